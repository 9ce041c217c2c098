"""CPU tests of the FP8 linear guardrails and the weight-cache design premise
(the reference's tests/test_precision.py:18-81 and tests/test_fp8_weight_cache.py:42-55)."""

import pytest
import torch
import torch.nn as nn

from flower_amd.precision import (Fp8Linear, _block_index, convert_model_to_fp8, fp8_module_filter,
                                  fp8_weight_cache, maybe_convert_fp8)


def test_block_index_parses_block_fqns():
    assert _block_index("blocks.0.ff.gate") == 0
    assert _block_index("blocks.19.attn.qkv") == 19


def test_block_index_returns_none_outside_blocks():
    assert _block_index("head") is None
    assert _block_index("mtp_heads.0") is None
    assert _block_index("token") is None


def test_filter_converts_interior_block_linears():
    keep = fp8_module_filter(num_layers=20, keep_bf16_blocks=1)
    aligned = nn.Linear(1280, 3392, bias=False)
    assert keep(aligned, "blocks.5.ff.gate") is True
    assert keep(aligned, "blocks.18.attn.qkv") is True


def test_filter_keeps_first_and_last_blocks_in_bf16():
    keep = fp8_module_filter(num_layers=20, keep_bf16_blocks=1)
    aligned = nn.Linear(1280, 3392, bias=False)
    assert keep(aligned, "blocks.0.ff.gate") is False
    assert keep(aligned, "blocks.19.ff.gate") is False


def test_filter_honours_wider_bf16_margin():
    keep = fp8_module_filter(num_layers=20, keep_bf16_blocks=4)
    aligned = nn.Linear(1280, 3392, bias=False)
    assert keep(aligned, "blocks.3.ff.gate") is False
    assert keep(aligned, "blocks.16.ff.gate") is False
    assert keep(aligned, "blocks.4.ff.gate") is True


def test_filter_never_converts_the_tied_lm_head():
    keep = fp8_module_filter(num_layers=20, keep_bf16_blocks=0)
    assert keep(nn.Linear(1280, 16384, bias=False), "head") is False


def test_filter_rejects_unaligned_dims():
    keep = fp8_module_filter(num_layers=20, keep_bf16_blocks=0)
    assert keep(nn.Linear(1280, 2730, bias=False), "blocks.5.ff.gate") is False
    assert keep(nn.Linear(2730, 1280, bias=False), "blocks.5.ff.down") is False
    assert keep(nn.Linear(1280, 2752, bias=False), "blocks.5.ff.gate") is True


def test_filter_ignores_non_linear_modules():
    keep = fp8_module_filter(num_layers=20, keep_bf16_blocks=0)
    assert keep(nn.RMSNorm(1280), "blocks.5.n1") is False
    assert keep(nn.Embedding(16384, 1280), "token") is False


def test_keep_zero_converts_every_aligned_block_linear():
    keep = fp8_module_filter(num_layers=20, keep_bf16_blocks=0)
    aligned = nn.Linear(1280, 3392, bias=False)
    assert keep(aligned, "blocks.0.ff.gate") is True
    assert keep(aligned, "blocks.19.ff.gate") is True


def test_version_counter_would_be_an_unsafe_invalidation_signal():
    p = nn.Parameter(torch.randn(4, 4))
    before = p._version
    with torch.no_grad():
        p.data -= 0.1
    assert p._version == before, "p.data -= now bumps _version; revisit the cache design"
    with torch.no_grad():
        p.add_(torch.ones(4, 4))
    assert p._version > before


class _Tiny(nn.Module):
    def __init__(self, n=4):
        super().__init__()
        self.blocks = nn.ModuleList(
            nn.ModuleDict({"qkv": nn.Linear(64, 192, bias=False), "odd": nn.Linear(64, 30)}) for _ in range(n))
        self.head = nn.Linear(64, 128, bias=False)


def test_convert_swaps_only_eligible_layers_and_keeps_parameters():
    m = _Tiny()
    params_before = {id(p) for p in m.parameters()}
    m, info = convert_model_to_fp8(m, keep_bf16_blocks=1, verbose=False)
    assert info["fp8_converted_linears"] == 2 and info["fp8_total_linears"] == 9
    assert isinstance(m.blocks[1]["qkv"], Fp8Linear) and isinstance(m.blocks[2]["qkv"], Fp8Linear)
    assert not isinstance(m.blocks[0]["qkv"], Fp8Linear) and not isinstance(m.blocks[3]["qkv"], Fp8Linear)
    assert not isinstance(m.head, Fp8Linear) and not isinstance(m.blocks[1]["odd"], Fp8Linear)
    assert {id(p) for p in m.parameters()} == params_before


def test_default_recipe_is_the_references_tensorwise():
    """convert_model_to_fp8(model) with no recipe, maybe_convert_fp8 with a config that carries none,
    and a bare Fp8Linear all take "tensorwise" (precision.py:137, config.py:593)."""
    m, info = convert_model_to_fp8(_Tiny(), verbose=False)
    assert info["fp8_recipe"] == "tensorwise"
    assert m.blocks[1]["qkv"].recipe == "tensorwise" and m.blocks[2]["qkv"].recipe == "tensorwise"
    assert Fp8Linear(32, 32).recipe == "tensorwise"
    assert Fp8Linear.from_linear(nn.Linear(32, 32)).recipe == "tensorwise"
    m2, info2 = convert_model_to_fp8(_Tiny(), recipe="rowwise", verbose=False)
    assert info2["fp8_recipe"] == "rowwise" and m2.blocks[1]["qkv"].recipe == "rowwise"


def test_convert_refuses_models_without_blocks_and_unknown_recipes():
    with pytest.raises(RuntimeError, match="no `blocks`"):
        convert_model_to_fp8(nn.Sequential(nn.Linear(16, 16)), verbose=False)
    with pytest.raises(RuntimeError, match="fp8_recipe"):
        convert_model_to_fp8(_Tiny(), recipe="int8", verbose=False)


def test_maybe_convert_guards():
    class Cfg:
        fp8_linear = True
        precision = "bf16"
        fp8_recipe = "rowwise"
        fp8_keep_bf16_blocks = 1

    assert maybe_convert_fp8(_Tiny(), type("Off", (), {"fp8_linear": False})(), torch.device("cpu"))[1] == {}
    with pytest.raises(RuntimeError, match="GPU"):
        maybe_convert_fp8(_Tiny(), Cfg(), torch.device("cpu"))
    Cfg.precision = "fp32"
    with pytest.raises(RuntimeError, match="bf16"):
        maybe_convert_fp8(_Tiny(), Cfg(), torch.device("cuda"))


def test_weight_cache_is_a_no_op_without_fp8_layers():
    """The cache only touches Fp8Linear layers; a bf16 model passes through untouched."""
    m = nn.Sequential(nn.Linear(8, 8))
    before = m[0].forward
    with fp8_weight_cache(m) as c:
        assert c.entries == []
    assert m[0].forward == before
