"""CPU: host logic of the attention module mirror (flower_amd.attention.CausalSelfAttention,
flower/models/base.py:553-665): config validation, parameter surface, the RoPE tables, and the
torch-side qkv_heads against the reference's expressions."""

from types import SimpleNamespace

import pytest
import torch


def _cfg(**kw):
    base = dict(d_model=128, num_heads=2, max_seq_len=64, rope_base=10000.0, use_bias=False, qk_norm=True,
                attn_precision="fp8")
    base.update(kw)
    return SimpleNamespace(**base)


def test_attn_precision_is_validated_like_the_reference():        # config.py:464-465
    from flower_amd.attention import CausalSelfAttention
    with pytest.raises(ValueError, match="attn_precision must be bf16|fp8"):
        CausalSelfAttention(_cfg(attn_precision="fp4"))
    with pytest.raises(ValueError, match="divisible"):
        CausalSelfAttention(_cfg(d_model=129))
    with pytest.raises(ValueError, match="rbf"):
        CausalSelfAttention(_cfg(local_attn_kernel_bias="rbf"))


def test_module_surface_matches_the_reference():
    """Parameter names and shapes of base.py:556-567 (qkv, out Linears; parameter-free QK-norm),
    bias following config.use_bias (default True, as base.py:562)."""
    from flower_amd.attention import CausalSelfAttention, HeadRMSNorm
    m = CausalSelfAttention(_cfg(), local_window=16)
    names = {n: tuple(p.shape) for n, p in m.named_parameters()}
    assert names == {"qkv.weight": (384, 128), "out.weight": (128, 128)}
    assert isinstance(m.qk_norm, HeadRMSNorm) and m.head_dim == 64 and m.local_window == 16
    cfg = _cfg(qk_norm=False)
    del cfg.use_bias
    m2 = CausalSelfAttention(cfg)
    assert m2.qk_norm is None and m2.qkv.bias is not None


def test_rope_tables_and_extension_follow_the_reference_construction():
    """base.py:444-457 (and the lazy extension, :471-476): cos / sin of position * base^(-2i/D),
    each frequency repeated for the pair (2i, 2i+1)."""
    from flower_amd.attention import RotaryEmbedding
    r = RotaryEmbedding(64, 32, base=500.0)
    inv = 1.0 / (500.0 ** (torch.arange(0, 64, 2).float() / 64))
    f = torch.outer(torch.arange(48).float(), inv)
    cos, sin = r.tables(48, torch.float32, "cpu")          # longer than max_seq_len: extended
    assert torch.equal(cos, f.cos().repeat_interleave(2, dim=-1))
    assert torch.equal(sin, f.sin().repeat_interleave(2, dim=-1))
    cb, _ = r.tables(48, torch.bfloat16, "cpu")
    assert cb.dtype == torch.bfloat16 and torch.equal(cb, cos.to(torch.bfloat16))


def test_qkv_heads_is_the_reference_pipeline():
    """qkv -> split -> HeadRMSNorm -> RoPE, written out with the reference's expressions."""
    from flower_amd.attention import CausalSelfAttention
    torch.manual_seed(0)
    m = CausalSelfAttention(_cfg(attn_precision="bf16"))
    x = torch.randn(2, 20, 128)
    q, k, v = m.qkv_heads(x)
    y = x @ m.qkv.weight.t()
    qs, ks, vs = (t.view(2, 20, 2, 64).transpose(1, 2) for t in y.chunk(3, dim=-1))

    def norm(t):
        return t.float() * t.float().pow(2).mean(-1, keepdim=True).add(1e-6).rsqrt()

    def rot(t):
        return torch.stack((-t[..., 1::2], t[..., ::2]), dim=-1).flatten(-2)
    cos, sin = m.rope.tables(20, torch.float32, "cpu")
    for got, src in ((q, qs), (k, ks)):
        n = norm(src)
        torch.testing.assert_close(got, n * cos + rot(n) * sin)
    torch.testing.assert_close(v, vs)


def test_attention_from_codes_refuses_mismatched_operands_on_the_host():
    """fp8_swa_attention_from_codes hands the kernel only q8's B, H, T, D and strides, so every
    other operand is checked against q8 before any launch (CPU tensors: the refusals come before
    the GPU check, nothing reaches the library's kernels)."""
    import os
    from flower_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libflower_amd.so not built")
    from flower_amd.kernels.fp8_swa_attention import fp8_swa_attention_from_codes as f
    B, H, T, D = 1, 2, 100, 64
    lib = _lib.load()
    q8 = torch.zeros(B, H, T, D, dtype=torch.uint8)
    vt = torch.zeros(lib.flw_vtile_bytes(B, H, T, D), dtype=torch.uint8)
    sc = torch.ones(3 * H)
    with pytest.raises(ValueError, match="k8"):
        f(q8, torch.zeros(B, H, T - 1, D, dtype=torch.uint8), vt, sc, 16)            # shorter K
    with pytest.raises(ValueError, match="e4m3 codes"):
        f(q8, q8.to(torch.int8), vt, sc, 16)                                          # wrong code dtype
    with pytest.raises(ValueError, match="e4m3 codes"):
        f(q8.float(), q8, vt, sc, 16)
    with pytest.raises(ValueError, match="tile buffer"):
        f(q8, q8, vt[:-64], sc, 16)                                                   # undersized V tiles
    with pytest.raises(ValueError, match="V codes"):
        f(q8, q8, torch.zeros(B, H, T + 1, D, dtype=torch.uint8), sc, 16)             # V of another T
    with pytest.raises(ValueError, match="out must be"):
        f(q8, q8, vt, sc, 16, out=torch.empty(B, H, T, D, dtype=torch.float32))       # out dtype != out_dtype
    with pytest.raises(ValueError, match="granularity"):
        f(q8, q8, vt, sc, 16, granularity="row")
    with pytest.raises(ValueError, match="scales"):
        f(q8, q8, vt, torch.ones(3), 16)                                              # per-tensor count for "head"
    with pytest.raises(ValueError, match="head_dim"):
        f(torch.zeros(B, H, T, 48, dtype=torch.uint8), q8, vt, sc, 16)
    with pytest.raises(ValueError, match="out_dtype"):
        f(q8, q8, vt, sc, 16, out_dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU"):                                    # consistent: only then the GPU check
        f(q8, q8, vt, sc, 16)
