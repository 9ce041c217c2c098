"""CPU: the training block's construction (flower_amd.block): the SwiGLU width rule of base.py:370-383
on known widths, the 450M vanilla_matched configuration as configs/sweep13_450m_longctx_fp8.yaml
:94-113 sets it, and the parameter names of the reference's TransformerBlock / FeedForward
(base.py:485-552, :698-722), which checkpoints and the FP8 conversion filter rely on."""

import pytest
import torch.nn as nn

from flower_amd.block import FeedForward, TransformerBlock, block_config, swiglu_hidden_dim


@pytest.mark.parametrize("ffn,want", [(5120, 3392), (4096, 2752), (3072, 2048), (64, 64), (96, 64), (1000, 640)])
def test_swiglu_width(ffn, want):
    # 2/3 of the width (integer division), rounded to the nearest multiple of 64, at least 64
    assert swiglu_hidden_dim(ffn) == want
    assert swiglu_hidden_dim(ffn, param_match=False) == ffn


def test_450m_block_config_and_names():
    conf = block_config()
    assert (conf.d_model, conf.num_heads, conf.ffn_dim, conf.local_window) == (1280, 20, 5120, 2048)
    assert conf.ffn_activation == "swiglu" and conf.qk_norm and not conf.use_bias
    blk = TransformerBlock(conf)
    names = {n: tuple(p.shape) for n, p in blk.named_parameters()}
    assert names == {"ln1.weight": (1280,), "attn.qkv.weight": (3840, 1280), "attn.out.weight": (1280, 1280),
                     "ln2.weight": (1280,), "ff.gate.weight": (3392, 1280), "ff.up.weight": (3392, 1280),
                     "ff.down.weight": (1280, 3392)}
    assert sum(isinstance(m, nn.Linear) for m in blk.modules()) == 5


def test_gelu_feedforward_layout():
    ff = FeedForward(block_config(d_model=256, num_heads=4, ffn_dim=1024, ffn_activation="gelu", use_bias=True))
    assert [n for n, _ in ff.named_parameters()] == ["net.0.weight", "net.0.bias", "net.3.weight", "net.3.bias"]
    with pytest.raises(ValueError):
        FeedForward(block_config(ffn_activation="relu"))
