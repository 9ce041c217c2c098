"""GPU: the training block (flower_amd.block.TransformerBlock, base.py:698-722 with the SwiGLU feed-
forward of base.py:485-552) forward and backward, with bf16 Linears and with its Linears converted
to FP8 by convert_model_to_fp8, against the same block computed in float32 torch from the same
parameters (RMSNorm, qkv, HeadRMSNorm of q and k, RoPE, masked softmax attention over the window,
out, SwiGLU, the two residual adds).

Gates (written here): bf16 Linears -- output and every gradient within 3 % (Frobenius, relative)
of float32, the bf16 rounding of each stage; FP8 Linears -- within 12 % for the output's update
(out - x) and the gradients (each FP8 GEMM adds 2-4 %, and a backward chains several), and the
tensorwise and rowwise recipes both inside that gate.
"""

import copy

import pytest
import torch
import torch.nn as nn

pytestmark = pytest.mark.gpu

SHAPE = dict(B=2, T=320)
CFG = dict(d_model=256, num_heads=4, ffn_dim=1536, local_window=96, max_seq_len=512)


def _block():
    from flower_amd.block import TransformerBlock, block_config, init_block_
    conf = block_config(**CFG)
    blk = init_block_(TransformerBlock(conf), std=0.05, seed=5)
    with torch.no_grad():
        for norm in (blk.ln1, blk.ln2):
            norm.weight.copy_(1.0 + 0.1 * torch.randn(norm.weight.shape, generator=torch.Generator().manual_seed(9)))
    return blk.to("cuda", torch.bfloat16), conf


def _reference(blk, conf, x, dy):
    """float32 forward and backward of the same block, from its parameters."""
    P = {n: p.detach().float().clone().requires_grad_(True) for n, p in blk.named_parameters()}
    x = x.detach().float().clone().requires_grad_(True)
    B, T, d = x.shape
    H, W = conf.num_heads, conf.local_window
    D = d // H

    def rms(t, w, eps=1e-6):
        return t * t.pow(2).mean(-1, keepdim=True).add(eps).rsqrt() * w

    h = rms(x, P["ln1.weight"])
    q, k, v = (h @ P["attn.qkv.weight"].t()).chunk(3, dim=-1)
    q, k, v = (t.reshape(B, T, H, D).transpose(1, 2) for t in (q, k, v))
    q, k = (t * t.pow(2).mean(-1, keepdim=True).add(blk.attn.qk_norm.eps).rsqrt() for t in (q, k))
    cos, sin = (t.to(x.device).float() for t in blk.attn.rope._tables(T))

    def rot(t):
        return torch.stack((-t[..., 1::2], t[..., ::2]), dim=-1).flatten(-2)
    q, k = q * cos + rot(q) * sin, k * cos + rot(k) * sin
    i = torch.arange(T, device=x.device)
    band = (i[:, None] >= i[None, :]) & (i[:, None] - i[None, :] < W)
    s = (q @ k.transpose(-1, -2)) / D ** 0.5
    a = torch.softmax(s.masked_fill(~band, float("-inf")), dim=-1) @ v
    x1 = x + a.transpose(1, 2).reshape(B, T, d) @ P["attn.out.weight"].t()
    h2 = rms(x1, P["ln2.weight"])
    f = torch.nn.functional.silu(h2 @ P["ff.gate.weight"].t()) * (h2 @ P["ff.up.weight"].t())
    y = x1 + f @ P["ff.down.weight"].t()
    y.backward(dy.float())
    return y.detach(), x.grad, {n: p.grad for n, p in P.items()}


def _run(blk, x, dy):
    x = x.clone().requires_grad_(True)
    y = blk(x)[0]
    y.backward(dy)
    return y.detach().float(), x.grad.float(), {n: p.grad.float() for n, p in blk.named_parameters()}


def _rel(a, b):
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _inputs(conf):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(SHAPE["B"], SHAPE["T"], conf.d_model, generator=g).to("cuda", torch.bfloat16)
    dy = torch.randn(SHAPE["B"], SHAPE["T"], conf.d_model, generator=g).to("cuda", torch.bfloat16)
    return x, dy


def test_block_shape_and_swiglu_width():
    blk, conf = _block()
    assert blk.ff.hidden_dim == 1024          # 2/3 of 1536, a multiple of 64
    x, _ = _inputs(conf)
    with torch.no_grad():
        y, mem = blk(x)
    assert y.shape == x.shape and y.dtype == torch.bfloat16 and mem is None


def test_bf16_block_forward_backward_against_fp32():
    blk, conf = _block()
    x, dy = _inputs(conf)
    y_ref, gx_ref, gp_ref = _reference(blk, conf, x, dy)
    y, gx, gp = _run(blk, x, dy)
    assert _rel(y - x.float(), y_ref - x.float()) < 0.03
    assert _rel(gx, gx_ref) < 0.03
    for name, g in gp.items():
        assert _rel(g, gp_ref[name]) < 0.03, name


@pytest.mark.parametrize("recipe", ["tensorwise", "rowwise"])
def test_fp8_block_forward_backward_against_fp32(recipe):
    from flower_amd.precision import Fp8Linear, convert_model_to_fp8
    blk, conf = _block()
    x, dy = _inputs(conf)
    y_ref, gx_ref, gp_ref = _reference(blk, conf, x, dy)
    stack = nn.Module()
    stack.blocks = nn.ModuleList([copy.deepcopy(blk)])
    info = convert_model_to_fp8(stack, recipe=recipe, keep_bf16_blocks=0, verbose=False)[1]
    fblk = stack.blocks[0]
    assert info["fp8_converted_linears"] == 5
    assert sum(isinstance(m, Fp8Linear) for m in fblk.modules()) == 5
    y, gx, gp = _run(fblk, x, dy)
    assert _rel(y - x.float(), y_ref - x.float()) < 0.12
    assert _rel(gx, gx_ref) < 0.12
    for name, g in gp.items():
        assert _rel(g, gp_ref[name]) < 0.12, name


@pytest.mark.parametrize("fp8", [False, True])
def test_residual_norm_route_bit_identical_to_the_module_route(fp8):
    """TransformerBlock.forward on bf16 GPU inputs (ln1 handing x on as the residual stream, the
    first residual add inside ln2's pass, the residual gradients added in the norms' backward
    passes; with tensorwise FP8 Linears also the fused gate / up / SwiGLU node that casts x once
    and takes the amax of h, dgate and dup in the SwiGLU passes) against the same block composed
    module by module -- each Linear on its own, _SwiGLUFn, torch's adds and autograd's gradient
    sums: output, input gradient and every parameter gradient equal bit for bit."""
    from flower_amd.block import _SwiGLUFn
    blk, conf = _block()
    if fp8:
        from flower_amd.precision import convert_model_to_fp8
        stack = nn.Module()
        stack.blocks = nn.ModuleList([blk])
        convert_model_to_fp8(stack, recipe="tensorwise", keep_bf16_blocks=0, verbose=False)
        blk = stack.blocks[0]
    x, dy = _inputs(conf)
    y, gx, gp = _run(blk, x, dy)
    blk.zero_grad(set_to_none=True)
    xx = x.clone().requires_grad_(True)
    h = xx + blk.attn(blk.ln1(xx))
    t = blk.ln2(h)
    y2 = h + blk.ff.down(_SwiGLUFn.apply(blk.ff.gate(t), blk.ff.up(t)))
    y2.backward(dy)
    assert torch.equal(y, y2.detach().float())
    assert torch.equal(gx, xx.grad.float())
    for n, p in blk.named_parameters():
        assert torch.equal(gp[n], p.grad.float()), n


def test_fused_fp8_routes_inside_the_weight_cache():
    """Inside fp8_weight_cache the fused gate / up / SwiGLU node and the down projection with the
    residual take the cached weight codes (forward) and the cached column codes (dgrad): two steps
    inside the cache equal two uncached steps bit for bit, and the cache quantises each weight's
    columns once."""
    from flower_amd.precision import convert_model_to_fp8, fp8_weight_cache
    blk, conf = _block()
    stack = nn.Module()
    stack.blocks = nn.ModuleList([blk])
    convert_model_to_fp8(stack, recipe="tensorwise", keep_bf16_blocks=0, verbose=False)
    blk = stack.blocks[0]
    x, dy = _inputs(conf)
    y0, gx0, gp0 = _run(blk, x, dy)
    blk.zero_grad(set_to_none=True)
    with fp8_weight_cache(stack):
        for _ in range(2):
            y1, gx1, _ = _run(blk, x, dy)
        cols = [m._fp8_cached_cols is not None for m in (blk.ff.gate, blk.ff.up, blk.ff.down)]
    assert all(cols)
    assert torch.equal(y0, y1) and torch.equal(gx0, gx1)
    for n, p in blk.named_parameters():
        assert torch.equal(p.grad.float(), 2 * gp0[n]), n


def test_fused_fp8_block_ragged_tokens_bit_identical():
    """A ragged token count (B1 x T77: 77 rows, the wgrad operands zero-padded to 128 columns,
    partial GEMM tiles, a partial last attention tile) through the fused tensorwise routes equals
    the module-by-module composition bit for bit."""
    from flower_amd.block import _SwiGLUFn
    from flower_amd.precision import convert_model_to_fp8
    blk, conf = _block()
    stack = nn.Module()
    stack.blocks = nn.ModuleList([blk])
    convert_model_to_fp8(stack, recipe="tensorwise", keep_bf16_blocks=0, verbose=False)
    blk = stack.blocks[0]
    g = torch.Generator().manual_seed(21)
    x = torch.randn(1, 77, conf.d_model, generator=g).to("cuda", torch.bfloat16)
    dy = torch.randn(1, 77, conf.d_model, generator=g).to("cuda", torch.bfloat16)
    y, gx, gp = _run(blk, x, dy)
    blk.zero_grad(set_to_none=True)
    xx = x.clone().requires_grad_(True)
    h = xx + blk.attn(blk.ln1(xx))
    t = blk.ln2(h)
    y2 = h + blk.ff.down(_SwiGLUFn.apply(blk.ff.gate(t), blk.ff.up(t)))
    y2.backward(dy)
    assert torch.equal(y, y2.detach().float()) and torch.equal(gx, xx.grad.float())
    for n, p in blk.named_parameters():
        assert torch.equal(gp[n], p.grad.float()), n


@pytest.mark.parametrize("T,cached", [(320, False), (77, False), (320, True)])
def test_fused_fp8_qkv_heads_node_bit_identical(T, cached, monkeypatch):
    """The qkv projection and the heads pass as one node (_Fp8QkvHeadsFn: the qkv_heads backward
    reports |dqkv|'s maximum, the gradient cast takes it in place of its amax pass) against the
    tensorwise Fp8Linear followed by _QkvHeadsFn (the default route; the node is opt-in through
    fused_fp8_qkv): q, k, v, x's gradient and the weight's equal bit for bit -- ragged tokens
    (B1 x T77) and inside fp8_weight_cache too."""
    from flower_amd.precision import convert_model_to_fp8, fp8_weight_cache
    blk, conf = _block()
    stack = nn.Module()
    stack.blocks = nn.ModuleList([blk])
    convert_model_to_fp8(stack, recipe="tensorwise", keep_bf16_blocks=0, verbose=False)
    attn = stack.blocks[0].attn
    g = torch.Generator().manual_seed(T)
    x = torch.randn(2 if T == 320 else 1, T, conf.d_model, generator=g).to("cuda", torch.bfloat16)
    dq, dk, dv = (torch.randn(x.shape[0], conf.num_heads, T, conf.d_model // conf.num_heads,
                              generator=g).to("cuda", torch.bfloat16) for _ in range(3))

    def run():
        xx = x.clone().requires_grad_(True)
        attn.qkv.weight.grad = None
        ctx = fp8_weight_cache(stack) if cached else torch.enable_grad()
        with ctx:
            q, k, v = attn.qkv_heads(xx)
            torch.autograd.backward((q, k, v), (dq, dk, dv))
        return q.detach(), k.detach(), v.detach(), xx.grad, attn.qkv.weight.grad.clone()

    assert not attn._fp8_qkv_ok(x.clone().requires_grad_(True))       # opt-in
    plain = run()
    monkeypatch.setattr(attn, "fused_fp8_qkv", True)
    assert attn._fp8_qkv_ok(x.clone().requires_grad_(True))
    fused = run()
    for a, b in zip(fused, plain):
        assert torch.equal(a, b)
