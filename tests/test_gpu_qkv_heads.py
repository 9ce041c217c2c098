"""GPU: the fused training pass of CausalSelfAttention.qkv_heads (flower/models/base.py:618-639:
split of the qkv projection into heads, HeadRMSNorm of q and k, base.py:341-357, RoPE,
base.py:436-483), forward (flw_qkv_heads_fwd) and backward (flw_qkv_heads_bwd), through the
module's autograd route.

Gates (written here):
  - forward: v bit for bit; q', k' against the oracle's head_rmsnorm + rope on the same inputs --
    RoPE alone bit for bit, with the norm < 0.2 % of values differing, each by <= 2^-7 (|v| + 1)
    (the mean of squares' summation order, then RoPE's sum that can cancel a one-ulp input);
  - backward: dv bit for bit; dq, dk against the oracle's rope_backward + head_rmsnorm_backward
    (torch autograd's roundings) -- RoPE alone bit for bit, with the norm < 0.5 % of values
    differing, each by <= 2^-7 |ref| + 2^-12 max|ref| of its head row (the norm's fp32 sums);
  - the module's qkv_heads outputs and gradients (fused route) against the reference's torch
    expressions on the same submodules under autograd: relative Frobenius < 1e-2; against float32
    autograd < 2 %, within 0.5 % of the torch route's own distance.
"""

import numpy as np
import pytest
import torch

from gpu_util import to_np
from oracle.block import head_rmsnorm, head_rmsnorm_backward, rope, rope_backward

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _mk(B, T, H, D, seed, pad=0):
    g = torch.Generator().manual_seed(seed)
    C = 3 * H * D
    base = (torch.randn(B, T, C + pad, generator=g) * 1.7).to("cuda", torch.bfloat16)
    y = base[..., :C]                                          # row stride C + pad when pad > 0
    grads = [torch.randn(B, H, T, D, generator=g).to("cuda", torch.bfloat16) for _ in range(3)]
    return y, grads


def _heads(y, H, D):
    B, T, _ = y.shape
    return [t.reshape(B, T, H, D).transpose(1, 2) for t in y.float().chunk(3, dim=-1)]


def _tables(T, D):
    from flower_amd.attention import RotaryEmbedding
    return RotaryEmbedding(D, T).tables(T, torch.bfloat16, "cuda")


def _oracle_fwd(y, H, D, norm, cos, sin):
    q, k, v = (to_np(t) for t in _heads(y, H, D))
    c, s = to_np(cos.float()), to_np(sin.float())
    out = []
    for t in (q, k):
        if norm:
            t = head_rmsnorm(t, EPS, "bf16")
        out.append(rope(t, c, s, "bf16"))
    return out + [v]


def _oracle_bwd(y, H, D, norm, cos, sin, grads):
    q, k, _ = (to_np(t) for t in _heads(y, H, D))
    c, s = to_np(cos.float()), to_np(sin.float())
    out = []
    for x, g in zip((q, k), grads[:2]):
        dn = rope_backward(to_np(g.float()), c, s, "bf16")
        out.append(head_rmsnorm_backward(x, dn, EPS, "bf16") if norm else dn)
    return out + [to_np(grads[2].float())]


def _fused(y, H, norm, cos, sin, grads):
    from flower_amd.attention import _QkvHeadsFn
    yy = y.detach().requires_grad_(True)
    q, k, v = _QkvHeadsFn.apply(yy, H, norm, EPS, cos, sin)
    torch.autograd.backward((q, k, v), grads)
    return (q, k, v), yy.grad


CASES = [(2, 77, 3, 32, True, 0), (2, 77, 3, 32, False, 0), (1, 130, 2, 64, True, 64),
         (1, 130, 2, 64, False, 0), (2, 65, 2, 128, True, 0), (1, 40, 5, 128, False, 128)]


@pytest.mark.parametrize("B,T,H,D,norm,pad", CASES)
def test_fused_heads_forward_against_oracle(B, T, H, D, norm, pad):
    y, grads = _mk(B, T, H, D, seed=T + D, pad=pad)
    cos, sin = _tables(T, D)
    (q, k, v), _ = _fused(y, H, norm, cos, sin, grads)
    for t in (q, k, v):
        assert t.shape == (B, H, T, D) and t.is_contiguous() and t.dtype == torch.bfloat16
    want = _oracle_fwd(y, H, D, norm, cos, sin)
    assert np.array_equal(to_np(v.float()).view(np.uint32), want[2].view(np.uint32))
    for got, ref in zip((q, k), want[:2]):
        got = to_np(got.float())
        if not norm:
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
            continue
        d = np.abs(got.astype(np.float64) - ref)
        assert (d > 0).mean() < 2e-3, (d > 0).mean()
        assert (d <= 2.0 ** -7 * (np.abs(ref) + 1.0)).all(), float(d.max())


@pytest.mark.parametrize("B,T,H,D,norm,pad", CASES)
def test_fused_heads_backward_against_oracle(B, T, H, D, norm, pad):
    y, grads = _mk(B, T, H, D, seed=3 * T + D, pad=pad)
    cos, sin = _tables(T, D)
    _, dy = _fused(y, H, norm, cos, sin, grads)
    assert dy.shape == y.shape
    dq, dk, dv = (to_np(t.float()) for t in _heads(dy, H, D))
    want = _oracle_bwd(y, H, D, norm, cos, sin, grads)
    assert np.array_equal(dv.view(np.uint32), want[2].view(np.uint32))
    for got, ref in zip((dq, dk), want[:2]):
        if not norm:
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
            continue
        d = np.abs(got.astype(np.float64) - ref)
        row = np.abs(ref).max(axis=-1, keepdims=True)
        assert (d > 0).mean() < 5e-3, (d > 0).mean()
        assert (d <= 2.0 ** -7 * np.abs(ref) + 2.0 ** -12 * row).all(), float(d.max())


def test_module_route_against_torch_autograd_and_fp32():
    """CausalSelfAttention.qkv_heads (bf16 on the GPU: the fused route) against the reference's
    torch expressions on the same module's submodules under autograd, and float32 autograd."""
    import flower_amd.attention as A
    from types import SimpleNamespace
    conf = SimpleNamespace(d_model=256, num_heads=4, max_seq_len=512, rope_base=10000.0,
                           use_bias=False, qk_norm=True, fp8_attention_sim=False, attn_precision="bf16")
    torch.manual_seed(2)
    mod = A.CausalSelfAttention(conf).to("cuda", torch.bfloat16)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(2, 200, 256, generator=g).to("cuda", torch.bfloat16)
    gq = [torch.randn(2, 4, 200, 64, generator=g).to("cuda", torch.bfloat16) for _ in range(3)]

    def run(fused, dtype):
        m = mod if dtype == torch.bfloat16 else _fp32_copy(mod)
        xx = x.to(dtype).detach().requires_grad_(True)
        outs = m.qkv_heads(xx) if fused else _torch_route(m, xx)
        torch.autograd.backward(outs, [t.to(dtype) for t in gq])
        return [o.detach().float() for o in outs], xx.grad.float(), m.qkv.weight.grad.float()

    def rel(a, b):
        return float((a - b).norm() / b.norm())

    mod.zero_grad()
    f_out, f_gx, f_gw = run(True, torch.bfloat16)
    mod.zero_grad()
    t_out, t_gx, t_gw = run(False, torch.bfloat16)
    r_out, r_gx, r_gw = run(False, torch.float32)
    for a, b in zip(f_out, t_out):
        assert rel(a, b) < 1e-2
    assert rel(f_gx, t_gx) < 1e-2 and rel(f_gw, t_gw) < 1e-2
    assert rel(f_gx, r_gx) < 2e-2 and rel(f_gw, r_gw) < 2e-2
    assert abs(rel(f_gx, r_gx) - rel(t_gx, r_gx)) < 5e-3


def _fp32_copy(mod):
    import copy
    m = copy.deepcopy(mod).float()
    m.zero_grad()
    return m


def _torch_route(m, x):
    """The reference's qkv_heads expressions (base.py:618-639) on the module's own submodules."""
    q, k, v = m.qkv(x).chunk(3, dim=-1)
    q, k, v = m._split(q), m._split(k), m._split(v)
    if m.qk_norm is not None:
        q, k = m.qk_norm(q), m.qk_norm(k)
    return (*m.rope(q, k), v)
