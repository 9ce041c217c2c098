"""GPU: the bf16 sliding-window attention (flower/kernels/swa_attention.py counterpart) through the
C ABI, against dense masked attention in float64 torch (autograd for the gradients) on the same
bf16 values. Gates: the reference's own (tests/test_swa_kernel.py:20-55: forward mean-relative
< 0.01, each gradient < 0.02) plus max |d| / max |ref| < 2e-2 per tensor, and the saved
log-sum-exp within 1e-3 of torch.logsumexp."""

import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def dense(q, k, v, W):
    T, D = q.shape[-2], q.shape[-1]
    s = (q @ k.transpose(-1, -2)) / math.sqrt(D)
    i = torch.arange(T)
    keep = (i[:, None] >= i[None, :]) & ((i[:, None] - i[None, :]) < W)
    s = s.masked_fill(~keep, float("-inf"))
    return torch.softmax(s, -1) @ v, torch.logsumexp(s, -1)


def inputs(B, H, T, D, seed=0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(B, H, T, D, generator=g).to(torch.bfloat16) for _ in range(3)]


def rel(got, want):
    got, want = got.double(), want.double()
    return float((got - want).abs().mean() / want.abs().mean()), float((got - want).abs().max() / want.abs().max())


SHAPES = [(1, 2, 256, 64, 128), (2, 3, 512, 64, 256), (2, 2, 512, 32, 512), (1, 2, 200, 128, 64),
          (1, 2, 130, 64, 1000), (1, 1, 96, 64, 17)]


@pytest.mark.parametrize("B,H,T,D,W", SHAPES)
def test_forward_and_lse_match_dense(B, H, T, D, W):
    from flower_amd import _lib as L
    q, k, v = inputs(B, H, T, D)
    lb = L.load()
    tq, tk, tv = q.cuda(), k.cuda(), v.cuda()
    out = torch.empty_like(tq)
    lse = torch.empty((B, H, T), dtype=torch.float32, device="cuda")
    L.check(lb.flw_swa_bf16_fwd(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), B, H, T, D, W, out.data_ptr(),
                                lse.data_ptr(), L.stream_of(tq)), "fwd")
    ref, ref_lse = dense(q.double(), k.double(), v.double(), W)
    mean_rel, max_rel = rel(out.cpu(), ref)
    assert mean_rel < 0.01 and max_rel < 2e-2, (mean_rel, max_rel)
    assert float((lse.cpu().double() - ref_lse).abs().max()) < 1e-3


def test_window_one_returns_v():
    """W = 1: every query attends only to itself, so out == v exactly and lse == q.k / sqrt(D)."""
    from flower_amd.kernels.swa_attention import swa_attention
    q, k, v = (t.cuda() for t in inputs(1, 2, 160, 64, seed=3))
    out = swa_attention(q, k, v, 1)
    assert torch.equal(out, v)


@pytest.mark.parametrize("B,H,T,D,W", [(1, 2, 256, 64, 128), (2, 2, 512, 64, 256), (1, 2, 200, 128, 64),
                                       (2, 2, 256, 32, 256), (1, 1, 130, 64, 1000)])
def test_gradients_match_dense(B, H, T, D, W):
    from flower_amd.kernels.swa_attention import swa_attention
    base = inputs(B, H, T, D, seed=1)
    g = torch.randn(B, H, T, D, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    q, k, v = (t.cuda().requires_grad_(True) for t in base)
    swa_attention(q, k, v, W).backward(g.cuda())
    qr, kr, vr = (t.double().requires_grad_(True) for t in base)
    dense(qr, kr, vr, W)[0].backward(g.double())
    for name, got, want in (("dq", q.grad, qr.grad), ("dk", k.grad, kr.grad), ("dv", v.grad, vr.grad)):
        assert torch.isfinite(got).all(), name
        mean_rel, max_rel = rel(got.cpu(), want)
        assert mean_rel < 0.02 and max_rel < 2e-2, (name, mean_rel, max_rel)


def test_rejections():
    from flower_amd.kernels.swa_attention import swa_attention
    q, k, v = (torch.randn(1, 2, 128, 64, device="cuda", dtype=torch.bfloat16) for _ in range(3))
    with pytest.raises(ValueError, match="window must be positive"):
        swa_attention(q, k, v, 0)
    with pytest.raises(ValueError, match="head_dim"):
        swa_attention(*(torch.randn(1, 2, 128, 96, device="cuda", dtype=torch.bfloat16) for _ in range(3)), 16)
    with pytest.raises(TypeError):
        swa_attention(q.float(), k.float(), v.float(), 16)
