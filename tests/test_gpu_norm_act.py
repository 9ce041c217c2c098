"""GPU: the training block's RMSNorm (flower/models/base.py:324-338) and SwiGLU product
(base.py:538-550) passes, forward and backward (flw_rmsnorm_fwd / _bwd, flw_swiglu_fwd / _bwd),
through the modules' autograd routes (flower_amd.block._RMSNormFn, _SwiGLUFn) and the C ABI.

Gates (written here), against the oracle (oracle/block.py: the torch expressions' roundings):
  - RMSNorm h and dx: < 0.5 % of values differ after the norm's fp32 sums (their order differs):
    h's by <= 2 bf16 ulps (a one-ulp flip of bf16(x r) becomes up to two after the gain's product
    is rounded again), dx's by <= 2^-7 |ref| + 2^-12 max|ref| of its row, since its difference of
    two rounded terms can cancel; dw (a sum over every row): within 2 bf16 ulps;
  - SwiGLU h, dgate, dup: < 0.5 % differ, each by one ulp (the device exp against a correctly
    rounded one), dgate's with the same cancellation allowance;
  - both against torch's bf16 autograd of the reference's expressions on the GPU: the same gates;
  - empty rows: dw is zero, nothing else written.
"""

import numpy as np
import pytest
import torch

from gpu_util import to_np
from oracle.block import rmsnorm, rmsnorm_backward, swiglu, swiglu_backward
from oracle.e4m3 import f32_to_bf16_bits

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _ulps(a, b):
    ia = f32_to_bf16_bits(np.asarray(a, np.float32)).astype(np.int64)
    ib = f32_to_bf16_bits(np.asarray(b, np.float32)).astype(np.int64)
    return np.abs(ia - ib)


def _close(got, ref, frac=5e-3, cancel=False, ulps=1):
    got, ref = np.asarray(got, np.float32), np.asarray(ref, np.float32)
    d = _ulps(got, ref)
    assert (d > 0).mean() < frac, (d > 0).mean()
    if cancel:
        row = np.abs(ref).max(axis=-1, keepdims=True)
        err = np.abs(got.astype(np.float64) - ref)
        assert (err <= 2.0 ** -7 * np.abs(ref) + 2.0 ** -12 * row).all(), float(err.max())
    else:
        assert d.max() <= ulps, int(d.max())


def _norm_inputs(rows, cols, seed, pad=0):
    g = torch.Generator().manual_seed(seed)
    base = (torch.randn(rows, cols + pad, generator=g) * 2.0).to("cuda", torch.bfloat16)
    x = base[:, :cols]
    w = (1.0 + 0.2 * torch.randn(cols, generator=g)).to("cuda", torch.bfloat16)
    dh = torch.randn(rows, cols, generator=g).to("cuda", torch.bfloat16)
    return x, w, dh


def _fused_norm(x, w, dh):
    from flower_amd.block import _RMSNormFn
    xx = x.detach().requires_grad_(True)
    ww = w.detach().requires_grad_(True)
    h = _RMSNormFn.apply(xx, ww, EPS)
    h.backward(dh)
    return h.detach(), xx.grad, ww.grad


NORM_CASES = [(513, 1280, 0), (300, 64, 0), (129, 1288, 16), (77, 4096, 0), (33, 8192, 0), (5, 520, 8)]


@pytest.mark.parametrize("rows,cols,pad", NORM_CASES)
def test_rmsnorm_forward_backward_against_oracle(rows, cols, pad):
    x, w, dh = _norm_inputs(rows, cols, seed=rows + cols, pad=pad)
    h, dx, dw = _fused_norm(x, w, dh)
    xn, wn, dn = to_np(x), to_np(w), to_np(dh)
    _close(to_np(h), rmsnorm(xn, wn, EPS), ulps=2)
    rdx, rdw = rmsnorm_backward(xn, wn, dn, EPS)
    _close(to_np(dx), rdx, cancel=True)
    assert _ulps(to_np(dw), rdw).max() <= 2


def test_rmsnorm_against_torch_autograd():
    x, w, dh = _norm_inputs(1024, 1280, seed=3)
    h, dx, dw = _fused_norm(x, w, dh)
    xx = x.detach().requires_grad_(True)
    ww = w.detach().requires_grad_(True)
    rms = xx.float().pow(2).mean(dim=-1, keepdim=True).add(EPS).rsqrt()      # base.py:337-338
    ht = (xx.float() * rms).to(torch.bfloat16) * ww
    ht.backward(dh)
    _close(to_np(h), to_np(ht), ulps=2)
    _close(to_np(dx), to_np(xx.grad), cancel=True)
    assert _ulps(to_np(dw), to_np(ww.grad)).max() <= 2


def test_rmsnorm_empty_rows_give_zero_weight_gradient():
    from flower_amd import _lib
    lib = _lib.load()
    x = torch.empty((0, 64), dtype=torch.bfloat16, device="cuda")
    w = torch.ones(64, dtype=torch.bfloat16, device="cuda")
    dw = torch.full((64,), 7.0, dtype=torch.bfloat16, device="cuda")
    s = _lib.stream_of(w)
    _lib.check(lib.flw_rmsnorm_bwd(w.data_ptr(), 0, 64, 64, w.data_ptr(), EPS, w.data_ptr(), 64, None, 0, w.data_ptr(), 64,
                                   dw.data_ptr(), None, 0, s), "rmsnorm bwd")
    _lib.check(lib.flw_rmsnorm_fwd(w.data_ptr(), 0, 64, 64, w.data_ptr(), EPS, w.data_ptr(), 64, s), "rmsnorm fwd")
    torch.cuda.synchronize()
    assert torch.equal(dw, torch.zeros_like(dw)) and torch.equal(w, torch.ones_like(w)) and x.numel() == 0


SWIGLU_CASES = [(2, 1000, 3392, 0), (1, 37, 64, 0), (3, 50, 1024, 64)]


@pytest.mark.parametrize("B,T,cols,pad", SWIGLU_CASES)
def test_swiglu_forward_backward_against_oracle(B, T, cols, pad):
    from flower_amd.block import _SwiGLUFn
    g = torch.Generator().manual_seed(cols + T)
    gu = (torch.randn(B, T, 2 * cols + pad, generator=g) * 3.0).to("cuda", torch.bfloat16)
    gate, up = gu[..., :cols], gu[..., cols:2 * cols]                   # row stride 2 cols + pad
    dh = torch.randn(B, T, cols, generator=g).to("cuda", torch.bfloat16)
    gg, uu = gate.detach().requires_grad_(True), up.detach().requires_grad_(True)
    h = _SwiGLUFn.apply(gg, uu)
    h.backward(dh)
    gn, un, dn = to_np(gate), to_np(up), to_np(dh)
    _close(to_np(h), swiglu(gn, un))
    rdg, rdu = swiglu_backward(gn, un, dn)
    _close(to_np(gg.grad), rdg, cancel=True)
    _close(to_np(uu.grad), rdu)
    # torch's bf16 autograd of the reference's expressions on the same inputs
    gt, ut = gate.detach().requires_grad_(True), up.detach().requires_grad_(True)
    ht = torch.nn.functional.silu(gt) * ut
    ht.backward(dh)
    _close(to_np(h), to_np(ht))
    _close(to_np(gg.grad), to_np(gt.grad), cancel=True)
    _close(to_np(uu.grad), to_np(ut.grad))


def test_add_rmsnorm_and_residual_gradient_against_torch():
    """flw_add_rmsnorm_fwd: s = bf16(x + a) bit for bit torch's add, h = the norm of s (the same
    kernel arithmetic as flw_rmsnorm_fwd on s); flw_rmsnorm_bwd with dres: bf16(dres + the norm's
    dx), bit for bit autograd's sum of the two bf16 gradients."""
    from flower_amd import _lib
    from flower_amd.block import _AddRMSNormFn, _RMSNormFn
    x, w, dh = _norm_inputs(333, 1280, seed=21)
    a, _, dres = _norm_inputs(333, 1280, seed=22)
    xx, aa = x.detach().requires_grad_(True), a.detach().requires_grad_(True)
    s, h = _AddRMSNormFn.apply(xx, aa, w, EPS)
    assert torch.equal(s, x + a)
    ss = (x + a).detach().requires_grad_(True)
    h_ref = _RMSNormFn.apply(ss, w, EPS)
    assert torch.equal(h, h_ref)
    torch.autograd.backward((s, h), (dres, dh))
    torch.autograd.backward((ss, h_ref), (dres, dh))       # autograd sums dres and the norm's dx
    assert torch.equal(xx.grad, ss.grad) and torch.equal(aa.grad, ss.grad)


def test_swiglu_amax_outputs_equal_the_maxima_of_what_they_wrote():
    """flw_swiglu_fwd's h_amax and flw_swiglu_bwd's [|dgate|, |dup|] maxima: the fp32 bit patterns
    of max |x| over the tensors they wrote (the amax pass's value), the tensors themselves equal to
    the calls without them; a NaN in gate makes the maxima NaN (0x7FC00000, above inf)."""
    from flower_amd import _lib
    lib = _lib.load()
    g = torch.Generator().manual_seed(31)
    M, H = 1000, 3392
    gate = (torch.randn(M, H, generator=g) * 3).to("cuda", torch.bfloat16)
    up = torch.randn(M, H, generator=g).to("cuda", torch.bfloat16)
    dh = torch.randn(M, H, generator=g).to("cuda", torch.bfloat16)
    s = _lib.stream_of(gate)
    ws = _lib.workspace(lib.flw_swiglu_amax_workspace_bytes(M, H), "cuda")

    def bits(t):
        return int(t.float().abs().max().view(torch.int32).item())
    for nan in (False, True):
        if nan:
            gate[17, 5] = float("nan")
        h0, h1 = torch.empty_like(gate), torch.empty_like(gate)
        am = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        _lib.check(lib.flw_swiglu_fwd(gate.data_ptr(), up.data_ptr(), M, H, H, H, h0.data_ptr(), H, None, None, 0, s), "f")
        _lib.check(lib.flw_swiglu_fwd(gate.data_ptr(), up.data_ptr(), M, H, H, H, h1.data_ptr(), H, am.data_ptr(),
                                      ws.data_ptr(), ws.numel(), s), "f amax")
        dg0, du0, dg1, du1 = (torch.empty_like(gate) for _ in range(4))
        am2 = torch.full((2,), -1, dtype=torch.int32, device="cuda")
        _lib.check(lib.flw_swiglu_bwd(gate.data_ptr(), up.data_ptr(), M, H, H, H, dh.data_ptr(), H, dg0.data_ptr(),
                                      du0.data_ptr(), H, None, None, 0, s), "b")
        _lib.check(lib.flw_swiglu_bwd(gate.data_ptr(), up.data_ptr(), M, H, H, H, dh.data_ptr(), H, dg1.data_ptr(),
                                      du1.data_ptr(), H, am2.data_ptr(), ws.data_ptr(), ws.numel(), s), "b amax")
        torch.cuda.synchronize()
        assert torch.equal(h0.view(torch.int16), h1.view(torch.int16))
        assert torch.equal(dg0.view(torch.int16), dg1.view(torch.int16))
        assert torch.equal(du0.view(torch.int16), du1.view(torch.int16))
        if nan:
            assert int(am.item()) == 0x7FC00000 and int(am2[0].item()) == 0x7FC00000
        else:
            assert int(am.item()) == bits(h1)
            assert int(am2[0].item()) == bits(dg1) and int(am2[1].item()) == bits(du1)
