"""GPU: the differentiable FP8 attention (flower_amd.kernels.fp8_swa_attention: the FP8 forward, the
e4m3 dequantiser flw_dequant_e4m3, the bf16 forward + backward run at the dequantised Q, K, V) and
the FP8 kernel's log-sum-exp output (flw_fp8_swa_fwd_lse), through the C ABI, against the float64
oracle.

What the op computes (the reference trains FP8 attention with `_fake_quant_e4m3`'s straight-through
quantisers, flower/models/base.py:167-203, and a bf16 attention backward that rebuilds P from row
statistics, flower/kernels/swa_attention.py:307-359): forward = the FP8 kernel on e4m3 codes;
gradients = those of attention at the dequantised values q8 * s_q, k8 * s_k, v8 * s_v (rounded to
bf16 for the bf16 backward). The oracle is oracle/swa_grad.py in float64 on those bf16 values (and,
reported, on the exact dequantised values).

Gates (written here):
  - dequantised values bit for bit against e4m3(code) * scale rounded to bf16 (both layouts);
  - the FP8 kernel's log-sum-exp within 2e-3 (absolute, natural log) of the oracle's on the
    dequantised values, and its output unchanged bit for bit by writing it;
  - the op's forward output bit for bit equal to fp8_swa_attention_forward's;
  - gradients (O and the log-sum-exp recomputed by the bf16 forward on the dequantised bf16
    values): against the oracle at the bf16 dequantised values (the point the backward runs at, and
    what `_fake_quant_e4m3` returns in a bf16 model) the reference's gate
    (tests/test_swa_kernel.py:35-55) mean-relative < 0.02 per tensor, and max |d| / max |ref| < 2e-2
    (the bf16 kernel's); the distance to the exact dequantised values' gradients is printed beside
    (the bf16 rounding of the operands, ~3 % mean-relative on the 450M shape's largest-scale head).
"""

import numpy as np
import pytest
import torch

from gpu_util import rel_errors, to_np, vtile_permute
from oracle.e4m3 import e4m3_to_f32, round_bf16
from oracle.quant import per_tensor_fp8
from oracle.swa_grad import swa_backward, swa_forward_lse

pytestmark = pytest.mark.gpu


def _inputs(B, H, T, D, seed, factor=True):
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(3):
        x = torch.randn(B, H, T, D, generator=g)
        if factor:
            x = x * torch.randn(1, H, 1, 1, generator=g).exp()
        out.append(x.to(torch.bfloat16).cuda())
    return out


def _dequant_oracle(t, gran):
    c, s = per_tensor_fp8(to_np(t), gran)
    return c, s, e4m3_to_f32(c).astype(np.float64) * np.asarray(s, np.float64)


@pytest.mark.parametrize("gran", ["head", "bh", "tensor"])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_dequantiser_matches_oracle_in_both_layouts(gran, D):
    from flower_amd import _lib as L
    from flower_amd.kernels import _per_tensor_fp8, dequantize_e4m3
    B, H, T = 2, 3, 200
    x = _inputs(B, H, T, D, 3 + D)[0]
    codes, scale = _per_tensor_fp8(x, gran)
    c_np = to_np(codes)
    want = e4m3_to_f32(c_np).astype(np.float32) * to_np(scale).reshape(
        (1, 1, 1, 1) if gran == "tensor" else ((1, H, 1, 1) if gran == "head" else (B, H, 1, 1)))
    got = dequantize_e4m3(codes, scale, (B, H, T, D), gran)
    assert np.array_equal(to_np(got).view(np.uint32), round_bf16(want.astype(np.float32)).view(np.uint32))
    got32 = dequantize_e4m3(codes, scale, (B, H, T, D), gran, out_dtype=torch.float32)
    assert np.array_equal(to_np(got32), want.astype(np.float32))
    vt = torch.from_numpy(vtile_permute(c_np)).cuda()
    got_v = dequantize_e4m3(vt, scale, (B, H, T, D), gran, layout="vtile")
    assert torch.equal(got_v, got)
    with pytest.raises(ValueError, match="codes"):
        dequantize_e4m3(vt[:-16], scale, (B, H, T, D), gran, layout="vtile")


def _lse_of(q, k, v, W, gran):
    """The FP8 kernel's output and log-sum-exp through flw_fp8_swa_fwd_lse on the quantiser's codes."""
    from flower_amd import _lib as L
    lib = L.load()
    B, H, T, D = q.shape
    G = {"tensor": 1, "head": H, "bh": B * H}[gran]
    q8 = torch.empty((B, H, T, D), dtype=torch.uint8, device="cuda")
    k8 = torch.empty_like(q8)
    vt = torch.empty(lib.flw_vtile_bytes(B, H, T, D), dtype=torch.uint8, device="cuda")
    sc = torch.empty(3 * G, dtype=torch.float32, device="cuda")
    ws = L.workspace(3 * lib.flw_quant_workspace_bytes(B, H, T, D), q.device)
    st = L.stream_of(q)
    L.check(lib.flw_quant_qkv_e4m3(q.data_ptr(), k.data_ptr(), v.data_ptr(), L.BF16, B, H, T, D,
                                   L.i64s(*q.stride()[:3], *k.stride()[:3], *v.stride()[:3]), L.GRANULARITY[gran],
                                   q8.data_ptr(), k8.data_ptr(), vt.data_ptr(), sc.data_ptr(), ws.data_ptr(),
                                   ws.numel(), st), "quant")
    out = torch.empty((B, H, T, D), dtype=torch.bfloat16, device="cuda")
    lse = torch.full((B, H, T), 7.0, dtype=torch.float32, device="cuda")
    s8 = L.i64s(H * T * D, T * D, D)
    base = sc.data_ptr()
    L.check(lib.flw_fp8_swa_fwd_lse(q8.data_ptr(), s8, k8.data_ptr(), s8, vt.data_ptr(), base, base + 4 * G,
                                    base + 8 * G, L.GRANULARITY[gran], out.data_ptr(), L.BF16,
                                    L.i64s(*out.stride()[:3]), B, H, T, D, W, lse.data_ptr(), st), "fwd lse")
    torch.cuda.synchronize()
    return out, lse


@pytest.mark.parametrize("B,H,T,D,W,gran", [(1, 2, 512, 64, 128, "head"), (2, 2, 300, 32, 64, "bh"),
                                            (1, 2, 257, 128, 1000, "tensor"), (1, 3, 200, 64, 1, "head")])
def test_log_sum_exp_matches_oracle(B, H, T, D, W, gran):
    """The kernel's log-sum-exp against the float64 one of the dequantised scores (q8 s_q . k8 s_k
    / sqrt(D)) over each query's band, W = 1 included (then it is the self score)."""
    from flower_amd.kernels import fp8_swa_attention_forward
    q, k, v = _inputs(B, H, T, D, 11 + D)
    out, lse = _lse_of(q, k, v, W, gran)
    want_out = fp8_swa_attention_forward(q, k, v, W, granularity=gran)
    torch.cuda.synchronize()
    assert torch.equal(out, want_out)           # the LSE output leaves O bit for bit unchanged
    dq = [_dequant_oracle(t, gran)[2] for t in (q, k, v)]
    _, want = swa_forward_lse(*dq, W, chunk=256)
    d = np.abs(to_np(lse).astype(np.float64) - want)
    assert d.max() < 2e-3, float(d.max())


def _grad_case(B, H, T, D, W, gran, seed, slices):
    from flower_amd.kernels import fp8_swa_attention, fp8_swa_attention_forward
    base = _inputs(B, H, T, D, seed)
    g = torch.randn(B, H, T, D, generator=torch.Generator().manual_seed(seed + 1)).to(torch.bfloat16)
    q, k, v = (t.clone().requires_grad_(True) for t in base)
    out = fp8_swa_attention(q, k, v, W, granularity=gran)
    out.backward(g.cuda())
    with torch.no_grad():
        ref_out = fp8_swa_attention_forward(*base, W, granularity=gran)
    torch.cuda.synchronize()
    assert torch.equal(out.detach(), ref_out)
    grads = [t.grad.detach() for t in (q, k, v)]
    for t in grads:
        assert t.dtype == torch.bfloat16 and torch.isfinite(t).all()
    deq = [_dequant_oracle(t, gran)[2] for t in base]
    gn = g.double().numpy()
    for b, h in slices:
        sl = (slice(b, b + 1), slice(h, h + 1))
        # the evaluation point: the dequantised values in bf16 (what the backward runs on, and what
        # `_fake_quant_e4m3` returns in a bf16 model); the exact dequantised values reported beside
        qd, kd, vd = (round_bf16(t[sl].astype(np.float32)).astype(np.float64) for t in deq)
        o, lse = swa_forward_lse(qd, kd, vd, W, chunk=512)
        want = swa_backward(qd, kd, vd, o, lse, gn[sl], W, chunk=512)
        qx, kx, vx = (t[sl] for t in deq)
        ox, lx = swa_forward_lse(qx, kx, vx, W, chunk=512)
        exact = swa_backward(qx, kx, vx, ox, lx, gn[sl], W, chunk=512)
        for name, got, w, wx in zip(("dq", "dk", "dv"), grads, want, exact):
            mx, mean = rel_errors(to_np(got[sl]), w)
            mxx, meanx = rel_errors(to_np(got[sl]), wx)
            print(f"[fp8 train] B{B} H{H} T{T} D{D} W{W} slice ({b}, {h}) {name}: mean-rel {mean:.4f} "
                  f"max-rel {mx:.4f} (at the exact dequantised values: {meanx:.4f} / {mxx:.4f})", flush=True)
            assert mean < 0.02 and mx < 2e-2, (name, b, h, mean, mx)


@pytest.mark.parametrize("B,H,T,D,W,gran", [(1, 2, 256, 64, 128, "head"), (2, 2, 512, 32, 256, "bh"),
                                            (1, 2, 300, 128, 64, "tensor"), (1, 1, 130, 64, 1000, "head")])
def test_gradients_match_the_fake_quant_oracle(B, H, T, D, W, gran):
    _grad_case(B, H, T, D, W, gran, 20 + D + W, [(b, h) for b in range(B) for h in range(H)])


def test_gradients_at_the_450m_shape():
    """B2 H20 T8192 D64 W2048 (the reference's 450M training shape), per-head scales: forward +
    backward through the op; slices (0, 0) and (1, 19) against the oracle."""
    print("[fp8 train] B2 H20 T8192 D64 W2048", flush=True)
    _grad_case(2, 20, 8192, 64, 2048, "head", 450, [(0, 0), (1, 19)])


def test_refusals():
    from flower_amd.kernels import fp8_swa_attention
    q = torch.randn(1, 2, 64, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="window must be positive"):
        fp8_swa_attention(q, q, q, 0)
    with pytest.raises(TypeError):
        fp8_swa_attention(q.half(), q.half(), q.half(), 16)
    with pytest.raises(ValueError, match="head_dim"):
        x = torch.randn(1, 2, 64, 48, device="cuda", dtype=torch.bfloat16)
        fp8_swa_attention(x, x, x, 16)
