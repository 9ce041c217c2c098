"""GPU parity: fused FP8 SWA attention (C ABI via flower_amd) vs the CPU oracle.

Gate (written here, as the tolerance of a floating-point kernel): against the kernel-faithful
FP8 simulator run on the SAME e4m3 codes and scales (which are themselves bit-exact, see
test_gpu_quant.py), max |d| / max |ref| <= 2e-2 and mean |d| / mean |ref| <= 5e-3. The
remaining difference is the exp2-with-folded-scale vs exp rounding, which can move a P value
across an e4m3 rounding boundary, and fp32 summation order.
Against plain fp32 attention the error is reported and bounded by the reference's own measured
FP8 band (mean relative ~0.05, fp8_swa_attention.py:48-57).
"""

import numpy as np
import pytest
import torch

from gpu_util import rel_errors, seeded, to_np
from oracle.quant import per_tensor_fp8
from oracle.swa import fp8_swa_simulate, swa_banded

pytestmark = pytest.mark.gpu

MAX_REL, MEAN_REL = 2e-2, 5e-3
# Rows of a slice that may exceed MAX_REL, each only within the simulator's MFMA allowance (P codes
# within the hardware dot product's error of an e4m3 rounding boundary); see the head_dim 32 / 128 test.
MAX_FLIP_ROWS = 4


def run(q, k, v, W, granularity="tensor"):
    from flower_amd.kernels.fp8_swa_attention import fp8_swa_attention_forward
    out = fp8_swa_attention_forward(q, k, v, W, granularity=granularity)
    torch.cuda.synchronize()
    return out


def oracle(q, k, v, W, granularity="tensor"):
    """Quantise with the oracle (bit-exact with the kernel's quantiser), then simulate."""
    q8, qs = per_tensor_fp8(to_np(q), granularity)
    k8, ks = per_tensor_fp8(to_np(k), granularity)
    v8, vs = per_tensor_fp8(to_np(v), granularity)
    return fp8_swa_simulate(q8, k8, v8, qs, ks, vs, W)


SHAPES = [
    # B, H, T, D, W  -- the reference's test shapes (test_swa_kernel.py:20-32) first
    (1, 2, 256, 64, 128),
    (2, 3, 512, 64, 256),
    (2, 2, 512, 32, 512),
    (1, 2, 200, 128, 77),        # ragged T, odd window
    (1, 1, 64, 64, 1),           # W = 1
    (1, 2, 130, 64, 1000),       # W > T: full causal
    (1, 1, 1, 64, 16),           # T = 1
    (2, 1, 1000, 64, 300),
]


@pytest.mark.parametrize("B,H,T,D,W", SHAPES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_matches_kernel_faithful_simulator(B, H, T, D, W, dtype):
    q, k, v = (seeded((B, H, T, D), s, dtype) for s in (0, 1, 2))
    out = run(q, k, v, W)
    assert out.dtype == dtype and out.shape == q.shape
    ref = oracle(q, k, v, W)
    mx, mean = rel_errors(to_np(out), ref)
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)


@pytest.mark.parametrize("granularity", ["head", "bh"])
def test_per_head_and_per_slice_scales(granularity):
    B, H, T, D, W = 2, 4, 384, 64, 192
    g = torch.Generator().manual_seed(9)
    base = [torch.randn(B, H, T, D, generator=g) * torch.randn(1, H, 1, 1, generator=g).exp() for _ in range(3)]
    q, k, v = (t.to(torch.bfloat16).cuda() for t in base)
    out = run(q, k, v, W, granularity)
    mx, mean = rel_errors(to_np(out), oracle(q, k, v, W, granularity))
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)


def test_config1_cpu_reference_shape_fp32():
    """B1 H8 T1024 D64 W256, fp32 N(0,1), per-tensor scales."""
    q, k, v = (seeded((1, 8, 1024, 64), s, torch.float32) for s in (10, 11, 12))
    out = to_np(run(q, k, v, 256))
    mx, mean = rel_errors(out, oracle(q, k, v, 256))
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)
    # vs the reference's FP8-simulated path (Q, K, V quantised, softmax and P in fp32): the P
    # quantisation's band (the reference measured 0.0261 mean-relative for it at its shape,
    # fp8_swa_attention.py:48-57); max |d| / max |ref| within the 2e-2 the path is held to
    q8, qs = per_tensor_fp8(to_np(q))
    k8, ks = per_tensor_fp8(to_np(k))
    v8, vs = per_tensor_fp8(to_np(v))
    sim_qkv = fp8_swa_simulate(q8, k8, v8, qs, ks, vs, 256, quantize_p=False)
    mx_q, mean_q = rel_errors(out, sim_qkv)
    max_abs_q = float(np.abs(out.astype(np.float64) - sim_qkv).max())
    assert mx_q <= 2e-2 and 0.01 < mean_q < 0.035, (mx_q, mean_q, max_abs_q)
    # vs plain fp32 attention: the reference's measured FP8 band (0.0511 at its shape)
    ref32 = swa_banded(to_np(q), to_np(k), to_np(v), 256)
    _, mean32 = rel_errors(out, ref32)
    assert 0.03 < mean32 < 0.07, mean32


def test_strided_inputs_from_the_model_layout():
    """q/k/v as CausalSelfAttention builds them: view(B, T, H, D).transpose(1, 2)."""
    B, T, H, D, W = 2, 320, 4, 64, 100
    qkv = seeded((B, T, 3 * H * D), 13, torch.bfloat16)
    q, k, v = (t.view(B, T, H, D).transpose(1, 2) for t in qkv.chunk(3, dim=-1))
    assert not q.is_contiguous()
    out = run(q, k, v, W)
    mx, mean = rel_errors(to_np(out), oracle(q.contiguous(), k.contiguous(), v.contiguous(), W))
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)


def test_window_nonpositive_gives_zeros_and_outputs_are_deterministic():
    q, k, v = (seeded((1, 2, 100, 64), s, torch.bfloat16) for s in (14, 15, 16))
    assert torch.count_nonzero(run(q, k, v, 0)) == 0
    a, b = run(q, k, v, 33), run(q, k, v, 33)
    assert torch.equal(a, b)


def test_window_one_returns_dequantised_v():
    q, k, v = (seeded((1, 2, 192, 64), s, torch.float32) for s in (17, 18, 19))
    out = to_np(run(q, k, v, 1))
    v8, vs = per_tensor_fp8(to_np(v))
    from oracle.quant import dequant
    np.testing.assert_allclose(out, dequant(v8, vs), rtol=1e-5, atol=1e-7)


def test_full_size_config3_rows_match_oracle_on_sampled_slices():
    """BASELINE config 3 at full size (B4 H16 T8192 D64 W1024, per-head scales, lognormal heads):
    two (b, h) slices checked against the simulator end to end."""
    B, H, T, D, W = 4, 16, 8192, 64, 1024
    g = torch.Generator().manual_seed(2024)
    mk = lambda: (torch.randn(B, H, T, D, generator=g) * torch.randn(1, H, 1, 1, generator=g).exp()).to(torch.bfloat16)  # noqa: E731
    q, k, v = mk().cuda(), mk().cuda(), mk().cuda()
    out = to_np(run(q, k, v, W, "head"))
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    q8, qs = per_tensor_fp8(qn, "head")
    k8, ks = per_tensor_fp8(kn, "head")
    v8, vs = per_tensor_fp8(vn, "head")
    for b, h in [(0, 0), (3, 11)]:
        ref = fp8_swa_simulate(q8[b:b + 1, h:h + 1], k8[b:b + 1, h:h + 1], v8[b:b + 1, h:h + 1],
                               qs[:, h:h + 1], ks[:, h:h + 1], vs[:, h:h + 1], W, chunk=1024)
        mx, mean = rel_errors(out[b:b + 1, h:h + 1], ref)
        assert mx <= MAX_REL and mean <= MEAN_REL, (b, h, mx, mean)
    assert np.isfinite(out).all()
    _all_slices_checks(q, k, v, W, out)


def test_full_size_config3_fp32_inputs():
    """C3's shape with fp32 Q, K, V (the quantisers' and the Q-on-load fp32 paths at full size):
    one slice against the simulator, every slice bit-identical to the two-pass path."""
    B, H, T, D, W = 4, 16, 8192, 64, 1024
    g = torch.Generator().manual_seed(4032)
    mk = lambda: (torch.randn(B, H, T, D, generator=g) * torch.randn(1, H, 1, 1, generator=g).exp()).cuda()  # noqa: E731
    q, k, v = mk(), mk(), mk()
    got = run(q, k, v, W, "head")
    out = to_np(got)
    q8, qs = per_tensor_fp8(to_np(q), "head")
    k8, ks = per_tensor_fp8(to_np(k), "head")
    v8, vs = per_tensor_fp8(to_np(v), "head")
    b, h = 2, 9
    ref = fp8_swa_simulate(q8[b:b + 1, h:h + 1], k8[b:b + 1, h:h + 1], v8[b:b + 1, h:h + 1],
                           qs[:, h:h + 1], ks[:, h:h + 1], vs[:, h:h + 1], W, chunk=1024)
    mx, mean = rel_errors(out[b:b + 1, h:h + 1], ref)
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)
    assert np.isfinite(out).all()
    want = _two_pass(q, k, v, W, "head")
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


def test_long_ragged_sequence():
    """T = 30001 (not a multiple of the 64-key tile or the 128-query workgroup), W = 4096, eight
    heads (slices split evenly over the XCDs): one slice against the simulator, every slice
    against the two-pass path and under a head reversal."""
    B, H, T, D, W = 1, 8, 30001, 64, 4096
    g = torch.Generator().manual_seed(30001)
    mk = lambda: (torch.randn(B, H, T, D, generator=g) * torch.randn(1, H, 1, 1, generator=g).exp()).to(torch.bfloat16)  # noqa: E731
    q, k, v = mk().cuda(), mk().cuda(), mk().cuda()
    out = to_np(run(q, k, v, W, "head"))
    q8, qs = per_tensor_fp8(to_np(q), "head")
    k8, ks = per_tensor_fp8(to_np(k), "head")
    v8, vs = per_tensor_fp8(to_np(v), "head")
    h = 5
    ref = fp8_swa_simulate(q8[:, h:h + 1], k8[:, h:h + 1], v8[:, h:h + 1], qs[:, h:h + 1], ks[:, h:h + 1],
                           vs[:, h:h + 1], W, chunk=1024)
    mx, mean = rel_errors(out[:, h:h + 1], ref)
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)
    assert np.isfinite(out).all()
    _all_slices_checks(q, k, v, W, out)


def _all_slices_checks(q, k, v, W, out, gran="head"):
    """Every (b, h) slice at full size, without the CPU oracle: the operator equals the explicit
    two-pass path (Q, K, V codes from flw_quant_qkv_e4m3, then flw_fp8_swa_fwd) bit for bit, and
    reversing the heads of q, k, v reverses the heads of the output bit for bit (per-head or
    per-(b, h) scales: no slice's result depends on another slice or on where its workgroups ran)."""
    got = run(q, k, v, W, gran)
    assert np.array_equal(to_np(got), out)                 # the operator is deterministic
    want = _two_pass(q, k, v, W, gran)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    flip = lambda t: t.flip(1).contiguous()  # noqa: E731
    rev = run(flip(q), flip(k), flip(v), W, gran)
    torch.cuda.synchronize()
    assert torch.equal(rev.flip(1).view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("D", [32, 128])
def test_full_size_other_head_dims_match_oracle_on_sampled_slices(D):
    """head_dim 32 and 128 at a long sequence (B2 H4 T8192, W = 1000: not a multiple of 32, so
    the band's partial blocks take the general per-score mask), per-(b, h) scales with lognormal
    per-slice factors: two slices against the simulator, and every slice against the two-pass
    path and under a head reversal.

    The gate is the attention tests' 2e-2 (max |d| / max |ref|), with one MFMA-aware exception:
    the FP8 MFMA's accumulation differs from the simulator's exact dot product by up to 2^-10 of
    the dot's largest product (tests/test_gpu_diag.py), so a P code whose 448 p lies that close to
    an e4m3 rounding boundary may round the other way (at D = 128, slice (1, 3): 448 p = 184.023,
    1.2e-4 above the 176 / 192 boundary, on a key holding 29 % of its row's weight, moves that row
    by 0.0201). The simulator reports, per output element, how far such flips can move it
    (``mfma_rel_err``); an element beyond 2e-2 must lie within 2e-2 plus that allowance, and at
    most MAX_FLIP_ROWS rows of a slice may need it -- a regression that moves many rows fails."""
    B, H, T, W = 2, 4, 8192, 1000
    g = torch.Generator().manual_seed(128 + D)
    mk = lambda: (torch.randn(B, H, T, D, generator=g) * torch.randn(B, H, 1, 1, generator=g).exp()).to(torch.bfloat16)  # noqa: E731
    q, k, v = mk().cuda(), mk().cuda(), mk().cuda()
    out = to_np(run(q, k, v, W, "bh"))
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    q8, qs = per_tensor_fp8(qn, "bh")
    k8, ks = per_tensor_fp8(kn, "bh")
    v8, vs = per_tensor_fp8(vn, "bh")
    for b, h in [(0, 1), (1, 3)]:
        sl = (slice(b, b + 1), slice(h, h + 1))
        ref, allow = fp8_swa_simulate(q8[sl], k8[sl], v8[sl], qs[sl], ks[sl], vs[sl], W, chunk=1024,
                                      mfma_rel_err=2.0 ** -10)
        mx, mean = rel_errors(out[sl], ref)
        tol = MAX_REL * np.abs(ref).max()
        d = np.abs(out[sl].astype(np.float64) - ref)
        beyond = d > tol
        rows = np.unique(np.nonzero(beyond)[2])
        print(f"[attn D{D}] slice ({b}, {h}): max-rel {mx:.4f} mean-rel {mean:.2e}; {beyond.sum()} elements in "
              f"{len(rows)} rows beyond {MAX_REL} (rows {rows.tolist()[:8]})", flush=True)
        assert mean <= MEAN_REL, (D, b, h, mean)
        assert (d[beyond] <= tol + allow[beyond]).all(), (D, b, h, float((d - allow)[beyond].max() / tol))
        assert len(rows) <= MAX_FLIP_ROWS, (D, b, h, rows.tolist())
    assert np.isfinite(out).all()
    _all_slices_checks(q, k, v, W, out, "bh")


def test_full_size_config4_rows_match_oracle_on_sampled_slices():
    """BASELINE config 4 at full size (B1 H16 T32768 D64 W4096, per-head scales; bf16 N(0,1) with
    Student-t (nu = 4) channels in 4 of the 64 dims): two slices against the simulator."""
    B, H, T, D, W = 1, 16, 32768, 64, 4096
    rng = np.random.default_rng(4096)

    def mk():
        x = rng.standard_normal((B, H, T, D), dtype=np.float32)
        x[..., [3, 17, 40, 61]] = rng.standard_t(4, size=(B, H, T, 4)).astype(np.float32)
        return torch.from_numpy(x).to(torch.bfloat16).cuda()

    q, k, v = mk(), mk(), mk()
    out = to_np(run(q, k, v, W, "head"))
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    q8, qs = per_tensor_fp8(qn, "head")
    k8, ks = per_tensor_fp8(kn, "head")
    v8, vs = per_tensor_fp8(vn, "head")
    for h in (0, 13):
        ref = fp8_swa_simulate(q8[:, h:h + 1], k8[:, h:h + 1], v8[:, h:h + 1],
                               qs[:, h:h + 1], ks[:, h:h + 1], vs[:, h:h + 1], W, chunk=1024)
        mx, mean = rel_errors(out[:, h:h + 1], ref)
        assert mx <= MAX_REL and mean <= MEAN_REL, (h, mx, mean)
    assert np.isfinite(out).all()
    _all_slices_checks(q, k, v, W, out)


def test_refuses_grad_tensors():                      # test_swa_kernel.py:68-78
    from flower_amd.kernels.fp8_swa_attention import fp8_swa_attention_forward
    q, k, v = (torch.randn(1, 2, 128, 64, device="cuda", dtype=torch.bfloat16).requires_grad_(True) for _ in range(3))
    with pytest.raises(RuntimeError, match="forward-only"):
        fp8_swa_attention_forward(q, k, v, 64)


def test_rejects_bad_shapes():
    from flower_amd.kernels.fp8_swa_attention import fp8_swa_attention_forward
    with pytest.raises(ValueError, match=r"\(B, H, T, D\)"):
        fp8_swa_attention_forward(*(torch.randn(2, 128, 64, device="cuda") for _ in range(3)), 8)
    with pytest.raises(ValueError, match="head_dim"):
        fp8_swa_attention_forward(*(torch.randn(1, 1, 16, 96, device="cuda") for _ in range(3)), 8)


def test_reference_swa_attention_api_matches_oracle():
    from flower_amd.kernels.fp8_swa_attention import reference_swa_attention
    q, k, v = (seeded((1, 2, 96, 32), s, torch.float32) for s in (20, 21, 22))
    got = to_np(reference_swa_attention(q, k, v, 17))
    from oracle.swa import swa_dense
    np.testing.assert_allclose(got, swa_dense(to_np(q), to_np(k), to_np(v), 17), rtol=1e-4, atol=1e-5)


def test_attention_with_producer_amax_is_identical():
    """fp8_swa_attention_forward(amax=...) with the per-head |q|, |k|, |v| maxima supplied (as the
    QKV GEMM epilogue supplies them) skips the amax pass and returns the same output bit for bit."""
    from flower_amd.kernels.fp8_swa_attention import amax_e4m3, fp8_swa_attention_forward
    g = torch.Generator().manual_seed(21)
    B, H, T, D, W = 2, 4, 300, 64, 96
    q, k, v = (torch.randn(B, H, T, D, generator=g).mul(torch.rand(1, H, 1, 1, generator=g) * 4)
               .to("cuda", torch.bfloat16) for _ in range(3))
    plain = fp8_swa_attention_forward(q, k, v, W, granularity="head")
    amax = torch.cat([t.float().abs().amax(dim=(0, 2, 3)) for t in (q, k, v)]).view(torch.int32).contiguous()
    given = fp8_swa_attention_forward(q, k, v, W, granularity="head", amax=amax)
    # the same maxima as float32 (the dtype amax_e4m3 returns) are accepted too
    amax_f = torch.cat([amax_e4m3(t, "head") for t in (q, k, v)])
    given_f = fp8_swa_attention_forward(q, k, v, W, granularity="head", amax=amax_f)
    torch.cuda.synchronize()
    assert torch.equal(plain, given)
    assert torch.equal(plain, given_f)
    with pytest.raises(ValueError, match="amax"):
        fp8_swa_attention_forward(q, k, v, W, granularity="head", amax=amax[:5])


@pytest.mark.parametrize("gran", ["tensor", "head", "bh"])
def test_scale_strides_entry_matches_the_granularity_entry(gran):
    """flw_fp8_swa_fwd_scale_strides (scales indexed by b * stride_b + h * stride_h, the boundary's
    form): 0/0, 0/1 and H/1 give the granularity entry point's output bit for bit, and per-(b, h)
    scales stored head-major (strides 1/B) give the same output as stored batch-major."""
    from flower_amd import _lib as L
    lib = L.load()
    B, H, T, D, W = 2, 3, 200, 64, 64
    q, k, v = (seeded((B, H, T, D), s, torch.bfloat16) for s in (91, 92, 93))
    G = {"tensor": 1, "head": H, "bh": B * H}[gran]
    q8 = torch.empty((B, H, T, D), dtype=torch.uint8, device="cuda")
    k8 = torch.empty_like(q8)
    vt = torch.empty(lib.flw_vtile_bytes(B, H, T, D), dtype=torch.uint8, device="cuda")
    sc = torch.empty(3 * G, dtype=torch.float32, device="cuda")
    ws = L.workspace(3 * lib.flw_quant_workspace_bytes(B, H, T, D), q.device)
    L.check(lib.flw_quant_qkv_e4m3(q.data_ptr(), k.data_ptr(), v.data_ptr(), L.BF16, B, H, T, D,
                                   L.i64s(*q.stride()[:3], *k.stride()[:3], *v.stride()[:3]), L.GRANULARITY[gran],
                                   q8.data_ptr(), k8.data_ptr(), vt.data_ptr(), sc.data_ptr(), ws.data_ptr(),
                                   ws.numel(), L.stream_of(q)), "quant")
    s8 = L.i64s(H * T * D, T * D, D)
    st = L.stream_of(q)

    def run(scales, ssb, ssh):
        out = torch.empty((B, H, T, D), dtype=torch.bfloat16, device="cuda")
        base = scales.data_ptr()
        n = scales.numel() // 3
        L.check(lib.flw_fp8_swa_fwd_scale_strides(q8.data_ptr(), s8, k8.data_ptr(), s8, vt.data_ptr(), base,
                                                  base + 4 * n, base + 8 * n, ssb, ssh, out.data_ptr(), L.BF16,
                                                  L.i64s(*out.stride()[:3]), B, H, T, D, W, st), "swa")
        return out

    want = torch.empty((B, H, T, D), dtype=torch.bfloat16, device="cuda")
    base = sc.data_ptr()
    L.check(lib.flw_fp8_swa_fwd(q8.data_ptr(), s8, k8.data_ptr(), s8, vt.data_ptr(), base, base + 4 * G,
                                base + 8 * G, L.GRANULARITY[gran], want.data_ptr(), L.BF16,
                                L.i64s(*want.stride()[:3]), B, H, T, D, W, st), "swa")
    ssb, ssh = {"tensor": (0, 0), "head": (0, 1), "bh": (H, 1)}[gran]
    got = run(sc, ssb, ssh)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    if gran == "bh":
        hm = sc.view(3, B, H).transpose(1, 2).contiguous().view(-1)      # [tensor][h][b]
        got_hm = run(hm, 1, B)
        torch.cuda.synchronize()
        assert torch.equal(got_hm.view(torch.int16), want.view(torch.int16))


def _given_amax_two_pass(q, k, v, W, amax_bits):
    """The operator under a given amax as explicit passes: each tensor through flw_quant_e4m3_amax
    (its codes checked against the given maximum, pinned against the oracle in
    tests/test_gpu_quant.py), V into the tile layout, then flw_fp8_swa_fwd on those codes."""
    from flower_amd import _lib as L
    lib = L.load()
    B, H, T, D = q.shape
    G = H
    codes, scales = [], torch.empty(3 * G, dtype=torch.float32, device="cuda")
    for i, (t, layout) in enumerate(((q, L.LAYOUT_BHTD), (k, L.LAYOUT_BHTD), (v, L.LAYOUT_VTILE))):
        n = lib.flw_vtile_bytes(B, H, T, D) if layout == L.LAYOUT_VTILE else B * H * T * D
        c = torch.empty(n, dtype=torch.uint8, device="cuda")
        L.check(lib.flw_quant_e4m3_amax(t.data_ptr(), L.dtype_code(t.dtype), B, H, T, D, *t.stride()[:3],
                                        L.SCALE_HEAD, layout, amax_bits[i * G:].data_ptr(), c.data_ptr(),
                                        scales[i * G:].data_ptr(), L.stream_of(t)), "quant")
        codes.append(c)
    out = torch.empty((B, H, T, D), dtype=q.dtype, device="cuda")
    s8 = L.i64s(H * T * D, T * D, D)
    base = scales.data_ptr()
    L.check(lib.flw_fp8_swa_fwd(codes[0].data_ptr(), s8, codes[1].data_ptr(), s8, codes[2].data_ptr(), base,
                                base + 4 * G, base + 8 * G, L.SCALE_HEAD, out.data_ptr(), L.dtype_code(q.dtype),
                                L.i64s(*out.stride()[:3]), B, H, T, D, W, L.stream_of(q)), "swa")
    return out


@pytest.mark.parametrize("factor", [0.5, 1.0, -1.0])
def test_q_on_load_under_a_given_amax_checks_it_like_the_quantiser(factor):
    """With a producer amax, fp8_swa_attention_forward quantises Q inside the attention kernel and
    checks every lane's values against the given maximum: with the maximum at 0.5x, 1x or -1x the
    data's own and inf / -inf / NaN / 1e30 planted in Q, the lanes beyond it take the exact path
    (IEEE division, clamp to +-448, the cast), so the output equals the attention over the
    given-amax quantiser's codes bit for bit."""
    from flower_amd.kernels.fp8_swa_attention import fp8_swa_attention_forward
    g = torch.Generator().manual_seed(31)
    B, H, T, D, W = 2, 4, 300, 64, 96
    q, k, v = (torch.randn(B, H, T, D, generator=g).mul(torch.rand(1, H, 1, 1, generator=g) * 4 + 0.5)
               .to(torch.bfloat16) for _ in range(3))
    amax = torch.cat([t.float().abs().amax(dim=(0, 2, 3)) for t in (q, k, v)]) * factor
    q[0, 1, 5, :4] = torch.tensor([float("inf"), float("-inf"), float("nan"), 1e30]).to(torch.bfloat16)
    q[1, 2, 7, 9] = 1e30
    q, k, v = q.cuda(), k.cuda(), v.cuda()
    bits = amax.cuda().contiguous().view(torch.int32)
    print(f"[amax-q-on-load] factor {factor}", flush=True)
    got = fp8_swa_attention_forward(q, k, v, W, granularity="head", amax=bits)
    want = _given_amax_two_pass(q, k, v, W, bits)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    if factor == 1.0:
        # rows that saw no planted value are finite; the planted rows carry the NaN / saturation
        assert bool(torch.isfinite(got[1, 0]).all())


def _two_pass(q, k, v, W, gran):
    """The operator as two explicit passes: flw_quant_qkv_e4m3 (Q, K, V codes) then
    flw_fp8_swa_fwd on those codes -- the path before Q was quantised on load."""
    from flower_amd import _lib as L
    lib = L.load()
    B, H, T, D = q.shape
    G = {"tensor": 1, "head": H, "bh": B * H}[gran]
    q8 = torch.empty((B, H, T, D), dtype=torch.uint8, device="cuda")
    k8 = torch.empty_like(q8)
    vt = torch.empty(lib.flw_vtile_bytes(B, H, T, D), dtype=torch.uint8, device="cuda")
    sc = torch.empty(3 * G, dtype=torch.float32, device="cuda")
    ws = L.workspace(3 * lib.flw_quant_workspace_bytes(B, H, T, D), q.device)
    L.check(lib.flw_quant_qkv_e4m3(q.data_ptr(), k.data_ptr(), v.data_ptr(), L.dtype_code(q.dtype), B, H, T, D,
                                   L.i64s(*q.stride()[:3], *k.stride()[:3], *v.stride()[:3]), L.GRANULARITY[gran],
                                   q8.data_ptr(), k8.data_ptr(), vt.data_ptr(), sc.data_ptr(), ws.data_ptr(),
                                   ws.numel(), L.stream_of(q)), "quant")
    out = torch.empty((B, H, T, D), dtype=q.dtype, device="cuda")
    s8 = L.i64s(H * T * D, T * D, D)
    base = sc.data_ptr()
    L.check(lib.flw_fp8_swa_fwd(q8.data_ptr(), s8, k8.data_ptr(), s8, vt.data_ptr(), base, base + 4 * G,
                                base + 8 * G, L.GRANULARITY[gran], out.data_ptr(), L.dtype_code(q.dtype),
                                L.i64s(*out.stride()[:3]), B, H, T, D, W, L.stream_of(q)), "swa")
    return out


@pytest.mark.parametrize("gran", ["tensor", "head", "bh"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_q_quantised_on_load_is_bit_identical_to_the_two_pass_path(D, dtype, gran):
    """fp8_swa_attention_forward quantises Q inside the attention kernel (flw_quant_qkv_e4m3_deferq +
    flw_fp8_swa_fwd_qx); with near-tie Q values (quotients within ulps of an e4m3 rounding midpoint)
    and strided Q, its output equals the two-pass path's bit for bit."""
    from test_oracle_quant import near_tie_input
    from flower_amd.kernels.fp8_swa_attention import fp8_swa_attention_forward
    B, H, T, W = 2, 3, 333, 100
    # heads scaled by powers of two: a head's quotients x / s are unchanged, so they stay near ties
    qn = near_tie_input((B, T, H, D), 81) * (2.0 ** np.arange(H, dtype=np.float32))[None, None, :, None]
    q = torch.from_numpy(qn).to(dtype).cuda().transpose(1, 2)          # (B, H, T, D) view, strided
    k, v = (seeded((B, H, T, D), s, dtype) for s in (82, 83))
    got = fp8_swa_attention_forward(q, k, v, W, granularity=gran)
    want = _two_pass(q, k, v, W, gran)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_q_on_load_leaves_non_finite_groups_to_the_quantiser():
    """A NaN in one head of Q (per-head scales): that group's codes come from the quantiser's exact
    path, the other heads' from the attention kernel's quantise-on-load; the output equals the
    two-pass path bit for bit (NaN rows in that head included) and an inf head too."""
    from flower_amd.kernels.fp8_swa_attention import fp8_swa_attention_forward
    B, H, T, D, W = 1, 4, 256, 64, 64
    q, k, v = (seeded((B, H, T, D), s, torch.bfloat16) for s in (84, 85, 86))
    q[0, 1, 17, 5] = float("nan")
    q[0, 2, 100, 0] = float("inf")
    got = fp8_swa_attention_forward(q, k, v, W, granularity="head")
    want = _two_pass(q, k, v, W, "head")
    torch.cuda.synchronize()
    assert torch.isnan(got[0, 1]).all()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("D,T", [(64, 300), (32, 64), (128, 130)])
def test_attention_from_bhtd_codes(D, T):
    """V codes in plain (B, H, T, D) layout (what _per_tensor_fp8 returns) reach the kernel through
    flw_vtile_from_bhtd: the permuted bytes equal the layout's definition (gpu_util.vtile_permute,
    keys past T zero), and attention on _per_tensor_fp8's own codes equals the fused operator."""
    from flower_amd import _lib as L
    from flower_amd.kernels.fp8_swa_attention import (_per_tensor_fp8, fp8_swa_attention_forward,
                                                      fp8_swa_attention_from_codes)
    from gpu_util import vtile_permute
    lib = L.load()
    B, H, W = 2, 3, 77
    q, k, v = (seeded((B, H, T, D), s, torch.bfloat16) for s in (87, 88, 89))
    codes = [_per_tensor_fp8(t, "head") for t in (q, k, v)]
    v8 = codes[2][0].view(torch.uint8)
    vt = torch.full((lib.flw_vtile_bytes(B, H, T, D),), 0x5A, dtype=torch.uint8, device="cuda")
    L.check(lib.flw_vtile_from_bhtd(v8.data_ptr(), B, H, T, D, *v8.stride()[:3], vt.data_ptr(),
                                    L.stream_of(v8)), "permute")
    scales = torch.cat([c[1] for c in codes])
    got = fp8_swa_attention_from_codes(codes[0][0], codes[1][0], codes[2][0], scales, W, granularity="head")
    want = fp8_swa_attention_forward(q, k, v, W, granularity="head")
    torch.cuda.synchronize()
    assert np.array_equal(to_np(vt), vtile_permute(to_np(v8)))
    assert torch.equal(got, want)


@pytest.mark.parametrize("D,T,gran", [(64, 300, "head"), (32, 64, "tensor"), (128, 130, "bh"), (64, 8192, "bh")])
def test_bhtd_v_entry_is_bit_identical_to_the_tiled_v_entry(D, T, gran):
    """flw_fp8_swa_fwd_bhtd (V as (B, H, T, D) codes, staged into the tile layout by the kernel)
    against flw_fp8_swa_fwd on flw_vtile_from_bhtd of the same codes: bit for bit, with V read
    through the model's (B, T, H, D) layout as a strided view (rows past T are the padding keys),
    the scales through the granularity's element strides, bf16 and fp32 outputs."""
    from flower_amd import _lib as L
    from flower_amd.kernels.fp8_swa_attention import _per_tensor_fp8
    lib = L.load()
    B, H, W = 2, 3, 77 if T < 8192 else 1024
    q, k = (seeded((B, H, T, D), s, torch.bfloat16) for s in (91, 92))
    v = seeded((B, H, T, D), 93, torch.bfloat16)
    (q8, qs), (k8, ks), (v8c, vs) = (_per_tensor_fp8(t, gran) for t in (q, k, v))
    q8, k8 = q8.view(torch.uint8), k8.view(torch.uint8)
    vbuf = torch.empty((B, T, H, D), dtype=torch.uint8, device="cuda")    # the model's layout
    vbuf.copy_(v8c.view(torch.uint8).transpose(1, 2))
    v8 = vbuf.transpose(1, 2)                                   # (B, H, T, D) view, strides (THD, D, HD)
    assert not v8.is_contiguous() and v8.stride()[:3] == (T * H * D, D, H * D)
    vt = torch.empty(lib.flw_vtile_bytes(B, H, T, D), dtype=torch.uint8, device="cuda")
    L.check(lib.flw_vtile_from_bhtd(v8.data_ptr(), B, H, T, D, *v8.stride()[:3], vt.data_ptr(), L.stream_of(v8)),
            "permute")
    ssb, ssh = {"tensor": (0, 0), "head": (0, 1), "bh": (H, 1)}[gran]
    s8, sk, sv = (L.i64s(*t.stride()[:3]) for t in (q8, k8, v8))
    for dt in (torch.bfloat16, torch.float32):
        want = torch.empty((B, H, T, D), dtype=dt, device="cuda")
        got = torch.full_like(want, float("nan"))
        so = L.i64s(*want.stride()[:3])
        L.check(lib.flw_fp8_swa_fwd_scale_strides(q8.data_ptr(), s8, k8.data_ptr(), sk, vt.data_ptr(), qs.data_ptr(),
                                                  ks.data_ptr(), vs.data_ptr(), ssb, ssh, want.data_ptr(),
                                                  L.dtype_code(dt), so, B, H, T, D, W, L.stream_of(q8)), "tiled")
        L.check(lib.flw_fp8_swa_fwd_bhtd(q8.data_ptr(), s8, k8.data_ptr(), sk, v8.data_ptr(), sv, qs.data_ptr(),
                                         ks.data_ptr(), vs.data_ptr(), ssb, ssh, got.data_ptr(), L.dtype_code(dt), so,
                                         B, H, T, D, W, L.stream_of(q8)), "bhtd")
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16 if dt == torch.bfloat16 else torch.int32),
                           want.view(torch.int16 if dt == torch.bfloat16 else torch.int32)), (D, T, gran, dt)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_small_and_large_grid_kernels_agree_bit_for_bit(dtype):
    """A slice's output does not depend on the grid it runs in (dispatch order, XCD grouping, the
    ramp-last tile order): the same (b, h) slices run in a small grid (2 heads) and inside a large
    one (the heads repeated 200 times, per-head scales so every copy gets the same scale) give
    identical outputs."""
    from flower_amd.kernels.fp8_swa_attention import fp8_swa_attention_forward
    q, k, v = (seeded((1, 2, 1024, 64), s, dtype) for s in (90, 91, 92))
    small = fp8_swa_attention_forward(q, k, v, 300, granularity="head")
    big = fp8_swa_attention_forward(*(t.repeat(1, 200, 1, 1) for t in (q, k, v)), 300, granularity="head")
    torch.cuda.synchronize()
    for r in (0, 57, 199):
        assert torch.equal(big[:, 2 * r:2 * r + 2], small), r
