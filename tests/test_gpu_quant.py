"""GPU parity: e4m3 quantisers (C ABI via flower_amd) vs the CPU oracle, bit-exact."""

import ctypes

import numpy as np
import pytest
import torch

from gpu_util import seeded, to_np, vtile_permute
from oracle.e4m3 import f32_to_e4m3
from oracle.quant import fake_quant_e4m3, per_tensor_fp8, rowwise_fp8

pytestmark = pytest.mark.gpu


def lib():
    from flower_amd import _lib
    return _lib


def near_ties(shape, seed, amax=3.0):
    from test_oracle_quant import near_tie_input
    return torch.from_numpy(near_tie_input(shape, seed, amax))


# ------------------------------------------------------------------ the hardware P conversion

def test_hw_fp8_convert_is_exact_on_the_attention_P_range():
    """v_cvt_pk_fp8_f32 (used for P * 448 in the attention kernel) against the library's exact
    rounding, on EVERY fp32 value in [0, 448 * (1 + 2^-20)], compared on the device."""
    L = lib()
    lb = L.load_diag()
    hi = int(np.array([448.0], np.float32).view(np.int32)[0]) + 16
    chunk = 1 << 26
    bad = 0
    for start in range(0, hi + 1, chunk):
        n = min(chunk, hi + 1 - start)
        n += n % 2
        x = torch.arange(start, start + n, dtype=torch.int64, device="cuda").to(torch.int32).view(torch.float32)
        hw = torch.empty(n, dtype=torch.uint8, device="cuda")
        sw = torch.empty(n, dtype=torch.uint8, device="cuda")
        s = L.stream_of(x)
        L.check(lb.flw_diag_cvt_e4m3(x.data_ptr(), hw.data_ptr(), n, 1, s), "hw", lb)
        L.check(lb.flw_diag_cvt_e4m3(x.data_ptr(), sw.data_ptr(), n, 0, s), "sw", lb)
        bad += int((hw != sw).sum())
    assert bad == 0, f"{bad} hardware conversions differ from exact RNE"


def test_hw_fp8_convert_is_exact_on_negative_quantiser_range():
    """The quantisers feed v_cvt_pk_fp8_f32 quotients in [-448 (1 + 2^-20), 448 (1 + 2^-20)]:
    the negative half, EVERY fp32 value, against the exact rounding."""
    L = lib()
    lb = L.load_diag()
    hi = int(np.array([448.0], np.float32).view(np.int32)[0]) + 16
    chunk = 1 << 26
    bad = 0
    for start in range(0, hi + 1, chunk):
        n = min(chunk, hi + 1 - start)
        n += n % 2
        u = torch.arange(start, start + n, dtype=torch.int64, device="cuda") | (1 << 31)
        x = u.to(torch.int32).view(torch.float32)          # sign bit set: -|x|
        hw = torch.empty(n, dtype=torch.uint8, device="cuda")
        sw = torch.empty(n, dtype=torch.uint8, device="cuda")
        s = L.stream_of(x)
        L.check(lb.flw_diag_cvt_e4m3(x.data_ptr(), hw.data_ptr(), n, 1, s), "hw", lb)
        L.check(lb.flw_diag_cvt_e4m3(x.data_ptr(), sw.data_ptr(), n, 0, s), "sw", lb)
        bad += int((hw != sw).sum())
    assert bad == 0, f"{bad} hardware conversions differ from exact RNE"


def _quotients(x, scales, mode):
    L = lib()
    lb = L.load_diag()
    xt = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    st = torch.from_numpy(np.ascontiguousarray(scales, np.float32)).cuda()
    out = torch.empty(x.size * scales.size, dtype=torch.int32, device="cuda")
    L.check(lb.flw_diag_quotient(xt.data_ptr(), x.size, st.data_ptr(), scales.size, out.data_ptr(),
                                 mode, L.stream_of(xt)), "quotient", lb)
    return out


def _scale_set(seed=0):
    """Scales the quantisers form: max(amax, 1e-12) / 448 for random and adversarial amax
    (all-ones and all-zeros mantissas, powers of two, tiny, huge), plus raw random mantissas."""
    rng = np.random.default_rng(seed)
    amax = np.concatenate([
        rng.standard_normal(700).astype(np.float32) ** 2 * 10,
        np.exp(rng.uniform(-30, 30, 300)).astype(np.float32),
        np.array([1.0, 2.0, 448.0, 3.0, 1e-12, 1e-30, 3e38, 65504.0], np.float32),
        (np.uint32(0x3FFFFFFF) - np.arange(32, dtype=np.uint32)).view(np.float32),   # 1.999..
        (np.uint32(0x3F800000) + np.arange(32, dtype=np.uint32)).view(np.float32),   # 1.000..
    ])
    s = (np.maximum(amax, np.float32(1e-12)) / np.float32(448.0)).astype(np.float32)
    raw = ((rng.integers(0, 1 << 23, 256, dtype=np.uint32)) | np.uint32(0x3F800000)).view(np.float32)
    return np.concatenate([s, raw]).astype(np.float32)


def test_reciprocal_correction_equals_ieee_division_on_every_bf16_input():
    """The quantisers' x / s (RN(1/s), one product, two FMAs) is the IEEE quotient bit for bit,
    for all 65,536 bf16 values x against ~1,300 scales, wherever |x / s| <= 2^9 (the quantiser
    never sees larger quotients: |x| <= amax and s >= amax / 448)."""
    bits = np.arange(1 << 16, dtype=np.uint32) << 16
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    scales = _scale_set()
    for lo in range(0, scales.size, 256):
        sc = scales[lo:lo + 256]
        ref = _quotients(x, sc, 0)
        got = _quotients(x, sc, 1)
        _check_quotients(ref, got, f"scales {lo}..{lo + sc.size}")


def _check_quotients(ref, got, what):
    """Bit-identical where 2^-20 <= |q| <= 2^9; below 2^-20 (an e4m3 zero) the sign must agree."""
    q = ref.view(torch.float32).abs()
    inside = q <= 512.0
    exact = inside & (q >= 2.0 ** -20)
    bad = int(((ref != got) & exact).sum())
    assert bad == 0, f"{bad} quotients differ ({what})"
    sign_bad = int((((ref ^ got) < 0) & inside).sum())
    assert sign_bad == 0, f"{sign_bad} quotient signs differ ({what})"


def test_reciprocal_correction_equals_ieee_division_on_random_fp32():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(1 << 18) * np.exp(rng.uniform(-20, 20, 1 << 18))).astype(np.float32)
    scales = _scale_set(2)[::5]
    x[:64] = np.float32(-0.0)
    ref = _quotients(x, scales, 0)
    got = _quotients(x, scales, 1)
    _check_quotients(ref, got, "random fp32")


def test_device_exact_rounding_matches_oracle():
    """The device's software e4m3 rounding (used by the quantisers) vs the oracle, on random
    bit patterns, every e4m3 midpoint +-4 ulp, NaN and inf."""
    L = lib()
    lb = L.load_diag()
    from test_oracle_e4m3 import _boundaries
    pts = _boundaries()
    u = pts.view(np.int32).astype(np.int64)
    cand = (u[:, None] + np.arange(-4, 5)[None, :]).reshape(-1)
    cand = cand[(cand >= -(2 ** 31)) & (cand < 2 ** 31)].astype(np.int32).view(np.float32)
    rnd = np.random.default_rng(0).integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([cand, rnd, np.array([np.nan, -np.nan, np.inf, -np.inf], np.float32)])
    xt = torch.from_numpy(x).cuda()
    out = torch.empty(x.size, dtype=torch.uint8, device="cuda")
    L.check(lb.flw_diag_cvt_e4m3(xt.data_ptr(), out.data_ptr(), x.size, 0, L.stream_of(xt)), "sw", lb)
    np.testing.assert_array_equal(out.cpu().numpy(), f32_to_e4m3(x))


# ------------------------------------------------------------------ _per_tensor_fp8

CASES = [
    # (shape, dtype, maker)
    ((2, 4, 256, 64), torch.float32, "randn"),
    ((2, 4, 256, 64), torch.bfloat16, "randn"),
    ((1, 8, 1024, 64), torch.float32, "randn"),          # BASELINE config 1 shape
    ((2, 3, 100, 32), torch.bfloat16, "randn"),          # ragged T
    ((2, 4, 64, 32), torch.float32, "ties"),
    ((2, 4, 64, 32), torch.float32, "zeros"),
    ((1, 2, 300, 128), torch.bfloat16, "lognormal_heads"),
    ((3, 5, 257, 64), torch.float32, "tiny"),
]


def make(shape, dtype, kind, seed=0):
    if kind == "randn":
        x = seeded(shape, seed, torch.float32, "cpu")
    elif kind == "ties":
        x = near_ties(shape, seed)
    elif kind == "zeros":
        x = torch.zeros(shape)
    elif kind == "lognormal_heads":
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(*shape, generator=g) * torch.randn(1, shape[1], 1, 1, generator=g).exp()
    elif kind == "tiny":
        x = seeded(shape, seed, torch.float32, "cpu") * 1e-30
        x.view(-1)[::7] = -0.0                                  # the sign of zero is kept
    else:
        raise ValueError(kind)
    return x.to(dtype).cuda()


@pytest.mark.parametrize("shape,dtype,kind", CASES)
@pytest.mark.parametrize("granularity", ["tensor", "head", "bh"])
def test_per_tensor_fp8_codes_and_scales_bit_exact(shape, dtype, kind, granularity):
    from flower_amd.kernels.fp8_swa_attention import _per_tensor_fp8
    x = make(shape, dtype, kind)
    q8, scale = _per_tensor_fp8(x, granularity)
    torch.cuda.synchronize()
    want_codes, want_scale = per_tensor_fp8(to_np(x), granularity)
    np.testing.assert_array_equal(to_np(q8), want_codes)
    np.testing.assert_array_equal(to_np(scale).view(np.uint32), want_scale.reshape(-1).view(np.uint32))


def test_per_tensor_fp8_strided_input():
    """q as the model produces it: x.view(B, T, H, D).transpose(1, 2) (base.py:612-614)."""
    from flower_amd.kernels.fp8_swa_attention import _per_tensor_fp8
    B, T, H, D = 2, 192, 4, 64
    x = seeded((B, T, H * D), 3, torch.bfloat16).view(B, T, H, D).transpose(1, 2)
    assert not x.is_contiguous()
    q8, scale = _per_tensor_fp8(x, "head")
    want_codes, want_scale = per_tensor_fp8(to_np(x.contiguous()), "head")
    np.testing.assert_array_equal(to_np(q8), want_codes)
    np.testing.assert_array_equal(to_np(scale), want_scale.reshape(-1))


def test_nan_input_gives_nan_scale_and_codes_like_the_reference():
    from flower_amd.kernels.fp8_swa_attention import _per_tensor_fp8
    x = seeded((1, 2, 64, 32), 4, torch.float32, "cpu")
    x[0, 1, 5, 7] = float("nan")
    q8, scale = _per_tensor_fp8(x.cuda(), "head")
    want_codes, want_scale = per_tensor_fp8(x.numpy(), "head")
    np.testing.assert_array_equal(to_np(q8), want_codes)
    s = to_np(scale)
    assert np.isnan(s[1]) and s[0] == want_scale.reshape(-1)[0]


@pytest.mark.parametrize("shape,dtype", [((2, 3, 100, 64), torch.bfloat16), ((1, 2, 64, 32), torch.float32),
                                         ((1, 1, 257, 128), torch.bfloat16), ((1, 2, 1, 64), torch.bfloat16),
                                         ((2, 1, 129, 32), torch.bfloat16), ((1, 1, 200, 128), torch.float32),
                                         ((1, 3, 63, 64), torch.float32)])
def test_vtile_layout_is_the_documented_permutation(shape, dtype):
    L = lib()
    lb = L.load()
    x = make(shape, dtype, "randn", seed=5)
    B, H, T, D = shape
    out = torch.empty(lb.flw_vtile_bytes(B, H, T, D), dtype=torch.uint8, device="cuda")
    sc = torch.empty(H, dtype=torch.float32, device="cuda")
    ws = L.workspace(lb.flw_quant_workspace_bytes(B, H, T, D), "cuda")
    sb, sh, st, _ = x.stride()
    L.check(lb.flw_quant_e4m3(x.data_ptr(), L.dtype_code(dtype), B, H, T, D, sb, sh, st, L.SCALE_HEAD,
                              L.LAYOUT_VTILE, out.data_ptr(), sc.data_ptr(), ws.data_ptr(), ws.numel(),
                              L.stream_of(x)), "vtile")
    want_codes, want_scale = per_tensor_fp8(to_np(x), "head")
    np.testing.assert_array_equal(out.cpu().numpy(), vtile_permute(want_codes))
    np.testing.assert_array_equal(to_np(sc), want_scale.reshape(-1))


@pytest.mark.parametrize("granularity", ["tensor", "head", "bh"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_qkv_entry_point_bit_exact(granularity, dtype):
    """flw_quant_qkv_e4m3: Q, K codes (BHTD), V codes (VTILE) and all scales in one call."""
    L = lib()
    lb = L.load()
    B, H, T, D = 2, 3, 200, 64
    xs = [make((B, H, T, D), dtype, kind, seed=s) for s, kind in ((7, "randn"), (8, "ties"), (9, "lognormal_heads"))]
    G = {"tensor": 1, "head": H, "bh": B * H}[granularity]
    q8 = torch.empty((B, H, T, D), dtype=torch.uint8, device="cuda")
    k8 = torch.empty_like(q8)
    vt = torch.empty(lb.flw_vtile_bytes(B, H, T, D), dtype=torch.uint8, device="cuda")
    sc = torch.empty(3 * G, dtype=torch.float32, device="cuda")
    ws = L.workspace(3 * lb.flw_quant_workspace_bytes(B, H, T, D), "cuda")
    strides = L.i64s(*xs[0].stride()[:3], *xs[1].stride()[:3], *xs[2].stride()[:3])
    L.check(lb.flw_quant_qkv_e4m3(xs[0].data_ptr(), xs[1].data_ptr(), xs[2].data_ptr(), L.dtype_code(dtype),
                                  B, H, T, D, strides, L.GRANULARITY[granularity], q8.data_ptr(),
                                  k8.data_ptr(), vt.data_ptr(), sc.data_ptr(), ws.data_ptr(), ws.numel(),
                                  L.stream_of(q8)), "qkv")
    want = [per_tensor_fp8(to_np(x), granularity) for x in xs]
    np.testing.assert_array_equal(q8.cpu().numpy(), want[0][0])
    np.testing.assert_array_equal(k8.cpu().numpy(), want[1][0])
    np.testing.assert_array_equal(vt.cpu().numpy(), vtile_permute(want[2][0]))
    got_sc = to_np(sc).view(np.uint32)
    for i in range(3):
        np.testing.assert_array_equal(got_sc[i * G:(i + 1) * G], want[i][1].reshape(-1).view(np.uint32))


def run_qkv(xs, granularity):
    """flw_quant_qkv_e4m3 on the three tensors; returns (q8, k8, vtiles, scales)."""
    L = lib()
    lb = L.load()
    B, H, T, D = xs[0].shape
    G = {"tensor": 1, "head": H, "bh": B * H}[granularity]
    q8 = torch.empty((B, H, T, D), dtype=torch.uint8, device="cuda")
    k8 = torch.empty_like(q8)
    vt = torch.empty(lb.flw_vtile_bytes(B, H, T, D), dtype=torch.uint8, device="cuda")
    sc = torch.empty(3 * G, dtype=torch.float32, device="cuda")
    ws = L.workspace(3 * lb.flw_quant_workspace_bytes(B, H, T, D), "cuda")
    strides = L.i64s(*xs[0].stride()[:3], *xs[1].stride()[:3], *xs[2].stride()[:3])
    L.check(lb.flw_quant_qkv_e4m3(xs[0].data_ptr(), xs[1].data_ptr(), xs[2].data_ptr(),
                                  L.dtype_code(xs[0].dtype), B, H, T, D, strides,
                                  L.GRANULARITY[granularity], q8.data_ptr(), k8.data_ptr(),
                                  vt.data_ptr(), sc.data_ptr(), ws.data_ptr(), ws.numel(),
                                  L.stream_of(q8)), "qkv")
    torch.cuda.synchronize()
    return q8, k8, vt, sc


def check_qkv_against_oracle(xs, granularity, got):
    q8, k8, vt, sc = got
    G = sc.numel() // 3
    want = [per_tensor_fp8(to_np(x), granularity) for x in xs]
    np.testing.assert_array_equal(q8.cpu().numpy(), want[0][0])
    np.testing.assert_array_equal(k8.cpu().numpy(), want[1][0])
    np.testing.assert_array_equal(vt.cpu().numpy(), vtile_permute(want[2][0]))
    got_sc = to_np(sc).view(np.uint32)
    for i in range(3):
        np.testing.assert_array_equal(got_sc[i * G:(i + 1) * G], want[i][1].reshape(-1).view(np.uint32))


def test_qkv_large_shape_repeated():
    """A 21 M-element-per-tensor call (2 x 4 x 40960 x 64, per head) against the oracle, then five
    more calls that must give the same bytes."""
    shape = (2, 4, 40960, 64)
    xs = [make(shape, torch.bfloat16, "lognormal_heads", seed=s) for s in (21, 22, 23)]
    first = run_qkv(xs, "head")
    check_qkv_against_oracle(xs, "head", first)
    ref = torch.cat([t.view(torch.uint8).reshape(-1) for t in first])
    for _ in range(5):
        again = run_qkv(xs, "head")
        assert torch.equal(torch.cat([t.view(torch.uint8).reshape(-1) for t in again]), ref)


def test_qkv_nan_group_and_strided_views():
    """A NaN in one head makes that head's scale and codes NaN exactly as the reference does; the
    inputs are the strided head views of a packed qkv projection (read in place)."""
    B, T, H, D = 2, 512, 4, 64
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(B, T, 3 * H * D, generator=g).to(torch.bfloat16)
    qkv[1, 17, H * D + 2 * D + 5] = float("nan")            # K, head 2
    qkv = qkv.cuda()
    xs = [t.view(B, T, H, D).transpose(1, 2) for t in qkv.chunk(3, dim=-1)]
    assert not xs[0].is_contiguous()
    got = run_qkv(xs, "head")
    check_qkv_against_oracle(xs, "head", got)
    assert np.isnan(to_np(got[3])[H + 2]) and not np.isnan(to_np(got[3])[H + 1])


def test_timing_hook_brackets_one_entry_point_call():
    """flw_time_next_launch: the quantiser pair records the armed events from its own dispatches
    (start with the first kernel, stop with the last), computes the same codes, and disarms."""
    L = lib()
    lb = L.load()
    B, H, T, D = 1, 2, 512, 64
    xs = [make((B, H, T, D), torch.bfloat16, "randn", seed=s) for s in (1, 2, 3)]
    outs = []
    for timed in (False, True):
        q8 = torch.empty((B, H, T, D), dtype=torch.uint8, device="cuda")
        k8 = torch.empty_like(q8)
        vt = torch.empty(lb.flw_vtile_bytes(B, H, T, D), dtype=torch.uint8, device="cuda")
        sc = torch.empty(3 * H, dtype=torch.float32, device="cuda")
        ws = L.workspace(3 * lb.flw_quant_workspace_bytes(B, H, T, D), "cuda")
        strides = L.i64s(*xs[0].stride()[:3], *xs[1].stride()[:3], *xs[2].stride()[:3])
        if timed:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            b.record()
            torch.cuda.synchronize()
            L.check(lb.flw_time_next_launch(a.cuda_event, b.cuda_event), "arm")
        for _ in range(2):              # the second call runs untimed: the hook is consumed
            L.check(lb.flw_quant_qkv_e4m3(xs[0].data_ptr(), xs[1].data_ptr(), xs[2].data_ptr(), L.BF16,
                                          B, H, T, D, strides, L.SCALE_HEAD, q8.data_ptr(), k8.data_ptr(),
                                          vt.data_ptr(), sc.data_ptr(), ws.data_ptr(), ws.numel(),
                                          L.stream_of(q8)), "qkv")
        torch.cuda.synchronize()
        outs.append(torch.cat([q8.view(-1), k8.view(-1), vt.view(-1), sc.view(torch.uint8)]))
        if timed:
            ms = a.elapsed_time(b)
            assert 0.0 < ms < 1000.0, ms
    assert torch.equal(outs[0], outs[1])
    assert lb.flw_time_next_launch(None, None) == 0
    x = torch.cuda.Event(enable_timing=True)
    x.record()
    assert lb.flw_time_next_launch(x.cuda_event, None) == 1      # both or neither


# ------------------------------------------------------------------ _fake_quant_e4m3

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kind", ["randn", "ties", "zeros", "tiny"])
def test_fake_quant_matches_reference_sequence_bit_exact(dtype, kind):
    from flower_amd.attention import _fake_quant_e4m3
    x = make((2, 2, 96, 64), dtype, kind, seed=6)
    y = _fake_quant_e4m3(x)
    want, _, _ = fake_quant_e4m3(to_np(x), "f32" if dtype == torch.float32 else "bf16")
    assert y.dtype == dtype and y.shape == x.shape
    np.testing.assert_array_equal(to_np(y).view(np.uint32), want.view(np.uint32))


def test_fake_quant_gradient_passes_straight_through():      # test_fp8_attention_sim.py:40-52
    from flower_amd.attention import _fake_quant_e4m3
    x = seeded((2, 2, 8, 16), 0).requires_grad_(True)
    y = _fake_quant_e4m3(x)
    g = seeded((2, 2, 8, 16), 1)
    y.backward(g)
    assert torch.equal(x.grad, g)


def test_fake_quant_is_actually_quantized_and_zero_safe():     # :23-29, :69-74
    from flower_amd.attention import _fake_quant_e4m3
    x = seeded((2, 2, 32, 16), 0) * 0.5
    y = _fake_quant_e4m3(x)
    assert not torch.equal(y, x) and (y - x).abs().mean() > 0
    z = torch.zeros(2, 2, 8, 16, device="cuda")
    assert torch.equal(_fake_quant_e4m3(z), z)


# ------------------------------------------------------------------ per-row (GEMM / weight cache)

@pytest.mark.parametrize("rows,cols,dtype,skew", [(128, 512, torch.bfloat16, 0.0), (100, 1024, torch.bfloat16, -2.5),
                                                  (37, 64, torch.float32, 0.0), (4096, 1024, torch.bfloat16, 0.0)])
def test_rowwise_quant_bit_exact(rows, cols, dtype, skew):
    from flower_amd import _lib as L
    lb = L.load()
    x = (seeded((rows, cols), 7, torch.float32) + skew).to(dtype)
    out = torch.empty((rows, cols), dtype=torch.uint8, device="cuda")
    sc = torch.empty(rows, dtype=torch.float32, device="cuda")
    L.check(lb.flw_quant_rows_e4m3(x.data_ptr(), L.dtype_code(dtype), rows, cols, cols, out.data_ptr(),
                                   sc.data_ptr(), L.stream_of(x)), "rows")
    want_codes, want_scale = rowwise_fp8(to_np(x))
    np.testing.assert_array_equal(to_np(out), want_codes)
    np.testing.assert_array_equal(to_np(sc), want_scale.reshape(-1))


def test_abi_rejects_bad_arguments():
    L = lib()
    lb = L.load()
    x = torch.zeros(1, 1, 64, 60, device="cuda")       # D not a multiple of 4? 60 is; use 62 bf16
    xb = torch.zeros(1, 1, 64, 62, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(64 * 62, dtype=torch.uint8, device="cuda")
    sc = torch.empty(1, device="cuda")
    ws = L.workspace(1024, "cuda")
    rc = lb.flw_quant_e4m3(xb.data_ptr(), L.BF16, 1, 1, 64, 62, 64 * 62, 64 * 62, 62, 0, 0, out.data_ptr(),
                           sc.data_ptr(), ws.data_ptr(), ws.numel(), None)
    assert rc == 2 and b"multiple" in lb.flw_last_error()
    rc = lb.flw_quant_e4m3(x.data_ptr(), L.F32, 1, 1, 64, 60, 64 * 60, 64 * 60, 60, 0, 0, out.data_ptr(),
                           sc.data_ptr(), ws.data_ptr(), 0, None)
    assert rc == 3 and b"workspace" in lb.flw_last_error()
    assert ctypes.c_int(rc).value == 3


# ------------------------------------------------------------------ fused producers of FP8 inputs

def _ulp(a, b):
    from oracle.e4m3 import f32_to_bf16_bits
    ia = f32_to_bf16_bits(np.asarray(a, np.float32)).astype(np.int32)
    ib = f32_to_bf16_bits(np.asarray(b, np.float32)).astype(np.int32)
    return np.abs(ia - ib)


@pytest.mark.parametrize("rows,cols", [(300, 1024), (17, 4096), (64, 520), (5, 8)])
def test_rmsnorm_quant_rows(rows, cols):
    """flw_rmsnorm_quant_rows_e4m3: h against the oracle's RMSNorm (last-place differences from
    the mean's summation order only), and the codes / scales bit-exact against the per-row
    quantiser applied to the kernel's own h."""
    from oracle.block import rmsnorm
    L = lib()
    lb = L.load()
    g = torch.Generator().manual_seed(rows)
    rs = cols + 16
    xbuf = (torch.randn(rows, rs, generator=g) * 3).to(torch.bfloat16)
    xbuf[rows // 2, :cols] = 0                      # an all-zero row: scale hits the 1e-12 floor
    w = (1 + 0.2 * torch.randn(cols, generator=g)).to(torch.bfloat16)
    tx, tw = xbuf.cuda(), w.cuda()
    codes = torch.empty((rows, cols), dtype=torch.uint8, device="cuda")
    sc = torch.empty(rows, dtype=torch.float32, device="cuda")
    h = torch.empty((rows, cols), dtype=torch.bfloat16, device="cuda")
    L.check(lb.flw_rmsnorm_quant_rows_e4m3(tx.data_ptr(), rows, cols, rs, tw.data_ptr(), 1e-6, codes.data_ptr(),
                                           sc.data_ptr(), h.data_ptr(), L.stream_of(tx)), "rmsnorm_quant")
    torch.cuda.synchronize()
    want_h = rmsnorm(xbuf[:, :cols].float().numpy(), w.float().numpy(), 1e-6)
    d = _ulp(h.float().cpu().numpy(), want_h)
    assert d.max() <= 1 and (d > 0).mean() < 1e-3, ((d > 0).mean(), d.max())
    want_c, want_s = rowwise_fp8(h.float().cpu().numpy())
    np.testing.assert_array_equal(codes.cpu().numpy(), want_c)
    np.testing.assert_array_equal(to_np(sc), want_s.reshape(-1))


@pytest.mark.parametrize("rows,cols", [(200, 4096), (33, 1024)])
def test_gelu_quant_rows(rows, cols):
    """flw_gelu_quant_rows_e4m3: h against the oracle's exact-erf GELU (the device erff differs in
    the last place; outputs under 1e-4 compared absolutely), codes / scales bit-exact against the
    per-row quantiser applied to the kernel's own h."""
    from oracle.block import gelu
    L = lib()
    lb = L.load()
    g = torch.Generator().manual_seed(cols)
    x = (torch.randn(rows, cols, generator=g) * 3).to(torch.bfloat16)
    tx = x.cuda()
    codes = torch.empty((rows, cols), dtype=torch.uint8, device="cuda")
    sc = torch.empty(rows, dtype=torch.float32, device="cuda")
    h = torch.empty((rows, cols), dtype=torch.bfloat16, device="cuda")
    L.check(lb.flw_gelu_quant_rows_e4m3(tx.data_ptr(), rows, cols, cols, codes.data_ptr(), sc.data_ptr(),
                                        h.data_ptr(), L.stream_of(tx)), "gelu_quant")
    torch.cuda.synchronize()
    got = h.float().cpu().numpy()
    want = gelu(x.float().numpy())
    big = np.abs(want) > 1e-4
    d = _ulp(got[big], want[big])
    assert d.max() <= 1 and (d > 0).mean() < 0.02, ((d > 0).mean(), d.max())
    assert np.abs(got[~big] - want[~big]).max() < 2e-6
    want_c, want_s = rowwise_fp8(got)
    np.testing.assert_array_equal(codes.cpu().numpy(), want_c)
    np.testing.assert_array_equal(to_np(sc), want_s.reshape(-1))


@pytest.mark.parametrize("act", ["rmsnorm", "gelu"])
def test_fused_row_quantisers_nan_rows(act):
    """A NaN in a row: h carries the canonical bf16 NaN 0x7FC0 (torch's float -> bf16 rounding) where
    it is NaN, and that row's scale and codes follow the per-row quantiser on the kernel's own h;
    the other rows are unaffected."""
    L = lib()
    lb = L.load()
    rows, cols = 8, 1024
    g = torch.Generator().manual_seed(99)
    x = (torch.randn(rows, cols, generator=g) * 3).to(torch.bfloat16)
    xn = x.clone()
    xn[3, 17] = float("nan")
    w = (1 + 0.2 * torch.randn(cols, generator=g)).to(torch.bfloat16).cuda()
    outs = []
    for inp in (x, xn):
        tx = inp.cuda()
        codes = torch.empty((rows, cols), dtype=torch.uint8, device="cuda")
        sc = torch.empty(rows, dtype=torch.float32, device="cuda")
        h = torch.empty((rows, cols), dtype=torch.bfloat16, device="cuda")
        if act == "rmsnorm":
            rc = lb.flw_rmsnorm_quant_rows_e4m3(tx.data_ptr(), rows, cols, cols, w.data_ptr(), 1e-6, codes.data_ptr(),
                                                sc.data_ptr(), h.data_ptr(), L.stream_of(tx))
        else:
            rc = lb.flw_gelu_quant_rows_e4m3(tx.data_ptr(), rows, cols, cols, codes.data_ptr(), sc.data_ptr(),
                                             h.data_ptr(), L.stream_of(tx))
        L.check(rc, act)
        torch.cuda.synchronize()
        outs.append((codes.cpu(), sc.cpu(), h.cpu()))
    (c0, s0, h0), (c1, s1, h1) = outs
    keep = torch.arange(rows) != 3
    assert torch.equal(c0[keep], c1[keep]) and torch.equal(s0[keep], s1[keep]) and torch.equal(h0[keep], h1[keep])
    hb = h1[3].view(torch.int16).numpy().astype(np.uint16)
    nan = np.isnan(h1[3].float().numpy())
    assert nan.any() and (hb[nan] == 0x7FC0).all()
    assert np.isnan(s1[3].item())
    want_c, _ = rowwise_fp8(h1[3:4].float().numpy())
    np.testing.assert_array_equal(c1[3:4].numpy(), want_c)


# ------------------------------------------------------------------ amax pass / given amax

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("gran", ["tensor", "head", "bh"])
def test_amax_pass_alone_matches_oracle(gran, dtype):
    """flw_amax_e4m3: |x| max per scale group, bit-exact against the oracle's amax (the amax of
    per_tensor_fp8, fp8_swa_attention.py:201), on a strided (B, T, H, D) view."""
    from flower_amd.kernels import amax_e4m3
    from oracle.quant import _amax, group_axes
    x = (seeded((2, 300, 3, 64), 41) * torch.exp(seeded((1, 1, 3, 1), 42))).to(dtype)
    xv = x.cuda().transpose(1, 2)                    # (B, H, T, D), non-contiguous
    got = amax_e4m3(xv, gran)
    ref = _amax(to_np(x.transpose(1, 2)), group_axes(4, gran)).reshape(-1)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(got).view(np.uint32), ref.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("gran", ["tensor", "head", "bh"])
def test_quantise_with_given_amax_equals_the_two_pass_quantiser(gran):
    """flw_quant_e4m3_amax(x, flw_amax_e4m3(x)) == flw_quant_e4m3(x), codes and scales bit for
    bit, and both equal the oracle (near-tie inputs, where x / s rounding decides codes)."""
    from flower_amd.kernels import _per_tensor_fp8, amax_e4m3, quantize_e4m3_with_amax
    x = near_ties((2, 3, 200, 64), 43).cuda()
    c1, s1 = _per_tensor_fp8(x, gran)
    c2, s2 = quantize_e4m3_with_amax(x, amax_e4m3(x, gran), gran)
    torch.cuda.synchronize()
    assert torch.equal(c1.view(torch.uint8), c2.view(torch.uint8))
    assert torch.equal(s1.view(torch.int32), s2.view(torch.int32))
    codes, scale = per_tensor_fp8(to_np(x), gran)
    assert np.array_equal(to_np(c2.view(torch.uint8)), codes)
    assert np.array_equal(to_np(s2).view(np.uint32), np.asarray(scale, np.float32).reshape(-1).view(np.uint32))


@pytest.mark.parametrize("gran", ["tensor", "head"])
def test_sequence_shards_quantised_with_the_combined_amax_match_the_whole(gran):
    """A sequence-sharded tensor (two T ranges, as two ranks would hold it): each shard's amax,
    combined by MAX on the int32 view (what an all_reduce(MAX) over RCCL would do), then each
    shard quantised with the combined amax, gives exactly the whole tensor's codes and scale.
    A NaN in one shard reaches the combined amax and every shard's scale."""
    from flower_amd.kernels import _per_tensor_fp8, amax_e4m3, quantize_e4m3_with_amax
    x = (seeded((1, 4, 512, 64), 44) * torch.exp(seeded((1, 4, 1, 1), 45))).to(torch.bfloat16).cuda()
    parts = [x[:, :, :192], x[:, :, 192:]]
    amax = torch.maximum(*(amax_e4m3(p, gran).view(torch.int32) for p in parts)).view(torch.float32)
    codes = [quantize_e4m3_with_amax(p, amax, gran) for p in parts]
    whole_c, whole_s = _per_tensor_fp8(x, gran)
    torch.cuda.synchronize()
    assert torch.equal(torch.cat([c.view(torch.uint8) for c, _ in codes], dim=2), whole_c.view(torch.uint8))
    for _, s in codes:
        assert torch.equal(s.view(torch.int32), whole_s.view(torch.int32))
    y = x.clone()
    y[0, 1, 300, 5] = float("nan")
    a = [amax_e4m3(p, gran) for p in (y[:, :, :192], y[:, :, 192:])]
    comb = torch.maximum(*(t.view(torch.int32) for t in a)).view(torch.float32)
    torch.cuda.synchronize()
    assert torch.isnan(comb[0 if gran == "tensor" else 1])


def test_given_amax_is_validated():
    from flower_amd.kernels import quantize_e4m3_with_amax
    x = seeded((1, 2, 64, 64), 46).cuda()
    with pytest.raises(ValueError, match="float32 tensor of 2"):
        quantize_e4m3_with_amax(x, torch.ones(3, device="cuda"), "head")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("factor", [0.5, 1.0, -1.0])
@pytest.mark.parametrize("gran", ["tensor", "head", "bh"])
def test_given_amax_below_the_data_max_clamps_like_the_reference(gran, factor, dtype):
    """A given amax smaller than the data's |x| max (a stale or wrong producer maximum): every
    quotient above 448 is clamped exactly as clamp(x / s, -448, 448) then the cast, with inf, NaN
    and a 1e30 among the inputs, bit-exact against the oracle with the same amax swapped in."""
    from flower_amd.kernels import quantize_e4m3_with_amax
    from oracle.quant import _amax, group_axes
    x = near_ties((2, 3, 200, 64), 47)
    axes = group_axes(4, gran)
    given = (_amax(x.numpy(), axes).reshape(-1) * np.float32(factor)).astype(np.float32)
    x[0, 1, 3, :4] = torch.tensor([float("inf"), float("-inf"), float("nan"), -float("nan")])
    x[1, 2, 5, 8] = 1e30
    x = x.to(dtype)
    xd = x.cuda()
    codes, scale = quantize_e4m3_with_amax(xd, torch.from_numpy(given).cuda(), gran)
    want_c, want_s = per_tensor_fp8(to_np(x), gran, amax=given)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(codes.view(torch.uint8)), want_c)
    assert np.array_equal(to_np(scale).view(np.uint32), np.asarray(want_s, np.float32).reshape(-1).view(np.uint32))
    if factor == 0.5:
        assert int(((codes.view(torch.uint8) & 0x7F) == 0x7E).sum()) > 1000
