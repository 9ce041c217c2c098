"""Pins the GEMM oracle (oracle/gemm.py): the scaled FP8 GEMM of ``CausalLM._fp8_head``
(flower/models/base.py:887-924) and the weight-only mode.

- float64 brute force over explicit loops on tiny shapes (a dropped scale, a transposed operand
  or a wrong scale axis fails it);
- torch.matmul on the dequantised operands (a library routine, independent of the numpy path);
- the reference's FP8-head acceptance bounds (tests/test_training_speedups.py:375-389 of the
  reference: Frobenius error < 0.05 and norm ratio in (0.9, 1.1) against the unquantised
  product), including rows whose largest magnitude is negative (:392-412).
"""

import numpy as np
import pytest
import torch

from oracle.e4m3 import e4m3_to_f32, round_bf16
from oracle.gemm import fp8_linear_a8w8, fp8_linear_w8a16, scaled_mm
from oracle.quant import rowwise_fp8


def _rnd(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def test_scaled_mm_equals_loop_brute_force():
    M, N, K = 3, 5, 7
    x8, sa = rowwise_fp8(_rnd((M, K), 0))
    w8, sb = rowwise_fp8(_rnd((N, K), 1, 0.02))
    got = scaled_mm(x8, w8, sa, sb.reshape(-1))
    xf, wf = e4m3_to_f32(x8).astype(np.float64), e4m3_to_f32(w8).astype(np.float64)
    want = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                acc += xf[m, k] * wf[n, k]
            want[m, n] = acc * float(sa[m, 0]) * float(sb[n, 0])
    np.testing.assert_allclose(got, want.astype(np.float32), rtol=1e-6, atol=0)


@pytest.mark.parametrize("M,N,K", [(16, 32, 64), (64, 48, 128)])
def test_scaled_mm_equals_torch_matmul_on_dequantised_operands(M, N, K):
    x8, sa = rowwise_fp8(_rnd((M, K), 2))
    w8, sb = rowwise_fp8(_rnd((N, K), 3, 0.02))
    xd = torch.from_numpy(e4m3_to_f32(x8).astype(np.float64)) * torch.from_numpy(sa.astype(np.float64))
    wd = torch.from_numpy(e4m3_to_f32(w8).astype(np.float64)) * torch.from_numpy(sb.astype(np.float64))
    want = (xd @ wd.T).numpy()
    np.testing.assert_allclose(scaled_mm(x8, w8, sa, sb.reshape(-1)), want, rtol=1e-6, atol=1e-30)


def test_per_tensor_scales_broadcast():
    x8, sa = rowwise_fp8(_rnd((8, 32), 4))
    w8, sb = rowwise_fp8(_rnd((4, 32), 5))
    full = scaled_mm(x8, w8, np.full((8, 1), 0.5, np.float32), np.full(4, 2.0, np.float32))
    scalar = scaled_mm(x8, w8, np.float32(0.5), np.float32(2.0))
    np.testing.assert_array_equal(full, scalar)


@pytest.mark.parametrize("shift", [0.0, -2.5])
def test_fp8_head_acceptance_bounds(shift):
    """The reference's FP8-head checks against the unquantised (bf16-level) product."""
    x = _rnd((32, 256), 6) + np.float32(shift)
    w = _rnd((64, 256), 7, 0.02)
    w8, sw = rowwise_fp8(w)
    y, _, _ = fp8_linear_a8w8(x, w8, sw.reshape(-1))
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert rel < 0.05
    assert 0.9 < np.linalg.norm(y) / np.linalg.norm(ref) < 1.1
    assert np.isfinite(y).all()


def test_w8a16_is_exact_widening_of_the_weight():
    x = round_bf16(_rnd((6, 64), 8))
    w8, sw = rowwise_fp8(_rnd((10, 64), 9, 0.02))
    got = fp8_linear_w8a16(x, w8, sw.reshape(-1))
    wd = e4m3_to_f32(w8).astype(np.float64)
    want = round_bf16(((x.astype(np.float64) @ wd.T) * sw.reshape(1, -1).astype(np.float64)).astype(np.float32))
    np.testing.assert_array_equal(got, want)


# ---------------------------------------------------------------- FP8 backward (dgrad / wgrad)

from oracle.gemm import cols_fp8, fp8_linear_backward, rows_fp8  # noqa: E402
from oracle.quant import per_tensor_fp8  # noqa: E402


def test_cols_fp8_is_the_row_recipe_of_the_transpose():
    x = _rnd((37, 24), 10)
    codes, s = cols_fp8(x, "column")
    assert codes.shape == (24, 37) and s.shape == (24,)
    for c in (0, 7, 23):
        amax = np.abs(x[:, c]).max()
        assert s[c] == np.float32(amax / np.float32(448.0))
        # every code is the e4m3 of x / s (within the e4m3 spacing of the quotient)
        q = e4m3_to_f32(codes[c]).astype(np.float64)
        ref = x[:, c].astype(np.float64) / s[c]
        assert np.all(np.abs(q - ref) <= np.abs(ref) * 2.0 ** -4 + 2.0 ** -10)
    tc, ts = cols_fp8(x, "tensor")
    c2, s2 = per_tensor_fp8(x, "tensor")
    np.testing.assert_array_equal(tc, c2.T)
    assert ts.shape == (1,) and ts[0] == np.float32(s2).reshape(-1)[0]


@pytest.mark.parametrize("recipe", ["rowwise", "tensorwise"])
@pytest.mark.parametrize("M,N,K", [(64, 48, 32), (200, 96, 80)])
def test_fp8_backward_against_float64_gradients(recipe, M, N, K):
    """The FP8-head acceptance bounds (Frobenius error < 0.05, norm ratio in (0.9, 1.1)) for both
    gradients against the float64 gradients of the unquantised operands."""
    g, x, w = _rnd((M, N), 11), _rnd((M, K), 12), _rnd((N, K), 13, 0.02)
    gx, gw = fp8_linear_backward(g, x, w, recipe)
    for got, want in ((gx, g.astype(np.float64) @ w), (gw, g.astype(np.float64).T @ x)):
        err = np.linalg.norm(got - want) / np.linalg.norm(want)
        ratio = np.linalg.norm(got) / np.linalg.norm(want)
        assert err < 0.05 and 0.9 < ratio < 1.1, (err, ratio)


def test_fp8_backward_equals_torch_matmul_on_dequantised_codes():
    M, N, K = 96, 64, 48
    g, x, w = _rnd((M, N), 14), _rnd((M, K), 15), _rnd((N, K), 16, 0.02)
    gx, gw = fp8_linear_backward(g, x, w, "rowwise")
    g8, sg = rows_fp8(g, "rowwise")
    w8c, swc = cols_fp8(w, "column")
    gd = torch.from_numpy(e4m3_to_f32(g8).astype(np.float64) * sg.astype(np.float64)[:, None])
    wd = torch.from_numpy(e4m3_to_f32(w8c).astype(np.float64) * swc.astype(np.float64)[:, None])
    want_gx = round_bf16(torch.matmul(gd, wd.T).numpy().astype(np.float32))
    np.testing.assert_array_equal(gx, want_gx)
    g8c, sgc = cols_fp8(g, "column")
    x8c, sxc = cols_fp8(x, "column")
    gcd = torch.from_numpy(e4m3_to_f32(g8c).astype(np.float64) * sgc.astype(np.float64)[:, None])
    xcd = torch.from_numpy(e4m3_to_f32(x8c).astype(np.float64) * sxc.astype(np.float64)[:, None])
    want_gw = round_bf16(torch.matmul(gcd, xcd.T).numpy().astype(np.float32))
    np.testing.assert_array_equal(gw, want_gw)


def test_wrong_axis_scale_is_caught():
    """A plausible mistake -- the weight's per-output-channel (row) scales used for dgrad instead
    of per-column scales -- breaks the acceptance bounds on a weight with uneven rows."""
    M, N, K = 64, 48, 32
    g, x = _rnd((M, N), 17), _rnd((M, K), 18)
    w = _rnd((N, K), 19, 0.02) * np.linspace(0.1, 10.0, N, dtype=np.float32)[:, None]
    g8, sg = rows_fp8(g, "rowwise")
    w8, sw = rowwise_fp8(w)                          # row scales, the forward's codes
    wrong = round_bf16(scaled_mm(g8, np.ascontiguousarray(w8.T), sg, np.full(K, sw.mean(), np.float32)))
    want = g.astype(np.float64) @ w
    assert np.linalg.norm(wrong - want) / np.linalg.norm(want) > 0.05
    gx, _ = fp8_linear_backward(g, x, w, "rowwise")
    assert np.linalg.norm(gx - want) / np.linalg.norm(want) < 0.05
