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
