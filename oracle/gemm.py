"""Closed form of the scaled FP8 GEMM on the path. TEST INFRASTRUCTURE ONLY.

The reference's self-contained FP8 GEMM is ``CausalLM._fp8_head`` (flower/models/base.py:887-924):
per-row activation scales ``scale_a[m]``, per-output-channel weight scales ``scale_b[n]``, e4m3
operands, ``torch._scaled_mm(x8, w8.t(), scale_a, scale_b, out_dtype=bf16)``, i.e.

    y[m, n] = bf16( (sum_k x8[m, k] * w8[n, k]) * scale_a[m] * scale_b[n] )

with fp32 accumulation. Here the sum is taken exactly in float64 (e4m3 products are exact) and
the scaled result is rounded once to fp32 and then to bf16, so a correct fp32-accumulating kernel
differs from it only by accumulation-order rounding (gated by a tolerance in the GPU tests).

``w8a16`` is the weight-only mode: y = bf16( (sum_k x[m, k] * w8[n, k]) * scale_b[n] ), with the
bf16 activations used as they are (e4m3 -> bf16 is exact, so the kernel may widen w8 in place).

Pinned by tests/test_oracle_gemm.py: float64 brute force over explicit loops on tiny shapes,
torch.matmul on the dequantised operands (a library routine), and the reference's FP8-head
acceptance bounds (tests/test_training_speedups.py:375-389: Frobenius error < 0.05, norm ratio
in (0.9, 1.1)) against the unquantised product.
"""

from __future__ import annotations

import numpy as np

from .e4m3 import e4m3_to_f32, round_bf16
from .quant import rowwise_fp8

F32 = np.float32


def scaled_mm(x8: np.ndarray, w8: np.ndarray, scale_a: np.ndarray, scale_b: np.ndarray) -> np.ndarray:
    """x8 [M, K] codes, w8 [N, K] codes, scale_a [M] or [M,1] (or scalar), scale_b [N] -> fp32 [M, N]
    (before the bf16 output rounding)."""
    xf = e4m3_to_f32(x8).astype(np.float64)
    wf = e4m3_to_f32(w8).astype(np.float64)
    acc = xf @ wf.T
    sa = np.asarray(scale_a, dtype=np.float64).reshape(-1, 1)
    sb = np.asarray(scale_b, dtype=np.float64).reshape(1, -1)
    return (acc * sa * sb).astype(F32)


def fp8_linear_a8w8(x: np.ndarray, w8: np.ndarray, w_scale: np.ndarray):
    """Per-row activation quantisation (base.py:912,917) then the scaled GEMM; bf16 values as fp32."""
    x8, sa = rowwise_fp8(x)
    return round_bf16(scaled_mm(x8, w8, sa, w_scale)), x8, sa


def fp8_linear_w8a16(x: np.ndarray, w8: np.ndarray, w_scale: np.ndarray) -> np.ndarray:
    """Weight-only FP8: dequantised weight times bf16 activations, fp32 accumulate, bf16 out."""
    wf = e4m3_to_f32(w8).astype(np.float64)
    acc = x.astype(np.float64) @ wf.T
    return round_bf16((acc * np.asarray(w_scale, np.float64).reshape(1, -1)).astype(F32))
