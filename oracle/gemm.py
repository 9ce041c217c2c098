"""Closed form of the scaled FP8 GEMM on the path. TEST INFRASTRUCTURE ONLY.

The reference's self-contained FP8 GEMM is ``CausalLM._fp8_head`` (flower/models/base.py:887-924):
per-row activation scales ``scale_a[m]``, per-output-channel weight scales ``scale_b[n]``, e4m3
operands, ``torch._scaled_mm(x8, w8.t(), scale_a, scale_b, out_dtype=bf16)``, i.e.

    y[m, n] = bf16( (sum_k x8[m, k] * w8[n, k]) * scale_a[m] * scale_b[n] )

with fp32 accumulation. Here the sum is taken exactly in float64 (e4m3 products are exact) and
the scaled result is rounded once to fp32 and then to bf16, so a correct fp32-accumulating kernel
differs from it only by accumulation-order rounding (gated by a tolerance in the GPU tests).

``cols_fp8`` / ``fp8_linear_backward``: the FP8 gradient GEMMs of y = x W^T that torchao's
Float8Linear runs under ``training.fp8_linear`` (flower/train.py:368-370; torchao 0.18.0,
uv.lock:1642-1644, is not vendored and not installed, so its own scale arithmetic is parity
unpinned — the recipes below reuse the path's two pinned quantisers):
    dgrad  gx = bf16( scaled_mm(rows(g), cols(W)^T) ),   gW = bf16( scaled_mm(cols(g)^T, cols(x)^T) )
with rows() = ``rowwise_fp8`` / cols() = ``rowwise_fp8`` of the transpose for "rowwise", and
``per_tensor_fp8`` (tensor) for both under "tensorwise".

``w8a16`` is the weight-only mode: y = bf16( (sum_k x[m, k] * w8[n, k]) * scale_b[n] ), with the
bf16 activations used as they are (e4m3 -> bf16 is exact, so the kernel may widen w8 in place).

Pinned by tests/test_oracle_gemm.py (the backward also: the float64 gradients g W and g^T x of
the unquantised operands within the FP8-head acceptance bounds, torch.matmul on the dequantised
codes, and a planted wrong-axis scale that must fail): float64 brute force over explicit loops on tiny shapes,
torch.matmul on the dequantised operands (a library routine), and the reference's FP8-head
acceptance bounds (tests/test_training_speedups.py:375-389: Frobenius error < 0.05, norm ratio
in (0.9, 1.1)) against the unquantised product.
"""

from __future__ import annotations

import numpy as np

from .e4m3 import e4m3_to_f32, round_bf16
from .quant import per_tensor_fp8, rowwise_fp8

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


def cols_fp8(x: np.ndarray, granularity: str = "column"):
    """e4m3 codes of each column of x [R, C], transposed ([C, R]), and the scales ([C] or [1]).
    "column": ``rowwise_fp8`` of x^T (the _fp8_head recipe per column); "tensor":
    ``per_tensor_fp8`` of x (the _per_tensor_fp8 recipe), transposed."""
    if granularity == "column":
        codes, s = rowwise_fp8(np.ascontiguousarray(x.T))
        return codes, s.reshape(-1).astype(F32)
    codes, s = per_tensor_fp8(x, "tensor")
    return np.ascontiguousarray(codes.T), np.asarray(s, F32).reshape(-1)


def rows_fp8(x: np.ndarray, recipe: str):
    """(codes [M, K], scales [M] or [1]) of the dgrad left operand."""
    if recipe == "rowwise":
        codes, s = rowwise_fp8(x)
        return codes, s.reshape(-1).astype(F32)
    codes, s = per_tensor_fp8(x, "tensor")
    return codes, np.asarray(s, F32).reshape(-1)


def fp8_linear_backward(g: np.ndarray, x: np.ndarray, w: np.ndarray, recipe: str = "rowwise"):
    """(gx [M, K], gW [N, K]) as bf16 values in fp32, for y = x W^T with g = dL/dy [M, N]."""
    gran = "column" if recipe == "rowwise" else "tensor"
    g8, sg = rows_fp8(g, recipe)
    w8c, swc = cols_fp8(w, gran)                    # [K, N]
    gx = round_bf16(scaled_mm(g8, w8c, sg, swc))
    g8c, sgc = cols_fp8(g, gran)                    # [N, M]
    x8c, sxc = cols_fp8(x, gran)                    # [K, M]
    gw = round_bf16(scaled_mm(g8c, x8c, sgc, sxc))
    return gx, gw
