"""Quantisation recipes of the reference's FP8 path, restated op by op in numpy.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Every function reproduces the reference's operation order and the dtype each intermediate is
rounded to, because the e4m3 codes and scales are gated bit-exact:

``per_tensor_fp8`` -- flower/kernels/fp8_swa_attention.py:195-205 (``_per_tensor_fp8``):
    amax = |x|.amax().float().clamp(min=1e-12)      (fp32)
    scale = amax / 448                              (fp32, IEEE division)
    code = e4m3( clamp(fp32(x) / scale, -448, 448) ) (fp32 IEEE division, NaN propagates)
  The reference returns the scale via ``.item()`` and divides by that Python float. On the CPU
  that is the same IEEE fp32 division restated here. (torch's CUDA kernel instead multiplies by
  the fp32 reciprocal when the divisor is a host scalar; this build follows the CPU semantics,
  which are also the ``_fake_quant_e4m3`` semantics below, where the divisor is a tensor.)

``group`` generalises the amax to per-head (amax over B,T,D for each h) and per-(b,h)
  (amax over T,D). The reference has no per-head code; the build defines it as the per-tensor
  recipe applied to each slice (fp8_swa_attention.py:57 reports a "per-head scales" row only).

``fake_quant_e4m3`` -- flower/models/base.py:167-203 (``_fake_quant_e4m3``), dtype-faithful:
    amax = |x|.amax().clamp(min=1e-12)   in x.dtype
    scale = amax / 448.0                 in x.dtype (fp32 maths rounded to x.dtype)
    y = clamp(x / scale, +-448)          division in fp32, rounded to x.dtype
    dq = e4m3(y).to(x.dtype) * scale     product rounded to x.dtype
    out = x + (dq - x)                   each op rounded to x.dtype (straight-through form)

``rowwise_fp8`` -- flower/models/base.py:911-918 (``_fp8_head``), per row of a 2-D tensor:
    scale = clamp_min( fp32(|x|.amax(-1)) / 448, 1e-12 )   (divide THEN clamp)
    code = e4m3( fp32(x) / scale )                         (no clamp before the cast)
  Used for the activation rows and the weight output-channels of the FP8 GEMM.

Pinned by tests/test_oracle_quant.py against the reference's formulas evaluated with torch's
own CPU operators (a separate implementation of the same ops), on seeded, adversarial and
special inputs (zeros, NaN, ties, subnormals, bf16 and fp32).
"""

from __future__ import annotations

import numpy as np

from .e4m3 import E4M3_MAX, e4m3_to_f32, f32_to_e4m3, round_bf16

F32 = np.float32
EPS = F32(1e-12)
QMAX = F32(E4M3_MAX)

GRANULARITIES = ("tensor", "head", "bh")


def _amax(x: np.ndarray, axes) -> np.ndarray:
    """|x|.amax over axes with NaN propagation (torch.amax propagates NaN)."""
    a = np.abs(x.astype(F32))
    return np.max(a, axis=axes, keepdims=True)


def group_axes(ndim: int, granularity: str):
    """Reduction axes for a (B, H, T, D) tensor at a given scale granularity."""
    if ndim != 4 and granularity != "tensor":
        raise ValueError("per-head / per-(b,h) scales need a (B, H, T, D) tensor")
    if granularity == "tensor":
        return tuple(range(ndim))
    if granularity == "head":
        return (0, 2, 3)
    if granularity == "bh":
        return (2, 3)
    raise ValueError(f"granularity must be one of {GRANULARITIES}, got {granularity!r}")


def scale_a2(amax: np.ndarray) -> np.ndarray:
    """fp8_swa_attention.py:203-204: clamp(min=1e-12) then /448, in fp32."""
    amax = amax.astype(F32)
    amax = np.where(amax < EPS, EPS, amax)          # torch.clamp keeps NaN
    return (amax / QMAX).astype(F32)


def per_tensor_fp8(x: np.ndarray, granularity: str = "tensor", amax: np.ndarray | None = None):
    """``_per_tensor_fp8`` (and its per-head / per-(b,h) extension).

    x: float32 array holding fp32 or bf16 values. Returns (codes uint8 same shape,
    scale float32 with keepdims shape of the group). ``amax`` (optional, one value per scale
    group, e.g. a producer's maximum or one combined across shards) replaces the amax of x in
    the scale; the clamp then bounds every quotient it leaves above 448.
    """
    xf = x.astype(F32)
    axes = group_axes(xf.ndim, granularity)
    if amax is None:
        amax = _amax(xf, axes)
    else:
        shape = [1 if i in axes else n for i, n in enumerate(xf.shape)]
        amax = np.asarray(amax, F32).reshape(shape)
    scale = scale_a2(amax)
    y = (xf / scale).astype(F32)
    y = np.where(y > QMAX, QMAX, np.where(y < -QMAX, -QMAX, y))   # clamp, NaN propagates
    return f32_to_e4m3(y), scale


def _round(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "f32":
        return x.astype(F32)
    if dtype == "bf16":
        return round_bf16(x.astype(F32))
    raise ValueError(dtype)


def fake_quant_scale(x: np.ndarray, dtype: str, granularity: str = "tensor") -> np.ndarray:
    """base.py:198-199 scale, kept in x.dtype (bf16 scale under autocast)."""
    amax = _amax(x, group_axes(x.ndim, granularity))                 # exact in any dtype
    eps = _round(np.array(EPS, dtype=F32), dtype)
    amax = np.where(amax < eps, eps, amax)
    return _round((amax / QMAX).astype(F32), dtype)


def fake_quant_e4m3(x: np.ndarray, dtype: str, granularity: str = "tensor"):
    """``_fake_quant_e4m3`` forward value; x holds values representable in ``dtype``.

    Returns (out, codes, scale), all rounded exactly as the reference's op sequence rounds.
    """
    xf = x.astype(F32)
    scale = fake_quant_scale(xf, dtype, granularity)
    y = _round((xf / scale).astype(F32), dtype)
    y = np.where(y > QMAX, QMAX, np.where(y < -QMAX, -QMAX, y))
    codes = f32_to_e4m3(y)
    dq = _round((e4m3_to_f32(codes) * scale).astype(F32), dtype)
    d = _round((dq - xf).astype(F32), dtype)
    out = _round((xf + d).astype(F32), dtype)
    return out, codes, scale


def rowwise_scale(x: np.ndarray) -> np.ndarray:
    """base.py:912-913: |x|.amax(-1).float() / 448, then clamp_min(1e-12). Shape [rows, 1]."""
    amax = _amax(x.astype(F32), (-1,))
    s = (amax / QMAX).astype(F32)
    return np.where(s < EPS, EPS, s)


def rowwise_fp8(x: np.ndarray):
    """base.py:917-918: e4m3(fp32(x) / scale) per row, no clamp. Returns (codes, scale[rows,1])."""
    xf = x.astype(F32)
    scale = rowwise_scale(xf)
    return f32_to_e4m3((xf / scale).astype(F32)), scale


def dequant(codes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """fp32 value of e4m3 codes times their scale (exact product rounded to fp32)."""
    return (e4m3_to_f32(codes) * scale.astype(F32)).astype(F32)
