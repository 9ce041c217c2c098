"""RMSNorm and GELU of the decoder block around the FP8 linears. TEST INFRASTRUCTURE ONLY.

``rmsnorm``  flower/models/base.py:324-338 on bf16 activations:
             h = bf16( bf16( x * rsqrt(mean(x^2) + eps) ) * w )
             (fp32 mean of squares and rsqrt, the product rounded to bf16, then the bf16 gain
             multiplied in fp32 and rounded to bf16 again, as torch does for bf16 tensors).
``gelu``     torch.nn.functional.gelu(approximate="none") on bf16 values:
             bf16( (0.5 x) * (1 + erf(x / sqrt 2)) ), evaluated in fp32 in that order with a
             correctly rounded erf.

Pinned by tests/test_oracle_block.py against torch's CPU operators on the same bf16 inputs (a
library routine): identical except for rare last-place differences from summation order and
the erf implementation.
"""

from __future__ import annotations

import math

import numpy as np

from .e4m3 import round_bf16

F32 = np.float32


def rmsnorm(x: np.ndarray, weight: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """x [rows, d] (bf16 values as fp32), weight [d] (bf16 values) -> bf16 values as fp32."""
    xf = np.asarray(x, dtype=F32)
    ms = np.mean(xf * xf, axis=-1, keepdims=True, dtype=F32)
    r = (F32(1.0) / np.sqrt(ms + F32(eps), dtype=F32)).astype(F32)
    h = round_bf16((xf * r).astype(F32))
    return round_bf16((h * np.asarray(weight, dtype=F32)).astype(F32))


_erf = np.vectorize(math.erf, otypes=[np.float64])


def gelu(x: np.ndarray) -> np.ndarray:
    """bf16 values in and out (as fp32): (0.5 x) (1 + erf(x / sqrt 2)) evaluated in fp32 in
    that order, erf correctly rounded to fp32 (so 1 + erf cancels to 0 below x ~ -5.3, exactly as
    an fp32 evaluation does)."""
    xf = np.asarray(x, dtype=F32)
    a = (xf * F32(1.0 / math.sqrt(2.0))).astype(F32)
    e = _erf(a.astype(np.float64)).astype(F32)
    return round_bf16(((F32(0.5) * xf).astype(F32) * (F32(1.0) + e).astype(F32)).astype(F32))
