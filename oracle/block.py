"""RMSNorm and GELU of the decoder block around the FP8 linears. TEST INFRASTRUCTURE ONLY.

``rmsnorm``  flower/models/base.py:324-338 on bf16 activations:
             h = bf16( bf16( x * rsqrt(mean(x^2) + eps) ) * w )
             (fp32 mean of squares and rsqrt, the product rounded to bf16, then the bf16 gain
             multiplied in fp32 and rounded to bf16 again, as torch does for bf16 tensors).
``rmsnorm_backward``  the gradients torch's autograd gives x and the gain of ``rmsnorm`` (two
             x.float() casts, each handing back a bf16 gradient, summed in bf16):
             dn = bf16(dh w), dx = bf16(bf16(dn r) - bf16(x r^3 sum(dn x) / d)),
             dw = bf16(sum over rows of bf16(dh n)), n = bf16(x r), the sum in fp32.
``swiglu``, ``swiglu_backward``  FeedForward's SwiGLU product (base.py:538-550, smooth_swiglu
             off) on bf16 values: s = bf16(g / (1 + exp(-g))), h = bf16(s u); backward
             ds = bf16(dh u), du = bf16(dh s), sig = 1 / (1 + exp(-g)),
             dg = bf16(ds sig (1 + g (1 - sig))) (torch's silu backward), fp32 maths with exp
             correctly rounded to fp32.
``gelu``     torch.nn.functional.gelu(approximate="none") on bf16 values:
             bf16( (0.5 x) * (1 + erf(x / sqrt 2)) ), evaluated in fp32 in that order with a
             correctly rounded erf.

``head_rmsnorm``  flower/models/base.py:341-357 (HeadRMSNorm, the QK-norm), per row of D:
             h = dtype( x * (1 / sqrt(mean(x^2) + eps)) ), fp32 maths.
``rope``     base.py:478-483 with rotate_half (:465-469), tables given ([T, D], already in the
             activations' dtype): out = dtype( dtype(x * cos) + dtype(rotate_half(x) * sin) ),
             rotate_half(x)[2i] = -x[2i+1], rotate_half(x)[2i+1] = x[2i].
``rope_backward``  the gradient torch's autograd gives x of ``rope`` in bf16 (the adjoint of the
             rotation, each op rounded as autograd rounds it): t1 = dtype(g cos), t2 = dtype(g sin),
             dx[2i] = dtype(t1[2i] + t2[2i+1]), dx[2i+1] = dtype(t1[2i+1] - t2[2i]).
``head_rmsnorm_backward``  the gradient torch's autograd gives x of ``head_rmsnorm`` (base.py:355-
             357: two x.float() casts, each handing back a gradient of x's dtype, summed in it):
             r = rsqrt(mean(x^2) + eps), dx = dtype(dtype(dn r) - dtype(x r^3 sum(dn x) / D)).

Pinned by tests/test_oracle_block.py against torch's CPU operators on the same bf16 inputs (a
library routine): identical except for rare last-place differences from summation order and
the erf implementation; the backwards also against torch's CPU autograd of the forward
expressions, against the adjoint identity <rope(x), g> = <x, rope_backward(g)> and against
central finite differences in float64.
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


def rmsnorm_backward(x: np.ndarray, weight: np.ndarray, dh: np.ndarray, eps: float = 1e-6):
    """x [rows, d], weight [d], dh = d/d rmsnorm(x) [rows, d] (bf16 values as fp32) -> (dx, dw)."""
    xf = np.asarray(x, dtype=F32)
    w = np.asarray(weight, dtype=F32)
    g = np.asarray(dh, dtype=F32)
    d = xf.shape[-1]
    ms = np.mean(xf * xf, axis=-1, keepdims=True, dtype=F32)
    r = (F32(1.0) / np.sqrt(ms + F32(eps), dtype=F32)).astype(F32)
    n = round_bf16((xf * r).astype(F32))
    dn = round_bf16((g * w).astype(F32))
    dw = round_bf16(np.sum(round_bf16((g * n).astype(F32)).astype(np.float64), axis=0).astype(F32))
    sd = np.sum(dn * xf, axis=-1, keepdims=True, dtype=F32)
    k = (sd * (r * r * r) / F32(d)).astype(F32)
    dx = round_bf16((round_bf16((dn * r).astype(F32)) - round_bf16((xf * k).astype(F32))).astype(F32))
    return dx, dw


def _exp_f32(x: np.ndarray) -> np.ndarray:
    """exp of fp32 values, correctly rounded to fp32 (via float64)."""
    return np.exp(np.asarray(x, dtype=np.float64)).astype(F32)


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """bf16 values in and out (as fp32): bf16(bf16(silu(gate)) up)."""
    g = np.asarray(gate, dtype=F32)
    s = round_bf16((g / (F32(1.0) + _exp_f32(-g))).astype(F32))
    return round_bf16((s * np.asarray(up, dtype=F32)).astype(F32))


def swiglu_backward(gate: np.ndarray, up: np.ndarray, dh: np.ndarray):
    """bf16 values in and out (as fp32): (dgate, dup) of swiglu for the gradient dh."""
    g = np.asarray(gate, dtype=F32)
    u = np.asarray(up, dtype=F32)
    d = np.asarray(dh, dtype=F32)
    den = (F32(1.0) + _exp_f32(-g)).astype(F32)
    s = round_bf16((g / den).astype(F32))
    ds = round_bf16((d * u).astype(F32))
    du = round_bf16((d * s).astype(F32))
    sig = (F32(1.0) / den).astype(F32)
    inner = (F32(1.0) + (g * (F32(1.0) - sig)).astype(F32)).astype(F32)
    dg = round_bf16(((ds * sig).astype(F32) * inner).astype(F32))
    return dg, du


_erf = np.vectorize(math.erf, otypes=[np.float64])


def gelu(x: np.ndarray) -> np.ndarray:
    """bf16 values in and out (as fp32): (0.5 x) (1 + erf(x / sqrt 2)) evaluated in fp32 in
    that order, erf correctly rounded to fp32 (so 1 + erf cancels to 0 below x ~ -5.3, exactly as
    an fp32 evaluation does)."""
    xf = np.asarray(x, dtype=F32)
    a = (xf * F32(1.0 / math.sqrt(2.0))).astype(F32)
    e = _erf(a.astype(np.float64)).astype(F32)
    return round_bf16(((F32(0.5) * xf).astype(F32) * (F32(1.0) + e).astype(F32)).astype(F32))


def _round_dtype(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return round_bf16(np.asarray(x, dtype=F32))
    if dtype == "f32":
        return np.asarray(x, dtype=F32)
    raise ValueError(dtype)


def head_rmsnorm(x: np.ndarray, eps: float = 1e-6, dtype: str = "bf16") -> np.ndarray:
    """x [..., D] (values of ``dtype`` as fp32) -> HeadRMSNorm(x) as fp32 values of ``dtype``."""
    xf = np.asarray(x, dtype=F32)
    ms = np.mean(xf * xf, axis=-1, keepdims=True, dtype=F32)
    r = (F32(1.0) / np.sqrt(ms + F32(eps), dtype=F32)).astype(F32)
    return _round_dtype((xf * r).astype(F32), dtype)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """x [..., T, D], cos / sin [T, D] (values of ``dtype``) -> x * cos + rotate_half(x) * sin with
    every product and the sum rounded to ``dtype``."""
    xf = np.asarray(x, dtype=F32)
    rot = np.empty_like(xf)
    rot[..., 0::2] = -xf[..., 1::2]
    rot[..., 1::2] = xf[..., 0::2]
    a = _round_dtype(xf * np.asarray(cos, F32), dtype)
    b = _round_dtype(rot * np.asarray(sin, F32), dtype)
    return _round_dtype(a + b, dtype)


def rope_backward(g: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """g = d/d rope(x) [..., T, D] -> d/dx, with torch autograd's roundings (see the header)."""
    gf = np.asarray(g, dtype=F32)
    t1 = _round_dtype(gf * np.asarray(cos, F32), dtype)
    t2 = _round_dtype(gf * np.asarray(sin, F32), dtype)
    dx = np.empty_like(gf)
    dx[..., 0::2] = t1[..., 0::2] + t2[..., 1::2]
    dx[..., 1::2] = t1[..., 1::2] - t2[..., 0::2]
    return _round_dtype(dx, dtype)


def head_rmsnorm_backward(x: np.ndarray, dn: np.ndarray, eps: float = 1e-6, dtype: str = "bf16") -> np.ndarray:
    """x [..., D] (the norm's input), dn = d/d head_rmsnorm(x) -> d/dx (see the header)."""
    xf = np.asarray(x, dtype=F32)
    dnf = np.asarray(dn, dtype=F32)
    D = xf.shape[-1]
    ms = np.mean(xf * xf, axis=-1, keepdims=True, dtype=F32)
    r = (F32(1.0) / np.sqrt(ms + F32(eps), dtype=F32)).astype(F32)
    sd = np.sum(dnf * xf, axis=-1, keepdims=True, dtype=F32)
    k = (sd * (r * r * r) / F32(D)).astype(F32)
    return _round_dtype(_round_dtype(dnf * r, dtype) - _round_dtype(xf * k, dtype), dtype)
