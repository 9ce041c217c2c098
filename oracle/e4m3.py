"""Bit-level codecs: fp32 -> e4m3fn, e4m3fn -> fp32, fp32 -> bf16 (RNE), bf16 -> fp32.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates the casts the reference path uses:
  - ``Tensor.to(torch.float8_e4m3fn)`` (fp8_swa_attention.py:205, base.py:200, base.py:917-918):
    OCP FP8 E4M3 "fn" format: 1 sign, 4 exponent (bias 7), 3 mantissa bits, no infinities,
    S.1111.111 is NaN, max finite 448 = S.1111.110. Round-to-nearest-even, NOT saturating:
    |x| > 464 (the midpoint between 448 and the next would-be value 480) becomes NaN, which is
    why the reference clamps to +-448 before casting. NaN and +-inf map to sign|0x7F.
  - ``Tensor.to(torch.bfloat16)``: round-to-nearest-even on the top 16 bits, NaN -> 0x7FC0|sign.

Pinned by tests/test_oracle_e4m3.py:
  - exhaustively over all 65,536 bf16 bit patterns against torch's CPU cast (a library routine);
  - over every fp32 value within +-4 ulp of every e4m3 rounding midpoint and boundary
    (the adversarial set where a wrong tie rule or exponent offset would show), against torch;
  - known-answer values of the OCP spec (448 -> 0x7E, 464 -> 0x7E, 2^-9 -> 0x01, ...).
"""

from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0          # fp8_swa_attention.py:92
E4M3_NAN = 0x7F


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    """fp32 -> e4m3fn code (uint8), RNE, non-saturating. Accepts any float32 array."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    sign = ((u >> 24) & 0x80).astype(np.uint32)
    a = u & np.uint32(0x7FFFFFFF)
    # Normal e4m3 range (|x| >= 2^-6): move the fp32 exponent bias (127) to e4m3's (7) and
    # round the 23-bit fraction to 3 bits, ties to even. Carries ripple into the exponent.
    r = a.astype(np.int64) - (120 << 23)
    lsb = (r >> 20) & 1
    normal = (r + 0x7FFFF + lsb) >> 20
    # Anything that rounds past 0x7E (>= 464 rounds up to 480, or inf / NaN) is NaN.
    normal = np.minimum(normal, E4M3_NAN)
    # Subnormal e4m3 range (|x| < 2^-6): the value is an integer multiple of 2^-9, 0..8,
    # round-half-even of |x| * 2^9 (exact scaling by a power of two).
    is_normal = a >= 0x3C800000
    small = np.where(is_normal, np.uint32(0), a).view(np.float32).astype(np.float64)
    sub = np.rint(small * 512.0).astype(np.int64)
    code = np.where(is_normal, normal, sub).astype(np.uint32)
    return (code | sign).astype(np.uint8)


_E4M3_TABLE = None


def e4m3_to_f32(c: np.ndarray) -> np.ndarray:
    """e4m3fn code (uint8) -> fp32 (exact). 0x7F / 0xFF decode to NaN."""
    global _E4M3_TABLE
    if _E4M3_TABLE is None:
        codes = np.arange(256, dtype=np.uint32)
        s = np.where(codes & 0x80, -1.0, 1.0)
        e = (codes >> 3) & 0xF
        m = codes & 0x7
        val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e.astype(np.float64) - 7.0))
        val = s * val
        val[(codes & 0x7F) == 0x7F] = np.nan
        _E4M3_TABLE = val.astype(np.float32)
    return _E4M3_TABLE[np.asarray(c, dtype=np.uint8)]


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> fp32 (exact)."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round-to-nearest-even; NaN -> 0x7FC0 with the input sign."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    rounded = ((u + 0x7FFF + lsb) >> 16).astype(np.uint32)
    nan = np.isnan(x)
    rounded = np.where(nan, (u.astype(np.uint32) >> 16) & 0x8000 | 0x7FC0, rounded)
    return rounded.astype(np.uint16)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bf16 value, returned as fp32 (i.e. ``x.to(bf16).float()``)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))
