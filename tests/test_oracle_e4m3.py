"""Pins the oracle's e4m3 / bf16 codecs against torch's CPU casts (library routines)."""

import numpy as np
import pytest
import torch

from oracle.e4m3 import bf16_bits_to_f32, e4m3_to_f32, f32_to_bf16_bits, f32_to_e4m3

E4M3 = torch.float8_e4m3fn


def torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(E4M3).view(torch.uint8).numpy()


def test_all_bf16_patterns_cast_like_torch():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = bf16_bits_to_f32(bits)
    np.testing.assert_array_equal(f32_to_e4m3(x), torch_e4m3(x))


def _boundaries() -> np.ndarray:
    """Every e4m3 value and every midpoint between neighbours, both signs, plus the
    overflow / underflow edges: the places a wrong rounding rule shows."""
    vals = e4m3_to_f32(np.arange(256, dtype=np.uint8)).astype(np.float64)
    vals = np.unique(vals[np.isfinite(vals)])
    mids = (vals[1:] + vals[:-1]) / 2
    extra = np.array([464.0, 480.0, 512.0, 2.0 ** -10, 2.0 ** -11, 1.5 * 2.0 ** -10,
                      3.4e38, 1e-40, 2.0 ** -126, 2.0 ** -149])
    pts = np.concatenate([vals, mids, extra, -vals, -mids, -extra]).astype(np.float32)
    return pts


def test_fp32_within_4ulp_of_every_boundary_cast_like_torch():
    pts = _boundaries()
    u = pts.view(np.int32).astype(np.int64)
    offs = np.arange(-4, 5, dtype=np.int64)
    cand = (u[:, None] + offs[None, :]).reshape(-1)
    cand = cand[(cand >= -(2 ** 31)) & (cand < 2 ** 31)].astype(np.int32)
    x = cand.view(np.float32)
    np.testing.assert_array_equal(f32_to_e4m3(x), torch_e4m3(x))


def test_random_fp32_bit_patterns_cast_like_torch():
    rng = np.random.default_rng(0)
    x = rng.integers(0, 2 ** 32, size=2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    np.testing.assert_array_equal(f32_to_e4m3(x), torch_e4m3(x))


@pytest.mark.parametrize("value,code", [
    (448.0, 0x7E), (464.0, 0x7E), (465.0, 0x7F), (-448.0, 0xFE), (2.0 ** -9, 0x01),
    (2.0 ** -10, 0x00), (1.5 * 2.0 ** -10, 0x01), (1.0625, 0x38), (1.0, 0x38), (-0.0, 0x80),
    (float("inf"), 0x7F), (float("-inf"), 0xFF), (float("nan"), 0x7F), (2.0 ** -6, 0x08),
])
def test_known_answers(value, code):
    assert int(f32_to_e4m3(np.array([value], np.float32))[0]) == code


def test_decode_all_codes_like_torch():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(E4M3).float().numpy()
    got = e4m3_to_f32(codes)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    np.testing.assert_array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))


def test_decode_then_encode_is_identity():
    codes = np.arange(256, dtype=np.uint8)
    finite = (codes & 0x7F) != 0x7F
    np.testing.assert_array_equal(f32_to_e4m3(e4m3_to_f32(codes[finite])), codes[finite])


def test_bf16_rounding_like_torch():
    rng = np.random.default_rng(1)
    x = rng.integers(0, 2 ** 32, size=1_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = f32_to_bf16_bits(x)
    nan = np.isnan(x)
    np.testing.assert_array_equal(got[~nan], want[~nan])
    # NaN stays NaN (torch's payload choice is not part of any contract on this path).
    assert np.all(np.isnan(bf16_bits_to_f32(got[nan])))
