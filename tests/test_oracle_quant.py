"""Pins the oracle's quantisation recipes against the reference's formulas run through torch's
own CPU operators (fp8_swa_attention.py:203-205, base.py:198-203, base.py:912-918).

torch is an independent implementation of every op here (its clamp, its bf16 scalar handling,
its division and its e4m3 cast), so a wrong op order, a scale kept in the wrong dtype or a
dropped clamp in the numpy restatement fails these tests.
"""

import numpy as np
import pytest
import torch

from oracle.e4m3 import bf16_bits_to_f32, e4m3_to_f32
from oracle.quant import (fake_quant_e4m3, group_axes, per_tensor_fp8, rowwise_fp8)

E4M3 = torch.float8_e4m3fn


# ---- the reference's expressions, evaluated by torch ------------------------------------

def torch_per_tensor_fp8(x: torch.Tensor, dims=None):
    """fp8_swa_attention.py:203-205 on the CPU (dims=None: whole tensor)."""
    if dims is None:
        amax = x.abs().amax().float().clamp(min=1e-12)
    else:
        amax = x.abs().amax(dim=dims, keepdim=True).float().clamp(min=1e-12)
    scale = amax / 448.0
    q = (x.float() / scale).clamp(-448.0, 448.0).to(E4M3)
    return q.view(torch.uint8).numpy(), scale.numpy()


def torch_fake_quant(x: torch.Tensor, dims=None):
    """base.py:198-203 forward value (x.detach() is irrelevant to the value)."""
    if dims is None:
        amax = x.abs().amax().clamp(min=1e-12)
    else:
        amax = x.abs().amax(dim=dims, keepdim=True).clamp(min=1e-12)
    scale = amax / 448.0
    q = (x / scale).clamp(-448.0, 448.0).to(E4M3)
    dq = q.to(x.dtype) * scale
    return x + (dq - x), q.view(torch.uint8).numpy(), scale


def torch_rowwise(x: torch.Tensor):
    """base.py:912, 917 (_fp8_head activation side; the weight side is the same per row)."""
    scale = x.abs().amax(dim=-1, keepdim=True).float().div(448.0).clamp_min(1e-12)
    return (x.float() / scale).to(E4M3).view(torch.uint8).numpy(), scale.numpy()


# ---- inputs ---------------------------------------------------------------------------------

def near_tie_input(shape, seed, amax=3.0):
    """Values whose quotient by the scale lands within a few fp32 ulps of an e4m3 rounding
    midpoint: the cases where IEEE division vs reciprocal multiply, or a wrong tie rule,
    change the code. One element pins the amax so the scale is known in advance."""
    rng = np.random.default_rng(seed)
    scale = np.float32(np.float32(amax) / np.float32(448.0))
    vals = e4m3_to_f32(np.arange(0, 0x7E, dtype=np.uint8)).astype(np.float64)
    mids = (vals[1:] + vals[:-1]) / 2
    n = int(np.prod(shape))
    m = rng.choice(mids, size=n)
    x = (m * np.float64(scale)).astype(np.float32)
    ulps = rng.integers(-3, 4, size=n).astype(np.int32)
    x = (x.view(np.int32) + ulps).view(np.float32)
    x *= np.where(rng.random(n) < 0.5, -1, 1).astype(np.float32)
    x = x.reshape(shape)
    x.reshape(-1)[0] = np.float32(amax)
    return x


CASES = [
    ("randn", lambda: np.random.default_rng(0).standard_normal((2, 4, 64, 32)).astype(np.float32)),
    ("ties", lambda: near_tie_input((2, 4, 64, 32), 1)),
    ("ties_small", lambda: near_tie_input((2, 4, 64, 32), 2, amax=1e-3)),
    ("tiny", lambda: (np.random.default_rng(3).standard_normal((2, 4, 64, 32)) * 1e-30).astype(np.float32)),
    ("zeros", lambda: np.zeros((2, 4, 64, 32), np.float32)),
]


@pytest.mark.parametrize("name,make", CASES)
@pytest.mark.parametrize("granularity", ["tensor", "head", "bh"])
def test_per_tensor_fp8_matches_reference_formula(name, make, granularity):
    x = make()
    dims = None if granularity == "tensor" else group_axes(4, granularity)
    want_codes, want_scale = torch_per_tensor_fp8(torch.from_numpy(x), dims)
    codes, scale = per_tensor_fp8(x, granularity)
    np.testing.assert_array_equal(codes, want_codes)
    np.testing.assert_array_equal(scale.reshape(np.shape(want_scale)).view(np.uint32),
                                  np.asarray(want_scale, np.float32).view(np.uint32))


@pytest.mark.parametrize("factor", [0.5, 1.0, 3.0, -1.0])
@pytest.mark.parametrize("granularity", ["tensor", "head", "bh"])
def test_per_tensor_fp8_with_a_given_amax_matches_clamp_then_cast(factor, granularity):
    """A given amax (a producer's or a cross-shard maximum, possibly below the data's own |x|
    max) replaces amax in the scale; the reference's clamp(x / s, -448, 448) then bounds the
    quotients, and inf / NaN inputs go through the cast as torch casts them. Checked against
    fp8_swa_attention.py:203-205's expressions in torch with the amax swapped in."""
    x = near_tie_input((2, 4, 64, 32), 7)
    dims = (0, 1, 2, 3) if granularity == "tensor" else group_axes(4, granularity)
    given = (np.max(np.abs(x), axis=dims, keepdims=True) * np.float32(factor)).astype(np.float32)
    x[0, 1, 3, :4] = [np.inf, -np.inf, np.nan, -np.nan]
    x[1, 2, 5, 7] = 1e30
    xt = torch.from_numpy(x)
    scale = torch.from_numpy(given).float().clamp(min=1e-12) / 448.0
    want = (xt.float() / scale).clamp(-448.0, 448.0).to(E4M3).view(torch.uint8).numpy()
    codes, sc = per_tensor_fp8(x, granularity, amax=given.reshape(-1))
    np.testing.assert_array_equal(codes, want)
    np.testing.assert_array_equal(sc.reshape(-1).view(np.uint32), scale.numpy().reshape(-1).view(np.uint32))
    if factor == 0.5:
        assert (codes & 0x7F == 0x7E).sum() > 100        # the clamp is exercised


@pytest.mark.parametrize("name,make", CASES)
@pytest.mark.parametrize("granularity", ["tensor", "head"])
def test_fake_quant_fp32_matches_reference_formula(name, make, granularity):
    x = make()
    dims = None if granularity == "tensor" else group_axes(4, granularity)
    want, want_codes, _ = torch_fake_quant(torch.from_numpy(x), dims)
    out, codes, _ = fake_quant_e4m3(x, "f32", granularity)
    np.testing.assert_array_equal(codes, want_codes)
    np.testing.assert_array_equal(out.view(np.uint32), want.numpy().view(np.uint32))


def _bf16(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(x).to(torch.bfloat16)


@pytest.mark.parametrize("name,make", CASES)
def test_fake_quant_bf16_matches_reference_formula(name, make):
    xb = _bf16(make())
    want, want_codes, want_scale = torch_fake_quant(xb)
    xf = xb.float().numpy()
    out, codes, scale = fake_quant_e4m3(xf, "bf16")
    np.testing.assert_array_equal(codes, want_codes)
    np.testing.assert_array_equal(scale.reshape(()).astype(np.float32), want_scale.float().numpy())
    np.testing.assert_array_equal(out.view(np.uint32), want.float().numpy().view(np.uint32))


def test_fake_quant_bf16_scale_for_every_bf16_amax():
    """The bf16 scale (amax / 448 rounded to bf16) for all 32,640 positive finite bf16 amax
    values, against torch. Covers the eps clamp and every rounding case of the scale."""
    bits = np.arange(1, 0x7F80, dtype=np.uint32).astype(np.uint16)
    amax = bf16_bits_to_f32(bits)
    t = torch.from_numpy(amax).to(torch.bfloat16)
    want = (t.clamp(min=1e-12) / 448.0).float().numpy()
    from oracle.quant import fake_quant_scale
    got = np.array([fake_quant_scale(np.array([a], np.float32), "bf16")[0] for a in amax[:64]])
    np.testing.assert_array_equal(got, want[:64])
    # vectorised over the rest: the scale is an elementwise function of amax
    eps = np.float32(torch.tensor(1e-12).to(torch.bfloat16).float().item())
    from oracle.e4m3 import round_bf16
    a = np.where(amax < eps, eps, amax)
    got_all = round_bf16((a / np.float32(448.0)).astype(np.float32))
    np.testing.assert_array_equal(got_all, want)


@pytest.mark.parametrize("name,make", CASES[:4])
def test_rowwise_matches_fp8_head_formula(name, make):
    x = make().reshape(-1, 32)
    want_codes, want_scale = torch_rowwise(torch.from_numpy(x))
    codes, scale = rowwise_fp8(x)
    np.testing.assert_array_equal(codes, want_codes)
    np.testing.assert_array_equal(scale, want_scale)


def test_rowwise_bf16_rows_with_negative_skew():
    """base.py:906-908 regression: the scale comes from |x|, not max(x)."""
    x = (np.random.default_rng(5).standard_normal((16, 64)) - 2.5).astype(np.float32)
    xb = _bf16(x)
    want_codes, want_scale = torch_rowwise(xb)
    codes, scale = rowwise_fp8(xb.float().numpy())
    np.testing.assert_array_equal(codes, want_codes)
    np.testing.assert_array_equal(scale, want_scale)
    assert np.all(scale > 0)


def test_nan_propagates_like_torch():
    x = np.random.default_rng(6).standard_normal((1, 2, 8, 16)).astype(np.float32)
    x[0, 1, 3, 5] = np.nan
    want_codes, _ = torch_per_tensor_fp8(torch.from_numpy(x), (0, 2, 3))
    codes, scale = per_tensor_fp8(x, "head")
    np.testing.assert_array_equal(codes, want_codes)
    assert np.isnan(scale[0, 1, 0, 0]) and not np.isnan(scale[0, 0, 0, 0])


# ---- the reference's own sim tests (tests/test_fp8_attention_sim.py), restated on the oracle --

def test_forward_is_actually_quantized():                     # :23-29
    x = (np.random.default_rng(0).standard_normal((2, 2, 32, 16)) * 0.5).astype(np.float32)
    y, _, _ = fake_quant_e4m3(x, "f32")
    assert not np.array_equal(y, x)
    assert np.abs(y - x).mean() > 0


def test_quantization_error_is_far_above_bf16():              # :55-66
    from oracle.e4m3 import round_bf16
    x = np.random.default_rng(0).standard_normal((4096, 64)).astype(np.float32)
    y, _, _ = fake_quant_e4m3(x, "f32")
    e_fp8 = np.abs(y - x).mean()
    e_bf16 = np.abs(round_bf16(x) - x).mean()
    assert e_fp8 > 5 * e_bf16


def test_handles_all_zero_input_without_nan():                # :69-74
    x = np.zeros((2, 2, 8, 16), np.float32)
    y, _, _ = fake_quant_e4m3(x, "f32")
    assert np.isfinite(y).all() and np.array_equal(y, x)
