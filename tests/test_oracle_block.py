"""CPU: the oracle's RMSNorm and GELU against torch's CPU operators on the same bf16 inputs."""

import numpy as np
import torch

from oracle.block import gelu, rmsnorm
from oracle.e4m3 import f32_to_bf16_bits


def _ulp_diff(a, b):
    ia = f32_to_bf16_bits(np.asarray(a, np.float32)).astype(np.int32)
    ib = f32_to_bf16_bits(np.asarray(b, np.float32)).astype(np.int32)
    return np.abs(ia - ib)


def test_rmsnorm_matches_torch_formula():
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(256, 1024, generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(1024, generator=g)).to(torch.bfloat16)
    eps = 1e-6
    rms = x.float().pow(2).mean(dim=-1, keepdim=True).add(eps).rsqrt()      # base.py:335-338
    want = ((x.float() * rms).to(torch.bfloat16) * w).float().numpy()
    got = rmsnorm(x.float().numpy(), w.float().numpy(), eps)
    d = _ulp_diff(got, want)
    assert d.max() <= 1 and (d > 0).mean() < 1e-3, ((d > 0).mean(), d.max())


def test_rmsnorm_plants_a_dropped_gain_and_fails():
    """A mistake (the gain left out) must be visible to the comparison above."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(8, 64, generator=g).to(torch.bfloat16)
    w = (2 + torch.rand(64, generator=g)).to(torch.bfloat16)
    good = rmsnorm(x.float().numpy(), w.float().numpy())
    bad = rmsnorm(x.float().numpy(), np.ones(64, np.float32))
    assert _ulp_diff(good, bad).max() > 10


def test_gelu_matches_torch_erf_gelu():
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(65536, generator=g) * 4).to(torch.bfloat16)
    want = torch.nn.functional.gelu(x.float()).to(torch.bfloat16).float().numpy()
    got = gelu(x.float().numpy())
    # 1 + erf cancels for negative x: a last-place difference between two fp32 erf implementations
    # (torch's CPU erf is off by up to 5e-4 relative there) flips ~1 % of the bf16 roundings and,
    # below x ~ -3, becomes a large relative but tiny absolute difference; outputs under 1e-4 are
    # compared absolutely.
    big = np.abs(want) > 1e-4
    d = _ulp_diff(got[big], want[big])
    assert d.max() <= 1 and (d > 0).mean() < 0.02, ((d > 0).mean(), d.max())
    assert np.abs(got[~big] - want[~big]).max() < 2e-6
    # closed-form points: gelu(0) = 0, gelu(x) -> x for large x, -> 0 for very negative x
    assert gelu(np.array([0.0, 10.0, -10.0], np.float32)).tolist() == [0.0, 10.0, 0.0]
    # gelu(1) = 0.5 (1 + erf(1 / sqrt 2)) = Phi(1) = 0.8413447...
    assert abs(gelu(np.array([1.0], np.float32))[0] - 0.8413447) < 2 ** -8


def _rope_tables(T, D, base=10000.0):
    """base.py:444-457's tables, built with torch as the reference builds them."""
    inv_freq = 1.0 / (base ** (torch.arange(0, D, 2).float() / D))
    freqs = torch.outer(torch.arange(T).float(), inv_freq)
    return freqs.cos().repeat_interleave(2, dim=-1), freqs.sin().repeat_interleave(2, dim=-1)


def _torch_rotate_half(x):
    x1, x2 = x[..., ::2], x[..., 1::2]
    return torch.stack((-x2, x1), dim=-1).flatten(-2)


def test_head_rmsnorm_and_rope_match_the_reference_expressions_in_torch():
    """oracle.block.head_rmsnorm / rope against base.py:355-357 and :478-483 evaluated by torch's
    CPU operators (a separate implementation) on bf16 and fp32 (B, H, T, D) inputs with the
    model's own cos / sin tables cast to the activations' dtype: the norm within one bf16 ulp in
    a small fraction of values (summation order), RoPE bit for bit."""
    from oracle.block import head_rmsnorm, rope
    g = torch.Generator().manual_seed(3)
    B, H, T, D, eps = 2, 3, 96, 64, 1e-6
    cos32, sin32 = _rope_tables(T, D)
    for dt, name in ((torch.bfloat16, "bf16"), (torch.float32, "f32")):
        x = (torch.randn(B, H, T, D, generator=g) * 2.5).to(dt)
        rms = x.float().pow(2).mean(dim=-1, keepdim=True).add(eps).rsqrt()
        normed = (x.float() * rms).to(dt)
        got_n = head_rmsnorm(x.float().numpy(), eps, name)
        if name == "bf16":
            d = _ulp_diff(got_n, normed.float().numpy())
            assert d.max() <= 1 and (d > 0).mean() < 2e-3, ((d > 0).mean(), d.max())
        else:
            np.testing.assert_allclose(got_n, normed.numpy(), rtol=3e-7, atol=0)
        cos, sin = cos32.to(dt), sin32.to(dt)
        want = (normed * cos + _torch_rotate_half(normed) * sin).float().numpy()
        got = rope(normed.float().numpy(), cos.float().numpy(), sin.float().numpy(), name)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_rope_plants_a_wrong_pair_sign_and_fails():
    """rotate_half with the sign on the wrong half (a plausible slip) must fail the comparison."""
    from oracle.block import rope
    g = torch.Generator().manual_seed(4)
    x = torch.randn(1, 1, 32, 64, generator=g).to(torch.bfloat16)
    cos, sin = (t.to(torch.bfloat16) for t in _rope_tables(32, 64))
    right = (x * cos + _torch_rotate_half(x) * sin).float().numpy()
    bad_rot = torch.stack((x[..., 1::2], -x[..., ::2]), dim=-1).flatten(-2)
    wrong = (x * cos + bad_rot * sin).float().numpy()
    got = rope(x.float().numpy(), cos.float().numpy(), sin.float().numpy(), "bf16")
    assert np.array_equal(got, right) and not np.array_equal(got, wrong)
