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
