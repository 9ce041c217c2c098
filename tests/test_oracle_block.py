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


def test_rope_and_head_rmsnorm_backward_match_torch_autograd():
    """oracle.block.rope_backward / head_rmsnorm_backward against torch's CPU autograd of the
    reference's expressions (base.py:355-357, :478-483) on bf16 (B, H, T, D) tensors: RoPE's
    gradient bit for bit; the norm's within one bf16 ulp in a small fraction of values (the fp32
    sums' order)."""
    from oracle.block import head_rmsnorm_backward, rope_backward
    g = torch.Generator().manual_seed(6)
    B, H, T, D, eps = 2, 3, 80, 64, 1e-6
    cos, sin = (t.to(torch.bfloat16) for t in _rope_tables(T, D))
    x = (torch.randn(B, H, T, D, generator=g) * 2.0).to(torch.bfloat16).requires_grad_(True)
    gy = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16)
    n = (x.float() * x.float().pow(2).mean(dim=-1, keepdim=True).add(eps).rsqrt()).to(torch.bfloat16)
    n.retain_grad()
    y = n * cos + _torch_rotate_half(n) * sin
    y.backward(gy)
    dn = rope_backward(gy.float().numpy(), cos.float().numpy(), sin.float().numpy(), "bf16")
    np.testing.assert_array_equal(dn.view(np.uint32), n.grad.float().numpy().view(np.uint32))
    dx = head_rmsnorm_backward(x.detach().float().numpy(), dn, eps, "bf16")
    d = _ulp_diff(dx, x.grad.float().numpy())
    assert d.max() <= 1 and (d > 0).mean() < 5e-3, ((d > 0).mean(), d.max())


def test_rope_backward_is_the_adjoint_and_norm_backward_the_derivative():
    """Independent of torch: in float64 terms, <rope(x), g> = <x, rope_backward(g)> (the rotation's
    adjoint; a swapped pair or sign fails it), and head_rmsnorm_backward against central finite
    differences of head_rmsnorm computed in float64 (a dropped r^3 term or a missing 1/D fails it)."""
    from oracle.block import head_rmsnorm_backward, rope_backward
    rng = np.random.default_rng(7)
    T, D = 16, 32
    cos32, sin32 = (t.numpy() for t in _rope_tables(T, D))
    x = rng.standard_normal((T, D)).astype(np.float32)
    gy = rng.standard_normal((T, D)).astype(np.float32)
    rot = np.empty_like(x, dtype=np.float64)
    rot[:, 0::2], rot[:, 1::2] = -x[:, 1::2], x[:, 0::2]
    lhs = float(np.sum((x * cos32.astype(np.float64) + rot * sin32) * gy))
    rhs = float(np.sum(x.astype(np.float64) * rope_backward(gy, cos32, sin32, "f32")))
    assert abs(lhs - rhs) <= 1e-4 * (abs(lhs) + 1.0)

    eps = 1e-6
    xr = rng.standard_normal((4, D)).astype(np.float64) * 1.5
    dn = rng.standard_normal((4, D))

    def f(v):
        return np.sum(dn * v / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + eps))
    fd = np.zeros_like(xr)
    h = 1e-6
    for i in range(xr.shape[0]):
        for j in range(D):
            e = np.zeros_like(xr)
            e[i, j] = h
            fd[i, j] = (f(xr + e) - f(xr - e)) / (2 * h)
    got = head_rmsnorm_backward(xr.astype(np.float32), dn.astype(np.float32), eps, "f32")
    np.testing.assert_allclose(got, fd, rtol=2e-4, atol=2e-5)


def test_rmsnorm_backward_matches_torch_autograd():
    """oracle.block.rmsnorm_backward against torch's CPU autograd of base.py:337-338 on bf16 rows
    and a bf16 gain: dx within one bf16 ulp in a small fraction of values (fp32 sums' order), dw
    (a sum over 512 rows) within one ulp."""
    from oracle.block import rmsnorm_backward
    g = torch.Generator().manual_seed(12)
    x = (torch.randn(512, 320, generator=g) * 2).to(torch.bfloat16).requires_grad_(True)
    w = (1 + 0.2 * torch.randn(320, generator=g)).to(torch.bfloat16).requires_grad_(True)
    dh = torch.randn(512, 320, generator=g).to(torch.bfloat16)
    eps = 1e-6
    rms = x.float().pow(2).mean(dim=-1, keepdim=True).add(eps).rsqrt()
    ((x.float() * rms).to(torch.bfloat16) * w).backward(dh)
    dx, dw = rmsnorm_backward(x.detach().float().numpy(), w.detach().float().numpy(), dh.float().numpy(), eps)
    d = _ulp_diff(dx, x.grad.float().numpy())
    assert d.max() <= 1 and (d > 0).mean() < 5e-3, ((d > 0).mean(), d.max())
    assert _ulp_diff(dw, w.grad.float().numpy()).max() <= 1


def test_rmsnorm_backward_is_the_derivative():
    """Independent of torch: rmsnorm_backward (bf16 roundings at every step, so the check is
    relative) against central finite differences of sum(dh * x r w) in float64: relative error of
    dx and dw below 2 %, which the norm's r^3 term dropped fails."""
    from oracle.block import rmsnorm_backward
    rng = np.random.default_rng(13)
    x = rng.standard_normal((6, 64)).astype(np.float32)
    w = (1 + 0.3 * rng.standard_normal(64)).astype(np.float32)
    dh = rng.standard_normal((6, 64)).astype(np.float32)
    eps = 1e-6

    def f(xv, wv):
        xv = xv.astype(np.float64)
        return float(np.sum(dh * xv / np.sqrt(np.mean(xv * xv, axis=-1, keepdims=True) + eps) * wv))
    h = 1e-6
    fx = np.zeros_like(x, dtype=np.float64)
    for i in range(x.shape[0]):
        for j in range(x.shape[1]):
            e = np.zeros_like(x, dtype=np.float64)
            e[i, j] = h
            fx[i, j] = (f(x + e, w) - f(x - e, w)) / (2 * h)
    fw = np.array([(f(x, w + h * np.eye(64)[j]) - f(x, w - h * np.eye(64)[j])) / (2 * h) for j in range(64)])
    dx, dw = rmsnorm_backward(x, w, dh, eps)
    assert np.linalg.norm(dx - fx) / np.linalg.norm(fx) < 0.02
    assert np.linalg.norm(dw - fw) / np.linalg.norm(fw) < 0.02
    n = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    dropped = dh * w / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    assert np.linalg.norm(dropped - fx) / np.linalg.norm(fx) > 0.1 and n.shape == x.shape


def test_swiglu_and_backward_match_torch_autograd():
    """oracle.block.swiglu / swiglu_backward against torch's CPU silu, product and autograd on bf16
    values: within one bf16 ulp in a small fraction of values (torch's CPU exp)."""
    from oracle.block import swiglu, swiglu_backward
    g = torch.Generator().manual_seed(14)
    gate = (torch.randn(64, 1024, generator=g) * 3).to(torch.bfloat16).requires_grad_(True)
    up = (torch.randn(64, 1024, generator=g) * 2).to(torch.bfloat16).requires_grad_(True)
    dh = torch.randn(64, 1024, generator=g).to(torch.bfloat16)
    h = torch.nn.functional.silu(gate) * up
    h.backward(dh)
    got = swiglu(gate.detach().float().numpy(), up.detach().float().numpy())
    d = _ulp_diff(got, h.detach().float().numpy())
    assert d.max() <= 1 and (d > 0).mean() < 5e-3, ((d > 0).mean(), d.max())
    dg, du = swiglu_backward(gate.detach().float().numpy(), up.detach().float().numpy(), dh.float().numpy())
    for a, b in ((dg, gate.grad), (du, up.grad)):
        d = _ulp_diff(a, b.float().numpy())
        assert d.max() <= 1 and (d > 0).mean() < 5e-3, ((d > 0).mean(), d.max())


def test_swiglu_closed_forms_and_derivative():
    """silu(0) = 0, silu(x) -> x for large x and -> 0 for very negative x; d silu / dx at 0 is 1/2;
    swiglu_backward against central differences of swiglu's float64 form (a sign slip in the
    (1 - sig) term fails it)."""
    from oracle.block import swiglu, swiglu_backward
    one = np.ones(3, np.float32)
    got = swiglu(np.array([0.0, 20.0, -30.0], np.float32), one)
    assert got[0] == 0.0 and got[1] == 20.0 and -1e-11 < got[2] < 0.0       # -30 / (1 + e^30)
    dg, du = swiglu_backward(np.zeros(1, np.float32), np.ones(1, np.float32), np.ones(1, np.float32))
    assert dg[0] == 0.5 and du[0] == 0.0
    rng = np.random.default_rng(15)
    gv = rng.standard_normal(256) * 2
    uv = rng.standard_normal(256)

    def sw(x):
        return x / (1 + np.exp(-x))
    h = 1e-6
    fd_g = (sw(gv + h) - sw(gv - h)) / (2 * h) * uv
    dg, du = swiglu_backward(gv.astype(np.float32), uv.astype(np.float32), np.ones(256, np.float32))
    assert np.abs(dg - fd_g).max() < 2e-2 * (np.abs(fd_g).max() + 1)
    assert np.abs(du - sw(gv)).max() < 2e-2 * (np.abs(sw(gv)).max() + 1)
    sig = 1 / (1 + np.exp(-gv))
    wrong = sig * (1 - gv * (1 - sig)) * uv
    assert np.abs(wrong - fd_g).max() > 0.1

