"""Pins the oracle of the bf16 sliding-window attention training op (forward + log-sum-exp +
backward): dense reference, a direct log-sum-exp, torch autograd, finite differences, and the
closed-form gradient identities."""

import math

import numpy as np
import pytest
import torch

from oracle.swa import swa_dense
from oracle.swa_grad import swa_backward, swa_forward_lse


def rnd(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def torch_dense(q, k, v, W):
    T, D = q.shape[-2], q.shape[-1]
    s = (q @ k.transpose(-1, -2)) / math.sqrt(D)
    i = torch.arange(T)
    keep = (i[:, None] >= i[None, :]) & ((i[:, None] - i[None, :]) < W)
    return torch.softmax(s.masked_fill(~keep, float("-inf")), -1) @ v


CASES = [(1, 2, 70, 16, 9), (2, 1, 300, 32, 64), (1, 1, 130, 64, 1000), (1, 2, 257, 8, 256)]


@pytest.mark.parametrize("B,H,T,D,W", CASES)
def test_forward_and_lse(B, H, T, D, W):
    q, k, v = (rnd((B, H, T, D), s) for s in (1, 2, 3))
    out, lse = swa_forward_lse(q, k, v, W, chunk=64)
    np.testing.assert_allclose(out, swa_dense(q, k, v, W), rtol=2e-5, atol=2e-5)
    # L_i = log sum_{j valid} exp(q_i . k_j / sqrt(D)), taken row by row
    for b, h, i in [(0, 0, 0), (B - 1, H - 1, T - 1), (0, H - 1, T // 2)]:
        js = [j for j in range(T) if j <= i and i - j < W]
        s = np.array([q[b, h, i] @ k[b, h, j] for j in js]) / math.sqrt(D)
        assert abs(lse[b, h, i] - np.log(np.exp(s).sum())) < 1e-12


@pytest.mark.parametrize("B,H,T,D,W", CASES)
def test_gradients_match_autograd(B, H, T, D, W):
    q, k, v, do = (rnd((B, H, T, D), s) for s in (4, 5, 6, 7))
    out, lse = swa_forward_lse(q, k, v, W, chunk=64)
    dq, dk, dv = swa_backward(q, k, v, out, lse, do, W, chunk=64)
    tq, tk, tv = (torch.tensor(t, requires_grad=True) for t in (q, k, v))
    torch_dense(tq, tk, tv, W).backward(torch.tensor(do))
    for got, want in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad)):
        np.testing.assert_allclose(got, want.numpy(), rtol=1e-9, atol=1e-10)


def test_gradients_match_finite_differences():
    B, H, T, D, W = 1, 1, 12, 4, 5
    q, k, v, do = (rnd((B, H, T, D), s) for s in (8, 9, 10, 11))
    out, lse = swa_forward_lse(q, k, v, W)
    grads = swa_backward(q, k, v, out, lse, do, W)
    eps = 1e-6
    for which, g in enumerate(grads):
        for idx in [(0, 0, 0, 0), (0, 0, 5, 2), (0, 0, 11, 3), (0, 0, 7, 1)]:
            xs = [q.copy(), k.copy(), v.copy()]
            xs[which][idx] += eps
            fp = np.sum(do * swa_forward_lse(*xs, W)[0])
            xs[which][idx] -= 2 * eps
            fm = np.sum(do * swa_forward_lse(*xs, W)[0])
            assert abs((fp - fm) / (2 * eps) - g[idx]) < 1e-7, (which, idx)


@pytest.mark.parametrize("B,H,T,D,W", CASES)
def test_closed_form_identities(B, H, T, D, W):
    q, k, v, do = (rnd((B, H, T, D), s) for s in (12, 13, 14, 15))
    out, lse = swa_forward_lse(q, k, v, W, chunk=64)
    dq, dk, dv = swa_backward(q, k, v, out, lse, do, W, chunk=64)
    np.testing.assert_allclose(dk.sum(axis=2), 0.0, atol=1e-9)
    np.testing.assert_allclose(dv.sum(axis=2), do.sum(axis=2), rtol=1e-10, atol=1e-10)


def test_window_one():
    q, k, v, do = (rnd((1, 2, 40, 16), s) for s in (16, 17, 18, 19))
    out, lse = swa_forward_lse(q, k, v, 1)
    np.testing.assert_array_equal(out, v)
    np.testing.assert_allclose(lse, np.sum(q * k, axis=-1) / 4.0, rtol=1e-13)
    dq, dk, dv = swa_backward(q, k, v, out, lse, do, 1)
    np.testing.assert_allclose(dq, 0.0, atol=1e-12)
    np.testing.assert_allclose(dk, 0.0, atol=1e-12)
    np.testing.assert_allclose(dv, do, rtol=1e-13)


def test_dropped_delta_is_caught():
    """The identity sum_j dK_j = 0 fails for a backward that forgets the Delta term."""
    q, k, v, do = (rnd((1, 1, 64, 8), s) for s in (20, 21, 22, 23))
    out, lse = swa_forward_lse(q, k, v, 16)
    _, dk, _ = swa_backward(q, k, v, np.zeros_like(out), lse, do, 16)   # Delta = 0
    assert np.abs(dk.sum(axis=2)).max() > 1e-3
