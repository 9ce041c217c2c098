"""Pins the attention oracle: mask truth table, brute force, library routines, invariants."""

import numpy as np
import pytest
import torch

from oracle.e4m3 import e4m3_to_f32
from oracle.quant import per_tensor_fp8
from oracle.swa import (attention_flops, causal_window_mask, fp8_swa_attention, fp8_swa_simulate,
                        in_window_pairs, swa_banded, swa_dense)


def rnd(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def test_local_causal_mask_truth_table():
    """tests/test_causal.py:10-21 of the reference, verbatim expectation."""
    expected = np.array([
        [True, False, False, False, False],
        [True, True, False, False, False],
        [False, True, True, False, False],
        [False, False, True, True, False],
        [False, False, False, True, True],
    ])
    np.testing.assert_array_equal(causal_window_mask(5, 2), expected)


def brute_force(q, k, v, W):
    """Explicit loops in float64."""
    B, H, T, D = q.shape
    out = np.zeros((B, H, T, D))
    for b in range(B):
        for h in range(H):
            for i in range(T):
                js = [j for j in range(T) if j <= i and i - j < W]
                s = np.array([np.dot(q[b, h, i].astype(np.float64), k[b, h, j]) / np.sqrt(D) for j in js])
                p = np.exp(s - s.max())
                p /= p.sum()
                out[b, h, i] = sum(pj * v[b, h, j].astype(np.float64) for pj, j in zip(p, js))
    return out


@pytest.mark.parametrize("T,W", [(9, 3), (16, 1), (12, 12), (12, 40)])
def test_dense_matches_float64_brute_force(T, W):
    q, k, v = rnd((1, 2, T, 8), 0), rnd((1, 2, T, 8), 1), rnd((1, 2, T, 8), 2)
    np.testing.assert_allclose(swa_dense(q, k, v, W), brute_force(q, k, v, W), rtol=1e-5, atol=1e-5)


def test_full_window_equals_torch_causal_sdpa():
    q, k, v = rnd((2, 3, 64, 16), 3), rnd((2, 3, 64, 16), 4), rnd((2, 3, 64, 16), 5)
    want = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), is_causal=True).numpy()
    np.testing.assert_allclose(swa_dense(q, k, v, 64), want, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(swa_dense(q, k, v, 10_000), want, rtol=1e-5, atol=1e-5)


def test_window_one_returns_v():
    q, k, v = rnd((1, 2, 32, 16), 6), rnd((1, 2, 32, 16), 7), rnd((1, 2, 32, 16), 8)
    np.testing.assert_array_equal(swa_dense(q, k, v, 1), v)


@pytest.mark.parametrize("T,W,chunk", [(100, 7, 16), (256, 64, 64), (200, 300, 32)])
def test_banded_equals_dense(T, W, chunk):
    q, k, v = rnd((1, 2, T, 16), 9), rnd((1, 2, T, 16), 10), rnd((1, 2, T, 16), 11)
    np.testing.assert_allclose(swa_banded(q, k, v, W, chunk=chunk), swa_dense(q, k, v, W),
                               rtol=1e-5, atol=1e-6)


def test_rows_ignore_keys_outside_band_and_slices_are_independent():
    T, W = 96, 16
    q, k, v = rnd((2, 2, T, 16), 12), rnd((2, 2, T, 16), 13), rnd((2, 2, T, 16), 14)
    base = swa_dense(q, k, v, W)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, :40] += 5.0            # keys 0..39 are outside the band of rows >= 40 + W - 1 = 55
    v2[:, :, :40] -= 3.0
    other = swa_dense(q, k2, v2, W)
    np.testing.assert_array_equal(other[:, :, 55:], base[:, :, 55:])
    q3 = q.copy()
    q3[1, 0] *= -2                  # one (b, h) slice changed, the others untouched
    third = swa_dense(q3, k, v, W)
    mask = np.ones((2, 2), bool)
    mask[1, 0] = False
    np.testing.assert_array_equal(third[mask], base[mask])


@pytest.mark.parametrize("block_n", [16, 32, 64])
def test_simulator_without_p_quant_equals_dense_on_dequantised_inputs(block_n):
    B, H, T, D, W = 1, 2, 160, 32, 48
    q, k, v = rnd((B, H, T, D), 15), rnd((B, H, T, D), 16), rnd((B, H, T, D), 17)
    q8, qs = per_tensor_fp8(q)
    k8, ks = per_tensor_fp8(k)
    v8, vs = per_tensor_fp8(v)
    deq = [(e4m3_to_f32(c) * s).astype(np.float32) for c, s in ((q8, qs), (k8, ks), (v8, vs))]
    sim = fp8_swa_simulate(q8, k8, v8, qs, ks, vs, W, block_n=block_n, quantize_p=False, chunk=64)
    np.testing.assert_allclose(sim, swa_dense(*deq, W), rtol=2e-4, atol=2e-5)


def test_simulator_error_vs_fp32_is_in_the_reference_band():
    """fp8_swa_attention.py:48-57: FP8 Q,K,V,P mean relative error ~0.051 vs fp32. The oracle
    must land in that band (a dropped P quantisation would give ~0.035, a dropped Q/K/V one
    ~0.026); measured at a smaller shape, so the band is wide but excludes both."""
    B, H, T, D, W = 1, 4, 1024, 64, 512
    q, k, v = rnd((B, H, T, D), 18), rnd((B, H, T, D), 19), rnd((B, H, T, D), 20)
    ref = swa_banded(q, k, v, W)
    out = fp8_swa_attention(q, k, v, W)
    rel = np.abs(out - ref).mean() / np.abs(ref).mean()
    assert 0.040 < rel < 0.065, rel


def test_window_nonpositive_gives_zeros():
    q, k, v = rnd((1, 1, 40, 16), 21), rnd((1, 1, 40, 16), 22), rnd((1, 1, 40, 16), 23)
    assert np.array_equal(fp8_swa_attention(q, k, v, 0), np.zeros_like(q))


def test_flop_count_closed_form():
    # In-window pair counts of the benchmark configs: C1 (B1 H8 T1024 W256), C3 (B4 H16 T8192
    # W1024), C4 (B1 H16 T32768 W4096); FLOPs = 4 * D * pairs.
    assert in_window_pairs(1024, 256) * 8 == 1_836_032
    assert in_window_pairs(8192, 1024) * 64 == 503_349_248
    assert in_window_pairs(32768, 4096) * 16 == 2_013_298_688
    assert attention_flops(4, 16, 8192, 64, 1024) == 4 * 64 * 503_349_248
    assert attention_flops(1, 16, 32768, 64, 4096) == 4 * 64 * 2_013_298_688
    T, W = 37, 11
    assert in_window_pairs(T, W) == int(causal_window_mask(T, W).sum())


def test_p_code_flip_marks_only_values_near_an_e4m3_boundary():
    """The e4m3 values 176 and 192 have their rounding boundary at 184: 184.023 (the value the
    gfx950 MFMA rounded the other way at D = 128) flips by 16 when the value may move 2e-4, not
    when it may move 1e-5; 180 never flips at 2e-4; 448 stays in range."""
    from oracle.swa import _p_code_flip
    x = np.array([184.023, 184.023, 180.0, 448.0, 0.0], np.float32)
    rel = np.array([2e-4, 1e-5, 2e-4, 1e-3, 1e-3])
    np.testing.assert_array_equal(_p_code_flip(x, rel), [16.0, 0.0, 0.0, 0.0, 0.0])


def test_mfma_allowance_covers_score_errors_within_the_bound():
    """Planted errors: every raw dot product moved by up to its bound (2^-10 of its largest
    |product|, random sign) changes the simulator's output by no more than the allowance the
    unperturbed run reports (plus the fp32-level change of l and the rescales, far below it); with
    no error allowed the allowance is zero."""
    from oracle.quant import per_tensor_fp8
    from oracle.swa import fp8_swa_simulate
    rng = np.random.default_rng(5)
    B, H, T, D, W = 1, 1, 384, 64, 160
    q, k, v = (rng.standard_normal((B, H, T, D)).astype(np.float32) * 2.5 for _ in range(3))
    c = [per_tensor_fp8(t, "bh") for t in (q, k, v)]
    args = (c[0][0], c[1][0], c[2][0], c[0][1], c[1][1], c[2][1], W)
    out, allow = fp8_swa_simulate(*args, mfma_rel_err=2.0 ** -10, chunk=128)
    assert np.array_equal(out, fp8_swa_simulate(*args, chunk=128))
    assert (allow > 0).any()
    _, zero = fp8_swa_simulate(*args, mfma_rel_err=0.0, chunk=128)
    assert not zero.any()

    def perturb(s, qa, ka):
        pmax = (np.abs(qa)[:, None, :] * np.abs(ka)[None, :, :]).max(axis=2)
        return s + rng.uniform(-1.0, 1.0, s.shape) * 2.0 ** -10 * pmax

    for _ in range(3):
        moved = fp8_swa_simulate(*args, chunk=128, score_perturb=perturb)
        d = np.abs(moved.astype(np.float64) - out)
        assert (d <= allow + 2e-3 * np.abs(out).max()).all(), float((d - allow).max())
    # the planted errors do flip codes: without the allowance some element moves further
    assert (np.abs(moved.astype(np.float64) - out) > 1e-3 * np.abs(out).max()).any()
