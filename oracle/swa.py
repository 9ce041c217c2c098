"""Causal sliding-window attention: mask, dense/banded fp32 references, FP8 kernel simulator.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

``causal_window_mask``   base.py:418-423 -- valid(i, j) <=> j <= i and i - j < W.
``swa_dense``            fp8_swa_attention.py:262-273 ``reference_swa_attention``: fp32
                         softmax(mask(Q K^T / sqrt(D))) V.  O(T^2): small T only.
``swa_banded``           the same mathematics chunked by query block, so that only the keys in
                         the band [i - W + 1, i] are materialised: O(T * W) memory, usable at
                         T = 8192 / 32768.
``fp8_swa_simulate``     the FP8 kernel's blockwise algorithm, fp8_swa_attention.py:129-192, on
                         e4m3 codes: per key block of ``block_n`` keys,
                           S = dot(q8, k8) * qk_scale ; masked -> -inf
                           m_new = max(m, rowmax S) ; m_safe = 0 if m_new == -inf
                           p = exp(S - m_safe) ; masked -> 0
                           alpha = exp(m - m_safe) (0 when m == -inf)
                           l = l * alpha + sum(p) ; acc = acc * alpha + e4m3(p * 448) @ v8
                         and finally acc * (v_scale / 448) / (l or 1).
                         With per-head / per-(b,h) scales the scalars become per-slice values.
                         ``quantize_p=False`` skips the e4m3 rounding of p (then it must equal
                         the dense reference on dequantised inputs up to fp32 rounding).
                         ``mfma_rel_err`` also returns, per output element, how far P codes that
                         sit within the hardware dot product's error of an e4m3 rounding
                         boundary can move it (the comparison with an MFMA kernel accepts either
                         rounding of those codes).
``fp8_swa_attention``    quantise Q/K/V (``quant.per_tensor_fp8`` at a granularity) then simulate:
                         the FP8-simulated path end to end.

Pinned by tests/test_oracle_swa.py: the 5x5 mask truth table of tests/test_causal.py:10-21;
float64 brute force on tiny shapes; W >= T equals torch's causal scaled_dot_product_attention
(a library routine); W = 1 returns V exactly; banded == dense; the simulator without
P-quantisation equals the dense reference on the dequantised inputs; rows do not depend on keys
outside their band; (b, h) slices are independent.
"""

from __future__ import annotations

import numpy as np

from .e4m3 import E4M3_MAX, e4m3_to_f32, f32_to_e4m3
from .quant import per_tensor_fp8

F32 = np.float32


def causal_window_mask(T: int, window: int | None) -> np.ndarray:
    idx = np.arange(T)
    mask = idx[:, None] >= idx[None, :]
    if window is not None:
        mask &= (idx[:, None] - idx[None, :]) < window
    return mask


def _softmax_rows(s: np.ndarray) -> np.ndarray:
    m = np.max(s, axis=-1, keepdims=True)
    m = np.where(np.isneginf(m), 0.0, m)
    e = np.exp(s - m)
    den = np.sum(e, axis=-1, keepdims=True)
    with np.errstate(invalid="ignore", divide="ignore"):
        return e / den


def swa_dense(q: np.ndarray, k: np.ndarray, v: np.ndarray, window: int) -> np.ndarray:
    """reference_swa_attention in fp32 (rows with no valid key give NaN, as torch.softmax does)."""
    B, H, T, D = q.shape
    qf, kf, vf = (t.astype(F32) for t in (q, k, v))
    scores = (qf @ np.swapaxes(kf, -1, -2)).astype(F32) / F32(D ** 0.5)
    scores = np.where(causal_window_mask(T, window), scores, -np.inf).astype(F32)
    return (_softmax_rows(scores).astype(F32) @ vf).astype(F32)


def swa_banded(q, k, v, window: int, chunk: int = 256, dtype=F32) -> np.ndarray:
    """Same result as ``swa_dense`` with O(T * (W + chunk)) memory per (b, h)."""
    B, H, T, D = q.shape
    out = np.empty((B, H, T, D), dtype=dtype)
    scale = dtype(D ** 0.5)
    for b in range(B):
        for h in range(H):
            qs, ks, vs = (t[b, h].astype(dtype) for t in (q, k, v))
            for i0 in range(0, T, chunk):
                i1 = min(T, i0 + chunk)
                j0 = max(0, i0 - window + 1)
                s = (qs[i0:i1] @ ks[j0:i1].T) / scale
                ii = np.arange(i0, i1)[:, None]
                jj = np.arange(j0, i1)[None, :]
                s = np.where((jj <= ii) & (ii - jj < window), s, -np.inf)
                out[b, h, i0:i1] = _softmax_rows(s) @ vs[j0:i1]
    return out


def _slice_scale(scale: np.ndarray, b: int, h: int) -> float:
    s = np.broadcast_to(scale, scale.shape)
    bi = 0 if s.shape[0] == 1 else b
    hi = 0 if s.shape[1] == 1 else h
    return float(s[bi, hi, 0, 0])


def _p_code_flip(x: np.ndarray, rel: np.ndarray) -> np.ndarray:
    """|e4m3(x') - e4m3(x)| over x' within a relative distance ``rel`` of x (x >= 0): the largest
    change of the P code value when the pre-rounding value 448 p can move that far -- nonzero only
    where 448 p lies within ``rel`` of an e4m3 rounding boundary."""
    c = e4m3_to_f32(f32_to_e4m3(x))
    lo = e4m3_to_f32(f32_to_e4m3((x * (1.0 - rel)).astype(F32)))
    hi = e4m3_to_f32(f32_to_e4m3(np.minimum(x * (1.0 + rel), E4M3_MAX).astype(F32)))
    return np.maximum(np.abs(hi - c), np.abs(c - lo)).astype(np.float64)


def fp8_swa_simulate(q8, k8, v8, q_scale, k_scale, v_scale, window: int, block_n: int = 64,
                     quantize_p: bool = True, chunk: int = 512, mfma_rel_err: float | None = None,
                     score_perturb=None):
    """Kernel-faithful FP8 SWA forward on e4m3 codes; returns fp32 (B, H, T, D).

    Scales are float32 arrays broadcastable to (B, H, 1, 1). Query rows are processed in
    chunks (vectorised), key blocks in the kernel's order, so the running max / rescale
    sequence matches a kernel that uses ``block_n``-key tiles aligned to multiples of
    ``block_n``.

    ``mfma_rel_err`` (e.g. 2^-10, the bound tests/test_gpu_diag.py measures for gfx950's e4m3
    MFMA): the hardware dot product may differ from the exact one by that fraction of the
    largest |product| of the dot (bounded here by max|q| max|k| of the two rows), so a score --
    and the row max it is compared with -- can move by that much, and a P code whose 448 p lies
    that close (relatively: qk_scale times the two score errors) to an e4m3 rounding boundary can
    round the other way. Then ``(out, allowance)`` is returned: allowance[b, h, i, d] bounds how
    far such flips can move out[b, h, i, d] (the flipped code-value changes times |v|, carried
    through the same rescales and normalisation as the output), so a kernel result is consistent
    with this simulator when |kernel - out| <= tolerance + allowance.

    ``score_perturb(s_raw, qa, ka) -> s_raw'`` (for the oracle's own tests): replaces each block's
    raw dot products (fp32, before the scale) -- e.g. by adding errors within the MFMA bound, to
    check that the allowance covers what such errors do to the output.
    """
    B, H, T, D = q8.shape
    out = np.zeros((B, H, T, D), dtype=F32)
    allow = np.zeros((B, H, T, D), dtype=np.float64) if mfma_rel_err is not None else None
    sm = 1.0 / (D ** 0.5)
    for b in range(B):
        for h in range(H):
            qs_, ks_, vs_ = (_slice_scale(s, b, h) for s in (q_scale, k_scale, v_scale))
            qk_scale = F32(qs_ * ks_ * sm)         # fp8_swa_attention.py:252 (double -> fp32)
            pv_scale = F32(vs_ / E4M3_MAX)         # :253
            qf = e4m3_to_f32(q8[b, h]).astype(np.float64)
            kf = e4m3_to_f32(k8[b, h]).astype(np.float64)
            vf = e4m3_to_f32(v8[b, h]).astype(np.float64)
            for i0 in range(0, T, chunk):
                i1 = min(T, i0 + chunk)
                ii = np.arange(i0, i1)[:, None]
                m = np.full((i1 - i0, 1), -np.inf, dtype=F32)
                l = np.zeros((i1 - i0, 1), dtype=F32)
                acc = np.zeros((i1 - i0, D), dtype=F32)
                lo = max(0, i0 - window + 1) // block_n * block_n
                if allow is not None:
                    al = np.zeros((i1 - i0, D), dtype=np.float64)
                    qa = np.abs(qf[i0:i1]).astype(F32)
                    pm = np.zeros((i1 - i0, 1), dtype=np.float64)   # largest |product| of the max's dot
                for n0 in range(lo, i1, block_n):
                    n1 = min(T, n0 + block_n)
                    jj = np.arange(n0, n1)[None, :]
                    valid = (jj <= ii) & (ii - jj < window)
                    # FP8 dot with fp32 accumulation: products of e4m3 values are exact; the
                    # sum is taken exactly (float64) and rounded once.
                    s = (qf[i0:i1] @ kf[n0:n1].T).astype(F32)
                    if score_perturb is not None:
                        s = score_perturb(s, qf[i0:i1], kf[n0:n1]).astype(F32)
                    s = s * qk_scale
                    s = np.where(valid, s, -np.inf).astype(F32)
                    if allow is not None:
                        # largest |q_d k_d| of each dot: the MFMA's error bound scales with it
                        pmax = (qa[:, None, :] * np.abs(kf[n0:n1]).astype(F32)[None, :, :]).max(axis=2)
                        bmax = np.max(s, axis=1, keepdims=True)
                        arg = np.argmax(s, axis=1)
                        pm = np.where(bmax > m, pmax[np.arange(i1 - i0), arg][:, None], pm)
                    m_new = np.maximum(m, np.max(s, axis=1, keepdims=True))
                    m_safe = np.where(np.isneginf(m_new), F32(0), m_new)
                    p = np.exp(s - m_safe).astype(F32)
                    p = np.where(valid, p, F32(0))
                    alpha = np.where(np.isneginf(m), F32(0), np.exp(m - m_safe)).astype(F32)
                    l = (l * alpha + p.sum(axis=1, keepdims=True, dtype=F32)).astype(F32)
                    acc = (acc * alpha).astype(F32)
                    if quantize_p:
                        pq = e4m3_to_f32(f32_to_e4m3((p * F32(E4M3_MAX)).astype(F32)))
                        acc = (acc + (pq.astype(np.float64) @ vf[n0:n1]).astype(F32)).astype(F32)
                        if allow is not None:
                            # 448 p moves by exp(qk_scale (ds - dm)): both dots' error bounds
                            rel = np.expm1(float(qk_scale) * mfma_rel_err * (pmax + pm))
                            flip = np.where(valid, _p_code_flip((p * F32(E4M3_MAX)).astype(F32), rel), 0.0)
                            al = al * alpha + flip @ np.abs(vf[n0:n1])
                    else:
                        acc = (acc + ((p * F32(E4M3_MAX)).astype(np.float64) @ vf[n0:n1])
                               .astype(F32)).astype(F32)
                    m = m_new
                acc = acc * pv_scale
                out[b, h, i0:i1] = acc / np.where(l == 0, F32(1), l)
                if allow is not None:
                    allow[b, h, i0:i1] = al * float(pv_scale) / np.where(l == 0, 1.0, l.astype(np.float64))
    return out if allow is None else (out, allow)


def fp8_swa_attention(q, k, v, window: int, granularity: str = "tensor", block_n: int = 64):
    """The FP8-simulated forward: quantise Q, K, V, then the blockwise FP8 simulator."""
    q8, qs = per_tensor_fp8(q, granularity)
    k8, ks = per_tensor_fp8(k, granularity)
    v8, vs = per_tensor_fp8(v, granularity)
    return fp8_swa_simulate(q8, k8, v8, qs, ks, vs, window, block_n=block_n)


def attention_flops(B: int, H: int, T: int, D: int, window: int) -> int:
    """4 * D * sum_{b,h} sum_i min(i + 1, W): in-window (q, k) pairs, QK^T plus PV."""
    W = max(0, window)
    full = max(0, T - W)
    ramp = min(T, W)
    pairs = ramp * (ramp + 1) // 2 + full * W
    return 4 * D * B * H * pairs


def in_window_pairs(T: int, window: int) -> int:
    W = max(0, window)
    ramp = min(T, W)
    return ramp * (ramp + 1) // 2 + max(0, T - W) * W


__all__ = [
    "causal_window_mask", "swa_dense", "swa_banded", "fp8_swa_simulate", "fp8_swa_attention",
    "attention_flops", "in_window_pairs",
]
