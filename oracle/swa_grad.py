"""bf16 sliding-window attention as a training op: forward with log-sum-exp, and the backward.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates flower/kernels/swa_attention.py (the reference's Triton forward / backward) in float64
numpy, query block by query block so that only the band [i - W + 1, i] of keys is materialised:

``swa_forward_lse``  _swa_fwd, swa_attention.py:84-160: O = softmax(mask(Q K^T * s)) V with
                     s = 1 / sqrt(D), and L = m + log(l) per query row (the combined form the
                     backward needs, P = exp(S - L)); a row with no valid key (none exist in
                     the causal band: key i is always valid for query i) would store L = log 1.
``swa_backward``     _swa_bwd_preprocess :163-181  Delta_i = sum_d dO_id O_id;
                     _swa_bwd_dkdv :184-241 and _swa_bwd_dq :244-292, per valid (i, j):
                         P_ij  = exp(S_ij - L_i)
                         dP_ij = dO_i . v_j
                         dS_ij = P_ij (dP_ij - Delta_i) s
                         dV_j += P_ij dO_i ;  dK_j += dS_ij q_i ;  dQ_i += dS_ij k_j
                     The reference computes dK/dV per key block and dQ per query block; the
                     sums are the same.

Pinned by tests/test_oracle_swa_grad.py: forward and L against ``swa.swa_dense`` and a log-sum-exp
taken directly; the gradients against torch.autograd through dense masked attention (a library
routine, float64), and against central finite differences of sum(dO * O) on a tiny case; the
closed-form invariants  sum_j dK_j = 0  (softmax is invariant to a shift of every score of a row,
so sum_j dS_ij = 0 -- the identity that a dropped Delta term breaks) and  sum_j dV_j = sum_i dO_i
(rows of P sum to 1); W = 1 (dQ = dK = 0, dV = dO).
"""

from __future__ import annotations

import numpy as np

F64 = np.float64


def _band(i0: int, i1: int, window: int):
    j0 = max(0, i0 - window + 1)
    ii = np.arange(i0, i1)[:, None]
    jj = np.arange(j0, i1)[None, :]
    return j0, (jj <= ii) & (ii - jj < window)


def swa_forward_lse(q, k, v, window: int, chunk: int = 256):
    """(out, lse): out (B, H, T, D) float64, lse (B, H, T) float64 (natural log)."""
    B, H, T, D = q.shape
    s = 1.0 / np.sqrt(D)
    out = np.empty((B, H, T, D), dtype=F64)
    lse = np.empty((B, H, T), dtype=F64)
    for b in range(B):
        for h in range(H):
            qs, ks, vs = (np.asarray(t[b, h], dtype=F64) for t in (q, k, v))
            for i0 in range(0, T, chunk):
                i1 = min(T, i0 + chunk)
                j0, valid = _band(i0, i1, window)
                sc = np.where(valid, (qs[i0:i1] @ ks[j0:i1].T) * s, -np.inf)
                m = sc.max(axis=1, keepdims=True)
                m = np.where(np.isneginf(m), 0.0, m)
                p = np.exp(sc - m)
                l = p.sum(axis=1, keepdims=True)
                l = np.where(l == 0.0, 1.0, l)
                out[b, h, i0:i1] = (p @ vs[j0:i1]) / l
                lse[b, h, i0:i1] = (m + np.log(l))[:, 0]
    return out, lse


def swa_backward(q, k, v, out, lse, dout, window: int, chunk: int = 256):
    """(dq, dk, dv), float64, from the saved forward output and log-sum-exp."""
    B, H, T, D = q.shape
    s = 1.0 / np.sqrt(D)
    dq = np.zeros((B, H, T, D), dtype=F64)
    dk = np.zeros((B, H, T, D), dtype=F64)
    dv = np.zeros((B, H, T, D), dtype=F64)
    for b in range(B):
        for h in range(H):
            qs, ks, vs, os_, dos = (np.asarray(t[b, h], dtype=F64) for t in (q, k, v, out, dout))
            delta = np.sum(dos * os_, axis=1)
            L = np.asarray(lse[b, h], dtype=F64)
            for i0 in range(0, T, chunk):
                i1 = min(T, i0 + chunk)
                j0, valid = _band(i0, i1, window)
                p = np.where(valid, np.exp((qs[i0:i1] @ ks[j0:i1].T) * s - L[i0:i1, None]), 0.0)
                dp = dos[i0:i1] @ vs[j0:i1].T
                ds = np.where(valid, p * (dp - delta[i0:i1, None]) * s, 0.0)
                dv[b, h, j0:i1] += p.T @ dos[i0:i1]
                dk[b, h, j0:i1] += ds.T @ qs[i0:i1]
                dq[b, h, i0:i1] = ds @ ks[j0:i1]
    return dq, dk, dv
