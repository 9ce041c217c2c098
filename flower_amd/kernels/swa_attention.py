"""bf16 causal sliding-window attention, forward + backward, on the HIP library (gfx950).

Mirrors flower/kernels/swa_attention.py: ``swa_attention(q, k, v, window, *, fwd_cfg, dkdv_cfg,
dq_cfg)`` (:362-380) is differentiable (``_SlidingWindowAttention``, :307-359); the forward saves
L = m + log(l) per query (``_swa_fwd``, :84-160) and the backward computes Delta = rowsum(dO * O)
(``_swa_bwd_preprocess``, :163-182), then dK / dV (one program per key block walking the query
blocks that see it, ``_swa_bwd_dkdv``, :184-242) and dQ (one per query block walking its keys,
``_swa_bwd_dq``, :244-305). The Triton launch-geometry tuples are accepted and ignored (the HIP
kernels use their own tiling).

Errors as in the reference (:373-379): ValueError for a non-(B, H, T, D) input, a head_dim outside
{32, 64, 128} or a window <= 0. The products run on bf16 MFMA: bf16 inputs are used as they are;
fp32 inputs (which the reference's Triton dots take at TF32 on its hardware) are rounded to bf16
on entry, and the output and the gradients come back in fp32. Other dtypes raise TypeError. No
CPU fallback.
"""

from __future__ import annotations

import torch

from .. import _lib

_FWD_CFG = (128, 64, 4, 2)
_DKDV_CFG = (128, 64, 4, 2)
_DQ_CFG = (128, 64, 4, 2)


class _SlidingWindowAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, window, token_major=False):
        lib = _lib.load()
        B, H, T, D = q.shape
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        # token_major: O stored (B, T, H, D) and returned as its (B, H, T, D) view, so that the
        # caller's transpose(1, 2).reshape(B, T, H D) is a view (no copy); the backward then takes
        # dO as that layout's view too.
        out = torch.empty((B, T, H, D) if token_major else (B, H, T, D), dtype=q.dtype, device=q.device)
        lse = torch.empty((B, H, T), device=q.device, dtype=torch.float32)
        layout = _lib.LAYOUT_BTHD if token_major else _lib.LAYOUT_BHTD
        rc = lib.flw_swa_bf16_fwd_layout(q.data_ptr(), k.data_ptr(), v.data_ptr(), B, H, T, D, int(window),
                                         out.data_ptr(), layout, lse.data_ptr(), _lib.stream_of(q))
        _lib.check(rc, "swa_attention forward")
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.window, ctx.layout = int(window), layout
        return out.transpose(1, 2) if token_major else out

    @staticmethod
    def backward(ctx, do):
        lib = _lib.load()
        q, k, v, out, lse = ctx.saved_tensors
        B, H, T, D = q.shape
        if do.dtype != q.dtype:
            do = do.to(q.dtype)
        # dO in the forward's O layout: a view of it when the gradient comes that way (the output
        # projection's gradient, token-major), a copy otherwise
        do = do.transpose(1, 2).contiguous() if ctx.layout == _lib.LAYOUT_BTHD else do.contiguous()
        dptr = do.data_ptr()
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        ws = _lib.workspace(lib.flw_swa_bf16_bwd_workspace_bytes(B, H, T, D), q.device)
        rc = lib.flw_swa_bf16_bwd_layout(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), dptr,
                                         ctx.layout, lse.data_ptr(), B, H, T, D, ctx.window, dq.data_ptr(),
                                         dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws.numel(),
                                         _lib.stream_of(q))
        _lib.check(rc, "swa_attention backward")
        return dq, dk, dv, None, None


def swa_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int, *,
                  fwd_cfg=_FWD_CFG, dkdv_cfg=_DKDV_CFG, dq_cfg=_DQ_CFG, token_major: bool = False) -> torch.Tensor:
    """Causal sliding-window attention. q/k/v: (B, H, T, D) bf16 or fp32 on the GPU. Differentiable.
    token_major (this build's addition): the (B, H, T, D) result is a view of a (B, T, H, D) tensor,
    so that ``out.transpose(1, 2).reshape(B, T, H * D)`` -- the output projection's input -- is a
    view, not a copy (bf16 inputs; the values are the same either way)."""
    del fwd_cfg, dkdv_cfg, dq_cfg
    try:
        _lib.load()
    except RuntimeError as e:
        raise RuntimeError(f"swa_attention requires the HIP library: {e}") from e
    if q.dim() != 4:
        raise ValueError(f"expected (B, H, T, D), got {tuple(q.shape)}")
    if q.shape[-1] not in (32, 64, 128):
        raise ValueError(f"head_dim must be 32/64/128, got {q.shape[-1]}")
    if window <= 0:
        raise ValueError("window must be positive; use flex for full-context attention")
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v shapes differ: {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"q, k, v must share a dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
    if q.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("swa_attention takes bfloat16 or float32 inputs; got " + str(q.dtype))
    _lib.require_gpu(q, k, v)
    if q.dtype == torch.float32:
        # bf16 MFMA products; the casts are differentiable, so the gradients return in fp32
        out = _SlidingWindowAttention.apply(q.to(torch.bfloat16), k.to(torch.bfloat16),
                                            v.to(torch.bfloat16), window)
        return out.to(torch.float32)
    return _SlidingWindowAttention.apply(q, k, v, window, bool(token_major))


__all__ = ["swa_attention"]
