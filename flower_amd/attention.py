"""Attention-side operators of the reference's model code, on the HIP library.

``_fake_quant_e4m3``  -- flower/models/base.py:167-203: straight-through e4m3
                         quantise-dequantise of Q/K/V (the ``model.fp8_attention_sim`` probe).
                         Forward value computed by one HIP amax pass + one fused
                         quantise/dequantise pass, rounded to x.dtype step by step exactly as the
                         reference's torch op sequence; backward is the identity.
``causal_mask``       -- base.py:418-423, the boolean (T, T) band mask (plain torch).
``fp8_attention``     -- the ``attn_precision: fp8`` route (config.py:373): Q/K/V after QK-norm
                         and RoPE go through the fused FP8 SWA kernel.
"""

from __future__ import annotations

import torch

from . import _lib
from .kernels.fp8_swa_attention import fp8_swa_attention_forward


class _FakeQuantE4M3(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: torch.Tensor, granularity: str) -> torch.Tensor:
        lib = _lib.load()
        _lib.require_gpu(x)
        shape = x.shape
        if granularity == "tensor":
            last = shape[-1] if x.dim() else 1
            x4 = x.detach().reshape(1, 1, -1, last) if x.dim() != 4 else x.detach()
        else:
            if x.dim() != 4:
                raise ValueError(f"per-{granularity} fake quantisation needs (B, H, T, D)")
            x4 = x.detach()
        vec = 4 if x.dtype == torch.float32 else 8
        sb, sh, st, sd = x4.stride()
        if sd != 1 or sb % vec or sh % vec or st % vec or x4.data_ptr() % 16:
            x4 = x4.contiguous()
            sb, sh, st, _ = x4.stride()
        B, H, T, D = x4.shape
        out = torch.empty((B, H, T, D), dtype=x.dtype, device=x.device)
        ws = _lib.workspace(lib.flw_quant_workspace_bytes(B, H, T, D) + 4 * B * H, x.device)
        rc = lib.flw_fake_quant_e4m3(x4.data_ptr(), _lib.dtype_code(x.dtype), B, H, T, D, sb, sh, st,
                                     _lib.GRANULARITY[granularity], out.data_ptr(), None,
                                     ws.data_ptr(), ws.numel(), _lib.stream_of(x))
        _lib.check(rc, "_fake_quant_e4m3")
        return out.reshape(shape)

    @staticmethod
    def backward(ctx, grad_out):
        # x + (dq - x).detach(): the gradient reaches x untouched (base.py:201-203).
        return grad_out, None


def _fake_quant_e4m3(x: torch.Tensor, granularity: str = "tensor") -> torch.Tensor:
    """Straight-through per-tensor e4m3 quantize-dequantize (base.py:167-203).

    Forward value: ``x + (dq - x)`` with ``dq = e4m3(clamp(x / s, +-448)) * s``,
    ``s = max(|x|.amax(), 1e-12) / 448`` kept in x.dtype; gradient: identity.
    """
    return _FakeQuantE4M3.apply(x, granularity)


def causal_mask(seq_len: int, device: torch.device, local_window: int | None = None) -> torch.Tensor:
    idx = torch.arange(seq_len, device=device)
    mask = idx[:, None] >= idx[None, :]
    if local_window is not None:
        mask &= (idx[:, None] - idx[None, :]) < local_window
    return mask


def fp8_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, local_window: int | None,
                  granularity: str = "head") -> torch.Tensor:
    """Forward-only FP8 attention for (B, H, T, D) Q/K/V; ``local_window=None`` is full causal."""
    window = q.shape[2] if local_window is None else local_window
    return fp8_swa_attention_forward(q, k, v, window, granularity=granularity)
