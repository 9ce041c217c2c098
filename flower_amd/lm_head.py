"""FP8 LM head, mirroring ``CausalLM._compute_logits`` / ``CausalLM._fp8_head``
(flower/models/base.py:865-924) on the HIP FP8 GEMM.

``fp8_head(x_normed, weight)``: per-row abs-amax activation scales and per-vocab-row weight scales,
``scale = max(amax / 448, 1e-12)`` in fp32, both operands divided by their scale before the e4m3
cast (no clamp), the product accumulated in fp32 and returned as bf16 logits (B, T, vocab) -- the
``_scaled_mm`` recipe of base.py:911-923, here as flw_quant_rows_e4m3 (the weight) +
flw_fp8_linear(A8W8) (the activations and the GEMM). The weight is quantised on every call, as
in the reference (it is a view of the tied embedding that training keeps changing).

``compute_logits(head, x_normed, fp8_lm_head, training)``: the reference's routing -- the FP8 head
only in eval, for bf16 activations on the GPU; otherwise the plain ``head`` Linear (the FP8 GEMM
has no backward).
"""

from __future__ import annotations

import torch
import torch.nn as nn

from .precision import fp8_linear_forward, quantize_weight


def fp8_head(x_normed: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """bf16 logits [B, T, vocab] = x_normed [B, T, D] @ weight [vocab, D]^T in FP8 (A8W8)."""
    B, T, D = x_normed.shape
    w8, w_scale = quantize_weight(weight, "rowwise")
    logits = fp8_linear_forward(x_normed.reshape(-1, D), w8, w_scale, "rowwise")
    return logits.view(B, T, -1)


def compute_logits(head: nn.Linear, x_normed: torch.Tensor, fp8_lm_head: bool,
                   training: bool) -> torch.Tensor:
    if fp8_lm_head and not training and x_normed.dtype == torch.bfloat16 and x_normed.is_cuda:
        return fp8_head(x_normed, head.weight)
    return head(x_normed)


__all__ = ["fp8_head", "compute_logits"]
