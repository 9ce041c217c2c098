"""An FP8 decoder block: the reference's TransformerBlock with every Linear on the HIP FP8 GEMM and
the attention on the fused FP8 sliding-window kernel.

Layout and parameter names follow flower/models/base.py:
  ``RMSNorm``                 base.py:324-338 (fp32 mean-square, rsqrt, then the gain)
  ``Fp8CausalSelfAttention``  base.py:553-665: ``qkv`` Linear(d, 3d) -> chunk -> heads as strided
                              (B, H, T, D) views (base.py:607-614, read in place by the
                              quantiser) -> FP8 SWA -> (B, T, d) -> ``out`` Linear(d, d);
                              forward-only like the FP8 kernel (fp8_swa_attention.py:71-76)
  ``Fp8FeedForward``          base.py:514-525 GELU layout (``net.0`` Linear(d, ffn), GELU,
                              ``net.3`` Linear(ffn, d); dropout is identity in eval)
  ``Fp8DecoderBlock``         base.py:698-722: x + attn(ln1(x)), then + ff(ln2(x))

Norms, GELU and residual adds are plain torch ops on the GPU; the linears, the quantisers and the
attention run in libflower_amd.so. Wrap calls in ``fp8_weight_cache(block)`` to quantise the
weights once.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from .kernels.fp8_swa_attention import fp8_swa_attention_forward
from .precision import Fp8Linear


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        rms = x.float().pow(2).mean(dim=-1, keepdim=True).add(self.eps).rsqrt()
        return (x.float() * rms).to(dtype=x.dtype) * self.weight


class Fp8CausalSelfAttention(nn.Module):
    def __init__(self, d_model: int, num_heads: int, local_window: int | None, *, bias: bool = False,
                 recipe: str = "rowwise", granularity: str = "head") -> None:
        super().__init__()
        if d_model % num_heads:
            raise ValueError("d_model must be divisible by num_heads")
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.local_window = local_window
        self.granularity = granularity
        self.qkv = Fp8Linear(d_model, 3 * d_model, bias=bias, recipe=recipe)
        self.out = Fp8Linear(d_model, d_model, bias=bias, recipe=recipe)

    def _split(self, x: torch.Tensor) -> torch.Tensor:
        bsz, seq_len, _ = x.shape
        return x.view(bsz, seq_len, self.num_heads, self.head_dim).transpose(1, 2)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        q, k, v = self.qkv(x).chunk(3, dim=-1)
        q, k, v = self._split(q), self._split(k), self._split(v)
        window = x.shape[1] if self.local_window is None else self.local_window
        out = fp8_swa_attention_forward(q, k, v, window, granularity=self.granularity)
        return self.out(out.transpose(1, 2).reshape(x.shape))


class Fp8FeedForward(nn.Module):
    def __init__(self, d_model: int, ffn_dim: int, *, bias: bool = False, recipe: str = "rowwise") -> None:
        super().__init__()
        self.net = nn.Sequential(
            Fp8Linear(d_model, ffn_dim, bias=bias, recipe=recipe),
            nn.GELU(),
            nn.Identity(),                     # the reference's Dropout slot (eval: identity)
            Fp8Linear(ffn_dim, d_model, bias=bias, recipe=recipe),
        )

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.net(x)


class Fp8DecoderBlock(nn.Module):
    def __init__(self, d_model: int = 1024, num_heads: int = 16, ffn_dim: int = 4096,
                 local_window: int | None = 4096, *, bias: bool = False, recipe: str = "rowwise",
                 granularity: str = "head") -> None:
        super().__init__()
        self.ln1 = RMSNorm(d_model)
        self.attn = Fp8CausalSelfAttention(d_model, num_heads, local_window, bias=bias, recipe=recipe,
                                           granularity=granularity)
        self.ln2 = RMSNorm(d_model)
        self.ff = Fp8FeedForward(d_model, ffn_dim, bias=bias, recipe=recipe)

    @torch.no_grad()
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.ln1(x))
        return x + self.ff(self.ln2(x))


def init_block_(block: Fp8DecoderBlock, std: float = 0.02, seed: int = 0) -> Fp8DecoderBlock:
    """Random init of BASELINE config 5: every Linear weight ~ N(0, std), norms at 1."""
    g = torch.Generator().manual_seed(seed)
    for mod in block.modules():
        if isinstance(mod, nn.Linear):
            w = torch.randn(mod.weight.shape, generator=g) * std
            mod.weight.data.copy_(w.to(mod.weight.dtype))
            if mod.bias is not None:
                mod.bias.data.zero_()
    return block


def block_flops(T: int, B: int, d_model: int, ffn_dim: int, num_heads: int, window: int) -> int:
    """Linear FLOPs (2 M N K over QKV, O, FF1, FF2) plus in-window attention FLOPs (4 D per pair)."""
    M = B * T
    linear = 2 * M * d_model * (3 * d_model + d_model + 2 * ffn_dim)
    W = min(window, T)
    pairs = W * (W + 1) // 2 + max(0, T - W) * W
    return linear + 4 * (d_model // num_heads) * B * num_heads * pairs


__all__ = ["RMSNorm", "Fp8CausalSelfAttention", "Fp8FeedForward", "Fp8DecoderBlock", "init_block_",
           "block_flops"]
