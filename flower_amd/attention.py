"""Attention-side operators and modules of the reference's model code, on the HIP library.

``_fake_quant_e4m3``    -- flower/models/base.py:167-203: straight-through e4m3
                           quantise-dequantise of Q/K/V (the ``model.fp8_attention_sim`` probe).
                           Forward value computed by one HIP amax pass + one fused
                           quantise/dequantise pass, rounded to x.dtype step by step exactly as the
                           reference's torch op sequence; backward is the identity.
``causal_mask``         -- base.py:418-423, the boolean (T, T) band mask (plain torch).
``HeadRMSNorm``         -- base.py:341-357, parameter-free QK-norm (torch ops, the reference maths).
``RotaryEmbedding``     -- base.py:436-483, RoPE with cached fp32 cos / sin tables.
``CausalSelfAttention`` -- base.py:553-665 with the ``attn_precision`` switch (config.py:373):
                           "fp8" routes the heads through the FP8 sliding-window kernel, with the
                           QK-norm, RoPE and the e4m3 quantisation of Q/K/V fused in one HIP pass
                           pair (the reference's quantisation point, "after QK-norm and RoPE",
                           base.py:634-637) -- and, in training, through the differentiable FP8
                           attention (bf16 backward, straight-through quantisers); "bf16"
                           through the HIP bf16 sliding-window kernel.
``fp8_attention``       -- the FP8 route on (B, H, T, D) Q/K/V that are already normed and rotated.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib
from .kernels.fp8_swa_attention import (fp8_swa_attention, fp8_swa_attention_forward,
                                        fp8_swa_attention_from_codes, qk_norm_rope_quant_e4m3)
from .kernels.swa_attention import swa_attention


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


class _QkvHeadsFn(torch.autograd.Function):
    """``qkv_heads``' split, HeadRMSNorm and RoPE on the qkv projection's bf16 output y [B, T, 3 H D]
    in one HIP pass each way (flw_qkv_heads_fwd / flw_qkv_heads_bwd): q', k', v as contiguous
    (B, H, T, D); the backward returns dy [B, T, 3 H D] as torch's autograd of the same expressions
    does (its bf16 roundings of the RoPE products, the norm's backward in fp32)."""

    @staticmethod
    def forward(ctx, y, num_heads, norm, eps, cos, sin):
        lib = _lib.load()
        B, T, C = y.shape
        D = C // (3 * num_heads)
        if y.stride(-1) != 1 or y.stride(0) != T * y.stride(1) or y.stride(1) % 8 or y.data_ptr() % 16:
            y = y.contiguous()
        q, k, v = (torch.empty((B, num_heads, T, D), dtype=y.dtype, device=y.device) for _ in range(3))
        rc = lib.flw_qkv_heads_fwd(y.data_ptr(), B, T, num_heads, D, y.stride(1), int(norm), float(eps),
                                   cos.data_ptr(), sin.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                   _lib.stream_of(y))
        _lib.check(rc, "qkv_heads")
        ctx.save_for_backward(y, cos, sin)
        ctx.meta = (num_heads, norm, eps, D)
        return q, k, v

    @staticmethod
    def backward(ctx, dq, dk, dv):
        y, cos, sin = ctx.saved_tensors
        H, norm, eps, D = ctx.meta
        B, T, C = y.shape
        grads = [(g if g is not None else torch.zeros((B, H, T, D), dtype=y.dtype, device=y.device))
                 .to(y.dtype).contiguous() for g in (dq, dk, dv)]
        dy = torch.empty((B, T, C), dtype=y.dtype, device=y.device)
        lib = _lib.load()
        rc = lib.flw_qkv_heads_bwd(y.data_ptr(), B, T, H, D, y.stride(1), int(norm), float(eps), cos.data_ptr(),
                                   sin.data_ptr(), grads[0].data_ptr(), grads[1].data_ptr(), grads[2].data_ptr(),
                                   dy.data_ptr(), C, None, None, 0, _lib.stream_of(y))
        _lib.check(rc, "qkv_heads backward")
        return dy, None, None, None, None, None


class _Fp8QkvHeadsFn(torch.autograd.Function):
    """The qkv projection as a tensorwise Fp8Linear followed by ``_QkvHeadsFn``'s pass, as one
    autograd node, so that the backward's qkv_heads pass also reports |dqkv|'s maximum and the
    projection's gradient cast takes it instead of an amax pass. Every code, scale and GEMM is the
    one the Fp8Linear and _QkvHeadsFn compute on their own: the same results bit for bit."""

    @staticmethod
    def forward(ctx, x, weight, qkv_mod, num_heads, norm, eps, cos, sin):
        from . import precision as P
        lib = _lib.load()
        B, T, d = x.shape
        x2 = x.reshape(B * T, d)
        if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
            x2 = x2.contiguous()
        M = B * T
        ld = ((M + 127) // 128) * 128
        x8, x8t, sx = P._quantize_tensorwise_t(x2, ld)
        w8, sw, w8t = qkv_mod.tensorwise_codes()
        y = P.scaled_mm_plain(x8, sx, w8, sw)
        C = y.shape[1]
        D = C // (3 * num_heads)
        q, k, v = (torch.empty((B, num_heads, T, D), dtype=y.dtype, device=y.device) for _ in range(3))
        _lib.check(lib.flw_qkv_heads_fwd(y.data_ptr(), B, T, num_heads, D, C, int(norm), float(eps), cos.data_ptr(),
                                         sin.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                         _lib.stream_of(y)), "qkv_heads")
        ctx.save_for_backward(y, cos, sin, x8t, sx, w8, sw, w8t)
        ctx.meta = (qkv_mod, num_heads, norm, eps, D, B, T, ld, x.shape)
        return q, k, v

    @staticmethod
    def backward(ctx, dq, dk, dv):
        from . import precision as P
        y, cos, sin, x8t, sx, w8, sw, w8t = ctx.saved_tensors
        qkv_mod, H, norm, eps, D, B, T, ld, x_shape = ctx.meta
        M, C = y.shape
        lib = _lib.load()
        grads = [(g if g is not None else torch.zeros((B, H, T, D), dtype=y.dtype, device=y.device))
                 .to(y.dtype).contiguous() for g in (dq, dk, dv)]
        dy = torch.empty((M, C), dtype=y.dtype, device=y.device)
        amax = torch.empty(1, dtype=torch.int32, device=y.device)
        ws = _lib.workspace(lib.flw_qkv_heads_amax_workspace_bytes(B, T, H, D), y.device)
        _lib.check(lib.flw_qkv_heads_bwd(y.data_ptr(), B, T, H, D, C, int(norm), float(eps), cos.data_ptr(),
                                         sin.data_ptr(), grads[0].data_ptr(), grads[1].data_ptr(), grads[2].data_ptr(),
                                         dy.data_ptr(), C, amax.data_ptr(), ws.data_ptr(), ws.numel(),
                                         _lib.stream_of(y)), "qkv_heads backward")
        g8, g8t, sg = P._quantize_tensorwise_t(dy, ld, amax)
        gx = gw = None
        if ctx.needs_input_grad[0]:
            if getattr(qkv_mod, "_fp8_cached", None) is not None:     # the weight cache's dgrad codes
                wc, swc = qkv_mod.weight_col_codes()
            else:
                wc, swc = (w8t if w8t is not None else P.transpose_codes(w8, C)), sw
            gx = P.scaled_mm(g8, sg, wc, swc).view(x_shape)
        if ctx.needs_input_grad[1]:
            gw = P.scaled_mm(g8t, sg, x8t, sx).to(qkv_mod.weight.dtype)
        return gx, gw, None, None, None, None, None, None


class HeadRMSNorm(nn.Module):
    """Parameter-free RMSNorm over the head dimension (QK-norm), base.py:341-357."""

    def __init__(self, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        rms = x.float().pow(2).mean(dim=-1, keepdim=True).add(self.eps).rsqrt()
        return (x.float() * rms).to(dtype=x.dtype)


class RotaryEmbedding(nn.Module):
    """RoPE with cached cos / sin tables (base.py:436-483): pairs (2i, 2i+1) rotate by
    position * base^(-2i / head_dim); the fp32 tables are built once on the CPU and cast to the
    activations' dtype at use, as the reference does, so the fused kernel and the torch path see
    the same table values."""

    def __init__(self, head_dim: int, max_seq_len: int, base: float = 10000.0) -> None:
        super().__init__()
        if head_dim % 2 != 0:
            raise ValueError("RoPE requires even head_dim")
        self._base = base
        self._head_dim = head_dim
        cos, sin = self._tables(max_seq_len)
        self.register_buffer("cos", cos, persistent=False)
        self.register_buffer("sin", sin, persistent=False)
        self._cast = {}

    def _tables(self, seq_len: int):
        inv_freq = 1.0 / (self._base ** (torch.arange(0, self._head_dim, 2).float() / self._head_dim))
        freqs = torch.outer(torch.arange(seq_len).float(), inv_freq)
        shape = (1, 1, seq_len, self._head_dim)
        return (freqs.cos().repeat_interleave(2, dim=-1).view(shape),
                freqs.sin().repeat_interleave(2, dim=-1).view(shape))

    def _extend_cache(self, seq_len: int) -> None:
        """Tables for longer sequences, built lazily (base.py:471-476)."""
        cos, sin = self._tables(seq_len)
        self.register_buffer("cos", cos, persistent=False)
        self.register_buffer("sin", sin, persistent=False)
        self._cast = {}

    @staticmethod
    def _rotate_half(x: torch.Tensor) -> torch.Tensor:
        x1 = x[..., ::2]
        x2 = x[..., 1::2]
        return torch.stack((-x2, x1), dim=-1).flatten(-2)

    def tables(self, seq_len: int, dtype: torch.dtype, device) -> tuple[torch.Tensor, torch.Tensor]:
        """(cos, sin) as contiguous [seq_len, head_dim] tensors of ``dtype`` on ``device``."""
        if seq_len > self.cos.shape[-2]:
            self._extend_cache(seq_len)
        key = (seq_len, dtype, torch.device(device), self.cos.data_ptr())
        hit = self._cast.get(key)
        if hit is None:
            hit = tuple(t[0, 0, :seq_len].to(device=device, dtype=dtype).contiguous() for t in (self.cos, self.sin))
            self._cast = {key: hit}
        return hit

    def forward(self, q: torch.Tensor, k: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        cos, sin = self.tables(q.shape[-2], q.dtype, q.device)
        return q * cos + self._rotate_half(q) * sin, k * cos + self._rotate_half(k) * sin


class CausalSelfAttention(nn.Module):
    """The reference's attention module (base.py:553-665) on this build's kernels.

    ``config`` carries the reference's fields: d_model, num_heads, max_seq_len, rope_base,
    use_bias (default True), qk_norm (False), fp8_attention_sim (False) and attn_precision
    ("bf16" | "fp8", config.py:373; validated as config.py:464-465), plus this build's
    ``fp8_attention_granularity`` ("head" by default: one e4m3 scale per head for each of Q, K, V).

    attn_precision "fp8", inference (no gradient needed): the qkv projection, then ONE HIP pass pair
    that applies QK-norm and RoPE to q and k and quantises q', k', v to e4m3 (the reference's
    quantisation point, base.py:634-637, "exactly the tensors a real FP8 attention kernel would
    consume"), then the FP8 sliding-window kernel writing the (B, T, H, D) output in place, then
    ``out``. ``forward_unfused`` is the same route with the heads built by ``qkv_heads`` in torch.
    attn_precision "fp8", training (gradients needed): ``qkv_heads`` in torch (its QK-norm and RoPE
    differentiate as usual), then the differentiable ``fp8_swa_attention`` -- the same FP8 forward,
    and the bf16 sliding-window backward at the dequantised q', k', v (straight-through
    quantisers, the estimator `_fake_quant_e4m3` trains with), then ``out``.
    attn_precision "bf16": ``qkv_heads`` then the differentiable HIP bf16 sliding-window kernel
    (a full causal window when ``local_window`` is None). The reference's flex / SDPA choice and
    its RBF distance bias (local_attn_kernel_bias "rbf") are not offered: rbf raises ValueError.
    ``fused_fp8_qkv`` (False): with a tensorwise Fp8Linear ``qkv`` in training, run the projection
    and the heads pass as one node whose backward hands |dqkv|'s maximum to the gradient cast
    (``_Fp8QkvHeadsFn``; the same results bit for bit).
    """

    fused_fp8_qkv = False

    def __init__(self, config, local_window: int | None = None) -> None:
        super().__init__()
        if config.d_model % config.num_heads != 0:
            raise ValueError("d_model must be divisible by num_heads")
        precision = getattr(config, "attn_precision", "bf16")
        if precision not in {"bf16", "fp8"}:
            raise ValueError(f"attn_precision must be bf16|fp8, got {precision!r}")
        if getattr(config, "local_attn_kernel_bias", "none") != "none":
            raise ValueError("local_attn_kernel_bias 'rbf' is not supported by the HIP attention kernels")
        self.num_heads = config.num_heads
        self.head_dim = config.d_model // config.num_heads
        self.local_window = local_window
        self.attn_precision = precision
        self.fp8_granularity = getattr(config, "fp8_attention_granularity", "head")
        self.rope = RotaryEmbedding(self.head_dim, getattr(config, "max_seq_len", 8192),
                                    base=getattr(config, "rope_base", 10000.0))
        bias = bool(getattr(config, "use_bias", True))
        self.qkv = nn.Linear(config.d_model, config.d_model * 3, bias=bias)
        self.out = nn.Linear(config.d_model, config.d_model, bias=bias)
        self.out._is_residual_out = True
        self.qk_norm = HeadRMSNorm() if bool(getattr(config, "qk_norm", False)) else None
        self.fp8_attention_sim = bool(getattr(config, "fp8_attention_sim", False))

    def _split(self, x: torch.Tensor) -> torch.Tensor:
        bsz, seq_len, _ = x.shape
        return x.view(bsz, seq_len, self.num_heads, self.head_dim).transpose(1, 2)

    def _window(self, seq_len: int) -> int:
        return seq_len if self.local_window is None else self.local_window

    def qkv_heads(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Project to per-head (q, k, v), apply QK-norm, then RoPE (base.py:618-639). bf16 on the
        GPU: the split, norm and RoPE run as one HIP pass each way (``_QkvHeadsFn``), q, k, v
        contiguous; otherwise the reference's torch expressions."""
        if self._fp8_qkv_ok(x):
            cos, sin = self.rope.tables(x.shape[1], x.dtype, x.device)
            eps = self.qk_norm.eps if self.qk_norm is not None else 0.0
            q, k, v = _Fp8QkvHeadsFn.apply(x, self.qkv.weight, self.qkv, self.num_heads, self.qk_norm is not None,
                                           eps, cos, sin)
            if self.fp8_attention_sim:
                q, k, v = _fake_quant_e4m3(q), _fake_quant_e4m3(k), _fake_quant_e4m3(v)
            return q, k, v
        y = self.qkv(x)
        if y.is_cuda and y.dtype == torch.bfloat16 and self.head_dim in (32, 64, 128):
            cos, sin = self.rope.tables(y.shape[1], y.dtype, y.device)
            eps = self.qk_norm.eps if self.qk_norm is not None else 0.0
            q, k, v = _QkvHeadsFn.apply(y, self.num_heads, self.qk_norm is not None, eps, cos, sin)
            if self.fp8_attention_sim:
                q, k, v = _fake_quant_e4m3(q), _fake_quant_e4m3(k), _fake_quant_e4m3(v)
            return q, k, v
        q, k, v = y.chunk(3, dim=-1)
        q, k, v = self._split(q), self._split(k), self._split(v)
        if self.qk_norm is not None:
            q, k = self.qk_norm(q), self.qk_norm(k)
        q, k = self.rope(q, k)
        if self.fp8_attention_sim:
            q, k, v = _fake_quant_e4m3(q), _fake_quant_e4m3(k), _fake_quant_e4m3(v)
        return q, k, v

    def _fp8_qkv_ok(self, x: torch.Tensor) -> bool:
        """``qkv`` a bias-free tensorwise Fp8Linear with the FP8 backward and 16-aligned widths, x a
        non-empty (B, T, d) bf16 GPU tensor, autocast off, a gradient to take, and ``fused_fp8_qkv`` set:
        _Fp8QkvHeadsFn's route. Off by default: on the 450M block the qkv_heads backward with the
        |dqkv| maximum takes ~8 us longer a call than without it (92.8 against 84.8 us), which is
        what the amax pass it spares the gradient cast costs, with a fold launch besides."""
        from .precision import Fp8Linear
        m = self.qkv
        return (self.fused_fp8_qkv and type(m) is Fp8Linear and m.recipe == "tensorwise" and getattr(m, "backward_fp8", True)
                and m.bias is None and m.in_features % 16 == 0 and m.out_features % 16 == 0
                and x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 3 and x.numel() > 0
                and not torch.is_autocast_enabled() and self.head_dim in (32, 64, 128)
                and m.out_features == 3 * self.num_heads * self.head_dim
                and torch.is_grad_enabled() and (x.requires_grad or m.weight.requires_grad))

    def _needs_grad(self, x: torch.Tensor) -> bool:
        return torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters()))

    def _forward_fp8_train(self, x: torch.Tensor) -> torch.Tensor:
        """The differentiable FP8 route: qkv_heads in torch, fp8_swa_attention, out."""
        q, k, v = self.qkv_heads(x)
        out = fp8_swa_attention(q, k, v, self._window(x.shape[1]), granularity=self.fp8_granularity)
        return self.out(out.transpose(1, 2).reshape(x.shape))

    def forward(self, x: torch.Tensor, trace: dict | None = None) -> torch.Tensor:
        if self.attn_precision == "fp8":
            if self._needs_grad(x):
                return self._forward_fp8_train(x)
            return self._forward_fp8(x, trace)
        q, k, v = self.qkv_heads(x)
        # token-major O: the transpose back to [B, T, H D] rows below is a view, in both directions
        out = swa_attention(q, k, v, self._window(x.shape[1]), token_major=q.dtype == torch.bfloat16)
        return self.out(out.transpose(1, 2).reshape(x.shape))

    def _forward_fp8(self, x: torch.Tensor, trace: dict | None = None) -> torch.Tensor:
        """qkv -> fused QK-norm + RoPE + e4m3 quantisation -> FP8 SWA -> out. ``trace`` (a dict,
        for checks) receives the projection "qkv", the transformed "q" / "k", the codes and scales,
        and the attention output "attn"."""
        B, T, d = x.shape
        y = self.qkv(x)
        q, k, v = (self._split(t) for t in y.chunk(3, dim=-1))
        cos, sin = self.rope.tables(T, y.dtype, y.device)
        res = qk_norm_rope_quant_e4m3(q, k, v, qk_norm=self.qk_norm is not None,
                                      eps=self.qk_norm.eps if self.qk_norm is not None else 0.0,
                                      rope_cos=cos, rope_sin=sin, granularity=self.fp8_granularity,
                                      return_transformed=trace is not None)
        q8, k8, vt, scales = res[:4]
        a = torch.empty((B, T, d), dtype=y.dtype, device=y.device)
        fp8_swa_attention_from_codes(q8, k8, vt, scales, self._window(T), granularity=self.fp8_granularity,
                                     out=a.view(B, T, self.num_heads, self.head_dim).transpose(1, 2))
        if trace is not None:
            trace.update(qkv=y, q=res[4], k=res[5], q8=q8, k8=k8, v_tiles=vt, scales=scales, attn=a)
        return self.out(a)

    def forward_unfused(self, x: torch.Tensor) -> torch.Tensor:
        """The FP8 route composed from the reference's pieces: ``qkv_heads`` in torch, then
        ``fp8_swa_attention_forward`` (its own quantisation), then ``out``; with gradients needed,
        the differentiable route."""
        if self._needs_grad(x):
            return self._forward_fp8_train(x)
        q, k, v = self.qkv_heads(x)
        out = fp8_swa_attention_forward(q, k, v, self._window(x.shape[1]), granularity=self.fp8_granularity)
        return self.out(out.transpose(1, 2).reshape(x.shape))
