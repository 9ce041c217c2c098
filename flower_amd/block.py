"""An FP8 decoder block: the reference's TransformerBlock with every Linear on the HIP FP8 GEMM and
the attention on the fused FP8 sliding-window kernel.

Layout and parameter names follow flower/models/base.py:
  ``RMSNorm``                 base.py:324-338 (fp32 mean-square, rsqrt, then the gain)
  ``Fp8CausalSelfAttention``  base.py:553-665: the module's ``attn_precision: "fp8"`` route
                              (flower_amd.attention.CausalSelfAttention) with both projections as
                              Fp8Linear: ``qkv`` Linear(d, 3d) -> heads as strided (B, H, T, D)
                              views (base.py:607-614) -> HeadRMSNorm of q, k when ``qk_norm``
                              (base.py:632-633; on by default, as the 450M FP8 configs set it,
                              configs/sweep13_450m_longctx_fp8.yaml:109) -> RoPE of q, k
                              (base.py:634, always, base ``rope_base``) -> e4m3 (the quantisation
                              point, base.py:636-637) -> FP8 SWA -> ``out`` Linear(d, d);
                              differentiable through fp8_swa_attention when gradients are needed
                              (the block's own fused ``forward`` runs without them)
  ``Fp8FeedForward``          base.py:514-525 GELU layout (``net.0`` Linear(d, ffn), GELU,
                              ``net.3`` Linear(ffn, d); dropout is identity in eval)
  ``Fp8DecoderBlock``         base.py:698-722: x + attn(ln1(x)), then + ff(ln2(x))

``forward`` runs the fused path on bf16 GPU inputs (RMSNorm and GELU fused with the next
linear's per-row e4m3 quantisation, QK-norm + RoPE and the per-head maxima in the QKV GEMM's
epilogue (or, with ``fuse_qk_epilogue = False``, in the Q / K / V quantiser), residual adds in the
GEMM epilogues, the attention writing its (B, T, H, D) output in place: library kernels
only, no torch elementwise kernels);
``forward_unfused`` is the module-by-module composition (the modules' own norms, GELU and torch
adds around the library's linears and attention). Wrap calls in ``fp8_weight_cache(block)`` to quantise the
weights once.
"""

from __future__ import annotations

from types import SimpleNamespace

import torch
import torch.nn as nn

from . import _lib
from .attention import CausalSelfAttention
from .kernels.fp8_swa_attention import (fp8_swa_attention_forward, fp8_swa_attention_from_codes,
                                        qk_norm_rope_quant_e4m3)
from .precision import Fp8Linear


def _rows(t: torch.Tensor) -> torch.Tensor:
    """t as a 2-D [rows, last] view with unit column stride and 16-byte aligned rows (a copy when
    its layout has none)."""
    t2 = t.reshape(-1, t.shape[-1])
    if t2.stride(-1) != 1 or t2.stride(0) % 8 or t2.data_ptr() % 16:
        t2 = t2.contiguous()
    return t2


def _rmsnorm_backward(x2, weight, eps, dh, dres, shape):
    """(dx, dweight) of RMSNorm on the saved rows x2 [rows, cols] for the gradient dh; dres (or None):
    the gradient x2 receives along the residual stream, added in the same pass (flw_rmsnorm_bwd)."""
    rows, cols = x2.shape
    lib = _lib.load()
    d2 = _rows(dh.to(x2.dtype))
    r2 = _rows(dres.to(x2.dtype)) if dres is not None else None
    dx = torch.empty((rows, cols), dtype=x2.dtype, device=x2.device)
    dw = torch.empty((cols,), dtype=weight.dtype, device=weight.device)
    ws = _lib.workspace(lib.flw_rmsnorm_bwd_workspace_bytes(rows, cols), x2.device)
    _lib.check(lib.flw_rmsnorm_bwd(x2.data_ptr(), rows, cols, x2.stride(0), weight.data_ptr(), eps,
                                   d2.data_ptr(), d2.stride(0), _lib.ptr(r2), r2.stride(0) if r2 is not None else 0,
                                   dx.data_ptr(), cols, dw.data_ptr(), ws.data_ptr(), ws.numel(),
                                   _lib.stream_of(x2)), "RMSNorm backward")
    return dx.view(shape), dw


class _RMSNormFn(torch.autograd.Function):
    """RMSNorm.forward on bf16 rows as one HIP pass (flw_rmsnorm_fwd), its autograd backward as one
    more plus the weight gradient's column sum (flw_rmsnorm_bwd), rounded as torch's autograd of the
    expression rounds (base.py:336-338)."""

    @staticmethod
    def forward(ctx, x, weight, eps):
        lib = _lib.load()
        x2 = _rows(x)
        rows, cols = x2.shape
        h = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        _lib.check(lib.flw_rmsnorm_fwd(x2.data_ptr(), rows, cols, x2.stride(0), weight.data_ptr(), float(eps),
                                       h.data_ptr(), cols, _lib.stream_of(x)), "RMSNorm")
        ctx.save_for_backward(x2, weight)
        ctx.eps, ctx.shape = float(eps), x.shape
        return h

    @staticmethod
    def backward(ctx, dh):
        x2, weight = ctx.saved_tensors
        dx, dw = _rmsnorm_backward(x2, weight, ctx.eps, dh, None, ctx.shape)
        return dx, dw, None


class _RMSNormResFn(torch.autograd.Function):
    """(RMSNorm(x), x) for the block's first norm: the second output is x itself (a view) as the
    residual stream, so that the gradient x receives along that stream reaches this backward, which
    adds it to the norm's gradient in its own pass -- the sum autograd would otherwise form with a
    separate kernel where x has two uses (ln1 and the residual add, base.py:719-720)."""

    @staticmethod
    def forward(ctx, x, weight, eps):
        h = _RMSNormFn.forward(ctx, x, weight, eps)
        return h, x.view_as(x)

    @staticmethod
    def backward(ctx, dh, dres):
        x2, weight = ctx.saved_tensors
        if dh is None:
            return dres, None, None
        dx, dw = _rmsnorm_backward(x2, weight, ctx.eps, dh, dres, ctx.shape)
        return dx, dw, None


class _AddRMSNormFn(torch.autograd.Function):
    """(s, RMSNorm(s)) with s = x + a: the block's first residual add and the ln2 that reads it
    (base.py:720-721) in one pass (flw_add_rmsnorm_fwd); the backward adds s's residual-stream
    gradient to the norm's in the norm's pass, and hands the sum to both x and a, as the add's
    autograd does."""

    @staticmethod
    def forward(ctx, x, a, weight, eps):
        lib = _lib.load()
        x2, a2 = _rows(x), _rows(a)
        rows, cols = x2.shape
        s = torch.empty((rows, cols), dtype=x.dtype, device=x.device)
        h = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        _lib.check(lib.flw_add_rmsnorm_fwd(x2.data_ptr(), a2.data_ptr(), rows, cols, x2.stride(0), a2.stride(0),
                                           weight.data_ptr(), float(eps), s.data_ptr(), cols, h.data_ptr(), cols,
                                           _lib.stream_of(x)), "residual add + RMSNorm")
        ctx.save_for_backward(s, weight)
        ctx.eps, ctx.shape = float(eps), x.shape
        return s.view(x.shape), h

    @staticmethod
    def backward(ctx, ds, dh):
        s2, weight = ctx.saved_tensors
        if dh is None:
            return ds, ds, None, None
        d, dw = _rmsnorm_backward(s2, weight, ctx.eps, dh, ds, ctx.shape)
        return d, d, dw, None


class _SwiGLUFn(torch.autograd.Function):
    """silu(gate) * up on bf16 rows as one HIP pass each way (flw_swiglu_fwd / flw_swiglu_bwd),
    rounded as torch's silu, product and their autograd round (base.py:540, 550)."""

    @staticmethod
    def forward(ctx, gate, up):
        lib = _lib.load()
        g2, u2 = _rows(gate), _rows(up)
        rows, cols = g2.shape
        h = torch.empty(gate.shape, dtype=gate.dtype, device=gate.device)
        _lib.check(lib.flw_swiglu_fwd(g2.data_ptr(), u2.data_ptr(), rows, cols, g2.stride(0), u2.stride(0),
                                      h.data_ptr(), cols, None, None, 0, _lib.stream_of(gate)), "SwiGLU")
        ctx.save_for_backward(g2, u2)
        ctx.shape = gate.shape
        return h

    @staticmethod
    def backward(ctx, dh):
        g2, u2 = ctx.saved_tensors
        rows, cols = g2.shape
        lib = _lib.load()
        d2 = _rows(dh.to(g2.dtype))
        dg = torch.empty((rows, cols), dtype=g2.dtype, device=g2.device)
        du = torch.empty((rows, cols), dtype=g2.dtype, device=g2.device)
        _lib.check(lib.flw_swiglu_bwd(g2.data_ptr(), u2.data_ptr(), rows, cols, g2.stride(0), u2.stride(0),
                                      d2.data_ptr(), d2.stride(0), dg.data_ptr(), du.data_ptr(), cols, None, None, 0,
                                      _lib.stream_of(g2)), "SwiGLU backward")
        return dg.view(ctx.shape), du.view(ctx.shape)


class _Fp8GatedFn(torch.autograd.Function):
    """silu(gate(x)) * up(x) for two tensorwise Fp8Linears (base.py:538-550) as one autograd node,
    returning (h, |h| max): x is cast once for both GEMMs (the two Linears would each compute the
    same codes), the SwiGLU pass also takes h's maximum (so the down projection's cast of h skips
    its amax pass), and the backward's SwiGLU pass takes dgate's and dup's maxima for their casts.
    Every code, scale and GEMM is the one the two Fp8Linears and _SwiGLUFn compute, so the result
    equals the module route bit for bit (the gradient sum for x included: bf16(dx_gate + dx_up))."""

    @staticmethod
    def forward(ctx, x, w_gate, w_up, gate_mod, up_mod):
        from . import precision as P
        lib = _lib.load()
        x2 = _rows(x)
        M, K = x2.shape
        H = gate_mod.out_features
        ld = ((M + 127) // 128) * 128
        x8, x8t, sx = P._quantize_tensorwise_t(x2, ld)
        wg8, swg, wg8t = gate_mod.tensorwise_codes()
        wu8, swu, wu8t = up_mod.tensorwise_codes()
        g = P.scaled_mm_plain(x8, sx, wg8, swg)
        u = P.scaled_mm_plain(x8, sx, wu8, swu)
        h = torch.empty((M, H), dtype=x.dtype, device=x.device)
        amax = torch.empty(1, dtype=torch.int32, device=x.device)
        ws = _lib.workspace(lib.flw_swiglu_amax_workspace_bytes(M, H), x.device)
        _lib.check(lib.flw_swiglu_fwd(g.data_ptr(), u.data_ptr(), M, H, H, H, h.data_ptr(), H, amax.data_ptr(),
                                      ws.data_ptr(), ws.numel(), _lib.stream_of(x)), "SwiGLU")
        ctx.save_for_backward(g, u, x8t, sx, wg8, swg, wu8, swu, wg8t, wu8t)
        ctx.mods, ctx.x_shape, ctx.ld = (gate_mod, up_mod), x.shape, ld
        ctx.mark_non_differentiable(amax)
        ctx.set_materialize_grads(False)          # no zeros for the maximum's (absent) gradient
        return h.view(*x.shape[:-1], H), amax

    @staticmethod
    def backward(ctx, dh, _amax_grad):
        from . import precision as P
        g, u, x8t, sx, wg8, swg, wu8, swu, wg8t, wu8t = ctx.saved_tensors
        if dh is None:
            return None, None, None, None, None
        gate_mod, up_mod = ctx.mods
        M, H = g.shape
        lib = _lib.load()
        d2 = _rows(dh.to(g.dtype))
        dg = torch.empty((M, H), dtype=g.dtype, device=g.device)
        du = torch.empty((M, H), dtype=g.dtype, device=g.device)
        amax = torch.empty(2, dtype=torch.int32, device=g.device)
        ws = _lib.workspace(lib.flw_swiglu_amax_workspace_bytes(M, H), g.device)
        _lib.check(lib.flw_swiglu_bwd(g.data_ptr(), u.data_ptr(), M, H, H, H, d2.data_ptr(), d2.stride(0),
                                      dg.data_ptr(), du.data_ptr(), H, amax.data_ptr(), ws.data_ptr(), ws.numel(),
                                      _lib.stream_of(g)), "SwiGLU backward")
        dg8, dg8t, sdg = P._quantize_tensorwise_t(dg, ctx.ld, amax[0:1])
        du8, du8t, sdu = P._quantize_tensorwise_t(du, ctx.ld, amax[1:2])

        def w_cols(mod, w8, sw, w8t):                # as _Fp8LinearFn's backward takes them
            if getattr(mod, "_fp8_cached", None) is not None:
                return mod.weight_col_codes()
            return (w8t if w8t is not None else P.transpose_codes(w8, mod.out_features)), sw
        gx = gwg = gwu = None
        if ctx.needs_input_grad[0]:
            gx = P.scaled_mm(dg8, sdg, *w_cols(gate_mod, wg8, swg, wg8t))
            K = gx.shape[1]
            if lib.flw_fp8_scaled_mm_workspace_bytes(M, K, H) == 0:
                # unsplit: the sum of the two dgrads in the second one's epilogue, bf16(a + bf16(b))
                # as autograd's add of the two bf16 gradients gives it
                gx = P.scaled_mm_residual(du8, sdu, *w_cols(up_mod, wu8, swu, wu8t), gx)
            else:
                gx = gx + P.scaled_mm(du8, sdu, *w_cols(up_mod, wu8, swu, wu8t))
            gx = gx.view(ctx.x_shape)
        if ctx.needs_input_grad[1]:
            gwg = P.scaled_mm(dg8t, sdg, x8t, sx).to(gate_mod.weight.dtype)
        if ctx.needs_input_grad[2]:
            gwu = P.scaled_mm(du8t, sdu, x8t, sx).to(up_mod.weight.dtype)
        return gx, gwg, gwu, None, None


def _fp8_gated_ok(x: torch.Tensor, ff) -> bool:
    """The FeedForward's gate, up and down are bias-free tensorwise Fp8Linears with the FP8
    backward and 16-aligned widths, x a non-empty bf16 GPU tensor, autocast off: _Fp8GatedFn's
    route."""
    from .precision import Fp8Linear
    mods = (ff.gate, ff.up, ff.down)
    return (x.is_cuda and x.dtype == torch.bfloat16 and x.numel() > 0 and not torch.is_autocast_enabled()
            and all(type(m) is Fp8Linear and m.recipe == "tensorwise" and getattr(m, "backward_fp8", True)
                    and m.bias is None and m.in_features % 16 == 0 and m.out_features % 16 == 0 for m in mods)
            and ff.gate.out_features == ff.up.out_features and x.shape[-1] == ff.gate.in_features)


def _hip_rows_ok(*ts: torch.Tensor) -> bool:
    """bf16 GPU tensors whose last dimension the row kernels take (a multiple of 8)."""
    return all(t.is_cuda and t.dtype == torch.bfloat16 for t in ts) and ts[0].shape[-1] % 8 == 0


class RMSNorm(nn.Module):
    """base.py:324-338. bf16 on the GPU (bf16 weight, width a multiple of 8 up to 8192): the HIP
    pass pair of ``_RMSNormFn``; otherwise the reference's torch expression."""

    def __init__(self, dim: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] <= 8192 and x.numel() > 0 and _hip_rows_ok(x, self.weight):
            return _RMSNormFn.apply(x, self.weight, self.eps)
        rms = x.float().pow(2).mean(dim=-1, keepdim=True).add(self.eps).rsqrt()
        return (x.float() * rms).to(dtype=x.dtype) * self.weight


class Fp8CausalSelfAttention(CausalSelfAttention):
    """The reference's attention module with ``attn_precision: "fp8"`` and FP8 projections."""

    def __init__(self, d_model: int, num_heads: int, local_window: int | None, *, bias: bool = False,
                 recipe: str = "rowwise", granularity: str = "head", qk_norm: bool = True,
                 rope_base: float = 10000.0, max_seq_len: int = 8192) -> None:
        cfg = SimpleNamespace(d_model=d_model, num_heads=num_heads, max_seq_len=max_seq_len, rope_base=rope_base,
                              use_bias=bias, qk_norm=qk_norm, attn_precision="fp8",
                              fp8_attention_granularity=granularity)
        super().__init__(cfg, local_window)
        self.granularity = granularity
        self.qkv = Fp8Linear.from_linear(self.qkv, recipe)
        self.out = Fp8Linear.from_linear(self.out, recipe)
        self.out._is_residual_out = True


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
    """BASELINE config 5's block. ``recipe`` defaults to "rowwise" (per-output-channel weight
    scales, the configuration's stated recipe); ``qk_norm`` / ``rope_base`` / ``max_seq_len`` as
    the reference's ModelConfig fields (the RoPE tables grow on demand past ``max_seq_len``)."""

    def __init__(self, d_model: int = 1024, num_heads: int = 16, ffn_dim: int = 4096,
                 local_window: int | None = 4096, *, bias: bool = False, recipe: str = "rowwise",
                 granularity: str = "head", qk_norm: bool = True, rope_base: float = 10000.0,
                 max_seq_len: int = 8192) -> None:
        super().__init__()
        self.ln1 = RMSNorm(d_model)
        self.attn = Fp8CausalSelfAttention(d_model, num_heads, local_window, bias=bias, recipe=recipe,
                                           granularity=granularity, qk_norm=qk_norm, rope_base=rope_base,
                                           max_seq_len=max_seq_len)
        self.ln2 = RMSNorm(d_model)
        self.ff = Fp8FeedForward(d_model, ffn_dim, bias=bias, recipe=recipe)
        # Fused path: QK-norm, RoPE and the per-head maxima in the QKV GEMM's epilogue (True) or in
        # the Q / K / V quantiser's pass pair (False); the two give the same q', k' bit for bit.
        self.fuse_qk_epilogue = True

    @torch.no_grad()
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self._fusable(x):
            return self._forward_fused(x)
        return self.forward_unfused(x)

    @torch.no_grad()
    def forward_unfused(self, x: torch.Tensor) -> torch.Tensor:
        """The reference composition, one module after the other (the attention through its
        qkv_heads -- the head split, QK-norm and RoPE -- and fp8_swa_attention_forward)."""
        x = x + self.attn.forward_unfused(self.ln1(x))
        return x + self.ff(self.ln2(x))

    def _linears(self):
        return self.attn.qkv, self.attn.out, self.ff.net[0], self.ff.net[3]

    def _fusable(self, x: torch.Tensor) -> bool:
        gelu = self.ff.net[1]
        return (x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 3 and x.shape[-1] % 8 == 0
                and x.shape[-1] <= 4096 and self.ff.net[0].out_features <= 4096
                and all(l.bias is None and l.recipe == "rowwise" for l in self._linears())
                and isinstance(gelu, nn.GELU) and gelu.approximate == "none"
                and self.ln1.weight.dtype == self.ln2.weight.dtype == torch.bfloat16)

    def _forward_fused(self, x: torch.Tensor, trace: dict | None = None) -> torch.Tensor:
        """The same block with the work around the FP8 GEMMs fused into the library's kernels:
        RMSNorm -> per-row e4m3 in one pass (flw_rmsnorm_quant_rows_e4m3), QK-norm + RoPE + the
        per-head maxima in the QKV GEMM's epilogue (flw_fp8_scaled_mm_qk_norm_rope_amax) and the
        Q / K / V e4m3 from those maxima (Q on load in the attention kernel), the attention writing
        its (B, T, H, D) output in place, the residual adds in the GEMM epilogues
        (flw_fp8_scaled_mm_residual), GELU -> per-row e4m3 in one pass (flw_gelu_quant_rows_e4m3).
        Every rounding step of the unfused composition is kept (bf16 norm / GELU outputs, bf16
        linear outputs before each residual add).

        ``trace`` (a dict, for stage-by-stage checks): receives every intermediate of the call --
        the row codes / scales of each linear's input ("c1"/"s1", "ca"/"sa", "c2"/"s2",
        "cg"/"sg"), the normed / activated rows the fused quantisers also write out when tracing
        ("h1", "h2", "hg"), the QKV output "qkv" (with the epilogue: q' and k' already QK-normed
        and rotated), the QK-normed and rotated "q" / "k" heads, with the epilogue the per-head
        maxima "amax" of q', k', v, without it the attention operands "q8" / "k8" / "v_tiles" /
        "scales"; the attention output "attn", "x1" and the FF1 output "f". The kernels and the
        result are the same."""
        lib = _lib.load()
        B, T, d = x.shape
        M = B * T
        dev = x.device
        stream = _lib.stream_of(x)
        x2 = x.reshape(M, d)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        qkv_l, out_l, ff1_l, ff2_l = self._linears()

        def codes_of(kind, src, cols, norm=None, h_name=None):
            c = torch.empty((M, cols), dtype=torch.uint8, device=dev)
            sc = torch.empty(M, dtype=torch.float32, device=dev)
            h = None
            if trace is not None and h_name is not None:
                h = trace[h_name] = torch.empty((M, cols), dtype=torch.bfloat16, device=dev)
            hp = None if h is None else h.data_ptr()
            if kind == "rmsnorm":
                rc = lib.flw_rmsnorm_quant_rows_e4m3(src.data_ptr(), M, cols, cols, norm.weight.data_ptr(),
                                                     float(norm.eps), c.data_ptr(), sc.data_ptr(), hp, stream)
            elif kind == "gelu":
                rc = lib.flw_gelu_quant_rows_e4m3(src.data_ptr(), M, cols, cols, c.data_ptr(), sc.data_ptr(),
                                                  hp, stream)
            else:
                rc = lib.flw_quant_rows_e4m3(src.data_ptr(), _lib.BF16, M, cols, cols, c.data_ptr(),
                                             sc.data_ptr(), stream)
            _lib.check(rc, kind)
            return c, sc

        def linear(codes, sc, lin, residual=None):
            w8, ws = lin.weight_codes()
            N, K = w8.shape
            y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            if residual is None:
                rc = lib.flw_fp8_scaled_mm(codes.data_ptr(), M, K, w8.data_ptr(), N, sc.data_ptr(), M,
                                           ws.data_ptr(), ws.numel(), y.data_ptr(), N, stream)
            else:
                rc = lib.flw_fp8_scaled_mm_residual(codes.data_ptr(), M, K, w8.data_ptr(), N, sc.data_ptr(), M,
                                                    ws.data_ptr(), ws.numel(), y.data_ptr(), N,
                                                    residual.data_ptr(), residual.stride(0), stream)
            _lib.check(rc, "fp8 linear")
            return y

        att = self.attn
        c1, s1 = codes_of("rmsnorm", x2, d, self.ln1, "h1")
        cos, sin = att.rope.tables(T, torch.bfloat16, dev)
        qk_norm = att.qk_norm is not None
        eps = att.qk_norm.eps if qk_norm else 0.0
        a = torch.empty((B, T, d), dtype=torch.bfloat16, device=dev)
        a_heads = a.view(B, T, att.num_heads, att.head_dim).transpose(1, 2)
        window = T if att.local_window is None else att.local_window
        if self.fuse_qk_epilogue and att.granularity == "head" and d % 128 == 0 and M * d < 2 ** 32 \
                and 3 * d * d < 2 ** 32:
            # The quantisation point of qkv_heads (base.py:630-637) in the QKV GEMM's epilogue: the q
            # and k heads are QK-normed and rotated before they are stored, and the per-head maxima
            # of q', k', v come with them, so the attention's quantiser runs only its quantise pass
            # (K / V codes; Q is quantised on load by the attention kernel). The 256 x 256 GEMM
            # (K % 128 == 0, operands < 2^32 bytes) carries this epilogue; other shapes take the
            # quantiser pair below.
            w8, ws = qkv_l.weight_codes()
            N, K = w8.shape
            qkv = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            amax = torch.empty(N // att.head_dim, dtype=torch.int32, device=dev)
            _lib.check(lib.flw_fp8_scaled_mm_qk_norm_rope_amax(
                c1.data_ptr(), M, K, w8.data_ptr(), N, s1.data_ptr(), M, ws.data_ptr(), ws.numel(), qkv.data_ptr(),
                N, att.head_dim, 2 * d, int(qk_norm), float(eps), cos.data_ptr(), sin.data_ptr(), T, amax.data_ptr(),
                stream), "qkv + qk-norm + rope + amax")
            qkv = qkv.view(B, T, 3 * d)
            q, k, v = (att._split(t) for t in qkv.chunk(3, dim=-1))
            fp8_swa_attention_forward(q, k, v, window, granularity="head", out=a_heads, amax=amax)
            if trace is not None:
                trace.update(q=q, k=k, amax=amax)
        else:
            # HeadRMSNorm and RoPE of q, k and the three e4m3 quantisations in one pass pair over the
            # strided head views of the projection.
            qkv = linear(c1, s1, qkv_l).view(B, T, 3 * d)
            q, k, v = (att._split(t) for t in qkv.chunk(3, dim=-1))
            res = qk_norm_rope_quant_e4m3(q, k, v, qk_norm=qk_norm, eps=eps, rope_cos=cos, rope_sin=sin,
                                          granularity=att.granularity, return_transformed=trace is not None)
            fp8_swa_attention_from_codes(*res[:4], window, granularity=att.granularity, out=a_heads)
            if trace is not None:
                trace.update(q=res[4], k=res[5], q8=res[0], k8=res[1], v_tiles=res[2], scales=res[3])
        ca, sa = codes_of("plain", a.view(M, d), d)
        x1 = linear(ca, sa, out_l, residual=x2)
        c2, s2 = codes_of("rmsnorm", x1, d, self.ln2, "h2")
        f = linear(c2, s2, ff1_l)
        cg, sg = codes_of("gelu", f, f.shape[1], h_name="hg")
        if trace is not None:
            trace.update(c1=c1, s1=s1, qkv=qkv, attn=a, ca=ca, sa=sa, x1=x1, c2=c2, s2=s2, f=f, cg=cg, sg=sg)
        return linear(cg, sg, ff2_l, residual=x1).view(B, T, d)


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


def swiglu_hidden_dim(ffn_dim: int, param_match: bool = True) -> int:
    """SwiGLU hidden width for a nominal ``ffn_dim`` (base.py:370-383): with ``param_match`` the
    three d x h matrices get the parameters of GELU's two, 2/3 of the width rounded to a multiple
    of 64 (5120 -> 3392)."""
    if not param_match:
        return ffn_dim
    return max(64, round(((ffn_dim * 2) // 3) / 64) * 64)


class FeedForward(nn.Module):
    """base.py:485-552 without dropout (0 in the 450M configs): the GELU MLP (``net.0``, GELU,
    ``net.3``) or SwiGLU (``down(silu(gate(x)) * up(x))``), by ``config.ffn_activation``. Plain
    nn.Linear layers, which ``convert_model_to_fp8`` replaces by Fp8Linear as the reference's
    conversion replaces them by Float8Linear."""

    def __init__(self, config) -> None:
        super().__init__()
        d, ffn = config.d_model, config.ffn_dim
        bias = bool(getattr(config, "use_bias", True))
        self.activation = getattr(config, "ffn_activation", "gelu")
        if self.activation not in {"gelu", "swiglu"}:
            raise ValueError(f"ffn_activation must be 'gelu' or 'swiglu', got {self.activation!r}")
        if self.activation == "gelu":
            self.net = nn.Sequential(nn.Linear(d, ffn, bias=bias), nn.GELU(), nn.Identity(),
                                     nn.Linear(ffn, d, bias=bias))
            self.net[-1]._is_residual_out = True
        else:
            hidden = swiglu_hidden_dim(ffn, bool(getattr(config, "ffn_param_match", True)))
            self.hidden_dim = hidden
            self.gate = nn.Linear(d, hidden, bias=bias)
            self.up = nn.Linear(d, hidden, bias=bias)
            self.down = nn.Linear(hidden, d, bias=bias)
            self.down._is_residual_out = True

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
        """residual: returns ``residual + ff(x)`` (the block's second residual add), inside the down
        projection's GEMM epilogue on the fused FP8 route."""
        if self.activation == "gelu":
            out = self.net(x)
        elif _fp8_gated_ok(x, self):
            h, h_amax = _Fp8GatedFn.apply(x, self.gate.weight, self.up.weight, self.gate, self.up)
            return self.down(h, x_amax=h_amax, residual=residual)
        else:
            gate, up = self.gate(x), self.up(x)
            if gate.numel() > 0 and _hip_rows_ok(gate, up):
                out = self.down(_SwiGLUFn.apply(gate, up))
            else:
                out = self.down(torch.nn.functional.silu(gate) * up)
        return out if residual is None else residual + out


class TransformerBlock(nn.Module):
    """base.py:698-722 for training: ``x + attn(ln1(x))``, then ``+ ff(ln2(x))``, returning
    ``(x, memory)`` as the reference's block does. The attention is ``CausalSelfAttention`` (the
    HIP bf16 sliding-window kernels, or the FP8 route with ``attn_precision: "fp8"``) with the
    config's window; RMSNorm norms (``norm_type: rmsnorm``, the 450M configs' choice)."""

    def __init__(self, config) -> None:
        super().__init__()
        if getattr(config, "norm_type", "rmsnorm") != "rmsnorm":
            raise ValueError("only norm_type 'rmsnorm' is built")
        self.ln1 = RMSNorm(config.d_model)
        self.attn = CausalSelfAttention(config, getattr(config, "local_window", None))
        self.ln2 = RMSNorm(config.d_model)
        self.ff = FeedForward(config)

    def forward(self, x: torch.Tensor, memory: torch.Tensor | None = None):
        d = x.shape[-1]
        if d % 8 == 0 and d <= 8192 and x.numel() > 0 and _hip_rows_ok(x, self.ln1.weight, self.ln2.weight):
            # bf16 on the GPU: ln1 hands x on as the residual stream and ln2 takes the first
            # residual add into its pass, so the norms' backward passes also add the residual
            # gradients (the same bf16 sums autograd forms for x's and x1's two uses).
            h1, xr = _RMSNormResFn.apply(x, self.ln1.weight, self.ln1.eps)
            x1, h2 = _AddRMSNormFn.apply(xr, self.attn(h1), self.ln2.weight, self.ln2.eps)
            return self.ff(h2, residual=x1), memory
        x = x + self.attn(self.ln1(x))
        x = x + self.ff(self.ln2(x))
        return x, memory


def block_config(**overrides) -> SimpleNamespace:
    """The 450M ``vanilla_matched`` block (configs/sweep13_450m_longctx_fp8.yaml:94-113): d_model
    1280, 20 heads, ffn 5120 as param-matched SwiGLU (3392), window 2048, RoPE 10000, QK-norm,
    RMSNorm, no biases, bf16 attention."""
    cfg = dict(d_model=1280, num_heads=20, ffn_dim=5120, ffn_activation="swiglu", ffn_param_match=True,
               local_window=2048, rope_base=10000.0, qk_norm=True, norm_type="rmsnorm", use_bias=False,
               max_seq_len=8192, attn_precision="bf16")
    cfg.update(overrides)
    return SimpleNamespace(**cfg)


__all__ = ["RMSNorm", "Fp8CausalSelfAttention", "Fp8FeedForward", "Fp8DecoderBlock", "init_block_",
           "block_flops", "swiglu_hidden_dim", "FeedForward", "TransformerBlock", "block_config"]
