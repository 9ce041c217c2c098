"""FP8 linear layers and the FP8 weight cache, on the HIP library (gfx950).

Mirrors flower/precision.py (the torchao-based FP8 conversion) with this build's own FP8 linear:

``_FP8_DIM_ALIGNMENT``, ``_block_index``, ``fp8_module_filter``  -- precision.py:56-98, the same
    guardrails (aligned dims, only Linears under ``blocks.<i>``, first/last ``keep`` blocks bf16).
``Fp8Linear``          -- replaces torchao ``Float8Linear``: forward is the HIP FP8 GEMM
    (e4m3 weight x e4m3 per-row activation, fp32 accumulate, bf16 out, the ``_fp8_head``
    recipe of base.py:911-923). recipe "rowwise": per-output-channel weight scales, per-row
    activation scales; "tensorwise": one weight scale and one activation scale; "weight_only":
    per-output-channel e4m3 weights times the bf16 activations as they are (W8A16: the weight is
    widened to bf16 in the kernel, bf16 MFMA; needs K % 64 == 0).
    Backward ("rowwise" / "tensorwise", as torchao's Float8Linear does under
    ``training.fp8_linear``): both gradient GEMMs in FP8 on the same kernel —
    dgrad  grad_x = g W:    per-row e4m3 g (per tensor for "tensorwise") x the weight's per-column
                            e4m3 codes stored transposed (cached with the forward codes);
    wgrad  grad_W = g^T x:  per-column e4m3 of g and of x (the token axis becomes the contiguous
                            reduction), written transposed by flw_quant_cols_e4m3.
    "weight_only" (and ``backward_fp8 = False``) keeps the bf16 matmul pair.
``convert_model_to_fp8`` / ``maybe_convert_fp8`` -- precision.py:134-195, 356-381.
``fp8_weight_cache``   -- precision.py:198-353: quantise every FP8 weight ONCE on entry, patch
    the layers' forwards to reuse it across grad-accumulation microsteps, restore the forwards
    on exit (also on an exception), and raise RuntimeError("...stale...") when a sampled
    fingerprint of any cached weight changed while the cache was live.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib

_FP8_DIM_ALIGNMENT = 16
RECIPES = ("rowwise", "tensorwise", "weight_only")


def _block_index(fqn: str) -> int | None:
    """Index of the ``blocks.<i>`` a module FQN sits under, or None."""
    parts = fqn.split(".")
    for a, b in zip(parts[:-1], parts[1:]):
        if a == "blocks" and b.isdigit():
            return int(b)
    return None


def fp8_module_filter(num_layers: int, keep_bf16_blocks: int):
    """``(module, fqn) -> bool``: which Linears become FP8 (precision.py:73-98 rules)."""

    def should_convert(module: nn.Module, fqn: str) -> bool:
        if not isinstance(module, nn.Linear):
            return False
        if module.in_features % _FP8_DIM_ALIGNMENT or module.out_features % _FP8_DIM_ALIGNMENT:
            return False
        idx = _block_index(fqn)
        if idx is None:                      # LM head, MTP heads, model-level projections
            return False
        if keep_bf16_blocks > 0 and (idx < keep_bf16_blocks or idx >= num_layers - keep_bf16_blocks):
            return False
        return True

    return should_convert


# ---------------------------------------------------------------- weight / activation quantisers

def quantize_weight(weight: torch.Tensor, recipe: str = "rowwise"):
    """(w8 [N, K] uint8 e4m3 codes, w_scale float32 [N] or [1]) on the weight's device."""
    lib = _lib.load()
    _lib.require_gpu(weight)
    w = weight.detach()
    if w.dtype not in (torch.float32, torch.bfloat16):
        w = w.to(torch.bfloat16)
    w = w.contiguous()
    N, K = w.shape
    w8 = torch.empty((N, K), dtype=torch.uint8, device=w.device)
    if recipe in ("rowwise", "weight_only"):
        scale = torch.empty(N, dtype=torch.float32, device=w.device)
        rc = lib.flw_quant_rows_e4m3(w.data_ptr(), _lib.dtype_code(w.dtype), N, K, K, w8.data_ptr(),
                                     scale.data_ptr(), _lib.stream_of(w))
        _lib.check(rc, "quantize_weight")
    elif recipe == "tensorwise":
        scale = torch.empty(1, dtype=torch.float32, device=w.device)
        ws = _lib.workspace(lib.flw_quant_workspace_bytes(1, 1, N, K), w.device)
        rc = lib.flw_quant_e4m3(w.data_ptr(), _lib.dtype_code(w.dtype), 1, 1, N, K, N * K, N * K, K,
                                _lib.SCALE_TENSOR, _lib.LAYOUT_BHTD, w8.data_ptr(), scale.data_ptr(),
                                ws.data_ptr(), ws.numel(), _lib.stream_of(w))
        _lib.check(rc, "quantize_weight")
    else:
        raise RuntimeError(f"training.fp8_recipe must be one of {sorted(RECIPES)}, got {recipe!r}")
    return w8, scale


def quantize_cols(x2: torch.Tensor, granularity: str, ld: int | None = None):
    """(codes_t [C, ld] uint8, scale float32 [C] or [1]): e4m3 of each column of x2 [R, C] (bf16 or
    fp32, rows contiguous), transposed; rows past R up to ld (a multiple of 16) are coded 0."""
    lib = _lib.load()
    _lib.require_gpu(x2)
    if x2.dtype not in (torch.float32, torch.bfloat16):
        x2 = x2.to(torch.bfloat16)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    R, C = x2.shape
    ld = ((R + 15) // 16) * 16 if ld is None else ld
    gran = _lib.SCALE_COLUMN if granularity == "column" else _lib.SCALE_TENSOR
    out = torch.empty((C, ld), dtype=torch.uint8, device=x2.device)
    scale = torch.empty(C if gran == _lib.SCALE_COLUMN else 1, dtype=torch.float32, device=x2.device)
    ws = _lib.workspace(lib.flw_quant_cols_workspace_bytes(R, C), x2.device)
    rc = lib.flw_quant_cols_e4m3(x2.data_ptr(), _lib.dtype_code(x2.dtype), R, C, x2.stride(0), gran,
                                 out.data_ptr(), ld, scale.data_ptr(), ws.data_ptr(), ws.numel(),
                                 _lib.stream_of(x2))
    _lib.check(rc, "quantize_cols")
    return out, scale


def quantize_weight_cols(weight: torch.Tensor, recipe: str = "rowwise"):
    """The weight's codes for dgrad: (w8c [K, N] = per-column e4m3 of W [N, K], transposed;
    scales [K] ("rowwise") or [1] ("tensorwise"))."""
    w = weight.detach()
    return quantize_cols(w, "column" if recipe == "rowwise" else "tensor", ld=w.shape[0])


def _quantize_rows(x2: torch.Tensor, recipe: str):
    """(x8 [M, K], scale [M] or [1]) of a contiguous bf16 / fp32 matrix, per row ("rowwise") or
    per tensor ("tensorwise")."""
    lib = _lib.load()
    M, K = x2.shape
    x8 = torch.empty((M, K), dtype=torch.uint8, device=x2.device)
    stream = _lib.stream_of(x2)
    if recipe == "rowwise":
        sx = torch.empty(M, dtype=torch.float32, device=x2.device)
        rc = lib.flw_quant_rows_e4m3(x2.data_ptr(), _lib.dtype_code(x2.dtype), M, K, x2.stride(0),
                                     x8.data_ptr(), sx.data_ptr(), stream)
    else:
        sx = torch.empty(1, dtype=torch.float32, device=x2.device)
        ws = _lib.workspace(lib.flw_quant_workspace_bytes(1, 1, M, K), x2.device)
        rc = lib.flw_quant_e4m3(x2.data_ptr(), _lib.dtype_code(x2.dtype), 1, 1, M, K, M * x2.stride(0),
                                M * x2.stride(0), x2.stride(0), _lib.SCALE_TENSOR, _lib.LAYOUT_BHTD,
                                x8.data_ptr(), sx.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "quantize rows")
    return x8, sx


def scaled_mm(a8: torch.Tensor, sa: torch.Tensor, b8: torch.Tensor, sb: torch.Tensor) -> torch.Tensor:
    """bf16 [M, N] = (a8 [M, K] . b8 [N, K]^T) * sa[m] * sb[n] through flw_fp8_scaled_mm_ws (split
    over K into a workspace when [M, N] has too few output tiles to fill the GPU)."""
    lib = _lib.load()
    M, K = a8.shape
    N = b8.shape[0]
    y = torch.empty((M, N), dtype=torch.bfloat16, device=a8.device)
    ws = _lib.workspace(lib.flw_fp8_scaled_mm_workspace_bytes(M, N, K), a8.device)
    rc = lib.flw_fp8_scaled_mm_ws(a8.data_ptr(), M, K, b8.data_ptr(), N, sa.data_ptr(), sa.numel(),
                                  sb.data_ptr(), sb.numel(), y.data_ptr(), N, ws.data_ptr(), ws.numel(),
                                  _lib.stream_of(a8))
    _lib.check(rc, "fp8_scaled_mm")
    return y


def fp8_linear_backward(g2: torch.Tensor, x2: torch.Tensor, w_cols, recipe: str,
                        need_x: bool = True, need_w: bool = True):
    """FP8 gradient GEMMs of y = x W^T: (grad_x [M, K], grad_W [N, K]), bf16.

    g2: [M, N] output gradient, x2: [M, K] the forward input, w_cols: (w8c [K, N], scale) from
    ``quantize_weight_cols`` (or a callable returning it). Row / column granularity per recipe:
    "rowwise" -> g per row for dgrad, g and x per column for wgrad; "tensorwise" -> one scale per
    tensor everywhere. The token axis is zero-padded to a multiple of 128 for wgrad."""
    gx = gw = None
    g2 = g2.to(torch.bfloat16).contiguous()
    if need_x:
        g8, sg = _quantize_rows(g2, recipe)
        w8c, swc = w_cols() if callable(w_cols) else w_cols
        gx = scaled_mm(g8, sg, w8c, swc)
    if need_w:
        gran = "column" if recipe == "rowwise" else "tensor"
        M = g2.shape[0]
        ld = ((M + 127) // 128) * 128
        g8c, sgc = quantize_cols(g2, gran, ld)
        x8c, sxc = quantize_cols(x2, gran, ld)
        gw = scaled_mm(g8c, sgc, x8c, sxc)
    return gx, gw


def fp8_linear_forward(x: torch.Tensor, w8: torch.Tensor, w_scale: torch.Tensor,
                       recipe: str = "rowwise") -> torch.Tensor:
    """bf16 y[..., N] = x[..., K] @ dequant(w8)^T through the HIP FP8 GEMM."""
    lib = _lib.load()
    _lib.require_gpu(x, w8)
    N, K = w8.shape
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    if x2.dtype != torch.bfloat16:
        x2 = x2.to(torch.bfloat16)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    M = x2.shape[0]
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    if M == 0:
        return y.reshape(*lead, N)
    stream = _lib.stream_of(x2)
    if recipe == "weight_only":
        rc = lib.flw_fp8_linear(x2.data_ptr(), M, K, x2.stride(0), w8.data_ptr(), N, w_scale.data_ptr(),
                                w_scale.numel(), _lib.GEMM_W8A16, y.data_ptr(), N, None, 0, stream)
        _lib.check(rc, "fp8_linear(weight_only)")
    elif recipe == "rowwise":
        ws = _lib.workspace(lib.flw_fp8_linear_workspace_bytes(M, K, _lib.GEMM_A8W8), x.device)
        rc = lib.flw_fp8_linear(x2.data_ptr(), M, K, x2.stride(0), w8.data_ptr(), N, w_scale.data_ptr(),
                                w_scale.numel(), _lib.GEMM_A8W8, y.data_ptr(), N, ws.data_ptr(),
                                ws.numel(), stream)
        _lib.check(rc, "fp8_linear")
    else:
        x8 = torch.empty((M, K), dtype=torch.uint8, device=x.device)
        sx = torch.empty(1, dtype=torch.float32, device=x.device)
        ws = _lib.workspace(lib.flw_quant_workspace_bytes(1, 1, M, K), x.device)
        rc = lib.flw_quant_e4m3(x2.data_ptr(), _lib.BF16, 1, 1, M, K, M * x2.stride(0), M * x2.stride(0),
                                x2.stride(0), _lib.SCALE_TENSOR, _lib.LAYOUT_BHTD, x8.data_ptr(),
                                sx.data_ptr(), ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, "fp8_linear(tensorwise activation)")
        rc = lib.flw_fp8_scaled_mm(x8.data_ptr(), M, K, w8.data_ptr(), N, sx.data_ptr(), 1,
                                   w_scale.data_ptr(), w_scale.numel(), y.data_ptr(), N, stream)
        _lib.check(rc, "fp8_scaled_mm")
    return y.reshape(*lead, N)


class _Fp8LinearFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, w8, w_scale, recipe, mod):
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        ctx.recipe, ctx.mod = recipe, mod
        y = fp8_linear_forward(x, w8, w_scale, recipe)
        if bias is not None:
            y = y + bias.to(y.dtype)
        return y

    @staticmethod
    def backward(ctx, g):
        x, weight = ctx.saved_tensors
        g2 = g.reshape(-1, g.shape[-1])
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        N, K = weight.shape
        # FP8 gradient GEMMs need 16-aligned dims (the conversion filter guarantees them; a
        # hand-built Fp8Linear may not): otherwise the bf16 pair below.
        fp8 = (ctx.recipe in ("rowwise", "tensorwise") and getattr(ctx.mod, "backward_fp8", True)
               and N % 16 == 0 and K % 16 == 0)
        gx = gw = None
        if fp8 and (need_x or need_w):
            x2 = x.reshape(-1, x.shape[-1])
            gx, gw = fp8_linear_backward(g2, x2, ctx.mod.weight_col_codes, ctx.recipe, need_x, need_w)
            gx = gx.reshape(x.shape).to(x.dtype) if gx is not None else None
            gw = gw.to(weight.dtype) if gw is not None else None
        else:
            w = weight.to(g2.dtype)
            gx = (g2 @ w).reshape(x.shape).to(x.dtype) if need_x else None
            if need_w:
                gw = (g2.t() @ x.reshape(-1, x.shape[-1]).to(g2.dtype)).to(weight.dtype)
        gb = g2.sum(0) if ctx.has_bias and ctx.needs_input_grad[2] else None
        return gx, gw, gb, None, None, None, None


class Fp8Linear(nn.Linear):
    """``nn.Linear`` whose forward runs the HIP FP8 GEMM (weights quantised on every call unless
    an ``fp8_weight_cache`` is active). Shares the Parameters of the Linear it was built from."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True, device=None,
                 dtype=None, *, recipe: str = "rowwise") -> None:
        if recipe not in RECIPES:
            raise RuntimeError(f"training.fp8_recipe must be one of {sorted(RECIPES)}, got {recipe!r}")
        super().__init__(in_features, out_features, bias=bias, device=device, dtype=dtype)
        self.recipe = recipe
        self.backward_fp8 = True

    @classmethod
    def from_linear(cls, lin: nn.Linear, recipe: str = "rowwise") -> "Fp8Linear":
        if recipe not in RECIPES:
            raise RuntimeError(f"training.fp8_recipe must be one of {sorted(RECIPES)}, got {recipe!r}")
        new = cls.__new__(cls)
        nn.Module.__init__(new)
        new.in_features, new.out_features = lin.in_features, lin.out_features
        # same Parameter objects: an optimizer built before or after conversion sees them
        new.register_parameter("weight", lin.weight)
        new.register_parameter("bias", lin.bias)
        new.recipe = recipe
        new.backward_fp8 = True
        new.train(lin.training)
        return new

    def quantize_weight(self):
        return quantize_weight(self.weight, self.recipe)

    def weight_codes(self):
        """(w8, w_scale): the fp8_weight_cache's copy while one is active, else quantised now."""
        cached = getattr(self, "_fp8_cached", None)
        return cached if cached is not None else self.quantize_weight()

    def weight_col_codes(self):
        """(w8c [K, N], scale) for the dgrad GEMM: quantised once per fp8_weight_cache context
        (on the first backward inside it), else on every call."""
        cached = getattr(self, "_fp8_cached_cols", None)
        if cached is not None:
            return cached
        codes = quantize_weight_cols(self.weight, self.recipe)
        if getattr(self, "_fp8_cached", None) is not None:       # a cache context is active
            self._fp8_cached_cols = codes
        return codes

    def forward_with(self, x: torch.Tensor, w8: torch.Tensor, w_scale: torch.Tensor) -> torch.Tensor:
        if torch.is_autocast_enabled():
            x = x.to(torch.get_autocast_gpu_dtype())
        return _Fp8LinearFn.apply(x, self.weight, self.bias, w8, w_scale, self.recipe, self)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        w8, w_scale = self.quantize_weight()
        return self.forward_with(x, w8, w_scale)

    def extra_repr(self) -> str:
        return super().extra_repr() + f", recipe={self.recipe}"


def convert_model_to_fp8(model: nn.Module, *, recipe: str = "rowwise", keep_bf16_blocks: int = 1,
                         use_fast_accum: bool = False, verbose: bool = True):
    """Swap eligible ``nn.Linear`` layers for ``Fp8Linear`` in place; returns (model, info).

    ``use_fast_accum`` is accepted for config compatibility; the MFMA accumulates in fp32 always.
    """
    if recipe not in RECIPES:
        raise RuntimeError(f"training.fp8_recipe must be one of {sorted(RECIPES)}, got {recipe!r}")
    num_layers = len(getattr(model, "blocks", []))
    if num_layers == 0:
        raise RuntimeError(
            "convert_model_to_fp8 found no `blocks` on the model; the block-range "
            "guardrail cannot be applied. Refusing to convert blindly.")
    keep = fp8_module_filter(num_layers, keep_bf16_blocks)
    eligible = [(fqn, m) for fqn, m in model.named_modules() if keep(m, fqn)]
    total_linear = sum(1 for _, m in model.named_modules() if isinstance(m, nn.Linear))
    for fqn, mod in eligible:
        parent_name, _, child = fqn.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        setattr(parent, child, Fp8Linear.from_linear(mod, recipe))
    info = {
        "fp8_recipe": recipe,
        "fp8_keep_bf16_blocks": keep_bf16_blocks,
        "fp8_use_fast_accum": use_fast_accum,
        "fp8_converted_linears": len(eligible),
        "fp8_total_linears": total_linear,
    }
    if verbose:
        print(f"[fp8] recipe={recipe} converted {len(eligible)}/{total_linear} Linear layers "
              f"(blocks {keep_bf16_blocks}..{num_layers - keep_bf16_blocks - 1} of {num_layers}; "
              f"first/last {keep_bf16_blocks} and the tied LM head stay bf16)", flush=True)
    return model, info


def maybe_convert_fp8(model: nn.Module, training_cfg, device):
    """Apply FP8 conversion if ``training.fp8_linear`` is set; otherwise a no-op."""
    if not getattr(training_cfg, "fp8_linear", False):
        return model, {}
    if device.type != "cuda":
        raise RuntimeError("training.fp8_linear requires a GPU (ROCm)")
    if training_cfg.precision != "bf16":
        raise RuntimeError(
            "training.fp8_linear requires training.precision: bf16 "
            f"(FP8 layers consume bf16 activations), got {training_cfg.precision!r}")
    return convert_model_to_fp8(
        model,
        recipe=getattr(training_cfg, "fp8_recipe", "rowwise"),
        keep_bf16_blocks=int(training_cfg.fp8_keep_bf16_blocks),
        use_fast_accum=bool(getattr(training_cfg, "fp8_use_fast_accum", False)),
    )


class fp8_weight_cache:
    """Cache each FP8 layer's quantised weight across accumulation microsteps.

    Usage:
        with fp8_weight_cache(model):
            for _ in range(accum):
                model(...).backward()
        optimizer.step()

    The cache is only valid while the weights do not change, which a version counter cannot
    tell (``p.data -= x`` does not bump ``_version``), so invalidation is explicit: the cache
    lives inside this context only, and on exit a sampled fingerprint of every cached weight is
    re-checked; a change raises RuntimeError ("stale") unless the context exits by an exception.
    """

    _FINGERPRINT_STRIDE = 4096

    def __init__(self, model: nn.Module, *, verify: bool = True) -> None:
        self.model = model
        self.verify = verify
        self._layers: list = []
        self._orig_forwards: dict = {}
        self._fingerprints: dict = {}

    @staticmethod
    def _fingerprint(w) -> float:
        flat = w.detach().reshape(-1)
        return float(flat[:: fp8_weight_cache._FINGERPRINT_STRIDE].float().sum())

    def __enter__(self):
        for mod in self.model.modules():
            if not isinstance(mod, Fp8Linear):
                continue
            w8, w_scale = mod.quantize_weight()

            def cached_forward(x, _mod=mod, _w8=w8, _s=w_scale):
                return _mod.forward_with(x, _w8, _s)

            self._orig_forwards[mod] = mod.forward
            mod.forward = cached_forward
            mod._fp8_cached = (w8, w_scale)
            self._layers.append(mod)
            if self.verify:
                self._fingerprints[mod] = self._fingerprint(mod.weight)
        return self

    def __exit__(self, exc_type, exc, tb):
        changed = []
        for mod in self._layers:
            mod.forward = self._orig_forwards[mod]
            mod._fp8_cached = None
            mod._fp8_cached_cols = None
            if self.verify and exc_type is None:
                if self._fingerprint(mod.weight) != self._fingerprints[mod]:
                    changed.append(mod)
        self._layers.clear()
        self._orig_forwards.clear()
        self._fingerprints.clear()
        if changed:
            raise RuntimeError(
                f"fp8_weight_cache: {len(changed)} weight(s) were modified while the cache was "
                "active, so the cached FP8 weights were stale. The cache must not span an "
                "optimizer step. This is raised rather than silently training on stale weights.")
        return False
