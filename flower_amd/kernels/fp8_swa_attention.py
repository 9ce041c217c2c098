"""FP8 sliding-window causal attention forward on MI355X (gfx950), reference-compatible API.

Same operator surface as flower/kernels/fp8_swa_attention.py:92-273:

  ``E4M3_MAX``                   -- :92
  ``_per_tensor_fp8(x)``         -- :195-205, returns the scale as a device tensor (no .item())
  ``fp8_swa_attention_forward``  -- :208-259, same signature; the Triton tuning keywords are
                                    accepted and ignored (the HIP kernel has one tuned geometry)
  ``reference_swa_attention``    -- :262-273, dense fp32 reference (plain torch, small T only)

Everything on the hot path runs in libflower_amd.so (HIP, gfx950): the amax + e4m3 quantisers
for Q, K, V and the fused FP8 MFMA attention kernel. Scales never leave the device, so a call
is fully asynchronous on the current stream (the reference does three ``.item()`` syncs).

``granularity`` (keyword-only, default "tensor" as in the reference) selects per-tensor,
per-head ("head": amax over B, T, D of each head) or per-(b, h) ("bh") e4m3 scales.
"""

from __future__ import annotations

import torch

from .. import _lib

E4M3_MAX = 448.0


def _check_bhtd(x: torch.Tensor, name: str) -> None:
    if x.dim() != 4:
        raise ValueError(f"expected (B, H, T, D), got {tuple(x.shape)}")
    if x.stride(-1) != 1:
        raise ValueError(f"{name} must be contiguous in its last dimension")


def _rowmajor_strides(x: torch.Tensor, vec: int):
    """(b, h, t) element strides if the kernel can read x in place, else None."""
    sb, sh, st, sd = x.stride()
    ok = sd == 1 and sb % vec == 0 and sh % vec == 0 and st % vec == 0 and x.data_ptr() % 16 == 0
    return (sb, sh, st) if ok else None


def _prepare(x: torch.Tensor):
    vec = 4 if x.dtype == torch.float32 else 8
    s = _rowmajor_strides(x, vec)
    if s is None:
        x = x.contiguous()
        s = _rowmajor_strides(x, vec)
    return x, s


def _as_bhtd(x: torch.Tensor, granularity: str):
    """x as a (B, H, T, D) tensor with 16-byte rows, its strides and its scale-group count."""
    if x.numel() == 0:
        raise ValueError("cannot quantise an empty tensor")
    shape = x.shape
    if x.dim() == 4:
        x4 = x
    elif granularity == "tensor":
        last = shape[-1] if x.dim() else 1
        x4 = x.reshape(1, 1, -1, last)
    else:
        raise ValueError(f"expected (B, H, T, D) for {granularity} scales, got {tuple(shape)}")
    x4, strides = _prepare(x4)
    B, H, T, D = x4.shape
    return x4, strides, {"tensor": 1, "head": H, "bh": B * H}[granularity]


def _per_tensor_fp8(x: torch.Tensor, granularity: str = "tensor"):
    """e4m3 quantisation with an amax scale: (x_e4m3, scale).

    scale = max(amax, 1e-12) / 448 in fp32; codes = e4m3(clamp(x / scale, -448, 448)), with IEEE
    division and round-to-nearest-even. ``scale`` is a float32 device tensor of 1 (tensor),
    H (head) or B*H (bh) elements; ``float(scale)`` is the reference's Python float.
    Accepts any shape for per-tensor scaling; per-head / per-(b, h) need (B, H, T, D).
    """
    lib = _lib.load()
    _lib.require_gpu(x)
    x4, (sb, sh, st), G = _as_bhtd(x, granularity)
    B, H, T, D = x4.shape
    out = torch.empty((B, H, T, D), dtype=torch.uint8, device=x.device)
    scale = torch.empty(G, dtype=torch.float32, device=x.device)
    ws = _lib.workspace(lib.flw_quant_workspace_bytes(B, H, T, D), x.device)
    rc = lib.flw_quant_e4m3(x4.data_ptr(), _lib.dtype_code(x.dtype), B, H, T, D, sb, sh, st,
                            _lib.GRANULARITY[granularity], _lib.LAYOUT_BHTD, out.data_ptr(),
                            scale.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(x))
    _lib.check(rc, "_per_tensor_fp8")
    return out.view(torch.float8_e4m3fn).reshape(x.shape), scale


def amax_e4m3(x: torch.Tensor, granularity: str = "tensor") -> torch.Tensor:
    """The amax pass of ``_per_tensor_fp8`` alone (fp8_swa_attention.py:201): |x| max per scale
    group as a float32 device tensor of 1, H or B*H elements (NaN propagates).

    For a tensor split across shards: each shard's amax, combined with an all_reduce(MAX) (it can
    run on ``amax.view(torch.int32)``: non-negative floats order like their bit patterns), then
    ``quantize_e4m3_with_amax`` on every shard gives the codes and scale of the whole tensor.
    """
    lib = _lib.load()
    _lib.require_gpu(x)
    x4, (sb, sh, st), G = _as_bhtd(x, granularity)
    B, H, T, D = x4.shape
    amax = torch.empty(G, dtype=torch.float32, device=x.device)
    ws = _lib.workspace(lib.flw_quant_workspace_bytes(B, H, T, D), x.device)
    rc = lib.flw_amax_e4m3(x4.data_ptr(), _lib.dtype_code(x.dtype), B, H, T, D, sb, sh, st,
                           _lib.GRANULARITY[granularity], amax.data_ptr(), ws.data_ptr(), ws.numel(),
                           _lib.stream_of(x))
    _lib.check(rc, "amax_e4m3")
    return amax


def quantize_e4m3_with_amax(x: torch.Tensor, amax: torch.Tensor, granularity: str = "tensor"):
    """``_per_tensor_fp8`` with the amax given (a float32 device tensor of 1, H or B*H elements,
    e.g. ``amax_e4m3`` combined across shards): (x_e4m3, scale), the quantise pass only."""
    lib = _lib.load()
    _lib.require_gpu(x)
    x4, (sb, sh, st), G = _as_bhtd(x, granularity)
    if amax.dtype != torch.float32 or amax.numel() != G or amax.device != x.device:
        raise ValueError(f"amax must be a float32 tensor of {G} elements on {x.device}")
    amax = amax.contiguous()
    B, H, T, D = x4.shape
    out = torch.empty((B, H, T, D), dtype=torch.uint8, device=x.device)
    scale = torch.empty(G, dtype=torch.float32, device=x.device)
    rc = lib.flw_quant_e4m3_amax(x4.data_ptr(), _lib.dtype_code(x.dtype), B, H, T, D, sb, sh, st,
                                 _lib.GRANULARITY[granularity], _lib.LAYOUT_BHTD, amax.data_ptr(),
                                 out.data_ptr(), scale.data_ptr(), _lib.stream_of(x))
    _lib.check(rc, "quantize_e4m3_with_amax")
    return out.view(torch.float8_e4m3fn).reshape(x.shape), scale


def fp8_swa_attention_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    window: int,
    *,
    block_m: int = 64,
    block_n: int = 32,
    num_warps: int = 4,
    num_stages: int = 3,
    granularity: str = "tensor",
    out: torch.Tensor | None = None,
    amax: torch.Tensor | None = None,
) -> torch.Tensor:
    """FP8 sliding-window causal attention forward.

    q/k/v: (B, H, T, D) bf16 or fp32 on the GPU. Returns (B, H, T, D) in q's dtype. ``out`` (an
    extension; the reference has no such argument): a (B, H, T, D) tensor of q's dtype, any
    strides with D contiguous -- e.g. the (B, T, H, D) head view of a (B, T, H*D) buffer -- that
    the kernel writes in place and that is returned. ``amax`` (an extension): the |x| maxima of q,
    k, v per scale group [3 * groups] on the GPU, float32 (as ``amax_e4m3`` returns them) or
    their int32 bit patterns (as ``flw_fp8_scaled_mm_group_amax`` writes them for the QKV
    projection): the quantiser then skips its amax pass, and the result is the same as without
    it. A given amax below the data's own maximum still gives the reference's clamp-then-cast
    codes for that amax (values beyond it saturate at 448).
    ``window``: each query attends to the ``window`` keys at or behind it (window <= 0 gives
    an all-zero output, as the reference's masking does).

    Inference/forward only -- raises on tensors that require grad rather than silently
    detaching them. ``block_m``/``block_n``/``num_warps``/``num_stages`` are the reference's
    Triton tuning knobs; they are accepted for call compatibility and ignored.
    """
    del block_m, block_n, num_warps, num_stages
    try:
        lib = _lib.load()
    except RuntimeError as e:
        raise RuntimeError(f"fp8_swa_attention_forward requires the HIP library: {e}") from e
    if q.requires_grad or k.requires_grad or v.requires_grad:
        raise RuntimeError(
            "fp8_swa_attention_forward is forward-only and has no backward; "
            "calling it on tensors that require grad would silently detach them.")
    if q.dim() != 4:
        raise ValueError(f"expected (B, H, T, D), got {tuple(q.shape)}")
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v shapes differ: {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k, v must share a dtype")
    B, H, T, D = q.shape
    if D not in (32, 64, 128):
        raise ValueError(f"head_dim must be 32/64/128 for the MFMA tiling, got {D}")
    if granularity not in _lib.GRANULARITY:
        raise ValueError(f"granularity must be one of {sorted(_lib.GRANULARITY)}, got {granularity!r}")
    _lib.require_gpu(q, k, v)
    if q.numel() == 0:
        return torch.empty_like(q)
    dt = _lib.dtype_code(q.dtype)
    q, sq = _prepare(q)
    k, sk = _prepare(k)
    v, sv = _prepare(v)
    if out is None:
        out = torch.empty((B, H, T, D), device=q.device, dtype=q.dtype)
    elif (out.shape != (B, H, T, D) or out.dtype != q.dtype or out.device != q.device
          or out.stride(-1) != 1):
        raise ValueError("out must be a (B, H, T, D) tensor of q's dtype and device with D contiguous")
    so = out.stride()[:3]
    ws = _lib.workspace(lib.flw_fp8_swa_workspace_bytes(B, H, T, D), q.device)
    strides = _lib.i64s(*sq, *sk, *sv, *so)
    if amax is None:
        rc = lib.flw_fp8_swa_attention_forward(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), dt, strides, B, H, T, D, int(window),
            _lib.GRANULARITY[granularity], out.data_ptr(), None, ws.data_ptr(), ws.numel(),
            _lib.stream_of(q))
    else:
        groups = {"tensor": 1, "head": H, "bh": B * H}[granularity]
        if amax.dtype == torch.float32:
            amax = amax.view(torch.int32)
        if (amax.dtype != torch.int32 or amax.numel() != 3 * groups or amax.device != q.device
                or not amax.is_contiguous()):
            raise ValueError(f"amax must be a contiguous float32 tensor (or its int32 bit patterns) of "
                             f"{3 * groups} elements on q's device")
        rc = lib.flw_fp8_swa_attention_forward_amax(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), dt, strides, B, H, T, D, int(window),
            _lib.GRANULARITY[granularity], amax.data_ptr(), out.data_ptr(), None, ws.data_ptr(), ws.numel(),
            _lib.stream_of(q))
    _lib.check(rc, "fp8_swa_attention_forward")
    return out


def reference_swa_attention(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int
) -> torch.Tensor:
    """Dense fp32 reference for correctness testing. O(T^2) memory -- small shapes only.

    softmax(mask(Q K^T / sqrt(D))) V with valid(i, j) <=> j <= i and i - j < window
    (fp8_swa_attention.py:262-273); returns q's dtype.
    """
    B, H, T, D = q.shape
    qf, kf, vf = q.float(), k.float(), v.float()
    scores = (qf @ kf.transpose(-1, -2).contiguous()) / (D ** 0.5)
    idx = torch.arange(T, device=q.device)
    keep = (idx[:, None] >= idx[None, :]) & ((idx[:, None] - idx[None, :]) < window)
    scores = scores.masked_fill(~keep, float("-inf"))
    return (torch.softmax(scores, dim=-1) @ vf).to(q.dtype)


def qk_norm_rope_quant_e4m3(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, qk_norm: bool,
                            eps: float = 1e-6, rope_cos: torch.Tensor | None = None,
                            rope_sin: torch.Tensor | None = None, granularity: str = "head",
                            return_transformed: bool = False):
    """The FP8 attention's quantisation point of ``CausalSelfAttention.qkv_heads``
    (flower/models/base.py:618-639) in one HIP pass pair: HeadRMSNorm (``qk_norm``, base.py:341-357)
    and RoPE (``rope_cos`` / ``rope_sin``: [T, D] tables, base.py:436-483) applied to q and k, then
    the three ``_per_tensor_fp8`` quantisations (fp8_swa_attention.py:242-244) of q', k', v -- the
    transformed q', k' never round-trip through HBM.

    q / k / v: (B, H, T, D) bf16 or fp32 on the GPU, any strides with D contiguous (e.g. the head
    views of the qkv projection's output). Returns ``(q8, k8, v_tiles, scales)``: e4m3 codes of q'
    and k' (uint8 (B, H, T, D)), v's codes in the attention kernel's tile layout, and the float32
    scales [3 * groups] in the order q, k, v; with ``return_transformed`` also (q', k') in the
    input dtype (for checks; it costs their extra write).
    """
    lib = _lib.load()
    _lib.require_gpu(q, k, v)
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"expected three (B, H, T, D) tensors of one shape, got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k, v must share a dtype")
    if granularity not in _lib.GRANULARITY:
        raise ValueError(f"granularity must be one of {sorted(_lib.GRANULARITY)}, got {granularity!r}")
    B, H, T, D = q.shape
    if D not in (32, 64, 128):
        raise ValueError(f"head_dim must be 32/64/128 for the MFMA tiling, got {D}")
    if (rope_cos is None) != (rope_sin is None):
        raise ValueError("pass both RoPE tables or neither")
    if rope_cos is not None:
        if rope_cos.shape != (T, D) or rope_sin.shape != (T, D):
            raise ValueError(f"RoPE tables must be [T, D] = [{T}, {D}]")
        rope_cos = rope_cos.to(device=q.device, dtype=q.dtype).contiguous()
        rope_sin = rope_sin.to(device=q.device, dtype=q.dtype).contiguous()
    q, sq = _prepare(q)
    k, sk = _prepare(k)
    v, sv = _prepare(v)
    G = {"tensor": 1, "head": H, "bh": B * H}[granularity]
    dev = q.device
    q8 = torch.empty((B, H, T, D), dtype=torch.uint8, device=dev)
    k8 = torch.empty_like(q8)
    vt = torch.empty(lib.flw_vtile_bytes(B, H, T, D), dtype=torch.uint8, device=dev)
    scales = torch.empty(3 * G, dtype=torch.float32, device=dev)
    qt = kt = None
    if return_transformed:
        qt = torch.empty((B, H, T, D), dtype=q.dtype, device=dev)
        kt = torch.empty_like(qt)
    ws = _lib.workspace(3 * lib.flw_quant_workspace_bytes(B, H, T, D), dev)
    rc = lib.flw_qk_norm_rope_quant_e4m3(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.dtype_code(q.dtype), B, H, T, D,
        _lib.i64s(*sq, *sk, *sv), int(bool(qk_norm)), float(eps), _lib.ptr(rope_cos), _lib.ptr(rope_sin),
        _lib.GRANULARITY[granularity], q8.data_ptr(), k8.data_ptr(), vt.data_ptr(), scales.data_ptr(),
        _lib.ptr(qt), _lib.ptr(kt), ws.data_ptr(), ws.numel(), _lib.stream_of(q))
    _lib.check(rc, "qk_norm_rope_quant_e4m3")
    if return_transformed:
        return q8, k8, vt, scales, qt, kt
    return q8, k8, vt, scales


_CODE_DTYPES = (torch.uint8, torch.float8_e4m3fn)


def _group_count(granularity: str, B: int, H: int) -> int:
    if granularity not in _lib.GRANULARITY:
        raise ValueError(f"granularity must be one of {sorted(_lib.GRANULARITY)}, got {granularity!r}")
    return {"tensor": 1, "head": H, "bh": B * H}[granularity]


# Element strides (b, h) of each granularity's scale array: per tensor 0/0, per head 0/1, per (b, h) H/1.
_SCALE_STRIDES = {"tensor": lambda H: (0, 0), "head": lambda H: (0, 1), "bh": lambda H: (H, 1)}


def fp8_swa_attention_from_codes(q8: torch.Tensor, k8: torch.Tensor, v_tiles: torch.Tensor,
                                 scales: torch.Tensor, window: int, *, granularity: str = "head",
                                 out_dtype: torch.dtype = torch.bfloat16,
                                 out: torch.Tensor | None = None) -> torch.Tensor:
    """The attention kernel alone on pre-quantised operands (the ``_fp8_swa_fwd_kernel`` launch,
    fp8_swa_attention.py:249-258): q8 / k8 (B, H, T, D) e4m3 codes (uint8 or float8_e4m3fn, as
    ``_per_tensor_fp8`` returns them), V either in the kernel's tile layout (1-D, as
    ``qk_norm_rope_quant_e4m3`` returns it) or as (B, H, T, D) codes (read as they are by
    flw_fp8_swa_fwd_bhtd, the kernel instance that stages V into the tile layout itself), scales
    [3 * groups] (q, k, v) float32 on the device.
    ``out``: optional (B, H, T, D) destination of ``out_dtype`` with D contiguous.

    The kernel is given only B, H, T, D and strides, so every operand's shape, dtype and size is
    checked here against q8's before anything is launched (ValueError otherwise)."""
    lib = _lib.load()
    if q8.dim() != 4:
        raise ValueError(f"expected (B, H, T, D), got {tuple(q8.shape)}")
    B, H, T, D = q8.shape
    if D not in (32, 64, 128):
        raise ValueError(f"head_dim must be 32/64/128 for the MFMA tiling, got {D}")
    for name, t in (("q8", q8), ("k8", k8), ("v_tiles", v_tiles)):
        if t.dtype not in _CODE_DTYPES:
            raise ValueError(f"{name} must hold e4m3 codes (uint8 or float8_e4m3fn), got {t.dtype}")
    if k8.shape != q8.shape:
        raise ValueError(f"k8 {tuple(k8.shape)} does not match q8 {tuple(q8.shape)}")
    if q8.stride(-1) != 1 or k8.stride(-1) != 1:
        raise ValueError("q8 and k8 must be contiguous in their last dimension")
    if v_tiles.dim() == 4:
        if v_tiles.shape != q8.shape:
            raise ValueError(f"V codes {tuple(v_tiles.shape)} do not match Q's {tuple(q8.shape)}")
    elif v_tiles.dim() != 1 or v_tiles.numel() != lib.flw_vtile_bytes(B, H, T, D) or not v_tiles.is_contiguous():
        raise ValueError(f"v_tiles must be (B, H, T, D) codes or a contiguous 1-D tile buffer of "
                         f"flw_vtile_bytes(B, H, T, D) = {lib.flw_vtile_bytes(B, H, T, D)} bytes, "
                         f"got {tuple(v_tiles.shape)}")
    G = _group_count(granularity, B, H)
    if scales.numel() != 3 * G or scales.dtype != torch.float32 or not scales.is_contiguous():
        raise ValueError(f"scales must be a contiguous float32 tensor of {3 * G} elements")
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"out_dtype must be bfloat16 or float32, got {out_dtype}")
    if out is not None and (out.shape != (B, H, T, D) or out.stride(-1) != 1 or out.dtype != out_dtype):
        raise ValueError(f"out must be a (B, H, T, D) tensor of {out_dtype} with D contiguous")
    devices = {t.device for t in (q8, k8, v_tiles, scales) + ((out,) if out is not None else ())}
    if len(devices) != 1:
        raise ValueError(f"all operands must be on one device, got {sorted(map(str, devices))}")
    _lib.require_gpu(q8, k8, v_tiles, scales)
    q8, k8, v_tiles = (t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t for t in (q8, k8, v_tiles))
    if out is None:
        out = torch.empty((B, H, T, D), dtype=out_dtype, device=q8.device)
    s8 = _lib.i64s(*q8.stride()[:3])
    sk = _lib.i64s(*k8.stride()[:3])
    so = _lib.i64s(*out.stride()[:3])
    base = scales.data_ptr()
    if v_tiles.dim() == 4:
        v4 = v_tiles if v_tiles.stride(-1) == 1 and all(s % 16 == 0 for s in v_tiles.stride()[:3]) \
            else v_tiles.contiguous()
        ssb, ssh = _SCALE_STRIDES[granularity](H)
        rc = lib.flw_fp8_swa_fwd_bhtd(q8.data_ptr(), s8, k8.data_ptr(), sk, v4.data_ptr(), _lib.i64s(*v4.stride()[:3]),
                                      base, base + 4 * G, base + 8 * G, ssb, ssh, out.data_ptr(),
                                      _lib.dtype_code(out.dtype), so, B, H, T, D, int(window), _lib.stream_of(q8))
    else:
        rc = lib.flw_fp8_swa_fwd(q8.data_ptr(), s8, k8.data_ptr(), sk, v_tiles.data_ptr(), base, base + 4 * G,
                                 base + 8 * G, _lib.GRANULARITY[granularity], out.data_ptr(),
                                 _lib.dtype_code(out.dtype), so, B, H, T, D, int(window), _lib.stream_of(q8))
    _lib.check(rc, "fp8_swa_attention_from_codes")
    return out


def dequantize_e4m3(codes: torch.Tensor, scales: torch.Tensor, shape, granularity: str = "head",
                    layout: str = "bhtd", out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """(B, H, T, D) values e4m3(code) * scale of the code's group, rounded to ``out_dtype``
    (flw_dequant_e4m3): ``codes`` as ``_per_tensor_fp8`` returns them (layout "bhtd", contiguous) or
    in the attention kernel's V tile layout ("vtile", 1-D); ``scales`` one group's float32 scales."""
    lib = _lib.load()
    B, H, T, D = shape
    if codes.dtype == torch.float8_e4m3fn:
        codes = codes.view(torch.uint8)
    G = _group_count(granularity, B, H)
    if scales.numel() != G or scales.dtype != torch.float32 or not scales.is_contiguous():
        raise ValueError(f"scales must be a contiguous float32 tensor of {G} elements")
    want = lib.flw_vtile_bytes(B, H, T, D) if layout == "vtile" else B * H * T * D
    if codes.dtype != torch.uint8 or codes.numel() != want or not codes.is_contiguous():
        raise ValueError(f"codes must be {want} contiguous e4m3 codes ({layout})")
    _lib.require_gpu(codes, scales)
    out = torch.empty((B, H, T, D), dtype=out_dtype, device=codes.device)
    rc = lib.flw_dequant_e4m3(codes.data_ptr(), _lib.LAYOUT_VTILE if layout == "vtile" else _lib.LAYOUT_BHTD,
                              B, H, T, D, scales.data_ptr(), _lib.GRANULARITY[granularity], out.data_ptr(),
                              _lib.dtype_code(out_dtype), _lib.stream_of(codes))
    _lib.check(rc, "dequantize_e4m3")
    return out


class _Fp8SwaAttention(torch.autograd.Function):
    """FP8 forward (the e4m3 quantiser pass pair, then the FP8 kernel) with the bf16 sliding-window
    backward (flw_swa_bf16_bwd) at the dequantised Q, K, V: the straight-through estimator of
    `_fake_quant_e4m3` (base.py:167-203, the gradient passes the quantisers unchanged) around the
    attention's own backward, which rebuilds P from saved row statistics as swa_attention.py:307-359
    does. The statistics (O and the log-sum-exp) are recomputed in the backward by the bf16 forward
    (flw_swa_bf16_fwd) on the dequantised bf16 Q, K, V, so P is rebuilt from the same operands it
    was normalised with: the gradient is that of bf16 attention at the dequantised point, which is
    what the reference's fake-quant training path (`_fake_quant_e4m3`, then bf16 attention)
    differentiates. (Rebuilding P from the FP8 forward's own log-sum-exp, which comes from the exact
    fp32 scores of the codes, against the bf16-rounded dequantised operands misnormalises P by
    exp(score difference): measured 7 % mean-relative on dQ at the 450M shape.)"""

    @staticmethod
    def forward(ctx, q, k, v, window, granularity):
        lib = _lib.load()
        B, H, T, D = q.shape
        dt = _lib.dtype_code(q.dtype)
        q, sq = _prepare(q.detach())
        k, sk = _prepare(k.detach())
        v, sv = _prepare(v.detach())
        G = _group_count(granularity, B, H)
        dev = q.device
        q8 = torch.empty((B, H, T, D), dtype=torch.uint8, device=dev)
        k8 = torch.empty_like(q8)
        vt = torch.empty(lib.flw_vtile_bytes(B, H, T, D), dtype=torch.uint8, device=dev)
        scales = torch.empty(3 * G, dtype=torch.float32, device=dev)
        ws = _lib.workspace(3 * lib.flw_quant_workspace_bytes(B, H, T, D), dev)
        stream = _lib.stream_of(q)
        _lib.check(lib.flw_quant_qkv_e4m3(q.data_ptr(), k.data_ptr(), v.data_ptr(), dt, B, H, T, D,
                                          _lib.i64s(*sq, *sk, *sv), _lib.GRANULARITY[granularity], q8.data_ptr(),
                                          k8.data_ptr(), vt.data_ptr(), scales.data_ptr(), ws.data_ptr(),
                                          ws.numel(), stream), "fp8_swa_attention (quantise)")
        out = torch.empty((B, H, T, D), dtype=q.dtype, device=dev)
        s8 = _lib.i64s(H * T * D, T * D, D)
        base = scales.data_ptr()
        rc = lib.flw_fp8_swa_fwd(q8.data_ptr(), s8, k8.data_ptr(), s8, vt.data_ptr(), base, base + 4 * G,
                                 base + 8 * G, _lib.GRANULARITY[granularity], out.data_ptr(), dt,
                                 _lib.i64s(*out.stride()[:3]), B, H, T, D, int(window), stream)
        _lib.check(rc, "fp8_swa_attention (forward)")
        ctx.save_for_backward(q8, k8, vt, scales)
        ctx.window, ctx.granularity, ctx.G, ctx.dtype = int(window), granularity, G, q.dtype
        return out

    @staticmethod
    def backward(ctx, dout):
        lib = _lib.load()
        q8, k8, vt, scales = ctx.saved_tensors
        B, H, T, D = q8.shape
        G, gran = ctx.G, ctx.granularity
        qd = dequantize_e4m3(q8, scales[:G], (B, H, T, D), gran)
        kd = dequantize_e4m3(k8, scales[G:2 * G], (B, H, T, D), gran)
        vd = dequantize_e4m3(vt, scales[2 * G:], (B, H, T, D), gran, layout="vtile")
        stream = _lib.stream_of(qd)
        ob = torch.empty_like(qd)
        lse = torch.empty((B, H, T), dtype=torch.float32, device=qd.device)
        _lib.check(lib.flw_swa_bf16_fwd(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), B, H, T, D, ctx.window,
                                        ob.data_ptr(), lse.data_ptr(), stream), "fp8_swa_attention (recompute)")
        do = dout.to(torch.bfloat16).contiguous()
        dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
        ws = _lib.workspace(lib.flw_swa_bf16_bwd_workspace_bytes(B, H, T, D), q8.device)
        _lib.check(lib.flw_swa_bf16_bwd(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), ob.data_ptr(), do.data_ptr(),
                                        lse.data_ptr(), B, H, T, D, ctx.window, dq.data_ptr(), dk.data_ptr(),
                                        dv.data_ptr(), ws.data_ptr(), ws.numel(), stream),
                   "fp8_swa_attention (backward)")
        dt = ctx.dtype
        return dq.to(dt), dk.to(dt), dv.to(dt), None, None


def fp8_swa_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int, *,
                      granularity: str = "head") -> torch.Tensor:
    """Differentiable FP8 sliding-window causal attention (an extension of the reference's
    forward-only kernel, fp8_swa_attention.py:71-76): the forward is ``fp8_swa_attention_forward``'s
    (e4m3 Q / K / V with amax scales, e4m3 P, fp32 accumulation); the backward is the bf16
    sliding-window backward at the dequantised Q, K, V (straight-through quantisers, as
    `_fake_quant_e4m3` trains), from row statistics the bf16 forward recomputes there.
    q / k / v: (B, H, T, D) bf16 or fp32 on the GPU, D in {32, 64, 128}; window > 0 (the
    backward's requirement, swa_attention.py:378)."""
    try:
        _lib.load()
    except RuntimeError as e:
        raise RuntimeError(f"fp8_swa_attention requires the HIP library: {e}") from e
    if q.dim() != 4:
        raise ValueError(f"expected (B, H, T, D), got {tuple(q.shape)}")
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v shapes differ: {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("q, k, v must share a dtype, bfloat16 or float32")
    if q.shape[-1] not in (32, 64, 128):
        raise ValueError(f"head_dim must be 32/64/128 for the MFMA tiling, got {q.shape[-1]}")
    if window <= 0:
        raise ValueError("window must be positive; use flex for full-context attention")
    _group_count(granularity, q.shape[0], q.shape[1])
    _lib.require_gpu(q, k, v)
    return _Fp8SwaAttention.apply(q, k, v, int(window), granularity)
