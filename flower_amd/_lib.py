"""ctypes binding of libflower_amd.so (the C ABI declared in include/flower_amd.h).

The shared object is built in-tree by ``flower_amd._build``. There is no fallback: if the
library is missing or the device is not a GPU, every operator raises RuntimeError.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int64, c_size_t, c_void_p

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libflower_amd.so")

F32, BF16 = 0, 1
SCALE_TENSOR, SCALE_HEAD, SCALE_BH, SCALE_COLUMN = 0, 1, 2, 3
LAYOUT_BHTD, LAYOUT_VTILE, LAYOUT_BTHD = 0, 1, 2
GEMM_A8W8, GEMM_W8A16 = 0, 1

GRANULARITY = {"tensor": SCALE_TENSOR, "head": SCALE_HEAD, "bh": SCALE_BH}

_P64 = POINTER(c_int64)

# name -> (restype, argtypes); must match include/flower_amd.h
SIGNATURES = {
    "flw_last_error": (c_char_p, []),
    "flw_abi_version": (c_int, []),
    "flw_time_next_launch": (c_int, [c_void_p, c_void_p]),
    "flw_quant_workspace_bytes": (c_size_t, [c_int64] * 4),
    "flw_vtile_bytes": (c_size_t, [c_int64] * 4),
    "flw_vtile_from_bhtd": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64,
                                    c_void_p, c_void_p]),
    "flw_quant_e4m3": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64,
                               c_int64, c_int, c_int, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "flw_amax_e4m3": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64,
                              c_int64, c_int, c_void_p, c_void_p, c_size_t, c_void_p]),
    "flw_quant_e4m3_amax": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64,
                                    c_int64, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p]),
    "flw_quant_qkv_e4m3": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_int64,
                                   c_int64, _P64, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                   c_void_p, c_size_t, c_void_p]),
    "flw_qk_norm_rope_quant_e4m3": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_int64,
                                            c_int64, _P64, c_int, c_float, c_void_p, c_void_p, c_int, c_void_p,
                                            c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                            c_void_p]),
    "flw_noalloc_scratch_bytes": (c_size_t, []),
    "flw_quant_qkv_e4m3_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_int64,
                                           c_int64, _P64, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                           c_void_p]),
    "flw_fake_quant_e4m3": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_int64, c_int64,
                                    c_int64, c_int64, c_int, c_void_p, c_void_p, c_void_p, c_size_t,
                                    c_void_p]),
    "flw_quant_rows_e4m3": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_void_p, c_void_p,
                                    c_void_p]),
    "flw_quant_cols_workspace_bytes": (c_size_t, [c_int64, c_int64]),
    "flw_quant_cols_e4m3": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_int, c_void_p, c_int64,
                                    c_void_p, c_void_p, c_size_t, c_void_p]),
    "flw_transpose_e4m3": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p]),
    "flw_qkv_heads_fwd": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_int, c_float, c_void_p,
                                  c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "flw_qkv_heads_bwd": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_int, c_float, c_void_p,
                                  c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p,
                                  c_size_t, c_void_p]),
    "flw_qkv_heads_amax_workspace_bytes": (c_size_t, [c_int64] * 4),
    "flw_quant_tensor_t_workspace_bytes": (c_size_t, [c_int64, c_int64]),
    "flw_quant_tensor_t_e4m3": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                        c_void_p, c_void_p, c_size_t, c_void_p]),
    "flw_quant_tensor_t_e4m3_amax": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_int64,
                                             c_void_p, c_int64, c_void_p, c_void_p]),
    "flw_rmsnorm_fwd": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_float, c_void_p, c_int64,
                                c_void_p]),
    "flw_rmsnorm_bwd_workspace_bytes": (c_size_t, [c_int64, c_int64]),
    "flw_add_rmsnorm_fwd": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p, c_float,
                                    c_void_p, c_int64, c_void_p, c_int64, c_void_p]),
    "flw_rmsnorm_bwd": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_float, c_void_p, c_int64,
                                c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_size_t, c_void_p]),
    "flw_swiglu_amax_workspace_bytes": (c_size_t, [c_int64, c_int64]),
    "flw_swiglu_fwd": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p, c_int64,
                               c_void_p, c_void_p, c_size_t, c_void_p]),
    "flw_swiglu_bwd": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p, c_int64,
                               c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_size_t, c_void_p]),
    "flw_rmsnorm_quant_rows_e4m3": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_float, c_void_p,
                                            c_void_p, c_void_p, c_void_p]),
    "flw_gelu_quant_rows_e4m3": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p,
                                         c_void_p]),
    "flw_fp8_swa_fwd": (c_int, [c_void_p, _P64, c_void_p, _P64, c_void_p, c_void_p, c_void_p, c_void_p,
                                c_int, c_void_p, c_int, _P64, c_int64, c_int64, c_int64, c_int64,
                                c_int64, c_void_p]),
    "flw_fp8_swa_fwd_scale_strides": (c_int, [c_void_p, _P64, c_void_p, _P64, c_void_p, c_void_p, c_void_p,
                                              c_void_p, c_int64, c_int64, c_void_p, c_int, _P64, c_int64,
                                              c_int64, c_int64, c_int64, c_int64, c_void_p]),
    "flw_fp8_swa_fwd_bhtd": (c_int, [c_void_p, _P64, c_void_p, _P64, c_void_p, _P64, c_void_p, c_void_p,
                                     c_void_p, c_int64, c_int64, c_void_p, c_int, _P64, c_int64, c_int64,
                                     c_int64, c_int64, c_int64, c_void_p]),
    "flw_fp8_swa_fwd_qx": (c_int, [c_void_p, _P64, c_void_p, c_void_p, c_void_p, _P64, c_void_p, c_void_p,
                                   c_void_p, c_void_p, c_int, c_void_p, c_int, _P64, c_int64, c_int64, c_int64,
                                   c_int64, c_int64, c_void_p]),
    "flw_fp8_swa_fwd_lse": (c_int, [c_void_p, _P64, c_void_p, _P64, c_void_p, c_void_p, c_void_p, c_void_p,
                                    c_int, c_void_p, c_int, _P64, c_int64, c_int64, c_int64, c_int64,
                                    c_int64, c_void_p, c_void_p]),
    "flw_dequant_e4m3": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_int64, c_void_p, c_int, c_void_p,
                                 c_int, c_void_p]),
    "flw_quant_qkv_e4m3_deferq": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_int64,
                                          c_int64, _P64, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                          c_void_p, c_size_t, c_void_p]),
    "flw_fp8_swa_workspace_bytes": (c_size_t, [c_int64] * 4),
    "flw_fp8_swa_attention_forward_amax": (c_int, [c_void_p, c_void_p, c_void_p, c_int, _P64, c_int64, c_int64,
                                                   c_int64, c_int64, c_int64, c_int, c_void_p, c_void_p, c_void_p,
                                                   c_void_p, c_size_t, c_void_p]),
    "flw_fp8_swa_attention_forward": (c_int, [c_void_p, c_void_p, c_void_p, c_int, _P64, c_int64,
                                              c_int64, c_int64, c_int64, c_int64, c_int, c_void_p,
                                              c_void_p, c_void_p, c_size_t, c_void_p]),
    "flw_swa_bf16_fwd": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64,
                                 c_void_p, c_void_p, c_void_p]),
    "flw_swa_bf16_fwd_layout": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64,
                                        c_int64, c_void_p, c_int, c_void_p, c_void_p]),
    "flw_swa_bf16_bwd_layout": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int64,
                                        c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p,
                                        c_size_t, c_void_p]),
    "flw_swa_bf16_bwd_workspace_bytes": (c_size_t, [c_int64] * 4),
    "flw_swa_bf16_bwd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64,
                                 c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                 c_void_p]),
    "flw_fp8_linear_workspace_bytes": (c_size_t, [c_int64, c_int64, c_int]),
    "flw_fp8_linear": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p,
                               c_int64, c_int, c_void_p, c_int64, c_void_p, c_size_t, c_void_p]),
    "flw_fp8_scaled_mm_group_amax": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                             c_void_p, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "flw_fp8_scaled_mm_qk_norm_rope_amax": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p,
                                                    c_int64, c_void_p, c_int64, c_void_p, c_int64, c_int64,
                                                    c_int64, c_int, c_float, c_void_p, c_void_p, c_int64,
                                                    c_void_p, c_void_p]),
    "flw_fp8_scaled_mm_workspace_bytes": (c_size_t, [c_int64, c_int64, c_int64]),
    "flw_fp8_scaled_mm_ws": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                     c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_size_t, c_void_p]),
    "flw_fp8_scaled_mm": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                  c_void_p, c_int64, c_void_p, c_int64, c_void_p]),
    "flw_fp8_scaled_mm_residual": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                           c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p]),
}

# The diagnostics library (flower_amd/csrc/diag/flw_diag.h): instruments for tests and bench.py.
DIAG_LIB_PATH = os.path.join(_HERE, "libflower_amd_diag.so")
DIAG_SIGNATURES = {
    "flw_last_error": (c_char_p, []),
    "flw_abi_version": (c_int, []),
    "flw_time_next_launch": (c_int, [c_void_p, c_void_p]),
    "flw_diag_cvt_e4m3": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_void_p]),
    "flw_diag_quotient": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int, c_void_p]),
    "flw_diag_issue_probe": (c_int, [c_int, c_void_p, c_int64, c_int, c_void_p]),
    "flw_diag_issue_probe_iters": (c_int, []),
    "flw_diag_mfma_e4m3_dot": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_void_p]),
}

_lib = None
_diag = None


def load() -> ctypes.CDLL:
    """Load (once) and type the shared library. Raises RuntimeError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"libflower_amd.so is not built ({LIB_PATH}); run `python -m flower_amd._build`")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.flw_abi_version() != 1:
        raise RuntimeError("libflower_amd ABI version mismatch")
    _lib = lib
    return lib


def load_diag() -> ctypes.CDLL:
    """Load (once) the diagnostics library. Raises RuntimeError if it is not built."""
    global _diag
    if _diag is not None:
        return _diag
    if not os.path.exists(DIAG_LIB_PATH):
        raise RuntimeError(
            f"libflower_amd_diag.so is not built ({DIAG_LIB_PATH}); run `python -m flower_amd._build`")
    lib = ctypes.CDLL(DIAG_LIB_PATH)
    for name, (res, args) in DIAG_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _diag = lib
    return lib


class FlowerError(RuntimeError):
    pass


def check(rc: int, what: str, lib: ctypes.CDLL | None = None) -> None:
    """Raise for a non-zero status; ``lib`` is the library that returned it (default: the product)."""
    if rc != 0:
        msg = (lib or load()).flw_last_error().decode(errors="replace")
        if rc in (1, 2):          # FLW_E_INVALID / FLW_E_UNSUPPORTED: caller error
            raise ValueError(f"{what}: {msg}")
        raise FlowerError(f"{what} failed ({rc}): {msg}")


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(
                "flower_amd operators run only on a ROCm GPU (gfx950); got a tensor on "
                f"{t.device}. There is no CPU fallback.")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    raise ValueError(f"unsupported dtype {dt} (float32 or bfloat16)")


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def i64s(*vals: int):
    return (c_int64 * len(vals))(*vals)


def workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


__all__ = ["load", "load_diag", "check", "require_gpu", "dtype_code", "stream_of", "ptr", "i64s", "workspace",
           "GRANULARITY", "SIGNATURES", "LIB_PATH", "DIAG_SIGNATURES", "DIAG_LIB_PATH"]
