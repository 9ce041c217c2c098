"""CPU: the C-ABI library loads and exports exactly what include/flower_amd.h declares; the
diagnostics library (flower_amd/csrc/diag/flw_diag.h) is separate and exports what it declares."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flower_amd.h")
DIAG_HEADER = os.path.join(ROOT, "flower_amd", "csrc", "diag", "flw_diag.h")


def _gpu_visible() -> bool:
    import torch
    return torch.cuda.is_available()


# The host-validation tests below hand the library made-up device addresses and rely on its
# argument checks refusing the call before any launch; they run only where no GPU is visible, so
# that a regression in those checks can never put a kernel on a fake address.
fake_pointers = pytest.mark.skipif(_gpu_visible(), reason="passes fake device pointers: CPU-only host check")


def declared_functions(header=HEADER):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(flw_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_path_entry_points():
    names = declared_functions()
    for must in ("flw_quant_e4m3", "flw_fake_quant_e4m3", "flw_quant_rows_e4m3", "flw_fp8_swa_fwd",
                 "flw_fp8_swa_attention_forward", "flw_fp8_linear", "flw_fp8_scaled_mm",
                 "flw_last_error", "flw_abi_version"):
        assert must in names


def test_library_loads_and_exports_every_declared_symbol():
    from flower_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libflower_amd.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in include/flower_amd.h but not exported"
    # the Python binding types exactly the declared set
    assert set(_lib.SIGNATURES) == set(declared_functions())
    # measurement instruments are not part of the product library
    assert not any(n.startswith("flw_diag") for n in declared_functions())
    for name in ("flw_diag_issue_probe", "flw_diag_cvt_e4m3", "flw_diag_quotient", "flw_diag_mfma_e4m3_dot"):
        assert not hasattr(lib, name), f"{name} leaked into the product library"


def test_diagnostics_library_exports_what_its_header_declares():
    from flower_amd import _lib
    if not os.path.exists(_lib.DIAG_LIB_PATH):
        pytest.skip("libflower_amd_diag.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_lib.DIAG_LIB_PATH)
    names = declared_functions(DIAG_HEADER)
    assert "flw_diag_issue_probe" in names
    for name in names:
        assert hasattr(lib, name), f"{name} declared in flw_diag.h but not exported"
    assert set(_lib.DIAG_SIGNATURES) == set(names)


@fake_pointers
def test_host_only_calls_work_without_a_gpu():
    from flower_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libflower_amd.so not built")
    lib = _lib.load()
    assert lib.flw_abi_version() == 1
    assert lib.flw_vtile_bytes(2, 3, 100, 64) == 2 * 3 * 128 * 64
    assert lib.flw_quant_workspace_bytes(1, 1, 1000, 64) == 8 * 4          # 8 chunks of 128 rows
    assert lib.flw_fp8_swa_workspace_bytes(4, 16, 8192, 64) >= 3 * 4 * 16 * 8192 * 64
    # argument validation happens on the host, before any device work
    rc = lib.flw_fp8_swa_fwd(None, None, None, None, None, None, None, None, 0, None, 0, None,
                             1, 1, 64, 64, 16, None)
    assert rc == 1 and b"null" in lib.flw_last_error()
    s = _lib.i64s(0, 0, 0)
    rc = lib.flw_fp8_swa_fwd(16, s, 16, s, 16, 16, 16, 16, 0, 16, 1, s, 1, 1, 64, 96, 16, None)
    assert rc == 2 and b"head_dim" in lib.flw_last_error()
    # V as (B, H, T, D) codes: strides checked before launch (multiples of 16 bytes)
    s16, s8 = _lib.i64s(64 * 64, 64 * 64, 64), _lib.i64s(64 * 64, 64 * 64, 72)
    rc = lib.flw_fp8_swa_fwd_bhtd(16, s16, 16, s16, 16, None, 16, 16, 16, 0, 1, 16, 1, s16, 1, 1, 64, 64, 16, None)
    assert rc == 1 and b"null v8 strides" in lib.flw_last_error()
    rc = lib.flw_fp8_swa_fwd_bhtd(16, s16, 16, s16, 16, s8, 16, 16, 16, 0, 1, 16, 1, s16, 1, 1, 64, 64, 16, None)
    assert rc == 1 and b"v8 strides" in lib.flw_last_error()
    rc = lib.flw_fp8_linear(16, 8, 64, 64, 16, 16, 16, 16, 7, 16, 16, 16, 1 << 20, None)
    assert rc == 1 and b"unknown GEMM mode" in lib.flw_last_error()
    rc = lib.flw_fp8_linear(16, 8, 80, 80, 16, 16, 16, 16, 1, 16, 16, None, 0, None)   # W8A16
    assert rc == 2 and b"multiple of 64" in lib.flw_last_error()
    assert lib.flw_fp8_scaled_mm_workspace_bytes(8192, 4096, 1024) == 0    # 512 tiles: no split
    assert lib.flw_fp8_scaled_mm_workspace_bytes(256, 256, 100) == 0       # K % 128: no split
    assert lib.flw_quant_cols_workspace_bytes(1000, 100) == 4 * 100 * 4   # 4 row chunks x 100 columns
    assert lib.flw_quant_cols_workspace_bytes(1000, 8) == 4 * 8 * 4
    rc = lib.flw_quant_cols_e4m3(16, 1, 100, 64, 64, _lib.SCALE_HEAD, 16, 112, 16, 16, 1 << 20, None)
    assert rc == 1 and b"granularity" in lib.flw_last_error()
    rc = lib.flw_quant_cols_e4m3(16, 1, 100, 64, 64, _lib.SCALE_COLUMN, 16, 96, 16, 16, 1 << 20, None)
    assert rc == 1 and b"ld must be" in lib.flw_last_error()
    rc = lib.flw_quant_cols_e4m3(16, 1, 100, 64, 64, _lib.SCALE_COLUMN, 16, 112, 16, 16, 4, None)
    assert rc != 0 and b"workspace" in lib.flw_last_error()


def test_operators_refuse_cpu_tensors():
    """No silent CPU fallback: the product path raises on host tensors."""
    import torch
    from flower_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libflower_amd.so not built")
    from flower_amd.kernels.fp8_swa_attention import _per_tensor_fp8, fp8_swa_attention_forward
    from flower_amd.attention import _fake_quant_e4m3
    x = torch.randn(1, 2, 64, 64)
    with pytest.raises(RuntimeError, match="GPU"):
        fp8_swa_attention_forward(x, x, x, 16)
    with pytest.raises(RuntimeError, match="GPU"):
        _per_tensor_fp8(x)
    with pytest.raises(RuntimeError, match="GPU"):
        _fake_quant_e4m3(x)


@fake_pointers
def test_limits_and_empty_shapes_are_refused_on_the_host():
    """Maximum sizes and empty inputs are turned into errors before any device work (fake,
    16-byte aligned pointers; nothing is dereferenced)."""
    from flower_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libflower_amd.so not built")
    lib = _lib.load()
    P = 1 << 20                                  # a fake aligned "device" address
    s64 = _lib.i64s(64 * 64, 64, 64)
    so = _lib.i64s(64 * 64, 64, 64)
    # one (b, h) slice of k8 must span < 2^31 bytes: T = 2^25 rows of D = 64 -> 2^31
    rc = lib.flw_fp8_swa_fwd(P, _lib.i64s(0, 0, 64), P, _lib.i64s(0, 0, 64), P, P, P, P, 0, P, 1,
                             _lib.i64s(0, 0, 64), 1, 1, 1 << 25, 64, 16, None)
    assert rc == 2 and b"2^31" in lib.flw_last_error()
    rc = lib.flw_fp8_swa_fwd(P, s64, P, s64, P, P, P, P, 0, P, 1, so, 1, 1, 0, 64, 16, None)
    assert rc == 1 and b"empty" in lib.flw_last_error()
    rc = lib.flw_swa_bf16_fwd(P, P, P, 1, 1, 128, 96, 16, P, P, None)
    assert rc == 2 and b"head_dim" in lib.flw_last_error()
    rc = lib.flw_swa_bf16_fwd(P, P, P, 1, 1, 128, 64, 0, P, P, None)
    assert rc == 1 and b"window" in lib.flw_last_error()
    rc = lib.flw_fp8_scaled_mm(P, 64, 40, P, 64, P, 64, P, 64, P, 64, None)
    assert rc == 2 and b"multiple of 16" in lib.flw_last_error()
    rc = lib.flw_fp8_scaled_mm(P, 0, 64, P, 64, P, 64, P, 64, P, 64, None)
    assert rc == 1 and b"empty" in lib.flw_last_error()
    rc = lib.flw_quant_rows_e4m3(P, _lib.BF16, 16, 12, 12, P, P, None)
    assert rc == 1 and b"multiples of 8" in lib.flw_last_error()
    rc = lib.flw_quant_cols_e4m3(P, _lib.BF16, 0, 64, 64, _lib.SCALE_COLUMN, P, 16, P, P, 1 << 20, None)
    assert rc == 1 and b"empty" in lib.flw_last_error()
    rc = lib.flw_quant_e4m3_amax(P, _lib.BF16, 1, 2, 64, 64, 8192, 4096, 64, _lib.SCALE_HEAD,
                                 _lib.LAYOUT_BHTD, None, P, P, None)
    assert rc == 1 and b"null amax" in lib.flw_last_error()
    rc = lib.flw_amax_e4m3(P, _lib.BF16, 1, 2, 64, 64, 8192, 4096, 64, _lib.SCALE_HEAD, P, P, 4, None)
    assert rc == 3 and b"workspace" in lib.flw_last_error()
    rc = lib.flw_amax_e4m3(P, _lib.BF16, 1, 2, 64, 64, 8192, 4096, 64, 7, P, P, 1 << 20, None)
    assert rc == 1 and b"granularity" in lib.flw_last_error()
    # the QKV GEMM's group amax exists only in the 256 x 256 kernel: operands past 2^32 bytes
    # (M * K = 2^32 here) are refused instead of returning an unwritten amax
    rc = lib.flw_fp8_scaled_mm_group_amax(P, 1 << 22, 1024, P, 256, P, 1 << 22, P, 256, P, 256, 64, P, None)
    assert rc == 2 and b"group amax" in lib.flw_last_error()


@fake_pointers
def test_issue_probe_refuses_bad_arguments_on_the_host():
    from flower_amd import _lib
    if not os.path.exists(_lib.DIAG_LIB_PATH):
        pytest.skip("libflower_amd_diag.so not built")
    lib = _lib.load_diag()
    assert lib.flw_diag_issue_probe_iters() > 0
    fake = 1 << 20
    assert lib.flw_diag_issue_probe(1, None, 256, 1, None) == 1           # null out
    assert lib.flw_diag_issue_probe(1, fake, 255, 1, None) == 1           # out too small
    assert lib.flw_diag_issue_probe(1, fake, 256, 0, None) == 1           # no workgroups
    assert lib.flw_diag_issue_probe(5, fake, 256, 1, None) == 1           # no such probe
    assert b"no issue probe" in lib.flw_last_error()


@fake_pointers
def test_mfma_dot_probe_refuses_bad_arguments_on_the_host():
    from flower_amd import _lib
    if not os.path.exists(_lib.DIAG_LIB_PATH):
        pytest.skip("libflower_amd_diag.so not built")
    lib = _lib.load_diag()
    f = 1 << 20
    assert lib.flw_diag_mfma_e4m3_dot(None, f, None, None, f, 1, 0, None) == 1        # null A
    assert b"null operand" in lib.flw_last_error()
    assert lib.flw_diag_mfma_e4m3_dot(f, f, None, f, f, 1, 1, None) == 1            # chain without A2
    assert lib.flw_diag_mfma_e4m3_dot(f, f, None, None, f, 0, 0, None) == 1         # no problems
    assert lib.flw_diag_mfma_e4m3_dot(f, f, None, None, f, 1 << 31, 0, None) == 1   # too many
    assert b"nprobe" in lib.flw_last_error()
    assert lib.flw_diag_mfma_e4m3_dot(f + 8, f, None, None, f, 1, 0, None) == 1     # misaligned A
    assert b"aligned" in lib.flw_last_error()


@fake_pointers
def test_scale_strides_are_validated_on_the_host():
    from flower_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libflower_amd.so not built")
    lib = _lib.load()
    P = 1 << 20                                  # a fake aligned "device" address
    s64 = _lib.i64s(64 * 64, 64, 64)
    rc = lib.flw_fp8_swa_fwd_scale_strides(P, s64, P, s64, P, P, P, P, -1, 1, P, 1, s64, 1, 1, 64, 64, 16, None)
    assert rc == 1 and b"scale strides" in lib.flw_last_error()
    rc = lib.flw_fp8_swa_fwd(P, s64, P, s64, P, P, P, P, 7, P, 1, s64, 1, 1, 64, 64, 16, None)
    assert rc == 1 and b"granularity" in lib.flw_last_error()


@fake_pointers
def test_noalloc_quantiser_refuses_shapes_beyond_its_scratch():
    """3 tensors x B*H*ceil(T/128) partials x 4 bytes: B1 H64 T1,048,576 needs 6 MiB against the
    1 MiB scratch array, refused on the host before the scratch address is even looked up."""
    from flower_amd import _lib as L
    if not os.path.exists(L.LIB_PATH):
        pytest.skip("libflower_amd.so not built")
    lib = L.load()
    assert lib.flw_noalloc_scratch_bytes() == 1 << 20
    P = 1 << 20
    strides = L.i64s(*([64 * 1048576 * 64, 1048576 * 64, 64] * 3))
    rc = lib.flw_quant_qkv_e4m3_noalloc(P, P, P, L.BF16, 1, 64, 1048576, 64, strides, L.SCALE_HEAD,
                                        P, P, P, P, None)
    assert rc == 2 and b"scratch" in lib.flw_last_error()
    rc = lib.flw_quant_qkv_e4m3_noalloc(P, P, P, L.BF16, 0, 64, 128, 64, strides, L.SCALE_HEAD, P, P, P, P, None)
    assert rc == 1 and b"empty" in lib.flw_last_error()


@fake_pointers
def test_qkv_epilogue_transform_refusals_on_the_host():
    """flw_fp8_scaled_mm_qk_norm_rope_amax checks its transform arguments before any launch."""
    from flower_amd import _lib as L
    if not os.path.exists(L.LIB_PATH):
        pytest.skip("libflower_amd.so not built")
    lib = L.load()
    P = 1 << 20

    def call(M, N, D, qk, T, cos, sin):
        return lib.flw_fp8_scaled_mm_qk_norm_rope_amax(P, M, 128, P, N, P, M, P, N, P, N, D, qk, 1, 1e-6, cos, sin,
                                                       T, P, None)
    assert call(128, 96, 48, 64, 128, None, None) == 2 and b"head_dim" in lib.flw_last_error()
    assert call(128, 192, 64, 96, 128, None, None) == 1 and b"qk_cols" in lib.flw_last_error()
    assert call(128, 192, 64, 128, 100, None, None) == 1 and b"seq_len" in lib.flw_last_error()
    assert call(128, 192, 64, 128, 128, P, None) == 1 and b"both RoPE" in lib.flw_last_error()
    rc = lib.flw_fp8_scaled_mm_qk_norm_rope_amax(P, 128, 128, P, 192, P, 128, P, 192, P, 192, 64, 128, 1, 1e-6,
                                                 None, None, 128, None, None)
    assert rc == 1 and b"null amax" in lib.flw_last_error()


@fake_pointers
def test_lse_forward_and_dequantiser_refusals_on_the_host():
    from flower_amd import _lib as L
    if not os.path.exists(L.LIB_PATH):
        pytest.skip("libflower_amd.so not built")
    lib = L.load()
    P = 1 << 20
    s64 = L.i64s(64 * 64, 64, 64)
    rc = lib.flw_fp8_swa_fwd_lse(P, s64, P, s64, P, P, P, P, L.SCALE_HEAD, P, L.BF16, s64, 1, 1, 64, 64, 16, None, None)
    assert rc == 1 and b"null lse" in lib.flw_last_error()
    rc = lib.flw_fp8_swa_fwd_lse(P, s64, P, s64, P, P, P, P, L.SCALE_HEAD, P, L.BF16, s64, 1, 1, 64, 64, 16, P + 2,
                                 None)
    assert rc == 1 and b"lse" in lib.flw_last_error()
    rc = lib.flw_dequant_e4m3(P, L.LAYOUT_BHTD, 1, 1, 64, 48, P, L.SCALE_HEAD, P, L.BF16, None)
    assert rc == 2 and b"head_dim" in lib.flw_last_error()
    rc = lib.flw_dequant_e4m3(P, 5, 1, 1, 64, 64, P, L.SCALE_HEAD, P, L.BF16, None)
    assert rc == 1 and b"layout" in lib.flw_last_error()
    rc = lib.flw_dequant_e4m3(P, L.LAYOUT_BHTD, 1, 1, 64, 64, P, 9, P, L.BF16, None)
    assert rc == 1 and b"granularity" in lib.flw_last_error()
    rc = lib.flw_dequant_e4m3(P, L.LAYOUT_BHTD, 1, 1, 0, 64, P, L.SCALE_HEAD, P, L.BF16, None)
    assert rc == 1 and b"empty" in lib.flw_last_error()
    rc = lib.flw_dequant_e4m3(P, L.LAYOUT_BHTD, 1, 1, 64, 64, P, L.SCALE_HEAD, P + 8, L.BF16, None)
    assert rc == 1 and b"aligned" in lib.flw_last_error()


@fake_pointers
def test_training_row_kernel_refusals_on_the_host():
    """qkv_heads, RMSNorm and SwiGLU training passes: unsupported widths, misaligned or short rows
    and an undersized workspace are refused before any launch (fake aligned pointers)."""
    from flower_amd import _lib as L
    if not os.path.exists(L.LIB_PATH):
        pytest.skip("libflower_amd.so not built")
    lib = L.load()
    P = 1 << 20
    rc = lib.flw_qkv_heads_fwd(P, 1, 16, 2, 48, 288, 1, 1e-6, P, P, P, P, P, None)
    assert rc == 2 and b"head_dim" in lib.flw_last_error()
    rc = lib.flw_qkv_heads_fwd(P, 1, 16, 2, 64, 320, 1, 1e-6, P, P, P, P, P, None)
    assert rc == 1 and b"3 H D" in lib.flw_last_error()
    rc = lib.flw_qkv_heads_bwd(P, 1, 16, 2, 64, 384, 1, 1e-6, P, P, P, P, P, P + 8, 384, None, None, 0, None)
    assert rc == 1 and b"aligned" in lib.flw_last_error()
    need = lib.flw_qkv_heads_amax_workspace_bytes(1, 16, 2, 64)           # one u32 per workgroup
    assert need == 4 * ((16 * 3 * 2 * 8 + 255) // 256)
    rc = lib.flw_qkv_heads_bwd(P, 1, 16, 2, 64, 384, 1, 1e-6, P, P, P, P, P, P, 384, P, P, need - 4, None)
    assert rc == 3 and b"workspace" in lib.flw_last_error()
    rc = lib.flw_rmsnorm_fwd(P, 4, 12, 16, P, 1e-6, P, 16, None)
    assert rc == 1 and b"multiple of 8" in lib.flw_last_error()
    rc = lib.flw_rmsnorm_fwd(P, 4, 8200, 8200, P, 1e-6, P, 8200, None)
    assert rc == 2 and b"8192" in lib.flw_last_error()
    rc = lib.flw_rmsnorm_fwd(P, 4, 64, 32, P, 1e-6, P, 64, None)
    assert rc == 1 and b"stride" in lib.flw_last_error()
    rc = lib.flw_rmsnorm_fwd(P, 4, 64, 64, P, -1.0, P, 64, None)
    assert rc == 1 and b"eps" in lib.flw_last_error()
    need = lib.flw_rmsnorm_bwd_workspace_bytes(1021, 1280)            # a workgroup per 4 rows
    assert need == 256 * 1280 * 4 and lib.flw_rmsnorm_bwd_workspace_bytes(0, 1280) == 0
    assert lib.flw_rmsnorm_bwd_workspace_bytes(1 << 20, 1280) == 768 * 1280 * 4   # at most 768
    rc = lib.flw_rmsnorm_bwd(P, 1021, 1280, 1280, P, 1e-6, P, 1280, None, 0, P, 1280, P, P, need - 16, None)
    assert rc == 1 and b"workspace" in lib.flw_last_error()
    rc = lib.flw_rmsnorm_bwd(P, 1021, 1280, 1280, P, 1e-6, P, 1280, P + 8, 1280, P, 1280, P, P, need, None)
    assert rc == 1 and b"dres" in lib.flw_last_error()
    rc = lib.flw_add_rmsnorm_fwd(P, None, 4, 64, 64, 64, P, 1e-6, P, 64, P, 64, None)
    assert rc == 1 and b"null" in lib.flw_last_error()
    rc = lib.flw_add_rmsnorm_fwd(P, P, 4, 64, 64, 32, P, 1e-6, P, 64, P, 64, None)
    assert rc == 1 and b"strides" in lib.flw_last_error()
    rc = lib.flw_swa_bf16_fwd_layout(P, P, P, 1, 4, 128, 64, 32, P, 7, P, None)
    assert rc == 1 and b"layout" in lib.flw_last_error()
    rc = lib.flw_swa_bf16_fwd_layout(P, P, P, 1, 64, 1 << 18, 64, 32, P, L.LAYOUT_BTHD, P, None)
    assert rc == 2 and b"2^31" in lib.flw_last_error()
    rc = lib.flw_swa_bf16_bwd_layout(P, P, P, P, P, L.LAYOUT_VTILE, P, 1, 4, 128, 64, 32, P, P, P, P, 1 << 20, None)
    assert rc == 1 and b"layout" in lib.flw_last_error()
    rc = lib.flw_swiglu_fwd(P, P, 4, 20, 24, 24, P, 24, None, None, 0, None)
    assert rc == 1 and b"multiple of 8" in lib.flw_last_error()
    rc = lib.flw_swiglu_bwd(P, P, 4, 64, 64, 64, P, 64, P, P + 4, 64, None, None, 0, None)
    assert rc == 1 and b"aligned" in lib.flw_last_error()
    rc = lib.flw_swiglu_fwd(P, P, 1 << 28, 128, 128, 128, P, 128, None, None, 0, None)
    assert rc == 2 and b"too many" in lib.flw_last_error()
    need = lib.flw_swiglu_amax_workspace_bytes(16384, 3392)                 # 2 x 8192 workgroups
    assert need == 2 * 8192 * 4 and lib.flw_swiglu_amax_workspace_bytes(2, 64) == 2 * 1 * 4
    rc = lib.flw_swiglu_fwd(P, P, 16384, 3392, 3392, 3392, P, 3392, P, P, need - 4, None)
    assert rc == 3 and b"workspace" in lib.flw_last_error()
    rc = lib.flw_swiglu_bwd(P, P, 0, 64, 64, 64, P, 64, P, P, 64, P, P, 64, None)
    assert rc == 1 and b"empty" in lib.flw_last_error()
    rc = lib.flw_quant_tensor_t_e4m3_amax(P, 64, 64, 64, None, P, 64, P, 64, P, None)
    assert rc == 1 and b"null amax" in lib.flw_last_error()
    need = lib.flw_quant_tensor_t_workspace_bytes(1000, 1280)              # 16 + one u32 per chunk
    assert need == 16 + 4 * ((1000 * 1280 // 64 + 127) // 128)
    rc = lib.flw_quant_tensor_t_e4m3(P, 1000, 1288, 1288, P, 1288, P, 1024, P, P, need, None)
    assert rc == 1 and b"multiple of 16" in lib.flw_last_error()
    rc = lib.flw_quant_tensor_t_e4m3(P, 1000, 1280, 1280, P, 1280, P, 992, P, P, need, None)
    assert rc == 1 and b"ld must be >= rows" in lib.flw_last_error()
    rc = lib.flw_quant_tensor_t_e4m3(P, 1000, 1280, 1280, P, 1280, P, 1024, P, P, need - 4, None)
    assert rc == 3 and b"workspace" in lib.flw_last_error()
    rc = lib.flw_quant_tensor_t_e4m3(P, 0, 1280, 1280, P, 1280, P, 1024, P, P, need, None)
    assert rc == 1 and b"empty" in lib.flw_last_error()
