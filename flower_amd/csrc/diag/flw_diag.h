/* Diagnostics library libflower_amd_diag.so (flower_amd/csrc/diag/flw_diag.hip): instruments for
 * tests and bench.py, built beside the product library and not part of it. None of these has a
 * counterpart in the reference. Status codes and flw_last_error() as in include/flower_amd.h (the
 * diagnostics library carries its own copy of the error state). */
#ifndef FLW_DIAG_H
#define FLW_DIAG_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char* flw_last_error(void);
int flw_abi_version(void);
int flw_time_next_launch(void* start_event, void* stop_event);

/* No counterpart in the reference. Converts n fp32 values to e4m3 codes on the device, with the
 * hardware instruction the attention kernel uses for P (hardware = 1, v_cvt_pk_fp8_f32, n even)
 * or with the library's exact software rounding (hardware = 0), so a test can check the two
 * agree bit for bit on the values the kernel feeds it. */
int flw_diag_cvt_e4m3(const float* x, uint8_t* out, int64_t n, int hardware, void* stream);

/* No counterpart in the reference. The quotient x[i] / scale[j] for every pair (i, j), as raw
 * fp32 bits in out[j * n + i]: mode 0 with the IEEE division, mode 1 with the quantisers'
 * reciprocal-and-correct sequence, so a test can check the two agree bit for bit. */
int flw_diag_quotient(const float* x, int64_t n, const float* scales, int64_t n_scales,
                      uint32_t* out, int mode, void* stream);

/* No counterpart in the reference. Issue-cost probe of the attention loop's instruction classes:
 * one kernel of `blocks` 256-thread workgroups in which every wave runs
 * flw_diag_issue_probe_iters() iterations of 32 independent instructions of each VALU class in
 * `mask` (1 v_fma_f32, 2 v_exp_f32, 4 v_max3_f32, 8 v_cvt_pk_fp8_f32, 16 v_mul_f32,
 * 32 v_permlane32_swap_b32) and / or 2 independent v_mfma_scale_f32_32x32x64_f8f6f4 (64).
 * Supported masks: 1, 2, 4, 8, 16, 32, 64, 65, 66, 68, 72, 80, 3, 67. out: blocks * 256 floats
 * (a checksum per thread). Armable with flw_time_next_launch. */
int flw_diag_issue_probe(int mask, float* out, int64_t out_count, int blocks, void* stream);
int flw_diag_issue_probe_iters(void);

/* No counterpart in the reference. The attention kernel's score product on given e4m3 operands,
 * so a test can measure how far the FP8 MFMA's fp32 accumulation is from the exact dot product:
 * nprobe independent 32 x 32 x 64 products d[p] = a[p] b[p] (+ a2[p] b2[p] when chain != 0, as
 * the two 64-deep chunks of head_dim 128 accumulate). a, b, a2, b2: nprobe x 2048 bytes in
 * fragment order (lane-major, 32 bytes per lane: A row lane % 32 / B column lane % 32, k =
 * 32 (lane / 32) + 0..31); d: nprobe x 1024 floats, d[p][64 v + lane] = row 8 (v / 4) +
 * 4 (lane / 32) + v % 4, column lane % 32. 16-byte aligned operands. */
int flw_diag_mfma_e4m3_dot(const uint8_t* a, const uint8_t* b, const uint8_t* a2, const uint8_t* b2,
                           float* d, int64_t nprobe, int chain, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLW_DIAG_H */
