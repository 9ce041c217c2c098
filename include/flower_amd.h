/*
 * libflower_amd -- C ABI of the MI355X (gfx950) FP8 sliding-window-attention path.
 *
 * Plain pointers and sizes only. Every pointer argument is device memory owned by the caller
 * (the library never allocates or frees). Every call is asynchronous on `stream` (a
 * hipStream_t passed as void*; NULL = the default stream) and returns 0 on success or a
 * FLW_E_* code, with a message available from flw_last_error() on the calling thread.
 * Strides are in elements. The innermost (D / K) dimension must be contiguous.
 *
 * Reference interfaces each entry point replaces are cited as path:line in sims1253/flower.
 */
#ifndef FLOWER_AMD_H
#define FLOWER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FLW_ABI_VERSION 1

enum flw_status {
  FLW_OK = 0,
  FLW_E_INVALID = 1,      /* bad shape / stride / alignment / null pointer */
  FLW_E_UNSUPPORTED = 2,  /* valid request this build does not implement (e.g. head_dim 96) */
  FLW_E_WORKSPACE = 3,    /* workspace too small */
  FLW_E_LAUNCH = 4        /* HIP launch error */
};

enum flw_dtype { FLW_F32 = 0, FLW_BF16 = 1 };

/* Scale granularity for a (B, H, T, D) tensor: one scale, one per head h (amax over B, T, D),
 * or one per (b, h) slice (amax over T, D). Scale arrays hold 1, H or B*H floats. */
enum flw_granularity { FLW_SCALE_TENSOR = 0, FLW_SCALE_HEAD = 1, FLW_SCALE_BH = 2, FLW_SCALE_COLUMN = 3 };

/* Layout of e4m3 codes written by flw_quant_e4m3:
 *   FLW_LAYOUT_BHTD  -- contiguous (B, H, T, D), one byte per element;
 *   FLW_LAYOUT_VTILE -- the attention kernel's V operand: per (b, h) slice, ceil(T/64) tiles of
 *     64 keys x D bytes (keys past T are zero). Inside a tile, element (key kk, dim d) sits at
 *        (d/32)*2048 + (kk/32)*1024 + ((d%32) + 32*h)*16 + b,
 *        r = kk%32, h = (r/4)%2, b = 4*(r/8) + r%4,
 *     i.e. each 16-byte run is one lane's share of a 32x32x64 FP8 MFMA operand of V^T. */
enum flw_layout { FLW_LAYOUT_BHTD = 0, FLW_LAYOUT_VTILE = 1, FLW_LAYOUT_BTHD = 2 };
/* FLW_LAYOUT_BTHD -- contiguous (B, T, H, D), token-major: the layout of the attention output the
 *   output projection reads as rows of H D values (the bf16 attention's O and dO, below). */

/* GEMM modes. A8W8: activations quantised per row to e4m3, FP8 x FP8 MFMA (the _fp8_head
 * recipe). W8A16: e4m3 weights widened to bf16 in the kernel, bf16 activations unquantised. */
enum flw_gemm_mode { FLW_GEMM_A8W8 = 0, FLW_GEMM_W8A16 = 1 };

const char* flw_last_error(void);
int flw_abi_version(void);

/* Measurement hook, no counterpart in the reference: arms two hipEvent_t (created with timing
 * enabled, passed as void*) on the calling thread. The next call on this thread of an entry point
 * that launches the quantisers, the attention kernel or the FP8 GEMM takes them: its first kernel
 * records `start` and its last kernel records `stop` from their own dispatch timestamps
 * (hipExtLaunchKernel), so hipEventElapsedTime(start, stop) spans exactly that call's kernels.
 * Both NULL disarms. */
int flw_time_next_launch(void* start_event, void* stop_event);

/* ---------------------------------------------------------------- quantisation */

/* Workspace for flw_quant_e4m3 / flw_fake_quant_e4m3 on a (B, H, T, D) tensor (amax partials). */
size_t flw_quant_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D);

/* The amax pass of `_per_tensor_fp8` (flower/kernels/fp8_swa_attention.py:201,
 * `x.abs().amax().float()`) on its own: |x| max per scale group (granularity: 1, H or B*H groups)
 * written to amax_out as the bit patterns of the fp32 values. Non-negative floats order like
 * their bit patterns, so shards can combine their amax with an integer all_reduce(MAX) before
 * quantising with flw_quant_e4m3_amax; NaN propagates (its pattern is above +inf's).
 * workspace: flw_quant_workspace_bytes(B, H, T, D). x as for flw_quant_e4m3. */
int flw_amax_e4m3(const void* x, int dtype, int64_t B, int64_t H, int64_t T, int64_t D,
                  int64_t stride_b, int64_t stride_h, int64_t stride_t, int granularity,
                  uint32_t* amax_out, void* workspace, size_t workspace_bytes, void* stream);

/* flw_quant_e4m3 with the amax given (amax: the groups' |x| max bit patterns, e.g. from
 * flw_amax_e4m3, combined across shards): the quantise pass only, no workspace. Same scale and
 * code arithmetic, so flw_quant_e4m3_amax(x, flw_amax_e4m3(x)) == flw_quant_e4m3(x) bit for bit.
 * An amax below the data's own |x| max still gives the reference's clamp(x / s, -448, 448)-then-
 * cast codes for that amax: values past it saturate at +-448 (inf too), NaN stays NaN. */
int flw_quant_e4m3_amax(const void* x, int dtype, int64_t B, int64_t H, int64_t T, int64_t D,
                        int64_t stride_b, int64_t stride_h, int64_t stride_t, int granularity,
                        int layout, const uint32_t* amax, uint8_t* out, float* scale_out,
                        void* stream);

/* Bytes of a FLW_LAYOUT_VTILE buffer for a (B, H, T, D) tensor: B*H*ceil(T/64)*64*D. */
size_t flw_vtile_bytes(int64_t B, int64_t H, int64_t T, int64_t D);

/* The attention kernel reads V only in FLW_LAYOUT_VTILE (V^T operand order, written by the
 * quantisers). For V codes held in plain (B, H, T, D) layout -- e.g. the e4m3 tensor
 * `_per_tensor_fp8(v)` returns (flower/kernels/fp8_swa_attention.py:195-205, :244) -- this
 * permutes them into v_tiles (flw_vtile_bytes bytes; keys past T zero), one pass over the codes.
 * codes: element (= byte) strides, 16-byte aligned rows; D in {32, 64, 128}. */
int flw_vtile_from_bhtd(const uint8_t* codes, int64_t B, int64_t H, int64_t T, int64_t D,
                        int64_t stride_b, int64_t stride_h, int64_t stride_t, uint8_t* v_tiles,
                        void* stream);

/* e4m3 quantisation with amax scales, replacing `_per_tensor_fp8`
 * (flower/kernels/fp8_swa_attention.py:195-205) and extending it to per-head / per-(b,h):
 *   scale = max(amax, 1e-12) / 448  (fp32),  code = e4m3_rne(clamp(x / scale, -448, 448)).
 * The scale stays on the device (scale_out: 1, H or B*H floats); no host synchronisation.
 * x: fp32 or bf16, strides in elements, D contiguous, 16-byte aligned rows. */
int flw_quant_e4m3(const void* x, int dtype, int64_t B, int64_t H, int64_t T, int64_t D,
                   int64_t stride_b, int64_t stride_h, int64_t stride_t, int granularity,
                   int layout, uint8_t* out, float* scale_out, void* workspace,
                   size_t workspace_bytes, void* stream);

/* flw_quant_e4m3 on three tensors of one shape in one pass pair (the three `_per_tensor_fp8`
 * calls of flower/kernels/fp8_swa_attention.py:242-244): q and k to FLW_LAYOUT_BHTD codes (q8,
 * k8), v to FLW_LAYOUT_VTILE (v_tiles). strides: 9 values, {b, h, t} of q, k, v. scales_out:
 * 3 x (1 | H | B*H) floats in the order q, k, v. workspace: 3 * flw_quant_workspace_bytes. */
int flw_quant_qkv_e4m3(const void* q, const void* k, const void* v, int dtype, int64_t B,
                       int64_t H, int64_t T, int64_t D, const int64_t* strides, int granularity,
                       uint8_t* q8, uint8_t* k8, uint8_t* v_tiles, float* scales_out,
                       void* workspace, size_t workspace_bytes, void* stream);

/* flw_quant_qkv_e4m3 with Q's codes deferred to the attention kernel (flw_fp8_swa_fwd_qx): the
 * amax pass covers q, k, v; the quantise pass writes k8, v_tiles and all scales, plus q_rcp_out
 * (1 | H | B*H floats, RN(1 / q scale)), and q8 codes only for Q's scale groups whose amax is not
 * finite (left to the quantiser's exact path). Half the `_per_tensor_fp8` calls of
 * flower/kernels/fp8_swa_attention.py:242-244 in full, the Q one split with the attention kernel. */
int flw_quant_qkv_e4m3_deferq(const void* q, const void* k, const void* v, int dtype, int64_t B,
                              int64_t H, int64_t T, int64_t D, const int64_t* strides, int granularity,
                              uint8_t* q8, uint8_t* k8, uint8_t* v_tiles, float* scales_out,
                              float* q_rcp_out, void* workspace, size_t workspace_bytes, void* stream);

/* The FP8 attention's quantisation point in `CausalSelfAttention.qkv_heads`
 * (flower/models/base.py:618-639: qkv -> heads -> HeadRMSNorm -> RoPE, "quantize AFTER QK-norm
 * and RoPE", :634-637) fused with the three `_per_tensor_fp8` calls it feeds
 * (flower/kernels/fp8_swa_attention.py:242-244): flw_quant_qkv_e4m3 on q', k', v where
 *   q' = rope(norm(q)), k' = rope(norm(k)), every step rounded to the input dtype as torch rounds:
 *   norm (qk_norm != 0; HeadRMSNorm, base.py:341-357): x' = dtype(x * (1 / sqrt(mean(x^2) + eps)))
 *     over each (b, h, t) row of D, fp32 maths (IEEE sqrt and division);
 *   rope (rope_cos / rope_sin: [T, D] contiguous tables in the input dtype, i.e. the module's
 *     cached cos / sin cast to it as base.py:478-483 casts them; both NULL: no RoPE):
 *     out[2i] = dtype(dtype(x'[2i] c[2i]) + dtype(-x'[2i+1] s[2i])),
 *     out[2i+1] = dtype(dtype(x'[2i+1] c[2i+1]) + dtype(x'[2i] s[2i+1]))  (rotate_half, :465-469).
 * The amax pass and the quantise pass both apply the transform, so q' and k' never go through
 * HBM; q_out / k_out (contiguous (B, H, T, D), input dtype, may be NULL) receive them if given.
 * Other arguments, layouts and the workspace as flw_quant_qkv_e4m3. */
int flw_qk_norm_rope_quant_e4m3(const void* q, const void* k, const void* v, int dtype, int64_t B,
                                int64_t H, int64_t T, int64_t D, const int64_t* strides, int qk_norm,
                                float eps, const void* rope_cos, const void* rope_sin, int granularity,
                                uint8_t* q8, uint8_t* k8, uint8_t* v_tiles, float* scales_out,
                                void* q_out, void* k_out, void* workspace, size_t workspace_bytes,
                                void* stream);

/* CausalSelfAttention.qkv_heads (flower/models/base.py:618-639) for training, bf16: the qkv
 * projection's output qkv [B T, qkv_row_stride] (q | k | v column blocks of H D values) split into
 * per-head q', k', v, contiguous (B, H, T, D) bf16, with HeadRMSNorm of q and k when qk_norm
 * (base.py:341-357) and RoPE of q and k from the [T, D] bf16 tables (base.py:436-483), rounded as
 * torch rounds them (the transform of flw_qk_norm_rope_quant_e4m3); one pass in place of the torch
 * ops' ~10 forward kernels. D in {32, 64, 128}; 16-byte aligned rows and tables. */
int flw_qkv_heads_fwd(const void* qkv, int64_t B, int64_t T, int64_t H, int64_t D, int64_t qkv_row_stride,
                      int qk_norm, float eps, const void* rope_cos, const void* rope_sin, void* q, void* k,
                      void* v, void* stream);

/* The backward of flw_qkv_heads_fwd, as torch's autograd of the same expressions computes it:
 * dq', dk', dv contiguous (B, H, T, D) bf16 and the forward's qkv -> dqkv [B T, dqkv_row_stride]
 * bf16. RoPE backward with torch's bf16 roundings (t1 = bf16(g cos), t2 = bf16(g sin),
 * dn[2i] = bf16(t1[2i] + t2[2i+1]), dn[2i+1] = bf16(t1[2i+1] - t2[2i])), then the HeadRMSNorm
 * backward in fp32 from the forward's input x (r = rsqrt(mean(x^2) + eps),
 * dx = bf16(bf16(dn r) - bf16(x r^3 sum(dn x) / D)), the two casts' gradients summed in bf16 as
 * autograd sums them); dv copied into the v columns. */
int flw_qkv_heads_bwd(const void* qkv, int64_t B, int64_t T, int64_t H, int64_t D, int64_t qkv_row_stride,
                      int qk_norm, float eps, const void* rope_cos, const void* rope_sin, const void* dq,
                      const void* dk, const void* dv, void* dqkv, int64_t dqkv_row_stride, uint32_t* dqkv_amax,
                      void* workspace, size_t workspace_bytes, void* stream);
/* dqkv_amax (may be NULL; then workspace may be NULL too): also |dqkv|'s maximum as an fp32 bit
 * pattern (NaN above inf), the amax half of the qkv projection's tensorwise gradient cast, from
 * per-workgroup maxima in a workspace of flw_qkv_heads_amax_workspace_bytes and a folding launch. */
size_t flw_qkv_heads_amax_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D);

/* RMSNorm forward for training, replacing RMSNorm.forward (flower/models/base.py:336-338) on bf16
 * rows: x [rows, cols] (row stride x_row_stride), bf16 weight [cols] -> h [rows, cols]
 * (h_row_stride), r = 1 / sqrt(mean(x^2) + eps) in fp32, h = bf16(bf16(x r) w). cols a multiple of
 * 8, at most 8192; 16-byte aligned rows. */
int flw_rmsnorm_fwd(const void* x, int64_t rows, int64_t cols, int64_t x_row_stride, const void* weight, float eps,
                    void* h, int64_t h_row_stride, void* stream);

/* Bytes of fp32 workspace flw_rmsnorm_bwd needs for its weight-gradient partial sums. */
size_t flw_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols);

/* x + a followed by RMSNorm, the residual add of Block.forward (flower/models/base.py:720) and the
 * ln2 that reads its result (:721), in one pass: sum = bf16(x + a) [rows, cols] (written: the
 * residual stream) and h = flw_rmsnorm_fwd of sum, bit for bit the two torch ops. */
int flw_add_rmsnorm_fwd(const void* x, const void* a, int64_t rows, int64_t cols, int64_t x_row_stride,
                        int64_t a_row_stride, const void* weight, float eps, void* sum, int64_t sum_row_stride,
                        void* h, int64_t h_row_stride, void* stream);

/* The backward of flw_rmsnorm_fwd as torch's autograd of base.py:337-338 computes it, from the
 * forward's x and weight and the gradient dh: dn = bf16(dh w),
 * dx = bf16(bf16(dn r) - bf16(x r^3 sum(dn x) / cols)) (the expression's two x.float() casts each
 * return a bf16 gradient, summed in bf16), dweight [cols] = bf16(sum over rows of bf16(dh n)),
 * n = bf16(x r), the sum in fp32 (over a fixed order: deterministic). dres (may be NULL): the
 * gradient x receives along the residual stream, added as autograd adds the two uses' gradients:
 * dx = bf16(dres + that). Two launches; the workspace holds partial sums only. */
int flw_rmsnorm_bwd(const void* x, int64_t rows, int64_t cols, int64_t x_row_stride, const void* weight, float eps,
                    const void* dh, int64_t dh_row_stride, const void* dres, int64_t dres_row_stride, void* dx,
                    int64_t dx_row_stride, void* dweight, void* workspace, size_t workspace_bytes, void* stream);

/* The SwiGLU product of FeedForward.forward (flower/models/base.py:538-550, smooth_swiglu off) on
 * bf16 rows: h = bf16(bf16(silu(gate)) up), silu(g) = g / (1 + exp(-g)) in fp32 (torch's silu).
 * gate, up, h [rows, cols] with their own row strides; cols a multiple of 8. h_amax (may be
 * NULL): also |h|'s maximum as an fp32 bit pattern (NaN above inf), the amax pass of the next FP8
 * linear's tensorwise cast done by this pass (per-workgroup maxima in the workspace of
 * flw_swiglu_amax_workspace_bytes, folded by a second launch). */
size_t flw_swiglu_amax_workspace_bytes(int64_t rows, int64_t cols);
int flw_swiglu_fwd(const void* gate, const void* up, int64_t rows, int64_t cols, int64_t gate_row_stride,
                   int64_t up_row_stride, void* h, int64_t h_row_stride, uint32_t* h_amax, void* workspace,
                   size_t workspace_bytes, void* stream);

/* The backward of flw_swiglu_fwd as torch's autograd computes it: ds = bf16(dh up),
 * dup = bf16(dh s) with s = bf16(silu(gate)), dgate = bf16(ds sig (1 + g (1 - sig))),
 * sig = 1 / (1 + exp(-g)) (torch's silu backward). dgate and dup share grad_row_stride.
 * grad_amax (may be NULL): [2] the |dgate| and |dup| maxima, as flw_swiglu_fwd's h_amax. */
int flw_swiglu_bwd(const void* gate, const void* up, int64_t rows, int64_t cols, int64_t gate_row_stride,
                   int64_t up_row_stride, const void* dh, int64_t dh_row_stride, void* dgate, void* dup,
                   int64_t grad_row_stride, uint32_t* grad_amax, void* workspace, size_t workspace_bytes,
                   void* stream);

/* flw_quant_qkv_e4m3 without a workspace: no counterpart in the reference. For callers that
 * cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): the amax partials live in a library-owned device array of
 * flw_noalloc_scratch_bytes() bytes (1 MiB) per GPU, held until the process ends; the call itself
 * allocates nothing. Limit: 3 * B * H * ceil(T / 128) * 4 bytes of partials must fit the array
 * (FLW_E_UNSUPPORTED otherwise). Outputs and their contract are those of flw_quant_qkv_e4m3. Calls
 * that overlap on one GPU (e.g. on two streams) share the array and race; serialise them. */
size_t flw_noalloc_scratch_bytes(void);
int flw_quant_qkv_e4m3_noalloc(const void* q, const void* k, const void* v, int dtype, int64_t B,
                               int64_t H, int64_t T, int64_t D, const int64_t* strides,
                               int granularity, uint8_t* q8, uint8_t* k8, uint8_t* v_tiles,
                               float* scales_out, void* stream);

/* Straight-through fake quantisation forward value, replacing `_fake_quant_e4m3`
 * (flower/models/base.py:167-203): out = x + (e4m3(x / s) * s - x), every step rounded to the
 * input dtype exactly as the reference's op sequence rounds (s itself in the input dtype).
 * out: contiguous (B, H, T, D) of the input dtype. scale_out may be NULL. */
int flw_fake_quant_e4m3(const void* x, int dtype, int64_t B, int64_t H, int64_t T, int64_t D,
                        int64_t stride_b, int64_t stride_h, int64_t stride_t, int granularity,
                        void* out, float* scale_out, void* workspace, size_t workspace_bytes,
                        void* stream);

/* Per-row e4m3 quantisation of a [rows, cols] matrix, replacing the scale / cast steps of
 * `CausalLM._fp8_head` (flower/models/base.py:912-918), used for GEMM activation rows and for
 * weight output channels (FP8 weight cache):
 *   scale[r] = max(amax_r / 448, 1e-12),  code = e4m3_rne(x / scale[r])  (no clamp).
 * out: contiguous [rows, cols]; scale_out: [rows]. */
int flw_quant_rows_e4m3(const void* x, int dtype, int64_t rows, int64_t cols, int64_t row_stride,
                        uint8_t* out, float* scale_out, void* stream);

/* Per-column e4m3 quantisation of a [rows, cols] matrix with the codes written TRANSPOSED,
 * out_t[cols, ld] (ld >= rows, ld % 16 == 0; rows past `rows` coded 0): the operands of the FP8
 * backward GEMMs that torchao's Float8Linear runs under `training.fp8_linear` (torchao 0.18.0,
 * uv.lock:1642-1644, not vendored; enabled at flower/train.py:368-370), where the reduction runs
 * over the rows (wgrad: tokens) or a weight is consumed along its other axis (dgrad).
 *   FLW_SCALE_COLUMN: scale[c] = max(amax_c / 448, 1e-12), code = e4m3_rne(x / scale[c])
 *                     (flw_quant_rows_e4m3 of the transpose); scale_out: [cols].
 *   FLW_SCALE_TENSOR: scale = max(amax, 1e-12) / 448, code = e4m3_rne(clamp(x / scale, +-448))
 *                     (flw_quant_e4m3's per-tensor codes, transposed); scale_out: [1].
 * cols and row_stride multiples of 8, rows 16-byte aligned. workspace: amax partials,
 * flw_quant_cols_workspace_bytes(rows, cols) bytes. */
size_t flw_quant_cols_workspace_bytes(int64_t rows, int64_t cols);
int flw_quant_cols_e4m3(const void* x, int dtype, int64_t rows, int64_t cols, int64_t row_stride,
                        int granularity, uint8_t* out_t, int64_t ld, float* scale_out, void* workspace,
                        size_t workspace_bytes, void* stream);

/* The tensorwise e4m3 cast of torchao Float8Linear (one scale for the whole matrix, the
 * reference's default recipe; torchao 0.18.0, not vendored, enabled at flower/train.py:368-370)
 * of a bf16 matrix x [rows, cols] written in both layouts the training GEMMs read: out8 [rows, cols]
 * (row stride ld8) for the forward / dgrad operand and out_t [cols, ldt] (ldt >= rows; columns
 * rows .. ldt - 1 zero) for the wgrad operand -- the codes of flw_quant_e4m3(FLW_SCALE_TENSOR) and
 * flw_transpose_e4m3 of them, bit for bit, from one read of x. scale_out[0] = the scale. Three
 * launches: the amax pass, its fold, the quantise-and-transpose pass. cols % 16 == 0; 16-byte
 * aligned rows; workspace of flw_quant_tensor_t_workspace_bytes(rows, cols). */
size_t flw_quant_tensor_t_workspace_bytes(int64_t rows, int64_t cols);
int flw_quant_tensor_t_e4m3(const void* x, int64_t rows, int64_t cols, int64_t row_stride, uint8_t* out8, int64_t ld8,
                            uint8_t* out_t, int64_t ldt, float* scale_out, void* workspace, size_t workspace_bytes,
                            void* stream);
/* flw_quant_tensor_t_e4m3 with x's |x| maximum given (a device fp32 bit pattern from its producer,
 * e.g. flw_swiglu_fwd's h_amax): the quantise-and-transpose pass alone, one launch. The codes are
 * those of flw_quant_tensor_t_e4m3 when amax is |x|'s true maximum. */
int flw_quant_tensor_t_e4m3_amax(const void* x, int64_t rows, int64_t cols, int64_t row_stride,
                                 const uint32_t* amax, uint8_t* out8, int64_t ld8, uint8_t* out_t, int64_t ldt,
                                 float* scale_out, void* stream);

/* e4m3 codes [rows, cols] transposed to out_t [cols, ld] (ld >= rows, ld % 16 == 0; columns
 * rows .. ld - 1 of out_t zero). With one scale for the whole matrix (the tensorwise recipe) a
 * matrix's per-column codes equal its per-row codes, so the transposed operands of the backward
 * GEMMs come from the forward's and the gradient's row codes by this byte transpose, as torchao's
 * Float8Linear reuses its tensorwise fp8 casts transposed (torchao 0.18.0, not vendored; enabled
 * at flower/train.py:368-370): flw_quant_cols_e4m3(FLW_SCALE_TENSOR) of the same matrix, bit for
 * bit, without reading it again in bf16. cols and row_stride multiples of 16, 16-byte aligned
 * codes and out_t. */
int flw_transpose_e4m3(const uint8_t* codes, int64_t rows, int64_t cols, int64_t row_stride, uint8_t* out_t,
                       int64_t ld, void* stream);

/* ---------------------------------------------------------------- attention */

/* FP8 causal sliding-window attention forward on pre-quantised operands, replacing the launch
 * of `_fp8_swa_fwd_kernel` (flower/kernels/fp8_swa_attention.py:249-258):
 *   q8, k8: (B, H, T, D) e4m3 with element strides q_strides[3] / k_strides[3] = {b, h, t};
 *   v_tiles: FLW_LAYOUT_VTILE e4m3 V (BHTD V codes: flw_fp8_swa_fwd_bhtd reads them as they are);
 *   scales: 1, H or B*H floats each (granularity);
 *   out: (B, H, T, D) fp32 or bf16 with strides out_strides[3].
 * Query i attends to keys j with j <= i and i - j < window; window <= 0 gives zeros.
 * D in {32, 64, 128}. */
int flw_fp8_swa_fwd(const uint8_t* q8, const int64_t* q_strides, const uint8_t* k8,
                    const int64_t* k_strides, const uint8_t* v_tiles, const float* q_scale,
                    const float* k_scale, const float* v_scale, int granularity, void* out,
                    int out_dtype, const int64_t* out_strides, int64_t B, int64_t H, int64_t T,
                    int64_t D, int64_t window, void* stream);

/* flw_fp8_swa_fwd with the scales indexed by element strides instead of a granularity, as the
 * boundary of flower/kernels/fp8_swa_attention.py:249-258 passes them: the scale of slice (b, h)
 * is q_scale[b * scale_stride_b + h * scale_stride_h] (likewise k, v); 0/0 is per tensor, 0/1 per
 * head, H/1 per (b, h), any other non-negative pair another layout of per-(b, h) scales. */
int flw_fp8_swa_fwd_scale_strides(const uint8_t* q8, const int64_t* q_strides, const uint8_t* k8,
                                  const int64_t* k_strides, const uint8_t* v_tiles, const float* q_scale,
                                  const float* k_scale, const float* v_scale, int64_t scale_stride_b,
                                  int64_t scale_stride_h, void* out, int out_dtype,
                                  const int64_t* out_strides, int64_t B, int64_t H, int64_t T, int64_t D,
                                  int64_t window, void* stream);

/* The launch of `_fp8_swa_fwd_kernel` (flower/kernels/fp8_swa_attention.py:249-258) with every
 * operand as the reference passes it: q8, k8, v8 (B, H, T, D) e4m3 codes as `_per_tensor_fp8`
 * returns them (:242-244), with byte strides {b, h, t} (multiples of 16, D contiguous), and the
 * scales indexed by element strides as in flw_fp8_swa_fwd_scale_strides. V is read in that layout
 * (no separate permutation pass): the kernel stages each V tile into the layout its MFMA operand
 * reads, so the output is flw_fp8_swa_fwd's on flw_vtile_from_bhtd(v8), bit for bit. */
int flw_fp8_swa_fwd_bhtd(const uint8_t* q8, const int64_t* q_strides, const uint8_t* k8,
                         const int64_t* k_strides, const uint8_t* v8, const int64_t* v_strides,
                         const float* q_scale, const float* k_scale, const float* v_scale,
                         int64_t scale_stride_b, int64_t scale_stride_h, void* out, int out_dtype,
                         const int64_t* out_strides, int64_t B, int64_t H, int64_t T, int64_t D,
                         int64_t window, void* stream);

/* flw_fp8_swa_fwd with Q in its input dtype, quantised on load by the attention kernel (the
 * `_per_tensor_fp8(q)` of flower/kernels/fp8_swa_attention.py:242 moved into the kernel's
 * prologue; every Q row is read by exactly one workgroup): q (B, H, T, D) bf16 or fp32 (= dtype,
 * also the output dtype) with element strides q_strides[3]; q_rcp: RN(1 / q_scale) per scale
 * group, and q8_nonfinite: contiguous (B, H, T, D) codes read only for groups whose scale is not
 * finite -- both as flw_quant_qkv_e4m3_deferq writes them. The codes, hence the output, are
 * those of flw_quant_qkv_e4m3 + flw_fp8_swa_fwd. */
int flw_fp8_swa_fwd_qx(const void* q, const int64_t* q_strides, const uint8_t* q8_nonfinite,
                       const float* q_rcp, const uint8_t* k8, const int64_t* k_strides,
                       const uint8_t* v_tiles, const float* q_scale, const float* k_scale,
                       const float* v_scale, int granularity, void* out, int dtype,
                       const int64_t* out_strides, int64_t B, int64_t H, int64_t T, int64_t D,
                       int64_t window, void* stream);

/* flw_fp8_swa_fwd that also writes the log-sum-exp of every query's scores, lse [B, H, T] fp32
 * (contiguous), natural log, in the units of the dequantised scores q . k / sqrt(D):
 * lse = m + ln(sum_j exp(s_j - m)) over the band, with the kernel's running maximum m and its fp32
 * row sum of the unquantised P (the sum the reference's l_i is, fp8_swa_attention.py:176) -- the
 * statistic flw_swa_bf16_bwd takes to rebuild P, so the FP8 forward can be trained through with
 * that backward (flower/kernels/swa_attention.py:307-359). -inf for a query with no key
 * in its band (window <= 0). */
int flw_fp8_swa_fwd_lse(const uint8_t* q8, const int64_t* q_strides, const uint8_t* k8,
                        const int64_t* k_strides, const uint8_t* v_tiles, const float* q_scale,
                        const float* k_scale, const float* v_scale, int granularity, void* out,
                        int out_dtype, const int64_t* out_strides, int64_t B, int64_t H, int64_t T,
                        int64_t D, int64_t window, float* lse, void* stream);

/* The dequantised values of e4m3 codes: out[b, h, t, d] = e4m3(code) * scale of (b, h)'s group
 * (granularity as above) as an fp32 product, rounded to out_dtype (FLW_BF16: nearest even). Codes in
 * FLW_LAYOUT_BHTD (contiguous) or FLW_LAYOUT_VTILE; out contiguous (B, H, T, D), 16-byte aligned.
 * The tensors the straight-through estimator of `_fake_quant_e4m3` (flower/models/base.py:167-203)
 * differentiates at: the backward of the FP8 attention runs on them. */
int flw_dequant_e4m3(const uint8_t* codes, int layout, int64_t B, int64_t H, int64_t T, int64_t D,
                     const float* scales, int granularity, void* out, int out_dtype, void* stream);

/* Workspace of flw_fp8_swa_attention_forward (e4m3 Q, K, tiled V, scales, amax partials). */
size_t flw_fp8_swa_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D);

/* The whole `fp8_swa_attention_forward(q, k, v, window)` of
 * flower/kernels/fp8_swa_attention.py:208-259: quantise Q, K, V (granularity as above), then
 * the fused FP8 attention; output in the input dtype. strides: 12 values, {b, h, t} of q, k, v,
 * out. scales_out (3 x 1|H|B*H floats: q, k, v) may be NULL. */
int flw_fp8_swa_attention_forward(const void* q, const void* k, const void* v, int dtype,
                                  const int64_t* strides, int64_t B, int64_t H, int64_t T,
                                  int64_t D, int64_t window, int granularity, void* out,
                                  float* scales_out, void* workspace, size_t workspace_bytes,
                                  void* stream);

/* flw_fp8_swa_attention_forward with the amax of Q, K and V supplied by their producer (u32
 * [3 * (1 | H | B*H)], |x| max fp32 bit patterns in the order q, k, v, e.g. from
 * flw_fp8_scaled_mm_group_amax): the quantiser's amax pass is skipped; scales, codes and the
 * output are those of flw_fp8_swa_attention_forward on the same inputs. A given maximum below the
 * data's own gives the reference's clamp(x / s, -448, 448)-then-cast codes for that maximum (Q is
 * checked against it inside the attention kernel, K and V in the quantiser). */
int flw_fp8_swa_attention_forward_amax(const void* q, const void* k, const void* v, int dtype,
                                       const int64_t* strides, int64_t B, int64_t H, int64_t T, int64_t D,
                                       int64_t window, int granularity, const uint32_t* amax, void* out,
                                       float* scales_out, void* workspace, size_t workspace_bytes,
                                       void* stream);

/* The producer of an FP8 linear's input fused with its per-row quantiser (flw_quant_rows_e4m3
 * semantics: scale = max(amax / 448, 1e-12) per row, codes = e4m3(h / scale), no clamp), one read
 * of the bf16 rows [rows, cols] (row stride in elements, cols <= 4096, multiples of 8):
 *   flw_rmsnorm_quant_rows_e4m3: h = bf16(bf16(x * (1 / sqrt(mean(x^2) + eps))) * weight[cols]),
 *     replacing RMSNorm (flower/models/base.py:324-338) followed by the next linear's activation
 *     quantisation (base.py:912,917 / torchao Float8Linear's input cast);
 *   flw_gelu_quant_rows_e4m3: h = bf16((0.5 x) (1 + erf(x / sqrt 2))), replacing the MLP's GELU
 *     (base.py:514-525) followed by the same quantisation.
 * h_out (bf16 [rows, cols], contiguous) receives h when not NULL. */
int flw_rmsnorm_quant_rows_e4m3(const void* x, int64_t rows, int64_t cols, int64_t row_stride,
                                const void* weight, float eps, uint8_t* out, float* scale_out,
                                void* h_out, void* stream);
int flw_gelu_quant_rows_e4m3(const void* x, int64_t rows, int64_t cols, int64_t row_stride,
                             uint8_t* out, float* scale_out, void* h_out, void* stream);

/* ---------------------------------------------------------------- bf16 sliding-window attention */

/* The differentiable bf16 causal sliding-window attention of flower/kernels/swa_attention.py
 * (`swa_attention`, :362-380; its Triton kernels :84-305). q, k, v, out, dout, dq, dk, dv:
 * contiguous (B, H, T, D) bf16, 16-byte aligned; D in {32, 64, 128}; window > 0 (query i attends
 * keys j with 0 <= i - j < window). Softmax and accumulation in fp32.
 * flw_swa_bf16_fwd: out, and lse = m + log(l) per query ([B, H, T] fp32, natural log) for the
 *   backward (the reference's _swa_fwd, :84-160).
 * flw_swa_bf16_bwd: dq, dk, dv from dout and the forward's out / lse (the reference's
 *   _swa_bwd_preprocess, _swa_bwd_dkdv and _swa_bwd_dq, :163-305); the workspace holds
 *   Delta = rowsum(dout * out). */
int flw_swa_bf16_fwd(const void* q, const void* k, const void* v, int64_t B, int64_t H, int64_t T,
                     int64_t D, int64_t window, void* out, float* lse, void* stream);
/* flw_swa_bf16_fwd writing O in out_layout: FLW_LAYOUT_BHTD (as flw_swa_bf16_fwd) or
 * FLW_LAYOUT_BTHD, O as (B, T, H, D) -- `a.transpose(1, 2).reshape(B, T, H D)` of
 * CausalSelfAttention.forward (flower/models/base.py:643-646) then is a view, no copy. */
int flw_swa_bf16_fwd_layout(const void* q, const void* k, const void* v, int64_t B, int64_t H, int64_t T,
                            int64_t D, int64_t window, void* out, int out_layout, float* lse, void* stream);
size_t flw_swa_bf16_bwd_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D);
int flw_swa_bf16_bwd(const void* q, const void* k, const void* v, const void* out, const void* dout,
                     const float* lse, int64_t B, int64_t H, int64_t T, int64_t D, int64_t window,
                     void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes,
                     void* stream);
/* flw_swa_bf16_bwd with O and dO in o_layout (FLW_LAYOUT_BHTD or FLW_LAYOUT_BTHD; q, k, v and the
 * gradients stay (B, H, T, D)): the forward's token-major O and the output projection's gradient
 * as it comes, without transposing either. */
int flw_swa_bf16_bwd_layout(const void* q, const void* k, const void* v, const void* out, const void* dout,
                            int o_layout, const float* lse, int64_t B, int64_t H, int64_t T, int64_t D,
                            int64_t window, void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes,
                            void* stream);

/* ---------------------------------------------------------------- GEMM */

/* Workspace of flw_fp8_linear (the per-row e4m3 activations and their scales in A8W8 mode; 0
 * bytes in W8A16 mode). */
size_t flw_fp8_linear_workspace_bytes(int64_t M, int64_t K, int mode);

/* y[M, N] (bf16) = x[M, K] (bf16) @ dequant(w8[N, K])^T, replacing the FP8 GEMM of
 * torchao Float8Linear / `torch._scaled_mm` (flower/models/base.py:919-923,
 * flower/precision.py:304-324). w_scale: N floats (per output channel) or 1 float
 * (w_scale_count = 1, per tensor). FLW_GEMM_A8W8 quantises x per row (flw_quant_rows_e4m3
 * semantics) into the workspace first, then FP8 x FP8 MFMA (K % 16 == 0). FLW_GEMM_W8A16 keeps x
 * in bf16, widens the e4m3 weight to bf16 in the kernel (exact) and multiplies on bf16 MFMA: no
 * workspace, K % 64 == 0, x rows 16-byte aligned. N % 4 == 0 in both modes. */
int flw_fp8_linear(const void* x, int64_t M, int64_t K, int64_t x_row_stride, const uint8_t* w8,
                   int64_t N, const float* w_scale, int64_t w_scale_count, int mode, void* y,
                   int64_t y_row_stride, void* workspace, size_t workspace_bytes, void* stream);

/* The scaled FP8 GEMM alone: y[M, N] (bf16) = (x8[M, K] . w8[N, K]) * x_scale[m] * w_scale[n],
 * fp32 accumulation (`torch._scaled_mm(x8, w8.t(), scale_a, scale_b, out_dtype=bf16)`,
 * flower/models/base.py:919-923). Scale counts: M or 1, and N or 1. */
int flw_fp8_scaled_mm(const uint8_t* x8, int64_t M, int64_t K, const uint8_t* w8, int64_t N,
                      const float* x_scale, int64_t x_scale_count, const float* w_scale,
                      int64_t w_scale_count, void* y, int64_t y_row_stride, void* stream);

/* flw_fp8_scaled_mm with a workspace for a split over K, for outputs with too few 256 x 256 tiles
 * to fill the GPU (the FP8 wgrad of a linear: [N, K] outputs reduced over the tokens): each tile's
 * K range is cut into up to 8 parts whose fp32 partial sums go to the workspace and are summed,
 * scaled and rounded to bf16 by a second kernel. Same result contract as flw_fp8_scaled_mm
 * (fp32 accumulation, summed in a different order). flw_fp8_scaled_mm_workspace_bytes returns 0
 * when no split applies; with a smaller workspace the call runs unsplit. */
/* flw_fp8_scaled_mm that also returns, for every group of group_cols consecutive output columns,
 * max |y| over all rows (as the fp32 bit pattern of the bf16 value, u32 [N / group_cols]): the
 * per-head amax of a QKV projection (group_cols = head_dim, groups ordered q heads, k heads,
 * v heads), so that the Q / K / V quantiser needs no amax pass of its own. This is the "fuse
 * quantisation into the producer" step of the path: `qkv_heads` (flower/models/base.py:618-639)
 * feeds `_per_tensor_fp8` (flower/kernels/fp8_swa_attention.py:195-205), whose amax this
 * replaces. group_cols: a power of two in [8, 256] dividing N; K % 64 == 0, N % 8 == 0,
 * 16-byte aligned y rows, M * K and N * K < 2^32 (other shapes return FLW_E_UNSUPPORTED; the
 * caller then takes the quantiser's own amax pass). amax_out is overwritten (cleared by the call
 * itself). */
int flw_fp8_scaled_mm_group_amax(const uint8_t* x8, int64_t M, int64_t K, const uint8_t* w8, int64_t N,
                                 const float* x_scale, int64_t x_scale_count, const float* w_scale,
                                 int64_t w_scale_count, void* y, int64_t y_row_stride, int64_t group_cols,
                                 uint32_t* amax_out, void* stream);

/* flw_fp8_scaled_mm_group_amax for a QKV projection whose q and k heads feed the FP8 attention
 * through `CausalSelfAttention.qkv_heads` (flower/models/base.py:618-639): before the q / k output
 * columns (n < qk_cols) are stored and before their maxima are taken, each head row of head_dim
 * values gets HeadRMSNorm (base.py:341-357, when qk_norm: fp32 maths, eps) and RoPE
 * (base.py:436-483, when rope_cos / rope_sin are given: [seq_len, head_dim] bf16 tables; output
 * row m is position m % seq_len), every step rounded to bf16 as the reference's torch ops round it
 * -- bit for bit the transform flw_qk_norm_rope_quant_e4m3 applies. y then holds q', k', v and
 * amax_out their per-head maxima, so the attention's quantiser needs neither an amax pass nor a
 * transform (flw_fp8_swa_attention_forward_amax). head_dim 32 / 64 / 128; qk_cols a multiple of
 * head_dim (2 * d_model for a fused QKV); seq_len divides M; the other requirements as
 * flw_fp8_scaled_mm_group_amax. */
int flw_fp8_scaled_mm_qk_norm_rope_amax(const uint8_t* x8, int64_t M, int64_t K, const uint8_t* w8, int64_t N,
                                        const float* x_scale, int64_t x_scale_count, const float* w_scale,
                                        int64_t w_scale_count, void* y, int64_t y_row_stride, int64_t head_dim,
                                        int64_t qk_cols, int qk_norm, float eps, const void* rope_cos,
                                        const void* rope_sin, int64_t seq_len, uint32_t* amax_out, void* stream);

size_t flw_fp8_scaled_mm_workspace_bytes(int64_t M, int64_t N, int64_t K);
int flw_fp8_scaled_mm_ws(const uint8_t* x8, int64_t M, int64_t K, const uint8_t* w8, int64_t N,
                         const float* x_scale, int64_t x_scale_count, const float* w_scale,
                         int64_t w_scale_count, void* y, int64_t y_row_stride, void* workspace,
                         size_t workspace_bytes, void* stream);

/* flw_fp8_scaled_mm with the block's residual add in the epilogue:
 * y = bf16(residual + bf16((x8 . w8^T) * x_scale[m] * w_scale[n])), i.e. `x + linear(h)` of
 * the decoder block (flower/models/base.py:698-722) with both terms rounded to bf16 as torch
 * adds them. residual: bf16 [M, N], row stride in elements; it may alias y. */
int flw_fp8_scaled_mm_residual(const uint8_t* x8, int64_t M, int64_t K, const uint8_t* w8, int64_t N,
                               const float* x_scale, int64_t x_scale_count, const float* w_scale,
                               int64_t w_scale_count, void* y, int64_t y_row_stride,
                               const void* residual, int64_t residual_row_stride, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLOWER_AMD_H */
