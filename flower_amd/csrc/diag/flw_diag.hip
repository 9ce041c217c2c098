// Diagnostics library (libflower_amd_diag.so), built beside the product library and never linked
// into it: instruments that check the device arithmetic the product kernels rely on, and price the
// attention loop's instruction classes. Nothing on the attention / quantiser / GEMM path calls it.
//
// flw_diag_cvt_e4m3      the hardware fp32 -> e4m3 converter (v_cvt_pk_fp8_f32, the attention
//                        kernel's P conversion and the quantisers' fast path) against the exact
//                        software rounding, on caller-given values.
// flw_diag_quotient      x / s by IEEE division against the quantisers' reciprocal-and-correct
//                        sequence (div_by_scale), on caller-given pairs.
// flw_diag_issue_probe   issue cost on one SIMD of the instruction classes the FP8 attention loop is
//                        made of, alone and with the QK^T / PV MFMA. Every probe kernel runs
//                        kIters iterations per lane of eight independent chains of one instruction
//                        (inline assembly, so the instruction is exactly the one named), and/or two
//                        independent chains of v_mfma_scale_f32_32x32x64_f8f6f4. Launched with
//                        256-thread workgroups, four per CU (four waves per SIMD, the attention
//                        kernel's occupancy). The host divides the kernel time by the instructions
//                        issued per SIMD.
// flw_diag_mfma_e4m3_dot the attention kernel's score product (the same MFMA on e4m3 operands in
//                        fragment order) on caller-given operands, so a test can measure its fp32
//                        accumulation against the exact dot product.
#include "flw_common.h"

namespace flw {

typedef int dv8i __attribute__((ext_vector_type(8)));
typedef float dv16f __attribute__((ext_vector_type(16)));

constexpr int kIters = 1024;

__global__ __launch_bounds__(256) void cvt_hw_kernel(const float* __restrict__ x, uint8_t* __restrict__ out,
                                                     int64_t npairs) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= npairs) return;
  const int w = __builtin_amdgcn_cvt_pk_fp8_f32(x[2 * i], x[2 * i + 1], 0, false);
  out[2 * i] = (uint8_t)(w & 0xFF);
  out[2 * i + 1] = (uint8_t)((w >> 8) & 0xFF);
}

__global__ __launch_bounds__(256) void cvt_sw_kernel(const float* __restrict__ x, uint8_t* __restrict__ out,
                                                     int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  out[i] = (uint8_t)(f32_to_e4m3(x[i]) & 0xFF);
}

// mode 0: IEEE x / s;  mode 1: the quantisers' reciprocal-and-correct quotient.
__global__ __launch_bounds__(256) void quotient_kernel(const float* __restrict__ x, int64_t n,
                                                       const float* __restrict__ s, int64_t ns,
                                                       uint32_t* __restrict__ out, int mode) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n * ns) return;
  const float xv = x[i % n], sv = s[i / n];
  const float q = mode == 0 ? xv / sv : div_by_scale(xv, sv, 1.0f / sv);
  out[i] = __float_as_uint(q);
}

enum : int {
  P_FMA = 1, P_EXP = 2, P_MAX3 = 4, P_CVT = 8, P_MUL = 16, P_PERM = 32, P_MFMA = 64,
};

template <int MASK>
__global__ __launch_bounds__(256) void issue_probe_kernel(float* out, float seed) {
  float x[8];
  int w[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    x[i] = seed * (float)(threadIdx.x + i) * 1e-6f - 0.5f;
    w[i] = (int)threadIdx.x * 7 + i;
  }
  dv16f acc0 = {}, acc1 = {};
  dv8i a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (int)(threadIdx.x * 0x01010101u) ^ i;
    b[i] = (int)(threadIdx.x * 0x00010001u) + i;
  }
  for (int it = 0; it < kIters; ++it) {
    if (MASK & P_MFMA) {
      acc0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc0, 0, 0, 0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, acc1, 0, 0, 0, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (MASK & P_FMA) asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(x[i]) : "v"(x[(i + 3) & 7]), "v"(x[(i + 5) & 7]));
        if (MASK & P_EXP) asm volatile("v_exp_f32 %0, %0" : "+v"(x[i]));
        if (MASK & P_MAX3) asm volatile("v_max3_f32 %0, %0, %1, %2" : "+v"(x[i]) : "v"(x[(i + 1) & 7]), "v"(x[(i + 2) & 7]));
        if (MASK & P_CVT) asm volatile("v_cvt_pk_fp8_f32 %0, %1, %2" : "+v"(w[i]) : "v"(x[i]), "v"(x[(i + 1) & 7]));
        if (MASK & P_MUL) asm volatile("v_mul_f32 %0, %0, %1" : "+v"(x[i]) : "v"(x[(i + 4) & 7]));
        if (MASK & P_PERM) asm volatile("v_permlane32_swap_b32 %0, %1" : "+v"(w[i]), "+v"(w[(i + 1) & 7]));
      }
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += x[i] + (float)w[i];
#pragma unroll
  for (int i = 0; i < 16; ++i) s += acc0[i] + acc1[i];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

// The attention kernel's score product on given operands: problem p computes the 32 x 32 block
// A_p B_p (+ A2_p B2_p when chain != 0, the two-chunk accumulation of head_dim 128) with
// v_mfma_scale_f32_32x32x64_f8f6f4 on e4m3 codes. Operands arrive in fragment order, 32 bytes per
// lane (A: row lane % 32, k = 32 (lane / 32) + 0..31; B: column lane % 32, the same k), and the
// lane's 16 results are written as d[p][64 v + lane] (column lane % 32, row 8 (v / 4) +
// 4 (lane / 32) + v % 4). Every access is inside problem p's 2 KB / 4 KB.
__global__ __launch_bounds__(64) void mfma_e4m3_dot_kernel(const uint8_t* __restrict__ a,
                                                           const uint8_t* __restrict__ b,
                                                           const uint8_t* __restrict__ a2,
                                                           const uint8_t* __restrict__ b2, float* __restrict__ d,
                                                           int chain) {
  const int64_t p = blockIdx.x;
  const int lane = threadIdx.x;
  auto frag = [&](const uint8_t* src) __attribute__((always_inline)) {
    const uint4* q = reinterpret_cast<const uint4*>(src + p * 2048 + 32 * lane);
    const uint4 x = q[0], y = q[1];
    return dv8i{(int)x.x, (int)x.y, (int)x.z, (int)x.w, (int)y.x, (int)y.y, (int)y.z, (int)y.w};
  };
  dv16f acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(frag(a), frag(b), dv16f{}, 0, 0, 0, 0, 0, 0);
  if (chain) acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(frag(a2), frag(b2), acc, 0, 0, 0, 0, 0, 0);
#pragma unroll
  for (int v = 0; v < 16; ++v) d[p * 1024 + 64 * v + lane] = acc[v];
}

}  // namespace flw

using namespace flw;

extern "C" int flw_diag_mfma_e4m3_dot(const uint8_t* a, const uint8_t* b, const uint8_t* a2, const uint8_t* b2,
                                      float* d, int64_t nprobe, int chain, void* stream) {
  FLW_REQUIRE(a != nullptr && b != nullptr && d != nullptr && (!chain || (a2 != nullptr && b2 != nullptr)),
              FLW_E_INVALID, "null operand");
  FLW_REQUIRE(nprobe > 0 && nprobe <= 0x7FFFFFFF, FLW_E_INVALID, "nprobe out of range");
  FLW_REQUIRE(((uintptr_t)a & 15) == 0 && ((uintptr_t)b & 15) == 0 && ((uintptr_t)d & 3) == 0 &&
              (!chain || (((uintptr_t)a2 & 15) == 0 && ((uintptr_t)b2 & 15) == 0)),
              FLW_E_INVALID, "operands must be 16-byte aligned");
  hipLaunchKernelGGL(mfma_e4m3_dot_kernel, dim3((unsigned)nprobe), dim3(64), 0, static_cast<hipStream_t>(stream),
                     a, b, a2, b2, d, chain);
  return check_launch("flw_diag_mfma_e4m3_dot");
}

// Instruction-class mask combinations the host may ask for (each is its own kernel).
#define FLW_ISSUE_PROBES(X)                                                                         \
  X(P_FMA) X(P_EXP) X(P_MAX3) X(P_CVT) X(P_MUL) X(P_PERM) X(P_MFMA) X(P_MFMA | P_FMA)             \
  X(P_MFMA | P_EXP) X(P_MFMA | P_MAX3) X(P_MFMA | P_CVT) X(P_MFMA | P_MUL) X(P_FMA | P_EXP)       \
  X(P_MFMA | P_FMA | P_EXP)

extern "C" int flw_diag_issue_probe(int mask, float* out, int64_t out_count, int blocks, void* stream) {
  FLW_REQUIRE(out != nullptr && blocks > 0 && out_count >= (int64_t)blocks * 256, FLW_E_INVALID,
              "out needs blocks * 256 floats");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const void* k = nullptr;
#define FLW_PICK(M) if (mask == (M)) k = reinterpret_cast<const void*>(&issue_probe_kernel<(M)>);
  FLW_ISSUE_PROBES(FLW_PICK)
#undef FLW_PICK
  FLW_REQUIRE(k != nullptr, FLW_E_INVALID, "no issue probe for mask %d", mask);
  const Timer t = take_timer();
  (void)launch_args(k, dim3((unsigned)blocks), dim3(256), 0, s, t.start, t.stop, out, 1.0f);
  return check_launch("flw_diag_issue_probe");
}

extern "C" int flw_diag_issue_probe_iters(void) { return kIters; }

extern "C" int flw_diag_cvt_e4m3(const float* x, uint8_t* out, int64_t n, int hardware, void* stream) {
  FLW_REQUIRE(x != nullptr && out != nullptr && n > 0, FLW_E_INVALID, "bad arguments");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (hardware) {
    FLW_REQUIRE(n % 2 == 0, FLW_E_INVALID, "hardware conversion works on pairs: n must be even");
    const int64_t np = n / 2;
    FLW_REQUIRE((np + 255) / 256 <= 0x7FFFFFFF, FLW_E_UNSUPPORTED, "too many values");
    hipLaunchKernelGGL(cvt_hw_kernel, dim3((unsigned)((np + 255) / 256)), dim3(256), 0, s, x, out, np);
  } else {
    FLW_REQUIRE((n + 255) / 256 <= 0x7FFFFFFF, FLW_E_UNSUPPORTED, "too many values");
    hipLaunchKernelGGL(cvt_sw_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, out, n);
  }
  return check_launch("flw_diag_cvt_e4m3");
}

extern "C" int flw_diag_quotient(const float* x, int64_t n, const float* scales, int64_t n_scales,
                                 uint32_t* out, int mode, void* stream) {
  FLW_REQUIRE(x && scales && out && n > 0 && n_scales > 0, FLW_E_INVALID, "bad arguments");
  FLW_REQUIRE(mode == 0 || mode == 1, FLW_E_INVALID, "mode must be 0 (IEEE) or 1 (reciprocal + correction)");
  const int64_t total = n * n_scales;
  FLW_REQUIRE((total + 255) / 256 <= 0x7FFFFFFF, FLW_E_UNSUPPORTED, "too many quotients");
  hipLaunchKernelGGL(quotient_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, n, scales, n_scales, out, mode);
  return check_launch("flw_diag_quotient");
}
