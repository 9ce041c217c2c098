// Diagnostic: issue cost on one SIMD of the instruction classes the FP8 attention loop is made of,
// alone and in combination with the QK^T / PV MFMA, so the kernel's time can be accounted for
// from measured per-instruction costs instead of nominal rates. Not part of the attention path.
//
// Every probe kernel runs kIters iterations per lane of eight independent chains of one
// instruction (inline assembly, so the instruction is exactly the one named), and/or two
// independent chains of v_mfma_scale_f32_32x32x64_f8f6f4 (the attention kernel's MFMA). Launched
// with 256-thread workgroups, four per CU (four waves per SIMD, the attention kernel's
// occupancy). The host divides the kernel time by the instructions issued per SIMD.
#include "flw_common.h"

namespace flw {

typedef int dv8i __attribute__((ext_vector_type(8)));
typedef float dv16f __attribute__((ext_vector_type(16)));

constexpr int kIters = 1024;

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

}  // namespace flw

using namespace flw;

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
