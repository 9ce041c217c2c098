// Diagnostic: run the hardware fp32 -> e4m3 conversion (v_cvt_pk_fp8_f32) that the attention
// kernel uses to quantise P, over caller-supplied values, so tests can compare it bit for bit
// with the exact rounding rule. Not part of the attention path itself.
#include "flw_common.h"

namespace flw {

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

}  // namespace flw

using namespace flw;

extern "C" int flw_diag_cvt_e4m3(const float* x, uint8_t* out, int64_t n, int hardware, void* stream) {
  FLW_REQUIRE(x != nullptr && out != nullptr && n > 0, FLW_E_INVALID, "bad arguments");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (hardware) {
    FLW_REQUIRE(n % 2 == 0, FLW_E_INVALID, "hardware conversion works on pairs: n must be even");
    const int64_t np = n / 2;
    hipLaunchKernelGGL(cvt_hw_kernel, dim3((unsigned)((np + 255) / 256)), dim3(256), 0, s, x, out, np);
  } else {
    hipLaunchKernelGGL(cvt_sw_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, out, n);
  }
  return check_launch("flw_diag_cvt_e4m3");
}
