// Shared device helpers and host-side error plumbing for libflower_amd (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/flower_amd.h"

namespace flw {

// ---------------------------------------------------------------- host: error state
// Every entry point returns 0 on success or a FLW_E* code; the message of the last failure on
// the calling thread is kept here for flw_last_error().
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

// Kernel timing: flw_time_next_launch() arms an event pair on the calling thread; the next entry
// point takes it (take_timer disarms) and hands `start` to its first launch and `stop` to its last.
// hipExtLaunchKernel records each event from that dispatch's own start / end timestamps.
struct Timer {
  hipEvent_t start = nullptr, stop = nullptr;
};
Timer take_timer();
// Re-arm (part of) a taken pair for an entry point that calls other entry points in turn.
void arm_timer(Timer t);
// Compute units of the current device (cached per device; 256 if the query fails).
int compute_units();

// e4m3 quantisation of 1-3 (B, H, T, D) tensors of one shape (flw_quant.hip): amax pass + quantise
// pass, or, with amax_given ([tensor][scale group] |x| max bit patterns from the producer), the
// quantise pass alone.
// Optional pre-quantisation transform of the first two tensors (q, k): HeadRMSNorm and / or RoPE
// (tables [T, D] in the input dtype), the transformed values written to qout / kout if non-null.
struct QkTransform {
  int norm = 0;
  float eps = 0.0f;
  const void* rcos = nullptr;
  const void* rsin = nullptr;
  void* qout = nullptr;
  void* kout = nullptr;
};
int quant_bhtd_n(int n, const void* const* xs, int dtype, int64_t B, int64_t H, int64_t T,
                 int64_t D, const int64_t* strides, int granularity, const int* layouts,
                 uint8_t* const* outs, float* const* scale_outs, void* ws, size_t ws_bytes,
                 hipStream_t stream, Timer tm, const uint32_t* amax_given = nullptr,
                 const QkTransform* xf = nullptr, float* q_rcp_deferred = nullptr);

// Launch of a kernel taking one parameter struct, optionally recording start / stop events.
template <typename P>
inline hipError_t launch_ext(const void* kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream,
                             P p, hipEvent_t start, hipEvent_t stop) {
  void* args[] = {static_cast<void*>(&p)};
  return hipExtLaunchKernel(kernel, grid, block, args, lds, stream, start, stop, 0);
}

// Launch of a kernel taking plain arguments. The argument types must be exactly the kernel's
// parameter types (no conversion happens through the void* array).
template <typename... A>
inline hipError_t launch_args(const void* kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream,
                              hipEvent_t start, hipEvent_t stop, A... a) {
  void* args[] = {static_cast<void*>(&a)...};
  return hipExtLaunchKernel(kernel, grid, block, args, lds, stream, start, stop, 0);
}

// A single-kernel entry point: the whole armed pair goes to its one launch.
template <typename P>
inline hipError_t launch_timed(const void* kernel, dim3 grid, dim3 block, hipStream_t stream, P p) {
  const Timer t = take_timer();
  return launch_ext(kernel, grid, block, 0, stream, p, t.start, t.stop);
}

#define FLW_REQUIRE(cond, code, ...)                      \
  do {                                                    \
    if (!(cond)) return ::flw::set_error((code), __VA_ARGS__); \
  } while (0)

// ---------------------------------------------------------------- device: number formats
constexpr float kE4m3Max = 448.0f;
constexpr float kEps = 1e-12f;   // the reference's amax / scale floor

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 bits, round to nearest even; NaN -> 0x7FC0 (quiet). The NaN test is on the bit
// pattern so it holds in translation units built with relaxed NaN handling.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  return (u & 0x7FFFFFFFu) > 0x7F800000u ? 0x7FC0u : r;
}
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16_bits(f)); }

// f32_to_bf16_bits of two values, packed lo | hi << 16, by the converter (v_cvt_pk_bf16_f32:
// round to nearest even, one instruction for both) with NaN made 0x7FC0 as above (the converter
// keeps NaN payloads).
typedef __bf16 flw_bf16x2 __attribute__((ext_vector_type(2)));
typedef float flw_f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16x2_rne_raw(float a, float b) {   // NaN payloads kept
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((flw_f32x2{a, b}), flw_bf16x2));
}
// Two 16-bit lanes of one register: max over packed halves is one v_pk_max_u16.
typedef unsigned short flw_u16x2 __attribute__((ext_vector_type(2)));
// Per-half max of |bf16| bit patterns (sign cleared; NaN orders above inf) of packed pair w into m.
__device__ __forceinline__ flw_u16x2 abs_max_bf16x2(flw_u16x2 m, uint32_t w) {
  return __builtin_elementwise_max(m, __builtin_bit_cast(flw_u16x2, w & 0x7FFF7FFFu));
}
// Every NaN half of a packed bf16 pair made 0x7FC0.
__device__ __forceinline__ uint32_t bf16x2_canon_nan(uint32_t w) {
  w = (w & 0x7FFFu) > 0x7F80u ? (w & 0xFFFF0000u) | 0x7FC0u : w;
  return (w & 0x7FFF0000u) > 0x7F800000u ? (w & 0x0000FFFFu) | 0x7FC00000u : w;
}
__device__ __forceinline__ uint32_t bf16x2_rne(float a, float b) {
  return bf16x2_canon_nan(bf16x2_rne_raw(a, b));
}

// fp32 -> OCP e4m3fn code, round to nearest even, NOT saturating (|x| >= 464+ -> NaN 0x7F),
// NaN / inf -> sign | 0x7F. Integer-exact; the low byte of the result is the code.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
  uint32_t u = __float_as_uint(x);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7FFFFFFFu;
  // normal range: rebias the exponent (127 -> 7) and round the fraction to 3 bits
  uint32_t r = a - (120u << 23);
  uint32_t nrm = (r + 0x7FFFFu + ((r >> 20) & 1u)) >> 20;
  nrm = nrm > 0x7Fu ? 0x7Fu : nrm;
  // subnormal range (|x| < 2^-6): multiples of 2^-9, round half to even
  uint32_t sub = (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);
  uint32_t code = a >= 0x3C800000u ? nrm : sub;
  return code | sign;
}

// e4m3fn code -> fp32 (exact); 0x7F / 0xFF -> NaN.
__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
  uint32_t s = (c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 0xFu;
  uint32_t m = c & 7u;
  float v = e == 0 ? (float)m * 0.001953125f                        // m * 2^-9
                   : __uint_as_float(((e + 120u) << 23) | (m << 20));
  v = ((c & 0x7Fu) == 0x7Fu) ? __uint_as_float(0x7FC00000u) : v;   // NaN, by its bit pattern
  return __uint_as_float(__float_as_uint(v) | s);
}

// x / s from r = RN(1 / s): one product and two FMAs, the correctly rounded quotient whenever
// |x / s| >= 2^-20 (below that the correction can underflow, but every such quotient is an e4m3
// zero); the sign is copied from x so that -0 and tiny negatives keep the reference's sign. Used
// by the quantisers and by the attention kernel's quantise-on-load of Q, so both produce the same
// codes.
__device__ __forceinline__ float div_by_scale(float x, float s, float r) {
  const float q0 = x * r;
  const float e = fmaf(-q0, s, x);
  return __builtin_copysignf(fmaf(e, r, q0), x);
}

// Finite test on the bit pattern (holds in translation units built without NaN semantics).
__device__ __forceinline__ bool finite_bits(float x) {
  return (__float_as_uint(x) & 0x7F800000u) != 0x7F800000u;
}

// |x| as an unsigned bit pattern: ordered like |x| for finite values, NaN above +inf, so an
// integer max over it is an abs-max that propagates NaN (as torch.amax does).
__device__ __forceinline__ uint32_t abs_bits(float x) { return __float_as_uint(x) & 0x7FFFFFFFu; }

// Wave64 reductions.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    uint32_t w = (uint32_t)__shfl_xor((int)v, o, 64);
    v = v > w ? v : w;
  }
  return v;
}

// Loads of 16 bytes of an input tensor, widened to fp32.
template <typename T> struct Vec16;
template <> struct Vec16<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void load(const void* p, float* out) {
    float4 v = *reinterpret_cast<const float4*>(p);
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  }
  __device__ __forceinline__ static void unpack(uint4 v, float* out) {
    out[0] = __uint_as_float(v.x); out[1] = __uint_as_float(v.y);
    out[2] = __uint_as_float(v.z); out[3] = __uint_as_float(v.w);
  }
};
template <> struct Vec16<uint16_t> {   // bf16
  static constexpr int N = 8;
  __device__ __forceinline__ static void load(const void* p, float* out) {
    unpack(*reinterpret_cast<const uint4*>(p), out);
  }
  __device__ __forceinline__ static void unpack(uint4 v, float* out) {
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __uint_as_float(w[i] << 16);
      out[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  }
};

// Rounding to the tensor's dtype (bf16: round to nearest even, NaN quietened; fp32: identity).
template <typename T>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (sizeof(T) == 2) return round_bf16(x);
  return x;
}

// Sum of x over an aligned group of `lanes` consecutive lanes (1, 2, 4, 8, 16 or 32), the same
// bits in every lane of the group: quad butterflies (lane ^ 1, lane ^ 2) by DPP, then the mirrored
// half row and row (lane 7 - i, 15 - i: the partner holds the other half's sum, and a + b == b + a),
// then lane ^ 16. The pairing is ((s0 + s1) + (s2 + s3)) + ((s4 + s5) + (s6 + s7)) ... at every width.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float group_sum(float x, int lanes) {
  if (lanes >= 2) x = x + dpp_f32<0xB1>(x);                        // quad_perm [1, 0, 3, 2]
  if (lanes >= 4) x = x + dpp_f32<0x4E>(x);                        // quad_perm [2, 3, 0, 1]
  if (lanes >= 8) x = x + dpp_f32<0x141>(x);                       // row_half_mirror
  if (lanes >= 16) x = x + dpp_f32<0x140>(x);                      // row_mirror
  if (lanes >= 32) x = x + __shfl_xor(x, 16, 64);
  return x;
}

// The pre-attention transform of CausalSelfAttention.qkv_heads (flower/models/base.py:630-637) on
// one lane's Vec16<T>::N consecutive values f of a head row of d values (d = 32, 64 or 128), every
// step rounded to the tensor's dtype as the reference's torch ops round it:
//   HeadRMSNorm (base.py:355-357, when `norm`): h = dtype(x * rsqrt(mean(x^2) + eps)), fp32 maths;
//     the row's sum of squares is an fma chain over the lane's values, then group_sum over the
//     `lanes` lanes that hold the row; the mean is an exact power-of-two scaling; rsqrt is the
//     hardware v_rsq_f32 (1 ulp, like the reference's GPU torch.rsqrt);
//   RoPE (base.py:478-483, rotate_half :465-469; when `rope`):
//     out[2i]   = dtype(dtype(h[2i] c) + dtype(-h[2i+1] s)),
//     out[2i+1] = dtype(dtype(h[2i+1] c) + dtype(h[2i] s)),
//     c / s the lane's N entries of the [T, D] tables' row for this position (already loaded).
// bf16 roundings go through the pair converter (v_cvt_pk_bf16_f32, nearest even) when every value
// the wave transforms is finite and the norm's eps is positive (no NaN can arise then); otherwise
// the wave takes the exact software rounding, which also makes every NaN the quiet 0x7FC0 that
// torch's bf16 rounding gives -- the two agree bit for bit on every finite result. With pk (bf16
// only), the words of the result pairs are also written there, packed as stored (value 2i in the
// low half), by the last step that ran; pk keeps what it held when no step runs. Every lane of a
// group must call this together (it exchanges lanes); an invalid lane (padding, zeros) uses no
// table values and keeps its zeros. c / sn always name register arrays (read only when `rope`): a
// pointer chosen at run time between an array and null would force the arrays into scratch memory.
template <typename T, bool HW>
__device__ __forceinline__ void head_norm_rope_core(float* f, bool norm, float eps, int d, int lanes, bool valid,
                                                    bool rope, const float* c, const float* sn,
                                                    uint32_t* pk = nullptr) {
  // Separate products and sums, as the reference's separate torch ops round them: no FMA
  // contraction in this function (hipcc contracts a * b + c by default, which would change the
  // fp32 results).
#pragma clang fp contract(off)
  constexpr int N = Vec16<T>::N;
  // Rounds a and b to T; for bf16 also returns them packed (a in the low half).
  auto rnd2 = [](float& a, float& b) __attribute__((always_inline)) -> uint32_t {
    if constexpr (sizeof(T) == 2) {
      if constexpr (HW) {
        const uint32_t w = bf16x2_rne_raw(a, b);
        a = __uint_as_float(w << 16);
        b = __uint_as_float(w & 0xFFFF0000u);
        return w;
      } else {
        a = round_bf16(a);
        b = round_bf16(b);
        return (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xFFFF0000u);
      }
    }
    return 0u;
  };
  if (norm) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < N; ++i) ss = fmaf(f[i], f[i], ss);
    ss = group_sum(ss, lanes);
    const float r = __builtin_amdgcn_rsqf(__builtin_ldexpf(ss, -__builtin_ctz((unsigned)d)) + eps);
#pragma unroll
    for (int i = 0; i < N; i += 2) {
      float a = f[i] * r, b = f[i + 1] * r;
      const uint32_t w = rnd2(a, b);
      f[i] = valid ? a : 0.0f;
      f[i + 1] = valid ? b : 0.0f;
      if (pk != nullptr) pk[i / 2] = valid ? w : 0u;
    }
  }
  if (rope && valid) {
#pragma unroll
    for (int i = 0; i < N; i += 2) {
      float a0 = f[i] * c[i], a1 = f[i + 1] * c[i + 1];
      float b0 = -f[i + 1] * sn[i], b1 = f[i] * sn[i + 1];
      rnd2(a0, a1);
      rnd2(b0, b1);
      float o0 = a0 + b0, o1 = a1 + b1;
      const uint32_t w = rnd2(o0, o1);
      f[i] = o0;
      f[i + 1] = o1;
      if (pk != nullptr) pk[i / 2] = w;
    }
  }
}

template <typename T>
__device__ __forceinline__ void head_norm_rope(float* f, bool norm, float eps, int d, int lanes, bool valid,
                                               bool rope, const float* c, const float* sn) {
  if constexpr (sizeof(T) == 2) {
    uint32_t mx = 0;
#pragma unroll
    for (int i = 0; i < Vec16<T>::N; ++i) { const uint32_t a = abs_bits(f[i]); mx = mx > a ? mx : a; }
    const bool bad = mx >= 0x7F800000u || (norm && !(eps > 0.0f));
    if (__builtin_amdgcn_ballot_w64(bad) == 0) {     // wave-uniform
      head_norm_rope_core<T, true>(f, norm, eps, d, lanes, valid, rope, c, sn);
      return;
    }
  }
  head_norm_rope_core<T, false>(f, norm, eps, d, lanes, valid, rope, c, sn);
}

// LDS pointer type: the 32-bit LDS address of a __shared__ object is (uint32_t)(lds_u8_t*)p.
typedef __attribute__((address_space(3))) uint8_t lds_u8_t;

// A 64-key x D tile of e4m3 codes (D = 32, 64, 128) staged in LDS as rows: row r (key r) at r D,
// its 16-byte chunk c at position c ^ vrow_swizzle(r, D). The swizzle keeps both accesses free of
// bank conflicts: writes of consecutive chunks of consecutive rows, and the transposed reads of
// vtile_run (a 16-lane group reads one 16-byte chunk of the 8 rows r0 + {0-3, 8-11}: row bits 3 and,
// at D = 128, 1 pick the chunk).
__device__ __forceinline__ int vrow_swizzle(int r, int D) {
  return D == 128 ? (((r >> 1) & 1) | (((r >> 3) & 1) << 1)) : ((r >> 3) & 1);
}
__device__ __forceinline__ int vrow_offset(int r, int c16, int D) { return r * D + 16 * (c16 ^ vrow_swizzle(r, D)); }

// One 16-byte run of the tiled-V layout (FLW_LAYOUT_VTILE: dim d, key block kb of 32 keys, half
// hb; byte 4 a + c = key 32 kb + 8 a + 4 hb + c) read from a row-staged tile, for lane n of a
// 16-lane group whose lanes take dims d0 .. d0 + 15 (d0 a multiple of 16) with the same kb, hb.
// ds_read_b64_tr_b8 works on groups of 16 lanes (measured lane layout): lane 2 j + a supplies the
// address of 8 consecutive bytes (row j, columns 8 a .. 8 a + 7 of the group's 16) and lane n
// receives column n of the 8 rows, byte j from row j. Two reads (rows 32 kb + 4 hb + {0-3, 8-11}
// and the same + 16) give the run. Every lane of the group must call this together.
__device__ __forceinline__ uint4 vtile_run(const uint8_t* tile, int D, int d0, int kb, int hb, int n) {
  typedef int v2i __attribute__((ext_vector_type(2)));
  typedef __attribute__((address_space(3))) v2i lds_v2i;
  const int j = n >> 1, a = n & 1;
  const int r0 = 32 * kb + 4 * hb + (j < 4 ? j : j + 4);      // r0 + 16 has the same swizzle
  const uint8_t* src = tile + vrow_offset(r0, d0 >> 4, D) + 8 * a;
  const v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(lds_u8_t*)src);
  const v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(lds_u8_t*)(src + 16 * D));
  return make_uint4((uint32_t)lo.x, (uint32_t)lo.y, (uint32_t)hi.x, (uint32_t)hi.y);
}

// s_waitcnt immediate that waits until at most n vector-memory operations are outstanding
// (gfx9 encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14; expcnt / lgkmcnt left free).
constexpr int vmcnt_imm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

// Workgroup barrier without the release fence __syncthreads() carries (which would drain every
// outstanding global load, i.e. the whole prefetch, at each K step). Callers wait for the loads
// they need with an explicit vmcnt first; the empty asm statements keep the compiler from moving
// memory operations across the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace flw
