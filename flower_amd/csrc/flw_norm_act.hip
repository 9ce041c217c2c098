// The block's RMSNorm (flower/models/base.py:324-338) and the SwiGLU product of its FeedForward
// (base.py:535-551 with smooth_swiglu off: act = silu(gate), down(act * up)) for training on bf16
// activations, forward and backward, each one memory-bound pass over the rows (plus a small column
// reduction for the norm's weight gradient), with the roundings of the reference's torch
// expressions under eager autograd:
//   RMSNorm forward:  r = 1 / sqrt(mean(x^2) + eps) in fp32, n = bf16(x r), h = bf16(n w);
//     with a residual input a (the block's x + attn(...) feeding ln2), x = bf16(x0 + a) first,
//     written out as the residual stream;
//   RMSNorm backward: dn = bf16(dh w); dw = bf16(sum over rows of bf16(dh n)), the sum in fp32;
//     dx = bf16(bf16(dn r) - bf16(x r^3 sum(dn x) / cols)) -- x.float() appears twice in the
//     expression, and each cast hands back its own bf16 gradient, summed in bf16; with the residual
//     stream's gradient dres, dx = bf16(dres + that), the sum autograd forms where x has two uses;
//   SwiGLU forward:   s = bf16(g / (1 + exp(-g))), h = bf16(s u);
//   SwiGLU backward:  ds = bf16(dh u), du = bf16(dh s), sig = 1 / (1 + exp(-g)),
//     dg = bf16(ds sig (1 + g (1 - sig))) (torch's silu backward).
// NaN results are written as the quiet 0x7FC0 that torch's bf16 rounding gives.
//
// Row kernels: a workgroup of 4 waves, one row per wave at a time; a lane holds chunks of 8 values
// (16 bytes) v = lane + 64 i, i < NV, so a row of up to 512 NV values stays in registers; the row's
// sums are wave butterflies. The backward's waves walk rows with a grid stride and keep their
// columns' dw partial sums in registers; a workgroup folds its 4 waves' partials through LDS into
// one row of a [blocks, cols] fp32 workspace, which rmsnorm_dw_kernel sums per column.

#include "flw_common.h"

namespace flw {

// Backward workgroups, the rows of the dw partials: 3 per CU, as many as the 1280-column instance
// keeps resident (3 waves per SIMD); 512 took 42 us a norm at the 450M shape, 768 takes 36.
constexpr int kNormBlocks = 768;

__device__ __forceinline__ float norm_wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// a, b rounded to bf16 (kept as fp32) by one pair conversion (nearest even; a NaN stays a NaN).
__device__ __forceinline__ void round2_bf16(float& a, float& b) {
  const uint32_t t = bf16x2_rne_raw(a, b);
  a = __uint_as_float(t << 16);
  b = __uint_as_float(t & 0xFFFF0000u);
}

__device__ __forceinline__ uint4 pack_bf16x8(const float* f) {
  return make_uint4(bf16x2_canon_nan(bf16x2_rne_raw(f[0], f[1])), bf16x2_canon_nan(bf16x2_rne_raw(f[2], f[3])),
                    bf16x2_canon_nan(bf16x2_rne_raw(f[4], f[5])), bf16x2_canon_nan(bf16x2_rne_raw(f[6], f[7])));
}

// The row's 1 / sqrt(mean(x^2) + eps): an fma chain over the lane's values, the wave butterfly,
// a division by cols, IEEE sqrt and division. Chunks past the row end hold zeros.
template <int NV>
__device__ __forceinline__ float row_rstd(const uint4* xb, int cols, float eps) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    float f[8];
    Vec16<uint16_t>::unpack(xb[i], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(f[e], f[e], ss);
  }
  const float ms = norm_wave_sum(ss) / (float)cols;
  return 1.0f / __builtin_sqrtf(ms + eps);
}

template <int NV>
__device__ __forceinline__ void load_row(const uint16_t* src, int nvec, int lane, uint4* out) {
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = lane + 64 * i;
    out[i] = v < nvec ? *reinterpret_cast<const uint4*>(src + 8 * v) : make_uint4(0, 0, 0, 0);
  }
}

template <int NV, bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(const uint16_t* __restrict__ x, int64_t rows, int cols,
                                                          int64_t xs, const uint16_t* __restrict__ w, float eps,
                                                          uint16_t* __restrict__ h, int64_t hs,
                                                          const uint16_t* __restrict__ a, int64_t as,
                                                          uint16_t* __restrict__ sum, int64_t ss) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;                        // wave-uniform
  const int lane = threadIdx.x & 63, nvec = cols >> 3;
  uint4 xb[NV];
  load_row<NV>(x + row * xs, nvec, lane, xb);
  if (ADD) {                                      // x = bf16(x0 + a), kept as the residual stream
    uint4 ab[NV];
    load_row<NV>(a + row * as, nvec, lane, ab);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float f[8], g[8];
      Vec16<uint16_t>::unpack(xb[i], f);
      Vec16<uint16_t>::unpack(ab[i], g);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] += g[e];
      xb[i] = pack_bf16x8(f);
      const int v = lane + 64 * i;
      if (v < nvec) *reinterpret_cast<uint4*>(sum + row * ss + 8 * v) = xb[i];
    }
  }
  const float r = row_rstd<NV>(xb, cols, eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = lane + 64 * i;
    if (v >= nvec) continue;
    float f[8], g[8], o[8];
    Vec16<uint16_t>::unpack(xb[i], f);
    Vec16<uint16_t>::load(w + 8 * v, g);
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
#pragma clang fp contract(off)
      float n0 = f[e] * r, n1 = f[e + 1] * r;
      round2_bf16(n0, n1);
      o[e] = n0 * g[e];
      o[e + 1] = n1 * g[e + 1];
    }
    *reinterpret_cast<uint4*>(h + row * hs + 8 * v) = pack_bf16x8(o);
  }
}

template <int NV, bool RES>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const uint16_t* __restrict__ x, int64_t rows, int cols,
                                                          int64_t xs, const uint16_t* __restrict__ w, float eps,
                                                          const uint16_t* __restrict__ dh, int64_t dhs,
                                                          uint16_t* __restrict__ dx, int64_t dxs,
                                                          float* __restrict__ part,
                                                          const uint16_t* __restrict__ dres, int64_t drs) {
  extern __shared__ float fold[];                 // [cols]: one wave's partials at a time
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nvec = cols >> 3;
  float acc[NV][8];
  uint4 wb[NV];
  load_row<NV>(w, nvec, lane, wb);
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[i][e] = 0.0f;
  for (int64_t row = (int64_t)blockIdx.x * 4 + wave; row < rows; row += (int64_t)gridDim.x * 4) {
    uint4 xb[NV], gb[NV];
    load_row<NV>(x + row * xs, nvec, lane, xb);
    load_row<NV>(dh + row * dhs, nvec, lane, gb);
    const float r = row_rstd<NV>(xb, cols, eps);
    uint32_t dn[NV][4];                           // bf16(dh w), packed as pairs
    float sd = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float f[8], g[8], wf[8];
      Vec16<uint16_t>::unpack(xb[i], f);
      Vec16<uint16_t>::unpack(gb[i], g);
      Vec16<uint16_t>::unpack(wb[i], wf);
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
#pragma clang fp contract(off)
        float n0 = f[e] * r, n1 = f[e + 1] * r;
        round2_bf16(n0, n1);
        float d0 = g[e] * wf[e], d1 = g[e + 1] * wf[e + 1];
        round2_bf16(d0, d1);
        float p0 = g[e] * n0, p1 = g[e + 1] * n1;
        round2_bf16(p0, p1);
        dn[i][e >> 1] = (__float_as_uint(d0) >> 16) | (__float_as_uint(d1) & 0xFFFF0000u);
        acc[i][e] += p0;
        acc[i][e + 1] += p1;
        sd = fmaf(d0, f[e], sd);
        sd = fmaf(d1, f[e + 1], sd);
      }
    }
    sd = norm_wave_sum(sd);
    const float k = sd * (r * r * r) / (float)cols;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int v = lane + 64 * i;
      if (v >= nvec) continue;
      float f[8], o[8];
      Vec16<uint16_t>::unpack(xb[i], f);
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
#pragma clang fp contract(off)
        float a0 = __uint_as_float(dn[i][e >> 1] << 16) * r;
        float a1 = __uint_as_float(dn[i][e >> 1] & 0xFFFF0000u) * r;
        float b0 = f[e] * k, b1 = f[e + 1] * k;
        round2_bf16(a0, a1);
        round2_bf16(b0, b1);
        o[e] = a0 - b0;
        o[e + 1] = a1 - b1;
      }
      if (RES) {                                  // bf16(dres + bf16(o)): autograd's sum
        float d[8];
        Vec16<uint16_t>::load(dres + row * drs + 8 * v, d);
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          round2_bf16(o[e], o[e + 1]);
          o[e] += d[e];
          o[e + 1] += d[e + 1];
        }
      }
      *reinterpret_cast<uint4*>(dx + row * dxs + 8 * v) = pack_bf16x8(o);
    }
  }
  // Fold the 4 waves' column partials into part[blockIdx.x] in a fixed order (wave 0 + 1 + 2 + 3):
  // waves 1, 2, 3 in turn hand theirs to wave 0 through one row of LDS.
  for (int q = 1; q < 4; ++q) {
    if (wave == q) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int v = lane + 64 * i;
        if (v >= nvec) continue;
        float4* dst = reinterpret_cast<float4*>(fold + 8 * v);
        dst[0] = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
        dst[1] = make_float4(acc[i][4], acc[i][5], acc[i][6], acc[i][7]);
      }
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int v = lane + 64 * i;
        if (v >= nvec) continue;
        const float4* src = reinterpret_cast<const float4*>(fold + 8 * v);
        const float4 a = src[0], b = src[1];
        acc[i][0] += a.x; acc[i][1] += a.y; acc[i][2] += a.z; acc[i][3] += a.w;
        acc[i][4] += b.x; acc[i][5] += b.y; acc[i][6] += b.z; acc[i][7] += b.w;
      }
    }
    __syncthreads();
  }
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int v = lane + 64 * i;
      if (v >= nvec) continue;
      float4* dst = reinterpret_cast<float4*>(part + (int64_t)blockIdx.x * cols + 8 * v);
      dst[0] = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
      dst[1] = make_float4(acc[i][4], acc[i][5], acc[i][6], acc[i][7]);
    }
  }
}

// dw[c] = bf16(sum over the nblk partial rows of part[., c]): 16 columns per workgroup, 16 slices
// of the rows each, folded through LDS in a fixed order.
__global__ __launch_bounds__(256) void rmsnorm_dw_kernel(const float* __restrict__ part, int nblk, int cols,
                                                         uint16_t* __restrict__ dw) {
  __shared__ float red[16][17];
  const int cl = threadIdx.x & 15, s = threadIdx.x >> 4;
  const int c = blockIdx.x * 16 + cl;
  float a = 0.0f;
  if (c < cols) {
#pragma unroll 8
    for (int b = s; b < nblk; b += 16) a += part[(int64_t)b * cols + c];
  }
  red[s][cl] = a;
  __syncthreads();
  if (s == 0 && c < cols) {
    float t = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) t += red[j][cl];
    dw[c] = (uint16_t)f32_to_bf16_bits(t);
  }
}

struct SwigluParams {
  const uint16_t* g;
  const uint16_t* u;
  const uint16_t* dh;           // backward
  uint16_t* out0;               // forward h; backward dgate
  uint16_t* out1;               // backward dup
  int64_t gs, us, dhs, os;
  int cpr;                      // 16-byte chunks per row
  int total;                    // rows * cpr
  uint32_t* part;               // with AMAX: [2][gridDim.x] per-workgroup |out0|, |out1| maxima
};

constexpr int kSwigluBlocks = 8192;   // grid-stride workgroups (at most): rows of the amax partials

// |value| maxima of 8 packed bf16 values folded into two 16-bit lanes (v_pk_max_u16 over the bit
// patterns with the sign cleared: the amax pass's ordering, NaN above inf); as_f32_bits widens the
// larger lane to the fp32 bit pattern of that bf16 value.
__device__ __forceinline__ flw_u16x2 absmax_bf16x8(uint4 w, flw_u16x2 m) {
  m = abs_max_bf16x2(m, w.x);
  m = abs_max_bf16x2(m, w.y);
  m = abs_max_bf16x2(m, w.z);
  return abs_max_bf16x2(m, w.w);
}
__device__ __forceinline__ uint32_t as_f32_bits(flw_u16x2 m) {
  return (uint32_t)(m[0] > m[1] ? m[0] : m[1]) << 16;
}

__device__ __forceinline__ uint32_t block_max_256(uint32_t m, uint32_t* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t t = (uint32_t)__shfl_xor((int)m, o, 64);
    m = m > t ? m : t;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  uint32_t r = red[0];
#pragma unroll
  for (int i = 1; i < 4; ++i) r = r > red[i] ? r : red[i];
  return r;
}

// 16-byte chunks (8 values) of the rows with a grid stride, chunk index i -> (row i / cpr,
// chunk i % cpr). With AMAX each workgroup also writes the |value| maxima of what it wrote.
template <bool AMAX>
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(SwigluParams p) {
  __shared__ uint32_t red[4];
  flw_u16x2 mx = {0, 0};
#pragma unroll 2
  for (int i = blockIdx.x * 256 + threadIdx.x; i < p.total; i += gridDim.x * 256) {
    const int64_t m = i / p.cpr;
    const int c = 8 * (i - (int)m * p.cpr);
    float g[8], u[8], o[8];
    Vec16<uint16_t>::load(p.g + m * p.gs + c, g);
    Vec16<uint16_t>::load(p.u + m * p.us + c, u);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = round_bf16(g[e] / (1.0f + expf(-g[e]))) * u[e];
    const uint4 w = pack_bf16x8(o);
    *reinterpret_cast<uint4*>(p.out0 + m * p.os + c) = w;
    if (AMAX) mx = absmax_bf16x8(w, mx);
  }
  if (AMAX) {
    const uint32_t m = block_max_256(as_f32_bits(mx), red);
    if (threadIdx.x == 0) p.part[blockIdx.x] = m;
  }
}

template <bool AMAX>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(SwigluParams p) {
  __shared__ uint32_t red[4];
  flw_u16x2 mg = {0, 0}, mu = {0, 0};
#pragma unroll 2
  for (int i = blockIdx.x * 256 + threadIdx.x; i < p.total; i += gridDim.x * 256) {
    const int64_t m = i / p.cpr;
    const int c = 8 * (i - (int)m * p.cpr);
    float g[8], u[8], d[8], dg[8], du[8];
    Vec16<uint16_t>::load(p.g + m * p.gs + c, g);
    Vec16<uint16_t>::load(p.u + m * p.us + c, u);
    Vec16<uint16_t>::load(p.dh + m * p.dhs + c, d);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float den = 1.0f + expf(-g[e]);     // silu's and sigmoid's 1 + exp(-g), one exp
      const float s = round_bf16(g[e] / den);
      const float ds = round_bf16(d[e] * u[e]);
      du[e] = d[e] * s;
      const float sig = 1.0f / den;
      dg[e] = ds * sig * (1.0f + g[e] * (1.0f - sig));
    }
    const uint4 wg = pack_bf16x8(dg), wu = pack_bf16x8(du);
    *reinterpret_cast<uint4*>(p.out0 + m * p.os + c) = wg;
    *reinterpret_cast<uint4*>(p.out1 + m * p.os + c) = wu;
    if (AMAX) {
      mg = absmax_bf16x8(wg, mg);
      mu = absmax_bf16x8(wu, mu);
    }
  }
  if (AMAX) {
    const uint32_t a = block_max_256(as_f32_bits(mg), red);
    __syncthreads();                               // red is reused
    const uint32_t b = block_max_256(as_f32_bits(mu), red);
    if (threadIdx.x == 0) {
      p.part[blockIdx.x] = a;
      p.part[gridDim.x + blockIdx.x] = b;
    }
  }
}

// One workgroup of 1024 per array (blockIdx.x) folds n partial maxima into out[blockIdx.x].
__global__ __launch_bounds__(1024) void fold_max_kernel(const uint32_t* __restrict__ part, int n,
                                                        uint32_t* __restrict__ out) {
  __shared__ uint32_t red[16];
  const uint32_t* src = part + (int64_t)blockIdx.x * n;
  uint32_t m = 0;
  for (int i = threadIdx.x; i < n; i += 1024) m = m > src[i] ? m : src[i];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t t = (uint32_t)__shfl_xor((int)m, o, 64);
    m = m > t ? m : t;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = red[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) r = r > red[i] ? r : red[i];
    out[blockIdx.x] = r;
  }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

static int norm_nv(int64_t cols) {
  const int64_t need = (cols / 8 + 63) / 64;
  for (int nv : {1, 2, 3, 4, 6, 8, 12, 16})
    if (need <= nv) return nv;
  return 0;
}

#define FLW_NORM_KERNELS(K, B) \
  {reinterpret_cast<const void*>(&K<1, B>), reinterpret_cast<const void*>(&K<2, B>),  \
   reinterpret_cast<const void*>(&K<3, B>), reinterpret_cast<const void*>(&K<4, B>),  \
   reinterpret_cast<const void*>(&K<6, B>), reinterpret_cast<const void*>(&K<8, B>),  \
   reinterpret_cast<const void*>(&K<12, B>), reinterpret_cast<const void*>(&K<16, B>)}

static const void* pick_nv(const void* const* table, int nv) {
  switch (nv) {
    case 1: return table[0];
    case 2: return table[1];
    case 3: return table[2];
    case 4: return table[3];
    case 6: return table[4];
    case 8: return table[5];
    case 12: return table[6];
    default: return table[7];
  }
}

static int norm_check(const void* x, int64_t rows, int64_t cols, int64_t xs, const void* w, float eps) {
  FLW_REQUIRE(x != nullptr && w != nullptr, FLW_E_INVALID, "null pointer");
  FLW_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0, FLW_E_INVALID, "cols must be a positive multiple of 8");
  FLW_REQUIRE(cols <= 8192, FLW_E_UNSUPPORTED, "cols must be <= 8192, got %lld", (long long)cols);
  FLW_REQUIRE(xs >= cols && xs % 8 == 0 && aligned16(x) && aligned16(w), FLW_E_INVALID,
              "rows must be 16-byte aligned with a stride >= cols");
  FLW_REQUIRE(eps >= 0.0f, FLW_E_INVALID, "eps must be non-negative");
  FLW_REQUIRE(rows <= 0x7FFFFFFFll * 4, FLW_E_UNSUPPORTED, "too many rows");
  return FLW_OK;
}

static int swiglu_check(const void* g, const void* u, int64_t rows, int64_t cols, int64_t gs, int64_t us) {
  FLW_REQUIRE(g != nullptr && u != nullptr, FLW_E_INVALID, "null pointer");
  FLW_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0, FLW_E_INVALID, "cols must be a positive multiple of 8");
  FLW_REQUIRE(gs >= cols && us >= cols && gs % 8 == 0 && us % 8 == 0 && aligned16(g) && aligned16(u),
              FLW_E_INVALID, "rows must be 16-byte aligned with a stride >= cols");
  // the grid-stride index stays below 2^31 through its last step
  FLW_REQUIRE(rows * (cols / 8) <= 0x7FFFFFFFll - (int64_t)kSwigluBlocks * 256, FLW_E_UNSUPPORTED, "too many elements");
  return FLW_OK;
}

}  // namespace flw

using namespace flw;

static int rmsnorm_fwd_launch(const void* x, int64_t rows, int64_t cols, int64_t xs, const void* weight, float eps,
                              void* h, int64_t hs, const void* a, int64_t as, void* sum, int64_t ss, void* stream,
                              const char* name) {
  int rc = norm_check(x, rows, cols, xs, weight, eps);
  if (rc) return rc;
  FLW_REQUIRE(h != nullptr && aligned16(h) && hs >= cols && hs % 8 == 0, FLW_E_INVALID,
              "h must be 16-byte aligned rows with a stride >= cols");
  if (a != nullptr)
    FLW_REQUIRE(sum != nullptr && aligned16(a) && aligned16(sum) && as >= cols && as % 8 == 0 && ss >= cols &&
                ss % 8 == 0, FLW_E_INVALID, "a and sum must be 16-byte aligned rows with strides >= cols");
  if (rows == 0) return FLW_OK;
  static const void* const plain[] = FLW_NORM_KERNELS(rmsnorm_fwd_kernel, false);
  static const void* const added[] = FLW_NORM_KERNELS(rmsnorm_fwd_kernel, true);
  const Timer tm = take_timer();
  (void)launch_args(pick_nv(a != nullptr ? added : plain, norm_nv(cols)), dim3((unsigned)((rows + 3) / 4)),
                    dim3(256), 0, static_cast<hipStream_t>(stream), tm.start, tm.stop,
                    static_cast<const uint16_t*>(x), rows, (int)cols, xs, static_cast<const uint16_t*>(weight), eps,
                    static_cast<uint16_t*>(h), hs, static_cast<const uint16_t*>(a), as, static_cast<uint16_t*>(sum),
                    ss);
  return check_launch(name);
}

extern "C" int flw_rmsnorm_fwd(const void* x, int64_t rows, int64_t cols, int64_t x_row_stride, const void* weight,
                               float eps, void* h, int64_t h_row_stride, void* stream) {
  return rmsnorm_fwd_launch(x, rows, cols, x_row_stride, weight, eps, h, h_row_stride, nullptr, 0, nullptr, 0,
                            stream, "flw_rmsnorm_fwd");
}

extern "C" int flw_add_rmsnorm_fwd(const void* x, const void* a, int64_t rows, int64_t cols, int64_t x_row_stride,
                                   int64_t a_row_stride, const void* weight, float eps, void* sum,
                                   int64_t sum_row_stride, void* h, int64_t h_row_stride, void* stream) {
  FLW_REQUIRE(a != nullptr && sum != nullptr, FLW_E_INVALID, "null pointer");
  return rmsnorm_fwd_launch(x, rows, cols, x_row_stride, weight, eps, h, h_row_stride, a, a_row_stride, sum,
                            sum_row_stride, stream, "flw_add_rmsnorm_fwd");
}

extern "C" size_t flw_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols) {
  const int64_t nblk = rows <= 0 ? 0 : std::min<int64_t>((rows + 3) / 4, kNormBlocks);
  return (size_t)(nblk * (cols > 0 ? cols : 0) * 4);
}

extern "C" int flw_rmsnorm_bwd(const void* x, int64_t rows, int64_t cols, int64_t x_row_stride, const void* weight,
                               float eps, const void* dh, int64_t dh_row_stride, const void* dres,
                               int64_t dres_row_stride, void* dx, int64_t dx_row_stride, void* dweight,
                               void* workspace, size_t workspace_bytes, void* stream) {
  int rc = norm_check(x, rows, cols, x_row_stride, weight, eps);
  if (rc) return rc;
  FLW_REQUIRE(dh != nullptr && dx != nullptr && dweight != nullptr && aligned16(dh) && aligned16(dx),
              FLW_E_INVALID, "dh, dx must be 16-byte aligned and dweight non-null");
  FLW_REQUIRE(dh_row_stride >= cols && dh_row_stride % 8 == 0 && dx_row_stride >= cols && dx_row_stride % 8 == 0,
              FLW_E_INVALID, "gradient rows need a stride >= cols, a multiple of 8");
  if (dres != nullptr)
    FLW_REQUIRE(aligned16(dres) && dres_row_stride >= cols && dres_row_stride % 8 == 0, FLW_E_INVALID,
                "dres must be 16-byte aligned rows with a stride >= cols");
  const size_t need = flw_rmsnorm_bwd_workspace_bytes(rows, cols);
  FLW_REQUIRE(workspace_bytes >= need && (need == 0 || (workspace != nullptr && aligned16(workspace))),
              FLW_E_INVALID, "workspace needs %zu bytes (16-byte aligned), got %zu", need, workspace_bytes);
  const int nblk = (int)std::min<int64_t>((rows + 3) / 4, kNormBlocks);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const Timer tm = take_timer();
  float* part = static_cast<float*>(workspace);
  if (nblk > 0) {
    static const void* const plain[] = FLW_NORM_KERNELS(rmsnorm_bwd_kernel, false);
    static const void* const withres[] = FLW_NORM_KERNELS(rmsnorm_bwd_kernel, true);
    (void)launch_args(pick_nv(dres != nullptr ? withres : plain, norm_nv(cols)), dim3((unsigned)nblk), dim3(256),
                      (size_t)(cols * 4), s, tm.start, nullptr, static_cast<const uint16_t*>(x), rows, (int)cols,
                      x_row_stride, static_cast<const uint16_t*>(weight), eps, static_cast<const uint16_t*>(dh),
                      dh_row_stride, static_cast<uint16_t*>(dx), dx_row_stride, part,
                      static_cast<const uint16_t*>(dres), dres_row_stride);
  }
  (void)launch_args(reinterpret_cast<const void*>(&rmsnorm_dw_kernel), dim3((unsigned)((cols + 15) / 16)),
                    dim3(256), 0, s, nblk > 0 ? nullptr : tm.start, tm.stop, static_cast<const float*>(part), nblk,
                    (int)cols, static_cast<uint16_t*>(dweight));
  return check_launch("flw_rmsnorm_bwd");
}

static int swiglu_blocks(int64_t rows, int64_t cols) {
  const int64_t total = rows * (cols / 8);
  return (int)std::min<int64_t>((total + 255) / 256, kSwigluBlocks);
}

extern "C" size_t flw_swiglu_amax_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return (size_t)(2 * swiglu_blocks(rows, cols) * 4);
}

// Launches `kernel` (the AMAX instance when amax_out is given, then the fold of its partials into
// amax_out[0 .. nout - 1]).
static int swiglu_launch(SwigluParams& p, const void* plain, const void* with_amax, int nout, uint32_t* amax_out,
                         void* ws, size_t ws_bytes, int64_t rows, int64_t cols, void* stream, const char* name) {
  const int blocks = swiglu_blocks(rows, cols);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (amax_out == nullptr) {
    (void)launch_timed(plain, dim3((unsigned)blocks), dim3(256), s, p);
    return check_launch(name);
  }
  const size_t need = flw_swiglu_amax_workspace_bytes(rows, cols);
  FLW_REQUIRE(ws != nullptr && aligned16(ws) && ws_bytes >= need, FLW_E_WORKSPACE,
              "workspace needs %zu bytes (16-byte aligned)", need);
  p.part = static_cast<uint32_t*>(ws);
  const Timer tm = take_timer();
  (void)launch_ext(with_amax, dim3((unsigned)blocks), dim3(256), 0, s, p, tm.start, nullptr);
  (void)launch_args(reinterpret_cast<const void*>(&fold_max_kernel), dim3((unsigned)nout), dim3(1024), 0, s,
                    nullptr, tm.stop, static_cast<const uint32_t*>(p.part), blocks, amax_out);
  return check_launch(name);
}

extern "C" int flw_swiglu_fwd(const void* gate, const void* up, int64_t rows, int64_t cols, int64_t gate_row_stride,
                              int64_t up_row_stride, void* h, int64_t h_row_stride, uint32_t* h_amax,
                              void* workspace, size_t workspace_bytes, void* stream) {
  int rc = swiglu_check(gate, up, rows, cols, gate_row_stride, up_row_stride);
  if (rc) return rc;
  FLW_REQUIRE(h != nullptr && aligned16(h) && h_row_stride >= cols && h_row_stride % 8 == 0, FLW_E_INVALID,
              "h must be 16-byte aligned rows with a stride >= cols");
  if (rows == 0) {
    FLW_REQUIRE(h_amax == nullptr, FLW_E_INVALID, "no amax of an empty matrix");
    return FLW_OK;
  }
  SwigluParams p{};
  p.g = static_cast<const uint16_t*>(gate); p.u = static_cast<const uint16_t*>(up);
  p.out0 = static_cast<uint16_t*>(h);
  p.gs = gate_row_stride; p.us = up_row_stride; p.os = h_row_stride;
  p.cpr = (int)(cols / 8); p.total = (int)(rows * p.cpr);
  return swiglu_launch(p, reinterpret_cast<const void*>(&swiglu_fwd_kernel<false>),
                       reinterpret_cast<const void*>(&swiglu_fwd_kernel<true>), 1, h_amax, workspace,
                       workspace_bytes, rows, cols, stream, "flw_swiglu_fwd");
}

extern "C" int flw_swiglu_bwd(const void* gate, const void* up, int64_t rows, int64_t cols, int64_t gate_row_stride,
                              int64_t up_row_stride, const void* dh, int64_t dh_row_stride, void* dgate, void* dup,
                              int64_t grad_row_stride, uint32_t* grad_amax, void* workspace, size_t workspace_bytes,
                              void* stream) {
  int rc = swiglu_check(gate, up, rows, cols, gate_row_stride, up_row_stride);
  if (rc) return rc;
  FLW_REQUIRE(dh != nullptr && dgate != nullptr && dup != nullptr && aligned16(dh) && aligned16(dgate) &&
              aligned16(dup), FLW_E_INVALID, "dh, dgate, dup must be non-null and 16-byte aligned");
  FLW_REQUIRE(dh_row_stride >= cols && dh_row_stride % 8 == 0 && grad_row_stride >= cols && grad_row_stride % 8 == 0,
              FLW_E_INVALID, "gradient rows need a stride >= cols, a multiple of 8");
  if (rows == 0) {
    FLW_REQUIRE(grad_amax == nullptr, FLW_E_INVALID, "no amax of an empty matrix");
    return FLW_OK;
  }
  SwigluParams p{};
  p.g = static_cast<const uint16_t*>(gate); p.u = static_cast<const uint16_t*>(up);
  p.dh = static_cast<const uint16_t*>(dh);
  p.out0 = static_cast<uint16_t*>(dgate); p.out1 = static_cast<uint16_t*>(dup);
  p.gs = gate_row_stride; p.us = up_row_stride; p.dhs = dh_row_stride; p.os = grad_row_stride;
  p.cpr = (int)(cols / 8); p.total = (int)(rows * p.cpr);
  return swiglu_launch(p, reinterpret_cast<const void*>(&swiglu_bwd_kernel<false>),
                       reinterpret_cast<const void*>(&swiglu_bwd_kernel<true>), 2, grad_amax, workspace,
                       workspace_bytes, rows, cols, stream, "flw_swiglu_bwd");
}
