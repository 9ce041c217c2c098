// e4m3 quantisers (HBM-bound): amax partials -> quantise, and the per-row quantiser.
//
// A (B, H, T, D) tensor is handled as B*H slices of T rows x D contiguous elements. Pass 1
// (amax_partial_kernel) reduces |x| over chunks of kRowsPerChunk rows of one slice into a
// partials array; pass 2 (quant_kernel) lets every workgroup fold the partials of its scale group
// (whole tensor / head / slice) itself -- no atomics, no zero-initialised buffer, no host sync --
// then quantises its chunk. Chunks are processed one tensor at a time, so on MI355X the second
// read of a 64 MiB Q/K/V tensor is served largely from the 256 MB Infinity Cache.
#include "flw_common.h"

namespace flw {

constexpr int kThreads = 256;
constexpr int64_t kRowsPerChunk = 256;   // multiple of 64: VTILE chunks hold whole key tiles

struct SliceParams {
  const void* x;
  int64_t d0, d1, d2, d3;      // B, H, T, D
  int64_t s0, s1, s2;          // element strides of b, h, t
  int64_t nchunks;             // chunks per slice
  uint32_t* partials;          // [d0*d1*nchunks] |x| max bit patterns
  int granularity;
  uint8_t* out8;               // codes (BHTD or VTILE)
  void* outx;                  // fake-quant output (input dtype, contiguous BHTD)
  float* scale_out;            // 1 | d1 | d0*d1
};

__device__ __forceinline__ uint32_t block_max_u32(uint32_t m, uint32_t* lds4) {
  m = wave_max_u32(m);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) lds4[wave] = m;
  __syncthreads();
  uint32_t r = lds4[0];
#pragma unroll
  for (int i = 1; i < kThreads / 64; ++i) r = r > lds4[i] ? r : lds4[i];
  return r;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void amax_partial_kernel(SliceParams p) {
  using V = Vec16<T>;
  __shared__ uint32_t red[kThreads / 64];
  const int64_t slice = blockIdx.y;
  const int64_t i0 = slice / p.d1, i1 = slice % p.d1;
  const int64_t r0 = (int64_t)blockIdx.x * kRowsPerChunk;
  const int64_t r1 = min(p.d2, r0 + kRowsPerChunk);
  const T* base = static_cast<const T*>(p.x) + i0 * p.s0 + i1 * p.s1;
  const int64_t vpr = p.d3 / V::N;
  const int64_t nvec = (r1 - r0) * vpr;
  uint32_t m = 0;
  for (int64_t v = threadIdx.x; v < nvec; v += kThreads) {
    const int64_t row = r0 + v / vpr, cv = v % vpr;
    float f[V::N];
    V::load(base + row * p.s2 + cv * V::N, f);
#pragma unroll
    for (int i = 0; i < V::N; ++i) { uint32_t a = abs_bits(f[i]); m = m > a ? m : a; }
  }
  m = block_max_u32(m, red);
  if (threadIdx.x == 0) p.partials[slice * p.nchunks + blockIdx.x] = m;
}

// Fold the partials of this workgroup's scale group.
__device__ __forceinline__ uint32_t group_amax(const SliceParams& p, int64_t slice, int64_t i1,
                                               uint32_t* red) {
  uint32_t m = 0;
  if (p.granularity == FLW_SCALE_TENSOR) {
    const int64_t n = p.d0 * p.d1 * p.nchunks;
    for (int64_t i = threadIdx.x; i < n; i += kThreads) { uint32_t a = p.partials[i]; m = m > a ? m : a; }
  } else if (p.granularity == FLW_SCALE_HEAD) {
    const int64_t n = p.d0 * p.nchunks;
    for (int64_t i = threadIdx.x; i < n; i += kThreads) {
      const int64_t b = i / p.nchunks, c = i % p.nchunks;
      uint32_t a = p.partials[(b * p.d1 + i1) * p.nchunks + c];
      m = m > a ? m : a;
    }
  } else {
    for (int64_t i = threadIdx.x; i < p.nchunks; i += kThreads) {
      uint32_t a = p.partials[slice * p.nchunks + i];
      m = m > a ? m : a;
    }
  }
  return block_max_u32(m, red);
}

__device__ __forceinline__ int64_t group_index(const SliceParams& p, int64_t slice, int64_t i1) {
  return p.granularity == FLW_SCALE_TENSOR ? 0 : (p.granularity == FLW_SCALE_HEAD ? i1 : slice);
}

__device__ __forceinline__ bool writes_scale(const SliceParams& p, int64_t slice, int64_t i0) {
  if (blockIdx.x != 0 || threadIdx.x != 0) return false;
  if (p.granularity == FLW_SCALE_TENSOR) return slice == 0;
  if (p.granularity == FLW_SCALE_HEAD) return i0 == 0;
  return true;
}

__device__ __forceinline__ float clamp448(float y) {
  // torch.clamp semantics: NaN stays NaN (both comparisons are false)
  y = y > kE4m3Max ? kE4m3Max : y;
  return y < -kE4m3Max ? -kE4m3Max : y;
}

// Byte offset of element (key kk, dim d) inside a 64 x D VTILE tile.
__device__ __forceinline__ uint32_t vtile_offset(uint32_t kk, uint32_t d) {
  const uint32_t r = kk & 31u;
  const uint32_t h = (r >> 2) & 1u;
  const uint32_t b = ((r >> 3) << 2) | (r & 3u);
  return (d >> 5) * 2048u + (kk >> 5) * 1024u + ((d & 31u) + 32u * h) * 16u + b;
}

// MODE 0: e4m3 codes with the _per_tensor_fp8 recipe. MODE 1: _fake_quant_e4m3 forward value.
template <typename T, int LAYOUT, int MODE>
__global__ __launch_bounds__(kThreads) void quant_kernel(SliceParams p) {
  using V = Vec16<T>;
  constexpr bool kBf16 = sizeof(T) == 2;
  __shared__ uint32_t red[kThreads / 64];
  extern __shared__ __align__(16) uint8_t tile_lds[];   // VTILE staging: kRowsPerChunk x D
  const int64_t slice = blockIdx.y;
  const int64_t i0 = slice / p.d1, i1 = slice % p.d1;

  const float amax = __uint_as_float(group_amax(p, slice, i1, red));
  float scale;
  if (MODE == 1 && kBf16) {
    // base.py:198-199 under bf16: clamp and /448 are bf16 tensor ops
    const float eps_b = round_bf16(kEps);
    scale = round_bf16((amax < eps_b ? eps_b : amax) / kE4m3Max);
  } else {
    scale = (amax < kEps ? kEps : amax) / kE4m3Max;     // IEEE fp32 division
  }
  if (writes_scale(p, slice, i0)) p.scale_out[group_index(p, slice, i1)] = scale;

  const int64_t r0 = (int64_t)blockIdx.x * kRowsPerChunk;
  const int64_t r1 = min(p.d2, r0 + kRowsPerChunk);
  // VTILE: cover whole 64-row tiles, padding rows past T become code 0.
  const int64_t r1p = LAYOUT == FLW_LAYOUT_VTILE ? min(r0 + kRowsPerChunk, (p.d2 + 63) & ~int64_t(63)) : r1;
  const T* base = static_cast<const T*>(p.x) + i0 * p.s0 + i1 * p.s1;
  const int64_t vpr = p.d3 / V::N;
  const int64_t nvec = (r1p - r0) * vpr;

  for (int64_t v = threadIdx.x; v < nvec; v += kThreads) {
    const int64_t row = r0 + v / vpr, cv = v % vpr;
    float f[V::N];
    if (row < p.d2) {
      V::load(base + row * p.s2 + cv * V::N, f);
    } else {
#pragma unroll
      for (int i = 0; i < V::N; ++i) f[i] = 0.0f;
    }
    uint32_t codes[V::N];
#pragma unroll
    for (int i = 0; i < V::N; ++i) {
      float y = f[i] / scale;                      // IEEE division, as the reference's CPU path
      if (MODE == 1 && kBf16) y = round_bf16(y);
      codes[i] = f32_to_e4m3(clamp448(y)) & 0xFFu;
      if (row >= p.d2) codes[i] = 0;
    }
    if (MODE == 0) {
      if (LAYOUT == FLW_LAYOUT_BHTD) {
        uint8_t* dst = p.out8 + (slice * p.d2 + row) * p.d3 + cv * V::N;
        if (V::N == 8) {
          uint2 w;
          w.x = codes[0] | (codes[1] << 8) | (codes[2] << 16) | (codes[3] << 24);
          w.y = codes[4] | (codes[5] << 8) | (codes[6] << 16) | (codes[7] << 24);
          *reinterpret_cast<uint2*>(dst) = w;
        } else {
          *reinterpret_cast<uint32_t*>(dst) =
              codes[0] | (codes[1] << 8) | (codes[2] << 16) | (codes[3] << 24);
        }
      } else {
        const uint32_t lrow = (uint32_t)(row - r0);
        uint8_t* t = tile_lds + (lrow >> 6) * (64u * (uint32_t)p.d3);
#pragma unroll
        for (int i = 0; i < V::N; ++i)
          t[vtile_offset(lrow & 63u, (uint32_t)(cv * V::N + i))] = (uint8_t)codes[i];
      }
    } else {
      // out = x + (dq - x), each step rounded to T (base.py:200-203)
      float o[V::N];
#pragma unroll
      for (int i = 0; i < V::N; ++i) {
        float dq = e4m3_to_f32(codes[i] | 0u) * scale;
        if (kBf16) dq = round_bf16(dq);
        float d = dq - f[i];
        if (kBf16) d = round_bf16(d);
        o[i] = f[i] + d;
      }
      T* dst = static_cast<T*>(p.outx) + (slice * p.d2 + row) * p.d3 + cv * V::N;
      if (kBf16) {
        uint4 w;
        w.x = f32_to_bf16_bits(o[0]) | (f32_to_bf16_bits(o[1]) << 16);
        w.y = f32_to_bf16_bits(o[2]) | (f32_to_bf16_bits(o[3]) << 16);
        w.z = f32_to_bf16_bits(o[4]) | (f32_to_bf16_bits(o[5]) << 16);
        w.w = f32_to_bf16_bits(o[6]) | (f32_to_bf16_bits(o[7]) << 16);
        *reinterpret_cast<uint4*>(dst) = w;
      } else {
        *reinterpret_cast<float4*>(dst) = make_float4(o[0], o[1], o[2], o[3]);
      }
    }
  }
  if (LAYOUT == FLW_LAYOUT_VTILE && MODE == 0) {
    __syncthreads();
    const int64_t ntiles = (p.d2 + 63) >> 6;
    const int64_t nbytes = (r1p - r0) * p.d3;
    uint8_t* dst = p.out8 + (slice * ntiles + (r0 >> 6)) * 64 * p.d3;
    for (int64_t o = threadIdx.x * 16; o < nbytes; o += kThreads * 16)
      *reinterpret_cast<uint4*>(dst + o) = *reinterpret_cast<const uint4*>(tile_lds + o);
  }
}

// One wave per row: amax, scale = max(amax / 448, 1e-12), codes = e4m3(x / scale).
template <typename T>
__global__ __launch_bounds__(kThreads) void rows_quant_kernel(const T* __restrict__ x, int64_t rows,
                                                              int64_t cols, int64_t rs,
                                                              uint8_t* __restrict__ out,
                                                              float* __restrict__ scale_out) {
  using V = Vec16<T>;
  const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;            // wave-uniform
  const int lane = threadIdx.x & 63;
  const T* src = x + row * rs;
  const int64_t nvec = cols / V::N;
  uint32_t m = 0;
  for (int64_t v = lane; v < nvec; v += 64) {
    float f[V::N];
    V::load(src + v * V::N, f);
#pragma unroll
    for (int i = 0; i < V::N; ++i) { uint32_t a = abs_bits(f[i]); m = m > a ? m : a; }
  }
  m = wave_max_u32(m);
  float s = __uint_as_float(m) / kE4m3Max;
  s = s < kEps ? kEps : s;
  if (lane == 0) scale_out[row] = s;
  uint8_t* dst = out + row * cols;
  for (int64_t v = lane; v < nvec; v += 64) {
    float f[V::N];
    V::load(src + v * V::N, f);
    uint32_t c[V::N];
#pragma unroll
    for (int i = 0; i < V::N; ++i) c[i] = f32_to_e4m3(f[i] / s) & 0xFFu;
    if (V::N == 8) {
      uint2 w;
      w.x = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
      w.y = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
      *reinterpret_cast<uint2*>(dst + v * 8) = w;
    } else {
      *reinterpret_cast<uint32_t*>(dst + v * 4) = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
    }
  }
}

// ---------------------------------------------------------------- host side

static int64_t nchunks_of(int64_t T) { return (T + kRowsPerChunk - 1) / kRowsPerChunk; }

static int check_tensor(const void* x, int dtype, int64_t B, int64_t H, int64_t T, int64_t D,
                        int64_t sb, int64_t sh, int64_t st) {
  FLW_REQUIRE(x != nullptr, FLW_E_INVALID, "null input pointer");
  FLW_REQUIRE(dtype == FLW_F32 || dtype == FLW_BF16, FLW_E_UNSUPPORTED, "dtype %d not supported (f32=0, bf16=1)", dtype);
  FLW_REQUIRE(B > 0 && H > 0 && T > 0 && D > 0, FLW_E_INVALID, "empty or negative shape (%lld,%lld,%lld,%lld)",
              (long long)B, (long long)H, (long long)T, (long long)D);
  const int64_t vec = dtype == FLW_F32 ? 4 : 8;
  FLW_REQUIRE(D % vec == 0, FLW_E_UNSUPPORTED, "last dim %lld must be a multiple of %lld", (long long)D, (long long)vec);
  FLW_REQUIRE(sb % vec == 0 && sh % vec == 0 && st % vec == 0, FLW_E_INVALID,
              "strides must be multiples of %lld elements (16-byte rows)", (long long)vec);
  FLW_REQUIRE(((uintptr_t)x & 15) == 0, FLW_E_INVALID, "input must be 16-byte aligned");
  FLW_REQUIRE(B * H <= 65535 && nchunks_of(T) <= 0x7FFFFFFF, FLW_E_UNSUPPORTED, "B*H must be <= 65535");
  return FLW_OK;
}

static size_t partial_bytes(int64_t B, int64_t H, int64_t T) {
  return (size_t)(B * H * nchunks_of(T)) * sizeof(uint32_t);
}

template <int LAYOUT, int MODE>
static int launch_slice(const SliceParams& p, int dtype, hipStream_t s, const char* name) {
  dim3 grid((unsigned)p.nchunks, (unsigned)(p.d0 * p.d1));
  size_t lds = LAYOUT == FLW_LAYOUT_VTILE ? (size_t)(kRowsPerChunk * p.d3) : 0;
  if (dtype == FLW_F32) {
    hipLaunchKernelGGL(amax_partial_kernel<float>, grid, dim3(kThreads), 0, s, p);
    hipLaunchKernelGGL((quant_kernel<float, LAYOUT, MODE>), grid, dim3(kThreads), lds, s, p);
  } else {
    hipLaunchKernelGGL(amax_partial_kernel<uint16_t>, grid, dim3(kThreads), 0, s, p);
    hipLaunchKernelGGL((quant_kernel<uint16_t, LAYOUT, MODE>), grid, dim3(kThreads), lds, s, p);
  }
  return check_launch(name);
}

int quant_bhtd(const void* x, int dtype, int64_t B, int64_t H, int64_t T, int64_t D, int64_t sb,
               int64_t sh, int64_t st, int granularity, int layout, uint8_t* out, float* scale_out,
               void* ws, size_t ws_bytes, hipStream_t stream) {
  int rc = check_tensor(x, dtype, B, H, T, D, sb, sh, st);
  if (rc) return rc;
  FLW_REQUIRE(granularity >= FLW_SCALE_TENSOR && granularity <= FLW_SCALE_BH, FLW_E_INVALID, "bad granularity %d", granularity);
  FLW_REQUIRE(layout == FLW_LAYOUT_BHTD || layout == FLW_LAYOUT_VTILE, FLW_E_INVALID, "bad layout %d", layout);
  FLW_REQUIRE(out != nullptr && scale_out != nullptr, FLW_E_INVALID, "null output pointer");
  FLW_REQUIRE(ws != nullptr && ws_bytes >= partial_bytes(B, H, T), FLW_E_WORKSPACE,
              "workspace needs %zu bytes", partial_bytes(B, H, T));
  if (layout == FLW_LAYOUT_VTILE) {
    FLW_REQUIRE(D == 32 || D == 64 || D == 128, FLW_E_UNSUPPORTED, "VTILE layout needs D in {32, 64, 128}");
    FLW_REQUIRE(((uintptr_t)out & 15) == 0, FLW_E_INVALID, "VTILE output must be 16-byte aligned");
  } else {
    FLW_REQUIRE(((uintptr_t)out & 7) == 0, FLW_E_INVALID, "output must be 8-byte aligned");
  }
  SliceParams p{};
  p.x = x; p.d0 = B; p.d1 = H; p.d2 = T; p.d3 = D; p.s0 = sb; p.s1 = sh; p.s2 = st;
  p.nchunks = nchunks_of(T); p.partials = static_cast<uint32_t*>(ws); p.granularity = granularity;
  p.out8 = out; p.scale_out = scale_out;
  if (layout == FLW_LAYOUT_BHTD) return launch_slice<FLW_LAYOUT_BHTD, 0>(p, dtype, stream, "flw_quant_e4m3");
  return launch_slice<FLW_LAYOUT_VTILE, 0>(p, dtype, stream, "flw_quant_e4m3(vtile)");
}

}  // namespace flw

using namespace flw;

extern "C" size_t flw_quant_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D) {
  (void)D;
  return partial_bytes(B, H, T);
}

extern "C" size_t flw_vtile_bytes(int64_t B, int64_t H, int64_t T, int64_t D) {
  return (size_t)(B * H * ((T + 63) / 64) * 64 * D);
}

extern "C" int flw_quant_e4m3(const void* x, int dtype, int64_t B, int64_t H, int64_t T, int64_t D,
                              int64_t stride_b, int64_t stride_h, int64_t stride_t, int granularity,
                              int layout, uint8_t* out, float* scale_out, void* workspace,
                              size_t workspace_bytes, void* stream) {
  return quant_bhtd(x, dtype, B, H, T, D, stride_b, stride_h, stride_t, granularity, layout, out,
                    scale_out, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int flw_fake_quant_e4m3(const void* x, int dtype, int64_t B, int64_t H, int64_t T,
                                   int64_t D, int64_t stride_b, int64_t stride_h, int64_t stride_t,
                                   int granularity, void* out, float* scale_out, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  int rc = check_tensor(x, dtype, B, H, T, D, stride_b, stride_h, stride_t);
  if (rc) return rc;
  FLW_REQUIRE(granularity >= FLW_SCALE_TENSOR && granularity <= FLW_SCALE_BH, FLW_E_INVALID, "bad granularity %d", granularity);
  FLW_REQUIRE(out != nullptr && ((uintptr_t)out & 15) == 0, FLW_E_INVALID, "output must be non-null and 16-byte aligned");
  FLW_REQUIRE(workspace != nullptr && workspace_bytes >= partial_bytes(B, H, T), FLW_E_WORKSPACE,
              "workspace needs %zu bytes", partial_bytes(B, H, T));
  SliceParams p{};
  p.x = x; p.d0 = B; p.d1 = H; p.d2 = T; p.d3 = D; p.s0 = stride_b; p.s1 = stride_h; p.s2 = stride_t;
  p.nchunks = nchunks_of(T); p.partials = static_cast<uint32_t*>(workspace); p.granularity = granularity;
  p.outx = out;
  p.scale_out = scale_out;
  if (scale_out == nullptr) {   // optional: park the scales in the tail of the workspace
    const size_t need = partial_bytes(B, H, T) + sizeof(float) * (size_t)(B * H);
    FLW_REQUIRE(workspace_bytes >= need, FLW_E_WORKSPACE, "workspace needs %zu bytes without scale_out", need);
    p.scale_out = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + partial_bytes(B, H, T));
  }
  return launch_slice<FLW_LAYOUT_BHTD, 1>(p, dtype, static_cast<hipStream_t>(stream), "flw_fake_quant_e4m3");
}

extern "C" int flw_quant_rows_e4m3(const void* x, int dtype, int64_t rows, int64_t cols,
                                   int64_t row_stride, uint8_t* out, float* scale_out, void* stream) {
  FLW_REQUIRE(x != nullptr && out != nullptr && scale_out != nullptr, FLW_E_INVALID, "null pointer");
  FLW_REQUIRE(dtype == FLW_F32 || dtype == FLW_BF16, FLW_E_UNSUPPORTED, "dtype %d not supported", dtype);
  FLW_REQUIRE(rows > 0 && cols > 0, FLW_E_INVALID, "empty matrix");
  const int64_t vec = dtype == FLW_F32 ? 4 : 8;
  FLW_REQUIRE(cols % vec == 0 && row_stride % vec == 0 && ((uintptr_t)x & 15) == 0, FLW_E_INVALID,
              "rows must be 16-byte aligned multiples of %lld elements", (long long)vec);
  FLW_REQUIRE(((uintptr_t)out & 7) == 0 && (cols % 8 == 0 || dtype == FLW_F32), FLW_E_INVALID, "output must be 8-byte aligned");
  FLW_REQUIRE((rows + 3) / 4 <= 0x7FFFFFFF, FLW_E_UNSUPPORTED, "too many rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid((unsigned)((rows + 3) / 4));
  if (dtype == FLW_F32)
    hipLaunchKernelGGL(rows_quant_kernel<float>, grid, dim3(kThreads), 0, s,
                       static_cast<const float*>(x), rows, cols, row_stride, out, scale_out);
  else
    hipLaunchKernelGGL(rows_quant_kernel<uint16_t>, grid, dim3(kThreads), 0, s,
                       static_cast<const uint16_t*>(x), rows, cols, row_stride, out, scale_out);
  return check_launch("flw_quant_rows_e4m3");
}
