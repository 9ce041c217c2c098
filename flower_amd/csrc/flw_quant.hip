// e4m3 quantisers (HBM-bound): amax partials -> quantise, and the per-row quantiser.
//
// A (B, H, T, D) tensor is handled as B*H slices of T rows x D contiguous elements, cut into
// chunks of kRowsPerChunk rows. Pass 1 (amax_kernel) reduces |x| over each chunk into a partials
// array; pass 2 (quant_kernel) lets every workgroup fold the partials of its scale group (whole
// tensor / head / slice) itself -- no atomics, no zero-initialised buffer, no host sync -- then
// quantises its chunk. Up to three tensors of one shape (Q, K, V) go through each pass in ONE
// launch (grid.z = tensor), and every thread keeps kUnroll 16-byte loads in flight. The second
// read of each tensor is partly served by the MI355X Infinity Cache (256 MB); pass 2 walks the
// chunks in the reverse of pass 1's order to make the most of it.
//
// Rounding. The reference computes e4m3(clamp(x / s, -448, 448)) with an IEEE fp32 division
// and round-to-nearest-even. For a scale group whose amax is finite, every |x / s| is at most
// 448 (s = max(amax, eps) / 448), so the clamp is inert and the quotient goes through
//   q0 = x * r,  e = fma(-q0, s, x),  q = fma(e, r, q0)       with r = RN(1 / s)
// (the reciprocal-then-correct sequence of Markstein, correctly rounded when r is the correctly
// rounded reciprocal) and the hardware RNE converter v_cvt_pk_fp8_f32, two values per
// instruction. Both are checked bit for bit on the device against the exact division and the
// exact software rounding (the diagnostics library and its tests). A group whose amax is NaN or
// infinite takes the exact path (IEEE division, clamp, software rounding) so that NaN and inf
// propagate exactly as in the reference.
#include <mutex>

#include "flw_common.h"

namespace flw {

constexpr int kThreads = 256;
// Chunk height and loads in flight per thread, swept together (64-1024 rows x 1-16 loads): 128 x 1
// ties 256 x 2 on the large shapes and is faster on small ones (more workgroups to spread).
constexpr int64_t kRowsPerChunk = 128;   // multiple of 64: VTILE chunks hold whole key tiles
constexpr int kUnroll = 1;               // 16-byte loads in flight per thread per iteration
// The amax pass without a transform keeps 4 loads in flight per thread: with chunks of wide rows
// (the tensorwise flat grid) a thread walks many vectors, and the max folds in any order.
constexpr int kAmaxUnroll = 4;

struct QTensor {
  const void* x;
  int64_t s0, s1, s2;          // element strides of b, h, t
  uint8_t* out8;               // codes (BHTD or VTILE)
  void* outx;                  // fake-quant output (input dtype, contiguous BHTD)
  float* scale_out;            // 1 | d1 | d0*d1
  int layout;
  int rows_packed;             // s2 == D: a chunk is one contiguous run of memory
  // Optional transform applied before the amax and the codes (XFORM kernels only): the
  // HeadRMSNorm and RoPE of CausalSelfAttention.qkv_heads, with the transformed values also
  // written to tout (contiguous (B, H, T, D), input dtype) when it is not null.
  int norm;                    // HeadRMSNorm over each row of D
  float eps;
  const void* rcos;            // RoPE tables [T, D] in the input dtype, or null
  const void* rsin;
  void* tout;
  // Deferred codes (the attention kernel quantises this tensor on load): the scale and its
  // reciprocal RN(1 / scale) (to rcp_out) are written, and codes only for scale groups whose amax
  // is not finite (the exact path, which the attention kernel leaves to this kernel).
  int defer;
  float* rcp_out;
};

struct QuantParams {
  QTensor t[3];
  int64_t d0, d1, d2, d3;      // B, H, T, D
  int64_t nchunks;             // chunks per slice
  uint32_t* partials;          // [tensor][d0*d1][nchunks] |x| max bit patterns
  int granularity;
  const uint32_t* amax_given;  // optional [tensor][groups] |x| max bit patterns (no amax pass)
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

// Element offset of the 16-byte vector v of chunk rows [r0, ...) inside a slice.
__device__ __forceinline__ int64_t vec_offset(const QTensor& t, int64_t r0, int64_t v, int64_t vpr,
                                              int n, int64_t d3) {
  if (t.rows_packed) return r0 * d3 + v * n;
  const int64_t row = r0 + v / vpr, cv = v % vpr;
  return row * t.s2 + cv * n;
}

// The pre-attention transform of CausalSelfAttention.qkv_heads on one 16-byte vector (column
// block cv of row `row` of a slice): head_norm_rope (flw_common.h) with the row's sum of squares
// reduced over the vpr lanes that hold the row. Every lane of a vpr group must call this together
// (valid or not: invalid lanes carry zeros and read no table).
template <typename T>
__device__ __forceinline__ void qk_transform(const QTensor& t, float* f, int64_t row, int64_t cv, int vpr,
                                             int64_t d3, bool valid) {
  constexpr int N = Vec16<T>::N;
  float c[N] = {}, sn[N] = {};
  const bool rope = t.rcos != nullptr && valid;
  if (rope) {
    const int64_t off = row * d3 + cv * N;
    Vec16<T>::load(static_cast<const T*>(t.rcos) + off, c);
    Vec16<T>::load(static_cast<const T*>(t.rsin) + off, sn);
  }
  head_norm_rope<T>(f, t.norm, t.eps, (int)d3, vpr, valid, t.rcos != nullptr, c, sn);
}

template <typename T, bool XFORM = false>
__global__ __launch_bounds__(kThreads) void amax_kernel(QuantParams p) {
  using V = Vec16<T>;
  __shared__ uint32_t red[kThreads / 64];
  const QTensor& t = p.t[blockIdx.z];
  const int64_t slice = blockIdx.y;
  const int64_t i0 = slice / p.d1, i1 = slice % p.d1;
  const int64_t r0 = (int64_t)blockIdx.x * kRowsPerChunk;
  const int64_t r1 = min(p.d2, r0 + kRowsPerChunk);
  const T* base = static_cast<const T*>(t.x) + i0 * t.s0 + i1 * t.s1;
  const int64_t vpr = p.d3 / V::N;
  const int64_t nvec = (r1 - r0) * vpr;
  constexpr int U = XFORM ? kUnroll : kAmaxUnroll;
  uint32_t m = 0;
  for (int64_t v0 = threadIdx.x; v0 < nvec; v0 += (int64_t)kThreads * U) {
    float f[U][V::N];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t v = v0 + (int64_t)u * kThreads;
      if (v < nvec) {
        V::load(base + vec_offset(t, r0, v, vpr, V::N, p.d3), f[u]);
      } else {
#pragma unroll
        for (int i = 0; i < V::N; ++i) f[u][i] = 0.0f;
      }
    }
    if (XFORM && (t.norm || t.rcos != nullptr)) {          // uniform over the workgroup
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t v = v0 + (int64_t)u * kThreads;
        qk_transform<T>(t, f[u], r0 + v / vpr, v % vpr, (int)vpr, p.d3, v < nvec);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < V::N; ++i) { const uint32_t a = abs_bits(f[u][i]); m = m > a ? m : a; }
  }
  m = block_max_u32(m, red);
  if (threadIdx.x == 0)
    p.partials[((int64_t)blockIdx.z * p.d0 * p.d1 + slice) * p.nchunks + blockIdx.x] = m;
}

// Fold the partials of this workgroup's scale group.
__device__ __forceinline__ uint32_t group_amax(const QuantParams& p, const uint32_t* part,
                                               int64_t slice, int64_t i1, uint32_t* red) {
  uint32_t m = 0;
  if (p.granularity == FLW_SCALE_TENSOR) {
    const int64_t n = p.d0 * p.d1 * p.nchunks;
    for (int64_t i = threadIdx.x; i < n; i += kThreads) { uint32_t a = part[i]; m = m > a ? m : a; }
  } else if (p.granularity == FLW_SCALE_HEAD) {
    const int64_t n = p.d0 * p.nchunks;
    for (int64_t i = threadIdx.x; i < n; i += kThreads) {
      const int64_t b = i / p.nchunks, c = i % p.nchunks;
      uint32_t a = part[(b * p.d1 + i1) * p.nchunks + c];
      m = m > a ? m : a;
    }
  } else {
    for (int64_t i = threadIdx.x; i < p.nchunks; i += kThreads) {
      uint32_t a = part[slice * p.nchunks + i];
      m = m > a ? m : a;
    }
  }
  return block_max_u32(m, red);
}

__device__ __forceinline__ int64_t group_index(int gran, int64_t slice, int64_t i1) {
  return gran == FLW_SCALE_TENSOR ? 0 : (gran == FLW_SCALE_HEAD ? i1 : slice);
}

__device__ __forceinline__ bool writes_scale(int gran, int64_t slice, int64_t i0) {
  if (blockIdx.x != 0 || threadIdx.x != 0) return false;
  if (gran == FLW_SCALE_TENSOR) return slice == 0;
  if (gran == FLW_SCALE_HEAD) return i0 == 0;
  return true;
}

__device__ __forceinline__ float clamp448(float y) {
  // torch.clamp semantics: NaN stays NaN (both comparisons are false)
  y = y > kE4m3Max ? kE4m3Max : y;
  return y < -kE4m3Max ? -kE4m3Max : y;
}


// e4m3 codes of N values, packed little-endian (N = 4 or 8), on the fast or the exact path.
template <int N>
__device__ __forceinline__ void codes_of(const float* f, float s, float r, bool fast, uint32_t* w) {
  if (fast) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      int c = __builtin_amdgcn_cvt_pk_fp8_f32(div_by_scale(f[4 * i], s, r),
                                              div_by_scale(f[4 * i + 1], s, r), 0, false);
      c = __builtin_amdgcn_cvt_pk_fp8_f32(div_by_scale(f[4 * i + 2], s, r),
                                          div_by_scale(f[4 * i + 3], s, r), c, true);
      w[i] = (uint32_t)c;
    }
  } else {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      uint32_t c = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        c |= (f32_to_e4m3(clamp448(f[4 * i + j] / s)) & 0xFFu) << (8 * j);   // IEEE division
      w[i] = c;
    }
  }
}

// MODE 0: e4m3 codes with the _per_tensor_fp8 recipe. MODE 1: _fake_quant_e4m3 forward value.
// XFORM: the q / k transform of qk_transform first (MODE 0 only).
template <typename T, int MODE, bool XFORM = false>
__global__ __launch_bounds__(kThreads) void quant_kernel(QuantParams p) {
  using V = Vec16<T>;
  constexpr bool kBf16 = sizeof(T) == 2;
  __shared__ uint32_t red[kThreads / 64];
  extern __shared__ __align__(16) uint8_t tile_lds[];   // VTILE staging: kRowsPerChunk x D
  // Blocks walk the tensors in the reverse of amax_kernel's order, so the first chunks quantised
  // are the ones the amax pass read last and that are most likely still in the Infinity Cache.
  const int zi = (int)(gridDim.z - 1 - blockIdx.z);
  const int64_t slice = (int64_t)(gridDim.y - 1 - blockIdx.y);
  const int64_t bx = (int64_t)(gridDim.x - 1 - blockIdx.x);
  const QTensor& t = p.t[zi];
  const int64_t i0 = slice / p.d1, i1 = slice % p.d1;
  const uint32_t* part = p.partials + (int64_t)zi * p.d0 * p.d1 * p.nchunks;

  const int64_t ngroups = p.granularity == FLW_SCALE_TENSOR ? 1 : (p.granularity == FLW_SCALE_HEAD ? p.d1 : p.d0 * p.d1);
  const float amax = p.amax_given
      ? __uint_as_float(p.amax_given[zi * ngroups + group_index(p.granularity, slice, i1)])
      : __uint_as_float(group_amax(p, part, slice, i1, red));
  float scale;
  if (MODE == 1 && kBf16) {
    // base.py:198-199 under bf16: clamp and /448 are bf16 tensor ops
    const float eps_b = round_bf16(kEps);
    scale = round_bf16((amax < eps_b ? eps_b : amax) / kE4m3Max);
  } else {
    scale = (amax < kEps ? kEps : amax) / kE4m3Max;     // IEEE fp32 division
  }
  const bool fast = MODE == 0 && __builtin_isfinite(amax);   // uniform over the workgroup
  const float rcp = 1.0f / scale;                            // IEEE: correctly rounded
  if (writes_scale(p.granularity, slice, i0)) {
    t.scale_out[group_index(p.granularity, slice, i1)] = scale;
    if (MODE == 0 && t.rcp_out != nullptr) t.rcp_out[group_index(p.granularity, slice, i1)] = rcp;
  }
  if (MODE == 0 && t.defer && fast) return;                  // codes made by the attention kernel
  // A given amax is the caller's claim about the data (a producer's epilogue maximum, or a
  // maximum combined across shards). The fast path relies on |x| <= amax (then |x / s| <= 448
  // and the clamp is inert), so with a given amax every vector is checked against it, and a
  // vector holding a larger |x|, an inf or a NaN takes the exact path (IEEE division, clamp,
  // software rounding): the reference's clamp(x / s, -448, 448) then the cast, whatever amax
  // was given. A negative amax admits no value to the fast path.
  const bool check_given = p.amax_given != nullptr;
  const uint32_t given_bits = amax > 0.0f ? __float_as_uint(amax) : 0u;

  const int64_t r0 = bx * kRowsPerChunk;
  const int64_t r1 = min(p.d2, r0 + kRowsPerChunk);
  const bool vtile = MODE == 0 && t.layout == FLW_LAYOUT_VTILE;
  // VTILE: cover whole 64-row tiles, padding rows past T become code 0.
  const int64_t r1p = vtile ? min(r0 + kRowsPerChunk, (p.d2 + 63) & ~int64_t(63)) : r1;
  const T* base = static_cast<const T*>(t.x) + i0 * t.s0 + i1 * t.s1;
  const int64_t vpr = p.d3 / V::N;
  const int64_t nvec = (r1 - r0) * vpr;        // vectors of real rows
  const int64_t nvec_p = (r1p - r0) * vpr;     // including VTILE padding rows

  for (int64_t v0 = threadIdx.x; v0 < nvec_p; v0 += (int64_t)kThreads * kUnroll) {
    float f[kUnroll][V::N];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t v = v0 + (int64_t)u * kThreads;
      if (v < nvec) {
        V::load(base + vec_offset(t, r0, v, vpr, V::N, p.d3), f[u]);
      } else {
#pragma unroll
        for (int i = 0; i < V::N; ++i) f[u][i] = 0.0f;
      }
    }
    if (XFORM && (t.norm || t.rcos != nullptr)) {          // uniform over the workgroup
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int64_t v = v0 + (int64_t)u * kThreads;
        qk_transform<T>(t, f[u], r0 + v / vpr, v % vpr, (int)vpr, p.d3, v < nvec);
        if (t.tout != nullptr && v < nvec) {
          T* dst = static_cast<T*>(t.tout) + (slice * p.d2 + r0) * p.d3 + v * V::N;
          if constexpr (sizeof(T) == 2) {
            *reinterpret_cast<uint4*>(dst) = make_uint4(
                f32_to_bf16_bits(f[u][0]) | (f32_to_bf16_bits(f[u][1]) << 16),
                f32_to_bf16_bits(f[u][2]) | (f32_to_bf16_bits(f[u][3]) << 16),
                f32_to_bf16_bits(f[u][4]) | (f32_to_bf16_bits(f[u][5]) << 16),
                f32_to_bf16_bits(f[u][6]) | (f32_to_bf16_bits(f[u][7]) << 16));
          } else {
            *reinterpret_cast<float4*>(dst) = make_float4(f[u][0], f[u][1], f[u][2], f[u][3]);
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t v = v0 + (int64_t)u * kThreads;
      if (v >= nvec_p) continue;
      if (MODE == 0) {
        uint32_t w[V::N / 4];
        bool fast_v = fast;
        if (check_given) {
          uint32_t m = 0;
#pragma unroll
          for (int i = 0; i < V::N; ++i) { const uint32_t a = abs_bits(f[u][i]); m = m > a ? m : a; }
          fast_v = fast_v && m <= given_bits;
        }
        codes_of<V::N>(f[u], scale, rcp, fast_v, w);
        if (!vtile) {
          uint8_t* dst = t.out8 + (slice * p.d2 + r0) * p.d3 + v * V::N;
          if (V::N == 8) *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
          else *reinterpret_cast<uint32_t*>(dst) = w[0];
        } else {
          // the chunk's rows staged as they are (vrow_offset), re-read in the tile order below
          const int lrow = (int)(v / vpr), d = (int)((v % vpr) * V::N), D = (int)p.d3;
          uint8_t* dst = tile_lds + (lrow >> 6) * 64 * D + vrow_offset(lrow & 63, d >> 4, D) + (d & 15);
          const bool pad = v >= nvec;
          if (V::N == 8) *reinterpret_cast<uint2*>(dst) = pad ? make_uint2(0, 0) : make_uint2(w[0], w[1]);
          else *reinterpret_cast<uint32_t*>(dst) = pad ? 0u : w[0];
        }
      } else {
        // out = x + (dq - x), each step rounded to T (base.py:200-203)
        float o[V::N];
#pragma unroll
        for (int i = 0; i < V::N; ++i) {
          float y = f[u][i] / scale;                 // IEEE division, as the reference's CPU path
          if (kBf16) y = round_bf16(y);
          float dq = e4m3_to_f32(f32_to_e4m3(clamp448(y)) & 0xFFu) * scale;
          if (kBf16) dq = round_bf16(dq);
          float d = dq - f[u][i];
          if (kBf16) d = round_bf16(d);
          o[i] = f[u][i] + d;
        }
        T* dst = static_cast<T*>(t.outx) + (slice * p.d2 + r0) * p.d3 + v * V::N;
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
  }
  if (vtile) {
    // Each 16-byte run of the tiled layout (run index i of a tile: dim 32 (i / 128) + i % 32, key
    // block (i / 64) % 2, half (i / 32) % 2) gathered from the staged rows by transposed reads; 16
    // consecutive runs per 16-lane group, stored contiguously. The chunk holds whole tiles of 4 D
    // runs each (a multiple of 128), so every 16-lane group is whole.
    __syncthreads();
    const int D = (int)p.d3;
    const int64_t ntiles = (p.d2 + 63) >> 6;
    const int nruns = (int)((r1p - r0) * D / 16), tile_runs = 4 * D;
    uint8_t* dst = t.out8 + (slice * ntiles + (r0 >> 6)) * 64 * p.d3;
    for (int i = threadIdx.x; i < nruns; i += kThreads) {
      const int tl = i / tile_runs, ir = i % tile_runs;
      const uint4 run = vtile_run(tile_lds + tl * 64 * D, D, 32 * (ir >> 7) + (ir & 16), (ir >> 6) & 1,
                                  (ir >> 5) & 1, ir & 15);
      *reinterpret_cast<uint4*>(dst + 16 * (int64_t)i) = run;
    }
  }
}

// One wave per row: amax, scale = max(amax / 448, 1e-12), codes = e4m3(x / scale) (no clamp:
// |x / scale| <= 448 whenever amax is finite).
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
  const float amax = __uint_as_float(m);
  float s = amax / kE4m3Max;
  s = s < kEps ? kEps : s;
  if (lane == 0) scale_out[row] = s;
  const bool fast = __builtin_isfinite(amax);
  const float rcp = 1.0f / s;
  uint8_t* dst = out + row * cols;
  for (int64_t v = lane; v < nvec; v += 64) {
    float f[V::N];
    V::load(src + v * V::N, f);
    uint32_t w[V::N / 4];
    if (fast) {
      codes_of<V::N>(f, s, rcp, true, w);
    } else {
#pragma unroll
      for (int i = 0; i < V::N / 4; ++i) {
        uint32_t c = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) c |= (f32_to_e4m3(f[4 * i + j] / s) & 0xFFu) << (8 * j);
        w[i] = c;
      }
    }
    if (V::N == 8) *reinterpret_cast<uint2*>(dst + v * 8) = make_uint2(w[0], w[1]);
    else *reinterpret_cast<uint32_t*>(dst + v * 4) = w[0];
  }
}

// ---------------------------------------------------------------- column quantiser, transposed out
//
// The operands of the FP8 backward GEMMs: for a [rows, cols] matrix (activations x, output
// gradient g, or a weight) the e4m3 codes of each COLUMN, written transposed as out_t[cols, ld]
// (ld >= rows, rows past `rows` coded 0), so that the reduction over rows becomes the contiguous
// K dimension of the "TN" FP8 GEMM. Scales:
//   per column (FLW_SCALE_COLUMN): the _fp8_head recipe on the column, s = max(amax / 448, 1e-12),
//     code = e4m3(x / s) (flw_quant_rows_e4m3 applied to the transpose);
//   per tensor (FLW_SCALE_TENSOR): the _per_tensor_fp8 recipe, s = max(amax, 1e-12) / 448,
//     code = e4m3(clamp(x / s, -448, 448)) (flw_quant_e4m3's codes, transposed).
// Pass 1 (cols_amax_kernel) writes one |x| max per 64 columns x 256 rows tile and column (per tile
// in tensor mode); pass 2 (cols_quant_t_kernel) folds the partials of its columns, quantises its
// 256 x 64 tile and transposes it through LDS so that every output row segment is written with
// 16-byte stores. A thread covers 8 rows x 8 columns (8 rows of one column pack into 8 bytes).
constexpr int kCT = 64, kRT = 256;               // tile: kRT rows x kCT columns
constexpr int kCTStride = kRT + 8;               // LDS bytes per transposed column (bank spread)

template <typename T>
__device__ __forceinline__ void load8(const T* src, float* f) {
  if constexpr (sizeof(T) == 2) {
    Vec16<uint16_t>::load(src, f);
  } else {
    Vec16<float>::load(src, f);
    Vec16<float>::load(src + 4, f + 4);
  }
}

template <typename T>
__device__ __forceinline__ void load_tile8(const T* x, int64_t rows, int64_t cols, int64_t rs, int64_t r0,
                                           int64_t c0, float (&f)[8][8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t r = r0 + i;
    if (r < rows && c0 < cols) {
      load8(x + r * rs + c0, f[i]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) f[i][j] = 0.0f;
    }
  }
}

template <typename T, bool TENSOR>
__global__ __launch_bounds__(kThreads) void cols_amax_kernel(const T* __restrict__ x, int64_t rows,
                                                             int64_t cols, int64_t rs,
                                                             uint32_t* __restrict__ partials) {
  __shared__ uint32_t red[kThreads / 8][kCT + 1];
  const int t = threadIdx.x, cg = t & 7, rg = t >> 3;
  const int64_t c0 = (int64_t)blockIdx.x * kCT + 8 * cg;
  const int64_t r0 = (int64_t)blockIdx.y * kRT + 8 * rg;
  float f[8][8];
  load_tile8(x, rows, cols, rs, r0, c0, f);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) { const uint32_t a = abs_bits(f[i][j]); m = m > a ? m : a; }
    red[rg][8 * cg + j] = m;
  }
  __syncthreads();
  if (t < kCT) {
    uint32_t m = 0;
    for (int g = 0; g < kThreads / 8; ++g) m = m > red[g][t] ? m : red[g][t];
    if (TENSOR) {
      m = wave_max_u32(m);
      if (t == 0) partials[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = m;
    } else if ((int64_t)blockIdx.x * kCT + t < cols) {
      partials[(int64_t)blockIdx.y * cols + (int64_t)blockIdx.x * kCT + t] = m;
    }
  }
}

template <typename T, bool TENSOR>
__global__ __launch_bounds__(kThreads) void cols_quant_t_kernel(const T* __restrict__ x, int64_t rows,
                                                                int64_t cols, int64_t rs,
                                                                const uint32_t* __restrict__ partials,
                                                                int64_t nchunks, int64_t ncb,
                                                                uint8_t* __restrict__ out, int64_t ld,
                                                                float* __restrict__ scale_out) {
  __shared__ __align__(16) uint8_t lt[kCT * kCTStride];
  __shared__ float sc[kCT], rc[kCT];
  __shared__ uint32_t red[kThreads / 64];
  const int t = threadIdx.x, cg = t & 7, rg = t >> 3;
  const int64_t cb0 = (int64_t)blockIdx.x * kCT;
  // Scales of this tile's columns.
  if (TENSOR) {
    uint32_t m = 0;
    for (int64_t i = t; i < nchunks * ncb; i += kThreads) m = m > partials[i] ? m : partials[i];
    m = block_max_u32(m, red);
    const float amax = __uint_as_float(m);
    const float s = (amax < kEps ? kEps : amax) / kE4m3Max;
    if (t < kCT) { sc[t] = s; rc[t] = 1.0f / s; }
    if (blockIdx.x == 0 && blockIdx.y == 0 && t == 0) scale_out[0] = s;
  } else {
    // Fold the column partials with all 256 threads (4 row-chunk lanes per column, several loads
    // in flight each): a single thread per column walking the chunks serialises their latency.
    __shared__ uint32_t fold[kThreads / kCT][kCT];
    const int cl = t & (kCT - 1), part = t / kCT;
    const int64_t c = cb0 + cl;
    uint32_t m = 0;
    if (c < cols) {
#pragma unroll 4
      for (int64_t k = part; k < nchunks; k += kThreads / kCT) {
        const uint32_t a = partials[k * cols + c];
        m = m > a ? m : a;
      }
    }
    fold[part][cl] = m;
    __syncthreads();
    if (t < kCT) {
#pragma unroll
      for (int q = 1; q < kThreads / kCT; ++q) m = m > fold[q][t] ? m : fold[q][t];
      const float amax = __uint_as_float(m);
      float s = amax / kE4m3Max;
      s = s < kEps ? kEps : s;
      sc[t] = s;
      rc[t] = 1.0f / s;
      if (blockIdx.y == 0 && c < cols) scale_out[c] = s;
    }
  }
  __syncthreads();

  const int64_t c0 = cb0 + 8 * cg;
  const int64_t r0 = (int64_t)blockIdx.y * kRT + 8 * rg;
  float f[8][8];
  load_tile8(x, rows, cols, rs, r0, c0, f);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int cj = 8 * cg + j;
    const float s = sc[cj], r = rc[cj];
    float col[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) col[i] = f[i][j];
    uint32_t w[2];
    if (__builtin_isfinite(s * kE4m3Max) && __builtin_isfinite(r)) {
      codes_of<8>(col, s, r, true, w);
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t c = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float q = col[4 * h + e] / s;
          c |= (f32_to_e4m3(TENSOR ? clamp448(q) : q) & 0xFFu) << (8 * e);
        }
        w[h] = c;
      }
    }
    *reinterpret_cast<uint2*>(lt + cj * kCTStride + 8 * rg) = make_uint2(w[0], w[1]);
  }
  __syncthreads();
  // Store: thread t writes column t / 4, rows 64 q + 16 (t % 4) .. +15 for q = 0..3, so that
  // each store instruction writes 64 contiguous bytes of every column it touches.
  const int cl = t >> 2, part = t & 3;
  const int64_t c = cb0 + cl;
  if (c < cols) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int rr = 64 * q + 16 * part;
      const int64_t r = (int64_t)blockIdx.y * kRT + rr;
      if (r < ld) {
        const uint2 a = *reinterpret_cast<const uint2*>(lt + cl * kCTStride + rr);
        const uint2 b = *reinterpret_cast<const uint2*>(lt + cl * kCTStride + rr + 8);
        *reinterpret_cast<uint4*>(out + c * ld + r) = make_uint4(a.x, a.y, b.x, b.y);
      }
    }
  }
}

// ---------------------------------------------------------------- activation + per-row quantiser
//
// The producer of an FP8 linear's input fused with its per-row quantiser (flw_quant_rows_e4m3
// semantics), one wave per row, the row held in registers between the reductions:
//   ACT_RMSNORM: h = bf16( bf16( x * (1 / sqrt(mean(x^2) + eps)) ) * w )   (base.py:324-338)
//   ACT_GELU:    h = bf16( (0.5 x) * (1 + erf(x / sqrt 2)) )                 (F.gelu, erf form)
// then scale = max(amax|h| / 448, 1e-12), code = e4m3(h / scale). bf16 in and out; the bf16 h
// is written too when h_out is given.
constexpr int kActRmsnorm = 0, kActGelu = 1, kActNone = 2;   // kActNone: h = x (flw_quant_rows_e4m3)

// GELU with erf by Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7): erf(|z|) = 1 - q(t) exp(-z^2),
// t = 1 / (1 + p |z|); two transcendental and six fused multiply-adds instead of the device
// library's full-precision erff, an error far below the bf16 rounding of the result. With
// z = x / sqrt 2 folded into the constants (p / sqrt 2, exp2(x * (x * -log2(e) / 2))) and
// u = 1 - q e = erf(|z|):
//   (0.5 x) (1 + erf(z)) = x * RN(0.5 +- 0.5 u)  (+ for x >= 0, - below; the same roundings as
//   RN(0.5 x) * RN(1 +- u), since scaling by 0.5 is exact), so 1 + erf still cancels to 0 for
//   very negative x, as the reference's fp32 evaluation does.
__device__ __forceinline__ float gelu_as(float x) {
  const float a = __builtin_fabsf(x);
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f * 0.70710678118654752f, a, 1.0f));
  float q = fmaf(1.061405429f, t, -1.453152027f);
  q = fmaf(q, t, 1.421413741f);
  q = fmaf(q, t, -0.284496736f);
  q = fmaf(q, t, 0.254829592f);
  q *= t;
  const float e = __builtin_amdgcn_exp2f(x * (x * (-0.5f * 1.4426950408889634f)));
  const float u = fmaf(-q, e, 1.0f);
  return x * fmaf(__builtin_copysignf(0.5f, x), u, 0.5f);
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <int ACT, int NV>
__global__ __launch_bounds__(kThreads) void rows_act_quant_kernel(
    const uint16_t* __restrict__ x, int64_t rows, int cols, int64_t rs, const uint16_t* __restrict__ w,
    float eps, uint8_t* __restrict__ out, float* __restrict__ scale_out, uint16_t* __restrict__ h_out) {
  const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;            // wave-uniform
  const int lane = threadIdx.x & 63;
  const int nvec = cols >> 3;
  const uint16_t* src = x + row * rs;
  // The row stays in registers as packed bf16 (h is a bf16 value at every step that is kept).
  uint4 hb[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = lane + 64 * i;
    hb[i] = v < nvec ? *reinterpret_cast<const uint4*>(src + 8 * v) : make_uint4(0, 0, 0, 0);
  }
  auto unpack = [](const uint4& q, float* f) __attribute__((always_inline)) { Vec16<uint16_t>::unpack(q, f); };
  // NaN halves keep their payload here and are made 0x7FC0 below, only in rows whose amax is NaN.
  auto pack = [](const float* f) __attribute__((always_inline)) {
    return make_uint4(bf16x2_rne_raw(f[0], f[1]), bf16x2_rne_raw(f[2], f[3]), bf16x2_rne_raw(f[4], f[5]),
                      bf16x2_rne_raw(f[6], f[7]));
  };
  if (ACT == kActRmsnorm) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float f[8];
      unpack(hb[i], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(f[e], f[e], ss);
    }
    const float ms = wave_sum_f32(ss) / (float)cols;
    const float r = 1.0f / __builtin_sqrtf(ms + eps);        // IEEE sqrt and division
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int v = lane + 64 * i;
      if (v >= nvec) continue;
      float f[8], g[8];
      unpack(hb[i], f);
      Vec16<uint16_t>::load(w + 8 * v, g);
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {       // bf16(bf16(x r) w), two values per conversion
        const uint32_t t = bf16x2_rne_raw(f[2 * e] * r, f[2 * e + 1] * r);
        o[e] = bf16x2_rne_raw(__uint_as_float(t << 16) * g[2 * e], __uint_as_float(t & 0xFFFF0000u) * g[2 * e + 1]);
      }
      hb[i] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  } else if (ACT == kActGelu) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float f[8];
      unpack(hb[i], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = gelu_as(f[e]);
      hb[i] = pack(f);
      __builtin_amdgcn_sched_barrier(0);        // one vector's erf at a time: bounded registers
    }
  }
  // |h| maxima as 16-bit halves (v_pk_max_u16 over the bf16 bit patterns: NaN above inf).
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  u16x2 m2 = {0, 0};
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const uint32_t q[4] = {hb[i].x, hb[i].y, hb[i].z, hb[i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, q[e] & 0x7FFF7FFFu));
  }
  uint32_t m = (uint32_t)(m2[0] > m2[1] ? m2[0] : m2[1]) << 16;
  m = wave_max_u32(m);
  const float amax = __uint_as_float(m);
  if (ACT != kActNone && __builtin_isnan(amax)) {   // wave-uniform, rare: NaN h as 0x7FC0
#pragma unroll
    for (int i = 0; i < NV; ++i)
      hb[i] = make_uint4(bf16x2_canon_nan(hb[i].x), bf16x2_canon_nan(hb[i].y), bf16x2_canon_nan(hb[i].z),
                         bf16x2_canon_nan(hb[i].w));
  }
  float sc = amax / kE4m3Max;
  sc = sc < kEps ? kEps : sc;
  if (lane == 0) scale_out[row] = sc;
  const bool fast = __builtin_isfinite(amax);
  const float rcp = 1.0f / sc;
  uint8_t* dst = out + row * cols;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = lane + 64 * i;
    if (v >= nvec) continue;
    float f[8];
    unpack(hb[i], f);
    uint32_t wd[2];
    if (fast) {
      codes_of<8>(f, sc, rcp, true, wd);
    } else {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        uint32_t c = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) c |= (f32_to_e4m3(f[4 * q + j] / sc) & 0xFFu) << (8 * j);
        wd[q] = c;
      }
    }
    *reinterpret_cast<uint2*>(dst + 8 * v) = make_uint2(wd[0], wd[1]);
    if (h_out) *reinterpret_cast<uint4*>(h_out + row * cols + 8 * v) = hb[i];
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

template <int MODE>
static int launch_quant(const QuantParams& p, int ntensors, int dtype, hipStream_t s, const char* name,
                        Timer tm) {
  dim3 grid((unsigned)p.nchunks, (unsigned)(p.d0 * p.d1), (unsigned)ntensors);
  bool any_vtile = false, xform = false;
  for (int i = 0; i < ntensors; ++i) {
    any_vtile |= p.t[i].layout == FLW_LAYOUT_VTILE;
    xform |= p.t[i].norm != 0 || p.t[i].rcos != nullptr;
  }
  const size_t lds = MODE == 0 && any_vtile ? (size_t)(kRowsPerChunk * p.d3) : 0;
  const bool f32 = dtype == FLW_F32;
  const void* ka = xform ? (f32 ? reinterpret_cast<const void*>(&amax_kernel<float, true>)
                                : reinterpret_cast<const void*>(&amax_kernel<uint16_t, true>))
                         : (f32 ? reinterpret_cast<const void*>(&amax_kernel<float>)
                                : reinterpret_cast<const void*>(&amax_kernel<uint16_t>));
  const void* kq = xform ? (f32 ? reinterpret_cast<const void*>(&quant_kernel<float, MODE, MODE == 0>)
                                : reinterpret_cast<const void*>(&quant_kernel<uint16_t, MODE, MODE == 0>))
                         : (f32 ? reinterpret_cast<const void*>(&quant_kernel<float, MODE>)
                                : reinterpret_cast<const void*>(&quant_kernel<uint16_t, MODE>));
  if (p.amax_given) {                     // amax from the producer: the quantise pass only
    (void)launch_ext(kq, grid, dim3(kThreads), lds, s, p, tm.start, tm.stop);
    return check_launch(name);
  }
  (void)launch_ext(ka, grid, dim3(kThreads), 0, s, p, tm.start, nullptr);
  (void)launch_ext(kq, grid, dim3(kThreads), lds, s, p, nullptr, tm.stop);
  return check_launch(name);
}

static void set_tensor(QTensor& t, const void* x, int64_t sb, int64_t sh, int64_t st, int64_t D,
                       int layout, uint8_t* out8, void* outx, float* scale_out) {
  t.x = x; t.s0 = sb; t.s1 = sh; t.s2 = st; t.layout = layout; t.out8 = out8; t.outx = outx;
  t.scale_out = scale_out; t.rows_packed = st == D ? 1 : 0;
}

// Quantise n (1..3) tensors of one shape, dtype and granularity in two launches.
int quant_bhtd_n(int n, const void* const* xs, int dtype, int64_t B, int64_t H, int64_t T,
                 int64_t D, const int64_t* strides, int granularity, const int* layouts,
                 uint8_t* const* outs, float* const* scale_outs, void* ws, size_t ws_bytes,
                 hipStream_t stream, Timer tm, const uint32_t* amax_given, const QkTransform* xf,
                 float* q_rcp_deferred) {
  FLW_REQUIRE(n >= 1 && n <= 3, FLW_E_INVALID, "1 to 3 tensors per call");
  FLW_REQUIRE(granularity >= FLW_SCALE_TENSOR && granularity <= FLW_SCALE_BH, FLW_E_INVALID, "bad granularity %d", granularity);
  FLW_REQUIRE(amax_given != nullptr || (ws != nullptr && ws_bytes >= (size_t)n * partial_bytes(B, H, T)),
              FLW_E_WORKSPACE, "workspace needs %zu bytes", (size_t)n * partial_bytes(B, H, T));
  QuantParams p{};
  for (int i = 0; i < n; ++i) {
    int rc = check_tensor(xs[i], dtype, B, H, T, D, strides[3 * i], strides[3 * i + 1], strides[3 * i + 2]);
    if (rc) return rc;
    FLW_REQUIRE(layouts[i] == FLW_LAYOUT_BHTD || layouts[i] == FLW_LAYOUT_VTILE, FLW_E_INVALID, "bad layout %d", layouts[i]);
    FLW_REQUIRE(outs[i] != nullptr && scale_outs[i] != nullptr, FLW_E_INVALID, "null output pointer");
    if (layouts[i] == FLW_LAYOUT_VTILE) {
      FLW_REQUIRE(D == 32 || D == 64 || D == 128, FLW_E_UNSUPPORTED, "VTILE layout needs D in {32, 64, 128}");
      FLW_REQUIRE(((uintptr_t)outs[i] & 15) == 0, FLW_E_INVALID, "VTILE output must be 16-byte aligned");
    } else {
      FLW_REQUIRE(((uintptr_t)outs[i] & 7) == 0, FLW_E_INVALID, "output must be 8-byte aligned");
    }
    set_tensor(p.t[i], xs[i], strides[3 * i], strides[3 * i + 1], strides[3 * i + 2], D, layouts[i], outs[i],
               nullptr, scale_outs[i]);
    if (xf != nullptr && i < 2) {
      FLW_REQUIRE(layouts[i] == FLW_LAYOUT_BHTD, FLW_E_INVALID, "q / k transforms need BHTD codes");
      p.t[i].norm = xf->norm;
      p.t[i].eps = xf->eps;
      p.t[i].rcos = xf->rcos;
      p.t[i].rsin = xf->rsin;
      p.t[i].tout = i == 0 ? xf->qout : xf->kout;
    }
  }
  if (q_rcp_deferred != nullptr) {
    FLW_REQUIRE(xf == nullptr && layouts[0] == FLW_LAYOUT_BHTD, FLW_E_INVALID,
                "deferred Q codes need no transform and BHTD codes");
    p.t[0].defer = 1;
    p.t[0].rcp_out = q_rcp_deferred;
  }
  p.d0 = B; p.d1 = H; p.d2 = T; p.d3 = D;
  p.nchunks = nchunks_of(T); p.partials = static_cast<uint32_t*>(ws); p.granularity = granularity;
  p.amax_given = amax_given;
  return launch_quant<0>(p, n, dtype, stream, "flw_quant_e4m3", tm);
}

int quant_bhtd(const void* x, int dtype, int64_t B, int64_t H, int64_t T, int64_t D, int64_t sb,
               int64_t sh, int64_t st, int granularity, int layout, uint8_t* out, float* scale_out,
               void* ws, size_t ws_bytes, hipStream_t stream) {
  const int64_t strides[3] = {sb, sh, st};
  return quant_bhtd_n(1, &x, dtype, B, H, T, D, strides, granularity, &layout, &out, &scale_out, ws,
                      ws_bytes, stream, take_timer());
}

// One workgroup per scale group (grid.x) folds that group's amax partials into amax_out.
__global__ __launch_bounds__(kThreads) void amax_fold_kernel(QuantParams p, uint32_t* __restrict__ amax_out) {
  __shared__ uint32_t red[kThreads / 64];
  const int64_t g = blockIdx.x;
  const int64_t slice = p.granularity == FLW_SCALE_BH ? g : 0;
  const int64_t i1 = p.granularity == FLW_SCALE_HEAD ? g : slice % p.d1;
  const uint32_t m = group_amax(p, p.partials, slice, i1, red);
  if (threadIdx.x == 0) amax_out[g] = m;
}

// The amax pass alone: |x| max per scale group, as the bit patterns of non-negative fp32 values.
int amax_bhtd(const void* x, int dtype, int64_t B, int64_t H, int64_t T, int64_t D, int64_t sb,
              int64_t sh, int64_t st, int granularity, uint32_t* amax_out, void* ws,
              size_t ws_bytes, hipStream_t stream) {
  int rc = check_tensor(x, dtype, B, H, T, D, sb, sh, st);
  if (rc) return rc;
  FLW_REQUIRE(granularity >= FLW_SCALE_TENSOR && granularity <= FLW_SCALE_BH, FLW_E_INVALID, "bad granularity %d", granularity);
  FLW_REQUIRE(amax_out != nullptr, FLW_E_INVALID, "null amax output");
  FLW_REQUIRE(ws != nullptr && ws_bytes >= partial_bytes(B, H, T), FLW_E_WORKSPACE, "workspace needs %zu bytes",
              partial_bytes(B, H, T));
  QuantParams p{};
  set_tensor(p.t[0], x, sb, sh, st, D, FLW_LAYOUT_BHTD, nullptr, nullptr, nullptr);
  p.d0 = B; p.d1 = H; p.d2 = T; p.d3 = D;
  p.nchunks = nchunks_of(T); p.partials = static_cast<uint32_t*>(ws); p.granularity = granularity;
  const int64_t G = granularity == FLW_SCALE_TENSOR ? 1 : (granularity == FLW_SCALE_HEAD ? H : B * H);
  const void* ka = dtype == FLW_F32 ? reinterpret_cast<const void*>(&amax_kernel<float>)
                                    : reinterpret_cast<const void*>(&amax_kernel<uint16_t>);
  const Timer tm = take_timer();
  (void)launch_ext(ka, dim3((unsigned)p.nchunks, (unsigned)(B * H), 1u), dim3(kThreads), 0, stream, p,
                   tm.start, nullptr);
  (void)launch_args(reinterpret_cast<const void*>(&amax_fold_kernel), dim3((unsigned)G), dim3(kThreads), 0,
                    stream, nullptr, tm.stop, p, amax_out);
  return check_launch("flw_amax_e4m3");
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

extern "C" int flw_amax_e4m3(const void* x, int dtype, int64_t B, int64_t H, int64_t T, int64_t D,
                             int64_t stride_b, int64_t stride_h, int64_t stride_t, int granularity,
                             uint32_t* amax_out, void* workspace, size_t workspace_bytes, void* stream) {
  return amax_bhtd(x, dtype, B, H, T, D, stride_b, stride_h, stride_t, granularity, amax_out, workspace,
                   workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int flw_quant_e4m3_amax(const void* x, int dtype, int64_t B, int64_t H, int64_t T, int64_t D,
                                   int64_t stride_b, int64_t stride_h, int64_t stride_t, int granularity,
                                   int layout, const uint32_t* amax, uint8_t* out, float* scale_out,
                                   void* stream) {
  FLW_REQUIRE(amax != nullptr, FLW_E_INVALID, "null amax");
  const int64_t strides[3] = {stride_b, stride_h, stride_t};
  return quant_bhtd_n(1, &x, dtype, B, H, T, D, strides, granularity, &layout, &out, &scale_out, nullptr, 0,
                      static_cast<hipStream_t>(stream), take_timer(), amax);
}

extern "C" int flw_quant_qkv_e4m3(const void* q, const void* k, const void* v, int dtype, int64_t B,
                                  int64_t H, int64_t T, int64_t D, const int64_t* strides,
                                  int granularity, uint8_t* q8, uint8_t* k8, uint8_t* v_tiles,
                                  float* scales_out, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  FLW_REQUIRE(strides != nullptr && scales_out != nullptr, FLW_E_INVALID, "null strides / scales");
  const int64_t G = granularity == FLW_SCALE_TENSOR ? 1 : (granularity == FLW_SCALE_HEAD ? H : B * H);
  const void* xs[3] = {q, k, v};
  const int layouts[3] = {FLW_LAYOUT_BHTD, FLW_LAYOUT_BHTD, FLW_LAYOUT_VTILE};
  uint8_t* outs[3] = {q8, k8, v_tiles};
  float* sc[3] = {scales_out, scales_out + G, scales_out + 2 * G};
  return quant_bhtd_n(3, xs, dtype, B, H, T, D, strides, granularity, layouts, outs, sc, workspace,
                      workspace_bytes, static_cast<hipStream_t>(stream), take_timer());
}

extern "C" int flw_quant_qkv_e4m3_deferq(const void* q, const void* k, const void* v, int dtype, int64_t B,
                                         int64_t H, int64_t T, int64_t D, const int64_t* strides,
                                         int granularity, uint8_t* q8, uint8_t* k8, uint8_t* v_tiles,
                                         float* scales_out, float* q_rcp_out, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  FLW_REQUIRE(strides != nullptr && scales_out != nullptr && q_rcp_out != nullptr, FLW_E_INVALID,
              "null strides / scales / q_rcp_out");
  const int64_t G = granularity == FLW_SCALE_TENSOR ? 1 : (granularity == FLW_SCALE_HEAD ? H : B * H);
  const void* xs[3] = {q, k, v};
  const int layouts[3] = {FLW_LAYOUT_BHTD, FLW_LAYOUT_BHTD, FLW_LAYOUT_VTILE};
  uint8_t* outs[3] = {q8, k8, v_tiles};
  float* sc[3] = {scales_out, scales_out + G, scales_out + 2 * G};
  return quant_bhtd_n(3, xs, dtype, B, H, T, D, strides, granularity, layouts, outs, sc, workspace,
                      workspace_bytes, static_cast<hipStream_t>(stream), take_timer(), nullptr, nullptr, q_rcp_out);
}

extern "C" int flw_qk_norm_rope_quant_e4m3(const void* q, const void* k, const void* v, int dtype, int64_t B,
                                           int64_t H, int64_t T, int64_t D, const int64_t* strides,
                                           int qk_norm, float eps, const void* rope_cos, const void* rope_sin,
                                           int granularity, uint8_t* q8, uint8_t* k8, uint8_t* v_tiles,
                                           float* scales_out, void* q_out, void* k_out, void* workspace,
                                           size_t workspace_bytes, void* stream) {
  FLW_REQUIRE(strides != nullptr && scales_out != nullptr, FLW_E_INVALID, "null strides / scales");
  FLW_REQUIRE((rope_cos == nullptr) == (rope_sin == nullptr), FLW_E_INVALID, "pass both RoPE tables or neither");
  FLW_REQUIRE(D % 2 == 0, FLW_E_INVALID, "RoPE needs an even head_dim");
  FLW_REQUIRE(((uintptr_t)rope_cos & 15) == 0 && ((uintptr_t)rope_sin & 15) == 0 && ((uintptr_t)q_out & 15) == 0 &&
              ((uintptr_t)k_out & 15) == 0, FLW_E_INVALID, "RoPE tables and q_out / k_out must be 16-byte aligned");
  FLW_REQUIRE(!(eps < 0.0f) && eps == eps, FLW_E_INVALID, "eps must be a non-negative number");
  const int64_t G = granularity == FLW_SCALE_TENSOR ? 1 : (granularity == FLW_SCALE_HEAD ? H : B * H);
  const void* xs[3] = {q, k, v};
  const int layouts[3] = {FLW_LAYOUT_BHTD, FLW_LAYOUT_BHTD, FLW_LAYOUT_VTILE};
  uint8_t* outs[3] = {q8, k8, v_tiles};
  float* sc[3] = {scales_out, scales_out + G, scales_out + 2 * G};
  QkTransform xf;
  xf.norm = qk_norm != 0;
  xf.eps = eps;
  xf.rcos = rope_cos;
  xf.rsin = rope_sin;
  xf.qout = q_out;
  xf.kout = k_out;
  return quant_bhtd_n(3, xs, dtype, B, H, T, D, strides, granularity, layouts, outs, sc, workspace,
                      workspace_bytes, static_cast<hipStream_t>(stream), take_timer(), nullptr, &xf);
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
  QuantParams p{};
  float* sc = scale_out;
  if (sc == nullptr) {   // optional: park the scales in the tail of the workspace
    const size_t need = partial_bytes(B, H, T) + sizeof(float) * (size_t)(B * H);
    FLW_REQUIRE(workspace_bytes >= need, FLW_E_WORKSPACE, "workspace needs %zu bytes without scale_out", need);
    sc = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + partial_bytes(B, H, T));
  }
  set_tensor(p.t[0], x, stride_b, stride_h, stride_t, D, FLW_LAYOUT_BHTD, nullptr, out, sc);
  p.d0 = B; p.d1 = H; p.d2 = T; p.d3 = D;
  p.nchunks = nchunks_of(T); p.partials = static_cast<uint32_t*>(workspace); p.granularity = granularity;
  return launch_quant<1>(p, 1, dtype, static_cast<hipStream_t>(stream), "flw_fake_quant_e4m3", take_timer());
}

template <int ACT>
static int rows_act_quant(const void* x, int64_t rows, int64_t cols, int64_t rs, const void* w, float eps,
                          uint8_t* out, float* scale_out, void* h_out, hipStream_t s, const char* name);

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
  // bf16 rows of up to 4096 elements: read once and kept in registers between the amax and the
  // codes (the generic kernel re-reads the row, which for long rows comes back from HBM).
  if (dtype == FLW_BF16 && cols <= 4096 && row_stride >= cols && ((uintptr_t)out & 7) == 0)
    return rows_act_quant<kActNone>(x, rows, cols, row_stride, nullptr, 0.0f, out, scale_out, nullptr, s,
                                    "flw_quant_rows_e4m3");
  dim3 grid((unsigned)((rows + 3) / 4));
  const Timer tm = take_timer();
  if (dtype == FLW_F32)
    (void)launch_args(reinterpret_cast<const void*>(&rows_quant_kernel<float>), grid, dim3(kThreads), 0, s,
                      tm.start, tm.stop, static_cast<const float*>(x), rows, cols, row_stride, out, scale_out);
  else
    (void)launch_args(reinterpret_cast<const void*>(&rows_quant_kernel<uint16_t>), grid, dim3(kThreads), 0, s,
                      tm.start, tm.stop, static_cast<const uint16_t*>(x), rows, cols, row_stride, out, scale_out);
  return check_launch("flw_quant_rows_e4m3");
}

extern "C" size_t flw_quant_cols_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  const int64_t nchunks = (rows + kRT - 1) / kRT, ncb = (cols + kCT - 1) / kCT;
  return (size_t)(nchunks * (cols > ncb ? cols : ncb)) * sizeof(uint32_t);
}

// ---------------------------------------------------------------- e4m3 codes transposed
//
// out_t [cols, ld] = codes [rows, cols] transposed, columns rows .. ld - 1 of out_t zero: the
// transposed operand of a GEMM from codes quantised with one scale for the whole matrix (the
// tensorwise recipe), where the column codes equal the row codes. 64 x 64-byte tiles through LDS:
// thread t loads 16 bytes of row t / 4 (64-byte rows of the tile, padded to 80 in LDS), then
// gathers the 16 bytes of output row t / 4 at input rows 16 (t % 4) .. + 15 and stores them
// as one 16-byte vector. Rows past `rows` read as zero, columns past `cols` are not stored.
constexpr int kTT = 64, kTPitch = 80;

__global__ __launch_bounds__(256) void transpose_u8_kernel(const uint8_t* __restrict__ src, int64_t rows,
                                                           int64_t cols, int64_t sld, uint8_t* __restrict__ dst,
                                                           int64_t dld) {
  __shared__ __align__(16) uint8_t t[kTT * kTPitch];
  const int tid = threadIdx.x;
  const int64_t c0 = (int64_t)blockIdx.x * kTT, r0 = (int64_t)blockIdx.y * kTT;
  {
    const int r = tid >> 2, q = tid & 3;
    const int64_t gr = r0 + r, gc = c0 + 16 * q;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (gr < rows && gc < cols) v = *reinterpret_cast<const uint4*>(src + gr * sld + gc);
    *reinterpret_cast<uint4*>(t + r * kTPitch + 16 * q) = v;
  }
  __syncthreads();
  const int c = tid >> 2, q = tid & 3;
  const int64_t oc = c0 + c, orow0 = r0 + 16 * q;
  if (oc >= cols || orow0 >= dld) return;
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t x = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) x |= (uint32_t)t[(16 * q + 4 * j + b) * kTPitch + c] << (8 * b);
    w[j] = x;
  }
  *reinterpret_cast<uint4*>(dst + oc * dld + orow0) = make_uint4(w[0], w[1], w[2], w[3]);
}

extern "C" int flw_transpose_e4m3(const uint8_t* codes, int64_t rows, int64_t cols, int64_t row_stride,
                                  uint8_t* out_t, int64_t ld, void* stream) {
  FLW_REQUIRE(codes != nullptr && out_t != nullptr, FLW_E_INVALID, "null pointer");
  FLW_REQUIRE(rows > 0 && cols > 0, FLW_E_INVALID, "empty matrix");
  FLW_REQUIRE(cols % 16 == 0 && row_stride % 16 == 0 && row_stride >= cols && ((uintptr_t)codes & 15) == 0,
              FLW_E_INVALID, "cols and row_stride must be multiples of 16, codes 16-byte aligned");
  FLW_REQUIRE(ld >= rows && ld % 16 == 0 && ((uintptr_t)out_t & 15) == 0, FLW_E_INVALID,
              "ld must be >= rows and a multiple of 16, out_t 16-byte aligned");
  const int64_t gx = (cols + kTT - 1) / kTT, gy = (ld + kTT - 1) / kTT;
  FLW_REQUIRE(gx <= 0x7FFFFFFF && gy <= 65535, FLW_E_UNSUPPORTED, "matrix too large");
  (void)launch_args(reinterpret_cast<const void*>(&transpose_u8_kernel), dim3((unsigned)gx, (unsigned)gy),
                    dim3(256), 0, static_cast<hipStream_t>(stream), nullptr, nullptr, codes, rows, cols,
                    row_stride, out_t, ld);
  return check_launch("flw_transpose_e4m3");
}

// Tensorwise e4m3 of a bf16 matrix writing both layouts in one pass: a 64 x 64 tile's codes go to
// out8 in rows and, staged in LDS, to out_t in columns (the transpose_u8_kernel gather). The scale
// comes from the tensor's |x| max (amax_bits, folded by the amax pass before this launch); the
// arithmetic is quant_kernel's, so both layouts hold exactly the tensorwise quantiser's codes.
// Rows of out_t past `rows` (up to ld, which grid.y covers) are zero.
// part != nullptr: amax_bits is unused and every workgroup folds the npart amax partials itself (a
// few hundred: a weight matrix), which spares the fold its own launch.
__global__ __launch_bounds__(256) void quant_tensor_t_kernel(const uint16_t* __restrict__ x, int64_t rows,
                                                             int64_t cols, int64_t xs,
                                                             const uint32_t* __restrict__ amax_bits,
                                                             uint8_t* __restrict__ out8, int64_t ld8,
                                                             uint8_t* __restrict__ out_t, int64_t ldt,
                                                             float* __restrict__ scale_out,
                                                             const uint32_t* __restrict__ part, int npart) {
  __shared__ __align__(16) uint8_t t[kTT * kTPitch];
  __shared__ uint32_t red[4];
  const int tid = threadIdx.x;
  const int64_t c0 = (int64_t)blockIdx.x * kTT, r0 = (int64_t)blockIdx.y * kTT;
  uint32_t amax_u;
  if (part != nullptr) {
    uint32_t m = 0;
    for (int i = tid; i < npart; i += 256) m = m > part[i] ? m : part[i];
    m = wave_max_u32(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    amax_u = red[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) amax_u = amax_u > red[i] ? amax_u : red[i];
  } else {
    amax_u = *amax_bits;
  }
  const float amax = __uint_as_float(amax_u);
  const float scale = (amax < kEps ? kEps : amax) / kE4m3Max;    // IEEE fp32 division
  const bool fast = __builtin_isfinite(amax);
  const float rcp = 1.0f / scale;
  if (blockIdx.x == 0 && blockIdx.y == 0 && tid == 0) scale_out[0] = scale;
  {
    const int r = tid >> 2, q = tid & 3;
    const int64_t gr = r0 + r, gc = c0 + 16 * q;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (gr < rows && gc < cols) {
      float f[16];
      Vec16<uint16_t>::load(x + gr * xs + gc, f);
      Vec16<uint16_t>::load(x + gr * xs + gc + 8, f + 8);
      uint32_t w[4];
      codes_of<8>(f, scale, rcp, fast, w);
      codes_of<8>(f + 8, scale, rcp, fast, w + 2);
      v = make_uint4(w[0], w[1], w[2], w[3]);
      *reinterpret_cast<uint4*>(out8 + gr * ld8 + gc) = v;
    }
    *reinterpret_cast<uint4*>(t + r * kTPitch + 16 * q) = v;
  }
  __syncthreads();
  const int c = tid >> 2, q = tid & 3;
  const int64_t oc = c0 + c, orow0 = r0 + 16 * q;
  if (oc >= cols || orow0 >= ldt) return;
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t v = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) v |= (uint32_t)t[(16 * q + 4 * j + b) * kTPitch + c] << (8 * b);
    w[j] = v;
  }
  *reinterpret_cast<uint4*>(out_t + oc * ldt + orow0) = make_uint4(w[0], w[1], w[2], w[3]);
}

// One workgroup of 1024 threads folds n amax partials into out[0]: eight independent loads in
// flight per thread, then the wave and workgroup maxima.
__global__ __launch_bounds__(1024) void amax_fold_tensor_kernel(const uint32_t* __restrict__ part, int64_t n,
                                                                uint32_t* __restrict__ out) {
  __shared__ uint32_t red[16];
  uint32_t m = 0;
  for (int64_t i0 = threadIdx.x; i0 < n; i0 += 1024 * 8) {
    uint32_t a[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t i = i0 + 1024 * u;
      a[u] = i < n ? part[i] : 0u;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) m = m > a[u] ? m : a[u];
  }
  m = wave_max_u32(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = red[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) r = r > red[i] ? r : red[i];
    out[0] = r;
  }
}

constexpr int64_t kInlineFold = 1024;   // amax partials every quantising workgroup folds itself

// The amax pass's rows for a contiguous matrix of n values: the narrowest of 64 .. 512 values that
// leaves at most kInlineFold chunks of 128 rows (so no fold launch), else 64; 0: not flat.
static int64_t tensor_t_flat_cols(int64_t n) {
  if (n % 64 != 0) return 0;
  for (int64_t c = 64; c <= 512; c *= 2)
    if (n % c == 0 && nchunks_of(n / c) <= kInlineFold) return c;
  return 64;
}

extern "C" size_t flw_quant_tensor_t_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  const int64_t n = rows * cols, fc = tensor_t_flat_cols(n);
  return 16 + partial_bytes(1, 1, fc ? n / fc : rows);     // the amax pass's chunk rows
}

static int quant_t_check(const void* x, int64_t rows, int64_t cols, int64_t row_stride, const uint8_t* out8,
                         int64_t ld8, const uint8_t* out_t, int64_t ldt, const float* scale_out) {
  FLW_REQUIRE(x != nullptr && out8 != nullptr && out_t != nullptr && scale_out != nullptr, FLW_E_INVALID,
              "null pointer");
  FLW_REQUIRE(rows > 0 && cols > 0, FLW_E_INVALID, "empty matrix");
  FLW_REQUIRE(cols % 16 == 0 && row_stride % 8 == 0 && row_stride >= cols && ((uintptr_t)x & 15) == 0,
              FLW_E_INVALID, "cols must be a multiple of 16, bf16 rows 16-byte aligned with a stride >= cols");
  FLW_REQUIRE(ld8 >= cols && ld8 % 16 == 0 && ((uintptr_t)out8 & 15) == 0, FLW_E_INVALID,
              "out8 rows must be 16-byte aligned with ld8 >= cols");
  FLW_REQUIRE(ldt >= rows && ldt % 16 == 0 && ((uintptr_t)out_t & 15) == 0, FLW_E_INVALID,
              "ld must be >= rows and a multiple of 16, out_t 16-byte aligned");
  FLW_REQUIRE((cols + kTT - 1) / kTT <= 0x7FFFFFFF && (ldt + kTT - 1) / kTT <= 65535, FLW_E_UNSUPPORTED,
              "matrix too large");
  return FLW_OK;
}

extern "C" int flw_quant_tensor_t_e4m3_amax(const void* x, int64_t rows, int64_t cols, int64_t row_stride,
                                            const uint32_t* amax, uint8_t* out8, int64_t ld8, uint8_t* out_t,
                                            int64_t ldt, float* scale_out, void* stream) {
  int rc = quant_t_check(x, rows, cols, row_stride, out8, ld8, out_t, ldt, scale_out);
  if (rc) return rc;
  FLW_REQUIRE(amax != nullptr, FLW_E_INVALID, "null amax");
  const int64_t gx = (cols + kTT - 1) / kTT, gy = (ldt + kTT - 1) / kTT;
  const Timer tm = take_timer();
  (void)launch_args(reinterpret_cast<const void*>(&quant_tensor_t_kernel), dim3((unsigned)gx, (unsigned)gy),
                    dim3(256), 0, static_cast<hipStream_t>(stream), tm.start, tm.stop,
                    static_cast<const uint16_t*>(x), rows, cols, row_stride, amax, out8, ld8, out_t, ldt, scale_out,
                    static_cast<const uint32_t*>(nullptr), 0);
  return check_launch("flw_quant_tensor_t_e4m3_amax");
}

extern "C" int flw_quant_tensor_t_e4m3(const void* x, int64_t rows, int64_t cols, int64_t row_stride, uint8_t* out8,
                                       int64_t ld8, uint8_t* out_t, int64_t ldt, float* scale_out, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  int rc = quant_t_check(x, rows, cols, row_stride, out8, ld8, out_t, ldt, scale_out);
  if (rc) return rc;
  const size_t need = flw_quant_tensor_t_workspace_bytes(rows, cols);
  FLW_REQUIRE(workspace != nullptr && ((uintptr_t)workspace & 15) == 0 && workspace_bytes >= need, FLW_E_WORKSPACE,
              "workspace needs %zu bytes (16-byte aligned)", need);
  const int64_t gx = (cols + kTT - 1) / kTT, gy = (ldt + kTT - 1) / kTT;
  // The amax pass over the matrix as flat rows when it is contiguous (chunks of 128 such rows
  // spread over the GPU), else over its own rows.
  const int64_t fc = row_stride == cols ? tensor_t_flat_cols(rows * cols) : 0;
  const bool flat = fc != 0;
  QuantParams p{};
  const int64_t d2 = flat ? rows * cols / fc : rows, d3 = flat ? fc : cols;
  set_tensor(p.t[0], x, d2 * (flat ? fc : row_stride), d2 * (flat ? fc : row_stride), flat ? fc : row_stride, d3,
             FLW_LAYOUT_BHTD, nullptr, nullptr, nullptr);
  p.d0 = 1; p.d1 = 1; p.d2 = d2; p.d3 = d3;
  p.nchunks = nchunks_of(d2);
  uint32_t* amax = static_cast<uint32_t*>(workspace);
  p.partials = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(workspace) + 16);
  p.granularity = FLW_SCALE_TENSOR;
  FLW_REQUIRE(p.nchunks <= 0x7FFFFFFF, FLW_E_UNSUPPORTED, "matrix too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const Timer tm = take_timer();
  (void)launch_ext(reinterpret_cast<const void*>(&amax_kernel<uint16_t>), dim3((unsigned)p.nchunks, 1u, 1u),
                   dim3(kThreads), 0, s, p, tm.start, nullptr);
  // Up to kInlineFold partials every quantising workgroup folds itself; more, one workgroup first.
  const bool inline_fold = p.nchunks <= kInlineFold;
  if (!inline_fold)
    (void)launch_args(reinterpret_cast<const void*>(&amax_fold_tensor_kernel), dim3(1u), dim3(1024), 0, s, nullptr,
                      nullptr, static_cast<const uint32_t*>(p.partials), (int64_t)p.nchunks, amax);
  (void)launch_args(reinterpret_cast<const void*>(&quant_tensor_t_kernel), dim3((unsigned)gx, (unsigned)gy),
                    dim3(256), 0, s, nullptr, tm.stop, static_cast<const uint16_t*>(x), rows, cols, row_stride,
                    static_cast<const uint32_t*>(amax), out8, ld8, out_t, ldt, scale_out,
                    static_cast<const uint32_t*>(inline_fold ? p.partials : nullptr), (int)p.nchunks);
  return check_launch("flw_quant_tensor_t_e4m3");
}

extern "C" int flw_quant_cols_e4m3(const void* x, int dtype, int64_t rows, int64_t cols, int64_t row_stride,
                                   int granularity, uint8_t* out_t, int64_t ld, float* scale_out,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  FLW_REQUIRE(x != nullptr && out_t != nullptr && scale_out != nullptr, FLW_E_INVALID, "null pointer");
  FLW_REQUIRE(dtype == FLW_F32 || dtype == FLW_BF16, FLW_E_UNSUPPORTED, "dtype %d not supported", dtype);
  FLW_REQUIRE(granularity == FLW_SCALE_TENSOR || granularity == FLW_SCALE_COLUMN, FLW_E_INVALID,
              "granularity must be FLW_SCALE_TENSOR or FLW_SCALE_COLUMN");
  FLW_REQUIRE(rows > 0 && cols > 0, FLW_E_INVALID, "empty matrix");
  FLW_REQUIRE(cols % 8 == 0 && row_stride % 8 == 0 && row_stride >= cols, FLW_E_INVALID,
              "cols and row_stride must be multiples of 8");
  const int64_t esz = dtype == FLW_F32 ? 4 : 2;
  FLW_REQUIRE(((uintptr_t)x & 15) == 0 && (row_stride * esz) % 16 == 0, FLW_E_INVALID, "rows must be 16-byte aligned");
  FLW_REQUIRE(ld >= rows && ld % 16 == 0 && ((uintptr_t)out_t & 15) == 0, FLW_E_INVALID,
              "ld must be >= rows and a multiple of 16, out_t 16-byte aligned");
  const int64_t nchunks = (rows + kRT - 1) / kRT, ncb = (cols + kCT - 1) / kCT;
  const int64_t oy = (ld + kRT - 1) / kRT;
  FLW_REQUIRE(ncb <= 0x7FFFFFFF && oy <= 65535, FLW_E_UNSUPPORTED, "matrix too large");
  const size_t need = flw_quant_cols_workspace_bytes(rows, cols);
  FLW_REQUIRE(workspace != nullptr && workspace_bytes >= need, FLW_E_WORKSPACE, "workspace needs %zu bytes", need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* part = static_cast<uint32_t*>(workspace);
  const dim3 g1((unsigned)ncb, (unsigned)nchunks), g2((unsigned)ncb, (unsigned)oy);
  const bool tensor = granularity == FLW_SCALE_TENSOR;
  const Timer tm = take_timer();   // start on the amax pass, stop on the quantise pass
#define FLW_COLS(T, TEN)                                                                                   \
  do {                                                                                                     \
    const T* xt = static_cast<const T*>(x);                                                                \
    (void)launch_args(reinterpret_cast<const void*>(&cols_amax_kernel<T, TEN>), g1, dim3(kThreads), 0, s, \
                      tm.start, nullptr, xt, rows, cols, row_stride, part);                                \
    (void)launch_args(reinterpret_cast<const void*>(&cols_quant_t_kernel<T, TEN>), g2, dim3(kThreads), 0, \
                      s, nullptr, tm.stop, xt, rows, cols, row_stride, static_cast<const uint32_t*>(part), \
                      nchunks, ncb, out_t, ld, scale_out);                                                 \
  } while (0)
  if (dtype == FLW_F32) {
    if (tensor) FLW_COLS(float, true); else FLW_COLS(float, false);
  } else {
    if (tensor) FLW_COLS(uint16_t, true); else FLW_COLS(uint16_t, false);
  }
#undef FLW_COLS
  return check_launch("flw_quant_cols_e4m3");
}

template <int ACT>
static int rows_act_quant(const void* x, int64_t rows, int64_t cols, int64_t rs, const void* w, float eps,
                          uint8_t* out, float* scale_out, void* h_out, hipStream_t s, const char* name) {
  FLW_REQUIRE(x != nullptr && out != nullptr && scale_out != nullptr && (ACT != kActRmsnorm || w != nullptr),
              FLW_E_INVALID, "null pointer");
  FLW_REQUIRE(rows > 0 && cols > 0, FLW_E_INVALID, "empty matrix");
  FLW_REQUIRE(cols % 8 == 0 && rs % 8 == 0 && rs >= cols && ((uintptr_t)x & 15) == 0 &&
              ((uintptr_t)out & 7) == 0 && ((uintptr_t)h_out & 15) == 0 && ((uintptr_t)w & 15) == 0,
              FLW_E_INVALID, "rows must be 16-byte aligned multiples of 8 bf16 elements");
  FLW_REQUIRE(cols <= 4096, FLW_E_UNSUPPORTED, "rows longer than 4096 elements are not supported, got %lld",
              (long long)cols);
  FLW_REQUIRE((rows + 3) / 4 <= 0x7FFFFFFF, FLW_E_UNSUPPORTED, "too many rows");
  dim3 grid((unsigned)((rows + 3) / 4));
  const int nv = (int)((cols / 8 + 63) / 64);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* wp = static_cast<const uint16_t*>(w);
  uint16_t* hp = static_cast<uint16_t*>(h_out);
  const Timer tm = take_timer();
#define FLW_ACT_CASE(N)                                                                               \
  if (nv <= N) {                                                                                      \
    (void)launch_args(reinterpret_cast<const void*>(&rows_act_quant_kernel<ACT, N>), grid, dim3(kThreads), \
                      0, s, tm.start, tm.stop, xp, rows, (int)cols, rs, wp, eps, out, scale_out, hp); \
    return check_launch(name);                                                                        \
  }
  FLW_ACT_CASE(2) FLW_ACT_CASE(4) FLW_ACT_CASE(8)
#undef FLW_ACT_CASE
  return set_error(FLW_E_UNSUPPORTED, "%s: row too long", name);
}

extern "C" int flw_rmsnorm_quant_rows_e4m3(const void* x, int64_t rows, int64_t cols, int64_t row_stride,
                                           const void* weight, float eps, uint8_t* out, float* scale_out,
                                           void* h_out, void* stream) {
  return rows_act_quant<kActRmsnorm>(x, rows, cols, row_stride, weight, eps, out, scale_out, h_out,
                                     static_cast<hipStream_t>(stream), "flw_rmsnorm_quant_rows_e4m3");
}

extern "C" int flw_gelu_quant_rows_e4m3(const void* x, int64_t rows, int64_t cols, int64_t row_stride,
                                        uint8_t* out, float* scale_out, void* h_out, void* stream) {
  return rows_act_quant<kActGelu>(x, rows, cols, row_stride, nullptr, 0.0f, out, scale_out, h_out,
                                  static_cast<hipStream_t>(stream), "flw_gelu_quant_rows_e4m3");
}

namespace flw {

// ---------------------------------------------------------------- BHTD codes -> V tile layout
//
// For callers that hold V's e4m3 codes in plain (B, H, T, D) layout (e.g. _per_tensor_fp8's
// output): one workgroup per (b, h) slice and 64-key tile stages the tile's rows in LDS with
// 16-byte loads (keys past T read as zero), then every thread assembles whole 16-byte runs of the
// tile layout (16 keys of one dim each) from LDS bytes and stores them with 16-byte stores.
__global__ __launch_bounds__(256) void bhtd_to_vtile_kernel(const uint8_t* __restrict__ src, int64_t sb,
                                                            int64_t sh, int64_t st, int64_t H, int64_t T,
                                                            int D, uint8_t* __restrict__ dst) {
  __shared__ __align__(16) uint8_t tile[64 * 128];
  const int64_t ntiles = (T + 63) >> 6;
  const int64_t slice = blockIdx.y, tt = blockIdx.x;
  const int64_t b = slice / H, h = slice % H;
  const uint8_t* base = src + b * sb + h * sh;
  const int cpr = D / 16;                               // 16-byte chunks per key row
  for (int i = threadIdx.x; i < 64 * cpr; i += 256) {
    const int kk = i / cpr, c = i % cpr;
    const int64_t key = tt * 64 + kk;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (key < T) v = *reinterpret_cast<const uint4*>(base + key * st + 16 * c);
    *reinterpret_cast<uint4*>(tile + kk * D + 16 * c) = v;
  }
  __syncthreads();
  uint8_t* out = dst + (slice * ntiles + tt) * 64 * D;
  for (int j = threadIdx.x; j < 4 * D; j += 256) {      // 16-byte runs of the tile
    const int dblk = j >> 7, kblk = (j >> 6) & 1, hh = (j >> 5) & 1, dd = j & 31;
    const int d = 32 * dblk + dd;
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t x = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int bi = 4 * q + e;                       // byte index inside the run
        const int r = 8 * (bi >> 2) + 4 * hh + (bi & 3);
        x |= (uint32_t)tile[(32 * kblk + r) * D + d] << (8 * e);
      }
      w[q] = x;
    }
    *reinterpret_cast<uint4*>(out + 16 * j) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

}  // namespace flw

extern "C" int flw_vtile_from_bhtd(const uint8_t* codes, int64_t B, int64_t H, int64_t T, int64_t D,
                                   int64_t stride_b, int64_t stride_h, int64_t stride_t, uint8_t* v_tiles,
                                   void* stream) {
  using namespace flw;
  FLW_REQUIRE(codes != nullptr && v_tiles != nullptr, FLW_E_INVALID, "null pointer argument");
  FLW_REQUIRE(B > 0 && H > 0 && T > 0, FLW_E_INVALID, "empty shape");
  FLW_REQUIRE(D == 32 || D == 64 || D == 128, FLW_E_UNSUPPORTED, "head_dim must be 32/64/128, got %lld", (long long)D);
  FLW_REQUIRE(stride_b % 16 == 0 && stride_h % 16 == 0 && stride_t % 16 == 0 && ((uintptr_t)codes & 15) == 0 &&
              ((uintptr_t)v_tiles & 15) == 0, FLW_E_INVALID, "codes rows and v_tiles must be 16-byte aligned");
  FLW_REQUIRE(B * H <= 65535 && (T + 63) / 64 <= 0x7FFFFFFF, FLW_E_UNSUPPORTED, "B*H must be <= 65535");
  const dim3 grid((unsigned)((T + 63) / 64), (unsigned)(B * H));
  const Timer tm = take_timer();
  (void)launch_args(reinterpret_cast<const void*>(&bhtd_to_vtile_kernel), grid, dim3(256), 0,
                    static_cast<hipStream_t>(stream), tm.start, tm.stop, codes, stride_b, stride_h, stride_t, H, T,
                    (int)D, v_tiles);
  return check_launch("flw_vtile_from_bhtd");
}

// ---------------------------------------------------------------- e4m3 codes -> values
//
// The dequantised tensor a straight-through FP8 path differentiates at: out[b, h, t, d] =
// e4m3(code) * scale of its group, rounded to the output dtype (bf16: nearest even). Codes in
// (B, H, T, D) rows or in the attention kernel's V tile layout; out contiguous (B, H, T, D). The
// codes are converted by v_cvt_pk_f32_fp8 (exact: every e4m3 value is an fp32 value).
namespace flw {

// Eight values e4m3(code) * scale to OutT (bf16: round to nearest even, NaN as 0x7FC0).
template <typename OutT>
__device__ __forceinline__ void dequant8_store(uint32_t w0, uint32_t w1, float sc, OutT* dst) {
  float v[8];
  const uint32_t w[2] = {w0, w1};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], false);     // bytes 0, 1
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], true);      // bytes 2, 3
    v[4 * i] = lo[0] * sc; v[4 * i + 1] = lo[1] * sc; v[4 * i + 2] = hi[0] * sc; v[4 * i + 3] = hi[1] * sc;
  }
  if constexpr (sizeof(OutT) == 2) {
    *reinterpret_cast<uint4*>(dst) = make_uint4(bf16x2_rne(v[0], v[1]), bf16x2_rne(v[2], v[3]),
                                                bf16x2_rne(v[4], v[5]), bf16x2_rne(v[6], v[7]));
  } else {
    float4* o = reinterpret_cast<float4*>(dst);
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// (B, H, T, D) codes: one thread per 8 consecutive values (n8 < 2^31).
template <typename OutT>
__global__ __launch_bounds__(256) void dequant_bhtd_kernel(const uint8_t* __restrict__ codes, int H, int T, int D,
                                                           const float* __restrict__ scales, int ssb, int ssh,
                                                           OutT* __restrict__ out, int n8) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const int per_row = D >> 3;
  const int row = i / per_row, bh = row / T;
  const float sc = scales[(bh / H) * ssb + (bh % H) * ssh];
  const uint2 w = *reinterpret_cast<const uint2*>(codes + (int64_t)i * 8);
  dequant8_store<OutT>(w.x, w.y, sc, out + (int64_t)i * 8);
}

// The attention's V tile layout: one workgroup per 64-key tile of a (b, h) slice. The tile is
// copied to LDS as it is (runs of 16 keys, run rho = 128 (d / 32) + 64 kb + 32 hb + d % 32 for dim
// d, key block kb, half hb; byte 4 a + c of a run = key 32 kb + 8 a + 4 hb + c), then each 16-lane
// group transposes 8 consecutive runs (dims d0 .. d0 + 7) with ds_read_b64_tr_b8 -- lane 2 j + a
// supplies the address of bytes 8 a .. 8 a + 7 of run j, lane n receives byte n of the 8 runs -- so
// lane n holds dims d0 .. d0 + 7 of key 32 kb + 8 (n / 4) + 4 hb + n % 4, stored as one row piece.
template <typename OutT>
__global__ __launch_bounds__(256) void dequant_vtile_kernel(const uint8_t* __restrict__ codes, int H, int T, int D,
                                                            const float* __restrict__ scales, int ssb, int ssh,
                                                            OutT* __restrict__ out) {
  typedef int v2i __attribute__((ext_vector_type(2)));
  typedef __attribute__((address_space(3))) v2i lds_v2i;
  __shared__ __align__(16) uint8_t lt[64 * 128];
  const int ntiles = (T + 63) >> 6;
  const int bh = blockIdx.x / ntiles, tile = blockIdx.x % ntiles;
  const float sc = scales[(bh / H) * ssb + (bh % H) * ssh];
  const uint8_t* src = codes + ((int64_t)bh * ntiles + tile) * 64 * D;
  for (int i = threadIdx.x; i < 4 * D; i += 256)
    *reinterpret_cast<uint4*>(lt + 16 * i) = *reinterpret_cast<const uint4*>(src + 16 * i);
  __syncthreads();
  const int lane16 = threadIdx.x & 15, j = lane16 >> 1, a = lane16 & 1;
  const int octs = D >> 3;                      // 8-dim groups per (kb, hb)
  for (int g = threadIdx.x >> 4; g < 4 * octs; g += 16) {   // uniform per 16-lane group
    const int d0 = 8 * (g % octs), hb = (g / octs) & 1, kb = g / (2 * octs);
    const int rho0 = 128 * (d0 >> 5) + 64 * kb + 32 * hb + (d0 & 31);
    const v2i r = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(lds_u8_t*)(lt + 16 * (rho0 + j) + 8 * a));
    const int t = 64 * tile + 32 * kb + 8 * (lane16 >> 2) + 4 * hb + (lane16 & 3);
    if (t < T) dequant8_store<OutT>((uint32_t)r.x, (uint32_t)r.y, sc, out + ((int64_t)bh * T + t) * D + d0);
  }
}

}  // namespace flw

extern "C" int flw_dequant_e4m3(const uint8_t* codes, int layout, int64_t B, int64_t H, int64_t T, int64_t D,
                                const float* scales, int granularity, void* out, int out_dtype, void* stream) {
  using namespace flw;
  FLW_REQUIRE(codes != nullptr && scales != nullptr && out != nullptr, FLW_E_INVALID, "null pointer argument");
  FLW_REQUIRE(B > 0 && H > 0 && T > 0, FLW_E_INVALID, "empty shape");
  FLW_REQUIRE(D == 32 || D == 64 || D == 128, FLW_E_UNSUPPORTED, "head_dim must be 32/64/128, got %lld", (long long)D);
  FLW_REQUIRE(layout == FLW_LAYOUT_BHTD || layout == FLW_LAYOUT_VTILE, FLW_E_INVALID, "bad layout %d", layout);
  FLW_REQUIRE(out_dtype == FLW_BF16 || out_dtype == FLW_F32, FLW_E_UNSUPPORTED, "output dtype %d", out_dtype);
  FLW_REQUIRE(granularity >= FLW_SCALE_TENSOR && granularity <= FLW_SCALE_BH, FLW_E_INVALID, "bad granularity %d",
              granularity);
  FLW_REQUIRE(((uintptr_t)codes & 7) == 0 && ((uintptr_t)out & 15) == 0, FLW_E_INVALID,
              "codes must be 8-byte, out 16-byte aligned");
  const int64_t n8 = B * H * T * D / 8;
  FLW_REQUIRE(n8 < ((int64_t)1 << 31) - 256 && B * H * ((T + 63) / 64) <= 0x7FFFFFFF, FLW_E_UNSUPPORTED,
              "tensor too large");
  const int ssb = granularity == FLW_SCALE_BH ? (int)H : 0, ssh = granularity == FLW_SCALE_TENSOR ? 0 : 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf = out_dtype == FLW_BF16;
  if (layout == FLW_LAYOUT_BHTD) {
    const dim3 grid((unsigned)((n8 + 255) / 256));
    if (bf)
      hipLaunchKernelGGL(dequant_bhtd_kernel<uint16_t>, grid, dim3(256), 0, s, codes, (int)H, (int)T, (int)D, scales,
                         ssb, ssh, static_cast<uint16_t*>(out), (int)n8);
    else
      hipLaunchKernelGGL(dequant_bhtd_kernel<float>, grid, dim3(256), 0, s, codes, (int)H, (int)T, (int)D, scales,
                         ssb, ssh, static_cast<float*>(out), (int)n8);
  } else {
    FLW_REQUIRE(((uintptr_t)codes & 15) == 0, FLW_E_INVALID, "tile-layout codes must be 16-byte aligned");
    const dim3 grid((unsigned)(B * H * ((T + 63) / 64)));
    if (bf)
      hipLaunchKernelGGL(dequant_vtile_kernel<uint16_t>, grid, dim3(256), 0, s, codes, (int)H, (int)T, (int)D, scales,
                         ssb, ssh, static_cast<uint16_t*>(out));
    else
      hipLaunchKernelGGL(dequant_vtile_kernel<float>, grid, dim3(256), 0, s, codes, (int)H, (int)T, (int)D, scales,
                         ssb, ssh, static_cast<float*>(out));
  }
  return check_launch("flw_dequant_e4m3");
}

// ---------------------------------------------------------------- allocation-free QKV quantiser
//
// flw_quant_qkv_e4m3 without a workspace argument, for callers that cannot allocate (code under
// graph capture, tight serving loops): the amax partials live in a file-scope device array, one
// copy per GPU, held until the process ends. Its device address is looked up once per device
// (hipGetSymbolAddress with that device current) and only that address is handed to the kernels
// -- the array's name in host code is a host-side stand-in, not a device address. Every entry of
// the partials is written by the amax pass before the quantise pass reads it, so the array needs
// no clearing between calls; two calls that overlap on one GPU (different streams) share the
// array and race.
namespace flw {

constexpr size_t kNoAllocScratchBytes = 1u << 20;   // 262,144 amax partials
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint32_t scratch[kNoAllocScratchBytes / sizeof(uint32_t)];

static int scratch_of_stream(hipStream_t stream, void** out) {
  int dev = -1;
  if (stream != nullptr) {
    FLW_REQUIRE(hipStreamGetDevice(stream, &dev) == hipSuccess, FLW_E_LAUNCH, "hipStreamGetDevice failed");
  } else {
    FLW_REQUIRE(hipGetDevice(&dev) == hipSuccess, FLW_E_LAUNCH, "hipGetDevice failed");
  }
  FLW_REQUIRE(dev >= 0 && dev < kMaxDevices, FLW_E_UNSUPPORTED, "device %d out of range", dev);
  static void* ptrs[kMaxDevices] = {};
  static std::mutex mu;
  std::lock_guard<std::mutex> lock(mu);
  if (ptrs[dev] == nullptr) {
    int cur = -1;
    FLW_REQUIRE(hipGetDevice(&cur) == hipSuccess, FLW_E_LAUNCH, "hipGetDevice failed");
    if (cur != dev) FLW_REQUIRE(hipSetDevice(dev) == hipSuccess, FLW_E_LAUNCH, "hipSetDevice(%d) failed", dev);
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    FLW_REQUIRE(e == hipSuccess && p != nullptr, FLW_E_LAUNCH, "hipGetSymbolAddress(scratch): %s",
                hipGetErrorString(e));
    ptrs[dev] = p;
  }
  *out = ptrs[dev];
  return FLW_OK;
}

}  // namespace flw

extern "C" size_t flw_noalloc_scratch_bytes(void) { return flw::kNoAllocScratchBytes; }

extern "C" int flw_quant_qkv_e4m3_noalloc(const void* q, const void* k, const void* v, int dtype, int64_t B,
                                          int64_t H, int64_t T, int64_t D, const int64_t* strides,
                                          int granularity, uint8_t* q8, uint8_t* k8, uint8_t* v_tiles,
                                          float* scales_out, void* stream) {
  FLW_REQUIRE(strides != nullptr && scales_out != nullptr, FLW_E_INVALID, "null strides / scales");
  FLW_REQUIRE(B > 0 && H > 0 && T > 0, FLW_E_INVALID, "empty or negative shape");
  FLW_REQUIRE(B * H <= 65535 && T < ((int64_t)1 << 40), FLW_E_UNSUPPORTED, "B*H must be <= 65535");
  const size_t need = 3 * partial_bytes(B, H, T);
  FLW_REQUIRE(need <= kNoAllocScratchBytes, FLW_E_UNSUPPORTED,
              "allocation-free quantiser: 3 * B * H * ceil(T / 128) amax partials must fit its %zu-byte "
              "scratch (this shape needs %zu bytes); use flw_quant_qkv_e4m3 with a workspace",
              kNoAllocScratchBytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  const int rc = scratch_of_stream(s, &ws);
  if (rc) return rc;
  const int64_t G = granularity == FLW_SCALE_TENSOR ? 1 : (granularity == FLW_SCALE_HEAD ? H : B * H);
  const void* xs[3] = {q, k, v};
  const int layouts[3] = {FLW_LAYOUT_BHTD, FLW_LAYOUT_BHTD, FLW_LAYOUT_VTILE};
  uint8_t* outs[3] = {q8, k8, v_tiles};
  float* sc[3] = {scales_out, scales_out + G, scales_out + 2 * G};
  return quant_bhtd_n(3, xs, dtype, B, H, T, D, strides, granularity, layouts, outs, sc, ws,
                      kNoAllocScratchBytes, s, take_timer());
}
