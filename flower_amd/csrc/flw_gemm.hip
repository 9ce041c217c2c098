// Scaled FP8 GEMM for gfx950: y[M, N] (bf16) = (x8[M, K] . w8[N, K]^T) * sx[m] * sw[n].
//
// Both operands are K-contiguous e4m3 ("TN"), which is exactly what the MFMA operand registers
// want: every lane holds 32 consecutive K bytes of one row. The kernel computes the transposed
// tile C^T = W X^T so that a lane of the 32x32 accumulator owns one output row m and 16 output
// columns n in runs of 4 (8-byte bf16 stores). Workgroup tile 128 (n) x 128 (m), 4 waves in a
// 2 x 2 grid of 64 x 64 wave tiles (2 x 2 v_mfma_f32_32x32x64_f8f6f4 per 64-deep K step);
// K advances 128 per stage through double-buffered LDS in fragment order (conflict-free
// ds_read_b128), the next stage's global loads overlapping the current stage's MFMAs.
#include <type_traits>

#include "flw_common.h"

// m0 is clobbered by the direct-to-LDS loads below; nothing else here uses it.
#pragma clang diagnostic ignored "-Winline-asm"

namespace flw {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16f gemm_mfma(v8i a, v8i b, v16f c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

constexpr int kGBN = 128;   // n per workgroup (MFMA rows)
constexpr int kGBM = 128;   // m per workgroup (MFMA columns)
constexpr int kGKS = 128;   // K per LDS stage
constexpr int kTileBytes = 128 * kGKS;           // one operand tile per stage (16 KiB)
constexpr int kChunks = kTileBytes / 16;         // 1024 16-byte chunks
constexpr int kCPT = kChunks / 256;              // 4 per thread

struct GemmParams {
  const uint8_t* x8;   // [M, K]
  const uint8_t* w8;   // [N, K]
  const float* sx;     // M or 1
  const float* sw;     // N or 1
  int sx_step, sw_step;
  uint16_t* y;         // [M, N] bf16
  int64_t ys;          // row stride of y (elements)
  int M, N, K;
  int tiles_n;         // output tiles along N
  int tiles_m;         // output tiles along M
  const uint16_t* res; // optional bf16 residual [M, N] (row stride rs): y = bf16(res + bf16(..))
  int64_t rs;
  float* part;         // split-K: fp32 partial sums [splits][M][N] instead of the bf16 epilogue
  int splits;          // K ranges per output tile (1: no split)
  int lds_epi;         // epilogue staged through LDS (N % 8 == 0, 16-byte aligned y / residual rows)
  uint32_t* gmax;      // optional: max |y| (fp32 bit patterns) per group of gcols output columns
  int gcols;           // power of two in [8, 256]
  // Optional with gmax (gcols = head_dim in {32, 64, 128}): the attention's pre-quantisation
  // transform of qkv_heads applied to the output columns n < xcols (the q and k heads) before
  // they are stored and before their maxima are taken -- HeadRMSNorm when xnorm, RoPE when rcos
  // is set ([xT, gcols] bf16 tables; output row m is position m % xT).
  int xcols;           // 0: no transform
  int xnorm;
  float xeps;
  int xT;
  const uint16_t* rcos;
  const uint16_t* rsin;
};

// The epilogue value of one output: bf16(v), or bf16(residual + bf16(v)) -- x + linear(h) with
// both terms in bf16, as the reference's residual adds compute it.
__device__ __forceinline__ float epi_value(float v, const uint16_t* res, int64_t idx) {
  return res ? round_bf16(v) + __uint_as_float((uint32_t)res[idx] << 16) : v;
}

__device__ __forceinline__ v8i gfrag(const uint8_t* lds, int off) {
  const uint4 a = *reinterpret_cast<const uint4*>(lds + off);
  const uint4 b = *reinterpret_cast<const uint4*>(lds + off + 1024);
  return v8i{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
}

// Byte offset in LDS of the 16-byte chunk (row r, k = 16 g .. 16 g + 15) of a 128 x 128 tile:
// fragment (rowblk = r/32, kc = k/64), half c = (k/16)%2, lane = r%32 + 32 * ((k/32)%2).
__device__ __forceinline__ int gtile_off(int r, int g) {
  const int rowblk = r >> 5, kc = g >> 2, h = (g >> 1) & 1, c = g & 1;
  return (((rowblk * 2 + kc) * 2 + c) * 64 + (r & 31) + 32 * h) * 16;
}

__global__ __launch_bounds__(256) void fp8_gemm_kernel(GemmParams p) {
  __shared__ __align__(16) uint8_t lw[2][kTileBytes];
  __shared__ __align__(16) uint8_t lx[2][kTileBytes];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave & 1, wm = wave >> 1;
  const int tn = blockIdx.x % p.tiles_n, tm = blockIdx.x / p.tiles_n;
  const int n0 = tn * kGBN, m0 = tm * kGBM;

  uint4 rw[kCPT], rx[kCPT];
  auto load = [&](int k0) {
#pragma unroll
    for (int j = 0; j < kCPT; ++j) {
      const int i = tid + 256 * j;
      const int r = i >> 3, g = i & 7;        // 8 chunks per 128-byte row
      const int k = k0 + 16 * g;
      const int n = n0 + r, m = m0 + r;
      rw[j] = (n < p.N && k < p.K) ? *reinterpret_cast<const uint4*>(p.w8 + (int64_t)n * p.K + k)
                                   : make_uint4(0, 0, 0, 0);
      rx[j] = (m < p.M && k < p.K) ? *reinterpret_cast<const uint4*>(p.x8 + (int64_t)m * p.K + k)
                                   : make_uint4(0, 0, 0, 0);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int j = 0; j < kCPT; ++j) {
      const int i = tid + 256 * j;
      const int off = gtile_off(i >> 3, i & 7);
      *reinterpret_cast<uint4*>(&lw[buf][off]) = rw[j];
      *reinterpret_cast<uint4*>(&lx[buf][off]) = rx[j];
    }
  };

  v16f acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = v16f{};

  load(0);
  store(0);
  __syncthreads();
  const int nstages = (p.K + kGKS - 1) / kGKS;
  for (int s = 0; s < nstages; ++s) {
    const int buf = s & 1;
    const bool more = s + 1 < nstages;
    if (more) load((s + 1) * kGKS);
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      v8i a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        a[i] = gfrag(lw[buf], (((2 * wn + i) * 2 + kc) * 2 * 64 + lane) * 16);
        b[i] = gfrag(lx[buf], (((2 * wm + i) * 2 + kc) * 2 * 64 + lane) * 16);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = gemm_mfma(a[i], b[j], acc[i][j]);
    }
    if (more) store(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: lane owns m = m0 + 64 wm + 32 j + lane%32 and n = n0 + 64 wn + 32 i + 8 g + 4 hh + 0..3
  const int hh = lane >> 5;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int m = m0 + 64 * wm + 32 * j + (lane & 31);
    if (m >= p.M) continue;
    const float sxm = p.sx[(int64_t)m * p.sx_step];
    uint16_t* yrow = p.y + (int64_t)m * p.ys;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + 64 * wn + 32 * i + 8 * g + 4 * hh;
        if (n >= p.N) continue;      // N % 4 == 0 is required on the host
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = epi_value(acc[i][j][4 * g + e] * sxm * p.sw[(int64_t)(n + e) * p.sw_step], p.res,
                           (int64_t)m * p.rs + n + e);
        uint2 w;
        w.x = f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16);
        w.y = f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16);
        *reinterpret_cast<uint2*>(yrow + n) = w;
      }
    }
  }
}

// ---------------------------------------------------------------- 256 x 256 tile, direct-to-LDS
//
// For K % 64 == 0 (every model shape; K % 128 == 64 ends on a 64-deep stage). Workgroup tile
// 256 (n) x 256 (m), 8 waves (two per SIMD)
// in a 2 x 4 grid of 128 (n) x 64 (m) wave tiles: per 64-deep K chunk a wave reads 4 + 2
// fragments (12 KB of LDS) for 8 v_mfma_f32_32x32x64_f8f6f4 (512 MFMA cycles), and the two waves
// of a SIMD interleave one's LDS reads with the other's MFMAs.
// Operand tiles move global -> LDS with global_load_lds_dwordx4 (no staging registers), 128 K
// bytes of each row per stage so that one instruction reads 8 whole 128-byte lines (8 lanes per
// row). In LDS a tile is row-major, 128 bytes per row, with the 16-byte chunk c of row r stored
// at position c ^ ((r >> 1) & 7): a lane's DMA slot is fixed (base + 16 lane), so the swizzle is
// applied by choosing which global chunk each lane fetches, and it makes the fragment reads (16
// consecutive rows, one chunk each) hit 16 distinct bank groups. Two LDS stages of 64 KB, one
// barrier per stage. Rows past M / N load a clamped valid row (their outputs are not stored).
constexpr int kFBN = 256, kFBM = 256, kFBK = 128;
constexpr int kFThreads = 512;
constexpr int kGroupM = 4;                        // m-tiles per tile group (L2 locality)
constexpr int kFOpBytes = 256 * kFBK;             // one operand tile per stage (32 KB)
constexpr int kFStageBytes = 2 * kFOpBytes;       // W tile then X tile

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{a, b}), bf16x2_t));
}

// Byte offset of chunk c (16 bytes) of row r in a swizzled 128-byte-row tile.
__device__ __forceinline__ int swz_off(int r, int c) { return r * 128 + 16 * (c ^ ((r >> 1) & 7)); }

// A 32 x 64 MFMA fragment of row block rb, K chunk kc: lane (row 32 rb + lane % 32, half h)
// takes the 32 bytes at K offset 64 kc + 32 h.
__device__ __forceinline__ v8i swz_frag(const uint8_t* tile, int rb, int kc, int lane) {
  const int r = 32 * rb + (lane & 31), c = 4 * kc + 2 * (lane >> 5);
  const uint4 a = *reinterpret_cast<const uint4*>(tile + swz_off(r, c));
  const uint4 b = *reinterpret_cast<const uint4*>(tile + swz_off(r, c + 1));
  return v8i{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
}

// Epilogue staged through LDS, shared by the 256 x 256 kernels (the stage buffers are free after
// the K loop, whose last step ends with a barrier): the scaled bf16 tile, 256 rows x 512 bytes,
// rows 0-127 in st0 and 128-255 in st1 (64 KB each), 16-byte chunk c of row r at c ^ (r & 31);
// then every wave stores whole row segments with 16-byte stores (a full 512-byte row per 32
// lanes) instead of 8-byte pieces of 32 rows, and adds the optional residual row-wise.
// Wave layout of acc (wave = 2 wm + wn): lane owns m = 64 wm + 32 j + lane % 32 and
// n = 128 wn + 32 i + 8 g + 4 (lane / 32) + 0..3. Needs N % 8 == 0 and 16-byte aligned rows.
// With gmax, the max |y| over the tile's rows for each group of gcols columns (the per-head amax of
// a QKV projection, gcols = head_dim) is reduced in the workgroup and folded into gmax with one
// atomic max per group and tile (bit patterns of non-negative floats order as unsigned integers).
//
// XD > 0 (= gcols, the head dim): the q / k transform of xf on the columns n < xf->xcols. A tile
// holding such columns is read head-major: lane = XD / 8 lanes per head row (its 8 columns at
// d = 8 (lane % (XD / 8))) x 512 / XD rows, each lane taking the same d of every head in the tile
// for its row, so one load of the row's RoPE table entries serves all 256 / XD heads (the tables
// are shared by every head of a position). The table loads of the next row batch are issued
// before the current batch is transformed, the first batch's before the staging.
template <int XD = 0>
__device__ __forceinline__ void staged_epilogue(const v16f (&acc)[4][2], const float (&sxm)[2], const float* sw,
                                                int sw_step, uint16_t* y, int64_t ys, const uint16_t* res,
                                                int64_t rs, int M, int N, uint8_t* st0, uint8_t* st1, int m0,
                                                int n0, int wave, int lane_id, uint32_t* gmax = nullptr,
                                                int gcols = 0, const GemmParams* xf = nullptr) {
  // In the transform instances the lane id reaches the epilogue through an opaque copy, so the LDS
  // addresses derived from it are computed per tile instead of being hoisted out of the tile loop
  // into registers held through every K loop (where they spilled and slowed the K loop).
  int lane = lane_id;
  if constexpr (XD > 0) asm volatile("" : "+v"(lane));
  constexpr int LPR = XD > 0 ? XD / 8 : 1;        // lanes per head row
  constexpr int RPP = 64 / LPR;                   // rows per batch
  constexpr int NB = XD > 0 ? 32 / RPP : 1;       // batches over the wave's 32 rows
  constexpr int HPT = XD > 0 ? 256 / XD : 1;      // heads per tile
  const bool xform = XD > 0 && n0 < xf->xcols;    // uniform
  const bool rope = XD > 0 && xform && xf->rcos != nullptr;
  // The head-major lane coordinates are recomputed in every epilogue: derived from an opaque copy
  // of the lane id, they and the LDS / table addresses built on them cannot be hoisted out of the
  // tile loop, where they would hold registers (or scratch) through every K loop.
  int xl = lane;
  if constexpr (XD > 0) asm volatile("" : "+v"(xl));
  const int xsub = xl / LPR, xdc = xl % LPR;
  // Table entries (8 columns from d = 8 xdc) of batch b's row; rows past M use the last row's.
  auto xtab = [&](int b, uint4& c, uint4& s) __attribute__((always_inline)) {
    const int m = min(m0 + 32 * wave + RPP * b + xsub, M - 1);
    const int64_t off = (int64_t)((uint32_t)m % (uint32_t)xf->xT) * XD + 8 * xdc;
    c = *reinterpret_cast<const uint4*>(xf->rcos + off);
    s = *reinterpret_cast<const uint4*>(xf->rsin + off);
  };
  uint4 tc = make_uint4(0, 0, 0, 0), tsn = tc;
  if (rope) xtab(0, tc, tsn);

  const int wn = wave & 1, wm = wave >> 1, hh = lane >> 5;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float swn[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = min(n0 + 128 * wn + 32 * i + 8 * g + 4 * hh, N - 4);
      if (sw_step) {
        const float4 v = *reinterpret_cast<const float4*>(sw + n);
        swn[4 * g] = v.x; swn[4 * g + 1] = v.y; swn[4 * g + 2] = v.z; swn[4 * g + 3] = v.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) swn[4 * g + e] = sw[0];
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int r = 64 * wm + 32 * j + (lane & 31);
      uint8_t* rowp = (r < 128 ? st0 : st1) + (r & 127) * 512;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const v16f& c = acc[i][j];
        const int ch = 16 * wn + 4 * i + g;      // 16-byte chunk (8 n) of the row
        uint2 w;
        w.x = pack_bf16x2(c[4 * g] * sxm[j] * swn[4 * g], c[4 * g + 1] * sxm[j] * swn[4 * g + 1]);
        w.y = pack_bf16x2(c[4 * g + 2] * sxm[j] * swn[4 * g + 2], c[4 * g + 3] * sxm[j] * swn[4 * g + 3]);
        *reinterpret_cast<uint2*>(rowp + 16 * (ch ^ (r & 31)) + 8 * hh) = w;
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);           // lgkmcnt(0)
  lds_barrier();
  // Stores chunk ch (8 columns) of tile row r, with the residual; mx takes its max |y| bf16 bits
  // (per 16-bit half).
  auto store_at = [&](int r, int ch, uint4 v, flw_u16x2& mx) __attribute__((always_inline)) {
    const int m = m0 + r, n = n0 + 8 * ch;
    if (m < M && n < N) {
      uint4 o = v;
      if (res) {
        const uint4 rr = *reinterpret_cast<const uint4*>(res + (int64_t)m * rs + n);
        const uint32_t a[4] = {v.x, v.y, v.z, v.w}, b[4] = {rr.x, rr.y, rr.z, rr.w};
        uint32_t ov[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          ov[e] = pack_bf16x2(__uint_as_float(a[e] << 16) + __uint_as_float(b[e] << 16),
                              __uint_as_float(a[e] & 0xFFFF0000u) + __uint_as_float(b[e] & 0xFFFF0000u));
        o = make_uint4(ov[0], ov[1], ov[2], ov[3]);
      }
      *reinterpret_cast<uint4*>(y + (int64_t)m * ys + n) = o;
      if (gmax) {
        mx = abs_max_bf16x2(mx, o.x);
        mx = abs_max_bf16x2(mx, o.y);
        mx = abs_max_bf16x2(mx, o.z);
        mx = abs_max_bf16x2(mx, o.w);
      }
    }
  };
  auto staged_at = [&](int r, int ch) __attribute__((always_inline)) {
    return *reinterpret_cast<const uint4*>((r < 128 ? st0 : st1) + (r & 127) * 512 + 16 * (ch ^ (r & 31)));
  };
  flw_u16x2 lm = {0, 0};                          // max |y| bf16 bits of this lane's chunks
  flw_u16x2 lmh[HPT];                             // head-major: per head of the tile
#pragma unroll
  for (int h = 0; h < HPT; ++h) lmh[h] = flw_u16x2{0, 0};
  if (XD > 0 && xform) {
    // One row batch: the transform of every q / k head of the tile on its 8 columns, with the
    // pair converter (HW) or the exact software rounding, chosen once for the batch.
    auto batch = [&](auto hw, int r, const uint4 (&v)[HPT], const float* cf, const float* sf)
        __attribute__((always_inline)) {
#pragma unroll
      for (int h = 0; h < HPT; ++h) {
        const int nh = n0 + h * XD;               // uniform
        if (nh >= N) break;
        uint4 o = v[h];
        if (nh < xf->xcols) {
          float f[8];
          Vec16<uint16_t>::unpack(o, f);
          uint32_t pk[4] = {o.x, o.y, o.z, o.w};
          head_norm_rope_core<uint16_t, decltype(hw)::value>(f, xf->xnorm != 0, xf->xeps, XD, LPR, true, rope,
                                                             cf, sf, pk);
          o = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        }
        store_at(r, h * LPR + xdc, o, lmh[h]);
      }
    };
#pragma unroll 1
    for (int b = 0; b < NB; ++b) {
      uint4 nc = tc, ns = tsn;
      if (rope && b + 1 < NB) xtab(b + 1, nc, ns);
      const int r = 32 * wave + RPP * b + xsub;
      uint4 v[HPT];
      flw_u16x2 fm = {0, 0};                      // max |x| of the values transformed
#pragma unroll
      for (int h = 0; h < HPT; ++h) {
        v[h] = staged_at(r, h * LPR + xdc);
        if (n0 + h * XD < min(N, xf->xcols)) {
          fm = abs_max_bf16x2(fm, v[h].x);
          fm = abs_max_bf16x2(fm, v[h].y);
          fm = abs_max_bf16x2(fm, v[h].z);
          fm = abs_max_bf16x2(fm, v[h].w);
        }
      }
      float cf[8] = {}, sf[8] = {};
      if (rope) {
        Vec16<uint16_t>::unpack(tc, cf);
        Vec16<uint16_t>::unpack(tsn, sf);
      }
      // The pair converter only where no NaN can arise: every input finite, eps > 0.
      const bool bad = (fm[0] > fm[1] ? fm[0] : fm[1]) >= 0x7F80u || (xf->xnorm != 0 && !(xf->xeps > 0.0f));
      if (__builtin_amdgcn_ballot_w64(bad) == 0)
        batch(std::true_type{}, r, v, cf, sf);
      else
        batch(std::false_type{}, r, v, cf, sf);
      tc = nc;
      tsn = ns;
    }
  } else {
    // Wave w stores rows 32 w .. 32 w + 31, two rows (2 x 512 bytes) per instruction.
#pragma unroll 4
    for (int q = 0; q < 16; ++q) {
      const int r = 32 * wave + 2 * q + (lane >> 5), ch = lane & 31;
      store_at(r, ch, staged_at(r, ch), lm);
    }
  }
  // The next tile's loads refill st0 / st1: every wave's reads of the staged tile are done.
  __builtin_amdgcn_s_waitcnt(0xC07F);           // lgkmcnt(0)
  lds_barrier();
  if (gmax) {
    uint32_t* red = reinterpret_cast<uint32_t*>(st0);          // [8 waves][32 groups at most]
    if (XD > 0 && xform) {
      // Every lane of the wave holds rows of every head: the wave's max per head.
#pragma unroll
      for (int h = 0; h < HPT; ++h) {
        uint32_t v = lmh[h][0] > lmh[h][1] ? lmh[h][0] : lmh[h][1];
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const uint32_t t = (uint32_t)__shfl_xor((int)v, o, 64);
          v = v > t ? v : t;
        }
        if (lane == 0) red[wave * 32 + h] = v;
      }
    } else {
      // Lanes ch .. ch + gcols / 8 - 1 of each half-wave cover one group's columns.
      const int lpg = gcols >> 3;
      uint32_t lmx = lm[0] > lm[1] ? lm[0] : lm[1];
      for (int o = 1; o < lpg; o <<= 1) {
        const uint32_t t = (uint32_t)__shfl_xor((int)lmx, o, 64);
        lmx = lmx > t ? lmx : t;
      }
      const uint32_t t = (uint32_t)__shfl_xor((int)lmx, 32, 64);
      lmx = lmx > t ? lmx : t;
      const int ch = lane & 31;
      if (lane < 32 && (ch & (lpg - 1)) == 0) red[wave * 32 + ch / lpg] = lmx;
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    lds_barrier();
    const int ngr = 256 / gcols, tid = wave * 64 + lane;
    if (tid < ngr && n0 + tid * gcols < N) {
      uint32_t mx = 0;
#pragma unroll
      for (int w = 0; w < 8; ++w) mx = mx > red[w * 32 + tid] ? mx : red[w * 32 + tid];
      atomicMax(gmax + (n0 / gcols) + tid, mx << 16);     // bf16 bits -> fp32 bits
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    lds_barrier();
  }
}

// One 256 x 256 output tile: K loop over two LDS stages, then the scaled bf16 epilogue.
template <int XD = 0, bool HALFK = false>
__device__ __forceinline__ void gemm_tile(const GemmParams& p, uint8_t* st0, uint8_t* st1, int m0,
                                          int n0, int wave, int lane, int sbase, int nst, int split) {
  const int wn = wave & 1, wm = wave >> 1;        // 128 n rows, 64 m columns
  // Loads: a stage is 2 x 256 rows x 128 bytes = 512 rows; wave w fills rows 64 w .. 64 w + 63
  // (waves 0-3: W, 4-7: X) with 8 instructions of 8 rows each. Lane i of instruction t covers
  // row 8 t + i / 8 of the wave's range, LDS position i % 8, i.e. global chunk (i % 8) ^ swz.
  const int op = wave >> 2;                       // uniform
  const uint8_t* gsrc = op == 0 ? p.w8 : p.x8;
  uint32_t goff[8];
  uint32_t hi_half = 0;                           // bit t: instruction t's chunk is in bytes 64-127
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int r = 64 * (wave & 3) + 8 * t + (lane >> 3);      // row within the operand tile
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    const int grow = op == 0 ? min(n0 + r, p.N - 1) : min(m0 + r, p.M - 1);
    goff[t] = (uint32_t)grow * (uint32_t)p.K + 16u * (uint32_t)c;
    hi_half |= (uint32_t)(c >> 2) << t;
  }
  // K % 128 == 64: the range's last stage holds 64 K bytes; its lanes for bytes 64-127 load
  // bytes 0-63 again (in bounds; that half of the stage is never read). Instances of their own
  // (HALFK), so that the K % 128 == 0 kernels keep their code.
  const bool half_last = HALFK && sbase + nst == (p.K + kFBK - 1) / kFBK;
  const int lbase = op * kFOpBytes + (64 * (wave & 3)) * 128;
  // Issued from inline assembly: the compiler then does not track these LDS writes and does not
  // drain the prefetch before every fragment read; the kernel orders them itself (an explicit
  // vmcnt wait for this wave's loads, then a workgroup barrier, before a stage is read).
  auto issue = [&](uint8_t* stage, int s) __attribute__((always_inline)) {
    const uint32_t k0 = (uint32_t)(sbase + s) * kFBK;
    const uint32_t back = half_last && s == nst - 1 ? 64u : 0u;
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_u8_t*)(stage + lbase);
#pragma unroll
    for (int t = 0; t < 8; ++t)
      asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                   :: "s"(lds + t * 1024), "v"(goff[t] + k0 - (((hi_half >> t) & 1u) ? back : 0u)), "s"(gsrc)
                   : "memory", "m0");
  };

  v16f acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v16f{};

  issue(st0, 0);

  // Stage s in `cur`: prefetch stage s+1 into `nxt` (its readers finished at the end of step
  // s-1, before the barrier below was passed by everyone... see the barrier at the step's end),
  // wait for stage s, publish it, then two K chunks of fragments + MFMAs.
  auto step = [&](int s, const uint8_t* cur, uint8_t* nxt) __attribute__((always_inline)) {
    if (s + 1 < nst) {
      issue(nxt, s + 1);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(8));   // this wave's loads of stage s landed
    } else {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    }
    lds_barrier();                                // ... and every wave's
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      if (kc == 1 && half_last && s == nst - 1) break;      // a 64-deep last stage
      v8i a[4], b[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = swz_frag(cur, 4 * wn + i, kc, lane);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = swz_frag(cur + kFOpBytes, 2 * wm + j, kc, lane);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = gemm_mfma(a[i], b[j], acc[i][j]);
    }
    // Everyone's fragment reads of `cur` are done before anyone refills it (next step + 1).
    __builtin_amdgcn_s_waitcnt(0xC07F);           // lgkmcnt(0)
    lds_barrier();
  };
  for (int s = 0; s < nst; s += 2) {
    step(s, st0, st1);
    if (s + 1 < nst) step(s + 1, st1, st0);
  }

  // Epilogue: lane owns m = m0 + 64 wm + 32 j + lane % 32, n = n0 + 128 wn + 32 i + 8 g + 4 hh + 0..3
  const int hh = lane >> 5;
  if (p.part) {                                   // split-K: unscaled fp32 partials, 16-byte stores
    float* base = p.part + (int64_t)split * p.M * p.N;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int m = m0 + 64 * wm + 32 * j + (lane & 31);
        if (m >= p.M) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + 128 * wn + 32 * i + 8 * g + 4 * hh;
          if (n >= p.N) continue;
          const v16f& c = acc[i][j];
          *reinterpret_cast<float4*>(base + (int64_t)m * p.N + n) =
              make_float4(c[4 * g], c[4 * g + 1], c[4 * g + 2], c[4 * g + 3]);
        }
      }
    return;
  }
  if (p.lds_epi) {
    float sxm[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int m = min(m0 + 64 * wm + 32 * j + (lane & 31), p.M - 1);
      sxm[j] = p.sx[(int64_t)m * p.sx_step];
    }
    staged_epilogue<XD>(acc, sxm, p.sw, p.sw_step, p.y, p.ys, p.res, p.rs, p.M, p.N, st0, st1, m0, n0, wave,
                        lane, p.gmax, p.gcols, XD > 0 ? &p : nullptr);
    return;
  }
  float sxm[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int m = min(m0 + 64 * wm + 32 * j + (lane & 31), p.M - 1);
    sxm[j] = p.sx[(int64_t)m * p.sx_step];
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float swn[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = min(n0 + 128 * wn + 32 * i + 8 * g + 4 * hh, p.N - 4);
      if (p.sw_step) {
        const float4 v = *reinterpret_cast<const float4*>(p.sw + n);
        swn[4 * g] = v.x; swn[4 * g + 1] = v.y; swn[4 * g + 2] = v.z; swn[4 * g + 3] = v.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) swn[4 * g + e] = p.sw[0];
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int m = m0 + 64 * wm + 32 * j + (lane & 31);
      if (m >= p.M) continue;
      uint16_t* yrow = p.y + (int64_t)m * p.ys;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + 128 * wn + 32 * i + 8 * g + 4 * hh;
        if (n >= p.N) continue;      // N % 4 == 0 is required on the host
        const v16f& c = acc[i][j];
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = c[4 * g + e] * sxm[j] * swn[4 * g + e];
        if (p.res) {
          const uint2 r = *reinterpret_cast<const uint2*>(p.res + (int64_t)m * p.rs + n);
          v[0] = round_bf16(v[0]) + __uint_as_float(r.x << 16);
          v[1] = round_bf16(v[1]) + __uint_as_float(r.x & 0xFFFF0000u);
          v[2] = round_bf16(v[2]) + __uint_as_float(r.y << 16);
          v[3] = round_bf16(v[3]) + __uint_as_float(r.y & 0xFFFF0000u);
        }
        uint2 w;
        w.x = pack_bf16x2(v[0], v[1]);
        w.y = pack_bf16x2(v[2], v[3]);
        *reinterpret_cast<uint2*>(yrow + n) = w;
      }
    }
  }
}

// One 256 (n) x 128 (m) output tile (or its K range under split-K), for outputs with fewer
// 256 x 256 tiles than compute units (twice the tiles, so the grid covers more of the GPU): 8 waves in a 4 x 2 grid of 64 x 64 wave tiles
// (2 x 2 MFMAs per 64-deep K chunk), a stage holding the 256 W rows and 128 X rows (48 of its
// 64 KB), the same swizzle, barriers and accumulation order as gemm_tile (the results are
// identical), and the epilogue staged through st0 (128 rows x 512 bytes).
template <bool HALFK = false>
__device__ __forceinline__ void gemm_tile_128(const GemmParams& p, uint8_t* st0, uint8_t* st1, int m0,
                                              int n0, int wave, int lane, int sbase, int nst, int split) {
  const int wn = wave & 3, wm = wave >> 2;        // 64 n rows, 64 m columns
  // Loads: 384 rows of 128 bytes per stage; wave w fills rows 48 w .. 48 w + 47 with 6
  // instructions of 8 rows, rows 256 .. 383 being X rows 0 .. 127. Instruction t of a wave reads
  // one operand (256 is a multiple of 8), so its base address is a scalar.
  uint32_t goff[6];
  uint32_t hi_half = 0;                           // bit t: instruction t's chunk is in bytes 64-127
#pragma unroll
  for (int t = 0; t < 6; ++t) {
    const int row0 = 48 * wave + 8 * t;
    const bool xop = row0 >= 256;
    const int r = (xop ? row0 - 256 : row0) + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    const int grow = xop ? min(m0 + r, p.M - 1) : min(n0 + r, p.N - 1);
    goff[t] = (uint32_t)grow * (uint32_t)p.K + 16u * (uint32_t)c;
    hi_half |= (uint32_t)(c >> 2) << t;
  }
  const bool half_last = HALFK && sbase + nst == (p.K + kFBK - 1) / kFBK;
  auto issue = [&](uint8_t* stage, int s) __attribute__((always_inline)) {
    const uint32_t k0 = (uint32_t)(sbase + s) * kFBK;
    const uint32_t back = half_last && s == nst - 1 ? 64u : 0u;
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_u8_t*)stage;
#pragma unroll
    for (int t = 0; t < 6; ++t) {
      const int row0 = 48 * wave + 8 * t;
      const bool xop = row0 >= 256;
      const uint32_t dst = lds + (xop ? kFOpBytes + (row0 - 256) * 128 : row0 * 128);
      const uint8_t* src = xop ? p.x8 : p.w8;
      asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                   :: "s"(dst), "v"(goff[t] + k0 - (((hi_half >> t) & 1u) ? back : 0u)), "s"(src)
                   : "memory", "m0");
    }
  };

  v16f acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v16f{};

  issue(st0, 0);
  auto step = [&](int s, const uint8_t* cur, uint8_t* nxt) __attribute__((always_inline)) {
    if (s + 1 < nst) {
      issue(nxt, s + 1);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(6));   // this wave's loads of stage s landed
    } else {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    }
    lds_barrier();                                // ... and every wave's
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      if (kc == 1 && half_last && s == nst - 1) break;      // a 64-deep last stage
      v8i a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = swz_frag(cur, 2 * wn + i, kc, lane);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = swz_frag(cur + kFOpBytes, 2 * wm + j, kc, lane);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = gemm_mfma(a[i], b[j], acc[i][j]);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);           // lgkmcnt(0)
    lds_barrier();
  };
  for (int s = 0; s < nst; s += 2) {
    step(s, st0, st1);
    if (s + 1 < nst) step(s + 1, st1, st0);
  }

  // Epilogue: lane owns m = m0 + 64 wm + 32 j + lane % 32, n = n0 + 64 wn + 32 i + 8 g + 4 hh + 0..3;
  // the scaled bf16 tile goes to st0 (row r = m - m0, 16-byte chunk c at c ^ (r & 31)), then
  // wave w stores rows 16 w .. 16 w + 15, two 512-byte rows per instruction. Split-K: unscaled
  // fp32 partials, 16-byte stores.
  const int hh = lane >> 5;
  if (p.part) {
    float* base = p.part + (int64_t)split * p.M * p.N;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int m = m0 + 64 * wm + 32 * j + (lane & 31);
        if (m >= p.M) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + 64 * wn + 32 * i + 8 * g + 4 * hh;
          if (n >= p.N) continue;
          const v16f& c = acc[i][j];
          *reinterpret_cast<float4*>(base + (int64_t)m * p.N + n) =
              make_float4(c[4 * g], c[4 * g + 1], c[4 * g + 2], c[4 * g + 3]);
        }
      }
    return;
  }
  float sxm[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int m = min(m0 + 64 * wm + 32 * j + (lane & 31), p.M - 1);
    sxm[j] = p.sx[(int64_t)m * p.sx_step];
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float swn[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = min(n0 + 64 * wn + 32 * i + 8 * g + 4 * hh, p.N - 4);
      if (p.sw_step) {
        const float4 v = *reinterpret_cast<const float4*>(p.sw + n);
        swn[4 * g] = v.x; swn[4 * g + 1] = v.y; swn[4 * g + 2] = v.z; swn[4 * g + 3] = v.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) swn[4 * g + e] = p.sw[0];
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int r = 64 * wm + 32 * j + (lane & 31);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const v16f& c = acc[i][j];
        const int ch = 8 * wn + 4 * i + g;
        uint2 w;
        w.x = pack_bf16x2(c[4 * g] * sxm[j] * swn[4 * g], c[4 * g + 1] * sxm[j] * swn[4 * g + 1]);
        w.y = pack_bf16x2(c[4 * g + 2] * sxm[j] * swn[4 * g + 2], c[4 * g + 3] * sxm[j] * swn[4 * g + 3]);
        *reinterpret_cast<uint2*>(st0 + r * 512 + 16 * (ch ^ (r & 31)) + 8 * hh) = w;
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);             // lgkmcnt(0)
  lds_barrier();
#pragma unroll 4
  for (int q = 0; q < 8; ++q) {
    const int r = 16 * wave + 2 * q + (lane >> 5), ch = lane & 31;
    const int m = m0 + r, n = n0 + 8 * ch;
    const uint4 v = *reinterpret_cast<const uint4*>(st0 + r * 512 + 16 * (ch ^ (r & 31)));
    if (m < p.M && n < p.N) {
      uint4 o = v;
      if (p.res) {
        const uint4 rr = *reinterpret_cast<const uint4*>(p.res + (int64_t)m * p.rs + n);
        const uint32_t a[4] = {v.x, v.y, v.z, v.w}, b[4] = {rr.x, rr.y, rr.z, rr.w};
        uint32_t ov[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          ov[e] = pack_bf16x2(__uint_as_float(a[e] << 16) + __uint_as_float(b[e] << 16),
                              __uint_as_float(a[e] & 0xFFFF0000u) + __uint_as_float(b[e] & 0xFFFF0000u));
        o = make_uint4(ov[0], ov[1], ov[2], ov[3]);
      }
      *reinterpret_cast<uint4*>(p.y + (int64_t)m * p.ys + n) = o;
    }
  }
  // The next tile's loads refill st0: every wave's reads of the staged tile are done.
  __builtin_amdgcn_s_waitcnt(0xC07F);
  lds_barrier();
}

// XD > 0: the q / k transform epilogue of flw_fp8_scaled_mm_qk_norm_rope_amax for head dim XD,
// compiled as instances of their own so that the other GEMMs keep their register allocation.
template <int TM, int XD = 0, bool HALFK = false>
__global__ __launch_bounds__(kFThreads, 1) void fp8_gemm_256_kernel(GemmParams p) {
  // One array per stage: every LDS access below names its stage at compile time, so the
  // compiler can see that the direct-to-LDS loads in flight write the other stage.
  __shared__ __align__(16) uint8_t st0[kFStageBytes];
  __shared__ __align__(16) uint8_t st1[kFStageBytes];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // Persistent over tiles: workgroup b takes tiles L, L + G, L + 2G, ... (G = grid size), so
  // the output stores of one tile drain while the next tile computes. L = (b % 8) (G / 8) + b / 8
  // gives the G/8 workgroups of XCD b % 8 consecutive tile numbers, and tiles are numbered in
  // groups of kGroupM m-tiles (m fastest): the 32 tiles an XCD runs at once are a 4 x 8 block
  // whose operands (3 MB) stay in its 4 MB L2.
  const int G = gridDim.x;
  const int L = (G & 7) == 0 ? (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int ntiles = p.tiles_n * p.tiles_m;

  // Split-K: work item t = split * ntiles + tile; split s covers K stages [s nst / S, (s+1) nst / S).
  const int nst_all = (p.K + kFBK - 1) / kFBK;     // the last one 64 deep when K % 128 == 64
  for (int t = L; t < ntiles * p.splits; t += G) {
    const int split = t / ntiles, tt = t % ntiles;
    const int group = tt / (kGroupM * p.tiles_n);
    const int first_m = group * kGroupM;
    const int gm = min(p.tiles_m - first_m, kGroupM);
    const int tm = first_m + (tt % (kGroupM * p.tiles_n)) % gm;
    const int tn = (tt % (kGroupM * p.tiles_n)) / gm;
    const int s0 = split * nst_all / p.splits, s1 = (split + 1) * nst_all / p.splits;
    if constexpr (TM == 256) gemm_tile<XD, HALFK>(p, st0, st1, tm * kFBM, tn * kFBN, wave, lane, s0, s1 - s0, split);
    else gemm_tile_128<HALFK>(p, st0, st1, tm * TM, tn * kFBN, wave, lane, s0, s1 - s0, split);
  }
}

// Split-K finish: y[m, n..n+3] = bf16( (sum_s part[s][m][n]) * sx[m] * sw[n] ) (+ residual as in
// the one-pass epilogue); one thread per 4 outputs.
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(GemmParams p) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_row = p.N / 4;
  if (q >= (int64_t)p.M * per_row) return;
  const int m = (int)(q / per_row), n = (int)(q % per_row) * 4;
  float4 a = *reinterpret_cast<const float4*>(p.part + (int64_t)m * p.N + n);
  for (int sp = 1; sp < p.splits; ++sp) {
    const float4 b = *reinterpret_cast<const float4*>(p.part + ((int64_t)sp * p.M + m) * p.N + n);
    a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
  }
  const float sx = p.sx[(int64_t)m * p.sx_step];
  const float sw[4] = {p.sw[(int64_t)n * p.sw_step], p.sw[(int64_t)(n + 1) * p.sw_step],
                       p.sw[(int64_t)(n + 2) * p.sw_step], p.sw[(int64_t)(n + 3) * p.sw_step]};
  float v[4] = {a.x * sx * sw[0], a.y * sx * sw[1], a.z * sx * sw[2], a.w * sx * sw[3]};
  if (p.res) {
    const uint2 r = *reinterpret_cast<const uint2*>(p.res + (int64_t)m * p.rs + n);
    v[0] = round_bf16(v[0]) + __uint_as_float(r.x << 16);
    v[1] = round_bf16(v[1]) + __uint_as_float(r.x & 0xFFFF0000u);
    v[2] = round_bf16(v[2]) + __uint_as_float(r.y << 16);
    v[3] = round_bf16(v[3]) + __uint_as_float(r.y & 0xFFFF0000u);
  }
  uint2 w;
  w.x = pack_bf16x2(v[0], v[1]);
  w.y = pack_bf16x2(v[2], v[3]);
  *reinterpret_cast<uint2*>(p.y + (int64_t)m * p.ys + n) = w;
}

// ---------------------------------------------------------------- W8A16: e4m3 weights x bf16 activations
//
// y[M, N] (bf16) = (x[M, K] . w8[N, K]^T) * sw[n] with x in bf16, unquantised. The weight codes are
// widened to bf16 in registers (v_cvt_scalef32_pk_bf16_fp8, exact: every e4m3 value is a bf16
// value) and the product runs on v_mfma_f32_32x32x16_bf16 (bf16 dense peak 2.5 PFLOP/s). Same
// persistent 256 x 256 tiles, wave grid, XCD / group-M tile order and direct-to-LDS staging as
// the FP8 kernel; a stage is 64 deep in K: a 256 x 128-byte X tile (bf16) and a 256 x 64-byte W
// tile (e4m3), 48 KB, in a ring of three (144 KB of LDS): the loads of stage s + 2 are issued
// while stage s computes, so two stages of MFMA work cover the load latency, and one barrier per
// stage both publishes stage s and retires every wave's reads of stage s - 1, whose buffer the
// loads issued right after it refill.
//
// K order inside a stage. An MFMA only needs A and B to agree on which K each lane holds, so
// k-step ks (16 deep) gives lane half h the K values 32 h + 8 ks .. +7: a lane then reads its W
// row's 32 contiguous bytes once (two ds_read_b128) for all four k-steps, and its X row's 16
// bytes at K offset 32 h + 8 ks (one ds_read_b128 per k-step).
//
// LDS layouts: X as the FP8 kernel's swizzled 128-byte rows (swz_off); W as 64-byte rows with
// 16-byte chunk c of row r at position c ^ ((r >> 2) & 3), so that the eight rows one
// ds_read_b128 phase touches fall in eight distinct bank groups.
constexpr int kWK = 64;                           // K per stage
constexpr int kWXBytes = 256 * 128;               // X tile per stage (32 KB)
constexpr int kWWBytes = 256 * 64;                // W tile per stage (16 KB)
constexpr int kWStageBytes = kWXBytes + kWWBytes;
constexpr int kWStages = 3;                       // LDS ring; the staged epilogue reuses its first 128 KB

typedef __bf16 v8bf_t __attribute__((ext_vector_type(8)));

struct W8A16Params {
  const uint16_t* x;   // [M, K] bf16, row stride xs
  int64_t xs;
  const uint8_t* w8;   // [N, K] e4m3
  const float* sw;     // N or 1
  int sw_step;
  uint16_t* y;         // [M, N] bf16
  int64_t ys;
  int M, N, K;
  int tiles_n, tiles_m;
  int lds_epi;         // epilogue staged through LDS (N % 8 == 0, 16-byte aligned y rows)
};

__device__ __forceinline__ int wswz_off(int r, int c) { return r * 64 + 16 * (c ^ ((r >> 2) & 3)); }

__device__ __forceinline__ v8bf_t bf16_frag(uint4 q) {
  return __builtin_bit_cast(v8bf_t, q);
}

// Eight e4m3 codes (two words) widened to eight bf16 values.
__device__ __forceinline__ v8bf_t widen8(uint32_t lo, uint32_t hi) {
  const bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)lo, 1.0f, false);
  const bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)lo, 1.0f, true);
  const bf16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)hi, 1.0f, false);
  const bf16x2_t d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)hi, 1.0f, true);
  return v8bf_t{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

__device__ __forceinline__ void w8a16_tile(const W8A16Params& p, uint8_t* lds, int m0, int n0, int wave,
                                           int lane) {
  const int wn = wave & 1, wm = wave >> 1;        // 128 n rows, 64 m columns
  // Direct-to-LDS loads: wave w fills X rows 32 w .. 32 w + 31 (four instructions of 8 rows x
  // 128 bytes) and W rows 32 w .. 32 w + 31 (two instructions of 16 rows x 64 bytes).
  uint32_t xoff[4], woff[2];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int r = 32 * wave + 8 * t + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    const int grow = min(m0 + r, p.M - 1);
    xoff[t] = (uint32_t)grow * (uint32_t)(p.xs * 2) + 16u * (uint32_t)c;
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int r = 32 * wave + 16 * t + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    const int grow = min(n0 + r, p.N - 1);
    woff[t] = (uint32_t)grow * (uint32_t)p.K + 16u * (uint32_t)c;
  }
  auto issue = [&](int buf, int s) __attribute__((always_inline)) {
    uint8_t* stage = lds + buf * kWStageBytes;
    const uint32_t kx = (uint32_t)s * kWK * 2, kw = (uint32_t)s * kWK;
    const uint32_t lx = (uint32_t)(uintptr_t)(lds_u8_t*)(stage + 32 * wave * 128);
    const uint32_t lw = (uint32_t)(uintptr_t)(lds_u8_t*)(stage + kWXBytes + 32 * wave * 64);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                   :: "s"(lx + t * 1024), "v"(xoff[t] + kx), "s"(p.x) : "memory", "m0");
#pragma unroll
    for (int t = 0; t < 2; ++t)
      asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                   :: "s"(lw + t * 1024), "v"(woff[t] + kw), "s"(p.w8) : "memory", "m0");
  };

  v16f acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v16f{};

  const int nst = p.K / kWK;
  const int h = lane >> 5;
  issue(0, 0);
  if (nst > 1) issue(1, 1);
  auto step = [&](int s, auto bufc) __attribute__((always_inline)) {
    constexpr int BUF = decltype(bufc)::value;
    // This wave's loads of stage s landed (only stage s + 1's six are issued after them) ...
    if (s + 1 < nst) __builtin_amdgcn_s_waitcnt(vmcnt_imm(6));
    else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    lds_barrier();                                // ... and every wave's; stage s - 1 is retired
    if (s + 2 < nst) issue((BUF + 2) % kWStages, s + 2);
    const uint8_t* cur = lds + BUF * kWStageBytes;
    // X fragments for both m blocks and all four k-steps: chunk 4 h + ks of row 32 (2 wm + j) + lane % 32.
    v8bf_t b[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int r = 32 * (2 * wm + j) + (lane & 31);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        b[j][ks] = bf16_frag(*reinterpret_cast<const uint4*>(cur + swz_off(r, 4 * h + ks)));
    }
    const uint8_t* wt = cur + kWXBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 32 * (4 * wn + i) + (lane & 31);
      const uint4 q0 = *reinterpret_cast<const uint4*>(wt + wswz_off(r, 2 * h));
      const uint4 q1 = *reinterpret_cast<const uint4*>(wt + wswz_off(r, 2 * h + 1));
      const v8bf_t a[4] = {widen8(q0.x, q0.y), widen8(q0.z, q0.w), widen8(q1.x, q1.y), widen8(q1.z, q1.w)};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ks], b[j][ks], acc[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);           // lgkmcnt(0): this wave's reads of `cur` done
  };
  for (int s = 0; s < nst; s += kWStages) {
    step(s, std::integral_constant<int, 0>{});
    if (s + 1 < nst) step(s + 1, std::integral_constant<int, 1>{});
    if (s + 2 < nst) step(s + 2, std::integral_constant<int, 2>{});
  }
  // The epilogue (and the next tile's first loads) overwrite the ring: every wave's reads of the
  // last stage are done.
  lds_barrier();

  if (p.lds_epi) {
    const float one[2] = {1.0f, 1.0f};
    staged_epilogue(acc, one, p.sw, p.sw_step, p.y, p.ys, nullptr, 0, p.M, p.N, lds, lds + 65536, m0, n0, wave,
                    lane);
    return;
  }
  // Epilogue: lane owns m = m0 + 64 wm + 32 j + lane % 32, n = n0 + 128 wn + 32 i + 8 g + 4 h + 0..3
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float swn[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = min(n0 + 128 * wn + 32 * i + 8 * g + 4 * h, p.N - 4);
      if (p.sw_step) {
        const float4 v = *reinterpret_cast<const float4*>(p.sw + n);
        swn[4 * g] = v.x; swn[4 * g + 1] = v.y; swn[4 * g + 2] = v.z; swn[4 * g + 3] = v.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) swn[4 * g + e] = p.sw[0];
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int m = m0 + 64 * wm + 32 * j + (lane & 31);
      if (m >= p.M) continue;
      uint16_t* yrow = p.y + (int64_t)m * p.ys;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + 128 * wn + 32 * i + 8 * g + 4 * h;
        if (n >= p.N) continue;      // N % 4 == 0 is required on the host
        const v16f& c = acc[i][j];
        uint2 w;
        w.x = pack_bf16x2(c[4 * g] * swn[4 * g], c[4 * g + 1] * swn[4 * g + 1]);
        w.y = pack_bf16x2(c[4 * g + 2] * swn[4 * g + 2], c[4 * g + 3] * swn[4 * g + 3]);
        *reinterpret_cast<uint2*>(yrow + n) = w;
      }
    }
  }
}

__global__ __launch_bounds__(kFThreads, 1) void w8a16_gemm_kernel(W8A16Params p) {
  // Three 48 KB stages; the staged epilogue uses the first 2 x 64 KB.
  __shared__ __align__(16) uint8_t lds[kWStages * kWStageBytes];
  static_assert(kWStages * kWStageBytes >= 2 * 65536, "the staged epilogue needs 128 KB");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x;
  const int L = (G & 7) == 0 ? (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int ntiles = p.tiles_n * p.tiles_m;
  for (int t = L; t < ntiles; t += G) {
    const int group = t / (kGroupM * p.tiles_n);
    const int first_m = group * kGroupM;
    const int gm = min(p.tiles_m - first_m, kGroupM);
    const int tm = first_m + (t % (kGroupM * p.tiles_n)) % gm;
    const int tn = (t % (kGroupM * p.tiles_n)) / gm;
    w8a16_tile(p, lds, tm * kFBM, tn * kFBN, wave, lane);
  }
}

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* p, int n, uint32_t v) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

// Compute units of the current device (queried once per device).

// K ranges per output tile for the 256 x 256 kernel: split when the tiles alone would leave more
// than half of the compute units idle and each range keeps at least 4 K stages of 128. (Measured
// at the C2 shapes: the wgrad output [4096, 1024], 64 tiles, 96 -> 54 us with 4 ranges; the dgrad
// output [8192, 1024], 128 tiles, gains nothing from 2.)
static int splitk_of(int64_t tiles, int64_t K) {
  const int cus = compute_units();
  if (tiles * 2 >= cus) return 1;     // half the GPU or more busy: the finish pass would cost more
  int sp = (int)(cus / tiles);
  sp = sp > 8 ? 8 : sp;
  while (sp > 1 && (K / kFBK) / sp < 4) --sp;
  return sp < 1 ? 1 : sp;
}

static size_t splitk_bytes(int64_t M, int64_t N, int64_t K) {
  if (K % 64 != 0) return 0;
  const int64_t tiles = ((N + kFBN - 1) / kFBN) * ((M + kFBM - 1) / kFBM);
  const int sp = splitk_of(tiles, K);
  return sp > 1 ? (size_t)sp * (size_t)M * (size_t)N * sizeof(float) : 0;
}

static int scaled_mm(const uint8_t* x8, int64_t M, int64_t K, const uint8_t* w8, int64_t N,
                     const float* sx, int64_t sx_count, const float* sw, int64_t sw_count,
                     void* y, int64_t ys, hipStream_t s, const void* res = nullptr, int64_t rs = 0,
                     void* workspace = nullptr, size_t workspace_bytes = 0, uint32_t* gmax = nullptr,
                     int gcols = 0, const GemmParams* xform = nullptr) {
  FLW_REQUIRE(x8 && w8 && sx && sw && y, FLW_E_INVALID, "null pointer argument");
  FLW_REQUIRE(M > 0 && N > 0 && K > 0, FLW_E_INVALID, "empty GEMM");
  FLW_REQUIRE(K % 16 == 0, FLW_E_UNSUPPORTED, "K must be a multiple of 16, got %lld", (long long)K);
  FLW_REQUIRE(N % 4 == 0 && ys % 4 == 0 && ys >= N, FLW_E_INVALID, "N and the output row stride must be multiples of 4");
  FLW_REQUIRE(sx_count == 1 || sx_count == M, FLW_E_INVALID, "x_scale count must be 1 or M");
  FLW_REQUIRE(sw_count == 1 || sw_count == N, FLW_E_INVALID, "w_scale count must be 1 or N");
  FLW_REQUIRE(((uintptr_t)x8 & 15) == 0 && ((uintptr_t)w8 & 15) == 0 && ((uintptr_t)y & 7) == 0,
              FLW_E_INVALID, "x8 / w8 must be 16-byte aligned, y 8-byte aligned");
  FLW_REQUIRE(M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31), FLW_E_UNSUPPORTED, "dimension too large");
  GemmParams p{};
  p.x8 = x8; p.w8 = w8; p.sx = sx; p.sw = sw;
  p.sx_step = sx_count == 1 ? 0 : 1; p.sw_step = sw_count == 1 ? 0 : 1;
  p.y = static_cast<uint16_t*>(y); p.ys = ys;
  p.M = (int)M; p.N = (int)N; p.K = (int)K;
  p.res = static_cast<const uint16_t*>(res); p.rs = rs;
  FLW_REQUIRE(res == nullptr || (rs >= N && rs % 4 == 0 && ((uintptr_t)res & 7) == 0), FLW_E_INVALID,
              "residual rows must be 8-byte aligned with a stride >= N, a multiple of 4");
  if (K % 64 == 0 && N * K < (1ll << 32) && M * K < (1ll << 32)) {
    p.tiles_n = (int)((N + kFBN - 1) / kFBN);
    p.tiles_m = (int)((M + kFBM - 1) / kFBM);
    const int64_t tiles = (int64_t)p.tiles_n * p.tiles_m;
    FLW_REQUIRE(tiles <= 0x7FFFFFFF, FLW_E_UNSUPPORTED, "grid too large");
    // Split-K into the caller's workspace when the output has too few tiles to fill the GPU.
    p.splits = 1;
    p.lds_epi = N % 8 == 0 && ys % 8 == 0 && ((uintptr_t)y & 15) == 0 &&
                (res == nullptr || (rs % 8 == 0 && ((uintptr_t)res & 15) == 0));
    const size_t need = splitk_bytes(M, N, K);
    if (need && workspace && workspace_bytes >= need && ((uintptr_t)workspace & 15) == 0 && N % 4 == 0) {
      p.splits = splitk_of(tiles, K);
      p.part = static_cast<float*>(workspace);
    }
    // Fewer 256 x 256 tiles than compute units: 256 x 128 tiles (twice as many), and then half
    // the K ranges of an even split (the same number of work items, half the partials to fold).
    // An odd split keeps its 256 x 256 tiles: halving 3 ranges to 1 would leave the items a
    // third of the GPU short (the 450M block's wgrad outputs [3392 | 3840, 1280] at K = 16384:
    // 70 / 75 tiles x 3 ranges, 97 / 92 us against 108 / 103 us as 135 / 150 narrow tiles).
    // More tiles than compute units: the narrow tiles too when they fill the last round of the
    // persistent grid enough better to pay their ~10 % higher cost per output (measured at
    // M = 16384: 320 tiles [N = 1280] 62.5 % -> 83 % filled, -10 to -19 %; 896 tiles 87.5 % ->
    // 100 %, -3 %; 960 or 512 tiles, equally filled either way, +3 to +13 % narrow).
    const int cus = compute_units();
    auto fill = [cus](int64_t items) { return (double)items / (double)(((items + cus - 1) / cus) * cus); };
    const bool narrow = p.lds_epi && gmax == nullptr && xform == nullptr &&
                        (tiles < cus ? (p.splits == 1 || p.splits % 2 == 0)
                                     : p.splits == 1 && fill(2 * tiles) > 1.1 * fill(tiles));
    if (narrow) {
      p.tiles_m = (int)((M + 127) / 128);
      p.splits = p.splits / 2 > 1 ? p.splits / 2 : 1;
      if (p.splits == 1) p.part = nullptr;
    }
    // K % 128 == 64 (no q / k transform: its entry point requires K % 128 == 0): the instances
    // whose last K stage is 64 deep.
    const bool halfk = K % kFBK != 0;
    const void* kern = narrow ? (halfk ? reinterpret_cast<const void*>(&fp8_gemm_256_kernel<128, 0, true>)
                                       : reinterpret_cast<const void*>(&fp8_gemm_256_kernel<128>))
                     : xform == nullptr ? (halfk ? reinterpret_cast<const void*>(&fp8_gemm_256_kernel<256, 0, true>)
                                                 : reinterpret_cast<const void*>(&fp8_gemm_256_kernel<256>))
                     : gcols == 32 ? reinterpret_cast<const void*>(&fp8_gemm_256_kernel<256, 32>)
                     : gcols == 64 ? reinterpret_cast<const void*>(&fp8_gemm_256_kernel<256, 64>)
                     : reinterpret_cast<const void*>(&fp8_gemm_256_kernel<256, 128>);
    // Persistent: one workgroup per CU (each holds 128 KB of LDS), at most one per work item.
    const int64_t items = (int64_t)p.tiles_n * p.tiles_m * p.splits;
    const int64_t grid = items < compute_units() ? items : compute_units();
    if (gmax) {
      FLW_REQUIRE(p.splits == 1 && p.lds_epi, FLW_E_UNSUPPORTED,
                  "the group amax needs an unsplit GEMM with N %% 8 == 0 and 16-byte aligned rows");
      p.gmax = gmax;
      p.gcols = gcols;
      if (xform != nullptr) {
        p.xcols = xform->xcols; p.xnorm = xform->xnorm; p.xeps = xform->xeps; p.xT = xform->xT;
        p.rcos = xform->rcos; p.rsin = xform->rsin;
      }
      const Timer tm = take_timer();
      const int ng = (int)(N / gcols);
      (void)launch_args(reinterpret_cast<const void*>(&fill_u32_kernel), dim3((unsigned)((ng + 255) / 256)),
                        dim3(256), 0, s, tm.start, nullptr, gmax, ng, 0u);
      (void)launch_ext(kern, dim3((unsigned)grid), dim3(kFThreads), 0, s, p, nullptr, tm.stop);
    } else if (p.splits == 1) {
      (void)launch_timed(kern, dim3((unsigned)grid), dim3(kFThreads), s, p);
    } else {
      const Timer tm = take_timer();
      (void)launch_ext(kern, dim3((unsigned)grid), dim3(kFThreads),
                       0, s, p, tm.start, nullptr);
      const int64_t quads = M * (N / 4);
      (void)launch_ext(reinterpret_cast<const void*>(&gemm_splitk_reduce_kernel), dim3((unsigned)((quads + 255) / 256)),
                       dim3(256), 0, s, p, nullptr, tm.stop);
    }
    return check_launch("flw_fp8_scaled_mm");
  }
  // The general kernel has no group-amax epilogue: refuse rather than leave amax_out unwritten.
  FLW_REQUIRE(gmax == nullptr, FLW_E_UNSUPPORTED,
              "the group amax needs K %% 64 == 0 and M*K, N*K < 2^32 (the 256 x 256 kernel)");
  p.tiles_n = (int)((N + kGBN - 1) / kGBN);
  const int64_t tiles = (int64_t)p.tiles_n * ((M + kGBM - 1) / kGBM);
  FLW_REQUIRE(tiles <= 0x7FFFFFFF, FLW_E_UNSUPPORTED, "grid too large");
  (void)launch_timed(reinterpret_cast<const void*>(&fp8_gemm_kernel), dim3((unsigned)tiles), dim3(256), s, p);
  return check_launch("flw_fp8_scaled_mm");
}

static int w8a16_mm(const uint16_t* x, int64_t M, int64_t K, int64_t xs, const uint8_t* w8, int64_t N,
                    const float* sw, int64_t sw_count, void* y, int64_t ys, hipStream_t s) {
  FLW_REQUIRE(x && w8 && sw && y, FLW_E_INVALID, "null pointer argument");
  FLW_REQUIRE(M > 0 && N > 0 && K > 0, FLW_E_INVALID, "empty GEMM");
  FLW_REQUIRE(K % kWK == 0, FLW_E_UNSUPPORTED, "W8A16 needs K a multiple of %d, got %lld", kWK, (long long)K);
  FLW_REQUIRE(N % 4 == 0 && ys % 4 == 0 && ys >= N, FLW_E_INVALID, "N and the output row stride must be multiples of 4");
  FLW_REQUIRE(xs >= K && xs % 8 == 0, FLW_E_INVALID, "x row stride must be >= K and a multiple of 8 elements");
  FLW_REQUIRE(sw_count == 1 || sw_count == N, FLW_E_INVALID, "w_scale count must be 1 or N");
  FLW_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)w8 & 15) == 0 && ((uintptr_t)y & 7) == 0 &&
              (sw_count == 1 || ((uintptr_t)sw & 15) == 0),
              FLW_E_INVALID, "x / w8 must be 16-byte aligned, y 8-byte aligned, per-channel scales 16-byte aligned");
  FLW_REQUIRE(M * xs * 2 < (1ll << 32) && N * K < (1ll << 32), FLW_E_UNSUPPORTED, "operand too large for 32-bit offsets");
  W8A16Params p{};
  p.x = x; p.xs = xs; p.w8 = w8; p.sw = sw; p.sw_step = sw_count == 1 ? 0 : 1;
  p.y = static_cast<uint16_t*>(y); p.ys = ys;
  p.M = (int)M; p.N = (int)N; p.K = (int)K;
  p.lds_epi = N % 8 == 0 && ys % 8 == 0 && ((uintptr_t)y & 15) == 0;
  p.tiles_n = (int)((N + kFBN - 1) / kFBN);
  p.tiles_m = (int)((M + kFBM - 1) / kFBM);
  const int64_t tiles = (int64_t)p.tiles_n * p.tiles_m;
  FLW_REQUIRE(tiles <= 0x7FFFFFFF, FLW_E_UNSUPPORTED, "grid too large");
  const int64_t grid = tiles < compute_units() ? tiles : compute_units();
  (void)launch_timed(reinterpret_cast<const void*>(&w8a16_gemm_kernel), dim3((unsigned)grid), dim3(kFThreads), s, p);
  return check_launch("flw_fp8_linear (W8A16)");
}

static size_t galign(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace flw

using namespace flw;

extern "C" int flw_fp8_scaled_mm(const uint8_t* x8, int64_t M, int64_t K, const uint8_t* w8,
                                 int64_t N, const float* x_scale, int64_t x_scale_count,
                                 const float* w_scale, int64_t w_scale_count, void* y,
                                 int64_t y_row_stride, void* stream) {
  return scaled_mm(x8, M, K, w8, N, x_scale, x_scale_count, w_scale, w_scale_count, y,
                   y_row_stride, static_cast<hipStream_t>(stream));
}

extern "C" size_t flw_fp8_scaled_mm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return splitk_bytes(M, N, K);
}

extern "C" int flw_fp8_scaled_mm_ws(const uint8_t* x8, int64_t M, int64_t K, const uint8_t* w8, int64_t N,
                                    const float* x_scale, int64_t x_scale_count, const float* w_scale,
                                    int64_t w_scale_count, void* y, int64_t y_row_stride, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  return scaled_mm(x8, M, K, w8, N, x_scale, x_scale_count, w_scale, w_scale_count, y, y_row_stride,
                   static_cast<hipStream_t>(stream), nullptr, 0, workspace, workspace_bytes);
}

extern "C" int flw_fp8_scaled_mm_group_amax(const uint8_t* x8, int64_t M, int64_t K, const uint8_t* w8,
                                            int64_t N, const float* x_scale, int64_t x_scale_count,
                                            const float* w_scale, int64_t w_scale_count, void* y,
                                            int64_t y_row_stride, int64_t group_cols, uint32_t* amax_out,
                                            void* stream) {
  FLW_REQUIRE(amax_out != nullptr, FLW_E_INVALID, "null amax_out");
  FLW_REQUIRE(group_cols >= 8 && group_cols <= 256 && (group_cols & (group_cols - 1)) == 0 && N % group_cols == 0,
              FLW_E_INVALID, "group_cols must be a power of two in [8, 256] dividing N");
  FLW_REQUIRE(K % 64 == 0, FLW_E_UNSUPPORTED, "the group amax needs K %% 64 == 0");
  return scaled_mm(x8, M, K, w8, N, x_scale, x_scale_count, w_scale, w_scale_count, y, y_row_stride,
                   static_cast<hipStream_t>(stream), nullptr, 0, nullptr, 0, amax_out, (int)group_cols);
}

extern "C" int flw_fp8_scaled_mm_qk_norm_rope_amax(const uint8_t* x8, int64_t M, int64_t K, const uint8_t* w8,
                                                  int64_t N, const float* x_scale, int64_t x_scale_count,
                                                  const float* w_scale, int64_t w_scale_count, void* y,
                                                  int64_t y_row_stride, int64_t head_dim, int64_t qk_cols, int qk_norm,
                                                  float eps, const void* rope_cos, const void* rope_sin,
                                                  int64_t seq_len, uint32_t* amax_out, void* stream) {
  FLW_REQUIRE(amax_out != nullptr, FLW_E_INVALID, "null amax_out");
  FLW_REQUIRE(head_dim == 32 || head_dim == 64 || head_dim == 128, FLW_E_UNSUPPORTED,
              "head_dim must be 32/64/128, got %lld", (long long)head_dim);
  FLW_REQUIRE(N % head_dim == 0 && qk_cols >= 0 && qk_cols <= N && qk_cols % head_dim == 0, FLW_E_INVALID,
              "qk_cols must be a multiple of head_dim within N");
  FLW_REQUIRE((rope_cos == nullptr) == (rope_sin == nullptr), FLW_E_INVALID, "pass both RoPE tables or neither");
  FLW_REQUIRE(seq_len > 0 && seq_len <= 0x7FFFFFFF && M % seq_len == 0, FLW_E_INVALID,
              "seq_len must divide M (rows are (batch, position) pairs)");
  FLW_REQUIRE(rope_cos == nullptr || (((uintptr_t)rope_cos & 15) == 0 && ((uintptr_t)rope_sin & 15) == 0),
              FLW_E_INVALID, "RoPE tables must be 16-byte aligned");
  FLW_REQUIRE(qk_norm == 0 || eps >= 0.0f, FLW_E_INVALID, "eps must be non-negative");
  FLW_REQUIRE(K % kFBK == 0, FLW_E_UNSUPPORTED, "the fused epilogue needs K %% %d == 0", kFBK);
  GemmParams xf{};
  xf.xcols = (int)qk_cols;
  xf.xnorm = qk_norm != 0;
  xf.xeps = eps;
  xf.xT = (int)seq_len;
  xf.rcos = static_cast<const uint16_t*>(rope_cos);
  xf.rsin = static_cast<const uint16_t*>(rope_sin);
  return scaled_mm(x8, M, K, w8, N, x_scale, x_scale_count, w_scale, w_scale_count, y, y_row_stride,
                   static_cast<hipStream_t>(stream), nullptr, 0, nullptr, 0, amax_out, (int)head_dim,
                   qk_cols > 0 ? &xf : nullptr);
}

extern "C" int flw_fp8_scaled_mm_residual(const uint8_t* x8, int64_t M, int64_t K, const uint8_t* w8,
                                          int64_t N, const float* x_scale, int64_t x_scale_count,
                                          const float* w_scale, int64_t w_scale_count, void* y,
                                          int64_t y_row_stride, const void* residual,
                                          int64_t residual_row_stride, void* stream) {
  FLW_REQUIRE(residual != nullptr, FLW_E_INVALID, "null residual");
  return scaled_mm(x8, M, K, w8, N, x_scale, x_scale_count, w_scale, w_scale_count, y, y_row_stride,
                   static_cast<hipStream_t>(stream), residual, residual_row_stride);
}

extern "C" size_t flw_fp8_linear_workspace_bytes(int64_t M, int64_t K, int mode) {
  if (mode != FLW_GEMM_A8W8) return 0;
  return galign((size_t)(M * K)) + galign(sizeof(float) * (size_t)M);
}

extern "C" int flw_fp8_linear(const void* x, int64_t M, int64_t K, int64_t x_row_stride,
                              const uint8_t* w8, int64_t N, const float* w_scale,
                              int64_t w_scale_count, int mode, void* y, int64_t y_row_stride,
                              void* workspace, size_t workspace_bytes, void* stream) {
  FLW_REQUIRE(mode == FLW_GEMM_A8W8 || mode == FLW_GEMM_W8A16, FLW_E_INVALID, "unknown GEMM mode %d", mode);
  if (mode == FLW_GEMM_W8A16)
    return w8a16_mm(static_cast<const uint16_t*>(x), M, K, x_row_stride, w8, N, w_scale, w_scale_count, y,
                    y_row_stride, static_cast<hipStream_t>(stream));
  const size_t need = flw_fp8_linear_workspace_bytes(M, K, mode);
  FLW_REQUIRE(workspace != nullptr && workspace_bytes >= need, FLW_E_WORKSPACE, "workspace needs %zu bytes", need);
  uint8_t* x8 = static_cast<uint8_t*>(workspace);
  float* sx = reinterpret_cast<float*>(x8 + galign((size_t)(M * K)));
  const Timer tm = take_timer();   // start on the row quantiser, stop on the GEMM
  arm_timer(Timer{tm.start, nullptr});
  int rc = flw_quant_rows_e4m3(x, FLW_BF16, M, K, x_row_stride, x8, sx, stream);
  if (rc) {
    arm_timer(Timer{});
    return rc;
  }
  arm_timer(Timer{nullptr, tm.stop});
  rc = scaled_mm(x8, M, K, w8, N, sx, M, w_scale, w_scale_count, y, y_row_stride,
                 static_cast<hipStream_t>(stream));
  if (rc) arm_timer(Timer{});
  return rc;
}
