// bf16 causal sliding-window attention, forward (with the log-sum-exp) and backward, for gfx950.
//
// The differentiable counterpart of the FP8 forward (flower/kernels/swa_attention.py): bf16 Q/K/V
// in, bf16 out, softmax and accumulation in fp32, v_mfma_f32_32x32x16_bf16 for every product.
//
// Forward: one workgroup = 4 waves = 128 queries of one (b, h); a wave owns 32 queries and walks
// the 64-key tiles of its band. S^T = K Q^T (keys are the MFMA rows, so a lane holds 16 scores of
// ONE query and the softmax row reductions are lane-local plus one v_permlane32_swap), the online
// softmax in base 2, P packed to bf16 straight from those registers into the B operand of
// O^T += V^T P^T. For that the K order of each 16-deep k-step is permuted: lane half h takes the
// keys {0-3, 8-11} + 4h of the step, exactly the scores it already holds, and the V^T tile in LDS
// is stored in that order (V is transposed while it is staged). L = m + log(l) is written for the
// backward.
//
// Backward (after Delta = rowsum(dO * O)):
//   dK / dV: one workgroup = 128 keys (4 waves x 32 keys, their K and V fragments in registers),
//     walking the 64-query tiles that see them. S = Q K^T and dP = dO V^T with queries as MFMA
//     rows, so a lane holds 16 queries of ONE key; P = exp(S - L), dS = P (dP - Delta) / sqrt(D)
//     feed dV += P^T dO and dK += dS^T Q directly as A operands (the same k-step permutation over
//     queries), with dO^T and Q^T staged transposed in LDS.
//   dQ: one workgroup = 128 queries (Q and dO fragments in registers), walking key tiles:
//     S^T = K Q^T, dP^T = V dO^T (keys as rows, one query per lane), dS^T, then
//     dQ^T += K^T dS^T with K^T staged transposed in LDS.
// Rows past T are loaded as zeros and never stored.
#include <math.h>

#include <type_traits>

#include "flw_common.h"

// m0 is clobbered by the direct-to-LDS tile loads (TileLoadLds); nothing else here uses it.
#pragma clang diagnostic ignored "-Winline-asm"

namespace flw {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ v16f mfma16(v8bf a, v8bf b, v16f c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v8bf as_v8bf(uint4 q) { return __builtin_bit_cast(v8bf, q); }
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v{a, b}), bf16x2v));
}

constexpr float kLog2eB = 1.4426950408889634f;

struct SwaB16Params {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;      // forward output (backward: read)
  const uint16_t* dout;   // backward only
  uint16_t* out;          // forward: O; dq kernel: dQ
  uint16_t* out2;         // dkdv kernel: dK
  uint16_t* out3;         // dkdv kernel: dV
  float* lse;             // [B, H, T]
  float* delta;           // [B, H, T]
  int H, T, W, nblk, nwg; // nblk: 128-row blocks per (b, h)
  int ramp;               // blocks per slice whose band is cut short by the sequence's start / end
  int group_slices;       // slices per dispatch group (one XCD's share when it is whole slices)
  float sm_scale;
  int64_t rows;           // B * H * T (delta kernel)
  int o_tmaj;             // O and dO token-major, (B, T, H, D): rows of a (b, h) slice H D apart
};

// O / dO of slice (b, h) = bh: its first row and its row stride in elements. Head-major (B, H, T, D)
// slices are contiguous; token-major (B, T, H, D) slices interleave with the other heads, which is
// the layout the output projection reads as [B T, H D] rows.
__device__ __forceinline__ int64_t o_base(const SwaB16Params& p, int bh, int D) {
  if (!p.o_tmaj) return (int64_t)bh * p.T * D;
  const int b = bh / p.H, h = bh - b * p.H;
  return ((int64_t)b * p.T * p.H + h) * D;
}
__device__ __forceinline__ int o_ld(const SwaB16Params& p, int D) { return p.o_tmaj ? p.H * D : D; }

// ---------------------------------------------------------------- LDS tile layouts
//
// A natural tile: 64 rows x D bf16 (2D bytes per row), 16-byte chunk c of row r at position
// c ^ swz(r). The swizzle serves both ways the tile is read:
//  - ds_read_b128 of one chunk by 16 consecutive rows (nat_frag) hits 16 distinct 16-byte bank
//    slots of the 256-byte bank space (a row of D = 64 is 128 bytes, so row parity picks the
//    half and swz must be a permutation over each parity class);
//  - ds_read_b64_tr_b16 (trr_frag) by a half-wave reads 4 consecutive rows x 64 bytes, which
//    must land in 4 distinct 64-byte quarters.
// D = 32 (64-byte rows) gets the quarters from the row address alone.
template <int D>
__device__ __forceinline__ int nat_off(int r, int c) {
  if (D == 32) return r * 64 + 16 * (c ^ ((r >> 2) & 3));
  if (D == 64) return r * 128 + 16 * (c ^ ((((r >> 1) & 1) << 2) | ((r >> 2) & 3)));
  return r * 256 + 16 * (c ^ (((r & 3) << 2) | ((r >> 2) & 3)));
}

// Buffer descriptors cover a slice's T rows, so rows past T read as zero with no compare; row
// offsets go into the VGPR offset, which the descriptor's range check covers.
constexpr int kBufferFlags = 0x00020000;   // buffer descriptor word 3 for raw dword access (gfx9)

// Global -> LDS for one 64-row tile of a (T, D) bf16 slice, straight into the natural swizzled
// layout (buffer_load_dwordx4 ... lds: each lane's 16 bytes land at M0 + 16 lane, no VGPR round
// trip, so a kernel holds no prefetch registers): wave w fills rows RPI (NI w + t) .. + RPI - 1
// with instruction t, the lane at LDS slot p of row r loading the global chunk that nat_off puts
// at slot p (the swizzle is an XOR, its own inverse). Rows past T read as zero through the
// descriptor's range check. Issued from inline assembly, so the compiler does not wait for these
// loads before every LDS read; callers wait (vmcnt) before the barrier that publishes a tile.
template <int D>
struct TileLoadLds {
  static constexpr int CPR = D / 8;                 // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;              // rows per wave instruction
  static constexpr int NI = 64 / RPI / 4;           // instructions per wave per tile
  __amdgpu_buffer_rsrc_t rs;
  uint32_t off[NI];
  uint32_t row_bytes;
  // Rows of D values `ld` elements apart (ld = D: a contiguous slice); rows past T read as zeros
  // (the descriptor ends with row T - 1).
  __device__ __forceinline__ void init(const uint16_t* base, int T, int wave, int lane, int ld = D) {
    row_bytes = (uint32_t)ld * 2;
    rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), 0, (T - 1) * ld * 2 + 2 * D, kBufferFlags);
#pragma unroll
    for (int t = 0; t < NI; ++t) {
      const int r = RPI * (NI * wave + t) + lane / CPR, slot = lane % CPR;
      const int c = (nat_off<D>(r, slot) - r * 2 * D) / 16;
      off[t] = (uint32_t)r * row_bytes + 16 * c;
    }
  }
  __device__ __forceinline__ void load(uint8_t* lds, int row0, int wave) const {
#pragma unroll
    for (int t = 0; t < NI; ++t) {
      const uint32_t dst = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)(lds + RPI * (NI * wave + t) * 2 * D);
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                   :: "s"(dst), "v"(off[t] + (uint32_t)row0 * row_bytes), "s"(rs) : "memory", "m0");
    }
  }
};

// Fragment of a natural tile for the rows 32 rb .. 32 rb + 31, k-step ks (K = model dim):
// lane (row rb*32 + lane%32, half h) takes dims 16 ks + 8 h .. +7.
template <int D>
__device__ __forceinline__ v8bf nat_frag(const uint8_t* lds, int rb, int ks, int lane) {
  return as_v8bf(*reinterpret_cast<const uint4*>(lds + nat_off<D>(32 * rb + (lane & 31), 2 * ks + (lane >> 5))));
}
// Fragment of a natural tile read transposed, for the dims 32 db .. 32 db + 31 (the MFMA row /
// column, lane % 32) with K = the tile's 64 rows, k-step g, in the permuted k-step order (lane
// half h holds rows 16 g + {0-3, 8-11} + 4 h). ds_read_b64_tr_b16 works on groups of 16 lanes:
// lane 4 j + a supplies the address of 4 consecutive bf16 (row j, dims 4 a .. 4 a + 3 of its
// group's 16 dims) and lane 4 a + e receives element e of the rows j = 0..3 supplied by lanes
// a, a + 4, a + 8, a + 12. Two reads (rows 16 g + 4 h + j and 16 g + 8 + 4 h + j) give the 8 values.
template <int D>
__device__ __forceinline__ v8bf trr_frag(const uint8_t* lds, int db, int g, int lane) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef short v8s __attribute__((ext_vector_type(8)));
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  const int s = lane & 15, j = s >> 2, a = s & 3, h = lane >> 5;
  const int d = 32 * db + 16 * ((lane >> 4) & 1) + 4 * a;
  const int r = 16 * g + 4 * h + j;
  const int cb = 2 * (d & 7);
  const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(lds + nat_off<D>(r, d >> 3) + cb));
  const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(lds + nat_off<D>(r + 8, d >> 3) + cb));
  const v8s w = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(v8bf, w);
}
// Fragment of a row of global memory: 8 dims 16 ks + 8 h of row `row` (zero past T).
template <int D>
__device__ __forceinline__ v8bf row_frag(const uint16_t* base, int row, int T, int ks, int lane, int ld = D) {
  if (row >= T) return as_v8bf(make_uint4(0, 0, 0, 0));
  return as_v8bf(*reinterpret_cast<const uint4*>(base + (int64_t)row * ld + 16 * ks + 8 * (lane >> 5)));
}

// The 16 values of a 32x32 C block, packed to bf16 as the B (or A) operand of the next product
// with K over the block's rows: k-step 2 b + s gets values 8 s .. 8 s + 7.
__device__ __forceinline__ v8bf pack_frag(const v16f& c, int s) {
  uint4 q;
  q.x = pk_bf16(c[8 * s + 0], c[8 * s + 1]);
  q.y = pk_bf16(c[8 * s + 2], c[8 * s + 3]);
  q.z = pk_bf16(c[8 * s + 4], c[8 * s + 5]);
  q.w = pk_bf16(c[8 * s + 6], c[8 * s + 7]);
  return as_v8bf(q);
}

__device__ __forceinline__ float pmax_pair(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float psum_pair(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Element v of a 32x32 C block held by lane (col, h) is row 8 (v / 4) + 4 h + v % 4.
__device__ __forceinline__ int crow(int v, int h) { return 8 * (v >> 2) + 4 * h + (v & 3); }

// Before a tile loop: every load issued so far (this lane's own row fragments, the first
// tile) has landed, and the first tile is published. Without the explicit wait the compiler's
// wait-count placement, merging the path that skips the first tile, would wait inside the loop
// for the row fragments and with them for the next tile's prefetch, every iteration.
__device__ __forceinline__ void wait_all_loads() {
  __builtin_amdgcn_s_waitcnt(0);   // vmcnt(0) expcnt(0) lgkmcnt(0)
  __syncthreads();
}

// XCD-contiguous work numbering (as in the FP8 kernel).
// Contiguous work per XCD when the slices split evenly over the 8 XCDs; otherwise round-robin
// over the XCDs, so each XCD gets an even share of the long and short work items.
__device__ __forceinline__ int xcd_id(const SwaB16Params& p) {
  int L = (int)blockIdx.x;
  if (p.group_slices * 8 * p.nblk == p.nwg) L = (L & 7) * (p.nwg >> 3) + (L >> 3);
  return L;
}

// (slice, 128-row block) of this workgroup. Inside one XCD's group of slices the blocks with a
// full-length band come first, slice by slice (consecutive blocks share K / V or Q / dO tiles in
// that XCD's L2), then the `ramp` short-band blocks in decreasing band length, so the short work
// items fill the grid's drain. Query-block kernels: the short blocks are a slice's first ones (their
// band starts at key 0); the key-block kernel: its last ones (their band ends at query T - 1).
__device__ __forceinline__ void band_order(const SwaB16Params& p, bool ramp_at_end, int& bh, int& blk) {
  const int L = xcd_id(p);
  const int gs = p.group_slices, R = p.ramp, nfull = p.nblk - R;
  const int gi = L / (gs * p.nblk), i = L % (gs * p.nblk);
  if (i < gs * nfull) {
    bh = gi * gs + i / nfull;
    blk = (ramp_at_end ? 0 : R) + i % nfull;
  } else {
    const int j = i - gs * nfull, r = j / gs;     // r-th longest short-band block
    bh = gi * gs + j % gs;
    blk = ramp_at_end ? nfull + r : R - 1 - r;
  }
}

// ---------------------------------------------------------------- forward

template <int D>
__global__ __launch_bounds__(256, 2) void swa_bf16_fwd_kernel(SwaB16Params p) {
  constexpr int KS = D / 16;                      // k-steps over the head dim
  constexpr int NDB = D / 32;                     // 32-row blocks of O^T
  constexpr int NAT = 64 * D * 2;                 // bytes of a natural / transposed tile
  __shared__ __align__(16) uint8_t lk[2][NAT];
  __shared__ __align__(16) uint8_t lv[2][NAT];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), h = lane >> 5, qc = lane & 31;
  int bh, mt;
  band_order(p, false, bh, mt);
  const int T = p.T, W = p.W;
  const int m0 = mt * 128, q0 = m0 + 32 * wave;
  const int64_t slice = (int64_t)bh * T * D;
  const uint16_t* Q = p.q + slice;
  const uint16_t* K = p.k + slice;
  const uint16_t* V = p.v + slice;
  const float c = p.sm_scale * kLog2eB;

  v8bf qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qf[ks] = row_frag<D>(Q, q0 + qc, T, ks, lane);

  const int lo_raw = m0 - W + 1;
  const int lo = lo_raw <= 0 ? 0 : (lo_raw & ~63);
  const int hi = min(T, m0 + 128);
  const int nt = hi > lo ? (hi - lo + 63) / 64 : 0;
  const int wk0 = max(0, q0 - W + 1), wk1 = min(q0 + 31, T - 1);
  const int ta = q0 < T ? (wk0 - lo) / 64 : 1;
  const int tb = q0 < T ? (wk1 - lo) / 64 : 0;

  v16f o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = v16f{};
  float m_run = -INFINITY, l_run = 0.0f;

  TileLoadLds<D> tk, tv;
  tk.init(K, T, wave, lane);
  tv.init(V, T, wave, lane);
  if (nt > 0) {
    tk.load(lk[0], lo, wave);
    tv.load(lv[0], lo, wave);
  }
  wait_all_loads();

  for (int j = 0; j < nt; ++j) {
    const int buf = j & 1;
    const bool pre = j + 1 < nt;
    if (pre) {
      tk.load(lk[buf ^ 1], lo + (j + 1) * 64, wave);
      tv.load(lv[buf ^ 1], lo + (j + 1) * 64, wave);
    }
    if (j >= ta && j <= tb) {
      const int n0 = lo + 64 * j;
      v16f s[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        s[b] = v16f{};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) s[b] = mfma16(nat_frag<D>(lk[buf], b, ks, lane), qf[ks], s[b]);
      }
      // mask: key n0 + 32 b + crow(v, h) against query q0 + qc
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int d0 = q0 + qc - (n0 + 32 * b);         // i - j for row 0 of the block
        const bool full = (q0 - (n0 + 32 * b) >= 31) && (q0 + 31 - (n0 + 32 * b) < W) && (n0 + 32 * b + 31 < T);
        if (!full) {
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int dd = d0 - crow(v, h);
            s[b][v] = (dd >= 0 && dd < W && n0 + 32 * b + crow(v, h) < T) ? s[b][v] : -INFINITY;
          }
        }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[b][v]);
      const float m_new = fmaxf(m_run, pmax_pair(mx));
      const float m_safe = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = __builtin_amdgcn_exp2f((m_run - m_safe) * c);
      const float nb = -m_safe * c;
      m_run = m_new;
      float ls = 0.0f;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          s[b][v] = __builtin_amdgcn_exp2f(fmaf(s[b][v], c, nb));
          ls += s[b][v];
        }
      l_run = fmaf(l_run, alpha, ls);
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        o[db] *= alpha;
#pragma unroll
        for (int g = 0; g < 4; ++g) o[db] = mfma16(trr_frag<D>(lv[buf], db, g, lane), pack_frag(s[g >> 1], g & 1), o[db]);
      }
    }
    // The other buffer was last read in step j - 1, which every wave finished before the barrier
    // that ended it; one barrier per tile publishes the new tile.
    __builtin_amdgcn_s_waitcnt(0x0F70);             // vmcnt(0): this wave's tile loads landed
    __syncthreads();
  }

  const float l_tot = psum_pair(l_run);
  const int qi = q0 + qc;
  if (qi < T) {
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    uint16_t* op = p.out + o_base(p, bh, D) + (int64_t)qi * o_ld(p, D);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = 32 * db + 8 * j + 4 * h;
        uint2 w;
        w.x = pk_bf16(o[db][4 * j] * inv, o[db][4 * j + 1] * inv);
        w.y = pk_bf16(o[db][4 * j + 2] * inv, o[db][4 * j + 3] * inv);
        *reinterpret_cast<uint2*>(op + d) = w;
      }
    if (h == 0) p.lse[(int64_t)bh * T + qi] = fmaf(m_run, p.sm_scale, __logf(l_tot));
  }
}

// ---------------------------------------------------------------- backward: Delta

// Delta[row] = sum_d dO[row, d] * O[row, d] in fp32; D / 8 consecutive lanes per row.
template <int D>
__global__ __launch_bounds__(256) void swa_bf16_delta_kernel(SwaB16Params p) {
  constexpr int LPR = D / 8;                      // lanes per row (8 elements each)
  const uint16_t* __restrict__ o = p.o;
  const uint16_t* __restrict__ dout = p.dout;
  const int64_t rows = p.rows;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gid / LPR;
  const int part = (int)(gid % LPR);
  float s = 0.0f;
  if (row < rows) {
    // row = (b H + h) T + t of the (B, H, T) statistics; O / dO's element offset of that row
    int64_t at = row * D;
    if (p.o_tmaj) {
      const int64_t bh = row / p.T, t = row - bh * p.T;
      at = o_base(p, (int)bh, D) + t * o_ld(p, D);
    }
    float a[8], b[8];
    Vec16<uint16_t>::load(o + at + 8 * part, a);
    Vec16<uint16_t>::load(dout + at + 8 * part, b);
#pragma unroll
    for (int e = 0; e < 8; ++e) s = fmaf(a[e], b[e], s);
  }
#pragma unroll
  for (int w = LPR / 2; w >= 1; w >>= 1) s += __shfl_xor(s, w, 64);
  if (row < rows && part == 0) p.delta[row] = s;
}

// ---------------------------------------------------------------- backward: dK, dV

template <int D>
__global__ __launch_bounds__(256, D == 128 ? 1 : 2) void swa_bf16_dkdv_kernel(SwaB16Params p) {
  constexpr int KS = D / 16, NDB = D / 32, NAT = 64 * D * 2;
  __shared__ __align__(16) uint8_t lq[2][NAT];     // Q tile: A operand of S, read transposed for dK
  __shared__ __align__(16) uint8_t ldo[2][NAT];    // dO tile: A operand of dP, read transposed for dV
  __shared__ __align__(16) float lstat[2][2][64];  // -L log2(e) and Delta of the tile's queries
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), h = lane >> 5, kc = lane & 31;
  int bh, nt0;
  band_order(p, true, bh, nt0);
  const int T = p.T, W = p.W;
  const int k0w = nt0 * 128, k0 = k0w + 32 * wave;     // this wave's 32 keys
  const int64_t slice = (int64_t)bh * T * D;
  const float* LSE = p.lse + (int64_t)bh * T;
  const float* DLT = p.delta + (int64_t)bh * T;
  const float c = p.sm_scale * kLog2eB;

  // K and V of this wave's keys as B operands (lane = key column, 8 dims per k-step).
  v8bf kf[KS], vf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    kf[ks] = row_frag<D>(p.k + slice, k0 + kc, T, ks, lane);
    vf[ks] = row_frag<D>(p.v + slice, k0 + kc, T, ks, lane);
  }
  v16f dk[NDB], dv[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) { dk[db] = v16f{}; dv[db] = v16f{}; }

  // Query tiles that see the workgroup's keys [k0w, k0w + 127]: queries [k0w, k0w + 127 + W - 1].
  const int lo = k0w & ~63;
  const int hi = min(T, k0w + 127 + W);
  const int nt = hi > lo ? (hi - lo + 63) / 64 : 0;
  // This wave's keys are seen by queries [k0, k0 + 31 + W - 1].
  const int wq1 = min(T - 1, k0 + 31 + W - 1);
  const int ta = k0 < T ? (k0 - lo) / 64 : 1;
  const int tb = k0 < T ? (wq1 - lo) / 64 : 0;

  // Queries past T: Q and dO load as zeros and their L / Delta stage as zeros, so P = 1,
  // dS = 1 * (0 - 0) = 0 and P^T dO = 0: they add nothing, without a compare. Keys past T are
  // computed on zeros and never stored. Only the band 0 <= i - j < W is masked, and only in
  // the 32 x 32 blocks it cuts.
  TileLoadLds<D> tq, tdo;
  tq.init(p.q + slice, T, wave, lane);
  tdo.init(p.dout + o_base(p, bh, D), T, wave, lane, o_ld(p, D));
  // Wave 0 carries L of the tile's 64 queries (stored as -L log2(e)), wave 1 their Delta; both
  // through buffer descriptors over the slice's T values, so queries past T read as 0.
  const __amdgpu_buffer_rsrc_t lrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(LSE), 0, T * 4, kBufferFlags);
  const __amdgpu_buffer_rsrc_t drs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(DLT), 0, T * 4, kBufferFlags);
  auto load_stat = [&](int r0) __attribute__((always_inline)) {
    float x = 0.0f;
    if (wave == 0) x = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(lrs, 4 * (r0 + lane), 0, 0));
    else if (wave == 1) x = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(drs, 4 * (r0 + lane), 0, 0));
    return x;
  };
  auto store_stat = [&](int buf, float x) __attribute__((always_inline)) {
    if (wave == 0) lstat[buf][0][lane] = -x * kLog2eB;
    else if (wave == 1) lstat[buf][1][lane] = x;
  };
  float st = 0.0f;
  if (nt > 0) {
    tq.load(lq[0], lo, wave);
    tdo.load(ldo[0], lo, wave);
    st = load_stat(lo);
    store_stat(0, st);
  }
  wait_all_loads();

  const int key = k0 + kc;
  for (int j = 0; j < nt; ++j) {
    const int buf = j & 1;
    const bool pre = j + 1 < nt;
    if (pre) {
      tq.load(lq[buf ^ 1], lo + (j + 1) * 64, wave);
      tdo.load(ldo[buf ^ 1], lo + (j + 1) * 64, wave);
      st = load_stat(lo + (j + 1) * 64);
    }
    if (j >= ta && j <= tb) {
      const int r0 = lo + 64 * j;                    // first query of the tile
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        // S and dP for queries r0 + 32 qb + crow(v, h) (rows) and key k0 + kc (column).
        v16f s = v16f{}, dp = v16f{};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          s = mfma16(nat_frag<D>(lq[buf], qb, ks, lane), kf[ks], s);
          dp = mfma16(nat_frag<D>(ldo[buf], qb, ks, lane), vf[ks], dp);
        }
        const int q0b = r0 + 32 * qb;
        if (!(q0b >= k0 + 31 && q0b + 31 - k0 < W)) {
#pragma unroll
          for (int v = 0; v < 16; ++v)
            if ((unsigned)(q0b + crow(v, h) - key) >= (unsigned)W) s[v] = -INFINITY;
        }
        // Rows crow(4 i + e, h) = 8 i + 4 h + e: four consecutive stats per i.
        const float4* nl4 = reinterpret_cast<const float4*>(&lstat[buf][0][32 * qb + 4 * h]);
        const float4* dl4 = reinterpret_cast<const float4*>(&lstat[buf][1][32 * qb + 4 * h]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 nl = nl4[2 * i], dl = dl4[2 * i];
          const float nla[4] = {nl.x, nl.y, nl.z, nl.w}, dla[4] = {dl.x, dl.y, dl.z, dl.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int v = 4 * i + e;
            const float pr = __builtin_amdgcn_exp2f(fmaf(s[v], c, nla[e]));
            s[v] = pr;
            dp[v] = pr * (dp[v] - dla[e]);           // dS / sm_scale
          }
        }
        // dV += P^T dO, dK += dS^T Q: A = this lane's key row, K = the 32 queries of block qb.
#pragma unroll
        for (int hs = 0; hs < 2; ++hs) {
          const v8bf pa = pack_frag(s, hs), da = pack_frag(dp, hs);
#pragma unroll
          for (int db = 0; db < NDB; ++db) {
            dv[db] = mfma16(pa, trr_frag<D>(ldo[buf], db, 2 * qb + hs, lane), dv[db]);
            dk[db] = mfma16(da, trr_frag<D>(lq[buf], db, 2 * qb + hs, lane), dk[db]);
          }
        }
      }
    }
    if (pre) store_stat(buf ^ 1, st);
    __builtin_amdgcn_s_waitcnt(0x0F70);             // vmcnt(0): this wave's tile loads landed
    __syncthreads();
  }

  // The A operands' rows were keys, the B operands' columns dims: lane (dim 32 db + lane % 32)
  // holds dK / dV of the keys k0 + crow(v, h). dK carries the softmax scale left out of dS.
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int kr = k0 + crow(v, h), d = 32 * db + kc;
      if (kr < T) {
        p.out2[slice + (int64_t)kr * D + d] = (uint16_t)f32_to_bf16_bits(dk[db][v] * p.sm_scale);
        p.out3[slice + (int64_t)kr * D + d] = (uint16_t)f32_to_bf16_bits(dv[db][v]);
      }
    }
}

// ---------------------------------------------------------------- backward: dQ

template <int D>
__global__ __launch_bounds__(256, D == 128 ? 1 : 3) void swa_bf16_dq_kernel(SwaB16Params p) {
  constexpr int KS = D / 16, NDB = D / 32, NAT = 64 * D * 2;
  __shared__ __align__(16) uint8_t lk[2][NAT];     // K tile: A operand of S^T, read transposed for dQ^T
  __shared__ __align__(16) uint8_t lv[2][NAT];     // V tile, natural (A operand of dP^T)
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), h = lane >> 5, qc = lane & 31;
  int bh, mt;
  band_order(p, false, bh, mt);
  const int T = p.T, W = p.W;
  const int m0 = mt * 128, q0 = m0 + 32 * wave;
  const int64_t slice = (int64_t)bh * T * D;
  const uint16_t* K = p.k + slice;
  const uint16_t* V = p.v + slice;
  const float c = p.sm_scale * kLog2eB;
  const int qi = q0 + qc;
  const float nlse2 = qi < T ? -p.lse[(int64_t)bh * T + qi] * kLog2eB : 0.0f;
  const float dl = qi < T ? p.delta[(int64_t)bh * T + qi] : 0.0f;

  v8bf qf[KS], df[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    qf[ks] = row_frag<D>(p.q + slice, qi, T, ks, lane);
    df[ks] = row_frag<D>(p.dout + o_base(p, bh, D), qi, T, ks, lane, o_ld(p, D));
  }
  v16f dq[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dq[db] = v16f{};

  const int lo_raw = m0 - W + 1;
  const int lo = lo_raw <= 0 ? 0 : (lo_raw & ~63);
  const int hi = min(T, m0 + 128);
  const int nt = hi > lo ? (hi - lo + 63) / 64 : 0;
  const int wk0 = max(0, q0 - W + 1), wk1 = min(q0 + 31, T - 1);
  const int ta = q0 < T ? (wk0 - lo) / 64 : 1;
  const int tb = q0 < T ? (wk1 - lo) / 64 : 0;

  TileLoadLds<D> tk, tv;
  tk.init(K, T, wave, lane);
  tv.init(V, T, wave, lane);
  if (nt > 0) {
    tk.load(lk[0], lo, wave);
    tv.load(lv[0], lo, wave);
  }
  wait_all_loads();

  for (int j = 0; j < nt; ++j) {
    const int buf = j & 1;
    const bool pre = j + 1 < nt;
    if (pre) {
      tk.load(lk[buf ^ 1], lo + (j + 1) * 64, wave);
      tv.load(lv[buf ^ 1], lo + (j + 1) * 64, wave);
    }
    if (j >= ta && j <= tb) {
      const int n0 = lo + 64 * j;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        v16f s = v16f{}, dp = v16f{};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          s = mfma16(nat_frag<D>(lk[buf], b, ks, lane), qf[ks], s);
          dp = mfma16(nat_frag<D>(lv[buf], b, ks, lane), df[ks], dp);
        }
        // Keys past T are zeros (S = 0, dP = 0) and meet K^T = 0 in dQ: no compare needed for
        // them; queries past T are never stored. Only the band 0 <= i - j < W is masked.
        const int kb0 = n0 + 32 * b;
        if (!(q0 >= kb0 + 31 && q0 + 31 - kb0 < W)) {
#pragma unroll
          for (int v = 0; v < 16; ++v)
            if ((unsigned)(qi - kb0 - crow(v, h)) >= (unsigned)W) s[v] = -INFINITY;
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float pr = __builtin_amdgcn_exp2f(fmaf(s[v], c, nlse2));
          dp[v] = pr * (dp[v] - dl);                  // dS / sm_scale
        }
        // dQ^T += K^T dS^T: A = K^T (dims as rows, keys of block b as K), B = dS^T (this lane's query).
#pragma unroll
        for (int hs = 0; hs < 2; ++hs) {
          const v8bf db_ = pack_frag(dp, hs);
#pragma unroll
          for (int db = 0; db < NDB; ++db) dq[db] = mfma16(trr_frag<D>(lk[buf], db, 2 * b + hs, lane), db_, dq[db]);
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);             // vmcnt(0): this wave's tile loads landed
    __syncthreads();
  }

  if (qi < T) {
    uint16_t* op = p.out + slice + (int64_t)qi * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = 32 * db + 8 * j + 4 * h;
        uint2 w;
        w.x = pk_bf16(dq[db][4 * j] * p.sm_scale, dq[db][4 * j + 1] * p.sm_scale);
        w.y = pk_bf16(dq[db][4 * j + 2] * p.sm_scale, dq[db][4 * j + 3] * p.sm_scale);
        *reinterpret_cast<uint2*>(op + d) = w;
      }
  }
}

// ---------------------------------------------------------------- host

static int check_b16(const void* a, const void* b, const void* c, int64_t B, int64_t H, int64_t T, int64_t D,
                     int64_t window) {
  FLW_REQUIRE(a && b && c, FLW_E_INVALID, "null pointer argument");
  FLW_REQUIRE(D == 32 || D == 64 || D == 128, FLW_E_UNSUPPORTED, "head_dim must be 32/64/128, got %lld", (long long)D);
  FLW_REQUIRE(B > 0 && H > 0 && T > 0, FLW_E_INVALID, "empty shape");
  FLW_REQUIRE(window > 0, FLW_E_INVALID, "window must be positive");
  FLW_REQUIRE(T <= (1 << 30) && B * H * ((T + 127) / 128) <= 0x7FFFFFFF, FLW_E_UNSUPPORTED, "shape too large");
  FLW_REQUIRE(((uintptr_t)a & 15) == 0 && ((uintptr_t)b & 15) == 0 && ((uintptr_t)c & 15) == 0, FLW_E_INVALID,
              "tensors must be 16-byte aligned");
  return FLW_OK;
}

// Query blocks whose band starts at key 0 (shorter than W + 127 keys): the first ceil(W / 128).
static int query_ramp(const SwaB16Params& p) {
  return p.W > 0 ? std::min(p.nblk, (p.W - 1) / 128 + 1) : 0;
}
// Key blocks whose band of queries ends at T - 1 before its full W + 127: the last ones.
static int key_ramp(const SwaB16Params& p) {
  const int64_t span = (int64_t)p.T - p.W - 127;
  const int nfull = span < 0 ? 0 : std::min<int64_t>(p.nblk, span / 128 + 1);
  return p.nblk - nfull;
}
static int group_slices(int64_t slices, int nwg) {
  return (slices % 8 == 0 && (nwg & 7) == 0) ? (int)(slices / 8) : (int)slices;
}

}  // namespace flw

using namespace flw;

static int o_layout_check(int layout, int64_t B, int64_t H, int64_t T, int64_t D) {
  FLW_REQUIRE(layout == FLW_LAYOUT_BHTD || layout == FLW_LAYOUT_BTHD, FLW_E_INVALID,
              "out layout must be FLW_LAYOUT_BHTD or FLW_LAYOUT_BTHD, got %d", layout);
  FLW_REQUIRE(layout == FLW_LAYOUT_BHTD || T * H * D * 2 <= 0x7FFFFFFFll, FLW_E_UNSUPPORTED,
              "a (B, T, H, D) slice must span < 2^31 bytes");
  (void)B;
  return FLW_OK;
}

static int swa_bf16_fwd(const void* q, const void* k, const void* v, int64_t B, int64_t H, int64_t T, int64_t D,
                        int64_t window, void* out, int out_layout, float* lse, void* stream, const char* name) {
  int rc = check_b16(q, k, v, B, H, T, D, window);
  if (rc) return rc;
  rc = o_layout_check(out_layout, B, H, T, D);
  if (rc) return rc;
  FLW_REQUIRE(out && lse && ((uintptr_t)out & 15) == 0, FLW_E_INVALID, "out / lse");
  SwaB16Params p{};
  p.o_tmaj = out_layout == FLW_LAYOUT_BTHD;
  p.q = static_cast<const uint16_t*>(q); p.k = static_cast<const uint16_t*>(k); p.v = static_cast<const uint16_t*>(v);
  p.out = static_cast<uint16_t*>(out); p.lse = lse;
  p.H = (int)H; p.T = (int)T; p.W = (int)(window < T ? window : T);
  p.nblk = (int)((T + 127) / 128); p.nwg = (int)(B * H * p.nblk);
  p.ramp = query_ramp(p);
  p.group_slices = group_slices(B * H, p.nwg);
  p.sm_scale = 1.0f / sqrtf((float)D);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)p.nwg);
  const void* kf = D == 32 ? reinterpret_cast<const void*>(&swa_bf16_fwd_kernel<32>)
                 : D == 64 ? reinterpret_cast<const void*>(&swa_bf16_fwd_kernel<64>)
                           : reinterpret_cast<const void*>(&swa_bf16_fwd_kernel<128>);
  (void)launch_timed(kf, grid, dim3(256), s, p);
  return check_launch(name);
}

extern "C" int flw_swa_bf16_fwd(const void* q, const void* k, const void* v, int64_t B, int64_t H,
                                int64_t T, int64_t D, int64_t window, void* out, float* lse,
                                void* stream) {
  return swa_bf16_fwd(q, k, v, B, H, T, D, window, out, FLW_LAYOUT_BHTD, lse, stream, "flw_swa_bf16_fwd");
}

extern "C" int flw_swa_bf16_fwd_layout(const void* q, const void* k, const void* v, int64_t B, int64_t H,
                                       int64_t T, int64_t D, int64_t window, void* out, int out_layout, float* lse,
                                       void* stream) {
  return swa_bf16_fwd(q, k, v, B, H, T, D, window, out, out_layout, lse, stream, "flw_swa_bf16_fwd_layout");
}

extern "C" size_t flw_swa_bf16_bwd_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D) {
  (void)D;
  return (size_t)(B * H * T) * sizeof(float);
}

static int swa_bf16_bwd(const void* q, const void* k, const void* v, const void* out, const void* dout,
                        int o_layout, const float* lse, int64_t B, int64_t H, int64_t T, int64_t D, int64_t window,
                        void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes, void* stream,
                        const char* name) {
  int rc = check_b16(q, k, v, B, H, T, D, window);
  if (rc) return rc;
  rc = o_layout_check(o_layout, B, H, T, D);
  if (rc) return rc;
  FLW_REQUIRE(out && dout && lse && dq && dk && dv, FLW_E_INVALID, "null pointer argument");
  FLW_REQUIRE(((uintptr_t)out & 15) == 0 && ((uintptr_t)dout & 15) == 0 && ((uintptr_t)dq & 15) == 0 &&
              ((uintptr_t)dk & 1) == 0 && ((uintptr_t)dv & 1) == 0, FLW_E_INVALID, "misaligned tensor");
  const size_t need = flw_swa_bf16_bwd_workspace_bytes(B, H, T, D);
  FLW_REQUIRE(workspace && workspace_bytes >= need, FLW_E_WORKSPACE, "workspace needs %zu bytes", need);
  SwaB16Params p{};
  p.q = static_cast<const uint16_t*>(q); p.k = static_cast<const uint16_t*>(k); p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<const uint16_t*>(out); p.dout = static_cast<const uint16_t*>(dout);
  p.o_tmaj = o_layout == FLW_LAYOUT_BTHD;
  p.lse = const_cast<float*>(lse); p.delta = static_cast<float*>(workspace);
  p.H = (int)H; p.T = (int)T; p.W = (int)(window < T ? window : T);
  p.nblk = (int)((T + 127) / 128); p.nwg = (int)(B * H * p.nblk);
  p.sm_scale = 1.0f / sqrtf((float)D);
  hipStream_t s = static_cast<hipStream_t>(stream);
  p.rows = B * H * T;
  const int64_t threads = p.rows * (D / 8);
  const dim3 dgrid((unsigned)((threads + 255) / 256));
  const dim3 grid((unsigned)p.nwg);
  p.group_slices = group_slices(B * H, p.nwg);
  SwaB16Params pk = p;
  pk.out2 = static_cast<uint16_t*>(dk); pk.out3 = static_cast<uint16_t*>(dv);
  pk.ramp = key_ramp(p);
  SwaB16Params pq = p;
  pq.out = static_cast<uint16_t*>(dq);
  pq.ramp = query_ramp(p);
  const void* kd = D == 32 ? reinterpret_cast<const void*>(&swa_bf16_delta_kernel<32>)
                 : D == 64 ? reinterpret_cast<const void*>(&swa_bf16_delta_kernel<64>)
                           : reinterpret_cast<const void*>(&swa_bf16_delta_kernel<128>);
  const void* kk = D == 32 ? reinterpret_cast<const void*>(&swa_bf16_dkdv_kernel<32>)
                 : D == 64 ? reinterpret_cast<const void*>(&swa_bf16_dkdv_kernel<64>)
                           : reinterpret_cast<const void*>(&swa_bf16_dkdv_kernel<128>);
  const void* kq = D == 32 ? reinterpret_cast<const void*>(&swa_bf16_dq_kernel<32>)
                 : D == 64 ? reinterpret_cast<const void*>(&swa_bf16_dq_kernel<64>)
                           : reinterpret_cast<const void*>(&swa_bf16_dq_kernel<128>);
  const Timer tm = take_timer();   // start on the delta kernel, stop on the dQ kernel
  (void)launch_ext(kd, dgrid, dim3(256), 0, s, p, tm.start, nullptr);
  (void)launch_ext(kk, grid, dim3(256), 0, s, pk, nullptr, nullptr);
  (void)launch_ext(kq, grid, dim3(256), 0, s, pq, nullptr, tm.stop);
  return check_launch(name);
}

extern "C" int flw_swa_bf16_bwd(const void* q, const void* k, const void* v, const void* out,
                                const void* dout, const float* lse, int64_t B, int64_t H, int64_t T,
                                int64_t D, int64_t window, void* dq, void* dk, void* dv,
                                void* workspace, size_t workspace_bytes, void* stream) {
  return swa_bf16_bwd(q, k, v, out, dout, FLW_LAYOUT_BHTD, lse, B, H, T, D, window, dq, dk, dv, workspace,
                      workspace_bytes, stream, "flw_swa_bf16_bwd");
}

extern "C" int flw_swa_bf16_bwd_layout(const void* q, const void* k, const void* v, const void* out,
                                       const void* dout, int o_layout, const float* lse, int64_t B, int64_t H,
                                       int64_t T, int64_t D, int64_t window, void* dq, void* dk, void* dv,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  return swa_bf16_bwd(q, k, v, out, dout, o_layout, lse, B, H, T, D, window, dq, dk, dv, workspace,
                      workspace_bytes, stream, "flw_swa_bf16_bwd_layout");
}
