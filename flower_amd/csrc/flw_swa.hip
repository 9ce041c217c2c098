// FP8 causal sliding-window attention forward for gfx950 (CDNA4).
//
// Work decomposition: one workgroup = 4 waves = 128 queries of one (b, h) slice; each wave owns
// 32 queries. The workgroup walks 64-key tiles over its band [m0 - W + 1, m0 + 127] only (tiles
// wholly outside the window are never visited); a wave computes only the tiles that meet its own
// 32-query band. Per tile a wave computes S^T = K Q^T with two v_mfma_f32_32x32x64_f8f6f4 (keys
// are the MFMA rows, queries the columns, so every lane holds 32 scores of ONE query and the row
// max / sum are lane-local plus one v_permlane32_swap with lane^32), runs the online softmax in
// base 2 with the softmax scale, log2(e) and the x448 P pre-scale folded into one FMA, packs P to
// e4m3 in registers (v_cvt_pk_fp8_f32) straight into the B operand of O^T += V^T P^T (D/32 more
// MFMAs, accumulators kept in VGPRs so the rescale is one multiply per element).
//
// The softmax is VALU-bound. Per score: one FMA, one v_exp_f32 and half a v_cvt_pk_fp8_f32
// (each of those two costs about three full-rate issue slots on gfx950), half a max3, one add,
// and D/64 rescale multiplies per tile; the MFMA work of a tile is about a third of its VALU
// time. Inside a wave every step depends on the previous one, so the MFMA time hides only under
// the other waves of the SIMD (four workgroups per CU at D <= 64: 120 VGPRs, 24 KB of LDS each);
// a wave raises its priority for its softmax and drops it to issue its MFMAs, which keeps the
// VALU fed. Software-pipelining the tiles inside a wave (the next tile's QK^T and the previous
// tile's PV issued between the current tile's exponentials) was measured slower.
//
// K tiles are staged in LDS in MFMA-fragment order (a permutation of 16-byte chunks of the
// row-major tile); V arrives already in that order from the quantiser (FLW_LAYOUT_VTILE), so every
// fragment read is a conflict-free linear ds_read_b128. Three LDS stages, one barrier per tile:
// the global loads of tile j+2 are in flight while tile j is consumed. Workgroups are dealt to
// the 8 XCDs so that each XCD works through contiguous query tiles of the same heads and re-reads
// K/V from its own L2.
#include <math.h>

#include <algorithm>

#include <type_traits>

#include "flw_common.h"

namespace flw {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16f mfma_32x32x64_f8(v8i a, v8i b, v16f c) {
  // cbsz = blgp = 0: both operands are FP8 E4M3; no block scales.
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

constexpr int kWaves = 4;
constexpr int kBM = 32 * kWaves;   // queries per workgroup
constexpr int kBN = 64;            // keys per tile
constexpr int kStages = 3;         // LDS ring of K/V tiles
constexpr int kBufferFlags = 0x00020000;   // buffer descriptor word 3 for raw dword access (gfx9)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLog2_448 = 8.807354922057604f;   // log2(448): P is produced pre-scaled by 448

struct SwaParams {
  const uint8_t* q8;
  const uint8_t* k8;
  const uint8_t* vt;
  int64_t qsb, qsh, qst;      // byte strides of q8
  int64_t ksb, ksh, kst;      // byte strides of k8
  int64_t vt_slice;           // bytes per (b, h) slice of the tiled V
  int64_t vsb, vsh, vst;      // byte strides of V when it is given as (B, H, T, D) codes (vt then
                              // points at those codes; the kernel instance with VB set)
  const float* qs;
  const float* ks;
  const float* vs;
  int64_t ssb, ssh;           // element strides of b and h in the scale arrays (0/0 tensor, 0/1 head, H/1 (b, h))
  void* out;
  int64_t osb, osh, ost;      // element strides of out
  int H, T, W, nM, nwg;
  int ramp;                   // query tiles per slice whose band starts at key 0 (fewer key tiles)
  int group_slices;           // slices per dispatch group (one XCD's share when it is whole slices)
  // Optional: Q in the output's dtype (element strides), quantised on load with the reciprocals
  // qr (RN(1 / q scale)) for scale groups whose scale is finite; q8 serves the others.
  const void* qx;
  int64_t xsb, xsh, xst;
  const float* qr;
  // Optional with qx: the caller-given |q| maximum of each scale group (fp32 bit patterns) that
  // the scale was derived from. A lane holding a larger |q| (a stale or wrong maximum) takes the
  // exact path for its values: IEEE division, clamp to +-448, then the cast.
  const uint32_t* qamax;
  // Optional: the log-sum-exp of each query's scores, [B, H, T] fp32, natural log, in the units of
  // the dequantised scores (q . k / sqrt(D)): lse = m + ln(sum_j exp(s_j - m)) -- what a
  // recomputing backward (flw_swa_bf16_bwd) needs to rebuild P.
  float* lse;
};

template <typename OutT> struct Store4;
template <> struct Store4<float> {
  __device__ __forceinline__ static void st(float* p, float a, float b, float c, float d) {
    *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
  }
};
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
template <> struct Store4<uint16_t> {
  // v_cvt_pk_bf16_f32: round to nearest even, two values per instruction.
  __device__ __forceinline__ static void st(uint16_t* p, float a, float b, float c, float d) {
    uint2 w;
    w.x = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), bf16x2));
    w.y = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{c, d}), bf16x2));
    *reinterpret_cast<uint2*>(p) = w;
  }
};

__device__ __forceinline__ v8i load_frag(const uint8_t* lds, int off) {
  const uint4 a = *reinterpret_cast<const uint4*>(lds + off);
  const uint4 b = *reinterpret_cast<const uint4*>(lds + off + 1024);
  v8i r;
  r[0] = (int)a.x; r[1] = (int)a.y; r[2] = (int)a.z; r[3] = (int)a.w;
  r[4] = (int)b.x; r[5] = (int)b.y; r[6] = (int)b.z; r[7] = (int)b.w;
  return r;
}

// The PV operand fragment of dims 32 db .. 32 db + 31 from a row-staged V tile (vrow_offset),
// byte for byte the tiled V's fragment (load_frag): lane (d = lane % 32, h = lane / 32) holds the
// runs of key blocks 0 and 1 for its dim (vtile_run).
template <int D>
__device__ __forceinline__ v8i vtr_frag(const uint8_t* lds, int db, int lane) {
  const int n = lane & 15, d0 = 32 * db + 16 * ((lane >> 4) & 1), h = lane >> 5;
  const uint4 a = vtile_run(lds, D, d0, 0, h, n), b = vtile_run(lds, D, d0, 1, h, n);
  return v8i{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
}

// A K fragment (32 keys x 64 bytes for this lane) from its swizzled region (offsets from the lane).
__device__ __forceinline__ v8i load_kfrag(const uint8_t* lds, int region, int x0, int x1) {
  const uint4 a = *reinterpret_cast<const uint4*>(lds + region + x0);
  const uint4 b = *reinterpret_cast<const uint4*>(lds + region + x1);
  return v8i{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
}

// clamp(y, -448, 448) on the bit pattern (this file is built without NaN semantics, so a float
// comparison could not be trusted to keep a NaN): |y| above 448, inf included, becomes +-448;
// NaN is kept.
__device__ __forceinline__ float clamp448_bits(float y) {
  const uint32_t u = __float_as_uint(y), a = u & 0x7FFFFFFFu;
  return a > 0x43E00000u && a <= 0x7F800000u ? __uint_as_float((u & 0x80000000u) | 0x43E00000u) : y;
}

// x combined with its value in lane ^ 32 (the other half of the same query's keys).
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Scores of one 64-key tile for one wave: S^T blocks of keys n0 .. n0+31 and n0+32 .. n0+63.
// Lane (qcol = lane % 32, hh = lane / 32), element v of block blk holds key
// n0 + 32 blk + 8 (v / 4) + 4 hh + v % 4 of query q0 + qcol.
struct Scores {
  v16f s0, s1;
};

// At D <= 64 the kernel takes 120 VGPRs (D = 32: 110), so four workgroups (16 waves) share a CU;
// the launch bound only asks for three. D = 128 asks for two (its O^T needs 64 VGPRs more).
// VB: V arrives as (B, H, T, D) e4m3 codes (the reference's layout, strides vsb / vsh / vst). Its
// tiles are staged as they are (64 key rows of D bytes, swizzled as vrow_offset places them)
// and the PV operand is read with ds_read_b64_tr_b8, which hands each lane one dim of 8 key rows:
// the same bytes in the same order as the tiled V's fragment reads, so the results are those of
// the tiled-V instance.
template <int D, typename OutT, bool VB = false>
__global__ __launch_bounds__(256, D == 128 ? 2 : 3) void swa_fwd_kernel(SwaParams p) {
  constexpr int NDC = D >= 64 ? D / 64 : 1;   // 64-deep K chunks of the QK^T product
  constexpr int NDB = D / 32;                  // 32-row blocks of O^T
  constexpr int KT_BYTES = 2 * NDC * 2048;     // one K tile in fragment order
  constexpr int VT_BYTES = 64 * D;             // one V tile (VTILE layout)
  constexpr int CPR = D / 16;                  // 16-byte chunks per K row
  constexpr int KCH = 64 * CPR;                // chunks per K tile (== V tile chunks)
  constexpr int CPT = (KCH + 255) / 256;       // chunks per thread
  __shared__ __align__(16) uint8_t lds_k[kStages][KT_BYTES];
  __shared__ __align__(16) uint8_t lds_v[kStages][VT_BYTES];

  // Work-item / group ids through the builtins (this file is built without IEEE mode, and the
  // device-library accessors are not inlined across that mode difference).
  const int tid = (int)__builtin_amdgcn_workitem_id_x(), lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar branches
  const int nwg = p.nwg;
  int L = (int)__builtin_amdgcn_workgroup_id_x();
  // Contiguous work per XCD when the slices split evenly over the 8 XCDs (each XCD then takes
  // whole slices); otherwise the workgroups stay dealt round-robin over the XCDs, so every XCD
  // gets an even share of the long and the short work items of the order below.
  if (p.group_slices * 8 * p.nM == nwg) L = (L & 7) * (nwg >> 3) + (L >> 3);
  // Inside a group of slices (one XCD's share), the full-band query tiles come first, slice by
  // slice (consecutive tiles share K / V tiles in that XCD's L2), then the causal-ramp tiles in
  // decreasing length, so the short work items fill the end of the grid as the long ones drain.
  int bh, mt;
  {
    const int gs = p.group_slices, nfull_t = p.nM - p.ramp;
    const int gi = L / (gs * p.nM), i = L % (gs * p.nM);
    if (i < gs * nfull_t) {
      bh = gi * gs + i / nfull_t;
      mt = p.ramp + i % nfull_t;
    } else {
      const int j = i - gs * nfull_t;
      bh = gi * gs + j % gs;
      mt = p.ramp - 1 - j / gs;
    }
  }
  const int b = bh / p.H, h = bh % p.H;
  const int T = p.T, W = p.W;
  const int m0 = mt * kBM;
  const int q0 = m0 + 32 * wave;
  const int qcol = lane & 31, hh = lane >> 5;

  const int64_t si = b * p.ssb + h * p.ssh;
  const float q_s = p.qs[si], k_s = p.ks[si], v_s = p.vs[si];
  const float rsd = D == 32 ? 0.17677669529663687f : (D == 64 ? 0.125f : 0.08838834764831845f);
  const float c = q_s * k_s * rsd * kLog2e;

  // Q fragments: B operand of S^T = K Q^T; lane (qcol, hh) holds Q[q][64 dc + 32 hh + 0..31].
  // With Q given in its input dtype, the lane quantises its 32 values here with the quantiser's
  // arithmetic (x / s as x * RN(1/s) plus one FMA correction, then v_cvt_pk_fp8_f32), so the
  // codes are the ones the quantise pass would have written; groups whose scale is not finite
  // (NaN / inf amax, the exact path) were coded by the quantiser and are read from q8.
  v8i qf[NDC];
  const int qi_ld = q0 + qcol < T ? q0 + qcol : T - 1;
  if (p.qx != nullptr && finite_bits(q_s)) {                  // uniform over the workgroup
    const float qrcp = p.qr[si];
    const OutT* qx = static_cast<const OutT*>(p.qx) + b * p.xsb + h * p.xsh + (int64_t)qi_ld * p.xst;
    using QV = Vec16<OutT>;
#pragma unroll
    for (int dc = 0; dc < NDC; ++dc) {
      if (D == 32 && hh) {
        qf[dc] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
        continue;
      }
      float f[32];
#pragma unroll
      for (int j = 0; j < 32 / QV::N; ++j) QV::load(qx + 64 * dc + 32 * hh + j * QV::N, f + j * QV::N);
      bool exact = false;
      if (p.qamax != nullptr) {                     // values beyond the given maximum?
        const uint32_t g = p.qamax[si];
        const uint32_t lim = (int32_t)g > 0 ? g : 0u;   // a given maximum <= 0 admits only zeros
        uint32_t m = 0;
#pragma unroll
        for (int j = 0; j < 32; ++j) { const uint32_t a = abs_bits(f[j]); m = m > a ? m : a; }
        exact = m > lim;
      }
      if (!exact) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          int c = __builtin_amdgcn_cvt_pk_fp8_f32(div_by_scale(f[4 * j], q_s, qrcp),
                                                  div_by_scale(f[4 * j + 1], q_s, qrcp), 0, false);
          c = __builtin_amdgcn_cvt_pk_fp8_f32(div_by_scale(f[4 * j + 2], q_s, qrcp),
                                              div_by_scale(f[4 * j + 3], q_s, qrcp), c, true);
          qf[dc][j] = c;
        }
      } else {                                      // rare: the reference's clamp, then the cast
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          uint32_t c = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            c |= (f32_to_e4m3(clamp448_bits(f[4 * j + e] / q_s)) & 0xFFu) << (8 * e);   // IEEE division
          qf[dc][j] = (int)c;
        }
      }
    }
  } else {
    const int qi = qi_ld;
    const uint8_t* qp = p.q8 + b * p.qsb + h * p.qsh + (int64_t)qi * p.qst;
#pragma unroll
    for (int dc = 0; dc < NDC; ++dc) {
      if (D == 32 && hh) {
        qf[dc] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
      } else {
        const uint4 a = *reinterpret_cast<const uint4*>(qp + 64 * dc + 32 * hh);
        const uint4 bq = *reinterpret_cast<const uint4*>(qp + 64 * dc + 32 * hh + 16);
        qf[dc] = v8i{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)bq.x, (int)bq.y, (int)bq.z, (int)bq.w};
      }
    }
  }

  // K rows: scalar tile base + a fixed 32-bit offset per thread; V tiles are contiguous.
  const uint8_t* kbase = p.k8 + b * p.ksb + h * p.ksh;
  const uint8_t* vbase = VB ? p.vt + b * p.vsb + h * p.vsh : p.vt + (int64_t)bh * p.vt_slice;
  uint32_t koff[CPT], ldsk[CPT];
  // VB: the chunk's V row offset and its swizzled place in the staged tile.
  uint32_t voff[VB ? CPT : 1], ldsv[VB ? CPT : 1];
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int i = min(tid + 256 * j, KCH - 1);
    const int kk = i / CPR, g = i % CPR;
    const int d0 = 16 * g;
    const int blk = kk >> 5, krow = kk & 31, dc = d0 >> 6, h2 = (d0 >> 5) & 1, cc = (d0 >> 4) & 1;
    koff[j] = (uint32_t)(kk * p.kst + 16 * g);
    if constexpr (VB) {
      voff[j] = (uint32_t)(kk * p.vst + 16 * g);
      ldsv[j] = (uint32_t)vrow_offset(kk, g, D);
    }
    // Chunk (krow + 32 h2) of fragment region (blk, dc, cc), its index XORed with 4 (h2 + 2 cc):
    // the 16 lanes of a ds_write_b128 phase (4 rows x 4 chunks) then fall in 16 distinct bank
    // groups, and the fragment reads below (one region and one lane half per phase) stay a
    // permutation of 16 consecutive chunks.
    ldsk[j] = (uint32_t)((((blk * NDC + dc) * 2 + cc) * 64 + ((krow + 32 * h2) ^ (4 * (h2 + 2 * cc)))) * 16);
  }
  uint4 kreg[CPT], vreg[CPT];

  // K and V tiles through buffer descriptors of the (b, h) slice: a fixed per-thread offset plus
  // the tile offset, both in the VGPR operand (the one the range check covers), so K rows past T
  // read as zero (they only meet queries past T, whose rows are not stored) and no load leaves
  // the slice. The host checks that the slice fits a 31-bit extent.
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(kbase), 0, (int)((int64_t)(T - 1) * p.kst + D), kBufferFlags);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(vbase), 0, VB ? (int)((int64_t)(T - 1) * p.vst + D) : (int)p.vt_slice, kBufferFlags);
  auto load_tile = [&](int n0) __attribute__((always_inline)) {
    const int ks = n0 * (int)p.kst, vs = (n0 >> 6) * VT_BYTES;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int i = tid + 256 * j;
      if (KCH % 256 == 0 || i < KCH) {
        const auto kv = __builtin_amdgcn_raw_buffer_load_b128(krs, (int)(koff[j] + (uint32_t)ks), 0, 0);
        kreg[j] = make_uint4(kv[0], kv[1], kv[2], kv[3]);
        // VB: V rows past T read as zero, the tiled V's padding keys
        std::remove_const_t<decltype(kv)> vv;
        if constexpr (VB) vv = __builtin_amdgcn_raw_buffer_load_b128(vrs, (int)(voff[j] + (uint32_t)(n0 * (int)p.vst)), 0, 0);
        else vv = __builtin_amdgcn_raw_buffer_load_b128(vrs, 16 * i, vs, 0);
        vreg[j] = make_uint4(vv[0], vv[1], vv[2], vv[3]);
      }
    }
  };
  auto store_tile = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int i = tid + 256 * j;
      if (KCH % 256 == 0 || i < KCH) {
        *reinterpret_cast<uint4*>(&lds_k[buf][ldsk[j]]) = kreg[j];
        if constexpr (VB) {
          *reinterpret_cast<uint4*>(&lds_v[buf][ldsv[j]]) = vreg[j];
        } else {
          *reinterpret_cast<uint4*>(&lds_v[buf][16 * i]) = vreg[j];
        }
      }
    }
  };

  // Key range of the workgroup, tile-aligned, and this wave's tiles [ta, tb] inside it.
  const int lo_raw = m0 - W + 1;
  const int lo = lo_raw <= 0 ? 0 : (lo_raw & ~(kBN - 1));
  const int hi = min(T, m0 + kBM);
  const int nt = hi > lo ? (hi - lo + kBN - 1) / kBN : 0;
  const int wk0 = max(0, q0 - W + 1), wk1 = min(q0 + 31, T - 1);
  const int ta = q0 < T ? (wk0 - lo) / kBN : 1;
  const int tb = q0 < T ? (wk1 - lo) / kBN : 0;

  v16f o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = v16f{};
  float m_run = -INFINITY, l_run = 0.0f;
  int pk[8] = {0, 0, 0, 0, 0, 0, 0, 0};     // e4m3 P of the current tile, packed 4 per word

  // This lane's swizzled chunk offsets in the two halves (cc = 0, 1) of a K fragment region.
  const int kx0 = (lane ^ (4 * hh)) * 16, kx1 = 1024 + (lane ^ (4 * hh + 8)) * 16;
  // S^T = K Q^T for the tile in LDS stage `buf`.
  auto qk = [&](Scores& s, int buf) __attribute__((always_inline)) {
    const uint8_t* lk = lds_k[buf];
    s.s0 = v16f{};
    s.s1 = v16f{};
#pragma unroll
    for (int dc = 0; dc < NDC; ++dc) {
      v8i k0 = load_kfrag(lk, (0 * NDC + dc) * 2 * 1024, kx0, kx1);
      v8i k1 = load_kfrag(lk, (1 * NDC + dc) * 2 * 1024, kx0, kx1);
      if (D == 32 && hh) { k0 = v8i{0, 0, 0, 0, 0, 0, 0, 0}; k1 = k0; }
      s.s0 = mfma_32x32x64_f8(k0, qf[dc], s.s0);
      s.s1 = mfma_32x32x64_f8(k1, qf[dc], s.s1);
    }
  };

  // Band masking per 32-key block of a tile. d0 = q0 - (first key of the block) is a multiple
  // of 32, so a block is partial under the causal condition only when d0 == 0, and then element
  // v of lane (qcol, hh) is valid iff kv(v) <= qcol - 4 hh (kv(v) = 8 (v / 4) + v % 4 is the
  // key's offset inside the block). When W is a multiple of 32 a block is partial under the
  // window condition only when d0 == W, with exactly the complementary pattern. Those 16
  // per-element lane masks are formed once (held as SGPR pairs), so masking such a block is one
  // v_cndmask per score. Blocks wholly outside the band become -inf; other windows fall back
  // to one unsigned compare of i - j against W per score.
  const bool w32 = (W & 31) == 0;
  bool diag[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) diag[v] = 8 * (v >> 2) + (v & 3) <= qcol - 4 * hh;

  auto mask_block = [&](v16f& sb, int blk, int n0) __attribute__((always_inline)) {
    const int d0 = q0 - n0 - 32 * blk;            // query q0 minus the block's first key
    const bool causal = d0 < 31;                   // some key of the block is after some query
    const bool window = d0 + 31 >= W;              // some pair is W or more apart
    if (!causal && !window) return;
    if (d0 < 0 || d0 - W > 30) {                   // no pair of the block is in the band
#pragma unroll
      for (int v = 0; v < 16; ++v) sb[v] = -INFINITY;
    } else if (causal && !window && d0 == 0) {
#pragma unroll
      for (int v = 0; v < 16; ++v) sb[v] = diag[v] ? sb[v] : -INFINITY;
    } else if (window && !causal && w32 && d0 == W) {
#pragma unroll
      for (int v = 0; v < 16; ++v) sb[v] = diag[v] ? -INFINITY : sb[v];
    } else {
      const int base = d0 + qcol - 4 * hh;         // i - j for element kv = 0 of this lane
#pragma unroll
      for (int v = 0; v < 16; ++v)
        sb[v] = (unsigned)(base - (8 * (v >> 2) + (v & 3))) < (unsigned)W ? sb[v] : -INFINITY;
    }
  };

  // Online softmax of one tile (the reference's update: m_new = max(m, rowmax S),
  // p = exp(S - m_new), alpha = exp(m - m_new), l = l alpha + sum p, O = O alpha + e4m3(448 p) V),
  // in base 2 with the scale folded in, then O^T += V^T P^T.
  auto softmax_pv = [&](Scores& s, int n0, int buf) __attribute__((always_inline)) {
    // A wave in its softmax issues ahead of the waves about to issue MFMAs (s_setprio 1 until
    // its PV), so the VALU stays fed and the matrix core works through the others' MFMAs.
    __builtin_amdgcn_s_setprio(1);
    // Keys past T only meet queries past T, whose rows are not stored.
    mask_block(s.s0, 0, n0);
    mask_block(s.s1, 1, n0);

    // Row max: four independent chains of v_max3 over 8 scores each.
    float mx[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float m = fmaxf(fmaxf(s.s0[4 * j], s.s0[4 * j + 1]), s.s0[4 * j + 2]);
      m = fmaxf(fmaxf(m, s.s0[4 * j + 3]), s.s1[4 * j]);
      m = fmaxf(fmaxf(m, s.s1[4 * j + 1]), s.s1[4 * j + 2]);
      mx[j] = fmaxf(m, s.s1[4 * j + 3]);
    }
    const float tmax = pair_max(fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3])));
    const float m_new = fmaxf(m_run, tmax);
    const float m_safe = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f((m_run - m_safe) * c);
    const float nb = kLog2_448 - m_safe * c;
    m_run = m_new;

    // P = 448 exp(S - m) as one FMA + exp2 per score, packed to e4m3 two at a time (the old
    // half of each packed word is overwritten, so last tile's codes serve as the old value).
    float ls[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a0 = __builtin_amdgcn_exp2f(fmaf(s.s0[4 * j + 0], c, nb));
      const float a1 = __builtin_amdgcn_exp2f(fmaf(s.s0[4 * j + 1], c, nb));
      const float a2 = __builtin_amdgcn_exp2f(fmaf(s.s0[4 * j + 2], c, nb));
      const float a3 = __builtin_amdgcn_exp2f(fmaf(s.s0[4 * j + 3], c, nb));
      const float b0 = __builtin_amdgcn_exp2f(fmaf(s.s1[4 * j + 0], c, nb));
      const float b1 = __builtin_amdgcn_exp2f(fmaf(s.s1[4 * j + 1], c, nb));
      const float b2 = __builtin_amdgcn_exp2f(fmaf(s.s1[4 * j + 2], c, nb));
      const float b3 = __builtin_amdgcn_exp2f(fmaf(s.s1[4 * j + 3], c, nb));
      ls[j] = ((a0 + a1) + (a2 + a3)) + ((b0 + b1) + (b2 + b3));
      pk[j] = __builtin_amdgcn_cvt_pk_fp8_f32(a0, a1, pk[j], false);
      pk[j] = __builtin_amdgcn_cvt_pk_fp8_f32(a2, a3, pk[j], true);
      pk[4 + j] = __builtin_amdgcn_cvt_pk_fp8_f32(b0, b1, pk[4 + j], false);
      pk[4 + j] = __builtin_amdgcn_cvt_pk_fp8_f32(b2, b3, pk[4 + j], true);
    }
    l_run = fmaf(l_run, alpha, (ls[0] + ls[1]) + (ls[2] + ls[3]));
    const v8i pf = v8i{pk[0], pk[1], pk[2], pk[3], pk[4], pk[5], pk[6], pk[7]};
    const uint8_t* lv = lds_v[buf];
    __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const v8i vf = VB ? vtr_frag<D>(lv, db, lane) : load_frag(lv, (db * 2 * 64 + lane) * 16);
      o[db] *= alpha;
      o[db] = mfma_32x32x64_f8(vf, pf, o[db]);
    }
  };

  // Prologue: stage tiles 0 and 1.
  if (nt > 0) { load_tile(lo); store_tile(0); }
  if (nt > 1) { load_tile(lo + kBN); store_tile(1); }
  // Retire every global load so far (Q fragments included) on all paths: the wait-count pass
  // then knows Q is resident inside the loop and does not drain the tile prefetch before each
  // QK^T MFMA. 0x0F70 = vmcnt(0), expcnt / lgkmcnt unconstrained.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();

  // One tile: prefetch tile j+2 (global -> registers), QK^T + softmax + PV of tile j from LDS
  // stage BUF (a compile-time constant, so LDS offsets are immediates), then park tile j+2 in
  // the stage tile j-1 used.
  Scores sc;
  auto step = [&](int j, auto bufc) __attribute__((always_inline)) {
    constexpr int BUF = decltype(bufc)::value;
    const bool pre = j + 2 < nt;
    if (pre) load_tile(lo + (j + 2) * kBN);
    if (j >= ta && j <= tb) {
      qk(sc, BUF);
      softmax_pv(sc, lo + j * kBN, BUF);
    }
    if (pre) store_tile((BUF + 2) % kStages);
    __syncthreads();
  };
  for (int j = 0; j < nt; j += kStages) {
    step(j, std::integral_constant<int, 0>{});
    if (j + 1 < nt) step(j + 1, std::integral_constant<int, 1>{});
    if (j + 2 < nt) step(j + 2, std::integral_constant<int, 2>{});
  }

  // Epilogue: out = O * v_scale / l   (l carries the x448 of P, matching pv_scale = v_s / 448)
  const float l_tot = pair_sum(l_run);
  const float inv = l_tot == 0.0f ? 0.0f : v_s / l_tot;
  const int qi = q0 + qcol;
  if (p.lse != nullptr && hh == 0 && qi < T) {
    // m c + log2(l / 448) is the base-2 log-sum-exp of the scores times log2(e): back to natural log
    constexpr float kLn2 = 0.6931471805599453f;
    p.lse[(int64_t)bh * T + qi] =
        l_tot == 0.0f ? -INFINITY : (fmaf(m_run, c, __builtin_amdgcn_logf(l_tot)) - kLog2_448) * kLn2;
  }
  if (qi < T) {
    OutT* op = static_cast<OutT*>(p.out) + b * p.osb + h * p.osh + (int64_t)qi * p.ost;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = 32 * db + 8 * j + 4 * hh;
        Store4<OutT>::st(op + d, o[db][4 * j] * inv, o[db][4 * j + 1] * inv,
                         o[db][4 * j + 2] * inv, o[db][4 * j + 3] * inv);
      }
    }
  }
}


template <int D>
static void launch_d(const SwaParams& p, int out_dtype, bool vb, dim3 grid, hipStream_t s, Timer tm) {
  const void* k = vb ? (out_dtype == FLW_F32 ? reinterpret_cast<const void*>(&swa_fwd_kernel<D, float, true>)
                                             : reinterpret_cast<const void*>(&swa_fwd_kernel<D, uint16_t, true>))
                     : (out_dtype == FLW_F32 ? reinterpret_cast<const void*>(&swa_fwd_kernel<D, float>)
                                             : reinterpret_cast<const void*>(&swa_fwd_kernel<D, uint16_t>));
  (void)launch_ext(k, grid, dim3(256), 0, s, p, tm.start, tm.stop);
}

static int swa_fwd(const uint8_t* q8, const int64_t* qst, const uint8_t* k8, const int64_t* kst,
                   const uint8_t* vt, const float* qs, const float* ks, const float* vs, int64_t ssb, int64_t ssh,
                   void* out, int out_dtype, const int64_t* ost, int64_t B, int64_t H, int64_t T,
                   int64_t D, int64_t window, hipStream_t stream, Timer tm, const void* qx = nullptr,
                   const int64_t* xst = nullptr, const float* qr = nullptr, const uint32_t* qamax = nullptr,
                   float* lse = nullptr, const int64_t* vst = nullptr) {
  FLW_REQUIRE(q8 && k8 && vt && qs && ks && vs && out && qst && kst && ost, FLW_E_INVALID, "null pointer argument");
  if (vst != nullptr) {
    for (int i = 0; i < 3; ++i)
      FLW_REQUIRE(vst[i] % 16 == 0 && vst[i] >= 0, FLW_E_INVALID, "v8 strides must be non-negative multiples of 16 bytes");
    FLW_REQUIRE((T - 1) * vst[2] + D < ((int64_t)1 << 31), FLW_E_UNSUPPORTED, "one (b, h) slice of v8 must span < 2^31 bytes");
  }
  if (qx != nullptr) {
    const int64_t vec = out_dtype == FLW_F32 ? 4 : 8;
    FLW_REQUIRE(xst != nullptr && qr != nullptr, FLW_E_INVALID, "null Q strides / reciprocals");
    FLW_REQUIRE(xst[0] % vec == 0 && xst[1] % vec == 0 && xst[2] % vec == 0 && ((uintptr_t)qx & 15) == 0,
                FLW_E_INVALID, "Q must have 16-byte aligned rows (strides multiples of %lld elements)", (long long)vec);
  }
  FLW_REQUIRE(D == 32 || D == 64 || D == 128, FLW_E_UNSUPPORTED, "head_dim must be 32/64/128, got %lld", (long long)D);
  FLW_REQUIRE(B > 0 && H > 0 && T > 0, FLW_E_INVALID, "empty shape");
  FLW_REQUIRE(out_dtype == FLW_F32 || out_dtype == FLW_BF16, FLW_E_UNSUPPORTED, "output dtype %d", out_dtype);
  FLW_REQUIRE(ssb >= 0 && ssh >= 0, FLW_E_INVALID, "scale strides must be non-negative");
  FLW_REQUIRE(T <= (int64_t)0x7FFFFF00, FLW_E_UNSUPPORTED, "T too large");
  for (int i = 0; i < 3; ++i) {
    FLW_REQUIRE(qst[i] % 16 == 0 && kst[i] % 16 == 0, FLW_E_INVALID, "q8/k8 strides must be multiples of 16 bytes");
    FLW_REQUIRE(ost[i] % 4 == 0, FLW_E_INVALID, "output strides must be multiples of 4 elements");
  }
  FLW_REQUIRE(((uintptr_t)q8 & 15) == 0 && ((uintptr_t)k8 & 15) == 0 && ((uintptr_t)vt & 15) == 0,
              FLW_E_INVALID, "q8 / k8 / v tiles must be 16-byte aligned");
  FLW_REQUIRE(((uintptr_t)out & 15) == 0, FLW_E_INVALID, "output must be 16-byte aligned");
  FLW_REQUIRE((T - 1) * kst[2] + D < ((int64_t)1 << 31) && (T + 63) / 64 * 64 * D < ((int64_t)1 << 31),
              FLW_E_UNSUPPORTED, "one (b, h) slice of k8 / v tiles must span < 2^31 bytes");
  const int64_t nM = (T + kBM - 1) / kBM;
  FLW_REQUIRE(B * H * nM <= 0x7FFFFFFF, FLW_E_UNSUPPORTED, "grid too large");
  int64_t W = window;
  if (W > T) W = T;       // i - j <= T - 1 < T: a window of T is already full causal
  if (W < 0) W = 0;
  SwaParams p{};
  p.q8 = q8; p.k8 = k8; p.vt = vt;
  p.qsb = qst[0]; p.qsh = qst[1]; p.qst = qst[2];
  p.ksb = kst[0]; p.ksh = kst[1]; p.kst = kst[2];
  p.vt_slice = ((T + 63) / 64) * 64 * D;
  if (vst != nullptr) { p.vsb = vst[0]; p.vsh = vst[1]; p.vst = vst[2]; }
  p.qs = qs; p.ks = ks; p.vs = vs; p.ssb = ssb; p.ssh = ssh;
  p.out = out; p.osb = ost[0]; p.osh = ost[1]; p.ost = ost[2];
  p.H = (int)H; p.T = (int)T; p.W = (int)W; p.nM = (int)nM;
  p.nwg = (int)(B * H * nM);
  p.qx = qx;
  p.qr = qr;
  p.qamax = qx != nullptr ? qamax : nullptr;
  p.lse = lse;
  FLW_REQUIRE(lse == nullptr || ((uintptr_t)lse & 3) == 0, FLW_E_INVALID, "lse must be 4-byte aligned");
  if (qx != nullptr) { p.xsb = xst[0]; p.xsh = xst[1]; p.xst = xst[2]; }
  p.ramp = W > 0 ? (int)std::min<int64_t>(nM, (W - 1) / kBM + 1) : 0;
  p.group_slices = ((B * H) % 8 == 0 && (p.nwg & 7) == 0) ? (int)(B * H / 8) : (int)(B * H);
  dim3 grid((unsigned)p.nwg);
  const bool vb = vst != nullptr;
  if (D == 32) launch_d<32>(p, out_dtype, vb, grid, stream, tm);
  else if (D == 64) launch_d<64>(p, out_dtype, vb, grid, stream, tm);
  else launch_d<128>(p, out_dtype, vb, grid, stream, tm);
  return check_launch("flw_fp8_swa_fwd");
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct SwaWorkspace {
  size_t q8, k8, vt, scales, qrcp, partials, total;
};

static SwaWorkspace swa_ws_layout(int64_t B, int64_t H, int64_t T, int64_t D) {
  SwaWorkspace w{};
  const size_t n = (size_t)(B * H * T * D);
  w.q8 = 0;
  w.k8 = align256(n);
  w.vt = w.k8 + align256(n);
  w.scales = w.vt + align256(flw_vtile_bytes(B, H, T, D));
  w.qrcp = w.scales + align256(3 * sizeof(float) * (size_t)(B * H));
  w.partials = w.qrcp + align256(sizeof(float) * (size_t)(B * H));
  w.total = w.partials + align256(3 * flw_quant_workspace_bytes(B, H, T, D));
  return w;
}

// Scale-array strides of a granularity: per tensor 0/0, per head 0/1, per (b, h) H/1.
static int scale_strides(int gran, int64_t H, int64_t* ssb, int64_t* ssh) {
  FLW_REQUIRE(gran >= FLW_SCALE_TENSOR && gran <= FLW_SCALE_BH, FLW_E_INVALID, "bad granularity %d", gran);
  *ssb = gran == FLW_SCALE_BH ? H : 0;
  *ssh = gran == FLW_SCALE_TENSOR ? 0 : 1;
  return FLW_OK;
}

}  // namespace flw

using namespace flw;

extern "C" int flw_fp8_swa_fwd_scale_strides(const uint8_t* q8, const int64_t* q_strides, const uint8_t* k8,
                                             const int64_t* k_strides, const uint8_t* v_tiles,
                                             const float* q_scale, const float* k_scale, const float* v_scale,
                                             int64_t scale_stride_b, int64_t scale_stride_h, void* out,
                                             int out_dtype, const int64_t* out_strides, int64_t B, int64_t H,
                                             int64_t T, int64_t D, int64_t window, void* stream) {
  return swa_fwd(q8, q_strides, k8, k_strides, v_tiles, q_scale, k_scale, v_scale, scale_stride_b,
                 scale_stride_h, out, out_dtype, out_strides, B, H, T, D, window,
                 static_cast<hipStream_t>(stream), take_timer());
}

extern "C" int flw_fp8_swa_fwd_bhtd(const uint8_t* q8, const int64_t* q_strides, const uint8_t* k8,
                                    const int64_t* k_strides, const uint8_t* v8, const int64_t* v_strides,
                                    const float* q_scale, const float* k_scale, const float* v_scale,
                                    int64_t scale_stride_b, int64_t scale_stride_h, void* out, int out_dtype,
                                    const int64_t* out_strides, int64_t B, int64_t H, int64_t T, int64_t D,
                                    int64_t window, void* stream) {
  FLW_REQUIRE(v_strides != nullptr, FLW_E_INVALID, "null v8 strides");
  return swa_fwd(q8, q_strides, k8, k_strides, v8, q_scale, k_scale, v_scale, scale_stride_b, scale_stride_h,
                 out, out_dtype, out_strides, B, H, T, D, window, static_cast<hipStream_t>(stream), take_timer(),
                 nullptr, nullptr, nullptr, nullptr, nullptr, v_strides);
}

extern "C" int flw_fp8_swa_fwd(const uint8_t* q8, const int64_t* q_strides, const uint8_t* k8,
                               const int64_t* k_strides, const uint8_t* v_tiles,
                               const float* q_scale, const float* k_scale, const float* v_scale,
                               int granularity, void* out, int out_dtype,
                               const int64_t* out_strides, int64_t B, int64_t H, int64_t T,
                               int64_t D, int64_t window, void* stream) {
  int64_t ssb, ssh;
  const int rc = scale_strides(granularity, H, &ssb, &ssh);
  if (rc) return rc;
  return swa_fwd(q8, q_strides, k8, k_strides, v_tiles, q_scale, k_scale, v_scale, ssb, ssh,
                 out, out_dtype, out_strides, B, H, T, D, window, static_cast<hipStream_t>(stream),
                 take_timer());
}

extern "C" int flw_fp8_swa_fwd_lse(const uint8_t* q8, const int64_t* q_strides, const uint8_t* k8,
                                   const int64_t* k_strides, const uint8_t* v_tiles, const float* q_scale,
                                   const float* k_scale, const float* v_scale, int granularity, void* out,
                                   int out_dtype, const int64_t* out_strides, int64_t B, int64_t H, int64_t T,
                                   int64_t D, int64_t window, float* lse, void* stream) {
  FLW_REQUIRE(lse != nullptr, FLW_E_INVALID, "null lse");
  int64_t ssb, ssh;
  const int rc = scale_strides(granularity, H, &ssb, &ssh);
  if (rc) return rc;
  return swa_fwd(q8, q_strides, k8, k_strides, v_tiles, q_scale, k_scale, v_scale, ssb, ssh, out, out_dtype,
                 out_strides, B, H, T, D, window, static_cast<hipStream_t>(stream), take_timer(), nullptr, nullptr,
                 nullptr, nullptr, lse);
}

extern "C" int flw_fp8_swa_fwd_qx(const void* q, const int64_t* q_strides, const uint8_t* q8_nonfinite,
                                  const float* q_rcp, const uint8_t* k8, const int64_t* k_strides,
                                  const uint8_t* v_tiles, const float* q_scale, const float* k_scale,
                                  const float* v_scale, int granularity, void* out, int dtype,
                                  const int64_t* out_strides, int64_t B, int64_t H, int64_t T, int64_t D,
                                  int64_t window, void* stream) {
  FLW_REQUIRE(q != nullptr, FLW_E_INVALID, "null q");
  int64_t ssb, ssh;
  const int rc = scale_strides(granularity, H, &ssb, &ssh);
  if (rc) return rc;
  const int64_t s8[3] = {H * T * D, T * D, D};
  return swa_fwd(q8_nonfinite, s8, k8, k_strides, v_tiles, q_scale, k_scale, v_scale, ssb, ssh, out, dtype,
                 out_strides, B, H, T, D, window, static_cast<hipStream_t>(stream), take_timer(), q, q_strides,
                 q_rcp);
}

extern "C" size_t flw_fp8_swa_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D) {
  return swa_ws_layout(B, H, T, D).total;
}

static int attention_forward(const void* q, const void* k, const void* v, int dtype, const int64_t* strides,
                             int64_t B, int64_t H, int64_t T, int64_t D, int64_t window, int granularity,
                             void* out, float* scales_out, void* workspace, size_t workspace_bytes,
                             void* stream, const uint32_t* amax) {
  FLW_REQUIRE(strides != nullptr && workspace != nullptr, FLW_E_INVALID, "null strides / workspace");
  FLW_REQUIRE(D == 32 || D == 64 || D == 128, FLW_E_UNSUPPORTED, "head_dim must be 32/64/128, got %lld", (long long)D);
  FLW_REQUIRE(B > 0 && H > 0 && T > 0, FLW_E_INVALID, "empty shape");
  const SwaWorkspace w = swa_ws_layout(B, H, T, D);
  FLW_REQUIRE(workspace_bytes >= w.total, FLW_E_WORKSPACE, "workspace needs %zu bytes", w.total);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const int64_t G = granularity == FLW_SCALE_TENSOR ? 1 : (granularity == FLW_SCALE_HEAD ? H : B * H);
  float* sc = scales_out ? scales_out : reinterpret_cast<float*>(ws + w.scales);
  uint8_t* q8 = ws + w.q8;
  uint8_t* k8 = ws + w.k8;
  uint8_t* vt = ws + w.vt;
  const void* xs[3] = {q, k, v};
  const int layouts[3] = {FLW_LAYOUT_BHTD, FLW_LAYOUT_BHTD, FLW_LAYOUT_VTILE};
  uint8_t* outs[3] = {q8, k8, vt};
  float* scs[3] = {sc, sc + G, sc + 2 * G};
  // An armed timer brackets the whole operator: start with the first quantiser launch, stop with
  // the attention kernel.
  const Timer tm = take_timer();
  // Q is quantised on load by the attention kernel: the quantise pass writes only Q's scale and its
  // reciprocal (and Q's codes for groups whose amax is not finite) and spends its bandwidth on K
  // and V. With a given amax the kernel also checks Q against it (the check the quantise pass
  // makes for K and V), so a stale maximum still gives the reference's clamp-then-cast codes.
  float* qrcp = reinterpret_cast<float*>(ws + w.qrcp);
  int rc = quant_bhtd_n(3, xs, dtype, B, H, T, D, strides, granularity, layouts, outs, scs,
                        ws + w.partials, w.total - w.partials, s, Timer{tm.start, nullptr}, amax, nullptr, qrcp);
  if (rc) return rc;
  const int64_t s8[3] = {H * T * D, T * D, D};
  int64_t ssb, ssh;
  rc = scale_strides(granularity, H, &ssb, &ssh);
  if (rc) return rc;
  return swa_fwd(q8, s8, k8, s8, vt, sc, sc + G, sc + 2 * G, ssb, ssh, out, dtype, strides + 9,
                 B, H, T, D, window, s, Timer{nullptr, tm.stop}, q, strides, qrcp, amax);
}

extern "C" int flw_fp8_swa_attention_forward(const void* q, const void* k, const void* v, int dtype,
                                             const int64_t* strides, int64_t B, int64_t H,
                                             int64_t T, int64_t D, int64_t window,
                                             int granularity, void* out, float* scales_out,
                                             void* workspace, size_t workspace_bytes,
                                             void* stream) {
  return attention_forward(q, k, v, dtype, strides, B, H, T, D, window, granularity, out, scales_out,
                           workspace, workspace_bytes, stream, nullptr);
}

extern "C" int flw_fp8_swa_attention_forward_amax(const void* q, const void* k, const void* v, int dtype,
                                                  const int64_t* strides, int64_t B, int64_t H, int64_t T,
                                                  int64_t D, int64_t window, int granularity,
                                                  const uint32_t* amax, void* out, float* scales_out,
                                                  void* workspace, size_t workspace_bytes, void* stream) {
  FLW_REQUIRE(amax != nullptr, FLW_E_INVALID, "null amax");
  return attention_forward(q, k, v, dtype, strides, B, H, T, D, window, granularity, out, scales_out,
                           workspace, workspace_bytes, stream, amax);
}
