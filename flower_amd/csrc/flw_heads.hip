// CausalSelfAttention.qkv_heads (flower/models/base.py:618-639) for training, forward and backward:
// the qkv projection's output [M = B T, 3 H D] split into per-head q, k, v, HeadRMSNorm of q and k
// over each head row (base.py:341-357, when qk_norm) and RoPE of q and k (base.py:436-483), with
// the reference's torch roundings, as two memory-bound passes in place of the ~20 torch kernels
// (forward and autograd backward) that the expressions take in eager torch.
//
// Work item: one 16-byte chunk (8 bf16 values) of a qkv row; the D / 8 lanes holding one head row
// are consecutive lanes of a wave (a token row holds 3 H D / 8 chunks, a multiple of D / 8), so the
// head row's sums are DPP reductions over an aligned lane group (group_sum).
//
// Forward: q, k = rope(norm(x)) through head_norm_rope (the same transform the FP8 quantisers and
// the QKV GEMM's epilogue apply), v copied; outputs contiguous (B, H, T, D).
// Backward, given dq', dk', dv (B, H, T, D) and the forward's input x:
//   RoPE (y = x cos + rot(x) sin, rot(x)[2i] = -x[2i+1], rot(x)[2i+1] = x[2i], each op rounded
//   to bf16 as torch's bf16 autograd rounds it): t1 = bf16(g cos), t2 = bf16(g sin),
//   dn[2i] = bf16(t1[2i] + t2[2i+1]), dn[2i+1] = bf16(t1[2i+1] - t2[2i]);
//   HeadRMSNorm (fp32 maths as torch's autograd of x.float() * rsqrt(mean(x.float()^2) + eps); the
//   two x.float() casts each hand back a bf16 gradient, summed in bf16): r = rsqrt(mean(x^2) + eps),
//   dx = bf16(bf16(dn r) - bf16(x r^3 sum(dn x) / D));
//   dv copied back into the qkv gradient's v columns.

#include "flw_common.h"

namespace flw {

struct HeadsParams {
  const uint16_t* qkv;          // [M, qs] bf16: q | k | v column blocks of H D
  int64_t qs;
  const uint16_t* cos;          // [T, D] bf16 RoPE tables
  const uint16_t* sin;
  uint16_t* out[3];             // forward: q', k', v as contiguous (B, H, T, D)
  const uint16_t* grad[3];      // backward: dq', dk', dv as contiguous (B, H, T, D)
  uint16_t* dqkv;               // backward: [M, ds]
  int64_t ds;
  uint32_t* part;               // backward with AMAX: per-workgroup |dqkv| maxima
  int64_t M;
  int T, H, norm;
  float eps;
};

// This lane's chunk: token row m, part (0 q, 1 k, 2 v), head h, chunk l of the head row; the
// element offset of the chunk in the (B, H, T, D) tensors.
template <int D>
struct HeadsChunk {
  int64_t m, bhtd;
  int part, h, l, t;
  // 32-bit index arithmetic (the host keeps the chunk count below 2^31): the divisions by the
  // run-time cpr, H and T are the kernel's largest instruction cost otherwise.
  __device__ __forceinline__ bool init(const HeadsParams& p) {
    constexpr uint32_t LPR = D / 8;
    const uint32_t cpr = 3u * (uint32_t)p.H * LPR;
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    const uint32_t mm = i / cpr;
    if ((int64_t)mm >= p.M) return false;       // a whole head row at a time (cpr % LPR == 0)
    m = mm;
    const uint32_t c = i - mm * cpr;
    const uint32_t hl = c / LPR;                 // part * H + h
    part = (int)(hl / (uint32_t)p.H);
    h = (int)(hl - (uint32_t)part * (uint32_t)p.H);
    l = (int)(c % LPR);
    const uint32_t b = mm / (uint32_t)p.T;
    t = (int)(mm - b * (uint32_t)p.T);
    bhtd = (((int64_t)b * p.H + h) * p.T + t) * D + 8 * l;
    return true;
  }
};

template <int D>
__global__ __launch_bounds__(256) void qkv_heads_fwd_kernel(HeadsParams p) {
  HeadsChunk<D> ch;
  if (!ch.init(p)) return;
  const int64_t src = ch.m * p.qs + ((int64_t)ch.part * p.H + ch.h) * D + 8 * ch.l;
  const uint4 raw = *reinterpret_cast<const uint4*>(p.qkv + src);
  if (ch.part == 2) {
    *reinterpret_cast<uint4*>(p.out[2] + ch.bhtd) = raw;
    return;
  }
  float f[8], c[8], sn[8];
  Vec16<uint16_t>::unpack(raw, f);
  Vec16<uint16_t>::load(p.cos + (int64_t)ch.t * D + 8 * ch.l, c);
  Vec16<uint16_t>::load(p.sin + (int64_t)ch.t * D + 8 * ch.l, sn);
  head_norm_rope<uint16_t>(f, p.norm != 0, p.eps, D, D / 8, true, true, c, sn);
  *reinterpret_cast<uint4*>(p.out[ch.part] + ch.bhtd) =
      make_uint4(bf16x2_rne_raw(f[0], f[1]), bf16x2_rne_raw(f[2], f[3]), bf16x2_rne_raw(f[4], f[5]),
                 bf16x2_rne_raw(f[6], f[7]));
}

template <int D, bool AMAX>
__global__ __launch_bounds__(256) void qkv_heads_bwd_kernel(HeadsParams p) {
  __shared__ uint32_t red[4];
  HeadsChunk<D> ch;
  const bool valid = ch.init(p);
  flw_u16x2 mx = {0, 0};
  if (valid) {
    const int64_t dst = ch.m * p.ds + ((int64_t)ch.part * p.H + ch.h) * D + 8 * ch.l;
    const uint4 graw = *reinterpret_cast<const uint4*>(p.grad[ch.part] + ch.bhtd);
    uint4 w = graw;
    if (ch.part != 2) {
      float g[8], x[8], c[8], sn[8], dn[8];
      Vec16<uint16_t>::unpack(graw, g);
      Vec16<uint16_t>::load(p.qkv + ch.m * p.qs + ((int64_t)ch.part * p.H + ch.h) * D + 8 * ch.l, x);
      Vec16<uint16_t>::load(p.cos + (int64_t)ch.t * D + 8 * ch.l, c);
      Vec16<uint16_t>::load(p.sin + (int64_t)ch.t * D + 8 * ch.l, sn);
      {
#pragma clang fp contract(off)
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          const float a0 = round_bf16(g[i] * c[i]), a1 = round_bf16(g[i + 1] * c[i + 1]);
          const float b0 = round_bf16(g[i] * sn[i]), b1 = round_bf16(g[i + 1] * sn[i + 1]);
          dn[i] = round_bf16(a0 + b1);
          dn[i + 1] = round_bf16(a1 - b0);
        }
      }
      float o[8];
      if (p.norm) {                                 // uniform over a head row's lanes
        float ss = 0.0f, sd = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          ss = fmaf(x[i], x[i], ss);
          sd = fmaf(dn[i], x[i], sd);
        }
        ss = group_sum(ss, D / 8);
        sd = group_sum(sd, D / 8);
        const float r = __builtin_amdgcn_rsqf(__builtin_ldexpf(ss, -__builtin_ctz((unsigned)D)) + p.eps);
        const float k = __builtin_ldexpf(sd * (r * r * r), -__builtin_ctz((unsigned)D));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
#pragma clang fp contract(off)
          o[i] = round_bf16(dn[i] * r) - round_bf16(x[i] * k);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = dn[i];
      }
      w = make_uint4(bf16x2_canon_nan(bf16x2_rne_raw(o[0], o[1])), bf16x2_canon_nan(bf16x2_rne_raw(o[2], o[3])),
                     bf16x2_canon_nan(bf16x2_rne_raw(o[4], o[5])), bf16x2_canon_nan(bf16x2_rne_raw(o[6], o[7])));
    }
    *reinterpret_cast<uint4*>(p.dqkv + dst) = w;
    if (AMAX) {
      mx = abs_max_bf16x2(mx, w.x);
      mx = abs_max_bf16x2(mx, w.y);
      mx = abs_max_bf16x2(mx, w.z);
      mx = abs_max_bf16x2(mx, w.w);
    }
  }
  if (AMAX) {                                       // this workgroup's |dqkv| maximum (fp32 bits)
    uint32_t m = (uint32_t)(mx[0] > mx[1] ? mx[0] : mx[1]) << 16;
    m = wave_max_u32(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t r = red[0];
#pragma unroll
      for (int i = 1; i < 4; ++i) r = r > red[i] ? r : red[i];
      p.part[blockIdx.x] = r;
    }
  }
}

// One workgroup of 1024 folds the n per-workgroup maxima into out[0].
__global__ __launch_bounds__(1024) void heads_fold_kernel(const uint32_t* __restrict__ part, int n,
                                                          uint32_t* __restrict__ out) {
  __shared__ uint32_t red[16];
  uint32_t m = 0;
  for (int i = threadIdx.x; i < n; i += 1024) m = m > part[i] ? m : part[i];
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

static int heads_check(const void* qkv, int64_t B, int64_t T, int64_t H, int64_t D, int64_t qs,
                       const void* rcos, const void* rsin, float eps, int qk_norm) {
  FLW_REQUIRE(qkv != nullptr && rcos != nullptr && rsin != nullptr, FLW_E_INVALID, "null pointer");
  FLW_REQUIRE(B > 0 && T > 0 && H > 0, FLW_E_INVALID, "empty shape");
  FLW_REQUIRE(D == 32 || D == 64 || D == 128, FLW_E_UNSUPPORTED, "head_dim must be 32/64/128, got %lld", (long long)D);
  FLW_REQUIRE(qs >= 3 * H * D && qs % 8 == 0 && ((uintptr_t)qkv & 15) == 0, FLW_E_INVALID,
              "qkv rows must hold 3 H D values, 16-byte aligned");
  FLW_REQUIRE(((uintptr_t)rcos & 15) == 0 && ((uintptr_t)rsin & 15) == 0, FLW_E_INVALID,
              "RoPE tables must be 16-byte aligned");
  FLW_REQUIRE(qk_norm == 0 || eps >= 0.0f, FLW_E_INVALID, "eps must be non-negative");
  FLW_REQUIRE(B * T * 3 * H * (D / 8) <= 0x7FFFFFFFll - 255 && H <= 65535, FLW_E_UNSUPPORTED,
              "shape too large (3 B T H D / 8 chunks must stay below 2^31)");
  return FLW_OK;
}

static void heads_launch(const void* fwd32, const void* fwd64, const void* fwd128, int64_t D, const HeadsParams& p,
                         hipStream_t s) {
  const int64_t chunks = p.M * 3 * p.H * (D / 8);
  const void* k = D == 32 ? fwd32 : D == 64 ? fwd64 : fwd128;
  (void)launch_timed(k, dim3((unsigned)((chunks + 255) / 256)), dim3(256), s, p);
}

}  // namespace flw

using namespace flw;

extern "C" int flw_qkv_heads_fwd(const void* qkv, int64_t B, int64_t T, int64_t H, int64_t D, int64_t qkv_row_stride,
                                 int qk_norm, float eps, const void* rope_cos, const void* rope_sin, void* q,
                                 void* k, void* v, void* stream) {
  int rc = heads_check(qkv, B, T, H, D, qkv_row_stride, rope_cos, rope_sin, eps, qk_norm);
  if (rc) return rc;
  FLW_REQUIRE(q && k && v && ((uintptr_t)q & 15) == 0 && ((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 15) == 0,
              FLW_E_INVALID, "q, k, v must be non-null and 16-byte aligned");
  HeadsParams p{};
  p.qkv = static_cast<const uint16_t*>(qkv); p.qs = qkv_row_stride;
  p.cos = static_cast<const uint16_t*>(rope_cos); p.sin = static_cast<const uint16_t*>(rope_sin);
  p.out[0] = static_cast<uint16_t*>(q); p.out[1] = static_cast<uint16_t*>(k); p.out[2] = static_cast<uint16_t*>(v);
  p.M = B * T; p.T = (int)T; p.H = (int)H; p.norm = qk_norm; p.eps = eps;
  heads_launch(reinterpret_cast<const void*>(&qkv_heads_fwd_kernel<32>),
               reinterpret_cast<const void*>(&qkv_heads_fwd_kernel<64>),
               reinterpret_cast<const void*>(&qkv_heads_fwd_kernel<128>), D, p, static_cast<hipStream_t>(stream));
  return check_launch("flw_qkv_heads_fwd");
}

extern "C" size_t flw_qkv_heads_amax_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D) {
  if (B <= 0 || T <= 0 || H <= 0 || D <= 0) return 0;
  return (size_t)((B * T * 3 * H * (D / 8) + 255) / 256) * 4;
}

extern "C" int flw_qkv_heads_bwd(const void* qkv, int64_t B, int64_t T, int64_t H, int64_t D, int64_t qkv_row_stride,
                                 int qk_norm, float eps, const void* rope_cos, const void* rope_sin, const void* dq,
                                 const void* dk, const void* dv, void* dqkv, int64_t dqkv_row_stride,
                                 uint32_t* dqkv_amax, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = heads_check(qkv, B, T, H, D, qkv_row_stride, rope_cos, rope_sin, eps, qk_norm);
  if (rc) return rc;
  FLW_REQUIRE(dq && dk && dv && dqkv && ((uintptr_t)dq & 15) == 0 && ((uintptr_t)dk & 15) == 0 &&
              ((uintptr_t)dv & 15) == 0 && ((uintptr_t)dqkv & 15) == 0, FLW_E_INVALID,
              "gradients must be non-null and 16-byte aligned");
  FLW_REQUIRE(dqkv_row_stride >= 3 * H * D && dqkv_row_stride % 8 == 0, FLW_E_INVALID,
              "dqkv rows must hold 3 H D values, 16-byte aligned");
  HeadsParams p{};
  p.qkv = static_cast<const uint16_t*>(qkv); p.qs = qkv_row_stride;
  p.cos = static_cast<const uint16_t*>(rope_cos); p.sin = static_cast<const uint16_t*>(rope_sin);
  p.grad[0] = static_cast<const uint16_t*>(dq); p.grad[1] = static_cast<const uint16_t*>(dk);
  p.grad[2] = static_cast<const uint16_t*>(dv);
  p.dqkv = static_cast<uint16_t*>(dqkv); p.ds = dqkv_row_stride;
  p.M = B * T; p.T = (int)T; p.H = (int)H; p.norm = qk_norm; p.eps = eps;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dqkv_amax == nullptr) {
    heads_launch(reinterpret_cast<const void*>(&qkv_heads_bwd_kernel<32, false>),
                 reinterpret_cast<const void*>(&qkv_heads_bwd_kernel<64, false>),
                 reinterpret_cast<const void*>(&qkv_heads_bwd_kernel<128, false>), D, p, s);
    return check_launch("flw_qkv_heads_bwd");
  }
  const size_t need = flw_qkv_heads_amax_workspace_bytes(B, T, H, D);
  FLW_REQUIRE(workspace != nullptr && ((uintptr_t)workspace & 15) == 0 && workspace_bytes >= need, FLW_E_WORKSPACE,
              "workspace needs %zu bytes (16-byte aligned)", need);
  p.part = static_cast<uint32_t*>(workspace);
  const int64_t chunks = p.M * 3 * p.H * (D / 8);
  const int nblk = (int)((chunks + 255) / 256);
  const void* k = D == 32 ? reinterpret_cast<const void*>(&qkv_heads_bwd_kernel<32, true>)
                : D == 64 ? reinterpret_cast<const void*>(&qkv_heads_bwd_kernel<64, true>)
                          : reinterpret_cast<const void*>(&qkv_heads_bwd_kernel<128, true>);
  const Timer tm = take_timer();
  (void)launch_ext(k, dim3((unsigned)nblk), dim3(256), 0, s, p, tm.start, nullptr);
  (void)launch_args(reinterpret_cast<const void*>(&heads_fold_kernel), dim3(1u), dim3(1024), 0, s, nullptr, tm.stop,
                    static_cast<const uint32_t*>(p.part), nblk, dqkv_amax);
  return check_launch("flw_qkv_heads_bwd");
}
