// Scaled FP8 GEMM for gfx950: y[M, N] (bf16) = (x8[M, K] . w8[N, K]^T) * sx[m] * sw[n].
//
// Both operands are K-contiguous e4m3 ("TN"), which is exactly what the MFMA operand registers
// want: every lane holds 32 consecutive K bytes of one row. The kernel computes the transposed
// tile C^T = W X^T so that a lane of the 32x32 accumulator owns one output row m and 16 output
// columns n in runs of 4 (8-byte bf16 stores). Workgroup tile 128 (n) x 128 (m), 4 waves in a
// 2 x 2 grid of 64 x 64 wave tiles (2 x 2 v_mfma_f32_32x32x64_f8f6f4 per 64-deep K step);
// K advances 128 per stage through double-buffered LDS in fragment order (conflict-free
// ds_read_b128), the next stage's global loads overlapping the current stage's MFMAs.
#include "flw_common.h"

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
  int tiles_n;         // ceil(N / 128)
};

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
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * g + e] * sxm * p.sw[(int64_t)(n + e) * p.sw_step];
        uint2 w;
        w.x = f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16);
        w.y = f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16);
        *reinterpret_cast<uint2*>(yrow + n) = w;
      }
    }
  }
}

static int scaled_mm(const uint8_t* x8, int64_t M, int64_t K, const uint8_t* w8, int64_t N,
                     const float* sx, int64_t sx_count, const float* sw, int64_t sw_count,
                     void* y, int64_t ys, hipStream_t s) {
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
  p.tiles_n = (int)((N + kGBN - 1) / kGBN);
  const int64_t tiles = (int64_t)p.tiles_n * ((M + kGBM - 1) / kGBM);
  FLW_REQUIRE(tiles <= 0x7FFFFFFF, FLW_E_UNSUPPORTED, "grid too large");
  hipLaunchKernelGGL(fp8_gemm_kernel, dim3((unsigned)tiles), dim3(256), 0, s, p);
  return check_launch("flw_fp8_scaled_mm");
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

extern "C" size_t flw_fp8_linear_workspace_bytes(int64_t M, int64_t K, int mode) {
  if (mode != FLW_GEMM_A8W8) return 0;
  return galign((size_t)(M * K)) + galign(sizeof(float) * (size_t)M);
}

extern "C" int flw_fp8_linear(const void* x, int64_t M, int64_t K, int64_t x_row_stride,
                              const uint8_t* w8, int64_t N, const float* w_scale,
                              int64_t w_scale_count, int mode, void* y, int64_t y_row_stride,
                              void* workspace, size_t workspace_bytes, void* stream) {
  FLW_REQUIRE(mode == FLW_GEMM_A8W8, FLW_E_UNSUPPORTED, "GEMM mode %d is not implemented in this build", mode);
  const size_t need = flw_fp8_linear_workspace_bytes(M, K, mode);
  FLW_REQUIRE(workspace != nullptr && workspace_bytes >= need, FLW_E_WORKSPACE, "workspace needs %zu bytes", need);
  uint8_t* x8 = static_cast<uint8_t*>(workspace);
  float* sx = reinterpret_cast<float*>(x8 + galign((size_t)(M * K)));
  int rc = flw_quant_rows_e4m3(x, FLW_BF16, M, K, x_row_stride, x8, sx, stream);
  if (rc) return rc;
  return scaled_mm(x8, M, K, w8, N, sx, M, w_scale, w_scale_count, y, y_row_stride,
                   static_cast<hipStream_t>(stream));
}
