// W8A16 GEMM for gfx950: y = x . (wq * scale)^T (+ bias)   (ops/triton_w8a16.py:11-51).
//
// The int8 weights are widened to fp16 in registers (exact: |w| <= 127), the contraction runs
// on v_mfma_f32_16x16x32_f16 with fp32 accumulation and the per-output-channel scale (and
// the bias) are applied once at the end, as the Triton kernel does.
//
// Everything is computed transposed, Y^T[N][M] = W[N][K] . X^T[K][M], so that both operands
// are row-contiguous loads: lane (c, g) holds W[n + c][k .. k+7] (8 bytes) as the A operand
// and X[m + c][k .. k+7] (16 bytes) as the B operand, and the result lane holds
// Y[m + c][n + 4g .. n + 4g + 3] (see common.h for the operand layouts).
//
//  * small M (<= 64): HBM-bound weight streaming. One wavefront owns 16 output channels and
//    a K range; lane (c, g) reads 16 contiguous weight bytes per 64-wide K step (64 bytes per
//    row and instruction). The K dimension is split over workgroups until the device is full;
//    fp32 partials are merged (and scaled) by a second kernel.
//  * large M: LDS-tiled MFMA GEMM, 128 x 128 output tile per workgroup of four wavefronts
//    (2 x 2, 64 x 64 each), K step 64, int8 tile kept as int8 in LDS and widened on read.
#include "common.h"

namespace ts {

// int8 -> fp16 for four packed bytes: 0x6400 | (b ^ 0x80) is the fp16 number 1024 + (b + 128);
// subtracting 1152 leaves b exactly.
__device__ __forceinline__ half4_t i8x4_to_half4(uint32_t w) {
  const uint32_t x = w ^ 0x80808080u;
  const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, x, 0x05010400u);   // [b0, 64, b1, 64]
  const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, x, 0x05030402u);   // [b2, 64, b3, 64]
  half2_t a = __builtin_bit_cast(half2_t, lo);
  half2_t b = __builtin_bit_cast(half2_t, hi);
  const half2_t off = {(half_t)1152.f, (half_t)1152.f};
  a -= off;
  b -= off;
  return {a[0], a[1], b[0], b[1]};
}

__device__ __forceinline__ half8_t i8x8_to_half8(int2_t w) {
  const half4_t a = i8x4_to_half4((uint32_t)w[0]);
  const half4_t b = i8x4_to_half4((uint32_t)w[1]);
  return {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

__device__ __forceinline__ float load_scale(const void* scale, int scale_is_fp16, int n) {
  return scale_is_fp16 ? (float)static_cast<const half_t*>(scale)[n]
                       : static_cast<const float*>(scale)[n];
}

// ------------------------------------------------------------------------------------------
// Small M: split-K weight streaming.
// ------------------------------------------------------------------------------------------
constexpr int kSmWaves = 4;        // wavefronts per workgroup = 4 x 16 output channels
constexpr int kSmKStep = 64;       // K per step: lane (c, g) covers k + 16g .. k + 16g + 15

template <int MT>   // number of 16-row m tiles (M <= 16 * MT)
__global__ void __launch_bounds__(kSmWaves * 64) w8a16_small_kernel(
    const half_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ wq,
    const void* __restrict__ scale, int scale_is_fp16, const half_t* __restrict__ bias,
    half_t* __restrict__ y, int64_t ldy, int M, int N, int K, int k_per_split,
    float* __restrict__ part) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int c = lane & 15, g = lane >> 4;
  const int n0 = (blockIdx.x * kSmWaves + w) * 16;
  const int ks = blockIdx.y;
  if (n0 >= N) return;
  const int kb = ks * k_per_split;
  const int ke = (kb + k_per_split < K) ? kb + k_per_split : K;
  const int n = n0 + c;
  const bool n_ok = n < N;
  const int8_t* wrow = wq + (int64_t)(n_ok ? n : 0) * K;
  const half_t* xrow[MT];
  bool m_ok[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int mm = mt * 16 + c;
    m_ok[mt] = mm < M;
    xrow[mt] = x + (int64_t)(m_ok[mt] ? mm : 0) * ldx;
  }
  float4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = {0.f, 0.f, 0.f, 0.f};

  const half8_t hz = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int k = kb; k < ke; k += kSmKStep) {
    // Two 8-element chunks per lane; K % 8 == 0, so a chunk is entirely inside or outside.
    const int ka = k + 16 * g, kb2 = ka + 8;
    const bool a_ok = ka < ke, b_ok = kb2 < ke;
    int2_t wa = {0, 0}, wb = {0, 0};
    if (n_ok && a_ok) wa = ld<int2_t>(wrow + ka);
    if (n_ok && b_ok) wb = ld<int2_t>(wrow + kb2);
    const half8_t fa = i8x8_to_half8(wa), fb = i8x8_to_half8(wb);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const half8_t xa = (m_ok[mt] && a_ok) ? ld<half8_t>(xrow[mt] + ka) : hz;
      const half8_t xb = (m_ok[mt] && b_ok) ? ld<half8_t>(xrow[mt] + kb2) : hz;
      acc[mt] = mfma16x16x32(fa, xa, acc[mt]);
      acc[mt] = mfma16x16x32(fb, xb, acc[mt]);
    }
  }
  // lane (c, g) holds Y[m = 16 mt + c][n0 + 4g + r]
  const int nn = n0 + 4 * g;
  if (part == nullptr) {
    float sc[4], bs[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = nn + r < N;
      sc[r] = ok ? load_scale(scale, scale_is_fp16, nn + r) : 0.f;
      bs[r] = (ok && bias) ? (float)bias[nn + r] : 0.f;
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int mm = mt * 16 + c;
      if (mm >= M) continue;
      half_t* yp = y + (int64_t)mm * ldy + nn;
      if (nn + 3 < N) {
        const half4_t v = {(half_t)(acc[mt][0] * sc[0] + bs[0]), (half_t)(acc[mt][1] * sc[1] + bs[1]),
                           (half_t)(acc[mt][2] * sc[2] + bs[2]), (half_t)(acc[mt][3] * sc[3] + bs[3])};
        st<half4_t>(yp, v);
      } else {
        for (int r = 0; r < 4; ++r)
          if (nn + r < N) yp[r] = (half_t)(acc[mt][r] * sc[r] + bs[r]);
      }
    }
  } else {
    float* pp = part + (int64_t)ks * M * N;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int mm = mt * 16 + c;
      if (mm >= M) continue;
      float* dst = pp + (int64_t)mm * N + nn;
      if (nn + 3 < N) {
        st<float4_t>(dst, acc[mt]);
      } else {
        for (int r = 0; r < 4; ++r)
          if (nn + r < N) dst[r] = acc[mt][r];
      }
    }
  }
}

// Sum of the split-K partials, then scale, bias and fp16 conversion.
__global__ void __launch_bounds__(256) w8a16_reduce_kernel(
    const float* __restrict__ part, int splits, const void* __restrict__ scale, int scale_is_fp16,
    const half_t* __restrict__ bias, half_t* __restrict__ y, int64_t ldy, int M, int N) {
  const int64_t total = (int64_t)M * N;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int mm = (int)(i / N), nn = (int)(i % N);
    float s = 0.f;
    for (int k = 0; k < splits; ++k) s += part[(int64_t)k * total + i];
    float v = s * load_scale(scale, scale_is_fp16, nn);
    if (bias) v += (float)bias[nn];
    y[(int64_t)mm * ldy + nn] = (half_t)v;
  }
}

// ------------------------------------------------------------------------------------------
// Large M: LDS-tiled MFMA GEMM.
// ------------------------------------------------------------------------------------------
constexpr int kLgBN = 128;     // output channels per workgroup
constexpr int kLgBM = 128;     // activation rows per workgroup
constexpr int kLgBK = 64;
constexpr int kLgWP = kLgBK + 16;   // padded int8 row (bytes)
constexpr int kLgXP = kLgBK + 8;    // padded fp16 row (halfs)

__global__ void __launch_bounds__(256) w8a16_large_kernel(
    const half_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ wq,
    const void* __restrict__ scale, int scale_is_fp16, const half_t* __restrict__ bias,
    half_t* __restrict__ y, int64_t ldy, int M, int N, int K) {
  __shared__ int8_t s_w[kLgBN][kLgWP];
  __shared__ half_t s_x[kLgBM][kLgXP];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int c = lane & 15, g = lane >> 4;
  const int wn = w >> 1, wm = w & 1;                 // 2 x 2 wavefronts, 64 x 64 each
  const int n_base = blockIdx.x * kLgBN, m_base = blockIdx.y * kLgBM;

  float4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = {0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < K; k0 += kLgBK) {
    // W tile: 128 rows x 64 bytes = 512 chunks of 16 bytes (K % 8 == 0: 8-byte granules).
    for (int u = tid; u < kLgBN * (kLgBK / 8); u += 256) {
      const int r = u / (kLgBK / 8), cc = u % (kLgBK / 8);
      const int n = n_base + r, k = k0 + 8 * cc;
      int2_t v = {0, 0};
      if (n < N && k < K) v = ld<int2_t>(wq + (int64_t)n * K + k);
      st<int2_t>(&s_w[r][8 * cc], v);
    }
    // X tile: 128 rows x 64 halfs = 1024 chunks of 16 bytes.
    for (int u = tid; u < kLgBM * (kLgBK / 8); u += 256) {
      const int r = u / (kLgBK / 8), cc = u % (kLgBK / 8);
      const int mm = m_base + r, k = k0 + 8 * cc;
      half8_t v = {0, 0, 0, 0, 0, 0, 0, 0};
      if (mm < M && k < K) v = ld<half8_t>(x + (int64_t)mm * ldx + k);
      st<half8_t>(&s_x[r][8 * cc], v);
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < kLgBK / 32; ++ks) {
      half8_t a[4], bq[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[i] = i8x8_to_half8(ld<int2_t>(&s_w[wn * 64 + 16 * i + c][32 * ks + 8 * g]));
#pragma unroll
      for (int j = 0; j < 4; ++j) bq[j] = ld<half8_t>(&s_x[wm * 64 + 16 * j + c][32 * ks + 8 * g]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x32(a[i], bq[j], acc[i][j]);
    }
    __syncthreads();
  }
  // lane (c, g) of tile (i, j) holds Y[m = .. + 16 j + c][n = .. + 16 i + 4g + r]
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int nn = n_base + wn * 64 + 16 * i + 4 * g;
    float sc[4], bs[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = nn + r < N;
      sc[r] = ok ? load_scale(scale, scale_is_fp16, nn + r) : 0.f;
      bs[r] = (ok && bias) ? (float)bias[nn + r] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int mm = m_base + wm * 64 + 16 * j + c;
      if (mm >= M) continue;
      half_t* yp = y + (int64_t)mm * ldy + nn;
      if (nn + 3 < N) {
        const half4_t v = {(half_t)(acc[i][j][0] * sc[0] + bs[0]), (half_t)(acc[i][j][1] * sc[1] + bs[1]),
                           (half_t)(acc[i][j][2] * sc[2] + bs[2]), (half_t)(acc[i][j][3] * sc[3] + bs[3])};
        st<half4_t>(yp, v);
      } else {
        for (int r = 0; r < 4; ++r)
          if (nn + r < N) yp[r] = (half_t)(acc[i][j][r] * sc[r] + bs[r]);
      }
    }
  }
}

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------
constexpr int kSmallMMax = 64;

struct GemmPlan {
  bool small;
  int mt;          // m tiles (small path)
  int splits;      // K splits (small path)
  int k_per_split;
};

static GemmPlan plan_gemm(int M, int N, int K, int cus) {
  GemmPlan p{M <= kSmallMMax, (M + 15) / 16, 1, K};
  if (!p.small) return p;
  // Fill the device with wavefronts (about eight per CU) by splitting K, keeping at least
  // 256 K per split and the partial traffic (splits * M * N * 4 bytes) below 1/8 of the
  // weight bytes.
  const int64_t wgs = (N + 16 * kSmWaves - 1) / (16 * kSmWaves);
  const int64_t target_wgs = 2LL * cus;
  int splits = (int)((target_wgs + wgs - 1) / wgs);
  const int max_by_k = K / 256 > 1 ? K / 256 : 1;
  const int max_by_traffic = (int)((int64_t)K / (32LL * M) > 1 ? (int64_t)K / (32LL * M) : 1);
  if (splits > max_by_k) splits = max_by_k;
  if (splits > max_by_traffic) splits = max_by_traffic;
  if (splits < 1) splits = 1;
  int kps = (K + splits - 1) / splits;
  kps = (kps + kSmKStep - 1) / kSmKStep * kSmKStep;
  p.splits = (K + kps - 1) / kps;
  p.k_per_split = kps;
  return p;
}

static size_t gemm_workspace(const GemmPlan& p, int M, int N) {
  return (p.small && p.splits > 1) ? (size_t)p.splits * M * N * sizeof(float) : 0;
}

}  // namespace ts

using namespace ts;

extern "C" size_t ts_w8a16_workspace_bytes(int32_t M, int32_t N, int32_t K, int32_t cu_count) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return gemm_workspace(plan_gemm(M, N, K, cu_count > 0 ? cu_count : 256), M, N);
}

extern "C" int ts_w8a16_gemm(const void* x, int64_t ldx, const int8_t* wq, const void* scale,
                             int32_t scale_is_fp16, const void* bias, void* y, int64_t ldy,
                             int32_t M, int32_t N, int32_t K, void* workspace,
                             size_t workspace_bytes, void* stream) {
  TS_REQUIRE(M >= 0 && N > 0 && K > 0, TS_ERR_INVALID_ARG, "w8a16: bad shape M=%d N=%d K=%d", M,
             N, K);
  if (M == 0) return TS_OK;
  TS_REQUIRE(x && wq && scale && y, TS_ERR_INVALID_ARG, "w8a16: null pointer argument");
  TS_REQUIRE(K % 8 == 0, TS_ERR_UNSUPPORTED, "w8a16: K=%d is not a multiple of 8", K);
  TS_REQUIRE(ldx >= K && ldx % 8 == 0 && ldy >= N && aligned(x, 16) && aligned(wq, 8) &&
                 aligned(y, 2),
             TS_ERR_INVALID_ARG, "w8a16: x must be 16-byte aligned rows (ldx %% 8 == 0), wq 8-byte aligned");
  TS_REQUIRE(!(ldy % 4) && aligned(y, 8), TS_ERR_INVALID_ARG,
             "w8a16: y rows must be 8-byte aligned (ldy %% 4 == 0)");
  int cus = 0;
  int st = device_cu_count(&cus);
  if (st != TS_OK) return st;
  const GemmPlan p = plan_gemm(M, N, K, cus);
  const size_t need = gemm_workspace(p, M, N);
  TS_REQUIRE(need == 0 || (workspace && workspace_bytes >= need && aligned(workspace, 16)),
             TS_ERR_WORKSPACE, "w8a16: workspace of %zu bytes needed, got %zu", need,
             workspace_bytes);
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const half_t* xp = static_cast<const half_t*>(x);
  const half_t* bp = static_cast<const half_t*>(bias);
  half_t* yp = static_cast<half_t*>(y);
  if (p.small) {
    float* part = p.splits > 1 ? static_cast<float*>(workspace) : nullptr;
    const dim3 grid((N + 16 * kSmWaves - 1) / (16 * kSmWaves), p.splits);
#define TS_SM_CASE(MTV)                                                                          \
  case MTV:                                                                                      \
    w8a16_small_kernel<MTV><<<grid, kSmWaves * 64, 0, s>>>(xp, ldx, wq, scale, scale_is_fp16,   \
                                                           bp, yp, ldy, M, N, K, p.k_per_split, \
                                                           part);                               \
    break;
    switch (p.mt) {
      TS_SM_CASE(1)
      TS_SM_CASE(2)
      TS_SM_CASE(3)
      TS_SM_CASE(4)
    }
#undef TS_SM_CASE
    if (p.splits > 1) {
      const int64_t total = (int64_t)M * N;
      const int64_t want = (total + 255) / 256;
      w8a16_reduce_kernel<<<(int)(want < 4096 ? want : 4096), 256, 0, s>>>(
          part, p.splits, scale, scale_is_fp16, bp, yp, ldy, M, N);
    }
  } else {
    const dim3 grid((N + kLgBN - 1) / kLgBN, (M + kLgBM - 1) / kLgBM);
    w8a16_large_kernel<<<grid, 256, 0, s>>>(xp, ldx, wq, scale, scale_is_fp16, bp, yp, ldy, M, N,
                                            K);
  }
  return check_launch("w8a16_gemm");
}
