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
//  * larger M: double-buffered LDS-tiled MFMA GEMM (128x128, 128x64 or 64x64 tiles chosen so
//    the grid covers the CUs, split-K when even the smallest tile does not), K step 64, int8
//    tile kept as int8 in LDS and widened on read.
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

// U K steps are loaded before any is multiplied, so each wavefront keeps U x (1 KiB of weights
// + MT x 2 KiB of activations) in flight instead of waiting one round trip per step.
template <int MT, bool WIDE>   // MT 16-row m tiles (M <= 16 MT); WIDE: 16-byte weight loads
__global__ void __launch_bounds__(kSmWaves * 64) w8a16_small_kernel(
    const half_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ wq,
    const void* __restrict__ scale, int scale_is_fp16, const half_t* __restrict__ bias,
    half_t* __restrict__ y, int64_t ldy, int M, int N, int K, int k_per_split,
    float* __restrict__ part) {
  constexpr int U = MT <= 2 ? 4 : 2;
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
  for (int k = kb; k < ke; k += U * kSmKStep) {
    int2_t wa[U], wb[U];
    half8_t xa[U][MT], xb[U][MT];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // lane (c, g): K columns ka .. ka+15 in two 8-element chunks; K % 8 == 0, so a chunk is
      // entirely inside or outside [kb, ke) (WIDE: K % 16 == 0 and the pair goes together).
      const int ka = k + u * kSmKStep + 16 * g, kb2 = ka + 8;
      const bool a_ok = ka < ke, b_ok = kb2 < ke;
      if constexpr (WIDE) {
        const int4_t v = (n_ok && a_ok) ? ld<int4_t>(wrow + ka) : int4_t{0, 0, 0, 0};
        wa[u] = {v[0], v[1]};
        wb[u] = {v[2], v[3]};
      } else {
        wa[u] = (n_ok && a_ok) ? ld<int2_t>(wrow + ka) : int2_t{0, 0};
        wb[u] = (n_ok && b_ok) ? ld<int2_t>(wrow + kb2) : int2_t{0, 0};
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        xa[u][mt] = (m_ok[mt] && a_ok) ? ld<half8_t>(xrow[mt] + ka) : hz;
        xb[u][mt] = (m_ok[mt] && b_ok) ? ld<half8_t>(xrow[mt] + kb2) : hz;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const half8_t fa = i8x8_to_half8(wa[u]), fb = i8x8_to_half8(wb[u]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[mt] = mfma16x16x32(fa, xa[u][mt], acc[mt]);
        acc[mt] = mfma16x16x32(fb, xb[u][mt], acc[mt]);
      }
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
// Larger M: LDS-tiled MFMA GEMM.
// ------------------------------------------------------------------------------------------
// Workgroup = 4 wavefronts (2 x 2) on a BN (output channels) x BM (activation rows) tile, K step
// 64. Each thread stages 8-column chunks of both tiles: weight chunks are widened to fp16 once,
// as they enter LDS (each weight is then read by the two wavefronts that share it without being
// converted twice), and both tiles are stored as rows of eight 16-byte chunks with chunk kc of
// row r at position kc ^ (r & 7), an XOR swizzle under which the MFMA operand reads (16 rows x
// one chunk, eight lanes per LDS cycle) and the staging writes (one row, eight chunks) touch
// eight distinct bank groups. Global loads run RD - 1 K steps ahead through a register ring, the
// LDS tiles are double-buffered, and every load is issued by every lane at an in-range address
// (rows past M or N repeat the last row, whose results are discarded; a K tail past the split
// end is read at column K - 8 and zeroed) so the loads in flight never depend on a branch. The
// per-channel scales and the bias are fetched before the loop. (Streaming the weights straight
// into A-operand registers instead halves the LDS traffic but measured slower: each weight row
// is then loaded and widened by two wavefronts.) With split-K (gridDim.z > 1) each workgroup
// covers k_per_split columns of K and writes fp32 partials for w8a16_reduce_kernel.
constexpr int kTileBK = 64;
constexpr int kTileChunks = kTileBK / 8;          // 16-byte fp16 chunks per tile row

template <int BN, int BM, int RD>
__global__ void __launch_bounds__(256) w8a16_tile_kernel(
    const half_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ wq,
    const void* __restrict__ scale, int scale_is_fp16, const half_t* __restrict__ bias,
    half_t* __restrict__ y, int64_t ldy, int M, int N, int K, int k_per_split,
    float* __restrict__ part) {
  constexpr int BK = kTileBK, CH = kTileChunks;
  constexpr int TN = BN / 32, TM = BM / 32;   // 16 x 16 MFMA tiles per wavefront
  constexpr int WPT = BN * CH / 256, XPT = BM * CH / 256;
  static_assert(WPT * 256 == BN * CH && XPT * 256 == BM * CH, "tile must split over 256 threads");
  static_assert(RD % 2 == 0, "register stages pair with the two LDS buffers");
  __shared__ half8_t s_w[2][BN * CH];
  __shared__ half8_t s_x[2][BM * CH];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int wn = w >> 1, wm = w & 1;
  const int n_base = blockIdx.x * BN, m_base = blockIdx.y * BM;
  const int kb = blockIdx.z * k_per_split;
  const int ke = (kb + k_per_split < K) ? kb + k_per_split : K;
  const int nk = (ke - kb + BK - 1) / BK;
  const bool k_tail = (ke - kb) % BK != 0;          // last step reaches past the split end

  // Chunk u = tid + 256 i of a tile is row u / CH, columns 8 (u % CH) .. + 7 of the K step.
  const int kc = tid % CH;
  const int8_t* wrow[WPT];
  const half_t* xrow[XPT];
  int wpos[WPT], xpos[XPT];
#pragma unroll
  for (int i = 0; i < WPT; ++i) {
    const int r = (tid + 256 * i) / CH, n = n_base + r;
    wrow[i] = wq + (int64_t)(n < N ? n : N - 1) * K;
    wpos[i] = r * CH + (kc ^ (r & 7));
  }
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int r = (tid + 256 * i) / CH, mm = m_base + r;
    xrow[i] = x + (int64_t)(mm < M ? mm : M - 1) * ldx;
    xpos[i] = r * CH + (kc ^ (r & 7));
  }
  // Output-channel scale and bias of this lane's four columns per tile, fetched up front.
  float sc[TN][4], bs[TN][4];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int nn = n_base + wn * (BN / 2) + 16 * i + 4 * g + r;
      const int nc = nn < N ? nn : N - 1;
      sc[i][r] = part ? 0.f : load_scale(scale, scale_is_fp16, nc);
      bs[i][r] = (part || !bias) ? 0.f : (float)bias[nc];
    }

  int2_t wreg[RD][WPT];
  half8_t xreg[RD][XPT];
  // Step kt's loads; steps past the split end repeat the last step (a cache hit that is never
  // used), so every lane issues the same loads in every iteration.
  auto gload = [&](int kt, int2_t (&wr)[WPT], half8_t (&xr)[XPT]) {
    const int k = kb + (kt < nk ? kt : nk - 1) * BK + 8 * kc;
    if (k_tail && kt >= nk - 1) {                   // rare: column K - 8 stands in, then zero
      const bool ok = k < ke;
      const int ka = ok ? k : K - 8;
#pragma unroll
      for (int i = 0; i < WPT; ++i) {
        const int2_t v = ld<int2_t>(wrow[i] + ka);
        wr[i] = ok ? v : int2_t{0, 0};
      }
#pragma unroll
      for (int i = 0; i < XPT; ++i) {
        const half8_t v = ld<half8_t>(xrow[i] + ka);
        xr[i] = ok ? v : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
      }
    } else {
#pragma unroll
      for (int i = 0; i < WPT; ++i) wr[i] = ld<int2_t>(wrow[i] + k);
#pragma unroll
      for (int i = 0; i < XPT; ++i) xr[i] = ld<half8_t>(xrow[i] + k);
    }
  };
  auto lstore = [&](int buf, const int2_t (&wr)[WPT], const half8_t (&xr)[XPT]) {
#pragma unroll
    for (int i = 0; i < WPT; ++i) s_w[buf][wpos[i]] = i8x8_to_half8(wr[i]);
#pragma unroll
    for (int i = 0; i < XPT; ++i) s_x[buf][xpos[i]] = xr[i];
  };

  float4_t acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = {0.f, 0.f, 0.f, 0.f};

  // Operand rows are 16 i + c past a multiple of 16, so their swizzle key is c & 7.
  auto mma_tile = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      const int pc = (4 * ks + g) ^ (c & 7);
      half8_t a[TN], b[TM];
#pragma unroll
      for (int i = 0; i < TN; ++i) a[i] = s_w[buf][(wn * (BN / 2) + 16 * i + c) * CH + pc];
#pragma unroll
      for (int j = 0; j < TM; ++j) b[j] = s_x[buf][(wm * (BM / 2) + 16 * j + c) * CH + pc];
#pragma unroll
      for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = mfma16x16x32(a[i], b[j], acc[i][j]);
    }
  };

  if (nk > 0) {
#pragma unroll
    for (int st_ = 0; st_ < RD - 1; ++st_) gload(st_, wreg[st_], xreg[st_]);
    lstore(0, wreg[0], xreg[0]);
  }
  __syncthreads();
  // Step kt sits in LDS buffer kt % 2 and came through register stage kt % RD (RD is even, so
  // both indices are compile-time constants within the unrolled group).
  for (int kt0 = 0; kt0 < nk; kt0 += RD) {
#pragma unroll
    for (int u = 0; u < RD; ++u) {
      const int kt = kt0 + u;
      gload(kt + RD - 1, wreg[(u + RD - 1) % RD], xreg[(u + RD - 1) % RD]);
      if (kt < nk) mma_tile(u & 1);
      lstore((u + 1) & 1, wreg[(u + 1) % RD], xreg[(u + 1) % RD]);
      __syncthreads();                           // the other buffer was last read before the
    }                                            // previous barrier
  }
  // lane (c, g) of tile (i, j) holds Y[m = .. + 16 j + c][n = .. + 16 i + 4g + r]
#pragma unroll
  for (int i = 0; i < TN; ++i) {
    const int nn = n_base + wn * (BN / 2) + 16 * i + 4 * g;
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      const int mm = m_base + wm * (BM / 2) + 16 * j + c;
      if (mm >= M) continue;
      if (part) {
        float* dst = part + ((int64_t)blockIdx.z * M + mm) * N + nn;
        if (nn + 3 < N) {
          st<float4_t>(dst, acc[i][j]);
        } else {
          for (int r = 0; r < 4; ++r)
            if (nn + r < N) dst[r] = acc[i][j][r];
        }
        continue;
      }
      half_t* yp = y + (int64_t)mm * ldy + nn;
      if (nn + 3 < N) {
        const half4_t v = {(half_t)(acc[i][j][0] * sc[i][0] + bs[i][0]), (half_t)(acc[i][j][1] * sc[i][1] + bs[i][1]),
                           (half_t)(acc[i][j][2] * sc[i][2] + bs[i][2]), (half_t)(acc[i][j][3] * sc[i][3] + bs[i][3])};
        st<half4_t>(yp, v);
      } else {
        for (int r = 0; r < 4; ++r)
          if (nn + r < N) yp[r] = (half_t)(acc[i][j][r] * sc[i][r] + bs[i][r]);
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
  int bn, bm;      // tile shape (tile path)
  int splits;      // K splits
  int k_per_split;
};

static GemmPlan plan_gemm(int M, int N, int K, int cus) {
  GemmPlan p{M <= kSmallMMax, (M + 15) / 16, 0, 0, 1, K};
  if (p.small) {
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
#ifdef TS_W8A16_FORCE_BN                          // tuning override (bn, bm, splits)
  if (!p.small) {
    p.bn = TS_W8A16_FORCE_BN;
    p.bm = TS_W8A16_FORCE_BM;
    const int nk = (K + kTileBK - 1) / kTileBK;
    const int steps = (nk + TS_W8A16_FORCE_SPLITS - 1) / TS_W8A16_FORCE_SPLITS;
    p.k_per_split = steps * kTileBK;
    p.splits = (K + p.k_per_split - 1) / p.k_per_split;
    return p;
  }
#endif
  // Largest tile whose grid covers every CU; the smallest tile otherwise.
  static const int tiles[3][2] = {{128, 128}, {128, 64}, {64, 64}};
  int64_t grid = 0;
  for (int t = 0; t < 3; ++t) {
    p.bn = tiles[t][0];
    p.bm = tiles[t][1];
    grid = (int64_t)((N + p.bn - 1) / p.bn) * ((M + p.bm - 1) / p.bm);
    if (grid >= cus) break;
  }
  // Still short of the CU count: split K, keeping >= 4 K steps per split and the fp32 partial
  // traffic (splits * M * N * 4 bytes) within half the weight bytes.
  if (grid < cus) {
    const int nk = (K + kTileBK - 1) / kTileBK;
    int splits = (int)((cus + grid - 1) / grid);
    const int by_k = nk / 4 > 1 ? nk / 4 : 1;
    const int64_t by_traffic64 = ((int64_t)N * K / 2) / ((int64_t)M * N * 4);
    const int by_traffic = by_traffic64 > 1 ? (int)by_traffic64 : 1;
    if (splits > by_k) splits = by_k;
    if (splits > by_traffic) splits = by_traffic;
    if (splits > 1) {
      const int steps = (nk + splits - 1) / splits;
      p.k_per_split = steps * kTileBK;
      p.splits = (K + p.k_per_split - 1) / p.k_per_split;
    }
  }
  return p;
}

static size_t gemm_workspace(const GemmPlan& p, int M, int N) {
  return p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
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
    const bool wide = K % 16 == 0 && aligned(wq, 16);
#define TS_SM_CASE(MTV)                                                                          \
  case MTV:                                                                                      \
    if (wide)                                                                                    \
      w8a16_small_kernel<MTV, true><<<grid, kSmWaves * 64, 0, s>>>(                             \
          xp, ldx, wq, scale, scale_is_fp16, bp, yp, ldy, M, N, K, p.k_per_split, part);        \
    else                                                                                         \
      w8a16_small_kernel<MTV, false><<<grid, kSmWaves * 64, 0, s>>>(                            \
          xp, ldx, wq, scale, scale_is_fp16, bp, yp, ldy, M, N, K, p.k_per_split, part);        \
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
    float* part = p.splits > 1 ? static_cast<float*>(workspace) : nullptr;
    const dim3 grid((N + p.bn - 1) / p.bn, (M + p.bm - 1) / p.bm, p.splits);
#define TS_TILE_LAUNCH(BNV, BMV)                                                                  \
  w8a16_tile_kernel<BNV, BMV, 4><<<grid, 256, 0, s>>>(xp, ldx, wq, scale, scale_is_fp16, bp, yp,  \
                                                      ldy, M, N, K, p.k_per_split, part)
    if (p.bn == 128 && p.bm == 128)
      TS_TILE_LAUNCH(128, 128);
    else if (p.bn == 128)
      TS_TILE_LAUNCH(128, 64);
    else
      TS_TILE_LAUNCH(64, 64);
#undef TS_TILE_LAUNCH
    if (p.splits > 1) {
      const int64_t total = (int64_t)M * N;
      const int64_t want = (total + 255) / 256;
      w8a16_reduce_kernel<<<(int)(want < 4096 ? want : 4096), 256, 0, s>>>(
          part, p.splits, scale, scale_is_fp16, bp, yp, ldy, M, N);
    }
  }
  return check_launch("w8a16_gemm");
}
