// W8A16 GEMM for gfx950: y = x . (wq * scale)^T (+ bias)   (ops/triton_w8a16.py:11-51).
//
// The int8 weights are widened to fp16 in registers (exact: |w| <= 127), the contraction runs
// on MFMAs with fp32 accumulation and the per-output-channel scale (and the bias) are applied
// once at the end, as the Triton kernel does.
//
// Everything is computed transposed, Y^T[N][M] = W[N][K] . X^T[K][M], so that both operands
// are row-contiguous loads (weights as the A operand, activations as the B operand).
//
//  * small M (<= 32, see use_small_path): HBM-bound weight streaming on v_mfma_f32_16x16x32_f16. One wavefront
//    owns 16 output channels and a K range; lane (c, g) reads 16 contiguous weight bytes per
//    64-wide K step (64 bytes per row and instruction). The K dimension is split over
//    workgroups until the device is full; fp32 partials are merged (and scaled) by a second
//    kernel.
//  * larger M: the wide-tile kernel on v_mfma_f32_32x32x16_f16 (128 x 128, 128 x 64 or 128 x 32 tiles of
//    Y^T, split-K when the grid is short of two workgroups per CU): weights stream straight
//    into the A operands of the wavefront that owns them, activations are DMA'd into a ring of
//    LDS stages that all four wavefronts read.
#include "common.h"
#include "rmsnorm.h"
#include "rope.h"

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

// Optional extras of the logits entry point: activation row r of the product is
// x[rows[r]] (clamped to [0, x_rows)) instead of x[r], and the result goes to the fp32 matrix yf
// as the fp16-rounded value widened (what the reference's fp16 product followed by .float()
// holds) instead of to the fp16 matrix y. glu = I > 0 selects the gated-MLP output of the
// fused gate_up entry point: the weights are [gate; up] (N = 2I rows) and y[m][i] =
// silu(Y[m][i]) * Y[m][I + i], an [M, I] matrix.
struct GemmIo {
  const int64_t* rows;
  int64_t x_rows;
  float* yf;
  int64_t ldyf;
  int glu;
  // The qkv product with RoPE and the K/V cache write in its epilogue (rope_cos set): each
  // 128-column tile is one head of 128 dims (q heads [0, rope_heads), then rope_kv_heads k and
  // rope_kv_heads v heads); rows at positions[m], K / V rows to slots[m] (as rope_kv_write).
  const int64_t* positions;
  const float* rope_cos;
  const float* rope_sin;
  int64_t rope_max_pos;
  int rope_heads;
  int rope_kv_heads;
  half_t* kc;
  half_t* vc;
  const int64_t* slots;
  int64_t num_slots;
};

// silu(gate) * up from the fp16 GEMM outputs, with the rounding points of the unfused pair
// (the silu_mul kernel, ops/reference.py:40-42): SiLU in fp32 rounded to fp16, then the product
// rounded to fp16.
__device__ __forceinline__ half_t silu_mul_h(half_t g, half_t u) {
  const float gf = (float)g;
  const half_t sl = (half_t)(gf / (1.f + expf(-gf)));
  return (half_t)((float)sl * (float)u);
}

__device__ __forceinline__ int64_t x_row(const GemmIo& io, int r) {
  if (!io.rows) return r;
  const int64_t v = io.rows[r];
  return v < 0 ? 0 : (v >= io.x_rows ? io.x_rows - 1 : v);
}

// Output columns nn .. nn + 3 of row mm (those below N) from their fp32 values.
__device__ __forceinline__ void store_out4(const GemmIo& io, half_t* y, int64_t ldy, int mm, int nn,
                                           int N, const float (&v)[4]) {
  const half4_t hv = {(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
  if (io.yf) {
    float* dst = io.yf + (int64_t)mm * io.ldyf + nn;
    if (nn + 3 < N) {
      st<float4_t>(dst, float4_t{(float)hv[0], (float)hv[1], (float)hv[2], (float)hv[3]});
    } else {
      for (int r = 0; r < 4; ++r)
        if (nn + r < N) dst[r] = (float)hv[r];
    }
  } else {
    half_t* dst = y + (int64_t)mm * ldy + nn;
    if (nn + 3 < N) {
      st<half4_t>(dst, hv);
    } else {
      for (int r = 0; r < 4; ++r)
        if (nn + r < N) dst[r] = hv[r];
    }
  }
}

// ------------------------------------------------------------------------------------------
// Small M: split-K weight streaming.
// ------------------------------------------------------------------------------------------
constexpr int kSmWaves = 4;        // wavefronts per workgroup = 4 x 16 output channels
constexpr int kSmKStep = 64;       // K per step: lane (c, g) covers k + 16g .. k + 16g + 15

// Two register stages of U K steps each: the loads of the next stage (if it starts inside the
// split) are issued before the current one is multiplied, so each wavefront keeps up to
// 2U x (1 KiB of weights + MT x 2 KiB of activations) in flight. Every load is at an in-range address (rows past M or N repeat the
// last row, whose results are not stored; columns past the split end repeat column K - 16 or
// K - 8) and columns past the split end are zeroed in the widened weights, where they are used:
// a select on a register whose load is in flight would wait for it.
template <int MT, bool WIDE>   // MT 16-row m tiles (M <= 16 MT); WIDE: 16-byte weight loads
__global__ void __launch_bounds__(kSmWaves * 64) w8a16_small_kernel(
    const half_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ wq,
    const void* __restrict__ scale, int scale_is_fp16, const half_t* __restrict__ bias,
    half_t* __restrict__ y, int64_t ldy, int M, int N, int K, int k_per_split,
    float* __restrict__ part, GemmIo io) {
  constexpr int U = 4;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int c = lane & 15, g = lane >> 4;
  const int n0 = (blockIdx.x * kSmWaves + w) * 16;
  const int ks = blockIdx.y;
  // GLU mode (N = 2I): wavefronts 0, 1 take gate rows g0 + 16w .. + 15 and wavefronts 2, 3
  // the matching up rows, so each gate value meets its up value in this workgroup. Every
  // wavefront then stays to the end (the epilogue has a barrier); rows past I are clamped.
  const int glu = io.glu;
  const int g0 = blockIdx.x * (kSmWaves / 2) * 16;
  auto weight_row = [&](int j) {                   // weight row of this wavefront's row j
    if (glu) {
      const int i = g0 + (w & 1) * 16 + j;
      return (w >= kSmWaves / 2 ? glu : 0) + (i < glu ? i : glu - 1);
    }
    return n0 + j < N ? n0 + j : N - 1;
  };
  if (!glu && n0 >= N) return;
  const int kb = ks * k_per_split;
  const int ke = (kb + k_per_split < K) ? kb + k_per_split : K;
  const int8_t* wrow = wq + (int64_t)weight_row(c) * K;
  const half_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int mm = mt * 16 + c;
    xrow[mt] = x + x_row(io, mm < M ? mm : M - 1) * ldx;
  }
  float4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = {0.f, 0.f, 0.f, 0.f};

  struct Stage {
    int2_t wa[U], wb[U];
    half8_t xa[U][MT], xb[U][MT];
  };
  // lane (c, g), step u of a stage at k: K columns k + 64u + 16g .. +15 in two 8-column pieces
  // (K % 8 == 0, so a piece is entirely inside or outside [kb, ke)).
  auto load = [&](int k, Stage& st) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int ka = k + u * kSmKStep + 16 * g, kb2 = ka + 8;
      const int xa_col = ka < ke ? ka : K - 8, xb_col = kb2 < ke ? kb2 : K - 8;
      if constexpr (WIDE) {
        const int4_t v = ld<int4_t>(wrow + (ka < ke ? ka : K - 16));
        st.wa[u] = {v[0], v[1]};
        st.wb[u] = {v[2], v[3]};
      } else {
        st.wa[u] = ld<int2_t>(wrow + xa_col);
        st.wb[u] = ld<int2_t>(wrow + xb_col);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        st.xa[u][mt] = ld<half8_t>(xrow[mt] + xa_col);
        st.xb[u][mt] = ld<half8_t>(xrow[mt] + xb_col);
      }
    }
  };
  const half8_t hz = {0, 0, 0, 0, 0, 0, 0, 0};
  auto compute = [&](int k, const Stage& st) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int ka = k + u * kSmKStep + 16 * g;
      const half8_t fa = ka < ke ? i8x8_to_half8(st.wa[u]) : hz;
      const half8_t fb = ka + 8 < ke ? i8x8_to_half8(st.wb[u]) : hz;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[mt] = mfma16x16x32(fa, st.xa[u][mt], acc[mt]);
        acc[mt] = mfma16x16x32(fb, st.xb[u][mt], acc[mt]);
      }
    }
  };
  constexpr int SK = U * kSmKStep;                 // K per stage
  Stage s0, s1;
  load(kb, s0);
  for (int k = kb; k < ke; k += 2 * SK) {
    const bool more1 = k + SK < ke, more2 = k + 2 * SK < ke;   // uniform
    if (more1) load(k + SK, s1);
    compute(k, s0);
    if (more2) load(k + 2 * SK, s0);
    if (more1) compute(k + SK, s1);
  }
  // lane (c, g) holds Y[m = 16 mt + c][weight_row(4g + r)]
  if (glu && !part) {
    // Up wavefronts pass their fp16 results to the gate wavefronts through LDS, in register
    // order; the values are formed exactly as the plain epilogue below forms them.
    __shared__ half4_t s_xch[2][MT][64];
    float sc[4], bs[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int nr = weight_row(4 * g + r);
      sc[r] = load_scale(scale, scale_is_fp16, nr);
      bs[r] = bias ? (float)bias[nr] : 0.f;
    }
    auto value = [&](int mt) {
      const float v[4] = {acc[mt][0] * sc[0] + bs[0], acc[mt][1] * sc[1] + bs[1],
                          acc[mt][2] * sc[2] + bs[2], acc[mt][3] * sc[3] + bs[3]};
      return half4_t{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
    };
    const int hw = w & 1;
    if (w >= kSmWaves / 2) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) s_xch[hw][mt][lane] = value(mt);
    }
    __syncthreads();
    if (w < kSmWaves / 2) {
      const int col = g0 + hw * 16 + 4 * g;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int mm = mt * 16 + c;
        if (mm >= M || col >= glu) continue;
        const half4_t gv = value(mt), uv = s_xch[hw][mt][lane];
        const half4_t o = {silu_mul_h(gv[0], uv[0]), silu_mul_h(gv[1], uv[1]),
                           silu_mul_h(gv[2], uv[2]), silu_mul_h(gv[3], uv[3])};
        half_t* dst = y + (int64_t)mm * ldy + col;
        if (col + 3 < glu) {
          st<half4_t>(dst, o);
        } else {
          for (int r = 0; r < 4; ++r)
            if (col + r < glu) dst[r] = o[r];
        }
      }
    }
    return;
  }
  // GLU partials go to the weight row's column of the [M, 2I] product (valid while the gate
  // index is below I); otherwise column n0 + 4g + r.
  const int nn = glu ? weight_row(4 * g) : n0 + 4 * g;
  const int nend = glu ? (w >= kSmWaves / 2 ? 2 * glu : glu) : N;
  const bool run_ok = !glu || g0 + (w & 1) * 16 + 4 * g < glu;
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
      const float v[4] = {acc[mt][0] * sc[0] + bs[0], acc[mt][1] * sc[1] + bs[1],
                          acc[mt][2] * sc[2] + bs[2], acc[mt][3] * sc[3] + bs[3]};
      store_out4(io, y, ldy, mm, nn, N, v);
    }
  } else {
    float* pp = part + (int64_t)ks * M * N;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int mm = mt * 16 + c;
      if (mm >= M || !run_ok) continue;
      float* dst = pp + (int64_t)mm * N + nn;
      if (nn + 3 < nend) {
        st<float4_t>(dst, acc[mt]);
      } else {
        for (int r = 0; r < 4; ++r)
          if (nn + r < nend) dst[r] = acc[mt][r];
      }
    }
  }
}

// Output channel nn from its fp32 K sum: scale, bias, fp16.
__device__ __forceinline__ half_t finish_channel(float s, const void* __restrict__ scale,
                                                 int scale_is_fp16, const half_t* __restrict__ bias,
                                                 int nn) {
  float v = s * load_scale(scale, scale_is_fp16, nn);
  if (bias) v += (float)bias[nn];
  return (half_t)v;
}

// Element i of the [M, N] product from its split-K partials: sum (in split order), scale, bias,
// fp16.
__device__ __forceinline__ half_t reduce_partials(const float* __restrict__ part, int splits,
                                                  int64_t total, int64_t i,
                                                  const void* __restrict__ scale, int scale_is_fp16,
                                                  const half_t* __restrict__ bias, int nn) {
  // Up to 8 partials requested before any is summed (a plain loop waits for each load in turn),
  // then summed in split order; rows past `splits` are skipped, not added as zeros (which would
  // turn a -0 sum into +0).
  constexpr int U = 8;
  float s = 0.f;
  for (int k0 = 0; k0 < splits; k0 += U) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = k0 + u < splits ? part[(int64_t)(k0 + u) * total + i] : 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (k0 + u < splits) s += v[u];
  }
  return finish_channel(s, scale, scale_is_fp16, bias, nn);
}

// Sum of the split-K partials, then scale, bias and fp16 conversion.
__global__ void __launch_bounds__(256) w8a16_reduce_kernel(
    const float* __restrict__ part, int splits, const void* __restrict__ scale, int scale_is_fp16,
    const half_t* __restrict__ bias, half_t* __restrict__ y, int64_t ldy, int M, int N,
    GemmIo io) {
  const int64_t total = (int64_t)M * N;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int mm = (int)(i / N), nn = (int)(i % N);
    const half_t hv = reduce_partials(part, splits, total, i, scale, scale_is_fp16, bias, nn);
    if (io.yf)
      io.yf[(int64_t)mm * io.ldyf + nn] = (float)hv;
    else
      y[(int64_t)mm * ldy + nn] = hv;
  }
}

// The gated-MLP form: partials of the [M, 2I] gate_up product in, y[m][i] = silu(gate) * up out.
__global__ void __launch_bounds__(256) w8a16_glu_reduce_kernel(
    const float* __restrict__ part, int splits, const void* __restrict__ scale, int scale_is_fp16,
    const half_t* __restrict__ bias, half_t* __restrict__ y, int64_t ldy, int M, int I) {
  const int64_t N = 2 * (int64_t)I, total = (int64_t)M * N, outs = (int64_t)M * I;
  for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < outs;
       o += (int64_t)gridDim.x * blockDim.x) {
    const int mm = (int)(o / I), ii = (int)(o % I);
    const int64_t i = (int64_t)mm * N + ii;
    const half_t g = reduce_partials(part, splits, total, i, scale, scale_is_fp16, bias, ii);
    const half_t u = reduce_partials(part, splits, total, i + I, scale, scale_is_fp16, bias, I + ii);
    y[(int64_t)mm * ldy + ii] = silu_mul_h(g, u);
  }
}

// Split-K epilogue of a product that a residual add and RMSNorm consume (o_proj and down_proj in
// a decoder layer): row t of y is reduced as w8a16_reduce_kernel reduces it (split order, scale,
// bias, fp16), then res_out = y + res and out = rmsnorm(res_out) * w as the standalone norm
// computes them, so the pair of launches replaces reduce + norm with the same values.
__global__ void __launch_bounds__(kRowThreads) w8a16_reduce_rmsnorm_kernel(
    const float* __restrict__ part, int splits, const void* __restrict__ scale, int scale_is_fp16,
    const half_t* __restrict__ bias, const half_t* __restrict__ res, int64_t res_st,
    const half_t* __restrict__ w, half_t* __restrict__ out, int64_t out_st,
    half_t* __restrict__ res_out, int64_t res_out_st, int M, int N, float eps) {
  const int64_t t = blockIdx.x;
  const int64_t total = (int64_t)M * N;
  auto load_x = [&](int i) {
    float4_t a = {0.f, 0.f, 0.f, 0.f}, b = {0.f, 0.f, 0.f, 0.f};
    constexpr int U = 4;                         // partials requested before any is summed
    for (int k0 = 0; k0 < splits; k0 += U) {
      float4_t va[U], vb[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (k0 + u < splits) {                   // uniform over the workgroup
          const float* pp = part + (int64_t)(k0 + u) * total + t * N + i;
          va[u] = ld<float4_t>(pp);
          vb[u] = ld<float4_t>(pp + 4);
        } else {
          va[u] = vb[u] = float4_t{0.f, 0.f, 0.f, 0.f};
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (k0 + u < splits) {                   // split order, as the plain reduction
          a += va[u];
          b += vb[u];
        }
    }
    half8_t v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = finish_channel(a[e], scale, scale_is_fp16, bias, i + e);
      v[4 + e] = finish_channel(b[e], scale, scale_is_fp16, bias, i + 4 + e);
    }
    return v;
  };
  rmsnorm_row<true>(load_x, res + t * res_st, w, out + t * out_st, res_out + t * res_out_st, N,
                    eps);
}

// ------------------------------------------------------------------------------------------
// Skinny products (M <= 64, a decode step's projections and the logits): no split-K launch.
// ------------------------------------------------------------------------------------------
// Workgroup = KW wavefronts on RT x 16 weight rows (output channels) and every row of x (MT
// 16-row m tiles), over the whole K: wavefront w takes a contiguous slice of the 64-wide K steps,
// so the workgroup streams each of its weight rows once, front to back, and reads x once. The
// KW partial accumulators meet in LDS (a tree: half the wavefronts hand theirs to the other
// half, log2 KW rounds) and wavefront 0 applies scale and bias and stores; no fp32 partials
// leave the workgroup and no reduction kernel follows.
//
// Per K step, lane (c, g) loads 16 bytes of weight row c of each row tile (columns 16g .. 16g+15
// of the step: 1 KiB per tile and instruction, every byte used once) and the same 16 columns of
// x row c of each m tile (two 16-byte loads), and multiplies them on v_mfma_f32_16x16x32_f16 as
// two K = 32 products (columns 16g .. 16g+7, then 16g+8 .. 16g+15; the contraction index is
// permuted the same way in both operands). Loads run P steps ahead in a register ring.
//
// TAIL (K % 64 != 0): in the last step, 8-column pieces at or past K read column K - 8 instead
// (in range) and their widened weights are zeroed. GLU mode (io.glu = I, N = 2I): row tiles
// rt < RT/2 hold gate rows, rt >= RT/2 the matching up rows, so wavefront 0 forms
// silu(gate) * up itself.
constexpr int kSkStep = 64;

template <int MT, int RT, int KW, int P, bool TAIL>
__global__ void __launch_bounds__(KW * 64) w8a16_skinny_kernel(
    const half_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ wq,
    const void* __restrict__ scale, int scale_is_fp16, const half_t* __restrict__ bias,
    half_t* __restrict__ y, int64_t ldy, int M, int N, int K, GemmIo io) {
  static_assert(KW == 4 || KW == 8 || KW == 16, "4, 8 or 16 wavefronts");
  static_assert(P >= 1 && P <= 8, "one to eight steps in flight");
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int glu = io.glu;
  // weight row of row tile rt, row j within the tile (clamped into the matrix)
  auto weight_row = [&](int rt, int j) {
    if (glu) {
      constexpr int HALF = RT / 2 > 0 ? RT / 2 : 1;
      const int i = blockIdx.x * 16 * HALF + 16 * (rt % HALF) + j;
      return (rt >= HALF ? glu : 0) + (i < glu ? i : glu - 1);
    }
    const int n = blockIdx.x * 16 * RT + 16 * rt + j;
    return n < N ? n : N - 1;
  };
  const int nsteps = (K + kSkStep - 1) / kSkStep;
  const int per = (nsteps + KW - 1) / KW;
  const int s0 = w * per;
  const int s1 = s0 + per < nsteps ? s0 + per : nsteps;
  const int8_t* wrow[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) wrow[rt] = wq + (int64_t)weight_row(rt, c) * K + 16 * g;
  const half_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int mm = 16 * mt + c;
    xrow[mt] = x + x_row(io, mm < M ? mm : M - 1) * ldx + 16 * g;
  }
  struct Step {
    int4_t wv[RT];
    half8_t xa[MT], xb[MT];
  };
  // Step s's loads (s < nsteps): column offsets of the lane's two 8-column pieces, clamped.
  auto load = [&](int s, Step& st) {
    const int k = s * kSkStep;
    if constexpr (TAIL) {
      const int ca = k + 16 * g < K ? k : K - 8 - 16 * g;
      const int cb = k + 16 * g + 8 < K ? k + 8 : K - 8 - 16 * g;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int2_t a = ld<int2_t>(wrow[rt] + ca), b = ld<int2_t>(wrow[rt] + cb);
        st.wv[rt] = {a[0], a[1], b[0], b[1]};
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        st.xa[mt] = ld<half8_t>(xrow[mt] + ca);
        st.xb[mt] = ld<half8_t>(xrow[mt] + cb);
      }
    } else {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) st.wv[rt] = ld<int4_t>(wrow[rt] + k);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        st.xa[mt] = ld<half8_t>(xrow[mt] + k);
        st.xb[mt] = ld<half8_t>(xrow[mt] + k + 8);
      }
    }
  };
  float4_t acc[RT][MT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[rt][mt] = {0.f, 0.f, 0.f, 0.f};
  const half8_t hz = {0, 0, 0, 0, 0, 0, 0, 0};
  auto compute = [&](int s, const Step& st) {
    const int k = s * kSkStep + 16 * g;
    const bool oka = !TAIL || k < K, okb = !TAIL || k + 8 < K;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const half8_t fa = oka ? i8x8_to_half8(int2_t{st.wv[rt][0], st.wv[rt][1]}) : hz;
      const half8_t fb = okb ? i8x8_to_half8(int2_t{st.wv[rt][2], st.wv[rt][3]}) : hz;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[rt][mt] = mfma16x16x32(fa, st.xa[mt], acc[rt][mt]);
        acc[rt][mt] = mfma16x16x32(fb, st.xb[mt], acc[rt][mt]);
      }
    }
  };
  // Ring of P register steps: step s lives in slot (s - s0) % P; every iteration computes one
  // step and refills its slot with the step P ahead.
  Step ring[P];
#pragma unroll
  for (int u = 0; u < P; ++u)
    if (s0 + u < s1) load(s0 + u, ring[u]);
  for (int s = s0; s < s1; s += P) {
#pragma unroll
    for (int u = 0; u < P; ++u) {
      if (s + u < s1) {
        compute(s + u, ring[u]);
        if (s + u + P < s1) load(s + u + P, ring[u]);
      }
    }
  }
  // Tree reduction of the KW accumulators: in round h, wavefronts [h, 2h) publish theirs and
  // wavefronts [0, h) add them.
  __shared__ float4_t red[KW / 2][RT * MT][64];
#pragma unroll
  for (int h = KW / 2; h >= 1; h /= 2) {
    if (w >= h && w < 2 * h) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) red[w - h][rt * MT + mt][lane] = acc[rt][mt];
    }
    __syncthreads();
    if (w < h) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[rt][mt] += red[w][rt * MT + mt][lane];
    }
    __syncthreads();
  }
  if (w != 0) return;
  // lane (c, g) of tile (rt, mt) holds Y[m = 16 mt + c][weight_row(rt, 4g + r)], r = 0..3; every
  // output value is fp16(acc * scale + bias) formed by this one expression (the GLU and the
  // plain epilogue must round identically)
  auto value = [&](int rt, int mt, int r) {
    const int nr = weight_row(rt, 4 * g + r);
    return (half_t)(acc[rt][mt][r] * load_scale(scale, scale_is_fp16, nr) +
                    (bias ? (float)bias[nr] : 0.f));
  };
  if (glu) {
    constexpr int HALF = RT / 2 > 0 ? RT / 2 : 1;
#pragma unroll
    for (int rt = 0; rt < HALF; ++rt) {
      const int col = blockIdx.x * 16 * HALF + 16 * rt + 4 * g;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int mm = 16 * mt + c;
        if (mm >= M || col >= glu) continue;
        half4_t o;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = silu_mul_h(value(rt, mt, r), value(rt + HALF, mt, r));
        half_t* dst = y + (int64_t)mm * ldy + col;
        if (col + 3 < glu) {
          st<half4_t>(dst, o);
        } else {
          for (int r = 0; r < 4; ++r)
            if (col + r < glu) dst[r] = o[r];
        }
      }
    }
    return;
  }
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int nn = blockIdx.x * 16 * RT + 16 * rt + 4 * g;
    if (nn >= N) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int mm = 16 * mt + c;
      if (mm >= M) continue;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = (float)value(rt, mt, r);   // columns past N not stored
      store_out4(io, y, ldy, mm, nn, N, v);
    }
  }
}

// ------------------------------------------------------------------------------------------
// M <= 4: weight rows streamed on the VALU.
// ------------------------------------------------------------------------------------------
// The MFMA kernels' 16-row weight tiles leave most CUs idle on the 1536-row products at M = 1
// (96 workgroups for the down projection). Here a workgroup of 256 threads takes R = 256 / LPR
// weight rows (GLU: R / 2 gate rows and the matching up rows), each row on LPR consecutive
// threads (LPR = 128: two wavefronts): K is cut into 16-column pieces and thread j of the row's
// group takes pieces j, j + LPR, ..., PP of them requested before any is used. A thread keeps
// one fp32 sum per activation row, accumulated piece by piece with v_dot2_f32_f16 on the exactly
// widened int8 weights; a row's threads are summed by a fixed butterfly (and, over two
// wavefronts, a fixed-order sum through LDS), so the result does not depend on timing, and
// every output is fp16(acc * scale + bias) as in the other kernels. Needs K % 16 == 0 and
// 16-byte aligned weights and activation rows (the host falls back to the skinny kernel).
constexpr int kGemvMaxM = 4;

template <int MR, int LPR, int RPT, int PP>
__global__ void __launch_bounds__(256) w8a16_gemv_kernel(
    const half_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ wq,
    const void* __restrict__ scale, int scale_is_fp16, const half_t* __restrict__ bias,
    half_t* __restrict__ y, int64_t ldy, int M, int N, int K, GemmIo io) {
  constexpr int G = 256 / LPR;                   // thread groups (each RPT weight rows)
  constexpr int R = G * RPT;                     // weight rows per workgroup
  constexpr int WPR = LPR > kWave ? LPR / kWave : 1;   // wavefronts per group
  constexpr int LW = LPR < kWave ? LPR : kWave;        // lanes of a group within one wavefront
  static_assert(MR >= 1 && MR <= kGemvMaxM && LPR >= 16 && LPR <= 256 && (LPR & (LPR - 1)) == 0 &&
                    (RPT == 1 || RPT == 2 || RPT == 4) && (R % 2 == 0 || RPT == 1),
                "gemv shape");
  __shared__ float s_part[R][WPR][MR];
  const int tid = threadIdx.x;
  const int grp = tid / LPR;                     // rows grp * RPT .. + RPT - 1 of the workgroup
  const int j = tid % LPR;
  const int glu = io.glu;
  // weight row of workgroup row r (clamped into the matrix; GLU: gate rows first, then up)
  auto weight_row = [&](int r) {
    if (glu) {
      const int i = blockIdx.x * (R / 2) + r % (R / 2);
      return (r >= R / 2 ? glu : 0) + (i < glu ? i : glu - 1);
    }
    const int n = blockIdx.x * R + r;
    return n < N ? n : N - 1;
  };
  const int8_t* wrow[RPT];
#pragma unroll
  for (int q = 0; q < RPT; ++q) wrow[q] = wq + (int64_t)weight_row(grp * RPT + q) * K;
  const half_t* xrow[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) xrow[m] = x + x_row(io, m < M ? m : M - 1) * ldx;
  const int C = K / 16;                          // pieces per row
  float acc[RPT][MR];
#pragma unroll
  for (int q = 0; q < RPT; ++q)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[q][m] = 0.f;
  for (int base = 0; base < C; base += PP * LPR) {
    int4_t wv[PP][RPT];
    half8_t xa[PP][MR], xb[PP][MR];
#pragma unroll
    for (int u = 0; u < PP; ++u) {
      int pc = base + u * LPR + j;
      pc = pc < C ? pc : C - 1;                  // past the row: its last piece, not summed
#pragma unroll
      for (int q = 0; q < RPT; ++q) wv[u][q] = ld<int4_t>(wrow[q] + 16 * pc);
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        xa[u][m] = ld<half8_t>(xrow[m] + 16 * pc);
        xb[u][m] = ld<half8_t>(xrow[m] + 16 * pc + 8);
      }
    }
#pragma unroll
    for (int u = 0; u < PP; ++u) {
      if (base + u * LPR + j >= C) continue;
#pragma unroll
      for (int q = 0; q < RPT; ++q) {
        const half8_t fa = i8x8_to_half8(int2_t{wv[u][q][0], wv[u][q][1]});
        const half8_t fb = i8x8_to_half8(int2_t{wv[u][q][2], wv[u][q][3]});
#pragma unroll
        for (int m = 0; m < MR; ++m) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            acc[q][m] = __builtin_amdgcn_fdot2(half2_t{fa[2 * e], fa[2 * e + 1]},
                                               half2_t{xa[u][m][2 * e], xa[u][m][2 * e + 1]},
                                               acc[q][m], false);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            acc[q][m] = __builtin_amdgcn_fdot2(half2_t{fb[2 * e], fb[2 * e + 1]},
                                               half2_t{xb[u][m][2 * e], xb[u][m][2 * e + 1]},
                                               acc[q][m], false);
        }
      }
    }
  }
#pragma unroll
  for (int q = 0; q < RPT; ++q)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
#pragma unroll
      for (int off = LW / 2; off > 0; off >>= 1) acc[q][m] += __shfl_xor(acc[q][m], off, kWave);
    }
  if (j % LW == 0) {
#pragma unroll
    for (int q = 0; q < RPT; ++q)
#pragma unroll
      for (int m = 0; m < MR; ++m) s_part[grp * RPT + q][j / LW][m] = acc[q][m];
  }
  __syncthreads();
  auto row_sum = [&](int r, int m) {
    float a = s_part[r][0][m];
#pragma unroll
    for (int k = 1; k < WPR; ++k) a += s_part[r][k][m];
    return a;
  };
  auto value = [&](float a, int nr) {
    return (half_t)(a * load_scale(scale, scale_is_fp16, nr) + (bias ? (float)bias[nr] : 0.f));
  };
  if (glu) {
    for (int t = tid; t < (R / 2) * MR; t += 256) {
      const int r = t / MR, m = t % MR;
      const int col = blockIdx.x * (R / 2) + r;
      if (m >= M || col >= glu) continue;
      y[(int64_t)m * ldy + col] =
          silu_mul_h(value(row_sum(r, m), col), value(row_sum(R / 2 + r, m), glu + col));
    }
    return;
  }
  for (int t = tid; t < R * MR; t += 256) {
    const int r = t / MR, m = t % MR;
    const int n = blockIdx.x * R + r;
    if (m >= M || n >= N) continue;
    const half_t v = value(row_sum(r, m), n);
    if (io.yf)
      io.yf[(int64_t)m * io.ldyf + n] = (float)v;
    else
      y[(int64_t)m * ldy + n] = v;
  }
}

constexpr int kTileBK = 64;
constexpr int kTileChunks = kTileBK / 8;          // 16-byte fp16 chunks per tile row

// ------------------------------------------------------------------------------------------
// Larger M, wide tiles: weights straight into registers, activations DMA'd into LDS, 32x32 MFMAs.
// ------------------------------------------------------------------------------------------
// Workgroup = 4 wavefronts stacked along N on a (128 WN) x (32 WM) tile of Y^T, K step 64, on
// v_mfma_f32_32x32x16_f16 (on gfx950 it sustains twice the rate of the 16x16x32 form). Operand
// layouts, lane l = 32h + r: A holds A[row r][k 8h .. 8h+7], B holds B[k 8h .. 8h+7][col r], and
// result element e is D[row 8(e / 4) + 4h + e % 4][col r].
//
// Each wavefront owns 32 WN weight rows: lane (h, r) of a 32-row subtile uses the 32 bytes
// W[n + r][k + 32h .. + 31] of each K step, MFMA q bytes 8q .. 8q+7 (the MFMA reduces over its K
// slots in any order as long as both operands use the same one). The B operand of MFMA q for
// lane (h, r) is chunk 4h + q of activation row r, and every wavefront reads the whole
// activation tile from LDS. Both tiles travel by global_load_lds_dwordx4 (each lane's 16 bytes
// land at the next 16-byte slot of LDS, so they need no registers); a lane picks the piece its
// slot must hold under the stage's swizzle:
//   activations: chunk kc of row r at slot kc ^ ((r >> 1) & 7), so one DMA instruction reads 8
//     rows x 128 bytes and each 16-lane group of an operand read (rows r .. r+15 at one chunk
//     index) covers the 64 banks once (an XOR with r & 7 left pairs of lanes on one bank:
//     measured 1-9 % slower);
//   weights (WIDE): 16-byte piece c of row n at slot c ^ ((n >> 2) & 3) of the row's four, so one
//     DMA instruction reads 16 rows x 64 bytes, and each 16-lane group of the ds_read_b128 that
//     fetches a lane's pieces (rows r .. r+15 at one piece index) covers the 64 banks once.
// Measured on MI355X: loads whose wavefront instruction reads 32 rows x 32 bytes (the pattern of
// lanes loading their own A operands straight from the weight rows) stream at most ~2.9 TB/s
// with every CU busy and ~1.8 TB/s on 140 CUs; 16 rows x 64 bytes by DMA reach ~5 TB/s and
// ~3.7 TB/s. Without 16-byte alignment (K % 64 != 0, or an unaligned weight pointer) the weights
// go straight to registers in 8-byte pieces instead, one register stage per LDS stage.
//
// Loads are issued one step ahead of a ring of PD + 1 stages; each step waits for the batch of
// the next step (PD - 1 younger batches may stay in flight) and then takes one barrier. The wait
// and the barrier are written out instead of __syncthreads(), whose release fence would wait for
// every LDS-bound load in flight; the barrier carries a memory clobber so no load or LDS read
// moves across it.
//
// K tail (only the last split can end inside a K step, and only if K % 64 != 0): weight columns
// past the split end are zeroed at conversion; activation chunks past it are read at column
// K - 8 (finite input data whose weights are zero).
template <int N>
__device__ __forceinline__ void wait_vmem_below() {
  // s_waitcnt immediate: vmcnt in bits 3:0 and 15:14; expcnt (bits 6:4) and lgkmcnt (bits 11:8)
  // left at their maxima. The builtin, unlike inline assembly, tells the compiler's own wait
  // insertion which loads are complete.
  static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// The same with every LDS access of this wavefront complete as well (lgkmcnt 0).
template <int N>
__device__ __forceinline__ void wait_vmem_below_lds_done() {
  static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}
__device__ __forceinline__ void workgroup_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Scheduling pattern for one half step: the LDS reads first, the widening of the first weight
// operand, then MFMAs each followed by an equal share of the remaining VALU work, so that the
// widening runs in the MFMA shadow instead of in blocks between MFMA runs.
template <int NMFMA, int NVALU, int NDS>
__device__ __forceinline__ void interleave_mfma_valu() {
  constexpr int first = NVALU >= 10 ? 10 : NVALU;
  constexpr int per = (NVALU - first + NMFMA - 1) / NMFMA;
  __builtin_amdgcn_sched_group_barrier(0x100, NDS, 0);        // LDS reads
  if constexpr (first > 0) __builtin_amdgcn_sched_group_barrier(0x002, first, 0);
#pragma unroll
  for (int m = 0; m < NMFMA; ++m) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);        // one MFMA
    if constexpr (per > 0) __builtin_amdgcn_sched_group_barrier(0x002, per, 0);
  }
}

typedef float float16_t __attribute__((ext_vector_type(16)));

template <int WN, int WM, int PD, bool WIDE, bool TAIL>
__global__ void __launch_bounds__(256) w8a16_wide_kernel(
    const half_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ wq,
    const void* __restrict__ scale, int scale_is_fp16, const half_t* __restrict__ bias,
    half_t* __restrict__ y, int64_t ldy, int M, int N, int K, int k_per_split,
    float* __restrict__ part, GemmIo io) {
  constexpr int BK = kTileBK, CH = kTileChunks;
  constexpr int BN = 128 * WN, BM = 32 * WM;
  constexpr int XPT = BM * CH / 256;              // activation DMAs per thread per step
  constexpr int S = PD + 1;                       // stages (LDS, and weight registers if !WIDE)
  constexpr int WP = BN * BK / 16;                // 16-byte weight pieces per step
  constexpr int WDMA = WP / 256;                  // weight DMAs per thread per step (WIDE)
  constexpr int BATCH = XPT + (WIDE ? WDMA : 4 * WN);   // vector memory loads per thread per step
  static_assert(XPT * 256 == BM * CH, "activation tile must split over 256 threads");
  static_assert(WDMA * 256 == WP, "weight tile must split over 256 threads");
  static_assert(BN <= 256, "one scale per thread");
  static_assert(S >= 2 && S <= 8, "two to eight LDS stages");
  static_assert(!(WIDE && TAIL), "weight DMA needs whole 16-byte pieces");
  // One array per stage: the compiler's wait insertion then sees that an LDS read of one stage
  // cannot alias a DMA in flight into another and does not wait for it (stage indices are
  // constants after unrolling, so stage() folds to one array).
  __shared__ half8_t s_x0[BM * CH], s_x1[BM * CH], s_x2[S > 2 ? BM * CH : 1], s_x3[S > 3 ? BM * CH : 1];
  __shared__ half8_t s_x4[S > 4 ? BM * CH : 1], s_x5[S > 5 ? BM * CH : 1];
  __shared__ half8_t s_x6[S > 6 ? BM * CH : 1], s_x7[S > 7 ? BM * CH : 1];
  constexpr int WS = WIDE ? WP : 1;
  __shared__ int4_t s_w0[WS], s_w1[WS], s_w2[S > 2 ? WS : 1], s_w3[S > 3 ? WS : 1];
  __shared__ int4_t s_w4[S > 4 ? WS : 1], s_w5[S > 5 ? WS : 1], s_w6[S > 6 ? WS : 1], s_w7[S > 7 ? WS : 1];
  __shared__ float s_sc[BN], s_bs[BN];
  auto stage = [&](int st) -> half8_t* {
    return st == 0 ? s_x0 : st == 1 ? s_x1 : st == 2 ? s_x2 : st == 3 ? s_x3
         : st == 4 ? s_x4 : st == 5 ? s_x5 : st == 6 ? s_x6 : s_x7;
  };
  auto wstage = [&](int st) -> int4_t* {
    return st == 0 ? s_w0 : st == 1 ? s_w1 : st == 2 ? s_w2 : st == 3 ? s_w3
         : st == 4 ? s_w4 : st == 5 ? s_w5 : st == 6 ? s_w6 : s_w7;
  };
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, h = lane >> 5;
  const int n_tile = blockIdx.x * BN;
  const int m_base = blockIdx.y * BM;
  // Weight row of tile column nl (clamped into the matrix). In GLU mode the tile holds the gate
  // rows g0 .. g0 + BN/2 - 1 in its first half (wavefronts 0, 1) and the matching up rows in
  // its second half (wavefronts 2, 3), so each gate value and its up value meet in one workgroup.
  const int glu = io.glu;
  const int g0 = blockIdx.x * (BN / 2);
  auto weight_row = [&](int nl) {
    if (glu) {
      const int i = g0 + nl % (BN / 2);
      return (nl >= BN / 2 ? glu : 0) + (i < glu ? i : glu - 1);
    }
    const int n = n_tile + nl;
    return n < N ? n : N - 1;
  };
  static_assert(WN == 1, "GLU mode pairs wavefronts 0, 1 with 2, 3 (32 rows each)");
  // Weight piece c (16 bytes) of tile row nl sits at slot 4 nl + (c ^ ((nl >> 2) & 3)) of a stage.
  auto wslot = [](int nl, int c) { return 4 * nl + (c ^ ((nl >> 2) & 3)); };
  const int kb = blockIdx.z * k_per_split;
  const int ke = (kb + k_per_split < K) ? kb + k_per_split : K;
  const int nk = (ke - kb + BK - 1) / BK;

  // Per-channel scale and bias of the tile, read once into LDS for the epilogue (published by
  // the barriers of the main loop, which runs at least once).
  if (tid < BN) {
    const int nc = weight_row(tid);
    s_sc[tid] = part ? 1.f : load_scale(scale, scale_is_fp16, nc);
    s_bs[tid] = (part || !bias) ? 0.f : (float)bias[nc];
  }
  const int8_t* wrow[WIDE ? WDMA : WN];
  if constexpr (WIDE) {
    // DMA j of thread t fills slot 256 j + t: tile row (256 j + t) / 4, which holds piece
    // (t % 4) ^ ((row >> 2) & 3) there.
#pragma unroll
    for (int j = 0; j < WDMA; ++j) {
      const int nl = (256 * j + tid) / 4;
      wrow[j] = wq + (int64_t)weight_row(nl) * K + 16 * ((tid % 4) ^ ((nl >> 2) & 3));
    }
  } else {
#pragma unroll
    for (int i = 0; i < WN; ++i) wrow[i] = wq + (int64_t)weight_row(w * 32 * WN + 32 * i + r) * K + 32 * h;
  }
  // DMA i of thread t fills slot 256 i + t of a stage: row (256 i + t) / 8, position t % 8,
  // which holds chunk (t % 8) ^ ((row >> 1) & 7) = (t % 8) ^ ((t / 16) & 7) for every i.
  const int kcx = (tid % CH) ^ ((tid / 16) & 7);
  const half_t* xrow[XPT];
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int mm = m_base + (256 * i + tid) / CH;
    xrow[i] = x + x_row(io, mm < M ? mm : M - 1) * ldx + 8 * kcx;
  }

  // Step kt's loads (steps past the split end repeat the last one), all at in-range addresses.
  // Weight piece p (8 bytes each) of lane (h, r) is columns 32h + 8p .. + 7 of the step.
  auto issue = [&](int kt, int st, int4_t (&wr)[WN][2]) {
    const int k = kb + (kt < nk ? kt : nk - 1) * BK;
    const int kx = !TAIL || k + 8 * kcx < ke ? k : K - 8 - 8 * kcx;
#pragma unroll
    for (int i = 0; i < XPT; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(xrow[i] + kx),
                                       (__attribute__((address_space(3))) void*)(stage(st) + 256 * i + 64 * w),
                                       16, 0, 0);
    if constexpr (WIDE) {
#pragma unroll
      for (int j = 0; j < WDMA; ++j)
        __builtin_amdgcn_global_load_lds((const void*)(wrow[j] + k),
                                         (__attribute__((address_space(3))) void*)(wstage(st) + 256 * j + 64 * w),
                                         16, 0, 0);
    } else {
      int kp[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) kp[q] = !TAIL || k + 32 * h + 8 * q < ke ? k + 8 * q : K - 8 - 32 * h;
#pragma unroll
      for (int i = 0; i < WN; ++i) {
        const int2_t p0 = ld<int2_t>(wrow[i] + kp[0]), p1 = ld<int2_t>(wrow[i] + kp[1]);
        const int2_t p2 = ld<int2_t>(wrow[i] + kp[2]), p3 = ld<int2_t>(wrow[i] + kp[3]);
        wr[i][0] = {p0[0], p0[1], p1[0], p1[1]};
        wr[i][1] = {p2[0], p2[1], p3[0], p3[1]};
      }
    }
  };

  float16_t acc[WN][WM];
#pragma unroll
  for (int i = 0; i < WN; ++i)
#pragma unroll
    for (int j = 0; j < WM; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // B operands of MFMAs q0 and q0 + 1 of a step.
  auto read_b = [&](int st, int q0, half8_t (&b)[2][WM]) {
    const half8_t* sx = stage(st);
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int j = 0; j < WM; ++j) b[q][j] = sx[(32 * j + r) * CH + ((4 * h + q0 + q) ^ ((r >> 1) & 7))];
  };
  // A operands of MFMAs q0 and q0 + 1 of step kt (K tail columns zeroed).
  auto convert = [&](const int4_t (&wr)[WN][2], int kt, int q0, half8_t (&a)[2][WN]) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int p = q0 + q;
      const bool ok = !TAIL || kb + kt * BK + 32 * h + 8 * p < ke;
#pragma unroll
      for (int i = 0; i < WN; ++i) {
        const int4_t v = wr[i][p >> 1];
        const int lo = (p & 1) * 2;
        a[q][i] = i8x8_to_half8(int2_t{ok ? v[lo] : 0, ok ? v[lo + 1] : 0});
      }
    }
  };
  // WIDE: lane (h, r)'s weight pieces 2h, 2h + 1 of each subtile row of a stage.
  auto read_a = [&](int st, int4_t (&wr)[WN][2]) {
    const int4_t* sw = wstage(st);
#pragma unroll
    for (int i = 0; i < WN; ++i) {
      const int nl = 32 * (w * WN + i) + r;
      wr[i][0] = sw[wslot(nl, 2 * h)];
      wr[i][1] = sw[wslot(nl, 2 * h + 1)];
    }
  };
  auto mma = [&](const half8_t (&a)[2][WN], const half8_t (&b)[2][WM]) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int i = 0; i < WN; ++i)
#pragma unroll
        for (int j = 0; j < WM; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[q][i], b[q][j], acc[i][j], 0, 0, 0);
  };

  // Weight operands: WIDE reads step t's pieces from its LDS stage into `araw` (just after the
  // barrier that publishes it); otherwise they wait in register stage t % S.
  int4_t wreg[WIDE ? 1 : S][WN][2];
  int4_t araw[WN][2];
  auto wsrc = [&](int u) -> int4_t (&)[WN][2] {
    if constexpr (WIDE) return araw; else return wreg[u];
  };
  half8_t b0[2][WM], b1[2][WM];
  // Step t lives in stage t % S, constants of the loops unrolled by S. The prologue issues steps
  // 0 .. S-1 and waits for step 0; each main-loop iteration computes step kt and then issues step
  // kt + S into the stage it has just released. The main loop holds only whole groups of S steps
  // and no branch, so the compiler's wait accounting stays exact across its back edge (the
  // prologue leaves the same loads in flight as a group does); the last nk % S steps follow it,
  // after waiting for everything.
  //
  // Each step is split into two halves (MFMAs q = 0, 1 and q = 2, 3) so that LDS reads overlap
  // MFMAs instead of following the barrier in lock step on all four wavefronts: the second
  // half's B operands are read while the first half multiplies, and the next step's first-half
  // B operands (and weight pieces) while the second half multiplies. The barrier between the
  // halves publishes step kt + 1's tiles (its batch has landed on every wavefront) and guarantees
  // that every wavefront has finished its reads of step kt's stage (the wait before it includes
  // this wavefront's LDS reads; both halves' A operands are widened before it), so step kt + S's
  // batch is issued right after it into that stage.
  //
  // The explicit waits count vector-memory operations, which retire in issue order on one
  // counter whatever their kind. Each batch issues its activation DMAs before its weight loads:
  // without WIDE the compiler may sink the prologue's last weight loads (registers only the main
  // loop reads) below the first wait, and with this order that only removes operations the
  // wait's count already allows to be outstanding, never ones between the awaited DMAs and the
  // wait.
#pragma unroll
  for (int u = 0; u < S; ++u) issue(u, u, wsrc(u));
  wait_vmem_below_lds_done<PD * BATCH>();
  workgroup_barrier();
  read_b(0, 0, b0);
  if constexpr (WIDE) read_a(0, araw);
  int kt0 = 0;
  for (; kt0 + S <= nk; kt0 += S) {
#pragma unroll
    for (int u = 0; u < S; ++u) {
      const int kt = kt0 + u;
      half8_t a0[2][WN], a1[2][WN];
      read_b(u, 2, b1);
      convert(wsrc(u), kt, 0, a0);
      convert(wsrc(u), kt, 2, a1);
      mma(a0, b0);
      interleave_mfma_valu<2 * WN * WM, 40 * WN, 2 * WM>();
      __builtin_amdgcn_sched_barrier(0);
      wait_vmem_below_lds_done<(PD - 1) * BATCH>();   // step kt + 1's batch has landed
      workgroup_barrier();
      issue(kt + S, u, wsrc(u));                      // step kt's stage (and registers)
      read_b((u + 1) % S, 0, b0);                     // past the last step: never used
      if constexpr (WIDE) read_a((u + 1) % S, araw);
      mma(a1, b1);
      interleave_mfma_valu<2 * WN * WM, 0, 2 * WM + (WIDE ? 2 * WN : 0)>();
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int u = 0; u < S - 1; ++u) {
    const int kt = kt0 + u;
    if (kt < nk) {
      half8_t a0[2][WN], a1[2][WN];
      read_b(u, 2, b1);
      convert(wsrc(u), kt, 0, a0);
      convert(wsrc(u), kt, 2, a1);
      mma(a0, b0);
      wait_vmem_below_lds_done<0>();
      workgroup_barrier();
      read_b((u + 1) % S, 0, b0);
      if constexpr (WIDE) read_a((u + 1) % S, araw);
      mma(a1, b1);
    }
  }
  // No DMA may still be writing this workgroup's LDS when it exits.
  wait_vmem_below<0>();
  // lane (h, r) of subtile (i, j), element e = 4a + c: Y[m][n] with m = m_base + 32 j + r and
  // n = weight_row(32 WN w + 32 i + 8a + 4h + c); the four c are one 8-byte store.
  if constexpr (WN == 1 && WIDE) {   // the host fuses only products on the weight-DMA path
    if (io.rope_cos != nullptr && !part) {
      // RoPE + K/V cache write (the qkv product of a layer step, rope_kv_write_kernel's work):
      // the tile is head hd, dims 0..127. Every wavefront puts its fp16 results in LDS, dims
      // [0, 64) in stage 0 and [64, 128) in stage 1 (both idle now), rows in place; then each
      // thread takes 8 rotation pairs of a row, rotates them with rope4 (q and k heads) exactly
      // as rope_kv_write_kernel does from the same fp16 values, stores the row's 16-byte pieces
      // and, for k and v heads, the cache row of its slot.
      __syncthreads();                                  // every wavefront is done with the stages
      half_t* x1s = reinterpret_cast<half_t*>(s_x0);    // [BM][64]
      half_t* x2s = reinterpret_cast<half_t*>(s_x1);
      static_assert(sizeof(s_x0) == (size_t)BM * 64 * sizeof(half_t), "a stage holds half a head");
#pragma unroll
      for (int j = 0; j < WM; ++j)
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
          const int nl = w * 32 + 8 * a4 + 4 * h;
          const float4_t sc = *reinterpret_cast<const float4_t*>(&s_sc[nl]);
          const float4_t bs = *reinterpret_cast<const float4_t*>(&s_bs[nl]);
          const float o[4] = {acc[0][j][4 * a4] * sc[0] + bs[0], acc[0][j][4 * a4 + 1] * sc[1] + bs[1],
                              acc[0][j][4 * a4 + 2] * sc[2] + bs[2], acc[0][j][4 * a4 + 3] * sc[3] + bs[3]};
          const half4_t hv = {(half_t)o[0], (half_t)o[1], (half_t)o[2], (half_t)o[3]};
          *reinterpret_cast<half4_t*>((nl < 64 ? x1s : x2s) + (32 * j + r) * 64 + (nl & 63)) = hv;
        }
      __syncthreads();
      const int hd = blockIdx.x;
      const int H = io.rope_heads, KVH = io.rope_kv_heads;
      const bool rotate = hd < H + KVH;
      const int kvh = hd < H + KVH ? hd - H : hd - H - KVH;   // cache head of k / v tiles
      half_t* cache = hd < H ? nullptr : (hd < H + KVH ? io.kc : io.vc);
      for (int it = tid; it < BM * 8; it += 256) {
        const int m = it >> 3, g = it & 7;
        const int mm = m_base + m;
        if (mm >= M) continue;
        half8_t y1 = *reinterpret_cast<const half8_t*>(x1s + m * 64 + 8 * g);
        half8_t y2 = *reinterpret_cast<const half8_t*>(x2s + m * 64 + 8 * g);
        if (rotate) {
          const int64_t prow = rope_row(io.positions[mm], io.rope_max_pos) * 64 + 8 * g;
          half4_t a1, a2, b1, b2;
          rope4(lo4(y1), lo4(y2), ld<float4_t>(io.rope_cos + prow), ld<float4_t>(io.rope_sin + prow),
                a1, a2);
          rope4(hi4(y1), hi4(y2), ld<float4_t>(io.rope_cos + prow + 4),
                ld<float4_t>(io.rope_sin + prow + 4), b1, b2);
          y1 = half8_t{a1[0], a1[1], a1[2], a1[3], b1[0], b1[1], b1[2], b1[3]};
          y2 = half8_t{a2[0], a2[1], a2[2], a2[3], b2[0], b2[1], b2[2], b2[3]};
        }
        half_t* dst = y + (int64_t)mm * ldy + n_tile + 8 * g;
        st<half8_t>(dst, y1);
        st<half8_t>(dst + 64, y2);
        if (cache != nullptr) {
          const int64_t slot = io.slots[mm];
          if (slot >= 0 && slot < io.num_slots) {             // -1 = padding row
            half_t* crow = cache + (((slot >> 4) * KVH + kvh) * kBlockSize + (slot & 15)) * 128 + 8 * g;
            st<half8_t>(crow, y1);
            st<half8_t>(crow + 64, y2);
          }
        }
      }
      return;
    }
  }
  if constexpr (WM % 2 == 0) {         // GLU tiles pair subtiles (no 32-row GLU tiles)
    if (glu && !part) {
      // Every wavefront puts its fp16 results in LDS (gate values in stage 0, up values in stage
      // 1, both idle now) in register order, slot ((half, j, a), lane); then wavefronts w and w + 2
      // share column half w % 2, w < 2 finishing subtiles j < WM / 2 and w >= 2 the rest, each
      // lane at the same (row, columns) its slot came from.
      __syncthreads();                                  // every wavefront is done with the stages
      half4_t* xg = reinterpret_cast<half4_t*>(s_x0);   // 2 halves x WM x 4 x 64 lanes x 8 B each
      half4_t* xu = reinterpret_cast<half4_t*>(s_x1);
      static_assert(sizeof(s_x0) == 2 * WM * 4 * 64 * sizeof(half4_t), "exchange fits one stage");
      static_assert(WM % 2 == 0, "subtiles split between the two wavefronts of a half");
      const int half_w = w & 1;
      const bool is_up = w >= 2;
  #pragma unroll
      for (int j = 0; j < WM; ++j)
  #pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
          const int nl = w * 32 + 8 * a4 + 4 * h;
          const float4_t sc = *reinterpret_cast<const float4_t*>(&s_sc[nl]);
          const float4_t bs = *reinterpret_cast<const float4_t*>(&s_bs[nl]);
          const float o[4] = {acc[0][j][4 * a4] * sc[0] + bs[0], acc[0][j][4 * a4 + 1] * sc[1] + bs[1],
                              acc[0][j][4 * a4 + 2] * sc[2] + bs[2], acc[0][j][4 * a4 + 3] * sc[3] + bs[3]};
          const half4_t hv = {(half_t)o[0], (half_t)o[1], (half_t)o[2], (half_t)o[3]};
          (is_up ? xu : xg)[((half_w * WM + j) * 4 + a4) * 64 + lane] = hv;
        }
      __syncthreads();
  #pragma unroll
      for (int jj = 0; jj < WM / 2; ++jj) {
        const int j = (is_up ? WM / 2 : 0) + jj;
        const int mm = m_base + 32 * j + r;
  #pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
          const int col = g0 + 32 * half_w + 8 * a4 + 4 * h;
          if (mm >= M || col >= glu) continue;
          const int slot = ((half_w * WM + j) * 4 + a4) * 64 + lane;
          const half4_t gv = xg[slot], uv = xu[slot];
          const half4_t o = {silu_mul_h(gv[0], uv[0]), silu_mul_h(gv[1], uv[1]), silu_mul_h(gv[2], uv[2]),
                             silu_mul_h(gv[3], uv[3])};
          half_t* dst = y + (int64_t)mm * ldy + col;
          if (col + 3 < glu) {
            st<half4_t>(dst, o);
          } else {
            for (int c = 0; c < 4; ++c)
              if (col + c < glu) dst[c] = o[c];
          }
        }
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < WN; ++i) {
#pragma unroll
    for (int a4 = 0; a4 < 4; ++a4) {
      const int nl = w * 32 * WN + 32 * i + 8 * a4 + 4 * h;   // column within the tile
      // GLU partials: column of the [M, 2I] product; the four columns are valid together or
      // stop at I (the gate index of each half is what may run past the matrix)
      const int gi = g0 + nl % (BN / 2);
      const int nn = glu ? (nl >= BN / 2 ? glu : 0) + gi : n_tile + nl;
      const int nend = glu ? nn - gi + glu : N;        // first column past this run
      if (nn >= nend) continue;
      const float4_t sc = *reinterpret_cast<const float4_t*>(&s_sc[nl]);
      const float4_t bs = *reinterpret_cast<const float4_t*>(&s_bs[nl]);
#pragma unroll
      for (int j = 0; j < WM; ++j) {
        const int mm = m_base + 32 * j + r;
        if (mm >= M) continue;
        const float4_t v = {acc[i][j][4 * a4], acc[i][j][4 * a4 + 1], acc[i][j][4 * a4 + 2],
                            acc[i][j][4 * a4 + 3]};
        if (part) {
          float* dst = part + ((int64_t)blockIdx.z * M + mm) * N + nn;
          if (nn + 3 < nend) {
            st<float4_t>(dst, v);
          } else {
            for (int c = 0; c < 4; ++c)
              if (nn + c < nend) dst[c] = v[c];
          }
          continue;
        }
        const float o[4] = {v[0] * sc[0] + bs[0], v[1] * sc[1] + bs[1], v[2] * sc[2] + bs[2],
                            v[3] * sc[3] + bs[3]};
        store_out4(io, y, ldy, mm, nn, N, o);
      }
    }
  }
}

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------
constexpr int kSmallMMax = 32;

// The weight-streaming kernel re-reads the activations once per wavefront (M x K x 2 bytes per
// 16 output channels), so its cost grows with M x N; the wide kernel shares them through LDS
// but pays a fixed ~10 us for the shortest K. Measured on the 1.5B projections, streaming wins
// for M <= 8 everywhere and up to M = 32 on the narrow, short-K ones (M x N <= 64K, K <= 2048).
static bool use_small_path(int M, int N, int K) {
  if (M <= 8) return true;
  return M <= kSmallMMax && (int64_t)M * N <= 65536 && K <= 2048;
}
// K steps of loads in flight (wide kernel). With weights in LDS as well, 128-column tiles take
// one step fewer so that two workgroups (3 x 24 KB of stages each) stay resident per CU; measured
// at M = 2048 on the gate_up product: 165 us at 2 steps, 186 us at 3 (one workgroup per CU).
// 192-column tiles keep one step in flight (2 x 32 KB of stages, two workgroups per CU).
constexpr int kWidePrefetch = 3;
constexpr int wide_prefetch(bool dma, int wm) {
  return wm == 6 ? 1 : (dma && wm == 4 ? 2 : kWidePrefetch);
}

struct GemmPlan {
  bool small;
  int mt;          // m tiles (small and skinny paths)
  int bn, bm;      // tile shape (wide path): 128 x 192, 128 x 128, 128 x 64 or 128 x 32
  int splits;      // K splits
  int k_per_split;
  int rt;          // skinny path: 16-row weight tiles per workgroup (0: not skinny)
  int kw;          // skinny path: wavefronts per workgroup (the K split inside it)
  int gv;          // VALU path: threads per weight-row group (0: not this path)
  int gvr;         // VALU path: weight rows per thread
};

// Variants a caller (a tuning table) may name instead of the planner's choice.
enum GemmVariant : int {
  kVarAuto = 0, kVarStream = 1, kVarWide64 = 2, kVarWide128 = 3, kVarWide32 = 4, kVarSkinny = 5,
  kVarWide192 = 6, kVarGemv = 7
};
constexpr int kSkinnyMMax = 64;

// Skinny plan (measured on the 1.5B projections and the lm head, cold weights): one 16-row weight
// tile per workgroup (a GLU product pairs a gate and an up tile); the most resident wavefronts
// win, each issuing its whole share of the row at once: 8 wavefronts when the grid is at most
// two workgroups per CU, else 4 (more workgroups per CU fit, and all of them in one round).
// M = 1: 2048 x 1536 7.3 -> 4.3 us, 17920 x 1536 13.4 -> 8.9 us, 1536 x 8960 13.2 -> 9.3 us.
static void skinny_shape(int N, int cus, bool glu, GemmPlan* p) {
  p->rt = glu ? 2 : 1;
  // from N alone, so a GLU product splits K exactly as the unfused [M, 2I] product does (the
  // fused result must equal the unfused pair bit for bit)
  p->kw = (int64_t)((N + 15) / 16) <= 2LL * cus ? 8 : 4;
}

// Auto plan: skinny for M <= 16, and up to M = 32 for short-K, narrow products (where the wide
// tiles would need a K split and its reduction); past that the activations re-read per 16-row
// tile cost more than the wide tiles' LDS sharing saves.
static bool use_skinny(int M, int N, int K) {
  return M <= 16 || (M <= 32 && K <= 2048 && N <= 4096);
}

constexpr int kMaxSplits = 256;

// VALU path (w8a16_gemv_kernel) shape, measured on the 1.5B projections (cold weights, M = 1 /
// 2): K >= 4096 (down, 560 pieces per row) takes a whole workgroup per group of two rows (768
// workgroups for 1536 rows: 5.75 / 6.78 us; one row per 128 threads 6.17 / 7.70, per 64 threads
// 6.81 / 9.46); shorter K takes 32 threads per row, one row each (qkv 3.57 / 3.95 us, o 3.51 /
// 3.92, gate_up at M = 1 7.97), two rows each for a GLU product at M >= 2 (gate_up 9.06 against
// 9.84), sharing its activation loads between them.
static void gemv_shape(int M, int K, bool glu, GemmPlan* p) {
  if (K / 16 >= 256) {
    p->gv = 256;
    p->gvr = 2;
  } else {
    p->gv = 32;
    p->gvr = glu && M >= 2 ? 2 : 1;
  }
}
// Auto plan: the VALU path for M <= 2, where it beat the skinny kernel on all four projections
// (M = 1: 20.8 against 29.3 us for the four, M = 2: 23.7 against 30.2 us), and up to M = 4 for
// long K (down at M = 3 / 4: 8.9 / 9.7 against 10.1 / 10.6 us skinny; at K = 1536 the skinny
// kernel is 0.1-0.2 us faster there).
constexpr int kGemvAutoM = 2;
static bool use_gemv(int M, int N, int K) {
  return K % 16 == 0 && (M <= kGemvAutoM || (M <= kGemvMaxM && K >= 4096));
}
// Long-K products whose 16-row skinny tiles would cover under half the CUs (the down projection,
// 1536 x 8960: 96 workgroups) take 128 x 32 wide tiles split over K instead, from M = 5 to 16
// (down at M = 8 / 12 / 16: 11.7 / 11.8 / 11.9 us with 8 splits, 10.1 / 10.4 / 10.5 us with the
// 16 of the rule below, against 12.4 / 14.1 / 15.4 us skinny).
static bool use_wide_long_k(int M, int N, int K, int cus) {
  return M <= 16 && K >= 4096 && (int64_t)((N + 15) / 16) * 2 < cus;
}
// Short-K products with many output channels past the streaming path (M = 9 to 32) take 128 x 32
// wide tiles with no K split when their grid covers at least half the CUs: each activation row
// is then read by 140 tiles instead of 1120 skinny ones (the gate_up projection, 17920 x 1536,
// cold weights: M = 12 / 16 / 24 / 32 11.5 / 11.6 / 11.8 / 12.0 us against 12.7 / 15.0 / 12.6 /
// 12.8 us for the skinny and 128 x 64 plans). The fused gated form follows the same plan (14.1 ->
// 14.3 us at M = 16, 13.6 -> 13.6 at M = 24), so its result stays equal to the unfused pair's.
static bool use_wide32_wide_n(int M, int N, int K, int cus) {
  return M > 8 && M <= kSmallMMax && K <= 2048 && (int64_t)((N + 127) / 128) * 2 >= cus;
}

// Weight streaming: fill the device with wavefronts (about eight per CU) by splitting K,
// keeping at least 256 K per split and the fp32 partials (splits * M * N * 4 bytes) within a
// quarter of the weight bytes or 2 MB.
static int stream_splits(int M, int N, int K, int cus) {
  const int64_t wgs = (N + 16 * kSmWaves - 1) / (16 * kSmWaves);
  const int64_t target_wgs = 2LL * cus;
  int splits = (int)((target_wgs + wgs - 1) / wgs);
  const int max_by_k = K / 256 > 1 ? K / 256 : 1;
  const int64_t budget = (int64_t)N * K / 4 > (2LL << 20) ? (int64_t)N * K / 4 : (2LL << 20);
  const int64_t by_traffic64 = budget / ((int64_t)M * N * 4);
  const int max_by_traffic = by_traffic64 > 1 ? (int)by_traffic64 : 1;
  if (splits > max_by_k) splits = max_by_k;
  if (splits > max_by_traffic) splits = max_by_traffic;
  return splits < 1 ? 1 : splits;
}

// 128 x 64 wide tiles: split over K while the grid holds fewer than two workgroups per CU, each
// split keeps at least 20 K steps (below that the reduction costs more than the split saves)
// and the fp32 partials (written and read once more by the reduction) stay within half the
// weight bytes or 8 MB. The 1536 x 8960 product at M = 96 / 128 / 192 (cold weights): 18.4 /
// 19.3 / 19.8 us with the earlier floor of 32 K steps (4, 4 and 4 splits), 15.7 / 16.6 / 17.6
// us at 6 splits.
static int wide64_splits(int M, int N, int K, int cus) {
  const int nk = (K + kTileBK - 1) / kTileBK;
  const int64_t tiles = (int64_t)((N + 127) / 128) * ((M + 63) / 64);
  const int64_t part_budget = (int64_t)N * K / 2 > (8LL << 20) ? (int64_t)N * K / 2 : (8LL << 20);
  int splits = 1;
  while (tiles * splits < 2LL * cus && nk / (splits + 1) >= 20 &&
         (int64_t)(splits + 1) * M * N * 4 <= part_budget)
    ++splits;
  return splits;
}

// The plan of a variant with `splits` K splits (0: the variant's own rule). kVarAuto: weight
// streaming when use_small_path says so; else 128 x 128 tiles (two workgroups per CU; the most
// work per CU of the shapes measured) once they cover more than half the CUs and M is past 64
// (below that most of their rows would be padding; at exactly half, 128 x 64 tiles give every
// CU one: the 2048 x 1536 product at M = 1024 17.0 -> 13.2 us), or 128 x 192 tiles where those fit one resident
// round and 128 x 128 tiles would not; else 128 x 64 tiles, or 128 x 32 tiles (four
// workgroups per CU) when M is past 64 but 128 x 64 tiles would cover fewer than half the CUs
// with no K split (short K): twice the workgroups for the same weights, which measured ~13 %
// faster on the 1536 x 1536 and 2048 x 1536 products at M = 256 and the former at M = 560;
// for M <= 64 (past the streaming path) 128 x 32 tiles split over K when 128 x 64 tiles would
// cover under a quarter of the CUs, and unsplit for short-K products with many output channels
// at M = 9 to 32 (use_wide32_wide_n). 128 x 32 tiles never split K by their own rule (splits 0),
// and GLU mode plans them as 128 x 64.
static GemmPlan plan_gemm_v(int M, int N, int K, int cus, int variant, int splits,
                            bool glu = false) {
  if (variant == kVarGemv || (variant == kVarAuto && use_gemv(M, N, K))) {
    GemmPlan p{false, 1, 0, 0, 1, K, 0, 0, 0, 0};
    gemv_shape(M, K, glu, &p);
    return p;
  }
  if (variant == kVarSkinny ||
      (variant == kVarAuto && use_skinny(M, N, K) && !use_wide_long_k(M, N, K, cus) &&
       !use_wide32_wide_n(M, N, K, cus))) {
    GemmPlan p{false, M <= 16 ? 1 : (M <= 32 ? 2 : 4), 0, 0, 1, K, 0, 0};
    skinny_shape(N, cus, glu, &p);
    return p;
  }
  if (variant == kVarAuto) {
    const int64_t n_tiles = (N + 127) / 128;
    variant = use_small_path(M, N, K) && !use_wide_long_k(M, N, K, cus)     ? kVarStream
              : (M > 64 && n_tiles * ((M + 127) / 128) * 2 > cus) ? kVarWide128
                                                                        : kVarWide64;
    splits = 0;
    // 128 x 64 tiles rather than 128 x 128 ones when they pad fewer rows and their grid still
    // fits one round of resident workgroups (the gated gate_up product at M = 192: 30.4 -> 25.8
    // us, plain 28.2 -> 25.6 us)
    if (variant == kVarWide128 && (M + 63) / 64 * 64 < (M + 127) / 128 * 128 &&
        n_tiles * ((M + 63) / 64) <= 2LL * cus)
      variant = kVarWide64;
    // 128 x 192 tiles when their grid fits one round of resident workgroups (two per CU) and the
    // 128 x 128 grid does not: the leftover partial round of 128-row tiles costs more than the
    // larger tiles. Measured on the gate_up product (17920 x 1536, cold weights) at M = 560:
    // 59.5 -> 48.3 us fused with SiLU.up, 56.3 -> 44.0 us plain; at M = 1024 and 2048, where
    // neither grid fits one round, 192-column tiles were no faster.
    if (variant == kVarWide128 && n_tiles * ((M + 191) / 192) <= 2LL * cus &&
        n_tiles * ((M + 127) / 128) > 2LL * cus)
      variant = kVarWide192;
    if (variant == kVarWide64 && M <= 96 && n_tiles * ((M + 63) / 64) * 4 < cus) {
      // Few rows and few columns (a decode step's projections): 128 x 32 tiles split over K
      // until about three workgroups per four CUs, at most 16 ways and at least 6 K steps each
      // (the reduction of M x N x 4-byte partials is cheap at this M). Measured at M = 48 and
      // 64: 2048 x 1536 11.1 -> 8.8 us, 1536 x 1536 11.0 -> 8.6 us, 1536 x 8960 18.6 -> 14.4 us
      // (8 splits); the 1536 x 8960 product at M = 5 / 16 / 32 with 16 splits instead of 8:
      // 11.7 / 12.0 / 12.5 -> 10.0 / 10.5 / 11.4 us (at M = 48 and 64, 8 splits stay fastest);
      // at M = 96 (three 32-row tiles): 1536 x 1536 10.0 -> 8.9 us, 2048 x 1536 10.3 -> 9.5 us,
      // 1536 x 8960 15.0 -> 14.4 us.
      const int64_t tiles32 = n_tiles * ((M + 31) / 32);
      const int nk = (K + kTileBK - 1) / kTileBK;
      int64_t sp = (3LL * cus / 4 + tiles32 - 1) / tiles32;
      sp = sp < 16 ? sp : 16;
      sp = sp < nk / 6 ? sp : nk / 6;
      variant = kVarWide32;
      splits = sp > 1 ? (int)sp : 1;
    }
    // 128 x 32 tiles, unsplit, past M = 64 when 128 x 64 tiles would cover at most half the CUs
    // and take no K split (the 2048 x 1536 product at M = 512: 12.3 -> 10.5 us)
    if (variant == kVarWide64 && M > 64 && n_tiles * ((M + 63) / 64) * 2 <= cus &&
        wide64_splits(M, N, K, cus) == 1)
      variant = kVarWide32;
    // Long K where the partial budget leaves 128 x 64 tiles unsplit on under 2/3 of the CUs:
    // 128 x 128 tiles split up to 3 ways instead (1536 x 8960, cold weights, at M = 768 / 896:
    // 47.8 / 48.5 -> 40.6 / 42.1 us; at M = 960, past the bound, 128 x 64 unsplit stays fastest)
    const int nk_all = (K + kTileBK - 1) / kTileBK;
    if (variant == kVarWide64 && M > 96 && nk_all >= 64 &&
        n_tiles * ((M + 63) / 64) * 3 < 2LL * cus && wide64_splits(M, N, K, cus) == 1) {
      const int64_t t128 = n_tiles * ((M + 127) / 128);
      const int64_t sp = cus / t128;
      if (sp >= 2) {
        variant = kVarWide128;
        splits = sp < 3 ? (int)sp : 3;
      }
    }
    if (use_wide32_wide_n(M, N, K, cus)) {
      variant = kVarWide32;
      splits = 1;
    }
  }
  GemmPlan p{variant == kVarStream, (M + 15) / 16, 128,
             variant == kVarWide192 ? 192
                                    : (variant == kVarWide128 ? 128 : (variant == kVarWide32 ? 32 : 64)),
             1, K, 0, 0};
  if (p.small) {
    if (splits == 0) splits = stream_splits(M, N, K, cus);
    int kps = (K + splits - 1) / splits;
    kps = (kps + kSmKStep - 1) / kSmKStep * kSmKStep;
    p.splits = (K + kps - 1) / kps;
    p.k_per_split = kps;
    return p;
  }
  if (splits == 0) splits = variant == kVarWide64 ? wide64_splits(M, N, K, cus) : 1;
  const int nk = (K + kTileBK - 1) / kTileBK;
  if (splits > nk) splits = nk;
  if (splits > 1) {
    const int steps = (nk + splits - 1) / splits;
    p.k_per_split = steps * kTileBK;
    p.splits = (K + p.k_per_split - 1) / p.k_per_split;
  }
  return p;
}

static GemmPlan plan_gemm(int M, int N, int K, int cus) { return plan_gemm_v(M, N, K, cus, kVarAuto, 0); }

// fp32 partials [splits][M][N] of split-K (in GLU mode N = 2I).
static size_t gemm_workspace(const GemmPlan& p, int M, int N) {
  return p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
}

}  // namespace ts

using namespace ts;

extern "C" size_t ts_w8a16_workspace_bytes(int32_t M, int32_t N, int32_t K, int32_t cu_count) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return gemm_workspace(plan_gemm(M, N, K, cu_count > 0 ? cu_count : 256), M, N);
}

static bool variant_valid(int variant, int splits, int M) {
  return variant >= kVarAuto && variant <= kVarGemv && splits >= 0 && splits <= kMaxSplits &&
         (variant != kVarGemv || (M <= kGemvMaxM && splits <= 1)) &&
         (variant != kVarStream || M <= kSmallMMax) &&
         (variant != kVarSkinny || (M <= kSkinnyMMax && splits <= 1));
}

extern "C" size_t ts_w8a16_workspace_bytes_v(int32_t M, int32_t N, int32_t K, int32_t variant,
                                             int32_t splits, int32_t cu_count) {
  if (M <= 0 || N <= 0 || K <= 0 || !variant_valid(variant, splits, M)) return 0;
  return gemm_workspace(plan_gemm_v(M, N, K, cu_count > 0 ? cu_count : 256, variant, splits), M,
                        N);
}

// Validated launch shared by the GEMM and logits entry points.
// With splits_out, a product planned with split K leaves its fp32 partials in the workspace
// (no reduction launch) and *splits_out says how many; otherwise *splits_out = 1 and y is
// written.
static int w8a16_launch(const half_t* xp, int64_t ldx, const int8_t* wq, const void* scale,
                        int32_t scale_is_fp16, const half_t* bp, half_t* yp, int64_t ldy,
                        int32_t M, int32_t N, int32_t K, void* workspace, size_t workspace_bytes,
                        hipStream_t s, const GemmIo& io, int variant, int splits,
                        int* splits_out = nullptr) {
  int cus = 0;
  int st = device_cu_count(s, &cus);
  if (st != TS_OK) return st;
  const bool glu = io.glu > 0;                    // N = 2 * io.glu, y is [M, io.glu]
  GemmPlan p = plan_gemm_v(M, N, K, cus, variant, splits, glu);
  if (p.gv > 0 && !(M <= kGemvMaxM && K % 16 == 0 && aligned(wq, 16) && aligned(xp, 16) &&
                    ldx % 8 == 0))
    p = plan_gemm_v(M, N, K, cus, kVarSkinny, 0, glu);   // the VALU path's alignment not met
  if (glu && p.bm == 32) p.bm = 64;               // GLU tiles pair 32-row subtiles (same splits)
  const size_t need = gemm_workspace(p, M, N);
  TS_REQUIRE(need == 0 || (workspace && workspace_bytes >= need && aligned(workspace, 16)),
             TS_ERR_WORKSPACE, "w8a16: workspace of %zu bytes needed, got %zu", need,
             workspace_bytes);
  if (splits_out) *splits_out = p.splits;
  auto reduce = [&](float* part) {
    if (splits_out) return;
    if (glu) {
      const int64_t want = ((int64_t)M * io.glu + 255) / 256;
      w8a16_glu_reduce_kernel<<<(int)(want < 4096 ? want : 4096), 256, 0, s>>>(
          part, p.splits, scale, scale_is_fp16, bp, yp, ldy, M, io.glu);
    } else {
      const int64_t want = ((int64_t)M * N + 255) / 256;
      w8a16_reduce_kernel<<<(int)(want < 4096 ? want : 4096), 256, 0, s>>>(
          part, p.splits, scale, scale_is_fp16, bp, yp, ldy, M, N, io);
    }
  };
  if (p.gv > 0) {
    const int rows = 256 / p.gv * p.gvr;
    const dim3 grid(glu ? (io.glu + rows / 2 - 1) / (rows / 2) : (N + rows - 1) / rows);
    const int per = (K / 16 + p.gv - 1) / p.gv;  // pieces per thread
#define TS_GV_LAUNCH(MR, LPR, RPT, PP)                                                             \
  w8a16_gemv_kernel<MR, LPR, RPT, PP><<<grid, 256, 0, s>>>(xp, ldx, wq, scale, scale_is_fp16, bp, \
                                                           yp, ldy, M, N, K, io)
    // pieces requested at once per thread: all of them where the registers allow
#define TS_GV_M(LPR, RPT)                                                                          \
  {                                                                                                \
    if (M == 1) {                                                                                  \
      if (per <= 3) TS_GV_LAUNCH(1, LPR, RPT, 3); else TS_GV_LAUNCH(1, LPR, RPT, 6);               \
    } else if (M == 2) {                                                                           \
      if (per <= 3) TS_GV_LAUNCH(2, LPR, RPT, 3); else TS_GV_LAUNCH(2, LPR, RPT, 6);               \
    } else {                                                                                       \
      if (per <= 3) TS_GV_LAUNCH(4, LPR, RPT, 3); else TS_GV_LAUNCH(4, LPR, RPT, 4);               \
    }                                                                                              \
  }
    if (p.gv == 256) {
      TS_GV_M(256, 2)
    } else if (p.gvr == 2) {
      TS_GV_M(32, 2)
    } else {
      TS_GV_M(32, 1)
    }
#undef TS_GV_M
#undef TS_GV_LAUNCH
  } else if (p.rt > 0) {
    // GLU: a workgroup covers 8 RT gate columns (its RT / 2 gate tiles and their up tiles)
    const int cols = glu ? io.glu : N;
    const int per_wg = glu ? 8 * p.rt : 16 * p.rt;
    const dim3 grid((cols + per_wg - 1) / per_wg);
    const bool tail = K % kSkStep != 0 || !aligned(wq, 16);
#define TS_SK_LAUNCH(MTV, RTV, KWV)                                                                \
  {                                                                                                \
    constexpr int PV = MTV == 4 ? 2 : (MTV == 2 || KWV == 8 ? 4 : 8);                              \
    if (tail)                                                                                      \
      w8a16_skinny_kernel<MTV, RTV, KWV, PV, true><<<grid, KWV * 64, 0, s>>>(                      \
          xp, ldx, wq, scale, scale_is_fp16, bp, yp, ldy, M, N, K, io);                            \
    else                                                                                           \
      w8a16_skinny_kernel<MTV, RTV, KWV, PV, false><<<grid, KWV * 64, 0, s>>>(                     \
          xp, ldx, wq, scale, scale_is_fp16, bp, yp, ldy, M, N, K, io);                            \
  }
#define TS_SK_RT(MTV)                                                                              \
  if (p.rt == 2) {                                                                                 \
    if (p.kw == 8) TS_SK_LAUNCH(MTV, 2, 8) else TS_SK_LAUNCH(MTV, 2, 4)                            \
  } else if (p.kw == 8) TS_SK_LAUNCH(MTV, 1, 8) else TS_SK_LAUNCH(MTV, 1, 4)
    if (p.mt == 1) {
      TS_SK_RT(1)
    } else if (p.mt == 2) {
      TS_SK_RT(2)
    } else {
      TS_SK_RT(4)
    }
#undef TS_SK_RT
#undef TS_SK_LAUNCH
  } else if (p.small) {
    float* part = p.splits > 1 ? static_cast<float*>(workspace) : nullptr;
    const int rows_per_wg = glu ? 16 * kSmWaves / 2 : 16 * kSmWaves;   // GLU: gate columns
    const dim3 grid(((glu ? io.glu : N) + rows_per_wg - 1) / rows_per_wg, p.splits);
    const bool wide = K % 16 == 0 && aligned(wq, 16);
#define TS_SM_CASE(MTV)                                                                          \
  case MTV:                                                                                      \
    if (wide)                                                                                    \
      w8a16_small_kernel<MTV, true><<<grid, kSmWaves * 64, 0, s>>>(                             \
          xp, ldx, wq, scale, scale_is_fp16, bp, yp, ldy, M, N, K, p.k_per_split, part, io);    \
    else                                                                                         \
      w8a16_small_kernel<MTV, false><<<grid, kSmWaves * 64, 0, s>>>(                            \
          xp, ldx, wq, scale, scale_is_fp16, bp, yp, ldy, M, N, K, p.k_per_split, part, io);    \
    break;
    switch (p.mt) {
      TS_SM_CASE(1)
      TS_SM_CASE(2)
    }
#undef TS_SM_CASE
    if (part) reduce(part);
  } else {
    float* part = p.splits > 1 ? static_cast<float*>(workspace) : nullptr;
    const int tiles_n = glu ? (io.glu + p.bn / 2 - 1) / (p.bn / 2) : (N + p.bn - 1) / p.bn;
    const dim3 grid(tiles_n, (M + p.bm - 1) / p.bm, p.splits);
    const bool fast = K % kTileBK == 0 && aligned(wq, 16);   // weight DMA, no K tail
#define TS_WIDE_LAUNCH(WNV, WMV)                                                                   \
  if (fast)                                                                                        \
    w8a16_wide_kernel<WNV, WMV, wide_prefetch(true, WMV), true, false><<<grid, 256, 0, s>>>(       \
        xp, ldx, wq, scale, scale_is_fp16, bp, yp, ldy, M, N, K, p.k_per_split, part, io);         \
  else                                                                                             \
    w8a16_wide_kernel<WNV, WMV, wide_prefetch(false, WMV), false, true><<<grid, 256, 0, s>>>(      \
        xp, ldx, wq, scale, scale_is_fp16, bp, yp, ldy, M, N, K, p.k_per_split, part, io)
    if (p.bm == 192) {
      TS_WIDE_LAUNCH(1, 6);
    } else if (p.bm == 128) {
      TS_WIDE_LAUNCH(1, 4);
    } else if (p.bm == 64) {
      TS_WIDE_LAUNCH(1, 2);
    } else {
      TS_WIDE_LAUNCH(1, 1);
    }
#undef TS_WIDE_LAUNCH
    if (part) reduce(part);
  }
  return TS_OK;
}

static int w8a16_gemm_checked(const void* x, int64_t ldx, const int8_t* wq, const void* scale,
                              int32_t scale_is_fp16, const void* bias, void* y, int64_t ldy,
                              int32_t M, int32_t N, int32_t K, int32_t variant, int32_t splits,
                              void* workspace, size_t workspace_bytes, void* stream) {
  TS_REQUIRE(M >= 0 && N > 0 && K > 0, TS_ERR_INVALID_ARG, "w8a16: bad shape M=%d N=%d K=%d", M,
             N, K);
  TS_REQUIRE(variant_valid(variant, splits, M < 1 ? 1 : M), TS_ERR_UNSUPPORTED,
             "w8a16: variant %d with %d splits is not available for M=%d", variant, splits, M);
  if (M == 0) return TS_OK;
  TS_REQUIRE(x && wq && scale && y, TS_ERR_INVALID_ARG, "w8a16: null pointer argument");
  TS_REQUIRE(K % 8 == 0, TS_ERR_UNSUPPORTED, "w8a16: K=%d is not a multiple of 8", K);
  TS_REQUIRE(ldx >= K && ldx % 8 == 0 && ldy >= N && aligned(x, 16) && aligned(wq, 8) &&
                 aligned(y, 2),
             TS_ERR_INVALID_ARG, "w8a16: x must be 16-byte aligned rows (ldx %% 8 == 0), wq 8-byte aligned");
  TS_REQUIRE(!(ldy % 4) && aligned(y, 8), TS_ERR_INVALID_ARG,
             "w8a16: y rows must be 8-byte aligned (ldy %% 4 == 0)");
  const GemmIo io{nullptr, 0, nullptr, 0, 0};
  const int st = w8a16_launch(static_cast<const half_t*>(x), ldx, wq, scale, scale_is_fp16,
                              static_cast<const half_t*>(bias), static_cast<half_t*>(y), ldy, M,
                              N, K, workspace, workspace_bytes,
                              reinterpret_cast<hipStream_t>(stream), io, variant, splits);
  if (st != TS_OK) return st;
  return check_launch("w8a16_gemm");
}

extern "C" int ts_w8a16_gemm(const void* x, int64_t ldx, const int8_t* wq, const void* scale,
                             int32_t scale_is_fp16, const void* bias, void* y, int64_t ldy,
                             int32_t M, int32_t N, int32_t K, void* workspace,
                             size_t workspace_bytes, void* stream) {
  ts::clear_error();
  return w8a16_gemm_checked(x, ldx, wq, scale, scale_is_fp16, bias, y, ldy, M, N, K, kVarAuto, 0,
                            workspace, workspace_bytes, stream);
}

extern "C" int ts_w8a16_gemm_v(const void* x, int64_t ldx, const int8_t* wq, const void* scale,
                               int32_t scale_is_fp16, const void* bias, void* y, int64_t ldy,
                               int32_t M, int32_t N, int32_t K, int32_t variant, int32_t splits,
                               void* workspace, size_t workspace_bytes, void* stream) {
  ts::clear_error();
  return w8a16_gemm_checked(x, ldx, wq, scale, scale_is_fp16, bias, y, ldy, M, N, K, variant,
                            splits, workspace, workspace_bytes, stream);
}

// The qkv product of a layer step with RoPE and the K/V cache write in the product's epilogue
// (linear, then rope_kv_write: model/qwen2.py:26-28, :89). Fused when each 128-column tile is
// one head (head_dim 128), the plan has one K split and the rows and tables are 16-byte
// aligned; otherwise the product and ts_rope_kv_write run as two launches. Same results either
// way: the epilogue rotates the product's own fp16 values with rope_kv_write's arithmetic.
extern "C" int ts_w8a16_qkv_rope_kv_write(
    const void* x, int64_t ldx, const int8_t* wq, const void* scale, int32_t scale_is_fp16,
    const void* bias, void* qkv, int64_t ld_qkv, int32_t M, int32_t K, int32_t num_heads,
    int32_t num_kv_heads, int32_t head_dim, const int64_t* positions, const float* cos_table,
    const float* sin_table, int64_t max_position, void* k_cache, void* v_cache,
    int64_t num_blocks, const int64_t* slot_mapping, int32_t variant, int32_t splits,
    void* workspace, size_t workspace_bytes, void* stream) {
  ts::clear_error();
  TS_REQUIRE(num_heads > 0 && num_kv_heads > 0 && head_dim > 0, TS_ERR_INVALID_ARG,
             "w8a16_qkv_rope_kv_write: bad head counts");
  const int N = (num_heads + 2 * num_kv_heads) * head_dim;
  if (M == 0) return TS_OK;
  TS_REQUIRE(M > 0, TS_ERR_INVALID_ARG, "w8a16_qkv_rope_kv_write: M=%d < 0", M);
  TS_REQUIRE(positions && cos_table && sin_table && max_position > 0 && k_cache && v_cache &&
                 slot_mapping && num_blocks > 0,
             TS_ERR_INVALID_ARG, "w8a16_qkv_rope_kv_write: null pointer, empty table or empty cache");
  int cus = 0;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int st = device_cu_count(s, &cus);
  if (st != TS_OK) return st;
  bool fuse = head_dim == 128 && variant_valid(variant, splits, M) && ld_qkv % 8 == 0 &&
              aligned(qkv, 16) && aligned(cos_table, 16) && aligned(sin_table, 16) &&
              aligned(k_cache, 16) && aligned(v_cache, 16);
  if (fuse) {
    const GemmPlan p = plan_gemm_v(M, N, K, cus, variant, splits);
    fuse = !p.small && p.rt == 0 && p.splits == 1 && p.bn == 128 && K % kTileBK == 0 &&
           aligned(wq, 16);                         // the weight-DMA wide kernel
  }
  if (!fuse) {
    st = w8a16_gemm_checked(x, ldx, wq, scale, scale_is_fp16, bias, qkv, ld_qkv, M, N, K, variant,
                            splits, workspace, workspace_bytes, stream);
    if (st != TS_OK) return st;
    return ts_rope_kv_write(qkv, ld_qkv, positions, cos_table, sin_table, max_position, M,
                            num_heads, num_kv_heads, head_dim, k_cache, v_cache, num_blocks,
                            slot_mapping, stream);
  }
  TS_REQUIRE(x && wq && scale, TS_ERR_INVALID_ARG, "w8a16_qkv_rope_kv_write: null pointer argument");
  TS_REQUIRE(K > 0 && K % 8 == 0, TS_ERR_UNSUPPORTED,
             "w8a16_qkv_rope_kv_write: K=%d is not a multiple of 8", K);
  TS_REQUIRE(ldx >= K && ldx % 8 == 0 && ld_qkv >= N && aligned(x, 16) && aligned(wq, 8),
             TS_ERR_INVALID_ARG,
             "w8a16_qkv_rope_kv_write: x must be 16-byte aligned rows (ldx %% 8 == 0), wq 8-byte aligned");
  GemmIo io{nullptr, 0, nullptr, 0, 0};
  io.positions = positions;
  io.rope_cos = cos_table;
  io.rope_sin = sin_table;
  io.rope_max_pos = max_position;
  io.rope_heads = num_heads;
  io.rope_kv_heads = num_kv_heads;
  io.kc = static_cast<half_t*>(k_cache);
  io.vc = static_cast<half_t*>(v_cache);
  io.slots = slot_mapping;
  io.num_slots = num_blocks * kBlockSize;
  st = w8a16_launch(static_cast<const half_t*>(x), ldx, wq, scale, scale_is_fp16,
                    static_cast<const half_t*>(bias), static_cast<half_t*>(qkv), ld_qkv, M, N, K,
                    workspace, workspace_bytes, s, io, variant, splits);
  if (st != TS_OK) return st;
  return check_launch("w8a16_qkv_rope_kv_write");
}

// Workspace of the fused product + residual add + RMSNorm: the split-K partials when the plan
// splits K, else the fp16 product rows the norm reads.
static size_t add_rmsnorm_workspace(const GemmPlan& p, int M, int N) {
  return p.splits > 1 ? gemm_workspace(p, M, N) : (size_t)M * N * sizeof(half_t);
}

extern "C" size_t ts_w8a16_add_rmsnorm_workspace_bytes(int32_t M, int32_t N, int32_t K,
                                                       int32_t variant, int32_t splits,
                                                       int32_t cu_count) {
  if (M <= 0 || N <= 0 || K <= 0 || !variant_valid(variant, splits, M)) return 0;
  return add_rmsnorm_workspace(plan_gemm_v(M, N, K, cu_count > 0 ? cu_count : 256, variant, splits),
                               M, N);
}

extern "C" int ts_w8a16_add_rmsnorm(const void* x, int64_t ldx, const int8_t* wq,
                                    const void* scale, int32_t scale_is_fp16, const void* bias,
                                    const void* residual, int64_t residual_stride,
                                    const void* norm_weight, void* out, int64_t out_stride,
                                    void* residual_out, int64_t residual_out_stride, int32_t M,
                                    int32_t N, int32_t K, float eps, int32_t variant,
                                    int32_t splits, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  ts::clear_error();
  TS_REQUIRE(M >= 0 && N > 0 && K > 0, TS_ERR_INVALID_ARG,
             "w8a16_add_rmsnorm: bad shape M=%d N=%d K=%d", M, N, K);
  TS_REQUIRE(variant_valid(variant, splits, M < 1 ? 1 : M), TS_ERR_UNSUPPORTED,
             "w8a16_add_rmsnorm: variant %d with %d splits is not available for M=%d", variant,
             splits, M);
  if (M == 0) return TS_OK;
  TS_REQUIRE(x && wq && scale && residual && norm_weight && out && residual_out,
             TS_ERR_INVALID_ARG, "w8a16_add_rmsnorm: null pointer argument");
  TS_REQUIRE(K % 8 == 0, TS_ERR_UNSUPPORTED, "w8a16_add_rmsnorm: K=%d is not a multiple of 8", K);
  TS_REQUIRE(N % kRowVec == 0 && N <= kRmsMaxIter * kRowThreads * kRowVec, TS_ERR_UNSUPPORTED,
             "w8a16_add_rmsnorm: N=%d must be a multiple of 8 and <= 8192", N);
  TS_REQUIRE(ldx >= K && ldx % 8 == 0 && aligned(x, 16) && aligned(wq, 8), TS_ERR_INVALID_ARG,
             "w8a16_add_rmsnorm: x must be 16-byte aligned rows (ldx %% 8 == 0), wq 8-byte aligned");
  TS_REQUIRE(residual_stride >= N && out_stride >= N && residual_out_stride >= N &&
                 residual_stride % kRowVec == 0 && out_stride % kRowVec == 0 &&
                 residual_out_stride % kRowVec == 0 && aligned(residual, 16) && aligned(out, 16) &&
                 aligned(residual_out, 16) && aligned(norm_weight, 16),
             TS_ERR_INVALID_ARG, "w8a16_add_rmsnorm: norm rows must be 16-byte aligned");
  int cus = 0;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (device_cu_count(stream, &cus) != TS_OK) return TS_ERR_DEVICE;
  const GemmPlan p = plan_gemm_v(M, N, K, cus, variant, splits);
  const size_t need = add_rmsnorm_workspace(p, M, N);
  TS_REQUIRE(workspace && workspace_bytes >= need && aligned(workspace, 16), TS_ERR_WORKSPACE,
             "w8a16_add_rmsnorm: workspace of %zu bytes needed, got %zu", need, workspace_bytes);
  const GemmIo io{nullptr, 0, nullptr, 0, 0};
  half_t* ytmp = static_cast<half_t*>(workspace);  // used only when K is not split
  int used_splits = 1;
  const int st = w8a16_launch(static_cast<const half_t*>(x), ldx, wq, scale, scale_is_fp16,
                              static_cast<const half_t*>(bias), ytmp, N, M, N, K, workspace,
                              workspace_bytes, s, io, variant, splits, &used_splits);
  if (st != TS_OK) return st;
  const half_t* rp = static_cast<const half_t*>(residual);
  const half_t* wp = static_cast<const half_t*>(norm_weight);
  half_t* op = static_cast<half_t*>(out);
  half_t* rop = static_cast<half_t*>(residual_out);
  if (used_splits > 1)
    w8a16_reduce_rmsnorm_kernel<<<dim3((unsigned)M), kRowThreads, 0, s>>>(
        static_cast<const float*>(workspace), used_splits, scale, scale_is_fp16,
        static_cast<const half_t*>(bias), rp, residual_stride, wp, op, out_stride, rop,
        residual_out_stride, M, N, eps);
  else
    rmsnorm_kernel<true><<<dim3((unsigned)M), kRowThreads, 0, s>>>(
        ytmp, N, rp, residual_stride, wp, op, out_stride, rop, residual_out_stride, N, eps);
  return check_launch("w8a16_add_rmsnorm");
}

extern "C" size_t ts_logits_int8_workspace_bytes(int32_t num_samples, int32_t vocab,
                                                  int32_t hidden_size, int32_t cu_count) {
  return ts_w8a16_workspace_bytes(num_samples, vocab, hidden_size, cu_count);
}

extern "C" int ts_logits_int8(const void* hidden, int64_t hidden_stride, int64_t hidden_rows,
                              const int64_t* sample_indices, int32_t num_samples, const int8_t* wq,
                              const void* scale, int32_t scale_is_fp16, float* logits,
                              int64_t logits_stride, int32_t vocab, int32_t hidden_size,
                              void* workspace, size_t workspace_bytes, void* stream) {
  ts::clear_error();
  TS_REQUIRE(num_samples >= 0 && vocab > 0 && hidden_size > 0, TS_ERR_INVALID_ARG,
             "logits_int8: bad shape S=%d V=%d H=%d", num_samples, vocab, hidden_size);
  if (num_samples == 0) return TS_OK;
  TS_REQUIRE(hidden && sample_indices && wq && scale && logits && hidden_rows > 0,
             TS_ERR_INVALID_ARG, "logits_int8: null pointer argument or no hidden rows");
  TS_REQUIRE(hidden_size % 8 == 0, TS_ERR_UNSUPPORTED,
             "logits_int8: hidden_size=%d is not a multiple of 8", hidden_size);
  TS_REQUIRE(hidden_stride >= hidden_size && hidden_stride % 8 == 0 && aligned(hidden, 16) &&
                 aligned(wq, 8) && aligned(sample_indices, 8),
             TS_ERR_INVALID_ARG, "logits_int8: hidden must be 16-byte aligned rows, wq 8-byte aligned");
  TS_REQUIRE(logits_stride >= vocab && logits_stride % 4 == 0 && aligned(logits, 16),
             TS_ERR_INVALID_ARG, "logits_int8: logits rows must be 16-byte aligned (stride %% 4 == 0)");
  const GemmIo io{sample_indices, hidden_rows, logits, logits_stride, 0};
  const int st = w8a16_launch(static_cast<const half_t*>(hidden), hidden_stride, wq, scale,
                              scale_is_fp16, nullptr, nullptr, 0, num_samples, vocab, hidden_size,
                              workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream), io,
                              kVarAuto, 0);
  if (st != TS_OK) return st;
  return check_launch("logits_int8");
}

extern "C" size_t ts_w8a16_glu_workspace_bytes(int32_t M, int32_t intermediate, int32_t K,
                                               int32_t variant, int32_t splits, int32_t cu_count) {
  if (M <= 0 || intermediate <= 0 || K <= 0 || !variant_valid(variant, splits, M)) return 0;
  const int N = 2 * intermediate;
  return gemm_workspace(plan_gemm_v(M, N, K, cu_count > 0 ? cu_count : 256, variant, splits), M,
                        N);
}

extern "C" int ts_w8a16_glu(const void* x, int64_t ldx, const int8_t* wq, const void* scale,
                            int32_t scale_is_fp16, const void* bias, void* out, int64_t ldo,
                            int32_t M, int32_t intermediate, int32_t K, int32_t variant,
                            int32_t splits, void* workspace, size_t workspace_bytes, void* stream) {
  ts::clear_error();
  TS_REQUIRE(M >= 0 && intermediate > 0 && intermediate <= (1 << 29) && K > 0, TS_ERR_INVALID_ARG,
             "w8a16_glu: bad shape M=%d I=%d K=%d", M, intermediate, K);
  TS_REQUIRE(variant_valid(variant, splits, M < 1 ? 1 : M), TS_ERR_UNSUPPORTED,
             "w8a16_glu: variant %d with %d splits is not available for M=%d", variant, splits, M);
  if (M == 0) return TS_OK;
  TS_REQUIRE(x && wq && scale && out, TS_ERR_INVALID_ARG, "w8a16_glu: null pointer argument");
  TS_REQUIRE(K % 8 == 0, TS_ERR_UNSUPPORTED, "w8a16_glu: K=%d is not a multiple of 8", K);
  TS_REQUIRE(ldx >= K && ldx % 8 == 0 && aligned(x, 16) && aligned(wq, 8), TS_ERR_INVALID_ARG,
             "w8a16_glu: x must be 16-byte aligned rows (ldx %% 8 == 0), wq 8-byte aligned");
  TS_REQUIRE(ldo >= intermediate && !(ldo % 4) && aligned(out, 8), TS_ERR_INVALID_ARG,
             "w8a16_glu: out rows must be 8-byte aligned (ldo %% 4 == 0)");
  const GemmIo io{nullptr, 0, nullptr, 0, intermediate};
  const int st = w8a16_launch(static_cast<const half_t*>(x), ldx, wq, scale, scale_is_fp16,
                              static_cast<const half_t*>(bias), static_cast<half_t*>(out), ldo, M,
                              2 * intermediate, K, workspace, workspace_bytes,
                              reinterpret_cast<hipStream_t>(stream), io, variant, splits);
  if (st != TS_OK) return st;
  return check_launch("w8a16_glu");
}
