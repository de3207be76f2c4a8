// RMSNorm of one token row with the residual add, shared by the standalone norm launch
// (small_ops.hip) and the W8A16 split-K epilogue that feeds it (w8a16.hip), so that both compute
// the same values with the same instructions (ops/triton_rmsnorm.py:10-46, twin
// ops/reference.py:13-22): the residual add is an fp32 add rounded to fp16; RMS is taken in fp32
// over the rounded sum and the normalised row is rounded to fp16 before the weight multiply.
#pragma once

#include "common.h"

namespace ts {

constexpr int kRowThreads = 256;
constexpr int kRowVec = 8;                 // halves per 16-byte access
constexpr int kRmsMaxIter = 4;             // N <= 4 * 256 * 8 = 8192

__device__ __forceinline__ float block_sum_256(float v, float* s_red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) s_red[w] = v;
  __syncthreads();
  return (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
}

// One row of N features by a workgroup of kRowThreads threads. load_x(i) returns features
// i .. i+7 of the row's input; with kRes, res is added and the sum written to res_out.
template <bool kRes, class LoadX>
__device__ __forceinline__ void rmsnorm_row(LoadX load_x, const half_t* __restrict__ res,
                                            const half_t* __restrict__ w, half_t* __restrict__ out,
                                            half_t* __restrict__ res_out, int N, float eps) {
  __shared__ float s_red[kRowThreads / kWave];
  const int tid = threadIdx.x;
  half8_t v[kRmsMaxIter];
  float ss = 0.f;
#pragma unroll
  for (int it = 0; it < kRmsMaxIter; ++it) {
    const int i = (it * kRowThreads + tid) * kRowVec;
    if (i < N) {
      half8_t a = load_x(i);
      if constexpr (kRes) {
        const half8_t b = ld<half8_t>(res + i);
#pragma unroll
        for (int e = 0; e < kRowVec; ++e) a[e] = (half_t)((float)a[e] + (float)b[e]);
        st<half8_t>(res_out + i, a);
      }
      v[it] = a;
#pragma unroll
      for (int e = 0; e < kRowVec; ++e) ss += (float)a[e] * (float)a[e];
    }
  }
  const float inv = rsqrtf(block_sum_256(ss, s_red) / (float)N + eps);
#pragma unroll
  for (int it = 0; it < kRmsMaxIter; ++it) {
    const int i = (it * kRowThreads + tid) * kRowVec;
    if (i < N) {
      const half8_t wv = ld<half8_t>(w + i);
      half8_t o;
#pragma unroll
      for (int e = 0; e < kRowVec; ++e) {
        const half_t y = (half_t)((float)v[it][e] * inv);          // cast before the weight
        o[e] = (half_t)((float)wv[e] * (float)y);
      }
      st<half8_t>(out + i, o);
    }
  }
}

// One workgroup per token row of N = hidden features.
template <bool kRes>
__global__ void __launch_bounds__(kRowThreads) rmsnorm_kernel(
    const half_t* __restrict__ x, int64_t x_st, const half_t* __restrict__ res, int64_t res_st,
    const half_t* __restrict__ w, half_t* __restrict__ out, int64_t out_st,
    half_t* __restrict__ res_out, int64_t res_out_st, int N, float eps) {
  const int64_t t = blockIdx.x;
  const half_t* xr = x + t * x_st;
  rmsnorm_row<kRes>([&](int i) { return ld<half8_t>(xr + i); }, kRes ? res + t * res_st : nullptr,
                    w, out + t * out_st, kRes ? res_out + t * res_out_st : nullptr, N, eps);
}

}  // namespace ts
