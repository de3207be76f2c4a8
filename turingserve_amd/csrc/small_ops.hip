// The per-layer elementwise ops around the attention / GEMM hot path, fused for gfx950
// (ops/triton_rmsnorm.py:10-46, ops/triton_rope.py:10-31, ops/triton_silu_mul.py:10-28; twins
// ops/reference.py:13-42). All three are HBM-bound row passes: one workgroup reads a token row
// once with 16-byte vector loads, computes in fp32 and writes the fp16 result once.
//
// Rounding follows the reference twins (HF numerics): the residual add is an fp32 add rounded to
// fp16; RMS is taken in fp32 over the rounded sum and the normalised row is rounded to fp16
// before the weight multiply; RoPE rounds the fp32 cos / sin tables to fp16 and rounds each
// product and each sum to fp16 like the twin's fp16 arithmetic (ops/reference.py:31-42; the
// Triton kernel keeps the products in fp32, which differs from the twin near cancellation);
// SiLU is computed in fp32 and rounded before the multiply by up.
#include <math.h>

#include "common.h"
#include "rmsnorm.h"
#include "rope.h"

namespace ts {

// One workgroup per token; the (H + KVH) rotated heads of the row are covered by 256 threads,
// each owning 4 consecutive frequency indices of one head (8-byte accesses of both halves).
__global__ void __launch_bounds__(kRowThreads) rope_kernel(
    half_t* __restrict__ qkv, int64_t qkv_st, const int64_t* __restrict__ positions,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int64_t max_pos,
    int heads, int D) {
  const int64_t t = blockIdx.x;
  const int half_d = D / 2, per_head = half_d / 4;
  int64_t pos = positions[t];
  pos = pos < 0 ? 0 : (pos >= max_pos ? max_pos - 1 : pos);
  const float* cp = cos_t + pos * half_d;
  const float* sp = sin_t + pos * half_d;
  for (int u = threadIdx.x; u < heads * per_head; u += kRowThreads) {
    const int h = u / per_head, i = (u % per_head) * 4;
    half_t* base = qkv + t * qkv_st + (int64_t)h * D;
    half4_t o1, o2;
    rope4(ld<half4_t>(base + i), ld<half4_t>(base + half_d + i), ld<float4_t>(cp + i),
          ld<float4_t>(sp + i), o1, o2);
    st<half4_t>(base + i, o1);
    st<half4_t>(base + half_d + i, o2);
  }
}

// RoPE and the cache write of one token row in one pass: the q and k heads are rotated in
// place as rope_kernel does, and when the token's slot lies in the cache the rotated k heads
// and the v heads are also written to K / V cache slot (block slot / 16, row slot % 16), as
// kv_write_kernel copies them. The row is read once and the rotated k is never re-read.
__global__ void __launch_bounds__(kRowThreads) rope_kv_write_kernel(
    half_t* __restrict__ qkv, int64_t qkv_st, const int64_t* __restrict__ positions,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int64_t max_pos, int H,
    int KVH, int D, half_t* __restrict__ kc, half_t* __restrict__ vc, int64_t num_slots,
    const int64_t* __restrict__ slots) {
  const int64_t t = blockIdx.x;
  const int half_d = D / 2, per_head = half_d / 4;
  int64_t pos = positions[t];
  pos = pos < 0 ? 0 : (pos >= max_pos ? max_pos - 1 : pos);
  const float* cp = cos_t + pos * half_d;
  const float* sp = sin_t + pos * half_d;
  const int64_t slot = slots[t];
  const bool cached = slot >= 0 && slot < num_slots;            // -1 = padding row
  const int64_t cache_row = ((slot >> 4) * KVH * kBlockSize + (slot & 15)) * D;  // + head * 16 D
  half_t* row = qkv + t * qkv_st;
  for (int u = threadIdx.x; u < (H + KVH) * per_head; u += kRowThreads) {
    const int h = u / per_head, i = (u % per_head) * 4;
    half_t* base = row + (int64_t)h * D;
    half4_t o1, o2;
    rope4(ld<half4_t>(base + i), ld<half4_t>(base + half_d + i), ld<float4_t>(cp + i),
          ld<float4_t>(sp + i), o1, o2);
    st<half4_t>(base + i, o1);
    st<half4_t>(base + half_d + i, o2);
    if (h >= H && cached) {
      half_t* dst = kc + cache_row + (int64_t)(h - H) * kBlockSize * D;
      st<half4_t>(dst + i, o1);
      st<half4_t>(dst + half_d + i, o2);
    }
  }
  if (!cached) return;
  const int pieces = D / kRowVec;
  const half_t* vrow = row + (int64_t)(H + KVH) * D;
  for (int u = threadIdx.x; u < KVH * pieces; u += kRowThreads) {
    const int kh = u / pieces, p = (u % pieces) * kRowVec;
    st<half8_t>(vc + cache_row + (int64_t)kh * kBlockSize * D + p,
                ld<half8_t>(vrow + (int64_t)kh * D + p));
  }
}

// gu = [gate | up] per row (I features each); grid (T, ceil(I / 2048)).
__global__ void __launch_bounds__(kRowThreads) silu_mul_kernel(
    const half_t* __restrict__ gu, int64_t gu_st, half_t* __restrict__ out, int64_t out_st,
    int I) {
  const int64_t t = blockIdx.x;
  const int i = (blockIdx.y * kRowThreads + threadIdx.x) * kRowVec;
  if (i >= I) return;
  const half8_t g = ld<half8_t>(gu + t * gu_st + i);
  const half8_t u = ld<half8_t>(gu + t * gu_st + I + i);
  half8_t o;
#pragma unroll
  for (int e = 0; e < kRowVec; ++e) {
    const float gf = (float)g[e];
    const half_t sl = (half_t)(gf / (1.f + expf(-gf)));           // silu in fp32, rounded
    o[e] = (half_t)((float)sl * (float)u[e]);
  }
  st<half8_t>(out + t * out_st + i, o);
}

}  // namespace ts

using namespace ts;

extern "C" int ts_rmsnorm(const void* x, int64_t x_stride, const void* residual,
                          int64_t residual_stride, const void* weight, void* out,
                          int64_t out_stride, void* residual_out, int64_t residual_out_stride,
                          int64_t num_tokens, int32_t hidden, float eps, void* stream) {
  ts::clear_error();
  TS_REQUIRE(num_tokens >= 0, TS_ERR_INVALID_ARG, "rmsnorm: num_tokens %lld < 0",
             (long long)num_tokens);
  if (num_tokens == 0) return TS_OK;
  TS_REQUIRE(x && weight && out && (!residual || residual_out), TS_ERR_INVALID_ARG,
             "rmsnorm: null pointer argument");
  TS_REQUIRE(hidden > 0 && hidden % kRowVec == 0 && hidden <= kRmsMaxIter * kRowThreads * kRowVec,
             TS_ERR_UNSUPPORTED, "rmsnorm: hidden %d must be a multiple of 8 and <= 8192", hidden);
  TS_REQUIRE(x_stride % kRowVec == 0 && out_stride % kRowVec == 0 &&
                 (!residual || (residual_stride % kRowVec == 0 && residual_out_stride % kRowVec == 0)) &&
                 aligned(x, 16) && aligned(out, 16) && aligned(weight, 16) &&
                 (!residual || (aligned(residual, 16) && aligned(residual_out, 16))),
             TS_ERR_INVALID_ARG, "rmsnorm: rows must be 16-byte aligned");
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const half_t* xp = static_cast<const half_t*>(x);
  const half_t* wp = static_cast<const half_t*>(weight);
  half_t* op = static_cast<half_t*>(out);
  if (residual) {
    rmsnorm_kernel<true><<<dim3((unsigned)num_tokens), kRowThreads, 0, s>>>(
        xp, x_stride, static_cast<const half_t*>(residual), residual_stride, wp, op, out_stride,
        static_cast<half_t*>(residual_out), residual_out_stride, hidden, eps);
  } else {
    rmsnorm_kernel<false><<<dim3((unsigned)num_tokens), kRowThreads, 0, s>>>(
        xp, x_stride, nullptr, 0, wp, op, out_stride, nullptr, 0, hidden, eps);
  }
  return check_launch("rmsnorm");
}

extern "C" int ts_rope(void* qkv, int64_t qkv_stride, const int64_t* positions,
                       const float* cos_table, const float* sin_table, int64_t max_position,
                       int64_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
                       int32_t head_dim, void* stream) {
  ts::clear_error();
  TS_REQUIRE(num_tokens >= 0, TS_ERR_INVALID_ARG, "rope: num_tokens %lld < 0", (long long)num_tokens);
  if (num_tokens == 0) return TS_OK;
  TS_REQUIRE(qkv && positions && cos_table && sin_table && max_position > 0, TS_ERR_INVALID_ARG,
             "rope: null pointer or empty table");
  TS_REQUIRE(num_heads > 0 && num_kv_heads > 0, TS_ERR_INVALID_ARG, "rope: bad head counts");
  TS_REQUIRE(head_dim % 8 == 0 && head_dim >= 8, TS_ERR_UNSUPPORTED,
             "rope: head_dim %d must be a multiple of 8", head_dim);
  TS_REQUIRE(qkv_stride % 4 == 0 && aligned(qkv, 8) && aligned(cos_table, 16) &&
                 aligned(sin_table, 16),
             TS_ERR_INVALID_ARG, "rope: misaligned qkv rows or tables");
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  rope_kernel<<<dim3((unsigned)num_tokens), kRowThreads, 0, s>>>(
      static_cast<half_t*>(qkv), qkv_stride, positions, cos_table, sin_table, max_position,
      num_heads + num_kv_heads, head_dim);
  return check_launch("rope");
}

extern "C" int ts_rope_kv_write(void* qkv, int64_t qkv_stride, const int64_t* positions,
                                const float* cos_table, const float* sin_table,
                                int64_t max_position, int64_t num_tokens, int32_t num_heads,
                                int32_t num_kv_heads, int32_t head_dim, void* k_cache,
                                void* v_cache, int64_t num_blocks, const int64_t* slot_mapping,
                                void* stream) {
  ts::clear_error();
  TS_REQUIRE(num_tokens >= 0, TS_ERR_INVALID_ARG, "rope_kv_write: num_tokens %lld < 0",
             (long long)num_tokens);
  if (num_tokens == 0) return TS_OK;
  TS_REQUIRE(qkv && positions && cos_table && sin_table && max_position > 0 && k_cache &&
                 v_cache && slot_mapping && num_blocks > 0,
             TS_ERR_INVALID_ARG, "rope_kv_write: null pointer, empty table or empty cache");
  TS_REQUIRE(num_heads > 0 && num_kv_heads > 0, TS_ERR_INVALID_ARG, "rope_kv_write: bad head counts");
  TS_REQUIRE(head_dim % 8 == 0 && head_dim >= 8, TS_ERR_UNSUPPORTED,
             "rope_kv_write: head_dim %d must be a multiple of 8", head_dim);
  TS_REQUIRE(qkv_stride >= (int64_t)(num_heads + 2 * num_kv_heads) * head_dim &&
                 qkv_stride % 8 == 0 && aligned(qkv, 16) && aligned(k_cache, 16) &&
                 aligned(v_cache, 16) && aligned(cos_table, 16) && aligned(sin_table, 16),
             TS_ERR_INVALID_ARG, "rope_kv_write: qkv rows, caches and tables must be 16-byte aligned");
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  rope_kv_write_kernel<<<dim3((unsigned)num_tokens), kRowThreads, 0, s>>>(
      static_cast<half_t*>(qkv), qkv_stride, positions, cos_table, sin_table, max_position,
      num_heads, num_kv_heads, head_dim, static_cast<half_t*>(k_cache),
      static_cast<half_t*>(v_cache), num_blocks * kBlockSize, slot_mapping);
  return check_launch("rope_kv_write");
}

extern "C" int ts_silu_mul(const void* gu, int64_t gu_stride, void* out, int64_t out_stride,
                           int64_t num_tokens, int32_t intermediate, void* stream) {
  ts::clear_error();
  TS_REQUIRE(num_tokens >= 0, TS_ERR_INVALID_ARG, "silu_mul: num_tokens %lld < 0",
             (long long)num_tokens);
  if (num_tokens == 0) return TS_OK;
  TS_REQUIRE(gu && out, TS_ERR_INVALID_ARG, "silu_mul: null pointer argument");
  TS_REQUIRE(intermediate > 0 && intermediate % kRowVec == 0, TS_ERR_UNSUPPORTED,
             "silu_mul: intermediate %d must be a multiple of 8", intermediate);
  TS_REQUIRE(gu_stride % kRowVec == 0 && out_stride % kRowVec == 0 && aligned(gu, 16) &&
                 aligned(out, 16),
             TS_ERR_INVALID_ARG, "silu_mul: rows must be 16-byte aligned");
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const unsigned gy = (unsigned)((intermediate + kRowThreads * kRowVec - 1) / (kRowThreads * kRowVec));
  silu_mul_kernel<<<dim3((unsigned)num_tokens, gy), kRowThreads, 0, s>>>(
      static_cast<const half_t*>(gu), gu_stride, static_cast<half_t*>(out), out_stride,
      intermediate);
  return check_launch("silu_mul");
}
