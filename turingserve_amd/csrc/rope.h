// Rotate-half RoPE arithmetic shared by the RoPE kernels and the decode kernel that rotates q
// and the new k itself (ops/triton_rope.py:10-25, twin ops/reference.py:31-42), so that every
// path rounds exactly alike.
#pragma once

#include "common.h"

namespace ts {

// Rotate-half RoPE of 4 consecutive frequency indices: x1 from the first half of the head, x2
// from the second, c4 / s4 the fp32 table entries.
__device__ __forceinline__ void rope4(half4_t x1, half4_t x2, float4_t c4, float4_t s4,
                                      half4_t& o1, half4_t& o2) {
  // Each product must round to fp16 before the sum, as in the twin: no fused multiply-add.
#pragma clang fp contract(off)
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    // fp16 x fp16 products are exact in fp32, so each rounds once to fp16, as the twin's
    // fp16 multiplies do; the sum of two fp16 values then rounds once more.
    const float c = (float)(half_t)c4[e], s = (float)(half_t)s4[e];
    const float a = (float)x1[e], b = (float)x2[e];
    o1[e] = (half_t)((float)(half_t)(a * c) - (float)(half_t)(b * s));
    o2[e] = (half_t)((float)(half_t)(b * c) + (float)(half_t)(a * s));
  }
}

// Clamped table row of a position (positions outside [0, max_pos) use the nearest row).
__device__ __forceinline__ int64_t rope_row(int64_t pos, int64_t max_pos) {
  return pos < 0 ? 0 : (pos >= max_pos ? max_pos - 1 : pos);
}

}  // namespace ts
