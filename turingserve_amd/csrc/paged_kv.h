// Loading paged K/V blocks straight into MFMA operand registers (shared by the decode and
// prefill kernels). One 16-token block of one KV head is 16 x D fp16, contiguous.
#pragma once

#include "common.h"

namespace ts {

template <int D>
struct KvRegs {
  // D >= 32: KK 16-byte pieces of K per lane; D == 16: one 8-byte piece.
  static constexpr int KK = D >= 32 ? D / 32 : 1;
  // V: each lane holds VW consecutive dims of 4 tokens; O^T is split into VW tiles of 16 dims.
  static constexpr int VW = D / 16;
  static constexpr int TILES = VW;
};

// K rows in their natural layout: lane (c, g) gets K[tok c][32kk + 8g .. +7] (16-byte loads).
template <int D>
__device__ __forceinline__ void load_k_block(const half_t* __restrict__ base, int c, int g,
                                             half8_t (&x)[KvRegs<D>::KK]) {
  if constexpr (D >= 32) {
#pragma unroll
    for (int kk = 0; kk < KvRegs<D>::KK; ++kk) x[kk] = ld<half8_t>(base + c * D + 32 * kk + 8 * g);
  } else {
    const half4_t t = ld<half4_t>(base + c * D + 4 * g);
    x[0] = {t[0], t[1], t[2], t[3], 0, 0, 0, 0};
  }
}

// Packed fp16 vector of VW elements (registers hold two halves each; VW = 1 uses a pair).
template <int VW>
struct HalfVec {
  typedef _Float16 type __attribute__((ext_vector_type(VW)));
};
template <>
struct HalfVec<1> {
  typedef half2_t type;
};

// V rows in their natural layout: lane (c, g) loads V[tok 4g + r][VW c .. VW c + VW-1] for
// r = 0..3 (16 lanes cover one whole token row, so every load is fully coalesced). Tile q of
// O^T then uses dims {VW i + q : i = 0..15}: its token-packed A operand for lane (c, g) is
// {x[0][q], x[1][q], x[2][q], x[3][q]}, two byte permutes and no transpose product.
template <int D>
__device__ __forceinline__ void load_v_rows(const half_t* __restrict__ base, int c, int g,
                                            typename HalfVec<KvRegs<D>::VW>::type (&x)[4]) {
  constexpr int VW = KvRegs<D>::VW;
  typedef typename HalfVec<VW>::type V;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const half_t* p = base + (4 * g + r) * D + VW * c;
    if constexpr (VW == 1) {
      x[r] = half2_t{p[0], (half_t)0.f};
    } else {
      x[r] = ld<V>(p);
    }
  }
}

// Tokens 4g .. 4g+3 of a V^T operand at or past seq_len are zeroed: a reused block may hold
// anything there, and 0 * NaN would reach the output.
__device__ __forceinline__ half4_t mask_tokens(half4_t v, int tok0, int seq_len) {
#pragma unroll
  for (int r = 0; r < 4; ++r) v[r] = (tok0 + r < seq_len) ? v[r] : (half_t)0.f;
  return v;
}

}  // namespace ts
