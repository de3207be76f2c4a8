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

// Token-packed A operand of O^T tile t over a pair of blocks (a, b): lane (c, g) gets tokens
// 4g .. 4g+3 of each block for dim VW c' + t, taken from the coalesced V rows (two byte permutes
// per block). Blocks with tokens at or past tok_hi are masked when `tail_*` is set.
template <int VW, typename VRow>
__device__ __forceinline__ half8_t vt_operand(const VRow (&va)[4], const VRow (&vb)[4], int t,
                                              bool tail_a, bool tail_b, int ta, int tb, int tok_hi) {
  half4_t x = {va[0][t], va[1][t], va[2][t], va[3][t]};
  half4_t y = {vb[0][t], vb[1][t], vb[2][t], vb[3][t]};
  if (tail_a) x = mask_tokens(x, ta, tok_hi);
  if (tail_b) y = mask_tokens(y, tb, tok_hi);
  return {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
}

// Online softmax with a lazy reference point (in scaled log2 units). A row's reference m moves
// only when a new score exceeds it by more than kRescaleLog2, so P = 2^(s - m) <= 2^8 stays well
// inside fp16 (with the same relative rounding as P <= 1) and the O accumulators are rescaled a
// few times per row instead of at every new maximum. O / l does not depend on the reference
// point, and merges weight each partial by 2^(m_i - max m), which is exact for any reference.
constexpr float kRescaleLog2 = 8.f;

// One step over 32 keys (a pair of 16-token blocks) for the 16 rows of a wavefront: sa / sb are
// the raw S^T tiles (lane (c, g): keys 4g + r of row c; masked keys already -inf) and
// sl2 = scale * log2(e) > 0. Updates the row's reference m and this lane's partial sum l and
// returns P^T rounded to fp16 (the B operand of v_mfma_f32_16x16x32_f16: keys 4g .. 4g+3 of
// block a, then of block b) with the factor alpha the O^T accumulators must be scaled by first
// when `rescale` is set (alpha is 1 for rows whose reference did not move, 0 on a row's first
// visible key, where O is still 0).
struct SoftmaxStep {
  half8_t p;
  float alpha;
  bool rescale;
};

__device__ __forceinline__ SoftmaxStep softmax_pair(const float4_t& sa, const float4_t& sb,
                                                    float sl2, float& m, float& l) {
  const float raw = vmax(vmax(vmax(sa[0], sa[1]), vmax(sa[2], sa[3])),
                         vmax(vmax(sb[0], sb[1]), vmax(sb[2], sb[3])));
  const float bm = rows_max(raw) * sl2;            // -inf when every key of the row is masked
  const bool move = bm > m + kRescaleLog2;         // m = -inf: the first visible key moves it
  SoftmaxStep st;
  st.rescale = __ballot(move) != 0;
  st.alpha = 1.f;
  if (st.rescale) {
    st.alpha = move ? fast_exp2(m - bm) : 1.f;     // m = -inf -> 0
    l *= st.alpha;
    m = move ? bm : m;
  }
  const float neg = m == -INFINITY ? 0.f : -m;     // rows with no visible key: every P is 0
  float p[8];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    p[r] = fast_exp2(fmaf(sa[r], sl2, neg));
    p[4 + r] = fast_exp2(fmaf(sb[r], sl2, neg));
  }
  l += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
  st.p = {(half_t)p[0], (half_t)p[1], (half_t)p[2], (half_t)p[3],
          (half_t)p[4], (half_t)p[5], (half_t)p[6], (half_t)p[7]};
  return st;
}

// O^T = alpha O^T + V^T . P^T over the pair for all TILES tiles. The scaling is unconditional
// (alpha is exactly 1 unless a reference point moved, so the result is the same as skipping it):
// a conditional multiply before the MFMAs left two accumulator sets live across the branch.
template <int TILES, typename VOperand>
__device__ __forceinline__ void pv_update(float4_t (&o)[TILES], const SoftmaxStep& st,
                                          VOperand vt) {
#pragma unroll
  for (int t = 0; t < TILES; ++t) o[t] = mfma16x16x32(vt(t), st.p, o[t] * st.alpha);
}

}  // namespace ts
