// Paged chunked-prefill attention for gfx950 (ops/triton_prefill_attention.py:17-79).
//
// Query row i of prefill sequence b sits at absolute position prefix + i with
// prefix = seq_len - q_len and attends to keys j <= prefix + i, j < seq_len (bottom-right
// causal mask, ops/reference.py:60-77). Online softmax in fp32; P is rounded to fp16 before
// the P.V product (ops/triton_prefill_attention.py:57).
//
// Workgroup = 32 query rows of one query head and four wavefronts. Every wavefront holds Q^T of
// all 32 rows (two 16-row column groups) in registers and reads 16-token K/V blocks straight
// from the paged cache into MFMA operand registers, the way the decode kernel does (K in its
// natural layout, V as coalesced rows permuted in registers); the wavefronts take the pairs of
// blocks round-robin, each keeping its next pair in flight while it multiplies the current one:
//   S^T[32 keys][16 rows] = K . Q^T        two v_mfma_f32_16x16x32_f16 chains per row group
//   O^T[D][16 rows]     += V^T . P^T      v_mfma_f32_16x16x32_f16 over the 32 keys of the pair
// so every per-row softmax statistic sits in lane column c = lane % 16 (see common.h). The four
// partial (m, l, O) states of a row are merged in LDS at the end, so a short chunk on a long
// prefix still spreads over the whole device without global partials. Pairs past the tile's
// causal limit are never loaded; workgroups are launched longest-first.
#include <math.h>

#include "common.h"
#include "paged_kv.h"

namespace ts {

constexpr float kLog2eP = 1.4426950408889634f;

#ifndef TS_PREFILL_ROW_GROUPS
#define TS_PREFILL_ROW_GROUPS 2
#endif
constexpr int kPsRows = 16 * TS_PREFILL_ROW_GROUPS;   // query rows per workgroup and wavefront
constexpr int kPsWaves = 4;

template <int D, int NW>
__global__ void __launch_bounds__(NW * 64) prefill_stream_kernel(
    const half_t* __restrict__ q, int64_t q_st, int64_t q_sh, half_t* __restrict__ out,
    int64_t o_st, int64_t num_tokens, const half_t* __restrict__ kc,
    const half_t* __restrict__ vc, int64_t NB, const int* __restrict__ bt, int64_t bt_st,
    int max_blocks, const int* __restrict__ seq_lens, const int* __restrict__ qsl,
    int num_decode, int H, int KVH, float sl2) {
  constexpr int KK = KvRegs<D>::KK, VW = KvRegs<D>::VW, TILES = KvRegs<D>::TILES;
  constexpr int RG = kPsRows / 16;
  constexpr int OROW = D + 4;
  __shared__ float s_o[NW][kPsRows][OROW];
  __shared__ float s_m[NW][kPsRows];
  __shared__ float s_l[NW][kPsRows];

  const int mtile = gridDim.x - 1 - blockIdx.x;       // longest (last) row tiles first
  const int b = num_decode + blockIdx.y;
  const int h = blockIdx.z;
  const int G = H / KVH, kvh = h / G;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: keeps loops scalar
  const int c = lane & 15, g = lane >> 4;

  const int q_start = __builtin_amdgcn_readfirstlane(qsl[b]);
  int q_len = __builtin_amdgcn_readfirstlane(qsl[b + 1]) - q_start;
  if (q_start < 0 || q_len < 0 || (int64_t)q_start + q_len > num_tokens) q_len = 0;  // bad metadata
  int seq_len = __builtin_amdgcn_readfirstlane(seq_lens[b]);
  seq_len = seq_len < 0 ? 0 : (seq_len > max_blocks * kBlockSize ? max_blocks * kBlockSize : seq_len);
  const int m0 = mtile * kPsRows;
  if (m0 >= q_len) return;
  const int prefix = seq_len - q_len;
  const int last_row = (m0 + kPsRows < q_len ? m0 + kPsRows : q_len) - 1;
  int kv_hi = prefix + last_row + 1;                   // keys any row of this tile may see
  kv_hi = kv_hi < seq_len ? kv_hi : seq_len;
  const int nblk = (kv_hi + kBlockSize - 1) / kBlockSize;
  const int npairs = (nblk + 1) / 2;

  // Q^T operands: lane (c, g) of group rg is row m0 + 16 rg + c (zeros past q_len).
  half8_t qf[RG][KK];
  int lim[RG];                                         // last key each lane's row may see
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    const int row = m0 + 16 * rg + c;
    const bool ok = row < q_len;
    lim[rg] = ok ? prefix + row : -1;
    const half_t* qp = q + (int64_t)(q_start + (ok ? row : 0)) * q_st + (int64_t)h * q_sh;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if constexpr (D >= 32) {
        qf[rg][kk] = ok ? ld<half8_t>(qp + 32 * kk + 8 * g) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
      } else {
        const half4_t t = ok ? ld<half4_t>(qp + 4 * g) : half4_t{0, 0, 0, 0};
        qf[rg][kk] = {t[0], t[1], t[2], t[3], 0, 0, 0, 0};
      }
    }
  }
  const float4_t zero4 = {0.f, 0.f, 0.f, 0.f};
  float4_t o[RG][TILES];
  float m[RG], l[RG];
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    m[rg] = -INFINITY;
    l[rg] = 0.f;
#pragma unroll
    for (int t = 0; t < TILES; ++t) o[rg][t] = zero4;
  }

  const int* btrow = bt + (int64_t)b * bt_st;
  const int64_t head_off = (int64_t)kvh * kBlockSize * D;
  const int64_t blk_stride = (int64_t)KVH * kBlockSize * D;
  // A pair index past the end re-reads the last block (a cache hit); its keys are masked.
  typedef typename HalfVec<VW>::type VRow;
  auto load_pair = [&](int pi, half8_t (&kf)[2][KK], VRow (&vr)[2][4]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      int bi = 2 * pi + j;
      bi = bi < nblk ? bi : nblk - 1;
      const int64_t off = clamp_block(btrow[bi], NB) * blk_stride + head_off;
      load_k_block<D>(kc + off, c, g, kf[j]);
      load_v_rows<D>(vc + off, c, g, vr[j]);
    }
  };
  auto compute_pair = [&](int pi, const half8_t (&kf)[2][KK], const VRow (&vr)[2][4]) {
    const int ta = 2 * pi * kBlockSize + 4 * g, tb = ta + kBlockSize;
    const bool tail_a = (2 * pi + 1) * kBlockSize > kv_hi;
    const bool tail_b = (2 * pi + 2) * kBlockSize > kv_hi;
    half8_t v8[TILES];                                    // V^T operands of the pair
#pragma unroll
    for (int t = 0; t < TILES; ++t) v8[t] = vt_operand<VW>(vr[0], vr[1], t, tail_a, tail_b, ta, tb, kv_hi);
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
      float4_t sa = zero4, sb = zero4;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        if constexpr (D >= 32) {
          sa = mfma16x16x32(kf[0][kk], qf[rg][kk], sa);
          sb = mfma16x16x32(kf[1][kk], qf[rg][kk], sb);
        } else {
          sa = mfma16x16x16(lo4(kf[0][kk]), lo4(qf[rg][kk]), sa);
          sb = mfma16x16x16(lo4(kf[1][kk]), lo4(qf[rg][kk]), sb);
        }
      }
      // Interior pair: every row of the group sees all 32 keys (rows past q_len are discarded),
      // so no key needs masking.
      const int last_key = (2 * pi + 2) * kBlockSize - 1;
      const bool interior = last_key < kv_hi && last_key <= prefix + m0 + 16 * rg;
      if (!interior) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sa[r] = (ta + r < kv_hi && ta + r <= lim[rg]) ? sa[r] : -INFINITY;
          sb[r] = (tb + r < kv_hi && tb + r <= lim[rg]) ? sb[r] : -INFINITY;
        }
      }
      const SoftmaxStep step = softmax_pair(sa, sb, sl2, m[rg], l[rg]);
      // lane (c, g) of tile t: dims VW (4g + r) + t
      pv_update<TILES>(o[rg], step, [&](int t) { return v8[t]; });
    }
  };
  // Two-deep register ring: the loads of pair p + NW are issued before pair p is computed.
  half8_t k0[2][KK], k1[2][KK];
  VRow v0[2][4], v1[2][4];
  int p = w;
  if (p < npairs) load_pair(p, k0, v0);
  for (; p < npairs; p += 2 * NW) {
    if (p + NW < npairs) load_pair(p + NW, k1, v1);
    compute_pair(p, k0, v0);
    if (p + NW >= npairs) break;
    if (p + 2 * NW < npairs) load_pair(p + 2 * NW, k0, v0);
    compute_pair(p + NW, k1, v1);
  }

  // Merge the NW wavefronts' partial softmax states for the 32 rows in LDS.
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    const float lt = rows_sum(l[rg]);
    if (g == 0) {
      s_m[w][16 * rg + c] = m[rg];
      s_l[w][16 * rg + c] = lt;
    }
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) s_o[w][16 * rg + c][VW * (4 * g + r) + t] = o[rg][t][r];
  }
  __syncthreads();
  for (int e = tid; e < kPsRows * D; e += NW * 64) {
    const int rr = e / D, d = e % D;
    const int row = m0 + rr;
    if (row >= q_len) continue;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, s_m[ww][rr]);
    const float Mr = M == -INFINITY ? 0.f : M;
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float wt = fast_exp2(s_m[ww][rr] - Mr);      // idle wavefront: m = -inf -> 0
      L += wt * s_l[ww][rr];
      O += wt * s_o[ww][rr][d];
    }
    out[(int64_t)(q_start + row) * o_st + (int64_t)h * D + d] = (half_t)(L == 0.f ? 0.f : O / L);
  }
}

}  // namespace ts

using namespace ts;

extern "C" int ts_prefill_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                    void* out, int64_t out_stride_t, int64_t num_tokens,
                                    const void* k_cache, const void* v_cache, int64_t num_blocks,
                                    const int32_t* block_tables, int64_t bt_stride,
                                    int32_t max_blocks_per_seq, const int32_t* seq_lens,
                                    const int32_t* query_start_loc, int32_t num_seqs,
                                    int32_t num_decode, int32_t max_query_len, int32_t num_heads,
                                    int32_t num_kv_heads, int32_t head_dim, float scale,
                                    void* stream) {
  TS_REQUIRE(num_seqs >= 0 && num_decode >= 0 && num_decode <= num_seqs, TS_ERR_INVALID_ARG,
             "prefill_attention: num_decode=%d num_seqs=%d", num_decode, num_seqs);
  const int P = num_seqs - num_decode;
  if (P == 0 || max_query_len <= 0) return TS_OK;
  TS_REQUIRE(q && out && k_cache && v_cache && block_tables && seq_lens && query_start_loc,
             TS_ERR_INVALID_ARG, "prefill_attention: null pointer argument");
  TS_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
             TS_ERR_INVALID_ARG, "prefill_attention: num_heads=%d not a multiple of num_kv_heads=%d",
             num_heads, num_kv_heads);
  TS_REQUIRE(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128,
             TS_ERR_UNSUPPORTED, "prefill_attention: head_dim %d not in {16, 32, 64, 128}", head_dim);
  TS_REQUIRE(num_blocks > 0 && max_blocks_per_seq > 0 && bt_stride >= max_blocks_per_seq,
             TS_ERR_INVALID_ARG, "prefill_attention: bad block table");
  TS_REQUIRE(num_tokens > 0, TS_ERR_INVALID_ARG, "prefill_attention: num_tokens %lld",
             (long long)num_tokens);
  const int vec = head_dim >= 32 ? 8 : 4;
  TS_REQUIRE(q_stride_t % vec == 0 && q_stride_h % vec == 0 && out_stride_t % 4 == 0 &&
                 aligned(q, 2 * vec) && aligned(out, 8) && aligned(k_cache, 16) &&
                 aligned(v_cache, 16),
             TS_ERR_INVALID_ARG, "prefill_attention: misaligned q / out / caches");
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((max_query_len + kPsRows - 1) / kPsRows, P, num_heads);
  const float sl2 = scale * kLog2eP;
#define TS_PF_CASE(DD)                                                                            \
  case DD:                                                                                        \
    prefill_stream_kernel<DD, kPsWaves><<<grid, kPsWaves * 64, 0, s>>>(                           \
        static_cast<const half_t*>(q), q_stride_t, q_stride_h, static_cast<half_t*>(out),        \
        out_stride_t, num_tokens, static_cast<const half_t*>(k_cache),                           \
        static_cast<const half_t*>(v_cache), num_blocks, block_tables, bt_stride,                \
        max_blocks_per_seq, seq_lens, query_start_loc, num_decode, num_heads, num_kv_heads, sl2); \
    break;
  switch (head_dim) {
    TS_PF_CASE(16)
    TS_PF_CASE(32)
    TS_PF_CASE(64)
    TS_PF_CASE(128)
  }
#undef TS_PF_CASE
  return check_launch("prefill_attention");
}
