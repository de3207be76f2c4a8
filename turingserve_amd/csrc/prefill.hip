// Paged chunked-prefill attention for gfx950 (ops/triton_prefill_attention.py:17-79).
//
// Query row i of prefill sequence b sits at absolute position prefix + i with
// prefix = seq_len - q_len and attends to keys j <= prefix + i, j < seq_len (bottom-right
// causal mask, ops/reference.py:60-77). Online softmax in fp32; P is rounded to fp16 before
// the P.V product (ops/triton_prefill_attention.py:57).
//
// Workgroup = BM = 64 query rows of one query head, four wavefronts of 16 rows each.
// Per key tile of BN = 64 keys the workgroup stages K[BN][D] (row-major) and V^T[D][BN]
// (transposed while storing: two keys packed per 4-byte LDS write) in LDS, gathered through
// the block table. Each wavefront then computes
//   S^T[64 keys][16 rows] = K . Q^T        v_mfma_f32_16x16x32_f16, Q^T kept in registers
//   O^T[D][16 rows]     += V^T . P^T      v_mfma_f32_16x16x32_f16, P^T straight from S^T
// so every per-row softmax statistic sits in lane column c = lane % 16 (see common.h).
// Tiles past a wavefront's causal limit are skipped; workgroups are launched longest-first.
#include <math.h>

#include "common.h"
#include "paged_kv.h"

namespace ts {

constexpr float kLog2eP = 1.4426950408889634f;
constexpr int kPfBM = 64;
constexpr int kPfBN = 64;
constexpr int kPfWaves = 4;

template <int D>
__global__ void __launch_bounds__(kPfWaves * 64) prefill_kernel(
    const half_t* __restrict__ q, int64_t q_st, int64_t q_sh, half_t* __restrict__ out,
    int64_t o_st, int64_t num_tokens, const half_t* __restrict__ kc,
    const half_t* __restrict__ vc, int64_t NB, const int* __restrict__ bt, int64_t bt_st,
    int max_blocks, const int* __restrict__ seq_lens, const int* __restrict__ qsl,
    int num_decode, int H, int KVH, float scale_log2) {
  constexpr int KP = D + 8;          // padded K row (halfs)
  constexpr int VP = kPfBN + 8;      // padded V^T row (halfs)
  constexpr int KK = D >= 32 ? D / 32 : 1;
  constexpr int TILES = D / 16;
  constexpr int NT = kPfBN / 16;     // 16-key sub-tiles per key tile
  __shared__ half_t s_k[kPfBN][KP];
  __shared__ half_t s_vt[D][VP];

  const int mtile = gridDim.x - 1 - blockIdx.x;       // longest (last) query tiles first
  const int b = num_decode + blockIdx.y;
  const int h = blockIdx.z;
  const int G = H / KVH, kvh = h / G;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int c = lane & 15, g = lane >> 4;

  const int q_start = qsl[b];
  int q_len = qsl[b + 1] - q_start;
  if (q_start < 0 || q_len < 0 || (int64_t)q_start + q_len > num_tokens) q_len = 0;  // bad metadata
  int seq_len = seq_lens[b];
  seq_len = seq_len < 0 ? 0 : (seq_len > max_blocks * kBlockSize ? max_blocks * kBlockSize : seq_len);
  const int m0 = mtile * kPfBM;
  if (m0 >= q_len) return;
  const int prefix = seq_len - q_len;
  const int last_row = (m0 + kPfBM < q_len ? m0 + kPfBM : q_len) - 1;
  int kv_hi = prefix + last_row + 1;
  kv_hi = kv_hi < seq_len ? kv_hi : seq_len;

  // This wavefront's rows and their Q^T operand (lane (c, g): row c, dims 32kk + 8g .. +7).
  const int row = m0 + 16 * w + c;
  const bool row_ok = row < q_len;
  const int w_last = (m0 + 16 * w + 15 < q_len ? m0 + 16 * w + 15 : q_len - 1);
  const int w_kv_hi = prefix + w_last + 1;            // keys this wavefront can see
  half8_t qf[KK];
  {
    const half_t* qp = q + (int64_t)(q_start + (row_ok ? row : 0)) * q_st + (int64_t)h * q_sh;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if constexpr (D >= 32) {
        qf[kk] = row_ok ? ld<half8_t>(qp + 32 * kk + 8 * g) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
      } else {
        const half4_t t = row_ok ? ld<half4_t>(qp + 4 * g) : half4_t{0, 0, 0, 0};
        qf[kk] = {t[0], t[1], t[2], t[3], 0, 0, 0, 0};
      }
    }
  }
  float4_t o[TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t) o[t] = {0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const int abs_row = prefix + row;                    // last key this row may see
  const int* btrow = bt + (int64_t)b * bt_st;
  const int64_t head_off = (int64_t)kvh * kBlockSize * D;
  const int64_t blk_stride = (int64_t)KVH * kBlockSize * D;

  for (int j0 = 0; j0 < kv_hi; j0 += kPfBN) {
    // ---- stage K (row-major) and V^T into LDS; keys >= seq_len are zero-filled ----
    constexpr int KCH = D / 8;                          // 16-byte chunks per key row
    for (int u = tid; u < kPfBN * KCH; u += kPfWaves * 64) {
      const int kr = u / KCH, cc = u % KCH;
      const int j = j0 + kr;
      half8_t val = {0, 0, 0, 0, 0, 0, 0, 0};
      if (j < seq_len) {
        const int64_t off = clamp_block(btrow[j >> 4], NB) * blk_stride + head_off +
                            (int64_t)(j & 15) * D + 8 * cc;
        val = ld<half8_t>(kc + off);
      }
      st<half8_t>(&s_k[kr][8 * cc], val);
    }
    for (int u = tid; u < (kPfBN / 2) * KCH; u += kPfWaves * 64) {
      const int cc = u / (kPfBN / 2), kp = u % (kPfBN / 2);
      const int j = j0 + 2 * kp;                       // keys j, j + 1 share a KV block
      half8_t v0 = {0, 0, 0, 0, 0, 0, 0, 0}, v1 = v0;
      if (j < seq_len) {
        const int64_t off = clamp_block(btrow[j >> 4], NB) * blk_stride + head_off +
                            (int64_t)(j & 15) * D + 8 * cc;
        v0 = ld<half8_t>(vc + off);
        if (j + 1 < seq_len) v1 = ld<half8_t>(vc + off + D);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) st<half2_t>(&s_vt[8 * cc + e][2 * kp], half2_t{v0[e], v1[e]});
    }
    __syncthreads();

    if (j0 < w_kv_hi) {
      // ---- S^T = K . Q^T for NT sub-tiles of 16 keys ----
      float4_t sacc[NT];
#pragma unroll
      for (int kt = 0; kt < NT; ++kt) {
        sacc[kt] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          if constexpr (D >= 32) {
            sacc[kt] = mfma16x16x32(ld<half8_t>(&s_k[16 * kt + c][32 * kk + 8 * g]), qf[kk], sacc[kt]);
          } else {
            sacc[kt] = mfma16x16x16(ld<half4_t>(&s_k[16 * kt + c][4 * g]), lo4(qf[kk]), sacc[kt]);
          }
        }
      }
      // ---- mask, online softmax (row statistics live in lane column c) ----
      float bmax = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < NT; ++kt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = j0 + 16 * kt + 4 * g + r;
          const bool ok = row_ok && j < seq_len && j <= abs_row;
          sacc[kt][r] = ok ? sacc[kt][r] * scale_log2 : -INFINITY;
          bmax = fmaxf(bmax, sacc[kt][r]);
        }
      }
      bmax = rows_max(bmax);
      const float m_new = fmaxf(m, bmax);
      // A row with no visible key in this tile keeps m = -inf: use 0 as the reference point.
      const float m_ref = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = fast_exp2(m - m_ref);
      float lsum = 0.f;
      half4_t pb[NT];
#pragma unroll
      for (int kt = 0; kt < NT; ++kt) {
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[r] = fast_exp2(sacc[kt][r] - m_ref);
          lsum += p[r];
        }
        pb[kt] = {(half_t)p[0], (half_t)p[1], (half_t)p[2], (half_t)p[3]};
      }
      l = l * alpha + lsum;
      m = m_new;
#pragma unroll
      for (int t = 0; t < TILES; ++t) o[t] *= alpha;
      // ---- O^T += V^T . P^T; each 16x16x32 step covers key sub-tiles 2u and 2u + 1 ----
#pragma unroll
      for (int u = 0; u < NT / 2; ++u) {
        const half8_t pu = {pb[2 * u][0], pb[2 * u][1], pb[2 * u][2], pb[2 * u][3],
                            pb[2 * u + 1][0], pb[2 * u + 1][1], pb[2 * u + 1][2], pb[2 * u + 1][3]};
#pragma unroll
        for (int t = 0; t < TILES; ++t) {
          const half_t* vr = &s_vt[16 * t + c][0];
          const half4_t a0 = ld<half4_t>(vr + 32 * u + 4 * g);
          const half4_t a1 = ld<half4_t>(vr + 32 * u + 16 + 4 * g);
          const half8_t va = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
          o[t] = mfma16x16x32(va, pu, o[t]);
        }
      }
    }
    __syncthreads();
  }

  // ---- epilogue: lane (c, g) holds dims 16t + 4g .. +3 of its row ----
  l = rows_sum(l);
  if (row_ok) {
    const float inv = 1.f / (l == 0.f ? 1.f : l);       // a row with no key writes zeros
    half_t* op = out + (int64_t)(q_start + row) * o_st + (int64_t)h * D;
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      const half4_t v = {(half_t)(o[t][0] * inv), (half_t)(o[t][1] * inv),
                         (half_t)(o[t][2] * inv), (half_t)(o[t][3] * inv)};
      st<half4_t>(op + 16 * t + 4 * g, v);
    }
  }
}

// ------------------------------------------------------------------------------------------
// Streaming variant (the one launched): a wavefront owns 32 query rows of one head (two 16-row
// column groups) and reads K/V 16-token blocks straight into registers, the way the decode
// kernel does (K in MFMA layout, V as coalesced rows permuted in registers), keeping the next
// two pairs of blocks in flight while the current pair is multiplied. The workgroup's wavefronts take
// the key pairs round-robin for the same 32 rows and merge their (m, l, acc) in LDS, so a short
// chunk on a long prefix still spreads over the whole device without global partials.
// ------------------------------------------------------------------------------------------
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
    int num_decode, int H, int KVH, float scale_log2) {
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
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int c = lane & 15, g = lane >> 4;

  const int q_start = qsl[b];
  int q_len = qsl[b + 1] - q_start;
  if (q_start < 0 || q_len < 0 || (int64_t)q_start + q_len > num_tokens) q_len = 0;  // bad metadata
  int seq_len = seq_lens[b];
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
    for (int t = 0; t < TILES; ++t) {
      half4_t va = {vr[0][0][t], vr[0][1][t], vr[0][2][t], vr[0][3][t]};
      half4_t vb = {vr[1][0][t], vr[1][1][t], vr[1][2][t], vr[1][3][t]};
      if (tail_a) va = mask_tokens(va, ta, kv_hi);
      if (tail_b) vb = mask_tokens(vb, tb, kv_hi);
      v8[t] = {va[0], va[1], va[2], va[3], vb[0], vb[1], vb[2], vb[3]};
    }
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
      float sca[4], scb[4];
      if (interior) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sca[r] = sa[r] * scale_log2;
          scb[r] = sb[r] * scale_log2;
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sca[r] = (ta + r < kv_hi && ta + r <= lim[rg]) ? sa[r] * scale_log2 : -INFINITY;
          scb[r] = (tb + r < kv_hi && tb + r <= lim[rg]) ? sb[r] * scale_log2 : -INFINITY;
        }
      }
      const float bmax = rows_max(fmaxf(fmaxf(fmaxf(sca[0], sca[1]), fmaxf(sca[2], sca[3])),
                                        fmaxf(fmaxf(scb[0], scb[1]), fmaxf(scb[2], scb[3]))));
      const float m_new = fmaxf(m[rg], bmax);
      // a row with no visible key so far keeps m = -inf: use 0 as the reference point
      const float m_ref = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = fast_exp2(m[rg] - m_ref);
      // O is rescaled only when some row's running max moved (alpha == 1 exactly otherwise).
      const bool rescale = __ballot(m_new != m[rg]) != 0;
      float pa[4], pb[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pa[r] = fast_exp2(sca[r] - m_ref);
        pb[r] = fast_exp2(scb[r] - m_ref);
      }
      l[rg] = l[rg] * alpha + (((pa[0] + pa[1]) + (pa[2] + pa[3])) + ((pb[0] + pb[1]) + (pb[2] + pb[3])));
      m[rg] = m_new;
      const half8_t p8 = {(half_t)pa[0], (half_t)pa[1], (half_t)pa[2], (half_t)pa[3],
                          (half_t)pb[0], (half_t)pb[1], (half_t)pb[2], (half_t)pb[3]};
      if (rescale) {
#pragma unroll
        for (int t = 0; t < TILES; ++t) o[rg][t] *= alpha;
      }
#pragma unroll
      for (int t = 0; t < TILES; ++t)
        o[rg][t] = mfma16x16x32(v8[t], p8, o[rg][t]);   // lane (c, g): dims VW (4g + r) + t
    }
  };
  // Three-deep register ring: the loads of pair p + 2 NW are issued before pair p is computed.
  // (Occupancy is one wavefront per SIMD at D = 128 anyway, so the ring costs no occupancy.)
  half8_t k0[2][KK], k1[2][KK], k2[2][KK];
  VRow v0[2][4], v1[2][4], v2[2][4];
  int p = w;
  if (p < npairs) load_pair(p, k0, v0);
  if (p + NW < npairs) load_pair(p + NW, k1, v1);
  for (; p < npairs; p += 3 * NW) {
    if (p + 2 * NW < npairs) load_pair(p + 2 * NW, k2, v2);
    compute_pair(p, k0, v0);
    if (p + NW >= npairs) break;
    if (p + 3 * NW < npairs) load_pair(p + 3 * NW, k0, v0);
    compute_pair(p + NW, k1, v1);
    if (p + 2 * NW >= npairs) break;
    if (p + 4 * NW < npairs) load_pair(p + 4 * NW, k1, v1);
    compute_pair(p + 2 * NW, k2, v2);
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
