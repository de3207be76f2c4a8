// Paged decode attention for gfx950: the v1 / v2 / v3 family of
// ops/triton_decode_attention.py:1-200 with the policy of ops/triton_ops.py:35-57.
//
//  v1  one wavefront per (sequence, query head); VALU dot products and 64-lane shuffles.
//      Reads every KV block once per query head; kept as the simple, any-group-size variant.
//  v2  one workgroup per (sequence, KV head, group of <= 16 query heads): the whole GQA group
//      shares each 16-token K/V block, which is read from HBM exactly once per KV head.
//  v3  v2 split over context partitions of `partition` tokens ("flash-decoding"): partials
//      (m, l, acc) in fp32 go to the workspace and a merge kernel combines them (sequences
//      that fit one split are finished by the first kernel).
//
// Inner loop of v2/v3 (one wavefront, a pair of 16-token blocks; lane l = 16 g + c):
//   S^T[16 tok][16 heads] = K[16 tok][D] . Q^T[D][16 heads]       v_mfma_f32_16x16x32_f16
//   K lane (c, g) loads K[tok c][32kk + 8g .. +7]: 16-byte loads, 64 contiguous bytes per token
//   per instruction; Q^T uses the same dim permutation, so no shuffles are needed.
//   The result leaves lane (c, g) holding tokens 4g..4g+3 of head c: every per-head softmax
//   statistic (running max m, sum l, rescale alpha) lives in lane column c.
//   V rows are loaded coalesced (lane (c, g): tokens 4g..4g+3, dims 8c..8c+7 at D = 128) and
//   tile t of O^T takes dims {8i + t}, so each lane's token-packed operand is two byte
//   permutes of what it loaded: O^T[D][16 heads] += V^T . P^T runs on v_mfma_f32_16x16x32_f16
//   over both blocks of the pair with no transpose; P is rounded to fp16 first, exactly like
//   ops/triton_decode_attention.py:91. Afterwards lane (c, g) owns dims 32g .. 32g+31 of head c.
// The waves of a workgroup take consecutive blocks and merge their (m, l, acc) in LDS.
#include <math.h>

#include "common.h"
#include "paged_kv.h"

namespace ts {

constexpr float kLog2e = 1.4426950408889634f;

// ------------------------------------------------------------------------------------------
// v1 (ops/triton_decode_attention.py:23-54)
// ------------------------------------------------------------------------------------------
template <int D>
__global__ void __launch_bounds__(64) decode_v1_kernel(
    const half_t* __restrict__ q, int64_t q_st, int64_t q_sh, half_t* __restrict__ out,
    int64_t o_st, const half_t* __restrict__ kc, const half_t* __restrict__ vc, int64_t NB,
    const int* __restrict__ bt, int64_t bt_st, int max_blocks, const int* __restrict__ seq_lens,
    int H, int KVH, float scale_log2) {
  constexpr int DQ = D / 4;                    // dims per lane: 4 lanes share one token row
  const int s = blockIdx.x, h = blockIdx.y;
  const int G = H / KVH, kvh = h / G;
  const int lane = threadIdx.x, tok = lane >> 2, part = lane & 3;
  int seq_len = seq_lens[s];
  seq_len = seq_len < 0 ? 0 : (seq_len > max_blocks * kBlockSize ? max_blocks * kBlockSize : seq_len);
  float qv[DQ], acc[DQ];
  const half_t* qp = q + (int64_t)s * q_st + (int64_t)h * q_sh + part * DQ;
#pragma unroll
  for (int d = 0; d < DQ; ++d) {
    qv[d] = (float)qp[d];
    acc[d] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int nblk = (seq_len + kBlockSize - 1) / kBlockSize;
  for (int i = 0; i < nblk; ++i) {
    const int phys = clamp_block(bt[(int64_t)s * bt_st + i], NB);
    const int64_t row = (((int64_t)phys * KVH + kvh) * kBlockSize + tok) * D + part * DQ;
    float sc = 0.f;
#pragma unroll
    for (int d = 0; d < DQ; ++d) sc += qv[d] * (float)kc[row + d];
    sc += shfl_xor(sc, 1);
    sc += shfl_xor(sc, 2);
    const bool valid = i * kBlockSize + tok < seq_len;
    sc = valid ? sc * scale_log2 : -INFINITY;
    float bm = sc;
    bm = fmaxf(bm, shfl_xor(bm, 4));
    bm = fmaxf(bm, shfl_xor(bm, 8));
    bm = fmaxf(bm, shfl_xor(bm, 16));
    bm = fmaxf(bm, shfl_xor(bm, 32));
    const float m_new = fmaxf(m, bm);          // finite: token 0 of the block is valid
    const float alpha = fast_exp2(m - m_new);
    const float p = valid ? fast_exp2(sc - m_new) : 0.f;
    float ps = p;                              // sum over the 16 tokens (lanes of equal part)
    ps += shfl_xor(ps, 4);
    ps += shfl_xor(ps, 8);
    ps += shfl_xor(ps, 16);
    ps += shfl_xor(ps, 32);
    l = l * alpha + ps;
#pragma unroll
    for (int d = 0; d < DQ; ++d) acc[d] = acc[d] * alpha + (valid ? p * (float)vc[row + d] : 0.f);
    m = m_new;
  }
#pragma unroll
  for (int d = 0; d < DQ; ++d) {
    float a = acc[d];
    a += shfl_xor(a, 4);
    a += shfl_xor(a, 8);
    a += shfl_xor(a, 16);
    a += shfl_xor(a, 32);
    acc[d] = a;
  }
  const float inv = 1.f / (l == 0.f ? 1.f : l);   // seq_len 0 -> zeros
  if (tok == 0) {
    half_t* op = out + (int64_t)s * o_st + (int64_t)h * D + part * DQ;
#pragma unroll
    for (int d = 0; d < DQ; ++d) op[d] = (half_t)(acc[d] * inv);
  }
}

// ------------------------------------------------------------------------------------------
// v2 / v3 (ops/triton_decode_attention.py:60-163)
// ------------------------------------------------------------------------------------------
// One workgroup = NW wavefronts = one (sequence, split, KV head, head group). A wavefront owns
// BPW consecutive 16-token blocks per round and issues all their loads before computing; the
// block-table entries, seq_len and q are requested together at the start. Blocks are consumed
// in pairs: two independent S^T chains, one online-softmax update per 32 tokens, and the P.V
// product as v_mfma_f32_16x16x32_f16 over the 32 tokens of the pair. A sequence with one active
// split writes its output here; otherwise the split's (m, l, acc) go to the workspace for
// decode_merge_kernel.
template <int D, int NW, int BPW>
__global__ void __launch_bounds__(NW * 64) decode_mfma_kernel(
    const half_t* __restrict__ q, int64_t q_st, int64_t q_sh, half_t* __restrict__ out,
    int64_t o_st, const half_t* __restrict__ kc, const half_t* __restrict__ vc, int64_t NB,
    const int* __restrict__ bt, int64_t bt_st, int max_blocks, const int* __restrict__ seq_lens,
    int H, int KVH, int G, int HG, float scale_log2, int part_blocks, int num_splits,
    float* __restrict__ ws_acc, float* __restrict__ ws_m, float* __restrict__ ws_l) {
  static_assert(BPW % 2 == 0, "blocks are consumed in pairs");
  constexpr int KK = KvRegs<D>::KK;
  constexpr int VW = KvRegs<D>::VW;
  constexpr int TILES = KvRegs<D>::TILES;
  constexpr int OROW = D + 4;                    // padded LDS row (floats) against bank conflicts
  __shared__ float s_o[NW][16][OROW];
  __shared__ float s_m[NW][16];
  __shared__ float s_l[NW][16];

  const int s = blockIdx.x, split = blockIdx.y;
  const int kvh = blockIdx.z / HG, hg = blockIdx.z % HG;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int c = lane & 15, g = lane >> 4;
  const int hq = hg * 16 + c;                    // query head within the GQA group
  const bool head_ok = hq < G;
  const int nh = (G - hg * 16) < 16 ? (G - hg * 16) : 16;   // real heads in this group
  const int head0 = kvh * G + hg * 16;           // first query head of this group
  const int blk_lo = split * part_blocks;
  const int* btrow = bt + (int64_t)s * bt_st;

  // Requests that do not depend on seq_len go out first, together.
  int seq_len = seq_lens[s];
  int r0 = blk_lo + w * BPW;
  int btv[BPW];
#pragma unroll
  for (int j = 0; j < BPW; ++j) btv[j] = btrow[(r0 + j) < max_blocks ? (r0 + j) : (max_blocks - 1)];
  half8_t qf[KK];
  {
    const half_t* qp = q + (int64_t)s * q_st + (int64_t)(kvh * G + hq) * q_sh;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if constexpr (D >= 32) {
        qf[kk] = head_ok ? ld<half8_t>(qp + 32 * kk + 8 * g) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
      } else {
        const half4_t t = head_ok ? ld<half4_t>(qp + 4 * g) : half4_t{0, 0, 0, 0};
        qf[kk] = {t[0], t[1], t[2], t[3], 0, 0, 0, 0};
      }
    }
  }

  seq_len = seq_len < 0 ? 0 : (seq_len > max_blocks * kBlockSize ? max_blocks * kBlockSize : seq_len);
  const int nblk = (seq_len + kBlockSize - 1) / kBlockSize;
  // A seq_len beyond the caller's max_seq_len is truncated to the launched splits, as the fixed
  // split grid of ops/triton_ops.py:50-51 does; it never indexes past the workspace.
  int n_active = (nblk + part_blocks - 1) / part_blocks;
  n_active = n_active < num_splits ? n_active : num_splits;
  // With split partials, every split slot that carries no partial (idle split, a sequence that
  // fits one split, seq_len 0) is marked m = -inf so the merge needs no seq_len.
  const bool idle = seq_len == 0 || blk_lo >= nblk;
  if ((idle || n_active == 1) && num_splits > 1 && tid < nh)
    ws_m[((int64_t)s * H + head0 + tid) * num_splits + split] = -INFINITY;
  if (seq_len == 0) {                            // padding row: zeros (ops/reference.py:99,104-105)
    if (split == 0) {
      for (int e = tid; e < nh * D; e += NW * 64)
        out[(int64_t)s * o_st + (int64_t)(head0 + e / D) * D + e % D] = (half_t)0.f;
    }
    return;
  }
  if (idle) return;                              // idle split of a short sequence
  const int blk_hi = (blk_lo + part_blocks) < nblk ? (blk_lo + part_blocks) : nblk;
  // Tokens this split may use: a pair's second block can lie past the split (or be a repeat of
  // its last block) while its tokens are still below seq_len.
  const int tok_hi = blk_hi * kBlockSize < seq_len ? blk_hi * kBlockSize : seq_len;

  const float4_t zero4 = {0.f, 0.f, 0.f, 0.f};
  float4_t o[TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t) o[t] = zero4;
  float m = -INFINITY, l = 0.f;

  const int64_t head_off = (int64_t)kvh * kBlockSize * D;
  const int64_t blk_stride = (int64_t)KVH * kBlockSize * D;
  for (; r0 < blk_hi; r0 += NW * BPW) {
    // Blocks past blk_hi repeat the last valid block (a cache hit, no extra HBM read), so the
    // loads below carry no branches; the repeated data is masked out of the softmax.
    int phys[BPW];
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
      int id = btv[j];
#pragma unroll
      for (int i = 0; i < BPW; ++i)
        if (r0 + j >= blk_hi && r0 + i == blk_hi - 1) id = btv[i];
      phys[j] = clamp_block(id, NB);
    }
    half8_t kf[BPW][KK];
    typename HalfVec<VW>::type vr[BPW][4];
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
      const int64_t off = phys[j] * blk_stride + head_off;
      load_k_block<D>(kc + off, c, g, kf[j]);
      load_v_rows<D>(vc + off, c, g, vr[j]);
    }
    const int r_next = r0 + NW * BPW;
    if (r_next < blk_hi) {                       // next round's table entries, early
#pragma unroll
      for (int j = 0; j < BPW; ++j)
        btv[j] = btrow[(r_next + j) < max_blocks ? (r_next + j) : (max_blocks - 1)];
    }
#pragma unroll
    for (int pr = 0; pr < BPW / 2; ++pr) {
      const int ja = 2 * pr, jb = 2 * pr + 1;
      const int ba = r0 + ja, bb = r0 + jb;
      if (ba >= blk_hi) break;
      // S^T = K . Q^T for both blocks: two independent MFMA chains
      float4_t sa = zero4, sb = zero4;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        if constexpr (D >= 32) {
          sa = mfma16x16x32(kf[ja][kk], qf[kk], sa);
          sb = mfma16x16x32(kf[jb][kk], qf[kk], sb);
        } else {
          sa = mfma16x16x16(lo4(kf[ja][kk]), lo4(qf[kk]), sa);
          sb = mfma16x16x16(lo4(kf[jb][kk]), lo4(qf[kk]), sb);
        }
      }
      const int ta = ba * kBlockSize + 4 * g, tb = bb * kBlockSize + 4 * g;
      const bool interior = (bb + 1) * kBlockSize <= tok_hi;   // every token of the pair valid
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
          sca[r] = (ta + r < tok_hi) ? sa[r] * scale_log2 : -INFINITY;
          scb[r] = (tb + r < tok_hi) ? sb[r] * scale_log2 : -INFINITY;
        }
      }
      const float bmax = rows_max(fmaxf(fmaxf(fmaxf(sca[0], sca[1]), fmaxf(sca[2], sca[3])),
                                        fmaxf(fmaxf(scb[0], scb[1]), fmaxf(scb[2], scb[3]))));
      const float m_new = fmaxf(m, bmax);        // finite: token 0 of block ba is valid
      const float alpha = fast_exp2(m - m_new);
      // O is rescaled only when some head's running max moved (alpha == 1 exactly otherwise),
      // which after the first blocks is rare: the accumulators then stay in the MFMA registers.
      const bool rescale = __ballot(m_new != m) != 0;
      float pa[4], pb[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pa[r] = fast_exp2(sca[r] - m_new);
        pb[r] = fast_exp2(scb[r] - m_new);
      }
      l = l * alpha + (((pa[0] + pa[1]) + (pa[2] + pa[3])) + ((pb[0] + pb[1]) + (pb[2] + pb[3])));
      m = m_new;
      const half8_t p8 = {(half_t)pa[0], (half_t)pa[1], (half_t)pa[2], (half_t)pa[3],
                          (half_t)pb[0], (half_t)pb[1], (half_t)pb[2], (half_t)pb[3]};
      const bool tail_a = (ba + 1) * kBlockSize > tok_hi;
      const bool tail_b = (bb + 1) * kBlockSize > tok_hi;
      if (rescale) {
#pragma unroll
        for (int t = 0; t < TILES; ++t) o[t] *= alpha;
      }
#pragma unroll
      for (int t = 0; t < TILES; ++t) {
        half4_t va = {vr[ja][0][t], vr[ja][1][t], vr[ja][2][t], vr[ja][3][t]};
        half4_t vb = {vr[jb][0][t], vr[jb][1][t], vr[jb][2][t], vr[jb][3][t]};
        if (tail_a) va = mask_tokens(va, ta, tok_hi);
        if (tail_b) vb = mask_tokens(vb, tb, tok_hi);
        const half8_t v8 = {va[0], va[1], va[2], va[3], vb[0], vb[1], vb[2], vb[3]};
        o[t] = mfma16x16x32(v8, p8, o[t]);        // lane (c, g): dims VW (4g + r) + t of head c
      }
    }
  }
  l = rows_sum(l);

  // Merge the NW wavefronts of this workgroup in LDS.
  if (g == 0) {
    s_m[w][c] = m;
    s_l[w][c] = l;
  }
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) s_o[w][c][VW * (4 * g + r) + t] = o[t][r];
  __syncthreads();
  const bool single = n_active == 1;
  for (int e = tid; e < nh * D; e += NW * 64) {
    const int hh = e / D, d = e % D;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, s_m[ww][hh]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float wt = fast_exp2(s_m[ww][hh] - M);    // idle wavefront: m = -inf -> 0
      L += wt * s_l[ww][hh];
      O += wt * s_o[ww][hh][d];
    }
    if (single) {
      out[(int64_t)s * o_st + (int64_t)(head0 + hh) * D + d] = (half_t)(O / L);
    } else {
      const int64_t pidx = ((int64_t)s * H + head0 + hh) * num_splits + split;
      ws_acc[pidx * D + d] = O;
      if (d == 0) {
        ws_m[pidx] = M;
        ws_l[pidx] = L;
      }
    }
  }
}

// Merge of the split partials (ops/triton_decode_attention.py:144-163): M = max m_j,
// w_j = 2^(m_j - M), out = sum w_j acc_j / sum w_j l_j. One workgroup per (sequence, KV head,
// head group), two dependent memory steps: every (head, split) statistic is loaded at once
// (slots without a partial hold m = -inf, so seq_len is not needed), then the partials of the
// active splits (a compact list, identical for all heads) are read without branches. A group
// whose slots are all -inf was finished by the first kernel.
template <int D>
__global__ void __launch_bounds__(256) decode_merge_kernel(
    const float* __restrict__ ws_acc, const float* __restrict__ ws_m,
    const float* __restrict__ ws_l, half_t* __restrict__ out, int64_t o_st, int H, int G, int HG,
    int num_splits) {
  constexpr int kMaxSplits = 256;               // the launcher caps num_splits
  __shared__ float s_w[16][kMaxSplits];
  __shared__ float s_l[16][kMaxSplits];
  __shared__ float s_inv[16];
  __shared__ int s_act[kMaxSplits];             // splits that carry a partial (same for all heads)
  __shared__ int s_nact;
  const int s = blockIdx.x, kvh = blockIdx.y / HG, hg = blockIdx.y % HG;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int nh = (G - hg * 16) < 16 ? (G - hg * 16) : 16;
  const int head0 = kvh * G + hg * 16;
  const int64_t base0 = ((int64_t)s * H + head0) * num_splits;
  for (int e = tid; e < nh * num_splits; e += 256) {
    const int hh = e / num_splits, j = e % num_splits;
    s_w[hh][j] = ws_m[base0 + (int64_t)hh * num_splits + j];
    s_l[hh][j] = ws_l[base0 + (int64_t)hh * num_splits + j];
  }
  __syncthreads();
  if (w == 0) {                                 // compact list of active splits (ballot + popcount)
    int n = 0;
    for (int j0 = 0; j0 < num_splits; j0 += 64) {
      const int j = j0 + lane;
      const bool act = j < num_splits && s_w[0][j] != -INFINITY;
      const uint64_t mask = __ballot(act);
      if (act) s_act[n + __popcll(mask & ((1ull << lane) - 1))] = j;
      n += __popcll(mask);
    }
    if (lane == 0) s_nact = n;
  }
  for (int hh = w; hh < nh; hh += 4) {
    float M = -INFINITY;
    for (int j = lane; j < num_splits; j += 64) M = fmaxf(M, s_w[hh][j]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, shfl_xor(M, off));
    float L = 0.f;
    for (int j = lane; j < num_splits; j += 64) {
      const float m = s_w[hh][j];
      const float wt = m == -INFINITY ? 0.f : fast_exp2(m - M);
      s_w[hh][j] = wt;
      L += m == -INFINITY ? 0.f : wt * s_l[hh][j];   // a slot without a partial holds garbage l
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) L += shfl_xor(L, off);
    if (lane == 0) s_inv[hh] = M == -INFINITY ? 0.f : 1.f / L;
  }
  __syncthreads();
  const int nact = s_nact;
  if (nact == 0) return;                        // finished (or zeroed) by the first kernel
  // Each thread owns up to EPT outputs; for every chunk of CH active splits all EPT x CH loads
  // are issued before any is consumed (indices past nact repeat the last split with weight 0).
  constexpr int EPT = 4, CH = 16;
  for (int e0 = tid; e0 < nh * D; e0 += 256 * EPT) {
    float O[EPT];
    const float* accp[EPT];
    int hh_[EPT];
    bool ok[EPT];
#pragma unroll
    for (int q = 0; q < EPT; ++q) {
      const int e = e0 + 256 * q;
      ok[q] = e < nh * D;
      const int ee = ok[q] ? e : 0;
      hh_[q] = ee / D;
      accp[q] = ws_acc + (base0 + (int64_t)hh_[q] * num_splits) * D + ee % D;
      O[q] = 0.f;
    }
    for (int t0 = 0; t0 < nact; t0 += CH) {
      float v[EPT][CH];
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int j = s_act[(t0 + u) < nact ? (t0 + u) : (nact - 1)];
#pragma unroll
        for (int q = 0; q < EPT; ++q) v[q][u] = accp[q][(int64_t)j * D];
      }
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int j = s_act[(t0 + u) < nact ? (t0 + u) : (nact - 1)];
#pragma unroll
        for (int q = 0; q < EPT; ++q) O[q] += (t0 + u < nact) ? s_w[hh_[q]][j] * v[q][u] : 0.f;
      }
    }
#pragma unroll
    for (int q = 0; q < EPT; ++q) {
      const int e = e0 + 256 * q;
      if (ok[q]) out[(int64_t)s * o_st + (int64_t)(head0 + hh_[q]) * D + e % D] = (half_t)(O[q] * s_inv[hh_[q]]);
    }
  }
}

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------
#ifndef TS_DECODE_WAVES
#define TS_DECODE_WAVES 4
#endif
#ifndef TS_DECODE_BLOCKS_PER_WAVE
#define TS_DECODE_BLOCKS_PER_WAVE 4
#endif
constexpr int kDecodeWaves = TS_DECODE_WAVES;               // wavefronts per workgroup
constexpr int kBlocksPerWave = TS_DECODE_BLOCKS_PER_WAVE;   // blocks loaded up front per round
constexpr int kDefaultPartition = kDecodeWaves * kBlocksPerWave * kBlockSize;   // 256 tokens

struct SplitPlan {
  int version;        // 1, 2 or 3 after resolving AUTO
  int part_blocks;    // blocks per split
  int num_splits;
};

static SplitPlan plan_decode(int version, int S, int H, int KVH, int max_seq_len, int partition,
                             int cu_count) {
  SplitPlan p{version, 1 << 30, 1};
  const int G = H / KVH;
  const int HG = (G + 15) / 16;
  if (version == TS_DECODE_AUTO) {
    // ops/triton_ops.py:44-45: split when the (sequence, KV head) grid cannot fill the device
    // twice over and the context is long; the CU count replaces the SM count.
    const bool use_split = (int64_t)S * KVH * HG < 2LL * cu_count && max_seq_len > 1024;
    p.version = use_split ? TS_DECODE_V3 : TS_DECODE_V2;
  }
  if (p.version == TS_DECODE_V3) {
    int part = partition > 0 ? partition : kDefaultPartition;
    part = ((part + kBlockSize - 1) / kBlockSize) * kBlockSize;
    p.part_blocks = part / kBlockSize;
    const int max_blk = (max_seq_len + kBlockSize - 1) / kBlockSize;
    p.num_splits = (max_blk + p.part_blocks - 1) / p.part_blocks;   // ops/triton_ops.py:50-51
    if (p.num_splits > 256) {                    // the merge keeps <= 256 split weights in LDS
      p.part_blocks = (max_blk + 255) / 256;
      p.num_splits = (max_blk + p.part_blocks - 1) / p.part_blocks;
    }
    if (p.num_splits < 1) p.num_splits = 1;
  }
  return p;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct WsLayout {
  size_t acc, m, l, total;
};

// [acc: S * H * splits * D fp32][m: S * H * splits][l: S * H * splits]
static WsLayout ws_layout(const SplitPlan& p, int S, int H, int D) {
  WsLayout w{0, 0, 0, 0};
  if (p.version != TS_DECODE_V3 || p.num_splits <= 1) return w;
  const size_t n = (size_t)S * H * p.num_splits;
  w.acc = 0;
  w.m = align256(n * D * sizeof(float));
  w.l = w.m + align256(n * sizeof(float));
  w.total = w.l + align256(n * sizeof(float));
  return w;
}

template <int D>
static void launch_decode(const SplitPlan& p, hipStream_t st, const half_t* q, int64_t q_st,
                          int64_t q_sh, half_t* out, int64_t o_st, const half_t* kc,
                          const half_t* vc, int64_t NB, const int* bt, int64_t bt_st,
                          int max_blocks, const int* sl, int S, int H, int KVH, float scale_log2,
                          void* ws) {
  const int G = H / KVH;
  if (p.version == TS_DECODE_V1) {
    decode_v1_kernel<D><<<dim3(S, H), 64, 0, st>>>(q, q_st, q_sh, out, o_st, kc, vc, NB, bt,
                                                   bt_st, max_blocks, sl, H, KVH, scale_log2);
    return;
  }
  const int HG = (G + 15) / 16;
  float *ws_acc = nullptr, *ws_m = nullptr, *ws_l = nullptr;
  if (p.num_splits > 1) {
    const WsLayout w = ws_layout(p, S, H, D);
    char* b = static_cast<char*>(ws);
    ws_acc = reinterpret_cast<float*>(b + w.acc);
    ws_m = reinterpret_cast<float*>(b + w.m);
    ws_l = reinterpret_cast<float*>(b + w.l);
  }
  decode_mfma_kernel<D, kDecodeWaves, kBlocksPerWave>
      <<<dim3(S, p.num_splits, KVH * HG), kDecodeWaves * 64, 0, st>>>(
          q, q_st, q_sh, out, o_st, kc, vc, NB, bt, bt_st, max_blocks, sl, H, KVH, G, HG,
          scale_log2, p.part_blocks, p.num_splits, ws_acc, ws_m, ws_l);
  if (p.num_splits > 1) {
    decode_merge_kernel<D><<<dim3(S, KVH * HG), 256, 0, st>>>(ws_acc, ws_m, ws_l, out, o_st, H,
                                                              G, HG, p.num_splits);
  }
}

static bool supported_head_dim(int D) {
  return D == 16 || D == 32 || D == 64 || D == 128 || D == 256;
}

}  // namespace ts

using namespace ts;

extern "C" size_t ts_decode_workspace_bytes(int32_t version, int32_t num_seqs, int32_t num_heads,
                                            int32_t num_kv_heads, int32_t head_dim,
                                            int32_t max_seq_len, int32_t partition,
                                            int32_t cu_count) {
  if (num_seqs <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return 0;
  const SplitPlan p = plan_decode(version, num_seqs, num_heads, num_kv_heads, max_seq_len,
                                  partition, cu_count > 0 ? cu_count : 256);
  return ws_layout(p, num_seqs, num_heads, head_dim).total;
}

extern "C" int ts_decode_attention(int32_t version, const void* q, int64_t q_stride_t,
                                   int64_t q_stride_h, void* out, int64_t out_stride_t,
                                   const void* k_cache, const void* v_cache, int64_t num_blocks,
                                   const int32_t* block_tables, int64_t bt_stride,
                                   int32_t max_blocks_per_seq, const int32_t* seq_lens,
                                   int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                   int32_t head_dim, float scale, int32_t max_seq_len,
                                   int32_t partition, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  TS_REQUIRE(version >= TS_DECODE_AUTO && version <= TS_DECODE_V3, TS_ERR_INVALID_ARG,
             "decode_attention: unknown version %d", version);
  TS_REQUIRE(num_seqs >= 0, TS_ERR_INVALID_ARG, "decode_attention: num_seqs %d < 0", num_seqs);
  if (num_seqs == 0) return TS_OK;
  TS_REQUIRE(q && out && k_cache && v_cache && block_tables && seq_lens, TS_ERR_INVALID_ARG,
             "decode_attention: null pointer argument");
  TS_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
             TS_ERR_INVALID_ARG, "decode_attention: num_heads=%d not a multiple of num_kv_heads=%d",
             num_heads, num_kv_heads);
  TS_REQUIRE(supported_head_dim(head_dim), TS_ERR_UNSUPPORTED,
             "decode_attention: head_dim %d not in {16, 32, 64, 128, 256}", head_dim);
  TS_REQUIRE(num_blocks > 0 && max_blocks_per_seq > 0 && bt_stride >= max_blocks_per_seq,
             TS_ERR_INVALID_ARG, "decode_attention: bad block table (num_blocks=%lld width=%d stride=%lld)",
             (long long)num_blocks, max_blocks_per_seq, (long long)bt_stride);
  TS_REQUIRE(partition >= 0 && partition % kBlockSize == 0, TS_ERR_INVALID_ARG,
             "decode_attention: partition %d is not a multiple of 16", partition);
  const int vec = head_dim >= 32 ? 8 : 4;
  TS_REQUIRE(q_stride_t % vec == 0 && q_stride_h % vec == 0 && aligned(q, 2 * vec) &&
                 aligned(k_cache, 2 * vec) && aligned(v_cache, 2 * vec),
             TS_ERR_INVALID_ARG, "decode_attention: q / caches must be %d-byte aligned", 2 * vec);
  int cus = 0;
  int st = device_cu_count(&cus);
  if (st != TS_OK) return st;
  const SplitPlan p = plan_decode(version, num_seqs, num_heads, num_kv_heads, max_seq_len,
                                  partition, cus);
  const size_t need = ws_layout(p, num_seqs, num_heads, head_dim).total;
  TS_REQUIRE(need == 0 || (workspace && workspace_bytes >= need && aligned(workspace, 256)),
             TS_ERR_WORKSPACE, "decode_attention: workspace of %zu bytes (256-aligned) needed, got %zu",
             need, workspace_bytes);
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const float sl2 = scale * kLog2e;
  const half_t* qp = static_cast<const half_t*>(q);
  half_t* op = static_cast<half_t*>(out);
  const half_t* kp = static_cast<const half_t*>(k_cache);
  const half_t* vp = static_cast<const half_t*>(v_cache);
#define TS_DECODE_CASE(DD)                                                                      \
  case DD:                                                                                      \
    launch_decode<DD>(p, s, qp, q_stride_t, q_stride_h, op, out_stride_t, kp, vp, num_blocks,  \
                      block_tables, bt_stride, max_blocks_per_seq, seq_lens, num_seqs, num_heads, \
                      num_kv_heads, sl2, workspace);                                            \
    break;
  switch (head_dim) {
    TS_DECODE_CASE(16)
    TS_DECODE_CASE(32)
    TS_DECODE_CASE(64)
    TS_DECODE_CASE(128)
    TS_DECODE_CASE(256)
  }
#undef TS_DECODE_CASE
  return check_launch("decode_attention");
}
