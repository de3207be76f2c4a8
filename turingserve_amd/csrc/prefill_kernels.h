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
#pragma once

#include <math.h>

#include "common.h"
#include "paged_kv.h"
namespace ts {

constexpr float kLog2eP = 1.4426950408889634f;

// Rows [row_lo, q_len) of query head h of a sequence, filled with NaN by the whole workgroup:
// what a tile gets whose rows the launch does not cover (host bounds below the batch's real
// q_len / seq_len), so the caller sees the understated bound instead of stale memory.
template <int D>
__device__ __forceinline__ void poison_rows(half_t* __restrict__ out, int64_t o_st, int q_start,
                                            int row_lo, int q_len, int h) {
  const half_t nan = __builtin_bit_cast(half_t, (unsigned short)0x7e00);
  const half4_t n4 = {nan, nan, nan, nan};
  const int per_row = D / 4;
  for (int e = (int)threadIdx.x; e < (q_len - row_lo) * per_row; e += (int)blockDim.x) {
    const int row = row_lo + e / per_row, d0 = 4 * (e % per_row);
    ts::st<half4_t>(out + (int64_t)(q_start + row) * o_st + (int64_t)h * D + d0, n4);
  }
}


constexpr int kPsRows = 32;           // query rows per workgroup and wavefront (two 16-row groups)
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
  if (mtile == (int)gridDim.x - 1 && (int64_t)gridDim.x * kPsRows < q_len)
    poison_rows<D>(out, o_st, q_start, (int)gridDim.x * kPsRows, q_len, h);   // q_len past the bound
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


// ------------------------------------------------------------------------------------------
// LDS-tiled prefill (D = 128, the Qwen2.5 attention shapes).
//
// Workgroup = 128 query rows of one query head, four wavefronts of 32 rows each. Every 64-key
// step (four 16-token blocks) is staged once in LDS and shared by the four wavefronts: K in its
// natural [key][dim] layout, V transposed to [dim][key] (16 bytes of padding per row keep the
// 16-lane groups of each 16-byte read on distinct banks). Wavefront w stages block w of the
// step, so its block-table entry is one scalar load. Per wavefront and step (lane l = 32 h + r):
//   S^T[32 keys][32 rows] = K . Q^T    v_mfma_f32_32x32x16_f16, two key halves x D/16 k-steps;
//       lane (r, h) of the result holds keys 8j + 4h + i (j, i = 0..3) of query row r, so every
//       per-row softmax statistic sits in lanes r and r + 32;
//   O^T[32 dims][32 rows] += V^T . P^T  for each of the D/32 dim tiles over four 16-key steps.
//       P^T is the S^T result rounded to fp16 as it lies in the registers (the contraction
//       index is permuted consistently: k-slot 8h + i is key 4h + i, k-slot 8h + 4 + i key
//       8 + 4h + i), which is why the staged V^T rows keep each 16-key group in the order
//       0-3, 8-11, 4-7, 12-15 (bits 2 and 3 of the key swapped): lane group h then reads its
//       eight keys as one 16-byte piece.
// Online softmax with the lazy reference point of the decode kernel; P is rounded to fp16
// before P.V (ops/triton_prefill_attention.py:57). The staging of step s + 1 (global loads
// into registers, then LDS) overlaps the MFMAs of step s; one barrier per step.
//
// Long key ranges are split: a tile with n steps runs as max(1, ceil(n / smax)) workgroups
// over consecutive step ranges, which leave fp32 partials (m, l, O) in the workspace; the
// merge kernel combines them. Launch slots of one (sequence, head) number the tiles longest
// first.
// ------------------------------------------------------------------------------------------
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int kTileRows = 128;
constexpr int kTileKeys = 64;
constexpr int kTileThreads = 256;
constexpr int kPrefillMinSteps = 4;   // fewest 64-key steps a split is given
constexpr int kMergeRows = 2;         // rows per merge thread (8 dims each)

template <int D>
struct TileLayout {
  static constexpr int KROW = 2 * D + 16;           // bytes per staged K row
  static constexpr int VROW = 2 * kTileKeys;        // bytes per staged V^T row (swizzled)
  static constexpr int KBYTES = kTileKeys * KROW;
  static constexpr int VBYTES = D * VROW;
  static constexpr int STAGE = KBYTES + VBYTES;
};

__device__ __forceinline__ float16_t mfma32x32x16(half8_t a, half8_t b, float16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// 16-byte piece p of staged V^T row d lives at piece p ^ vt_swz(d): the 8 lanes of one LDS
// phase hit 8 distinct pieces both when they read rows d0 .. d0+7 (MFMA operands) and when they
// write rows 4l + j, l = 0..7 (staging), so neither side has bank conflicts.
__device__ __forceinline__ int vt_swz(int d) { return (d ^ (d >> 3)) & 7; }

// Reductions over the two lanes of a query row (r and r + 32): v_permlane32_swap(x, x) returns
// the lower and the upper half of x in every lane.
__device__ __forceinline__ float pair_max(float v) {
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return vmax(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float pair_sum(float v) {
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

struct TileSlot {
  int tile, split, nsplit, lo, hi;   // steps [lo, hi) of tile `tile`; tile -1: idle slot
};

// Launch slot -> (tile, split) for one (sequence, head item): tiles of `tr` query rows longest
// first, tile i with n_i steps gets max(1, ceil(n_i / smax)) splits of balanced step ranges,
// numbered consecutively.
__device__ __forceinline__ TileSlot tile_slot(int slot, int q_len, int prefix, int seq_len, int smax,
                                              int tr) {
  const int tiles = (q_len + tr - 1) / tr;
  int base = 0;
  for (int i = tiles - 1; i >= 0; --i) {
    const int last = ((i + 1) * tr < q_len ? (i + 1) * tr : q_len) - 1;
    int hi = prefix + last + 1 < seq_len ? prefix + last + 1 : seq_len;
    hi = hi < 0 ? 0 : hi;
    const int n = (hi + kTileKeys - 1) / kTileKeys;
    const int ns = n <= smax ? 1 : (n + smax - 1) / smax;
    if (slot < base + ns) {
      const int j = slot - base;
      return {i, j, ns, (int)((int64_t)n * j / ns), (int)((int64_t)n * (j + 1) / ns)};
    }
    base += ns;
  }
  return {-1, 0, 0, 0, 0};
}

// First launch slot and split count of tile `tile` (the inverse of tile_slot).
__device__ __forceinline__ int2_t tile_span(int tile, int q_len, int prefix, int seq_len, int smax,
                                            int tr) {
  const int tiles = (q_len + tr - 1) / tr;
  int base = 0;
  for (int i = tiles - 1; i >= tile; --i) {
    const int last = ((i + 1) * tr < q_len ? (i + 1) * tr : q_len) - 1;
    int hi = prefix + last + 1 < seq_len ? prefix + last + 1 : seq_len;
    hi = hi < 0 ? 0 : hi;
    const int n = (hi + kTileKeys - 1) / kTileKeys;
    const int ns = n <= smax ? 1 : (n + smax - 1) / smax;
    if (i == tile) return {base, ns};
    base += ns;
  }
  return {0, 0};
}

// The lowest tile (of `tr` rows) whose splits run past a launch of `slots` slots, or -1: with
// host bounds below the batch's real q_len / seq_len the tiles a launch misses are the lowest
// ones (slots number the tiles longest first).
__device__ __forceinline__ int first_cut_tile(int q_len, int prefix, int seq_len, int smax, int tr,
                                              int slots) {
  const int tiles = (q_len + tr - 1) / tr;
  int base = 0;
  for (int i = tiles - 1; i >= 0; --i) {
    const int last_row = ((i + 1) * tr < q_len ? (i + 1) * tr : q_len) - 1;
    int hi = prefix + last_row + 1 < seq_len ? prefix + last_row + 1 : seq_len;
    hi = hi < 0 ? 0 : hi;
    const int n = (hi + kTileKeys - 1) / kTileKeys;
    base += n <= smax ? 1 : (n + smax - 1) / smax;
    if (base > slots) return i;
  }
  return -1;
}

struct PrefillSeq {
  int q_start, q_len, seq_len, prefix;
};

__device__ __forceinline__ PrefillSeq prefill_seq(const int* __restrict__ qsl,
                                                  const int* __restrict__ seq_lens, int b,
                                                  int64_t num_tokens, int max_blocks) {
  PrefillSeq p;
  p.q_start = __builtin_amdgcn_readfirstlane(qsl[b]);
  p.q_len = __builtin_amdgcn_readfirstlane(qsl[b + 1]) - p.q_start;
  if (p.q_start < 0 || p.q_len < 0 || (int64_t)p.q_start + p.q_len > num_tokens) p.q_len = 0;
  int sl = __builtin_amdgcn_readfirstlane(seq_lens[b]);
  p.seq_len = sl < 0 ? 0 : (sl > max_blocks * kBlockSize ? max_blocks * kBlockSize : sl);
  p.prefix = p.seq_len - p.q_len;
  return p;
}

// Workspace of the split path: per-split rows O (unnormalised) [slots_total][128][D] fp32, then
// (m, l) pairs [slots_total][128][2] fp32, slots_total = P * H * slots.
template <int D>
__device__ __forceinline__ void prefill_tile_body(
    const half_t* __restrict__ q, int64_t q_st, int64_t q_sh, half_t* __restrict__ out,
    int64_t o_st, int64_t num_tokens, const half_t* __restrict__ kc,
    const half_t* __restrict__ vc, int64_t NB, const int* __restrict__ bt, int64_t bt_st,
    int max_blocks, const int* __restrict__ seq_lens, const int* __restrict__ qsl,
    int num_decode, int H, int KVH, float sl2, int smax, int slots, int P,
    float* __restrict__ ws,
    int bx, char* __restrict__ lds) {
  static_assert(D == 128, "the staging roles below assume D = 128");
  using L = TileLayout<D>;
  constexpr int KK = D / 16;                       // k-steps of S^T
  constexpr int DT = D / 32;                       // 32-dim tiles of O^T

  // Work items of one KV head are (slot, sequence, query head of the group), slot-major. When
  // the KV heads divide the eight XCDs (launch ids l are dispatched round-robin, XCD l % 8),
  // XCD x serves KV head x / (8 / KVH) and takes every (8 / KVH)-th item of it: each XCD L2
  // holds one KV head's K/V, workgroups running together there share key steps, and the
  // slots past a sequence's last split (at the end of the order) fall evenly on the XCDs.
  const int G = H / KVH;
  const int per_kvh = slots * P * G;
  int kvh, rem;
  if (8 % KVH == 0) {
    const int xpk = 8 / KVH;
    const int xcd = (bx & 7);
    kvh = xcd / xpk;
    rem = (bx >> 3) * xpk + xcd % xpk;
  } else {
    kvh = bx / per_kvh;
    rem = bx - kvh * per_kvh;
  }
  if (kvh >= KVH || rem >= per_kvh) return;
  const int slot = rem / (P * G);
  rem -= slot * (P * G);
  const int pi = rem / G;
  const int h = kvh * G + (rem - pi * G);
  const int b = num_decode + pi;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, hh = lane >> 5;

  const PrefillSeq sq = prefill_seq(qsl, seq_lens, b, num_tokens, max_blocks);
  if (slot == slots - 1) {
    // Rows of tiles the launch misses are written by no other workgroup.
    const int cut = first_cut_tile(sq.q_len, sq.prefix, sq.seq_len, smax, kTileRows, slots);
    if (cut >= 0) {
      const int m_end = (cut + 1) * kTileRows < sq.q_len ? (cut + 1) * kTileRows : sq.q_len;
      poison_rows<D>(out, o_st, sq.q_start, 0, m_end, h);
    }
  }
  const TileSlot tsl = tile_slot(slot, sq.q_len, sq.prefix, sq.seq_len, smax, kTileRows);
  if (tsl.tile < 0) return;
  const int m0 = tsl.tile * kTileRows;
  const int last = (m0 + kTileRows < sq.q_len ? m0 + kTileRows : sq.q_len) - 1;
  int kv_hi = sq.prefix + last + 1 < sq.seq_len ? sq.prefix + last + 1 : sq.seq_len;
  kv_hi = kv_hi < 0 ? 0 : kv_hi;
  const int nblk = (kv_hi + kBlockSize - 1) / kBlockSize;
  const int r0 = m0 + 32 * w;                      // first query row of this wavefront
  const int row = r0 + r;
  const bool row_ok = row < sq.q_len;

  // Q^T operands: lane (r, h) holds dims 16 kk + 8 h .. +7 of its row (zeros past q_len).
  half8_t qf[KK];
  {
    const half_t* qp = q + (int64_t)(sq.q_start + (row_ok ? row : 0)) * q_st + (int64_t)h * q_sh + 8 * hh;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      qf[kk] = row_ok ? ld<half8_t>(qp + 16 * kk) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
  }

  const int64_t head_off = (int64_t)kvh * kBlockSize * D;
  const int64_t blk_stride = (int64_t)KVH * kBlockSize * D;
  const int* btrow = bt + (int64_t)b * bt_st;
  // Staging: wavefront w loads block w of the step. K: lane -> token lane / 4, dims
  // 32 (lane % 4) .. +31 (four 16-byte pieces). V: lane -> tokens {4 v + i, 8 + 4 v + i}
  // (v = lane / 32, i = 0..3), dims 4 (lane % 32) .. +3 (eight 8-byte pieces; 32 lanes cover a
  // token row): exactly the eight keys of V^T piece 2w + v, so each lane writes four whole
  // 16-byte pieces, one per dim.
  half8_t skA[4], skB[4];                         // two steps in flight (register double buffer)
  half4_t svA[8], svB[8];
  auto stage_load = [&](int st, half8_t (&sk)[4], half4_t (&sv)[8]) {
    int bi = st * 4 + w;
    bi = bi < nblk ? bi : nblk - 1;                // past the tile's keys: repeat (masked)
    const int64_t off = clamp_block(btrow[bi], NB) * blk_stride + head_off;
    const half_t* kp = kc + off + (lane >> 2) * D + 32 * (lane & 3);
#pragma unroll
    for (int i = 0; i < 4; ++i) sk[i] = ld<half8_t>(kp + 8 * i);
    const half_t* vp = vc + off + 4 * (lane >> 5) * D + 4 * (lane & 31);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sv[i] = ld<half4_t>(vp + i * D);
      sv[4 + i] = ld<half4_t>(vp + (8 + i) * D);
    }
  };
  auto stage_store = [&](int st, int buf, const half8_t (&sk)[4], const half4_t (&sv)[8]) {
    char* kb = lds + buf * L::STAGE;
    char* vb = kb + L::KBYTES;
    char* kd = kb + (16 * w + (lane >> 2)) * L::KROW + 64 * (lane & 3);
#pragma unroll
    for (int i = 0; i < 4; ++i) ts::st<half8_t>(kd + 16 * i, sk[i]);
    // V^T: the eight keys of this lane, transposed; keys at or past kv_hi are zeroed (a reused
    // block may hold NaN there, and 0 * NaN would reach the output).
    const int vv = lane >> 5;
    const int key0 = st * kTileKeys + 16 * w + 4 * vv;
    const half4_t z4 = {0, 0, 0, 0};
    half4_t x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = sv[i];
    if ((st + 1) * kTileKeys > kv_hi) {            // the tile's last step only
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[i] = key0 + i < kv_hi ? sv[i] : z4;
        x[4 + i] = key0 + 8 + i < kv_hi ? sv[4 + i] : z4;
      }
    }
    const int piece = 2 * w + vv;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 4 * (lane & 31) + j;
      const half8_t t8 = {x[0][j], x[1][j], x[2][j], x[3][j], x[4][j], x[5][j], x[6][j], x[7][j]};
      ts::st<half8_t>(vb + d * L::VROW + 16 * (piece ^ vt_swz(d)), t8);
    }
  };

  float16_t o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[t][e] = 0.f;
  float m = -INFINITY, l = 0.f;
  const int lim = sq.prefix + row < kv_hi - 1 ? sq.prefix + row : kv_hi - 1;   // last visible key

  auto compute = [&](int st, int buf) {
    const int k0 = st * kTileKeys;
    if (r0 >= sq.q_len || k0 > sq.prefix + r0 + 31) return;   // nothing visible to this wave
    const char* kb = lds + buf * L::STAGE;
    const char* vb = kb + L::KBYTES;
    // S^T for both key halves: the two MFMA chains alternate and the K operands of k-step
    // kk + 1 are requested before the MFMAs of k-step kk, so each LDS read has two MFMAs of
    // cover.
    float16_t s[2];
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int e = 0; e < 16; ++e) s[x][e] = 0.f;
    const char* kr0 = kb + r * L::KROW + 16 * hh;
    const char* kr1 = kr0 + 32 * L::KROW;
    half8_t ka[2][2];
    ka[0][0] = ld<half8_t>(kr0);
    ka[1][0] = ld<half8_t>(kr1);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if (kk + 1 < KK) {
        ka[0][(kk + 1) & 1] = ld<half8_t>(kr0 + 32 * (kk + 1));
        ka[1][(kk + 1) & 1] = ld<half8_t>(kr1 + 32 * (kk + 1));
      }
      s[0] = mfma32x32x16(ka[0][kk & 1], qf[kk], s[0]);
      s[1] = mfma32x32x16(ka[1][kk & 1], qf[kk], s[1]);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // the two reads ...
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);   // ... then the two MFMAs
    }
    if (k0 + kTileKeys - 1 > sq.prefix + r0) {     // diagonal or tail step: per-key mask
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = k0 + 32 * x + 8 * (e >> 2) + 4 * hh + (e & 3);
          s[x][e] = key <= lim ? s[x][e] : -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) mx = vmax(mx, vmax(s[0][e], s[1][e]));
    const float bm = pair_max(mx) * sl2;
    const bool move = bm > m + kRescaleLog2;       // m = -inf: the first visible key moves it
    if (__ballot(move) != 0) {
      const float alpha = move ? fast_exp2(m - bm) : 1.f;   // m = -inf -> 0
      l *= alpha;
      m = move ? bm : m;
#pragma unroll
      for (int t = 0; t < DT; ++t) o[t] *= alpha;
    }
    const float neg = m == -INFINITY ? 0.f : -m;   // rows with no visible key: every P is 0
    half8_t p[4];
    float ls = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float pv = fast_exp2(fmaf(s[u >> 1][8 * (u & 1) + i], sl2, neg));
        ls += pv;
        p[u][i] = (half_t)pv;
      }
    l += ls;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int t = 0; t < DT; ++t)
        o[t] = mfma32x32x16(
            ld<half8_t>(vb + (32 * t + r) * L::VROW + 16 * ((2 * u + hh) ^ vt_swz(32 * t + r))),
            p[u], o[t]);
  };

  // Step s sits in LDS buffer (s - lo) % 2 while the registers hold step s + 1 (loaded one
  // step earlier) and receive step s + 2. The loads are unconditional (past the range they
  // repeat its last step, a cache hit), so each wait covers exactly the registers it needs.
  if (tsl.lo < tsl.hi) {
    const int hi1 = tsl.hi - 1;
    stage_load(tsl.lo, skA, svA);
    stage_load(tsl.lo + 1 < hi1 ? tsl.lo + 1 : hi1, skB, svB);
    stage_store(tsl.lo, 0, skA, svA);
    __syncthreads();
    for (int st = tsl.lo; st < tsl.hi; st += 2) {
      stage_load(st + 2 < hi1 ? st + 2 : hi1, skA, svA);
      compute(st, 0);
      if (st + 1 < tsl.hi) stage_store(st + 1, 1, skB, svB);
      __syncthreads();
      if (st + 1 >= tsl.hi) break;
      stage_load(st + 3 < hi1 ? st + 3 : hi1, skB, svB);
      compute(st + 1, 1);
      if (st + 2 < tsl.hi) stage_store(st + 2, 0, skA, svA);
      __syncthreads();
    }
  }

  const float lt = pair_sum(l);
  if (!row_ok) return;
  if (tsl.nsplit == 1) {
    const float inv = lt == 0.f ? 0.f : 1.f / lt;
    half_t* op = out + (int64_t)(sq.q_start + row) * o_st + (int64_t)h * D + 4 * hh;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const half4_t v4 = {(half_t)(o[t][4 * j] * inv), (half_t)(o[t][4 * j + 1] * inv),
                            (half_t)(o[t][4 * j + 2] * inv), (half_t)(o[t][4 * j + 3] * inv)};
        ts::st<half4_t>(op + 32 * t + 8 * j, v4);
      }
  } else {
    // Partial of this split: the row's O and (m, l), all fp32, as the reference keeps a
    // split's state (ops/triton_decode_attention.py:190-192).
    const int64_t wslot = ((int64_t)pi * H + h) * slots + slot;
    const int64_t total = (int64_t)P * H * slots;
    float* wo = ws + (wslot * kTileRows + 32 * w + r) * D + 4 * hh;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        ts::st<float4_t>(wo + 32 * t + 8 * j,
                         float4_t{o[t][4 * j], o[t][4 * j + 1], o[t][4 * j + 2], o[t][4 * j + 3]});
    if (hh == 0) {
      float* wml = ws + total * kTileRows * D + (wslot * kTileRows + 32 * w + r) * 2;
      wml[0] = m;
      wml[1] = lt;
    }
  }
}

template <int D>
__global__ void __launch_bounds__(kTileThreads, 2) prefill_tile_kernel(
    const half_t* __restrict__ q, int64_t q_st, int64_t q_sh, half_t* __restrict__ out,
    int64_t o_st, int64_t num_tokens, const half_t* __restrict__ kc,
    const half_t* __restrict__ vc, int64_t NB, const int* __restrict__ bt, int64_t bt_st,
    int max_blocks, const int* __restrict__ seq_lens, const int* __restrict__ qsl,
    int num_decode, int H, int KVH, float sl2, int smax, int slots, int P,
    float* __restrict__ ws) {
  __shared__ __attribute__((aligned(16))) char lds[2 * TileLayout<D>::STAGE];
  prefill_tile_body<D>(q, q_st, q_sh, out, o_st, num_tokens, kc, vc, NB, bt, bt_st, max_blocks,
                       seq_lens, qsl, num_decode, H, KVH, sl2, smax, slots, P, ws,
                       (int)blockIdx.x, lds);
}

// Merge of split partials (each the split's fp32 (O_j, m_j, l_j), O_j unnormalised):
// M = max m_j, w_j = 2^(m_j - M), out = sum w_j O_j / sum w_j l_j (empty splits have m = -inf and
// weigh 0). A thread owns 8 dims (d0, two 16-byte loads per partial row) of kMergeRows rows; the
// partials sit at slot indices base .. base + cnt - 1 of a workspace of total_slots slots x
// slot_rows rows, the thread's rows at row0 + kMergeRowStride * k of each slot, and go to dst[k]
// (nullptr: not wanted). The partials are taken kMergeBatch at a time, all of a batch's loads
// requested together (cnt is uniform over the workgroup, so the unused ones are not issued).
constexpr int kMergeRowStride = kTileThreads / 16;   // 16 rows per pass of a 256-thread group
constexpr int kMergeBatch = 4;

template <int D>
__device__ __forceinline__ void merge_partials(const float* __restrict__ ws, int64_t total_slots,
                                               int slot_rows, int64_t base, int cnt, int row0,
                                               int d0, half_t* const (&dst)[kMergeRows]) {
  constexpr int NR = kMergeRows;
  constexpr int RG = kMergeRowStride;
  constexpr int B = kMergeBatch;
  const float* wo = ws;
  const float* wml = ws + total_slots * slot_rows * D;
  float M[NR], Lsum[NR], acc[NR][8];
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    M[k] = -INFINITY;
    Lsum[k] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[k][e] = 0.f;
  }
  for (int j = 0; j < cnt; j += B) {
    float2_t ml[B][NR];
    float4_t a[B][NR][2];
#pragma unroll
    for (int u = 0; u < B; ++u)
#pragma unroll
      for (int k = 0; k < NR; ++k) {
        if (j + u < cnt) {
          const int64_t rix = (base + j + u) * slot_rows + row0 + RG * k;
          ml[u][k] = ld<float2_t>(wml + rix * 2);
          a[u][k][0] = ld<float4_t>(wo + rix * D + d0);
          a[u][k][1] = ld<float4_t>(wo + rix * D + d0 + 4);
        } else {
          ml[u][k] = float2_t{-INFINITY, 0.f};
          a[u][k][0] = float4_t{0.f, 0.f, 0.f, 0.f};
          a[u][k][1] = float4_t{0.f, 0.f, 0.f, 0.f};
        }
      }
#pragma unroll
    for (int k = 0; k < NR; ++k) {
      float cm = M[k];
#pragma unroll
      for (int u = 0; u < B; ++u) cm = fmaxf(cm, ml[u][k][0]);
      const float alpha = M[k] == -INFINITY ? 0.f : fast_exp2(M[k] - cm);
      Lsum[k] *= alpha;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[k][e] *= alpha;
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const float mu = ml[u][k][0];
        const float wt = mu == -INFINITY ? 0.f : fast_exp2(mu - cm);
        Lsum[k] += wt * ml[u][k][1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[k][e] += wt * a[u][k][0][e];
          acc[k][e + 4] += wt * a[u][k][1][e];
        }
      }
      M[k] = cm;
    }
  }
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    if (dst[k] == nullptr) continue;
    const float inv = Lsum[k] == 0.f ? 0.f : 1.f / Lsum[k];
    half4_t o0, o1;                              // two 8-byte stores: out rows are 8-byte aligned
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o0[e] = (half_t)(acc[k][e] * inv);
      o1[e] = (half_t)(acc[k][e + 4] * inv);
    }
    ts::st<half4_t>(dst[k], o0);
    ts::st<half4_t>(dst[k] + 4, o1);
  }
}

// Merge of the 4-wavefront tile kernel's split tiles (the mixed-step kernel's prefill part).
// Grid (4 * tiles, P, H): workgroup (4 i + q) merges rows 32q .. 32q+31 of tile i if it was split;
// partials are slot-major per (sequence, head), kTileRows rows per slot.
template <int D>
__device__ __forceinline__ void prefill_merge_body(
    const float* __restrict__ ws, half_t* __restrict__ out, int64_t o_st, int64_t num_tokens,
    int max_blocks, const int* __restrict__ seq_lens, const int* __restrict__ qsl,
    int num_decode, int H, int smax, int slots, int P, int bx, int by, int bz, int tile_stride) {
  constexpr int TPR = D / 8;                       // threads per row
  constexpr int RG = kMergeRowStride;              // row groups per workgroup (16)
  constexpr int NR = kMergeRows;                   // rows per thread
  static_assert(RG * NR * 4 == kTileRows && TPR * RG == kTileThreads, "four workgroups per tile");
  const int part = bx & 3;
  const int b = num_decode + by, h = bz;
  const PrefillSeq sq = prefill_seq(qsl, seq_lens, b, num_tokens, max_blocks);
  const int rbase = part * RG * NR + (int)(threadIdx.x / TPR);   // rows rbase + RG * k
  const int d0 = 8 * (int)(threadIdx.x % TPR);
  const int64_t total = (int64_t)P * H * slots;
  // The grid covers the tiles the host bounds foresee; a sequence with more (bounds below its
  // real q_len) has its further tiles taken in turn, so every tile whose splits all ran is
  // merged (the tile kernel fills the rows of the others with NaN).
  for (int tile = bx >> 2; tile * kTileRows < sq.q_len; tile += tile_stride) {
    if (tile * kTileRows + rbase >= sq.q_len) continue;
    const int2_t span = tile_span(tile, sq.q_len, sq.prefix, sq.seq_len, smax, kTileRows);
    const int slot = span[0], nsplit = span[1];
    if (nsplit <= 1 || slot + nsplit > slots) continue;   // unsplit, or splits past the launch
    half_t* dst[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) {
      const int row = tile * kTileRows + rbase + RG * k;
      dst[k] = row < sq.q_len ? out + (int64_t)(sq.q_start + row) * o_st + (int64_t)h * D + d0
                              : nullptr;
    }
    merge_partials<D>(ws, total, kTileRows, ((int64_t)by * H + h) * slots + slot, nsplit, rbase,
                      d0, dst);
  }
}

template <int D>
__global__ void __launch_bounds__(kTileThreads) prefill_merge_kernel(
    const float* __restrict__ ws, half_t* __restrict__ out, int64_t o_st, int64_t num_tokens,
    int max_blocks, const int* __restrict__ seq_lens, const int* __restrict__ qsl,
    int num_decode, int H, int smax, int slots) {
  prefill_merge_body<D>(ws, out, o_st, num_tokens, max_blocks, seq_lens, qsl, num_decode, H, smax,
                        slots, (int)gridDim.y, (int)blockIdx.x, (int)blockIdx.y,
                        (int)blockIdx.z, (int)gridDim.x / 4);
}

// Host-side plan of the 4-wavefront tiled path: the most steps one split may take (smax) and the
// launch slots per (sequence, head), from host bounds of the batch (max_query_len, max_seq_len).
struct TilePlan {
  int smax, slots;
  size_t ws_bytes;
  int64_t est_wg;     // workgroups with work, estimated from the host bounds
};

inline int cdiv(int a, int b) { return (a + b - 1) / b; }

inline TilePlan tile_plan(int P, int H, int D, int max_query_len, int max_seq_len, int cu_count,
                          bool split, int64_t round = 0) {
  const int tiles = cdiv(max_query_len, kTileRows);
  const int seq = max_seq_len > max_query_len ? max_seq_len : max_query_len;
  const int nmax = cdiv(seq, kTileKeys);           // most steps any tile can have
  TilePlan pl{nmax > 0 ? nmax : 1, tiles, 0, (int64_t)tiles * P * H};
  if (!split || nmax <= 1) return pl;
  // Workgroups of the batch for a given smax, as if every sequence had the longest chunk on the
  // longest prefix (the tiles' step counts n_i then follow from the host bounds).
  const int prefix = seq - max_query_len;
  auto workgroups = [&](int smax) {
    int64_t n_wg = 0;
    for (int i = 0; i < tiles; ++i) {
      const int hi = prefix + ((i + 1) * kTileRows < max_query_len ? (i + 1) * kTileRows : max_query_len);
      const int n = cdiv(hi, kTileKeys);
      n_wg += n <= smax ? 1 : cdiv(n, smax);
    }
    return n_wg * P * H;
  };
  // Every split tile must run in the first round of resident workgroups (two per CU, or the
  // `round` a caller leaves to this kernel): a second, partial round would leave most of the
  // device idle while it runs. So take the smallest smax whose workgroups fit one round; if the
  // unsplit tiles already fill it, do not split.
  if (round <= 0) round = 2 * (int64_t)(cu_count > 0 ? cu_count : 256);
  if (workgroups(nmax) >= round) return pl;
  int smax = kPrefillMinSteps;
  while (smax < nmax && workgroups(smax) > round) ++smax;
  if (smax >= nmax) return pl;
  pl.smax = smax;
  pl.est_wg = workgroups(smax);
  pl.slots = tiles * cdiv(nmax, smax);
  pl.ws_bytes = (size_t)P * H * pl.slots * kTileRows * (D + 2) * sizeof(float);
  return pl;
}

}  // namespace ts
