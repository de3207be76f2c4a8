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
#pragma once

#include <math.h>

#include <type_traits>

#include "common.h"
#include "paged_kv.h"
#include "rope.h"
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
// Dense split map of v3. Sequence s has nb_s = ceil(len_s / 16) blocks (len_s clamped to
// cap_blocks * 16) cut into n_s = ceil(nb_s / P_s) splits of P_s blocks; the splits of the batch
// are numbered densely in sequence order (split j of sequence s is launch slot C_s + j with
// C_s = sum_{t<s} n_t), so the busy workgroups come first in the launch. With a caller
// partition, P_s = partition. With part_blocks == 0 (the default, own-length schedule) a
// sequence is cut into n = min(max_splits, ceil(nb_s / kOwnPartBlocks)) splits of equal size,
// P_s = ceil(nb_s / n) rounded up to a multiple of kMinPartBlocks (one pair per wavefront, so
// every wavefront of a full split gets the same number of pairs). Either way a sequence's split
// boundaries depend on its own length only, as in the reference's fixed grid
// (ops/triton_ops.py:47-53), so a row's result does not depend on the rest of the batch.
// Split j of sequence s leaves its partial in workspace row s * max_splits + j, so the merge
// can request a sequence's partials without knowing the other sequences' lengths.
constexpr int kMinPartBlocks = 8;
constexpr int kOwnPartBlocks = 24;           // the own-length schedule's longest split (blocks)
constexpr int kOwnMaxSplits = 32;

struct SplitSlot {
  int seq;     // sequence owning the slot (-1: the slot is past the batch's last split)
  int first;   // C_s
  int count;   // n_s
  int part;    // P_s in blocks
  int len;     // clamped seq_len
};

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ int wave_inclusive_sum(int v, int lane) {
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int t = __shfl_up(v, d, kWave);
    if (lane >= d) v += t;
  }
  return v;
}

__device__ __forceinline__ int round_part(int blocks) {
  return (blocks + kMinPartBlocks - 1) / kMinPartBlocks * kMinPartBlocks;
}

// Splits of a sequence of nb blocks cut into ps-block pieces: a sequence with no blocks (a
// padding row, seq_len 0) still gets one split, whose workgroup writes the row's zeros.
__device__ __forceinline__ int split_count(int nb, int ps) { return nb > 0 ? (nb + ps - 1) / ps : 1; }

// P_s of a sequence of nb blocks: the caller's partition P, or (P <= 0, the own-length
// schedule) nb cut into min(max_splits, ceil(nb / kOwnPartBlocks)) near-equal splits.
__device__ __forceinline__ int seq_part(int P, int nb, int max_splits) {
  if (P > 0) return P;
  int n = (nb + kOwnPartBlocks - 1) / kOwnPartBlocks;
  n = n < 1 ? 1 : (n > max_splits ? max_splits : n);
  const int ps = round_part((nb + n - 1) / n);
  return ps > kMinPartBlocks ? ps : kMinPartBlocks;
}

// Called by every thread of an NT-thread workgroup (S >= 1): finds the sequence that owns
// launch slot `slot`. s_map holds NT / 64 + 5 ints of LDS.
template <int NT>
__device__ SplitSlot split_lookup(const int* __restrict__ seq_lens, int S, int cap_blocks,
                                  int part_blocks, int max_splits, int slot, int* s_map) {
  constexpr int NWV = NT / kWave;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int cap = cap_blocks * kBlockSize;
  auto clamp_len = [&](int len) { return len < 0 ? 0 : (len > cap ? cap : len); };
  const int len0 = tid < S ? clamp_len(seq_lens[tid]) : 0;
  if (tid == 0) {
    s_map[NWV] = -1;
    s_map[NWV + 1] = 0;
    s_map[NWV + 2] = 0;
    s_map[NWV + 3] = 0;
    s_map[NWV + 4] = part_blocks;
  }
  int base = 0;
  for (int c0 = 0; c0 < S; c0 += NT) {
    const int i = c0 + tid;
    const int len = c0 == 0 ? len0 : (i < S ? clamp_len(seq_lens[i]) : 0);
    const int nb = (len + kBlockSize - 1) / kBlockSize;
    const int ps = seq_part(part_blocks, nb, max_splits);
    const int n = i < S ? split_count(nb, ps) : 0;
    const int incl = wave_inclusive_sum(n, lane);
    if (lane == kWave - 1) s_map[w] = incl;
    __syncthreads();
    int off = base, tot = 0;
#pragma unroll
    for (int k = 0; k < NWV; ++k) {
      const int v = s_map[k];
      off += k < w ? v : 0;
      tot += v;
    }
    const int excl = off + incl - n;
    if (i < S && slot >= excl && slot < excl + n) {
      s_map[NWV] = i;
      s_map[NWV + 1] = excl;
      s_map[NWV + 2] = n;
      s_map[NWV + 3] = len;
      s_map[NWV + 4] = ps;
    }
    base += tot;
    __syncthreads();
  }
  return {__builtin_amdgcn_readfirstlane(s_map[NWV]), __builtin_amdgcn_readfirstlane(s_map[NWV + 1]),
          __builtin_amdgcn_readfirstlane(s_map[NWV + 2]), __builtin_amdgcn_readfirstlane(s_map[NWV + 4]),
          __builtin_amdgcn_readfirstlane(s_map[NWV + 3])};
}

// Per-step split map: the result of split_lookup for every launch slot, plus the block ids its
// wavefronts request first, built once per step by decode_split_map_kernel and read by every
// layer's v3 launch in place of split_lookup (the layers of a step share seq_lens, the block
// tables and the plan). A workgroup then issues its first K/V requests one scalar load after it
// starts instead of after a seq_lens load, a block-wide scan and a block-table load. Layout
// (int32): a header of kMapHeader ints {kMapMagic, S, slots, part_blocks, 0, max_splits,
// cap_blocks, 0} naming the plan it was built for (a launch whose plan differs ignores the map
// and runs split_lookup), then kMapEntry ints per slot: {seq (-1: past the last split), C_s,
// n_s, clamped seq_len, first block, end block, block id of the sequence's last token, P_s}
// and the block ids of pairs 0 .. kMapPairs - 1 of the split as blk_id gives them to the
// wavefronts' first loads (a pair past the range repeats the id its wavefront falls back to).
constexpr int kMapMagic = 0x314d5354;
constexpr int kMapHeader = 8;
constexpr int kMapEntry = 32;
constexpr int kMapPairs = 8;                 // two pairs per wavefront of a 4-wavefront launch
constexpr int kMapMaxSeqs = 4096;            // sequences per step the builder handles
constexpr int kMapThreads = 256;
constexpr int kMapMaxGroups = 64;            // workgroups of the builder (each kMapThreads slots)

__device__ __forceinline__ int4 int4_of(int a, int b, int c, int d) { return int4{a, b, c, d}; }

template <int NT>
__global__ void __launch_bounds__(NT) decode_split_map_kernel(
    const int* __restrict__ seq_lens, const int* __restrict__ bt, int64_t bt_st, int64_t NB,
    int S, int cap_blocks, int part_blocks, int max_splits, int nslots, int n_counters,
    int* __restrict__ map) {
  constexpr int NWV = NT / kWave;
  __shared__ int s_first[kMapMaxSeqs];
  __shared__ int s_len[kMapMaxSeqs];
  __shared__ int s_part[kMapMaxSeqs];
  __shared__ int s_red[NWV];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int cap = cap_blocks * kBlockSize;
  for (int i = tid; i < S; i += NT) {
    int len = seq_lens[i];
    len = len < 0 ? 0 : (len > cap ? cap : len);
    s_len[i] = len;
  }
  __syncthreads();                             // s_len complete
  int base = 0;
  for (int c0 = 0; c0 < S; c0 += NT) {         // exclusive prefix of the split counts
    const int i = c0 + tid;
    int n = 0;
    if (i < S) {
      const int nb = (s_len[i] + kBlockSize - 1) / kBlockSize;
      const int ps = seq_part(part_blocks, nb, max_splits);
      s_part[i] = ps;
      n = split_count(nb, ps);
    }
    const int incl = wave_inclusive_sum(n, lane);
    if (lane == kWave - 1) s_red[w] = incl;
    __syncthreads();
    int off = base, tot = 0;
#pragma unroll
    for (int k = 0; k < NWV; ++k) {
      const int v = s_red[k];
      off += k < w ? v : 0;
      tot += v;
    }
    if (i < S) s_first[i] = off + incl - n;
    base += tot;
    __syncthreads();
  }
  // the arrival counters of the split kernel's in-launch merge start at zero (each merge resets
  // its counter, so the map stays valid for every layer of the step)
  int* counters = map + kMapHeader + (int64_t)nslots * kMapEntry;
  if (blockIdx.x == 0) {
    for (int i = tid; i < n_counters; i += NT) counters[i] = 0;
    if (tid == 0) {
      int4* h = reinterpret_cast<int4*>(map);
      h[0] = int4_of(kMapMagic, S, nslots, part_blocks);
      h[1] = int4_of(0, max_splits, cap_blocks, 0);
    }
  }
  // Every workgroup computed the prefix above; the slots are shared among them.
  constexpr int NWF = kMapPairs / 2;           // wavefronts of the consuming launch
  for (int slot = blockIdx.x * NT + tid; slot < nslots; slot += gridDim.x * NT) {
    int lo = 0, hi = S - 1;                    // last sequence whose first split is <= slot
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_first[mid] <= slot) lo = mid;
      else hi = mid - 1;
    }
    const int i = lo, len = s_len[i], ps = s_part[i];
    const int nb = (len + kBlockSize - 1) / kBlockSize;
    const int n = split_count(nb, ps);
    int4* dst = reinterpret_cast<int4*>(map + kMapHeader + (int64_t)slot * kMapEntry);
    const int j = slot - s_first[i];
    if (j >= n) {                              // past the batch's last split
      dst[0] = int4_of(-1, 0, 0, 0);
#pragma unroll
      for (int k = 1; k < kMapEntry / 4; ++k) dst[k] = int4_of(0, 0, 0, 0);
      continue;
    }
    const int* btrow = bt + (int64_t)i * bt_st;
    const int blk_lo = j * ps;
    const int blk_hi = blk_lo + ps < nb ? blk_lo + ps : nb;
    const int npairs = (blk_hi - blk_lo + 1) >> 1;
    int ids[2 * kMapPairs];
#pragma unroll
    for (int q = 0; q < kMapPairs; ++q) {
      const int qq = q < npairs ? q : (q >= NWF ? q - NWF : q);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        int bi = blk_lo + 2 * qq + h;
        bi = bi < blk_hi ? bi : blk_hi - 1;
        ids[2 * q + h] = nb > 0 ? clamp_block(btrow[bi], NB) : 0;   // no blocks: nothing read
      }
    }
    const int last = len > 0 ? clamp_block(btrow[(len - 1) / kBlockSize], NB) : 0;
    dst[0] = int4_of(i, s_first[i], n, len);
    dst[1] = int4_of(blk_lo, blk_hi, last, ps);
#pragma unroll
    for (int k = 0; k < kMapPairs / 2; ++k)
      dst[2 + k] = int4_of(ids[4 * k], ids[4 * k + 1], ids[4 * k + 2], ids[4 * k + 3]);
#pragma unroll
    for (int k = 2 + kMapPairs / 2; k < kMapEntry / 4; ++k) dst[k] = int4_of(0, 0, 0, 0);
  }
}

// One workgroup = NW wavefronts = one (split slot, KV head, head group) in v3 or one (sequence,
// KV head, head group) in v2 (ws_acc == nullptr). The blocks of the range are consumed in pairs,
// pair p by wavefront p % NW: two S^T chains, one online-softmax step per 32 tokens and the P.V
// product as v_mfma_f32_16x16x32_f16 over the pair. Each wavefront keeps the next pair's loads in
// flight while it multiplies the current one (with KDMA the next two pairs', K through a ring in
// LDS); block-table entries are wave-uniform scalar loads issued a pair further ahead, so they
// never wait behind the K/V vector loads. The wavefronts
// merge their (m, l, acc) in LDS; a sequence with one split writes its output here, otherwise
// the split's partial goes to the workspace for decode_merge_kernel.
// LDS of one decode workgroup: per-wavefront O^T rows, m and l, and the split lookup's scratch.
template <int D, int NW>
struct DecodeLds {
  static constexpr int OROW = D + 4;
  static constexpr int M = NW * 16 * OROW * 4;
  static constexpr int L = M + NW * 16 * 4;
  static constexpr int MAP = L + NW * 16 * 4;
  static constexpr int BYTES = MAP + (NW + 5) * 4;
};

// The step's new K/V rows (one per decode row), for the launch that also performs kv_write
// (and, with cos_t set, the RoPE of q and of the new k rows first).
struct NewRows {
  const half_t* k;
  const half_t* v;
  int64_t k_st, k_sh, v_st, v_sh;
  const int64_t* slots;     // slot_mapping [S] (-1: padding row, not written)
  int64_t num_slots;        // NB * 16: slots at or past it are not written (as kv_write)
  // RoPE (ops/triton_rope.py:10-31): row s of q and k rotated at positions[s] with the fp32
  // tables [max_pos, D / 2]; qkv / qkv_st / H describe the packed rows for the host's fallback.
  const int64_t* positions;
  const float* cos_t;
  const float* sin_t;
  int64_t max_pos;
  void* qkv;
  int64_t qkv_st;
};

template <int D, int NW, bool WRITE = false, bool ROPE = false, bool KDMA = false>
__device__ __forceinline__ void decode_mfma_body(
    const half_t* __restrict__ q, int64_t q_st, int64_t q_sh, half_t* __restrict__ out,
    int64_t o_st, const half_t* __restrict__ kc, const half_t* __restrict__ vc, int64_t NB,
    const int* __restrict__ bt, int64_t bt_st, int max_blocks, const int* __restrict__ seq_lens,
    int S, int H, int KVH, int G, int HG, float sl2, int cap_blocks, int part_blocks,
    int max_splits, float* __restrict__ ws_acc, float* __restrict__ ws_m,
    float* __restrict__ ws_l, int* __restrict__ ws_cnt,
    int bx, int bz, char* __restrict__ lds, const NewRows& nr = NewRows{},
    int* __restrict__ smap = nullptr, int nslots = 0, half8_t* kr0 = nullptr,
    half8_t* kr1 = nullptr) {
  constexpr int KK = KvRegs<D>::KK;
  constexpr int VW = KvRegs<D>::VW;
  constexpr int TILES = KvRegs<D>::TILES;
  constexpr int OROW = D + 4;                    // padded LDS row (floats) against bank conflicts
  typedef typename HalfVec<VW>::type VRow;
  float (*s_o)[16][OROW] = reinterpret_cast<float (*)[16][OROW]>(lds);
  float (*s_m)[16] = reinterpret_cast<float (*)[16]>(lds + DecodeLds<D, NW>::M);
  float (*s_l)[16] = reinterpret_cast<float (*)[16]>(lds + DecodeLds<D, NW>::L);
  int* s_map = reinterpret_cast<int*>(lds + DecodeLds<D, NW>::MAP);

  const int kvh = bz / HG, hg = bz % HG;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int hq = hg * 16 + c;                    // query head within the GQA group
  const bool head_ok = hq < G;
  const int nh = (G - hg * 16) < 16 ? (G - hg * 16) : 16;   // real heads in this group
  const int head0 = kvh * G + hg * 16;           // first query head of this group
  const bool split = ws_acc != nullptr;

  int s, seq_len, blk_lo, blk_hi, nsplit, split_j = 0;
  // With a split map built for this launch's plan (header equal to the plan; smap is only
  // passed by decode_mfma_kernel, with its slot count nslots) the slot's entry replaces
  // split_lookup, and the first two pairs' block ids of this wavefront come with it. The header
  // and the entry are requested together (the host checked that the map holds every slot).
  bool mapped = false;
  int m_last = 0, m_id[4] = {0, 0, 0, 0};
  SplitSlot sp{-1, 0, 0, 0, 0};
  if constexpr (2 * NW == kMapPairs) {
    if (split && smap != nullptr) {
      const int* e = smap + kMapHeader + (int64_t)bx * kMapEntry;
      mapped = smap[0] == kMapMagic && smap[1] == S && smap[2] == nslots &&
               smap[3] == part_blocks && smap[5] == max_splits &&
               smap[6] == cap_blocks;
      sp = {e[0], e[1], e[2], e[7], e[3]};
      m_last = e[6];
      m_id[0] = e[8 + 2 * w];
      m_id[1] = e[9 + 2 * w];
      m_id[2] = e[8 + 2 * (w + NW)];
      m_id[3] = e[9 + 2 * (w + NW)];
    }
  }
  if (split) {
    if (!mapped)
      sp = split_lookup<NW * 64>(seq_lens, S, cap_blocks, part_blocks, max_splits, bx, s_map);
    if (sp.seq < 0) return;                      // slot past the batch's last split
    s = sp.seq;
    seq_len = sp.len;
    nsplit = sp.count;
    split_j = bx - sp.first;
    if (smap != nullptr && !mapped) {
      // A map whose header names another plan: the launch has no merge kernel after it (the
      // map's workgroups merge in-launch), so the rows are poisoned, loudly, not attended.
      if (split_j == 0)
        for (int e = tid; e < nh * D; e += NW * 64)
          out[(int64_t)s * o_st + (int64_t)(head0 + e / D) * D + e % D] = (half_t)__builtin_nanf("");
      return;
    }
    if (split_j == 0 && tid == 0) ws_cnt[s] = nsplit;   // read by the merge kernel
    if (seq_len == 0) {                          // padding row: zeros (ops/reference.py:99,104-105)
      for (int e = tid; e < nh * D; e += NW * 64)
        out[(int64_t)s * o_st + (int64_t)(head0 + e / D) * D + e % D] = (half_t)0.f;
      return;
    }
    const int nblk = (seq_len + kBlockSize - 1) / kBlockSize;
    blk_lo = split_j * sp.part;
    blk_hi = (blk_lo + sp.part) < nblk ? (blk_lo + sp.part) : nblk;
  } else {
    s = bx;
    seq_len = seq_lens[s];
    seq_len = seq_len < 0 ? 0 : (seq_len > max_blocks * kBlockSize ? max_blocks * kBlockSize : seq_len);
    seq_len = __builtin_amdgcn_readfirstlane(seq_len);
    nsplit = 1;
    blk_lo = 0;
    blk_hi = (seq_len + kBlockSize - 1) / kBlockSize;
    if (seq_len == 0) {                          // padding row: zeros (ops/reference.py:99,104-105)
      for (int e = tid; e < nh * D; e += NW * 64)
        out[(int64_t)s * o_st + (int64_t)(head0 + e / D) * D + e % D] = (half_t)0.f;
      return;
    }
  }
  bool poison = false;                           // fused write with a non-conforming slot
  if constexpr (WRITE) {
    // kv_write of sequence s's new row (ops/reference.py:50-57) for this KV head, by the
    // workgroup whose range ends the sequence (it holds position seq_len - 1, where every input
    // builder puts slot_mapping[s]; the launch has one head group per KV head, so no other
    // workgroup reads that block). The rows are stored before any wavefront requests K/V:
    // the stores complete in L2 (vmcnt 0) before the barrier, and no wavefront of this CU has
    // requested those lines in this kernel, so the loads after it see the new row. The cache
    // pointers are the same restrict pointers the loads use, so the compiler orders them too.
    if (split_j == nsplit - 1) {
      const int64_t slot = nr.slots[s];
      // The precondition of the fusion: the slot is that of position seq_len - 1. Any other
      // slot would put the row in a block another workgroup may be reading; it is not written,
      // and the sequence's output becomes NaN so the caller sees the broken precondition.
      const int last_blk =
          mapped ? m_last
                 : clamp_block(table_entry(bt + (int64_t)s * bt_st + (seq_len - 1) / kBlockSize), NB);
      const int64_t want = (int64_t)last_blk * kBlockSize + (seq_len - 1) % kBlockSize;
      poison = slot >= 0 && slot < nr.num_slots && slot != want;
      if (slot >= 0 && slot < nr.num_slots && !poison) {
        const int64_t row = (((slot >> 4) * KVH + kvh) * kBlockSize + (slot & 15)) * D;
        const half_t* ksrc = nr.k + (int64_t)s * nr.k_st + (int64_t)kvh * nr.k_sh;
        const half_t* vsrc = nr.v + (int64_t)s * nr.v_st + (int64_t)kvh * nr.v_sh;
        constexpr int PIECES = D / 8;              // 16-byte pieces per row
        constexpr int PK = ROPE ? D / 16 : PIECES; // threads writing K (with RoPE: 8 frequencies)
        if (tid < PK) {
          if constexpr (ROPE) {
            // frequencies 8 tid .. 8 tid + 7: dims d0.. of the first half and d0 + D/2.. of the
            // second, rotated as rope_kv_write_kernel rotates them
            const int d0 = 8 * tid;
            const float* cp = nr.cos_t + rope_row(nr.positions[s], nr.max_pos) * (D / 2) + d0;
            const float* sp = nr.sin_t + (cp - nr.cos_t);
            const half8_t x1 = ld<half8_t>(ksrc + d0), x2 = ld<half8_t>(ksrc + D / 2 + d0);
            half4_t o1a, o2a, o1b, o2b;
            rope4(lo4(x1), lo4(x2), ld<float4_t>(cp), ld<float4_t>(sp), o1a, o2a);
            rope4(hi4(x1), hi4(x2), ld<float4_t>(cp + 4), ld<float4_t>(sp + 4), o1b, o2b);
            half_t* krow = const_cast<half_t*>(kc) + row;
            st<half8_t>(krow + d0, half8_t{o1a[0], o1a[1], o1a[2], o1a[3], o1b[0], o1b[1], o1b[2], o1b[3]});
            st<half8_t>(krow + D / 2 + d0,
                        half8_t{o2a[0], o2a[1], o2a[2], o2a[3], o2b[0], o2b[1], o2b[2], o2b[3]});
          } else {
            st<half8_t>(const_cast<half_t*>(kc) + row + 8 * tid, ld<half8_t>(ksrc + 8 * tid));
          }
        } else if (tid < PK + PIECES) {
          const int pc = tid - PK;
          st<half8_t>(const_cast<half_t*>(vc) + row + 8 * pc, ld<half8_t>(vsrc + 8 * pc));
        }
      }
      __builtin_amdgcn_s_waitcnt(kWaitVmcntZero);
      __syncthreads();
    }
  }
  // Tokens this range may use: a pair's second block can lie past the range (it then repeats
  // the range's last block, a cache hit) while its tokens are still below seq_len.
  const int tok_hi = blk_hi * kBlockSize < seq_len ? blk_hi * kBlockSize : seq_len;
  const int npairs = (blk_hi - blk_lo + 1) >> 1;
  const int* btrow = bt + (int64_t)s * bt_st;
  auto blk_id = [&](int p, int j) {
    int bi = blk_lo + 2 * p + j;
    bi = bi < blk_hi ? bi : blk_hi - 1;
    return clamp_block(table_entry(btrow + bi), NB);
  };

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
    if constexpr (ROPE) {
      // q rotated in registers, as rope_kernel rotates it in memory: lane (c, g) holds dims
      // 32 kk + 8 g .. + 7, and dims d and d + D / 2 (kk and kk + KK / 2) are a rotation pair.
      static_assert(KK % 2 == 0, "RoPE pairs must sit in one lane (head_dim a multiple of 64)");
      const int64_t trow = rope_row(nr.positions[s], nr.max_pos) * (D / 2);
#pragma unroll
      for (int kk = 0; kk < KK / 2; ++kk) {
        const float* cp = nr.cos_t + trow + 32 * kk + 8 * g;
        const float* sp = nr.sin_t + trow + 32 * kk + 8 * g;
        half4_t o1a, o2a, o1b, o2b;
        rope4(lo4(qf[kk]), lo4(qf[kk + KK / 2]), ld<float4_t>(cp), ld<float4_t>(sp), o1a, o2a);
        rope4(hi4(qf[kk]), hi4(qf[kk + KK / 2]), ld<float4_t>(cp + 4), ld<float4_t>(sp + 4), o1b,
              o2b);
        qf[kk] = half8_t{o1a[0], o1a[1], o1a[2], o1a[3], o1b[0], o1b[1], o1b[2], o1b[3]};
        qf[kk + KK / 2] = half8_t{o2a[0], o2a[1], o2a[2], o2a[3], o2b[0], o2b[1], o2b[2], o2b[3]};
      }
    }
  }
  const float4_t zero4 = {0.f, 0.f, 0.f, 0.f};
  float4_t o[TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t) o[t] = zero4;
  float m = -INFINITY, l = 0.f;

  const int64_t head_off = (int64_t)kvh * kBlockSize * D;
  const int64_t blk_stride = (int64_t)KVH * kBlockSize * D;
  // Two pipelines. KDMA (decode_mfma_kernel at D = 128 without RoPE, and the ragged launch): K
  // of two pairs in a per-wavefront LDS ring filled by LDS DMA, V of two pairs in registers, so
  // each pair's K and V are requested two pairs ahead. Otherwise: K of one pair in registers
  // (refilled for the next pair as soon as the S^T MFMAs have consumed it) and V of two pairs
  // (the next pair's V is requested a whole iteration before its P.V product). Either form keeps
  // the kernel at two wavefronts per SIMD at D = 128; the remaining latency is hidden by the
  // other resident wavefronts. The refills are unconditional (past a wavefront's last pair they
  // repeat its current pair, a cache hit) so every iteration has the same loads in flight and
  // each wait covers exactly what it needs. Block-table entries are scalar loads issued two
  // pairs ahead.
  auto load_k = [&](const int (&id)[2], half8_t (&kf)[2][KK]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) load_k_block<D>(kc + id[j] * blk_stride + head_off, c, g, kf[j]);
  };
  auto load_v = [&](const int (&id)[2], VRow (&vr)[2][4]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) load_v_rows<D>(vc + id[j] * blk_stride + head_off, c, g, vr[j]);
  };
  auto ids_of = [&](int pp, int (&id)[2]) {
    id[0] = blk_id(pp, 0);
    id[1] = blk_id(pp, 1);
  };

  auto last_or = [&](int pp, int fallback) { return pp < npairs ? pp : fallback; };
  // A map built for another step (other lengths or block tables, same plan) poisons the rows
  // it would attend wrongly: the entry's clamped length and last block must be this step's.
  // These loads follow the first K/V requests, off their critical path.
  auto stale = [&]() {
    const int cap = cap_blocks * kBlockSize;
    int cur = seq_lens[s];
    cur = cur < 0 ? 0 : (cur > cap ? cap : cur);
    const int cur_last = clamp_block(table_entry(btrow + (seq_len - 1) / kBlockSize), NB);
    return cur != seq_len || cur_last != m_last;
  };
  if constexpr (KDMA) {
    static_assert(D == 128, "LDS-staged K: 16 pieces of 16 bytes per token row");
    // This wavefront's 8 KB of each ring slot (a pair of blocks, 4 KB each). Token row r of a
    // block holds its 16-byte piece q at position q ^ r, so the 16 lanes of an operand read
    // (rows 0..15 at one piece index) cover the 64 banks once.
    half8_t* kslot0 = kr0 + w * 512;
    half8_t* kslot1 = kr1 + w * 512;
    const int lr = lane >> 4, lq = lane & 15;
    // The DMAs are issued from inline assembly, outside the compiler's wait bookkeeping (it
    // would drain every load in flight before any LDS read after an LDS DMA in a loop); their
    // waits are written out: each K pair's eight DMAs are followed, before the pair is read, by
    // at least 24 younger vector memory operations (its own V loads and the next pair's DMAs
    // and V loads), so vmcnt(24) means the pair has landed. The compiler's own waits for the V
    // registers count only its own loads and so also cover the DMAs issued before them.
    auto dma_k = [&](const int (&id)[2], half8_t* slot) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the slot's last reads are done
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const half_t* base = kc + id[j] * blk_stride + head_off;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * i + lr;
          const unsigned dst = (unsigned)(size_t)(__attribute__((address_space(3))) half8_t*)(
              slot + 256 * j + 64 * i);
          asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                       :: "v"(base + r * D + 8 * (lq ^ r)), "{m0}"(dst) : "memory");
        }
      }
    };
    int idn[2] = {0, 0};
    auto stepk = [&](int p, VRow (&vr)[2][4], half8_t* slot) {
      int idnn[2];
      ids_of(last_or(p + 3 * NW, last_or(p + 2 * NW, last_or(p + NW, p))), idnn);
      const int ba = blk_lo + 2 * p;
      const int ta = ba * kBlockSize + 4 * g, tb = ta + kBlockSize;
      half8_t kf[2][KK];
      asm volatile("s_waitcnt vmcnt(24)" ::: "memory");    // this pair's K has landed
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) kf[j][kk] = slot[256 * j + 16 * c + ((4 * kk + g) ^ c)];
      float4_t sa = zero4, sb = zero4;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        sa = mfma16x16x32(kf[0][kk], qf[kk], sa);
        sb = mfma16x16x32(kf[1][kk], qf[kk], sb);
      }
      auto finish = [&](auto masked) {
        constexpr bool kMasked = decltype(masked)::value;
        const bool tail_a = kMasked && (ba + 1) * kBlockSize > tok_hi;
        if constexpr (kMasked) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            sa[r] = ta + r < tok_hi ? sa[r] : -INFINITY;
            sb[r] = tb + r < tok_hi ? sb[r] : -INFINITY;
          }
        }
        const SoftmaxStep st = softmax_pair(sa, sb, sl2, m, l);
        pv_update<TILES>(o, st, [&](int t) {
          return vt_operand<VW>(vr[0], vr[1], t, tail_a, kMasked, ta, tb, tok_hi);
        });
      };
      if ((ba + 2) * kBlockSize > tok_hi)
        finish(std::true_type());
      else
        finish(std::false_type());
      dma_k(idn, slot);
      load_v(idn, vr);
      idn[0] = idnn[0];
      idn[1] = idnn[1];
    };
    VRow vA[2][4], vB[2][4];
    int p = w;
    if (p < npairs) {
      int id0[2], id1[2];
      if (mapped) {
        id0[0] = m_id[0];
        id0[1] = m_id[1];
        id1[0] = m_id[2];
        id1[1] = m_id[3];
      } else {
        ids_of(p, id0);
        ids_of(last_or(p + NW, p), id1);
      }
      dma_k(id0, kslot0);
      dma_k(id1, kslot1);
      load_v(id0, vA);
      load_v(id1, vB);
      ids_of(last_or(p + 2 * NW, last_or(p + NW, p)), idn);
    }
    // The loop sits on the prologue's path only, so the compiler's wait state at its head is the
    // prologue's (q and the prologue loads in flight), not that of a path with no loads.
    if (p < npairs) {
      if (mapped) poison = poison || stale();
      for (; p < npairs; p += 2 * NW) {
        stepk(p, vA, kslot0);
        if (p + NW >= npairs) break;
        stepk(p + NW, vB, kslot1);
      }
    } else if (mapped) {
      poison = poison || stale();
    }
    // the ring's memory is reused by the merge below: every DMA of every wavefront has landed
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  } else {
    half8_t kf[2][KK];
    VRow vA[2][4], vB[2][4];
    int idk[2] = {0, 0}, idv[2] = {0, 0};        // next K refill / next V refill (two pairs on)
    // Pair p: S^T from kf, refill kf with pair p + NW, softmax, P.V from vr, refill vr with pair
    // p + 2 NW.
    auto step = [&](int p, VRow (&vr)[2][4]) {
      int idk_next[2], idv_next[2];
      ids_of(last_or(p + 2 * NW, last_or(p + NW, p)), idk_next);
      ids_of(last_or(p + 3 * NW, last_or(p + 2 * NW, last_or(p + NW, p))), idv_next);
      const int ba = blk_lo + 2 * p;
      const int ta = ba * kBlockSize + 4 * g, tb = ta + kBlockSize;
      float4_t sa = zero4, sb = zero4;             // S^T = K . Q^T: two independent MFMA chains
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        if constexpr (D >= 32) {
          sa = mfma16x16x32(kf[0][kk], qf[kk], sa);
          sb = mfma16x16x32(kf[1][kk], qf[kk], sb);
        } else {
          sa = mfma16x16x16(lo4(kf[0][kk]), lo4(qf[kk]), sa);
          sb = mfma16x16x16(lo4(kf[1][kk]), lo4(qf[kk]), sb);
        }
      }
      load_k(idk, kf);
      // Only the last pair of a range can reach past tok_hi (token 0 of block a never does), so
      // the masked form is a separate, rarely taken path and the common one carries no selects.
      auto finish = [&](auto masked) {
        constexpr bool kMasked = decltype(masked)::value;
        const bool tail_a = kMasked && (ba + 1) * kBlockSize > tok_hi;
        if constexpr (kMasked) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            sa[r] = ta + r < tok_hi ? sa[r] : -INFINITY;
            sb[r] = tb + r < tok_hi ? sb[r] : -INFINITY;
          }
        }
        const SoftmaxStep st = softmax_pair(sa, sb, sl2, m, l);
        // lane (c, g) of tile t: dims VW (4g + r) + t of head c
        pv_update<TILES>(o, st, [&](int t) {
          return vt_operand<VW>(vr[0], vr[1], t, tail_a, kMasked, ta, tb, tok_hi);
        });
      };
      if ((ba + 2) * kBlockSize > tok_hi)
        finish(std::true_type());
      else
        finish(std::false_type());
      load_v(idv, vr);
      idk[0] = idk_next[0];
      idk[1] = idk_next[1];
      idv[0] = idv_next[0];
      idv[1] = idv_next[1];
    };
    int p = w;
    if (p < npairs) {
      int id0[2], id1[2];
      if (mapped) {
        id0[0] = m_id[0];
        id0[1] = m_id[1];
        id1[0] = m_id[2];
        id1[1] = m_id[3];
      } else {
        ids_of(p, id0);
        ids_of(last_or(p + NW, p), id1);
      }
      load_k(id0, kf);
      load_v(id0, vA);
      load_v(id1, vB);
      ids_of(last_or(p + NW, p), idk);
      ids_of(last_or(p + 2 * NW, last_or(p + NW, p)), idv);
    }
    if (mapped) poison = poison || stale();
    for (; p < npairs; p += 2 * NW) {
      step(p, vA);
      if (p + NW >= npairs) break;
      step(p + NW, vB);
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
    if (poison) L = __builtin_nanf("");             // reaches the output through the merge too
    if (nsplit == 1) {
      out[(int64_t)s * o_st + (int64_t)(head0 + hh) * D + d] = (half_t)(O / L);
    } else if (!mapped) {
      const int64_t pidx = ((int64_t)s * max_splits + split_j) * H + head0 + hh;
      ws_acc[pidx * D + d] = O;                  // fp32 (acc, m, l), as the reference keeps them
      if (d == 0) {
        ws_m[pidx] = M;
        ws_l[pidx] = L;
      }
    } else {                                     // for the in-launch merge: device-coherent stores
      // (offsets within sequence s's rows of the workspace: resources from its first row)
      const int pj = split_j * H + head0 + hh;
      coherent_store(coherent_rsrc(ws_acc + (int64_t)s * max_splits * H * D), (pj * D + d) * 4, O);
      if (d == 0) {
        coherent_store(coherent_rsrc(ws_m + (int64_t)s * max_splits * H), pj * 4, M);
        coherent_store(coherent_rsrc(ws_l + (int64_t)s * max_splits * H), pj * 4, L);
      }
    }
  }
  if (!mapped || nsplit == 1) return;
  // In-launch merge (a launch with the step's map): the last split of (sequence, KV head, head
  // group) to finish merges all of them, as decode_merge_kernel would, and resets the counter.
  // Its partial reaches the coherence point (vmcnt 0) before its arrival counts; the others are
  // read from there.
  __builtin_amdgcn_s_waitcnt(kWaitVmcntZero);
  __syncthreads();
  int* counter = smap + kMapHeader + (int64_t)nslots * kMapEntry + (int64_t)s * (KVH * HG) + bz;
  if (tid == 0)
    s_map[0] = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               nsplit - 1;
  __syncthreads();
  if (!s_map[0]) return;
  constexpr int TPH = D / 8;                     // threads per head (8 dims each), as the merge
  constexpr int HPP = NW * 64 / TPH;             // kernel's workgroup
  static_assert(NW * 64 == 256, "the merge layout is that of decode_merge_kernel");
  const auto r_acc = coherent_rsrc(ws_acc + (int64_t)s * max_splits * H * D);
  const auto r_m = coherent_rsrc(ws_m + (int64_t)s * max_splits * H);
  const auto r_l = coherent_rsrc(ws_l + (int64_t)s * max_splits * H);
  for (int hp = 0; hp < nh; hp += HPP) {
    const int hh = hp + tid / TPH, d0 = (tid % TPH) * 8;
    if (hh >= nh) continue;
    const int64_t hoff = head0 + hh;
    float4_t O0, O1;
    float L;
    merge_dims8(nsplit, [&](int j, float& mj, float& lj, float4_t& a0, float4_t& a1) {
      const int pj = j * H + (int)hoff;
      mj = coherent_load(r_m, pj * 4);
      lj = coherent_load(r_l, pj * 4);
      a0 = coherent_load4(r_acc, (pj * D + d0) * 4);
      a1 = coherent_load4(r_acc, (pj * D + d0 + 4) * 4);
    }, O0, O1, L);
    half_t* dst = out + (int64_t)s * o_st + hoff * D + d0;
    st<half4_t>(dst, to_half4(O0 / L));
    st<half4_t>(dst + 4, to_half4(O1 / L));
  }
  if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int D, int NW, bool WRITE = false, bool ROPE = false>
__global__ void __launch_bounds__(NW * 64) decode_mfma_kernel(
    const half_t* __restrict__ q, int64_t q_st, int64_t q_sh, half_t* __restrict__ out,
    int64_t o_st, const half_t* __restrict__ kc, const half_t* __restrict__ vc, int64_t NB,
    const int* __restrict__ bt, int64_t bt_st, int max_blocks, const int* __restrict__ seq_lens,
    int S, int H, int KVH, int G, int HG, float sl2, int cap_blocks, int part_blocks,
    int max_splits, float* __restrict__ ws_acc, float* __restrict__ ws_m,
    float* __restrict__ ws_l, int* __restrict__ ws_cnt, const NewRows nr,
    int* __restrict__ smap) {
  // One-dimensional grid of slots x (KV head, head group), the latter fastest: the launch
  // bounds the slot count from max_seq_len (S times the longest sequence's split count), so
  // most slots past the batch's last split exit at once; numbered last, they no longer hold
  // resident slots ahead of the second KV head's splits.
  const int zh = KVH * HG;
  const int bx = (int)blockIdx.x / zh, bz = (int)blockIdx.x - bx * zh;
  if constexpr (D == 128 && !ROPE) {
    // The K ring: two slots of NW x 8 KB (a pair of 4 KB blocks per wavefront). The merge's LDS
    // (O^T rows, m, l, the lookup scratch) reuses the first slot once every DMA has landed, so
    // the workgroup holds 64 KB plus the part of the merge's LDS past 32 KB (two per CU). Not
    // with RoPE: the compiler's waits for q and the RoPE tables, which count only the loads it
    // sees, then also wait for the ring's first DMAs before the rotation, and the model step
    // measured 2.230 against 2.246-2.251 ms with the register form.
    constexpr int kMergeVecs = (DecodeLds<D, NW>::BYTES + 15) / 16;
    constexpr int R0 = NW * 512 > kMergeVecs ? NW * 512 : kMergeVecs;
    __shared__ __attribute__((aligned(16))) half8_t s_k0[R0];
    __shared__ __attribute__((aligned(16))) half8_t s_k1[NW * 512];
    decode_mfma_body<D, NW, WRITE, ROPE, true>(q, q_st, q_sh, out, o_st, kc, vc, NB, bt, bt_st,
                                   max_blocks, seq_lens, S, H, KVH, G, HG, sl2, cap_blocks,
                                   part_blocks, max_splits, ws_acc, ws_m, ws_l, ws_cnt, bx, bz,
                                   reinterpret_cast<char*>(s_k0), nr, smap, (int)gridDim.x / zh,
                                   s_k0, s_k1);
  } else {
    __shared__ __attribute__((aligned(16))) char lds[DecodeLds<D, NW>::BYTES];
    decode_mfma_body<D, NW, WRITE, ROPE>(q, q_st, q_sh, out, o_st, kc, vc, NB, bt, bt_st, max_blocks,
                                   seq_lens, S, H, KVH, G, HG, sl2, cap_blocks, part_blocks,
                                   max_splits, ws_acc, ws_m, ws_l, ws_cnt, bx, bz, lds, nr, smap,
                                   (int)gridDim.x / zh);
  }
}

// Merge of the split partials (ops/triton_decode_attention.py:144-163): each split leaves its
// fp32 (acc_j, m_j, l_j), acc_j unnormalised; M = max m_j, w_j = 2^(m_j - M),
// out = sum w_j acc_j / sum w_j l_j. One workgroup per (sequence, KV head, head group), one
// thread per 8 output dims of a head (two 16-byte partial loads per split). A sequence's partials sit in rows
// s * max_splits + j; the split count written by the first kernel is read first and only the
// rows below it are requested (a second memory step, but a few hundred KB instead of kMergeChunk
// rows for every sequence: measured faster than requesting a fixed chunk together with the
// count). Sequences with one split were finished by the first kernel; a sequence with none
// (seq_len 0) gets zeros here.
constexpr int kMaxSplits = 256;
constexpr int kMergeChunk = 16;

// One thread's share of a merge: dims d0 .. d0 + 7 of one query head over the n split partials
// that load(j, m, l, a0, a1) returns (split j's m, l and acc[d0 .. d0 + 7]), taken CH at a time,
// all of a chunk's loads requested together. O0 / O1 / L come back unnormalised. The merge
// kernel and the split kernel's last workgroup both merge through this function, so a row merged
// either way has the same value.
template <class Load>
__device__ __forceinline__ void merge_dims8(int n, Load load, float4_t& O0, float4_t& O1,
                                            float& L) {
  constexpr int CH = kMergeChunk;
  float mv[CH], lv[CH];
  float4_t av[CH][2];
  auto load_chunk = [&](int j0) {
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      if (j0 + u < n) {                          // uniform over the workgroup
        load(j0 + u, mv[u], lv[u], av[u][0], av[u][1]);
      } else {
        mv[u] = -INFINITY;
        lv[u] = 0.f;
        av[u][0] = float4_t{0.f, 0.f, 0.f, 0.f};
        av[u][1] = float4_t{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
  load_chunk(0);
  float M = -INFINITY;
  L = 0.f;
  O0 = float4_t{0.f, 0.f, 0.f, 0.f};
  O1 = float4_t{0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < n; j0 += CH) {
    if (j0 > 0) load_chunk(j0);
    float cm = M;
#pragma unroll
    for (int u = 0; u < CH; ++u) cm = (j0 + u < n) ? fmaxf(cm, mv[u]) : cm;
    const float alpha = fast_exp2(M - cm);       // M = -inf on the first chunk -> 0
    L *= alpha;
    O0 *= alpha;
    O1 *= alpha;
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      // rows past n are skipped, not weighted by 0: their stale contents may be inf or NaN
      const float wt = fast_exp2(mv[u] - cm);
      L = (j0 + u < n) ? L + wt * lv[u] : L;
      const float4_t o0 = O0 + wt * av[u][0], o1 = O1 + wt * av[u][1];
      O0 = (j0 + u < n) ? o0 : O0;
      O1 = (j0 + u < n) ? o1 : O1;
    }
    M = cm;
  }
}

template <int D>
__device__ __forceinline__ void decode_merge_body(
    const float* __restrict__ ws_acc, const float* __restrict__ ws_m,
    const float* __restrict__ ws_l, const int* __restrict__ ws_cnt, half_t* __restrict__ out,
    int64_t o_st, const int* __restrict__ seq_lens, int H, int G, int HG, int max_splits, int bx, int by) {
  constexpr int TPH = D / 8;                     // threads per head (8 dims each)
  constexpr int HPP = 256 / TPH;                 // heads per pass
  const int s = bx, kvh = by / HG, hg = by % HG;
  const int tid = threadIdx.x;
  const int nh = (G - hg * 16) < 16 ? (G - hg * 16) : 16;
  const int head0 = kvh * G + hg * 16;
  const int len = __builtin_amdgcn_readfirstlane(seq_lens[s]);
  const int cnt = __builtin_amdgcn_readfirstlane(ws_cnt[s]);
  const int64_t row0 = (int64_t)s * max_splits;
  for (int hp = 0; hp < nh; hp += HPP) {
    const int hh = hp + tid / TPH, d0 = (tid % TPH) * 8;
    if (hh >= nh) continue;                      // no head for this thread (no barrier below)
    const int64_t hoff = head0 + hh;
    half_t* dst = out + (int64_t)s * o_st + (head0 + hh) * (int64_t)D + d0;
    if (len <= 0) {                              // padding row: zeros (ops/reference.py:99,104-105)
      st<half4_t>(dst, half4_t{0, 0, 0, 0});     // output rows are 8-byte aligned: two stores
      st<half4_t>(dst + 4, half4_t{0, 0, 0, 0});
      continue;
    }
    const int n = cnt < 1 ? 1 : (cnt > max_splits ? max_splits : cnt);
    if (n == 1) return;                          // written by the first kernel
    // rows past n are neither requested nor used: their stale contents may be inf or NaN
    float4_t O0, O1;
    float L;
    merge_dims8(n, [&](int j, float& mj, float& lj, float4_t& a0, float4_t& a1) {
      const int64_t pidx = (row0 + j) * H + hoff;
      mj = ws_m[pidx];
      lj = ws_l[pidx];
      a0 = ld<float4_t>(ws_acc + pidx * D + d0);
      a1 = ld<float4_t>(ws_acc + pidx * D + d0 + 4);
    }, O0, O1, L);
    st<half4_t>(dst, to_half4(O0 / L));
    st<half4_t>(dst + 4, to_half4(O1 / L));
  }
}

template <int D>
__global__ void __launch_bounds__(256) decode_merge_kernel(
    const float* __restrict__ ws_acc, const float* __restrict__ ws_m,
    const float* __restrict__ ws_l, const int* __restrict__ ws_cnt, half_t* __restrict__ out,
    int64_t o_st, const int* __restrict__ seq_lens, int H, int G, int HG, int max_splits) {
  decode_merge_body<D>(ws_acc, ws_m, ws_l, ws_cnt, out, o_st, seq_lens, H, G, HG, max_splits,
                       (int)blockIdx.x, (int)blockIdx.y);
}

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------
constexpr int kDecodeWaves = 4;                              // wavefronts per workgroup
static_assert(2 * kDecodeWaves == kMapPairs, "split map entries hold two pairs per wavefront");

// Workgroups of decode_mfma_kernel resident per CU (4 wavefronts each, one per SIMD), from the
// kernel's VGPR use (512 per SIMD lane): 6 waves per SIMD up to D = 32, 3 at D = 64, 2 at
// D = 128 (236 VGPRs), 1 at D = 256.
static int decode_wgs_per_cu(int D) { return D <= 32 ? 6 : (D == 64 ? 3 : (D == 128 ? 2 : 1)); }

struct SplitPlan {
  int version;        // 1, 2 or 3 after resolving AUTO
  int part_blocks;    // v3: blocks per split, 0 = the own-length schedule
  int nslots;         // v3: launched split slots per (KV head, head group)
  int cap_blocks;     // v3: blocks of a sequence covered by the launched splits
  int max_splits;     // v3: workspace rows per sequence (bound on its split count)
};

// Explicit v3 partition (ops/triton_ops.py:50-51): num_splits = ceil(max_seq_len / partition)
// splits per sequence at most; partition = 0 selects the own-length schedule (seq_part). AUTO
// splits whenever one workgroup per (sequence, KV head, head group) cannot fill the device and
// contexts are longer than two minimum splits (the reference's rule, ops/triton_ops.py:44-45,
// with the CU count and this kernel's residency). With a fixed partition a sequence longer than
// max_seq_len is attended over the launched grid's tokens, as in the reference's grid.
static SplitPlan plan_decode(int version, int S, int H, int KVH, int D, int max_seq_len,
                             int partition, int cu_count) {
  SplitPlan p{version, 0, 0, 0, 0};
  const int G = H / KVH;
  const int HG = (G + 15) / 16;
  const int64_t groups = (int64_t)KVH * HG;
  const int64_t wg_slots = (int64_t)cu_count * decode_wgs_per_cu(D);
  if (version == TS_DECODE_AUTO) {
    const bool use_split = (int64_t)S * groups < wg_slots && max_seq_len > 2 * kMinPartBlocks * kBlockSize;
    p.version = use_split ? TS_DECODE_V3 : TS_DECODE_V2;
  }
  if (p.version != TS_DECODE_V3) return p;
  const int max_blk = (max_seq_len + kBlockSize - 1) / kBlockSize;
  if (partition > 0) {
    p.part_blocks = partition / kBlockSize;
    int num_splits = (max_blk + p.part_blocks - 1) / p.part_blocks;
    if (num_splits > kMaxSplits) {               // bounds the workspace rows per sequence
      p.part_blocks = (max_blk + kMaxSplits - 1) / kMaxSplits;
      num_splits = (max_blk + p.part_blocks - 1) / p.part_blocks;
    }
    num_splits = num_splits < 1 ? 1 : num_splits;
    p.cap_blocks = num_splits * p.part_blocks;
    p.nslots = S * num_splits;
    p.max_splits = num_splits;
  } else {
    // The own-length schedule: a sequence of nb <= max_blk blocks has at most
    // per_seq = min(kOwnMaxSplits, ceil(max_blk / kOwnPartBlocks)) splits, and seq_part caps
    // every sequence at max_splits = per_seq splits (only a sequence longer than max_seq_len,
    // which the caller promises not to pass, gets longer splits than its own length implies;
    // it is still attended in full). So S * per_seq slots cover every batch; the slots past
    // the batch's last split exit at once.
    int per_seq = (max_blk + kOwnPartBlocks - 1) / kOwnPartBlocks;
    per_seq = per_seq < 1 ? 1 : (per_seq > kOwnMaxSplits ? kOwnMaxSplits : per_seq);
    p.cap_blocks = 1 << 30;
    p.nslots = S * per_seq;
    p.max_splits = per_seq;
  }
  return p;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct WsLayout {
  size_t acc, m, l, cnt, total;
};

// [acc: rows * H * D fp32][m: rows * H fp32][l: rows * H fp32][count: S int32] with
// rows = S * max_splits: split j of sequence s keeps query head h's partial in row
// s * max_splits + j, column h.
static WsLayout ws_layout(const SplitPlan& p, int S, int H, int D) {
  WsLayout w{0, 0, 0, 0, 0};
  if (p.version != TS_DECODE_V3) return w;
  const size_t n = (size_t)S * p.max_splits * H;
  w.acc = 0;
  w.m = align256(n * D * sizeof(float));
  w.l = w.m + align256(n * sizeof(float));
  w.cnt = w.l + align256(n * sizeof(float));
  w.total = w.cnt + align256((size_t)S * sizeof(int));
  return w;
}

// Bytes of the per-step split map of plan p (0: the plan does not split): header, entries and
// one arrival counter per (sequence, KV head, head group).
static size_t map_bytes_of(const SplitPlan& p, int S, int groups) {
  if (p.version != TS_DECODE_V3) return 0;
  return ((size_t)kMapHeader + (size_t)p.nslots * kMapEntry + (size_t)S * groups) * sizeof(int);
}

// The cap_blocks a v3 launch of plan p passes to its kernels (and the map records).
static int launch_cap_blocks(const SplitPlan& p, int max_blocks) {
  return p.cap_blocks < max_blocks ? p.cap_blocks : max_blocks;
}

static void launch_split_map(const SplitPlan& p, hipStream_t st, const int* sl, const int* bt,
                             int64_t bt_st, int64_t NB, int max_blocks, int S, int groups,
                             int* map) {
  int groups_x = (p.nslots + kMapThreads - 1) / kMapThreads;
  groups_x = groups_x < 1 ? 1 : (groups_x > kMapMaxGroups ? kMapMaxGroups : groups_x);
  decode_split_map_kernel<kMapThreads><<<groups_x, kMapThreads, 0, st>>>(
      sl, bt, bt_st, NB, S, launch_cap_blocks(p, max_blocks), p.part_blocks, p.max_splits,
      p.nslots, S * groups, map);
}

// With nr.k set (kv_write fused into the launch; v2 / v3 with one head group per KV head only)
// the MFMA kernel first writes the new rows, as in decode_mfma_body; with nr.cos_t set too
// (head_dim a multiple of 64) it also rotates q and the new k rows first.
template <int D>
static void launch_decode(const SplitPlan& p, hipStream_t st, const half_t* q, int64_t q_st,
                          int64_t q_sh, half_t* out, int64_t o_st, const half_t* kc,
                          const half_t* vc, int64_t NB, const int* bt, int64_t bt_st,
                          int max_blocks, const int* sl, int S, int H, int KVH, float scale_log2,
                          void* ws, const NewRows& nr = NewRows{}, int* smap = nullptr) {
  const int G = H / KVH;
  const bool write = nr.k != nullptr;
  const bool rope = write && nr.cos_t != nullptr;     // only for head_dim % 64 == 0
  if (p.version == TS_DECODE_V1) {
    decode_v1_kernel<D><<<dim3(S, H), 64, 0, st>>>(q, q_st, q_sh, out, o_st, kc, vc, NB, bt,
                                                   bt_st, max_blocks, sl, H, KVH, scale_log2);
    return;
  }
  const int HG = (G + 15) / 16;
  if (p.version == TS_DECODE_V2) {
#define TS_V2_LAUNCH(W, R)                                                                       \
  decode_mfma_kernel<D, kDecodeWaves, W, R><<<dim3(S * KVH * HG), kDecodeWaves * 64, 0, st>>>(  \
      q, q_st, q_sh, out, o_st, kc, vc, NB, bt, bt_st, max_blocks, sl, S, H, KVH, G, HG,        \
      scale_log2, 0, 0, 0, nullptr, nullptr, nullptr, nullptr, nr, nullptr)
    if constexpr (D % 64 == 0) {
      if (rope) {
        TS_V2_LAUNCH(true, true);
        return;
      }
    }
    if (write)
      TS_V2_LAUNCH(true, false);
    else
      TS_V2_LAUNCH(false, false);
#undef TS_V2_LAUNCH
    return;
  }
  const WsLayout w = ws_layout(p, S, H, D);
  char* b = static_cast<char*>(ws);
  float* ws_acc = reinterpret_cast<float*>(b + w.acc);
  float* ws_m = reinterpret_cast<float*>(b + w.m);
  float* ws_l = reinterpret_cast<float*>(b + w.l);
  int* ws_cnt = reinterpret_cast<int*>(b + w.cnt);
  const int cap = launch_cap_blocks(p, max_blocks);
#define TS_V3_LAUNCH(W, R)                                                                       \
  decode_mfma_kernel<D, kDecodeWaves, W, R><<<dim3(p.nslots * KVH * HG), kDecodeWaves * 64, 0,  \
                                              st>>>(                                             \
      q, q_st, q_sh, out, o_st, kc, vc, NB, bt, bt_st, max_blocks, sl, S, H, KVH, G, HG,        \
      scale_log2, cap, p.part_blocks, p.max_splits, ws_acc, ws_m, ws_l, ws_cnt, nr, smap)
  bool launched = false;
  if constexpr (D % 64 == 0) {
    if (rope) {
      TS_V3_LAUNCH(true, true);
      launched = true;
    }
  }
  if (!launched) {
    if (write)
      TS_V3_LAUNCH(true, false);
    else
      TS_V3_LAUNCH(false, false);
  }
#undef TS_V3_LAUNCH
  if (smap != nullptr) return;                 // the split kernel merged in-launch
  decode_merge_kernel<D><<<dim3(S, KVH * HG), 256, 0, st>>>(ws_acc, ws_m, ws_l, ws_cnt, out, o_st,
                                                             sl, H, G, HG, p.max_splits);
}

static bool supported_head_dim(int D) {
  return D == 16 || D == 32 || D == 64 || D == 128 || D == 256;
}

}  // namespace ts
