// Paired-unit prefill tiles for head_dim 128: the standalone chunked-prefill kernel
// (ops/triton_prefill_attention.py:17-79; bottom-right causal mask of ops/reference.py:60-77,
// online softmax in fp32, P rounded to fp16 before the P.V product).
//
// Workgroup = 512 threads: two groups of four wavefronts, each group owning one 128-row unit.
// With an even GQA group size the two units are the same 128 query rows of two query heads that
// share a KV head; otherwise two consecutive 128-row tiles of one query head. Every 64-key step
// of K and V is staged in LDS once for both units (eight wavefronts, 256 query rows). Per step s
// and wavefront (32 query rows of its unit), on v_mfma_f32_32x32x16_f16 (operand layouts as in the
// 4-wavefront tile kernel):
//   MFMA phase M(s):  S^T(s) = K(s) . Q^T (16 MFMAs) alternating with O^T += V^T(s-1) . P^T(s-1)
//                     (16 MFMAs, the previous step's P), operands requested kPairAhead MFMAs
//                     ahead; the wavefront's share of staging step s + 1 (4 LDS writes, 10 global
//                     loads) is spread between the MFMAs
//   VALU phase V(s):  causal mask and online softmax of S^T(s) -> P(s) in fp16
// Keeping P(s) for the next MFMA phase puts 32 mutually independent MFMAs in every MFMA phase.
// The groups run half a step apart -- group 0: M(s) | V(s), group 1: V(s-1) | M(s) -- with a
// workgroup barrier between phases, so on every SIMD (one wavefront of each group) one
// wavefront's softmax runs beside the other's MFMAs. (Measured on MI355X: one wavefront's LDS
// operand reads feed an MFMA only about every 55 cycles, which bounds each MFMA phase; running
// both groups' MFMA phases together, one barrier per step, measured about as fast.)
//
// Launch: with a workspace, each work item's (sequence, head item) steps, tiles longest first,
// are shared evenly over its launch slots (stream-K) and cut at tile boundaries into segments; a
// tile covered by one segment is written directly, otherwise its segments' partials are combined
// by prefill_pair_merge_kernel. Without one, each slot takes one whole tile.
//
// LDS: two K buffers [64 keys][256 bytes + 16 pad] and two V^T buffers laid out as
// [16-key block u][dim d][32 bytes]: the 32 bytes are the two 8-key halves that lanes h = 0, 1
// of the PV MFMA of block u read, swapped when bits 2 and 3 of d differ, so that operand reads
// and staging writes fall on distinct banks. K(s) is in buffer (s - lo) % 2, V(s) in buffer
// (s - lo) % 2; during step s the staging writes K(s + 1) and V(s) into the buffers that step
// s - 1 released, and loads K(s + 2), V(s + 1) into registers.
#pragma once

#include "prefill_kernels.h"

namespace ts {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kPairThreads = 512;
constexpr int kPairSlotRows = 256;     // partial rows per launch slot: the two 128-row units
constexpr int kPairAhead = 7;         // LDS operand reads in flight ahead of the MFMAs

template <bool B>
struct Flag {
  static constexpr bool value = B;
};

struct PairLayout {
  static constexpr int D = 128;
  static constexpr int KROW = 2 * D + 16;            // staged K row: 256 bytes + 16 of padding
  static constexpr int KBYTES = kTileKeys * KROW;
  static constexpr int VBYTES = 4 * D * 32;          // V^T: [u][d][32 bytes]
  static constexpr int BYTES = 2 * KBYTES + 2 * VBYTES;
};

// Whether the two units of a workgroup are two query heads (even group size) or two tiles.
__host__ __device__ inline bool pair_heads(int H, int KVH) { return (H / KVH) % 2 == 0; }

// Launch plan of the paired kernel, from host bounds of the batch. With a workspace and fewer work
// items (sequence, head item) than CUs, each item gets `slots` launch slots that share its steps
// evenly (stream-K, one workgroup per CU); otherwise one slot per tile (seg_cap = 0).
struct PairPlan {
  int slots;          // launch slots per work item
  int seg_cap;        // partial segments per work item in the workspace (0: no partials)
  size_t ws_bytes;
};

inline PairPlan pair_plan(int P, int H, int KVH, int max_query_len, int max_seq_len, int cu_count,
                          bool split) {
  const bool heads = pair_heads(H, KVH);
  const int tr = heads ? kTileRows : 2 * kTileRows;
  const int items = P * (H / (heads ? 2 : 1));
  const int tiles = cdiv(max_query_len, tr);
  const int seq = max_seq_len > max_query_len ? max_seq_len : max_query_len;
  const int cus = cu_count > 0 ? cu_count : 256;
  PairPlan pl{tiles, 0, 0};
  if (!split || cdiv(seq, kTileKeys) <= 1 || 2 * items > cus) return pl;
  pl.slots = cus / items;
  pl.seg_cap = tiles + pl.slots;
  pl.ws_bytes = (size_t)items * pl.seg_cap * kPairSlotRows * (PairLayout::D + 2) * sizeof(float);
  return pl;
}

__device__ __forceinline__ void prefill_pair_body(
    const half_t* __restrict__ q, int64_t q_st, int64_t q_sh, half_t* __restrict__ out,
    int64_t o_st, int64_t num_tokens, const half_t* __restrict__ kc,
    const half_t* __restrict__ vc, int64_t NB, const int* __restrict__ bt, int64_t bt_st,
    int max_blocks, const int* __restrict__ seq_lens, const int* __restrict__ qsl,
    int num_decode, int H, int KVH, float sl2, int slots, int seg_cap, int P,
    float* __restrict__ ws, int bx, char* __restrict__ lds) {
  constexpr int D = PairLayout::D;
  using L = PairLayout;
  constexpr int KK = D / 16;                       // k-steps of S^T
  constexpr int DT = D / 32;                       // 32-dim tiles of O^T
  const int G = H / KVH;
  const bool heads = pair_heads(H, KVH);
  const int hp = heads ? 2 : 1;                    // query heads per work item
  const int tr = heads ? kTileRows : 2 * kTileRows;
  const int HI = G / hp;                           // work items per KV head and tile

  // Work items of one KV head are (slot, sequence, head item), slot-major; with the KV heads
  // dividing the eight XCDs, XCD x serves KV head x / (8 / KVH) (launch ids go round-robin over
  // the XCDs), so each XCD L2 holds one KV head's K/V.
  const int per_kvh = slots * P * HI;
  int kvh, rem;
  if (8 % KVH == 0) {
    const int xpk = 8 / KVH;
    const int xcd = bx & 7;
    kvh = xcd / xpk;
    rem = (bx >> 3) * xpk + xcd % xpk;
  } else {
    kvh = bx / per_kvh;
    rem = bx - kvh * per_kvh;
  }
  if (kvh >= KVH || rem >= per_kvh) return;
  const int slot = rem / (P * HI);
  rem -= slot * (P * HI);
  const int pi = rem / HI;
  const int item = kvh * HI + (rem - pi * HI);     // query heads item * hp .. + hp - 1
  const int b = num_decode + pi;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = w >> 2, wi = w & 3;
  const int r = lane & 31, hh = lane >> 5;
  const int h = item * hp + (heads ? g : 0);

  const PrefillSeq sq = prefill_seq(qsl, seq_lens, b, num_tokens, max_blocks);
  const int tiles = (sq.q_len + tr - 1) / tr;
  // 64-key steps of tile t: up to the causal limit of its last row.
  auto tile_steps = [&](int t) {
    const int last_row = ((t + 1) * tr < sq.q_len ? (t + 1) * tr : sq.q_len) - 1;
    int k_hi = sq.prefix + last_row + 1 < sq.seq_len ? sq.prefix + last_row + 1 : sq.seq_len;
    k_hi = k_hi < 0 ? 0 : k_hi;
    return (k_hi + kTileKeys - 1) / kTileKeys;
  };

  // Steps [lo, hi) of tile `tile` for both units; whole: the tile's full key range (written to the
  // output), else a partial at segment index seg of the work item (dropped if seg >= seg_cap).
  auto run_segment = [&](int tile, int lo, int hi, bool whole, int seg) {
  const int m0 = tile * tr;
  const int last = (m0 + tr < sq.q_len ? m0 + tr : sq.q_len) - 1;
  int kv_hi = sq.prefix + last + 1 < sq.seq_len ? sq.prefix + last + 1 : sq.seq_len;
  kv_hi = kv_hi < 0 ? 0 : kv_hi;
  const int nblk = (kv_hi + kBlockSize - 1) / kBlockSize;
  const int r0 = m0 + (heads ? 0 : kTileRows * g) + 32 * wi;   // first query row of this wave
  const int row = r0 + r;
  const bool row_ok = row < sq.q_len;
  const int n = hi - lo;
  // Steps this wavefront computes: [lo, whi), up to its last visible key.
  int whi = lo;
  if (r0 < sq.q_len) {
    const int kmax = sq.prefix + r0 + 31 < kv_hi - 1 ? sq.prefix + r0 + 31 : kv_hi - 1;
    if (kmax >= 0) whi = kmax / kTileKeys + 1 < hi ? kmax / kTileKeys + 1 : hi;
    whi = whi < lo ? lo : whi;
  }

  // Q^T operands: lane (r, h) holds dims 16 kk + 8 h .. +7 of its row (zeros past q_len).
  half8_t qf[KK];
  {
    const half_t* qp = q + (int64_t)(sq.q_start + (row_ok ? row : 0)) * q_st + (int64_t)h * q_sh + 8 * hh;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      qf[kk] = row_ok ? ld<half8_t>(qp + 16 * kk) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
  }

  // Staging share of wavefront w: block ub = w / 2 of the step.
  //  K: rows 8w .. 8w+7; lane -> row 8w + lane % 8, 16-byte pieces kpc and kpc + 4 with
  //     kpc = lane / 16 + 8 ((lane / 8) % 2): 16 consecutive lanes write pieces {c, c + 8} of
  //     eight rows, which the 272-byte row pitch puts on distinct banks.
  //  V: keys {4v + i, 8 + 4v + i} (v = lane / 32, i = 0..3) of block ub -- the 8-key half v of
  //     the PV operand -- and dims 64 (w % 2) + 2 (lane % 32) + {0, 1}, one dword per key.
  const int64_t head_off = (int64_t)kvh * kBlockSize * D;
  const int64_t blk_stride = (int64_t)KVH * kBlockSize * D;
  const int* btrow = bt + (int64_t)b * bt_st;
  const int ub = w >> 1;
  const int krow = 8 * w + (lane & 7);
  const int kpc = (lane >> 4) + 8 * ((lane >> 3) & 1);
  const int k_g = (krow & 15) * D + 8 * kpc;       // halves within the cache block
  const int k_l = krow * L::KROW + 16 * kpc;       // bytes within a K buffer
  const int vvh = lane >> 5, vcol = lane & 31;
  const int vd0 = 64 * (w & 1) + 2 * vcol;
  const int v_g = 4 * vvh * D + vd0;
  const int v_l = ub * (D * 32) + vd0 * 32 + 16 * (vvh ^ (((vcol >> 1) ^ (vcol >> 2)) & 1));
  // MFMA operand bases: S^T reads K row 32 x + r at piece 2 kk + h; PV reads V^T row 32 t + r of
  // block u at the half h (swapped by bits 2 and 3 of r).
  const int k_rd = r * L::KROW + 16 * hh;
  const int v_rd = r * 32 + 16 * (hh ^ (((r >> 2) ^ (r >> 3)) & 1));

  // Staging registers: each step's loads are issued one step before they are written to LDS.
  int4_t kra[2];
  uint32_t vra[8];
  const int hi1 = hi - 1;
  // Cache offset of this wavefront's block at step st (past the range: the range's last step,
  // past the tile's keys: its last block; those keys are masked or zeroed). The block ids come
  // from a window of 64 steps held one per lane and read with v_readlane, so the staging never
  // waits on a scalar load (whose wait would also drain the wavefront's LDS writes). Callers ask
  // for non-decreasing steps, so the window moves forward once per 64 steps; a step outside it
  // (either side) reloads it.
  int bwin = 0, win = -kWave;
  auto block_at = [&](int st) -> int64_t {
    st = st < hi1 ? st : hi1;
    if (st < win || st - win >= kWave) {
      win = st;
      int sl = win + lane;
      sl = sl < hi1 ? sl : hi1;
      int bi = sl * 4 + ub;
      bi = bi < nblk ? bi : nblk - 1;
      bwin = clamp_block(btrow[bi], NB);
    }
    return (int64_t)__builtin_amdgcn_readlane(bwin, st - win) * blk_stride + head_off;
  };
  auto load_k = [&](int64_t off, int4_t (&kr)[2]) {
    const half_t* p = kc + off + k_g;
    kr[0] = ld<int4_t>(p);
    kr[1] = ld<int4_t>(p + 32);
  };
  auto load_v = [&](int64_t off, uint32_t (&vr)[8]) {
    const half_t* p = vc + off + v_g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      vr[i] = ld<uint32_t>(p + i * D);
      vr[4 + i] = ld<uint32_t>(p + (8 + i) * D);
    }
  };
  auto store_k = [&](int buf, const int4_t (&kr)[2]) {
    char* d = lds + buf * L::KBYTES + k_l;
    ts::st<int4_t>(d, kr[0]);
    ts::st<int4_t>(d + 64, kr[1]);
  };
  auto store_v = [&](int buf, int st, const uint32_t (&vr)[8]) {
    uint32_t x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = vr[i];
    if ((st + 1) * kTileKeys > kv_hi) {
      // The tile's last step: keys at or past kv_hi are zeroed (a reused block may hold NaN
      // there, and 0 * NaN would reach the output).
      const int key0 = st * kTileKeys + 16 * ub + 4 * vvh;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[i] = key0 + i < kv_hi ? vr[i] : 0u;
        x[4 + i] = key0 + 8 + i < kv_hi ? vr[4 + i] : 0u;
      }
    }
    // Dim vd0 is the low half of every key's dword, dim vd0 + 1 the high half.
    u32x4_t lo4, hi4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo4[i] = __builtin_amdgcn_perm(x[2 * i + 1], x[2 * i], 0x05040100u);
      hi4[i] = __builtin_amdgcn_perm(x[2 * i + 1], x[2 * i], 0x07060302u);
    }
    char* d = lds + 2 * L::KBYTES + buf * L::VBYTES + v_l;
    ts::st<u32x4_t>(d, lo4);
    ts::st<u32x4_t>(d + 32, hi4);
  };

  float16_t o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[t][e] = 0.f;
  float16_t s[2];
  half8_t p[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) p[u] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
  float m = -INFINITY, l = 0.f;
  const int lim = sq.prefix + row < kv_hi - 1 ? sq.prefix + row : kv_hi - 1;   // last visible key

  // MFMA phase of step st: S^T(st) from K buffer (st - lo) % 2 and O^T += V^T(st - 1) . P^T(st - 1)
  // from V buffer (st - lo - 1) % 2; MFMA i of the issue order reads operand i, S and PV
  // alternating. At st = lo, P is zero and the V buffer zero-filled; S^T of steps past the
  // wavefront's range (st >= whi, including st = hi) is computed but never used.
  // With `staged`, the block also holds a staging's 4 LDS writes and 10 global loads: the writes
  // go first, the loads one after every third MFMA, so the vector memory path takes them a few at
  // a time instead of stalling the wavefront on a burst.
  auto mphase = [&](int st, auto staged) {
    constexpr int N = 32;
    const char* kb = lds + ((st - lo) & 1) * L::KBYTES + k_rd;
    const char* vb = lds + 2 * L::KBYTES + ((st - lo + 1) & 1) * L::VBYTES + v_rd;
    half8_t op[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int j = i >> 1;
      op[i] = (i & 1) == 0 ? ld<half8_t>(kb + (j & 1) * 32 * L::KROW + (j >> 1) * 32)
                           : ld<half8_t>(vb + (j >> 2) * (D * 32) + (j & 3) * 1024);
    }
    const float16_t zero = {};
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int j = i >> 1;
      if ((i & 1) == 0)
        s[j & 1] = mfma32x32x16(op[i], qf[j >> 1], j < 2 ? zero : s[j & 1]);
      else
        o[j & 3] = mfma32x32x16(op[i], p[j >> 2], o[j & 3]);
    }
    constexpr bool STAGED = decltype(staged)::value;
    if (STAGED) __builtin_amdgcn_sched_group_barrier(0x200, 4, 0);  // staging LDS writes
    __builtin_amdgcn_sched_group_barrier(0x100, kPairAhead, 0);      // the first reads ...
#pragma unroll
    for (int i = 0; i < N; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);             // ... then each MFMA
      if (i < N - kPairAhead)                                        //     followed by the read
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);           //     kPairAhead ahead
      if (STAGED && i % 3 == 1 && i / 3 < 10)
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);           //     and a global load
    }
  };
  // Online softmax of S^T(st) into P(st) (lazy rescale: the reference maximum moves only when a
  // new score exceeds it by more than kRescaleLog2). Outside [lo, whi) every key is masked, which
  // leaves m, l and O unchanged and makes P zero.
  auto vstep = [&](int st) {
    const int k0 = st * kTileKeys;
    const bool none = st < lo || st >= whi;
    if (none || k0 + kTileKeys - 1 > sq.prefix + r0) {   // diagonal or tail step: per-key mask
      const int lm = none ? -1 : lim;
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = k0 + 32 * x + 8 * (e >> 2) + 4 * hh + (e & 3);
          s[x][e] = key <= lm ? s[x][e] : -INFINITY;
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
  };

  if (n > 0) {
    __syncthreads();                               // the previous segment's last LDS reads
    load_k(block_at(lo), kra);                     // K(lo)
    store_k(0, kra);
    {
      // V buffer 1 is read (times P = 0) by the first MFMA phase: zero, not stale bits.
      const u32x4_t z = {0u, 0u, 0u, 0u};
      char* d = lds + 2 * L::KBYTES + L::VBYTES + v_l;
      ts::st<u32x4_t>(d, z);
      ts::st<u32x4_t>(d + 32, z);
    }
    // K(lo + 1), V(lo), in the order in which every staging issues its loads.
    load_k(block_at(lo + 1), kra);
    load_v(block_at(lo), vra);
    __syncthreads();
    // Staging of step index j from the registers holding K(lo + j + 1) and V(lo + j): write them
    // to LDS, then load K(lo + j + 2) and V(lo + j + 1).
    auto staging = [&](int j, int4_t (&kr)[2], uint32_t (&vr)[8]) {
      const int st = lo + j;
      const int64_t bv = block_at(st + 1);         // steps in increasing order (see block_at)
      const int64_t bk = block_at(st + 2);
      store_v(j & 1, st, vr);
      store_k((j + 1) & 1, kr);                    // at j = n - 1 a copy of K(hi - 1), unused
      load_k(bk, kr);
      load_v(bv, vr);
    };
    // Phase 2j + g: group g stages step index j and runs M(lo + j); phase 2j + 1 + g: it runs
    // the softmax of step lo + j. Every wavefront runs every phase (past its own key range on
    // zero P), so the loop has no branches besides the causal mask and the rescale.
    if (g == 1) __syncthreads();                   // phase 0 belongs to group 0
    for (int j = 0; j < n; ++j) {
      // Raised priority over the MFMA phase: of the two wavefronts on a SIMD, the one issuing
      // MFMAs is served first.
      __builtin_amdgcn_s_setprio(2);
      staging(j, kra, vra);
      mphase(lo + j, Flag<true>{});
      __builtin_amdgcn_s_setprio(0);
      __syncthreads();
      vstep(lo + j);
      __syncthreads();
    }
    __builtin_amdgcn_s_setprio(2);
    mphase(hi, Flag<false>{});                     // O += V^T(hi - 1) . P^T(hi - 1)
    __builtin_amdgcn_s_setprio(0);
    if (g == 0) __syncthreads();                   // phase 2n + 1 belongs to group 1
  }

  const float lt = pair_sum(l);
  if (!row_ok || (!whole && seg >= seg_cap)) return;
  if (whole) {
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
    // Partial of this segment: the row's O and (m, l), all fp32, as the reference keeps a
    // split's state (ops/triton_decode_attention.py:190-192), at row 32 w + r of the segment.
    const int64_t wseg = ((int64_t)pi * (H / hp) + item) * seg_cap + seg;
    const int64_t total = (int64_t)P * (H / hp) * seg_cap;
    const int64_t prow = wseg * kPairSlotRows + 32 * w + r;
    float* op = ws + prow * D + 4 * hh;
    if (hh == 0) {
      float* wml = ws + total * kPairSlotRows * D + prow * 2;
      wml[0] = m;
      wml[1] = lt;
    }
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        ts::st<float4_t>(op + 32 * t + 8 * j,
                         float4_t{o[t][4 * j], o[t][4 * j + 1], o[t][4 * j + 2], o[t][4 * j + 3]});
  }
  };

  if (seg_cap == 0) {
    // One tile per launch slot, longest first, written to the output. Rows of tiles the launch
    // misses (host bounds below the real q_len / seq_len) are written by no other workgroup.
    if (slot == slots - 1 && tiles > slots) {
      const int m_end = (tiles - slots) * tr < sq.q_len ? (tiles - slots) * tr : sq.q_len;
      for (int x = 0; x < hp; ++x) poison_rows<D>(out, o_st, sq.q_start, 0, m_end, item * hp + x);
    }
    if (slot < tiles) {
      const int t = tiles - 1 - slot;
      run_segment(t, 0, tile_steps(t), true, 0);
    }
    return;
  }
  // Stream-K split: the work item's tiles, longest first, form one sequence of N steps; launch
  // slot k takes steps [k T, (k + 1) T), T = ceil(N / slots), cut at tile boundaries into
  // segments. The segment holding step g is numbered (position of its tile) + g / T.
  int total_steps = 0;
  for (int t = 0; t < tiles; ++t) total_steps += tile_steps(t);
  const int per = (total_steps + slots - 1) / slots;
  const int g0 = slot * per, g1 = g0 + per < total_steps ? g0 + per : total_steps;
  int gbase = 0;
  for (int pos = 0; pos < tiles && gbase < g1; ++pos) {
    const int t = tiles - 1 - pos;
    const int nt = tile_steps(t);
    const int lo = g0 > gbase ? g0 - gbase : 0;
    const int hi = g1 - gbase < nt ? g1 - gbase : nt;
    if (lo < hi) run_segment(t, lo, hi, lo == 0 && hi == nt, pos + slot);
    gbase += nt;
  }
}

__global__ void __launch_bounds__(kPairThreads) prefill_pair_kernel(
    const half_t* __restrict__ q, int64_t q_st, int64_t q_sh, half_t* __restrict__ out,
    int64_t o_st, int64_t num_tokens, const half_t* __restrict__ kc,
    const half_t* __restrict__ vc, int64_t NB, const int* __restrict__ bt, int64_t bt_st,
    int max_blocks, const int* __restrict__ seq_lens, const int* __restrict__ qsl,
    int num_decode, int H, int KVH, float sl2, int slots, int seg_cap, int P,
    float* __restrict__ ws) {
  __shared__ __attribute__((aligned(16))) char lds[PairLayout::BYTES];
  prefill_pair_body(q, q_st, q_sh, out, o_st, num_tokens, kc, vc, NB, bt, bt_st, max_blocks,
                    seq_lens, qsl, num_decode, H, KVH, sl2, slots, seg_cap, P, ws, (int)blockIdx.x,
                    lds);
}

// Merge of the stream-K segments: grid (4 * blocks, P, H) over 128-row blocks of each sequence
// and head; workgroup (4 c + q) merges rows 32q .. 32q+31 of block c if its tile was cut into
// segments. Block c of head h is unit (h % hp) + (128 c % tr) / 128 of tile 128 c / tr of item
// h / hp; its tile at position pos (longest first) starting at step G of the item's sequence has
// segments pos + k, k = G / T .. (G + n - 1) / T. A tile with a segment past seg_cap (host bounds
// below the real lengths) gets NaN rows.
__global__ void __launch_bounds__(kTileThreads) prefill_pair_merge_kernel(
    const float* __restrict__ ws, half_t* __restrict__ out, int64_t o_st, int64_t num_tokens,
    int max_blocks, const int* __restrict__ seq_lens, const int* __restrict__ qsl,
    int num_decode, int H, int KVH, int slots, int seg_cap) {
  constexpr int D = PairLayout::D;
  constexpr int TPR = D / 8;
  constexpr int RG = kMergeRowStride;
  constexpr int NR = kMergeRows;
  static_assert(RG * NR * 4 == kTileRows && TPR * RG == kTileThreads, "four workgroups per block");
  const int bx = (int)blockIdx.x, by = (int)blockIdx.y, h = (int)blockIdx.z;
  const int part = bx & 3;
  const PrefillSeq sq = prefill_seq(qsl, seq_lens, num_decode + by, num_tokens, max_blocks);
  const bool heads = pair_heads(H, KVH);
  const int hp = heads ? 2 : 1;
  const int tr = heads ? kTileRows : 2 * kTileRows;
  const int tiles = (sq.q_len + tr - 1) / tr;
  auto tile_steps = [&](int t) {
    const int last_row = ((t + 1) * tr < sq.q_len ? (t + 1) * tr : sq.q_len) - 1;
    int k_hi = sq.prefix + last_row + 1 < sq.seq_len ? sq.prefix + last_row + 1 : sq.seq_len;
    k_hi = k_hi < 0 ? 0 : k_hi;
    return (k_hi + kTileKeys - 1) / kTileKeys;
  };
  int total_steps = 0;
  for (int t = 0; t < tiles; ++t) total_steps += tile_steps(t);
  const int per = (total_steps + slots - 1) / slots;
  const int rbase = part * RG * NR + (int)(threadIdx.x / TPR);
  const int d0 = 8 * (int)(threadIdx.x % TPR);
  const int64_t total = (int64_t)gridDim.y * (H / hp) * seg_cap;
  const half_t nan = __builtin_bit_cast(half_t, (unsigned short)0x7e00);
  // The grid covers the blocks the host bounds foresee; a longer sequence has its further blocks
  // taken in turn.
  for (int blk = bx >> 2; blk * kTileRows < sq.q_len; blk += (int)gridDim.x / 4) {
    if (blk * kTileRows + rbase >= sq.q_len) continue;
    const int t = blk * kTileRows / tr;
    const int unit = h % hp + (blk * kTileRows - t * tr) / kTileRows;
    const int pos = tiles - 1 - t;
    int gstart = 0;
    for (int u = tiles - 1; u > t; --u) gstart += tile_steps(u);
    const int nt = tile_steps(t);
    if (nt == 0 || per == 0) continue;
    const int k0 = gstart / per, k1 = (gstart + nt - 1) / per;
    if (k0 == k1) continue;                        // one segment: written by the tile kernel
    half_t* dst[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) {
      const int row = blk * kTileRows + rbase + RG * k;
      dst[k] = row < sq.q_len ? out + (int64_t)(sq.q_start + row) * o_st + (int64_t)h * D + d0
                              : nullptr;
    }
    if (pos + k1 >= seg_cap) {
#pragma unroll
      for (int k = 0; k < NR; ++k)
        if (dst[k] != nullptr) {
          ts::st<half4_t>(dst[k], half4_t{nan, nan, nan, nan});
          ts::st<half4_t>(dst[k] + 4, half4_t{nan, nan, nan, nan});
        }
      continue;
    }
    merge_partials<D>(ws, total, kPairSlotRows, ((int64_t)by * (H / hp) + h / hp) * seg_cap + pos + k0,
                      k1 - k0 + 1, unit * kTileRows + rbase, d0, dst);
  }
}

}  // namespace ts
