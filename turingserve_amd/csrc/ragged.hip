// One ragged paged-attention step over a flat batch of decode rows and prefill chunks
// (ops/triton_ops.py:60-71, twin ops/reference.py:94-111).
//
// The reference runs the decode kernel on rows [0, num_decode) and then the prefill kernel on
// the remaining sequences. Neither fills an MI355X on a mixed step by itself: the decode split
// kernel is bound by HBM bandwidth and the prefill tiles by MFMA and LDS latency. Here both run
// in one launch: the workgroups of the prefill tile plan come first, the decode split slots take
// the remaining resident slots (two workgroups per CU), and one merge launch then combines the
// split partials of both. The decode part uses the own-length split schedule of
// ts_decode_attention, the prefill part a split plan sized for 6/8 of the resident slots (the
// decode splits fill what the prefill tiles leave and free as they finish). Each workgroup
// runs exactly the code of its standalone kernel (decode_mfma_body / prefill_tile_body), so the
// results equal the standalone launches with the same plans.
//
// The fused path needs head_dim 128, the automatic decode policy resolving to v3 with the
// own-length schedule (partition 0), at least one decode row and one prefill sequence, and a
// workspace of ts_paged_attention_workspace_bytes(); otherwise the two kernels run one after
// the other on the stream, sharing the workspace.
#include "decode_kernels.h"
#include "prefill_kernels.h"

namespace ts {

struct RaggedArgs {
  const half_t* q;
  int64_t q_st, q_sh;
  half_t* out;
  int64_t o_st, num_tokens;
  const half_t* kc;
  const half_t* vc;
  int64_t NB;
  const int* bt;
  int64_t bt_st;
  int max_blocks;
  const int* seq_lens;
  const int* qsl;
  int num_decode, H, KVH, G, HG;
  float sl2;
  // prefill tiles: launch ids [0, pf_launch)
  int pf_launch, smax, slots, P;
  float* pf_ws;
  // decode splits: launch ids [pf_launch, pf_launch + nslots * KVH * HG), slot-major (the slots
  // past the batch's last split, which exit at once, come last)
  int nslots, cap_blocks, max_splits;
  float* ws_acc;
  float* ws_m;
  float* ws_l;
  int* ws_cnt;
  // merge: decode (sequence, KV head group) workgroups first, then prefill (quarter tile, seq,
  // head) workgroups
  int dm_launch, pm_x;
};

// Share of the resident workgroup slots, in eighths, that the prefill tiles' plan gets as one
// round; the decode splits take the slots the prefill leaves. Measured on the config 5
// attention shape with the own-length decode splits and fp32 partials (cold caches, µs per call
// with the merge): 2/8 50.8, 3/8 35.9, 4/8 33.9-34.2, 5/8 31.4-32.2, 6/8 31.3-31.4, 7/8 31.9,
// 8/8 37.7.
constexpr int kRaggedPfShare = 6;

constexpr int kRaggedLds = 2 * TileLayout<128>::STAGE > DecodeLds<128, kDecodeWaves>::BYTES
                               ? 2 * TileLayout<128>::STAGE
                               : DecodeLds<128, kDecodeWaves>::BYTES;

// The decode splits' K ring: slot 0 at the start of the LDS (at least the merge's LDS long), slot
// 1 after it, kDecodeWaves x 8 KB each.
constexpr int kRaggedRing1 = (DecodeLds<128, kDecodeWaves>::BYTES + 15) / 16 > kDecodeWaves * 512
                                 ? (DecodeLds<128, kDecodeWaves>::BYTES + 15) / 16
                                 : kDecodeWaves * 512;
static_assert((kRaggedRing1 + kDecodeWaves * 512) * 16 <= kRaggedLds,
              "the decode K ring must fit in the ragged launch's LDS");

__global__ void __launch_bounds__(256, 2) ragged_split_kernel(const RaggedArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[kRaggedLds];
  const int bx = (int)blockIdx.x;
  if (bx < a.pf_launch) {
    prefill_tile_body<128>(a.q, a.q_st, a.q_sh, a.out, a.o_st, a.num_tokens, a.kc, a.vc, a.NB,
                           a.bt, a.bt_st, a.max_blocks, a.seq_lens, a.qsl, a.num_decode, a.H,
                           a.KVH, a.sl2, a.smax, a.slots, a.P, a.pf_ws, bx, lds);
  } else {
    // the decode splits run the LDS-ring form of decode_mfma_kernel: its two K slots fit in the
    // prefill tiles' LDS, the first one shared with the merge's LDS as there
    const int d = bx - a.pf_launch;
    half8_t* ring = reinterpret_cast<half8_t*>(lds);
    decode_mfma_body<128, kDecodeWaves, false, false, true>(
        a.q, a.q_st, a.q_sh, a.out, a.o_st, a.kc, a.vc, a.NB, a.bt, a.bt_st, a.max_blocks,
        a.seq_lens, a.num_decode, a.H, a.KVH, a.G, a.HG, a.sl2, a.cap_blocks, 0, a.max_splits,
        a.ws_acc, a.ws_m, a.ws_l, a.ws_cnt, d / (a.KVH * a.HG), d % (a.KVH * a.HG), lds,
        NewRows{}, nullptr, 0, ring, ring + kRaggedRing1);
  }
}

__global__ void __launch_bounds__(256) ragged_merge_kernel(const RaggedArgs a) {
  const int bx = (int)blockIdx.x;
  if (bx < a.dm_launch) {
    decode_merge_body<128>(a.ws_acc, a.ws_m, a.ws_l, a.ws_cnt, a.out, a.o_st, a.seq_lens, a.H,
                           a.G, a.HG, a.max_splits, bx % a.num_decode, bx / a.num_decode);
  } else {
    const int p = bx - a.dm_launch;
    const int x = p % a.pm_x, rest = p / a.pm_x;
    prefill_merge_body<128>(a.pf_ws, a.out, a.o_st, a.num_tokens, a.max_blocks, a.seq_lens,
                            a.qsl, a.num_decode, a.H, a.smax, a.slots, a.P, x, rest % a.P,
                            rest / a.P, a.pm_x / 4);
  }
}

// The fused plan: the prefill tiles get one round of 6/8 of the resident slots, the decode
// splits follow (the own-length schedule, as in ts_decode_attention, so a decode row's result
// does not depend on the prefill beside it). ok = false when the batch does not qualify.
struct RaggedPlan {
  bool ok;
  TilePlan pf;
  SplitPlan dec;
  size_t dec_bytes, total_bytes;
};

static RaggedPlan ragged_plan(int num_seqs, int num_decode, int max_query_len, int max_seq_len,
                              int max_prefill_seq_len, int H, int KVH, int D, int decode_version,
                              int partition, int cu_count) {
  RaggedPlan r{};
  const int P = num_seqs - num_decode;
  if (D != 128 || num_decode <= 0 || P <= 0 || max_query_len <= 0 || partition != 0 ||
      (decode_version != TS_DECODE_AUTO && decode_version != TS_DECODE_V3) || H % KVH != 0)
    return r;
  const int cus = cu_count > 0 ? cu_count : 256;
  const int64_t slots = (int64_t)cus * decode_wgs_per_cu(D);
  const int pf_seq = max_prefill_seq_len > 0 ? max_prefill_seq_len : max_seq_len;
  r.pf = tile_plan(P, H, D, max_query_len, pf_seq, cus, true, slots * kRaggedPfShare / 8);
  r.dec = plan_decode(decode_version, num_decode, H, KVH, D, max_seq_len, 0, cus);
  if (r.dec.version != TS_DECODE_V3) return r;
  r.dec_bytes = align256(ws_layout(r.dec, num_decode, H, D).total);
  r.total_bytes = r.dec_bytes + r.pf.ws_bytes;
  r.ok = true;
  return r;
}

}  // namespace ts

using namespace ts;

extern "C" size_t ts_paged_attention_workspace_bytes(int32_t num_seqs, int32_t num_decode,
                                                     int32_t max_query_len, int32_t max_seq_len,
                                                     int32_t max_prefill_seq_len,
                                                     int32_t num_heads, int32_t num_kv_heads,
                                                     int32_t head_dim, int32_t decode_version,
                                                     int32_t partition, int32_t cu_count) {
  if (num_seqs <= 0 || num_decode < 0 || num_decode > num_seqs || num_heads <= 0 ||
      num_kv_heads <= 0 || num_heads % num_kv_heads)
    return 0;
  const int pf_seq = max_prefill_seq_len > 0 ? max_prefill_seq_len : max_seq_len;
  size_t seq = 0;
  if (num_decode > 0)
    seq = ts_decode_workspace_bytes(decode_version, num_decode, num_heads, num_kv_heads, head_dim,
                                    max_seq_len, partition, cu_count);
  const size_t pf = ts_prefill_workspace_bytes(num_seqs - num_decode, num_heads, head_dim,
                                               max_query_len, pf_seq, cu_count);
  seq = seq > pf ? seq : pf;
  const RaggedPlan r = ragged_plan(num_seqs, num_decode, max_query_len, max_seq_len,
                                   max_prefill_seq_len, num_heads, num_kv_heads, head_dim,
                                   decode_version, partition, cu_count);
  return r.ok && r.total_bytes > seq ? r.total_bytes : seq;
}

extern "C" int ts_paged_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                  void* out, int64_t out_stride_t, int64_t num_tokens,
                                  const void* k_cache, const void* v_cache, int64_t num_blocks,
                                  const int32_t* block_tables, int64_t bt_stride,
                                  int32_t max_blocks_per_seq, const int32_t* seq_lens,
                                  const int32_t* query_start_loc, int32_t num_seqs,
                                  int32_t num_decode, int32_t max_query_len, int32_t max_seq_len,
                                  int32_t max_prefill_seq_len, int32_t num_heads,
                                  int32_t num_kv_heads, int32_t head_dim, float scale,
                                  int32_t decode_version, int32_t partition, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  ts::clear_error();
  TS_REQUIRE(num_decode >= 0 && num_decode <= num_seqs, TS_ERR_INVALID_ARG,
             "paged_attention: num_decode=%d outside [0, num_seqs=%d]", num_decode, num_seqs);
  TS_REQUIRE(num_decode <= num_tokens, TS_ERR_INVALID_ARG,
             "paged_attention: num_decode=%d exceeds num_tokens=%lld", num_decode,
             (long long)num_tokens);
  const int pf_seq = max_prefill_seq_len > 0 ? max_prefill_seq_len : max_seq_len;
  int cus = 0;
  if (num_decode > 0 && num_seqs > num_decode && head_dim == 128 && workspace != nullptr) {
    const int st = device_cu_count(stream, &cus);
    if (st != TS_OK) return st;
    const RaggedPlan r = ragged_plan(num_seqs, num_decode, max_query_len, max_seq_len,
                                     max_prefill_seq_len, num_heads, num_kv_heads, head_dim,
                                     decode_version, partition, cus);
    if (r.ok && workspace_bytes >= r.total_bytes && aligned(workspace, 256)) {
      // The argument checks of the two standalone entry points, which the sequential path
      // below performs as it calls them.
      TS_REQUIRE(q && out && k_cache && v_cache && block_tables && seq_lens && query_start_loc,
                 TS_ERR_INVALID_ARG, "paged_attention: null pointer argument");
      TS_REQUIRE(num_blocks > 0 && max_blocks_per_seq > 0 && bt_stride >= max_blocks_per_seq,
                 TS_ERR_INVALID_ARG, "paged_attention: bad block table");
      TS_REQUIRE(q_stride_t % 8 == 0 && q_stride_h % 8 == 0 && out_stride_t % 4 == 0 &&
                     aligned(q, 16) && aligned(out, 8) && aligned(k_cache, 16) &&
                     aligned(v_cache, 16),
                 TS_ERR_INVALID_ARG, "paged_attention: misaligned q / out / caches");
      const int P = num_seqs - num_decode;
      RaggedArgs a{};
      a.q = static_cast<const half_t*>(q);
      a.q_st = q_stride_t;
      a.q_sh = q_stride_h;
      a.out = static_cast<half_t*>(out);
      a.o_st = out_stride_t;
      a.num_tokens = num_tokens;
      a.kc = static_cast<const half_t*>(k_cache);
      a.vc = static_cast<const half_t*>(v_cache);
      a.NB = num_blocks;
      a.bt = block_tables;
      a.bt_st = bt_stride;
      a.max_blocks = max_blocks_per_seq;
      a.seq_lens = seq_lens;
      a.qsl = query_start_loc;
      a.num_decode = num_decode;
      a.H = num_heads;
      a.KVH = num_kv_heads;
      a.G = num_heads / num_kv_heads;
      a.HG = (a.G + 15) / 16;
      a.sl2 = scale * kLog2e;
      const int per_kvh = r.pf.slots * P * a.G;
      a.pf_launch = 8 % num_kv_heads == 0 ? 8 * cdiv(per_kvh, 8 / num_kv_heads)
                                          : per_kvh * num_kv_heads;
      a.smax = r.pf.ws_bytes > 0 ? r.pf.smax : 1 << 30;   // unsplit: no tile leaves partials
      a.slots = r.pf.slots;
      a.P = P;
      char* ws = static_cast<char*>(workspace);
      a.pf_ws = reinterpret_cast<float*>(ws + r.dec_bytes);
      const WsLayout w = ws_layout(r.dec, num_decode, num_heads, head_dim);
      a.ws_acc = reinterpret_cast<float*>(ws + w.acc);
      a.ws_m = reinterpret_cast<float*>(ws + w.m);
      a.ws_l = reinterpret_cast<float*>(ws + w.l);
      a.ws_cnt = reinterpret_cast<int*>(ws + w.cnt);
      a.nslots = r.dec.nslots;
      a.cap_blocks = r.dec.cap_blocks < max_blocks_per_seq ? r.dec.cap_blocks : max_blocks_per_seq;
      a.max_splits = r.dec.max_splits;
      a.dm_launch = num_decode * num_kv_heads * a.HG;
      a.pm_x = 4 * cdiv(max_query_len, kTileRows);
      const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
      const int n_split = a.pf_launch + a.nslots * num_kv_heads * a.HG;
      ragged_split_kernel<<<n_split, 256, 0, s>>>(a);
      ragged_merge_kernel<<<a.dm_launch + a.pm_x * P * num_heads, 256, 0, s>>>(a);
      return check_launch("paged_attention");
    }
  }
  if (num_decode > 0) {
    const int st = ts_decode_attention(decode_version, q, q_stride_t, q_stride_h, out,
                                       out_stride_t, k_cache, v_cache, num_blocks, block_tables,
                                       bt_stride, max_blocks_per_seq, seq_lens, num_decode,
                                       num_heads, num_kv_heads, head_dim, scale, max_seq_len,
                                       partition, workspace, workspace_bytes, stream,
                                       nullptr, 0);
    if (st != TS_OK) return st;
  }
  if (num_seqs > num_decode) {
    // Stream-ordered after the decode kernels, so the prefill reuses the same workspace.
    const int st = ts_prefill_attention_ws(q, q_stride_t, q_stride_h, out, out_stride_t,
                                           num_tokens, k_cache, v_cache, num_blocks, block_tables,
                                           bt_stride, max_blocks_per_seq, seq_lens,
                                           query_start_loc, num_seqs, num_decode, max_query_len,
                                           pf_seq, num_heads, num_kv_heads, head_dim, scale,
                                           workspace, workspace_bytes, stream);
    if (st != TS_OK) return st;
  }
  return TS_OK;
}
