// Paged chunked-prefill attention for gfx950 (ops/triton_prefill_attention.py:17-79).
// Host entry points; the kernels and their launch plans are in prefill_kernels.h (head_dim < 128)
// and prefill_pair.h (head_dim 128).
#include "prefill_pair.h"

using namespace ts;

namespace {

// head_dim 128 runs one of two kernels. The paired kernel (two 128-row units per 512-thread
// workgroup, one workgroup per CU, stream-K key-range slots) wins when each launch slot has many
// key steps; with few steps per slot its per-segment prologue, partials and merge dominate and
// the 4-wavefront tile kernel (two workgroups per CU, split plan sized for one resident round)
// is faster. Measured on MI355X (H 12, KVH 2; us per call, tile / paired, and the host-bound
// steps per paired slot): 512 rows on a 1037 prefix 28.0 / 34.0 (2.4), 2048 on 0 39.6 / 43.3
// (12.2), 1024 on 0 21.8 / 28.9 (3.0), 2048 on 2048 67.8 / 65.7 (24.4), 2048 on 4096 99.6 / 89.7
// (36.6), 1856 on 6144 125.5 / 106.2 (44.6).
constexpr int kPairMinSlotSteps = 16;

bool pair_pays(const PairPlan& pl, int num_heads, int num_kv_heads, int max_query_len,
               int max_seq_len) {
  if (pl.seg_cap == 0) return true;                // no split: the paired kernel as is
  const int tr = pair_heads(num_heads, num_kv_heads) ? kTileRows : 2 * kTileRows;
  const int seq = max_seq_len > max_query_len ? max_seq_len : max_query_len;
  const int64_t bound = (int64_t)cdiv(max_query_len, tr) * cdiv(seq, kTileKeys);
  return bound >= (int64_t)kPairMinSlotSteps * pl.slots;
}

// Shared body of the prefill entry points. With `workspace` the head_dim 128 kernels may split
// long key ranges; a workspace smaller than the plan needs runs the paired kernel unsplit.
int prefill_launch(const void* q, int64_t q_stride_t, int64_t q_stride_h, void* out,
                   int64_t out_stride_t, int64_t num_tokens, const void* k_cache,
                   const void* v_cache, int64_t num_blocks, const int32_t* block_tables,
                   int64_t bt_stride, int32_t max_blocks_per_seq, const int32_t* seq_lens,
                   const int32_t* query_start_loc, int32_t num_seqs, int32_t num_decode,
                   int32_t max_query_len, int32_t max_seq_len, int32_t num_heads,
                   int32_t num_kv_heads, int32_t head_dim, float scale, void* workspace,
                   size_t workspace_bytes, void* stream) {
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
  const float sl2 = scale * kLog2eP;
  if (head_dim == 128) {
    int cus = 0;
    if (workspace != nullptr && device_cu_count(stream, &cus) != TS_OK) return TS_ERR_DEVICE;
    PairPlan pl = pair_plan(P, num_heads, num_kv_heads, max_query_len, max_seq_len, cus,
                            workspace != nullptr);
    if (!pair_pays(pl, num_heads, num_kv_heads, max_query_len, max_seq_len)) {
      TilePlan tp = tile_plan(P, num_heads, head_dim, max_query_len, max_seq_len, cus, true);
      if (tp.ws_bytes <= workspace_bytes && (tp.ws_bytes == 0 || aligned(workspace, 16))) {
        if (tp.ws_bytes == 0) tp.smax = 1 << 30;     // unsplit: no tile leaves partials
        const int per_kvh = tp.slots * P * (num_heads / num_kv_heads);
        const int n_launch = 8 % num_kv_heads == 0 ? 8 * cdiv(per_kvh, 8 / num_kv_heads)
                                                    : per_kvh * num_kv_heads;
        prefill_tile_kernel<128><<<n_launch, kTileThreads, 0, s>>>(
            static_cast<const half_t*>(q), q_stride_t, q_stride_h, static_cast<half_t*>(out),
            out_stride_t, num_tokens, static_cast<const half_t*>(k_cache),
            static_cast<const half_t*>(v_cache), num_blocks, block_tables, bt_stride,
            max_blocks_per_seq, seq_lens, query_start_loc, num_decode, num_heads, num_kv_heads,
            sl2, tp.smax, tp.slots, P, static_cast<float*>(workspace));
        if (tp.ws_bytes > 0)
          prefill_merge_kernel<128><<<dim3(4 * cdiv(max_query_len, kTileRows), P, num_heads),
                                      kTileThreads, 0, s>>>(
              static_cast<const float*>(workspace), static_cast<half_t*>(out), out_stride_t,
              num_tokens, max_blocks_per_seq, seq_lens, query_start_loc, num_decode, num_heads,
              tp.smax, tp.slots);
        return check_launch("prefill_attention");
      }
    }
    if (pl.ws_bytes > workspace_bytes || (pl.ws_bytes > 0 && !aligned(workspace, 16)))
      pl = pair_plan(P, num_heads, num_kv_heads, max_query_len, max_seq_len, cus, false);
    const bool heads = pair_heads(num_heads, num_kv_heads);
    const int per_kvh = pl.slots * P * (num_heads / num_kv_heads / (heads ? 2 : 1));
    const int n_launch = 8 % num_kv_heads == 0 ? 8 * cdiv(per_kvh, 8 / num_kv_heads)
                                                : per_kvh * num_kv_heads;
    prefill_pair_kernel<<<n_launch, kPairThreads, 0, s>>>(
        static_cast<const half_t*>(q), q_stride_t, q_stride_h, static_cast<half_t*>(out),
        out_stride_t, num_tokens, static_cast<const half_t*>(k_cache),
        static_cast<const half_t*>(v_cache), num_blocks, block_tables, bt_stride,
        max_blocks_per_seq, seq_lens, query_start_loc, num_decode, num_heads, num_kv_heads, sl2,
        pl.slots, pl.seg_cap, P, static_cast<float*>(workspace));
    if (pl.seg_cap > 0)
      prefill_pair_merge_kernel<<<dim3(4 * cdiv(max_query_len, kTileRows), P, num_heads),
                                  kTileThreads, 0, s>>>(
          static_cast<const float*>(workspace), static_cast<half_t*>(out), out_stride_t,
          num_tokens, max_blocks_per_seq, seq_lens, query_start_loc, num_decode, num_heads,
          num_kv_heads, pl.slots, pl.seg_cap);
    return check_launch("prefill_attention");
  }
  const dim3 grid((max_query_len + kPsRows - 1) / kPsRows, P, num_heads);
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
  }
#undef TS_PF_CASE
  return check_launch("prefill_attention");
}

}  // namespace

extern "C" size_t ts_prefill_workspace_bytes(int32_t num_prefill, int32_t num_heads,
                                             int32_t head_dim, int32_t max_query_len,
                                             int32_t max_seq_len, int32_t cu_count) {
  if (num_prefill <= 0 || num_heads <= 0 || head_dim != 128 || max_query_len <= 0) return 0;
  // The paired plan depends on whether the GQA group size is even (not an argument here), and
  // short splits take the tile plan instead: enough for every form.
  const size_t a = pair_plan(num_prefill, num_heads, 1, max_query_len, max_seq_len, cu_count,
                             true).ws_bytes;
  const size_t b = pair_plan(num_prefill, num_heads, num_heads, max_query_len, max_seq_len,
                             cu_count, true).ws_bytes;
  const size_t c = tile_plan(num_prefill, num_heads, head_dim, max_query_len, max_seq_len,
                             cu_count, true).ws_bytes;
  const size_t ab = a > b ? a : b;
  return ab > c ? ab : c;
}

extern "C" int ts_prefill_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                    void* out, int64_t out_stride_t, int64_t num_tokens,
                                    const void* k_cache, const void* v_cache, int64_t num_blocks,
                                    const int32_t* block_tables, int64_t bt_stride,
                                    int32_t max_blocks_per_seq, const int32_t* seq_lens,
                                    const int32_t* query_start_loc, int32_t num_seqs,
                                    int32_t num_decode, int32_t max_query_len, int32_t num_heads,
                                    int32_t num_kv_heads, int32_t head_dim, float scale,
                                    void* stream) {
  ts::clear_error();
  return prefill_launch(q, q_stride_t, q_stride_h, out, out_stride_t, num_tokens, k_cache,
                        v_cache, num_blocks, block_tables, bt_stride, max_blocks_per_seq, seq_lens,
                        query_start_loc, num_seqs, num_decode, max_query_len, max_query_len,
                        num_heads, num_kv_heads, head_dim, scale, nullptr, 0, stream);
}

extern "C" int ts_prefill_attention_ws(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                       void* out, int64_t out_stride_t, int64_t num_tokens,
                                       const void* k_cache, const void* v_cache,
                                       int64_t num_blocks, const int32_t* block_tables,
                                       int64_t bt_stride, int32_t max_blocks_per_seq,
                                       const int32_t* seq_lens, const int32_t* query_start_loc,
                                       int32_t num_seqs, int32_t num_decode,
                                       int32_t max_query_len, int32_t max_seq_len,
                                       int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                       float scale, void* workspace, size_t workspace_bytes,
                                       void* stream) {
  ts::clear_error();
  return prefill_launch(q, q_stride_t, q_stride_h, out, out_stride_t, num_tokens, k_cache,
                        v_cache, num_blocks, block_tables, bt_stride, max_blocks_per_seq, seq_lens,
                        query_start_loc, num_seqs, num_decode, max_query_len, max_seq_len,
                        num_heads, num_kv_heads, head_dim, scale, workspace, workspace_bytes,
                        stream);
}
