// Paged decode attention for gfx950 (ops/triton_decode_attention.py, ops/triton_ops.py:35-57).
// Host entry points; the kernels and their launch plans are in decode_kernels.h.
#include <mutex>

#include "decode_kernels.h"

using namespace ts;

extern "C" size_t ts_decode_workspace_bytes(int32_t version, int32_t num_seqs, int32_t num_heads,
                                            int32_t num_kv_heads, int32_t head_dim,
                                            int32_t max_seq_len, int32_t partition,
                                            int32_t cu_count) {
  if (num_seqs <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return 0;
  const SplitPlan p = plan_decode(version, num_seqs, num_heads, num_kv_heads, head_dim,
                                  max_seq_len, partition, cu_count > 0 ? cu_count : 256);
  return ws_layout(p, num_seqs, num_heads, head_dim).total;
}

extern "C" size_t ts_decode_split_map_bytes(int32_t version, int32_t num_seqs, int32_t num_heads,
                                            int32_t num_kv_heads, int32_t head_dim,
                                            int32_t max_seq_len, int32_t partition,
                                            int32_t cu_count) {
  if (num_seqs <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return 0;
  if (num_seqs > kMapMaxSeqs) return 0;
  const SplitPlan p = plan_decode(version, num_seqs, num_heads, num_kv_heads, head_dim,
                                  max_seq_len, partition, cu_count > 0 ? cu_count : 256);
  return map_bytes_of(p, num_seqs, num_kv_heads * ((num_heads / num_kv_heads + 15) / 16));
}

extern "C" int ts_decode_split_map(int32_t version, const int32_t* block_tables, int64_t bt_stride,
                                   int32_t max_blocks_per_seq, int64_t num_blocks,
                                   const int32_t* seq_lens, int32_t num_seqs, int32_t num_heads,
                                   int32_t num_kv_heads, int32_t head_dim, int32_t max_seq_len,
                                   int32_t partition, void* split_map, size_t split_map_bytes,
                                   void* stream) {
  ts::clear_error();
  TS_REQUIRE(version >= TS_DECODE_AUTO && version <= TS_DECODE_V3, TS_ERR_INVALID_ARG,
             "decode_split_map: unknown version %d", version);
  TS_REQUIRE(num_seqs >= 0 && num_seqs <= kMapMaxSeqs, TS_ERR_UNSUPPORTED,
             "decode_split_map: %d sequences (the map builder handles 0 .. %d; launch without a map)",
             num_seqs, kMapMaxSeqs);
  if (num_seqs == 0) return TS_OK;
  TS_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
             TS_ERR_INVALID_ARG, "decode_split_map: num_heads=%d not a multiple of num_kv_heads=%d",
             num_heads, num_kv_heads);
  TS_REQUIRE(block_tables && seq_lens, TS_ERR_INVALID_ARG, "decode_split_map: null pointer argument");
  TS_REQUIRE(num_blocks > 0 && max_blocks_per_seq > 0 && bt_stride >= max_blocks_per_seq,
             TS_ERR_INVALID_ARG, "decode_split_map: bad block table (num_blocks=%lld width=%d stride=%lld)",
             (long long)num_blocks, max_blocks_per_seq, (long long)bt_stride);
  TS_REQUIRE(partition >= 0 && partition % kBlockSize == 0, TS_ERR_INVALID_ARG,
             "decode_split_map: partition %d is not a multiple of 16", partition);
  int cus = 0;
  int st = device_cu_count(stream, &cus);
  if (st != TS_OK) return st;
  const SplitPlan p = plan_decode(version, num_seqs, num_heads, num_kv_heads, head_dim,
                                  max_seq_len, partition, cus);
  const int groups = num_kv_heads * ((num_heads / num_kv_heads + 15) / 16);
  const size_t need = map_bytes_of(p, num_seqs, groups);
  if (need == 0) return TS_OK;                 // this plan does not split: no map
  TS_REQUIRE(split_map && split_map_bytes >= need && aligned(split_map, 16), TS_ERR_WORKSPACE,
             "decode_split_map: map of %zu bytes (16-byte aligned) needed, got %zu", need,
             split_map_bytes);
  launch_split_map(p, reinterpret_cast<hipStream_t>(stream), seq_lens, block_tables, bt_stride,
                   num_blocks, max_blocks_per_seq, num_seqs, groups, static_cast<int*>(split_map));
  return check_launch("decode_split_map");
}

// Shared by the entry points; nr.k set: kv_write fused into the attention launch.
static int decode_entry(int32_t version, const void* q, int64_t q_stride_t, int64_t q_stride_h,
                        void* out, int64_t out_stride_t, const void* k_cache, const void* v_cache,
                        int64_t num_blocks, const int32_t* block_tables, int64_t bt_stride,
                        int32_t max_blocks_per_seq, const int32_t* seq_lens, int32_t num_seqs,
                        int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float scale,
                        int32_t max_seq_len, int32_t partition, void* workspace,
                        size_t workspace_bytes, void* stream, const NewRows& nr,
                        const void* split_map, size_t split_map_bytes) {
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
  int st = device_cu_count(stream, &cus);
  if (st != TS_OK) return st;
  const SplitPlan p = plan_decode(version, num_seqs, num_heads, num_kv_heads, head_dim,
                                  max_seq_len, partition, cus);
  const size_t need = ws_layout(p, num_seqs, num_heads, head_dim).total;
  TS_REQUIRE(need == 0 || (workspace && workspace_bytes >= need && aligned(workspace, 256)),
             TS_ERR_WORKSPACE, "decode_attention: workspace of %zu bytes (256-aligned) needed, got %zu",
             need, workspace_bytes);
  const size_t map_need =
      split_map ? map_bytes_of(p, num_seqs, num_kv_heads * ((num_heads / num_kv_heads + 15) / 16)) : 0;
  TS_REQUIRE(map_need == 0 || (split_map_bytes >= map_need && aligned(split_map, 16)),
             TS_ERR_INVALID_ARG,
             "decode_attention: split map of %zu bytes (16-byte aligned) needed for this plan, got %zu",
             map_need, split_map_bytes);
  // the map's arrival counters are written in place (and left at zero) by the in-launch merge
  int* smap = map_need ? static_cast<int*>(const_cast<void*>(split_map)) : nullptr;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (nr.k) {
    // The fused write needs the MFMA kernels with one head group per KV head (so the workgroup
    // that writes a block is the only one reading it) and 16-byte row pieces, the fused RoPE
    // also a head_dim that keeps each rotation pair in one lane; otherwise the rows go through
    // kv_write's (or rope_kv_write's) own launch first.
    const bool rope = nr.cos_t != nullptr;
    const bool fused = p.version != TS_DECODE_V1 && num_heads / num_kv_heads <= 16 &&
                       head_dim % 8 == 0 && nr.k_st % 8 == 0 && nr.k_sh % 8 == 0 &&
                       nr.v_st % 8 == 0 && nr.v_sh % 8 == 0 && aligned(nr.k, 16) &&
                       aligned(nr.v, 16) && aligned(k_cache, 16) && aligned(v_cache, 16) &&
                       (!rope || head_dim % 64 == 0);
    if (!fused) {
      if (rope)
        st = ts_rope_kv_write(nr.qkv, nr.qkv_st, nr.positions, nr.cos_t, nr.sin_t, nr.max_pos,
                              num_seqs, num_heads, num_kv_heads, head_dim,
                              const_cast<void*>(k_cache), const_cast<void*>(v_cache), num_blocks,
                              nr.slots, stream);
      else
        st = ts_kv_write(nr.k, nr.v, nr.k_st, nr.k_sh, nr.v_st, nr.v_sh,
                         const_cast<void*>(k_cache), const_cast<void*>(v_cache), num_blocks,
                         nr.slots, num_seqs, num_kv_heads, head_dim, stream);
      if (st != TS_OK) return st;
      return decode_entry(version, q, q_stride_t, q_stride_h, out, out_stride_t, k_cache, v_cache,
                          num_blocks, block_tables, bt_stride, max_blocks_per_seq, seq_lens,
                          num_seqs, num_heads, num_kv_heads, head_dim, scale, max_seq_len,
                          partition, workspace, workspace_bytes, stream, NewRows{}, split_map,
                          split_map_bytes);
    }
  }
  const float sl2 = scale * kLog2e;
  const half_t* qp = static_cast<const half_t*>(q);
  half_t* op = static_cast<half_t*>(out);
  const half_t* kp = static_cast<const half_t*>(k_cache);
  const half_t* vp = static_cast<const half_t*>(v_cache);
#define TS_DECODE_CASE(DD)                                                                      \
  case DD:                                                                                      \
    launch_decode<DD>(p, s, qp, q_stride_t, q_stride_h, op, out_stride_t, kp, vp, num_blocks,  \
                      block_tables, bt_stride, max_blocks_per_seq, seq_lens, num_seqs, num_heads, \
                      num_kv_heads, sl2, workspace, nr, smap);                                  \
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

extern "C" int ts_decode_attention(int32_t version, const void* q, int64_t q_stride_t,
                                   int64_t q_stride_h, void* out, int64_t out_stride_t,
                                   const void* k_cache, const void* v_cache, int64_t num_blocks,
                                   const int32_t* block_tables, int64_t bt_stride,
                                   int32_t max_blocks_per_seq, const int32_t* seq_lens,
                                   int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                   int32_t head_dim, float scale, int32_t max_seq_len,
                                   int32_t partition, void* workspace, size_t workspace_bytes,
                                   void* stream, const void* split_map, size_t split_map_bytes) {
  ts::clear_error();
  return decode_entry(version, q, q_stride_t, q_stride_h, out, out_stride_t, k_cache, v_cache,
                      num_blocks, block_tables, bt_stride, max_blocks_per_seq, seq_lens, num_seqs,
                      num_heads, num_kv_heads, head_dim, scale, max_seq_len, partition, workspace,
                      workspace_bytes, stream, NewRows{}, split_map, split_map_bytes);
}

extern "C" int ts_decode_attention_kv_write(
    int32_t version, const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k,
    const void* v, int64_t k_stride_t, int64_t k_stride_h, int64_t v_stride_t,
    int64_t v_stride_h, const int64_t* slot_mapping, void* out, int64_t out_stride_t,
    void* k_cache, void* v_cache, int64_t num_blocks, const int32_t* block_tables,
    int64_t bt_stride, int32_t max_blocks_per_seq, const int32_t* seq_lens, int32_t num_seqs,
    int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float scale, int32_t max_seq_len,
    int32_t partition, void* workspace, size_t workspace_bytes, void* stream,
    const void* split_map, size_t split_map_bytes) {
  ts::clear_error();
  TS_REQUIRE(num_seqs >= 0, TS_ERR_INVALID_ARG, "decode_attention_kv_write: num_seqs %d < 0",
             num_seqs);
  if (num_seqs == 0) return TS_OK;
  TS_REQUIRE(k && v && slot_mapping, TS_ERR_INVALID_ARG,
             "decode_attention_kv_write: null pointer argument");
  TS_REQUIRE(k_stride_t >= 0 && k_stride_h >= 0 && v_stride_t >= 0 && v_stride_h >= 0,
             TS_ERR_INVALID_ARG, "decode_attention_kv_write: negative stride");
  const NewRows nr{static_cast<const half_t*>(k), static_cast<const half_t*>(v), k_stride_t,
                   k_stride_h, v_stride_t, v_stride_h, slot_mapping,
                   num_blocks * (int64_t)kBlockSize, nullptr, nullptr, nullptr, 0, nullptr, 0};
  return decode_entry(version, q, q_stride_t, q_stride_h, out, out_stride_t, k_cache, v_cache,
                      num_blocks, block_tables, bt_stride, max_blocks_per_seq, seq_lens, num_seqs,
                      num_heads, num_kv_heads, head_dim, scale, max_seq_len, partition, workspace,
                      workspace_bytes, stream, nr, split_map, split_map_bytes);
}

// ---------------------------------------------------------------------------------------------
// ts_decode_attention_kv_write_noalloc: the same launch with its split-K scratch in `scratch`,
// a library-owned device array (one copy per GPU, held until the process ends), so the call
// allocates nothing. The split kernel writes every partial row, and every split count, that the
// merge kernel reads in the same call (rows past a sequence's split count are skipped, a padding
// row reads none), so stale contents from an earlier call never matter and nothing is cleared.
// Calls that overlap on one GPU (two streams, two threads) share the array and race.
// ---------------------------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[TS_NOALLOC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
static void* g_scratch_addr[kMaxDevices];      // device address of `scratch`, per device

// Device address of `scratch` on `dev`, looked up once per device with that device current (the
// host-side name of a __device__ array is not a device address).
static int scratch_address(int dev, void** addr) {
  TS_REQUIRE(dev >= 0 && dev < kMaxDevices, TS_ERR_DEVICE, "noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || p == nullptr)
      return set_error(TS_ERR_DEVICE, "noalloc: hipGetSymbolAddress of the scratch failed: %s",
                       hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return TS_OK;
}

extern "C" int ts_decode_attention_kv_write_noalloc(
    int32_t version, const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k,
    const void* v, int64_t k_stride_t, int64_t k_stride_h, int64_t v_stride_t,
    int64_t v_stride_h, const int64_t* slot_mapping, void* out, int64_t out_stride_t,
    void* k_cache, void* v_cache, int64_t num_blocks, const int32_t* block_tables,
    int64_t bt_stride, int32_t max_blocks_per_seq, const int32_t* seq_lens, int32_t num_seqs,
    int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float scale, int32_t max_seq_len,
    int32_t partition, void* stream) {
  ts::clear_error();
  TS_REQUIRE(num_seqs >= 0, TS_ERR_INVALID_ARG,
             "decode_attention_kv_write_noalloc: num_seqs %d < 0", num_seqs);
  if (num_seqs == 0) return TS_OK;
  int dev = 0, cus = 0;
  int st = stream_device(stream, &dev);
  if (st == TS_OK) st = ts_device_cu_count(dev, &cus);
  if (st != TS_OK) return st;
  const size_t need = ts_decode_workspace_bytes(version, num_seqs, num_heads, num_kv_heads,
                                                head_dim, max_seq_len, partition, cus);
  TS_REQUIRE(need <= TS_NOALLOC_SCRATCH_BYTES, TS_ERR_WORKSPACE,
             "decode_attention_kv_write_noalloc: this batch (%d sequences, %d heads, head_dim %d) "
             "needs %zu bytes of split scratch, the static scratch holds %zu; call "
             "ts_decode_attention_kv_write with a workspace instead",
             num_seqs, num_heads, head_dim, need, (size_t)TS_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0) {
    st = scratch_address(dev, &ws);
    if (st != TS_OK) return st;
  }
  return ts_decode_attention_kv_write(version, q, q_stride_t, q_stride_h, k, v, k_stride_t,
                                      k_stride_h, v_stride_t, v_stride_h, slot_mapping, out,
                                      out_stride_t, k_cache, v_cache, num_blocks, block_tables,
                                      bt_stride, max_blocks_per_seq, seq_lens, num_seqs, num_heads,
                                      num_kv_heads, head_dim, scale, max_seq_len, partition, ws,
                                      need > 0 ? (size_t)TS_NOALLOC_SCRATCH_BYTES : 0, stream,
                                      nullptr, 0);
}

extern "C" int ts_decode_rope_kv_write_attention(
    int32_t version, void* qkv, int64_t qkv_stride, const int64_t* positions,
    const float* cos_table, const float* sin_table, int64_t max_position, void* out,
    int64_t out_stride_t, void* k_cache, void* v_cache, int64_t num_blocks,
    const int64_t* slot_mapping, const int32_t* block_tables, int64_t bt_stride,
    int32_t max_blocks_per_seq, const int32_t* seq_lens, int32_t num_seqs, int32_t num_heads,
    int32_t num_kv_heads, int32_t head_dim, float scale, int32_t max_seq_len, int32_t partition,
    void* workspace, size_t workspace_bytes, void* stream, const void* split_map,
    size_t split_map_bytes) {
  ts::clear_error();
  TS_REQUIRE(num_seqs >= 0, TS_ERR_INVALID_ARG,
             "decode_rope_kv_write_attention: num_seqs %d < 0", num_seqs);
  if (num_seqs == 0) return TS_OK;
  TS_REQUIRE(qkv && positions && cos_table && sin_table && slot_mapping && max_position > 0,
             TS_ERR_INVALID_ARG, "decode_rope_kv_write_attention: null pointer or empty table");
  TS_REQUIRE(num_heads > 0 && num_kv_heads > 0 && head_dim > 0 && head_dim % 8 == 0,
             TS_ERR_INVALID_ARG, "decode_rope_kv_write_attention: bad heads or head_dim %d",
             head_dim);
  TS_REQUIRE(qkv_stride >= (int64_t)(num_heads + 2 * num_kv_heads) * head_dim &&
                 qkv_stride % 8 == 0 && aligned(qkv, 16) && aligned(cos_table, 16) &&
                 aligned(sin_table, 16),
             TS_ERR_INVALID_ARG,
             "decode_rope_kv_write_attention: qkv rows and tables must be 16-byte aligned");
  half_t* base = static_cast<half_t*>(qkv);
  const int64_t kv_off = (int64_t)num_heads * head_dim;
  const NewRows nr{base + kv_off, base + kv_off + (int64_t)num_kv_heads * head_dim, qkv_stride,
                   head_dim, qkv_stride, head_dim, slot_mapping,
                   num_blocks * (int64_t)kBlockSize, positions, cos_table, sin_table,
                   max_position, qkv, qkv_stride};
  return decode_entry(version, qkv, qkv_stride, head_dim, out, out_stride_t, k_cache, v_cache,
                      num_blocks, block_tables, bt_stride, max_blocks_per_seq, seq_lens, num_seqs,
                      num_heads, num_kv_heads, head_dim, scale, max_seq_len, partition, workspace,
                      workspace_bytes, stream, nr, split_map, split_map_bytes);
}
