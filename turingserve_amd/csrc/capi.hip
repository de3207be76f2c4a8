// C ABI plumbing: version, thread-local error messages, device queries and the
// paged_attention dispatcher (decode rows, then prefill sequences), which mirrors
// ops/triton_ops.py:60-71.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace ts {

static thread_local char g_err[512] = "";

int set_error(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return status;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(TS_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return TS_OK;
}

int device_cu_count(int* out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(TS_ERR_DEVICE, "hipGetDevice failed");
  return ts_device_cu_count(dev, out);
}

}  // namespace ts

extern "C" const char* ts_version(void) { return "turingserve_hip 0.1.0 gfx950"; }

extern "C" const char* ts_last_error(void) { return ts::g_err; }

extern "C" int ts_device_cu_count(int device, int* cu_count) {
  TS_REQUIRE(cu_count != nullptr, TS_ERR_INVALID_ARG, "device_cu_count: null output");
  // One cached answer per device (a startup query, like utils/gpu.py:19-24 behind lru_cache).
  static int cache[64] = {0};
  if (device >= 0 && device < 64 && cache[device] > 0) {
    *cu_count = cache[device];
    return TS_OK;
  }
  int n = 0;
  hipError_t e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device);
  if (e != hipSuccess || n <= 0)
    return ts::set_error(TS_ERR_DEVICE, "device_cu_count: hipDeviceGetAttribute failed: %s",
                         hipGetErrorString(e));
  if (device >= 0 && device < 64) cache[device] = n;
  *cu_count = n;
  return TS_OK;
}

extern "C" int ts_paged_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                  void* out, int64_t out_stride_t, int64_t num_tokens,
                                  const void* k_cache, const void* v_cache, int64_t num_blocks,
                                  const int32_t* block_tables, int64_t bt_stride,
                                  int32_t max_blocks_per_seq, const int32_t* seq_lens,
                                  const int32_t* query_start_loc, int32_t num_seqs,
                                  int32_t num_decode, int32_t max_query_len, int32_t max_seq_len,
                                  int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                  float scale, int32_t decode_version, int32_t partition,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  TS_REQUIRE(num_decode >= 0 && num_decode <= num_seqs, TS_ERR_INVALID_ARG,
             "paged_attention: num_decode=%d outside [0, num_seqs=%d]", num_decode, num_seqs);
  TS_REQUIRE(num_decode <= num_tokens, TS_ERR_INVALID_ARG,
             "paged_attention: num_decode=%d exceeds num_tokens=%lld", num_decode,
             (long long)num_tokens);
  if (num_decode > 0) {
    int st = ts_decode_attention(decode_version, q, q_stride_t, q_stride_h, out, out_stride_t,
                                 k_cache, v_cache, num_blocks, block_tables, bt_stride,
                                 max_blocks_per_seq, seq_lens, num_decode, num_heads, num_kv_heads,
                                 head_dim, scale, max_seq_len, partition, workspace,
                                 workspace_bytes, stream);
    if (st != TS_OK) return st;
  }
  if (num_seqs > num_decode) {
    // Stream-ordered after the decode kernels, so the prefill reuses the same workspace.
    int st = ts_prefill_attention_ws(q, q_stride_t, q_stride_h, out, out_stride_t, num_tokens,
                                     k_cache, v_cache, num_blocks, block_tables, bt_stride,
                                     max_blocks_per_seq, seq_lens, query_start_loc, num_seqs,
                                     num_decode, max_query_len, max_seq_len, num_heads,
                                     num_kv_heads, head_dim, scale, workspace, workspace_bytes,
                                     stream);
    if (st != TS_OK) return st;
  }
  return TS_OK;
}
