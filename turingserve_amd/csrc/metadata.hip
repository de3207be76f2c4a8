// Per-step attention metadata built on the GPU from compact per-sequence descriptors
// (runner/input_builder.py:81-150 and the decode-graph padding of runner/cuda_graphs.py:62-78).
//
// The host uploads one packed int32 buffer (one copy instead of seven) and this kernel expands it
// into the flat token rows and per-sequence tables the attention kernels read:
//   desc[i]   = {start, n_tokens, sample (0 none, 1 last, 2 all), table_offset, table_len}
//   tokens    = the n_tokens ids of every sequence, in order
//   block ids = every sequence's block table, concatenated (table_offset / table_len index it)
// Row t of sequence i (token offset off_i = n_0 + ... + n_{i-1}) gets
//   input_ids = token, position = start + t,
//   slot_mapping = table[(start + t) / 16] * 16 + (start + t) % 16   (-1 past the table),
// and the sequence gets query_start_loc[i + 1] = off_i + n_i, seq_lens[i] = start + n_i, its
// table row padded with block 0 (the null block) to bt_width, and its sample rows (the last
// row, every row or none) at the running sample offset. Sequences num_seqs .. pad_seqs - 1 are
// padding rows of a captured decode graph: one token 0 at position 0 with slot -1, seq_len 0,
// an all-zero table row.
//
// One workgroup per (possibly padding) sequence; each sums the token and sample counts of the
// sequences before it (a block-wide reduction; at most max_seqs descriptors), so no separate scan
// launch is needed.
#include "common.h"

namespace ts {

constexpr int kMetaThreads = 256;
constexpr int kDescWords = 5;

__device__ __forceinline__ int block_sum_int(int v, int* s_red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  __syncthreads();                                  // s_red may hold a previous sum
  if (lane == 0) s_red[w] = v;
  __syncthreads();
  return (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
}

__global__ void __launch_bounds__(kMetaThreads) step_metadata_kernel(
    const int32_t* __restrict__ packed, int num_seqs, int64_t num_tokens, int64_t num_block_ids,
    int bt_width, int64_t bt_stride, int64_t* __restrict__ input_ids,
    int64_t* __restrict__ positions, int64_t* __restrict__ slot_mapping,
    int32_t* __restrict__ qsl, int32_t* __restrict__ seq_lens, int32_t* __restrict__ block_tables,
    int64_t* __restrict__ sample_indices) {
  __shared__ int s_red[kMetaThreads / kWave];
  const int i = blockIdx.x, tid = threadIdx.x;
  const int32_t* desc = packed;
  const int32_t* tokens = packed + (int64_t)kDescWords * num_seqs;
  const int32_t* blocks = tokens + num_tokens;
  int32_t* bt_row = block_tables + (int64_t)i * bt_stride;

  if (i >= num_seqs) {                              // padding sequence of a decode graph
    const int64_t row = num_tokens + (i - num_seqs);
    if (tid == 0) {
      input_ids[row] = 0;
      positions[row] = 0;
      slot_mapping[row] = -1;
      seq_lens[i] = 0;
      qsl[i + 1] = (int32_t)(row + 1);
      if (i == 0) qsl[0] = 0;
    }
    for (int j = tid; j < bt_width; j += kMetaThreads) bt_row[j] = 0;
    return;
  }

  int tok = 0, smp = 0;
  for (int j = tid; j < i; j += kMetaThreads) {
    const int n = desc[kDescWords * j + 1], mode = desc[kDescWords * j + 2];
    tok += n;
    smp += mode == 1 ? (n > 0 ? 1 : 0) : (mode == 2 ? n : 0);
  }
  const int64_t off = block_sum_int(tok, s_red);
  const int64_t s_off = block_sum_int(smp, s_red);
  const int start = desc[kDescWords * i], n = desc[kDescWords * i + 1];
  const int mode = desc[kDescWords * i + 2];
  const int64_t t_off = desc[kDescWords * i + 3];
  const int t_len = desc[kDescWords * i + 4];
  // block id j of this sequence's table; entries past the uploaded ids read as block 0
  auto table = [&](int j) -> int64_t {
    const int64_t k = t_off + j;
    return (j < t_len && k >= 0 && k < num_block_ids) ? blocks[k] : 0;
  };

  for (int t = tid; t < n; t += kMetaThreads) {
    const int64_t row = off + t;
    if (row >= num_tokens) break;                   // descriptors claim more tokens than sent
    const int64_t pos = (int64_t)start + t;
    const int64_t blk = pos / kBlockSize;
    input_ids[row] = tokens[row];
    positions[row] = pos;
    slot_mapping[row] = blk < t_len ? table((int)blk) * kBlockSize + pos % kBlockSize : -1;
    if (mode == 2 && sample_indices) sample_indices[s_off + t] = row;
  }
  for (int j = tid; j < bt_width; j += kMetaThreads) bt_row[j] = (int32_t)table(j);
  if (tid == 0) {
    qsl[i + 1] = (int32_t)(off + n);
    seq_lens[i] = start + n;
    if (i == 0) qsl[0] = 0;
    if (mode == 1 && n > 0 && sample_indices) sample_indices[s_off] = off + n - 1;
  }
}

}  // namespace ts

using namespace ts;

extern "C" int ts_step_metadata(const int32_t* packed, int32_t num_seqs, int64_t num_tokens,
                                int64_t num_block_ids, int32_t pad_seqs, int32_t bt_width,
                                int64_t bt_stride, int64_t* input_ids, int64_t* positions,
                                int64_t* slot_mapping, int32_t* query_start_loc,
                                int32_t* seq_lens, int32_t* block_tables,
                                int64_t* sample_indices, void* stream) {
  ts::clear_error();
  TS_REQUIRE(num_seqs >= 0 && pad_seqs >= num_seqs && num_tokens >= 0 && num_block_ids >= 0,
             TS_ERR_INVALID_ARG, "step_metadata: num_seqs=%d pad_seqs=%d num_tokens=%lld",
             num_seqs, pad_seqs, (long long)num_tokens);
  if (pad_seqs == 0) return TS_OK;
  TS_REQUIRE(bt_width >= 1 && bt_stride >= bt_width, TS_ERR_INVALID_ARG,
             "step_metadata: bt_width=%d bt_stride=%lld", bt_width, (long long)bt_stride);
  TS_REQUIRE((packed || num_seqs == 0) && input_ids && positions && slot_mapping &&
                 query_start_loc && seq_lens && block_tables,
             TS_ERR_INVALID_ARG, "step_metadata: null pointer argument");
  step_metadata_kernel<<<pad_seqs, kMetaThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      packed, num_seqs, num_tokens, num_block_ids, bt_width, bt_stride, input_ids, positions,
      slot_mapping, query_start_loc, seq_lens, block_tables, sample_indices);
  return check_launch("step_metadata");
}
