// kv_write: scatter the new K/V rows of a step into their paged-cache slots.
//
// Reference behaviour: ops/triton_kv_write.py:10-35 (twin ops/reference.py:50-57):
//   k_cache[slot // 16, h, slot % 16, :] = k[t, h, :] for slot = slot_mapping[t] >= 0.
// The copy is bit-exact. Each thread moves one VEC-element piece of one (token, head) row for
// both K and V, so a wavefront writes whole 16-token-block rows with 16-byte stores; the grid
// is flat (tokens x heads x pieces) so even a 64-token decode step fills many CUs.
#include "common.h"

namespace ts {

template <int VEC>
struct VecT;
template <>
struct VecT<8> { typedef int4_t type; };     // 16 bytes
template <>
struct VecT<2> { typedef int type; };        // 4 bytes
template <>
struct VecT<1> { typedef uint16_t type; };   // 2 bytes

template <int VEC>
__global__ void __launch_bounds__(256) kv_write_kernel(
    const half_t* __restrict__ k, const half_t* __restrict__ v, int64_t k_st, int64_t k_sh,
    int64_t v_st, int64_t v_sh, half_t* __restrict__ kc, half_t* __restrict__ vc,
    int64_t num_slots, const int64_t* __restrict__ slots, int64_t total, int KVH, int D) {
  typedef typename VecT<VEC>::type V;
  const int pieces = D / VEC;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int p = (int)(i % pieces);
    const int64_t th = i / pieces;
    const int h = (int)(th % KVH);
    const int64_t t = th / KVH;
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= num_slots) continue;          // -1 = padding row (and out-of-range)
    const int64_t blk = slot >> 4, off = slot & 15;
    const int64_t dst = ((blk * KVH + h) * kBlockSize + off) * D + (int64_t)p * VEC;
    st<V>(kc + dst, ld<V>(k + t * k_st + h * k_sh + p * VEC));
    st<V>(vc + dst, ld<V>(v + t * v_st + h * v_sh + p * VEC));
  }
}

}  // namespace ts

using namespace ts;

extern "C" int ts_kv_write(const void* k, const void* v, int64_t k_stride_t, int64_t k_stride_h,
                           int64_t v_stride_t, int64_t v_stride_h, void* k_cache, void* v_cache,
                           int64_t num_blocks, const int64_t* slot_mapping, int64_t num_tokens,
                           int32_t num_kv_heads, int32_t head_dim, void* stream) {
  ts::clear_error();
  TS_REQUIRE(num_tokens >= 0, TS_ERR_INVALID_ARG, "kv_write: num_tokens %lld < 0",
             (long long)num_tokens);
  if (num_tokens == 0) return TS_OK;     // ops/triton_kv_write.py:32-33
  TS_REQUIRE(k && v && k_cache && v_cache && slot_mapping, TS_ERR_INVALID_ARG,
             "kv_write: null pointer argument");
  TS_REQUIRE(num_kv_heads > 0 && head_dim > 0 && num_blocks > 0, TS_ERR_INVALID_ARG,
             "kv_write: num_kv_heads=%d head_dim=%d num_blocks=%lld must be positive",
             num_kv_heads, head_dim, (long long)num_blocks);
  TS_REQUIRE(k_stride_t >= 0 && k_stride_h >= 0 && v_stride_t >= 0 && v_stride_h >= 0,
             TS_ERR_INVALID_ARG, "kv_write: negative stride");
  const int64_t total_rows = num_tokens * num_kv_heads;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool v16 = head_dim % 8 == 0 && k_stride_t % 8 == 0 && k_stride_h % 8 == 0 &&
                   v_stride_t % 8 == 0 && v_stride_h % 8 == 0 && aligned(k, 16) &&
                   aligned(v, 16) && aligned(k_cache, 16) && aligned(v_cache, 16);
  const bool v4 = head_dim % 2 == 0 && k_stride_t % 2 == 0 && k_stride_h % 2 == 0 &&
                  v_stride_t % 2 == 0 && v_stride_h % 2 == 0 && aligned(k, 4) &&
                  aligned(v, 4) && aligned(k_cache, 4) && aligned(v_cache, 4);
  const int vec = v16 ? 8 : (v4 ? 2 : 1);
  const int64_t total = total_rows * (head_dim / vec);
  const int threads = 256;
  const int64_t want = (total + threads - 1) / threads;
  const int grid = (int)(want < 65536 ? want : 65536);
  const half_t* kp = static_cast<const half_t*>(k);
  const half_t* vp = static_cast<const half_t*>(v);
  half_t* kcp = static_cast<half_t*>(k_cache);
  half_t* vcp = static_cast<half_t*>(v_cache);
  const int64_t num_slots = num_blocks * kBlockSize;
  if (vec == 8)
    kv_write_kernel<8><<<grid, threads, 0, s>>>(kp, vp, k_stride_t, k_stride_h, v_stride_t,
                                                v_stride_h, kcp, vcp, num_slots, slot_mapping,
                                                total, num_kv_heads, head_dim);
  else if (vec == 2)
    kv_write_kernel<2><<<grid, threads, 0, s>>>(kp, vp, k_stride_t, k_stride_h, v_stride_t,
                                                v_stride_h, kcp, vcp, num_slots, slot_mapping,
                                                total, num_kv_heads, head_dim);
  else
    kv_write_kernel<1><<<grid, threads, 0, s>>>(kp, vp, k_stride_t, k_stride_h, v_stride_t,
                                                v_stride_h, kcp, vcp, num_slots, slot_mapping,
                                                total, num_kv_heads, head_dim);
  return check_launch("kv_write");
}
