// Measurement probes (no counterpart in the reference). They give the roofline figures that
// bench.py reports beside the spec peaks a measured ceiling on this device:
//  * gather: reads a list of equal-size chunks at arbitrary byte offsets with no arithmetic
//    and no dependent metadata loads -- with the chunk list of a decode step (every cached
//    (block, KV head) K and V chunk once, in block-table order), the fastest that step's bytes
//    can be gathered;
//  * mfma: back-to-back independent v_mfma_f32_32x32x16_f16 chains, the matrix-core rate.
#include "common.h"

namespace ts {

constexpr int kProbeThreads = 256;
constexpr int kChunksPerGroup = 8;        // two chunks per wavefront

// Workgroup b reads chunks 8b .. 8b+7 (wavefront w: 8b + 2w, 8b + 2w + 1; past the list the
// last chunk again); each chunk of PIECES KiB is read with 16-byte lane loads, all issued before
// any is used. The XOR of the loaded words goes to sink[b] so no load is dead.
template <int PIECES>
__global__ void __launch_bounds__(kProbeThreads) gather_probe_kernel(
    const uint8_t* __restrict__ base, const int64_t* __restrict__ offsets, int n_chunks,
    uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int4_t v[2][PIECES];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    int chunk = blockIdx.x * kChunksPerGroup + 2 * w + c;
    chunk = chunk < n_chunks ? chunk : n_chunks - 1;
    const uint8_t* p = base + offsets[chunk] + lane * 16;
#pragma unroll
    for (int i = 0; i < PIECES; ++i) v[c][i] = ld<int4_t>(p + i * 1024);
  }
  int4_t acc = {0, 0, 0, 0};
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int i = 0; i < PIECES; ++i) acc ^= v[c][i];
  const int x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (threadIdx.x == 0) sink[blockIdx.x] = (uint32_t)x;
  if (x == 0x7fffffff) sink[blockIdx.x] = 1;       // keeps every lane's loads live
}

// Each wavefront runs `iters` rounds of four independent 32x32x16 fp16 MFMA chains (2 * 32 * 32
// * 16 flops each) on operands built from its lane id; the accumulators' sum goes to sink.
__global__ void __launch_bounds__(kProbeThreads) mfma_probe_kernel(int iters,
                                                                  float* __restrict__ sink) {
  typedef float float16v __attribute__((ext_vector_type(16)));
  const int lane = threadIdx.x & 63;
  half8_t a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (half_t)(0.001f * (lane + i));
    b[i] = (half_t)(0.002f * (lane - i));
  }
  float16v c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int it = 0; it < iters; ++it) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, a, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, a, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, b, c3, 0, 0, 0);
  }
  float s = 0.f;
  for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i];
  if (lane == 0) sink[blockIdx.x * (kProbeThreads / 64) + (threadIdx.x >> 6)] = s;
}

}  // namespace ts

using namespace ts;

extern "C" int ts_probe_gather(const void* base, const int64_t* chunk_offsets, int32_t n_chunks,
                               int32_t chunk_bytes, uint32_t* sink, void* stream) {
  ts::clear_error();
  TS_REQUIRE(base && chunk_offsets && sink && n_chunks >= 0, TS_ERR_INVALID_ARG,
             "probe_gather: null pointer or negative count");
  TS_REQUIRE((chunk_bytes == 2048 || chunk_bytes == 4096) && aligned(base, 16),
             TS_ERR_INVALID_ARG, "probe_gather: chunk_bytes %d must be 2048 or 4096 (one block "
             "of one KV head at head_dim 64 or 128), base 16-byte aligned", chunk_bytes);
  if (n_chunks == 0) return TS_OK;
  const int groups = (n_chunks + kChunksPerGroup - 1) / kChunksPerGroup;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const uint8_t* b = static_cast<const uint8_t*>(base);
  if (chunk_bytes == 4096)
    gather_probe_kernel<4><<<groups, kProbeThreads, 0, s>>>(b, chunk_offsets, n_chunks, sink);
  else
    gather_probe_kernel<2><<<groups, kProbeThreads, 0, s>>>(b, chunk_offsets, n_chunks, sink);
  return check_launch("probe_gather");
}

extern "C" int ts_probe_mfma(int32_t workgroups, int32_t iters, float* sink, void* stream) {
  ts::clear_error();
  TS_REQUIRE(sink && workgroups > 0 && iters > 0, TS_ERR_INVALID_ARG,
             "probe_mfma: null sink or non-positive size");
  mfma_probe_kernel<<<workgroups, kProbeThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      iters, sink);
  return check_launch("probe_mfma");
}
