// Measurement probes (no counterpart in the reference). They give the roofline figures that
// bench.py reports beside the spec peaks a measured ceiling on this device:
//  * gather: reads a list of equal-size chunks at arbitrary byte offsets with no arithmetic
//    and no dependent metadata loads -- with the chunk list of a decode step (every cached
//    (block, KV head) K and V chunk once, in block-table order), the fastest that step's bytes
//    can be gathered;
//  * k-operand gather: the same, with each K chunk read in the decode kernel's K operand layout
//    (64 bytes of each of 16 token rows per load instruction) instead of whole KiBs;
//  * persistent gather: the same chunk list read by a few resident workgroups per CU, each
//    wavefront streaming its own contiguous range with 4 or 8 loads in flight;
//  * mfma: back-to-back independent v_mfma_f32_32x32x16_f16 chains, the matrix-core rate.
#include "common.h"

namespace ts {

constexpr int kProbeThreads = 256;
constexpr int kChunksPerGroup = 8;        // two chunks per wavefront

// Workgroup b reads chunks 8b .. 8b+7 (wavefront w: 8b + 2w, 8b + 2w + 1; past the list the
// last chunk again); each chunk of PIECES KiB is read with 16-byte lane loads, all issued before
// any is used. The XOR of the loaded words goes to sink[b] so no load is dead.
// KOP = false: every load instruction reads one contiguous KiB. KOP = true: a wavefront's first
// chunk (the K chunk in a decode step's list, whose chunks alternate K and V of one block) is
// read as the decode kernel reads its K operand -- load i of lane (c, g) (c = lane % 16,
// g = lane / 16) takes bytes 64 i + 16 g of the chunk's token row c, so one instruction reads
// 64 bytes of each of 16 rows -- and the second chunk (V) as whole KiBs, as the decode kernel
// reads V rows.
template <int PIECES, bool KOP>
__global__ void __launch_bounds__(kProbeThreads) gather_probe_kernel(
    const uint8_t* __restrict__ base, const int64_t* __restrict__ offsets, int n_chunks,
    uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  constexpr int kRowBytes = PIECES * 1024 / 16;   // one token row of the chunk
  int4_t v[2][PIECES];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    int chunk = blockIdx.x * kChunksPerGroup + 2 * w + c;
    chunk = chunk < n_chunks ? chunk : n_chunks - 1;
    const uint8_t* p = base + offsets[chunk] +
                       (KOP && c == 0 ? (lane & 15) * kRowBytes + (lane >> 4) * 16 : lane * 16);
#pragma unroll
    for (int i = 0; i < PIECES; ++i) v[c][i] = ld<int4_t>(p + i * (KOP && c == 0 ? 64 : 1024));
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

// Persistent gather: a grid of at most a few workgroups per CU in which wavefront w reads the
// w-th of the grid's equal ranges of the chunk list's 1 KiB pieces (PPC pieces per chunk) in
// order, DEPTH loads in flight at all times, each load one whole 1 KiB piece (16 bytes per lane).
// LDS = false loads into registers; LDS = true issues the loads as LDS DMA
// (global_load_lds_dwordx4) into a per-wavefront ring of DEPTH 1 KiB slots. A wavefront's range
// touches at most 64 chunks (the host checks), whose offsets it holds one per lane.
template <int PPC, int DEPTH, bool LDS>
__global__ void __launch_bounds__(kProbeThreads) gather_persistent_kernel(
    const uint8_t* __restrict__ base, const int64_t* __restrict__ offsets, int n_chunks,
    uint32_t* __restrict__ sink) {
  constexpr int kWaves = kProbeThreads / 64;
  __shared__ int4_t ring[LDS ? kWaves : 1][LDS ? DEPTH : 1][64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t waves = (int64_t)gridDim.x * kWaves, wid = (int64_t)blockIdx.x * kWaves + w;
  const int64_t pieces = (int64_t)PPC * n_chunks;
  const int p0 = (int)(pieces * wid / waves), p1 = (int)(pieces * (wid + 1) / waves);
  if (p0 >= p1) return;
  const int c0 = p0 / PPC;
  const int64_t mine = offsets[min(c0 + lane, n_chunks - 1)];
  const int lo = (int)mine, hi = (int)(mine >> 32);
  auto piece = [&](int p) {                        // address of this lane's 16 bytes of piece p
    p = p < p1 ? p : p1 - 1;                       // past the range: the last piece again
    const int c = p / PPC - c0;
    const int64_t off = (int64_t)(uint32_t)__builtin_amdgcn_readlane(lo, c) |
                        ((int64_t)__builtin_amdgcn_readlane(hi, c) << 32);
    return base + off + (p % PPC) * 1024 + lane * 16;
  };
  uint32_t acc = 0;
  if constexpr (LDS) {
#pragma unroll
    for (int i = 0; i < DEPTH; ++i)
      __builtin_amdgcn_global_load_lds((const void*)piece(p0 + i),
                                       (__attribute__((address_space(3))) void*)&ring[w][i][0], 16, 0, 0);
    for (int p = p0; p < p1; p += DEPTH) {
#pragma unroll
      for (int i = 0; i < DEPTH; ++i) {
        // slot i has landed once at most DEPTH - 1 younger DMAs are outstanding
        __builtin_amdgcn_s_waitcnt((DEPTH - 1) | (7 << 4) | (15 << 8));
        acc ^= (uint32_t)ring[w][i][lane][0];
        __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));   // LDS read done
        __builtin_amdgcn_global_load_lds((const void*)piece(p + DEPTH + i),
                                         (__attribute__((address_space(3))) void*)&ring[w][i][0],
                                         16, 0, 0);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);                 // no DMA outstanding at exit
  } else {
    int4_t r[DEPTH];
#pragma unroll
    for (int i = 0; i < DEPTH; ++i) r[i] = ld<int4_t>(piece(p0 + i));
    for (int p = p0; p < p1; p += DEPTH) {
#pragma unroll
      for (int i = 0; i < DEPTH; ++i) {
        acc ^= (uint32_t)(r[i][0] ^ r[i][1] ^ r[i][2] ^ r[i][3]);
        r[i] = ld<int4_t>(piece(p + DEPTH + i));
      }
    }
#pragma unroll
    for (int i = 0; i < DEPTH; ++i) acc ^= (uint32_t)r[i][0];
  }
  if (acc == 0x7fffffffu) sink[wid] = 1;           // keeps the loads live
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
    gather_probe_kernel<4, false><<<groups, kProbeThreads, 0, s>>>(b, chunk_offsets, n_chunks, sink);
  else
    gather_probe_kernel<2, false><<<groups, kProbeThreads, 0, s>>>(b, chunk_offsets, n_chunks, sink);
  return check_launch("probe_gather");
}

extern "C" int ts_probe_gather_k_operand(const void* base, const int64_t* chunk_offsets,
                                         int32_t n_chunks, int32_t chunk_bytes, uint32_t* sink,
                                         void* stream) {
  ts::clear_error();
  TS_REQUIRE(base && chunk_offsets && sink && n_chunks >= 0, TS_ERR_INVALID_ARG,
             "probe_gather_k_operand: null pointer or negative count");
  TS_REQUIRE((chunk_bytes == 2048 || chunk_bytes == 4096) && aligned(base, 16),
             TS_ERR_INVALID_ARG, "probe_gather_k_operand: chunk_bytes %d must be 2048 or 4096, "
             "base 16-byte aligned", chunk_bytes);
  if (n_chunks == 0) return TS_OK;
  const int groups = (n_chunks + kChunksPerGroup - 1) / kChunksPerGroup;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const uint8_t* b = static_cast<const uint8_t*>(base);
  if (chunk_bytes == 4096)
    gather_probe_kernel<4, true><<<groups, kProbeThreads, 0, s>>>(b, chunk_offsets, n_chunks, sink);
  else
    gather_probe_kernel<2, true><<<groups, kProbeThreads, 0, s>>>(b, chunk_offsets, n_chunks, sink);
  return check_launch("probe_gather_k_operand");
}

extern "C" int ts_probe_gather_persistent(const void* base, const int64_t* chunk_offsets,
                                          int32_t n_chunks, int32_t chunk_bytes,
                                          int32_t workgroups, int32_t depth, int32_t use_lds,
                                          uint32_t* sink, void* stream) {
  ts::clear_error();
  TS_REQUIRE(base && chunk_offsets && sink && n_chunks >= 0 && workgroups > 0, TS_ERR_INVALID_ARG,
             "probe_gather_persistent: null pointer, negative count or no workgroups");
  TS_REQUIRE((chunk_bytes == 2048 || chunk_bytes == 4096) && aligned(base, 16) &&
                 (depth == 4 || depth == 8),
             TS_ERR_INVALID_ARG,
             "probe_gather_persistent: chunk_bytes %d (2048 or 4096), depth %d (4 or 8), base "
             "16-byte aligned", chunk_bytes, depth);
  if (n_chunks == 0) return TS_OK;
  const int ppc = chunk_bytes / 1024;
  const int64_t waves = (int64_t)workgroups * (kProbeThreads / 64);
  const int64_t per_wave = ((int64_t)ppc * n_chunks + waves - 1) / waves;
  TS_REQUIRE(per_wave / ppc + 2 <= 64, TS_ERR_INVALID_ARG,
             "probe_gather_persistent: %lld pieces per wavefront span more than 64 chunks; use "
             "more workgroups", (long long)per_wave);
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const uint8_t* b = static_cast<const uint8_t*>(base);
#define TS_PG(PPC, DEPTH, LDS)                                                                    \
  gather_persistent_kernel<PPC, DEPTH, LDS><<<workgroups, kProbeThreads, 0, s>>>(b, chunk_offsets, \
                                                                               n_chunks, sink)
#define TS_PG_D(PPC, LDS) \
  if (depth == 4) TS_PG(PPC, 4, LDS); else TS_PG(PPC, 8, LDS);
#define TS_PG_L(PPC) \
  if (use_lds) { TS_PG_D(PPC, true) } else { TS_PG_D(PPC, false) }
  if (ppc == 4) {
    TS_PG_L(4)
  } else {
    TS_PG_L(2)
  }
#undef TS_PG_L
#undef TS_PG_D
#undef TS_PG
  return check_launch("probe_gather_persistent");
}

extern "C" int ts_probe_mfma(int32_t workgroups, int32_t iters, float* sink, void* stream) {
  ts::clear_error();
  TS_REQUIRE(sink && workgroups > 0 && iters > 0, TS_ERR_INVALID_ARG,
             "probe_mfma: null sink or non-positive size");
  mfma_probe_kernel<<<workgroups, kProbeThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      iters, sink);
  return check_launch("probe_mfma");
}
