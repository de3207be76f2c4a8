// Shared device and host helpers of the gfx950 hot-path kernels.
//
// MFMA operand layouts used throughout (CDNA3/CDNA4 matrix cores, 64-lane wavefront).
// Lane l is split into c = l % 16 and g = l / 16.
//   v_mfma_f32_16x16x16_f16  A[16][16] x B[16][16]: lane holds A[c][4g .. 4g+3] and
//                            B[4g .. 4g+3][c]; result lane holds D[4g + r][c], r = 0..3.
//   v_mfma_f32_16x16x32_f16  A[16][32] x B[32][16]: lane holds A[c][8g .. 8g+7] and
//                            B[8g .. 8g+7][c]; result as above.
// The contraction index k may be permuted freely as long as A and B use the same
// permutation; the kernels use that freedom so that every operand is a contiguous
// 8- or 16-byte load of the natural memory layout.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/turingserve_hip.h"

namespace ts {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef int int4_t __attribute__((ext_vector_type(4)));
typedef int int2_t __attribute__((ext_vector_type(2)));

constexpr int kBlockSize = 16;    // tokens per KV block (config.py:74-75)
constexpr int kWave = 64;         // CDNA wavefront width
// s_waitcnt operand waiting for every vector memory operation of the wavefront (loads and
// stores: vmcnt 0; expcnt and lgkmcnt at their maxima, i.e. not waited for).
constexpr int kWaitVmcntZero = (7 << 4) | (15 << 8);

__device__ __forceinline__ float4_t mfma16x16x16(half4_t a, half4_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ half4_t lo4(half8_t v) { return {v[0], v[1], v[2], v[3]}; }
__device__ __forceinline__ half4_t hi4(half8_t v) { return {v[4], v[5], v[6], v[7]}; }

// Device-coherent (sc1) buffer accesses: data one workgroup stores and another, on any XCD,
// loads in the same launch after an agent-scope atomic has ordered them (the stores are waited
// for, vmcnt 0, before the atomic). The resource is built from a wave-uniform base, the lane's
// byte offset (below 2 GiB) travels in a VGPR; the raw buffer builtins move 32-bit words, so
// floats travel as their bits.
constexpr int kCoherentPolicy = 16;            // buffer cache policy bits: sc1
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const void* uniform_base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(uniform_base), (short)0, 0x7fffffff,
                                           0x00020000);
}
__device__ __forceinline__ void coherent_store(__amdgpu_buffer_rsrc_t r, int off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, off, 0, kCoherentPolicy);
}
__device__ __forceinline__ float coherent_load(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kCoherentPolicy));
}
__device__ __forceinline__ float4_t coherent_load4(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCoherentPolicy));
}

__device__ __forceinline__ half4_t to_half4(float4_t v) {
  return {(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
}

// Base-2 exponential on the hardware transcendental unit (v_exp_f32).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float shfl_xor(float v, int mask) { return __shfl_xor(v, mask, kWave); }

// NaN-propagating maximum (llvm.maximum, v_maximum3_f32 on gfx950). Unlike fmaxf it needs no
// quieting of its inputs in IEEE mode, so reductions over MFMA results cost one op per value.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Max / sum over the four 16-lane rows of a wavefront (lanes c, c+16, c+32, c+48), on the VALU:
// v_permlane16_swap(x, x) returns rows (0, 0, 2, 2) and (1, 1, 3, 3) of x, v_permlane32_swap(x, x)
// returns (lo, lo) and (hi, hi) halves, so combining each pair is an all-reduce over 2 then 4
// rows with no LDS round trip (gfx950 instructions).
__device__ __forceinline__ float rows_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = vmax(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return vmax(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ int clamp_block(int blk, int64_t num_blocks) {
  return (blk >= 0 && (int64_t)blk < num_blocks) ? blk : 0;
}

// One entry of a table the kernel only reads (block tables), read through the constant address
// space: at a wave-uniform address this is a scalar load even when the compiler cannot prove
// that no store of the kernel aliases the table (pointers that come in a struct argument carry
// no restrict), so the entry does not wait behind the wavefront's vector loads.
__device__ __forceinline__ int table_entry(const int* p) {
  return *reinterpret_cast<const __attribute__((address_space(4))) int*>(
      reinterpret_cast<uintptr_t>(p));
}

// 16-byte vector load / store through the vector memory path.
template <typename T>
__device__ __forceinline__ T ld(const void* p) { return *reinterpret_cast<const T*>(p); }
template <typename T>
__device__ __forceinline__ void st(void* p, T v) { *reinterpret_cast<T*>(p) = v; }

}  // namespace ts

// ---------------------------------------------------------------------------------------------
// Host side: error reporting shared by every entry point (defined in capi.hip).
// ---------------------------------------------------------------------------------------------
namespace ts {
constexpr int kMaxDevices = 64;                 // per-device host caches (CU counts, scratch)
int set_error(int status, const char* fmt, ...);
void clear_error();
int check_launch(const char* what);
int stream_device(void* stream, int* device);
int device_cu_count(void* stream, int* out);
inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
}  // namespace ts

#define TS_REQUIRE(cond, status, ...)                 \
  do {                                                \
    if (!(cond)) return ::ts::set_error((status), __VA_ARGS__); \
  } while (0)
