// Paged decode attention for gfx950: the v1 / v2 / v3 family of
// ops/triton_decode_attention.py:1-200 with the policy of ops/triton_ops.py:35-57.
//
//  v1  one wavefront per (sequence, query head); VALU dot products and 64-lane shuffles.
//      Reads every KV block once per query head; kept as the simple, any-group-size variant.
//  v2  one workgroup per (sequence, KV head, group of <= 16 query heads): the whole GQA group
//      shares each 16-token K/V block, which is read from HBM exactly once per KV head.
//  v3  v2 split over context partitions of `partition` tokens ("flash-decoding"): partials
//      (m, l, acc) in fp32 go to the workspace and a second kernel merges them.
//
// Inner loop of v2/v3 (one wavefront, one 16-token block; lane l = 16 g + c):
//   S^T[16 tok][16 heads] = K[16 tok][D] . Q^T[D][16 heads]       v_mfma_f32_16x16x32_f16
//   K lane (c, g) loads K[tok c][32kk + 8g .. +7]: 16-byte loads, 64 contiguous bytes per token
//   per instruction; Q^T uses the same dim permutation, so no shuffles are needed.
//   The result leaves lane (c, g) holding tokens 4g..4g+3 of head c: every per-head softmax
//   statistic (running max m, sum l, rescale alpha) lives in lane column c.
//   V is transposed in registers by one v_mfma_f32_16x16x16_f16 against the identity (exact:
//   one non-zero product per output), which turns V[tok][dim] rows into the token-packed A
//   operand of O^T[D][16 heads] += V^T . P^T (v_mfma_f32_16x16x16_f16, P rounded to fp16
//   exactly like ops/triton_decode_attention.py:91).
//   Afterwards lane (c, g) owns dims 32kk + 8g .. +7 of head c: 16-byte stores.
// The waves of a workgroup take interleaved blocks and merge their (m, l, acc) in LDS.
#include <math.h>

#include "common.h"

namespace ts {

constexpr float kLog2e = 1.4426950408889634f;

// ------------------------------------------------------------------------------------------
// v1 (ops/triton_decode_attention.py:23-54)
// ------------------------------------------------------------------------------------------
template <int D>
__global__ void __launch_bounds__(64) decode_v1_kernel(
    const half_t* __restrict__ q, int64_t q_st, int64_t q_sh, half_t* __restrict__ out,
    int64_t o_st, const half_t* __restrict__ kc, const half_t* __restrict__ vc, int64_t NB,
    const int* __restrict__ bt, int64_t bt_st, int max_blocks, const int* __restrict__ seq_lens,
    int H, int KVH, float scale_log2) {
  constexpr int DQ = D / 4;                    // dims per lane: 4 lanes share one token row
  const int s = blockIdx.x, h = blockIdx.y;
  const int G = H / KVH, kvh = h / G;
  const int lane = threadIdx.x, tok = lane >> 2, part = lane & 3;
  int seq_len = seq_lens[s];
  seq_len = seq_len < 0 ? 0 : (seq_len > max_blocks * kBlockSize ? max_blocks * kBlockSize : seq_len);
  float qv[DQ], acc[DQ];
  const half_t* qp = q + (int64_t)s * q_st + (int64_t)h * q_sh + part * DQ;
#pragma unroll
  for (int d = 0; d < DQ; ++d) {
    qv[d] = (float)qp[d];
    acc[d] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int nblk = (seq_len + kBlockSize - 1) / kBlockSize;
  for (int i = 0; i < nblk; ++i) {
    const int phys = clamp_block(bt[(int64_t)s * bt_st + i], NB);
    const int64_t row = (((int64_t)phys * KVH + kvh) * kBlockSize + tok) * D + part * DQ;
    float sc = 0.f;
#pragma unroll
    for (int d = 0; d < DQ; ++d) sc += qv[d] * (float)kc[row + d];
    sc += shfl_xor(sc, 1);
    sc += shfl_xor(sc, 2);
    const bool valid = i * kBlockSize + tok < seq_len;
    sc = valid ? sc * scale_log2 : -INFINITY;
    float bm = sc;
    bm = fmaxf(bm, shfl_xor(bm, 4));
    bm = fmaxf(bm, shfl_xor(bm, 8));
    bm = fmaxf(bm, shfl_xor(bm, 16));
    bm = fmaxf(bm, shfl_xor(bm, 32));
    const float m_new = fmaxf(m, bm);          // finite: token 0 of the block is valid
    const float alpha = fast_exp2(m - m_new);
    const float p = valid ? fast_exp2(sc - m_new) : 0.f;
    float ps = p;                              // sum over the 16 tokens (lanes of equal part)
    ps += shfl_xor(ps, 4);
    ps += shfl_xor(ps, 8);
    ps += shfl_xor(ps, 16);
    ps += shfl_xor(ps, 32);
    l = l * alpha + ps;
#pragma unroll
    for (int d = 0; d < DQ; ++d) acc[d] = acc[d] * alpha + (valid ? p * (float)vc[row + d] : 0.f);
    m = m_new;
  }
#pragma unroll
  for (int d = 0; d < DQ; ++d) {
    float a = acc[d];
    a += shfl_xor(a, 4);
    a += shfl_xor(a, 8);
    a += shfl_xor(a, 16);
    a += shfl_xor(a, 32);
    acc[d] = a;
  }
  const float inv = 1.f / (l == 0.f ? 1.f : l);   // seq_len 0 -> zeros
  if (tok == 0) {
    half_t* op = out + (int64_t)s * o_st + (int64_t)h * D + part * DQ;
#pragma unroll
    for (int d = 0; d < DQ; ++d) op[d] = (half_t)(acc[d] * inv);
  }
}

// ------------------------------------------------------------------------------------------
// v2 / v3 partial kernel (ops/triton_decode_attention.py:60-141)
// ------------------------------------------------------------------------------------------
template <int D>
struct DecodeRegs {
  // D >= 32: KK 16-byte pieces per lane; D == 16: one 8-byte piece.
  static constexpr int KK = D >= 32 ? D / 32 : 1;
  static constexpr int TILES = D / 16;           // 16-dim output tiles of O^T
};

template <int D>
__device__ __forceinline__ void load_kv_block(const half_t* __restrict__ base, int c, int g,
                                              half8_t (&x)[DecodeRegs<D>::KK]) {
  if constexpr (D >= 32) {
#pragma unroll
    for (int kk = 0; kk < DecodeRegs<D>::KK; ++kk) x[kk] = ld<half8_t>(base + c * D + 32 * kk + 8 * g);
  } else {
    const half4_t t = ld<half4_t>(base + c * D + 4 * g);
    x[0] = {t[0], t[1], t[2], t[3], 0, 0, 0, 0};
  }
}

template <int D, int NW>
__global__ void __launch_bounds__(NW * 64) decode_mfma_kernel(
    const half_t* __restrict__ q, int64_t q_st, int64_t q_sh, half_t* __restrict__ out,
    int64_t o_st, const half_t* __restrict__ kc, const half_t* __restrict__ vc, int64_t NB,
    const int* __restrict__ bt, int64_t bt_st, int max_blocks, const int* __restrict__ seq_lens,
    int H, int KVH, int G, int HG, float scale_log2, int part_blocks, int num_splits,
    float* __restrict__ ws_acc, float* __restrict__ ws_m, float* __restrict__ ws_l) {
  constexpr int KK = DecodeRegs<D>::KK;
  constexpr int TILES = DecodeRegs<D>::TILES;
  constexpr int OROW = D + 4;                    // padded LDS row (floats) against bank conflicts
  __shared__ float s_o[NW][16][OROW];
  __shared__ float s_m[NW][16];
  __shared__ float s_l[NW][16];

  const int split = blockIdx.x, s = blockIdx.y;
  const int kvh = blockIdx.z / HG, hg = blockIdx.z % HG;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int c = lane & 15, g = lane >> 4;
  const int hq = hg * 16 + c;                    // query head within the GQA group
  const bool head_ok = hq < G;
  const int nh = (G - hg * 16) < 16 ? (G - hg * 16) : 16;   // real heads in this group

  int seq_len = seq_lens[s];
  seq_len = seq_len < 0 ? 0 : (seq_len > max_blocks * kBlockSize ? max_blocks * kBlockSize : seq_len);
  const int nblk = (seq_len + kBlockSize - 1) / kBlockSize;
  // A seq_len beyond the caller's max_seq_len is truncated to the launched splits, as the fixed
  // split grid of ops/triton_ops.py:50-51 does; it never indexes past the workspace.
  int n_active = (nblk + part_blocks - 1) / part_blocks;
  n_active = n_active < num_splits ? n_active : num_splits;
  if (seq_len == 0) {                            // padding row: zeros (ops/reference.py:99,104-105)
    if (split == 0) {
      for (int e = tid; e < nh * D; e += NW * 64) {
        const int hh = e / D, d = e % D;
        out[(int64_t)s * o_st + (int64_t)(kvh * G + hg * 16 + hh) * D + d] = (half_t)0.f;
      }
    }
    return;
  }
  const int blk_lo = split * part_blocks;
  if (blk_lo >= nblk) return;                    // idle split of a short sequence
  const int blk_hi = (blk_lo + part_blocks) < nblk ? (blk_lo + part_blocks) : nblk;

  // Q^T operand: lane (c, g) holds Q[head c][32kk + 8g .. +7] (zeros for padding heads).
  half8_t qf[KK];
  {
    const half_t* qp = q + (int64_t)s * q_st + (int64_t)(kvh * G + hq) * q_sh;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if constexpr (D >= 32) {
        qf[kk] = head_ok ? ld<half8_t>(qp + 32 * kk + 8 * g) : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
      } else {
        const half4_t t = head_ok ? ld<half4_t>(qp + 4 * g) : half4_t{0, 0, 0, 0};
        qf[kk] = {t[0], t[1], t[2], t[3], 0, 0, 0, 0};
      }
    }
  }
  // Identity B operand for the register transpose: B[4g + r][c] = (4g + r == c).
  const half4_t ident = {(half_t)(4 * g + 0 == c ? 1.f : 0.f), (half_t)(4 * g + 1 == c ? 1.f : 0.f),
                         (half_t)(4 * g + 2 == c ? 1.f : 0.f), (half_t)(4 * g + 3 == c ? 1.f : 0.f)};

  float4_t o[TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t) o[t] = {0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;

  const int* btrow = bt + (int64_t)s * bt_st;
  const int64_t head_off = (int64_t)kvh * kBlockSize * D;
  const int64_t blk_stride = (int64_t)KVH * kBlockSize * D;
  half8_t kf[KK], vf[KK], kn[KK], vn[KK];
  // V rows past seq_len are zeroed so stale cache contents never reach P.V (0 * NaN).
  const half8_t hz = {0, 0, 0, 0, 0, 0, 0, 0};
  int i = blk_lo + w;
  if (i < blk_hi) {
    const int64_t off = clamp_block(btrow[i], NB) * blk_stride + head_off;
    load_kv_block<D>(kc + off, c, g, kf);
    load_kv_block<D>(vc + off, c, g, vf);
    if (i * kBlockSize + c >= seq_len) {
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) vf[kk] = hz;
    }
  }
  for (; i < blk_hi; i += NW) {
    const int inext = i + NW;
    if (inext < blk_hi) {                        // prefetch the next block of this wave
      const int64_t off = clamp_block(btrow[inext], NB) * blk_stride + head_off;
      load_kv_block<D>(kc + off, c, g, kn);
      load_kv_block<D>(vc + off, c, g, vn);
      if (inext * kBlockSize + c >= seq_len) {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) vn[kk] = hz;
      }
    }
    // S^T = K . Q^T
    float4_t st4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if constexpr (D >= 32) st4 = mfma16x16x32(kf[kk], qf[kk], st4);
      else st4 = mfma16x16x16(lo4(kf[kk]), lo4(qf[kk]), st4);
    }
    const int tok0 = i * kBlockSize + 4 * g;
    float sc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[r] = (tok0 + r < seq_len) ? st4[r] * scale_log2 : -INFINITY;
    const float bmax = rows_max(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
    const float m_new = fmaxf(m, bmax);          // finite: token 0 of every block is valid
    const float alpha = fast_exp2(m - m_new);
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = fast_exp2(sc[r] - m_new);
    l = l * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    m = m_new;
    const half4_t pb = {(half_t)p[0], (half_t)p[1], (half_t)p[2], (half_t)p[3]};
#pragma unroll
    for (int t = 0; t < TILES; ++t) o[t] *= alpha;
    // O^T += V^T . P^T, V transposed through the identity product.
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const float4_t zero = {0.f, 0.f, 0.f, 0.f};
      const half4_t va = to_half4(mfma16x16x16(lo4(vf[kk]), ident, zero));
      o[2 * kk] = mfma16x16x16(va, pb, o[2 * kk]);
      if constexpr (D >= 32) {
        const half4_t vb = to_half4(mfma16x16x16(hi4(vf[kk]), ident, zero));
        o[2 * kk + 1] = mfma16x16x16(vb, pb, o[2 * kk + 1]);
      }
    }
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      kf[kk] = kn[kk];
      vf[kk] = vn[kk];
    }
  }
  l = rows_sum(l);

  // Merge the NW waves of this workgroup.
  if (g == 0) {
    s_m[w][c] = m;
    s_l[w][c] = l;
  }
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    if constexpr (D >= 32) {
      float* dst = &s_o[w][c][32 * kk + 8 * g];
      st<float4_t>(dst, o[2 * kk]);
      st<float4_t>(dst + 4, o[2 * kk + 1]);
    } else {
      st<float4_t>(&s_o[w][c][4 * g], o[0]);
    }
  }
  __syncthreads();
  const bool final_out = n_active == 1;
  for (int e = tid; e < nh * D; e += NW * 64) {
    const int hh = e / D, d = e % D;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, s_m[ww][hh]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float wt = fast_exp2(s_m[ww][hh] - M);    // idle wave: m = -inf -> 0
      L += wt * s_l[ww][hh];
      O += wt * s_o[ww][hh][d];
    }
    const int head = kvh * G + hg * 16 + hh;
    if (final_out) {
      out[(int64_t)s * o_st + (int64_t)head * D + d] = (half_t)(O / L);
    } else {
      const int64_t pidx = ((int64_t)s * H + head) * num_splits + split;
      ws_acc[pidx * D + d] = O;
      if (d == 0) {
        ws_m[pidx] = M;
        ws_l[pidx] = L;
      }
    }
  }
}

// Merge of the split partials (ops/triton_decode_attention.py:144-163): M = max m_j,
// w_j = 2^(m_j - M), out = sum w_j acc_j / sum w_j l_j. Sequences with a single active split
// were finished by the partial kernel.
template <int D>
__global__ void __launch_bounds__(D < 64 ? 64 : D) decode_reduce_kernel(
    const float* __restrict__ ws_acc, const float* __restrict__ ws_m,
    const float* __restrict__ ws_l, half_t* __restrict__ out, int64_t o_st,
    const int* __restrict__ seq_lens, int max_blocks, int H, int part_blocks, int num_splits) {
  const int s = blockIdx.x, h = blockIdx.y;
  int seq_len = seq_lens[s];
  seq_len = seq_len < 0 ? 0 : (seq_len > max_blocks * kBlockSize ? max_blocks * kBlockSize : seq_len);
  const int nblk = (seq_len + kBlockSize - 1) / kBlockSize;
  int n_active = (nblk + part_blocks - 1) / part_blocks;
  n_active = n_active < num_splits ? n_active : num_splits;
  if (n_active <= 1) return;
  const int64_t base = ((int64_t)s * H + h) * num_splits;
  float M = -INFINITY;
  for (int j = 0; j < n_active; ++j) M = fmaxf(M, ws_m[base + j]);
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float L = 0.f, O = 0.f;
    for (int j = 0; j < n_active; ++j) {
      const float wt = fast_exp2(ws_m[base + j] - M);
      L += wt * ws_l[base + j];
      O += wt * ws_acc[(base + j) * D + d];
    }
    out[(int64_t)s * o_st + (int64_t)h * D + d] = (half_t)(O / L);
  }
}

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------
constexpr int kDecodeWaves = 4;
constexpr int kDefaultPartition = 256;     // tokens per v3 split (multiple of 16 * kDecodeWaves)

struct SplitPlan {
  int version;        // 1, 2 or 3 after resolving AUTO
  int part_blocks;    // blocks per split
  int num_splits;
};

static SplitPlan plan_decode(int version, int S, int H, int KVH, int max_seq_len, int partition,
                             int cu_count) {
  SplitPlan p{version, 1 << 30, 1};
  const int G = H / KVH;
  const int HG = (G + 15) / 16;
  if (version == TS_DECODE_AUTO) {
    // ops/triton_ops.py:44-45: split when the (sequence, KV head) grid cannot fill the device
    // twice over and the context is long; the CU count replaces the SM count.
    const bool use_split = (int64_t)S * KVH * HG < 2LL * cu_count && max_seq_len > 1024;
    p.version = use_split ? TS_DECODE_V3 : TS_DECODE_V2;
  }
  if (p.version == TS_DECODE_V3) {
    int part = partition > 0 ? partition : kDefaultPartition;
    part = ((part + kBlockSize - 1) / kBlockSize) * kBlockSize;
    p.part_blocks = part / kBlockSize;
    const int max_blk = (max_seq_len + kBlockSize - 1) / kBlockSize;
    p.num_splits = (max_blk + p.part_blocks - 1) / p.part_blocks;   // ops/triton_ops.py:50-51
    if (p.num_splits < 1) p.num_splits = 1;
  }
  return p;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static size_t workspace_for(const SplitPlan& p, int S, int H, int D) {
  if (p.version != TS_DECODE_V3 || p.num_splits <= 1) return 0;
  const size_t n = (size_t)S * H * p.num_splits;
  return align256(n * D * sizeof(float)) + 2 * align256(n * sizeof(float));
}

template <int D>
static void launch_decode(const SplitPlan& p, hipStream_t st, const half_t* q, int64_t q_st,
                          int64_t q_sh, half_t* out, int64_t o_st, const half_t* kc,
                          const half_t* vc, int64_t NB, const int* bt, int64_t bt_st,
                          int max_blocks, const int* sl, int S, int H, int KVH, float scale_log2,
                          void* ws) {
  const int G = H / KVH;
  if (p.version == TS_DECODE_V1) {
    decode_v1_kernel<D><<<dim3(S, H), 64, 0, st>>>(q, q_st, q_sh, out, o_st, kc, vc, NB, bt,
                                                   bt_st, max_blocks, sl, H, KVH, scale_log2);
    return;
  }
  const int HG = (G + 15) / 16;
  float *ws_acc = nullptr, *ws_m = nullptr, *ws_l = nullptr;
  if (p.num_splits > 1) {
    const size_t n = (size_t)S * H * p.num_splits;
    char* b = static_cast<char*>(ws);
    ws_acc = reinterpret_cast<float*>(b);
    ws_m = reinterpret_cast<float*>(b + align256(n * D * sizeof(float)));
    ws_l = reinterpret_cast<float*>(b + align256(n * D * sizeof(float)) + align256(n * sizeof(float)));
  }
  decode_mfma_kernel<D, kDecodeWaves><<<dim3(p.num_splits, S, KVH * HG), kDecodeWaves * 64, 0, st>>>(
      q, q_st, q_sh, out, o_st, kc, vc, NB, bt, bt_st, max_blocks, sl, H, KVH, G, HG, scale_log2,
      p.part_blocks, p.num_splits, ws_acc, ws_m, ws_l);
  if (p.num_splits > 1) {
    decode_reduce_kernel<D><<<dim3(S, H), D < 64 ? 64 : D, 0, st>>>(
        ws_acc, ws_m, ws_l, out, o_st, sl, max_blocks, H, p.part_blocks, p.num_splits);
  }
}

static bool supported_head_dim(int D) {
  return D == 16 || D == 32 || D == 64 || D == 128 || D == 256;
}

}  // namespace ts

using namespace ts;

extern "C" size_t ts_decode_workspace_bytes(int32_t version, int32_t num_seqs, int32_t num_heads,
                                            int32_t num_kv_heads, int32_t head_dim,
                                            int32_t max_seq_len, int32_t partition,
                                            int32_t cu_count) {
  if (num_seqs <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return 0;
  const SplitPlan p = plan_decode(version, num_seqs, num_heads, num_kv_heads, max_seq_len,
                                  partition, cu_count > 0 ? cu_count : 256);
  return workspace_for(p, num_seqs, num_heads, head_dim);
}

extern "C" int ts_decode_attention(int32_t version, const void* q, int64_t q_stride_t,
                                   int64_t q_stride_h, void* out, int64_t out_stride_t,
                                   const void* k_cache, const void* v_cache, int64_t num_blocks,
                                   const int32_t* block_tables, int64_t bt_stride,
                                   int32_t max_blocks_per_seq, const int32_t* seq_lens,
                                   int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                   int32_t head_dim, float scale, int32_t max_seq_len,
                                   int32_t partition, void* workspace, size_t workspace_bytes,
                                   void* stream) {
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
  int st = device_cu_count(&cus);
  if (st != TS_OK) return st;
  const SplitPlan p = plan_decode(version, num_seqs, num_heads, num_kv_heads, max_seq_len,
                                  partition, cus);
  const size_t need = workspace_for(p, num_seqs, num_heads, head_dim);
  TS_REQUIRE(need == 0 || (workspace && workspace_bytes >= need && aligned(workspace, 256)),
             TS_ERR_WORKSPACE, "decode_attention: workspace of %zu bytes (256-aligned) needed, got %zu",
             need, workspace_bytes);
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const float sl2 = scale * kLog2e;
  const half_t* qp = static_cast<const half_t*>(q);
  half_t* op = static_cast<half_t*>(out);
  const half_t* kp = static_cast<const half_t*>(k_cache);
  const half_t* vp = static_cast<const half_t*>(v_cache);
#define TS_DECODE_CASE(DD)                                                                      \
  case DD:                                                                                      \
    launch_decode<DD>(p, s, qp, q_stride_t, q_stride_h, op, out_stride_t, kp, vp, num_blocks,  \
                      block_tables, bt_stride, max_blocks_per_seq, seq_lens, num_seqs, num_heads, \
                      num_kv_heads, sl2, workspace);                                            \
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
