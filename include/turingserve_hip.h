/*
 * turingserve_hip.h -- C ABI of the MI355X (gfx950) per-step hot path of TuringServe.
 *
 * One shared library, libturingserve_hip.so, exports these entry points. They replace the
 * Triton kernels behind the reference's op namespace (turingserve/ops/__init__.py:22-35):
 *
 *   ts_kv_write            <- ops/triton_kv_write.py:28-35   (twin ops/reference.py:50-57)
 *   ts_decode_attention    <- ops/triton_ops.py:35-57 (_decode) and
 *                             ops/triton_decode_attention.py:169-200 (v1 / v2 / v3 launchers)
 *   ts_decode_attention_kv_write  (kv_write + decode attention of a pure-decode step, fused)
 *   ts_decode_rope_kv_write_attention  (rope + kv_write + decode attention, fused)
 *   ts_prefill_attention   <- ops/triton_prefill_attention.py:66-79
 *   ts_prefill_attention_ws   (the same with split key ranges, + ts_prefill_workspace_bytes)
 *   ts_paged_attention     <- ops/triton_ops.py:60-71        (twin ops/reference.py:94-111)
 *                             (+ ts_paged_attention_workspace_bytes)
 *   ts_w8a16_gemm          <- ops/triton_w8a16.py:38-51 and ops/triton_ops.py:74-91
 *   ts_w8a16_gemm_v        <- the same with the tuned per-bucket config (autopilot/tuner.py)
 *   ts_w8a16_glu           <- model/qwen2.py:35-36, silu_mul(linear(x, gate_up)) fused
 *                             (ops/triton_ops.py:74-91 + ops/triton_silu_mul.py:21-28)
 *   ts_w8a16_add_rmsnorm   <- model/qwen2.py:84-92, rmsnorm_residual(linear(x, proj), residual)
 *                             fused (ops/triton_ops.py:74-91 + ops/triton_rmsnorm.py:30-46)
 *   ts_logits_int8         <- model/qwen2.py:94-99 with ops/triton_ops.py:88-91 (gather, int8
 *                             lm head and .float() fused)
 *   ts_step_metadata       <- runner/input_builder.py:81-150 (host arrays + seven copies) and
 *                             the decode-graph padding of runner/cuda_graphs.py:62-78
 *   ts_rmsnorm             <- ops/triton_rmsnorm.py:30-46   (twins ops/reference.py:13-23)
 *   ts_rope                <- ops/triton_rope.py:27-31      (twin ops/reference.py:31-42)
 *   ts_rope_kv_write       <- rope then kv_write of one layer, fused (model/qwen2.py:26-28, :89)
 *   ts_silu_mul            <- ops/triton_silu_mul.py:21-28  (twin ops/reference.py:26-28)
 *                             (twin ops/reference.py:45-47 + quant/int8.py:15-16)
 *
 * Conventions shared by every entry point
 *  - Plain pointers to device memory; the caller owns every buffer. The library never
 *    allocates or frees device memory; scratch space comes in through `workspace`.
 *  - Activations, K/V caches and outputs are IEEE fp16 (the reference's serving dtype).
 *    Strides are in elements, not bytes.
 *  - `stream` is a hipStream_t passed as void*; every launch is stream-ordered and no entry
 *    point synchronises with the host, so all of them can be captured into a hipGraph.
 *  - Return value: TS_OK (0) or a negative status. On error nothing has been launched and
 *    ts_last_error() returns a message (thread-local) naming the offending argument.
 *  - Paged KV cache of one layer: k_cache / v_cache are [num_blocks, num_kv_heads, 16, head_dim]
 *    contiguous (the per-layer views kv_cache[l, 0] / kv_cache[l, 1] of the reference's
 *    [L, 2, num_blocks, KVH, 16, D] tensor, engine/builder.py:76-80). Block 0 is the null block.
 *  - Memory safety instead of undefined behaviour: slot ids outside [0, num_blocks*16) are
 *    skipped like -1, block ids outside [0, num_blocks) read block 0, and a sequence whose
 *    seq_len exceeds 16 * max_blocks_per_seq attends only to the blocks its table holds.
 */
#ifndef TURINGSERVE_HIP_H
#define TURINGSERVE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TS_OK 0
#define TS_ERR_INVALID_ARG (-1)   /* null pointer, negative size, bad stride, bad alignment */
#define TS_ERR_UNSUPPORTED (-2)   /* a shape the kernels are not built for (e.g. head_dim 96) */
#define TS_ERR_WORKSPACE (-3)     /* workspace missing or smaller than *_workspace_bytes() */
#define TS_ERR_LAUNCH (-4)        /* the HIP runtime refused a launch */
#define TS_ERR_DEVICE (-5)        /* device query failed */

/* Decode kernel versions (ops/triton_decode_attention.py:1-10). */
#define TS_DECODE_AUTO 0          /* split (v3) when one workgroup per (seq, KV head) leaves CUs idle */
#define TS_DECODE_V1 1            /* one wavefront per (sequence, query head), VALU only */
#define TS_DECODE_V2 2            /* one workgroup per (sequence, KV head), GQA group on MFMA */
#define TS_DECODE_V3 3            /* v2 split over context partitions + reduction of the partials */

/* Library version string, e.g. "turingserve_hip 0.1.0 gfx950". */
const char* ts_version(void);

/* Message of the most recent call on this host thread: its error, or "" if it succeeded. */
const char* ts_last_error(void);

/* Number of compute units of `device` (the reference's num_sms, utils/gpu.py:19-24). */
int ts_device_cu_count(int device, int* cu_count);

/*
 * kv_write: for every token t with s = slot_mapping[t] >= 0,
 *   k_cache[s / 16, h, s % 16, :] = k[t, h, :] and v_cache[...] = v[t, h, :]  for all h.
 * Bit-exact copy. k and v may be strided views of the fused qkv activation
 * (stride over tokens k_stride_t, over heads k_stride_h, unit stride over head_dim).
 * Replaces ops/triton_kv_write.py:28-35 (twin ops/reference.py:50-57).
 */
int ts_kv_write(const void* k, const void* v,
                int64_t k_stride_t, int64_t k_stride_h,
                int64_t v_stride_t, int64_t v_stride_h,
                void* k_cache, void* v_cache, int64_t num_blocks,
                const int64_t* slot_mapping, int64_t num_tokens,
                int32_t num_kv_heads, int32_t head_dim, void* stream);

/*
 * Decode attention over the first num_seqs rows of the flat batch (one query token each,
 * q row s belongs to sequence s). out[s, h*D:(h+1)*D] = softmax(q_s,h . K^T * scale) . V over
 * the seq_lens[s] cached tokens of sequence s; rows with seq_len 0 are written as zeros.
 * version: TS_DECODE_*. partition: tokens per split for v3 (multiple of 16). partition > 0
 * gives the reference's fixed split grid: ceil(max_seq_len / partition) splits per sequence
 * (ops/triton_ops.py:50-51), tokens past max_seq_len are not attended. partition = 0 gives the
 * own-length schedule: sequence s of nb_s blocks is cut into min(R, ceil(nb_s / 24)) splits of
 * near-equal size, R = min(32, ceil(max_seq_len / 384)) (a longer sequence than max_seq_len gets
 * R longer splits and is still attended in full), so a row's result does not depend on the rest
 * of the batch; the splits of the batch are numbered densely, busy workgroups first.
 * max_seq_len: a host-side upper bound of seq_lens (inside graphs: max_model_len).
 * Workspace: ts_decode_workspace_bytes() bytes, 256-byte aligned (0 bytes for v1 / v2).
 * split_map / split_map_bytes: NULL / 0, or a map that ts_decode_split_map built from the same
 * seq_lens, block tables and plan arguments (version, num_seqs, heads, head_dim, max_seq_len,
 * partition, max_blocks_per_seq): the v3 split kernel then reads its split and its first block
 * ids from the map instead of scanning seq_lens, and merges its splits in the same launch (the
 * last split workgroup of each sequence and head group merges them, counted in the map; no
 * merge launch follows). The results are identical either way. A map built for another plan
 * poisons the rows (NaN); one smaller than the plan needs is an error; one built from other
 * seq_lens or block tables (an earlier step) poisons the rows whose length or last block moved.
 * The map must be rebuilt whenever seq_lens or the block tables change, and calls that share a
 * map must not overlap in time (its counters are shared; one stream orders them).
 * Replaces ops/triton_ops.py:35-57 and ops/triton_decode_attention.py:169-200.
 */
size_t ts_decode_workspace_bytes(int32_t version, int32_t num_seqs, int32_t num_heads,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t max_seq_len,
                                 int32_t partition, int32_t cu_count);
int ts_decode_attention(int32_t version,
                        const void* q, int64_t q_stride_t, int64_t q_stride_h,
                        void* out, int64_t out_stride_t,
                        const void* k_cache, const void* v_cache, int64_t num_blocks,
                        const int32_t* block_tables, int64_t bt_stride, int32_t max_blocks_per_seq,
                        const int32_t* seq_lens, int32_t num_seqs,
                        int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                        float scale, int32_t max_seq_len, int32_t partition,
                        void* workspace, size_t workspace_bytes, void* stream,
                        const void* split_map, size_t split_map_bytes);

/*
 * The per-step split map of the v3 decode schedule: for every launch slot of the plan the
 * sequence, split and block range it covers and the first block ids its wavefronts load. Built
 * once per step (one small launch) and passed to every layer's decode call of that step, it
 * replaces the per-workgroup seq_lens scan and block-table load that otherwise precede a split's
 * first K/V request. No counterpart in the reference (its split kernel needs no lookup: the
 * fixed grid of ops/triton_decode_attention.py:187-200 maps program ids to splits directly);
 * it belongs with the step metadata (runner/input_builder.py). ts_decode_split_map_bytes():
 * bytes for the plan, 0 when the plan does not split (v1 / v2) or for more than 4096 sequences
 * (then no map is built and the decode calls take NULL). The arguments mean what they mean for
 * ts_decode_attention. Stream-ordered: the decode calls that read the map follow it on the
 * same stream.
 */
size_t ts_decode_split_map_bytes(int32_t version, int32_t num_seqs, int32_t num_heads,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t max_seq_len,
                                 int32_t partition, int32_t cu_count);
int ts_decode_split_map(int32_t version, const int32_t* block_tables, int64_t bt_stride,
                        int32_t max_blocks_per_seq, int64_t num_blocks,
                        const int32_t* seq_lens, int32_t num_seqs, int32_t num_heads,
                        int32_t num_kv_heads, int32_t head_dim, int32_t max_seq_len,
                        int32_t partition, void* split_map, size_t split_map_bytes,
                        void* stream);

/*
 * ts_kv_write of the step's new rows followed by ts_decode_attention, as one launch: the
 * decode-only layer step of model/qwen2.py:26-28 with ops/triton_kv_write.py:28-35 and
 * ops/triton_ops.py:60-71 (pure decode). Row i of k / v ([num_seqs, num_kv_heads, head_dim],
 * strides in elements) goes to slot_mapping[i] exactly as ts_kv_write writes it, and the
 * attention then sees it. Precondition (what every input builder produces, incl. the graph
 * padding of runner/cuda_graphs.py:62-78): slot_mapping[i] is the slot of position
 * seq_lens[i] - 1, and a row with seq_lens[i] == 0 carries slot -1 (such a row is not written).
 * A row whose in-range slot is any other one is not written and its output row is NaN (the
 * write could not be ordered against other workgroups' reads of that block): use ts_kv_write
 * and ts_decode_attention for such rows.
 * The write is fused for v2 / v3 with at most 16 query heads per KV head and 16-byte aligned
 * rows; otherwise it runs as ts_kv_write's own launch before the attention. Same workspace and
 * split map as ts_decode_attention (ts_decode_workspace_bytes(), ts_decode_split_map()).
 */
int ts_decode_attention_kv_write(int32_t version,
                                 const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                 const void* k, const void* v, int64_t k_stride_t,
                                 int64_t k_stride_h, int64_t v_stride_t, int64_t v_stride_h,
                                 const int64_t* slot_mapping,
                                 void* out, int64_t out_stride_t,
                                 void* k_cache, void* v_cache, int64_t num_blocks,
                                 const int32_t* block_tables, int64_t bt_stride,
                                 int32_t max_blocks_per_seq, const int32_t* seq_lens,
                                 int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                 int32_t head_dim, float scale, int32_t max_seq_len,
                                 int32_t partition, void* workspace, size_t workspace_bytes,
                                 void* stream, const void* split_map, size_t split_map_bytes);

/*
 * ts_decode_attention_kv_write without a workspace argument: the split-K scratch is a static
 * device array of TS_NOALLOC_SCRATCH_BYTES inside the library (one per GPU, held until the
 * process ends), so this call allocates nothing. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under hipGraph capture, serving loops and
 * harnesses that forbid hipMalloc). Same arguments, results and preconditions as
 * ts_decode_attention_kv_write; a batch whose split scratch (ts_decode_workspace_bytes()) exceeds
 * TS_NOALLOC_SCRATCH_BYTES is rejected with TS_ERR_WORKSPACE before anything is launched. The
 * first call on a device looks up the array's device address (make it outside graph capture).
 * Calls that overlap on one GPU share the array and race: serialise them (one stream).
 */
#define TS_NOALLOC_SCRATCH_BYTES (16u << 20)
int ts_decode_attention_kv_write_noalloc(int32_t version,
                                         const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                         const void* k, const void* v, int64_t k_stride_t,
                                         int64_t k_stride_h, int64_t v_stride_t,
                                         int64_t v_stride_h, const int64_t* slot_mapping,
                                         void* out, int64_t out_stride_t,
                                         void* k_cache, void* v_cache, int64_t num_blocks,
                                         const int32_t* block_tables, int64_t bt_stride,
                                         int32_t max_blocks_per_seq, const int32_t* seq_lens,
                                         int32_t num_seqs, int32_t num_heads,
                                         int32_t num_kv_heads, int32_t head_dim, float scale,
                                         int32_t max_seq_len, int32_t partition, void* stream);

/*
 * ts_rope_kv_write followed by ts_decode_attention, as one launch: the whole attention half of a
 * pure-decode layer step (model/qwen2.py:26-28, :89 with ops/triton_rope.py:27-31,
 * ops/triton_kv_write.py:28-35 and ops/triton_ops.py:60-71). qkv rows as for ts_rope_kv_write
 * ([num_seqs, (H + 2 KVH) head_dim], 16-byte aligned, one decode row per sequence); q and the
 * new k rows are rotated at positions[i] with exactly ts_rope's arithmetic, the rotated k and the
 * v rows land in slot_mapping[i] and the attention sees them. The output and the caches are
 * bit-identical to the two calls; qkv itself is left unrotated when the launch is fused (the
 * rotated q and k exist only in registers and the cache) and rotated in place otherwise.
 * Preconditions, workspace and split map as ts_decode_attention_kv_write; fused for v2 / v3 with
 * at most 16 query heads per KV head and head_dim a multiple of 64, else ts_rope_kv_write runs
 * first.
 */
int ts_decode_rope_kv_write_attention(int32_t version, void* qkv, int64_t qkv_stride,
                                      const int64_t* positions, const float* cos_table,
                                      const float* sin_table, int64_t max_position,
                                      void* out, int64_t out_stride_t,
                                      void* k_cache, void* v_cache, int64_t num_blocks,
                                      const int64_t* slot_mapping,
                                      const int32_t* block_tables, int64_t bt_stride,
                                      int32_t max_blocks_per_seq, const int32_t* seq_lens,
                                      int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                      int32_t head_dim, float scale, int32_t max_seq_len,
                                      int32_t partition, void* workspace, size_t workspace_bytes,
                                      void* stream, const void* split_map,
                                      size_t split_map_bytes);

/*
 * Chunked-prefill attention for sequences num_decode .. num_seqs-1 of the flat batch.
 * Query row i of sequence b (rows query_start_loc[b] .. query_start_loc[b+1]-1) sits at
 * absolute position prefix + i, prefix = seq_lens[b] - q_len; it attends to keys
 * j <= prefix + i (bottom-right causal mask) read through block_tables[b].
 * num_tokens bounds every q / out row the kernel touches.
 * Without a workspace every 128-row query tile runs as one workgroup.
 * Replaces ops/triton_prefill_attention.py:66-79.
 */
int ts_prefill_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                         void* out, int64_t out_stride_t, int64_t num_tokens,
                         const void* k_cache, const void* v_cache, int64_t num_blocks,
                         const int32_t* block_tables, int64_t bt_stride, int32_t max_blocks_per_seq,
                         const int32_t* seq_lens, const int32_t* query_start_loc,
                         int32_t num_seqs, int32_t num_decode, int32_t max_query_len,
                         int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                         float scale, void* stream);

/*
 * The same with a workspace of ts_prefill_workspace_bytes() bytes (16-byte aligned): at
 * head_dim 128 the key range of a long query tile is then split over several workgroups whose
 * fp32 partials a merge kernel combines, so short chunks on long prefixes still fill the
 * device. max_seq_len: a host-side upper bound of the prefill sequences' seq_lens. A smaller
 * workspace (or none) runs the tiles unsplit. Same results up to fp32 summation order.
 * Replaces ops/triton_prefill_attention.py:66-79 (the launch grid of :72-79).
 */
size_t ts_prefill_workspace_bytes(int32_t num_prefill, int32_t num_heads, int32_t head_dim,
                                  int32_t max_query_len, int32_t max_seq_len, int32_t cu_count);
int ts_prefill_attention_ws(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                            void* out, int64_t out_stride_t, int64_t num_tokens,
                            const void* k_cache, const void* v_cache, int64_t num_blocks,
                            const int32_t* block_tables, int64_t bt_stride,
                            int32_t max_blocks_per_seq, const int32_t* seq_lens,
                            const int32_t* query_start_loc, int32_t num_seqs, int32_t num_decode,
                            int32_t max_query_len, int32_t max_seq_len, int32_t num_heads,
                            int32_t num_kv_heads, int32_t head_dim, float scale,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * paged_attention: decode attention on rows [0, num_decode), chunked-prefill attention on the
 * remaining sequences; one call per layer. With a workspace of
 * ts_paged_attention_workspace_bytes() bytes (256-byte aligned), head_dim 128, the automatic
 * (or v3) decode policy with partition 0 and both kinds of rows present, the two run in ONE
 * launch (prefill tiles and decode splits side by side) followed by one merge launch;
 * otherwise they run one after the other on `stream`, sharing the workspace (then the larger
 * of ts_decode_workspace_bytes() and ts_prefill_workspace_bytes() suffices). Same results
 * either way, up to fp32 summation order. max_seq_len bounds every seq_len (decode policy);
 * max_prefill_seq_len bounds the prefill rows' seq_lens (the prefill split plan; 0 = use
 * max_seq_len).
 * Replaces ops/triton_ops.py:60-71.
 */
size_t ts_paged_attention_workspace_bytes(int32_t num_seqs, int32_t num_decode,
                                          int32_t max_query_len, int32_t max_seq_len,
                                          int32_t max_prefill_seq_len, int32_t num_heads,
                                          int32_t num_kv_heads, int32_t head_dim,
                                          int32_t decode_version, int32_t partition,
                                          int32_t cu_count);
int ts_paged_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                       void* out, int64_t out_stride_t, int64_t num_tokens,
                       const void* k_cache, const void* v_cache, int64_t num_blocks,
                       const int32_t* block_tables, int64_t bt_stride, int32_t max_blocks_per_seq,
                       const int32_t* seq_lens, const int32_t* query_start_loc,
                       int32_t num_seqs, int32_t num_decode, int32_t max_query_len,
                       int32_t max_seq_len, int32_t max_prefill_seq_len,
                       int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                       float scale, int32_t decode_version, int32_t partition,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * W8A16 GEMM: y[M, N] = x[M, K] . (wq[N, K] * scale[N])^T (+ bias[N]), fp32 accumulation,
 * the per-output-channel scale applied once after the int8 x fp16 contraction
 * (ops/triton_w8a16.py:11-35). x, y fp16 row-major with leading dimensions ldx, ldy;
 * wq int8 row-major [N, K]; scale fp32 (scale_is_fp16 = 0, quant/int8.py:8-12) or fp16
 * (scale_is_fp16 = 1); bias fp16 or NULL.
 * Workspace: ts_w8a16_workspace_bytes() bytes (split-K partials for small M).
 */
size_t ts_w8a16_workspace_bytes(int32_t M, int32_t N, int32_t K, int32_t cu_count);
int ts_w8a16_gemm(const void* x, int64_t ldx, const int8_t* wq, const void* scale,
                  int32_t scale_is_fp16, const void* bias, void* y, int64_t ldy,
                  int32_t M, int32_t N, int32_t K,
                  void* workspace, size_t workspace_bytes, void* stream);

/*
 * The same product with a named kernel variant, the choice a tuning table makes for a shape
 * bucket (the role of the reference's per-bucket W8A16 configs, autopilot/tuner.py:116-134 and
 * ops/triton_ops.py:74-86): variant 0 = the library's own plan (as ts_w8a16_gemm), 1 = weight
 * streaming (M <= 32 only), 2 = 128 x 64 wide tiles, 3 = 128 x 128 wide tiles, 4 = 128 x 32
 * wide tiles (planned as 128 x 64 by ts_w8a16_glu), 5 = skinny (M <= 64, whole K per workgroup),
 * 6 = 128 x 192 wide tiles (128 weight rows x 192 activation rows), 7 = weight rows streamed on
 * the VALU (M <= 4, no split-K; it needs K % 16 == 0 and 16-byte aligned x rows and weights, and
 * runs the skinny kernel otherwise); splits = the
 * number of K splits (0 = the variant's own rule, at most 256; splits > 1 sum fp32 partials in
 * the workspace). Every variant computes the same product up to fp32 summation order.
 * Unavailable combinations return TS_ERR_UNSUPPORTED.
 */
size_t ts_w8a16_workspace_bytes_v(int32_t M, int32_t N, int32_t K, int32_t variant,
                                  int32_t splits, int32_t cu_count);
int ts_w8a16_gemm_v(const void* x, int64_t ldx, const int8_t* wq, const void* scale,
                    int32_t scale_is_fp16, const void* bias, void* y, int64_t ldy,
                    int32_t M, int32_t N, int32_t K, int32_t variant, int32_t splits,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * The gated MLP activation from the fused gate_up W8A16 linear, in one call:
 *   out[m][i] = fp16( fp16(silu(g)) * u ),  g = G[m][i], u = G[m][I + i],
 *   G = fp16( x . (wq * scale)^T + bias ), an [M, 2I] product never written to memory,
 * where silu(g) = g / (1 + exp(-g)) in fp32. This is model/qwen2.py:35-36's
 * silu_mul(linear(x, gate_up)) (ops/triton_silu_mul.py:21-28 after ops/triton_ops.py:74-91)
 * and equals, bit for bit, ts_silu_mul applied to ts_w8a16_gemm_v's output with the same
 * variant and splits: the product is planned for the [M, 2I] shape, and each gate value meets
 * its up value in the GEMM epilogue (or in the split-K reduction). wq int8 [2 * intermediate, K]
 * = [gate rows; up rows], scale / bias [2 * intermediate]; out fp16 [M, intermediate] with a
 * row stride that is a multiple of 4; x and variant / splits as for ts_w8a16_gemm_v.
 * Workspace: ts_w8a16_glu_workspace_bytes() bytes (the split-K partials, as for
 * ts_w8a16_gemm_v on the [M, 2I] shape).
 */
size_t ts_w8a16_glu_workspace_bytes(int32_t M, int32_t intermediate, int32_t K, int32_t variant,
                                    int32_t splits, int32_t cu_count);
int ts_w8a16_glu(const void* x, int64_t ldx, const int8_t* wq, const void* scale,
                 int32_t scale_is_fp16, const void* bias, void* out, int64_t ldo,
                 int32_t M, int32_t intermediate, int32_t K, int32_t variant, int32_t splits,
                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * A W8A16 product consumed by the residual add and RMSNorm of a decoder layer (o_proj before
 * post_attention_layernorm, down_proj before the next layer's input_layernorm or the final
 * norm: model/qwen2.py:84-92's rmsnorm_residual(linear(x, proj), residual)):
 *   y = fp16( x . (wq * scale)^T + bias ),   residual_out = y + residual,
 *   out = rmsnorm(residual_out) * norm_weight
 * equal, bit for bit, to ts_w8a16_gemm_v (same variant and splits) followed by ts_rmsnorm with
 * the residual. When the plan splits K, the norm launch reduces the fp32 partials itself (in the
 * split-K reduction's order) instead of a separate reduction launch; otherwise the product rows
 * go through the workspace to the norm. y is not written to memory. x, wq, scale, bias, M, N, K,
 * variant and splits as for ts_w8a16_gemm_v; residual, norm_weight, out, residual_out as for
 * ts_rmsnorm with hidden = N (a multiple of 8, at most 8192). Workspace:
 * ts_w8a16_add_rmsnorm_workspace_bytes() bytes (16-byte aligned; never zero for M > 0).
 */
size_t ts_w8a16_add_rmsnorm_workspace_bytes(int32_t M, int32_t N, int32_t K, int32_t variant,
                                            int32_t splits, int32_t cu_count);
int ts_w8a16_add_rmsnorm(const void* x, int64_t ldx, const int8_t* wq, const void* scale,
                         int32_t scale_is_fp16, const void* bias, const void* residual,
                         int64_t residual_stride, const void* norm_weight, void* out,
                         int64_t out_stride, void* residual_out, int64_t residual_out_stride,
                         int32_t M, int32_t N, int32_t K, float eps, int32_t variant,
                         int32_t splits, void* workspace, size_t workspace_bytes, void* stream);

/*
 * The qkv product of a layer step followed by RoPE and the K/V cache write (model/qwen2.py:26-28,
 * :89: linear(x, qkv_proj), then rope_ and kv_write, as ts_w8a16_gemm_v then ts_rope_kv_write):
 *   qkv = fp16( x . (wq * scale)^T + bias )  [M, (H + 2 KVH) head_dim] at row stride ld_qkv,
 * then q and k heads rotated in place at positions[m] and the rotated k and the v rows written to
 * slot_mapping[m] (slot -1 or past the cache: not written), bit for bit what the two calls leave.
 * With head_dim 128, a plan of wide tiles with one K split, K % 64 == 0, a 16-byte aligned
 * weight and 16-byte aligned qkv rows, tables and caches, the rotation and the cache rows happen
 * in the product's epilogue (one launch, the unrotated rows never reach memory); otherwise the two
 * launches run. x, wq, scale, bias, M, K, variant, splits and the workspace as for
 * ts_w8a16_gemm_v with N = (H + 2 KVH) head_dim; positions, tables and caches as for
 * ts_rope_kv_write. No separate counterpart in the reference (its layer makes the three calls).
 */
int ts_w8a16_qkv_rope_kv_write(const void* x, int64_t ldx, const int8_t* wq, const void* scale,
                               int32_t scale_is_fp16, const void* bias, void* qkv, int64_t ld_qkv,
                               int32_t M, int32_t K, int32_t num_heads, int32_t num_kv_heads,
                               int32_t head_dim, const int64_t* positions, const float* cos_table,
                               const float* sin_table, int64_t max_position, void* k_cache,
                               void* v_cache, int64_t num_blocks, const int64_t* slot_mapping,
                               int32_t variant, int32_t splits, void* workspace,
                               size_t workspace_bytes, void* stream);

/*
 * Logits of the sampling rows through the int8 tied lm head, in one launch (plus the split-K
 * reduction when num_samples is small): for s < num_samples,
 *   logits[s][v] = (float) fp16( sum_k hidden[sample_indices[s]][k] * wq[v][k] * scale[v] )
 * which is what the reference computes as hidden[sample_indices] (a gather), lm_head_int8
 * (the W8A16 product, fp16 result) and .float(): model/qwen2.py:94-99 with
 * ops/triton_ops.py:88-91. hidden fp16 [hidden_rows, hidden_size] (row stride hidden_stride,
 * 16-byte aligned rows); sample_indices int64 on the device (clamped to [0, hidden_rows));
 * wq int8 [vocab, hidden_size] and scale as for ts_w8a16_gemm; logits fp32
 * [num_samples, vocab] with a row stride that is a multiple of 4. The values equal those of
 * ts_w8a16_gemm on the gathered rows, widened to fp32.
 * Workspace: ts_logits_int8_workspace_bytes() bytes.
 */
size_t ts_logits_int8_workspace_bytes(int32_t num_samples, int32_t vocab, int32_t hidden_size,
                                      int32_t cu_count);
int ts_logits_int8(const void* hidden, int64_t hidden_stride, int64_t hidden_rows,
                   const int64_t* sample_indices, int32_t num_samples, const int8_t* wq,
                   const void* scale, int32_t scale_is_fp16, float* logits, int64_t logits_stride,
                   int32_t vocab, int32_t hidden_size, void* workspace, size_t workspace_bytes,
                   void* stream);

/*
 * One step's attention metadata built on the device from a compact packed int32 upload
 * (replaces the host builder of runner/input_builder.py:81-150 and the padding copies of
 * runner/cuda_graphs.py:62-78). `packed` (device memory) holds, in order:
 *   num_seqs descriptors of 5 int32 {start, n_tokens, sample (0 none, 1 last, 2 all),
 *   table_offset, table_len}, then num_tokens token ids, then num_block_ids block ids (the
 *   sequences' block tables concatenated; table_offset / table_len index them).
 * Writes, for the token rows in sequence order (row offset off_i = n_0 + ... + n_{i-1}):
 *   input_ids[row] = token, positions[row] = start + t,
 *   slot_mapping[row] = table[pos / 16] * 16 + pos % 16 (-1 when pos / 16 >= table_len);
 * per sequence: query_start_loc[i + 1] = off_i + n_i (query_start_loc[0] = 0),
 *   seq_lens[i] = start + n_i, block_tables row i (stride bt_stride) = the table padded with
 *   block 0 to bt_width entries; sample_indices (may be NULL) = the last row of each 'last'
 *   sequence with n_i > 0 and every row of each 'all' sequence, in order.
 * Sequences num_seqs .. pad_seqs - 1 become padding rows of a captured decode graph: one token
 * (id 0, position 0, slot -1) each after the real rows, seq_len 0, a zero table row, and
 * query_start_loc advancing by one. Output sizes: num_tokens + pad_seqs - num_seqs token rows,
 * pad_seqs + 1 query_start_loc entries, pad_seqs seq_lens and table rows.
 * Block ids past num_block_ids read as 0 and token rows past num_tokens are not written.
 */
int ts_step_metadata(const int32_t* packed, int32_t num_seqs, int64_t num_tokens,
                     int64_t num_block_ids, int32_t pad_seqs, int32_t bt_width, int64_t bt_stride,
                     int64_t* input_ids, int64_t* positions, int64_t* slot_mapping,
                     int32_t* query_start_loc, int32_t* seq_lens, int32_t* block_tables,
                     int64_t* sample_indices, void* stream);

/*
 * RMSNorm with optional fused residual add, one token row of `hidden` features at a time:
 *   r = residual ? fp16(x + residual) : x;  out = fp16(w * fp16(r * rsqrt(mean(r^2) + eps)))
 * with the mean in fp32; residual_out receives r when residual is given (ops/triton_rmsnorm.py:
 * 10-27). fp16 rows, 16-byte aligned; hidden a multiple of 8, at most 8192.
 * Replaces ops/triton_rmsnorm.py:30-46 (rmsnorm_residual / rmsnorm).
 */
int ts_rmsnorm(const void* x, int64_t x_stride, const void* residual, int64_t residual_stride,
               const void* weight, void* out, int64_t out_stride, void* residual_out,
               int64_t residual_out_stride, int64_t num_tokens, int32_t hidden, float eps,
               void* stream);

/*
 * In-place rotate-half RoPE on the first num_heads + num_kv_heads heads (q, then k) of each
 * token row of qkv [T, (H + 2 KVH) * D] fp16: with c, s the fp32 tables [max_position, D / 2]
 * rounded to fp16 at positions[t] (int64; clamped to the table), x1' = x1 c - x2 s and
 * x2' = x2 c + x1 s with every product and sum rounded to fp16, the twin's arithmetic
 * (ops/reference.py:31-42). head_dim a multiple of 8.
 * Replaces ops/triton_rope.py:27-31.
 */
int ts_rope(void* qkv, int64_t qkv_stride, const int64_t* positions, const float* cos_table,
            const float* sin_table, int64_t max_position, int64_t num_tokens, int32_t num_heads,
            int32_t num_kv_heads, int32_t head_dim, void* stream);

/*
 * ts_rope followed by ts_kv_write of the rotated k heads and the v heads of the same qkv rows,
 * in one pass over each row (the per-layer sequence rope -> kv_write of model/qwen2.py:26-28
 * and :89, ops/triton_rope.py:27-31 then ops/triton_kv_write.py:28-35): the q and k heads of
 * qkv [T, (H + 2 KVH) D] are rotated in place, and for slot_mapping[t] in [0, num_blocks * 16)
 * k_cache / v_cache [num_blocks, KVH, 16, D] receive row t's rotated k and its v at that slot.
 * The same bits as the two calls. qkv rows, caches and tables 16-byte aligned (qkv_stride a
 * multiple of 8); head_dim a multiple of 8.
 */
int ts_rope_kv_write(void* qkv, int64_t qkv_stride, const int64_t* positions,
                     const float* cos_table, const float* sin_table, int64_t max_position,
                     int64_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
                     int32_t head_dim, void* k_cache, void* v_cache, int64_t num_blocks,
                     const int64_t* slot_mapping, void* stream);

/*
 * out[t, i] = fp16(fp16(silu(g)) * u) for gu[t] = [g (intermediate) | u (intermediate)], silu in
 * fp32 (ops/triton_silu_mul.py:10-18). fp16 rows, 16-byte aligned; intermediate a multiple of 8.
 * Replaces ops/triton_silu_mul.py:21-28.
 */
int ts_silu_mul(const void* gu, int64_t gu_stride, void* out, int64_t out_stride,
                int64_t num_tokens, int32_t intermediate, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* TURINGSERVE_HIP_H */
