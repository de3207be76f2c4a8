/*
 * libturingserve_probes.so: measurement probes. NOT part of the product ABI: a separate,
 * measurement-only library (built beside libturingserve_hip.so and linked against it for its
 * status codes and ts_last_error), loaded only by bench.py to measure the ceilings that its
 * roofline fractions are read against. No counterpart in the reference.
 */
#ifndef TURINGSERVE_PROBES_H
#define TURINGSERVE_PROBES_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * ts_probe_gather: reads n_chunks chunks of chunk_bytes (2048 or 4096) at base + chunk_offsets[i]
 * (bytes, 16-byte aligned) with no arithmetic; writes one word per 8 chunks to sink
 * (ceil(n_chunks / 8) words). ts_probe_mfma: `workgroups` workgroups of 4 wavefronts, each
 * wavefront runs `iters` rounds of four independent v_mfma_f32_32x32x16_f16 (4 * 32768 flops);
 * writes one float per wavefront to sink. Status codes and the error message as in
 * turingserve_hip.h.
 */
int ts_probe_gather(const void* base, const int64_t* chunk_offsets, int32_t n_chunks,
                    int32_t chunk_bytes, uint32_t* sink, void* stream);
int ts_probe_mfma(int32_t workgroups, int32_t iters, float* sink, void* stream);

/*
 * ts_probe_gather_k_operand: as ts_probe_gather, but the first of each wavefront's two chunks
 * (the K chunk of a block in a decode step's chunk list, which alternates K and V) is read in the
 * decode kernel's K operand layout: each load instruction takes 64 bytes of each of the chunk's
 * 16 token rows instead of one contiguous KiB. The second chunk is read as in ts_probe_gather.
 */
int ts_probe_gather_k_operand(const void* base, const int64_t* chunk_offsets, int32_t n_chunks,
                              int32_t chunk_bytes, uint32_t* sink, void* stream);

/*
 * ts_probe_gather_persistent: the same chunk list read by `workgroups` workgroups of 4
 * wavefronts, each wavefront streaming an equal contiguous range of the list's 1 KiB pieces with
 * `depth` (4 or 8) whole-piece loads in flight; use_lds != 0 issues them as LDS DMA into a ring.
 * A wavefront's range must span at most 62 chunks (else TS_ERR_INVALID_ARG: more workgroups).
 * sink: at least 4 * workgroups words.
 */
int ts_probe_gather_persistent(const void* base, const int64_t* chunk_offsets, int32_t n_chunks,
                               int32_t chunk_bytes, int32_t workgroups, int32_t depth,
                               int32_t use_lds, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* TURINGSERVE_PROBES_H */
