/* Read-bandwidth probes used by bench.py to state the practical HBM read
 * ceilings beside the decode kernel's figure (library libbw_probe_gfx950.so,
 * source vllm-inference-engine_amd/probes/bw_probe.hip). Measurement
 * infrastructure: no counterpart in the reference, whose benchmark states a
 * device-copy line instead (README.md:86). Return 0 on success, 1 on a bad
 * argument, 4 when the launch fails. Asynchronous on `stream` (a hipStream_t). */
#ifndef BW_PROBE_H
#define BW_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BWP_API __attribute__((visibility("default")))

/* Reads `bytes` (a multiple of 8 KB is read; 16-byte aligned buffer) once
 * with `grid` workgroups of eight wavefronts; `sink` is a 4-byte device word
 * that is written only if the data's XOR equals a fixed constant. */
BWP_API int bwp_read_stream(const void* buf, int64_t bytes, void* sink, int grid, void* stream);

/* Reads blocks ids[0 .. n_ids) of a pool of num_blocks blocks of block_bytes
 * (1, 2, 3 or 4 KB; ids clamped into the pool) in list order, wavefront i
 * taking blocks i, i + W, ... (W wavefronts in `grid` workgroups of eight),
 * four blocks in flight per wavefront. */
BWP_API int bwp_gather_blocks(const void* pool, int num_blocks, int block_bytes,
                              const int32_t* ids, int n_ids, void* sink, int grid, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BW_PROBE_H */
