/* libphantom_attn_tiles.so: tile and occupancy alternatives of the fused MFMA kernel, for the
 * counter-driven tile choice only (phantom-a100_amd/autotune/select_tiles.py). Not on the
 * attention path: cuda_attn never loads it.
 *
 * The reference chooses among compiled tile shapes at run time through
 * attn::launch_fused_tuned_cfg (csrc/kernels/fused_tuned.cuh:192-228) and scores them with its
 * simulator's counters (autotune/hw_counters.py:33-76, autotune/diagnose.py:17-77). fused_tc
 * here launches one tile per head dim (include/phantom_attn.h); this library launches the
 * alternatives that choice was made against, so each can be timed and profiled on the device.
 *
 * Status codes and dtype codes are those of phantom_attn.h; errors leave a message for
 * pa_tiles_last_error(). Nothing here allocates; launches go to the caller's stream. */
#ifndef PHANTOM_ATTN_TILES_H
#define PHANTOM_ATTN_TILES_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Number of compiled candidates; they are indexed 0 .. count - 1. */
int pa_tiles_count(void);

/* The candidate's label, e.g. "br128_bc64_2stage_persistent" ("" for a bad index). */
const char* pa_tiles_label(int index);

/* The candidate's input dtype, head dim, query rows per workgroup (br), keys per tile (bc), LDS
 * stages and launch form (persistent 1: as many workgroups as fit at once walk the query blocks;
 * 0: one workgroup per query block), and for a persistent candidate the most workgroups it
 * places per CU (0: as many as fit). */
int pa_tiles_describe(int index, int* dtype, int* d, int* br, int* bc, int* stages, int* persistent,
                      int* wgs_per_cu);

/* O = softmax(Q K^T / sqrt(d)) V with candidate `index`, as pa_fused_tc_fwd (output in the input
 * dtype). Only non-causal calls of the candidate's dtype and head dim; the persistent candidates
 * also need N a multiple of 2 * bc. */
int pa_tiles_fwd(int index, const void* q, const void* k, const void* v, void* o, int dtype, int64_t bh, int64_t n,
                 int64_t d, int causal, void* stream);

/* The instantiation and grid pa_tiles_fwd launches for (bh, n), as text. */
const char* pa_tiles_kernel(int index, int64_t bh, int64_t n);

/* Message of the last failed call on this thread. */
const char* pa_tiles_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* PHANTOM_ATTN_TILES_H */
