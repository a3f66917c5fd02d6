/*
 * phantom_attn.h - C ABI of the MI355X (gfx950) attention-forward library libphantom_attn.so.
 *
 * This is the drop-in boundary for the reference's attention forward path. Each entry point
 * replaces one reference launcher (L1, csrc/kernels/<name>.cuh) together with the torch glue
 * around it (L2, csrc/attn_<name>.cu); the Python package cuda_attn binds these through ctypes
 * in place of the reference's pybind11 module cuda_attn._C (csrc/bindings.cpp:40-54).
 *
 * Conventions shared by every entry point
 *   - q, k, v, o are device pointers to contiguous [BH][N][d] arrays (the reference's
 *     (B, H, N, d) tensors viewed as [B*H][N][d], csrc/bindings.cpp:12-22). Inputs are only
 *     read; o is only written. The library never allocates or frees device memory: outputs and
 *     the score workspace of the unfused paths are allocated by the caller (pa_tiled_fwd_noalloc
 *     instead uses a fixed array compiled into the library).
 *   - dtype / out_dtype take the PA_DTYPE_* codes below. out_dtype lets a caller ask for fp32
 *     output from fp16/bf16 inputs (the reference always writes o in the input dtype).
 *   - stream is a hipStream_t passed as void* (NULL = the null stream). Launches are
 *     asynchronous; nothing synchronises.
 *   - Return value: 0 on success; a positive hipError_t from the HIP runtime; or a negative
 *     PA_ERR_* code for a rejected argument. pa_last_error() then returns a message for the
 *     calling thread (the reference turned cudaError_t into RuntimeError through ATTN_CHECK,
 *     csrc/common.cuh:21-25).
 *   - Every entry point is re-entrant; the only state is a thread-local error string and a
 *     per-device attribute cache.
 */
#ifndef PHANTOM_ATTN_H_
#define PHANTOM_ATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum pa_dtype { PA_DTYPE_F32 = 0, PA_DTYPE_F16 = 1, PA_DTYPE_BF16 = 2 };

enum pa_status {
  PA_OK = 0,
  PA_ERR_INVALID = -1,     /* bad pointer, size, dtype or flag */
  PA_ERR_UNSUPPORTED = -2  /* shape/dtype/tile combination that is not compiled */
};

/* v1 naive: three kernels, fp32 N x N scores in the caller's workspace s (BH*N*N floats).
 * dtype: F32 or F16 (out in the same dtype); any d >= 1.
 * Replaces attn::launch_naive (csrc/kernels/naive.cuh:55-64) and naive_forward
 * (csrc/attn_naive.cu:5-14). */
int pa_naive_fwd(const void* q, const void* k, const void* v, void* o, float* s,
                 int dtype, int64_t bh, int64_t n, int64_t d, int causal, void* stream);

/* v2 tiled: LDS-tiled scores and P.V, one wave per softmax row; fp32 scores in workspace s.
 * dtype: F32 or F16; any d >= 1.
 * Replaces attn::launch_tiled (csrc/kernels/tiled.cuh:108-117) and tiled_forward
 * (csrc/attn_tiled.cu:5-14). */
int pa_tiled_fwd(const void* q, const void* k, const void* v, void* o, float* s,
                 int dtype, int64_t bh, int64_t n, int64_t d, int causal, void* stream);

/* tiled_forward without allocation: pa_tiled_fwd with the score workspace taken from a static
 * device array of the library instead of the caller. For callers that cannot allocate device
 * memory (code under stream/graph capture, serving loops, harnesses that forbid hipMalloc).
 * Limit: B*H*N*N <= 16777216 scores (64 MiB, held by every GPU the library runs on until the
 * process ends); larger calls return PA_ERR_UNSUPPORTED and should use pa_tiled_fwd. Calls no
 * allocating routine. Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (two streams, two host threads) race and must be serialised by the caller.
 * No counterpart in the reference (its glue always allocates the workspace with torch,
 * csrc/attn_tiled.cu:5-14). */
int pa_tiled_fwd_noalloc(const void* q, const void* k, const void* v, void* o,
                         int dtype, int64_t bh, int64_t n, int64_t d, int causal, void* stream);

/* v3 fused: online softmax with fp32 arithmetic throughout (fp32 MFMA, P kept in fp32).
 * dtype: F32 or F16; out_dtype: dtype or F32; d == 64.
 * Replaces attn::launch_fused<T> (csrc/kernels/fused.cuh:106-112) and fused_forward
 * (csrc/attn_fused.cu:5-14). */
int pa_fused_fwd(const void* q, const void* k, const void* v, void* o,
                 int dtype, int out_dtype, int64_t bh, int64_t n, int64_t d, int causal, void* stream);

/* v3.1/v3.2 fused_tuned: the fp16 MFMA kernel at query tile br and key tile bc, with
 * (double_buffer=1) or without (0) the two-stage LDS pipeline.
 * dtype: F16; out_dtype: F16 or F32; d == 64; (br, bc) in {(64,32),(64,64),(128,32),(128,64)}.
 * Replaces attn::launch_fused_tuned (csrc/kernels/fused_tuned.cuh:212-228) and
 * fused_tuned_forward (csrc/attn_fused_tuned.cu:5-21). */
int pa_fused_tuned_fwd(const void* q, const void* k, const void* v, void* o,
                       int dtype, int out_dtype, int64_t bh, int64_t n, int64_t d, int causal,
                       int double_buffer, int br, int bc, void* stream);

/* v4 fused_tc: QK^T and PV on MFMA (fp16/bf16 in, fp32 accumulate), online softmax between.
 * dtype: F16 or BF16; out_dtype: dtype or F32; d in {64, 128}.
 * The launch is persistent (as many workgroups as fit on the device at once, walking the query
 * blocks) for causal == 0 with an even number of 64-key tiles (or an odd number, above one, of
 * full ones), and for every causal != 0 call (its walk over the query blocks chosen from the
 * shape); unless pa_set_persistent(0) switched that off (see below). Otherwise one workgroup per
 * query block. pa_fused_tc_kernel names the choice.
 * Both launches give the same bits.
 * Replaces attn::launch_fused_tc (csrc/kernels/fused_tc.cuh:187-196) and fused_tc_forward
 * (csrc/attn_fused_tc.cu:5-19). */
int pa_fused_tc_fwd(const void* q, const void* k, const void* v, void* o,
                    int dtype, int out_dtype, int64_t bh, int64_t n, int64_t d, int causal,
                    void* stream);

/* The kernel instantiation and launch shape pa_fused_tc_fwd would use for these arguments, as
 * text ("" if the combination is not compiled). For reports and profiles; no GPU needed (without
 * a device the persistent launch is not chosen, as in pa_fused_tc_fwd).
 * No reference counterpart: the reference launches one fixed kernel (csrc/kernels/fused_tc.cuh:187-196). */
const char* pa_fused_tc_kernel(int dtype, int out_dtype, int64_t bh, int64_t n, int64_t d, int causal);

/* Process-wide switch of fused_tc's persistent launch: enable = 0 selects one workgroup
 * per query block, nonzero the persistent launch. Returns the previous setting. The initial
 * setting is read once, when the library is loaded, from the environment variable
 * PA_PERSISTENT ("0" = off; unset or anything else = on). For A/B measurements and tests; calls
 * already launched are not affected.
 * No reference counterpart (the reference has one launch form). */
int pa_set_persistent(int enable);

/* LDS bytes one workgroup of fused_tuned needs, or -1 if (br, bc, d, dtype) is not compiled.
 * Replaces fused_tuned_smem_bytes (csrc/kernels/fused_tuned.cuh:188-190). No GPU needed. */
int64_t pa_fused_tuned_lds_bytes(int br, int bc, int double_buffer, int64_t d, int dtype);

/* LDS bytes one workgroup of fused_tc needs, or -1 if (d, dtype) is not compiled: the largest of
 * its launch forms (the persistent forms add rows that stage O before its stores).
 * Replaces fused_tc_smem_bytes (csrc/kernels/fused_tc.cuh:184). No GPU needed. */
int64_t pa_fused_tc_lds_bytes(int64_t d, int dtype);

/* LDS bytes one workgroup may use on `device`, written to *bytes.
 * Replaces smem_optin_bytes (csrc/common.cuh:35-40). */
int pa_device_lds_limit(int device, int64_t* bytes);

/* Message for the last nonzero status returned on this thread ("" if none). */
const char* pa_last_error(void);

/* Library version and the offload architecture it was compiled for. */
const char* pa_version(void);

#ifdef __cplusplus
}
#endif

#endif /* PHANTOM_ATTN_H_ */
