// libphantom_attn_tiles.so: the tile and occupancy alternatives of the fused MFMA kernel, compiled
// beside the library for the counter-driven tile choice (autotune/select_tiles.py) and nothing
// else. fused_tc launches one tile per head dim; this library launches the shapes that choice was
// made against, so that each can be timed and profiled with rocprofv3 on the same inputs:
//   d = 128: 128-query workgroups (two per CU), 32- and 128-key tiles, one LDS stage;
//   d = 64:  256-query workgroups, 64-query workgroups, 32-key tiles, 128-key tiles, and the
//            shipped tile's persistent launch held to two workgroups per CU.
// The shipped tiles themselves are measured through libphantom_attn.so (both its launch forms).
// Declarations: include/phantom_attn_tiles.h. Non-causal calls only; same argument checks and
// status convention as libphantom_attn.so.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <type_traits>

#include "phantom_attn.h"
#include "phantom_attn_tiles.h"
#include "kernels/fa_mfma.hpp"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

// dry: only compute the grid (into *grid_out), launch nothing.
typedef hipError_t (*launch_fn)(const void*, const void*, const void*, void*, int, int, hipStream_t, int*, bool);

// One candidate: the kernel's template arguments and whether it takes the persistent launch (as
// many workgroups as fit at once, or at most wgs_cap per CU, walking the query blocks of their
// XCD; needs N a multiple of 2 * BN, as the shipped persistent form without its ragged copy).
struct Candidate {
  const char* label;
  int dtype, d, br, bc, stages, persistent, wgs_cap;
  launch_fn fn;
};

template <typename T, int D, int BM, int BN, int ST, bool PERSIST, int CAP>
hipError_t launch(const void* q, const void* k, const void* v, void* o, int bh, int n, hipStream_t stream,
                  int* grid_out, bool dry) {
  // fp16 two-stage candidates take the packed-max check, as fused_tc's fp16 tiles do on these
  // (non-causal) calls, so that they compare like with like.
  constexpr bool kCheck = std::is_same<T, pa::f16>::value && ST == 2;
  auto kernel = pa::fa_mfma_fwd<T, D, BM, BN, ST, T, 1, PERSIST, false, false, kCheck>;
  const int threads = BM / 32 * pa::kWave;
  const int qblocks = (n + BM - 1) / BM;
  const long long total = (long long)qblocks * bh;
  if (total > INT_MAX) return hipErrorInvalidConfiguration;
  int grid = (int)total, cus_per_xcd = 0;
  if constexpr (PERSIST) {
    int dev = 0, cus = 0, per_cu = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0);
    if (e != hipSuccess) return e;
    if (per_cu <= 0) return hipErrorInvalidConfiguration;
    if (CAP > 0) per_cu = std::min(per_cu, CAP);
    cus_per_xcd = cus / pa::kNumXcd;
    const long long per_xcd = (total + pa::kNumXcd - 1) / pa::kNumXcd;
    grid = (int)std::min<long long>((long long)cus_per_xcd * per_cu, per_xcd) * pa::kNumXcd;
  }
  if (grid_out) *grid_out = grid;
  if (dry) return hipSuccess;
  hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(threads), 0, stream, static_cast<const T*>(q),
                     static_cast<const T*>(k), static_cast<const T*>(v), static_cast<T*>(o), n, qblocks, (int)total,
                     pa::kLog2e / sqrtf((float)D), 0, cus_per_xcd, 0);
  return hipGetLastError();
}

#define PA_CAND(label, T, code, D, BM, BN, ST, P, CAP) \
  Candidate { label, code, D, BM, BN, ST, P, CAP, &launch<T, D, BM, BN, ST, P, CAP> }

const Candidate kCandidates[] = {
    PA_CAND("br128_bc64_2stage_persistent", pa::bf16, PA_DTYPE_BF16, 128, 128, 64, 2, true, 0),
    PA_CAND("br128_bc64_2stage", pa::bf16, PA_DTYPE_BF16, 128, 128, 64, 2, false, 0),
    PA_CAND("br256_bc32_2stage_persistent", pa::bf16, PA_DTYPE_BF16, 128, 256, 32, 2, true, 0),
    PA_CAND("br256_bc128_1stage", pa::bf16, PA_DTYPE_BF16, 128, 256, 128, 1, false, 0),
    PA_CAND("br256_bc64_1stage", pa::bf16, PA_DTYPE_BF16, 128, 256, 64, 1, false, 0),
    // fused_tc's general d = 128 tile, persistent: the alternative on the grids where fused_tc
    // launches the 128-query tile (a grid where fused_tc launches this one skips it as a duplicate)
    PA_CAND("br256_bc64_2stage_persistent_d128", pa::bf16, PA_DTYPE_BF16, 128, 256, 64, 2, true, 0),
    PA_CAND("br256_bc64_2stage_persistent", pa::f16, PA_DTYPE_F16, 64, 256, 64, 2, true, 0),
    PA_CAND("br64_bc64_2stage_persistent", pa::f16, PA_DTYPE_F16, 64, 64, 64, 2, true, 0),
    PA_CAND("br128_bc32_2stage_persistent", pa::f16, PA_DTYPE_F16, 64, 128, 32, 2, true, 0),
    PA_CAND("br128_bc128_1stage", pa::f16, PA_DTYPE_F16, 64, 128, 128, 1, false, 0),
    PA_CAND("br128_bc64_2stage_persistent_2wg", pa::f16, PA_DTYPE_F16, 64, 128, 64, 2, true, 2),
};
constexpr int kCount = (int)(sizeof(kCandidates) / sizeof(kCandidates[0]));

const Candidate* find(int index) { return index >= 0 && index < kCount ? &kCandidates[index] : nullptr; }

}  // namespace

extern "C" {

int pa_tiles_count(void) { return kCount; }

const char* pa_tiles_label(int index) {
  const Candidate* c = find(index);
  return c ? c->label : "";
}

int pa_tiles_describe(int index, int* dtype, int* d, int* br, int* bc, int* stages, int* persistent,
                      int* wgs_per_cu) {
  const Candidate* c = find(index);
  if (!c) return fail(PA_ERR_INVALID, "pa_tiles_describe: no candidate %d (there are %d)", index, kCount);
  if (!dtype || !d || !br || !bc || !stages || !persistent || !wgs_per_cu)
    return fail(PA_ERR_INVALID, "pa_tiles_describe: null output");
  *dtype = c->dtype;
  *d = c->d;
  *br = c->br;
  *bc = c->bc;
  *stages = c->stages;
  *persistent = c->persistent;
  *wgs_per_cu = c->wgs_cap;
  return PA_OK;
}

int pa_tiles_fwd(int index, const void* q, const void* k, const void* v, void* o, int dtype, int64_t bh, int64_t n,
                 int64_t d, int causal, void* stream) {
  const Candidate* c = find(index);
  if (!c) return fail(PA_ERR_INVALID, "pa_tiles_fwd: no candidate %d (there are %d)", index, kCount);
  if (!q || !k || !v || !o) return fail(PA_ERR_INVALID, "%s: null tensor pointer", c->label);
  if (bh <= 0 || n <= 0 || bh > INT_MAX || n > INT_MAX)
    return fail(PA_ERR_INVALID, "%s: B*H and N must be in [1, 2^31-1]", c->label);
  for (const void* p : {q, k, v, static_cast<const void*>(o)})
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return fail(PA_ERR_INVALID, "%s: inputs must be 16-byte aligned", c->label);
  if (dtype != c->dtype || d != c->d)
    return fail(PA_ERR_UNSUPPORTED, "%s: compiled for dtype %d, d = %d only", c->label, c->dtype, c->d);
  if (causal) return fail(PA_ERR_UNSUPPORTED, "%s: non-causal calls only", c->label);
  if ((uint64_t)n * (uint64_t)d * 2 >= (1ull << 31))
    return fail(PA_ERR_UNSUPPORTED, "%s: one head (N*d*2 bytes) must stay below 2 GiB", c->label);
  if (c->persistent && n % (2 * c->bc) != 0)
    return fail(PA_ERR_UNSUPPORTED, "%s: the persistent candidates need N a multiple of %d", c->label, 2 * c->bc);
  int grid = 0;
  const hipError_t e = c->fn(q, k, v, o, (int)bh, (int)n, static_cast<hipStream_t>(stream), &grid, false);
  if (e != hipSuccess) return fail((int)e, "%s: HIP error: %s", c->label, hipGetErrorString(e));
  return PA_OK;
}

const char* pa_tiles_kernel(int index, int64_t bh, int64_t n) {
  thread_local char desc[256];
  const Candidate* c = find(index);
  if (!c || bh <= 0 || n <= 0) return "";
  static const char* dt_name[] = {"f32", "f16", "bf16"};
  int grid = (int)std::min<long long>((n + c->br - 1) / c->br * bh, INT_MAX);
  if (c->persistent && c->fn(nullptr, nullptr, nullptr, nullptr, (int)bh, (int)n, nullptr, &grid, true) != hipSuccess)
    grid = 0;   // no device: the grid is unknown
  char cap[48] = "";
  if (c->wgs_cap > 0) snprintf(cap, sizeof(cap), " (at most %d workgroups per CU)", c->wgs_cap);
  const bool check = c->dtype == PA_DTYPE_F16 && c->stages == 2;   // as in launch()
  snprintf(desc, sizeof(desc), "fa_mfma_fwd<%s, D=%d, BM=%d, BN=%d, %d stages, out %s%s%s> grid %d x %d threads%s",
           dt_name[c->dtype], c->d, c->br, c->bc, c->stages, dt_name[c->dtype], c->persistent ? ", persistent" : "",
           check ? ", packed-max check" : "", grid, c->br / 32 * pa::kWave, cap);
  return desc;
}

const char* pa_tiles_last_error(void) { return g_err; }

}  // extern "C"
