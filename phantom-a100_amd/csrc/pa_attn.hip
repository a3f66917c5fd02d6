// C ABI of libphantom_attn.so: argument validation, dispatch to the compiled kernel
// instantiations, launch on the caller's stream. Declarations and the reference interface each
// entry replaces are in include/phantom_attn.h.
//
// Host-side rules: no allocation, no synchronisation, no per-call hipFuncSetAttribute (all LDS
// is static, so a launch needs no opt-in call; the reference set the attribute on every call,
// /root/reference/csrc/kernels/fused_tc.cuh:189-191). Errors come back as status codes with a
// thread-local message.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <vector>

#include "phantom_attn.h"
#include "kernels/fa_f32.hpp"
#include "kernels/fa_mfma.hpp"
#include "kernels/unfused.hpp"
#include "launch_model.hpp"

#ifndef PA_VERSION_STRING
#define PA_VERSION_STRING "0.1.0"
#endif

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* name) {
  if (e == hipSuccess) return PA_OK;
  return fail((int)e, "%s: HIP error: %s", name, hipGetErrorString(e));
}

size_t dtype_bytes(int dt) { return dt == PA_DTYPE_F32 ? 4 : 2; }

// The fused kernels address one head through a 32-bit buffer offset (N*d elements per head).
int check_head_bytes(const char* name, int64_t n, int64_t d, int dtype) {
  if ((uint64_t)n * (uint64_t)d * dtype_bytes(dtype) >= (1ull << 31))
    return fail(PA_ERR_UNSUPPORTED, "%s: one head (N*d*%zu bytes) must stay below 2 GiB", name, dtype_bytes(dtype));
  return PA_OK;
}

// Shared argument checks. Pointers must be non-null and 16-byte aligned (the kernels move
// 16-byte vectors); sizes must keep every in-kernel 32-bit index in range.
int check_common(const char* name, const void* q, const void* k, const void* v, const void* o,
                 int64_t bh, int64_t n, int64_t d) {
  if (!q || !k || !v || !o) return fail(PA_ERR_INVALID, "%s: null tensor pointer", name);
  if (bh <= 0 || n <= 0 || d <= 0) return fail(PA_ERR_INVALID, "%s: inputs must be non-empty", name);
  if (bh > INT_MAX || n > INT_MAX || d > INT_MAX)
    return fail(PA_ERR_INVALID, "%s: tensor dimension exceeds 2^31-1", name);
  return PA_OK;
}

int check_aligned16(const char* name, const void* q, const void* k, const void* v, const void* o) {
  for (const void* p : {q, k, v, o})
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return fail(PA_ERR_INVALID, "%s: inputs must be 16-byte aligned", name);
  return PA_OK;
}

float scale_log2_for(int64_t d) { return pa::kLog2e / sqrtf((float)d); }

// ------------------------------------------------------------------ fused MFMA (fp16 / bf16)
// Compute units of the current device (looked up once per device), 0 if unknown.
int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// The persistent d = 128 launch is on unless the environment sets PA_PERSISTENT=0 when the library
// is loaded; pa_set_persistent() switches it afterwards (a process-wide flag, read once per launch).
int persistent_from_env() {
  const char* e = getenv("PA_PERSISTENT");
  return (e && e[0] == '0') ? 0 : 1;
}
std::atomic<int> g_persistent{persistent_from_env()};
bool persistent_enabled() { return g_persistent.load(std::memory_order_relaxed) != 0; }

// fused_tc, non-causal, an even number of key tiles or an odd number of full ones: the persistent
// form. As many workgroups as fit on the device at once (d = 128: one 8-wave workgroup per CU;
// d = 64: three 4-wave workgroups per CU) each walk the query blocks of their XCD, so the
// next block's first tiles load during the current block's last two. Measured on MI355X,
// TFLOP/s with one workgroup per query block -> persistent: B x H x N = 4x32x4096 / 2x16x8192 /
// 1x64x2048 / 16x16x1024 at
// d = 128: bf16 1125 / 1198 / 1062 / 929 -> 1184 / 1247 / 1126 / 1049, fp16 1021 / 1081 / 967 /
// 868 -> 1043 / 1099 / 1002 / 941; at d = 64 fp16 (three workgroups per CU): C3 681 -> 708,
// C5 845 -> 890 (back to back), 605 -> 627 and 821 -> 859 under the flushing protocol.
// Causal rows take the CAUSAL form for any N (a head's last block then ends past N, with rows that
// are computed and not stored) and any B*H, with the walk persistent_grid_for picks: faster than
// one workgroup per block (which leaves CUs idle between blocks of unequal length and ends with the
// most loaded CU) in every causal shape measured (launch_model.hpp).
// (Only the two-stage fused_tc kernels without a key split have persistent forms; the caller,
// persistent_grid_for, is instantiated for those alone.)
bool persistent_launch(int64_t n, int bn, int causal) {
  if (!persistent_enabled()) return false;
  // (An odd count of full tiles is padded with an empty one; a single tile is not, since a bf16
  // row of one tile takes its P as two terms, which only the per-block launch does.)
  return causal || (n + bn - 1) / bn % 2 == 0 || (n % bn == 0 && n > bn);
}
// Workgroups of the persistent launch: wgs_per_cu per CU, at most as many per XCD as the XCD has
// blocks.
int persistent_grid(long long total_blocks, int wgs_per_cu) {
  const long long per_xcd = (total_blocks + pa::kNumXcd - 1) / pa::kNumXcd;
  return (int)std::min<long long>((long long)device_cus() / pa::kNumXcd * wgs_per_cu, per_xcd) * pa::kNumXcd;
}

// Workgroups of an fa_mfma_fwd instantiation that fit on one CU of the current device (queried
// once per device), 0 if unknown.
template <typename T, int D, int BM, int BN, int ST, typename OutT, int KS, bool PERSIST, bool RAGGED, bool CAUSAL,
          bool CHECK = false>
int wgs_per_cu() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, pa::fa_mfma_fwd<T, D, BM, BN, ST, OutT, KS, PERSIST, RAGGED, CAUSAL, CHECK>,
                                                     BM / 32 * pa::kWave * KS, 0) != hipSuccess || n <= 0)
      return 0;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Grid of the persistent launch of this call, 0 for one workgroup per query block. A call that
// needs the RAGGED form keeps the persistent launch only if that kernel fits as many workgroups
// per CU as the clean one. It does at d = 128 (one workgroup per CU either way; padding an odd
// tile count gained, bf16 4x32x4032 1190 -> 1221, 16x16x960 930 -> 960 TFLOP/s) and at d = 64,
// where it is held to three (fp16 unconstrained took 217 VGPRs, two workgroups per CU, and lost
// to the per-block launch: 4x16x4032 864 vs 895, 8x16x960 672 vs 724; held, with no spill, per
// block -> persistent 4x16x4032 904 -> 905, 8x16x960 728 -> 720, 16x16x1000 775 -> 800,
// 8x16x4050 908 -> 894, 1x16x8000 883 -> 920).
struct PersistentPlan {
  int grid = 0;      // workgroups of the persistent launch, 0 for one workgroup per query block
  int walk = 0;      // causal walk: 0 per-XCD lists head by head, 1 per-XCD lists by length, 2 one list
};
template <typename T, int D, int BM, int BN, int ST, typename OutT, int KS>
PersistentPlan persistent_grid_for(int64_t n, int64_t bh, int causal) {
  static_assert(ST == 2 && KS == 1, "persistent forms: two stages, no key split");
  if (!persistent_launch(n, BN, causal)) return {};
  const long long total = (n + BM - 1) / BM * bh;
  if (causal) {
    const int wpc = wgs_per_cu<T, D, BM, BN, ST, OutT, KS, true, false, true>();
    const int cus = device_cus() / pa::kNumXcd;
    // Per-XCD lists (each XCD owning whole heads) need B*H a multiple of 8, or else at most 25 %
    // more heads on the busiest XCD than the mean and a block for every workgroup on every XCD
    // (measured per XCD against the per-block launch, TFLOP/s: bf16 d = 128 N = 4096 B*H = 63 / 42
    // / 20: 961 -> 1182, 877 -> 931, 738 -> 886; B*H = 100, N = 1024: 485 -> 694; fp16 d = 64,
    // B*H = 81, N = 2048: 558 -> 715; outside the rule: B*H = 12 (N = 4096, d = 128) 619 -> 601,
    // fp16 d = 64 B*H = 42 N = 2048, under a block per workgroup, 453 -> 374). Otherwise the walk
    // takes one list over the device.
    const bool per_xcd = bh % pa::kNumXcd == 0 ||
                         ((bh + pa::kNumXcd - 1) / pa::kNumXcd * pa::kNumXcd * 4 <= bh * 5 &&
                          bh / pa::kNumXcd * ((n + BM - 1) / BM) >= (long long)cus * wpc);
    const int grid = persistent_grid(total, wpc);
    if (grid <= 0) return {};
    return {grid, pa::causal_walk(n, bh, BM, BN, grid / pa::kNumXcd, cus, D == 64, per_xcd)};
  }
  constexpr bool kCheck = std::is_same<T, pa::f16>::value;   // the fp16 non-causal forms' packed-max check
  const int clean = wgs_per_cu<T, D, BM, BN, ST, OutT, KS, true, false, false, kCheck>();
  if (n % (2 * BN) == 0) return {persistent_grid(total, clean), 0};
  const int ragged = wgs_per_cu<T, D, BM, BN, ST, OutT, KS, true, true, false, kCheck>();
  return ragged >= clean ? PersistentPlan{persistent_grid(total, ragged), 0} : PersistentPlan{};
}

// fused_tc with fp16 inputs on non-causal rows (two stages, no key split) uses the packed-max
// check instead of the per-tile row max (kernel template argument CHECK) in its persistent forms,
// and at d = 128 also in the per-block form (so both launch forms of a d = 128 call give the same
// bits); causal rows, the d = 64 per-block form, the key split and the fused_tuned tiles keep the
// row max. Measured back to back, row max -> packed-max check (TFLOP/s), persistent: d = 64
// 8x16x1024 (C3) 777 -> 806 and 694 -> 728, 1x16x8192 with Q, K x3 (C5) 926 -> 944 and 945 -> 966,
// 4x16x4096 888 -> 927, 16x16x2048 863 -> 899, 4x16x4032 (ragged) 863 -> 898, 8x16x1000 (ragged)
// 748 -> 744; d = 128 4x32x4096 1080 -> 1152. Per block: d = 128 4x32x4096 1048 -> 1100, 1x32x1030
// 487 -> 524; d = 64 it lost (2 waves per SIMD, 194 VGPRs: C3 716 -> 696, 8x16x1025 602 -> 554;
// held to 3 with 16 VGPRs spilled: 437), and on causal d = 64 rows 9 % at 8x16x1024.
template <typename T, int D, int BM, int BN, int ST, typename OutT, int KS = 1, bool TC = false>
hipError_t launch_mfma(const void* q, const void* k, const void* v, void* o, int bh, int n, int causal,
                       hipStream_t stream) {
  const int qblocks = (n + BM - 1) / BM;
  const long long total = (long long)qblocks * bh;
  if (total > INT_MAX) return hipErrorInvalidConfiguration;
  constexpr bool kCheck = TC && ST == 2 && KS == 1 && std::is_same<T, pa::f16>::value;
  constexpr bool kCheckPerBlock = kCheck && D == 128;
  if constexpr (TC && ST == 2 && KS == 1) {
    {
      const PersistentPlan plan = persistent_grid_for<T, D, BM, BN, ST, OutT, KS>(n, bh, causal);
      if (plan.grid > 0) {
        // Non-causal with N a multiple of 2 * BN: an even number of full tiles. Otherwise (an
        // even tile count whose last tile is partial, or an odd count of full tiles, padded with
        // an empty one) the RAGGED form, whose wrap copies mask the keys past N.
        auto kernel = causal ? pa::fa_mfma_fwd<T, D, BM, BN, ST, OutT, KS, true, false, true>
                      : n % (2 * BN) == 0 ? pa::fa_mfma_fwd<T, D, BM, BN, ST, OutT, KS, true, false, false, kCheck>
                                          : pa::fa_mfma_fwd<T, D, BM, BN, ST, OutT, KS, true, true, false, kCheck>;
        hipLaunchKernelGGL(kernel, dim3((unsigned)plan.grid), dim3(BM / 32 * pa::kWave * KS), 0, stream,
                           static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                           static_cast<OutT*>(o), n, qblocks, (int)total, scale_log2_for(D), causal,
                           device_cus() / pa::kNumXcd, plan.walk);
        return hipGetLastError();
      }
    }
  }
  auto kernel = kCheckPerBlock && !causal ? pa::fa_mfma_fwd<T, D, BM, BN, ST, OutT, KS, false, false, false, kCheckPerBlock>
                                          : pa::fa_mfma_fwd<T, D, BM, BN, ST, OutT, KS>;
  hipLaunchKernelGGL(kernel, dim3((unsigned)total), dim3(BM / 32 * pa::kWave * KS), 0, stream,
                     static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                     static_cast<OutT*>(o), n, qblocks, (int)total, scale_log2_for(D), causal, 0, 0);
  return hipGetLastError();
}

typedef hipError_t (*mfma_fn)(const void*, const void*, const void*, void*, int, int, int, hipStream_t);

struct MfmaEntry {
  int dtype, out_dtype, d, br, bc, db, ks;
  mfma_fn fn;
  int64_t lds;
  bool tc;                 // fused_tc entry: may take the persistent launch
  PersistentPlan (*persistent_grid)(int64_t n, int64_t bh, int causal);   // its persistent launch (tc entries)
};

template <typename T> constexpr int dt_code();
template <> constexpr int dt_code<pa::f16>() { return PA_DTYPE_F16; }
template <> constexpr int dt_code<pa::bf16>() { return PA_DTYPE_BF16; }
template <> constexpr int dt_code<float>() { return PA_DTYPE_F32; }

template <typename T, int D, int BM, int BN, int ST, typename OutT, int KS, bool TC>
constexpr PersistentPlan (*persistent_grid_fn())(int64_t, int64_t, int) {
  if constexpr (TC && ST == 2 && KS == 1) return &persistent_grid_for<T, D, BM, BN, ST, OutT, KS>;
  else return nullptr;
}

template <typename T, int D, int BM, int BN, int ST, typename OutT, int KS = 1, bool TC = false>
constexpr MfmaEntry mfma_entry() {
  // LDS: the K/V stages, plus the O staging rows where the entry can take a persistent form.
  constexpr int64_t lds = (int64_t)pa::MfmaLds<D, BN, ST>::BYTES * KS +
                          (persistent_grid_fn<T, D, BM, BN, ST, OutT, KS, TC>() ? pa::MfmaOStage<D, BM, OutT>::BYTES : 0);
  return MfmaEntry{dt_code<T>(), dt_code<OutT>(), D, BM, BN, ST == 2 ? 1 : 0, KS, &launch_mfma<T, D, BM, BN, ST, OutT, KS, TC>,
                   lds, TC, persistent_grid_fn<T, D, BM, BN, ST, OutT, KS, TC>()};
}

#define PA_TC_BOTH_OUT(T, D, BM, BN, ST) mfma_entry<T, D, BM, BN, ST, T, 1, true>(), mfma_entry<T, D, BM, BN, ST, float, 1, true>()
#define PA_TUNED_BOTH_OUT(T, D, BM, BN, ST) mfma_entry<T, D, BM, BN, ST, T>(), mfma_entry<T, D, BM, BN, ST, float>()
#define PA_TC_SPLIT_BOTH_OUT(T, D, BM, BN) mfma_entry<T, D, BM, BN, 2, T, 2>(), mfma_entry<T, D, BM, BN, 2, float, 2>()

// fused_tc: one tile configuration per (dtype, d), chosen by measurement on MI355X. d = 128
// uses 8 waves (256 queries) per workgroup: one workgroup per CU, so each K/V tile is staged
// into LDS once per 256 queries instead of once per 128 (+3 % on C4); d = 64 keeps 4 waves,
// whose shorter rows leave the grid too few workgroups at 256.
const MfmaEntry kTcTable[] = {
    PA_TC_BOTH_OUT(pa::f16, 64, 128, 64, 2),
    PA_TC_BOTH_OUT(pa::bf16, 64, 128, 64, 2),
    PA_TC_BOTH_OUT(pa::f16, 128, 256, 64, 2),
    PA_TC_BOTH_OUT(pa::bf16, 128, 256, 64, 2),
};
// Small grids at d = 64: 64-query workgroups whose keys are split over two groups of 2 waves, so
// each wave walks half the tiles and the extra waves land on otherwise idle CUs; the groups merge
// at the end. Taken for rows of 2-4 key tiles with at most one such workgroup per CU (measured at
// BH = 42: N = 128 7.76 vs 8.44 us, N = 256 9.48 vs 10.16 us), and for rows of any length whose
// 128-query blocks fill at most half the CUs: back to back against the persistent launch, fp16,
// B*H x N from 1 x 512 to 32 x 512, 1 x 16384 and 2 x 8192, time ratio 0.85-0.92 non-causal and
// 0.79-0.83 causal. Causal rows of 4096 keys or more keep it up to one such block per CU (their
// blocks' lengths differ, so the longest one bounds the launch): 6x4096 0.92, 5x4096 (bf16) 0.94,
// 7x4096 0.92, 4x8192 0.86, 2x16384 1.00, 1x8x4096 0.83; between half and all of the CUs it lost
// non-causal (1.13-1.20) and tied or lost causal at shorter rows (28x1024 1.00, 1x16x2048 1.03).
// Slower with one tile or a grid that already fills the chip.
constexpr int kCUs = 256;   // MI355X / gfx950
const MfmaEntry kTcSplitTable[] = {
    PA_TC_SPLIT_BOTH_OUT(pa::f16, 64, 64, 64),
    PA_TC_SPLIT_BOTH_OUT(pa::bf16, 64, 64, 64),
};
bool use_key_split(int64_t d, int64_t n, int64_t bh, int causal) {
  if (d != 64 || n <= 64) return false;
  const int64_t blocks = (n + 127) / 128 * bh;
  return (n <= 256 && (n + 63) / 64 * bh <= kCUs) || blocks <= kCUs / 2 || (causal && n >= 4096 && blocks <= kCUs);
}
// d = 128 grids the 256-query blocks would leave partly idle: 128-query workgroups (4 waves, two
// per CU) where those blocks fill at most half the CUs (causal: at most all), so the work spreads
// over twice the CUs, and non-causal past one round where the last round is far from full. Every
// wave computes exactly as in the 256-query tile (same bits). Measured back to back against it,
// TFLOP/s, non-causal bf16: 1x8x1024 176 -> 234, 1x16x1024 356 -> 458, 1x32x1024 687 -> 813,
// 1x16x2048 833 -> 954, 1x4x4096 467 -> 629, 2x8x2048 813 -> 948, 1x2x8192 489 -> 654, 1x64x512
// 534 -> 652; causal: bf16 1x8x2048 203 -> 277, 1x16x1024 171 -> 222, 1x4x4096 227 -> 322, 1x8x1000
// 82 -> 109, fp16 1x2x8192 197 -> 284, 1x32x1024 290 -> 373. Causal rows keep it up to one such
// block per CU (bf16 12x4096 645 -> 828, 10x4096 550 -> 719, 28x2048 632 -> 704, 16x4096 763 ->
// 937, 2x16x2048 711 -> 716; fp16 14x4096 626 -> 733); non-causal between half and all of the CUs
// it lost (bf16 40x1024 795 -> 724, 48x1024 873 -> 801, 2x32x1024 1008 -> 957). Non-causal beyond
// one round of 256-query blocks it wins where the last round is far from full (rounds R, idle
// share of the launch 1 - R / ceil(R)): bf16 1x72x1024 (R 1.125) 724 -> 845, 1x20x4096 (1.25) 955
// -> 1078, 3x32x1024 (1.5) 883 -> 1005, 1x36x4096 (2.25) 1081 -> 1161, 1x18x8192 (2.25) 1104 ->
// 1180, 5x16x2048 (2.5) 1108 -> 1163, 1x80x2048 (2.5) 1119 -> 1171; fp16 1x24x4096 (1.5) 1055 ->
// 1100, 1x144x1024 (2.25) 822 -> 910; and loses where it is nearly full or full: 1x112x1024 (1.75)
// 1005 -> 950, 1x56x4096 (3.5) 1216 -> 1221, 2x32x2048 (2) 1128 -> 1068, C4 (8) 1290 -> 1195.
// Causal rows beyond one round lost with it (3x32x2048 970 -> 863, 1x40x4096 1070 -> 975). Where
// a row's last 256-query block is mostly padding, the 128-query tile computes fewer rows: non-causal
// bf16 past one round 4x256x128 263 -> 371, 1x512x384 659 -> 774, 2x128x896 976 -> 1033, fp16
// 2x256x640 833 -> 896; 1x256x1100 (11 % padding) 946 -> 946, 1x256x1536 (none) 1137 -> 1071;
// within one round 1x256x128 233 -> 270, 1x200x100 107 -> 127, but 1x100x384 500 -> 474 and
// 1x40x1100 754 -> 693.
const MfmaEntry kTcSmallGridTable[] = {
    PA_TC_BOTH_OUT(pa::f16, 128, 128, 64, 2),
    PA_TC_BOTH_OUT(pa::bf16, 128, 128, 64, 2),
};
bool use_small_grid_tile(int64_t d, int64_t n, int64_t bh, int causal) {
  if (d != 128) return false;
  const int64_t blocks = (n + 255) / 256 * bh;   // 256-query blocks, one workgroup per CU at a time
  if (causal) return blocks <= kCUs;
  if (blocks <= kCUs / 2) return true;
  // Rows of a head computed by each tile: a row's last block is padded to the tile (rows past N
  // are computed and not stored).
  const int64_t rows256 = (n + 255) / 256 * 256, rows128 = (n + 127) / 128 * 128;
  if (blocks <= kCUs) return n <= 128;   // one round: where half of every 256-query block is padding
  // More than one round of 256-query blocks: the 128-query tile where at least 14 % of the
  // 256-query tile's rows are padding, or where its last round would leave at least 15 % of the
  // launch's CU time idle (the half-size blocks fill that round's CUs better).
  if (100 * rows256 >= 114 * rows128) return true;
  const int64_t rounds = (blocks + kCUs - 1) / kCUs, last = blocks - (rounds - 1) * kCUs;
  return 100 * (kCUs - last) >= 15 * rounds * kCUs;
}

// fused_tuned: the reference's tile sweep set (fused_tuned.cuh:207) x {one, two} LDS stages.
#define PA_TUNED(BR, BC) PA_TUNED_BOTH_OUT(pa::f16, 64, BR, BC, 1), PA_TUNED_BOTH_OUT(pa::f16, 64, BR, BC, 2)
const MfmaEntry kTunedTable[] = {PA_TUNED(64, 32), PA_TUNED(64, 64), PA_TUNED(128, 32), PA_TUNED(128, 64)};

const MfmaEntry* find_tc(int dtype, int out_dtype, int64_t d, int64_t n, int64_t bh, int causal) {
  if (use_key_split(d, n, bh, causal))
    for (const auto& e : kTcSplitTable)
      if (e.dtype == dtype && e.out_dtype == out_dtype && e.d == d) return &e;
  if (use_small_grid_tile(d, n, bh, causal))
    for (const auto& e : kTcSmallGridTable)
      if (e.dtype == dtype && e.out_dtype == out_dtype && e.d == d) return &e;
  for (const auto& e : kTcTable)
    if (e.dtype == dtype && e.out_dtype == out_dtype && e.d == d) return &e;
  return nullptr;
}
const MfmaEntry* find_tuned(int dtype, int out_dtype, int64_t d, int br, int bc, int db) {
  for (const auto& e : kTunedTable)
    if (e.dtype == dtype && e.out_dtype == out_dtype && e.d == d && e.br == br && e.bc == bc && e.db == (db ? 1 : 0))
      return &e;
  return nullptr;
}

// ------------------------------------------------------------------ fused fp32 arithmetic
// 32 query rows per workgroup, keys split over kF32KS waves (merged through LDS at the end).
constexpr int kF32KS = 4;

template <typename T, typename OutT>
hipError_t launch_f32(const void* q, const void* k, const void* v, void* o, int bh, int n, int causal,
                      hipStream_t stream) {
  const int qblocks = (n + 31) / 32;
  const long long total = (long long)qblocks * bh;
  if (total > INT_MAX) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((pa::fa_f32_fwd<T, 64, kF32KS, OutT>), dim3((unsigned)total), dim3(kF32KS * pa::kWave),
                     0, stream, static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                     static_cast<OutT*>(o), n, qblocks, (int)total, scale_log2_for(64), causal);
  return hipGetLastError();
}

// ------------------------------------------------------------------ unfused
template <typename T>
hipError_t launch_naive(const void* q, const void* k, const void* v, void* o, float* s, int bh, int n, int d,
                        int causal, hipStream_t stream) {
  const float scale = 1.f / sqrtf((float)d);
  // Four waves per workgroup, one wave per (row, 64 columns); the heads in y.
  const long long key_blocks = (n + 63) / 64, dim_blocks = (d + 63) / 64;
  const long long score_units = (long long)n * key_blocks, pv_units = (long long)n * dim_blocks;
  const long long rows = (long long)n * bh;
  if (score_units > INT_MAX - 4 || pv_units > INT_MAX - 4 || (rows + 3) / 4 > INT_MAX)   // 32-bit unit indices
    return hipErrorInvalidConfiguration;
  // Rows of whole 16-byte pieces, 16-byte aligned: the scores read them a piece per load.
  const bool pieces = d * (int)sizeof(T) % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(k) % 16 == 0;
  auto scores = pieces ? pa::naive_scores<T, true> : pa::naive_scores<T, false>;
  hipLaunchKernelGGL(scores, dim3((unsigned)((score_units + 3) / 4), bh), dim3(256), 0, stream,
                     static_cast<const T*>(q), static_cast<const T*>(k), s, n, d, scale, causal, (int)key_blocks);
  hipLaunchKernelGGL(pa::naive_softmax, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, s, n, rows);
  auto pv = n % 4 == 0 && reinterpret_cast<uintptr_t>(s) % 16 == 0 ? pa::naive_pv<T, true> : pa::naive_pv<T, false>;
  hipLaunchKernelGGL(pv, dim3((unsigned)((pv_units + 3) / 4), bh), dim3(256), 0, stream, s,
                     static_cast<const T*>(v), static_cast<T*>(o), n, d, (int)dim_blocks);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_tiled(const void* q, const void* k, const void* v, void* o, float* s, int bh, int n, int d,
                        int causal, hipStream_t stream) {
  const float scale = 1.f / sqrtf((float)d);
  const int nt = (n + pa::kTile - 1) / pa::kTile;
  bool mfma_scores = false;
  if constexpr (std::is_same<T, pa::f16>::value) {
    // fp16 rows of 16 * {2, 4, 5, 6, 8} dims, 16-byte aligned, one head below 2 GiB.
    const bool aligned = reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0;
    const int nt128 = (n + 127) / 128;
    auto launch = [&](auto kernel) {
      hipLaunchKernelGGL(kernel, dim3(nt128, nt128, bh), dim3(256), 0, stream, static_cast<const pa::f16*>(q),
                         static_cast<const pa::f16*>(k), s, n, scale, causal);
      mfma_scores = true;
    };
    if (aligned && (int64_t)n * d * 2 < (1ll << 31)) {
      switch (d) {
        case 32: launch(pa::tiled_scores_mfma<2>); break;
        case 64: launch(pa::tiled_scores_mfma<4>); break;
        case 80: launch(pa::tiled_scores_mfma<5>); break;
        case 96: launch(pa::tiled_scores_mfma<6>); break;
        case 128: launch(pa::tiled_scores_mfma<8>); break;
        default: break;
      }
    }
  }
  if constexpr (std::is_same<T, float>::value) {
    // fp32 rows of 64 or 128 dims, 16-byte aligned, one head below 2 GiB.
    const bool aligned = reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0;
    if (aligned && (d == 64 || d == 128) && (int64_t)n * d * 4 < (1ll << 31)) {
      const int nt128 = (n + 127) / 128;
      hipLaunchKernelGGL(d == 64 ? pa::tiled_scores_mfma_f32<64> : pa::tiled_scores_mfma_f32<128>,
                         dim3(nt128, nt128, bh), dim3(256), 0, stream, static_cast<const float*>(q),
                         static_cast<const float*>(k), s, n, scale, causal);
      mfma_scores = true;
    }
  }
  if (!mfma_scores)
    hipLaunchKernelGGL(pa::tiled_scores<T>, dim3(nt, nt, bh), dim3(256), 0, stream, static_cast<const T*>(q),
                       static_cast<const T*>(k), s, n, d, scale, causal);
  const dim3 sm_grid((n + 3) / 4, bh);
  if (n <= 256) hipLaunchKernelGGL(pa::tiled_softmax_rows<4>, sm_grid, dim3(256), 0, stream, s, n);
  else if (n <= 1024) hipLaunchKernelGGL(pa::tiled_softmax_rows<16>, sm_grid, dim3(256), 0, stream, s, n);
  else if (n <= 2048) hipLaunchKernelGGL(pa::tiled_softmax_rows<32>, sm_grid, dim3(256), 0, stream, s, n);
  else if (n <= 4096) hipLaunchKernelGGL(pa::tiled_softmax_rows<64>, sm_grid, dim3(256), 0, stream, s, n);
  else if (n <= 8192) hipLaunchKernelGGL(pa::tiled_softmax_rows<128>, sm_grid, dim3(256), 0, stream, s, n);
  else if (n <= 16384) hipLaunchKernelGGL(pa::tiled_softmax_segments<64>, dim3(n, bh), dim3(256), 0, stream, s, n);
  else hipLaunchKernelGGL(pa::tiled_softmax_segments<128>, dim3(n, bh), dim3(256), 0, stream, s, n);
  bool mfma_pv = false;
  if constexpr (std::is_same<T, pa::f16>::value) {
    // fp16 V with d in {64, 128}, 16-byte aligned rows of P (N a multiple of 4) and V, one head's
    // P and V each below 2 GiB.
    const bool ok = (d == 64 || d == 128) && n % 4 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(s) % 16 == 0 && (int64_t)n * n * 4 < (1ll << 31) &&
                    (int64_t)n * d * 2 < (1ll << 31);
    if (ok) {
      auto kernel = d == 64 ? pa::tiled_pv_mfma<64> : pa::tiled_pv_mfma<128>;
      hipLaunchKernelGGL(kernel, dim3((n + 127) / 128, bh), dim3(256), 0, stream, s, static_cast<const pa::f16*>(v),
                         static_cast<pa::f16*>(o), n, causal);
      mfma_pv = true;
    }
  }
  if constexpr (std::is_same<T, float>::value) {
    const bool ok = (d == 64 || d == 128) && n % 4 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(s) % 16 == 0 && (int64_t)n * n * 4 < (1ll << 31) &&
                    (int64_t)n * d * 4 < (1ll << 31);
    if (ok) {
      hipLaunchKernelGGL(d == 64 ? pa::tiled_pv_mfma_f32<64> : pa::tiled_pv_mfma_f32<128>, dim3((n + 127) / 128, bh),
                         dim3(256), 0, stream, s, static_cast<const float*>(v), static_cast<float*>(o), n, causal);
      mfma_pv = true;
    }
  }
  if (!mfma_pv)
    hipLaunchKernelGGL(pa::tiled_pv<T>, dim3((d + pa::kTile - 1) / pa::kTile, nt, bh), dim3(256), 0, stream, s,
                       static_cast<const T*>(v), static_cast<T*>(o), n, d, causal);
  return hipGetLastError();
}

int unfused_common(const char* name, const void* q, const void* k, const void* v, void* o, int dtype, int64_t bh,
                   int64_t n, int64_t d) {
  if (int rc = check_common(name, q, k, v, o, bh, n, d)) return rc;
  if (dtype != PA_DTYPE_F32 && dtype != PA_DTYPE_F16)
    return fail(PA_ERR_UNSUPPORTED, "%s: only float32 and float16 are supported", name);
  if (bh > 65535) return fail(PA_ERR_UNSUPPORTED, "%s: B*H must be at most 65535", name);
  if ((n + 3) / 4 > 65535) return fail(PA_ERR_UNSUPPORTED, "%s: N must be at most 262140", name);
  return PA_OK;
}

// ------------------------------------------------------------------ tiled without allocation
// Score workspace of pa_tiled_fwd_noalloc: a fixed device array instead of a caller-allocated
// buffer. Every GPU the library runs on holds its own copy until the process ends. The tiled
// kernels write every score before reading it, so nothing needs clearing between calls.
constexpr int64_t kScratchFloats = 16ll << 20;   // 64 MiB: BH * N * N <= 16 Mi scores
static __device__ __align__(256) float scratch[kScratchFloats];

// Device address of this device's `scratch`, looked up once per device (the host-side name of a
// __device__ array is only a handle for the runtime, never a pointer to pass to a kernel).
std::mutex g_scratch_mu;
void* g_scratch_ptr[64];

int scratch_for_current_device(const char* name, float** out) {
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return hip_status(e, name);
  if (dev < 0 || dev >= 64) return fail(PA_ERR_UNSUPPORTED, "%s: device index %d out of range", name, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)); e != hipSuccess) return hip_status(e, name);
    if (!ptr) return fail(PA_ERR_INVALID, "%s: no device address for the scratch array", name);
    g_scratch_ptr[dev] = ptr;
  }
  *out = static_cast<float*>(g_scratch_ptr[dev]);
  return PA_OK;
}

// Per-device LDS limit, queried once per device.
std::mutex g_lds_mu;
int64_t g_lds_limit[64];
bool g_lds_known[64];

}  // namespace

extern "C" {

int pa_naive_fwd(const void* q, const void* k, const void* v, void* o, float* s, int dtype, int64_t bh, int64_t n,
                 int64_t d, int causal, void* stream) {
  const char* name = "naive_forward";
  if (int rc = unfused_common(name, q, k, v, o, dtype, bh, n, d)) return rc;
  if (!s) return fail(PA_ERR_INVALID, "%s: null score workspace", name);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = dtype == PA_DTYPE_F32 ? launch_naive<float>(q, k, v, o, s, (int)bh, (int)n, (int)d, causal, st)
                                       : launch_naive<pa::f16>(q, k, v, o, s, (int)bh, (int)n, (int)d, causal, st);
  return hip_status(e, name);
}

int pa_tiled_fwd(const void* q, const void* k, const void* v, void* o, float* s, int dtype, int64_t bh, int64_t n,
                 int64_t d, int causal, void* stream) {
  const char* name = "tiled_forward";
  if (int rc = unfused_common(name, q, k, v, o, dtype, bh, n, d)) return rc;
  if (!s) return fail(PA_ERR_INVALID, "%s: null score workspace", name);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = dtype == PA_DTYPE_F32 ? launch_tiled<float>(q, k, v, o, s, (int)bh, (int)n, (int)d, causal, st)
                                       : launch_tiled<pa::f16>(q, k, v, o, s, (int)bh, (int)n, (int)d, causal, st);
  return hip_status(e, name);
}

int pa_tiled_fwd_noalloc(const void* q, const void* k, const void* v, void* o, int dtype, int64_t bh, int64_t n,
                         int64_t d, int causal, void* stream) {
  const char* name = "tiled_forward_noalloc";
  if (int rc = unfused_common(name, q, k, v, o, dtype, bh, n, d)) return rc;
  if (n > kScratchFloats / bh / n)   // bh * n * n > kScratchFloats, without overflow
    return fail(PA_ERR_UNSUPPORTED,
                "%s: B*H*N*N = %.0f scores exceed the static scratch of %lld (use tiled_forward with a workspace)",
                name, (double)bh * (double)n * (double)n, (long long)kScratchFloats);
  float* s = nullptr;
  if (int rc = scratch_for_current_device(name, &s)) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = dtype == PA_DTYPE_F32 ? launch_tiled<float>(q, k, v, o, s, (int)bh, (int)n, (int)d, causal, st)
                                       : launch_tiled<pa::f16>(q, k, v, o, s, (int)bh, (int)n, (int)d, causal, st);
  return hip_status(e, name);
}

int pa_fused_fwd(const void* q, const void* k, const void* v, void* o, int dtype, int out_dtype, int64_t bh, int64_t n,
                 int64_t d, int causal, void* stream) {
  const char* name = "fused_forward";
  if (int rc = check_common(name, q, k, v, o, bh, n, d)) return rc;
  if (d != 64) return fail(PA_ERR_UNSUPPORTED, "%s: only head dimension 64 is compiled (got %lld)", name, (long long)d);
  if (int rc = check_aligned16(name, q, k, v, o)) return rc;
  if (int rc = check_head_bytes(name, n, d, dtype)) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (dtype == PA_DTYPE_F32 && out_dtype == PA_DTYPE_F32)
    e = launch_f32<float, float>(q, k, v, o, (int)bh, (int)n, causal, st);
  else if (dtype == PA_DTYPE_F16 && out_dtype == PA_DTYPE_F16)
    e = launch_f32<pa::f16, pa::f16>(q, k, v, o, (int)bh, (int)n, causal, st);
  else if (dtype == PA_DTYPE_F16 && out_dtype == PA_DTYPE_F32)
    e = launch_f32<pa::f16, float>(q, k, v, o, (int)bh, (int)n, causal, st);
  else
    return fail(PA_ERR_UNSUPPORTED, "%s: only float32 and float16 are supported", name);
  return hip_status(e, name);
}

int pa_fused_tuned_fwd(const void* q, const void* k, const void* v, void* o, int dtype, int out_dtype, int64_t bh,
                       int64_t n, int64_t d, int causal, int double_buffer, int br, int bc, void* stream) {
  const char* name = "fused_tuned";
  if (int rc = check_common(name, q, k, v, o, bh, n, d)) return rc;
  if (dtype != PA_DTYPE_F16) return fail(PA_ERR_UNSUPPORTED, "%s: float16 only", name);
  if (d != 64) return fail(PA_ERR_UNSUPPORTED, "%s: only head dimension 64 is compiled (got %lld)", name, (long long)d);
  if (int rc = check_aligned16(name, q, k, v, o)) return rc;
  if (int rc = check_head_bytes(name, n, d, dtype)) return rc;
  const MfmaEntry* e = find_tuned(dtype, out_dtype, d, br, bc, double_buffer);
  if (!e)
    return fail(PA_ERR_UNSUPPORTED,
                "%s: (br, bc) = (%d, %d) not compiled; available: (64,32) (64,64) (128,32) (128,64)", name, br, bc);
  return hip_status(e->fn(q, k, v, o, (int)bh, (int)n, causal, static_cast<hipStream_t>(stream)), name);
}

int pa_fused_tc_fwd(const void* q, const void* k, const void* v, void* o, int dtype, int out_dtype, int64_t bh,
                    int64_t n, int64_t d, int causal, void* stream) {
  const char* name = "fused_tc";
  if (int rc = check_common(name, q, k, v, o, bh, n, d)) return rc;
  if (dtype != PA_DTYPE_F16 && dtype != PA_DTYPE_BF16) return fail(PA_ERR_UNSUPPORTED, "%s: float16 or bfloat16 only", name);
  if (d != 64 && d != 128)
    return fail(PA_ERR_UNSUPPORTED, "%s: only head dimensions 64 and 128 are compiled (got %lld)", name, (long long)d);
  if (int rc = check_aligned16(name, q, k, v, o)) return rc;
  if (int rc = check_head_bytes(name, n, d, dtype)) return rc;
  const MfmaEntry* e = find_tc(dtype, out_dtype, d, n, bh, causal);
  if (!e) return fail(PA_ERR_UNSUPPORTED, "%s: output dtype must be the input dtype or float32", name);
  return hip_status(e->fn(q, k, v, o, (int)bh, (int)n, causal, static_cast<hipStream_t>(stream)), name);
}

const char* pa_fused_tc_kernel(int dtype, int out_dtype, int64_t bh, int64_t n, int64_t d, int causal) {
  thread_local char desc[256];
  const MfmaEntry* e = (bh > 0 && n > 0) ? find_tc(dtype, out_dtype, d, n, bh, causal) : nullptr;
  if (!e) return "";
  static const char* dt_name[] = {"f32", "f16", "bf16"};
  const long long total = (n + e->br - 1) / e->br * bh;
  const PersistentPlan plan = e->persistent_grid ? e->persistent_grid(n, bh, causal) : PersistentPlan{};
  const bool pers = plan.grid > 0;   // as in launch_mfma: no device (grid 0) means one workgroup per block
  const bool check = e->dtype == PA_DTYPE_F16 && e->tc && e->db && e->ks == 1 && !causal && (pers || e->d == 128);   // as in launch_mfma
  snprintf(desc, sizeof(desc), "fa_mfma_fwd<%s, D=%d, BM=%d, BN=%d, %d stages, out %s%s%s%s%s> grid %d x %d threads",
           dt_name[e->dtype], e->d, e->br, e->bc, e->db ? 2 : 1, dt_name[e->out_dtype],
           e->ks == 2 ? ", key split 2" : "", pers ? ", persistent" : "",
           !pers ? "" : !causal ? (n % (2 * e->bc) ? ", ragged" : "")
                      : plan.walk == 2 ? ", causal, device list" : plan.walk == 1 ? ", causal, by rank" : ", causal",
           check ? ", packed-max check" : "", pers ? plan.grid : (int)total, e->br / 32 * pa::kWave * e->ks);
  return desc;
}

int pa_set_persistent(int enable) {
  return g_persistent.exchange(enable ? 1 : 0, std::memory_order_relaxed);
}

int64_t pa_fused_tuned_lds_bytes(int br, int bc, int double_buffer, int64_t d, int dtype) {
  const MfmaEntry* e = find_tuned(dtype, dtype, d, br, bc, double_buffer);
  return e ? e->lds : -1;
}

int64_t pa_fused_tc_lds_bytes(int64_t d, int dtype) {
  // the larger of the general and the short-row (key-split) tile
  const MfmaEntry* e = find_tc(dtype, dtype, d, 1 << 20, 1024, 0);
  const MfmaEntry* s = find_tc(dtype, dtype, d, 128, 1, 0);
  if (!e) return -1;
  return s && s->lds > e->lds ? s->lds : e->lds;
}

int pa_device_lds_limit(int device, int64_t* bytes) {
  if (!bytes) return fail(PA_ERR_INVALID, "pa_device_lds_limit: null output pointer");
  if (device < 0 || device >= 64) return fail(PA_ERR_INVALID, "pa_device_lds_limit: bad device %d", device);
  std::lock_guard<std::mutex> lock(g_lds_mu);
  if (!g_lds_known[device]) {
    int v = 0;
    hipError_t e = hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, device);
    if (e != hipSuccess) return hip_status(e, "pa_device_lds_limit");
    g_lds_limit[device] = v;
    g_lds_known[device] = true;
  }
  *bytes = g_lds_limit[device];
  return PA_OK;
}

const char* pa_last_error(void) { return g_err; }

const char* pa_version(void) { return "phantom_attn " PA_VERSION_STRING " (gfx950)"; }

}  // extern "C"
