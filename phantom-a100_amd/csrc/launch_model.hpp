// The causal launch's walk, chosen on the host (and checked by a host-only test). Host code: it
// includes the kernels' shared helpers only for the walk the kernels themselves take
// (causal_walk_block).
#pragma once

#include <algorithm>
#include <cstdint>
#include <mutex>
#include <vector>

#include "kernels/common.hpp"

namespace pa {

// Causal rows take the persistent form with one of three walks (kernel argument `walk`): per-XCD
// lists head by head (0), per-XCD lists by length (1), or one list over the device by length (2).
// Head by head, the serpentine passes pair every CU's long and short blocks only when the blocks per
// head tile the passes (4 to 64 blocks per head at 32 CUs per XCD); other counts leave some CU
// 1.4-2.2x above the mean. By length, the passes deal a sorted list and the busiest CU stays within
// ~10 % of the bound for any count, but the blocks running at once on an XCD come from more heads
// and share less K/V in its L2. Measured on MI355X (TFLOP/s, head by head -> by length, bitwise
// equal): d = 128 where head by head balances, bf16 4x32x4096 1157 -> 1124, 2x16x8192 1236 -> 1233,
// 4x32x1024 836 -> 812, and B*H = 100 N = 1024 720 -> 677 (equal busiest CUs); where it does not,
// bf16 4x32x1536 829 -> 938, 2x16x3072 783 -> 998, 1x32x6144 1041 -> 1150, 1x42x4096 938 -> 1015. At
// d = 64 (three workgroups per CU) by length was faster everywhere: fp16 8x16x1024 644 -> 682,
// 1x16x8192 840 -> 890, 8x16x1030 461 -> 584, 1x16x8000 696 -> 884, 4x16x1536 572 -> 732,
// 2x16x3072 602 -> 792, 1x16x6144 694 -> 823. So d = 64 walks by length, and d = 128 by length only
// where its busiest CU (key tiles summed over the blocks dealt to each CU of XCD 0, which owns the
// most heads) is lower than head by head. Where per-XCD lists are not allowed (few heads, or heads
// uneven over the XCDs) the walk takes one list over the device.
//
// Against one workgroup per query block, the persistent form with these walks was faster in every
// causal shape measured (per block -> persistent, TFLOP/s): bf16 d = 128 4x32x4096 972 -> 1124,
// 2x16x8192 1129 -> 1196, 4x32x768 479 -> 639, 2x16x3072 781 -> 980, 1x100x1024 492 -> 685,
// 1x1x65536 661 -> 881, 4x16384 (B*H x N) 807 -> 862, 42x1024 411 -> 433; fp16 d = 64 8x16x1024
// 472 -> 658, 8x16x1030 452 -> 571, 1x16x8000 690 -> 865, 10x8192 500 -> 733; bf16 d = 64 4x16x4096
// 759 -> 910. (A model of the per-block launch, a processor-sharing simulation of its dispatch,
// agreed within its error; it decided nothing once the walks by length existed, and simulating on
// every new shape cost about as much as a short launch, so it is not run.)

// Key tiles a causal query block qb walks: its keys up to min(N, its last row + 1), the count
// padded to even, as the kernel pads it.
inline long long causal_block_tiles(long long qb, int64_t n, int bm, int bn) {
  const long long t = (std::min<long long>(n, (qb + 1) * bm) + bn - 1) / bn;
  return t + (t & 1);
}

// Key tiles of the busiest CU under the walk of list 0 of `lists` (XCD 0 of the per-XCD lists,
// the most heads; or the device's one list), wgs workgroups over cus CUs. One step per block of
// the list.
inline long long causal_walk_busiest(int64_t n, int64_t bh, int bm, int bn, int wgs, int cus, int by_rank, int lists) {
  const int nq = (int)((n + bm - 1) / bm);
  std::vector<long long> load((size_t)cus, 0);
  for (int c = 0; c < wgs; ++c) {
    for (int j = 0;; ++j) {
      const int blk = causal_walk_block(j, c, 0, wgs, cus, (int)bh, nq, by_rank, lists);
      if (blk < 0) break;
      load[(size_t)(c % cus)] += causal_block_tiles(blk % nq, n, bm, bn);
    }
  }
  return *std::max_element(load.begin(), load.end());
}

// Per-XCD lists by length (1) or head by head (0), whichever leaves XCD 0's busiest CU fewer tiles.
inline int causal_walk_uncached(int64_t n, int64_t bh, int bm, int bn, int wgs, int cus) {
  return causal_walk_busiest(n, bh, bm, bn, wgs, cus, 1, kNumXcd) < causal_walk_busiest(n, bh, bm, bn, wgs, cus, 0, kNumXcd)
             ? 1
             : 0;
}

// The last shapes whose walk was counted (the count walks up to 64 list entries per CU and costs
// up to ~75 us on the host; a serving loop repeats few shapes). A small ring under a mutex.
struct CausalWalkCache {
  struct Entry {
    int64_t n = -1, bh = -1;
    int bm = 0, bn = 0, wgs = 0, cus = 0, walk = 0;
  };
  static constexpr int kSlots = 16;
  std::mutex mu;
  Entry slot[kSlots];
  int next = 0;
};
inline CausalWalkCache& causal_walk_cache() {
  static CausalWalkCache cache;
  return cache;
}

// The walk for causal rows. wgs: workgroups per XCD of the persistent launch, cus: CUs per XCD.
// per_xcd: whether the per-XCD lists may be used (the launcher's heads rule); rank_only: no
// head-by-head lists (d = 64). Beyond 64 blocks per CU, where a pass's pattern averages out over
// many passes, head by head is kept without counting.
inline int causal_walk(int64_t n, int64_t bh, int bm, int bn, int wgs, int cus, bool rank_only, bool per_xcd) {
  if (!per_xcd) return 2;
  if (rank_only) return 1;
  const long long nq = (n + bm - 1) / bm, heads = (bh + kNumXcd - 1) / kNumXcd;
  if (wgs <= 0 || cus <= 0 || heads * nq > 64LL * cus) return 0;
  CausalWalkCache& c = causal_walk_cache();
  {
    std::lock_guard<std::mutex> lock(c.mu);
    for (const auto& e : c.slot)
      if (e.n == n && e.bh == bh && e.bm == bm && e.bn == bn && e.wgs == wgs && e.cus == cus) return e.walk;
  }
  const int walk = causal_walk_uncached(n, bh, bm, bn, wgs, cus);   // counted outside the lock
  std::lock_guard<std::mutex> lock(c.mu);
  c.slot[c.next] = CausalWalkCache::Entry{n, bh, bm, bn, wgs, cus, walk};
  c.next = (c.next + 1) % CausalWalkCache::kSlots;
  return walk;
}

}  // namespace pa
