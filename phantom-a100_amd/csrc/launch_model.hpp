// Host-side model of the causal launches, used by the launcher to choose between them (and by
// a host-only test). Host code: it includes the kernels' shared helpers only for the walk and the
// block mapping the kernels themselves use (causal_walk_block, xcd_remap).
#pragma once

#include <algorithm>
#include <cstdint>
#include <mutex>
#include <vector>

#include "kernels/common.hpp"

namespace pa {

// Causal rows: which walk and which launch finish first, from a model in key tiles at one CU's
// rate, the rate of a CU being shared by the workgroups it holds. The persistent launch ends with
// its busiest CU (of XCD 0, which owns the most heads, for per-XCD lists): each CU's tiles summed
// over the blocks the walk (causal_walk_block) deals its workgroups. The per-block launch is
// simulated: its blocks in dispatch order (workgroup g to XCD g % 8, block xcd_remap(g)), each CU
// holding up to its occupancy of them, a freed slot taking the next block on the CU that holds
// fewest.
// The walk's list runs head by head or by length. Head by head, the serpentine passes pair every
// CU's long and short blocks only when the blocks per head tile the passes (4 to 64 blocks per head
// at 32 CUs per XCD); other counts leave some CU 1.4-2.2x above the mean. By length, the passes
// deal a sorted list and the busiest CU stays within ~10 % of the bound for any count. Measured on
// MI355X (TFLOP/s, head by head -> by length, bitwise equal): d = 128 where head by head balances,
// bf16 4x32x4096 1157 -> 1124, 2x16x8192 1236 -> 1233, 4x32x1024 836 -> 812 (the blocks at once
// on an XCD share fewer heads' K/V in its L2), and B*H = 100 N = 1024 720 -> 677 (equal busiest
// CUs); where it does not, bf16 4x32x1536 829 -> 938, 2x16x3072 783 -> 998, 1x32x6144 1041 -> 1150,
// 1x42x4096 938 -> 1015. At d = 64 (three workgroups per CU) by length was faster everywhere:
// fp16 8x16x1024 644 -> 682, 1x16x8192 840 -> 890, 8x16x1030 461 -> 584, 1x16x8000 696 -> 884,
// 4x16x1536 572 -> 732, 2x16x3072 602 -> 792, 1x16x6144 694 -> 823. So d = 64 walks by length, and
// d = 128 by length only where the model's busiest CU is lower that way. Where per-XCD lists are
// not allowed (few heads, or heads uneven over the XCDs) one list over the device, by length, is
// modelled on all CUs; against the per-block launch it measured, TFLOP/s, bf16 d = 128 B*H x N =
// 1x65536 661 -> 881, 4x16384 807 -> 862, 12x4096 607 -> 653, 42x1024 411 -> 433, fp16 d = 64
// 4x16384 606 -> 681, 10x8192 500 -> 733, 42x2048 441 -> 651. The per-block launch is simulated on
// every XCD, since with few heads `xcd_remap` gives one XCD the longest eighth of a head.
// The persistent launch is then taken while the model's per-block time is at least 0.85 of the
// persistent one: the measured per-block / persistent time ratio ran at the model's times 0.9-1.25
// (the persistent launch also hides each block's start); e.g. head by head, model -> measured,
// bf16 d = 128 B*H = 32 N = 3072 0.71 -> 0.87, B*H = 128 N = 768 0.83 -> 1.00, B*H = 128 N = 1000
// 1.40 -> 1.33, fp16 d = 64 B*H = 128 N = 1030 0.73 -> 0.92, B*H = 81 N = 2048 1.35 -> 1.28. The
// model runs once per shape (cached); beyond 64 blocks per CU, where a pass's pattern averages out
// over many passes, the persistent launch is taken without it.
inline long long causal_block_tiles(long long qb, int64_t n, int bm, int bn) {
  const long long t = (std::min<long long>(n, (qb + 1) * bm) + bn - 1) / bn;
  return t + (t & 1);   // padded to even, as the kernel pads it
}

// Key tiles of the busiest CU under the walk of list 0 of `lists` (XCD 0 of the per-XCD lists,
// the most heads; or the device's one list), wgs workgroups over cus CUs.
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

// When the per-block launch's last block on XCD x ends (its cus CUs, `slots` blocks per CU).
inline double per_block_makespan(int64_t n, int64_t bh, int bm, int bn, int slots, int cus, int x) {
  const long long nq = (n + bm - 1) / bm, total = nq * bh;
  std::vector<double> done((size_t)cus, 0.0);          // work each resident block of a CU has had
  std::vector<std::vector<double>> ends((size_t)cus);  // `done` at which each resident block ends
  double now = 0.0;
  long long g = x;   // next workgroup id of XCD x
  while (true) {
    while (g < total) {
      size_t cu = 0;
      for (size_t c = 1; c < ends.size(); ++c)
        if (ends[c].size() < ends[cu].size()) cu = c;
      if ((int)ends[cu].size() >= slots) break;
      const long long blk = xcd_remap((int)g, (int)total);
      ends[cu].push_back(done[cu] + (double)causal_block_tiles(nq - 1 - blk % nq, n, bm, bn));
      g += kNumXcd;
    }
    double dt = 0.0;
    bool any = false;
    for (size_t c = 0; c < ends.size(); ++c) {
      if (ends[c].empty()) continue;
      const double left = (*std::min_element(ends[c].begin(), ends[c].end()) - done[c]) * (double)ends[c].size();
      if (!any || left < dt) dt = left;
      any = true;
    }
    if (!any) break;
    now += dt;
    for (size_t c = 0; c < ends.size(); ++c) {
      if (ends[c].empty()) continue;
      done[c] += dt / (double)ends[c].size();
      const double at = done[c] + 1e-9 * (1.0 + done[c]);
      ends[c].erase(std::remove_if(ends[c].begin(), ends[c].end(), [&](double e) { return e <= at; }), ends[c].end());
    }
  }
  return now;
}

// The launch and walk for causal rows: walk 0 (per-XCD lists head by head), 1 (per-XCD lists by
// length) or 2 (one list over the device by length). wgs: workgroups per XCD of the persistent
// launch, slots: blocks per CU of the per-block launch, cus: CUs per XCD. per_xcd: whether the
// per-XCD lists may be used (the launcher's heads rule); rank_only: no head-by-head lists. The
// device list is taken over the per-XCD ones only where its busiest CU is 5 % lower (its blocks
// of a head run on every XCD, so they share less K/V in L2).
struct CausalChoice {
  bool persistent = false;
  int walk = 0;
};
inline CausalChoice causal_choice(int64_t n, int64_t bh, int bm, int bn, int wgs, int slots, int cus, bool rank_only,
                                  bool per_xcd) {
  if (wgs <= 0 || slots <= 0 || cus <= 0) return {};
  const long long nq = (n + bm - 1) / bm, heads = (bh + kNumXcd - 1) / kNumXcd;
  if (per_xcd && heads * nq > 64LL * cus) return {true, rank_only ? 1 : 0};
  if (!per_xcd && bh * nq > 64LL * cus * kNumXcd) return {true, 2};
  struct Entry {
    int64_t n = -1, bh = -1;
    int bm = 0, wgs = 0, slots = 0, cus = 0;
    bool rank_only = false, per_xcd = false;
    CausalChoice choice;
  };
  static std::mutex mu;
  static Entry cache[64];
  Entry& e = cache[(size_t)((uint64_t)(n * 1000003 + bh * 131 + bm + wgs) % 64)];
  {
    std::lock_guard<std::mutex> lock(mu);
    if (e.n == n && e.bh == bh && e.bm == bm && e.wgs == wgs && e.slots == slots && e.cus == cus &&
        e.rank_only == rank_only && e.per_xcd == per_xcd)
      return e.choice;
  }
  CausalChoice choice;
  double best = 0.0;
  if (per_xcd) {
    const long long by_rank = causal_walk_busiest(n, bh, bm, bn, wgs, cus, 1, kNumXcd);
    const long long by_head = rank_only ? by_rank + 1 : causal_walk_busiest(n, bh, bm, bn, wgs, cus, 0, kNumXcd);
    choice.walk = by_rank < by_head ? 1 : 0;
    best = (double)std::min(by_rank, by_head);
  }
  const double device = (double)causal_walk_busiest(n, bh, bm, bn, wgs * kNumXcd, cus * kNumXcd, 1, 1);
  if (!per_xcd || device < 0.95 * best) {
    choice.walk = 2;
    best = device;
  }
  double per_block = 0.0;
  for (int x = 0; x < kNumXcd; ++x) per_block = std::max(per_block, per_block_makespan(n, bh, bm, bn, slots, cus, x));
  choice.persistent = per_block >= 0.85 * best;
  std::lock_guard<std::mutex> lock(mu);
  e.n = n; e.bh = bh; e.bm = bm; e.wgs = wgs; e.slots = slots; e.cus = cus; e.rank_only = rank_only;
  e.per_xcd = per_xcd;
  e.choice = choice;
  return choice;
}

}  // namespace pa
