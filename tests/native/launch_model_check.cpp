// Host-only checks of the causal walk and of the launch model (phantom-a100_amd/csrc/launch_model.hpp),
// compiled and run by tests/test_launch_model.py on the CPU. Exit status 0 when every check holds;
// each failure prints one line starting with FAIL.
//
// 1. The walk (causal_walk_block, the function the causal persistent kernel calls) hands every
//    query block to exactly one workgroup: with per-XCD lists on the XCD that owns the block's
//    head, for both list orders, and with one list over the device; for both dealing branches
//    (workgroups filling whole slots of the CUs, or not) and grids of one to three workgroups per
//    CU, as the launcher sizes them.
// 2. The busiest CU's key tiles under each per-XCD walk, for whole-head shapes, against an
//    independent restatement, and the walk the launcher then takes.
// 3. The walk cache: a second call agrees, evicted entries are counted afresh, and eight threads
//    reading and replacing entries at once all get the uncached answer (the test also builds this
//    file with ThreadSanitizer on the host code where the toolchain has its runtime).
#include <atomic>
#include <cstdio>
#include <thread>
#include <vector>

#include "launch_model.hpp"

static int failures = 0;
#define CHECK(cond, ...)                    \
  do {                                      \
    if (!(cond)) {                          \
      ++failures;                           \
      std::printf("FAIL: " __VA_ARGS__);    \
      std::printf("\n");                    \
    }                                       \
  } while (0)

// walk: 0 / 1 per-XCD lists head by head / by length, 2 one list over the device (by length).
static void check_walk(int bh, int nq, int wpc, int cus, int walk) {
  const long long total = (long long)bh * nq;
  const int per_xcd = (int)((total + pa::kNumXcd - 1) / pa::kNumXcd);
  const int wgs = std::min(std::max(cus, 32) * wpc, per_xcd);   // the launcher's grid per XCD
  std::vector<int> seen((size_t)total, 0);
  for (int x = 0; x < pa::kNumXcd; ++x)
    for (int c = 0; c < wgs; ++c)
      for (int j = 0;; ++j) {
        const int g = c * pa::kNumXcd + x;   // the workgroup id; the kernel's XCD is g % 8
        const int blk = walk == 2 ? pa::causal_walk_block(j, g, 0, wgs * pa::kNumXcd, cus * pa::kNumXcd, bh, nq, 1, 1)
                                  : pa::causal_walk_block(j, c, x, wgs, cus, bh, nq, walk, pa::kNumXcd);
        if (blk < 0) break;
        if (blk >= total) {
          CHECK(false, "bh=%d nq=%d wgs=%d cus=%d walk=%d: block %d out of range", bh, nq, wgs, cus, walk, blk);
          break;
        }
        CHECK(walk == 2 || (blk / nq) % pa::kNumXcd == x, "bh=%d nq=%d walk=%d: block %d on XCD %d", bh, nq, walk, blk, x);
        ++seen[(size_t)blk];
      }
  int missing = 0, repeated = 0;
  for (int s : seen) {
    missing += s == 0;
    repeated += s > 1;
  }
  CHECK(missing == 0 && repeated == 0, "bh=%d nq=%d wgs=%d cus=%d walk=%d: %d blocks missing, %d repeated", bh, nq,
        wgs, cus, walk, missing, repeated);
}

int main() {
  int walks = 0;
  for (int bh : {1, 2, 3, 5, 7, 8, 9, 12, 13, 16, 20, 42, 63, 64, 100, 128})
    for (int nq : {1, 2, 3, 4, 5, 8, 9, 12, 16, 24, 63, 64})
      for (int wpc : {1, 2, 3})
        for (int cus : {32, 0})
          for (int walk : {0, 1, 2}) {
            check_walk(bh, nq, wpc, cus, walk);
            ++walks;
          }
  std::printf("walks checked: %d\n", walks);

  struct Case {
    int bh, n, d, slots;
    long long by_head, by_rank;
    int walk;
  };
  // Figures of the independent restatement; the walk follows from them (d = 64 by length, d = 128
  // by length only where its busiest CU is lower).
  const Case cases[] = {
      {128, 4096, 128, 1, 272, 272, 0},
      {32, 3072, 128, 1, 84, 48, 1},
      {128, 768, 128, 1, 24, 12, 1},
      {128, 1030, 64, 3, 82, 46, 1},
      {16, 8000, 64, 3, 376, 252, 1},
      {64, 4096, 64, 3, 264, 264, 1},
  };
  for (const Case& k : cases) {
    const int bm = k.d == 128 ? 256 : 128, bn = 64, cus = 32;
    const long long total = (long long)(k.n + bm - 1) / bm * k.bh;
    const int wgs = (int)std::min<long long>((long long)cus * k.slots, (total + 7) / 8);
    const long long h = pa::causal_walk_busiest(k.n, k.bh, bm, bn, wgs, cus, 0, pa::kNumXcd);
    const long long r = pa::causal_walk_busiest(k.n, k.bh, bm, bn, wgs, cus, 1, pa::kNumXcd);
    const int walk = pa::causal_walk(k.n, k.bh, bm, bn, wgs, cus, k.d == 64, true);
    std::printf("B*H=%d N=%d d=%d: busiest CU head by head %lld, by length %lld -> walk %d\n", k.bh, k.n, k.d, h, r, walk);
    CHECK(h == k.by_head && r == k.by_rank, "B*H=%d N=%d d=%d: busiest %lld / %lld, expected %lld / %lld", k.bh, k.n,
          k.d, h, r, k.by_head, k.by_rank);
    CHECK(walk == k.walk, "B*H=%d N=%d d=%d: walk %d, expected %d", k.bh, k.n, k.d, walk, k.walk);
    // The second call of a shape comes from the walk cache and must agree.
    CHECK(pa::causal_walk(k.n, k.bh, bm, bn, wgs, cus, k.d == 64, true) == walk, "B*H=%d N=%d: cached walk differs",
          k.bh, k.n);
  }
  // More shapes than the cache holds, then the first again: evicted entries are counted afresh.
  for (int i = 0; i < 40; ++i) {
    const int n = 1024 + 64 * i, wgs = 32;
    const int want = pa::causal_walk_uncached(n, 128, 256, 64, wgs, 32);
    CHECK(pa::causal_walk(n, 128, 256, 64, wgs, 32, false, true) == want, "N=%d: walk differs from the count", n);
    CHECK(pa::causal_walk(n, 128, 256, 64, wgs, 32, false, true) == want, "N=%d: cached walk differs", n);
  }
  // Heads the per-XCD lists may not take walk one list over the device.
  CHECK(pa::causal_walk(16384, 4, 256, 64, 8, 32, false, false) == 2, "B*H=4: walk not the device list");
  // Eight threads asking for 48 shapes at once (three times what the cache holds, so entries are
  // evicted while others are read): every answer equals the uncached count.
  {
    std::vector<int> want(48);
    for (int i = 0; i < 48; ++i) want[i] = pa::causal_walk_uncached(2048 + 64 * i, 96, 256, 64, 32, 32);
    std::atomic<int> wrong{0};
    std::vector<std::thread> pool;
    for (int t = 0; t < 8; ++t)
      pool.emplace_back([&, t] {
        for (int r = 0; r < 20; ++r)
          for (int i = 0; i < 48; ++i) {
            const int j = (i * 7 + t * 5 + r) % 48;
            if (pa::causal_walk(2048 + 64 * j, 96, 256, 64, 32, 32, false, true) != want[j]) ++wrong;
          }
      });
    for (auto& th : pool) th.join();
    CHECK(wrong.load() == 0, "threads: %d cached walks differ from the count", wrong.load());
  }
  std::printf("%s\n", failures ? "FAILED" : "ok");
  return failures ? 1 : 0;
}
