// Fused online-softmax attention forward on CDNA4 MFMA (fp16 / bf16 in, fp32 accumulate).
//
// Computes O = softmax(Q K^T / sqrt(d)) V for one (head, BM-query block) per workgroup without
// materialising the N x N scores. Same math as the reference's v4 kernel
// (/root/reference/csrc/kernels/fused_tc.cuh:45-179): scores scaled by log2(e)/sqrt(d) in fp32,
// a reference max m and sum l per query row, alpha = 2^(m_old - m_new), P = 2^(S c - m) rounded
// to the input dtype as the P.V operand, output O / l. Two deliberate differences, both exact
// in real arithmetic (O / l does not depend on which m is used, as long as numerator and
// denominator use the same one):
//  * l sums the rounded P, the values the P.V MFMAs multiply, so the normalisation is
//    consistent with the numerator (the reference sums the unrounded P). On a row dominated by
//    one key the rounding of that key's P then cancels in O / l.
//  * Lazy rescale: m is raised (and O, l multiplied by alpha) only when some row of the wave
//    would exceed it by more than 2^8 (2^18 under the fp16 packed-max check, CHECK); otherwise
//    the stale m is kept and P <= 2^8 (2^18). The reference rescales at every tile.
//
// gfx950 design (not a translation of the WMMA kernel):
//  * Each wave owns 32 query rows. Both products are computed transposed so that every
//    per-row quantity stays in one lane:
//        S^T (keys x queries) = K . Q^T        v_mfma_f32_32x32x16_{f16,bf16}, A = K from LDS,
//                                              B = Q^T resident in VGPRs for the whole kernel
//        O^T (d x queries)   += V^T . P^T      A = V^T read from LDS with ds_read_b64_tr_b16,
//                                              B = P^T taken straight from the S^T accumulator
//    In the 32x32 accumulator, lane l holds column l%32 (= one query) and 16 of its 32 rows
//    (keys, or head dims); the other 16 sit in lane l^32. So a row max is a 16-element in-lane
//    reduction plus one v_permlane32_swap, the rescale of O is lane-local,
//    and P^T needs no LDS round trip: register r of the S^T block holds key
//    8*(r/4) + 4*(l/32) + r%4, exactly the key that the PV MFMA's B operand expects in k-slot
//    8*(l/32) + (r%8) once the A operand (V^T) is read in the same key order.
//  * The row sum l of the rounded P also runs on the matrix core: one 16x16x32 MFMA per 16-key
//    step multiplies a constant 0/1 operand by the P^T operand, which leaves every lane with the
//    sum of its own query. It replaces 16 v_dot2 per tile, which cost 4-5 % of the kernel's
//    time on the VALU; the extra MFMAs cost most of that back (net, measured: C3 +1.1 %,
//    C4 +1.2 %, C5 +1.5 %).
//  * K and V tiles of BN keys go HBM -> LDS with buffer_load ... lds (16 bytes per lane, no
//    VGPR staging; rows past N arrive as zeros). One such load writes 1 KB of LDS contiguously,
//    so rows are unpadded and 16-byte chunks are XOR-swizzled per row instead: the K operand
//    reads (ds_read_b128, 16 consecutive rows at one column) and the transposed V reads
//    (4 rows x 4 chunks per 32 lanes) each touch all 64 banks once.
//  * STAGES == 2 (default): software pipeline inside each wave. For fp16 (causal rows, key split
//    and the fused_tuned tiles), iteration t runs
//        phase A: MFMAs of S(t+1) = K(t+1).Q^T   interleaved with the VALU work that turns S(t)
//                                                 into P(t) (exp2, rounding; at d = 64 only its
//                                                 second half)
//        phase B: MFMAs of O += V(t)^T.P(t)^T    interleaved with the row sum of P(t), the row
//                                                 max of S(t+1) and, at d = 64, the first half
//                                                 of P(t+1)
//    For bf16, and for the fp16 fused_tc tiles on non-causal rows (CHECK), the row max leaves the
//    fast path: P is computed against the stale reference max and checked afterwards, bf16 for
//    overflow past 2^8 with one OR over its packed patterns, fp16 for reaching 2^14 with a packed
//    max (see the branch below), and the exponentials are split evenly over the two phases (the second
//    half of P(t) in phase A, the first half of P(t+1) in phase B), so each MFMA phase carries
//    about the same VALU work.
//    The interleave is fixed with scheduling-group barriers on a branch-free fast path (tile
//    t+1 needs no mask); masked tiles (the N tail, causal diagonal) take a generic path. K and
//    V have their own two-stage LDS rings (K is consumed one tile ahead of V); the loads of
//    K(t+2) and V(t+1) fly during iteration t; one barrier per tile.
//  * O and l are rescaled only in tiles where some row's max outgrew the reference max by
//    more than 2^8, or 2^18 under CHECK (a wave-uniform branch, rare after the first tile); on
//    the fp16 row-max fast path the rescale runs inside phase A, whose QK MFMAs do not touch O.
//  * KSPLIT == 2 (short rows on a small grid): the workgroup's waves form two key groups; group
//    g walks the key tiles g, g + 2, ... through its own half of every LDS stage, with its own
//    (m, l, O), so each wave walks half the tiles. At the end group 1 hands (m, l, O) to the
//    lane of group 0 holding the same query and dims, through the freed stages, and group 0
//    merges them with the online-softmax rule and stores.
//  * STAGES == 1: no prefetch (the reference's v3.1 structure): load tile, wait, compute.
//  * Workgroup ids are remapped so that all query blocks of a head run on one XCD (shared L2).
//  * PERSIST (two stages, no key split; launched for non-causal rows with an even tile count or
//    an odd count of full tiles): as many workgroups as fit at once walk the query blocks of
//    their XCD's range. The last two
//    iterations of a block are separate copies of the iteration (compile-time WRAP) whose loads
//    past the block's last tile fetch the next block's K(0), K(1), V(0) and Q, so a block starts
//    with its first tiles already in LDS and the per-block start-up (workgroup launch, first
//    loads) is hidden behind the previous block. When every tile is full (N a multiple of
//    2 * BN, RAGGED = false) the mask code is compiled out and all but a block's last iteration
//    take the fast path without a runtime test. RAGGED: the same walk for an even tile count
//    whose last tile is partial, or an odd count of full tiles padded with one empty tile; both
//    wrap iterations then take the generic path and mask the tiles past N.
//  * CAUSAL (the persistent form for causal rows; XCD x owns the heads x, x + 8, ...): a block
//    of query rows [q0, q0 + BM) sees its c = q0 / BN first key tiles unmasked in every wave, and
//    then BM / BN diagonal tiles, of which wave w needs the first w / 2 + 1 (the last one masked).
//    When N is not a multiple of BM, a head's last block holds the tiles up to N, padded to an
//    even count; its waves need the tiles up to min(N, their last row + 1). The c clean tiles run the clean persistent iterations; the diagonal tiles (with
//    the two before them) run copies (DIAG) in which each wave takes the fast path up to its last
//    tile and idles after it, the fast path masking S(t+1) when t+1 is the wave's diagonal tile;
//    only the block's very last tile (the last wrap copy) takes the generic path. An XCD's blocks
//    are listed head by head (longest first within a head; the blocks running at once then share
//    the K/V of few heads in its L2) or by length across its heads, or the device's blocks by
//    length in one list (for few heads), and dealt to the CUs in serpentine passes, so that a CU
//    that gets one pass's long block gets the next pass's short one (causal_walk_block in
//    common.hpp; the launcher picks the list).
//  * The persistent forms stage each wave's block of O in LDS and store it as whole rows with
//    non-temporal stores (store_block), so few dirty O lines are left for the end of the launch.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace pa {

template <int D, int BN, int STAGES>
struct MfmaLds {
  static constexpr int ROW_BYTES = D * 2;
  static constexpr int TILE_BYTES = BN * ROW_BYTES;
  static constexpr int BYTES = STAGES * 2 * TILE_BYTES;   // K stages then V stages
};

// The persistent forms' O staging rows: each wave stages its 32 rows of O in ROWS-row passes that
// fit LIMIT bytes per workgroup (three d = 64 workgroups per CU: 3 x (32 + 16) KB; one 256-query
// d = 128 workgroup: 64 + 64 KB; two 128-query d = 128 workgroups: 2 x (64 + 16) KB), so BYTES of
// LDS per workgroup beside the K/V stages.
template <int D, int BM, typename OutT>
struct MfmaOStage {
  static constexpr int ROW = D * (int)sizeof(OutT);       // bytes of one O row
  static constexpr int CHUNKS = ROW / 16;                  // its 16-byte chunks
  static constexpr int LIMIT = (D == 64 || BM < 256) ? 16384 : 65536;
  static constexpr int PASSES = (BM * ROW + LIMIT - 1) / LIMIT;
  static constexpr int ROWS = 32 / PASSES;                 // rows of a wave per pass
  static constexpr int BYTES = BM / 32 * ROWS * ROW;
};

// XOR swizzle of the 16-byte chunk index within a row (CR chunks per row).
// K: consecutive rows r..r+15 read at one logical chunk land in 16 distinct bank groups.
// V: rows r..r+3 (r % 4 == 0) x chunks 4q..4q+3 land in 16 distinct bank groups.
template <int CR> __device__ __forceinline__ int k_swz(int row) { return CR == 16 ? (row & 15) : ((row >> 1) & 7); }
template <int CR> __device__ __forceinline__ int v_swz(int row) { return CR == 16 ? 4 * (row & 3) : 4 * ((row >> 1) & 1); }

// Minimum waves per SIMD the register allocator must allow (1: no constraint; PA_MFMA_MIN_WAVES
// overrides it for every instantiation). Three 4-wave d = 64 workgroups per CU need at most 168
// VGPRs: the fp16 causal persistent form takes 169 unconstrained, the bf16 non-causal persistent
// forms 169-171 (held to 168 they spill 1-2 VGPRs and still run 3.5-6 % faster), the bf16 causal
// form 193 (held to 168 it spills 10 VGPRs and runs 4-26 % faster: B*H x N = 256 x 512 404 -> 422,
// 128 x 1024 516 -> 584, 128 x 2048 641 -> 794, 64 x 4096 692 -> 873, 16 x 8192 713 -> 887
// TFLOP/s); the fp16 persistent forms with the packed-max check (CHECK) take 169-171 and are held
// to 168 (1 VGPR spilled; the ragged one 21).
#ifndef PA_MFMA_MIN_WAVES
#define PA_MFMA_MIN_WAVES 0
#endif
template <typename T, int D, bool PERSIST, bool RAGGED, bool CAUSAL, bool CHECK>
constexpr int mfma_min_waves() {
  return PA_MFMA_MIN_WAVES > 0 ? PA_MFMA_MIN_WAVES
                               : (PERSIST && D == 64 && (std::is_same<T, bf16>::value || RAGGED || CAUSAL || CHECK)) ? 3 : 1;
}

// CHECK (fp16, two stages, no key split, not the causal form): the lazy rescale is triggered by a
// check on the computed P' (as the bf16 kernels always do) instead of the row max of S before the
// exponentials; see the branch below.
template <typename T, int D, int BM, int BN, int STAGES, typename OutT, int KSPLIT = 1, bool PERSIST = false,
          bool RAGGED = false, bool CAUSAL = false, bool CHECK = false>
__global__ void __launch_bounds__(BM / 32 * kWave * KSPLIT)
__attribute__((amdgpu_waves_per_eu(mfma_min_waves<T, D, PERSIST, RAGGED, CAUSAL, CHECK>())))
fa_mfma_fwd(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
            OutT* __restrict__ O, int N, int num_qblocks, int total_blocks, float scale_log2, int causal,
            int cus_per_xcd, int walk) {
  typedef typename vec8<T>::type V8;
  typedef MfmaLds<D, BN, STAGES> L;
  constexpr float kLazyLog2 = 8.f;       // P stays below 2^kLazyLog2 between rescales
  constexpr int NW = BM / 32;
  constexpr int THREADS = NW * kWave;
  constexpr int QK_STEPS = D / 16;       // MFMA k-steps over the head dim
  constexpr int NKB = BN / 32;           // 32-key blocks per tile
  constexpr int NDB = D / 32;            // 32-dim blocks of O^T
  constexpr int PV_STEPS = BN / 16;      // MFMA k-steps over the keys of a tile
  constexpr int CR = D / 8;              // 16-byte chunks per K/V row
  constexpr int RB = L::ROW_BYTES;
  constexpr int QK_MFMAS = NKB * QK_STEPS;
  constexpr int PV_MFMAS = PV_STEPS * NDB;
  static_assert(D == 64 || D == 128, "head dim");
  static_assert(BM % 32 == 0 && BN % 32 == 0, "tile shape");
  static_assert((BN * CR) % THREADS == 0, "K/V tile must split evenly over the workgroup");
  constexpr int CPT = BN * CR / THREADS; // 16-byte chunks per thread per matrix per tile
  static_assert(STAGES == 1 || STAGES == 2, "one or two LDS stages");
  // Operand reads address the stages through ds_read's 16-bit immediate offset; a stage above
  // 64 KB would need its addresses built in extra VGPRs (measured: -11 % at d = 128).
  static_assert(L::BYTES * KSPLIT <= 65536, "K/V stages must fit ds_read's 64 KB offset reach");
  static_assert(KSPLIT == 1 || (KSPLIT == 2 && STAGES == 2 && (BM / 32) % 2 == 0),
                "key groups: two-stage pipeline, an even number of query waves");
  static_assert(!PERSIST || (KSPLIT == 1 && STAGES == 2), "persistent form: two stages, no key split");
  static_assert(!RAGGED || PERSIST, "RAGGED selects the persistent form whose last key tile is partial");
  static_assert(!CAUSAL || (PERSIST && !RAGGED && BM % (2 * BN) == 0), "CAUSAL selects the persistent causal form");
  static_assert(!CHECK || (std::is_same<T, f16>::value && STAGES == 2 && KSPLIT == 1 && !CAUSAL),
                "CHECK: the fp16 two-stage forms without key split, not the causal one");

  // One LDS object per stage and matrix: the compiler then sees that a tile load into one stage
  // cannot alias the operand reads from another, and does not make those reads wait for it.
  // With KSPLIT key groups each object holds one tile per group.
  __shared__ __attribute__((aligned(1024))) unsigned char k_lds0[L::TILE_BYTES * KSPLIT];
  __shared__ __attribute__((aligned(1024))) unsigned char v_lds0[L::TILE_BYTES * KSPLIT];
  __shared__ __attribute__((aligned(1024))) unsigned char k_lds1[STAGES == 2 ? L::TILE_BYTES * KSPLIT : 16];
  __shared__ __attribute__((aligned(1024))) unsigned char v_lds1[STAGES == 2 ? L::TILE_BYTES * KSPLIT : 16];
  // Persistent forms: each wave's block of O goes through its own LDS rows (MfmaOStage) and leaves
  // as whole rows, 16 bytes per lane. The smaller alignment places o_lds after the K/V stages,
  // which keep their ds_read immediate offsets.
  typedef MfmaOStage<D, BM, OutT> OS;
  constexpr int OROW = OS::ROW;
  constexpr int OCR = OS::CHUNKS;
  constexpr int ORW = OS::ROWS;
  static_assert(32 % OS::PASSES == 0 && (ORW * OCR) % kWave == 0, "O passes: whole rows, whole wave reads");
  __shared__ __attribute__((aligned(16))) unsigned char o_lds[PERSIST ? OS::BYTES : 16];
  const std::integral_constant<int, 0> even{};
  const std::integral_constant<int, 1> odd{};

  // Waves are (key group g) x (query wave): group g takes the key tiles g, g + KSPLIT, ...
  const int g = KSPLIT == 1 ? 0 : (int)threadIdx.x / THREADS;
  const int tid = KSPLIT == 1 ? (int)threadIdx.x : (int)threadIdx.x % THREADS;
  // The persistent form keeps the wave index in an SGPR, so the LDS destinations of its tile
  // loads (M0) are scalar arithmetic instead of v_readfirstlane per load (C4 +0.6 %); the
  // per-block forms spill or lose occupancy with it.
  const int wave = PERSIST ? __builtin_amdgcn_readfirstlane(tid / kWave) : tid / kWave;
  const int lane = tid % kWave;
  auto k_stage = [&](auto par) -> unsigned char* {
    if constexpr (decltype(par)::value) return k_lds1 + g * L::TILE_BYTES; else return k_lds0 + g * L::TILE_BYTES;
  };
  auto v_stage = [&](auto par) -> unsigned char* {
    if constexpr (decltype(par)::value) return v_lds1 + g * L::TILE_BYTES; else return v_lds0 + g * L::TILE_BYTES;
  };
  // Key tile of this group's iteration j.
  auto tile_of = [&](int j) { return j * KSPLIT + g; };
  const int lq = lane % 32;   // query column of this lane in the wave's 32-query tile
  const int hi = lane / 32;   // which half of the 32 accumulator rows this lane holds

  // Query block blk = (head, BM-query block). The persistent form walks the blocks of its XCD's
  // range (blk = x * range + c + C * j for the c-th of the C workgroups on XCD x), so that all
  // blocks of a head still run on one XCD.
  // CAUSAL: a list of query blocks per XCD, XCD x owning the heads x, x + 8, x + 16, ... below
  // B*H, head by head (walk 0) or by length (walk 1); or one list for the device, by length
  // (walk 2). A list is dealt out in serpentine passes over its CUs (causal_walk_block), so the
  // workgroups sharing a CU take blocks from opposite ends of the length order.
  const uint32_t head_bytes = (uint32_t)((size_t)N * D * sizeof(T));
  int blk = 0, blk_step = 0, blk_end = 0, step = 0;
  auto causal_block = [&](int j) -> int {
    const int lists = walk == 2 ? 1 : kNumXcd;   // workgroup g is entry g / lists of list g % lists
    return causal_walk_block(j, (int)blockIdx.x / lists, (int)blockIdx.x % lists, (int)gridDim.x / lists,
                             cus_per_xcd * (kNumXcd / lists), total_blocks / num_qblocks, num_qblocks, walk != 0, lists);
  };
  if constexpr (CAUSAL) {
    blk = causal_block(0);
    if (blk < 0) return;   // more workgroups than blocks on this XCD
  } else if constexpr (PERSIST) {
    const int range = (total_blocks + kNumXcd - 1) / kNumXcd;
    const int x = (int)blockIdx.x % kNumXcd;
    blk_step = (int)gridDim.x / kNumXcd;
    blk_end = min(total_blocks, (x + 1) * range);
    blk = x * range + (int)blockIdx.x / kNumXcd;
    if (blk >= blk_end) return;   // more workgroups than blocks on this XCD
  } else {
    blk = xcd_remap(blockIdx.x, total_blocks);
  }
  int qb = blk % num_qblocks;
  if (causal && !CAUSAL) qb = num_qblocks - 1 - qb;  // longest causal rows first
  int q0 = qb * BM;
  int q0w = q0 + wave * 32;
  int qrow = q0w + lq;
  size_t base = (size_t)(blk / num_qblocks) * N * D;
  rsrc_t q_rs = make_rsrc(Q + base, head_bytes);
  rsrc_t k_rs = make_rsrc(K + base, head_bytes);
  rsrc_t v_rs = make_rsrc(V + base, head_bytes);

  // ---- Q^T operand: lane holds Q[qrow][16*kk + 8*hi + j], j < 8, for every k-step kk
  // (rows past N read as zero).
  V8 qf[QK_STEPS];
  auto load_q = [&](rsrc_t rs, int row) {
    // hi * 16 from the lane id read afresh (an asm the compiler cannot merge across the two calls):
    // held from the prologue to the next block's load, it was the one VGPR the persistent fp16
    // d = 64 kernel spilled.
    uint32_t lane_now;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane_now));
    const uint32_t hi16 = (lane_now >> 1) & 16u;
#pragma unroll
    for (int kk = 0; kk < QK_STEPS; ++kk)
      qf[kk] = __builtin_bit_cast(V8, load16(rs, (uint32_t)(row * RB + kk * 32) + hi16));
  };
  load_q(q_rs, qrow);

  // ---- Direct HBM -> LDS loads. Load i of this thread fills LDS slot i*THREADS + tid of the
  // tile (16 bytes each, slots in lane order), i.e. row slot/CR at physical chunk slot%CR, which
  // holds logical chunk (slot%CR) ^ swz(row). The per-lane source offsets are fixed; the tile
  // start goes in the scalar offset.
  uint32_t k_src[CPT], v_src[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int slot = i * THREADS + tid;
    const int row = slot / CR, pc = slot % CR;
    k_src[i] = (uint32_t)(row * RB + ((pc ^ k_swz<CR>(row)) * 16));
    v_src[i] = (uint32_t)(row * RB + ((pc ^ v_swz<CR>(row)) * 16));
  }
  auto load_tile = [&](rsrc_t rs, const uint32_t (&src)[CPT], unsigned char* stage, int j0) {
#pragma unroll
    for (int i = 0; i < CPT; ++i)
      load16_to_lds(rs, stage + (i * THREADS + wave * kWave) * 16, src[i], (uint32_t)(j0 * RB));
  };

  // ---- Operand read addresses (byte offsets inside a stage).
  // K operand of k-step kk: row 32b + lq, logical chunk 2kk + hi.
  int k_addr[QK_STEPS];
#pragma unroll
  for (int kk = 0; kk < QK_STEPS; ++kk) k_addr[kk] = lq * RB + (((2 * kk + hi) ^ k_swz<CR>(lq)) * 16);
  // V^T operand (transposed read): in each 16-lane group g, lane i supplies row 4*hi + i/4
  // (+16*ks, +8 for the second half) and logical dims 32*db + 16*(g%2) + 4*(i%4) .. +3;
  // ds_read_b64_tr_b16 then hands lane i the element i%4 of the rows supplied by lanes
  // 4t + i/4, i.e. V[row0 + t][32*db + 16*(g%2) + i], t < 4.
  const int g16 = lane / 16, i16 = lane % 16;
  const int v_row = hi * 4 + i16 / 4;
  const int v_cl = 2 * (g16 % 2) + (i16 % 4) / 2;   // logical chunk within the 4-chunk dim block
  int v_addr[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
    v_addr[db] = v_row * RB + (((4 * db + v_cl) ^ v_swz<CR>(v_row)) * 16) + 8 * (i16 % 2);

  float m_run = -INFINITY;  // running max of the log2-domain scores of row qrow
  float m_out = -INFINITY;  // the exponent reference O and l are scaled by, for the key-group merge
  // Row sum on the matrix core: lacc += ONES . P^T per 16-key step (16x16x32). The P^T operand
  // of lane l holds 8 keys of query l%32; with A[m][8g+j] = 1 iff (m/4)%2 == g%2, output rows
  // 4g..4g+3 of column n sum both key halves of query n + 16*(g%2), so every lane ends with the
  // sum of its own query (all 4 registers equal).
  f32x4 lacc = {0.f, 0.f, 0.f, 0.f};
  V8 ones;
  {
    const bool on = (((lane % 16) / 4) % 2) == ((lane / 16) % 2);
#pragma unroll
    for (int j = 0; j < 8; ++j) ones[j] = from_f32<T>(on ? 1.f : 0.f);
  }
  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = f32x16{};

  const int kv_end = causal ? min(N, q0 + BM) : N;
  // (CAUSAL: the block's tile counts, set again for every block of the walk.)
  int ntiles = (kv_end + BN - 1) / BN;
  const int wave_kv_end = causal ? min(kv_end, q0w + 32) : kv_end;  // keys this wave can see
  int wave_tiles = (wave_kv_end + BN - 1) / BN;
  // RAGGED with an odd tile count (every tile full): one more tile, entirely past N (it loads as
  // zeros and is masked to P = 0), makes the count even for the wrap copies. CAUSAL: the same
  // padding for a last query block that ends past N; the padded tile lies past every wave's last
  // tile, so no wave computes on it.
  if constexpr (RAGGED) {
    ntiles += ntiles & 1;
    wave_tiles = ntiles;
  }
  if constexpr (CAUSAL) ntiles += ntiles & 1;
  const int nit = (ntiles + KSPLIT - 1) / KSPLIT;   // iterations of every key group
  // Tiles [0, clean_tiles) need no mask for this wave: all keys < N and (causal) all keys at or
  // before the wave's first query.
  const int clean_tiles = causal ? min(N / BN, (q0w + 1) / BN) : N / BN;

  // S^T = K . Q^T for the tile in K stage `ks`; the 32-key blocks alternate so that
  // consecutive MFMAs never depend on each other.
  auto qk = [&](f32x16 (&s)[NKB], const unsigned char* ks) {
#pragma unroll
    for (int b = 0; b < NKB; ++b) s[b] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < QK_STEPS; ++kk)
#pragma unroll
      for (int b = 0; b < NKB; ++b) {
        const V8 a = *reinterpret_cast<const V8*>(ks + b * 32 * RB + k_addr[kk]);
        s[b] = mfma32x32x16(a, qf[kk], s[b]);
      }
  };

  // Mask keys past N and (causal) keys after the query.
  // Persistent form: the wrap copies mask the same tile index in every block; an offset the
  // compiler cannot see through keeps it from hoisting the mask's comparisons out of the block
  // loop (~84 predicate pairs, which spill).
  auto opaque_offset = [](int j0) __attribute__((always_inline)) {
    if constexpr (RAGGED) asm volatile("" : "+s"(j0));
    return j0;
  };
  // CAUSAL form: the causal mask of the wave's diagonal tile (a key past N comes after every row
  // before N, so this mask hides it too; rows past N, whose keys past N read as zeros, are never
  // stored). Key j0 + off (off = 32 b + 8 (r / 4) + 4 hi + r % 4) is visible iff
  // 32 b + 8 (r / 4) + r % 4 <= qrow - j0 - 4 hi; that limit is hidden from the compiler, which
  // would otherwise hoist the 32 per-lane terms qrow - off out of the block loop (they spill).
  auto mask_diag = [&](f32x16 (&s)[NKB], int j0) {
    int lim = qrow - j0 - 4 * hi;
    asm volatile("" : "+v"(lim));
#pragma unroll
    for (int b = 0; b < NKB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (b * 32 + (r / 4) * 8 + (r % 4) > lim) s[b][r] = -INFINITY;
  };
  auto mask = [&](f32x16 (&s)[NKB], int j0) {
#pragma unroll
    for (int b = 0; b < NKB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = j0 + b * 32 + (r / 4) * 8 + hi * 4 + (r % 4);
        if (key >= N || (causal && key > qrow)) s[b][r] = -INFINITY;
      }
  };

  // Row max of a masked tile. `rescale` is set, wave-uniform, when some row's max exceeds its
  // reference max m_run by more than 2^kLazyLog2; then every row whose max grew takes it as its
  // new m_run. Returns alpha = 2^(m_old - m_new): 0 on a row's first visible tile, exactly 1
  // where m_run is kept.
  auto update_max = [&](const f32x16 (&s)[NKB], bool& rescale) -> float {
    float mx = -INFINITY;
#pragma unroll
    for (int b = 0; b < NKB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[b][r]);
    const float m_new = fmaxf(m_run, half_max(mx) * scale_log2);
    rescale = __builtin_amdgcn_ballot_w64(m_new > m_run + kLazyLog2) != 0;
    const bool upd = rescale && m_new > m_run;
    const float alpha = upd ? exp2_fast(m_run - m_new) : 1.f;  // m_run = -inf -> 0
    m_run = upd ? m_new : m_run;
    return alpha;
  };

  // P = 2^(S*c - m) rounded to T: the PV operand.
  auto exponentiate = [&](const f32x16 (&s)[NKB], V8 (&pf)[PV_STEPS]) {
    const float neg_m = (m_run == -INFINITY) ? 0.f : -m_run;  // fully masked row: P = 0
#pragma unroll
    for (int b = 0; b < NKB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) pf[b * 2 + r / 8][r % 8] = from_f32<T>(exp2_fast(fmaf(s[b][r], scale_log2, neg_m)));
  };
  // l += sum of the rounded P: 16x16x32 MFMAs of the 0/1 operand by P^T (exact products, fp32
  // accumulation).
  auto row_sum = [&](const V8 (&pf)[PV_STEPS]) {
#pragma unroll
    for (int ks_ = 0; ks_ < PV_STEPS; ++ks_) lacc = mfma16x16x32(ones, pf[ks_], lacc);
  };

  auto rescale_o = [&](float alpha) {
    lacc *= alpha;
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] *= alpha;
  };

  // O^T += V^T . P^T for the tile in V stage `vs`.
  auto pv = [&](const V8 (&pf)[PV_STEPS], const unsigned char* vs) {
#pragma unroll
    for (int ks_ = 0; ks_ < PV_STEPS; ++ks_) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const unsigned char* p0 = vs + ks_ * 16 * RB + v_addr[db];
        const i16x4 a0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr<i16x4>)(p0));
        const i16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr<i16x4>)(p0 + 8 * RB));
        const i16x8 a = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        o[db] = mfma32x32x16(__builtin_bit_cast(V8, a), pf[ks_], o[db]);
      }
    }
  };

  // O = O^T / l for the current block. Register r of block db holds dim 32*db + 8*(r/4) + 4*hi + r%4.
  // Staged stores: each wave writes its 32 rows of O into LDS rows of its own (16-byte chunks
  // XOR-swizzled by row) and reads them back as whole rows, for non-temporal 16-byte buffer stores
  // that each cover whole rows. O is written once and not read again, and whole-row stores let the
  // lines leave L2 during the kernel instead of with the cache writeback at its end (persistent C3
  // +4 %, per-block launches at the C3 / C4 shapes +3 / +1.4 %; stores of the lane's 8-byte pieces,
  // non-temporal or write-through, were 13-15 % slower). Rows past N fall outside the buffer and
  // are dropped. The persistent forms stage in o_lds; the two-stage per-block forms, which end with
  // their block, in the K/V stages: wave w in stage object w % 4 at slot w / 4. The key-split and
  // single-stage forms store each lane's pieces directly (staged, C2 was 2 % slower, and the
  // single-stage 128 x 32 tile lost a wave per SIMD).
  constexpr bool PB_STAGED = !PERSIST && KSPLIT == 1 && STAGES == 2;
  constexpr int PB_SLOT = L::TILE_BYTES / ((NW + 3) / 4);   // staging bytes per wave
  constexpr int PB_ROWS = PB_SLOT >= 32 * OROW ? 32 : PB_SLOT >= 16 * OROW ? 16 : PB_SLOT >= 8 * OROW ? 8 : 4;
  static_assert(!PB_STAGED || ((PB_ROWS * OCR) % kWave == 0 && PB_ROWS * OROW <= PB_SLOT),
                "per-block O staging: whole wave reads");
  auto store_rows = [&](unsigned char* ws, auto rows_c) {   // rows_c: rows per pass
    constexpr int R = decltype(rows_c)::value;
    constexpr int PASSES = 32 / R;
    constexpr int kNonTemporal = 2;   // buffer store cache policy: nt
    typedef OutT OutV4 __attribute__((ext_vector_type(4)));
    const float inv = 1.f / lacc[0];
    const rsrc_t o_rs = make_rsrc(O + base, (uint32_t)((size_t)N * OROW));
    // Lane-derived offsets behind an empty asm: hoisted out of the block loop they cost ~14 VGPRs.
    int ln = lane;
    asm volatile("" : "+v"(ln));
    // Chunk swizzle of a staged row: 128-byte rows (8 chunks) pair up rows as the K tiles do, so
    // the 32 rows written at one chunk spread over all 64 banks; longer rows XOR by row % chunks.
    auto o_swz = [](int row) { return OCR == 8 ? (row >> 1) & 7 : row % OCR; };
    const int lq_ = ln % 32, hi_ = ln / 32;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      if (lq_ / R == p) {
        const int row = lq_ % R;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            OutV4 w;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) w[rr] = from_f32<OutT>(o[db][g4 * 4 + rr] * inv);
            const int byte = (32 * db + 8 * g4 + 4 * hi_) * (int)sizeof(OutT);
            *reinterpret_cast<OutV4*>(ws + row * OROW + (((byte / 16) ^ o_swz(row)) * 16) + byte % 16) = w;
          }
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): the wave's rows are in LDS
#pragma unroll
      for (int i = 0; i < R * OCR / kWave; ++i) {
        const int c16 = i * kWave + ln, row = c16 / OCR, c = c16 % OCR;
        const u32x4 d = *reinterpret_cast<const u32x4*>(ws + row * OROW + ((c ^ o_swz(row)) * 16));
        // (fp32 O: a head can span up to 4 GiB, so the offset is unsigned.)
        __builtin_amdgcn_raw_buffer_store_b128(d, o_rs, (uint32_t)(q0w + p * R + row) * (uint32_t)OROW + c * 16, 0,
                                               kNonTemporal);
      }
      if (p + 1 < PASSES) __builtin_amdgcn_s_waitcnt(0xc07f);   // reads done before the next pass
    }
  };
  auto store_block = [&]() {
    if constexpr (PERSIST) {
      store_rows(o_lds + wave * ORW * OROW, std::integral_constant<int, ORW>{});
    } else if constexpr (PB_STAGED) {
      __syncthreads();   // every wave is done with the K/V stages
      const int obj = wave % 4;
      unsigned char* st = obj == 0 ? k_lds0 : obj == 1 ? v_lds0 : obj == 2 ? k_lds1 : v_lds1;
      store_rows(st + (wave / 4) * PB_SLOT, std::integral_constant<int, PB_ROWS>{});
    } else if (g == 0 && qrow < N) {
      typedef OutT OutV4 __attribute__((ext_vector_type(4)));
      const float inv = 1.f / lacc[0];
      OutT* orow = O + base + (size_t)qrow * D;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          OutV4 w;
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) w[rr] = from_f32<OutT>(o[db][g4 * 4 + rr] * inv);
          *reinterpret_cast<OutV4*>(orow + db * 32 + g4 * 8 + hi * 4) = w;
        }
    }
  };

  // Two-stage prologue: the first tiles into LDS, all in flight together. The persistent forms
  // (at least two tiles per block) load K(0), V(0) and K(1) and wait for Q, K(0) and V(0) only
  // (vmcnt counts these loads in issue order), so the first tile's MFMAs run while K(1) arrives;
  // the wait after the first tile covers it before iteration 0. Their V(1) comes with iteration 0.
  // The per-block forms load K(0), V(0), K(1), V(1) and wait for all of them.
  auto prologue_loads = [&]() {
    if constexpr (PERSIST) {
      load_tile(k_rs, k_src, k_stage(even), 0);
      load_tile(v_rs, v_src, v_stage(even), 0);
      load_tile(k_rs, k_src, k_stage(odd), BN);
      __builtin_amdgcn_s_waitcnt(CPT);   // vmcnt(CPT) expcnt(0) lgkmcnt(0): all but K(1)
    } else {
      if (KSPLIT == 1 || tile_of(0) < ntiles) {   // a workgroup always has a first tile
        load_tile(k_rs, k_src, k_stage(even), tile_of(0) * BN);
        load_tile(v_rs, v_src, v_stage(even), tile_of(0) * BN);
      }
      if (tile_of(1) < ntiles) {
        load_tile(k_rs, k_src, k_stage(odd), tile_of(1) * BN);
        load_tile(v_rs, v_src, v_stage(odd), tile_of(1) * BN);
      }
      __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();
  };
  static_assert(CPT < 16, "prologue wait: vmcnt(CPT) in the low vmcnt bits");

  if constexpr (STAGES == 2 && (std::is_same<T, bf16>::value || CHECK)) {
    // bf16 (and fp16 with CHECK): overflow check instead of a row max. The exponent's reference point is
    // m_ref = m + kShift, so the P.V operand is P' = 2^(S c - m_ref) = P 2^-kShift and
    // "some P > 2^kLazyLog2" is "some rounded P' >= 2": bit 14 of the bf16 pattern (the top
    // exponent bit), tested by one OR over the packed P' registers. bf16 has fp32's exponent
    // range, so the 2^-7 scale loses nothing, and O / l is unchanged (numerator and denominator
    // carry the same scale). When the check fires (wave-uniform, rare after the first tile) the
    // exact row max is taken, O and l are rescaled and P'(t) is recomputed: the same update as
    // the fp16 path, done after the exponentials instead of before them. The finite start value
    // of m_ref makes every finite score of a row's first visible tile overflow (a rescale) and
    // keeps a masked score at P' = 0 without a NaN.
    // fp16 (CHECK): fp16 has no room below for the 2^-7 shift (P' would turn subnormal 7 octaves
    // earlier), and one exponent bit gives no larger window. The check is instead the packed fp16
    // max of the P' registers (v_pk_maximum3_f16, as many instructions as the OR), compared once
    // with 2^14; with m_ref = m + 4 that lets a row's max grow 18 octaves past the reference
    // before a rescale (P' <= 2^14 < fp16's 65504; the P' of keys within 10 octaves of the
    // reference stay normal). Peaked rows (C5: scores spread ~13 octaves) then rescale about once
    // instead of at every new maximum. A P' that overflowed fp16 reads as inf in the max and fires.
    constexpr bool kPackedMax = std::is_same<T, f16>::value;
    constexpr float kShift = kPackedMax ? 4.f : kLazyLog2 - 1.f;
    constexpr float kFireF16 = 16384.f;         // fp16: fire when some rounded P' >= 2^14
    constexpr uint32_t kTopExp = 0x40004000u;   // bf16: exponent MSB of both halves (P' >= 2)
    // A check word that fires: the bf16 bits, or fp16 (inf, inf) for the packed max.
    constexpr uint32_t kForce = kPackedMax ? 0x7C007C00u : kTopExp;
    constexpr int HALF = PV_STEPS / 2;
    float m_ref = -3.0e38f;
    // The check word of one operand register folded into acc: bf16, the OR of the P' patterns
    // (the check fires when some lane of the wave has the top exponent bit set); fp16, the packed
    // max of the P' values (it fires when some lane's max reaches 2^14).
    typedef _Float16 H2 __attribute__((ext_vector_type(2)));
    auto check_acc = [&](const V8& a, uint32_t acc) __attribute__((always_inline)) -> uint32_t {
      if constexpr (kPackedMax) {
        // (pairs taken with shufflevector: with this compiler, bit-casting single elements of the
        // u32x4 view of the register read element 0 for every index)
        H2 mx = __builtin_bit_cast(H2, acc);
        mx = __builtin_elementwise_maximum(__builtin_elementwise_maximum(mx, __builtin_shufflevector(a, a, 0, 1)),
                                           __builtin_shufflevector(a, a, 2, 3));
        mx = __builtin_elementwise_maximum(__builtin_elementwise_maximum(mx, __builtin_shufflevector(a, a, 4, 5)),
                                           __builtin_shufflevector(a, a, 6, 7));
        return __builtin_bit_cast(uint32_t, mx);
      } else {
        const u32x4 x = __builtin_bit_cast(u32x4, a);
        return acc | x[0] | x[1] | x[2] | x[3];
      }
    };
    auto check_fires = [&](uint32_t acc) __attribute__((always_inline)) -> bool {
      if constexpr (kPackedMax) {
        const H2 mx = __builtin_bit_cast(H2, acc);
        return __builtin_amdgcn_ballot_w64(fmaxf((float)mx[0], (float)mx[1]) >= kFireF16) != 0;
      } else {
        return __builtin_amdgcn_ballot_w64((acc & kTopExp) != 0) != 0;
      }
    };
    // `opaque` hides -m_ref behind an empty asm so that the fast path's exponentials are not
    // merged with the generic path's and hoisted out of the MFMA phases.
    auto exp_range = [&](const f32x16 (&s_)[NKB], V8 (&pf)[PV_STEPS], int lo, int hi, bool opaque) __attribute__((always_inline)) {
      float nm = -m_ref;
      if (opaque) asm("" : "+v"(nm));
#pragma unroll
      for (int i = 0; i < PV_STEPS; ++i)
        if (i >= lo && i < hi)
#pragma unroll
          for (int j = 0; j < 8; ++j) pf[i][j] = from_f32<T>(exp2_fast(fmaf(s_[i / 2][8 * (i % 2) + j], scale_log2, nm)));
    };
    // Rare path: exact row max of S(t); rows whose max grew take m_ref = max + kShift and
    // rescale O and l by 2^(m_ref_old - m_ref_new) (0 on a row's first visible tile).
    auto exact_rescale = [&](const f32x16 (&s_)[NKB]) __attribute__((always_inline)) {
      float mx = -INFINITY;
#pragma unroll
      for (int b = 0; b < NKB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s_[b][r]);
      const float mrow = half_max(mx) * scale_log2 + kShift;   // -inf on a fully masked row
      const bool upd = mrow > m_ref;
      const float alpha = upd ? exp2_fast(m_ref - mrow) : 1.f;
      m_ref = upd ? mrow : m_ref;
      rescale_o(alpha);
    };
    constexpr int c0 = 0, ch = HALF, cf = PV_STEPS;

    // Prologue: the first tiles into LDS together (one memory latency instead of two for short
    // rows); S(0).
    prologue_loads();

    // Score and P' buffers swap roles every iteration (the loop is unrolled by two so the swap
    // costs no register moves). On the fast path the first HALF P' registers of tile t and
    // their OR (`or_c`) come from iteration t-1 (for tile 0, from the prologue, after the first
    // tile's exact max).
    f32x16 sa[NKB], sb[NKB];
    V8 pa[PV_STEPS], pb[PV_STEPS];
    uint32_t or_c = kForce;
    // S(0) and the first half of P'(0) of a block (the arrays are parameters, not captures:
    // capturing them here changes how the compiler allocates the whole kernel).
    auto first_tile = [&](f32x16 (&s0)[NKB], V8 (&p0)[PV_STEPS]) {
      if (tile_of(0) < wave_tiles) {
        qk(s0, k_stage(even));
        if (!PERSIST && tile_of(0) >= clean_tiles) mask(s0, tile_of(0) * BN);
        if (CAUSAL && wave_tiles == 1) mask_diag(s0, 0);
        exact_rescale(s0);   // the first tile's exact max: m_ref set, O and l stay 0
        exp_range(s0, p0, c0, ch, false);
        uint32_t nb = 0;
#pragma unroll
        for (int i = 0; i < HALF; ++i) nb = check_acc(p0[i], nb);
        or_c = nb;
      }
    };
    first_tile(sa, pa);
    // Iteration 0 loads K(2) into K(0)'s stage: every wave must have read K(0) first (and, in the
    // persistent forms, K(1) must have landed).
    if constexpr (PERSIST) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // Persistent form: whether this workgroup has a next query block, and its index. The current
    // block's last two iterations (the "wrap" copies) load that block's K(0), K(1), V(0) and Q.
    bool has_next = false;
    int blk_n = 0;
    auto next_base = [&]() { return (size_t)(blk_n / num_qblocks) * N * D; };

    // `par` is the parity of t as a compile-time constant, so every stage below is a fixed LDS
    // object: K(t+1) in k_stage(!par), V(t) in v_stage(par).
    auto iteration = [&](auto par, auto wrap, int t, f32x16 (&s)[NKB], f32x16 (&sn)[NKB], V8 (&pf)[PV_STEPS],
                         V8 (&pn)[PV_STEPS]) {
      constexpr int P = decltype(par)::value;
      // WRAP: the persistent form's last two iterations of a block (t = nit-2, nit-1): loads past
      // the block's last tile fetch the next block's first tiles instead; the last one has no
      // S(t+1) and therefore no fast-path copy. DIAG (CAUSAL form): an iteration at or after the
      // block's last clean tile pair, whose path is chosen per wave.
      constexpr bool WRAP = (decltype(wrap)::value & 1) != 0;
      constexpr bool DIAG = (decltype(wrap)::value & 2) != 0;
      constexpr bool kMayBeFast = !(WRAP && P == 1);
      const std::integral_constant<int, P> cur{};
      const std::integral_constant<int, 1 - P> nxt{};
      // K(t+2) replaces K(t) (read in iteration t-1; K(0) by the first tile, before the barrier
      // above); V(t+1) replaces V(t-1) (V(1) came with the prologue). Every wave issues its
      // share of both loads in every iteration: on the fast path inside phase A (so the 8 waves
      // leaving the barrier do not queue them all at once; +1.4 % on C4), otherwise here. They
      // are waited for before the iteration's closing barrier.
      // Persistent form: every tile but (RAGGED) the last is full, so every iteration outside the
      // wrap copies takes the fast path; the last wrap copy never does, the first only when the
      // last tile is full. DIAG: the fast path up to the wave's last tile (S(t+1) masked before
      // phase B when t+1 is the wave's diagonal tile; on the last tile itself S(t+1) is computed
      // and not used, which keeps the generic path, and its registers, out of these copies),
      // idle after it.
      const bool fast = DIAG ? (kMayBeFast && t < wave_tiles)
                             : PERSIST ? (kMayBeFast && !(WRAP && RAGGED))
                                       : (tile_of(t) < wave_tiles && tile_of(t + 1) < clean_tiles);
      if (!fast) {
        if (tile_of(t + 2) < ntiles) load_tile(k_rs, k_src, k_stage(cur), tile_of(t + 2) * BN);
        else if (WRAP && has_next) load_tile(make_rsrc(K + next_base(), head_bytes), k_src, k_stage(cur), (tile_of(t + 2) - ntiles) * BN);
        if ((PERSIST || t >= 1) && tile_of(t + 1) < ntiles) load_tile(v_rs, v_src, v_stage(nxt), tile_of(t + 1) * BN);
        else if (WRAP && has_next && tile_of(t + 1) == ntiles) load_tile(make_rsrc(V + next_base(), head_bytes), v_src, v_stage(nxt), 0);
        if constexpr (WRAP && P == 1) {
          if (has_next) load_q(make_rsrc(Q + next_base(), head_bytes), (blk_n % num_qblocks) * BM + wave * 32 + lq);
        }
      }
      if ((PERSIST && !DIAG) || tile_of(t) < wave_tiles) {
        const unsigned char* kn = k_stage(nxt);
        const unsigned char* vc = v_stage(cur);
        if (fast) {
          // Fast path, straight-line. Phase A: S(t+1) MFMAs with the second half of P'(t) and
          // the overflow check of all of P'(t).
          // VALU instructions placed after each MFMA: the per-phase totals spread evenly, except
          // at d = 128, where 2 and 2 measured fastest (C4, against (2, 3) +0.8 %, (3, 2) -1 %,
          // (3, 3) -2 %, (4, x) -3 to -5 %; with the row sum on the matrix core, phase B has 20
          // MFMAs for ~46 VALU instructions).
          constexpr int VA = D == 128 ? 2 : (HALF * 20 + 6 + QK_MFMAS - 1) / QK_MFMAS;
          constexpr int VB = D == 128 ? 2 : (HALF * 20 + PV_STEPS * 4 + 3 + PV_MFMAS - 1) / PV_MFMAS;
          // Phase A runs at wave priority 2 (0 again after it), so the SIMD's issue arbitration
          // favours a wave starting its S(t+1) MFMAs over the other waves' phase B. Measured back
          // to back against priority 0 throughout (bits unchanged): C4 +0.4-0.9 %, C3 +2.4-2.6 %,
          // C5 +1.0-1.8 %, fp16 4x32x4096 d = 128 +0.5-2.7 %, bf16 8x16x2048 d = 64 +2.5 %, causal
          // C4 +0.5 %, the bf16 key split on causal 1x5x4096 +4 %; priority 1 or 3 within 0.2 % of
          // 2; priority raised for phase B instead lost 0.4-0.9 % at d = 64.
          __builtin_amdgcn_s_setprio(2);
          qk(sn, kn);
          // This iteration's tile loads, issued inside phase A (unconditionally, to keep the phase
          // branch-free: past the last tile K reloads the last tile into the free stage, and at
          // t = 0 V(1) is written again over itself).
          if constexpr (WRAP) {
            // t = nit-2: K(t+2) is the next block's K(0) (or, after the last block, this block's
            // last tile again into the free stage).
            load_tile(make_rsrc(K + (has_next ? next_base() : base), head_bytes), k_src, k_stage(cur), has_next ? 0 : (ntiles - 1) * BN);
          } else {
            load_tile(k_rs, k_src, k_stage(cur), min(tile_of(t + 2), ntiles - 1) * BN);
          }
          load_tile(v_rs, v_src, v_stage(nxt), tile_of(t + 1) * BN);
          exp_range(s, pf, ch, cf, true);
          uint32_t bits = or_c;
#pragma unroll
          for (int i = HALF; i < PV_STEPS; ++i) bits = check_acc(pf[i], bits);
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
#pragma unroll
          for (int i = 0; i < QK_MFMAS; ++i) {
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedValu, VA, 0);
          }
          __builtin_amdgcn_sched_barrier(0);
          __builtin_amdgcn_s_setprio(0);
          if constexpr (DIAG) {
            if (t + 2 == wave_tiles) mask_diag(sn, (t + 1) * BN);
          }
          if (check_fires(bits)) {
            exact_rescale(s);
            exp_range(s, pf, c0, cf, false);
          }
          if constexpr (DIAG) {
            // A row of one tile (the generic path's two bf16 terms, below): the low terms first.
            if (wave_tiles == 1) {
              const float nm = -m_ref;
#pragma unroll
              for (int i = 0; i < PV_STEPS; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                  const float x = exp2_fast(fmaf(s[i / 2][8 * (i % 2) + j], scale_log2, nm));
                  pn[i][j] = from_f32<T>(x - to_f32(pf[i][j]));
                }
              row_sum(pn);
              pv(pn, vc);
            }
          }
          // Phase B: PV(t) MFMAs with the row sum of P'(t) and the first half of P'(t+1).
          pv(pf, vc);
          row_sum(pf);
          exp_range(sn, pn, c0, ch, true);
          uint32_t nb = 0;
#pragma unroll
          for (int i = 0; i < HALF; ++i) nb = check_acc(pn[i], nb);
          or_c = nb;
          // V operand reads (two per MFMA) run two MFMAs ahead of their use.
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4, 0);
#pragma unroll
          for (int i = 0; i < PV_MFMAS + PV_STEPS; ++i) {
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedValu, VB, 0);
          }
          __builtin_amdgcn_sched_barrier(0);
        } else {
          // Generic path: the next tile is masked or absent. P'(t) is computed here in full.
          const bool ahead = tile_of(t + 1) < wave_tiles;
          exp_range(s, pf, c0, cf, false);
          uint32_t bits = 0;
#pragma unroll
          for (int i = 0; i < PV_STEPS; ++i) bits = check_acc(pf[i], bits);
          if (check_fires(bits)) {
            exact_rescale(s);
            exp_range(s, pf, c0, cf, false);
          }
          if constexpr (!PERSIST) {
            // Rows of at most BN keys (one tile: short causal rows, N <= BN): P' is taken as two
            // bf16 terms, hi = round(P') (in pf) and lo = round(P' - hi) (in pn, unused without
            // a next tile), and both go through P.V and the row sum. With few keys a single bf16
            // P' per key (8 significant bits) leaves up to half an ulp of max|V| in O; the two
            // terms carry ~16 bits. Longer rows average the rounding over their keys.
            if (wave_tiles == 1) {
              const float nm = -m_ref;
#pragma unroll
              for (int i = 0; i < PV_STEPS; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                  const float x = exp2_fast(fmaf(s[i / 2][8 * (i % 2) + j], scale_log2, nm));
                  pn[i][j] = from_f32<T>(x - to_f32(pf[i][j]));
                }
              row_sum(pn);
              pv(pn, vc);
            }
          }
          row_sum(pf);
          pv(pf, vc);
          if (ahead) {
            qk(sn, kn);
            if constexpr (!PERSIST || RAGGED) mask(sn, opaque_offset(tile_of(t + 1) * BN));
          }
          or_c = kForce;   // no P'(t+1) half was made: a fast iteration after this one recomputes
        }
      }
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    };

    const std::false_type no_wrap{};
    if constexpr (!PERSIST) {
      for (int t = 0; t < nit; t += 2) {
        iteration(even, no_wrap, t, sa, sb, pa, pb);
        if (t + 1 < nit) iteration(odd, no_wrap, t + 1, sb, sa, pb, pa);
      }
    } else {
      // The launcher guarantees an even tile count nit = ntiles >= 2 in every block: the block's
      // last two iterations are the wrap copies. Non-causal: only the last tile can be partial
      // (RAGGED), and the query block is blk % num_qblocks. CAUSAL: only a head's last query
      // block can end past N (its tile count padded to even).
      const std::true_type with_wrap{};
      const std::integral_constant<int, 2> diag{};
      const std::integral_constant<int, 3> diag_wrap{};
      while (true) {
        if constexpr (CAUSAL) {
          blk_n = causal_block(step + 1);
          has_next = blk_n >= 0;
          // Tiles [0, c) are clean in every wave; the per-wave copies start two tiles before c.
          const int c = q0 / BN;
          for (int t = 0; t < c - 2; t += 2) {
            iteration(even, no_wrap, t, sa, sb, pa, pb);
            iteration(odd, no_wrap, t + 1, sb, sa, pb, pa);
          }
          for (int t = max(c - 2, 0); t < ntiles - 2; t += 2) {
            iteration(even, diag, t, sa, sb, pa, pb);
            iteration(odd, diag, t + 1, sb, sa, pb, pa);
          }
          iteration(even, diag_wrap, ntiles - 2, sa, sb, pa, pb);
          iteration(odd, diag_wrap, ntiles - 1, sb, sa, pb, pa);
        } else {
          blk_n = blk + blk_step;
          has_next = blk_n < blk_end;
          for (int t = 0; t < nit - 2; t += 2) {
            iteration(even, no_wrap, t, sa, sb, pa, pb);
            iteration(odd, no_wrap, t + 1, sb, sa, pb, pa);
          }
          iteration(even, with_wrap, nit - 2, sa, sb, pa, pb);
          iteration(odd, with_wrap, nit - 1, sb, sa, pb, pa);
        }
        store_block();
        if (!has_next) break;
        ++step;
        blk = blk_n;
        q0 = (blk % num_qblocks) * BM;
        q0w = q0 + wave * 32;
        qrow = q0w + lq;
        if constexpr (CAUSAL) {
          // (Not clamped at N: that differs only for a wave whose rows all lie past N, which
          // computes on keys that read as zeros and stores nothing; the clamp costs 3 VGPRs and a
          // spill in the bf16 d = 128 kernel. Every load and barrier is independent of wave_tiles.)
          ntiles = (min(N, q0 + BM) + 2 * BN - 1) / (2 * BN) * 2;
          wave_tiles = (q0w + 32 + BN - 1) / BN;
        }
        base = (size_t)(blk / num_qblocks) * N * D;
        q_rs = make_rsrc(Q + base, head_bytes);
        k_rs = make_rsrc(K + base, head_bytes);
        v_rs = make_rsrc(V + base, head_bytes);
#pragma unroll
        for (int db = 0; db < NDB; ++db) o[db] = f32x16{};
        lacc = f32x4{0.f, 0.f, 0.f, 0.f};
        m_ref = -3.0e38f;
        // K(0), K(1), V(0) and Q landed with the last iteration's wait; V(1) comes with
        // iteration 0's phase A, as for the first block.
        first_tile(sa, pa);
        __syncthreads();
      }
    }
    m_out = m_ref;
  } else if constexpr (STAGES == 2) {
    // fp16: the row max of S(t+1) decides the rescale before its exponentials.
    // Prologue: the first tiles into LDS together (one memory latency instead of two for short
    // rows); S(0) and its row max.
    prologue_loads();

    // Two score buffers swap roles every iteration (the loop is unrolled by two so the swap
    // costs no register moves).
    f32x16 sa[NKB], sb[NKB];
    V8 pa[PV_STEPS], pb[PV_STEPS];
    bool rescale = false;
    float alpha = 1.f;
    // The first QB P operand registers of tile t+1 are made in phase B of iteration t, right after
    // its row max, the rest in phase A of iteration t+1, so both MFMA phases carry about the same
    // VALU work. `opaque` keeps the fast path's exponentials from being merged with the generic
    // path's and hoisted out of the MFMA phases. Measured per tile: at d = 64 every tile but the
    // 64 x 64 one runs 2-7 % faster with the split; that tile (6 %) and d = 128 (1 %, where 16
    // MFMAs per phase already carry the exponentials) run faster with all of P(t) in phase A.
    constexpr int QB = (D == 128 || (BM == 64 && BN == 64)) ? 0 : PV_STEPS / 2;
    auto exp_part = [&](const f32x16 (&s_)[NKB], V8 (&p_)[PV_STEPS], int lo, int hi, bool opaque) __attribute__((always_inline)) {
      float nm = (m_run == -INFINITY) ? 0.f : -m_run;  // fully masked row: P = 0
      if (opaque) asm("" : "+v"(nm));
#pragma unroll
      for (int i = 0; i < PV_STEPS; ++i)
        if (i >= lo && i < hi)
#pragma unroll
          for (int j = 0; j < 8; ++j) p_[i][j] = from_f32<T>(exp2_fast(fmaf(s_[i / 2][8 * (i % 2) + j], scale_log2, nm)));
    };
    // S(0), its row max and the first QB P registers of a block (arrays as parameters, not
    // captures, as on the bf16 path).
    auto first_tile = [&](f32x16 (&s0)[NKB], V8 (&p0)[PV_STEPS]) {
      if (tile_of(0) < wave_tiles) {
        qk(s0, k_stage(even));
        if (!PERSIST && tile_of(0) >= clean_tiles) mask(s0, tile_of(0) * BN);
        if (CAUSAL && wave_tiles == 1) mask_diag(s0, 0);
        alpha = update_max(s0, rescale);
        exp_part(s0, p0, 0, QB, false);
      }
    };
    first_tile(sa, pa);
    // Iteration 0 loads K(2) into K(0)'s stage: every wave must have read K(0) first (and, in the
    // persistent forms, K(1) must have landed).
    if constexpr (PERSIST) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // Persistent form: the next query block of this workgroup, loaded by the wrap copies (as on
    // the bf16 path).
    bool has_next = false;
    int blk_n = 0;
    auto next_base = [&]() { return (size_t)(blk_n / num_qblocks) * N * D; };

    // `par` is the parity of t as a compile-time constant, so every stage below is a fixed LDS
    // object: K(t+1) in k_stage(!par), V(t) in v_stage(par).
    auto iteration = [&](auto par, auto wrap, int t, f32x16 (&s)[NKB], f32x16 (&sn)[NKB], V8 (&pf)[PV_STEPS],
                         V8 (&pn)[PV_STEPS]) {
      constexpr int P = decltype(par)::value;
      // WRAP: the persistent form's last two iterations of a block; the loads past the block's
      // last tile fetch the next block's K(0), K(1), V(0) and Q (as on the bf16 path). DIAG: as
      // on the bf16 path.
      constexpr bool WRAP = (decltype(wrap)::value & 1) != 0;
      constexpr bool DIAG = (decltype(wrap)::value & 2) != 0;
      const std::integral_constant<int, P> cur{};
      const std::integral_constant<int, 1 - P> nxt{};
      // K(t+2) replaces K(t) (read in iteration t-1; K(0) by the first tile, before the barrier
      // above); V(t+1) replaces V(t-1) (V(1) came with the prologue). Issued first so they have
      // the whole iteration to land; waited for before its closing barrier.
      if (tile_of(t + 2) < ntiles) load_tile(k_rs, k_src, k_stage(cur), tile_of(t + 2) * BN);
      else if (WRAP && has_next) load_tile(make_rsrc(K + next_base(), head_bytes), k_src, k_stage(cur), (tile_of(t + 2) - ntiles) * BN);
      // (The persistent form also loads V(1) at t = 0: after the first block, V(1) is not in the
      // prologue's loads. For the first block it writes the same data again.)
      if ((PERSIST || t >= 1) && tile_of(t + 1) < ntiles) load_tile(v_rs, v_src, v_stage(nxt), tile_of(t + 1) * BN);
      else if (WRAP && has_next && tile_of(t + 1) == ntiles) load_tile(make_rsrc(V + next_base(), head_bytes), v_src, v_stage(nxt), 0);
      if constexpr (WRAP && P == 1) {
        if (has_next) load_q(make_rsrc(Q + next_base(), head_bytes), (blk_n % num_qblocks) * BM + wave * 32 + lq);
      }
      if ((PERSIST && !DIAG) || tile_of(t) < wave_tiles) {
        const unsigned char* kn = k_stage(nxt);
        const unsigned char* vc = v_stage(cur);
        // Persistent form: as on the bf16 path, the wrap copies of a RAGGED block take the
        // generic path, the last wrap copy always does, every other iteration the fast path.
        const bool fast = DIAG ? (!(WRAP && P == 1) && t < wave_tiles)
                               : PERSIST ? (!(WRAP && P == 1) && !(WRAP && RAGGED)) : (tile_of(t + 1) < clean_tiles);
        if (fast) {
          // Fast path, straight-line. Phase A: S(t+1) MFMAs with the exp2/round of S(t) and,
          // if m moved, the rescale of O and l. Two copies so the common case carries no muls.
          auto phase_a = [&](auto with_rescale) {
            constexpr bool RS = decltype(with_rescale)::value;
            // (the fused_tc d = 64 tile measured fastest at 4 and, in phase B, 8: C3 +0.5 %,
            // C5 +0.6 % over the per-phase totals 5 and 11, within 1 % for 4-6 and 4-11)
            constexpr int VA = (D == 64 && BM == 128 && BN == 64 && !RS)
                                   ? 4 : ((PV_STEPS - QB) * 20 + (RS ? NDB * 16 + 2 : 0) + QK_MFMAS - 1) / QK_MFMAS;
            // Phase A at wave priority 2, as on the bf16 path (causal fp16 d = 64 4x16x1024 +2.1-3.1 %,
            // 1x16x2048 +1.0-1.2 %); not in the key split, which lost 8 % with it (C2, 1x4x8192).
            if constexpr (KSPLIT == 1) __builtin_amdgcn_s_setprio(2);
            qk(sn, kn);
            if constexpr (RS) rescale_o(alpha);
            exp_part(s, pf, QB, PV_STEPS, true);
            // K operand reads run two MFMAs ahead of their use.
            __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
#pragma unroll
            for (int i = 0; i < QK_MFMAS; ++i) {
              __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
              __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
              __builtin_amdgcn_sched_group_barrier(kSchedValu, VA, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (KSPLIT == 1) __builtin_amdgcn_s_setprio(0);
          };
          if (rescale) phase_a(std::true_type{});
          else phase_a(std::false_type{});
          if constexpr (DIAG) {
            if (t + 2 == wave_tiles) mask_diag(sn, (t + 1) * BN);
          }
          // Phase B: PV(t) MFMAs with the row sum of P(t) and the row max of S(t+1).
          constexpr int VB = (D == 64 && BM == 128 && BN == 64) ? 8 : (NKB * 8 + 10 + QB * 20 + PV_MFMAS - 1) / PV_MFMAS;
          pv(pf, vc);
          row_sum(pf);
          alpha = update_max(sn, rescale);
          exp_part(sn, pn, 0, QB, true);
          // V operand reads (two per MFMA) run two MFMAs ahead of their use.
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4, 0);
#pragma unroll
          for (int i = 0; i < PV_MFMAS + PV_STEPS; ++i) {
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedValu, VB, 0);
          }
          __builtin_amdgcn_sched_barrier(0);
          // Keep the first P(t+1) registers made here: their only use is in the next phase A, and
          // without this the compiler moves their exponentials there in every other iteration
          // (across the barrier), leaving that phase A 32 exponentials against 8 MFMAs and the
          // phase B before it none (C3, C5 +0.8 %, 8 fewer VGPRs).
#pragma unroll
          for (int i = 0; i < QB; ++i) asm volatile("" : "+v"(pn[i]));
        } else {
          // Generic path: the next tile is masked or absent.
          const bool ahead = tile_of(t + 1) < wave_tiles;
          if (rescale) rescale_o(alpha);
          exp_part(s, pf, QB, PV_STEPS, false);
          row_sum(pf);
          pv(pf, vc);
          if (ahead) {
            qk(sn, kn);
            if constexpr (!PERSIST || RAGGED) mask(sn, opaque_offset(tile_of(t + 1) * BN));
            alpha = update_max(sn, rescale);
            exp_part(sn, pn, 0, QB, false);
          }
        }
      }
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    };

    const std::false_type no_wrap{};
    if constexpr (!PERSIST) {
      for (int t = 0; t < nit; t += 2) {
        iteration(even, no_wrap, t, sa, sb, pa, pb);
        if (t + 1 < nit) iteration(odd, no_wrap, t + 1, sb, sa, pb, pa);
      }
    } else {
      // Same launch guarantees, block walks and iteration copies as the bf16 path.
      const std::true_type with_wrap{};
      const std::integral_constant<int, 2> diag{};
      const std::integral_constant<int, 3> diag_wrap{};
      while (true) {
        if constexpr (CAUSAL) {
          blk_n = causal_block(step + 1);
          has_next = blk_n >= 0;
          // Tiles [0, c) are clean in every wave; the per-wave copies start two tiles before c.
          const int c = q0 / BN;
          for (int t = 0; t < c - 2; t += 2) {
            iteration(even, no_wrap, t, sa, sb, pa, pb);
            iteration(odd, no_wrap, t + 1, sb, sa, pb, pa);
          }
          for (int t = max(c - 2, 0); t < ntiles - 2; t += 2) {
            iteration(even, diag, t, sa, sb, pa, pb);
            iteration(odd, diag, t + 1, sb, sa, pb, pa);
          }
          iteration(even, diag_wrap, ntiles - 2, sa, sb, pa, pb);
          iteration(odd, diag_wrap, ntiles - 1, sb, sa, pb, pa);
        } else {
          blk_n = blk + blk_step;
          has_next = blk_n < blk_end;
          for (int t = 0; t < nit - 2; t += 2) {
            iteration(even, no_wrap, t, sa, sb, pa, pb);
            iteration(odd, no_wrap, t + 1, sb, sa, pb, pa);
          }
          iteration(even, with_wrap, nit - 2, sa, sb, pa, pb);
          iteration(odd, with_wrap, nit - 1, sb, sa, pb, pa);
        }
        store_block();
        if (!has_next) break;
        ++step;
        blk = blk_n;
        q0 = (blk % num_qblocks) * BM;
        q0w = q0 + wave * 32;
        qrow = q0w + lq;
        if constexpr (CAUSAL) {
          ntiles = (min(N, q0 + BM) + 2 * BN - 1) / (2 * BN) * 2;
          wave_tiles = (q0w + 32 + BN - 1) / BN;
        }
        base = (size_t)(blk / num_qblocks) * N * D;
        q_rs = make_rsrc(Q + base, head_bytes);
        k_rs = make_rsrc(K + base, head_bytes);
        v_rs = make_rsrc(V + base, head_bytes);
#pragma unroll
        for (int db = 0; db < NDB; ++db) o[db] = f32x16{};
        lacc = f32x4{0.f, 0.f, 0.f, 0.f};
        m_run = -INFINITY;
        rescale = false;
        alpha = 1.f;
        first_tile(sa, pa);
        __syncthreads();
      }
    }
    m_out = m_run;
  } else {
    for (int t = 0; t < ntiles; ++t) {
      const int j0 = t * BN;
      __syncthreads();  // previous tile fully consumed
      load_tile(k_rs, k_src, k_stage(even), j0);
      load_tile(v_rs, v_src, v_stage(even), j0);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (t < wave_tiles) {
        f32x16 s[NKB];
        V8 pf[PV_STEPS];
        bool rescale;
        qk(s, k_stage(even));
        if (t >= clean_tiles) mask(s, j0);
        const float alpha = update_max(s, rescale);
        if (rescale) rescale_o(alpha);
        exponentiate(s, pf);
        row_sum(pf);
        pv(pf, v_stage(even));
      }
    }
  }

  // ---- Key groups: group 1 hands (m, l, O) to the lane of group 0 that holds the same query and
  // dims, through the (now free) K/V stages; group 0 merges them with the online-softmax rule
  // (m = max, l and O scaled by 2^(m_g - m); a group that saw no key of the row adds nothing).
  if constexpr (KSPLIT == 2) {
    static_assert(NW * NDB * 16 * kWave * 4 <= 2 * L::TILE_BYTES * KSPLIT, "merge fits two stages");
    __syncthreads();   // every group is done with the stages
    float* red_o = reinterpret_cast<float*>(wave < NW / 2 ? k_lds0 : v_lds0) + (wave % (NW / 2)) * (NDB * 16 * kWave);
    float* red_ml = reinterpret_cast<float*>(k_lds1) + wave * 2 * kWave;
    if (g == 1) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) red_o[(db * 16 + r) * kWave + lane] = o[db][r];
      red_ml[lane] = m_out;
      red_ml[kWave + lane] = lacc[0];
    }
    __syncthreads();
    if (g == 0) {
      const float m1 = red_ml[lane], l1 = red_ml[kWave + lane];
      const float m = fmaxf(m_out, m1);
      const float sc0 = (m_out == -INFINITY) ? 0.f : exp2_fast(m_out - m);
      const float sc1 = (m1 == -INFINITY) ? 0.f : exp2_fast(m1 - m);
      lacc = sc0 * lacc + sc1 * l1;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = sc0 * o[db][r] + sc1 * red_o[(db * 16 + r) * kWave + lane];
    }
  }

  // ---- Epilogue (the persistent form stores each block where it ends).
  if constexpr (!PERSIST) store_block();
}

}  // namespace pa
