// Unfused attention paths (the `naive` and `tiled` entries): the full fp32 score matrix S is
// written to a caller-provided [BH][N][N] workspace, normalised in place, then multiplied by V.
// They exist for API completeness and as an independent GPU cross-check of the fused kernels;
// any head dim d >= 1 is accepted, fp32 or fp16 storage, fp32 arithmetic.
//
//   naive (/root/reference/csrc/kernels/naive.cuh:10-64): the same three passes (scores, softmax
//         by row max / sum / normalise, P.V) as plain loops, one wave per row of each product.
//   tiled (/root/reference/csrc/kernels/tiled.cuh:16-117): both products on the matrix core
//         for fp16 inputs (scores at d a multiple of 16, P.V at d = 64 / 128) and for fp32 inputs
//         at d = 64 / 128 (tiled_*_mfma, tiled_*_mfma_f32); otherwise 64x64 output tiles with 4x4
//         register blocking per thread and LDS-staged operands. Softmax with one wave per row,
//         the row held in registers up to 8192 keys (one read of S); longer rows take one
//         workgroup per row, in register-held segments whose max the workgroup agrees on before
//         their sums (one read of S up to 32768 keys, two beyond). Causal P.V skips key tiles
//         right of the diagonal.
#pragma once

#include "common.hpp"
#include "fa_mfma.hpp"   // v_swz: the V tile layout of the fused kernel, reused by tiled_pv_mfma

namespace pa {

// ------------------------------------------------------------------------------------ naive
// The reference's three unfused passes, each a plain loop per lane, laid out by waves: every
// workgroup is 4 waves, and a wave owns one row of the product it writes (64 keys of a score row,
// a whole softmax row, 64 head dims of an output row), so the operand that row shares (the query
// row, the P row) is the same address in every lane, and the per-lane operand (a K row, a V
// column) is a different one. Grids are flattened into x: N rows times column blocks.

// S[h][i][j0 + lane] for the wave's query row i and 64 keys from j0; keys after i are -inf when
// causal. PIECES (rows of whole 16-byte pieces, 16-byte aligned): each lane reads its K row, and
// the wave its Q row, a 16-byte piece per load instead of an element per load (one load then
// touches the wave's 64 K rows once per piece, not once per element); the products are summed in
// the same order either way.
template <typename T, bool PIECES>
__global__ void __launch_bounds__(256)
naive_scores(const T* __restrict__ Q, const T* __restrict__ K, float* __restrict__ S, int N, int d,
             float scale, int causal, int key_blocks) {
  const int unit = (int)blockIdx.x * 4 + (int)threadIdx.x / kWave;   // (query row, 64-key block)
  const int i = unit / key_blocks;
  const int j = (unit % key_blocks) * kWave + (int)threadIdx.x % kWave;
  if (i >= N || j >= N) return;
  const size_t head = (size_t)blockIdx.y * N;
  float* srow = S + (head + i) * N;
  if (causal && j > i) {   // masked: the product is not needed
    srow[j] = -INFINITY;
    return;
  }
  const T* qi = Q + (head + i) * d;
  const T* kj = K + (head + j) * d;
  float dot = 0.f;
  if constexpr (PIECES) {
    constexpr int E = 16 / (int)sizeof(T);   // elements per piece
    for (int c = 0; c < d; c += E) {
      // (the loaded vector is bit-cast as a whole before its elements are taken)
      const u32x4 qw = *reinterpret_cast<const u32x4*>(qi + c);
      const u32x4 kw = *reinterpret_cast<const u32x4*>(kj + c);
      if constexpr (sizeof(T) == 4) {
        const f32x4 qv = __builtin_bit_cast(f32x4, qw), kv = __builtin_bit_cast(f32x4, kw);
#pragma unroll
        for (int e = 0; e < E; ++e) dot = fmaf(qv[e], kv[e], dot);
      } else {
        const typename vec8<T>::type qv = __builtin_bit_cast(typename vec8<T>::type, qw);
        const typename vec8<T>::type kv = __builtin_bit_cast(typename vec8<T>::type, kw);
#pragma unroll
        for (int e = 0; e < E; ++e) dot = fmaf(to_f32(qv[e]), to_f32(kv[e]), dot);
      }
    }
  } else {
    for (int c = 0; c < d; ++c) dot = fmaf(to_f32(qi[c]), to_f32(kj[c]), dot);
  }
  srow[j] = scale * dot;
}

// Row r of S in place: max, sum of exp(s - max), then exp(s - max) / sum, each a strided pass
// of the wave's 64 lanes over the row followed by a wave all-reduce (DPP and lane swaps).
__global__ void __launch_bounds__(256)
naive_softmax(float* __restrict__ S, int N, long long rows) {
  const long long r = (long long)blockIdx.x * 4 + threadIdx.x / kWave;
  if (r >= rows) return;
  const int lane = (int)threadIdx.x % kWave;
  float* srow = S + r * N;
  float mx = -INFINITY;
  for (int j = lane; j < N; j += kWave) mx = fmaxf(mx, srow[j]);
  mx = wave_allreduce(mx, MaxOp{});
  float sum = 0.f;
  for (int j = lane; j < N; j += kWave) sum += expf(srow[j] - mx);
  sum = wave_allreduce(sum, SumOp{});
  const float rcp = 1.f / sum;
  for (int j = lane; j < N; j += kWave) srow[j] = expf(srow[j] - mx) * rcp;
}

// O[h][i][c0 + lane] = sum over keys j of P[h][i][j] V[h][j][c0 + lane], for the wave's row i and
// 64 head dims from c0. PIECES (N a multiple of 4, P 16-byte aligned): the wave reads its P row
// four probabilities per load; the products are summed in the same order either way.
template <typename T, bool PIECES>
__global__ void __launch_bounds__(256)
naive_pv(const float* __restrict__ P, const T* __restrict__ V, T* __restrict__ O, int N, int d, int dim_blocks) {
  const int unit = (int)blockIdx.x * 4 + (int)threadIdx.x / kWave;   // (query row, 64-dim block)
  const int i = unit / dim_blocks;
  const int c = (unit % dim_blocks) * kWave + (int)threadIdx.x % kWave;
  if (i >= N || c >= d) return;
  const size_t head = (size_t)blockIdx.y * N;
  const float* pi = P + (head + i) * N;
  const T* vc = V + head * d + c;
  float acc = 0.f;
  if constexpr (PIECES) {
    for (int j = 0; j < N; j += 4) {
      const f32x4 p4 = *reinterpret_cast<const f32x4*>(pi + j);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = fmaf(p4[e], to_f32(vc[(size_t)(j + e) * d]), acc);
    }
  } else {
    for (int j = 0; j < N; ++j) acc = fmaf(pi[j], to_f32(vc[(size_t)j * d]), acc);
  }
  O[(head + i) * d + c] = from_f32<T>(acc);
}

// ------------------------------------------------------------------------------------ tiled
constexpr int kTile = 64;   // output tile edge
constexpr int kTk = 16;     // reduction chunk

// S[i0:i0+64, j0:j0+64] = scale * Q_tile . K_tile^T (keys after the query -> -inf when causal).
// Operands are staged transposed ([k][row]) so each thread reads its 4 rows / 4 columns as one
// float4 from LDS.
template <typename T>
__global__ void __launch_bounds__(256)
tiled_scores(const T* __restrict__ Q, const T* __restrict__ K, float* __restrict__ S, int N, int d,
             float scale, int causal) {
  __shared__ __attribute__((aligned(16))) float qs[kTk][kTile + 4];
  __shared__ __attribute__((aligned(16))) float ksm[kTk][kTile + 4];
  const int bh = blockIdx.z;
  const int i0 = blockIdx.y * kTile, j0 = blockIdx.x * kTile;
  const int tid = threadIdx.x, tx = tid % 16, ty = tid / 16;
  const T* Qb = Q + (size_t)bh * N * d;
  const T* Kb = K + (size_t)bh * N * d;
  float acc[4][4] = {};
  for (int c0 = 0; c0 < d; c0 += kTk) {
    // 64 rows x 16 dims per operand = 1024 elements, 4 per thread; consecutive threads read
    // consecutive dims of one row.
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int idx = tid + e * 256;
      const int r = idx / kTk, c = idx % kTk;
      const int qi = i0 + r, kj = j0 + r, cc = c0 + c;
      qs[c][r] = (qi < N && cc < d) ? to_f32(Qb[(size_t)qi * d + cc]) : 0.f;
      ksm[c][r] = (kj < N && cc < d) ? to_f32(Kb[(size_t)kj * d + cc]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kTk; ++c) {
      const float4 a = *reinterpret_cast<const float4*>(&qs[c][ty * 4]);
      const float4 b = *reinterpret_cast<const float4*>(&ksm[c][tx * 4]);
      const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int w = 0; w < 4; ++w) acc[u][w] = fmaf(av[u], bv[w], acc[u][w]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = i0 + ty * 4 + u;
    if (i >= N) continue;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int j = j0 + tx * 4 + w;
      if (j < N) S[((size_t)bh * N + i) * N + j] = (causal && j > i) ? -INFINITY : acc[u][w] * scale;
    }
  }
}

// S = scale * Q K^T on the matrix core, for fp16 storage and d = 16 * KSTEPS (the tiled_scores
// result up to the order of the fp32 sums: products of fp16 values are exact in fp32). A 128 x 128
// tile per workgroup, a 64 x 64 quarter per wave as 2 x 2 v_mfma_f32_32x32x16_f16 blocks, whose
// operands are read straight from memory in the MFMA layout: lane l takes dims
// 16 kk + 8 (l / 32) .. + 7 of row l % 32 of its 32-row block (16 bytes, rows 16-byte aligned);
// rows past N read as zero through the buffer's range. Register r of a block holds row
// 8 (r / 4) + 4 (l / 32) + r % 4 and column l % 32, so each store instruction writes 128
// contiguous bytes of two rows. With causal, a quarter entirely right of the diagonal skips its
// products and stores -inf.
template <int KSTEPS>
__global__ void __launch_bounds__(256)
tiled_scores_mfma(const f16* __restrict__ Q, const f16* __restrict__ K, float* __restrict__ S, int N,
                  float scale, int causal) {
  constexpr int D = 16 * KSTEPS;
  const int bh = blockIdx.z;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int r0 = blockIdx.y * 128 + (wave / 2) * 64;
  const int c0 = blockIdx.x * 128 + (wave % 2) * 64;
  const int lr = lane % 32, hk = lane / 32;
  const uint32_t head_bytes = (uint32_t)((size_t)N * D * sizeof(f16));
  const rsrc_t q_rs = make_rsrc(Q + (size_t)bh * N * D, head_bytes);
  const rsrc_t k_rs = make_rsrc(K + (size_t)bh * N * D, head_bytes);
  f32x16 acc[2][2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) acc[rb][cb] = f32x16{};
  if (!(causal && c0 > r0 + 63)) {
    f16x8 a[KSTEPS][2], b[KSTEPS][2];
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk)
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        a[kk][x] = __builtin_bit_cast(f16x8, load16(q_rs, (uint32_t)(((r0 + 32 * x + lr) * D + 16 * kk + 8 * hk) * 2)));
        b[kk][x] = __builtin_bit_cast(f16x8, load16(k_rs, (uint32_t)(((c0 + 32 * x + lr) * D + 16 * kk + 8 * hk) * 2)));
      }
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) acc[rb][cb] = mfma32x32x16(a[kk][rb], b[kk][cb], acc[rb][cb]);
  }
  float* Sb = S + (size_t)bh * N * N;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = r0 + 32 * rb + 8 * (r / 4) + 4 * hk + r % 4;
        const int j = c0 + 32 * cb + lr;
        if (i < N && j < N) Sb[(size_t)i * N + j] = (causal && j > i) ? -INFINITY : acc[rb][cb][r] * scale;
      }
}

// S = scale * Q K^T on the fp32 matrix core (v_mfma_f32_32x32x2_f32) for fp32 storage and
// D in {64, 128}; the tiled_scores result up to the order of its fp32 sums. 128 x 128 tile per
// workgroup, 64 x 64 per wave as 2 x 2 blocks. The dot product's dims are walked in an order that
// keeps every lane's reads contiguous: within each 64-dim chunk, k-step kk of lane l takes dim
// 32 (l / 32) + kk of its row (l % 32 of the block), in Q and K alike, so a lane reads 32
// consecutive floats (8 x 16 bytes) per row and chunk. Rows past N read as zero.
template <int D>
__global__ void __launch_bounds__(256)
tiled_scores_mfma_f32(const float* __restrict__ Q, const float* __restrict__ K, float* __restrict__ S, int N,
                      float scale, int causal) {
  static_assert(D % 64 == 0, "64-dim chunks");
  const int bh = blockIdx.z;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int r0 = blockIdx.y * 128 + (wave / 2) * 64;
  const int c0 = blockIdx.x * 128 + (wave % 2) * 64;
  const int lr = lane % 32, hk = lane / 32;
  const uint32_t head_bytes = (uint32_t)((size_t)N * D * sizeof(float));
  const rsrc_t q_rs = make_rsrc(Q + (size_t)bh * N * D, head_bytes);
  const rsrc_t k_rs = make_rsrc(K + (size_t)bh * N * D, head_bytes);
  f32x16 acc[2][2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) acc[rb][cb] = f32x16{};
  if (!(causal && c0 > r0 + 63)) {
#pragma unroll 1
    for (int ch = 0; ch < D / 64; ++ch) {
      f32x4 a[2][8], b[2][8];
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const uint32_t col = (uint32_t)(64 * ch + 32 * hk + 4 * v);
          a[x][v] = __builtin_bit_cast(f32x4, load16(q_rs, (uint32_t)((r0 + 32 * x + lr) * D + col) * 4));
          b[x][v] = __builtin_bit_cast(f32x4, load16(k_rs, (uint32_t)((c0 + 32 * x + lr) * D + col) * 4));
        }
#pragma unroll
      for (int kk = 0; kk < 32; ++kk)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int cb = 0; cb < 2; ++cb)
            acc[rb][cb] = mfma32x32x2(a[rb][kk / 4][kk % 4], b[cb][kk / 4][kk % 4], acc[rb][cb]);
    }
  }
  float* Sb = S + (size_t)bh * N * N;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = r0 + 32 * rb + 8 * (r / 4) + 4 * hk + r % 4;
        const int j = c0 + 32 * cb + lr;
        if (i < N && j < N) Sb[(size_t)i * N + j] = (causal && j > i) ? -INFINITY : acc[rb][cb][r] * scale;
      }
}

// One wave per row, the whole row held in registers (rows of at most 64 * VPL keys): S is read
// once and P written once, 8 bytes per score (the naive softmax reads S three times). The max
// first, then the sum of exp(x - max) kept in place, then P = e / sum; element j of the row sits in
// lane j % 64, slot j / 64, so every load and store of a wave covers 256 contiguous bytes.
template <int VPL>
__global__ void __launch_bounds__(256)
tiled_softmax_rows(float* __restrict__ S, int N) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int bh = blockIdx.y;
  const int i = blockIdx.x * 4 + wave;
  if (i >= N) return;  // whole wave leaves together
  float* row = S + ((size_t)bh * N + i) * N;
  float x[VPL];
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int j = lane + k * kWave;
    x[k] = j < N ? row[j] : -INFINITY;
    m = fmaxf(m, x[k]);
  }
  m = wave_allreduce(m, MaxOp{});
  float l = 0.f;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    x[k] = expf(x[k] - m);   // -inf (masked or past N) -> 0; every row has a finite score
    l += x[k];
  }
  l = wave_allreduce(l, SumOp{});
  const float inv = 1.f / l;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int j = lane + k * kWave;
    if (j < N) row[j] = x[k] * inv;
  }
}

// Rows longer than the one-wave register kernel holds (N > 64 * 128): one 256-lane workgroup per
// row. The row is cut into segments of 256 * VPL keys, each held in registers (key
// j0 + 256 k + t in slot k of thread t, so every load and store of a wave covers 256 contiguous
// bytes). Per segment, the workgroup first agrees on the segment's max (wave all-reduce, then the
// four wave maxima through LDS); where it exceeds the row's running max m, the per-thread sums are
// multiplied by exp(m - m_new) once, and then every key of the segment adds exp(x - m) against the
// same, workgroup-uniform m. So m needs no per-lane state and the end is a plain sum. A row of one
// segment (N <= 256 * VPL) keeps its exponentials in registers and writes P from them (S read
// once); longer rows read each segment again for P = exp(x - m) / l.
template <int VPL>
__global__ void __launch_bounds__(256)
tiled_softmax_segments(float* __restrict__ S, int N) {
  constexpr int SEG = 256 * VPL;
  // Two slots so that consecutive reductions need one barrier each: reduction r writes slot r % 2
  // after every thread has passed reduction r - 1's barrier, i.e. after the reads of slot r % 2 by
  // reduction r - 2.
  __shared__ float part[2][4];
  const int t = (int)threadIdx.x, wave = t / kWave, lane = t % kWave;
  float* row = S + ((size_t)blockIdx.y * N + blockIdx.x) * N;
  int slot = 0;
  auto block_reduce = [&](float v, auto op) {
    v = wave_allreduce(v, op);
    if (lane == 0) part[slot][wave] = v;
    __syncthreads();
    const float r = op(op(part[slot][0], part[slot][1]), op(part[slot][2], part[slot][3]));
    slot ^= 1;
    return r;
  };
  const int segments = (N + SEG - 1) / SEG;
  float x[VPL];
  float m = -INFINITY, l = 0.f;
  for (int sg = 0; sg < segments; ++sg) {
    const int j0 = sg * SEG;
    float smax = -INFINITY;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int j = j0 + k * 256 + t;
      x[k] = j < N ? row[j] : -INFINITY;
      smax = fmaxf(smax, x[k]);
    }
    smax = block_reduce(smax, MaxOp{});
    if (smax > m) {   // workgroup-uniform; l is still 0 while m is -inf
      l = m == -INFINITY ? 0.f : l * expf(m - smax);
      m = smax;
    }
    // Key 0 is visible in every row (causal or not), so m is finite from the first segment on.
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      x[k] = expf(x[k] - m);   // masked or past N: exp(-inf) = 0
      l += x[k];
    }
  }
  const float inv = 1.f / block_reduce(l, SumOp{});
  if (segments == 1) {
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int j = k * 256 + t;
      if (j < N) row[j] = x[k] * inv;
    }
  } else {
    for (int j = t; j < N; j += 256) row[j] = expf(row[j] - m) * inv;
  }
}

// O = P V on the matrix core for fp16 V with D in {64, 128} (the fused kernel's V operand path),
// computed transposed as O^T += V^T P^T per 16-key step with v_mfma_f32_32x32x16_f16: A = V^T,
// read from a swizzled LDS tile of 64 keys with ds_read_b64_tr_b16; B = P^T, lane l taking the 8
// probabilities of its query row l % 32 at the keys the V reads pair with them (two runs of 4
// consecutive keys) straight from the fp32 workspace. P is fed as two fp16 terms of 1024 P
// (hi = round(1024 P), lo = round(1024 P - hi)): ~22 significant bits while lo is a normal fp16
// (|lo| ~ 2^-11 |hi| >= 2^-14, i.e. P >= ~2^-13); below that lo lands on fp16's subnormal spacing
// 2^-24, so the pair is off by at most 2^-25 in 1024 P, 2^-35 in P. Both products are exact in
// fp32 and summed in fp32; O is scaled back by 2^-10. 128 queries per workgroup (32 per wave),
// two V stages; the next tile's V (to LDS) and P (to registers) load during the current one.
// Reads past the head (query or key rows past N) return zero through the buffers' ranges, and
// keys past N meet zero V rows. With causal, keys after the block's last query are skipped (their
// P is zero).
template <int D>
__global__ void __launch_bounds__(256)
tiled_pv_mfma(const float* __restrict__ P, const f16* __restrict__ V, f16* __restrict__ O, int N, int causal) {
  constexpr int BN = 64, THREADS = 256, NDB = D / 32, CR = D / 8, RB = D * 2;
  constexpr int TILE_BYTES = BN * RB;
  constexpr int CPT = BN * CR / THREADS;   // 16-byte V chunks per thread per tile
  static_assert(D == 64 || D == 128, "V layout of the fused kernel");
  __shared__ __attribute__((aligned(1024))) unsigned char v_lds[2 * TILE_BYTES];
  const int bh = blockIdx.y;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int lq = lane % 32, hi = lane / 32;
  const int q0 = blockIdx.x * 128;
  const int qrow = q0 + wave * 32 + lq;
  const rsrc_t v_rs = make_rsrc(V + (size_t)bh * N * D, (uint32_t)((size_t)N * D * sizeof(f16)));
  const rsrc_t p_rs = make_rsrc(P + (size_t)bh * N * N, (uint32_t)((size_t)N * N * sizeof(float)));
  uint32_t v_src[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int slot = i * THREADS + tid;
    const int row = slot / CR, pc = slot % CR;
    v_src[i] = (uint32_t)(row * RB + ((pc ^ v_swz<CR>(row)) * 16));
  }
  auto load_v = [&](int stage, int k0) {
#pragma unroll
    for (int i = 0; i < CPT; ++i)
      load16_to_lds(v_rs, v_lds + stage * TILE_BYTES + (i * THREADS + wave * kWave) * 16, v_src[i], (uint32_t)(k0 * RB));
  };
  const int g16 = lane / 16, i16 = lane % 16;
  const int v_row = hi * 4 + i16 / 4;
  const int v_cl = 2 * (g16 % 2) + (i16 % 4) / 2;
  int v_addr[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
    v_addr[db] = v_row * RB + (((4 * db + v_cl) ^ v_swz<CR>(v_row)) * 16) + 8 * (i16 % 2);
  // P^T operands of one 64-key tile: for 16-key step ks, k-slot j of this lane holds key
  // 16 ks + 8 (j / 4) + 4 hi + j % 4 of its query row, the key order in which the transposed
  // V reads hand out the A operand (rows 4 hi .. 4 hi + 3, then 8 + 4 hi .. 8 + 4 hi + 3).
  auto load_p = [&](u32x4 (&pr)[8], int k0) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        pr[2 * ks + h] = load16(p_rs, (uint32_t)(((size_t)qrow * N + k0 + 16 * ks + 8 * h + 4 * hi) * sizeof(float)));
  };
  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = f32x16{};
  const int k_end = causal ? min(N, q0 + 128) : N;
  const int ntiles = (k_end + BN - 1) / BN;
  u32x4 pc[8], pn[8];
  load_v(0, 0);
  load_p(pc, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    if (t + 1 < ntiles) {
      load_v((t + 1) & 1, (t + 1) * BN);
      load_p(pn, (t + 1) * BN);
    }
    const unsigned char* vs = v_lds + (t & 1) * TILE_BYTES;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      f16x8 ph, pl;
      // (the whole u32x4 is bit-cast to f32x4: casting one element of a loaded u32x4 to float
      // miscompiles with this hipcc, every element then reading element 0)
      const f32x4 p4[2] = {__builtin_bit_cast(f32x4, pc[2 * ks]), __builtin_bit_cast(f32x4, pc[2 * ks + 1])};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float x = 1024.f * p4[j / 4][j % 4];
        const f16 h = (f16)x;
        ph[j] = h;
        pl[j] = (f16)(x - (float)h);
      }
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const unsigned char* p0 = vs + ks * 16 * RB + v_addr[db];
        const i16x4 a0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr<i16x4>)(p0));
        const i16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr<i16x4>)(p0 + 8 * RB));
        const f16x8 a = __builtin_bit_cast(f16x8, i16x8{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]});
        acc[db] = mfma32x32x16(a, ph, acc[db]);
        acc[db] = mfma32x32x16(a, pl, acc[db]);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) pc[i] = pn[i];
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  // Register r of block db holds dim 32 db + 8 (r / 4) + 4 hi + r % 4 of query qrow.
  if (qrow < N) {
    f16* orow = O + ((size_t)bh * N + qrow) * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        typedef f16 F16x4 __attribute__((ext_vector_type(4)));
        F16x4 w;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) w[rr] = (f16)(acc[db][g4 * 4 + rr] * (1.f / 1024.f));
        *reinterpret_cast<F16x4*>(orow + db * 32 + g4 * 8 + hi * 4) = w;
      }
  }
}

// O = P V on the fp32 matrix core for fp32 V and D in {64, 128}: A = P (lane l: 32 consecutive
// probabilities of its query row l % 32 per 64-key tile, the keys of k-step kk being
// 32 (l / 32) + kk, read straight from the workspace), B = V from a 64-key LDS tile (lane l reads
// key 32 (l / 32) + kk, dim l % 32 of its 32-dim block). 128 queries per workgroup, 32 per wave;
// the next tile's V (to LDS) and P (to registers) load during the current one. Reads past the
// head return zero; keys past N meet zero V rows. With causal, keys after the block's last query
// are skipped.
template <int D>
__global__ void __launch_bounds__(256)
tiled_pv_mfma_f32(const float* __restrict__ P, const float* __restrict__ V, float* __restrict__ O, int N, int causal) {
  constexpr int BN = 64, THREADS = 256, NDB = D / 32;
  constexpr int ROW = D + 4;                       // LDS row pitch in floats (padding spreads banks)
  static_assert(D == 64 || D == 128, "head dim");
  __shared__ __attribute__((aligned(16))) float v_lds[2][BN * ROW];
  const int bh = blockIdx.y;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int lq = lane % 32, hi = lane / 32;
  const int q0 = blockIdx.x * 128;
  const int qrow = q0 + wave * 32 + lq;
  const rsrc_t v_rs = make_rsrc(V + (size_t)bh * N * D, (uint32_t)((size_t)N * D * sizeof(float)));
  const rsrc_t p_rs = make_rsrc(P + (size_t)bh * N * N, (uint32_t)((size_t)N * N * sizeof(float)));
  // V tile: 64 keys x D floats, 16 bytes per thread per load, rows of D / 4 chunks.
  constexpr int CH = BN * D / 4 / THREADS;
  auto load_v = [&](u32x4 (&vr)[CH], int k0) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int slot = i * THREADS + tid, row = slot / (D / 4), c4 = slot % (D / 4);
      vr[i] = load16(v_rs, (uint32_t)(((k0 + row) * D + 4 * c4) * 4));
    }
  };
  auto store_v = [&](const u32x4 (&vr)[CH], int stage) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int slot = i * THREADS + tid, row = slot / (D / 4), c4 = slot % (D / 4);
      *reinterpret_cast<f32x4*>(&v_lds[stage][row * ROW + 4 * c4]) = __builtin_bit_cast(f32x4, vr[i]);
    }
  };
  auto load_p = [&](u32x4 (&pr)[8], int k0) {
#pragma unroll
    for (int v = 0; v < 8; ++v)
      pr[v] = load16(p_rs, (uint32_t)(((size_t)qrow * N + k0 + 32 * hi + 4 * v) * sizeof(float)));
  };
  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = f32x16{};
  const int k_end = causal ? min(N, q0 + 128) : N;
  const int ntiles = (k_end + BN - 1) / BN;
  u32x4 vr[CH], pc[8], pn[8];
  load_v(vr, 0);
  load_p(pc, 0);
  store_v(vr, 0);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const bool more = t + 1 < ntiles;
    if (more) {
      load_v(vr, (t + 1) * BN);
      load_p(pn, (t + 1) * BN);
    }
    const float* vs = v_lds[t & 1];
#pragma unroll
    for (int kk = 0; kk < 32; ++kk) {
      const float a = __builtin_bit_cast(f32x4, pc[kk / 4])[kk % 4];
#pragma unroll
      for (int db = 0; db < NDB; ++db) acc[db] = mfma32x32x2(a, vs[(32 * hi + kk) * ROW + 32 * db + lq], acc[db]);
    }
    if (more) store_v(vr, (t + 1) & 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) pc[i] = pn[i];
    __syncthreads();
  }
  // Register r of block db holds query 8 (r / 4) + 4 hi + r % 4 of the wave and dim 32 db + l % 32.
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int q = q0 + wave * 32 + 8 * (r / 4) + 4 * hi + r % 4;
      if (q < N) O[((size_t)bh * N + q) * D + 32 * db + lq] = acc[db][r];
    }
}

// O[i0:i0+64, c0:c0+64] = P_rows . V_cols; with causal, P is zero right of the diagonal so
// the key loop stops at the tile's last row.
template <typename T>
__global__ void __launch_bounds__(256)
tiled_pv(const float* __restrict__ P, const T* __restrict__ V, T* __restrict__ O, int N, int d, int causal) {
  __shared__ __attribute__((aligned(16))) float ps[kTk][kTile + 4];
  __shared__ __attribute__((aligned(16))) float vsm[kTk][kTile + 4];
  const int bh = blockIdx.z;
  const int i0 = blockIdx.y * kTile, c0 = blockIdx.x * kTile;
  const int tid = threadIdx.x, tx = tid % 16, ty = tid / 16;
  const float* Pb = P + (size_t)bh * N * N;
  const T* Vb = V + (size_t)bh * N * d;
  const int k_end = causal ? min(N, i0 + kTile) : N;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < k_end; k0 += kTk) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int idx = tid + e * 256;
      // P: 64 rows x 16 keys, consecutive threads read consecutive keys of one row.
      const int r = idx / kTk, kk = idx % kTk;
      const int pi = i0 + r, pj = k0 + kk;
      ps[kk][r] = (pi < N && pj < N) ? Pb[(size_t)pi * N + pj] : 0.f;
      // V: 16 keys x 64 dims, consecutive threads read consecutive dims of one key.
      const int vk = idx / kTile, vc = idx % kTile;
      const int gk = k0 + vk, gc = c0 + vc;
      vsm[vk][vc] = (gk < N && gc < d) ? to_f32(Vb[(size_t)gk * d + gc]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kTk; ++kk) {
      const float4 a = *reinterpret_cast<const float4*>(&ps[kk][ty * 4]);
      const float4 b = *reinterpret_cast<const float4*>(&vsm[kk][tx * 4]);
      const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int w = 0; w < 4; ++w) acc[u][w] = fmaf(av[u], bv[w], acc[u][w]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = i0 + ty * 4 + u;
    if (i >= N) continue;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int c = c0 + tx * 4 + w;
      if (c < d) O[((size_t)bh * N + i) * d + c] = from_f32<T>(acc[u][w]);
    }
  }
}

}  // namespace pa
