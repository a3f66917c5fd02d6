// Unfused attention paths (the `naive` and `tiled` entries): the full fp32 score matrix S is
// written to a caller-provided [BH][N][N] workspace, normalised in place, then multiplied by V.
// They exist for API completeness and as an independent GPU cross-check of the fused kernels;
// any head dim d >= 1 is accepted, fp32 or fp16 storage, fp32 arithmetic.
//
//   naive (/root/reference/csrc/kernels/naive.cuh:10-64): one thread per score, one thread per
//         softmax row (three passes: max, sum, normalise), one thread per output element.
//   tiled (/root/reference/csrc/kernels/tiled.cuh:16-117): 64x64 output tiles with 4x4 register
//         blocking per thread and LDS-staged operands for both products; softmax with one wave
//         per row (online max/sum per lane, then a 6-step butterfly merge across the 64 lanes);
//         causal P.V skips key tiles right of the diagonal.
#pragma once

#include "common.hpp"

namespace pa {

// ------------------------------------------------------------------------------------ naive
template <typename T>
__global__ void __launch_bounds__(256)
naive_scores(const T* __restrict__ Q, const T* __restrict__ K, float* __restrict__ S, int N, int d,
             float scale, int causal) {
  const int bh = blockIdx.z;
  const int i = blockIdx.y * 4 + threadIdx.y;
  const int j = blockIdx.x * 64 + threadIdx.x;
  if (i >= N || j >= N) return;
  const T* q = Q + ((size_t)bh * N + i) * d;
  const T* k = K + ((size_t)bh * N + j) * d;
  float acc = 0.f;
  for (int c = 0; c < d; ++c) acc = fmaf(to_f32(q[c]), to_f32(k[c]), acc);
  S[((size_t)bh * N + i) * N + j] = (causal && j > i) ? -INFINITY : acc * scale;
}

__global__ void __launch_bounds__(256)
naive_softmax(float* __restrict__ S, int N) {
  const int bh = blockIdx.y;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= N) return;
  float* row = S + ((size_t)bh * N + i) * N;
  float m = -INFINITY;
  for (int j = 0; j < N; ++j) m = fmaxf(m, row[j]);
  float l = 0.f;
  for (int j = 0; j < N; ++j) l += expf(row[j] - m);
  const float inv = 1.f / l;
  for (int j = 0; j < N; ++j) row[j] = expf(row[j] - m) * inv;
}

template <typename T>
__global__ void __launch_bounds__(256)
naive_pv(const float* __restrict__ P, const T* __restrict__ V, T* __restrict__ O, int N, int d) {
  const int bh = blockIdx.z;
  const int i = blockIdx.y * 4 + threadIdx.y;
  const int c = blockIdx.x * 64 + threadIdx.x;
  if (i >= N || c >= d) return;
  const float* p = P + ((size_t)bh * N + i) * N;
  const T* v = V + (size_t)bh * N * d;
  float acc = 0.f;
  for (int j = 0; j < N; ++j) acc = fmaf(p[j], to_f32(v[(size_t)j * d + c]), acc);
  O[((size_t)bh * N + i) * d + c] = from_f32<T>(acc);
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

// Merge partial softmax states (m, l) with l = sum exp(x - m); empty states have m = -inf.
__device__ __forceinline__ void merge_state(float& m, float& l, float m2, float l2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  l = l * expf(m - mn) + l2 * expf(m2 - mn);
  m = mn;
}

// One wave per row, 4 rows per 256-thread workgroup.
__global__ void __launch_bounds__(256)
tiled_softmax(float* __restrict__ S, int N) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int bh = blockIdx.y;
  const int i = blockIdx.x * 4 + wave;
  if (i >= N) return;  // whole wave leaves together
  float* row = S + ((size_t)bh * N + i) * N;
  float m = -INFINITY, l = 0.f;
  for (int j = lane; j < N; j += kWave) {
    const float x = row[j];
    if (x > m) {
      l = l * expf(m - x) + 1.f;
      m = x;
    } else if (x != -INFINITY) {
      l += expf(x - m);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float m2 = __shfl_xor(m, off);
    const float l2 = __shfl_xor(l, off);
    merge_state(m, l, m2, l2);
  }
  const float inv = 1.f / l;
  for (int j = lane; j < N; j += kWave) row[j] = expf(row[j] - m) * inv;
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
