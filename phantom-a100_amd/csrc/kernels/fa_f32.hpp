// Fused online-softmax attention forward with fp32 arithmetic throughout (the `fused` entry).
//
// Same algorithm and numerics as the reference's v3 kernel
// (/root/reference/csrc/kernels/fused.cuh:26-102): Q pre-scaled by log2(e)/sqrt(d) in fp32
// registers, scores, running max/sum and P all fp32 (P is never rounded), inputs fp32 or fp16
// widened to fp32 when staged. On gfx950 both products run on the fp32 matrix core
// (v_mfma_f32_32x32x2_f32) instead of one thread per row on scalar FMAs:
//   S^T (keys x queries) = K . Q^T   A = K from LDS (ds_read_b128 feeds 4 k-steps),
//                                    B = scaled Q^T in VGPRs, k-slot h of step kk = dim h*D/2+kk
//   O^T (d x queries)   += V^T . P^T  B = P^T straight from the S^T accumulator (k-slot h of
//                                    step r = key 8*(r/4) + 4*h + r%4), A = V read row-major
//                                    from LDS (32 consecutive dims per half-wave, no transpose)
// Each wave owns 32 query rows; lane l keeps all state of query l%32 (see fa_mfma.hpp).
#pragma once

#include "common.hpp"

namespace pa {

template <int D, int BN>
struct F32Lds {
  static constexpr int LDK = D + 4;   // +16 B: 8/16 consecutive K rows at one column hit distinct banks
  static constexpr int LDV = D + 8;   // +32 B: the two half-waves read rows 4 apart on distinct banks
  static constexpr int BYTES = BN * (LDK + LDV) * 4;
};

template <typename T, int D, int BM, int BN, typename OutT>
__global__ void __launch_bounds__(BM / 32 * kWave)
fa_f32_fwd(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
           OutT* __restrict__ O, int N, int num_qblocks, int total_blocks, float scale_log2, int causal) {
  typedef F32Lds<D, BN> L;
  constexpr int NW = BM / 32;
  constexpr int THREADS = NW * kWave;
  constexpr int NKB = BN / 32;
  constexpr int NDB = D / 32;
  constexpr int HALF = D / 2;
  constexpr int QUADS = BN * D / 4;          // 4-element groups per K/V tile
  static_assert(D % 32 == 0 && BN % 32 == 0 && BM % 32 == 0, "tile shape");
  static_assert(QUADS % THREADS == 0, "K/V tile must split evenly over the workgroup");
  constexpr int QPT = QUADS / THREADS;

  __shared__ __attribute__((aligned(16))) float ks[BN * L::LDK];
  __shared__ __attribute__((aligned(16))) float vs[BN * L::LDV];

  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int lq = lane % 32;
  const int hi = lane / 32;

  const int blk = xcd_remap(blockIdx.x, total_blocks);
  const int bh = blk / num_qblocks;
  int qb = blk % num_qblocks;
  if (causal) qb = num_qblocks - 1 - qb;
  const int q0 = qb * BM;
  const int q0w = q0 + wave * 32;
  const int qrow = q0w + lq;
  const size_t base = (size_t)bh * N * D;
  const T* __restrict__ Qb = Q + base;
  const T* __restrict__ Kb = K + base;
  const T* __restrict__ Vb = V + base;

  // Scaled Q^T operand: k-slot `hi` of step kk is dim hi*HALF + kk.
  float qf[HALF];
  {
    const bool ok = qrow < N;
#pragma unroll
    for (int c = 0; c < HALF; ++c) qf[c] = ok ? to_f32(Qb[(size_t)qrow * D + hi * HALF + c]) * scale_log2 : 0.f;
  }

  float m_run = -INFINITY, l_run = 0.f;
  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = f32x16{};

  const int kv_end = causal ? min(N, q0 + BM) : N;
  const int wave_kv_end = causal ? min(kv_end, q0w + 32) : kv_end;

  for (int j0 = 0; j0 < kv_end; j0 += BN) {
    // Stage K/V rows [j0, j0 + BN) as fp32 (zeros past N).
    float4 kq[QPT], vq[QPT];
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int c = tid + i * THREADS;
      const int row = c / (D / 4), col = (c % (D / 4)) * 4;
      const int key = j0 + row;
      float4 kk = {0.f, 0.f, 0.f, 0.f}, vv = {0.f, 0.f, 0.f, 0.f};
      if (key < N) {
        const T* kp = Kb + (size_t)key * D + col;
        const T* vp = Vb + (size_t)key * D + col;
        kk = make_float4(to_f32(kp[0]), to_f32(kp[1]), to_f32(kp[2]), to_f32(kp[3]));
        vv = make_float4(to_f32(vp[0]), to_f32(vp[1]), to_f32(vp[2]), to_f32(vp[3]));
      }
      kq[i] = kk;
      vq[i] = vv;
    }
    __syncthreads();  // previous tile fully consumed
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int c = tid + i * THREADS;
      const int row = c / (D / 4), col = (c % (D / 4)) * 4;
      *reinterpret_cast<float4*>(ks + row * L::LDK + col) = kq[i];
      *reinterpret_cast<float4*>(vs + row * L::LDV + col) = vq[i];
    }
    __syncthreads();
    if (j0 >= wave_kv_end) continue;  // causal: no key of this tile is visible to this wave

    f32x16 s[NKB];
#pragma unroll
    for (int b = 0; b < NKB; ++b) {
      s[b] = f32x16{};
#pragma unroll
      for (int u = 0; u < HALF / 4; ++u) {
        const float4 kf = *reinterpret_cast<const float4*>(ks + (b * 32 + lq) * L::LDK + hi * HALF + 4 * u);
        s[b] = mfma32x32x2(kf.x, qf[4 * u + 0], s[b]);
        s[b] = mfma32x32x2(kf.y, qf[4 * u + 1], s[b]);
        s[b] = mfma32x32x2(kf.z, qf[4 * u + 2], s[b]);
        s[b] = mfma32x32x2(kf.w, qf[4 * u + 3], s[b]);
      }
    }

    const bool need_mask = (j0 + BN > N) || (causal && j0 + BN - 1 > q0w);
    if (need_mask) {
#pragma unroll
      for (int b = 0; b < NKB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = j0 + b * 32 + (r / 4) * 8 + hi * 4 + (r % 4);
          if (key >= N || (causal && key > qrow)) s[b][r] = -INFINITY;
        }
    }

    float mx = -INFINITY;
#pragma unroll
    for (int b = 0; b < NKB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[b][r]);
    mx = half_max(mx);
    const float m_new = fmaxf(m_run, mx);
    // A row whose keys are all masked so far keeps l = 0 and O = 0 (the reference skips the
    // update, /root/reference/csrc/kernels/fused.cuh:78); alpha = 0 and P = 0 give the same
    // state without a lane-divergent branch around the MFMAs.
    const bool dead = (m_new == -INFINITY);
    const float alpha = dead ? 0.f : exp2_fast(m_run - m_new);
    const float sub_m = dead ? 0.f : m_new;
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] *= alpha;

#pragma unroll
    for (int b = 0; b < NKB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = exp2_fast(s[b][r] - sub_m);
        l_run += p;
        const int key = b * 32 + (r / 4) * 8 + hi * 4 + (r % 4);
#pragma unroll
        for (int db = 0; db < NDB; ++db) o[db] = mfma32x32x2(vs[key * L::LDV + db * 32 + lq], p, o[db]);
      }
  }

  const float l_tot = half_sum(l_run);
  const float inv = 1.f / l_tot;
  if (qrow < N) {
    OutT* orow = O + base + (size_t)qrow * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        typedef OutT OutV4 __attribute__((ext_vector_type(4)));
        OutV4 w;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) w[rr] = from_f32<OutT>(o[db][g4 * 4 + rr] * inv);
        *reinterpret_cast<OutV4*>(orow + db * 32 + g4 * 8 + hi * 4) = w;
      }
  }
}

}  // namespace pa
