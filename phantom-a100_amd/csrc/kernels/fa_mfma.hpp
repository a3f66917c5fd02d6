// Fused online-softmax attention forward on CDNA4 MFMA (fp16 / bf16 in, fp32 accumulate).
//
// Computes O = softmax(Q K^T / sqrt(d)) V for one (head, BM-query block) per workgroup without
// materialising the N x N scores. Same math as the reference's v4 kernel
// (/root/reference/csrc/kernels/fused_tc.cuh:45-179): scores scaled by log2(e)/sqrt(d) in fp32,
// running max m and sum l per query row, alpha = 2^(m_old - m_new), P rounded to the input
// dtype only as the P.V operand while l sums the unrounded fp32 P, output O / l.
//
// gfx950 design (not a translation of the WMMA kernel):
//  * Each wave owns 32 query rows. Both products are computed transposed so that every
//    per-row quantity stays in one lane:
//        S^T (keys x queries) = K . Q^T        v_mfma_f32_32x32x16_{f16,bf16}, A = K from LDS,
//                                              B = Q^T resident in VGPRs for the whole kernel
//        O^T (d x queries)   += V^T . P^T      A = V^T read from LDS with ds_read_b64_tr_b16,
//                                              B = P^T taken straight from the S^T accumulator
//    In the 32x32 accumulator, lane l holds column l%32 (= one query) and 16 of its 32 rows
//    (keys, or head dims), the other 16 sit in lane l^32. So a row max / row sum is a
//    16-element in-lane reduction plus one v_permlane32_swap, the rescale of O by alpha is
//    lane-local, and P^T needs no LDS round trip: register r of the S^T block holds key
//    8*(r/4) + 4*(l/32) + r%4, exactly the key that the PV MFMA's B operand expects in k-slot
//    8*(l/32) + (r%8) once the A operand (V^T) is read with the same key order.
//  * K and V tiles of BN keys are staged row-major in LDS (16-byte coalesced global loads,
//    16-byte LDS writes). With STAGES == 2 the global loads for tile t+1 are issued before the
//    MFMAs of tile t and written to the other LDS stage afterwards: one barrier per tile.
//  * LDS rows are padded so that the K operand reads (ds_read_b128, 8..16 consecutive rows at
//    one column) and the transposed V reads (4 rows x 32 bytes per 16 lanes) hit distinct banks.
//  * Workgroup ids are remapped so that all query blocks of a head run on one XCD (shared L2).
#pragma once

#include "common.hpp"

namespace pa {

template <int D, int BN, int STAGES>
struct MfmaLds {
  static constexpr int LDK = D + 8;    // K row pitch in elements (+16 B)
  static constexpr int LDV = D + 16;   // V row pitch in elements (+32 B)
  static constexpr int K_ELEMS = BN * LDK;
  static constexpr int V_ELEMS = BN * LDV;
  static constexpr int STAGE_ELEMS = K_ELEMS + V_ELEMS;
  static constexpr int ELEMS = STAGES * STAGE_ELEMS;
  static constexpr int BYTES = ELEMS * 2;
};

template <typename T, int D, int BM, int BN, int STAGES, typename OutT>
__global__ void __launch_bounds__(BM / 32 * kWave)
fa_mfma_fwd(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
            OutT* __restrict__ O, int N, int num_qblocks, int total_blocks, float scale_log2, int causal) {
  typedef typename vec8<T>::type V8;
  typedef MfmaLds<D, BN, STAGES> L;
  constexpr int NW = BM / 32;
  constexpr int THREADS = NW * kWave;
  constexpr int QK_STEPS = D / 16;       // MFMA k-steps over the head dim
  constexpr int NKB = BN / 32;           // 32-key blocks per tile
  constexpr int NDB = D / 32;            // 32-dim blocks of O^T
  constexpr int PV_STEPS = BN / 16;      // MFMA k-steps over the keys of a tile
  constexpr int CHUNKS_ROW = D / 8;      // 16-byte chunks per K/V row
  constexpr int CHUNKS = BN * CHUNKS_ROW;
  static_assert(BM % 32 == 0 && BN % 32 == 0 && D % 32 == 0, "tile shape");
  static_assert(CHUNKS % THREADS == 0, "K/V tile must split evenly over the workgroup");
  constexpr int CPT = CHUNKS / THREADS;  // 16-byte chunks per thread per matrix
  static_assert(STAGES == 1 || STAGES == 2, "one or two LDS stages");

  __shared__ __attribute__((aligned(16))) T lds[L::ELEMS];

  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int lq = lane % 32;   // query column of this lane in the wave's 32-query tile
  const int hi = lane / 32;   // which half of the 32 accumulator rows this lane holds

  const int blk = xcd_remap(blockIdx.x, total_blocks);
  const int bh = blk / num_qblocks;
  int qb = blk % num_qblocks;
  if (causal) qb = num_qblocks - 1 - qb;  // longest causal rows first
  const int q0 = qb * BM;
  const int q0w = q0 + wave * 32;
  const int qrow = q0w + lq;
  const size_t base = (size_t)bh * N * D;
  const T* __restrict__ Qb = Q + base;
  const T* __restrict__ Kb = K + base;
  const T* __restrict__ Vb = V + base;

  // ---- Q^T operand: lane holds Q[qrow][16*kk + 8*hi + j], j < 8, for every k-step kk.
  V8 qf[QK_STEPS];
  {
    const bool ok = qrow < N;
#pragma unroll
    for (int kk = 0; kk < QK_STEPS; ++kk) {
      V8 z = {};
      qf[kk] = ok ? *reinterpret_cast<const V8*>(Qb + (size_t)qrow * D + kk * 16 + hi * 8) : z;
    }
  }

  // ---- K/V staging: thread handles chunks tid + i*THREADS (row-major, coalesced).
  u32x4 kreg[CPT], vreg[CPT];
  auto gload = [&](int j0) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * THREADS;
      const int row = c / CHUNKS_ROW, col = (c % CHUNKS_ROW) * 8;
      const int key = j0 + row;
      u32x4 z = {0u, 0u, 0u, 0u};
      const bool ok = key < N;
      kreg[i] = ok ? *reinterpret_cast<const u32x4*>(Kb + (size_t)key * D + col) : z;
      vreg[i] = ok ? *reinterpret_cast<const u32x4*>(Vb + (size_t)key * D + col) : z;
    }
  };
  auto sstore = [&](int st) {
    T* ks = lds + st * L::STAGE_ELEMS;
    T* vs = ks + L::K_ELEMS;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * THREADS;
      const int row = c / CHUNKS_ROW, col = (c % CHUNKS_ROW) * 8;
      *reinterpret_cast<u32x4*>(ks + row * L::LDK + col) = kreg[i];
      *reinterpret_cast<u32x4*>(vs + row * L::LDV + col) = vreg[i];
    }
  };

  // Per-lane source offsets of the transposed V read. In each 16-lane group g, lane i supplies
  // row (i / 4) and columns 16*(g%2) + 4*(i%4) .. +3; ds_read_b64_tr_b16 then hands lane i the
  // element (i % 4) of the rows supplied by lanes 4t + i/4, i.e. V[row0 + t][col0 + i], t < 4.
  const int g16 = lane / 16, i16 = lane % 16;
  const int v_lane_off = (hi * 4 + i16 / 4) * L::LDV + 16 * (g16 % 2) + 4 * (i16 % 4);

  float m_run = -INFINITY;  // running max of the log2-domain scores of row qrow
  float l_run = 0.f;        // running sum over the 16 keys per 32 held by this lane
  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = f32x16{};

  const int kv_end = causal ? min(N, q0 + BM) : N;
  const int ntiles = (kv_end + BN - 1) / BN;
  const int wave_kv_end = causal ? min(kv_end, q0w + 32) : kv_end;  // keys this wave can see

  auto compute = [&](int st, int j0) {
    const T* ks = lds + st * L::STAGE_ELEMS;
    const T* vs = ks + L::K_ELEMS;

    // S^T = K . Q^T for each 32-key block.
    f32x16 s[NKB];
#pragma unroll
    for (int b = 0; b < NKB; ++b) {
      s[b] = f32x16{};
#pragma unroll
      for (int kk = 0; kk < QK_STEPS; ++kk) {
        const V8 a = *reinterpret_cast<const V8*>(ks + (b * 32 + lq) * L::LDK + kk * 16 + hi * 8);
        s[b] = mfma32x32x16(a, qf[kk], s[b]);
      }
    }

    // Mask keys past N and (causal) keys after the query; only tiles that need it pay.
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

    // Online softmax update of this row's state (log2 domain).
    float mx = -INFINITY;
#pragma unroll
    for (int b = 0; b < NKB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[b][r]);
    mx = half_max(mx);
    const float m_new = fmaxf(m_run, mx * scale_log2);
    const bool dead = (m_new == -INFINITY);  // every key so far masked
    const float alpha = dead ? 0.f : exp2_fast(m_run - m_new);
    const float neg_m = dead ? 0.f : -m_new;
    m_run = m_new;

    V8 pf[PV_STEPS];
    float psum = 0.f;
#pragma unroll
    for (int b = 0; b < NKB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = exp2_fast(fmaf(s[b][r], scale_log2, neg_m));
        psum += p;
        pf[b * 2 + r / 8][r % 8] = from_f32<T>(p);
      }
    l_run = l_run * alpha + psum;

#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] *= alpha;

    // O^T += V^T . P^T
#pragma unroll
    for (int ks_ = 0; ks_ < PV_STEPS; ++ks_) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const T* p0 = vs + ks_ * 16 * L::LDV + db * 32 + v_lane_off;
        const i16x4 a0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr<i16x4>)(p0));
        const i16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr<i16x4>)(p0 + 8 * L::LDV));
        const i16x8 a = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        o[db] = mfma32x32x16(__builtin_bit_cast(V8, a), pf[ks_], o[db]);
      }
    }
  };

  if constexpr (STAGES == 2) {
    gload(0);
    sstore(0);
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
      const int j0 = t * BN;
      if (t + 1 < ntiles) gload(j0 + BN);          // in flight while tile t is computed
      if (j0 < wave_kv_end) compute(t & 1, j0);
      if (t + 1 < ntiles) sstore((t + 1) & 1);
      __syncthreads();
    }
  } else {
    for (int t = 0; t < ntiles; ++t) {
      const int j0 = t * BN;
      gload(j0);
      __syncthreads();  // previous tile fully consumed
      sstore(0);
      __syncthreads();
      if (j0 < wave_kv_end) compute(0, j0);
    }
  }

  // ---- Epilogue: O = O^T / l. Register r of block db holds dim 32*db + 8*(r/4) + 4*hi + r%4.
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
