// Fused online-softmax attention forward with fp32 arithmetic throughout (the `fused` entry).
//
// Same algorithm and numerics as the reference's v3 kernel
// (/root/reference/csrc/kernels/fused.cuh:26-102): Q pre-scaled by log2(e)/sqrt(d) in fp32
// registers, scores, running max/sum and P all fp32 (P is never rounded), inputs fp32 or fp16
// widened to fp32 on load. Both products run on the fp32 matrix core (v_mfma_f32_32x32x2_f32):
//   S^T (keys x queries) = K . Q^T   A = K (lane: one key row, 32 consecutive dims),
//                                    B = scaled Q^T in VGPRs, k-slot h of step kk = dim h*D/2+kk
//   O^T (d x queries)   += V^T . P^T  B = P^T straight from the S^T accumulator (k-slot h of
//                                    step r = key 8*(r/4) + 4*h + r%4), A = V (lane: one dim of
//                                    the two keys of the step)
// Each lane keeps all state of query l%32 (see fa_mfma.hpp). Row i of the two 32-row O^T blocks
// is dim 2i (block 0) and dim 2i + 1 (block 1), so each lane reads the V values of both blocks
// with one 8-byte load (fp32; 4 bytes for fp16) instead of two scalar loads; the merge puts the
// dims back in order.
//
// gfx950 shape: the fp32 matrix core does 64 FLOP per cycle per SIMD, so a 32-query x 32-key
// tile costs a wave ~4K cycles; at the reference's sizes (N = 128) a wave per 32 queries leaves
// most SIMDs idle and runs four tiles back to back. Here a workgroup of KS waves owns 32 query
// rows and SPLITS THE KEYS: wave w takes key tiles w, w+KS, w+2KS, ... with its own running
// (m, l, O); the KS partial states are merged once through LDS at the end with the same rule
// the online softmax applies between tiles (m = max m_w, l = sum l_w 2^(m_w - m),
// O = sum O_w 2^(m_w - m)), the reference's merge_ml (tiled.cuh:48-53) extended to O. Each wave
// reads its K/V rows straight from HBM/L2 into the operand registers (no tile is shared between
// waves, so no LDS staging), one tile ahead of its use.
#pragma once

#include "common.hpp"

namespace pa {

template <int D, int KS>
struct F32Lds {
  static constexpr int LDO = D + 4;   // +16 B per query row: the 32 rows written at one column hit distinct banks
  static constexpr int BYTES = KS * 32 * (LDO + 2) * 4;
};

// 32 consecutive elements of a row, widened to fp32 (offsets past the buffer read as zero).
// The loaded vector is bit-cast as a whole before its elements are taken: bit-casting an element
// extracted from the u32x4 miscompiles with this toolchain (every element read as element 0).
template <typename T>
__device__ __forceinline__ void load_row32(rsrc_t rs, uint32_t byte_off, float (&x)[32]) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const f32x4 w = __builtin_bit_cast(f32x4, load16(rs, byte_off + 16 * i));
#pragma unroll
      for (int j = 0; j < 4; ++j) x[4 * i + j] = w[j];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 w = load16(rs, byte_off + 16 * i);
      const f16x8 h = __builtin_bit_cast(f16x8, w);
#pragma unroll
      for (int j = 0; j < 8; ++j) x[8 * i + j] = (float)h[j];
    }
  }
}

template <typename T>
__device__ __forceinline__ float load_one(rsrc_t rs, uint32_t byte_off) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, byte_off, 0, 0));
  } else {
    return (float)__builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(rs, byte_off, 0, 0));
  }
}

// Two consecutive elements of a row, widened to fp32 (offsets past the buffer read as zero).
template <typename T>
__device__ __forceinline__ void load_pair(rsrc_t rs, uint32_t byte_off, float& a, float& b) {
  if constexpr (sizeof(T) == 4) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 w = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, byte_off, 0, 0));
    a = w[0];
    b = w[1];
  } else {
    const f16x2 h = __builtin_bit_cast(f16x2, __builtin_amdgcn_raw_buffer_load_b32(rs, byte_off, 0, 0));
    a = (float)h[0];
    b = (float)h[1];
  }
}

template <typename T, int D, int KS, typename OutT>
__global__ void __launch_bounds__(KS * kWave)
fa_f32_fwd(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
           OutT* __restrict__ O, int N, int num_qblocks, int total_blocks, float scale_log2, int causal) {
  typedef F32Lds<D, KS> L;
  constexpr int BN = 32;                     // keys per tile
  constexpr int NDB = D / 32;
  constexpr int HALF = D / 2;
  constexpr int ES = sizeof(T);
  static_assert(D == 64, "the fp32 path is compiled for d = 64");

  __shared__ __attribute__((aligned(16))) float red_o[KS * 32 * L::LDO];
  __shared__ float red_m[KS * 32];
  __shared__ float red_l[KS * 32];

  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int lq = lane % 32;
  const int hi = lane / 32;

  const int blk = xcd_remap(blockIdx.x, total_blocks);
  const int bh = blk / num_qblocks;
  int qb = blk % num_qblocks;
  if (causal) qb = num_qblocks - 1 - qb;
  const int q0 = qb * 32;
  const int qrow = q0 + lq;
  const size_t base = (size_t)bh * N * D;
  const uint32_t head_bytes = (uint32_t)((size_t)N * D * ES);
  const rsrc_t q_rs = make_rsrc(Q + base, head_bytes);
  const rsrc_t k_rs = make_rsrc(K + base, head_bytes);
  const rsrc_t v_rs = make_rsrc(V + base, head_bytes);

  // Scaled Q^T operand: k-slot `hi` of step kk is dim hi*HALF + kk (rows past N read as zero).
  float qf[HALF];
  load_row32<T>(q_rs, (uint32_t)((qrow * D + hi * HALF) * ES), qf);
#pragma unroll
  for (int c = 0; c < HALF; ++c) qf[c] *= scale_log2;

  float m_run = -INFINITY, l_run = 0.f;
  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = f32x16{};

  const int kv_end = causal ? min(N, q0 + 32) : N;
  const int ntiles = (kv_end + BN - 1) / BN;

  // Operands of one tile: K row (key j0 + lq, dims hi*HALF ..) and V (dim db*32 + lq of the key
  // that k-slot hi of step r holds).
  struct Tile {
    float k[HALF];
    float v[16][NDB];
  };
  auto load_tile = [&](Tile& tl, int j0) {
    load_row32<T>(k_rs, (uint32_t)(((j0 + lq) * D + hi * HALF) * ES), tl.k);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = j0 + 8 * (r / 4) + 4 * hi + (r % 4);
      load_pair<T>(v_rs, (uint32_t)((key * D + 2 * lq) * ES), tl.v[r][0], tl.v[r][1]);   // dims 2 lq, 2 lq + 1
    }
  };

  auto compute = [&](const Tile& tl, int j0) {
    f32x16 s = f32x16{};
#pragma unroll
    for (int kk = 0; kk < HALF; ++kk) s = mfma32x32x2(tl.k[kk], qf[kk], s);
    if (j0 + BN > N || (causal && j0 + BN - 1 > q0)) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = j0 + 8 * (r / 4) + 4 * hi + (r % 4);
        if (key >= N || (causal && key > qrow)) s[r] = -INFINITY;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
    const float m_new = fmaxf(m_run, half_max(mx));
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
    for (int r = 0; r < 16; ++r) {
      const float p = exp2_fast(s[r] - sub_m);
      l_run += p;
#pragma unroll
      for (int db = 0; db < NDB; ++db) o[db] = mfma32x32x2(tl.v[r][db], p, o[db]);
    }
  };

  // This wave's tiles: wave, wave + KS, ...; the next one is loaded while the current computes.
  if (wave < ntiles) {
    Tile cur, nxt;
    load_tile(cur, wave * BN);
    for (int t = wave; t < ntiles; t += KS) {
      const bool more = t + KS < ntiles;
      if (more) load_tile(nxt, (t + KS) * BN);
      compute(cur, t * BN);
      if (more) cur = nxt;
    }
  }

  // ---- Merge the KS partial states (m, l, O) of the 32 queries through LDS.
  const float l_w = half_sum(l_run);
  if (hi == 0) {
    red_m[wave * 32 + lq] = m_run;
    red_l[wave * 32 + lq] = l_w;
  }
  // Register r of block db holds row i = 8*(r/4) + 4*hi + r%4, i.e. dim 2i + db: registers
  // 4 g4 .. 4 g4 + 3 of both blocks are the 8 consecutive dims 16 g4 + 8 hi .. + 7.
#pragma unroll
  for (int g4 = 0; g4 < 4; ++g4) {
    const f32x4 w0 = {o[0][4 * g4], o[1][4 * g4], o[0][4 * g4 + 1], o[1][4 * g4 + 1]};
    const f32x4 w1 = {o[0][4 * g4 + 2], o[1][4 * g4 + 2], o[0][4 * g4 + 3], o[1][4 * g4 + 3]};
    float* dst = red_o + (wave * 32 + lq) * L::LDO + 16 * g4 + 8 * hi;
    *reinterpret_cast<f32x4*>(dst) = w0;
    *reinterpret_cast<f32x4*>(dst + 4) = w1;
  }
  __syncthreads();

  float m_all = -INFINITY;
#pragma unroll
  for (int w = 0; w < KS; ++w) m_all = fmaxf(m_all, red_m[w * 32 + lq]);
  float sc[KS];
  float l_all = 0.f;
#pragma unroll
  for (int w = 0; w < KS; ++w) {
    const float mw = red_m[w * 32 + lq];
    sc[w] = (mw == -INFINITY) ? 0.f : exp2_fast(mw - m_all);   // a wave without visible keys adds nothing
    l_all += sc[w] * red_l[w * 32 + lq];
  }
  const float inv = 1.f / l_all;
  // Wave w finalises the (db, g4) groups w, w + KS, ... of its lanes' rows (4 dims each).
  if (qrow < N) {
    OutT* orow = O + base + (size_t)qrow * D;
    for (int grp = wave; grp < NDB * 4; grp += KS) {
      const int db = grp / 4, g4 = grp % 4;
      const int dim = db * 32 + 8 * g4 + 4 * hi;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < KS; ++w) acc += sc[w] * *reinterpret_cast<const f32x4*>(red_o + (w * 32 + lq) * L::LDO + dim);
      typedef OutT OutV4 __attribute__((ext_vector_type(4)));
      OutV4 out;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) out[rr] = from_f32<OutT>(acc[rr] * inv);
      *reinterpret_cast<OutV4*>(orow + dim) = out;
    }
  }
}

}  // namespace pa
