// Device-side helpers shared by every attention kernel (gfx950 / CDNA4, wave64).
//
// Storage types are the compiler's native _Float16 and __bf16; all softmax arithmetic is fp32.
// Nothing here depends on PyTorch: the kernels are reached only through the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pa {

typedef _Float16 f16;
typedef __bf16 bf16;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWave = 64;
constexpr int kNumXcd = 8;  // MI355X: 8 accelerator complex dies, each with its own L2

// LDS pointer type for builtins that take an address_space(3) operand.
template <typename T>
using lds_ptr = __attribute__((address_space(3))) T*;

// Vector of 8 storage elements, the per-lane operand of a K=16 (32x32) / K=32 (16x16) MFMA.
template <typename T> struct vec8;
template <> struct vec8<f16> { typedef f16x8 type; };
template <> struct vec8<bf16> { typedef bf16x8 type; };

// D = A * B + C on a 32x32x16 tile. Lane l holds A[l%32][8*(l/32)+j], B[8*(l/32)+j][l%32] and
// C[8*(r/4) + 4*(l/32) + r%4][l%32] in register r (layouts checked on the device).
__device__ __forceinline__ f32x16 mfma32x32x16(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// D = A * B + C on a 16x16x32 tile. Lane l holds A[l%16][8*(l/16)+j], B[8*(l/16)+j][l%16] and
// C[4*(l/16) + r][l%16] in register r (the row sums of the fused kernels depend on this layout;
// the GPU parity tests check them against the oracle).
__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// fp32 32x32x2: lane l holds A[l%32][l/32], B[l/32][l%32]; C as above.
__device__ __forceinline__ f32x16 mfma32x32x2(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// x[l ^ 32]: the value held by the same column in the other half of the wave.
// v_permlane32_swap(vdst = x, vsrc = x) leaves vdst = {x[l%32]} and vsrc = {x[l%32 + 32]} in every
// lane, so the partner is vsrc in the low half and vdst in the high half. The two results are
// selected by lane half on purpose: combining them symmetrically (r0 + r1) is compiled by this
// hipcc as r0 + r0, which drops the other half.
__device__ __forceinline__ float partner32(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}
// All-reduce across the two 32-lane halves: lanes l and l^32 both get op(x[l], x[l^32]).
__device__ __forceinline__ float half_max(float x) { return fmaxf(x, partner32(x)); }
__device__ __forceinline__ float half_sum(float x) { return x + partner32(x); }

// x[l ^ 16], on v_permlane16_swap: with vdst = vsrc = x it leaves vdst = x of the even 16-lane row
// of each pair and vsrc = x of the odd one, so the partner is vsrc in even rows and vdst in odd
// ones (the same selection by lane bit as partner32).
__device__ __forceinline__ float partner16(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 16) ? r[0] : r[1]);
}

// x of another lane of the same 16-lane row through a DPP move (CTRL: quad_perm 0x00-0xff,
// row_mirror 0x140, row_half_mirror 0x141).
template <int CTRL>
__device__ __forceinline__ float dpp_move(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}

// Wave64 all-reduce without LDS or ds_bpermute: every lane ends with op over all 64 lanes. Within
// a 16-lane row, two quad permutations (lane ^ 1, lane ^ 2) make every quad uniform, the half-row
// mirror (lane 7 - i within 8) pairs the two quads of an 8-lane half and the row mirror (lane
// 15 - i) the two halves; then the 16- and 32-lane partner swaps join the four rows. op must be
// commutative and associative (max, or + up to the order of its roundings, fixed per lane).
template <typename Op>
__device__ __forceinline__ float wave_allreduce(float x, Op op) {
  x = op(x, dpp_move<0xB1>(x));    // quad_perm [1, 0, 3, 2]
  x = op(x, dpp_move<0x4E>(x));    // quad_perm [2, 3, 0, 1]
  x = op(x, dpp_move<0x141>(x));   // row_half_mirror
  x = op(x, dpp_move<0x140>(x));   // row_mirror
  x = op(x, partner16(x));
  return op(x, partner32(x));
}
struct MaxOp {
  __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct SumOp {
  __device__ float operator()(float a, float b) const { return a + b; }
};

// Buffer resource over [base, base + bytes): raw buffer loads at offsets past `bytes` return 0
// without touching memory, which makes the tails of K/V/Q tiles branch-free.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 load16(rsrc_t r, uint32_t byte_offset) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, byte_offset, 0, 0);
}

// 16 bytes per lane from the buffer straight into LDS: lane i writes lds_base + 16*i
// (lds_base must be wave-uniform); offsets past the buffer's size write zeros.
__device__ __forceinline__ void load16_to_lds(rsrc_t r, void* lds_base, uint32_t voffset, uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_base, 16, voffset,
                                           soffset, 0, 0);
}

// Scheduling-group masks for __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedValu = 0x002;
constexpr int kSchedMfma = 0x008;
constexpr int kSchedVmemRead = 0x020;
constexpr int kSchedDsRead = 0x100;

// 2^x on the transcendental unit (v_exp_f32). exp2(-inf) = 0.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Storage conversions, round to nearest even.
template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ f16 from_f32<f16>(float x) { return (f16)x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(f16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }

// Maps the hardware workgroup id to a logical one so that consecutive logical ids run on the
// same XCD: the dispatcher sends workgroup g to XCD g % 8, so logical id
// (g % 8) * (total / 8) + g / 8 keeps a contiguous range of (head, query-block) pairs - the
// blocks that re-read the same K/V rows - inside one XCD's L2. Identity when total % 8 != 0.
__device__ __forceinline__ int xcd_remap(int g, int total) {
  if (total % kNumXcd != 0) return g;
  return (g % kNumXcd) * (total / kNumXcd) + g / kNumXcd;
}

// The causal walk's dealing: the entry of an XCD's block list taken at step j by workgroup c of
// the XCD's wgs workgroups. Workgroup c runs on the XCD's CU u = c % cus_per_xcd (the dispatcher
// places an XCD's workgroups on its CUs in turn) as slot c / cus_per_xcd; step j is pass
// p = j * slots + slot of the list over the CUs, entry p * cus_per_xcd + u in even passes and
// p * cus_per_xcd + cus_per_xcd - 1 - u in odd ones (serpentine). Where the workgroups do not
// fill whole slots (cus_per_xcd 0, or fewer workgroups than the XCD has CUs times its slots), the
// passes run over the workgroups instead. The launcher evaluates the same function on the host.
__host__ __device__ __forceinline__ int causal_walk_entry(int j, int c, int wgs, int cus_per_xcd) {
  if (cus_per_xcd > 0 && wgs % cus_per_xcd == 0) {
    const int u = c % cus_per_xcd, p = j * (wgs / cus_per_xcd) + c / cus_per_xcd;
    return p * cus_per_xcd + ((p & 1) ? cus_per_xcd - 1 - u : u);
  }
  return j * wgs + ((j & 1) ? wgs - 1 - c : c);
}

// The causal walk: the query block (head * num_qblocks + block) that workgroup c of the wgs on
// list x takes at step j, -1 past the end of the list. The heads below bh are split over `lists`
// lists, list x owning the heads x, x + lists, ...: one list per XCD (lists = kNumXcd, c and wgs
// counted within the XCD, cus the XCD's CUs), or one for the device (lists = 1, c the workgroup
// id, cus every CU: workgroup g runs on the device's CU g % cus, since the dispatcher sends g to
// XCD g % 8 and places an XCD's workgroups on its CUs in turn). A list holds its blocks head by
// head, longest (last) block first within a head (by_rank = 0), or by length, the longest block
// of every head first (by_rank = 1), and is dealt out by causal_walk_entry. Head by head, the
// blocks running at once on an XCD share the K/V of few heads in its L2, and the serpentine
// passes pair long and short blocks on a CU exactly when the blocks per head tile the passes; by
// length, the passes deal a sorted list, which is near the longest-first greedy assignment for any
// block count.
__host__ __device__ __forceinline__ int causal_walk_block(int j, int c, int x, int wgs, int cus, int bh,
                                                          int num_qblocks, int by_rank, int lists) {
  const int heads = (bh - x + lists - 1) / lists;
  const int e = causal_walk_entry(j, c, wgs, cus);
  if (e >= heads * num_qblocks) return -1;
  const int h = by_rank ? e % heads : e / num_qblocks;
  const int r = by_rank ? e / heads : e % num_qblocks;
  return (x + lists * h) * num_qblocks + (num_qblocks - 1 - r);
}

}  // namespace pa
