// Shared device helpers for the gfx950 attention kernels: b16 vector types,
// MFMA wrappers, LDS address-space casts and the XCD-aware block remap.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace afa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define AFA_LDS __attribute__((address_space(3)))

// Storage type tags. DT_BF16 and DT_F16 are the values of the C-ABI `dtype`.
enum { DT_BF16 = 0, DT_F16 = 1 };

template <int DT> struct B16;
template <> struct B16<DT_BF16> {
  typedef __bf16 scalar;
  typedef bf16x8 x8;
  typedef bf16x4 x4;
  static __device__ __forceinline__ f32x4 mfma(x8 a, x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ x4 read_tr(const AFA_LDS void* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((x4 AFA_LDS*)p);
  }
};
template <> struct B16<DT_F16> {
  typedef _Float16 scalar;
  typedef f16x8 x8;
  typedef f16x4 x4;
  static __device__ __forceinline__ f32x4 mfma(x8 a, x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ x4 read_tr(const AFA_LDS void* p) {
    typedef __fp16 fp16x4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
    return __builtin_bit_cast(x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((fp16x4 AFA_LDS*)p));
  }
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Reductions over the four lanes {l, l^16, l^32, l^48} that hold the same
// MFMA output column, with the gfx950 half-swaps v_permlane32_swap (lanes
// 32..63 <-> 0..31) and v_permlane16_swap (16..31 <-> 0..15 in each half):
// swapping a value with itself leaves each lane holding both partners.
__device__ __forceinline__ void swap32(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ void swap16(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_over_lane_groups(float v) {
  float a, b;
  swap16(v, a, b);
  v = fmaxf(a, b);
  swap32(v, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float sum_over_lane_groups(float v) {
  float a, b;
  swap16(v, a, b);
  v = a + b;
  swap32(v, a, b);
  return a + b;
}

// Inclusive prefix sum over the 64 lanes of a wave (every lane active), in
// DPP moves rather than LDS permutes: shifts by 1, 2, 4 and 8 within each row
// of 16 lanes (lanes shifted in from outside the row add 0), then row 0's
// total is added to row 1 and row 2's to row 3 (row_bcast:15 into rows 1, 3),
// then the total of rows 0-1 to rows 2 and 3 (row_bcast:31 into rows 2, 3).
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

// gfx950 LDS serves 64 four-byte banks (256 bytes) per cycle. Measured lane
// grouping: a 16-byte read (ds_read_b128) serves, within each 32-lane half, the
// 16 lanes whose quad index (lane >> 2) & 7 has even parity, then the odd ones;
// an 8-byte transposing read (ds_read_b64_tr_b16) serves lanes 0..31, then
// 32..63. Unit u (16 bytes) of KV row r lives at u ^ (r & 15). With the row
// permutation sigma below:
//  - QK fragment reads (lane (g, i) reads row sigma(i), unit 4j + g): each
//    16-lane group touches 16 distinct 16-byte bank groups, because
//    sigma({0..3} u {12..15}) and sigma({4..11}) are unions of row pairs
//    {2k, 2k+1};
//  - transposing reads (lane group g reads rows sigma(4g..4g+3), 32 bytes each):
//    each 32-lane half touches 8 distinct 32-byte bank groups, because the
//    rows of lane groups {0,1} and of {2,3} have distinct r >> 1.
__device__ __forceinline__ int swz(int row, int unit) { return unit ^ (row & 15); }

// Chunk row held at MFMA output row m of a 16-row S^T tile:
// sigma(m) = 2*(m & 3) + {0, 8, 9, 1}[m >> 2], i.e. lane groups 0..3 of a
// transposing read take the rows {0,2,4,6}, {8,10,12,14}, {9,11,13,15}, {1,3,5,7}.
__device__ __forceinline__ int sigma(int m) { return ((m & 3) << 1) + ((0x1980 >> ((m >> 2) << 2)) & 15); }

// Load-to-LDS (global_load_lds_*): the LDS destination is M0, set by an
// s_mov_b32 in the same asm statement. GFX9 needs one wait state between an
// SALU write of M0 and an LDS-DMA instruction that reads it; the compiler
// inserts it for its own code but cannot see inside inline asm, so every such
// statement here carries its own s_nop 0 between the two.

// LDS byte address of a __shared__ object, and an LDS pointer from one.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return (uint32_t)(uintptr_t)(const AFA_LDS void*)p;
}
template <typename T>
__device__ __forceinline__ const AFA_LDS T* lds_at(uint32_t address) {
  return (const AFA_LDS T*)(uintptr_t)address;
}

// Returns v unchanged but hides how it was formed. A per-iteration LDS base
// laundered this way stays one register, and the constant parts of each
// fragment address go into the DS instruction's offset field; without it the
// compiler keeps one precomputed address per fragment and rebuilds each one
// with two VALU operations every iteration.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  __asm__("" : "+v"(v));
  return v;
}
// The same for a wave-uniform value, kept in a scalar register.
__device__ __forceinline__ uint32_t opaque_uniform(uint32_t v) {
  __asm__("" : "+s"(v));
  return v;
}

// s_waitcnt immediate for lgkmcnt(0) alone (gfx9 encoding: vmcnt[3:0] |
// expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14, all other fields at max).
constexpr int WAIT_LGKM0 = 0xC07F;
// s_waitcnt vmcnt(N) alone: wait until at most N vector memory operations of
// this wave are in flight. The kernels use N > 0 only where every operation in
// flight is a load (loads and loads to LDS retire in issue order, so this waits
// for all but the N most recent); behind stores they wait with N = 0, since
// stores are not relied on to retire in order with loads.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}
// Workgroup barrier without the memory fence of __syncthreads(): global loads
// of later chunks stay in flight across it. The caller's own LDS stores are
// complete (lgkmcnt(0)) before it signals; the empty asm statements keep the
// compiler from moving LDS accesses across the barrier.
__device__ __forceinline__ void block_barrier() {
  __builtin_amdgcn_s_waitcnt(WAIT_LGKM0);
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

// Blocks are dispatched round-robin over the 8 XCDs of an MI355X. Map the
// hardware block id to a logical id so that each XCD receives a contiguous
// range of logical ids (neighbouring work shares that XCD's L2).
__device__ __forceinline__ uint32_t xcd_contiguous(uint32_t b, uint32_t n) {
  const uint32_t x = b & 7u, local = b >> 3;
  const uint32_t per = n >> 3, extra = n & 7u;
  return x * per + (x < extra ? x : extra) + local;
}

}  // namespace afa
