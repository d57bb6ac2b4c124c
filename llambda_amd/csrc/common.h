// common.h -- shared device helpers for the gfx950 kernels of libllambda_hip.
//
// Block formats are GGML's, as llambda reads them (llambda.lisp:2126-2155,
// 4338-4506):
//   Q4_K  144 B / 256 weights: fp16 d, fp16 dmin, 12 B packed 6-bit
//         scales/mins, 128 B nibbles.
//   Q6_K  210 B / 256 weights: 128 B low nibbles (ql), 64 B 2-bit highs (qh),
//         16 int8 scales, fp16 d.
//   Q5_0  22 B / 32 weights:   fp16 d, u32 high bits, 16 B nibbles.
//   Q8_0  34 B / 32 weights:   fp16 d, 32 int8.
//   F32   4 B / weight.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llhip {

enum GgmlType : int {
  kF32 = 0,
  kQ5_0 = 6,
  kQ8_0 = 8,
  kQ4_K = 12,
  kQ6_K = 14,
};

constexpr int kWave = 64;

// Bytes and weights per block for each supported type.
__host__ __device__ constexpr int block_bytes(int type) {
  return type == kQ4_K ? 144 : type == kQ6_K ? 210 : type == kQ5_0 ? 22 : type == kQ8_0 ? 34 : 4;
}
__host__ __device__ constexpr int block_weights(int type) {
  return (type == kQ4_K || type == kQ6_K) ? 256 : (type == kQ5_0 || type == kQ8_0) ? 32 : 1;
}

// Device allocations of packed weights carry this many readable bytes past
// their end: the dword-granular loads of 2-byte-aligned blocks may touch up to
// 3 bytes beyond the last block, and the grouped expert kernels stage whole
// 256-element chunks (up to 288 bytes) of a row's last, partial chunk.
constexpr size_t kWeightPad = 512;

// A dword-aligned 16-byte vector: lets the compiler emit global_load_dwordx4
// at 4-byte alignment (the hardware requires dword alignment only).
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// Five consecutive dwords starting at the dword containing byte address p,
// returned as the 16 bytes at p (p must be 2-byte aligned; the fifth dword is
// read even when p is dword aligned, hence kWeightPad).
__device__ __forceinline__ uint4 load16_unaligned2(const uint8_t* p) {
  // pointer arithmetic (not an integer round trip) keeps the global address
  // space visible to the compiler, so these become global_load, not flat_load
  const uint32_t shift = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3u);
  const uint32_t* base = reinterpret_cast<const uint32_t*>(p - shift);
  u32x4a4 v = *reinterpret_cast<const u32x4a4*>(base);
  uint32_t e = base[4];
  uint4 r;
  r.x = __builtin_amdgcn_alignbyte(v.y, v.x, shift);
  r.y = __builtin_amdgcn_alignbyte(v.z, v.y, shift);
  r.z = __builtin_amdgcn_alignbyte(v.w, v.z, shift);
  r.w = __builtin_amdgcn_alignbyte(e, v.w, shift);
  return r;
}

__device__ __forceinline__ uint4 load16_aligned(const uint8_t* p) {
  return *reinterpret_cast<const uint4*>(p);
}

__device__ __forceinline__ float ubyte(uint32_t v, int k) {
  return (float)((v >> (8 * k)) & 0xFFu);
}

// Hides a value's provenance from the optimiser.  Used on nibble masks such
// as (v >> 4) & 0x0F0F0F0F so that their bytes convert with
// v_cvt_f32_ubyte0..3 (one instruction per weight) instead of being folded
// into a v_bfe_u32 per weight.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm("" : "+v"(v));
  return v;
}

// DPP lane permutations within rows of 16 lanes (gfx9 encodings).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <- 7-i within 8
constexpr int kDppMirror = 0x140;      // lane i <- 15-i within 16
constexpr int kDppRowRor8 = 0x128;     // lane i <- (i+8) mod 16 within 16, i.e. i ^ 8

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// Maximum / minimum over the wavefront, every lane receiving it: DPP within
// rows of 16 lanes, then the four row results.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppMirror>(v));
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
__device__ __forceinline__ int wave_max_i(int v) {
  v = max(v, dpp_i<kDppXor1>(v));
  v = max(v, dpp_i<kDppXor2>(v));
  v = max(v, dpp_i<kDppHalfMirror>(v));
  v = max(v, dpp_i<kDppMirror>(v));
  return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ int wave_min(int v) {
  v = min(v, dpp_i<kDppXor1>(v));
  v = min(v, dpp_i<kDppXor2>(v));
  v = min(v, dpp_i<kDppHalfMirror>(v));
  v = min(v, dpp_i<kDppMirror>(v));
  return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// v + v of lane i ^ 16 (rows 0/1 and 2/3 of 16 lanes) and v + v of lane
// i ^ 32 (the two halves), by gfx950's row swaps: with v in both operands,
// v_permlane16_swap leaves (rows 0,0,2,2) in the first and (rows 1,1,3,3) in
// the second, v_permlane32_swap (lanes 0-31 twice) and (lanes 32-63 twice);
// their sum is each lane's own value plus its partner's (the sum commutes).
// Written as assembly with both registers as in/out operands (the compiler's
// builtin returned the first register twice), with two wait states on each
// side of the swap.  Every lane must be active.
__device__ __forceinline__ float row_pair_sum(float v) {
  float a = v, b = v;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  return a + b;
}
__device__ __forceinline__ float half_pair_sum(float v) {
  float a = v, b = v;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  return a + b;
}

// Sum over aligned groups of 2^log2w lanes; every lane of a group receives
// its group's sum.
__device__ __forceinline__ float group_sum(float v, int log2w) {
  if (log2w >= 1) v += dpp<kDppXor1>(v);
  if (log2w >= 2) v += dpp<kDppXor2>(v);
  if (log2w >= 3) v += dpp<kDppHalfMirror>(v);
  if (log2w >= 4) v += dpp<kDppMirror>(v);
  if (log2w >= 5) v = row_pair_sum(v);
  if (log2w >= 6) v = half_pair_sum(v);
  return v;
}

// Sum over the wavefront, every lane receiving it: rows of 16 lanes by DPP
// (group_sum), then the four row sums as (r0 + r1) + (r2 + r3).
__device__ __forceinline__ float wave_total(float v) {
  const int b = __builtin_bit_cast(int, group_sum(v, 4));
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
}

// Sum across `width` consecutive lanes (width a power of two <= 64).
template <int WIDTH>
__device__ __forceinline__ float segment_sum(float v) {
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float segment_sum_dyn(float v, int width) {
  for (int off = width / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

}  // namespace llhip
