// mfma.h -- shared helpers of the MFMA kernels (gemv_mfma.hip, moe_mfma.hip):
// operand types, exact bf16 code fragments, the activation hi/lo split, and
// the global -> LDS DMA used to stage raw super-block bytes.
#pragma once

#include "common.h"

namespace llhip {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// A code byte q < 128 next to the filler byte 0x43 is the bf16 bit pattern of
// exactly 128 + q (0x4300 = 128.0, one unit in the last place = 1).
constexpr uint32_t kFiller = 0x43434343u;
constexpr uint32_t kSelLo = 0x04010400u;  // {b0, F, b1, F}
constexpr uint32_t kSelHi = 0x04030402u;  // {b2, F, b3, F}

__device__ __forceinline__ uint32_t bf16_bits_rne(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// x = hi + lo with hi, lo bf16 (bits returned); |x - hi - lo| <= 2^-17 |x|.
// hi + lo (as fp32) is returned in sum.
__device__ __forceinline__ void split_bf16(float x, uint32_t& hi, uint32_t& lo, float& sum) {
  hi = bf16_bits_rne(x);
  const float fh = __builtin_bit_cast(float, hi << 16);
  lo = bf16_bits_rne(x - fh);
  sum = fh + __builtin_bit_cast(float, lo << 16);
}

// Two elements split at once: (x0, x1) = (hi0 + lo0, hi1 + lo1), the bf16
// pairs packed with x0 in the low half (split_bf16's hi0 | hi1 << 16), by
// v_cvt_pk_bf16_f32, whose round-to-nearest-even equals bf16_bits_rne on
// every finite value and infinity; the fp32 sums hi + lo in s0, s1.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void split_bf16_pair(float x0, float x1, uint32_t& hi, uint32_t& lo,
                                                float& s0, float& s1) {
  hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(floatx2{x0, x1}, bf16x2));
  const float h0 = __builtin_bit_cast(float, hi << 16);
  const float h1 = __builtin_bit_cast(float, hi & 0xFFFF0000u);
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(floatx2{x0 - h0, x1 - h1}, bf16x2));
  s0 = h0 + __builtin_bit_cast(float, lo << 16);
  s1 = h1 + __builtin_bit_cast(float, lo & 0xFFFF0000u);
}

// 8 codes (two dwords of code bytes, each < 128) -> 8 bf16 of 128 + q.
__device__ __forceinline__ bf16x8 codes_to_b(uint32_t c0, uint32_t c1) {
  u32x4 v;
  v.x = __builtin_amdgcn_perm(kFiller, c0, kSelLo);
  v.y = __builtin_amdgcn_perm(kFiller, c0, kSelHi);
  v.z = __builtin_amdgcn_perm(kFiller, c1, kSelLo);
  v.w = __builtin_amdgcn_perm(kFiller, c1, kSelHi);
  return __builtin_bit_cast(bf16x8, v);
}

// 4 codes (one dword) -> 4 bf16 of 128 + q.
__device__ __forceinline__ shortx4 codes4_to_b(uint32_t c) {
  u32x2 v;
  v.x = __builtin_amdgcn_perm(kFiller, c, kSelLo);
  v.y = __builtin_amdgcn_perm(kFiller, c, kSelHi);
  return __builtin_bit_cast(shortx4, v);
}

// D = A B + C on 16 x 16 tiles.  Lane l holds A row (l & 15), B column
// (l & 15), the K slice selected by l >> 4, and D rows 4 (l >> 4) .. +3 of
// column (l & 15).
__device__ __forceinline__ floatx4 mfma32(const bf16x8& a, const bf16x8& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mfma16(const shortx4& a, const shortx4& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mfma4f32(float a, float b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------- LDS staging
typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return (uint32_t)(uintptr_t)(lds_ptr_t)(p);
}

// An 8-byte LDS read that the compiler does not pair with another into one
// ds_read2_b64: a paired read serves 16 lanes a cycle, so the rows n and
// n + 8 of a stage (rows of 144 or 240 bytes) meet in one bank; single
// 8-byte reads serve 32 lanes a cycle and see none (measured with the LDS
// bank-conflict counter).  The address passes through an empty asm, so no
// two reads share a base register; equal addresses still combine.
__device__ __forceinline__ uint2 lds_read8(const void* p) {
  uint32_t a = lds_address(p);
  asm("" : "+v"(a));
  typedef unsigned int pair_t __attribute__((ext_vector_type(2)));
  const pair_t v = *reinterpret_cast<const __attribute__((address_space(3))) pair_t*>(a);
  return make_uint2(v.x, v.y);
}

// 64 lanes x 16 bytes from base + voff[lane] to LDS lds + 16 * lane (vector
// memory load with LDS destination).  base and lds are wavefront-uniform.
__device__ __forceinline__ void load_lds16(const uint8_t* base, uint32_t voff, uint32_t lds) {
  asm volatile(
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(voff), "s"(base), "{m0}"(lds)
      : "memory");
}

// load_lds16 with the non-temporal policy: for streams read once (packed
// weight rows), which then stay out of the caches' way.  Measured on one
// MI355X over a 431 MB buffer: 7.0 TB/s against 6.0 TB/s with the default
// policy.
__device__ __forceinline__ void load_lds16_nt(const uint8_t* base, uint32_t voff, uint32_t lds) {
  asm volatile(
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1 nt"
      :
      : "v"(voff), "s"(base), "{m0}"(lds)
      : "memory");
}

// 64 lanes x 4 bytes from base + voff[lane] to LDS lds + 4 * lane.
__device__ __forceinline__ void load_lds4(const uint8_t* base, uint32_t voff, uint32_t lds) {
  asm volatile(
      "s_nop 0\n\t"
      "global_load_lds_dword %0, %1"
      :
      : "v"(voff), "s"(base), "{m0}"(lds)
      : "memory");
}

template <int N>
__device__ __forceinline__ void wait_loads() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const uint8_t*>(((uint64_t)hi << 32) | lo);
}

}  // namespace llhip
