// positions.h -- per-lane dequant-dot of one 64-weight "position" of a packed
// row, with the lane's 64 activations held in registers.
//
// The batch-1 GEMV (gemv.hip, gemv_rows_kernel) gives every lane a fixed
// position of K, loads that position's activations once, and then streams
// rows past it: per row a lane loads only its position's bytes, so each byte
// of W is fetched by exactly one lane (the Q4_K header and the Q6_K d, shared
// within a block, aside) and no activation traffic is repeated.
//
//   Q4_K  position (block b, j):  header 16 B + qs bytes [32j, 32j+32):
//         sub-block 2j (low nibbles) and 2j+1 (high nibbles).
//   Q6_K  position (block b, h, half):  ql [64h+16half, +16) and
//         [64h+32+16half, +16), qh [128+32h+16half, +16), scales
//         sc[8h+half+2k] (k = 0..3) and d.  Element 128h + 32k + l,
//         l in [16half, 16half+16): the q_k of llambda.lisp:4203-4310.
//   Q8_0, Q5_0  position = two consecutive 32-weight blocks.
//
// Every dot is  sum_g delta_g * (sum_i u_i x_i - c_g * sum_i x_i)  over the
// position's scale groups g (u: unsigned code, c_g: code offset), with the
// group sums of x precomputed in registers.
#pragma once

#include "common.h"

namespace llhip {

template <int TYPE>
struct Pos;

// Sum of 16 consecutive x values (registers).
__device__ __forceinline__ float sum16(const float* x) {
  float a = (x[0] + x[1]) + (x[2] + x[3]);
  float b = (x[4] + x[5]) + (x[6] + x[7]);
  float c = (x[8] + x[9]) + (x[10] + x[11]);
  float d = (x[12] + x[13]) + (x[14] + x[15]);
  return (a + b) + (c + d);
}

// ------------------------------------------------------------------ Q4_K
template <>
struct Pos<kQ4_K> {
  static constexpr int kGroups = 2;
  struct Raw {
    uint4 hdr;
    uint4 q0, q1;
  };
  // activation index of element e (0..63) of the position
  static __device__ __forceinline__ int x_index(int pos, int e) {
    return (pos >> 2) * 256 + (pos & 3) * 64 + e;
  }
  static __device__ __forceinline__ void group_sums(const float (&x)[64], float (&g)[kGroups]) {
    g[0] = sum16(x) + sum16(x + 16);
    g[1] = sum16(x + 32) + sum16(x + 48);
  }
  static __device__ __forceinline__ Raw load(const uint8_t* row, int pos) {
    const uint8_t* blk = row + (pos >> 2) * 144;
    const int j = pos & 3;
    Raw r;
    r.hdr = load16_aligned(blk);
    r.q0 = load16_aligned(blk + 16 + 32 * j);
    r.q1 = load16_aligned(blk + 32 + 32 * j);
    return r;
  }
  static __device__ __forceinline__ float dot(const Raw& r, int pos, const float (&x)[64],
                                              const float (&g)[kGroups]) {
    const int j = pos & 3;
    const int b = (2 * j) & 3;  // byte index of sub-block 2j (and 2j+1 = b+1)
    const bool high = j >= 2;
    const uint32_t s0 = r.hdr.y, s4 = r.hdr.z, s8 = r.hdr.w;
    // get-scale-min-k4-at (llambda.lisp:4316-4336) for sub-blocks 2j, 2j+1
    const uint32_t B0a = (s0 >> (8 * b)) & 0xFFu, B0b = (s0 >> (8 * b + 8)) & 0xFFu;
    const uint32_t B4a = (s4 >> (8 * b)) & 0xFFu, B4b = (s4 >> (8 * b + 8)) & 0xFFu;
    const uint32_t B8a = (s8 >> (8 * b)) & 0xFFu, B8b = (s8 >> (8 * b + 8)) & 0xFFu;
    const uint32_t sc0 = high ? ((B8a & 15u) | ((B0a >> 6) << 4)) : (B0a & 63u);
    const uint32_t m0 = high ? ((B8a >> 4) | ((B4a >> 6) << 4)) : (B4a & 63u);
    const uint32_t sc1 = high ? ((B8b & 15u) | ((B0b >> 6) << 4)) : (B0b & 63u);
    const uint32_t m1 = high ? ((B8b >> 4) | ((B4b >> 6) << 4)) : (B4b & 63u);
    const float d = half_bits_to_float(r.hdr.x & 0xFFFFu);
    const float dmin = half_bits_to_float(r.hdr.x >> 16);
    const uint32_t qw[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    float al = 0.f, ah = 0.f;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const uint32_t lo = opaque(qw[w] & 0x0F0F0F0Fu);
      const uint32_t hi = opaque((qw[w] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        al = fmaf(ubyte(lo, k), x[4 * w + k], al);
        ah = fmaf(ubyte(hi, k), x[32 + 4 * w + k], ah);
      }
    }
    float v = (d * (float)sc0) * al;
    v = fmaf(-(dmin * (float)m0), g[0], v);
    v = fmaf(d * (float)sc1, ah, v);
    v = fmaf(-(dmin * (float)m1), g[1], v);
    return v;
  }
};

// ------------------------------------------------------------------ Q6_K
template <>
struct Pos<kQ6_K> {
  static constexpr int kGroups = 4;
  // Every field of a position sits at an offset from the block start that is
  // a multiple of 4, so one shift (block start & 3, which is 0 or 2) realigns
  // them all.
  struct Raw {
    uint32_t qla[5], qlb[5], qh[5];
    uint32_t sc[3];  // bytes [192+8h, 200+8h): scales 8h..8h+7
    uint32_t dw;     // dword holding d (bytes 208..209)
    uint32_t shift;
  };
  // element 16k + i of the position -> 256 b + 128 h + 32 k + 16 half + i
  static __device__ __forceinline__ int x_index(int pos, int e) {
    const int q = pos & 3, h = q >> 1, half = q & 1;
    return (pos >> 2) * 256 + 128 * h + 32 * (e >> 4) + 16 * half + (e & 15);
  }
  static __device__ __forceinline__ void group_sums(const float (&x)[64], float (&g)[kGroups]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) g[k] = sum16(x + 16 * k);
  }
  template <int N>
  static __device__ __forceinline__ void load_words(const uint32_t* base, uint32_t (&out)[N]) {
    if constexpr (N == 5) {
      const u32x4a4 v = *reinterpret_cast<const u32x4a4*>(base);
      out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
      out[4] = base[4];
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) out[i] = base[i];
    }
  }
  static __device__ __forceinline__ Raw load(const uint8_t* row, int pos) {
    const uint8_t* blk = row + (pos >> 2) * 210;
    const int q = pos & 3, h = q >> 1, half = q & 1;
    Raw r;
    r.shift = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3u);
    const uint32_t* base = reinterpret_cast<const uint32_t*>(blk - r.shift);
    load_words(base + 16 * h + 4 * half, r.qla);        // byte 64h + 16half
    load_words(base + 16 * h + 8 + 4 * half, r.qlb);    // byte 64h + 32 + 16half
    load_words(base + 32 + 8 * h + 4 * half, r.qh);     // byte 128 + 32h + 16half
    load_words(base + 48 + 2 * h, r.sc);                // byte 192 + 8h
    r.dw = base[52];                                    // byte 208
    return r;
  }
  static __device__ __forceinline__ uint32_t get(const uint32_t* w, int i, uint32_t shift) {
    return __builtin_amdgcn_alignbyte(w[i + 1], w[i], shift);
  }
  static __device__ __forceinline__ float dot(const Raw& r, int pos, const float (&x)[64],
                                              const float (&g)[kGroups]) {
    const int half = pos & 1;
    const float d = half_bits_to_float((r.dw >> (8 * r.shift)) & 0xFFFFu);
    // scales sc[8h + half + 2k], k = 0..3: bytes half, half+2, half+4, half+6 of sc
    const uint32_t t0 = get(r.sc, 0, r.shift), t1 = get(r.sc, 1, r.shift);
    float delta[4];
    delta[0] = d * (float)(int)(int8_t)((t0 >> (8 * half)) & 0xFFu);
    delta[1] = d * (float)(int)(int8_t)((t0 >> (8 * half + 16)) & 0xFFu);
    delta[2] = d * (float)(int)(int8_t)((t1 >> (8 * half)) & 0xFFu);
    delta[3] = d * (float)(int)(int8_t)((t1 >> (8 * half + 16)) & 0xFFu);
    float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t la = get(r.qla, w, r.shift), lb = get(r.qlb, w, r.shift);
      const uint32_t hq = get(r.qh, w, r.shift);
      const uint32_t q0 = (la & 0x0F0F0F0Fu) | ((hq & 0x03030303u) << 4);
      const uint32_t q1 = (lb & 0x0F0F0F0Fu) | (((hq >> 2) & 0x03030303u) << 4);
      const uint32_t q2 = ((la >> 4) & 0x0F0F0F0Fu) | (((hq >> 4) & 0x03030303u) << 4);
      const uint32_t q3 = ((lb >> 4) & 0x0F0F0F0Fu) | (((hq >> 6) & 0x03030303u) << 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        s[0] = fmaf(ubyte(q0, k), x[4 * w + k], s[0]);
        s[1] = fmaf(ubyte(q1, k), x[16 + 4 * w + k], s[1]);
        s[2] = fmaf(ubyte(q2, k), x[32 + 4 * w + k], s[2]);
        s[3] = fmaf(ubyte(q3, k), x[48 + 4 * w + k], s[3]);
      }
    }
    float v = delta[0] * fmaf(-32.f, g[0], s[0]);
#pragma unroll
    for (int k = 1; k < 4; ++k) v = fmaf(delta[k], fmaf(-32.f, g[k], s[k]), v);
    return v;
  }
};

// ------------------------------------------------------- Q8_0 (two blocks)
template <>
struct Pos<kQ8_0> {
  static constexpr int kGroups = 2;
  struct Raw {
    uint32_t w[18];  // 68 bytes of two blocks (+ alignment), realigned lazily
    uint32_t shift;
  };
  static __device__ __forceinline__ int x_index(int pos, int e) { return pos * 64 + e; }
  static __device__ __forceinline__ void group_sums(const float (&x)[64], float (&g)[kGroups]) {
    g[0] = sum16(x) + sum16(x + 16);
    g[1] = sum16(x + 32) + sum16(x + 48);
  }
  static __device__ __forceinline__ Raw load(const uint8_t* row, int pos) {
    const uint8_t* p = row + pos * 68;
    Raw r;
    r.shift = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint32_t* base = reinterpret_cast<const uint32_t*>(p - r.shift);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4a4 v = *reinterpret_cast<const u32x4a4*>(base + 4 * i);
      r.w[4 * i] = v.x; r.w[4 * i + 1] = v.y; r.w[4 * i + 2] = v.z; r.w[4 * i + 3] = v.w;
    }
    r.w[16] = base[16];
    r.w[17] = base[17];
    return r;
  }
  static __device__ __forceinline__ uint32_t byte4(const Raw& r, int off) {
    // 4 bytes at byte offset `off` (even) of the two-block span
    const int i = off >> 2;
    const uint32_t s = r.shift + (uint32_t)(off & 3);
    return s >= 4 ? __builtin_amdgcn_alignbyte(r.w[i + 2], r.w[i + 1], s - 4)
                  : __builtin_amdgcn_alignbyte(r.w[i + 1], r.w[i], s);
  }
  static __device__ __forceinline__ float dot(const Raw& r, int pos, const float (&x)[64],
                                              const float (&g)[kGroups]) {
    float v = 0.f;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      const float d = half_bits_to_float(byte4(r, 34 * blk) & 0xFFFFu);
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        const uint32_t q = byte4(r, 34 * blk + 2 + 4 * w) ^ 0x80808080u;
#pragma unroll
        for (int k = 0; k < 4; ++k) s = fmaf(ubyte(q, k), x[32 * blk + 4 * w + k], s);
      }
      v = fmaf(d, fmaf(-128.f, g[blk], s), v);
    }
    return v;
  }
};

// ------------------------------------------------------- Q5_0 (two blocks)
template <>
struct Pos<kQ5_0> {
  static constexpr int kGroups = 2;
  struct Raw {
    uint32_t w[12];  // 44 bytes of two blocks (+ alignment)
    uint32_t shift;
  };
  static __device__ __forceinline__ int x_index(int pos, int e) { return pos * 64 + e; }
  static __device__ __forceinline__ void group_sums(const float (&x)[64], float (&g)[kGroups]) {
    g[0] = sum16(x) + sum16(x + 16);
    g[1] = sum16(x + 32) + sum16(x + 48);
  }
  static __device__ __forceinline__ Raw load(const uint8_t* row, int pos) {
    const uint8_t* p = row + pos * 44;
    Raw r;
    r.shift = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint32_t* base = reinterpret_cast<const uint32_t*>(p - r.shift);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const u32x4a4 v = *reinterpret_cast<const u32x4a4*>(base + 4 * i);
      r.w[4 * i] = v.x; r.w[4 * i + 1] = v.y; r.w[4 * i + 2] = v.z; r.w[4 * i + 3] = v.w;
    }
    return r;
  }
  static __device__ __forceinline__ uint32_t byte4(const Raw& r, int off) {
    const int i = off >> 2;
    const uint32_t s = r.shift + (uint32_t)(off & 3);
    return s >= 4 ? __builtin_amdgcn_alignbyte(r.w[i + 2], r.w[i + 1], s - 4)
                  : __builtin_amdgcn_alignbyte(r.w[i + 1], r.w[i], s);
  }
  static __device__ __forceinline__ uint32_t spread4(uint32_t nib) {
    return ((nib * 0x00204081u) & 0x01010101u) << 4;
  }
  static __device__ __forceinline__ float dot(const Raw& r, int pos, const float (&x)[64],
                                              const float (&g)[kGroups]) {
    float v = 0.f;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      const float d = half_bits_to_float(byte4(r, 22 * blk) & 0xFFFFu);
      const uint32_t qh = byte4(r, 22 * blk + 2);
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t qs = byte4(r, 22 * blk + 6 + 4 * w);
        const uint32_t lo = (qs & 0x0F0F0F0Fu) | spread4((qh >> (4 * w)) & 0xFu);
        const uint32_t hi = ((qs >> 4) & 0x0F0F0F0Fu) | spread4((qh >> (16 + 4 * w)) & 0xFu);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          s = fmaf(ubyte(lo, k), x[32 * blk + 4 * w + k], s);
          s = fmaf(ubyte(hi, k), x[32 * blk + 16 + 4 * w + k], s);
        }
      }
      v = fmaf(d, fmaf(-16.f, g[blk], s), v);
    }
    return v;
  }
};

}  // namespace llhip
