// units.h -- per-lane dequant-dot of one 32-weight "unit" of a packed row.
//
// Every supported block type is cut into units of 32 weights so that one
// lane handles one unit and a wavefront sweeps a row 64 units (2048 weights)
// at a time:
//   Q4_K: 8 units per 144-byte super-block.  Unit t holds qs bytes
//         [16t, 16t+16): 16 low nibbles of sub-block 2j and 16 high nibbles
//         of sub-block 2j+1 (j = t/2), the pairing of llambda.lisp:4360-4382.
//   Q6_K: 8 units per 210-byte super-block.  Unit t holds ql bytes
//         [16t, 16t+16) and the matching 16 qh bytes; its weights are the
//         q_k pairs (k, k+2) of llambda.lisp:4203-4310 for one half.
//   Q5_0, Q8_0: one unit per 32-weight block.
//
// The dot is evaluated as  sum_g delta_g * (sum_i u_i * x_i  -  c_g * sum_i x_i)
// per 16-weight group g, where u_i is the unsigned code read from the bits,
// c_g the code offset (Q4_K: min/delta, Q6_K: 32, Q5_0: 16, Q8_0: 128) and
// sum_i x_i comes precomputed from LDS.  The reference forms each weight
// first (w = fl(fl(q*delta) - min)) and accumulates w*x; the two orders agree
// to fp32 rounding, which the parity bound 1e-4 * sum|w*x| per row covers.
//
// Loads are split from arithmetic (Raw structs) so a caller can issue the
// loads of several rows before the first multiply.
#pragma once

#include "common.h"

namespace llhip {

// x for NT tokens lives in LDS as xs[tok * xs_stride + k] and the sums of
// its 16-element groups as xg[tok * xg_stride + k/16].
struct XView {
  const float* xs;
  const float* xg;
  int xs_stride;
  int xg_stride;
};

template <int TYPE>
struct Unit;

// ---------------------------------------------------------------- Q4_K
template <>
struct Unit<kQ4_K> {
  struct Raw {
    uint4 hdr;  // d, dmin, scales[0..11]
    uint4 q;    // 16 qs bytes
  };
  static __device__ __forceinline__ const uint8_t* block_ptr(const uint8_t* row, int unit) {
    return row + (unit >> 3) * 144;
  }
  static __device__ __forceinline__ Raw load(const uint8_t* row, int unit) {
    const uint8_t* blk = block_ptr(row, unit);
    Raw r;
    r.hdr = load16_aligned(blk);
    r.q = load16_aligned(blk + 16 + 16 * (unit & 7));
    return r;
  }
  // (scale, min) of sub-block s per get-scale-min-k4-at (llambda.lisp:4316-4336).
  static __device__ __forceinline__ void scale_min(const uint4& hdr, int s, int& sc, int& m) {
    int b = s & 3;
    uint32_t B0 = (hdr.y >> (8 * b)) & 0xFFu;  // S[b]
    uint32_t B4 = (hdr.z >> (8 * b)) & 0xFFu;  // S[b+4]
    uint32_t B8 = (hdr.w >> (8 * b)) & 0xFFu;  // S[b+8]
    if (s < 4) {
      sc = (int)(B0 & 63u);
      m = (int)(B4 & 63u);
    } else {
      sc = (int)((B8 & 15u) | ((B0 >> 6) << 4));
      m = (int)((B8 >> 4) | ((B4 >> 6) << 4));
    }
  }
  template <int NT>
  static __device__ __forceinline__ void dot(const Raw& r, int unit, const XView& xv, float (&acc)[NT]) {
    const int t = unit & 7, j = t >> 1, half = t & 1;
    int sc0, m0, sc1, m1;
    scale_min(r.hdr, 2 * j, sc0, m0);
    scale_min(r.hdr, 2 * j + 1, sc1, m1);
    const float d = half_bits_to_float(r.hdr.x & 0xFFFFu);
    const float dmin = half_bits_to_float(r.hdr.x >> 16);
    const float delta0 = d * (float)sc0, off0 = dmin * (float)m0;
    const float delta1 = d * (float)sc1, off1 = dmin * (float)m1;
    float wl[16], wh[16];
    const uint32_t qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t lo = opaque(qw[w] & 0x0F0F0F0Fu);
      uint32_t hi = opaque((qw[w] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        wl[4 * w + k] = ubyte(lo, k);
        wh[4 * w + k] = ubyte(hi, k);
      }
    }
    const int xl = (unit >> 3) * 256 + 64 * j + 16 * half;
    const int xh = xl + 32;
#pragma unroll
    for (int tok = 0; tok < NT; ++tok) {
      const float4* pl = reinterpret_cast<const float4*>(xv.xs + tok * xv.xs_stride + xl);
      const float4* ph = reinterpret_cast<const float4*>(xv.xs + tok * xv.xs_stride + xh);
      float al = 0.f, ah = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        float4 a = pl[w];
        float4 b = ph[w];
        al = fmaf(wl[4 * w + 0], a.x, al);
        al = fmaf(wl[4 * w + 1], a.y, al);
        al = fmaf(wl[4 * w + 2], a.z, al);
        al = fmaf(wl[4 * w + 3], a.w, al);
        ah = fmaf(wh[4 * w + 0], b.x, ah);
        ah = fmaf(wh[4 * w + 1], b.y, ah);
        ah = fmaf(wh[4 * w + 2], b.z, ah);
        ah = fmaf(wh[4 * w + 3], b.w, ah);
      }
      const float gl = xv.xg[tok * xv.xg_stride + (xl >> 4)];
      const float gh = xv.xg[tok * xv.xg_stride + (xh >> 4)];
      float v = acc[tok];
      v = fmaf(delta0, al, v);
      v = fmaf(-off0, gl, v);
      v = fmaf(delta1, ah, v);
      v = fmaf(-off1, gh, v);
      acc[tok] = v;
    }
  }
};

// ---------------------------------------------------------------- Q6_K
template <>
struct Unit<kQ6_K> {
  struct Raw {
    uint4 ql;
    uint4 qh;
    uint4 sc;       // scales[0..15]
    uint32_t dword; // d in the low 16 bits
  };
  static __device__ __forceinline__ Raw load(const uint8_t* row, int unit) {
    const uint8_t* blk = row + (unit >> 3) * 210;
    const int t = unit & 7, h = t >> 2, half = t & 1;
    Raw r;
    r.ql = load16_unaligned2(blk + 16 * t);
    r.qh = load16_unaligned2(blk + 128 + 32 * h + 16 * half);
    // scales at 192..207 and d at 208..209, from the dwords that hold them
    const uint32_t shift = (uint32_t)(reinterpret_cast<uintptr_t>(blk + 192) & 3u);
    const uint32_t* base = reinterpret_cast<const uint32_t*>(blk + 192 - shift);
    u32x4a4 v = *reinterpret_cast<const u32x4a4*>(base);
    uint32_t e = base[4];
    r.sc.x = __builtin_amdgcn_alignbyte(v.y, v.x, shift);
    r.sc.y = __builtin_amdgcn_alignbyte(v.z, v.y, shift);
    r.sc.z = __builtin_amdgcn_alignbyte(v.w, v.z, shift);
    r.sc.w = __builtin_amdgcn_alignbyte(e, v.w, shift);
    r.dword = e >> (8 * shift);
    return r;
  }
  static __device__ __forceinline__ int scale_at(const uint4& sc, int i) {
    uint32_t w = (i < 4) ? sc.x : (i < 8) ? sc.y : (i < 12) ? sc.z : sc.w;
    return (int)(int8_t)((w >> (8 * (i & 3))) & 0xFFu);
  }
  template <int NT>
  static __device__ __forceinline__ void dot(const Raw& r, int unit, const XView& xv, float (&acc)[NT]) {
    const int t = unit & 7, h = t >> 2, part = (t >> 1) & 1, half = t & 1;
    const float d = half_bits_to_float(r.dword & 0xFFFFu);
    const int ia = 8 * h + half + 2 * part;  // scale of q_k, k = part
    const float delta_a = d * (float)scale_at(r.sc, ia);
    const float delta_b = d * (float)scale_at(r.sc, ia + 4);  // k = part + 2
    const int sa = 2 * part, sb = 4 + 2 * part;
    float wa[16], wb[16];
    const uint32_t lqw[4] = {r.ql.x, r.ql.y, r.ql.z, r.ql.w};
    const uint32_t hqw[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t qa = (lqw[w] & 0x0F0F0F0Fu) | (((hqw[w] >> sa) & 0x03030303u) << 4);
      uint32_t qb = ((lqw[w] >> 4) & 0x0F0F0F0Fu) | (((hqw[w] >> sb) & 0x03030303u) << 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        wa[4 * w + k] = ubyte(qa, k);
        wb[4 * w + k] = ubyte(qb, k);
      }
    }
    const int xa = (unit >> 3) * 256 + 128 * h + 32 * part + 16 * half;
    const int xb = xa + 64;
#pragma unroll
    for (int tok = 0; tok < NT; ++tok) {
      const float4* pa = reinterpret_cast<const float4*>(xv.xs + tok * xv.xs_stride + xa);
      const float4* pb = reinterpret_cast<const float4*>(xv.xs + tok * xv.xs_stride + xb);
      float sa_ = 0.f, sb_ = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        float4 a = pa[w];
        float4 b = pb[w];
        sa_ = fmaf(wa[4 * w + 0], a.x, sa_);
        sa_ = fmaf(wa[4 * w + 1], a.y, sa_);
        sa_ = fmaf(wa[4 * w + 2], a.z, sa_);
        sa_ = fmaf(wa[4 * w + 3], a.w, sa_);
        sb_ = fmaf(wb[4 * w + 0], b.x, sb_);
        sb_ = fmaf(wb[4 * w + 1], b.y, sb_);
        sb_ = fmaf(wb[4 * w + 2], b.z, sb_);
        sb_ = fmaf(wb[4 * w + 3], b.w, sb_);
      }
      const float ga = xv.xg[tok * xv.xg_stride + (xa >> 4)];
      const float gb = xv.xg[tok * xv.xg_stride + (xb >> 4)];
      float v = acc[tok];
      v = fmaf(delta_a, fmaf(-32.f, ga, sa_), v);
      v = fmaf(delta_b, fmaf(-32.f, gb, sb_), v);
      acc[tok] = v;
    }
  }
};

// ------------------------------------------------------ 32-weight blocks
// Reads the `ND` dwords at the 2-byte-aligned address p (ND+1 dword loads).
template <int ND>
__device__ __forceinline__ void load_dwords_unaligned2(const uint8_t* p, uint32_t (&out)[ND]) {
  const uint32_t shift = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3u);
  const uint32_t* base = reinterpret_cast<const uint32_t*>(p - shift);
  uint32_t raw[ND + 1];
#pragma unroll
  for (int i = 0; i <= ND; ++i) raw[i] = base[i];
#pragma unroll
  for (int i = 0; i < ND; ++i) out[i] = __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], shift);
}

// Q8_0: d, 32 x int8.  Code u = q ^ 0x80 (0..255) so q = u - 128.
template <>
struct Unit<kQ8_0> {
  struct Raw {
    uint32_t w[9];  // bytes 0..35 of the block (the last 2 are padding)
  };
  static __device__ __forceinline__ Raw load(const uint8_t* row, int unit) {
    Raw r;
    load_dwords_unaligned2<9>(row + unit * 34, r.w);
    return r;
  }
  template <int NT>
  static __device__ __forceinline__ void dot(const Raw& r, int unit, const XView& xv, float (&acc)[NT]) {
    const float d = half_bits_to_float(r.w[0] & 0xFFFFu);
    float u[32];
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      // quant byte 4w+k sits at block byte 2+4w+k
      uint32_t v = __builtin_amdgcn_alignbyte(r.w[w + 1], r.w[w], 2) ^ 0x80808080u;
#pragma unroll
      for (int k = 0; k < 4; ++k) u[4 * w + k] = ubyte(v, k);
    }
    const int x0 = unit * 32;
#pragma unroll
    for (int tok = 0; tok < NT; ++tok) {
      const float4* p = reinterpret_cast<const float4*>(xv.xs + tok * xv.xs_stride + x0);
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        float4 a = p[w];
        s = fmaf(u[4 * w + 0], a.x, s);
        s = fmaf(u[4 * w + 1], a.y, s);
        s = fmaf(u[4 * w + 2], a.z, s);
        s = fmaf(u[4 * w + 3], a.w, s);
      }
      const float g = xv.xg[tok * xv.xg_stride + 2 * unit] + xv.xg[tok * xv.xg_stride + 2 * unit + 1];
      acc[tok] = fmaf(d, fmaf(-128.f, g, s), acc[tok]);
    }
  }
};

// Q5_0: d, u32 qh, 16 nibble bytes.  Code u = nibble | high bit << 4, q = u - 16.
template <>
struct Unit<kQ5_0> {
  struct Raw {
    uint32_t w[6];  // bytes 0..23 (the last 2 are padding)
  };
  static __device__ __forceinline__ Raw load(const uint8_t* row, int unit) {
    Raw r;
    load_dwords_unaligned2<6>(row + unit * 22, r.w);
    return r;
  }
  // bits b0..b3 -> bit 4 of bytes 0..3
  static __device__ __forceinline__ uint32_t spread4(uint32_t nib) {
    return ((nib * 0x00204081u) & 0x01010101u) << 4;
  }
  template <int NT>
  static __device__ __forceinline__ void dot(const Raw& r, int unit, const XView& xv, float (&acc)[NT]) {
    const float d = half_bits_to_float(r.w[0] & 0xFFFFu);
    const uint32_t qh = __builtin_amdgcn_alignbyte(r.w[1], r.w[0], 2);
    float ul[16], uh[16];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      // qs bytes 4w..4w+3 sit at block bytes 6+4w..
      uint32_t qs = __builtin_amdgcn_alignbyte(r.w[w + 2], r.w[w + 1], 2);
      uint32_t lo = (qs & 0x0F0F0F0Fu) | spread4((qh >> (4 * w)) & 0xFu);
      uint32_t hi = ((qs >> 4) & 0x0F0F0F0Fu) | spread4((qh >> (16 + 4 * w)) & 0xFu);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        ul[4 * w + k] = ubyte(lo, k);
        uh[4 * w + k] = ubyte(hi, k);
      }
    }
    const int x0 = unit * 32;
#pragma unroll
    for (int tok = 0; tok < NT; ++tok) {
      const float4* p = reinterpret_cast<const float4*>(xv.xs + tok * xv.xs_stride + x0);
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        float4 a = p[w];
        float4 b = p[4 + w];
        s = fmaf(ul[4 * w + 0], a.x, s);
        s = fmaf(ul[4 * w + 1], a.y, s);
        s = fmaf(ul[4 * w + 2], a.z, s);
        s = fmaf(ul[4 * w + 3], a.w, s);
        s = fmaf(uh[4 * w + 0], b.x, s);
        s = fmaf(uh[4 * w + 1], b.y, s);
        s = fmaf(uh[4 * w + 2], b.z, s);
        s = fmaf(uh[4 * w + 3], b.w, s);
      }
      const float g = xv.xg[tok * xv.xg_stride + 2 * unit] + xv.xg[tok * xv.xg_stride + 2 * unit + 1];
      acc[tok] = fmaf(d, fmaf(-16.f, g, s), acc[tok]);
    }
  }
};

// ------------------------------------------------------------------ staging
// Copy NT activation rows into LDS (rows with a null source become zero) and
// form the sums of each 16-element group.  Four consecutive threads stage one
// group, so the group sum is two shuffles.  K must be a multiple of 32.
template <int NT>
__device__ __forceinline__ void stage_rows(float* xs, float* xg, const float* const* src, int K) {
  const int n4 = K >> 2;
  const int total = NT * n4;
  for (int i = threadIdx.x; i < total; i += blockDim.x) {
    const int tok = i / n4, k4 = i - tok * n4;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (src[tok]) v = reinterpret_cast<const float4*>(src[tok])[k4];
    reinterpret_cast<float4*>(xs + tok * K)[k4] = v;
    float s = (v.x + v.y) + (v.z + v.w);
    s += __shfl_xor(s, 1, kWave);
    s += __shfl_xor(s, 2, kWave);
    if ((k4 & 3) == 0) xg[tok * (K >> 4) + (k4 >> 2)] = s;
  }
}

template <int NT>
__device__ __forceinline__ void stage_x(float* xs, float* xg, const float* __restrict__ x,
                                        int64_t x_stride, int ntok, int K) {
  const float* src[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) src[t] = t < ntok ? x + t * x_stride : nullptr;
  stage_rows<NT>(xs, xg, src, K);
}

// Dot of R packed rows (row pointers rp) with NT staged activations: lane l of
// a `lpr`-lane slot covers units l, l + lpr, ...; the caller sums the slot.
template <int TYPE, int NT, int R>
__device__ __forceinline__ void rows_dot(const uint8_t* const (&rp)[R], const bool (&valid)[R],
                                         int l, int lpr, int units, const XView& xv,
                                         float (&acc)[R][NT]) {
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[r][t] = 0.f;
  for (int u0 = 0; u0 < units; u0 += lpr) {
    const int u = u0 + l;
    typename Unit<TYPE>::Raw raw[R];
    bool ok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      ok[r] = (u < units) && valid[r];
      if (ok[r]) raw[r] = Unit<TYPE>::load(rp[r], u);
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (ok[r]) Unit<TYPE>::template dot<NT>(raw[r], u, xv, acc[r]);
  }
}

__host__ __device__ inline int lanes_per_row_log2(int K) {
  const int units = K >> 5;
  int l = 0;
  while ((1 << l) < units && l < 6) ++l;
  return l;
}

}  // namespace llhip
