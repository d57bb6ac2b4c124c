// moe_mfma.hip -- the routed-MoE products on MFMA.
//
//   router_mfma_kernel  the F32 router as a GEMM on v_mfma_f32_16x16x4_f32
//                       (fp32 products, fp32 accumulation) in K slices of 512,
//                       and the tokens' "split rows": every element as two
//                       bf16 (hi + lo, |x - hi - lo| <= 2^-17 |x|) plus the
//                       sum of each 16-element group of fl(hi) + fl(lo).
//   moe_gemm_kernel     the grouped expert products over the chunk table
//                       (expert, up to 16*MT (token, rank) pairs): gate/up
//                       with silu(g)*u or relu(u)^2 fused, or down.
//
// Expert products.  The weights stay the tensor's GGUF super-blocks.  Each
// wavefront owns 16-row subtiles of one or two matrices (gate and up side by
// side) and streams them through LDS in 256-element K chunks
// (global_load_lds_dwordx4: coalesced, no VGPR round trip).  Per chunk every
// lane first decodes the scales of its share of the chunk's scale groups into
// a per-wave table (delta, -c), then, group by group, turns its 8 (or 4)
// codes into exact bf16 values 128 + q (v_perm_b32 with the filler byte 0x43)
// -- the B operand of a 16x16x32 (Q6_K's 16-weight groups: 16x16x16) bf16
// MFMA whose A operand is 16 tokens' hi, then lo, activations.  Per scale
// group g of row n
//     sum_k w_k x_k = delta_g * sum_k (128 + q_k) x_k  -  c_g * sum_k x_k
// with c_g = 128 delta_g + mu_g (Q4_K), 160 delta_g (Q6_K: q - 32),
// 144 delta_g (Q5_0: q - 16), 128 delta_g (Q8_0: codes q ^ 0x80).  The first
// term is one VALU fma per output per group; the second is itself a product
// over groups, done at the end of each chunk as v_mfma_f32_16x16x4_f32 of the
// group sums (A) with -c (B).  The reference forms every weight first
// (w = fl(fl(q delta) - mu)) and accumulates w x in fp32; both are fp32
// evaluations of the same sum and differ by rounding, inside the bound
// 1e-4 sum|w x| per output.
//
// The two batch pipelines share that arithmetic instruction for instruction,
// so a token's output does not depend on the batch (of two or more) it runs
// in:
//   kPipeWide    2 token tiles (chunks of up to 32 pairs): 4 waves x 64
//                rows, one LDS stage per wave; latency is hidden by the
//                other waves of the SIMD, the MFMA work per chunk is long.
//                The chunk's group sums and first group's activations load
//                with its rows, later groups' activations two groups ahead.
//   kPipeDouble  1 token tile: 4 waves x 32 rows (16 + 16 for gate and
//                up), in one of three forms chosen by what fits:
//                16-byte fragments whose rows fit 53 KB with the chunk's
//                activations: those shared through LDS (a quarter loaded by
//                each wave), one row stage per wave, three workgroups per
//                CU; otherwise, when one row stage fits 53 KB, the wide
//                loop above with one row stage; else two LDS stages per
//                wave, chunk kc + 1 (rows by DMA, activations and group sums
//                into registers) loading while chunk kc computes, and with
//                at most four chunks in K two row tiles per workgroup.
// In every pipeline the LDS words of group j + 1 are read while group j
// decodes and multiplies, and rows sit an odd number of 16-byte pieces apart
// in LDS so that the 16 rows of one read fall in different bank quads.
//   moe_group_kernel  4 token tiles (chunks of up to 64 pairs), 32-weight
//                block types only: the chunk's activations staged once per
//                workgroup by DMA and shared by its four waves, every DMA
//                instruction reading whole 16-byte runs of a few rows (see
//                below).
//   kPipeDecode  one token: 4 waves share 32 rows and split K (wave w takes
//                chunks w, w + 4, ...), each through a ring of up to 8 LDS
//                stages of rows, the token's activations and group sums,
//                loaded by DMA ahead of use; the four partial sums are added
//                in wave order.  Its sums therefore run in another order than
//                the batch pipelines' (same bound).
#include "activations.h"
#include "mfma.h"
#include "moe.h"
#include "moe_gate.h"

#include <algorithm>
#include <type_traits>

namespace llhip {

// s_waitcnt immediates (gfx9 encoding: vmcnt [3:0] and [15:14], expcnt
// [6:4], lgkmcnt [11:8]).  Issued through the builtin so the compiler's own
// wait insertion knows the counters were drained.
constexpr int waitcnt_vm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }
constexpr int kWaitLgkm0 = 0xC07F;

// ------------------------------------------------------------ split rows
// Row r of K elements (K % 32 == 0):
//   q + r * q_stride (u16): for each 32-group j, [64j, 64j + 32) = hi bf16 of
//       elements 32j .. 32j + 31 and [64j + 32, 64j + 64) = their lo bf16.
//   s + r * s_stride (f32): [0, K/16) = sums of the 16-groups, each of
//       fl(hi) + fl(lo) over the group.  A 32-group's sum is always formed as
//       s[2j] + s[2j + 1].
// Octet o (elements 8o .. 8o+7) of a row; lanes o and o ^ 1 must both run it.
__device__ __forceinline__ void split_octet(const float* __restrict__ xrow, int o,
                                            uint16_t* __restrict__ qrow, float* __restrict__ srow) {
  const float4* xp = reinterpret_cast<const float4*>(xrow + 8 * o);
  const float4 a = xp[0], b = xp[1];
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t hi[4], lo[4];
  float t[8];
#pragma unroll
  for (int e = 0; e < 8; e += 2) split_bf16_pair(v[e], v[e + 1], hi[e / 2], lo[e / 2], t[e], t[e + 1]);
  float sum = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) sum += t[e];
  uint16_t* dst = qrow + 64 * (o >> 2) + 8 * (o & 3);
  *reinterpret_cast<u32x4*>(dst) = u32x4{hi[0], hi[1], hi[2], hi[3]};
  *reinterpret_cast<u32x4*>(dst + 32) = u32x4{lo[0], lo[1], lo[2], lo[3]};
  const float s16 = sum + dpp<kDppXor1>(sum);
  if ((o & 1) == 0) srow[o >> 1] = s16;
}

// One thread per octet of the T rows (a row's K / 8 octets are a multiple of
// four, so octets o and o ^ 1 always sit in neighbouring lanes).
__global__ void __launch_bounds__(256)
split_rows_kernel(const float* __restrict__ x, int T, int K, int64_t x_stride,
                  uint16_t* __restrict__ q, int64_t q_stride, float* __restrict__ s,
                  int64_t s_stride) {
  const int octets = K >> 3;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)T * octets) return;
  const int t = (int)(idx / octets), o = (int)(idx - (int64_t)t * octets);
  split_octet(x + t * x_stride, o, q + t * q_stride, s + t * s_stride);
}

hipError_t split_rows_launch(const float* x, int T, int K, int64_t x_stride, uint16_t* q,
                             int64_t q_stride, float* s, int64_t s_stride, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  if (K <= 0 || K % 32 || x_stride % 4 || q_stride % 8) return hipErrorInvalidValue;
  const int64_t threads = (int64_t)T * (K >> 3);
  hipLaunchKernelGGL(split_rows_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     stream, x, T, K, x_stride, q, q_stride, s, s_stride);
  return hipGetLastError();
}

// -------------------------------------------------------------------- router
// Router logits sum_h x[t][h] R[e][h] (dot-product-with-f32-tensor-data,
// llambda.lisp:4096-4107, in another fp32 order), in one fixed order for
// every batch size: K is cut into slices of 512; for each 16 x 16 (token,
// expert) tile and slice, the slice's 32 pieces of 16 elements are added on
// v_mfma_f32_16x16x4_f32 -- wave w of 8 takes pieces 4w .. 4w+3, adds them as
// (p0 + p1) + (p2 + p3), and the wave sums meet as ((w0 + w1) + (w2 + w3)) +
// ((w4 + w5) + (w6 + w7)) -- and the slice's partial sum goes to
// part[slice][t][e]; the top-k kernel adds the slices in order.  A workgroup
// takes one token tile, one slice and GE expert tiles; those of the first
// expert tiles also write their tokens' split rows over their slice.
constexpr int kRouterWaves = 8;
constexpr int kRouterSlice = 512;

// GE expert tiles per workgroup: each wave loads its token tile's x pieces
// once and runs the expert tiles' products in turn (a batch's x is then read
// once per GE expert tiles instead of once per tile); wave w < GE adds the
// eight wave sums of expert tile w.  Every tile's arithmetic is the same for
// any GE.
template <int GE>
__global__ void __launch_bounds__(64 * kRouterWaves)
router_mfma_kernel(const float* __restrict__ x, int T, const float* __restrict__ R, int Er, int H,
                   float* __restrict__ part, int ld, uint16_t* __restrict__ q, int64_t q_stride,
                   float* __restrict__ s, int64_t s_stride) {
  __shared__ floatx4 red[GE][kRouterWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, kg = lane >> 4;
  const int t0 = blockIdx.y * 16, eg = blockIdx.x * 16 * GE, k0 = blockIdx.z * kRouterSlice;
  const int tiles = min(GE, (Er - eg + 15) >> 4);  // expert tiles of this workgroup
  // the products' operands are requested first, so that the split below
  // (expert-group 0) overlaps their round trip instead of preceding it
  const float* xr = x + (int64_t)min(t0 + i, T - 1) * H + 4 * kg;
  auto load_r = [&](int e0, float4 (&rb)[4]) {
    const float* rr = R + (int64_t)min(e0 + i, Er - 1) * H + 4 * kg;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int k = k0 + 64 * wave + 16 * c;
      rb[c] = k < H ? *reinterpret_cast<const float4*>(rr + k) : float4{0.f, 0.f, 0.f, 0.f};
    }
  };
  float4 xa[4], rb[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int k = k0 + 64 * wave + 16 * c;
    xa[c] = k < H ? *reinterpret_cast<const float4*>(xr + k) : float4{0.f, 0.f, 0.f, 0.f};
  }
  load_r(eg, rb);
  if (blockIdx.x == 0) {
    const int octets = min(kRouterSlice, H - k0) >> 3, ofirst = k0 >> 3;
    for (int idx = threadIdx.x; idx < 16 * octets; idx += 64 * kRouterWaves) {
      const int tt = idx / octets, o = ofirst + idx - tt * octets;
      if (t0 + tt < T)
        split_octet(x + (int64_t)(t0 + tt) * H, o, q + (int64_t)(t0 + tt) * q_stride,
                    s + (int64_t)(t0 + tt) * s_stride);
    }
  }
#pragma unroll
  for (int ge = 0; ge < GE; ++ge) {
    if (ge < tiles) {
      float4 rn[4];
      if (ge + 1 < tiles) load_r(eg + 16 * (ge + 1), rn);
      floatx4 acc[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        acc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
        if (k0 + 64 * wave + 16 * c < H) {
          acc[c] = mfma4f32(xa[c].x, rb[c].x, acc[c]);
          acc[c] = mfma4f32(xa[c].y, rb[c].y, acc[c]);
          acc[c] = mfma4f32(xa[c].z, rb[c].z, acc[c]);
          acc[c] = mfma4f32(xa[c].w, rb[c].w, acc[c]);
        }
      }
      red[ge][wave][lane] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
      if (ge + 1 < tiles)
#pragma unroll
        for (int c = 0; c < 4; ++c) rb[c] = rn[c];
    }
  }
  __syncthreads();
  for (int ge = wave; ge < tiles; ge += kRouterWaves) {
    const floatx4(&r8)[kRouterWaves][64] = red[ge];
    const floatx4 v = ((r8[0][lane] + r8[1][lane]) + (r8[2][lane] + r8[3][lane])) +
                      ((r8[4][lane] + r8[5][lane]) + (r8[6][lane] + r8[7][lane]));
    const int e = eg + 16 * ge + i;
    if (e >= Er) continue;
    float* out = part + (int64_t)blockIdx.z * T * ld;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 4 * kg + r;
      if (t < T) out[(int64_t)t * ld + e] = v[r];
    }
  }
}

int router_slices(int H) { return (H + kRouterSlice - 1) / kRouterSlice; }

hipError_t router_mfma_launch(const float* x, int T, const float* R, int Er, int H, float* part,
                              int ld, uint16_t* q, int64_t q_stride, float* s, int64_t s_stride,
                              hipStream_t stream) {
  // batches of 32 token tiles or more take eight expert tiles per
  // workgroup, of 16 or more four (a grid of 576 workgroups for 256 tokens
  // and 513 rows: Qwen3Next B=256 0.408 -> 0.404 ms against eight), smaller
  // ones one (their grid is already short)
  const int etiles = (Er + 15) / 16, ttiles = (T + 15) / 16;
  if (ttiles >= 32) {
    const dim3 grid((etiles + 7) / 8, ttiles, router_slices(H));
    hipLaunchKernelGGL(router_mfma_kernel<8>, grid, dim3(64 * kRouterWaves), 0, stream, x, T, R, Er,
                       H, part, ld, q, q_stride, s, s_stride);
  } else if (ttiles >= 16) {
    const dim3 grid((etiles + 3) / 4, ttiles, router_slices(H));
    hipLaunchKernelGGL(router_mfma_kernel<4>, grid, dim3(64 * kRouterWaves), 0, stream, x, T, R, Er,
                       H, part, ld, q, q_stride, s, s_stride);
  } else {
    const dim3 grid(etiles, ttiles, router_slices(H));
    hipLaunchKernelGGL(router_mfma_kernel<1>, grid, dim3(64 * kRouterWaves), 0, stream, x, T, R, Er,
                       H, part, ld, q, q_stride, s, s_stride);
  }
  return hipGetLastError();
}

// ------------------------------------------------------ B operand per type
// `row` is the dword-aligned LDS image of one row's chunk; the chunk's first
// byte is at row + sh (sh < 4; 0 for Q4_K).  fetch(): the LDS words holding
// lane g's codes of scale group j; decode(): those codes as bf16 128 + q
// (split so that the next group's reads are in flight while this group
// decodes and multiplies).  scale(): the group's delta and c.
// kPieces 16-byte pieces hold a chunk and its shift; rows sit kPitch bytes
// apart in LDS, an odd number of pieces, so that the 16 rows one read
// instruction touches start in 16 different bank quads (an even pitch of
// 12 or 14 pieces puts them in 2 or 4 and serialises the reads 8- or
// 4-fold).  The pad piece of each row is a second copy of its last piece.
__host__ __device__ constexpr int odd_pitch(int pieces) { return 16 * (pieces | 1); }

__device__ __forceinline__ uint32_t lds_dword(const uint8_t* row, uint32_t i) {
  return reinterpret_cast<const uint32_t*>(row)[i];
}
__device__ __forceinline__ uint32_t lds_u16_even(const uint8_t* row, uint32_t o) {
  return (lds_dword(row, o >> 2) >> (8 * (o & 3u))) & 0xFFFFu;
}
__device__ __forceinline__ uint32_t lds_u8(const uint8_t* row, uint32_t o) {
  return (lds_dword(row, o >> 2) >> (8 * (o & 3u))) & 0xFFu;
}

// Bit i of a nibble v at bit 8i: v * 0x204081 masked to bits 0, 8, 16, 24.
// Written as the 24-bit multiply (full rate) because the compiler, once it
// keeps the constant in a scalar register, emits the quarter-rate 32-bit one.
__device__ __forceinline__ uint32_t spread_nibble(uint32_t v) {
  uint32_t r;
  asm("v_mul_u32_u24 %0, 0x204081, %1" : "=v"(r) : "v"(v));
  return r & 0x01010101u;
}

template <int TYPE>
struct GemmB;

// Q4_K: chunk = one super-block (144 B), 8 groups (sub-blocks) of 32.  Lane
// g takes elements 8g .. 8g+7 of sub-block j: qs bytes 32 (j/2) + 8g .. +7,
// low nibbles for even j, high for odd (llambda.lisp:4145-4201, 6815-6859).
template <>
struct GemmB<kQ4_K> {
  static constexpr int kSpan = 144, kPieces = 9, kPitch = odd_pitch(kPieces), kSteps = 8,
                       kStepK = 32;
  static constexpr int kTilePitch = 144;  // tile-major row chunk (0: packed rows)
  static constexpr bool kWide = true;
  // c = kCd * delta (0: c also carries the block minimum)
  static constexpr float kCd = 0.f;
  typedef bf16x8 Frag;
  typedef uint2 Raw;
  static __device__ __forceinline__ Raw fetch(const uint8_t* row, uint32_t, int j, int g) {
    return lds_read8(row + 16 + 32 * (j >> 1) + 8 * g);
  }
  static __device__ __forceinline__ Frag decode(const Raw& q, uint32_t, int j, int) {
    const uint32_t c0 = (j & 1) ? (q.x >> 4) & 0x0F0F0F0Fu : q.x & 0x0F0F0F0Fu;
    const uint32_t c1 = (j & 1) ? (q.y >> 4) & 0x0F0F0F0Fu : q.y & 0x0F0F0F0Fu;
    return codes_to_b(c0, c1);
  }
  // get-scale-min-k4-at (llambda.lisp:4316-4336)
  static __device__ __forceinline__ void scale(const uint8_t* row, uint32_t, int j, float& delta,
                                               float& c) {
    const uint4 h = *reinterpret_cast<const uint4*>(row);
    const int k = j & 3;
    const uint32_t B0 = (h.y >> (8 * k)) & 0xFFu, B4 = (h.z >> (8 * k)) & 0xFFu;
    uint32_t sc, m;
    if (j < 4) {
      sc = B0 & 63u;
      m = B4 & 63u;
    } else {
      const uint32_t B8 = (h.w >> (8 * k)) & 0xFFu;
      sc = (B8 & 15u) | ((B0 >> 6) << 4);
      m = (B8 >> 4) | ((B4 >> 6) << 4);
    }
    const float d = half_bits_to_float(h.x & 0xFFFFu);
    const float dmin = half_bits_to_float(h.x >> 16);
    delta = d * (float)sc;
    c = fmaf(128.f, delta, dmin * (float)m);
  }
};

// Q6_K: chunk = one super-block (210 B), 16 scale groups of 16 elements.
// Element e = 128h + 32k + l has scale sc[e / 16] (llambda.lisp:4203-4310,
// 6919-6978); lane g takes l = 16s + 4g .. +3 of group u = 8h + 2k + s.
// The tile-major rows (moe_tile_launch) hold each 32-byte run of ql and qh
// with the words of groups 2t and 2t + 1 that lane g reads side by side
// (dword 2g + s of the run instead of 4s + g), so that one 8-byte read per
// lane serves both groups and a half wave's reads meet 32 different bank
// pairs (four-byte reads of rows 240 bytes apart put rows n and n + 8 in one
// bank).
template <>
struct GemmB<kQ6_K> {
  static constexpr int kSpan = 210, kPieces = 14, kPitch = odd_pitch(kPieces), kSteps = 16,
                       kStepK = 16;
  static constexpr int kTilePitch = 212;
  static constexpr bool kWide = false;
  static constexpr float kCd = 160.f;
  typedef shortx4 Frag;
  typedef u32x4 Raw;
  static __device__ __forceinline__ Raw fetch(const uint8_t* row, uint32_t, int u, int g) {
    const int h = u >> 3, k = (u >> 1) & 3, s = u & 1;
    const uint2 l2 = lds_read8(row + 64 * h + 32 * (k & 1) + 8 * g);
    const uint2 q2 = lds_read8(row + 128 + 32 * h + 8 * g);
    return u32x4{s ? l2.y : l2.x, 0u, s ? q2.y : q2.x, 0u};
  }
  static __device__ __forceinline__ Frag decode(const Raw& w, uint32_t, int u, int) {
    const int k = (u >> 1) & 3;
    const uint32_t ql = w[0], qh = w[2];  // tile-major: rows start on dwords
    const uint32_t nib = (ql >> (4 * (k >> 1))) & 0x0F0F0F0Fu;
    const uint32_t hb = ((qh >> (2 * k)) & 0x03030303u) << 4;
    return codes4_to_b(nib | hb);
  }
  static __device__ __forceinline__ void scale(const uint8_t* row, uint32_t sh, int u, float& delta,
                                               float& c) {
    const int sc = (int)(int8_t)lds_u8(row, sh + 192u + (uint32_t)u);
    const float d = half_bits_to_float(lds_u16_even(row, sh + 208u));
    delta = d * (float)sc;
    c = 160.f * delta;
  }
};

// Q5_0: chunk = 8 blocks of 22 B (llambda.lisp:3965-3990, 4037-4066).
// Lane g takes elements 8g .. 8g+7: qs bytes 8 (g & 1) .. +7, low nibbles
// for g < 2, high for g >= 2, fifth bits from qh bits 8g .. 8g+7, each
// moved to bit 4 of its code byte: for a nibble v, v * 0x204081 puts bit i
// of v at bit 8i (the copies shifted by 0, 7, 14 and 21 occupy disjoint
// bits, so nothing carries), and the mask keeps bits 0, 8, 16 and 24.
template <>
struct GemmB<kQ5_0> {
  static constexpr int kSpan = 176, kPieces = 12, kPitch = odd_pitch(kPieces), kSteps = 8,
                       kStepK = 32;
  static constexpr int kTilePitch = 0;
  static constexpr bool kWide = true;
  static constexpr float kCd = 144.f;
  typedef bf16x8 Frag;
  typedef u32x4 Raw;  // three words from the qs bytes' dword, the qh byte's word
  static __device__ __forceinline__ Raw fetch(const uint8_t* row, uint32_t sh, int j, int g) {
    const uint32_t o = sh + 22u * (uint32_t)j;
    const uint32_t os = (o + 6u + 8u * (uint32_t)(g & 1)) >> 2, ob = (o + 2u + (uint32_t)g) >> 2;
    return u32x4{lds_dword(row, os), lds_dword(row, os + 1u), lds_dword(row, os + 2u),
                 lds_dword(row, ob)};
  }
  static __device__ __forceinline__ Frag decode(const Raw& w, uint32_t sh, int j, int g) {
    const uint32_t o = sh + 22u * (uint32_t)j;
    const uint32_t a = (o + 6u + 8u * (uint32_t)(g & 1)) & 3u;  // 0 or 2
    const uint32_t shift = 4u * (uint32_t)(g >> 1);
    const uint32_t q0 = __builtin_amdgcn_alignbyte(w[1], w[0], a) >> shift;
    const uint32_t q1 = __builtin_amdgcn_alignbyte(w[2], w[1], a) >> shift;
    const uint32_t bit = 8u * ((o + 2u + (uint32_t)g) & 3u);
    const uint32_t h0 = spread_nibble(__builtin_amdgcn_ubfe(w[3], bit, 4u));
    const uint32_t h1 = spread_nibble(__builtin_amdgcn_ubfe(w[3], bit + 4u, 4u));
    return codes_to_b((q0 & 0x0F0F0F0Fu) | (h0 << 4), (q1 & 0x0F0F0F0Fu) | (h1 << 4));
  }
  static __device__ __forceinline__ void scale(const uint8_t* row, uint32_t sh, int j, float& delta,
                                               float& c) {
    delta = half_bits_to_float(lds_u16_even(row, sh + 22u * (uint32_t)j));
    c = 144.f * delta;
  }
};

// Q8_0: chunk = 8 blocks of 34 B (llambda.lisp:3992-4009, 4068-4094).  The
// code u = q ^ 0x80 = q + 128 (0..255) is exact in bf16 (8 significant bits).
template <>
struct GemmB<kQ8_0> {
  static constexpr int kSpan = 272, kPieces = 18, kPitch = odd_pitch(kPieces), kSteps = 8,
                       kStepK = 32;
  static constexpr int kTilePitch = 0;
  static constexpr bool kWide = true;
  static constexpr float kCd = 128.f;
  typedef bf16x8 Frag;
  static __device__ __forceinline__ uint32_t pack2(uint32_t u, int k) {
    const float f0 = (float)((u >> (8 * k)) & 0xFFu), f1 = (float)((u >> (8 * k + 8)) & 0xFFu);
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f1), __builtin_bit_cast(uint32_t, f0),
                                 0x07060302u);
  }
  typedef u32x4 Raw;  // three words from the codes' dword
  static __device__ __forceinline__ Raw fetch(const uint8_t* row, uint32_t sh, int j, int g) {
    const uint32_t os = (sh + 34u * (uint32_t)j + 2u + 8u * (uint32_t)g) >> 2;
    return u32x4{lds_dword(row, os), lds_dword(row, os + 1u), lds_dword(row, os + 2u), 0u};
  }
  static __device__ __forceinline__ Frag decode(const Raw& w, uint32_t sh, int j, int g) {
    const uint32_t a = (sh + 34u * (uint32_t)j + 2u + 8u * (uint32_t)g) & 3u;
    const uint32_t u0 = __builtin_amdgcn_alignbyte(w[1], w[0], a) ^ 0x80808080u;
    const uint32_t u1 = __builtin_amdgcn_alignbyte(w[2], w[1], a) ^ 0x80808080u;
    u32x4 v = {pack2(u0, 0), pack2(u0, 2), pack2(u1, 0), pack2(u1, 2)};
    return __builtin_bit_cast(bf16x8, v);
  }
  static __device__ __forceinline__ void scale(const uint8_t* row, uint32_t sh, int j, float& delta,
                                               float& c) {
    delta = half_bits_to_float(lds_u16_even(row, sh + 34u * (uint32_t)j));
    c = 128.f * delta;
  }
};

// A fragments of lane (t, g) for group j of chunk kc: hi then lo (8 bf16
// each for 32-groups, 4 for 16-groups).  `row` is the token's split row.
template <bool WIDE>
struct AFrag;
template <>
struct AFrag<true> {
  bf16x8 hi, lo;
  static __device__ __forceinline__ int offset(int j, int g) { return 64 * j + 8 * g; }
  __device__ __forceinline__ void load(const uint16_t* p) {
    hi = *reinterpret_cast<const bf16x8*>(p);
    lo = *reinterpret_cast<const bf16x8*>(p + 32);
  }
  // one token: the hi part in the even rows of the A operand, the lo part in
  // the odd ones (into `hi`), so one product yields both sums (rows 0, 1)
  __device__ __forceinline__ void load_pair(const uint16_t* p, int n) {
    hi = *reinterpret_cast<const bf16x8*>(p + 32 * (n & 1));
  }
  __device__ __forceinline__ void zero() {
    hi = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
    lo = hi;
  }
};
template <>
struct AFrag<false> {
  shortx4 hi, lo;
  static __device__ __forceinline__ int offset(int u, int g) {
    return 64 * (u >> 1) + 16 * (u & 1) + 4 * g;
  }
  __device__ __forceinline__ void load(const uint16_t* p) {
    hi = *reinterpret_cast<const shortx4*>(p);
    lo = *reinterpret_cast<const shortx4*>(p + 32);
  }
  __device__ __forceinline__ void load_pair(const uint16_t* p, int n) {
    hi = *reinterpret_cast<const shortx4*>(p + 32 * (n & 1));
  }
  __device__ __forceinline__ void zero() {
    hi = shortx4{0, 0, 0, 0};
    lo = hi;
  }
};

__device__ __forceinline__ floatx4 mfma_b(const bf16x8& a, const bf16x8& b, const floatx4& c) {
  return mfma32(a, b, c);
}
__device__ __forceinline__ floatx4 mfma_b(const shortx4& a, const shortx4& b, const floatx4& c) {
  return mfma16(a, b, c);
}

// ------------------------------------------------------------ tile shape
enum GemmPipe : int { kPipeWide = 0, kPipeDouble = 1, kPipeDecode = 2 };

#ifndef LLHIP_DECODE_WAVES
#define LLHIP_DECODE_WAVES 4
#endif
template <int TYPE, int EPI, int PIPE>
struct GemmShape {
  using B = GemmB<TYPE>;
  static constexpr int kWaves = PIPE == kPipeDecode ? LLHIP_DECODE_WAVES : 4;
  static constexpr int NB = EPI == kEpiSwiglu ? 2 : 1;             // gate and up side by side
  static constexpr int NS = (PIPE == kPipeWide ? 4 : 2) / NB;      // 16-row subtiles per matrix
  static constexpr int ROWS = 16 * NS;                              // rows per matrix and wave
  static constexpr int PPR = B::kPitch / 16;                        // 16-byte pieces per row
  static constexpr int PIECES = ROWS * PPR;
  static constexpr int LOADS = (PIECES + 63) / 64;                  // per matrix
  static constexpr int MATBUF = 1024 * LOADS;                       // one matrix's rows
  static constexpr int ROWBUF = MATBUF * NB;                        // rows of one chunk
  // (delta, -c) per group and row; delta alone where c = kCd * delta
  static constexpr int TABLE = NS * NB * B::kSteps * 16 * (B::kCd != 0.f ? 4 : 8);
  static constexpr int A_OFF = ROWBUF;                              // decode: the token's chunk
  static constexpr int S_OFF = ROWBUF + 1024;                       // decode: its 16 group sums
  static constexpr int STAGE = PIPE == kPipeDecode ? ROWBUF + 1024 + 256 : ROWBUF;
  static constexpr int DEPTH = PIPE == kPipeWide ? 1 : PIPE == kPipeDecode ? 8 : 2;
  static constexpr int DMA = NB * LOADS + (PIPE == kPipeDecode ? 2 : 0);  // loads per stage
  // decode: the waves' partial sums, added in wave order
  static constexpr int RED = PIPE == kPipeDecode ? kWaves * NS * NB * 64 * 16 : 0;
  // rows per workgroup: the decode waves share their rows and split K
  static constexpr int WG_ROWS = PIPE == kPipeDecode ? ROWS : kWaves * ROWS;
};

// The double pipeline with 16-byte activation fragments: the chunk's split
// activations (16 tokens x 1 KB) go into LDS once per workgroup, a quarter
// loaded by each wave, instead of every wave holding all 16 KB of the
// current and the next chunk in its registers; with one row stage per wave
// (the next chunk's rows load once the products have read the stage) the
// workgroup fits 53 KB and 160 registers, three workgroups per CU instead of
// two, whose waves cover each other's waits (Qwen3Next B=256 gate|up:
// 0.493 -> 0.452 ms for the layer).
constexpr int kShareABytes = 16 * 1024;
template <int TYPE, int EPI, int PIPE>
constexpr bool gemm_share_a() {
  using Sh = GemmShape<TYPE, EPI, PIPE>;
  return PIPE == kPipeDouble && GemmB<TYPE>::kWide &&
         Sh::RED + Sh::kWaves * (Sh::STAGE + Sh::TABLE) + kShareABytes <= 53 * 1024;
}

// The double pipeline otherwise (8-byte fragments, or rows too wide to
// share the activations beside them): when one row stage per wave and the
// scale tables fit 53 KB, it runs the wide pipeline's loop -- one stage,
// each group's activations loaded two groups ahead -- so that no wave holds
// a whole chunk's activations (current and next) in registers and three or
// four workgroups share a CU (Q6_K: 112 registers, 40 KB).
template <int TYPE, int EPI, int PIPE>
constexpr bool gemm_jit_a() {
  using Sh = GemmShape<TYPE, EPI, PIPE>;
  return PIPE == kPipeDouble && !gemm_share_a<TYPE, EPI, PIPE>() &&
         Sh::RED + Sh::kWaves * (Sh::STAGE + Sh::TABLE) <= 53 * 1024;
}

template <int TYPE, int EPI, int PIPE>
constexpr int gemm_lds_bytes(int depth) {
  using Sh = GemmShape<TYPE, EPI, PIPE>;
  if constexpr (gemm_share_a<TYPE, EPI, PIPE>())
    return Sh::RED + Sh::kWaves * (Sh::STAGE + Sh::TABLE) + kShareABytes;
  if constexpr (gemm_jit_a<TYPE, EPI, PIPE>()) return Sh::RED + Sh::kWaves * (Sh::STAGE + Sh::TABLE);
  return Sh::RED + Sh::kWaves * (depth * Sh::STAGE + Sh::TABLE);
}

// ------------------------------------------------------------ the kernel
// ALIGNED: row_bytes % 4 == 0, so every row's chunk starts at the same offset
// from a dword (Q4_K, Q5_0, Q8_0: 0; Q6_K: 2 in odd chunks).
// GATE (single-token pipeline, one token): the launch also selects and
// gates the token (gate_token) instead of reading a chunk table.
template <int TYPE, int EPI, int MT, int PIPE, bool ALIGNED, bool GATE = false>
// (two workgroups per CU: within that budget of 256 registers the compiler
// writes the MFMA results to ordinary registers instead of accumulation
// registers it then reads back one by one -- a quarter of the double
// pipeline's main-loop VALU; except for the wide pipeline of the 32-weight
// block types, whose decode state does not fit: they ran with 52-500 bytes
// of scratch per lane)
__global__ void __launch_bounds__((64 * GemmShape<TYPE, EPI, PIPE>::kWaves),
                                  (PIPE != kPipeWide || (TYPE != kQ5_0 && TYPE != kQ8_0) ? 2 : 1))
moe_gemm_kernel(MoeGemmArgs args) {
  using B = GemmB<TYPE>;
  using Sh = GemmShape<TYPE, EPI, PIPE>;
  constexpr int NB = Sh::NB, NS = Sh::NS, NQ = B::kSteps / 4, KS = B::kSteps;
  constexpr bool TILED = B::kTilePitch != 0;  // tile-major weights (K-quants)
  static_assert(!TILED || ALIGNED, "tile-major rows start on dwords");
  typedef AFrag<B::kWide> AF;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  // (chunk, row tile) of this workgroup.  Batch pipelines: a 1-D grid in
  // which the row tiles of chunk c take the workgroup ids
  // (c / 8) * 8 T + 8 k + c % 8 (k < T tiles): workgroups are dealt to the
  // eight XCDs by id modulo 8, so every row tile of a chunk runs on one XCD,
  // close in time, and the chunk's activations are fetched into its L2 once.
  int bx = blockIdx.x, by = blockIdx.y;
  if constexpr (PIPE != kPipeDecode) {
    const int T = args.row_tiles, L = blockIdx.x;
    bx = (L / (8 * T)) * 8 + (L & 7);
    by = (L >> 3) % T;
  }
  const int* cc = args.chunk_counts;
  // joint launches: routed chunks, then the shared expert's (their entries
  // follow the routed ones in the table).  Except for a separate shared
  // launch, the entry's index does not depend on the counts, and it is read
  // together with them (the table has room for every workgroup of the grid).
  MoeChunk ch;
  bool shared_chunk;
  int gate_pair = 0;  // GATE: the pair id of this workgroup's chunk
  if constexpr (GATE) {
    static_assert(PIPE == kPipeDecode && MT == 1, "the gate runs with the single-token pipeline");
    // x index 0: the shared expert (when the launch carries it), which does
    // not wait for the gate; then the token's valid ranks in rank order.
    // Wave 0 selects and gates the token; the workgroup of the first rank's
    // row tile 0 also stores the gate's outputs and the chunk table, which
    // the later launches read.
    __shared__ int gate_lds[2 * kMoeMaxTopK + 1];
    const int has_sh = args.joint;
    if (has_sh && bx == 0) {
      ch = MoeChunk{0, args.top_k, 1};
      shared_chunk = true;
      gate_pair = args.top_k;
    } else {
      const int pos = bx - has_sh;
      if (threadIdx.x < 64) {
        const bool write = pos == 0 && by == 0;
        // the selection's scratch: the start of the dynamic LDS, whose
        // stages and sums are first written after the barrier below
        static_assert(Sh::RED >= kSelectScratch * (int)sizeof(int64_t), "selection scratch");
        int64_t* sel = reinterpret_cast<int64_t*>(lds);
        GateRank r{};
        switch (args.gate_jpl) {
          case 1: r = gate_token<1>(args.plan, 0, 1, write, sel); break;
          case 2: r = gate_token<2>(args.plan, 0, 1, write, sel); break;
          case 4: r = gate_token<4>(args.plan, 0, 1, write, sel); break;
          case 8: r = gate_token<8>(args.plan, 0, 1, write, sel); break;
          default: r = gate_token<16>(args.plan, 0, 1, write, sel); break;
        }
        const int l = threadIdx.x;
        const uint64_t mask = __ballot(r.valid);
        if (r.valid) {
          const int pp = __popcll(mask & ((1ull << l) - 1ull));
          gate_lds[pp] = r.idx;
          gate_lds[kMoeMaxTopK + pp] = l;
        }
        if (l == 0) gate_lds[2 * kMoeMaxTopK] = __popcll(mask);
        if (write) gate_chunk_table(args.plan, r.valid, r.idx);
      }
      __syncthreads();
      if (pos >= gate_lds[2 * kMoeMaxTopK]) return;
      ch = MoeChunk{gate_lds[pos], pos, 1};
      gate_pair = gate_lds[kMoeMaxTopK + pos];
      shared_chunk = false;
    }
  } else {
    ch = args.chunks[(!args.joint && args.group ? cc[0] : 0) + bx];
    const int all_chunks = cc[0] + cc[1];
    const int nchunks = args.joint ? all_chunks : cc[args.group];
    if (bx >= nchunks) return;
    shared_chunk = args.joint && bx >= cc[0];
  }
  MoeGemmArgs a = args;
  if (shared_chunk) {
    a.w0 = args.s_w0;
    a.w1 = args.s_w1;
    a.row_bytes = args.s_row_bytes;
    a.expert_stride = 0;
    a.N = args.s_N;
    a.K = args.s_K;
  }
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;

  // first rows of this wave (the double pipeline's workgroups take
  // tiles_per_wg consecutive row tiles of the chunk, one after the other)
  const int n0 = PIPE == kPipeDecode ? by * Sh::ROWS
                                     : by * a.tiles_per_wg * Sh::WG_ROWS + wave * Sh::ROWS;
  // shared activations: every wave of the workgroup takes part in their
  // loads and barriers, also one whose rows lie past the last
  constexpr bool SHARE_A = gemm_share_a<TYPE, EPI, PIPE>();
  constexpr bool JIT_A = gemm_jit_a<TYPE, EPI, PIPE>();
  if (SHARE_A ? n0 - wave * Sh::ROWS >= a.N : n0 >= a.N) return;  // uniform (decode, SHARE_A)
  const int depth = PIPE == kPipeDecode ? a.depth : SHARE_A || JIT_A ? 1 : Sh::DEPTH;
  uint8_t* wlds = lds + Sh::RED + wave * (depth * Sh::STAGE + Sh::TABLE);
  using TableEntry = std::conditional_t<B::kCd != 0.f, float, float2>;
  TableEntry* table = reinterpret_cast<TableEntry*>(wlds + depth * Sh::STAGE);
  const uint32_t wlds_addr = lds_address(wlds);

  // split rows of this lane's tokens (tile row t = n of each token tile)
  const uint16_t* arow[MT];
  const float* srow[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int tk = 16 * i + n;
    const int q = GATE ? gate_pair : a.perm[ch.start + (tk < ch.count ? tk : 0)];
    const int64_t r = a.a_by_token ? (q < a.pairs ? q / a.top_k : q - a.pairs) : q;
    arow[i] = a.aq + r * a.aq_stride;
    srow[i] = a.as + r * a.as_stride;
  }
  // the pairs whose outputs this lane writes (tokens 16 i + 4 g + r of each
  // tile), read now rather than after the products
  int qout[MT][4];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tk = 16 * i + 4 * g + r;
      qout[i][r] = tk < ch.count ? (GATE ? gate_pair : a.perm[ch.start + tk]) : 0;
    }
  const uint8_t* base[NB];
  base[0] = uniform_ptr(a.w0 + (int64_t)ch.expert * a.expert_stride);
  if constexpr (NB == 2) base[NB - 1] = uniform_ptr(a.w1 + (int64_t)ch.expert * a.expert_stride);
  const uint32_t rb = (uint32_t)a.row_bytes;

  // byte offsets of this lane's rows (their chunks' shift when rows are not
  // dword multiples)
  uint32_t brow[NS];
  auto set_rows = [&](int n0t) {
#pragma unroll
    for (int m = 0; m < NS; ++m) brow[m] = (uint32_t)min(n0t + 16 * m + n, a.N - 1) * rb;
  };
  set_rows(n0);

  const int groups = a.K / B::kStepK;
  const int nchunk = (a.K + 255) >> 8;
  const int last_tile = (a.N - 1) >> 4;  // tile-major: the slab's last 16-row tile

  // Issue chunk kc's loads into stage `slot`: the rows; for the decode
  // pipeline also the token's 256 split elements (1 KB) and 16 group sums.
  // Lane l of load instruction i carries piece 64 i + l of the stage: row
  // r = piece / PPR, its 16-byte piece p = piece % PPR (the pad piece p =
  // PPR - 1 repeats the last one).  Tile-major weights: the stage's rows of
  // one 16-row tile are one contiguous run (row r at r * kTilePitch); a
  // tile past the slab's last re-reads that one, whose outputs are dropped.
  // The offsets are formed anew at every issue (the empty asm keeps the
  // compiler from holding them in registers across the products, where the
  // wide pipeline has none to spare).
  auto issue = [&](int kc, int slot, int n0t) {
    const uint32_t koff = (uint32_t)kc * (uint32_t)B::kSpan;
    const uint32_t st = wlds_addr + (uint32_t)(slot * Sh::STAGE);
    int lane_v = lane;
    asm volatile("" : "+v"(lane_v));
#pragma unroll
    for (int i = 0; i < Sh::LOADS; ++i) {
      const int idx = min(64 * i + lane_v, Sh::PIECES - 1);
      const int r = idx / Sh::PPR;
      const uint32_t piece = 16u * (uint32_t)min(idx - r * Sh::PPR, B::kPieces - 1);
      uint32_t off;
      if constexpr (TILED) {
        const uint32_t tile = (uint32_t)min((n0t + r) >> 4, last_tile);
        off = ((tile * (uint32_t)nchunk + (uint32_t)kc) * 16u + (uint32_t)(r & 15)) *
                  (uint32_t)B::kTilePitch + piece;
      } else {
        off = (((uint32_t)min(n0t + r, a.N - 1) * rb + koff) & ~3u) + piece;
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        load_lds16(base[nb], off, st + (uint32_t)(nb * Sh::MATBUF + 1024 * i));
    }
    if constexpr (PIPE == kPipeDecode) {
      // lane l: 16 bytes [16 l, 16 l + 16) of the token's chunk; the sums
      // (16 floats; lanes past them re-read the last one into slack)
      const uint8_t* abase = uniform_ptr(reinterpret_cast<const uint8_t*>(arow[0] + 512 * kc));
      load_lds16(abase, 16u * (uint32_t)lane, st + Sh::A_OFF);
      const uint8_t* sbase = uniform_ptr(reinterpret_cast<const uint8_t*>(srow[0] + 16 * kc));
      const int smax = min(16, (a.K >> 4) - 16 * kc) - 1;
      load_lds4(sbase, 4u * (uint32_t)min(lane, smax), st + Sh::S_OFF);
    }
  };

  floatx4 tot[MT][NS][NB];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int m = 0; m < NS; ++m)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) tot[i][m][nb] = floatx4{0.f, 0.f, 0.f, 0.f};

  // ---- one chunk: scale table, then groups, then offsets
  // get_a(i, j, af) fills tile i's fragments of group j; get_s(i, q)
  // returns the sum of the group (4q + g) of tile i's lane token.
  // FULL: all KS groups of the chunk lie inside K (always for Q4_K and Q6_K,
  // whose K is a multiple of 256); only the last chunk of a Q5_0 / Q8_0 row
  // may be partial.
  auto compute = [&](auto full, int kc, const uint8_t* stage, auto get_a, auto get_s) {
    constexpr bool FULL = decltype(full)::value;
    const uint32_t koff = (uint32_t)kc * (uint32_t)B::kSpan;
    const int valid = FULL ? KS : min(KS, groups - kc * KS);
    uint32_t sh[NS];
#pragma unroll
    for (int m = 0; m < NS; ++m)
      sh[m] = TILED ? 0u : ALIGNED ? (koff & 3u) : ((brow[m] + koff) & 3u);
    // scale table: lane (n, g) decodes groups g, g + 4, ... of row n (the
    // four lane groups' entries then sit in different banks)
#pragma unroll
    for (int m = 0; m < NS; ++m)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const uint8_t* row = stage + nb * Sh::MATBUF + (16 * m + n) * B::kPitch;
#pragma unroll
        for (int e = 0; e < KS / 4; ++e) {
          const int j = g + 4 * e;
          float delta, c;
          B::scale(row, sh[m], j, delta, c);
          const bool ok = j < valid;
          if constexpr (B::kCd != 0.f) table[((m * NB + nb) * KS + j) * 16 + n] = ok ? delta : 0.f;
          else table[((m * NB + nb) * KS + j) * 16 + n] = float2{ok ? delta : 0.f, ok ? -c : 0.f};
        }
      }
    // Software pipeline over the groups: the LDS words (codes and delta) of
    // group j + 1 and, in the wide pipeline, whose activations come from
    // memory, those of group j + 2 are requested before group j decodes and
    // multiplies, so that neither latency stalls the group's MFMAs.
    constexpr int kAhead = PIPE == kPipeWide || JIT_A ? 2 : SHARE_A ? 1 : 0;
    typename B::Raw raw[2][NS][NB];
    float dl[2][NS][NB];
    AF af[kAhead + 1][MT];
    auto fetch = [&](int j, typename B::Raw (&r)[NS][NB], float (&d)[NS][NB]) {
#pragma unroll
      for (int m = 0; m < NS; ++m)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const uint8_t* row = stage + nb * Sh::MATBUF + (16 * m + n) * B::kPitch;
          r[m][nb] = B::fetch(row, sh[m], j, g);
          if constexpr (B::kCd != 0.f) d[m][nb] = table[((m * NB + nb) * KS + j) * 16 + n];
          else d[m][nb] = table[((m * NB + nb) * KS + j) * 16 + n].x;
        }
    };
#pragma unroll
    for (int j = 0; j < kAhead; ++j)
      if (FULL || j < valid)
#pragma unroll
        for (int i = 0; i < MT; ++i) get_a(i, j, af[j][i]);
    fetch(0, raw[0], dl[0]);
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      if (FULL || j < valid) {
        if (j + kAhead < KS && (FULL || j + kAhead < valid))
#pragma unroll
          for (int i = 0; i < MT; ++i) get_a(i, j + kAhead, af[(j + kAhead) % (kAhead + 1)][i]);
        if (j + 1 < KS && (FULL || j + 1 < valid)) fetch(j + 1, raw[(j + 1) & 1], dl[(j + 1) & 1]);
#pragma unroll
        for (int m = 0; m < NS; ++m)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            const typename B::Frag bf = B::decode(raw[j & 1][m][nb], sh[m], j, g);
            const float delta = dl[j & 1][m][nb];
#pragma unroll
            for (int i = 0; i < MT; ++i) {
              const AF& a_ = af[j % (kAhead + 1)][i];
              floatx4& t = tot[i][m][nb];
              if constexpr (PIPE == kPipeDecode) {
                // one token, hi and lo in alternate rows (load_pair): its
                // sums are rows 0 and 1, lane group 0 elements 0 and 1
                const floatx4 d = mfma_b(a_.hi, bf, floatx4{0.f, 0.f, 0.f, 0.f});
                t[0] = fmaf(delta, d[0] + d[1], t[0]);
              } else {
                floatx4 d = mfma_b(a_.hi, bf, floatx4{0.f, 0.f, 0.f, 0.f});
                d = mfma_b(a_.lo, bf, d);
                t[0] = fmaf(delta, d[0], t[0]);
                t[1] = fmaf(delta, d[1], t[1]);
                t[2] = fmaf(delta, d[2], t[2]);
                t[3] = fmaf(delta, d[3], t[3]);
              }
            }
          }
      }
    }
    // offsets: group 4q + g of the chunk in K slice g of MFMA q
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      float cb[NS][NB];
#pragma unroll
      for (int m = 0; m < NS; ++m)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          // -c as the table held it: -(kCd * delta), 0 for a group past K
          if constexpr (B::kCd != 0.f)
            cb[m][nb] = 4 * q + g < valid ? -(B::kCd * table[((m * NB + nb) * KS + 4 * q + g) * 16 + n])
                                          : 0.f;
          else cb[m][nb] = table[((m * NB + nb) * KS + 4 * q + g) * 16 + n].y;
        }
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const float sv = get_s(i, q);
#pragma unroll
        for (int m = 0; m < NS; ++m)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) tot[i][m][nb] = mfma4f32(sv, cb[m][nb], tot[i][m][nb]);
      }
    }
  };

  auto run_chunk = [&](int kc, const uint8_t* stage, auto get_a, auto get_s) {
    if (kc * KS + KS <= groups) compute(std::true_type{}, kc, stage, get_a, get_s);
    else compute(std::false_type{}, kc, stage, get_a, get_s);
  };

  // group sum of element group gi of a split row (16-groups; a 32-group is
  // the sum of its two halves)
  auto row_sum = [&](const float* s, int gi) -> float {
    if constexpr (B::kStepK == 32) return s[2 * gi] + s[2 * gi + 1];
    else return s[gi];
  };

  // activations and group sums of chunk kc of the lane's token into registers
  auto load_regs = [&](int kc, AF (&ar)[KS], float (&sr)[NQ]) {
    const int valid = min(KS, groups - kc * KS);
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      if (j < valid) ar[j].load(arow[0] + 512 * kc + AF::offset(j, g));
      else ar[j].zero();
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) sr[q] = row_sum(srow[0], min(kc * KS + 4 * q + g, groups - 1));
  };

  // ---------------------------------------------------------- epilogue
  // lane (n, G) holds tokens 16 i + 4 G + r of rows n0t + 16 m + n
  auto finish = [&](int n0t) {
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tk = 16 * i + 4 * g + r;
        const bool ok_t = tk < ch.count;
        const int q = qout[i][r];
        if constexpr (EPI == kEpiDown) {
#pragma unroll
          for (int m = 0; m < NS; ++m) {
            const int row = n0t + 16 * m + n;
            if (ok_t && row < a.N) a.out[(int64_t)q * a.out_stride + row] = tot[i][m][0][r];
          }
        } else {
          uint16_t* oq = a.oq + (int64_t)q * a.oq_stride;
          float* os = a.os + (int64_t)q * a.os_stride;
#pragma unroll
          for (int m = 0; m < NS; ++m) {
            const int row = n0t + 16 * m + n;
            float act;
            if constexpr (EPI == kEpiSwiglu) {
#pragma clang fp contract(off)
              act = silu_ref(tot[i][m][0][r]) * tot[i][m][1][r];  // llambda.lisp:5386-5401
            } else {
              act = relu2_ref(tot[i][m][0][r]);  // llambda.lisp:5921-5926
            }
            uint32_t hb, lb;
            float sum;
            split_bf16(act, hb, lb, sum);
            const bool ok = ok_t && row < a.N;
            if (ok) {
              uint16_t* p = oq + 64 * (row >> 5) + (row & 31);
              p[0] = (uint16_t)hb;
              p[32] = (uint16_t)lb;
            }
            // the 16 rows of the subtile are one 16-group of the activation row
            const float s16 = group_sum(ok ? sum : 0.f, 4);
            if (n == 0 && ok) os[row >> 4] = s16;
          }
        }
      }
    }
  };

  if constexpr (PIPE == kPipeWide || JIT_A) {
    for (int kc = 0; kc < nchunk; ++kc) {
      const int gbase = kc * KS;
      // The chunk's group sums and its first group's activations are
      // requested with its rows, under the one wait; the later groups'
      // activations load two groups ahead of use (two groups here would not
      // fit the registers).  Lanes of padding tokens read the chunk's first
      // token (their outputs are dropped).
      AF a_first[1][MT];
      float sv[MT][NQ];
#pragma unroll
      for (int j = 0; j < 1; ++j)
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          if (gbase + j < groups) a_first[j][i].load(arow[i] + 512 * kc + AF::offset(j, g));
          else a_first[j][i].zero();
        }
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int q = 0; q < NQ; ++q) sv[i][q] = row_sum(srow[i], min(gbase + 4 * q + g, groups - 1));
      issue(kc, 0, n0);
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
      run_chunk(
          kc, wlds,
          [&](int i, int j, AF& af) {
            if (j < 1) af = a_first[j][i];
            else af.load(arow[i] + 512 * kc + AF::offset(j, g));
          },
          [&](int i, int q) { return sv[i][q]; });
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    }
  } else if constexpr (PIPE == kPipeDouble && SHARE_A) {
    // As below, with the chunk's activations in LDS: wave w loads tokens
    // 4w .. 4w+3 (lane l: token 4w + (l >> 4), 16-byte pieces (l & 15) +
    // 16 k, k < 4, of its 1 KB) into registers while the step computes, and
    // stores them once every wave is done with the step's; piece P of token t
    // sits in slot P ^ t of the token's 1 KB, so a fragment's 16 tokens read
    // 16 different bank quads, and the 16 lanes of a store write 16.  The steps and barriers are the workgroup's: a
    // wave without rows in a tile loads its quarter and waits with the rest.
    const int n0w = n0 - wave * Sh::ROWS;
    const int ntile = min(a.tiles_per_wg, (a.N - n0w + Sh::WG_ROWS - 1) / Sh::WG_ROWS);
    const int steps = ntile * nchunk;
    uint8_t* alds = lds + Sh::RED + Sh::kWaves * (Sh::STAGE + Sh::TABLE);
    const int qt = 4 * wave + (lane >> 4);
    const uint64_t ap = reinterpret_cast<uint64_t>(arow[0]);  // lane qt holds token qt's row
    const uint32_t ap_lo = (uint32_t)__shfl((int)(uint32_t)ap, qt);
    const uint32_t ap_hi = (uint32_t)__shfl((int)(uint32_t)(ap >> 32), qt);
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(((uint64_t)ap_hi << 32) | ap_lo);
    u32x4 qa[4];
    auto load_quarter = [&](int kc) {
      const int valid = min(KS, groups - kc * KS);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int piece = (lane & 15) + 16 * k;  // group piece >> 3
        qa[k] = (piece >> 3) < valid
                    ? *reinterpret_cast<const u32x4*>(qrow + 512 * kc + 8 * piece)
                    : u32x4{0u, 0u, 0u, 0u};
      }
    };
    auto store_quarter = [&]() {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int piece = (lane & 15) + 16 * k;
        *reinterpret_cast<u32x4*>(alds + qt * 1024 + 16 * (piece ^ qt)) = qa[k];
      }
    };
    auto load_sums = [&](int kc, float (&sr)[NQ]) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) sr[q] = row_sum(srow[0], min(kc * KS + 4 * q + g, groups - 1));
    };
    auto get_a_lds = [&](int, int j, AF& af) {
      af.hi = *reinterpret_cast<const bf16x8*>(alds + n * 1024 + 16 * ((8 * j + g) ^ n));
      af.lo = *reinterpret_cast<const bf16x8*>(alds + n * 1024 + 16 * ((8 * j + 4 + g) ^ n));
    };
    float scur[NQ], snext[NQ];
    if (n0 < a.N) issue(0, 0, n0);
    load_quarter(0);
    load_sums(0, scur);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    store_quarter();
    __syncthreads();
    for (int st = 0, tt = 0, kc = 0; st < steps; ++st) {
      const bool more = st + 1 < steps;
      const int kc1 = kc + 1 < nchunk ? kc + 1 : 0;
      const int tt1 = kc + 1 < nchunk ? tt : tt + 1;
      const bool live = n0 + tt * Sh::WG_ROWS < a.N;
      if (more) {
        load_quarter(kc1);
        load_sums(kc1, snext);
      }
      if (live)
        run_chunk(kc, wlds, get_a_lds, [&](int, int q) { return scur[q]; });
      // one row stage per wave: the next step's rows load once this step's
      // products have read them (the other workgroups' waves cover the wait)
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      if (more && n0 + tt1 * Sh::WG_ROWS < a.N) issue(kc1, 0, n0 + tt1 * Sh::WG_ROWS);
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
      if (kc + 1 == nchunk) {
        if (live) finish(n0 + tt * Sh::WG_ROWS);
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int m = 0; m < NS; ++m)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) tot[i][m][nb] = floatx4{0.f, 0.f, 0.f, 0.f};
        if (more && !ALIGNED) set_rows(n0 + tt1 * Sh::WG_ROWS);
      }
      __syncthreads();  // every wave is done with this chunk's activations
      if (more) {
        store_quarter();
#pragma unroll
        for (int q = 0; q < NQ; ++q) scur[q] = snext[q];
      }
      __syncthreads();  // the next chunk's activations are in place
      kc = kc1;
      tt = tt1;
    }
  } else if constexpr (PIPE == kPipeDouble) {
    // Steps (tile, chunk) over the workgroup's row tiles that hold rows of
    // this wave, tile by tile; the rows (by DMA) and the activations and
    // sums (into registers) of the next step load while a step computes, so
    // the chain of dependent loads before the first step is paid once for
    // tiles_per_wg tiles.
    const int ntile = min(a.tiles_per_wg, (a.N - n0 + Sh::WG_ROWS - 1) / Sh::WG_ROWS);
    const int steps = ntile * nchunk;
    AF acur[KS], anext[KS];
    float scur[NQ], snext[NQ];
    issue(0, 0, n0);
    load_regs(0, acur, scur);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    for (int st = 0, tt = 0, kc = 0; st < steps; ++st) {
      const bool more = st + 1 < steps;
      const int kc1 = kc + 1 < nchunk ? kc + 1 : 0;
      const int tt1 = kc + 1 < nchunk ? tt : tt + 1;
      if (more) {
        issue(kc1, (st + 1) & 1, n0 + tt1 * Sh::WG_ROWS);
        load_regs(kc1, anext, snext);
      }
      run_chunk(
          kc, wlds + (st & 1) * Sh::STAGE, [&](int, int j, AF& af) { af = acur[j]; },
          [&](int, int q) { return scur[q]; });
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      if (kc + 1 == nchunk) {
        finish(n0 + tt * Sh::WG_ROWS);
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int m = 0; m < NS; ++m)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) tot[i][m][nb] = floatx4{0.f, 0.f, 0.f, 0.f};
        if (more && !ALIGNED) set_rows(n0 + tt1 * Sh::WG_ROWS);
      }
      if (more) {
#pragma unroll
        for (int j = 0; j < KS; ++j) acur[j] = anext[j];
#pragma unroll
        for (int q = 0; q < NQ; ++q) scur[q] = snext[q];
      }
      kc = kc1;
      tt = tt1;
    }
  } else {
    // decode: one token; wave w takes chunks w, w + 4, ... through a ring of
    // `depth` stages filled ahead of use
    const int mine = (nchunk - wave + Sh::kWaves - 1) / Sh::kWaves;
    const int first = min(depth, mine);
    for (int s = 0; s < first; ++s) issue(wave + Sh::kWaves * s, s, n0);
    for (int it = 0; it < mine; ++it) {
      const int kc = wave + Sh::kWaves * it;
      const int ahead = min(mine, it + depth) - it - 1;  // stages issued after this one
      // at most `ahead` stages (DMA loads each) may still be in flight; the
      // counter holds 63, beyond which the wait is stricter than needed
      switch (ahead) {
        case 0: __builtin_amdgcn_s_waitcnt(waitcnt_vm(0)); break;
        case 1: __builtin_amdgcn_s_waitcnt(waitcnt_vm(std::min(63, 1 * Sh::DMA))); break;
        case 2: __builtin_amdgcn_s_waitcnt(waitcnt_vm(std::min(63, 2 * Sh::DMA))); break;
        case 3: __builtin_amdgcn_s_waitcnt(waitcnt_vm(std::min(63, 3 * Sh::DMA))); break;
        case 4: __builtin_amdgcn_s_waitcnt(waitcnt_vm(std::min(63, 4 * Sh::DMA))); break;
        case 5: __builtin_amdgcn_s_waitcnt(waitcnt_vm(std::min(63, 5 * Sh::DMA))); break;
        case 6: __builtin_amdgcn_s_waitcnt(waitcnt_vm(std::min(63, 6 * Sh::DMA))); break;
        default: __builtin_amdgcn_s_waitcnt(waitcnt_vm(std::min(63, 7 * Sh::DMA))); break;
      }
      const int slot = it % depth;
      const uint8_t* stage = wlds + slot * Sh::STAGE;
      const float* ssum = reinterpret_cast<const float*>(stage + Sh::S_OFF);
      // every tile row reads the one token (rows t > 0 are dropped)
      run_chunk(
          kc, stage,
          [&](int, int j, AF& af) {
            af.load_pair(reinterpret_cast<const uint16_t*>(stage + Sh::A_OFF) + AF::offset(j, g), n);
          },
          [&](int, int q) {
            const int gi = min(kc * KS + 4 * q + g, groups - 1) - kc * KS;
            if constexpr (B::kStepK == 32) return ssum[2 * gi] + ssum[2 * gi + 1];
            else return ssum[gi];
          });
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      if (it + depth < mine) issue(kc + Sh::kWaves * depth, slot, n0);
    }
    // partial sums of the four K slices, added in wave order by wave 0
    floatx4* red = reinterpret_cast<floatx4*>(lds);
#pragma unroll
    for (int m = 0; m < NS; ++m)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) red[((wave * NS + m) * NB + nb) * 64 + lane] = tot[0][m][nb];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int m = 0; m < NS; ++m)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        floatx4 v = red[(m * NB + nb) * 64 + lane];
#pragma unroll
        for (int w = 1; w < Sh::kWaves; ++w) v = v + red[((w * NS + m) * NB + nb) * 64 + lane];
        tot[0][m][nb] = v;
      }
  }

  if constexpr (PIPE != kPipeDouble || JIT_A) finish(n0);
}

// ------------------------------------------------ one token: down + combine
// The down products of one token's chunks (its valid ranks' experts in rank
// order, then the shared expert) and their weighted combine, in one launch.
// Workgroup r takes rows 16 r .. 16 r + 15 of every chunk.  The work units
// are the chunks' 256-element K steps (chunk by chunk, steps in order); wave
// w of 16 takes units w, w + 16, ..., streaming each unit's rows by DMA with
// the pair's 256 split activations and their 16 group sums through a ring of
// LDS stages filled ahead of use.  A unit leaves the partial sums of its 16
// rows in LDS; after one barrier lanes 0..15 of wave 0 add each chunk's
// partials in K order (the single-token pipeline's split-K sum) and combine
// the chunks as moe_combine_kernel does: rank order, every product and sum
// rounded separately (llambda.lisp:3465-3489; 5359, 5409, 5426, 5914, 5932,
// 5949).  At batch 1 the chunk table has chunk c = {expert, start c, one
// pair} and perm[c] = its rank (the shared chunk: perm[c] = top_k), as
// topk_gate_kernel writes them.
constexpr int kCombineSlots = 64;   // chunks of one token: top_k + 1 (read back by readlane)
constexpr int kCombineUnits = 128;  // (chunk, K step) units of one token

template <int TYPE>
struct CombineShape {
  using B = GemmB<TYPE>;
  // sixteen waves: a unit's decode and products are a chain of dependent
  // VALU work, so four waves per SIMD cover each other's latencies where two
  // did not (Qwen3Next B=1 25.3 -> 23.0 us; the ring is one stage deep then)
  static constexpr int kWaves = 16;
  static constexpr int PPR = B::kPitch / 16;       // 16-byte pieces per row
  static constexpr int PIECES = 16 * PPR;          // 16 rows
  static constexpr int LOADS = (PIECES + 63) / 64;
  static constexpr int ROWBUF = 1024 * LOADS;
  static constexpr int A_OFF = ROWBUF;             // the pair's 256 split elements (1 KB)
  static constexpr int S_OFF = ROWBUF + 1024;      // their 16 group sums
  static constexpr int STAGE = ROWBUF + 1024 + 256;
  static constexpr int DEPTH = 4;
  static constexpr int DMA = LOADS + 2;            // loads per stage
  static constexpr int TABLE = B::kSteps * 16 * 8;  // (delta, -c) per group and row
  static constexpr int OUT = kCombineUnits * 16 * 4;
};

template <int TYPE>
constexpr int combine_lds_bytes(int depth) {
  using Sh = CombineShape<TYPE>;
  return Sh::OUT + Sh::kWaves * (depth * Sh::STAGE + Sh::TABLE);
}

// One 256-element K step of a wave's 16 rows for the one token: the body of
// moe_gemm_kernel's per-chunk computation with one subtile, one matrix and
// one token tile (scale table, groups with the next group's LDS words
// fetched ahead, then the chunk's offsets).
template <int TYPE, bool ALIGNED, bool FULL>
__device__ __forceinline__ void combine_step(int kc, const uint8_t* stage, uint32_t brow,
                                             int groups, float2* table, int n, int g,
                                             floatx4& tot) {
  using B = GemmB<TYPE>;
  using Sh = CombineShape<TYPE>;
  constexpr int NQ = B::kSteps / 4, KS = B::kSteps;
  typedef AFrag<B::kWide> AF;
  const uint32_t koff = (uint32_t)kc * (uint32_t)B::kSpan;
  const int valid = FULL ? KS : min(KS, groups - kc * KS);
  const uint32_t sh = B::kTilePitch ? 0u : ALIGNED ? (koff & 3u) : ((brow + koff) & 3u);
  const uint8_t* row = stage + n * B::kPitch;
  // scale table: lane (n, g) decodes groups g, g + 4, ... of row n (the four
  // lane groups' entries then sit in different banks)
#pragma unroll
  for (int e = 0; e < KS / 4; ++e) {
    const int j = g + 4 * e;
    float delta, c;
    B::scale(row, sh, j, delta, c);
    const bool ok = j < valid;
    table[j * 16 + n] = float2{ok ? delta : 0.f, ok ? -c : 0.f};
  }
  typename B::Raw raw[2];
  float dl[2];
  auto fetch = [&](int j, typename B::Raw& r, float& d) {
    r = B::fetch(row, sh, j, g);
    d = table[j * 16 + n].x;
  };
  fetch(0, raw[0], dl[0]);
#pragma unroll
  for (int j = 0; j < KS; ++j) {
    if (FULL || j < valid) {
      AF af;
      af.load_pair(reinterpret_cast<const uint16_t*>(stage + Sh::A_OFF) + AF::offset(j, g), n);
      if (j + 1 < KS && (FULL || j + 1 < valid)) fetch(j + 1, raw[(j + 1) & 1], dl[(j + 1) & 1]);
      const typename B::Frag bf = B::decode(raw[j & 1], sh, j, g);
      const float delta = dl[j & 1];
      // hi and lo in alternate A rows: the token's two sums are rows 0 and 1
      const floatx4 d = mfma_b(af.hi, bf, floatx4{0.f, 0.f, 0.f, 0.f});
      tot[0] = fmaf(delta, d[0] + d[1], tot[0]);
    }
  }
  // offsets: group 4q + g of the chunk in K slice g of MFMA q
  const float* ssum = reinterpret_cast<const float*>(stage + Sh::S_OFF);
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const float cb = table[(4 * q + g) * 16 + n].y;
    const int gi = min(kc * KS + 4 * q + g, groups - 1) - kc * KS;
    float sv;
    if constexpr (B::kStepK == 32) sv = ssum[2 * gi] + ssum[2 * gi + 1];
    else sv = ssum[gi];
    tot = mfma4f32(sv, cb, tot);
  }
}

template <int TYPE, bool ALIGNED>
__global__ void __launch_bounds__(64 * CombineShape<TYPE>::kWaves)
moe_down_combine_kernel(MoeGemmArgs a, MoeCombineArgs cb) {
  using B = GemmB<TYPE>;
  using Sh = CombineShape<TYPE>;
  constexpr int KS = B::kSteps, W = Sh::kWaves;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int K = a.top_k;
  float* parts = reinterpret_cast<float*>(lds);  // [kCombineUnits][16]
  const int depth = a.depth;
  uint8_t* wlds = lds + Sh::OUT + wave * (depth * Sh::STAGE + Sh::TABLE);
  float2* table = reinterpret_cast<float2*>(wlds + depth * Sh::STAGE);
  const uint32_t wlds_addr = lds_address(wlds);

  // lane i: the entry and the pair of chunk i, read with the counts (chunk
  // c's pair is perm[c] at batch 1), and its K, K steps and row bytes, read
  // back by readlane
  const int ci = min(lane, K);
  const int ex = a.chunks[ci].expert;
  const int pq = a.perm[ci];
  // wave 0: the gating weight of routed chunk `lane` (its rank perm[lane];
  // lanes past the token's chunks read a clamped, unused entry)
  float wl = 0.f;
  if (wave == 0) wl = cb.top_w[max(0, min(a.perm[ci], K - 1))];
  const float shw = cb.shared_scaled ? cb.shared_w[0] : 0.f;
  const int nv = a.chunk_counts[0], ns = a.chunk_counts[1];
  const bool lane_shared = lane >= nv;
  const int kv = lane_shared ? a.s_K : a.K;
  const int rbv = (int)(lane_shared ? a.s_row_bytes : a.row_bytes);
  const int nk_r = (a.K + 255) >> 8, nk_s = ns ? (a.s_K + 255) >> 8 : 0;
  const int routed_units = nv * nk_r;
  const int units = routed_units + nk_s;
  const int mine = units > wave ? (units - wave + W - 1) / W : 0;  // units of this wave
  // unit u: chunk u / nk_r, step u % nk_r (routed), or the shared chunk nv
  auto chunk_of = [=](int u) { return u < routed_units ? u / nk_r : nv; };
  auto step_of = [=](int u) { return u < routed_units ? u - (u / nk_r) * nk_r : u - routed_units; };

  auto issue = [&](int i, int slot) __attribute__((always_inline)) {
    const int u = wave + W * i;
    const int c = chunk_of(u), kc = step_of(u);
    const int e = __builtin_amdgcn_readlane(ex, c);
    const int q = __builtin_amdgcn_readlane(pq, c);
    const uint8_t* base =
        uniform_ptr(c >= nv ? a.s_w0 : a.w0 + (int64_t)e * a.expert_stride);
    const uint32_t rb = (uint32_t)__builtin_amdgcn_readlane(rbv, c);
    const int Kc = __builtin_amdgcn_readlane(kv, c);
    const uint32_t koff = (uint32_t)kc * (uint32_t)B::kSpan;
    const uint32_t st = wlds_addr + (uint32_t)(slot * Sh::STAGE);
    // tile-major weights: this workgroup's tile of chunk kc, one run
    const uint32_t run = ((uint32_t)blockIdx.x * (uint32_t)((Kc + 255) >> 8) + (uint32_t)kc) *
                         16u * (uint32_t)B::kTilePitch;
#pragma unroll
    for (int l = 0; l < Sh::LOADS; ++l) {
      const int idx = min(64 * l + lane, Sh::PIECES - 1);
      const int r = idx / Sh::PPR;
      const uint32_t piece = 16u * (uint32_t)min(idx - r * Sh::PPR, B::kPieces - 1);
      const uint32_t off =
          B::kTilePitch ? run + (uint32_t)r * (uint32_t)B::kTilePitch + piece
                        : (((uint32_t)min(n0 + r, a.N - 1) * rb + koff) & ~3u) + piece;
      load_lds16(base, off, st + (uint32_t)(1024 * l));
    }
    const uint8_t* abase = uniform_ptr(
        reinterpret_cast<const uint8_t*>(a.aq + (int64_t)q * a.aq_stride + 512 * kc));
    load_lds16(abase, 16u * (uint32_t)lane, st + Sh::A_OFF);
    const uint8_t* sbase =
        uniform_ptr(reinterpret_cast<const uint8_t*>(a.as + (int64_t)q * a.as_stride + 16 * kc));
    const int smax = min(16, (Kc >> 4) - 16 * kc) - 1;
    load_lds4(sbase, 4u * (uint32_t)min(lane, smax), st + Sh::S_OFF);
  };

  const int first = min(depth, mine);
  for (int i = 0; i < first; ++i) issue(i, i);
  for (int i = 0; i < mine; ++i) {
    const int ahead = min(mine, i + depth) - i - 1;  // stages issued after this one
    switch (ahead) {
      case 0: __builtin_amdgcn_s_waitcnt(waitcnt_vm(0)); break;
      case 1: __builtin_amdgcn_s_waitcnt(waitcnt_vm(std::min(63, 1 * Sh::DMA))); break;
      case 2: __builtin_amdgcn_s_waitcnt(waitcnt_vm(std::min(63, 2 * Sh::DMA))); break;
      default: __builtin_amdgcn_s_waitcnt(waitcnt_vm(std::min(63, 3 * Sh::DMA))); break;
    }
    const int slot = i % depth;
    const uint8_t* stage = wlds + slot * Sh::STAGE;
    const int u = wave + W * i;
    const int c = chunk_of(u), kc = step_of(u);
    const int groups = __builtin_amdgcn_readlane(kv, c) / B::kStepK;
    const uint32_t rb = (uint32_t)__builtin_amdgcn_readlane(rbv, c);
    const uint32_t brow = (uint32_t)min(n0 + n, a.N - 1) * rb;
    floatx4 tot = floatx4{0.f, 0.f, 0.f, 0.f};
    if (kc * KS + KS <= groups)
      combine_step<TYPE, ALIGNED, true>(kc, stage, brow, groups, table, n, g, tot);
    else
      combine_step<TYPE, ALIGNED, false>(kc, stage, brow, groups, table, n, g, tot);
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    if (i + depth < mine) issue(i + depth, slot);
    // lane (n, 0) holds row n0 + n of the unit's one token
    if (g == 0) parts[u * 16 + n] = tot[0];
  }
  __syncthreads();
  if (wave != 0 || g != 0) return;
  {
#pragma clang fp contract(off)
    auto chunk_sum = [&](int u0, int nk) {
      float d = parts[u0 * 16 + n];
      for (int k = 1; k < nk; ++k) d = d + parts[(u0 + k) * 16 + n];
      return d;
    };
    float acc = 0.f;
    for (int c = 0; c < nv; ++c) {
      const float w = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), c));
      const float prod = w * chunk_sum(c * nk_r, nk_r);
      acc = acc + prod;
    }
    if (ns) {
      const float d = chunk_sum(routed_units, nk_s);
      if (cb.shared_scaled) {
        const float prod = shw * d;
        acc = acc + prod;
      } else {
        acc = acc + d;
      }
    }
    if (n0 + n < a.N) cb.y[n0 + n] = acc;
    if (cb.error_out && blockIdx.x == 0 && n == 0) *cb.error_out = *cb.error;
  }
}

// ------------------------------------------------------ group pipeline
// Batches whose experts average more than 16 pairs, with 32-weight block
// types (Q5_0, Q8_0): chunks of up to 64 (token, rank) pairs of one expert,
// four 16-token tiles.  A workgroup of four waves takes 64 rows per wave (32
// of gate and 32 of up for silu-gate products) and streams K in stages of two
// 32-groups through a double-buffered LDS ring, both operands by DMA, with
// every DMA instruction's 64 lanes reading whole 16-byte runs of a few rows
// (one row per lane made each instruction touch 64 cache lines and bound the
// pipeline on the requests):
//   the chunk's split activations, once per workgroup and shared by its
//   waves: instruction k takes tokens 4k .. 4k + 3, a token's 256 bytes of
//   the stage in 16 consecutive lanes, and writes 1 KB block k of the stage
//   with piece P of token t in 16-byte slot 16 (t & 3) + (P ^ (t & 15)), so
//   that the 16 tokens of one MFMA fragment fall in 16 different slots of
//   the 256-byte bank window; the group sums, 16 bytes per token, one lane
//   per token;
//   each wave's weight rows (one matrix): row-major lines of PIECES 16-byte
//   pieces, instruction q taking line slots 64 q .. 64 q + 63 -- a run of
//   whole lines (a line pitch of 48 or 80 bytes puts the 16 rows of a
//   fragment in 16 different banks); the silu-gate pair (two matrices)
//   keeps the piece-major [piece][row][16 bytes] stage, one row per lane.
// One barrier per stage: after it, every wave's DMA of the stage has landed
// and every wave is done with the other buffer, which then takes the next
// stage's DMA while this one computes.  The per-output arithmetic is the
// other batch pipelines' instruction for instruction (exact bf16 codes, hi
// then lo MFMA, per-group delta fma in group order, the -c * sum offsets of
// each 256-element chunk after its eight groups), so a token's output does
// not depend on the pipeline, and hence on the batch, it runs in.
// Q5_0 in the stage-major plane order (moe_repack_launch): a wave's stage
// of 64 rows is 704 dwords -- [64 (4j + g) + (r ^ 16 g)] = lane g's code
// fields of block j of row r (byte b: all five bits of code 8g + b, the low
// three of code 8g + 4 + b above them), [512 + 64 j + r] = block j's word of
// the other bits, [640 + r] = both deltas -- so that the 64 lanes' reads of
// one subtile (rows 16 m + n, lanes g) fall in 64 different banks.  Codes
// and scales equal GemmB<kQ5_0>'s.
__device__ __forceinline__ u32x4 staged_q5_fetch(const uint8_t* run, int r, int j, int g) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(run);
  return u32x4{w[64 * (4 * j + g) + (r ^ (16 * g))], w[512 + 64 * j + r], 0u, 0u};
}
__device__ __forceinline__ bf16x8 staged_q5_decode(const u32x4& w, int g) {
  // the word rotated right by 2g puts bits 3 and 4 of code 8g + 4 + b at
  // bits 8b + 3 and 8b + 4
  const uint32_t r = __builtin_amdgcn_alignbit(w[1], w[1], 2u * (uint32_t)g);
  const uint32_t c0 = w[0] & 0x1F1F1F1Fu;
  const uint32_t c1 = ((w[0] >> 5) & 0x07070707u) | (r & 0x18181818u);
  return codes_to_b(c0, c1);
}
__device__ __forceinline__ uint32_t staged_q5_deltas(const uint8_t* run, int r) {
  return reinterpret_cast<const uint32_t*>(run)[640 + r];
}
__device__ __forceinline__ void staged_q5_scale(const uint8_t* run, int r, int j, float& delta,
                                                float& c) {
  const uint32_t d = staged_q5_deltas(run, r);
  delta = half_bits_to_float(j ? d >> 16 : d & 0xFFFFu);
  c = 144.f * delta;
}
// Q8_0 in the stage-major order: row r holds the codes q + 128 of blocks 0
// and 1 in dwords [0, 16), both deltas in [16].  Codes and scales equal
// GemmB<kQ8_0>'s.
__device__ __forceinline__ u32x4 staged_q8_fetch(const uint8_t* row, int j, int g) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(row);
  return u32x4{w[8 * j + 2 * g], w[8 * j + 2 * g + 1], 0u, 0u};
}
__device__ __forceinline__ bf16x8 staged_q8_decode(const u32x4& w) {
  using B = GemmB<kQ8_0>;
  u32x4 v = {B::pack2(w[0], 0), B::pack2(w[0], 2), B::pack2(w[1], 0), B::pack2(w[1], 2)};
  return __builtin_bit_cast(bf16x8, v);
}
__device__ __forceinline__ void staged_q8_scale(const uint8_t* row, int j, float& delta, float& c) {
  const uint32_t d = reinterpret_cast<const uint32_t*>(row)[16];
  delta = half_bits_to_float(j ? d >> 16 : d & 0xFFFFu);
  c = 128.f * delta;
}

// Row waves per set (64 rows each): a build knob.
#ifndef LLHIP_GROUP_ROW_WAVES
#define LLHIP_GROUP_ROW_WAVES 4
#endif
constexpr int kGroupWaves = LLHIP_GROUP_ROW_WAVES;
constexpr int kGroupTiles = 4;    // 16-token tiles per set
static_assert(kGroupWaves == 4 || kGroupWaves == 8, "row waves: 4 or 8");

template <int TYPE>
struct GroupB;
template <>
struct GroupB<kQ5_0> {
  static constexpr int kBlock = 22, kPieces = 3;  // two blocks + a 0..3-byte shift
};
template <>
struct GroupB<kQ8_0> {
  static constexpr int kBlock = 34, kPieces = 5;
};

// SETS wave sets share the workgroup's weight rows: set s takes token tiles
// 4 s .. 4 s + 3 of a chunk of up to 64 SETS pairs, so each stage of rows
// comes from HBM once for 64 SETS tokens.
template <int TYPE, int EPI, int SETS>
struct GroupShape {
  static constexpr int NB = EPI == kEpiSwiglu ? 2 : 1;
  static constexpr int RUN = 128 * GroupB<TYPE>::kBlock;  // stage-major run: 64 rows x 2 blocks
  static constexpr int RP = 2 * GroupB<TYPE>::kBlock;     // a row's bytes in the run
  static constexpr int ROWS = 64 / NB;  // rows per matrix and wave
  static constexpr int NS = ROWS / 16;
  // row waves of a set (the silu-gate pair's two matrices keep four)
  static constexpr int RW = NB == 2 ? 4 : kGroupWaves;
  static constexpr int WAVES = RW * SETS;
  static constexpr int WG_ROWS = RW * ROWS;
  static constexpr int PIECES = GroupB<TYPE>::kPieces;
  static constexpr int TOKENS = 64 * SETS;                  // pairs per chunk
  static constexpr int A_BYTES = TOKENS * 256 + TOKENS * 16;  // + each token's 4 group sums
  // per wave of a set: one matrix, the run itself (the last DMA instruction
  // takes only the lanes inside it); two, piece-major
  static constexpr int B_BYTES = NB == 1 ? RUN : PIECES * NB * 1024;
  static constexpr int STAGE = A_BYTES + RW * B_BYTES;
  static constexpr int LDS = 2 * STAGE;
  static_assert(RUN % 16 == 0 && STAGE % 16 == 0, "16-byte DMA slots");
  static constexpr bool FITS = LDS <= 160 * 1024;  // else the launch is refused
};

// Dword i of row r of a wave's weight stage (matrix nb): one matrix, the
// stage-major run (rows RP = two blocks' bytes apart); two, piece-major.
template <int NB, int P, int RP>
__device__ __forceinline__ uint32_t pm_dword(const uint8_t* wbuf, int nb, int r, uint32_t i) {
  if constexpr (NB == 1) return *reinterpret_cast<const uint32_t*>(wbuf + r * RP + 4 * i);
  return *reinterpret_cast<const uint32_t*>(wbuf + (((i >> 2) * NB + nb) * 64 + r) * 16 + 4 * (i & 3));
}

// The words GemmB<TYPE>::fetch reads and the scale of group j, from the
// piece-major stage (byte o of the row image: dword o >> 2).
template <int TYPE, int NB>
__device__ __forceinline__ typename GemmB<TYPE>::Raw group_fetch(const uint8_t* wbuf, int nb, int r,
                                                                 uint32_t sh, int j, int g) {
  if constexpr (TYPE == kQ5_0) {
    const uint32_t o = sh + 22u * (uint32_t)j;
    const uint32_t os = (o + 6u + 8u * (uint32_t)(g & 1)) >> 2, ob = (o + 2u + (uint32_t)g) >> 2;
    constexpr int P = GroupB<TYPE>::kPieces, RP = 2 * GroupB<TYPE>::kBlock;
    return u32x4{pm_dword<NB, P, RP>(wbuf, nb, r, os), pm_dword<NB, P, RP>(wbuf, nb, r, os + 1u),
                 pm_dword<NB, P, RP>(wbuf, nb, r, os + 2u), pm_dword<NB, P, RP>(wbuf, nb, r, ob)};
  } else {
    const uint32_t os = (sh + 34u * (uint32_t)j + 2u + 8u * (uint32_t)g) >> 2;
    constexpr int P = GroupB<TYPE>::kPieces, RP = 2 * GroupB<TYPE>::kBlock;
    return u32x4{pm_dword<NB, P, RP>(wbuf, nb, r, os), pm_dword<NB, P, RP>(wbuf, nb, r, os + 1u),
                 pm_dword<NB, P, RP>(wbuf, nb, r, os + 2u), 0u};
  }
}
template <int TYPE, int NB>
__device__ __forceinline__ void group_scale(const uint8_t* wbuf, int nb, int r, uint32_t sh, int j,
                                            float& delta, float& c) {
  const uint32_t o = sh + (uint32_t)GroupB<TYPE>::kBlock * (uint32_t)j;  // even
  const uint32_t bits = (pm_dword<NB, GroupB<TYPE>::kPieces, 2 * GroupB<TYPE>::kBlock>(
                             wbuf, nb, r, o >> 2) >> (8 * (o & 3u))) & 0xFFFFu;
  delta = half_bits_to_float(bits);
  if constexpr (TYPE == kQ5_0) c = 144.f * delta;
  else c = 128.f * delta;
}

template <int TYPE, int EPI, int SETS>
__global__ void __launch_bounds__((64 * GroupShape<TYPE, EPI, SETS>::WAVES), 2)
moe_group_kernel(MoeGemmArgs args) {
  using B = GemmB<TYPE>;
  using Sh = GroupShape<TYPE, EPI, SETS>;
  constexpr int NB = Sh::NB, NS = Sh::NS, MT = kGroupTiles;
  // one matrix: the stage-major rows in lane order
  constexpr bool kStagedQ5 = TYPE == kQ5_0 && NB == 1, kStagedQ8 = TYPE == kQ8_0 && NB == 1;
  constexpr int BB = GroupB<TYPE>::kBlock;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  // (chunk, row tile) from the XCD-grouped 1-D grid of the batch pipelines
  const int T = args.row_tiles, L = blockIdx.x;
  const int bx = (L / (8 * T)) * 8 + (L & 7);
  const int by = (L >> 3) % T;
  const int* cc = args.chunk_counts;
  const int nchunks = args.joint ? cc[0] + cc[1] : cc[args.group];
  if (bx >= nchunks) return;  // the whole workgroup, before any barrier
  // a joint launch takes the shared expert's chunks (all full) first, so
  // that routed chunks, many of them short, make up the launch's last round
  const int cx = args.joint ? (bx < cc[1] ? cc[0] + bx : bx - cc[1]) : bx;
  const MoeChunk ch = args.chunks[(!args.joint && args.group ? cc[0] : 0) + cx];
  MoeGemmArgs a = args;
  if (args.joint && cx >= cc[0]) {
    a.w0 = args.s_w0;
    a.w1 = args.s_w1;
    a.row_bytes = args.s_row_bytes;
    a.expert_stride = 0;
    a.N = args.s_N;
    a.K = args.s_K;
  }
  const int wg_row0 = by * Sh::WG_ROWS;
  if (wg_row0 >= a.N) return;  // the whole workgroup
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rw = wave & (Sh::RW - 1), set = wave / Sh::RW;  // row group, token set
  const int n = lane & 15, g = lane >> 4;
  // rows of this wave (a wave past the last row still takes part in every
  // barrier: its rows clamp to the last one and its outputs are dropped)
  const int n0 = wg_row0 + rw * Sh::ROWS;
  const int count = __builtin_amdgcn_readfirstlane(ch.count);
  const int start = __builtin_amdgcn_readfirstlane(ch.start);
  const int expert = __builtin_amdgcn_readfirstlane(ch.expert);
  const int nt = (count + 15) >> 4;  // token tiles holding pairs
  const int nt_set = min(max(nt - kGroupTiles * set, 0), kGroupTiles);  // this wave's

  // lane l = token l of the chunk (and token 64 + l with two sets): its
  // split row and group sums (tokens past the count read the first token's)
  uint32_t a_off[SETS], s_off[SETS];
  int q_l[SETS];
#pragma unroll
  for (int k = 0; k < SETS; ++k) {
    const int tk = 64 * k + lane;
    q_l[k] = a.perm[start + (tk < count ? tk : 0)];
    const int64_t r_l = a.a_by_token ? (q_l[k] < a.pairs ? q_l[k] / a.top_k : q_l[k] - a.pairs)
                                     : q_l[k];
    a_off[k] = (uint32_t)(r_l * a.aq_stride * 2);
    s_off[k] = (uint32_t)(r_l * a.as_stride * 4);
  }
  const uint8_t* aq_base = uniform_ptr(reinterpret_cast<const uint8_t*>(a.aq));
  const uint8_t* as_base = uniform_ptr(reinterpret_cast<const uint8_t*>(a.as));
  const uint8_t* base[NB];
  base[0] = uniform_ptr(a.w0 + (int64_t)expert * a.expert_stride);
  if constexpr (NB == 2) base[1] = uniform_ptr(a.w1 + (int64_t)expert * a.expert_stride);
  const uint32_t rb = (uint32_t)a.row_bytes;
  // weight DMA: two matrices, lane l takes row (l mod ROWS) of each; one
  // matrix, instruction q takes line slot 64 q + l = row r, piece c
  // (offsets without the stage's, 4-byte aligned: a stage spans a multiple
  // of 4 bytes)
  const uint32_t brow = (uint32_t)min(n0 + (lane & (Sh::ROWS - 1)), a.N - 1) * rb;
  // one matrix: the stage-major layout (moe_repack_launch), this wave's run
  // of each stage read whole -- instruction q takes its bytes 1024 q ..
  // 1024 q + 1023, lanes past the run re-reading its last piece
  uint32_t wdma[Sh::PIECES];
#pragma unroll
  for (int q = 0; q < Sh::PIECES; ++q) wdma[q] = (uint32_t)min(16 * (64 * q + lane), Sh::RUN - 16);
  // activation DMA: this wave's instructions k = wave + WAVES u take token
  // 4 k + (l >> 4) and piece (l & 15) ^ (token & 15) into slot l of block k
  uint32_t adma[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = 4 * (wave + Sh::WAVES * u) + (lane >> 4);
    int ao = __shfl((int)a_off[0], t & 63);
    if constexpr (SETS == 2) {
      const int ao1 = __shfl((int)a_off[1], t & 63);
      ao = t < 64 ? ao : ao1;
    }
    adma[u] = (uint32_t)ao + 16u * (uint32_t)((lane & 15) ^ (t & 15));
  }
  // fetch rows 16 m + n: their byte shift within a dword is the same at
  // every stage (2 blocks span a multiple of 4 bytes) and for every m (rows
  // 16 apart: row_bytes * 16 is a multiple of 4), so the subtiles' LDS words
  // sit at constant offsets from one address.  (A row past the last one
  // reads the clamped row's bytes at this shift; its outputs are dropped.)
  const uint32_t sh0 = NB == 1 ? 0u : ((uint32_t)(n0 + n) * rb) & 3u;  // runs: rows on dwords
  uint32_t sh[NS];
#pragma unroll
  for (int m = 0; m < NS; ++m) sh[m] = sh0;

  const int groups = a.K >> 5;
  const int nstage = (groups + 1) >> 1;
  const uint32_t lds0 = lds_address(lds);

  // (the token blocks of tiles past the chunk's are never read; a wave
  // whose rows all lie past the last loads no rows and computes nothing, nor
  // does a wave whose set holds no token tile; the first set loads the rows)
  const bool live = n0 < a.N;
  const bool work = live && nt_set > 0;
  auto issue = [&](int st, int buf) {
    const uint32_t stg = lds0 + (uint32_t)(buf * Sh::STAGE);
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (wave + Sh::WAVES * u < 4 * nt)
        load_lds16(aq_base, adma[u] + 256u * (uint32_t)st,
                   stg + 1024u * (uint32_t)(wave + Sh::WAVES * u));
    if (wave < SETS)  // wave k: the sums of tokens 64 k .. 64 k + 63
      load_lds16(as_base, (wave == 0 ? s_off[0] : s_off[SETS - 1]) + 16u * (uint32_t)st,
                 stg + (uint32_t)(Sh::TOKENS * 256 + 1024 * wave));
    if (!live || set > 0) return;
    const uint32_t wst = stg + Sh::A_BYTES + (uint32_t)rw * Sh::B_BYTES;
    const uint32_t sto = (uint32_t)st * (uint32_t)(2 * BB);
    if constexpr (NB == 1) {
      const uint8_t* run =
          uniform_ptr(base[0] + (int64_t)((n0 >> 6) * nstage + st) * Sh::RUN);
#pragma unroll
      for (int q = 0; q < Sh::PIECES; ++q)
        if (16 * (64 * q + lane) < Sh::RUN)  // lane 0 always: every instruction issues
          load_lds16(run, wdma[q], wst + 1024u * (uint32_t)q);
    } else {
      const uint32_t off = (brow + sto) & ~3u;
#pragma unroll
      for (int k = 0; k < Sh::PIECES; ++k)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          load_lds16(base[nb], off + 16u * (uint32_t)k, wst + (uint32_t)((k * NB + nb) * 1024));
    }
  };

  floatx4 tot[MT][NS][NB];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int m = 0; m < NS; ++m)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) tot[i][m][nb] = floatx4{0.f, 0.f, 0.f, 0.f};
  // offsets of the current 256-element chunk: -c of group 4 q + g of the
  // lane's rows, and the lane token's sum of that group.  The stage-major
  // rows keep, instead of -c, the word holding the deltas of the stage
  // with the lane's group (c is formed from it when the offsets apply, the
  // same product as the scale's).
  constexpr bool kStaged = kStagedQ5 || kStagedQ8;
  float cneg[NS][NB][2];
  uint32_t cdw[NS][2];
  float sv[MT][2];
  auto clear_offsets = [&]() {
#pragma unroll
    for (int m = 0; m < NS; ++m) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) cneg[m][nb][0] = cneg[m][nb][1] = 0.f;
      cdw[m][0] = cdw[m][1] = 0u;
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) sv[i][0] = sv[i][1] = 0.f;
  };
  clear_offsets();

  // The token-tile count is a compile-time parameter of the stage loop (four
  // copies, one chosen per workgroup): no branch may separate an MFMA from
  // the VALU instruction that reads its result, or the wait states the
  // result needs can be lost on the branch path.
  auto apply_offsets = [&](auto ntc) {
    constexpr int NT = decltype(ntc)::value;
    if constexpr (kStaged) {
      // (a cleared word -- a group past the last -- gives -c = -0, which
      // leaves the sums as +0 does: they start at +0 and never become -0)
      constexpr float kC = kStagedQ5 ? 144.f : 128.f;
#pragma unroll
      for (int m = 0; m < NS; ++m)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const uint32_t bits = (g & 1) ? cdw[m][q] >> 16 : cdw[m][q] & 0xFFFFu;
          cneg[m][0][q] = -(kC * half_bits_to_float(bits));
        }
    }
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int i = 0; i < NT; ++i)
#pragma unroll
        for (int m = 0; m < NS; ++m)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            tot[i][m][nb] = mfma4f32(sv[i][q], cneg[m][nb][q], tot[i][m][nb]);
    clear_offsets();
  };

  auto compute = [&](auto ntc, int st, auto bufc) {
    constexpr int NT = decltype(ntc)::value;
    const uint8_t* stg = lds + decltype(bufc)::value * Sh::STAGE;
    const uint8_t* wbuf = stg + Sh::A_BYTES + rw * Sh::B_BYTES;
    const int ls = st & 3;  // stage within the 256-element chunk
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      if (2 * st + jj < groups) {
        const int j8 = 2 * ls + jj;  // group within the chunk
        typename B::Raw raw[NS][NB];
        float dl[NS][NB];
#pragma unroll
        for (int m = 0; m < NS; ++m)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            float c;
            if constexpr (kStagedQ5) {
              raw[m][nb] = staged_q5_fetch(wbuf, 16 * m + n, jj, g);
              staged_q5_scale(wbuf, 16 * m + n, jj, dl[m][nb], c);
            } else if constexpr (kStagedQ8) {
              const uint8_t* row = wbuf + (16 * m + n) * Sh::RP;
              raw[m][nb] = staged_q8_fetch(row, jj, g);
              staged_q8_scale(row, jj, dl[m][nb], c);
            } else {
              raw[m][nb] = group_fetch<TYPE, NB>(wbuf, nb, 16 * m + n, sh[m], jj, g);
              group_scale<TYPE, NB>(wbuf, nb, 16 * m + n, sh[m], jj, dl[m][nb], c);
            }
            if constexpr (!kStaged) {
              // (q = j8 >> 2 is uniform: a select per lane, not an indexed write)
              const bool mine = (j8 & 3) == g;
              cneg[m][nb][0] = (mine && j8 < 4) ? -c : cneg[m][nb][0];
              cneg[m][nb][1] = (mine && j8 >= 4) ? -c : cneg[m][nb][1];
            }
          }
        // token 16 i + n of the set: block 4 i + (n >> 2), slot 16 (n & 3) +
        // (piece ^ n)
        bf16x8 hi[NT], lo[NT];
        const uint8_t* at = stg + set * 16384 + (n >> 2) * 1024 + (n & 3) * 256;
#pragma unroll
        for (int i = 0; i < NT; ++i) {
          hi[i] = *reinterpret_cast<const bf16x8*>(at + 4096 * i + 16 * ((jj * 8 + g) ^ n));
          lo[i] = *reinterpret_cast<const bf16x8*>(at + 4096 * i + 16 * ((jj * 8 + 4 + g) ^ n));
        }
#pragma unroll
        for (int m = 0; m < NS; ++m)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            typename B::Frag bf;
            if constexpr (kStagedQ5) bf = staged_q5_decode(raw[m][nb], g);
            else if constexpr (kStagedQ8) bf = staged_q8_decode(raw[m][nb]);
            else bf = B::decode(raw[m][nb], sh[m], jj, g);
            const float delta = dl[m][nb];
#pragma unroll
            for (int i = 0; i < NT; ++i) {
              floatx4 d = mfma_b(hi[i], bf, floatx4{0.f, 0.f, 0.f, 0.f});
              d = mfma_b(lo[i], bf, d);
              floatx4& t = tot[i][m][nb];
              t[0] = fmaf(delta, d[0], t[0]);
              t[1] = fmaf(delta, d[1], t[1]);
              t[2] = fmaf(delta, d[2], t[2]);
              t[3] = fmaf(delta, d[3], t[3]);
            }
          }
      }
    }
    // this stage holds groups 2 st and 2 st + 1: lanes whose offset group
    // 4 q + g is one of them take the lane token's sum of it (the sum of
    // its two 16-halves, as the other pipelines form it) and, stage-major,
    // the word of its rows' deltas
    {
      const bool mine = (g >> 1) == (ls & 1);
      const bool ok = 2 * st + (g & 1) < groups;
      if constexpr (kStaged) {
#pragma unroll
        for (int m = 0; m < NS; ++m) {
          const uint32_t dw =
              kStagedQ5 ? staged_q5_deltas(wbuf, 16 * m + n)
                        : reinterpret_cast<const uint32_t*>(wbuf + (16 * m + n) * Sh::RP)[16];
          cdw[m][0] = (mine && ok && ls < 2) ? dw : cdw[m][0];
          cdw[m][1] = (mine && ok && ls >= 2) ? dw : cdw[m][1];
        }
      }
#pragma unroll
      for (int i = 0; i < NT; ++i) {
        const float* sp = reinterpret_cast<const float*>(
            stg + Sh::TOKENS * 256 + (64 * set + 16 * i + n) * 16);
        const float v = sp[2 * (g & 1)] + sp[2 * (g & 1) + 1];
        const float val = ok ? v : 0.f;
        sv[i][0] = (mine && ls < 2) ? val : sv[i][0];
        sv[i][1] = (mine && ls >= 2) ? val : sv[i][1];
      }
    }
  };

  // epilogue: lane (n, g) holds tokens 16 i + 4 g + r of rows n0 + 16 m + n
  auto finish = [&](auto ntc) {
    constexpr int NT = decltype(ntc)::value;
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      int qout[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tk = 64 * set + 16 * i + 4 * g + r;
        int q = __shfl(q_l[0], tk & 63);  // lane tk holds the pair of token tk
        if constexpr (SETS == 2) {
          const int q1 = __shfl(q_l[1], tk & 63);
          q = tk < 64 ? q : q1;
        }
        qout[r] = tk < count ? q : 0;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tk = 64 * set + 16 * i + 4 * g + r;
        const bool ok_t = tk < count;
        const int q = qout[r];
        if constexpr (EPI == kEpiDown) {
#pragma unroll
          for (int m = 0; m < NS; ++m) {
            const int row = n0 + 16 * m + n;
            if (ok_t && row < a.N) a.out[(int64_t)q * a.out_stride + row] = tot[i][m][0][r];
          }
        } else {
          uint16_t* oq = a.oq + (int64_t)q * a.oq_stride;
          float* os = a.os + (int64_t)q * a.os_stride;
#pragma unroll
          for (int m = 0; m < NS; ++m) {
            const int row = n0 + 16 * m + n;
            float act;
            if constexpr (EPI == kEpiSwiglu) {
#pragma clang fp contract(off)
              act = silu_ref(tot[i][m][0][r]) * tot[i][m][1][r];  // llambda.lisp:5386-5401
            } else {
              act = relu2_ref(tot[i][m][0][r]);  // llambda.lisp:5921-5926
            }
            uint32_t hb, lb;
            float sum;
            split_bf16(act, hb, lb, sum);
            const bool ok = ok_t && row < a.N;
            if (ok) {
              uint16_t* p = oq + 64 * (row >> 5) + (row & 31);
              p[0] = (uint16_t)hb;
              p[32] = (uint16_t)lb;
            }
            const float s16 = group_sum(ok ? sum : 0.f, 4);
            if (n == 0 && ok) os[row >> 4] = s16;
          }
        }
      }
    }
  };

  // the stages; each 256-element chunk's offsets follow its last stage (the
  // final chunk's after the loop, in line with the epilogue)
  // (two stages per iteration: the buffer of each is a compile-time
  // constant, folded into the LDS instructions' offsets.  Deeper rings, of
  // both operands or of either, measured slower.)
  auto stage = [&](auto ntc, int st, auto bufc) {
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();
    if (st + 1 < nstage) issue(st + 1, 1 - decltype(bufc)::value);
    if (work) {
      compute(ntc, st, bufc);
      if ((st & 3) == 3 && st + 1 < nstage) apply_offsets(ntc);
    }
  };
  auto run = [&](auto ntc) {
    issue(0, 0);
    for (int st = 0; st < nstage; st += 2) {
      stage(ntc, st, std::integral_constant<int, 0>{});
      if (st + 1 < nstage) stage(ntc, st + 1, std::integral_constant<int, 1>{});
    }
    if (work) {
      apply_offsets(ntc);
      finish(ntc);
    }
  };
  switch (nt_set) {
    case 1: run(std::integral_constant<int, 1>{}); break;
    case 2: run(std::integral_constant<int, 2>{}); break;
    case 3: run(std::integral_constant<int, 3>{}); break;
    default: run(std::integral_constant<int, 4>{}); break;
  }

}

// ------------------------------------------------------------------ host

template <int TYPE, int EPI, int MT, int PIPE, bool ALIGNED, bool GATE = false>
static hipError_t launch_gemm_t(const MoeGemmArgs& a_in, int max_chunks, hipStream_t stream) {
  using Sh = GemmShape<TYPE, EPI, PIPE>;
  MoeGemmArgs a = a_in;
  const int nchunk = (std::max(a.K, a.joint ? a.s_K : 0) + 255) / 256;
  const int per_wave = (nchunk + Sh::kWaves - 1) / Sh::kWaves;
  // the decode ring: at most DEPTH stages, no more than a wave's chunks, and
  // no more than fit the 160 KB of LDS a workgroup may hold
  constexpr int kLdsMax = 160 * 1024;
  const int fit = (kLdsMax - gemm_lds_bytes<TYPE, EPI, PIPE>(0)) / (Sh::kWaves * Sh::STAGE);
  a.depth = PIPE == kPipeDecode ? std::max(1, std::min({Sh::DEPTH, per_wave, fit})) : Sh::DEPTH;
  const int lds = gemm_lds_bytes<TYPE, EPI, PIPE>(a.depth);
  const auto kernel = moe_gemm_kernel<TYPE, EPI, MT, PIPE, ALIGNED, GATE>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
  }
  const int rows = a.joint ? std::max(a.N, a.s_N) : a.N;
  const int tiles = (rows + Sh::WG_ROWS - 1) / Sh::WG_ROWS;
  // the double pipeline's workgroups take two row tiles when K is short (at
  // most 4 chunks), so that their prologue is paid once for both (measured
  // on Qwen3Next B=256: one, two and four tiles within 2% of each other,
  // two ahead)
  a.tiles_per_wg = PIPE == kPipeDouble && nchunk <= 4 && !gemm_jit_a<TYPE, EPI, PIPE>() ? 2 : 1;
  a.row_tiles = (tiles + a.tiles_per_wg - 1) / a.tiles_per_wg;
  // batch pipelines: the XCD-grouped 1-D grid (chunks padded to a multiple of 8)
  const dim3 grid = PIPE == kPipeDecode ? dim3(max_chunks, tiles)
                                        : dim3(((max_chunks + 7) / 8) * 8 * a.row_tiles);
  hipLaunchKernelGGL(kernel, grid, dim3(64 * Sh::kWaves), lds, stream, a);
  return hipGetLastError();
}

template <int TYPE, int EPI, bool ALIGNED>
static hipError_t launch_gemm_mt(const MoeGemmArgs& a, int mt, int max_chunks, hipStream_t s) {
  switch (mt) {
    case 0:
      if constexpr (EPI != kEpiDown)
        if (a.fused_gate) return launch_gemm_t<TYPE, EPI, 1, kPipeDecode, ALIGNED, true>(a, max_chunks, s);
      return launch_gemm_t<TYPE, EPI, 1, kPipeDecode, ALIGNED>(a, max_chunks, s);
    case 1: return launch_gemm_t<TYPE, EPI, 1, kPipeDouble, ALIGNED>(a, max_chunks, s);
    case 2:
      // (Q5_0 rows that are not dword multiples take 16-pair chunks: the
      // launcher never asks for these)
      if constexpr (TYPE == kQ5_0 && !ALIGNED && EPI != kEpiSwiglu) return hipErrorInvalidValue;
      else return launch_gemm_t<TYPE, EPI, 2, kPipeWide, ALIGNED>(a, max_chunks, s);
    default: return hipErrorInvalidValue;
  }
}

template <int TYPE, int EPI>
static hipError_t launch_gemm_al(const MoeGemmArgs& a, int mt, int max_chunks, hipStream_t s) {
  // tile-major (K-quant) rows start on dwords; packed rows are aligned when
  // their bytes are dword multiples (a joint launch: the shared expert's too)
  constexpr bool kTiled = GemmB<TYPE>::kTilePitch != 0;
  const bool aligned = a.row_bytes % 4 == 0 && (!a.joint || a.s_row_bytes % 4 == 0);
  if (kTiled || aligned) return launch_gemm_mt<TYPE, EPI, true>(a, mt, max_chunks, s);
  if constexpr (!kTiled) return launch_gemm_mt<TYPE, EPI, false>(a, mt, max_chunks, s);
  return hipErrorInvalidValue;
}

template <int EPI>
static hipError_t launch_gemm_epi(int type, const MoeGemmArgs& a, int mt, int max_chunks,
                                  hipStream_t s) {
  switch (type) {
    case kQ4_K: return launch_gemm_al<kQ4_K, EPI>(a, mt, max_chunks, s);
    case kQ6_K: return launch_gemm_al<kQ6_K, EPI>(a, mt, max_chunks, s);
    case kQ5_0: return launch_gemm_al<kQ5_0, EPI>(a, mt, max_chunks, s);
    case kQ8_0: return launch_gemm_al<kQ8_0, EPI>(a, mt, max_chunks, s);
    default: return hipErrorInvalidValue;
  }
}

template <int TYPE, int EPI, int SETS>
static hipError_t launch_group_t(const MoeGemmArgs& a_in, int max_chunks, hipStream_t stream) {
  using Sh = GroupShape<TYPE, EPI, SETS>;
  if constexpr (!Sh::FITS) {
    return hipErrorInvalidValue;  // this build's row waves leave no room in LDS
  } else {
    MoeGemmArgs a = a_in;
    const auto kernel = moe_group_kernel<TYPE, EPI, SETS>;
    if (Sh::LDS > 65536) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, Sh::LDS);
      if (e != hipSuccess) return e;
    }
    const int rows = a.joint ? std::max(a.N, a.s_N) : a.N;
    a.row_tiles = (rows + Sh::WG_ROWS - 1) / Sh::WG_ROWS;
    a.tiles_per_wg = 1;
    a.depth = 2;
    const dim3 grid(((max_chunks + 7) / 8) * 8 * a.row_tiles);
    hipLaunchKernelGGL(kernel, grid, dim3(64 * Sh::WAVES), Sh::LDS, stream, a);
    return hipGetLastError();
  }
}

template <int EPI, int SETS>
static hipError_t launch_group_epi(int type, const MoeGemmArgs& a, int max_chunks, hipStream_t s) {
  // the stage offsets (256 bytes of split row, 16 of sums per stage) are
  // 32-bit: the launcher only chooses this pipeline when they fit
  if (a.K % 32 || (a.joint && a.s_K % 32)) return hipErrorInvalidValue;
  switch (type) {
    case kQ5_0: return launch_group_t<kQ5_0, EPI, SETS>(a, max_chunks, s);
    case kQ8_0: return launch_group_t<kQ8_0, EPI, SETS>(a, max_chunks, s);
    default: return hipErrorInvalidValue;
  }
}

bool moe_group_pipeline_types(int type) { return type == kQ5_0 || type == kQ8_0; }

// The stage-major layout of the group pipeline's one-matrix launches: per
// slab, per 64-row tile, per stage of two blocks, the tile's 64 rows' two
// blocks back to back (a wave's stage then comes in as one contiguous run;
// rows past the slab's and the block past an odd count are zeros).  The
// blocks are reordered so that MFMA lane g decodes its eight codes from
// aligned dwords in a few instructions: Q8_0 rows as the 64 codes q + 128
// then the two deltas (staged_q8_decode); Q5_0 as planes of one dword of
// five- and three-bit fields per lane, block and row, swizzled so that a
// subtile's 64 reads hit 64 banks, a word of the remaining bits per block
// and row, rotated into place per lane (staged_q5_decode), and the deltas.
static int64_t repack_slab_bytes(int type, int64_t rows, int64_t columns) {
  const int64_t bb = block_bytes(type), nblk = columns / 32;
  return (rows + 63) / 64 * ((nblk + 1) / 2) * 128 * bb;
}
int64_t moe_repack_bytes(int type, int64_t slabs, int64_t rows, int64_t columns) {
  return slabs * repack_slab_bytes(type, rows, columns);
}

__global__ void __launch_bounds__(256)
moe_repack_kernel(const uint8_t* __restrict__ src, int64_t rows, int64_t rb, int nblk, int bb,
                  int ntile, int nstage, uint8_t* __restrict__ dst, int64_t total) {
  const int64_t run = 128 * (int64_t)bb;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    int64_t q = i / run;
    const int o = (int)(i - q * run);
    const int stage = (int)(q % nstage);
    q /= nstage;
    const int tile = (int)(q % ntile);
    const int64_t slab = q / ntile;
    const int r = o / (2 * bb), rest = o - r * 2 * bb;
    const int64_t row = (int64_t)tile * 64 + r;
    const uint8_t* rsrc = src + (slab * rows + row) * rb;
    uint8_t v = 0;
    if (bb == 22) {
      // Q5_0, plane order (staged_q5_fetch): the run's dword D = o / 4
      const int D = o >> 2, byte = o & 3;
      int pr, j, kind, g = 0;  // kind 0: code fields, 1: the word of other bits, 2: deltas
      if (D < 512) {
        kind = 0;
        j = (D >> 6) >> 2;
        g = (D >> 6) & 3;
        pr = (D & 63) ^ (16 * g);
      } else if (D < 640) {
        kind = 1;
        j = (D - 512) >> 6;
        pr = (D - 512) & 63;
      } else {
        kind = 2;
        j = byte >> 1;
        pr = D - 640;
      }
      const int64_t prow = (int64_t)tile * 64 + pr;
      const int blk = 2 * stage + j;
      if (prow < rows && blk < nblk) {
        const uint8_t* blkp = src + (slab * rows + prow) * rb + (int64_t)blk * bb;
        const uint32_t qh = blkp[2] | (uint32_t)blkp[3] << 8 | (uint32_t)blkp[4] << 16 |
                            (uint32_t)blkp[5] << 24;
        auto code = [&](int e) -> uint32_t {  // q of element e (0..31)
          const uint32_t nib = e < 16 ? blkp[6 + e] & 15 : blkp[6 + e - 16] >> 4;
          return nib | ((qh >> e) & 1u) << 4;
        };
        if (kind == 0) {
          v = (uint8_t)(code(8 * g + byte) | (code(8 * g + 4 + byte) & 7u) << 5);
        } else if (kind == 1) {
          // bits 3 and 4 of code 8g + 4 + b at bits (8b + 3 + 2g) and
          // (8b + 4 + 2g) mod 32 of the word
          uint32_t bits = 0;
          for (int k = 0; k < 8; ++k) {
            const int p = 8 * byte + k;
            for (int gg = 0; gg < 4; ++gg) {  // the one lane whose bit p is
              const int sft = (p - 3 - 2 * gg) & 31;
              if ((sft & 7) < 2)
                bits |= ((code(8 * gg + 4 + (sft >> 3)) >> (3 + (sft & 7))) & 1u) << k;
            }
          }
          v = (uint8_t)bits;
        } else {
          v = blkp[byte & 1];
        }
      }
    } else {
      // Q8_0: [0, 64) the two blocks' codes as q + 128 (q ^ 0x80), [64, 68)
      // the deltas
      const int j = rest < 64 ? rest >> 5 : (rest - 64) >> 1;
      const int blk = 2 * stage + j;
      if (row < rows && blk < nblk) {
        const uint8_t* blkp = rsrc + (int64_t)blk * bb;
        v = rest < 64 ? (uint8_t)(blkp[2 + (rest & 31)] ^ 0x80u) : blkp[(rest - 64) & 1];
      }
    }
    dst[i] = v;
  }
}

hipError_t moe_repack_launch(int type, const uint8_t* src, int64_t slabs, int64_t rows,
                             int64_t columns, uint8_t* dst, hipStream_t stream) {
  if (!moe_group_pipeline_types(type) || columns % 32 || rows <= 0 || slabs <= 0)
    return hipErrorInvalidValue;
  const int bb = block_bytes(type), nblk = (int)(columns / 32);
  const int ntile = (int)((rows + 63) / 64), nstage = (nblk + 1) / 2;
  const int64_t total = moe_repack_bytes(type, slabs, rows, columns);
  const int grid = (int)std::min<int64_t>((total + 255) / 256, 65536);
  hipLaunchKernelGGL(moe_repack_kernel, dim3(grid), dim3(256), 0, stream, src, rows,
                     nblk * (int64_t)bb, nblk, bb, ntile, nstage, dst, total);
  return hipGetLastError();
}

// The tile-major copy (moe.h): the grid strides over the destination's
// 16-bit halves (every chunk length and offset is even), each one row r of
// tile t, chunk kc of slab s: zeros in a row's dword pad and past the slab.
__global__ void __launch_bounds__(256)
moe_tile_kernel(const uint16_t* __restrict__ src, int64_t rows, int64_t row_halves, int nchunk,
                int span_halves, int pitch_halves, int64_t tiles, int pair_halves,
                uint16_t* __restrict__ dst, int64_t total) {
  const int64_t chunk_halves = 16 * (int64_t)pitch_halves;
  const int64_t tile_halves = nchunk * chunk_halves;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t_all = i / tile_halves;  // slab * tiles + tile
    const int64_t in_tile = i - t_all * tile_halves;
    const int kc = (int)(in_tile / chunk_halves);
    const int in_chunk = (int)(in_tile - kc * chunk_halves);
    const int r = in_chunk / pitch_halves, h = in_chunk - r * pitch_halves;
    const int64_t slab = t_all / tiles, row = (t_all - slab * tiles) * 16 + r;
    // the first pair_halves halves: 32-byte runs whose dword d' = 2g + s
    // comes from dword 4s + g of the source run
    int hs = h;
    if (h < pair_halves) {
      const int d = (h & 15) >> 1;
      hs = (h & ~15) + 2 * (4 * (d & 1) + (d >> 1)) + (h & 1);
    }
    uint16_t v = 0;
    if (row < rows && h < span_halves)
      v = src[(slab * rows + row) * row_halves + (int64_t)kc * span_halves + hs];
    dst[i] = v;
  }
}

bool moe_tiled_type(int type) { return type == kQ4_K || type == kQ6_K; }

int64_t moe_slab_bytes(int type, int64_t rows, int64_t columns) {
  if (!moe_tiled_type(type)) return rows * (columns / block_weights(type)) * block_bytes(type);
  const int pitch = type == kQ4_K ? GemmB<kQ4_K>::kTilePitch : GemmB<kQ6_K>::kTilePitch;
  return (rows + 15) / 16 * (columns / 256) * 16 * pitch;
}

hipError_t moe_tile_launch(int type, const uint8_t* src, int64_t slabs, int64_t rows,
                           int64_t columns, uint8_t* dst, hipStream_t stream) {
  if (!moe_tiled_type(type) || columns % 256 || rows <= 0 || slabs <= 0)
    return hipErrorInvalidValue;
  const int span = type == kQ4_K ? GemmB<kQ4_K>::kSpan : GemmB<kQ6_K>::kSpan;
  const int pitch = type == kQ4_K ? GemmB<kQ4_K>::kTilePitch : GemmB<kQ6_K>::kTilePitch;
  const int nchunk = (int)(columns / 256);
  const int64_t total = slabs * moe_slab_bytes(type, rows, columns) / 2;
  const int grid = (int)std::min<int64_t>((total + 255) / 256, 65536);
  hipLaunchKernelGGL(moe_tile_kernel, dim3(grid), dim3(256), 0, stream,
                     reinterpret_cast<const uint16_t*>(src), rows, (int64_t)nchunk * span / 2,
                     nchunk, span / 2, pitch / 2, (rows + 15) / 16, type == kQ6_K ? 96 : 0,
                     reinterpret_cast<uint16_t*>(dst), total);
  return hipGetLastError();
}

template <int TYPE, bool ALIGNED>
static hipError_t launch_combine_t(const MoeGemmArgs& a_in, const MoeCombineArgs& c,
                                   hipStream_t stream) {
  using Sh = CombineShape<TYPE>;
  MoeGemmArgs a = a_in;
  constexpr int kLdsMax = 160 * 1024;
  const int fit = (kLdsMax - combine_lds_bytes<TYPE>(0)) / (Sh::kWaves * Sh::STAGE);
  a.depth = std::max(1, std::min(Sh::DEPTH, fit));
  const int lds = combine_lds_bytes<TYPE>(a.depth);
  const auto kernel = moe_down_combine_kernel<TYPE, ALIGNED>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kernel, dim3((a.N + 15) / 16), dim3(64 * Sh::kWaves), lds, stream, a, c);
  return hipGetLastError();
}

bool moe_down_combine_supported(int type, const MoeGemmArgs& a) {
  if (a.top_k < 1 || a.top_k + 1 > kCombineSlots || a.N <= 0) return false;
  const int64_t units = (int64_t)a.top_k * ((a.K + 255) / 256) + (a.joint ? (a.s_K + 255) / 256 : 0);
  if (units > kCombineUnits) return false;
  return type == kQ4_K || type == kQ6_K || type == kQ5_0 || type == kQ8_0;
}

hipError_t moe_down_combine_launch(int type, const MoeGemmArgs& a, const MoeCombineArgs& c,
                                   hipStream_t stream) {
  if (!moe_down_combine_supported(type, a)) return hipErrorInvalidValue;
  const bool aligned = a.row_bytes % 4 == 0 && (!a.joint || a.s_row_bytes % 4 == 0);
  switch (type) {
    // (K-quants: tile-major rows, which start on dwords)
    case kQ4_K: return launch_combine_t<kQ4_K, true>(a, c, stream);
    case kQ6_K: return launch_combine_t<kQ6_K, true>(a, c, stream);
    case kQ5_0:
      return aligned ? launch_combine_t<kQ5_0, true>(a, c, stream)
                     : launch_combine_t<kQ5_0, false>(a, c, stream);
    case kQ8_0:
      return aligned ? launch_combine_t<kQ8_0, true>(a, c, stream)
                     : launch_combine_t<kQ8_0, false>(a, c, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t moe_gemm_launch(int type, int epi, const MoeGemmArgs& a, int mt, int max_chunks,
                           hipStream_t stream) {
  if (max_chunks <= 0 || a.N <= 0) return hipSuccess;
  if (mt == 4 || mt == 8) {
    const bool two = mt == 8;
    switch (epi) {
      case kEpiSwiglu:
        return two ? launch_group_epi<kEpiSwiglu, 2>(type, a, max_chunks, stream)
                   : launch_group_epi<kEpiSwiglu, 1>(type, a, max_chunks, stream);
      case kEpiRelu2:
        return two ? launch_group_epi<kEpiRelu2, 2>(type, a, max_chunks, stream)
                   : launch_group_epi<kEpiRelu2, 1>(type, a, max_chunks, stream);
      case kEpiDown:
        return two ? launch_group_epi<kEpiDown, 2>(type, a, max_chunks, stream)
                   : launch_group_epi<kEpiDown, 1>(type, a, max_chunks, stream);
      default: return hipErrorInvalidValue;
    }
  }
  switch (epi) {
    case kEpiSwiglu: return launch_gemm_epi<kEpiSwiglu>(type, a, mt, max_chunks, stream);
    case kEpiRelu2: return launch_gemm_epi<kEpiRelu2>(type, a, mt, max_chunks, stream);
    case kEpiDown: return launch_gemm_epi<kEpiDown>(type, a, mt, max_chunks, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace llhip
