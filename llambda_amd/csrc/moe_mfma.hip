// moe_mfma.hip -- the multi-token routed-MoE products on MFMA.
//
// Three kernels serve batches of two or more tokens:
//
//   split_rows_kernel   fp32 activation rows -> "split rows": every element
//                       as two bf16 (hi + lo, |x - hi - lo| <= 2^-17 |x|) plus
//                       the sums of each 16- and 32-element group of hi + lo.
//   router_mfma_kernel  the F32 router as a GEMM on v_mfma_f32_16x16x4_f32
//                       (fp32 products, fp32 accumulation).
//   moe_gemm_kernel     the grouped expert products over the chunk table
//                       (expert, up to 16*MT (token, rank) pairs): gate/up
//                       with silu(g)*u or relu(u)^2 fused, or down.
//
// Expert products.  The weights stay the tensor's GGUF super-blocks.  Each
// wavefront stages the raw bytes of its rows for one 256-element K chunk in
// LDS (global_load_lds_dwordx4 -- coalesced, no VGPR round trip), then every
// lane turns its 8 (or 4) codes of one scale group into exact bf16 values
// 128 + q (a v_perm_b32 with the filler byte 0x43) -- the B operand of a
// 16x16x32 (or, for Q6_K's 16-weight groups, 16x16x16) bf16 MFMA whose A
// operand is 16 tokens' hi, then lo, activations.  Per scale group g of row n
//     sum_k w_k x_k = delta_g * sum_k (128 + q_k) x_k  -  c_g * sum_k x_k
// with c_g = 128 delta_g + mu_g (Q4_K), 160 delta_g (Q6_K: q - 32),
// 144 delta_g (Q5_0: q - 16), 128 delta_g (Q8_0: codes q ^ 0x80).  The first
// term is one VALU fma per output per group (the MFMA result scaled by the
// row's delta); the second is itself a product over groups, done at the end
// of each chunk as a v_mfma_f32_16x16x4_f32 of the group sums (A) with -c (B).
// The reference forms every weight first (w = fl(fl(q delta) - mu)) and
// accumulates w x in fp32; both are fp32 evaluations of the same sum and
// differ by rounding, inside the bound 1e-4 sum|w x| per output.
#include "activations.h"
#include "mfma.h"
#include "moe.h"

#include <algorithm>

namespace llhip {

// ---------------------------------------------------------------- split rows
// Row r of K elements (K % 32 == 0):
//   q + r * q_stride (u16): for each 32-group j, [64j, 64j + 32) = hi bf16 of
//       elements 32j .. 32j + 31 and [64j + 32, 64j + 64) = their lo bf16.
//   s + r * s_stride (f32): [0, K/16) = sums of the 16-groups, then
//       [K/16, K/16 + K/32) = sums of the 32-groups, each of fl(hi) + fl(lo).
__global__ void __launch_bounds__(256) split_rows_kernel(const float* __restrict__ x, int rows,
                                                         int K, uint16_t* __restrict__ q,
                                                         int64_t q_stride, float* __restrict__ s,
                                                         int64_t s_stride) {
  const int octets = K >> 3;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  // octets is a multiple of 4 and so is the block size: the four octets of
  // a 32-group are all in range or all out, so the shuffles below stay
  // within active lanes
  if (gid >= (int64_t)rows * octets) return;
  const int row = (int)(gid / octets), o = (int)(gid - (int64_t)row * octets);
  const float4* xp = reinterpret_cast<const float4*>(x + (int64_t)row * K + 8 * o);
  const float4 a = xp[0], b = xp[1];
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t hi[8], lo[8];
  float sum = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float t;
    split_bf16(v[e], hi[e], lo[e], t);
    sum += t;
  }
  uint16_t* dst = q + (int64_t)row * q_stride + 64 * (o >> 2) + 8 * (o & 3);
  *reinterpret_cast<u32x4*>(dst) = u32x4{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16),
                                         hi[4] | (hi[5] << 16), hi[6] | (hi[7] << 16)};
  *reinterpret_cast<u32x4*>(dst + 32) = u32x4{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16),
                                              lo[4] | (lo[5] << 16), lo[6] | (lo[7] << 16)};
  const float s16 = sum + __shfl_xor(sum, 1, 64);
  const float s32 = s16 + __shfl_xor(s16, 2, 64);
  float* srow = s + (int64_t)row * s_stride;
  if ((o & 1) == 0) srow[o >> 1] = s16;
  if ((o & 3) == 0) srow[(K >> 4) + (o >> 2)] = s32;
}

hipError_t split_rows_launch(const float* x, int rows, int K, uint16_t* q, int64_t q_stride,
                             float* s, int64_t s_stride, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  const int64_t threads = (int64_t)rows * (K >> 3);
  const int grid = (int)((threads + 255) / 256);
  hipLaunchKernelGGL(split_rows_kernel, dim3(grid), dim3(256), 0, stream, x, rows, K, q, q_stride,
                     s, s_stride);
  return hipGetLastError();
}

// -------------------------------------------------------------------- router
// logits[t * ld + e] = sum_h x[t][h] R[e][h] (dot-product-with-f32-tensor-data,
// llambda.lisp:4096-4107, in another fp32 order).  A workgroup owns a 16 x 16
// (token, expert) tile; its four wavefronts take interleaved 16-element K
// slices and their partial tiles are added in wave order.
__global__ void __launch_bounds__(256) router_mfma_kernel(const float* __restrict__ x, int T,
                                                          const float* __restrict__ R, int Er,
                                                          int H, float* __restrict__ logits,
                                                          int ld) {
  __shared__ floatx4 red[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, kg = lane >> 4;
  const int t0 = blockIdx.y * 16, e0 = blockIdx.x * 16;
  const float* xr = x + (int64_t)min(t0 + i, T - 1) * H + 4 * kg;
  const float* rr = R + (int64_t)min(e0 + i, Er - 1) * H + 4 * kg;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int k = 16 * wave; k < H; k += 64) {
    const float4 xa = *reinterpret_cast<const float4*>(xr + k);
    const float4 rb = *reinterpret_cast<const float4*>(rr + k);
    acc = mfma4f32(xa.x, rb.x, acc);
    acc = mfma4f32(xa.y, rb.y, acc);
    acc = mfma4f32(xa.z, rb.z, acc);
    acc = mfma4f32(xa.w, rb.w, acc);
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  const floatx4 v = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
  const int e = e0 + i;
  if (e >= Er) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = t0 + 4 * kg + r;
    if (t < T) logits[(int64_t)t * ld + e] = v[r];
  }
}

hipError_t router_mfma_launch(const float* x, int T, const float* R, int Er, int H, float* logits,
                              int ld, hipStream_t stream) {
  const dim3 grid((Er + 15) / 16, (T + 15) / 16);
  hipLaunchKernelGGL(router_mfma_kernel, grid, dim3(256), 0, stream, x, T, R, Er, H, logits, ld);
  return hipGetLastError();
}

// ------------------------------------------------------ B operand per type
// step(): for lane (n, g), its codes of scale group j of the chunk as bf16
// 128 + q, the row's delta and offset c for that group.  `row` is the
// dword-aligned LDS image of the row's chunk; the chunk's first byte is at
// row + sh (sh < 4; 0 for Q4_K).

__device__ __forceinline__ uint32_t lds_dword(const uint8_t* row, int i) {
  return reinterpret_cast<const uint32_t*>(row)[i];
}
// Four bytes at byte offset o (o % 4 == 0) of a chunk that starts sh bytes
// past the dword-aligned row image.
__device__ __forceinline__ uint32_t lds_dword_at(const uint8_t* row, uint32_t sh, int o) {
  return __builtin_amdgcn_alignbyte(lds_dword(row, (o >> 2) + 1), lds_dword(row, o >> 2), sh);
}
// Four bytes at byte offset o (o even, o % 4 unknown) of the dword-aligned image.
__device__ __forceinline__ uint32_t lds_dword_even(const uint8_t* row, uint32_t o) {
  const uint32_t* q = reinterpret_cast<const uint32_t*>(row) + (o >> 2);
  return __builtin_amdgcn_alignbyte(q[1], q[0], o & 3u);
}
__device__ __forceinline__ uint32_t lds_u16_even(const uint8_t* row, uint32_t o) {
  return (reinterpret_cast<const uint32_t*>(row)[o >> 2] >> (8 * (o & 3u))) & 0xFFFFu;
}
__device__ __forceinline__ uint32_t lds_u8(const uint8_t* row, uint32_t o) {
  return (reinterpret_cast<const uint32_t*>(row)[o >> 2] >> (8 * (o & 3u))) & 0xFFu;
}

// Bits 0..3 of b to bit 4 of bytes 0..3.
__device__ __forceinline__ uint32_t spread4_bit4(uint32_t b) {
  return (((b & 0xFu) * 0x00204081u) & 0x01010101u) << 4;
}

template <int TYPE>
struct GemmB;

// Q4_K: chunk = one super-block (144 B), 8 groups (sub-blocks) of 32.  Lane
// g takes elements 8g .. 8g+7 of sub-block j: qs bytes 32 (j/2) + 8g .. +7,
// low nibbles for even j, high for odd (llambda.lisp:4145-4201, 6815-6859).
template <>
struct GemmB<kQ4_K> {
  static constexpr int kSpan = 144, kPitch = 144, kSteps = 8, kStepK = 32;
  static constexpr bool kWide = true;
  typedef bf16x8 Frag;
  static __device__ __forceinline__ void step(const uint8_t* row, uint32_t, int j, int g, Frag& b,
                                              float& delta, float& c) {
    const uint4 h = *reinterpret_cast<const uint4*>(row);
    const uint2 q = *reinterpret_cast<const uint2*>(row + 16 + 32 * (j >> 1) + 8 * g);
    const uint32_t c0 = (j & 1) ? (q.x >> 4) & 0x0F0F0F0Fu : q.x & 0x0F0F0F0Fu;
    const uint32_t c1 = (j & 1) ? (q.y >> 4) & 0x0F0F0F0Fu : q.y & 0x0F0F0F0Fu;
    b = codes_to_b(c0, c1);
    // get-scale-min-k4-at (llambda.lisp:4316-4336)
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
template <>
struct GemmB<kQ6_K> {
  static constexpr int kSpan = 210, kPitch = 224, kSteps = 16, kStepK = 16;
  static constexpr bool kWide = false;
  typedef shortx4 Frag;
  static __device__ __forceinline__ void step(const uint8_t* row, uint32_t sh, int u, int g,
                                              Frag& b, float& delta, float& c) {
    const int h = u >> 3, k = (u >> 1) & 3, s = u & 1;
    const uint32_t ql = lds_dword_at(row, sh, 64 * h + 32 * (k & 1) + 16 * s + 4 * g);
    const uint32_t qh = lds_dword_at(row, sh, 128 + 32 * h + 16 * s + 4 * g);
    const uint32_t nib = (ql >> (4 * (k >> 1))) & 0x0F0F0F0Fu;
    const uint32_t hb = ((qh >> (2 * k)) & 0x03030303u) << 4;
    b = codes4_to_b(nib | hb);
    const int sc = (int)(int8_t)lds_u8(row, sh + 192u + (uint32_t)u);
    const float d = half_bits_to_float(lds_u16_even(row, sh + 208u));
    delta = d * (float)sc;
    c = 160.f * delta;
  }
};

// Q5_0: chunk = 8 blocks of 22 B (llambda.lisp:3965-3990, 4037-4066).
// Lane g takes elements 8g .. 8g+7: qs bytes 8 (g & 1) .. +7, low nibbles
// for g < 2, high for g >= 2, fifth bits from qh bits 8g .. 8g+7.
template <>
struct GemmB<kQ5_0> {
  static constexpr int kSpan = 176, kPitch = 192, kSteps = 8, kStepK = 32;
  static constexpr bool kWide = true;
  typedef bf16x8 Frag;
  static __device__ __forceinline__ void step(const uint8_t* row, uint32_t sh, int j, int g,
                                              Frag& b, float& delta, float& c) {
    const uint32_t o = sh + 22u * (uint32_t)j;
    const uint32_t os = o + 6u + 8u * (uint32_t)(g & 1);
    uint32_t q0 = lds_dword_even(row, os), q1 = lds_dword_even(row, os + 4u);
    if (g >= 2) {
      q0 >>= 4;
      q1 >>= 4;
    }
    const uint32_t hb = lds_u8(row, o + 2u + (uint32_t)g);
    const uint32_t c0 = (q0 & 0x0F0F0F0Fu) | spread4_bit4(hb);
    const uint32_t c1 = (q1 & 0x0F0F0F0Fu) | spread4_bit4(hb >> 4);
    b = codes_to_b(c0, c1);
    delta = half_bits_to_float(lds_u16_even(row, o));
    c = 144.f * delta;
  }
};

// Q8_0: chunk = 8 blocks of 34 B (llambda.lisp:3992-4009, 4068-4094).  The
// code u = q ^ 0x80 = q + 128 (0..255) is exact in bf16 (8 significant bits).
template <>
struct GemmB<kQ8_0> {
  static constexpr int kSpan = 272, kPitch = 288, kSteps = 8, kStepK = 32;
  static constexpr bool kWide = true;
  typedef bf16x8 Frag;
  static __device__ __forceinline__ uint32_t pack2(uint32_t u, int k) {
    const float f0 = (float)((u >> (8 * k)) & 0xFFu), f1 = (float)((u >> (8 * k + 8)) & 0xFFu);
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f1), __builtin_bit_cast(uint32_t, f0),
                                 0x07060302u);
  }
  static __device__ __forceinline__ void step(const uint8_t* row, uint32_t sh, int j, int g,
                                              Frag& b, float& delta, float& c) {
    const uint32_t o = sh + 34u * (uint32_t)j;
    const uint32_t os = o + 2u + 8u * (uint32_t)g;
    const uint32_t u0 = lds_dword_even(row, os) ^ 0x80808080u;
    const uint32_t u1 = lds_dword_even(row, os + 4u) ^ 0x80808080u;
    u32x4 v = {pack2(u0, 0), pack2(u0, 2), pack2(u1, 0), pack2(u1, 2)};
    b = __builtin_bit_cast(bf16x8, v);
    delta = half_bits_to_float(lds_u16_even(row, o));
    c = 128.f * delta;
  }
};

// A fragments of lane (t, g) for group j of the chunk starting at element
// 256 kc: hi then lo (8 bf16 each for 32-groups, 4 for 16-groups).
template <bool WIDE>
struct AFrag;
template <>
struct AFrag<true> {
  bf16x8 hi, lo;
  __device__ __forceinline__ void load(const uint16_t* row, int kc, int j, int g) {
    const uint16_t* p = row + 512 * kc + 64 * j + 8 * g;
    hi = *reinterpret_cast<const bf16x8*>(p);
    lo = *reinterpret_cast<const bf16x8*>(p + 32);
  }
};
template <>
struct AFrag<false> {
  shortx4 hi, lo;
  __device__ __forceinline__ void load(const uint16_t* row, int kc, int u, int g) {
    const uint16_t* p = row + 512 * kc + 64 * (u >> 1) + 16 * (u & 1) + 4 * g;
    hi = *reinterpret_cast<const shortx4*>(p);
    lo = *reinterpret_cast<const shortx4*>(p + 32);
  }
};

__device__ __forceinline__ floatx4 mfma_b(const bf16x8& a, const bf16x8& b, const floatx4& c) {
  return mfma32(a, b, c);
}
__device__ __forceinline__ floatx4 mfma_b(const shortx4& a, const shortx4& b, const floatx4& c) {
  return mfma16(a, b, c);
}

// ------------------------------------------------------------ grouped GEMM
constexpr int kGemmWaves = 4;

template <int EPI>
struct EpiShape {
  static constexpr int kMats = EPI == kEpiSwiglu ? 2 : 1;  // gate and up rows side by side
  static constexpr int kSub = EPI == kEpiSwiglu ? 2 : 4;   // 16-row subtiles per matrix
};

template <int TYPE, int EPI>
constexpr int gemm_lds_bytes() {
  using B = GemmB<TYPE>;
  using S = EpiShape<EPI>;
  constexpr int pieces = 16 * S::kSub * B::kPitch / 16;
  return kGemmWaves * S::kMats * 1024 * ((pieces + 63) / 64);
}

template <int TYPE, int EPI, int MT>
__global__ void __launch_bounds__(64 * kGemmWaves) moe_gemm_kernel(MoeGemmArgs a) {
  using B = GemmB<TYPE>;
  using S = EpiShape<EPI>;
  constexpr int NB = S::kMats, NS = S::kSub, ROWS = 16 * NS;
  constexpr int PPR = B::kPitch / 16;  // 16-byte pieces per row
  constexpr int PIECES = ROWS * PPR;
  constexpr int LOADS = (PIECES + 63) / 64;
  constexpr int BUF = 1024 * LOADS;
  constexpr int NQ = B::kSteps / 4;  // offset MFMAs per chunk
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  const int nchunks = a.chunk_counts[a.group];
  if ((int)blockIdx.x >= nchunks) return;
  const MoeChunk ch = a.chunks[(a.group ? a.chunk_counts[0] : 0) + blockIdx.x];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int n0 = (blockIdx.y * kGemmWaves + wave) * ROWS;
  if (n0 >= a.N) return;

  // A rows of this lane's token (tile row t = n) in each token tile
  const uint16_t* arow[MT];
  const float* srow[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int tk = 16 * i + n;
    const int q = a.perm[ch.start + (tk < ch.count ? tk : 0)];
    const int64_t r = a.a_by_token ? (q < a.pairs ? q / a.top_k : q - a.pairs) : q;
    arow[i] = a.aq + r * a.aq_stride;
    srow[i] = a.as + r * a.as_stride + (B::kStepK == 32 ? a.as32_off : 0);
  }
  const uint8_t* base[NB];
  base[0] = uniform_ptr(a.w0 + (int64_t)ch.expert * a.expert_stride);
  if constexpr (NB == 2) base[NB - 1] = uniform_ptr(a.w1 + (int64_t)ch.expert * a.expert_stride);
  uint8_t* buf = lds + wave * NB * BUF;
  const uint32_t buf_lds = lds_address(buf);
  const uint32_t rb = (uint32_t)a.row_bytes;

  // this lane's DMA pieces: (row, piece) per load instruction
  uint32_t prow[LOADS], ppc[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int idx = min(64 * i + lane, PIECES - 1);
    const int r = idx / PPR;
    prow[i] = (uint32_t)min(n0 + r, a.N - 1) * rb;
    ppc[i] = 16u * (uint32_t)(idx - r * PPR);
  }
  // this lane's B rows (one per subtile)
  uint32_t brow[NS];
#pragma unroll
  for (int m = 0; m < NS; ++m) brow[m] = (uint32_t)min(n0 + 16 * m + n, a.N - 1) * rb;

  floatx4 tot[MT][NS][NB];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int m = 0; m < NS; ++m)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) tot[i][m][nb] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int groups = a.K / B::kStepK;  // scale groups along K
  const int nchunk = (a.K + 255) >> 8;
  for (int kc = 0; kc < nchunk; ++kc) {
    const uint32_t koff = (uint32_t)kc * (uint32_t)B::kSpan;
    // stage the wave's rows of this chunk
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < LOADS; ++i)
        load_lds16(base[nb], ((prow[i] + koff) & ~3u) + ppc[i],
                   buf_lds + (uint32_t)(nb * BUF + 1024 * i));
    wait_loads<0>();

    const int gbase = kc * B::kSteps;  // first scale group of the chunk
    float cq[NS][NB][NQ];
#pragma unroll
    for (int m = 0; m < NS; ++m)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int q = 0; q < NQ; ++q) cq[m][nb][q] = 0.f;

#pragma unroll
    for (int j = 0; j < B::kSteps; ++j) {
      if (gbase + j < groups) {
        AFrag<B::kWide> af[MT];
#pragma unroll
        for (int i = 0; i < MT; ++i) af[i].load(arow[i], kc, j, g);
#pragma unroll
        for (int m = 0; m < NS; ++m) {
          const uint32_t sh = (brow[m] + koff) & 3u;
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            typename B::Frag bf;
            float delta, c;
            B::step(buf + nb * BUF + (16 * m + n) * B::kPitch, sh, j, g, bf, delta, c);
            if ((j & 3) == g) cq[m][nb][j >> 2] = -c;
#pragma unroll
            for (int i = 0; i < MT; ++i) {
              floatx4 d = mfma_b(af[i].hi, bf, floatx4{0.f, 0.f, 0.f, 0.f});
              d = mfma_b(af[i].lo, bf, d);
              floatx4& t = tot[i][m][nb];
              t[0] = fmaf(delta, d[0], t[0]);
              t[1] = fmaf(delta, d[1], t[1]);
              t[2] = fmaf(delta, d[2], t[2]);
              t[3] = fmaf(delta, d[3], t[3]);
            }
          }
        }
      }
    }
    // offsets: sum over the chunk's groups of (-c) x (group sum), 4 groups
    // per MFMA (K slice g = lane >> 4 is group 4q + g)
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int gi = min(gbase + 4 * q + g, groups - 1);
        const float sv = srow[i][gi];
#pragma unroll
        for (int m = 0; m < NS; ++m)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) tot[i][m][nb] = mfma4f32(sv, cq[m][nb][q], tot[i][m][nb]);
      }
    }
    // every LDS read of this chunk has returned before the next DMA writes
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }

  // ---------------------------------------------------------- epilogue
  // lane (n, G) holds tokens 16 i + 4 G + r of row n0 + 16 m + n
#pragma unroll
  for (int i = 0; i < MT; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tk = 16 * i + 4 * g + r;
      const bool tok_ok = tk < ch.count;
      const int q = tok_ok ? a.perm[ch.start + tk] : 0;
      if constexpr (EPI == kEpiDown) {
#pragma unroll
        for (int m = 0; m < NS; ++m) {
          const int row = n0 + 16 * m + n;
          if (tok_ok && row < a.N) a.out[(int64_t)q * a.out_stride + row] = tot[i][m][0][r];
        }
      } else {
        uint16_t* oq = a.oq + (int64_t)q * a.oq_stride;
        float* os = a.os + (int64_t)q * a.os_stride;
        float s16[NS];
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
          const bool ok = tok_ok && row < a.N;
          if (ok) {
            uint16_t* p = oq + 64 * (row >> 5) + (row & 31);
            p[0] = (uint16_t)hb;
            p[32] = (uint16_t)lb;
          }
          s16[m] = group_sum(ok ? sum : 0.f, 4);
        }
        if (n == 0 && tok_ok) {
#pragma unroll
          for (int m = 0; m < NS; ++m) {
            const int row = n0 + 16 * m;
            if (row < a.N) {
              os[row >> 4] = s16[m];
              if ((m & 1) == 0) os[a.os32_off + (row >> 5)] = s16[m] + s16[m + 1];
            }
          }
        }
      }
    }
  }
}

// ------------------------------------------------------------------ host

template <int TYPE, int EPI, int MT>
static hipError_t launch_gemm_t(const MoeGemmArgs& a, int max_chunks, hipStream_t stream) {
  constexpr int lds = gemm_lds_bytes<TYPE, EPI>();
  const auto kernel = moe_gemm_kernel<TYPE, EPI, MT>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
  }
  constexpr int rows_per_block = kGemmWaves * 16 * EpiShape<EPI>::kSub;
  const dim3 grid(max_chunks, (a.N + rows_per_block - 1) / rows_per_block);
  hipLaunchKernelGGL(kernel, grid, dim3(64 * kGemmWaves), lds, stream, a);
  return hipGetLastError();
}

template <int TYPE, int EPI>
static hipError_t launch_gemm_mt(const MoeGemmArgs& a, int mt, int max_chunks, hipStream_t s) {
  switch (mt) {
    case 1: return launch_gemm_t<TYPE, EPI, 1>(a, max_chunks, s);
    case 2: return launch_gemm_t<TYPE, EPI, 2>(a, max_chunks, s);
    case 4: return launch_gemm_t<TYPE, EPI, 4>(a, max_chunks, s);
    default: return hipErrorInvalidValue;
  }
}

template <int EPI>
static hipError_t launch_gemm_epi(int type, const MoeGemmArgs& a, int mt, int max_chunks,
                                  hipStream_t s) {
  switch (type) {
    case kQ4_K: return launch_gemm_mt<kQ4_K, EPI>(a, mt, max_chunks, s);
    case kQ6_K: return launch_gemm_mt<kQ6_K, EPI>(a, mt, max_chunks, s);
    case kQ5_0: return launch_gemm_mt<kQ5_0, EPI>(a, mt, max_chunks, s);
    case kQ8_0: return launch_gemm_mt<kQ8_0, EPI>(a, mt, max_chunks, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t moe_gemm_launch(int type, int epi, const MoeGemmArgs& a, int mt, int max_chunks,
                           hipStream_t stream) {
  if (max_chunks <= 0 || a.N <= 0) return hipSuccess;
  switch (epi) {
    case kEpiSwiglu: return launch_gemm_epi<kEpiSwiglu>(type, a, mt, max_chunks, stream);
    case kEpiRelu2: return launch_gemm_epi<kEpiRelu2>(type, a, mt, max_chunks, stream);
    case kEpiDown: return launch_gemm_epi<kEpiDown>(type, a, mt, max_chunks, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace llhip
