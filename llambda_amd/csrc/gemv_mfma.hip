// gemv_mfma.hip -- batch-1 Q4_K / Q6_K GEMV with the unpacked codes fed to
// MFMA (v_mfma_f32_16x16x32_bf16), so the VALU only unpacks bits.
//
// One wavefront computes 16 rows of W (the MFMA's 16 B-columns) over all of
// K.  For every super-block:
//   B operand  lane (n, g) = (lane & 15, lane >> 4) holds 8 codes of row n as
//              bf16 (128 + q): the code byte and a 0x43 filler byte are
//              interleaved by one v_perm_b32, 0x43qq being exactly 128 + q.
//   A operand  the activations, split x = x_hi + x_lo into two bf16 (each
//              within 2^-9 of its remainder, so |x - x_hi - x_lo| <= 2^-18 |x|),
//              arranged so that A row a carries scale group "slot" a >> 1 (hi
//              for even a, lo for odd a) and zeros elsewhere.  Lanes whose A
//              row has no data in an MFMA read a zero line.  The table is built
//              once per workgroup in LDS.
//   D          lane (n, G) then holds, for row n, the (hi, lo) sums of slots
//              2G and 2G+1; it applies those groups' scale and offset once:
//                sum_i (q_i - c) x_i = (D_hi + D_lo) - (128 + c) * sum_i x~_i
//              with c the code offset (Q4_K: min/delta handled through dmin,
//              Q6_K: 32) and sum x~ precomputed per group.
//   Q4_K       slots = the 8 sub-blocks; 8 MFMAs per block, MFMA m takes
//              elements 4m..4m+3 of sub-blocks 2g (low nibbles) and 2g+1
//              (high nibbles) from lane g's 32 qs bytes [32g, 32g+32).
//   Q6_K       per half h, slots = the 8 scale groups (k, half) of
//              llambda.lisp:4203-4310; 4 MFMAs per half, MFMA m takes q_m of
//              l = 8g .. 8g+7 from lane g's ql/qh bytes.
// The row sums of the four G lanes meet by two cross-lane adds.
#include "activations.h"
#include "gemv.h"
#include "mfma.h"

#include <algorithm>
#include <type_traits>
#include <utility>

namespace llhip {

// Sum over the four lanes n, n+16, n+32, n+48.
__device__ __forceinline__ float sum_lane_groups(float v) {
  return half_pair_sum(row_pair_sum(v));
}

// ------------------------------------------------------------ row staging
// A wavefront streams its 16-row tile through LDS in chunks of C blocks per
// row.  Piece j (16 bytes) of row r of the chunk is load lane (r * kPitch +
// j): global_load_lds_dwordx4 writes lane i's 16 bytes to M0 + 16 i, so the
// LDS image of a chunk is the rows' byte ranges kRow bytes apart, with no
// VGPR staging.  kPitch is kPieces rounded up to an odd count (the pad piece
// repeats the row's last piece), so the 16 rows' reads of one offset fall in
// 16 different bank quads.  Each row's range starts at the dword at or
// below the chunk's first byte (row starts need only be 2-byte aligned) and
// may run up to 18 bytes past the chunk (the allocation's pad covers the last
// row).  Two buffers per wave: the next chunk loads while this one computes.
template <int BB, int C, bool ALIGNED>
struct Chunk {
  static constexpr int kSpan = C * BB;
  static constexpr int kPieces = (kSpan + (ALIGNED ? 0 : 3) + 15) / 16;
  static constexpr int kPitch = kPieces | 1;
  static constexpr int kRow = 16 * kPitch;
  static constexpr int kLoads = (16 * kPitch + 63) / 64;
  static constexpr int kBuffer = 1024 * kLoads;  // per buffer; lanes past 16 rows write slack
};

// ------------------------------------------------------------------ Q4_K
// LDS table per block: 8 MFMAs x 16 A rows x 16 B (only lane g = a >> 2
// reads its row's entry; others read the zero line), then 8 group sums.
constexpr int kQ4Table = 8 * 16 * 16;  // bytes per block
constexpr int kQ6Table = 2 * 4 * 8 * 16;

// Zero lines (LDS [0, 2 KB) is zero) for A lanes without data, in a bank
// quad (16-byte slot modulo 256 bytes) that no data lane served in the same
// cycle reads: a 16-byte read serves the lanes of octets 0 and 3, then 1 and
// 2, of each half wave (measured with the LDS bank-conflict counter).  Q4_K:
// the data lanes of lane group g read slots 4g .. 4g+3 of each 256-byte MFMA
// row (the table and its blocks are 256-byte aligned), so groups 0 and 1 read
// their zero line in slot 8, groups 2 and 3 in slot 0; Q6_K: the data lanes
// of MFMA m of half h read slots 8m .. 8m+7 (modulo 16) at h * 512 + m * 128,
// the zero lanes 128 bytes further.
__device__ __forceinline__ uint32_t zero_line_q4(int g) { return g < 2 ? 128u : 0u; }
constexpr uint32_t kZeroLineQ6 = 128;

// Table items: Q4_K item i = (block, sub-block s, 4-element step m); Q6_K
// item i = (block, half, k, l-octet): 8 activations.  first(i) is the item's
// first element; emit() writes the split values of its elements and, with
// the lanes sharing its scale group, the group's sum.
struct Q4Items {
  static constexpr int kEl = 4, kPerBlock = 64;
  __device__ static int first(int i) {
    const int b = i >> 6, s = (i >> 3) & 7, m = i & 7;
    return b * 256 + 32 * s + 4 * m;
  }
  __device__ static void emit(uint8_t* table, float* gsum, int i, const float* v) {
    const int b = i >> 6, s = (i >> 3) & 7, m = i & 7;
    uint32_t hi[2], lo[2];
    float sum[4];
    split_bf16_pair(v[0], v[1], hi[0], lo[0], sum[0], sum[1]);
    split_bf16_pair(v[2], v[3], hi[1], lo[1], sum[2], sum[3]);
    float part = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) part += sum[e];
    // rows a = 2s (hi) and 2s+1 (lo); the data sits in half (s & 1) of the 8 slots
    const int half = s & 1;
    u32x4 vh = {0u, 0u, 0u, 0u}, vl = {0u, 0u, 0u, 0u};
    vh[2 * half] = hi[0];
    vh[2 * half + 1] = hi[1];
    vl[2 * half] = lo[0];
    vl[2 * half + 1] = lo[1];
    uint8_t* base = table + b * kQ4Table + m * 256;
    *reinterpret_cast<u32x4*>(base + (2 * s) * 16) = vh;
    *reinterpret_cast<u32x4*>(base + (2 * s + 1) * 16) = vl;
    // group sum over the sub-block's 32 elements: 8 threads m = 0..7 share it
    part = group_sum(part, 3);
    if (m == 0) gsum[b * 8 + s] = part;
  }
};

// The bytes of one Q4_K block that lane (n, g) uses: the 16-byte header and
// its 32 qs bytes, read from the block's 144 bytes in LDS (16-byte aligned).
struct Q4Raw {
  uint4 h, c0, c1;
};
__device__ __forceinline__ Q4Raw q4k_fetch(const uint8_t* p, int g) {
  return {*reinterpret_cast<const uint4*>(p), *reinterpret_cast<const uint4*>(p + 16 + 32 * g),
          *reinterpret_cast<const uint4*>(p + 32 + 32 * g)};
}

// One Q4_K block of lane (n, g)'s row from its fetched bytes; a = the lane's
// A address for this block (a zero line when its A row carries no data).
__device__ __forceinline__ float q4k_block(const Q4Raw& r, const uint8_t* lds, uint32_t a,
                                           const float* gs, int g) {
  const uint4 h = r.h, c0 = r.c0, c1 = r.c1;
  const uint32_t qw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  floatx4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const bf16x8 av = *reinterpret_cast<const bf16x8*>(lds + a + m * 256);
    const uint32_t lo = opaque(qw[m] & 0x0F0F0F0Fu);
    const uint32_t hi = opaque((qw[m] >> 4) & 0x0F0F0F0Fu);
    d = mfma32(av, codes_to_b(lo, hi), d);
  }
  // sub-blocks 2g (D rows 4g, 4g+1) and 2g+1 (4g+2, 4g+3); scale and min per
  // get-scale-min-k4-at (llambda.lisp:4316-4336)
  const int bsel = (2 * g) & 3;
  const bool high = g >= 2;
  const uint32_t B0a = (h.y >> (8 * bsel)) & 0xFFu, B0b = (h.y >> (8 * bsel + 8)) & 0xFFu;
  const uint32_t B4a = (h.z >> (8 * bsel)) & 0xFFu, B4b = (h.z >> (8 * bsel + 8)) & 0xFFu;
  const uint32_t B8a = (h.w >> (8 * bsel)) & 0xFFu, B8b = (h.w >> (8 * bsel + 8)) & 0xFFu;
  const uint32_t sc0 = high ? ((B8a & 15u) | ((B0a >> 6) << 4)) : (B0a & 63u);
  const uint32_t m0 = high ? ((B8a >> 4) | ((B4a >> 6) << 4)) : (B4a & 63u);
  const uint32_t sc1 = high ? ((B8b & 15u) | ((B0b >> 6) << 4)) : (B0b & 63u);
  const uint32_t m1 = high ? ((B8b >> 4) | ((B4b >> 6) << 4)) : (B4b & 63u);
  const float dd = half_bits_to_float(h.x & 0xFFFFu);
  const float dm = half_bits_to_float(h.x >> 16);
  const float delta0 = dd * (float)sc0, delta1 = dd * (float)sc1;
  const float off0 = fmaf(128.f, delta0, dm * (float)m0);
  const float off1 = fmaf(128.f, delta1, dm * (float)m1);
  const float2 gsv = *reinterpret_cast<const float2*>(gs + 2 * g);
  float v = delta0 * (d[0] + d[1]);
  v = fmaf(-off0, gsv.x, v);
  v = fmaf(delta1, d[2] + d[3], v);
  v = fmaf(-off1, gsv.y, v);
  return v;
}

// ------------------------------------------------------------------ Q6_K
// LDS table per block: 2 halves x 4 MFMAs x 8 entries x 16 B, then 16 group
// sums.  Entry (a & 3) * 2 + (g & 1) of MFMA m serves A row a = 4m + (a & 3)
// for lane g when (a >> 1) & 1 == g >> 1.
struct Q6Items {
  static constexpr int kEl = 8, kPerBlock = 32;
  __device__ static int first(int i) {
    const int b = i >> 5, h = (i >> 4) & 1, k = (i >> 2) & 3, g = i & 3;
    return b * 256 + 128 * h + 32 * k + 8 * g;
  }
  __device__ static void emit(uint8_t* table, float* gsum, int i, const float* v) {
    const int b = i >> 5, h = (i >> 4) & 1, k = (i >> 2) & 3, g = i & 3;
    uint32_t hi[4], lo[4];
    float sum[8];
#pragma unroll
    for (int e = 0; e < 8; e += 2)
      split_bf16_pair(v[e], v[e + 1], hi[e / 2], lo[e / 2], sum[e], sum[e + 1]);
    float part = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) part += sum[e];
    // slot = 2k + (g >> 1): A rows 4k + 2(g >> 1) (hi) and +1 (lo)
    const int ahi = 2 * (g >> 1);
    uint8_t* base = table + b * kQ6Table + (h * 4 + k) * 128;
    const u32x4 vh = {hi[0], hi[1], hi[2], hi[3]};
    const u32x4 vl = {lo[0], lo[1], lo[2], lo[3]};
    *reinterpret_cast<u32x4*>(base + (ahi * 2 + (g & 1)) * 16) = vh;
    *reinterpret_cast<u32x4*>(base + ((ahi + 1) * 2 + (g & 1)) * 16) = vl;
    // group (h, k, half = g >> 1) sums 16 elements: threads g, g ^ 1
    part = group_sum(part, 1);
    if ((g & 1) == 0) gsum[b * 16 + h * 8 + 2 * k + (g >> 1)] = part;
  }
};

// 8 bytes at byte offset o of the dword-aligned q (the block starts SH bytes
// past q).
template <int SH>
__device__ __forceinline__ uint2 read8(const uint32_t* q, int o) {
  if constexpr (SH == 0) {
    return make_uint2(q[o / 4], q[o / 4 + 1]);
  } else {
    const uint32_t r0 = q[o / 4], r1 = q[o / 4 + 1], r2 = q[o / 4 + 2];
    return make_uint2(__builtin_amdgcn_alignbyte(r1, r0, SH), __builtin_amdgcn_alignbyte(r2, r1, SH));
  }
}
__device__ __forceinline__ uint2 read8(const uint32_t* q, int o, uint32_t sh) {
  const uint32_t r0 = q[o / 4], r1 = q[o / 4 + 1], r2 = q[o / 4 + 2];
  return make_uint2(__builtin_amdgcn_alignbyte(r1, r0, sh), __builtin_amdgcn_alignbyte(r2, r1, sh));
}

// The bytes of one Q6_K block that lane (n, g) uses, read from the block's
// 210 bytes p in LDS (2-byte aligned; SH = p & 3 when known at compile time,
// -1: read it from p): per half its 8 ql bytes of each 32-lane run, its 8 qh
// bytes and its two scales, and the block's d.
struct Q6Raw {
  uint2 la[2], lb[2], qh[2];
  uint32_t sv[2];
  uint32_t d;
};
template <int SH>
__device__ __forceinline__ Q6Raw q6k_fetch(const uint8_t* p, int g) {
  const uint32_t sh = SH >= 0 ? (uint32_t)SH : (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3u);
  const uint32_t* q = reinterpret_cast<const uint32_t*>(p - sh);
  Q6Raw r;
  r.d = *reinterpret_cast<const uint16_t*>(p + 208);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if constexpr (SH >= 0) {
      r.la[h] = read8<SH>(q, 64 * h + 8 * g);
      r.lb[h] = read8<SH>(q, 64 * h + 32 + 8 * g);
      r.qh[h] = read8<SH>(q, 128 + 32 * h + 8 * g);
    } else {
      r.la[h] = read8(q, 64 * h + 8 * g + 0, sh);
      r.lb[h] = read8(q, 64 * h + 32 + 8 * g, sh);
      r.qh[h] = read8(q, 128 + 32 * h + 8 * g, sh);
    }
    r.sv[h] = *reinterpret_cast<const uint16_t*>(p + 192 + 8 * h + 2 * g);
  }
  return r;
}

// One Q6_K block of lane (n, g)'s row from its fetched bytes.  am[m] = the
// lane's A address for MFMA m of the block (kZeroLineQ6: zero line).
__device__ __forceinline__ float q6k_block(const Q6Raw& r, const uint8_t* lds, const uint32_t am[4],
                                           const float* gs, int g) {
  const float dd = half_bits_to_float(r.d);
  float v = 0.f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint2 la = r.la[h], lb = r.lb[h], qh = r.qh[h];
    floatx4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint2 l = (m & 1) ? lb : la;
      const uint32_t l0 = (m & 2) ? (l.x >> 4) : l.x;
      const uint32_t l1 = (m & 2) ? (l.y >> 4) : l.y;
      const uint32_t h0 = (qh.x >> (2 * m)) & 0x03030303u;
      const uint32_t h1 = (qh.y >> (2 * m)) & 0x03030303u;
      const uint32_t c0 = opaque((l0 & 0x0F0F0F0Fu) | (h0 << 4));
      const uint32_t c1 = opaque((l1 & 0x0F0F0F0Fu) | (h1 << 4));
      const bf16x8 av = *reinterpret_cast<const bf16x8*>(lds + am[m] + h * 512 + m * 128);
      d = mfma32(av, codes_to_b(c0, c1), d);
    }
    // D rows 4g .. 4g+3 of column n: groups (k = g, l-half 0 / 1) of half h,
    // i.e. scales sc[8h + 2g] and sc[8h + 2g + 1] (llambda.lisp:4203-4310)
    const uint32_t sv = r.sv[h];
    const float delta0 = dd * (float)(int)(int8_t)(sv & 0xFFu);
    const float delta1 = dd * (float)(int)(int8_t)(sv >> 8);
    const float2 gsv = *reinterpret_cast<const float2*>(gs + h * 8 + 2 * g);
    v = fmaf(delta0, fmaf(-160.f, gsv.x, d[0] + d[1]), v);
    v = fmaf(delta1, fmaf(-160.f, gsv.y, d[2] + d[3]), v);
  }
  return v;
}

// ------------------------------------------------------------- fusion
// 1 / sqrt(mean(x^2) + eps) over K elements (rms-norm-into,
// llambda.lisp:859-879; the sum of squares runs in another order than
// sum-square-elements' serial loop).  red: kMfmaWaves floats of LDS.
template <int WAVES>
__device__ float rms_scale(const float* __restrict__ x, int K, float eps, float* red) {
  float acc = 0.f;
  for (int i = threadIdx.x; i < K; i += 64 * WAVES) acc += x[i] * x[i];
  acc = wave_total(acc);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  float sum = red[0];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) sum += red[w];
  __syncthreads();
  const float mean = sum / (float)K;
  return 1.f / sqrtf(mean + eps);
}

// One batch of the activation table: the thread's items base + threadIdx.x
// + j * T (j < kMaxI) with their elements v (and, with a fused rms-norm-into,
// norm weights wv) loaded.  A table of one batch takes the rms scale from
// the loaded elements (sum of squares over the workgroup); then x (or
// (x * w) * scale, rounded as the reference rounds) is split into the table.
template <typename IT, int WAVES>
__device__ __forceinline__ void table_batch(float (&v)[16 / IT::kEl][IT::kEl],
                                            const float (&wv)[16 / IT::kEl][IT::kEl], int base,
                                            int items, bool one_batch, float& nscale,
                                            const float* __restrict__ nw, int nblk, float eps,
                                            float* red, uint8_t* table, float* gsum) {
  constexpr int T = 64 * WAVES, EL = IT::kEl, kMaxI = 16 / EL;
  if (nw && one_batch) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < kMaxI; ++j)
      if (base + threadIdx.x + j * T < items)
#pragma unroll
        for (int e = 0; e < EL; ++e) acc += v[j][e] * v[j][e];
    acc = wave_total(acc);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    float sum = red[0];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) sum += red[w];
    __syncthreads();
    nscale = 1.f / sqrtf(sum / (float)(nblk * 256) + eps);
  }
#pragma unroll
  for (int j = 0; j < kMaxI; ++j) {
    const int i = base + threadIdx.x + j * T;
    if (i < items) {
      if (nw) {
#pragma unroll
        for (int e = 0; e < EL; ++e) v[j][e] = (v[j][e] * wv[j][e]) * nscale;
      }
      IT::emit(table, gsum, i, v[j]);
    }
  }
}

// The activation table of one workgroup: every thread loads the elements of
// its items (up to kMaxI items, 16 floats, at once: one memory latency),
// with a fused rms-norm-into (llambda.lisp:859-879) also their norm weights
// and the sum of squares; then splits x into the table.  x is 16-byte
// aligned.  red: kMfmaWaves floats of LDS.
template <typename IT, int WAVES>
__device__ void build_table(uint8_t* table, float* gsum, const float* __restrict__ x, int nblk,
                            const float* __restrict__ nw, float eps, float* red) {
  constexpr int T = 64 * WAVES, EL = IT::kEl, kMaxI = 16 / EL;
  const int items = nblk * IT::kPerBlock;
  const bool one_batch = items <= T * kMaxI;
  float nscale = 1.f;
  if (nw && !one_batch) nscale = rms_scale<WAVES>(x, nblk * 256, eps, red);
  for (int base = 0; base < items; base += T * kMaxI) {
    float v[kMaxI][EL], wv[kMaxI][EL];
#pragma unroll
    for (int j = 0; j < kMaxI; ++j) {
      const int i = base + threadIdx.x + j * T;
      const int x0 = IT::first(min(i, items - 1));
#pragma unroll
      for (int e = 0; e < EL; e += 4) {
        const float4 a = *reinterpret_cast<const float4*>(x + x0 + e);
        v[j][e] = a.x; v[j][e + 1] = a.y; v[j][e + 2] = a.z; v[j][e + 3] = a.w;
        if (nw) {
          const float4 c = *reinterpret_cast<const float4*>(nw + x0 + e);
          wv[j][e] = c.x; wv[j][e + 1] = c.y; wv[j][e + 2] = c.z; wv[j][e + 3] = c.w;
        }
      }
    }
    table_batch<IT, WAVES>(v, wv, base, items, one_batch, nscale, nw, nblk, eps, red, table, gsum);
  }
}

// true when the table of nblk blocks is one batch of per-thread items
template <typename IT, int WAVES>
__host__ __device__ constexpr bool table_one_batch(int nblk) {
  return nblk * IT::kPerBlock <= 64 * WAVES * (16 / IT::kEl);
}

// The loads of a one-batch table and of a wave's first stage in one asm
// statement: the thread's four 16-byte x loads and four norm-weight loads
// (x again without a norm), then the stage's NL DMAs (lane i of load k:
// 16 bytes from wb + wo[k] to LDS dst + 1024 k + 16 i), then a wait until
// only the DMAs are in flight (vector loads complete in issue order).  The
// x registers are outputs of the statement, defined only after its wait, so
// no instruction can read them while their loads are in flight; the table
// is then built while the stage streams in.
#define LLHIP_PRO_DMA(k, imm) \
  "s_add_u32 m0, %[dst], " #imm "\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %[w" #k "], %[wb]\n\t"
#define LLHIP_PRO_DMA1 LLHIP_PRO_DMA(0, 0)
#define LLHIP_PRO_DMA2 LLHIP_PRO_DMA1 LLHIP_PRO_DMA(1, 0x400)
#define LLHIP_PRO_DMA3 LLHIP_PRO_DMA2 LLHIP_PRO_DMA(2, 0x800)
#define LLHIP_PRO_DMA4 LLHIP_PRO_DMA3 LLHIP_PRO_DMA(3, 0xc00)
#define LLHIP_PRO_DMA5 LLHIP_PRO_DMA4 LLHIP_PRO_DMA(4, 0x1000)
#define LLHIP_PRO_DMA6 LLHIP_PRO_DMA5 LLHIP_PRO_DMA(5, 0x1400)
#define LLHIP_PRO_DMA7 LLHIP_PRO_DMA6 LLHIP_PRO_DMA(6, 0x1800)
#define LLHIP_PRO_ASM(NL)                                                                   \
  asm volatile("global_load_dwordx4 %[v0], %[o0], %[xb]\n\t"                                \
               "global_load_dwordx4 %[v1], %[o1], %[xb]\n\t"                                \
               "global_load_dwordx4 %[v2], %[o2], %[xb]\n\t"                                \
               "global_load_dwordx4 %[v3], %[o3], %[xb]\n\t"                                \
               "global_load_dwordx4 %[v4], %[o0], %[nb]\n\t"                                \
               "global_load_dwordx4 %[v5], %[o1], %[nb]\n\t"                                \
               "global_load_dwordx4 %[v6], %[o2], %[nb]\n\t"                                \
               "global_load_dwordx4 %[v7], %[o3], %[nb]\n\t" LLHIP_PRO_DMA##NL            \
               "s_waitcnt vmcnt(" #NL ")"                                                   \
               : [m0o] "=&{m0}"(m0_out), [v0] "=&v"(r[0]), [v1] "=&v"(r[1]),               \
                 [v2] "=&v"(r[2]), [v3] "=&v"(r[3]), [v4] "=&v"(r[4]), [v5] "=&v"(r[5]),   \
                 [v6] "=&v"(r[6]), [v7] "=&v"(r[7])                                         \
               : [o0] "v"(xo[0]), [o1] "v"(xo[1]), [o2] "v"(xo[2]), [o3] "v"(xo[3]),        \
                 [xb] "s"(xb), [nb] "s"(nb), [wb] "s"(wb), [dst] "s"(dst), [w0] "v"(o[0]),  \
                 [w1] "v"(o[1]), [w2] "v"(o[2]), [w3] "v"(o[3]), [w4] "v"(o[4]),            \
                 [w5] "v"(o[5]), [w6] "v"(o[6])                                             \
               : "memory", "scc")

template <int NL>
__device__ __forceinline__ void prologue_loads(floatx4 (&r)[8], const float* xb, const float* nb,
                                               const uint32_t (&xo)[4], const uint8_t* wb,
                                               const uint32_t* wo, uint32_t dst) {
  static_assert(NL >= 1 && NL <= 7, "stage loads per wave");
  uint32_t o[7] = {0u, 0u, 0u, 0u, 0u, 0u, 0u};
#pragma unroll
  for (int k = 0; k < NL; ++k) o[k] = wo[k];
  uint32_t m0_out;
  if constexpr (NL == 1) LLHIP_PRO_ASM(1);
  else if constexpr (NL == 2) LLHIP_PRO_ASM(2);
  else if constexpr (NL == 3) LLHIP_PRO_ASM(3);
  else if constexpr (NL == 4) LLHIP_PRO_ASM(4);
  else if constexpr (NL == 5) LLHIP_PRO_ASM(5);
  else if constexpr (NL == 6) LLHIP_PRO_ASM(6);
  else LLHIP_PRO_ASM(7);
  (void)m0_out;
}

// A one-batch table built while stage 0 (NL loads from wb + wo to LDS dst)
// streams in: the same items, values and arithmetic as build_table.
template <typename IT, int WAVES, int NL>
__device__ __forceinline__ void build_table_overlapped(uint8_t* table, float* gsum,
                                                       const float* __restrict__ x, int nblk,
                                                       const float* __restrict__ nw, float eps,
                                                       float* red, const uint8_t* wb,
                                                       const uint32_t* wo, uint32_t dst) {
  constexpr int T = 64 * WAVES, EL = IT::kEl, kMaxI = 16 / EL;
  static_assert(kMaxI * EL == 16, "four 16-byte loads of x per thread");
  const int items = nblk * IT::kPerBlock;
  uint32_t xo[4];
#pragma unroll
  for (int j = 0; j < kMaxI; ++j) {
    const int x0 = IT::first(min((int)threadIdx.x + j * T, items - 1));
#pragma unroll
    for (int e = 0; e < EL; e += 4) xo[(j * EL + e) / 4] = (uint32_t)(x0 + e) * 4u;
  }
  floatx4 r[8];
  prologue_loads<NL>(r, x, nw ? nw : x, xo, wb, wo, dst);
  float v[kMaxI][EL], wv[kMaxI][EL];
#pragma unroll
  for (int j = 0; j < kMaxI; ++j)
#pragma unroll
    for (int e = 0; e < EL; ++e) {
      v[j][e] = r[(j * EL + e) / 4][e & 3];
      wv[j][e] = r[4 + (j * EL + e) / 4][e & 3];
    }
  float nscale = 1.f;
  table_batch<IT, WAVES>(v, wv, 0, items, true, nscale, nw, nblk, eps, red, table, gsum);
}

// Store the value v of row `row` (every lane of the wavefront calls this with
// its own row; `writer` lanes store).  Pairs of rows for the rotation and
// gate / up rows for SwiGLU are lanes n ^ 1 and n ^ 8 of the same 16 rows.
__device__ __forceinline__ void store_row(const GemvFuse& f, float* __restrict__ y, int rows,
                                          int row, float v, bool writer) {
#pragma clang fp contract(off)
  switch (f.epi) {
    case kGemvAdd:
      if (writer && row < rows) y[row] = f.res[row] + v;
      return;
    case kGemvSwiglu8: {
      // apply-silu-into then vector-elementwise-multiply-into
      // (llambda.lisp:6433-6441)
      const float u = dpp<kDppRowRor8>(v);  // lane n ^ 8
      if (writer && (row & 8) == 0 && row < rows) y[((row >> 4) << 3) | (row & 7)] = silu_ref(v) * u;
      return;
    }
    case kGemvRope:
    case kGemvCache: {
      const int hd = f.head_dim;
      float out = v;
      if (f.epi == kGemvRope) {
        // apply-rope-head-in-place (llambda.lisp:3760-3795): the pair
        // (x0, x1) rotated in double, each result rounded to single
        const float other = dpp<kDppXor1>(v);  // lane n ^ 1
        const int local = (row < f.split ? row : row - f.split) % hd;
        const int pair = local >> 1;
        if (pair < f.rope_pairs) {
          const double c = f.rope_cs[2 * pair], sn = f.rope_cs[2 * pair + 1];
          const double x0 = (local & 1) ? other : v, x1 = (local & 1) ? v : other;
          out = (local & 1) ? (float)(x0 * sn + x1 * c) : (float)(x0 * c - x1 * sn);
        }
        if (writer && row < rows && row < f.split) {
          y[row] = out * f.q_scale;  // vector-scale-into (llambda.lisp:6391)
          return;
        }
      }
      if (!writer || row >= rows) return;
      const int r = f.epi == kGemvRope ? row - f.split : row;
      float* base = f.epi == kGemvRope ? f.y1 : y;
      base[(int64_t)(r / hd) * f.head_stride + (int64_t)(*f.pos) * hd + r % hd] = out;
      return;
    }
    default:
      if (writer && row < rows) y[row] = v;
      return;
  }
}

// ------------------------------------------------------------------ kernel
template <int TYPE>
struct MfmaType {
  static constexpr int kBB = TYPE == kQ4_K ? 144 : 210;
  static constexpr int kTable = TYPE == kQ4_K ? kQ4Table : kQ6Table;
  static constexpr int kSums = TYPE == kQ4_K ? 8 : 16;
  static constexpr int kZero = 2048;  // zero lines read by A lanes without data
};

// Waves per workgroup, blocks per staged chunk and LDS stages per wave of the
// batch-1 GEMV, as measured best on the Q6_K output head and the 4096 x 4096
// Q4_K projection (deeper rings and longer chunks read HBM more slowly).
#ifndef LLHIP_GEMV_WAVES
#define LLHIP_GEMV_WAVES 8
#endif
#ifndef LLHIP_GEMV_CHUNK
#define LLHIP_GEMV_CHUNK 2
#endif
constexpr int kMfmaWaves = LLHIP_GEMV_WAVES;
#ifndef LLHIP_GEMV_DEPTH
#define LLHIP_GEMV_DEPTH 2
#endif
constexpr int kGemvDepth = LLHIP_GEMV_DEPTH;

// s_waitcnt vmcnt(n) and lgkmcnt(0) (gfx9 encoding, other counters left alone)
constexpr int waitcnt_vm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }
constexpr int kWaitLgkm0 = 0xC07F;

// LDS layout: [0, kZero) zeros | table (nblk * kTable) | group sums | stages
// (nbuf per wave) | split-K partial row sums.
template <int TYPE, int C, bool ALIGNED>
constexpr size_t mfma_lds_bytes(int nblk, int nbuf) {
  using T = MfmaType<TYPE>;
  using Ch = Chunk<T::kBB, C, ALIGNED>;
  return (size_t)T::kZero + (size_t)nblk * (T::kTable + 4 * T::kSums) +
         (size_t)kMfmaWaves * nbuf * Ch::kBuffer + kMfmaWaves * 64 * sizeof(float);
}

// ALIGNED: the weights, row_bytes and the chunk span are multiples of 4, so
// every row's chunk starts on a dword.  D: depth of the ring of stages per
// wave; nbuf = min(D, steps of any wave) stages are allocated, step s uses
// stage s % nbuf, all of them are filled once the activation table is
// built, and each is refilled as soon as it has been read.  S: waves per
// 16-row tile (rows are taken in rounds; see the step mapping below); with
// S > 1 a tile's partial sums meet in LDS and are added in wave order.
// The arguments of one batch-1 GEMV launch.
struct MfmaArgs {
  const uint8_t* w;
  int64_t row_bytes;
  int rows, nblk;
  const float* x;
  float* y;
  GemvFuse f;
  int nbuf;
  // weight stages with the non-temporal policy: launches of eight rounds or
  // more, whose rows stream far past what the caches keep (the Q6_K head
  // 128256 x 4096: 76.9 -> 74.3 us); shorter ones keep the default policy,
  // under which they measured faster (4096^2 Q4_K 5.7 us against 5.9)
  int nt;
};

// Workgroup `wg` of `nwg` working on one GEMV (the body of gemv_mfma_kernel
// and of each half of gemv_mfma_pair_kernel).
template <int TYPE, int C, bool ALIGNED, int D, int S>
__device__ __forceinline__ void gemv_mfma_body(uint8_t* lds, int wg, int nwg, const MfmaArgs& args) {
  const uint8_t* __restrict__ w = args.w;
  const int64_t row_bytes = args.row_bytes;
  const int rows = args.rows, nblk = args.nblk;
  const float* __restrict__ x = args.x;
  float* __restrict__ y = args.y;
  const GemvFuse& f = args.f;
  const int nbuf = args.nbuf;
  using T = MfmaType<TYPE>;
  using Ch = Chunk<T::kBB, C, ALIGNED>;
  const uint32_t table_off = T::kZero;
  uint8_t* table = lds + table_off;
  float* gsum = reinterpret_cast<float*>(table + nblk * T::kTable);
  uint8_t* stages = reinterpret_cast<uint8_t*>(gsum + nblk * T::kSums);
  float* partial = reinterpret_cast<float*>(stages + kMfmaWaves * nbuf * Ch::kBuffer);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4, a = lane & 15;
  // A addressing: lane_a = the lane's table entry in block 0, or a zero line
  // in MFMAs where its A row carries no data (zero_line_q4 / kZeroLineQ6).
  uint32_t a_base;
  bool a_m[4];
  if constexpr (TYPE == kQ4_K) {
    a_base = (g == (a >> 2)) ? table_off + (uint32_t)(a * 16) : zero_line_q4(g);
  } else {
    const bool act = ((a >> 1) & 1) == (g >> 1);
    a_base = table_off + (uint32_t)(((a & 3) * 2 + (g & 1)) * 16);
#pragma unroll
    for (int m = 0; m < 4; ++m) a_m[m] = act && (a >> 2) == m;
  }
  const uint32_t a_stride = (TYPE == kQ4_K && g != (a >> 2)) ? 0u : (uint32_t)T::kTable;

  const uint8_t* stage = stages + wave * nbuf * Ch::kBuffer;
  const uint32_t stage_lds = lds_address(stage);
  const int tiles = (rows + 15) >> 4;
  const int chunks = nblk / C;
  // Step s of this wave: (tile, chunk).  The workgroup owns a contiguous
  // range of tiles (HBM streams each workgroup's own region faster than
  // interleaved ones), taken in rounds of kGroups tiles: group grp (S waves)
  // takes tile first + r * kGroups + grp of round r, wave sw of the group its
  // chunks sw, sw + S, ...  With S = kMfmaWaves a round is one tile whose
  // bytes the whole workgroup loads at once.
  constexpr int kGroups = kMfmaWaves / S;
  const int grp = wave / S, sw = wave - grp * S;
  // Workgroups b and b + nwg / 2 (dispatched to the same CU when the grid
  // is two per CU) take the adjacent ranges 2 b and 2 b + 1 (measured: the
  // Llama decode token -1.2%, the head unchanged).
  const int half = (nwg + 1) >> 1;
  const int rix = wg < half ? 2 * wg : 2 * (wg - half) + 1;
  const int wg_first = (int)(((int64_t)rix * tiles) / nwg);
  const int wg_end = (int)(((int64_t)(rix + 1) * tiles) / nwg);
  const int rounds = (wg_end - wg_first + kGroups - 1) / kGroups;  // same for every group
  const int first_tile = wg_first + grp;
  const int tile_step = kGroups;
  const int cpt = S == 1 ? chunks : (chunks - sw + S - 1) / S;  // chunks per tile
  const int my_tiles =
      first_tile < wg_end ? (wg_end - first_tile + tile_step - 1) / tile_step : 0;
  const int steps = my_tiles * cpt;
  const uint32_t rb = (uint32_t)row_bytes;
  auto tile_of = [&](int s) { return first_tile + (s / cpt) * tile_step; };
  auto chunk_of = [&](int s) {
    const int c = s - (s / cpt) * cpt;
    return S == 1 ? c : sw + S * c;
  };

  // per load instruction i: this lane's (row, piece) and byte offset in the tile
  uint32_t voff[Ch::kLoads];
#pragma unroll
  for (int i = 0; i < Ch::kLoads; ++i) {
    const int idx = min(64 * i + lane, 16 * Ch::kPitch - 1);
    const int r = idx / Ch::kPitch;
    voff[i] = (uint32_t)r * rb + 16u * (uint32_t)min(idx - r * Ch::kPitch, Ch::kPieces - 1);
  }

  // Row r of the tile starts at base + r * rb; its range is read from the
  // dword at or below that, i.e. from base_al + ((bsh + r * rb) & ~3) with
  // base_al = base & ~3 and bsh = base & 3 (offsets stay non-negative).
  auto stage_src = [&](int s, uint32_t (&o)[Ch::kLoads]) {
    const int tile = tile_of(s);
    const int chunk = chunk_of(s);
    const uint8_t* base =
        uniform_ptr(w + (int64_t)tile * 16 * row_bytes + (int64_t)chunk * Ch::kSpan);
    const uint32_t bsh = ALIGNED ? 0u : (uint32_t)(reinterpret_cast<uintptr_t>(base) & 3u);
    const int rmax = rows - 1 - tile * 16;
    if (ALIGNED && rmax >= 15) {
#pragma unroll
      for (int i = 0; i < Ch::kLoads; ++i) o[i] = voff[i];
    } else {
      // unaligned rows, or the last, partial tile (rows past the end re-read
      // the last row)
#pragma unroll
      for (int i = 0; i < Ch::kLoads; ++i) {
        const int idx = min(64 * i + lane, 16 * Ch::kPitch - 1);
        const int r = idx / Ch::kPitch;
        const uint32_t rr = (uint32_t)min(r, rmax);
        o[i] = ((bsh + rr * rb) & ~3u) + 16u * (uint32_t)min(idx - r * Ch::kPitch, Ch::kPieces - 1);
      }
    }
    return base - bsh;
  };
  auto issue = [&](int s) {
    uint32_t o[Ch::kLoads];
    const uint8_t* base_al = stage_src(s, o);
    const uint32_t dst = stage_lds + (uint32_t)((s % nbuf) * Ch::kBuffer);
    if (args.nt) {
#pragma unroll
      for (int i = 0; i < Ch::kLoads; ++i) load_lds16_nt(base_al, o[i], dst + 1024u * i);
    } else {
#pragma unroll
      for (int i = 0; i < Ch::kLoads; ++i) load_lds16(base_al, o[i], dst + 1024u * i);
    }
  };

  for (int i = threadIdx.x; i < T::kZero / 16; i += blockDim.x)
    reinterpret_cast<u32x4*>(lds)[i] = u32x4{0u, 0u, 0u, 0u};
  using IT = std::conditional_t<TYPE == kQ4_K, Q4Items, Q6Items>;
  const int first = min(nbuf, steps);
  // (the overlapped form holds a stage of at most seven loads: four-block
  // chunks take the plain one)
  bool overlapped = false;
  if constexpr (Ch::kLoads <= 7) {
    if (table_one_batch<IT, kMfmaWaves>(nblk) && first == 1) {
      // one stage per wave: its DMA is issued right behind the table's loads
      // and streams in while the table is built (never for a wave without
      // steps -- small matrices leave some waves no tile -- whose step 0
      // would lie past the rows)
      uint32_t o[Ch::kLoads];
      const uint8_t* base_al = stage_src(0, o);
      build_table_overlapped<IT, kMfmaWaves, Ch::kLoads>(table, gsum, x, nblk, f.norm_w,
                                                          f.norm_eps, partial, base_al, o,
                                                          stage_lds);
      overlapped = true;
    }
  }
  if (!overlapped) {
    // activation table first: its loads would otherwise queue behind the
    // weight stages' and hold every wave's first step back (measured: the
    // 4096 x 4096 Q4_K GEMV 7.5 -> 6.2 us, the Llama decode token -5%)
    build_table<IT, kMfmaWaves>(table, gsum, x, nblk, f.norm_w, f.norm_eps, partial);
    // then every stage is filled
    for (int s = 0; s < first; ++s) issue(s);
  }
  __syncthreads();

  float acc = 0.f;
  int s = 0;
  for (int r = 0; r < rounds; ++r) {
  const int round_end = S == 1 ? steps : (r < my_tiles ? s + cpt : s);
  for (; s < round_end; ++s) {
    const int tile = tile_of(s);
    const int chunk = chunk_of(s);
    // steps up to s + nbuf - 1 are issued; at most `ahead` later steps' loads
    // may still be in flight (a y store in between only makes the wait
    // stricter)
    const int ahead = min(steps, s + nbuf) - s - 1;
    if constexpr (D <= 2) {
      if (ahead == 0) __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
      else __builtin_amdgcn_s_waitcnt(waitcnt_vm(Ch::kLoads));
    } else {
      switch (ahead) {
        case 0: __builtin_amdgcn_s_waitcnt(waitcnt_vm(0)); break;
        case 1: __builtin_amdgcn_s_waitcnt(waitcnt_vm(Ch::kLoads)); break;
        case 2: __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * Ch::kLoads)); break;
        default: __builtin_amdgcn_s_waitcnt(waitcnt_vm(3 * Ch::kLoads)); break;
      }
    }
    const uint8_t* buf = stage + (s % nbuf) * Ch::kBuffer;
    const uint8_t* rowp = buf + n * Ch::kRow;
    if constexpr (!ALIGNED) {
      const int row = min(tile * 16 + n, rows - 1);
      rowp += (reinterpret_cast<uintptr_t>(w + (int64_t)row * row_bytes + (int64_t)chunk * Ch::kSpan) & 3u);
    }
    // this lane's bytes of the stage into registers, then the stage is
    // refilled (its LDS reads drained first) while the blocks compute
    using Raw = std::conditional_t<TYPE == kQ4_K, Q4Raw, Q6Raw>;
    Raw raw[C];
    [&]<int... BL>(std::integer_sequence<int, BL...>) {
      ((raw[BL] = [&] {
         const uint8_t* p = rowp + BL * T::kBB;
         if constexpr (TYPE == kQ4_K) return q4k_fetch(p, g);
         else if constexpr (ALIGNED) return q6k_fetch<(BL * 210) & 3>(p, g);
         else return q6k_fetch<-1>(p, g);
       }()), ...);
    }(std::make_integer_sequence<int, C>{});
    if (s + nbuf < steps) {
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      issue(s + nbuf);
    }
#pragma unroll
    for (int bl = 0; bl < C; ++bl) {
      const int b = chunk * C + bl;
      const float* gs = gsum + b * T::kSums;
      if constexpr (TYPE == kQ4_K) {
        acc += q4k_block(raw[bl], lds, a_base + (uint32_t)b * a_stride, gs, g);
      } else {
        const uint32_t ab = a_base + (uint32_t)b * (uint32_t)T::kTable;
        const uint32_t am[4] = {a_m[0] ? ab : kZeroLineQ6, a_m[1] ? ab : kZeroLineQ6,
                                a_m[2] ? ab : kZeroLineQ6, a_m[3] ? ab : kZeroLineQ6};
        acc += q6k_block(raw[bl], lds, am, gs, g);
      }
    }
    if (S == 1 && chunk == chunks - 1) {
      const float v = sum_lane_groups(acc);
      store_row(f, y, rows, tile * 16 + n, v, g == 0);
      acc = 0.f;
    }
  }
  if constexpr (S > 1) {
    // the round's tiles: each group's row sums, in wave order
    // (partial sums alternate between two halves by round, so one barrier
    // per round suffices: a half is written again two rounds later, after
    // the next round's barrier, which its readers reach only when done)
    float* part = partial + (r & 1) * (kMfmaWaves * 16);
    const float v = sum_lane_groups(acc);
    acc = 0.f;
    if (g == 0) part[wave * 16 + n] = v;
    __syncthreads();
    const int tile = first_tile + r * tile_step;
    if (sw == 0 && r < my_tiles) {
      float t = part[wave * 16 + n];
#pragma unroll
      for (int k = 1; k < S; ++k) t = t + part[(wave + k) * 16 + n];
      store_row(f, y, rows, tile * 16 + n, t, g == 0);
    }
  } else {
    break;  // S = 1: every step of the wave ran in the one pass
  }
  }
}

template <int TYPE, int C, bool ALIGNED, int D, int S>
__global__ void __launch_bounds__(64 * kMfmaWaves) gemv_mfma_kernel(const MfmaArgs args) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  gemv_mfma_body<TYPE, C, ALIGNED, D, S>(lds, blockIdx.x, gridDim.x, args);
}

// ------------------------------------------------------------ tile rounds
// The batch-1 GEMV of long launches whose row is one chunk per wave (K =
// C x kMfmaWaves blocks, dword-aligned rows): a round is one 16-row tile of
// the workgroup's contiguous range, and its bytes -- contiguous in HBM --
// come in by non-temporal DMA as one contiguous run per wave into a tile
// buffer whose rows sit an odd number of 16-byte pieces apart (a row's pad
// piece re-reads its last piece, in the same instruction).  Each wave then
// reads its own chunk of the 16 rows from the buffer and computes it exactly
// as gemv_mfma_body does, and wave 0 adds the eight partial sums in wave
// order: the outputs are that kernel's, bit for bit.  (There each wave DMAs
// its chunk of every row, so the 128-byte lines on chunk boundaries are two
// waves' requests; non-temporal, they are fetched twice: 1.07x the bytes.
// One run per wave reads 1.00x.)
constexpr int kTileMaxLoads = 8;  // DMA instructions (1 KB) per wave and tile

__host__ __device__ constexpr int tile_pitch_pieces(int64_t row_bytes) {
  return (int)(row_bytes / 16) | 1;  // odd: a fragment's 16 rows in 16 bank quads
}
__host__ __device__ constexpr int tile_loads(int64_t row_bytes) {
  return (16 * tile_pitch_pieces(row_bytes) + 63) / 64;
}
// LDS: [0, kZero) zeros | table | group sums | tile buffer | partials (two
// rounds x waves x 16 rows)
template <int TYPE>
constexpr size_t tile_lds_bytes(int nblk, int64_t row_bytes) {
  using T = MfmaType<TYPE>;
  return (size_t)T::kZero + (size_t)nblk * (T::kTable + 4 * T::kSums) +
         1024 * (size_t)tile_loads(row_bytes) + 2 * kMfmaWaves * 16 * sizeof(float);
}

template <int TYPE, int C>
__global__ void __launch_bounds__(64 * kMfmaWaves) gemv_tile_kernel(const MfmaArgs args) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int S = kMfmaWaves;
  using T = MfmaType<TYPE>;
  const uint8_t* __restrict__ w = args.w;
  const int64_t row_bytes = args.row_bytes;
  const int rows = args.rows, nblk = args.nblk;
  const GemvFuse& f = args.f;
  const int pitch = tile_pitch_pieces(row_bytes), loads = tile_loads(row_bytes);
  uint8_t* table = lds + T::kZero;
  float* gsum = reinterpret_cast<float*>(table + nblk * T::kTable);
  uint8_t* tbuf = reinterpret_cast<uint8_t*>(gsum + nblk * T::kSums);
  float* partial = reinterpret_cast<float*>(tbuf + 1024 * loads);
  const uint32_t tbuf_lds = lds_address(tbuf);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4, a = lane & 15;
  const uint32_t table_off = T::kZero;
  uint32_t a_base;
  bool a_m[4];
  if constexpr (TYPE == kQ4_K) {
    a_base = (g == (a >> 2)) ? table_off + (uint32_t)(a * 16) : zero_line_q4(g);
  } else {
    const bool act = ((a >> 1) & 1) == (g >> 1);
    a_base = table_off + (uint32_t)(((a & 3) * 2 + (g & 1)) * 16);
#pragma unroll
    for (int m = 0; m < 4; ++m) a_m[m] = act && (a >> 2) == m;
  }
  const uint32_t a_stride = (TYPE == kQ4_K && g != (a >> 2)) ? 0u : (uint32_t)T::kTable;

  // the workgroup's contiguous tile range (workgroups b and b + nwg / 2 --
  // one CU when the grid is two per CU -- take adjacent ranges)
  const int tiles = (rows + 15) >> 4, nwg = gridDim.x, wg = blockIdx.x;
  const int half = (nwg + 1) >> 1;
  const int rix = wg < half ? 2 * wg : 2 * (wg - half) + 1;
  const int wg_first = (int)(((int64_t)rix * tiles) / nwg);
  const int wg_end = (int)(((int64_t)(rix + 1) * tiles) / nwg);
  const int ntiles = wg_end - wg_first;

  // this wave's run: loads [l0, l0 + nl) of the tile; lane i of load l
  // writes slot 64 l + i = (row, piece) of the buffer
  const int per = loads / S, extra = loads - per * S;
  const int l0 = wave * per + min(wave, extra), nl = per + (wave < extra ? 1 : 0);
  const uint32_t rb = (uint32_t)row_bytes;
  const int rp = (int)(row_bytes / 16);  // pieces of a row
  uint32_t voff[kTileMaxLoads];
  int vrow[kTileMaxLoads];
#pragma unroll
  for (int l = 0; l < kTileMaxLoads; ++l) {
    const int slot = min(64 * (l0 + l) + lane, 16 * pitch - 1);
    const int r = slot / pitch;
    vrow[l] = r;
    voff[l] = (uint32_t)r * rb + 16u * (uint32_t)min(slot - r * pitch, rp - 1);
  }
  auto issue = [&](int tile) {
    const uint8_t* base = uniform_ptr(w + (int64_t)tile * 16 * row_bytes);
    const int rmax = rows - 1 - tile * 16;  // rows past the end re-read the last one
#pragma unroll
    for (int l = 0; l < kTileMaxLoads; ++l) {
      if (l < nl) {
        const uint32_t o = rmax >= 15 ? voff[l]
                                      : voff[l] - (uint32_t)(vrow[l] - min(vrow[l], rmax)) * rb;
        load_lds16_nt(base, o, tbuf_lds + 1024u * (uint32_t)(l0 + l));
      }
    }
  };

  for (int i = threadIdx.x; i < T::kZero / 16; i += blockDim.x)
    reinterpret_cast<u32x4*>(lds)[i] = u32x4{0u, 0u, 0u, 0u};
  using IT = std::conditional_t<TYPE == kQ4_K, Q4Items, Q6Items>;
  // the first tile's DMA streams in while the activation table is built
  // (the table's loads wait behind it; head 71.3 -> 70.5 us by events)
  if (ntiles > 0) issue(wg_first);
  build_table<IT, S>(table, gsum, args.x, nblk, f.norm_w, f.norm_eps, partial);
  __syncthreads();

  auto finish_round = [&](int r) {  // wave 0: the round's row sums, in wave order
    const float* part = partial + (r & 1) * (S * 16);
    float t = part[n];
#pragma unroll
    for (int k = 1; k < S; ++k) t = t + part[k * 16 + n];
    store_row(f, args.y, rows, (wg_first + r) * 16 + n, t, g == 0);
  };
  using Raw = std::conditional_t<TYPE == kQ4_K, Q4Raw, Q6Raw>;
  const uint8_t* rowp = tbuf + n * (16 * pitch) + wave * (C * T::kBB);
  for (int r = 0; r < ntiles; ++r) {
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();  // the tile is in LDS; the last round's partial sums too
    if (r > 0 && wave == 0) finish_round(r - 1);
    Raw raw[C];
    [&]<int... BL>(std::integer_sequence<int, BL...>) {
      ((raw[BL] = [&] {
         const uint8_t* p = rowp + BL * T::kBB;
         if constexpr (TYPE == kQ4_K) return q4k_fetch(p, g);
         else return q6k_fetch<(BL * 210) & 3>(p, g);
       }()), ...);
    }(std::make_integer_sequence<int, C>{});
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    __syncthreads();  // every wave has its chunk: the buffer takes the next tile
    if (r + 1 < ntiles) issue(wg_first + r + 1);
    float acc = 0.f;
#pragma unroll
    for (int bl = 0; bl < C; ++bl) {
      const int b = wave * C + bl;
      const float* gs = gsum + b * T::kSums;
      if constexpr (TYPE == kQ4_K) {
        acc += q4k_block(raw[bl], lds, a_base + (uint32_t)b * a_stride, gs, g);
      } else {
        const uint32_t ab = a_base + (uint32_t)b * (uint32_t)T::kTable;
        const uint32_t am[4] = {a_m[0] ? ab : kZeroLineQ6, a_m[1] ? ab : kZeroLineQ6,
                                a_m[2] ? ab : kZeroLineQ6, a_m[3] ? ab : kZeroLineQ6};
        acc += q6k_block(raw[bl], lds, am, gs, g);
      }
    }
    const float v = sum_lane_groups(acc);
    if (g == 0) partial[(r & 1) * (S * 16) + wave * 16 + n] = v;
  }
  if (ntiles > 0) {
    __syncthreads();
    if (wave == 0) finish_round(ntiles - 1);
  }
}

// Two independent GEMVs in one launch (the decoder's q|k and v rows): the
// first `grid_a` workgroups run the first, the rest the second, so the
// second's fixed latency (table, first loads, epilogue) overlaps the first's
// instead of following it.
template <int TA, int CA, bool AA, int TB, int CB, bool AB>
__global__ void __launch_bounds__(64 * kMfmaWaves)
gemv_mfma_pair_kernel(const MfmaArgs a, const MfmaArgs b, int grid_a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  if ((int)blockIdx.x < grid_a)
    gemv_mfma_body<TA, CA, AA, kGemvDepth, kMfmaWaves>(lds, blockIdx.x, grid_a, a);
  else
    gemv_mfma_body<TB, CB, AB, kGemvDepth, kMfmaWaves>(lds, blockIdx.x - grid_a,
                                                        gridDim.x - grid_a, b);
}

// ------------------------------------------------------------------ host


template <int TYPE>
struct MfmaChoice {
  int chunk;
  bool aligned;
  int depth;  // ring depth per wave
  int waves;  // waves per tile (S)
};

// Stages a wave needs: the ring depth, or fewer when no wave has that many
// steps (S > 1: one tile's chunks shared by S waves).
static int mfma_nbuf(int depth, int waves, int chunks) {
  if (waves == 1) return depth;
  return std::max(1, std::min(depth, (chunks + waves - 1) / waves));
}
template <int TYPE>
static int mfma_nbuf(const MfmaChoice<TYPE>& c, int nblk) {
  return mfma_nbuf(c.depth, c.waves, nblk / c.chunk);
}

// Waves per tile: as many as the tile has chunks, up to the workgroup (a
// round of a workgroup then loads one contiguous tile at once; measured best
// for every decode shape, 4096..128256 rows).
#ifndef LLHIP_GEMV_WAVES_PER_TILE
#define LLHIP_GEMV_WAVES_PER_TILE 8
#endif
static int mfma_waves_per_tile(int64_t chunks) {
  int S = 1;
  while (S < LLHIP_GEMV_WAVES_PER_TILE && S < kMfmaWaves && chunks >= 2 * S) S *= 2;
  return S;
}

template <int TYPE>
static size_t mfma_lds_for(const MfmaChoice<TYPE>& c, int nblk) {
  const int nb = mfma_nbuf(c, nblk);
  if (c.chunk == 4)
    return c.aligned ? mfma_lds_bytes<TYPE, 4, true>(nblk, nb)
                     : mfma_lds_bytes<TYPE, 4, false>(nblk, nb);
  if (c.chunk == 2)
    return c.aligned ? mfma_lds_bytes<TYPE, 2, true>(nblk, nb)
                     : mfma_lds_bytes<TYPE, 2, false>(nblk, nb);
  return c.aligned ? mfma_lds_bytes<TYPE, 1, true>(nblk, nb)
                   : mfma_lds_bytes<TYPE, 1, false>(nblk, nb);
}

template <int TYPE>
static MfmaChoice<TYPE> mfma_choice(const GemvProblem& p) {
  const int64_t nblk = p.columns / 256;
  MfmaChoice<TYPE> c;
  c.chunk = nblk % LLHIP_GEMV_CHUNK == 0 ? LLHIP_GEMV_CHUNK : nblk % 2 == 0 ? 2 : 1;
  c.depth = kGemvDepth;
  // long rows: shorter chunks, then fewer stages, until the LDS holds the
  // activation table and the stages
  for (;;) {
    const int64_t span = (int64_t)c.chunk * MfmaType<TYPE>::kBB;
    c.aligned = p.row_bytes % 4 == 0 && span % 4 == 0;
    c.waves = mfma_waves_per_tile(nblk / c.chunk);
    if (mfma_lds_for(c, (int)nblk) <= kMaxLdsBytes) break;
    if (c.chunk > 1) c.chunk /= 2;
    else if (c.depth > 2) c.depth = 2;
    else break;
  }
  return c;
}

bool gemv_mfma_supported(const GemvProblem& p) {
  if (p.tokens != 1 || p.columns % 256 != 0 || p.rows < 1) return false;
  if (p.row_bytes * 16 >= (int64_t)1 << 31) return false;
  // row ranges are read from the dword at or below their start: the
  // weights must start on a dword (Q4_K: rows 16-byte aligned, its blocks
  // are read from LDS with 16-byte loads)
  if (reinterpret_cast<uintptr_t>(p.weights) & 3u) return false;
  // activations are read as float4
  if (reinterpret_cast<uintptr_t>(p.x) & 15u) return false;
  if (p.type == kQ4_K) {
    const MfmaChoice<kQ4_K> c = mfma_choice<kQ4_K>(p);
    return (reinterpret_cast<uintptr_t>(p.weights) & 15u) == 0 && p.row_bytes % 16 == 0 &&
           mfma_lds_for(c, (int)(p.columns / 256)) <= kMaxLdsBytes;
  }
  if (p.type == kQ6_K) {
    const MfmaChoice<kQ6_K> c = mfma_choice<kQ6_K>(p);
    return mfma_lds_for(c, (int)(p.columns / 256)) <= kMaxLdsBytes;
  }
  return false;
}

// The tile-round kernel, on the same persistent grid rule as launch_mfma;
// hipErrorInvalidValue when its LDS does not allow one workgroup per CU.
template <int TYPE, int C>
static hipError_t launch_tile(const GemvProblem& p, const MfmaArgs& args, int tiles,
                              hipStream_t stream) {
  const size_t lds = tile_lds_bytes<TYPE>(args.nblk, p.row_bytes);
  if (lds > kMaxLdsBytes) return hipErrorInvalidValue;
  const auto kernel = gemv_tile_kernel<TYPE, C>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kernel),
                                                   64 * kMfmaWaves, lds) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  const int cap = device_cu_count() * per_cu;
  const int nrounds = (tiles + cap - 1) / cap;
  const int grid = std::max(1, (tiles + nrounds - 1) / nrounds);
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(64 * kMfmaWaves), lds, stream, args);
  return hipGetLastError();
}

template <int TYPE, int C, bool ALIGNED, int D, int S>
static hipError_t launch_mfma(const GemvProblem& p, const GemvFuse& f, hipStream_t stream) {
  const int nblk = (int)(p.columns / 256);
  const int nbuf = mfma_nbuf(D, S, nblk / C);
  const size_t lds = mfma_lds_bytes<TYPE, C, ALIGNED>(nblk, nbuf);
  const auto kernel = gemv_mfma_kernel<TYPE, C, ALIGNED, D, S>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  const int tiles = (int)((p.rows + 15) / 16);
  // persistent: at most the resident workgroups, each a contiguous tile range
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kernel),
                                                   64 * kMfmaWaves, lds) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  const int needed = (tiles + kMfmaWaves / S - 1) / (kMfmaWaves / S);
  const int cap = device_cu_count() * per_cu;
  // Long launches take the smallest grid with the same number of rounds, so
  // that every workgroup has as many (the Q6_K head: 501 workgroups of 16
  // tiles instead of 512 of 15 or 16, 77.1 -> 76.7 us sustained); for a few
  // rounds that changed nothing or lost (the decode token's gate|up: 448 of
  // 4 instead of 512 of 3 or 4, +0.2%).
  const int nrounds = (needed + cap - 1) / cap;
  const int grid = std::max(1, nrounds >= 8 ? (needed + nrounds - 1) / nrounds : std::min(needed, cap));
  const MfmaArgs args{p.weights, p.row_bytes, (int)p.rows, nblk, p.x, p.y, f, nbuf, nrounds >= 8};
  if constexpr (ALIGNED && S == kMfmaWaves) {
    if (nrounds >= 8 && nblk == C * S && p.row_bytes % 16 == 0 &&
        tile_loads(p.row_bytes) <= kTileMaxLoads * S)
      return launch_tile<TYPE, C>(p, args, tiles, stream);
  }
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(64 * kMfmaWaves), lds, stream, args);
  return hipGetLastError();
}

template <int TYPE, int C, bool ALIGNED>
static hipError_t launch_mfma_ds(const MfmaChoice<TYPE>& c, const GemvProblem& p,
                                 const GemvFuse& f, hipStream_t s) {
  if (c.depth != kGemvDepth) {  // shallower ring where the LDS is short
    switch (c.waves) {
      case 8: return launch_mfma<TYPE, C, ALIGNED, 2, (kMfmaWaves >= 8 ? 8 : kMfmaWaves)>(p, f, s);
      case 4: return launch_mfma<TYPE, C, ALIGNED, 2, (kMfmaWaves >= 4 ? 4 : kMfmaWaves)>(p, f, s);
      case 2: return launch_mfma<TYPE, C, ALIGNED, 2, 2>(p, f, s);
      default: return launch_mfma<TYPE, C, ALIGNED, 2, 1>(p, f, s);
    }
  }
  switch (c.waves) {
    case 8: return launch_mfma<TYPE, C, ALIGNED, kGemvDepth, (kMfmaWaves >= 8 ? 8 : kMfmaWaves)>(p, f, s);
    case 4: return launch_mfma<TYPE, C, ALIGNED, kGemvDepth, (kMfmaWaves >= 4 ? 4 : kMfmaWaves)>(p, f, s);
    case 2: return launch_mfma<TYPE, C, ALIGNED, kGemvDepth, 2>(p, f, s);
    default: return launch_mfma<TYPE, C, ALIGNED, kGemvDepth, 1>(p, f, s);
  }
}

template <int TYPE>
static hipError_t launch_mfma_type(const GemvProblem& p, const GemvFuse& f, hipStream_t stream) {
  const MfmaChoice<TYPE> c = mfma_choice<TYPE>(p);
#if LLHIP_GEMV_CHUNK == 4
  if (c.chunk == 4)
    return c.aligned ? launch_mfma_ds<TYPE, 4, true>(c, p, f, stream)
                     : launch_mfma_ds<TYPE, 4, false>(c, p, f, stream);
#endif
  if (c.chunk == 2)
    return c.aligned ? launch_mfma_ds<TYPE, 2, true>(c, p, f, stream)
                     : launch_mfma_ds<TYPE, 2, false>(c, p, f, stream);
  return c.aligned ? launch_mfma_ds<TYPE, 1, true>(c, p, f, stream)
                   : launch_mfma_ds<TYPE, 1, false>(c, p, f, stream);
}

hipError_t gemv_mfma_launch(const GemvProblem& p, hipStream_t stream) {
  const GemvFuse plain;
  return p.type == kQ4_K ? launch_mfma_type<kQ4_K>(p, plain, stream)
                         : launch_mfma_type<kQ6_K>(p, plain, stream);
}

static bool fuse_ok(const GemvProblem& p, const GemvFuse& f) {
  if (!gemv_mfma_supported(p)) return false;
  if ((f.epi == kGemvRope || f.epi == kGemvCache) && (f.head_dim <= 0 || f.head_dim % 2 || !f.pos))
    return false;
  if (f.epi == kGemvSwiglu8 && p.rows % 16) return false;
  if (f.epi == kGemvAdd && !f.res) return false;
  return true;
}

hipError_t gemv_fused_launch(const GemvProblem& p, const GemvFuse& f, hipStream_t stream) {
  if (!fuse_ok(p, f)) return hipErrorInvalidValue;
  return p.type == kQ4_K ? launch_mfma_type<kQ4_K>(p, f, stream)
                         : launch_mfma_type<kQ6_K>(p, f, stream);
}

// The pair kernel is instantiated for the shape of the Llama-style q|k (Q4_K)
// and v (Q6_K) rows whose K is a multiple of 512 (two-block chunks, dword
// aligned rows, whole workgroups on a tile); other pairs run as two launches.
template <int TYPE>
static bool pair_shape(const GemvProblem& p) {
  const MfmaChoice<TYPE> c = mfma_choice<TYPE>(p);
  return c.chunk == 2 && c.aligned && c.depth == kGemvDepth && c.waves == kMfmaWaves;
}

hipError_t gemv_fused_pair_launch(const GemvProblem& pa, const GemvFuse& fa, const GemvProblem& pb,
                                  const GemvFuse& fb, hipStream_t stream) {
  if (!fuse_ok(pa, fa) || !fuse_ok(pb, fb)) return hipErrorInvalidValue;
  if (!(pa.type == kQ4_K && pb.type == kQ6_K && pair_shape<kQ4_K>(pa) && pair_shape<kQ6_K>(pb))) {
    const hipError_t e = gemv_fused_launch(pa, fa, stream);
    return e != hipSuccess ? e : gemv_fused_launch(pb, fb, stream);
  }
  const int na = (int)(pa.columns / 256), nb = (int)(pb.columns / 256);
  const int bufa = mfma_nbuf(kGemvDepth, kMfmaWaves, na / 2);
  const int bufb = mfma_nbuf(kGemvDepth, kMfmaWaves, nb / 2);
  const size_t lds = std::max(mfma_lds_bytes<kQ4_K, 2, true>(na, bufa),
                              mfma_lds_bytes<kQ6_K, 2, true>(nb, bufb));
  const auto kernel = gemv_mfma_pair_kernel<kQ4_K, 2, true, kQ6_K, 2, true>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kernel),
                                                   64 * kMfmaWaves, lds) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  const int slots = device_cu_count() * per_cu;
  const int ta = (int)((pa.rows + 15) / 16), tb = (int)((pb.rows + 15) / 16);
  // resident slots shared in proportion to the tiles (each part >= 1)
  int ga = std::min(ta, std::max(1, (int)((int64_t)slots * ta / (ta + tb))));
  int gb = std::min(tb, std::max(1, slots - ga));
  const MfmaArgs a{pa.weights, pa.row_bytes, (int)pa.rows, na, pa.x, pa.y, fa, bufa};
  const MfmaArgs b{pb.weights, pb.row_bytes, (int)pb.rows, nb, pb.x, pb.y, fb, bufb};
  hipLaunchKernelGGL(kernel, dim3(ga + gb), dim3(64 * kMfmaWaves), lds, stream, a, b, ga);
  return hipGetLastError();
}

}  // namespace llhip
