// gemv.hip -- dequant-fused GEMV kernels for gfx950.
//
// y[tok][row] = sum_k W[row][k] * x[tok][k] for packed rows of Q4_K, Q6_K,
// Q5_0, Q8_0 (units.h) and F32, i.e. %gguf-model-matrix-vector-multiply-into
// (llambda.lisp:4542-4658) on one MI355X.
//
// Launch shape: 256-thread workgroups (4 wavefronts).  Each workgroup copies
// the activations of up to NT tokens into LDS once, with the sums of every
// 16-element group, then its wavefronts stream rows: a wavefront owns
// `slots` row slots of `lpr` lanes (lpr = min(64, pow2ceil(K/32))), every lane
// dequantises one 32-weight unit per step with 16-byte loads, and the row's
// lanes are summed with cross-lane shuffles.  R rows per slot are loaded
// before the first multiply so each lane keeps 2R 16-byte loads in flight.
#include "gemv.h"
#include "positions.h"

#include <algorithm>

namespace llhip {

template <int TYPE, int NT, int R>
__global__ void __launch_bounds__(256)
gemv_kernel(const uint8_t* __restrict__ w, int64_t row_bytes, int rows, int K,
            const float* __restrict__ x, int64_t x_stride, int ntok,
            float* __restrict__ y, int64_t y_stride, int lpr_log2) {
  extern __shared__ float smem[];
  float* xs = smem;
  float* xg = smem + NT * K;
  stage_x<NT>(xs, xg, x, x_stride, ntok, K);
  __syncthreads();
  const XView xv{xs, xg, K, K >> 4};

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lpr = 1 << lpr_log2;
  const int slot = lane >> lpr_log2;
  const int l = lane & (lpr - 1);
  const int slots = kWave >> lpr_log2;
  const int units = K >> 5;
  const int waves_per_block = blockDim.x >> 6;
  const int rows_per_iter = slots * R;
  const int stride = gridDim.x * waves_per_block * rows_per_iter;

  for (int base = (blockIdx.x * waves_per_block + wave) * rows_per_iter; base < rows; base += stride) {
    float acc[R][NT];
    const uint8_t* rp[R];
    bool valid[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = base + r * slots + slot;
      valid[r] = row < rows;
      rp[r] = w + (int64_t)(valid[r] ? row : 0) * row_bytes;
    }
    rows_dot<TYPE, NT, R>(rp, valid, l, lpr, units, xv, acc);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = base + r * slots + slot;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const float v = segment_sum_dyn(acc[r][t], lpr);
        if (l == 0 && row < rows && t < ntok) y[t * y_stride + row] = v;
      }
    }
  }
}

// ------------------------------------------------------------------------
// Batch-1 row-streaming GEMV: every lane owns one 64-weight position of K
// (positions.h) with its activations in registers, and streams rows.
//   positions P = K/64 <= 64: a wavefront covers a row with L = pow2ceil(P)
//     lanes, 64/L rows side by side; four independent wavefronts per block.
//   P > 64: K is split over `kwaves` wavefronts of one block (<= 64
//     positions each); their row sums meet in LDS.
// R rows are loaded per lane before the first multiply.
constexpr int kRowsMaxWaves = 8;

// Rows loaded per lane before the first multiply (compile-time tuning).
#ifndef LLHIP_ROWS_Q4K
#define LLHIP_ROWS_Q4K 2
#endif
#ifndef LLHIP_ROWS_Q6K
#define LLHIP_ROWS_Q6K 1
#endif

template <int TYPE, int R>
__global__ void __launch_bounds__(512)
gemv_rows_kernel(const uint8_t* __restrict__ w, int64_t row_bytes, int rows, int positions,
                 const float* __restrict__ x, float* __restrict__ y, int lanes_log2, int kwaves) {
  using P = Pos<TYPE>;
  __shared__ float partial[kRowsMaxWaves][R];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int L = 1 << lanes_log2;
  const int slot = lane >> lanes_log2;
  const int l = lane & (L - 1);
  const int slots = kWave >> lanes_log2;
  int pos, rows_per_iter, base, stride;
  if (kwaves == 1) {
    pos = l;
    rows_per_iter = slots * R;
    const int waves_per_block = blockDim.x >> 6;
    base = (blockIdx.x * waves_per_block + wave) * rows_per_iter;
    stride = gridDim.x * waves_per_block * rows_per_iter;
  } else {
    const int per_wave = (positions + kwaves - 1) / kwaves;
    pos = wave * per_wave + l;
    if (l >= per_wave) pos = positions;  // idle lane
    rows_per_iter = R;
    base = blockIdx.x * R;
    stride = gridDim.x * R;
  }
  const bool active = pos < positions;
  float xr[64];
  float g[P::kGroups];
  if (active) {
#pragma unroll
    for (int e = 0; e < 64; e += 4) {
      const float4 v = *reinterpret_cast<const float4*>(x + P::x_index(pos, e));
      xr[e] = v.x; xr[e + 1] = v.y; xr[e + 2] = v.z; xr[e + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 64; ++e) xr[e] = 0.f;
  }
  P::group_sums(xr, g);

  for (; base < rows; base += stride) {
    typename P::Raw raw[R];
    bool ok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = base + (kwaves == 1 ? r * slots + slot : r);
      ok[r] = active && row < rows;
      if (ok[r]) raw[r] = P::load(w + (int64_t)row * row_bytes, pos);
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = ok[r] ? P::dot(raw[r], pos, xr, g) : 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = group_sum(acc[r], lanes_log2);
    if (kwaves == 1) {
      if (l == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int row = base + r * slots + slot;
          if (row < rows) y[row] = acc[r];
        }
      }
    } else {
      if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) partial[wave][r] = acc[r];
      }
      __syncthreads();
      if (threadIdx.x < R && base + (int)threadIdx.x < rows) {
        float v = 0.f;
        for (int q = 0; q < kwaves; ++q) v += partial[q][threadIdx.x];
        y[base + threadIdx.x] = v;
      }
      __syncthreads();
    }
  }
}

// F32 rows (the router): one float4 of W per lane per step.
template <int NT>
__global__ void __launch_bounds__(256)
gemv_f32_kernel(const float* __restrict__ w, int rows, int K, const float* __restrict__ x,
                int64_t x_stride, int ntok, float* __restrict__ y, int64_t y_stride) {
  extern __shared__ float smem[];
  float* xs = smem;
  for (int i = threadIdx.x; i < NT * K; i += blockDim.x) {
    const int tok = i / K, k = i - tok * K;
    xs[i] = tok < ntok ? x[tok * x_stride + k] : 0.f;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves_per_block = blockDim.x >> 6;
  const int n4 = K >> 2;
  for (int row = blockIdx.x * waves_per_block + wave; row < rows; row += gridDim.x * waves_per_block) {
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.f;
    const float4* wr = reinterpret_cast<const float4*>(w + (int64_t)row * K);
    for (int k4 = lane; k4 < n4; k4 += kWave) {
      const float4 a = wr[k4];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const float4 b = reinterpret_cast<const float4*>(xs + t * K)[k4];
        acc[t] = fmaf(a.x, b.x, acc[t]);
        acc[t] = fmaf(a.y, b.y, acc[t]);
        acc[t] = fmaf(a.z, b.z, acc[t]);
        acc[t] = fmaf(a.w, b.w, acc[t]);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float v = segment_sum<kWave>(acc[t]);
      if (lane == 0 && t < ntok) y[t * y_stride + row] = v;
    }
  }
}

// ------------------------------------------------------------------------
// Exact dequantisation (bit-identical to llambda.lisp:6815-6859, 6919-6978,
// 3965-4009): one thread per 32-weight unit, every product and difference
// rounded separately.
template <int TYPE>
__global__ void dequant_kernel(const uint8_t* __restrict__ w, int64_t row_bytes, int rows, int K,
                               float* __restrict__ out, const int* __restrict__ row_sel) {
#pragma clang fp contract(off)
  // row_sel: one row, its index read from device memory (a token's embedding)
  if (row_sel) w += (int64_t)(*row_sel) * row_bytes;
  const int units = K >> 5;
  const int64_t total = (int64_t)rows * units;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int row = (int)(i / units);
    const int u = (int)(i - (int64_t)row * units);
    const uint8_t* rp = w + (int64_t)row * row_bytes;
    float* o = out + (int64_t)row * K;
    if constexpr (TYPE == kQ4_K) {
      const auto raw = Unit<kQ4_K>::load(rp, u);
      const int t = u & 7, j = t >> 1, half = t & 1;
      int sc0, m0, sc1, m1;
      Unit<kQ4_K>::scale_min(raw.hdr, 2 * j, sc0, m0);
      Unit<kQ4_K>::scale_min(raw.hdr, 2 * j + 1, sc1, m1);
      const float d = half_bits_to_float(raw.hdr.x & 0xFFFFu);
      const float dmin = half_bits_to_float(raw.hdr.x >> 16);
      const float delta0 = d * (float)sc0, off0 = dmin * (float)m0;
      const float delta1 = d * (float)sc1, off1 = dmin * (float)m1;
      const uint32_t qw[4] = {raw.q.x, raw.q.y, raw.q.z, raw.q.w};
      const int xl = (u >> 3) * 256 + 64 * j + 16 * half;
      for (int b = 0; b < 16; ++b) {
        const uint32_t p = (qw[b >> 2] >> (8 * (b & 3))) & 0xFFu;
        const float pl = delta0 * (float)(p & 15u);
        const float ph = delta1 * (float)(p >> 4);
        o[xl + b] = pl - off0;
        o[xl + 32 + b] = ph - off1;
      }
    } else if constexpr (TYPE == kQ6_K) {
      const auto raw = Unit<kQ6_K>::load(rp, u);
      const int t = u & 7, h = t >> 2, part = (t >> 1) & 1, half = t & 1;
      const float d = half_bits_to_float(raw.dword & 0xFFFFu);
      const int ia = 8 * h + half + 2 * part;
      const float delta_a = d * (float)Unit<kQ6_K>::scale_at(raw.sc, ia);
      const float delta_b = d * (float)Unit<kQ6_K>::scale_at(raw.sc, ia + 4);
      const uint32_t lqw[4] = {raw.ql.x, raw.ql.y, raw.ql.z, raw.ql.w};
      const uint32_t hqw[4] = {raw.qh.x, raw.qh.y, raw.qh.z, raw.qh.w};
      const int xa = (u >> 3) * 256 + 128 * h + 32 * part + 16 * half;
      for (int b = 0; b < 16; ++b) {
        const uint32_t lq = (lqw[b >> 2] >> (8 * (b & 3))) & 0xFFu;
        const uint32_t hq = (hqw[b >> 2] >> (8 * (b & 3))) & 0xFFu;
        const int qa = (int)((lq & 15u) | (((hq >> (2 * part)) & 3u) << 4)) - 32;
        const int qb = (int)((lq >> 4) | (((hq >> (4 + 2 * part)) & 3u) << 4)) - 32;
        o[xa + b] = delta_a * (float)qa;
        o[xa + 64 + b] = delta_b * (float)qb;
      }
    } else if constexpr (TYPE == kQ8_0) {
      const auto raw = Unit<kQ8_0>::load(rp, u);
      const float d = half_bits_to_float(raw.w[0] & 0xFFFFu);
      for (int b = 0; b < 32; ++b) {
        const int byte = 2 + b;
        const int q = (int)(int8_t)((raw.w[byte >> 2] >> (8 * (byte & 3))) & 0xFFu);
        o[u * 32 + b] = d * (float)q;
      }
    } else if constexpr (TYPE == kQ5_0) {
      const auto raw = Unit<kQ5_0>::load(rp, u);
      const float d = half_bits_to_float(raw.w[0] & 0xFFFFu);
      const uint32_t qh = __builtin_amdgcn_alignbyte(raw.w[1], raw.w[0], 2);
      for (int b = 0; b < 16; ++b) {
        const int byte = 6 + b;
        const uint32_t p = (raw.w[byte >> 2] >> (8 * (byte & 3))) & 0xFFu;
        const int q0 = (int)((p & 15u) | (((qh >> b) & 1u) << 4)) - 16;
        const int q1 = (int)((p >> 4) | (((qh >> (b + 16)) & 1u) << 4)) - 16;
        o[u * 32 + b] = d * (float)q0;
        o[u * 32 + 16 + b] = d * (float)q1;
      }
    }
  }
}

// fp16 fields with exponent 31 (Inf/NaN) are rejected by the reference's
// decoder (llambda.lisp:727-728).  Finds the first block holding one.
template <int TYPE>
__global__ void validate_kernel(const uint8_t* __restrict__ w, int64_t nblocks,
                                unsigned long long* __restrict__ first_bad) {
  for (int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; b < nblocks;
       b += (int64_t)gridDim.x * blockDim.x) {
    const uint8_t* p = w + b * block_bytes(TYPE);
    bool bad;
    if constexpr (TYPE == kQ4_K) {
      const uint32_t h0 = p[0] | (p[1] << 8), h1 = p[2] | (p[3] << 8);
      bad = ((h0 >> 10) & 31u) == 31u || ((h1 >> 10) & 31u) == 31u;
    } else if constexpr (TYPE == kQ6_K) {
      const uint32_t h0 = p[208] | (p[209] << 8);
      bad = ((h0 >> 10) & 31u) == 31u;
    } else {
      const uint32_t h0 = p[0] | (p[1] << 8);
      bad = ((h0 >> 10) & 31u) == 31u;
    }
    if (bad) atomicMin(first_bad, (unsigned long long)b);
  }
}

// ------------------------------------------------------------------------
// Host launchers

int device_cu_count() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (cus <= 0) cus = 256;
  }
  return cus;
}

template <typename Kernel>
static hipError_t launch_with_lds(Kernel k, int grid, size_t lds, hipStream_t stream,
                                  auto... args) {
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(k, dim3(grid), dim3(256), lds, stream, args...);
  return hipGetLastError();
}

template <int TYPE, int NT, int R>
static hipError_t launch_packed(const GemvProblem& p, hipStream_t stream) {
  const int lpr_log2 = lanes_per_row_log2((int)p.columns);
  const int slots = kWave >> lpr_log2;
  const int rows_per_block = 4 * slots * R;
  const int needed = (int)((p.rows + rows_per_block - 1) / rows_per_block);
  const size_t lds = (size_t)NT * (p.columns + (p.columns >> 4)) * sizeof(float);
  // Enough workgroups for 8 per CU; beyond that, workgroups loop over rows so
  // the activation staging is amortised.
  const int grid = std::max(1, std::min(needed, device_cu_count() * 8));
  return launch_with_lds(gemv_kernel<TYPE, NT, R>, grid, lds, stream, p.weights, p.row_bytes,
                         (int)p.rows, (int)p.columns, p.x, p.x_stride, p.tokens, p.y, p.y_stride,
                         lpr_log2);
}

template <int NT>
static hipError_t launch_f32(const GemvProblem& p, hipStream_t stream) {
  const int needed = (int)((p.rows + 3) / 4);
  const size_t lds = (size_t)NT * p.columns * sizeof(float);
  const int grid = std::max(1, std::min(needed, device_cu_count() * 8));
  return launch_with_lds(gemv_f32_kernel<NT>, grid, lds, stream,
                         reinterpret_cast<const float*>(p.weights), (int)p.rows, (int)p.columns,
                         p.x, p.x_stride, p.tokens, p.y, p.y_stride);
}

template <int NT>
static hipError_t launch_nt(const GemvProblem& p, hipStream_t stream) {
  switch (p.type) {
    case kQ4_K: return launch_packed<kQ4_K, NT, 2>(p, stream);
    case kQ6_K: return launch_packed<kQ6_K, NT, 2>(p, stream);
    case kQ5_0: return launch_packed<kQ5_0, NT, 2>(p, stream);
    case kQ8_0: return launch_packed<kQ8_0, NT, 2>(p, stream);
    case kF32: return launch_f32<NT>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int TYPE, int R>
static hipError_t launch_rows(const GemvProblem& p, hipStream_t stream) {
  const int positions = (int)(p.columns / 64);
  int lanes_log2 = 0, kwaves = 1;
  if (positions <= 64) {
    while ((1 << lanes_log2) < positions) ++lanes_log2;
  } else {
    lanes_log2 = 6;
    kwaves = (positions + 63) / 64;
  }
  const int block = kwaves == 1 ? 256 : 64 * kwaves;
  const auto kernel = gemv_rows_kernel<TYPE, R>;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kernel),
                                                   block, 0) != hipSuccess || per_cu < 1)
    per_cu = 1;
  const int rows_per_block = kwaves == 1 ? (block / 64) * (kWave >> lanes_log2) * R : R;
  const int needed = (int)((p.rows + rows_per_block - 1) / rows_per_block);
  const int grid = std::max(1, std::min(needed, device_cu_count() * per_cu));
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(block), 0, stream, p.weights, p.row_bytes,
                     (int)p.rows, positions, p.x, p.y, lanes_log2, kwaves);
  return hipGetLastError();
}

// The row-streaming kernel serves one token when K is a multiple of 64.
static bool rows_path(const GemvProblem& p) {
  return p.tokens == 1 && p.type != kF32 && p.columns % 64 == 0 &&
         p.columns / 64 <= 64 * kRowsMaxWaves;
}

#ifndef LLHIP_GEMV_MFMA
#define LLHIP_GEMV_MFMA 1
#endif

hipError_t gemv_launch(const GemvProblem& p, hipStream_t stream) {
  if (LLHIP_GEMV_MFMA && gemv_mfma_supported(p)) return gemv_mfma_launch(p, stream);
  if (rows_path(p)) {
    switch (p.type) {
      case kQ4_K: return launch_rows<kQ4_K, LLHIP_ROWS_Q4K>(p, stream);
      case kQ6_K: return launch_rows<kQ6_K, LLHIP_ROWS_Q6K>(p, stream);
      case kQ5_0: return launch_rows<kQ5_0, 2>(p, stream);
      case kQ8_0: return launch_rows<kQ8_0, 2>(p, stream);
      default: break;
    }
  }
  // Tokens are processed up to NT at a time (each chunk re-reads the
  // weights); NT is capped so the staged activations fit in LDS.
  const size_t per_token = p.type == kF32 ? (size_t)p.columns * sizeof(float)
                                          : (size_t)(p.columns + (p.columns >> 4)) * sizeof(float);
  const int fit = (int)std::min<size_t>(4, kMaxLdsBytes / per_token);
  if (fit < 1) return hipErrorInvalidValue;
  const int chunk = fit >= 4 ? 4 : fit >= 2 ? 2 : 1;
  GemvProblem q = p;
  for (int t0 = 0; t0 < p.tokens; t0 += chunk) {
    q.tokens = std::min(chunk, p.tokens - t0);
    q.x = p.x + (int64_t)t0 * p.x_stride;
    q.y = p.y + (int64_t)t0 * p.y_stride;
    hipError_t e;
    if (q.tokens == 1) e = launch_nt<1>(q, stream);
    else if (q.tokens == 2) e = launch_nt<2>(q, stream);
    else e = launch_nt<4>(q, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t dequant_launch(int type, const uint8_t* w, int64_t row_bytes, int64_t rows,
                          int64_t columns, float* out, hipStream_t stream, const int* row_sel) {
  const int64_t units = rows * (columns >> 5);
  const int grid = (int)std::min<int64_t>((units + 255) / 256, 65536);
  switch (type) {
    case kQ4_K:
      hipLaunchKernelGGL(dequant_kernel<kQ4_K>, dim3(grid), dim3(256), 0, stream, w, row_bytes,
                         (int)rows, (int)columns, out, row_sel);
      break;
    case kQ6_K:
      hipLaunchKernelGGL(dequant_kernel<kQ6_K>, dim3(grid), dim3(256), 0, stream, w, row_bytes,
                         (int)rows, (int)columns, out, row_sel);
      break;
    case kQ5_0:
      hipLaunchKernelGGL(dequant_kernel<kQ5_0>, dim3(grid), dim3(256), 0, stream, w, row_bytes,
                         (int)rows, (int)columns, out, row_sel);
      break;
    case kQ8_0:
      hipLaunchKernelGGL(dequant_kernel<kQ8_0>, dim3(grid), dim3(256), 0, stream, w, row_bytes,
                         (int)rows, (int)columns, out, row_sel);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t validate_launch(int type, const uint8_t* w, int64_t nblocks,
                           unsigned long long* first_bad, hipStream_t stream) {
  const int grid = (int)std::max<int64_t>(1, std::min<int64_t>((nblocks + 255) / 256, 16384));
  switch (type) {
    case kQ4_K:
      hipLaunchKernelGGL(validate_kernel<kQ4_K>, dim3(grid), dim3(256), 0, stream, w, nblocks, first_bad);
      break;
    case kQ6_K:
      hipLaunchKernelGGL(validate_kernel<kQ6_K>, dim3(grid), dim3(256), 0, stream, w, nblocks, first_bad);
      break;
    case kQ5_0:
      hipLaunchKernelGGL(validate_kernel<kQ5_0>, dim3(grid), dim3(256), 0, stream, w, nblocks, first_bad);
      break;
    case kQ8_0:
      hipLaunchKernelGGL(validate_kernel<kQ8_0>, dim3(grid), dim3(256), 0, stream, w, nblocks, first_bad);
      break;
    default: return hipSuccess;  // F32 has no fp16 fields
  }
  return hipGetLastError();
}

}  // namespace llhip

// ------------------------------------------------------- streaming read
// The read rate this device sustains over one contiguous buffer: the
// ceiling the GEMV kernels are measured against.  Each wave streams one
// contiguous slice with 16-byte non-temporal loads (the policy the weight
// streams use), four in flight per lane; the XOR of everything a wave read
// goes to out[wave], so the loads cannot be dropped.
namespace llhip {

constexpr int kStreamWaves = 8;

__global__ void __launch_bounds__(64 * kStreamWaves)
stream_read_kernel(const u32x4a4* __restrict__ p, int64_t n16, uint32_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * kStreamWaves + (threadIdx.x >> 6);
  const int64_t waves = (int64_t)gridDim.x * kStreamWaves;
  const int64_t per = (((n16 + waves - 1) / waves) + 63) & ~(int64_t)63;  // whole wave rows
  const int64_t begin = wave * per;
  const int64_t end = begin + per < n16 ? begin + per : n16;
  uint32_t acc = 0;
  int64_t j = begin;
  for (; j + 256 <= end; j += 256) {
    const u32x4a4 a = __builtin_nontemporal_load(p + j + lane),
                  b = __builtin_nontemporal_load(p + j + 64 + lane),
                  c = __builtin_nontemporal_load(p + j + 128 + lane),
                  d = __builtin_nontemporal_load(p + j + 192 + lane);
    acc ^= (a.x ^ a.y ^ a.z ^ a.w) ^ (b.x ^ b.y ^ b.z ^ b.w) ^ (c.x ^ c.y ^ c.z ^ c.w) ^
           (d.x ^ d.y ^ d.z ^ d.w);
  }
  for (; j < end; j += 64)
    if (j + lane < end) {
      const u32x4a4 a = __builtin_nontemporal_load(p + j + lane);
      acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
  for (int off = 32; off; off >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, off);
  if (lane == 0) out[wave] = acc;
}

hipError_t stream_read_launch(const void* data, size_t bytes, uint32_t* out, hipStream_t stream) {
  if (!data || !out || bytes == 0 || bytes % 16 || reinterpret_cast<uintptr_t>(data) % 16)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(stream_read_kernel, dim3(kStreamReadWords / kStreamWaves),
                     dim3(64 * kStreamWaves), 0, stream, static_cast<const u32x4a4*>(data),
                     (int64_t)(bytes / 16), out);
  return hipGetLastError();
}

}  // namespace llhip
