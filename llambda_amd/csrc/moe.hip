// moe.hip -- routed-MoE feed-forward kernels for gfx950 (see moe.h).
#include "moe.h"
#include "activations.h"

#include <algorithm>
#include <cfloat>
#include <climits>

namespace llhip {

// ------------------------------------------------------------------ top-k
// select-top-k-logits-into (llambda.lisp:5265-5292) keeps, in descending
// order, the k largest logits strictly above most-negative-single-float,
// lower index first among equal values, never NaN; unfilled slots stay
// (-1, -FLT_MAX).  Here one wavefront holds JPL logits per lane and takes k
// rounds of a wave-wide (value desc, index asc) arg-max.  `bias` (optional)
// is added first and the biased logits are written back.
template <int JPL>
__device__ __forceinline__ void wave_select(float* lg, const float* bias, int E, int K, int lane,
                                            int* out_idx, float* out_val) {
  float vals[JPL];
#pragma unroll
  for (int j = 0; j < JPL; ++j) {
    const int e = lane + kWave * j;
    float v = -INFINITY;
    if (e < E) {
      float raw = lg[e];
      if (bias) {
        raw = __fadd_rn(raw, bias[e]);
        lg[e] = raw;
      }
      v = raw > -FLT_MAX ? raw : -INFINITY;  // NaN, -inf, -FLT_MAX never qualify
    }
    vals[j] = v;
  }
  for (int r = 0; r < K; ++r) {
    float bv = -INFINITY;
    int bi = INT_MAX;
#pragma unroll
    for (int j = 0; j < JPL; ++j) {
      if (vals[j] > bv) {
        bv = vals[j];
        bi = lane + kWave * j;
      }
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, kWave);
      const int oi = __shfl_xor(bi, off, kWave);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (bi != INT_MAX && (bi & (kWave - 1)) == lane) {
#pragma unroll
      for (int j = 0; j < JPL; ++j)
        if (j == (bi >> 6)) vals[j] = -INFINITY;
    }
    if (lane == 0) {
      out_idx[r] = bi == INT_MAX ? -1 : bi;
      out_val[r] = bi == INT_MAX ? -FLT_MAX : bv;
    }
  }
}

template <int JPL>
__global__ void __launch_bounds__(256) topk_kernel(const float* __restrict__ logits, int n, int k,
                                                   int batch, int* __restrict__ idx,
                                                   float* __restrict__ val) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= batch) return;
  wave_select<JPL>(const_cast<float*>(logits + (int64_t)t * n), nullptr, n, k,
                   threadIdx.x & 63, idx + (int64_t)t * k, val + (int64_t)t * k);
}

// Top-k plus the gating weights of llambda.lisp:5365-5379 (qwen3next:
// sigmoid, renormalise, error when the sum is not positive) or 5894-5913
// (nemotron: bias before selection, sigmoid, optional renormalise, scale);
// then the expert histogram.
template <int JPL>
__global__ void __launch_bounds__(256) topk_gate_kernel(MoePlan p, int tokens) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= tokens) return;
  const int E = p.experts, K = p.top_k;
  float* lg = p.logits + (int64_t)t * (E + 1);
  int* ti = p.top_idx + (int64_t)t * K;
  float* tw = p.top_w + (int64_t)t * K;
  wave_select<JPL>(lg, p.variant == kNemotronH ? p.bias : nullptr, E, K, lane, ti, tw);
  if (lane != 0) return;
  int err = 0;
  float sum = 0.f;
  for (int r = 0; r < K; ++r) {
    if (ti[r] < 0) err |= 1;
    const float w = sigmoid_ref(tw[r]);
    tw[r] = w;
    sum = sum + w;
  }
  if (p.variant == kQwen3Next || p.weights_norm) {
    if (!(sum > 0.f)) {
      err |= 2;
    } else {
      for (int r = 0; r < K; ++r) tw[r] = tw[r] / sum;
    }
  }
  if (p.variant == kNemotronH)
    for (int r = 0; r < K; ++r) tw[r] = p.weights_scale * tw[r];
  p.shared_w[t] = p.variant == kQwen3Next ? sigmoid_ref(lg[E]) : 1.f;
  for (int r = 0; r < K; ++r)
    if (ti[r] >= 0) atomicAdd(&p.counts[ti[r]], 1);
  if (err) atomicOr(p.error, err);
}

// ------------------------------------------------------------ scan/scatter
// One workgroup: exclusive scans of the expert histogram (pairs and chunks),
// the chunk table, and the permutation that groups (token, rank) pairs by
// expert.  Pair id p = token * k + rank; the shared expert's pairs are
// tokens * k + token.  Leaves the histogram zeroed for the next run.
constexpr int kScanThreads = 1024;

__global__ void __launch_bounds__(kScanThreads) moe_scan_kernel(MoePlan p, int tokens, int nt,
                                                                int has_shared) {
  __shared__ int s_cnt[kMoeMaxExperts];
  __shared__ int s_off[kMoeMaxExperts + 1];
  __shared__ int s_coff[kMoeMaxExperts + 1];
  __shared__ int s_cur[kMoeMaxExperts];
  __shared__ int s_part[kScanThreads];
  __shared__ int s_cpart[kScanThreads];
  const int E = p.experts, K = p.top_k, tid = threadIdx.x;
  for (int e = tid; e < E; e += kScanThreads) {
    s_cnt[e] = p.counts[e];
    s_cur[e] = 0;
    p.counts[e] = 0;
  }
  __syncthreads();
  const int per = (E + kScanThreads - 1) / kScanThreads;
  const int e0 = tid * per, e1 = min(e0 + per, E);
  int sum = 0, csum = 0;
  for (int e = e0; e < e1; ++e) {
    sum += s_cnt[e];
    csum += (s_cnt[e] + nt - 1) / nt;
  }
  s_part[tid] = sum;
  s_cpart[tid] = csum;
  __syncthreads();
  for (int off = 1; off < kScanThreads; off <<= 1) {
    const int v = tid >= off ? s_part[tid - off] : 0;
    const int cv = tid >= off ? s_cpart[tid - off] : 0;
    __syncthreads();
    s_part[tid] += v;
    s_cpart[tid] += cv;
    __syncthreads();
  }
  int run = tid ? s_part[tid - 1] : 0, crun = tid ? s_cpart[tid - 1] : 0;
  for (int e = e0; e < e1; ++e) {
    s_off[e] = run;
    s_coff[e] = crun;
    run += s_cnt[e];
    crun += (s_cnt[e] + nt - 1) / nt;
  }
  if (tid == kScanThreads - 1) {
    s_off[E] = s_part[tid];
    s_coff[E] = s_cpart[tid];
  }
  __syncthreads();
  const int routed_pairs = s_off[E], routed_chunks = s_coff[E];
  for (int e = tid; e < E; e += kScanThreads) {
    const int c = s_cnt[e];
    for (int j = 0; j * nt < c; ++j) {
      MoeChunk ch;
      ch.expert = e;
      ch.start = s_off[e] + j * nt;
      ch.count = min(nt, c - j * nt);
      p.chunks[s_coff[e] + j] = ch;
    }
  }
  const int P = tokens * K;
  int shared_chunks = 0;
  if (has_shared) {
    shared_chunks = (tokens + nt - 1) / nt;
    for (int j = tid; j < shared_chunks; j += kScanThreads) {
      MoeChunk ch;
      ch.expert = 0;
      ch.start = routed_pairs + j * nt;
      ch.count = min(nt, tokens - j * nt);
      p.chunks[routed_chunks + j] = ch;
    }
    for (int t = tid; t < tokens; t += kScanThreads) p.perm[routed_pairs + t] = P + t;
  }
  if (tid == 0) {
    p.chunk_counts[0] = routed_chunks;
    p.chunk_counts[1] = shared_chunks;
  }
  for (int q = tid; q < P; q += kScanThreads) {
    const int e = p.top_idx[q];
    if (e >= 0 && e < E) {
      const int pos = atomicAdd(&s_cur[e], 1);
      p.perm[s_off[e] + pos] = q;
    }
  }
}

// ------------------------------------------------------- grouped experts
// One group is either the routed experts (slabs of E experts, chunk table
// entries [0, chunk_counts[0])) or the shared expert (one slab, entries
// after the routed ones).
struct MoeGroup {
  int group;              // 0 routed, 1 shared
  const uint8_t* gate;    // qwen3next gate rows (null for nemotron)
  const uint8_t* up;
  int64_t up_row_bytes;
  int64_t up_expert_stride;  // bytes between experts' gate/up slabs
  int ffn;                   // rows per expert of gate/up = columns of down
  const uint8_t* down;
  int64_t down_row_bytes;
  int64_t down_expert_stride;
  int act_stride;            // floats per pair row of act
  int up_iters;              // row iterations per workgroup (up kernel)
  int down_iters;            // row iterations per workgroup (down kernel)
};

template <int NT>
__device__ __forceinline__ bool load_chunk(const MoePlan& p, const MoeGroup& g, int tokens,
                                           MoeChunk& c, int* pair_of) {
  const int nchunks = p.chunk_counts[g.group];
  if ((int)blockIdx.x >= nchunks) return false;
  const int cbase = g.group == 0 ? 0 : p.chunk_counts[0];
  c = p.chunks[cbase + blockIdx.x];
  if (threadIdx.x < NT)
    pair_of[threadIdx.x] = (int)threadIdx.x < c.count ? p.perm[c.start + threadIdx.x] : -1;
  (void)tokens;
  return true;
}

// gate/up rows of one expert against the chunk's tokens, activation fused:
// qwen3next  act = fl(silu(g) * u)  (llambda.lisp:5386-5401)
// nemotron   act = relu(u)^2        (llambda.lisp:5921-5926)
template <int TU, int NT, int VARIANT>
__global__ void __launch_bounds__(256) moe_up_kernel(MoePlan p, MoeGroup g,
                                                     const float* __restrict__ x, int tokens) {
#pragma clang fp contract(off)
  __shared__ int pair_of[NT];
  __shared__ const float* src[NT];
  MoeChunk c;
  if (!load_chunk<NT>(p, g, tokens, c, pair_of)) return;
  const int H = p.hidden, K = p.top_k, P = tokens * K;
  __syncthreads();
  if (threadIdx.x < NT) {
    const int q = pair_of[threadIdx.x];
    src[threadIdx.x] = q < 0 ? nullptr : x + (int64_t)(q < P ? q / K : q - P) * H;
  }
  __syncthreads();
  extern __shared__ float smem[];
  float* xs = smem;
  float* xg = smem + NT * H;
  stage_rows<NT>(xs, xg, src, H);
  __syncthreads();
  const XView xv{xs, xg, H, H >> 4};

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lpr_log2 = lanes_per_row_log2(H);
  const int lpr = 1 << lpr_log2, slot = lane >> lpr_log2, l = lane & (lpr - 1);
  const int slots = kWave >> lpr_log2;
  const int units = H >> 5;
  const uint8_t* gate_e = g.gate + (int64_t)c.expert * g.up_expert_stride;
  const uint8_t* up_e = g.up + (int64_t)c.expert * g.up_expert_stride;
  // rows handled per wave iteration: qwen3next 1 (gate+up), nemotron 2
  constexpr int ITEMS = VARIANT == kQwen3Next ? 1 : 2;
  const int per_iter = 4 * slots * ITEMS;
  const int tile0 = blockIdx.y * per_iter * g.up_iters;
  for (int it = 0; it < g.up_iters; ++it) {
    const int f0 = tile0 + it * per_iter + (wave * slots + slot) * ITEMS;
    const uint8_t* rp[2];
    bool valid[2];
    int f[2];
    if constexpr (VARIANT == kQwen3Next) {
      f[0] = f[1] = f0;
      valid[0] = valid[1] = f0 < g.ffn;
      rp[0] = gate_e + (int64_t)(valid[0] ? f0 : 0) * g.up_row_bytes;
      rp[1] = up_e + (int64_t)(valid[1] ? f0 : 0) * g.up_row_bytes;
    } else {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        f[r] = f0 + r;
        valid[r] = f[r] < g.ffn;
        rp[r] = up_e + (int64_t)(valid[r] ? f[r] : 0) * g.up_row_bytes;
      }
    }
    float acc[2][NT];
    rows_dot<TU, NT, 2>(rp, valid, l, lpr, units, xv, acc);
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[r][t] = segment_sum_dyn(acc[r][t], lpr);
    if (l == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int q = pair_of[t];
        if (q < 0) continue;
        float* row = p.act + (int64_t)q * g.act_stride;
        if constexpr (VARIANT == kQwen3Next) {
          if (valid[0]) row[f0] = silu_ref(acc[0][t]) * acc[1][t];
        } else {
#pragma unroll
          for (int r = 0; r < 2; ++r)
            if (valid[r]) row[f[r]] = relu2_ref(acc[r][t]);
        }
      }
    }
  }
}

// down rows of one expert against the chunk's activations, one output row
// per pair: down_out[pair][i] (llambda.lisp:5402-5408, 5927-5931).
template <int TD, int NT>
__global__ void __launch_bounds__(256) moe_down_kernel(MoePlan p, MoeGroup g, int tokens) {
  __shared__ int pair_of[NT];
  __shared__ const float* src[NT];
  MoeChunk c;
  if (!load_chunk<NT>(p, g, tokens, c, pair_of)) return;
  const int H = p.hidden, F = g.ffn;
  __syncthreads();
  if (threadIdx.x < NT) {
    const int q = pair_of[threadIdx.x];
    src[threadIdx.x] = q < 0 ? nullptr : p.act + (int64_t)q * g.act_stride;
  }
  __syncthreads();
  extern __shared__ float smem[];
  float* xs = smem;
  float* xg = smem + NT * F;
  stage_rows<NT>(xs, xg, src, F);
  __syncthreads();
  const XView xv{xs, xg, F, F >> 4};

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lpr_log2 = lanes_per_row_log2(F);
  const int lpr = 1 << lpr_log2, slot = lane >> lpr_log2, l = lane & (lpr - 1);
  const int slots = kWave >> lpr_log2;
  const int units = F >> 5;
  const uint8_t* down_e = g.down + (int64_t)c.expert * g.down_expert_stride;
  constexpr int R = 2;
  const int per_iter = 4 * slots * R;
  const int tile0 = blockIdx.y * per_iter * g.down_iters;
  for (int it = 0; it < g.down_iters; ++it) {
    const int i0 = tile0 + it * per_iter + (wave * slots + slot) * R;
    const uint8_t* rp[R];
    bool valid[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      valid[r] = i0 + r < H;
      rp[r] = down_e + (int64_t)(valid[r] ? i0 + r : 0) * g.down_row_bytes;
    }
    float acc[R][NT];
    rows_dot<TD, NT, R>(rp, valid, l, lpr, units, xv, acc);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[r][t] = segment_sum_dyn(acc[r][t], lpr);
    if (l == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int q = pair_of[t];
        if (q < 0) continue;
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (valid[r]) p.down_out[(int64_t)q * H + i0 + r] = acc[r][t];
      }
    }
  }
}

// Weighted combine in rank order, then the shared expert, every product and
// sum rounded separately as in vector-add-scaled-in-place /
// vector-add-bias-in-place (llambda.lisp:3465-3489; 5359, 5409, 5426, 5914,
// 5932, 5949).
__global__ void __launch_bounds__(256) moe_combine_kernel(MoePlan p, float* __restrict__ y,
                                                          int tokens, int has_shared) {
#pragma clang fp contract(off)
  const int t = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const int H = p.hidden, K = p.top_k;
  if (i >= H) return;
  float acc = 0.f;
  for (int r = 0; r < K; ++r) {
    const int q = t * K + r;
    if (p.top_idx[q] < 0) continue;
    const float prod = p.top_w[q] * p.down_out[(int64_t)q * H + i];
    acc = acc + prod;
  }
  if (has_shared) {
    const float d = p.down_out[(int64_t)(tokens * K + t) * H + i];
    if (p.variant == kQwen3Next) {
      const float prod = p.shared_w[t] * d;
      acc = acc + prod;
    } else {
      acc = acc + d;
    }
  }
  y[(int64_t)t * H + i] = acc;
}

__global__ void moe_reset_kernel(int* counts, int n, int* error) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    counts[i] = 0;
  if (blockIdx.x == 0 && threadIdx.x == 0) *error = 0;
}

// ------------------------------------------------------------------ host

int64_t moe_max_chunks(const MoePlan& p, int64_t tokens, int nt) {
  const int64_t pairs = tokens * p.top_k;
  return pairs / nt + std::min<int64_t>(p.experts, pairs) + (tokens + nt - 1) / nt + 1;
}

template <typename Kernel, typename... Args>
static hipError_t launch(Kernel k, dim3 grid, dim3 block, size_t lds, hipStream_t s, Args... args) {
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(k, grid, block, lds, s, args...);
  return hipGetLastError();
}

static int jpl_for(int E) {
  int j = 1;
  while (j * kWave < E) j <<= 1;
  return j;
}

template <int NT, int VARIANT>
static hipError_t launch_up(const MoePlan& p, const MoeGroup& g, int type, int chunks,
                            const float* x, int tokens, hipStream_t s) {
  const int slots = kWave >> lanes_per_row_log2(p.hidden);
  const int items = VARIANT == kQwen3Next ? 1 : 2;
  const int per_block = 4 * slots * items * g.up_iters;
  const dim3 grid(chunks, (g.ffn + per_block - 1) / per_block);
  const size_t lds = (size_t)NT * (p.hidden + (p.hidden >> 4)) * sizeof(float);
  switch (type) {
    case kQ4_K: return launch(moe_up_kernel<kQ4_K, NT, VARIANT>, grid, dim3(256), lds, s, p, g, x, tokens);
    case kQ6_K: return launch(moe_up_kernel<kQ6_K, NT, VARIANT>, grid, dim3(256), lds, s, p, g, x, tokens);
    case kQ5_0: return launch(moe_up_kernel<kQ5_0, NT, VARIANT>, grid, dim3(256), lds, s, p, g, x, tokens);
    case kQ8_0: return launch(moe_up_kernel<kQ8_0, NT, VARIANT>, grid, dim3(256), lds, s, p, g, x, tokens);
    default: return hipErrorInvalidValue;
  }
}

template <int NT>
static hipError_t launch_down(const MoePlan& p, const MoeGroup& g, int type, int chunks,
                              int tokens, hipStream_t s) {
  const int slots = kWave >> lanes_per_row_log2(g.ffn);
  const int per_block = 4 * slots * 2 * g.down_iters;
  const dim3 grid(chunks, (p.hidden + per_block - 1) / per_block);
  const size_t lds = (size_t)NT * (g.ffn + (g.ffn >> 4)) * sizeof(float);
  switch (type) {
    case kQ4_K: return launch(moe_down_kernel<kQ4_K, NT>, grid, dim3(256), lds, s, p, g, tokens);
    case kQ6_K: return launch(moe_down_kernel<kQ6_K, NT>, grid, dim3(256), lds, s, p, g, tokens);
    case kQ5_0: return launch(moe_down_kernel<kQ5_0, NT>, grid, dim3(256), lds, s, p, g, tokens);
    case kQ8_0: return launch(moe_down_kernel<kQ8_0, NT>, grid, dim3(256), lds, s, p, g, tokens);
    default: return hipErrorInvalidValue;
  }
}

static int64_t row_bytes_of(int type, int64_t columns) {
  return columns / block_weights(type) * block_bytes(type);
}

template <int NT>
static hipError_t launch_groups(const MoePlan& p, const float* x, int tokens, hipStream_t s) {
  const int has_shared = p.shared_ffn > 0;
  const int act_stride = std::max(p.ffn, p.shared_ffn);
  const int64_t pairs = (int64_t)tokens * p.top_k;
  const int routed_chunks = (int)(pairs / NT + std::min<int64_t>(p.experts, pairs));
  const int shared_chunks = (tokens + NT - 1) / NT;
  MoeGroup routed{};
  routed.group = 0;
  routed.gate = p.gate;
  routed.up = p.up;
  routed.up_row_bytes = row_bytes_of(p.up_type, p.hidden);
  routed.up_expert_stride = routed.up_row_bytes * p.ffn;
  routed.ffn = p.ffn;
  routed.down = p.down;
  routed.down_row_bytes = row_bytes_of(p.down_type, p.ffn);
  routed.down_expert_stride = routed.down_row_bytes * p.hidden;
  routed.act_stride = act_stride;
  routed.up_iters = 4;
  routed.down_iters = 4;
  MoeGroup shared = routed;
  shared.group = 1;
  shared.gate = p.sh_gate;
  shared.up = p.sh_up;
  shared.up_row_bytes = row_bytes_of(p.sh_up_type, p.hidden);
  shared.up_expert_stride = 0;
  shared.ffn = p.shared_ffn;
  shared.down = p.sh_down;
  shared.down_row_bytes = row_bytes_of(p.sh_down_type, p.shared_ffn);
  shared.down_expert_stride = 0;

  hipError_t e;
  if (p.variant == kQwen3Next) {
    e = launch_up<NT, kQwen3Next>(p, routed, p.up_type, routed_chunks, x, tokens, s);
    if (e == hipSuccess && has_shared)
      e = launch_up<NT, kQwen3Next>(p, shared, p.sh_up_type, shared_chunks, x, tokens, s);
  } else {
    e = launch_up<NT, kNemotronH>(p, routed, p.up_type, routed_chunks, x, tokens, s);
    if (e == hipSuccess && has_shared)
      e = launch_up<NT, kNemotronH>(p, shared, p.sh_up_type, shared_chunks, x, tokens, s);
  }
  if (e != hipSuccess) return e;
  e = launch_down<NT>(p, routed, p.down_type, routed_chunks, tokens, s);
  if (e == hipSuccess && has_shared)
    e = launch_down<NT>(p, shared, p.sh_down_type, shared_chunks, tokens, s);
  return e;
}

// Token-tile count (16 tokens each) of the grouped MFMA chunks: enough to
// cover the average (token, rank) pairs per expert, at most 4.
static int moe_mfma_tiles(const MoePlan& p, int tokens) {
  if (tokens == 1) return 0;  // the decode pipeline: one token per chunk
  const int64_t avg = ((int64_t)tokens * p.top_k + p.experts - 1) / p.experts;
  return avg <= 16 ? 1 : avg <= 40 ? 2 : 4;
}

// The multi-token forward on MFMA (moe_mfma.hip): split x, router GEMM,
// top-k, scan, grouped gate/up and down products, combine.
static hipError_t moe_forward_mfma(const MoePlan& p, const float* x, float* y, int tokens,
                                   hipStream_t s) {
  const int has_shared = p.shared_ffn > 0;
  const int H = p.hidden, E = p.experts, K = p.top_k;
  const int act_w = std::max(p.ffn, p.shared_ffn);
  const int64_t xs_stride = H / 16, as_stride = act_w / 16;
  hipError_t e = split_rows_launch(x, tokens, H, p.xq, 2 * (int64_t)H, p.xsum, xs_stride, s);
  if (e != hipSuccess) return e;
  const int er = E + ((p.variant == kQwen3Next && has_shared) ? 1 : 0);
  e = router_mfma_launch(x, tokens, p.router, er, H, p.logits, E + 1, s);
  if (e != hipSuccess) return e;
  const dim3 tgrid((tokens + 3) / 4);
  switch (jpl_for(E)) {
    case 1: e = launch(topk_gate_kernel<1>, tgrid, dim3(256), 0, s, p, tokens); break;
    case 2: e = launch(topk_gate_kernel<2>, tgrid, dim3(256), 0, s, p, tokens); break;
    case 4: e = launch(topk_gate_kernel<4>, tgrid, dim3(256), 0, s, p, tokens); break;
    case 8: e = launch(topk_gate_kernel<8>, tgrid, dim3(256), 0, s, p, tokens); break;
    case 16: e = launch(topk_gate_kernel<16>, tgrid, dim3(256), 0, s, p, tokens); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess) return e;
  const int mt = moe_mfma_tiles(p, tokens), nt = 16 * std::max(mt, 1);
  e = launch(moe_scan_kernel, dim3(1), dim3(kScanThreads), 0, s, p, tokens, nt, has_shared);
  if (e != hipSuccess) return e;
  const int64_t pairs = (int64_t)tokens * K;
  const int routed_chunks = (int)(pairs / nt + std::min<int64_t>(E, pairs));
  const int shared_chunks = (tokens + nt - 1) / nt;

  MoeGemmArgs up{};
  up.chunks = p.chunks;
  up.chunk_counts = p.chunk_counts;
  up.perm = p.perm;
  up.pairs = (int)pairs;
  up.top_k = K;
  up.a_by_token = 1;
  up.aq = p.xq;
  up.aq_stride = 2 * (int64_t)H;
  up.as = p.xsum;
  up.as_stride = xs_stride;
  up.K = H;
  up.oq = p.aq;
  up.oq_stride = 2 * (int64_t)act_w;
  up.os = p.asum;
  up.os_stride = as_stride;
  const int epi = p.variant == kQwen3Next ? kEpiSwiglu : kEpiRelu2;

  MoeGemmArgs a = up;
  a.group = 0;
  a.w0 = p.variant == kQwen3Next ? p.gate : p.up;
  a.w1 = p.up;
  a.row_bytes = row_bytes_of(p.up_type, H);
  a.expert_stride = a.row_bytes * p.ffn;
  a.N = p.ffn;
  e = moe_gemm_launch(p.up_type, epi, a, mt, routed_chunks, s);
  if (e != hipSuccess) return e;
  if (has_shared) {
    a = up;
    a.group = 1;
    a.w0 = p.variant == kQwen3Next ? p.sh_gate : p.sh_up;
    a.w1 = p.sh_up;
    a.row_bytes = row_bytes_of(p.sh_up_type, H);
    a.expert_stride = 0;
    a.N = p.shared_ffn;
    e = moe_gemm_launch(p.sh_up_type, epi, a, mt, shared_chunks, s);
    if (e != hipSuccess) return e;
  }

  MoeGemmArgs down{};
  down.chunks = p.chunks;
  down.chunk_counts = p.chunk_counts;
  down.perm = p.perm;
  down.pairs = (int)pairs;
  down.top_k = K;
  down.a_by_token = 0;
  down.aq = p.aq;
  down.aq_stride = 2 * (int64_t)act_w;
  down.as = p.asum;
  down.as_stride = as_stride;
  down.N = H;
  down.out = p.down_out;
  down.out_stride = H;
  a = down;
  a.group = 0;
  a.K = p.ffn;
  a.w0 = p.down;
  a.row_bytes = row_bytes_of(p.down_type, p.ffn);
  a.expert_stride = a.row_bytes * H;
  e = moe_gemm_launch(p.down_type, kEpiDown, a, mt, routed_chunks, s);
  if (e != hipSuccess) return e;
  if (has_shared) {
    a = down;
    a.group = 1;
    a.K = p.shared_ffn;
    a.w0 = p.sh_down;
    a.row_bytes = row_bytes_of(p.sh_down_type, p.shared_ffn);
    a.expert_stride = 0;
    e = moe_gemm_launch(p.sh_down_type, kEpiDown, a, mt, shared_chunks, s);
    if (e != hipSuccess) return e;
  }
  return launch(moe_combine_kernel, dim3((H + 255) / 256, tokens), dim3(256), 0, s, p, y, tokens,
                has_shared);
}

hipError_t moe_forward_launch(const MoePlan& p, const float* x, float* y, int tokens,
                              hipStream_t s) {
  if (tokens <= 0) return hipSuccess;
  if (tokens > p.capacity) return hipErrorInvalidValue;
  // the MFMA path reads x with 16-byte loads
  if (p.xq && (reinterpret_cast<uintptr_t>(x) & 15u) == 0)
    return moe_forward_mfma(p, x, y, tokens, s);
  const int has_shared = p.shared_ffn > 0;
  // 1 router (+ the shared-gate row for qwen3next)
  GemvProblem r{};
  r.type = kF32;
  r.weights = reinterpret_cast<const uint8_t*>(p.router);
  r.row_bytes = (int64_t)p.hidden * 4;
  r.rows = p.experts + ((p.variant == kQwen3Next && has_shared) ? 1 : 0);
  r.columns = p.hidden;
  r.x = x;
  r.x_stride = p.hidden;
  r.tokens = tokens;
  r.y = p.logits;
  r.y_stride = p.experts + 1;
  hipError_t e = gemv_launch(r, s);
  if (e != hipSuccess) return e;
  // 2 top-k + gating
  const dim3 tgrid((tokens + 3) / 4);
  switch (jpl_for(p.experts)) {
    case 1: e = launch(topk_gate_kernel<1>, tgrid, dim3(256), 0, s, p, tokens); break;
    case 2: e = launch(topk_gate_kernel<2>, tgrid, dim3(256), 0, s, p, tokens); break;
    case 4: e = launch(topk_gate_kernel<4>, tgrid, dim3(256), 0, s, p, tokens); break;
    case 8: e = launch(topk_gate_kernel<8>, tgrid, dim3(256), 0, s, p, tokens); break;
    case 16: e = launch(topk_gate_kernel<16>, tgrid, dim3(256), 0, s, p, tokens); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess) return e;
  // 3 scan + scatter
  const int nt = tokens == 1 ? 1 : kMoeChunkTokens;
  e = launch(moe_scan_kernel, dim3(1), dim3(kScanThreads), 0, s, p, tokens, nt, has_shared);
  if (e != hipSuccess) return e;
  // 4, 5 grouped experts
  e = nt == 1 ? launch_groups<1>(p, x, tokens, s) : launch_groups<kMoeChunkTokens>(p, x, tokens, s);
  if (e != hipSuccess) return e;
  // 6 combine
  return launch(moe_combine_kernel, dim3((p.hidden + 255) / 256, tokens), dim3(256), 0, s, p, y,
                tokens, has_shared);
}

hipError_t moe_reset_launch(const MoePlan& p, hipStream_t s) {
  return launch(moe_reset_kernel, dim3(4), dim3(256), 0, s, p.counts, p.experts, p.error);
}

hipError_t topk_launch(const float* logits, int n, int k, int batch, int* idx, float* val,
                       hipStream_t s) {
  const dim3 grid((batch + 3) / 4);
  switch (jpl_for(n)) {
    case 1: return launch(topk_kernel<1>, grid, dim3(256), 0, s, logits, n, k, batch, idx, val);
    case 2: return launch(topk_kernel<2>, grid, dim3(256), 0, s, logits, n, k, batch, idx, val);
    case 4: return launch(topk_kernel<4>, grid, dim3(256), 0, s, logits, n, k, batch, idx, val);
    case 8: return launch(topk_kernel<8>, grid, dim3(256), 0, s, logits, n, k, batch, idx, val);
    case 16: return launch(topk_kernel<16>, grid, dim3(256), 0, s, logits, n, k, batch, idx, val);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace llhip
