// moe.hip -- routed-MoE feed-forward: routing, permutation, combine and the
// forward's launch sequence (the expert products are in moe_mfma.hip).
#include "moe.h"
#include "activations.h"
#include "moe_gate.h"

#include <algorithm>
#include <cfloat>
#include <climits>

namespace llhip {

template <int JPL>
__global__ void __launch_bounds__(256) topk_kernel(const float* __restrict__ logits, int n, int k,
                                                   int batch, int* __restrict__ idx,
                                                   float* __restrict__ val) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= batch) return;
  const int lane = threadIdx.x & 63;
  float vals[JPL];
#pragma unroll
  for (int j = 0; j < JPL; ++j) {
    const int e = lane + kWave * j;
    vals[j] = e < n ? selectable(logits[(int64_t)t * n + e]) : -INFINITY;
  }
  __shared__ int64_t sel[4][kSelectScratch];
  int mi;
  float mv;
  wave_select<JPL>(vals, k, lane, sel[threadIdx.x >> 6], mi, mv);
  if (lane < k) {
    idx[(int64_t)t * k + lane] = mi;
    val[(int64_t)t * k + lane] = mv;
  }
}

// Top-k and gating, one wavefront per token (gate_token); for a single token
// also the chunk table: one chunk per selected expert in rank order, then
// the shared expert.
template <int JPL>
__global__ void __launch_bounds__(256) topk_gate_kernel(MoePlan p, int tokens, int single) {
  __shared__ int64_t sel[4][kSelectScratch];
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= tokens) return;
  const GateRank r = gate_token<JPL>(p, t, tokens, true, sel[threadIdx.x >> 6]);
  if (!single) return;  // the scan kernel counts the experts' pairs
  gate_chunk_table(p, r.valid, r.idx);
}

// ------------------------------------------------------------ scan/scatter
// One workgroup: the expert histogram of the top-k indices (in LDS), its
// exclusive scans (pairs and chunks), the chunk table, and the permutation
// that groups (token, rank) pairs by expert.  Pair id p = token * k + rank;
// the shared expert's pairs are tokens * k + token.
constexpr int kScanThreads = 1024;
constexpr int kMaxChunkPairs = 128;  // pairs per chunk: 16, 32, 64 or 128

__global__ void __launch_bounds__(kScanThreads) moe_scan_kernel(MoePlan p, int tokens, int nt,
                                                                int has_shared) {
  __shared__ int s_cnt[kMoeMaxExperts];
  __shared__ int s_off[kMoeMaxExperts + 1];
  __shared__ int s_coff[kMoeMaxExperts + 1];
  __shared__ int s_cur[kMoeMaxExperts];
  __shared__ int s_part[kScanThreads / 64];
  __shared__ int s_cpart[kScanThreads / 64];
  const int E = p.experts, K = p.top_k, tid = threadIdx.x;
  const int P = tokens * K;
  for (int e = tid; e < E; e += kScanThreads) {
    s_cnt[e] = 0;
    s_cur[e] = 0;
  }
  __syncthreads();
  // the histogram of the selected experts, in LDS (global atomics on a hot
  // expert's counter serialise hundreds of increments)
  for (int q = tid; q < P; q += kScanThreads) {
    const int e = p.top_idx[q];
    if (e >= 0 && e < E) atomicAdd(&s_cnt[e], 1);
  }
  __syncthreads();
  const int per = (E + kScanThreads - 1) / kScanThreads;
  const int e0 = tid * per, e1 = min(e0 + per, E);
  int sum = 0, csum = 0;
  for (int e = e0; e < e1; ++e) {
    sum += s_cnt[e];
    csum += (s_cnt[e] + nt - 1) / nt;
  }
  // exclusive prefix sums of both counts in thread order: wavefront scans,
  // then the wavefronts' totals
  const int lane = tid & 63, wave = tid >> 6;
  int inc = sum, cinc = csum;
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(inc, o, 64), cv = __shfl_up(cinc, o, 64);
    if (lane >= o) {
      inc += v;
      cinc += cv;
    }
  }
  if (lane == 63) {
    s_part[wave] = inc;
    s_cpart[wave] = cinc;
  }
  __syncthreads();
  int run = inc - sum, crun = cinc - csum;
  for (int w = 0; w < wave; ++w) {
    run += s_part[w];
    crun += s_cpart[w];
  }
  for (int e = e0; e < e1; ++e) {
    s_off[e] = run;
    s_coff[e] = crun;
    run += s_cnt[e];
    crun += (s_cnt[e] + nt - 1) / nt;
  }
  if (tid == kScanThreads - 1) {
    s_off[E] = run;
    s_coff[E] = crun;
  }
  __syncthreads();
  const int routed_pairs = s_off[E], routed_chunks = s_coff[E];
  // The chunk table in decreasing pair count -- every full chunk, then the
  // experts' partial last chunks, counting-sorted by size -- so that the
  // launch's last workgroups are its shortest.  (A chunk's outputs do not
  // depend on where it sits in the table.)
  __shared__ int s_hoff[kMaxChunkPairs + 1];
  __shared__ int s_full;
  if (tid <= kMaxChunkPairs) s_hoff[tid] = 0;
  if (tid == 0) s_full = 0;
  __syncthreads();
  for (int e = tid; e < E; e += kScanThreads) {
    const int r = s_cnt[e] % nt;
    if (r) atomicAdd(&s_hoff[r], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int run = routed_chunks;  // the partial chunks end the routed table
    for (int v = 1; v < nt; ++v) {
      run -= s_hoff[v];
      s_hoff[v] = run;
    }
  }
  __syncthreads();
  for (int e = tid; e < E; e += kScanThreads) {
    const int c = s_cnt[e], f = c / nt, r = c - f * nt;
    const int base = f ? atomicAdd(&s_full, f) : 0;
    for (int j = 0; j < f; ++j) p.chunks[base + j] = MoeChunk{e, s_off[e] + j * nt, nt};
    if (r) p.chunks[atomicAdd(&s_hoff[r], 1)] = MoeChunk{e, s_off[e] + f * nt, r};
  }
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

// Weighted combine in rank order, then the shared expert, every product and
// sum rounded separately as in vector-add-scaled-in-place /
// vector-add-bias-in-place (llambda.lisp:3465-3489; 5359, 5409, 5426, 5914,
// 5932, 5949).  `width` outputs per token (hidden; latent_out where
// ffn_latent_up follows, then without the shared expert, which
// moe_latent_finish_kernel adds after it).
__global__ void __launch_bounds__(256) moe_combine_kernel(MoePlan p, float* __restrict__ y,
                                                          int tokens, int width, int has_shared,
                                                          int* __restrict__ error_out) {
#pragma clang fp contract(off)
  const int t = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const int K = p.top_k;
  const int64_t ow = p.out_w;
  if (error_out && i == 0 && t == 0) *error_out = *p.error;
  if (i >= width) return;
  // the ranks' outputs (just written by another launch, on other XCDs) are
  // loaded 8 ranks at a time before the sums, which run in rank order
  const float dsh = has_shared ? p.down_out[(int64_t)(tokens * K + t) * ow + i] : 0.f;
  float acc = 0.f;
  constexpr int kBatch = 8;
  for (int r0 = 0; r0 < K; r0 += kBatch) {
    float d[kBatch], wv[kBatch];
    int ix[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int q = t * K + min(r0 + b, K - 1);
      ix[b] = p.top_idx[q];
      wv[b] = p.top_w[q];
      d[b] = p.down_out[(int64_t)q * ow + i];
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      if (r0 + b >= K || ix[b] < 0) continue;
      const float prod = wv[b] * d[b];
      acc = acc + prod;
    }
  }
  if (has_shared) {
    const float d = dsh;
    if (p.variant == kQwen3Next) {
      const float prod = p.shared_w[t] * d;
      acc = acc + prod;
    } else {
      acc = acc + d;
    }
  }
  y[(int64_t)t * width + i] = acc;
}

// After ffn_latent_up (llambda.lisp:5933-5938): y = its output, plus the
// shared expert's (vector-add-bias-in-place, :5939-5949) when there is one.
__global__ void __launch_bounds__(256) moe_latent_finish_kernel(MoePlan p, float* __restrict__ y,
                                                                int tokens, int has_shared,
                                                                int* __restrict__ error_out) {
#pragma clang fp contract(off)
  const int t = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const int H = p.hidden;
  if (error_out && i == 0 && t == 0) *error_out = *p.error;
  if (i >= H) return;
  float v = p.lat_y[(int64_t)t * H + i];
  if (has_shared) v = v + p.down_out[(int64_t)(tokens * p.top_k + t) * p.out_w + i];
  y[(int64_t)t * H + i] = v;
}

__global__ void moe_reset_kernel(int* error) {
  if (threadIdx.x == 0) *error = 0;
}

// OR a run's error flags into another flag word (one thread).
__global__ void moe_error_merge_kernel(const int* __restrict__ src, int* __restrict__ dst) {
  if (threadIdx.x == 0) {
    const int f = *src;
    if (f) atomicOr(dst, f);
  }
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

static int64_t row_bytes_of(int type, int64_t columns) {
  return columns / block_weights(type) * block_bytes(type);
}

// Pipeline of the grouped MFMA products and its chunk size: 0 = the
// single-token pipeline, 1 = one 16-token tile per chunk (double-buffered),
// 2 = two 16-token tiles per chunk (32 pairs), 4 and 8 = the group pipeline
// with one or two wave sets (64 or 128 pairs per chunk).
#ifndef LLHIP_GROUP_PAIRS
#define LLHIP_GROUP_PAIRS 64
#endif
static int moe_mfma_tiles(const MoePlan& p, int tokens) {
  if (tokens == 1) return 0;
  const int64_t avg = ((int64_t)tokens * p.top_k + p.experts - 1) / p.experts;
  if (avg <= 16) return 1;
  // the group pipeline (64-pair chunks) for 32-weight block types, while its
  // 32-bit byte offsets into the split rows and their sums fit
  const bool types = moe_group_pipeline_types(p.up_type) && moe_group_pipeline_types(p.down_type) &&
                     (p.shared_ffn == 0 || (moe_group_pipeline_types(p.sh_up_type) &&
                                            moe_group_pipeline_types(p.sh_down_type)));
  const int64_t act_w = std::max(p.ffn, p.shared_ffn);
  const int64_t split_bytes = std::max((int64_t)tokens * (p.top_k + 1) * 4 * act_w,
                                       (int64_t)tokens * 4 * std::max(p.hidden, p.latent_in));
  // the wide pipeline's relu^2 and down kernels for Q5_0 rows of an odd
  // number of blocks (not dword multiples) do not fit the registers: layers
  // with such rows keep 16-pair chunks
  auto odd_q5 = [](int type, int64_t k) { return type == kQ5_0 && ((k / 32) & 1); };
  const bool odd = odd_q5(p.up_type, p.latent_in ? p.latent_in : p.hidden) ||
                   odd_q5(p.down_type, p.ffn) ||
                   (p.shared_ffn && (odd_q5(p.sh_up_type, p.hidden) ||
                                     odd_q5(p.sh_down_type, p.shared_ffn)));
  if (!types || split_bytes >= ((int64_t)1 << 31)) return odd ? 1 : 2;
  return LLHIP_GROUP_PAIRS / 16;
}
static int moe_chunk_tokens(int mt) { return mt == 0 ? 1 : 16 * mt; }

// One forward: router GEMM (+ split x), top-k and gating, scan (batches),
// grouped gate/up and down products, combine.
hipError_t moe_forward_launch(const MoePlan& p, const float* x, float* y, int tokens,
                              hipStream_t s, int* error_out) {
  if (tokens <= 0) return hipSuccess;
  if (tokens > p.capacity) return hipErrorInvalidValue;
  // the router and the split read x with 16-byte loads
  if (reinterpret_cast<uintptr_t>(x) & 15u) return hipErrorInvalidValue;
  const int has_shared = p.shared_ffn > 0;
  const int H = p.hidden, E = p.experts, K = p.top_k;
  const int Li = p.latent_in, Lo = p.latent_out;
  const int din = Li ? Li : H, dout = Lo ? Lo : H;  // routed experts' input, output widths
  const int act_w = std::max(p.ffn, p.shared_ffn);
  const int64_t xs_stride = H / 16, as_stride = act_w / 16;
  const int er = E + ((p.variant == kQwen3Next && has_shared) ? 1 : 0);
  hipError_t e = router_mfma_launch(x, tokens, p.router, er, H, p.router_part, E + 1, p.xq,
                                    2 * (int64_t)H, p.xsum, xs_stride, s);
  if (e != hipSuccess) return e;
  if (Li) {
    // the experts' input ffn_latent_down * x (llambda.lisp:5883-5887) and
    // its split rows; the router and the shared expert keep x's
    GemvProblem g{p.lat_down_type, p.lat_down, row_bytes_of(p.lat_down_type, H), Li, H, x, H,
                  tokens, p.lat, Li};
    e = gemv_launch(g, s);
    if (e != hipSuccess) return e;
    e = split_rows_launch(p.lat, tokens, Li, Li, p.lq, 2 * (int64_t)Li, p.lsum, Li / 16, s);
    if (e != hipSuccess) return e;
  }
  const int single = tokens == 1;
  const int mt = moe_mfma_tiles(p, tokens), nt = moe_chunk_tokens(mt);
  // routed and shared up products share a launch when they share a weight
  // type and an input
  const bool joint_up = has_shared && p.sh_up_type == p.up_type && !Li;
  // one token whose up products run in one launch: that launch selects and
  // gates the token itself (one launch fewer)
  const bool fuse_gate = single && mt == 0 && (!has_shared || joint_up) && K <= kMoeMaxTopK &&
                         jpl_for(E) <= 16;
  if (!fuse_gate) {
    const dim3 tgrid((tokens + 3) / 4);
    switch (jpl_for(E)) {
      case 1: e = launch(topk_gate_kernel<1>, tgrid, dim3(256), 0, s, p, tokens, single); break;
      case 2: e = launch(topk_gate_kernel<2>, tgrid, dim3(256), 0, s, p, tokens, single); break;
      case 4: e = launch(topk_gate_kernel<4>, tgrid, dim3(256), 0, s, p, tokens, single); break;
      case 8: e = launch(topk_gate_kernel<8>, tgrid, dim3(256), 0, s, p, tokens, single); break;
      case 16: e = launch(topk_gate_kernel<16>, tgrid, dim3(256), 0, s, p, tokens, single); break;
      default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
  }
  if (!single) {
    e = launch(moe_scan_kernel, dim3(1), dim3(kScanThreads), 0, s, p, tokens, nt, has_shared);
    if (e != hipSuccess) return e;
  }
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

  // routed, then shared, gate/up products: one launch when the types agree
  MoeGemmArgs a = up;
  a.group = 0;
  if (Li) {
    a.aq = p.lq;
    a.aq_stride = 2 * (int64_t)Li;
    a.as = p.lsum;
    a.as_stride = Li / 16;
    a.K = Li;
  }
  a.w0 = p.variant == kQwen3Next ? p.gate : p.up;
  a.w1 = p.up;
  a.row_bytes = row_bytes_of(p.up_type, din);
  a.expert_stride = moe_slab_bytes(p.up_type, p.ffn, din);
  a.N = p.ffn;
  if (joint_up) {
    a.joint = 1;
    a.s_w0 = p.variant == kQwen3Next ? p.sh_gate : p.sh_up;
    a.s_w1 = p.sh_up;
    a.s_row_bytes = row_bytes_of(p.sh_up_type, H);
    a.s_N = p.shared_ffn;
    a.s_K = H;
  }
  if (fuse_gate) {
    a.fused_gate = 1;
    a.gate_jpl = jpl_for(E);
    a.plan = p;
  }
  const bool staged_up = mt >= 4 && epi == kEpiRelu2;  // one matrix: the stage-major copies
  if (staged_up) {
    a.w0 = p.up_g;
    a.expert_stride = p.up_g_stride;
    a.s_w0 = p.sh_up_g;
  }
  e = moe_gemm_launch(p.up_type, epi, a, mt,
                      fuse_gate ? K + (joint_up ? 1 : 0)
                                : routed_chunks + (joint_up ? shared_chunks : 0),
                      s);
  if (e != hipSuccess) return e;
  if (has_shared && !joint_up) {
    a = up;
    a.group = 1;
    a.w0 = staged_up ? p.sh_up_g : p.variant == kQwen3Next ? p.sh_gate : p.sh_up;
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
  down.out_stride = p.out_w;
  a = down;
  a.group = 0;
  a.K = p.ffn;
  a.N = dout;
  a.w0 = p.down;
  a.row_bytes = row_bytes_of(p.down_type, p.ffn);
  a.expert_stride = moe_slab_bytes(p.down_type, dout, p.ffn);
  const bool joint_down = has_shared && p.sh_down_type == p.down_type;
  if (joint_down) {
    a.joint = 1;
    a.s_w0 = p.sh_down;
    a.s_row_bytes = row_bytes_of(p.sh_down_type, p.shared_ffn);
    a.s_N = H;
    a.s_K = p.shared_ffn;
  }
  // one token: the down products and the combine in one launch
  if (single && !Lo && (!has_shared || joint_down) &&
      moe_down_combine_supported(p.down_type, a)) {
    MoeCombineArgs c{};
    c.y = y;
    c.top_w = p.top_w;
    c.shared_w = p.shared_w;
    c.shared_scaled = p.variant == kQwen3Next;
    c.error = p.error;
    c.error_out = error_out;
    return moe_down_combine_launch(p.down_type, a, c, s);
  }
  if (mt >= 4) {
    a.w0 = p.down_g;
    a.expert_stride = p.down_g_stride;
    a.s_w0 = p.sh_down_g;
  }
  e = moe_gemm_launch(p.down_type, kEpiDown, a, mt, routed_chunks + (joint_down ? shared_chunks : 0), s);
  if (e != hipSuccess) return e;
  if (has_shared && !joint_down) {
    a = down;
    a.group = 1;
    a.K = p.shared_ffn;
    a.w0 = mt >= 4 ? p.sh_down_g : p.sh_down;
    a.row_bytes = row_bytes_of(p.sh_down_type, p.shared_ffn);
    a.expert_stride = 0;
    e = moe_gemm_launch(p.sh_down_type, kEpiDown, a, mt, shared_chunks, s);
    if (e != hipSuccess) return e;
  }
  // (a separate launch: combining in the last workgroup of each row tile,
  // behind a device-scope fence and an atomic per workgroup, measured 10 us
  // slower for one Qwen3Next token)
  if (!Lo)
    return launch(moe_combine_kernel, dim3((H + 255) / 256, tokens), dim3(256), 0, s, p, y, tokens,
                  H, has_shared, error_out);
  // the Lo-wide weighted sum, ffn_latent_up, then the shared expert
  e = launch(moe_combine_kernel, dim3((Lo + 255) / 256, tokens), dim3(256), 0, s, p, p.lat, tokens,
             Lo, 0, static_cast<int*>(nullptr));
  if (e != hipSuccess) return e;
  GemvProblem g{p.lat_up_type, p.lat_up, row_bytes_of(p.lat_up_type, Lo), H, Lo, p.lat, Lo, tokens,
                p.lat_y, H};
  e = gemv_launch(g, s);
  if (e != hipSuccess) return e;
  return launch(moe_latent_finish_kernel, dim3((H + 255) / 256, tokens), dim3(256), 0, s, p, y,
                tokens, has_shared, error_out);
}

hipError_t moe_reset_launch(const MoePlan& p, hipStream_t s) {
  return launch(moe_reset_kernel, dim3(1), dim3(64), 0, s, p.error);
}

hipError_t moe_error_merge_launch(const int* src, int* dst, hipStream_t s) {
  return launch(moe_error_merge_kernel, dim3(1), dim3(64), 0, s, src, dst);
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
