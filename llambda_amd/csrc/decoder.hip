// decoder.hip -- the Llama-layout decode token (decoder.h): state, rotation
// table, grouped-query attention over the fp32 KV cache, and the step's
// launch sequence over the fused batch-1 GEMV (gemv_mfma.hip).
#include "decoder.h"

#include <algorithm>
#include <cmath>

namespace llhip {

// The state word and the rotation table of the position: cos and sin of
// angle = position / denom[i] per rotary pair (apply-rope-head-in-place,
// llambda.lisp:3760-3795: the angle in double; denom[i] = factor_i *
// theta^(2i/d) is formed on the host, +inf where the factor exceeds 1e20 so
// that the angle is 0).
__global__ void decoder_state_kernel(int* __restrict__ state, int token, int position,
                                     const double* __restrict__ denom, int pairs,
                                     double* __restrict__ cs) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i == 0) {
    state[0] = token;
    state[1] = position;
  }
  if (i >= pairs) return;
  const double angle = (double)position / denom[i];
  cs[2 * i] = cos(angle);
  cs[2 * i + 1] = sin(angle);
}

hipError_t decoder_state_launch(const DecoderPlan& p, int token, int position,
                                hipStream_t stream) {
  const int blocks = std::max(1, (p.rope_pairs + 63) / 64);
  hipLaunchKernelGGL(decoder_state_kernel, dim3(blocks), dim3(64), 0, stream, p.state, token,
                     position, p.rope_denom, p.rope_pairs, p.rope_cs);
  return hipGetLastError();
}

// ----------------------------------------------------------------- attention
// compute-gemma4-attention-into as the llama step calls it
// (llambda.lisp:5122-5167 with dot-product 3491-3500, softmax-into 5075-5096,
// weighted-sum-head-into 5097-5115): for query head h of kv head h / G,
// scores s_p = q_h . k_p over cache slots p = 0..position, probabilities
// exp(s_p - max) / sum, context = sum_p prob_p v_p.
//
// Workgroup (chunk, kv head) takes slots [P chunk, P chunk + P), P =
// kAttnChunk, for the G query heads of its kv head: scores (16 lanes per
// slot, xor-shuffle reduction), the chunk's max m_c, e_p = exp(s_p - m_c) and
// their sum S_c, and the unnormalised sum_p e_p v_p.  A second launch
// combines the chunks (four quarters of them in order, then the quarters):
// M = max m_c, a_c = exp(m_c - M),
// context = (sum_c a_c pv_c) / (sum_c a_c S_c).  The reference normalises
// every probability before the weighted sum; the two agree to rounding
// (single-precision exp of each difference, computed in double as SBCL
// does).
constexpr int kAttnWaves = 8;

__device__ __forceinline__ float4 operator+(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
__device__ __forceinline__ float4 scale4(float s, float4 a) {
  return make_float4(s * a.x, s * a.y, s * a.z, s * a.w);
}

template <int D, int G>
__global__ void __launch_bounds__(64 * kAttnWaves)
attention_kernel(const float* __restrict__ q, const float* __restrict__ kc,
                 const float* __restrict__ vc, int64_t head_stride, const int* __restrict__ state,
                 float* __restrict__ part, float* __restrict__ pmax, float* __restrict__ psum,
                 int max_chunks) {
  constexpr int P = kAttnChunk;
  constexpr int T = 64 * kAttnWaves;
  constexpr int DL = D / 16;  // dims per lane in the scores
  constexpr int DQ = D / 4;   // float4 columns of a row
  constexpr int NP = T / DQ;  // slot parts in the weighted sum
  constexpr int PPP = P / NP;  // slots per part
  constexpr int SPW = P / kAttnWaves;  // slots per wave in the scores
  constexpr int ST = SPW / 4;          // four slots per step
  constexpr int E = P / 64;            // slots per lane in the softmax
  static_assert((P == 64 || P == 128) && D % 16 == 0 && G <= kAttnWaves && NP * PPP == P &&
                    ST * 4 * kAttnWaves == P,
                "attention shape");
  __shared__ float sc[G][P];
  __shared__ float4 pv[NP][G][DQ];

  const int n = state[1] + 1;
  const int chunk = blockIdx.x, kvh = blockIdx.y;
  const int nchunks = (n + P - 1) / P;
  if (chunk >= nchunks) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float* kh = kc + (int64_t)kvh * head_stride;
  const float* vh = vc + (int64_t)kvh * head_stride;
  const int p0 = chunk * P;

  // scores: lane (grp, sub) holds dims [DL sub, DL sub + DL); wave w takes
  // slots 16w .. 16w+15 of the chunk, four per step
  {
    const int sub = lane & 15, grp = lane >> 4;
    float qr[G][DL];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int j = 0; j < DL; j += 4) {
        const float4 v =
            *reinterpret_cast<const float4*>(q + (int64_t)(kvh * G + h) * D + DL * sub + j);
        qr[h][j] = v.x; qr[h][j + 1] = v.y; qr[h][j + 2] = v.z; qr[h][j + 3] = v.w;
      }
    float kr[ST][DL];
#pragma unroll
    for (int st = 0; st < ST; ++st) {
      const int p = min(p0 + SPW * wave + 4 * st + grp, n - 1);
#pragma unroll
      for (int j = 0; j < DL; j += 4) {
        const float4 v = *reinterpret_cast<const float4*>(kh + (int64_t)p * D + DL * sub + j);
        kr[st][j] = v.x; kr[st][j + 1] = v.y; kr[st][j + 2] = v.z; kr[st][j + 3] = v.w;
      }
    }

#pragma unroll
    for (int st = 0; st < ST; ++st) {
      const int pl = SPW * wave + 4 * st + grp;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < DL; ++j) s += qr[h][j] * kr[st][j];
        s = group_sum(s, 4);  // the 16 lanes of the slot
        if (sub == 0) sc[h][pl] = p0 + pl < n ? s : -INFINITY;
      }
    }
  }
  // the value rows of the weighted sum, requested now so that they load
  // while the softmax runs: thread (prt, col) takes float4 column col of
  // slots prt, prt + NP, ...
  const int col = threadIdx.x % DQ, prt = threadIdx.x / DQ;
  float4 vr[PPP];
#pragma unroll
  for (int i = 0; i < PPP; ++i) {
    const int p = min(p0 + prt + NP * i, n - 1);
    vr[i] = *reinterpret_cast<const float4*>(vh + (int64_t)p * D + 4 * col);
  }
  __syncthreads();

  // chunk max, e_p = exp(s_p - m) rounded to single, and the chunk sum
  if (wave < G) {
    const int h = wave;
    float sv[E];
    float m = -INFINITY;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      sv[e] = sc[h][lane + 64 * e];
      m = fmaxf(m, sv[e]);
    }
    m = wave_max(m);
    float t = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float ev = p0 + lane + 64 * e < n ? (float)exp((double)(sv[e] - m)) : 0.f;
      sc[h][lane + 64 * e] = ev;
      t += ev;
    }
    t = wave_total(t);
    if (lane == 0) {
      pmax[((int64_t)kvh * max_chunks + chunk) * G + h] = m;
      psum[((int64_t)kvh * max_chunks + chunk) * G + h] = t;
    }
  }
  __syncthreads();

  // unnormalised weighted sum of the chunk's value rows
  {
    float4 acc[G];
#pragma unroll
    for (int h = 0; h < G; ++h) acc[h] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < PPP; ++i) {
      const int pl = prt + NP * i;
      if (p0 + pl < n) {
#pragma unroll
        for (int h = 0; h < G; ++h) acc[h] = acc[h] + scale4(sc[h][pl], vr[i]);
      }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) pv[prt][h][col] = acc[h];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < G * DQ; i += T) {
    const int h = i / DQ, c = i % DQ;
    float4 t = pv[0][h][c];
    for (int r = 1; r < NP; ++r) t = t + pv[r][h][c];
    *reinterpret_cast<float4*>(part + (((int64_t)kvh * max_chunks + chunk) * G + h) * D + 4 * c) = t;
  }
}

// Chunks of one query head combined: M = max m_c, a_c = exp(m_c - M)
// (single, computed in double), S = sum a_c S_c, out = (sum a_c pv_c) / S.
// Workgroup h; thread (q, d) = (t / D, t % D) takes element d over quarter q
// of the chunks, in chunk order, and the four quarters' sums are added in
// quarter order.  (The partials were just written by workgroups on other
// XCDs, so every dependent round of loads is slow: a thread requests its
// quarter's values, up to kCombineLoads, at once -- a wave holds at most 63
// vector loads in flight -- and the maxima and sums go through LDS.)
constexpr int kCombineQuarters = 4;
constexpr int kCombineLoads = 32;
template <int D, int G>
__global__ void __launch_bounds__(kCombineQuarters * D)
attention_combine_kernel(const float* __restrict__ part, const float* __restrict__ pmax,
                         const float* __restrict__ psum, const int* __restrict__ state,
                         int max_chunks, float* __restrict__ out) {
  constexpr int T = kCombineQuarters * D, U = kCombineLoads;
  __shared__ float alpha[kAttnMaxChunks], ssum[kAttnMaxChunks];
  __shared__ float red[T / 64];
  __shared__ float qacc[kCombineQuarters][D], qs[kCombineQuarters];
  const int h = blockIdx.x, t = threadIdx.x, lane = t & 63;
  const int q = t / D, d = t - q * D;
  const int kvh = h / G, hh = h % G;
  const int nchunks = (state[1] + kAttnChunk) / kAttnChunk;
  const int per = (nchunks + kCombineQuarters - 1) / kCombineQuarters;
  const int c_lo = q * per, c_hi = min(nchunks, c_lo + per);
  const int64_t base = (int64_t)kvh * max_chunks * G + hh;  // chunk c at base + c * G
  const float* pc = part + base * D + d;
  float pv[U];
#pragma unroll
  for (int u = 0; u < U; ++u) pv[u] = pc[(int64_t)max(0, min(c_lo + u, c_hi - 1)) * G * D];
  float m = -INFINITY;
  for (int c = t; c < nchunks; c += T) {
    const float v = pmax[base + (int64_t)c * G];
    alpha[c] = v;
    ssum[c] = psum[base + (int64_t)c * G];
    m = fmaxf(m, v);
  }
  m = wave_max(m);
  if (lane == 0) red[t >> 6] = m;
  __syncthreads();
  m = red[0];
#pragma unroll
  for (int w = 1; w < T / 64; ++w) m = fmaxf(m, red[w]);
  for (int c = t; c < nchunks; c += T) alpha[c] = (float)exp((double)(alpha[c] - m));
  __syncthreads();
  float S = 0.f, acc = 0.f;
  for (int c0 = c_lo; c0 < c_hi; c0 += U) {
    if (c0 > c_lo) {
#pragma unroll
      for (int u = 0; u < U; ++u) pv[u] = pc[(int64_t)min(c0 + u, c_hi - 1) * G * D];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (c0 + u < c_hi) {
        const float a = alpha[c0 + u];
        S += a * ssum[c0 + u];
        acc += a * pv[u];
      }
    }
  }
  qacc[q][d] = acc;
  if (d == 0) qs[q] = S;
  __syncthreads();
  if (q == 0) {
    float sa = qacc[0][d], ss = qs[0];
#pragma unroll
    for (int i = 1; i < kCombineQuarters; ++i) {
      sa += qacc[i][d];
      ss += qs[i];
    }
    out[(int64_t)h * D + d] = sa / ss;
  }
}

bool decoder_head_supported(int head_dim, int group) {
  return (head_dim == 64 || head_dim == 128) &&
         (group == 1 || group == 2 || group == 4 || group == 8);
}

template <int D, int G>
static hipError_t launch_attention_t(const DecoderPlan& p, const float* q, const float* kc,
                                     const float* vc, float* out, hipStream_t stream) {
  const dim3 grid(p.att_chunks, p.kv_heads);
  hipLaunchKernelGGL((attention_kernel<D, G>), grid, dim3(64 * kAttnWaves), 0, stream, q, kc, vc,
                     (int64_t)p.context * D, p.state, p.att_part, p.att_max, p.att_sum,
                     p.att_chunks);
  hipLaunchKernelGGL((attention_combine_kernel<D, G>), dim3(p.heads), dim3(kCombineQuarters * D), 0,
                     stream,
                     p.att_part, p.att_max, p.att_sum, p.state, p.att_chunks, out);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_attention_d(const DecoderPlan& p, const float* q, const float* kc,
                                     const float* vc, float* out, hipStream_t s) {
  switch (p.heads / p.kv_heads) {
    case 1: return launch_attention_t<D, 1>(p, q, kc, vc, out, s);
    case 2: return launch_attention_t<D, 2>(p, q, kc, vc, out, s);
    case 4: return launch_attention_t<D, 4>(p, q, kc, vc, out, s);
    case 8: return launch_attention_t<D, 8>(p, q, kc, vc, out, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t decoder_attention_launch(const DecoderPlan& p, const float* q, const float* kc,
                                    const float* vc, float* out, hipStream_t s) {
  if (p.kv_heads <= 0 || p.heads % p.kv_heads || !decoder_head_supported(p.head_dim, p.heads / p.kv_heads) ||
      p.att_chunks <= 0 || p.att_chunks > kAttnMaxChunks || (int64_t)p.att_chunks * kAttnChunk < p.context)
    return hipErrorInvalidValue;
  return p.head_dim == 64 ? launch_attention_d<64>(p, q, kc, vc, out, s)
                          : launch_attention_d<128>(p, q, kc, vc, out, s);
}

// ---------------------------------------------------------------- the step
static GemvProblem problem(const DecoderMatrix& m, const float* x, float* y) {
  GemvProblem g{};
  g.type = m.type;
  g.weights = m.w;
  g.row_bytes = m.row_bytes;
  g.rows = m.rows;
  g.columns = m.columns;
  g.x = x;
  g.x_stride = m.columns;
  g.tokens = 1;
  g.y = y;
  g.y_stride = m.rows;
  return g;
}

#define DEC_CHECK(expr)                 \
  do {                                  \
    const hipError_t e_ = (expr);       \
    if (e_ != hipSuccess) return e_;    \
  } while (0)

hipError_t decoder_step_launch(const DecoderPlan& p, float* logits, hipStream_t st) {
  const int D = p.head_dim;
  // token row (gguf-model-token-row-into, llambda.lisp:4977-4982); the
  // rotation table came with the state
  DEC_CHECK(dequant_launch(p.embd.type, p.embd.w, p.embd.row_bytes, 1, p.hidden, p.x, st, p.state));
  for (int l = 0; l < p.layer_count; ++l) {
    const DecoderLayer& L = p.layers[l];
    GemvFuse rope;
    rope.norm_w = L.attn_norm;
    rope.norm_eps = p.eps;
    rope.epi = kGemvRope;
    rope.y1 = L.kcache;
    rope.head_dim = D;
    rope.rope_pairs = p.rope_pairs;
    rope.rope_cs = p.rope_cs;
    rope.q_scale = p.q_scale;
    rope.pos = p.state + 1;
    rope.head_stride = (int64_t)p.context * D;
    GemvFuse cache;
    cache.norm_w = L.attn_norm;
    cache.norm_eps = p.eps;
    cache.epi = kGemvCache;
    cache.head_dim = D;
    cache.pos = p.state + 1;
    cache.head_stride = (int64_t)p.context * D;
    if (L.qk.w) {
      // q|k and v rows in one launch where their shapes allow
      rope.split = p.heads * D;
      DEC_CHECK(gemv_fused_pair_launch(problem(L.qk, p.x, p.q), rope,
                                       problem(L.v, p.x, L.vcache), cache, st));
    } else {
      rope.split = p.heads * D;  // every row a query row
      DEC_CHECK(gemv_fused_launch(problem(L.q, p.x, p.q), rope, st));
      rope.split = 0;  // every row a key row
      DEC_CHECK(gemv_fused_launch(problem(L.k, p.x, p.q), rope, st));
      DEC_CHECK(gemv_fused_launch(problem(L.v, p.x, L.vcache), cache, st));
    }
    DEC_CHECK(decoder_attention_launch(p, p.q, L.kcache, L.vcache, p.ctx, st));
    // x += o(context) (vector-add-into, llambda.lisp:6404)
    GemvFuse add;
    add.epi = kGemvAdd;
    add.res = p.x;
    DEC_CHECK(gemv_fused_launch(problem(L.o, p.ctx, p.x), add, st));
    GemvFuse swiglu;
    swiglu.norm_w = L.ffn_norm;
    swiglu.norm_eps = p.eps;
    swiglu.epi = kGemvSwiglu8;
    DEC_CHECK(gemv_fused_launch(problem(L.gate_up, p.x, p.h), swiglu, st));
    DEC_CHECK(gemv_fused_launch(problem(L.down, p.h, p.x), add, st));
  }
  GemvFuse head;
  head.norm_w = p.output_norm;
  head.norm_eps = p.eps;
  return gemv_fused_launch(problem(p.output, p.x, logits), head, st);
}

}  // namespace llhip
