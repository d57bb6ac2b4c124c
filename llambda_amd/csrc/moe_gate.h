// moe_gate.h -- top-k selection and gating of one token by one wavefront,
// shared by the top-k launch (moe.hip) and the one-token up products, which
// run it in their prologue (moe_mfma.hip).
#pragma once

#include "activations.h"
#include "moe.h"

#include <cfloat>
#include <climits>

namespace llhip {

// ------------------------------------------------------------------ top-k
// select-top-k-logits-into (llambda.lisp:5265-5292) keeps, in descending
// order, the k largest logits strictly above most-negative-single-float,
// lower index first among equal values, never NaN; unfilled slots stay
// (-1, -FLT_MAX).  Here one wavefront holds JPL logits per lane and takes k
// rounds of a wave-wide (value desc, index asc) arg-max; lane r keeps rank
// r.  `bias` (optional) is added first and the biased logits are written
// back.
template <int JPL>
__device__ __forceinline__ void wave_select(float (&vals)[JPL], int K, int lane, int& my_idx,
                                            float& my_val) {
  my_idx = -1;
  my_val = -FLT_MAX;
  for (int r = 0; r < K; ++r) {
    // the lane's best (lowest index among equals), then the wave's
    float lv = -INFINITY;
    int li = INT_MAX;
#pragma unroll
    for (int j = 0; j < JPL; ++j) {
      if (vals[j] > lv) {
        lv = vals[j];
        li = lane + kWave * j;
      }
    }
    const float bv = wave_max(lv);
    const int bi = wave_min(lv == bv ? li : INT_MAX);
    const bool own = bi != INT_MAX && (bi & (kWave - 1)) == lane;
#pragma unroll
    for (int j = 0; j < JPL; ++j) vals[j] = (own && j == (bi >> 6)) ? -INFINITY : vals[j];
    if (lane == r && bi != INT_MAX) {
      my_idx = bi;
      my_val = bv;
    }
  }
}

// The selectable logits of one token: NaN, -inf and -FLT_MAX never qualify.
__device__ __forceinline__ float selectable(float raw) { return raw > -FLT_MAX ? raw : -INFINITY; }

// Top-k plus the gating weights of llambda.lisp:5365-5379 (qwen3next:
// sigmoid, renormalise, error when the sum is not positive) or 5894-5913
// (nemotron: bias before selection, sigmoid, optional renormalise, scale).
// The weight sum runs over the ranks in order, as the reference's loop does.
// Run by one wavefront for token t; with `write` it stores the token's
// logits, top-k indices and weights, shared weight and error flags.  Lane r
// < k returns rank r: its expert (-1 where fewer than k logits qualify), its
// weight and whether the expert is valid.
struct GateRank {
  int idx;
  float w;
  bool valid;
};

template <int JPL>
__device__ __forceinline__ GateRank gate_token(const MoePlan& p, int t, int tokens, bool write) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int E = p.experts, K = p.top_k;
  const int ld = E + 1;
  float* lg = p.logits + (int64_t)t * ld;
  // router logits: the K-slice partial sums in slice order (the router's
  // fixed order), then nemotron's bias; written back for the caller.  The
  // lane's JPL logits (and, on lane 0, the shared-gate logit in slot JPL)
  // load slice by slice, all slots of a slice at once.
  const bool has_shared_row = p.variant == kQwen3Next && p.shared_ffn > 0;
  // (loads are unconditional from a clamped column -- rows have ld = E + 1
  // entries -- and unused slots are dropped by the selects)
  float acc[JPL + 1];
  int col[JPL + 1];
  bool use[JPL + 1];
  float bias[JPL];
#pragma unroll
  for (int j = 0; j <= JPL; ++j) {
    const int e = j < JPL ? lane + kWave * j : E;
    use[j] = j < JPL ? e < E : (lane == 0 && has_shared_row);
    col[j] = min(e, E);
    const float v = p.router_part[(int64_t)t * ld + col[j]];
    acc[j] = use[j] ? v : 0.f;
  }
#pragma unroll
  for (int j = 0; j < JPL; ++j)
    bias[j] = p.variant == kNemotronH ? p.bias[min(lane + kWave * j, E - 1)] : 0.f;
  // The slices were just written by the router launch, on other XCDs: up to
  // kMaxSlices of them are requested in one round (rather than one round
  // per slice), then added in slice order.
  constexpr int kMaxSlices = 8;
  if (p.router_ks <= kMaxSlices) {
    float v[kMaxSlices - 1][JPL + 1];
#pragma unroll
    for (int ks = 1; ks < kMaxSlices; ++ks)
      if (ks < p.router_ks) {
        const float* part = p.router_part + ((int64_t)ks * tokens + t) * ld;
#pragma unroll
        for (int j = 0; j <= JPL; ++j) v[ks - 1][j] = part[col[j]];
      }
#pragma unroll
    for (int ks = 1; ks < kMaxSlices; ++ks)
      if (ks < p.router_ks)
#pragma unroll
        for (int j = 0; j <= JPL; ++j) acc[j] = use[j] ? acc[j] + v[ks - 1][j] : 0.f;
  } else {
    for (int ks = 1; ks < p.router_ks; ++ks) {
      const float* part = p.router_part + ((int64_t)ks * tokens + t) * ld;
      float v[JPL + 1];
#pragma unroll
      for (int j = 0; j <= JPL; ++j) v[j] = part[col[j]];
#pragma unroll
      for (int j = 0; j <= JPL; ++j) acc[j] = use[j] ? acc[j] + v[j] : 0.f;
    }
  }
  float vals[JPL];
#pragma unroll
  for (int j = 0; j < JPL; ++j) {
    const int e = lane + kWave * j;
    float v = -INFINITY;
    if (e < E) {
      float raw = acc[j];
      if (p.variant == kNemotronH) raw = __fadd_rn(raw, bias[j]);
      if (write) lg[e] = raw;
      v = selectable(raw);
    }
    vals[j] = v;
  }
  const float shared_logit = acc[JPL];
  if (write && lane == 0 && has_shared_row) lg[E] = shared_logit;
  int mi;
  float mv;
  wave_select<JPL>(vals, K, lane, mi, mv);
  const bool has = lane < K;
  float w = has ? sigmoid_ref(mv) : 0.f;
  float sum = 0.f;
  for (int r = 0; r < K; ++r)
    sum = sum + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), r));
  int err = (has && mi < 0) ? 1 : 0;
  if (p.variant == kQwen3Next || p.weights_norm) {
    if (!(sum > 0.f)) err |= 2;
    else w = w / sum;
  }
  if (p.variant == kNemotronH) w = p.weights_scale * w;
  if (write && has) {
    p.top_idx[(int64_t)t * K + lane] = mi;
    p.top_w[(int64_t)t * K + lane] = w;
  }
  if (write && lane == 0) p.shared_w[t] = has_shared_row ? sigmoid_ref(shared_logit) : 1.f;
  if (write && err) atomicOr(p.error, err);
  return GateRank{mi, w, has && mi >= 0 && mi < E};
}

// The chunk table of a single token (one wavefront, lane r holding rank
// r's expert and validity): one chunk per valid rank in rank order, then the
// shared expert; pair id of rank r is r, the shared pair is top_k.
__device__ __forceinline__ void gate_chunk_table(const MoePlan& p, bool valid, int mi) {
  const int lane = threadIdx.x & 63;
  const int K = p.top_k;
  const uint64_t mask = __ballot(valid);
  const int pos = __popcll(mask & ((1ull << lane) - 1ull));
  const int nvalid = __popcll(mask);
  if (valid) {
    p.chunks[pos] = MoeChunk{mi, pos, 1};
    p.perm[pos] = lane;
  }
  if (lane == 0) {
    const int has_shared = p.shared_ffn > 0;
    if (has_shared) {
      p.chunks[nvalid] = MoeChunk{0, nvalid, 1};
      p.perm[nvalid] = K;
    }
    p.chunk_counts[0] = nvalid;
    p.chunk_counts[1] = has_shared;
  }
}

}  // namespace llhip
