// moe_gate.h -- top-k selection and gating of one token by one wavefront,
// shared by the top-k launch (moe.hip) and the one-token up products, which
// run it in their prologue (moe_mfma.hip).
#pragma once

#include "activations.h"
#include "moe.h"

#include <cfloat>
#include <climits>
#include <utility>

namespace llhip {

// ------------------------------------------------------------------ top-k
// select-top-k-logits-into (llambda.lisp:5265-5292) keeps, in descending
// order, the k largest logits strictly above most-negative-single-float,
// lower index first among equal values, never NaN; unfilled slots stay
// (-1, -FLT_MAX).  Here one wavefront holds JPL logits per lane (-inf where
// not selectable) and takes k rounds of a wave-wide (value desc, index asc)
// arg-max; lane r keeps rank r.
//
// A candidate is the entry (key << 32) | (~index << 1) | (value is -0), a
// signed 64-bit integer: a larger entry is a larger value, or an equal value
// at a lower index.  Values map to integers that order as the floats do, -0
// to the key of +0, which it equals (NaN never occurs: `selectable` turns it
// into -inf); the entry's lowest bit keeps the sign of a zero, so the
// selected value is returned bit for bit.
//
// Selection by threshold (a fixed number of steps, not k dependent rounds):
// the k-th largest of the 64 lanes' maxima, t, is found by counting ranks;
// every entry of the top k is at least t (the k largest maxima are k entries
// >= t), and only the k lanes whose maximum is >= t hold such entries, so
// at most k * JPL candidates remain.  They are compacted into LDS by ballot
// prefix counts and ranked by counting; more than 64 (possible only when
// k * JPL > 64) take the round-by-round selection instead.
__device__ __forceinline__ int order_key(float v) {
  const int b = __builtin_bit_cast(int, v == 0.f ? 0.f : v);
  return b >= 0 ? b : b ^ 0x7FFFFFFF;
}
__device__ __forceinline__ float order_value(int k) {
  return __builtin_bit_cast(float, k >= 0 ? k : k ^ 0x7FFFFFFF);
}

// The list operations below index the candidates with compile-time
// constants only (template recursion, fold expressions), so the array lives
// in registers from the start: written as loops, a select between two of its
// entries can become an access at a computed index, lowered to a chain of
// compares and selects per entry.
constexpr int kSelectNone = (int)0x807FFFFF;  // order_key(-inf): nothing selectable
// LDS a wavefront's selection uses (int64 entries)
constexpr int kSelectScratch = 2 * kWave + 1;

__device__ __forceinline__ int64_t select_entry(float v, int index) {
  const uint32_t neg0 = __builtin_bit_cast(uint32_t, v) == 0x80000000u ? 1u : 0u;
  return (int64_t)((uint64_t)(uint32_t)order_key(v) << 32 |
                   ((uint32_t)~(uint32_t)index << 1 | neg0));
}
__device__ __forceinline__ void select_decode(int64_t e, int& idx, float& val) {
  const int k = (int)(e >> 32);
  idx = (int)(~(uint32_t)e >> 1);
  val = (k == 0 && (e & 1)) ? -0.f : order_value(k);
}

// descending bitonic sort: stage (KB, J), comparator I
template <int JPL, int KB, int J, int I>
__device__ __forceinline__ void select_sort(int64_t (&c)[JPL]) {
  if constexpr (I < JPL) {
    constexpr int L = I ^ J;
    if constexpr (L > I) {
      constexpr bool kDesc = (I & KB) == 0;
      const bool sw = kDesc ? c[L] > c[I] : c[I] > c[L];
      const int64_t a = sw ? c[L] : c[I], b = sw ? c[I] : c[L];
      c[I] = a;
      c[L] = b;
    }
    select_sort<JPL, KB, J, I + 1>(c);
  } else if constexpr (J > 1) {
    select_sort<JPL, KB, J / 2, 0>(c);
  } else if constexpr (KB < JPL) {
    select_sort<JPL, KB * 2, KB, 0>(c);
  }
}

template <int JPL, int... J>
__device__ __forceinline__ void select_fill(int64_t (&c)[JPL], const float (&vals)[JPL], int lane,
                                            std::integer_sequence<int, J...>) {
  ((c[J] = select_entry(vals[J], lane + kWave * J)), ...);
}

// drop the head of the list where `own`
template <int JPL, int... J>
__device__ __forceinline__ void select_pop(int64_t (&c)[JPL], bool own,
                                           std::integer_sequence<int, J...>) {
  ((c[J] = own ? c[J + 1] : c[J]), ...);
  c[JPL - 1] = own ? (int64_t)((uint64_t)(uint32_t)kSelectNone << 32) : c[JPL - 1];
}

__device__ __forceinline__ int64_t readlane64(int64_t v, int l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), l);
  return (int64_t)((uint64_t)hi << 32 | lo);
}

// Round by round: each lane's list sorted, then per round the wave's largest
// head (an integer max, then an index min over the lanes holding it) and a
// shift of the winning lane's list.
template <int JPL>
__device__ __forceinline__ void wave_select_rounds(int64_t (&c)[JPL], int K, int lane, int& my_idx,
                                                float& my_val) {
  if constexpr (JPL > 1) select_sort<JPL, 2, 1, 0>(c);
  for (int r = 0; r < K; ++r) {
    const int hk = (int)(c[0] >> 32);
    const int m = wave_max_i(hk);
    if (m == kSelectNone) break;  // uniform: the remaining slots stay unfilled
    const int hi = (int)(~(uint32_t)c[0] >> 1);
    const int bi = wave_min(hk == m ? hi : INT_MAX);
    const bool own = (bi & (kWave - 1)) == lane;
    float v = order_value(m);
    if (m == 0 && (__builtin_amdgcn_readlane((int)(uint32_t)c[0], bi & (kWave - 1)) & 1)) v = -0.f;
    select_pop<JPL>(c, own, std::make_integer_sequence<int, JPL - 1>{});
    if (lane == r) {
      my_idx = bi;
      my_val = v;
    }
  }
}

// `s`: kSelectScratch int64 entries of LDS owned by this wavefront.
template <int JPL>
__device__ __forceinline__ void wave_select(const float (&vals)[JPL], int K, int lane, int64_t* s,
                                            int& my_idx, float& my_val) {
  int64_t c[JPL];
  select_fill<JPL>(c, vals, lane, std::make_integer_sequence<int, JPL>{});
  my_idx = -1;
  my_val = -FLT_MAX;
  // the threshold: the lane maximum of rank K - 1 (ranks are distinct, the
  // indices being distinct, and K <= 64)
  int64_t h = c[0];
#pragma unroll
  for (int j = 1; j < JPL; ++j) h = c[j] > h ? c[j] : h;
  s[lane] = h;
  int rank = 0;
#pragma unroll
  for (int i = 0; i < kWave; ++i) rank += s[i] > h ? 1 : 0;
  const int tl = (int)__builtin_ctzll(__ballot(rank == K - 1));
  const int64_t t = readlane64(h, tl);
  // the candidates: selectable entries >= t, and their exclusive prefix
  // count over the lanes (at most 16 per lane: 5 bits)
  bool take[JPL];
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < JPL; ++j) {
    take[j] = c[j] >= t && (int)(c[j] >> 32) != kSelectNone;
    cnt += take[j] ? 1 : 0;
  }
  int pre = 0, total = 0;
#pragma unroll
  for (int b = 0; b < 5; ++b) {
    const uint64_t m = __ballot((cnt >> b) & 1);
    pre += (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u)) << b;
    total += __popcll(m) << b;
  }
  if (total > kWave) {
    wave_select_rounds<JPL>(c, K, lane, my_idx, my_val);
    return;
  }
  // compact into s[64 .. 64 + total) (non-candidates write the spare entry
  // s[128]); the wavefront's LDS accesses execute in order, so the reads of
  // the maxima above are done before these writes
  int64_t* cs = s + kWave;
  int at = pre;
#pragma unroll
  for (int j = 0; j < JPL; ++j) {
    cs[take[j] ? at : kWave] = c[j];
    at += take[j] ? 1 : 0;
  }
  // entries past the candidates read as the smallest entry, so the ranks
  // are counted eight at a time
  if (lane >= total) cs[lane] = INT64_MIN;
  const int64_t mine = cs[lane];
  int r2 = 0;
  for (int i0 = 0; i0 < total; i0 += 8)
#pragma unroll
    for (int i = i0; i < i0 + 8; ++i) r2 += cs[i] > mine ? 1 : 0;
  // rank r2 of the first min(K, total) to lane r2, through s[0 .. K)
  const int filled = min(K, total);
  if (lane < total && r2 < filled) s[r2] = mine;
  if (lane < filled) select_decode(s[lane], my_idx, my_val);
}

// The selectable logits of one token: NaN, -inf and -FLT_MAX never qualify.
__device__ __forceinline__ float selectable(float raw) { return raw > -FLT_MAX ? raw : -INFINITY; }

// Top-k plus the gating weights of llambda.lisp:5365-5379 (qwen3next:
// sigmoid, renormalise, error when the sum is not positive) or 5894-5913
// (nemotron: bias before selection, sigmoid, optional renormalise, scale).
// The weight sum runs over the ranks in order, as the reference's loop does.
// Run by one wavefront for token t (`sel`: its kSelectScratch entries of
// LDS); with `write` it stores the token's
// logits, top-k indices and weights, shared weight and error flags.  Lane r
// < k returns rank r: its expert (-1 where fewer than k logits qualify), its
// weight and whether the expert is valid.
struct GateRank {
  int idx;
  float w;
  bool valid;
};

template <int JPL>
__device__ __forceinline__ GateRank gate_token(const MoePlan& p, int t, int tokens, bool write,
                                               int64_t* sel) {
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
  wave_select<JPL>(vals, K, lane, sel, mi, mv);
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
