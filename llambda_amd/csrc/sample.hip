// sample.hip -- sample-token-id-from-logits (llambda.lisp:1272-1317) on the
// device, for an output head's logits (sample.h).
//
// A first launch of kPrepGroups workgroups, each over one contiguous slice
// of the row:
//   1 copy the logits to the scratch row with the repetition penalty applied
//     to the distinct history tokens (apply-repetition-penalty, 1036-1086;
//     the slice's tokens marked in an LDS bitmap), NaN flagged; and, for
//     k <= kPrepCap, the slice's candidates: every logit >= the slice's k-th
//     largest (ties included; more than kPrepCap of them is an overflow).
//     The k largest of the row are among the union of the slices'.
// Then one workgroup of 1024 threads:
//   2 top-k (apply-top-k-with-workspace, 1088-1150): the reference keeps every
//     logit >= the root of a min-heap of the k largest, i.e. the k-th largest
//     value; here the k-th largest of the slices' candidates by a 4-pass
//     radix select (8 bits per pass) over order-preserving keys of the
//     floats.  Larger k, or a slice overflow: a threshold T0 (the k-th
//     largest of the 1024 threads' maxima over the scratch row, so at least
//     k logits are >= T0), the logits >= T0 compacted into LDS, and their
//     k-th largest by the radix select
//   3 the survivors (logit >= cutoff) ordered by index
//   4 top-p (apply-top-p-with-workspace, 1163-1240) on the survivors: a
//     stable descending order by rank, then the reference's serial
//     single-precision sums in that order
//   5 apply-temperature, softmax (1009-1034) and the draw
//     (sample-from-probabilities, 1253-1270): masked logits have probability
//     exactly 0, so the reference's serial sums over the whole row equal the
//     serial sums over the survivors in index order, done here by one thread.
// With top-k the result is the reference's token bit for bit.  Rows without
// top-k (k = 0 or k >= n) take sample_exp_kernel (the exponentials, over the
// slices) and sample_row_kernel instead of steps 2-5.
#include "sample.h"

#include <cmath>

namespace llhip {

constexpr int kSampleThreads = 1024;
constexpr int kPrepGroups = 64;    // first-pass workgroups (row slices)
constexpr int kPrepThreads = 256;
constexpr int kPrepCap = 64;       // candidates a slice may pass on
constexpr int kPrepSlice = kSampleMaxVocab / kPrepGroups;  // longest slice
static_assert(kPrepGroups * kPrepCap <= kSampleMaxSurvivors, "candidates must fit the LDS lists");
constexpr float kMaskedLogit = -1.0e30f;  // llambda.lisp:1098, 1172

// Order-preserving key of a float (larger float -> larger key; -0 < +0).
__device__ __forceinline__ uint32_t float_key(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __builtin_bit_cast(float, u);
}

// Sum over the block in a fixed order (waves' sums added in wave order).
__device__ float block_sum(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = red[0];
  for (int w = 1; w < kSampleThreads / 64; ++w) s += red[w];
  __syncthreads();
  return s;
}

// Exclusive prefix sum over the block, in thread order.
__device__ float block_exclusive_scan(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float inc = v;
  for (int o = 1; o < 64; o <<= 1) {
    const float t = __shfl_up(inc, o, 64);
    if (lane >= o) inc += t;
  }
  if (lane == 63) red[wave] = inc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float acc = 0.f;
    for (int w = 0; w < kSampleThreads / 64; ++w) {
      const float t = red[w];
      red[w] = acc;
      acc += t;
    }
  }
  __syncthreads();
  const float out = red[wave] + (inc - v);
  __syncthreads();
  return out;
}

// The key of the k-th largest of vals[0..m) (generic pointer: LDS or global),
// by a 4-pass radix select over order-preserving keys; every thread calls.
// hist: 256 ints of LDS, sel: 3 words of LDS.  The bins of each pass are
// scanned from the top by wavefront 0 (four bins per lane, a lane prefix sum
// and a ballot).
template <int THREADS = kSampleThreads>
__device__ uint32_t radix_select(const float* vals, int m, int k, int* hist, uint32_t* sel) {
  const int tid = threadIdx.x;
  if (tid == 0) {
    sel[0] = 0u;
    sel[1] = 0u;
    sel[2] = (uint32_t)k;
  }
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int b = tid; b < 256; b += THREADS) hist[b] = 0;
    __syncthreads();
    const uint32_t prefix = sel[0], mask = sel[1];
    for (int i = tid; i < m; i += THREADS) {
      const uint32_t key = float_key(vals[i]);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
    }
    __syncthreads();
    if (tid < 64) {
      const int lane = tid;
      const uint32_t r = sel[2];
      uint32_t c[4], sum = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = (uint32_t)hist[255 - 4 * lane - j];
        sum += c[j];
      }
      uint32_t inc = sum;
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(inc, o, 64);
        if (lane >= o) inc += t;
      }
      const unsigned long long hit = __ballot(inc >= r);
      const int first = hit ? __ffsll(hit) - 1 : 63;
      if (lane == first) {
        uint32_t acc = inc - sum;
        int bin = 255 - 4 * lane - 3;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (acc + c[j] >= r) {
            bin = 255 - 4 * lane - j;
            break;
          }
          acc += c[j];
        }
        sel[0] = prefix | ((uint32_t)bin << shift);
        sel[1] = mask | (255u << shift);
        sel[2] = r - acc;
      }
    }
    __syncthreads();
  }
  return sel[0];
}

// Scratch layout after the row (n rounded up to 4 floats): candidates
// [kPrepGroups][kPrepCap] values, then their indices, then per slice
// (count, nan, cutoff key).  A count above kPrepCap is an overflow; the
// cutoff key is 0 for a slice of at most k logits.
struct PrepScratch {
  float* val;
  int* idx;
  int* count;
  int* nan;
  uint32_t* cut;
  float* smax;  // the slice's maximum of x / T
  float* ssum;  // rows without top-k: the slice's sum of exp(x / T - max)
  int* sact;    // and its logits above the mask value
};
__device__ __host__ inline PrepScratch prep_scratch(float* work, int n) {
  float* base = work + ((n + 3) & ~3);
  PrepScratch ps;
  ps.val = base;
  ps.idx = reinterpret_cast<int*>(base + kPrepGroups * kPrepCap);
  ps.count = ps.idx + kPrepGroups * kPrepCap;
  ps.nan = ps.count + kPrepGroups;
  ps.cut = reinterpret_cast<uint32_t*>(ps.nan + kPrepGroups);
  ps.smax = reinterpret_cast<float*>(ps.cut + kPrepGroups);
  ps.ssum = ps.smax + kPrepGroups;
  ps.sact = reinterpret_cast<int*>(ps.ssum + kPrepGroups);
  return ps;
}

// Top-p without top-k: the row's exponentials, after the prep scratch.
__device__ __host__ inline size_t prep_work_floats(int n) {
  return (size_t)((n + 3) & ~3) + 2 * kPrepGroups * kPrepCap + 6 * kPrepGroups;
}
static_assert((2 * kPrepGroups * kPrepCap + 6 * kPrepGroups) % 4 == 0,
              "the exponentials start on 16 bytes");
__device__ __host__ inline float* topp_scratch(float* work, int n) {
  return work + prep_work_floats(n);
}

size_t sample_work_floats(int n) { return prep_work_floats(n) + (size_t)((n + 3) & ~3); }

__global__ void __launch_bounds__(kPrepThreads)
sample_prep_kernel(const float* __restrict__ logits, float* __restrict__ work, SampleParams p) {
#pragma clang fp contract(off)
  __shared__ uint32_t bitmap[kPrepSlice / 32];
  __shared__ float vals[kPrepSlice];
  __shared__ int hist[256];
  __shared__ uint32_t sel[3];
  __shared__ int nan_flag, count;
  __shared__ float wmax[kPrepThreads / 64];
  const int g = blockIdx.x, tid = threadIdx.x, n = p.n;
  const int lo = (int)((int64_t)g * n / kPrepGroups), hi = (int)((int64_t)(g + 1) * n / kPrepGroups);
  const int m = hi - lo;
  const PrepScratch ps = prep_scratch(work, n);
  for (int w = tid; w < kPrepSlice / 32; w += kPrepThreads) bitmap[w] = 0u;
  if (tid == 0) {
    nan_flag = 0;
    count = 0;
  }
  __syncthreads();
  for (int i = tid; i < p.nh; i += kPrepThreads) {
    const int t = (p.history ? p.history[i] : p.hist_inline[i]) - lo;
    if (t >= 0 && t < m) atomicOr(&bitmap[t >> 5], 1u << (t & 31));
  }
  __syncthreads();
  // the slice's logits in one round of loads (they were just written by
  // another launch), then the penalty
  constexpr int kPer = kPrepSlice / kPrepThreads;
  float lv[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = tid + kPrepThreads * j;
    lv[j] = i < m ? logits[lo + i] : 0.f;
  }
  int nan = 0;
  float vmax = -INFINITY;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = tid + kPrepThreads * j;
    if (i < m) {
      float v = lv[j];
      if (bitmap[i >> 5] & (1u << (i & 31))) {
        if (v > 0.0f) v = v / p.penalty;
        else if (v < 0.0f) v = v * p.penalty;
      }
      nan |= v != v;
      work[lo + i] = v;
      vals[i] = v;
      vmax = fmaxf(vmax, v / p.temperature);
    }
  }
  if (nan) nan_flag = 1;
  vmax = wave_max(vmax);
  if ((tid & 63) == 0) wmax[tid >> 6] = vmax;
  __syncthreads();
  const bool topk = p.top_k > 0 && p.top_k < n;
  uint32_t ck = 0u;
  if (topk && p.top_k <= kPrepCap && !nan_flag) {
    // every logit >= the slice's k-th largest (all of them when m <= k),
    // compared as floats as the reference compares, so that -0 and +0 tie
    // at a cutoff of zero (their keys differ)
    ck = m > p.top_k ? radix_select<kPrepThreads>(vals, m, p.top_k, hist, sel) : 0u;
    const float cut = key_float(ck);
    for (int i = tid; i < m; i += kPrepThreads) {
      if (ck == 0u || !(vals[i] < cut)) {
        const int slot = atomicAdd(&count, 1);
        if (slot < kPrepCap) {
          ps.val[g * kPrepCap + slot] = vals[i];
          ps.idx[g * kPrepCap + slot] = lo + i;
        }
      }
    }
    __syncthreads();
  }
  if (tid == 0) {
    ps.count[g] = count;
    ps.nan[g] = nan_flag;
    ps.cut[g] = ck;
    float sm = wmax[0];
    for (int w = 1; w < kPrepThreads / 64; ++w) sm = fmaxf(sm, wmax[w]);
    ps.smax[g] = sm;
  }
}

// Rows without top-k: exp(x / T - max) rounded to single (computed in double
// as the reference computes it) per position of the slice, into the scratch
// after the prep words, with the slice's sum (threads' strided sums, added
// in wave order) and its logits above the mask value.  The maximum is the
// slices' (written by the prep launch).
__global__ void __launch_bounds__(kPrepThreads)
sample_exp_kernel(float* __restrict__ work, SampleParams p) {
#pragma clang fp contract(off)
  __shared__ float wred[kPrepThreads / 64];
  __shared__ int wact[kPrepThreads / 64];
  __shared__ float s_mx;
  const int g = blockIdx.x, tid = threadIdx.x, n = p.n, lane = tid & 63, wave = tid >> 6;
  const int lo = (int)((int64_t)g * n / kPrepGroups), hi = (int)((int64_t)(g + 1) * n / kPrepGroups);
  const PrepScratch ps = prep_scratch(work, n);
  if (wave == 0) {
    float v = lane < kPrepGroups ? ps.smax[lane] : -INFINITY;
    v = wave_max(v);
    if (lane == 0) s_mx = v;
  }
  __syncthreads();
  const float mx = s_mx;
  float* ex = topp_scratch(work, n);
  constexpr int kPer = kPrepSlice / kPrepThreads;
  float xv[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = lo + tid + kPrepThreads * j;
    xv[j] = i < hi ? work[i] : 0.f;
  }
  float local = 0.f;
  int act = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = lo + tid + kPrepThreads * j;
    if (i < hi) {
      const float e = (float)exp((double)(xv[j] / p.temperature - mx));
      ex[i] = e;
      local += e;
      act += xv[j] > kMaskedLogit;
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    local += __shfl_xor(local, o, 64);
    act += __shfl_xor(act, o, 64);
  }
  if (lane == 0) {
    wred[wave] = local;
    wact[wave] = act;
  }
  __syncthreads();
  if (tid == 0) {
    float t = wred[0];
    int a = wact[0];
    for (int w = 1; w < kPrepThreads / 64; ++w) {
      t += wred[w];
      a += wact[w];
    }
    ps.ssum[g] = t;
    ps.sact[g] = a;
  }
}

__global__ void __launch_bounds__(kSampleThreads)
sample_kernel(float* __restrict__ work, SampleParams p, int* __restrict__ result) {
#pragma clang fp contract(off)
  __shared__ int hist[256];
  __shared__ int red[kSampleThreads / 64 + 1];
  __shared__ float fred[kSampleThreads / 64 + 1];
  __shared__ uint32_t sel[3];
  __shared__ int flag, ncand;
  __shared__ float s_tmax[kSampleThreads];
  __shared__ int s_cnt[kPrepGroups], s_nan[kPrepGroups];
  __shared__ uint32_t s_cut[kPrepGroups];
  __shared__ int c_idx[kSampleMaxSurvivors];
  __shared__ float c_val[kSampleMaxSurvivors];
  __shared__ int s_idx[kSampleMaxSurvivors];
  __shared__ float s_val[kSampleMaxSurvivors];
  __shared__ float s_e[kSampleMaxSurvivors];
  __shared__ int s_order[kSampleMaxSurvivors];
  const int n = p.n, tid = threadIdx.x;

  // the slices' words, one thread each (they were just written on other
  // XCDs: one round of loads, not one per slice); NaN in any slice is the
  // reference's error
  const PrepScratch ps = prep_scratch(work, n);
  if (tid < kPrepGroups) {
    s_cnt[tid] = ps.count[tid];
    s_cut[tid] = ps.cut[tid];
    s_nan[tid] = ps.nan[tid];
  }
  __syncthreads();
  if (tid == 0) {
    int any = 0;
#pragma unroll 16
    for (int g = 0; g < kPrepGroups; ++g) any |= s_nan[g];
    flag = any;
    ncand = 0;
  }
  __syncthreads();
  if (flag) {
    if (tid == 0) {
      result[0] = -1;
      result[1] = kSampleErrNaN;
    }
    return;
  }

  // 2. top-k cutoff.  The slices' candidates when every slice passed all
  // of its own (k <= kPrepCap, no overflow).  Two lower bounds of the row's
  // k-th largest prune them: each slice's k-th largest (the slice alone holds
  // k logits >= it), and the k-th largest of the slices' maxima (k slices
  // each hold a logit >= it; k <= kPrepCap = kPrepGroups).  The larger one
  // keeps about k candidates, and at least k.
  if (tid == 0) {
    int ok = p.top_k <= kPrepCap;
    uint32_t cmax = 0u;
#pragma unroll 16
    for (int g = 0; g < kPrepGroups; ++g) {
      ok &= s_cnt[g] <= kPrepCap;
      cmax = max(cmax, s_cut[g]);
    }
    red[0] = ok;
    sel[0] = cmax;
    sel[1] = 0u;
  }
  __syncthreads();
  const bool gathered = red[0] != 0;
  if (gathered) {
    // every slot's value and index into LDS in one round of loads (s_val /
    // s_idx are free until the survivors)
    constexpr int kSlots = kPrepGroups * kPrepCap / kSampleThreads;
    static_assert(kSlots * kSampleThreads == kPrepGroups * kPrepCap, "slot split");
    float sv[kSlots];
    int si[kSlots];
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
      sv[j] = ps.val[tid + kSampleThreads * j];
      si[j] = ps.idx[tid + kSampleThreads * j];
    }
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
      s_val[tid + kSampleThreads * j] = sv[j];
      s_idx[tid + kSampleThreads * j] = si[j];
    }
    __syncthreads();
    // slice maxima (key 0: an empty slice), then the k-th largest of them by
    // counting: the g with #{> key_g} < k <= #{>= key_g}
    if (tid < kPrepGroups) {
      uint32_t mx = 0u;
#pragma unroll 8
      for (int slot = 0; slot < s_cnt[tid]; ++slot)
        mx = max(mx, float_key(s_val[tid * kPrepCap + slot]));
      s_cut[tid] = mx;
    }
    __syncthreads();
    if (tid < kPrepGroups) {
      const uint32_t v = s_cut[tid];
      int gt = 0, ge = 0;
#pragma unroll 16
      for (int h = 0; h < kPrepGroups; ++h) {
        gt += s_cut[h] > v;
        ge += s_cut[h] >= v;
      }
      if (gt < p.top_k && p.top_k <= ge) sel[1] = v;  // equal keys write equal values
    }
    __syncthreads();
    // (compared as floats, as the reference compares: -0 >= +0)
    const float tlow = key_float(max(sel[0], sel[1]));
    for (int c = tid; c < kPrepGroups * kPrepCap; c += kSampleThreads) {
      const int g = c / kPrepCap, slot = c - g * kPrepCap;
      if (slot < s_cnt[g]) {
        const float v = s_val[c];
        if (!(v < tlow)) {
          const int pos = atomicAdd(&ncand, 1);
          c_val[pos] = v;
          c_idx[pos] = s_idx[c];
        }
      }
    }
    __syncthreads();
  }
  // ... else T0 = the k-th largest of the per-thread maxima over the scratch
  // row: at least k logits are >= T0, so the k-th largest logit is >= T0 and
  // lies among the candidates (logits >= T0), which are compacted into LDS.
  // (k above the thread count: the k-th largest of the whole row itself)
  float t0 = 0.f;
  if (!gathered) {
    float tmax = -INFINITY;
    for (int i = tid; i < n; i += kSampleThreads) tmax = fmaxf(tmax, work[i]);
    s_tmax[tid] = tmax;
    __syncthreads();
    t0 = key_float(p.top_k <= kSampleThreads
                       ? radix_select(s_tmax, kSampleThreads, p.top_k, hist, sel)
                       : radix_select(work, n, p.top_k, hist, sel));
  }
  auto candidate = [&](int i, float v) {
    if (!(v < t0)) {
      const int slot = atomicAdd(&ncand, 1);
      if (slot < kSampleMaxSurvivors) {
        c_val[slot] = v;
        c_idx[slot] = i;
      }
    }
  };
  for (int attempt = 0; attempt < 2 && !gathered; ++attempt) {
    const int n4 = n >> 2;
    const float4* w4 = reinterpret_cast<const float4*>(work);
    constexpr int U = 4;
    for (int base = tid; base < n4; base += U * kSampleThreads) {
      float4 a[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = base + u * kSampleThreads;
        a[u] = j < n4 ? w4[j] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = base + u * kSampleThreads;
        if (j < n4) {
          candidate(4 * j, a[u].x);
          candidate(4 * j + 1, a[u].y);
          candidate(4 * j + 2, a[u].z);
          candidate(4 * j + 3, a[u].w);
        }
      }
    }
    for (int i = 4 * n4 + tid; i < n; i += kSampleThreads) candidate(i, work[i]);
    __syncthreads();
    if (ncand <= kSampleMaxSurvivors || attempt == 1) break;
    // too many candidates above the threshold: the k-th largest of the whole
    // row is the threshold instead (only ties at it can then overflow)
    t0 = key_float(radix_select(work, n, p.top_k, hist, sel));
    __syncthreads();
    if (tid == 0) ncand = 0;
    __syncthreads();
  }
  const int cand = ncand;
  if (cand > kSampleMaxSurvivors) {
    if (tid == 0) {
      result[0] = -1;
      result[1] = kSampleErrTies;
    }
    return;
  }
  // the k-th largest candidate: by counting when they fit one per thread
  // (the c with #{> v_c} < k <= #{>= v_c}), else the radix select
  float cutoff;
  if (cand <= kSampleThreads) {
    if (tid < cand) {
      const float v = c_val[tid];
      int gt = 0, ge = 0;
#pragma unroll 8
      for (int d = 0; d < cand; ++d) {
        const float cv = c_val[d];
        gt += (int)(cv > v);
        ge += (int)(cv >= v);
      }
      if (gt < p.top_k && p.top_k <= ge) fred[0] = v;  // equal values write equal values
    }
    __syncthreads();
    cutoff = fred[0];
    __syncthreads();
  } else {
    cutoff = key_float(radix_select(c_val, cand, p.top_k, hist, sel));
  }

  // 3. survivors (candidates >= cutoff) in index order
  if (tid == 0) flag = 0;
  __syncthreads();
  for (int c = tid; c < cand; c += kSampleThreads) {
    if (c_val[c] < cutoff) continue;
    const int idx = c_idx[c];
    int pos = 0;
#pragma unroll 8
    for (int d = 0; d < cand; ++d) pos += (int)!(c_val[d] < cutoff) & (int)(c_idx[d] < idx);
    s_idx[pos] = idx;
    s_val[pos] = c_val[c];
    atomicAdd(&flag, 1);
  }
  __syncthreads();
  const int total = flag;

  // 4. top-p over the survivors above the mask value
  if (p.top_p < 1.0f) {
    // active survivors keep their index order; rank = stable descending position
    for (int a = tid; a < total; a += kSampleThreads) {
      const float v = s_val[a];
      int rank = 0;
      if (v > kMaskedLogit) {
#pragma unroll 8
        for (int b = 0; b < total; ++b) {
          const float w = s_val[b];
          rank += (int)(w > kMaskedLogit) & ((int)(w > v) | ((int)(w == v) & (int)(b < a)));
        }
        s_order[rank] = a;
      }
    }
    __syncthreads();
    if (tid == 0) {
      int active = 0;
#pragma unroll 8
      for (int a = 0; a < total; ++a) active += s_val[a] > kMaskedLogit;
      red[0] = active;
    }
    __syncthreads();
    const int active = red[0];
    if (active > 1) {
      const float max_scaled = s_val[s_order[0]] / p.temperature;
      for (int j = tid; j < active; j += kSampleThreads)
        s_e[j] = (float)exp((double)(s_val[s_order[j]] / p.temperature - max_scaled));
      __syncthreads();
      // the reference's serial single-precision sums, run by every lane of
      // wavefront 0 (the same loads in the same order: equal results), each
      // lane dividing its own terms by the sum in between
      if (tid < kWave) {
        float sum = 0.0f;
#pragma unroll 8
        for (int j = 0; j < active; ++j) sum += s_e[j];
        for (int j = tid; j < active; j += kWave) s_e[j] = s_e[j] / sum;
        float cumulative = 0.0f;
        int at = active - 1;
        for (int j0 = 0; j0 < active; j0 += 8) {
          float q[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) q[u] = j0 + u < active ? s_e[j0 + u] : 0.f;
          int hit = -1;
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            if (hit < 0 && j0 + u < active) {
              cumulative += q[u];
              if (cumulative >= p.top_p) hit = j0 + u;
            }
          }
          if (hit >= 0) {
            at = hit;
            break;
          }
        }
        if (tid == 0) fred[0] = s_val[s_order[at]];
      }
      __syncthreads();
      {
        const float cut = fred[0];
        for (int a = tid; a < total; a += kSampleThreads)
          if (s_val[a] < cut) s_val[a] = kMaskedLogit;
      }
      __syncthreads();
    }
  }

  // 5. temperature, softmax, draw (masked logits contribute exactly 0).
  // Wavefront 0: the maximum (order-free) and each exp (rounded to single as
  // the reference rounds it) across its lanes; the reference's serial sums
  // in index order by every lane (the same loads in the same order: equal
  // results), each lane dividing its own terms by the sum in between.  The
  // wavefront's LDS accesses execute in order, so no barrier is needed.
  for (int a = tid; a < total; a += kSampleThreads) s_e[a] = s_val[a] / p.temperature;
  __syncthreads();
  if (tid >= kWave) return;
  float mx = -INFINITY;
  for (int a = tid; a < total; a += kWave) mx = fmaxf(mx, s_e[a]);
  mx = wave_max(mx);
  for (int a = tid; a < total; a += kWave) s_e[a] = (float)exp((double)(s_e[a] - mx));
  float sum = 0.0f;
#pragma unroll 8
  for (int a = 0; a < total; ++a) sum += s_e[a];
  for (int a = tid; a < total; a += kWave) s_e[a] = s_e[a] / sum;
  int token = n - 1;
  if (p.roll <= 0.0f) {
    token = 0;
  } else {
    float running = 0.0f;
    for (int a0 = 0; a0 < total; a0 += 8) {
      float q[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) q[u] = a0 + u < total ? s_e[a0 + u] : 0.f;
      int hit = -1;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (hit < 0 && a0 + u < total) {
          running += q[u];
          if (p.roll <= running) hit = a0 + u;
        }
      }
      if (hit >= 0) {
        token = s_idx[hit];
        break;
      }
    }
  }
  if (tid == 0) {
    result[0] = token;
    result[1] = 0;
  }
}

// Rows without top-k (k = 0 or k >= n: every logit survives apply-top-k).
// Top-p (apply-top-p-with-workspace, llambda.lisp:1163-1240), when p < 1:
// the logits above the mask value ranked by value, descending, exp(x / T -
// max / T) per rank, and the first rank at which the running sum of
// exp / sum reaches p gives the cut value; every logit below it is masked
// (ties with the cut kept).  Only the cut value is needed, not the ranking:
// it is the value whose keys' probability mass first brings the running sum
// to p, found by a radix select over descending keys (12, 8, 8 and 4 bits a
// pass, most significant first) that carries each bin's mass.  Masses are 32-bit
// fixed-point probabilities (floor(2^32 exp / sum), exp / sum rounded to
// single as the reference forms it) added in 64-bit integers, so every order
// of addition gives the same bins; the sums are exact where the reference's
// serial single sums round (the cut can move by a rank where the running sum
// meets p within that rounding).  A row whose total never reaches p keeps
// every logit (the reference's cut is then its smallest one).
// Then apply-temperature, softmax (1009-1034) and the draw
// (sample-from-probabilities, 1253-1270) over the masked row: masked logits
// have probability exactly 0.  Wavefront w owns a contiguous segment of the
// row, read 256 positions at a time (lane l: positions 4l .. 4l+3, one
// float4), so the running sums follow index order up to the rounding of
// the wavefront scans and of the scan over the segments' totals; the
// reference adds serially, so the token matches wherever the random value is
// not within rounding of a cumulative boundary.  The exponentials, the
// slices' sums and their active counts come from sample_exp_kernel.
constexpr int kRowWaves = kSampleThreads / 64;

// Exclusive prefix sum of one 64-bit integer per thread over the block, in
// thread order (red: kRowWaves words of LDS).
__device__ unsigned long long block_exclusive_scan_u64(unsigned long long v,
                                                       unsigned long long* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  unsigned long long inc = v;
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned long long t = __shfl_up(inc, o, 64);
    if (lane >= o) inc += t;
  }
  if (lane == 63) red[wave] = inc;
  __syncthreads();
  unsigned long long before = 0;
  for (int w = 0; w < wave; ++w) before += red[w];
  __syncthreads();
  return before + inc - v;
}

// Inclusive scan of v over the wavefront's lanes, in lane order.
__device__ __forceinline__ float wave_inclusive_scan(float v) {
  const int lane = threadIdx.x & 63;
  for (int o = 1; o < 64; o <<= 1) {
    const float t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

__global__ void __launch_bounds__(kSampleThreads)
sample_row_kernel(float* __restrict__ work, SampleParams p, int* __restrict__ result) {
#pragma clang fp contract(off)
  __shared__ unsigned long long mass[4096];
  __shared__ unsigned long long ured[kRowWaves];
  __shared__ float fred[kRowWaves + 1];
  __shared__ float wtot[kRowWaves];
  __shared__ int s_active, s_token, s_none;
  __shared__ uint32_t s_key;  // descending key of the selected prefix
  __shared__ unsigned long long s_before;
  const int n = p.n, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const PrepScratch ps = prep_scratch(work, n);
  if (tid == 0) {
    s_active = 0;
    s_token = n - 1;
    s_none = 0;
    s_key = 0;
    s_before = 0;
  }
  // NaN in any slice is the reference's error (the slices' words were just
  // written on other XCDs: one round of loads)
  if (__syncthreads_or(tid < kPrepGroups ? ps.nan[tid] : 0)) {
    if (tid == 0) {
      result[0] = -1;
      result[1] = kSampleErrNaN;
    }
    return;
  }
  float* ex = topp_scratch(work, n);
  // this wavefront's segment [wlo, whi): a multiple of 256 positions long
  const int seg = (n + 256 * kRowWaves - 1) / (256 * kRowWaves) * 256;
  const int wlo = min(n, wave * seg), whi = min(n, wlo + seg);
  constexpr int kB = 8;  // float4 loads per lane in flight
  // each round of kB chunks of 256: the row's (and, with EX, the
  // exponentials') float4s loaded at once, then visit(chunk start, x[4],
  // e[4], count) per chunk in order; the row is padded to 4 floats, so a
  // float4 that starts inside it is read whole
  auto sweep = [&](auto with_ex, auto&& visit) {
    constexpr bool EX = decltype(with_ex)::value;
    for (int c0 = wlo; c0 < whi; c0 += 256 * kB) {
      float4 xv[kB], ev[kB];
#pragma unroll
      for (int b = 0; b < kB; ++b) {
        const int i = c0 + 256 * b + 4 * lane;
        xv[b] = i < whi ? *reinterpret_cast<const float4*>(work + i) : make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (EX)
          ev[b] = i < whi ? *reinterpret_cast<const float4*>(ex + i) : make_float4(0.f, 0.f, 0.f, 0.f);
        else
          ev[b] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int b = 0; b < kB; ++b) {
        const int c = c0 + 256 * b;
        if (c >= whi) break;  // uniform
        const int i = c + 4 * lane;
        const float xs[4] = {xv[b].x, xv[b].y, xv[b].z, xv[b].w};
        const float es[4] = {ev[b].x, ev[b].y, ev[b].z, ev[b].w};
        visit(i, xs, es, max(0, min(4, whi - i)));
      }
    }
  };
  using NoEx = std::integral_constant<bool, false>;
  using WithEx = std::integral_constant<bool, true>;

  // the row's sum of exponentials (the slices' sums in slice order) and its
  // logits above the mask value
  if (tid == 0) {
    float t = 0.f;
    int a = 0;
    for (int g = 0; g < kPrepGroups; ++g) {
      t += ps.ssum[g];
      a += ps.sact[g];
    }
    fred[0] = t;
    s_active = a;
  }
  __syncthreads();
  const float sum = fred[0];
  __syncthreads();

  float cut = -INFINITY;  // logits below it are masked
  if (p.top_p < 1.0f && s_active > 1) {
    const unsigned long long target = (unsigned long long)ceil((double)p.top_p * 4294967296.0);
    auto dkey = [](float x) { return ~float_key(x == 0.0f ? 0.0f : x); };  // -0 ranks with +0
    // passes over key bits 31..20 (sign, exponent, 3 mantissa bits: a
    // row's logits spread over many bins, so few lanes of an instruction
    // add to one), 19..12, 11..4 and 3..0
    constexpr int kShift[4] = {20, 12, 4, 0}, kWidth[4] = {12, 8, 8, 4};
    for (int pass = 0; pass < 4; ++pass) {
      const int shift = kShift[pass], width = kWidth[pass], nb = 1 << width;
      for (int i = tid; i < nb; i += kSampleThreads) mass[i] = 0ull;
      __syncthreads();
      const uint32_t prefix = s_key;
      const int top = shift + width;  // bits above the pass's are the prefix's
      sweep(WithEx{}, [&](int, const float (&x)[4], const float (&e)[4], int cnt) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (u >= cnt || !(x[u] > kMaskedLogit)) continue;
          const uint32_t k = dkey(x[u]);
          if (top < 32 && (k >> top) != (prefix >> top)) continue;
          // floor(2^32 q): the scaling is exact in single, the conversion truncates
          const float qs = (e[u] / sum) * 4294967296.0f;
          const uint32_t q = qs < 4294967296.0f ? (uint32_t)qs : 0xFFFFFFFFu;
          if (q) atomicAdd(&mass[(k >> shift) & (uint32_t)(nb - 1)], (unsigned long long)q);
        }
      });
      __syncthreads();
      // thread t: bins 4t .. 4t+3; the running mass before them; the one
      // thread whose bins bring it to the target picks the bin
      unsigned long long mine = 0;
      if (4 * tid < nb)
        for (int j = 0; j < 4; ++j) mine += mass[4 * tid + j];
      unsigned long long run = s_before + block_exclusive_scan_u64(mine, ured);
      if (4 * tid < nb && run < target && run + mine >= target) {
        for (int j = 0; j < 4; ++j) {
          const unsigned long long bm = mass[4 * tid + j];
          if (run + bm >= target) {
            s_key = (prefix & ~((uint32_t)(nb - 1) << shift)) | ((uint32_t)(4 * tid + j) << shift);
            s_before = run;
            break;
          }
          run += bm;
        }
        s_none = 2;  // picked
      }
      __syncthreads();
      const bool picked = s_none == 2;
      __syncthreads();
      if (!picked) break;  // the total never reaches p (first pass): no cut
      if (tid == 0) s_none = 0;
      if (pass == 3) cut = key_float(~s_key);
    }
  }

  // the draw over the masked row: its sum, each chunk's running sums of
  // exp / sum (lanes' four in order, then a lane scan), chunks in order, the
  // segments' totals scanned in wavefront order; the first position whose
  // running sum reaches the roll
  float msum = sum;
  if (cut > -INFINITY) {
    float ls = 0.f;
    sweep(WithEx{}, [&](int, const float (&x)[4], const float (&e)[4], int cnt) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (u < cnt && x[u] >= cut) ls += e[u];
    });
    msum = block_sum(ls, fred);
  }
  auto probs = [&](const float (&x)[4], const float (&e)[4], int cnt, float (&q)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) q[u] = u < cnt && x[u] >= cut ? e[u] / msum : 0.f;
  };
  float seg_run = 0.f;  // the segment's running sum at its current chunk
  sweep(WithEx{}, [&](int, const float (&x)[4], const float (&e)[4], int cnt) {
    float q[4];
    probs(x, e, cnt, q);
    const float incl = wave_inclusive_scan(((q[0] + q[1]) + q[2]) + q[3]);
    seg_run += __shfl(incl, 63, 64);
  });
  if (lane == 0) wtot[wave] = seg_run;
  __syncthreads();
  float run = 0.f;  // the running sum before this segment
  for (int w = 0; w < wave; ++w) run += wtot[w];
  bool found = false;
  sweep(WithEx{}, [&](int i, const float (&x)[4], const float (&e)[4], int cnt) {
    if (found) return;  // uniform
    float q[4];
    probs(x, e, cnt, q);
    const float incl = wave_inclusive_scan(((q[0] + q[1]) + q[2]) + q[3]);
    const float before = __shfl_up(incl, 1, 64);
    float r = run + (lane > 0 ? before : 0.f);
    int hit = 4;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      r += q[u];
      if (hit == 4 && u < cnt && p.roll <= r) hit = u;
    }
    const uint64_t any = __ballot(hit < 4);
    if (any) {
      if (lane == __builtin_ctzll(any)) atomicMin(&s_token, i + hit);
      found = true;
    }
    run += __shfl(incl, 63, 64);
  });
  __syncthreads();
  if (tid == 0) {
    result[0] = s_token;
    result[1] = 0;
  }
}

hipError_t sample_launch(const float* logits, float* work, const SampleParams& p, int* result,
                         hipStream_t stream) {
  if (p.n <= 0 || p.n > kSampleMaxVocab) return hipErrorInvalidValue;
  hipLaunchKernelGGL(sample_prep_kernel, dim3(kPrepGroups), dim3(kPrepThreads), 0, stream, logits,
                     work, p);
  const bool topk = p.top_k > 0 && p.top_k < p.n;
  if (topk) {
    hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(kSampleThreads), 0, stream, work, p, result);
  } else {
    hipLaunchKernelGGL(sample_exp_kernel, dim3(kPrepGroups), dim3(kPrepThreads), 0, stream, work, p);
    hipLaunchKernelGGL(sample_row_kernel, dim3(1), dim3(kSampleThreads), 0, stream, work, p, result);
  }
  return hipGetLastError();
}

}  // namespace llhip
