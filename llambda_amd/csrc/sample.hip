// sample.hip -- sample-token-id-from-logits (llambda.lisp:1272-1317) on the
// device, for an output head's logits (sample.h).
//
// One workgroup of 1024 threads:
//   1 copy the logits to the scratch row with the repetition penalty applied
//     to the distinct history tokens (apply-repetition-penalty, 1036-1086;
//     the tokens marked in an LDS bitmap), NaN rejected
//   2 top-k (apply-top-k-with-workspace, 1088-1150): the reference keeps every
//     logit >= the root of a min-heap of the k largest, i.e. the k-th largest
//     value; here: a threshold T0 (the k-th largest of the 1024 threads'
//     maxima, so at least k logits are >= T0), the logits >= T0 compacted
//     into LDS, and the k-th largest of those by a 4-pass radix select
//     (8 bits per pass) over order-preserving keys of the floats
//   3 the survivors (logit >= cutoff) ordered by index
//   4 top-p (apply-top-p-with-workspace, 1163-1240) on the survivors: a
//     stable descending order by rank, then the reference's serial
//     single-precision sums in that order
//   5 apply-temperature, softmax (1009-1034) and the draw
//     (sample-from-probabilities, 1253-1270): masked logits have probability
//     exactly 0, so the reference's serial sums over the whole row equal the
//     serial sums over the survivors in index order, done here by one thread.
// With top-k the result is the reference's token bit for bit.  Without top-k
// (k = 0 or k >= n; top-p must then be 1) every logit survives and the sums
// run as a parallel tree: the token then matches wherever the random value
// is not within rounding of a cumulative boundary.
#include "sample.h"

#include <cmath>

namespace llhip {

constexpr int kSampleThreads = 1024;
constexpr int kSampleBitmapWords = kSampleMaxVocab / 32;
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
__device__ uint32_t radix_select(const float* vals, int m, int k, int* hist, uint32_t* sel) {
  const int tid = threadIdx.x;
  if (tid == 0) {
    sel[0] = 0u;
    sel[1] = 0u;
    sel[2] = (uint32_t)k;
  }
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int b = tid; b < 256; b += kSampleThreads) hist[b] = 0;
    __syncthreads();
    const uint32_t prefix = sel[0], mask = sel[1];
    for (int i = tid; i < m; i += kSampleThreads) {
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

__global__ void __launch_bounds__(kSampleThreads)
sample_kernel(const float* __restrict__ logits, float* __restrict__ work, SampleParams p,
              int* __restrict__ result) {
#pragma clang fp contract(off)
  __shared__ int hist[256];
  __shared__ int red[kSampleThreads / 64 + 1];
  __shared__ float fred[kSampleThreads / 64 + 1];
  __shared__ uint32_t sel[3];
  __shared__ int flag, ncand;
  __shared__ float s_tmax[kSampleThreads];
  __shared__ uint32_t bitmap[kSampleBitmapWords];
  __shared__ int c_idx[kSampleMaxSurvivors];
  __shared__ float c_val[kSampleMaxSurvivors];
  __shared__ int s_idx[kSampleMaxSurvivors];
  __shared__ float s_val[kSampleMaxSurvivors];
  __shared__ float s_e[kSampleMaxSurvivors];
  __shared__ int s_order[kSampleMaxSurvivors];
  const int n = p.n, tid = threadIdx.x;

  // 1. copy with the repetition penalty applied (history tokens marked in an
  // LDS bitmap), NaN rejected; each thread's maximum over its float4s
  if (tid == 0) {
    flag = 0;
    ncand = 0;
  }
  for (int w = tid; w < kSampleBitmapWords; w += kSampleThreads) bitmap[w] = 0u;
  __syncthreads();
  for (int i = tid; i < p.nh; i += kSampleThreads) {
    const int t = p.history[i];
    atomicOr(&bitmap[t >> 5], 1u << (t & 31));
  }
  __syncthreads();
  auto penalized = [&](int i, float v) {
    if (bitmap[i >> 5] & (1u << (i & 31))) {
      if (v > 0.0f) return v / p.penalty;
      if (v < 0.0f) return v * p.penalty;
    }
    return v;
  };
  float tmax = -INFINITY;
  int nan = 0;
  {
    const int n4 = n >> 2;
    const float4* src = reinterpret_cast<const float4*>(logits);
    float4* dst = reinterpret_cast<float4*>(work);
    constexpr int U = 4;
    for (int base = tid; base < n4; base += U * kSampleThreads) {
      float4 a[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = base + u * kSampleThreads;
        a[u] = j < n4 ? src[j] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = base + u * kSampleThreads;
        if (j < n4) {
          float4 v = a[u];
          v.x = penalized(4 * j, v.x);
          v.y = penalized(4 * j + 1, v.y);
          v.z = penalized(4 * j + 2, v.z);
          v.w = penalized(4 * j + 3, v.w);
          nan |= (v.x != v.x) | (v.y != v.y) | (v.z != v.z) | (v.w != v.w);
          tmax = fmaxf(fmaxf(tmax, fmaxf(v.x, v.y)), fmaxf(v.z, v.w));
          dst[j] = v;
        }
      }
    }
    for (int i = 4 * n4 + tid; i < n; i += kSampleThreads) {
      const float v = penalized(i, logits[i]);
      nan |= v != v;
      tmax = fmaxf(tmax, v);
      work[i] = v;
    }
  }
  if (nan) flag = 1;
  s_tmax[tid] = tmax;
  __syncthreads();
  if (flag) {
    if (tid == 0) {
      result[0] = -1;
      result[1] = kSampleErrNaN;
    }
    return;
  }

  const bool topk = p.top_k > 0 && p.top_k < n;
  if (!topk) {
    // every logit survives: the tree path (top-p must be 1); thread t owns
    // the contiguous range [t * per, (t + 1) * per) so that its prefix sums
    // follow index order
    const int per = (n + kSampleThreads - 1) / kSampleThreads;
    const int lo = min(n, tid * per), hi = min(n, lo + per);
    float m = -INFINITY;
    for (int i = lo; i < hi; ++i) m = fmaxf(m, work[i] / p.temperature);
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if ((tid & 63) == 0) fred[tid >> 6] = m;
    __syncthreads();
    float mx = fred[0];
    for (int w = 1; w < kSampleThreads / 64; ++w) mx = fmaxf(mx, fred[w]);
    __syncthreads();
    float local = 0.f;
    for (int i = lo; i < hi; ++i) local += (float)exp((double)(work[i] / p.temperature - mx));
    const float sum = block_sum(local, fred);
    float mine = 0.f;
    for (int i = lo; i < hi; ++i) mine += (float)exp((double)(work[i] / p.temperature - mx)) / sum;
    float run = block_exclusive_scan(mine, fred);
    if (tid == 0) flag = n - 1;
    __syncthreads();
    for (int i = lo; i < hi; ++i) {
      run += (float)exp((double)(work[i] / p.temperature - mx)) / sum;
      if (p.roll <= run) {
        atomicMin(&flag, i);
        break;
      }
    }
    __syncthreads();
    if (tid == 0) {
      result[0] = flag;
      result[1] = 0;
    }
    return;
  }

  // 2. top-k cutoff.  T0 = the k-th largest of the per-thread maxima: at
  // least k logits are >= T0, so the k-th largest logit is >= T0 and lies
  // among the candidates (logits >= T0), which are compacted into LDS.
  // (k above the thread count: the k-th largest of the whole row itself)
  float t0 = key_float(p.top_k <= kSampleThreads
                           ? radix_select(s_tmax, kSampleThreads, p.top_k, hist, sel)
                           : radix_select(work, n, p.top_k, hist, sel));
  auto candidate = [&](int i, float v) {
    if (!(v < t0)) {
      const int slot = atomicAdd(&ncand, 1);
      if (slot < kSampleMaxSurvivors) {
        c_val[slot] = v;
        c_idx[slot] = i;
      }
    }
  };
  for (int attempt = 0; attempt < 2; ++attempt) {
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
  const float cutoff = key_float(radix_select(c_val, cand, p.top_k, hist, sel));

  // 3. survivors (candidates >= cutoff) in index order
  if (tid == 0) flag = 0;
  __syncthreads();
  for (int c = tid; c < cand; c += kSampleThreads) {
    if (c_val[c] < cutoff) continue;
    const int idx = c_idx[c];
    int pos = 0;
    for (int d = 0; d < cand; ++d) pos += !(c_val[d] < cutoff) && c_idx[d] < idx;
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
        for (int b = 0; b < total; ++b) {
          const float w = s_val[b];
          rank += (w > kMaskedLogit) && (w > v || (w == v && b < a));
        }
        s_order[rank] = a;
      }
    }
    __syncthreads();
    if (tid == 0) {
      int active = 0;
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
      if (tid == 0) {
        float sum = 0.0f;
        for (int j = 0; j < active; ++j) sum += s_e[j];
        float cumulative = 0.0f, cut = s_val[s_order[active - 1]];
        for (int j = 0; j < active; ++j) {
          cumulative += s_e[j] / sum;
          if (cumulative >= p.top_p) {
            cut = s_val[s_order[j]];
            break;
          }
        }
        for (int a = 0; a < total; ++a)
          if (s_val[a] < cut) s_val[a] = kMaskedLogit;
      }
      __syncthreads();
    }
  }

  // 5. temperature, softmax, draw (masked logits contribute exactly 0)
  for (int a = tid; a < total; a += kSampleThreads) s_e[a] = s_val[a] / p.temperature;
  __syncthreads();
  if (tid == 0) {
    float mx = s_e[0];
    for (int a = 1; a < total; ++a)
      if (s_e[a] > mx) mx = s_e[a];
    float sum = 0.0f;
    for (int a = 0; a < total; ++a) {
      const float e = (float)exp((double)(s_e[a] - mx));
      s_e[a] = e;
      sum += e;
    }
    int token = n - 1;
    float running = 0.0f;
    if (p.roll <= 0.0f) {
      token = 0;
    } else {
      for (int a = 0; a < total; ++a) {
        running += s_e[a] / sum;
        if (p.roll <= running) {
          token = s_idx[a];
          break;
        }
      }
    }
    result[0] = token;
    result[1] = 0;
  }
}

hipError_t sample_launch(const float* logits, float* work, const SampleParams& p, int* result,
                         hipStream_t stream) {
  hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(kSampleThreads), 0, stream, logits, work, p,
                     result);
  return hipGetLastError();
}

}  // namespace llhip
