// activations.h -- the reference's scalar activations, evaluated as it
// evaluates them (llambda.lisp:926-940).
#pragma once

#include <hip/hip_runtime.h>

namespace llhip {

// sigmoid / silu as llambda.lisp:926-930 evaluates them: exp of the single
// argument is formed in double and rounded to single, 1 + e and the quotient
// are double, the result is rounded to single.
__device__ __forceinline__ float sigmoid_ref(float v) {
  const float e = (float)exp(-(double)v);
  return (float)(1.0 / (1.0 + (double)e));
}
__device__ __forceinline__ float silu_ref(float v) {
  const float e = (float)exp(-(double)v);
  return (float)((double)v / (1.0 + (double)e));
}
// relu-squared, llambda.lisp:938-940
__device__ __forceinline__ float relu2_ref(float v) {
  const float r = v > 0.f ? v : 0.f;
  return __fmul_rn(r, r);
}

}  // namespace llhip
