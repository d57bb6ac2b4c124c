// sample.h -- sample-token-id-from-logits (llambda.lisp:1272-1317) on the
// device (sample.hip).
#pragma once

#include "common.h"

namespace llhip {

// Survivors of top-k (ties included) the exact path holds in LDS.
constexpr int kSampleMaxSurvivors = 4096;
// Longest logits row (the history bitmap lives in LDS).
constexpr int kSampleMaxVocab = 262144;

enum SampleError : int {
  kSampleErrNaN = 1,   // a NaN logit
  kSampleErrTies = 2,  // more than kSampleMaxSurvivors logits tie at or above the cutoff
};

// Histories of up to this many distinct tokens travel in the launch's
// arguments (no copy to the device before the launch).
constexpr int kSampleInlineHistory = 128;

struct SampleParams {
  int n;               // logits
  const int* history;  // device, distinct token ids < n (host-validated), or
                       // null: the ids are hist_inline[0 .. nh)
  int nh;
  float penalty;       // repetition penalty (> 0)
  int top_k;           // 0 or >= n: no top-k (top_p must then be 1); at most
                       // kSampleMaxSurvivors
  float top_p;         // (0, 1]
  float temperature;   // > 0
  float roll;          // random value in [0, 1)
  int hist_inline[kSampleInlineHistory];
};

// Scratch floats sample_launch needs for n logits: the penalised row, the
// first pass's candidates and its per-workgroup counts.
size_t sample_work_floats(int n);

// result[0] = token (-1 on error), result[1] = SampleError or 0.  work:
// sample_work_floats(n) floats of scratch.  logits and work 16-byte aligned.
// Two launches: a multi-workgroup pass over the row, then one workgroup.
hipError_t sample_launch(const float* logits, float* work, const SampleParams& p, int* result,
                         hipStream_t stream);

}  // namespace llhip
