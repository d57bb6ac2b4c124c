// gemv.h -- launchers of the dequant-fused GEMV kernels (gemv.hip).
#pragma once

#include "units.h"

namespace llhip {

// y[t * y_stride + r] = dot(row r of `weights`, x + t * x_stride) for
// r < rows, t < tokens.  Every pointer is device memory; `weights` carries
// kWeightPad readable bytes past rows * row_bytes.
struct GemvProblem {
  int type;
  const uint8_t* weights;
  int64_t row_bytes;
  int64_t rows;
  int64_t columns;
  const float* x;
  int64_t x_stride;
  int tokens;
  float* y;
  int64_t y_stride;
};

// LDS per workgroup on gfx950.
constexpr size_t kMaxLdsBytes = 160 * 1024;

// Columns a packed GEMV session accepts (one token's activations and their
// group sums must fit in LDS).
constexpr int64_t kMaxColumns = 32768;

hipError_t gemv_launch(const GemvProblem& p, hipStream_t stream);

// Batch-1 Q4_K / Q6_K GEMV on MFMA (gemv_mfma.hip).
bool gemv_mfma_supported(const GemvProblem& p);
hipError_t gemv_mfma_launch(const GemvProblem& p, hipStream_t stream);

// Compute units of the current device (cached after the first call).
int device_cu_count();

// out[r * columns + k] = the reference's dequantised weight (bit-exact).
hipError_t dequant_launch(int type, const uint8_t* w, int64_t row_bytes, int64_t rows,
                          int64_t columns, float* out, hipStream_t stream);

// *first_bad = min(*first_bad, index of the first block whose fp16 scale
// field is Inf/NaN).
hipError_t validate_launch(int type, const uint8_t* w, int64_t nblocks,
                           unsigned long long* first_bad, hipStream_t stream);

}  // namespace llhip
