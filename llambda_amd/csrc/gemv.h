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

// Fused prologue and epilogue of the batch-1 MFMA GEMV, used by the decoder's
// projections.  The default is the plain y[r] = dot(row r, x).
enum GemvEpilogue : int {
  kGemvStore = 0,    // y[r] = v
  kGemvAdd = 1,      // y[r] = res[r] + v                       (vector-add-into)
  kGemvSwiglu8 = 2,  // rows come in groups of 16: 8 gate rows, then the same
                     // 8 up rows; y[8 (r / 16) + i] = silu(g_i) * u_i
  kGemvRope = 3,     // rows < split: query rows, rotated then times q_scale,
                     // to y[r]; rows >= split: key rows, rotated, to the cache
                     // y1 (layout as kGemvCache)
  kGemvCache = 4,    // row r -> y[(r / head_dim) * head_stride +
                     //            pos * head_dim + r % head_dim]
};

struct GemvFuse {
  const float* norm_w = nullptr;  // non-null: x -> rms-norm-into(x, norm_w)
  float norm_eps = 0.f;
  int epi = kGemvStore;
  const float* res = nullptr;     // kGemvAdd (may alias y)
  float* y1 = nullptr;            // kGemvRope key cache
  int split = 0;                  // kGemvRope: first key row
  int head_dim = 0;               // kGemvRope, kGemvCache
  int rope_pairs = 0;             // rotated pairs per head
  const double* rope_cs = nullptr;  // [rope_pairs][2]: cos, sin of this position
  float q_scale = 1.f;
  const int* pos = nullptr;       // device: the token's cache position
  int64_t head_stride = 0;        // cache floats per kv head
};

// Batch-1 GEMV with a fused prologue / epilogue (Q4_K / Q6_K on MFMA only;
// hipErrorInvalidValue for problems the MFMA kernel does not take).
hipError_t gemv_fused_launch(const GemvProblem& p, const GemvFuse& f, hipStream_t stream);

// Two independent fused GEMVs (no shared outputs) in one launch where the
// pair's shapes allow it (Q4_K then Q6_K), else two launches.
hipError_t gemv_fused_pair_launch(const GemvProblem& pa, const GemvFuse& fa, const GemvProblem& pb,
                                  const GemvFuse& fb, hipStream_t stream);

// Batch-1 Q4_K / Q6_K GEMV on MFMA (gemv_mfma.hip).
bool gemv_mfma_supported(const GemvProblem& p);
hipError_t gemv_mfma_launch(const GemvProblem& p, hipStream_t stream);

// Compute units of the current device (cached after the first call).
int device_cu_count();

// out[r * columns + k] = the reference's dequantised weight (bit-exact).
// With row_sel (device int), the one row w + *row_sel * row_bytes (rows = 1).
hipError_t dequant_launch(int type, const uint8_t* w, int64_t row_bytes, int64_t rows,
                          int64_t columns, float* out, hipStream_t stream,
                          const int* row_sel = nullptr);

// A plain read of `bytes` (a multiple of 16, 16-byte aligned device memory)
// by kStreamReadWords waves, each streaming one contiguous slice; out
// (kStreamReadWords words) receives each wave's XOR of what it read.
constexpr int kStreamReadWords = 4096;
hipError_t stream_read_launch(const void* data, size_t bytes, uint32_t* out, hipStream_t stream);

// *first_bad = min(*first_bad, index of the first block whose fp16 scale
// field is Inf/NaN).
hipError_t validate_launch(int type, const uint8_t* w, int64_t nblocks,
                           unsigned long long* first_bad, hipStream_t stream);

}  // namespace llhip
