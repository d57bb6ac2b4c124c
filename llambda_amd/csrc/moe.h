// moe.h -- routed-MoE feed-forward on one GPU (moe.hip).
//
// One forward of qwen3next-moe-into (llambda.lisp:5321-5426) or
// nemotron-h-moe-ffn-into (llambda.lisp:5827-5949) for a batch of tokens,
// as a fixed sequence of launches on one stream:
//   1 router GEMV (F32)              logits[t][e]  (+ shared-gate dot, qwen3next)
//   2 top-k + gating, one wavefront per token; expert histogram
//   3 scan + scatter (one workgroup): token-to-expert permutation and the
//     chunk table of (expert, first pair, pair count) work items
//   4 grouped up: gate/up rows of each expert against its chunk of tokens,
//     activation fused (silu(g)*u, or relu(u)^2)
//   5 grouped down: down rows against the chunk's activations, per pair
//   6 combine in rank order, then the shared expert
#pragma once

#include "gemv.h"

namespace llhip {

enum MoeVariant : int { kQwen3Next = 0, kNemotronH = 1 };

// Chunk work item of the grouped expert kernels.
struct MoeChunk {
  int expert;  // slab index within its group (routed: expert id; shared: 0)
  int start;   // first entry of the permutation
  int count;   // pairs in this chunk (1..kMoeChunkTokens)
};

constexpr int kMoeChunkTokens = 4;  // tokens per chunk (grouped kernels, batch > 1)
constexpr int kMoeMaxExperts = 1024;
constexpr int kMoeMaxTopK = 64;

// Device-side description of one layer and its scratch, all device pointers.
struct MoePlan {
  int variant;
  int hidden, experts, top_k, ffn, shared_ffn;
  float weights_scale;
  int weights_norm;
  // weights
  const float* router;   // [(experts + (variant == qwen3next && shared)) ][hidden]
  const float* bias;     // [experts], nemotron
  int gate_type, up_type, down_type;
  const uint8_t* gate;   // [experts * ffn] rows of hidden (qwen3next)
  const uint8_t* up;     // [experts * ffn] rows of hidden
  const uint8_t* down;   // [experts * hidden] rows of ffn
  int sh_gate_type, sh_up_type, sh_down_type;
  const uint8_t* sh_gate;  // [shared_ffn] rows of hidden (qwen3next)
  const uint8_t* sh_up;    // [shared_ffn] rows of hidden
  const uint8_t* sh_down;  // [hidden] rows of shared_ffn
  // scratch, sized for `capacity` tokens
  int capacity;
  float* logits;       // [capacity][experts + 1]
  int* top_idx;        // [capacity][top_k]
  float* top_w;        // [capacity][top_k]
  float* shared_w;     // [capacity]
  int* counts;         // [experts]          zero between runs
  int* perm;           // [capacity * (top_k + 1)]
  MoeChunk* chunks;    // [max_chunks(capacity)]
  int* chunk_counts;   // [2]: routed chunks, shared chunks
  float* act;          // [capacity * (top_k + 1)][max(ffn, shared_ffn)]
  float* down_out;     // [capacity * (top_k + 1)][hidden]
  int* error;          // [1] nonzero after a run that hit a reference error
};

// Upper bound of the chunk table for `tokens` tokens with chunk size nt.
int64_t moe_max_chunks(const MoePlan& p, int64_t tokens, int nt);

// Enqueue one forward for `tokens` tokens: x, y are [tokens][hidden] on the
// device.  `error` codes (bit flags): 1 = fewer than k finite router logits,
// 2 = non-positive weight sum, 4 = expert index out of range.
hipError_t moe_forward_launch(const MoePlan& p, const float* x, float* y, int tokens,
                              hipStream_t stream);

// Zero the histogram and the error flag (session set-up; every run leaves
// the histogram zeroed again).
hipError_t moe_reset_launch(const MoePlan& p, hipStream_t stream);

// Batched device top-k with the reference's selection rule (test hook).
hipError_t topk_launch(const float* logits, int n, int k, int batch, int* idx, float* val,
                       hipStream_t stream);

}  // namespace llhip
