// decoder.h -- one Llama-layout decode token on the device (decoder.hip).
//
// The step of make-llama-step-function (llambda.lisp:6294-6441) as a fixed
// sequence of launches on one stream, every intermediate resident in HBM:
//   token row of token_embd -> x; cos / sin of this position per rotary pair
//   per layer:
//     q|k rows      rms-norm(x) fused in, rotation (+ query scale) fused out,
//                   keys written to the cache slot of this position
//     v rows        rms-norm(x) fused in, values written to the cache slot
//                   (one launch with the q|k rows where their shapes allow)
//     attention     GQA over cache slots 0..position (split over position
//                   chunks of 128, the chunks combined by a second launch)
//     o rows        x += o(context)
//     gate|up rows  rms-norm(x) fused in, silu(g) * u fused out
//     down rows     x += down(h)
//   output rows     rms-norm(x) fused in -> logits
// The token and position are read from device memory (`state`), so one
// captured graph serves every step.
#pragma once

#include "gemv.h"

namespace llhip {

struct DecoderMatrix {
  int type = 0;
  const uint8_t* w = nullptr;
  int64_t row_bytes = 0;
  int64_t rows = 0, columns = 0;
};

struct DecoderLayer {
  const float* attn_norm = nullptr;
  const float* ffn_norm = nullptr;
  // q and k rows in one matrix (q rows first) when their types match;
  // otherwise q and k separately (qk.w == nullptr)
  DecoderMatrix qk, q, k, v, o;
  DecoderMatrix gate_up;  // gate and up rows interleaved in groups of 8
  DecoderMatrix down;
  float* kcache = nullptr;  // [kv_heads][context][head_dim]
  float* vcache = nullptr;
};

struct DecoderPlan {
  int hidden = 0, heads = 0, kv_heads = 0, head_dim = 0, ffn = 0, vocab = 0;
  int context = 0, rope_pairs = 0;
  float eps = 0.f, q_scale = 1.f;
  DecoderMatrix embd, output;
  const float* output_norm = nullptr;
  const DecoderLayer* layers = nullptr;  // host array
  int layer_count = 0;
  // device scratch
  int* state = nullptr;            // [2]: token, position
  const double* rope_denom = nullptr;  // [rope_pairs]: angle = position / denom
  double* rope_cs = nullptr;       // [rope_pairs][2]
  float* x = nullptr;              // [hidden]
  float* q = nullptr;              // [heads * head_dim]
  float* ctx = nullptr;            // [heads * head_dim]
  float* h = nullptr;              // [ffn]
  float* att_part = nullptr;       // [kv_heads][att_chunks][group][head_dim]
  float* att_max = nullptr;        // [kv_heads][att_chunks][group]
  float* att_sum = nullptr;        // [kv_heads][att_chunks][group]
  int att_chunks = 0;              // chunks of the context
};

// Positions per attention workgroup and the longest context.
#ifndef LLHIP_ATTN_CHUNK
#define LLHIP_ATTN_CHUNK 64
#endif
constexpr int kAttnChunk = LLHIP_ATTN_CHUNK;
constexpr int kAttnMaxChunks = 32768 / kAttnChunk;
constexpr int kDecoderMaxContext = kAttnChunk * kAttnMaxChunks;

bool decoder_head_supported(int head_dim, int group);

// state <- (token, position) and the rotation table of the position, as a
// kernel so a captured graph that reads them can follow it on the stream.
hipError_t decoder_state_launch(const DecoderPlan& p, int token, int position, hipStream_t stream);

// Everything after the state: embedding row, the layers and the output rows
// into logits (device, [vocab]).
hipError_t decoder_step_launch(const DecoderPlan& p, float* logits, hipStream_t stream);

// Attention of one layer alone (test hook): q [heads][head_dim] (rotated and
// scaled), caches [kv_heads][context][head_dim], slots 0..state[1].
hipError_t decoder_attention_launch(const DecoderPlan& p, const float* q, const float* kcache,
                                    const float* vcache, float* out, hipStream_t stream);

}  // namespace llhip
