// moe.h -- routed-MoE feed-forward on one GPU (moe.hip).
//
// One forward of qwen3next-moe-into (llambda.lisp:5321-5426) or
// nemotron-h-moe-ffn-into (llambda.lisp:5827-5949) for a batch of tokens,
// as a fixed sequence of launches on one stream:
//   1 router GEMV (F32)              logits[t][e]  (+ shared-gate dot, qwen3next)
//   2 top-k + gating, one wavefront per token
//   3 histogram, scan + scatter (one workgroup): token-to-expert permutation
//     and the chunk table of (expert, first pair, pair count) work items
//   4 grouped up: gate/up rows of each expert against its chunk of tokens,
//     activation fused (silu(g)*u, or relu(u)^2)
//   5 grouped down: down rows against the chunk's activations, per pair
//   6 combine in rank order, then the shared expert
// A Nemotron-H layer with ffn_latent_down also runs that projection on x
// and splits its output after 1 (the routed up products read it); with
// ffn_latent_up, 6 forms the latent-wide weighted sum, then ffn_latent_up and
// the shared expert's addition follow.
#pragma once

#include "gemv.h"

namespace llhip {

enum MoeVariant : int { kQwen3Next = 0, kNemotronH = 1 };

// Chunk work item of the grouped expert kernels.
struct MoeChunk {
  int expert;  // slab index within its group (routed: expert id; shared: 0)
  int start;   // first entry of the permutation
  int count;   // pairs in this chunk (1..64)
};

constexpr int kMoeMaxExperts = 1024;
constexpr int kMoeMaxTopK = 64;

// Device-side description of one layer and its scratch, all device pointers.
struct MoePlan {
  int variant;
  int hidden, experts, top_k, ffn, shared_ffn;
  float weights_scale;
  int weights_norm;
  // weights.  Expert tensors of a K-quant type (Q4_K, Q6_K) are held in the
  // tile-major layout (moe_tile_launch), the others as packed GGUF rows;
  // moe_slab_bytes gives one expert's bytes in either.
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
  // ffn_latent_down [latent_in] rows of hidden and ffn_latent_up [hidden]
  // rows of latent_out (nemotron, each optional: 0 = absent).  The routed
  // up rows are latent_in (else hidden) wide, the routed down rows number
  // latent_out (else hidden).
  int latent_in, latent_out;
  int lat_down_type, lat_up_type;
  const uint8_t* lat_down;
  const uint8_t* lat_up;
  int out_w;           // row stride of down_out: max(hidden, latent_out)
  // the group pipeline's one-matrix launches (Q5_0 / Q8_0: relu^2 up, down)
  // read these stage-major copies (moe_repack_launch); slab strides in bytes
  const uint8_t* up_g;
  const uint8_t* down_g;
  const uint8_t* sh_up_g;
  const uint8_t* sh_down_g;
  int64_t up_g_stride, down_g_stride;
  // scratch, sized for `capacity` tokens
  int capacity;
  float* logits;       // [capacity][experts + 1]
  float* router_part;  // [router_ks][capacity][experts + 1]  router K-slice sums
  int router_ks;
  int* top_idx;        // [capacity][top_k]
  float* top_w;        // [capacity][top_k]
  float* shared_w;     // [capacity]
  int* perm;           // [capacity * (top_k + 1)]
  MoeChunk* chunks;    // [max_chunks(capacity)]
  int* chunk_counts;   // [2]: routed chunks, shared chunks
  // split rows (moe_mfma.hip) of the multi-token path
  uint16_t* xq;        // [capacity][2 hidden]           x as bf16 hi/lo
  float* xsum;         // [capacity][hidden/16]          16-group sums
  uint16_t* aq;        // [capacity * (top_k + 1)][2 act_width]  activations
  float* asum;         // [capacity * (top_k + 1)][act_width/16]
  float* down_out;     // [capacity * (top_k + 1)][out_w]
  // latent layers only
  float* lat;          // [capacity][latent_in], later [capacity][latent_out]:
                       // the experts' input, then their weighted sum
  uint16_t* lq;        // [capacity][2 latent_in]        its split rows
  float* lsum;         // [capacity][latent_in/16]       and their sums
  float* lat_y;        // [capacity][hidden]             ffn_latent_up output
  int* error;          // [1] nonzero after a run that hit a reference error
};

// Grouped expert product over a chunk table (moe_mfma.hip).
enum MoeEpilogue : int {
  kEpiSwiglu = 0,  // gate and up rows -> split silu(g) * u
  kEpiRelu2 = 1,   // up rows -> split relu(u)^2
  kEpiDown = 2,    // down rows -> fp32 output per pair
};

struct MoeGemmArgs {
  // work: chunk table entries of `group` (routed 0, shared 1)
  const MoeChunk* chunks;
  const int* chunk_counts;
  int group;
  const int* perm;
  int pairs;       // tokens * top_k: pair ids >= pairs are shared-expert pairs
  int top_k;
  int a_by_token;  // A row = the pair's token (1) or the pair itself (0)
  // A: split rows
  const uint16_t* aq;
  int64_t aq_stride;  // u16 per row
  const float* as;
  int64_t as_stride;  // floats per row (16-group sums)
  int K;
  // B: expert slabs of packed rows
  const uint8_t* w0;  // gate (swiglu) or up / down
  const uint8_t* w1;  // up (swiglu)
  int64_t row_bytes;
  int64_t expert_stride;
  int N;
  // output: split activations (swiglu, relu2) or fp32 rows (down)
  uint16_t* oq;
  int64_t oq_stride;
  float* os;
  int64_t os_stride;
  float* out;
  int64_t out_stride;
  int depth;      // LDS stages per wave (set by the launcher)
  int row_tiles;  // row-tile groups of the grid (set by the launcher)
  int tiles_per_wg;  // consecutive row tiles per workgroup (set by the launcher)
  // routed and shared chunks in one launch (same weight type): the shared
  // expert's tensors, rows and K
  int joint;
  const uint8_t* s_w0;
  const uint8_t* s_w1;
  int64_t s_row_bytes;
  int s_N, s_K;
  // one token, up products: the launch selects and gates the token itself
  // (top-k over router_part, gate_jpl = logits per lane); x index 0 is the
  // shared expert (joint), then the valid ranks in rank order
  int fused_gate;
  int gate_jpl;
  MoePlan plan;
};

// Router logits of T tokens (fp32 MFMA) as router_slices(H) partial sums
// part[slice][t][e] (row stride ld), and the split rows of x (q, s).
int router_slices(int H);
hipError_t router_mfma_launch(const float* x, int T, const float* R, int Er, int H, float* part,
                              int ld, uint16_t* q, int64_t q_stride, float* s, int64_t s_stride,
                              hipStream_t stream);
// The split rows (format above router_mfma_launch's q, s) of T rows of K
// fp32 elements, K % 32 == 0, rows x_stride floats apart.
hipError_t split_rows_launch(const float* x, int T, int K, int64_t x_stride, uint16_t* q,
                             int64_t q_stride, float* s, int64_t s_stride, hipStream_t stream);
// mt: 0 = one token (K split over four wavefronts), 1 = chunks of up to 16
// pairs (double-buffered), 2 = chunks of up to 32 pairs, 4 = chunks of up to
// 64 pairs, activations shared by the workgroup (32-weight block types only:
// moe_group_pipeline_types).
hipError_t moe_gemm_launch(int type, int epi, const MoeGemmArgs& a, int mt, int max_chunks,
                           hipStream_t stream);
bool moe_group_pipeline_types(int type);
// The stage-major copy of `slabs` slabs of `rows` packed rows of `columns`
// (Q5_0 / Q8_0) that the group pipeline's one-matrix launches read: per slab,
// per 64-row tile, per stage of two 32-blocks, the 64 rows' two blocks back
// to back (zeros past the slab's rows and past an odd block count).
int64_t moe_repack_bytes(int type, int64_t slabs, int64_t rows, int64_t columns);
hipError_t moe_repack_launch(int type, const uint8_t* src, int64_t slabs, int64_t rows,
                             int64_t columns, uint8_t* dst, hipStream_t stream);
// The tile-major layout of K-quant (Q4_K, Q6_K) expert tensors, which the
// grouped products and the one-token down+combine read: per slab, per
// 16-row tile, per 256-weight chunk, the 16 rows' chunks back to back, each
// padded to a dword (Q4_K 144 bytes, Q6_K 212); rows past the slab's are
// zeros.  A wave's stage of a chunk is then one contiguous run whose rows
// start on dwords.  In a Q6_K chunk each 32-byte run of ql and qh (its first
// 192 bytes) holds dword 4s + g of the GGUF run at dword 2g + s.  moe_slab_bytes: one slab's bytes in the device layout of
// `type` (tile-major for K-quants, packed rows otherwise).
bool moe_tiled_type(int type);
int64_t moe_slab_bytes(int type, int64_t rows, int64_t columns);
hipError_t moe_tile_launch(int type, const uint8_t* src, int64_t slabs, int64_t rows,
                           int64_t columns, uint8_t* dst, hipStream_t stream);

// One token's down products and their combine in one launch (moe_mfma.hip):
// a.chunks / a.chunk_counts / a.perm as topk_gate_kernel writes them for a
// single token; routed and shared down rows of one weight type (a.joint, or
// no shared expert).  y = sum over valid ranks r (in order) of top_w[r] *
// down_r, then + shared_w * down_shared (shared_scaled) or + down_shared.
struct MoeCombineArgs {
  float* y;               // [hidden]
  const float* top_w;     // [top_k] gating weights by rank
  const float* shared_w;  // [1] shared-expert gate
  int shared_scaled;      // 1: Qwen3Next's sigmoid-gated shared expert; 0: Nemotron-H's
  const int* error;       // [1] the run's error word
  int* error_out;         // [1] optional copy of it (see moe_forward_launch)
};
bool moe_down_combine_supported(int type, const MoeGemmArgs& a);
hipError_t moe_down_combine_launch(int type, const MoeGemmArgs& a, const MoeCombineArgs& c,
                                   hipStream_t stream);

// Upper bound of the chunk table for `tokens` tokens with chunk size nt.
int64_t moe_max_chunks(const MoePlan& p, int64_t tokens, int nt);

// Enqueue one forward for `tokens` tokens: x, y are [tokens][hidden] in
// memory the device can address.  `error` codes (bit flags): 1 = fewer than
// k finite router logits, 2 = non-positive weight sum, 4 = expert index out
// of range.  With `error_out`, the final launch also stores the run's error
// word there (host-mapped memory, read after the stream is synchronised).
hipError_t moe_forward_launch(const MoePlan& p, const float* x, float* y, int tokens,
                              hipStream_t stream, int* error_out = nullptr);

// Zero the error flag (a fill kernel, so that a captured graph replays it).
hipError_t moe_reset_launch(const MoePlan& p, hipStream_t stream);

// OR the flags at src into dst (one thread; no host round trip).
hipError_t moe_error_merge_launch(const int* src, int* dst, hipStream_t stream);

// Batched device top-k with the reference's selection rule (test hook).
hipError_t topk_launch(const float* logits, int n, int k, int batch, int* idx, float* val,
                       hipStream_t stream);

}  // namespace llhip
