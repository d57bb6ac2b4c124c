/*
 * llambda_oracle.h -- CPU restatement of llambda's quantized decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path and the source of the reported CPU baseline.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the checker or the baseline, never as the thing measured or shipped.
 *
 * Every function restates one function of the reference (Common Lisp,
 * llambda.lisp) and cites the file:line it follows.  Arithmetic order is the
 * reference's: single-precision products and sums are rounded separately
 * (the library is compiled with -ffp-contract=off) and only the reference's
 * explicit f32.8-fmadd steps use fmaf().
 *
 * Parity pins (what checks each function beyond retyping it):
 *   fp16 decode          all 65536 bit patterns vs numpy.float16 (tests)
 *   get_scale_min_k4     independent bit-field decode of all 256 values of
 *                        each scale byte position (tests)
 *   dequantize Q4_K/Q6_K reference KATs tests.lisp:2386-2450, 2324-2367
 *   fused Q4_K/Q6_K dot  reference KATs tests.lisp:2257-2322 plus float64
 *                        dot of the dequantised row on random blocks
 *   Q5_0/Q8_0            float64 closed forms of the block formulas
 *   f32 dot              numpy float32 sequential accumulate (bit-exact)
 *   select_top_k         stable descending sort with NaN excluded
 *   sigmoid/silu/relu2   float64 closed forms
 *   MoE layers           float64 restatement from dequantised weights
 *   Nemotron latent      float64 restatement with ffn_latent_down/up; identity
 *                        down and permutation up equal the latent-free layer
 *                        permuted, bit for bit
 *                        (independent of the fused kernels)
 *   rms_norm, silu,      reference KATs tests.lisp:298-345 (rms-norm of
 *   rope, softmax        (3 4) by (1 2), silu 2, rotation by cos/sin 1,
 *                        softmax of (2 1 0)), plus closed forms: rotation
 *                        preserves the pair's norm and is the identity at
 *                        position 0, softmax sums to 1 and is shift
 *                        invariant, rms of the output equals rms of w
 *   attention            float64 restatement; one slot returns its value
 *                        row, identical keys return the mean value row
 *   llama step           float64 restatement of the layer from dequantised
 *                        weights (tests)
 *   sampling             reference KATs tests.lisp:1258-1375 (penalty, top-k,
 *                        top-p, draw, the default top-k of 40); top-k against
 *                        a sort (the k-th largest value, ties kept); top-p
 *                        against a float64 cumulative on a stable sort
 *   horizontal+ of the 8-lane accumulator: sb-simd's internal order is not
 *   published; this file sums lanes 0..7 left to right.  Parity unpinned for
 *   that order; it moves results by a few ulp, far inside the 1e-4 bound.
 */
#ifndef LLAMBDA_ORACLE_H
#define LLAMBDA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type tags, llambda.lisp:24-31. */
enum {
  ORACLE_TYPE_F32 = 0,
  ORACLE_TYPE_Q5_0 = 6,
  ORACLE_TYPE_Q8_0 = 8,
  ORACLE_TYPE_Q4_K = 12,
  ORACLE_TYPE_Q6_K = 14
};

const char* oracle_last_error(void);

/* llambda.lisp:2126-2155 */
int64_t oracle_type_block_elements(int type);
int64_t oracle_type_block_bytes(int type);
int64_t oracle_row_bytes(int type, int64_t columns); /* -1 on error */

/* llambda.lisp:716-733 (fp16-to-single-float) */
int oracle_fp16_to_f32(uint16_t bits, float* out);

/* llambda.lisp:6794-6813 and 4316-4336 */
void oracle_get_scale_min_k4(const uint8_t* scales, int index, int* scale, int* min);

/* Scalar dequantisers: llambda.lisp:6815-6859, 6919-6978, 3965-4009 */
int oracle_dequantize(int type, const uint8_t* src, int64_t elements, float* dst);

/* Fused row dots: llambda.lisp:4338-4382 (Q4_K), 4446-4506 (Q6_K),
 * 4037-4094 (Q5_0, Q8_0), 4096-4107 (F32). */
int oracle_dot_row(int type, const uint8_t* row, const float* x, int64_t columns, float* out);

/* llambda.lisp:3491-3500 (dot-product) */
float oracle_dot_product(const float* left, const float* right, int64_t n);

/* Row-parallel GEMV, llambda.lisp:4542-4658 with the worker runtime of
 * 769-817: Q4_K/Q6_K use min(rows, threads) contiguous parts when
 * rows >= 96; other types run serially.  threads <= 0 means 1. */
int oracle_gemv(int type, const uint8_t* matrix, int64_t rows, int64_t columns,
                const float* x, float* y, int threads);

/* llambda.lisp:5265-5292 */
void oracle_select_top_k(const float* logits, int64_t n, int64_t k,
                         int64_t* top_indices, float* top_logits);

/* llambda.lisp:926-940 */
float oracle_sigmoid(float x);
float oracle_silu(float x);
float oracle_relu_squared(float x);

/* One routed-MoE layer description.  Expert tensors are the flat GGUF
 * [E * rows][columns] slabs (llambda.lisp:4951-4971). */
typedef struct oracle_moe_desc {
  int variant;                 /* 0 = qwen3next, 1 = nemotron_h_moe */
  int64_t hidden;              /* H */
  int64_t expert_count;        /* E */
  int64_t top_k;               /* k, already min(E, used count) */
  int64_t expert_ffn;          /* F */
  int64_t shared_ffn;          /* Fs, 0 when there is no shared expert */
  const float* router;         /* F32 [E][H] */
  const float* shared_gate_inp;/* F32 [H], qwen3next only */
  const float* router_bias;    /* F32 [E], nemotron only (exp_probs_b.bias) */
  float expert_weights_scale;  /* nemotron only */
  int expert_weights_norm;     /* nemotron only */
  int gate_type;  const uint8_t* gate_exps;   /* qwen3next only: [E*F][H] */
  int up_type;    const uint8_t* up_exps;     /* [E*F][H] */
  int down_type;  const uint8_t* down_exps;   /* [E*H][F] */
  int shared_gate_type; const uint8_t* shared_gate; /* [Fs][H], qwen3next */
  int shared_up_type;   const uint8_t* shared_up;   /* [Fs][H] */
  int shared_down_type; const uint8_t* shared_down; /* [H][Fs] */
  /* nemotron only, each optional (llambda.lisp:5845-5864): ffn_latent_down
   * [Li][H] gives the routed experts an Li-wide input (up_exps [E*F][Li]);
   * ffn_latent_up [H][Lo] maps their Lo-wide weighted sum back to H
   * (down_exps [E*Lo][F]).  0 when the layer has no such tensor. */
  int64_t latent_in;            /* Li: rows of ffn_latent_down */
  int latent_down_type; const uint8_t* latent_down;
  int latent_up_type;   const uint8_t* latent_up;
  int64_t latent_out;           /* Lo: columns of ffn_latent_up */
} oracle_moe_desc;

/* llambda.lisp:5321-5426 (qwen3next-moe-into) and 5827-5949
 * (nemotron-h-moe-ffn-into), run token by token as the reference's
 * prefill does (llambda.lisp:1319-1341).  x, y: [tokens][H].  The optional
 * outputs receive the selected experts and their final weights per token
 * ([tokens][k]) and the router logits ([tokens][E], after the bias for
 * nemotron). */
int oracle_moe_forward(const oracle_moe_desc* desc, const float* x, float* y,
                       int64_t tokens, int64_t* top_indices, float* top_weights,
                       float* router_logits, int threads);

/* ---- Llama decode token (llambda.lisp:6294-6441) ---------------------- */

/* llambda.lisp:819-828, 859-879 */
void oracle_rms_norm(const float* x, const float* w, int64_t n, float eps, float* out);
/* llambda.lisp:3760-3795 */
void oracle_rope_head(float* head, int64_t len, int64_t position, int64_t rope_dim,
                      float theta_base, const float* factors, int64_t n_factors);
/* llambda.lisp:5075-5096 */
void oracle_softmax(const float* logits, int64_t n, float* out);
/* llambda.lisp:5122-5167: q [heads][D], caches [kv_heads][cap][D], slots 0..n-1 */
int oracle_attention(const float* q, const float* kc, const float* vc, int64_t cap, int64_t n,
                     int64_t heads, int64_t kv_heads, int64_t D, float* out);

typedef struct oracle_tensor {
  int type;
  const uint8_t* data;
} oracle_tensor;

typedef struct oracle_llama_layer {
  const float* attn_norm;
  oracle_tensor attn_q, attn_k, attn_v, attn_output;
  const float* ffn_norm;
  oracle_tensor ffn_gate, ffn_up, ffn_down;
} oracle_llama_layer;

typedef struct oracle_llama_desc {
  int64_t hidden, layer_count, heads, kv_heads, ffn, vocab, rope_dim;
  float norm_eps, rope_base;
  const float* rope_factors;
  int64_t rope_factor_count;
  oracle_tensor token_embd, output;
  const float* output_norm;
  const oracle_llama_layer* layers;
} oracle_llama_desc;

/* llambda.lisp:6315-6441; kv: [layers][2][kv_heads][cap][head_dim] */
int oracle_llama_step(const oracle_llama_desc* m, float* kv, int64_t cap, int64_t token,
                      int64_t position, float* logits, int threads);
int oracle_llama_step_hidden(const oracle_llama_desc* m, float* kv, int64_t cap, int64_t token,
                             int64_t position, float* logits, float* hidden, int threads);

/* ---- sampling (llambda.lisp:1036-1317) ------------------------------ */
int oracle_repetition_penalty(float* logits, int64_t n, const int64_t* history, int64_t nh,
                              float penalty);                       /* 1036-1086 */
int oracle_top_k(float* logits, int64_t n, int64_t k);              /* 1088-1150 */
int oracle_top_p(float* logits, int64_t n, float p, float temperature); /* 1163-1240 */
int64_t oracle_sample_from_probabilities(const float* probs, int64_t n, float roll); /* 1253-1270 */
int oracle_sample_token(float* logits, int64_t n, const int64_t* history, int64_t nh,
                        float penalty, int64_t top_k, float top_p, float temperature, float roll,
                        int64_t* token);                            /* 1272-1317 */

#ifdef __cplusplus
}
#endif

#endif
