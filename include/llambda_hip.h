/*
 * llambda_hip.h -- C ABI of libllambda_hip.so, the MI355X (gfx950) backend
 * for llambda's quantized decode hot path.
 *
 * The library mirrors the conventions of the reference's native bridge
 * (native/llambda_npu.h:1-70, native/llambda_npu.cpp:1-539):
 *   - every function is extern "C" and takes plain pointers and sizes;
 *   - status ints: 0 = success, -1 = failure with llambda_hip_last_error()
 *     describing it (thread-local; cleared on entry of every call that can
 *     fail); C++ exceptions never cross the boundary;
 *   - status -2 (MoE runs only, LLAMBDA_HIP_INPUT_ERROR): the reference's
 *     own error for this input, last_error holding its text; the session
 *     is healthy and the next call runs normally.  The adapter signals a
 *     plain error for it, not the backend's condition, so the runtime
 *     fallback re-signals it without disabling the layer, as the
 *     reference's CPU body would for that call alone;
 *   - sessions are opaque, owned by the caller, destroyed with a null-safe
 *     destroy; element-count getters return 0 for null;
 *   - a run is synchronous on host pointers: input copied to the device, the
 *     kernels, output copied back, stream synchronised, before returning
 *     (llambda.lisp:294-295, 343-344 pin Lisp arrays only for the call).
 * One session may not be run from two threads at once (the Lisp side holds
 * a per-projection run-mutex, llambda.lisp:4726); different sessions may.
 *
 * GGML type tags are llambda's (llambda.lisp:24-31): F32 = 0, Q5_0 = 6,
 * Q8_0 = 8, Q4_K = 12, Q6_K = 14.  Packed rows are GGUF super-block bytes,
 * verbatim; row r of an N x K tensor starts at r * row_bytes(type, K)
 * (llambda.lisp:2147-2155, 3909-3927).
 */
#ifndef LLAMBDA_HIP_H
#define LLAMBDA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LLAMBDA_HIP_INPUT_ERROR (-2)

typedef struct llambda_hip_session llambda_hip_session;
typedef struct llambda_hip_moe_session llambda_hip_moe_session;
typedef struct llambda_hip_llama_session llambda_hip_llama_session;
typedef struct llambda_hip_sampler llambda_hip_sampler;
typedef struct llambda_hip_gguf llambda_hip_gguf;

/* ---- probe, versions, errors -------------------------------------- */

/* 1 = a gfx950 device is usable, 0 = none, -1 = error (last_error set).
 * Replaces llambda_gpu_probe / llambda_npu_probe (native/llambda_npu.h:25, 45). */
int llambda_hip_probe(void);

/* Replaces llambda_npu_bridge_version (native/llambda_npu.h:26). */
const char* llambda_hip_bridge_version(void);

/* HIP runtime and driver versions.  Replaces llambda_npu_runtime_version
 * (native/llambda_npu.h:27). */
const char* llambda_hip_runtime_version(void);

/* Thread-local description of the last failure.  Replaces
 * llambda_npu_last_error (native/llambda_npu.h:28). */
const char* llambda_hip_last_error(void);

/* Lower-case hex SHA-256 of data into output (output_size >= 65).  Replaces
 * llambda_npu_sha256 (native/llambda_npu.h:29-33), used for projection cache
 * keys (llambda.lisp:2894-2993). */
int llambda_hip_sha256(const void* data, size_t data_size, char* output, size_t output_size);

/* ---- 2-D projection sessions -------------------------------------- */

/* Open a packed-projection file written by the backend's exporter:
 *   bytes 0..7   magic "LLHIPPRJ"
 *   8..11        u32 format version (1)
 *   12..15       u32 GGML type tag
 *   16..23       u64 rows (N)
 *   24..31       u64 columns (K)
 *   32..39       u64 payload bytes (= N * row_bytes(type, K))
 *   40..         payload: the tensor's GGUF bytes, verbatim
 * cache_dir and cache_key are accepted for signature compatibility and not
 * used.  Replaces llambda_npu_session_create (native/llambda_npu.h:35-39),
 * called by make-session-function (accelerator.lisp:42-45). */
int llambda_hip_session_create(const char* model_path, const char* cache_dir,
                               const char* cache_key, llambda_hip_session** result);

/* Upload an N x K tensor straight from host bytes (e.g. the GGUF mapping at
 * the tensor's data offset).  No counterpart in the reference's bridge; it is
 * the zero-copy form of session_create for callers that hold the mapping. */
int llambda_hip_session_create_packed(const void* data, size_t data_size, int ggml_type,
                                      int64_t rows, int64_t columns,
                                      llambda_hip_session** result);

/* Null-safe.  Replaces llambda_npu_session_destroy (native/llambda_npu.h:40). */
void llambda_hip_session_destroy(llambda_hip_session* session);

/* K and N; 0 for null.  Replace llambda_npu_session_{input,output}_element_count
 * (native/llambda_npu.h:41-44), checked at registration (llambda.lisp:2686-2703). */
size_t llambda_hip_session_input_element_count(const llambda_hip_session* session);
size_t llambda_hip_session_output_element_count(const llambda_hip_session* session);

/* output[N] = W x for input[K], synchronous.  -1 on null or count mismatch.
 * Replaces llambda_npu_session_run (native/llambda_npu.h:45-50); the same
 * contract as %gguf-model-matrix-vector-multiply-into (llambda.lisp:4542-4658). */
int llambda_hip_session_run(llambda_hip_session* session, const float* input,
                            size_t input_element_count, float* output,
                            size_t output_element_count);

/* Multi-token form: input [batch][K], output [batch][N], synchronous.  No
 * counterpart in the reference (its prefill is one token at a time,
 * llambda.lisp:1319-1341); row t equals session_run on row t. */
int llambda_hip_session_run_batch(llambda_hip_session* session, const float* input,
                                  size_t input_element_count, float* output,
                                  size_t output_element_count, size_t batch);

/* Device-resident form: input/output are device pointers ([batch][K],
 * [batch][N]); the kernels are enqueued on `stream` (a hipStream_t, or null
 * for the session's own stream) and the call returns without waiting.
 * For callers that keep activations in HBM (and for benchmarking). */
int llambda_hip_session_run_device(llambda_hip_session* session, const float* input,
                                   float* output, size_t batch, void* stream);

/* output[N*K] = the dequantised weights, bit-identical to dequantize-q4-k-m
 * / dequantize-q6-k / dequantize-q5-0 / dequantize-q8-0 (llambda.lisp:
 * 6815-6978, 3965-4009).  Verification hook; synchronous. */
int llambda_hip_session_dequantize(llambda_hip_session* session, float* output,
                                   size_t output_element_count);

/* ---- routed-MoE layer sessions ------------------------------------ */

enum {
  LLAMBDA_HIP_MOE_QWEN3NEXT = 0, /* qwen3next-moe-into, llambda.lisp:5321-5426 */
  LLAMBDA_HIP_MOE_NEMOTRON_H = 1 /* nemotron-h-moe-ffn-into, llambda.lisp:5827-5949 */
};

/* One MoE layer's tensors (host memory, copied at creation).  Expert tensors
 * are the flat GGUF 3-D slabs: rows [e*rows, (e+1)*rows) belong to expert e
 * (llambda.lisp:4951-4971).  Tensor names per llambda.lisp:5321-5426 and
 * 5827-5949 (blk.N.<name>): */
typedef struct llambda_hip_moe_desc {
  int variant;                /* LLAMBDA_HIP_MOE_* */
  int64_t hidden;             /* H */
  int64_t expert_count;       /* E (rows of ffn_gate_inp) */
  int64_t top_k;              /* min(E, expert_used_count) */
  int64_t expert_ffn;         /* F (rows per expert of ffn_up_exps) */
  int64_t shared_ffn;         /* Fs (rows of ffn_up_shexp); 0 = no shared expert */
  const float* router;        /* ffn_gate_inp, F32 [E][H] */
  const float* shared_gate_inp; /* ffn_gate_inp_shexp, F32 [H] (qwen3next) */
  const float* router_bias;   /* exp_probs_b.bias, F32 [E] (nemotron) */
  float expert_weights_scale; /* nemotron_h_moe.expert_weights_scale (default 1) */
  int expert_weights_norm;    /* nemotron_h_moe.expert_weights_norm */
  int gate_type;              /* ffn_gate_exps [E*F][H] (qwen3next) */
  const void* gate_exps;
  int up_type;                /* ffn_up_exps [E*F][H] */
  const void* up_exps;
  int down_type;              /* ffn_down_exps [E*H][F] */
  const void* down_exps;
  int shared_gate_type;       /* ffn_gate_shexp [Fs][H] (qwen3next) */
  const void* shared_gate;
  int shared_up_type;         /* ffn_up_shexp [Fs][H] */
  const void* shared_up;
  int shared_down_type;       /* ffn_down_shexp [H][Fs] */
  const void* shared_down;
  /* ffn_latent_down [Li][H] and ffn_latent_up [H][Lo] (nemotron, each
   * optional, llambda.lisp:5845-5864, 5883-5887, 5933-5938).  With
   * ffn_latent_down the routed experts' input is ffn_latent_down * x, Li
   * wide (ffn_up_exps [E*F][Li]); with ffn_latent_up their weighted sum is
   * Lo wide (ffn_down_exps [E*Lo][F]) and ffn_latent_up maps it back to H
   * before the shared expert is added.  Types: F32, Q4_K, Q6_K, Q5_0, Q8_0. */
  int latent_down_type;
  const void* latent_down;
  int latent_up_type;
  const void* latent_up;
  int64_t latent_in;          /* Li: rows of ffn_latent_down; 0 = none */
  int64_t latent_out;         /* Lo: columns of ffn_latent_up; 0 = none */
} llambda_hip_moe_desc;

/* Upload one layer.  No counterpart in the reference's bridge (its routed
 * experts bypass the accelerator store, llambda.lisp:4951-4971); this is the
 * per-layer hook, bound per layer index in a table of its own beside the
 * tensor-indexed projection store (never under a tensor name, so the 2-D
 * router projection blk.N.ffn_gate_inp.weight stays a 2-D binding). */
int llambda_hip_moe_session_create(const llambda_hip_moe_desc* desc,
                                   llambda_hip_moe_session** result);

void llambda_hip_moe_session_destroy(llambda_hip_moe_session* session);

/* H; 0 for null.  Registration checks it against the columns of the layer's
 * ffn_gate_inp (the MoE counterpart of the N x K check, llambda.lisp:2686-2703). */
size_t llambda_hip_moe_session_hidden_size(const llambda_hip_moe_session* session);

/* E (rows of ffn_gate_inp); 0 for null. */
size_t llambda_hip_moe_session_expert_count(const llambda_hip_moe_session* session);

/* output[batch][H] = the layer's FFN output (before the residual add) for
 * input[batch][H], token by token as the reference computes it.  Synchronous.
 * top_indices / top_weights (optional, [batch][k]) receive the selected
 * experts in rank order and their final weights; router_logits (optional,
 * [batch][E]) the router logits (after the bias for nemotron).  Returns
 * LLAMBDA_HIP_INPUT_ERROR (-2) with the reference's error text when it would
 * have signalled one for this input (non-positive weight sum,
 * llambda.lisp:5373-5375 and 5903-5905; fewer than k selectable logits);
 * output then holds no result.  -1 for every other failure. */
int llambda_hip_moe_session_run(llambda_hip_moe_session* session, const float* input,
                                size_t input_element_count, float* output,
                                size_t output_element_count, size_t batch,
                                int64_t* top_indices, float* top_weights,
                                float* router_logits);

/* Device-resident form; enqueues on `stream` (null = the session's stream)
 * and returns without waiting.  Errors raised by the kernels are reported by
 * the next llambda_hip_moe_session_sync. */
int llambda_hip_moe_session_run_device(llambda_hip_moe_session* session, const float* input,
                                       float* output, size_t batch, void* stream);

/* Wait for `stream` (null = the session's stream) and report any error flag
 * raised by the kernels since the last check (LLAMBDA_HIP_INPUT_ERROR, as
 * llambda_hip_moe_session_run). */
int llambda_hip_moe_session_sync(llambda_hip_moe_session* session, void* stream);

/* The device-resident run above with no allocation of any kind (no hipMalloc,
 * hipFree or allocating library call), for callers that cannot allocate:
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * it.  No counterpart in the reference.  The forward's scratch (router
 * logits and slice sums, top-k, histogram, permutation, chunk table, split
 * activations, per-pair expert outputs) lives in one file-scope device array
 * of 32 MiB per GPU, held until the process ends; a call whose batch needs
 * more (the layer's per-token scratch times `batch`; e.g. Qwen3Next-shaped
 * layers up to 251 tokens, Nemotron-H-shaped ones up to 166) is
 * refused with an error, before anything is enqueued.  Every call on a GPU
 * shares that GPU's array, which keeps the last call's contents, so the calls
 * are ordered on the device: each call's stream first waits for the previous
 * call's last launch (an event recorded on its stream), whatever stream or
 * session it came from.  Under stream capture no wait or record is made:
 * the graph orders its own calls, and replays of graphs holding such calls
 * must not overlap on one GPU.  Errors raised by the kernels reach the
 * session's flag and are reported by llambda_hip_moe_session_sync. */
int llambda_hip_moe_session_run_device_noalloc(llambda_hip_moe_session* session,
                                               const float* input, float* output, size_t batch,
                                               void* stream);

/* ---- routing primitive ---------------------------------------------- */

/* For each of `batch` rows of n logits, the k selected by
 * select-top-k-logits-into (llambda.lisp:5265-5292): descending, lower
 * index first among equal values, NaN and values <= -FLT_MAX never chosen,
 * unfilled slots (-1, -FLT_MAX).  Host pointers, synchronous, on the device. */
int llambda_hip_select_top_k(const float* logits, size_t n, size_t k, size_t batch,
                             int64_t* top_indices, float* top_logits);

/* ---- measurement ------------------------------------------------------ */

#define LLAMBDA_HIP_STREAM_READ_WORDS 4096

/* A plain streaming read of `bytes` of device memory (16-byte aligned, a
 * multiple of 16): LLAMBDA_HIP_STREAM_READ_WORDS wavefronts each read one
 * contiguous slice with 16-byte loads and store the XOR of what they read in
 * out[wave] (device memory, LLAMBDA_HIP_STREAM_READ_WORDS words).  Enqueued
 * on `stream` (null = the null stream), not waited for.  No counterpart in
 * the reference: it measures the HBM read rate the device sustains, the
 * ceiling beside 8 TB/s against which bench.py reads the GEMV figures. */
int llambda_hip_stream_read(const void* data, size_t bytes, uint32_t* out, void* stream);

/* ---- Llama-layout decode token ---------------------------------------- */

/* One packed 2-D tensor: GGML type tag and its rows (rows * row_bytes bytes,
 * host memory, or device memory when the descriptor says so). */
typedef struct llambda_hip_tensor_ref {
  int type;
  const void* data;
  size_t bytes;
} llambda_hip_tensor_ref;

/* Tensors of layer N (blk.N.<name>.weight, llambda.lisp:6294-6441). */
typedef struct llambda_hip_llama_layer {
  const float* attn_norm;             /* attn_norm, F32 [hidden], host */
  llambda_hip_tensor_ref attn_q;      /* [heads * head_dim][hidden] */
  llambda_hip_tensor_ref attn_k;      /* [kv_heads * head_dim][hidden] */
  llambda_hip_tensor_ref attn_v;      /* [kv_heads * head_dim][hidden] */
  llambda_hip_tensor_ref attn_output; /* [hidden][heads * head_dim] */
  const float* ffn_norm;              /* ffn_norm, F32 [hidden], host */
  llambda_hip_tensor_ref ffn_gate;    /* [ffn][hidden] */
  llambda_hip_tensor_ref ffn_up;      /* [ffn][hidden] */
  llambda_hip_tensor_ref ffn_down;    /* [hidden][ffn] */
} llambda_hip_llama_layer;

/* Model hyper-parameters as load-llama-model reads them
 * (llambda.lisp:6269-6292) and its tensors.  Quantised tensors must be
 * Q4_K or Q6_K with a column count divisible by 256; q and k (and gate and
 * up) of a layer that share a type are stored side by side on the device. */
typedef struct llambda_hip_llama_desc {
  int64_t hidden;             /* llama.embedding_length */
  int64_t layer_count;        /* llama.block_count */
  int64_t head_count;         /* llama.attention.head_count */
  int64_t kv_head_count;      /* llama.attention.head_count_kv */
  int64_t ffn;                /* llama.feed_forward_length */
  int64_t vocab;              /* rows of token_embd and output */
  int64_t rope_dimension;     /* llama.rope.dimension_count */
  float norm_epsilon;         /* llama.attention.layer_norm_rms_epsilon */
  float rope_base;            /* llama.rope.freq_base */
  const float* rope_factors;  /* rope_freqs.weight, host, NULL if absent */
  int64_t rope_factor_count;
  int64_t context;            /* KV cache slots (positions) to allocate */
  int weights_on_device;      /* 1: tensor data pointers are device memory */
  llambda_hip_tensor_ref token_embd;  /* [vocab][hidden] */
  llambda_hip_tensor_ref output;      /* [vocab][hidden] */
  const float* output_norm;           /* output_norm, F32 [hidden], host */
  const llambda_hip_llama_layer* layers; /* [layer_count] */
} llambda_hip_llama_desc;

/* Upload a model for device-resident decoding, with a zeroed fp32 KV cache
 * of `context` slots per layer.  No counterpart in the reference's bridge:
 * this is the model-level hook for make-llama-step-function
 * (llambda.lisp:6294-6441), whose step runs every projection, norm,
 * rotation and attention of a token on the device. */
int llambda_hip_llama_session_create(const llambda_hip_llama_desc* desc,
                                     llambda_hip_llama_session** result);

void llambda_hip_llama_session_destroy(llambda_hip_llama_session* session);

/* vocab; 0 for null. */
size_t llambda_hip_llama_session_vocab(const llambda_hip_llama_session* session);

/* One decode step of the step function (token-id position) -> logits
 * (llambda.lisp:6315-6441): the token's keys and values go to cache slot
 * `position`, attention covers slots 0..position.  logits: host [vocab].
 * Synchronous. */
int llambda_hip_llama_session_step(llambda_hip_llama_session* session, int64_t token,
                                   int64_t position, float* logits, size_t logits_count);

/* Device-resident form: logits is device memory [vocab] (null = the
 * session's own logits buffer, read back with llambda_hip_llama_session_logits);
 * enqueued on `stream` (null = the session's stream).  use_graph = 1 replays
 * a HIP graph of the step captured on the first call for these logits.
 * Steps of one session are ordered whatever streams they are given: each
 * waits on the device for the previous one (they share the position word,
 * the cache and the logits), and _logits, _sample, _read_kv, _write_kv and
 * _sync wait for the last one. */
int llambda_hip_llama_session_step_device(llambda_hip_llama_session* session, int64_t token,
                                          int64_t position, float* logits, void* stream,
                                          int use_graph);

/* Copy the session's own logits buffer (the last step_device with null
 * logits) to host memory after waiting for the session's stream. */
int llambda_hip_llama_session_logits(llambda_hip_llama_session* session, float* logits,
                                     size_t logits_count);

/* Copy cache slots [first, first + count) of `layer` in or out: keys and
 * values are [kv_heads][count][head_dim] fp32 (host memory, or device
 * memory for write when on_device = 1).  Synchronous. */
int llambda_hip_llama_session_write_kv(llambda_hip_llama_session* session, int64_t layer,
                                       int64_t first, int64_t count, const float* keys,
                                       const float* values, int on_device);
int llambda_hip_llama_session_read_kv(llambda_hip_llama_session* session, int64_t layer,
                                      int64_t first, int64_t count, float* keys, float* values);

/* Wait for `stream` (null = the session's stream). */
int llambda_hip_llama_session_sync(llambda_hip_llama_session* session, void* stream);

/* ---- sampling ------------------------------------------------------------ */

/* Keyword arguments of sample-token-id-from-logits (llambda.lisp:1272-1317),
 * with the random value explicit (the reference's :random-value). */
typedef struct llambda_hip_sampling {
  const int64_t* history;     /* host, token ids already generated (may repeat) */
  size_t history_count;
  float repetition_penalty;   /* reference default 1.15 */
  int64_t top_k;              /* reference default 40; 0 disables */
  float top_p;                /* reference default 0.95; 1 disables */
  float temperature;          /* reference default 1.0 */
  float random_value;         /* in [0, 1) */
} llambda_hip_sampling;

/* Device scratch for logits rows of up to `vocab` entries.  No counterpart in
 * the reference's bridge: sampling runs in Lisp there (llambda.lisp:1036-1317). */
int llambda_hip_sampler_create(size_t vocab, llambda_hip_sampler** result);
void llambda_hip_sampler_destroy(llambda_hip_sampler* sampler);

/* The token sample-token-id-from-logits draws from logits[count] (host
 * memory, or device memory when logits_on_device = 1); the logits are not
 * modified.  With top-k (1 <= top_k < count) the token is the reference's bit
 * for bit; without top-k the token matches wherever the random value, and with
 * top_p < 1 the running sum at the top-p cut, is not within rounding of a
 * cumulative boundary (the whole row is ranked and summed in a fixed tree
 * order).  Errors: the reference's argument errors, NaN logits, more than 4096
 * logits tied at or above the top-k cutoff.  Synchronous. */
int llambda_hip_sampler_sample(llambda_hip_sampler* sampler, const float* logits, size_t count,
                               int logits_on_device, const llambda_hip_sampling* params,
                               int64_t* token);

/* Sample from a llama session's own logits buffer (after
 * llambda_hip_llama_session_step_device with null logits). */
int llambda_hip_llama_session_sample(llambda_hip_llama_session* session,
                                     llambda_hip_sampler* sampler,
                                     const llambda_hip_sampling* params, int64_t* token);

/* ---- GGUF files ------------------------------------------------------------ */

/* One tensor info of read-gguf-tensor-infos (llambda.lisp:2147-2238).  name
 * and data point into the mapping (valid until close; name is not
 * NUL-terminated). */
typedef struct llambda_hip_gguf_tensor {
  const char* name;
  size_t name_length;
  uint32_t dimension_count;    /* 1..4 */
  uint64_t dimensions[4];      /* GGUF order: dimensions[0] = columns */
  uint32_t type;               /* GGML type tag */
  uint64_t offset;             /* relative to the tensor data start */
  uint64_t element_count;
  int supported;               /* supported-ggml-type-p */
  uint64_t byte_size;          /* 0 when unsupported */
  uint64_t data_offset;        /* absolute file offset */
  const void* data;            /* mapping + data_offset */
} llambda_hip_gguf_tensor;

/* One metadata value (read-gguf-value, llambda.lisp:1985-2045): the key
 * (metadata entries only), the GGUF value type (0 u8, 1 i8, 2 u16, 3 i16,
 * 4 u32, 5 i32, 6 f32, 7 bool, 8 string, 9 array, 10 u64, 11 i64, 12 f64),
 * integers in u / i, floats in f, booleans as u = 0 / 1, strings as bytes
 * in the mapping (not NUL-terminated), arrays as element_type and count. */
typedef struct llambda_hip_gguf_value {
  const char* key;
  size_t key_length;
  uint32_t type;
  uint32_t element_type;
  uint64_t count;
  uint64_t u;
  int64_t i;
  double f;
  const char* string;
  size_t string_length;
} llambda_hip_gguf_value;

/* Open and map a GGUF file read-only and parse its header, metadata and
 * tensor infos with every read bounded by the file length; errors carry the
 * reference's texts ("... exceeds mapped file length ...", "Invalid GGUF
 * magic", "... invalid dimension count ...").  Replaces call-with-file and
 * with-mapped-file (llambda.lisp:489-675, Win32) with open/fstat/mmap. */
int llambda_hip_gguf_open(const char* path, llambda_hip_gguf** result);
void llambda_hip_gguf_close(llambda_hip_gguf* file);

/* read-gguf-header (llambda.lisp:2047-2059) plus the alignment
 * (general.alignment, default 32) and the tensor data start. */
int llambda_hip_gguf_header(const llambda_hip_gguf* file, uint32_t* version,
                            uint64_t* tensor_count, uint64_t* kv_count, uint64_t* alignment,
                            uint64_t* data_start);

/* The mapping (size in *size); tensor data for zero-copy uploads. */
const void* llambda_hip_gguf_mapping(const llambda_hip_gguf* file, size_t* size);

int llambda_hip_gguf_tensor_info(const llambda_hip_gguf* file, uint64_t index,
                                 llambda_hip_gguf_tensor* out);
/* Index of the first tensor named `name`, -1 when absent (find-gguf-tensor-info). */
int64_t llambda_hip_gguf_find_tensor(const llambda_hip_gguf* file, const char* name);

/* Metadata entry `index` in file order; array elements by
 * llambda_hip_gguf_kv_element. */
int llambda_hip_gguf_kv(const llambda_hip_gguf* file, uint64_t index, llambda_hip_gguf_value* out);
int llambda_hip_gguf_kv_element(const llambda_hip_gguf* file, uint64_t index, uint64_t element,
                                llambda_hip_gguf_value* out);

#ifdef __cplusplus
}
#endif

#endif
