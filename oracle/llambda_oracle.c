/*
 * llambda_oracle.c -- CPU restatement of llambda's quantized decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the CPU baseline.  The
 * product (libllambda_hip.so) never links or calls this file.
 *
 * Build: oracle/Makefile, with -ffp-contract=off so that only the explicit
 * fmaf() calls (the reference's f32.8-fmadd) fuse.
 */
#include "llambda_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define QK_K 256           /* llambda.lisp:21 +qk-k+ */
#define K_SCALE_SIZE 12    /* llambda.lisp:22 +k-scale-size+ */
#define Q4_K_BYTES 144     /* 4 + 12 + 128, llambda.lisp:2142 */
#define Q6_K_BYTES 210     /* 2 + 16 + 192, llambda.lisp:2144 */
#define Q5_0_BYTES 22      /* llambda.lisp:2139 */
#define Q8_0_BYTES 34      /* llambda.lisp:2140 */
#define PARALLEL_MIN_ROWS 96 /* llambda.lisp:37 *gemv-min-parallel-rows* */

static __thread char g_error[512];

const char* oracle_last_error(void) { return g_error; }

static int fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof g_error, fmt, ap);
  va_end(ap);
  return -1;
}

/* ------------------------------------------------------------------ */
/* Type table, llambda.lisp:2126-2155                                  */

int64_t oracle_type_block_elements(int type) {
  switch (type) {
    case ORACLE_TYPE_F32: return 1;
    case ORACLE_TYPE_Q5_0:
    case ORACLE_TYPE_Q8_0: return 32;
    case ORACLE_TYPE_Q4_K:
    case ORACLE_TYPE_Q6_K: return QK_K;
    default: return -1;
  }
}

int64_t oracle_type_block_bytes(int type) {
  switch (type) {
    case ORACLE_TYPE_F32: return 4;
    case ORACLE_TYPE_Q5_0: return Q5_0_BYTES;
    case ORACLE_TYPE_Q8_0: return Q8_0_BYTES;
    case ORACLE_TYPE_Q4_K: return Q4_K_BYTES;
    case ORACLE_TYPE_Q6_K: return Q6_K_BYTES;
    default: return -1;
  }
}

/* ggml-tensor-byte-size: errors when the count is not a block multiple. */
int64_t oracle_row_bytes(int type, int64_t columns) {
  int64_t be = oracle_type_block_elements(type);
  if (be <= 0) { fail("Unsupported GGML tensor type tag %d.", type); return -1; }
  if (columns % be != 0) {
    fail("Tensor element count %lld is not a multiple of block size %lld for type %d.",
         (long long)columns, (long long)be, type);
    return -1;
  }
  return columns / be * oracle_type_block_bytes(type);
}

/* ------------------------------------------------------------------ */
/* Byte readers, llambda.lisp:676-760                                  */

static inline uint16_t rd_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t rd_u32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static inline int rd_s8(const uint8_t* p) { return (int)(int8_t)p[0]; }

/* fp16-to-single-float, llambda.lisp:716-733.  The value is built in double
 * (exact for every half) and rounded once to single; exponent 31 (Inf/NaN)
 * is an error, as in the reference. */
int oracle_fp16_to_f32(uint16_t bits, float* out) {
  float sign = (bits & 0x8000) ? -1.0f : 1.0f;
  int exponent = (bits >> 10) & 31;
  int fraction = bits & 1023;
  if (exponent == 0) {
    if (fraction == 0) {
      *out = sign * 0.0f;
    } else {
      *out = (float)((double)sign * ldexp(fraction / 1024.0, -14));
    }
    return 0;
  }
  if (exponent == 31) return fail("Unsupported fp16 special value: %x.", bits);
  *out = (float)((double)sign * ldexp(1.0 + fraction / 1024.0, exponent - 15));
  return 0;
}

static inline int read_fp16(const uint8_t* p, float* out) { return oracle_fp16_to_f32(rd_u16(p), out); }

/* get-scale-min-k4, llambda.lisp:6794-6813; twin get-scale-min-k4-at,
 * llambda.lisp:4316-4336. */
void oracle_get_scale_min_k4(const uint8_t* s, int index, int* scale, int* min) {
  int byte0 = s[index];
  int byte4 = s[index + 4];
  if (index < 4) {
    *scale = byte0 & 63;
    *min = byte4 & 63;
  } else {
    *scale = (byte4 & 0x0F) | (((s[index - 4] & 0xC0) >> 6) << 4);
    *min = (byte4 >> 4) | (((s[index] & 0xC0) >> 6) << 4);
  }
}

/* ------------------------------------------------------------------ */
/* Scalar dequantisers                                                 */

/* dequantize-q4-k-m, llambda.lisp:6815-6859 */
static int dequant_q4_k(const uint8_t* src, int64_t n, float* dst) {
  if (n % QK_K) return fail("Q4_K_M dequantization requires ELEMENT-COUNT to be a multiple of 256.");
  for (int64_t b = 0; b < n / QK_K; ++b) {
    const uint8_t* blk = src + b * Q4_K_BYTES;
    float d, dmin;
    if (read_fp16(blk, &d) || read_fp16(blk + 2, &dmin)) return -1;
    const uint8_t* scales = blk + 4;
    const uint8_t* qs = blk + 4 + K_SCALE_SIZE;
    float* out = dst + b * QK_K;
    int scale_index = 0;
    for (int chunk = 0; chunk < QK_K / 64; ++chunk) {
      int sc0, m0, sc1, m1;
      oracle_get_scale_min_k4(scales, scale_index, &sc0, &m0);
      oracle_get_scale_min_k4(scales, scale_index + 1, &sc1, &m1);
      float delta0 = d * (float)sc0, offset0 = dmin * (float)m0;
      float delta1 = d * (float)sc1, offset1 = dmin * (float)m1;
      for (int lane = 0; lane < 32; ++lane) {
        int packed = qs[chunk * 32 + lane];
        out[chunk * 64 + lane] = delta0 * (float)(packed & 0x0F) - offset0;
        out[chunk * 64 + 32 + lane] = delta1 * (float)(packed >> 4) - offset1;
      }
      scale_index += 2;
    }
  }
  return 0;
}

/* dequantize-q6-k, llambda.lisp:6919-6978: (* d scale q) = fl(fl(d*scale)*q) */
static int dequant_q6_k(const uint8_t* src, int64_t n, float* dst) {
  if (n % QK_K) return fail("Q6_K dequantization requires ELEMENT-COUNT to be a multiple of 256.");
  for (int64_t b = 0; b < n / QK_K; ++b) {
    const uint8_t* blk = src + b * Q6_K_BYTES;
    float d;
    if (read_fp16(blk + Q6_K_BYTES - 2, &d)) return -1;
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + QK_K / 2;
    const uint8_t* sc = blk + QK_K / 2 + QK_K / 4;
    float* out = dst + b * QK_K;
    for (int chunk = 0; chunk < 2; ++chunk) {
      const uint8_t* cql = ql + chunk * 64;
      const uint8_t* cqh = qh + chunk * 32;
      const uint8_t* csc = sc + chunk * 8;
      for (int lane = 0; lane < 32; ++lane) {
        int si = lane / 16;
        int lo = cql[lane], hi = cql[32 + lane], top = cqh[lane];
        int q1 = ((lo & 0x0F) | ((top & 3) << 4)) - 32;
        int q2 = ((hi & 0x0F) | (((top >> 2) & 3) << 4)) - 32;
        int q3 = ((lo >> 4) | (((top >> 4) & 3) << 4)) - 32;
        int q4 = ((hi >> 4) | (((top >> 6) & 3) << 4)) - 32;
        out[chunk * 128 + lane] = (d * (float)rd_s8(csc + si + 0)) * (float)q1;
        out[chunk * 128 + 32 + lane] = (d * (float)rd_s8(csc + si + 2)) * (float)q2;
        out[chunk * 128 + 64 + lane] = (d * (float)rd_s8(csc + si + 4)) * (float)q3;
        out[chunk * 128 + 96 + lane] = (d * (float)rd_s8(csc + si + 6)) * (float)q4;
      }
    }
  }
  return 0;
}

/* dequantize-q5-0, llambda.lisp:3965-3990 */
static int dequant_q5_0(const uint8_t* src, int64_t n, float* dst) {
  if (n % 32) return fail("Q5_0 dequantization requires ELEMENT-COUNT to be a multiple of 32.");
  for (int64_t b = 0; b < n / 32; ++b) {
    const uint8_t* blk = src + b * Q5_0_BYTES;
    float d;
    if (read_fp16(blk, &d)) return -1;
    uint32_t qh = rd_u32(blk + 2);
    const uint8_t* qs = blk + 6;
    for (int i = 0; i < 16; ++i) {
      int packed = qs[i];
      int xh0 = ((qh >> i) & 1) ? 0x10 : 0;
      int xh1 = ((qh >> (i + 16)) & 1) ? 0x10 : 0;
      int q0 = ((packed & 0x0F) | xh0) - 16;
      int q1 = ((packed >> 4) | xh1) - 16;
      dst[b * 32 + i] = d * (float)q0;
      dst[b * 32 + 16 + i] = d * (float)q1;
    }
  }
  return 0;
}

/* dequantize-q8-0, llambda.lisp:3992-4009 */
static int dequant_q8_0(const uint8_t* src, int64_t n, float* dst) {
  if (n % 32) return fail("Q8_0 dequantization requires ELEMENT-COUNT to be a multiple of 32.");
  for (int64_t b = 0; b < n / 32; ++b) {
    const uint8_t* blk = src + b * Q8_0_BYTES;
    float d;
    if (read_fp16(blk, &d)) return -1;
    for (int i = 0; i < 32; ++i) dst[b * 32 + i] = d * (float)rd_s8(blk + 2 + i);
  }
  return 0;
}

int oracle_dequantize(int type, const uint8_t* src, int64_t n, float* dst) {
  switch (type) {
    case ORACLE_TYPE_F32: memcpy(dst, src, (size_t)n * 4); return 0;
    case ORACLE_TYPE_Q4_K: return dequant_q4_k(src, n, dst);
    case ORACLE_TYPE_Q6_K: return dequant_q6_k(src, n, dst);
    case ORACLE_TYPE_Q5_0: return dequant_q5_0(src, n, dst);
    case ORACLE_TYPE_Q8_0: return dequant_q8_0(src, n, dst);
    default: return fail("Unsupported GGML tensor type tag %d.", type);
  }
}

/* ------------------------------------------------------------------ */
/* Fused row dots                                                      */

/* f32.8-horizontal+: sb-simd's lane order is unpublished; lanes are summed
 * 0..7 left to right here (parity unpinned for this order only). */
static inline float horizontal_sum8(const float a[8]) {
  float s = a[0];
  for (int t = 1; t < 8; ++t) s = s + a[t];
  return s;
}

/* dot-product-with-q4-k-m-tensor-data, llambda.lisp:4338-4382, with the
 * group body of expand-q4-k-body, llambda.lisp:4145-4201. */
static int dot_q4_k(const uint8_t* row, const float* x, int64_t n, float* out) {
  if (n % QK_K) return fail("Q4_K_M dot product requires ELEMENT-COUNT to be a multiple of 256.");
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t b = 0; b < n / QK_K; ++b) {
    const uint8_t* blk = row + b * Q4_K_BYTES;
    float d, dmin;
    if (read_fp16(blk, &d) || read_fp16(blk + 2, &dmin)) return -1;
    const uint8_t* scales = blk + 4;
    const uint8_t* qs = blk + 4 + K_SCALE_SIZE;
    const float* vb = x + b * QK_K;
    for (int j = 0; j < 4; ++j) { /* accumulate-body (2j 2j+1 32j 64j) */
      int sc0, m0, sc1, m1;
      oracle_get_scale_min_k4(scales, 2 * j, &sc0, &m0);
      oracle_get_scale_min_k4(scales, 2 * j + 1, &sc1, &m1);
      float delta0 = d * (float)sc0, offset0 = dmin * (float)m0;
      float delta1 = d * (float)sc1, offset1 = dmin * (float)m1;
      const uint8_t* q = qs + 32 * j;
      const float* v = vb + 64 * j;
      for (int g = 0; g < 4; ++g) {
        for (int t = 0; t < 8; ++t) {
          int packed = q[8 * g + t];
          float wlo = (float)(packed & 0x0F) * delta0 - offset0;
          float whi = (float)(packed >> 4) * delta1 - offset1;
          acc[t] = fmaf(wlo, v[8 * g + t], acc[t]);
          acc[t] = fmaf(whi, v[32 + 8 * g + t], acc[t]);
        }
      }
    }
  }
  *out = horizontal_sum8(acc);
  return 0;
}

/* dot-product-with-q6-k-tensor-data, llambda.lisp:4446-4506, with the group
 * body of expand-q6-k-group, llambda.lisp:4203-4310. */
static int dot_q6_k(const uint8_t* row, const float* x, int64_t n, float* out) {
  if (n % QK_K) return fail("Q6_K dot product requires ELEMENT-COUNT to be a multiple of 256.");
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t b = 0; b < n / QK_K; ++b) {
    const uint8_t* blk = row + b * Q6_K_BYTES;
    float d;
    if (read_fp16(blk + Q6_K_BYTES - 2, &d)) return -1;
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + QK_K / 2;
    const uint8_t* sc = blk + QK_K / 2 + QK_K / 4;
    const float* vb = x + b * QK_K;
    for (int h = 0; h < 2; ++h) {
      const uint8_t* cql = ql + 64 * h;
      const uint8_t* cqh = qh + 32 * h;
      const uint8_t* csc = sc + 8 * h;
      const float* cv = vb + 128 * h;
      for (int pass = 0; pass < 2; ++pass) { /* start-lane 0 then 16 */
        float delta[4];
        for (int k = 0; k < 4; ++k) delta[k] = d * (float)rd_s8(csc + 2 * k + pass);
        for (int g = 0; g < 2; ++g) {
          for (int t = 0; t < 8; ++t) {
            int L = 16 * pass + 8 * g + t;
            int lo = cql[L], hi = cql[32 + L], top = cqh[L];
            int q1 = ((lo & 0x0F) | ((top & 3) << 4)) - 32;
            int q2 = ((hi & 0x0F) | (((top >> 2) & 3) << 4)) - 32;
            int q3 = ((lo >> 4) | (((top >> 4) & 3) << 4)) - 32;
            int q4 = ((hi >> 4) | (((top >> 6) & 3) << 4)) - 32;
            float w1 = (float)q1 * delta[0];
            float w2 = (float)q2 * delta[1];
            float w3 = (float)q3 * delta[2];
            float w4 = (float)q4 * delta[3];
            acc[t] = fmaf(w1, cv[L], acc[t]);
            acc[t] = fmaf(w2, cv[32 + L], acc[t]);
            acc[t] = fmaf(w3, cv[64 + L], acc[t]);
            acc[t] = fmaf(w4, cv[96 + L], acc[t]);
          }
        }
      }
    }
  }
  *out = horizontal_sum8(acc);
  return 0;
}

/* dot-product-with-q5-0-tensor-data, llambda.lisp:4037-4066:
 * sum += d * (q0*v0 + q1*v1), every operation rounded. */
static int dot_q5_0(const uint8_t* row, const float* x, int64_t n, float* out) {
  if (n % 32) return fail("Q5_0 dot product requires ELEMENT-COUNT to be a multiple of 32.");
  float sum = 0.0f;
  for (int64_t b = 0; b < n / 32; ++b) {
    const uint8_t* blk = row + b * Q5_0_BYTES;
    float d;
    if (read_fp16(blk, &d)) return -1;
    uint32_t qh = rd_u32(blk + 2);
    const uint8_t* qs = blk + 6;
    const float* v = x + b * 32;
    for (int i = 0; i < 16; ++i) {
      int packed = qs[i];
      int xh0 = ((qh >> i) & 1) ? 0x10 : 0;
      int xh1 = ((qh >> (i + 16)) & 1) ? 0x10 : 0;
      int q0 = ((packed & 0x0F) | xh0) - 16;
      int q1 = ((packed >> 4) | xh1) - 16;
      float pair = (float)q0 * v[i] + (float)q1 * v[16 + i];
      sum = sum + d * pair;
    }
  }
  *out = sum;
  return 0;
}

/* dot-product-with-q8-0-tensor-data, llambda.lisp:4068-4094:
 * sum += (d * q) * v. */
static int dot_q8_0(const uint8_t* row, const float* x, int64_t n, float* out) {
  if (n % 32) return fail("Q8_0 dot product requires ELEMENT-COUNT to be a multiple of 32.");
  float sum = 0.0f;
  for (int64_t b = 0; b < n / 32; ++b) {
    const uint8_t* blk = row + b * Q8_0_BYTES;
    float d;
    if (read_fp16(blk, &d)) return -1;
    const float* v = x + b * 32;
    for (int i = 0; i < 32; ++i) sum = sum + (d * (float)rd_s8(blk + 2 + i)) * v[i];
  }
  *out = sum;
  return 0;
}

/* dot-product-with-f32-tensor-data, llambda.lisp:4096-4107 */
static float dot_f32(const float* w, const float* x, int64_t n) {
  float sum = 0.0f;
  for (int64_t i = 0; i < n; ++i) sum = sum + x[i] * w[i];
  return sum;
}

int oracle_dot_row(int type, const uint8_t* row, const float* x, int64_t n, float* out) {
  switch (type) {
    case ORACLE_TYPE_F32:
      /* rows of an F32 tensor are 4-byte aligned in GGUF */
      *out = dot_f32((const float*)(const void*)row, x, n);
      return 0;
    case ORACLE_TYPE_Q4_K: return dot_q4_k(row, x, n, out);
    case ORACLE_TYPE_Q6_K: return dot_q6_k(row, x, n, out);
    case ORACLE_TYPE_Q5_0: return dot_q5_0(row, x, n, out);
    case ORACLE_TYPE_Q8_0: return dot_q8_0(row, x, n, out);
    default: return fail("Unsupported GGML tensor type tag %d.", type);
  }
}

/* dot-product, llambda.lisp:3491-3500 */
float oracle_dot_product(const float* left, const float* right, int64_t n) {
  float sum = 0.0f;
  for (int64_t i = 0; i < n; ++i) sum = sum + left[i] * right[i];
  return sum;
}

/* ------------------------------------------------------------------ */
/* Persistent worker pool (the lparallel kernel of llambda.lisp:769-817) */

typedef struct gemv_job {
  int type;
  const uint8_t* matrix;
  int64_t row_bytes, columns, rows, parts;
  const float* x;
  float* y;
  int status;              /* first failing part's status */
  char error[512];
  pthread_mutex_t error_lock;
} gemv_job;

typedef struct pool {
  pthread_mutex_t lock;
  pthread_cond_t start, done;
  pthread_t* threads;
  int size;                /* worker threads (the caller is one more part) */
  int ready;               /* workers that have registered their generation */
  unsigned long generation;
  int pending;             /* workers still inside the current job */
  int next_part;
  gemv_job* job;
} pool;

static pool g_pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER,
                      PTHREAD_COND_INITIALIZER, NULL, 0, 0, 0, 0, 0, NULL};
static pthread_mutex_t g_pool_use = PTHREAD_MUTEX_INITIALIZER;

/* lparallel:pdotimes over `parts` contiguous chunks of [0, rows). */
static void run_part(gemv_job* job, int64_t part) {
  int64_t base = job->rows / job->parts, extra = job->rows % job->parts;
  int64_t start = part * base + (part < extra ? part : extra);
  int64_t count = base + (part < extra ? 1 : 0);
  for (int64_t r = start; r < start + count; ++r) {
    float v;
    if (oracle_dot_row(job->type, job->matrix + r * job->row_bytes, job->x, job->columns, &v)) {
      pthread_mutex_lock(&job->error_lock);
      if (job->status == 0) {
        job->status = -1;
        snprintf(job->error, sizeof job->error, "%s", g_error);
      }
      pthread_mutex_unlock(&job->error_lock);
      return;
    }
    job->y[r] = v;
  }
}

static void drain_parts(pool* p, gemv_job* job) {
  for (;;) {
    pthread_mutex_lock(&p->lock);
    int part = p->next_part < job->parts ? p->next_part++ : -1;
    pthread_mutex_unlock(&p->lock);
    if (part < 0) return;
    run_part(job, part);
  }
}

static void* worker_main(void* arg) {
  pool* p = (pool*)arg;
  /* a new worker joins at the current generation, so it never runs a job
   * dispatched before it existed */
  pthread_mutex_lock(&p->lock);
  unsigned long seen = p->generation;
  p->ready++;
  pthread_cond_broadcast(&p->done);
  pthread_mutex_unlock(&p->lock);
  for (;;) {
    pthread_mutex_lock(&p->lock);
    while (p->generation == seen) pthread_cond_wait(&p->start, &p->lock);
    seen = p->generation;
    gemv_job* job = p->job;
    pthread_mutex_unlock(&p->lock);
    drain_parts(p, job);
    pthread_mutex_lock(&p->lock);
    if (--p->pending == 0) pthread_cond_signal(&p->done);
    pthread_mutex_unlock(&p->lock);
  }
  return NULL;
}

/* ensure-gemv-kernel, llambda.lisp:774-792: grow the pool to threads-1
 * workers (the caller works too). */
static void ensure_pool(int threads) {
  int want = threads - 1;
  if (g_pool.size >= want) return;
  g_pool.threads = (pthread_t*)realloc(g_pool.threads, sizeof(pthread_t) * (size_t)want);
  for (int i = g_pool.size; i < want; ++i) {
    pthread_create(&g_pool.threads[i], NULL, worker_main, &g_pool);
    pthread_detach(g_pool.threads[i]);
  }
  g_pool.size = want;
  pthread_mutex_lock(&g_pool.lock);
  while (g_pool.ready < g_pool.size) pthread_cond_wait(&g_pool.done, &g_pool.lock);
  pthread_mutex_unlock(&g_pool.lock);
}

int oracle_gemv(int type, const uint8_t* matrix, int64_t rows, int64_t columns,
                const float* x, float* y, int threads) {
  int64_t row_bytes = oracle_row_bytes(type, columns);
  if (row_bytes < 0) return -1;
  if (threads <= 0) threads = 1;
  int parallel = (type == ORACLE_TYPE_Q4_K || type == ORACLE_TYPE_Q6_K) &&
                 rows >= PARALLEL_MIN_ROWS && threads > 1;
  gemv_job job;
  memset(&job, 0, sizeof job);
  job.type = type; job.matrix = matrix; job.row_bytes = row_bytes;
  job.columns = columns; job.rows = rows; job.x = x; job.y = y;
  pthread_mutex_init(&job.error_lock, NULL);
  if (!parallel) {
    job.parts = 1;
    run_part(&job, 0);
  } else {
    job.parts = rows < threads ? rows : threads; /* parallel-gemv-part-count */
    pthread_mutex_lock(&g_pool_use);
    ensure_pool(threads);
    pthread_mutex_lock(&g_pool.lock);
    g_pool.job = &job;
    g_pool.next_part = 0;
    g_pool.pending = g_pool.size; /* every worker acknowledges every job */
    g_pool.generation++;
    pthread_cond_broadcast(&g_pool.start);
    pthread_mutex_unlock(&g_pool.lock);
    drain_parts(&g_pool, &job);
    pthread_mutex_lock(&g_pool.lock);
    while (g_pool.pending > 0) pthread_cond_wait(&g_pool.done, &g_pool.lock);
    pthread_mutex_unlock(&g_pool.lock);
    pthread_mutex_unlock(&g_pool_use);
  }
  pthread_mutex_destroy(&job.error_lock);
  if (job.status) {
    if (parallel) snprintf(g_error, sizeof g_error, "%s", job.error);
    return -1;
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* Routing and activations                                             */

/* select-top-k-logits-into, llambda.lisp:5265-5292: sorted insertion with
 * strict >, slots start at (-1, most-negative-single-float). */
void oracle_select_top_k(const float* logits, int64_t n, int64_t k,
                         int64_t* idx, float* val) {
  for (int64_t i = 0; i < k; ++i) { idx[i] = -1; val[i] = -FLT_MAX; }
  if (k <= 0) return;
  for (int64_t li = 0; li < n; ++li) {
    float v = logits[li];
    if (v > val[k - 1]) {
      int64_t ins = k - 1;
      while (ins > 0 && v > val[ins - 1]) {
        val[ins] = val[ins - 1];
        idx[ins] = idx[ins - 1];
        --ins;
      }
      val[ins] = v;
      idx[ins] = li;
    }
  }
}

/* sigmoid, llambda.lisp:929-930: (exp (- x)) of a single-float is a single
 * (computed in double and rounded); 1 + e and the quotient are double; the
 * result is rounded to single.  SBCL traps the rounding overflow that
 * exp(-x) > FLT_MAX would cause (x < -88.72); this restatement yields the
 * IEEE limit (0) there instead. */
float oracle_sigmoid(float x) {
  float e = (float)exp((double)(-x));
  return (float)(1.0 / (1.0 + (double)e));
}

/* silu, llambda.lisp:926-927 */
float oracle_silu(float x) {
  float e = (float)exp((double)(-x));
  return (float)((double)x / (1.0 + (double)e));
}

/* relu-squared, llambda.lisp:938-940 */
float oracle_relu_squared(float x) {
  float r = x > 0.0f ? x : 0.0f;
  return r * r;
}

/* ------------------------------------------------------------------ */
/* Routed MoE layers                                                   */

static int expert_gemv(int type, const uint8_t* slab, int64_t expert, int64_t rows,
                       int64_t columns, const float* x, float* y, int threads) {
  /* gguf-model-expert-matrix-vector-multiply-into, llambda.lisp:4951-4971:
   * expert e's rows are [e*rows, (e+1)*rows) of the flat matrix. */
  int64_t row_bytes = oracle_row_bytes(type, columns);
  if (row_bytes < 0) return -1;
  return oracle_gemv(type, slab + expert * rows * row_bytes, rows, columns, x, y, threads);
}

/* qwen3next-moe-into, llambda.lisp:5321-5426, for one token. */
static int qwen3next_token(const oracle_moe_desc* m, const float* x, float* dest,
                           int64_t* top_idx, float* top_w, float* logits, float* work,
                           int threads) {
  const int64_t H = m->hidden, E = m->expert_count, K = m->top_k, F = m->expert_ffn,
                Fs = m->shared_ffn;
  float* top_logits = work;                 /* [K] */
  float* gate = top_logits + K;             /* [max(F, Fs)] */
  int64_t FF = F > Fs ? F : Fs;
  float* up = gate + FF;
  float* down = up + FF;                    /* [H] */
  for (int64_t i = 0; i < H; ++i) dest[i] = 0.0f;                       /* :5359 */
  if (oracle_gemv(ORACLE_TYPE_F32, (const uint8_t*)m->router, E, H, x, logits, threads))
    return -1;                                                          /* :5360-5363 */
  oracle_select_top_k(logits, E, K, top_idx, top_logits);              /* :5364 */
  float weight_sum = 0.0f;                                              /* :5365-5379 */
  for (int64_t r = 0; r < K; ++r) {
    float w = oracle_sigmoid(top_logits[r]);
    top_w[r] = w;
    weight_sum = weight_sum + w;
  }
  if (!(weight_sum > 0.0f))
    return fail("Qwen3Next layer router produced non-positive top-k weight sum.");
  for (int64_t r = 0; r < K; ++r) top_w[r] = top_w[r] / weight_sum;
  for (int64_t r = 0; r < K; ++r) {                                     /* :5380-5409 */
    int64_t e = top_idx[r];
    if (e < 0 || e >= E) return fail("Expert index %lld is out of range.", (long long)e);
    if (expert_gemv(m->gate_type, m->gate_exps, e, F, H, x, gate, threads)) return -1;
    if (expert_gemv(m->up_type, m->up_exps, e, F, H, x, up, threads)) return -1;
    for (int64_t i = 0; i < F; ++i) gate[i] = oracle_silu(gate[i]);
    for (int64_t i = 0; i < F; ++i) gate[i] = gate[i] * up[i];
    if (expert_gemv(m->down_type, m->down_exps, e, H, F, gate, down, threads)) return -1;
    for (int64_t i = 0; i < H; ++i) dest[i] = dest[i] + top_w[r] * down[i];
  }
  if (Fs > 0) {                                                         /* :5410-5426 */
    float shared_weight = oracle_sigmoid(oracle_dot_product(m->shared_gate_inp, x, H));
    if (oracle_gemv(m->shared_gate_type, m->shared_gate, Fs, H, x, gate, threads)) return -1;
    if (oracle_gemv(m->shared_up_type, m->shared_up, Fs, H, x, up, threads)) return -1;
    for (int64_t i = 0; i < Fs; ++i) gate[i] = oracle_silu(gate[i]);
    for (int64_t i = 0; i < Fs; ++i) gate[i] = gate[i] * up[i];
    if (oracle_gemv(m->shared_down_type, m->shared_down, H, Fs, gate, down, threads)) return -1;
    for (int64_t i = 0; i < H; ++i) dest[i] = dest[i] + shared_weight * down[i];
  }
  return 0;
}

/* nemotron-h-moe-ffn-into, llambda.lisp:5827-5949, for one token.  The
 * optional latent projections are independent, as in the reference: with
 * ffn_latent_down the experts' input is ffn_latent_down * x (:5883-5887),
 * Li wide; with ffn_latent_up their weighted sum is Lo wide and
 * ffn_latent_up maps it back to H (:5933-5938); without it the sum is
 * formed in dest.  The router and the shared expert read x itself. */
static int nemotron_token(const oracle_moe_desc* m, const float* x, float* dest,
                          int64_t* top_idx, float* top_w, float* logits, float* work,
                          int threads) {
  const int64_t H = m->hidden, E = m->expert_count, K = m->top_k, F = m->expert_ffn,
                Fs = m->shared_ffn;
  const int64_t Li = m->latent_in, Lo = m->latent_out;
  const int64_t Din = Li > 0 ? Li : H;      /* width of the experts' input */
  const int64_t Dout = Lo > 0 ? Lo : H;     /* width of their outputs */
  const int64_t FF = F > Fs ? F : Fs;
  float* top_logits = work;                 /* [K] */
  float* up = top_logits + K;               /* [FF] */
  float* down = up + FF;                    /* [max(H, Lo)] */
  float* expert_in = down + (H > Lo ? H : Lo); /* [Li] */
  float* moe_out = expert_in + Li;          /* [Lo] */
  const float* ein = x;
  float* acc = Lo > 0 ? moe_out : dest;
  if (Li > 0) {                                                         /* :5883-5887 */
    if (oracle_gemv(m->latent_down_type, m->latent_down, Li, H, x, expert_in, threads))
      return -1;
    ein = expert_in;
  }
  if (oracle_gemv(ORACLE_TYPE_F32, (const uint8_t*)m->router, E, H, x, logits, threads))
    return -1;                                                          /* :5888-5891 */
  for (int64_t e = 0; e < E; ++e) logits[e] = logits[e] + m->router_bias[e]; /* :5892 */
  oracle_select_top_k(logits, E, K, top_idx, top_logits);              /* :5893 */
  float weight_sum = 0.0f;                                              /* :5894-5913 */
  for (int64_t r = 0; r < K; ++r) {
    float w = oracle_sigmoid(top_logits[r]);
    top_w[r] = w;
    weight_sum = weight_sum + w;
  }
  if (m->expert_weights_norm) {
    if (!(weight_sum > 0.0f))
      return fail("Nemotron-H MoE layer router produced non-positive top-k weight sum.");
    for (int64_t r = 0; r < K; ++r) top_w[r] = top_w[r] / weight_sum;
  }
  for (int64_t r = 0; r < K; ++r) top_w[r] = m->expert_weights_scale * top_w[r];
  for (int64_t i = 0; i < Dout; ++i) acc[i] = 0.0f;                    /* :5914 */
  for (int64_t r = 0; r < K; ++r) {                                     /* :5915-5932 */
    int64_t e = top_idx[r];
    if (e < 0 || e >= E) return fail("Expert index %lld is out of range.", (long long)e);
    if (expert_gemv(m->up_type, m->up_exps, e, F, Din, ein, up, threads)) return -1;
    for (int64_t i = 0; i < F; ++i) up[i] = oracle_relu_squared(up[i]);
    if (expert_gemv(m->down_type, m->down_exps, e, Dout, F, up, down, threads)) return -1;
    for (int64_t i = 0; i < Dout; ++i) acc[i] = acc[i] + top_w[r] * down[i];
  }
  if (Lo > 0 &&                                                         /* :5933-5938 */
      oracle_gemv(m->latent_up_type, m->latent_up, H, Lo, moe_out, dest, threads))
    return -1;
  if (Fs > 0) {                                                         /* :5939-5949 */
    if (oracle_gemv(m->shared_up_type, m->shared_up, Fs, H, x, up, threads)) return -1;
    for (int64_t i = 0; i < Fs; ++i) up[i] = oracle_relu_squared(up[i]);
    if (oracle_gemv(m->shared_down_type, m->shared_down, H, Fs, up, down, threads)) return -1;
    for (int64_t i = 0; i < H; ++i) dest[i] = dest[i] + down[i];
  }
  return 0;
}

int oracle_moe_forward(const oracle_moe_desc* m, const float* x, float* y, int64_t tokens,
                       int64_t* top_indices, float* top_weights, float* router_logits,
                       int threads) {
  if (!m || !x || !y) return fail("null argument");
  if (m->top_k <= 0 || m->top_k > m->expert_count) return fail("top_k out of range");
  int64_t FF = m->expert_ffn > m->shared_ffn ? m->expert_ffn : m->shared_ffn;
  const int64_t Li = m->latent_in, Lo = m->latent_out;
  if (Li < 0 || Lo < 0 || (Li > 0) != (m->latent_down != NULL) ||
      (Lo > 0) != (m->latent_up != NULL))
    return fail("latent projections: a width for each tensor given, and only for those");
  if ((Li > 0 || Lo > 0) && m->variant != 1)
    return fail("latent projections belong to Nemotron-H layers");
  /* qwen3next: top logits, gate, up, down [H]; nemotron: top logits, up,
   * down [max(H, Lo)], expert input [Li], weighted sum [Lo] */
  const int64_t wide = m->hidden > Lo ? m->hidden : Lo;
  size_t work_floats = (size_t)(m->top_k + 2 * FF + wide + Li + Lo);
  float* work = (float*)malloc((work_floats + (size_t)m->expert_count) * sizeof(float));
  int64_t* idx = (int64_t*)malloc((size_t)m->top_k * sizeof(int64_t));
  float* w = (float*)malloc((size_t)m->top_k * sizeof(float));
  float* logits = work + work_floats;
  int status = 0;
  for (int64_t t = 0; t < tokens && status == 0; ++t) {
    const float* xt = x + t * m->hidden;
    float* yt = y + t * m->hidden;
    if (m->variant == 0)
      status = qwen3next_token(m, xt, yt, idx, w, logits, work, threads);
    else if (m->variant == 1)
      status = nemotron_token(m, xt, yt, idx, w, logits, work, threads);
    else
      status = fail("unknown MoE variant %d", m->variant);
    if (status == 0) {
      if (top_indices) memcpy(top_indices + t * m->top_k, idx, (size_t)m->top_k * sizeof(int64_t));
      if (top_weights) memcpy(top_weights + t * m->top_k, w, (size_t)m->top_k * sizeof(float));
      if (router_logits)
        memcpy(router_logits + t * m->expert_count, logits, (size_t)m->expert_count * sizeof(float));
    }
  }
  free(work);
  free(idx);
  free(w);
  return status;
}

/* ================================================== Llama decode token */

/* sum-square-elements (llambda.lisp:819-828) and rms-norm-into (859-879):
 * serial fp32 sum of squares, mean = sum / n, scale = 1 / sqrt(mean + eps),
 * out = (x * w) * scale. */
void oracle_rms_norm(const float* x, const float* w, int64_t n, float eps, float* out) {
  float sum = 0.0f;
  for (int64_t i = 0; i < n; ++i) sum += x[i] * x[i];
  const float mean = sum / (float)n;
  const float scale = 1.0f / sqrtf(mean + eps);
  for (int64_t i = 0; i < n; ++i) out[i] = (x[i] * w[i]) * scale;
}

/* apply-rope-head-in-place (llambda.lisp:3760-3795).  The power
 * (expt theta-base (/ (* 2 i) even)) has a single-float base and a rational
 * exponent, so Common Lisp returns a single-float: pow in double, rounded.
 * The angle, cos, sin and the rotation are double; results rounded. */
void oracle_rope_head(float* head, int64_t len, int64_t position, int64_t rope_dim,
                      float theta_base, const float* factors, int64_t n_factors) {
  const int64_t factor_limit = factors ? 2 * n_factors : rope_dim;
  int64_t eff = rope_dim < factor_limit ? rope_dim : factor_limit;
  if (len < eff) eff = len;
  const int64_t even = 2 * (eff / 2), pairs = even / 2;
  for (int64_t i = 0; i < pairs; ++i) {
    const double factor = (factors && i < n_factors) ? (double)factors[i] : 1.0;
    double angle = 0.0;
    if (!(factor > 1.0e20)) {
      const float power = (float)pow((double)theta_base, (double)(2 * i) / (double)even);
      angle = (double)position / (factor * (double)power);
    }
    const double c = cos(angle), s = sin(angle);
    const float x0 = head[2 * i], x1 = head[2 * i + 1];
    head[2 * i] = (float)((double)x0 * c - (double)x1 * s);
    head[2 * i + 1] = (float)((double)x0 * s + (double)x1 * c);
  }
}

/* softmax-into (llambda.lisp:5075-5096) with max-single-float-element
 * (841-857): exp of the single-float difference (computed in double,
 * rounded), serial sum, each value divided by the sum. */
void oracle_softmax(const float* logits, int64_t n, float* out) {
  float mx = logits[0];
  for (int64_t i = 1; i < n; ++i)
    if (logits[i] > mx) mx = logits[i];
  float sum = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    const float v = (float)exp((double)(logits[i] - mx));
    out[i] = v;
    sum += v;
  }
  for (int64_t i = 0; i < n; ++i) out[i] = out[i] / sum;
}

/* compute-gemma4-attention-into as the llama step uses it
 * (llambda.lisp:5122-5167): query head h reads kv head h / (heads / kv);
 * scores by dot-product (3491-3500) over slots 0..n-1, softmax-into, then
 * weighted-sum-head-into (5097-5115), slot by slot.  q: [heads][D],
 * caches: [kv][cap][D], out: [heads][D]. */
int oracle_attention(const float* q, const float* kc, const float* vc, int64_t cap, int64_t n,
                     int64_t heads, int64_t kv_heads, int64_t D, float* out) {
  if (n <= 0 || n > cap) return fail("attention: %lld slots outside the cache", (long long)n);
  if (kv_heads <= 0 || heads % kv_heads) return fail("attention: bad head counts");
  float* scores = (float*)malloc((size_t)n * 2 * sizeof(float));
  if (!scores) return fail("attention: out of memory");
  float* probs = scores + n;
  const int64_t group = heads / kv_heads;
  for (int64_t h = 0; h < heads; ++h) {
    const int64_t kvh = h / group;
    const float* qh = q + h * D;
    for (int64_t s = 0; s < n; ++s)
      scores[s] = oracle_dot_product(qh, kc + (kvh * cap + s) * D, D);
    oracle_softmax(scores, n, probs);
    float* dst = out + h * D;
    for (int64_t e = 0; e < D; ++e) dst[e] = 0.0f;
    for (int64_t s = 0; s < n; ++s) {
      const float* vh = vc + (kvh * cap + s) * D;
      for (int64_t e = 0; e < D; ++e) dst[e] += probs[s] * vh[e];
    }
  }
  free(scores);
  return 0;
}

/* One step of make-llama-step-function (llambda.lisp:6294-6441) for token
 * `token` at `position`: the embedding row (gguf-model-token-row-into,
 * 4977-4982, via the dequantisers), per layer rms-norm, q/k/v projections,
 * rotation of every q and k head, q scaled by 1/sqrt(head size), k and v
 * appended (here: written to cache slot `position`), attention over slots
 * 0..position, x += o(context), rms-norm, silu(gate) * up, x += down(h);
 * then rms-norm with output_norm and the output rows.
 * kv: [layers][2][kv_heads][cap][head_dim]. */
int oracle_llama_step(const oracle_llama_desc* m, float* kv, int64_t cap, int64_t token,
                      int64_t position, float* logits, int threads) {
  return oracle_llama_step_hidden(m, kv, cap, token, position, logits, NULL, threads);
}

/* The same step; `hidden` (optional, [hidden]) receives the output rows'
 * input, rms-norm(x) * output_norm, for per-row bounds of the logits. */
int oracle_llama_step_hidden(const oracle_llama_desc* m, float* kv, int64_t cap, int64_t token,
                             int64_t position, float* logits, float* hidden, int threads) {
  if (!m || !kv || !logits) return fail("llama step: null argument");
  const int64_t H = m->hidden, NH = m->heads, NKV = m->kv_heads, F = m->ffn;
  if (H <= 0 || NH <= 0 || NKV <= 0 || H % NH || NH % NKV) return fail("llama step: bad dims");
  if (token < 0 || token >= m->vocab) return fail("llama step: token out of range");
  if (position < 0 || position >= cap) return fail("llama step: position outside the cache");
  const int64_t D = H / NH;
  const float scale = 1.0f / sqrtf((float)D);
  const size_t nbuf = (size_t)(5 * H + 2 * NKV * D + 2 * F + NH * D);
  float* buf = (float*)malloc(nbuf * sizeof(float));
  if (!buf) return fail("llama step: out of memory");
  float *x = buf, *xin = x + H, *q = xin + H, *k = q + NH * D, *v = k + NKV * D;
  float *ctx = v + NKV * D, *ao = ctx + NH * D, *g = ao + H, *u = g + F;
  int status = 0;
  const int64_t erb = oracle_row_bytes(m->token_embd.type, H);
  if (erb < 0 || oracle_dequantize(m->token_embd.type, m->token_embd.data + token * erb, H, x))
    status = fail("llama step: token row: %s", g_error);
  for (int64_t l = 0; l < m->layer_count && status == 0; ++l) {
    const oracle_llama_layer* L = m->layers + l;
    float* kc = kv + (size_t)(2 * l) * NKV * cap * D;
    float* vc = kc + (size_t)NKV * cap * D;
    oracle_rms_norm(x, L->attn_norm, H, m->norm_eps, xin);
    if (oracle_gemv(L->attn_q.type, L->attn_q.data, NH * D, H, xin, q, threads) ||
        oracle_gemv(L->attn_k.type, L->attn_k.data, NKV * D, H, xin, k, threads) ||
        oracle_gemv(L->attn_v.type, L->attn_v.data, NKV * D, H, xin, v, threads)) {
      status = -1;
      break;
    }
    for (int64_t h = 0; h < NH; ++h)
      oracle_rope_head(q + h * D, D, position, m->rope_dim, m->rope_base, m->rope_factors,
                       m->rope_factor_count);
    for (int64_t h = 0; h < NKV; ++h)
      oracle_rope_head(k + h * D, D, position, m->rope_dim, m->rope_base, m->rope_factors,
                       m->rope_factor_count);
    for (int64_t i = 0; i < NH * D; ++i) q[i] = q[i] * scale;
    for (int64_t h = 0; h < NKV; ++h) {
      memcpy(kc + (h * cap + position) * D, k + h * D, (size_t)D * sizeof(float));
      memcpy(vc + (h * cap + position) * D, v + h * D, (size_t)D * sizeof(float));
    }
    if (oracle_attention(q, kc, vc, cap, position + 1, NH, NKV, D, ctx)) {
      status = -1;
      break;
    }
    if (oracle_gemv(L->attn_output.type, L->attn_output.data, H, NH * D, ctx, ao, threads)) {
      status = -1;
      break;
    }
    for (int64_t i = 0; i < H; ++i) x[i] = x[i] + ao[i];
    oracle_rms_norm(x, L->ffn_norm, H, m->norm_eps, xin);
    if (oracle_gemv(L->ffn_gate.type, L->ffn_gate.data, F, H, xin, g, threads) ||
        oracle_gemv(L->ffn_up.type, L->ffn_up.data, F, H, xin, u, threads)) {
      status = -1;
      break;
    }
    for (int64_t i = 0; i < F; ++i) g[i] = oracle_silu(g[i]);
    for (int64_t i = 0; i < F; ++i) g[i] = g[i] * u[i];
    if (oracle_gemv(L->ffn_down.type, L->ffn_down.data, H, F, g, ao, threads)) {
      status = -1;
      break;
    }
    for (int64_t i = 0; i < H; ++i) x[i] = x[i] + ao[i];
  }
  if (status == 0) {
    oracle_rms_norm(x, m->output_norm, H, m->norm_eps, xin);
    if (hidden) memcpy(hidden, xin, (size_t)H * sizeof(float));
    if (oracle_gemv(m->output.type, m->output.data, m->vocab, H, xin, logits, threads)) status = -1;
  }
  free(buf);
  return status;
}

/* ========================================================== sampling */

#define MASKED_LOGIT (-1.0e30f) /* llambda.lisp:1098, 1172 */

/* apply-repetition-penalty (llambda.lisp:1036-1086): every distinct history
 * token once, positive logits divided by the penalty, negative multiplied. */
int oracle_repetition_penalty(float* logits, int64_t n, const int64_t* history, int64_t nh,
                              float penalty) {
  if (!(penalty > 0.0f)) return fail("PENALTY must be positive, got %g.", (double)penalty);
  for (int64_t i = 0; i < nh; ++i) {
    const int64_t t = history[i];
    int seen = 0;
    for (int64_t j = 0; j < i; ++j)
      if (history[j] == t) {
        seen = 1;
        break;
      }
    if (seen) continue;
    if (t < 0 || t >= n)
      return fail("History token id %lld is out of bounds for logits length %lld.", (long long)t,
                  (long long)n);
    const float l = logits[t];
    if (l > 0.0f) logits[t] = l / penalty;
    else if (l < 0.0f) logits[t] = l * penalty;
  }
  return 0;
}

static void heapify_down(float* heap, int64_t k, int64_t start) {
  const float value = heap[start];
  int64_t index = start;
  for (;;) {
    const int64_t left = 2 * index + 1;
    if (left >= k) break;
    const int64_t right = left + 1;
    const int64_t smaller = (right < k && heap[right] < heap[left]) ? right : left;
    if (value <= heap[smaller]) break;
    heap[index] = heap[smaller];
    index = smaller;
  }
  heap[index] = value;
}

/* apply-top-k-with-workspace (llambda.lisp:1088-1150): a min-heap of the
 * first k logits, each later logit greater than the root replaces it; every
 * logit below the final root is masked (ties with the root survive). */
int oracle_top_k(float* logits, int64_t n, int64_t k) {
  if (k < 0) return fail("TOP-K must be non-negative, got %lld.", (long long)k);
  if (k == 0 || k >= n) return 0;
  float* heap = (float*)malloc((size_t)k * sizeof(float));
  if (!heap) return fail("top-k: out of memory");
  memcpy(heap, logits, (size_t)k * sizeof(float));
  for (int64_t i = (k - 2) / 2; i >= 0; --i) heapify_down(heap, k, i);
  for (int64_t i = k; i < n; ++i)
    if (logits[i] > heap[0]) {
      heap[0] = logits[i];
      heapify_down(heap, k, 0);
    }
  const float cutoff = heap[0];
  for (int64_t i = 0; i < n; ++i)
    if (logits[i] < cutoff) logits[i] = MASKED_LOGIT;
  free(heap);
  return 0;
}

/* apply-top-p-with-workspace (llambda.lisp:1163-1240): the unmasked logits
 * in index order, insertion-sorted descending (stable), softmax of
 * logit / temperature accumulated in that order until the cumulative
 * probability reaches p; logits below the cutoff are masked. */
int oracle_top_p(float* logits, int64_t n, float p, float temperature) {
  if (!(p > 0.0f) || p > 1.0f) return fail("TOP-P must satisfy 0.0 < p <= 1.0, got %g.", (double)p);
  if (!(temperature > 0.0f))
    return fail("TEMPERATURE must be positive, got %g.", (double)temperature);
  if (p == 1.0f) return 0;
  float* val = (float*)malloc((size_t)n * sizeof(float));
  int64_t* idx = (int64_t*)malloc((size_t)n * sizeof(int64_t));
  if (!val || !idx) {
    free(val);
    free(idx);
    return fail("top-p: out of memory");
  }
  int64_t active = 0;
  for (int64_t i = 0; i < n; ++i)
    if (logits[i] > MASKED_LOGIT) {
      val[active] = logits[i];
      idx[active] = i;
      ++active;
    }
  if (active > 1) {
    for (int64_t i = 1; i < active; ++i) {
      const float v = val[i];
      const int64_t t = idx[i];
      int64_t j = i;
      while (j > 0 && !(val[j - 1] >= v)) {
        val[j] = val[j - 1];
        idx[j] = idx[j - 1];
        --j;
      }
      val[j] = v;
      idx[j] = t;
    }
    const float max_scaled = val[0] / temperature;
    float sum = 0.0f;
    for (int64_t i = 0; i < active; ++i) sum += (float)exp((double)(val[i] / temperature - max_scaled));
    float cumulative = 0.0f, cutoff = val[active - 1];
    for (int64_t i = 0; i < active; ++i) {
      cumulative += (float)exp((double)(val[i] / temperature - max_scaled)) / sum;
      if (cumulative >= p) {
        cutoff = val[i];
        break;
      }
    }
    for (int64_t i = 0; i < n; ++i)
      if (logits[i] < cutoff) logits[i] = MASKED_LOGIT;
  }
  free(val);
  free(idx);
  return 0;
}

/* sample-from-probabilities (llambda.lisp:1253-1270): the first index whose
 * running total reaches the roll, else the last index. */
int64_t oracle_sample_from_probabilities(const float* probs, int64_t n, float roll) {
  float running = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    running += probs[i];
    if (roll <= running) return i;
  }
  return n - 1;
}

/* sample-token-id-from-logits (llambda.lisp:1272-1317) with an explicit
 * random value: repetition penalty (when history is given), top-k, top-p,
 * apply-temperature (1009-1015), softmax (1017-1034), the draw.  logits are
 * modified in place as the reference modifies them. */
int oracle_sample_token(float* logits, int64_t n, const int64_t* history, int64_t nh,
                        float penalty, int64_t top_k, float top_p, float temperature, float roll,
                        int64_t* token) {
  if (n <= 0 || !token) return fail("sample: empty logits");
  if (!(roll >= 0.0f && roll < 1.0f))
    return fail("RANDOM-VALUE must satisfy 0.0 <= value < 1.0, got %g.", (double)roll);
  if (!(top_p > 0.0f) || top_p > 1.0f)
    return fail("TOP-P must satisfy 0.0 < p <= 1.0, got %g.", (double)top_p);
  if (top_k < 0) return fail("TOP-K must be a nonnegative fixnum or NIL, got %lld.", (long long)top_k);
  if (nh > 0 && oracle_repetition_penalty(logits, n, history, nh, penalty)) return -1;
  if (oracle_top_k(logits, n, top_k)) return -1;
  if (oracle_top_p(logits, n, top_p, temperature)) return -1;
  float* probs = (float*)malloc((size_t)n * sizeof(float));
  if (!probs) return fail("sample: out of memory");
  for (int64_t i = 0; i < n; ++i) probs[i] = logits[i] / temperature;
  oracle_softmax(probs, n, probs);
  *token = oracle_sample_from_probabilities(probs, n, roll);
  free(probs);
  return 0;
}
