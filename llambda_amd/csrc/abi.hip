// abi.hip -- the extern "C" boundary of libllambda_hip.so (include/llambda_hip.h).
//
// Conventions follow the reference's native bridge (native/llambda_npu.cpp):
// thread-local last error cleared on entry, status 0 / -1, exceptions caught
// at the boundary, null-safe destroy, synchronous runs on host pointers.
#include "../../include/llambda_hip.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cmath>
#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "decoder.h"
#include "gemv.h"
#include "gguf.h"
#include "moe.h"
#include "sample.h"
#include "sha256.h"

using namespace llhip;

namespace {

thread_local std::string g_last_error;

struct Failure : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// The reference's own error for this input (the MoE functions' `error`
// calls): the call fails with status -2 and the session stays usable.
struct InputError : Failure {
  using Failure::Failure;
};

[[noreturn]] void failf(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  throw Failure(buf);
}

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) failf("%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
}
#define HIPC(expr) hip_check((expr), #expr)

template <typename F>
int guarded(F&& f) {
  g_last_error.clear();
  try {
    f();
    return 0;
  } catch (const InputError& e) {
    g_last_error = e.what();
    return -2;
  } catch (const std::exception& e) {
    g_last_error = e.what();
  } catch (...) {
    g_last_error = "unknown C++ exception";
  }
  return -1;
}

bool supported_type(int t) {
  return t == kF32 || t == kQ4_K || t == kQ6_K || t == kQ5_0 || t == kQ8_0;
}

const char* type_name(int t) {
  switch (t) {
    case kF32: return "F32";
    case kQ4_K: return "Q4_K";
    case kQ6_K: return "Q6_K";
    case kQ5_0: return "Q5_0";
    case kQ8_0: return "Q8_0";
    default: return "?";
  }
}

// ggml-tensor-byte-size (llambda.lisp:2147-2155) for one row of K columns,
// plus the layout limits of the kernels (units of 32 weights).
int64_t checked_row_bytes(int type, int64_t columns, const char* what) {
  if (!supported_type(type)) failf("%s: unsupported GGML tensor type tag %d", what, type);
  const int be = block_weights(type);
  if (columns <= 0) failf("%s: column count %lld must be positive", what, (long long)columns);
  if (columns % be)
    failf("%s: Tensor element count %lld is not a multiple of block size %d for type %s.", what,
          (long long)columns, be, type_name(type));
  if (type == kF32 && columns % 4)
    failf("%s: F32 rows need a column count divisible by 4, got %lld", what, (long long)columns);
  if (columns > kMaxColumns)
    failf("%s: column count %lld exceeds the supported %lld", what, (long long)columns,
          (long long)kMaxColumns);
  return columns / be * block_bytes(type);
}

// RAII device buffer.
struct DevBuf {
  void* ptr = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() { reset(); }
  void reset() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
  }
  void alloc(size_t n, const char* what) {
    reset();
    if (n == 0) n = 16;
    hipError_t e = hipMalloc(&ptr, n);
    if (e != hipSuccess) {
      ptr = nullptr;
      failf("hipMalloc of %zu bytes for %s failed: %s", n, what, hipGetErrorString(e));
    }
    bytes = n;
  }
  template <typename T>
  T* as() const { return static_cast<T*>(ptr); }
  void swap(DevBuf& o) {
    std::swap(ptr, o.ptr);
    std::swap(bytes, o.bytes);
  }
};

// Pinned host memory staging the host-pointer runs.  A copy from or to it
// is one DMA transfer, where a pageable buffer first goes through the
// runtime's own bounce buffer (measured 26 us against 18 us for a 16 KB
// vector in and out around a trivial kernel).  A `mapped` buffer is also
// fine-grained and coherent: kernels store into it directly through `dev`,
// visible to the host once the stream has been synchronised.
struct HostBuf {
  void* ptr = nullptr;
  void* dev = nullptr;
  size_t bytes = 0;
  HostBuf() = default;
  HostBuf(const HostBuf&) = delete;
  HostBuf& operator=(const HostBuf&) = delete;
  ~HostBuf() { reset(); }
  void reset() {
    if (ptr) (void)hipHostFree(ptr);
    ptr = dev = nullptr;
    bytes = 0;
  }
  void alloc(size_t n, bool mapped, const char* what) {
    reset();
    if (n == 0) n = 16;
    const unsigned flags = mapped ? (hipHostMallocMapped | hipHostMallocCoherent) : hipHostMallocDefault;
    hipError_t e = hipHostMalloc(&ptr, n, flags);
    if (e != hipSuccess) {
      ptr = nullptr;
      failf("hipHostMalloc of %zu bytes for %s failed: %s", n, what, hipGetErrorString(e));
    }
    bytes = n;
    if (mapped) {
      e = hipHostGetDevicePointer(&dev, ptr, 0);
      if (e != hipSuccess) {
        reset();
        failf("hipHostGetDevicePointer for %s failed: %s", what, hipGetErrorString(e));
      }
    }
  }
  template <typename T>
  T* as() const { return static_cast<T*>(ptr); }
  template <typename T>
  T* dev_as() const { return static_cast<T*>(dev); }
};

int current_device_checked() {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0) failf("no HIP device available");
  int dev = 0;
  HIPC(hipGetDevice(&dev));
  return dev;
}

// Upload packed bytes with kWeightPad readable (zeroed) bytes after them and
// reject Inf/NaN fp16 scale fields as fp16-to-single-float does
// (llambda.lisp:727-728).
void upload_weights(DevBuf& buf, const void* host, size_t bytes, int type, int64_t nblocks,
                    hipStream_t stream, const char* what) {
  buf.alloc(bytes + kWeightPad, what);
  HIPC(hipMemcpyAsync(buf.ptr, host, bytes, hipMemcpyHostToDevice, stream));
  std::vector<uint8_t> zeros(kWeightPad, 0);
  HIPC(hipMemcpyAsync(buf.as<uint8_t>() + bytes, zeros.data(), kWeightPad, hipMemcpyHostToDevice,
                      stream));
  if (type == kF32) {
    HIPC(hipStreamSynchronize(stream));
    return;
  }
  DevBuf flag;
  flag.alloc(sizeof(unsigned long long), "validation flag");
  const unsigned long long none = ULLONG_MAX;
  HIPC(hipMemcpyAsync(flag.ptr, &none, sizeof none, hipMemcpyHostToDevice, stream));
  HIPC(validate_launch(type, buf.as<uint8_t>(), nblocks, flag.as<unsigned long long>(), stream));
  unsigned long long first_bad = 0;
  HIPC(hipMemcpyAsync(&first_bad, flag.ptr, sizeof first_bad, hipMemcpyDeviceToHost, stream));
  HIPC(hipStreamSynchronize(stream));
  if (first_bad != ULLONG_MAX)
    failf("%s: Unsupported fp16 special value (Inf/NaN scale) in block %llu.", what, first_bad);
}

}  // namespace

// ------------------------------------------------------------------ sessions

struct llambda_hip_session {
  std::mutex run_mutex;
  int device = 0;
  int type = 0;
  int64_t rows = 0, columns = 0, row_bytes = 0;
  hipStream_t stream = nullptr;
  DevBuf weights;
  DevBuf x, y;    // device staging for the host-pointer runs
  HostBuf hx, hy;  // their pinned host side; hy is mapped
  size_t staged_tokens = 0;
  ~llambda_hip_session() {
    if (stream) (void)hipStreamDestroy(stream);
  }
  void ensure_staging(size_t batch) {
    if (batch <= staged_tokens) return;
    x.alloc(batch * (size_t)columns * sizeof(float), "session input");
    y.alloc(batch * (size_t)rows * sizeof(float), "session output");
    hx.alloc(batch * (size_t)columns * sizeof(float), false, "session input (host)");
    hy.alloc(batch * (size_t)rows * sizeof(float), true, "session output (host)");
    staged_tokens = batch;
  }
  void launch(const float* dx, float* dy, size_t batch, hipStream_t s) {
    GemvProblem p{};
    p.type = type;
    p.weights = weights.as<uint8_t>();
    p.row_bytes = row_bytes;
    p.rows = rows;
    p.columns = columns;
    p.x = dx;
    p.x_stride = columns;
    p.tokens = (int)batch;
    p.y = dy;
    p.y_stride = rows;
    HIPC(gemv_launch(p, s));
  }
};

static llambda_hip_session* make_session(const void* data, size_t size, int type, int64_t rows,
                                         int64_t columns) {
  const int64_t rb = checked_row_bytes(type, columns, "session");
  if (rows <= 0 || rows > INT_MAX) failf("session: row count %lld out of range", (long long)rows);
  if ((uint64_t)rows * (uint64_t)rb != size)
    failf("session: %zu bytes do not hold %lld rows of %lld %s columns (%lld bytes)", size,
          (long long)rows, (long long)columns, type_name(type), (long long)(rows * rb));
  if (!data) failf("session: null tensor data");
  auto* s = new llambda_hip_session();
  try {
    s->device = current_device_checked();
    s->type = type;
    s->rows = rows;
    s->columns = columns;
    s->row_bytes = rb;
    HIPC(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking));
    const int64_t nblocks = rows * (columns / block_weights(type));
    upload_weights(s->weights, data, size, type, nblocks, s->stream, "session");
  } catch (...) {
    delete s;
    throw;
  }
  return s;
}

extern "C" {

int llambda_hip_probe(void) {
  g_last_error.clear();
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e == hipErrorNoDevice || (e == hipSuccess && count == 0)) return 0;
  if (e != hipSuccess) {
    g_last_error = std::string("hipGetDeviceCount failed: ") + hipGetErrorString(e);
    return -1;
  }
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return -1;
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

const char* llambda_hip_bridge_version(void) { return "llambda-hip 0.1.0 (gfx950)"; }

const char* llambda_hip_runtime_version(void) {
  thread_local std::string text;
  int rt = 0, drv = 0;
  const bool ok_rt = hipRuntimeGetVersion(&rt) == hipSuccess;
  const bool ok_drv = hipDriverGetVersion(&drv) == hipSuccess;
  char buf[128];
  snprintf(buf, sizeof buf, "HIP runtime %d, driver %d", ok_rt ? rt : -1, ok_drv ? drv : -1);
  text = buf;
  return text.c_str();
}

const char* llambda_hip_last_error(void) { return g_last_error.c_str(); }

int llambda_hip_sha256(const void* data, size_t data_size, char* output, size_t output_size) {
  return guarded([&] {
    if (!output || output_size < 65) failf("sha256: output buffer must hold 65 bytes");
    if (!data && data_size) failf("sha256: null data");
    sha256_hex(data ? data : "", data_size, output);
  });
}

int llambda_hip_session_create(const char* model_path, const char* cache_dir,
                               const char* cache_key, llambda_hip_session** result) {
  (void)cache_dir;
  (void)cache_key;
  return guarded([&] {
    if (!result) failf("session_create: null result pointer");
    *result = nullptr;
    if (!model_path) failf("session_create: null model path");
    const int fd = open(model_path, O_RDONLY);
    if (fd < 0) failf("session_create: cannot open %s", model_path);
    struct stat st;
    if (fstat(fd, &st) != 0) {
      close(fd);
      failf("session_create: cannot stat %s", model_path);
    }
    const size_t size = (size_t)st.st_size;
    if (size < 40) {
      close(fd);
      failf("session_create: %s is not a packed projection (too short)", model_path);
    }
    void* map = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) failf("session_create: cannot map %s", model_path);
    struct Unmap {
      void* p;
      size_t n;
      ~Unmap() { munmap(p, n); }
    } unmap{map, size};
    const uint8_t* b = static_cast<const uint8_t*>(map);
    if (std::memcmp(b, "LLHIPPRJ", 8) != 0)
      failf("session_create: %s is not a packed projection (bad magic)", model_path);
    uint32_t version, type;
    uint64_t rows, columns, payload;
    std::memcpy(&version, b + 8, 4);
    std::memcpy(&type, b + 12, 4);
    std::memcpy(&rows, b + 16, 8);
    std::memcpy(&columns, b + 24, 8);
    std::memcpy(&payload, b + 32, 8);
    if (version != 1) failf("session_create: unsupported packed projection version %u", version);
    if (payload != size - 40)
      failf("session_create: %s payload size %llu does not match the file (%zu bytes)", model_path,
            (unsigned long long)payload, size - 40);
    *result = make_session(b + 40, (size_t)payload, (int)type, (int64_t)rows, (int64_t)columns);
  });
}

int llambda_hip_session_create_packed(const void* data, size_t data_size, int ggml_type,
                                      int64_t rows, int64_t columns,
                                      llambda_hip_session** result) {
  return guarded([&] {
    if (!result) failf("session_create_packed: null result pointer");
    *result = nullptr;
    *result = make_session(data, data_size, ggml_type, rows, columns);
  });
}

void llambda_hip_session_destroy(llambda_hip_session* session) { delete session; }

size_t llambda_hip_session_input_element_count(const llambda_hip_session* session) {
  return session ? (size_t)session->columns : 0;
}

size_t llambda_hip_session_output_element_count(const llambda_hip_session* session) {
  return session ? (size_t)session->rows : 0;
}

int llambda_hip_session_run_batch(llambda_hip_session* s, const float* input, size_t n_in,
                                  float* output, size_t n_out, size_t batch) {
  return guarded([&] {
    if (!s) failf("session_run: null session");
    if (!input || !output) failf("session_run: null input or output");
    if (batch == 0) failf("session_run: batch must be positive");
    if (batch > (size_t)INT_MAX / 2) failf("session_run: batch too large");
    if (n_in != batch * (size_t)s->columns)
      failf("session_run: input element count %zu does not match %zu x %lld", n_in, batch,
            (long long)s->columns);
    if (n_out != batch * (size_t)s->rows)
      failf("session_run: output element count %zu does not match %zu x %lld", n_out, batch,
            (long long)s->rows);
    std::lock_guard<std::mutex> lock(s->run_mutex);
    HIPC(hipSetDevice(s->device));
    s->ensure_staging(batch);
    std::memcpy(s->hx.ptr, input, n_in * sizeof(float));
    HIPC(hipMemcpyAsync(s->x.ptr, s->hx.ptr, n_in * sizeof(float), hipMemcpyHostToDevice, s->stream));
    if (batch == 1) {
      // one token's rows are stored by the kernel straight into host memory
      s->launch(s->x.as<float>(), s->hy.dev_as<float>(), batch, s->stream);
    } else {
      s->launch(s->x.as<float>(), s->y.as<float>(), batch, s->stream);
      HIPC(hipMemcpyAsync(s->hy.ptr, s->y.ptr, n_out * sizeof(float), hipMemcpyDeviceToHost, s->stream));
    }
    HIPC(hipStreamSynchronize(s->stream));
    std::memcpy(output, s->hy.ptr, n_out * sizeof(float));
  });
}

int llambda_hip_session_run(llambda_hip_session* s, const float* input, size_t n_in,
                            float* output, size_t n_out) {
  return llambda_hip_session_run_batch(s, input, n_in, output, n_out, 1);
}

int llambda_hip_session_run_device(llambda_hip_session* s, const float* input, float* output,
                                   size_t batch, void* stream) {
  return guarded([&] {
    if (!s) failf("session_run_device: null session");
    if (!input || !output) failf("session_run_device: null input or output");
    if (batch == 0 || batch > (size_t)INT_MAX / 2) failf("session_run_device: bad batch %zu", batch);
    HIPC(hipSetDevice(s->device));
    s->launch(input, output, batch, stream ? static_cast<hipStream_t>(stream) : s->stream);
  });
}

int llambda_hip_session_dequantize(llambda_hip_session* s, float* output, size_t n_out) {
  return guarded([&] {
    if (!s) failf("session_dequantize: null session");
    if (!output) failf("session_dequantize: null output");
    if (n_out != (size_t)(s->rows * s->columns))
      failf("session_dequantize: output element count %zu does not match %lld x %lld", n_out,
            (long long)s->rows, (long long)s->columns);
    std::lock_guard<std::mutex> lock(s->run_mutex);
    HIPC(hipSetDevice(s->device));
    DevBuf out;
    out.alloc(n_out * sizeof(float), "dequantized weights");
    if (s->type == kF32) {
      HIPC(hipMemcpyAsync(out.ptr, s->weights.ptr, n_out * sizeof(float), hipMemcpyDeviceToDevice,
                          s->stream));
    } else {
      HIPC(dequant_launch(s->type, s->weights.as<uint8_t>(), s->row_bytes, s->rows, s->columns,
                          out.as<float>(), s->stream));
    }
    HIPC(hipMemcpyAsync(output, out.ptr, n_out * sizeof(float), hipMemcpyDeviceToHost, s->stream));
    HIPC(hipStreamSynchronize(s->stream));
  });
}

}  // extern "C"

// ------------------------------------------------------------- MoE sessions

// Bytes of each per-run scratch buffer of one MoE forward over T tokens, as
// the kernels index them.
struct MoeScratchBytes {
  size_t logits, router_part, top_idx, top_w, shared_w, perm, chunks, down_out, xq, xsum, aq,
      asum, lat, lq, lsum, lat_y;
};

static MoeScratchBytes moe_scratch_bytes(const MoePlan& p, size_t T) {
  const size_t K = (size_t)p.top_k, E = (size_t)p.experts, H = (size_t)p.hidden;
  const size_t pairs = T * (K + 1);
  const size_t act_w = (size_t)std::max(p.ffn, p.shared_ffn);
  MoeScratchBytes b;
  b.logits = T * (E + 1) * sizeof(float);
  b.router_part = (size_t)router_slices(p.hidden) * T * (E + 1) * sizeof(float);
  b.top_idx = T * K * sizeof(int);
  b.top_w = T * K * sizeof(float);
  b.shared_w = T * sizeof(float);
  b.perm = pairs * sizeof(int);
  // (+ 8: the batch products read the entry of every workgroup of their
  // grid, which is padded to a multiple of 8, before they compare its index
  // with the count)
  b.chunks = (size_t)(moe_max_chunks(p, (int64_t)T, 1) + 8) * sizeof(MoeChunk);
  b.down_out = pairs * (size_t)p.out_w * sizeof(float);
  // the decode pipeline stages whole 256-element chunks (1 KB of split row)
  // of a row's last, partial chunk: 1 KB of readable slack
  b.xq = T * 2 * H * sizeof(uint16_t) + 1024;
  // (+ 256: the group pipeline stages the sums of two 32-groups at a time
  // and reads past a row whose group count is odd)
  b.xsum = T * (H / 16) * sizeof(float) + 256;
  b.aq = pairs * 2 * act_w * sizeof(uint16_t) + 1024;
  b.asum = pairs * (act_w / 16) * sizeof(float) + 256;
  // latent layers: the experts' input (then their weighted sum), its split
  // rows (the same slack as x's), the ffn_latent_up output
  const size_t Li = (size_t)p.latent_in, Lo = (size_t)p.latent_out;
  b.lat = T * std::max(Li, Lo) * sizeof(float);
  b.lq = Li ? T * 2 * Li * sizeof(uint16_t) + 1024 : 0;
  b.lsum = Li ? T * (Li / 16) * sizeof(float) + 256 : 0;
  b.lat_y = Lo ? T * H * sizeof(float) : 0;
  return b;
}

struct llambda_hip_moe_session {
  std::mutex run_mutex;
  int device = 0;
  hipStream_t stream = nullptr;
  MoePlan plan{};
  DevBuf router, bias, gate, up, down, sh_gate, sh_up, sh_down, lat_down, lat_up;
  DevBuf up_g, down_g, sh_up_g, sh_down_g;  // stage-major copies (group pipeline)
  DevBuf logits, router_part, top_idx, top_w, shared_w, perm, chunks, chunk_counts,
      down_out, error, xq, xsum, aq, asum, lat, lq, lsum, lat_y;
  DevBuf x, y;     // device staging for the host-pointer runs
  HostBuf hx, hy;  // their pinned host side; hy is mapped, the error word after the rows
  int staged = 0;
  ~llambda_hip_moe_session() {
    if (stream) (void)hipStreamDestroy(stream);
  }
  // Size the scratch for `tokens` tokens (grows only).
  void ensure_capacity(int tokens) {
    if (tokens <= plan.capacity) return;
    MoePlan& p = plan;
    const MoeScratchBytes b = moe_scratch_bytes(p, (size_t)tokens);
    p.router_ks = router_slices(p.hidden);
    logits.alloc(b.logits, "router logits");
    router_part.alloc(b.router_part, "router slice sums");
    top_idx.alloc(b.top_idx, "top-k indices");
    top_w.alloc(b.top_w, "top-k weights");
    shared_w.alloc(b.shared_w, "shared weights");
    perm.alloc(b.perm, "permutation");
    chunks.alloc(b.chunks, "chunk table");
    down_out.alloc(b.down_out, "expert outputs");
    xq.alloc(b.xq, "split input");
    xsum.alloc(b.xsum, "input group sums");
    aq.alloc(b.aq, "split activations");
    asum.alloc(b.asum, "activation group sums");
    lat.alloc(b.lat, "latent vectors");
    lq.alloc(b.lq, "split latent input");
    lsum.alloc(b.lsum, "latent input group sums");
    lat_y.alloc(b.lat_y, "ffn_latent_up output");
    p.capacity = tokens;
    p.router_part = router_part.as<float>();
    p.xq = xq.as<uint16_t>();
    p.xsum = xsum.as<float>();
    p.aq = aq.as<uint16_t>();
    p.asum = asum.as<float>();
    p.logits = logits.as<float>();
    p.top_idx = top_idx.as<int>();
    p.top_w = top_w.as<float>();
    p.shared_w = shared_w.as<float>();
    p.perm = perm.as<int>();
    p.chunks = chunks.as<MoeChunk>();
    p.down_out = down_out.as<float>();
    p.lat = lat.as<float>();
    p.lq = lq.as<uint16_t>();
    p.lsum = lsum.as<float>();
    p.lat_y = lat_y.as<float>();
  }
  void ensure_staging(int tokens) {
    if (tokens <= staged) return;
    const size_t bytes = (size_t)tokens * plan.hidden * sizeof(float);
    x.alloc(bytes, "MoE input");
    y.alloc(bytes, "MoE output");
    hx.alloc(bytes, false, "MoE input (host)");
    hy.alloc(bytes + 64, true, "MoE output (host)");
    staged = tokens;
  }
  int take_error(hipStream_t s) {
    int flag = 0;
    HIPC(hipMemcpyAsync(&flag, plan.error, sizeof flag, hipMemcpyDeviceToHost, s));
    HIPC(hipStreamSynchronize(s));
    if (flag) {
      const int zero = 0;
      HIPC(hipMemcpyAsync(plan.error, &zero, sizeof zero, hipMemcpyHostToDevice, s));
      HIPC(hipStreamSynchronize(s));
    }
    return flag;
  }
};

// The kernels' error word: bit 1 = a non-positive top-k weight sum
// (llambda.lisp:5373-5375, 5903-5905), bit 0 = fewer than k selectable
// logits, where the reference's expert lookup fails on index -1.  Both are
// the reference's own errors for the input, so they take status -2.
[[noreturn]] static void raise_moe_error(int flag, int variant) {
  const char* layer = variant == kQwen3Next ? "Qwen3Next" : "Nemotron-H MoE";
  char buf[256];
  if (flag & 2)
    snprintf(buf, sizeof buf, "%s layer router produced non-positive top-k weight sum.", layer);
  else if (flag & 1)
    snprintf(buf, sizeof buf,
             "%s layer router produced fewer than top-k selectable logits (Expert index -1 is out of range).",
             layer);
  else
    failf("%s layer failed (error flags %d)", layer, flag);
  throw InputError(buf);
}

extern "C" {

int llambda_hip_moe_session_create(const llambda_hip_moe_desc* d,
                                   llambda_hip_moe_session** result) {
  return guarded([&] {
    if (!result) failf("moe_session_create: null result pointer");
    *result = nullptr;
    if (!d) failf("moe_session_create: null description");
    if (d->variant != LLAMBDA_HIP_MOE_QWEN3NEXT && d->variant != LLAMBDA_HIP_MOE_NEMOTRON_H)
      failf("moe_session_create: unknown variant %d", d->variant);
    const bool qwen = d->variant == LLAMBDA_HIP_MOE_QWEN3NEXT;
    const int64_t Li = d->latent_in, Lo = d->latent_out;
    if ((d->latent_down || d->latent_up || Li || Lo) && qwen)
      failf("moe_session_create: ffn_latent_down / ffn_latent_up belong to Nemotron-H layers");
    const int64_t H = d->hidden, E = d->expert_count, K = d->top_k, F = d->expert_ffn,
                  Fs = d->shared_ffn;
    if (H <= 0 || H % 32 || H > (1 << 16)) failf("moe_session_create: hidden %lld unsupported", (long long)H);
    if (E <= 0 || E > kMoeMaxExperts)
      failf("moe_session_create: expert count %lld outside 1..%d", (long long)E, kMoeMaxExperts);
    if (K <= 0 || K > E || K > kMoeMaxTopK)
      failf("moe_session_create: top_k %lld outside 1..min(E, %d)", (long long)K, kMoeMaxTopK);
    if (F <= 0 || F % 32 || F > (1 << 16)) failf("moe_session_create: expert ffn %lld unsupported", (long long)F);
    if (Fs < 0 || Fs % 32 || Fs > (1 << 16)) failf("moe_session_create: shared ffn %lld unsupported", (long long)Fs);
    if (!d->router) failf("moe_session_create: missing router (ffn_gate_inp)");
    if (!d->up_exps || !d->down_exps) failf("moe_session_create: missing expert tensors");
    if (qwen && !d->gate_exps) failf("moe_session_create: missing ffn_gate_exps");
    if (qwen && d->gate_type != d->up_type)
      failf("moe_session_create: ffn_gate_exps and ffn_up_exps must share a type");
    if (!qwen && !d->router_bias) failf("moe_session_create: missing exp_probs_b.bias");
    if ((Li != 0) != (d->latent_down != nullptr) || Li < 0 || Li % 32 || Li > (1 << 16))
      failf("moe_session_create: ffn_latent_down needs its row count (latent_in %lld), a positive "
            "multiple of 32 up to 65536", (long long)Li);
    if ((Lo != 0) != (d->latent_up != nullptr) || Lo < 0 || Lo > (1 << 16))
      failf("moe_session_create: ffn_latent_up needs its column count (latent_out %lld), "
            "positive and up to 65536", (long long)Lo);
    const int64_t din = Li ? Li : H, dout = Lo ? Lo : H;
    if (Fs > 0) {
      if (!d->shared_up || !d->shared_down) failf("moe_session_create: missing shared expert tensors");
      if (qwen && (!d->shared_gate || !d->shared_gate_inp))
        failf("moe_session_create: missing ffn_gate_shexp or ffn_gate_inp_shexp");
      if (qwen && d->shared_gate_type != d->shared_up_type)
        failf("moe_session_create: ffn_gate_shexp and ffn_up_shexp must share a type");
    }
    const int types[] = {d->up_type, d->down_type, Fs > 0 ? d->shared_up_type : kQ4_K,
                         Fs > 0 ? d->shared_down_type : kQ4_K};
    for (int t : types)
      if (t == kF32 || !supported_type(t))
        failf("moe_session_create: expert tensors must be Q4_K, Q6_K, Q5_0 or Q8_0 (got tag %d)", t);
    const int64_t up_rb = checked_row_bytes(d->up_type, din, "ffn_up_exps");
    const int64_t down_rb = checked_row_bytes(d->down_type, F, "ffn_down_exps");
    // the expert kernels address one expert's slab (in its device layout)
    // with 32-bit offsets
    if (std::max(F * up_rb, moe_slab_bytes(d->up_type, F, din)) + (int64_t)kWeightPad >=
            ((int64_t)1 << 31) ||
        std::max(dout * down_rb, moe_slab_bytes(d->down_type, dout, F)) + (int64_t)kWeightPad >=
            ((int64_t)1 << 31))
      failf("moe_session_create: one expert's slab exceeds 2 GiB");
    const int64_t ld_rb = Li ? checked_row_bytes(d->latent_down_type, H, "ffn_latent_down") : 0;
    const int64_t lu_rb = Lo ? checked_row_bytes(d->latent_up_type, Lo, "ffn_latent_up") : 0;

    auto* s = new llambda_hip_moe_session();
    try {
      s->device = current_device_checked();
      HIPC(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking));
      MoePlan& p = s->plan;
      p.variant = qwen ? kQwen3Next : kNemotronH;
      p.hidden = (int)H;
      p.experts = (int)E;
      p.top_k = (int)K;
      p.ffn = (int)F;
      p.shared_ffn = (int)Fs;
      p.weights_scale = qwen ? 1.0f : d->expert_weights_scale;
      p.weights_norm = qwen ? 1 : (d->expert_weights_norm ? 1 : 0);
      // router [E (+1 shared gate row)][H]
      const size_t rbytes = (size_t)(E + 1) * H * sizeof(float);
      s->router.alloc(rbytes, "router");
      HIPC(hipMemcpyAsync(s->router.ptr, d->router, (size_t)E * H * sizeof(float),
                          hipMemcpyHostToDevice, s->stream));
      if (qwen && Fs > 0)
        HIPC(hipMemcpyAsync(s->router.as<float>() + E * H, d->shared_gate_inp, (size_t)H * sizeof(float),
                            hipMemcpyHostToDevice, s->stream));
      p.router = s->router.as<float>();
      if (!qwen) {
        s->bias.alloc((size_t)E * sizeof(float), "router bias");
        HIPC(hipMemcpyAsync(s->bias.ptr, d->router_bias, (size_t)E * sizeof(float),
                            hipMemcpyHostToDevice, s->stream));
        p.bias = s->bias.as<float>();
      }
      const int64_t up_blocks = E * F * (din / block_weights(d->up_type));
      const int64_t down_blocks = E * dout * (F / block_weights(d->down_type));
      p.up_type = d->up_type;
      p.down_type = d->down_type;
      p.gate_type = qwen ? d->gate_type : d->up_type;
      if (qwen) {
        upload_weights(s->gate, d->gate_exps, (size_t)(E * F * up_rb), d->gate_type, up_blocks,
                       s->stream, "ffn_gate_exps");
        p.gate = s->gate.as<uint8_t>();
      }
      upload_weights(s->up, d->up_exps, (size_t)(E * F * up_rb), d->up_type, up_blocks, s->stream,
                     "ffn_up_exps");
      upload_weights(s->down, d->down_exps, (size_t)(E * dout * down_rb), d->down_type, down_blocks,
                     s->stream, "ffn_down_exps");
      p.up = s->up.as<uint8_t>();
      p.down = s->down.as<uint8_t>();
      p.latent_in = (int)Li;
      p.latent_out = (int)Lo;
      p.out_w = (int)std::max(H, Lo);
      if (Li) {
        upload_weights(s->lat_down, d->latent_down, (size_t)(Li * ld_rb), d->latent_down_type,
                       Li * (H / block_weights(d->latent_down_type)), s->stream, "ffn_latent_down");
        p.lat_down_type = d->latent_down_type;
        p.lat_down = s->lat_down.as<uint8_t>();
      }
      if (Lo) {
        upload_weights(s->lat_up, d->latent_up, (size_t)(H * lu_rb), d->latent_up_type,
                       H * (Lo / block_weights(d->latent_up_type)), s->stream, "ffn_latent_up");
        p.lat_up_type = d->latent_up_type;
        p.lat_up = s->lat_up.as<uint8_t>();
      }
      if (Fs > 0) {
        const int64_t sh_up_rb = checked_row_bytes(d->shared_up_type, H, "ffn_up_shexp");
        const int64_t sh_down_rb = checked_row_bytes(d->shared_down_type, Fs, "ffn_down_shexp");
        p.sh_up_type = d->shared_up_type;
        p.sh_down_type = d->shared_down_type;
        p.sh_gate_type = qwen ? d->shared_gate_type : d->shared_up_type;
        if (qwen) {
          upload_weights(s->sh_gate, d->shared_gate, (size_t)(Fs * sh_up_rb), d->shared_gate_type,
                         Fs * (H / block_weights(d->shared_gate_type)), s->stream, "ffn_gate_shexp");
          p.sh_gate = s->sh_gate.as<uint8_t>();
        }
        upload_weights(s->sh_up, d->shared_up, (size_t)(Fs * sh_up_rb), d->shared_up_type,
                       Fs * (H / block_weights(d->shared_up_type)), s->stream, "ffn_up_shexp");
        upload_weights(s->sh_down, d->shared_down, (size_t)(H * sh_down_rb), d->shared_down_type,
                       H * (Fs / block_weights(d->shared_down_type)), s->stream, "ffn_down_shexp");
        p.sh_up = s->sh_up.as<uint8_t>();
        p.sh_down = s->sh_down.as<uint8_t>();
      }
      // the group pipeline's stage-major copies of the one-matrix launches
      // weights (Q5_0 / Q8_0 relu^2 up and every down), made on the device
      auto stage_major = [&](DevBuf& dst, const DevBuf& src, int type, int64_t slabs, int64_t rows,
                             int64_t columns, const char* what) -> const uint8_t* {
        if (!moe_group_pipeline_types(type)) return nullptr;
        dst.alloc((size_t)moe_repack_bytes(type, slabs, rows, columns) + kWeightPad, what);
        HIPC(moe_repack_launch(type, src.as<uint8_t>(), slabs, rows, columns, dst.as<uint8_t>(),
                               s->stream));
        return dst.as<uint8_t>();
      };
      if (!qwen) {
        p.up_g = stage_major(s->up_g, s->up, d->up_type, E, F, din, "ffn_up_exps (stage-major)");
        p.up_g_stride = moe_repack_bytes(d->up_type, 1, F, din);
      }
      p.down_g = stage_major(s->down_g, s->down, d->down_type, E, dout, F,
                             "ffn_down_exps (stage-major)");
      p.down_g_stride = moe_repack_bytes(d->down_type, 1, dout, F);
      if (Fs > 0) {
        if (!qwen)
          p.sh_up_g = stage_major(s->sh_up_g, s->sh_up, d->shared_up_type, 1, Fs, H,
                                  "ffn_up_shexp (stage-major)");
        p.sh_down_g = stage_major(s->sh_down_g, s->sh_down, d->shared_down_type, 1, H, Fs,
                                  "ffn_down_shexp (stage-major)");
      }
      // K-quant expert tensors: the tile-major layout replaces the packed rows
      auto tile_major = [&](DevBuf& buf, int type, int64_t slabs, int64_t rows, int64_t columns,
                            const uint8_t*& ptr, const char* what) {
        if (!moe_tiled_type(type)) return;
        const int64_t bytes = slabs * moe_slab_bytes(type, rows, columns);
        DevBuf t;
        t.alloc((size_t)bytes + kWeightPad, what);
        HIPC(hipMemsetAsync(t.as<uint8_t>() + bytes, 0, kWeightPad, s->stream));
        HIPC(moe_tile_launch(type, buf.as<uint8_t>(), slabs, rows, columns, t.as<uint8_t>(),
                             s->stream));
        HIPC(hipStreamSynchronize(s->stream));
        buf.swap(t);
        ptr = buf.as<uint8_t>();
      };
      if (qwen) tile_major(s->gate, d->gate_type, E, F, din, p.gate, "ffn_gate_exps (tile-major)");
      tile_major(s->up, d->up_type, E, F, din, p.up, "ffn_up_exps (tile-major)");
      tile_major(s->down, d->down_type, E, dout, F, p.down, "ffn_down_exps (tile-major)");
      if (Fs > 0) {
        if (qwen)
          tile_major(s->sh_gate, d->shared_gate_type, 1, Fs, H, p.sh_gate,
                     "ffn_gate_shexp (tile-major)");
        tile_major(s->sh_up, d->shared_up_type, 1, Fs, H, p.sh_up, "ffn_up_shexp (tile-major)");
        tile_major(s->sh_down, d->shared_down_type, 1, H, Fs, p.sh_down,
                   "ffn_down_shexp (tile-major)");
      }
      s->chunk_counts.alloc(2 * sizeof(int), "chunk counts");
      s->error.alloc(sizeof(int), "error flag");
      p.chunk_counts = s->chunk_counts.as<int>();
      p.error = s->error.as<int>();
      p.capacity = 0;
      s->ensure_capacity(1);
      HIPC(moe_reset_launch(p, s->stream));
      HIPC(hipStreamSynchronize(s->stream));
    } catch (...) {
      delete s;
      throw;
    }
    *result = s;
  });
}

void llambda_hip_moe_session_destroy(llambda_hip_moe_session* session) { delete session; }

size_t llambda_hip_moe_session_hidden_size(const llambda_hip_moe_session* session) {
  return session ? (size_t)session->plan.hidden : 0;
}

size_t llambda_hip_moe_session_expert_count(const llambda_hip_moe_session* session) {
  return session ? (size_t)session->plan.experts : 0;
}

int llambda_hip_moe_session_run(llambda_hip_moe_session* s, const float* input, size_t n_in,
                                float* output, size_t n_out, size_t batch, int64_t* top_indices,
                                float* top_weights, float* router_logits) {
  return guarded([&] {
    if (!s) failf("moe_session_run: null session");
    if (!input || !output) failf("moe_session_run: null input or output");
    if (batch == 0 || batch > (1u << 20)) failf("moe_session_run: bad batch %zu", batch);
    const size_t H = (size_t)s->plan.hidden;
    if (n_in != batch * H || n_out != batch * H)
      failf("moe_session_run: element counts %zu/%zu do not match %zu x %zu", n_in, n_out, batch, H);
    std::lock_guard<std::mutex> lock(s->run_mutex);
    HIPC(hipSetDevice(s->device));
    const int T = (int)batch;
    s->ensure_capacity(T);
    s->ensure_staging(T);
    std::memcpy(s->hx.ptr, input, n_in * sizeof(float));
    HIPC(hipMemcpyAsync(s->x.ptr, s->hx.ptr, n_in * sizeof(float), hipMemcpyHostToDevice, s->stream));
    // the final launch stores the error word after the rows in mapped host
    // memory, and one token's rows too
    float* rows_dev = T == 1 ? s->hy.dev_as<float>() : s->y.as<float>();
    volatile int* flag_host = reinterpret_cast<int*>(s->hy.as<float>() + n_out);
    int* flag_dev = reinterpret_cast<int*>(s->hy.dev_as<float>() + n_out);
    *flag_host = -1;
    HIPC(moe_forward_launch(s->plan, s->x.as<float>(), rows_dev, T, s->stream, flag_dev));
    if (T > 1)
      HIPC(hipMemcpyAsync(s->hy.ptr, s->y.ptr, n_out * sizeof(float), hipMemcpyDeviceToHost, s->stream));
    const size_t K = (size_t)s->plan.top_k, E = (size_t)s->plan.experts;
    std::vector<int> idx;
    if (top_indices) {
      idx.resize(batch * K);
      HIPC(hipMemcpyAsync(idx.data(), s->plan.top_idx, idx.size() * sizeof(int),
                          hipMemcpyDeviceToHost, s->stream));
    }
    if (top_weights)
      HIPC(hipMemcpyAsync(top_weights, s->plan.top_w, batch * K * sizeof(float),
                          hipMemcpyDeviceToHost, s->stream));
    if (router_logits)
      HIPC(hipMemcpy2DAsync(router_logits, E * sizeof(float), s->plan.logits, (E + 1) * sizeof(float),
                            E * sizeof(float), batch, hipMemcpyDeviceToHost, s->stream));
    HIPC(hipStreamSynchronize(s->stream));
    std::memcpy(output, s->hy.ptr, n_out * sizeof(float));
    const int flag = *flag_host;
    if (flag < 0) failf("moe_session_run: the forward did not report its error word");
    if (flag) {
      HIPC(moe_reset_launch(s->plan, s->stream));
      HIPC(hipStreamSynchronize(s->stream));
    }
    for (size_t i = 0; i < idx.size(); ++i) top_indices[i] = idx[i];
    if (flag) raise_moe_error(flag, s->plan.variant);
  });
}

int llambda_hip_moe_session_run_device(llambda_hip_moe_session* s, const float* input,
                                       float* output, size_t batch, void* stream) {
  return guarded([&] {
    if (!s) failf("moe_session_run_device: null session");
    if (!input || !output) failf("moe_session_run_device: null input or output");
    if (batch == 0 || batch > (1u << 20)) failf("moe_session_run_device: bad batch %zu", batch);
    if (reinterpret_cast<uintptr_t>(input) & 15u)
      failf("moe_session_run_device: input must be 16-byte aligned");
    std::lock_guard<std::mutex> lock(s->run_mutex);
    HIPC(hipSetDevice(s->device));
    const int T = (int)batch;
    if (T > s->plan.capacity) {
      // growing frees scratch that queued work may still use
      HIPC(hipStreamSynchronize(stream ? static_cast<hipStream_t>(stream) : s->stream));
      HIPC(hipStreamSynchronize(s->stream));
      s->ensure_capacity(T);
    }
    HIPC(moe_forward_launch(s->plan, input, output, T,
                            stream ? static_cast<hipStream_t>(stream) : s->stream));
  });
}

int llambda_hip_moe_session_sync(llambda_hip_moe_session* s, void* stream) {
  return guarded([&] {
    if (!s) failf("moe_session_sync: null session");
    std::lock_guard<std::mutex> lock(s->run_mutex);
    HIPC(hipSetDevice(s->device));
    const int flag = s->take_error(stream ? static_cast<hipStream_t>(stream) : s->stream);
    if (flag) raise_moe_error(flag, s->plan.variant);
  });
}

}  // extern "C"

// ----------------------------------------------- no-allocation MoE runs
// One MoE forward's scratch for llambda_hip_moe_session_run_device_noalloc:
// a file-scope device array, one per GPU, held until the process ends.  Its
// name is a host-side stand-in: host code uses only the device address that
// hipGetSymbolAddress returns for the current device (kept per device).
constexpr size_t kMoeNoallocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[kMoeNoallocScratchBytes];

namespace {

constexpr int kMaxScratchDevices = 64;
// g_scratch_mutex is held across a whole call (wait, launches, record), so
// the calls' order on the device is the order they took the mutex.
std::mutex g_scratch_mutex;
uint8_t* g_scratch[kMaxScratchDevices];
// Recorded after each call's last launch on its stream; the next call's
// stream waits for it first, so calls on one GPU never overlap on the device
// whatever stream or session they come from.
hipEvent_t g_scratch_done[kMaxScratchDevices];

// Set-up, once per device (current): the device address of `scratch` and
// the ordering event.  The caller holds g_scratch_mutex.
uint8_t* noalloc_scratch(int device) {
  if (device < 0 || device >= kMaxScratchDevices)
    failf("moe_session_run_device_noalloc: device %d beyond the %d tracked", device,
          kMaxScratchDevices);
  if (!g_scratch[device]) {
    void* ptr = nullptr;
    HIPC(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (!ptr) failf("moe_session_run_device_noalloc: no device address for the scratch array");
    if (!g_scratch_done[device])
      HIPC(hipEventCreateWithFlags(&g_scratch_done[device], hipEventDisableTiming));
    g_scratch[device] = static_cast<uint8_t*>(ptr);
  }
  return g_scratch[device];
}

// Point p's per-run buffers into [base, base + limit) for T tokens; returns
// the bytes the layout needs (nothing is assigned when that exceeds limit).
size_t carve_moe_scratch(MoePlan& p, int T, uint8_t* base, size_t limit) {
  const MoeScratchBytes b = moe_scratch_bytes(p, (size_t)T);
  const size_t sizes[] = {b.logits, b.router_part, b.top_idx, b.top_w, b.shared_w, b.perm,
                          b.chunks, b.down_out, b.xq, b.xsum, b.aq, b.asum, 2 * sizeof(int),
                          sizeof(int), b.lat, b.lq, b.lsum, b.lat_y};
  constexpr int kBuffers = sizeof(sizes) / sizeof(sizes[0]);
  size_t off[kBuffers], total = 0;
  for (int i = 0; i < kBuffers; ++i) {
    off[i] = total;
    total += (sizes[i] + 255) & ~(size_t)255;
  }
  if (total > limit) return total;
  p.logits = reinterpret_cast<float*>(base + off[0]);
  p.router_part = reinterpret_cast<float*>(base + off[1]);
  p.top_idx = reinterpret_cast<int*>(base + off[2]);
  p.top_w = reinterpret_cast<float*>(base + off[3]);
  p.shared_w = reinterpret_cast<float*>(base + off[4]);
  p.perm = reinterpret_cast<int*>(base + off[5]);
  p.chunks = reinterpret_cast<MoeChunk*>(base + off[6]);
  p.down_out = reinterpret_cast<float*>(base + off[7]);
  p.xq = reinterpret_cast<uint16_t*>(base + off[8]);
  p.xsum = reinterpret_cast<float*>(base + off[9]);
  p.aq = reinterpret_cast<uint16_t*>(base + off[10]);
  p.asum = reinterpret_cast<float*>(base + off[11]);
  p.chunk_counts = reinterpret_cast<int*>(base + off[12]);
  p.error = reinterpret_cast<int*>(base + off[13]);
  p.lat = reinterpret_cast<float*>(base + off[14]);
  p.lq = reinterpret_cast<uint16_t*>(base + off[15]);
  p.lsum = reinterpret_cast<float*>(base + off[16]);
  p.lat_y = reinterpret_cast<float*>(base + off[17]);
  p.router_ks = router_slices(p.hidden);
  p.capacity = T;
  return total;
}

}  // namespace

extern "C" {

int llambda_hip_moe_session_run_device_noalloc(llambda_hip_moe_session* s, const float* input,
                                               float* output, size_t batch, void* stream) {
  return guarded([&] {
    if (!s) failf("moe_session_run_device_noalloc: null session");
    if (!input || !output) failf("moe_session_run_device_noalloc: null input or output");
    if (batch == 0 || batch > (1u << 20))
      failf("moe_session_run_device_noalloc: bad batch %zu", batch);
    if (reinterpret_cast<uintptr_t>(input) & 15u)
      failf("moe_session_run_device_noalloc: input must be 16-byte aligned");
    std::lock_guard<std::mutex> lock(s->run_mutex);
    HIPC(hipSetDevice(s->device));
    const int T = (int)batch;
    MoePlan p = s->plan;  // the session's weights and knobs; the scratch is replaced
    const size_t need = carve_moe_scratch(p, T, nullptr, 0);
    if (need > kMoeNoallocScratchBytes)
      failf("moe_session_run_device_noalloc: %zu tokens of this layer need %zu bytes of scratch; "
            "the no-allocation entry point holds %zu (run fewer tokens per call, or use "
            "llambda_hip_moe_session_run_device)",
            batch, need, kMoeNoallocScratchBytes);
    std::lock_guard<std::mutex> order(g_scratch_mutex);
    uint8_t* base = noalloc_scratch(s->device);
    carve_moe_scratch(p, T, base, kMoeNoallocScratchBytes);
    const hipStream_t st = stream ? static_cast<hipStream_t>(stream) : s->stream;
    // Outside stream capture, wait for the previous call's last launch.  A
    // captured call is ordered by the graph it joins: replays of graphs that
    // hold such calls must not overlap on one GPU.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    HIPC(hipStreamIsCapturing(st, &capture));
    const bool ordered = capture == hipStreamCaptureStatusNone;
    if (ordered) HIPC(hipStreamWaitEvent(st, g_scratch_done[s->device], 0));
    // the error flag must start at zero (the array keeps the last call's
    // contents); a fill kernel, not a memset, so that a captured graph
    // replays it faithfully
    HIPC(moe_reset_launch(p, st));
    HIPC(moe_forward_launch(p, input, output, T, st));
    // errors reach the session's own flag, reported by moe_session_sync
    HIPC(moe_error_merge_launch(p.error, s->plan.error, st));
    if (ordered) HIPC(hipEventRecord(g_scratch_done[s->device], st));
  });
}

int llambda_hip_stream_read(const void* data, size_t bytes, uint32_t* out, void* stream) {
  return guarded([&] {
    static_assert(LLAMBDA_HIP_STREAM_READ_WORDS == kStreamReadWords, "one out word per wave");
    if (!data || !out) failf("stream_read: null argument");
    if (bytes == 0 || bytes % 16 || reinterpret_cast<uintptr_t>(data) % 16)
      failf("stream_read: %zu bytes at %p: need a positive multiple of 16, 16-byte aligned", bytes,
            data);
    HIPC(stream_read_launch(data, bytes, out, static_cast<hipStream_t>(stream)));
  });
}

int llambda_hip_select_top_k(const float* logits, size_t n, size_t k, size_t batch,
                             int64_t* top_indices, float* top_logits) {
  return guarded([&] {
    if (!logits || !top_indices || !top_logits) failf("select_top_k: null argument");
    if (n == 0 || n > (size_t)kMoeMaxExperts) failf("select_top_k: n must be in 1..%d", kMoeMaxExperts);
    if (k == 0 || k > (size_t)kMoeMaxTopK) failf("select_top_k: k must be in 1..%d", kMoeMaxTopK);
    if (batch == 0 || batch > (1u << 20)) failf("select_top_k: bad batch %zu", batch);
    current_device_checked();
    hipStream_t stream;
    HIPC(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
    struct StreamGuard {
      hipStream_t s;
      ~StreamGuard() { (void)hipStreamDestroy(s); }
    } guard{stream};
    DevBuf dl, di, dv;
    dl.alloc(batch * n * sizeof(float), "logits");
    di.alloc(batch * k * sizeof(int), "indices");
    dv.alloc(batch * k * sizeof(float), "values");
    HIPC(hipMemcpyAsync(dl.ptr, logits, batch * n * sizeof(float), hipMemcpyHostToDevice, stream));
    HIPC(topk_launch(dl.as<float>(), (int)n, (int)k, (int)batch, di.as<int>(), dv.as<float>(), stream));
    std::vector<int> idx(batch * k);
    HIPC(hipMemcpyAsync(idx.data(), di.ptr, idx.size() * sizeof(int), hipMemcpyDeviceToHost, stream));
    HIPC(hipMemcpyAsync(top_logits, dv.ptr, batch * k * sizeof(float), hipMemcpyDeviceToHost, stream));
    HIPC(hipStreamSynchronize(stream));
    for (size_t i = 0; i < idx.size(); ++i) top_indices[i] = idx[i];
  });
}

}  // extern "C"

// ---------------------------------------------------------- Llama decoder

struct llambda_hip_llama_session {
  std::mutex run_mutex;
  int device = 0;
  hipStream_t stream = nullptr;
  DecoderPlan plan{};
  std::vector<DecoderLayer> layers;
  std::vector<std::unique_ptr<DevBuf>> weights;
  DevBuf norms, kv, state, rope_denom, rope_cs, x, q, ctx, h, att_part, att_max, att_sum, logits;
  int64_t layer_count = 0;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  float* graph_logits = nullptr;
  // recorded after every step on the stream it ran on: the next step (on
  // any stream), logits and sample wait for it, so steps that share the
  // session's state word, cache and logits never overlap
  hipEvent_t done = nullptr;
  ~llambda_hip_llama_session() {
    if (done) (void)hipEventDestroy(done);
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    if (stream) (void)hipStreamDestroy(stream);
  }
  DevBuf& new_weights() {
    weights.emplace_back(new DevBuf());
    return *weights.back();
  }
  float* kcache(int64_t l) const {
    return kv.as<float>() + (size_t)(2 * l) * plan.kv_heads * plan.context * plan.head_dim;
  }
  float* vcache(int64_t l) const { return kcache(l) + (size_t)plan.kv_heads * plan.context * plan.head_dim; }
};

namespace {

int64_t decoder_row_bytes(const llambda_hip_tensor_ref& t, int64_t rows, int64_t columns,
                          bool gemv, const char* what) {
  if (gemv && t.type != kQ4_K && t.type != kQ6_K)
    failf("%s: tensor type %s is not supported by the decoder (Q4_K or Q6_K)", what,
          type_name(t.type));
  if (!gemv && t.type != kQ4_K && t.type != kQ6_K && t.type != kQ5_0 && t.type != kQ8_0)
    failf("%s: tensor type %s is not supported for the token embedding", what, type_name(t.type));
  const int64_t rb = checked_row_bytes(t.type, columns, what);
  if (!t.data) failf("%s: null tensor data", what);
  if ((uint64_t)rows * (uint64_t)rb != t.bytes)
    failf("%s: %zu bytes do not hold %lld rows of %lld %s columns", what, t.bytes,
          (long long)rows, (long long)columns, type_name(t.type));
  return rb;
}

void validate_device(const DevBuf& b, int type, size_t bytes, hipStream_t s, const char* what) {
  DevBuf flag;
  flag.alloc(sizeof(unsigned long long), "validation flag");
  const unsigned long long none = ULLONG_MAX;
  HIPC(hipMemcpyAsync(flag.ptr, &none, sizeof none, hipMemcpyHostToDevice, s));
  HIPC(validate_launch(type, b.as<uint8_t>(), (int64_t)(bytes / block_bytes(type)),
                       flag.as<unsigned long long>(), s));
  unsigned long long first_bad = 0;
  HIPC(hipMemcpyAsync(&first_bad, flag.ptr, sizeof first_bad, hipMemcpyDeviceToHost, s));
  HIPC(hipStreamSynchronize(s));
  if (first_bad != ULLONG_MAX)
    failf("%s: Unsupported fp16 special value (Inf/NaN scale) in block %llu.", what, first_bad);
}

// Copy `parts` tensors (same type and columns) into one slab, rows of part i
// after those of part i - 1; with interleave8 (two parts) rows go in groups
// of 8: part 0 rows 8t..8t+7, then part 1 rows 8t..8t+7.
DecoderMatrix upload_slab(llambda_hip_llama_session* s, const llambda_hip_tensor_ref* parts,
                          const int64_t* rows, int n, int64_t columns, bool interleave8,
                          bool on_device, const char* what) {
  DecoderMatrix m;
  m.type = parts[0].type;
  m.columns = columns;
  int64_t total = 0;
  for (int i = 0; i < n; ++i) {
    if (parts[i].type != m.type) failf("%s: parts of one slab differ in type", what);
    m.row_bytes = decoder_row_bytes(parts[i], rows[i], columns, true, what);
    total += rows[i];
  }
  m.rows = total;
  const size_t bytes = (size_t)total * m.row_bytes;
  DevBuf& buf = s->new_weights();
  buf.alloc(bytes + kWeightPad, what);
  HIPC(hipMemsetAsync(buf.as<uint8_t>() + bytes, 0, kWeightPad, s->stream));
  const hipMemcpyKind kind = on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
  if (interleave8) {
    if (n != 2 || rows[0] != rows[1] || rows[0] % 8)
      failf("%s: gate and up need equal row counts divisible by 8", what);
    const size_t w = 8 * (size_t)m.row_bytes;
    for (int i = 0; i < 2; ++i)
      HIPC(hipMemcpy2DAsync(buf.as<uint8_t>() + i * w, 2 * w, parts[i].data, w, w,
                            (size_t)(rows[i] / 8), kind, s->stream));
  } else {
    size_t off = 0;
    for (int i = 0; i < n; ++i) {
      HIPC(hipMemcpyAsync(buf.as<uint8_t>() + off, parts[i].data, parts[i].bytes, kind, s->stream));
      off += parts[i].bytes;
    }
  }
  validate_device(buf, m.type, bytes, s->stream, what);
  m.w = buf.as<uint8_t>();
  return m;
}

}  // namespace

extern "C" {

int llambda_hip_llama_session_create(const llambda_hip_llama_desc* d,
                                     llambda_hip_llama_session** result) {
  return guarded([&] {
    if (!result) failf("llama session: null result pointer");
    *result = nullptr;
    if (!d) failf("llama session: null descriptor");
    const int64_t H = d->hidden, NH = d->head_count, NKV = d->kv_head_count;
    if (H <= 0 || NH <= 0 || NKV <= 0 || d->layer_count <= 0 || d->ffn <= 0 || d->vocab <= 0)
      failf("llama session: non-positive dimension");
    if (H % NH) failf("Llama hidden size %lld is not divisible by head count %lld.", (long long)H,
                      (long long)NH);
    if (NH % NKV)
      failf("Llama head count %lld is not divisible by KV head count %lld.", (long long)NH,
            (long long)NKV);
    const int64_t D = H / NH;
    if (!decoder_head_supported((int)D, (int)(NH / NKV)))
      failf("llama session: head size %lld with %lld query heads per kv head is not supported "
            "(head size 64 or 128, group 1, 2, 4 or 8)", (long long)D, (long long)(NH / NKV));
    if (d->context <= 0 || d->context > kDecoderMaxContext)
      failf("llama session: context %lld out of range (1..%d)", (long long)d->context,
            kDecoderMaxContext);
    if (d->ffn % 16) failf("llama session: ffn %lld must be a multiple of 16", (long long)d->ffn);
    if (!d->layers || !d->output_norm) failf("llama session: null layer list or output_norm");
    if (d->rope_factor_count < 0 || (d->rope_factor_count > 0 && !d->rope_factors))
      failf("llama session: bad rope factors");
    const bool dev = d->weights_on_device != 0;

    std::unique_ptr<llambda_hip_llama_session> s(new llambda_hip_llama_session());
    s->device = current_device_checked();
    HIPC(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking));
    HIPC(hipEventCreateWithFlags(&s->done, hipEventDisableTiming));
    HIPC(hipEventRecord(s->done, s->stream));
    DecoderPlan& p = s->plan;
    p.hidden = (int)H;
    p.heads = (int)NH;
    p.kv_heads = (int)NKV;
    p.head_dim = (int)D;
    p.ffn = (int)d->ffn;
    p.vocab = (int)d->vocab;
    p.context = (int)d->context;
    p.eps = d->norm_epsilon;
    // (coerce (/ (sqrt head-size)) 'single-float), llambda.lisp:6304
    p.q_scale = 1.f / sqrtf((float)D);
    s->layer_count = d->layer_count;

    // rotation: apply-rope-head-in-place (llambda.lisp:3760-3795)
    const int64_t factor_limit = d->rope_factor_count > 0 ? 2 * d->rope_factor_count
                                                          : d->rope_dimension;
    const int64_t eff = std::min(std::min(d->rope_dimension, factor_limit), D);
    const int64_t even = 2 * (eff / 2);
    p.rope_pairs = (int)(even / 2);
    std::vector<double> denom((size_t)std::max<int64_t>(p.rope_pairs, 1), 1.0);
    for (int64_t i = 0; i < p.rope_pairs; ++i) {
      const double factor = (d->rope_factors && i < d->rope_factor_count)
                                ? (double)d->rope_factors[i] : 1.0;
      // (expt theta-base (/ (* 2 i) even)): single-float base, rational
      // power -> single-float result
      const float power = (float)pow((double)d->rope_base, (double)(2 * i) / (double)even);
      denom[(size_t)i] = factor > 1.0e20 ? INFINITY : factor * (double)power;
    }

    // norms: attn and ffn per layer, then output
    const size_t nvec = (size_t)(2 * d->layer_count + 1);
    s->norms.alloc(nvec * (size_t)H * sizeof(float), "norm vectors");
    for (int64_t l = 0; l < d->layer_count; ++l) {
      const llambda_hip_llama_layer& L = d->layers[l];
      if (!L.attn_norm || !L.ffn_norm) failf("llama session: layer %lld: null norm vector", (long long)l);
      HIPC(hipMemcpyAsync(s->norms.as<float>() + (size_t)(2 * l) * H, L.attn_norm, H * sizeof(float),
                          hipMemcpyHostToDevice, s->stream));
      HIPC(hipMemcpyAsync(s->norms.as<float>() + (size_t)(2 * l + 1) * H, L.ffn_norm,
                          H * sizeof(float), hipMemcpyHostToDevice, s->stream));
    }
    HIPC(hipMemcpyAsync(s->norms.as<float>() + (nvec - 1) * H, d->output_norm, H * sizeof(float),
                        hipMemcpyHostToDevice, s->stream));
    p.output_norm = s->norms.as<float>() + (nvec - 1) * H;

    // KV cache, zeroed
    const size_t kv_floats = (size_t)d->layer_count * 2 * NKV * d->context * D;
    s->kv.alloc(kv_floats * sizeof(float), "KV cache");
    HIPC(hipMemsetAsync(s->kv.ptr, 0, kv_floats * sizeof(float), s->stream));

    // tensors
    {
      const int64_t rows[1] = {d->vocab};
      char what[64];
      snprintf(what, sizeof what, "token_embd");
      decoder_row_bytes(d->token_embd, d->vocab, H, false, what);
      DevBuf& buf = s->new_weights();
      buf.alloc(d->token_embd.bytes + kWeightPad, what);
      HIPC(hipMemsetAsync(buf.as<uint8_t>() + d->token_embd.bytes, 0, kWeightPad, s->stream));
      HIPC(hipMemcpyAsync(buf.ptr, d->token_embd.data, d->token_embd.bytes,
                          dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, s->stream));
      validate_device(buf, d->token_embd.type, d->token_embd.bytes, s->stream, what);
      p.embd.type = d->token_embd.type;
      p.embd.w = buf.as<uint8_t>();
      p.embd.row_bytes = checked_row_bytes(p.embd.type, H, what);
      p.embd.rows = d->vocab;
      p.embd.columns = H;
      p.output = upload_slab(s.get(), &d->output, rows, 1, H, false, dev, "output");
    }
    s->layers.resize((size_t)d->layer_count);
    for (int64_t l = 0; l < d->layer_count; ++l) {
      const llambda_hip_llama_layer& L = d->layers[l];
      DecoderLayer& o = s->layers[(size_t)l];
      char what[64];
      o.attn_norm = s->norms.as<float>() + (size_t)(2 * l) * H;
      o.ffn_norm = s->norms.as<float>() + (size_t)(2 * l + 1) * H;
      const int64_t qr = NH * D, kr = NKV * D;
      if (L.attn_q.type == L.attn_k.type) {
        const llambda_hip_tensor_ref parts[2] = {L.attn_q, L.attn_k};
        const int64_t rows[2] = {qr, kr};
        snprintf(what, sizeof what, "blk.%lld.attn_q|attn_k", (long long)l);
        o.qk = upload_slab(s.get(), parts, rows, 2, H, false, dev, what);
      } else {
        snprintf(what, sizeof what, "blk.%lld.attn_q", (long long)l);
        o.q = upload_slab(s.get(), &L.attn_q, &qr, 1, H, false, dev, what);
        snprintf(what, sizeof what, "blk.%lld.attn_k", (long long)l);
        o.k = upload_slab(s.get(), &L.attn_k, &kr, 1, H, false, dev, what);
      }
      snprintf(what, sizeof what, "blk.%lld.attn_v", (long long)l);
      o.v = upload_slab(s.get(), &L.attn_v, &kr, 1, H, false, dev, what);
      snprintf(what, sizeof what, "blk.%lld.attn_output", (long long)l);
      o.o = upload_slab(s.get(), &L.attn_output, &H, 1, qr, false, dev, what);
      {
        const llambda_hip_tensor_ref parts[2] = {L.ffn_gate, L.ffn_up};
        const int64_t rows[2] = {d->ffn, d->ffn};
        snprintf(what, sizeof what, "blk.%lld.ffn_gate|ffn_up", (long long)l);
        o.gate_up = upload_slab(s.get(), parts, rows, 2, H, true, dev, what);
      }
      snprintf(what, sizeof what, "blk.%lld.ffn_down", (long long)l);
      o.down = upload_slab(s.get(), &L.ffn_down, &H, 1, d->ffn, false, dev, what);
      o.kcache = s->kcache(l);
      o.vcache = s->vcache(l);
    }
    p.layers = s->layers.data();
    p.layer_count = (int)d->layer_count;

    // scratch
    p.att_chunks = (p.context + kAttnChunk - 1) / kAttnChunk;
    s->state.alloc(2 * sizeof(int), "decoder state");
    s->rope_denom.alloc(denom.size() * sizeof(double), "rope denominators");
    HIPC(hipMemcpyAsync(s->rope_denom.ptr, denom.data(), denom.size() * sizeof(double),
                        hipMemcpyHostToDevice, s->stream));
    s->rope_cs.alloc(denom.size() * 2 * sizeof(double), "rope table");
    s->x.alloc((size_t)H * sizeof(float), "hidden state");
    s->q.alloc((size_t)NH * D * sizeof(float), "queries");
    s->ctx.alloc((size_t)NH * D * sizeof(float), "attention context");
    s->h.alloc((size_t)d->ffn * sizeof(float), "ffn activations");
    s->att_part.alloc((size_t)NH * p.att_chunks * D * sizeof(float), "attention partial sums");
    s->att_max.alloc((size_t)NH * p.att_chunks * sizeof(float), "attention chunk maxima");
    s->att_sum.alloc((size_t)NH * p.att_chunks * sizeof(float), "attention chunk sums");
    s->logits.alloc((size_t)d->vocab * sizeof(float), "logits");
    p.state = s->state.as<int>();
    p.rope_denom = s->rope_denom.as<double>();
    p.rope_cs = s->rope_cs.as<double>();
    p.x = s->x.as<float>();
    p.q = s->q.as<float>();
    p.ctx = s->ctx.as<float>();
    p.h = s->h.as<float>();
    p.att_part = s->att_part.as<float>();
    p.att_max = s->att_max.as<float>();
    p.att_sum = s->att_sum.as<float>();
    HIPC(hipStreamSynchronize(s->stream));
    *result = s.release();
  });
}

void llambda_hip_llama_session_destroy(llambda_hip_llama_session* session) { delete session; }

size_t llambda_hip_llama_session_vocab(const llambda_hip_llama_session* session) {
  return session ? (size_t)session->plan.vocab : 0;
}

static void check_token(const llambda_hip_llama_session* s, int64_t token, int64_t position) {
  if (token < 0 || token >= s->plan.vocab)
    failf("token id %lld out of range (vocab %d)", (long long)token, s->plan.vocab);
  if (position < 0 || position >= s->plan.context)
    failf("position %lld outside the KV cache (context %d)", (long long)position, s->plan.context);
}

int llambda_hip_llama_session_step(llambda_hip_llama_session* s, int64_t token, int64_t position,
                                   float* logits, size_t logits_count) {
  return guarded([&] {
    if (!s) failf("llama step: null session");
    if (!logits || logits_count != (size_t)s->plan.vocab)
      failf("llama step: logits count %zu does not match vocab %d", logits_count, s->plan.vocab);
    check_token(s, token, position);
    std::lock_guard<std::mutex> lock(s->run_mutex);
    HIPC(hipSetDevice(s->device));
    HIPC(hipStreamWaitEvent(s->stream, s->done, 0));
    HIPC(decoder_state_launch(s->plan, (int)token, (int)position, s->stream));
    HIPC(decoder_step_launch(s->plan, s->logits.as<float>(), s->stream));
    HIPC(hipMemcpyAsync(logits, s->logits.ptr, logits_count * sizeof(float), hipMemcpyDeviceToHost,
                        s->stream));
    HIPC(hipEventRecord(s->done, s->stream));
    HIPC(hipStreamSynchronize(s->stream));
  });
}

int llambda_hip_llama_session_step_device(llambda_hip_llama_session* s, int64_t token,
                                          int64_t position, float* logits, void* stream,
                                          int use_graph) {
  return guarded([&] {
    if (!s) failf("llama step: null session");
    check_token(s, token, position);
    std::lock_guard<std::mutex> lock(s->run_mutex);
    HIPC(hipSetDevice(s->device));
    hipStream_t st = stream ? static_cast<hipStream_t>(stream) : s->stream;
    if (!logits) logits = s->logits.as<float>();
    if (use_graph && (!s->exec || s->graph_logits != logits)) {
      if (s->exec) HIPC(hipGraphExecDestroy(s->exec));
      if (s->graph) HIPC(hipGraphDestroy(s->graph));
      s->exec = nullptr;
      s->graph = nullptr;
      // capture on the session's own stream, after whatever `st` holds and
      // the previous step
      HIPC(hipStreamSynchronize(st));
      HIPC(hipEventSynchronize(s->done));
      HIPC(hipStreamBeginCapture(s->stream, hipStreamCaptureModeRelaxed));
      const hipError_t e = decoder_step_launch(s->plan, logits, s->stream);
      hipGraph_t g = nullptr;
      const hipError_t e2 = hipStreamEndCapture(s->stream, &g);
      HIPC(e);
      HIPC(e2);
      s->graph = g;
      HIPC(hipGraphInstantiate(&s->exec, s->graph, nullptr, nullptr, 0));
      s->graph_logits = logits;
    }
    HIPC(hipStreamWaitEvent(st, s->done, 0));
    HIPC(decoder_state_launch(s->plan, (int)token, (int)position, st));
    if (use_graph) HIPC(hipGraphLaunch(s->exec, st));
    else HIPC(decoder_step_launch(s->plan, logits, st));
    HIPC(hipEventRecord(s->done, st));
  });
}

int llambda_hip_llama_session_logits(llambda_hip_llama_session* s, float* logits,
                                     size_t logits_count) {
  return guarded([&] {
    if (!s || !logits) failf("llama logits: null argument");
    if (logits_count != (size_t)s->plan.vocab)
      failf("llama logits: count %zu does not match vocab %d", logits_count, s->plan.vocab);
    std::lock_guard<std::mutex> lock(s->run_mutex);
    HIPC(hipSetDevice(s->device));
    // the last step may have run on a caller's stream
    HIPC(hipStreamWaitEvent(s->stream, s->done, 0));
    HIPC(hipMemcpyAsync(logits, s->logits.ptr, logits_count * sizeof(float), hipMemcpyDeviceToHost,
                        s->stream));
    HIPC(hipStreamSynchronize(s->stream));
  });
}

int llambda_hip_llama_session_write_kv(llambda_hip_llama_session* s, int64_t layer, int64_t first,
                                       int64_t count, const float* keys, const float* values,
                                       int on_device) {
  return guarded([&] {
    if (!s || !keys || !values) failf("write_kv: null argument");
    if (layer < 0 || layer >= s->layer_count) failf("write_kv: layer %lld out of range", (long long)layer);
    if (first < 0 || count < 0 || first + count > s->plan.context)
      failf("write_kv: slots [%lld, %lld) outside the context %d", (long long)first,
            (long long)(first + count), s->plan.context);
    if (count == 0) return;
    std::lock_guard<std::mutex> lock(s->run_mutex);
    HIPC(hipSetDevice(s->device));
    HIPC(hipStreamWaitEvent(s->stream, s->done, 0));
    const size_t D = (size_t)s->plan.head_dim, C = (size_t)s->plan.context;
    const hipMemcpyKind kind = on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
    const size_t w = (size_t)count * D * sizeof(float);
    HIPC(hipMemcpy2DAsync(s->kcache(layer) + first * D, C * D * sizeof(float), keys, w, w,
                          (size_t)s->plan.kv_heads, kind, s->stream));
    HIPC(hipMemcpy2DAsync(s->vcache(layer) + first * D, C * D * sizeof(float), values, w, w,
                          (size_t)s->plan.kv_heads, kind, s->stream));
    HIPC(hipStreamSynchronize(s->stream));
  });
}

int llambda_hip_llama_session_read_kv(llambda_hip_llama_session* s, int64_t layer, int64_t first,
                                      int64_t count, float* keys, float* values) {
  return guarded([&] {
    if (!s || !keys || !values) failf("read_kv: null argument");
    if (layer < 0 || layer >= s->layer_count) failf("read_kv: layer %lld out of range", (long long)layer);
    if (first < 0 || count < 0 || first + count > s->plan.context)
      failf("read_kv: slots [%lld, %lld) outside the context %d", (long long)first,
            (long long)(first + count), s->plan.context);
    if (count == 0) return;
    std::lock_guard<std::mutex> lock(s->run_mutex);
    HIPC(hipSetDevice(s->device));
    HIPC(hipStreamWaitEvent(s->stream, s->done, 0));
    const size_t D = (size_t)s->plan.head_dim, C = (size_t)s->plan.context;
    const size_t w = (size_t)count * D * sizeof(float);
    HIPC(hipMemcpy2DAsync(keys, w, s->kcache(layer) + first * D, C * D * sizeof(float), w,
                          (size_t)s->plan.kv_heads, hipMemcpyDeviceToHost, s->stream));
    HIPC(hipMemcpy2DAsync(values, w, s->vcache(layer) + first * D, C * D * sizeof(float), w,
                          (size_t)s->plan.kv_heads, hipMemcpyDeviceToHost, s->stream));
    HIPC(hipStreamSynchronize(s->stream));
  });
}

int llambda_hip_llama_session_sync(llambda_hip_llama_session* s, void* stream) {
  return guarded([&] {
    if (!s) failf("llama sync: null session");
    HIPC(hipStreamSynchronize(stream ? static_cast<hipStream_t>(stream) : s->stream));
    HIPC(hipEventSynchronize(s->done));
  });
}

}  // extern "C"

// ---------------------------------------------------------------- sampling

struct llambda_hip_sampler {
  std::mutex run_mutex;
  int device = 0;
  hipStream_t stream = nullptr;
  int64_t vocab = 0;
  DevBuf work, logits, history;
  size_t history_cap = 0;
  // pinned host staging of long histories (a small copy without a pageable
  // bounce) and the mapped result the kernel writes
  int* host_history = nullptr;
  int* host_result = nullptr;
  int* dev_result = nullptr;  // host_result as the device addresses it
  ~llambda_hip_sampler() {
    if (host_history) (void)hipHostFree(host_history);
    if (host_result) (void)hipHostFree(host_result);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

namespace {

// Validate the arguments as sample-token-id-from-logits does and enqueue the
// sampling kernel on the sampler's stream; returns the token.
int64_t run_sampler(llambda_hip_sampler* s, const float* dev_logits, int64_t n,
                    const llambda_hip_sampling* a) {
  if (!a) failf("sample: null parameters");
  if (n <= 0 || n > s->vocab) failf("sample: %lld logits do not fit the sampler (vocab %lld)",
                                    (long long)n, (long long)s->vocab);
  if (!(a->random_value >= 0.0f && a->random_value < 1.0f))
    failf("RANDOM-VALUE must satisfy 0.0 <= value < 1.0, got %g.", (double)a->random_value);
  if (a->top_k < 0) failf("TOP-K must be a nonnegative fixnum or NIL, got %lld.", (long long)a->top_k);
  if (!(a->top_p > 0.0f && a->top_p <= 1.0f))
    failf("TOP-P must satisfy 0.0 < p <= 1.0, got %g.", (double)a->top_p);
  if (!(a->temperature > 0.0f)) failf("TEMPERATURE must be positive, got %g.", (double)a->temperature);
  if (a->temperature > 1.0e20f)
    failf("sample: temperature %g is outside the device path (masked logits must underflow)",
          (double)a->temperature);
  // distinct history tokens, checked in the reference's order
  std::vector<int> distinct;
  if (a->history_count > 0) {
    if (!a->history) failf("sample: null history");
    if (!(a->repetition_penalty > 0.0f))
      failf("PENALTY must be positive, got %g.", (double)a->repetition_penalty);
    std::vector<int64_t> seen;
    for (size_t i = 0; i < a->history_count; ++i) {
      const int64_t t = a->history[i];
      bool dup = false;
      for (int64_t u : seen)
        if (u == t) {
          dup = true;
          break;
        }
      if (dup) continue;
      if (t < 0 || t >= n)
        failf("History token id %lld is out of bounds for logits length %lld.", (long long)t,
              (long long)n);
      seen.push_back(t);
      distinct.push_back((int)t);
    }
  }
  const bool topk = a->top_k > 0 && a->top_k < n;
  if (topk && a->top_k > kSampleMaxSurvivors)
    failf("sample: top-k %lld above %d is not supported on the device", (long long)a->top_k,
          kSampleMaxSurvivors);
  const bool inline_history = distinct.size() <= (size_t)kSampleInlineHistory;
  if (!inline_history && distinct.size() > s->history_cap) {
    const size_t cap = std::max<size_t>(distinct.size(), 2 * s->history_cap);
    s->history.alloc(cap * sizeof(int), "sampling history");
    if (s->host_history) HIPC(hipHostFree(s->host_history));
    s->host_history = nullptr;
    HIPC(hipHostMalloc((void**)&s->host_history, cap * sizeof(int), hipHostMallocDefault));
    s->history_cap = cap;
  }
  SampleParams p;
  p.n = (int)n;
  p.nh = (int)distinct.size();
  if (inline_history) {
    p.history = nullptr;
    std::copy(distinct.begin(), distinct.end(), p.hist_inline);
  } else {
    std::copy(distinct.begin(), distinct.end(), s->host_history);
    HIPC(hipMemcpyAsync(s->history.ptr, s->host_history, distinct.size() * sizeof(int),
                        hipMemcpyHostToDevice, s->stream));
    p.history = s->history.as<int>();
  }
  p.penalty = a->repetition_penalty;
  p.top_k = (int)std::min<int64_t>(a->top_k, n);
  p.top_p = a->top_p;
  p.temperature = a->temperature;
  p.roll = a->random_value;
  int* res = s->host_result;
  res[0] = -1;
  res[1] = -1;
  HIPC(sample_launch(dev_logits, s->work.as<float>(), p, s->dev_result, s->stream));
  HIPC(hipStreamSynchronize(s->stream));
  if (res[1] == kSampleErrNaN) failf("sample: NaN logit");
  if (res[1] == kSampleErrTies)
    failf("sample: more than %d logits tie at or above the top-k cutoff", kSampleMaxSurvivors);
  if (res[1] != 0 || res[0] < 0) failf("sample: device error %d", res[1]);
  return res[0];
}

}  // namespace

extern "C" {

int llambda_hip_sampler_create(size_t vocab, llambda_hip_sampler** result) {
  return guarded([&] {
    if (!result) failf("sampler: null result pointer");
    *result = nullptr;
    if (vocab == 0 || vocab > (size_t)kSampleMaxVocab)
      failf("sampler: vocab %zu out of range (1..%d)", vocab, kSampleMaxVocab);
    std::unique_ptr<llambda_hip_sampler> s(new llambda_hip_sampler());
    s->device = current_device_checked();
    s->vocab = (int64_t)vocab;
    HIPC(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking));
    s->work.alloc(sample_work_floats((int)vocab) * sizeof(float), "sampling row");
    s->logits.alloc(vocab * sizeof(float), "sampling input");
    // the result lands in mapped, coherent pinned memory: the kernel writes
    // it there and no copy follows the launches
    HIPC(hipHostMalloc((void**)&s->host_result, 2 * sizeof(int),
                       hipHostMallocMapped | hipHostMallocCoherent));
    HIPC(hipHostGetDevicePointer((void**)&s->dev_result, s->host_result, 0));
    *result = s.release();
  });
}

void llambda_hip_sampler_destroy(llambda_hip_sampler* sampler) { delete sampler; }

int llambda_hip_sampler_sample(llambda_hip_sampler* s, const float* logits, size_t count,
                               int logits_on_device, const llambda_hip_sampling* params,
                               int64_t* token) {
  return guarded([&] {
    if (!s || !logits || !token) failf("sample: null argument");
    std::lock_guard<std::mutex> lock(s->run_mutex);
    HIPC(hipSetDevice(s->device));
    if (count == 0 || count > (size_t)s->vocab)
      failf("sample: %zu logits do not fit the sampler (vocab %lld)", count, (long long)s->vocab);
    const float* dev = logits;
    if (logits_on_device && (reinterpret_cast<uintptr_t>(logits) & 15u))
      failf("sample: device logits must be 16-byte aligned");
    if (!logits_on_device) {
      HIPC(hipMemcpyAsync(s->logits.ptr, logits, count * sizeof(float), hipMemcpyHostToDevice,
                          s->stream));
      dev = s->logits.as<float>();
    }
    *token = run_sampler(s, dev, (int64_t)count, params);
  });
}

int llambda_hip_llama_session_sample(llambda_hip_llama_session* session,
                                     llambda_hip_sampler* s, const llambda_hip_sampling* params,
                                     int64_t* token) {
  return guarded([&] {
    if (!session || !s || !token) failf("sample: null argument");
    std::lock_guard<std::mutex> lock(s->run_mutex);
    HIPC(hipSetDevice(s->device));
    // the last step wrote the logits, on whichever stream it was given
    {
      std::lock_guard<std::mutex> slock(session->run_mutex);
      HIPC(hipEventSynchronize(session->done));
    }
    *token = run_sampler(s, session->logits.as<float>(), session->plan.vocab, params);
  });
}

}  // extern "C"

// -------------------------------------------------------------------- GGUF

struct llambda_hip_gguf {
  std::unique_ptr<GgufFile> file;
};

static void fill_value(const GgufValue& v, llambda_hip_gguf_value* out) {
  out->type = v.type;
  out->element_type = v.elem_type;
  out->count = v.type == 9 ? v.items.size() : 0;
  out->u = v.u;
  out->i = v.i;
  out->f = v.f;
  out->string = v.str;
  out->string_length = v.str_len;
}

extern "C" {

int llambda_hip_gguf_open(const char* path, llambda_hip_gguf** result) {
  return guarded([&] {
    if (!result) failf("gguf: null result pointer");
    *result = nullptr;
    std::unique_ptr<llambda_hip_gguf> g(new llambda_hip_gguf());
    g->file.reset(gguf_open(path));
    *result = g.release();
  });
}

void llambda_hip_gguf_close(llambda_hip_gguf* file) { delete file; }

int llambda_hip_gguf_header(const llambda_hip_gguf* g, uint32_t* version, uint64_t* tensor_count,
                            uint64_t* kv_count, uint64_t* alignment, uint64_t* data_start) {
  return guarded([&] {
    if (!g) failf("gguf: null file");
    if (version) *version = g->file->version;
    if (tensor_count) *tensor_count = g->file->tensor_count;
    if (kv_count) *kv_count = g->file->kv_count;
    if (alignment) *alignment = g->file->alignment;
    if (data_start) *data_start = g->file->data_start;
  });
}

const void* llambda_hip_gguf_mapping(const llambda_hip_gguf* g, size_t* size) {
  if (!g) return nullptr;
  if (size) *size = (size_t)g->file->size;
  return g->file->base;
}

int llambda_hip_gguf_tensor_info(const llambda_hip_gguf* g, uint64_t index,
                                 llambda_hip_gguf_tensor* out) {
  return guarded([&] {
    if (!g || !out) failf("gguf: null argument");
    if (index >= g->file->tensors.size()) failf("gguf: tensor index %llu out of range", (unsigned long long)index);
    const GgufTensor& t = g->file->tensors[index];
    out->name = t.name;
    out->name_length = (size_t)t.name_len;
    out->dimension_count = t.dimension_count;
    for (int d = 0; d < 4; ++d) out->dimensions[d] = t.dimensions[d];
    out->type = t.type;
    out->offset = t.offset;
    out->element_count = t.element_count;
    out->supported = t.supported;
    out->byte_size = t.byte_size;
    out->data_offset = t.data_offset;
    out->data = g->file->base + t.data_offset;
  });
}

int64_t llambda_hip_gguf_find_tensor(const llambda_hip_gguf* g, const char* name) {
  if (!g || !name) return -1;
  const size_t n = strlen(name);
  for (size_t i = 0; i < g->file->tensors.size(); ++i) {
    const GgufTensor& t = g->file->tensors[i];
    if (t.name_len == n && memcmp(t.name, name, n) == 0) return (int64_t)i;
  }
  return -1;
}

int llambda_hip_gguf_kv(const llambda_hip_gguf* g, uint64_t index, llambda_hip_gguf_value* out) {
  return guarded([&] {
    if (!g || !out) failf("gguf: null argument");
    if (index >= g->file->kv.size()) failf("gguf: metadata index %llu out of range", (unsigned long long)index);
    const GgufKv& kv = g->file->kv[index];
    fill_value(kv.value, out);
    out->key = kv.key;
    out->key_length = (size_t)kv.key_len;
  });
}

int llambda_hip_gguf_kv_element(const llambda_hip_gguf* g, uint64_t index, uint64_t element,
                                llambda_hip_gguf_value* out) {
  return guarded([&] {
    if (!g || !out) failf("gguf: null argument");
    if (index >= g->file->kv.size()) failf("gguf: metadata index %llu out of range", (unsigned long long)index);
    const GgufValue& v = g->file->kv[index].value;
    if (v.type != 9 || element >= v.items.size())
      failf("gguf: metadata %llu has no element %llu", (unsigned long long)index, (unsigned long long)element);
    fill_value(v.items[element], out);
    out->key = nullptr;
    out->key_length = 0;
  });
}

}  // extern "C"
