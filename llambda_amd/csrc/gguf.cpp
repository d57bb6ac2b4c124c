// gguf.cpp -- the bounded GGUF parser over open/mmap (gguf.h).
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>

namespace llhip {

namespace {

[[noreturn]] void gguf_fail(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  throw std::runtime_error(buf);
}

// ensure-mapped-range (llambda.lisp:561-574)
void ensure_range(const GgufFile& f, uint64_t offset, uint64_t length, const char* what) {
  if (!(offset <= f.size && length <= f.size - offset))
    gguf_fail("%s byte range [%llu, %llu) exceeds mapped file length %llu.", what,
              (unsigned long long)offset, (unsigned long long)(offset + length),
              (unsigned long long)f.size);
}

uint32_t read_u32(const GgufFile& f, uint64_t off, const char* what) {
  ensure_range(f, off, 4, what);
  uint32_t v;
  memcpy(&v, f.base + off, 4);
  return v;
}

uint64_t read_u64(const GgufFile& f, uint64_t off, const char* what) {
  ensure_range(f, off, 8, what);
  uint64_t v;
  memcpy(&v, f.base + off, 8);
  return v;
}

// gguf-value-minimum-byte-size (llambda.lisp:1954-1962)
uint64_t value_min_size(uint32_t type) {
  switch (type) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 8: case 10: case 11: case 12: return 8;
    case 9: return 12;
    default: gguf_fail("Unsupported GGUF metadata value type: %u.", type);
  }
}

// ensure-gguf-count-fits (llambda.lisp:1964-1975)
void ensure_count_fits(const GgufFile& f, uint64_t offset, uint64_t count, uint64_t min_size,
                       const char* what) {
  const uint64_t remaining = offset <= f.size ? f.size - offset : 0;
  if (offset > f.size || count > remaining / min_size)
    gguf_fail("%s count %llu cannot fit in the %llu mapped bytes remaining.", what,
              (unsigned long long)count, (unsigned long long)remaining);
}

// read-gguf-string (llambda.lisp:1977-1983)
uint64_t read_string(const GgufFile& f, uint64_t off, const char** s, uint64_t* len) {
  const uint64_t n = read_u64(f, off, "GGUF string length");
  ensure_range(f, off + 8, n, "GGUF string");
  *s = reinterpret_cast<const char*>(f.base + off + 8);
  *len = n;
  return off + 8 + n;
}

// read-gguf-value (llambda.lisp:1985-2045)
uint64_t read_value(const GgufFile& f, uint64_t off, uint32_t type, GgufValue& v) {
  v.type = type;
  switch (type) {
    case 0:
      ensure_range(f, off, 1, "GGUF uint8 metadata value");
      v.u = f.base[off];
      v.i = (int64_t)v.u;
      return off + 1;
    case 1:
      ensure_range(f, off, 1, "GGUF int8 metadata value");
      v.i = (int8_t)f.base[off];
      return off + 1;
    case 2: {
      ensure_range(f, off, 2, "GGUF uint16 metadata value");
      uint16_t t;
      memcpy(&t, f.base + off, 2);
      v.u = t;
      v.i = t;
      return off + 2;
    }
    case 3: {
      ensure_range(f, off, 2, "GGUF int16 metadata value");
      int16_t t;
      memcpy(&t, f.base + off, 2);
      v.i = t;
      return off + 2;
    }
    case 4:
      v.u = read_u32(f, off, "GGUF uint32 metadata value");
      v.i = (int64_t)v.u;
      return off + 4;
    case 5:
      v.i = (int32_t)read_u32(f, off, "GGUF int32 metadata value");
      return off + 4;
    case 6: {
      ensure_range(f, off, 4, "GGUF float32 metadata value");
      float t;
      memcpy(&t, f.base + off, 4);
      v.f = t;
      return off + 4;
    }
    case 7:
      ensure_range(f, off, 1, "GGUF boolean metadata value");
      v.u = f.base[off] != 0;
      v.i = (int64_t)v.u;
      return off + 1;
    case 8:
      return read_string(f, off, &v.str, &v.str_len);
    case 9: {
      v.elem_type = read_u32(f, off, "GGUF metadata array element type");
      const uint64_t n = read_u64(f, off + 4, "GGUF metadata array length");
      uint64_t cur = off + 12;
      if (v.elem_type == 9) gguf_fail("Nested GGUF metadata arrays are unsupported.");
      ensure_count_fits(f, cur, n, value_min_size(v.elem_type), "GGUF metadata array");
      v.items.resize(n);
      for (uint64_t j = 0; j < n; ++j) cur = read_value(f, cur, v.elem_type, v.items[j]);
      return cur;
    }
    case 10:
      v.u = read_u64(f, off, "GGUF uint64 metadata value");
      v.i = (int64_t)v.u;
      return off + 8;
    case 11:
      v.i = (int64_t)read_u64(f, off, "GGUF int64 metadata value");
      return off + 8;
    case 12: {
      ensure_range(f, off, 8, "GGUF float64 metadata value");
      memcpy(&v.f, f.base + off, 8);
      return off + 8;
    }
    default:
      gguf_fail("Unsupported GGUF metadata value type: %u.", type);
  }
}

// supported-ggml-type-p, ggml-type-block-size, ggml-type-size
// (llambda.lisp:2097-2145)
bool type_supported(uint32_t t) {
  return t == 0 || t == 1 || t == 6 || t == 8 || t == 30 || t == 12 || t == 13 || t == 14;
}
uint64_t type_block(uint32_t t) {
  return (t == 0 || t == 1 || t == 30) ? 1 : (t == 6 || t == 8) ? 32 : 256;
}
uint64_t type_size(uint32_t t) {
  switch (t) {
    case 0: return 4;
    case 1: case 30: return 2;
    case 6: return 2 + 4 + 16;
    case 8: return 2 + 32;
    case 12: return 4 + 12 + 128;
    case 13: return 4 + 12 + 32 + 128;
    default: return 2 + 16 + 192;  // 14
  }
}
const char* type_name(uint32_t t) {
  switch (t) {
    case 0: return "F32";
    case 1: return "F16";
    case 6: return "Q5_0";
    case 8: return "Q8_0";
    case 30: return "BF16";
    case 12: return "Q4_K";
    case 13: return "Q5_K";
    case 14: return "Q6_K";
    default: return "?";
  }
}

}  // namespace

GgufFile::~GgufFile() {
  if (base && size) munmap(const_cast<uint8_t*>(base), size);
  if (fd >= 0) close(fd);
}

GgufFile* gguf_open(const char* path) {
  if (!path) gguf_fail("GGUF path is null.");
  std::unique_ptr<GgufFile> f(new GgufFile());
  f->fd = open(path, O_RDONLY | O_CLOEXEC);
  if (f->fd < 0) gguf_fail("Cannot open %s: %s.", path, strerror(errno));
  struct stat st;
  if (fstat(f->fd, &st) != 0) gguf_fail("Cannot stat %s: %s.", path, strerror(errno));
  f->size = (uint64_t)st.st_size;
  if (f->size > 0) {
    void* m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
    if (m == MAP_FAILED) gguf_fail("Cannot map %s: %s.", path, strerror(errno));
    f->base = static_cast<const uint8_t*>(m);
  }

  // read-gguf-header (llambda.lisp:2047-2059)
  ensure_range(*f, 0, 4, "GGUF magic");
  if (memcmp(f->base, "GGUF", 4) != 0)
    gguf_fail("Invalid GGUF magic: \"%c%c%c%c\".", f->base[0], f->base[1], f->base[2], f->base[3]);
  f->version = read_u32(*f, 4, "GGUF version");
  f->tensor_count = read_u64(*f, 8, "GGUF tensor count");
  f->kv_count = read_u64(*f, 16, "GGUF metadata count");

  // read-gguf-metadata-section (llambda.lisp:2061-2082)
  uint64_t cur = 24;
  ensure_count_fits(*f, cur, f->kv_count, 13, "GGUF metadata");
  f->kv.resize(f->kv_count);
  for (uint64_t k = 0; k < f->kv_count; ++k) {
    GgufKv& kv = f->kv[k];
    const uint64_t key_end = read_string(*f, cur, &kv.key, &kv.key_len);
    const uint32_t type = read_u32(*f, key_end, "GGUF metadata value type");
    cur = read_value(*f, key_end + 4, type, kv.value);
  }

  // gguf-alignment (llambda.lisp:2090-2100)
  for (const GgufKv& kv : f->kv) {
    if (kv.key_len == 17 && memcmp(kv.key, "general.alignment", 17) == 0) {
      const GgufValue& v = kv.value;
      const bool integer = v.type <= 5 || v.type == 10 || v.type == 11;
      const int64_t a = v.i;
      if (!integer || a <= 0 || (a & (a - 1)) != 0)
        gguf_fail("GGUF alignment must be a positive power of two, got %lld.", (long long)a);
      f->alignment = (uint64_t)a;
    }
  }

  // read-gguf-tensor-infos (llambda.lisp:2147-2238)
  ensure_count_fits(*f, cur, f->tensor_count, 24, "GGUF tensor info");
  f->tensors.resize(f->tensor_count);
  for (uint64_t t = 0; t < f->tensor_count; ++t) {
    GgufTensor& ti = f->tensors[t];
    const uint64_t name_end = read_string(*f, cur, &ti.name, &ti.name_len);
    ti.dimension_count = read_u32(*f, name_end, "GGUF tensor dimension count");
    const uint64_t dc = name_end + 4;
    if (ti.dimension_count < 1 || ti.dimension_count > 4)
      gguf_fail("Tensor \"%.*s\" has invalid dimension count %u; GGUF permits 1 through 4.",
                (int)ti.name_len, ti.name, ti.dimension_count);
    ensure_range(*f, dc, ti.dimension_count * 8 + 12, "GGUF tensor dimensions, type, and offset");
    uint64_t elements = 1;
    bool positive = true, overflow = false;
    for (uint32_t d = 0; d < ti.dimension_count; ++d) {
      ti.dimensions[d] = read_u64(*f, dc + 8 * d, "GGUF tensor dimension");
      if (ti.dimensions[d] == 0) positive = false;
      else if (elements > UINT64_MAX / ti.dimensions[d]) overflow = true;
      else elements *= ti.dimensions[d];
    }
    const uint64_t tc = dc + 8 * ti.dimension_count;
    ti.type = read_u32(*f, tc, "GGUF tensor type");
    ti.offset = read_u64(*f, tc + 4, "GGUF tensor offset");
    cur = tc + 12;
    if (overflow) gguf_fail("Tensor \"%.*s\" element count overflows.", (int)ti.name_len, ti.name);
    ti.element_count = elements;
    ti.supported = type_supported(ti.type);
    if (ti.supported) {
      const uint64_t bs = type_block(ti.type);
      if (elements % bs)
        gguf_fail("Tensor element count %llu is not a multiple of block size %llu for type %s.",
                  (unsigned long long)elements, (unsigned long long)bs, type_name(ti.type));
      ti.byte_size = elements / bs * type_size(ti.type);
    }
    if (!positive) {
      char dims[128];
      int o = snprintf(dims, sizeof dims, "(");
      for (uint32_t d = 0; d < ti.dimension_count; ++d)
        o += snprintf(dims + o, sizeof dims - o, d ? " %llu" : "%llu",
                      (unsigned long long)ti.dimensions[d]);
      snprintf(dims + o, sizeof dims - o, ")");
      gguf_fail("Tensor \"%.*s\" has non-positive dimensions %s.", (int)ti.name_len, ti.name, dims);
    }
  }
  // align-offset (llambda.lisp:2087-2088)
  f->data_start = (cur + f->alignment - 1) / f->alignment * f->alignment;
  if (f->tensor_count) ensure_range(*f, f->data_start, 0, "GGUF tensor data start");
  for (GgufTensor& ti : f->tensors) {
    if (ti.offset > UINT64_MAX - f->data_start) gguf_fail("GGUF tensor offset overflows.");
    ti.data_offset = f->data_start + ti.offset;
    char what[160];
    snprintf(what, sizeof what, "GGUF tensor \"%.*s\"", (int)ti.name_len, ti.name);
    ensure_range(*f, ti.data_offset, ti.byte_size, what);
  }
  return f.release();
}

}  // namespace llhip
