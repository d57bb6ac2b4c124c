// gguf.h -- GGUF v3 files over open/mmap with a bounded parser (gguf.cpp).
//
// The reference maps the file with CreateFileMapping / MapViewOfFile
// (llambda.lisp:489-675) and parses it with read-gguf-header,
// read-gguf-metadata-section and read-gguf-tensor-infos
// (llambda.lisp:1937-2238); every read is checked against the mapped length
// (ensure-mapped-range, llambda.lisp:561-574) and every count against the
// bytes left (ensure-gguf-count-fits).  This is the same parser on POSIX
// open/fstat/mmap, with the reference's error texts.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace llhip {

struct GgufValue {
  uint32_t type = 0;          // GGUF value type 0..12
  uint64_t u = 0;             // unsigned integers, bool (0 / 1)
  int64_t i = 0;              // signed integers (and unsigned, when they fit)
  double f = 0.0;             // float32 / float64
  const char* str = nullptr;  // strings: bytes in the mapping
  uint64_t str_len = 0;
  uint32_t elem_type = 0;     // arrays
  std::vector<GgufValue> items;
};

struct GgufKv {
  const char* key = nullptr;  // bytes in the mapping
  uint64_t key_len = 0;
  GgufValue value;
};

struct GgufTensor {
  const char* name = nullptr;
  uint64_t name_len = 0;
  uint32_t dimension_count = 0;
  uint64_t dimensions[4] = {0, 0, 0, 0};
  uint32_t type = 0;
  uint64_t offset = 0;         // relative to the tensor data start
  uint64_t element_count = 0;
  bool supported = false;      // the reference's supported-ggml-type-p
  uint64_t byte_size = 0;      // 0 when unsupported (the reference's NIL)
  uint64_t data_offset = 0;    // absolute in the file
};

struct GgufFile {
  int fd = -1;
  const uint8_t* base = nullptr;
  uint64_t size = 0;
  uint32_t version = 0;
  uint64_t tensor_count = 0, kv_count = 0;
  std::vector<GgufKv> kv;
  std::vector<GgufTensor> tensors;
  uint64_t alignment = 32;
  uint64_t data_start = 0;
  ~GgufFile();
};

// Open, map and parse; throws std::runtime_error with the reference's text.
GgufFile* gguf_open(const char* path);

}  // namespace llhip
