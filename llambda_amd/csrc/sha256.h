// sha256.h -- SHA-256 of a byte range as 64 lower-case hex digits.
#pragma once

#include <cstddef>
#include <cstdint>

namespace llhip {

void sha256_hex(const void* data, size_t size, char out[65]);

}  // namespace llhip
