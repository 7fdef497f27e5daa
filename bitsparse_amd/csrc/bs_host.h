// Host-side helpers of libbitsparse_hip.so: error reporting and the
// workspace layout shared by the compress and fp8 entry points.
#pragma once

#include <stdint.h>

#include "bitsparse_hip.h"

namespace bs {

// Workspace layout: [0, 256) header, then one uint64 status word per tile.
//   header +0  : uint64 amax slot ((epoch << 32) | bf16 magnitude bits)
//   header +8  : uint32 look-back fallback counter
constexpr int64_t kWsHeaderBytes = 256;
constexpr int64_t kWsAmaxOffset = 0;
constexpr int64_t kWsFallbackOffset = 8;

// Records a formatted message for bs_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

}  // namespace bs
