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

// Largest matrix accepted by the codec, gradient and GEMM entry points:
// fewer than 2^31 elements.  The reference forms element offsets in int32
// (lib_sparse/src/triton_kernels.py:80), so this is its domain as well.  The
// kernels here index with 64-bit offsets and a uint32 prefix, but a GPU run at
// 2^31 + 2^21 elements faulted without a cause found in this code, so shapes
// from 2^31 elements up are refused until such a run passes.
constexpr uint64_t kMaxElems = 1ull << 31;

// Records a formatted message for bs_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

}  // namespace bs
