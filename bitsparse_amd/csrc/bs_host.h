// Host-side helpers of libbitsparse_hip.so: error reporting and the
// workspace layout shared by the compress and fp8 entry points.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bitsparse_hip.h"

namespace bs {

// Workspace layout: [0, 256) header, then one uint64 status word per tile.
//   header +0  : uint64 amax slot ((epoch << 32) | bf16 magnitude bits)
//   header +8  : uint32 look-back fallback counter
constexpr int64_t kWsHeaderBytes = 256;
constexpr int64_t kWsAmaxOffset = 0;
constexpr int64_t kWsFallbackOffset = 8;

// Largest matrix accepted: fewer than 2^32 elements, the range of the uint32
// tile prefix (the kernels index HBM with 64-bit element offsets), on the
// paths run past 2^31 elements on the GPU (raw bf16 compress: into a value
// buffer, or count + values of the standalone path; bf16 decompress; the
// bf16 dW GEMM); every other entry point (fp8
// or packed storage, quantizing compress, gradients, the fp8 dW GEMM, the
// fused up-projection, the reference-API pieces) stops at 2^31 until its
// own run past that size exists.  The reference forms element offsets in
// int32 (lib_sparse/src/triton_kernels.py:80), so its domain ends at 2^31.
constexpr uint64_t kMaxElems = 1ull << 32;
constexpr uint64_t kMaxElemsUntested = 1ull << 31;

// Kernels that stream a dense matrix at least this large use nontemporal
// (`nt`) loads and stores for it: nothing of it can stay in the 256 MiB last
// level cache for a later kernel, and the streaming hint raises the HBM rate
// (read-only 6.0 -> 6.8 TB/s; the 16384^2 compress 200 -> 173 us).  Smaller
// matrices keep plain accesses, which leave them cached for the next kernel
// (the configs[3]-sized fp8 unpack: 34 us plain, 41 us nontemporal).
// BITSPARSE_NT_MIN_BYTES overrides the threshold (tuning runs).
bool use_nontemporal(int64_t dense_bytes);

// Launch timing (bs_launch_timing): the next start/stop event pair for a
// kernel launch of the given kind (0 compress, 1 decompress), or false when
// timing is off on this thread.
bool timing_next(int kind, hipEvent_t* start, hipEvent_t* stop);

// hipLaunchKernelGGL, or hipExtLaunchKernelGGL with a timing event pair while
// launch timing is on.
template <typename F, typename... Args>
inline void launch_timed(int kind, F kernel, dim3 grid, dim3 block, uint32_t shmem, hipStream_t st,
                         Args... args)
{
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (timing_next(kind, &e0, &e1))
        hipExtLaunchKernelGGL(kernel, grid, block, shmem, st, e0, e1, 0u, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, shmem, st, args...);
}

// BS_ERR_INVALID when `stream` is capturing into a HIP graph.  Entry points
// whose device state is tagged with a host-chosen epoch (the compress
// look-back's status words, the fp8 amax slot) call it: a graph would replay
// the same epoch and take the previous replay's values for current ones.
int refuse_capture(hipStream_t stream, const char* what);

// The device a stream belongs to (the current device for the null stream).
hipError_t stream_device(hipStream_t stream, int* dev);

// amax of a bf16 array (of relu(x) with `relu`) into the amax slot of
// `workspace` under `epoch` (bs_amax / bs_amax_relu without clear_error();
// `check_capture` = refuse a capturing stream).
int amax_launch(const void* x, int64_t n, void* workspace, int64_t workspace_bytes, uint32_t epoch,
                void* stream, bool relu, bool check_capture);

// Records a formatted message for bs_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

}  // namespace bs
