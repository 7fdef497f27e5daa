// Error reporting, version and launch-timing entry points of libbitsparse_hip.so.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <atomic>
#include <vector>

#include "bs_host.h"

namespace bs {

static thread_local char g_err[512];

int set_error(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_err[0] = '\0'; }

// Launch timing (per thread): while enabled, every compress / decompress
// kernel launch takes the next pair of events from a pool that grows as
// needed; hipExtLaunchKernel records them at the kernel's start and end.
namespace {
struct TimedLaunch {
    hipEvent_t start, stop;
    int kind;
};
struct LaunchTiming {
    bool on = false;
    size_t used = 0;
    std::vector<TimedLaunch> pool;
};
thread_local LaunchTiming g_timing;
}  // namespace

bool timing_next(int kind, hipEvent_t* start, hipEvent_t* stop)
{
    LaunchTiming& t = g_timing;
    if (!t.on) return false;
    if (t.used == t.pool.size()) {
        TimedLaunch l{nullptr, nullptr, 0};
        if (hipEventCreate(&l.start) != hipSuccess) return false;
        if (hipEventCreate(&l.stop) != hipSuccess) {
            (void)hipEventDestroy(l.start);
            return false;
        }
        t.pool.push_back(l);
    }
    TimedLaunch& l = t.pool[t.used++];
    l.kind = kind;
    *start = l.start;
    *stop = l.stop;
    return true;
}

constexpr int64_t kNtMinBytesDefault = int64_t(192) << 20;

static int64_t nt_min_bytes_initial()
{
    if (const char* ev = getenv("BITSPARSE_NT_MIN_BYTES")) {
        char* end = nullptr;
        const long long v = strtoll(ev, &end, 10);
        if (end != ev && v >= 0) return (int64_t)v;
    }
    return kNtMinBytesDefault;
}

static std::atomic<int64_t> g_nt_min_bytes{nt_min_bytes_initial()};

bool use_nontemporal(int64_t dense_bytes)
{
    return dense_bytes >= g_nt_min_bytes.load(std::memory_order_relaxed);
}

hipError_t stream_device(hipStream_t stream, int* dev)
{
    if (stream == nullptr) return hipGetDevice(dev);
    return hipStreamGetDevice(stream, dev);
}

int refuse_capture(hipStream_t stream, const char* what)
{
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess) {
        (void)hipGetLastError();
        return BS_OK;
    }
    if (cs != hipStreamCaptureStatusNone)
        return set_error(BS_ERR_INVALID,
                         "%s cannot be captured into a HIP graph: its device state is tagged with a "
                         "per-call epoch that a replay would repeat", what);
    return BS_OK;
}

}  // namespace bs

using namespace bs;

extern "C" const char* bs_last_error(void) { return bs::g_err; }

extern "C" int bs_abi_version(void) { return 15; }

extern "C" int bs_host_device_pointer(void* host_ptr, void** device_ptr)
{
    clear_error();
    if (host_ptr == nullptr || device_ptr == nullptr)
        return set_error(BS_ERR_INVALID, "bs_host_device_pointer: null pointer");
    void* d = nullptr;
    const hipError_t e = hipHostGetDevicePointer(&d, host_ptr, 0);
    if (e != hipSuccess || d == nullptr) {
        (void)hipGetLastError();
        return set_error(BS_ERR_HIP, "bs_host_device_pointer: %s is not mapped pinned host memory (%s)",
                         "the pointer", hipGetErrorString(e));
    }
    *device_ptr = d;
    return BS_OK;
}

extern "C" int64_t bs_nontemporal_min_bytes(int64_t bytes)
{
    clear_error();
    return g_nt_min_bytes.exchange(bytes < 0 ? nt_min_bytes_initial() : bytes);
}

extern "C" int bs_launch_timing(int enable)
{
    clear_error();
    g_timing.on = enable != 0;
    g_timing.used = 0;
    return BS_OK;
}

extern "C" int bs_launch_timing_read(float* ms_out, int* kinds_out, int max_n, int* n_out)
{
    clear_error();
    if (n_out == nullptr) return set_error(BS_ERR_INVALID, "bs_launch_timing_read: null n_out");
    const int n = (int)g_timing.used;
    *n_out = n;
    for (int i = 0; i < n && i < max_n; i++) {
        const TimedLaunch& l = g_timing.pool[i];
        hipError_t e = hipEventSynchronize(l.stop);
        float ms = 0.0f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, l.start, l.stop);
        if (e != hipSuccess)
            return set_error(BS_ERR_HIP, "bs_launch_timing_read: %s", hipGetErrorString(e));
        if (ms_out) ms_out[i] = ms;
        if (kinds_out) kinds_out[i] = l.kind;
    }
    g_timing.used = 0;
    return BS_OK;
}
