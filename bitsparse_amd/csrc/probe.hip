// Streaming probes of the codec's HBM access mixes (measurement only; no
// counterpart in the reference).  They move exactly the bytes of a compress or
// a decompress launch, in the same load / store instructions and the same
// per-workgroup layout, with no scan, no compaction and no gather, so their
// duration is the floor those kernels are measured against:
//
//   compress mix   (mode 0): workgroup u reads the 8 64x64 bf16 tiles of unit u
//                  (8 waves, lane chunks of 16 bytes, each load covering 8 whole
//                  tile rows, nontemporal), stores one bitmask byte per chunk
//                  (64 bytes per store instruction) and `vals_per_unit` bytes of
//                  values at u * vals_per_unit with 16-byte stores;
//   decompress mix (mode 1): workgroup u loads those bitmask bytes and value
//                  bytes and stores the unit's 8 tiles (16-byte chunks,
//                  nontemporal).
//
// The data written is formed from the data read, so no access is dead.
#include <hip/hip_runtime.h>

#include "bitsparse_hip.h"
#include "bs_device.h"
#include "bs_host.h"

namespace bs {

constexpr int kProbeU = 8;      // tiles per workgroup (the compress unit)

template <int MODE, bool NT>
__global__ __launch_bounds__(64 * kProbeU) __attribute__((amdgpu_waves_per_eu(8)))
void stream_probe_kernel(uint8_t* big, int64_t N, uint32_t grid_n, uint8_t* vals, uint32_t vals_per_unit,
                         uint8_t* bitmask)
{
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const uint32_t u = blockIdx.x;
    const uint32_t t = u * kProbeU + (uint32_t)wave;
    const uint32_t tm = t / grid_n, tn = t - tm * grid_n;
    // the chunk of lane `lane` in row 8k of the tile: rows 8k + lane/8, columns 8(lane%8)..+7
    uint8_t* const org = big + ((uint64_t)tm * 64 * (uint64_t)N + (uint64_t)tn * 64 + (uint64_t)(lane >> 3) * (uint64_t)N +
                                (uint64_t)((lane & 7) * 8)) * 2;
    // this wave's share of the unit's value bytes: 16-byte slots j = 64 i + lane
    const uint32_t wslots = vals_per_unit / (16u * kProbeU);
    uint8_t* const wv = vals + (uint64_t)u * vals_per_unit + (uint64_t)wave * wslots * 16u;
    uint8_t* const bm = bitmask + (uint64_t)t * kTileBytes + lane;
    if constexpr (MODE == 0) {
        uint4 d[8];
#pragma unroll
        for (int k = 0; k < 8; k++) d[k] = ld16<NT>(org + (uint64_t)(8 * k) * (uint64_t)N * 2);
#pragma unroll
        for (int k = 0; k < 8; k++) bm[64 * k] = (uint8_t)(d[k].x ^ d[k].w);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t j = 64u * k + (uint32_t)lane;
            if (j < wslots) st16<NT>(wv + (uint64_t)j * 16u, d[k]);
        }
    } else {
        uint4 v[8];
        uint32_t m[8];
#pragma unroll
        for (int k = 0; k < 8; k++) m[k] = bm[64 * k];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t j = 64u * k + (uint32_t)lane;
            v[k] = j < wslots ? ld16<NT>(wv + (uint64_t)j * 16u) : uint4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint4 w = {v[k].x ^ m[k], v[k].y, v[k].z, v[k].w};
            st16<NT>(org + (uint64_t)(8 * k) * (uint64_t)N * 2, w);
        }
    }
}

}  // namespace bs

using namespace bs;

extern "C" int bs_stream_probe(int mode, void* dense, int64_t M, int64_t N, void* vals, int64_t vals_bytes,
                               int64_t vals_per_unit, uint8_t* bitmask, int64_t bitmask_bytes, int nontemporal,
                               void* stream)
{
    clear_error();
    if (mode != 0 && mode != 1) return set_error(BS_ERR_INVALID, "bs_stream_probe: mode must be 0 or 1");
    if (!dense || !vals || !bitmask) return set_error(BS_ERR_INVALID, "bs_stream_probe: null pointer");
    if (M <= 0 || N <= 0 || M % 64 || N % 64)
        return set_error(BS_ERR_INVALID, "bs_stream_probe: M and N must be positive multiples of 64");
    const int64_t T = (M / 64) * (N / 64);
    if (T % kProbeU || T / kProbeU > INT32_MAX || (uint64_t)M * (uint64_t)N >= kMaxElems)
        return set_error(BS_ERR_INVALID, "bs_stream_probe: tile count must be a multiple of 8 below 2^32 elements");
    if (vals_per_unit < 0 || vals_per_unit > 2 * kTileNumel * kProbeU || vals_per_unit % (16 * kProbeU))
        return set_error(BS_ERR_INVALID, "bs_stream_probe: vals_per_unit must be a multiple of 128 in [0, 65536]");
    if (vals_bytes < (T / kProbeU) * vals_per_unit || bitmask_bytes < T * kTileBytes)
        return set_error(BS_ERR_INVALID, "bs_stream_probe: vals or bitmask buffer too small");
    if ((((uintptr_t)dense) | ((uintptr_t)vals)) & 15u)
        return set_error(BS_ERR_INVALID, "bs_stream_probe: dense and vals must be 16-byte aligned");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const dim3 grid((uint32_t)(T / kProbeU)), block(64 * kProbeU);
    auto* d = reinterpret_cast<uint8_t*>(dense);
    auto* v = reinterpret_cast<uint8_t*>(vals);
    const uint32_t gn = (uint32_t)(N / 64), vpu = (uint32_t)vals_per_unit;
    if (mode == 0) {
        if (nontemporal) hipLaunchKernelGGL((stream_probe_kernel<0, true>), grid, block, 0, st, d, N, gn, v, vpu, bitmask);
        else hipLaunchKernelGGL((stream_probe_kernel<0, false>), grid, block, 0, st, d, N, gn, v, vpu, bitmask);
    } else {
        if (nontemporal) hipLaunchKernelGGL((stream_probe_kernel<1, true>), grid, block, 0, st, d, N, gn, v, vpu, bitmask);
        else hipLaunchKernelGGL((stream_probe_kernel<1, false>), grid, block, 0, st, d, N, gn, v, vpu, bitmask);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_stream_probe: %s", hipGetErrorString(e));
    return BS_OK;
}
