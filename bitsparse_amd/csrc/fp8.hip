// e4m3fn quantisation for gfx950: amax reduction and the quantize pass that
// together replace lib_sparse/fp8.py:123-129 (to_fp8).
//
// scale = max(fp32(amax|x|) / 448, 1e-9); q = e4m3fn_RNE(fp32(x) / scale)
// with one correctly rounded fp32 division per value: the quantize pass reads
// each code from a table of the scale's 24-exponent window (quant_chunk_tab),
// which every workgroup builds in LDS from exact divisions.
#include <cmath>

#include "bs_device.h"
#include "bs_host.h"

namespace bs {

constexpr int kFp8Threads = 256;

// max over |x| as bf16 magnitude bits; NaN patterns sort above Inf, so a NaN
// anywhere wins the max and the decoded amax is NaN.  Each thread keeps four
// independent 16-byte loads in flight per pass; the grid is a few workgroups
// per CU, so the per-workgroup device-scope atomicMax on the one slot (the
// only serialised step) stays at a few hundred.
constexpr int kAmaxUnroll = 4;

// RELU: amax of relu(x) (x <= 0 counts as 0; NaN is kept by relu, so it still wins).
template <bool RELU>
__device__ __forceinline__ uint32_t mag_bits(uint32_t b)
{
    const uint32_t m = b & 0x7fffu;
    if constexpr (RELU) return ((b & 0x8000u) && m <= 0x7f80u) ? 0u : m;
    else return m;
}

// NT: nontemporal loads of x.
template <bool RELU, bool NT>
__global__ __launch_bounds__(kFp8Threads) void amax_bf16_kernel(const uint16_t* x, int64_t n,
                                                                uint64_t* slot, uint32_t epoch)
{
    __shared__ uint32_t s_w[kFp8Threads / 64];
    const int tid = threadIdx.x;
    uint32_t m = 0;
    const int64_t nvec = ((((uintptr_t)x) & 15u) == 0) ? n / 8 : 0;
    const int64_t stride = (int64_t)gridDim.x * kFp8Threads;
    const uint4* xv = reinterpret_cast<const uint4*>(x);
    int64_t i = (int64_t)blockIdx.x * kFp8Threads + tid;
    for (; i + (kAmaxUnroll - 1) * stride < nvec; i += kAmaxUnroll * stride) {
        uint4 v[kAmaxUnroll];
#pragma unroll
        for (int u = 0; u < kAmaxUnroll; u++) v[u] = ld16<NT>(xv + i + u * stride);
#pragma unroll
        for (int u = 0; u < kAmaxUnroll; u++) {
            const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                m = max(m, mag_bits<RELU>(w[k] & 0xffffu));
                m = max(m, mag_bits<RELU>(w[k] >> 16));
            }
        }
    }
    for (; i < nvec; i += stride) {
        const uint4 v = ld16<NT>(xv + i);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            m = max(m, mag_bits<RELU>(w[k] & 0xffffu));
            m = max(m, mag_bits<RELU>(w[k] >> 16));
        }
    }
    for (int64_t j = nvec * 8 + (int64_t)blockIdx.x * kFp8Threads + tid; j < n; j += stride)
        m = max(m, mag_bits<RELU>((uint32_t)x[j]));
    m = wave_max_u32(m);
    if ((tid & 63) == 0) s_w[tid >> 6] = m;
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kFp8Threads / 64; w++) m = max(m, s_w[w]);
        atomicMax((unsigned long long*)slot, (unsigned long long)(((uint64_t)epoch << 32) | m));
    }
}

__device__ __forceinline__ float fp8_scale_from_slot(const uint64_t* slot, uint32_t epoch)
{
    uint64_t s = *slot;
    float amax = ((uint32_t)(s >> 32) == epoch) ? bf16_to_f32((uint32_t)s & 0xffffu) : 0.0f;
    float sc = amax / 448.0f;
    return (sc < 1e-9f) ? 1e-9f : sc;
}

// The code table of `scale` (qtab_build_kernel's layout) built in LDS by the
// workgroup: the positive half from div2_to_e4m3 on pairs of magnitudes
// (exact: f32_to_e4m3 of the correctly rounded quotient), the negative half
// with the sign bit set; a NaN scale gives the scale's NaN for every non-NaN
// magnitude and x's own NaN otherwise, as the division does.
__device__ __forceinline__ void qtab_build_lds(uint8_t* tab, float scale, float rcp, int tid)
{
    const int qoff = qtab_offset(scale);
    const bool nan_s = scale != scale;
    static_assert(kQtabEntries % 2 == 0, "entries come in pairs");
    for (int p = tid; p < kQtabEntries / 2; p += kFp8Threads) {
        const int m0 = min(max(qoff + 2 * p, 0), 0x7fff), m1 = min(max(qoff + 2 * p + 1, 0), 0x7fff);
        uint32_t pos, neg;
        if (nan_s) {
            pos = 0x7f7fu;
            neg = (m0 > 0x7f80 ? 0xffu : 0x7fu) | ((m1 > 0x7f80 ? 0xffu : 0x7fu) << 8);
        } else {
            pos = div2_to_e4m3(bf16_to_f32((uint32_t)m0), bf16_to_f32((uint32_t)m1), scale, rcp);
            neg = pos | 0x8080u;
        }
        *reinterpret_cast<uint16_t*>(tab + 2 * p) = (uint16_t)pos;
        *reinterpret_cast<uint16_t*>(tab + kQtabEntries + 2 * p) = (uint16_t)neg;
    }
}

// NT: nontemporal loads of x and stores of q.  Each thread's first chunk is
// loaded before the table is built.
template <bool NT>
__global__ __launch_bounds__(kFp8Threads) void quantize_e4m3_kernel(const uint16_t* x, int64_t n,
                                                                    uint8_t* q, float* scale_out,
                                                                    const uint64_t* slot,
                                                                    uint32_t epoch)
{
    __shared__ __align__(16) uint8_t s_tab[kQtabBytes];
    const float scale = fp8_scale_from_slot(slot, epoch);
    const float rcp = 1.0f / scale;
    const int tid = threadIdx.x;
    if (blockIdx.x == 0 && tid == 0 && scale_out) *scale_out = scale;
    const bool vec = ((((uintptr_t)x) & 15u) == 0) && ((((uintptr_t)q) & 7u) == 0);
    const int64_t nvec = vec ? n / 8 : 0;
    const int64_t stride = (int64_t)gridDim.x * kFp8Threads;
    int64_t i = (int64_t)blockIdx.x * kFp8Threads + tid;
    uint4 v = i < nvec ? ld16<NT>(reinterpret_cast<const uint4*>(x) + i) : uint4{0u, 0u, 0u, 0u};
    qtab_build_lds(s_tab, scale, rcp, tid);
    __syncthreads();
    const int qoff = qtab_offset(scale);
    for (; i < nvec; i += stride) {
        const int64_t inext = i + stride;
        const uint4 vn = inext < nvec ? ld16<NT>(reinterpret_cast<const uint4*>(x) + inext) : uint4{0u, 0u, 0u, 0u};
        st8<NT>(reinterpret_cast<uint2*>(q) + i, quant_chunk_tab(v, s_tab, qoff));
        v = vn;
    }
    for (int64_t j = nvec * 8 + (int64_t)blockIdx.x * kFp8Threads + tid; j < n; j += stride) {
        const uint32_t b = x[j];
        q[j] = (uint8_t)qtab_code(s_tab, b & 0x7fffu, b >> 15, qoff);
    }
}

static uint32_t grid_for(int64_t n)
{
    int64_t g = (n / 8 + kFp8Threads - 1) / kFp8Threads;
    if (g < 1) g = 1;
    if (g > 4096) g = 4096;
    return (uint32_t)g;
}

// the quantize pass: at least 8 chunks per thread where n allows (each
// workgroup builds the 6 KiB code table first), at most 2048 workgroups
static uint32_t quantize_grid(int64_t n)
{
    int64_t g = (n / 8 + 8 * kFp8Threads - 1) / (8 * kFp8Threads);
    if (g < 1) g = 1;
    if (g > 2048) g = 2048;
    return (uint32_t)g;
}


// Byte transpose out[c * ld_out + r] = in[r * ld_in + c] (r < R, c < C): the
// fp8 GEMM operand layout change (row-major <-> column-major) that hipBLASLt's
// fp8 path needs.  A 256-thread workgroup moves a 128 x 128 tile: 16-byte
// loads (eight lanes cover one 128-byte input row), the tile in LDS as
// dwords with the dword column XOR-swizzled by row / 4, then per lane a 4 x 4
// byte block (four LDS dwords from four consecutive rows) transposed in
// registers with v_perm_b32 and stored as one dword of each of four output
// rows, 32 lanes covering one 128-byte output row.  Needs C % 16 == 0,
// R % 4 == 0, ld_in % 16 == 0, ld_out % 4 == 0 and in / out 16 / 4-byte
// aligned (the host checks).
constexpr int kTrTile = 128;

__device__ __forceinline__ void transpose4x4_bytes(const uint32_t (&a)[4], uint32_t (&o)[4])
{
    // a[k] = bytes (k, 0..3); o[i] = bytes (0..3, i)
    const uint32_t t0 = __builtin_amdgcn_perm(a[1], a[0], 0x05010400u);   // a0.b0 a1.b0 a0.b1 a1.b1
    const uint32_t t1 = __builtin_amdgcn_perm(a[1], a[0], 0x07030602u);   // a0.b2 a1.b2 a0.b3 a1.b3
    const uint32_t u0 = __builtin_amdgcn_perm(a[3], a[2], 0x05010400u);
    const uint32_t u1 = __builtin_amdgcn_perm(a[3], a[2], 0x07030602u);
    o[0] = __builtin_amdgcn_perm(u0, t0, 0x05040100u);
    o[1] = __builtin_amdgcn_perm(u0, t0, 0x07060302u);
    o[2] = __builtin_amdgcn_perm(u1, t1, 0x05040100u);
    o[3] = __builtin_amdgcn_perm(u1, t1, 0x07060302u);
}

__global__ __launch_bounds__(256) void transpose_u8_kernel(const uint8_t* in, int64_t R, int64_t C, int64_t ld_in,
                                                           uint8_t* out, int64_t ld_out, uint32_t tiles_c)
{
    __shared__ uint32_t s[kTrTile * 32];
    const int t = threadIdx.x;
    const uint32_t tr = blockIdx.x / tiles_c, tc = blockIdx.x - tr * tiles_c;
    const int64_t r0 = (int64_t)tr * kTrTile, c0 = (int64_t)tc * kTrTile;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int rr = t / 8 + 32 * q, cc = 16 * (t % 8);
        const int64_t r = r0 + rr, c = c0 + cc;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (r < R && c < C) v = *reinterpret_cast<const uint4*>(in + r * ld_in + c);
        const int sw = (rr >> 2) & 31, d0 = cc / 4;
        uint32_t* row = s + rr * 32;
        row[(d0 + 0) ^ sw] = v.x;
        row[(d0 + 1) ^ sw] = v.y;
        row[(d0 + 2) ^ sw] = v.z;
        row[(d0 + 3) ^ sw] = v.w;
    }
    __syncthreads();
    const int rb = t % 32;                  // input rows 4 rb .. 4 rb + 3 (swizzle rb)
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const int cb = t / 32 + 8 * p;      // input dword column: columns 4 cb .. 4 cb + 3
        uint32_t a[4], o[4];
#pragma unroll
        for (int k = 0; k < 4; k++) a[k] = s[(4 * rb + k) * 32 + (cb ^ rb)];
        transpose4x4_bytes(a, o);
        const int64_t orow = c0 + 4 * cb, ocol = r0 + 4 * rb;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (orow + i < C && ocol < R) *reinterpret_cast<uint32_t*>(out + (orow + i) * ld_out + ocol) = o[i];
    }
}


// e4m3fn -> bf16 bits, exact (every e4m3fn value is a bf16 value); NaN codes
// give 0x7fc0, the quiet NaN torch's float8 -> bfloat16 cast produces
__device__ __forceinline__ uint32_t e4m3_to_bf16_bits(uint32_t c)
{
    const uint32_t s = (c & 0x80u) << 8, a = c & 0x7fu;
    if (a == 0x7fu) return 0x7fc0u;
    const uint32_t e = a >> 3, m = a & 7u;
    if (e != 0u) return s | ((e + 120u) << 7) | (m << 4);
    if (m == 0u) return s;
    const uint32_t p = 31u - (uint32_t)__builtin_clz(m);       // subnormal m 2^-9 = 1.f 2^(p-9)
    return s | ((p + 118u) << 7) | ((m << (7u - p)) & 0x7fu);
}

// bf16 bits of the four e4m3fn codes of w, two per dword: the hardware
// conversion to fp32 (v_cvt_pk_f32_fp8: every e4m3fn value is a bf16 value,
// so the fp32's high half is exact), NaN codes (0x7f / 0xff) as 0x7fc0
__device__ __forceinline__ void widen4_e4m3(uint32_t w, uint32_t& lo, uint32_t& hi)
{
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
    const f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    lo = __builtin_amdgcn_perm(__float_as_uint(a.y), __float_as_uint(a.x), 0x07060302u);
    hi = __builtin_amdgcn_perm(__float_as_uint(b.y), __float_as_uint(b.x), 0x07060302u);
    const uint32_t nan = ((w & 0x7f7f7f7fu) + 0x01010101u) & 0x80808080u;   // bit 7 of each NaN byte
    if (nan) {
        if (nan & 0x00000080u) lo = (lo & 0xffff0000u) | 0x7fc0u;
        if (nan & 0x00008000u) lo = (lo & 0x0000ffffu) | 0x7fc00000u;
        if (nan & 0x00800000u) hi = (hi & 0xffff0000u) | 0x7fc0u;
        if (nan & 0x80000000u) hi = (hi & 0x0000ffffu) | 0x7fc00000u;
    }
}

// out[i] = bf16(in[i]) for e4m3fn codes: 16 codes per lane (one 16-byte load,
// two 16-byte stores), grid-stride; a tail of n % 16 codes element by element
__global__ __launch_bounds__(256) void widen_e4m3_kernel(const uint8_t* in, int64_t n, uint16_t* out)
{
    const int64_t groups = n / 16;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x; g < groups; g += stride) {
        const uint4 v = *reinterpret_cast<const uint4*>(in + g * 16);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint32_t o[8];
#pragma unroll
        for (int k = 0; k < 4; k++) widen4_e4m3(w[k], o[2 * k], o[2 * k + 1]);
        uint4* dst = reinterpret_cast<uint4*>(out + g * 16);
        dst[0] = uint4{o[0], o[1], o[2], o[3]};
        dst[1] = uint4{o[4], o[5], o[6], o[7]};
    }
    if (blockIdx.x == 0 && threadIdx.x < (unsigned)(n - groups * 16)) {
        const int64_t i = groups * 16 + threadIdx.x;
        out[i] = (uint16_t)e4m3_to_bf16_bits(in[i]);
    }
}


// The ReLU^2 forward's h = k * r^2 (relu2_sq_bits) written back in place,
// with amax|h| into the slot: the square and scale passes and the amax pass
// of to_fp8(h) in one read and one write of r.

template <bool NT>
__global__ __launch_bounds__(kFp8Threads) void relu2_square_amax_kernel(uint16_t* x, int64_t n, float k,
                                                                        uint64_t* slot, uint32_t epoch)
{
    __shared__ uint32_t s_w[kFp8Threads / 64];
    const int tid = threadIdx.x;
    uint32_t m = 0;
    const int64_t nvec = ((((uintptr_t)x) & 15u) == 0) ? n / 8 : 0;
    const int64_t stride = (int64_t)gridDim.x * kFp8Threads;
    uint4* xv = reinterpret_cast<uint4*>(x);
    for (int64_t i = (int64_t)blockIdx.x * kFp8Threads + tid; i < nvec; i += stride) {
        const uint4 v = ld16<NT>(xv + i);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t lo = relu2_sq_bits(w[q] & 0xffffu, k), hi = relu2_sq_bits(w[q] >> 16, k);
            m = max(m, max(lo & 0x7fffu, hi & 0x7fffu));
            o[q] = lo | (hi << 16);
        }
        st16<NT>(xv + i, uint4{o[0], o[1], o[2], o[3]});
    }
    for (int64_t j = nvec * 8 + (int64_t)blockIdx.x * kFp8Threads + tid; j < n; j += stride) {
        const uint32_t h = relu2_sq_bits(x[j], k);
        m = max(m, h & 0x7fffu);
        x[j] = (uint16_t)h;
    }
    m = wave_max_u32(m);
    if ((tid & 63) == 0) s_w[tid >> 6] = m;
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kFp8Threads / 64; w++) m = max(m, s_w[w]);
        atomicMax((unsigned long long*)slot, (unsigned long long)(((uint64_t)epoch << 32) | m));
    }
}

// amax|k r^2| (relu2_sq_bits) from the amax of r = relu(z) in the slot, for
// a finite k: the map is non-decreasing on r >= 0 and NaN, so the amax of the
// squared tensor is that of its largest element; written under epoch_out
// (slot = amax 0 when the slot does not hold epoch_in).
__global__ void amax_relu2_from_kernel(uint64_t* slot, uint32_t epoch_in, uint32_t epoch_out, float k)
{
    if (threadIdx.x != 0) return;
    const uint64_t s = *slot;
    const uint32_t m = (uint32_t)(s >> 32) == epoch_in ? (uint32_t)s & 0x7fffu : 0u;
    *slot = ((uint64_t)epoch_out << 32) | (relu2_sq_bits(m, k) & 0x7fffu);
}

}  // namespace bs

using namespace bs;

extern "C" int bs_amax_relu2_from(void* workspace, int64_t workspace_bytes, uint32_t epoch_in, uint32_t epoch_out,
                                  float k, void* stream)
{
    clear_error();
    if (workspace == nullptr || workspace_bytes < kWsHeaderBytes)
        return set_error(BS_ERR_INVALID, "bs_amax_relu2_from: workspace too small");
    if (epoch_in == 0 || epoch_in >= (1u << 30) || epoch_out == 0 || epoch_out >= (1u << 30))
        return set_error(BS_ERR_INVALID, "bs_amax_relu2_from: epoch out of range");
    if (!std::isfinite(k)) return set_error(BS_ERR_INVALID, "bs_amax_relu2_from: k must be finite");
    if (int rc = refuse_capture((hipStream_t)stream, "bs_amax_relu2_from")) return rc;
    uint64_t* slot = reinterpret_cast<uint64_t*>((uint8_t*)workspace + kWsAmaxOffset);
    hipLaunchKernelGGL(amax_relu2_from_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, slot, epoch_in, epoch_out,
                       k);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_amax_relu2_from launch: %s", hipGetErrorString(e));
    return BS_OK;
}

int bs::amax_launch(const void* x, int64_t n, void* workspace, int64_t workspace_bytes, uint32_t epoch,
                    void* stream, bool relu, bool check_capture)
{
    if (n < 0) return set_error(BS_ERR_INVALID, "bs_amax: negative n");
    if (workspace == nullptr || workspace_bytes < kWsHeaderBytes)
        return set_error(BS_ERR_INVALID, "bs_amax: workspace too small");
    if (epoch == 0 || epoch >= (1u << 30)) return set_error(BS_ERR_INVALID, "bs_amax: epoch out of range");
    if (n > 0 && x == nullptr) return set_error(BS_ERR_INVALID, "bs_amax: null input");
    if (((uintptr_t)x) & 1u) return set_error(BS_ERR_INVALID, "bs_amax: input misaligned");
    if (check_capture) {
        if (int rc = refuse_capture((hipStream_t)stream, "bs_amax")) return rc;
    }
    if (n == 0) return BS_OK;   // slot keeps an older epoch: readers then see amax = 0
    uint64_t* slot = reinterpret_cast<uint64_t*>((uint8_t*)workspace + kWsAmaxOffset);
    int dev = 0, cus = 0;
    if (stream_device((hipStream_t)stream, &dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
        cus = 256;
    uint32_t grid = grid_for(n);
    if (grid > (uint32_t)(2 * cus)) grid = (uint32_t)(2 * cus);
    const bool nt = use_nontemporal(2 * n);
    auto kernel = relu ? (nt ? amax_bf16_kernel<true, true> : amax_bf16_kernel<true, false>)
                       : (nt ? amax_bf16_kernel<false, true> : amax_bf16_kernel<false, false>);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kFp8Threads), 0, (hipStream_t)stream, (const uint16_t*)x, n,
                       slot, epoch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_amax launch: %s", hipGetErrorString(e));
    return BS_OK;
}

extern "C" int bs_amax(const void* x, int64_t n, void* workspace, int64_t workspace_bytes, uint32_t epoch,
                       void* stream)
{
    clear_error();
    return amax_launch(x, n, workspace, workspace_bytes, epoch, stream, false, true);
}

extern "C" int bs_amax_relu(const void* preact, int64_t n, void* workspace, int64_t workspace_bytes,
                            uint32_t epoch, void* stream)
{
    clear_error();
    return amax_launch(preact, n, workspace, workspace_bytes, epoch, stream, true, true);
}

extern "C" int bs_quantize_e4m3fn(const void* x, int64_t n, void* q_out, float* scale_out,
                                  const void* workspace, int64_t workspace_bytes, uint32_t epoch,
                                  void* stream)
{
    clear_error();
    if (n < 0) return set_error(BS_ERR_INVALID, "bs_quantize_e4m3fn: negative n");
    if (workspace == nullptr || workspace_bytes < kWsHeaderBytes)
        return set_error(BS_ERR_INVALID, "bs_quantize_e4m3fn: workspace too small");
    if (n > 0 && (x == nullptr || q_out == nullptr))
        return set_error(BS_ERR_INVALID, "bs_quantize_e4m3fn: null pointer");
    if (((uintptr_t)x) & 1u) return set_error(BS_ERR_INVALID, "bs_quantize_e4m3fn: input misaligned");
    const uint64_t* slot = reinterpret_cast<const uint64_t*>((const uint8_t*)workspace + kWsAmaxOffset);
    auto kernel = use_nontemporal(2 * n) ? quantize_e4m3_kernel<true> : quantize_e4m3_kernel<false>;
    hipLaunchKernelGGL(kernel, dim3(quantize_grid(n)), dim3(kFp8Threads), 0, (hipStream_t)stream,
                       (const uint16_t*)x, n, (uint8_t*)q_out, scale_out, slot, epoch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_quantize_e4m3fn launch: %s", hipGetErrorString(e));
    return BS_OK;
}

extern "C" int bs_transpose_u8(const void* in, int64_t R, int64_t C, int64_t ld_in, void* out, int64_t ld_out,
                               void* stream)
{
    clear_error();
    if (R < 0 || C < 0) return set_error(BS_ERR_INVALID, "bs_transpose_u8: negative size");
    if (R == 0 || C == 0) return BS_OK;
    if (in == nullptr || out == nullptr) return set_error(BS_ERR_INVALID, "bs_transpose_u8: null pointer");
    if (C % 16 != 0 || R % 4 != 0)
        return set_error(BS_ERR_INVALID, "bs_transpose_u8: C must be a multiple of 16 and R of 4");
    if (ld_in < C || ld_in % 16 != 0 || ld_out < R || ld_out % 4 != 0)
        return set_error(BS_ERR_INVALID, "bs_transpose_u8: ld_in >= C, multiple of 16; ld_out >= R, multiple of 4");
    if (((uintptr_t)in) % 16 != 0 || ((uintptr_t)out) % 4 != 0)
        return set_error(BS_ERR_INVALID, "bs_transpose_u8: in must be 16-byte and out 4-byte aligned");
    const uint64_t tiles_r = (uint64_t)((R + kTrTile - 1) / kTrTile), tiles_c = (uint64_t)((C + kTrTile - 1) / kTrTile);
    if (tiles_r * tiles_c >= (1ull << 31) || tiles_c >= (1ull << 32))
        return set_error(BS_ERR_INVALID, "bs_transpose_u8: too many tiles");
    hipLaunchKernelGGL(transpose_u8_kernel, dim3((uint32_t)(tiles_r * tiles_c)), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)in, R, C, ld_in, (uint8_t*)out, ld_out, (uint32_t)tiles_c);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_transpose_u8 launch: %s", hipGetErrorString(e));
    return BS_OK;
}

extern "C" int bs_widen_e4m3fn(const void* in, int64_t n, void* out, void* stream)
{
    clear_error();
    if (n < 0) return set_error(BS_ERR_INVALID, "bs_widen_e4m3fn: negative n");
    if (n == 0) return BS_OK;
    if (in == nullptr || out == nullptr) return set_error(BS_ERR_INVALID, "bs_widen_e4m3fn: null pointer");
    if (((uintptr_t)in) % 16 != 0 || ((uintptr_t)out) % 16 != 0)
        return set_error(BS_ERR_INVALID, "bs_widen_e4m3fn: in and out must be 16-byte aligned");
    const int64_t groups = n / 16;
    int64_t blocks = (groups + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(widen_e4m3_kernel, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)in, n, (uint16_t*)out);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_widen_e4m3fn launch: %s", hipGetErrorString(e));
    return BS_OK;
}

extern "C" int bs_relu2_square_amax(void* r, int64_t n, float k, void* workspace, int64_t workspace_bytes,
                                    uint32_t epoch, void* stream)
{
    clear_error();
    if (n < 0) return set_error(BS_ERR_INVALID, "bs_relu2_square_amax: negative n");
    if (workspace == nullptr || workspace_bytes < kWsHeaderBytes)
        return set_error(BS_ERR_INVALID, "bs_relu2_square_amax: workspace too small");
    if (epoch == 0 || epoch >= (1u << 30)) return set_error(BS_ERR_INVALID, "bs_relu2_square_amax: epoch out of range");
    if (n > 0 && r == nullptr) return set_error(BS_ERR_INVALID, "bs_relu2_square_amax: null input");
    if (((uintptr_t)r) & 1u) return set_error(BS_ERR_INVALID, "bs_relu2_square_amax: input misaligned");
    if (int rc = refuse_capture((hipStream_t)stream, "bs_relu2_square_amax")) return rc;
    if (n == 0) return BS_OK;
    uint64_t* slot = reinterpret_cast<uint64_t*>((uint8_t*)workspace + kWsAmaxOffset);
    int dev = 0, cus = 0;
    if (stream_device((hipStream_t)stream, &dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
        cus = 256;
    uint32_t grid = grid_for(n);
    if (grid > (uint32_t)(4 * cus)) grid = (uint32_t)(4 * cus);
    auto kernel = use_nontemporal(2 * n) ? relu2_square_amax_kernel<true> : relu2_square_amax_kernel<false>;
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kFp8Threads), 0, (hipStream_t)stream, (uint16_t*)r, n, k, slot,
                       epoch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_relu2_square_amax launch: %s", hipGetErrorString(e));
    return BS_OK;
}
