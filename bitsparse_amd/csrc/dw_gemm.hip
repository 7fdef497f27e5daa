// Reconstruct-into-LDS MFMA GEMM for gfx950:  C[M, N] = At^T @ B
// where At is a dense [K, M] bf16 matrix (m contiguous; the MLP backward
// passes dY itself) and B is a compressed [K, N] activation (64x64-tile
// bitmask + prefix + values) that is never written to HBM in dense form.
//
// Replaces the "decompress B to HBM, then library GEMM" of the reference's
// AspB / AspRelu2B (lib_sparse/src/sparse_matmul.py:24-28, :109-113).  In the
// MLP backward K = tokens, At = dY [tokens, d_out], B = h [tokens, d_ff],
// C = dW2 [d_out, d_ff].
//
// Workgroup = 256 threads (4 waves), output tile 256 x 64, K-step = one
// compressed B tile (64 tokens).  Both operands stay in their natural
// row-major (k-outer) layout in LDS: A_s[k][m] straight from dY, B_s[k][n]
// decoded row by row (8 columns = one bitmask byte per 16-byte store).  The
// k-contiguous MFMA operands are read with ds_read_b64_tr_b16: within each
// 16-lane group, output lane i receives element i%4 of source lanes
// 4c + i/4 (c = 0..3), so pointing source lane j at row k0 + j/4, columns
// n0 + 4*(j%4) gives lane i the column B[k0..k0+3][n0+i].
// LDS is double-buffered: while the MFMAs consume step k, the data waves
// decode step k+1 into the other buffer and the loads of step k+2 are in
// flight; two barriers per step.
#include "bs_device.h"
#include "bs_host.h"

namespace bs {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kGM = 256;           // C rows per workgroup
constexpr int kGN = 64;            // C columns per workgroup (one B tile column)
constexpr int kGK = 64;            // K per step (one B tile row)
constexpr int kGThreads = 256;
constexpr int kAP = kGM + 8;       // A_s row pitch (elements): 528 bytes
constexpr int kBP = kGN + 8;       // B_s row pitch (elements): 144 bytes
constexpr int kRunSlots = 4096 / 8 + 2;   // one tile's bf16 value run, 16-byte slots
constexpr int kMaxSteps = 256;     // K-steps per workgroup (prefixes held in LDS)

struct GemmArgs {
    const uint16_t* At;           // [K, M] bf16, row stride ldat
    int64_t M, K, ldat;
    const uint8_t* vals;          // compressed B
    int64_t vals_numel;
    const uint8_t* bitmask;
    const uint32_t* prefix;
    const int64_t* vals_offset;
    int64_t N;
    uint32_t grid_n;              // B tiles along N
    float relu2_scale;
    const float* b_scale;         // square + fp8 storage: multiply by bf16(scale^2)
    uint16_t* C;                  // [M, N] bf16 (no split)
    float* part;                  // [split, M, N] fp32 partial sums (split > 1)
    uint32_t ksteps;              // total K-steps = ceil(K / 64)
    uint32_t ksteps_per_split;
};

// B element after the transform, as bf16 bits.
template <int V_T, bool SQUARE, bool HAS_SCALE>
__device__ __forceinline__ uint32_t b_elem(uint32_t raw, float k, float s2b)
{
    uint32_t x;
    if constexpr (SQUARE) {
        if constexpr (V_T == DT_BF16) {
            const float v = bf16_to_f32(raw);
            x = f32_to_bf16(bf16_to_f32(f32_to_bf16(k * v)) * v);
        } else {
            const float v = fp8_to_f32<V_T>(raw);
            x = f32_to_bf16((k * v) * v);
        }
        if constexpr (HAS_SCALE) x = f32_to_bf16(bf16_to_f32(x) * s2b);
    } else {
        x = raw;   // bf16 storage only
    }
    return x;
}

// Two transposing 64-bit LDS reads -> one 8 x bf16 MFMA operand fragment:
// lane gets rows k0..k0+7 of column (n0 + lane%16) of a row-major LDS tile.
__device__ __forceinline__ bf16x8_t tr_frag(const uint16_t* tile, int pitch, int k0, int n0, int j)
{
    const uint16_t* p = tile + (k0 + (j >> 2)) * pitch + n0 + 4 * (j & 3);
    typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 4 * pitch));
    // whole-vector shuffle + bit cast: element-wise __bf16 accesses of the
    // loaded vectors are not what the MFMA operand needs here
    const i16x8_t r = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8_t, r);
}

template <int V_T, bool SQUARE, bool HAS_SCALE>
__global__ __launch_bounds__(kGThreads, 1) void gemm_cb_kernel(GemmArgs a)
{
    constexpr int VB = V_T == DT_BF16 ? 2 : 1;
    constexpr int EPS = 16 / VB;

    __shared__ __align__(16) uint16_t A_s[2][kGK * kAP];
    __shared__ __align__(16) uint16_t B_s[2][kGK * kBP];
    __shared__ __align__(16) uint4 run_s[kRunSlots];
    __shared__ uint64_t bm_s[64];
    __shared__ uint32_t rowpre_s[64];
    __shared__ uint32_t pre_s[2][kMaxSteps];
    __shared__ int run_meta_s[2];   // phase of the staged run

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t nt = blockIdx.x;
    const int64_t m0 = (int64_t)blockIdx.y * kGM;
    const uint32_t kt0 = blockIdx.z * a.ksteps_per_split;
    const uint32_t kt1 = min(a.ksteps, kt0 + a.ksteps_per_split);
    const int nsteps = kt1 > kt0 ? (int)(kt1 - kt0) : 0;
    const int64_t vo = a.vals_offset ? *a.vals_offset : 0;
    float s2b = 1.0f;
    if constexpr (HAS_SCALE) {
        const float s = *a.b_scale;
        s2b = bf16_to_f32(f32_to_bf16(s * s));
    }
    const bool a_vec = (a.M % 8 == 0) && (a.ldat % 8 == 0) && ((((uintptr_t)a.At) & 15) == 0);

    // prefixes of every tile this workgroup visits
    for (int s = tid; s < nsteps; s += kGThreads) {
        const size_t t = (size_t)(kt0 + s) * a.grid_n + nt;
        pre_s[0][s] = a.prefix[t];
        pre_s[1][s] = a.prefix[t + 1];
    }
    __syncthreads();

    // ---- register stage of one K-step
    uint4 areg[8];          // At rows: chunk c = i*256 + tid -> row c/32, 8 m at (c%32)*8
    uint64_t bmreg = 0;     // bitmask row `lane` (wave 0)
    uint4 rreg[3];          // value-run slots tid, tid+256, tid+512
    int rphase = 0;

    auto load_step = [&](int s) {
        const uint32_t kt = kt0 + (uint32_t)s;
        const int64_t k0 = (int64_t)kt * kGK;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = i * kGThreads + tid;
            const int64_t k = k0 + (c >> 5);
            const int64_t m = m0 + (c & 31) * 8;
            uint4 v = {0u, 0u, 0u, 0u};
            if (k < a.K && m < a.M) {
                const uint16_t* p = a.At + k * a.ldat + m;
                if (a_vec) {
                    v = *reinterpret_cast<const uint4*>(p);
                } else {
                    uint32_t w[4] = {0u, 0u, 0u, 0u};
                    for (int e = 0; e < 8; e++)
                        if (m + e < a.M) w[e >> 1] |= (uint32_t)p[e] << ((e & 1) * 16);
                    v = uint4{w[0], w[1], w[2], w[3]};
                }
            }
            areg[i] = v;
        }
        const size_t t = (size_t)kt * a.grid_n + nt;
        if (wave == 0) bmreg = reinterpret_cast<const uint64_t*>(a.bitmask + t * kTileBytes)[lane];
        const uint32_t p0 = pre_s[0][s], p1 = pre_s[1][s];
        const int64_t run0 = vo + p0;
        int64_t cnt = (int64_t)p1 - (int64_t)p0;
        cnt = cnt < 0 ? 0 : (cnt > kTileNumel ? kTileNumel : cnt);
        rphase = (int)((((uintptr_t)a.vals) / VB + (uint64_t)run0) % EPS);
        const int nslots = (rphase + (int)cnt + EPS - 1) / EPS;
#pragma unroll
        for (int i = 0; i < 3; i++) {
            const int sl = i * kGThreads + tid;
            uint4 v = {0u, 0u, 0u, 0u};
            if (sl < nslots) {
                const int64_t e0 = run0 - rphase + (int64_t)sl * EPS;
                if (e0 >= 0 && e0 + EPS <= a.vals_numel) {
                    v = *reinterpret_cast<const uint4*>(a.vals + e0 * VB);
                } else {
                    uint32_t w[4] = {0u, 0u, 0u, 0u};
                    for (int e = 0; e < EPS; e++) {
                        const int64_t idx = e0 + e;
                        if (idx >= 0 && idx < a.vals_numel) {
                            const uint32_t x = VB == 2 ? (uint32_t)reinterpret_cast<const uint16_t*>(a.vals)[idx]
                                                       : (uint32_t)a.vals[idx];
                            w[(e * VB) >> 2] |= x << ((e * VB * 8) & 31);
                        }
                    }
                    v = uint4{w[0], w[1], w[2], w[3]};
                }
            }
            rreg[i] = v;
        }
    };
    // registers -> LDS (A into buffer `buf`, run + bitmask rows + row prefixes)
    auto store_step = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = i * kGThreads + tid;
            *reinterpret_cast<uint4*>(&A_s[buf][(c >> 5) * kAP + (c & 31) * 8]) = areg[i];
        }
#pragma unroll
        for (int i = 0; i < 3; i++) {
            const int sl = i * kGThreads + tid;
            if (sl < kRunSlots) run_s[sl] = rreg[i];
        }
        if (wave == 0) {
            const uint32_t c = (uint32_t)__popcll(bmreg);
            uint32_t x = c;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t y = __shfl_up(x, o, 64);
                if (lane >= o) x += y;
            }
            bm_s[lane] = bmreg;
            rowpre_s[lane] = x - c;
            if (lane == 0) run_meta_s[0] = rphase;
        }
    };
    // decode the staged tile row-wise into B_s[buf][k][n]
    auto decode_step = [&](int buf) {
        const int phase = run_meta_s[0];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int b = h * kGThreads + tid;   // chunk: row b/8, columns 8*(b%8)..+7
            const int k = b >> 3, n0 = (b & 7) * 8;
            const uint64_t mrow = bm_s[k];
            const uint32_t byte = (uint32_t)(mrow >> n0) & 0xffu;
            const uint64_t below = n0 == 0 ? 0ull : (mrow & (~0ull >> (64 - n0)));
            uint32_t r = (uint32_t)phase + rowpre_s[k] + (uint32_t)__popcll(below);
            uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                uint32_t x = 0;
                if ((byte >> e) & 1u) {
                    const uint32_t raw = VB == 2 ? (uint32_t)reinterpret_cast<const uint16_t*>(run_s)[r]
                                                 : (uint32_t)reinterpret_cast<const uint8_t*>(run_s)[r];
                    x = b_elem<V_T, SQUARE, HAS_SCALE>(raw, a.relu2_scale, s2b);
                    r++;
                } else if constexpr (HAS_SCALE) {
                    x = f32_to_bf16(0.0f * s2b);
                }
                w[e >> 1] |= x << ((e & 1) * 16);
            }
            *reinterpret_cast<uint4*>(&B_s[buf][k * kBP + n0]) = uint4{w[0], w[1], w[2], w[3]};
        }
    };

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    if (nsteps > 0) {
        load_step(0);
        store_step(0);
        __syncthreads();
        decode_step(0);
        if (nsteps > 1) load_step(1);
        __syncthreads();
        const int g = lane >> 4, j = lane & 15;
        for (int s = 0; s < nsteps; s++) {
            const int cur = s & 1, nxt = cur ^ 1;
            if (s + 1 < nsteps) store_step(nxt);
            __syncthreads();   // B1: step s+1 staged
            if (s + 2 < nsteps) load_step(s + 2);
            if (s + 1 < nsteps) decode_step(nxt);
            // ---- MFMA on step s: wave rows [64*wave, +64) x 64 columns
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const int k0 = kk * 16 + 8 * (g >> 1);
                bf16x8_t af[2], bfr[2];
#pragma unroll
                for (int i = 0; i < 2; i++)
                    af[i] = tr_frag(A_s[cur], kAP, k0, wave * 64 + i * 32 + 16 * (g & 1), j);
#pragma unroll
                for (int jj = 0; jj < 2; jj++)
                    bfr[jj] = tr_frag(B_s[cur], kBP, k0, jj * 32 + 16 * (g & 1), j);
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int jj = 0; jj < 2; jj++)
                        acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[jj], acc[i][jj], 0, 0, 0);
            }
            __syncthreads();   // B2: buffers swap
        }
    }

    // ---- epilogue: lane l, element r of a 32x32 block sits at
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32
    const int64_t n0 = (int64_t)nt * kGN;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int jj = 0; jj < 2; jj++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t row = m0 + wave * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int64_t col = n0 + jj * 32 + (lane & 31);
                if (row < a.M && col < a.N) {
                    if (a.part)
                        a.part[((int64_t)blockIdx.z * a.M + row) * a.N + col] = acc[i][jj][r];
                    else
                        a.C[row * a.N + col] = (uint16_t)f32_to_bf16(acc[i][jj][r]);
                }
            }
}

// C = bf16(sum over splits of part), summed in split order.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* part, int split, int64_t n,
                                                            uint16_t* C)
{
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
        float s = 0.0f;
        for (int k = 0; k < split; k++) s += part[(int64_t)k * n + i];
        C[i] = (uint16_t)f32_to_bf16(s);
    }
}

static int gemm_split(int64_t M, int64_t N, int64_t K)
{
    const int64_t base = ((N + kGN - 1) / kGN) * ((M + kGM - 1) / kGM);
    const int64_t ksteps = (K + kGK - 1) / kGK;
    int64_t split = (256 + base - 1) / base;       // at least one workgroup per CU
    if (split > ksteps / 8) split = ksteps / 8;    // keep >= 8 steps per workgroup
    if (split < 1) split = 1;
    const int64_t min_split = (ksteps + kMaxSteps - 1) / kMaxSteps;
    if (split < min_split) split = min_split;
    return (int)split;
}

}  // namespace bs

using namespace bs;

extern "C" int64_t bs_gemm_compressed_b_workspace_bytes(int64_t M, int64_t N, int64_t K)
{
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    const int split = gemm_split(M, N, K);
    return split > 1 ? (int64_t)split * M * N * 4 : 0;
}

extern "C" int bs_gemm_compressed_b(const void* At, int64_t M, int64_t K, int64_t ldat, const void* vals,
                                    int vals_dtype, int64_t vals_numel, const uint8_t* bitmask,
                                    const uint32_t* prefix, const int64_t* vals_offset, int64_t N,
                                    int square, float relu2_scale, const float* b_scale, void* C,
                                    void* workspace, int64_t workspace_bytes, void* stream)
{
    clear_error();
    if (M < 0 || N < 0 || K < 0) return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: negative shape");
    if (vals_dtype < 0 || vals_dtype > 2) return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: bad dtype");
    if (!square && vals_dtype != DT_BF16)
        return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: fp8 storage needs square=1");
    if (b_scale != nullptr && !square)
        return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: b_scale is only applied with square=1");
    if (ldat < M) return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: ldat < M");
    if ((uint64_t)K * (uint64_t)N >= (1ull << 32))
        return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: K*N must be < 2^32");
    if (M == 0 || N == 0) return BS_OK;
    if (At == nullptr || C == nullptr || bitmask == nullptr || prefix == nullptr ||
        (vals_numel > 0 && vals == nullptr))
        return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: null pointer");
    if ((((uintptr_t)At) & 1) || (((uintptr_t)C) & 1))
        return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: At / C misaligned");
    const int vb = vals_dtype == DT_BF16 ? 2 : 1;
    if (((uintptr_t)vals) % vb) return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: vals misaligned");
    hipStream_t st = (hipStream_t)stream;
    GemmArgs g{};
    g.At = (const uint16_t*)At;
    g.M = M;
    g.K = K;
    g.ldat = ldat;
    g.vals = (const uint8_t*)vals;
    g.vals_numel = vals_numel;
    g.bitmask = bitmask;
    g.prefix = prefix;
    g.vals_offset = vals_offset;
    g.N = N;
    g.grid_n = (uint32_t)((N + 63) / 64);
    g.relu2_scale = relu2_scale;
    g.b_scale = b_scale;
    g.C = (uint16_t*)C;
    g.ksteps = (uint32_t)((K + kGK - 1) / kGK);
    if (g.ksteps == 0) {
        hipError_t e = hipMemsetAsync(C, 0, (size_t)M * N * 2, st);
        return e == hipSuccess ? BS_OK : set_error(BS_ERR_HIP, "bs_gemm_compressed_b: %s", hipGetErrorString(e));
    }
    const int split = gemm_split(M, N, K);
    if (split > 1) {
        const int64_t need = (int64_t)split * M * N * 4;
        if (workspace == nullptr || workspace_bytes < need)
            return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: workspace too small (%lld < %lld)",
                             (long long)workspace_bytes, (long long)need);
        if (((uintptr_t)workspace) & 15) return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: workspace misaligned");
        g.part = (float*)workspace;
    }
    g.ksteps_per_split = (g.ksteps + split - 1) / split;
    if (g.ksteps_per_split > (uint32_t)kMaxSteps)
        return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: internal split error");
    dim3 grid(g.grid_n, (uint32_t)((M + kGM - 1) / kGM), (uint32_t)split);
#define BS_GEMM_LAUNCH(VT, SQ, SC) \
    hipLaunchKernelGGL((gemm_cb_kernel<VT, SQ, SC>), grid, dim3(kGThreads), 0, st, g)
    const bool sc = b_scale != nullptr;
    switch (vals_dtype) {
    case DT_BF16:
        if (!square) BS_GEMM_LAUNCH(DT_BF16, false, false);
        else if (!sc) BS_GEMM_LAUNCH(DT_BF16, true, false);
        else BS_GEMM_LAUNCH(DT_BF16, true, true);
        break;
    case DT_E4M3FN:
        if (!sc) BS_GEMM_LAUNCH(DT_E4M3FN, true, false);
        else BS_GEMM_LAUNCH(DT_E4M3FN, true, true);
        break;
    default:
        if (!sc) BS_GEMM_LAUNCH(DT_E5M2, true, false);
        else BS_GEMM_LAUNCH(DT_E5M2, true, true);
        break;
    }
#undef BS_GEMM_LAUNCH
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && split > 1) {
        const int64_t n = M * N;
        int64_t blocks = (n + 255) / 256;
        if (blocks > 4096) blocks = 4096;
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3((uint32_t)blocks), dim3(256), 0, st,
                           (const float*)workspace, split, n, (uint16_t*)C);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_gemm_compressed_b launch: %s", hipGetErrorString(e));
    return BS_OK;
}
