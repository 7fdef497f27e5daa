// Reconstruct-into-LDS MFMA GEMM for gfx950:  C[M, N] = A[M, K] @ B[K, N]
// where B is a compressed activation (64x64-tile bitmask + prefix + values)
// and is never written to HBM in dense form.
//
// Replaces the "decompress B to HBM, then library GEMM" of the reference's
// AspB / AspRelu2B (lib_sparse/src/sparse_matmul.py:24-28, :109-113).  In the
// MLP backward, A = dY^T (d_out x tokens, made k-contiguous by the caller),
// B = h (tokens x d_ff), C = dW2 (d_out x d_ff).
//
// Per workgroup (256 threads = 4 waves): a 256 x 64 tile of C.  Each K-step
// covers one compressed tile of B (64 tokens x 64 columns):
//   * A rows [m0, m0+256) x 64 k go global -> registers -> LDS (k-contiguous);
//   * the B tile's bitmask rows, row prefixes and value run are staged in LDS
//     and decoded column-wise, so every thread writes 8 consecutive k of one
//     column as one 16-byte LDS store: B_s is k-contiguous, which is the
//     operand layout of v_mfma_f32_32x32x16_bf16;
//   * each wave runs 2 x 2 MFMA 32x32x16 blocks per 16-k slice (64 rows x 64
//     columns of C per wave).
// The next K-step's A rows, bitmask and value run are loaded into registers
// before the MFMAs of the current step, so their latency hides behind them.
// Small grids split K; the partial sums are reduced in a fixed order.
#include "bs_device.h"
#include "bs_host.h"

namespace bs {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kGM = 256;          // C rows per workgroup
constexpr int kGN = 64;           // C columns per workgroup (one B tile column)
constexpr int kGK = 64;           // K per step (one B tile row)
constexpr int kGThreads = 256;
constexpr int kPitch = kGK + 8;   // LDS row pitch in bf16 elements (144 bytes)
constexpr int kRunSlots = 4096 / 8 + 2;   // bf16 value run of one tile, 16-byte slots

struct GemmArgs {
    const uint16_t* A;            // [M, K] bf16, row stride lda (k-contiguous)
    int64_t M, K, lda;
    const uint8_t* vals;          // compressed B
    int64_t vals_numel;
    const uint8_t* bitmask;
    const uint32_t* prefix;
    const int64_t* vals_offset;
    int64_t N;
    uint32_t grid_n;              // B tiles along N
    float relu2_scale;
    const float* b_scale;         // square + fp8 storage: multiply by bf16(scale^2)
    uint16_t* C;                  // [M, N] bf16 (split == 1)
    float* part;                  // [split, M, N] fp32 partial sums (split > 1)
    uint32_t ksteps;              // total K-steps = ceil(K / 64)
    uint32_t ksteps_per_split;
};

// Value of B after the element transform, as bf16 bits (0 for an unset bit).
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

template <int V_T, bool SQUARE, bool HAS_SCALE>
__global__ __launch_bounds__(kGThreads, 2) void gemm_cb_kernel(GemmArgs a)
{
    constexpr int VB = V_T == DT_BF16 ? 2 : 1;
    constexpr int EPS = 16 / VB;

    __shared__ __align__(16) uint16_t A_s[kGM * kPitch];
    __shared__ __align__(16) uint16_t B_s[kGN * kPitch];
    __shared__ uint64_t bm_s[64];
    __shared__ uint32_t rowpre_s[64];
    __shared__ __align__(16) uint4 run_s[kRunSlots];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t nt = blockIdx.x;
    const int64_t m0 = (int64_t)blockIdx.y * kGM;
    const uint32_t kt0 = blockIdx.z * a.ksteps_per_split;
    const uint32_t kt1 = min(a.ksteps, kt0 + a.ksteps_per_split);
    const int64_t vo = a.vals_offset ? *a.vals_offset : 0;
    float s2b = 1.0f;
    if constexpr (HAS_SCALE) {
        const float s = *a.b_scale;
        s2b = bf16_to_f32(f32_to_bf16(s * s));
    }
    const bool a_vec = (a.K % 8 == 0) && (a.lda % 8 == 0) && ((((uintptr_t)a.A) & 15) == 0);

    // ---- register stage of one K-step
    uint4 areg[8];          // A: chunk c = i*256 + tid -> row c/8, 8 k at (c%8)*8
    uint64_t bmreg = 0;     // bitmask row `lane` (wave 0)
    uint4 rreg[3];          // value-run slots tid, tid+256, tid+512
    int rphase = 0, rcount = 0;

    auto load_a = [&](uint32_t kt) {
        const int64_t k0 = (int64_t)kt * kGK;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = i * kGThreads + tid;
            const int64_t row = m0 + (c >> 3);
            const int64_t k = k0 + (c & 7) * 8;
            uint4 v = {0u, 0u, 0u, 0u};
            if (row < a.M && k < a.K) {
                const uint16_t* p = a.A + row * a.lda + k;
                if (a_vec) {
                    v = *reinterpret_cast<const uint4*>(p);
                } else {
                    uint32_t w[4] = {0u, 0u, 0u, 0u};
                    for (int e = 0; e < 8; e++)
                        if (k + e < a.K) w[e >> 1] |= (uint32_t)p[e] << ((e & 1) * 16);
                    v = uint4{w[0], w[1], w[2], w[3]};
                }
            }
            areg[i] = v;
        }
    };
    auto load_b = [&](uint32_t kt, uint32_t p0, uint32_t p1) {
        const size_t t = (size_t)kt * a.grid_n + nt;
        if (wave == 0) bmreg = reinterpret_cast<const uint64_t*>(a.bitmask + t * kTileBytes)[lane];
        const int64_t run0 = vo + p0;
        int64_t cnt = (int64_t)p1 - (int64_t)p0;
        cnt = cnt < 0 ? 0 : (cnt > kTileNumel ? kTileNumel : cnt);
        rphase = (int)((((uintptr_t)a.vals) / VB + (uint64_t)run0) % EPS);
        rcount = (int)cnt;
        const int nslots = (rphase + rcount + EPS - 1) / EPS;
#pragma unroll
        for (int i = 0; i < 3; i++) {
            const int s = i * kGThreads + tid;
            uint4 v = {0u, 0u, 0u, 0u};
            if (s < nslots) {
                const int64_t e0 = run0 - rphase + (int64_t)s * EPS;
                if (e0 >= 0 && e0 + EPS <= a.vals_numel) {
                    v = *reinterpret_cast<const uint4*>(a.vals + e0 * VB);
                } else {
                    uint32_t w[4] = {0u, 0u, 0u, 0u};
                    for (int e = 0; e < EPS; e++) {
                        const int64_t idx = e0 + e;
                        if (idx >= 0 && idx < a.vals_numel) {
                            const uint32_t x = VB == 2 ? (uint32_t)reinterpret_cast<const uint16_t*>(a.vals)[idx]
                                                       : (uint32_t)a.vals[idx];
                            const int sh = (e * VB * 8) & 31;
                            w[(e * VB) >> 2] |= x << sh;
                        }
                    }
                    v = uint4{w[0], w[1], w[2], w[3]};
                }
            }
            rreg[i] = v;
        }
    };

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    if (kt0 < kt1) {
        uint32_t pc0 = a.prefix[(size_t)kt0 * a.grid_n + nt];
        uint32_t pc1 = a.prefix[(size_t)kt0 * a.grid_n + nt + 1];
        load_a(kt0);
        load_b(kt0, pc0, pc1);
        for (uint32_t kt = kt0; kt < kt1; kt++) {
            // ---- registers -> LDS
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int c = i * kGThreads + tid;
                *reinterpret_cast<uint4*>(&A_s[(c >> 3) * kPitch + (c & 7) * 8]) = areg[i];
            }
#pragma unroll
            for (int i = 0; i < 3; i++) {
                const int s = i * kGThreads + tid;
                if (s < kRunSlots) run_s[s] = rreg[i];
            }
            const int phase = rphase;
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
            }
            __syncthreads();
            // ---- decode the B tile column-wise into B_s[n][k]
            {
                const int n = tid & 63;
                const uint64_t below = (n == 0) ? 0ull : (~0ull >> (64 - n));
#pragma unroll
                for (int half = 0; half < 2; half++) {
                    const int kc = (tid >> 6) + 4 * half;   // 8-row group
                    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        const int r = kc * 8 + i;
                        const uint64_t mrow = bm_s[r];
                        uint32_t x = 0;
                        if ((mrow >> n) & 1ull) {
                            const uint32_t rank = rowpre_s[r] + (uint32_t)__popcll(mrow & below);
                            const uint32_t li = (uint32_t)phase + rank;
                            const uint32_t raw = VB == 2 ? (uint32_t)reinterpret_cast<const uint16_t*>(run_s)[li]
                                                         : (uint32_t)reinterpret_cast<const uint8_t*>(run_s)[li];
                            x = b_elem<V_T, SQUARE, HAS_SCALE>(raw, a.relu2_scale, s2b);
                        } else if constexpr (HAS_SCALE) {
                            x = f32_to_bf16(0.0f * s2b);
                        }
                        w[i >> 1] |= x << ((i & 1) * 16);
                    }
                    *reinterpret_cast<uint4*>(&B_s[n * kPitch + kc * 8]) = uint4{w[0], w[1], w[2], w[3]};
                }
            }
            __syncthreads();
            // ---- prefetch the next K-step while the MFMAs run
            if (kt + 1 < kt1) {
                const uint32_t pn0 = a.prefix[(size_t)(kt + 1) * a.grid_n + nt];
                const uint32_t pn1 = a.prefix[(size_t)(kt + 1) * a.grid_n + nt + 1];
                load_a(kt + 1);
                load_b(kt + 1, pn0, pn1);
            }
            // ---- MFMA: wave rows [64*wave, +64) x 64 columns, 4 slices of 16 k
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const int k = kk * 16 + (lane >> 5) * 8;
                bf16x8_t af[2], bfr[2];
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const int row = wave * 64 + i * 32 + (lane & 31);
                    af[i] = *reinterpret_cast<const bf16x8_t*>(&A_s[row * kPitch + k]);
                }
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int n = j * 32 + (lane & 31);
                    bfr[j] = *reinterpret_cast<const bf16x8_t*>(&B_s[n * kPitch + k]);
                }
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
            }
            __syncthreads();
        }
    }

    // ---- epilogue: lane l, element r of a 32x32 block sits at
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32
    const int64_t n0 = (int64_t)nt * kGN;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t row = m0 + wave * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int64_t col = n0 + j * 32 + (lane & 31);
                if (row < a.M && col < a.N) {
                    if (a.part)
                        a.part[((int64_t)blockIdx.z * a.M + row) * a.N + col] = acc[i][j][r];
                    else
                        a.C[row * a.N + col] = (uint16_t)f32_to_bf16(acc[i][j][r]);
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

}  // namespace bs

using namespace bs;

extern "C" int64_t bs_gemm_compressed_b_workspace_bytes(int64_t M, int64_t N, int64_t K)
{
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    const int64_t base = ((N + kGN - 1) / kGN) * ((M + kGM - 1) / kGM);
    const int64_t ksteps = (K + kGK - 1) / kGK;
    int64_t split = (512 + base - 1) / base;
    if (split > ksteps / 4) split = ksteps / 4;
    if (split < 1) split = 1;
    return split > 1 ? split * M * N * 4 : 0;
}

extern "C" int bs_gemm_compressed_b(const void* A, int64_t M, int64_t K, int64_t lda, const void* vals,
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
    if (lda < K) return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: lda < K");
    if ((uint64_t)K * (uint64_t)N >= (1ull << 32))
        return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: K*N must be < 2^32");
    if (M == 0 || N == 0) return BS_OK;
    if (A == nullptr || C == nullptr || bitmask == nullptr || prefix == nullptr ||
        (vals_numel > 0 && vals == nullptr))
        return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: null pointer");
    if ((((uintptr_t)A) & 1) || (((uintptr_t)C) & 1))
        return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: A / C misaligned");
    const int vb = vals_dtype == DT_BF16 ? 2 : 1;
    if (((uintptr_t)vals) % vb) return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: vals misaligned");
    hipStream_t st = (hipStream_t)stream;
    GemmArgs g{};
    g.A = (const uint16_t*)A;
    g.M = M;
    g.K = K;
    g.lda = lda;
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
    const int64_t need = bs_gemm_compressed_b_workspace_bytes(M, N, K);
    int split = 1;
    if (need > 0) {
        split = (int)(need / (M * N * 4));
        if (workspace == nullptr || workspace_bytes < need)
            return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: workspace too small (%lld < %lld)",
                             (long long)workspace_bytes, (long long)need);
        if (((uintptr_t)workspace) & 15) return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: workspace misaligned");
        g.part = (float*)workspace;
    }
    g.ksteps_per_split = (g.ksteps + split - 1) / split;
    if (g.ksteps == 0) {
        hipError_t e = hipMemsetAsync(C, 0, (size_t)M * N * 2, st);
        return e == hipSuccess ? BS_OK : set_error(BS_ERR_HIP, "bs_gemm_compressed_b: %s", hipGetErrorString(e));
    }
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
