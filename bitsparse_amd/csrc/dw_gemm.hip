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
// Workgroup = 512 threads in two roles, output tile 256 (M) x 128 (N), one
// K-step = one row of compressed B tiles (64 tokens, two tiles wide):
//   * waves 0-3 (consumers) run the MFMAs, each on a 128 x 64 block of C
//     (4 x 2 v_mfma_f32_32x32x16_bf16 accumulators);
//   * waves 4-7 (producers) stage dY rows into LDS, stage the compressed
//     value runs, and decode B row by row into LDS (one 16-byte store per
//     bitmask byte), one step ahead of the consumers.
// Two waves share each SIMD, so the producers' VALU/LDS work issues while
// the consumers' MFMAs execute.  Both operands stay in their natural
// k-outer layout in LDS; the k-contiguous MFMA fragments are read with
// ds_read_b64_tr_b16.  Everything is double-buffered and one barrier per
// K-step orders producers and consumers.
//
// Launch order: workgroups are dispatched round-robin over the 8 XCDs, so
// the linear workgroup id is remapped to give each XCD a contiguous range of
// output tiles (N fastest): the workgroups resident on one XCD share their
// dY rows, which then stay in that XCD's L2.
#include "bs_device.h"
#include "bs_host.h"

namespace bs {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBM = 256;              // C rows per workgroup
constexpr int kBN = 128;              // C columns per workgroup (two B tiles)
constexpr int kBK = 64;               // K per step (one B tile row)
constexpr int kThreads = 512;
constexpr int kProducer0 = 256;       // first producer thread
#ifndef BS_GEMM_AP
#define BS_GEMM_AP (kBM + 32)
#endif
#ifndef BS_GEMM_BP
#define BS_GEMM_BP (kBN + 32)
#endif
// Row pitches are 64 bytes past a multiple of 256 (LDS has 64 4-byte banks):
// the four rows read by one 16-lane group of ds_read_b64_tr_b16 then start
// 16 banks apart and the two column halves of a 32-lane half-wave fill the
// other 8-bank gaps, so fragment reads are conflict-free.
constexpr int kAP = BS_GEMM_AP;       // A_s row pitch (elements): 576 bytes
constexpr int kBP = BS_GEMM_BP;       // B_s row pitch (elements): 320 bytes
constexpr int kRunSlots = kTileNumel / 8 + 2;   // one tile's value run + phase, 16-byte slots
constexpr int kMaxSteps = 256;        // K-steps per workgroup (prefixes held in LDS)
constexpr int kCus = 256;             // MI355X compute units (split-K sizing)
constexpr int kXcds = 8;

// LDS carve-up (bytes)
constexpr int kOffA = 0;                                   // A_s[2][64][kAP] bf16
constexpr int kOffB = kOffA + 2 * kBK * kAP * 2;           // B_s[2][64][kBP] bf16
constexpr int kOffRun = kOffB + 2 * kBK * kBP * 2;         // run_s[2][2 tiles][kRunSlots] uint4
constexpr int kOffBm = kOffRun + 2 * 2 * kRunSlots * 16;   // bm_s[2][2][64] uint64
constexpr int kOffRp = kOffBm + 2 * 2 * 64 * 8;           // rp_s[2][2][64] uint32 (row prefixes)
constexpr int kOffMeta = kOffRp + 2 * 2 * 64 * 4;         // meta_s[2][4] int (run phases)
constexpr int kOffLut = kOffMeta + 2 * 4 * 4;             // lut_s[256] uint4 byte-permute selectors
constexpr int kLds = kOffLut + 256 * 16;
// epilogue staging (after the main loop), 128 rows per consumer wave
constexpr int kStF = 64 + 4;          // fp32 staging pitch (floats)
constexpr int kStH = 64 + 8;          // bf16 staging pitch (elements)
static_assert(4 * 128 * kStF * 4 <= kLds, "fp32 staging does not fit");
static_assert(kLds <= 160 * 1024, "LDS budget");

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
    uint32_t tiles_m, tiles_n;    // C tiles (kBM x kBN)
    float relu2_scale;
    const float* b_scale;         // square + fp8 storage: multiply by bf16(scale^2)
    uint16_t* C;                  // [M, N] bf16 (no split)
    float* part;                  // [split, M, N] fp32 partial sums (split > 1)
    uint32_t ksteps;              // total K-steps = ceil(K / 64)
    uint32_t ksteps_per_split;
};

// fp32 -> bf16 bits with the hardware conversion (round to nearest even).
__device__ __forceinline__ uint32_t hw_bf16(float f)
{
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// B element after the transform, as bf16 bits.
template <int V_T, bool SQUARE, bool HAS_SCALE>
__device__ __forceinline__ uint32_t b_elem(uint32_t raw, float k, float s2b)
{
    uint32_t x;
    if constexpr (SQUARE) {
        if constexpr (V_T == DT_BF16) {
            const float v = bf16_to_f32(raw);
            x = hw_bf16(bf16_to_f32(hw_bf16(k * v)) * v);
        } else {
            const float v = V_T == DT_E4M3FN ? __builtin_amdgcn_cvt_f32_fp8(raw, 0)
                                             : __builtin_amdgcn_cvt_f32_bf8(raw, 0);
            x = hw_bf16((k * v) * v);
        }
        if constexpr (HAS_SCALE) x = hw_bf16(bf16_to_f32(x) * s2b);
    } else {
        x = raw;   // bf16 storage only
    }
    return x;
}

// Two transposing 64-bit LDS reads -> one 8 x bf16 MFMA operand fragment:
// lane gets rows k0..k0+7 of column (n0 + lane%16) of a row-major LDS tile.
// Within each 16-lane group ds_read_b64_tr_b16 hands output lane i element
// i%4 of source lanes 4c + i/4 (c = 0..3), so source lane j points at row
// k0 + j/4, columns n0 + 4*(j%4).
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

// Raw buffer access (gfx9 resource word 3 = 0x00020000): reads at or past
// `bytes` return zero instead of touching memory.
typedef __amdgpu_buffer_rsrc_t bs_rsrc;
__device__ __forceinline__ bs_rsrc make_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 load16(bs_rsrc rs, uint32_t off)
{
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, 0));
}
__device__ __forceinline__ uint64_t load8(bs_rsrc rs, uint32_t off)
{
    typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)off, 0, 0);
    return (uint64_t)v[0] | ((uint64_t)v[1] << 32);
}
// 16 bytes at `off` read one element at a time (each element range-checked)
template <int VB>
__device__ __forceinline__ uint4 load16_tail(bs_rsrc rs, uint32_t off)
{
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < 16 / VB; e++) {
        const uint32_t x = VB == 2 ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)(off + 2 * e), 0, 0)
                                   : (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rs, (int)(off + e), 0, 0);
        w[(e * VB) >> 2] |= x << ((e * VB * 8) & 31);
    }
    return uint4{w[0], w[1], w[2], w[3]};
}

// The 4 stored values starting at element r of a run staged in LDS, from
// dword-aligned reads (unaligned LDS reads stall for tens of cycles):
// bf16 -> 8 bytes from three dwords, fp8 -> 4 bytes (in .x) from two.
template <int VB>
__device__ __forceinline__ uint2 window(const uint32_t* run32, uint32_t r)
{
    const uint32_t o = r * VB, q = o >> 2, sh = o & 3;
    const uint32_t d0 = run32[q], d1 = run32[q + 1];
    if constexpr (VB == 2) {
        const uint32_t d2 = run32[q + 2];
        return uint2{__builtin_amdgcn_alignbyte(d1, d0, sh), __builtin_amdgcn_alignbyte(d2, d1, sh)};
    } else {
        return uint2{__builtin_amdgcn_alignbyte(d1, d0, sh), 0u};
    }
}

// compile-time register-set index
template <int P>
struct IC {
    static constexpr int value = P;
};

template <int V_T, bool SQUARE, bool HAS_SCALE>
__global__ __launch_bounds__(kThreads, 1) void gemm_cb_kernel(GemmArgs a)
{
    constexpr int VB = V_T == DT_BF16 ? 2 : 1;
    constexpr int EPS = 16 / VB;                                 // elements per 16-byte slot
    constexpr int RUN_REGS = (kTileNumel / EPS + 2 + 255) / 256; // run slots per producer lane per tile

    __shared__ __align__(16) uint8_t lds[kLds];
    uint16_t* A_s = reinterpret_cast<uint16_t*>(lds + kOffA);
    uint16_t* B_s = reinterpret_cast<uint16_t*>(lds + kOffB);
    uint4* run_s = reinterpret_cast<uint4*>(lds + kOffRun);
    uint64_t* bm_s = reinterpret_cast<uint64_t*>(lds + kOffBm);
    uint32_t* rp_s = reinterpret_cast<uint32_t*>(lds + kOffRp);
    int* meta_s = reinterpret_cast<int*>(lds + kOffMeta);
    uint4* lut_s = reinterpret_cast<uint4*>(lds + kOffLut);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

    // ---- XCD-aware tile order: XCD x runs a contiguous range of tile ids
    const uint32_t nb = gridDim.x, b = blockIdx.x;
    const uint32_t xcd = b % kXcds, q = b / kXcds;
    const uint32_t per = nb / kXcds, rem = nb % kXcds;
    const uint32_t id = xcd * per + min(xcd, rem) + q;
    const uint32_t tn = id % a.tiles_n;
    const uint32_t rest = id / a.tiles_n;
    const uint32_t tm = rest % a.tiles_m;
    const uint32_t split = rest / a.tiles_m;

    const uint32_t nt0 = tn * 2;                       // first B tile column
    const bool two = nt0 + 1 < a.grid_n;               // second B tile exists
    const int64_t m0 = (int64_t)tm * kBM;
    const uint32_t kt0 = split * a.ksteps_per_split;
    const uint32_t kt1 = min(a.ksteps, kt0 + a.ksteps_per_split);
    const int nsteps = kt1 > kt0 ? (int)(kt1 - kt0) : 0;

    // Byte-permute selectors per bitmask byte b.  A chunk's values are read
    // as two windows of 4 stored values: window A from the chunk's first rank
    // (elements 0-3 draw from it), window B from the rank of element 4.
    // Selector byte x picks byte x of the window, 0x0c gives 0x00.
    //   bf16: dword d = elements 2d, 2d+1 (d < 2: window A, else window B)
    //   fp8 : dword h = elements 4h..4h+3 (h = 0: window A, 1: window B)
    if (tid >= kProducer0) {
        const uint32_t b = (uint32_t)(tid - kProducer0);
        uint32_t sel[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint32_t nib = e < 4 ? (b & 15u) : (b >> 4);
            const int ee = e & 3;
            const uint32_t bit = (nib >> ee) & 1u;
            const uint32_t rank = (uint32_t)__builtin_popcount(nib & ((1u << ee) - 1u));
            if constexpr (VB == 2) {
                const uint32_t lo = bit ? 2u * rank : 12u, hi = bit ? 2u * rank + 1u : 12u;
                sel[e >> 1] |= (lo | (hi << 8)) << (16 * (e & 1));
            } else {
                sel[e >> 2] |= (bit ? rank : 12u) << (8 * ee);
            }
        }
        lut_s[b] = uint4{sel[0], sel[1], sel[2], sel[3]};
    }
    __syncthreads();

    f32x16_t acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    // Pipeline (both roles keep two register sets, R = 0, 1, so global loads
    // are issued two steps before their data is stored to LDS).  At the top
    // of iteration s: A_s/B_s[s&1] hold step s; run_s[(s+1)&1] holds run(s+1);
    // consumer set (s+1)&1 holds A(s+1), set s&1 holds A(s+2); producer set
    // s&1 holds run(s+2), set (s+1)&1 holds run(s+3).  Loads past the last
    // step re-read it.  Every global read is a raw buffer load through a
    // wave-uniform resource whose size stops at the operand's end, so
    // out-of-range lanes read zeros without branches.
    const int last = nsteps - 1;
    const IC<0> R0;
    const IC<1> R1;
    if (tid >= kProducer0) {
        // =================== producers: value runs, bitmask, decode ===================
        const int p = tid - kProducer0;                // 0..255
        const int64_t vo = a.vals_offset ? *a.vals_offset : 0;
        float s2b = 1.0f;
        if constexpr (HAS_SCALE) {
            const float sc = *a.b_scale;
            s2b = bf16_to_f32(f32_to_bf16(sc * sc));
        }
        const uint32_t zero_b = HAS_SCALE ? hw_bf16(0.0f * s2b) : 0u;
        const uint32_t zero_pair = zero_b | (zero_b << 16);
        const float kr = a.relu2_scale;
        const bool k_plain = kr >= 0.0f;           // k*0*0 is +0: expanded zeros need no fix-up
        // tile whose bitmask row `lane` this wave loads (two waves per tile)
        const int ub = __builtin_amdgcn_readfirstlane((p >> 6) & 1);

        uint4 rreg[2][2][RUN_REGS];
        int nsl[2][2] = {{0, 0}, {0, 0}};              // slots of the staged runs in rreg
        int phs[2][2] = {{0, 0}, {0, 0}};              // their phases
        uint64_t bmreg[2] = {0ull, 0ull};

        // prefix[t], prefix[t+1], prefix[t+2] of every step this workgroup
        // visits, loaded once: lane l of register w holds step 64*w + l
        // (nsteps <= kMaxSteps = 256); the loop picks them with v_readlane
        uint32_t pq[3][kMaxSteps / 64];
#pragma unroll
        for (int w = 0; w < kMaxSteps / 64; w++) {
            const int st = 64 * w + lane;
            uint32_t v0 = 0u, v1 = 0u, v2 = 0u;
            if (st < nsteps) {
                const size_t t = (size_t)(kt0 + (uint32_t)st) * a.grid_n + nt0;
                v0 = a.prefix[t];
                v1 = a.prefix[t + 1];
                v2 = two ? a.prefix[t + 2] : v1;
            }
            pq[0][w] = v0;
            pq[1][w] = v1;
            pq[2][w] = v2;
        }
        uint32_t pf[3];
        auto load_pre = [&](int s) __attribute__((always_inline)) {
            const int w = s >> 6, l = s & 63;
#pragma unroll
            for (int c = 0; c < 3; c++) {
                const uint32_t x0 = (uint32_t)__builtin_amdgcn_readlane((int)pq[c][0], l);
                const uint32_t x1 = (uint32_t)__builtin_amdgcn_readlane((int)pq[c][1], l);
                const uint32_t x2 = (uint32_t)__builtin_amdgcn_readlane((int)pq[c][2], l);
                const uint32_t x3 = (uint32_t)__builtin_amdgcn_readlane((int)pq[c][3], l);
                pf[c] = w == 0 ? x0 : w == 1 ? x1 : w == 2 ? x2 : x3;
            }
        };
        // value run of tile u of the step whose prefixes are in pf
        // (wave-uniform): 16-byte aligned start e0 (elements), phase = run
        // start - e0, nslots 16-byte slots
        auto run_geom = [&](int u, int64_t& e0, int& phase, int& nslots) __attribute__((always_inline)) {
            const uint32_t p0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(u ? pf[1] : pf[0]));
            const uint32_t p1 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(u ? pf[2] : pf[1]));
            const int64_t run0 = vo + (int64_t)p0;
            int64_t cnt = (int64_t)p1 - (int64_t)p0;
            cnt = cnt < 0 ? 0 : (cnt > kTileNumel ? kTileNumel : cnt);
            phase = (int)(run0 & (EPS - 1));             // vals itself is 16-byte aligned
            e0 = run0 - phase;
            nslots = (phase + (int)cnt + EPS - 1) / EPS;
        };
        // bitmask rows and the 16-byte-aligned value runs of step s's two tiles
        auto load_run = [&](int s, auto R) __attribute__((always_inline)) {
            constexpr int RS = decltype(R)::value;
            const size_t t0 = (size_t)(kt0 + (uint32_t)s) * a.grid_n + nt0;
            {
                const bs_rsrc rs = make_rsrc(a.bitmask + (t0 + ub) * kTileBytes,
                                             (ub == 0 || two) ? (uint32_t)kTileBytes : 0u);
                bmreg[RS] = load8(rs, (uint32_t)lane * 8u);
            }
#pragma unroll
            for (int u = 0; u < 2; u++) {
                int64_t e0;
                int phase, nslots;
                run_geom(u, e0, phase, nslots);
                nsl[RS][u] = nslots;
                phs[RS][u] = phase;
                const int64_t avail = a.vals_numel - e0;        // elements readable from e0
                const bool ok = e0 >= 0 && avail > 0;
                int64_t bytes = ok ? avail * VB : 0;
                if (bytes > (int64_t)nslots * 16) bytes = (int64_t)nslots * 16;
                const bs_rsrc rs = make_rsrc(ok ? a.vals + e0 * VB : a.vals, (uint32_t)bytes);
#pragma unroll
                for (int i = 0; i < RUN_REGS; i++) {
                    const int sl = i * 256 + p;
                    uint4 v = load16(rs, (uint32_t)sl * 16u);
                    // the slot holding the end of `vals` is read element by element
                    if ((int64_t)(sl + 1) * EPS > avail && (int64_t)sl * EPS < avail && sl < nslots)
                        v = load16_tail<VB>(rs, (uint32_t)sl * 16u);
                    rreg[RS][u][i] = v;
                }
            }
            load_pre(min(s + 1, last));
        };
        auto store_run = [&](int buf, auto R) __attribute__((always_inline)) {
            constexpr int RS = decltype(R)::value;
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int i = 0; i < RUN_REGS; i++) {
                    const int sl = i * 256 + p;
                    if (sl < nsl[RS][u]) run_s[(buf * 2 + u) * kRunSlots + sl] = rreg[RS][u][i];
                }
            if (p < 128) {                             // producer waves 0 and 1: one tile each
                // exclusive scan of the row popcounts (0..64, 7 bits) from
                // one ballot per bit: no LDS round trip
                const uint32_t c = (uint32_t)__popcll(bmreg[RS]);
                uint32_t x = 0;
#pragma unroll
                for (int bit = 0; bit < 7; bit++) x += popc_below(__ballot(c & (1u << bit))) << bit;
                bm_s[(buf * 2 + ub) * 64 + lane] = bmreg[RS];
                rp_s[(buf * 2 + ub) * 64 + lane] = x;
                if (lane < 2) meta_s[buf * 4 + lane] = phs[RS][lane];
            }
        };
        // decode step s from run/bitmask buffer rb into B_s[bb]; chunk
        // c = i*256 + p covers row c/16, tile (c/8)%2, 8 columns at 8*(c%8).
        // Each chunk reads two 4-value windows of its tile's staged run and
        // expands them with v_perm_b32 (selectors from lut_s, 0x00 for cleared
        // bits).  All LDS reads of the four chunks precede the writes.
        const int du = (p >> 3) & 1, dn0 = (p & 7) * 8;
        const uint64_t below_mask = dn0 == 0 ? 0ull : (~0ull >> (64 - dn0));
        auto decode = [&](int rb, int bb) __attribute__((always_inline)) {
            const uint32_t* run32 = reinterpret_cast<const uint32_t*>(run_s + (rb * 2 + du) * kRunSlots);
            const uint32_t phu = (uint32_t)meta_s[rb * 4 + du];
            uint64_t mrow[4];
            uint32_t rp[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int k = 16 * i + (p >> 4);
                mrow[i] = bm_s[(rb * 2 + du) * 64 + k];
                rp[i] = rp_s[(rb * 2 + du) * 64 + k];
            }
            uint32_t byte[4];
            uint4 sel[4];
            uint2 wa[4], wb[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                byte[i] = (uint32_t)(mrow[i] >> dn0) & 0xffu;
                const uint32_t ra = phu + rp[i] + (uint32_t)__popcll(mrow[i] & below_mask);
                const uint32_t rbk = ra + (uint32_t)__builtin_popcount(byte[i] & 15u);
                sel[i] = lut_s[byte[i]];
                wa[i] = window<VB>(run32, ra);
                wb[i] = window<VB>(run32, rbk);
            }
            uint16_t* dst = B_s + bb * (kBK * kBP);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t w[4];
                if constexpr (VB == 2) {
                    w[0] = __builtin_amdgcn_perm(wa[i].y, wa[i].x, sel[i].x);
                    w[1] = __builtin_amdgcn_perm(wa[i].y, wa[i].x, sel[i].y);
                    w[2] = __builtin_amdgcn_perm(wb[i].y, wb[i].x, sel[i].z);
                    w[3] = __builtin_amdgcn_perm(wb[i].y, wb[i].x, sel[i].w);
                    if constexpr (SQUARE) {
#pragma unroll
                        for (int d = 0; d < 4; d++)
                            w[d] = b_elem<V_T, SQUARE, HAS_SCALE>(w[d] & 0xffffu, kr, s2b) |
                                   (b_elem<V_T, SQUARE, HAS_SCALE>(w[d] >> 16, kr, s2b) << 16);
                    }
                } else {
                    const uint32_t d0 = __builtin_amdgcn_perm(wa[i].x, wa[i].x, sel[i].x);
                    const uint32_t d1 = __builtin_amdgcn_perm(wb[i].x, wb[i].x, sel[i].y);
#pragma unroll
                    for (int d = 0; d < 4; d++) {
                        const uint32_t src = d < 2 ? d0 : d1;
                        const uint32_t sh = 16 * (d & 1);
                        w[d] = b_elem<V_T, SQUARE, HAS_SCALE>((src >> sh) & 0xffu, kr, s2b) |
                               (b_elem<V_T, SQUARE, HAS_SCALE>((src >> (sh + 8)) & 0xffu, kr, s2b) << 16);
                    }
                }
                if constexpr (SQUARE) {
                    if (!k_plain) {   // negative or NaN k: cleared elements must stay zero_b
#pragma unroll
                        for (int d = 0; d < 4; d++) {
                            const uint32_t keep = (((byte[i] >> (2 * d)) & 1u) ? 0x0000ffffu : 0u) |
                                                  (((byte[i] >> (2 * d + 1)) & 1u) ? 0xffff0000u : 0u);
                            w[d] = (w[d] & keep) | (zero_pair & ~keep);
                        }
                    }
                }
                const int k = 16 * i + (p >> 4);
                *reinterpret_cast<uint4*>(&dst[k * kBP + du * 64 + dn0]) = uint4{w[0], w[1], w[2], w[3]};
            }
        };

        if (nsteps > 0) {
            load_pre(0);
            load_run(0, R0);
            store_run(0, R0);
            load_run(min(1, last), R1);
            load_run(min(2, last), R0);
        }
        __syncthreads();
        if (nsteps > 0) {
            decode(0, 0);
            store_run(1, R1);
            load_run(min(3, last), R1);
        }
        __syncthreads();
        // iteration s (R = register set s&1): the consumers multiply step s
        auto iteration = [&](int s, auto R) __attribute__((always_inline)) {
            constexpr int P = decltype(R)::value;
            store_run(P, R);                              // run(s+2)
            load_run(min(s + 4, last), R);
            if (s + 1 < nsteps) decode(P ^ 1, P ^ 1);     // B(s+1)
            __syncthreads();
        };
        int s = 0;
        for (; s + 1 < nsteps; s += 2) {
            iteration(s, R0);
            iteration(s + 1, R1);
        }
        if (s < nsteps) iteration(s, R0);
    } else {
        // =================== consumers: dY tile and MFMAs ===================
        uint4 areg[2][8];
        // dY rows of step s: chunk c = i*256 + tid -> row c/32, 8 m at (c%32)*8.
        // Rows past K lie outside the resource and read as zero; columns past M
        // only feed C rows that are never stored.
        auto load_a = [&](int s, auto R) __attribute__((always_inline)) {
            const int64_t k0 = (int64_t)(kt0 + (uint32_t)s) * kBK;
            const int64_t rows = a.K - k0 < kBK ? a.K - k0 : kBK;
            const bs_rsrc rs = make_rsrc(a.At + k0 * a.ldat, (uint32_t)(rows * a.ldat * 2));
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int c = i * 256 + tid;
                const uint32_t off = (uint32_t)(((c >> 5) * a.ldat + m0 + (c & 31) * 8) * 2);
                areg[decltype(R)::value][i] = load16(rs, off);
            }
        };
        auto store_a = [&](int buf, auto R) __attribute__((always_inline)) {
            uint16_t* dst = A_s + buf * (kBK * kAP);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int c = i * 256 + tid;
                *reinterpret_cast<uint4*>(&dst[(c >> 5) * kAP + (c & 31) * 8]) = areg[decltype(R)::value][i];
            }
        };
        if (nsteps > 0) {
            load_a(0, R0);
            store_a(0, R0);
            load_a(min(1, last), R1);
            load_a(min(2, last), R0);
        }
        __syncthreads();
        __syncthreads();
        const int wm = wave & 1, wn = wave >> 1;
        const int g = lane >> 4, j = lane & 15;
        auto iteration = [&](int s, auto R) __attribute__((always_inline)) {
            constexpr int P = decltype(R)::value;
            const IC<P ^ 1> Rn;
            const uint16_t* As = A_s + P * (kBK * kAP);
            const uint16_t* Bs = B_s + P * (kBK * kBP);
            // A(s+1) is stored to the other buffer and A(s+3) loaded in
            // quarters between the MFMA blocks
            const int64_t k0n = (int64_t)(kt0 + (uint32_t)min(s + 3, last)) * kBK;
            const int64_t rows_n = a.K - k0n < kBK ? a.K - k0n : kBK;
            const bs_rsrc rs_n = make_rsrc(a.At + k0n * a.ldat, (uint32_t)(rows_n * a.ldat * 2));
            uint16_t* dst_n = A_s + (P ^ 1) * (kBK * kAP);
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const int k0 = kk * 16 + 8 * (g >> 1);
                bf16x8_t af[4], bfr[2];
#pragma unroll
                for (int i = 0; i < 4; i++) af[i] = tr_frag(As, kAP, k0, wm * 128 + i * 32 + 16 * (g & 1), j);
#pragma unroll
                for (int jj = 0; jj < 2; jj++) bfr[jj] = tr_frag(Bs, kBP, k0, wn * 64 + jj * 32 + 16 * (g & 1), j);
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int jj = 0; jj < 2; jj++)
                        acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[jj], acc[i][jj], 0, 0, 0);
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int i = kk * 2 + h;
                    const int c = i * 256 + tid;
                    *reinterpret_cast<uint4*>(&dst_n[(c >> 5) * kAP + (c & 31) * 8]) = areg[P ^ 1][i];
                    areg[P ^ 1][i] = load16(rs_n, (uint32_t)(((c >> 5) * a.ldat + m0 + (c & 31) * 8) * 2));
                }
            }
            __syncthreads();
        };
        int s = 0;
        for (; s + 1 < nsteps; s += 2) {
            iteration(s, R0);
            iteration(s + 1, R1);
        }
        if (s < nsteps) iteration(s, R0);
    }

    // ---- epilogue: consumers stage their 128 x 64 block in LDS, then write
    // rows with 16-byte stores.  Accumulator element r of lane l of a 32x32
    // block sits at row 8*(r/4) + 4*(l/32) + r%4, column l%32.
    __syncthreads();
    const bool consumer = tid < kProducer0;
    const int wm = wave & 1, wn = (wave >> 1) & 1;
    const int64_t row0 = m0 + wm * 128;
    const int64_t col0 = (int64_t)nt0 * 64 + wn * 64;
    const bool out_vec = (a.N % 8 == 0);
    if (a.part) {
        float* st = reinterpret_cast<float*>(lds) + (wave & 3) * (128 * kStF);
        if (consumer) {
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int jj = 0; jj < 2; jj++)
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        st[(i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * kStF + jj * 32 + (lane & 31)] =
                            acc[i][jj][r];
        }
        __syncthreads();
        if (!consumer) return;
        float* dst = a.part + (int64_t)split * a.M * a.N;
        for (int it = 0; it < 32; it++) {
            const int rr = it * 4 + (lane >> 4), c4 = (lane & 15) * 4;
            const int64_t row = row0 + rr, col = col0 + c4;
            if (row >= a.M || col >= a.N) continue;
            const float* s = st + rr * kStF + c4;
            if (out_vec) {
                *reinterpret_cast<float4*>(&dst[row * a.N + col]) = *reinterpret_cast<const float4*>(s);
            } else {
                for (int e = 0; e < 4; e++)
                    if (col + e < a.N) dst[row * a.N + col + e] = s[e];
            }
        }
    } else {
        uint16_t* st = reinterpret_cast<uint16_t*>(lds) + (wave & 3) * (128 * kStH);
        if (consumer) {
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int jj = 0; jj < 2; jj++)
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        st[(i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * kStH + jj * 32 + (lane & 31)] =
                            (uint16_t)hw_bf16(acc[i][jj][r]);
        }
        __syncthreads();
        if (!consumer) return;
        const bool c_vec = out_vec && ((((uintptr_t)a.C) & 15) == 0);
        for (int it = 0; it < 16; it++) {
            const int rr = it * 8 + (lane >> 3), c8 = (lane & 7) * 8;
            const int64_t row = row0 + rr, col = col0 + c8;
            if (row >= a.M || col >= a.N) continue;
            const uint16_t* s = st + rr * kStH + c8;
            if (c_vec) {
                *reinterpret_cast<uint4*>(&a.C[row * a.N + col]) = *reinterpret_cast<const uint4*>(s);
            } else {
                for (int e = 0; e < 8; e++)
                    if (col + e < a.N) a.C[row * a.N + col + e] = s[e];
            }
        }
    }
}

// C = bf16(sum over splits of part), summed in split order; four elements
// per thread with 16-byte partial reads when n % 4 == 0 (scalar tail / path
// otherwise).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* part, int split, int64_t n,
                                                            uint16_t* C)
{
    const int64_t stride = (int64_t)gridDim.x * 256;
    const int64_t n4 = (n % 4 == 0 && (((uintptr_t)part) & 15) == 0 && (((uintptr_t)C) & 7) == 0) ? n / 4 : 0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
        float4 acc = reinterpret_cast<const float4*>(part)[i];
        for (int k = 1; k < split; k++) {
            const float4 v = reinterpret_cast<const float4*>(part + (int64_t)k * n)[i];
            acc.x += v.x;
            acc.y += v.y;
            acc.z += v.z;
            acc.w += v.w;
        }
        const uint32_t lo = f32_to_bf16(acc.x) | (f32_to_bf16(acc.y) << 16);
        const uint32_t hi = f32_to_bf16(acc.z) | (f32_to_bf16(acc.w) << 16);
        reinterpret_cast<uint2*>(C)[i] = uint2{lo, hi};
    }
    for (int64_t i = 4 * n4 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
        float s = 0.0f;
        for (int k = 0; k < split; k++) s += part[(int64_t)k * n + i];
        C[i] = (uint16_t)f32_to_bf16(s);
    }
}

// Split-K factor: fewest "rounds x steps" with one workgroup per CU on kCus
// CUs, a small charge for the partial-sum pass, <= kMaxSteps per workgroup
// and >= 8 steps per workgroup where possible.
static int gemm_split(int64_t M, int64_t N, int64_t K)
{
    const int64_t tiles = ((N + 2 * kTile - 1) / (2 * kTile)) * ((M + kBM - 1) / kBM);
    const int64_t ksteps = (K + kBK - 1) / kBK;
    const int64_t min_split = (ksteps + kMaxSteps - 1) / kMaxSteps;
    int64_t best = min_split, best_cost = -1;
    for (int64_t s = min_split; s <= 64; s++) {
        if (s > min_split && ksteps / s < 8) break;
        const int64_t rounds = (tiles * s + kCus - 1) / kCus;
        const int64_t cost = rounds * ((ksteps + s - 1) / s) + (s > 1 ? 2 : 0);
        if (best_cost < 0 || cost < best_cost) {
            best = s;
            best_cost = cost;
        }
    }
    return (int)best;
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
    if ((((uintptr_t)At) & 15) || (ldat % 8) != 0)
        return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: At must be 16-byte aligned with ldat %% 8 == 0");
    if (ldat >= (1ll << 24)) return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: ldat must be < 2^24");
    if (((uintptr_t)C) & 1) return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: C misaligned");
    if (((uintptr_t)vals) & 15) return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: vals must be 16-byte aligned");
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
    g.grid_n = (uint32_t)((N + kTile - 1) / kTile);
    g.tiles_n = (g.grid_n + 1) / 2;
    g.tiles_m = (uint32_t)((M + kBM - 1) / kBM);
    g.relu2_scale = relu2_scale;
    g.b_scale = b_scale;
    g.C = (uint16_t*)C;
    g.ksteps = (uint32_t)((K + kBK - 1) / kBK);
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
    const uint64_t blocks = (uint64_t)g.tiles_m * g.tiles_n * (uint64_t)split;
    if (blocks >= (1ull << 31)) return set_error(BS_ERR_INVALID, "bs_gemm_compressed_b: grid too large");
#define BS_GEMM_LAUNCH(VT, SQ, SC) \
    hipLaunchKernelGGL((gemm_cb_kernel<VT, SQ, SC>), dim3((uint32_t)blocks), dim3(kThreads), 0, st, g)
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
        int64_t nblk = (n / 4 + 255) / 256;
        if (nblk > 2048) nblk = 2048;
        if (nblk < 1) nblk = 1;
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3((uint32_t)nblk), dim3(256), 0, st,
                           (const float*)workspace, split, n, (uint16_t*)C);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_gemm_compressed_b launch: %s", hipGetErrorString(e));
    return BS_OK;
}
