// Reconstruct-into-LDS MFMA GEMM for gfx950:  C[M, N] = A @ B
// where A is a dense bf16 [M, K] matrix and B is a compressed [K, N]
// activation (64x64-tile bitmask + prefix + values) that is never written to
// HBM in dense form.
//
// Replaces the "decompress B to HBM, then library GEMM" of the reference's
// AspB / AspRelu2B (lib_sparse/src/sparse_matmul.py:24-28, :109-113).  In the
// MLP backward K = tokens, A = dY^T [d_out, tokens], B = h [tokens, d_ff],
// C = dW2 [d_out, d_ff].
//
// Workgroup = 256 threads: four waves, one per SIMD, output tile 256 x 256,
// one K-step = one row of compressed B tiles (64 tokens, four tiles wide).
// Every wave
//   * multiplies a 128 x 128 block of C (4 x 4 v_mfma_f32_32x32x16_bf16
//     accumulators = 256 registers per lane, kept in AGPRs), with its A
//     fragments read straight from global memory: A is consumed k-contiguous
//     (row-major [M, K]; a dY handed over as [K, M] is transposed once into
//     the workspace), so A takes no LDS bandwidth;
//   * decodes one B tile per step into the shared LDS tile: the tile's value
//     run is loaded one step ahead and staged in LDS as bf16, then every
//     8-element chunk is expanded from the run with v_perm_b32 byte selectors.
//     The ReLU^2 square and the fp8 widening are applied once per stored value
//     while the run is staged, not once per expanded element.
// B fragments are read with ds_read_b64_tr_b16 (k-contiguous out of the
// row-major tile).  B is double-buffered; one barrier per K-step.
//
// Launch order: workgroups are dispatched round-robin over the 8 XCDs, so
// the linear workgroup id is remapped to give each XCD a contiguous range of
// output tiles (N fastest): the workgroups resident on one XCD share their
// A rows, which then stay in that XCD's L2.
#include <algorithm>
#include <type_traits>
#include <utility>

#include "bs_device.h"
#include "bs_host.h"
#include "gemm_common.h"

namespace bs {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x8_t __attribute__((ext_vector_type(8)));

constexpr int kRunSlots = kTileNumel / 8 + 2;   // one bf16-staged run + phase, 16-byte slots

// Workgroup shape: a WGM x WGN grid of waves, each owning a WM x WN block of
// C.  A K-step decodes BN/64 B tiles; each is decoded by NWAVES/NT waves.
//   Cfg256: 256 x 256, 4 waves (one per SIMD), 128 x 128 per wave
//   Cfg512: 512 x 128, 8 waves (two per SIMD), 64 x 128 per wave: every
//           decoded B element feeds 512 rows instead of 256, half the decode
//           instructions per MFMA
template <int WGM_, int WGN_, int WM_, int WN_, bool AQ_, int MINB_ = 1>
struct GemmCfg {
    static constexpr int MINB = MINB_;                           // workgroups per CU (launch bound)
    // AQ: A fragments are loaded one k-quarter ahead (2 register sets) instead
    // of one K-step ahead (4 sets); with two waves per SIMD the other wave
    // covers the shorter lead
    static constexpr bool AQ = AQ_;
    static constexpr int ASETS = AQ_ ? 2 : 4;
    static constexpr int WGM = WGM_, WGN = WGN_, NWAVES = WGM_ * WGN_, THREADS = 64 * NWAVES;
    static constexpr int WAVE_M = WM_, WAVE_N = WN_;
    static constexpr int IM = WAVE_M / 32, JN = WAVE_N / 32;    // 32x32 accumulator blocks per wave
    static constexpr int BM = WAVE_M * WGM, BN = WAVE_N * WGN;
    static constexpr int NT = BN / 64;                           // B tiles per K-step
    static constexpr int DW = NWAVES / NT;                       // waves decoding one B tile
    static constexpr int CH = 8 / DW;                            // decode chunk iterations per lane per step
    // B_s row pitch (elements): 64 bytes past a multiple of 256 bytes (LDS has
    // 64 4-byte banks): the four rows read by one 16-lane group of
    // ds_read_b64_tr_b16 start 16 banks apart and the two column halves of a
    // 32-lane half-wave fill the other 8-bank gaps, so fragment reads are
    // conflict-free
    static constexpr int BP = ((BN * 2 + 255) / 256 * 256 + 64) / 2;
    static constexpr int SEG = 4 * IM * JN;                      // MFMAs (segments) per K-step
    static constexpr int PER = SEG / CH;                         // segments per decoded chunk
    // LDS carve-up (bytes)
    static constexpr int OFF_B = 0;                              // B_s[2][64][BP] bf16
    static constexpr int OFF_RUN = OFF_B + 2 * kBK * BP * 2;     // run_s[2][NT][kRunSlots] uint4
    static constexpr int OFF_BM = OFF_RUN + 2 * NT * kRunSlots * 16;   // bm_s[NWAVES][64] uint64
    static constexpr int OFF_RP = OFF_BM + NWAVES * 64 * 8;     // rp_s[NWAVES][64] uint32
    static constexpr int OFF_LUT = OFF_RP + NWAVES * 64 * 4;    // lut_s[256] uint4
    static constexpr int LDS = OFF_LUT + 256 * 16;
    static constexpr int ST_P = WAVE_N + 4;                      // epilogue staging pitch (floats)
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static_assert(NWAVES * 16 * ST_P * 4 <= LDS, "epilogue staging does not fit");
    static_assert(NWAVES % NT == 0 && 8 % DW == 0 && SEG % CH == 0, "decode split");
};
using Cfg256 = GemmCfg<2, 2, 128, 128, false>;
// 8 x 1 waves of 64 x 128: each A row block is read by one wave (a 4 x 2 grid
// of 128 x 64 reads every A block twice and measured 4% slower)
using Cfg512 = GemmCfg<8, 1, 64, 128, false>;
//   Cfg768: 768 x 64, 8 waves (two per SIMD) of 96 x 64: a C tile spans up
//           to 768 rows (the MLP dW shapes with d_out <= 768), so each B tile
//           is decoded once per K-step for all of M; one tile per step, one
//           decoded chunk per lane
using Cfg768 = GemmCfg<8, 1, 96, 64, false>;
//   Cfg256h: 256 x 128, 4 waves of 128 x 64 (2 x 2), two workgroups per CU:
//            with a wave of the other workgroup on every SIMD, the value-run
//            and A loads of one workgroup hide behind the other's MFMAs
//   Cfg256v: 256 x 128, 4 waves of 64 x 128 (4 x 1), two workgroups per CU
using Cfg256h = GemmCfg<2, 2, 128, 64, true, 2>;
using Cfg256v = GemmCfg<4, 1, 64, 128, true, 2>;

struct GemmArgs {
    const uint16_t* Apk;          // A in MFMA-fragment order (pack_a_*_kernel)
    int64_t M, K;
    uint32_t nkb;                 // 16-wide k blocks per 32-row block of Apk
    uint32_t nrb;                 // 32-row blocks of Apk
    const uint8_t* vals;          // compressed B
    int64_t vals_numel;
    const uint8_t* bitmask;
    const uint32_t* prefix;
    const int64_t* vals_offset;
    int64_t N;
    uint32_t grid_n;              // B tiles along N
    uint32_t tiles_m, tiles_n;    // C tiles (BM x BN of the launch configuration)
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
            const float v = V_T == DT_E4M3FN ? __builtin_amdgcn_cvt_f32_fp8(raw, 0)
                                             : __builtin_amdgcn_cvt_f32_bf8(raw, 0);
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

// A staging unit of the value run: 16 bytes (plain bf16 runs), 8 bytes
// (bf16 runs to square) or 4 bytes (fp8 runs).
template <int UB>
using RunUnit = typename std::conditional<UB == 16, uint4,
                                          typename std::conditional<UB == 8, uint2, uint32_t>::type>::type;

template <int UB>
__device__ __forceinline__ RunUnit<UB> load_unit(bs_rsrc rs, uint32_t off)
{
    if constexpr (UB == 16) return load16(rs, off);
    else if constexpr (UB == 8) return load8(rs, off);
    else return load4(rs, off);
}

// The unit at `off` read one element at a time: used for the unit that holds
// the end of `vals`, where a whole-unit read would cross the buffer's end.
template <int UB, int VB>
__device__ __forceinline__ RunUnit<UB> load_unit_tail(bs_rsrc rs, uint32_t off)
{
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < UB / VB; e++) {
        const uint32_t x = VB == 2 ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)(off + 2 * e), 0, 0)
                                   : (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rs, (int)(off + e), 0, 0);
        w[(e * VB) >> 2] |= x << ((e * VB * 8) & 31);
    }
    if constexpr (UB == 16) return uint4{w[0], w[1], w[2], w[3]};
    else if constexpr (UB == 8) return uint2{w[0], w[1]};
    else return w[0];
}

template <typename CFG, int V_T, bool SQUARE, bool HAS_SCALE>
__global__ __launch_bounds__(CFG::THREADS, CFG::MINB) void gemm_cb_kernel(GemmArgs a)
{
    constexpr int NT = CFG::NT, DW = CFG::DW, CH = CFG::CH, BP = CFG::BP, IM = CFG::IM, JN = CFG::JN;
    constexpr int VB = V_T == DT_BF16 ? 2 : 1;                   // stored value bytes
    constexpr int GV = SQUARE ? 4 : 8;                           // values per staging unit
    constexpr int UB = GV * VB;                                  // stored bytes per unit
    constexpr int RX = ((GV - 1 + kTileNumel + GV - 1) / GV + 63) / 64;   // units per lane, worst case
    // units per lane loaded one step ahead (<= 20 registers: 2560 plain bf16
    // values, 1536 bf16 / 1024 fp8 values to square); a denser tile's
    // remaining units are loaded when the run is staged
    // (two workgroups per CU: 2 units, the 50% zeros tile of a plain run,
    // to stay within 256 registers)
    constexpr int RXP0 = CFG::MINB > 1 ? 2 : (UB == 16 ? 5 : (UB == 8 ? 6 : 4));
    // the DW waves decoding one tile stage its run together: unit u is staged
    // by lane u % 64 of wave (u / 64) % DW, in pass u / (64 DW)
    constexpr int RXD = (RX + DW - 1) / DW;                      // passes per wave, worst case
    constexpr int RXP = RXP0 < RXD ? RXP0 : RXD;
    typedef RunUnit<UB> Unit;

    __shared__ __align__(16) uint8_t lds[CFG::LDS];
    uint16_t* B_s = reinterpret_cast<uint16_t*>(lds + CFG::OFF_B);
    uint4* run_s = reinterpret_cast<uint4*>(lds + CFG::OFF_RUN);
    uint64_t* bm_s = reinterpret_cast<uint64_t*>(lds + CFG::OFF_BM);
    uint32_t* rp_s = reinterpret_cast<uint32_t*>(lds + CFG::OFF_RP);
    uint4* lut_s = reinterpret_cast<uint4*>(lds + CFG::OFF_LUT);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // ---- XCD-aware tile order: XCD x runs a contiguous range of tile ids
    const uint32_t nb = gridDim.x, b = blockIdx.x;
    const uint32_t xcd = b % kXcds, q = b / kXcds;
    const uint32_t per = nb / kXcds, rem = nb % kXcds;
    const uint32_t id = xcd * per + min(xcd, rem) + q;
    // the divisions run on the VALU: pin their (uniform) results to SGPRs so
    // the buffer descriptors built from them stay scalar
    const uint32_t tn = (uint32_t)__builtin_amdgcn_readfirstlane((int)(id % a.tiles_n));
    const uint32_t rest = id / a.tiles_n;
    const uint32_t tm = (uint32_t)__builtin_amdgcn_readfirstlane((int)(rest % a.tiles_m));
    const uint32_t split = (uint32_t)__builtin_amdgcn_readfirstlane((int)(rest / a.tiles_m));

    const uint32_t nt0 = tn * NT;                      // first B tile column
    const int tw = wave / DW;                          // the B tile this wave helps decode
    const int tq = wave % DW;                          // its share: rows 64/DW * tq .. +64/DW
    const uint32_t tcol = nt0 + (uint32_t)tw;
    const bool has_tile = tcol < a.grid_n;
    const int64_t m0 = (int64_t)tm * CFG::BM;
    const uint32_t kt0 = split * a.ksteps_per_split;
    const uint32_t kt1 = min(a.ksteps, kt0 + a.ksteps_per_split);
    const int nsteps = kt1 > kt0 ? (int)(kt1 - kt0) : 0;
    const int last = nsteps - 1;

    // Byte-permute selectors per bitmask byte b for a bf16 run.  A chunk's
    // values are read as two windows of 4 values: window A from the chunk's
    // first rank (elements 0-3 draw from it), window B from the rank of
    // element 4.  Selector byte x picks byte x of the window, 0x0c gives 0x00;
    // dword d = elements 2d, 2d+1 (d < 2: window A, else window B).
    if (tid < 256) {
        const uint32_t bb = (uint32_t)tid;
        uint32_t sel[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint32_t nib = e < 4 ? (bb & 15u) : (bb >> 4);
            const int ee = e & 3;
            const uint32_t bit = (nib >> ee) & 1u;
            const uint32_t rank = (uint32_t)__builtin_popcount(nib & ((1u << ee) - 1u));
            const uint32_t lo = bit ? 2u * rank : 12u, hi = bit ? 2u * rank + 1u : 12u;
            sel[e >> 1] |= (lo | (hi << 8)) << (16 * (e & 1));
        }
        lut_s[bb] = uint4{sel[0], sel[1], sel[2], sel[3]};
    }

    // ---- value transform constants (ReLU^2 square, fp8 scale^2)
    float s2b = 1.0f;
    if constexpr (HAS_SCALE) {
        const float sc = *a.b_scale;
        s2b = bf16_to_f32(f32_to_bf16(sc * sc));
    }
    const float kr = a.relu2_scale;
    // a cleared bit decodes to the transform of 0 (+0 unless k < 0, or the
    // scale makes it NaN); the permutes produce +0, fixed up when different
    const uint32_t zero_b = SQUARE ? b_elem<V_T, SQUARE, HAS_SCALE>(0u, kr, s2b) : 0u;
    const uint32_t zero_pair = zero_b | (zero_b << 16);
    const bool zfix = SQUARE && zero_b != 0u;

    // ---- prefix[t], prefix[t+1] of every step of this wave's tile column,
    // loaded once: lane l of register w holds step 64*w + l
    // (nsteps <= kMaxSteps = 256); steps are picked with v_readlane
    uint32_t pq[2][kMaxSteps / 64];
#pragma unroll
    for (int w = 0; w < kMaxSteps / 64; w++) {
        const int st = 64 * w + lane;
        uint32_t v0 = 0u, v1 = 0u;
        if (has_tile && st < nsteps) {
            const size_t t = (size_t)(kt0 + (uint32_t)st) * a.grid_n + tcol;
            v0 = a.prefix[t];
            v1 = a.prefix[t + 1];
        }
        pq[0][w] = v0;
        pq[1][w] = v1;
    }
    const int64_t vo = a.vals_offset ? *a.vals_offset : 0;
    // value run of step s (wave-uniform): GV-aligned start e0 (elements),
    // phase = run start - e0, nunits staging units
    auto run_geom = [&](int s, int64_t& e0, int& phase, int& nunits) __attribute__((always_inline)) {
        const int w = s >> 6, l = s & 63;
        uint32_t p[2];
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const uint32_t x0 = (uint32_t)__builtin_amdgcn_readlane((int)pq[c][0], l);
            const uint32_t x1 = (uint32_t)__builtin_amdgcn_readlane((int)pq[c][1], l);
            const uint32_t x2 = (uint32_t)__builtin_amdgcn_readlane((int)pq[c][2], l);
            const uint32_t x3 = (uint32_t)__builtin_amdgcn_readlane((int)pq[c][3], l);
            p[c] = w == 0 ? x0 : w == 1 ? x1 : w == 2 ? x2 : x3;
        }
        // wave-uniform: 32-bit tests (a 64-bit compare is a vector
        // instruction on this target and takes a VGPR temporary)
        const uint32_t cnt = p[1] >= p[0] ? min(p[1] - p[0], (uint32_t)kTileNumel) : 0u;
        const int64_t run0 = vo + (int64_t)p[0];
        phase = (int)(run0 & (GV - 1));
        e0 = run0 - phase;
        nunits = cnt == 0 ? 0 : (phase + (int)cnt + GV - 1) / GV;
    };

    // ---- run staging: units of step s are loaded into registers one
    // iteration before they are written to LDS
    Unit rr[RXP];
    int rr_nunits = 0;
    uint32_t rr_avail = 0;
    bool rr_tail = false;
    bs_rsrc rr_rs;
    auto unit_at = [&](int u) __attribute__((always_inline)) -> Unit {
        Unit v = load_unit<UB>(rr_rs, (uint32_t)u * UB);
        if (rr_tail && (uint32_t)(u + 1) * GV > rr_avail && (uint32_t)u * GV < rr_avail)
            v = load_unit_tail<UB, VB>(rr_rs, (uint32_t)u * UB);
        return v;
    };
    auto load_run = [&](int s) __attribute__((always_inline)) {
        int64_t e0;
        int phase, nunits;
        run_geom(s, e0, phase, nunits);
        const int64_t avail = a.vals_numel - e0;       // elements readable from e0
        // 64-bit tests by sign and high bits, which stay scalar instructions;
        // avail32 = avail clamped to 2^24 (a run holds at most 4096 elements)
        const bool ok = ((uint64_t)e0 >> 63) == 0 && ((uint64_t)(avail - 1) >> 63) == 0 && nunits > 0;
        const uint32_t avail32 = ((uint64_t)avail >> 24) != 0 ? (1u << 24) : (uint32_t)avail;
        const uint32_t bytes = ok ? min(avail32 * (uint32_t)VB, (uint32_t)nunits * (uint32_t)UB) : 0u;
        rr_nunits = ok ? nunits : 0;
        rr_avail = avail32;
        rr_rs = make_rsrc(ok ? a.vals + e0 * VB : a.vals, bytes);
        rr_tail = ok && (uint32_t)nunits * GV > avail32;   // the run's last unit crosses the end of vals
        // the prefetched passes are issued whatever the run's length (units
        // past it read zeros through the resource's range check): a load
        // skipped on some paths makes the compiler's count of loads in flight
        // a lower bound, and the waits for A would then cover these loads too
#pragma unroll
        for (int x = 0; x < RXP; x++) rr[x] = unit_at((x * DW + tq) * 64 + lane);
    };
    auto store_run = [&](int buf) __attribute__((always_inline)) {
        uint8_t* dst = reinterpret_cast<uint8_t*>(run_s + (buf * NT + tw) * kRunSlots);
#pragma unroll
        for (int x = 0; x < RXD; x++) {
            if ((x * DW + tq) * 64 < rr_nunits) {
                const int u = (x * DW + tq) * 64 + lane;
                if (x >= RXP) rr[x % RXP] = unit_at(u);
                if (u < rr_nunits) {
                    if constexpr (!SQUARE) {
                        *reinterpret_cast<uint4*>(dst + u * 16) = rr[x % RXP];
                    } else {
                        uint32_t y[4];
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            uint32_t raw;
                            const Unit ux = rr[x % RXP];
                            if constexpr (VB == 2) raw = ((e < 2 ? ux.x : ux.y) >> (16 * (e & 1))) & 0xffffu;
                            else raw = (ux >> (8 * e)) & 0xffu;
                            y[e] = b_elem<V_T, SQUARE, HAS_SCALE>(raw, kr, s2b);
                        }
                        *reinterpret_cast<uint2*>(dst + u * 8) = uint2{y[0] | (y[1] << 16), y[2] | (y[3] << 16)};
                    }
                }
            }
        }
    };

    // ---- bitmask rows: lane r holds row r of this wave's tile of step s
    auto load_bm = [&](int s) __attribute__((always_inline)) -> uint64_t {
        const size_t t = (size_t)(kt0 + (uint32_t)s) * a.grid_n + tcol;
        const bs_rsrc rs = make_rsrc(a.bitmask + (has_tile ? t : 0) * kTileBytes,
                                     has_tile ? (uint32_t)kTileBytes : 0u);
        const uint2 v = load8(rs, (uint32_t)lane * 8u);
        return (uint64_t)v.x | ((uint64_t)v.y << 32);
    };

    // ---- decode step s (run in run_s[rb], bitmask rows bmr) into B_s[bb],
    // columns 64*tw .. +64, rows rbase .. rbase + 8 CH.  Lane l handles chunk
    // c = l%8 (8 columns at 8c) of CH rows, row = rbase + 8i + roff(l/8); roff
    // pairs rows two apart in each 16-lane group so the 16-byte stores of a
    // group hit disjoint banks.
    const int dc = lane & 7, dg = lane >> 3;
    const int roff = ((dg & 1) << 1) | ((dg >> 1) & 1) | (dg & 4);
    const uint64_t below_mask = dc == 0 ? 0ull : (~0ull >> (64 - 8 * dc));
    const int rbase = 8 * CH * tq;
    // row table of step s: bm_s = bitmask rows, rp_s = run index of each
    // row's first value (phase + exclusive prefix of the row popcounts)
    auto decode_rows = [&](int s, uint64_t bmr) __attribute__((always_inline)) {
        int64_t e0;
        int phase, nunits;
        run_geom(s, e0, phase, nunits);
        const uint32_t c = (uint32_t)__popcll(bmr);
        const uint32_t rp = wave_incl_scan(c) - c;
        bm_s[wave * 64 + lane] = bmr;
        rp_s[wave * 64 + lane] = rp + (uint32_t)phase;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // The decode of one chunk in three stages (compile-time chunk index C,
    // row 8C + roff), so that the stages of successive chunks can be spread
    // between the MFMAs of the step being multiplied:
    //   stage_r: the row's bitmask word and run index from the row table
    //            (each wave keeps its own copy of its tile's table)
    //   stage_s: ranks; issues the reads of the byte-permute selectors and of
    //            the dwords under the two value windows
    //   stage_w: aligns the windows, permutes and stores 16 bytes into B_s
    struct DecR {
        uint64_t mrow;
        uint32_t rpr;
    };
    struct DecS {
        uint4 sel;
        uint32_t a0, a1, a2, b0, b1, b2;    // dwords under window A / window B
        uint32_t sha, shb;                  // their byte offsets within the first dword
    };
    DecR dr[2];
    DecS dq[2];
    auto stage_r = [&](auto CI) __attribute__((always_inline)) {
        constexpr int C = decltype(CI)::value;
        const int row = rbase + 8 * C + roff;
        dr[C & 1].mrow = bm_s[wave * 64 + row];
        dr[C & 1].rpr = rp_s[wave * 64 + row];
    };
    auto stage_s = [&](auto CI, const uint32_t* run32) __attribute__((always_inline)) {
        constexpr int C = decltype(CI)::value;
        const uint64_t mrow = dr[C & 1].mrow;
        const uint32_t byte = (uint32_t)(mrow >> (8 * dc)) & 0xffu;
        const uint32_t ra = dr[C & 1].rpr + (uint32_t)__popcll(mrow & below_mask);
        const uint32_t rbk = ra + (uint32_t)__builtin_popcount(byte & 15u);
        DecS& q = dq[C & 1];
        q.sel = lut_s[byte];
        const uint32_t qa = ra >> 1, qb = rbk >> 1;     // bf16 value r sits in dword r/2
        q.sha = (ra & 1u) * 2u;
        q.shb = (rbk & 1u) * 2u;
        q.a0 = run32[qa];
        q.a1 = run32[qa + 1];
        q.a2 = run32[qa + 2];
        q.b0 = run32[qb];
        q.b1 = run32[qb + 1];
        q.b2 = run32[qb + 2];
    };
    auto stage_w = [&](auto CI, uint16_t* dst) __attribute__((always_inline)) {
        constexpr int C = decltype(CI)::value;
        const DecS& q = dq[C & 1];
        const uint32_t wax = __builtin_amdgcn_alignbyte(q.a1, q.a0, q.sha);
        const uint32_t way = __builtin_amdgcn_alignbyte(q.a2, q.a1, q.sha);
        const uint32_t wbx = __builtin_amdgcn_alignbyte(q.b1, q.b0, q.shb);
        const uint32_t wby = __builtin_amdgcn_alignbyte(q.b2, q.b1, q.shb);
        const uint32_t w0 = __builtin_amdgcn_perm(way, wax, q.sel.x);
        const uint32_t w1 = __builtin_amdgcn_perm(way, wax, q.sel.y);
        const uint32_t w2 = __builtin_amdgcn_perm(wby, wbx, q.sel.z);
        const uint32_t w3 = __builtin_amdgcn_perm(wby, wbx, q.sel.w);
        *reinterpret_cast<uint4*>(&dst[(rbase + 8 * C + roff) * BP]) = uint4{w0, w1, w2, w3};
    };
    auto run_ptr = [&](int rb) __attribute__((always_inline)) {
        return reinterpret_cast<const uint32_t*>(run_s + (rb * NT + tw) * kRunSlots);
    };
    auto dst_ptr = [&](int bb) __attribute__((always_inline)) {
        return B_s + bb * (kBK * BP) + tw * 64 + dc * 8;
    };
    // whole decode of the run in run_s[rb] into B_s[bb] (prologue)
    auto decode = [&](int rb, int bb) __attribute__((always_inline)) {
        const uint32_t* run32 = run_ptr(rb);
        uint16_t* dst = dst_ptr(bb);
        static_for<CH>([&](auto CI) __attribute__((always_inline)) {
            stage_r(CI);
            stage_s(CI, run32);
            stage_w(CI, dst);
        });
    };

    // cleared elements of B_s[bb] (this wave's columns) -> zero_b
    auto zero_fixup = [&](int bb) __attribute__((always_inline)) {
        uint16_t* dst = dst_ptr(bb);
        for (int i = 0; i < CH; i++) {
            const int row = rbase + 8 * i + roff;
            const uint32_t byte = (uint32_t)(bm_s[wave * 64 + row] >> (8 * dc)) & 0xffu;
            uint4 v = *reinterpret_cast<const uint4*>(&dst[row * BP]);
            uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int d = 0; d < 4; d++) {
                const uint32_t keep = (((byte >> (2 * d)) & 1u) ? 0x0000ffffu : 0u) |
                                      (((byte >> (2 * d + 1)) & 1u) ? 0xffff0000u : 0u);
                w[d] = (w[d] & keep) | (zero_pair & ~keep);
            }
            *reinterpret_cast<uint4*>(&dst[row * BP]) = uint4{w[0], w[1], w[2], w[3]};
        }
    };

    // ---- A fragments: lane (col = l%32, h = l/32) of block i holds row
    // 32i + col, k = 16kk + 8h .. +7 of the step.  Apk stores exactly these
    // 16-byte pieces lane after lane, one 1 KiB block per (32 rows, 16 k), so
    // every fragment load is one contiguous 1 KiB read; rows past M and k past
    // K are zero in Apk, blocks past its end read as zero.
    const int wm = wave % CFG::WGM, wn = wave / CFG::WGM;
    const int g = lane >> 4, j = lane & 15, hh = lane >> 5, col = lane & 31;
    const int64_t arow0 = m0 + wm * CFG::WAVE_M;
    const uint32_t rb0 = (uint32_t)(arow0 / 32);
    const uint32_t nrbw = rb0 < a.nrb ? min((uint32_t)IM, a.nrb - rb0) : 0u;   // row blocks of this wave
    const bs_rsrc rsA = make_rsrc(nrbw ? a.Apk + (int64_t)rb0 * a.nkb * 512 : a.Apk, nrbw * a.nkb * 1024u);
    bf16x8_t areg[IM][CFG::ASETS];   // [i][kk] (whole step) or [i][kk & 1] (AQ)
    auto a_off = [&](int s, int i, int kk) __attribute__((always_inline)) -> uint32_t {
        return ((uint32_t)i * a.nkb + (kt0 + (uint32_t)s) * 4u + (uint32_t)kk) * 1024u + (uint32_t)lane * 16u;
    };
    auto load_a = [&](int s, int kk) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < IM; i++)
            areg[i][kk % CFG::ASETS] = __builtin_bit_cast(bf16x8_t, load16(rsA, a_off(s, i, kk)));
    };

    f32x16_t acc[IM][JN];
#pragma unroll
    for (int i = 0; i < IM; i++)
#pragma unroll
        for (int jj = 0; jj < JN; jj++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][jj][r] = 0.0f;

    // B fragments of one k-quarter: lo / hi halves of the transposing reads,
    // two sets (k-quarter parity)
    i16x4_t blo[2][JN], bhi[2][JN];
    auto read_b = [&](const uint16_t* Bs, int kk, int jj, int half, int set) __attribute__((always_inline)) {
        const uint16_t* p = Bs + (16 * kk + 8 * hh + (j >> 2) + 4 * half) * BP + wn * CFG::WAVE_N + jj * 32 +
                            16 * (g & 1) + 4 * (j & 3);
        typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
        const i16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p);
        if (half) bhi[set][jj] = v;
        else blo[set][jj] = v;
    };

    // One K-step as SEG segments, one MFMA each (k-quarter kk, block i, jj),
    // fenced by sched_barrier so the order below is the issue order.  A
    // segment also carries: the reload of A(i, kk) for the next step after its
    // last use; in the second half of a k-quarter, one transposing read of the
    // next quarter's B fragments; and one stage of the software-pipelined
    // decode of the next step (chunk X/PER: stage_r at X%PER == 0, stage_s
    // half a period later, stage_w at the next chunk's stage_r).  Each segment
    // issues a few VALU / LDS instructions in the shadow of its MFMA.
    auto step = [&](int s_cur, int s_next, auto PI) __attribute__((always_inline)) {
        constexpr int P = decltype(PI)::value;
        constexpr int PER = CFG::PER, QB = IM * JN;    // segments per chunk / per k-quarter
        const uint16_t* Bs = B_s + P * (kBK * BP);
        const uint32_t* run32 = run_ptr(P ^ 1);
        uint16_t* dst = dst_ptr(P ^ 1);
        static_for<JN>([&](auto JI) __attribute__((always_inline)) {
            read_b(Bs, 0, decltype(JI)::value, 0, 0);
            read_b(Bs, 0, decltype(JI)::value, 1, 0);
        });
        static_for<CFG::SEG>([&](auto XI) __attribute__((always_inline)) {
            constexpr int X = decltype(XI)::value;
            constexpr int kk = X / QB, m = X % QB, i = m / JN, jj = m % JN;
            const i16x8_t bw = __builtin_shufflevector(blo[kk & 1][jj], bhi[kk & 1][jj], 0, 1, 2, 3, 4, 5, 6, 7);
            acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(areg[i][kk % CFG::ASETS],
                                                                 __builtin_bit_cast(bf16x8_t, bw), acc[i][jj], 0, 0, 0);
            // after the last use of A(i, kk): reload its register set with the
            // fragment needed ASETS quarters later
            if constexpr (jj == JN - 1) {
                if constexpr (CFG::AQ) {
                    if constexpr (kk < 2)
                        areg[i][kk % 2] = __builtin_bit_cast(bf16x8_t, load16(rsA, a_off(s_cur, i, kk + 2)));
                    else
                        areg[i][kk % 2] = __builtin_bit_cast(bf16x8_t, load16(rsA, a_off(s_next, i, kk - 2)));
                } else {
                    areg[i][kk] = __builtin_bit_cast(bf16x8_t, load16(rsA, a_off(s_next, i, kk)));
                }
            }
            if constexpr (kk < 3 && m >= QB - 2 * JN) {
                constexpr int r = m - (QB - 2 * JN);
                read_b(Bs, kk + 1, r / 2, r % 2, (kk + 1) & 1);
            }
            if constexpr (X % PER == 0) stage_r(IC<X / PER>{});
            if constexpr (X % PER == PER / 2) stage_s(IC<X / PER>{}, run32);
            if constexpr (X % PER == 0 && X >= PER) stage_w(IC<X / PER - 1>{}, dst);
            __builtin_amdgcn_sched_barrier(0);
        });
        stage_w(IC<CH - 1>{}, dst);
    };

    // Pipeline.  At the top of iteration s: B_s[s&1] holds B(s), run_s[(s+1)&1]
    // holds run(s+1), bm_cur holds the bitmask rows of step s+1 and areg A(s).
    // The iteration loads run(s+2) and the rows of step s+2, multiplies step s
    // while decoding B(s+1) and streaming in A(s+1), stages run(s+2) and meets
    // the other waves at the barrier.  Loads past the last step re-read it.
    uint64_t bm_cur = 0ull;
    __syncthreads();                                   // lut_s
    if (nsteps > 0) {
#pragma unroll
        for (int kk = 0; kk < CFG::ASETS; kk++) load_a(0, kk);
        load_run(0);
        bm_cur = load_bm(0);
        store_run(0);
    }
    // the DW waves of a tile stage its run together: all of it must be in LDS
    // before any of them decodes (nsteps is uniform, every wave gets here)
    __syncthreads();
    if (nsteps > 0) {
        decode_rows(0, bm_cur);
        decode(0, 0);
        if (zfix) zero_fixup(0);
        load_run(min(1, last));
        bm_cur = load_bm(min(1, last));
        store_run(1);
    }
    __syncthreads();
    auto iteration = [&](int s, auto R) __attribute__((always_inline)) {
        constexpr int P = decltype(R)::value;          // s & 1
        const int s1 = min(s + 1, last), s2 = min(s + 2, last);
        load_run(s2);
        const uint64_t bm_next = load_bm(s2);
        decode_rows(s1, bm_cur);
        step(s, s1, R);
        if (zfix) zero_fixup(P ^ 1);
        store_run(P);
        bm_cur = bm_next;
        __syncthreads();
    };
    int s = 0;
    for (; s + 1 < nsteps; s += 2) {
        iteration(s, IC<0>{});
        iteration(s + 1, IC<1>{});
    }
    if (s < nsteps) iteration(s, IC<0>{});

    // ---- epilogue: half a 32-row block of accumulators at a time, staged in
    // LDS (each wave its own 16 x WAVE_N fp32 area), then written as 16-byte
    // row segments.  Accumulator element r of lane l of a 32x32 block sits at
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32: elements r < 8 are rows 0-15.
    constexpr int ST_P = CFG::ST_P;
    constexpr int LPR = CFG::WAVE_N / 4;               // lanes per staged row (4 columns each)
    constexpr int RPI = 64 / LPR;                      // rows written per pass
    float* st = reinterpret_cast<float*>(lds) + wave * (16 * ST_P);
    const int64_t col0 = (int64_t)nt0 * 64 + wn * CFG::WAVE_N;
    const bool cvec = (a.N % 4 == 0) && (a.part != nullptr || (((uintptr_t)a.C) & 7) == 0);
    __syncthreads();                                   // last reads of B_s / run_s
#pragma unroll
    for (int i = 0; i < IM; i++) {
#pragma unroll
        for (int half = 0; half < 2; half++) {
#pragma unroll
            for (int jj = 0; jj < JN; jj++)
#pragma unroll
                for (int r = 8 * half; r < 8 * half + 8; r++)
                    st[(8 * ((r >> 2) & 1) + 4 * hh + (r & 3)) * ST_P + jj * 32 + col] = acc[i][jj][r];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // lane l: columns 4*(l%LPR) .. +3 of staged row RPI*it + l/LPR, which
            // is block row 16*half + that row
#pragma unroll
            for (int it = 0; it < 16 / RPI; it++) {
                const int rr2 = RPI * it + lane / LPR;
                const int64_t row = arow0 + i * 32 + 16 * half + rr2;
                const int64_t c4 = col0 + 4 * (lane % LPR);
                const float4 v = *reinterpret_cast<const float4*>(&st[rr2 * ST_P + 4 * (lane % LPR)]);
                if (row >= a.M || c4 >= a.N) continue;
                if (a.part) {
                    float* dst = a.part + ((int64_t)split * a.M + row) * a.N + c4;
                    if (cvec) {
                        *reinterpret_cast<float4*>(dst) = v;
                    } else {
                        const float e[4] = {v.x, v.y, v.z, v.w};
                        for (int x = 0; x < 4 && c4 + x < a.N; x++) dst[x] = e[x];
                    }
                } else {
                    uint16_t* dst = a.C + row * a.N + c4;
                    const uint32_t b0 = f32_to_bf16(v.x), b1 = f32_to_bf16(v.y), b2 = f32_to_bf16(v.z), b3 = f32_to_bf16(v.w);
                    if (cvec) {
                        *reinterpret_cast<uint2*>(dst) = uint2{b0 | (b1 << 16), b2 | (b3 << 16)};
                    } else {
                        const uint32_t e[4] = {b0, b1, b2, b3};
                        for (int x = 0; x < 4 && c4 + x < a.N; x++) dst[x] = (uint16_t)e[x];
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }
}

// A -> Apk, the MFMA-fragment order read by gemm_cb_kernel: for row block rb
// (32 rows) and k block kb (16 k), the 1 KiB block (rb * nkb + kb) holds, at
// lane l, A[32 rb + l%32][16 kb + 8 (l/32) .. +7]; zero past M and K.
__device__ __forceinline__ int64_t apk_index(int64_t m, int64_t k, uint32_t nkb)
{
    const int64_t rb = m >> 5, kb = k >> 4;
    const int l = (int)(m & 31) + 32 * (int)((k >> 3) & 1);
    return ((rb * nkb + kb) * 64 + l) * 8;
}

// from At [K, M] (row stride ldat, m contiguous): 64 x 64 blocks through LDS
__global__ __launch_bounds__(256) void pack_a_t_kernel(const uint16_t* At, int64_t K, int64_t M, int64_t ldat,
                                                       uint16_t* Apk, uint32_t nkb)
{
    __shared__ __align__(16) uint16_t t[64][64 + 8];
    const int tid = threadIdx.x;
    const int64_t k0 = (int64_t)blockIdx.x * 64, m0 = (int64_t)blockIdx.y * 64;
#pragma unroll
    for (int it = 0; it < 2; it++) {
        const int idx = it * 256 + tid, row = idx >> 3, c8 = (idx & 7) * 8;
        const int64_t k = k0 + row, m = m0 + c8;
        uint4 v = {0u, 0u, 0u, 0u};
        if (k < K && m < M) {
            const uint16_t* src = At + k * ldat + m;
            if (m + 8 <= M) {
                v = *reinterpret_cast<const uint4*>(src);
            } else {
                uint32_t w[4] = {0u, 0u, 0u, 0u};
                for (int e = 0; e < 8 && m + e < M; e++) w[e >> 1] |= (uint32_t)src[e] << (16 * (e & 1));
                v = uint4{w[0], w[1], w[2], w[3]};
            }
        }
        *reinterpret_cast<uint4*>(&t[row][c8]) = v;
    }
    __syncthreads();
    const int64_t mrows = (M + 31) / 32 * 32;          // Apk rows (whole 32-row blocks)
#pragma unroll
    for (int it = 0; it < 2; it++) {
        const int idx = it * 256 + tid, mm = idx >> 3, kc = (idx & 7) * 8;
        if (m0 + mm < mrows) {
            uint32_t w[4];
#pragma unroll
            for (int d = 0; d < 4; d++) w[d] = (uint32_t)t[kc + 2 * d][mm] | ((uint32_t)t[kc + 2 * d + 1][mm] << 16);
            *reinterpret_cast<uint4*>(Apk + apk_index(m0 + mm, k0 + kc, nkb)) = uint4{w[0], w[1], w[2], w[3]};
        }
    }
}

// from A [M, K] (row stride lda, k contiguous, K % 8 == 0): one 16-byte piece
// per thread
__global__ __launch_bounds__(256) void pack_a_n_kernel(const uint16_t* A, int64_t K, int64_t M, int64_t lda,
                                                       uint16_t* Apk, uint32_t nkb, int64_t pieces)
{
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x; p < pieces; p += stride) {
        const int64_t blk = p >> 6;
        const int l = (int)(p & 63);
        const int64_t rb = blk / nkb, kb = blk % nkb;
        const int64_t m = rb * 32 + (l & 31), k = kb * 16 + 8 * (l >> 5);
        uint4 v = {0u, 0u, 0u, 0u};
        if (m < M && k < K) v = *reinterpret_cast<const uint4*>(A + m * lda + k);
        reinterpret_cast<uint4*>(Apk)[p] = v;
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

// Packed bf16 storage (pack_sbit): value i of the stream at bits [15 i,
// 15 i + 15), least significant first, the value's low 15 bits (sign 0).
// The run [vo + prefix[0], vo + prefix[T]) is unpacked into out[0, n) as bf16
// (n = the run's length, within the stream's whole values and cap; cap a
// multiple of 8, so the 16-byte stores stay inside out), and *out_vo =
// -prefix[0]: the GEMM then stages tile t's run from out[prefix[t] + *out_vo]
// as it would stored bf16 values.  8 values per thread and pass: the five
// dwords from the one holding the group's first bit (whole-dword reads while
// inside the stream, else byte by byte), funnel-shifted to that bit.
__global__ __launch_bounds__(256) void unpack15_kernel(const uint8_t* stream, int64_t nbytes, const uint32_t* prefix,
                                                       int64_t T, const int64_t* vals_offset, uint16_t* out,
                                                       int64_t cap, int64_t* out_vo)
{
    const int64_t vo = vals_offset ? *vals_offset : 0;
    const int64_t p0 = (int64_t)prefix[0];
    const int64_t b0 = vo + p0;
    const int64_t whole = nbytes * 8 / 15;               // values wholly inside the stream
    int64_t n = (int64_t)prefix[T] - p0;
    if (b0 < 0 || b0 >= whole) n = 0;
    else if (n > whole - b0) n = whole - b0;
    if (n > cap) n = cap;
    if (blockIdx.x == 0 && threadIdx.x == 0) *out_vo = -p0;
    if (n <= 0) return;
    const int64_t base = ((b0 * 15) >> 5) * 4;           // the dword holding the run's first bit
    const int64_t readable = std::min<int64_t>(nbytes - base, 0xffffffffll);
    const bs_rsrc rs = make_rsrc(stream + base, (uint32_t)readable);
    const uint64_t bit0 = (uint64_t)(b0 * 15 - base * 8);
    const int64_t stride = (int64_t)gridDim.x * 256 * 8;
    for (int64_t j = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8; j < n; j += stride) {
        const uint64_t bit = bit0 + (uint64_t)j * 15u;
        const uint32_t o4 = (uint32_t)(bit >> 5) * 4u, sb = (uint32_t)(bit & 31u);
        uint32_t w[5];
        if ((int64_t)o4 + 20 <= readable) {
            const uint4 v = load16(rs, o4);
            w[0] = v.x, w[1] = v.y, w[2] = v.z, w[3] = v.w;
            w[4] = load4(rs, o4 + 16u);
        } else {
            w[0] = w[1] = w[2] = w[3] = w[4] = 0u;
            for (int e = 0; e < 20; e++)
                w[e >> 2] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rs, (int)(o4 + (uint32_t)e), 0, 0)
                             << (8 * (e & 3));
        }
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = __builtin_amdgcn_alignbit(w[i + 1], w[i], sb);
        uint32_t o[4];
#pragma unroll
        for (int d = 0; d < 4; d++) {
            uint32_t v2[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int b = 15 * (2 * d + h), wi = b >> 5, bs = b & 31;
                const uint32_t raw = bs + 15 <= 32 ? q[wi] >> bs : __builtin_amdgcn_alignbit(q[min(wi + 1, 3)], q[wi], bs);
                v2[h] = raw & 0x7fffu;
            }
            o[d] = v2[0] | (v2[1] << 16);
        }
        *reinterpret_cast<uint4*>(out + j) = uint4{o[0], o[1], o[2], o[3]};
    }
}

// C[0, n) = 0 (bf16 bits), grid-stride
__global__ __launch_bounds__(256) void zero_fill_u16_kernel(uint16_t* C, int64_t n)
{
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) C[i] = 0;
}

// Split-K factor: fewest "rounds x steps" with `per_cu` workgroups per CU on
// kCus CUs, a small charge for the partial-sum pass, <= kMaxSteps per workgroup
// and >= 8 steps per workgroup where possible.
static int gemm_split(int64_t M, int64_t N, int64_t K, int64_t bm, int64_t bn, int per_cu)
{
    const int64_t slots = (int64_t)kCus * per_cu;
    const int64_t tiles = ((N + bn - 1) / bn) * ((M + bm - 1) / bm);
    const int64_t ksteps = (K + kBK - 1) / kBK;
    const int64_t min_split = (ksteps + kMaxSteps - 1) / kMaxSteps;
    int64_t best = min_split, best_cost = -1;
    for (int64_t s = min_split; s <= 64; s++) {
        if (s > min_split && ksteps / s < 8) break;
        const int64_t rounds = (tiles * s + slots - 1) / slots;
        const int64_t cost = rounds * ((ksteps + s - 1) / s) + (s > 1 ? 2 : 0);
        if (best_cost < 0 || cost < best_cost) {
            best = s;
            best_cost = cost;
        }
    }
    return (int)best;
}

// Apk geometry: k padded to whole K-steps, rows to whole 32-row blocks
static int64_t apk_nkb(int64_t K) { return (K + kBK - 1) / kBK * (kBK / 16); }
static int64_t apk_bytes(int64_t M, int64_t K) { return (M + 31) / 32 * apk_nkb(K) * 1024; }

// Launch plan: 512-row workgroups when they cover M with no more padding
// than 256-row ones (half the decode work per MFMA); else 256 x 128 with two
// workgroups per CU (configs[1]'s 768 x 8192 x 3072: 78 us per call against
// 87 us with one 256 x 256 workgroup per CU, and 104 us with 768 x 64
// workgroups, which decode each B tile once but re-read A for every 64
// columns).  BITSPARSE_DW_CFG (256 / 512 / 768 / 2561 for 256h / 2562 for
// 256v) forces a shape (tuning runs).
enum { CFG_256 = 0, CFG_512 = 1, CFG_768 = 2, CFG_256H = 3, CFG_256V = 4 };
struct GemmPlan {
    int cfg;
    int64_t bm, bn;
    int split;
};
static GemmPlan gemm_plan(int64_t M, int64_t N, int64_t K)
{
    GemmPlan p;
    const int64_t pad512 = (M + Cfg512::BM - 1) / Cfg512::BM * Cfg512::BM;
    const int64_t pad256 = (M + Cfg256::BM - 1) / Cfg256::BM * Cfg256::BM;
    if (M >= Cfg512::BM && pad512 <= pad256) p.cfg = CFG_512;
    else p.cfg = CFG_256V;
    if (const char* ev = getenv("BITSPARSE_DW_CFG")) {
        const int v = atoi(ev);
        if (v == 256) p.cfg = CFG_256;
        else if (v == 512) p.cfg = CFG_512;
        else if (v == 768) p.cfg = CFG_768;
        else if (v == 2561) p.cfg = CFG_256H;
        else if (v == 2562) p.cfg = CFG_256V;
    }
    switch (p.cfg) {
    case CFG_768: p.bm = Cfg768::BM; p.bn = Cfg768::BN; break;
    case CFG_512: p.bm = Cfg512::BM; p.bn = Cfg512::BN; break;
    case CFG_256H: p.bm = Cfg256h::BM; p.bn = Cfg256h::BN; break;
    case CFG_256V: p.bm = Cfg256v::BM; p.bn = Cfg256v::BN; break;
    default: p.bm = Cfg256::BM; p.bn = Cfg256::BN; break;
    }
    const int per_cu = (p.cfg == CFG_256H || p.cfg == CFG_256V) ? 2 : 1;
    p.split = gemm_split(M, N, K, p.bm, p.bn, per_cu);
    return p;
}
static int64_t align_up256(int64_t x) { return (x + 255) / 256 * 256; }

}  // namespace bs

using namespace bs;

// packed: the unpacked bf16 value run (room for K N values, whole 16-byte
// units) and its offset word follow A's packed copy
static int64_t unpack_run_cap(int64_t K, int64_t N) { return (K * N + 7) / 8 * 8; }

extern "C" int64_t bs_gemm_compressed_b_packed_workspace_bytes(int64_t M, int64_t N, int64_t K, int a_layout)
{
    const int64_t base = bs_gemm_compressed_b_workspace_bytes(M, N, K, a_layout);
    if (M <= 0 || N <= 0 || K <= 0) return base;
    return align_up256(base) + align_up256(unpack_run_cap(K, N) * 2) + 256;
}

extern "C" int64_t bs_gemm_compressed_b_workspace_bytes(int64_t M, int64_t N, int64_t K, int a_layout)
{
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    const int split = gemm_plan(M, N, K).split;
    int64_t bytes = split > 1 ? align_up256((int64_t)split * M * N * 4) : 0;
    (void)a_layout;
    bytes += apk_bytes(M, K);
    return bytes;
}

// packed: vals is a packed value stream of vals_numel bytes (4-byte aligned)
static int gemm_cb_impl(const void* A, int64_t M, int64_t K, int64_t lda, int a_layout, const void* vals,
                        int vals_dtype, int64_t vals_numel, const uint8_t* bitmask, const uint32_t* prefix,
                        const int64_t* vals_offset, int64_t N, int square, float relu2_scale, const float* b_scale,
                        void* C, void* workspace, int64_t workspace_bytes, void* stream, bool packed, const char* fn)
{
    clear_error();
    if (M < 0 || N < 0 || K < 0) return set_error(BS_ERR_INVALID, "%s: negative shape", fn);
    if (a_layout != 0 && a_layout != 1) return set_error(BS_ERR_INVALID, "%s: bad a_layout", fn);
    if (vals_dtype < 0 || vals_dtype > 2) return set_error(BS_ERR_INVALID, "%s: bad dtype", fn);
    if (!square && vals_dtype != DT_BF16)
        return set_error(BS_ERR_INVALID, "%s: fp8 storage needs square=1", fn);
    if (b_scale != nullptr && !square)
        return set_error(BS_ERR_INVALID, "%s: b_scale is only applied with square=1", fn);
    if (a_layout == 0 && lda < M) return set_error(BS_ERR_INVALID, "%s: lda < M", fn);
    if (a_layout == 1 && lda < K) return set_error(BS_ERR_INVALID, "%s: lda < K", fn);
    if (a_layout == 1 && K % 8 != 0)
        return set_error(BS_ERR_INVALID, "%s: a_layout 1 needs K %% 8 == 0", fn);
    // bf16 storage without the square runs past 2^31 elements on the GPU
    const bool big_ok = !packed && vals_dtype == DT_BF16 && !square;
    if ((uint64_t)K * (uint64_t)N >= (big_ok ? kMaxElems : kMaxElemsUntested))
        return set_error(BS_ERR_INVALID, "%s: K*N must be < 2^%d on this path", fn, big_ok ? 32 : 31);
    if (M == 0 || N == 0) return BS_OK;
    if (C == nullptr) return set_error(BS_ERR_INVALID, "%s: null C", fn);
    if (((uintptr_t)C) & 1) return set_error(BS_ERR_INVALID, "%s: C misaligned", fn);
    hipStream_t st = (hipStream_t)stream;
    const uint32_t ksteps = (uint32_t)((K + kBK - 1) / kBK);
    if (ksteps == 0) {
        // an empty sum: C = 0, written by a kernel (a memset node in a captured
        // graph is avoided, so this path captures like the others)
        const int64_t n = M * N;
        const uint32_t nblk = (uint32_t)std::min<int64_t>((n + 255) / 256, 2048);
        hipLaunchKernelGGL(zero_fill_u16_kernel, dim3(nblk), dim3(256), 0, st, (uint16_t*)C, n);
        hipError_t e = hipGetLastError();
        return e == hipSuccess ? BS_OK : set_error(BS_ERR_HIP, "%s: %s", fn, hipGetErrorString(e));
    }
    if (A == nullptr || bitmask == nullptr || prefix == nullptr || (vals_numel > 0 && vals == nullptr))
        return set_error(BS_ERR_INVALID, "%s: null pointer", fn);
    if ((((uintptr_t)A) & 15) || (lda % 8) != 0)
        return set_error(BS_ERR_INVALID, "%s: A must be 16-byte aligned with lda %% 8 == 0", fn);
    if (lda >= (1ll << 24)) return set_error(BS_ERR_INVALID, "%s: lda must be < 2^24", fn);
    if (((uintptr_t)vals) & (packed ? 3 : 15))
        return set_error(BS_ERR_INVALID, "%s: vals must be %d-byte aligned", fn, packed ? 4 : 16);
    if (packed && vals_dtype != DT_BF16)
        return set_error(BS_ERR_INVALID, "%s: packed fp8 values go to bs_gemm_compressed_b_fp8_packed", fn);
    const GemmPlan plan = gemm_plan(M, N, K);
    const int split = plan.split;
    const int64_t part_bytes = split > 1 ? align_up256((int64_t)split * M * N * 4) : 0;
    const int64_t nkb = apk_nkb(K), nrb = (M + 31) / 32;
    if (nkb >= (1ll << 20)) return set_error(BS_ERR_INVALID, "%s: K too large", fn);
    const int64_t need = packed ? bs_gemm_compressed_b_packed_workspace_bytes(M, N, K, a_layout)
                                : part_bytes + apk_bytes(M, K);
    {
        if (workspace == nullptr || workspace_bytes < need)
            return set_error(BS_ERR_INVALID, "%s: workspace too small (%lld < %lld)", fn,
                             (long long)workspace_bytes, (long long)need);
        if (((uintptr_t)workspace) & 15) return set_error(BS_ERR_INVALID, "%s: workspace misaligned", fn);
    }
    GemmArgs g{};
    g.M = M;
    g.K = K;
    g.vals = (const uint8_t*)vals;
    g.vals_numel = vals_numel;
    g.bitmask = bitmask;
    g.prefix = prefix;
    g.vals_offset = vals_offset;
    g.N = N;
    g.grid_n = (uint32_t)((N + kTile - 1) / kTile);
    const uint32_t nt = (uint32_t)(plan.bn / kTile);
    g.tiles_n = (g.grid_n + nt - 1) / nt;
    g.tiles_m = (uint32_t)((M + plan.bm - 1) / plan.bm);
    g.relu2_scale = relu2_scale;
    g.b_scale = b_scale;
    g.C = (uint16_t*)C;
    g.part = split > 1 ? (float*)workspace : nullptr;
    g.ksteps = ksteps;
    g.ksteps_per_split = (ksteps + split - 1) / split;
    if (g.ksteps_per_split > (uint32_t)kMaxSteps)
        return set_error(BS_ERR_INVALID, "%s: internal split error", fn);
    const uint64_t blocks = (uint64_t)g.tiles_m * g.tiles_n * (uint64_t)split;
    if (blocks >= (1ull << 31)) return set_error(BS_ERR_INVALID, "%s: grid too large", fn);
    // A into MFMA-fragment order (workspace after the partial sums)
    uint16_t* apk = (uint16_t*)((uint8_t*)workspace + part_bytes);
    if (a_layout == 0) {
        hipLaunchKernelGGL(pack_a_t_kernel, dim3((uint32_t)(nkb / 4), (uint32_t)((M + 63) / 64)), dim3(256), 0, st,
                           (const uint16_t*)A, K, M, lda, apk, (uint32_t)nkb);
    } else {
        const int64_t pieces = nrb * nkb * 64;
        int64_t nblk = (pieces + 255) / 256;
        if (nblk > 4096) nblk = 4096;
        hipLaunchKernelGGL(pack_a_n_kernel, dim3((uint32_t)nblk), dim3(256), 0, st, (const uint16_t*)A, K, M, lda, apk,
                           (uint32_t)nkb, pieces);
    }
    g.Apk = apk;
    g.nkb = (uint32_t)nkb;
    g.nrb = (uint32_t)nrb;
    if (packed) {
        // the stream's run unpacked to bf16 after A's packed copy; the GEMM
        // stages it as stored values
        const int64_t cap = unpack_run_cap(K, N);
        uint16_t* run = reinterpret_cast<uint16_t*>((uint8_t*)workspace + align_up256(part_bytes + apk_bytes(M, K)));
        int64_t* run_vo = reinterpret_cast<int64_t*>((uint8_t*)run + align_up256(cap * 2));
        const int64_t T = (int64_t)ksteps * g.grid_n;
        const uint32_t ublk = (uint32_t)std::min<int64_t>((cap + 2047) / 2048, 2048);
        hipLaunchKernelGGL(unpack15_kernel, dim3(ublk), dim3(256), 0, st, (const uint8_t*)vals, vals_numel, prefix, T,
                           vals_offset, run, cap, run_vo);
        g.vals = reinterpret_cast<const uint8_t*>(run);
        g.vals_numel = cap;
        g.vals_offset = run_vo;
    }
#define BS_GEMM_LAUNCH(VT, SQ, SC)                                                                              \
    do {                                                                                                        \
        if (plan.cfg == CFG_768)                                                                                \
            hipLaunchKernelGGL((gemm_cb_kernel<Cfg768, VT, SQ, SC>), dim3((uint32_t)blocks), dim3(Cfg768::THREADS), \
                               0, st, g);                                                                       \
        else if (plan.cfg == CFG_256H)                                                                          \
            hipLaunchKernelGGL((gemm_cb_kernel<Cfg256h, VT, SQ, SC>), dim3((uint32_t)blocks),                   \
                               dim3(Cfg256h::THREADS), 0, st, g);                                               \
        else if (plan.cfg == CFG_256V)                                                                          \
            hipLaunchKernelGGL((gemm_cb_kernel<Cfg256v, VT, SQ, SC>), dim3((uint32_t)blocks),                   \
                               dim3(Cfg256v::THREADS), 0, st, g);                                               \
        else if (plan.cfg == CFG_512)                                                                           \
            hipLaunchKernelGGL((gemm_cb_kernel<Cfg512, VT, SQ, SC>), dim3((uint32_t)blocks), dim3(Cfg512::THREADS), \
                               0, st, g);                                                                       \
        else                                                                                                    \
            hipLaunchKernelGGL((gemm_cb_kernel<Cfg256, VT, SQ, SC>), dim3((uint32_t)blocks), dim3(Cfg256::THREADS), \
                               0, st, g);                                                                       \
    } while (0)
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
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "%s launch: %s", fn, hipGetErrorString(e));
    return BS_OK;
}

extern "C" int bs_gemm_compressed_b(const void* A, int64_t M, int64_t K, int64_t lda, int a_layout,
                                    const void* vals, int vals_dtype, int64_t vals_numel,
                                    const uint8_t* bitmask, const uint32_t* prefix, const int64_t* vals_offset,
                                    int64_t N, int square, float relu2_scale, const float* b_scale, void* C,
                                    void* workspace, int64_t workspace_bytes, void* stream)
{
    return gemm_cb_impl(A, M, K, lda, a_layout, vals, vals_dtype, vals_numel, bitmask, prefix, vals_offset, N,
                        square, relu2_scale, b_scale, C, workspace, workspace_bytes, stream, false,
                        "bs_gemm_compressed_b");
}

extern "C" int bs_gemm_compressed_b_packed(const void* A, int64_t M, int64_t K, int64_t lda, int a_layout,
                                           const void* stream_bytes, int vals_dtype, int64_t stream_nbytes,
                                           const uint8_t* bitmask, const uint32_t* prefix,
                                           const int64_t* vals_offset, int64_t N, int square, float relu2_scale,
                                           const float* b_scale, void* C, void* workspace,
                                           int64_t workspace_bytes, void* stream)
{
    return gemm_cb_impl(A, M, K, lda, a_layout, stream_bytes, vals_dtype, stream_nbytes, bitmask, prefix,
                        vals_offset, N, square, relu2_scale, b_scale, C, workspace, workspace_bytes, stream, true,
                        "bs_gemm_compressed_b_packed");
}
