// Reconstruct-into-LDS fp8 MFMA GEMM for gfx950:
//     C[M, N] = bf16(sA * sB * (A @ Bq))
// A: e4m3fn codes [M, K] with fp32 scale sA (in the MLP backward A = dY^T,
// quantized by to_fp8).  B: a compressed [K, N] fp8 activation (64x64-tile
// bitmask + prefix + values), decoded tile by tile into LDS and never
// written to HBM in dense form:
//   * square = 0 (AspB): Bq = the stored codes, sB = their stored scale;
//   * square = 1 (AspRelu2B): Bq, sB = to_fp8(D) of the bf16 dense operand
//     D = bf16(bf16((k r) r) * bf16(s^2)) that the reference decompresses and
//     re-quantizes (lib_sparse/src/sparse_matmul.py:109-113,
//     lib_sparse/src/triton_operators.py:160-161, lib_sparse/fp8.py:123-129).
//     D is a function of the stored code alone, so is Bq: a 256-entry table
//     code -> Bq code, built on the device before the GEMM from sB =
//     max(amax|D| / 448, 1e-9).  amax|D| is |D(c)| of the stored code c of
//     largest magnitude (|D| grows with |r|: each rounding is monotone; a NaN
//     code sorts above every finite one, as in the amax kernel), or |D(0)| of
//     the cleared elements.  Bq(c) = e4m3fn_RNE(D(c) / sB) with one correctly
//     rounded division, the to_fp8 rule, so the decoded operand is bit for
//     bit to_fp8(unpack_relu2_batch_(B)).  The tensor's value run is mapped
//     through the table once, into the workspace (nnz bytes read and
//     written), and the GEMM stages the mapped codes: every row block of C
//     reads the run, so mapping while staging would repeat the table lookups
//     once per row block.
// Replaces "decompress B to HBM, re-quantize, library fp8 GEMM" (hipBLASLt
// scaled_mm) of the reference's fp8 AspB / AspRelu2B.
//
// Workgroup: a WGM x WGN grid of waves, each owning a WAVE_M x WAVE_N block
// of C in v_mfma_scale_f32_32x32x64_f8f6f4 accumulators (e4m3 x e4m3, or
// e4m3 x e5m2 for square = 0 from e5m2 storage; unit block scales).  One
// K-step = 64 tokens = one row of B tiles = one MFMA deep.  Per step:
//   * the step's B tiles are decoded into a double-buffered LDS tile (one
//     8-byte chunk per lane per decode row): value runs are loaded one step
//     ahead, staged in LDS, and
//     each chunk is built from an 8-byte window of its run with v_alignbyte
//     and two v_perm_b32 (selectors from a 256-entry table per bitmask byte);
//   * B fragments come out of the row-major tile with ds_read_b64_tr_b8
//     (within a 16-lane group, output lane i byte b = source lane 2b + i/8,
//     byte i%8), four per 32-column block;
//   * A fragments (32 contiguous k of one row per lane) come from a packed
//     copy of A in MFMA-fragment order, one 2 KiB block per (32 rows, 64 k),
//     double-buffered across steps.
// Workgroup ids are remapped so each XCD walks a contiguous range of C tiles.
#include <algorithm>

#include "bs_device.h"
#include "bs_host.h"
#include "gemm_common.h"

namespace bs {

typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));

constexpr int kRun8Slots = kTileNumel / 16 + 2;   // one fp8 run + its phase, 16-byte slots

template <int WGM_, int WGN_, int WM_, int WN_, int MINB_ = 1>
struct Gemm8Cfg {
    static constexpr int MINB = MINB_;                           // workgroups per CU (launch bound)
    static constexpr int WGM = WGM_, WGN = WGN_, NWAVES = WGM_ * WGN_, THREADS = 64 * NWAVES;
    static constexpr int WAVE_M = WM_, WAVE_N = WN_;
    static constexpr int IM = WAVE_M / 32, JN = WAVE_N / 32;    // 32x32 accumulator blocks per wave
    static constexpr int BM = WAVE_M * WGM, BN = WAVE_N * WGN;
    static constexpr int NT = BN / 64;                           // B tiles per K-step
    static constexpr int DW = NWAVES / NT;                       // waves decoding one B tile
    static constexpr int CH = 8 / DW;                            // decode rows per lane per step
    // B_s row pitch (bytes): BN + 32, an odd multiple of 32 bytes past a
    // multiple of 256: any 8 consecutive rows start 8 banks apart around all
    // 64, so a transposing fragment read (16 rows x 32 bytes) and a decode
    // store (8 rows x 64 bytes) touch every bank exactly twice
    static constexpr int BP = BN + 32;
    static constexpr int SEG = IM * JN;                          // MFMAs per K-step
    static constexpr int PER = SEG / CH;                         // MFMAs per decoded chunk
    static constexpr int OFF_B = 0;                              // B_s[2][64][BP] bytes
    static constexpr int OFF_RUN = OFF_B + 2 * kBK * BP;         // run_s[3][NT][kRun8Slots] uint4
    // row tables of two steps (the one decoded now, the one built for later)
    static constexpr int OFF_BM = OFF_RUN + 3 * NT * kRun8Slots * 16;   // bm_s[2][NWAVES][64] uint64
    static constexpr int OFF_RP = OFF_BM + 2 * NWAVES * 64 * 8;     // rp_s[2][NWAVES][64] uint32
    static constexpr int OFF_SEL = OFF_RP + 2 * NWAVES * 64 * 4;    // sel_s[256] uint2
    static constexpr int OFF_PF = OFF_SEL + 256 * 8;            // pf_s[NT][kMaxSteps] uint2: prefix[t], prefix[t+1]
    static constexpr int ST_P = WAVE_N + 4;                      // epilogue staging pitch (floats)
    static constexpr int LDS_MAIN = OFF_PF + NT * kMaxSteps * 8;
    static constexpr int LDS_EPI = NWAVES * 16 * ST_P * 4;      // the epilogue reuses the space
    static constexpr int LDS = LDS_MAIN > LDS_EPI ? LDS_MAIN : LDS_EPI;
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static_assert(NWAVES * 16 * ST_P * 4 <= LDS, "epilogue staging does not fit");
    static_assert(NWAVES % NT == 0 && 8 % DW == 0 && SEG % CH == 0, "decode split");
    static_assert(BP % 256 == 32 || BP % 256 == 160, "fragment-read bank spread");
};
// 8 x 1 waves of 64 x 128 (two per SIMD, 128 VGPRs + 128 AGPRs each, the
// accumulators in the AGPRs): each decoded B byte feeds 512 rows.
using Cfg8_512 = Gemm8Cfg<8, 1, 64, 128>;
// 2 x 2 waves of 128 x 128 (one per SIMD)
using Cfg8_256 = Gemm8Cfg<2, 2, 128, 128>;

struct Gemm8Args {
    const uint8_t* Apk;           // A codes in MFMA-fragment order (pack_a8_*_kernel)
    int64_t M, K;
    uint32_t nkb;                 // 64-wide k blocks of Apk
    uint32_t nrb;                 // 32-row blocks of Apk (per k block)
    const uint8_t* vals;          // compressed B
    int64_t vals_numel;
    const uint8_t* bitmask;
    const uint32_t* prefix;
    const int64_t* vals_offset;
    int64_t N;
    uint32_t grid_n;              // B tiles along N
    uint32_t tiles_m, tiles_n;    // C tiles
    const float* a_scale;
    const float* b_scale;         // sB
    uint16_t* C;                  // [M, N] bf16 (no split)
    float* part;                  // [split, M, N] fp32 unscaled partial sums (split > 1)
    uint32_t ksteps;
    uint32_t ksteps_per_split;
};

// FMT_B: MFMA format of B (0 e4m3, 1 e5m2).
template <typename CFG, int FMT_B>
__global__ __launch_bounds__(CFG::THREADS, CFG::MINB) void gemm_cb8_kernel(Gemm8Args a)
{
    constexpr int NT = CFG::NT, DW = CFG::DW, CH = CFG::CH, BP = CFG::BP, IM = CFG::IM, JN = CFG::JN;
    constexpr int RX = (15 + kTileNumel + 15) / 16;              // 16-byte units of a run, worst case
    constexpr int RXD = (RX + 64 * DW - 1) / (64 * DW);          // per lane, worst case

    __shared__ __align__(16) uint8_t lds[CFG::LDS];
    uint8_t* B_s = lds + CFG::OFF_B;
    uint4* run_s = reinterpret_cast<uint4*>(lds + CFG::OFF_RUN);
    uint64_t* bm_s = reinterpret_cast<uint64_t*>(lds + CFG::OFF_BM);
    uint32_t* rp_s = reinterpret_cast<uint32_t*>(lds + CFG::OFF_RP);
    uint2* sel_s = reinterpret_cast<uint2*>(lds + CFG::OFF_SEL);
    uint2* pf_s = reinterpret_cast<uint2*>(lds + CFG::OFF_PF);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // ---- XCD-aware tile order: XCD x runs a contiguous range of tile ids
    const uint32_t nb = gridDim.x, b = blockIdx.x;
    const uint32_t xcd = b % kXcds, q = b / kXcds;
    const uint32_t per = nb / kXcds, rem = nb % kXcds;
    const uint32_t id = xcd * per + min(xcd, rem) + q;
    const uint32_t tn = (uint32_t)__builtin_amdgcn_readfirstlane((int)(id % a.tiles_n));
    const uint32_t rest = id / a.tiles_n;
    const uint32_t tm = (uint32_t)__builtin_amdgcn_readfirstlane((int)(rest % a.tiles_m));
    const uint32_t split = (uint32_t)__builtin_amdgcn_readfirstlane((int)(rest / a.tiles_m));

    const uint32_t nt0 = tn * NT;                      // first B tile column
    const int tw = wave / DW;                          // the B tile this wave helps decode
    const int tq = wave % DW;                          // its share: rows 8 CH tq .. +8 CH
    const uint32_t tcol = nt0 + (uint32_t)tw;
    const bool has_tile = tcol < a.grid_n;
    const int64_t m0 = (int64_t)tm * CFG::BM;
    const uint32_t kt0 = split * a.ksteps_per_split;
    const uint32_t kt1 = min(a.ksteps, kt0 + a.ksteps_per_split);
    const int nsteps = kt1 > kt0 ? (int)(kt1 - kt0) : 0;
    const int last = nsteps - 1;

    // selectors of bitmask byte x: set element e takes window byte rank(e),
    // 0x0c gives 0x00
    if (tid < 256) {
        uint32_t sel[2] = {0x0c0c0c0cu, 0x0c0c0c0cu};
        uint32_t rank = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            if ((tid >> e) & 1) {
                sel[e >> 2] = (sel[e >> 2] & ~(0xffu << (8 * (e & 3)))) | (rank << (8 * (e & 3)));
                rank++;
            }
        }
        sel_s[tid] = uint2{sel[0], sel[1]};
    }
    // A cleared element decodes to 0x00.  For square = 1 the reference's
    // operand holds to_fp8(D(0)) there: +0 (0x00), -0 (0x80, for k < 0) or
    // NaN.  -0 in place of +0 leaves every output bit unchanged (its products
    // are zeros, and the fp32 accumulators start at +0, to which a zero of
    // either sign adds nothing); a NaN D(0) makes amax, sB and so every
    // output NaN whatever B holds.

    // ---- prefix[t], prefix[t+1] of every step of each B tile column of the
    // workgroup, in LDS (nsteps <= kMaxSteps)
    for (int i = tid; i < NT * kMaxSteps; i += CFG::THREADS) {
        const int tc = i / kMaxSteps, st = i % kMaxSteps;
        const uint32_t col = nt0 + (uint32_t)tc;
        uint2 v = {0u, 0u};
        if (col < a.grid_n && st < nsteps) {
            const size_t t = (size_t)(kt0 + (uint32_t)st) * a.grid_n + col;
            v = uint2{a.prefix[t], a.prefix[t + 1]};
        }
        pf_s[i] = v;
    }
    const int64_t vo = a.vals_offset ? *a.vals_offset : 0;
    // value run of step s (wave-uniform): 16-byte aligned start e0, phase =
    // run start - e0, nunits 16-byte staging units
    auto run_geom = [&](int s, int64_t& e0, int& phase, int& nunits) __attribute__((always_inline)) {
        const uint2 pv = pf_s[tw * kMaxSteps + s];
        const uint32_t p[2] = {uniform_u32(pv.x), uniform_u32(pv.y)};
        // wave-uniform: 32-bit tests (a 64-bit compare is a vector
        // instruction on this target and takes a VGPR temporary)
        const uint32_t cnt = p[1] >= p[0] ? min(p[1] - p[0], (uint32_t)kTileNumel) : 0u;
        const int64_t run0 = vo + (int64_t)p[0];
        phase = (int)(run0 & 15);
        e0 = run0 - phase;
        nunits = cnt == 0 ? 0 : (phase + (int)cnt + 15) / 16;
    };

    // ---- run staging: the units of step s are loaded into registers one
    // iteration before they are written to LDS (unit u by lane u % 64 of
    // wave (u / 64) % DW of the tile's waves, pass u / (64 DW))
    uint4 rr[2][RXD];
    int rr_nunits[2] = {0, 0};
    auto load_run_at = [&](int64_t e0, int nunits, auto SL) __attribute__((always_inline)) {
        constexpr int SLOT = decltype(SL)::value;
        const int64_t avail = a.vals_numel - e0;       // bytes readable from e0
        // 64-bit tests by sign and high bits, which stay scalar instructions;
        // avail32 = avail clamped to 2^24 (a run holds at most 4096 bytes)
        const bool ok = ((uint64_t)e0 >> 63) == 0 && ((uint64_t)(avail - 1) >> 63) == 0 && nunits > 0;
        const uint32_t avail32 = ((uint64_t)avail >> 24) != 0 ? (1u << 24) : (uint32_t)avail;
        const uint32_t bytes = ok ? min(avail32, (uint32_t)nunits * 16u) : 0u;
        rr_nunits[SLOT] = ok ? nunits : 0;
        const bs_rsrc rs = make_rsrc(ok ? a.vals + e0 : a.vals, bytes);
        const bool tail = ok && (uint32_t)nunits * 16u > avail32;   // the run's last unit crosses the end of vals
        // Every pass is issued whatever the run's length (units past it read
        // zeros through the resource's range check): a load skipped on some
        // paths would make the compiler's count of loads in flight a lower
        // bound, and the waits for A before the MFMAs would then also wait
        // for the run and bitmask loads issued in the same iteration.
#pragma unroll
        for (int x = 0; x < RXD; x++) {
            const int u = (x * DW + tq) * 64 + lane;
            uint4 v = load16(rs, (uint32_t)u * 16u);
            if (tail && (uint32_t)(u + 1) * 16u > avail32 && (uint32_t)u * 16u < avail32) {
                uint32_t w[4] = {0u, 0u, 0u, 0u};
                for (int e = 0; e < 16; e++)
                    w[e >> 2] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rs, (int)(u * 16 + e), 0, 0)
                                 << (8 * (e & 3));
                v = uint4{w[0], w[1], w[2], w[3]};
            }
            rr[SLOT][x] = v;
        }
    };
    auto load_run = [&](int s, auto SL) __attribute__((always_inline)) {
        int64_t e0;
        int phase, nunits;
        run_geom(s, e0, phase, nunits);
        load_run_at(e0, nunits, SL);
    };
    auto store_run = [&](int buf, auto SL) __attribute__((always_inline)) {
        constexpr int SLOT = decltype(SL)::value;
        uint4* dst = run_s + (buf * NT + tw) * kRun8Slots;
#pragma unroll
        for (int x = 0; x < RXD; x++) {
            const int u = (x * DW + tq) * 64 + lane;
            if ((x * DW + tq) * 64 < rr_nunits[SLOT] && u < rr_nunits[SLOT]) dst[u] = rr[SLOT][x];
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

    // ---- decode: lane l handles chunk dc = l%8 (8 bytes at column 8 dc) of
    // CH rows, row = rbase + 8i + l/8
    const int dc = lane & 7, dg = lane >> 3;
    const uint64_t below_mask = dc == 0 ? 0ull : (~0ull >> (64 - 8 * dc));
    const int rbase = 8 * CH * tq;
    // row table tb (step parity): lane r's row word and the run index of its
    // first value (phase + exclusive prefix of the row popcounts)
    auto decode_rows_at = [&](int phase, uint64_t bmr, int tb) __attribute__((always_inline)) {
        const uint32_t c = (uint32_t)__popcll(bmr);
        const uint32_t rp = wave_incl_scan(c) - c;
        bm_s[(tb * CFG::NWAVES + wave) * 64 + lane] = bmr;
        rp_s[(tb * CFG::NWAVES + wave) * 64 + lane] = rp + (uint32_t)phase;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    auto decode_rows = [&](int s, uint64_t bmr, int tb) __attribute__((always_inline)) {
        int64_t e0;
        int phase, nunits;
        run_geom(s, e0, phase, nunits);
        decode_rows_at(phase, bmr, tb);
    };
    struct Dec {
        uint64_t mrow;
        uint32_t rpr;
        uint2 sel;
        uint32_t d0, d1, d2, sh;
    };
    Dec dq[2];
    auto stage_r = [&](auto CI, int tb) __attribute__((always_inline)) {
        constexpr int C = decltype(CI)::value;
        const int row = rbase + 8 * C + dg;
        dq[C & 1].mrow = bm_s[(tb * CFG::NWAVES + wave) * 64 + row];
        dq[C & 1].rpr = rp_s[(tb * CFG::NWAVES + wave) * 64 + row];
    };
    auto stage_s = [&](auto CI, const uint32_t* run32) __attribute__((always_inline)) {
        constexpr int C = decltype(CI)::value;
        Dec& d = dq[C & 1];
        const uint32_t byte = (uint32_t)(d.mrow >> (8 * dc)) & 0xffu;
        const uint32_t ra = d.rpr + (uint32_t)__popcll(d.mrow & below_mask);
        d.sel = sel_s[byte];
        d.sh = ra & 3u;
        d.d0 = run32[(ra >> 2)];
        d.d1 = run32[(ra >> 2) + 1];
        d.d2 = run32[(ra >> 2) + 2];
    };
    auto stage_w = [&](auto CI, uint8_t* dst) __attribute__((always_inline)) {
        constexpr int C = decltype(CI)::value;
        const Dec& d = dq[C & 1];
        const uint32_t w0 = __builtin_amdgcn_alignbyte(d.d1, d.d0, d.sh);
        const uint32_t w1 = __builtin_amdgcn_alignbyte(d.d2, d.d1, d.sh);
        const uint32_t o0 = __builtin_amdgcn_perm(w1, w0, d.sel.x);
        const uint32_t o1 = __builtin_amdgcn_perm(w1, w0, d.sel.y);
        *reinterpret_cast<uint2*>(&dst[(rbase + 8 * C + dg) * BP]) = uint2{o0, o1};
    };
    auto run_ptr = [&](int rb) __attribute__((always_inline)) {
        return reinterpret_cast<const uint32_t*>(run_s + (rb * NT + tw) * kRun8Slots);
    };
    auto dst_ptr = [&](int bb) __attribute__((always_inline)) {
        return B_s + bb * (kBK * BP) + tw * 64 + dc * 8;
    };
    auto decode = [&](int rb, int bb, int tb) __attribute__((always_inline)) {
        const uint32_t* run32 = run_ptr(rb);
        uint8_t* dst = dst_ptr(bb);
        static_for<CH>([&](auto CI) __attribute__((always_inline)) {
            stage_r(CI, tb);
            stage_s(CI, run32);
            stage_w(CI, dst);
        });
    };

    // ---- A fragments: lane l of block i holds row 32i + l%32, k = 32(l/32)
    // .. +31 of the step: the 16 bytes at 16 l and at 1024 + 16 l of its
    // 2 KiB block of Apk
    const int wm = wave % CFG::WGM, wn = wave / CFG::WGM;
    const int64_t arow0 = m0 + wm * CFG::WAVE_M;
    const uint32_t rb0 = (uint32_t)(arow0 / 32);
    // Apk holds at most 2^31 bytes (host check): an offset of 2^31 or more
    // reads zeros, for row blocks past M
    const bs_rsrc rsA = make_rsrc(a.Apk, a.nrb * a.nkb * 2048u);
    i32x8_t areg[2][IM];
    auto load_a = [&](int s, auto SI) __attribute__((always_inline)) {
        constexpr int SET = decltype(SI)::value;
#pragma unroll
        for (int i = 0; i < IM; i++) {
            const uint32_t rb = rb0 + (uint32_t)i;
            const uint32_t off = rb < a.nrb ? ((kt0 + (uint32_t)s) * a.nrb + rb) * 2048u + (uint32_t)lane * 16u
                                            : 0x80000000u;
            const uint4 lo = load16(rsA, off), hi = load16(rsA, off + 1024u);
            areg[SET][i] = i32x8_t{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
    };

    f32x16_t acc[IM][JN];
#pragma unroll
    for (int i = 0; i < IM; i++)
#pragma unroll
        for (int jj = 0; jj < JN; jj++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][jj][r] = 0.0f;

    // ---- B fragments of column block jj: lane L (group g = L/16, j = L%16)
    // points read c at row 32(g/2) + 8c + j/2, columns 16(g%2) + 8(j%2) ..+7
    // of the wave's block; the four reads are k = 8c .. 8c+7 of its column
    const int fg = lane >> 4, fj = lane & 15;
    const int fr = 32 * (fg >> 1) + (fj >> 1);
    const int fc = wn * CFG::WAVE_N + 16 * (fg & 1) + 8 * (fj & 1);
    i32x8_t breg[2];
    auto read_b = [&](const uint8_t* Bs, int jj, int set) __attribute__((always_inline)) {
        typedef __attribute__((address_space(3))) i32x2_t lds_i32x2;
        i32x2_t v[4];
#pragma unroll
        for (int c = 0; c < 4; c++)
            v[c] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(Bs + (fr + 8 * c) * BP + fc + jj * 32));
        breg[set] = i32x8_t{v[0][0], v[0][1], v[1][0], v[1][1], v[2][0], v[2][1], v[3][0], v[3][1]};
    };

    // One K-step: SEG MFMAs (column block jj outer, row block i inner), fenced
    // by sched_barrier so the order below is the issue order.  The next column
    // block's B fragments are read during the current one; one stage of the
    // software-pipelined decode of the next step goes with each MFMA (chunk
    // X/PER: stage_r at X%PER == 0, stage_s half a period later, stage_w at
    // the next chunk's stage_r), and `ld` issues the iteration's global loads
    // behind MFMAs already issued (a burst of them ahead of the first MFMA
    // stalled the issue while the TA queue drained, with the MFMA pipe idle:
    // 0.360 -> 0.345 ms at configs[3]).
    auto step = [&](int s, auto RI, auto&& ld) __attribute__((always_inline)) {
        constexpr int P = decltype(RI)::value;          // s & 1: B_s buffer and A register set
        constexpr int AS = P;
        constexpr int PER = CFG::PER;
        const uint8_t* Bs = B_s + P * (kBK * BP);
        const uint32_t* run32 = run_ptr((s + 1) % 3);   // run(s+1) -> B_s[P ^ 1]
        uint8_t* dst = dst_ptr(P ^ 1);
        read_b(Bs, 0, 0);
        static_for<CFG::SEG>([&](auto XI) __attribute__((always_inline)) {
            constexpr int X = decltype(XI)::value;
            constexpr int jj = X / IM, i = X % IM;
            if constexpr (i == 0 && jj + 1 < JN) read_b(Bs, jj + 1, (jj + 1) & 1);
            acc[i][jj] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(areg[AS][i], breg[jj & 1], acc[i][jj],
                                                                       0, FMT_B, 0, 127, 0, 127);
            // keep the MFMA in its segment: its result is next needed a step
            // later, and the compiler would otherwise sink all of them past
            // the run staging to the end of the iteration
            asm volatile("" : "+a"(acc[i][jj]));
            ld(XI);
            if constexpr (X % PER == 0) stage_r(IC<X / PER>{}, P ^ 1);
            if constexpr (X % PER == PER / 2) stage_s(IC<X / PER>{}, run32);
            if constexpr (X % PER == 0 && X >= PER) stage_w(IC<X / PER - 1>{}, dst);
            __builtin_amdgcn_sched_barrier(0);
        });
        stage_w(IC<CH - 1>{}, dst);
    };

    // Pipeline.  Step j: run(j) staged in run_s[j % 3] through register slot
    // j & 1, bitmask rows in bmq[j & 1], row table j & 1, A(j) in
    // areg[j & 1], B(j) decoded into B_s[j & 1].  Iteration s multiplies step
    // s while decoding B(s+1) from run_s[(s+1) % 3] with row table (s+1) & 1,
    // and issues behind its MFMAs, in this order (loads complete in order,
    // and A is needed an iteration before the run): A(s+1), the rows and run
    // of step s+3, the row table of step s+2 (into table s & 1, which the
    // decode of B(s) last read an iteration ago) and the staging of run(s+2),
    // loaded an iteration ago, into run_s[(s+2) % 3] (freed by the decode of
    // step s-1).  It then meets the other waves at the barrier.  Runs thus
    // get two iterations to arrive, A one.  Loads past the last step re-read
    // it.
    uint64_t bmq[2] = {0ull, 0ull};
    __syncthreads();                                   // sel_s, pf_s
    if (nsteps > 0) {
        load_run(0, IC<0>{});
        store_run(0, IC<0>{});
        load_run(min(1, last), IC<1>{});
        store_run(1, IC<1>{});
        bmq[0] = load_bm(0);
        bmq[1] = load_bm(min(1, last));
        load_a(0, IC<0>{});
    }
    __syncthreads();
    if (nsteps > 0) {
        decode_rows(0, bmq[0], 0);
        decode(0, 0, 0);
        decode_rows(min(1, last), bmq[1], 1);
        bmq[0] = load_bm(min(2, last));
        load_run(min(2, last), IC<0>{});
    }
    __syncthreads();
    auto iteration = [&](int s, auto RI) __attribute__((always_inline)) {
        constexpr int P = decltype(RI)::value;         // s & 1
        const int s1 = min(s + 1, last), s2 = min(s + 2, last), s3 = min(s + 3, last);
        // both steps' run geometry first: the two prefix reads share one
        // LDS round trip (the row-table stores would otherwise order them)
        int64_t e0a, e0b;
        int pha, phb, nua, nub;
        run_geom(s2, e0a, pha, nua);
        run_geom(s3, e0b, phb, nub);
        step(s, RI, [&](auto XI) __attribute__((always_inline)) {
            constexpr int X = decltype(XI)::value;
            if constexpr (X == 0) load_a(s1, IC<P ^ 1>{});
            if constexpr (X == CFG::SEG / 4) bmq[P ^ 1] = load_bm(s3);
            if constexpr (X == CFG::SEG / 2) load_run_at(e0b, nub, IC<P ^ 1>{});
            if constexpr (X == CFG::SEG / 2 + 1) decode_rows_at(pha, bmq[P], P);
            if constexpr (X == CFG::SEG * 3 / 4) store_run((s + 2) % 3, IC<P>{});
        });
        __syncthreads();
    };
    int s = 0;
    for (; s + 1 < nsteps; s += 2) {
        iteration(s, IC<0>{});
        iteration(s + 1, IC<1>{});
    }
    if (s < nsteps) iteration(s, IC<0>{});

    // ---- epilogue: as the bf16 GEMM's (half a 32-row block at a time through
    // LDS, 16-byte row segments), scaled by sA * sB; split partials unscaled
    const float sc = (*a.a_scale) * (*a.b_scale);
    constexpr int ST_P = CFG::ST_P;
    constexpr int LPR = CFG::WAVE_N / 4;
    constexpr int RPI = 64 / LPR;
    const int hh = lane >> 5, col = lane & 31;
    float* st = reinterpret_cast<float*>(lds) + wave * (16 * ST_P);
    const int64_t col0 = (int64_t)nt0 * 64 + wn * CFG::WAVE_N;
    const bool cvec = (a.N % 4 == 0) && (a.part != nullptr || (((uintptr_t)a.C) & 7) == 0);
    __syncthreads();
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
                    const uint32_t b0 = f32_to_bf16(v.x * sc), b1 = f32_to_bf16(v.y * sc);
                    const uint32_t b2 = f32_to_bf16(v.z * sc), b3 = f32_to_bf16(v.w * sc);
                    if (cvec) {
                        // nontemporal: C is written once and larger than the caches
                        // at the shapes this kernel serves (configs[3]: 128 MiB)
                        st8<true>(dst, uint2{b0 | (b1 << 16), b2 | (b3 << 16)});
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

// A codes -> Apk8: block (kb * nrb + rb) of 2 KiB holds the 32 fragment
// bytes of lane l -- A[32 rb + l%32][64 kb + 32 (l/32) .. +31] -- as two
// 16-byte halves, at 16 l (bytes 0..15) and 1024 + 16 l (16..31), so that
// each of a wave's two 16-byte loads reads 1 KiB of whole cache lines; zero
// past M and K.  k-block major: the A rows a workgroup reads in one step
// are one contiguous range (spread over all L2 channels).
__device__ __forceinline__ int64_t apk8_index(int64_t m, int64_t k, uint32_t nrb)
{
    const int64_t rb = m >> 5, kb = k >> 6;
    const int l = (int)(m & 31) + 32 * (int)((k >> 5) & 1);
    return (kb * nrb + rb) * 2048 + ((k >> 4) & 1) * 1024 + l * 16 + (k & 15);
}

// from At [K, M] (row stride ldat, m contiguous): 64 x 64 blocks through LDS
__global__ __launch_bounds__(256) void pack_a8_t_kernel(const uint8_t* At, int64_t K, int64_t M, int64_t ldat,
                                                        uint8_t* Apk, uint32_t nrb)
{
    __shared__ __align__(16) uint8_t t[64][64 + 16];
    const int tid = threadIdx.x;
    const int64_t k0 = (int64_t)blockIdx.x * 64, m0 = (int64_t)blockIdx.y * 64;
    {
        const int row = tid >> 2, c16 = (tid & 3) * 16;          // k row, 16 m
        const int64_t k = k0 + row, m = m0 + c16;
        uint4 v = {0u, 0u, 0u, 0u};
        if (k < K && m < M) {
            const uint8_t* src = At + k * ldat + m;
            if (m + 16 <= M && (((uintptr_t)src) & 15) == 0) {
                v = *reinterpret_cast<const uint4*>(src);
            } else {
                uint32_t w[4] = {0u, 0u, 0u, 0u};
                for (int e = 0; e < 16 && m + e < M; e++) w[e >> 2] |= (uint32_t)src[e] << (8 * (e & 3));
                v = uint4{w[0], w[1], w[2], w[3]};
            }
        }
        *reinterpret_cast<uint4*>(&t[row][c16]) = v;
    }
    __syncthreads();
    const int64_t mrows = (M + 31) / 32 * 32;           // Apk rows (whole 32-row blocks)
    {
        const int mm = tid >> 2, kc = (tid & 3) * 16;           // m row, 16 k
        if (m0 + mm < mrows) {
            uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int e = 0; e < 16; e++) w[e >> 2] |= (uint32_t)t[kc + e][mm] << (8 * (e & 3));
            *reinterpret_cast<uint4*>(Apk + apk8_index(m0 + mm, k0 + kc, nrb)) = uint4{w[0], w[1], w[2], w[3]};
        }
    }
}

// from A [M, K] (row stride lda, k contiguous): one 16-byte piece per thread
__global__ __launch_bounds__(256) void pack_a8_n_kernel(const uint8_t* A, int64_t K, int64_t M, int64_t lda,
                                                        uint8_t* Apk, uint32_t nrb, int64_t pieces)
{
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x; p < pieces; p += stride) {
        const int64_t blk = p >> 7;                    // 128 pieces per 2 KiB block
        const int l = (int)(p & 63), h = (int)((p >> 6) & 1);   // half h of lane l's fragment
        const int64_t rb = blk % nrb, kb = blk / nrb;
        const int64_t m = rb * 32 + (l & 31), k = kb * 64 + 32 * (l >> 5) + 16 * h;
        uint4 v = {0u, 0u, 0u, 0u};
        if (m < M && k < K) {
            const uint8_t* src = A + m * lda + k;
            if (k + 16 <= K && (((uintptr_t)src) & 15) == 0) {
                v = *reinterpret_cast<const uint4*>(src);
            } else {
                uint32_t w[4] = {0u, 0u, 0u, 0u};
                for (int e = 0; e < 16 && k + e < K; e++) w[e >> 2] |= (uint32_t)src[e] << (8 * (e & 3));
                v = uint4{w[0], w[1], w[2], w[3]};
            }
        }
        reinterpret_cast<uint4*>(Apk)[p] = v;
    }
}

// ---------------------------------------------------------------------------
// square = 1: the code table and sB
// ---------------------------------------------------------------------------
struct Lut8Args {
    const uint8_t* vals;
    int64_t vals_numel;
    const uint32_t* prefix;       // prefix[0], prefix[T]: the tensor's run relative to vals_offset
    int64_t T;
    const int64_t* vals_offset;
    int64_t dense_numel;          // K * N (cleared elements exist iff nnz < this)
    float relu2_scale;
    const float* r_scale;         // stored values' scale (may be null: bf16(scale^2) not applied)
    uint32_t* cmax;               // per-block maxima of code_max_kernel (kCodeMaxBlocks)
    float* b_scale;               // sB
    float* b_scale_out;           // optional copy for the caller
};

constexpr int kCodeMaxBlocks = 256;

// magnitude order of a stored code: its low 7 bits (e4m3fn / e5m2 codes of
// equal sign sort like their values; NaN codes above every finite one).
// Block b writes the largest magnitude of its 16-byte units of the run
// [vo + prefix[0], vo + prefix[T]) to cmax[b] (every block writes, so the
// slots need no clearing).
__global__ __launch_bounds__(256) void code_max_kernel(Lut8Args a)
{
    const int64_t vo = a.vals_offset ? *a.vals_offset : 0;
    int64_t b0 = vo + (int64_t)a.prefix[0];
    int64_t b1 = vo + (int64_t)a.prefix[a.T];
    if (b0 < 0) b0 = 0;
    if (b1 > a.vals_numel) b1 = a.vals_numel;
    uint32_t m = 0;
    if (b1 > b0) {
        const int64_t u0 = b0 >> 4, u1 = (b1 + 15) >> 4;
        const bs_rsrc rs = make_rsrc(a.vals + u0 * 16, (uint32_t)std::min<int64_t>(a.vals_numel - u0 * 16, 0xffffffffll));
        const int64_t stride = (int64_t)gridDim.x * 256;
        for (int64_t u = u0 + (int64_t)blockIdx.x * 256 + threadIdx.x; u < u1; u += stride) {
            const int64_t e0 = u * 16;
            uint32_t w[4];
            if (e0 + 16 <= a.vals_numel) {
                const uint4 v = load16(rs, (uint32_t)((u - u0) * 16));
                w[0] = v.x, w[1] = v.y, w[2] = v.z, w[3] = v.w;
            } else {
                // the unit crosses the end of vals: its readable bytes one by one
                w[0] = w[1] = w[2] = w[3] = 0u;
                for (int e = 0; e < 16 && e0 + e < a.vals_numel; e++)
                    w[e >> 2] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rs, (int)((u - u0) * 16 + e), 0, 0)
                                 << (8 * (e & 3));
            }
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const uint32_t c = (w[e >> 2] >> (8 * (e & 3))) & 0x7fu;
                const bool in = e0 + e >= b0 && e0 + e < b1;
                m = max(m, in ? c : 0u);
            }
        }
    }
    m = wave_max_u32(m);
    __shared__ uint32_t s_w[4];
    if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) a.cmax[blockIdx.x] = max(max(s_w[0], s_w[1]), max(s_w[2], s_w[3]));
}

// D(c) of code c as bf16 bits: the ReLU^2 unpack of fp8 storage
// (bf16((k v) v), then bf16(. * bf16(s^2)) with a scale)
template <int V_T>
__device__ __forceinline__ uint32_t relu2_dense_bits(uint32_t c, float k, bool has_scale, float s2b)
{
    const float v = fp8_to_f32<V_T>(c);
    uint32_t x = f32_to_bf16((k * v) * v);
    if (has_scale) x = f32_to_bf16(bf16_to_f32(x) * s2b);
    return x;
}

// The code table of square = 1 into tab[256] (all 256 threads of the block
// call this): sB = max(amax / 448, 1e-9) from code_max_kernel's maxima, and
// tab[c] = e4m3fn_RNE(D(c) / sB); the block with write_scale stores sB.
template <int V_T>
__device__ __forceinline__ void relu2_table(const Lut8Args& a, uint8_t* tab, bool write_scale)
{
    __shared__ float s_scale;
    const uint32_t c = threadIdx.x;
    const bool has_scale = a.r_scale != nullptr;
    float s2b = 1.0f;
    if (has_scale) {
        const float s = *a.r_scale;
        s2b = bf16_to_f32(f32_to_bf16(s * s));
    }
    const float k = a.relu2_scale;
    // code 0 stands for the cleared elements, which the ReLU^2 unpack writes
    // as bf16(0 * bf16(s^2)) (0 without a scale); stored codes are positive
    const uint32_t zero_x = has_scale ? f32_to_bf16(0.0f * s2b) : 0u;
    const uint32_t x = c == 0 ? zero_x : relu2_dense_bits<V_T>(c, k, has_scale, s2b);
    // the stored codes' largest magnitude, over code_max_kernel's blocks
    __shared__ uint32_t s_cm[4];
    const uint32_t cmw = wave_max_u32(c < (uint32_t)kCodeMaxBlocks ? a.cmax[c] : 0u);
    if ((c & 63) == 0) s_cm[c >> 6] = cmw;
    __syncthreads();
    if (c == 0) {
        const uint32_t cmax = max(max(s_cm[0], s_cm[1]), max(s_cm[2], s_cm[3]));
        const int64_t nnz = (int64_t)a.prefix[a.T] - (int64_t)a.prefix[0];
        // amax over |D| of the stored codes (the one of largest magnitude) and
        // of the cleared elements; NaN magnitudes sort above Inf
        uint32_t amag = 0;
        if (cmax != 0u) amag = relu2_dense_bits<V_T>(cmax, k, has_scale, s2b) & 0x7fffu;
        if (nnz < a.dense_numel) amag = max(amag, zero_x & 0x7fffu);
        const float amax = bf16_to_f32(amag);
        const float sc = amax / 448.0f;
        s_scale = (sc < 1e-9f) ? 1e-9f : sc;
        if (write_scale) {
            *a.b_scale = s_scale;
            if (a.b_scale_out) *a.b_scale_out = s_scale;
        }
    }
    __syncthreads();
    tab[c] = (uint8_t)f32_to_e4m3(bf16_to_f32(x) / s_scale);
    __syncthreads();
}

// square = 1: out[i] = table[vals[vo + prefix[0] + i]] for i < n, n = the
// run's length (prefix[T] - prefix[0], within vals and cap; cap a multiple of
// 16, so the whole 16-byte units the GEMM reads stay inside out), and
// *out_vo = -prefix[0]: the GEMM then finds tile t's run at out[prefix[t] +
// *out_vo].  Every block forms the code table itself (256 entries, a few
// instructions each; no separate launch); block 0 stores sB.  16 codes per
// thread and pass.
template <int V_T>
__global__ __launch_bounds__(256) void map_codes_kernel(Lut8Args a, uint8_t* out, int64_t cap, int64_t* out_vo)
{
    __shared__ uint8_t t[256];
    relu2_table<V_T>(a, t, blockIdx.x == 0);
    const int64_t vo = a.vals_offset ? *a.vals_offset : 0;
    const int64_t p0 = (int64_t)a.prefix[0];
    const int64_t b0 = vo + p0;
    int64_t n = (int64_t)a.prefix[a.T] - p0;
    if (n > cap) n = cap;
    if (b0 < 0 || b0 >= a.vals_numel) n = 0;
    else if (n > a.vals_numel - b0) n = a.vals_numel - b0;
    if (blockIdx.x == 0 && threadIdx.x == 0) *out_vo = -p0;
    if (n <= 0) return;
    // dword-aligned source base; sh = the run start's byte within its dword
    const int64_t base = b0 & ~(int64_t)3;
    const uint32_t sh = (uint32_t)(b0 & 3);
    const int64_t readable = std::min<int64_t>(a.vals_numel - base, 0xffffffffll);
    const bs_rsrc rs = make_rsrc(a.vals + base, (uint32_t)readable);
    const int64_t stride = (int64_t)gridDim.x * 256 * 16;
    for (int64_t j = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 16; j < n; j += stride) {
        uint32_t w[5];
        if (j + 20 <= readable) {
            const uint4 v = load16(rs, (uint32_t)j);
            w[0] = v.x, w[1] = v.y, w[2] = v.z, w[3] = v.w;
            w[4] = load4(rs, (uint32_t)j + 16u);
        } else {
            // the window crosses the end of vals: its readable bytes one by one
            w[0] = w[1] = w[2] = w[3] = w[4] = 0u;
            for (int e = 0; e < 20 && j + e < readable; e++)
                w[e >> 2] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rs, (int)(j + e), 0, 0) << (8 * (e & 3));
        }
        uint32_t o[4];
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const uint32_t x = __builtin_amdgcn_alignbyte(w[d + 1], w[d], sh);
            o[d] = (uint32_t)t[x & 0xffu] | ((uint32_t)t[(x >> 8) & 0xffu] << 8) |
                   ((uint32_t)t[(x >> 16) & 0xffu] << 16) | ((uint32_t)t[x >> 24] << 24);
        }
        *reinterpret_cast<uint4*>(out + j) = uint4{o[0], o[1], o[2], o[3]};
    }
}

// ---------------------------------------------------------------------------
// packed fp8 storage (pack_sbit): value i of the stream at bits [7 i, 7 i + 7)
// (least significant first), the code's low 7 bits (its sign bit is 0).  The
// GEMM stages unpacked codes, so the stream is unpacked by the pass that maps
// the codes (square = 1) or, for square = 0, by the same pass with the
// identity for its table: into the workspace run the GEMM reads.
// ---------------------------------------------------------------------------

// 16 consecutive codes from stream bit `bit` (counted from the resource's
// first byte, which is dword aligned): the five dwords from the one holding
// `bit` -- whole-dword reads while they lie inside the `readable` bytes, else
// byte by byte (bytes past the resource read 0) -- then code e at bits
// [7 e, 7 e + 7) past `bit`.
__device__ __forceinline__ uint4 packed7_x16(bs_rsrc rs, uint64_t bit, int64_t readable)
{
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
    uint32_t o[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const int b = 7 * e, wi = b >> 5, bs = b & 31;
        const uint32_t raw = bs + 7 <= 32 ? q[wi] >> bs : __builtin_amdgcn_alignbit(q[min(wi + 1, 3)], q[wi], bs);
        o[e >> 2] |= (raw & 0x7fu) << (8 * (e & 3));
    }
    return uint4{o[0], o[1], o[2], o[3]};
}

// The run [vo + prefix[0], vo + prefix[T]) of a packed stream (vals_numel
// bytes): its first value index b0, its length n (values wholly inside the
// stream), the resource from the dword holding value b0's first bit, and that
// bit's offset in the resource.
struct PackedRun {
    int64_t b0, n;
    bs_rsrc rs;
    int64_t readable;
    uint64_t bit0;
};
__device__ __forceinline__ PackedRun packed_run(const Lut8Args& a)
{
    PackedRun r;
    const int64_t vo = a.vals_offset ? *a.vals_offset : 0;
    r.b0 = vo + (int64_t)a.prefix[0];
    const int64_t whole = a.vals_numel * 8 / 7;         // values wholly inside the stream
    r.n = (int64_t)a.prefix[a.T] - (int64_t)a.prefix[0];
    if (r.b0 < 0 || r.b0 >= whole) r.n = 0;
    else if (r.n > whole - r.b0) r.n = whole - r.b0;
    const int64_t base = r.n > 0 ? ((r.b0 * 7) >> 5) * 4 : 0;
    r.readable = r.n > 0 ? std::min<int64_t>(a.vals_numel - base, 0xffffffffll) : 0;
    r.rs = make_rsrc(a.vals + base, (uint32_t)r.readable);
    r.bit0 = r.n > 0 ? (uint64_t)(r.b0 * 7 - base * 8) : 0;
    return r;
}

// code_max_kernel over a packed run
__global__ __launch_bounds__(256) void code_max_packed_kernel(Lut8Args a)
{
    const PackedRun r = packed_run(a);
    uint32_t m = 0;
    const int64_t stride = (int64_t)gridDim.x * 256 * 16;
    for (int64_t j = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 16; j < r.n; j += stride) {
        const uint4 v = packed7_x16(r.rs, r.bit0 + (uint64_t)j * 7u, r.readable);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 16; e++) m = max(m, j + e < r.n ? (w[e >> 2] >> (8 * (e & 3))) & 0x7fu : 0u);
    }
    m = wave_max_u32(m);
    __shared__ uint32_t s_w[4];
    if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) a.cmax[blockIdx.x] = max(max(s_w[0], s_w[1]), max(s_w[2], s_w[3]));
}

// map_codes_kernel reading a packed run; IDENT (square = 0): out[i] = the
// code itself, and the stored scale is copied to sB by copy_scale_kernel
template <int V_T, bool IDENT>
__global__ __launch_bounds__(256) void map_packed_kernel(Lut8Args a, uint8_t* out, int64_t cap, int64_t* out_vo)
{
    __shared__ uint8_t t[256];
    if constexpr (!IDENT) relu2_table<V_T>(a, t, blockIdx.x == 0);
    const PackedRun r = packed_run(a);
    const int64_t n = std::min<int64_t>(r.n, cap);
    if (blockIdx.x == 0 && threadIdx.x == 0) *out_vo = -(int64_t)a.prefix[0];
    const int64_t stride = (int64_t)gridDim.x * 256 * 16;
    for (int64_t j = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 16; j < n; j += stride) {
        const uint4 v = packed7_x16(r.rs, r.bit0 + (uint64_t)j * 7u, r.readable);
        uint32_t o[4] = {v.x, v.y, v.z, v.w};
        if constexpr (!IDENT) {
#pragma unroll
            for (int d = 0; d < 4; d++) {
                const uint32_t x = o[d];
                o[d] = (uint32_t)t[x & 0xffu] | ((uint32_t)t[(x >> 8) & 0xffu] << 8) |
                       ((uint32_t)t[(x >> 16) & 0xffu] << 16) | ((uint32_t)t[x >> 24] << 24);
            }
        }
        *reinterpret_cast<uint4*>(out + j) = uint4{o[0], o[1], o[2], o[3]};
    }
}

__global__ void copy_scale_kernel(const float* src, float* dst, float* dst2)
{
    if (threadIdx.x == 0) {
        *dst = *src;
        if (dst2) *dst2 = *src;
    }
}

// C = bf16(scale * sum over splits of part), summed in split order
__global__ __launch_bounds__(256) void splitk_reduce_scaled_kernel(const float* part, int split, int64_t n,
                                                                   const float* a_scale, const float* b_scale,
                                                                   uint16_t* C)
{
    const float sc = (*a_scale) * (*b_scale);
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
        float s = part[i];
        for (int k = 1; k < split; k++) s += part[(int64_t)k * n + i];
        C[i] = (uint16_t)f32_to_bf16(s * sc);
    }
}

__global__ __launch_bounds__(256) void zero_fill_u16_8_kernel(uint16_t* C, int64_t n)
{
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) C[i] = 0;
}

static int gemm8_split(int64_t M, int64_t N, int64_t K, int64_t bm, int64_t bn, int per_cu)
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

enum { CFG8_512 = 0, CFG8_256 = 1 };
struct Gemm8Plan {
    int cfg;
    int64_t bm, bn;
    int split;
};
template <typename CFG>
static void gemm8_shape(Gemm8Plan& p, int64_t M, int64_t N, int64_t K)
{
    p.bm = CFG::BM;
    p.bn = CFG::BN;
    p.split = gemm8_split(M, N, K, p.bm, p.bn, CFG::MINB);
}
static Gemm8Plan gemm8_plan(int64_t M, int64_t N, int64_t K)
{
    Gemm8Plan p;
    const int64_t pad512 = (M + Cfg8_512::BM - 1) / Cfg8_512::BM * Cfg8_512::BM;
    const int64_t pad256 = (M + Cfg8_256::BM - 1) / Cfg8_256::BM * Cfg8_256::BM;
    p.cfg = M >= Cfg8_512::BM && pad512 <= pad256 ? CFG8_512 : CFG8_256;
    // BITSPARSE_DW8_CFG selects a shape for tuning runs: 512 (8 waves of
    // 64 x 128) or 256 (2 x 2 waves of 128 x 128)
    if (const char* ev = getenv("BITSPARSE_DW8_CFG")) {
        const int v = atoi(ev);
        if (v == 512) p.cfg = CFG8_512;
        else if (v == 256) p.cfg = CFG8_256;
    }
    if (p.cfg == CFG8_512) gemm8_shape<Cfg8_512>(p, M, N, K);
    else gemm8_shape<Cfg8_256>(p, M, N, K);
    return p;
}

static int64_t apk8_nkb(int64_t K) { return (K + kBK - 1) / kBK; }
static int64_t apk8_bytes(int64_t M, int64_t K) { return (M + 31) / 32 * apk8_nkb(K) * 2048; }
static int64_t up256(int64_t x) { return (x + 255) / 256 * 256; }
constexpr int64_t kLutAreaBytes = 512 + 4 * kCodeMaxBlocks;     // sB at 256, code_max_kernel's maxima at 512
// square = 1: room for the mapped value run (at most K N codes, whole 16-byte
// units) and its offset word
static int64_t map8_cap(int64_t K, int64_t N) { return (K * N + 15) / 16 * 16; }
static int64_t map8_area(int64_t K, int64_t N) { return up256(map8_cap(K, N)) + 256; }

}  // namespace bs

using namespace bs;

extern "C" int64_t bs_gemm_compressed_b_fp8_workspace_bytes(int64_t M, int64_t N, int64_t K, int a_layout,
                                                            int square)
{
    (void)a_layout;
    if (M <= 0 || N <= 0 || K <= 0) return kLutAreaBytes;
    const int split = gemm8_plan(M, N, K).split;
    int64_t bytes = split > 1 ? up256((int64_t)split * M * N * 4) : 0;
    bytes += up256(apk8_bytes(M, K));
    if (square) bytes += map8_area(K, N);
    return bytes + kLutAreaBytes;
}

// packed: vals is a packed stream of vals_numel bytes (7-bit codes), unpacked
// (and for square = 1 mapped) into the workspace run the GEMM stages
static int gemm8_impl(const void* A, const float* a_scale, int64_t M, int64_t K, int64_t lda, int a_layout,
                      const void* vals, int vals_dtype, int64_t vals_numel, const uint8_t* bitmask,
                      const uint32_t* prefix, const int64_t* vals_offset, int64_t N, int square, float relu2_scale,
                      const float* b_scale, void* C, float* b_scale_out, void* workspace, int64_t workspace_bytes,
                      void* stream, bool packed, const char* fn)
{
    clear_error();
    if (M < 0 || N < 0 || K < 0) return set_error(BS_ERR_INVALID, "%s: negative shape", fn);
    if (a_layout != 0 && a_layout != 1) return set_error(BS_ERR_INVALID, "%s: bad a_layout", fn);
    if (vals_dtype != DT_E4M3FN && vals_dtype != DT_E5M2)
        return set_error(BS_ERR_INVALID, "%s: B must hold fp8 (e4m3fn or e5m2) values", fn);
    if (!square && b_scale == nullptr) return set_error(BS_ERR_INVALID, "%s: square=0 needs the stored scale", fn);
    if (a_scale == nullptr) return set_error(BS_ERR_INVALID, "%s: null a_scale", fn);
    if (a_layout == 0 && lda < M) return set_error(BS_ERR_INVALID, "%s: lda < M", fn);
    if (a_layout == 1 && lda < K) return set_error(BS_ERR_INVALID, "%s: lda < K", fn);
    if ((uint64_t)K * (uint64_t)N >= kMaxElemsUntested) return set_error(BS_ERR_INVALID, "%s: K*N must be < 2^31", fn);
    if (lda >= (1ll << 31)) return set_error(BS_ERR_INVALID, "%s: lda must be < 2^31", fn);
    if (M == 0 || N == 0) return BS_OK;
    if (C == nullptr) return set_error(BS_ERR_INVALID, "%s: null C", fn);
    if (((uintptr_t)C) & 1) return set_error(BS_ERR_INVALID, "%s: C misaligned", fn);
    // packed: the unpacked run takes the room of square = 1's mapped run
    const int64_t need = bs_gemm_compressed_b_fp8_workspace_bytes(M, N, K, a_layout, square || packed);
    if (workspace == nullptr || workspace_bytes < need)
        return set_error(BS_ERR_INVALID, "%s: workspace too small (%lld < %lld)", fn, (long long)workspace_bytes,
                         (long long)need);
    if (((uintptr_t)workspace) & 255) return set_error(BS_ERR_INVALID, "%s: workspace must be 256-byte aligned", fn);
    hipStream_t st = (hipStream_t)stream;
    const uint32_t ksteps = (uint32_t)((K + kBK - 1) / kBK);
    uint8_t* lut_area = (uint8_t*)workspace + need - kLutAreaBytes;
    float* sB = reinterpret_cast<float*>(lut_area + 256);
    uint32_t* cmax = reinterpret_cast<uint32_t*>(lut_area + 512);
    if (ksteps == 0) {
        // an empty sum: C = 0 (a fill kernel, no memset node in a captured graph)
        const int64_t n = M * N;
        const uint32_t nblk = (uint32_t)std::min<int64_t>((n + 255) / 256, 2048);
        hipLaunchKernelGGL(zero_fill_u16_8_kernel, dim3(nblk), dim3(256), 0, st, (uint16_t*)C, n);
        hipError_t e = hipGetLastError();
        return e == hipSuccess ? BS_OK : set_error(BS_ERR_HIP, "%s: %s", fn, hipGetErrorString(e));
    }
    if (A == nullptr || bitmask == nullptr || prefix == nullptr || (vals_numel > 0 && vals == nullptr))
        return set_error(BS_ERR_INVALID, "%s: null pointer", fn);
    if (((uintptr_t)vals) & (packed ? 3 : 15))
        return set_error(BS_ERR_INVALID, "%s: vals must be %d-byte aligned", fn, packed ? 4 : 16);
    const Gemm8Plan plan = gemm8_plan(M, N, K);
    const int split = plan.split;
    const int64_t part_bytes = split > 1 ? up256((int64_t)split * M * N * 4) : 0;
    const int64_t nkb = apk8_nkb(K), nrb = (M + 31) / 32;
    // A fragment offsets (row block < 4 of a wave, k block, lane) are 32-bit
    if (nkb >= (1ll << 18)) return set_error(BS_ERR_INVALID, "%s: K must be < 2^24", fn);
    if (apk8_bytes(M, K) > (1ll << 31))
        return set_error(BS_ERR_INVALID, "%s: M*K must be < 2^31 (A's fragment-order copy)", fn);
    const int64_t grid_n = (N + kTile - 1) / kTile;
    const int64_t T = (int64_t)ksteps * grid_n;

    // B code table and scale
    Lut8Args la{};
    la.vals = (const uint8_t*)vals;
    la.vals_numel = vals_numel;
    la.prefix = prefix;
    la.T = T;
    la.vals_offset = vals_offset;
    la.dense_numel = K * N;
    la.relu2_scale = relu2_scale;
    la.r_scale = b_scale;
    la.cmax = cmax;
    la.b_scale = sB;
    la.b_scale_out = b_scale_out;
    // square / packed: the mapped (or unpacked) value run after A's packed copy
    const int64_t map_cap = map8_cap(K, N);
    uint8_t* map_out = (uint8_t*)workspace + part_bytes + up256(apk8_bytes(M, K));
    int64_t* map_vo = reinterpret_cast<int64_t*>(map_out + up256(map_cap));
    const uint32_t mblk = (uint32_t)std::min<int64_t>((map_cap + 4095) / 4096, 2048);
    if (packed) {
        if (square) {
            hipLaunchKernelGGL(code_max_packed_kernel, dim3(kCodeMaxBlocks), dim3(256), 0, st, la);
            if (vals_dtype == DT_E4M3FN)
                hipLaunchKernelGGL((map_packed_kernel<DT_E4M3FN, false>), dim3(mblk), dim3(256), 0, st, la, map_out,
                                   map_cap, map_vo);
            else
                hipLaunchKernelGGL((map_packed_kernel<DT_E5M2, false>), dim3(mblk), dim3(256), 0, st, la, map_out,
                                   map_cap, map_vo);
        } else {
            hipLaunchKernelGGL(copy_scale_kernel, dim3(1), dim3(64), 0, st, b_scale, sB, b_scale_out);
            hipLaunchKernelGGL((map_packed_kernel<DT_E4M3FN, true>), dim3(mblk), dim3(256), 0, st, la, map_out,
                               map_cap, map_vo);
        }
    } else if (square) {
        hipLaunchKernelGGL(code_max_kernel, dim3(kCodeMaxBlocks), dim3(256), 0, st, la);
        if (vals_dtype == DT_E4M3FN)
            hipLaunchKernelGGL(map_codes_kernel<DT_E4M3FN>, dim3(mblk), dim3(256), 0, st, la, map_out, map_cap, map_vo);
        else
            hipLaunchKernelGGL(map_codes_kernel<DT_E5M2>, dim3(mblk), dim3(256), 0, st, la, map_out, map_cap, map_vo);
    } else {
        hipLaunchKernelGGL(copy_scale_kernel, dim3(1), dim3(64), 0, st, b_scale, sB, b_scale_out);
    }

    // A into MFMA-fragment order (workspace after the partial sums)
    uint8_t* apk = (uint8_t*)workspace + part_bytes;
    if (a_layout == 0) {
        hipLaunchKernelGGL(pack_a8_t_kernel, dim3((uint32_t)nkb, (uint32_t)((M + 63) / 64)), dim3(256), 0, st,
                           (const uint8_t*)A, K, M, lda, apk, (uint32_t)nrb);
    } else {
        const int64_t pieces = nrb * nkb * 128;
        int64_t nblk = (pieces + 255) / 256;
        if (nblk > 4096) nblk = 4096;
        hipLaunchKernelGGL(pack_a8_n_kernel, dim3((uint32_t)nblk), dim3(256), 0, st, (const uint8_t*)A, K, M, lda,
                           apk, (uint32_t)nrb, pieces);
    }
    Gemm8Args g{};
    g.Apk = apk;
    g.M = M;
    g.K = K;
    g.nkb = (uint32_t)nkb;
    g.nrb = (uint32_t)nrb;
    const bool mapped = square || packed;
    g.vals = mapped ? map_out : (const uint8_t*)vals;
    g.vals_numel = mapped ? map_cap : vals_numel;
    g.bitmask = bitmask;
    g.prefix = prefix;
    g.vals_offset = mapped ? map_vo : vals_offset;
    g.N = N;
    g.grid_n = (uint32_t)grid_n;
    const uint32_t nt = (uint32_t)(plan.bn / kTile);
    g.tiles_n = (g.grid_n + nt - 1) / nt;
    g.tiles_m = (uint32_t)((M + plan.bm - 1) / plan.bm);
    g.a_scale = a_scale;
    g.b_scale = sB;
    g.C = (uint16_t*)C;
    g.part = split > 1 ? (float*)workspace : nullptr;
    g.ksteps = ksteps;
    g.ksteps_per_split = (ksteps + split - 1) / split;
    if (g.ksteps_per_split > (uint32_t)kMaxSteps) return set_error(BS_ERR_INVALID, "%s: internal split error", fn);
    const uint64_t blocks = (uint64_t)g.tiles_m * g.tiles_n * (uint64_t)split;
    if (blocks >= (1ull << 31)) return set_error(BS_ERR_INVALID, "%s: grid too large", fn);
#define BS_GEMM8_GO(CFG, FMT) \
    hipLaunchKernelGGL((gemm_cb8_kernel<CFG, FMT>), dim3((uint32_t)blocks), dim3(CFG::THREADS), 0, st, g)
#define BS_GEMM8_LAUNCH(FMT)                                     \
    do {                                                         \
        if (plan.cfg == CFG8_512) BS_GEMM8_GO(Cfg8_512, FMT);   \
        else BS_GEMM8_GO(Cfg8_256, FMT);                         \
    } while (0)
    // square: the mapped codes are e4m3fn (to_fp8's); else the stored format
    if (square || vals_dtype == DT_E4M3FN) BS_GEMM8_LAUNCH(0);
    else BS_GEMM8_LAUNCH(1);
#undef BS_GEMM8_LAUNCH
#undef BS_GEMM8_GO
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && split > 1) {
        const int64_t n = M * N;
        int64_t nblk = (n + 255) / 256;
        if (nblk > 2048) nblk = 2048;
        hipLaunchKernelGGL(splitk_reduce_scaled_kernel, dim3((uint32_t)nblk), dim3(256), 0, st,
                           (const float*)workspace, split, n, a_scale, (const float*)sB, (uint16_t*)C);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "%s launch: %s", fn, hipGetErrorString(e));
    return BS_OK;
}

extern "C" int bs_gemm_compressed_b_fp8(const void* A, const float* a_scale, int64_t M, int64_t K, int64_t lda,
                                        int a_layout, const void* vals, int vals_dtype, int64_t vals_numel,
                                        const uint8_t* bitmask, const uint32_t* prefix, const int64_t* vals_offset,
                                        int64_t N, int square, float relu2_scale, const float* b_scale, void* C,
                                        float* b_scale_out, void* workspace, int64_t workspace_bytes, void* stream)
{
    return gemm8_impl(A, a_scale, M, K, lda, a_layout, vals, vals_dtype, vals_numel, bitmask, prefix, vals_offset, N,
                      square, relu2_scale, b_scale, C, b_scale_out, workspace, workspace_bytes, stream, false,
                      "bs_gemm_compressed_b_fp8");
}

extern "C" int bs_gemm_compressed_b_fp8_packed(const void* A, const float* a_scale, int64_t M, int64_t K,
                                               int64_t lda, int a_layout, const void* stream_bytes, int vals_dtype,
                                               int64_t stream_nbytes, const uint8_t* bitmask, const uint32_t* prefix,
                                               const int64_t* vals_offset, int64_t N, int square, float relu2_scale,
                                               const float* b_scale, void* C, float* b_scale_out, void* workspace,
                                               int64_t workspace_bytes, void* stream)
{
    return gemm8_impl(A, a_scale, M, K, lda, a_layout, stream_bytes, vals_dtype, stream_nbytes, bitmask, prefix,
                      vals_offset, N, square, relu2_scale, b_scale, C, b_scale_out, workspace, workspace_bytes,
                      stream, true, "bs_gemm_compressed_b_fp8_packed");
}
