// Up-projection GEMM with the ReLU and the compress in its epilogue (gfx950):
//     z = bf16(bf16(x @ W^T) + b),  h = relu(z)
//     h -> 64x64-tile bitmask + prefix + values (the BitsparseTensor format)
// in one kernel, so the activation is never read back from HBM to be
// compressed.  Replaces the reference's z = x @ W1^T; z = z + b1;
// h = z.relu_(); dense_to_tilesparse(h) (lib_sparse/layers.py:86-89, :29, :37;
// lib_sparse/src/functions.py:55-99).  The two bf16 roundings (the GEMM's
// output, then the bias add) are the reference's; the fp32 accumulation order
// is this kernel's own.
//
// GEMM: a workgroup is 4 waves (2 x 2) on a 128 x 192 tile of z; each wave
// holds 64 x 96 in 2 x 3 v_mfma_f32_32x32x16_bf16 accumulators (96 VGPRs), so
// that a wave needs at most 256 VGPRs and the workgroup 80 KiB of LDS: two
// workgroups share a CU, and one's epilogue (VALU, LDS and memory latency)
// runs beside the other's MFMAs.  x [M, K] and W [N, K] are both
// k-contiguous, so a K-step (64) stages a 128 x 64 slab of x and a 192 x 64
// slab of W in LDS as 16-byte chunks, eight per row.  The chunk index is
// XOR-swizzled with (row / 2) % 8: 16 lanes storing two rows, or reading one
// chunk of 16 rows, then touch all 64 banks once.  Slabs are double-buffered
// (one barrier per step); the next step's slabs are loaded into registers
// while the current step's MFMAs run.
//
// Epilogue: the tile (bias, roundings, torch's GPU relu) is staged in LDS as
// bf16 over the slab buffers; elements outside the matrix are staged as 0.
// Tile row u of the workgroup (three format tiles) is one look-back "unit",
// shared by waves u and u + 2, each taking half of its 24 chunk rounds in
// run order.  Units are consecutive in tile order (unit (tm, cb) = tiles
// tm * grid_n + 3 cb .. +2), so the decoupled look-back of the codec applies
// unchanged.  The two waves of a unit
//   * write its 64 rows of h (16-byte stores) and the tiles' bitmask bytes,
//   * exchange their counts through LDS; one publishes the unit's count,
//   * compact the tiles' set elements into one LDS run (v_perm selectors per
//     mask byte), each its half,
//   * both resolve the unit's offset from the preceding units' status words
//     (one publishes the inclusive prefix and writes the prefix entries),
//   * and store the run with 16-byte stores, with element stores at its two
//     partial ends.
//
// Look-back order: unit (tm, cb) waits for every unit before it in tile
// order, among them (tm - 1, NB - 1), the last workgroup of the same
// 128-row strip when tm is not the strip's first tile row: a workgroup
// dispatched after it.  Every workgroup publishes its counts before it waits
// for anything, so a strip completes once all of its NB workgroups have been
// resident.  The host bounds NB by half the workgroups the GPU holds at once
// (the occupancy API's count per CU times the CUs).  Work from other streams
// can still lower residency below that: a wait then ends after the caller's
// patience with the time-out flag set (its own word, never the capacity
// flags), the unit's offset is wrong, and the caller must discard the result.
#include <algorithm>
#include <atomic>

#include "bs_device.h"
#include "bs_host.h"
#include "compact.h"
#include "gemm_common.h"

namespace bs {

typedef __bf16 up_bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int kUpBM = 128, kUpBN = 192;
constexpr int kUpIM = 2, kUpJN = 3;                     // 32x32 accumulator blocks per wave
constexpr int kUpUnits = kUpBM / kTile;                 // units (tile rows) per workgroup
constexpr int kUpTiles = kUpBN / kTile;                 // format tiles per unit
constexpr int kUpAStage = kUpBM * 128;                  // x slab: 128 rows x 64 k bf16
constexpr int kUpBStage = kUpBN * 128;                  // W slab: 192 rows x 64 k bf16
constexpr int kUpMainLds = 2 * (kUpAStage + kUpBStage);
constexpr int kUpHP = kUpBN * 2 + 16;                   // staged h row pitch, bytes
// after the main loop: staged h, the compaction selectors (8 dwords per
// mask byte) and the units' count exchange, all inside the slab buffers
constexpr int kUpOffSel = kUpBM * kUpHP;
constexpr int kUpOffCnt = kUpOffSel + 256 * 32;
constexpr int kUpEpiLds = kUpOffCnt + kUpUnits * 2 * 4 * 4;
constexpr int kUpLds = kUpMainLds > kUpEpiLds ? kUpMainLds : kUpEpiLds;
constexpr int kUpHalfRounds = 4 * kUpTiles;             // chunk rounds of half a unit, at most
// the epilogue: four waves, two per unit; per-tile counts kept for three tiles
static_assert(kUpUnits == 2 && kUpTiles == 3, "epilogue layout");
// a unit's compacted run (phase <= 7, three tiles, the 8-element write
// overrun) fits in the wave's 64 staged rows, where it is built
static_assert(2 * (7 + kUpTiles * kTileNumel + 8) <= 64 * kUpHP, "unit run");
// two workgroups per CU (160 KiB of LDS)
static_assert(kUpLds <= 80 * 1024, "LDS budget");

struct UpArgs {
    const uint16_t* x;            // [M, K], row stride ldx
    const uint16_t* w;            // [N, K], row stride ldw
    const uint16_t* bias;         // [N] or null
    uint16_t* h;                  // [M, N], row stride ldh, or null
    int64_t ldx, ldw, ldh;
    int64_t M, N, K;
    uint32_t grid_n, grid_m;      // format tiles
    uint32_t nb;                  // workgroups (units) per tile row
    uint32_t T;
    uint8_t* bitmask;
    uint32_t* prefix;
    uint16_t* vals;
    int64_t vals_capacity;        // elements
    const int64_t* offset_in;
    int32_t align8;
    int64_t* offset_out;
    int64_t* start_out;
    int32_t* err;
    int32_t* timeout;             // set to 1 when a look-back wait gave up (device or mapped host memory)
    uint64_t* status;             // one word per unit
    uint32_t epoch;
    uint64_t patience;            // ticks a look-back wait may last (0: give up at once)
};

// torch's GPU relu on bf16 bits: x <= 0 (either zero included) -> +0, NaN
// and positive values keep their bits
__device__ __forceinline__ uint32_t relu_bf16_bits(uint32_t b) { return (b - 0x8000u) < 0x7f81u ? 0u : b; }

// Default look-back patience (s_memrealtime ticks, 100 MHz: 20 ms).  A wait
// longer than the patience ends with *timeout set: every predecessor
// publishes before it waits for anything, so with all of a strip's
// workgroups resident no wait comes near it; it guarantees that every wave
// ends when they are not.  Patience 0 makes every unit but the first give up
// without waiting (the tests force the time-out path that way).
constexpr uint64_t kUpLookbackGiveUpTicks = 2000000;

// Exclusive prefix of unit u from the status words of units 0 .. u-1.  Each
// read covers kUpLbWords * 64 units: lane j
// takes units pos - kUpLbWords j - i, i < kUpLbWords, nearest first, and the
// walk sums values back to the nearest inclusive prefix; it re-reads while a
// word it needs is unpublished.
constexpr int kUpLbWords = 4;

// The time-out flag takes a plain store at system scope (no read-modify-write,
// so it may live in mapped pinned host memory, where atomics need the bus's
// support); every writer stores the same 1.
__device__ __forceinline__ void set_timeout(int32_t* f)
{
    __hip_atomic_store(f, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ uint32_t up_lookback(const UpArgs& a, uint32_t u, int lane)
{
    uint32_t excl = 0;
    int64_t pos = (int64_t)u - 1;
    if (a.patience == 0 && pos >= 0) {          // the forced time-out: no wait at all
        if (lane == 0 && a.timeout) set_timeout(a.timeout);
        return 0u;
    }
    const uint64_t t0 = wall_clock64();
    while (pos >= 0) {
        uint32_t sum = 0;
        bool unpub = false, inc = false;
        // all of the lane's words in flight at once: unconditional loads (a
        // word before unit 0 reads unit 0 and is replaced by an inclusive 0)
        uint64_t w[kUpLbWords];
#pragma unroll
        for (int i = 0; i < kUpLbWords; i++) {
            const int64_t q = pos - kUpLbWords * lane - i;
            w[i] = ld_relaxed(&a.status[q >= 0 ? q : 0]);
        }
#pragma unroll
        for (int i = 0; i < kUpLbWords; i++) {
            const int64_t q = pos - kUpLbWords * lane - i;
            const uint64_t s = q >= 0 ? w[i] : pack_status(a.epoch, kFlagInc, 0u);
            const uint32_t flag = (uint32_t)(s >> 34) == a.epoch ? (uint32_t)(s >> 32) & 3u : 0u;
            if (!inc) {                  // words up to the lane's nearest inclusive prefix
                unpub |= flag == 0u;
                sum += (uint32_t)s;
                inc = flag == kFlagInc;
            }
        }
        const uint64_t incs = __ballot(inc);
        const int first = incs ? __ffsll((unsigned long long)incs) - 1 : 63;   // last lane needed
        const uint64_t need = first == 63 ? ~0ull : ((2ull << first) - 1ull);
        if (__ballot(unpub) & need) {
            if (wall_clock64() - t0 > a.patience) {
                if (lane == 0 && a.timeout) set_timeout(a.timeout);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
            continue;
        }
        excl += wave_sum_u32(lane <= first ? sum : 0u);
        if (incs) break;
        pos -= 64 * kUpLbWords;
    }
    return excl;
}

__global__ __launch_bounds__(256, 2) void up_relu_compress_kernel(UpArgs a)
{
    __shared__ __align__(16) uint8_t lds[kUpLds];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const uint32_t strip = blockIdx.x / a.nb, cb = blockIdx.x % a.nb;
    const int64_t m0 = (int64_t)strip * kUpBM, n0 = (int64_t)cb * kUpBN;

    uint32_t* sel_s = reinterpret_cast<uint32_t*>(lds + kUpOffSel);
    // the cursor, read at the start: a load issued in the epilogue waits for
    // every earlier h / bitmask store as well (one vmcnt counts both)
    int64_t start = a.offset_in ? *a.offset_in : 0;
    if (a.align8) start = (start + 7) & ~(int64_t)7;

    // ---- slab loads: thread t moves chunk t % 8 of rows t / 8 + 32 i; rows
    // past the matrix read zero through the resources, chunks past K are
    // zeroed when stored (K % 8 == 0: a chunk is wholly inside or outside)
    const int64_t rows_a = std::min<int64_t>(kUpBM, a.M - m0);
    const int64_t rows_b = std::min<int64_t>(kUpBN, a.N - n0);
    const bs_rsrc rsx = make_rsrc(a.x + m0 * a.ldx, (uint32_t)(((rows_a - 1) * a.ldx + a.K) * 2));
    const bs_rsrc rsw = make_rsrc(a.w + n0 * a.ldw, (uint32_t)(((rows_b - 1) * a.ldw + a.K) * 2));
    const int c8 = tid & 7, r8 = tid >> 3;
    const uint32_t swz = (uint32_t)((r8 >> 1) & 7);        // rows r8 + 32 i share it
    const uint32_t xrow = (uint32_t)(r8 * a.ldx * 2), xstep = (uint32_t)(32 * a.ldx * 2);
    const uint32_t wrow = (uint32_t)(r8 * a.ldw * 2), wstep = (uint32_t)(32 * a.ldw * 2);
    // two register sets: slab s + 2 is loaded while slab s + 1, loaded a
    // step earlier, waits to be stored -- each load gets two steps of MFMAs
    uint4 ga[2][kUpBM / 32], gb[2][kUpBN / 32];
    auto gload = [&](int s, auto SET) __attribute__((always_inline)) {
        constexpr int R = decltype(SET)::value;
        const uint32_t koff = (uint32_t)(s * 64 + 8 * c8) * 2u;
#pragma unroll
        for (int i = 0; i < kUpBM / 32; i++) ga[R][i] = load16(rsx, xrow + (uint32_t)i * xstep + koff);
#pragma unroll
        for (int i = 0; i < kUpBN / 32; i++) gb[R][i] = load16(rsw, wrow + (uint32_t)i * wstep + koff);
    };
    auto lstore = [&](int s, int buf, auto SET) __attribute__((always_inline)) {
        constexpr int R = decltype(SET)::value;
        // a mask, not a select of two values: a select of an array element
        // becomes a load through a selected pointer, which puts the array in
        // scratch memory
        const uint32_t km = (int64_t)s * 64 + 8 * c8 < a.K ? 0xffffffffu : 0u;
        uint8_t* As = lds + buf * kUpAStage;
        uint8_t* Bs = lds + 2 * kUpAStage + buf * kUpBStage;
        const uint32_t coff = ((uint32_t)c8 ^ swz) << 4;
#pragma unroll
        for (int i = 0; i < kUpBM / 32; i++)
            *reinterpret_cast<uint4*>(As + (r8 + 32 * i) * 128 + coff) =
                uint4{ga[R][i].x & km, ga[R][i].y & km, ga[R][i].z & km, ga[R][i].w & km};
#pragma unroll
        for (int i = 0; i < kUpBN / 32; i++)
            *reinterpret_cast<uint4*>(Bs + (r8 + 32 * i) * 128 + coff) =
                uint4{gb[R][i].x & km, gb[R][i].y & km, gb[R][i].z & km, gb[R][i].w & km};
    };

    // one chunk of the slab traffic: n < 8 the x rows r8 + 32 n, else the W
    // rows r8 + 32 (n - 8)
    auto gload1 = [&](int s, auto SET, auto NI) __attribute__((always_inline)) {
        constexpr int R = decltype(SET)::value, n = decltype(NI)::value;
        const uint32_t koff = (uint32_t)(s * 64 + 8 * c8) * 2u;
        if constexpr (n < kUpBM / 32) ga[R][n] = load16(rsx, xrow + (uint32_t)n * xstep + koff);
        else gb[R][n - kUpBM / 32] = load16(rsw, wrow + (uint32_t)(n - kUpBM / 32) * wstep + koff);
    };
    auto lstore1 = [&](int buf, uint32_t km, auto SET, auto NI) __attribute__((always_inline)) {
        constexpr int R = decltype(SET)::value, n = decltype(NI)::value;
        const uint32_t coff = ((uint32_t)c8 ^ swz) << 4;
        if constexpr (n < kUpBM / 32) {
            uint8_t* As = lds + buf * kUpAStage;
            *reinterpret_cast<uint4*>(As + (r8 + 32 * n) * 128 + coff) =
                uint4{ga[R][n].x & km, ga[R][n].y & km, ga[R][n].z & km, ga[R][n].w & km};
        } else {
            constexpr int nb = n - kUpBM / 32;
            uint8_t* Bs = lds + 2 * kUpAStage + buf * kUpBStage;
            *reinterpret_cast<uint4*>(Bs + (r8 + 32 * nb) * 128 + coff) =
                uint4{gb[R][nb].x & km, gb[R][nb].y & km, gb[R][nb].z & km, gb[R][nb].w & km};
        }
    };
    constexpr int kChunks = kUpBM / 32 + kUpBN / 32;     // slab chunks per thread per step

    // ---- fragments of k-slice ks (16 k): lane l reads row 32 i + l % 32,
    // chunk 2 ks + l / 32 of its wave's rows
    const int fl = lane & 31;
    const uint32_t fswz = (uint32_t)((fl >> 1) & 7);
    const int arow = wm * 64 + fl, brow = wn * 96 + fl;
    up_bf16x8_t fa[2][kUpIM], fb[2][kUpJN];
    auto fread = [&](int buf, int ks, auto SET) __attribute__((always_inline)) {
        constexpr int S = decltype(SET)::value;
        const uint8_t* As = lds + buf * kUpAStage;
        const uint8_t* Bs = lds + 2 * kUpAStage + buf * kUpBStage;
        const uint32_t coff = (((uint32_t)(2 * ks + (lane >> 5))) ^ fswz) << 4;
#pragma unroll
        for (int i = 0; i < kUpIM; i++)
            fa[S][i] = __builtin_bit_cast(up_bf16x8_t, *reinterpret_cast<const uint4*>(As + (arow + 32 * i) * 128 + coff));
#pragma unroll
        for (int j = 0; j < kUpJN; j++)
            fb[S][j] = __builtin_bit_cast(up_bf16x8_t, *reinterpret_cast<const uint4*>(Bs + (brow + 32 * j) * 128 + coff));
    };

    f32x16_t acc[kUpIM][kUpJN];
#pragma unroll
    for (int i = 0; i < kUpIM; i++)
#pragma unroll
        for (int j = 0; j < kUpJN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    // Step s: slab s in LDS buffer s & 1, its k-slice ks fragments in set
    // ks & 1 (the next slice's read during the current slice's MFMAs).
    // During step s, slab s + 2 is loaded into register set s & 1 and slab
    // s + 1 (register set (s + 1) & 1, loaded during step s - 1) is stored
    // into the other LDS buffer, each load and store behind an MFMA; one
    // barrier ends the step.
    const int nsteps = (int)((a.K + 63) / 64);
    if (nsteps > 0) {
        gload(0, IC<0>{});
        gload(std::min(1, nsteps - 1), IC<1>{});
        lstore(0, 0, IC<0>{});
    }
    __syncthreads();
    if (nsteps > 0) fread(0, 0, IC<0>{});
    auto step = [&](int s, auto PI) __attribute__((always_inline)) {
        constexpr int P = decltype(PI)::value;           // s & 1
        // slab s + 2 (past the end: the last slab again, so the loads in
        // flight, and the waits that count them, are the same on every path)
        // streams into register set P and slab s + 1 out of set P ^ 1 into
        // LDS buffer P ^ 1 (unused during this step; after the last step the
        // store is harmless), one chunk after each of the first MFMAs
        const int sl = std::min(s + 2, nsteps - 1);
        const uint32_t km = (int64_t)(s + 1) * 64 + 8 * c8 < a.K ? 0xffffffffu : 0u;
        static_for<4>([&](auto KS) __attribute__((always_inline)) {
            constexpr int ks = decltype(KS)::value, cur = ks & 1;
            // the next slice's fragment reads first, then this slice's twelve
            // MFMAs (the sched barriers fix the issue order)
            if constexpr (ks < 3) fread(P, ks + 1, IC<cur ^ 1>{});
            __builtin_amdgcn_sched_barrier(0);
            static_for<kUpIM * kUpJN>([&](auto MI) __attribute__((always_inline)) {
                constexpr int m = decltype(MI)::value, i = m / kUpJN, j = m % kUpJN;
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[cur][i], fb[cur][j], acc[i][j], 0, 0, 0);
                constexpr int q = ks * kUpIM * kUpJN + m;
                if constexpr (q < 2 * kChunks) {
                    if constexpr (q % 2 == 0) lstore1(P ^ 1, km, IC<P ^ 1>{}, IC<q / 2>{});
                    else gload1(sl, IC<P>{}, IC<q / 2>{});
                }
                __builtin_amdgcn_sched_barrier(0);
            });
        });
        __syncthreads();
        if (s + 1 < nsteps) fread(P ^ 1, 0, IC<0>{});
    };
    int s = 0;
    for (; s + 1 < nsteps; s += 2) {
        step(s, IC<0>{});
        step(s + 1, IC<1>{});
    }
    if (s < nsteps) step(s, IC<0>{});

    // ---- stage h = relu(bf16(bf16(acc) + b)) as bf16 (0 outside the matrix).
    // Accumulator element r of lane l of a 32x32 block is row 8 (r / 4) +
    // 4 (l / 32) + r % 4, column l % 32; elements r, r + 1 (r even) are two
    // consecutive rows of one column and are converted together.  Without a
    // bias the add is skipped: adding +0 can only turn -0 into +0, which the
    // relu does anyway.
    uint8_t* hs = lds;
    {
        const int rq = 4 * (lane >> 5);
        const int rows_in = (int)std::min<int64_t>(kUpBM, a.M - m0);
        typedef float f32x2_t __attribute__((ext_vector_type(2)));
        typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
        typedef short i16x2_t __attribute__((ext_vector_type(2)));
        // torch's GPU relu of two bf16 halves (x <= 0 -> +0, NaN kept): a half
        // is kept iff its bits are >= -127 as int16 (+0, positive values, +Inf
        // and every NaN; -0, negative values and -Inf are below), i.e. iff its
        // saturating int16 sum with 127 is nonnegative: three packed ops
        auto relu2x = [](uint32_t hp) __attribute__((always_inline)) {
            const i16x2_t d = __builtin_elementwise_add_sat(__builtin_bit_cast(i16x2_t, hp), (i16x2_t)(127));
            return hp & ~__builtin_bit_cast(uint32_t, (i16x2_t)(d >> (i16x2_t)(15)));
        };
        auto stage = [&](auto BOUNDS, auto BIAS) __attribute__((always_inline)) {
            constexpr bool BD = decltype(BOUNDS)::value, HB = decltype(BIAS)::value;
#pragma unroll
            for (int j = 0; j < kUpJN; j++) {
                const int col = wn * 96 + 32 * j + fl;
                const bool cin = n0 + col < a.N;
                float bj = 0.0f;
                if constexpr (HB) bj = cin ? bf16_to_f32(a.bias[n0 + col]) : 0.0f;
                uint8_t* cp = hs + col * 2;
#pragma unroll
                for (int i = 0; i < kUpIM; i++) {
#pragma unroll
                    for (int r = 0; r < 16; r += 2) {
                        const int row = wm * 64 + 32 * i + 8 * (r >> 2) + rq + (r & 3);
                        uint32_t hp = __builtin_bit_cast(
                            uint32_t, __builtin_convertvector(f32x2_t{acc[i][j][r], acc[i][j][r + 1]}, bf16x2_t));
                        if constexpr (HB) {
                            const f32x2_t zb = {__uint_as_float(hp << 16) + bj, __uint_as_float(hp & 0xffff0000u) + bj};
                            hp = __builtin_bit_cast(uint32_t, __builtin_convertvector(zb, bf16x2_t));
                        }
                        uint32_t h2 = relu2x(hp);
                        if constexpr (BD)
                            h2 &= (cin && row < rows_in ? 0x0000ffffu : 0u) | (cin && row + 1 < rows_in ? 0xffff0000u : 0u);
                        *reinterpret_cast<uint16_t*>(cp + row * kUpHP) = (uint16_t)h2;
                        *reinterpret_cast<uint16_t*>(cp + (row + 1) * kUpHP) = (uint16_t)(h2 >> 16);
                    }
                }
            }
        };
        const bool whole = rows_in == kUpBM && n0 + kUpBN <= a.N;
        if (a.bias == nullptr) {
            if (whole) stage(IC<false>{}, IC<false>{});
            else stage(IC<true>{}, IC<false>{});
        } else {
            if (whole) stage(IC<false>{}, IC<true>{});
            else stage(IC<true>{}, IC<true>{});
        }
    }
    {
        uint32_t sel[8];
        compaction_selectors<2>((uint32_t)tid, sel);
        *reinterpret_cast<uint4*>(&sel_s[tid * 8]) = uint4{sel[0], sel[1], sel[2], sel[3]};
        *reinterpret_cast<uint4*>(&sel_s[tid * 8 + 4]) = uint4{sel[4], sel[5], sel[6], sel[7]};
    }
    __syncthreads();

    // ---- epilogue.  Unit ui (tile row ui of the workgroup: rows 64 ui .. +63
    // of hs, three format tiles) is shared by waves ui and ui + kUpUnits.  Its
    // 8 * ntiles chunk rounds -- tile tt, round k: lane l takes chunk 64 k + l,
    // tile row 8 k + l / 8, columns 8 (l % 8) .. +7, the format's byte order --
    // split into two halves in run order: half 0 takes the first 4 * ntiles,
    // half 1 the rest.  Every wave passes the same barriers; the waves of a
    // unit past the matrix do no work.
    const int ui = wave % kUpUnits, half = wave / kUpUnits;
    const uint32_t tm = strip * (uint32_t)kUpUnits + (uint32_t)ui;
    const bool active = tm < a.grid_m;
    const uint8_t* hw = hs + ui * 64 * kUpHP;
    const int64_t grow0 = m0 + (int64_t)ui * 64;
    const uint32_t t0 = tm * a.grid_n + cb * (uint32_t)kUpTiles;
    const int ntiles = (int)std::min<uint32_t>((uint32_t)kUpTiles, a.grid_n - cb * (uint32_t)kUpTiles);
    const int nr = 4 * ntiles, r0 = half * nr;          // the half's rounds: r0 .. r0 + nr - 1
    const int lrow = lane >> 3, lcol = (lane & 7) * 16;   // byte offset of the lane's chunk in a tile row
    uint32_t* cnt_s = reinterpret_cast<uint32_t*>(lds + kUpOffCnt);   // [unit][half][tile] counts

    // bitmask bytes and the half's per-tile counts.  Every round's chunk is
    // read first (rounds past nr read staged rows of the same tile row: in
    // bounds, their masks are dropped); a half spans at most two tiles, ta
    // for its rounds i < bnd and ta + 1 after, so two lane counts packed in
    // one word take one wave sum.
    uint32_t mk[kUpHalfRounds / 4] = {};                // the half's mask bytes, 4 per register
    uint4 hv[kUpHalfRounds];                            // the lane's chunks, reused by the compaction
    const int ta = r0 >> 3, bnd = 8 - (r0 & 7);
    if (active) {
#pragma unroll
        for (int i = 0; i < kUpHalfRounds; i++) {
            const int r = r0 + i, tt = r >> 3, k = r & 7;
            hv[i] = *reinterpret_cast<const uint4*>(hw + (8 * k + lrow) * kUpHP + tt * 128 + lcol);
        }
        uint32_t cab = 0;                               // lane counts: tile ta in bits 0-15, ta + 1 above
#pragma unroll
        for (int i = 0; i < kUpHalfRounds; i++) {
            const uint32_t m = mask_bf16x8_pk(hv[i]) & (0u - (uint32_t)(i < nr));
            mk[i >> 2] |= m << (8 * (i & 3));
            cab += (uint32_t)__popc(m) << (i < bnd ? 0 : 16);
        }
#pragma unroll
        for (int i = 0; i < kUpHalfRounds; i++) {
            if (i < nr) {
                const int r = r0 + i, tt = r >> 3, k = r & 7;
                a.bitmask[(size_t)(t0 + tt) * kTileBytes + 64 * k + lane] = (uint8_t)(mk[i >> 2] >> (8 * (i & 3)));
            }
        }
        const uint32_t tot = wave_total(cab);           // a tile's count is at most 4096
        if (lane < kUpTiles)
            cnt_s[(ui * 2 + half) * 4 + lane] = lane == ta ? (tot & 0xffffu) : lane == ta + 1 ? (tot >> 16) : 0u;
    }
    __syncthreads();                                    // both halves' counts

    uint32_t toff[kUpTiles + 1], seg0 = 0;             // tile offsets in the unit's run; half 0's length
    toff[0] = 0;
#pragma unroll
    for (int tt = 0; tt < kUpTiles; tt++) {
        const uint32_t c0 = cnt_s[(ui * 2) * 4 + tt], c1 = cnt_s[(ui * 2 + 1) * 4 + tt];
        toff[tt + 1] = toff[tt] + c0 + c1;
        seg0 += c0;
    }
    const uint32_t unit_total = toff[kUpTiles];
    const uint32_t u = tm * a.nb + cb;
    if (active && half == 0 && lane == 0)
        st_relaxed(&a.status[u], pack_status(a.epoch, u == 0 ? kFlagInc : kFlagAgg, unit_total));

    // the dense h stores go out while the preceding units publish: half h
    // stores rows 32 h .. +31 of the unit, 24 chunks each, 16-byte stores
    // (N % 8 == 0, ldh % 8 == 0)
    if (active && a.h != nullptr) {
#pragma unroll 4
        for (int q = lane; q < 32 * (kUpBN / 8); q += 64) {
            const int row = 32 * half + q / (kUpBN / 8), cc = q % (kUpBN / 8);
            const int64_t grow = grow0 + row, gcol = n0 + cc * 8;
            if (grow < a.M && gcol < a.N)
                *reinterpret_cast<uint4*>(a.h + grow * a.ldh + gcol) =
                    *reinterpret_cast<const uint4*>(hw + row * kUpHP + cc * 16);
        }
    }
    __syncthreads();                                    // the unit's staged rows are read: the run replaces them

    // ---- values, first into LDS: the unit's runs are consecutive in vals,
    // so its two halves compact all of them into one run at phase 0 -- in the
    // unit's 64 staged rows, whose values they hold in registers.  This needs
    // no offset, so the preceding units have this long to publish before the
    // look-back below.  A compacted chunk's 8 elements are written in
    // descending order, its elements past the count landing on the following
    // chunks' positions, which later writes replace; half 0 writes nothing
    // past its own run, whose following positions are half 1's (its chunks
    // near that end store their elements one by one, clipped there).
    uint16_t* run = reinterpret_cast<uint16_t*>(hs + ui * 64 * kUpHP);
    if (active) {
        // every round's selector rows first; rounds past nr have empty masks
        uint4 s0[kUpHalfRounds], s1[kUpHalfRounds];
#pragma unroll
        for (int i = 0; i < kUpHalfRounds; i++) {
            const uint32_t m = (mk[i >> 2] >> (8 * (i & 3))) & 0xffu;
            s0[i] = *reinterpret_cast<const uint4*>(&sel_s[m * 8]);
            s1[i] = *reinterpret_cast<const uint4*>(&sel_s[m * 8 + 4]);
        }
        // each round's lane offsets and total: three rounds per wave scan, in
        // 10-bit fields (a round's total is at most 512)
        uint32_t ex[kUpHalfRounds], rt[kUpHalfRounds];
#pragma unroll
        for (int g = 0; g < kUpHalfRounds / 3; g++) {
            uint32_t cp = 0;
#pragma unroll
            for (int j = 0; j < 3; j++) cp |= (uint32_t)__popc((mk[(3 * g + j) >> 2] >> (8 * ((3 * g + j) & 3))) & 0xffu) << (10 * j);
            const uint32_t incl = wave_incl_scan(cp);
            const uint32_t last = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
#pragma unroll
            for (int j = 0; j < 3; j++) {
                ex[3 * g + j] = ((incl - cp) >> (10 * j)) & 1023u;
                rt[3 * g + j] = (last >> (10 * j)) & 1023u;
            }
        }
        uint32_t P = half == 0 ? 0u : seg0;            // run offset of the round
#pragma unroll
        for (int i = 0; i < kUpHalfRounds; i++) {
            const uint32_t m = (mk[i >> 2] >> (8 * (i & 3))) & 0xffu;
            const uint32_t base = P;
            P += rt[i];
            if (m != 0u) {
                const uint4 w = hv[i];
                uint4 o;
                o.x = __builtin_amdgcn_perm(w.y, w.x, s0[i].x) | __builtin_amdgcn_perm(w.w, w.z, s1[i].x);
                o.y = __builtin_amdgcn_perm(w.y, w.x, s0[i].y) | __builtin_amdgcn_perm(w.w, w.z, s1[i].y);
                o.z = __builtin_amdgcn_perm(w.y, w.x, s0[i].z) | __builtin_amdgcn_perm(w.w, w.z, s1[i].z);
                o.w = __builtin_amdgcn_perm(w.y, w.x, s0[i].w) | __builtin_amdgcn_perm(w.w, w.z, s1[i].w);
                uint8_t* dst = reinterpret_cast<uint8_t*>(run + (int)base + (int)ex[i]);
                // half 0: elements before half 1's run (at least the chunk's count)
                const uint32_t lim = half == 0 ? seg0 - (base + ex[i]) : 8u;
                if (__ballot(lim < 8u) == 0ull) {
                    write_compacted<2>(dst, o);
                } else {                                // the whole wave: same descending order
                    const uint32_t ow[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                    for (int e = 7; e >= 0; e--) {
                        if ((uint32_t)e < lim)
                            *reinterpret_cast<uint16_t*>(dst + 2 * e) = (uint16_t)(ow[e >> 1] >> (16 * (e & 1)));
                        asm volatile("" ::: "memory");
                    }
                }
            }
        }
    }
    __syncthreads();                                    // the unit's run is complete

    // ---- offset: look-back (both halves, read-only but for half 0's
    // inclusive status), prefix entries, cursor and flags
    if (!active) return;
    uint32_t excl = 0;
    if (u != 0) {
        excl = up_lookback(a, u, lane);
        if (half == 0 && lane == 0) st_relaxed(&a.status[u], pack_status(a.epoch, kFlagInc, excl + unit_total));
    }
    const uint32_t nunits = a.grid_m * a.nb;
    if (half == 0) {
#pragma unroll
        for (int tt = 0; tt < kUpTiles; tt++)
            if (lane == tt && tt < ntiles) a.prefix[t0 + tt] = excl + toff[tt];
        if (lane == 0 && u == nunits - 1) {
            a.prefix[a.T] = excl + unit_total;
            const int64_t end = start + (int64_t)(excl + unit_total);
            if (a.offset_out) *a.offset_out = end;
            if (a.start_out) *a.start_out = start;
            if (a.err && end > a.vals_capacity) atomicOr(a.err, 1);
            if (a.err && start < 0) atomicOr(a.err, 2);
        }
    }
    if (start < 0) return;

    // ---- values out: run element p is vals element g + p.  16-byte vals
    // slot j holds elements g - a0 + 8 j .. +7 (a0 = g mod 8), run elements
    // 8 j - a0 .. +7: its 16 bytes start at run byte 16 j - 2 a0, inside the
    // 8-byte-aligned 24 bytes from (16 j - 2 a0) & ~7, at byte offset
    // (-2 a0) mod 8 (the same for every slot).  Partial slots at the two ends
    // take element stores; elements past the capacity are not written.  The
    // two halves take alternate 64-slot groups.
    const int64_t g = start + (int64_t)excl;
    const int a0 = (int)(g & 7);
    const int64_t room = a.vals_capacity - g;
    const int endr = (int)std::max<int64_t>(0, std::min<int64_t>((int64_t)unit_total, room));
    const int nslots = (a0 + endr + 7) >> 3;
    uint16_t* const vbase = a.vals + (g - a0);             // 16-byte aligned
    const uint32_t off = (uint32_t)((8 - 2 * a0) & 7);     // byte offset in the window
    const uint8_t* runb = reinterpret_cast<const uint8_t*>(run);
    // three slots per pass, all their windows read before any is stored;
    // windows of partial slots and of slots past the end read clamped
    // addresses inside the workgroup's LDS and go unused
    auto store_slots = [&](auto SHIFT) __attribute__((always_inline)) {
        constexpr int S = decltype(SHIFT)::value;           // off >= 4: the window's first dword is skipped
        const uint32_t ob = off & 3u;
        for (int j = lane + 64 * half; j < nslots; j += 3 * 128) {
            uint32_t d[3][6];
#pragma unroll
            for (int v = 0; v < 3; v++) {
                const uint8_t* wp = runb + std::max(0, (16 * (j + 128 * v) - 2 * a0) & ~7);
                const uint2 q0 = *reinterpret_cast<const uint2*>(wp);
                const uint2 q1 = *reinterpret_cast<const uint2*>(wp + 8);
                const uint2 q2 = *reinterpret_cast<const uint2*>(wp + 16);
                d[v][0] = q0.x; d[v][1] = q0.y; d[v][2] = q1.x; d[v][3] = q1.y; d[v][4] = q2.x; d[v][5] = q2.y;
            }
#pragma unroll
            for (int v = 0; v < 3; v++) {
                const int jj = j + 128 * v;
                if (jj >= nslots) break;
                const int lo = std::max(8 * jj, a0), hi = std::min(8 * jj + 8, a0 + endr);
                if (lo == 8 * jj && hi == 8 * jj + 8) {
                    uint32_t o[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) o[i] = __builtin_amdgcn_alignbyte(d[v][i + 1 + S], d[v][i + S], ob);
                    *reinterpret_cast<uint4*>(vbase + 8 * jj) = uint4{o[0], o[1], o[2], o[3]};
                } else {
                    for (int e = lo; e < hi; e++) vbase[e] = run[e - a0];
                }
            }
        }
    };
    if (off >= 4) store_slots(IC<1>{});
    else store_slots(IC<0>{});
}

// Workgroups per tile row the launch accepts on device `dev`: half of what
// the device holds at once (the occupancy API's count per CU times its CUs),
// so that a strip's workgroups are co-resident with room to spare; 0 if the
// queries fail.
static int64_t up_max_nb(int dev)
{
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, up_relu_compress_kernel, 256, 0) != hipSuccess ||
        per_cu <= 0)
        return 0;
    return (int64_t)cus * per_cu / 2;
}

// up_max_nb per device, queried once (the occupancy query costs host time
// on every launch otherwise); 0 until known
static int64_t up_max_nb_cached(int dev)
{
    static std::atomic<int64_t> known[64];
    if (dev < 0 || dev >= 64) return up_max_nb(dev);
    int64_t v = known[dev].load(std::memory_order_relaxed);
    if (v <= 0) {
        v = up_max_nb(dev);
        if (v > 0) known[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

}  // namespace bs

using namespace bs;

extern "C" int64_t bs_linear_relu_compress_max_n(int device)
{
    clear_error();
    const int64_t nb = up_max_nb_cached(device);
    if (nb <= 0) {
        set_error(BS_ERR_HIP, "bs_linear_relu_compress_max_n: occupancy query failed");
        return -1;
    }
    return nb * kUpBN;
}

extern "C" int bs_linear_relu_compress(const void* x, int64_t M, int64_t K, int64_t ldx, const void* w, int64_t N,
                                       int64_t ldw, const void* bias, void* h_out, int64_t ldh, uint8_t* bitmask,
                                       uint32_t* prefix, void* vals, int64_t vals_capacity,
                                       const int64_t* vals_offset_in, int align8, int64_t* vals_offset_out,
                                       int64_t* vals_start_out, int32_t* err_flags, int32_t* timeout_flag,
                                       int64_t patience_ticks, void* workspace, int64_t workspace_bytes,
                                       uint32_t epoch, void* stream)
{
    clear_error();
    const char* fn = "bs_linear_relu_compress";
    if (M <= 0 || N <= 0 || K < 0) return set_error(BS_ERR_INVALID, "%s: needs M, N > 0 and K >= 0", fn);
    if (K % 8 || N % 8) return set_error(BS_ERR_INVALID, "%s: K and N must be multiples of 8", fn);
    if ((uint64_t)M * (uint64_t)N >= kMaxElemsUntested) return set_error(BS_ERR_INVALID, "%s: M*N must be < 2^31", fn);
    if (x == nullptr || w == nullptr || bitmask == nullptr || prefix == nullptr)
        return set_error(BS_ERR_INVALID, "%s: null pointer", fn);
    if (ldx < K || ldw < K || ldx % 8 || ldw % 8)
        return set_error(BS_ERR_INVALID, "%s: row strides must be >= K and multiples of 8", fn);
    // 32-bit buffer offsets: the rows of an x slab (128) and of a W slab
    // (192) stay below 2^31 bytes from their base
    if ((int64_t)std::max(kUpBM, kUpBN) * std::max(ldx, ldw) * 2 >= (1ll << 31))
        return set_error(BS_ERR_INVALID, "%s: row stride too large", fn);
    if ((((uintptr_t)x) & 15) || (((uintptr_t)w) & 15))
        return set_error(BS_ERR_INVALID, "%s: x and W must be 16-byte aligned", fn);
    if (bias != nullptr && (((uintptr_t)bias) & 1)) return set_error(BS_ERR_INVALID, "%s: bias misaligned", fn);
    if (h_out != nullptr && ((((uintptr_t)h_out) & 15) || ldh < N || ldh % 8))
        return set_error(BS_ERR_INVALID, "%s: h must be 16-byte aligned with a row stride >= N, a multiple of 8",
                         fn);
    if (vals_capacity < 0) return set_error(BS_ERR_INVALID, "%s: negative capacity", fn);
    if (vals_capacity > 0 && vals == nullptr) return set_error(BS_ERR_INVALID, "%s: null vals", fn);
    if (((uintptr_t)vals) & 15) return set_error(BS_ERR_INVALID, "%s: vals must be 16-byte aligned", fn);
    if (vals_offset_out != nullptr && vals_offset_out == vals_offset_in)
        return set_error(BS_ERR_INVALID, "%s: vals_offset_out aliases vals_offset_in", fn);
    if (epoch == 0 || epoch >= (1u << 30)) return set_error(BS_ERR_INVALID, "%s: epoch must be in [1, 2^30)", fn);
    const int64_t nb = (N + kUpBN - 1) / kUpBN;
    int dev = 0;
    if (stream_device((hipStream_t)stream, &dev) != hipSuccess)
        return set_error(BS_ERR_HIP, "%s: cannot resolve the stream's device", fn);
    const int64_t max_nb = up_max_nb_cached(dev);
    if (max_nb <= 0) return set_error(BS_ERR_HIP, "%s: occupancy query failed", fn);
    if (nb > max_nb)
        return set_error(BS_ERR_INVALID, "%s: N must be at most %lld on this device", fn,
                         (long long)(max_nb * kUpBN));
    if (int rc = refuse_capture((hipStream_t)stream, fn)) return rc;
    if (workspace == nullptr || workspace_bytes < bs_compress_workspace_bytes(M, N))
        return set_error(BS_ERR_INVALID, "%s: workspace too small (%lld < %lld bytes)", fn, (long long)workspace_bytes,
                         (long long)bs_compress_workspace_bytes(M, N));
    UpArgs a{};
    a.x = (const uint16_t*)x;
    a.w = (const uint16_t*)w;
    a.bias = (const uint16_t*)bias;
    a.h = (uint16_t*)h_out;
    a.ldx = ldx;
    a.ldw = ldw;
    a.ldh = ldh;
    a.M = M;
    a.N = N;
    a.K = K;
    a.grid_n = (uint32_t)((N + kTile - 1) / kTile);
    a.grid_m = (uint32_t)((M + kTile - 1) / kTile);
    a.nb = (uint32_t)nb;
    a.T = a.grid_m * a.grid_n;
    a.bitmask = bitmask;
    a.prefix = prefix;
    a.vals = (uint16_t*)vals;
    a.vals_capacity = vals_capacity;
    a.offset_in = vals_offset_in;
    a.align8 = align8 ? 1 : 0;
    a.offset_out = vals_offset_out;
    a.start_out = vals_start_out;
    a.err = err_flags;
    a.timeout = timeout_flag;
    a.status = reinterpret_cast<uint64_t*>((uint8_t*)workspace + kWsHeaderBytes);
    a.epoch = epoch;
    a.patience = patience_ticks < 0 ? kUpLookbackGiveUpTicks : (uint64_t)patience_ticks;
    const int64_t strips = (M + kUpBM - 1) / kUpBM;
    const int64_t blocks = strips * nb;
    if (blocks >= (1ll << 31)) return set_error(BS_ERR_INVALID, "%s: grid too large", fn);
    hipLaunchKernelGGL(up_relu_compress_kernel, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "%s launch: %s", fn, hipGetErrorString(e));
    return BS_OK;
}
