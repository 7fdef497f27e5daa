// BitSparse codec kernels for gfx950: single-pass compress (and the count /
// values passes of the standalone path), decompress, and the two gradient
// kernels.
//
// Compress runs one wave per tile (lane l owns chunks 64k + l, k < 8) and a
// look-back unit of 8 tiles per workgroup.  The gather kernels (decompress,
// gradients) use a workgroup of 256 threads (4 wave64) per "unit" of U
// consecutive tiles: for each tile, thread i handles chunks i and i+256 (rows
// i/8 and 32+i/8), so one wave instruction covers 8 full tile rows = 8 x 128
// contiguous bytes of bf16.
#include "bs_device.h"
#include "bs_host.h"
#include "compact.h"

#include <algorithm>
#include <cstdlib>
#include <cmath>
#include <functional>
#include <mutex>


namespace bs {

constexpr int kThreads = 256;




// Elements of one chunk as raw bits.
template <int B>
__device__ __forceinline__ uint32_t elem(const typename Raw<B>::T& v, int e)
{
    if constexpr (B == 2) return get16(v, e);
    else return get8(v, e);
}

template <int B>
__device__ __forceinline__ void set_elem(typename Raw<B>::T& v, int e, uint32_t x)
{
    if constexpr (B == 2) {
        uint32_t* w = e < 2 ? &v.x : e < 4 ? &v.y : e < 6 ? &v.z : &v.w;
        int sh = (e & 1) * 16;
        *w = (*w & ~(0xffffu << sh)) | ((x & 0xffffu) << sh);
    } else {
        uint32_t* w = e < 4 ? &v.x : &v.y;
        int sh = (e & 3) * 8;
        *w = (*w & ~(0xffu << sh)) | ((x & 0xffu) << sh);
    }
}

// Load chunk (row, col0..col0+7) of a row-major matrix, zeros outside [M, N].
// VEC: N % 8 == 0 and 8-element alignment, so a chunk is all in or all out.
template <int B, bool VEC, bool NT = false>
__device__ __forceinline__ typename Raw<B>::T load_chunk(const uint8_t* base, int64_t M, int64_t N,
                                                         int64_t row, int64_t col0)
{
    using T = typename Raw<B>::T;
    T v = {};
    if (row >= M || col0 >= N) return v;
    const uint8_t* p = base + (row * N + col0) * B;
    if constexpr (VEC) {
        v = ld_chunk<NT, T>(p);
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            if (col0 + e < N) {
                uint32_t x = (B == 2) ? (uint32_t)reinterpret_cast<const uint16_t*>(p)[e]
                                      : (uint32_t)p[e];
                set_elem<B>(v, e, x);
            }
        }
    }
    return v;
}

template <int B, bool VEC, bool NT = false>
__device__ __forceinline__ void store_chunk(uint8_t* base, int64_t M, int64_t N, int64_t row,
                                            int64_t col0, const typename Raw<B>::T& v)
{
    using T = typename Raw<B>::T;
    if (row >= M || col0 >= N) return;
    uint8_t* p = base + (row * N + col0) * B;
    if constexpr (VEC) {
        st_chunk<NT, T>(p, v);
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            if (col0 + e < N) {
                if (B == 2) reinterpret_cast<uint16_t*>(p)[e] = (uint16_t)elem<B>(v, e);
                else p[e] = (uint8_t)elem<B>(v, e);
            }
        }
    }
}

// fp32 scale of the e4m3fn quantizer from the amax slot: max(amax/448, 1e-9);
// a NaN amax gives a NaN scale (torch's clamp keeps NaN).
__device__ __forceinline__ float scale_from_slot(const uint64_t* slot, uint32_t epoch)
{
    uint64_t s = *slot;
    float amax = ((uint32_t)(s >> 32) == epoch) ? bf16_to_f32((uint32_t)s & 0xffffu) : 0.0f;
    float sc = amax / 448.0f;
    return (sc < 1e-9f) ? 1e-9f : sc;
}

__device__ __forceinline__ uint2 quant_chunk(const uint4 v, float scale, float rcp)
{
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t p[4];
#pragma unroll
    for (int k = 0; k < 4; k++) p[k] = div2_to_e4m3(bf16_to_f32(w[k] & 0xffffu), bf16_to_f32(w[k] >> 16), scale, rcp);
    return uint2{p[0] | (p[1] << 16), p[2] | (p[3] << 16)};
}

// entry i of each half stands for magnitude base + i - 1 (the end entries
// for every magnitude past them); scale from the amax slot
__global__ __launch_bounds__(256) void qtab_build_kernel(const uint64_t* slot, uint32_t epoch, uint8_t* qtab)
{
    const int i = (int)(blockIdx.x * 256 + threadIdx.x);
    if (i >= kQtabEntries) return;
    const float scale = scale_from_slot(slot, epoch);
    const int m = min(max(qtab_offset(scale) + i, 0), 0x7fff);
    const uint32_t c = f32_to_e4m3(bf16_to_f32((uint32_t)m) / scale);
    if (scale != scale) {
        qtab[i] = 0x7fu;
        qtab[kQtabEntries + i] = m > 0x7f80 ? 0xffu : 0x7fu;
    } else {
        qtab[i] = (uint8_t)c;
        qtab[kQtabEntries + i] = (uint8_t)(c | 0x80u);
    }
}

// Chunk geometry inside tile t of a [*, N] matrix.
__device__ __forceinline__ void chunk_pos(uint32_t t, uint32_t grid_n, int b, int64_t& row,
                                          int64_t& col0)
{
    uint32_t tm = t / grid_n, tn = t - tm * grid_n;
    row = (int64_t)tm * 64 + (b >> 3);
    col0 = (int64_t)tn * 64 + (b & 7) * 8;
}

// ===========================================================================
// compress
// ===========================================================================
enum { MODE_FUSED = 0, MODE_COUNT = 1, MODE_VALS = 2 };

struct CompressArgs {
    const uint8_t* dense;
    int64_t M, N;
    uint32_t grid_n;
    uint32_t T;
    const uint64_t* amax_slot;
    uint32_t amax_epoch;
    float* scale_out;
    uint8_t* dense_q_out;
    uint8_t* bitmask;           // written (FUSED/COUNT) or read (VALS)
    uint32_t* prefix;           // written (FUSED/COUNT) or read (VALS)
    uint8_t* vals;
    int64_t vals_capacity;
    const int64_t* offset_in;
    int32_t align8;
    int64_t* offset_out;
    int64_t* start_out;
    uint32_t tile0;             // first tile of unit 0 (VALS: also the prefix base)
    uint32_t tend;              // one past the last tile of this launch
    int32_t relu;               // 1: `dense` is a pre-activation, compress relu(dense)
    uint8_t* relu_out;          // nullable (may alias dense): receives relu(dense)
    uint64_t* status;
    uint64_t* gstat;            // one status word per group of kGroupUnits units
    uint32_t epoch;
    int32_t* err;
    uint32_t* fallbacks;
    uint64_t patience;          // look-back wait (s_memrealtime ticks) before counting a unit itself
    const uint8_t* qtab;        // quantize: the code table (kQtabBytes), copied into LDS
    float relu_k;               // RSQ: relu_out receives bf16(bf16(r * r) * relu_k), r = relu(dense)
};

// 200 us at the 100 MHz s_memrealtime clock: waiting longer than this for a
// predecessor makes the waiter count that predecessor's tiles itself (a
// safety net: in-order workgroup dispatch never needs it, and normal waits
// behind slow predecessors stay well below it).  The environment variable
// BITSPARSE_LOOKBACK_PATIENCE (ticks) overrides it; 0 makes every wait take
// the fallback, which is how the tests exercise that path.
constexpr uint64_t kLookbackPatienceTicks = 20000;

template <int IN_T, bool QUANT>
struct CompressTraits {
    static constexpr int INB = IN_T == DT_BF16 ? 2 : 1;
    static constexpr int OUTB = (IN_T == DT_BF16 && !QUANT) ? 2 : 1;
    static constexpr int MASK_T = QUANT ? DT_E4M3FN : IN_T;
    static constexpr int PB = OUTB == 2 ? 15 : 7;       // packed stream bits per value
};

// Positive-bit byte of a loaded chunk (after quantisation when QUANT).
// TAB: quantize through the code table `qtab` (LDS) instead of dividing.
template <int IN_T, bool QUANT, bool TAB = false>
__device__ __forceinline__ uint32_t chunk_mask(const typename Raw<CompressTraits<IN_T, QUANT>::INB>::T& d,
                                               typename Raw<CompressTraits<IN_T, QUANT>::OUTB>::T& o,
                                               float scale, float rcp, const uint8_t* qtab = nullptr,
                                               int qoff = 0)
{
    if constexpr (QUANT) {
        if constexpr (TAB) o = quant_chunk_tab(d, qtab, qoff);
        else o = quant_chunk(d, scale, rcp);
        return mask_fp8x8<DT_E4M3FN>(o);
    } else if constexpr (IN_T == DT_BF16) {
        o = d;
        return mask_bf16x8(d);
    } else {
        o = d;
        return mask_fp8x8<IN_T>(d);
    }
}

template <int IN_T, bool QUANT, bool TAB = false>
__device__ __forceinline__ uint32_t stream_chunk_mask(const typename Raw<CompressTraits<IN_T, QUANT>::INB>::T& d,
                                                      typename Raw<CompressTraits<IN_T, QUANT>::OUTB>::T& o,
                                                      float scale, float rcp, const uint8_t* qtab = nullptr,
                                                      int qoff = 0)
{
    if constexpr (IN_T == DT_BF16 && !QUANT) {
        o = d;
        return mask_bf16x8_pk(d);
    } else {
        return chunk_mask<IN_T, QUANT, TAB>(d, o, scale, rcp, qtab, qoff);
    }
}

// relu(x) of a loaded chunk with the semantics of torch's GPU relu: x <= 0
// becomes +0 (so -0 does too), NaN and positives keep their bits (bit
// patterns: bf16 [0x8000, 0xff80], e4m3fn [0x80, 0xfe], e5m2 [0x80, 0xfc] are
// the non-positive non-NaN values besides +0).
template <int DT>
__device__ __forceinline__ typename Raw<DT == DT_BF16 ? 2 : 1>::T relu_chunk(typename Raw<DT == DT_BF16 ? 2 : 1>::T v)
{
    if constexpr (DT == DT_BF16) {
        uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lo = w[i] & 0xffffu, hi = w[i] >> 16;
            w[i] = ((lo - 0x8000u) < 0x7f81u ? 0u : lo) | (((hi - 0x8000u) < 0x7f81u ? 0u : hi) << 16);
        }
        return uint4{w[0], w[1], w[2], w[3]};
    } else {
        constexpr uint32_t span = DT == DT_E4M3FN ? 0x7fu : 0x7du;   // zeroed: [0x80, 0x80 + span)
        uint32_t w[2] = {v.x, v.y};
#pragma unroll
        for (int i = 0; i < 2; i++) {
            uint32_t r = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const uint32_t x = (w[i] >> (8 * b)) & 0xffu;
                r |= ((x - 0x80u) < span ? 0u : x) << (8 * b);
            }
            w[i] = r;
        }
        return uint2{w[0], w[1]};
    }
}

// Nonzero count of compress unit q computed straight from the dense input by
// one wave (look-back fallback).
template <int IN_T, bool QUANT, bool VEC, int U>
__device__ uint32_t unit_count_wave(const CompressArgs& a, uint32_t q, float scale, int lane)
{
    using TR = CompressTraits<IN_T, QUANT>;
    uint32_t t0 = a.tile0 + q * U;
    uint32_t nt = min((uint32_t)U, a.tend - t0);
    uint32_t c = 0;
    for (uint32_t k = lane; k < nt * kChunksPerTile; k += kWave) {
        int64_t row, col0;
        chunk_pos(t0 + (k >> 9), a.grid_n, (int)(k & 511), row, col0);
        auto d = load_chunk<TR::INB, VEC>(a.dense, a.M, a.N, row, col0);
        if constexpr (IN_T == DT_BF16 && !QUANT) {
            // count only (no mask byte): few live registers on this rare path
            const uint32_t w[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
            for (int i = 0; i < 4; i++)
                c += pos_bf16(w[i] & 0xffffu) + pos_bf16(w[i] >> 16);
        } else {
            typename Raw<TR::OUTB>::T o;
            c += __popc(stream_chunk_mask<IN_T, QUANT>(d, o, scale, 1.0f / scale));
        }
    }
    return (uint32_t)__builtin_amdgcn_readlane((int)wave_incl_scan(c), 63);
}

__device__ __forceinline__ uint64_t bcast_lane0(uint64_t v)
{
    const uint32_t lo = uniform_u32((uint32_t)v);
    const uint32_t hi = uniform_u32((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// Two-level decoupled look-back of the streaming kernel, run by one wave.
// Units form groups of kGroupUnits; besides its unit status word, the last
// unit of a group publishes a group status word: the group aggregate when its
// own walk passes the group start seeing aggregates only, then the group's
// inclusive prefix once it has resolved.  A walk adds whole groups (64 group
// words per read) wherever a group word is out and falls back to that
// group's unit words otherwise, so a unit resolves in a few reads however far
// the nearest inclusive prefix is.  Only unit words are ever waited for; a
// unit that stays unpublished for kLookbackPatienceTicks is counted from the
// dense input instead.  Returns the exclusive prefix of unit u in every lane.
constexpr int kGroupUnits = 64;

template <int IN_T, bool QUANT, bool VEC, int U>
__device__ uint32_t wave_lookback_grouped(const CompressArgs& a, uint32_t u, uint32_t unit_total,
                                          float scale, int lane)
{
    uint32_t excl = 0;
    int64_t pos = (int64_t)u - 1;           // next unit still to be added
    const int64_t my_lo = (int64_t)u & ~(int64_t)(kGroupUnits - 1);
    const bool group_last = ((u + 1) & (kGroupUnits - 1)) == 0;
    bool units_only = false;                // the group word at pos was not out
    uint64_t since = wall_clock64();
    while (pos >= 0) {
        const int64_t lo = pos & ~(int64_t)(kGroupUnits - 1);
        if (!units_only && pos == lo + kGroupUnits - 1) {
            const int64_t gq = (pos / kGroupUnits) - lane;
            const uint64_t s = gq >= 0 ? ld_relaxed(&a.gstat[gq]) : pack_status(a.epoch, kFlagInc, 0);
            const uint32_t val = (uint32_t)s, flag = (uint32_t)(s >> 32) & 3u;
            const bool valid = (uint32_t)(s >> 34) == a.epoch && flag != 0u;
            const uint64_t notv = ~__ballot(valid);
            const uint64_t incm = __ballot(valid && flag == (uint32_t)kFlagInc);
            const int fi = notv ? __ffsll((unsigned long long)notv) - 1 : 64;
            const int fc = incm ? __ffsll((unsigned long long)incm) - 1 : 64;
            if (fc < fi) return excl + wave_total(lane <= fc ? val : 0u);
            excl += wave_total(lane < fi ? val : 0u);
            pos -= (int64_t)fi * kGroupUnits;
            units_only = fi < 64;
            if (fi > 0) since = wall_clock64();
            continue;
        }
        units_only = false;
        const int n = (int)(pos - lo) + 1;  // units pos, pos-1, ..., lo
        const uint64_t s = lane < n ? ld_relaxed(&a.status[pos - lane]) : 0ull;
        const uint32_t val = (uint32_t)s, flag = (uint32_t)(s >> 32) & 3u;
        const bool valid = lane < n && (uint32_t)(s >> 34) == a.epoch && flag != 0u;
        const uint64_t inwin = n == 64 ? ~0ull : ((1ull << n) - 1ull);
        const uint64_t notv = ~__ballot(valid) & inwin;
        const uint64_t incm = __ballot(valid && flag == (uint32_t)kFlagInc);
        const int fi = notv ? __ffsll((unsigned long long)notv) - 1 : n;
        const int fc = incm ? __ffsll((unsigned long long)incm) - 1 : 64;
        if (fc < fi) return excl + wave_total(lane <= fc ? val : 0u);
        excl += wave_total(lane < fi ? val : 0u);
        pos -= fi;
        if (fi > 0) since = wall_clock64();
        if (fi == n) {
            // the group start passed with aggregates only: publish the group's
            // aggregate if this unit closes it
            if (group_last && lo == my_lo && lane == 0)
                st_relaxed(&a.gstat[u / kGroupUnits], pack_status(a.epoch, kFlagAgg, excl + unit_total));
            continue;
        }
        // unit pos is not out yet: poll it alone (patience counts from here)
        since = wall_clock64();
        while (true) {
            uint64_t s0 = 0;
            if (lane == 0) s0 = ld_relaxed(&a.status[pos]);
            s0 = bcast_lane0(s0);
            const uint32_t f0 = (uint32_t)(s0 >> 32) & 3u;
            if ((uint32_t)(s0 >> 34) == a.epoch && f0 != 0u) {
                if (f0 == (uint32_t)kFlagInc) return excl + (uint32_t)s0;
                excl += (uint32_t)s0;
                break;
            }
            if (wall_clock64() - since > a.patience) {
                excl += unit_count_wave<IN_T, QUANT, VEC, U>(a, (uint32_t)pos, scale, lane);
                if (lane == 0 && a.fallbacks) atomicAdd(a.fallbacks, 1u);
                break;
            }
            __builtin_amdgcn_s_sleep(4);
        }
        pos -= 1;
        since = wall_clock64();
        if (pos == lo - 1 && group_last && lo == my_lo && lane == 0)
            st_relaxed(&a.gstat[u / kGroupUnits], pack_status(a.epoch, kFlagAgg, excl + unit_total));
    }
    return excl;
}

// ===========================================================================
// streaming compress (bs_compress FUSED / COUNT)
//
// One wave per tile, U tiles (one look-back unit) per workgroup; unit u is
// workgroup u (workgroups are dispatched in id order, so every unit's
// predecessors are already resident or done when it starts).  Lane l owns chunks
// 64k + l (k < 8) of its tile: rows 8k + l/8, columns 8(l%8)..+7, so every
// load instruction covers 8 whole tile rows and the tile's value run is
// produced in eight in-order rounds of 64 chunks.  The loaded chunks stay in
// registers while wave 0 runs the look-back, and are compacted there in the
// meantime (v_perm with selectors from a 256-entry table indexed by the mask
// byte: the set elements move to the front; this needs no prefix).  After
// the look-back each wave streams its run through a private LDS ring:
//   * a compacted chunk's 8 elements are written
//     at the chunk's run position in descending element order: the elements
//     past the chunk's count land on the positions of the following chunks,
//     which later (lower-index) writes of those chunks overwrite, so no
//     element needs an address or a predicate of its own;
//   * ring slot 0 always holds the output's pending 16-byte slot (the one the
//     next element falls in); every slot a round completes is stored with one
//     16-byte write, then the new pending slot is copied back to ring slot 0;
//   * the partial slots at the two ends of the run, shared with the
//     neighbouring runs, get element stores.
// ===========================================================================
#ifndef BS_STREAM_ROUNDS
#define BS_STREAM_ROUNDS 2
#endif
constexpr int kRoundsPerPass = BS_STREAM_ROUNDS;   // rounds written before each store pass
// >= 15 (pending) + 512 per round + 8 (overrun), a multiple of 16
constexpr int kRingElems = 512 * kRoundsPerPass + 32;

#ifndef BS_STREAM_WAVES_PER_EU
#define BS_STREAM_WAVES_PER_EU 8
#endif

__device__ __forceinline__ void opaque(uint4& v)
{
    asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
}
__device__ __forceinline__ void opaque(uint2& v) { asm volatile("" : "+v"(v.x), "+v"(v.y)); }

// PACKED (MODE_FUSED only): the values go to a 15/7-bit stream (pack_sbit
// storage) instead of raw elements: a.vals is the stream (4-byte aligned) and
// a.vals_capacity its size in dwords.  Each wave still compacts its run into
// the ring; every pass then builds the stream dwords its values complete (one
// dword per lane from the <= 4 / <= 6 values overlapping it; the dwords at the
// two ends of the run, shared with the neighbouring runs, are merged with
// disjoint-bit atomics) and carries the values the next dword still needs to
// the front of the ring.
__device__ __forceinline__ void wave_sync_lds()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Merge `word` into out[D] keeping the bits outside `mask` (disjoint-bit
// atomics commute with any other writer of other bits of the dword).
__device__ __forceinline__ void merge_word(uint32_t* out, int64_t D, uint32_t word, uint32_t mask)
{
    if (mask == 0xffffffffu) {
        out[D] = word;
    } else if (mask != 0u) {
        atomicAnd(&out[D], ~mask);
        atomicOr(&out[D], word & mask);
    }
}

// Bits [lb, hb) of a dword as a mask, 0 <= lb <= hb <= 32.
__device__ __forceinline__ uint32_t bit_range_mask(uint32_t lb, uint32_t hb)
{
    const uint32_t hi = hb >= 32u ? 0xffffffffu : ((1u << hb) - 1u);
    const uint32_t lo = lb >= 32u ? 0xffffffffu : ((1u << lb) - 1u);
    return hi & ~lo;
}

// Packed stream phase of one wave's run: values [0, cnt) of the tile's run
// (compacted chunks o[k] of round k at run position P[k] + in-round rank) go
// to stream bits [g*PB, (g+cnt)*PB) of a.vals (a.vals_capacity dwords).
// ring[i] holds run value base + i.
// The run's partial dwords (shared with the neighbouring runs) are OR-ed into
// s_edge[b], b the first unit boundary (0..U) whose dword they are; the unit
// writes those dwords afterwards (packed_unit_edges).  s_toff[b] is the run
// offset of boundary b inside the unit, whose run starts at value gu.
template <int OUTB, int PB, int U>
__device__ __forceinline__ void stream_packed(const CompressArgs& a, int64_t g, int cnt, const uint32_t* P,
                                              const uint32_t* mp, const typename Raw<OUTB>::T* o,
                                              uint8_t* ring, int lane, int64_t gu, const uint32_t* s_toff,
                                              uint32_t* s_edge)
{
    constexpr int MAXV = PB == 15 ? 4 : 6;      // values overlapping one stream dword
    constexpr uint32_t VMASK = (1u << PB) - 1u;
    if (cnt == 0) return;
    // boundary slots of the run's first and last dwords
    const int64_t bdw = ((gu + (int64_t)s_toff[min(lane, U)]) * PB) >> 5;
    const uint64_t mf = __ballot(lane <= U && bdw == ((g * PB) >> 5));
    const uint64_t ml = __ballot(lane <= U && bdw == (((g + cnt) * PB - 1) >> 5));
    const int slot_first = mf ? __ffsll((unsigned long long)mf) - 1 : -1;
    const int slot_last = ml ? __ffsll((unsigned long long)ml) - 1 : -1;
    // dwords and bits are counted from the run's first dword D0 (32-bit math)
    const int64_t D0 = (g * PB) >> 5;
    uint32_t* const out = reinterpret_cast<uint32_t*>(a.vals) + D0;
    const int sb = (int)((g * PB) & 31), eb = sb + cnt * PB;   // run bits [sb, eb)
    const int dend = (eb + 31) >> 5;
    const int64_t capw = a.vals_capacity - D0;                 // dwords left in the stream (64-bit: a
    const int dcap = capw <= 0 ? 0 : (int)min<int64_t>(capw, (int64_t)dend);   // far cursor must not wrap)
    int dn = 0;                                  // next dword to produce
    int base = 0;
    // rounds are written into the ring until the next one might not fit
    // (a round adds <= 512 values and 8 of overrun); each flush then builds
    // the dwords its values complete
#pragma unroll
    for (int k = 0; k < 8; k++) {
        {
            const uint32_t m = (mp[k >> 2] >> (8 * (k & 3))) & 0xffu;
            const uint32_t c = (uint32_t)__popc(m);
            const uint32_t ex = wave_incl_scan(c) - c;
            if (c != 0u) write_compacted<OUTB>(ring + ((int)P[k] - base + (int)ex) * OUTB, o[k]);
        }
        if (k < 7 && (int)P[k + 1] - base + 520 <= kRingElems) continue;
        wave_sync_lds();
        const int done = (int)P[k + 1];
        const int dl = done == cnt ? dend : ((sb + done * PB) >> 5);
        const int dlw = min(dl, dcap);
        for (int d = dn + lane; d < dlw; d += 64) {
            const int lo = max(d * 32, sb), hi = min(d * 32 + 32, eb);
            const int v0 = (lo - sb) / PB, v1 = (hi - 1 - sb) / PB;
            // values v0 .. v1 side by side in a 64-bit window (value v0 + j at
            // bit PB j, MAXV PB <= 60 bits), then shifted so that stream bit
            // 32 d lands on bit 0: by s0 = 32 d - (sb + v0 PB), which is in
            // [0, PB) inside the run and negative only for its first dword
            uint64_t win = 0;
#pragma unroll
            for (int j = 0; j < MAXV; j++) {
                const int v = v0 + j;
                uint32_t x = 0;
                if (v <= v1) {
                    if constexpr (OUTB == 2) x = reinterpret_cast<const uint16_t*>(ring)[v - base];
                    else x = ring[v - base];
                }
                win |= (uint64_t)(x & VMASK) << (PB * j);
            }
            const int s0 = d * 32 - (sb + v0 * PB);
            const uint32_t word = s0 >= 0 ? (uint32_t)(win >> s0) : (uint32_t)(win << (-s0));
            if (lo == d * 32 && hi == d * 32 + 32) {
                out[d] = word;
            } else {
                const int slot = d == 0 ? slot_first : slot_last;
                if (slot >= 0) atomicOr(&s_edge[slot], word);
                else merge_word(out, d, word, bit_range_mask((uint32_t)(lo - d * 32), (uint32_t)(hi - d * 32)));
            }
        }
        if (dl > dn) dn = dl;
        if (done == cnt) break;
        {
            // values [vf, done) overlap dword dn, which a later flush completes
            const int rel = dn * 32 - sb;
            const int vf = rel > 0 ? rel / PB : 0;
            const int np = done - vf;            // <= MAXV
            uint32_t x = 0;
            if (lane < np) {
                if constexpr (OUTB == 2) x = reinterpret_cast<const uint16_t*>(ring)[vf - base + lane];
                else x = ring[vf - base + lane];
            }
            wave_sync_lds();
            if (lane < np) {
                if constexpr (OUTB == 2) reinterpret_cast<uint16_t*>(ring)[lane] = (uint16_t)x;
                else ring[lane] = (uint8_t)x;
            }
            base = vf;
        }
        wave_sync_lds();
    }
}

// Write the unit's boundary dwords collected in s_edge (wave 0, lane b =
// boundary b; the unit's run starts at value gu).  A dword is written by the
// first boundary in it, and only if some run saw it as partial: a boundary
// inside it, or the unit's range covering part of it.  Dwords inside the unit
// are stored whole; the two at the unit's ends, shared with the neighbouring
// units, are merged with disjoint-bit atomics.
template <int PB, int U>
__device__ __forceinline__ void packed_unit_edges(const CompressArgs& a, int64_t gu, const uint32_t* s_toff,
                                                  const uint32_t* s_edge, int lane)
{
    const int64_t us = gu * PB, ue = (gu + (int64_t)s_toff[U]) * PB;
    if (ue <= us || lane > U) return;
    const int b = lane;
    const int64_t Bb = (gu + (int64_t)s_toff[b]) * PB, Db = Bb >> 5;
    if (b > 0 && (((gu + (int64_t)s_toff[b - 1]) * PB) >> 5) == Db) return;   // not the first in its dword
    bool inner = false;
    for (int b2 = b; b2 <= U; b2++) {
        const int64_t B2 = (gu + (int64_t)s_toff[b2]) * PB;
        if ((B2 >> 5) != Db) break;
        inner |= (B2 & 31) != 0;
    }
    const int64_t lo = max(Db * 32, us), hi = min(Db * 32 + 32, ue);
    if (lo < hi && Db < a.vals_capacity && (inner || lo > Db * 32 || hi < Db * 32 + 32))
        merge_word(reinterpret_cast<uint32_t*>(a.vals), Db, s_edge[b],
                   bit_range_mask((uint32_t)(lo - Db * 32), (uint32_t)(hi - Db * 32)));
}

#ifndef BS_QUANT_WAVES_PER_EU
#define BS_QUANT_WAVES_PER_EU 8
#endif

#ifndef BS_PACKED_WAVES_PER_EU
#define BS_PACKED_WAVES_PER_EU 7
#endif

// NT: nontemporal loads of the dense input and stores of the value slots.
// RSQ: the fused ReLU's write-back is the ReLU^2 layer's in-place square
// (relu2_sq_bits of relu(dense)); the compressed form is that of relu(dense).
template <int IN_T, bool QUANT, bool VEC, int MODE, int U, bool PACKED, bool NT, bool RSQ = false>
__global__ __launch_bounds__(64 * U) __attribute__((amdgpu_waves_per_eu(
    QUANT ? BS_QUANT_WAVES_PER_EU : (PACKED ? BS_PACKED_WAVES_PER_EU : BS_STREAM_WAVES_PER_EU))))
void compress_stream_kernel(CompressArgs a)
{
    static_assert(!(QUANT && MODE == MODE_VALS), "the values pass copies stored values");
    static_assert(!PACKED || MODE == MODE_FUSED, "the packed stream is written by the fused pass");
    static_assert(!RSQ || (IN_T == DT_BF16 && MODE == MODE_FUSED && !PACKED), "the ReLU^2 write-back");
    constexpr bool WRITE_VALS = MODE != MODE_COUNT;
    using TR = CompressTraits<IN_T, QUANT>;
    constexpr int INB = TR::INB, OUTB = TR::OUTB;
    constexpr int EPS = 16 / OUTB;          // elements per 16-byte slot
    constexpr int NSEL = OUTB == 2 ? 8 : 2; // selector dwords per mask byte
    using RawIn = typename Raw<INB>::T;
    using RawOut = typename Raw<OUTB>::T;
    static_assert(U >= 1 && U <= 16, "one wave per tile, at most 16 waves");

    __shared__ uint32_t s_cnt[U];
    __shared__ uint32_t s_toff[U + 1];      // tile offsets inside the unit's run; [U] = unit total
    __shared__ uint32_t s_edge[PACKED ? U + 1 : 1];   // packed: boundary dwords of the unit's runs
    __shared__ uint32_t s_excl[1];
    __shared__ __align__(16) uint32_t s_sel[WRITE_VALS ? 256 * NSEL : 4];
    // the quantizer's code table is read only while the chunks are masked,
    // the value rings only after the look-back's barrier: they share LDS
    constexpr int kRingBytes = WRITE_VALS ? U * kRingElems * OUTB : 16;
    constexpr int kShared = QUANT && kQtabBytes > kRingBytes ? kQtabBytes : kRingBytes;
    __shared__ __align__(16) uint8_t s_area[kShared];
    uint8_t* const s_ring = s_area;
    uint8_t* const s_qtab = s_area;

    // the wave index in a scalar register: branches on it are scalar
    // branches, not exec masks, so nothing the compiler places at their joins
    // (register spills among them) runs with some lanes switched off
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    if constexpr (PACKED) {
        if (tid <= U) s_edge[tid] = 0u;
    }

    float scale = 1.0f;
    if constexpr (QUANT) scale = scale_from_slot(a.amax_slot, a.amax_epoch);
    const float rcp = 1.0f / scale;
    const int qoff = QUANT ? qtab_offset(scale) : 0;
    int64_t start = 0;
    if (a.offset_in) start = *a.offset_in;
    if (a.align8) start = (start + 7) & ~(int64_t)7;
    // no barrier here: the dense loads below go out at once, and the
    // selector table (and the packed edge slots) are next read after the
    // barrier that follows the masks (or, for the values pass, the one below)

    {
        const uint32_t u = blockIdx.x;

        const uint32_t t0 = a.tile0 + u * U;
        const int ntiles = (int)min((uint32_t)U, a.tend - t0);
        const bool tile_ok = wave < ntiles;     // wave-uniform
        const uint32_t t = t0 + (uint32_t)wave;

        // ---- loads: all eight chunks of the lane in flight together.  Waves
        // past the last tile read the last tile again; with VEC, rows and
        // columns past the matrix read a clamped in-range address.  Either way
        // the chunk's mask byte is forced to 0, so no load is conditional (a
        // conditional load makes the compiler wait for it before the next).
        const uint32_t tc = tile_ok ? t : a.tend - 1;
        const uint32_t tm = tc / a.grid_n, tn = tc - tm * a.grid_n;
        const int64_t row0 = (int64_t)tm * 64 + (lane >> 3);
        const int64_t col0 = (int64_t)tn * 64 + (lane & 7) * 8;
        RawIn d[8];
        uint32_t vm[8];                         // MODE_VALS: the given bitmask bytes
        // chunk k is inside the matrix iff 8k < rows_in (rows_in <= 0: none)
        const int64_t rows_in = (tile_ok && col0 < a.N) ? a.M - row0 : 0;
        // VEC addressing: the tile origin and chunk k's row step are uniform
        // over the wave (64-bit, scalar registers); the lane's place in the
        // tile is one 32-bit register, (lane/8) rows of N elements plus its
        // column (< 8 N elements: the host takes this path only when 8 N
        // elements of the widest operand fit 32 bits)
        const uint64_t t_org = (uint64_t)tm * 64 * (uint64_t)a.N + (uint64_t)tn * 64;
        const uint32_t r_in = (uint32_t)(lane >> 3) * (uint32_t)a.N;
        const uint32_t c_in = (uint32_t)(min(col0, a.N - 8) - (int64_t)tn * 64);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int64_t row = row0 + 8 * k;
            if constexpr (VEC) {
                // rows past the matrix read the tile's first row (in range)
                const uint32_t lo = (row < a.M ? r_in : 0u) + c_in;
                d[k] = ld_chunk<NT, RawIn>(a.dense + (t_org + (uint64_t)(8 * k) * (uint64_t)a.N) * INB +
                                           (uint64_t)(lo * (uint32_t)INB));
            } else {
                d[k] = tile_ok ? load_chunk<INB, false>(a.dense, a.M, a.N, row, col0) : RawIn{};
            }
            if constexpr (MODE == MODE_VALS) vm[k] = a.bitmask[(size_t)tc * kTileBytes + 64 * k + lane];
        }
        // the compaction selector table, while the loads are in flight
        if constexpr (WRITE_VALS) {
            if (tid < 256) {
                uint32_t sel[NSEL];
                compaction_selectors<OUTB>((uint32_t)tid, sel);
#pragma unroll
                for (int i = 0; i < NSEL; i += 2)
                    *reinterpret_cast<uint2*>(&s_sel[tid * NSEL + i]) = make_uint2(sel[i], sel[i + 1]);
            }
        }
        if constexpr (QUANT) {
            // the code table into LDS, behind the dense loads (16-byte copies)
            for (int i = tid; i < kQtabBytes / 16; i += 64 * U)
                reinterpret_cast<uint4*>(s_qtab)[i] = reinterpret_cast<const uint4*>(a.qtab)[i];
            __syncthreads();
        }
        if constexpr (MODE != MODE_VALS) {
            if (a.relu) {
#pragma unroll
                for (int k = 0; k < 8; k++) d[k] = relu_chunk<IN_T>(d[k]);
            }
        }

        // ---- masks, bitmask bytes, round totals
        RawOut o[8];
        uint32_t mp[2] = {0u, 0u};              // the eight mask bytes, four per register
        uint32_t P[9];                          // wave-uniform run offset of each round
        P[0] = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            uint32_t m;
            if constexpr (MODE == MODE_VALS) {
                o[k] = d[k];
                m = tile_ok ? vm[k] & 0xffu : 0u;
            } else {
                m = stream_chunk_mask<IN_T, QUANT, QUANT>(d[k], o[k], scale, rcp, s_qtab, qoff) &
                    (8 * k < rows_in ? 0xffu : 0u);
                if (tile_ok) {
                    if constexpr (VEC) {
                        // in range, the lane's unclamped place in the tile
                        const uint64_t ko = t_org + (uint64_t)(8 * k) * (uint64_t)a.N;
                        const uint32_t lo = r_in + c_in;
                        if (a.relu_out != nullptr && 8 * k < rows_in) {
                            if constexpr (RSQ)
                                st_chunk<false, RawIn>(a.relu_out + ko * INB + (uint64_t)(lo * (uint32_t)INB),
                                                       relu2_sq_chunk(d[k], a.relu_k));
                            else
                                st_chunk<false, RawIn>(a.relu_out + ko * INB + (uint64_t)(lo * (uint32_t)INB), d[k]);
                        }
                        if constexpr (QUANT) {
                            if (a.dense_q_out != nullptr && 8 * k < rows_in)
                                st_chunk<false, RawOut>(a.dense_q_out + ko + (uint64_t)lo, o[k]);
                        }
                    } else {
                        if (a.relu_out != nullptr) {
                            if constexpr (RSQ)
                                store_chunk<INB, VEC>(a.relu_out, a.M, a.N, row0 + 8 * k, col0,
                                                      relu2_sq_chunk(d[k], a.relu_k));
                            else
                                store_chunk<INB, VEC>(a.relu_out, a.M, a.N, row0 + 8 * k, col0, d[k]);
                        }
                        if constexpr (QUANT) {
                            if (a.dense_q_out != nullptr)
                                store_chunk<1, VEC>(a.dense_q_out, a.M, a.N, row0 + 8 * k, col0, o[k]);
                        }
                    }
                    // wave 0 stores its bytes after the look-back: a store
                    // ahead of a status read delays the read until it is
                    // acknowledged (vector memory counts retire in order)
                    if (wave != 0) a.bitmask[(size_t)t * kTileBytes + 64 * k + lane] = (uint8_t)m;
                }
            }
            mp[k >> 2] |= m << (8 * (k & 3));
            P[k + 1] = P[k] + wave_sum_count(__popc(m));
        }
        if constexpr (MODE != MODE_VALS) {
            if (lane == 0) s_cnt[wave] = P[8];
        }
        __syncthreads();                        // s_cnt; the selector table

        // ---- unit total and aggregate (wave 0)
        uint32_t v = 0, x = 0, unit_total = 0;
        if (MODE != MODE_VALS && wave == 0) {
            v = lane < U ? s_cnt[lane] : 0u;
            x = v;
#pragma unroll
            for (int off = 1; off < U; off <<= 1) {
                const uint32_t y = __shfl_up(x, off, 64);
                if (lane >= off) x += y;
            }
            unit_total = __shfl(x, U - 1, 64);
            if (lane < U) s_toff[lane] = x - v;
            if (lane == U - 1) s_toff[U] = x;
            if (U == 1 && lane == 0)
                st_relaxed(&a.status[u], pack_status(a.epoch, u == 0 ? kFlagInc : kFlagAgg, unit_total));
        }
        if (MODE != MODE_VALS && U > 1 && wave == 1) {
            // the unit's aggregate is published by wave 1, so that wave 0
            // enters the look-back with no store outstanding.  Wave 0's
            // inclusive word may land first and this aggregate over it: a
            // walk that reads the aggregate adds the unit's total and goes
            // on, so either word gives the same prefix.
            const uint32_t total = wave_total(lane < U ? s_cnt[lane] : 0u);
            if (lane == 0) st_relaxed(&a.status[u], pack_status(a.epoch, u == 0 ? kFlagInc : kFlagAgg, total));
        }
        // ---- compaction of every chunk in registers, which needs no prefix:
        // the mask byte indexes a table of v_perm selectors that move the set
        // elements to the front.  Waves 1.. do it while wave 0 waits in the
        // look-back; o[k] is replaced by its compacted form.
        if constexpr (WRITE_VALS) {
            if (tile_ok) {
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const uint32_t m = (mp[k >> 2] >> (8 * (k & 3))) & 0xffu;
                    if constexpr (OUTB == 2) {
                        const uint4 s0 = *reinterpret_cast<const uint4*>(&s_sel[m * NSEL]);
                        const uint4 s1 = *reinterpret_cast<const uint4*>(&s_sel[m * NSEL + 4]);
                        const uint4 w = o[k];
                        o[k].x = __builtin_amdgcn_perm(w.y, w.x, s0.x) | __builtin_amdgcn_perm(w.w, w.z, s1.x);
                        o[k].y = __builtin_amdgcn_perm(w.y, w.x, s0.y) | __builtin_amdgcn_perm(w.w, w.z, s1.y);
                        o[k].z = __builtin_amdgcn_perm(w.y, w.x, s0.z) | __builtin_amdgcn_perm(w.w, w.z, s1.z);
                        o[k].w = __builtin_amdgcn_perm(w.y, w.x, s0.w) | __builtin_amdgcn_perm(w.w, w.z, s1.w);
                    } else {
                        const uint2 s0 = *reinterpret_cast<const uint2*>(&s_sel[m * NSEL]);
                        const uint2 w = o[k];
                        o[k].x = __builtin_amdgcn_perm(w.y, w.x, s0.x);
                        o[k].y = __builtin_amdgcn_perm(w.y, w.x, s0.y);
                    }
                }
            }
        }
        // ---- look-back, prefix entries (wave 0)
        if (MODE != MODE_VALS && wave == 0) {
            uint32_t excl = 0;
            if (u != 0) {
                excl = wave_lookback_grouped<IN_T, QUANT, VEC, U>(a, u, unit_total, scale, lane);
                if (lane == 0) st_relaxed(&a.status[u], pack_status(a.epoch, kFlagInc, excl + unit_total));
            }
            if (lane == 0 && ((u + 1) & (kGroupUnits - 1)) == 0)
                st_relaxed(&a.gstat[u / kGroupUnits], pack_status(a.epoch, kFlagInc, excl + unit_total));
            if (lane == 0) s_excl[0] = excl;
            if (tile_ok) {
#pragma unroll
                for (int k = 0; k < 8; k++)
                    a.bitmask[(size_t)t * kTileBytes + 64 * k + lane] = (uint8_t)(mp[k >> 2] >> (8 * (k & 3)));
            }
            if (lane < ntiles) a.prefix[t0 + lane] = excl + (x - v);
            if (lane == 0 && t0 + ntiles == a.tend) {
                a.prefix[a.tend] = excl + unit_total;
                const int64_t end = start + (int64_t)(excl + unit_total);
                if (a.offset_out) *a.offset_out = end;
                if (a.start_out) *a.start_out = start;
                if constexpr (PACKED) {
                    if (a.err && end * TR::PB > a.vals_capacity * 32) atomicOr(a.err, 1);
                } else {
                    if (a.err && end > a.vals_capacity && WRITE_VALS) atomicOr(a.err, 1);
                }
                if (start < 0 && a.err && WRITE_VALS) atomicOr(a.err, 2);
            }
            if constexpr (QUANT) {
                if (u == 0 && lane == 0 && a.scale_out) *a.scale_out = scale;
            }
        }
        if constexpr (WRITE_VALS) {
            if constexpr (MODE == MODE_VALS) {
                if (start < 0 && tid == 0 && a.err) atomicOr(a.err, 2);
            } else {
                __syncthreads();
            }
            if (tile_ok && start >= 0) {
                int64_t g;
                if constexpr (MODE == MODE_VALS)
                    g = start + (int64_t)(a.prefix[t] - a.prefix[a.tile0]);
                else
                    g = start + (int64_t)uniform_u32(s_excl[0]) + (int64_t)uniform_u32(s_toff[wave]);
                const int cnt = (int)P[8];
                if constexpr (PACKED) {
                    stream_packed<OUTB, TR::PB, U>(a, g, cnt, P, mp, o, s_ring + wave * (kRingElems * OUTB), lane,
                                                   start + (int64_t)uniform_u32(s_excl[0]),
                                                   s_toff, s_edge);
                } else {
                if (MODE == MODE_VALS && a.err && lane == 0 && g + cnt > a.vals_capacity) atomicOr(a.err, 1);
                const int a0 = (int)((((uintptr_t)a.vals) + (uint64_t)g * OUTB) & 15u) / OUTB;
                const int64_t room = a.vals_capacity - g;
                const int endr = (int)max<int64_t>(0, min<int64_t>((int64_t)cnt, room));
                uint8_t* const slot_base = a.vals + (g - a0) * OUTB;      // 16-byte aligned
                uint8_t* const ring = s_ring + wave * (kRingElems * OUTB);
                const int j_lo = a0 ? 1 : 0;                              // first whole slot
                const int j_hi = (a0 + endr) / EPS;                       // one past the last whole slot
                const int front_n = a0 ? min(endr, EPS - a0) : 0;         // leading partial slot
                const int back_s = max(j_hi, j_lo) * EPS - a0;            // trailing partial slot
                bool front_done = front_n == 0;
                bool back_done = back_s >= endr;
                int pend = 0;                   // output slot held in ring slot 0
#pragma unroll
                for (int k0 = 0; k0 < 8; k0 += kRoundsPerPass) {
                    if (front_done && back_done && max(pend, j_lo) >= j_hi) break;
                    // one pass at a time: nothing of a later pass is computed early
                    asm volatile("" : "+v"(mp[0]), "+v"(mp[1]) : : "memory");
#pragma unroll
                    for (int kk = 0; kk < kRoundsPerPass; kk++) {
                        const int k = k0 + kk;
                        const uint32_t m = (mp[k >> 2] >> (8 * (k & 3))) & 0xffu;
                        const uint32_t c = (uint32_t)__popc(m);
                        const uint32_t ex = wave_incl_scan(c) - c;
                        const int rb = a0 + (int)P[k] - pend * EPS;       // ring index of the round's first element
                        if (c != 0u) write_compacted<OUTB>(ring + (rb + (int)ex) * OUTB, o[k]);
                    }
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                    const int done = (int)P[k0 + kRoundsPerPass];
                    const int npend = (a0 + done) / EPS;
                    if (!front_done && done >= front_n) {
                        front_done = true;          // pend is still 0 here
                        if (lane < front_n) ring_elem_store<OUTB>(a.vals, g + lane, ring, a0 + lane);
                    }
                    const int jh = min(j_hi, npend);
                    for (int j = max(pend, j_lo) + lane; j < jh; j += 64)
                        st16<NT>(slot_base + (int64_t)j * 16,
                                        *reinterpret_cast<const uint4*>(ring + (j - pend) * 16));
                    if (!back_done && done >= endr) {
                        back_done = true;
                        const int r = back_s + lane;
                        if (lane < EPS && r < endr)
                            ring_elem_store<OUTB>(a.vals, g + r, ring, a0 + r - pend * EPS);
                    }
                    if (npend > pend) {
                        if (lane == 0)
                            *reinterpret_cast<uint4*>(ring) =
                                *reinterpret_cast<const uint4*>(ring + (npend - pend) * 16);
                        pend = npend;
                    }
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                }
                }
            }
            if constexpr (PACKED) {
                __syncthreads();
                if (wave == 0 && start >= 0)
                    packed_unit_edges<TR::PB, U>(a, start + (int64_t)s_excl[0], s_toff, s_edge, lane);
            }
        }
    }
}

// ===========================================================================
// bitstream packing (pack_sbit storage)
//
// Value i of a packed stream occupies stream bits [i*PB, (i+1)*PB), LSB first
// (byte i*PB/8 holds the low bits); the payload is the low PB bits of the
// stored value (15 for bf16, 7 for fp8: the sign bit of a ReLU value is 0).
// The kernel packs raw[0, count) to stream indices [start, start + count):
// one thread per output dword, each gathering the <= 4 (bf16) / <= 6 (fp8)
// values that overlap it.  Dwords shared with bits outside the run keep those
// bits (atomicAnd of the run's bit mask complement, then atomicOr of the
// run's bits: concurrent writers of disjoint bits commute).
// ===========================================================================

constexpr int kPackThreads = 256;

template <int VB, int PB>
__global__ __launch_bounds__(kPackThreads) void pack_bits_kernel(const uint8_t* raw, const uint32_t* count_ptr,
                                                                 int64_t count_max, uint32_t* out,
                                                                 int64_t out_words, const int64_t* start_ptr,
                                                                 int32_t* err, int raw_vec)
{
    // one 8-value group per thread: PB bytes of stream (15 / 7), staged here
    __shared__ uint32_t s_out[kPackThreads * PB / 4 + 2];
    const int tid = threadIdx.x;
    const int64_t start = start_ptr ? *start_ptr : 0;
    int64_t count = count_max;
    if (count_ptr) count = min((int64_t)*count_ptr, count_max);
    if (start < 0) {
        if (err && blockIdx.x == 0 && tid == 0) atomicOr(err, 2);
        return;
    }
    const int64_t S = start * PB, E = (start + count) * PB;   // stream bits of the run
    if (count <= 0) return;
    if (E > out_words * 32) {                                 // past the storage: flag, pack what fits
        if (err && blockIdx.x == 0 && tid == 0) atomicOr(err, 1);
    }

    if ((start & 7) != 0 || !raw_vec) {
        // general start (or raw values not aligned for vector loads): one
        // thread per output dword, gathering the <= 4 / <= 6
        // values that overlap it
        const int64_t D0 = S >> 5, D1 = min((E + 31) >> 5, out_words);
        for (int64_t D = D0 + (int64_t)blockIdx.x * kPackThreads + tid; D < D1;
             D += (int64_t)gridDim.x * kPackThreads) {
            const int64_t lo = max(D * 32, S), hi = min(D * 32 + 32, E);
            const int64_t v0 = (lo - S) / PB, v1 = (hi - 1 - S) / PB;
            uint64_t acc = 0;
            for (int64_t v = v0; v <= v1; v++) {
                const uint32_t x = (VB == 2 ? (uint32_t)reinterpret_cast<const uint16_t*>(raw)[v]
                                            : (uint32_t)raw[v]) & ((1u << PB) - 1u);
                const int64_t pos = S + v * PB - D * 32;       // > -PB
                acc |= pos >= 0 ? ((uint64_t)x << pos) : ((uint64_t)x >> (-pos));
            }
            merge_word(out, D, (uint32_t)acc, bit_range_mask((uint32_t)(lo - D * 32), (uint32_t)(hi - D * 32)));
        }
        return;
    }

    // start % 8 == 0 (and raw aligned to 8 values): group g (values 8g..8g+7) is exactly PB stream bytes at
    // byte S/8 + g*PB.  A workgroup packs 256 consecutive groups in registers,
    // stages their bytes contiguously in LDS at the dword phase of the output,
    // and stores whole dwords; only the two dwords at the ends of its span
    // (shared with the neighbouring workgroups or outside bits) are merged.
    const int64_t ngroups = (count + 7) / 8;
    const int64_t byte_base = S >> 3;
    for (int64_t gb = (int64_t)blockIdx.x * kPackThreads; gb < ngroups; gb += (int64_t)gridDim.x * kPackThreads) {
        const int64_t g = gb + tid;
        uint32_t w[8];
        const int64_t v0 = g * 8;
        if (v0 + 8 <= count) {
            if constexpr (VB == 2) {
                const uint4 r = *reinterpret_cast<const uint4*>(raw + v0 * 2);
                w[0] = r.x & 0xffffu; w[1] = r.x >> 16; w[2] = r.y & 0xffffu; w[3] = r.y >> 16;
                w[4] = r.z & 0xffffu; w[5] = r.z >> 16; w[6] = r.w & 0xffffu; w[7] = r.w >> 16;
            } else {
                const uint2 r = *reinterpret_cast<const uint2*>(raw + v0);
#pragma unroll
                for (int e = 0; e < 8; e++) w[e] = ((e < 4 ? r.x : r.y) >> (8 * (e & 3))) & 0xffu;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++)
                w[e] = (v0 + e < count) ? (VB == 2 ? (uint32_t)reinterpret_cast<const uint16_t*>(raw)[v0 + e]
                                                   : (uint32_t)raw[v0 + e]) : 0u;
        }
        // 8 x PB bits, LSB first, into up to 4 dwords
        uint64_t lo64 = 0, hi64 = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint64_t x = w[e] & ((1u << PB) - 1u);
            const int pos = e * PB;
            if (pos < 64) {
                lo64 |= x << pos;
                if (pos + PB > 64) hi64 |= x >> (64 - pos);
            } else {
                hi64 |= x << (pos - 64);
            }
        }
        const int64_t gbytes0 = byte_base + gb * PB;               // the span's first byte
        const int phase = (int)(gbytes0 & 3);
        uint8_t* sb = reinterpret_cast<uint8_t*>(s_out);
        const int o = phase + tid * PB;
#pragma unroll
        for (int k = 0; k < PB; k++) {
            const uint64_t src = k < 8 ? lo64 : hi64;
            sb[o + k] = (uint8_t)(src >> (8 * (k & 7)));
        }
        __syncthreads();
        // stream bits this span covers: [Sb, Eb)
        const int64_t Sb = gbytes0 * 8;
        const int64_t Eb = min(E, (byte_base + min(gb + kPackThreads, ngroups) * PB) * 8);
        const int64_t D0 = gbytes0 >> 2, D1 = min((Eb + 31) >> 5, out_words);
        for (int64_t D = D0 + tid; D < D1; D += kPackThreads) {
            const uint32_t word = s_out[D - D0];
            const int64_t lo = max(D * 32, Sb), hi = min(D * 32 + 32, Eb);
            merge_word(out, D, word, bit_range_mask((uint32_t)(lo - D * 32), (uint32_t)(hi - D * 32)));
        }
        __syncthreads();
    }
}

// ===========================================================================
// tile_pack: bitmask + int32 counts (reference API shape)
// ===========================================================================
template <int IN_T, bool VEC>
__global__ __launch_bounds__(kThreads) void tile_pack_kernel(const uint8_t* dense, int64_t M, int64_t N,
                                                             uint32_t grid_n, int32_t* counts,
                                                             uint8_t* bitmask)
{
    constexpr int INB = IN_T == DT_BF16 ? 2 : 1;
    __shared__ uint32_t s_tot[4];
    const int tid = threadIdx.x;
    const uint32_t t = blockIdx.x;
    uint32_t c = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        int b = h * 256 + tid;
        int64_t row, col0;
        chunk_pos(t, grid_n, b, row, col0);
        auto d = load_chunk<INB, VEC>(dense, M, N, row, col0);
        typename Raw<INB>::T o;
        uint32_t mk = chunk_mask<IN_T, false>(d, o, 1.0f, 1.0f);
        bitmask[(size_t)t * kTileBytes + b] = (uint8_t)mk;
        c += __popc(mk);
    }
    c = wave_sum_u32(c);
    if ((tid & 63) == 0) s_tot[tid >> 6] = c;
    __syncthreads();
    if (tid == 0) counts[t] = (int32_t)(s_tot[0] + s_tot[1] + s_tot[2] + s_tot[3]);
}

// ===========================================================================
// prefix from counts: one workgroup, 1024 threads, carries across blocks
// ===========================================================================
__global__ __launch_bounds__(1024) void prefix_kernel(const int32_t* counts, int64_t T, uint32_t* prefix)
{
    __shared__ uint32_t s_w[16];
    __shared__ uint32_t s_carry;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    if (tid == 0) { s_carry = 0; prefix[0] = 0; }
    __syncthreads();
    for (int64_t base = 0; base < T; base += 1024) {
        int64_t i = base + tid;
        uint32_t v = i < T ? (uint32_t)counts[i] : 0u;
        // inclusive wave scan
        uint32_t x = v;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            uint32_t y = __shfl_up(x, o, 64);
            if (lane >= o) x += y;
        }
        if (lane == 63) s_w[wave] = x;
        __syncthreads();
        uint32_t wb = 0, all = 0;
        for (int w = 0; w < 16; w++) {
            uint32_t tw = s_w[w];
            if (w < wave) wb += tw;
            all += tw;
        }
        uint32_t carry = s_carry;
        if (i < T) prefix[i + 1] = carry + wb + x;
        __syncthreads();
        if (tid == 0) s_carry = carry + all;
        __syncthreads();
    }
}

// ===========================================================================
// decompress / relu2-gradient value gather
// ===========================================================================
struct GatherArgs {
    const uint8_t* vals;
    int64_t vals_numel;
    const uint8_t* bitmask;
    const uint32_t* prefix;
    const int64_t* vals_offset;
    uint8_t* out;          // decompress: [rows, K] output; relu2: the gradient
    int64_t first_m_tile;
    uint32_t grid_n;
    int64_t K;             // columns of out
    int64_t rows;          // rows of out
    uint32_t num_tiles;
    float relu2_scale;
    const float* scale;
};

// Stage the value run of tiles [t0, t0+ntiles) in LDS; returns its phase.
// The run is [vo + prefix[t0], vo + prefix[t0+ntiles]).
template <int VB, bool NT>
__device__ __forceinline__ int stage_run(const GatherArgs& a, int64_t run0, int64_t run1,
                                         int64_t max_count, uint8_t* s_vals, int tid)
{
    constexpr int EPS = 16 / VB;
    const int p = (int)((((uintptr_t)a.vals) / VB + (uint64_t)run0) % EPS);
    // a consistent prefix gives 0 <= count <= 4096 per tile; clamp so that a
    // corrupt one can never index past the staging buffer
    int64_t cnt64 = run1 - run0;
    cnt64 = cnt64 < 0 ? 0 : (cnt64 > max_count ? max_count : cnt64);
    const int count = (int)cnt64;
    const int nslots = (p + count + EPS - 1) / EPS;
    for (int s = tid; s < nslots; s += kThreads) {
        const int64_t e0 = run0 - p + (int64_t)s * EPS;
        uint4 v = {0u, 0u, 0u, 0u};
        if (e0 >= 0 && e0 + EPS <= a.vals_numel) {
            v = ld16<NT>(a.vals + e0 * VB);
        } else {
            for (int e = 0; e < EPS; e++) {
                int64_t i = e0 + e;
                if (i >= 0 && i < a.vals_numel) {
                    if (VB == 2) {
                        uint32_t x = reinterpret_cast<const uint16_t*>(a.vals)[i];
                        uint32_t* w = e < 2 ? &v.x : e < 4 ? &v.y : e < 6 ? &v.z : &v.w;
                        *w |= x << ((e & 1) * 16);
                    } else {
                        uint32_t x = a.vals[i];
                        uint32_t* w = e < 4 ? &v.x : e < 8 ? &v.y : e < 12 ? &v.z : &v.w;
                        *w |= x << ((e & 3) * 8);
                    }
                }
            }
        }
        *reinterpret_cast<uint4*>(s_vals + s * 16) = v;
    }
    return p;
}

// Packed variant: stage the stream bytes holding bits [run0*PB, run1*PB) of
// a PB-bit value stream (vals_numel = stream bytes) from a 16-byte aligned
// byte, plus one more 16-byte slot so two-dword reads never leave the staged
// data.  Returns the bit position of value run0 inside the staged bytes.
template <int PB, bool NT>
__device__ __forceinline__ int stage_run_packed(const GatherArgs& a, int64_t run0, int64_t run1,
                                                int64_t max_count, uint8_t* s_vals, int tid)
{
    int64_t cnt64 = run1 - run0;
    cnt64 = cnt64 < 0 ? 0 : (cnt64 > max_count ? max_count : cnt64);
    const int64_t bit0 = run0 * PB;
    const int64_t sb = (bit0 >> 3) & ~(int64_t)15;                 // first staged byte
    const int64_t eb = (bit0 + cnt64 * PB + 7) >> 3;               // one past the last needed byte
    const int nslots = (int)((eb - sb + 15) >> 4) + 1;
    for (int s = tid; s < nslots; s += kThreads) {
        const int64_t b0 = sb + (int64_t)s * 16;
        uint4 v = {0u, 0u, 0u, 0u};
        if (b0 >= 0 && b0 + 16 <= a.vals_numel) {
            v = ld16<NT>(a.vals + b0);
        } else {
            for (int e = 0; e < 16; e++) {
                const int64_t i = b0 + e;
                if (i >= 0 && i < a.vals_numel) {
                    uint32_t* w = e < 4 ? &v.x : e < 8 ? &v.y : e < 12 ? &v.z : &v.w;
                    *w |= (uint32_t)a.vals[i] << ((e & 3) * 8);
                }
            }
        }
        *reinterpret_cast<uint4*>(s_vals + s * 16) = v;
    }
    return (int)(bit0 - sb * 8);
}

// Shared front half of decompress and relu2_grad: bitmask bytes, in-tile
// ranks, run staging.  Fills m[][], r0[][] (LDS element index of each chunk's
// first value) and returns after a barrier.
// M_LOADED: the caller already holds the mask bytes in m and prefix[t0 + tid]
// (tid <= ntiles) in pf.  vo: the run's cursor (*vals_offset, 0 without),
// which callers read at their start with the mask bytes, so that the staging
// waits for one memory round trip before it rather than two.
template <int VB, int PB, int U, bool NT, bool M_LOADED = false>
__device__ __forceinline__ int gather_prepare(const GatherArgs& a, uint32_t t0, int ntiles,
                                              uint32_t (&m)[U][2], uint32_t (&r0)[U][2],
                                              uint32_t* s_pref, uint32_t (*s_wtot)[2][4],
                                              uint8_t* s_vals, int tid, int64_t vo, uint32_t pf = 0u)
{
    const int wave = tid >> 6, lane = tid & 63;
    if constexpr (!M_LOADED) {
#pragma unroll
        for (int j = 0; j < U; j++)
#pragma unroll
            for (int h = 0; h < 2; h++)
                m[j][h] = j < ntiles ? a.bitmask[(size_t)(t0 + j) * kTileBytes + h * 256 + tid] : 0u;
        if (tid <= ntiles) pf = a.prefix[t0 + tid];
    }
    if (tid <= ntiles) s_pref[tid] = pf;
    uint32_t ex[U][2];
#pragma unroll
    for (int j = 0; j < U; j++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            // DPP prefix sum: the four chunks' scans are independent, so their
            // DPP steps interleave (fewer VALU instructions than bit-plane
            // ballots and mbcnt)
            const uint32_t c = (uint32_t)__popc(m[j][h]);
            const uint32_t incl = wave_incl_scan(c);
            ex[j][h] = incl - c;
            const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
            if (lane == 0) s_wtot[j][h][wave] = tot;
        }
    __syncthreads();
    const uint32_t pb = s_pref[0];
    int p = 0, bitbase = 0;
    if constexpr (PB > 0)
        bitbase = stage_run_packed<PB, NT>(a, vo + pb, vo + s_pref[ntiles], (int64_t)ntiles * kTileNumel,
                                       s_vals, tid);
    else
        p = stage_run<VB, NT>(a, vo + pb, vo + s_pref[ntiles], (int64_t)ntiles * kTileNumel, s_vals, tid);
#pragma unroll
    for (int j = 0; j < U; j++) {
        uint32_t tb = j < ntiles ? min(s_pref[j] - pb, (uint32_t)(j * kTileNumel)) : 0u;
        uint32_t h0 = 0, h0w = 0, h1w = 0;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            uint32_t a0 = s_wtot[j][0][w], a1 = s_wtot[j][1][w];
            h0 += a0;
            if (w < wave) { h0w += a0; h1w += a1; }
        }
        r0[j][0] = (uint32_t)p + tb + h0w + ex[j][0];
        r0[j][1] = (uint32_t)p + tb + h0 + h1w + ex[j][1];
    }
    __syncthreads();
    return bitbase;
}

// Stored bits of the i-th staged value.  Packed (PB > 0): bits
// [bitbase + i*PB, +PB) of the staged stream, from two aligned dword reads.
template <int V_T, int PB>
__device__ __forceinline__ uint32_t lds_val(const uint8_t* s_vals, uint32_t i, int bitbase)
{
    if constexpr (PB > 0) {
        const uint32_t bit = (uint32_t)bitbase + i * PB;
        const uint32_t* w = reinterpret_cast<const uint32_t*>(s_vals) + (bit >> 5);
        return __builtin_amdgcn_alignbit(w[1], w[0], bit & 31u) & ((1u << PB) - 1u);
    } else if constexpr (V_T == DT_BF16) {
        return reinterpret_cast<const uint16_t*>(s_vals)[i];
    } else {
        return s_vals[i];
    }
}

// k*v*v as bf16 bits: bf16 storage squares in bf16 ((k*v) rounded, then *v
// rounded); fp8 storage widens to fp32 and rounds once.
template <int V_T>
__device__ __forceinline__ uint32_t relu2_square(uint32_t raw, float k)
{
    if constexpr (V_T == DT_BF16) {
        float v = bf16_to_f32(raw);
        float kv = bf16_to_f32(f32_to_bf16(k * v));
        return f32_to_bf16(kv * v);
    } else {
        float v = fp8_to_f32<V_T>(raw);
        return f32_to_bf16((k * v) * v);
    }
}

template <int V_T>
__device__ __forceinline__ float val_f32(uint32_t raw)
{
    if constexpr (V_T == DT_BF16) return bf16_to_f32(raw);
    else return fp8_to_f32<V_T>(raw);
}

// NT: nontemporal staging loads and dense output stores.
template <int V_T, bool SQUARE, bool HAS_SCALE, bool VEC, int U, bool PACKED, bool NT>
__global__ __launch_bounds__(kThreads) void decompress_kernel(GatherArgs a)
{
    constexpr int VB = V_T == DT_BF16 ? 2 : 1;
    constexpr int PB = PACKED ? (V_T == DT_BF16 ? 15 : 7) : 0;
    constexpr int OB = SQUARE ? 2 : VB;
    __shared__ uint32_t s_pref[U + 1];
    __shared__ uint32_t s_wtot[U][2][4];
    // raw run: 16-byte phase + the run; packed run: 16-byte phase, the run
    // (PB/8 < VB bytes per value) and a guard slot
    __shared__ __align__(16) uint8_t s_vals[U * kTileNumel * VB + 32];
    // SQUARE from fp8 storage: every staged value converted once (k v^2, times
    // bf16(scale^2)) instead of in each of the 8 slots of every chunk; bf16
    // storage squares inline (its conversion is short and a second 16 KiB
    // buffer would halve the resident workgroups)
    constexpr bool STAGE = SQUARE && V_T != DT_BF16;
    constexpr int kSq = U * kTileNumel + 32;
    __shared__ __align__(16) uint16_t s_sq[STAGE ? kSq : 1];
    // plain bf16 values: each half (4 elements) of a chunk is built from a
    // 4-value window of the staged run at its first rank (three aligned dword
    // reads and two v_alignbyte) with two v_perm_b32, whose selectors come
    // from this table per mask nibble (element e takes window halfword
    // rank(e), bytes 2 rank(e) and 2 rank(e) + 1; 0x0c gives 0x00).  The
    // reads past a run's last value stay inside s_vals (its 32-byte slack)
    // and feed only cleared elements.
    constexpr bool PERM = V_T == DT_BF16 && !SQUARE && !HAS_SCALE;
    __shared__ uint2 s_sel4[PERM ? 16 : 1];
    const int tid = threadIdx.x;
    const uint32_t pid0 = blockIdx.x * U;
    const int ntiles = (int)min((uint32_t)U, a.num_tiles - pid0);
    const uint32_t t0 = (uint32_t)a.first_m_tile * a.grid_n + pid0;
    if constexpr (PERM) {
        if (tid < 16) {
            uint32_t sel[2] = {0x0c0c0c0cu, 0x0c0c0c0cu}, k = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if ((tid >> e) & 1) {
                    const uint32_t pair = (2u * k) | ((2u * k + 1u) << 8);
                    sel[e >> 1] = (sel[e >> 1] & ~(0xffffu << (16 * (e & 1)))) | (pair << (16 * (e & 1)));
                    k++;
                }
            }
            s_sel4[tid] = uint2{sel[0], sel[1]};      // ordered by gather_prepare's barriers
        }
    }

    uint32_t m[U][2], r0[U][2];
    // cursor and scale read with the front half's loads
    const int64_t vo = a.vals_offset ? *a.vals_offset : 0;
    float s = 1.0f;
    if constexpr (HAS_SCALE) s = *a.scale;
    const int bitbase = gather_prepare<VB, PB, U, NT>(a, t0, ntiles, m, r0, s_pref, s_wtot, s_vals, tid, vo);

    float s2b = 1.0f;
    if constexpr (HAS_SCALE) s2b = bf16_to_f32(f32_to_bf16(s * s));
    // an unset element: 0, or bf16(0 * bf16(scale^2)) (NaN for an infinite or NaN scale)
    const uint32_t zero_x = HAS_SCALE ? f32_to_bf16(0.0f * s2b) : 0u;
    if constexpr (STAGE) {
        // staged indices [0, count + 16) cover the run and its <= 15-element
        // phase (count clamped as the staging clamps it)
        const int64_t cnt = (int64_t)s_pref[ntiles] - (int64_t)s_pref[0];
        const int n_conv = (int)min<int64_t>(max<int64_t>(cnt, 0), (int64_t)ntiles * kTileNumel) + 16;
        for (int i = tid; i < n_conv; i += kThreads) {
            uint32_t x = relu2_square<V_T>(lds_val<V_T, PB>(s_vals, (uint32_t)i, bitbase), a.relu2_scale);
            if constexpr (HAS_SCALE) x = f32_to_bf16(bf16_to_f32(x) * s2b);
            s_sq[i] = (uint16_t)x;
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < U; j++) {
        if (j >= ntiles) break;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            typename Raw<OB>::T ov = {};
            uint32_t r = r0[j][h];
            const uint32_t mm = m[j][h];
            if constexpr (PERM) {
                const uint32_t* s32 = reinterpret_cast<const uint32_t*>(s_vals);
                uint32_t o[4];
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const uint32_t nib = (mm >> (4 * q)) & 15u;
                    uint32_t lo, hi;
                    if constexpr (PACKED) {
                        // the four 15-bit fields from stream bit bitbase + 15 r
                        // (a 64-bit window), widened to halfwords
                        const uint32_t bit = (uint32_t)bitbase + r * 15u;
                        const uint32_t d = bit >> 5, sh = bit & 31u;
                        const uint32_t w0 = s32[d], w1 = s32[d + 1], w2 = s32[d + 2];
                        const uint32_t x0 = __builtin_amdgcn_alignbit(w1, w0, sh);
                        const uint32_t x1 = __builtin_amdgcn_alignbit(w2, w1, sh);
                        lo = (x0 & 0x7fffu) | ((x0 << 1) & 0x7fff0000u);
                        hi = (((x0 >> 30) | (x1 << 2)) & 0x7fffu) | ((x1 << 3) & 0x7fff0000u);
                    } else {
                        const uint32_t d = r >> 1, sh = (r & 1u) * 2u;
                        const uint32_t w0 = s32[d], w1 = s32[d + 1], w2 = s32[d + 2];
                        lo = __builtin_amdgcn_alignbyte(w1, w0, sh);
                        hi = __builtin_amdgcn_alignbyte(w2, w1, sh);
                    }
                    const uint2 sel = s_sel4[nib];
                    o[2 * q] = __builtin_amdgcn_perm(hi, lo, sel.x);
                    o[2 * q + 1] = __builtin_amdgcn_perm(hi, lo, sel.y);
                    r += (uint32_t)__popc(nib);
                }
                ov = uint4{o[0], o[1], o[2], o[3]};
            }
#pragma unroll
            for (int e = 0; e < (PERM ? 0 : 8); e++) {
                uint32_t x;
                if constexpr (STAGE) {
                    x = ((mm >> e) & 1u) ? (uint32_t)s_sq[r] : zero_x;
                } else {
                    x = 0u;
                    if ((mm >> e) & 1u) {
                        x = lds_val<V_T, PB>(s_vals, r, bitbase);
                        if constexpr (SQUARE) x = relu2_square<V_T>(x, a.relu2_scale);
                    }
                    if constexpr (HAS_SCALE) x = f32_to_bf16(bf16_to_f32(x) * s2b);
                }
                r += (mm >> e) & 1u;
                set_elem<OB>(ov, e, x);
            }
            int64_t row, col0;
            chunk_pos(pid0 + j, a.grid_n, h * 256 + tid, row, col0);
            store_chunk<OB, VEC, NT>(a.out, a.rows, a.K, row, col0, ov);
        }
    }
}

// Plain decompress of fp8 storage (the stored e4m3fn / e5m2 bytes come back
// unchanged).  A workgroup takes a pair of horizontally adjacent tiles (tile
// columns 2c, 2c+1 of one tile row; the last tile of an odd row alone), so a
// 128-byte line of the output -- one row across both tiles -- is written by
// eight lanes of one store instruction: thread i owns, in pass h, row
// 32h + i/8 and the 16 elements of piece i%8 (pieces 0-3 in the first tile,
// 4-7 in the second), i.e. two bitmask bytes.  (A chunk-per-thread layout
// writes half lines, each finished later by another store.)  From raw storage
// the 16 outputs are built without a read per element: the thread's value
// window (16 bytes from its first rank) comes from five dword-aligned LDS
// reads and v_alignbyte, and each mask byte expands its 8 outputs with two
// v_perm_b32 whose selectors come from a 256-entry LDS table (selector byte
// 0x0c gives 0x00); the second byte's window starts popcount(first byte)
// values later.  Packed storage first widens the 16 7-bit fields from the
// thread's first rank (a 128-bit window of the staged stream) to bytes, then
// expands them the same way.  Needs K % 16 == 0 and
// a 16-byte aligned output.
template <int V_T, int NP, bool PACKED, bool NT>
__global__ __launch_bounds__(kThreads) void decompress_fp8_kernel(GatherArgs a, uint32_t groups_per_row)
{
    constexpr int PB = PACKED ? 7 : 0;
    constexpr int NTL = 2 * NP;             // tiles per workgroup: NP adjacent pairs of one tile row
    __shared__ uint32_t s_pref[NTL + 1];
    __shared__ uint32_t s_wtot[2][NTL][4];  // [pass][tile][wave]
    // the run, its <= 15-byte phase, and room for the last window's reads
    __shared__ __align__(16) uint8_t s_vals[NTL * kTileNumel + 48];
    __shared__ uint2 s_sel[256];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t tm = blockIdx.x / groups_per_row;
    const uint32_t tn0 = NTL * (blockIdx.x - tm * groups_per_row);
    const int ntiles = (int)min((uint32_t)NTL, a.grid_n - tn0);
    const uint32_t tb0 = tm * a.grid_n + tn0;                       // first tile, batch-relative
    const uint32_t t0 = (uint32_t)a.first_m_tile * a.grid_n + tb0;  // in the compressed tensor
    const int piece = tid & 7, jt = piece >> 2, pc = piece & 3;    // tile of the pair, piece in it

    const int64_t vo = a.vals_offset ? *a.vals_offset : 0;      // with the mask bytes
    uint32_t m[NP][2], ex[NP][2];
#pragma unroll
    for (int k = 0; k < NP; k++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int row = 32 * h + (tid >> 3), tile = 2 * k + jt;
            m[k][h] = tile < ntiles ? (uint32_t)*reinterpret_cast<const uint16_t*>(
                                          a.bitmask + (size_t)(t0 + tile) * kTileBytes + row * 8 + 2 * pc)
                                    : 0u;
        }
    if (tid <= ntiles) s_pref[tid] = a.prefix[t0 + tid];
    // the selector table while the mask bytes and prefixes are in flight
    {
        // selectors of mask byte tid: set element e takes window byte rank(e)
        uint32_t sel[2] = {0x0c0c0c0cu, 0x0c0c0c0cu};
        uint32_t rank = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            if ((tid >> e) & 1) {
                sel[e >> 2] = (sel[e >> 2] & ~(0xffu << (8 * (e & 3)))) | (rank << (8 * (e & 3)));
                rank++;
            }
        }
        s_sel[tid] = uint2{sel[0], sel[1]};
    }
#pragma unroll
    for (int k = 0; k < NP; k++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            // both tiles' counts in one DPP prefix sum, tile jt in bits
            // [16 jt, 16 jt + 16) (a wave's sum, <= 64 * 16, stays in its half)
            const uint32_t c = (uint32_t)__popc(m[k][h]);
            const uint32_t v = c << (16 * jt);
            const uint32_t incl = wave_incl_scan(v);
            ex[k][h] = ((incl - v) >> (16 * jt)) & 0xffffu;
            const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
            if (lane == 0) {
                s_wtot[h][2 * k][wave] = tot & 0xffffu;
                s_wtot[h][2 * k + 1][wave] = tot >> 16;
            }
        }
    __syncthreads();
    const uint32_t pb = s_pref[0];
    int p = 0, bitbase = 0;
    if constexpr (PACKED)
        bitbase = stage_run_packed<PB, NT>(a, vo + pb, vo + s_pref[ntiles], (int64_t)ntiles * kTileNumel, s_vals, tid);
    else
        p = stage_run<1, NT>(a, vo + pb, vo + s_pref[ntiles], (int64_t)ntiles * kTileNumel, s_vals, tid);
    // first value of this thread's piece: tile start + earlier pass + earlier
    // waves of this pass + the in-wave rank
    uint32_t r0[NP][2];
#pragma unroll
    for (int k = 0; k < NP; k++) {
        const int tile = 2 * k + jt;
        const uint32_t tstart = tile < ntiles ? min(s_pref[tile] - pb, (uint32_t)(tile * kTileNumel)) : 0u;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            uint32_t below = 0;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                if (h == 1) below += s_wtot[0][tile][w];
                if (w < wave) below += s_wtot[h][tile][w];
            }
            r0[k][h] = (uint32_t)p + tstart + below + ex[k][h];
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < NP; k++)
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t mm = m[k][h];
        uint4 o;
        {
            const uint32_t r = r0[k][h];
            uint32_t w0, w1, w2, w3;            // the 16 values from rank r, one byte each
            if constexpr (PACKED) {
                // the 16 7-bit fields from stream bit bitbase + 7 r: a 128-bit
                // window (five aligned dword reads, v_alignbit), each field
                // widened to its byte (a stored e4m3fn code: sign bit 0)
                const uint32_t bit = (uint32_t)bitbase + r * (uint32_t)PB;
                const uint32_t* sv = reinterpret_cast<const uint32_t*>(s_vals) + (bit >> 5);
                const uint32_t sh = bit & 31u;
                const uint32_t u0 = sv[0], u1 = sv[1], u2 = sv[2], u3 = sv[3], u4 = sv[4];
                const uint32_t x[5] = {__builtin_amdgcn_alignbit(u1, u0, sh), __builtin_amdgcn_alignbit(u2, u1, sh),
                                       __builtin_amdgcn_alignbit(u3, u2, sh), __builtin_amdgcn_alignbit(u4, u3, sh),
                                       0u};
                uint32_t wb[4] = {0u, 0u, 0u, 0u};
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    constexpr int kPB = PB > 0 ? PB : 1;
                    const int lo = j * kPB, q = lo >> 5, off = lo & 31;
                    uint32_t f = x[q] >> off;
                    if (off + kPB > 32) f |= x[q + 1] << (32 - off);
                    wb[j >> 2] |= (f & ((1u << kPB) - 1u)) << (8 * (j & 3));
                }
                w0 = wb[0], w1 = wb[1], w2 = wb[2], w3 = wb[3];
            } else {
                const uint32_t* sv = reinterpret_cast<const uint32_t*>(s_vals) + (r >> 2);
                const uint32_t sh = r & 3u;
                const uint32_t d0 = sv[0], d1 = sv[1], d2 = sv[2], d3 = sv[3], d4 = sv[4];
                w0 = __builtin_amdgcn_alignbyte(d1, d0, sh);
                w1 = __builtin_amdgcn_alignbyte(d2, d1, sh);
                w2 = __builtin_amdgcn_alignbyte(d3, d2, sh);
                w3 = __builtin_amdgcn_alignbyte(d4, d3, sh);
            }
            const uint32_t m0 = mm & 0xffu, m1 = mm >> 8;
            const uint2 sa = s_sel[m0], sb = s_sel[m1];
            // window of the second byte: bytes c0 .. c0+7, c0 = popcount(m0) <= 8
            const uint32_t c0 = (uint32_t)__popc(m0), q = c0 >> 2, t = c0 & 3u;
            const uint32_t x0 = q == 0 ? w0 : (q == 1 ? w1 : w2);
            const uint32_t x1 = q == 0 ? w1 : (q == 1 ? w2 : w3);
            const uint32_t x2 = q == 0 ? w2 : w3;      // q == 2 has t == 0: unused
            const uint32_t v0 = __builtin_amdgcn_alignbyte(x1, x0, t);
            const uint32_t v1 = __builtin_amdgcn_alignbyte(x2, x1, t);
            o = uint4{__builtin_amdgcn_perm(w1, w0, sa.x), __builtin_amdgcn_perm(w1, w0, sa.y),
                      __builtin_amdgcn_perm(v1, v0, sb.x), __builtin_amdgcn_perm(v1, v0, sb.y)};
        }
        const int tile = 2 * k + jt;
        const int64_t row = (int64_t)tm * 64 + 32 * h + (tid >> 3);
        const int64_t col0 = (int64_t)(tn0 + tile) * 64 + 16 * pc;
        if (tile < ntiles && row < a.rows && col0 < a.K) st16<NT>(a.out + row * a.K + col0, o);
    }
}

// grad = bit ? bf16(grad * (2k * r)) : 0, then optionally grad = bf16(grad * bf16(scale))
// NT: nontemporal gradient loads / stores and staging loads.
template <int V_T, bool HAS_SCALE, bool VEC, int U, bool PACKED, bool NT>
__global__ __launch_bounds__(kThreads) void relu2_grad_kernel(GatherArgs a)
{
    constexpr int VB = V_T == DT_BF16 ? 2 : 1;
    constexpr int PB = PACKED ? (V_T == DT_BF16 ? 15 : 7) : 0;
    __shared__ uint32_t s_pref[U + 1];
    __shared__ uint32_t s_wtot[U][2][4];
    __shared__ __align__(16) uint8_t s_vals[U * kTileNumel * VB + 32];
    // fp8 or packed storage: each staged value widened once to its bf16 bits
    // (exact: every e4m3fn / e5m2 value is a bf16 value)
    constexpr bool WIDEN = V_T != DT_BF16 || PACKED;
    constexpr int kRv = U * kTileNumel + 32;
    __shared__ __align__(16) uint16_t s_rv[WIDEN ? kRv : 1];
    const int tid = threadIdx.x;
    const uint32_t t0 = blockIdx.x * U;
    const int ntiles = (int)min((uint32_t)U, a.num_tiles - t0);

    // mask bytes first: a chunk with no bit set is written without reading
    // its gradient (at 90% zeros 43% of the chunks); cursor and scale with them.
    // Memory still moves the 128-byte line of a tile row whenever any of its
    // eight chunks is read, so the skip saves no HBM traffic below whole
    // rows, but it keeps the unused chunks out of the CU: reading every chunk
    // of a live row measured 55.7 against 51.7 us at the configs[3] shape.
    const int64_t vo = a.vals_offset ? *a.vals_offset : 0;
    float sc = 1.0f;
    if constexpr (HAS_SCALE) sc = *a.scale;
    uint32_t m[U][2], r0[U][2];
#pragma unroll
    for (int j = 0; j < U; j++)
#pragma unroll
        for (int h = 0; h < 2; h++)
            m[j][h] = j < ntiles ? a.bitmask[(size_t)(t0 + j) * kTileBytes + h * 256 + tid] : 0u;
    const uint32_t pf = tid <= ntiles ? a.prefix[t0 + tid] : 0u;
    uint4 g[U][2];
#pragma unroll
    for (int j = 0; j < U; j++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            g[j][h] = uint4{0u, 0u, 0u, 0u};
            if (m[j][h] != 0u) {
                int64_t row, col0;
                chunk_pos(t0 + j, a.grid_n, h * 256 + tid, row, col0);
                g[j][h] = load_chunk<2, VEC, NT>(a.out, a.rows, a.K, row, col0);
            }
        }
    const int bitbase = gather_prepare<VB, PB, U, NT, true>(a, t0, ntiles, m, r0, s_pref, s_wtot, s_vals, tid, vo, pf);

    if constexpr (WIDEN) {
        // staged indices [0, count + 16) cover the run and its <= 15-element phase
        const int64_t cnt = (int64_t)s_pref[ntiles] - (int64_t)s_pref[0];
        const int n_conv = (int)min<int64_t>(max<int64_t>(cnt, 0), (int64_t)ntiles * kTileNumel) + 16;
        for (int i = tid; i < n_conv; i += kThreads)
            s_rv[i] = (uint16_t)(__float_as_uint(val_f32<V_T>(lds_val<V_T, PB>(s_vals, (uint32_t)i, bitbase))) >> 16);
        __syncthreads();
    }
    float sb = 1.0f;
    if constexpr (HAS_SCALE) sb = bf16_to_f32(f32_to_bf16(sc));
    const uint32_t zero_x = HAS_SCALE ? f32_to_bf16(0.0f * sb) : 0u;
    const float k2 = 2.0f * a.relu2_scale;
#pragma unroll
    for (int j = 0; j < U; j++) {
        if (j >= ntiles) break;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            uint4 ov = {0u, 0u, 0u, 0u};
            uint32_t r = r0[j][h];
            const uint32_t mm = m[j][h];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                uint32_t x = zero_x;
                if ((mm >> e) & 1u) {
                    float rv;
                    if constexpr (WIDEN) rv = bf16_to_f32(s_rv[r]);
                    else rv = val_f32<V_T>(lds_val<V_T, PB>(s_vals, r, bitbase));
                    x = f32_to_bf16(bf16_to_f32(get16(g[j][h], e)) * (k2 * rv));
                    if constexpr (HAS_SCALE) x = f32_to_bf16(bf16_to_f32(x) * sb);
                }
                r += (mm >> e) & 1u;
                set_elem<2>(ov, e, x);
            }
            int64_t row, col0;
            chunk_pos(t0 + j, a.grid_n, h * 256 + tid, row, col0);
            store_chunk<2, VEC, NT>(a.out, a.rows, a.K, row, col0, ov);
        }
    }
}

// ===========================================================================
// ReLU mask gradient (in place)
// ===========================================================================
// NT: nontemporal gradient loads / stores.
template <bool VEC, int U, bool NT>
__global__ __launch_bounds__(kThreads) void relu_grad_kernel(uint8_t* grad, int64_t M, int64_t N,
                                                             uint32_t grid_n, uint32_t T,
                                                             const uint8_t* bitmask)
{
    const int tid = threadIdx.x;
    const uint32_t t0 = blockIdx.x * U;
    const int ntiles = (int)min((uint32_t)U, T - t0);
    uint32_t m[U][2];
#pragma unroll
    for (int j = 0; j < U; j++)
#pragma unroll
        for (int h = 0; h < 2; h++)
            m[j][h] = j < ntiles ? bitmask[(size_t)(t0 + j) * kTileBytes + h * 256 + tid] : 0xffu;
    uint4 g[U][2];
#pragma unroll
    for (int j = 0; j < U; j++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            g[j][h] = uint4{0u, 0u, 0u, 0u};
            if (m[j][h] != 0u && m[j][h] != 0xffu) {
                int64_t row, col0;
                chunk_pos(t0 + j, grid_n, h * 256 + tid, row, col0);
                g[j][h] = load_chunk<2, VEC, NT>(grad, M, N, row, col0);
            }
        }
#pragma unroll
    for (int j = 0; j < U; j++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t mm = m[j][h];
            if (mm == 0xffu) continue;    // all kept: nothing to write
            uint4 v = g[j][h];
            // byte mask -> 16-bit lane masks (all-zero byte stores zeros)
            uint32_t k0 = ((mm & 1u) ? 0xffffu : 0u) | ((mm & 2u) ? 0xffff0000u : 0u);
            uint32_t k1 = ((mm & 4u) ? 0xffffu : 0u) | ((mm & 8u) ? 0xffff0000u : 0u);
            uint32_t k2 = ((mm & 16u) ? 0xffffu : 0u) | ((mm & 32u) ? 0xffff0000u : 0u);
            uint32_t k3 = ((mm & 64u) ? 0xffffu : 0u) | ((mm & 128u) ? 0xffff0000u : 0u);
            v.x &= k0; v.y &= k1; v.z &= k2; v.w &= k3;
            int64_t row, col0;
            chunk_pos(t0 + j, grid_n, h * 256 + tid, row, col0);
            store_chunk<2, VEC, NT>(grad, M, N, row, col0, v);
        }
}

// Empty input (T = 0): prefix = [0]; the cursor outputs take the input
// cursor (or 0) unchanged.
__global__ void empty_compress_kernel(uint32_t* prefix, const int64_t* offset_in, int64_t* offset_out,
                                      int64_t* start_out)
{
    if (threadIdx.x != 0) return;
    prefix[0] = 0u;
    const int64_t c = offset_in ? *offset_in : 0;
    if (offset_out) *offset_out = c;
    if (start_out) *start_out = c;
}

// ===========================================================================
// host launchers
// ===========================================================================
// compress unit: tiles per workgroup and workgroup size
#ifndef BS_GATHER_U
#define BS_GATHER_U 2
#endif
constexpr int kGatherU = BS_GATHER_U;
// adjacent tile pairs per workgroup of the plain fp8 decompress
#ifndef BS_FP8_PAIRS
#define BS_FP8_PAIRS 2
#endif
constexpr int kFp8Pairs = BS_FP8_PAIRS;

constexpr int kMaskU = 4;

static inline bool aligned16(const void* p) { return (((uintptr_t)p) & 15u) == 0; }
static inline bool aligned8(const void* p) { return (((uintptr_t)p) & 7u) == 0; }


#ifndef BS_STREAM_U
#define BS_STREAM_U 8
#endif
constexpr int kStreamU = BS_STREAM_U;

// The streaming compress addresses a lane's chunk inside its tile with a
// 32-bit byte offset below 8 rows of N elements of `eb` bytes.
static bool vec_rows_fit(int64_t N, int eb) { return 8 * N * (int64_t)eb < (int64_t(1) << 32); }

template <int IN_T, bool QUANT, int MODE, bool PACKED>
static hipError_t launch_compress_mode(const CompressArgs& a, bool vec, bool nt, hipStream_t st, bool rsq = false)
{
    const uint32_t units = (a.tend - a.tile0 + kStreamU - 1) / kStreamU;
    // the streaming hint is built for the fused pass over a vector-loadable input
    constexpr bool kHasNt = MODE == MODE_FUSED;
    if constexpr (IN_T == DT_BF16 && MODE == MODE_FUSED && !PACKED) {
        if (rsq) {
            if (vec && nt)
                launch_timed(0, compress_stream_kernel<IN_T, QUANT, true, MODE, kStreamU, PACKED, true, true>,
                             dim3(units), dim3(64 * kStreamU), 0, st, a);
            else if (vec)
                launch_timed(0, compress_stream_kernel<IN_T, QUANT, true, MODE, kStreamU, PACKED, false, true>,
                             dim3(units), dim3(64 * kStreamU), 0, st, a);
            else
                launch_timed(0, compress_stream_kernel<IN_T, QUANT, false, MODE, kStreamU, PACKED, false, true>,
                             dim3(units), dim3(64 * kStreamU), 0, st, a);
            return hipGetLastError();
        }
    }
    if (vec && nt && kHasNt)
        launch_timed(0, compress_stream_kernel<IN_T, QUANT, true, MODE, kStreamU, PACKED, kHasNt>, dim3(units),
                     dim3(64 * kStreamU), 0, st, a);
    else if (vec)
        launch_timed(0, compress_stream_kernel<IN_T, QUANT, true, MODE, kStreamU, PACKED, false>, dim3(units),
                     dim3(64 * kStreamU), 0, st, a);
    else
        launch_timed(0, compress_stream_kernel<IN_T, QUANT, false, MODE, kStreamU, PACKED, false>, dim3(units),
                     dim3(64 * kStreamU), 0, st, a);
    return hipGetLastError();
}

template <int MODE, bool PACKED = false>
static hipError_t launch_compress(const CompressArgs& a, int in_dtype, bool quant, bool vec, bool nt,
                                  hipStream_t st, bool rsq = false)
{
    if constexpr (MODE != MODE_VALS) {
        if (quant) return launch_compress_mode<DT_BF16, true, MODE, PACKED>(a, vec, nt, st, rsq);
    }
    switch (in_dtype) {
    case DT_BF16: return launch_compress_mode<DT_BF16, false, MODE, PACKED>(a, vec, nt, st, rsq);
    case DT_E4M3FN: return launch_compress_mode<DT_E4M3FN, false, MODE, PACKED>(a, vec, nt, st);
    default: return launch_compress_mode<DT_E5M2, false, MODE, PACKED>(a, vec, nt, st);
    }
}

}  // namespace bs

using namespace bs;

// The quantizer's code table sits after the status words (256-byte aligned).
static int64_t ws_qtab_offset(int64_t T) { return (kWsHeaderBytes + 8 * (T + 2) + 255) / 256 * 256; }

extern "C" int64_t bs_compress_workspace_bytes(int64_t M, int64_t N)
{
    if (M < 0 || N < 0) return -1;
    int64_t T = ((M + 63) / 64) * ((N + 63) / 64);
    // status words: one per tile covers the units and the unit groups of the
    // streaming kernel (T/8 + T/512 words) and the units of the others; then
    // the quantizer's code table
    return ws_qtab_offset(T) + kQtabBytes;
}

extern "C" const uint64_t* bs_workspace_amax_slot(const void* ws, int64_t)
{
    return reinterpret_cast<const uint64_t*>(reinterpret_cast<const uint8_t*>(ws) + kWsAmaxOffset);
}

extern "C" const uint32_t* bs_workspace_fallback_counter(const void* ws, int64_t)
{
    return reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(ws) + kWsFallbackOffset);
}

static int check_dense(const void* dense, int dtype, int64_t M, int64_t N, const char* what,
                       uint64_t max_elems = kMaxElemsUntested)
{
    if (dtype < 0 || dtype > 2) return set_error(BS_ERR_INVALID, "%s: unknown dtype code %d", what, dtype);
    if (M < 0 || N < 0) return set_error(BS_ERR_INVALID, "%s: negative shape", what);
    if ((M > 0 && N > 0) && dense == nullptr) return set_error(BS_ERR_INVALID, "%s: null input", what);
    if ((uint64_t)M * (uint64_t)N >= max_elems)
        return set_error(BS_ERR_INVALID, "%s: M*N must be < 2^%d on this path", what,
                         max_elems == kMaxElems ? 32 : 31);
    int elem = dtype == DT_BF16 ? 2 : 1;
    if (((uintptr_t)dense) % elem)
        return set_error(BS_ERR_INVALID, "%s: input not aligned to its element size", what);
    return BS_OK;
}

static int compress_impl(const void* dense, int in_dtype, int64_t M, int64_t N, int quantize,
                         const uint64_t* amax_slot, uint32_t amax_epoch, float* scale_out,
                         void* dense_q_out, uint8_t* bitmask, uint32_t* prefix, void* vals,
                         int64_t vals_capacity, const int64_t* vals_offset_in, int align8,
                         int64_t* vals_offset_out, int64_t* vals_start_out, int write_vals,
                         int32_t* err_flags, void* workspace, int64_t workspace_bytes,
                         uint32_t epoch, void* stream, bool relu, void* relu_out, bool packed = false,
                         bool check_capture = true, const std::function<int()>& before_launch = nullptr,
                         bool relu_sq = false, float relu_k = 1.0f)
{
    if (relu_sq) {
        // the ReLU^2 write-back: bf16 pre-activation, values into a buffer
        if (!relu || relu_out == nullptr || in_dtype != DT_BF16 || packed || !write_vals)
            return set_error(BS_ERR_INVALID, "bs_compress_relu2: needs a bf16 pre-activation, relu_out and "
                                             "write_vals = 1");
        if (!std::isfinite(relu_k)) return set_error(BS_ERR_INVALID, "bs_compress_relu2: k must be finite");
    }
    if (packed) {
        // vals is the packed stream and vals_capacity its size in bytes
        if (!write_vals) return set_error(BS_ERR_INVALID, "bs_compress_packed: write_vals must be 1");
        if (((uintptr_t)vals) & 3u)
            return set_error(BS_ERR_INVALID, "bs_compress_packed: stream not 4-byte aligned");
        if (M > 0 && N > 0 && vals_capacity > 0 && vals == nullptr)
            return set_error(BS_ERR_INVALID, "bs_compress_packed: null stream");
        if (M == 0 || N == 0)
            return set_error(BS_ERR_INVALID, "bs_compress_packed: empty input (the cursor is not advanced here)");
    }
    if (relu_out != nullptr && !relu)
        return set_error(BS_ERR_INVALID, "bs_compress: relu_out without relu");
    if (relu_out != nullptr && (((uintptr_t)relu_out) % (in_dtype == DT_BF16 ? 2 : 1)))
        return set_error(BS_ERR_INVALID, "bs_compress_relu: relu_out misaligned");
    // raw bf16 compress (values into a buffer, or the count pass of the
    // standalone path) runs past 2^31 elements on the GPU; the quantizing,
    // fp8-input and packed variants stop at 2^31
    const bool big_ok = in_dtype == DT_BF16 && !quantize && !packed;
    if (int rc = check_dense(dense, in_dtype, M, N, "bs_compress", big_ok ? kMaxElems : kMaxElemsUntested))
        return rc;
    if (quantize && in_dtype != DT_BF16)
        return set_error(BS_ERR_INVALID, "bs_compress: quantize needs bf16 input");
    if (quantize && amax_slot == nullptr)
        return set_error(BS_ERR_INVALID, "bs_compress: quantize needs the amax slot");
    const int64_t T = ((M + 63) / 64) * ((N + 63) / 64);
    if (prefix == nullptr) return set_error(BS_ERR_INVALID, "bs_compress: null prefix");
    if (T > 0 && bitmask == nullptr) return set_error(BS_ERR_INVALID, "bs_compress: null bitmask");
    if (write_vals && vals_capacity > 0 && vals == nullptr)
        return set_error(BS_ERR_INVALID, "bs_compress: null vals");
    if (vals_capacity < 0) return set_error(BS_ERR_INVALID, "bs_compress: negative capacity");
    if (vals_offset_out != nullptr && vals_offset_out == vals_offset_in)
        return set_error(BS_ERR_INVALID, "bs_compress: vals_offset_out aliases vals_offset_in");
    if (epoch == 0 || epoch >= (1u << 30))
        return set_error(BS_ERR_INVALID, "bs_compress: epoch must be in [1, 2^30)");
    if (check_capture) {
        if (int rc = refuse_capture((hipStream_t)stream, "bs_compress")) return rc;
    }
    if (workspace == nullptr || workspace_bytes < bs_compress_workspace_bytes(M, N))
        return set_error(BS_ERR_INVALID, "bs_compress: workspace too small (%lld < %lld bytes)",
                         (long long)workspace_bytes, (long long)bs_compress_workspace_bytes(M, N));
    const int outb = (in_dtype == DT_BF16 && !quantize) ? 2 : 1;
    if (write_vals && !packed && ((uintptr_t)vals) % outb)
        return set_error(BS_ERR_INVALID, "bs_compress: vals not aligned to its element size");
    hipStream_t st = (hipStream_t)stream;
    // every argument is checked: launches may start (the caller's own first)
    if (before_launch) {
        if (int rc = before_launch()) return rc;
    }
    if (T == 0) {
        // empty input: prefix = [0], cursor unchanged (one small kernel, so the
        // no-allocation variant stays capturable)
        hipLaunchKernelGGL(empty_compress_kernel, dim3(1), dim3(64), 0, st, prefix, vals_offset_in,
                           vals_offset_out, vals_start_out);
        hipError_t e = hipGetLastError();
        return e == hipSuccess ? BS_OK : set_error(BS_ERR_HIP, "bs_compress: %s", hipGetErrorString(e));
    }
    CompressArgs a{};
    a.dense = (const uint8_t*)dense;
    a.M = M;
    a.N = N;
    a.grid_n = (uint32_t)((N + 63) / 64);
    a.T = (uint32_t)T;
    a.amax_slot = amax_slot;
    a.amax_epoch = amax_epoch;
    a.scale_out = scale_out;
    a.dense_q_out = (uint8_t*)dense_q_out;
    a.bitmask = bitmask;
    a.prefix = prefix;
    a.vals = (uint8_t*)vals;
    a.vals_capacity = packed ? vals_capacity / 4 : vals_capacity;   // packed: stream dwords
    a.offset_in = vals_offset_in;
    a.align8 = packed ? 1 : align8;
    a.offset_out = vals_offset_out;
    a.start_out = vals_start_out;
    a.tile0 = 0;
    a.tend = (uint32_t)T;
    a.relu = relu ? 1 : 0;
    a.relu_out = (uint8_t*)relu_out;
    a.relu_k = relu_k;
    a.status = reinterpret_cast<uint64_t*>((uint8_t*)workspace + kWsHeaderBytes);
    a.epoch = epoch;
    a.err = err_flags;
    a.fallbacks = reinterpret_cast<uint32_t*>((uint8_t*)workspace + kWsFallbackOffset);
    a.patience = kLookbackPatienceTicks;
    if (const char* ev = getenv("BITSPARSE_LOOKBACK_PATIENCE")) {
        char* end = nullptr;
        const unsigned long long v = strtoull(ev, &end, 10);
        if (end != ev) a.patience = (uint64_t)v;
    }
    a.gstat = a.status + (T + kStreamU - 1) / kStreamU;
    if (quantize) {
        // the code table of this call's scale, built after the amax it reads
        uint8_t* qtab = (uint8_t*)workspace + ws_qtab_offset(T);
        hipLaunchKernelGGL(qtab_build_kernel, dim3((kQtabEntries + 255) / 256), dim3(256), 0, st, amax_slot, amax_epoch,
                           qtab);
        a.qtab = qtab;
    }
    const int inb = in_dtype == DT_BF16 ? 2 : 1;
    bool vec = (N % 8 == 0) && (((uintptr_t)dense) % (8 * inb) == 0) && vec_rows_fit(N, inb) &&
               (dense_q_out == nullptr || aligned8(dense_q_out)) &&
               (relu_out == nullptr || ((uintptr_t)relu_out) % (8 * inb) == 0);
    const bool nt = use_nontemporal(M * N * inb);
    hipError_t e = packed     ? launch_compress<MODE_FUSED, true>(a, in_dtype, quantize != 0, vec, nt, st)
                 : write_vals ? launch_compress<MODE_FUSED>(a, in_dtype, quantize != 0, vec, nt, st, relu_sq)
                              : launch_compress<MODE_COUNT>(a, in_dtype, quantize != 0, vec, nt, st);
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_compress launch: %s", hipGetErrorString(e));
    return BS_OK;
}

extern "C" int bs_compress(const void* dense, int in_dtype, int64_t M, int64_t N, int quantize,
                           const uint64_t* amax_slot, uint32_t amax_epoch, float* scale_out,
                           void* dense_q_out, uint8_t* bitmask, uint32_t* prefix, void* vals,
                           int64_t vals_capacity, const int64_t* vals_offset_in, int align8,
                           int64_t* vals_offset_out, int64_t* vals_start_out, int write_vals,
                           int32_t* err_flags, void* workspace, int64_t workspace_bytes,
                           uint32_t epoch, void* stream)
{
    clear_error();
    return compress_impl(dense, in_dtype, M, N, quantize, amax_slot, amax_epoch, scale_out, dense_q_out,
                         bitmask, prefix, vals, vals_capacity, vals_offset_in, align8, vals_offset_out,
                         vals_start_out, write_vals, err_flags, workspace, workspace_bytes, epoch, stream,
                         false, nullptr);
}

extern "C" int bs_compress_relu(const void* preact, int in_dtype, int64_t M, int64_t N, int quantize,
                                const uint64_t* amax_slot, uint32_t amax_epoch, float* scale_out,
                                void* dense_q_out, uint8_t* bitmask, uint32_t* prefix, void* vals,
                                int64_t vals_capacity, const int64_t* vals_offset_in, int align8,
                                int64_t* vals_offset_out, int64_t* vals_start_out, int write_vals,
                                int32_t* err_flags, void* workspace, int64_t workspace_bytes,
                                uint32_t epoch, void* relu_out, void* stream)
{
    clear_error();
    return compress_impl(preact, in_dtype, M, N, quantize, amax_slot, amax_epoch, scale_out, dense_q_out,
                         bitmask, prefix, vals, vals_capacity, vals_offset_in, align8, vals_offset_out,
                         vals_start_out, write_vals, err_flags, workspace, workspace_bytes, epoch, stream,
                         true, relu_out);
}

extern "C" int bs_compress_relu2(const void* preact, int quantize, int64_t M, int64_t N,
                                 const uint64_t* amax_slot, uint32_t amax_epoch, float* scale_out,
                                 void* dense_q_out, uint8_t* bitmask, uint32_t* prefix, void* vals,
                                 int64_t vals_capacity, const int64_t* vals_offset_in, int64_t* vals_offset_out,
                                 int32_t* err_flags, void* workspace, int64_t workspace_bytes, uint32_t epoch,
                                 void* relu_out, float k, void* stream)
{
    clear_error();
    return compress_impl(preact, DT_BF16, M, N, quantize, amax_slot, amax_epoch, scale_out, dense_q_out,
                         bitmask, prefix, vals, vals_capacity, vals_offset_in, 0, vals_offset_out, nullptr, 1,
                         err_flags, workspace, workspace_bytes, epoch, stream, true, relu_out, false, true, nullptr,
                         true, k);
}

extern "C" int bs_compress_packed(const void* dense, int in_dtype, int64_t M, int64_t N, int quantize,
                                  const uint64_t* amax_slot, uint32_t amax_epoch, float* scale_out,
                                  void* dense_q_out, uint8_t* bitmask, uint32_t* prefix,
                                  void* stream_bytes, int64_t stream_nbytes, const int64_t* vals_offset_in,
                                  int64_t* vals_offset_out, int64_t* vals_start_out, int32_t* err_flags,
                                  void* workspace, int64_t workspace_bytes, uint32_t epoch, int relu,
                                  void* relu_out, void* stream)
{
    clear_error();
    return compress_impl(dense, in_dtype, M, N, quantize, amax_slot, amax_epoch, scale_out, dense_q_out,
                         bitmask, prefix, stream_bytes, stream_nbytes, vals_offset_in, 1, vals_offset_out,
                         vals_start_out, 1, err_flags, workspace, workspace_bytes, epoch, stream,
                         relu != 0, relu_out, true);
}

extern "C" int bs_compact_vals(const void* dense, int in_dtype, int64_t M, int64_t N,
                               const uint8_t* bitmask, const uint32_t* prefix, void* vals,
                               int64_t vals_capacity, const int64_t* vals_offset, int64_t first_tile,
                               int64_t num_tiles, int32_t* err_flags, void* stream)
{
    clear_error();
    // the bf16 values pass of the standalone path runs past 2^31 elements on the GPU
    if (int rc = check_dense(dense, in_dtype, M, N, "bs_compact_vals",
                             in_dtype == DT_BF16 ? kMaxElems : kMaxElemsUntested))
        return rc;
    const int64_t T = ((M + 63) / 64) * ((N + 63) / 64);
    if (first_tile < 0 || num_tiles < 0 || first_tile + num_tiles > T)
        return set_error(BS_ERR_INVALID, "bs_compact_vals: tile range [%lld, %lld) outside [0, %lld)",
                         (long long)first_tile, (long long)(first_tile + num_tiles), (long long)T);
    if (num_tiles == 0) return BS_OK;
    if (bitmask == nullptr || prefix == nullptr)
        return set_error(BS_ERR_INVALID, "bs_compact_vals: null bitmask/prefix");
    if (vals_capacity < 0) return set_error(BS_ERR_INVALID, "bs_compact_vals: negative capacity");
    if (vals_capacity > 0 && vals == nullptr) return set_error(BS_ERR_INVALID, "bs_compact_vals: null vals");
    const int eb = in_dtype == DT_BF16 ? 2 : 1;
    if (((uintptr_t)vals) % eb) return set_error(BS_ERR_INVALID, "bs_compact_vals: vals misaligned");
    CompressArgs a{};
    a.dense = (const uint8_t*)dense;
    a.M = M;
    a.N = N;
    a.grid_n = (uint32_t)((N + 63) / 64);
    a.T = (uint32_t)T;
    a.bitmask = (uint8_t*)bitmask;
    a.prefix = (uint32_t*)prefix;
    a.vals = (uint8_t*)vals;
    a.vals_capacity = vals_capacity;
    a.offset_in = vals_offset;
    a.tile0 = (uint32_t)first_tile;
    a.tend = (uint32_t)(first_tile + num_tiles);
    a.err = err_flags;
    a.patience = kLookbackPatienceTicks;       // no look-back in this mode
    bool vec = (N % 8 == 0) && (((uintptr_t)dense) % (8 * eb) == 0) && vec_rows_fit(N, eb);
    hipError_t e = launch_compress<MODE_VALS>(a, in_dtype, false, vec, false, (hipStream_t)stream);
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_compact_vals launch: %s", hipGetErrorString(e));
    return BS_OK;
}

extern "C" int bs_tile_pack(const void* dense, int in_dtype, int64_t M, int64_t N, int32_t* tile_counts,
                            uint8_t* bitmask, void* stream)
{
    clear_error();
    if (int rc = check_dense(dense, in_dtype, M, N, "bs_tile_pack")) return rc;
    const int64_t T = ((M + 63) / 64) * ((N + 63) / 64);
    if (T == 0) return BS_OK;
    if (tile_counts == nullptr || bitmask == nullptr)
        return set_error(BS_ERR_INVALID, "bs_tile_pack: null output");
    const int eb = in_dtype == DT_BF16 ? 2 : 1;
    bool vec = (N % 8 == 0) && (((uintptr_t)dense) % (8 * eb) == 0);
    uint32_t gn = (uint32_t)((N + 63) / 64);
    hipStream_t st = (hipStream_t)stream;
    const uint8_t* d = (const uint8_t*)dense;
#define BS_TP(DT, V) hipLaunchKernelGGL((tile_pack_kernel<DT, V>), dim3((uint32_t)T), dim3(kThreads), 0, st, \
                                        d, M, N, gn, tile_counts, bitmask)
    switch (in_dtype) {
    case DT_BF16: if (vec) BS_TP(DT_BF16, true); else BS_TP(DT_BF16, false); break;
    case DT_E4M3FN: if (vec) BS_TP(DT_E4M3FN, true); else BS_TP(DT_E4M3FN, false); break;
    default: if (vec) BS_TP(DT_E5M2, true); else BS_TP(DT_E5M2, false); break;
    }
#undef BS_TP
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_tile_pack launch: %s", hipGetErrorString(e));
    return BS_OK;
}

extern "C" int bs_prefix_from_counts(const int32_t* tile_counts, int64_t T, uint32_t* prefix, void* stream)
{
    clear_error();
    if (T < 0) return set_error(BS_ERR_INVALID, "bs_prefix_from_counts: negative T");
    if (prefix == nullptr || (T > 0 && tile_counts == nullptr))
        return set_error(BS_ERR_INVALID, "bs_prefix_from_counts: null pointer");
    hipLaunchKernelGGL(prefix_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, tile_counts, T, prefix);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_prefix_from_counts launch: %s", hipGetErrorString(e));
    return BS_OK;
}

template <int V_T, bool SQ, bool SC, bool PK>
static void launch_decompress_t(const GatherArgs& a, bool vec, bool nt, hipStream_t st)
{
    const uint32_t blocks = (a.num_tiles + kGatherU - 1) / kGatherU;
    if constexpr (V_T != DT_BF16 && !SQ) {
        // fp8 bytes out: 16-byte stores when rows are whole 16-byte pieces
        if (a.K % 16 == 0 && aligned16(a.out) && a.num_tiles % a.grid_n == 0) {
            // one workgroup per kFp8Pairs adjacent tile pairs of a tile row
            const uint32_t gpr = (a.grid_n + 2 * kFp8Pairs - 1) / (2 * kFp8Pairs);
            const uint32_t b8 = (a.num_tiles / a.grid_n) * gpr;
            if (nt)
                launch_timed(1, decompress_fp8_kernel<V_T, kFp8Pairs, PK, true>, dim3(b8), dim3(kThreads), 0, st, a, gpr);
            else
                launch_timed(1, decompress_fp8_kernel<V_T, kFp8Pairs, PK, false>, dim3(b8), dim3(kThreads), 0, st, a, gpr);
            return;
        }
    }
    if (vec && nt)
        launch_timed(1, decompress_kernel<V_T, SQ, SC, true, kGatherU, PK, true>, dim3(blocks), dim3(kThreads), 0, st, a);
    else if (vec)
        launch_timed(1, decompress_kernel<V_T, SQ, SC, true, kGatherU, PK, false>, dim3(blocks), dim3(kThreads), 0, st, a);
    else
        launch_timed(1, decompress_kernel<V_T, SQ, SC, false, kGatherU, PK, false>, dim3(blocks), dim3(kThreads), 0, st, a);
}

template <int V_T, bool PK>
static void launch_decompress_v(const GatherArgs& a, bool sq, bool sc, bool vec, bool nt, hipStream_t st)
{
    if (!sq) launch_decompress_t<V_T, false, false, PK>(a, vec, nt, st);
    else if (!sc) launch_decompress_t<V_T, true, false, PK>(a, vec, nt, st);
    else launch_decompress_t<V_T, true, true, PK>(a, vec, nt, st);
}

static int check_gather(const void* vals, int vals_dtype, int64_t vals_numel, const uint8_t* bitmask,
                        const uint32_t* prefix, const char* what, bool packed = false)
{
    if (vals_dtype < 0 || vals_dtype > 2) return set_error(BS_ERR_INVALID, "%s: unknown dtype %d", what, vals_dtype);
    if (vals_numel < 0) return set_error(BS_ERR_INVALID, "%s: negative vals_numel", what);
    if (bitmask == nullptr || prefix == nullptr) return set_error(BS_ERR_INVALID, "%s: null bitmask/prefix", what);
    if (vals_numel > 0 && vals == nullptr) return set_error(BS_ERR_INVALID, "%s: null vals", what);
    int vb = (vals_dtype == DT_BF16 && !packed) ? 2 : 1;
    if (((uintptr_t)vals) % vb) return set_error(BS_ERR_INVALID, "%s: vals misaligned", what);
    return BS_OK;
}

static int decompress_impl(const void* vals, int vals_dtype, int64_t vals_numel, const uint8_t* bitmask,
                           const uint32_t* prefix, const int64_t* vals_offset, void* out,
                           int64_t first_m_tile, int64_t grid_n, int64_t K, int64_t batch_rows,
                           int64_t num_tiles_in_batch, int square, float relu2_scale, const float* scale,
                           void* stream, bool packed)
{
    clear_error();
    if (int rc = check_gather(vals, vals_dtype, vals_numel, bitmask, prefix, "bs_decompress", packed)) return rc;
    if (grid_n <= 0 || K < 0 || batch_rows < 0 || num_tiles_in_batch < 0 || first_m_tile < 0)
        return set_error(BS_ERR_INVALID, "bs_decompress: bad batch geometry");
    if (num_tiles_in_batch == 0 || K == 0 || batch_rows == 0) return BS_OK;
    if (out == nullptr) return set_error(BS_ERR_INVALID, "bs_decompress: null output");
    if (scale != nullptr && !square)
        return set_error(BS_ERR_INVALID, "bs_decompress: scale is only applied with square=1");
    if ((uint64_t)(first_m_tile * grid_n + num_tiles_in_batch) >= (1ull << 32))
        return set_error(BS_ERR_INVALID, "bs_decompress: tile ids exceed 32 bits");
    // bf16 values without the square run past 2^31 elements on the GPU
    const bool big_ok = vals_dtype == DT_BF16 && !square && !packed;
    if ((uint64_t)batch_rows * (uint64_t)K >= (big_ok ? kMaxElems : kMaxElemsUntested))
        return set_error(BS_ERR_INVALID, "bs_decompress: batch_rows*K must be < 2^%d on this path",
                         big_ok ? 32 : 31);
    const int ob = square ? 2 : (vals_dtype == DT_BF16 ? 2 : 1);
    if (((uintptr_t)out) % ob) return set_error(BS_ERR_INVALID, "bs_decompress: output misaligned");
    GatherArgs a{};
    a.vals = (const uint8_t*)vals;
    a.vals_numel = vals_numel;
    a.bitmask = bitmask;
    a.prefix = prefix;
    a.vals_offset = vals_offset;
    a.out = (uint8_t*)out;
    a.first_m_tile = first_m_tile;
    a.grid_n = (uint32_t)grid_n;
    a.K = K;
    a.rows = batch_rows;
    a.num_tiles = (uint32_t)num_tiles_in_batch;
    a.relu2_scale = relu2_scale;
    a.scale = scale;
    bool vec = (K % 8 == 0) && (((uintptr_t)out) % (8 * ob) == 0);
    const bool nt = use_nontemporal(batch_rows * K * ob);
    hipStream_t st = (hipStream_t)stream;
    const bool sc = scale != nullptr;
    switch (vals_dtype) {
    case DT_BF16:
        if (packed) launch_decompress_v<DT_BF16, true>(a, square, sc, vec, nt, st);
        else launch_decompress_v<DT_BF16, false>(a, square, sc, vec, nt, st);
        break;
    case DT_E4M3FN:
        if (packed) launch_decompress_v<DT_E4M3FN, true>(a, square, sc, vec, nt, st);
        else launch_decompress_v<DT_E4M3FN, false>(a, square, sc, vec, nt, st);
        break;
    default:
        if (packed) launch_decompress_v<DT_E5M2, true>(a, square, sc, vec, nt, st);
        else launch_decompress_v<DT_E5M2, false>(a, square, sc, vec, nt, st);
        break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_decompress launch: %s", hipGetErrorString(e));
    return BS_OK;
}

extern "C" int bs_decompress(const void* vals, int vals_dtype, int64_t vals_numel, const uint8_t* bitmask,
                             const uint32_t* prefix, const int64_t* vals_offset, void* out,
                             int64_t first_m_tile, int64_t grid_n, int64_t K, int64_t batch_rows,
                             int64_t num_tiles_in_batch, int square, float relu2_scale, const float* scale,
                             void* stream)
{
    return decompress_impl(vals, vals_dtype, vals_numel, bitmask, prefix, vals_offset, out, first_m_tile,
                           grid_n, K, batch_rows, num_tiles_in_batch, square, relu2_scale, scale, stream, false);
}

extern "C" int bs_decompress_packed(const void* stream_bytes, int vals_dtype, int64_t stream_nbytes,
                                    const uint8_t* bitmask, const uint32_t* prefix,
                                    const int64_t* vals_offset, void* out, int64_t first_m_tile,
                                    int64_t grid_n, int64_t K, int64_t batch_rows,
                                    int64_t num_tiles_in_batch, int square, float relu2_scale,
                                    const float* scale, void* stream)
{
    return decompress_impl(stream_bytes, vals_dtype, stream_nbytes, bitmask, prefix, vals_offset, out,
                           first_m_tile, grid_n, K, batch_rows, num_tiles_in_batch, square, relu2_scale,
                           scale, stream, true);
}

extern "C" int bs_relu_grad(void* grad, int64_t M, int64_t N, const uint8_t* bitmask, void* stream)
{
    clear_error();
    if (M < 0 || N < 0) return set_error(BS_ERR_INVALID, "bs_relu_grad: negative shape");
    const int64_t T = ((M + 63) / 64) * ((N + 63) / 64);
    if (T == 0) return BS_OK;
    if (grad == nullptr || bitmask == nullptr) return set_error(BS_ERR_INVALID, "bs_relu_grad: null pointer");
    if ((uint64_t)M * (uint64_t)N >= kMaxElemsUntested)
        return set_error(BS_ERR_INVALID, "bs_relu_grad: M*N must be < 2^31");
    if (((uintptr_t)grad) & 1u) return set_error(BS_ERR_INVALID, "bs_relu_grad: grad misaligned");
    bool vec = (N % 8 == 0) && aligned16(grad);
    uint32_t gn = (uint32_t)((N + 63) / 64);
    const uint32_t blocks = (uint32_t)((T + kMaskU - 1) / kMaskU);
    hipStream_t st = (hipStream_t)stream;
    if (vec && use_nontemporal(2 * M * N))
        hipLaunchKernelGGL((relu_grad_kernel<true, kMaskU, true>), dim3(blocks), dim3(kThreads), 0, st,
                           (uint8_t*)grad, M, N, gn, (uint32_t)T, bitmask);
    else if (vec)
        hipLaunchKernelGGL((relu_grad_kernel<true, kMaskU, false>), dim3(blocks), dim3(kThreads), 0, st,
                           (uint8_t*)grad, M, N, gn, (uint32_t)T, bitmask);
    else
        hipLaunchKernelGGL((relu_grad_kernel<false, kMaskU, false>), dim3(blocks), dim3(kThreads), 0, st,
                           (uint8_t*)grad, M, N, gn, (uint32_t)T, bitmask);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_relu_grad launch: %s", hipGetErrorString(e));
    return BS_OK;
}

template <int V_T, bool SC, bool PK>
static void launch_relu2_t(const GatherArgs& a, bool vec, bool nt, hipStream_t st)
{
    const uint32_t blocks = (a.num_tiles + kGatherU - 1) / kGatherU;
    if (vec && nt)
        hipLaunchKernelGGL((relu2_grad_kernel<V_T, SC, true, kGatherU, PK, true>), dim3(blocks), dim3(kThreads), 0, st, a);
    else if (vec)
        hipLaunchKernelGGL((relu2_grad_kernel<V_T, SC, true, kGatherU, PK, false>), dim3(blocks), dim3(kThreads), 0, st, a);
    else
        hipLaunchKernelGGL((relu2_grad_kernel<V_T, SC, false, kGatherU, PK, false>), dim3(blocks), dim3(kThreads), 0, st, a);
}

template <int V_T, bool PK>
static void launch_relu2_v(const GatherArgs& a, bool sc, bool vec, bool nt, hipStream_t st)
{
    if (sc) launch_relu2_t<V_T, true, PK>(a, vec, nt, st);
    else launch_relu2_t<V_T, false, PK>(a, vec, nt, st);
}

static int relu2_grad_impl(void* grad, int64_t M, int64_t N, const void* vals, int vals_dtype,
                           int64_t vals_numel, const uint8_t* bitmask, const uint32_t* prefix,
                           const int64_t* vals_offset, float relu2_scale, const float* scale, void* stream,
                           bool packed)
{
    clear_error();
    if (int rc = check_gather(vals, vals_dtype, vals_numel, bitmask, prefix, "bs_relu2_grad", packed)) return rc;
    if (M < 0 || N < 0) return set_error(BS_ERR_INVALID, "bs_relu2_grad: negative shape");
    const int64_t T = ((M + 63) / 64) * ((N + 63) / 64);
    if (T == 0) return BS_OK;
    if (grad == nullptr) return set_error(BS_ERR_INVALID, "bs_relu2_grad: null grad");
    if ((uint64_t)M * (uint64_t)N >= kMaxElemsUntested)
        return set_error(BS_ERR_INVALID, "bs_relu2_grad: M*N must be < 2^31");
    if (((uintptr_t)grad) & 1u) return set_error(BS_ERR_INVALID, "bs_relu2_grad: grad misaligned");
    GatherArgs a{};
    a.vals = (const uint8_t*)vals;
    a.vals_numel = vals_numel;
    a.bitmask = bitmask;
    a.prefix = prefix;
    a.vals_offset = vals_offset;
    a.out = (uint8_t*)grad;
    a.first_m_tile = 0;
    a.grid_n = (uint32_t)((N + 63) / 64);
    a.K = N;
    a.rows = M;
    a.num_tiles = (uint32_t)T;
    a.relu2_scale = relu2_scale;
    a.scale = scale;
    bool vec = (N % 8 == 0) && aligned16(grad);
    const bool nt = use_nontemporal(2 * M * N);
    hipStream_t st = (hipStream_t)stream;
    const bool sc = scale != nullptr;
    switch (vals_dtype) {
    case DT_BF16:
        if (packed) launch_relu2_v<DT_BF16, true>(a, sc, vec, nt, st);
        else launch_relu2_v<DT_BF16, false>(a, sc, vec, nt, st);
        break;
    case DT_E4M3FN:
        if (packed) launch_relu2_v<DT_E4M3FN, true>(a, sc, vec, nt, st);
        else launch_relu2_v<DT_E4M3FN, false>(a, sc, vec, nt, st);
        break;
    default:
        if (packed) launch_relu2_v<DT_E5M2, true>(a, sc, vec, nt, st);
        else launch_relu2_v<DT_E5M2, false>(a, sc, vec, nt, st);
        break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_relu2_grad launch: %s", hipGetErrorString(e));
    return BS_OK;
}

extern "C" int bs_relu2_grad(void* grad, int64_t M, int64_t N, const void* vals, int vals_dtype,
                             int64_t vals_numel, const uint8_t* bitmask, const uint32_t* prefix,
                             const int64_t* vals_offset, float relu2_scale, const float* scale, void* stream)
{
    return relu2_grad_impl(grad, M, N, vals, vals_dtype, vals_numel, bitmask, prefix, vals_offset,
                           relu2_scale, scale, stream, false);
}

extern "C" int bs_relu2_grad_packed(void* grad, int64_t M, int64_t N, const void* stream_bytes,
                                    int vals_dtype, int64_t stream_nbytes, const uint8_t* bitmask,
                                    const uint32_t* prefix, const int64_t* vals_offset, float relu2_scale,
                                    const float* scale, void* stream)
{
    return relu2_grad_impl(grad, M, N, stream_bytes, vals_dtype, stream_nbytes, bitmask, prefix, vals_offset,
                           relu2_scale, scale, stream, true);
}

extern "C" int bs_pack_bits(const void* raw, int vals_dtype, const uint32_t* count_ptr, int64_t count_max,
                            void* stream_bytes, int64_t stream_nbytes, const int64_t* start_index,
                            int32_t* err_flags, void* stream)
{
    clear_error();
    if (vals_dtype < 0 || vals_dtype > 2) return set_error(BS_ERR_INVALID, "bs_pack_bits: unknown dtype %d", vals_dtype);
    if (count_max < 0 || stream_nbytes < 0) return set_error(BS_ERR_INVALID, "bs_pack_bits: negative size");
    if (count_max == 0) return BS_OK;
    if (raw == nullptr || stream_bytes == nullptr) return set_error(BS_ERR_INVALID, "bs_pack_bits: null pointer");
    const int vb = vals_dtype == DT_BF16 ? 2 : 1, pb = vals_dtype == DT_BF16 ? 15 : 7;
    if (((uintptr_t)raw) % vb) return set_error(BS_ERR_INVALID, "bs_pack_bits: raw values misaligned");
    if (((uintptr_t)stream_bytes) & 3u) return set_error(BS_ERR_INVALID, "bs_pack_bits: stream not 4-byte aligned");
    if (count_max > (int64_t)1 << 40) return set_error(BS_ERR_INVALID, "bs_pack_bits: count too large");
    // enough threads for one 8-value group each (aligned start) and for one
    // output dword each (any other start); the kernel loops over the rest
    const int64_t work = std::max((count_max + 7) / 8, (count_max * pb + 62) / 32 + 1);
    const uint32_t blocks = (uint32_t)std::min<int64_t>((work + kPackThreads - 1) / kPackThreads, 8192);
    hipStream_t st = (hipStream_t)stream;
    const uint8_t* r = (const uint8_t*)raw;
    const bool raw_vec = (((uintptr_t)raw) % (8 * vb)) == 0;
    uint32_t* o = (uint32_t*)stream_bytes;
    const int64_t ow = stream_nbytes / 4;
    if (vals_dtype == DT_BF16)
        hipLaunchKernelGGL((pack_bits_kernel<2, 15>), dim3(blocks), dim3(kPackThreads), 0, st, r, count_ptr,
                           count_max, o, ow, start_index, err_flags, (int)raw_vec);
    else
        hipLaunchKernelGGL((pack_bits_kernel<1, 7>), dim3(blocks), dim3(kPackThreads), 0, st, r, count_ptr,
                           count_max, o, ow, start_index, err_flags, (int)raw_vec);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_pack_bits launch: %s", hipGetErrorString(e));
    return BS_OK;
}

// ===========================================================================
// bs_compress_noalloc: bs_compress / bs_compress_relu with the look-back
// status words and the amax slot in a library-owned device array instead of
// a caller-allocated workspace.  Each call clears the part of the array it
// uses (one small kernel) and runs with epoch 1, so no state carries over
// between calls and the call sequence can be captured into a HIP graph.
// ===========================================================================
namespace bs {

constexpr int64_t kScratchMaxTiles = int64_t(1) << 19;                 // 2^31 elements in 64x64 tiles (half the codec range)
constexpr int64_t kScratchBytes = (kWsHeaderBytes + 8 * (kScratchMaxTiles + 2) + 255) / 256 * 256 + kQtabBytes;
constexpr int kScratchMaxDevices = 64;

// One copy per GPU, held until the process ends.  Host code never uses this
// name as an address: scratch_base() looks the device address up once per
// device with hipGetSymbolAddress.
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kScratchMaxDevices];

// Device address of `scratch` on the device of `st`.
static int scratch_base(hipStream_t st, uint8_t** out)
{
    int dev = 0;
    hipError_t e = stream_device(st, &dev);
    if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_compress_noalloc: stream device: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kScratchMaxDevices)
        return set_error(BS_ERR_INVALID, "bs_compress_noalloc: device %d beyond %d", dev, kScratchMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        int cur = 0;
        e = hipGetDevice(&cur);
        if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
        void* p = nullptr;
        if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) (void)hipSetDevice(cur);
        if (e != hipSuccess || p == nullptr)
            return set_error(BS_ERR_HIP, "bs_compress_noalloc: scratch address: %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = static_cast<uint8_t*>(g_scratch_ptr[dev]);
    return BS_OK;
}

__global__ __launch_bounds__(256) void zero_words_kernel(uint64_t* p, int64_t n)
{
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) p[i] = 0ull;
}

}  // namespace bs

extern "C" int64_t bs_compress_noalloc_max_tiles(void) { return kScratchMaxTiles; }

extern "C" int bs_compress_noalloc(const void* dense, int in_dtype, int64_t M, int64_t N, int quantize, int relu,
                                   float* scale_out, void* dense_q_out, uint8_t* bitmask, uint32_t* prefix,
                                   void* vals, int64_t vals_capacity, const int64_t* vals_offset_in, int align8,
                                   int64_t* vals_offset_out, int64_t* vals_start_out, int write_vals,
                                   int32_t* err_flags, void* relu_out, void* stream)
{
    clear_error();
    if (M < 0 || N < 0) return set_error(BS_ERR_INVALID, "bs_compress_noalloc: negative shape");
    const int64_t T = ((M + 63) / 64) * ((N + 63) / 64);
    if (T > kScratchMaxTiles)
        return set_error(BS_ERR_INVALID, "bs_compress_noalloc: %lld tiles, at most %lld (the scratch array's size)",
                         (long long)T, (long long)kScratchMaxTiles);
    if (quantize && in_dtype != DT_BF16)
        return set_error(BS_ERR_INVALID, "bs_compress_noalloc: quantize needs bf16 input");
    if (quantize && ((uintptr_t)dense) & 1u) return set_error(BS_ERR_INVALID, "bs_compress_noalloc: input misaligned");
    hipStream_t st = (hipStream_t)stream;
    uint8_t* ws = nullptr;
    if (int rc = scratch_base(st, &ws)) return rc;
    constexpr uint32_t kEpoch = 1;
    // after compress_impl has checked every argument: clear the header (amax
    // slot, fallback counter) and the status words this shape uses (one per
    // unit of kStreamU tiles, one per unit group), then the amax if quantizing
    auto prepare = [&]() -> int {
        const int64_t units = (T + kStreamU - 1) / kStreamU;
        const int64_t words = kWsHeaderBytes / 8 + units + (units + kGroupUnits - 1) / kGroupUnits + 2;
        const uint32_t nblk = (uint32_t)std::min<int64_t>((words + 255) / 256, 1024);
        hipLaunchKernelGGL(zero_words_kernel, dim3(nblk), dim3(256), 0, st, reinterpret_cast<uint64_t*>(ws), words);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return set_error(BS_ERR_HIP, "bs_compress_noalloc launch: %s", hipGetErrorString(e));
        if (quantize) return amax_launch(dense, M * N, ws, kScratchBytes, kEpoch, stream, relu != 0, false);
        return BS_OK;
    };
    const uint64_t* slot = reinterpret_cast<const uint64_t*>(ws + kWsAmaxOffset);
    return compress_impl(dense, in_dtype, M, N, quantize, quantize ? slot : nullptr, kEpoch, scale_out, dense_q_out,
                         bitmask, prefix, vals, vals_capacity, vals_offset_in, align8, vals_offset_out,
                         vals_start_out, write_vals, err_flags, ws, kScratchBytes, kEpoch, stream, relu != 0,
                         relu_out, false, false, prepare);
}
