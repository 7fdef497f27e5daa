// Device-side building blocks shared by the BitSparse HIP kernels (gfx950).
//
// Format facts used everywhere (reference lib_sparse/src/triton_kernels.py:1-17,
// lib_sparse/bitsparse.py:120-127):
//   * 64x64 tiles, tile id t = tm * grid_n + tn;
//   * a "chunk" is 8 consecutive elements of one tile row; chunk b of a tile
//     (0..511) covers tile-flat indices 8b..8b+7, i.e. row b/8, columns
//     8*(b%8)..+7, and owns exactly bitmask byte t*512 + b (LSB = first column);
//   * "positive" is the strict IEEE compare x > 0 evaluated on bit patterns.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bs {

enum : int { DT_BF16 = 0, DT_E4M3FN = 1, DT_E5M2 = 2 };

constexpr int kTile = 64;
constexpr int kTileNumel = 4096;
constexpr int kTileBytes = 512;     // bitmask bytes per tile
constexpr int kChunksPerTile = 512; // 8-element chunks per tile
constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// streaming (nontemporal) global accesses: data read or written once.  The
// `nt` bit keeps the line out of the caches' retained set, which on gfx950
// raises a pure streaming read from ~6.0 to ~6.8 TB/s.
// ---------------------------------------------------------------------------
typedef uint32_t bs_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t bs_u32x2 __attribute__((ext_vector_type(2)));

template <bool NT>
__device__ __forceinline__ uint4 ld16(const void* p)
{
    if constexpr (NT) {
        const bs_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const bs_u32x4*>(p));
        return uint4{v.x, v.y, v.z, v.w};
    } else {
        return *reinterpret_cast<const uint4*>(p);
    }
}
template <bool NT>
__device__ __forceinline__ uint2 ld8(const void* p)
{
    if constexpr (NT) {
        const bs_u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const bs_u32x2*>(p));
        return uint2{v.x, v.y};
    } else {
        return *reinterpret_cast<const uint2*>(p);
    }
}
template <bool NT>
__device__ __forceinline__ void st16(void* p, const uint4 v)
{
    if constexpr (NT) {
        const bs_u32x4 w = {v.x, v.y, v.z, v.w};
        __builtin_nontemporal_store(w, reinterpret_cast<bs_u32x4*>(p));
    } else {
        *reinterpret_cast<uint4*>(p) = v;
    }
}
template <bool NT>
__device__ __forceinline__ void st8(void* p, const uint2 v)
{
    if constexpr (NT) {
        const bs_u32x2 w = {v.x, v.y};
        __builtin_nontemporal_store(w, reinterpret_cast<bs_u32x2*>(p));
    } else {
        *reinterpret_cast<uint2*>(p) = v;
    }
}
// a chunk (uint4 = 8 bf16, uint2 = 8 fp8) of either width
template <bool NT, typename T>
__device__ __forceinline__ T ld_chunk(const void* p)
{
    if constexpr (sizeof(T) == 16) return ld16<NT>(p);
    else return ld8<NT>(p);
}
template <bool NT, typename T>
__device__ __forceinline__ void st_chunk(void* p, const T& v)
{
    if constexpr (sizeof(T) == 16) st16<NT>(p, v);
    else st8<NT>(p, v);
}

// ---------------------------------------------------------------------------
// positive tests on raw bits: x > 0 <=> bits in (0, +Inf]
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pos_bf16(uint32_t b) { return (b - 1u) < 0x7f80u; }

// ---------------------------------------------------------------------------
// scalar conversions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// fp32 -> bf16 bits, round to nearest even, NaN kept quiet: the hardware
// conversion (v_cvt_pk_bf16_f32), one instruction where the integer form
// (NaN test, add 0x7fff + lsb, shift) takes five.
__device__ __forceinline__ uint32_t f32_to_bf16(float f)
{
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// e4m3fn bits -> fp32 (exact). 0x7f / 0xff are NaN.
__device__ __forceinline__ float e4m3_to_f32(uint32_t b)
{
    uint32_t e = (b >> 3) & 15u, m = b & 7u;
    float v;
    if (e == 0u) v = (float)m * 0.001953125f;                       // m * 2^-9
    else v = __uint_as_float(((e + 120u) << 23) | (m << 20));        // 1.m * 2^(e-7)
    if (e == 15u && m == 7u) v = __uint_as_float(0x7fc00000u);
    return (b & 0x80u) ? -v : v;
}

// e5m2 bits -> fp32 (exact): the top byte of an IEEE half.
__device__ __forceinline__ float e5m2_to_f32(uint32_t b)
{
    uint32_t e = (b >> 2) & 31u, m = b & 3u;
    float v;
    if (e == 0u) v = (float)m * 1.52587890625e-05f;                  // m * 2^-16
    else if (e == 31u) v = __uint_as_float(m ? 0x7fc00000u : 0x7f800000u);
    else v = __uint_as_float(((e + 112u) << 23) | (m << 21));
    return (b & 0x80u) ? -v : v;
}

template <int DT>
__device__ __forceinline__ float fp8_to_f32(uint32_t b)
{
    return DT == DT_E4M3FN ? e4m3_to_f32(b) : e5m2_to_f32(b);
}

// fp32 -> e4m3fn bits, round to nearest even, no saturation: |x| > 464,
// Inf and NaN give NaN (0x7f | sign); 464 itself rounds to 448.
__device__ __forceinline__ uint32_t f32_to_e4m3(float f)
{
    uint32_t u = __float_as_uint(f);
    uint32_t sign = (u >> 24) & 0x80u;
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x43e80000u) return sign | 0x7fu;                        // > 464.0, Inf, NaN
    if (a < 0x3c800000u) {                                           // < 2^-6: subnormal grid 2^-9
        float t = __builtin_rintf(__uint_as_float(a) * 512.0f);
        return sign | (uint32_t)t;
    }
    a += 0x7ffffu + ((a >> 20) & 1u);                                // RNE at mantissa bit 20
    return sign | ((((a >> 23) - 120u) << 3) | ((a >> 20) & 7u));
}

// The plain product y = x * r (r = 1/s rounded, one more rounding in the
// product: |y - x/s| <= 2^-23 |x/s|) lies within 3 ulp of the correctly
// rounded quotient (itself within 2^-24 |x/s|), so y converts to the
// quotient's e4m3 code when y is in e4m3's normal range and no rounding tie
// is within 3 ulp of it.
__device__ __forceinline__ bool e4m3_product_safe(uint32_t yb)
{
    return ((((yb >> 23) & 0xffu) - 121u) <= 14u) && (((yb & 0xfffffu) - 0x7fffdu) > 6u);
}

// f32_to_e4m3(x0 / s) | f32_to_e4m3(x1 / s) << 8 for a scale s > 0 (or NaN)
// with r = 1/s: one packed hardware conversion of the two products; x = +-0
// converts as +-0 (= x/s for every such s that is not NaN); anything else
// outside the safe region takes the exact division.
__device__ __forceinline__ uint32_t div2_to_e4m3(float x0, float x1, float s, float r)
{
    const float y0 = x0 * r, y1 = x1 * r;
    uint32_t out = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y0, y1, 0, false) & 0xffffu;
    const bool s_ok = s == s;
    const bool ok0 = e4m3_product_safe(__float_as_uint(y0)) || ((__float_as_uint(x0) << 1) == 0u && s_ok);
    const bool ok1 = e4m3_product_safe(__float_as_uint(y1)) || ((__float_as_uint(x1) << 1) == 0u && s_ok);
    if (!ok0) out = (out & 0xff00u) | f32_to_e4m3(x0 / s);
    if (!ok1) out = (out & 0x00ffu) | (f32_to_e4m3(x1 / s) << 8);
    return out;
}

// The ReLU^2 layer's h = k * r^2 as torch forms it in place (h.square_()
// then h.mul_(k)): bf16(bf16(r * r) * k), a NaN as torch's 0x7fc0.  For
// r >= 0 (or NaN) and a finite k, |h| is non-decreasing in r (the square is
// exact in fp32, each rounding is monotonic), so max |h| = |h(max r)|.
__device__ __forceinline__ uint32_t relu2_sq_bits(uint32_t b, float k)
{
    const float r = bf16_to_f32(b);
    const uint32_t sq = f32_to_bf16(r * r);
    const uint32_t h = f32_to_bf16(bf16_to_f32(sq) * k);
    return (h & 0x7fffu) > 0x7f80u ? 0x7fc0u : h;
}

// relu2_sq_bits of the 8 bf16 values of a chunk
__device__ __forceinline__ uint4 relu2_sq_chunk(const uint4 v, float k)
{
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = relu2_sq_bits(w[i] & 0xffffu, k) | (relu2_sq_bits(w[i] >> 16, k) << 16);
    return uint4{o[0], o[1], o[2], o[3]};
}

// ---------------------------------------------------------------------------
// 8-element chunks: bitmask byte of 8 values held in registers
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t mask_bf16x8(const uint4 v)
{
    return pos_bf16(v.x & 0xffffu) | (pos_bf16(v.x >> 16) << 1) |
           (pos_bf16(v.y & 0xffffu) << 2) | (pos_bf16(v.y >> 16) << 3) |
           (pos_bf16(v.z & 0xffffu) << 4) | (pos_bf16(v.z >> 16) << 5) |
           (pos_bf16(v.w & 0xffffu) << 6) | (pos_bf16(v.w >> 16) << 7);
}

// Positive-bit byte of 8 fp8 codes, byte-parallel (13 VALU ops): a code is
// positive iff its sign bit is clear and its low 7 bits l satisfy
// 1 <= l <= MAXP (0x7e e4m3fn, 0x7c e5m2: above are NaN / Inf).  Per byte,
// l + 0x7f has bit 7 set iff l != 0 and l + (0x7f - MAXP) has it set iff
// l > MAXP; neither sum carries out of its byte.  Two byte dot products with
// 0x08040201 / 0x80402010 gather the eight bit-7 flags.
template <int DT>
__device__ __forceinline__ uint32_t mask_fp8x8(const uint2 v)
{
    constexpr uint32_t MAXP = DT == DT_E4M3FN ? 0x7eu : 0x7cu;
    auto flags = [](uint32_t w) __attribute__((always_inline)) {
        const uint32_t l = w & 0x7f7f7f7fu;
        return (l + 0x7f7f7f7fu) & ~(l + (0x7fu - MAXP) * 0x01010101u) & ~w & 0x80808080u;
    };
    const uint32_t d = __builtin_amdgcn_udot4(flags(v.y), 0x80402010u,
                                              __builtin_amdgcn_udot4(flags(v.x), 0x08040201u, 0u, false), false);
    return d >> 7;
}

__device__ __forceinline__ uint32_t get16(const uint4 v, int e)
{
    uint32_t w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
    return (e & 1) ? (w >> 16) : (w & 0xffffu);
}

__device__ __forceinline__ uint32_t get8(const uint2 v, int e)
{
    return ((e < 4 ? v.x : v.y) >> (8 * (e & 3))) & 0xffu;
}

// ---------------------------------------------------------------------------
// wave / lane helpers (wave64)
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

// Lane 0's value of a uint32 in every lane (a scalar register).  The builtin
// takes and returns int, so a value of 2^31 or more (a tile prefix, which
// reaches 2^32 - 1) must be widened from the unsigned result: converting the
// int straight to int64 sign-extends it.
__device__ __forceinline__ uint32_t uniform_u32(uint32_t x)
{
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)x);
}

// number of set bits of `m` in lanes strictly below this lane
__device__ __forceinline__ uint32_t popc_below(uint64_t m)
{
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Exclusive prefix and total over the wave of a per-lane count in [0, 15],
// built from four ballots (one per bit of the count).
__device__ __forceinline__ void wave_scan_count(uint32_t c, uint32_t& excl, uint32_t& total)
{
    uint64_t b0 = __ballot(c & 1u), b1 = __ballot(c & 2u);
    uint64_t b2 = __ballot(c & 4u), b3 = __ballot(c & 8u);
    excl = popc_below(b0) + 2u * popc_below(b1) + 4u * popc_below(b2) + 8u * popc_below(b3);
    total = (uint32_t)(__popcll(b0) + 2 * __popcll(b1) + 4 * __popcll(b2) + 8 * __popcll(b3));
}

// The same for a count in [0, 16] (five ballots).
__device__ __forceinline__ void wave_scan_count16(uint32_t c, uint32_t& excl, uint32_t& total)
{
    uint64_t b0 = __ballot(c & 1u), b1 = __ballot(c & 2u), b2 = __ballot(c & 4u);
    uint64_t b3 = __ballot(c & 8u), b4 = __ballot(c & 16u);
    excl = popc_below(b0) + 2u * popc_below(b1) + 4u * popc_below(b2) + 8u * popc_below(b3) +
           16u * popc_below(b4);
    total = (uint32_t)(__popcll(b0) + 2 * __popcll(b1) + 4 * __popcll(b2) + 8 * __popcll(b3) +
                       16 * __popcll(b4));
}

// Inclusive wave64 prefix sum (row shifts inside 16-lane rows, then the row
// broadcasts of lanes 15 and 31).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x)
{
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, false);   // row_shr:1
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, false);   // row_shr:2
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, false);   // row_shr:4
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, false);   // row_shr:8
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false);   // row_bcast:15
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false);   // row_bcast:31
    return x;
}

// Wave total of a per-lane count in [0, 15] (four ballots, scalar result).
__device__ __forceinline__ uint32_t wave_sum_count(uint32_t c)
{
    return (uint32_t)(__popcll(__ballot(c & 1u)) + 2 * __popcll(__ballot(c & 2u)) +
                      4 * __popcll(__ballot(c & 4u)) + 8 * __popcll(__ballot(c & 8u)));
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor(v, o, 64));
    return v;
}

// relaxed device-scope atomics: the status words carry their whole payload,
// so no fence is needed around them
__device__ __forceinline__ uint64_t ld_relaxed(const uint64_t* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_relaxed(uint64_t* p, uint64_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// The quantizer through a code table.  For a fixed scale s, f32_to_e4m3(x / s)
// of a bf16 x depends only on x's 15 magnitude bits m (RNE and the NaN rule
// are symmetric, so the sign bit is x's), and only a window of 24 exponents
// around s's gives codes other than 0 and 0x7f.  With Es the biased exponent
// of s (s < 2^(Es-126)):
//   * m below (Es - 12) * 128 is x < 2^(Es-139) <= s * 2^-12: the quotient
//     rounds below 2^-12 and converts to 0;
//   * m at or above (Es + 12) * 128 is x >= 2^(Es-115) > s * 2^11: the
//     quotient is above 464 (or Inf / NaN for the Inf and NaN magnitudes)
//     and converts to 0x7f.
// A NaN scale makes every code NaN: the scale's own (positive, 0x7f) for a
// non-NaN x, x's for a NaN x (a quotient with one NaN operand is that NaN).
// An infinite scale puts the window past the Inf/NaN exponent, whose entries
// are then computed like the others.
// Table, one half per sign of x (kQtabEntries each, negative half second):
// [0] the code of every magnitude below the window, [1 + i] the code of
// magnitude base + i (i < 3072), [3073] the code of every magnitude above it,
// each from one correctly rounded division (the quantizer's own rule); a
// lookup is qtab[clamp(m - base + 1, 0, 3073) + sign * kQtabEntries].
constexpr int kQwinExps = 24;
constexpr int kQtabEntries = kQwinExps * 128 + 2;
constexpr int kQtabBytes = (2 * kQtabEntries + 15) / 16 * 16;     // the table's space (16-byte copies)

// window base (a magnitude) of a scale, minus 1: the lookup's offset
__device__ __forceinline__ int qtab_offset(float scale)
{
    return ((int)((__float_as_uint(scale) >> 23) & 0xffu) - kQwinExps / 2) * 128 - 1;
}

__device__ __forceinline__ uint32_t qtab_code(const uint8_t* qtab, uint32_t m, uint32_t sign, int qoff)
{
    const int i = min(max((int)m - qoff, 0), kQtabEntries - 1);
    return (uint32_t)qtab[i + (int)sign * kQtabEntries];
}

// qtab_code of 8 bf16 values, the table indices formed two at a time with
// packed 16-bit arithmetic: clamp(m - qoff, 0, E - 1) = clamp(m, L, L') - qoff
// with L = max(qoff, 0), L' = qoff + E - 1 (qoff >= -1537, so L <= L' < 2^16),
// the subtraction taken mod 2^16 (its result is in [0, E - 1]); + E for x < 0.
__device__ __forceinline__ uint2 quant_chunk_tab(const uint4 v, const uint8_t* qtab, int qoff)
{
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const u16x2 lo = (u16x2)(unsigned short)(qoff > 0 ? qoff : 0);
    const u16x2 hi = (u16x2)(unsigned short)(qoff + kQtabEntries - 1);
    const u16x2 off = (u16x2)(unsigned short)(uint32_t)qoff;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t p[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const u16x2 h = __builtin_bit_cast(u16x2, w[k]);
        const u16x2 m = h & (u16x2)(unsigned short)0x7fff;
        const u16x2 i = __builtin_elementwise_min(__builtin_elementwise_max(m, lo), hi) - off +
                        (h >> (u16x2)(unsigned short)15) * (u16x2)(unsigned short)kQtabEntries;
        const uint32_t ii = __builtin_bit_cast(uint32_t, i);
        p[k] = (uint32_t)qtab[ii & 0xffffu] | ((uint32_t)qtab[ii >> 16] << 8);
    }
    return uint2{p[0] | (p[1] << 16), p[2] | (p[3] << 16)};
}

}  // namespace bs
