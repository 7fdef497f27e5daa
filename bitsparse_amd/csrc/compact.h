// Pieces of the compress kernels shared with the fused up-projection GEMM:
// chunk register types, the look-back status word, and the compaction of an
// 8-element chunk's set elements (v_perm selectors indexed by its mask byte).
#pragma once

#include "bs_device.h"

namespace bs {

template <int B> struct Raw;
template <> struct Raw<2> { using T = uint4; };   // 8 x bf16
template <> struct Raw<1> { using T = uint2; };   // 8 x fp8

// status word: [63:34] epoch, [33:32] flag (1 aggregate, 2 inclusive), [31:0] value
constexpr uint64_t kFlagAgg = 1, kFlagInc = 2;
__device__ __forceinline__ uint64_t pack_status(uint32_t epoch, uint64_t flag, uint32_t v)
{
    return ((uint64_t)epoch << 34) | (flag << 32) | v;
}

// Positive-bit byte of 8 bf16 values (x > 0: bits in [1, 0x7f80]) with
// packed 16-bit arithmetic, 13 VALU ops.  Per half, ((bits + 0x807f) mod 2^16)
// saturating-minus 0x80 has bit 15 set exactly for those bits: [1, 0x7f80]
// goes to [0x8080, 0xffff] and then [0x8000, 0xff7f]; 0 and the negative NaNs
// [0xff81, 0xffff] go to [0x8000, 0x807f] and then below 0x8000; the rest
// ([0x7f81, 0xff80]) wraps to [0, 0x7fff] and stays below.  v_perm selectors
// 8-11 replicate bits 15 / 31 of the second and first source into whole
// bytes, the masks keep bit k of byte k (values 0-3) and bit 4 + k (values
// 4-7), and a dot product with 0x01010101 adds (ORs) the four bytes.
__device__ __forceinline__ uint32_t mask_bf16x8_pk(const uint4 v)
{
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t u[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const u16x2 t = __builtin_bit_cast(u16x2, w[i]) + (u16x2)(0x807f);
        u[i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_sub_sat(t, (u16x2)(0x80)));
    }
    const uint32_t x = __builtin_amdgcn_perm(u[1], u[0], 0x0b0a0908u);   // values 0-3: 0xff / 0 bytes
    const uint32_t y = __builtin_amdgcn_perm(u[3], u[2], 0x0b0a0908u);   // values 4-7
    return __builtin_amdgcn_udot4((y & 0x80402010u) | (x & 0x08040201u), 0x01010101u, 0u, false);
}

// wave total of a per-lane value (every lane)
__device__ __forceinline__ uint32_t wave_total(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_readlane((int)wave_incl_scan(v), 63);
}

// Compaction selectors of mask byte m: the set elements move to the front.
// bf16 (OUTB 2): output dword j = perm(D1, D0, s[j]) | perm(D3, D2, s[4 + j]);
// fp8 (OUTB 1): output dword j = perm(D1, D0, s[j]), j < 2.
template <int OUTB>
__device__ __forceinline__ void compaction_selectors(uint32_t m, uint32_t* s)
{
    constexpr int NS = OUTB == 2 ? 8 : 2;
#pragma unroll
    for (int i = 0; i < NS; i++) s[i] = 0x0c0c0c0cu;   // 0x0c selects a zero byte
    uint32_t q = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        if ((m >> e) & 1u) {
            if constexpr (OUTB == 2) {
                const uint32_t ee = (uint32_t)(e & 3);
                const uint32_t pair = (2u * ee) | ((2u * ee + 1u) << 8);
                const uint32_t sh = (q & 1u) * 16u;
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if ((uint32_t)j == (q >> 1)) {
                        uint32_t& w = s[(e < 4 ? 0 : 4) + j];
                        w = (w & ~(0xffffu << sh)) | (pair << sh);
                    }
            } else {
                const uint32_t sh = (q & 3u) * 8u;
#pragma unroll
                for (int j = 0; j < 2; j++)
                    if ((uint32_t)j == (q >> 2)) s[j] = (s[j] & ~(0xffu << sh)) | ((uint32_t)e << sh);
            }
            q++;
        }
    }
}

// Write the 8 elements of a compacted chunk at consecutive positions from p,
// last element first, one store instruction per position.  Chunks compacted
// to exclusive offsets overlap: the zero tail of a chunk lands on the first
// elements of the chunks after it, which are written by later instructions
// (a lower element index), so every position ends up holding its set element.
// A chunk with no set element must not be written at all: its tail would
// land, in the same instruction, where the next chunk's element goes.
template <int OUTB>
__device__ __forceinline__ void write_compacted(uint8_t* p, const typename Raw<OUTB>::T& c)
{
    if constexpr (OUTB == 2) {
        const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
        for (int i = 7; i >= 0; i--) {
            *reinterpret_cast<uint16_t*>(p + 2 * i) = (uint16_t)(w[i >> 1] >> (16 * (i & 1)));
            asm volatile("" ::: "memory");
        }
    } else {
        const uint32_t w[2] = {c.x, c.y};
#pragma unroll
        for (int i = 7; i >= 0; i--) {
            p[i] = (uint8_t)(w[i >> 2] >> (8 * (i & 3)));
            asm volatile("" ::: "memory");
        }
    }
}

template <int OUTB>
__device__ __forceinline__ void ring_elem_store(uint8_t* vals, int64_t gi, const uint8_t* ring, int idx)
{
    if constexpr (OUTB == 2)
        reinterpret_cast<uint16_t*>(vals)[gi] = reinterpret_cast<const uint16_t*>(ring)[idx];
    else
        vals[gi] = ring[idx];
}

}  // namespace bs
