// Helpers shared by the reconstruct-into-LDS GEMMs (bf16 and fp8 operand):
// raw buffer loads through wave-uniform resources and compile-time loops.
#pragma once

#include <type_traits>
#include <utility>

#include "bs_device.h"

namespace bs {

constexpr int kBK = 64;               // K per step (one B tile row)
constexpr int kMaxSteps = 256;        // K-steps per workgroup (prefixes held in registers)
constexpr int kCus = 256;             // MI355X compute units (split-K sizing)
constexpr int kXcds = 8;

typedef float f32x16_t __attribute__((ext_vector_type(16)));

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
__device__ __forceinline__ uint2 load8(bs_rsrc rs, uint32_t off)
{
    typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)off, 0, 0);
    return uint2{v[0], v[1]};
}
__device__ __forceinline__ uint32_t load4(bs_rsrc rs, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b32(rs, (int)off, 0, 0);
}

// compile-time register-set index
template <int P>
struct IC {
    static constexpr int value = P;
};

// f(IC<0>{}), ..., f(IC<N-1>{}) with compile-time indices
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>)
{
    (f(IC<I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f)
{
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

}  // namespace bs
