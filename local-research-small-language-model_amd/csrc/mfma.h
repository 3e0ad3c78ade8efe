// gfx950 matrix-core helpers shared by the prefill and decode kernels:
// bf16 operand vectors, LDS operand reads (plain and transposed) and the
// lane-pair reductions over the row-swap permutes.
#pragma once

#include "common.h"

namespace sparda {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 lds_read8(const uint16_t* p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}

// Transposed read (ds_read_b64_tr_b16). Within each 16-lane group, output
// lane i, element e is element i%4 of the 8-byte chunk addressed by lane
// 4e + i/4 of the group.
__device__ __forceinline__ i16x4 lds_read_tr(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        reinterpret_cast<__attribute__((address_space(3))) i16x4*>(
            reinterpret_cast<uintptr_t>(p)));
}

// Reductions over lane pairs (l, l^16) and (l, l^32) with the gfx950 VALU
// row swaps: permlane16_swap(x, x) hands every lane the values of rows
// {2r, 2r+1} at its column, permlane32_swap(x, x) those of rows {r, r+2};
// both lanes of a pair combine the same two values in the same order.
__device__ __forceinline__ float pair16_max(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair32_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair16_sum(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair32_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace sparda
