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
// The pointer is converted with an address-space cast (not through an integer)
// so that constant offsets from a common base fold into the instruction.
__device__ __forceinline__ i16x4 lds_read_tr(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4*)(const_cast<uint16_t*>(p)));
}

// Reductions over lane pairs (l, l^16) and (l, l^32) with the gfx950 VALU
// row swaps: permlane16_swap(x, x) hands every lane the values of rows
// {2r, 2r+1} at its column, permlane32_swap(x, x) those of rows {r, r+2};
// both lanes of a pair combine the same two values in the same order.
// Maxima of values that are never NaN (attention scores: finite, or -inf where
// masked). fmaxf in IEEE mode adds a quieting max per operand; these issue
// v_max3_f32 / v_max_f32 as is.
__device__ __forceinline__ float max3_nn(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
__device__ __forceinline__ float max_nn(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
// max of the 16 accumulator values s[0..3][0..3]: 8 instructions
__device__ __forceinline__ float max16_nn(const f32x4 (&s)[4]) {
    const float a = max3_nn(s[0][0], s[0][1], s[0][2]);
    const float b = max3_nn(s[0][3], s[1][0], s[1][1]);
    const float c = max3_nn(s[1][2], s[1][3], s[2][0]);
    const float d = max3_nn(s[2][1], s[2][2], s[2][3]);
    const float e = max3_nn(s[3][0], s[3][1], s[3][2]);
    return max_nn(max3_nn(a, b, c), max3_nn(d, e, s[3][3]));
}
// max of the 8 accumulator values s[0..1][0..3] (a 32-key block): 4 instructions
__device__ __forceinline__ float max8_nn(const f32x4 (&s)[2]) {
    return max_nn(max3_nn(max3_nn(s[0][0], s[0][1], s[0][2]), max3_nn(s[0][3], s[1][0], s[1][1]), s[1][2]), s[1][3]);
}
// the maximum of a lane's scores of one block: 4 sub-tiles of 16 keys (64-key
// block) or 2 (32-key block)
__device__ __forceinline__ float max_sub_nn(const f32x4 (&s)[4]) { return max16_nn(s); }
__device__ __forceinline__ float max_sub_nn(const f32x4 (&s)[2]) { return max8_nn(s); }
// max with the lane 16 (SWAP16) or 32 lanes away. One asm block: a VALU write
// of a register needs two wait states before a permlane swap reads it, and the
// compiler does not count inline-assembly results as VALU writes, so the copy,
// the s_nop and the swap stay together.
__device__ __forceinline__ float pair16_max(float x) {
    float t;
    asm("v_mov_b32 %1, %0\n\ts_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\tv_max_f32 %0, %0, %1"
        : "+v"(x), "=&v"(t));
    return x;
}
__device__ __forceinline__ float pair32_max(float x) {
    float t;
    asm("v_mov_b32 %1, %0\n\ts_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\tv_max_f32 %0, %0, %1"
        : "+v"(x), "=&v"(t));
    return x;
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
