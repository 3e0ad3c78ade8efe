// Shared device/host helpers of libsparda (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include "../../include/sparda.h"

namespace sparda {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// element loads (bf16 is widened exactly to fp32)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

template <int DT>
__device__ __forceinline__ float load_elem(const void* p, int64_t i) {
    if constexpr (DT == SPARDA_F32) {
        return static_cast<const float*>(p)[i];
    } else {
        return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    }
}

// Two consecutive elements (i must be even-aligned for bf16 / 8-byte for f32).
template <int DT>
__device__ __forceinline__ float2 load_pair(const void* p, int64_t i) {
    if constexpr (DT == SPARDA_F32) {
        return *reinterpret_cast<const float2*>(static_cast<const float*>(p) + i);
    } else {
        uint32_t w = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(p) + i);
        return make_float2(__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u));
    }
}

template <int DT>
__device__ __forceinline__ void store_elem(void* p, int64_t i, float v) {
    if constexpr (DT == SPARDA_F32) {
        static_cast<float*>(p)[i] = v;
    } else {
        static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
    }
}

// ---------------------------------------------------------------------------
// canonical ranking of scores: larger first, equal scores by lower index.
// order_key is monotone in the float value, maps -0.0 onto +0.0.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ uint32_t order_key_bits(uint32_t u) {
    if (u == 0x80000000u) u = 0;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ uint32_t order_key(float x) { return order_key_bits(__float_as_uint(x)); }

// 64-bit rank: higher is better. Low word = ~index so that lower index wins ties.
__device__ __forceinline__ uint64_t rank64(float x, int32_t idx) {
    return (static_cast<uint64_t>(order_key(x)) << 32) | static_cast<uint32_t>(~static_cast<uint32_t>(idx));
}
__device__ __forceinline__ int32_t rank64_index(uint64_t r) {
    return static_cast<int32_t>(~static_cast<uint32_t>(r & 0xffffffffu));
}

// ---------------------------------------------------------------------------
// wavefront reductions (64 lanes)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        uint64_t w = __shfl_xor(v, o, kWave);
        v = w > v ? w : v;
    }
    return v;
}
__device__ __forceinline__ int wave_min_i32(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, kWave));
    return v;
}

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace sparda

// ---------------------------------------------------------------------------
// host-side error reporting (thread-local last error), used by the ABI layer
// ---------------------------------------------------------------------------
namespace sparda {
int set_error(int code, const char* fmt, ...);
int check_hip(hipError_t e, const char* what);
}  // namespace sparda

#define SPARDA_REQUIRE(cond, code, ...)                        \
    do {                                                       \
        if (!(cond)) return ::sparda::set_error((code), __VA_ARGS__); \
    } while (0)

#define SPARDA_HIP(call)                                       \
    do {                                                       \
        hipError_t e_ = (call);                                \
        if (e_ != hipSuccess) return ::sparda::check_hip(e_, #call); \
    } while (0)
