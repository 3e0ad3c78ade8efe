// Shared device/host helpers of libsparda (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include "../../include/sparda.h"

namespace sparda {

constexpr int kWave = 64;
constexpr int kMaxSelCap = 34;    // selection list capacity: top_k (<= 32) + sink + own block
constexpr int kMaxHeadDim = 128;

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
// wavefront reductions (64 lanes), all on the VALU: DPP within rows of 16
// lanes (quad_perm xor 1 and xor 2, row_half_mirror, row_mirror), then the
// gfx950 row swaps across rows (permlane16_swap, permlane32_swap). Every
// pairing step combines the same two values on both lanes, so all lanes end
// with the identical result.
// ---------------------------------------------------------------------------
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // row_half_mirror
constexpr int kDppMirror = 0x140;     // row_mirror

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float2 rows16_swap(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float2 rows32_swap(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<kDppXor1>(v));
    v = fmaxf(v, dpp_f32<kDppXor2>(v));
    v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_f32<kDppMirror>(v));
    float2 r = rows16_swap(v);
    v = fmaxf(r.x, r.y);
    r = rows32_swap(v);
    return fmaxf(r.x, r.y);
}
__device__ __forceinline__ float wave_sum(float v) {
    v = v + dpp_f32<kDppXor1>(v);
    v = v + dpp_f32<kDppXor2>(v);
    v = v + dpp_f32<kDppHalfMirror>(v);
    v = v + dpp_f32<kDppMirror>(v);
    float2 r = rows16_swap(v);
    v = r.x + r.y;
    r = rows32_swap(v);
    return r.x + r.y;
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

// Query window of workgroup `id` in a grid of BH (sequence, KV head) pairs x
// NBq windows, heaviest (latest) windows first. Workgroups go to the chip's 8
// XCDs in turn (XCD id % 8), each XCD with its own L2. With fewer pairs than
// XCDs, a pair's windows are cut into 2S chunks (S = 8 / BH XCDs per pair) and
// XCD slot s takes chunk s, then its mirror 2S-1-s, each heaviest first: the
// XCD reads the K/V blocks of two window ranges of one pair instead of the
// whole sequence, and the slots get about equal work when a window's cost
// grows with its position. Otherwise consecutive ids cycle through the pairs.
__device__ __forceinline__ void window_order(int64_t id, int64_t BH, int64_t NBq, int64_t& bg, int64_t& qw) {
    constexpr int64_t kXcd = 8;
    if (BH < kXcd && kXcd % BH == 0 && NBq % (2 * (kXcd / BH)) == 0) {
        const int64_t x = id % kXcd, j = id / kXcd;
        const int64_t S = kXcd / BH, s = x / BH, c = NBq / (2 * S);
        bg = x % BH;
        const int64_t chunk = j < c ? s : 2 * S - 1 - s;
        qw = NBq - 1 - (chunk * c + (j < c ? j : j - c));
    } else {
        bg = id % BH;
        qw = NBq - 1 - id / BH;
    }
}

// VEC consecutive elements widened to fp32 (the index must be VEC-aligned).
template <int DT, int VEC>
__device__ __forceinline__ void load_vec(const void* p, int64_t i, float (&o)[VEC]) {
    if constexpr (VEC == 1) {
        o[0] = load_elem<DT>(p, i);
    } else if constexpr (VEC == 2) {
        const float2 v = load_pair<DT>(p, i);
        o[0] = v.x;
        o[1] = v.y;
    } else if constexpr (DT == SPARDA_F32) {
        const float4 v = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    } else {
        const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
        o[0] = __uint_as_float(w.x << 16);
        o[1] = __uint_as_float(w.x & 0xffff0000u);
        o[2] = __uint_as_float(w.y << 16);
        o[3] = __uint_as_float(w.y & 0xffff0000u);
    }
}

// Sum of one block of key rows, sequential in s (the canonical prototype
// order): acc[v] = ((0 + k[s0]) + k[s0+1]) + ... for VEC adjacent elements.
// For a full block of UNROLL rows every load is issued before the additions.
template <int DT, int VEC, int UNROLL>
__device__ __forceinline__ void block_sum(const void* __restrict__ kc, int64_t base, int64_t s0, int64_t s1,
                                          int64_t ss, float (&acc)[VEC]) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = 0.0f;
    if (UNROLL > 0 && s1 - s0 == UNROLL) {
        float buf[UNROLL > 0 ? UNROLL : 1][VEC];
#pragma unroll
        for (int i = 0; i < UNROLL; ++i) load_vec<DT, VEC>(kc, base + (s0 + i) * ss, buf[i]);
#pragma unroll
        for (int i = 0; i < UNROLL; ++i)
#pragma unroll
            for (int v = 0; v < VEC; ++v) acc[v] = acc[v] + buf[i][v];
    } else {
#pragma unroll 8
        for (int64_t s = s0; s < s1; ++s) {
            float x[VEC];
            load_vec<DT, VEC>(kc, base + s * ss, x);
#pragma unroll
            for (int v = 0; v < VEC; ++v) acc[v] = acc[v] + x[v];
        }
    }
}

}  // namespace sparda

// ---------------------------------------------------------------------------
// host-side error reporting (thread-local last error), used by the ABI layer
// ---------------------------------------------------------------------------
namespace sparda {
int set_error(int code, const char* fmt, ...);
int check_hip(hipError_t e, const char* what);
// sum over each 16-lane group of a wavefront
__device__ __forceinline__ float row16_sum(float v) {
    v += __shfl_xor(v, 8, 16);
    v += __shfl_xor(v, 4, 16);
    v += __shfl_xor(v, 2, 16);
    v += __shfl_xor(v, 1, 16);
    return v;
}

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
