// Decode-shape products (a few token rows against a weight matrix) shared by
// the decode producer and the feed-forward kernels, on the matrix cores: a
// workgroup owns 16 weight rows (output columns) per tile; v_mfma_f32_16x16x32_bf16
// takes the 16 weight rows as its A operand and up to 16 x rows as its B
// operand (rows m >= M read as zero), so a launch costs the same for 1 and 16
// rows and is bound by the weight stream. The K dimension is split over the
// workgroup's waves in 128-element blocks; the wave partials are added in LDS
// in wave order (the result does not depend on timing).
#pragma once

#include "common.h"
#include "mfma.h"

namespace sparda {

constexpr int kRowsMaxM = 16;    // x rows per launch
constexpr int kRowsWaves = 4;    // waves per workgroup (K split)
constexpr int kRowsMaxKB = 4;    // 128-element K blocks per wave: K <= 2048

__device__ __forceinline__ float sq8(const uint4& xv) {
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float x0 = __builtin_bit_cast(float, xw[e] << 16);
        const float x1 = __builtin_bit_cast(float, xw[e] & 0xFFFF0000u);
        ss = __builtin_fmaf(x0, x0, ss);
        ss = __builtin_fmaf(x1, x1, ss);
    }
    return ss;
}

// This wave's share of C_t[r][m] = sum_k W_t[r][k] x[m][k] for NT weight
// tiles (r = 0..15: the tile's 16 rows; wrow[t] = this lane's row r = lane % 16
// of tile t, K elements), over the K blocks kb = wave, wave + kRowsWaves, ...
// Lane l (m = l % 16, g = l / 16) reads, for block kb, elements
// 128 kb + 32 g .. +32 of its W rows and of x row m, one 8-element slice per
// MFMA step: A and B lanes with the same (l % 16, g) carry the same k, which
// is all the product needs. Result layout (MFMA C): lane l, element i holds
// r = 4 (l / 16) + i, m = l % 16. ss = this lane's part of sum_k x[m][k]^2.
template <int NT>
__device__ __forceinline__ void rows_mfma(const uint16_t* __restrict__ x, int64_t x_st, int M, int K,
                                          const uint16_t* const (&wrow)[NT], int wave, f32x4 (&acc)[NT],
                                          float& ss) {
    const int lane = threadIdx.x % kWave;
    const int m = lane % 16, g = lane / 16;
    const bool mv = m < M;
    const uint16_t* xr = x + static_cast<int64_t>(mv ? m : 0) * x_st + 32 * g;
    const int nkb = K / 128;
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    ss = 0.0f;
    uint4 xv[kRowsMaxKB][4], wv[kRowsMaxKB][NT][4];
    // every load of the wave in flight before the first product
#pragma unroll
    for (int b = 0; b < kRowsMaxKB; ++b) {
        const int kb = wave + b * kRowsWaves;
        if (kb < nkb) {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                xv[b][s] = mv ? *reinterpret_cast<const uint4*>(xr + 128 * kb + 8 * s) : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    wv[b][t][s] = *reinterpret_cast<const uint4*>(wrow[t] + 128 * kb + 32 * g + 8 * s);
            }
        }
    }
#pragma unroll
    for (int b = 0; b < kRowsMaxKB; ++b) {
        const int kb = wave + b * kRowsWaves;
        if (kb < nkb) {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wv[b][t][s]),
                                                                     __builtin_bit_cast(bf16x8, xv[b][s]), acc[t],
                                                                     0, 0, 0);
                ss += sq8(xv[b][s]);
            }
        }
    }
}

// LDS for rows_reduce: the waves' partial tiles and sums of squares
template <int NT>
struct RowsRed {
    f32x4 part[NT][kRowsWaves][kWave];
    float ss[kRowsWaves][16];
};

// Adds the waves' partials in wave order: y[t][m][r] = C_t[r][m], and with
// want_ss rs[m] = sum_k x[m][k]^2. Called by the whole workgroup (two
// barriers); y and rs are LDS arrays the epilogue reads.
template <int NT>
__device__ __forceinline__ void rows_reduce(RowsRed<NT>& red, const f32x4 (&acc)[NT], float ss, int wave,
                                            bool want_ss, float (*y)[kRowsMaxM][16], float* rs) {
    const int tid = threadIdx.x;
    const int lane = tid % kWave;
#pragma unroll
    for (int t = 0; t < NT; ++t) red.part[t][wave][lane] = acc[t];
    if (want_ss) {
        ss += __shfl_xor(ss, 16, kWave);
        ss += __shfl_xor(ss, 32, kWave);
        if (lane < 16) red.ss[wave][lane] = ss;
    }
    __syncthreads();
    // thread tid -> (m, r) = (tid % 16, tid / 16): lane m + 16 (r / 4), element r % 4
    {
        const int m = tid % 16, r = tid / 16;
        const int src = m + 16 * (r / 4);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < kRowsWaves; ++w) v += red.part[t][w][src][r % 4];
            y[t][m][r] = v;
        }
        if (want_ss && tid < 16) {
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < kRowsWaves; ++w) s += red.ss[w][tid];
            rs[tid] = s;
        }
    }
    __syncthreads();
}

}  // namespace sparda
