// Decode-shape products (a few token rows against a weight matrix) shared by
// the decode producer and the feed-forward kernels: x rows are staged in LDS
// once, then each 16-lane group holds a slice of its weight row(s) in
// registers and accumulates one partial dot product per x row (all rows'
// LDS reads independent, so they overlap instead of paying one memory
// latency per row).
#pragma once

#include "common.h"

namespace sparda {

constexpr int kRowsMaxM = 16;  // x rows per launch

__device__ __forceinline__ void dot8(const uint4& xv, const uint4& wv, float& acc) {
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
    const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        acc = __builtin_fmaf(__builtin_bit_cast(float, xw[e] << 16), __builtin_bit_cast(float, ww[e] << 16), acc);
        acc = __builtin_fmaf(__builtin_bit_cast(float, xw[e] & 0xFFFF0000u),
                             __builtin_bit_cast(float, ww[e] & 0xFFFF0000u), acc);
    }
}

__device__ __forceinline__ void sq8(const uint4& xv, float& ss) {
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float x0 = __builtin_bit_cast(float, xw[e] << 16);
        const float x1 = __builtin_bit_cast(float, xw[e] & 0xFFFF0000u);
        ss = __builtin_fmaf(x0, x0, ss);
        ss = __builtin_fmaf(x1, x1, ss);
    }
}

// x [M, C] bf16 (row stride x_st) -> xs [M][C] in LDS, 16-byte chunks; ends with a barrier
__device__ __forceinline__ void stage_rows(const uint16_t* __restrict__ x, int64_t x_st, int M, int C,
                                           uint16_t* xs) {
    const int cpr = C / 8;
    for (int c = threadIdx.x; c < M * cpr; c += blockDim.x) {
        const int m = c / cpr, kk = c % cpr;
        *reinterpret_cast<uint4*>(xs + m * C + kk * 8) = *reinterpret_cast<const uint4*>(x + m * x_st + kk * 8);
    }
    __syncthreads();
}

// acc[r][m] += x[m, :] . w_r (this lane's slice: chunks i -> elements 128 i + 8 li .. +8),
// ss[m] += x[m, :]^2 over the same slice when SS
template <int NW, int MAXCH, bool SS>
__device__ __forceinline__ void rows_dot(const uint16_t* xs, int M, int C, int nch, int li,
                                         const uint4 (&w)[NW][MAXCH], float (&acc)[NW][kRowsMaxM],
                                         float (&ss)[kRowsMaxM]) {
#pragma unroll
    for (int m = 0; m < kRowsMaxM; ++m) {
        if (m < M) {
            const uint16_t* xr = xs + m * C + li * 8;
#pragma unroll
            for (int i = 0; i < MAXCH; ++i) {
                if (i < nch) {
                    const uint4 xv = *reinterpret_cast<const uint4*>(xr + i * 128);
#pragma unroll
                    for (int r = 0; r < NW; ++r) dot8(xv, w[r][i], acc[r][m]);
                    if constexpr (SS) sq8(xv, ss[m]);
                }
            }
        }
    }
}

}  // namespace sparda
