// Feed-forward half of a block for decode-sized batches (M <= 16 rows):
// RMSNorm + SwiGLU + residual (model/transformer.py:18-31, 126-129 with
// model/norm.py:15-21) in two launches instead of the ~12 small kernels the
// framework issues for ffn_norm / w_gate / w_up / silu / mul / w_down / add.
//
//   a[m, f]   = bf16( bf16(silu(g)) * u ),  g = bf16(x.Wg'[f] / rms(x)),  u = bf16(x.Wu'[f] / rms(x))
//   out[m, n] = bf16( x[m, n] + bf16(a[m, :] . Wd[n, :]) )
//
// with Wg' = w_gate * norm_weight and Wu' = w_up * norm_weight (the norm
// weight folded into the columns by the caller: w_gate_up = [Wg'; Wu'],
// [2F, C] bf16). The bf16 roundings sit where the unfused sequence rounds
// (the projections' outputs, silu, the product, the down projection, the
// residual sum); the norm is a per-row scale applied in fp32 after the
// product instead of a rounded normalised activation.
//
// Both launches use the decode producer's layout: a 256-thread workgroup owns
// 16 output columns, a 16-lane group per column keeps that column's weight
// row(s) in registers (C/128 16-byte chunks per lane) and forms the dot
// product with every x row, reduced across the group; the same lanes see the
// whole x row, so the gate/up launch also forms sum(x^2) for 1/rms. The x
// rows are staged in LDS first (rows.h).
#include "common.h"
#include "kernels.h"
#include "rows.h"

namespace sparda {

constexpr int kFfnThreads = 256;
constexpr int kFfnGuChunks = 8;     // gate/up: C <= 1024 (two weight rows per group)
constexpr int kFfnDownChunks = 16;  // down: F <= 2048

__device__ __forceinline__ float bf16_round(float v) { return static_cast<float>(static_cast<__bf16>(v)); }

// grid F/16: act[m, f] for 16 columns f per workgroup
__global__ void __launch_bounds__(kFfnThreads)
ffn_gate_up_kernel(const uint16_t* __restrict__ x, int64_t x_st, const uint16_t* __restrict__ wgu, int M, int C,
                   int F, float eps, uint16_t* __restrict__ act) {
    extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // [M][C]
    __shared__ float alds[kRowsMaxM][16];
    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int li = lane % 16;
    const int lc = 4 * (tid / kWave) + lane / 16;
    const int f = blockIdx.x * 16 + lc;
    const int nch = C / 128;
    uint4 w[2][kFfnGuChunks];
    const uint16_t* gr = wgu + static_cast<int64_t>(f) * C + li * 8;
    const uint16_t* ur = wgu + static_cast<int64_t>(F + f) * C + li * 8;
#pragma unroll
    for (int i = 0; i < kFfnGuChunks; ++i) {
        if (i < nch) {
            w[0][i] = *reinterpret_cast<const uint4*>(gr + i * 128);
            w[1][i] = *reinterpret_cast<const uint4*>(ur + i * 128);
        }
    }
    stage_rows(x, x_st, M, C, xs);
    float acc[2][kRowsMaxM], ss[kRowsMaxM];
#pragma unroll
    for (int m = 0; m < kRowsMaxM; ++m) acc[0][m] = acc[1][m] = ss[m] = 0.0f;
    rows_dot<2, kFfnGuChunks, true>(xs, M, C, nch, li, w, acc, ss);
#pragma unroll
    for (int m = 0; m < kRowsMaxM; ++m) {
        if (m < M) {
            const float ag = row16_sum(acc[0][m]);
            const float au = row16_sum(acc[1][m]);
            const float s2 = row16_sum(ss[m]);
            if (li == 0) {
                const float inv = 1.0f / __builtin_sqrtf(s2 / static_cast<float>(C) + eps);
                const float g = bf16_round(ag * inv);
                const float u = bf16_round(au * inv);
                const float s = bf16_round(g / (1.0f + expf(-g)));
                alds[m][lc] = bf16_round(s * u);
            }
        }
    }
    __syncthreads();
    for (int t = tid; t < M * 16; t += kFfnThreads) {
        const int m = t / 16, c = t % 16;
        act[static_cast<int64_t>(m) * F + blockIdx.x * 16 + c] =
            __builtin_bit_cast(uint16_t, static_cast<__bf16>(alds[m][c]));
    }
}

// grid N/16: out[m, n] = bf16(res[m, n] + bf16(a[m, :] . W[n, :])), W [N, K]
__global__ void __launch_bounds__(kFfnThreads)
ffn_down_kernel(const uint16_t* __restrict__ a, int64_t a_st, const uint16_t* __restrict__ w, int M, int K, int N,
                const uint16_t* __restrict__ res, int64_t res_st, uint16_t* __restrict__ out, int64_t out_st) {
    extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // [M][K]
    __shared__ float ylds[kRowsMaxM][16];
    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int li = lane % 16;
    const int lc = 4 * (tid / kWave) + lane / 16;
    const int n = blockIdx.x * 16 + lc;
    const int nch = K / 128;
    uint4 wr[1][kFfnDownChunks];
    const uint16_t* wrow = w + static_cast<int64_t>(n) * K + li * 8;
#pragma unroll
    for (int i = 0; i < kFfnDownChunks; ++i)
        if (i < nch) wr[0][i] = *reinterpret_cast<const uint4*>(wrow + i * 128);
    stage_rows(a, a_st, M, K, xs);
    float acc[1][kRowsMaxM], unused[kRowsMaxM];
#pragma unroll
    for (int m = 0; m < kRowsMaxM; ++m) acc[0][m] = 0.0f;
    rows_dot<1, kFfnDownChunks, false>(xs, M, K, nch, li, wr, acc, unused);
#pragma unroll
    for (int m = 0; m < kRowsMaxM; ++m) {
        if (m < M) {
            const float y = row16_sum(acc[0][m]);
            if (li == 0) ylds[m][lc] = y;
        }
    }
    __syncthreads();
    for (int t = tid; t < M * 16; t += kFfnThreads) {
        const int m = t / 16, c = t % 16;
        const int64_t col = static_cast<int64_t>(blockIdx.x) * 16 + c;
        const float r = __builtin_bit_cast(float, static_cast<uint32_t>(res[m * res_st + col]) << 16);
        out[m * out_st + col] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(r + bf16_round(ylds[m][c])));
    }
}

int launch_ffn_decode(const void* x, int64_t x_st, const void* w_gate_up, const void* w_down, int64_t M,
                      int64_t C, int64_t F, float eps, void* act, void* out, int64_t out_st, hipStream_t stream) {
    hipLaunchKernelGGL(ffn_gate_up_kernel, dim3(static_cast<unsigned>(F / 16)), dim3(kFfnThreads),
                       static_cast<size_t>(M * C) * 2, stream,
                       static_cast<const uint16_t*>(x), x_st, static_cast<const uint16_t*>(w_gate_up),
                       static_cast<int>(M), static_cast<int>(C), static_cast<int>(F), eps,
                       static_cast<uint16_t*>(act));
    int rc = check_hip(hipGetLastError(), "ffn_gate_up_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(ffn_down_kernel, dim3(static_cast<unsigned>(C / 16)), dim3(kFfnThreads),
                       static_cast<size_t>(M * F) * 2, stream,
                       static_cast<const uint16_t*>(act), F, static_cast<const uint16_t*>(w_down),
                       static_cast<int>(M), static_cast<int>(F), static_cast<int>(C),
                       static_cast<const uint16_t*>(x), x_st, static_cast<uint16_t*>(out), out_st);
    return check_hip(hipGetLastError(), "ffn_down_kernel");
}

// grid N/16: out[m, n] = bf16((x[m, :] . W'[n, :]) / rms(x[m])), W' [N, C] with the
// norm weight folded into its columns: the final RMSNorm and the output
// projection of a decode step in one launch
__global__ void __launch_bounds__(kFfnThreads)
norm_gemv_kernel(const uint16_t* __restrict__ x, int64_t x_st, const uint16_t* __restrict__ w, int M, int C,
                 float eps, uint16_t* __restrict__ out, int64_t out_st) {
    extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // [M][C]
    __shared__ float ylds[kRowsMaxM][16];
    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int li = lane % 16;
    const int lc = 4 * (tid / kWave) + lane / 16;
    const int n = blockIdx.x * 16 + lc;
    const int nch = C / 128;
    uint4 wr[1][kFfnGuChunks];
    const uint16_t* wrow = w + static_cast<int64_t>(n) * C + li * 8;
#pragma unroll
    for (int i = 0; i < kFfnGuChunks; ++i)
        if (i < nch) wr[0][i] = *reinterpret_cast<const uint4*>(wrow + i * 128);
    stage_rows(x, x_st, M, C, xs);
    float acc[1][kRowsMaxM], ss[kRowsMaxM];
#pragma unroll
    for (int m = 0; m < kRowsMaxM; ++m) acc[0][m] = ss[m] = 0.0f;
    rows_dot<1, kFfnGuChunks, true>(xs, M, C, nch, li, wr, acc, ss);
#pragma unroll
    for (int m = 0; m < kRowsMaxM; ++m) {
        if (m < M) {
            const float a = row16_sum(acc[0][m]);
            const float s2 = row16_sum(ss[m]);
            if (li == 0) ylds[m][lc] = a / __builtin_sqrtf(s2 / static_cast<float>(C) + eps);
        }
    }
    __syncthreads();
    for (int t = tid; t < M * 16; t += kFfnThreads) {
        const int m = t / 16, c = t % 16;
        out[m * out_st + static_cast<int64_t>(blockIdx.x) * 16 + c] =
            __builtin_bit_cast(uint16_t, static_cast<__bf16>(ylds[m][c]));
    }
}

int launch_norm_gemv(const void* x, int64_t x_st, const void* w, int64_t M, int64_t C, int64_t N, float eps,
                     void* out, int64_t out_st, hipStream_t stream) {
    hipLaunchKernelGGL(norm_gemv_kernel, dim3(static_cast<unsigned>(N / 16)), dim3(kFfnThreads),
                       static_cast<size_t>(M * C) * 2, stream, static_cast<const uint16_t*>(x), x_st,
                       static_cast<const uint16_t*>(w), static_cast<int>(M), static_cast<int>(C), eps,
                       static_cast<uint16_t*>(out), out_st);
    return check_hip(hipGetLastError(), "norm_gemv_kernel");
}

int launch_rows_residual(const void* a, int64_t a_st, const void* w, int64_t M, int64_t K, int64_t N,
                         const void* res, int64_t res_st, void* out, int64_t out_st, hipStream_t stream) {
    hipLaunchKernelGGL(ffn_down_kernel, dim3(static_cast<unsigned>(N / 16)), dim3(kFfnThreads),
                       static_cast<size_t>(M * K) * 2, stream, static_cast<const uint16_t*>(a), a_st,
                       static_cast<const uint16_t*>(w), static_cast<int>(M), static_cast<int>(K),
                       static_cast<int>(N), static_cast<const uint16_t*>(res), res_st, static_cast<uint16_t*>(out),
                       out_st);
    return check_hip(hipGetLastError(), "ffn_down_kernel");
}

}  // namespace sparda
