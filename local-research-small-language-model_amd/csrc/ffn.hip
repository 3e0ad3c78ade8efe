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
// Both launches use the decode producer's layout (rows.h): a workgroup owns 16
// output columns, the x rows are the B operand of the matrix-core products, and
// the gate/up launch also forms sum(x^2) for 1/rms from the same x slices.
#include "common.h"
#include "kernels.h"
#include "prefetch.h"
#include "rows.h"

namespace sparda {

constexpr int kFfnThreads = kRowsWaves * kWave;

__device__ __forceinline__ float bf16_round(float v) { return static_cast<float>(static_cast<__bf16>(v)); }

// Both launches may carry a share of the next layer's prefetch copy (stage 2):
// workgroups n_out, n_out + 1, ... copy it for (sequence, KV head) = the
// index past n_out, beside the product workgroups.
#define SPARDA_CARRIED_COPY()                                                                          \
    do {                                                                                               \
        if (static_cast<int>(blockIdx.x) >= n_out) {                                                  \
            __shared__ int32_t pf_sel[kMaxSelCap];                                                     \
            const int idx = static_cast<int>(blockIdx.x) - n_out;                                      \
            prefetch_copy_workgroup(pf, static_cast<int>(idx % pf.H), static_cast<int>(idx / pf.H), pos_dev, \
                                    pf_sel);                                                           \
            return;                                                                                    \
        }                                                                                              \
    } while (0)

// grid F/16: act[m, f] for 16 columns f per workgroup
__global__ void __launch_bounds__(kFfnThreads)
ffn_gate_up_kernel(const uint16_t* __restrict__ x, int64_t x_st, const uint16_t* __restrict__ wgu, int M, int C,
                   int F, float eps, uint16_t* __restrict__ act, int n_out, PrefetchDev pf,
                   const int64_t* __restrict__ pos_dev) {
    SPARDA_CARRIED_COPY();
    __shared__ RowsRed<2> red;
    __shared__ float y[2][kRowsMaxM][16];
    __shared__ float rs[16];
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int r = tid % 16;
    const int f0 = blockIdx.x * 16;
    const uint16_t* wrow[2] = {wgu + static_cast<int64_t>(f0 + r) * C, wgu + static_cast<int64_t>(F + f0 + r) * C};
    f32x4 acc[2];
    float ss;
    rows_mfma<2>(x, x_st, M, C, wrow, wave, acc, ss);
    rows_reduce<2>(red, acc, ss, wave, true, y, rs);
    if (tid < M * 16) {
        const int m = tid / 16, c = tid % 16;
        const float inv = 1.0f / __builtin_sqrtf(rs[m] / static_cast<float>(C) + eps);
        const float g = bf16_round(y[0][m][c] * inv);
        const float u = bf16_round(y[1][m][c] * inv);
        const float sl = bf16_round(g / (1.0f + expf(-g)));
        act[static_cast<int64_t>(m) * F + f0 + c] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(sl * u));
    }
}

// grid N/16: out[m, n] = bf16(res[m, n] + bf16(a[m, :] . W[n, :])), W [N, K]
__global__ void __launch_bounds__(kFfnThreads)
ffn_down_kernel(const uint16_t* __restrict__ a, int64_t a_st, const uint16_t* __restrict__ w, int M, int K, int N,
                const uint16_t* __restrict__ res, int64_t res_st, uint16_t* __restrict__ out, int64_t out_st,
                int n_out, PrefetchDev pf, const int64_t* __restrict__ pos_dev) {
    SPARDA_CARRIED_COPY();
    __shared__ RowsRed<1> red;
    __shared__ float y[1][kRowsMaxM][16];
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int n0 = blockIdx.x * 16;
    const uint16_t* wrow[1] = {w + static_cast<int64_t>(n0 + tid % 16) * K};
    f32x4 acc[1];
    float ss;
    rows_mfma<1>(a, a_st, M, K, wrow, wave, acc, ss);
    rows_reduce<1>(red, acc, ss, wave, false, y, nullptr);
    if (tid < M * 16) {
        const int m = tid / 16, c = tid % 16;
        const int64_t col = n0 + c;
        const float rv = __builtin_bit_cast(float, static_cast<uint32_t>(res[m * res_st + col]) << 16);
        out[m * out_st + col] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(rv + bf16_round(y[0][m][c])));
    }
}

int launch_ffn_decode(const void* x, int64_t x_st, const void* w_gate_up, const void* w_down, int64_t M,
                      int64_t C, int64_t F, float eps, void* act, void* out, int64_t out_st, hipStream_t stream,
                      const PrefetchDev* pf_gate_up, const PrefetchDev* pf_down, int64_t pf_groups,
                      const int64_t* pos_dev) {
    const int n_gu = static_cast<int>(F / 16), n_dn = static_cast<int>(C / 16);
    const PrefetchDev none{};
    hipLaunchKernelGGL(ffn_gate_up_kernel,
                       dim3(static_cast<unsigned>(n_gu + (pf_gate_up != nullptr ? pf_groups : 0))),
                       dim3(kFfnThreads), 0, stream, static_cast<const uint16_t*>(x), x_st,
                       static_cast<const uint16_t*>(w_gate_up), static_cast<int>(M), static_cast<int>(C),
                       static_cast<int>(F), eps, static_cast<uint16_t*>(act), n_gu,
                       pf_gate_up != nullptr ? *pf_gate_up : none, pos_dev);
    int rc = check_hip(hipGetLastError(), "ffn_gate_up_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(ffn_down_kernel, dim3(static_cast<unsigned>(n_dn + (pf_down != nullptr ? pf_groups : 0))),
                       dim3(kFfnThreads), 0, stream, static_cast<const uint16_t*>(act), F,
                       static_cast<const uint16_t*>(w_down), static_cast<int>(M), static_cast<int>(F),
                       static_cast<int>(C), static_cast<const uint16_t*>(x), x_st, static_cast<uint16_t*>(out),
                       out_st, n_dn, pf_down != nullptr ? *pf_down : none, pos_dev);
    return check_hip(hipGetLastError(), "ffn_down_kernel");
}

// grid N/16: out[m, n] = bf16((x[m, :] . W'[n, :]) / rms(x[m])), W' [N, C] with the
// norm weight folded into its columns: the final RMSNorm and the output
// projection of a decode step in one launch
__global__ void __launch_bounds__(kFfnThreads)
norm_gemv_kernel(const uint16_t* __restrict__ x, int64_t x_st, const uint16_t* __restrict__ w, int M, int C,
                 float eps, uint16_t* __restrict__ out, int64_t out_st) {
    __shared__ RowsRed<1> red;
    __shared__ float y[1][kRowsMaxM][16];
    __shared__ float rs[16];
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;
    const uint16_t* wrow[1] = {w + (n0 + tid % 16) * C};
    f32x4 acc[1];
    float ss;
    rows_mfma<1>(x, x_st, M, C, wrow, wave, acc, ss);
    rows_reduce<1>(red, acc, ss, wave, true, y, rs);
    if (tid < M * 16) {
        const int m = tid / 16, c = tid % 16;
        const float v = y[0][m][c] / __builtin_sqrtf(rs[m] / static_cast<float>(C) + eps);
        out[m * out_st + n0 + c] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
    }
}

int launch_norm_gemv(const void* x, int64_t x_st, const void* w, int64_t M, int64_t C, int64_t N, float eps,
                     void* out, int64_t out_st, hipStream_t stream) {
    hipLaunchKernelGGL(norm_gemv_kernel, dim3(static_cast<unsigned>(N / 16)), dim3(kFfnThreads), 0, stream,
                       static_cast<const uint16_t*>(x), x_st,
                       static_cast<const uint16_t*>(w), static_cast<int>(M), static_cast<int>(C), eps,
                       static_cast<uint16_t*>(out), out_st);
    return check_hip(hipGetLastError(), "norm_gemv_kernel");
}

int launch_rows_residual(const void* a, int64_t a_st, const void* w, int64_t M, int64_t K, int64_t N,
                         const void* res, int64_t res_st, void* out, int64_t out_st, hipStream_t stream) {
    hipLaunchKernelGGL(ffn_down_kernel, dim3(static_cast<unsigned>(N / 16)), dim3(kFfnThreads), 0, stream,
                       static_cast<const uint16_t*>(a), a_st,
                       static_cast<const uint16_t*>(w), static_cast<int>(M), static_cast<int>(K),
                       static_cast<int>(N), static_cast<const uint16_t*>(res), res_st, static_cast<uint16_t*>(out),
                       out_st, static_cast<int>(N / 16), PrefetchDev{}, nullptr);
    return check_hip(hipGetLastError(), "ffn_down_kernel");
}

}  // namespace sparda
