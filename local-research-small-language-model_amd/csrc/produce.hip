// Producer of a layer's attention inputs: RMSNorm + the q / k / v / forecast
// projections + RoPE in one kernel (model/transformer.py:104-107 with
// model/norm.py:15-21, model/forecast.py:30-40, the projections of
// model/attention/base.py:38-52 and model/rope.py:34-65).
//
//   y[m, n] = (sum_c x[m, c] * W'[n, c]) / rms(x[m, :]),  W'[n, c] = W[n, c] * w_norm[c]
//
// W' stacks the q, k, v and forecast weights ([Hq*D; Hkv*D; Hkv*D; Hf*Df] rows,
// the RMSNorm weight folded into its columns by the caller), so the norm is a
// per-row scale applied after the product. rms is accumulated in fp32 from the
// A fragments the product streams anyway. q and k columns are rotated in the
// epilogue (pairs (i, i + D/2) of a head, fp32 cos / sin tables), and every
// region is written in its own [M, heads * D] layout.
//
// Tiling (D = 64): a 256-thread workgroup computes a 128 x 128 tile of y, each
// wavefront 64 x 64 = one head of one region, as 4 x 4 tiles of
// v_mfma_f32_16x16x32_bf16. A and B (rows of x and of W', both row-major over
// c) are staged per 32-wide step of c in LDS, the next step in flight in
// registers. In the MFMA result layout lane l holds column l % 16 of a tile, so
// the rotation partner of column i (i + 32 or i - 32) is in the same lane, two
// tiles away.
#include "common.h"
#include "kernels.h"
#include "mfma.h"
#include "rows.h"

namespace sparda {

constexpr int kPBM = 128;          // rows of y per workgroup
constexpr int kPBN = 128;          // columns of y per workgroup
constexpr int kPBK = 32;           // reduction step
constexpr int kPRow = kPBK + 8;    // LDS row (bf16 elements): 80 B, 16-B aligned
constexpr int kPThreads = 256;

struct ProduceSmem {
    uint16_t a[2][kPBM * kPRow];
    uint16_t b[2][kPBN * kPRow];
    float inv_rms[kPBM];
};

template <int ODT>
__device__ __forceinline__ void store_out(void* out, int64_t i, float v) {
    if constexpr (ODT == SPARDA_F32) {
        static_cast<float*>(out)[i] = v;
    } else {
        static_cast<__bf16*>(out)[i] = static_cast<__bf16>(v);
    }
}

template <int FDT>
__global__ void __launch_bounds__(kPThreads, 2)
produce_kernel(const uint16_t* __restrict__ x, int64_t x_st, const uint16_t* __restrict__ w,
               int64_t M, int C, int Nq, int Nk, int Nf, float eps,
               const float* __restrict__ cosv, const float* __restrict__ sinv, int64_t T, int64_t pos0,
               uint16_t* __restrict__ q, uint16_t* __restrict__ k, uint16_t* __restrict__ v,
               void* __restrict__ f, const int64_t* __restrict__ pos_dev, int64_t rope_len) {
    __shared__ ProduceSmem sm;
    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int wave = tid / kWave;
    const int col16 = lane % 16;
    const int grp = lane / 16;
    const int wm = wave / 2, wn = wave % 2;          // 2 x 2 wavefronts of 64 x 64
    const int64_t m0 = static_cast<int64_t>(blockIdx.x) * kPBM;
    const int n0 = blockIdx.y * kPBN;

    // staging: 128 rows x 32 c = 512 chunks of 16 B per operand, two per thread
    const int r_lo = tid / 4, r_hi = tid / 4 + 64, cc = (tid % 4) * 8;
    int64_t ra_lo = m0 + r_lo, ra_hi = m0 + r_hi;
    ra_lo = ra_lo < M ? ra_lo : M - 1;                // rows past M repeat row M-1 (not stored)
    ra_hi = ra_hi < M ? ra_hi : M - 1;
    const uint16_t* xa_lo = x + ra_lo * x_st + cc;
    const uint16_t* xa_hi = x + ra_hi * x_st + cc;
    const uint16_t* wb_lo = w + static_cast<int64_t>(n0 + r_lo) * C + cc;
    const uint16_t* wb_hi = w + static_cast<int64_t>(n0 + r_hi) * C + cc;
    uint4 a_lo = *reinterpret_cast<const uint4*>(xa_lo);
    uint4 a_hi = *reinterpret_cast<const uint4*>(xa_hi);
    uint4 b_lo = *reinterpret_cast<const uint4*>(wb_lo);
    uint4 b_hi = *reinterpret_cast<const uint4*>(wb_hi);

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    float ss[4] = {0.f, 0.f, 0.f, 0.f};  // sum of squares of row 16*tm + col16 (this lane's k slice)

    const int steps = C / kPBK;
    for (int st = 0; st < steps; ++st) {
        const int buf = st & 1;
        *reinterpret_cast<uint4*>(&sm.a[buf][r_lo * kPRow + cc]) = a_lo;
        *reinterpret_cast<uint4*>(&sm.a[buf][r_hi * kPRow + cc]) = a_hi;
        *reinterpret_cast<uint4*>(&sm.b[buf][r_lo * kPRow + cc]) = b_lo;
        *reinterpret_cast<uint4*>(&sm.b[buf][r_hi * kPRow + cc]) = b_hi;
        __syncthreads();
        if (st + 1 < steps) {
            const int c1 = (st + 1) * kPBK;
            a_lo = *reinterpret_cast<const uint4*>(xa_lo + c1);
            a_hi = *reinterpret_cast<const uint4*>(xa_hi + c1);
            b_lo = *reinterpret_cast<const uint4*>(wb_lo + c1);
            b_hi = *reinterpret_cast<const uint4*>(wb_hi + c1);
        }
        bf16x8 af[4], bfr[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            af[t] = lds_read8(&sm.a[buf][(64 * wm + 16 * t + col16) * kPRow + 8 * grp]);
            bfr[t] = lds_read8(&sm.b[buf][(64 * wn + 16 * t + col16) * kPRow + 8 * grp]);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float xv = static_cast<float>(af[t][e]);
                ss[t] = __builtin_fmaf(xv, xv, ss[t]);
            }
        }
#pragma unroll
        for (int tm = 0; tm < 4; ++tm)
#pragma unroll
            for (int tn = 0; tn < 4; ++tn)
                acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[tm], bfr[tn], acc[tm][tn], 0, 0, 0);
        // the buffer written next step was last read before this step's barrier
    }

    // 1/rms of the workgroup's rows: the 4 lane groups hold disjoint c slices
    if (wn == 0) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float s = pair32_sum(pair16_sum(ss[t]));
            if (grp == 0) sm.inv_rms[64 * wm + 16 * t + col16] = 1.0f / __builtin_sqrtf(s / static_cast<float>(C) + eps);
        }
    }
    __syncthreads();

    // epilogue: this wavefront's 64 columns are one head of one region
    const int nh = n0 + 64 * wn;                     // first column of the head
    const int Nv = Nk;
    int region, head;
    if (nh < Nq) { region = 0; head = nh / 64; }
    else if (nh < Nq + Nk) { region = 1; head = (nh - Nq) / 64; }
    else if (nh < Nq + Nk + Nv) { region = 2; head = (nh - Nq - Nk) / 64; }
    else { region = 3; head = (nh - Nq - Nk - Nv) / 64; }
    const int ld = region == 0 ? Nq : (region == 3 ? Nf : Nk);  // row stride of the output
    const int64_t t_first = m0 % T;                  // position of row m0 within its sequence
    // a device-held offset (a decode step at token *pos_dev): positions clamped into the tables
    const int64_t pos_base = pos0 + (pos_dev != nullptr ? *pos_dev : 0);
    const int64_t pos_hi = pos_dev != nullptr ? rope_len - 1 : INT64_MAX;
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rloc = 64 * wm + 16 * tm + 4 * grp + i;
            const int64_t m = m0 + rloc;
            if (m >= M) continue;
            const float sc = sm.inv_rms[rloc];
            int64_t t = t_first + rloc;
            while (t >= T) t -= T;
            int64_t pos = pos_base + t;
            pos = pos < 0 ? 0 : (pos > pos_hi ? pos_hi : pos);
            float y[4];
#pragma unroll
            for (int tn = 0; tn < 4; ++tn) y[tn] = acc[tm][tn][i] * sc;
            if (region <= 1) {
                // columns d = 16*tn + col16: pairs (d, d + 32) are tiles (0, 2) and (1, 3)
#pragma unroll
                for (int tn = 0; tn < 2; ++tn) {
                    const int d = 16 * tn + col16;
                    const float c = cosv[pos * 32 + d], s = sinv[pos * 32 + d];
                    const float x1 = y[tn], x2 = y[tn + 2];
                    y[tn] = x1 * c - x2 * s;
                    y[tn + 2] = x2 * c + x1 * s;
                }
            }
            const int64_t base = m * ld + 64 * head + col16;
#pragma unroll
            for (int tn = 0; tn < 4; ++tn) {
                if (region == 0) store_out<SPARDA_BF16>(q, base + 16 * tn, y[tn]);
                else if (region == 1) store_out<SPARDA_BF16>(k, base + 16 * tn, y[tn]);
                else if (region == 2) store_out<SPARDA_BF16>(v, base + 16 * tn, y[tn]);
                else store_out<FDT>(f, base + 16 * tn, y[tn]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Decode shapes (M <= kRowsMaxM rows, a few tokens): the tiled kernel would
// run N/128 workgroups and stream all of W' through a dozen CUs. Here a
// workgroup owns 16 columns of one head (8 RoPE pairs: d0+p and d0+p+32,
// p < 8), so N/16 workgroups share the weight read; the 16 columns' rows of W'
// are the A operand of matrix-core products with the x rows (rows.h), which
// also yield sum(x^2) for 1/rms. Results go through LDS to the threads that
// rotate and store the pairs.
// ---------------------------------------------------------------------------
template <int FDT>
__global__ void __launch_bounds__(kPThreads)
produce_rows_kernel(const uint16_t* __restrict__ x, int64_t x_st, const uint16_t* __restrict__ w, int M, int C,
                    int Nq, int Nk, int Nf, float eps, const float* __restrict__ cosv,
                    const float* __restrict__ sinv, int64_t T, int64_t pos0, uint16_t* __restrict__ q,
                    uint16_t* __restrict__ k, uint16_t* __restrict__ v, void* __restrict__ f,
                    const int64_t* __restrict__ pos_dev, int64_t rope_len, uint16_t* __restrict__ kc,
                    uint16_t* __restrict__ vc, int64_t c_sb, int64_t c_st, int64_t c_sh, int64_t cap) {
    static_assert(kPThreads == kRowsWaves * kWave, "one rows_mfma workgroup");
    __shared__ RowsRed<1> red;
    __shared__ float ylds[1][kRowsMaxM][16];
    __shared__ float rs[16];
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int nh = (blockIdx.x / 4) * 64;            // first column of the head
    const int d0 = (blockIdx.x % 4) * 8;
    // local column lc = tile row: pair lc/2, half lc%2
    const int lr = tid % 16;
    const uint16_t* wrow[1] = {w + static_cast<int64_t>(nh + d0 + lr / 2 + 32 * (lr % 2)) * C};
    f32x4 acc[1];
    float ss;
    rows_mfma<1>(x, x_st, M, C, wrow, wave, acc, ss);
    rows_reduce<1>(red, acc, ss, wave, true, ylds, rs);
    if (tid < M * 16) {
        const int m = tid / 16, c = tid % 16;
        ylds[0][m][c] = ylds[0][m][c] / __builtin_sqrtf(rs[m] / static_cast<float>(C) + eps);
    }
    __syncthreads();

    const int Nv = Nk;
    int region, head;
    if (nh < Nq) { region = 0; head = nh / 64; }
    else if (nh < Nq + Nk) { region = 1; head = (nh - Nq) / 64; }
    else if (nh < Nq + Nk + Nv) { region = 2; head = (nh - Nq - Nk) / 64; }
    else { region = 3; head = (nh - Nq - Nk - Nv) / 64; }
    const int ld = region == 0 ? Nq : (region == 3 ? Nf : Nk);
    const int64_t pos_base = pos0 + (pos_dev != nullptr ? *pos_dev : 0);
    const int64_t pos_hi = pos_dev != nullptr ? rope_len - 1 : INT64_MAX;
    for (int t = tid; t < M * 8; t += kPThreads) {
        const int m = t / 8, p = t % 8;
        float y1 = ylds[0][m][2 * p], y2 = ylds[0][m][2 * p + 1];
        const int d = d0 + p;
        if (region <= 1) {
            int64_t pos = pos_base + m % T;
            pos = pos < 0 ? 0 : (pos > pos_hi ? pos_hi : pos);
            const float c = cosv[pos * 32 + d], sn = sinv[pos * 32 + d];
            const float r1 = y1 * c - y2 * sn;
            const float r2 = y2 * c + y1 * sn;
            y1 = r1;
            y2 = r2;
        }
        const int64_t base = static_cast<int64_t>(m) * ld + 64 * head + d;
        if (region == 0) { store_out<SPARDA_BF16>(q, base, y1); store_out<SPARDA_BF16>(q, base + 32, y2); }
        else if (region == 1) { store_out<SPARDA_BF16>(k, base, y1); store_out<SPARDA_BF16>(k, base + 32, y2); }
        else if (region == 2) { store_out<SPARDA_BF16>(v, base, y1); store_out<SPARDA_BF16>(v, base + 32, y2); }
        else { store_out<FDT>(f, base, y1); store_out<FDT>(f, base + 32, y2); }
        if (kc != nullptr && (region == 1 || region == 2)) {
            // the new key / value also as row p of sequence m / T in the caches
            int64_t p = pos_base + m % T;
            p = p < 0 ? 0 : (p > cap - 1 ? cap - 1 : p);
            const int64_t ci = (m / T) * c_sb + p * c_st + head * c_sh + d;
            uint16_t* dst = region == 1 ? kc : vc;
            store_out<SPARDA_BF16>(dst, ci, y1);
            store_out<SPARDA_BF16>(dst, ci + 32, y2);
        }
    }
}

int launch_produce(const void* x, int64_t x_st, const void* w, int64_t M, int64_t C, int64_t Nq, int64_t Nk,
                   int64_t Nf, float eps, const float* cosv, const float* sinv, int64_t T, int64_t pos0,
                   void* q, void* k, void* v, void* f, int f_dtype, hipStream_t stream,
                   const int64_t* pos_dev, int64_t rope_len, void* kc, void* vc, int64_t c_sb, int64_t c_st,
                   int64_t c_sh, int64_t cap) {
    const int64_t N = Nq + 2 * Nk + Nf;
    if (M <= kRowsMaxM && C % 128 == 0 && C / 128 <= kRowsWaves * kRowsMaxKB) {
        const size_t lds = 0;
#define SPARDA_PRODUCE_ROWS(FDT_)                                                                            \
    hipLaunchKernelGGL((produce_rows_kernel<FDT_>), dim3(static_cast<unsigned>(N / 16)), dim3(kPThreads), lds, \
                       stream, static_cast<const uint16_t*>(x), x_st, static_cast<const uint16_t*>(w),        \
                       static_cast<int>(M), static_cast<int>(C), static_cast<int>(Nq), static_cast<int>(Nk),  \
                       static_cast<int>(Nf), eps, cosv, sinv, T, pos0, static_cast<uint16_t*>(q),             \
                       static_cast<uint16_t*>(k), static_cast<uint16_t*>(v), f, pos_dev, rope_len,             \
                       static_cast<uint16_t*>(kc), static_cast<uint16_t*>(vc), c_sb, c_st, c_sh, cap)
        if (f_dtype == SPARDA_F32) SPARDA_PRODUCE_ROWS(SPARDA_F32);
        else SPARDA_PRODUCE_ROWS(SPARDA_BF16);
#undef SPARDA_PRODUCE_ROWS
        return check_hip(hipGetLastError(), "produce_rows_kernel");
    }
    if (kc != nullptr) return set_error(SPARDA_ERR_SHAPE, "produce: cache rows are written for M <= %d only",
                                        kRowsMaxM);
    dim3 grid(static_cast<unsigned>(cdiv(M, kPBM)), static_cast<unsigned>(N / kPBN));
#define SPARDA_PRODUCE(FDT_)                                                                              \
    hipLaunchKernelGGL((produce_kernel<FDT_>), grid, dim3(kPThreads), 0, stream,                          \
                       static_cast<const uint16_t*>(x), x_st, static_cast<const uint16_t*>(w), M,        \
                       static_cast<int>(C), static_cast<int>(Nq), static_cast<int>(Nk),                   \
                       static_cast<int>(Nf), eps, cosv, sinv, T, pos0, static_cast<uint16_t*>(q),         \
                       static_cast<uint16_t*>(k), static_cast<uint16_t*>(v), f, pos_dev, rope_len)
    if (f_dtype == SPARDA_F32) SPARDA_PRODUCE(SPARDA_F32);
    else SPARDA_PRODUCE(SPARDA_BF16);
#undef SPARDA_PRODUCE
    return check_hip(hipGetLastError(), "produce_kernel");
}

}  // namespace sparda
