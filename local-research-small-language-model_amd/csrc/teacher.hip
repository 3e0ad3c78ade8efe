// Teacher block mass for routing-quality evaluation (model/forecast.py:133-193,
// TeacherBlockSelector): the dense attention probability of every query row on
// every KV block, averaged over the query heads of a KV head,
//
//   mass[b, g, t, j] = (1/R) sum_{h in g} sum_{s in block j} softmax_s(q[b,t,h] . k[b,s,g] / sqrt(D))
//
// (causal: keys s <= t, blocks j > t / bs get 0), without materialising the
// [B, Hq, T, T] weights the reference builds. bf16 inputs, D = 64, bs = 64.
//
// One workgroup (4 wavefronts) per (b, g, query block of 64 tokens); wavefront
// w owns tokens 16w .. 16w+15 for all R heads as R tiles of 16 columns (column
// c -> token c / R, head c % R), like the sparse prefill. K blocks are staged in
// LDS (double-buffered, the next block in flight in registers) and shared by
// the four wavefronts; S^T = K Q^T per block and tile with
// v_mfma_f32_16x16x32_bf16. Pass 1 walks the blocks for every column's max and
// sum of exponentials (fp32, log2 domain); pass 2 walks them again and sums the
// normalised probabilities of each block per column in fp32; the R columns of a
// token are averaged through the wavefront's LDS slot and written as one value.
#include "common.h"
#include "kernels.h"
#include "mfma.h"

namespace sparda {

constexpr int kTBs = 64;           // block size
constexpr int kTD = 64;            // head dim
constexpr int kTThreads = 256;
constexpr int kTKRow = kTD + 8;    // K row in LDS (bf16 elements, 144 B)

template <int R>
struct TeacherSmem {
    uint16_t k[2][kTBs * kTKRow];
    float colmass[4][16 * R];      // per wavefront: the block mass of each column
};

template <int R>
__global__ void __launch_bounds__(kTThreads, 2)
teacher_mass_kernel(const uint16_t* __restrict__ q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                    const uint16_t* __restrict__ k, int64_t k_sb, int64_t k_st, int64_t k_sh,
                    int64_t T, int H, int64_t NBq, int64_t NB, int causal, float scale_log2,
                    float* __restrict__ mass) {
    __shared__ TeacherSmem<R> sm;
    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int wave = tid / kWave;
    const int col16 = lane % 16;
    const int grp = lane / 16;
    // heaviest query blocks first
    const int64_t BH = static_cast<int64_t>(gridDim.x) / NBq;
    const int64_t bg = blockIdx.x % BH;
    const int64_t qb = NBq - 1 - blockIdx.x / BH;
    const int b = static_cast<int>(bg / H);
    const int g = static_cast<int>(bg % H);
    const int64_t t0 = qb * kTBs;
    const int64_t jmax = causal ? qb : NB - 1;

    // Q operands of this wavefront's tiles, straight from memory
    int tok[R];
    bf16x8 qreg[R][2];
#pragma unroll
    for (int tt = 0; tt < R; ++tt) {
        const int c = 16 * tt + col16;
        tok[tt] = 16 * wave + c / R;
        int64_t t = t0 + tok[tt];
        t = t < T ? t : T - 1;
        const uint16_t* qp = q + b * q_sb + t * q_st + static_cast<int64_t>(g * R + c % R) * q_sh + 8 * grp;
        qreg[tt][0] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(qp));
        qreg[tt][1] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(qp + 32));
    }

    // K staging: chunk c = tid, tid + 256 -> row c / 8, 16-byte chunk c % 8
    const uint16_t* kbase = k + b * k_sb + static_cast<int64_t>(g) * k_sh;
    const int c_lo = tid, c_hi = tid + kTThreads;
    const int lds_lo = (c_lo / 8) * kTKRow + (c_lo % 8) * 8, lds_hi = (c_hi / 8) * kTKRow + (c_hi % 8) * 8;
    auto fetch = [&](int64_t j, uint4& lo, uint4& hi) {
        int64_t s_lo = j * kTBs + c_lo / 8, s_hi = j * kTBs + c_hi / 8;
        s_lo = s_lo < T ? s_lo : T - 1;  // rows past T repeat row T-1 (masked)
        s_hi = s_hi < T ? s_hi : T - 1;
        lo = *reinterpret_cast<const uint4*>(kbase + s_lo * k_st + (c_lo % 8) * 8);
        hi = *reinterpret_cast<const uint4*>(kbase + s_hi * k_st + (c_hi % 8) * 8);
    };

    // S^T of block j for tile tt, masked keys at -inf
    auto scores = [&](int buf, int64_t j, int tt, f32x4 (&s)[4]) {
        bf16x8 ka[4][2];
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
                ka[n][kk] = lds_read8(&sm.k[buf][(16 * n + col16) * kTKRow + 32 * kk + 8 * grp]);
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            s[n] = f32x4{0.f, 0.f, 0.f, 0.f};
            s[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[n][0], qreg[tt][0], s[n], 0, 0, 0);
            s[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[n][1], qreg[tt][1], s[n], 0, 0, 0);
        }
        // causal diagonal: key <= token; any block: key < T
        const int64_t lim_t = T - 1 - j * kTBs;
        const int64_t lim = (causal && j == qb) ? (tok[tt] < lim_t ? tok[tt] : lim_t) : lim_t;
        if (lim < kTBs - 1) {
#pragma unroll
            for (int n = 0; n < 4; ++n)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (16 * n + 4 * grp + i > lim) s[n][i] = -__builtin_inff();
        }
    };

    float m[R], l[R];
#pragma unroll
    for (int tt = 0; tt < R; ++tt) {
        m[tt] = -__builtin_inff();
        l[tt] = 0.0f;
    }

    for (int pass = 0; pass < 2; ++pass) {
        uint4 ka_lo, ka_hi;
        fetch(0, ka_lo, ka_hi);
        __syncthreads();  // the previous pass has read its last buffer
        *reinterpret_cast<uint4*>(&sm.k[0][lds_lo]) = ka_lo;
        *reinterpret_cast<uint4*>(&sm.k[0][lds_hi]) = ka_hi;
        if (jmax >= 1) fetch(1, ka_lo, ka_hi);
        __syncthreads();
        for (int64_t j = 0; j <= jmax; ++j) {
            const int buf = static_cast<int>(j & 1);
#pragma unroll
            for (int tt = 0; tt < R; ++tt) {
                f32x4 s[4];
                scores(buf, j, tt, s);
                if (pass == 0) {
                    float mx = pair32_max(pair16_max(max16_nn(s))) * scale_log2;
                    const float m_new = __builtin_fmaxf(m[tt], mx);
                    float acc = 0.0f;
#pragma unroll
                    for (int n = 0; n < 4; ++n)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            acc += __builtin_amdgcn_exp2f(__builtin_fmaf(s[n][i], scale_log2, -m_new));
                    acc = pair32_sum(pair16_sum(acc));
                    l[tt] = l[tt] * (m_new == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m[tt] - m_new)) + acc;
                    m[tt] = m_new;
                } else {
                    float acc = 0.0f;
#pragma unroll
                    for (int n = 0; n < 4; ++n)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            acc += __builtin_amdgcn_exp2f(__builtin_fmaf(s[n][i], scale_log2, -m[tt]));
                    acc = pair32_sum(pair16_sum(acc));
                    if (grp == 0) sm.colmass[wave][16 * tt + col16] = acc / l[tt];
                }
            }
            if (pass == 1 && lane < 16) {
                // average of the R head columns of token 16*wave + lane
                float v = 0.0f;
#pragma unroll
                for (int hh = 0; hh < R; ++hh) v += sm.colmass[wave][R * lane + hh];
                const int64_t t = t0 + 16 * wave + lane;
                if (t < T) mass[((static_cast<int64_t>(b) * H + g) * T + t) * NB + j] = v / static_cast<float>(R);
            }
            if (j + 1 <= jmax) {
                *reinterpret_cast<uint4*>(&sm.k[buf ^ 1][lds_lo]) = ka_lo;
                *reinterpret_cast<uint4*>(&sm.k[buf ^ 1][lds_hi]) = ka_hi;
                if (j + 2 <= jmax) fetch(j + 2, ka_lo, ka_hi);
            }
            __syncthreads();
        }
    }
    // blocks past the causal limit carry no probability
    if (jmax + 1 < NB && lane < 16) {
        const int64_t t = t0 + 16 * wave + lane;
        if (t < T) {
            float* row = mass + ((static_cast<int64_t>(b) * H + g) * T + t) * NB;
            for (int64_t j = jmax + 1; j < NB; ++j) row[j] = 0.0f;
        }
    }
}

int launch_teacher_mass(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k, int64_t k_sb,
                        int64_t k_st, int64_t k_sh, int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int causal,
                        float scale, float* mass, hipStream_t stream) {
    const int64_t NBq = cdiv(T, kTBs);
    const int64_t NB = NBq;
    const float scale_log2 = scale * 1.4426950408889634f;
    dim3 grid(static_cast<unsigned>(B * Hkv * NBq));
    const int R = static_cast<int>(Hq / Hkv);
#define SPARDA_TEACHER(R_)                                                                                  \
    hipLaunchKernelGGL((teacher_mass_kernel<R_>), grid, dim3(kTThreads), 0, stream,                         \
                       static_cast<const uint16_t*>(q), q_sb, q_st, q_sh, static_cast<const uint16_t*>(k),  \
                       k_sb, k_st, k_sh, T, static_cast<int>(Hkv), NBq, NB, causal, scale_log2, mass)
    switch (R) {
        case 1: SPARDA_TEACHER(1); break;
        case 2: SPARDA_TEACHER(2); break;
        case 3: SPARDA_TEACHER(3); break;
        default: return set_error(SPARDA_ERR_SHAPE, "teacher_mass: Hq/Hkv = %d not in {1, 2, 3}", R);
    }
#undef SPARDA_TEACHER
    return check_hip(hipGetLastError(), "teacher_mass_kernel");
}

}  // namespace sparda
