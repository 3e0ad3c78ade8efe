// Block-sparse GQA prefill: dispatch and the general VALU kernel.
//
// The general kernel covers every supported shape and dtype (fp32 inputs,
// head dims 16..128, any block size, any GQA ratio up to 16). One workgroup
// serves one (sequence, KV head, query token): it walks the token's selected
// blocks, stages each block's keys/values of that KV head in LDS once and runs
// the online softmax for all Hq/Hkv query heads of the group, one wavefront
// per head. bf16 inputs with D = 64 take the MFMA kernel instead.
#include "common.h"
#include "kernels.h"
#include "attend.h"

namespace sparda {

constexpr float kLog2eP = 1.4426950408889634f;
constexpr int kPrefillThreads = 256;
constexpr int kPrefillWaves = kPrefillThreads / kWave;
constexpr int kPrefillMaxGroup = 16;

template <int DT, int DH>
__global__ void __launch_bounds__(kPrefillThreads)
prefill_general_kernel(const void* __restrict__ q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                       const void* __restrict__ k, const void* __restrict__ v,
                       int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                       const int32_t* __restrict__ sel, const int32_t* __restrict__ n_sel, int64_t cap,
                       int64_t T, int Hq, int H, int bs, int causal, float scale_log2,
                       void* __restrict__ out, int64_t out_sb, int64_t out_st) {
    constexpr int KS = DH + 1;
    __shared__ float k_lds[kChunkKeys * KS];
    __shared__ float v_lds[kChunkKeys * KS];
    __shared__ float q_lds[kPrefillMaxGroup * DH];
    __shared__ float p_lds[kPrefillWaves][kChunkKeys];

    const int64_t t = blockIdx.x;
    const int g = blockIdx.y;
    const int b = blockIdx.z;
    const int R = Hq / H;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int64_t NB = cdiv(T, bs);
    const int64_t row = (static_cast<int64_t>(b) * H + g) * T + t;
    const int64_t limit = causal ? t + 1 : T;  // keys [0, limit)

    int n;
    if (sel == nullptr) {
        n = static_cast<int>(causal ? t / bs + 1 : NB);
    } else {
        n = n_sel[row] < cap ? n_sel[row] : static_cast<int>(cap);
    }

    for (int e = threadIdx.x; e < R * DH; e += kPrefillThreads) {
        const int hh = e / DH, d = e % DH;
        q_lds[e] = load_elem<DT>(q, b * q_sb + t * q_st + static_cast<int64_t>(g * R + hh) * q_sh + d) *
                   scale_log2;
    }
    constexpr int MAXR = kPrefillMaxGroup / kPrefillWaves;
    HeadAcc<DH> acc[MAXR];
#pragma unroll
    for (int r = 0; r < MAXR; ++r) acc[r].init();

    for (int i = 0; i < n; ++i) {
        const int64_t j = sel == nullptr ? i : sel[row * cap + i];
        if (j < 0 || j >= NB) continue;
        const int64_t s0 = j * bs;
        int64_t s1 = s0 + bs;
        if (s1 > limit) s1 = limit;
        for (int64_t c0 = s0; c0 < s1; c0 += kChunkKeys) {
            const int nk = static_cast<int>((s1 - c0) < kChunkKeys ? (s1 - c0) : kChunkKeys);
            __syncthreads();
            for (int e = threadIdx.x; e < nk * DH; e += kPrefillThreads) {
                const int kk = e / DH, d = e % DH;
                const int64_t src = b * kv_sb + (c0 + kk) * kv_st + g * kv_sh + d;
                k_lds[kk * KS + d] = load_elem<DT>(k, src);
                v_lds[kk * KS + d] = load_elem<DT>(v, src);
            }
            __syncthreads();
#pragma unroll
            for (int r = 0; r < MAXR; ++r) {
                const int hh = wave + r * kPrefillWaves;
                if (hh < R)
                    attend_chunk<DH, KS>(q_lds + hh * DH, k_lds, v_lds, nk, p_lds[wave], acc[r],
                                         [](int) { return true; });
            }
        }
    }

#pragma unroll
    for (int r = 0; r < MAXR; ++r) {
        const int hh = wave + r * kPrefillWaves;
        if (hh >= R) continue;
        const int h = g * R + hh;
        const float inv = 1.0f / acc[r].l;
#pragma unroll
        for (int i = 0; i < HeadAcc<DH>::DPL; ++i) {
            const int d = lane + i * kWave;
            if (d < DH) store_elem<DT>(out, b * out_sb + t * out_st + static_cast<int64_t>(h) * DH + d, acc[r].o[i] * inv);
        }
    }
}

int launch_prefill_mfma(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k,
                        const void* v, int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                        const int32_t* sel, const int32_t* n_sel, int64_t cap, int64_t B, int64_t T,
                        int64_t Hq, int64_t Hkv, int64_t bs, int causal, float scale, void* out,
                        int64_t out_sb, int64_t out_st, hipStream_t stream);
bool prefill_mfma_supported(int dtype, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t bs,
                            int64_t q_sb, int64_t q_st, int64_t q_sh, int64_t kv_sb, int64_t kv_st,
                            int64_t kv_sh, int64_t out_sb, int64_t out_st, const void* q, const void* k,
                            const void* v, const void* out);

// ---------------------------------------------------------------------------
// Masked prefill with optional attention weights (the reference's masked SDPA
// with an explicit additive mask and return_attn_weights, sparse.py:206-221,
// 255-281). One workgroup per (query token t, KV head g, sequence b), one
// wavefront per query head of the group (heads w, w+4, ...). The row's
// allowed keys are its listed blocks (or every block), keys <= t when causal;
// the additive mask is added to each allowed score. Pass 1 forms the row
// maximum and the sum of exponentials, pass 2 the normalised probabilities:
// written to `weights` (zeros elsewhere in the row) and accumulated into the
// output. Scores in log2 units: q * scale * log2 e . k + mask * log2 e.
// ---------------------------------------------------------------------------
constexpr int kWMaxList = 64;  // distinct listed blocks per row (selection capacity <= 34)

template <int DT, int DH>
__global__ void __launch_bounds__(kPrefillThreads)
prefill_weights_kernel(const void* __restrict__ q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                       const void* __restrict__ k, const void* __restrict__ v,
                       int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                       const int32_t* __restrict__ sel, const int32_t* __restrict__ n_sel, int64_t cap,
                       int64_t T, int Hq, int H, int bs, int causal, float scale_log2,
                       const void* __restrict__ mask, int mask_dt, int64_t m_sb, int64_t m_sh, int64_t m_st,
                       int64_t m_ss, void* __restrict__ out, int64_t out_sb, int64_t out_st,
                       void* __restrict__ weights, int64_t w_sb, int64_t w_sh, int64_t w_st) {
    constexpr int KS = DH + 1;
    __shared__ float k_lds[kChunkKeys * KS];
    __shared__ float v_lds[kChunkKeys * KS];
    __shared__ float q_lds[kPrefillMaxGroup * DH];
    __shared__ float p_lds[kPrefillWaves][kChunkKeys];
    __shared__ int32_t blocks[kWMaxList];
    __shared__ int n_blocks;
    __shared__ int dead[kPrefillMaxGroup];  // query head of the group with no finite score in its row

    const int64_t t = blockIdx.x;
    const int g = blockIdx.y;
    const int b = blockIdx.z;
    const int R = Hq / H;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int64_t NB = cdiv(T, bs);
    const int64_t row = (static_cast<int64_t>(b) * H + g) * T + t;
    const int64_t limit = causal ? t + 1 : T;  // keys [0, limit)
    const float kL2e = kLog2eP;

    // the row's blocks as a set: listed entries inside [0, NB) once each
    if (threadIdx.x == 0 && sel != nullptr) {
        int n = 0;
        if (sel != nullptr) {
            const int64_t m = n_sel[row] < cap ? n_sel[row] : cap;
            for (int64_t i = 0; i < m; ++i) {
                const int32_t j = sel[row * cap + i];
                bool seen = j < 0 || j >= NB;
                for (int e = 0; e < n && !seen; ++e) seen = blocks[e] == j;
                if (!seen && n < kWMaxList) blocks[n++] = j;
            }
        }
        n_blocks = n;
    }
    for (int e = threadIdx.x; e < R * DH; e += kPrefillThreads) {
        const int hh = e / DH, d = e % DH;
        q_lds[e] = load_elem<DT>(q, b * q_sb + t * q_st + static_cast<int64_t>(g * R + hh) * q_sh + d) * scale_log2;
    }
    __syncthreads();
    const int64_t nblk = sel != nullptr ? n_blocks : NB;  // dense: every block, in order

    auto mask_at = [&](int h, int64_t s) -> float {
        if (mask == nullptr) return 0.0f;
        const int64_t mi = b * m_sb + static_cast<int64_t>(h) * m_sh + t * m_st + s * m_ss;
        return (mask_dt == SPARDA_F32 ? load_elem<SPARDA_F32>(mask, mi) : load_elem<SPARDA_BF16>(mask, mi)) * kL2e;
    };
    constexpr int MAXR = kPrefillMaxGroup / kPrefillWaves;
    float m_row[MAXR], l_row[MAXR];
    float o_acc[MAXR][HeadAcc<DH>::DPL];
#pragma unroll
    for (int r = 0; r < MAXR; ++r) {
        m_row[r] = -__builtin_inff();
        l_row[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < HeadAcc<DH>::DPL; ++i) o_acc[r][i] = 0.0f;
    }
    for (int pass = 0; pass < 2; ++pass) {
        if (pass == 1 && weights != nullptr) {
            // the weights rows: zero outside the allowed set (its entries are
            // written below), except a row with no finite score at all, which
            // is NaN throughout, as the reference's F.softmax over an all -inf
            // row gives it (sparse.py:266-268; 0/0); the output of such a row
            // is then NaN too. Without weights the reference calls SDPA, which
            // returns 0 for such a row, and so does this kernel.
#pragma unroll
            for (int r = 0; r < MAXR; ++r) {
                const int hh = wave + r * kPrefillWaves;
                if (hh < R && lane == 0) dead[hh] = l_row[r] == 0.0f;
            }
            __syncthreads();
            for (int64_t e = threadIdx.x; e < static_cast<int64_t>(R) * T; e += kPrefillThreads) {
                const int hh = static_cast<int>(e / T);
                const int64_t s = e % T;
                store_elem<DT>(weights, b * w_sb + static_cast<int64_t>(g * R + hh) * w_sh + t * w_st + s,
                               dead[hh] ? __builtin_nanf("") : 0.0f);
            }
            __syncthreads();  // the fill is ordered before the allowed entries' stores
#pragma unroll
            for (int r = 0; r < MAXR; ++r)
                if (l_row[r] == 0.0f) l_row[r] = __builtin_nanf("");  // p = x / NaN below: NaN
        }
        for (int64_t bi = 0; bi < nblk; ++bi) {
            const int64_t s0 = (sel != nullptr ? static_cast<int64_t>(blocks[bi]) : bi) * bs;
            int64_t s1 = s0 + bs;
            if (s1 > limit) s1 = limit;
            for (int64_t c0 = s0; c0 < s1; c0 += kChunkKeys) {
                const int nk = static_cast<int>((s1 - c0) < kChunkKeys ? (s1 - c0) : kChunkKeys);
                __syncthreads();
                for (int e = threadIdx.x; e < nk * DH; e += kPrefillThreads) {
                    const int kk = e / DH, d = e % DH;
                    const int64_t src = b * kv_sb + (c0 + kk) * kv_st + g * kv_sh + d;
                    k_lds[kk * KS + d] = load_elem<DT>(k, src);
                    if (pass == 1) v_lds[kk * KS + d] = load_elem<DT>(v, src);
                }
                __syncthreads();
#pragma unroll
                for (int r = 0; r < MAXR; ++r) {
                    const int hh = wave + r * kPrefillWaves;
                    if (hh >= R) continue;
                    const int h = g * R + hh;
                    float sc = -__builtin_inff();
                    if (lane < nk) {
                        float a = 0.0f;
#pragma unroll
                        for (int d = 0; d < DH; ++d) a = fmaf(q_lds[hh * DH + d], k_lds[lane * KS + d], a);
                        sc = a + mask_at(h, c0 + lane);
                    }
                    if (pass == 0) {
                        const float mc = wave_max(sc);
                        if (mc == -__builtin_inff()) continue;  // wave-uniform
                        const float m_new = fmaxf(m_row[r], mc);
                        const float p = sc == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(sc - m_new);
                        l_row[r] = l_row[r] * __builtin_amdgcn_exp2f(m_row[r] - m_new) + wave_sum(p);
                        m_row[r] = m_new;
                    } else {
                        const float p = l_row[r] != l_row[r]
                                            ? l_row[r]  // a row with no finite score, weights wanted: NaN
                                            : (sc == -__builtin_inff() ? 0.0f
                                                                       : __builtin_amdgcn_exp2f(sc - m_row[r]) / l_row[r]);
                        if (weights != nullptr && lane < nk)
                            store_elem<DT>(weights, b * w_sb + static_cast<int64_t>(h) * w_sh + t * w_st + c0 + lane, p);
                        p_lds[wave][lane] = p;
                        __builtin_amdgcn_wave_barrier();
#pragma unroll
                        for (int i = 0; i < HeadAcc<DH>::DPL; ++i) {
                            const int d = lane + i * kWave;
                            if (d < DH)
                                for (int key = 0; key < nk; ++key) o_acc[r][i] = fmaf(p_lds[wave][key], v_lds[key * KS + d], o_acc[r][i]);
                        }
                        __builtin_amdgcn_wave_barrier();
                    }
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < MAXR; ++r) {
        const int hh = wave + r * kPrefillWaves;
        if (hh >= R) continue;
        const int h = g * R + hh;
#pragma unroll
        for (int i = 0; i < HeadAcc<DH>::DPL; ++i) {
            const int d = lane + i * kWave;
            // NaN l: no finite score and weights wanted (also when no key was visited)
            const float o = l_row[r] != l_row[r] ? l_row[r] : o_acc[r][i];
            if (d < DH) store_elem<DT>(out, b * out_sb + t * out_st + static_cast<int64_t>(h) * DH + d, o);
        }
    }
}

int launch_prefill_weights(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k, const void* v,
                           int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int dtype, const int32_t* sel,
                           const int32_t* n_sel, int64_t cap, int64_t B, int64_t T, int64_t Hq, int64_t Hkv,
                           int64_t D, int64_t bs, int causal, float scale, const void* mask, int mask_dt,
                           int64_t m_sb, int64_t m_sh, int64_t m_st, int64_t m_ss, void* out, int64_t out_sb,
                           int64_t out_st, void* weights, int64_t w_sb, int64_t w_sh, int64_t w_st,
                           hipStream_t stream) {
    dim3 grid(static_cast<unsigned>(T), static_cast<unsigned>(Hkv), static_cast<unsigned>(B));
    const float sl = scale * kLog2eP;
#define SPARDA_PW(DT_, DH_)                                                                                   \
    hipLaunchKernelGGL((prefill_weights_kernel<DT_, DH_>), grid, dim3(kPrefillThreads), 0, stream, q, q_sb, q_st, \
                       q_sh, k, v, kv_sb, kv_st, kv_sh, sel, n_sel, cap, T, static_cast<int>(Hq),            \
                       static_cast<int>(Hkv), static_cast<int>(bs), causal, sl, mask, mask_dt, m_sb, m_sh, m_st,  \
                       m_ss, out, out_sb, out_st, weights, w_sb, w_sh, w_st)
#define SPARDA_PW_D(DT_)                    \
    switch (D) {                            \
        case 16: SPARDA_PW(DT_, 16); break; \
        case 32: SPARDA_PW(DT_, 32); break; \
        case 64: SPARDA_PW(DT_, 64); break; \
        default: SPARDA_PW(DT_, 128); break; \
    }
    if (dtype == SPARDA_BF16) {
        SPARDA_PW_D(SPARDA_BF16);
    } else {
        SPARDA_PW_D(SPARDA_F32);
    }
#undef SPARDA_PW_D
#undef SPARDA_PW
    return check_hip(hipGetLastError(), "prefill_weights_kernel");
}

bool prefill_compact_supported(int dtype, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t bs,
                               const int32_t* sel, int64_t cap, int64_t q_sb, int64_t q_st, int64_t q_sh,
                               int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int64_t out_sb, int64_t out_st,
                               const void* q, const void* k, const void* v, const void* out);
int launch_prefill_compact(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k,
                           const void* v, int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                           const int32_t* sel, const int32_t* n_sel, int64_t cap, int64_t B, int64_t T,
                           int64_t Hq, int64_t Hkv, int64_t bs, int causal, float scale, void* out,
                           int64_t out_sb, int64_t out_st, hipStream_t stream);

int launch_prefill(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k,
                   const void* v, int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int dtype,
                   const int32_t* sel, const int32_t* n_sel, int64_t cap, int64_t B, int64_t T,
                   int64_t Hq, int64_t Hkv, int64_t D, int64_t bs, int causal, float scale,
                   void* out, int64_t out_sb, int64_t out_st, hipStream_t stream) {
    // per-token selections: columns compacted per block; dense steps (no
    // selection lists): the dense kernel; wider selections: the
    // union-of-blocks matrix-core kernel.
    // Without lists every key up to the query (or every key) is attended, so
    // the block size does not enter the result and the 64-key kernel serves
    // any block size.
    if (sel == nullptr) bs = 64;
    // no lists: every key up to the token (or every key), the dense kernel
    if (sel == nullptr && prefill_dense_supported(dtype, Hq, Hkv, D, q_sb, q_st, q_sh, kv_sb, kv_st, kv_sh, out_sb,
                                                  out_st, q, k, v, out))
        return launch_prefill_dense(q, q_sb, q_st, q_sh, k, v, kv_sb, kv_st, kv_sh, B, T, Hq, Hkv, causal, scale,
                                    out, out_sb, out_st, stream);
    if (prefill_compact_supported(dtype, T, Hq, Hkv, D, bs, sel, cap, q_sb, q_st, q_sh, kv_sb, kv_st, kv_sh,
                                  out_sb, out_st, q, k, v, out))
        return launch_prefill_compact(q, q_sb, q_st, q_sh, k, v, kv_sb, kv_st, kv_sh, sel, n_sel, cap, B, T, Hq,
                                      Hkv, bs, causal, scale, out, out_sb, out_st, stream);
    if (prefill_mfma_supported(dtype, T, Hq, Hkv, D, bs, q_sb, q_st, q_sh, kv_sb, kv_st, kv_sh, out_sb,
                               out_st, q, k, v, out))
        return launch_prefill_mfma(q, q_sb, q_st, q_sh, k, v, kv_sb, kv_st, kv_sh, sel, n_sel, cap,
                                   B, T, Hq, Hkv, bs, causal, scale, out, out_sb, out_st, stream);
    dim3 grid(static_cast<unsigned>(T), static_cast<unsigned>(Hkv), static_cast<unsigned>(B));
    const float sl = scale * kLog2eP;
#define SPARDA_PF(DT_, DH_)                                                                          \
    hipLaunchKernelGGL((prefill_general_kernel<DT_, DH_>), grid, dim3(kPrefillThreads), 0, stream, q, \
                       q_sb, q_st, q_sh, k, v, kv_sb, kv_st, kv_sh, sel, n_sel, cap, T,              \
                       static_cast<int>(Hq), static_cast<int>(Hkv), static_cast<int>(bs), causal, sl, \
                       out, out_sb, out_st)
#define SPARDA_PF_D(DT_)                    \
    switch (D) {                            \
        case 16: SPARDA_PF(DT_, 16); break; \
        case 32: SPARDA_PF(DT_, 32); break; \
        case 64: SPARDA_PF(DT_, 64); break; \
        default: SPARDA_PF(DT_, 128); break; \
    }
    if (dtype == SPARDA_BF16) {
        SPARDA_PF_D(SPARDA_BF16);
    } else {
        SPARDA_PF_D(SPARDA_F32);
    }
#undef SPARDA_PF_D
#undef SPARDA_PF
    return check_hip(hipGetLastError(), "prefill_general_kernel");
}

}  // namespace sparda
