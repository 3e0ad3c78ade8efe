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

bool prefill_compact_supported(int dtype, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t bs,
                               const int32_t* sel, int64_t cap, int64_t q_sb, int64_t q_st, int64_t q_sh,
                               int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int64_t out_sb, int64_t out_st,
                               const void* q, const void* k, const void* v, const void* out);
int launch_prefill_compact(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k,
                           const void* v, int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                           const int32_t* sel, const int32_t* n_sel, int64_t cap, int64_t B, int64_t T,
                           int64_t Hq, int64_t Hkv, int causal, float scale, void* out,
                           int64_t out_sb, int64_t out_st, hipStream_t stream);

int launch_prefill(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k,
                   const void* v, int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int dtype,
                   const int32_t* sel, const int32_t* n_sel, int64_t cap, int64_t B, int64_t T,
                   int64_t Hq, int64_t Hkv, int64_t D, int64_t bs, int causal, float scale,
                   void* out, int64_t out_sb, int64_t out_st, hipStream_t stream) {
    // per-token selections: columns compacted per block; dense (no selection
    // lists) and wider selections: the union-of-blocks matrix-core kernel
    if (prefill_compact_supported(dtype, T, Hq, Hkv, D, bs, sel, cap, q_sb, q_st, q_sh, kv_sb, kv_st, kv_sh,
                                  out_sb, out_st, q, k, v, out))
        return launch_prefill_compact(q, q_sb, q_st, q_sh, k, v, kv_sb, kv_st, kv_sh, sel, n_sel, cap, B, T, Hq,
                                      Hkv, causal, scale, out, out_sb, out_st, stream);
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
