// Wavefront online-softmax over one staged chunk of keys (VALU, fp32).
// Shared by the decode split-K kernel and the general prefill kernel.
#pragma once

#include "common.h"

namespace sparda {

constexpr int kChunkKeys = 64;  // keys staged in LDS per pass (one per lane)

template <int DH>
struct HeadAcc {
    static constexpr int DPL = (DH + kWave - 1) / kWave;  // output dims per lane
    float m;
    float l;
    float o[DPL];
    __device__ __forceinline__ void init() {
        m = -__builtin_inff();
        l = 0.0f;
#pragma unroll
        for (int i = 0; i < DPL; ++i) o[i] = 0.0f;
    }
};

// Scores are in log2 units: q_row already holds q * scale * log2(e).
// k_lds / v_lds: [nk][KS] fp32 rows; p_wave: 64 floats private to this wave.
// valid(i) masks keys; a chunk with no valid key leaves the state unchanged.
template <int DH, int KS, typename Valid>
__device__ __forceinline__ void attend_chunk(const float* q_row, const float* k_lds,
                                             const float* v_lds, int nk, float* p_wave,
                                             HeadAcc<DH>& acc, Valid valid) {
    const int lane = threadIdx.x % kWave;
    float s = -__builtin_inff();
    if (lane < nk && valid(lane)) {
        float a = 0.0f;
#pragma unroll
        for (int d = 0; d < DH; ++d) a = fmaf(q_row[d], k_lds[lane * KS + d], a);
        s = a;
    }
    const float mc = wave_max(s);
    if (mc == -__builtin_inff()) return;  // wave-uniform
    const float m_new = fmaxf(acc.m, mc);
    const float alpha = __builtin_amdgcn_exp2f(acc.m - m_new);
    const float p = (s == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f(s - m_new);
    acc.l = acc.l * alpha + wave_sum(p);
    acc.m = m_new;
    p_wave[lane] = p;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < HeadAcc<DH>::DPL; ++i) {
        const int d = lane + i * kWave;
        float o = acc.o[i] * alpha;
        if (d < DH) {
            for (int key = 0; key < nk; ++key) o = fmaf(p_wave[key], v_lds[key * KS + d], o);
        }
        acc.o[i] = o;
    }
    __builtin_amdgcn_wave_barrier();
}

}  // namespace sparda
