// One set of 64 consecutive query rows routed by a group of wavefronts of
// one workgroup (lane = row): forecast x prototype scores (the
// canonical fma chain), the per-row top-k of route keys, merged across the
// waves. Shared by the stand-alone router and the prefill kernel that routes
// its own query window, so both produce the same picks bit for bit.
#pragma once

#include "common.h"
#include "select.h"

namespace sparda {

constexpr int kRouteWaves = 4;
constexpr int kRouteThreads = kRouteWaves * kWave;

// N consecutive fp32 values (N in {1, 2, 4, 8}), 4*N-byte aligned
template <int N>
__device__ __forceinline__ void load_f32(const float* __restrict__ p, float (&o)[N]) {
    if constexpr (N == 1) {
        o[0] = p[0];
    } else if constexpr (N == 2) {
        const float2 v = *reinterpret_cast<const float2*>(p);
        o[0] = v.x; o[1] = v.y;
    } else {
#pragma unroll
        for (int q = 0; q < N; q += 4) {
            const float4 v = *reinterpret_cast<const float4*>(p + q);
            o[q] = v.x; o[q + 1] = v.y; o[q + 2] = v.z; o[q + 3] = v.w;
        }
    }
}

// Two fma chains, one step: acc[c] = fma(a, element of lane I of this lane's
// 16-lane row of p[c], acc[c]), each a v_fmac_f32 with a DPP row_newbcast
// source (a separate DPP move does not fold into the fma, which is a VOP3 op
// at that point). A DPP instruction needs two wait states after a VALU write
// of any register it reads. The compiler does not track that for inline
// assembly, so the steps carry their own: the two fmas of a step write
// different accumulators and end with s_nop 0, so an accumulator is read two
// wait states after its last write, and the steps that first read the
// prototype registers (FIRST) start with s_nop 1. What the compiler places
// between steps (spill reloads, copies) is checked on the built code by the
// test suite. (Four chains without the s_nop measured no faster: the nop
// costs the wave an issue cycle, not the SIMD, whose other wave issues.)
template <int I, bool FIRST>
__device__ __forceinline__ void fma_row_bcast(float (&acc)[2], float a, const float (&p)[2]) {
    if constexpr (FIRST)
        asm("s_nop 1\n\tv_fmac_f32_dpp %0, %2, %4 row_newbcast:%5 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %1, %3, %4 row_newbcast:%5 row_mask:0xf bank_mask:0xf\n\ts_nop 0"
            : "+v"(acc[0]), "+v"(acc[1]) : "v"(p[0]), "v"(p[1]), "v"(a), "n"(I));
    else
        asm("v_fmac_f32_dpp %0, %2, %4 row_newbcast:%5 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %1, %3, %4 row_newbcast:%5 row_mask:0xf bank_mask:0xf\n\ts_nop 0"
            : "+v"(acc[0]), "+v"(acc[1]) : "v"(p[0]), "v"(p[1]), "v"(a), "n"(I));
}
// acc[c] = fma chain over d = E*I + e (I = I0..15, e = 0..E-1) with element d
// of prototype c taken from lane I of the row (register pc[e][c])
template <int E, int DF, int C, int I0 = 0>
__device__ __forceinline__ void row_fma_chains(const float (&fr)[DF], const float (&pc)[E][C],
                                               float (&acc)[C]) {
    if constexpr (I0 < 16) {
#pragma unroll
        for (int e = 0; e < E; ++e) fma_row_bcast<I0, I0 == 0>(acc, fr[E * I0 + e], pc[e]);
        row_fma_chains<E, DF, C, I0 + 1>(fr, pc, acc);
    }
}

// The DF forecast elements at element offset `base` as fp32: 16-byte vector
// loads where every row is 16-byte aligned (vec, uniform), else one element
// at a time.
template <int FDT, int DF>
__device__ __forceinline__ void load_forecast_row(const void* __restrict__ f, int64_t base, bool vec,
                                                  float (&fr)[DF]) {
    if (vec) {
        if constexpr (FDT == SPARDA_F32) {
            const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(f) + base);
#pragma unroll
            for (int q = 0; q < DF / 4; ++q) {
                const float4 w = src[q];
                fr[4 * q] = w.x; fr[4 * q + 1] = w.y; fr[4 * q + 2] = w.z; fr[4 * q + 3] = w.w;
            }
        } else {
            const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(f) + base);
#pragma unroll
            for (int q = 0; q < DF / 8; ++q) {
                const uint4 w = src[q];
                const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    fr[8 * q + 2 * e] = __uint_as_float(u[e] << 16);
                    fr[8 * q + 2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
                }
            }
        }
    } else {
#pragma unroll
        for (int d = 0; d < DF; ++d) fr[d] = load_elem<FDT>(f, base + d);
    }
}

// Routes rows set*64 + lane of (b, h) on NW wavefronts. The waves split the
// candidate blocks (wave w scores j = w, w + NW, ...), so the block index is uniform
// across a wavefront: every 16-lane row loads the block's prototype with one
// coalesced load (lane i of the row holds elements E*i .. E*i+E-1, E = DF/16),
// one block ahead of its use, and the fma chain takes element d from lane d/E
// of the row through a DPP row broadcast. Each lane keeps its row's KMAX best
// route keys; wave m merges the waves' lists through `lists` (LDS,
// [NW][KMAX][64] doubles) and returns true with the row's picks
// (slots i >= ke: -1; slots no candidate filled: block i, the masked blocks
// in ascending order); the other waves return false. With scores non-null,
// every score of the row (-inf where masked) is written to scores[row * NB].
// Called by every wavefront of the workgroup (two barriers inside).
template <int FDT, int DF, int KMAX, int NW = kRouteWaves>
__device__ __forceinline__ bool route_set(const void* __restrict__ f, int64_t fsb, int64_t fst, int64_t fsh,
                                          const float* __restrict__ protos, int b, int h, int H, int64_t set,
                                          int64_t Tq, int64_t NB, int bs, int ke, int causal, int64_t score_pos0,
                                          float scale, float* __restrict__ scores, int m, double* lists,
                                          int32_t (&picks)[KMAX]) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x % kWave;
    // the wave within its group of NW (a workgroup may route several sets at once)
    const int w = __builtin_amdgcn_readfirstlane(static_cast<int>((threadIdx.x / kWave) % NW));
    const float* __restrict__ pbh = protos + (static_cast<int64_t>(b) * NB * H + h) * DF;
    const int64_t pstride = static_cast<int64_t>(H) * DF;
    const int64_t t = set * kWave + lane;
    const bool active = t < Tq;
    const int64_t tc = active ? t : Tq - 1;
    const int64_t t_last = (set * kWave + kWave < Tq ? set * kWave + kWave : Tq) - 1;
    int64_t limit = causal ? (score_pos0 + tc) / bs : NB - 1;
    if (limit > NB - 1) limit = NB - 1;
    int64_t jmax64 = causal ? (score_pos0 + t_last) / bs : NB - 1;
    if (jmax64 > NB - 1) jmax64 = NB - 1;
    // uniform: the block loop and the prototype addresses stay on the scalar unit
    const int jmax = __builtin_amdgcn_readfirstlane(static_cast<int>(jmax64));

    float fr[DF];
    {
        constexpr int64_t V = FDT == SPARDA_F32 ? 4 : 8;  // elements per 16 bytes
        const bool vec = (reinterpret_cast<uintptr_t>(f) & 15u) == 0 && fsb % V == 0 && fst % V == 0 && fsh % V == 0;
        load_forecast_row<FDT, DF>(f, b * fsb + tc * fst + h * fsh, vec, fr);
    }
    const int64_t row = (static_cast<int64_t>(b) * H + h) * Tq + t;
    float* srow = (scores != nullptr && active) ? scores + row * NB : nullptr;

    KeyTopK<KMAX> best;
    best.init();
    constexpr int E = DF / 16;
    constexpr int C = 2;  // blocks scored side by side
    const int loff = (lane % 16) * E;  // this lane's elements of a prototype row
    // prototype row of block min(jc, jmax) (a wave-uniform address), this lane's E elements
    auto load_proto = [&](int jc, float (&o)[E]) __attribute__((always_inline)) {
        const float* __restrict__ pb = pbh + static_cast<int64_t>(jc < jmax ? jc : jmax) * pstride;
        load_f32<E>(pb + loff, o);
    };
    // scores blocks j, j + NW, ... (C of them, prototypes in pc) and
    // pushes their keys
    auto score = [&](int j, const float (&pc)[E][C]) __attribute__((always_inline)) {
        float acc[C];
#pragma unroll
        for (int c = 0; c < C; ++c) acc[c] = 0.0f;
        row_fma_chains<E, DF, C>(fr, pc, acc);
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const int jc = j + c * NW;
            const float sc = acc[c] * scale;
            const bool ok = jc <= limit;  // limit <= jmax
            if (srow && ok) srow[jc] = sc;
            best.push(ok ? route_key(sc, static_cast<int32_t>(jc)) : 0.0);
        }
    };
    // two prototype buffers used in turn, each loaded one step ahead of its use
    constexpr int kStep = C * NW;
    float pa[E][C], pz[E][C];
    float tmp[E];
#pragma unroll
    for (int c = 0; c < C; ++c) {
        load_proto(w + c * NW, tmp);
#pragma unroll
        for (int e = 0; e < E; ++e) pa[e][c] = tmp[e];
    }
    for (int j = w; j <= jmax; j += 2 * kStep) {
#pragma unroll
        for (int c = 0; c < C; ++c) {
            load_proto(j + kStep + c * NW, tmp);
#pragma unroll
            for (int e = 0; e < E; ++e) pz[e][c] = tmp[e];
        }
        score(j, pa);
        if (j + kStep > jmax) break;  // uniform
#pragma unroll
        for (int c = 0; c < C; ++c) {
            load_proto(j + 2 * kStep + c * NW, tmp);
#pragma unroll
            for (int e = 0; e < E; ++e) pa[e][c] = tmp[e];
        }
        score(j + kStep, pz);
    }
    if (srow) {
        for (int64_t j = w; j < NB; j += NW)
            if (j > limit) srow[j] = -__builtin_inff();
    }

    // merge the waves' lists in the merging wave
    __syncthreads();  // the previous set's merger has read its lists
    if (w != m) {
#pragma unroll
        for (int i = 0; i < KMAX; ++i) lists[(w * KMAX + i) * kWave + lane] = best.r[i];
    }
    __syncthreads();
    if (w != m) return false;
    for (int o = 0; o < NW; ++o) {
        if (o == m) continue;
        double other[KMAX];
#pragma unroll
        for (int i = 0; i < KMAX; ++i) other[i] = lists[(o * KMAX + i) * kWave + lane];
        best.merge(other);
    }
    // slots not filled by a candidate take the masked blocks in ascending order
#pragma unroll
    for (int i = 0; i < KMAX; ++i) picks[i] = (i < ke) ? (best.r[i] == 0.0 ? i : route_key_index(best.r[i])) : -1;
    return true;
}

}  // namespace sparda
