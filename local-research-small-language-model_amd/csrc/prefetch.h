// Decode-time block selection from fp32 block sums, and the prefetch of the
// next layer's blocks that a decode attention launch carries as extra
// workgroups (the prefetch of AsyncForecastOffloadAttention,
// model/attention/async_offload.py:170-294, overlapped with the current
// layer's attention inside one launch instead of on a second stream).
#pragma once

#include "common.h"
#include "kernels.h"
#include "select.h"

namespace sparda {

// 16-byte copy unit of the prefetch (a vector type: arrays of it stay in registers)
typedef uint32_t pf_u32x4 __attribute__((ext_vector_type(4)));

// Selection of one (sequence b, KV head g) by a whole workgroup (every thread
// calls it; it synchronises the workgroup). Blocks j < n_present are scored
// from their sums (p = sum / bs, the canonical fma chain, times scale; -inf for
// j > score_limit) into key_lds; wave 0 then takes {0, own} U top-k restricted
// to <= own, or every block 0..own while own + 1 <= k + 2, and adds the own
// block when it holds no token yet (own >= n_present). sel_lds receives the
// ascending list; the returned length is the same in every thread.
//   sums: the sums of block 0 of (b, g); consecutive blocks are jstride floats apart
template <int CHMAX, int DH, bool POW2>
__device__ __forceinline__ int select_from_sums(const void* f, bool f_bf16, int64_t f_off, const float* sums,
                                                int64_t jstride, int64_t n_present, int64_t score_limit, int own,
                                                int k, int bs, float scale, float* f_lds, uint32_t* key_lds,
                                                int32_t* sel_lds, uint32_t* ck_lds, int32_t* ci_lds, int* m_lds) {
    const int tid = static_cast<int>(threadIdx.x);
    const int nthr = static_cast<int>(blockDim.x);
    const int lane = tid % kWave;
    for (int d = tid; d < DH; d += nthr)
        f_lds[d] = f_bf16 ? load_elem<SPARDA_BF16>(f, f_off + d) : load_elem<SPARDA_F32>(f, f_off + d);
    __syncthreads();
    const bool dense = own + 1 <= k + 2;
    if (!dense) {
        // every thread scores blocks tid, tid + nthr, ...; all DH/4 loads of a
        // block are issued before its chain. For a power-of-two bs, sum * (1/bs)
        // is the same correctly rounded value as sum / bs (the reciprocal is exact).
        const float den = static_cast<float>(bs);
        const float inv = 1.0f / den;
        for (int64_t j = tid; j < n_present; j += nthr) {
            const float s = j <= score_limit ? score_from_sum<DH, POW2>(sums + j * jstride, f_lds, den, inv, scale)
                                             : -__builtin_inff();
            key_lds[j] = order_key(s);
        }
    }
    __syncthreads();
    if (tid < kWave) {
        int m;
        if (dense) {
            m = own + 1;
            if (lane < m) sel_lds[lane] = lane;
        } else {
            m = select_keys_upto<CHMAX>(key_lds, static_cast<int>(n_present), k, own, sel_lds, lane, ck_lds, ci_lds);
            if (own >= n_present) {  // the own block holds no token yet: it has no score but is attended
                if (lane == 0) sel_lds[m] = own;
                m += 1;
            }
        }
        if (lane == 0) *m_lds = m;
    }
    __syncthreads();
    return *m_lds;
}

// The copy of (b, g)'s selected blocks (m slots of sel_lds, rows below the
// arena length p = *pos_dev clamped into [0, Smax]) from the arena into the
// compact slots: share pf.part of pf.parts, the slots s with s % parts ==
// part. Wavefront w copies the share's slots w, w + nwaves, ...: 2 x 8
// sixteen-byte loads in flight per lane for a 64 x 128-byte block of K and of V.
__device__ __forceinline__ void prefetch_copy(const PrefetchDev& pf, int64_t bg, int64_t p, const int32_t* sel_lds,
                                             int m) {
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int nwaves = static_cast<int>(blockDim.x) / kWave;
    const int64_t len = p < 0 ? 0 : (p > pf.Smax ? pf.Smax : p);
    constexpr int kIn = 8;  // 16-byte chunks of K (and of V) in flight per lane
    const int parts = pf.parts >= 1 ? pf.parts : 1;  // (the host passes parts >= 1, part < parts)
    const int part = pf.part >= 0 && pf.part < parts ? pf.part : 0;
    for (int i = wave;; i += nwaves) {
        const int slot = part + parts * i;
        if (slot >= m || slot >= pf.cap) break;
        const int64_t j = sel_lds[slot];
        if (j < 0 || j * pf.bs >= len) continue;
        const int64_t rows = (j + 1) * pf.bs < len ? pf.bs : len - j * pf.bs;
        const int64_t chunks = rows * pf.row_bytes / 16;
        const pf_u32x4* sk = reinterpret_cast<const pf_u32x4*>(pf.ak + (bg * pf.Smax + j * pf.bs) * pf.row_bytes);
        const pf_u32x4* sv = reinterpret_cast<const pf_u32x4*>(pf.av + (bg * pf.Smax + j * pf.bs) * pf.row_bytes);
        pf_u32x4* tk = reinterpret_cast<pf_u32x4*>(pf.dk + (bg * pf.cap + slot) * pf.bs * pf.row_bytes);
        pf_u32x4* tv = reinterpret_cast<pf_u32x4*>(pf.dv + (bg * pf.cap + slot) * pf.bs * pf.row_bytes);
        for (int c0 = lane; c0 < chunks; c0 += kIn * kWave) {
            // chunks past the block's rows re-read its last chunk (in bounds) and are not stored
            pf_u32x4 kr[kIn], vr[kIn];
#pragma unroll
            for (int i2 = 0; i2 < kIn; ++i2) {
                const int c = c0 + i2 * kWave < chunks ? c0 + i2 * kWave : static_cast<int>(chunks) - 1;
                kr[i2] = sk[c];
                vr[i2] = sv[c];
            }
#pragma unroll
            for (int i2 = 0; i2 < kIn; ++i2) {
                const int c = c0 + i2 * kWave;
                if (c < chunks) {
                    tk[c] = kr[i2];
                    tv[c] = vr[i2];
                }
            }
        }
    }
}

// The selection an earlier launch of the stream wrote for (b, g), into
// sel_lds (every thread calls it; it synchronises the workgroup); returns its
// length, clamped into [0, cap].
__device__ __forceinline__ int prefetch_read_selection(const PrefetchDev& pf, int64_t bg, int32_t* sel_lds) {
    int m = pf.n_sel[bg];
    m = m < 0 ? 0 : (m > pf.cap ? pf.cap : m);
    for (int i = static_cast<int>(threadIdx.x); i < m; i += static_cast<int>(blockDim.x))
        sel_lds[i] = pf.sel[bg * pf.cap + i];
    __syncthreads();
    return m;
}

// The prefetch of (b, g) by one workgroup: the selection with lookahead at
// token p = *pos_dev (len = p: the blocks before the token is appended), its
// list written to pf.sel / pf.n_sel, then the selected blocks copied
// (prefetch_copy). Stage 1 stops after the selection; stage 2 copies the
// selection found in pf.sel / pf.n_sel.
template <int CHMAX, int DH>
__device__ __forceinline__ void prefetch_workgroup(const PrefetchDev& pf, int g, int b, const int64_t* pos_dev,
                                                   float* f_lds, uint32_t* key_lds, int32_t* sel_lds,
                                                   uint32_t* ck_lds, int32_t* ci_lds, int* m_lds) {
    const int tid = static_cast<int>(threadIdx.x);
    const int64_t bg = static_cast<int64_t>(b) * pf.H + g;
    const int64_t p = *pos_dev;
    int m;
    if (pf.stage != 2) {
        const int64_t pos = p < 0 ? 0 : (p > pf.pos_max ? pf.pos_max : p);
        const int64_t n_present = (pos + pf.bs - 1) / pf.bs;
        const int64_t score_limit = (pf.absolute ? pos : 0) / pf.bs;
        const int own = static_cast<int>(pos / pf.bs);
        const float* sums = pf.sums + (static_cast<int64_t>(b) * pf.nb_stride * pf.H + g) * DH;
        const int64_t f_off = b * pf.f_sb + g * pf.f_sh;
        m = pf.pow2 ? select_from_sums<CHMAX, DH, true>(pf.f, pf.f_bf16 != 0, f_off, sums, pf.H * DH, n_present,
                                                        score_limit, own, pf.k, pf.bs, pf.scale, f_lds, key_lds,
                                                        sel_lds, ck_lds, ci_lds, m_lds)
                    : select_from_sums<CHMAX, DH, false>(pf.f, pf.f_bf16 != 0, f_off, sums, pf.H * DH, n_present,
                                                         score_limit, own, pf.k, pf.bs, pf.scale, f_lds, key_lds,
                                                         sel_lds, ck_lds, ci_lds, m_lds);
        for (int i = tid; i < pf.cap; i += static_cast<int>(blockDim.x))
            pf.sel[bg * pf.cap + i] = i < m ? sel_lds[i] : -1;
        if (tid == 0) pf.n_sel[bg] = m;
        if (pf.stage == 1) return;
    } else {
        m = prefetch_read_selection(pf, bg, sel_lds);
    }
    prefetch_copy(pf, bg, p, sel_lds, m);
}

// A launch that carries only a share of the copy (stage 2): (b, g)'s selection
// from pf.sel / pf.n_sel, then its share of the blocks. Needs kMaxSelCap ints of LDS.
__device__ __forceinline__ void prefetch_copy_workgroup(const PrefetchDev& pf, int g, int b, const int64_t* pos_dev,
                                                        int32_t* sel_lds) {
    const int64_t bg = static_cast<int64_t>(b) * pf.H + g;
    const int m = prefetch_read_selection(pf, bg, sel_lds);
    prefetch_copy(pf, bg, *pos_dev, sel_lds, m);
}

}  // namespace sparda
