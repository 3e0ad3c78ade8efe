// The list of one query block of the chunked-gather prefill
// (model/attention/sparse.py:303-333), built by a whole workgroup in LDS:
// {0, bq} U (the union of the block's rows' top-k picks when they are given and
// bq > 0, else the static window [bq-k+1, bq]), picks past bq dropped, then the
// lowest `cut` = min(NB, k + 2) block indices, ascending (torch.topk over the
// reference's 0/1 mask leaves the choice among equal entries open; the lowest
// indices are this library's tie rule). Used by chunk_select_kernel (lists
// only) and by the chunked attention kernel (lists built in the launch).
#pragma once

#include "common.h"

namespace sparda {

constexpr int kChunkMaxNB = 4096;  // blocks one list bitmap covers

struct ChunkLds {
    uint32_t bits[kChunkMaxNB / 32];
    int32_t lst[kMaxSelCap];
    int m;
};

// rows: the block's first row of top-k picks (nrows rows of ke entries), or
// nullptr for the static window. Every thread of the workgroup calls it; on
// return c.lst[0..c.m) holds the list, visible to all of them.
__device__ __forceinline__ void chunk_list(ChunkLds& c, const int32_t* __restrict__ rows, int64_t nrows, int ke,
                                           int bq, int k, int64_t NB, int cut) {
    const int tid = static_cast<int>(threadIdx.x);
    const int nt = static_cast<int>(blockDim.x);
    const int nw = static_cast<int>((NB + 31) / 32);
    for (int i = tid; i < nw; i += nt) c.bits[i] = 0u;
    __syncthreads();
    if (tid == 0) {
        atomicOr(&c.bits[0], 1u);
        atomicOr(&c.bits[bq / 32], 1u << (bq % 32));
    }
    if (rows != nullptr && bq > 0) {
        const int64_t n = nrows * ke;
        for (int64_t e = tid; e < n; e += nt) {
            const int j = rows[e];
            if (j >= 0 && j <= bq) atomicOr(&c.bits[j / 32], 1u << (j % 32));
        }
    } else {
        const int lo = bq - k + 1 > 0 ? bq - k + 1 : 0;
        for (int j = lo + tid; j <= bq; j += nt) atomicOr(&c.bits[j / 32], 1u << (j % 32));
    }
    __syncthreads();
    // the first wavefront scans 64 bitmap words at a time: lane l takes word
    // base + l, an inclusive prefix sum of the words' bit counts places its bits
    if (tid < kWave) {
        int m = 0;
        for (int base = 0; base < nw && m < cut; base += kWave) {  // m is wave-uniform
            const int w = base + tid;
            uint32_t x = w < nw ? c.bits[w] : 0u;
            const int cnt = __popc(x);
            int inc = cnt;
            for (int d = 1; d < kWave; d <<= 1) {
                const int y = __shfl_up(inc, d, kWave);
                if (tid >= d) inc += y;
            }
            int pos = m + inc - cnt;
            while (x != 0u && pos < cut) {
                c.lst[pos++] = 32 * w + __builtin_ctz(x);
                x &= x - 1u;
            }
            m += __shfl(inc, kWave - 1, kWave);
        }
        if (tid == 0) c.m = m < cut ? m : cut;
    }
    __syncthreads();
}

// every row of the block receives the list (cap entries, -1 padded) and its length
__device__ __forceinline__ void chunk_write(const ChunkLds& c, int64_t row0, int64_t nrows, int cap,
                                            int32_t* __restrict__ sel, int32_t* __restrict__ n_sel) {
    const int tid = static_cast<int>(threadIdx.x);
    const int nt = static_cast<int>(blockDim.x);
    const int m = c.m;
    for (int64_t e = tid; e < nrows * cap; e += nt) {
        const int i = static_cast<int>(e % cap);
        sel[(row0 + e / cap) * cap + i] = i < m ? c.lst[i] : -1;
    }
    for (int64_t t = tid; t < nrows; t += nt) n_sel[row0 + t] = m;
}

}  // namespace sparda
