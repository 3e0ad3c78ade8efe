// Single-token decode step of the sparse attention layer, two launches:
//
//  1. decode_select_kernel, grid (NB, B): each workgroup streams one KV block
//     of the cache (all KV heads), forms its prototypes (sequential fp32 sum,
//     / bs) and the forecast score of every head; the last workgroup to arrive
//     for a sequence runs the top-k and writes the sorted selection lists.
//     This is the HBM-bound pass: it reads the whole K cache once.
//  2. decode_attend_kernel, grid (k+2, Hkv, B): one workgroup per selected
//     block and KV head reads that block's K/V once into LDS and serves all
//     Hq/Hkv query heads of the group (split-K partial: m, l, o); the last
//     workgroup of a (sequence, KV head) merges the partials in slot order.
//
// Dense (NB <= k+2) and static-window (no forecast) steps skip launch 1: the
// attend kernel derives those selections from the block counts.
#pragma clang fp contract(off)

#include "common.h"
#include "kernels.h"
#include "select.h"
#include "attend.h"

namespace sparda {

constexpr float kLog2e = 1.4426950408889634f;

static size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

DecodeWs decode_ws_layout(void* base, int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D,
                          int64_t bs, int64_t k) {
    const int64_t NB = cdiv(S, bs);
    const int64_t cap = k + 2;
    char* p = static_cast<char*>(base);
    size_t off = 0;
    DecodeWs w{};
    w.cnt_b = reinterpret_cast<int32_t*>(p + off);
    w.cnt_bg = w.cnt_b + B;
    off += align256(static_cast<size_t>(B + B * Hkv) * 4);
    w.scores = reinterpret_cast<float*>(p + off);
    off += align256(static_cast<size_t>(B * Hkv * NB) * 4);
    w.sel = reinterpret_cast<int32_t*>(p + off);
    off += align256(static_cast<size_t>(B * Hkv * cap) * 4);
    w.n_sel = reinterpret_cast<int32_t*>(p + off);
    off += align256(static_cast<size_t>(B * Hkv) * 4);
    w.part = reinterpret_cast<float*>(p + off);
    off += align256(static_cast<size_t>(B * Hq * cap * (D + 2)) * 4);
    w.bytes = off;
    return w;
}

// ---------------------------------------------------------------------------
// launch 1: compress + score + (last arrival) select
// block = H*D/VEC threads, thread -> (h, d-group)
// ---------------------------------------------------------------------------
template <int DT, int FDT, int VEC>
__global__ void __launch_bounds__(1024)
decode_select_kernel(const void* __restrict__ kc, int64_t kv_sb, int64_t kv_ss, int64_t kv_sh,
                     int64_t S, int H, int D, int bs, int64_t NB,
                     const void* __restrict__ f, int64_t f_sb, int64_t f_sh, float scale,
                     int64_t score_pos0, const float* __restrict__ protos_in,
                     float* __restrict__ protos_out, int ke, int cap,
                     int32_t* cnt_b, float* ws_scores, int32_t* ws_sel, int32_t* ws_nsel,
                     int32_t* __restrict__ sel_out, int32_t* __restrict__ n_sel_out) {
    extern __shared__ float smem[];
    float* p_lds = smem;            // [H*D]
    float* f_lds = smem + H * D;    // [H*D]
    uint64_t* ranks = reinterpret_cast<uint64_t*>(smem + 2 * H * D);  // [NB] (last arrival only)
    __shared__ uint64_t wave_best[16];
    __shared__ int32_t picks[64];
    __shared__ int is_last;

    const int j = blockIdx.x;
    const int b = blockIdx.y;
    const int groups = D / VEC;
    const int HD = H * D;

    // 1. prototypes of block j for every head
    for (int e = threadIdx.x; e < H * groups; e += blockDim.x) {
        const int h = e / groups;
        const int d = (e % groups) * VEC;
        const int64_t pidx = ((static_cast<int64_t>(b) * NB + j) * H + h) * D + d;
        if (protos_in != nullptr) {
#pragma unroll
            for (int v = 0; v < VEC; ++v) p_lds[h * D + d + v] = protos_in[pidx + v];
        } else {
            const int64_t base = b * kv_sb + h * kv_sh + d;
            const int64_t s0 = static_cast<int64_t>(j) * bs;
            const int64_t s1 = s0 + bs < S ? s0 + bs : S;
            const float den = static_cast<float>(bs);
            if constexpr (VEC == 2) {
                float ax = 0.0f, ay = 0.0f;
#pragma unroll 8
                for (int64_t s = s0; s < s1; ++s) {
                    const float2 v = load_pair<DT>(kc, base + s * kv_ss);
                    ax = ax + v.x;
                    ay = ay + v.y;
                }
                p_lds[h * D + d] = ax / den;
                p_lds[h * D + d + 1] = ay / den;
            } else {
                float a = 0.0f;
#pragma unroll 8
                for (int64_t s = s0; s < s1; ++s) a = a + load_elem<DT>(kc, base + s * kv_ss);
                p_lds[h * D + d] = a / den;
            }
            if (protos_out != nullptr) {
#pragma unroll
                for (int v = 0; v < VEC; ++v) protos_out[pidx + v] = p_lds[h * D + d + v];
            }
        }
    }
    // 2. forecast rows of sequence b
    for (int e = threadIdx.x; e < HD; e += blockDim.x)
        f_lds[e] = load_elem<FDT>(f, b * f_sb + (e / D) * f_sh + (e % D));
    __syncthreads();

    // 3. scores (fma chain over d, canonical order), causal mask at score_pos0
    int64_t limit = score_pos0 / bs;
    if (limit > NB - 1) limit = NB - 1;
    for (int h = threadIdx.x; h < H; h += blockDim.x) {
        float s = -__builtin_inff();
        if (j <= limit) {
            float acc = 0.0f;
            for (int d = 0; d < D; ++d) acc = __fmaf_rn(f_lds[h * D + d], p_lds[h * D + d], acc);
            s = acc * scale;
        }
        ws_scores[(static_cast<int64_t>(b) * H + h) * NB + j] = s;
    }

    // 4. arrival; the last workgroup of sequence b selects for all heads
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) is_last = (atomicAdd(&cnt_b[b], 1) == static_cast<int>(NB) - 1);
    __syncthreads();
    if (!is_last) return;
    __threadfence();

    const int64_t cb = (S - 1) / bs;
    for (int h = 0; h < H; ++h) {
        const float* srow = ws_scores + (static_cast<int64_t>(b) * H + h) * NB;
        for (int64_t jj = threadIdx.x; jj < NB; jj += blockDim.x)
            ranks[jj] = rank64(__builtin_nontemporal_load(srow + jj), static_cast<int32_t>(jj));
        __syncthreads();
        wg_topk(ranks, static_cast<int>(NB), ke, picks, wave_best);
        if (threadIdx.x == 0) {
            int32_t c[34];
            c[0] = 0;
            c[1] = static_cast<int32_t>(cb);
#pragma unroll
            for (int i = 0; i < 32; ++i) c[i + 2] = i < ke ? picks[i] : -1;
            const int64_t r = static_cast<int64_t>(b) * H + h;
            emit_selection(c, static_cast<int>(cb), true, ws_sel + r * cap, cap, ws_nsel + r);
            if (sel_out != nullptr) {
                for (int i = 0; i < cap; ++i) sel_out[r * cap + i] = ws_sel[r * cap + i];
                n_sel_out[r] = ws_nsel[r];
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) cnt_b[b] = 0;
}

// ---------------------------------------------------------------------------
// launch 2: split-K attention over the selected blocks + last-arrival combine
// sel_mode: 0 lists from launch 1, 1 dense (all blocks), 2 window {0} U [cb-k+1, cb]
// ---------------------------------------------------------------------------
constexpr int kAttendThreads = 256;
constexpr int kAttendWaves = kAttendThreads / kWave;
constexpr int kMaxGroup = 16;  // query heads per KV head

template <int DT, int DH>
__global__ void __launch_bounds__(kAttendThreads)
decode_attend_kernel(const void* __restrict__ q, int64_t q_sb, int64_t q_sh,
                     const void* __restrict__ kc, const void* __restrict__ vc,
                     int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int64_t S, int Hq, int H, int bs,
                     int64_t NB, int k, int sel_mode, int cap, float scale_log2,
                     const int32_t* ws_sel, const int32_t* ws_nsel, int32_t* cnt_bg, float* part,
                     int32_t* __restrict__ sel_out, int32_t* __restrict__ n_sel_out,
                     void* __restrict__ out, int64_t out_sb) {
    constexpr int KS = DH + 1;  // padded LDS row (conflict-free column walks)
    __shared__ float k_lds[kChunkKeys * KS];
    __shared__ float v_lds[kChunkKeys * KS];
    __shared__ float q_lds[kMaxGroup * DH];
    __shared__ float p_lds[kAttendWaves][kChunkKeys];
    __shared__ int is_last;

    const int slot = blockIdx.x;
    const int g = blockIdx.y;
    const int b = blockIdx.z;
    const int R = Hq / H;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int64_t bg = static_cast<int64_t>(b) * H + g;
    const int64_t cb = (S - 1) / bs;

    int n;
    int64_t j;
    if (sel_mode == 0) {
        n = ws_nsel[bg];
        j = slot < n ? ws_sel[bg * cap + slot] : 0;
    } else if (sel_mode == 1) {
        n = static_cast<int>(cb + 1);
        j = slot;
        if (slot == 0 && sel_out != nullptr && threadIdx.x == 0) {
            for (int i = 0; i < cap; ++i) sel_out[bg * cap + i] = i < n ? i : -1;
            n_sel_out[bg] = n;
        }
    } else {
        int64_t lo = cb - k + 1;
        if (lo < 0) lo = 0;
        const int lead = lo > 0 ? 1 : 0;
        n = static_cast<int>(cb - lo + 1) + lead;
        j = (lead && slot == 0) ? 0 : lo + slot - lead;
        if (slot == 0 && sel_out != nullptr && threadIdx.x == 0) {
            for (int i = 0; i < cap; ++i) {
                int64_t ji = -1;
                if (i < n) ji = (lead && i == 0) ? 0 : lo + i - lead;
                sel_out[bg * cap + i] = static_cast<int32_t>(ji);
            }
            n_sel_out[bg] = n;
        }
    }
    if (slot >= n) return;

    const int64_t s_begin = j * bs;
    int64_t s_end = s_begin + bs;
    if (s_end > S) s_end = S;

    for (int e = threadIdx.x; e < R * DH; e += kAttendThreads) {
        const int hh = e / DH, d = e % DH;
        q_lds[e] = load_elem<DT>(q, b * q_sb + static_cast<int64_t>(g * R + hh) * q_sh + d) * scale_log2;
    }
    constexpr int MAXR = kMaxGroup / kAttendWaves;  // heads per wave
    HeadAcc<DH> acc[MAXR];
#pragma unroll
    for (int r = 0; r < MAXR; ++r) acc[r].init();

    for (int64_t c0 = s_begin; c0 < s_end; c0 += kChunkKeys) {
        const int nk = static_cast<int>((s_end - c0) < kChunkKeys ? (s_end - c0) : kChunkKeys);
        __syncthreads();
        for (int e = threadIdx.x; e < nk * DH; e += kAttendThreads) {
            const int i = e / DH, d = e % DH;
            const int64_t src = b * kv_sb + (c0 + i) * kv_ss + g * kv_sh + d;
            k_lds[i * KS + d] = load_elem<DT>(kc, src);
            v_lds[i * KS + d] = load_elem<DT>(vc, src);
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < MAXR; ++r) {
            const int hh = wave + r * kAttendWaves;
            if (hh < R)
                attend_chunk<DH, KS>(q_lds + hh * DH, k_lds, v_lds, nk, p_lds[wave], acc[r],
                                     [](int) { return true; });
        }
    }

    // partial (m, l, o) of each head handled by this wave
#pragma unroll
    for (int r = 0; r < MAXR; ++r) {
        const int hh = wave + r * kAttendWaves;
        if (hh >= R) continue;
        const int h = g * R + hh;
        float* pp = part + ((static_cast<int64_t>(b) * Hq + h) * cap + slot) * (DH + 2);
        if (lane == 0) {
            pp[0] = acc[r].m;
            pp[1] = acc[r].l;
        }
#pragma unroll
        for (int i = 0; i < HeadAcc<DH>::DPL; ++i) {
            const int d = lane + i * kWave;
            if (d < DH) pp[2 + d] = acc[r].o[i];
        }
    }

    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) is_last = (atomicAdd(&cnt_bg[bg], 1) == n - 1);
    __syncthreads();
    if (!is_last) return;
    __threadfence();

    for (int e = threadIdx.x; e < R * DH; e += kAttendThreads) {
        const int hh = e / DH, d = e % DH;
        const int h = g * R + hh;
        const float* pb = part + (static_cast<int64_t>(b) * Hq + h) * cap * (DH + 2);
        float M = -__builtin_inff();
        for (int s = 0; s < n; ++s) M = fmaxf(M, __builtin_nontemporal_load(pb + s * (DH + 2)));
        float num = 0.0f, den = 0.0f;
        for (int s = 0; s < n; ++s) {
            const float* ps = pb + s * (DH + 2);
            const float w = exp2f(__builtin_nontemporal_load(ps) - M);
            den = den + w * __builtin_nontemporal_load(ps + 1);
            num = num + w * __builtin_nontemporal_load(ps + 2 + d);
        }
        store_elem<DT>(out, b * out_sb + static_cast<int64_t>(h) * DH + d, num / den);
    }
    if (threadIdx.x == 0) cnt_bg[bg] = 0;
}

// ---------------------------------------------------------------------------
int launch_decode(const void* q, int64_t q_sb, int64_t q_sh, const void* kc, const void* vc,
                  int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int dtype, const void* f, int fdtype,
                  int64_t f_sb, int64_t f_sh, int64_t B, int64_t S, int64_t Hq, int64_t Hkv,
                  int64_t D, int64_t bs, int64_t k, int routing, float scale, const float* protos_in,
                  float* protos_out, int32_t* sel_out, int32_t* n_sel_out, void* out, int64_t out_sb,
                  const DecodeWs& ws, hipStream_t stream) {
    const int64_t NB = cdiv(S, bs);
    const int cap = static_cast<int>(k + 2);
    int sel_mode;
    if (NB <= k + 2) {
        sel_mode = 1;
    } else if (f == nullptr) {
        sel_mode = 2;
    } else {
        sel_mode = 0;
        const bool aligned = (D % 2 == 0) && (kv_sb % 2 == 0) && (kv_ss % 2 == 0) && (kv_sh % 2 == 0) &&
                             (reinterpret_cast<uintptr_t>(kc) % (dtype == SPARDA_F32 ? 8 : 4) == 0);
        const int vec = aligned ? 2 : 1;
        int threads = static_cast<int>(Hkv * D / vec);
        if (threads > 1024) threads = 1024;
        threads = ((threads + kWave - 1) / kWave) * kWave;
        const size_t lds = static_cast<size_t>(2 * Hkv * D) * sizeof(float) + static_cast<size_t>(NB) * 8;
        const int64_t score_pos0 = (routing == SPARDA_ROUTE_ABSOLUTE) ? S - 1 : 0;
        dim3 grid(static_cast<unsigned>(NB), static_cast<unsigned>(B));
#define SPARDA_SEL(DT_, FDT_, V_)                                                                 \
    hipLaunchKernelGGL((decode_select_kernel<DT_, FDT_, V_>), grid, dim3(threads), lds, stream,  \
                       kc, kv_sb, kv_ss, kv_sh, S, static_cast<int>(Hkv), static_cast<int>(D),   \
                       static_cast<int>(bs), NB, f, f_sb, f_sh, scale, score_pos0, protos_in,    \
                       protos_out, static_cast<int>(k), cap, ws.cnt_b, ws.scores, ws.sel,        \
                       ws.n_sel, sel_out, n_sel_out)
        if (dtype == SPARDA_BF16) {
            if (fdtype == SPARDA_BF16) {
                if (vec == 2) SPARDA_SEL(SPARDA_BF16, SPARDA_BF16, 2); else SPARDA_SEL(SPARDA_BF16, SPARDA_BF16, 1);
            } else {
                if (vec == 2) SPARDA_SEL(SPARDA_BF16, SPARDA_F32, 2); else SPARDA_SEL(SPARDA_BF16, SPARDA_F32, 1);
            }
        } else {
            if (fdtype == SPARDA_BF16) {
                if (vec == 2) SPARDA_SEL(SPARDA_F32, SPARDA_BF16, 2); else SPARDA_SEL(SPARDA_F32, SPARDA_BF16, 1);
            } else {
                if (vec == 2) SPARDA_SEL(SPARDA_F32, SPARDA_F32, 2); else SPARDA_SEL(SPARDA_F32, SPARDA_F32, 1);
            }
        }
#undef SPARDA_SEL
        int rc = check_hip(hipGetLastError(), "decode_select_kernel");
        if (rc) return rc;
    }
    dim3 grid2(static_cast<unsigned>(cap), static_cast<unsigned>(Hkv), static_cast<unsigned>(B));
    const float scale_log2 = scale * kLog2e;
#define SPARDA_ATT(DT_, DH_)                                                                       \
    hipLaunchKernelGGL((decode_attend_kernel<DT_, DH_>), grid2, dim3(kAttendThreads), 0, stream,   \
                       q, q_sb, q_sh, kc, vc, kv_sb, kv_ss, kv_sh, S, static_cast<int>(Hq),        \
                       static_cast<int>(Hkv), static_cast<int>(bs), NB, static_cast<int>(k),       \
                       sel_mode, cap, scale_log2, ws.sel, ws.n_sel, ws.cnt_bg, ws.part,            \
                       sel_mode == 0 ? nullptr : sel_out, n_sel_out, out, out_sb)
#define SPARDA_ATT_D(DT_)                                                                          \
    switch (D) {                                                                                   \
        case 16: SPARDA_ATT(DT_, 16); break;                                                       \
        case 32: SPARDA_ATT(DT_, 32); break;                                                       \
        case 64: SPARDA_ATT(DT_, 64); break;                                                       \
        default: SPARDA_ATT(DT_, 128); break;                                                      \
    }
    if (dtype == SPARDA_BF16) {
        SPARDA_ATT_D(SPARDA_BF16);
    } else {
        SPARDA_ATT_D(SPARDA_F32);
    }
#undef SPARDA_ATT_D
#undef SPARDA_ATT
    return check_hip(hipGetLastError(), "decode_attend_kernel");
}

}  // namespace sparda
