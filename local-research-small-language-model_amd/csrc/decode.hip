// Single-token decode step of the sparse attention layer, two launches and
// no cross-workgroup synchronisation inside a kernel (a device-scope fence
// writes back and invalidates the XCD's L2 on this part, which serialises
// thousands of workgroups):
//
//  1. decode_score_kernel, grid (NB, B): each workgroup streams one KV block
//     of the cache (all KV heads), forms its prototypes (sequential fp32 sum,
//     / bs) and the forecast score of every head. This is the HBM-bound pass:
//     it reads the whole K cache once.
//  2. decode_attend_kernel, grid (Hkv, B): one workgroup per (sequence, KV
//     head) derives the selection from the scores with a wavefront ballot
//     threshold search (the k-th largest orderable key, ties by lower index),
//     then one wavefront per selected block reads that block's K/V once and
//     serves all Hq/Hkv query heads of the group (split-K partial: m, l, o);
//     the partials are merged in LDS in slot order.
//
// Dense (NB <= k+2) and static-window (no forecast) steps skip launch 1: the
// attend kernel derives those selections from the block counts.
#pragma clang fp contract(off)

#include "common.h"
#include "kernels.h"
#include "attend.h"

namespace sparda {

[[maybe_unused]] constexpr float kLog2e = 1.4426950408889634f;

static size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

DecodeWs decode_ws_layout(void* base, int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D,
                          int64_t bs, int64_t k) {
    (void)Hq;
    (void)D;
    (void)k;
    const int64_t NB = cdiv(S, bs);
    char* p = static_cast<char*>(base);
    size_t off = 0;
    DecodeWs w{};
    w.scores = reinterpret_cast<float*>(p + off);
    off += align256(static_cast<size_t>(B * Hkv * NB) * 4);
    w.bytes = off;
    return w;
}

// ---------------------------------------------------------------------------
// launch 1: compress + score; block = H*D/VEC threads, thread -> (h, d-group)
// ---------------------------------------------------------------------------
template <int DT, int FDT, int VEC, int UNROLL>
__global__ void __launch_bounds__(256)
decode_score_kernel(const void* __restrict__ kc, int64_t kv_sb, int64_t kv_ss, int64_t kv_sh,
                    int64_t S, int H, int D, int bs, int64_t NB,
                    const void* __restrict__ f, int64_t f_sb, int64_t f_sh, float scale,
                    int64_t score_pos0, const float* __restrict__ protos_in,
                    float* __restrict__ protos_out, float* __restrict__ ws_scores) {
    extern __shared__ float smem[];
    float* p_lds = smem;            // [H*D]
    float* f_lds = smem + H * D;    // [H*D]
    const int j = blockIdx.x;
    const int b = blockIdx.y;
    const int groups = D / VEC;
    const int HD = H * D;

    for (int e = threadIdx.x; e < H * groups; e += blockDim.x) {
        const int h = e / groups;
        const int d = (e % groups) * VEC;
        const int64_t pidx = ((static_cast<int64_t>(b) * NB + j) * H + h) * D + d;
        if (protos_in != nullptr) {
#pragma unroll
            for (int v = 0; v < VEC; ++v) p_lds[h * D + d + v] = protos_in[pidx + v];
        } else {
            const int64_t s0 = static_cast<int64_t>(j) * bs;
            const int64_t s1 = s0 + bs < S ? s0 + bs : S;
            float acc[VEC];
            block_sum<DT, VEC, UNROLL>(kc, b * kv_sb + h * kv_sh + d, s0, s1, kv_ss, acc);
            const float den = static_cast<float>(bs);
#pragma unroll
            for (int v = 0; v < VEC; ++v) {
                const float p = acc[v] / den;
                p_lds[h * D + d + v] = p;
                if (protos_out != nullptr) protos_out[pidx + v] = p;
            }
        }
    }
    for (int e = threadIdx.x; e < HD; e += blockDim.x)
        f_lds[e] = load_elem<FDT>(f, b * f_sb + (e / D) * f_sh + (e % D));
    __syncthreads();

    // scores: fma chain over d (canonical order), causal mask at score_pos0
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
}

// ---------------------------------------------------------------------------
// Wavefront top-k selection by ballot threshold search.
// The wave holds keys[j] (orderable score keys, index = block) for
// j = e*64 + lane in kreg[e]. Writes to sel_lds the ascending list
// ({0, own} U topk) restricted to blocks <= own, returns its length.
// topk = the k largest keys, equal keys by lower index. Called by a whole
// wavefront; all control flow is wave-uniform.
// ---------------------------------------------------------------------------
template <int CH>
__device__ __forceinline__ int wave_select(const uint32_t (&kreg)[CH], int n, int k, int own,
                                           int32_t* sel_lds) {
    const int lane = threadIdx.x % kWave;
    // T = the k-th largest key: the largest T with count(key >= T) >= k
    uint32_t T = 0;
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t c = T | (1u << bit);
        int cnt = 0;
#pragma unroll
        for (int e = 0; e < CH; ++e) cnt += __popcll(__ballot(e * kWave + lane < n && kreg[e] >= c));
        if (cnt >= k) T = c;
    }
    int above = 0;
#pragma unroll
    for (int e = 0; e < CH; ++e) above += __popcll(__ballot(e * kWave + lane < n && kreg[e] > T));
    int need_eq = k - above;  // keys equal to T, taken in index order
    const uint64_t lanes_below = (1ull << lane) - 1ull;
    int m = 0;
#pragma unroll
    for (int e = 0; e < CH; ++e) {
        const int j = e * kWave + lane;
        const bool in = j < n;
        const uint64_t gt = __ballot(in && kreg[e] > T);
        uint64_t eq = __ballot(in && kreg[e] == T);
        uint64_t keep = 0;
        for (; need_eq > 0 && eq != 0; --need_eq) {
            const uint64_t low = eq & (~eq + 1ull);
            keep |= low;
            eq ^= low;
        }
        const uint64_t forced = __ballot(in && (j == 0 || j == own));
        const uint64_t take = (gt | keep | forced) & __ballot(in && j <= own);
        if ((take >> lane) & 1ull) sel_lds[m + __popcll(take & lanes_below)] = j;
        m += __popcll(take);
    }
    return m;
}

// ---------------------------------------------------------------------------
// launch 2: selection + attention over the selected blocks + merge, one
// workgroup per (sequence, KV head), W wavefronts; wavefront w serves the
// selected blocks w, w+W, ... sel_mode: 0 top-k of the launch-1 scores,
// 1 dense (all blocks), 2 window {0} U [cb-k+1, cb].
// For a block, lane i holds key row j*bs + i of K in registers and stages
// the V row in the wave's LDS region (16-byte loads); it scores the R query
// heads of the group (4 at a time), keeps a running (m, l, o) per head over
// the block's 64-key chunks, and parks the block's partial in its slot's LDS
// region. After a barrier the partials are merged in slot order.
// ---------------------------------------------------------------------------
constexpr int kMaxGroup = 16;   // query heads per KV head
constexpr int kMaxSlots = 34;   // k + 2 with k <= 32
constexpr int kHeadBatch = 4;

template <int DT>
struct KvElem { using T = float; };
template <>
struct KvElem<SPARDA_BF16> { using T = uint16_t; };

template <int DT, int DH>
__host__ __device__ constexpr int v_row_elems() { return DT == SPARDA_BF16 ? DH + 8 : DH + 4; }

template <int DT, int DH>
__host__ __device__ constexpr size_t attend_wave_bytes() {
    return static_cast<size_t>(kHeadBatch * 64) * 4 +
           static_cast<size_t>(64 * v_row_elems<DT, DH>()) * (DT == SPARDA_BF16 ? 2 : 4);
}

constexpr int kAttendMaxWaves = 12;

template <int DT, int DH, int CH>
__global__ void __launch_bounds__(kAttendMaxWaves * 64)
decode_attend_kernel(const void* __restrict__ q, int64_t q_sb, int64_t q_sh,
                     const void* __restrict__ kc, const void* __restrict__ vc,
                     int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int64_t S, int Hq, int H, int bs,
                     int64_t NB, int k, int sel_mode, int cap, float scale_log2,
                     const float* __restrict__ ws_scores,
                     int32_t* __restrict__ sel_out, int32_t* __restrict__ n_sel_out,
                     void* __restrict__ out, int64_t out_sb) {
    using E = typename KvElem<DT>::T;
    constexpr int VR = v_row_elems<DT, DH>();
    constexpr int KW = DT == SPARDA_BF16 ? DH / 2 : DH;  // K row words per lane
    constexpr int DPL = (DH + kWave - 1) / kWave;         // output dims per lane
    extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];
    __shared__ float q_lds[kMaxGroup * DH];
    __shared__ int32_t sel_lds[kMaxSlots + 6];
    __shared__ int n_lds;

    const int g = blockIdx.x;
    const int b = blockIdx.y;
    const int R = Hq / H;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int nwaves = blockDim.x / kWave;
    const int64_t bg = static_cast<int64_t>(b) * H + g;
    const int cb = static_cast<int>((S - 1) / bs);
    float* part_all = reinterpret_cast<float*>(dyn);                       // [cap][R][DH+2]
    const size_t part_bytes = ((static_cast<size_t>(cap) * R * (DH + 2) * 4) + 15) & ~static_cast<size_t>(15);
    unsigned char* wbase = dyn + part_bytes + wave * attend_wave_bytes<DT, DH>();
    float* p_lds = reinterpret_cast<float*>(wbase);                         // [4][64]
    E* v_lds = reinterpret_cast<E*>(wbase + kHeadBatch * 64 * 4);           // [64][VR]

    for (int e = threadIdx.x; e < R * DH; e += blockDim.x) {
        const int hh = e / DH, d = e % DH;
        q_lds[e] = load_elem<DT>(q, b * q_sb + static_cast<int64_t>(g * R + hh) * q_sh + d) * scale_log2;
    }
    if (wave == 0) {
        int m = 0;
        if (sel_mode == 0) {
            const float* srow = ws_scores + bg * NB;
            uint32_t kreg[CH];
#pragma unroll
            for (int e = 0; e < CH; ++e) {
                const int j = e * kWave + lane;
                kreg[e] = j < NB ? order_key(srow[j]) : 0u;
            }
            m = wave_select<CH>(kreg, static_cast<int>(NB), k, cb, sel_lds);
        } else if (sel_mode == 1) {
            for (int j = lane; j <= cb; j += kWave) sel_lds[j] = j;
            m = cb + 1;
        } else {
            int lo = cb - k + 1;
            if (lo < 0) lo = 0;
            const int lead = lo > 0 ? 1 : 0;
            m = cb - lo + 1 + lead;
            if (lane < m) sel_lds[lane] = (lead && lane == 0) ? 0 : lo + lane - lead;
        }
        if (lane == 0) n_lds = m;
    }
    __syncthreads();
    const int n = n_lds;
    if (threadIdx.x < cap) {
        if (sel_out != nullptr) sel_out[bg * cap + threadIdx.x] = threadIdx.x < n ? sel_lds[threadIdx.x] : -1;
        if (threadIdx.x == 0 && n_sel_out != nullptr) n_sel_out[bg] = n;
    }

    for (int w = wave; w < n; w += nwaves) {
        const int64_t j = sel_lds[w];
        const int64_t s0 = j * bs;
        const int64_t s1 = s0 + bs < S ? s0 + bs : S;
        float* part = part_all + static_cast<int64_t>(w) * R * (DH + 2);
        for (int hb = 0; hb < R; hb += kHeadBatch) {
            const int nh = R - hb < kHeadBatch ? R - hb : kHeadBatch;
            float mrun[kHeadBatch], lrun[kHeadBatch], orun[kHeadBatch][DPL];
#pragma unroll
            for (int hh = 0; hh < kHeadBatch; ++hh) {
                mrun[hh] = -__builtin_inff();
                lrun[hh] = 0.0f;
#pragma unroll
                for (int i = 0; i < DPL; ++i) orun[hh][i] = 0.0f;
            }
            for (int64_t c0 = s0; c0 < s1; c0 += kWave) {
                const int nk = static_cast<int>(s1 - c0 < kWave ? s1 - c0 : kWave);
                // coalesced block reads: chunk c -> row c / RC, 16-byte column c % RC
                constexpr int EPV = 16 / sizeof(E);     // elements per 16-byte chunk
                constexpr int RC = DH / EPV;            // chunks per row
                constexpr int NC = 64 * RC / kWave;     // chunks per lane
                uint4 kraw[NC], vraw[NC];
                const int64_t base = b * kv_sb + c0 * kv_ss + g * kv_sh;
#pragma unroll
                for (int i = 0; i < NC; ++i) {
                    const int c = lane + i * kWave;
                    const int row = c / RC, col = (c % RC) * EPV;
                    if (row < nk) {
                        kraw[i] = *reinterpret_cast<const uint4*>(static_cast<const E*>(kc) + base + row * kv_ss + col);
                        vraw[i] = *reinterpret_cast<const uint4*>(static_cast<const E*>(vc) + base + row * kv_ss + col);
                    } else {
                        kraw[i] = make_uint4(0u, 0u, 0u, 0u);
                        vraw[i] = make_uint4(0u, 0u, 0u, 0u);
                    }
                }
                // K through the wave's LDS buffer into lane = key rows
#pragma unroll
                for (int i = 0; i < NC; ++i) {
                    const int c = lane + i * kWave;
                    *reinterpret_cast<uint4*>(v_lds + (c / RC) * VR + (c % RC) * EPV) = kraw[i];
                }
                __builtin_amdgcn_wave_barrier();
                uint32_t kw[KW];
#pragma unroll
                for (int i = 0; i < RC; ++i) {
                    const uint4 w4 = *reinterpret_cast<const uint4*>(v_lds + lane * VR + i * EPV);
                    kw[4 * i] = w4.x;
                    kw[4 * i + 1] = w4.y;
                    kw[4 * i + 2] = w4.z;
                    kw[4 * i + 3] = w4.w;
                }
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int i = 0; i < NC; ++i) {
                    const int c = lane + i * kWave;
                    *reinterpret_cast<uint4*>(v_lds + (c / RC) * VR + (c % RC) * EPV) = vraw[i];
                }
                for (int hh = 0; hh < nh; ++hh) {
                    const float* qh = q_lds + (hb + hh) * DH;
                    float sc = -__builtin_inff();
                    if (lane < nk) {
                        float a = 0.0f;
#pragma unroll
                        for (int i = 0; i < KW; ++i) {
                            if constexpr (DT == SPARDA_BF16) {
                                a = fmaf(qh[2 * i], __uint_as_float(kw[i] << 16), a);
                                a = fmaf(qh[2 * i + 1], __uint_as_float(kw[i] & 0xffff0000u), a);
                            } else {
                                a = fmaf(qh[i], __uint_as_float(kw[i]), a);
                            }
                        }
                        sc = a;
                    }
                    const float mc = wave_max(sc);
                    const float m_new = fmaxf(mrun[hh], mc);
                    const float alpha = exp2f(mrun[hh] - m_new);
                    const float p = lane < nk ? exp2f(sc - m_new) : 0.0f;
                    lrun[hh] = lrun[hh] * alpha + wave_sum(p);
                    mrun[hh] = m_new;
                    p_lds[hh * 64 + lane] = p;
#pragma unroll
                    for (int i = 0; i < DPL; ++i) orun[hh][i] *= alpha;
                }
                __builtin_amdgcn_wave_barrier();
                // o[d] += sum_key p[key] * V[key][d]; rows >= nk are zero with p = 0
#pragma unroll
                for (int i = 0; i < DPL; ++i) {
                    const int d = lane + i * kWave;
                    if (d < DH) {
                        float acc[kHeadBatch] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 16
                        for (int key = 0; key < 64; key += 4) {
                            float vv[4];
#pragma unroll
                            for (int u = 0; u < 4; ++u) {
                                if constexpr (DT == SPARDA_BF16) vv[u] = bf16_to_f32(v_lds[(key + u) * VR + d]);
                                else vv[u] = v_lds[(key + u) * VR + d];
                            }
#pragma unroll
                            for (int hh = 0; hh < kHeadBatch; ++hh) {
                                if (hh < nh) {
                                    const float4 p4 = *reinterpret_cast<const float4*>(p_lds + hh * 64 + key);
                                    acc[hh] = fmaf(p4.x, vv[0], acc[hh]);
                                    acc[hh] = fmaf(p4.y, vv[1], acc[hh]);
                                    acc[hh] = fmaf(p4.z, vv[2], acc[hh]);
                                    acc[hh] = fmaf(p4.w, vv[3], acc[hh]);
                                }
                            }
                        }
#pragma unroll
                        for (int hh = 0; hh < kHeadBatch; ++hh)
                            if (hh < nh) orun[hh][i] += acc[hh];
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
            for (int hh = 0; hh < nh; ++hh) {
                float* pp = part + (hb + hh) * (DH + 2);
                if (lane == 0) {
                    pp[0] = mrun[hh];
                    pp[1] = lrun[hh];
                }
#pragma unroll
                for (int i = 0; i < DPL; ++i) {
                    const int d = lane + i * kWave;
                    if (d < DH) pp[2 + d] = orun[hh][i];
                }
            }
        }
    }
    __syncthreads();

    // merge the partials in slot order
    for (int e = threadIdx.x; e < R * DH; e += blockDim.x) {
        const int hh = e / DH, d = e % DH;
        float M = -__builtin_inff();
        for (int w = 0; w < n; ++w) M = fmaxf(M, part_all[(w * R + hh) * (DH + 2)]);
        float num = 0.0f, den = 0.0f;
        for (int w = 0; w < n; ++w) {
            const float* ps = part_all + (w * R + hh) * (DH + 2);
            const float wt = exp2f(ps[0] - M);
            den = den + wt * ps[1];
            num = num + wt * ps[2 + d];
        }
        store_elem<DT>(out, b * out_sb + static_cast<int64_t>(g * R + hh) * DH + d, num / den);
    }
    __syncthreads();
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
        const int esz = dtype == SPARDA_F32 ? 4 : 2;
        auto fits = [&](int v) {
            return (D % v == 0) && (kv_sb % v == 0) && (kv_ss % v == 0) && (kv_sh % v == 0) &&
                   (reinterpret_cast<uintptr_t>(kc) % (static_cast<uintptr_t>(v) * esz) == 0);
        };
        // 4-byte (2 x bf16) loads per lane measured faster than 8-byte ones for this pass
        const int vec = fits(2) ? 2 : 1;
        int threads = static_cast<int>(Hkv * D / vec);
        if (threads > 256) threads = 256;
        threads = ((threads + kWave - 1) / kWave) * kWave;
        const size_t lds = static_cast<size_t>(2 * Hkv * D) * sizeof(float);
        const int64_t score_pos0 = (routing == SPARDA_ROUTE_ABSOLUTE) ? S - 1 : 0;
        dim3 grid(static_cast<unsigned>(NB), static_cast<unsigned>(B));
#define SPARDA_SC(DT_, FDT_, V_, U_)                                                              \
    hipLaunchKernelGGL((decode_score_kernel<DT_, FDT_, V_, U_>), grid, dim3(threads), lds, stream, \
                       kc, kv_sb, kv_ss, kv_sh, S, static_cast<int>(Hkv), static_cast<int>(D),   \
                       static_cast<int>(bs), NB, f, f_sb, f_sh, scale, score_pos0, protos_in,    \
                       protos_out, ws.scores)
#define SPARDA_SC_U(DT_, FDT_, V_)                      \
    if (bs == 64) SPARDA_SC(DT_, FDT_, V_, 64);         \
    else if (bs == 32) SPARDA_SC(DT_, FDT_, V_, 32);    \
    else SPARDA_SC(DT_, FDT_, V_, 0);
#define SPARDA_SC_V(DT_, FDT_)                          \
    if (vec == 4) { SPARDA_SC_U(DT_, FDT_, 4) }         \
    else if (vec == 2) { SPARDA_SC_U(DT_, FDT_, 2) }    \
    else { SPARDA_SC_U(DT_, FDT_, 1) }
        if (dtype == SPARDA_BF16) {
            if (fdtype == SPARDA_BF16) { SPARDA_SC_V(SPARDA_BF16, SPARDA_BF16) }
            else { SPARDA_SC_V(SPARDA_BF16, SPARDA_F32) }
        } else {
            if (fdtype == SPARDA_BF16) { SPARDA_SC_V(SPARDA_F32, SPARDA_BF16) }
            else { SPARDA_SC_V(SPARDA_F32, SPARDA_F32) }
        }
#undef SPARDA_SC_V
#undef SPARDA_SC_U
#undef SPARDA_SC
        int rc = check_hip(hipGetLastError(), "decode_score_kernel");
        if (rc) return rc;
    }
    const float scale_log2 = scale * kLog2e;
    const int Hq_i = static_cast<int>(Hq), Hkv_i = static_cast<int>(Hkv);
    const size_t part_bytes = ((static_cast<size_t>(cap) * (Hq / Hkv) * (D + 2) * 4) + 15) & ~static_cast<size_t>(15);
    constexpr size_t kLdsBudget = 150 * 1024;
    dim3 grid2(static_cast<unsigned>(Hkv), static_cast<unsigned>(B));
#define SPARDA_ATT(DT_, DH_, CH_)                                                                        \
    do {                                                                                                 \
        const size_t wb = attend_wave_bytes<DT_, DH_>();                                                 \
        int waves = cap < kAttendMaxWaves ? cap : kAttendMaxWaves;                                                                 \
        while (waves > 1 && part_bytes + waves * wb > kLdsBudget) --waves;                              \
        hipLaunchKernelGGL((decode_attend_kernel<DT_, DH_, CH_>), grid2, dim3(waves * kWave),            \
                           part_bytes + waves * wb, stream, q, q_sb, q_sh, kc, vc, kv_sb, kv_ss, kv_sh,   \
                           S, Hq_i, Hkv_i, static_cast<int>(bs), NB, static_cast<int>(k), sel_mode, cap, \
                           scale_log2, ws.scores, sel_out, n_sel_out, out, out_sb);                      \
    } while (0)
#define SPARDA_ATT_C(DT_, DH_)                            \
    if (NB <= 256) SPARDA_ATT(DT_, DH_, 4);               \
    else if (NB <= 1024) SPARDA_ATT(DT_, DH_, 16);        \
    else SPARDA_ATT(DT_, DH_, 64);
#define SPARDA_ATT_D(DT_)                                         \
    switch (D) {                                                  \
        case 16: { SPARDA_ATT_C(DT_, 16) } break;                 \
        case 32: { SPARDA_ATT_C(DT_, 32) } break;                 \
        case 64: { SPARDA_ATT_C(DT_, 64) } break;                 \
        default: { SPARDA_ATT_C(DT_, 128) } break;                \
    }
    if (dtype == SPARDA_BF16) {
        SPARDA_ATT_D(SPARDA_BF16);
    } else {
        SPARDA_ATT_D(SPARDA_F32);
    }
#undef SPARDA_ATT_D
#undef SPARDA_ATT_C
#undef SPARDA_ATT
    return check_hip(hipGetLastError(), "decode_attend_kernel");
}

}  // namespace sparda
