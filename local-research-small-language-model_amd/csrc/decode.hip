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
#include "mfma.h"
#include "prefetch.h"
#include "select.h"

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
            if (D == 64) {
                // the same chain; the operands of each 16 steps read with 16-byte
                // LDS loads ahead of their fmas (the chain, not the reads, is serial)
                const float4* fr4 = reinterpret_cast<const float4*>(f_lds + h * 64);
                const float4* pr4 = reinterpret_cast<const float4*>(p_lds + h * 64);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    float4 fv[4], pv[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        fv[i] = fr4[4 * c + i];
                        pv[i] = pr4[4 * c + i];
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        acc = __fmaf_rn(fv[i].x, pv[i].x, acc);
                        acc = __fmaf_rn(fv[i].y, pv[i].y, acc);
                        acc = __fmaf_rn(fv[i].z, pv[i].z, acc);
                        acc = __fmaf_rn(fv[i].w, pv[i].w, acc);
                    }
                }
            } else {
                for (int d = 0; d < D; ++d) acc = __fmaf_rn(f_lds[h * D + d], p_lds[h * D + d], acc);
            }
            s = acc * scale;
        }
        ws_scores[(static_cast<int64_t>(b) * H + h) * NB + j] = s;
    }
}

// ---------------------------------------------------------------------------
// launch 2: selection + attention over the selected blocks + merge, one
// workgroup per (sequence, KV head), W wavefronts; wavefront w serves the
// selected blocks w, w+W, ... sel_mode: 0 top-k of the launch-1 scores,
// 1 dense (all blocks), 2 window {0} U [cb-k+1, cb] (every block while
// cb+1 <= k+2), 3 the caller's list, 4 top-k of scores formed here from
// block sums (cached prototypes; every block while cb+1 <= k+2). With pos_dev
// the length comes from device memory (S = *pos_dev + 1, clamped to the S
// argument).
// For a block, lane i holds key row j*bs + i of K in registers and stages
// the V row in the wave's LDS region (16-byte loads); it scores the R query
// heads of the group (4 at a time), keeps a running (m, l, o) per head over
// the block's 64-key chunks, and parks the block's partial in its slot's LDS
// region. After a barrier the partials are merged in slot order.
// ---------------------------------------------------------------------------
constexpr int kMaxGroup = 16;   // query heads per KV head
constexpr int kMaxSlots = kMaxSelCap;
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

// Matrix-core block attention (bf16, D = 64, bs = 64): per block and wave,
// S^T[key, head] = K . Q^T with v_mfma_f32_16x16x32_bf16 (the group's query
// heads are the 16 columns; K operands are read straight from memory),
// softmax in fp32 registers, O^T += V^T . P^T (V staged row-major in the
// wave's LDS region, read transposed), row sums on the matrix cores.
constexpr int kDVRow = 80;  // V row in LDS for the matrix-core path, bf16 elements

template <int DT, int DH, int CH, bool MF, int MBS = 64>
__global__ void __launch_bounds__(kAttendMaxWaves * 64)
decode_attend_kernel(const void* __restrict__ q, int64_t q_sb, int64_t q_sh,
                     const void* __restrict__ kc, const void* __restrict__ vc,
                     int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int64_t S_arg, int Hq, int H, int bs,
                     int64_t NB, int k, int sel_mode, int cap, float scale_log2,
                     const float* __restrict__ ws_scores,
                     const int32_t* __restrict__ sel_in, const int32_t* __restrict__ n_sel_in,
                     int compact, const void* __restrict__ k_new, const void* __restrict__ v_new,
                     int64_t new_sb, int64_t new_sh,
                     int32_t* __restrict__ sel_out, int32_t* __restrict__ n_sel_out,
                     void* __restrict__ out, int64_t out_sb, const int64_t* __restrict__ pos_dev,
                     float* sums, int64_t nb_stride, int update_sums, const void* __restrict__ fsel,
                     int fsel_bf16, int64_t fs_sb, int64_t fs_sh, int absolute, float fscale, int pow2,
                     PrefetchDev pf, int nsplit, int split_blocks, float* __restrict__ ws_part) {
    using E = typename KvElem<DT>::T;
    constexpr int VR = v_row_elems<DT, DH>();
    constexpr int KW = DT == SPARDA_BF16 ? DH / 2 : DH;  // K row words per lane
    constexpr int DPL = (DH + kWave - 1) / kWave;         // output dims per lane
    extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];
    __shared__ float q_lds[kMaxGroup * DH];
    __shared__ int32_t sel_lds[kMaxSlots + 6];
    __shared__ uint32_t ck_lds[kWave];  // selection candidates (keys, block indices)
    __shared__ int32_t ci_lds[kWave];
    __shared__ float fsel_lds[DH];      // forecast of the selection from block sums
    __shared__ int n_lds;

    const int g = blockIdx.x;
    const int b = blockIdx.y;
    // blockIdx.z < nsplit: split z of the (sequence, KV head)'s slots, slots
    // [z * split_blocks, (z + 1) * split_blocks) (nsplit > 1 only for the
    // matrix-core dense mode with a workspace)
    const int split = static_cast<int>(blockIdx.z);
    if constexpr (MF) {
        // blockIdx.z = nsplit: the next layer's prefetch for (b, g), carried by
        // this launch so that its selection and host-link copy run beside the
        // attention workgroups (the host adds that z only with pf filled in)
        if (split >= nsplit) {
            prefetch_workgroup<CH, DH>(pf, g, b, pos_dev, fsel_lds, reinterpret_cast<uint32_t*>(dyn), sel_lds, ck_lds,
                                       ci_lds, &n_lds);
            return;
        }
    }
    const int R = Hq / H;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int nwaves = blockDim.x / kWave;
    const int64_t bg = static_cast<int64_t>(b) * H + g;
    // with pos_dev the query is token *pos_dev (clamped into [0, S_arg)): S = *pos_dev + 1
    int64_t S = S_arg;
    if (pos_dev != nullptr) {
        const int64_t p = *pos_dev;
        S = p < 0 ? 1 : (p >= S_arg ? S_arg : p + 1);
    }
    const int cb = static_cast<int>((S - 1) / bs);
    float* part_all = reinterpret_cast<float*>(dyn);                       // [nwaves][R][DH+2]
    const size_t part_bytes = ((static_cast<size_t>(nwaves) * R * (DH + 2) * 4) + 15) & ~static_cast<size_t>(15);
    unsigned char* wbase = dyn + part_bytes + wave * attend_wave_bytes<DT, DH>();
    float* p_lds = reinterpret_cast<float*>(wbase);                         // [4][64]
    E* v_lds = reinterpret_cast<E*>(wbase + kHeadBatch * 64 * 4);           // [64][VR]

    if constexpr (!MF) {  // the matrix-core path reads q into registers instead
        for (int e = threadIdx.x; e < R * DH; e += blockDim.x) {
            const int hh = e / DH, d = e % DH;
            q_lds[e] = load_elem<DT>(q, b * q_sb + static_cast<int64_t>(g * R + hh) * q_sh + d) * scale_log2;
        }
    }
    // sel_mode 4: every thread scores present blocks from the block sums (as
    // select_decode_kernel does), keys parked in the dynamic region until the
    // selection is made
    uint32_t* key_lds = reinterpret_cast<uint32_t*>(dyn);
    const bool dense4 = cb + 1 <= k + 2;
    constexpr int kSumBatch = DH / 4 < 4 ? DH / 4 : 4;  // 16-byte loads in flight per score (register budget)
    if (sel_mode == 4) {
        for (int d = threadIdx.x; d < DH; d += blockDim.x) {
            const int64_t fi = b * fs_sb + g * fs_sh + d;
            fsel_lds[d] = fsel_bf16 ? load_elem<SPARDA_BF16>(fsel, fi) : load_elem<SPARDA_F32>(fsel, fi);
        }
        __syncthreads();  // fsel_lds
        // the last DH/2 threads re-sum the current block while the others
        // score the blocks before it; its score follows in wave 0
        const int rs0 = static_cast<int>(blockDim.x) - DH / 2;
        if (update_sums && static_cast<int>(threadIdx.x) >= rs0) {
            // the current block's sums of head g from its rows [cb*bs, S), in
            // row order (block_sums_kernel's order), 32 row loads in flight
            const int dd = 2 * (static_cast<int>(threadIdx.x) - rs0);
            const int64_t s0 = static_cast<int64_t>(cb) * bs;
            const int nr = static_cast<int>(S - s0);
            const int64_t base = b * kv_sb + g * kv_sh + dd;
            float a0 = 0.0f, a1 = 0.0f;
            for (int c0 = 0; c0 < nr; c0 += 32) {
                float buf[32][2];
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    const int r = c0 + i < nr ? c0 + i : nr - 1;
                    load_vec<DT, 2>(kc, base + (s0 + r) * kv_ss, buf[i]);
                }
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    if (c0 + i < nr) {
                        a0 = a0 + buf[i][0];
                        a1 = a1 + buf[i][1];
                    }
                }
            }
            float* cur = sums + ((b * nb_stride + cb) * H + g) * DH + dd;
            cur[0] = a0;
            cur[1] = a1;
        }
        if (!dense4) {
            const float den = static_cast<float>(bs);
            const float inv = 1.0f / den;
            const int limit = absolute ? cb : 0;
            const int jend = update_sums ? cb - 1 : cb;  // the current block is scored after the re-sum
            for (int j = threadIdx.x; j <= jend; j += blockDim.x) {
                const float* sp = sums + ((b * nb_stride + j) * H + g) * DH;
                const float sc = j > limit ? -__builtin_inff()
                                           : (pow2 ? score_from_sum<DH, true, kSumBatch>(sp, fsel_lds, den, inv, fscale)
                                                   : score_from_sum<DH, false, kSumBatch>(sp, fsel_lds, den, inv,
                                                                                          fscale));
                key_lds[j] = order_key(sc);
            }
        }
        __syncthreads();
    }
    if (wave == 0) {
        int m = 0;
        if (sel_mode == 4 && update_sums && !dense4) {
            // the current block's key from its fresh sums (stored before the barrier)
            if (lane == 0) {
                const float den = static_cast<float>(bs);
                const float* sp = sums + ((b * nb_stride + cb) * H + g) * DH;
                const float sc = cb > (absolute ? cb : 0)
                                     ? -__builtin_inff()
                                     : (pow2 ? score_from_sum<DH, true, kSumBatch>(sp, fsel_lds, den, 1.0f / den, fscale)
                                             : score_from_sum<DH, false, kSumBatch>(sp, fsel_lds, den, 1.0f / den,
                                                                                    fscale));
                key_lds[cb] = order_key(sc);
            }
            __builtin_amdgcn_wave_barrier();
        }
        if (sel_mode == 4) {
            if (dense4) {
                m = cb + 1;  // every block 0..cb
                if (lane < m) sel_lds[lane] = lane;
            } else {
                m = select_keys_upto<CH>(key_lds, cb + 1, k, cb, sel_lds, lane, ck_lds, ci_lds);
            }
        } else if (sel_mode == 0) {
            const float* srow = ws_scores + bg * NB;
            uint32_t kreg[CH];
#pragma unroll
            for (int e = 0; e < CH; ++e) {
                const int j = e * kWave + lane;
                kreg[e] = j < NB ? order_key(srow[j]) : 0u;
            }
            m = wave_select_pre<CH>(kreg, static_cast<int>(NB), k, cb, sel_lds, ck_lds, ci_lds);
        } else if (sel_mode == 1) {
            m = cb + 1;  // slot w is block w; sel_lds is not used
        } else if (sel_mode == 3) {
            m = n_sel_in[bg];
            m = m < 0 ? 0 : (m > cap ? cap : m);
            if (lane < m) sel_lds[lane] = sel_in[bg * cap + lane];
        } else if (cb + 1 <= k + 2) {
            m = cb + 1;  // window mode on a short cache: every block (the host picks mode 1 for these)
            if (lane < m) sel_lds[lane] = lane;
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
    // this workgroup's slots [s_lo, s_hi): all of them, or those of split `split`
    const int s_per = nsplit > 1 ? split_blocks : n;
    const int s_lo = split * s_per < n ? split * s_per : n;
    const int s_hi = s_lo + s_per < n ? s_lo + s_per : n;
    if (split == 0 && threadIdx.x < cap) {
        const int i = threadIdx.x;
        if (sel_out != nullptr) sel_out[bg * cap + i] = i < n ? (sel_mode == 1 ? i : sel_lds[i]) : -1;
        if (i == 0 && n_sel_out != nullptr) n_sel_out[bg] = n;
    }

    float* part = part_all + static_cast<int64_t>(wave) * R * (DH + 2);
    if constexpr (MF) {
        static_assert(DH == 64, "matrix-core decode path is for head dim 64");
        const int col16 = lane % 16;
        const int grp = lane / 16;
        constexpr int kBs = MBS;           // keys per block: 64 or 32
        constexpr int kSub = kBs / 16;     // 16-key sub-tiles (the M side of S^T)
        constexpr int kHalf = kBs / 32;    // 32-key halves (the K side of O^T)
        constexpr int kVC = kBs / 8;       // 16-byte V chunks per lane
        static_assert(kBs == 64 || kBs == 32, "matrix-core decode: blocks of 64 or 32 keys");
        constexpr float kLazy = 8.0f;
        uint16_t* vt = reinterpret_cast<uint16_t*>(wbase);  // [64][kDVRow]
        const uint16_t* qh = static_cast<const uint16_t*>(q);
        const uint16_t* kh = static_cast<const uint16_t*>(kc);
        const uint16_t* vh = static_cast<const uint16_t*>(vc);
        const uint16_t* knh = static_cast<const uint16_t*>(k_new);
        const uint16_t* vnh = static_cast<const uint16_t*>(v_new);
        // B operand of S^T: column col16 = query head of the group (zero past R)
        bf16x8 qb0, qb1;
        {
            uint4 a = make_uint4(0u, 0u, 0u, 0u), c = a;
            if (col16 < R) {
                const uint16_t* qp = qh + b * q_sb + static_cast<int64_t>(g * R + col16) * q_sh + 8 * grp;
                a = *reinterpret_cast<const uint4*>(qp);
                c = *reinterpret_cast<const uint4*>(qp + 32);
            }
            qb0 = __builtin_bit_cast(bf16x8, a);
            qb1 = __builtin_bit_cast(bf16x8, c);
        }
        bf16x8 ones_a;
#pragma unroll
        for (int e = 0; e < 8; ++e) ones_a[e] = static_cast<__bf16>(col16 == 0 ? 1.0f : 0.0f);
        f32x4 o[4], ol = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        float m_run = -__builtin_inff();
        const int64_t nbase = b * new_sb + g * new_sh;
        for (int w = s_lo + wave; w < s_hi; w += nwaves) {
            const int64_t j = sel_mode == 1 ? w : sel_lds[w];
            if (j < 0 || j > cb) continue;  // not a block of [0, S): nothing to attend
            const int64_t s0 = j * kBs;
            const int nk = static_cast<int>(S - s0 < kBs ? S - s0 : kBs);
            const int64_t row0 = compact ? static_cast<int64_t>(w) * kBs : s0;
            const int64_t base = b * kv_sb + row0 * kv_ss + g * kv_sh;
            // the row holding position S-1 when its K/V come from k_new/v_new (else -1)
            const int rnew = (knh != nullptr && S - 1 - s0 < kBs) ? static_cast<int>(S - 1 - s0) : -1;
            // V rows: 512 chunks of 16 B, lane -> chunks lane + 64 i (row c/8, chunk c%8,
            // the same chunk column lane%8 for every i); rows past S repeat row nk-1
            // (finite values; their P is 0)
            const uint16_t* vrow0 = vh + base + (lane % 8) * 8;
            uint4 vr[kVC];
#pragma unroll
            for (int i = 0; i < kVC; ++i) {
                int r = (lane + 64 * i) / 8;
                r = r < nk ? r : nk - 1;
                vr[i] = *reinterpret_cast<const uint4*>(vrow0 + r * kv_ss);
            }
            // K A operands: key 16n + col16, dims 32kk + 8grp .. +7
            const uint16_t* krow0 = kh + base + 8 * grp;
            bf16x8 ka[kSub][2];
#pragma unroll
            for (int nn = 0; nn < kSub; ++nn) {
                int r = 16 * nn + col16;
                r = r < nk ? r : nk - 1;
#pragma unroll
                for (int kk = 0; kk < 2; ++kk)
                    ka[nn][kk] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(krow0 + r * kv_ss + 32 * kk));
            }
            if (rnew >= 0) {  // wave-uniform: the new token's row from k_new / v_new
                const uint4 vn = *reinterpret_cast<const uint4*>(vnh + nbase + (lane % 8) * 8);
                const bf16x8 kn0 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(knh + nbase + 8 * grp));
                const bf16x8 kn1 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(knh + nbase + 32 + 8 * grp));
#pragma unroll
                for (int i = 0; i < kVC; ++i) {
                    // compare the clamped row: rows past S were read from row nk-1
                    int r = (lane + 64 * i) / 8;
                    r = r < nk ? r : nk - 1;
                    const bool hit = r == rnew;
                    vr[i].x = hit ? vn.x : vr[i].x;
                    vr[i].y = hit ? vn.y : vr[i].y;
                    vr[i].z = hit ? vn.z : vr[i].z;
                    vr[i].w = hit ? vn.w : vr[i].w;
                }
#pragma unroll
                for (int nn = 0; nn < kSub; ++nn) {
                    int r = 16 * nn + col16;
                    r = r < nk ? r : nk - 1;
                    const bool hit = r == rnew;
                    ka[nn][0] = hit ? kn0 : ka[nn][0];
                    ka[nn][1] = hit ? kn1 : ka[nn][1];
                }
            }
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int i = 0; i < kVC; ++i) {
                const int c = lane + 64 * i;
                *reinterpret_cast<uint4*>(vt + (c / 8) * kDVRow + (c % 8) * 8) = vr[i];
            }
            __builtin_amdgcn_wave_barrier();
            f32x4 sc[kSub];
#pragma unroll
            for (int nn = 0; nn < kSub; ++nn) {
                sc[nn] = f32x4{0.f, 0.f, 0.f, 0.f};
                sc[nn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[nn][0], qb0, sc[nn], 0, 0, 0);
                sc[nn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[nn][1], qb1, sc[nn], 0, 0, 0);
            }
            bf16x8 va[4][kHalf];
            {
                const int rsub = 4 * grp + col16 / 4;
                const int csub = 4 * (col16 % 4);
#pragma unroll
                for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                    for (int mm = 0; mm < kHalf; ++mm) {
                        const uint16_t* vb = vt + (32 * mm + rsub) * kDVRow + 16 * dt + csub;
                        const i16x4 lo = lds_read_tr(vb);
                        const i16x4 hi = lds_read_tr(vb + 16 * kDVRow);
                        va[dt][mm] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                    }
            }
            if (nk < kBs) {
#pragma unroll
                for (int nn = 0; nn < kSub; ++nn)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (16 * nn + 4 * grp + i >= nk) sc[nn][i] = -__builtin_inff();
            }
            float mx = max_sub_nn(sc);
            mx = pair32_max(pair16_max(mx));
            const float cand = mx * scale_log2;
            const float m_new = cand > m_run + kLazy ? cand : m_run;
            const float alpha = m_new != m_run ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
            m_run = m_new;
            uint4 pw[kHalf];
#pragma unroll
            for (int mm = 0; mm < kHalf; ++mm) {
                bf16x8 pb;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    pb[i] = static_cast<__bf16>(__builtin_amdgcn_exp2f(__builtin_fmaf(sc[2 * mm][i], scale_log2, -m_new)));
                    pb[4 + i] = static_cast<__bf16>(__builtin_amdgcn_exp2f(__builtin_fmaf(sc[2 * mm + 1][i], scale_log2, -m_new)));
                }
                pw[mm] = __builtin_bit_cast(uint4, pb);
            }
            if (__ballot(alpha != 1.0f) != 0ull) {
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
                ol *= alpha;
            }
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int mm = 0; mm < kHalf; ++mm)
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt][mm], __builtin_bit_cast(bf16x8, pw[mm]), o[dt],
                                                                    0, 0, 0);
#pragma unroll
            for (int mm = 0; mm < kHalf; ++mm)
                ol = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones_a, __builtin_bit_cast(bf16x8, pw[mm]), ol, 0, 0, 0);
            __builtin_amdgcn_wave_barrier();  // the next block overwrites vt
        }
        // the wave's partial of head col16: m (log2 units), l (lane group 0, element 0), o[16dt+4grp+i]
        const float lsum = __shfl(ol[0], col16, kWave);
        if (col16 < R) {
            float* pp = part + col16 * (DH + 2);
            if (grp == 0) {
                pp[0] = m_run;
                pp[1] = lsum;
            }
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i) pp[2 + 16 * dt + 4 * grp + i] = o[dt][i];
        }
    } else {
    // this wave's running partial (m, l, o[DH]) per head, merged block by block
    for (int hh = 0; hh < R; ++hh) {
        if (lane == 0) {
            part[hh * (DH + 2)] = -__builtin_inff();
            part[hh * (DH + 2) + 1] = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
            const int d = lane + i * kWave;
            if (d < DH) part[hh * (DH + 2) + 2 + d] = 0.0f;
        }
    }
    __builtin_amdgcn_wave_barrier();

    for (int w = s_lo + wave; w < s_hi; w += nwaves) {
        const int64_t j = sel_mode == 1 ? w : sel_lds[w];
        if (j < 0 || j > cb) continue;  // not a block of [0, S): nothing to attend
        const int64_t s0 = j * bs;
        const int64_t s1 = s0 + bs < S ? s0 + bs : S;
        // storage row of position s0: the cache row, or slot w of a compact buffer
        const int64_t row0 = compact ? static_cast<int64_t>(w) * bs : s0;
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
                const int64_t base = b * kv_sb + (row0 + (c0 - s0)) * kv_ss + g * kv_sh;
                const int64_t nbase = b * new_sb + g * new_sh;
#pragma unroll
                for (int i = 0; i < NC; ++i) {
                    const int c = lane + i * kWave;
                    const int row = c / RC, col = (c % RC) * EPV;
                    if (row < nk) {
                        if (k_new != nullptr && c0 + row == S - 1) {
                            // the new token, supplied apart from the (prefetched) blocks
                            kraw[i] = *reinterpret_cast<const uint4*>(static_cast<const E*>(k_new) + nbase + col);
                            vraw[i] = *reinterpret_cast<const uint4*>(static_cast<const E*>(v_new) + nbase + col);
                        } else {
                            kraw[i] = *reinterpret_cast<const uint4*>(static_cast<const E*>(kc) + base + row * kv_ss + col);
                            vraw[i] = *reinterpret_cast<const uint4*>(static_cast<const E*>(vc) + base + row * kv_ss + col);
                        }
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
                    const float alpha = __builtin_amdgcn_exp2f(mrun[hh] - m_new);
                    const float p = lane < nk ? __builtin_amdgcn_exp2f(sc - m_new) : 0.0f;
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
            // merge this block's (m, l, o) into the wave's partial
            for (int hh = 0; hh < nh; ++hh) {
                float* pp = part + (hb + hh) * (DH + 2);
                const float pm = pp[0];
                const float M = fmaxf(pm, mrun[hh]);
                const float a_old = __builtin_amdgcn_exp2f(pm - M);
                const float a_new = __builtin_amdgcn_exp2f(mrun[hh] - M);
#pragma unroll
                for (int i = 0; i < DPL; ++i) {
                    const int d = lane + i * kWave;
                    if (d < DH) pp[2 + d] = pp[2 + d] * a_old + orun[hh][i] * a_new;
                }
                __builtin_amdgcn_wave_barrier();
                if (lane == 0) {
                    pp[0] = M;
                    pp[1] = pp[1] * a_old + lrun[hh] * a_new;
                }
                __builtin_amdgcn_wave_barrier();
            }
        }
    }
    }  // !MF
    __syncthreads();

    // merge the wave partials in wave order (waves without a block hold m = -inf, l = 0)
    const int nw = s_hi - s_lo < nwaves ? s_hi - s_lo : nwaves;
    for (int e = threadIdx.x; e < R * DH; e += blockDim.x) {
        const int hh = e / DH, d = e % DH;
        float M = -__builtin_inff();
        for (int w = 0; w < nw; ++w) M = fmaxf(M, part_all[(w * R + hh) * (DH + 2)]);
        float num = 0.0f, den = 0.0f;
        for (int w = 0; w < nw; ++w) {
            const float* ps = part_all + (w * R + hh) * (DH + 2);
            const float wt = __builtin_amdgcn_exp2f(ps[0] - M);
            den = den + wt * ps[1];
            num = num + wt * ps[2 + d];
        }
        if (nsplit == 1) {
            store_elem<DT>(out, b * out_sb + static_cast<int64_t>(g * R + hh) * DH + d, num / den);
        } else {
            // the split's partial (m, l, o[DH]) of head hh, unnormalised (an
            // empty split: m = -inf, l = 0, o = 0), merged by decode_merge_kernel
            float* pw = ws_part + ((bg * nsplit + split) * R + hh) * (DH + 2);
            if (d == 0) {
                pw[0] = M;
                pw[1] = den;
            }
            pw[2 + d] = num;
        }
    }
    __syncthreads();
}

// The splits of a dense decode (decode_attend_kernel with nsplit > 1): one
// workgroup per (sequence, KV head) folds the nsplit partials of each of its
// R heads. Thread (q, e) of Q groups takes the splits q, q + Q, q + 2Q, ...
// of element e = (head, dim) in split order (32 loads in flight), keeping a
// running (m, l, o) that is rescaled when a split's maximum exceeds it; the
// groups are then combined in group order. A split's group depends on its
// index alone and an empty split (m = -inf, l = 0, o = 0) adds exact zeros,
// so the splits past the last block (a launch sized for a longer cache)
// change nothing.
constexpr int kMergeThreads = 768;

template <int DT, int DH>
__global__ void __launch_bounds__(kMergeThreads)
decode_merge_kernel(const float* __restrict__ ws_part, int nsplit, int R, int H, int Q, void* __restrict__ out,
                    int64_t out_sb) {
    __shared__ float m_q[kMergeThreads], l_q[kMergeThreads], o_q[kMergeThreads];
    constexpr int U = 32;
    const int g = blockIdx.x;
    const int b = blockIdx.y;
    const int64_t bg = static_cast<int64_t>(b) * H + g;
    const int RD = R * DH;
    const int per = static_cast<int>(blockDim.x) / Q;  // elements per round
    const int t = static_cast<int>(threadIdx.x);
    const int q = t / per;
    const int step = R * (DH + 2);
    for (int e0 = 0; e0 < RD; e0 += per) {  // the same trip count in every thread
        const int e = e0 + t % per;
        const bool live = q < Q && e < RD;
        const int hh = live ? e / DH : 0, d = live ? e % DH : 0;
        const float* p0 = ws_part + (bg * nsplit * R + hh) * (DH + 2);
        // this group's splits q + Q j; indices past the last re-read split q
        // (in bounds) and are not added
        const int nj = live && q < nsplit ? (nsplit - q + Q - 1) / Q : 0;
        float M = -__builtin_inff(), num = 0.0f, den = 0.0f;
        for (int j0 = 0; j0 < nj; j0 += U) {
            float mv[U], lv[U], ov[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int off = (q + Q * (j0 + u < nj ? j0 + u : 0)) * step;
                mv[u] = p0[off];
                lv[u] = p0[off + 1];
                ov[u] = p0[off + 2 + d];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (j0 + u < nj && mv[u] != -__builtin_inff()) {
                    if (mv[u] > M) {
                        const float sc = __builtin_amdgcn_exp2f(M - mv[u]);
                        num = num * sc;
                        den = den * sc;
                        M = mv[u];
                    }
                    const float wt = __builtin_amdgcn_exp2f(mv[u] - M);
                    den = den + wt * lv[u];
                    num = num + wt * ov[u];
                }
            }
        }
        m_q[t] = M;
        l_q[t] = den;
        o_q[t] = num;
        __syncthreads();
        if (live && q == 0) {
            float Mall = -__builtin_inff();
            for (int r = 0; r < Q; ++r) Mall = fmaxf(Mall, m_q[r * per + t]);
            float n_all = 0.0f, d_all = 0.0f;
            for (int r = 0; r < Q; ++r) {
                const float mr = m_q[r * per + t];
                if (mr == -__builtin_inff()) continue;  // a group without a block
                const float wt = __builtin_amdgcn_exp2f(mr - Mall);
                n_all = n_all + wt * o_q[r * per + t];
                d_all = d_all + wt * l_q[r * per + t];
            }
            store_elem<DT>(out, b * out_sb + static_cast<int64_t>(g * R + hh) * DH + d, n_all / d_all);
        }
        __syncthreads();  // m_q, l_q, o_q are rewritten by the next round
    }
}

// ---------------------------------------------------------------------------
struct AttendArgs {
    const void* q; int64_t q_sb, q_sh;
    const void* kc; const void* vc; int64_t kv_sb, kv_ss, kv_sh;
    int dtype; int64_t B, S, Hq, Hkv, D, bs, k;
    int sel_mode; int cap; float scale;
    const float* scores;
    const int32_t* sel_in; const int32_t* n_sel_in; int compact;
    const void* k_new; const void* v_new; int64_t new_sb, new_sh;
    int32_t* sel_out; int32_t* n_sel_out;
    void* out; int64_t out_sb;
    const int64_t* pos_dev = nullptr;  // S = *pos_dev + 1, S the bound (window / list modes)
    // sel_mode 4: selection from block sums [B, nb_stride, Hkv, D] and a forecast [B, Hkv, D];
    // update_sums: recompute the current block's sums first
    float* sums = nullptr; int64_t nb_stride = 0; int update_sums = 0;
    const void* fsel = nullptr; int fsel_bf16 = 0; int64_t fs_sb = 0, fs_sh = 0;
    int absolute = 0; float fscale = 0.0f;
    const PrefetchDev* pf = nullptr;  // the next layer's prefetch carried by the launch (matrix-core path)
    // dense mode on the matrix cores: a workspace for split partials (nullptr: one workgroup per (b, g))
    float* ws_part = nullptr; size_t ws_bytes = 0;
};

// Splits of a dense decode: kSplitBlocks blocks per workgroup (more when the
// workspace holds fewer splits, or past kMaxSplits), so that the split of a
// block, and with it the result, depends on the length alone, not on the
// capacity a launch is sized for; no split below two.
constexpr int64_t kSplitBlocks = 4;
constexpr int64_t kMaxSplits = 4096;

struct DenseSplit {
    int n = 1;       // splits per (sequence, KV head)
    int blocks = 0;  // blocks per split
};

static int64_t dense_split_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t D) {
    return B * Hkv * (Hq / Hkv) * (D + 2) * static_cast<int64_t>(sizeof(float));
}

static DenseSplit dense_split(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t NB, size_t ws_bytes) {
    int64_t fit = static_cast<int64_t>(ws_bytes) / dense_split_bytes(B, Hq, Hkv, D);
    fit = fit < kMaxSplits ? fit : kMaxSplits;
    if (fit < 2) return DenseSplit{};
    int64_t per = kSplitBlocks;
    if (cdiv(NB, per) > fit) per = cdiv(NB, fit);
    const int64_t n = cdiv(NB, per);
    if (n < 2) return DenseSplit{};
    return DenseSplit{static_cast<int>(n), static_cast<int>(per)};
}

size_t decode_dense_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t S, int64_t bs) {
    if (B <= 0 || Hkv <= 0 || Hq % Hkv != 0 || S <= 0 || bs <= 0) return 0;
    const DenseSplit sp = dense_split(B, Hq, Hkv, D, cdiv(S, bs), static_cast<size_t>(-1) / 2);
    return sp.n >= 2 ? static_cast<size_t>(sp.n * dense_split_bytes(B, Hq, Hkv, D)) : 0;
}

bool decode_at_matrix_core(int dtype, int64_t D, int64_t bs, int64_t q_sb, int64_t q_sh, const void* q) {
    return dtype == SPARDA_BF16 && D == 64 && (bs == 64 || bs == 32) && (q_sb % 8) == 0 && (q_sh % 8) == 0 &&
           (reinterpret_cast<uintptr_t>(q) & 15u) == 0;
}

static int launch_attend(const AttendArgs& a, hipStream_t stream) {
    const int64_t NB = cdiv(a.S, a.bs);
    const float scale_log2 = a.scale * kLog2e;
    const int Hq_i = static_cast<int>(a.Hq), Hkv_i = static_cast<int>(a.Hkv);
    const int64_t R = a.Hq / a.Hkv;
    // matrix-core block attention: bf16, D = 64, bs = 64, 16-byte aligned q rows
    const bool mf = decode_at_matrix_core(a.dtype, a.D, a.bs, a.q_sb, a.q_sh, a.q);
    // dense on the matrix cores with a workspace: the blocks split over nsplit
    // workgroups per (sequence, KV head), then decode_merge_kernel
    const DenseSplit split = (mf && a.sel_mode == 1 && a.ws_part != nullptr)
                                 ? dense_split(a.B, a.Hq, a.Hkv, a.D, NB, a.ws_bytes)
                                 : DenseSplit{};
    const int nsplit = split.n;
    // most blocks one workgroup can attend: the selection capacity, or its share of every block when dense
    const int64_t max_blocks = a.sel_mode == 1 ? (nsplit > 1 ? split.blocks : NB) : a.cap;
    if (a.pf != nullptr && !mf)
        return set_error(SPARDA_ERR_MODE, "decode: a carried prefetch needs the bf16 D=64 matrix-core attention");
    const PrefetchDev pf = a.pf != nullptr ? *a.pf : PrefetchDev{};
    constexpr size_t kLdsBudget = 150 * 1024;
    const int pow2 = (a.bs & (a.bs - 1)) == 0 ? 1 : 0;
    dim3 grid2(static_cast<unsigned>(a.Hkv), static_cast<unsigned>(a.B),
               static_cast<unsigned>(nsplit) + (a.pf != nullptr ? 1u : 0u));
#define SPARDA_ATT(DT_, DH_, CH_)                                                                        \
    do {                                                                                                 \
        if constexpr (DT_ == SPARDA_BF16 && DH_ == 64) {                                                 \
            if (mf) {                                                                                    \
                if (a.bs == 32) SPARDA_ATT_K(DT_, DH_, CH_, true, 32);                                   \
                else SPARDA_ATT_K(DT_, DH_, CH_, true, 64);                                              \
                break;                                                                                   \
            }                                                                                            \
        }                                                                                                \
        SPARDA_ATT_K(DT_, DH_, CH_, false, 64);                                                          \
    } while (0)
#define SPARDA_ATT_K(DT_, DH_, CH_, MF_, MBS_)                                                           \
    do {                                                                                                 \
        const size_t wb = attend_wave_bytes<DT_, DH_>();                                                 \
        const size_t pb = static_cast<size_t>(R) * (DH_ + 2) * 4;                                        \
        int waves = max_blocks < kAttendMaxWaves ? static_cast<int>(max_blocks) : kAttendMaxWaves;       \
        while (waves > 1 && ((waves * pb + 15) & ~static_cast<size_t>(15)) + waves * wb > kLdsBudget) --waves; \
        size_t lds = ((waves * pb + 15) & ~static_cast<size_t>(15)) + waves * wb;                        \
        if ((a.sel_mode == 4 || a.pf != nullptr) && lds < static_cast<size_t>(NB) * 4)                  \
            lds = static_cast<size_t>(NB) * 4;                                                           \
        hipLaunchKernelGGL((decode_attend_kernel<DT_, DH_, CH_, MF_, MBS_>), grid2, dim3(waves * kWave), lds, stream, \
                           a.q, a.q_sb, a.q_sh, a.kc, a.vc, a.kv_sb, a.kv_ss, a.kv_sh, a.S, Hq_i, Hkv_i,  \
                           static_cast<int>(a.bs), NB, static_cast<int>(a.k), a.sel_mode, a.cap,         \
                           scale_log2, a.scores, a.sel_in, a.n_sel_in, a.compact, a.k_new, a.v_new,     \
                           a.new_sb, a.new_sh, a.sel_out, a.n_sel_out, a.out, a.out_sb, a.pos_dev, a.sums, \
                           a.nb_stride, a.update_sums, a.fsel, a.fsel_bf16, a.fs_sb, a.fs_sh, a.absolute,       \
                           a.fscale, pow2, pf, nsplit, split.blocks, a.ws_part);                               \
        if (nsplit > 1) {                                                                                \
            const int rd = static_cast<int>(R) * DH_;                                                    \
            const int qg = rd >= kMergeThreads ? 1 : (kMergeThreads / rd < 4 ? kMergeThreads / rd : 4);  \
            const int thr = rd >= kMergeThreads ? kMergeThreads : rd * qg;                               \
            hipLaunchKernelGGL((decode_merge_kernel<DT_, DH_>), dim3(static_cast<unsigned>(a.Hkv),       \
                               static_cast<unsigned>(a.B)), dim3(thr), 0, stream, a.ws_part, nsplit,     \
                               static_cast<int>(R), Hkv_i, qg, a.out, a.out_sb);                         \
        }                                                                                                \
    } while (0)
#define SPARDA_ATT_C(DT_, DH_)                            \
    if (NB <= 256) SPARDA_ATT(DT_, DH_, 4);               \
    else if (NB <= 512) SPARDA_ATT(DT_, DH_, 8);          \
    else if (NB <= 1024) SPARDA_ATT(DT_, DH_, 16);        \
    else SPARDA_ATT(DT_, DH_, 64);
#define SPARDA_ATT_D(DT_)                                         \
    switch (a.D) {                                                \
        case 16: { SPARDA_ATT_C(DT_, 16) } break;                 \
        case 32: { SPARDA_ATT_C(DT_, 32) } break;                 \
        case 64: { SPARDA_ATT_C(DT_, 64) } break;                 \
        default: { SPARDA_ATT_C(DT_, 128) } break;                \
    }
    if (a.dtype == SPARDA_BF16) {
        SPARDA_ATT_D(SPARDA_BF16);
    } else {
        SPARDA_ATT_D(SPARDA_F32);
    }
#undef SPARDA_ATT_D
#undef SPARDA_ATT_C
#undef SPARDA_ATT_K
#undef SPARDA_ATT
    return check_hip(hipGetLastError(), "decode_attend_kernel");
}

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
    AttendArgs a{q, q_sb, q_sh, kc, vc, kv_sb, kv_ss, kv_sh, dtype, B, S, Hq, Hkv, D, bs, k,
                 sel_mode, cap, scale, ws.scores, nullptr, nullptr, 0, nullptr, nullptr, 0, 0,
                 sel_out, n_sel_out, out, out_sb};
    return launch_attend(a, stream);
}

int launch_decode_selected(const void* q, int64_t q_sb, int64_t q_sh, const void* k, const void* v,
                           int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int dtype, int compact,
                           const int32_t* sel, const int32_t* n_sel, int64_t cap, const void* k_new,
                           const void* v_new, int64_t new_sb, int64_t new_sh, int64_t B, int64_t S,
                           int64_t Hq, int64_t Hkv, int64_t D, int64_t bs, float scale, void* out,
                           int64_t out_sb, hipStream_t stream, void* ws, size_t ws_bytes) {
    AttendArgs a{q, q_sb, q_sh, k, v, kv_sb, kv_ss, kv_sh, dtype, B, S, Hq, Hkv, D, bs, cap > 2 ? cap - 2 : 0,
                 sel == nullptr ? 1 : 3, static_cast<int>(sel == nullptr ? 0 : cap), scale, nullptr,
                 sel, n_sel, compact, k_new, v_new, new_sb, new_sh, nullptr, nullptr, out, out_sb};
    a.ws_part = static_cast<float*>(ws);
    a.ws_bytes = ws_bytes;
    return launch_attend(a, stream);
}

int launch_decode_sums(const void* q, int64_t q_sb, int64_t q_sh, const void* k, const void* v, int64_t kv_sb,
                       int64_t kv_ss, int64_t kv_sh, int dtype, const void* f, int f_dtype, int64_t f_sb,
                       int64_t f_sh, float* sums, int64_t nb_stride, int update_sums, int64_t B, int64_t S,
                       const int64_t* pos_dev, int64_t Hq, int64_t Hkv, int64_t D, int64_t bs, int64_t top_k,
                       int routing, float scale, float fscale, int32_t* sel_out, int32_t* n_sel_out, void* out,
                       int64_t out_sb, hipStream_t stream) {
    AttendArgs a{q, q_sb, q_sh, k, v, kv_sb, kv_ss, kv_sh, dtype, B, S, Hq, Hkv, D, bs, top_k, 4,
                 static_cast<int>(top_k + 2), scale, nullptr, nullptr, nullptr, 0, nullptr, nullptr, 0, 0,
                 sel_out, n_sel_out, out, out_sb, pos_dev};
    a.sums = sums;
    a.nb_stride = nb_stride;
    a.update_sums = update_sums;
    a.fsel = f;
    a.fsel_bf16 = f_dtype == SPARDA_BF16 ? 1 : 0;
    a.fs_sb = f_sb;
    a.fs_sh = f_sh;
    a.absolute = routing == SPARDA_ROUTE_ABSOLUTE ? 1 : 0;
    a.fscale = fscale;
    return launch_attend(a, stream);
}

int launch_decode_at(const void* q, int64_t q_sb, int64_t q_sh, const void* k, const void* v, int64_t kv_sb,
                     int64_t kv_ss, int64_t kv_sh, int dtype, int compact, const int32_t* sel,
                     const int32_t* n_sel, int64_t cap, int64_t window_k, const void* k_new, const void* v_new,
                     int64_t new_sb, int64_t new_sh, int64_t B, int64_t S_max, const int64_t* pos_dev,
                     int64_t Hq, int64_t Hkv, int64_t D, int64_t bs, float scale, void* out, int64_t out_sb,
                     hipStream_t stream, const PrefetchDev* pf, void* ws, size_t ws_bytes) {
    int mode, cap_i;
    int64_t kk;
    if (sel != nullptr) {
        mode = 3, cap_i = static_cast<int>(cap), kk = cap > 2 ? cap - 2 : 0;
    } else if (window_k > 0) {
        mode = 2, cap_i = static_cast<int>(window_k + 2), kk = window_k;
    } else {
        mode = 1, cap_i = 0, kk = 0;
    }
    AttendArgs a{q, q_sb, q_sh, k, v, kv_sb, kv_ss, kv_sh, dtype, B, S_max, Hq, Hkv, D, bs, kk, mode, cap_i, scale,
                 nullptr, sel, n_sel, compact, k_new, v_new, new_sb, new_sh, nullptr, nullptr, out, out_sb,
                 pos_dev};
    a.pf = pf;
    a.ws_part = static_cast<float*>(ws);
    a.ws_bytes = ws_bytes;
    return launch_attend(a, stream);
}

}  // namespace sparda
