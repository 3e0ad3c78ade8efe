// bf16 dense GQA prefill on the gfx950 matrix cores (D = 64), causal or not:
// the reference's dense fallback (model/attention/sparse.py:201-224: layer 0,
// no forecast, or at most two KV blocks) without selection lists.
//
// One workgroup of 8 wavefronts serves one (sequence b, KV head g, window of
// 128 query tokens); wavefront w owns tokens [16w, 16w+16) of the window for
// all R = Hq/Hkv query heads of the group: 16R columns (column c -> token
// 16w + c / R, head c % R), R tiles of 16 columns whose Q operands stay in
// registers. The workgroup walks the KV blocks of 64 keys in ascending order
// up to its last token's block; each block's K and V are staged once in LDS
// (double-buffered; the next block is loaded into registers while the
// current one is computed) and shared by all 128 tokens and R heads. Per tile
// and block, with v_mfma_f32_16x16x32_bf16:
//     S^T[key, col] = K[key, :] . Q[col, :]           (8 MFMA)
//     P = exp2(S * scale log2 e - ref[col]), bf16      (fp32 exponent)
//     O^T[d, col]  += V^T[d, key] . P^T[key, col]      (8 MFMA)
//     l[col]       += 1^T P^T                           (2 MFMA, a ones A operand)
// ref[col] is the column's maximum over block 0 (which every column attends,
// key 0 being allowed to every token), taken when block 0 is computed; later
// blocks take no maxima and never rescale. A score more than 64 log2-units
// above the reference shows as a row sum past 2^64 at the end; the window is
// then walked once for the exact column maxima and again against them (every
// P <= 1).
// A wavefront whose tokens all lie before a block skips it (the causal
// triangle is not computed); the diagonal block masks the keys past each
// column's token. No per-token membership logic: every key up to the token
// (or every key) is attended.
//
// The chunked-gather prefill (model/attention/sparse.py:284-364) runs the same
// kernel with LISTED: one workgroup of 4 wavefronts per query block of 64
// tokens, which builds the block's list in LDS first (chunk.h: {0, own} U the
// union of its rows' non-causal top-k, cut to min(NB, k+2)) and walks the
// listed blocks instead of every block up to the diagonal; all 64 tokens share
// the list, so every tile is full. The first listed block sets the references
// (its key 0 is allowed to every token, since listed blocks never lie past
// the own one).
#include "chunk.h"
#include "common.h"
#include "kernels.h"
#include "mfma.h"

namespace sparda {

namespace {

constexpr int kDBs = 64;                 // keys per KV block
constexpr int kDD = 64;                  // head dim
constexpr int kDWaves = 8;               // wavefronts per workgroup (dense)
constexpr int kLWaves = 4;               // wavefronts per workgroup (listed: one 64-token query block)
constexpr int kDKRow = kDD + 8;          // K row in LDS, bf16 elements (144 B)
constexpr int kDVRow = kDD + 16;         // V row in LDS, bf16 elements (160 B)
constexpr float kDLog2e = 1.4426950408889634f;
constexpr float kDGuard = 18446744073709551616.0f;  // 2^64: a row sum past it means a score far above ref

struct DenseSmem {
    uint16_t k[2][kDBs * kDKRow];
    uint16_t v[2][kDBs * kDVRow];
    int flag;                             // some column's row sum passed kDGuard
};

// the chunked lists' inputs and outputs (LISTED only)
struct ChunkArgs {
    const int32_t* topk;  // [B, Hkv, T, ke] non-causal top-k, or nullptr: the static window
    int ke, k, cut;       // top-k width, top_k, list length cap min(NB, k + 2)
    int32_t* sel;         // optional [B, Hkv, T, cap] / [B, Hkv, T]: the lists as sparda_select_chunked writes them
    int32_t* n_sel;
    int cap;
};

}  // namespace

template <int R, bool LISTED>
__global__ void __launch_bounds__((LISTED ? kLWaves : kDWaves) * kWave, 2)
prefill_dense_kernel(const uint16_t* __restrict__ q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                     const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int64_t kv_sb, int64_t kv_st,
                     int64_t kv_sh, int64_t T, int H, int64_t NBq, int causal, float scale_log2,
                     uint16_t* __restrict__ out, int64_t out_sb, int64_t out_st, ChunkArgs ch) {
    constexpr int kNW = LISTED ? kLWaves : kDWaves;
    constexpr int kThreads = kNW * kWave;
    constexpr int kWin = 16 * kNW;               // query tokens per workgroup
    constexpr int kSR = kDBs * 8 / kThreads;     // 16-byte K (and V) chunks each thread stages per block
    __shared__ DenseSmem sm;
    __shared__ ChunkLds cl;
    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int wave = tid / kWave;
    const int col16 = lane % 16;
    const int grp = lane / 16;

    // heaviest windows first, XCD-aware when there are few (b, g) pairs
    const int64_t BH = static_cast<int64_t>(gridDim.x) / NBq;
    int64_t bg, qw;
    window_order(blockIdx.x, BH, NBq, bg, qw);
    const int b = static_cast<int>(bg / H);
    const int g = static_cast<int>(bg % H);
    const int64_t t0 = qw * kWin;
    const int64_t NB = cdiv(T, kDBs);
    const int t_valid = static_cast<int>(T - t0 < kWin ? T - t0 : kWin);
    const int64_t w_first = t0 + 16 * wave;  // this wavefront's first token
    int64_t w_last = w_first + 15;
    w_last = w_last < T - 1 ? w_last : T - 1;
    const bool w_live = w_first < T;
    // Q operands of this wavefront's tiles (column col16 of tile tt; rows past T read row T-1)
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

    f32x4 o[R][4], ol[R];
    float ref[R];  // the columns' references, log2 units
    bf16x8 ones_a;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones_a[e] = static_cast<__bf16>(col16 == 0 ? 1.0f : 0.0f);
    auto clear = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int tt = 0; tt < R; ++tt) {
            ol[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) o[tt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };
    clear();
#pragma unroll
    for (int tt = 0; tt < R; ++tt) ref[tt] = -__builtin_inff();
    if (tid == 0) sm.flag = 0;  // ordered before its uses by the staging barrier

    // staging: thread -> 16-byte chunks (rows tid / 8 + i * kThreads / 8, column
    // tid % 8) of K and of V; rows past T (a ragged last block) read row T-1
    // (finite values, masked)
    const uint16_t* kbase = k + b * kv_sb + static_cast<int64_t>(g) * kv_sh;
    const uint16_t* vbase = v + b * kv_sb + static_cast<int64_t>(g) * kv_sh;
    const int srow = tid / 8, scol = (tid % 8) * 8;
    constexpr int kRowStep = kThreads / 8;
    // the chunks in flight live in one vector register tuple (an array of
    // uint4 handed between the lambdas would be placed in scratch memory)
    typedef unsigned int StageV __attribute__((ext_vector_type(4 * kSR)));
    auto fetch = [&](int j, StageV& kv_k, StageV& kv_v) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kSR; ++i) {
            int64_t s = static_cast<int64_t>(j) * kDBs + srow + i * kRowStep;
            s = s < T ? s : T - 1;
            const uint4 a = *reinterpret_cast<const uint4*>(kbase + s * kv_st + scol);
            const uint4 c = *reinterpret_cast<const uint4*>(vbase + s * kv_st + scol);
            kv_k[4 * i] = a.x; kv_k[4 * i + 1] = a.y; kv_k[4 * i + 2] = a.z; kv_k[4 * i + 3] = a.w;
            kv_v[4 * i] = c.x; kv_v[4 * i + 1] = c.y; kv_v[4 * i + 2] = c.z; kv_v[4 * i + 3] = c.w;
        }
    };
    auto stash = [&](int buf, const StageV& kv_k, const StageV& kv_v) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kSR; ++i) {
            *reinterpret_cast<uint4*>(&sm.k[buf][(srow + i * kRowStep) * kDKRow + scol]) =
                uint4{kv_k[4 * i], kv_k[4 * i + 1], kv_k[4 * i + 2], kv_k[4 * i + 3]};
            *reinterpret_cast<uint4*>(&sm.v[buf][(srow + i * kRowStep) * kDVRow + scol]) =
                uint4{kv_v[4 * i], kv_v[4 * i + 1], kv_v[4 * i + 2], kv_v[4 * i + 3]};
        }
    };

    // blocks of the workgroup and of this wavefront: dense causal, every block up
    // to the last token's; dense non-causal, every block; listed, the list, built
    // while the Q rows and block 0 (the first entry of every list) are in flight
    int nblk, w_nblk;
    StageV nk0{}, nv0{};
    if constexpr (LISTED) {
        fetch(0, nk0, nv0);
        const int64_t row0 = bg * T + t0;  // (b * Hkv + g) * T + t0
        chunk_list(cl, ch.topk != nullptr ? ch.topk + row0 * ch.ke : nullptr, t_valid, ch.ke, static_cast<int>(qw),
                   ch.k, NB, ch.cut);
        if (ch.sel != nullptr) chunk_write(cl, row0, t_valid, ch.cap, ch.sel, ch.n_sel);
        nblk = cl.m;
        w_nblk = w_live ? nblk : 0;
    } else {
        const int64_t last_tok = t0 + t_valid - 1;
        nblk = static_cast<int>(causal ? last_tok / kDBs + 1 : NB);
        w_nblk = !w_live ? 0 : static_cast<int>(causal ? w_last / kDBs + 1 : NB);
    }
    // the u-th block walked
    auto blk = [&](int u) __attribute__((always_inline)) -> int {
        if constexpr (LISTED) return cl.lst[u];
        else return u;
    };

    // mode 0: P against the references (the first block walked sets them
    // unless `keep`); mode 1: scores only, the exact column maxima into ref
    auto compute = [&](int buf, int j, bool first, int mode, bool keep) __attribute__((always_inline)) {
        // K A operands: key 16n + col16, dims 32kk + 8grp .. +7
        bf16x8 ka[4][2];
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
                ka[n][kk] = lds_read8(&sm.k[buf][(16 * n + col16) * kDKRow + 32 * kk + 8 * grp]);
        // V^T A operands, read transposed from the row-major tile
        bf16x8 va[4][2];
        if (mode == 0) {
            const int rsub = 4 * grp + col16 / 4;
            const int csub = 4 * (col16 % 4);
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    const uint16_t* base = &sm.v[buf][(32 * m + rsub) * kDVRow + 16 * dt + csub];
                    const i16x4 lo = lds_read_tr(base);
                    const i16x4 hi = lds_read_tr(base + 16 * kDVRow);
                    va[dt][m] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                }
        }
        // keys past a column's token (causal diagonal) or past T (ragged tail) are masked
        const int64_t key0 = static_cast<int64_t>(j) * kDBs;
        const bool edge = causal ? key0 + kDBs - 1 > w_first : key0 + kDBs > T;
#pragma unroll
        for (int tt = 0; tt < R; ++tt) {
            f32x4 s[4];
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                s[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[n][0], qreg[tt][0], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                s[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[n][1], qreg[tt][1], s[n], 0, 0, 0);
            }
            if (edge) {
                const int64_t lim64 = causal ? t0 + tok[tt] - key0 : T - 1 - key0;  // keys <= lim are allowed
                const int lim = static_cast<int>(lim64 < kDBs ? lim64 : kDBs);
#pragma unroll
                for (int n = 0; n < 4; ++n)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (16 * n + 4 * grp + i > lim) s[n][i] = -__builtin_inff();
            }
            if (mode == 1 || (first && !keep)) {  // wave-uniform
                const float cand = pair32_max(pair16_max(max16_nn(s))) * scale_log2;  // block's column max, log2 units
                ref[tt] = mode == 1 ? fmaxf(ref[tt], cand) : cand;
                if (mode == 1) continue;
            }
            // a column with no allowed key (ref -inf) gets P = 0 throughout
            const float neg = ref[tt] == -__builtin_inff() ? -__builtin_inff() : -ref[tt];
            uint4 pw[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                bf16x8 pb;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    pb[i] = static_cast<__bf16>(__builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * m][i], scale_log2, neg)));
                    pb[4 + i] =
                        static_cast<__bf16>(__builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * m + 1][i], scale_log2, neg)));
                }
                pw[m] = __builtin_bit_cast(uint4, pb);
            }
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                o[tt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt][0], __builtin_bit_cast(bf16x8, pw[0]),
                                                                    o[tt][dt], 0, 0, 0);
                o[tt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt][1], __builtin_bit_cast(bf16x8, pw[1]),
                                                                    o[tt][dt], 0, 0, 0);
            }
            ol[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones_a, __builtin_bit_cast(bf16x8, pw[0]), ol[tt], 0, 0, 0);
            ol[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones_a, __builtin_bit_cast(bf16x8, pw[1]), ol[tt], 0, 0, 0);
        }
    };

    // block u is computed from buffer u & 1 while block u + 1 is in registers;
    // one barrier per block orders its stash before the reads of the next
    // (nk, nv: block blk(0) already loaded when have0)
    auto walk = [&](int mode, bool keep, StageV nk, StageV nv, bool have0) __attribute__((always_inline)) {
        if (!have0) fetch(blk(0), nk, nv);
        stash(0, nk, nv);
        if (nblk > 1) fetch(blk(1), nk, nv);
        __syncthreads();
        for (int u = 0; u < nblk; ++u) {
            const int buf = u & 1;
            // wave-uniform: blocks past this wavefront's tokens are skipped
            if (u < w_nblk) compute(buf, blk(u), u == 0, mode, keep);
            if (u + 1 < nblk) {
                stash(buf ^ 1, nk, nv);
                if (u + 2 < nblk) fetch(blk(u + 2), nk, nv);
            }
            __syncthreads();
        }
    };
    walk(0, false, nk0, nv0, LISTED);
    // a row sum past 2^64 (or not finite): a score more than 64 log2-units above
    // its column's reference somewhere; the row sums sit in lanes 0..15, element 0
    {
        bool bad = false;
#pragma unroll
        for (int tt = 0; tt < R; ++tt) bad = bad || (w_live && lane < 16 && !(ol[tt][0] <= kDGuard));
        if (__ballot(bad) != 0ull && lane == 0) atomicOr(&sm.flag, 1);
    }
    __syncthreads();
    if (sm.flag != 0) {  // workgroup-uniform: every wave walks again
#pragma unroll
        for (int tt = 0; tt < R; ++tt) ref[tt] = -__builtin_inff();
        walk(1, true, nk0, nv0, false);  // the exact column maxima
        clear();
        walk(0, true, nk0, nv0, false);  // against them: every P <= 1
    }

    // ---- epilogue: out[b, t, h*64 + d] = O / l ----
#pragma unroll
    for (int tt = 0; tt < R; ++tt) {
        // the row sum of column col16 sits in lane col16 (lane group 0), element 0
        const float lsum = __shfl(ol[tt][0], col16, kWave);
        if (tok[tt] >= t_valid) continue;
        const int c = 16 * tt + col16;
        const float inv = 1.0f / lsum;
        uint16_t* orow = out + b * out_sb + (t0 + tok[tt]) * out_st + static_cast<int64_t>(g * R + c % R) * kDD;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            bf16x4 w;
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = static_cast<__bf16>(o[tt][dt][i] * inv);
            *reinterpret_cast<bf16x4*>(orow + 16 * dt + 4 * grp) = w;
        }
    }
}

bool prefill_dense_supported(int dtype, int64_t Hq, int64_t Hkv, int64_t D, int64_t q_sb, int64_t q_st,
                             int64_t q_sh, int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int64_t out_sb,
                             int64_t out_st, const void* q, const void* k, const void* v, const void* out) {
    if (dtype != SPARDA_BF16 || D != kDD || Hq % Hkv != 0) return false;
    const int64_t R = Hq / Hkv;
    if (R < 1 || R > 4) return false;
    auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!al16(q) || !al16(k) || !al16(v) || (reinterpret_cast<uintptr_t>(out) & 7u)) return false;
    if ((q_sb % 8) || (q_st % 8) || (q_sh % 8) || (kv_sb % 8) || (kv_st % 8) || (kv_sh % 8)) return false;
    if ((out_sb % 4) || (out_st % 4)) return false;
    return true;
}

int launch_prefill_dense(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k, const void* v,
                         int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int64_t B, int64_t T, int64_t Hq,
                         int64_t Hkv, int causal, float scale, void* out, int64_t out_sb, int64_t out_st,
                         hipStream_t stream) {
    const int64_t NBq = cdiv(T, 16 * kDWaves);
    const int64_t R = Hq / Hkv;
    dim3 grid(static_cast<unsigned>(B * Hkv * NBq));
    const float sl = scale * kDLog2e;
#define SPARDA_DN(R_)                                                                                      \
    hipLaunchKernelGGL((prefill_dense_kernel<R_, false>), grid, dim3(kDWaves * kWave), 0, stream,          \
                       static_cast<const uint16_t*>(q), q_sb, q_st, q_sh, static_cast<const uint16_t*>(k), \
                       static_cast<const uint16_t*>(v), kv_sb, kv_st, kv_sh, T, static_cast<int>(Hkv), NBq, \
                       causal, sl, static_cast<uint16_t*>(out), out_sb, out_st, ChunkArgs{})
    switch (R) {
        case 1: SPARDA_DN(1); break;
        case 2: SPARDA_DN(2); break;
        case 3: SPARDA_DN(3); break;
        default: SPARDA_DN(4); break;
    }
#undef SPARDA_DN
    return check_hip(hipGetLastError(), "prefill_dense_kernel");
}

int launch_prefill_chunked(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k, const void* v,
                           int64_t kv_sb, int64_t kv_st, int64_t kv_sh, const int32_t* topk, int64_t ke,
                           int64_t top_k, int32_t* sel, int32_t* n_sel, int64_t cap, int64_t B, int64_t T,
                           int64_t Hq, int64_t Hkv, float scale, void* out, int64_t out_sb, int64_t out_st,
                           hipStream_t stream) {
    const int64_t NB = cdiv(T, kDBs);
    if (NB > kChunkMaxNB)
        return set_error(SPARDA_ERR_SHAPE, "prefill_chunked: more than %d blocks", kChunkMaxNB);
    const int64_t cut = NB < top_k + 2 ? NB : top_k + 2;
    if (sel != nullptr && (cap < cut || cap > kMaxSelCap))
        return set_error(SPARDA_ERR_SHAPE, "prefill_chunked: sel_cap %lld outside [%lld, %d]", (long long)cap,
                         (long long)cut, kMaxSelCap);
    const int64_t NBq = NB;  // one workgroup per 64-token query block
    const int64_t R = Hq / Hkv;
    dim3 grid(static_cast<unsigned>(B * Hkv * NBq));
    const float sl = scale * kDLog2e;
    const ChunkArgs ch{topk, static_cast<int>(ke), static_cast<int>(top_k), static_cast<int>(cut), sel, n_sel,
                       static_cast<int>(sel != nullptr ? cap : 0)};
#define SPARDA_CH(R_)                                                                                      \
    hipLaunchKernelGGL((prefill_dense_kernel<R_, true>), grid, dim3(kLWaves * kWave), 0, stream,           \
                       static_cast<const uint16_t*>(q), q_sb, q_st, q_sh, static_cast<const uint16_t*>(k), \
                       static_cast<const uint16_t*>(v), kv_sb, kv_st, kv_sh, T, static_cast<int>(Hkv), NBq, \
                       1, sl, static_cast<uint16_t*>(out), out_sb, out_st, ch)
    switch (R) {
        case 1: SPARDA_CH(1); break;
        case 2: SPARDA_CH(2); break;
        case 3: SPARDA_CH(3); break;
        default: SPARDA_CH(4); break;
    }
#undef SPARDA_CH
    return check_hip(hipGetLastError(), "prefill_dense_kernel (chunked)");
}

}  // namespace sparda
