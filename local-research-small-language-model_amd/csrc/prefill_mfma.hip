// bf16 block-sparse GQA prefill on the gfx950 matrix cores (D = 64, bs = 64).
//
// One workgroup (4 wavefronts) serves one (sequence b, KV head g, query block
// qb): 64 query tokens x R = Hq/Hkv query heads. Wavefront w owns tokens
// [16w, 16w+16) of the block for all R heads, i.e. 16R "columns"
// (column c -> token c / R, head c % R), processed as R tiles of 16 columns.
//
// The workgroup walks the union of its tokens' selected KV blocks in
// ascending order. Each block's K and V are staged once in LDS, row-major
// (double-buffered, with a second block in flight in registers), and shared
// by all R heads; a tile skips a block none of its columns selected, and
// columns that did not select it contribute nothing. Per tile and block,
// with v_mfma_f32_16x16x32_bf16:
//     S^T[key, col] = K[key, :] . Q[col, :]           (8 MFMA)
//     online softmax per column (fp32, log2 domain)
//     O^T[d, col]  += V^T[d, key] . P^T[key, col]      (8 MFMA)
// S^T leaves each lane with 4 consecutive keys of 4 key tiles for one column,
// which is directly the B operand of the PV product when the 32-key k-axis is
// enumerated as {32m + 4g + e, 32m + 16 + 4g + e} (g = lane / 16); the V^T A
// operand is read from the row-major V tile with the same enumeration by the
// LDS transpose read (ds_read_b64_tr_b16).
#include "common.h"
#include "kernels.h"
#include "mfma.h"

namespace sparda {

constexpr int kMBs = 64;          // block size (keys per KV block)
constexpr int kMD = 64;           // head dim
constexpr int kMThreads = 256;    // 4 wavefronts
constexpr int kKRow = kMD + 8;    // K row in LDS, bf16 elements (144 B)
constexpr int kVRow = kMD + 16;   // V row in LDS, bf16 elements (160 B: 4 rows cover all banks)
constexpr int kMaxNBWords = 32;   // selection bitmask words per token (NB <= 1024)
constexpr float kLog2eM = 1.4426950408889634f;
// KV blocks kept in flight in registers ahead of the one being computed (1 or 2)
#ifndef SPARDA_PREFILL_PREFETCH
#define SPARDA_PREFILL_PREFETCH 2
#endif
// 1: the running max is only raised when a block's max exceeds it by more than
// 2^kLazyLog2 (probabilities stay <= 2^8, exact in fp32 accumulation), so the
// output is rarely rescaled. 0: raised on every increase.
#ifndef SPARDA_PF_LAZY
#define SPARDA_PF_LAZY 1
#endif
constexpr float kLazyLog2 = 8.0f;

struct MfmaSmem {
    uint16_t k[2][kMBs * kKRow];
    uint16_t v[2][kMBs * kVRow];
    uint32_t mask[64 * kMaxNBWords];
    uint16_t list[kMaxNBWords * 32];
    int n_list;
};

// 1: the wave's Q operands are held in registers for the whole kernel
#ifndef SPARDA_PF_QREG
#define SPARDA_PF_QREG 1
#endif
// resident workgroups per CU the register budget is sized for
#ifndef SPARDA_PF_OCCUPANCY
#define SPARDA_PF_OCCUPANCY 2
#endif

template <int R>
__global__ void __launch_bounds__(kMThreads, SPARDA_PF_OCCUPANCY)
prefill_mfma_kernel(const uint16_t* __restrict__ q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                    int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                    const int32_t* __restrict__ sel, const int32_t* __restrict__ n_sel, int64_t cap,
                    int64_t T, int H, int64_t NBq, int causal, float scale_log2,
                    uint16_t* __restrict__ out, int64_t out_sb, int64_t out_st) {
    __shared__ MfmaSmem sm;
    __shared__ uint16_t qs[64 * R * kKRow];  // Q rows (token, head) of this query block
    __shared__ uint32_t uni[kMaxNBWords];
    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int wave = tid / kWave;
    const int col16 = lane % 16;   // column within a tile
    const int grp = lane / 16;     // lane group

    // heaviest query blocks first; consecutive ids cycle through (b, g)
    const int64_t BH = static_cast<int64_t>(gridDim.x) / NBq;
    const int64_t bg = blockIdx.x % BH;
    const int64_t qb = NBq - 1 - blockIdx.x / BH;
    const int b = static_cast<int>(bg / H);
    const int g = static_cast<int>(bg % H);
    const int64_t t0 = qb * 64;
    const int64_t NB = cdiv(T, kMBs);
    const int nbw = static_cast<int>((NB + 31) / 32);
    const int t_valid = static_cast<int>(T - t0 < 64 ? T - t0 : 64);  // tokens of this block

    // ---- selection bitmask per token, and the workgroup's union of blocks ----
    for (int i = tid; i < 64 * nbw; i += kMThreads) sm.mask[i] = 0u;
    __syncthreads();
    if (tid < 64 && tid < t_valid) {
        const int64_t t = t0 + tid;
        uint32_t* row = sm.mask + tid * nbw;
        if (sel != nullptr) {
            const int64_t r = (static_cast<int64_t>(b) * H + g) * T + t;
            const int n = min(static_cast<int64_t>(n_sel[r]), cap);
            for (int i = 0; i < n; ++i) {
                const int j = sel[r * cap + i];
                if (j >= 0 && j < NB) row[j >> 5] |= 1u << (j & 31);
            }
        } else {
            const int64_t jmax = causal ? qb : NB - 1;
            for (int64_t j = 0; j <= jmax; ++j) row[j >> 5] |= 1u << (j & 31);
        }
    }
    __syncthreads();
    // union of the tokens' blocks, then its ascending list (one lane per block)
    if (tid < nbw) {
        uint32_t u = 0;
        for (int tt = 0; tt < 64; ++tt) u |= sm.mask[tt * nbw + tid];
        uni[tid] = u;
    }
    __syncthreads();
    if (wave == 0) {
        int base = 0;
        const uint64_t below = (1ull << lane) - 1ull;
        for (int c0 = 0; c0 < NB; c0 += kWave) {
            const int j = c0 + lane;
            const bool bit = j < NB && ((uni[j >> 5] >> (j & 31)) & 1u);
            const uint64_t bal = __ballot(bit);
            if (bit) sm.list[base + __popcll(bal & below)] = static_cast<uint16_t>(j);
            base += __popcll(bal);
        }
        if (lane == 0) sm.n_list = base;
    }
    // Q rows of the block: row (token * R + head), 128 B each
    for (int c = tid; c < 64 * R * 8; c += kMThreads) {
        const int row = c / 8, ch = c % 8;
        const int tk = row / R, hh = row % R;
        uint4 val = make_uint4(0u, 0u, 0u, 0u);
        if (tk < t_valid)
            val = *reinterpret_cast<const uint4*>(q + b * q_sb + (t0 + tk) * q_st +
                                                  static_cast<int64_t>(g * R + hh) * q_sh + ch * 8);
        *reinterpret_cast<uint4*>(&qs[row * kKRow + ch * 8]) = val;
    }

    // column c of tile tt is Q row 16*wave*R + c: token 16*wave + c/R, head c%R
    int tok[R];
#pragma unroll
    for (int tt = 0; tt < R; ++tt) tok[tt] = 16 * wave + (16 * tt + col16) / R;
    const uint16_t* qrow0 = qs + (16 * wave * R + col16) * kKRow + 8 * grp;

    f32x4 o[R][4];
    float m_run[R];
    // Row sums of P on the matrix cores: a constant A operand whose row 0 is
    // ones (2 MFMA per tile) replaces 16 VALU adds and the cross-lane
    // reductions; ol[tt][0] on lane group 0 holds the sum of column col16.
    f32x4 ol[R];
    bf16x8 ones_a;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones_a[e] = static_cast<__bf16>(col16 == 0 ? 1.0f : 0.0f);
#pragma unroll
    for (int tt = 0; tt < R; ++tt) {
        m_run[tt] = -__builtin_inff();
        ol[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[tt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // ---- staging: thread -> 16 B chunks (row c/8, chunk c%8), c = tid, tid+256 ----
    const uint16_t* kbase = k + b * kv_sb + static_cast<int64_t>(g) * kv_sh;
    const uint16_t* vbase = v + b * kv_sb + static_cast<int64_t>(g) * kv_sh;
    // two prefetch sets of plain registers: (ka, kb, va, vb) = K and V chunks
    // c = tid and c = tid + 256 (row c/8, 16-byte chunk c%8) of one block
    uint4 k0a, k0b, v0a, v0b, k1a, k1b, v1a, v1b;
    const int c_lo = tid, c_hi = tid + kMThreads;
    const int64_t col_lo = (c_lo % 8) * 8, col_hi = (c_hi % 8) * 8;
    const int lds_k_lo = (c_lo / 8) * kKRow + (c_lo % 8) * 8, lds_k_hi = (c_hi / 8) * kKRow + (c_hi % 8) * 8;
    const int lds_v_lo = (c_lo / 8) * kVRow + (c_lo % 8) * 8, lds_v_hi = (c_hi / 8) * kVRow + (c_hi % 8) * 8;
    // Rows past T (a ragged last block) load row T-1 instead: unconditional
    // loads keep the register sets free of writes while loads are in flight,
    // and those keys are masked (causal / tail) so only finite V values matter.
    auto row_off = [&](int64_t j, int c, int64_t col) {
        int64_t s = j * kMBs + c / 8;
        s = s < T ? s : T - 1;
        return s * kv_st + col;
    };
    // a whole block (the common case): a uniform block offset plus a fixed
    // per-thread offset, no clamp
    const int64_t own_lo = static_cast<int64_t>(c_lo / 8) * kv_st + col_lo;
    const int64_t own_hi = static_cast<int64_t>(c_hi / 8) * kv_st + col_hi;
#define SPARDA_FETCH(KA, KB, VA, VB, J)                                                   \
    do {                                                                                  \
        const int64_t jb_ = static_cast<int64_t>(J) * kMBs;                               \
        int64_t o_lo_, o_hi_;                                                             \
        if (jb_ + kMBs <= T) {                                                            \
            o_lo_ = jb_ * kv_st + own_lo;                                                 \
            o_hi_ = jb_ * kv_st + own_hi;                                                 \
        } else {                                                                          \
            o_lo_ = row_off((J), c_lo, col_lo);                                           \
            o_hi_ = row_off((J), c_hi, col_hi);                                           \
        }                                                                                 \
        KA = *reinterpret_cast<const uint4*>(kbase + o_lo_);                              \
        VA = *reinterpret_cast<const uint4*>(vbase + o_lo_);                              \
        KB = *reinterpret_cast<const uint4*>(kbase + o_hi_);                              \
        VB = *reinterpret_cast<const uint4*>(vbase + o_hi_);                              \
    } while (0)
#define SPARDA_STASH(KA, KB, VA, VB, BUF)                                                 \
    do {                                                                                  \
        *reinterpret_cast<uint4*>(&sm.k[BUF][lds_k_lo]) = KA;                             \
        *reinterpret_cast<uint4*>(&sm.v[BUF][lds_v_lo]) = VA;                             \
        *reinterpret_cast<uint4*>(&sm.k[BUF][lds_k_hi]) = KB;                             \
        *reinterpret_cast<uint4*>(&sm.v[BUF][lds_v_hi]) = VB;                             \
    } while (0)

#if SPARDA_PF_QREG
    bf16x8 qreg[R][2];  // filled once qs is complete
#endif
    // ---- one KV block against this wave's tiles ----
    // Per tile: S^T = K Q^T, online softmax, O^T += V^T P^T. Columns that did
    // not select the block get an exponent offset of -inf (P = 0) instead of
    // per-element selects; a tile none of whose columns selected the block is
    // skipped.
    auto compute = [&](int buf, int j) {
        // causal diagonal block / ragged non-causal tail: keys are masked (wave-uniform)
        const bool edge = (causal && j == qb) || (!causal && (j + 1) * kMBs > T);
        bool member[R];
        bool any = false;
#pragma unroll
        for (int tt = 0; tt < R; ++tt) {
            member[tt] = (sm.mask[tok[tt] * nbw + (j >> 5)] >> (j & 31)) & 1u;
            any = any || member[tt];
        }
        if (__ballot(any) == 0ull) return;
        bf16x8 ka[4][2];
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
                ka[n][kk] = lds_read8(&sm.k[buf][(16 * n + col16) * kKRow + 32 * kk + 8 * grp]);
        bf16x8 va[4][2];
        {
            // transposed A operand of V^T: source lane (grp, col16) points at
            // row 32m + 4grp + col16/4 (+16 for the upper half), columns 16dt + 4(col16%4)
            const int rsub = 4 * grp + col16 / 4;
            const int csub = 4 * (col16 % 4);
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    const uint16_t* base = &sm.v[buf][(32 * m + rsub) * kVRow + 16 * dt + csub];
                    const i16x4 lo = lds_read_tr(base);
                    const i16x4 hi = lds_read_tr(base + 16 * kVRow);
                    va[dt][m] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                }
        }
        const int lim_tail = static_cast<int>(T - static_cast<int64_t>(j) * kMBs) - 1;
        auto qk = [&](int tt, f32x4 (&s)[4]) {
#if SPARDA_PF_QREG
            const bf16x8 qb0 = qreg[tt][0];
            const bf16x8 qb1 = qreg[tt][1];
#else
            const bf16x8 qb0 = lds_read8(qrow0 + 16 * tt * kKRow);
            const bf16x8 qb1 = lds_read8(qrow0 + 16 * tt * kKRow + 32);
#endif
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                s[n] = f32x4{0.f, 0.f, 0.f, 0.f};
                s[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[n][0], qb0, s[n], 0, 0, 0);
                s[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[n][1], qb1, s[n], 0, 0, 0);
            }
        };
#pragma unroll
        for (int tt = 0; tt < R; ++tt) {
            if (__ballot(member[tt]) == 0ull) continue;
            f32x4 s[4];
            qk(tt, s);
            if (edge) {
                // causal diagonal: key <= token; non-causal tail: key < T
                const int l = causal ? tok[tt] : lim_tail;
#pragma unroll
                for (int n = 0; n < 4; ++n)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (16 * n + 4 * grp + i > l) s[n][i] = -__builtin_inff();
            }
            float mx = max16_nn(s);
            mx = member[tt] ? mx : -__builtin_inff();
            mx = pair32_max(pair16_max(mx));
            const float cand = mx * scale_log2;  // this block's column max, log2 units
#if SPARDA_PF_LAZY
            // m_run = -inf takes any finite max; otherwise raise only past 2^kLazyLog2
            const float m_new = cand > m_run[tt] + kLazyLog2 ? cand : m_run[tt];
#else
            const float m_new = __builtin_fmaxf(m_run[tt], cand);
#endif
            // non-members: offset -inf gives P = 0 and leaves the running state alone
            const float neg = member[tt] ? -m_new : -__builtin_inff();
            const float alpha = m_new != m_run[tt] ? __builtin_amdgcn_exp2f(m_run[tt] - m_new) : 1.0f;
            m_run[tt] = m_new;
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
            if (__ballot(alpha != 1.0f) != 0ull) {
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) o[tt][dt] *= alpha;
                ol[tt] *= alpha;
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

    __syncthreads();
    const int n_list = sm.n_list;
#if SPARDA_PF_QREG
    // the wave's Q operands do not change across blocks: read them once
#pragma unroll
    for (int tt = 0; tt < R; ++tt) {
        qreg[tt][0] = lds_read8(qrow0 + 16 * tt * kKRow);
        qreg[tt][1] = lds_read8(qrow0 + 16 * tt * kKRow + 32);
    }
#endif
#if SPARDA_PREFILL_PREFETCH == 2
    // prologue: block 0 staged, block 1 in flight
    SPARDA_FETCH(k0a, k0b, v0a, v0b, sm.list[0]);
    if (n_list > 1) SPARDA_FETCH(k1a, k1b, v1a, v1b, sm.list[1]);
    SPARDA_STASH(k0a, k0b, v0a, v0b, 0);
    __syncthreads();
    // iteration u computes block u from buffer u&1, keeps block u+1 in
    // flight in register set (u+1)&1 and issues block u+2 into set u&1
    for (int u = 0; u < n_list; u += 2) {
        if (u + 2 < n_list) SPARDA_FETCH(k0a, k0b, v0a, v0b, sm.list[u + 2]);
        compute(0, sm.list[u]);
        if (u + 1 < n_list) SPARDA_STASH(k1a, k1b, v1a, v1b, 1);
        __syncthreads();
        if (u + 1 >= n_list) break;
        if (u + 3 < n_list) SPARDA_FETCH(k1a, k1b, v1a, v1b, sm.list[u + 3]);
        compute(1, sm.list[u + 1]);
        if (u + 2 < n_list) SPARDA_STASH(k0a, k0b, v0a, v0b, 0);
        __syncthreads();
    }
#else
    SPARDA_FETCH(k0a, k0b, v0a, v0b, sm.list[0]);
    SPARDA_STASH(k0a, k0b, v0a, v0b, 0);
    __syncthreads();
    for (int u = 0; u < n_list; u += 2) {
        if (u + 1 < n_list) SPARDA_FETCH(k0a, k0b, v0a, v0b, sm.list[u + 1]);
        compute(0, sm.list[u]);
        if (u + 1 < n_list) SPARDA_STASH(k0a, k0b, v0a, v0b, 1);
        __syncthreads();
        if (u + 1 >= n_list) break;
        if (u + 2 < n_list) SPARDA_FETCH(k0a, k0b, v0a, v0b, sm.list[u + 2]);
        compute(1, sm.list[u + 1]);
        if (u + 2 < n_list) SPARDA_STASH(k0a, k0b, v0a, v0b, 0);
        __syncthreads();
    }
#endif
#undef SPARDA_FETCH
#undef SPARDA_STASH

    // ---- epilogue: out[b, t, h*64 + d] = O / l ----
#pragma unroll
    for (int tt = 0; tt < R; ++tt) {
        // row sum of column col16 sits in lane col16 (lane group 0), element 0;
        // read by every lane before any lane leaves
        const float lsum = __shfl(ol[tt][0], col16, kWave);
        if (tok[tt] >= t_valid) continue;
        const int c = 16 * tt + col16;
        const int hh = c % R;
        const float inv = 1.0f / lsum;
        uint16_t* orow = out + b * out_sb + (t0 + tok[tt]) * out_st + static_cast<int64_t>(g * R + hh) * kMD;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            bf16x4 w;
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = static_cast<__bf16>(o[tt][dt][i] * inv);
            *reinterpret_cast<bf16x4*>(orow + 16 * dt + 4 * grp) = w;
        }
    }
}

bool prefill_mfma_supported(int dtype, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t bs,
                            int64_t q_sb, int64_t q_st, int64_t q_sh, int64_t kv_sb, int64_t kv_st,
                            int64_t kv_sh, int64_t out_sb, int64_t out_st, const void* q, const void* k,
                            const void* v, const void* out) {
    if (dtype != SPARDA_BF16 || D != kMD || bs != kMBs) return false;
    if (cdiv(T, kMBs) > kMaxNBWords * 32) return false;
    const int64_t R = Hq / Hkv;
    if (R < 1 || R > 4) return false;
    auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!al16(q) || !al16(k) || !al16(v) || (reinterpret_cast<uintptr_t>(out) & 7u)) return false;
    if ((q_sb % 8) || (q_st % 8) || (q_sh % 8) || (kv_sb % 8) || (kv_st % 8) || (kv_sh % 8)) return false;
    if ((out_sb % 4) || (out_st % 4)) return false;
    return true;
}

int launch_prefill_mfma(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k,
                        const void* v, int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                        const int32_t* sel, const int32_t* n_sel, int64_t cap, int64_t B, int64_t T,
                        int64_t Hq, int64_t Hkv, int64_t bs, int causal, float scale, void* out,
                        int64_t out_sb, int64_t out_st, hipStream_t stream) {
    (void)bs;
    const int64_t NBq = cdiv(T, kMBs);
    const int64_t R = Hq / Hkv;
    dim3 grid(static_cast<unsigned>(B * Hkv * NBq));
    const float sl = scale * kLog2eM;
#define SPARDA_MF(R_)                                                                                     \
    hipLaunchKernelGGL((prefill_mfma_kernel<R_>), grid, dim3(kMThreads), 0, stream,                       \
                       static_cast<const uint16_t*>(q), q_sb, q_st, q_sh, static_cast<const uint16_t*>(k), \
                       static_cast<const uint16_t*>(v), kv_sb, kv_st, kv_sh, sel, n_sel, cap, T,           \
                       static_cast<int>(Hkv), NBq, causal, sl, static_cast<uint16_t*>(out), out_sb, out_st)
    switch (R) {
        case 1: SPARDA_MF(1); break;
        case 2: SPARDA_MF(2); break;
        case 3: SPARDA_MF(3); break;
        default: SPARDA_MF(4); break;
    }
#undef SPARDA_MF
    return check_hip(hipGetLastError(), "prefill_mfma_kernel");
}

}  // namespace sparda
