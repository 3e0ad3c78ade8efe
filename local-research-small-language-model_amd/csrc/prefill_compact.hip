// bf16 block-sparse GQA prefill over compacted tiles (D = 64, KV blocks of
// BS = 64 or 32 keys, at most 10 selected blocks per token).
//
// One workgroup of 12 wavefronts (one per CU, three per SIMD) serves one
// (sequence b, KV head g, query window qb): W = 128 query tokens (64 for
// R = 4, whose 128-token accumulators would not fit the LDS) x R = Hq/Hkv
// query heads = W*R columns, column c = token * R + head. Every query token picks its own blocks, so a KV block
// is attended by only some of the window's columns. For each block j in the
// union of the window's selections, the columns that selected j are packed,
// in token order, into tiles of 16 (the N side of v_mfma_f32_16x16x32_bf16):
//     S^T[key, slot] = K[key, :] . Q[col(slot), :]          (8 MFMA)
//     P = exp2(S^T * scale * log2 e - m_ref[col])            (VALU, bf16)
//     O^T[d, slot]  += V^T[d, key] . P^T[key, slot]          (8 MFMA, C = acc)
// so a tile wastes only its padding slots (and the masked half of the causal
// diagonal block).
//
// Accumulation. P is taken against a fixed per-column reference m_ref: the
// score of the first key of the column's first listed block (key 0, the sink,
// for router lists), computed in the set-up. It is the score of an allowed
// key, so it never exceeds the row maximum and the row keeps a term P ~ 1.
// Contributions are then plain sums (no rescaling): each tile's O^T and row
// sums are formed from zero and added into fp32 accumulators acc[col][d],
// lsum[col] in LDS. Work items (a block and up to three of its tiles) are
// taken by the waves from a shared counter in block order; a column's
// contributions are added in ascending block order, each tile waiting until
// the column's earlier blocks have been added (vers[col] = blocks added so
// far), so the result does not depend on timing. A block whose row sum passes
// 2^64 (a score more than 64 log2-units above the reference) trips a flag;
// the workgroup then takes the exact row maxima in a scores-only pass and
// redoes the window against them.
//
// K A operands are read straight from memory; V is staged per wavefront in
// LDS, half a block at a time (XOR-swizzled 16-byte chunks), and read
// transposed with ds_read_b64_tr_b16.
#include "common.h"
#include "kernels.h"
#include "mfma.h"
#include "route_rows.h"

namespace sparda {

// Per-device status word: SPARDA_STATUS_* bits set by kernels that had to
// abandon work (read and cleared by sparda_status). Each GPU holds its own copy.
__device__ uint32_t g_sparda_status;

namespace {

constexpr int kCMaxCap = 10;                    // selection entries per token

constexpr int kCMaxNB = 1024;                   // KV blocks
// wavefronts per workgroup: one workgroup per CU, three wavefronts per SIMD
constexpr int kCWaves = 12;
constexpr int kCThreads = kCWaves * kWave;

// a query window of W tokens (128; 64 for R = 4, whose accumulators for 128
// tokens would not fit the LDS) per workgroup. Its 64-token sets are routed
// by kSetWaves waves each, whose first wave then holds the set's tokens
// (lane = token) through the set-up.
template <int W>
struct Win {
    static_assert(W == 64 || W == 128, "windows of 64 or 128 tokens");
    static constexpr int kMaxPairs = W * kCMaxCap;               // (token, block) pairs of a window
    static constexpr int kMaxUnion = kMaxPairs < kCMaxNB ? kMaxPairs : kCMaxNB;  // distinct blocks
    static constexpr int kSetWaves = kCWaves / (W / 64);
};

// the tokens of a window that selected a block: bit t of word t / 64
template <int W>
struct TokMask {
    unsigned long long w[W / 64];
};
template <int W>
__device__ __forceinline__ bool mask_any(const TokMask<W>& m) {
    bool a = false;
#pragma unroll
    for (int i = 0; i < W / 64; ++i) a = a || m.w[i] != 0ull;
    return a;
}
template <int W>
__device__ __forceinline__ int mask_count(const TokMask<W>& m) {
    int n = 0;
#pragma unroll
    for (int i = 0; i < W / 64; ++i) n += __popcll(m.w[i]);
    return n;
}
// selecting tokens before token t
template <int W>
__device__ __forceinline__ int mask_count_below(const TokMask<W>& m, int t) {
    int n = 0;
#pragma unroll
    for (int i = 0; i < W / 64; ++i) {
        const int lo = 64 * i;
        n += t >= lo + 64 ? __popcll(m.w[i]) : (t > lo ? __popcll(m.w[i] & ((1ull << (t - lo)) - 1ull)) : 0);
    }
    return n;
}
constexpr float kCLog2e = 1.4426950408889634f;
constexpr float kCGuard = 18446744073709551616.0f;  // 2^64
constexpr uint32_t kCSpinLimit = 1u << 20;  // polls of one ordering wait before it is abandoned
constexpr int kSentinel = 0x7fffffff;
constexpr int kCRouteK = kCMaxCap - 2;         // router picks per token when the kernel routes
constexpr int kCRouteDf = 64;                   // forecast dimension when the kernel routes

template <int R, int W>
struct CompactSmem {
    static constexpr int kCols = W * R;
    static constexpr int kMaxUnion = Win<W>::kMaxUnion;
    static constexpr int kMaxItems = (R * Win<W>::kMaxPairs) / 16 + kMaxUnion;
    // fp32 accumulators, slab layout: acc[s * kCols + col] = O[col][4s .. 4s+3].
    // During the set-up the same bytes hold the per-block token bitmaps, the
    // block -> union map and per-token facts.
    float4 acc[16 * kCols];
    uint16_t vstage[kCWaves][32 * 64];          // half a V block per wave, swizzled
    uint32_t items[kMaxItems];                  // u | first tile << 16
    float mref[kCols];                          // log2 units
    float lsum[kCols];                          // row sums (exact-max pass: order keys)
    int32_t vers[kCols];                        // blocks added to the column so far
    uint16_t ulist[kMaxUnion];                  // block index of union entry u
    uint16_t uofs[kMaxUnion + 1];               // records of union block u: uofs[u] .. uofs[u+1]-1
    uint8_t rankbuf[Win<W>::kMaxPairs];         // per record: rank of the block in the token's list
    uint8_t toklist[Win<W>::kMaxPairs];         // per record: the selecting token (ascending)
    int n_union, n_items, next_item, flag;
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int swz(int r) { return 2 * ((r >> 1) & 3); }
// element index of (local row r, element col) in a swizzled V half-stage
__device__ __forceinline__ int vidx(int r, int col) { return r * 64 + (((col >> 3) ^ swz(r)) << 3) + (col & 7); }

__device__ __forceinline__ float key_to_float(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

}  // namespace

// W = 128 (R <= 3) or 64 (R = 4): one workgroup of 12 wavefronts per CU; the
// wider window's tiles are fuller when each token's selections are spread
// over many blocks.
// BS: keys per KV block (64 or 32).
// FDT < 0: the token lists come from sel / n_sel. FDT = the forecast's dtype:
// the kernel routes its own window first (the router's per-set code, so the
// lists are the router's bit for bit) and, with rt.sel set, also writes them
// out as the router does.
template <int R, int BS, int FDT, int W>
__global__ void __launch_bounds__(kCThreads, 1)
prefill_compact_kernel(const uint16_t* __restrict__ q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                       const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                       int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                       const int32_t* __restrict__ sel, const int32_t* __restrict__ n_sel, int64_t cap,
                       int64_t T, int H, int64_t NBq, int causal, float scale_log2,
                       uint16_t* __restrict__ out, int64_t out_sb, int64_t out_st, CompactRoute rt,
                       uint32_t spin_limit) {
    using Smem = CompactSmem<R, W>;
    using Mask = TokMask<W>;
    constexpr int kCols = Smem::kCols;
    constexpr int kT = kCThreads;
    constexpr int kSetWaves = Win<W>::kSetWaves;
    constexpr int kMaxNB = kCMaxNB;
    __shared__ Smem sm;
    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int wave = tid / kWave;
    const int col16 = lane % 16;
    const int grp = lane / 16;
    const uint64_t below = (1ull << lane) - 1ull;
    // token tok of the window is held by lane tok % 64 of wave kSetWaves * (tok / 64)
    const bool owner = wave % kSetWaves == 0;
    const int tok = (wave / kSetWaves) * 64 + lane;

    // heaviest query windows first, XCD-aware when there are few (b, g) pairs
    const int64_t BH = static_cast<int64_t>(gridDim.x) / NBq;
    int64_t bg, qb;
    window_order(blockIdx.x, BH, NBq, bg, qb);
    const int b = static_cast<int>(bg / H);
    const int g = static_cast<int>(bg % H);
    static_assert(BS == 64 || BS == 32, "KV blocks of 64 or 32 keys");
    constexpr int kSub = BS / 16;  // 16-key sub-tiles of a block (the M side of S^T)
    constexpr int kHalf = BS / 32; // 32-key halves of a block (the K side of O^T)
    // tiles per work item: three for 64-key blocks, two for 32-key blocks
    // (whose items then hold fewer keys; three measured 6-7% slower there,
    // 1-13% faster for 64-key blocks)
    constexpr int kCChunk = BS == 64 ? 3 : 2;
    const int64_t t0 = qb * W;
    const int64_t NB = cdiv(T, BS);
    const int t_valid = static_cast<int>(T - t0 < W ? T - t0 : W);
    const bool has_tok = owner && tok < t_valid;
    // highest block a token here may attend
    const int jmax = static_cast<int>(causal ? (t0 + t_valid - 1) / BS : NB - 1);
    const uint16_t* kbase = k + b * kv_sb + static_cast<int64_t>(g) * kv_sh;
    const uint16_t* vbase = v + b * kv_sb + static_cast<int64_t>(g) * kv_sh;
    const uint16_t* qbase = q + b * q_sb + t0 * q_st + static_cast<int64_t>(g * R) * q_sh;
    // element offsets inside a window / a block fit in 32 bits (checked by the host)
    const int q_st32 = static_cast<int>(q_st), q_sh32 = static_cast<int>(q_sh), kv_st32 = static_cast<int>(kv_st);

    static_assert(kMaxNB * (sizeof(Mask) + sizeof(uint16_t)) <= sizeof(sm.acc), "set-up aliases fit in acc");
    static_assert(sizeof(Smem) <= 160 * 1024, "one workgroup's LDS");
    Mask* bitmap = reinterpret_cast<Mask*>(sm.acc);                   // [kMaxNB], set-up only
    uint16_t* jmap = reinterpret_cast<uint16_t*>(bitmap + kMaxNB);    // [kMaxNB], set-up only

    // ---- set-up 1: this thread's token list (sorted, repeats and out-of-range entries dropped) ----
    int lst[kCMaxCap];
#pragma unroll
    for (int i = 0; i < kCMaxCap; ++i) lst[i] = kSentinel;
    // blocks past the token's own (no key of theirs is allowed) are dropped
    const int tlim = static_cast<int>(causal ? (t0 + tok) / BS : NB - 1);
    if constexpr (FDT >= 0) {
        // each group of kSetWaves waves routes 64 of the window's tokens,
        // every wave scoring its share of the candidate blocks; the group's
        // first wave merges (through the group's V staging bytes, unused
        // until the tiles: 4 KB per wave, one wave's key lists) and holds
        // token tok's picks
        int32_t picks[kCRouteK];
        if (route_set<FDT, kCRouteDf, kCRouteK, kSetWaves>(
                rt.f, rt.fsb, rt.fst, rt.fsh, rt.protos, b, g, H, qb * (W / 64) + wave / kSetWaves, T, NB, BS,
                rt.ke, causal, 0, rt.scale, nullptr, 0,
                reinterpret_cast<double*>(&sm.vstage[kSetWaves * (wave / kSetWaves)][0]), picks) &&
            tok < t_valid) {
            // {0, own} U picks, own = the token's block (prefill positions start at 0)
            const int own = static_cast<int>((t0 + tok) / BS);
            int raw[kCMaxCap];
            raw[0] = 0;
            raw[1] = own;
#pragma unroll
            for (int i = 0; i < kCRouteK; ++i) raw[i + 2] = picks[i];
#pragma unroll
            for (int i = 0; i < kCMaxCap; ++i) lst[i] = (raw[i] >= 0 && raw[i] <= tlim) ? raw[i] : kSentinel;
        }
    } else if (has_tok) {
        const int64_t r = (static_cast<int64_t>(b) * H + g) * T + t0 + tok;
        const int32_t* row = sel + r * cap;
        int raw[kCMaxCap];
#pragma unroll
        for (int i = 0; i < kCMaxCap; ++i) raw[i] = i < cap ? row[i] : -1;  // issued with the count's load
        const int64_t nr = n_sel[r];
        const int n = static_cast<int>(nr < 0 ? 0 : (nr > cap ? cap : nr));
#pragma unroll
        for (int i = 0; i < kCMaxCap; ++i) lst[i] = (i < n && raw[i] >= 0 && raw[i] <= tlim) ? raw[i] : kSentinel;
    }
    if (has_tok) {
        // ascending, repeats dropped (odd-even transposition sort, twice)
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
            for (int rd = 0; rd < kCMaxCap; ++rd)
#pragma unroll
                for (int i = rd & 1; i + 1 < kCMaxCap; i += 2) {
                    const int a = lst[i], c = lst[i + 1];
                    lst[i] = a < c ? a : c;
                    lst[i + 1] = a < c ? c : a;
                }
            if (pass == 0) {
#pragma unroll
                for (int i = kCMaxCap - 1; i > 0; --i)
                    if (lst[i] == lst[i - 1]) lst[i] = kSentinel;
            }
        }
        if constexpr (FDT >= 0) {
            if (rt.sel != nullptr) {
                // the router's output rows: the list, -1 padding, the count
                const int64_t r = (static_cast<int64_t>(b) * H + g) * T + t0 + tok;
                int32_t* orow = rt.sel + r * rt.cap;
                int n = 0;
#pragma unroll
                for (int i = 0; i < kCMaxCap; ++i) n += lst[i] != kSentinel;
#pragma unroll
                for (int i = 0; i < kCMaxCap; ++i)
                    if (i < rt.cap) orow[i] = lst[i] != kSentinel ? lst[i] : -1;
                for (int i = kCMaxCap; i < rt.cap; ++i) orow[i] = -1;
                rt.n_sel[r] = n;
            }
        }
    }
    // the first key of the token's first listed block (always an allowed key),
    // or -1: its score is the column's reference (set-up 2). Held in the row
    // sums' bytes until set-up 3 clears them.
    if (owner) reinterpret_cast<int*>(sm.lsum)[tok] = (has_tok && lst[0] != kSentinel) ? lst[0] * BS : -1;
    for (int i = tid; i <= jmax; i += kT) bitmap[i] = Mask{};
    __syncthreads();
    if (has_tok) {
#pragma unroll
        for (int i = 0; i < kCMaxCap; ++i)
            if (lst[i] != kSentinel) atomicOr(&bitmap[lst[i]].w[tok / 64], 1ull << (tok % 64));
    }
    __syncthreads();

    // ---- set-up 2: union of the selected blocks, work items, rank offsets (wave 0) ----
    if (wave == 0) {
        int nu = 0, ni = 0, nrk = 0;
        for (int c0 = 0; c0 <= jmax; c0 += kWave) {
            const int j = c0 + lane;
            const Mask M = j <= jmax ? bitmap[j] : Mask{};
            const bool nz = mask_any(M);
            const uint64_t bal = __ballot(nz);
            const int nt = mask_count(M);
            const int tiles = (R * nt + 15) / 16;
            const int chunks = nz ? (tiles + kCChunk - 1) / kCChunk : 0;
            const int rk = nz ? nt : 0;
            int sc = chunks, sr = rk;  // inclusive prefix sums over the lanes
#pragma unroll
            for (int o = 1; o < kWave; o <<= 1) {
                const int a = __shfl_up(sc, o, kWave), c = __shfl_up(sr, o, kWave);
                if (lane >= o) {
                    sc += a;
                    sr += c;
                }
            }
            if (nz) {
                const int pos = nu + __popcll(bal & below);
                const int item0 = ni + sc - chunks;
                sm.ulist[pos] = static_cast<uint16_t>(j);
                sm.uofs[pos] = static_cast<uint16_t>(nrk + sr - rk);
                jmap[j] = static_cast<uint16_t>(pos);
                for (int cc = 0; cc < chunks; ++cc)
                    sm.items[item0 + cc] = static_cast<uint32_t>(pos) | (static_cast<uint32_t>(cc * kCChunk) << 16);
            }
            nu += __popcll(bal);
            ni += __shfl(sc, kWave - 1, kWave);
            nrk += __shfl(sr, kWave - 1, kWave);
        }
        if (lane == 0) {
            sm.n_union = nu;
            sm.n_items = ni;
            sm.uofs[nu] = static_cast<uint16_t>(nrk);
            sm.next_item = 0;
            sm.flag = 0;
        }
    } else {
        // meanwhile the other waves take each column's reference: the score
        // (log2 units) of the first key of the column's first listed block.
        // Any allowed score serves (the row keeps a term near 1, so the sums
        // neither underflow nor, short of a score 64 log2-units above it,
        // overflow); fixing it before the tiles leaves no tile waiting for
        // another tile's maximum.
        for (int c = tid - kWave; c < kCols; c += kT - kWave) {
            const int tk = c / R, h = c - (c / R) * R;
            const int s0 = reinterpret_cast<const int*>(sm.lsum)[tk];
            float ref = 0.0f;
            if (s0 >= 0) {
                const uint16_t* qr = qbase + tk * q_st32 + h * q_sh32;
                const uint16_t* kr = kbase + static_cast<int64_t>(s0) * kv_st;
                u32x4 qv[8], kv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    qv[i] = *reinterpret_cast<const u32x4*>(qr + 8 * i);
                    kv[i] = *reinterpret_cast<const u32x4*>(kr + 8 * i);
                }
                float a = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        a = __builtin_fmaf(__uint_as_float(qv[i][e] << 16), __uint_as_float(kv[i][e] << 16), a);
                        a = __builtin_fmaf(__uint_as_float(qv[i][e] & 0xffff0000u),
                                           __uint_as_float(kv[i][e] & 0xffff0000u), a);
                    }
                ref = a * scale_log2;
            }
            sm.mref[c] = ref;
        }
    }
    __syncthreads();

    // ---- set-up 3: ranks (position of each block in a token's list) ----
    if (has_tok) {
#pragma unroll
        for (int i = 0; i < kCMaxCap; ++i) {
            if (lst[i] != kSentinel) {
                const int u = jmap[lst[i]];
                const int e = sm.uofs[u] + mask_count_below(bitmap[lst[i]], tok);
                sm.rankbuf[e] = static_cast<uint8_t>(i);
                sm.toklist[e] = static_cast<uint8_t>(tok);
            }
        }
    }
    for (int c = tid; c < kCols; c += kT) {
        sm.lsum[c] = 0.0f;
        sm.vers[c] = 0;
    }
    __syncthreads();  // the set-up aliases in acc are dead from here
    for (int i = tid; i < 16 * kCols; i += kT) sm.acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    __syncthreads();

    // ---- the tiles ----
    bf16x8 ones_a;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones_a[e] = static_cast<__bf16>(col16 == 0 ? 1.0f : 0.0f);
    // per-lane element offsets inside a block: K A operand (key 16n + col16,
    // dims 32kk + 8grp), V rows (chunk lane + 64i: row lane/8 + 8i, 16-byte column lane%8)
    constexpr int kKR = 2 * kSub;  // K operand registers (u32x4) per block
    constexpr int kVR = BS / 8;    // V row chunks (u32x4) per lane per block
    const int koff = col16 * kv_st32 + 8 * grp;
    const int voff = (lane / 8) * kv_st32 + (lane % 8) * 8;
    const int64_t last_row = T - 1;

    auto grab = [&]() __attribute__((always_inline)) -> int {
        int it = 0;
        if (lane == 0) it = atomicAdd(&sm.next_item, 1);
        return __builtin_amdgcn_readfirstlane(it);
    };
    // rows past T (a ragged last block) read row T-1: finite values, masked
    auto load_k = [&](int item, u32x4 (&kr)[kKR]) __attribute__((always_inline)) {
        const int64_t r0 = static_cast<int64_t>(sm.ulist[item & 0xffff]) * BS;
        if (r0 + BS <= T) {
            const uint16_t* blk = kbase + r0 * kv_st;
#pragma unroll
            for (int n = 0; n < kSub; ++n)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk)
                    kr[2 * n + kk] = *reinterpret_cast<const u32x4*>(blk + koff + 16 * n * kv_st32 + 32 * kk);
        } else {
#pragma unroll
            for (int n = 0; n < kSub; ++n) {
                int64_t row = r0 + 16 * n + col16;
                row = row < last_row ? row : last_row;
#pragma unroll
                for (int kk = 0; kk < 2; ++kk)
                    kr[2 * n + kk] = *reinterpret_cast<const u32x4*>(kbase + row * kv_st + 32 * kk + 8 * grp);
            }
        }
    };
    auto load_v = [&](int item, u32x4 (&vr)[kVR]) __attribute__((always_inline)) {
        const int64_t r0 = static_cast<int64_t>(sm.ulist[item & 0xffff]) * BS;
        if (r0 + BS <= T) {
            const uint16_t* blk = vbase + r0 * kv_st;
#pragma unroll
            for (int i = 0; i < kVR; ++i) vr[i] = *reinterpret_cast<const u32x4*>(blk + voff + 8 * i * kv_st32);
        } else {
#pragma unroll
            for (int i = 0; i < kVR; ++i) {
                int64_t row = r0 + lane / 8 + 8 * i;
                row = row < last_row ? row : last_row;
                vr[i] = *reinterpret_cast<const u32x4*>(vbase + row * kv_st + (lane % 8) * 8);
            }
        }
    };

    uint16_t* vst = sm.vstage[wave];
    const int rsub = 4 * grp + col16 / 4;
    const int csub = 4 * (col16 % 4);

    // column of slot col16 in tile i of the current item
    struct Slot {
        int tr;     // rank of the slot's token among the block's selecting tokens
        int c;      // window column (token * R + head)
        int qoff;   // element offset of the slot's q row (+ 8 grp) from qbase
        bool valid;
    };
    auto slot = [&](int i, int ncol, int rofs) __attribute__((always_inline)) -> Slot {
        const int e = 16 * i + col16;
        Slot s_;
        s_.valid = e < ncol;
        const int ei = s_.valid ? e : ncol - 1;  // padding slots repeat the last column, masked
        s_.tr = ei / R;
        const int h = ei - s_.tr * R;
        const int tk = sm.toklist[rofs + s_.tr];
        s_.c = tk * R + h;
        s_.qoff = tk * q_st32 + h * q_sh32 + 8 * grp;
        return s_;
    };

    // one work item (packed word: union entry u | first tile i0 << 16): the
    // up to kCChunk tiles [i0, i1) of union block u, processed phase by phase
    // so that their latencies overlap: K, V and q loads with the columns'
    // references, S = K Q^T, P, O = V^T P^T, then one wait and one
    // read-add-write of every column. (The loads are not issued an item ahead: three waves per SIMD
    // cover their latency, and the registers that would hold the next item's
    // K and V are what lets the third wave fit.)
    // mode 0: P against the columns' references; 1: scores only, the exact
    // column maxima (into the row sums' bytes)
    auto process = [&](int item, int mode) __attribute__((always_inline)) {
        u32x4 kr[kKR], vr[kVR];
        load_k(item, kr);
        load_v(item, vr);
        const int u = item & 0xffff;
        const int i0 = item >> 16;
        const int j = sm.ulist[u];
        const int rofs = sm.uofs[u];
        const int ncol = R * (sm.uofs[u + 1] - rofs);
        const int tiles = (ncol + 15) / 16;
        const int nt = (i0 + kCChunk < tiles ? i0 + kCChunk : tiles) - i0;  // 1 .. kCChunk
        // causal: a block that ends past the window's first token holds keys
        // beyond some selecting tokens (key j*BS + i is allowed up to token t0 + tk)
        const bool diag = causal && (static_cast<int64_t>(j) + 1) * BS - 1 > t0;
        const int dbase = static_cast<int>(t0 - static_cast<int64_t>(j) * BS);
        const int lim_tail = (!causal && (static_cast<int64_t>(j) + 1) * BS > T) ? static_cast<int>(T - j * static_cast<int64_t>(BS)) : BS;
        const bool masked = diag || lim_tail < BS;  // causal diagonal or ragged tail block

        Slot sl[kCChunk];
        u32x4 qa[kCChunk], qc[kCChunk];
        int rank[kCChunk];
        float ref[kCChunk];
#pragma unroll
        for (int t = 0; t < kCChunk; ++t) {
            if (t < nt) {
                sl[t] = slot(i0 + t, ncol, rofs);
                qa[t] = *reinterpret_cast<const u32x4*>(qbase + sl[t].qoff);
                qc[t] = *reinterpret_cast<const u32x4*>(qbase + sl[t].qoff + 32);
                rank[t] = sm.rankbuf[rofs + sl[t].tr];
                ref[t] = sm.mref[sl[t].c];
            }
        }
        // S^T = K Q^T for every tile (every key sub-tile: on the causal
        // diagonal the masks below remove what lies past a column's token;
        // skipping those sub-tiles costs more in branches than it saves)
        f32x4 s[kCChunk][kSub];
#pragma unroll
        for (int t = 0; t < kCChunk; ++t) {
            if (t < nt) {
#pragma unroll
                for (int n = 0; n < kSub; ++n) {
                    s[t][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[2 * n]),
                                                                      __builtin_bit_cast(bf16x8, qa[t]),
                                                                      f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    s[t][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[2 * n + 1]),
                                                                      __builtin_bit_cast(bf16x8, qc[t]), s[t][n], 0, 0, 0);
                }
            }
        }
        // V^T operands: stage each half of the block, read it transposed
        bf16x8 va[4][kHalf];
#pragma unroll
        for (int m = 0; m < kHalf; ++m) {
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = lane / 8 + 8 * i;
                *reinterpret_cast<u32x4*>(vst + vidx(r, (lane % 8) * 8)) = vr[4 * m + i];
            }
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const i16x4 lo = lds_read_tr(vst + vidx(rsub, 16 * dt + csub));
                const i16x4 hi = lds_read_tr(vst + vidx(rsub + 16, 16 * dt + csub));
                va[dt][m] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            }
        }
        __builtin_amdgcn_wave_barrier();

        // masks: keys past a column's token on the causal diagonal, keys past T
        // in a ragged last block
        bool own[kCChunk];
#pragma unroll
        for (int t = 0; t < kCChunk; ++t) {
            if (t < nt) {
                own[t] = sl[t].valid && grp == 0;
                if (masked) {
                    const int lim = diag ? dbase + sl[t].c / R : lim_tail - 1;  // keys <= lim are allowed
#pragma unroll
                    for (int n = 0; n < kSub; ++n)
#pragma unroll
                        for (int ii = 0; ii < 4; ++ii)
                            if (16 * n + 4 * grp + ii > lim) s[t][n][ii] = -__builtin_inff();
                }
            }
        }
        if (mode == 1) {
            // exact column maxima (order keys of the maxima, in the row sums' bytes)
#pragma unroll
            for (int t = 0; t < kCChunk; ++t) {
                if (t < nt) {
                    const float cm = pair32_max(pair16_max(max_sub_nn(s[t]))) * scale_log2;
                    if (own[t]) atomicMax(reinterpret_cast<uint32_t*>(sm.lsum) + sl[t].c, order_key(cm));
                }
            }
            return;
        }
        // P = exp2(S * scale log2 e - reference), bf16
        uint4 pw[kCChunk][kHalf];
#pragma unroll
        for (int t = 0; t < kCChunk; ++t) {
            if (t < nt) {
                const float neg = sl[t].valid ? -ref[t] : -__builtin_inff();
#pragma unroll
                for (int mm = 0; mm < kHalf; ++mm) {
                    bf16x8 pb;
#pragma unroll
                    for (int ii = 0; ii < 4; ++ii) {
                        pb[ii] = static_cast<__bf16>(
                            __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][2 * mm][ii], scale_log2, neg)));
                        pb[4 + ii] = static_cast<__bf16>(
                            __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][2 * mm + 1][ii], scale_log2, neg)));
                    }
                    pw[t][mm] = __builtin_bit_cast(uint4, pb);
                }
            }
        }
        // O^T = V^T P^T and the row sums, from zero
        f32x4 o[kCChunk][4], ol[kCChunk];
#pragma unroll
        for (int t = 0; t < kCChunk; ++t) {
            if (t < nt) {
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    o[t][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt][0], __builtin_bit_cast(bf16x8, pw[t][0]),
                                                                       f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                    for (int mm = 1; mm < kHalf; ++mm)
                        o[t][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            va[dt][mm], __builtin_bit_cast(bf16x8, pw[t][mm]), o[t][dt], 0, 0, 0);
                }
                ol[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones_a, __builtin_bit_cast(bf16x8, pw[t][0]),
                                                                f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int mm = 1; mm < kHalf; ++mm)
                    ol[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones_a, __builtin_bit_cast(bf16x8, pw[t][mm]),
                                                                    ol[t], 0, 0, 0);
            }
        }
        // add into every column after its earlier blocks (read-add-write, in block
        // order). The wave issues ahead of the SIMD's other waves until its
        // columns are committed: later items of the same columns wait on them
        // (1-3.5% faster than equal priority); its polls sleep, so a waiting
        // wave does not hold back the one it waits for.
        __builtin_amdgcn_s_setprio(2);
        for (uint32_t spins = 0;; ++spins) {
            bool ready = true;
#pragma unroll
            for (int t = 0; t < kCChunk; ++t)
                if (t < nt && own[t])
                    ready = ready && __hip_atomic_load(&sm.vers[sl[t].c], __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_WORKGROUP) >= rank[t];
            if (__ballot(!ready) == 0ull) break;
            if (spins >= spin_limit) {
                if (lane == 0) atomicOr(&sm.flag, 2);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
#pragma unroll
        for (int t = 0; t < kCChunk; ++t) {
            if (t < nt) {
                if (sl[t].valid) {
#pragma unroll
                    for (int dt = 0; dt < 4; ++dt) {
                        float4* a = &sm.acc[(4 * dt + grp) * kCols + sl[t].c];
                        const float4 w = *a;
                        *a = make_float4(w.x + o[t][dt][0], w.y + o[t][dt][1], w.z + o[t][dt][2], w.w + o[t][dt][3]);
                    }
                }
                if (own[t]) {
                    sm.lsum[sl[t].c] += ol[t][0];
                    if (!(ol[t][0] <= kCGuard)) atomicOr(&sm.flag, 1);
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
#pragma unroll
        for (int t = 0; t < kCChunk; ++t)
            if (t < nt && own[t])
                __hip_atomic_store(&sm.vers[sl[t].c], rank[t] + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        __builtin_amdgcn_s_setprio(0);
    };

    // every wave takes items until none is left
    auto run = [&](int mode) __attribute__((always_inline)) {
        const int n_items = sm.n_items;
        while (true) {
            const int idx = grab();
            if (idx >= n_items) break;
            process(static_cast<int>(sm.items[idx]), mode);
        }
    };

    run(0);
    __syncthreads();
    if (sm.flag & 1) {
        // a block's row sum passed 2^64: a score more than 64 log2-units above
        // the column's reference. Exact maxima (order keys of max(reference,
        // every allowed score)), then the window again against them.
        for (int c = tid; c < kCols; c += kT) reinterpret_cast<uint32_t*>(sm.lsum)[c] = order_key(sm.mref[c]);
        if (tid == 0) sm.next_item = 0;
        __syncthreads();
        run(1);
        __syncthreads();
        for (int c = tid; c < kCols; c += kT) {
            sm.mref[c] = key_to_float(reinterpret_cast<uint32_t*>(sm.lsum)[c]);
            sm.lsum[c] = 0.0f;
            sm.vers[c] = 0;
        }
        {
            // an opaque copy of tid: the addresses are recomputed here rather
            // than kept live (in scratch) from the first clearing
            int i0 = tid;
            asm volatile("" : "+v"(i0));
            for (int i = i0; i < 16 * kCols; i += kT) sm.acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (tid == 0) {
            sm.next_item = 0;
            sm.flag &= ~1;
        }
        __syncthreads();
        run(0);  // the references are now the exact maxima: every P <= 1
        __syncthreads();
    }

    // ---- epilogue: out[b, t, h*64 + d] = O / l, 16-byte stores ----
    // a wait ran out (never expected): the window is poisoned with NaN and
    // the device's status word records it for the host (sparda_status)
    const bool broken = (sm.flag & 2) != 0;
    if (broken && tid == 0) atomicOr(&g_sparda_status, static_cast<uint32_t>(SPARDA_STATUS_PREFILL_WAIT_TIMEOUT));
    int e0 = tid;
    asm volatile("" : "+v"(e0));  // addresses computed here, not carried (in scratch) through the tiles
    for (int e = e0; e < kCols * 8; e += kT) {
        const int c = e / 8, ch = e % 8;
        const int tk = c / R, h = c % R;
        if (tk >= t_valid) continue;
        const float4 a = sm.acc[(2 * ch) * kCols + c];
        const float4 bq = sm.acc[(2 * ch + 1) * kCols + c];
        const float inv = broken ? __builtin_nanf("") : 1.0f / sm.lsum[c];
        bf16x8 w;
        w[0] = static_cast<__bf16>(a.x * inv);
        w[1] = static_cast<__bf16>(a.y * inv);
        w[2] = static_cast<__bf16>(a.z * inv);
        w[3] = static_cast<__bf16>(a.w * inv);
        w[4] = static_cast<__bf16>(bq.x * inv);
        w[5] = static_cast<__bf16>(bq.y * inv);
        w[6] = static_cast<__bf16>(bq.z * inv);
        w[7] = static_cast<__bf16>(bq.w * inv);
        uint16_t* op = out + b * out_sb + (t0 + tk) * out_st + static_cast<int64_t>(g * R + h) * 64 + 8 * ch;
        *reinterpret_cast<uint4*>(op) = __builtin_bit_cast(uint4, w);
    }
}

// window- and block-relative element offsets are 32-bit in the kernel; every
// vector access is 16 bytes
static bool compact_layout_ok(int64_t R, int64_t q_sb, int64_t q_st, int64_t q_sh, int64_t kv_sb, int64_t kv_st,
                              int64_t kv_sh, int64_t out_sb, int64_t out_st, const void* q, const void* k,
                              const void* v, const void* out) {
    auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!al16(q) || !al16(k) || !al16(v) || !al16(out)) return false;
    if ((q_sb % 8) || (q_st % 8) || (q_sh % 8) || (kv_sb % 8) || (kv_st % 8) || (kv_sh % 8)) return false;
    if ((out_sb % 8) || (out_st % 8)) return false;
    if (128 * q_st + R * q_sh + 64 >= (int64_t(1) << 30) || 64 * kv_st + 64 >= (int64_t(1) << 30)) return false;
    return true;
}

// 128-token windows wherever their LDS fits (R <= 3): twice the tokens of a
// 64-token window fill the tiles of each selected block. Measured faster at
// every tested length, with the same output bit for bit (each column's sums do
// not depend on its tile mates).
static int pick_window(int64_t R) { return R <= 3 ? 128 : 64; }

// Polls an ordering wait makes before the workgroup abandons it (the window
// is then NaN and the status word flags it). SPARDA_PREFILL_WAIT_LIMIT
// overrides the default, read once per process: failure-handling tests set
// it to 0 so that any wait not ready at its first poll is abandoned, with
// every wave still finishing its work normally.
static uint32_t wait_limit() {
    static const uint32_t lim = [] {
        const char* e = getenv("SPARDA_PREFILL_WAIT_LIMIT");
        return e != nullptr ? static_cast<uint32_t>(strtoul(e, nullptr, 10)) : kCSpinLimit;
    }();
    return lim;
}

bool prefill_compact_supported(int dtype, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t bs,
                               const int32_t* sel, int64_t cap, int64_t q_sb, int64_t q_st, int64_t q_sh,
                               int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int64_t out_sb, int64_t out_st,
                               const void* q, const void* k, const void* v, const void* out) {
    if (dtype != SPARDA_BF16 || D != 64 || (bs != 64 && bs != 32) || sel == nullptr) return false;
    if (cap < 1 || cap > kCMaxCap || cdiv(T, bs) > kCMaxNB) return false;
    if (Hq % Hkv != 0) return false;
    const int64_t R = Hq / Hkv;
    if (R < 1 || R > 4) return false;
    return compact_layout_ok(R, q_sb, q_st, q_sh, kv_sb, kv_st, kv_sh, out_sb, out_st, q, k, v, out);
}

bool prefill_routed_supported(int dtype, int f_dtype, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t Df,
                              int64_t bs, int64_t ke, int64_t q_sb, int64_t q_st, int64_t q_sh, int64_t kv_sb,
                              int64_t kv_st, int64_t kv_sh, int64_t out_sb, int64_t out_st, const void* q,
                              const void* k, const void* v, const void* out, const float* protos) {
    if (dtype != SPARDA_BF16 || D != 64 || (bs != 64 && bs != 32)) return false;
    if (Df != kCRouteDf || ke < 1 || ke > kCRouteK || (f_dtype != SPARDA_BF16 && f_dtype != SPARDA_F32)) return false;
    if (cdiv(T, bs) > kCMaxNB || (reinterpret_cast<uintptr_t>(protos) & 15u) != 0) return false;
    if (Hq % Hkv != 0) return false;
    const int64_t R = Hq / Hkv;
    if (R < 1 || R > 4) return false;
    return compact_layout_ok(R, q_sb, q_st, q_sh, kv_sb, kv_st, kv_sh, out_sb, out_st, q, k, v, out);
}

template <int FDT>
static int launch_compact(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k, const void* v,
                          int64_t kv_sb, int64_t kv_st, int64_t kv_sh, const int32_t* sel, const int32_t* n_sel,
                          int64_t cap, const CompactRoute& rt, int64_t B, int64_t T, int64_t Hq, int64_t Hkv,
                          int64_t bs, int causal, float scale, void* out, int64_t out_sb, int64_t out_st,
                          hipStream_t stream) {
    const int64_t R = Hq / Hkv;
    const int W = pick_window(R);  // 128, or 64 for R = 4
    const int64_t NBq = cdiv(T, W);  // query windows per (sequence, KV head)
    dim3 grid(static_cast<unsigned>(B * Hkv * NBq));
    const float sl = scale * kCLog2e;
    const uint32_t spin = wait_limit();
#define SPARDA_PC(R_, W_)                                                                                    \
    if (bs == 32) SPARDA_PCB(R_, 32, W_); else SPARDA_PCB(R_, 64, W_)
#define SPARDA_PCB(R_, BS_, W_)                                                                              \
    hipLaunchKernelGGL((prefill_compact_kernel<R_, BS_, FDT, W_>), grid, dim3(kCThreads), 0, stream,          \
                       static_cast<const uint16_t*>(q), q_sb, q_st, q_sh, static_cast<const uint16_t*>(k),    \
                       static_cast<const uint16_t*>(v), kv_sb, kv_st, kv_sh, sel, n_sel, cap, T,              \
                       static_cast<int>(Hkv), NBq, causal, sl, static_cast<uint16_t*>(out), out_sb, out_st, rt, \
                       spin)
    switch (R) {
        case 1: SPARDA_PC(1, 128); break;
        case 2: SPARDA_PC(2, 128); break;
        case 3: SPARDA_PC(3, 128); break;
        default: SPARDA_PC(4, 64); break;
    }
#undef SPARDA_PCB
#undef SPARDA_PC
    return check_hip(hipGetLastError(), "prefill_compact_kernel");
}

int launch_prefill_compact(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k,
                           const void* v, int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                           const int32_t* sel, const int32_t* n_sel, int64_t cap, int64_t B, int64_t T,
                           int64_t Hq, int64_t Hkv, int64_t bs, int causal, float scale, void* out,
                           int64_t out_sb, int64_t out_st, hipStream_t stream) {
    const CompactRoute none{};
    return launch_compact<-1>(q, q_sb, q_st, q_sh, k, v, kv_sb, kv_st, kv_sh, sel, n_sel, cap, none, B, T, Hq, Hkv,
                              bs, causal, scale, out, out_sb, out_st, stream);
}

int launch_prefill_routed(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k, const void* v,
                          int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int f_dtype, const CompactRoute& rt,
                          int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t bs, int causal, float scale,
                          void* out, int64_t out_sb, int64_t out_st, hipStream_t stream) {
    if (f_dtype == SPARDA_F32)
        return launch_compact<SPARDA_F32>(q, q_sb, q_st, q_sh, k, v, kv_sb, kv_st, kv_sh, nullptr, nullptr, 0, rt,
                                          B, T, Hq, Hkv, bs, causal, scale, out, out_sb, out_st, stream);
    return launch_compact<SPARDA_BF16>(q, q_sb, q_st, q_sh, k, v, kv_sb, kv_st, kv_sh, nullptr, nullptr, 0, rt, B,
                                       T, Hq, Hkv, bs, causal, scale, out, out_sb, out_st, stream);
}

__global__ void read_status_kernel(uint32_t* __restrict__ out, int clear) {
    if (threadIdx.x == 0) {
        *out = clear ? atomicExch(&g_sparda_status, 0u) : atomicOr(&g_sparda_status, 0u);
    }
}

int launch_read_status(uint32_t* out, int clear, hipStream_t stream) {
    hipLaunchKernelGGL(read_status_kernel, dim3(1), dim3(kWave), 0, stream, out, clear);
    return check_hip(hipGetLastError(), "read_status_kernel");
}

}  // namespace sparda
