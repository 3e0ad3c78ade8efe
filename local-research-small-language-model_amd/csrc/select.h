// Device-side selection helpers shared by the router and the decode step:
// per-lane top-k insertion lists, workgroup top-k, selection-list emission.
#pragma once

#include "common.h"

namespace sparda {

// ---------------------------------------------------------------------------
// per-lane top-k list: ranks sorted descending in registers. Slots >= ke hold
// UINT64_MAX so an inserted rank can never displace them; the rank falling off
// slot ke-1 is carried out and dropped.
// ---------------------------------------------------------------------------
template <int KMAX>
struct LaneTopK {
    uint64_t r[KMAX];
    uint64_t thr;  // rank at slot ke-1 (0 while the list is not full)
    int ke;

    __device__ __forceinline__ void init(int ke_) {
        ke = ke_;
#pragma unroll
        for (int i = 0; i < KMAX; ++i) r[i] = i < ke ? 0ull : ~0ull;
        thr = 0;
    }
    __device__ __forceinline__ void push(uint64_t x) {
        if (x > thr) {
#pragma unroll
            for (int i = 0; i < KMAX; ++i) {
                const uint64_t cur = r[i];
                const bool sw = x > cur;
                r[i] = sw ? x : cur;
                x = sw ? cur : x;
            }
            uint64_t t = 0;
#pragma unroll
            for (int i = 0; i < KMAX; ++i) t = (i == ke - 1) ? r[i] : t;
            thr = t;
        }
    }
};

// ---------------------------------------------------------------------------
// route keys: a (score, index) pair as a non-negative double whose bit pattern
// holds order_key(score) in bits 62..31 and 0x7FFFFFFF - index in bits 30..0.
// A larger key is a larger score, equal scores the lower index. Non-negative
// doubles order exactly as their bit patterns, so a compare-exchange of two
// keys is one max and one min. Key 0 (+0.0) marks an empty slot; every real
// key is above it. order_key is capped at 0xFFDFFFFF so that no key is a NaN
// (only NaN scores whose two top mantissa bits are set reach the cap).
// ---------------------------------------------------------------------------
__device__ __forceinline__ double route_key(float s, int32_t idx) {
    uint32_t ok = order_key(s);
    ok = ok < 0xFFDFFFFFu ? ok : 0xFFDFFFFFu;
    const uint32_t lo = (ok << 31) | (0x7FFFFFFFu - static_cast<uint32_t>(idx));
    return __hiloint2double(static_cast<int>(ok >> 1), static_cast<int>(lo));
}
__device__ __forceinline__ int32_t route_key_index(double k) {
    return static_cast<int32_t>(0x7FFFFFFFu - (static_cast<uint32_t>(__double2loint(k)) & 0x7FFFFFFFu));
}

// max / min of two route keys. Keys are never NaN, so the quieting of inputs
// that IEEE-mode maxnum would add is not needed: issue the instructions as is.
__device__ __forceinline__ double key_max(double a, double b) {
    double r;
    asm("v_max_f64 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ double key_min(double a, double b) {
    double r;
    asm("v_min_f64 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// per-lane list of the KMAX largest route keys, descending
template <int KMAX>
struct KeyTopK {
    double r[KMAX];

    __device__ __forceinline__ void init() {
#pragma unroll
        for (int i = 0; i < KMAX; ++i) r[i] = 0.0;
    }
    __device__ __forceinline__ void push(double x) {
#pragma unroll
        for (int i = 0; i < KMAX; ++i) {
            const double lo = key_min(r[i], x);
            asm("v_max_f64 %0, %0, %1" : "+v"(r[i]) : "v"(x));
            x = lo;
        }
    }
    // r <- the KMAX largest of r and o (both descending): bitonic merge
    __device__ __forceinline__ void merge(const double (&o)[KMAX]) {
        static_assert((KMAX & (KMAX - 1)) == 0, "KMAX must be a power of two");
#pragma unroll
        for (int i = 0; i < KMAX; ++i) r[i] = key_max(r[i], o[KMAX - 1 - i]);
#pragma unroll
        for (int s = KMAX / 2; s > 0; s >>= 1) {
#pragma unroll
            for (int i = 0; i < KMAX; ++i) {
                if ((i & s) == 0) {
                    const double a = r[i], c = r[i + s];
                    r[i] = key_max(a, c);
                    r[i + s] = key_min(a, c);
                }
            }
        }
    }
};

// Sorted, de-duplicated selection list ({0, own} U picks, restricted to <= own
// when causal) written to sel[0..cap), count to *n_out.
template <int N>
__device__ __forceinline__ void emit_selection(int32_t (&c)[N], int own, bool causal,
                                               int32_t* __restrict__ sel, int cap,
                                               int32_t* __restrict__ n_out) {
    constexpr int32_t kNone = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (c[i] < 0 || (causal && c[i] > own)) c[i] = kNone;
    // odd-even transposition sort, ascending
#pragma unroll
    for (int pass = 0; pass < N; ++pass) {
#pragma unroll
        for (int i = pass & 1; i + 1 < N; i += 2) {
            const int32_t a = c[i], bb = c[i + 1];
            c[i] = a < bb ? a : bb;
            c[i + 1] = a < bb ? bb : a;
        }
    }
    int m = 0;
    int32_t last = -1;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        if (c[i] != kNone && c[i] != last) {
            sel[m] = c[i];
            ++m;
            last = c[i];
        }
    }
    for (int i = m; i < cap; ++i) sel[i] = -1;
    *n_out = m;
}

// ---------------------------------------------------------------------------
// workgroup-level top-k over `n` ranks held in LDS (consumed: taken entries
// are zeroed). ke rounds of workgroup arg-max built on wavefront reductions.
// All threads of the workgroup must call it.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void wg_topk(uint64_t* ranks, int n, int ke, int32_t* out_lds, uint64_t* wave_best) {
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int nwaves = (blockDim.x + kWave - 1) / kWave;
    for (int i = 0; i < ke; ++i) {
        uint64_t m = 0;
        for (int j = threadIdx.x; j < n; j += blockDim.x) m = ranks[j] > m ? ranks[j] : m;
        m = wave_max_u64(m);
        if (lane == 0) wave_best[wave] = m;
        __syncthreads();
        if (threadIdx.x == 0) {
            uint64_t w = 0;
            for (int q = 0; q < nwaves; ++q) w = wave_best[q] > w ? wave_best[q] : w;
            const int32_t idx = rank64_index(w);
            out_lds[i] = idx;
            ranks[idx] = 0;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Wavefront top-k selection by ballot threshold search.
// The wave holds keys[j] (orderable score keys, index = block) for
// j = e*64 + lane in kreg[e]; slots j >= n must hold key 0, which no
// threshold counts (every score, -inf included, has a key >= 0x007FFFFF).
// Writes to sel_lds the ascending list ({0, own} U topk) restricted to blocks
// <= own, returns its length. topk = the k largest keys, equal keys by lower
// index; n >= k. Called by a whole wavefront; control flow is wave-uniform.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int ballot_count(bool p) {
    return __builtin_popcountll(__builtin_amdgcn_ballot_w64(p));
}

template <int CH>
__device__ __forceinline__ int wave_select(const uint32_t (&kreg)[CH], int n, int k, int own,
                                           int32_t* sel_lds) {
    const int lane = threadIdx.x % kWave;
    // T = the k-th largest key: the largest T with count(key >= T) >= k,
    // one bit per round (a compare and a popcount per key register)
    uint32_t T = 0;
#pragma unroll 4
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t c = T | (1u << bit);
        int cnt = 0;
#pragma unroll
        for (int e = 0; e < CH; ++e) cnt += ballot_count(kreg[e] >= c);
        T = cnt >= k ? c : T;
    }
    int above = 0;
#pragma unroll
    for (int e = 0; e < CH; ++e) above += ballot_count(kreg[e] > T);
    int need_eq = k - above;  // keys equal to T, taken in index order
    const uint64_t lanes_below = (1ull << lane) - 1ull;
    int m = 0;
#pragma unroll
    for (int e = 0; e < CH; ++e) {
        const int j = e * kWave + lane;
        const bool in = j < n;
        const uint64_t gt = __builtin_amdgcn_ballot_w64(kreg[e] > T);
        uint64_t eq = __builtin_amdgcn_ballot_w64(kreg[e] == T);
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

// The k-th largest of one key per lane (keys of empty lanes 0): the largest
// T with count(v >= T) >= k, two bits per round (the three candidate counts
// of a round are independent ballots, so a round costs little more than one).
__device__ __forceinline__ uint32_t wave_kth_largest(uint32_t v, int k) {
    uint32_t T = 0;
#pragma unroll 4
    for (int bit = 30; bit >= 0; bit -= 2) {
        const uint32_t c1 = T | (1u << bit), c2 = T | (2u << bit), c3 = T | (3u << bit);
        const int n1 = ballot_count(v >= c1), n2 = ballot_count(v >= c2), n3 = ballot_count(v >= c3);
        T = n3 >= k ? c3 : (n2 >= k ? c2 : (n1 >= k ? c1 : T));
    }
    return T;
}

// wave_select with a candidate pre-filter. A lower bound T0 of the k-th
// largest key (at least k keys are >= T0) confines the top-k to the keys
// >= T0: the minimum of G >= k group maxima, or, when that admits more than
// 64 keys, the k-th largest of the 64 lane maxima (the k lanes whose maximum
// is >= T0 hold k keys >= T0; the keys fill lanes 0.. first, so at least
// min(n, 64) >= k lanes hold one). When the keys >= T0 fit in one register
// per lane they are compacted in index order through ck_lds / ci_lds (64
// entries each) and ranked against each other (C lane reads instead of the
// threshold search's 32 ballot rounds over CH key registers, ~40 cycles per
// register per round). Otherwise wave_select runs as is. Same result as
// wave_select; called by a whole wavefront (wave-uniform flow).
template <int CH>
__device__ __forceinline__ int wave_select_pre(const uint32_t (&kreg)[CH], int n, int k, int own,
                                               int32_t* sel_lds, uint32_t* ck_lds, int32_t* ci_lds) {
    const int lane = threadIdx.x % kWave;
    uint32_t lm = kreg[0];
#pragma unroll
    for (int e = 1; e < CH; ++e) lm = kreg[e] > lm ? kreg[e] : lm;
    // First a cheaper bound: the lanes form G >= k groups (G a power of two),
    // and the smallest of the G group maxima has at least G >= k keys at or
    // above it (one per group). Six lane exchanges instead of a search.
    int G = 1;
    while (G < k && G < kWave) G <<= 1;
    const int gs = kWave / G;
    uint32_t gm = lm;
    for (int o = 1; o < gs; o <<= 1) {
        const uint32_t x = static_cast<uint32_t>(__shfl_xor(static_cast<int>(gm), o, kWave));
        gm = x > gm ? x : gm;
    }
    for (int o = gs; o < kWave; o <<= 1) {
        const uint32_t x = static_cast<uint32_t>(__shfl_xor(static_cast<int>(gm), o, kWave));
        gm = x < gm ? x : gm;
    }
    uint32_t T0 = __builtin_amdgcn_readfirstlane(gm);
    int C = 0;
#pragma unroll
    for (int e = 0; e < CH; ++e) C += ballot_count(kreg[e] >= T0);
    if (C > kWave) {
        // too many keys at or above it: the k-th largest lane maximum
        T0 = wave_kth_largest(lm, k);
        C = 0;
#pragma unroll
        for (int e = 0; e < CH; ++e) C += ballot_count(kreg[e] >= T0);
    }
    if (C > kWave) return wave_select<CH>(kreg, n, k, own, sel_lds);
    const uint64_t lanes_below = (1ull << lane) - 1ull;
    int base = 0;
#pragma unroll
    for (int e = 0; e < CH; ++e) {
        const uint64_t msk = __builtin_amdgcn_ballot_w64(kreg[e] >= T0);
        if ((msk >> lane) & 1ull) {
            const int slot = base + __popcll(msk & lanes_below);
            ck_lds[slot] = kreg[e];
            ci_lds[slot] = e * kWave + lane;
        }
        base += __popcll(msk);
    }
    __builtin_amdgcn_wave_barrier();  // LDS operations of one wavefront complete in order
    const uint32_t ck = lane < C ? ck_lds[lane] : 0u;
    const int ci = lane < C ? ci_lds[lane] : 0x7fffffff;
    // the candidates' ranks (keys above, equal keys at lower index: lanes are
    // in index order); the top k are the ranks below k
    int rank = 0;
    for (int j = 0; j < C; ++j) {
        const uint32_t kj = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(ck), j));
        rank += (kj > ck || (kj == ck && j < lane)) ? 1 : 0;
    }
    // candidates are in ascending index order, all <= own when taken: the
    // sink block 0 goes first and the own block last unless already taken
    const uint64_t take = __builtin_amdgcn_ballot_w64(lane < C && rank < k) & __builtin_amdgcn_ballot_w64(ci <= own);
    const bool mine = (take >> lane) & 1ull;
    const bool has0 = __builtin_amdgcn_ballot_w64(mine && ci == 0) != 0;
    const bool has_own = __builtin_amdgcn_ballot_w64(mine && ci == own) != 0;
    int m = 0;
    if (!has0) {
        if (lane == 0) sel_lds[0] = 0;
        m = 1;
    }
    if (mine) sel_lds[m + __popcll(take & lanes_below)] = ci;
    m += __popcll(take);
    if (!has_own && own != 0 && own < n) {
        if (lane == 0) sel_lds[m] = own;
        m += 1;
    }
    return m;
}

// Decode score of one block from its fp32 sum: p = sum / bs, then the
// canonical fma chain over d (f . p, d ascending), times scale. BATCH 16-byte
// loads are issued before the part of the chain that consumes them (all DH/4
// by default). For a power-of-two bs, sum * (1/bs) is the same correctly
// rounded value as sum / bs (the reciprocal is exact), at the cost of one
// multiply.
template <int DH, bool POW2, int BATCH = DH / 4>
__device__ __forceinline__ float score_from_sum(const float* __restrict__ sum, const float* f_lds, float den,
                                                float inv, float scale) {
    static_assert((DH / 4) % BATCH == 0, "BATCH must divide DH/4");
    const float4* p = reinterpret_cast<const float4*>(sum);
    float acc = 0.0f;
#pragma unroll
    for (int c0 = 0; c0 < DH / 4; c0 += BATCH) {
        float4 v[BATCH];
#pragma unroll
        for (int c = 0; c < BATCH; ++c) v[c] = p[c0 + c];
#pragma unroll
        for (int c = 0; c < BATCH; ++c) {
            const float x[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
            for (int e = 0; e < 4; ++e)
                acc = __fmaf_rn(f_lds[4 * (c0 + c) + e], POW2 ? x[e] * inv : x[e] / den, acc);
        }
    }
    return acc * scale;
}

// top-k selection over the first n keys of key_lds, CH keys per lane
template <int CH>
__device__ __forceinline__ int select_keys(const uint32_t* key_lds, int n, int k, int own, int32_t* sel_lds,
                                           int lane, uint32_t* ck_lds, int32_t* ci_lds) {
    uint32_t kreg[CH];
#pragma unroll
    for (int e = 0; e < CH; ++e) {
        const int j = e * kWave + lane;
        kreg[e] = j < n ? key_lds[j] : 0u;
    }
    return wave_select_pre<CH>(kreg, n, k, own, sel_lds, ck_lds, ci_lds);
}

// select_keys with the smallest key-register count (4, 8, 16 or 64, at most
// CHMAX) holding n keys: a length known only on the device may be far below
// the bound CHMAX was chosen for
template <int CHMAX>
__device__ __forceinline__ int select_keys_upto(const uint32_t* key_lds, int n, int k, int own, int32_t* sel_lds,
                                                int lane, uint32_t* ck_lds, int32_t* ci_lds) {
    if (CHMAX >= 64 && n > 1024)
        return select_keys<(CHMAX >= 64 ? 64 : CHMAX)>(key_lds, n, k, own, sel_lds, lane, ck_lds, ci_lds);
    if (CHMAX >= 16 && n > 512)
        return select_keys<(CHMAX >= 16 ? 16 : CHMAX)>(key_lds, n, k, own, sel_lds, lane, ck_lds, ci_lds);
    if (CHMAX >= 8 && n > 256)
        return select_keys<(CHMAX >= 8 ? 8 : CHMAX)>(key_lds, n, k, own, sel_lds, lane, ck_lds, ci_lds);
    return select_keys<4>(key_lds, n, k, own, sel_lds, lane, ck_lds, ci_lds);
}

}  // namespace sparda
