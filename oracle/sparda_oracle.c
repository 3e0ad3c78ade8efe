/*
 * sparda_oracle.c — CPU restatement of the reference's block compressor,
 * forecast scorer, top-k selector and selection-set rules.
 *
 * TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the reference results
 * are compared with. The product (libsparda.so and the Python package) never
 * links or calls it.
 *
 * Arithmetic contract (shared with the HIP kernels so that results are
 * bit-comparable):
 *   prototype = (((0 + k[s0]) + k[s1]) + ... + k[s_last]) / bs   in fp32,
 *               s increasing, division by bs (model/forecast.py:66-77);
 *   score     = fmaf-chain over d starting at 0, then * scale       in fp32
 *               (model/forecast.py:113-118), -inf where causal and
 *               j > (score_pos0 + t) / bs (model/forecast.py:120-126);
 *   top-k     = largest scores first, equal scores (incl. -inf) ordered by
 *               lower block index; -0.0 equals +0.0 (torch.topk at
 *               model/forecast.py:128-129 with its tie order fixed).
 * Build with -ffp-contract=off so the compiler adds no contractions.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* Monotone map from fp32 to uint32: a < b (as floats, no NaN) <=> key(a) < key(b). */
static inline uint32_t order_key(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if (u == 0x80000000u) u = 0; /* -0.0 ties with +0.0 */
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* a ranks before b: larger score, then lower index. */
static inline int ranks_before(uint32_t ka, int32_t ia, uint32_t kb, int32_t ib) {
    return ka > kb || (ka == kb && ia < ib);
}

/* KVBlockCompressor.forward, model/forecast.py:57-78. k is fp32 (bf16 inputs
 * are widened exactly by the caller). out: [B,NB,H,D] contiguous. */
void oracle_compress(const float* k, int64_t B, int64_t S, int64_t H, int64_t D,
                     int64_t sb, int64_t ss, int64_t sh, int64_t bs, float* out) {
    int64_t NB = (S + bs - 1) / bs;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t j = 0; j < NB; ++j)
            for (int64_t h = 0; h < H; ++h)
                for (int64_t d = 0; d < D; ++d) {
                    float acc = 0.0f;
                    int64_t s_end = (j + 1) * bs < S ? (j + 1) * bs : S;
                    for (int64_t s = j * bs; s < s_end; ++s)
                        acc = acc + k[b * sb + s * ss + h * sh + d];
                    out[((b * NB + j) * H + h) * D + d] = acc / (float)bs;
                }
}

/* ForecastBlockSelector scores, model/forecast.py:108-126.
 * f: [B,Tq,H,Df] strides (fsb, fst, fsh, 1); P: [B,NB,H,Df] contiguous;
 * scores: [B,H,Tq,NB] contiguous. */
void oracle_scores(const float* f, int64_t fsb, int64_t fst, int64_t fsh,
                   const float* P, int64_t B, int64_t Tq, int64_t H, int64_t Df,
                   int64_t NB, int64_t bs, int causal, int64_t score_pos0,
                   float scale, float* scores) {
    for (int64_t b = 0; b < B; ++b)
        for (int64_t h = 0; h < H; ++h)
            for (int64_t t = 0; t < Tq; ++t) {
                const float* fr = f + b * fsb + t * fst + h * fsh;
                int64_t limit = (score_pos0 + t) / bs;
                float* out = scores + ((b * H + h) * Tq + t) * NB;
                for (int64_t j = 0; j < NB; ++j) {
                    if (causal && j > limit) {
                        out[j] = -INFINITY;
                        continue;
                    }
                    const float* pr = P + ((b * NB + j) * H + h) * Df;
                    float acc = 0.0f;
                    for (int64_t d = 0; d < Df; ++d) acc = fmaf(fr[d], pr[d], acc);
                    out[j] = acc * scale;
                }
            }
}

/* Canonical top-k of each score row by exhaustive selection (O(NB*k)).
 * scores: [rows, NB]; out: [rows, min(k, NB)]. */
void oracle_topk(const float* scores, int64_t rows, int64_t NB, int64_t k,
                 int32_t* out) {
    int64_t ke = k < NB ? k : NB;
    unsigned char used[1 << 16];
    for (int64_t r = 0; r < rows; ++r) {
        const float* row = scores + r * NB;
        memset(used, 0, (size_t)NB);
        for (int64_t i = 0; i < ke; ++i) {
            int32_t best = -1;
            uint32_t bk = 0;
            for (int64_t j = 0; j < NB; ++j) {
                if (used[j]) continue;
                uint32_t kj = order_key(row[j]);
                if (best < 0 || ranks_before(kj, (int32_t)j, bk, best)) {
                    best = (int32_t)j;
                    bk = kj;
                }
            }
            used[best] = 1;
            out[r * ke + i] = best;
        }
    }
}

/* Selection set of one query row: ({0, own} U topk) restricted to <= own when
 * causal, ascending, unique, -1 padded. Mirrors the allowed-block rule of the
 * prefill (model/attention/sparse.py:231-253) and the decode selection
 * (model/attention/sparse.py:126-154).
 * topk: [rows, ke]; own: [rows]; sel: [rows, cap]; n_sel: [rows]. */
void oracle_sel_from_topk(const int32_t* topk, int64_t rows, int64_t ke,
                          const int64_t* own, int causal, int64_t cap,
                          int32_t* sel, int32_t* n_sel) {
    for (int64_t r = 0; r < rows; ++r) {
        int32_t buf[512];
        int64_t n = 0;
        int64_t o = own[r];
        buf[n++] = 0;
        buf[n++] = (int32_t)o;
        for (int64_t i = 0; i < ke; ++i) buf[n++] = topk[r * ke + i];
        /* insertion sort ascending */
        for (int64_t i = 1; i < n; ++i) {
            int32_t v = buf[i];
            int64_t p = i - 1;
            while (p >= 0 && buf[p] > v) { buf[p + 1] = buf[p]; --p; }
            buf[p + 1] = v;
        }
        int64_t m = 0;
        for (int64_t i = 0; i < n; ++i) {
            if (causal && buf[i] > o) continue;
            if (m > 0 && sel[r * cap + m - 1] == buf[i]) continue;
            sel[r * cap + m++] = buf[i];
        }
        n_sel[r] = (int32_t)m;
        for (int64_t i = m; i < cap; ++i) sel[r * cap + i] = -1;
    }
}
