// Block compressor, forecast router (score + top-k + selection list), the
// stand-alone top-k stage, forecast-free selections and the block gather.
//
// Arithmetic contract (bit-exact with the oracle):
//   prototype = sequential fp32 sum over the block's tokens, then / bs
//   score     = fma chain over d starting at 0, then * scale
//   top-k     = larger score first, equal scores by lower block index
#pragma clang fp contract(off)

#include "chunk.h"
#include "common.h"
#include "kernels.h"
#include "select.h"
#include "route_rows.h"

namespace sparda {

// ---------------------------------------------------------------------------
// compressor: grid (NB, B, ceil(H/heads_per_wg)), block = heads_per_wg*D/VEC.
// Thread (h, d-group) walks the block's tokens in order, one VEC-wide load per
// token; a wavefront reads a contiguous run of the token row.
// ---------------------------------------------------------------------------
template <int DT, int VEC, int UNROLL>
__global__ void __launch_bounds__(256)
compress_kernel(const void* __restrict__ k, int64_t S, int H, int D,
                int64_t sb, int64_t ss, int64_t sh, int bs, int heads_per_wg,
                float* __restrict__ protos, int64_t NB) {
    const int j = blockIdx.x;
    const int b = blockIdx.y;
    const int groups = D / VEC;
    const int h = blockIdx.z * heads_per_wg + threadIdx.x / groups;
    const int d = (threadIdx.x % groups) * VEC;
    if (h >= H) return;
    const int64_t s0 = static_cast<int64_t>(j) * bs;
    const int64_t s1 = s0 + bs < S ? s0 + bs : S;
    float acc[VEC];
    block_sum<DT, VEC, UNROLL>(k, b * sb + h * sh + d, s0, s1, ss, acc);
    float* out = protos + ((static_cast<int64_t>(b) * NB + j) * H + h) * D + d;
    const float den = static_cast<float>(bs);
#pragma unroll
    for (int v = 0; v < VEC; ++v) out[v] = acc[v] / den;
}

int launch_compress(const void* k, int dtype, int64_t B, int64_t S, int64_t H, int64_t D,
                    int64_t sb, int64_t ss, int64_t sh, int64_t bs, float* protos,
                    hipStream_t stream) {
    const int64_t NB = cdiv(S, bs);
    const bool aligned = (D % 2 == 0) && (sb % 2 == 0) && (ss % 2 == 0) && (sh % 2 == 0) &&
                         (reinterpret_cast<uintptr_t>(k) % (dtype == SPARDA_F32 ? 8 : 4) == 0);
    const int vec = aligned ? 2 : 1;
    const int groups = static_cast<int>(D / vec);
    int hpw = static_cast<int>(256 / groups);
    if (hpw < 1) hpw = 1;
    if (groups > 256) return set_error(SPARDA_ERR_SHAPE, "compress: D/VEC > 256");
    if (hpw > H) hpw = static_cast<int>(H);
    dim3 grid(static_cast<unsigned>(NB), static_cast<unsigned>(B), static_cast<unsigned>(cdiv(H, hpw)));
    dim3 block(static_cast<unsigned>(groups * hpw));
#define SPARDA_COMPRESS(DT_, V_, U_)                                                      \
    hipLaunchKernelGGL((compress_kernel<DT_, V_, U_>), grid, block, 0, stream, k, S,      \
                       static_cast<int>(H), static_cast<int>(D), sb, ss, sh,              \
                       static_cast<int>(bs), hpw, protos, NB)
#define SPARDA_COMPRESS_U(DT_, V_)                                                        \
    if (bs == 64) SPARDA_COMPRESS(DT_, V_, 64);                                           \
    else if (bs == 32) SPARDA_COMPRESS(DT_, V_, 32);                                      \
    else SPARDA_COMPRESS(DT_, V_, 0);
    if (dtype == SPARDA_F32) {
        if (vec == 2) { SPARDA_COMPRESS_U(SPARDA_F32, 2) } else { SPARDA_COMPRESS_U(SPARDA_F32, 1) }
    } else {
        if (vec == 2) { SPARDA_COMPRESS_U(SPARDA_BF16, 2) } else { SPARDA_COMPRESS_U(SPARDA_BF16, 1) }
    }
#undef SPARDA_COMPRESS_U
#undef SPARDA_COMPRESS
    return check_hip(hipGetLastError(), "compress_kernel");
}

// ---------------------------------------------------------------------------
// router: one lane per query row. Under the causal mask a workgroup of
// kRouteWaves wavefronts takes two sets of 64 consecutive rows of one (b, h):
// set p and its mirror NS-1-p, so that every workgroup scores about the same
// number of (row, block) pairs; without it every set has the same work and a
// workgroup takes one (twice the workgroups, four wavefronts per SIMD instead
// of two at B=1, T=16384). Within a set the waves split the candidate blocks
// (wave w scores the blocks j = w mod kRouteWaves), so the block index is
// uniform across the wavefront: every 16-lane row of the wavefront loads the
// block's prototype with one coalesced load (lane i of the row holds elements
// E*i .. E*i+E-1, E = DF/16), one block ahead of its use, and the fma chain
// takes element d from lane d/E of the row through a DPP row broadcast. Every
// lane keeps a descending list of route keys; after a set the waves' lists are
// merged through LDS by one wave (rotating with the set), which writes the
// rows' outputs.
// ---------------------------------------------------------------------------
template <int FDT, int DF, int KMAX>
__global__ void __launch_bounds__(kRouteThreads)
route_rows_kernel(const void* __restrict__ f, int64_t fsb, int64_t fst, int64_t fsh,
                  const float* __restrict__ protos, int64_t Tq, int H, int64_t NB, int bs,
                  int ke, int causal, int64_t score_pos0, int64_t query_pos0, float scale,
                  int32_t* __restrict__ topk, float* __restrict__ scores,
                  int32_t* __restrict__ sel, int32_t* __restrict__ n_sel, int cap) {
    extern __shared__ double lists[];  // [kRouteWaves][KMAX][kWave]
    const int lane = threadIdx.x % kWave;
    const int h = blockIdx.y;
    const int b = blockIdx.z;
    const int64_t NS = cdiv(Tq, kWave);
    const int64_t pair = blockIdx.x;

    for (int pass = 0; pass < 2; ++pass) {
        const int64_t set = pass == 0 ? pair : NS - 1 - pair;
        if (pass == 1 && (!causal || set == pair)) break;  // one set without the mask; an odd count's middle set
        const int m = static_cast<int>((2 * pair + pass) % kRouteWaves);
        int32_t picks[KMAX];
        if (!route_set<FDT, DF, KMAX>(f, fsb, fst, fsh, protos, b, h, H, set, Tq, NB, bs, ke, causal, score_pos0,
                                      scale, scores, m, lists, picks))
            continue;
        const int64_t t = set * kWave + lane;
        if (t >= Tq) continue;
        const int64_t row = (static_cast<int64_t>(b) * H + h) * Tq + t;
        if (topk) {
            int32_t* tr = topk + row * ke;
#pragma unroll
            for (int i = 0; i < KMAX; ++i)
                if (i < ke) tr[i] = picks[i];
        }
        if (sel) {
            int64_t own = (query_pos0 + t) / bs;
            if (own > NB - 1) own = NB - 1;
            int32_t c[KMAX + 2];
            c[0] = 0;
            c[1] = static_cast<int32_t>(own);
#pragma unroll
            for (int i = 0; i < KMAX; ++i) c[i + 2] = picks[i];
            emit_selection(c, static_cast<int>(own), causal != 0, sel + row * cap, cap, n_sel + row);
        }
    }
}

template <int FDT, int DF>
static int launch_route_df(const void* f, int64_t fsb, int64_t fst, int64_t fsh, const float* protos,
                           int64_t B, int64_t Tq, int64_t H, int64_t NB, int64_t bs, int ke,
                           int causal, int64_t score_pos0, int64_t query_pos0, float scale,
                           int32_t* topk, float* scores, int32_t* sel, int32_t* n_sel, int cap,
                           hipStream_t stream) {
    const int64_t pairs = causal ? cdiv(cdiv(Tq, kWave), 2) : cdiv(Tq, kWave);
    dim3 grid(static_cast<unsigned>(pairs), static_cast<unsigned>(H), static_cast<unsigned>(B));
#define SPARDA_ROUTE(KM_)                                                                          \
    hipLaunchKernelGGL((route_rows_kernel<FDT, DF, KM_>), grid, dim3(kRouteThreads),               \
                       static_cast<size_t>(kRouteWaves) * KM_ * kWave * sizeof(double), stream,    \
                       f, fsb, fst, fsh, protos, Tq, static_cast<int>(H), NB,                      \
                       static_cast<int>(bs), ke, causal, score_pos0, query_pos0, scale,            \
                       topk, scores, sel, n_sel, cap)
    if (ke <= 8) { SPARDA_ROUTE(8); }
    else if (ke <= 16) { SPARDA_ROUTE(16); }
    else { SPARDA_ROUTE(32); }
#undef SPARDA_ROUTE
    return check_hip(hipGetLastError(), "route_rows_kernel");
}

int launch_route(const void* f, int fdtype, int64_t fsb, int64_t fst, int64_t fsh,
                 const float* protos, int64_t B, int64_t Tq, int64_t H, int64_t Df, int64_t NB,
                 int64_t bs, int ke, int causal, int64_t score_pos0, int64_t query_pos0,
                 float scale, int32_t* topk, float* scores, int32_t* sel, int32_t* n_sel,
                 int cap, hipStream_t stream) {
#define SPARDA_DF(FDT_, DF_)                                                                   \
    return launch_route_df<FDT_, DF_>(f, fsb, fst, fsh, protos, B, Tq, H, NB, bs, ke, causal,  \
                                      score_pos0, query_pos0, scale, topk, scores, sel, n_sel, \
                                      cap, stream)
    if (fdtype == SPARDA_F32) {
        switch (Df) {
            case 16: SPARDA_DF(SPARDA_F32, 16);
            case 32: SPARDA_DF(SPARDA_F32, 32);
            case 64: SPARDA_DF(SPARDA_F32, 64);
            case 128: SPARDA_DF(SPARDA_F32, 128);
        }
    } else {
        switch (Df) {
            case 16: SPARDA_DF(SPARDA_BF16, 16);
            case 32: SPARDA_DF(SPARDA_BF16, 32);
            case 64: SPARDA_DF(SPARDA_BF16, 64);
            case 128: SPARDA_DF(SPARDA_BF16, 128);
        }
    }
#undef SPARDA_DF
    return set_error(SPARDA_ERR_SHAPE, "route: forecast dim %lld not in {16,32,64,128}",
                     static_cast<long long>(Df));
}

// one workgroup per row; ranks of the row staged in LDS
constexpr int kWaveTopkThreads = 256;

__global__ void __launch_bounds__(kWaveTopkThreads)
topk_wave_kernel(const float* __restrict__ scores, int64_t NB, int ke, int32_t* __restrict__ topk) {
    extern __shared__ uint64_t ranks[];
    __shared__ uint64_t wave_best[kWaveTopkThreads / kWave];
    __shared__ int32_t picks[64];
    const int64_t row = blockIdx.x;
    const float* s = scores + row * NB;
    for (int j = threadIdx.x; j < NB; j += blockDim.x) ranks[j] = rank64(s[j], j);
    __syncthreads();
    wg_topk(ranks, static_cast<int>(NB), ke, picks, wave_best);
    for (int i = threadIdx.x; i < ke; i += blockDim.x) topk[row * ke + i] = picks[i];
}

// one lane per row (scores read from global)
template <int KMAX>
__global__ void __launch_bounds__(64)
topk_rows_kernel(const float* __restrict__ scores, int64_t rows, int64_t NB, int ke,
                 int32_t* __restrict__ topk) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
    if (row >= rows) return;
    const float* s = scores + row * NB;
    LaneTopK<KMAX> best;
    best.init(ke);
    for (int64_t j = 0; j < NB; ++j) best.push(rank64(s[j], static_cast<int32_t>(j)));
#pragma unroll
    for (int i = 0; i < KMAX; ++i)
        if (i < ke) topk[row * ke + i] = rank64_index(best.r[i]);
}

int launch_topk_scores(const float* scores, int64_t rows, int64_t NB, int ke, int algo,
                       int32_t* topk, hipStream_t stream) {
    if (algo == SPARDA_TOPK_AUTO) algo = (rows < 2048 && NB >= 128 && NB <= 4096) ? SPARDA_TOPK_WAVE : SPARDA_TOPK_ROWS;
    if (algo == SPARDA_TOPK_WAVE) {
        hipLaunchKernelGGL(topk_wave_kernel, dim3(static_cast<unsigned>(rows)), dim3(kWaveTopkThreads),
                           static_cast<size_t>(NB) * sizeof(uint64_t), stream, scores, NB, ke, topk);
        return check_hip(hipGetLastError(), "topk_wave_kernel");
    }
    dim3 grid(static_cast<unsigned>(cdiv(rows, 64)));
    if (ke <= 8)
        hipLaunchKernelGGL((topk_rows_kernel<8>), grid, dim3(64), 0, stream, scores, rows, NB, ke, topk);
    else if (ke <= 16)
        hipLaunchKernelGGL((topk_rows_kernel<16>), grid, dim3(64), 0, stream, scores, rows, NB, ke, topk);
    else
        hipLaunchKernelGGL((topk_rows_kernel<32>), grid, dim3(64), 0, stream, scores, rows, NB, ke, topk);
    return check_hip(hipGetLastError(), "topk_rows_kernel");
}

// ---------------------------------------------------------------------------
// forecast-free selection lists, one thread per (b,h,t) row
// ---------------------------------------------------------------------------
__global__ void select_fixed_kernel(int mode, int64_t rows, int64_t Tq, int64_t NB, int bs, int k,
                                    int64_t query_pos0, int32_t* __restrict__ sel,
                                    int32_t* __restrict__ n_sel, int cap) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const int64_t t = row % Tq;
    int64_t own = (query_pos0 + t) / bs;
    if (own > NB - 1) own = NB - 1;
    int32_t* out = sel + row * cap;
    int m = 0;
    if (mode == SPARDA_SEL_DENSE) {
        for (int64_t j = 0; j <= own; ++j) out[m++] = static_cast<int32_t>(j);
    } else {
        const int64_t width = (mode == SPARDA_SEL_WINDOW_DECODE) ? k : k + 1;
        int64_t lo = own - width + 1;
        if (lo < 0) lo = 0;
        if (lo > 0) out[m++] = 0;
        for (int64_t j = lo; j <= own; ++j) out[m++] = static_cast<int32_t>(j);
    }
    for (int i = m; i < cap; ++i) out[i] = -1;
    n_sel[row] = m;
}

int launch_select_fixed(int mode, int64_t B, int64_t Tq, int64_t H, int64_t NB, int64_t bs, int64_t k,
                        int64_t query_pos0, int32_t* sel, int32_t* n_sel, int cap, hipStream_t stream) {
    const int64_t rows = B * H * Tq;
    hipLaunchKernelGGL(select_fixed_kernel, dim3(static_cast<unsigned>(cdiv(rows, 256))), dim3(256), 0,
                       stream, mode, rows, Tq, NB, static_cast<int>(bs), static_cast<int>(k), query_pos0,
                       sel, n_sel, cap);
    return check_hip(hipGetLastError(), "select_fixed_kernel");
}

// ---------------------------------------------------------------------------
// chunked-gather lists (model/attention/sparse.py:303-333): one workgroup per
// (query block bq, head h, sequence b) builds the block's list (chunk.h) and
// writes it to every row of the block (cap entries, -1 padded).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
chunk_select_kernel(const int32_t* __restrict__ topk, int ke, int64_t T, int H, int bs, int64_t NB, int k, int cut,
                    int cap, int32_t* __restrict__ sel, int32_t* __restrict__ n_sel) {
    __shared__ ChunkLds c;
    const int bq = blockIdx.x;
    const int h = blockIdx.y;
    const int b = blockIdx.z;
    const int64_t r0 = static_cast<int64_t>(bq) * bs;
    const int64_t r1 = r0 + bs < T ? r0 + bs : T;
    const int64_t row0 = (static_cast<int64_t>(b) * H + h) * T + r0;
    chunk_list(c, topk != nullptr ? topk + row0 * ke : nullptr, r1 - r0, ke, bq, k, NB, cut);
    chunk_write(c, row0, r1 - r0, cap, sel, n_sel);
}

int launch_chunk_select(const int32_t* topk, int64_t ke, int64_t B, int64_t H, int64_t T, int64_t bs, int64_t k,
                        int32_t* sel, int32_t* n_sel, int64_t cap, hipStream_t stream) {
    const int64_t NB = cdiv(T, bs);
    if (NB > kChunkMaxNB) return set_error(SPARDA_ERR_SHAPE, "select_chunked: more than %d blocks", kChunkMaxNB);
    const int64_t cut = NB < k + 2 ? NB : k + 2;
    if (cut > cap || cap > kMaxSelCap)
        return set_error(SPARDA_ERR_SHAPE, "select_chunked: sel_cap %lld outside [%lld, %d]", (long long)cap,
                         (long long)cut, kMaxSelCap);
    hipLaunchKernelGGL(chunk_select_kernel, dim3(static_cast<unsigned>(NB), static_cast<unsigned>(H),
                       static_cast<unsigned>(B)), dim3(256), 0, stream, topk, static_cast<int>(ke), T,
                       static_cast<int>(H), static_cast<int>(bs), NB, static_cast<int>(k), static_cast<int>(cut),
                       static_cast<int>(cap), sel, n_sel);
    return check_hip(hipGetLastError(), "chunk_select_kernel");
}

// ---------------------------------------------------------------------------
// gather: grid (n, H, B); each workgroup copies one block of K and of V
// ---------------------------------------------------------------------------
template <int DT>
__global__ void gather_kernel(const void* __restrict__ k, const void* __restrict__ v, int64_t sb,
                              int64_t sh, int64_t ss, const int32_t* __restrict__ idx, int64_t S,
                              int D, int64_t n, int bs, void* __restrict__ ko, void* __restrict__ vo) {
    const int i = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int H = gridDim.y;
    const int64_t j = idx[(static_cast<int64_t>(b) * H + h) * n + i];
    const int64_t obase = ((static_cast<int64_t>(b) * H + h) * n + i) * bs * D;
    for (int e = threadIdx.x; e < bs * D; e += blockDim.x) {
        const int r = e / D, d = e % D;
        const int64_t s = j * bs + r;
        float kv = 0.0f, vv = 0.0f;
        if (j >= 0 && s < S) {
            const int64_t src = b * sb + h * sh + s * ss + d;
            kv = load_elem<DT>(k, src);
            vv = load_elem<DT>(v, src);
        }
        store_elem<DT>(ko, obase + e, kv);
        store_elem<DT>(vo, obase + e, vv);
    }
}

int launch_gather(const void* k, const void* v, int dtype, int64_t sb, int64_t sh, int64_t ss,
                  const int32_t* idx, int64_t B, int64_t H, int64_t S, int64_t D, int64_t n,
                  int64_t bs, void* ko, void* vo, hipStream_t stream) {
    dim3 grid(static_cast<unsigned>(n), static_cast<unsigned>(H), static_cast<unsigned>(B));
    if (dtype == SPARDA_F32)
        hipLaunchKernelGGL((gather_kernel<SPARDA_F32>), grid, dim3(256), 0, stream, k, v, sb, sh, ss, idx,
                           S, static_cast<int>(D), n, static_cast<int>(bs), ko, vo);
    else
        hipLaunchKernelGGL((gather_kernel<SPARDA_BF16>), grid, dim3(256), 0, stream, k, v, sb, sh, ss, idx,
                           S, static_cast<int>(D), n, static_cast<int>(bs), ko, vo);
    return check_hip(hipGetLastError(), "gather_kernel");
}

}  // namespace sparda
