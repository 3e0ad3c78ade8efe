// KV cache held in pinned host memory, with forecast-driven block fetch.
//
// The arena of one cache (one layer) is [B][Hkv][Smax][D] in the cache dtype,
// allocated with hipHostMalloc (mapped, coherent), so the token rows of one
// KV head are contiguous and one KV block of one head is one contiguous run of
// bs*D elements (8 KiB for bs = D = 64, bf16): a block is one DMA or one tile.
//
//  * append: new tokens go from device memory straight into the arena through
//    its device mapping (vector stores over the host link), and the fp32 block
//    sums that back the prototypes are updated on the GPU for the touched
//    blocks only (sequential in s from the block start, so sum/bs is bit-equal
//    to the full-cache compression the reference redoes every step).
//  * select: decode-time routing from the block sums: scores of the blocks
//    present, top-k by wavefront ballot threshold search, sink + own block.
//  * fetch: the selected blocks into a compact device buffer
//    [B][Hkv][cap][bs][D] (slot i of (b, g) holds block sel[b,g,i]), either by
//    a gather kernel reading the arena through its device mapping (indices
//    stay on the GPU; no host synchronisation) or by the DMA engines
//    (hipMemcpyAsync per contiguous run of blocks; the selection is copied to
//    the host first, which waits for the stream once).
#pragma clang fp contract(off)

#include <stdlib.h>
#include <string.h>

#include <new>
#include <type_traits>

#include "common.h"
#include "kernels.h"
#include "prefetch.h"
#include "select.h"

struct sparda_offload {
    int64_t B, Smax, H, D;
    int dtype;
    int64_t esz;
    char* host;          // [2][B][H][Smax][D]: K arena then V arena
    char* dev;           // device address of `host`
    int32_t* staging;    // pinned host copy of a selection (DMA fetch)
    int64_t staging_cap; // int32 entries in `staging`
    int device;
};

namespace sparda {

constexpr int kSelThreads = 256;
constexpr int kSelMaxBlocks = 4096;  // blocks a selection can score (LDS key array)

static size_t arena_bytes(const sparda_offload* h) {
    return static_cast<size_t>(h->B * h->H * h->Smax * h->D * h->esz);
}

int offload_create(int64_t B, int64_t Smax, int64_t H, int64_t D, int dtype, sparda_offload_t* out) {
    sparda_offload* h = new (std::nothrow) sparda_offload{};
    if (h == nullptr) return set_error(SPARDA_ERR_CAPACITY, "offload_create: out of host memory");
    h->B = B;
    h->Smax = Smax;
    h->H = H;
    h->D = D;
    h->dtype = dtype;
    h->esz = dtype == SPARDA_F32 ? 4 : 2;
    int rc = check_hip(hipGetDevice(&h->device), "hipGetDevice");
    if (rc) {
        delete h;
        return rc;
    }
    const size_t bytes = 2 * arena_bytes(h);
    void* p = nullptr;
    rc = check_hip(hipHostMalloc(&p, bytes, hipHostMallocMapped | hipHostMallocCoherent), "hipHostMalloc(arena)");
    if (rc) {
        delete h;
        return rc;
    }
    memset(p, 0, bytes);  // rows never written read as zeros, like the reference's torch.zeros cache
    h->host = static_cast<char*>(p);
    void* d = nullptr;
    rc = check_hip(hipHostGetDevicePointer(&d, p, 0), "hipHostGetDevicePointer");
    if (rc) {
        (void)hipHostFree(p);
        delete h;
        return rc;
    }
    h->dev = static_cast<char*>(d);
    h->staging_cap = B * H * (kMaxFetchSlots + 1);
    void* st = nullptr;
    rc = check_hip(hipHostMalloc(&st, static_cast<size_t>(h->staging_cap) * 4, hipHostMallocDefault),
                   "hipHostMalloc(staging)");
    if (rc) {
        (void)hipHostFree(p);
        delete h;
        return rc;
    }
    h->staging = static_cast<int32_t*>(st);
    *out = h;
    return 0;
}

int offload_destroy(sparda_offload_t h) {
    int rc = 0;
    if (h->staging != nullptr) rc = check_hip(hipHostFree(h->staging), "hipHostFree(staging)");
    if (h->host != nullptr) {
        const int rc2 = check_hip(hipHostFree(h->host), "hipHostFree(arena)");
        if (rc == 0) rc = rc2;
    }
    delete h;
    return rc;
}

int64_t offload_max_seq(sparda_offload_t h) { return h->Smax; }
int64_t offload_batch(sparda_offload_t h) { return h->B; }
int64_t offload_heads(sparda_offload_t h) { return h->H; }
int64_t offload_head_dim(sparda_offload_t h) { return h->D; }
int offload_dtype(sparda_offload_t h) { return h->dtype; }

void offload_prefetch_dev(sparda_offload_t h, PrefetchDev* pf) {
    pf->ak = h->dev;
    pf->av = h->dev + arena_bytes(h);
    pf->H = h->H;
    pf->Smax = h->Smax;
    pf->row_bytes = h->D * h->esz;
}

void offload_host(sparda_offload_t h, void** k, void** v) {
    *k = h->host;
    *v = h->host + arena_bytes(h);
}

// ---------------------------------------------------------------------------
// append: token rows [pos, pos+n) of k/v ([B,n,H,D], strides sb, st, sh)
// into the arena; one thread per VEC-element chunk of a row.
// ---------------------------------------------------------------------------
template <int VEC_BYTES>
__global__ void __launch_bounds__(256)
arena_store_kernel(const char* __restrict__ k, const char* __restrict__ v, int64_t sb, int64_t st,
                   int64_t sh, int64_t n, int64_t pos, int64_t esz, int64_t row_bytes, int64_t H,
                   int64_t Smax, char* __restrict__ ak, char* __restrict__ av) {
    using W = typename std::conditional<VEC_BYTES == 16, uint4, typename std::conditional<VEC_BYTES == 8, uint2,
                                        typename std::conditional<VEC_BYTES == 4, uint32_t, uint16_t>::type>::type>::type;
    const int64_t chunks = row_bytes / VEC_BYTES;
    const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= n * chunks) return;
    const int64_t t = e / chunks;
    const int64_t c = e % chunks;
    const int64_t g = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int64_t src = (b * sb + t * st + g * sh) * esz + c * VEC_BYTES;
    const int64_t dst = ((b * H + g) * Smax + pos + t) * row_bytes + c * VEC_BYTES;
    const W kw = *reinterpret_cast<const W*>(k + src);
    const W vw = *reinterpret_cast<const W*>(v + src);
    *reinterpret_cast<W*>(ak + dst) = kw;
    *reinterpret_cast<W*>(av + dst) = vw;
}

// fp32 block sums of the blocks touched by tokens [pos, pos+n): for each
// (b, block j, g, d) continue the sequential sum from the block start
// (restart at 0 when pos is at or before the block start).
// k: [B,n,H,D] strides (sb, st, sh) holding tokens pos..pos+n-1.
template <int DT>
__global__ void __launch_bounds__(256)
block_sums_kernel(const void* __restrict__ k, int64_t sb, int64_t st, int64_t sh, int64_t pos, int64_t n,
                  int64_t H, int64_t D, int64_t bs, int64_t nb_stride, float* __restrict__ sums) {
    constexpr int U = 32;  // token loads in flight per thread, added in token order
    const int64_t j = pos / bs + blockIdx.x;
    const int64_t b = blockIdx.y;
    const int64_t s_lo = j * bs > pos ? j * bs : pos;
    const int64_t s_hi = (j + 1) * bs < pos + n ? (j + 1) * bs : pos + n;
    for (int64_t e = threadIdx.x; e < H * D; e += blockDim.x) {
        const int64_t g = e / D, d = e % D;
        float* out = sums + ((b * nb_stride + j) * H + g) * D + d;
        const int64_t base = b * sb + g * sh + d;
        float acc = s_lo == j * bs ? 0.0f : *out;
        // a partial last batch reads its last token again and skips the repeats
        for (int64_t s = s_lo; s < s_hi; s += U) {
            float x[U];
#pragma unroll
            for (int u = 0; u < U; ++u) x[u] = load_elem<DT>(k, base + ((s + u < s_hi ? s + u : s_hi - 1) - pos) * st);
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (s + u < s_hi) acc = acc + x[u];
        }
        *out = acc;
    }
}

int launch_block_sums(const void* k, int dtype, int64_t sb, int64_t st, int64_t sh, int64_t pos,
                      int64_t n, int64_t B, int64_t H, int64_t D, int64_t bs, int64_t nb_stride,
                      float* sums, hipStream_t stream) {
    const int64_t nblk = (pos + n - 1) / bs - pos / bs + 1;
    dim3 grid(static_cast<unsigned>(nblk), static_cast<unsigned>(B));
    int threads = static_cast<int>(H * D < 256 ? H * D : 256);
    threads = ((threads + kWave - 1) / kWave) * kWave;
    if (dtype == SPARDA_BF16)
        hipLaunchKernelGGL(block_sums_kernel<SPARDA_BF16>, grid, dim3(threads), 0, stream, k, sb, st, sh, pos, n,
                           H, D, bs, nb_stride, sums);
    else
        hipLaunchKernelGGL(block_sums_kernel<SPARDA_F32>, grid, dim3(threads), 0, stream, k, sb, st, sh, pos, n,
                           H, D, bs, nb_stride, sums);
    return check_hip(hipGetLastError(), "block_sums_kernel");
}

// Decode-step append at a device-held position p = *pos_dev (clamped into
// [0, max_len)), one workgroup per sequence: with k_new, the token's K and V
// rows are written into the caches at row p; the fp32 sums of the block
// holding p are recomputed over [p - p % bs, p] in token order (the sums
// block_sums_kernel gives), row p taken from k_new, so that no thread reads a
// row another thread writes. Workgroups past the first n_append carry the
// selection stage of the next layer's prefetch (pf, D = 64), one per
// (sequence, KV head) of that layer.
template <int DT>
__global__ void __launch_bounds__(256)
append_at_kernel(void* __restrict__ kc, void* __restrict__ vc, int64_t sb, int64_t st, int64_t sh,
                 const void* __restrict__ k_new, const void* __restrict__ v_new, int64_t n_sb, int64_t n_sh,
                 int64_t H, int64_t D, int64_t bs, int64_t max_len, int64_t nb_stride,
                 const int64_t* __restrict__ pos_dev, float* __restrict__ sums, int n_append, PrefetchDev pf) {
    using E = typename std::conditional<DT == SPARDA_BF16, uint16_t, float>::type;
    constexpr int U = 32;
    if (static_cast<int>(blockIdx.x) >= n_append) {
        __shared__ float f_lds[kMaxHeadDim];
        __shared__ uint32_t key_lds[kSelMaxBlocks];
        __shared__ int32_t sel_lds[kMaxSelCap + 2];
        __shared__ uint32_t ck_lds[kWave];
        __shared__ int32_t ci_lds[kWave];
        __shared__ int m_lds;
        const int idx = static_cast<int>(blockIdx.x) - n_append;
        prefetch_workgroup<64, 64>(pf, idx % static_cast<int>(pf.H), idx / static_cast<int>(pf.H), pos_dev, f_lds,
                                   key_lds, sel_lds, ck_lds, ci_lds, &m_lds);
        return;
    }
    const int64_t b = blockIdx.x;
    int64_t p = *pos_dev;
    p = p < 0 ? 0 : (p >= max_len ? max_len - 1 : p);
    const int64_t j = p / bs;
    // rows read from the cache (none when only the new row is written)
    const int64_t s_hi = sums == nullptr ? j * bs : (k_new != nullptr ? p : p + 1);
    E* kce = static_cast<E*>(kc);
    for (int64_t e = threadIdx.x; e < H * D; e += blockDim.x) {
        const int64_t g = e / D, d = e % D;
        const int64_t base = b * sb + g * sh + d;
        // rows in batches of U loads in flight (a partial last batch reads its
        // last row again and skips the repeats), added in row order
        float acc = 0.0f;
        for (int64_t s = j * bs; s < s_hi; s += U) {
            float x[U];
#pragma unroll
            for (int u = 0; u < U; ++u) x[u] = load_elem<DT>(kc, base + (s + u < s_hi ? s + u : s_hi - 1) * st);
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (s + u < s_hi) acc = acc + x[u];
        }
        if (k_new != nullptr) {
            const int64_t ni = b * n_sb + g * n_sh + d;
            const E kv = static_cast<const E*>(k_new)[ni];
            kce[base + p * st] = kv;
            static_cast<E*>(vc)[base + p * st] = static_cast<const E*>(v_new)[ni];
            acc = acc + load_elem<DT>(k_new, ni);
        }
        if (sums != nullptr) sums[((b * nb_stride + j) * H + g) * D + d] = acc;
    }
}

static int launch_append_at_pf(void* kc, void* vc, int dtype, int64_t sb, int64_t st, int64_t sh,
                               const void* k_new, const void* v_new, int64_t n_sb, int64_t n_sh, int64_t B,
                               int64_t H, int64_t D, int64_t bs, int64_t max_len, int64_t nb_stride,
                               const int64_t* pos_dev, float* sums, hipStream_t stream, const PrefetchDev* pf) {
    int threads = static_cast<int>(H * D < 256 ? H * D : 256);
    threads = ((threads + kWave - 1) / kWave) * kWave;
    // a carried selection takes workgroups of kSelThreads (the append's own need fewer at small H*D)
    if (pf != nullptr) threads = kSelThreads;
    const int64_t n_pf = pf != nullptr ? B * pf->H : 0;  // the next layer's batch is B too
    dim3 grid(static_cast<unsigned>(B + n_pf));
    const PrefetchDev pfv = pf != nullptr ? *pf : PrefetchDev{};
    if (dtype == SPARDA_BF16)
        hipLaunchKernelGGL(append_at_kernel<SPARDA_BF16>, grid, dim3(threads), 0, stream, kc, vc, sb, st, sh, k_new,
                           v_new, n_sb, n_sh, H, D, bs, max_len, nb_stride, pos_dev, sums, static_cast<int>(B), pfv);
    else
        hipLaunchKernelGGL(append_at_kernel<SPARDA_F32>, grid, dim3(threads), 0, stream, kc, vc, sb, st, sh, k_new,
                           v_new, n_sb, n_sh, H, D, bs, max_len, nb_stride, pos_dev, sums, static_cast<int>(B), pfv);
    return check_hip(hipGetLastError(), "append_at_kernel");
}

int launch_append_at(void* kc, void* vc, int dtype, int64_t sb, int64_t st, int64_t sh, const void* k_new,
                     const void* v_new, int64_t n_sb, int64_t n_sh, int64_t B, int64_t H, int64_t D, int64_t bs,
                     int64_t max_len, int64_t nb_stride, const int64_t* pos_dev, float* sums, hipStream_t stream) {
    return launch_append_at_pf(kc, vc, dtype, sb, st, sh, k_new, v_new, n_sb, n_sh, B, H, D, bs, max_len, nb_stride,
                               pos_dev, sums, stream, nullptr);
}

int offload_append(sparda_offload_t h, const void* k, const void* v, int64_t sb, int64_t st, int64_t sh,
                   int64_t pos, int64_t n, int64_t bs, float* sums, hipStream_t stream) {
    const int64_t row_bytes = h->D * h->esz;
    char* ak = h->dev;
    char* av = h->dev + arena_bytes(h);
    auto aligned = [&](int64_t vb) {
        const int64_t ve = vb / h->esz;
        return row_bytes % vb == 0 && sb % ve == 0 && st % ve == 0 && sh % ve == 0 &&
               reinterpret_cast<uintptr_t>(k) % vb == 0 && reinterpret_cast<uintptr_t>(v) % vb == 0;
    };
    const int vb = aligned(16) ? 16 : aligned(8) ? 8 : aligned(4) ? 4 : static_cast<int>(h->esz);
    const int64_t total = n * (row_bytes / vb);
    dim3 grid(static_cast<unsigned>(cdiv(total, 256)), static_cast<unsigned>(h->H), static_cast<unsigned>(h->B));
#define SPARDA_STORE(VB)                                                                                 \
    hipLaunchKernelGGL(arena_store_kernel<VB>, grid, dim3(256), 0, stream, static_cast<const char*>(k),  \
                       static_cast<const char*>(v), sb, st, sh, n, pos, h->esz, row_bytes, h->H, h->Smax, \
                       ak, av)
    if (vb == 16) SPARDA_STORE(16);
    else if (vb == 8) SPARDA_STORE(8);
    else if (vb == 4) SPARDA_STORE(4);
    else SPARDA_STORE(2);
#undef SPARDA_STORE
    int rc = check_hip(hipGetLastError(), "arena_store_kernel");
    if (rc || sums == nullptr) return rc;
    return launch_block_sums(k, h->dtype, sb, st, sh, pos, n, h->B, h->H, h->D, bs, cdiv(h->Smax, bs), sums,
                             stream);
}

int offload_append_at(sparda_offload_t h, const void* k, const void* v, int64_t n_sb, int64_t n_sh,
                      const int64_t* pos_dev, int64_t bs, float* sums, hipStream_t stream, const PrefetchDev* pf) {
    // the arena through its device mapping: [B][H][Smax][D] -> strides (H*Smax*D, D, Smax*D)
    return launch_append_at_pf(h->dev, h->dev + arena_bytes(h), h->dtype, h->H * h->Smax * h->D, h->D,
                               h->Smax * h->D, k, v, n_sb, n_sh, h->B, h->H, h->D, bs, h->Smax, cdiv(h->Smax, bs),
                               pos_dev, sums, stream, pf);
}

int offload_rebuild_sums(sparda_offload_t h, int64_t len, int64_t bs, float* sums, hipStream_t stream) {
    // the arena read through its device mapping: [B][H][Smax][D] -> strides (H*Smax*D, D, Smax*D)
    return launch_block_sums(h->dev, h->dtype, h->H * h->Smax * h->D, h->D, h->Smax * h->D, 0, len, h->B, h->H,
                             h->D, bs, cdiv(h->Smax, bs), sums, stream);
}

// ---------------------------------------------------------------------------
// decode selection from block sums, one wavefront per (sequence, KV head).
// Blocks j < n_present = ceil(len/bs) are scored with p = sums/bs:
//   score_j = (fma chain over d of f[d]*p_j[d]) * scale, -inf for j > score_pos/bs
// own = pos/bs. If own+1 <= k+2 every block 0..own is selected (the dense
// fallback); otherwise sel = ascending {0, own} U top-k (ties by lower index).
// ---------------------------------------------------------------------------

template <int FDT, int CH, int DH, bool POW2>
__global__ void __launch_bounds__(kSelThreads)
select_decode_kernel(const void* __restrict__ f, int64_t f_sb, int64_t f_sh, const float* __restrict__ sums,
                     int64_t H, int64_t nb_stride, int64_t n_present_arg, int64_t pos_arg, int64_t score_pos_arg,
                     int64_t bs, int k, float scale, int32_t* __restrict__ sel, int32_t* __restrict__ n_sel,
                     int cap, const int64_t* __restrict__ pos_dev, int absolute, int lookahead) {
    __shared__ float f_lds[kMaxHeadDim];
    __shared__ uint32_t key_lds[kSelMaxBlocks];
    __shared__ int32_t sel_lds[kMaxSelCap + 2];
    __shared__ uint32_t ck_lds[kWave];
    __shared__ int32_t ci_lds[kWave];
    __shared__ int m_lds;
    const int g = blockIdx.x;
    const int b = blockIdx.y;
    const int tid = threadIdx.x;
    const int64_t bg = static_cast<int64_t>(b) * H + g;
    // with pos_dev: a decode step at token p = *pos_dev (clamped into [0, pos_arg]),
    // len = p + 1, or with lookahead the prefetch before token p is appended,
    // len = p; otherwise the host's len / pos
    int64_t pos = pos_arg, n_present = n_present_arg, score_pos = score_pos_arg;
    if (pos_dev != nullptr) {
        const int64_t p = *pos_dev;
        pos = p < 0 ? 0 : (p > pos_arg ? pos_arg : p);
        n_present = lookahead ? (pos + bs - 1) / bs : pos / bs + 1;
        score_pos = absolute ? pos : 0;
    }
    const int own = static_cast<int>(pos / bs);
    const int m = select_from_sums<CH, DH, POW2>(f, FDT == SPARDA_BF16, b * f_sb + g * f_sh,
                                                 sums + (b * nb_stride * H + g) * DH, H * DH, n_present,
                                                 score_pos / bs, own, k, static_cast<int>(bs), scale, f_lds,
                                                 key_lds, sel_lds, ck_lds, ci_lds, &m_lds);
    for (int i = tid; i < cap; i += kSelThreads) sel[bg * cap + i] = i < m ? sel_lds[i] : -1;
    if (tid == 0) n_sel[bg] = m;
}

int launch_select_decode(const void* f, int fdtype, int64_t f_sb, int64_t f_sh, const float* sums, int64_t B,
                         int64_t H, int64_t D, int64_t nb_stride, int64_t len, int64_t pos, int64_t bs,
                         int64_t k, int routing, float scale, int32_t* sel, int32_t* n_sel, int64_t cap,
                         hipStream_t stream, const int64_t* pos_dev, int lookahead) {
    // with pos_dev, len bounds the device length (pos = len - 1 is the largest position)
    const int64_t n_present = cdiv(len, bs);
    const int64_t score_pos = routing == SPARDA_ROUTE_ABSOLUTE ? pos : 0;
    const bool pow2 = (bs & (bs - 1)) == 0;
    dim3 grid(static_cast<unsigned>(H), static_cast<unsigned>(B));
#define SPARDA_SEL(FDT_, CH_, DH_, P2_)                                                                     \
    hipLaunchKernelGGL((select_decode_kernel<FDT_, CH_, DH_, P2_>), grid, dim3(kSelThreads), 0, stream, f,  \
                       f_sb, f_sh, sums, H, nb_stride, n_present, pos, score_pos, bs, static_cast<int>(k),  \
                       scale, sel, n_sel, static_cast<int>(cap), pos_dev,                                   \
                       routing == SPARDA_ROUTE_ABSOLUTE ? 1 : 0, lookahead)
#define SPARDA_SEL_P(FDT_, CH_, DH_)                    \
    if (pow2) SPARDA_SEL(FDT_, CH_, DH_, true);         \
    else SPARDA_SEL(FDT_, CH_, DH_, false);
#define SPARDA_SEL_D(FDT_, CH_)                         \
    switch (D) {                                        \
        case 16: SPARDA_SEL_P(FDT_, CH_, 16) break;     \
        case 32: SPARDA_SEL_P(FDT_, CH_, 32) break;     \
        case 64: SPARDA_SEL_P(FDT_, CH_, 64) break;     \
        default: SPARDA_SEL_P(FDT_, CH_, 128) break;    \
    }
#define SPARDA_SEL_C(FDT_)                                  \
    if (n_present <= 256) { SPARDA_SEL_D(FDT_, 4) }         \
    else if (n_present <= 1024) { SPARDA_SEL_D(FDT_, 16) }  \
    else { SPARDA_SEL_D(FDT_, 64) }
    if (fdtype == SPARDA_BF16) {
        SPARDA_SEL_C(SPARDA_BF16)
    } else {
        SPARDA_SEL_C(SPARDA_F32)
    }
#undef SPARDA_SEL_C
#undef SPARDA_SEL_D
#undef SPARDA_SEL_P
#undef SPARDA_SEL
    return check_hip(hipGetLastError(), "select_decode_kernel");
}

// ---------------------------------------------------------------------------
// fetch by gather kernel: workgroup (slot, g, b) copies block sel[b,g,slot]
// (rows below len) from the arena into slot `slot` of the compact buffers.
// All 16-byte loads of a thread are issued before its stores.
// ---------------------------------------------------------------------------
constexpr int kFetchThreads = 256;

__global__ void __launch_bounds__(kFetchThreads)
fetch_blocks_kernel(const char* __restrict__ ak, const char* __restrict__ av, const int32_t* __restrict__ sel,
                    const int32_t* __restrict__ n_sel, int cap, int64_t H, int64_t Smax, int64_t row_bytes,
                    int64_t bs, int64_t len_arg, char* __restrict__ dk, char* __restrict__ dv,
                    const int64_t* __restrict__ len_dev) {
    // with len_dev the arena length is read when the kernel runs (clamped into [0, Smax])
    int64_t len = len_arg;
    if (len_dev != nullptr) {
        len = *len_dev;
        len = len < 0 ? 0 : (len > Smax ? Smax : len);
    }
    const int slot = blockIdx.x;
    const int64_t g = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int64_t bg = b * H + g;
    if (slot >= n_sel[bg]) return;
    const int64_t j = sel[bg * cap + slot];
    if (j < 0 || j * bs >= len) return;
    const int64_t rows = (j + 1) * bs < len ? bs : len - j * bs;
    const int64_t chunks = rows * row_bytes / 16;
    const uint4* sk = reinterpret_cast<const uint4*>(ak + (bg * Smax + j * bs) * row_bytes);
    const uint4* sv = reinterpret_cast<const uint4*>(av + (bg * Smax + j * bs) * row_bytes);
    uint4* tk = reinterpret_cast<uint4*>(dk + (bg * cap + slot) * bs * row_bytes);
    uint4* tv = reinterpret_cast<uint4*>(dv + (bg * cap + slot) * bs * row_bytes);
    // two chunks of K and two of V in flight per thread (a 64 x 128 B block is 512 chunks)
    for (int64_t c = threadIdx.x; c < chunks; c += 2 * kFetchThreads) {
        const int64_t c2 = c + kFetchThreads;
        const bool two = c2 < chunks;
        const uint4 k0 = sk[c];
        const uint4 v0 = sv[c];
        uint4 k1 = make_uint4(0u, 0u, 0u, 0u), v1 = k1;
        if (two) {
            k1 = sk[c2];
            v1 = sv[c2];
        }
        tk[c] = k0;
        tv[c] = v0;
        if (two) {
            tk[c2] = k1;
            tv[c2] = v1;
        }
    }
}

int offload_fetch(sparda_offload_t h, const int32_t* sel, const int32_t* n_sel, int64_t cap, int64_t bs,
                  int64_t len, int method, void* k_dst, void* v_dst, hipStream_t stream, const int64_t* len_dev) {
    const int64_t row_bytes = h->D * h->esz;
    const size_t ab = arena_bytes(h);
    if (method == SPARDA_FETCH_KERNEL) {
        dim3 grid(static_cast<unsigned>(cap), static_cast<unsigned>(h->H), static_cast<unsigned>(h->B));
        hipLaunchKernelGGL(fetch_blocks_kernel, grid, dim3(kFetchThreads), 0, stream, h->dev, h->dev + ab, sel,
                           n_sel, static_cast<int>(cap), h->H, h->Smax, row_bytes, bs, len,
                           static_cast<char*>(k_dst), static_cast<char*>(v_dst), len_dev);
        return check_hip(hipGetLastError(), "fetch_blocks_kernel");
    }
    // DMA: the selection to the host (one wait on the stream), then one copy
    // per run of consecutive blocks, per tensor.
    const int64_t BH = h->B * h->H;
    int32_t* hs = h->staging;
    int32_t* hn = h->staging + BH * cap;
    int rc = check_hip(hipMemcpyAsync(hs, sel, static_cast<size_t>(BH * cap) * 4, hipMemcpyDeviceToHost, stream),
                       "hipMemcpyAsync(sel)");
    if (rc) return rc;
    rc = check_hip(hipMemcpyAsync(hn, n_sel, static_cast<size_t>(BH) * 4, hipMemcpyDeviceToHost, stream),
                   "hipMemcpyAsync(n_sel)");
    if (rc) return rc;
    rc = check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize(fetch)");
    if (rc) return rc;
    const int64_t blk = bs * row_bytes;
    for (int64_t bg = 0; bg < BH; ++bg) {
        const int64_t n = hn[bg] < cap ? hn[bg] : cap;
        const int32_t* s = hs + bg * cap;
        int64_t i = 0;
        while (i < n) {
            const int64_t j0 = s[i];
            int64_t i1 = i + 1;
            while (i1 < n && s[i1] == s[i1 - 1] + 1) ++i1;
            if (j0 >= 0 && j0 * bs < len) {
                const int64_t jl = s[i1 - 1];
                int64_t end = (jl + 1) * bs;
                if (end > len) end = len;
                const size_t bytes = static_cast<size_t>((end - j0 * bs) * row_bytes);
                const int64_t src = (bg * h->Smax + j0 * bs) * row_bytes;
                const int64_t dst = (bg * cap + i) * blk;
                rc = check_hip(hipMemcpyAsync(static_cast<char*>(k_dst) + dst, h->host + src, bytes,
                                              hipMemcpyHostToDevice, stream), "hipMemcpyAsync(K run)");
                if (rc) return rc;
                rc = check_hip(hipMemcpyAsync(static_cast<char*>(v_dst) + dst, h->host + ab + src, bytes,
                                              hipMemcpyHostToDevice, stream), "hipMemcpyAsync(V run)");
                if (rc) return rc;
            }
            i = i1;
        }
    }
    return 0;
}

}  // namespace sparda
