/*
 * sparda.h — C ABI of libsparda.so, the MI355X (gfx950) implementation of
 * SparDA's forecast-guided block-sparse attention path.
 *
 * Every entry point is `extern "C"`, takes plain pointers, element strides
 * and sizes, and returns an int status:
 *     0   success
 *    >0   a hipError_t raised by a HIP call (message in sparda_last_error())
 *    <0   an argument error, detected before any HIP call is made
 * No exception crosses the boundary. All tensor pointers are device pointers
 * owned by the caller unless stated otherwise. `stream` is a hipStream_t
 * (NULL = the legacy default stream); every call is stream-ordered and never
 * synchronises the device, with one exception: sparda_offload_fetch with
 * SPARDA_FETCH_DMA waits on the host for `stream` (the selection must reach
 * the host to build the copies), so that form cannot be captured into a HIP
 * graph; SPARDA_FETCH_KERNEL is the capturable form. Calls are re-entrant;
 * the offload handle is the only stateful object.
 *
 * Layout vocabulary (the reference's own): B batch, S/T sequence length,
 * Hq query heads, Hkv key/value heads (== forecast heads), D head dim,
 * Df forecast dim (== D), bs block size, NB = ceil(S/bs) KV blocks,
 * k top-k blocks. Query head h uses KV head h / (Hq/Hkv).
 *
 * Reference citations are into tyborra/local-research-Small-Language-Model.
 */
#ifndef SPARDA_H
#define SPARDA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPARDA_API __attribute__((visibility("default")))

/* Element types of tensors crossing the boundary. */
enum {
    SPARDA_F32 = 0,
    SPARDA_BF16 = 1,
};

/* Argument-error status codes (all negative). */
enum {
    SPARDA_ERR_NULL = -1,     /* a required pointer is NULL */
    SPARDA_ERR_SHAPE = -2,    /* a size is out of range or inconsistent */
    SPARDA_ERR_DTYPE = -3,    /* unsupported element type */
    SPARDA_ERR_WORKSPACE = -4,/* workspace missing or too small */
    SPARDA_ERR_STRIDE = -5,   /* unsupported stride (innermost must be 1) */
    SPARDA_ERR_MODE = -6,     /* unknown mode / routing value */
    SPARDA_ERR_HANDLE = -7,   /* invalid offload handle or layer */
    SPARDA_ERR_CAPACITY = -8, /* cache/arena capacity exceeded */
};

/* Decode routing modes (sparda_decode). */
enum {
    /* Score the forecast with the causal mask taken at query row 0, as the
     * reference's decode does (model/forecast.py:120-126 called from
     * model/attention/sparse.py:139): only block 0 is finite, the other
     * k-1 picks are -inf ties, resolved here by lower block index. */
    SPARDA_ROUTE_REFERENCE = 0,
    /* Score with the mask at the query's absolute position S-1: every block
     * up to the current one competes (forecast routing as intended). */
    SPARDA_ROUTE_ABSOLUTE = 1,
};

/* Fixed (forecast-free) selections (sparda_select_fixed). */
enum {
    SPARDA_SEL_DENSE = 0,         /* every block <= own block
                                     (model/attention/sparse.py:113-123) */
    SPARDA_SEL_WINDOW_DECODE = 1, /* {0} U [own-k+1, own]
                                     (model/attention/sparse.py:142-147) */
    SPARDA_SEL_WINDOW_PREFILL = 2,/* {0} U [own-k, own]
                                     (model/attention/sparse.py:250-251) */
};

/* Transfer methods of sparda_offload_fetch. */
enum {
    SPARDA_FETCH_KERNEL = 0, /* gather kernel reading the arena through its device
                                mapping; indices stay on the GPU */
    SPARDA_FETCH_DMA = 1,    /* hipMemcpyAsync per run of consecutive blocks; the
                                selection is copied to the host first: the call
                                waits on the host for the stream (one
                                hipStreamSynchronize), not capturable */
};

/* Host-resident KV cache of one layer (opaque; see sparda_offload_create). */
typedef struct sparda_offload* sparda_offload_t;

/* Top-k algorithm selector for sparda_topk_scores. */
enum {
    SPARDA_TOPK_AUTO = 0,
    SPARDA_TOPK_ROWS = 1,   /* one lane per row, register insertion list */
    SPARDA_TOPK_WAVE = 2,   /* one workgroup per row, wavefront arg-max rounds */
};

/* Version of this ABI (major*100 + minor). */
SPARDA_API int sparda_version(void);

/* Message describing the last non-zero status returned on this thread. */
SPARDA_API const char* sparda_last_error(void);

/* Bits of the per-device status word (sparda_status). */
enum {
    /* A compacted prefill workgroup gave up an ordering wait after its poll
     * limit (never expected: waits end when earlier tiles commit). Its query
     * window's output rows were written as NaN. */
    SPARDA_STATUS_PREFILL_WAIT_TIMEOUT = 1,
};

/*
 * Status word of the current device: the SPARDA_STATUS_* conditions raised by
 * kernels since it was last cleared. Writes it to `out` (one uint32, device
 * memory), clearing it when `clear` != 0; stream-ordered like every other
 * call (the word reflects the launches queued on `stream` before it), with no
 * host wait, so it can be captured into a HIP graph. No counterpart in the
 * reference, which has no kernels that can abandon work; the caller reads
 * `out` when the stream has reached it.
 */
SPARDA_API int sparda_status(uint32_t* out, int clear, void* stream);

/*
 * KV block compressor.
 * Replaces KVBlockCompressor.forward (model/forecast.py:57-78).
 *   protos[b,j,h,d] = (sum_{s = j*bs}^{min((j+1)*bs, S)-1} k[b,s,h,d]) / bs
 * The sum runs in fp32, sequentially in increasing s, and is then divided by
 * bs (not by the count of present tokens: the reference zero-pads the last
 * block, model/forecast.py:68-77).
 *   k:      [B,S,H,D] of `dtype`, strides (stride_b, stride_s, stride_h, 1)
 *   protos: [B,NB,H,D] fp32, contiguous, NB = ceil(S/bs)
 */
SPARDA_API int sparda_compress(const void* k, int dtype,
                               int64_t B, int64_t S, int64_t H, int64_t D,
                               int64_t stride_b, int64_t stride_s, int64_t stride_h,
                               int64_t block_size, float* protos, void* stream);

/*
 * Fused forecast score + top-k block router.
 * Replaces ForecastBlockSelector.forward (model/forecast.py:89-130) and the
 * selection-set construction of the sparse backend
 * (model/attention/sparse.py:126-154 decode, 231-247 prefill).
 *   score[b,h,t,j] = (fma-chain_d f[b,t,h,d]*protos[b,j,h,d]) * scale, fp32,
 *                    -inf where causal && j > (score_pos0 + t) / bs
 *   topk[b,h,t,:]  = the min(top_k, NB) blocks with the largest scores,
 *                    ordered by score descending, ties (including -inf
 *                    ties) by lower block index
 *   sel[b,h,t,:]   = ({0, own} U topk) restricted to blocks <= own when
 *                    causal, sorted ascending, no duplicates, padded with -1;
 *                    own = min((query_pos0 + t) / bs, NB-1); n_sel = count
 *   forecast: [B,Tq,H,Df] of f_dtype, strides (f_sb, f_st, f_sh, 1)
 *   protos:   [B,NB,H,Df] fp32 contiguous, 16-byte aligned (sparda_compress output)
 * Any of topk / scores / sel (+n_sel) may be NULL. sel_cap >= min(top_k,NB)+2.
 * The reference's prefill uses score_pos0 = query_pos0 = 0.
 */
SPARDA_API int sparda_route(const void* forecast, int f_dtype,
                            int64_t f_sb, int64_t f_st, int64_t f_sh,
                            const float* protos,
                            int64_t B, int64_t Tq, int64_t H, int64_t Df, int64_t NB,
                            int64_t block_size, int64_t top_k, int causal,
                            int64_t score_pos0, int64_t query_pos0, float scale,
                            int32_t* topk, float* scores,
                            int32_t* sel, int32_t* n_sel, int64_t sel_cap,
                            void* stream);

/*
 * Canonical top-k over given fp32 score rows (no masking applied here).
 * The selection stage of sparda_route fed with caller-provided scores, so
 * that index parity can be checked on identical fp32 scores
 * (torch.topk at model/forecast.py:129 with ties broken by lower index).
 *   scores: [rows, NB] fp32 contiguous;  topk: [rows, min(top_k, NB)] int32
 */
SPARDA_API int sparda_topk_scores(const float* scores, int64_t rows, int64_t NB,
                                  int64_t top_k, int algo, int32_t* topk,
                                  void* stream);

/*
 * Per-query-block lists of the chunked-gather prefill. Replaces the
 * selection of SparseAttention._forward_chunked_gather
 * (model/attention/sparse.py:303-333): for query block bq (rows
 * bq*bs .. min(T, (bq+1)*bs) - 1) the set {0, bq} U the union of those rows'
 * top-k picks (topk [B,H,T,top_k_width] int32: sparda_route's non-causal
 * top-k, used for bq > 0) or, with topk NULL or at bq = 0, U the static
 * window [max(0, bq-top_k+1), bq]; blocks past bq dropped; then its lowest
 * min(NB, top_k+2) indices (the reference cuts with torch.topk over a 0/1
 * mask, whose order among the equal entries is unspecified; the lowest
 * indices are the library's tie rule). Every row of the block gets the
 * block's list: sel/n_sel [B,H,T,sel_cap] / [B,H,T] int32, ascending, -1
 * padded, min(NB, top_k+2) <= sel_cap <= 34, NB = ceil(T/bs) <= 4096.
 * sparda_prefill over these lists is the chunked path's attention.
 */
SPARDA_API int sparda_select_chunked(const int32_t* topk, int64_t top_k_width, int64_t B, int64_t H, int64_t T,
                                     int64_t block_size, int64_t top_k, int32_t* sel, int32_t* n_sel,
                                     int64_t sel_cap, void* stream);

/*
 * Forecast-free selection lists: dense causal fallback and the static
 * sink + sliding-window modes.
 * Replaces model/attention/sparse.py:113-123 (decode dense fallback),
 * 142-147 (decode window), 250-251 (prefill window).
 *   own = min((query_pos0 + t) / bs, NB-1) for t in [0, Tq)
 *   sel/n_sel: [B,H,Tq,sel_cap] int32 / [B,H,Tq] int32, ascending, -1 padded
 */
SPARDA_API int sparda_select_fixed(int mode, int64_t B, int64_t Tq, int64_t H,
                                   int64_t NB, int64_t block_size, int64_t top_k,
                                   int64_t query_pos0,
                                   int32_t* sel, int32_t* n_sel, int64_t sel_cap,
                                   void* stream);

/*
 * Materialised block gather.
 * Replaces gather_kv_blocks (model/attention/sparse.py:19-62).
 *   k, v:  [B,H,S,D] of dtype, strides (sb, sh, ss, 1)
 *   idx:   [B,H,n] int32 block indices in [0, NB)
 *   k_out, v_out: [B,H,n*bs,D] contiguous; tokens >= S are zero (the
 *          reference pads the sequence to NB*bs, sparse.py:41-43)
 */
SPARDA_API int sparda_gather_blocks(const void* k, const void* v, int dtype,
                                    int64_t sb, int64_t sh, int64_t ss,
                                    const int32_t* idx,
                                    int64_t B, int64_t H, int64_t S, int64_t D,
                                    int64_t n, int64_t block_size,
                                    void* k_out, void* v_out, void* stream);

/*
 * Block-sparse GQA prefill attention.
 * Replaces the mask build + masked SDPA of SparseAttention._forward_masked_sdpa
 * (model/attention/sparse.py:226-281), including its GQA expansion
 * (repeat_interleave, sparse.py:264-270): query head h reads KV head
 * h / (Hq/Hkv) directly.
 *   out[b,t,h*D+d] = sum_{s in A(b,g,t)} softmax_s(q.k_s * scale) v_s[d]
 *   A(b,g,t) = { s < T : s/bs in sel[b,g,t,:n_sel] } and s <= t if causal.
 * sel == NULL means dense (every block), the fallback of sparse.py:201-224.
 *   q: [B,T,Hq,D] strides (q_sb,q_st,q_sh,1); k,v: [B,T,Hkv,D] strides
 *   (kv_sb,kv_st,kv_sh,1); sel/n_sel from sparda_route or
 *   sparda_select_fixed ([B,Hkv,T,sel_cap] / [B,Hkv,T]);
 *   out: [B,T,Hq*D] of dtype, strides (out_sb, out_st, 1)
 */
SPARDA_API int sparda_prefill(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                              const void* k, const void* v,
                              int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                              int dtype,
                              const int32_t* sel, const int32_t* n_sel, int64_t sel_cap,
                              int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                              int64_t block_size, int causal, float scale,
                              void* out, int64_t out_sb, int64_t out_st,
                              void* stream);

/*
 * Routed block-sparse GQA prefill: sparda_route with score_pos0 = query_pos0
 * = 0 followed by sparda_prefill on its lists, in one launch where the shape
 * allows. Replaces the prefill forward of ForecastBlockSelector
 * (model/forecast.py:89-130) and SparseAttention's selection + masked SDPA
 * (model/attention/sparse.py:231-281).
 *   q, k, v, out, scale: as in sparda_prefill
 *   forecast: [B,T,Hkv,Df] of f_dtype, strides (f_sb, f_st, f_sh, 1)
 *   protos:   [B,ceil(T/bs),Hkv,Df] fp32 contiguous, 16-byte aligned
 *             (sparda_compress of k)
 *   top_k, route_scale: the router's (route_scale is its score scale)
 *   sel, n_sel: optional [B,Hkv,T,sel_cap] / [B,Hkv,T], sel_cap >=
 *             min(top_k, NB) + 2: receive exactly what sparda_route writes.
 * One launch (the attention kernel routes each 64-token window itself, with
 * the router's code, so lists and output equal the two-call sequence bit for
 * bit) for bf16, D = Df = 64, bs 32 or 64, min(top_k, NB) <= 8, Hq/Hkv <= 4,
 * ceil(T/bs) <= 1024, 16-byte aligned rows. Other shapes run the router and
 * the prefill as two launches and need sel / n_sel as the hand-off buffers
 * (SPARDA_ERR_SHAPE without them).
 */
SPARDA_API int sparda_prefill_routed(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                                     const void* k, const void* v,
                                     int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                                     int dtype,
                                     const void* forecast, int f_dtype,
                                     int64_t f_sb, int64_t f_st, int64_t f_sh,
                                     const float* protos, int64_t Df,
                                     int64_t top_k, float route_scale,
                                     int32_t* sel, int32_t* n_sel, int64_t sel_cap,
                                     int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                                     int64_t block_size, int causal, float scale,
                                     void* out, int64_t out_sb, int64_t out_st,
                                     void* stream);

/*
 * Chunked-gather prefill: sparda_select_chunked's lists and causal
 * sparda_prefill over them, in one launch where the shape allows (bf16,
 * D = 64, block_size 64, Hq/Hkv in 1..4, 16-byte aligned q/k/v rows): each
 * workgroup builds its 64-token query block's list in LDS and attends every
 * token of the block over it. Replaces SparseAttention._forward_chunked_gather
 * after its router call (model/attention/sparse.py:303-364).
 *   q, k, v, out, scale, dtype: as in sparda_prefill (causal)
 *   topk: [B,Hkv,T,top_k_width] int32, sparda_route's non-causal top-k; NULL:
 *         the static window (the reference's chunked path without a forecast)
 *   sel, n_sel: optional [B,Hkv,T,sel_cap] / [B,Hkv,T], min(NB, top_k+2) <=
 *         sel_cap <= 34: receive exactly what sparda_select_chunked writes.
 *         Other shapes run sparda_select_chunked + sparda_prefill as two
 *         launches through them, and fail without them.
 * The output equals sparda_prefill over the same lists within rounding (the
 * one-launch kernel sums in another order), not bit for bit.
 */
SPARDA_API int sparda_prefill_chunked(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                                      const void* k, const void* v,
                                      int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                                      int dtype,
                                      const int32_t* topk, int64_t top_k_width, int64_t top_k,
                                      int32_t* sel, int32_t* n_sel, int64_t sel_cap,
                                      int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                                      int64_t block_size, float scale,
                                      void* out, int64_t out_sb, int64_t out_st,
                                      void* stream);

/*
 * Block-sparse GQA prefill with an explicit additive mask and, optionally, the
 * attention weights. Replaces the masked-SDPA path of
 * SparseAttention._forward_masked_sdpa with `mask` and return_attn_weights
 * (model/attention/sparse.py:206-221 dense, 255-281 sparse), and the dense
 * backend's weights output used by scripts/benchmark_forecast.py:86-93.
 *   allowed(b,g,t,s) as in sparda_prefill (sel == NULL: every block;
 *   repeated or out-of-range list entries count once / not at all);
 *   score = q.k_s * scale + mask[b,h,t,s] on allowed keys, -inf elsewhere;
 *   weights[b,h,t,s] = softmax_s(score) (0 outside the allowed set),
 *   out[b,t,h*D+d] = sum_s weights[b,h,t,s] v_s[d].
 *   mask: optional, fp32 or the input dtype, element strides (m_sb, m_sh,
 *     m_st, m_ss) over [B, Hq, T, T] (0 to broadcast a dimension), h the
 *     query head; natural-log units, as added before the reference's softmax.
 *   weights: optional [B,Hq,T,T] of dtype, strides (w_sb, w_sh, w_st, 1).
 * A general (VALU) kernel: for the evaluation and debugging callers of these
 * options, not the sparse fast path (sparda_prefill).
 */
SPARDA_API int sparda_prefill_masked(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                                     const void* k, const void* v,
                                     int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                                     int dtype,
                                     const int32_t* sel, const int32_t* n_sel, int64_t sel_cap,
                                     int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                                     int64_t block_size, int causal, float scale,
                                     const void* mask, int mask_dtype,
                                     int64_t m_sb, int64_t m_sh, int64_t m_st, int64_t m_ss,
                                     void* out, int64_t out_sb, int64_t out_st,
                                     void* weights, int64_t w_sb, int64_t w_sh, int64_t w_st,
                                     void* stream);

/* Workspace bytes sparda_decode needs for these sizes. */
SPARDA_API size_t sparda_decode_workspace_bytes(int64_t B, int64_t S, int64_t Hq,
                                                int64_t Hkv, int64_t D,
                                                int64_t block_size, int64_t top_k);

/*
 * One single-token decode step of the sparse attention layer.
 * Replaces SparseAttention._forward_decode_gather (model/attention/sparse.py:99-183)
 * after the projections: block compression of the whole cache (sparse.py:133-135),
 * forecast routing (sparse.py:139-141), sink + current block (126-130),
 * removal of future blocks (150-151), the gather (157) and masked SDPA over the
 * gathered keys (160-181), as split-K attention over the selected blocks with
 * a merge (two kernel launches, no host synchronisation).
 * Dense over all S keys when NB <= top_k+2 (sparse.py:113-123);
 * static window {0} U [cb-k+1, cb] when forecast == NULL (sparse.py:142-147).
 *   q:        [B,Hq,D] of dtype, strides (q_sb, q_sh, 1) (position S-1)
 *   k_cache, v_cache: [B,Smax,Hkv,D] strides (kv_sb, kv_ss, kv_sh, 1);
 *             tokens [0,S) are valid, S includes the new token
 *   forecast: [B,Hkv,Df] of f_dtype, strides (f_sb, f_sh, 1), or NULL
 *   protos_in: optional cached prototypes [B,NB,Hkv,D] fp32 (skips the
 *             compression pass; must equal sparda_compress of the cache)
 *   protos_out: optional, receives the prototypes computed this step
 *   sel_out/n_sel_out: optional [B,Hkv,top_k+2] / [B,Hkv] int32
 *   out: [B,Hq*D] of dtype, stride out_sb
 *   workspace: >= sparda_decode_workspace_bytes(), 256-byte aligned; it
 *             holds the block scores of the step (no state survives the call). Calls sharing one workspace
 *             must be ordered on one stream.
 */
SPARDA_API int sparda_decode(const void* q, int64_t q_sb, int64_t q_sh,
                             const void* k_cache, const void* v_cache,
                             int64_t kv_sb, int64_t kv_ss, int64_t kv_sh,
                             int dtype,
                             const void* forecast, int f_dtype, int64_t f_sb, int64_t f_sh,
                             int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D,
                             int64_t block_size, int64_t top_k, int routing, float scale,
                             const float* protos_in, float* protos_out,
                             int32_t* sel_out, int32_t* n_sel_out,
                             void* out, int64_t out_sb,
                             void* workspace, size_t workspace_bytes,
                             void* stream);

/*
 * sparda_decode without a workspace argument. No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops and harnesses that forbid hipMalloc). The
 * step's block scores live in a static device array of 1 MiB per GPU
 * (B * Hkv * ceil(S/block_size) <= 262,144 scores; larger steps return
 * SPARDA_ERR_CAPACITY). The call itself allocates nothing; the caller passes
 * every input and output as for sparda_decode, whose arguments and results
 * this matches exactly. Uses the current device's array: the stream must
 * belong to the current device, and calls that overlap in time on one GPU
 * race on the array.
 */
SPARDA_API int sparda_decode_noalloc(const void* q, int64_t q_sb, int64_t q_sh,
                                     const void* k_cache, const void* v_cache,
                                     int64_t kv_sb, int64_t kv_ss, int64_t kv_sh,
                                     int dtype,
                                     const void* forecast, int f_dtype, int64_t f_sb, int64_t f_sh,
                                     int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D,
                                     int64_t block_size, int64_t top_k, int routing, float scale,
                                     const float* protos_in, float* protos_out,
                                     int32_t* sel_out, int32_t* n_sel_out,
                                     void* out, int64_t out_sb,
                                     void* stream);

/*
 * Single-token decode attention over a given block selection.
 * Replaces the gather + validity mask + SDPA over selected blocks of
 * SparseAttention._forward_decode_gather (model/attention/sparse.py:154-181)
 * and of the offload backends (model/attention/offload.py:247-278,
 * model/attention/async_offload.py:380-489).
 *   sel/n_sel: [B,Hkv,sel_cap] / [B,Hkv] int32 (sel_cap <= 34); blocks
 *     outside [0, (S-1)/bs] are skipped, n_sel must be >= 1 and should include
 *     the block of position S-1. sel == NULL: every block of [0, S) (dense,
 *     any length).
 *   compact == 0: k/v are the cache [B,Smax,Hkv,D] strides (kv_sb, kv_ss,
 *     kv_sh, 1), blocks are read in place.
 *   compact == 1: k/v are compact block buffers, slot i of (b, g) holding
 *     block sel[b,g,i]: element (b, g, i, r, d) at
 *     b*kv_sb + g*kv_sh + (i*bs + r)*kv_ss + d (sparda_offload_fetch output).
 *   k_new/v_new: optional [B,Hkv,D] (strides new_sb, new_sh, 1): the key and
 *     value of position S-1, used instead of what k/v hold there.
 *   q: [B,Hq,D]; out: [B,Hq*D] stride out_sb. 16-byte aligned rows.
 *   workspace (optional, 16-byte aligned, may be NULL): with sel == NULL on
 *     the matrix-core attention (bf16, D = 64, blocks of 64 or 32 keys) the
 *     blocks are split over workgroups, four per workgroup (more when
 *     workspace_bytes / (B*Hkv*(Hq/Hkv)*(D+2)*4) splits do not cover them),
 *     whose partials a second launch merges (flash-decoding); NULL or too
 *     small for two splits: one workgroup per (sequence, KV head). The split
 *     changes no selection, only the order in which partial softmax sums are
 *     combined. sparda_decode_dense_workspace_bytes gives the size of the
 *     full split for a length.
 */
SPARDA_API int sparda_decode_selected(const void* q, int64_t q_sb, int64_t q_sh,
                                      const void* k, const void* v,
                                      int64_t kv_sb, int64_t kv_ss, int64_t kv_sh,
                                      int dtype, int compact,
                                      const int32_t* sel, const int32_t* n_sel, int64_t sel_cap,
                                      const void* k_new, const void* v_new,
                                      int64_t new_sb, int64_t new_sh,
                                      int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D,
                                      int64_t block_size, float scale,
                                      void* out, int64_t out_sb,
                                      void* workspace, size_t workspace_bytes, void* stream);

/*
 * Workspace bytes for which a dense decode (sparda_decode_selected with sel
 * NULL, sparda_decode_at / sparda_decode_at_prefetch with sel NULL and
 * window_k 0) of up to max_len tokens takes its full split: four blocks
 * per workgroup (more only past 4096 workgroups per (sequence, KV head)),
 * so that which split holds a block, and with it the result, depends on the
 * length and not on max_len; 0 when it would not split. Only the
 * matrix-core attention (bf16, D = 64, blocks of 64 or 32 keys) splits;
 * other calls ignore a workspace. No counterpart in the reference: the
 * reference attends densely with SDPA (model/attention/offload.py:180-200,
 * model/attention/async_offload.py:399-417).
 */
SPARDA_API size_t sparda_decode_dense_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                                      int64_t max_len, int64_t block_size);

/*
 * Teacher block mass for routing-quality evaluation: the dense attention
 * probability of each query row on each KV block, averaged over the Hq/Hkv
 * query heads of a KV head (TeacherBlockSelector.forward, model/forecast.py:
 * 141-193, steps 1-3, computed from q and k without materialising the
 * [B,Hq,T,T] weights the reference takes as input).
 *   q: [B,T,Hq,64], k: [B,T,Hkv,64] bf16 (post-RoPE), element strides
 *      (sb, st, sh, 1), rows 16-byte aligned; Hq / Hkv in {1, 2, 3}.
 *   mass: [B,Hkv,T,NB] fp32, NB = ceil(T/64); causal: keys s <= t and blocks
 *      j > t/64 hold 0. scale = 1/sqrt(64) in the reference.
 */
SPARDA_API int sparda_teacher_mass(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k,
                                   int64_t k_sb, int64_t k_st, int64_t k_sh, int dtype, int64_t B, int64_t T,
                                   int64_t Hq, int64_t Hkv, int64_t D, int64_t block_size, int causal, float scale,
                                   float* mass, void* stream);

/*
 * Producer of one layer's attention inputs, fused: RMSNorm + the q, k, v and
 * forecast projections + RoPE of q and k. Replaces, for the HIP model, the
 * sequence attn_norm -> ForecastProjection -> wq / wk / wv -> RotaryEmbedding
 * of TransformerBlock.forward (model/transformer.py:104-107, 118-125;
 * model/norm.py:15-21; model/forecast.py:30-40; model/attention/base.py:38-52;
 * model/rope.py:34-65). Head dim 64.
 *   x: [M, C] bf16 rows (row stride x_stride_row), M = B * T, row b*T + t is
 *      position pos0 + t.
 *   w: [Nq + 2*Nk + Nf, C] bf16 = [wq; wk; wv; wf] with the RMSNorm weight
 *      folded into the columns (w[n, c] * norm_weight[c]).
 *   rope_cos / rope_sin: [rope_len, 32] fp32 tables (angle pos * theta^(-2i/64)).
 *   q: [M, Nq], k, v: [M, Nk] bf16; f: [M, Nf] of f_dtype (SPARDA_BF16 / F32).
 *   y = (x w^T) / sqrt(mean(x^2) + eps) per row; q and k rotated by position.
 */
SPARDA_API int sparda_produce(const void* x, int64_t x_stride_row, const void* w, int64_t M, int64_t C,
                              int64_t Nq, int64_t Nk, int64_t Nf, float eps, const float* rope_cos,
                              const float* rope_sin, int64_t rope_len, int64_t T, int64_t pos0, void* q, void* k,
                              void* v, void* f, int f_dtype, void* stream);

/*
 * Feed-forward half of a block for decode-sized batches, fused: RMSNorm +
 * SwiGLU + residual. Replaces, for the HIP model, ffn_norm -> SwiGLU -> add of
 * TransformerBlock.forward (model/transformer.py:18-31, 126-129;
 * model/norm.py:15-21) when M = B*T <= 16.
 *   x: [M, C] bf16 rows (stride x_stride_row), C a multiple of 128 up to 1024.
 *   w_gate_up: [2F, C] bf16 = [w_gate; w_up] with the RMSNorm weight folded
 *     into the columns (w[f, c] * norm_weight[c]); w_down: [C, F] bf16, F a
 *     multiple of 128 up to 2048.
 *   act: [M, F] bf16 scratch (the SwiGLU activation); out: [M, C] bf16
 *     (stride out_stride_row), out = x + w_down . (silu(g) * u),
 *     g / u = (x . w_gate_up rows) / sqrt(mean(x^2) + eps), each projection,
 *     silu, product and the down projection rounded to bf16 as the unfused
 *     sequence rounds them.
 */
SPARDA_API int sparda_ffn_decode(const void* x, int64_t x_stride_row, const void* w_gate_up, const void* w_down,
                                 int64_t M, int64_t C, int64_t F, float eps, void* act, void* out,
                                 int64_t out_stride_row, void* stream);

/*
 * The final RMSNorm and the output projection of a decode-sized batch in one
 * kernel: logits = final_norm(x) . W^T (SparDAResearchModel.forward,
 * model/model.py:79-157, with the tied embedding weight; RMSNorm as
 * model/norm.py:15-21), as out[m, n] = (x[m] . W'[n]) / sqrt(mean(x[m]^2) + eps)
 * in fp32, rounded to bf16 once, with W' = W * norm_weight (folded into the
 * columns by the caller).
 *   x: [M, C] bf16 (stride x_stride_row), M in 1..16, C a multiple of 128 up
 *     to 1024; w: [N, C] bf16 contiguous, N a multiple of 16
 *   out: [M, N] bf16 (stride out_stride_row)
 */
SPARDA_API int sparda_norm_gemv(const void* x, int64_t x_stride_row, const void* w, int64_t M, int64_t C,
                                int64_t N, float eps, void* out, int64_t out_stride_row, void* stream);

/*
 * The attention's output projection and residual of a decode-sized batch in
 * one kernel: out = x + attn . wo^T (TransformerBlock.forward,
 * model/transformer.py:118-126: x + attention(...) whose last step is
 * self.wo(...), model/attention/sparse.py:183), rounded as the unfused pair
 * rounds (the projection to bf16, then the sum).
 *   a: [M, K] bf16 (stride a_stride_row), M in 1..16, K a multiple of 128 up
 *     to 2048; w: [N, K] bf16 contiguous (nn.Linear layout), N a multiple of 16
 *   res / out: [M, N] bf16 (strides res_stride_row / out_stride_row)
 */
SPARDA_API int sparda_rows_residual(const void* a, int64_t a_stride_row, const void* w, int64_t M, int64_t K,
                                    int64_t N, const void* res, int64_t res_stride_row, void* out,
                                    int64_t out_stride_row, void* stream);

/*
 * fp32 block sums of a device KV cache, kept current across decode steps so
 * that decode selection (sparda_select_decode) reads the sums instead of
 * recompressing the whole cache every step as the reference's decode does
 * (KVBlockCompressor over all S keys, model/attention/sparse.py:133-135 with
 * model/forecast.py:66-78). prototype = sum / bs, so the sums give the same
 * prototypes as sparda_compress bit for bit.
 *   k: [B,S,Hkv,D] cache base, strides (sb, st, sh, 1); tokens pos..pos+n-1
 *     are read.
 *   block_sums: [B,nb_stride,Hkv,D] fp32. A block whose first token is in
 *     [pos, pos+n) is summed from zero; a block entered mid-way continues its
 *     stored sum. With pos = j*bs the blocks j.. are recomputed from scratch,
 *     which makes a per-step update of the current block idempotent.
 */
SPARDA_API int sparda_block_sums(const void* k, int dtype, int64_t sb, int64_t st, int64_t sh,
                                 int64_t B, int64_t Hkv, int64_t D, int64_t pos, int64_t n,
                                 int64_t block_size, int64_t nb_stride, float* block_sums, void* stream);

/*
 * Decode-time block selection from fp32 block sums (prototype = sum / bs).
 * Replaces the selection step of AsyncForecastOffloadAttention.prefetch
 * (model/attention/async_offload.py:241-260) and of
 * ForecastOffloadAttention._forward_offload_decode (offload.py:218-240)
 * without the full-K host-to-device copy and recompression they do.
 *   block_sums: [B,nb_stride,Hkv,D] fp32 covering tokens [0, len)
 *     (sparda_offload_append / sparda_offload_rebuild_sums)
 *   pos: the query position (len for the one-token lookahead of a prefetch);
 *     own = pos / bs. If own + 1 <= top_k + 2 every block 0..own is selected.
 *     Otherwise blocks j < ceil(len/bs) are scored as in sparda_route (mask
 *     j > pos/bs in SPARDA_ROUTE_ABSOLUTE, j > 0 in SPARDA_ROUTE_REFERENCE)
 *     and sel = ascending {0, own} U top-k, ties by lower index.
 *   forecast: [B,Hkv,D] strides (f_sb, f_sh, 1), D in {16, 32, 64, 128};
 *   sel/n_sel: [B,Hkv,sel_cap] / [B,Hkv]
 */
SPARDA_API int sparda_select_decode(const void* forecast, int f_dtype, int64_t f_sb, int64_t f_sh,
                                    const float* block_sums,
                                    int64_t B, int64_t Hkv, int64_t D, int64_t nb_stride,
                                    int64_t len, int64_t pos, int64_t block_size, int64_t top_k,
                                    int routing, float scale,
                                    int32_t* sel, int32_t* n_sel, int64_t sel_cap, void* stream);

/*
 * One decode step with cached prototypes, in a single launch. Replaces the
 * decode branch of SparseAttention.forward after the projections
 * (model/attention/sparse.py:99-183) for a cache whose fp32 block sums are kept
 * current (PrototypeKVCache): instead of recompressing all S keys
 * (sparse.py:133-135) the blocks are scored from the sums (prototype = sum /
 * bs, model/forecast.py:66-78, scored as sparda_select_decode does), the
 * ascending {0, cb} U top-k selected (sparse.py:126-154; every block 0..cb
 * while cb + 1 <= top_k + 2) and attended in place (sparse.py:157-181).
 *   q: [B,Hq,D] at position S-1; k/v: [B,Smax,Hkv,D] strides (kv_sb, kv_ss,
 *     kv_sh, 1), rows 16-byte aligned; forecast: [B,Hkv,D] strides (f_sb,
 *     f_sh, 1); D in {16, 32, 64, 128}
 *   block_sums: [B,nb_stride,Hkv,D] fp32, 16-byte aligned, covering [0, S).
 *     With update_current != 0 the sums of the current block cb are first
 *     recomputed from its rows [cb*bs, S) in row order (what sparda_block_sums
 *     with pos = cb*bs does) and stored, so a caller that appended the token
 *     at S-1 needs no separate sums launch; the other blocks must be current.
 *   pos_dev: NULL, or an 8-byte aligned int64 in device memory: then the
 *     query is token *pos_dev (S = *pos_dev + 1, clamped into [1, S]) read
 *     when the kernel runs
 *   route_scale: the score scale (1/sqrt(D) in the reference); scale: the
 *     attention scale
 *   sel_out/n_sel_out: optional [B,Hkv,top_k+2] / [B,Hkv] int32 (together)
 *   out: [B,Hq*D] of dtype, stride out_sb
 */
SPARDA_API int sparda_decode_sums(const void* q, int64_t q_sb, int64_t q_sh, const void* k, const void* v,
                                  int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int dtype,
                                  const void* forecast, int f_dtype, int64_t f_sb, int64_t f_sh,
                                  float* block_sums, int64_t nb_stride, int update_current,
                                  int64_t B, int64_t S, const int64_t* pos_dev,
                                  int64_t Hq, int64_t Hkv, int64_t D, int64_t block_size, int64_t top_k,
                                  int routing, float scale, float route_scale,
                                  int32_t* sel_out, int32_t* n_sel_out, void* out, int64_t out_sb,
                                  void* stream);

/*
 * Decode steps at a device-held position, so that one recorded sequence of
 * launches (a HIP graph) serves every step of a generation loop. The
 * reference's loop (SparDAResearchModel.generate, model/model.py:159-195, one
 * forward per token through KVCache.update, model/attention/base.py:11-32, and
 * the decode branch of SparseAttention.forward, model/attention/sparse.py:99-183)
 * passes the cache length from the host every step; these entries read the
 * position p of the token being decoded from *pos_dev (an int64 in device
 * memory, 8-byte aligned) when the kernels run. The cache holds p + 1 tokens
 * (token p appended by the caller before the attention). p is clamped into
 * [0, max_len) (the RoPE table length for produce): a position outside it
 * never reads out of bounds, but its results are those of the clamped one.
 *
 * sparda_produce_at: sparda_produce with positions *pos_dev + t.
 * sparda_produce_cache_at: sparda_produce_at that also writes the rotated key
 *   and the value of row m as row p = *pos_dev + m % T (clamped into
 *   [0, max_len)) of sequence m / T in the caches [B,Smax,Hkv,64] bf16
 *   (strides (sb, st, sh, 1)), the append of KVCache.update
 *   (model/attention/base.py:19-29) done by the producer; decode-sized
 *   batches only (M <= 16). The block sums are left to the decode launch
 *   (sparda_decode_sums with update_current).
 * sparda_append_at: per sequence, writes k_new / v_new ([B,Hkv,D], strides
 *   (new_sb, new_sh, 1)) as row p of the caches [B,Smax,Hkv,D] (strides
 *   (sb, st, sh, 1); KVCache.update, model/attention/base.py:19-29) and
 *   recomputes the fp32 sums of the block holding p over [p - p % bs, p], as
 *   sparda_block_sums(k, ..., pos = p - p % bs, n = p % bs + 1) does. With
 *   k_new / v_new NULL only the sums are recomputed (v_cache may be NULL);
 *   with block_sums NULL only the rows are written.
 * sparda_select_decode_at: sparda_select_decode with len = p + 1, pos = p;
 *   with lookahead != 0, len = p, pos = p (the selection a prefetch makes
 *   before token p is appended, async_offload.py:196-260).
 * sparda_decode_at: sparda_decode_selected with S = p + 1 over the caller's
 *   list (sel / n_sel; compact != 0: the fetched block buffers of
 *   sparda_offload_fetch_at; k_new / v_new: the key and value of position p),
 *   or, with sel NULL and window_k > 0, the static window
 *   {0} U [cb - window_k + 1, cb] (cb = p / bs; every block while cb + 1 <=
 *   window_k + 2) that sparda_decode uses without a forecast, or every block
 *   (sel NULL, window_k 0; split over the workgroups a workspace allows, as
 *   in sparda_decode_selected).
 * sparda_offload_fetch_at: sparda_offload_fetch (gather kernel) with
 *   len = *len_dev, clamped into [0, max_seq].
 * sparda_offload_append_at: appends one token (k / v [B,Hkv,D], strides
 *   (new_sb, new_sh, 1)) as row *pos_dev of the arena through its device
 *   mapping (OffloadedKVCache.update, offload.py:67-77) and, with block_sums,
 *   recomputes that block's sums from the arena, as sparda_append_at does.
 */
SPARDA_API int sparda_produce_at(const void* x, int64_t x_stride_row, const void* w, int64_t M, int64_t C,
                                 int64_t Nq, int64_t Nk, int64_t Nf, float eps, const float* rope_cos,
                                 const float* rope_sin, int64_t rope_len, int64_t T, const int64_t* pos_dev,
                                 void* q, void* k, void* v, void* f, int f_dtype, void* stream);
SPARDA_API int sparda_produce_cache_at(const void* x, int64_t x_stride_row, const void* w, int64_t M, int64_t C,
                                       int64_t Nq, int64_t Nk, int64_t Nf, float eps, const float* rope_cos,
                                       const float* rope_sin, int64_t rope_len, int64_t T, const int64_t* pos_dev,
                                       void* q, void* k, void* v, void* f, int f_dtype, void* k_cache,
                                       void* v_cache, int64_t sb, int64_t st, int64_t sh, int64_t max_len,
                                       void* stream);
SPARDA_API int sparda_append_at(void* k_cache, void* v_cache, int dtype, int64_t sb, int64_t st, int64_t sh,
                                const void* k_new, const void* v_new, int64_t new_sb, int64_t new_sh, int64_t B,
                                int64_t Hkv, int64_t D, int64_t max_len, const int64_t* pos_dev,
                                int64_t block_size, int64_t nb_stride, float* block_sums, void* stream);
SPARDA_API int sparda_select_decode_at(const void* forecast, int f_dtype, int64_t f_sb, int64_t f_sh,
                                       const float* block_sums, int64_t B, int64_t Hkv, int64_t D,
                                       int64_t nb_stride, int64_t max_len, const int64_t* pos_dev,
                                       int64_t block_size, int64_t top_k, int routing, float scale,
                                       int32_t* sel, int32_t* n_sel, int64_t sel_cap, int lookahead,
                                       void* stream);
SPARDA_API int sparda_decode_at(const void* q, int64_t q_sb, int64_t q_sh, const void* k, const void* v,
                                int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int dtype, int compact,
                                const int32_t* sel, const int32_t* n_sel, int64_t sel_cap, int64_t window_k,
                                const void* k_new, const void* v_new, int64_t new_sb, int64_t new_sh, int64_t B,
                                int64_t max_len, const int64_t* pos_dev, int64_t Hq, int64_t Hkv, int64_t D,
                                int64_t block_size, float scale, void* out, int64_t out_sb, void* workspace,
                                size_t workspace_bytes, void* stream);
SPARDA_API int sparda_offload_fetch_at(sparda_offload_t h, const int32_t* sel, const int32_t* n_sel,
                                       int64_t sel_cap, int64_t block_size, const int64_t* len_dev, void* k_dst,
                                       void* v_dst, void* stream);

/*
 * The next layer's prefetch carried by a decode attention launch.
 * The reference issues the prefetch of layer L+1 on a transfer stream before
 * layer L's attention (AsyncForecastOffloadAttention.prefetch,
 * model/attention/async_offload.py:170-294, called from
 * model/transformer.py:110-115) so that the copy runs under layer L's
 * attention and FFN. Here the same selection and copy run as extra
 * workgroups of layer L's sparda_decode_at launch, one per (sequence, KV
 * head), beside its attention workgroups: one stream, no cross-stream
 * join, capturable. The results equal sparda_select_decode_at (lookahead)
 * followed by sparda_offload_fetch_at (len_dev = pos_dev) bit for bit.
 *   arena: the next layer's arena; its batch, KV heads, head dim and dtype
 *     must be those of the attended layer
 *   forecast: [B,Hkv,D] (strides f_sb, f_sh, 1), the forecast that routes
 *     the next layer
 *   block_sums: the next layer's [B,nb_stride,Hkv,D] fp32 sums (16-byte
 *     aligned) covering the tokens before p
 *   top_k, routing, scale: as sparda_select_decode_at (scale: the routing
 *     scale)
 *   sel / n_sel: [B,Hkv,sel_cap] / [B,Hkv] int32 receiving the selection
 *   k_dst / v_dst: [B,Hkv,sel_cap,block_size,D] compact buffers (16-byte
 *     aligned) receiving the blocks
 */
typedef struct sparda_prefetch_args {
    sparda_offload_t arena;
    const void* forecast;
    int f_dtype;
    int64_t f_sb, f_sh;
    const float* block_sums;
    int64_t nb_stride;
    int64_t top_k;
    int routing;
    float scale;
    int32_t* sel;
    int32_t* n_sel;
    int64_t sel_cap;
    void* k_dst;
    void* v_dst;
    int stage;   /* 0: selection and copy; 1: the selection only (into sel / n_sel);
                    2: the copy only, of the selection in sel / n_sel (left there by a
                    stage-1 launch earlier on the stream; forecast and block_sums unused) */
    int parts;   /* stage 2: the copy in `parts` shares (0 or 1: all of it), of which
                    this launch copies share `part`: the slots s with s % parts == part */
    int part;
} sparda_prefetch_args;

/*
 * sparda_decode_at (same arguments, same result) whose launch also carries
 * `next`'s prefetch at the same position p = *pos_dev (the selection before
 * token p is appended to the next layer). Needs the matrix-core attention:
 * bf16, D = 64, blocks of 64 or 32 keys, 16-byte aligned q rows.
 */
/*
 * sparda_offload_append_at (same arguments, same result) whose launch also
 * carries `next`'s prefetch stage (normally 1, the selection, so that the
 * attention launch that follows carries only the copy, stage 2). max_len:
 * the positions' bound, as sparda_decode_at's (the selection clamps p into
 * [0, max_len - 1]). Needs bf16, D = 64.
 */
SPARDA_API int sparda_offload_append_at_prefetch(sparda_offload_t h, const void* k, const void* v, int64_t new_sb,
                                                 int64_t new_sh, const int64_t* pos_dev, int64_t block_size,
                                                 float* block_sums, int64_t max_len,
                                                 const sparda_prefetch_args* next, void* stream);

SPARDA_API int sparda_decode_at_prefetch(const void* q, int64_t q_sb, int64_t q_sh, const void* k, const void* v,
                                         int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int dtype, int compact,
                                         const int32_t* sel, const int32_t* n_sel, int64_t sel_cap,
                                         int64_t window_k, const void* k_new, const void* v_new, int64_t new_sb,
                                         int64_t new_sh, int64_t B, int64_t max_len, const int64_t* pos_dev,
                                         int64_t Hq, int64_t Hkv, int64_t D, int64_t block_size, float scale,
                                         void* out, int64_t out_sb, const sparda_prefetch_args* next,
                                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * sparda_ffn_decode (same arguments, same result) whose two launches also
 * carry a share of the next layer's prefetch copy: gate_up_next and
 * down_next (either may be NULL) are stage-2 prefetch arguments (the copy of
 * the selection a stage-1 launch left in sel / n_sel) with `parts` / `part`
 * naming the share, at position p = *pos_dev (the arena length p, as in
 * sparda_decode_at_prefetch); block_size: the arena's blocks. The arenas'
 * batch must be M (one row per sequence). No counterpart in the reference:
 * it spreads the copy that transformer.py:110-115 issues on a transfer
 * stream over the attention and feed-forward launches of the same layer.
 */
SPARDA_API int sparda_ffn_decode_prefetch(const void* x, int64_t x_stride_row, const void* w_gate_up,
                                          const void* w_down, int64_t M, int64_t C, int64_t F, float eps, void* act,
                                          void* out, int64_t out_stride_row, const sparda_prefetch_args* gate_up_next,
                                          const sparda_prefetch_args* down_next, const int64_t* pos_dev,
                                          int64_t block_size, void* stream);
SPARDA_API int sparda_offload_append_at(sparda_offload_t h, const void* k, const void* v, int64_t new_sb,
                                        int64_t new_sh, const int64_t* pos_dev, int64_t block_size,
                                        float* block_sums, void* stream);

/*
 * Host-resident KV cache of one layer: pinned host arena (hipHostMalloc,
 * mapped) of K and V, each [B][Hkv][max_seq][D] in `dtype`, zero-filled.
 * Replaces the pinned cpu_k / cpu_v of OffloadedKVCache
 * (model/attention/offload.py:29-65); the library owns the memory until
 * sparda_offload_destroy. A handle is not re-entrant: calls on one handle
 * must come from one host thread.
 */
SPARDA_API int sparda_offload_create(int64_t B, int64_t max_seq, int64_t Hkv, int64_t D, int dtype,
                                     sparda_offload_t* out);
SPARDA_API int sparda_offload_destroy(sparda_offload_t h);
/* Host addresses of the K and V arenas ([B][Hkv][max_seq][D] each). */
SPARDA_API int sparda_offload_host(sparda_offload_t h, void** k_host, void** v_host);

/*
 * Append tokens [pos, pos+n) from device memory to the arena.
 * Replaces OffloadedKVCache.update (model/attention/offload.py:67-77).
 *   k, v: [B,n,Hkv,D] device, strides (sb, st, sh, 1)
 *   block_sums: optional [B,ceil(max_seq/bs),Hkv,D] fp32 device array; the
 *     blocks touched get their sums continued sequentially from the block
 *     start (restarted at 0 when pos <= the block start).
 */
SPARDA_API int sparda_offload_append(sparda_offload_t h, const void* k, const void* v,
                                     int64_t sb, int64_t st, int64_t sh, int64_t pos, int64_t n,
                                     int64_t block_size, float* block_sums, void* stream);

/* Recompute block_sums of tokens [0, len) from the arena (through its device mapping). */
SPARDA_API int sparda_offload_rebuild_sums(sparda_offload_t h, int64_t len, int64_t block_size,
                                           float* block_sums, void* stream);

/*
 * Copy selected blocks (token rows below len) from the arena into compact
 * device buffers k_dst/v_dst [B][Hkv][sel_cap][bs][D] (contiguous): slot i of
 * (b, g) receives block sel[b,g,i] for i < n_sel[b,g]; rows at or beyond len
 * and unused slots are not written.
 * Replaces OffloadedKVCache.transfer_selected_blocks (offload.py:83-123) and
 * AsyncOffloadedKVCache.async_transfer_selected_blocks (async_offload.py:55-112):
 * no host gather, no per-call pinning. method: SPARDA_FETCH_KERNEL (never
 * waits; graph-capturable) or SPARDA_FETCH_DMA (sel_cap <= 1024). The DMA
 * form blocks the calling thread: it copies the selection to pinned host
 * memory and calls hipStreamSynchronize(stream) before it can issue one
 * hipMemcpyAsync per run of consecutive blocks, so it returns only after
 * everything queued on `stream` before it has finished, and it must not be
 * called under stream capture.
 */
SPARDA_API int sparda_offload_fetch(sparda_offload_t h, const int32_t* sel, const int32_t* n_sel,
                                    int64_t sel_cap, int64_t block_size, int64_t len, int method,
                                    void* k_dst, void* v_dst, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPARDA_H */
