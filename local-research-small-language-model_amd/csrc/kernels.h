// Internal launcher declarations (host side). The extern "C" layer in abi.cpp
// validates arguments and calls these; each returns 0 or a status code.
#pragma once

#include "common.h"

namespace sparda {

int launch_compress(const void* k, int dtype, int64_t B, int64_t S, int64_t H, int64_t D,
                    int64_t sb, int64_t ss, int64_t sh, int64_t bs, float* protos,
                    hipStream_t stream);

int launch_route(const void* f, int fdtype, int64_t fsb, int64_t fst, int64_t fsh,
                 const float* protos, int64_t B, int64_t Tq, int64_t H, int64_t Df, int64_t NB,
                 int64_t bs, int ke, int causal, int64_t score_pos0, int64_t query_pos0,
                 float scale, int32_t* topk, float* scores, int32_t* sel, int32_t* n_sel,
                 int cap, hipStream_t stream);

// forecast routing folded into the compacted bf16 prefill (prefill_compact.hip)
struct CompactRoute {
    const void* f;          // forecast [B, T, Hkv, 64], element strides (fsb, fst, fsh, 1)
    int64_t fsb, fst, fsh;
    const float* protos;    // [B, ceil(T/bs), Hkv, 64] fp32, contiguous
    int ke;                 // router picks per token, <= 8
    float scale;            // router score scale
    int32_t* sel;           // optional: the router's lists [B, Hkv, T, cap] and counts [B, Hkv, T]
    int32_t* n_sel;
    int cap;
};
bool prefill_routed_supported(int dtype, int f_dtype, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t Df,
                              int64_t bs, int64_t ke, int64_t q_sb, int64_t q_st, int64_t q_sh, int64_t kv_sb,
                              int64_t kv_st, int64_t kv_sh, int64_t out_sb, int64_t out_st, const void* q,
                              const void* k, const void* v, const void* out, const float* protos);
int launch_prefill_routed(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k, const void* v,
                          int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int f_dtype, const CompactRoute& rt,
                          int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t bs, int causal, float scale,
                          void* out, int64_t out_sb, int64_t out_st, hipStream_t stream);

// copy the device's status word (SPARDA_STATUS_* bits) to out, clearing it when asked
int launch_read_status(uint32_t* out, int clear, hipStream_t stream);

// dense (no selection lists) bf16 prefill, D = 64 (prefill_dense.hip)
bool prefill_dense_supported(int dtype, int64_t Hq, int64_t Hkv, int64_t D, int64_t q_sb, int64_t q_st,
                             int64_t q_sh, int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int64_t out_sb,
                             int64_t out_st, const void* q, const void* k, const void* v, const void* out);
int launch_prefill_dense(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k, const void* v,
                         int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int64_t B, int64_t T, int64_t Hq,
                         int64_t Hkv, int causal, float scale, void* out, int64_t out_sb, int64_t out_st,
                         hipStream_t stream);
// the chunked-gather prefill over 64-key blocks: each query block's list built in
// the launch from the non-causal top-k (or the static window), causal attention
// over it (same shape limits as the dense kernel)
int launch_prefill_chunked(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k, const void* v,
                           int64_t kv_sb, int64_t kv_st, int64_t kv_sh, const int32_t* topk, int64_t ke,
                           int64_t top_k, int32_t* sel, int32_t* n_sel, int64_t cap, int64_t B, int64_t T,
                           int64_t Hq, int64_t Hkv, float scale, void* out, int64_t out_sb, int64_t out_st,
                           hipStream_t stream);

int launch_produce(const void* x, int64_t x_st, const void* w, int64_t M, int64_t C, int64_t Nq, int64_t Nk,
                   int64_t Nf, float eps, const float* cosv, const float* sinv, int64_t T, int64_t pos0,
                   void* q, void* k, void* v, void* f, int f_dtype, hipStream_t stream,
                   const int64_t* pos_dev = nullptr, int64_t rope_len = 0, void* kc = nullptr,
                   void* vc = nullptr, int64_t c_sb = 0, int64_t c_st = 0, int64_t c_sh = 0, int64_t cap = 0);

// decode-sized feed-forward half of a block: RMSNorm (folded) + SwiGLU + residual
// out[m, n] = bf16((x[m] . W'[n]) / rms(x[m])) for M <= 16 rows: W' [N, C] bf16, C <= 1024
int launch_norm_gemv(const void* x, int64_t x_st, const void* w, int64_t M, int64_t C, int64_t N, float eps,
                     void* out, int64_t out_st, hipStream_t stream);
// out[m] = bf16(res[m] + bf16(a[m] . W^T)) for M <= 16 rows: W [N, K] bf16, K <= 2048
int launch_rows_residual(const void* a, int64_t a_st, const void* w, int64_t M, int64_t K, int64_t N,
                         const void* res, int64_t res_st, void* out, int64_t out_st, hipStream_t stream);
struct PrefetchDev;
// pf_gate_up / pf_down (optional): a share of the next layer's prefetch copy
// (stage 2) carried by the gate/up and the down launch, pf_groups = B * Hkv
// workgroups each after the product workgroups
int launch_ffn_decode(const void* x, int64_t x_st, const void* w_gate_up, const void* w_down, int64_t M,
                      int64_t C, int64_t F, float eps, void* act, void* out, int64_t out_st, hipStream_t stream,
                      const PrefetchDev* pf_gate_up = nullptr, const PrefetchDev* pf_down = nullptr,
                      int64_t pf_groups = 0, const int64_t* pos_dev = nullptr);

int launch_teacher_mass(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k, int64_t k_sb,
                        int64_t k_st, int64_t k_sh, int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int causal,
                        float scale, float* mass, hipStream_t stream);

int launch_topk_scores(const float* scores, int64_t rows, int64_t NB, int ke, int algo,
                       int32_t* topk, hipStream_t stream);

// chunked-gather lists: per query block of bs rows, {0, bq} U the rows' top-k
// picks (topk [B,H,T,ke]; NULL: the static window of k blocks) up to bq, the
// lowest cap of them; NB = ceil(T / bs) <= 4096
int launch_chunk_select(const int32_t* topk, int64_t ke, int64_t B, int64_t H, int64_t T, int64_t bs, int64_t k,
                        int32_t* sel, int32_t* n_sel, int64_t cap, hipStream_t stream);
int launch_select_fixed(int mode, int64_t B, int64_t Tq, int64_t H, int64_t NB, int64_t bs,
                        int64_t k, int64_t query_pos0, int32_t* sel, int32_t* n_sel, int cap,
                        hipStream_t stream);

int launch_gather(const void* k, const void* v, int dtype, int64_t sb, int64_t sh, int64_t ss,
                  const int32_t* idx, int64_t B, int64_t H, int64_t S, int64_t D, int64_t n,
                  int64_t bs, void* ko, void* vo, hipStream_t stream);

int launch_prefill_weights(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k, const void* v,
                           int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int dtype, const int32_t* sel,
                           const int32_t* n_sel, int64_t cap, int64_t B, int64_t T, int64_t Hq, int64_t Hkv,
                           int64_t D, int64_t bs, int causal, float scale, const void* mask, int mask_dt,
                           int64_t m_sb, int64_t m_sh, int64_t m_st, int64_t m_ss, void* out, int64_t out_sb,
                           int64_t out_st, void* weights, int64_t w_sb, int64_t w_sh, int64_t w_st,
                           hipStream_t stream);

// Workspace carve-up of the decode step.
struct DecodeWs {
    float* scores;     // [B*Hkv*NB]
    size_t bytes;
};
DecodeWs decode_ws_layout(void* base, int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D,
                          int64_t bs, int64_t k);

// Argument checks of one decode step (before any HIP call); 0 or a negative status.
int check_decode_args(const void* q, const void* k_cache, const void* v_cache, int64_t kv_sb, int64_t kv_ss,
                      int64_t kv_sh, int dtype, const void* forecast, int f_dtype, int64_t B, int64_t S, int64_t Hq,
                      int64_t Hkv, int64_t D, int64_t block_size, int64_t top_k, int routing,
                      const int32_t* sel_out, const int32_t* n_sel_out, const void* out);

int launch_decode(const void* q, int64_t q_sb, int64_t q_sh, const void* kc, const void* vc,
                  int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int dtype, const void* f, int fdtype,
                  int64_t f_sb, int64_t f_sh, int64_t B, int64_t S, int64_t Hq, int64_t Hkv,
                  int64_t D, int64_t bs, int64_t k, int routing, float scale, const float* protos_in,
                  float* protos_out, int32_t* sel_out, int32_t* n_sel_out, void* out, int64_t out_sb,
                  const DecodeWs& ws, hipStream_t stream);

int launch_decode_selected(const void* q, int64_t q_sb, int64_t q_sh, const void* k, const void* v,
                           int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int dtype, int compact,
                           const int32_t* sel, const int32_t* n_sel, int64_t cap, const void* k_new,
                           const void* v_new, int64_t new_sb, int64_t new_sh, int64_t B, int64_t S,
                           int64_t Hq, int64_t Hkv, int64_t D, int64_t bs, float scale, void* out,
                           int64_t out_sb, hipStream_t stream, void* ws = nullptr, size_t ws_bytes = 0);
// bytes of the split partials a dense decode of S tokens uses (0: it does not split)
size_t decode_dense_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t S, int64_t bs);

int launch_select_decode(const void* f, int fdtype, int64_t f_sb, int64_t f_sh, const float* sums, int64_t B,
                         int64_t H, int64_t D, int64_t nb_stride, int64_t len, int64_t pos, int64_t bs,
                         int64_t k, int routing, float scale, int32_t* sel, int32_t* n_sel, int64_t cap,
                         hipStream_t stream, const int64_t* pos_dev = nullptr, int lookahead = 0);

// decode step selecting from fp32 block sums inside the attention kernel
// (S = host length, or *pos_dev + 1 clamped to S)
int launch_decode_sums(const void* q, int64_t q_sb, int64_t q_sh, const void* k, const void* v, int64_t kv_sb,
                       int64_t kv_ss, int64_t kv_sh, int dtype, const void* f, int f_dtype, int64_t f_sb,
                       int64_t f_sh, float* sums, int64_t nb_stride, int update_sums, int64_t B, int64_t S,
                       const int64_t* pos_dev, int64_t Hq, int64_t Hkv, int64_t D, int64_t bs, int64_t top_k,
                       int routing, float scale, float fscale, int32_t* sel_out, int32_t* n_sel_out, void* out,
                       int64_t out_sb, hipStream_t stream);

// The prefetch of the next layer's blocks carried by another launch as extra
// workgroups, one per (sequence, KV head): the selection of
// launch_select_decode with pos_dev and lookahead (blocks of [0, p) scored from
// the block sums; p = *pos_dev clamped into [0, pos_max]), then the copy of
// offload_fetch's gather kernel from the arena into the compact buffers
// (arena length p, clamped into [0, Smax]). stage: 0 both, 1 the selection
// only, 2 the copy only (of the selection a stage-1 launch left in sel/n_sel).
struct PrefetchDev {
    const void* f;          // forecast [B, H, D], element strides (f_sb, f_sh, 1)
    int64_t f_sb, f_sh;
    int f_bf16;
    const float* sums;      // [B, nb_stride, H, D] fp32, 16-byte aligned
    int64_t nb_stride;
    int64_t pos_max;
    int bs, k, cap, absolute, pow2;
    float scale;
    int32_t* sel;           // [B, H, cap]
    int32_t* n_sel;         // [B, H]
    const char* ak;         // arena device mappings, [B][H][Smax][row_bytes] each
    const char* av;
    int64_t H, Smax, row_bytes;
    char* dk;               // compact buffers [B][H][cap][bs][row_bytes] each
    char* dv;
    int stage;
    int parts, part;        // the copy of the slots s with s % parts == part (parts >= 1)
};
// the arena fields of a PrefetchDev (ak, av, H, Smax, row_bytes)
void offload_prefetch_dev(sparda_offload_t h, PrefetchDev* pf);
int64_t offload_batch(sparda_offload_t h);
int64_t offload_heads(sparda_offload_t h);
int64_t offload_head_dim(sparda_offload_t h);
int offload_dtype(sparda_offload_t h);

// attention at a device-held position: S = *pos_dev + 1 (clamped to S_max);
// the caller's list (sel), the window of window_k blocks, or every block.
// pf (optional, bf16 D = 64 matrix-core attention only): the next layer's
// prefetch in the same launch. ws (optional): the dense mode's split partials.
int launch_decode_at(const void* q, int64_t q_sb, int64_t q_sh, const void* k, const void* v, int64_t kv_sb,
                     int64_t kv_ss, int64_t kv_sh, int dtype, int compact, const int32_t* sel,
                     const int32_t* n_sel, int64_t cap, int64_t window_k, const void* k_new, const void* v_new,
                     int64_t new_sb, int64_t new_sh, int64_t B, int64_t S_max, const int64_t* pos_dev,
                     int64_t Hq, int64_t Hkv, int64_t D, int64_t bs, float scale, void* out, int64_t out_sb,
                     hipStream_t stream, const PrefetchDev* pf = nullptr, void* ws = nullptr,
                     size_t ws_bytes = 0);
// whether launch_decode_at takes the matrix-core attention (which can carry a prefetch)
bool decode_at_matrix_core(int dtype, int64_t D, int64_t bs, int64_t q_sb, int64_t q_sh, const void* q);

// host-resident KV arena (offload.hip)
constexpr int64_t kMaxFetchSlots = 1024;  // selection capacity of a DMA fetch
int offload_create(int64_t B, int64_t Smax, int64_t H, int64_t D, int dtype, sparda_offload_t* out);
int offload_destroy(sparda_offload_t h);
void offload_host(sparda_offload_t h, void** k, void** v);
int64_t offload_max_seq(sparda_offload_t h);
int offload_append(sparda_offload_t h, const void* k, const void* v, int64_t sb, int64_t st, int64_t sh,
                   int64_t pos, int64_t n, int64_t bs, float* sums, hipStream_t stream);
int offload_rebuild_sums(sparda_offload_t h, int64_t len, int64_t bs, float* sums, hipStream_t stream);

// fp32 block sums of tokens pos..pos+n-1; k points at token pos (strides sb, st, sh)
int launch_block_sums(const void* k, int dtype, int64_t sb, int64_t st, int64_t sh, int64_t pos,
                      int64_t n, int64_t B, int64_t H, int64_t D, int64_t bs, int64_t nb_stride,
                      float* sums, hipStream_t stream);
// decode-step append of k_new / v_new (optional) at row *pos_dev of the caches
// and the fp32 sums of the block holding it
int launch_append_at(void* kc, void* vc, int dtype, int64_t sb, int64_t st, int64_t sh, const void* k_new,
                     const void* v_new, int64_t n_sb, int64_t n_sh, int64_t B, int64_t H, int64_t D, int64_t bs,
                     int64_t max_len, int64_t nb_stride, const int64_t* pos_dev, float* sums, hipStream_t stream);
int offload_fetch(sparda_offload_t h, const int32_t* sel, const int32_t* n_sel, int64_t cap, int64_t bs,
                  int64_t len, int method, void* k_dst, void* v_dst, hipStream_t stream,
                  const int64_t* len_dev = nullptr);
// decode-step append of one token at row *pos_dev of the arena (device mapping) + its block's sums
int offload_append_at(sparda_offload_t h, const void* k, const void* v, int64_t n_sb, int64_t n_sh,
                      const int64_t* pos_dev, int64_t bs, float* sums, hipStream_t stream,
                      const PrefetchDev* pf = nullptr);

int launch_prefill(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k,
                   const void* v, int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int dtype,
                   const int32_t* sel, const int32_t* n_sel, int64_t cap, int64_t B, int64_t T,
                   int64_t Hq, int64_t Hkv, int64_t D, int64_t bs, int causal, float scale,
                   void* out, int64_t out_sb, int64_t out_st, hipStream_t stream);

}  // namespace sparda
