// extern "C" entry points of libsparda: argument validation (before any HIP
// call), then the kernel launchers. Status: 0 ok, >0 hipError_t, <0 argument error.
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "common.h"
#include "kernels.h"

namespace sparda {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return 0;
    return set_error(static_cast<int>(e), "%s: %s", what, hipGetErrorString(e));
}

static bool dtype_ok(int dt) { return dt == SPARDA_F32 || dt == SPARDA_BF16; }
static bool head_dim_ok(int64_t d) { return d == 16 || d == 32 || d == 64 || d == 128; }
constexpr int64_t kMaxTopK = 32;
constexpr int64_t kMaxGroupAbi = 16;

int check_decode_args(const void* q, const void* k_cache, const void* v_cache, int64_t kv_sb, int64_t kv_ss,
                      int64_t kv_sh, int dtype, const void* forecast, int f_dtype, int64_t B, int64_t S, int64_t Hq,
                      int64_t Hkv, int64_t D, int64_t block_size, int64_t top_k, int routing,
                      const int32_t* sel_out, const int32_t* n_sel_out, const void* out) {
    SPARDA_REQUIRE(q && k_cache && v_cache && out, SPARDA_ERR_NULL, "decode: null q/k/v/out");
    SPARDA_REQUIRE(!sel_out == !n_sel_out, SPARDA_ERR_NULL, "decode: sel_out and n_sel_out go together");
    SPARDA_REQUIRE(dtype_ok(dtype), SPARDA_ERR_DTYPE, "decode: dtype %d unsupported", dtype);
    SPARDA_REQUIRE(!forecast || dtype_ok(f_dtype), SPARDA_ERR_DTYPE, "decode: forecast dtype %d", f_dtype);
    SPARDA_REQUIRE(routing == SPARDA_ROUTE_REFERENCE || routing == SPARDA_ROUTE_ABSOLUTE, SPARDA_ERR_MODE,
                   "decode: unknown routing %d", routing);
    SPARDA_REQUIRE(B > 0 && S > 0 && Hq > 0 && Hkv > 0 && block_size > 0, SPARDA_ERR_SHAPE,
                   "decode: sizes must be positive");
    SPARDA_REQUIRE(head_dim_ok(D), SPARDA_ERR_SHAPE, "decode: head dim %lld not in {16,32,64,128}",
                   (long long)D);
    SPARDA_REQUIRE(Hq % Hkv == 0 && Hq / Hkv <= kMaxGroupAbi, SPARDA_ERR_SHAPE,
                   "decode: Hq must be a multiple of Hkv with ratio <= 16");
    SPARDA_REQUIRE(top_k >= 1 && top_k <= kMaxTopK, SPARDA_ERR_SHAPE, "decode: top_k out of range");
    SPARDA_REQUIRE(Hkv * D <= 2048, SPARDA_ERR_SHAPE, "decode: Hkv*D > 2048");
    const int64_t NB = cdiv(S, block_size);
    SPARDA_REQUIRE(NB <= 4096, SPARDA_ERR_SHAPE, "decode: more than 4096 blocks");
    SPARDA_REQUIRE(B <= 65535, SPARDA_ERR_SHAPE, "decode: B too large");
    const int64_t ve = 16 / (dtype == SPARDA_F32 ? 4 : 2);
    const bool al = (reinterpret_cast<uintptr_t>(k_cache) & 15u) == 0 &&
                    (reinterpret_cast<uintptr_t>(v_cache) & 15u) == 0 && kv_sb % ve == 0 && kv_ss % ve == 0 &&
                    kv_sh % ve == 0;
    SPARDA_REQUIRE(al, SPARDA_ERR_STRIDE, "decode: K/V cache rows must be 16-byte aligned");
    return 0;
}

}  // namespace sparda

using namespace sparda;

extern "C" {

SPARDA_API int sparda_version(void) { return 100; }

SPARDA_API const char* sparda_last_error(void) { return g_last_error; }

SPARDA_API int sparda_status(uint32_t* out, int clear, void* stream) {
    SPARDA_REQUIRE(out, SPARDA_ERR_NULL, "status: null out");
    return launch_read_status(out, clear != 0, static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_compress(const void* k, int dtype, int64_t B, int64_t S, int64_t H, int64_t D,
                               int64_t stride_b, int64_t stride_s, int64_t stride_h,
                               int64_t block_size, float* protos, void* stream) {
    SPARDA_REQUIRE(k && protos, SPARDA_ERR_NULL, "compress: null pointer");
    SPARDA_REQUIRE(dtype_ok(dtype), SPARDA_ERR_DTYPE, "compress: dtype %d unsupported", dtype);
    SPARDA_REQUIRE(B > 0 && S > 0 && H > 0 && D > 0 && block_size > 0, SPARDA_ERR_SHAPE,
                   "compress: sizes must be positive (B=%lld S=%lld H=%lld D=%lld bs=%lld)",
                   (long long)B, (long long)S, (long long)H, (long long)D, (long long)block_size);
    SPARDA_REQUIRE(D <= 1024, SPARDA_ERR_SHAPE, "compress: head dim %lld > 1024", (long long)D);
    SPARDA_REQUIRE(cdiv(S, block_size) <= 0x7fffffff && B <= 65535 && H <= 65535, SPARDA_ERR_SHAPE,
                   "compress: grid too large");
    SPARDA_REQUIRE(stride_b >= 0 && stride_s >= 0 && stride_h >= 0, SPARDA_ERR_STRIDE,
                   "compress: negative stride");
    return launch_compress(k, dtype, B, S, H, D, stride_b, stride_s, stride_h, block_size, protos,
                           static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_route(const void* forecast, int f_dtype, int64_t f_sb, int64_t f_st, int64_t f_sh,
                            const float* protos, int64_t B, int64_t Tq, int64_t H, int64_t Df, int64_t NB,
                            int64_t block_size, int64_t top_k, int causal, int64_t score_pos0,
                            int64_t query_pos0, float scale, int32_t* topk, float* scores, int32_t* sel,
                            int32_t* n_sel, int64_t sel_cap, void* stream) {
    SPARDA_REQUIRE(forecast && protos, SPARDA_ERR_NULL, "route: null forecast/protos");
    SPARDA_REQUIRE(topk || scores || sel, SPARDA_ERR_NULL, "route: no output requested");
    SPARDA_REQUIRE(!sel == !n_sel, SPARDA_ERR_NULL, "route: sel and n_sel go together");
    SPARDA_REQUIRE(dtype_ok(f_dtype), SPARDA_ERR_DTYPE, "route: dtype %d unsupported", f_dtype);
    SPARDA_REQUIRE(B > 0 && Tq > 0 && H > 0 && NB > 0 && block_size > 0, SPARDA_ERR_SHAPE,
                   "route: sizes must be positive");
    SPARDA_REQUIRE(head_dim_ok(Df), SPARDA_ERR_SHAPE, "route: forecast dim %lld not in {16,32,64,128}",
                   (long long)Df);
    SPARDA_REQUIRE(top_k >= 1 && top_k <= kMaxTopK, SPARDA_ERR_SHAPE, "route: top_k %lld not in [1,%lld]",
                   (long long)top_k, (long long)kMaxTopK);
    SPARDA_REQUIRE(score_pos0 >= 0 && query_pos0 >= 0, SPARDA_ERR_SHAPE, "route: negative position");
    SPARDA_REQUIRE(NB < (1ll << 31) && B <= 65535 && H <= 65535, SPARDA_ERR_SHAPE, "route: too large");
    const int64_t ke = top_k < NB ? top_k : NB;
    SPARDA_REQUIRE(!sel || sel_cap >= ke + 2, SPARDA_ERR_SHAPE, "route: sel_cap %lld < %lld",
                   (long long)sel_cap, (long long)(ke + 2));
    SPARDA_REQUIRE(f_sb >= 0 && f_st >= 0 && f_sh >= 0, SPARDA_ERR_STRIDE, "route: negative stride");
    SPARDA_REQUIRE(reinterpret_cast<uintptr_t>(protos) % 16 == 0, SPARDA_ERR_STRIDE,
                   "route: prototypes must be 16-byte aligned");
    return launch_route(forecast, f_dtype, f_sb, f_st, f_sh, protos, B, Tq, H, Df, NB, block_size,
                        static_cast<int>(ke), causal != 0, score_pos0, query_pos0, scale, topk, scores,
                        sel, n_sel, static_cast<int>(sel ? sel_cap : 0), static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_topk_scores(const float* scores, int64_t rows, int64_t NB, int64_t top_k, int algo,
                                  int32_t* topk, void* stream) {
    SPARDA_REQUIRE(scores && topk, SPARDA_ERR_NULL, "topk_scores: null pointer");
    SPARDA_REQUIRE(rows > 0 && NB > 0 && rows < (1ll << 31), SPARDA_ERR_SHAPE, "topk_scores: bad sizes");
    SPARDA_REQUIRE(top_k >= 1 && top_k <= kMaxTopK, SPARDA_ERR_SHAPE, "topk_scores: top_k out of range");
    SPARDA_REQUIRE(algo >= SPARDA_TOPK_AUTO && algo <= SPARDA_TOPK_WAVE, SPARDA_ERR_MODE,
                   "topk_scores: unknown algo %d", algo);
    SPARDA_REQUIRE(algo != SPARDA_TOPK_WAVE || NB <= 4096, SPARDA_ERR_SHAPE,
                   "topk_scores: wave algo supports NB <= 4096");
    const int64_t ke = top_k < NB ? top_k : NB;
    return launch_topk_scores(scores, rows, NB, static_cast<int>(ke), algo, topk,
                              static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_select_chunked(const int32_t* topk, int64_t top_k_width, int64_t B, int64_t H, int64_t T,
                                     int64_t block_size, int64_t top_k, int32_t* sel, int32_t* n_sel,
                                     int64_t sel_cap, void* stream) {
    SPARDA_REQUIRE(sel && n_sel, SPARDA_ERR_NULL, "select_chunked: null sel / n_sel");
    SPARDA_REQUIRE(B > 0 && H > 0 && T > 0 && block_size > 0 && top_k >= 1 && top_k <= kMaxTopK, SPARDA_ERR_SHAPE,
                   "select_chunked: bad sizes");
    SPARDA_REQUIRE(!topk || (top_k_width >= 1 && top_k_width <= top_k), SPARDA_ERR_SHAPE,
                   "select_chunked: top-k width %lld not in [1, top_k]", (long long)top_k_width);
    SPARDA_REQUIRE(B <= 65535 && H <= 65535, SPARDA_ERR_SHAPE, "select_chunked: grid too large");
    return launch_chunk_select(topk, top_k_width, B, H, T, block_size, top_k, sel, n_sel, sel_cap,
                               static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_select_fixed(int mode, int64_t B, int64_t Tq, int64_t H, int64_t NB,
                                   int64_t block_size, int64_t top_k, int64_t query_pos0, int32_t* sel,
                                   int32_t* n_sel, int64_t sel_cap, void* stream) {
    SPARDA_REQUIRE(sel && n_sel, SPARDA_ERR_NULL, "select_fixed: null pointer");
    SPARDA_REQUIRE(mode >= SPARDA_SEL_DENSE && mode <= SPARDA_SEL_WINDOW_PREFILL, SPARDA_ERR_MODE,
                   "select_fixed: unknown mode %d", mode);
    SPARDA_REQUIRE(B > 0 && Tq > 0 && H > 0 && NB > 0 && block_size > 0 && top_k >= 1 && query_pos0 >= 0,
                   SPARDA_ERR_SHAPE, "select_fixed: bad sizes");
    int64_t need;
    if (mode == SPARDA_SEL_DENSE) {
        int64_t own_max = (query_pos0 + Tq - 1) / block_size;
        need = (own_max < NB - 1 ? own_max : NB - 1) + 1;
    } else {
        need = top_k + 2;
    }
    SPARDA_REQUIRE(sel_cap >= need, SPARDA_ERR_SHAPE, "select_fixed: sel_cap %lld < %lld",
                   (long long)sel_cap, (long long)need);
    return launch_select_fixed(mode, B, Tq, H, NB, block_size, top_k, query_pos0, sel, n_sel,
                               static_cast<int>(sel_cap), static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_gather_blocks(const void* k, const void* v, int dtype, int64_t sb, int64_t sh,
                                    int64_t ss, const int32_t* idx, int64_t B, int64_t H, int64_t S,
                                    int64_t D, int64_t n, int64_t block_size, void* k_out, void* v_out,
                                    void* stream) {
    SPARDA_REQUIRE(k && v && idx && k_out && v_out, SPARDA_ERR_NULL, "gather: null pointer");
    SPARDA_REQUIRE(dtype_ok(dtype), SPARDA_ERR_DTYPE, "gather: dtype %d unsupported", dtype);
    SPARDA_REQUIRE(B > 0 && H > 0 && S > 0 && D > 0 && n > 0 && block_size > 0, SPARDA_ERR_SHAPE,
                   "gather: sizes must be positive");
    SPARDA_REQUIRE(n <= 0x7fffffff && H <= 65535 && B <= 65535, SPARDA_ERR_SHAPE, "gather: too large");
    return launch_gather(k, v, dtype, sb, sh, ss, idx, B, H, S, D, n, block_size, k_out, v_out,
                         static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_prefill(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k,
                              const void* v, int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int dtype,
                              const int32_t* sel, const int32_t* n_sel, int64_t sel_cap, int64_t B,
                              int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t block_size, int causal,
                              float scale, void* out, int64_t out_sb, int64_t out_st, void* stream) {
    SPARDA_REQUIRE(q && k && v && out, SPARDA_ERR_NULL, "prefill: null q/k/v/out");
    SPARDA_REQUIRE(!sel == !n_sel, SPARDA_ERR_NULL, "prefill: sel and n_sel go together");
    SPARDA_REQUIRE(dtype_ok(dtype), SPARDA_ERR_DTYPE, "prefill: dtype %d unsupported", dtype);
    SPARDA_REQUIRE(B > 0 && T > 0 && Hq > 0 && Hkv > 0 && block_size > 0, SPARDA_ERR_SHAPE,
                   "prefill: sizes must be positive");
    SPARDA_REQUIRE(head_dim_ok(D), SPARDA_ERR_SHAPE, "prefill: head dim %lld not in {16,32,64,128}",
                   (long long)D);
    SPARDA_REQUIRE(Hq % Hkv == 0 && Hq / Hkv <= kMaxGroupAbi, SPARDA_ERR_SHAPE,
                   "prefill: Hq %lld must be a multiple of Hkv %lld with ratio <= 16", (long long)Hq,
                   (long long)Hkv);
    SPARDA_REQUIRE(!sel || sel_cap >= 1, SPARDA_ERR_SHAPE, "prefill: sel_cap must be >= 1");
    SPARDA_REQUIRE(T < (1ll << 31) && B <= 65535 && Hkv <= 65535, SPARDA_ERR_SHAPE, "prefill: too large");
    return launch_prefill(q, q_sb, q_st, q_sh, k, v, kv_sb, kv_st, kv_sh, dtype, sel, n_sel, sel_cap, B, T,
                          Hq, Hkv, D, block_size, causal != 0, scale, out, out_sb, out_st,
                          static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_prefill_routed(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k,
                                     const void* v, int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int dtype,
                                     const void* forecast, int f_dtype, int64_t f_sb, int64_t f_st, int64_t f_sh,
                                     const float* protos, int64_t Df, int64_t top_k, float route_scale,
                                     int32_t* sel, int32_t* n_sel, int64_t sel_cap, int64_t B, int64_t T,
                                     int64_t Hq, int64_t Hkv, int64_t D, int64_t block_size, int causal,
                                     float scale, void* out, int64_t out_sb, int64_t out_st, void* stream) {
    SPARDA_REQUIRE(q && k && v && out && forecast && protos, SPARDA_ERR_NULL,
                   "prefill_routed: null q/k/v/out/forecast/protos");
    SPARDA_REQUIRE(!sel == !n_sel, SPARDA_ERR_NULL, "prefill_routed: sel and n_sel go together");
    SPARDA_REQUIRE(dtype_ok(dtype) && dtype_ok(f_dtype), SPARDA_ERR_DTYPE, "prefill_routed: dtype %d / %d unsupported",
                   dtype, f_dtype);
    SPARDA_REQUIRE(B > 0 && T > 0 && Hq > 0 && Hkv > 0 && block_size > 0, SPARDA_ERR_SHAPE,
                   "prefill_routed: sizes must be positive");
    SPARDA_REQUIRE(head_dim_ok(D) && head_dim_ok(Df), SPARDA_ERR_SHAPE,
                   "prefill_routed: head dim %lld / forecast dim %lld not in {16,32,64,128}", (long long)D,
                   (long long)Df);
    SPARDA_REQUIRE(Hq % Hkv == 0 && Hq / Hkv <= kMaxGroupAbi, SPARDA_ERR_SHAPE,
                   "prefill_routed: Hq must be a multiple of Hkv with ratio <= 16");
    SPARDA_REQUIRE(top_k >= 1 && top_k <= kMaxTopK, SPARDA_ERR_SHAPE, "prefill_routed: top_k %lld not in [1,%lld]",
                   (long long)top_k, (long long)kMaxTopK);
    SPARDA_REQUIRE(T < (1ll << 31) && B <= 65535 && Hkv <= 65535, SPARDA_ERR_SHAPE, "prefill_routed: too large");
    SPARDA_REQUIRE(f_sb >= 0 && f_st >= 0 && f_sh >= 0, SPARDA_ERR_STRIDE, "prefill_routed: negative stride");
    SPARDA_REQUIRE(reinterpret_cast<uintptr_t>(protos) % 16 == 0, SPARDA_ERR_STRIDE,
                   "prefill_routed: prototypes must be 16-byte aligned");
    const int64_t NB = cdiv(T, block_size);
    const int64_t ke = top_k < NB ? top_k : NB;
    SPARDA_REQUIRE(!sel || sel_cap >= ke + 2, SPARDA_ERR_SHAPE, "prefill_routed: sel_cap %lld < %lld",
                   (long long)sel_cap, (long long)(ke + 2));
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (prefill_routed_supported(dtype, f_dtype, T, Hq, Hkv, D, Df, block_size, ke, q_sb, q_st, q_sh, kv_sb, kv_st,
                                 kv_sh, out_sb, out_st, q, k, v, out, protos)) {
        CompactRoute rt{forecast, f_sb, f_st, f_sh, protos, static_cast<int>(ke), route_scale,
                        sel, n_sel, static_cast<int>(sel ? sel_cap : 0)};
        return launch_prefill_routed(q, q_sb, q_st, q_sh, k, v, kv_sb, kv_st, kv_sh, f_dtype, rt, B, T, Hq, Hkv,
                                     block_size, causal != 0, scale, out, out_sb, out_st, st);
    }
    // other shapes: the router's lists handed to the prefill through the caller's buffers
    SPARDA_REQUIRE(sel != nullptr, SPARDA_ERR_SHAPE,
                   "prefill_routed: this shape takes two launches and needs sel/n_sel as their hand-off buffers");
    SPARDA_REQUIRE(NB < (1ll << 31), SPARDA_ERR_SHAPE, "prefill_routed: too large");
    int rc = launch_route(forecast, f_dtype, f_sb, f_st, f_sh, protos, B, T, Hkv, Df, NB, block_size,
                          static_cast<int>(ke), causal != 0, 0, 0, route_scale, nullptr, nullptr, sel, n_sel,
                          static_cast<int>(sel_cap), st);
    if (rc != 0) return rc;
    return launch_prefill(q, q_sb, q_st, q_sh, k, v, kv_sb, kv_st, kv_sh, dtype, sel, n_sel, sel_cap, B, T, Hq, Hkv,
                          D, block_size, causal != 0, scale, out, out_sb, out_st, st);
}

SPARDA_API int sparda_prefill_chunked(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k,
                                      const void* v, int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int dtype,
                                      const int32_t* topk, int64_t top_k_width, int64_t top_k, int32_t* sel,
                                      int32_t* n_sel, int64_t sel_cap, int64_t B, int64_t T, int64_t Hq,
                                      int64_t Hkv, int64_t D, int64_t block_size, float scale, void* out,
                                      int64_t out_sb, int64_t out_st, void* stream) {
    SPARDA_REQUIRE(q && k && v && out, SPARDA_ERR_NULL, "prefill_chunked: null q/k/v/out");
    SPARDA_REQUIRE(!sel == !n_sel, SPARDA_ERR_NULL, "prefill_chunked: sel and n_sel go together");
    SPARDA_REQUIRE(dtype_ok(dtype), SPARDA_ERR_DTYPE, "prefill_chunked: dtype %d unsupported", dtype);
    SPARDA_REQUIRE(B > 0 && T > 0 && Hq > 0 && Hkv > 0 && block_size > 0, SPARDA_ERR_SHAPE,
                   "prefill_chunked: sizes must be positive");
    SPARDA_REQUIRE(head_dim_ok(D), SPARDA_ERR_SHAPE, "prefill_chunked: head dim %lld not in {16,32,64,128}",
                   (long long)D);
    SPARDA_REQUIRE(Hq % Hkv == 0 && Hq / Hkv <= kMaxGroupAbi, SPARDA_ERR_SHAPE,
                   "prefill_chunked: Hq must be a multiple of Hkv with ratio <= 16");
    SPARDA_REQUIRE(top_k >= 1 && top_k <= kMaxTopK, SPARDA_ERR_SHAPE, "prefill_chunked: top_k %lld not in [1,%lld]",
                   (long long)top_k, (long long)kMaxTopK);
    SPARDA_REQUIRE(!topk || (top_k_width >= 1 && top_k_width <= top_k), SPARDA_ERR_SHAPE,
                   "prefill_chunked: top-k width %lld not in [1, top_k]", (long long)top_k_width);
    SPARDA_REQUIRE(T < (1ll << 31) && B <= 65535 && Hkv <= 65535, SPARDA_ERR_SHAPE, "prefill_chunked: too large");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (block_size == 64 && B * Hkv * cdiv(T, 64) < (1ll << 31) &&
        prefill_dense_supported(dtype, Hq, Hkv, D, q_sb, q_st, q_sh, kv_sb, kv_st, kv_sh, out_sb, out_st, q, k, v,
                                out))
        return launch_prefill_chunked(q, q_sb, q_st, q_sh, k, v, kv_sb, kv_st, kv_sh, topk, top_k_width, top_k, sel,
                                      n_sel, sel_cap, B, T, Hq, Hkv, scale, out, out_sb, out_st, st);
    // other shapes: the lists handed to the prefill through the caller's buffers
    SPARDA_REQUIRE(sel != nullptr, SPARDA_ERR_SHAPE,
                   "prefill_chunked: this shape takes two launches and needs sel/n_sel as their hand-off buffers");
    int rc = launch_chunk_select(topk, top_k_width, B, Hkv, T, block_size, top_k, sel, n_sel, sel_cap, st);
    if (rc != 0) return rc;
    return launch_prefill(q, q_sb, q_st, q_sh, k, v, kv_sb, kv_st, kv_sh, dtype, sel, n_sel, sel_cap, B, T, Hq, Hkv,
                          D, block_size, true, scale, out, out_sb, out_st, st);
}

SPARDA_API int sparda_prefill_masked(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k,
                                     const void* v, int64_t kv_sb, int64_t kv_st, int64_t kv_sh, int dtype,
                                     const int32_t* sel, const int32_t* n_sel, int64_t sel_cap, int64_t B,
                                     int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t block_size,
                                     int causal, float scale, const void* mask, int mask_dtype, int64_t m_sb,
                                     int64_t m_sh, int64_t m_st, int64_t m_ss, void* out, int64_t out_sb,
                                     int64_t out_st, void* weights, int64_t w_sb, int64_t w_sh, int64_t w_st,
                                     void* stream) {
    SPARDA_REQUIRE(q && k && v && out, SPARDA_ERR_NULL, "prefill_masked: null q/k/v/out");
    SPARDA_REQUIRE(!sel == !n_sel, SPARDA_ERR_NULL, "prefill_masked: sel and n_sel go together");
    SPARDA_REQUIRE(dtype_ok(dtype), SPARDA_ERR_DTYPE, "prefill_masked: dtype %d unsupported", dtype);
    SPARDA_REQUIRE(!mask || dtype_ok(mask_dtype), SPARDA_ERR_DTYPE, "prefill_masked: mask dtype %d", mask_dtype);
    SPARDA_REQUIRE(B > 0 && T > 0 && Hq > 0 && Hkv > 0 && block_size > 0, SPARDA_ERR_SHAPE,
                   "prefill_masked: sizes must be positive");
    SPARDA_REQUIRE(head_dim_ok(D), SPARDA_ERR_SHAPE, "prefill_masked: head dim %lld not in {16,32,64,128}",
                   (long long)D);
    SPARDA_REQUIRE(Hq % Hkv == 0 && Hq / Hkv <= kMaxGroupAbi, SPARDA_ERR_SHAPE,
                   "prefill_masked: Hq must be a multiple of Hkv with ratio <= 16");
    SPARDA_REQUIRE(!sel || (sel_cap >= 1 && sel_cap <= kMaxSelCap), SPARDA_ERR_SHAPE,
                   "prefill_masked: sel_cap must be in [1, %d]", kMaxSelCap);
    SPARDA_REQUIRE(T < (1ll << 31) && B <= 65535 && Hkv <= 65535, SPARDA_ERR_SHAPE, "prefill_masked: too large");
    SPARDA_REQUIRE(m_sb >= 0 && m_sh >= 0 && m_st >= 0 && m_ss >= 0 && w_sb >= 0 && w_sh >= 0 && w_st >= 0,
                   SPARDA_ERR_STRIDE, "prefill_masked: negative stride");
    return launch_prefill_weights(q, q_sb, q_st, q_sh, k, v, kv_sb, kv_st, kv_sh, dtype, sel, n_sel, sel_cap, B, T,
                                  Hq, Hkv, D, block_size, causal != 0, scale, mask, mask_dtype, m_sb, m_sh, m_st,
                                  m_ss, out, out_sb, out_st, weights, w_sb, w_sh, w_st,
                                  static_cast<hipStream_t>(stream));
}

SPARDA_API size_t sparda_decode_workspace_bytes(int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D,
                                                int64_t block_size, int64_t top_k) {
    if (B <= 0 || S <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || block_size <= 0 || top_k <= 0) return 0;
    return decode_ws_layout(nullptr, B, S, Hq, Hkv, D, block_size, top_k).bytes;
}

SPARDA_API int sparda_decode(const void* q, int64_t q_sb, int64_t q_sh, const void* k_cache,
                             const void* v_cache, int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int dtype,
                             const void* forecast, int f_dtype, int64_t f_sb, int64_t f_sh, int64_t B,
                             int64_t S, int64_t Hq, int64_t Hkv, int64_t D, int64_t block_size,
                             int64_t top_k, int routing, float scale, const float* protos_in,
                             float* protos_out, int32_t* sel_out, int32_t* n_sel_out, void* out,
                             int64_t out_sb, void* workspace, size_t workspace_bytes, void* stream) {
    const int rc = check_decode_args(q, k_cache, v_cache, kv_sb, kv_ss, kv_sh, dtype, forecast, f_dtype, B, S, Hq,
                                     Hkv, D, block_size, top_k, routing, sel_out, n_sel_out, out);
    if (rc) return rc;
    SPARDA_REQUIRE(workspace, SPARDA_ERR_WORKSPACE, "decode: workspace is required");
    const DecodeWs ws = decode_ws_layout(workspace, B, S, Hq, Hkv, D, block_size, top_k);
    SPARDA_REQUIRE(workspace_bytes >= ws.bytes, SPARDA_ERR_WORKSPACE, "decode: workspace %zu < %zu bytes",
                   workspace_bytes, ws.bytes);
    SPARDA_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255u) == 0, SPARDA_ERR_WORKSPACE,
                   "decode: workspace must be 256-byte aligned");
    return launch_decode(q, q_sb, q_sh, k_cache, v_cache, kv_sb, kv_ss, kv_sh, dtype, forecast, f_dtype, f_sb,
                         f_sh, B, S, Hq, Hkv, D, block_size, top_k, routing, scale, protos_in, protos_out,
                         sel_out, n_sel_out, out, out_sb, ws, static_cast<hipStream_t>(stream));
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

SPARDA_API int sparda_decode_selected(const void* q, int64_t q_sb, int64_t q_sh, const void* k, const void* v,
                                      int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int dtype, int compact,
                                      const int32_t* sel, const int32_t* n_sel, int64_t sel_cap,
                                      const void* k_new, const void* v_new, int64_t new_sb, int64_t new_sh,
                                      int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D,
                                      int64_t block_size, float scale, void* out, int64_t out_sb,
                                      void* workspace, size_t workspace_bytes, void* stream) {
    SPARDA_REQUIRE(q && k && v && out, SPARDA_ERR_NULL, "decode_selected: null q/k/v/out");
    SPARDA_REQUIRE(!workspace || aligned16(workspace), SPARDA_ERR_WORKSPACE,
                   "decode_selected: workspace must be 16-byte aligned");
    SPARDA_REQUIRE(!sel == !n_sel, SPARDA_ERR_NULL, "decode_selected: sel and n_sel go together");
    SPARDA_REQUIRE(!k_new == !v_new, SPARDA_ERR_NULL, "decode_selected: k_new and v_new go together");
    SPARDA_REQUIRE(!compact || sel, SPARDA_ERR_MODE, "decode_selected: compact buffers need a selection");
    SPARDA_REQUIRE(dtype_ok(dtype), SPARDA_ERR_DTYPE, "decode_selected: dtype %d unsupported", dtype);
    SPARDA_REQUIRE(B > 0 && S > 0 && Hq > 0 && Hkv > 0 && block_size > 0, SPARDA_ERR_SHAPE,
                   "decode_selected: sizes must be positive");
    SPARDA_REQUIRE(head_dim_ok(D), SPARDA_ERR_SHAPE, "decode_selected: head dim %lld not in {16,32,64,128}",
                   (long long)D);
    SPARDA_REQUIRE(Hq % Hkv == 0 && Hq / Hkv <= kMaxGroupAbi, SPARDA_ERR_SHAPE,
                   "decode_selected: Hq must be a multiple of Hkv with ratio <= 16");
    SPARDA_REQUIRE(!sel || (sel_cap >= 1 && sel_cap <= kMaxSelCap), SPARDA_ERR_SHAPE,
                   "decode_selected: sel_cap must be in [1, %d]", kMaxSelCap);
    SPARDA_REQUIRE(B <= 65535 && Hkv <= 65535, SPARDA_ERR_SHAPE, "decode_selected: grid too large");
    const int64_t ve = 16 / (dtype == SPARDA_F32 ? 4 : 2);
    SPARDA_REQUIRE(aligned16(k) && aligned16(v) && kv_sb % ve == 0 && kv_ss % ve == 0 && kv_sh % ve == 0,
                   SPARDA_ERR_STRIDE, "decode_selected: K/V rows must be 16-byte aligned");
    SPARDA_REQUIRE(!k_new || (aligned16(k_new) && aligned16(v_new) && new_sb % ve == 0 && new_sh % ve == 0),
                   SPARDA_ERR_STRIDE, "decode_selected: k_new/v_new rows must be 16-byte aligned");
    return launch_decode_selected(q, q_sb, q_sh, k, v, kv_sb, kv_ss, kv_sh, dtype, compact, sel, n_sel, sel_cap,
                                  k_new, v_new, new_sb, new_sh, B, S, Hq, Hkv, D, block_size, scale, out,
                                  out_sb, static_cast<hipStream_t>(stream), workspace,
                                  workspace ? workspace_bytes : 0);
}

SPARDA_API size_t sparda_decode_dense_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                                      int64_t max_len, int64_t block_size) {
    return decode_dense_workspace_bytes(B, Hq, Hkv, D, max_len, block_size);
}

SPARDA_API int sparda_select_decode(const void* forecast, int f_dtype, int64_t f_sb, int64_t f_sh,
                                    const float* block_sums, int64_t B, int64_t Hkv, int64_t D,
                                    int64_t nb_stride, int64_t len, int64_t pos, int64_t block_size,
                                    int64_t top_k, int routing, float scale, int32_t* sel, int32_t* n_sel,
                                    int64_t sel_cap, void* stream) {
    SPARDA_REQUIRE(forecast && block_sums && sel && n_sel, SPARDA_ERR_NULL, "select_decode: null pointer");
    SPARDA_REQUIRE(dtype_ok(f_dtype), SPARDA_ERR_DTYPE, "select_decode: forecast dtype %d", f_dtype);
    SPARDA_REQUIRE(routing == SPARDA_ROUTE_REFERENCE || routing == SPARDA_ROUTE_ABSOLUTE, SPARDA_ERR_MODE,
                   "select_decode: unknown routing %d", routing);
    SPARDA_REQUIRE(B > 0 && Hkv > 0 && head_dim_ok(D) && block_size > 0, SPARDA_ERR_SHAPE,
                   "select_decode: bad sizes (D must be one of 16, 32, 64, 128)");
    SPARDA_REQUIRE((reinterpret_cast<uintptr_t>(block_sums) & 15u) == 0, SPARDA_ERR_STRIDE,
                   "select_decode: block_sums must be 16-byte aligned");
    SPARDA_REQUIRE(len >= 1 && pos >= len - 1, SPARDA_ERR_SHAPE,
                   "select_decode: need len >= 1 and pos >= len-1 (len=%lld pos=%lld)", (long long)len,
                   (long long)pos);
    SPARDA_REQUIRE(top_k >= 1 && top_k <= kMaxTopK, SPARDA_ERR_SHAPE, "select_decode: top_k out of range");
    SPARDA_REQUIRE(sel_cap >= top_k + 2 && sel_cap <= kMaxSelCap, SPARDA_ERR_SHAPE,
                   "select_decode: sel_cap must be in [top_k+2, %d]", kMaxSelCap);
    SPARDA_REQUIRE(nb_stride >= cdiv(len, block_size), SPARDA_ERR_SHAPE, "select_decode: nb_stride too small");
    SPARDA_REQUIRE(cdiv(len, block_size) <= 4096, SPARDA_ERR_SHAPE, "select_decode: more than 4096 blocks");
    SPARDA_REQUIRE(B <= 65535 && Hkv <= 65535, SPARDA_ERR_SHAPE, "select_decode: grid too large");
    return launch_select_decode(forecast, f_dtype, f_sb, f_sh, block_sums, B, Hkv, D, nb_stride, len, pos,
                                block_size, top_k, routing, scale, sel, n_sel, sel_cap,
                                static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_select_decode_at(const void* forecast, int f_dtype, int64_t f_sb, int64_t f_sh,
                                       const float* block_sums, int64_t B, int64_t Hkv, int64_t D,
                                       int64_t nb_stride, int64_t max_len, const int64_t* pos_dev,
                                       int64_t block_size, int64_t top_k, int routing, float scale, int32_t* sel,
                                       int32_t* n_sel, int64_t sel_cap, int lookahead, void* stream) {
    SPARDA_REQUIRE(pos_dev, SPARDA_ERR_NULL, "select_decode_at: null pos_dev");
    SPARDA_REQUIRE((reinterpret_cast<uintptr_t>(pos_dev) & 7u) == 0, SPARDA_ERR_STRIDE,
                   "select_decode_at: pos_dev must be 8-byte aligned");
    SPARDA_REQUIRE(forecast && block_sums && sel && n_sel, SPARDA_ERR_NULL, "select_decode_at: null pointer");
    SPARDA_REQUIRE(dtype_ok(f_dtype), SPARDA_ERR_DTYPE, "select_decode_at: forecast dtype %d", f_dtype);
    SPARDA_REQUIRE(routing == SPARDA_ROUTE_REFERENCE || routing == SPARDA_ROUTE_ABSOLUTE, SPARDA_ERR_MODE,
                   "select_decode_at: unknown routing %d", routing);
    SPARDA_REQUIRE(B > 0 && Hkv > 0 && head_dim_ok(D) && block_size > 0 && max_len >= 1, SPARDA_ERR_SHAPE,
                   "select_decode_at: bad sizes (D must be one of 16, 32, 64, 128)");
    SPARDA_REQUIRE((reinterpret_cast<uintptr_t>(block_sums) & 15u) == 0, SPARDA_ERR_STRIDE,
                   "select_decode_at: block_sums must be 16-byte aligned");
    SPARDA_REQUIRE(top_k >= 1 && top_k <= kMaxTopK, SPARDA_ERR_SHAPE, "select_decode_at: top_k out of range");
    SPARDA_REQUIRE(sel_cap >= top_k + 2 && sel_cap <= kMaxSelCap, SPARDA_ERR_SHAPE,
                   "select_decode_at: sel_cap must be in [top_k+2, %d]", kMaxSelCap);
    SPARDA_REQUIRE(nb_stride >= cdiv(max_len, block_size), SPARDA_ERR_SHAPE,
                   "select_decode_at: nb_stride too small");
    SPARDA_REQUIRE(cdiv(max_len, block_size) <= 4096, SPARDA_ERR_SHAPE, "select_decode_at: more than 4096 blocks");
    SPARDA_REQUIRE(B <= 65535 && Hkv <= 65535, SPARDA_ERR_SHAPE, "select_decode_at: grid too large");
    return launch_select_decode(forecast, f_dtype, f_sb, f_sh, block_sums, B, Hkv, D, nb_stride, max_len,
                                max_len - 1, block_size, top_k, routing, scale, sel, n_sel, sel_cap,
                                static_cast<hipStream_t>(stream), pos_dev, lookahead != 0);
}

static int decode_at_checked(const void* q, int64_t q_sb, int64_t q_sh, const void* k, const void* v,
                             int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int dtype, int compact,
                             const int32_t* sel, const int32_t* n_sel, int64_t sel_cap, int64_t window_k,
                             const void* k_new, const void* v_new, int64_t new_sb, int64_t new_sh, int64_t B,
                             int64_t max_len, const int64_t* pos_dev, int64_t Hq, int64_t Hkv, int64_t D,
                             int64_t block_size, float scale, void* out, int64_t out_sb, void* workspace,
                             size_t workspace_bytes, void* stream, const sparda::PrefetchDev* pf) {
    SPARDA_REQUIRE(q && k && v && out && pos_dev, SPARDA_ERR_NULL, "decode_at: null q/k/v/out/pos_dev");
    SPARDA_REQUIRE(!workspace || aligned16(workspace), SPARDA_ERR_WORKSPACE,
                   "decode_at: workspace must be 16-byte aligned");
    SPARDA_REQUIRE((reinterpret_cast<uintptr_t>(pos_dev) & 7u) == 0, SPARDA_ERR_STRIDE,
                   "decode_at: pos_dev must be 8-byte aligned");
    SPARDA_REQUIRE(!sel == !n_sel, SPARDA_ERR_NULL, "decode_at: sel and n_sel go together");
    SPARDA_REQUIRE(!k_new == !v_new, SPARDA_ERR_NULL, "decode_at: k_new and v_new go together");
    SPARDA_REQUIRE(!compact || sel, SPARDA_ERR_MODE, "decode_at: compact buffers need a selection");
    SPARDA_REQUIRE(!sel || window_k == 0, SPARDA_ERR_MODE, "decode_at: a selection list or a window, not both");
    SPARDA_REQUIRE(dtype_ok(dtype), SPARDA_ERR_DTYPE, "decode_at: dtype %d unsupported", dtype);
    SPARDA_REQUIRE(B > 0 && max_len > 0 && Hq > 0 && Hkv > 0 && block_size > 0, SPARDA_ERR_SHAPE,
                   "decode_at: sizes must be positive");
    SPARDA_REQUIRE(head_dim_ok(D), SPARDA_ERR_SHAPE, "decode_at: head dim %lld not in {16,32,64,128}",
                   (long long)D);
    SPARDA_REQUIRE(Hq % Hkv == 0 && Hq / Hkv <= kMaxGroupAbi, SPARDA_ERR_SHAPE,
                   "decode_at: Hq must be a multiple of Hkv with ratio <= 16");
    SPARDA_REQUIRE(!sel || (sel_cap >= 1 && sel_cap <= kMaxSelCap), SPARDA_ERR_SHAPE,
                   "decode_at: sel_cap must be in [1, %d]", kMaxSelCap);
    SPARDA_REQUIRE(window_k >= 0 && window_k <= kMaxTopK, SPARDA_ERR_SHAPE, "decode_at: window_k out of range");
    SPARDA_REQUIRE(B <= 65535 && Hkv <= 65535, SPARDA_ERR_SHAPE, "decode_at: grid too large");
    const int64_t ve = 16 / (dtype == SPARDA_F32 ? 4 : 2);
    SPARDA_REQUIRE(aligned16(k) && aligned16(v) && kv_sb % ve == 0 && kv_ss % ve == 0 && kv_sh % ve == 0,
                   SPARDA_ERR_STRIDE, "decode_at: K/V rows must be 16-byte aligned");
    SPARDA_REQUIRE(!k_new || (aligned16(k_new) && aligned16(v_new) && new_sb % ve == 0 && new_sh % ve == 0),
                   SPARDA_ERR_STRIDE, "decode_at: k_new/v_new rows must be 16-byte aligned");
    return launch_decode_at(q, q_sb, q_sh, k, v, kv_sb, kv_ss, kv_sh, dtype, compact, sel, n_sel, sel_cap, window_k,
                            k_new, v_new, new_sb, new_sh, B, max_len, pos_dev, Hq, Hkv, D, block_size, scale, out,
                            out_sb, static_cast<hipStream_t>(stream), pf, workspace,
                            workspace ? workspace_bytes : 0);
}

SPARDA_API int sparda_decode_at(const void* q, int64_t q_sb, int64_t q_sh, const void* k, const void* v,
                                int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int dtype, int compact,
                                const int32_t* sel, const int32_t* n_sel, int64_t sel_cap, int64_t window_k,
                                const void* k_new, const void* v_new, int64_t new_sb, int64_t new_sh, int64_t B,
                                int64_t max_len, const int64_t* pos_dev, int64_t Hq, int64_t Hkv, int64_t D,
                                int64_t block_size, float scale, void* out, int64_t out_sb, void* workspace,
                                size_t workspace_bytes, void* stream) {
    return decode_at_checked(q, q_sb, q_sh, k, v, kv_sb, kv_ss, kv_sh, dtype, compact, sel, n_sel, sel_cap, window_k,
                             k_new, v_new, new_sb, new_sh, B, max_len, pos_dev, Hq, Hkv, D, block_size, scale, out,
                             out_sb, workspace, workspace_bytes, stream, nullptr);
}

// The device form of a prefetch carried by another launch, after the checks
// both carrying entries make (the next layer's arena: batch B, Hkv KV heads,
// head dim 64, dtype bf16 like the carrying layer).
static int prefetch_dev(const sparda_prefetch_args* next, int64_t B, int64_t Hkv, int64_t D, int dtype,
                        int64_t max_len, int64_t block_size, const char* who, PrefetchDev* pf) {
    SPARDA_REQUIRE(next, SPARDA_ERR_NULL, "%s: null prefetch arguments", who);
    const sparda_prefetch_args& n = *next;
    SPARDA_REQUIRE(n.arena, SPARDA_ERR_HANDLE, "%s: null arena handle", who);
    SPARDA_REQUIRE(n.stage >= 0 && n.stage <= 2, SPARDA_ERR_MODE, "%s: stage %d not in {0, 1, 2}", who, n.stage);
    SPARDA_REQUIRE(n.sel && n.n_sel, SPARDA_ERR_NULL, "%s: null sel / n_sel", who);
    SPARDA_REQUIRE(n.stage == 2 || (n.forecast && n.block_sums), SPARDA_ERR_NULL, "%s: null forecast / block_sums",
                   who);
    SPARDA_REQUIRE(n.stage == 1 || (n.k_dst && n.v_dst), SPARDA_ERR_NULL, "%s: null destinations", who);
    SPARDA_REQUIRE(n.parts >= 0 && n.parts <= kMaxSelCap && (n.parts <= 1 ? n.part == 0 : n.part >= 0 && n.part < n.parts),
                   SPARDA_ERR_SHAPE, "%s: copy share %d of %d", who, n.part, n.parts);
    SPARDA_REQUIRE(n.parts <= 1 || n.stage == 2, SPARDA_ERR_MODE, "%s: a share of the copy needs stage 2", who);
    SPARDA_REQUIRE(D == 64 && dtype == SPARDA_BF16, SPARDA_ERR_MODE, "%s: a carried prefetch needs bf16, D=64", who);
    SPARDA_REQUIRE(offload_batch(n.arena) == B && offload_heads(n.arena) == Hkv && offload_head_dim(n.arena) == D &&
                       offload_dtype(n.arena) == dtype,
                   SPARDA_ERR_SHAPE, "%s: the arena's batch, KV heads, head dim and dtype must be the carrying "
                   "layer's", who);
    SPARDA_REQUIRE(n.stage == 2 || dtype_ok(n.f_dtype), SPARDA_ERR_DTYPE, "%s: forecast dtype %d", who, n.f_dtype);
    SPARDA_REQUIRE(n.routing == SPARDA_ROUTE_REFERENCE || n.routing == SPARDA_ROUTE_ABSOLUTE, SPARDA_ERR_MODE,
                   "%s: unknown routing %d", who, n.routing);
    SPARDA_REQUIRE(n.stage == 2 || (reinterpret_cast<uintptr_t>(n.block_sums) & 15u) == 0, SPARDA_ERR_STRIDE,
                   "%s: block_sums must be 16-byte aligned", who);
    SPARDA_REQUIRE(n.top_k >= 1 && n.top_k <= kMaxTopK, SPARDA_ERR_SHAPE, "%s: top_k out of range", who);
    SPARDA_REQUIRE(n.sel_cap >= n.top_k + 2 && n.sel_cap <= kMaxSelCap, SPARDA_ERR_SHAPE,
                   "%s: sel_cap must be in [top_k+2, %d]", who, kMaxSelCap);
    SPARDA_REQUIRE(block_size > 0 && max_len >= 1 && (n.stage == 2 || n.nb_stride >= cdiv(max_len, block_size)),
                   SPARDA_ERR_SHAPE, "%s: nb_stride too small", who);
    SPARDA_REQUIRE(cdiv(max_len, block_size) <= 4096, SPARDA_ERR_SHAPE, "%s: more than 4096 blocks", who);
    SPARDA_REQUIRE(n.stage == 1 || (aligned16(n.k_dst) && aligned16(n.v_dst)), SPARDA_ERR_STRIDE,
                   "%s: destinations must be 16-byte aligned", who);
    *pf = PrefetchDev{};
    pf->f = n.forecast;
    pf->f_sb = n.f_sb;
    pf->f_sh = n.f_sh;
    pf->f_bf16 = n.f_dtype == SPARDA_BF16 ? 1 : 0;
    pf->sums = n.block_sums;
    pf->nb_stride = n.nb_stride;
    pf->pos_max = max_len - 1;
    pf->bs = static_cast<int>(block_size);
    pf->k = static_cast<int>(n.top_k);
    pf->cap = static_cast<int>(n.sel_cap);
    pf->absolute = n.routing == SPARDA_ROUTE_ABSOLUTE ? 1 : 0;
    pf->pow2 = (block_size & (block_size - 1)) == 0 ? 1 : 0;
    pf->scale = n.scale;
    pf->sel = n.sel;
    pf->n_sel = n.n_sel;
    pf->dk = static_cast<char*>(n.k_dst);
    pf->dv = static_cast<char*>(n.v_dst);
    pf->stage = n.stage;
    pf->parts = n.parts >= 1 ? n.parts : 1;
    pf->part = n.parts >= 1 ? n.part : 0;
    offload_prefetch_dev(n.arena, pf);
    return 0;
}

SPARDA_API int sparda_decode_at_prefetch(const void* q, int64_t q_sb, int64_t q_sh, const void* k, const void* v,
                                         int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int dtype, int compact,
                                         const int32_t* sel, const int32_t* n_sel, int64_t sel_cap,
                                         int64_t window_k, const void* k_new, const void* v_new, int64_t new_sb,
                                         int64_t new_sh, int64_t B, int64_t max_len, const int64_t* pos_dev,
                                         int64_t Hq, int64_t Hkv, int64_t D, int64_t block_size, float scale,
                                         void* out, int64_t out_sb, const sparda_prefetch_args* next,
                                         void* workspace, size_t workspace_bytes, void* stream) {
    SPARDA_REQUIRE(decode_at_matrix_core(dtype, D, block_size, q_sb, q_sh, q), SPARDA_ERR_MODE,
                   "decode_at_prefetch: needs the matrix-core attention (bf16, D=64, blocks of 64 or 32 keys, "
                   "16-byte aligned q rows)");
    PrefetchDev pf;
    const int rc = prefetch_dev(next, B, Hkv, D, dtype, max_len, block_size, "decode_at_prefetch", &pf);
    if (rc) return rc;
    return decode_at_checked(q, q_sb, q_sh, k, v, kv_sb, kv_ss, kv_sh, dtype, compact, sel, n_sel, sel_cap, window_k,
                             k_new, v_new, new_sb, new_sh, B, max_len, pos_dev, Hq, Hkv, D, block_size, scale, out,
                             out_sb, workspace, workspace_bytes, stream, &pf);
}

SPARDA_API int sparda_offload_create(int64_t B, int64_t max_seq, int64_t Hkv, int64_t D, int dtype,
                                     sparda_offload_t* out) {
    SPARDA_REQUIRE(out, SPARDA_ERR_NULL, "offload_create: null output handle");
    *out = nullptr;
    SPARDA_REQUIRE(dtype_ok(dtype), SPARDA_ERR_DTYPE, "offload_create: dtype %d unsupported", dtype);
    SPARDA_REQUIRE(B > 0 && max_seq > 0 && Hkv > 0 && head_dim_ok(D), SPARDA_ERR_SHAPE,
                   "offload_create: bad sizes (D must be 16/32/64/128)");
    SPARDA_REQUIRE(B <= 65535 && Hkv <= 65535 && max_seq <= (int64_t(1) << 31), SPARDA_ERR_SHAPE,
                   "offload_create: sizes too large");
    return offload_create(B, max_seq, Hkv, D, dtype, out);
}

SPARDA_API int sparda_offload_destroy(sparda_offload_t h) {
    SPARDA_REQUIRE(h, SPARDA_ERR_HANDLE, "offload_destroy: null handle");
    return offload_destroy(h);
}

SPARDA_API int sparda_offload_host(sparda_offload_t h, void** k_host, void** v_host) {
    SPARDA_REQUIRE(h, SPARDA_ERR_HANDLE, "offload_host: null handle");
    SPARDA_REQUIRE(k_host && v_host, SPARDA_ERR_NULL, "offload_host: null output");
    offload_host(h, k_host, v_host);
    return 0;
}

SPARDA_API int sparda_offload_append(sparda_offload_t h, const void* k, const void* v, int64_t sb, int64_t st,
                                     int64_t sh, int64_t pos, int64_t n, int64_t block_size, float* block_sums,
                                     void* stream) {
    SPARDA_REQUIRE(h, SPARDA_ERR_HANDLE, "offload_append: null handle");
    SPARDA_REQUIRE(k && v, SPARDA_ERR_NULL, "offload_append: null k/v");
    SPARDA_REQUIRE(n >= 1 && pos >= 0, SPARDA_ERR_SHAPE, "offload_append: need n >= 1, pos >= 0");
    SPARDA_REQUIRE(pos + n <= offload_max_seq(h), SPARDA_ERR_CAPACITY,
                   "offload_append: tokens [%lld, %lld) exceed the capacity %lld", (long long)pos,
                   (long long)(pos + n), (long long)offload_max_seq(h));
    SPARDA_REQUIRE(sb >= 0 && st >= 0 && sh >= 0, SPARDA_ERR_STRIDE, "offload_append: negative stride");
    SPARDA_REQUIRE(!block_sums || block_size > 0, SPARDA_ERR_SHAPE, "offload_append: block_size must be > 0");
    SPARDA_REQUIRE(n <= (int64_t(1) << 24), SPARDA_ERR_SHAPE, "offload_append: too many tokens in one call");
    return offload_append(h, k, v, sb, st, sh, pos, n, block_size, block_sums, static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_offload_rebuild_sums(sparda_offload_t h, int64_t len, int64_t block_size,
                                           float* block_sums, void* stream) {
    SPARDA_REQUIRE(h, SPARDA_ERR_HANDLE, "offload_rebuild_sums: null handle");
    SPARDA_REQUIRE(block_sums, SPARDA_ERR_NULL, "offload_rebuild_sums: null block_sums");
    SPARDA_REQUIRE(block_size > 0 && len >= 1 && len <= offload_max_seq(h), SPARDA_ERR_SHAPE,
                   "offload_rebuild_sums: bad len/block_size");
    return offload_rebuild_sums(h, len, block_size, block_sums, static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_teacher_mass(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k,
                                   int64_t k_sb, int64_t k_st, int64_t k_sh, int dtype, int64_t B, int64_t T,
                                   int64_t Hq, int64_t Hkv, int64_t D, int64_t block_size, int causal, float scale,
                                   float* mass, void* stream) {
    SPARDA_REQUIRE(q && k && mass, SPARDA_ERR_NULL, "teacher_mass: null pointer");
    SPARDA_REQUIRE(dtype == SPARDA_BF16, SPARDA_ERR_DTYPE, "teacher_mass: bf16 q and k only");
    SPARDA_REQUIRE(D == 64 && block_size == 64, SPARDA_ERR_SHAPE, "teacher_mass: head dim and block size 64 only");
    SPARDA_REQUIRE(B >= 1 && T >= 1 && Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0 && Hq / Hkv <= 3, SPARDA_ERR_SHAPE,
                   "teacher_mass: need Hq = R * Hkv with R in {1, 2, 3}");
    SPARDA_REQUIRE(q_sb % 8 == 0 && q_st % 8 == 0 && q_sh % 8 == 0 && k_sb % 8 == 0 && k_st % 8 == 0 &&
                       k_sh % 8 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(k) % 16 == 0,
                   SPARDA_ERR_STRIDE, "teacher_mass: q and k rows must be 16-byte aligned");
    SPARDA_REQUIRE(B * Hkv * cdiv(T, 64) < (int64_t(1) << 31), SPARDA_ERR_SHAPE, "teacher_mass: too large");
    return launch_teacher_mass(q, q_sb, q_st, q_sh, k, k_sb, k_st, k_sh, B, T, Hq, Hkv, causal != 0, scale, mass,
                               static_cast<hipStream_t>(stream));
}

static int produce_impl(const void* x, int64_t x_stride_row, const void* w, int64_t M, int64_t C, int64_t Nq,
                        int64_t Nk, int64_t Nf, float eps, const float* rope_cos, const float* rope_sin,
                        int64_t rope_len, int64_t T, int64_t pos0, const int64_t* pos_dev, void* q, void* k,
                        void* v, void* f, int f_dtype, void* stream, void* kc = nullptr, void* vc = nullptr,
                        int64_t c_sb = 0, int64_t c_st = 0, int64_t c_sh = 0, int64_t cap = 0) {
    SPARDA_REQUIRE(x && w && rope_cos && rope_sin && q && k && v && f, SPARDA_ERR_NULL, "produce: null pointer");
    SPARDA_REQUIRE(f_dtype == SPARDA_F32 || f_dtype == SPARDA_BF16, SPARDA_ERR_DTYPE,
                   "produce: forecast dtype %d unsupported", f_dtype);
    SPARDA_REQUIRE(M >= 1 && T >= 1 && M % T == 0 && pos0 >= 0, SPARDA_ERR_SHAPE,
                   "produce: need M >= 1 rows, a multiple of T >= 1, pos0 >= 0");
    SPARDA_REQUIRE(C >= 32 && C % 32 == 0 && C <= 65536, SPARDA_ERR_SHAPE,
                   "produce: model width %lld must be a positive multiple of 32", (long long)C);
    SPARDA_REQUIRE(Nq > 0 && Nk > 0 && Nf > 0 && Nq % 64 == 0 && Nk % 64 == 0 && Nf % 64 == 0 &&
                       (Nq + 2 * Nk + Nf) % 128 == 0,
                   SPARDA_ERR_SHAPE, "produce: regions must be whole 64-wide heads, %lld columns in all a "
                   "multiple of 128", (long long)(Nq + 2 * Nk + Nf));
    SPARDA_REQUIRE(pos0 + T <= rope_len, SPARDA_ERR_SHAPE, "produce: positions up to %lld beyond the RoPE "
                   "tables (%lld)", (long long)(pos0 + T), (long long)rope_len);
    SPARDA_REQUIRE(!pos_dev || (reinterpret_cast<uintptr_t>(pos_dev) & 7u) == 0, SPARDA_ERR_STRIDE,
                   "produce_at: pos_dev must be 8-byte aligned");
    SPARDA_REQUIRE(x_stride_row >= C && x_stride_row % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(w) % 16 == 0,
                   SPARDA_ERR_STRIDE, "produce: x rows and w must be 16-byte aligned");
    SPARDA_REQUIRE(M / 128 < (int64_t(1) << 31), SPARDA_ERR_SHAPE, "produce: too many rows");
    return launch_produce(x, x_stride_row, w, M, C, Nq, Nk, Nf, eps, rope_cos, rope_sin, T, pos0, q, k, v, f,
                          f_dtype, static_cast<hipStream_t>(stream), pos_dev, rope_len, kc, vc, c_sb, c_st, c_sh,
                          cap);
}

SPARDA_API int sparda_produce(const void* x, int64_t x_stride_row, const void* w, int64_t M, int64_t C,
                              int64_t Nq, int64_t Nk, int64_t Nf, float eps, const float* rope_cos,
                              const float* rope_sin, int64_t rope_len, int64_t T, int64_t pos0, void* q, void* k,
                              void* v, void* f, int f_dtype, void* stream) {
    return produce_impl(x, x_stride_row, w, M, C, Nq, Nk, Nf, eps, rope_cos, rope_sin, rope_len, T, pos0, nullptr,
                        q, k, v, f, f_dtype, stream);
}

SPARDA_API int sparda_produce_at(const void* x, int64_t x_stride_row, const void* w, int64_t M, int64_t C,
                                 int64_t Nq, int64_t Nk, int64_t Nf, float eps, const float* rope_cos,
                                 const float* rope_sin, int64_t rope_len, int64_t T, const int64_t* pos_dev,
                                 void* q, void* k, void* v, void* f, int f_dtype, void* stream) {
    SPARDA_REQUIRE(pos_dev, SPARDA_ERR_NULL, "produce_at: null pos_dev");
    return produce_impl(x, x_stride_row, w, M, C, Nq, Nk, Nf, eps, rope_cos, rope_sin, rope_len, T, 0, pos_dev, q,
                        k, v, f, f_dtype, stream);
}

SPARDA_API int sparda_produce_cache_at(const void* x, int64_t x_stride_row, const void* w, int64_t M, int64_t C,
                                       int64_t Nq, int64_t Nk, int64_t Nf, float eps, const float* rope_cos,
                                       const float* rope_sin, int64_t rope_len, int64_t T, const int64_t* pos_dev,
                                       void* q, void* k, void* v, void* f, int f_dtype, void* k_cache,
                                       void* v_cache, int64_t sb, int64_t st, int64_t sh, int64_t max_len,
                                       void* stream) {
    SPARDA_REQUIRE(pos_dev && k_cache && v_cache, SPARDA_ERR_NULL, "produce_cache_at: null pos_dev or cache");
    SPARDA_REQUIRE(M >= 1 && M <= 16 && C % 128 == 0 && C / 128 <= 16, SPARDA_ERR_SHAPE,
                   "produce_cache_at: decode-sized batches only (M <= 16 rows, C a multiple of 128 up to 2048)");
    SPARDA_REQUIRE(max_len >= 1 && sb > 0 && st > 0 && sh > 0, SPARDA_ERR_SHAPE,
                   "produce_cache_at: cache strides and capacity must be positive");
    return produce_impl(x, x_stride_row, w, M, C, Nq, Nk, Nf, eps, rope_cos, rope_sin, rope_len, T, 0, pos_dev, q,
                        k, v, f, f_dtype, stream, k_cache, v_cache, sb, st, sh, max_len);
}

SPARDA_API int sparda_decode_sums(const void* q, int64_t q_sb, int64_t q_sh, const void* k, const void* v,
                                  int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int dtype, const void* forecast,
                                  int f_dtype, int64_t f_sb, int64_t f_sh, float* block_sums,
                                  int64_t nb_stride, int update_current, int64_t B, int64_t S,
                                  const int64_t* pos_dev, int64_t Hq,
                                  int64_t Hkv, int64_t D, int64_t block_size, int64_t top_k, int routing,
                                  float scale, float route_scale, int32_t* sel_out, int32_t* n_sel_out, void* out,
                                  int64_t out_sb, void* stream) {
    SPARDA_REQUIRE(q && k && v && out && forecast && block_sums, SPARDA_ERR_NULL, "decode_sums: null pointer");
    SPARDA_REQUIRE(!sel_out == !n_sel_out, SPARDA_ERR_NULL, "decode_sums: sel_out and n_sel_out go together");
    SPARDA_REQUIRE(!pos_dev || (reinterpret_cast<uintptr_t>(pos_dev) & 7u) == 0, SPARDA_ERR_STRIDE,
                   "decode_sums: pos_dev must be 8-byte aligned");
    SPARDA_REQUIRE(dtype_ok(dtype) && dtype_ok(f_dtype), SPARDA_ERR_DTYPE, "decode_sums: dtype %d / %d unsupported",
                   dtype, f_dtype);
    SPARDA_REQUIRE(routing == SPARDA_ROUTE_REFERENCE || routing == SPARDA_ROUTE_ABSOLUTE, SPARDA_ERR_MODE,
                   "decode_sums: unknown routing %d", routing);
    SPARDA_REQUIRE(B > 0 && S > 0 && Hq > 0 && Hkv > 0 && block_size > 0, SPARDA_ERR_SHAPE,
                   "decode_sums: sizes must be positive");
    SPARDA_REQUIRE(head_dim_ok(D), SPARDA_ERR_SHAPE, "decode_sums: head dim %lld not in {16,32,64,128}",
                   (long long)D);
    SPARDA_REQUIRE(Hq % Hkv == 0 && Hq / Hkv <= kMaxGroupAbi, SPARDA_ERR_SHAPE,
                   "decode_sums: Hq must be a multiple of Hkv with ratio <= 16");
    SPARDA_REQUIRE(top_k >= 1 && top_k <= kMaxTopK, SPARDA_ERR_SHAPE, "decode_sums: top_k out of range");
    SPARDA_REQUIRE(nb_stride >= cdiv(S, block_size) && cdiv(S, block_size) <= 4096, SPARDA_ERR_SHAPE,
                   "decode_sums: need ceil(S/bs) <= nb_stride and <= 4096 blocks");
    SPARDA_REQUIRE((reinterpret_cast<uintptr_t>(block_sums) & 15u) == 0, SPARDA_ERR_STRIDE,
                   "decode_sums: block_sums must be 16-byte aligned");
    SPARDA_REQUIRE(B <= 65535 && Hkv <= 65535, SPARDA_ERR_SHAPE, "decode_sums: grid too large");
    const int64_t ve = 16 / (dtype == SPARDA_F32 ? 4 : 2);
    SPARDA_REQUIRE(aligned16(k) && aligned16(v) && kv_sb % ve == 0 && kv_ss % ve == 0 && kv_sh % ve == 0,
                   SPARDA_ERR_STRIDE, "decode_sums: K/V rows must be 16-byte aligned");
    return launch_decode_sums(q, q_sb, q_sh, k, v, kv_sb, kv_ss, kv_sh, dtype, forecast, f_dtype, f_sb, f_sh,
                              block_sums, nb_stride, update_current, B, S, pos_dev, Hq, Hkv, D, block_size, top_k,
                              routing, scale,
                              route_scale, sel_out, n_sel_out, out, out_sb, static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_ffn_decode(const void* x, int64_t x_stride_row, const void* w_gate_up, const void* w_down,
                                 int64_t M, int64_t C, int64_t F, float eps, void* act, void* out,
                                 int64_t out_stride_row, void* stream) {
    SPARDA_REQUIRE(x && w_gate_up && w_down && act && out, SPARDA_ERR_NULL, "ffn_decode: null pointer");
    SPARDA_REQUIRE(M >= 1 && M <= 16, SPARDA_ERR_SHAPE, "ffn_decode: %lld rows (decode batches of 1..16)",
                   (long long)M);
    SPARDA_REQUIRE(C >= 128 && C % 128 == 0 && C <= 1024, SPARDA_ERR_SHAPE,
                   "ffn_decode: model width %lld must be a multiple of 128 up to 1024", (long long)C);
    SPARDA_REQUIRE(F >= 128 && F % 128 == 0 && F <= 2048, SPARDA_ERR_SHAPE,
                   "ffn_decode: hidden width %lld must be a multiple of 128 up to 2048", (long long)F);
    SPARDA_REQUIRE(x_stride_row >= C && x_stride_row % 8 == 0 && out_stride_row >= C && out_stride_row % 8 == 0 &&
                       aligned16(x) && aligned16(w_gate_up) && aligned16(w_down) && aligned16(act) && aligned16(out),
                   SPARDA_ERR_STRIDE, "ffn_decode: rows and weights must be 16-byte aligned");
    return launch_ffn_decode(x, x_stride_row, w_gate_up, w_down, M, C, F, eps, act, out, out_stride_row,
                             static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_ffn_decode_prefetch(const void* x, int64_t x_stride_row, const void* w_gate_up,
                                          const void* w_down, int64_t M, int64_t C, int64_t F, float eps, void* act,
                                          void* out, int64_t out_stride_row, const sparda_prefetch_args* gate_up_next,
                                          const sparda_prefetch_args* down_next, const int64_t* pos_dev,
                                          int64_t block_size, void* stream) {
    SPARDA_REQUIRE(gate_up_next || down_next, SPARDA_ERR_NULL, "ffn_decode_prefetch: no prefetch arguments");
    SPARDA_REQUIRE(pos_dev && (reinterpret_cast<uintptr_t>(pos_dev) & 7u) == 0, SPARDA_ERR_NULL,
                   "ffn_decode_prefetch: pos_dev must be a non-null, 8-byte aligned int64");
    SPARDA_REQUIRE(x && w_gate_up && w_down && act && out, SPARDA_ERR_NULL, "ffn_decode_prefetch: null pointer");
    SPARDA_REQUIRE(M >= 1 && M <= 16, SPARDA_ERR_SHAPE, "ffn_decode_prefetch: %lld rows (decode batches of 1..16)",
                   (long long)M);
    SPARDA_REQUIRE(C >= 128 && C % 128 == 0 && C <= 1024, SPARDA_ERR_SHAPE,
                   "ffn_decode_prefetch: model width %lld must be a multiple of 128 up to 1024", (long long)C);
    SPARDA_REQUIRE(F >= 128 && F % 128 == 0 && F <= 2048, SPARDA_ERR_SHAPE,
                   "ffn_decode_prefetch: hidden width %lld must be a multiple of 128 up to 2048", (long long)F);
    SPARDA_REQUIRE(x_stride_row >= C && x_stride_row % 8 == 0 && out_stride_row >= C && out_stride_row % 8 == 0 &&
                       aligned16(x) && aligned16(w_gate_up) && aligned16(w_down) && aligned16(act) && aligned16(out),
                   SPARDA_ERR_STRIDE, "ffn_decode_prefetch: rows and weights must be 16-byte aligned");
    // the copy (stage 2) uses no position bound: max_len 1 passes the selection's checks
    PrefetchDev pg, pd;
    int64_t heads = 0;
    for (int i = 0; i < 2; ++i) {
        const sparda_prefetch_args* n = i == 0 ? gate_up_next : down_next;
        if (!n) continue;
        SPARDA_REQUIRE(n->stage == 2, SPARDA_ERR_MODE, "ffn_decode_prefetch: the carried prefetch must be stage 2");
        SPARDA_REQUIRE(n->arena, SPARDA_ERR_HANDLE, "ffn_decode_prefetch: null arena handle");
        const int64_t h = offload_heads(n->arena);
        SPARDA_REQUIRE(heads == 0 || h == heads, SPARDA_ERR_SHAPE, "ffn_decode_prefetch: the two arenas' heads differ");
        heads = h;
        const int rc = prefetch_dev(n, M, h, 64, SPARDA_BF16, 1, block_size, "ffn_decode_prefetch",
                                    i == 0 ? &pg : &pd);
        if (rc) return rc;
    }
    return launch_ffn_decode(x, x_stride_row, w_gate_up, w_down, M, C, F, eps, act, out, out_stride_row,
                             static_cast<hipStream_t>(stream), gate_up_next ? &pg : nullptr,
                             down_next ? &pd : nullptr, M * heads, pos_dev);
}

SPARDA_API int sparda_norm_gemv(const void* x, int64_t x_stride_row, const void* w, int64_t M, int64_t C,
                                int64_t N, float eps, void* out, int64_t out_stride_row, void* stream) {
    SPARDA_REQUIRE(x && w && out, SPARDA_ERR_NULL, "norm_gemv: null pointer");
    SPARDA_REQUIRE(M >= 1 && M <= 16, SPARDA_ERR_SHAPE, "norm_gemv: %lld rows (decode batches of 1..16)",
                   (long long)M);
    SPARDA_REQUIRE(C >= 128 && C % 128 == 0 && C <= 1024, SPARDA_ERR_SHAPE,
                   "norm_gemv: width %lld must be a multiple of 128 up to 1024", (long long)C);
    SPARDA_REQUIRE(N >= 16 && N % 16 == 0 && N / 16 < (int64_t(1) << 31), SPARDA_ERR_SHAPE,
                   "norm_gemv: %lld outputs, need a multiple of 16", (long long)N);
    SPARDA_REQUIRE(x_stride_row >= C && x_stride_row % 8 == 0 && out_stride_row >= N && aligned16(x) && aligned16(w),
                   SPARDA_ERR_STRIDE, "norm_gemv: rows and weights must be 16-byte aligned");
    return launch_norm_gemv(x, x_stride_row, w, M, C, N, eps, out, out_stride_row, static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_rows_residual(const void* a, int64_t a_stride_row, const void* w, int64_t M, int64_t K,
                                    int64_t N, const void* res, int64_t res_stride_row, void* out,
                                    int64_t out_stride_row, void* stream) {
    SPARDA_REQUIRE(a && w && res && out, SPARDA_ERR_NULL, "rows_residual: null pointer");
    SPARDA_REQUIRE(M >= 1 && M <= 16, SPARDA_ERR_SHAPE, "rows_residual: %lld rows (decode batches of 1..16)",
                   (long long)M);
    SPARDA_REQUIRE(K >= 128 && K % 128 == 0 && K <= 2048, SPARDA_ERR_SHAPE,
                   "rows_residual: input width %lld must be a multiple of 128 up to 2048", (long long)K);
    SPARDA_REQUIRE(N >= 16 && N % 16 == 0, SPARDA_ERR_SHAPE, "rows_residual: output width %lld must be a multiple "
                   "of 16", (long long)N);
    SPARDA_REQUIRE(a_stride_row >= K && a_stride_row % 8 == 0 && res_stride_row >= N && out_stride_row >= N &&
                       aligned16(a) && aligned16(w),
                   SPARDA_ERR_STRIDE, "rows_residual: input rows and weights must be 16-byte aligned");
    return launch_rows_residual(a, a_stride_row, w, M, K, N, res, res_stride_row, out, out_stride_row,
                                static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_append_at(void* k_cache, void* v_cache, int dtype, int64_t sb, int64_t st, int64_t sh,
                                const void* k_new, const void* v_new, int64_t new_sb, int64_t new_sh, int64_t B,
                                int64_t Hkv, int64_t D, int64_t max_len, const int64_t* pos_dev,
                                int64_t block_size, int64_t nb_stride, float* block_sums, void* stream) {
    SPARDA_REQUIRE(k_cache && pos_dev, SPARDA_ERR_NULL, "append_at: null k_cache/pos_dev");
    SPARDA_REQUIRE(!k_new == !v_new, SPARDA_ERR_NULL, "append_at: k_new and v_new go together");
    SPARDA_REQUIRE(k_new || block_sums, SPARDA_ERR_NULL, "append_at: nothing to do (no new rows, no block sums)");
    SPARDA_REQUIRE(!k_new || v_cache, SPARDA_ERR_NULL, "append_at: appending needs v_cache");
    SPARDA_REQUIRE((reinterpret_cast<uintptr_t>(pos_dev) & 7u) == 0, SPARDA_ERR_STRIDE,
                   "append_at: pos_dev must be 8-byte aligned");
    SPARDA_REQUIRE(dtype_ok(dtype), SPARDA_ERR_DTYPE, "append_at: dtype %d unsupported", dtype);
    SPARDA_REQUIRE(B > 0 && Hkv > 0 && D > 0 && block_size > 0 && nb_stride > 0 && max_len >= 1, SPARDA_ERR_SHAPE,
                   "append_at: sizes must be positive");
    SPARDA_REQUIRE((max_len - 1) / block_size < nb_stride, SPARDA_ERR_CAPACITY,
                   "append_at: max_len %lld needs more than nb_stride %lld blocks", (long long)max_len,
                   (long long)nb_stride);
    SPARDA_REQUIRE(sb >= 0 && st >= 0 && sh >= 0 && new_sb >= 0 && new_sh >= 0, SPARDA_ERR_STRIDE,
                   "append_at: negative stride");
    SPARDA_REQUIRE(B <= 65535, SPARDA_ERR_SHAPE, "append_at: too large");
    return launch_append_at(k_cache, v_cache, dtype, sb, st, sh, k_new, v_new, new_sb, new_sh, B, Hkv, D, block_size,
                            max_len, nb_stride, pos_dev, block_sums, static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_block_sums(const void* k, int dtype, int64_t sb, int64_t st, int64_t sh, int64_t B,
                                 int64_t Hkv, int64_t D, int64_t pos, int64_t n, int64_t block_size,
                                 int64_t nb_stride, float* block_sums, void* stream) {
    SPARDA_REQUIRE(k && block_sums, SPARDA_ERR_NULL, "block_sums: null k/block_sums");
    SPARDA_REQUIRE(dtype_ok(dtype), SPARDA_ERR_DTYPE, "block_sums: dtype %d unsupported", dtype);
    SPARDA_REQUIRE(B > 0 && Hkv > 0 && D > 0 && block_size > 0 && nb_stride > 0, SPARDA_ERR_SHAPE,
                   "block_sums: sizes must be positive");
    SPARDA_REQUIRE(pos >= 0 && n >= 1, SPARDA_ERR_SHAPE, "block_sums: need pos >= 0, n >= 1");
    SPARDA_REQUIRE((pos + n - 1) / block_size < nb_stride, SPARDA_ERR_CAPACITY,
                   "block_sums: block %lld beyond nb_stride %lld", (long long)((pos + n - 1) / block_size),
                   (long long)nb_stride);
    SPARDA_REQUIRE(sb >= 0 && st >= 0 && sh >= 0, SPARDA_ERR_STRIDE, "block_sums: negative stride");
    SPARDA_REQUIRE(B <= 65535 && (pos + n - 1) / block_size - pos / block_size < (int64_t(1) << 31),
                   SPARDA_ERR_SHAPE, "block_sums: too large");
    const char* kp = static_cast<const char*>(k) + pos * st * (dtype == SPARDA_F32 ? 4 : 2);
    return launch_block_sums(kp, dtype, sb, st, sh, pos, n, B, Hkv, D, block_size, nb_stride, block_sums,
                             static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_offload_fetch(sparda_offload_t h, const int32_t* sel, const int32_t* n_sel,
                                    int64_t sel_cap, int64_t block_size, int64_t len, int method, void* k_dst,
                                    void* v_dst, void* stream) {
    SPARDA_REQUIRE(h, SPARDA_ERR_HANDLE, "offload_fetch: null handle");
    SPARDA_REQUIRE(sel && n_sel && k_dst && v_dst, SPARDA_ERR_NULL, "offload_fetch: null pointer");
    SPARDA_REQUIRE(method == SPARDA_FETCH_KERNEL || method == SPARDA_FETCH_DMA, SPARDA_ERR_MODE,
                   "offload_fetch: unknown method %d", method);
    SPARDA_REQUIRE(block_size > 0 && len >= 0 && len <= offload_max_seq(h), SPARDA_ERR_SHAPE,
                   "offload_fetch: bad len/block_size");
    SPARDA_REQUIRE(sel_cap >= 1 && sel_cap <= (method == SPARDA_FETCH_DMA ? kMaxFetchSlots : 65535),
                   SPARDA_ERR_SHAPE, "offload_fetch: sel_cap %lld out of range", (long long)sel_cap);
    SPARDA_REQUIRE(aligned16(k_dst) && aligned16(v_dst), SPARDA_ERR_STRIDE,
                   "offload_fetch: destinations must be 16-byte aligned");
    return offload_fetch(h, sel, n_sel, sel_cap, block_size, len, method, k_dst, v_dst,
                         static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_offload_fetch_at(sparda_offload_t h, const int32_t* sel, const int32_t* n_sel,
                                       int64_t sel_cap, int64_t block_size, const int64_t* len_dev, void* k_dst,
                                       void* v_dst, void* stream) {
    SPARDA_REQUIRE(h, SPARDA_ERR_HANDLE, "offload_fetch_at: null handle");
    SPARDA_REQUIRE(sel && n_sel && k_dst && v_dst && len_dev, SPARDA_ERR_NULL, "offload_fetch_at: null pointer");
    SPARDA_REQUIRE((reinterpret_cast<uintptr_t>(len_dev) & 7u) == 0, SPARDA_ERR_STRIDE,
                   "offload_fetch_at: len_dev must be 8-byte aligned");
    SPARDA_REQUIRE(block_size > 0, SPARDA_ERR_SHAPE, "offload_fetch_at: bad block_size");
    SPARDA_REQUIRE(sel_cap >= 1 && sel_cap <= 65535, SPARDA_ERR_SHAPE, "offload_fetch_at: sel_cap %lld out of range",
                   (long long)sel_cap);
    SPARDA_REQUIRE(aligned16(k_dst) && aligned16(v_dst), SPARDA_ERR_STRIDE,
                   "offload_fetch_at: destinations must be 16-byte aligned");
    return offload_fetch(h, sel, n_sel, sel_cap, block_size, 0, SPARDA_FETCH_KERNEL, k_dst, v_dst,
                         static_cast<hipStream_t>(stream), len_dev);
}

SPARDA_API int sparda_offload_append_at(sparda_offload_t h, const void* k, const void* v, int64_t new_sb,
                                        int64_t new_sh, const int64_t* pos_dev, int64_t block_size,
                                        float* block_sums, void* stream) {
    SPARDA_REQUIRE(h, SPARDA_ERR_HANDLE, "offload_append_at: null handle");
    SPARDA_REQUIRE(k && v && pos_dev, SPARDA_ERR_NULL, "offload_append_at: null k/v/pos_dev");
    SPARDA_REQUIRE((reinterpret_cast<uintptr_t>(pos_dev) & 7u) == 0, SPARDA_ERR_STRIDE,
                   "offload_append_at: pos_dev must be 8-byte aligned");
    SPARDA_REQUIRE(new_sb >= 0 && new_sh >= 0, SPARDA_ERR_STRIDE, "offload_append_at: negative stride");
    SPARDA_REQUIRE(!block_sums || block_size > 0, SPARDA_ERR_SHAPE, "offload_append_at: block_size must be > 0");
    return offload_append_at(h, k, v, new_sb, new_sh, pos_dev, block_sums ? block_size : 1, block_sums,
                             static_cast<hipStream_t>(stream));
}

SPARDA_API int sparda_offload_append_at_prefetch(sparda_offload_t h, const void* k, const void* v, int64_t new_sb,
                                                 int64_t new_sh, const int64_t* pos_dev, int64_t block_size,
                                                 float* block_sums, int64_t max_len,
                                                 const sparda_prefetch_args* next, void* stream) {
    SPARDA_REQUIRE(h, SPARDA_ERR_HANDLE, "offload_append_at_prefetch: null handle");
    SPARDA_REQUIRE(k && v && pos_dev, SPARDA_ERR_NULL, "offload_append_at_prefetch: null k/v/pos_dev");
    SPARDA_REQUIRE((reinterpret_cast<uintptr_t>(pos_dev) & 7u) == 0, SPARDA_ERR_STRIDE,
                   "offload_append_at_prefetch: pos_dev must be 8-byte aligned");
    SPARDA_REQUIRE(new_sb >= 0 && new_sh >= 0, SPARDA_ERR_STRIDE, "offload_append_at_prefetch: negative stride");
    SPARDA_REQUIRE(block_size > 0, SPARDA_ERR_SHAPE, "offload_append_at_prefetch: block_size must be > 0");
    PrefetchDev pf;
    const int rc = prefetch_dev(next, offload_batch(h), offload_heads(h), offload_head_dim(h), offload_dtype(h),
                                max_len, block_size, "offload_append_at_prefetch", &pf);
    if (rc) return rc;
    return offload_append_at(h, k, v, new_sb, new_sh, pos_dev, block_size, block_sums,
                             static_cast<hipStream_t>(stream), &pf);
}

}  // extern "C"
