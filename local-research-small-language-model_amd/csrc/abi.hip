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

}  // namespace sparda

using namespace sparda;

extern "C" {

SPARDA_API int sparda_version(void) { return 100; }

SPARDA_API const char* sparda_last_error(void) { return g_last_error; }

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
    SPARDA_REQUIRE(q && k_cache && v_cache && out, SPARDA_ERR_NULL, "decode: null q/k/v/out");
    SPARDA_REQUIRE(workspace, SPARDA_ERR_WORKSPACE, "decode: workspace is required");
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
    const DecodeWs ws = decode_ws_layout(workspace, B, S, Hq, Hkv, D, block_size, top_k);
    SPARDA_REQUIRE(workspace_bytes >= ws.bytes, SPARDA_ERR_WORKSPACE, "decode: workspace %zu < %zu bytes",
                   workspace_bytes, ws.bytes);
    SPARDA_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255u) == 0, SPARDA_ERR_WORKSPACE,
                   "decode: workspace must be 256-byte aligned");
    return launch_decode(q, q_sb, q_sh, k_cache, v_cache, kv_sb, kv_ss, kv_sh, dtype, forecast, f_dtype, f_sb,
                         f_sh, B, S, Hq, Hkv, D, block_size, top_k, routing, scale, protos_in, protos_out,
                         sel_out, n_sel_out, out, out_sb, ws, static_cast<hipStream_t>(stream));
}

}  // extern "C"
