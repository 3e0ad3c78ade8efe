// Allocation-free decode step: sparda_decode with its workspace (the block
// scores of the step) in a file-scope device array instead of caller memory,
// for callers that cannot allocate (code under HIP graph capture, serving
// loops that forbid allocation). The kernels are the ones sparda_decode runs.
//
// Every GPU the library runs on holds its own copy of `scratch` for the life
// of the process. Its device address is looked up once per device, with that
// device current, through hipGetSymbolAddress; host code uses only that
// address (the array's name on the host is a stand-in, not device memory).
// Calls on one GPU share the array: two calls that overlap in time on one
// GPU (different streams without ordering between them) race on it.
#include <mutex>

#include "common.h"
#include "kernels.h"

namespace sparda {

constexpr size_t kScratchBytes = size_t(1) << 20;  // 1 MiB: B * Hkv * NB <= 262,144 block scores
constexpr int kMaxScratchDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxScratchDevices];

// Device address of the current device's copy of `scratch` (looked up on the
// first call on that device).
static int scratch_address(void** out) {
    int dev = -1;
    SPARDA_HIP(hipGetDevice(&dev));
    SPARDA_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, SPARDA_ERR_SHAPE,
                   "decode_noalloc: device %d beyond the %d the library tracks", dev, kMaxScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return check_hip(e, "hipGetSymbolAddress(scratch)");
        SPARDA_REQUIRE(ptr != nullptr && (reinterpret_cast<uintptr_t>(ptr) & 255u) == 0, SPARDA_ERR_WORKSPACE,
                       "decode_noalloc: scratch address %p is not 256-byte aligned", ptr);
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

}  // namespace sparda

using namespace sparda;

extern "C" {

SPARDA_API int sparda_decode_noalloc(const void* q, int64_t q_sb, int64_t q_sh, const void* k_cache,
                                     const void* v_cache, int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int dtype,
                                     const void* forecast, int f_dtype, int64_t f_sb, int64_t f_sh, int64_t B,
                                     int64_t S, int64_t Hq, int64_t Hkv, int64_t D, int64_t block_size,
                                     int64_t top_k, int routing, float scale, const float* protos_in,
                                     float* protos_out, int32_t* sel_out, int32_t* n_sel_out, void* out,
                                     int64_t out_sb, void* stream) {
    int rc = check_decode_args(q, k_cache, v_cache, kv_sb, kv_ss, kv_sh, dtype, forecast, f_dtype, B, S, Hq, Hkv, D,
                               block_size, top_k, routing, sel_out, n_sel_out, out);
    if (rc) return rc;
    const size_t need = decode_ws_layout(nullptr, B, S, Hq, Hkv, D, block_size, top_k).bytes;
    SPARDA_REQUIRE(need <= kScratchBytes, SPARDA_ERR_CAPACITY,
                   "decode_noalloc: the step needs %zu bytes of scratch, more than the %zu the library holds "
                   "(use sparda_decode with a workspace)", need, kScratchBytes);
    void* ws_ptr = nullptr;
    rc = scratch_address(&ws_ptr);
    if (rc) return rc;
    // every score the attend launch reads is written by the score launch of
    // the same call: nothing in the scratch has to start at zero
    const DecodeWs ws = decode_ws_layout(ws_ptr, B, S, Hq, Hkv, D, block_size, top_k);
    return launch_decode(q, q_sb, q_sh, k_cache, v_cache, kv_sb, kv_ss, kv_sh, dtype, forecast, f_dtype, f_sb, f_sh,
                         B, S, Hq, Hkv, D, block_size, top_k, routing, scale, protos_in, protos_out, sel_out,
                         n_sel_out, out, out_sb, ws, static_cast<hipStream_t>(stream));
}

}  // extern "C"
