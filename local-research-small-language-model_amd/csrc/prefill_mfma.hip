// bf16 block-sparse GQA prefill on the gfx950 matrix cores (D = 64, bs = 64).
//
// One workgroup (4 wavefronts) serves one (sequence b, KV head g, query block
// qb): 64 query tokens x R = Hq/Hkv query heads. Wavefront w owns tokens
// [16w, 16w+16) of the block for all R heads, i.e. 16R "columns"
// (column c -> token c / R, head c % R), processed as R tiles of 16 columns.
//
// The workgroup walks the union of its tokens' selected KV blocks in
// ascending order. Each block's K (row-major) and V (transposed) are staged
// once in LDS (double-buffered) and shared by all R heads; a tile skips a
// block none of its columns selected, and columns that did not select it are
// masked. Per tile and block, with v_mfma_f32_16x16x32_bf16:
//     S^T[key, col] = K[key, :] . Q[col, :]           (8 MFMA)
//     online softmax per column (fp32, log2 domain)
//     O^T[d, col]  += V^T[d, key] . P^T[key, col]      (8 MFMA)
// S^T leaves each lane with 4 consecutive keys of 4 key tiles for one column,
// which is directly the B operand of the PV product when the 32-key k-axis is
// enumerated as {32m + 4g + e, 32m + 16 + 4g + e} (g = lane / 16); the V^T A
// operand is read from LDS with the same enumeration.
#include "common.h"
#include "kernels.h"

namespace sparda {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMBs = 64;          // block size (keys per KV block)
constexpr int kMD = 64;           // head dim
constexpr int kMThreads = 256;    // 4 wavefronts
constexpr int kKRow = kMD + 8;    // K row in LDS, bf16 elements (144 B: 16 B aligned)
constexpr int kVRow = kMBs + 4;   // V^T row in LDS, bf16 elements (136 B)
constexpr int kMaxNBWords = 32;   // selection bitmask words per token (NB <= 1024)
constexpr float kLog2eM = 1.4426950408889634f;

struct MfmaSmem {
    uint16_t k[2][kMBs * kKRow];
    uint16_t vt[2][kMD * kVRow];
    uint32_t mask[64 * kMaxNBWords];
    uint16_t list[kMaxNBWords * 32];
    int n_list;
};

__device__ __forceinline__ bf16x8 lds_read8(const uint16_t* p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}
__device__ __forceinline__ bf16x8 lds_read4x2(const uint16_t* p0, const uint16_t* p1) {
    const uint2 a = *reinterpret_cast<const uint2*>(p0);
    const uint2 c = *reinterpret_cast<const uint2*>(p1);
    return __builtin_bit_cast(bf16x8, make_uint4(a.x, a.y, c.x, c.y));
}

template <int R>
__global__ void __launch_bounds__(kMThreads, 2)
prefill_mfma_kernel(const uint16_t* __restrict__ q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                    int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                    const int32_t* __restrict__ sel, const int32_t* __restrict__ n_sel, int64_t cap,
                    int64_t T, int H, int64_t NBq, int causal, float scale_log2,
                    uint16_t* __restrict__ out, int64_t out_sb, int64_t out_st) {
    __shared__ MfmaSmem sm;
    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int wave = tid / kWave;
    const int col16 = lane % 16;   // column within a tile
    const int grp = lane / 16;     // lane group (k / row sub-block)

    // heaviest query blocks first; consecutive ids cycle through (b, g)
    const int64_t BH = static_cast<int64_t>(gridDim.x) / NBq;
    const int64_t bg = blockIdx.x % BH;
    const int64_t qb = NBq - 1 - blockIdx.x / BH;
    const int b = static_cast<int>(bg / H);
    const int g = static_cast<int>(bg % H);
    const int64_t t0 = qb * 64;
    const int64_t NB = cdiv(T, kMBs);
    const int nbw = static_cast<int>((NB + 31) / 32);

    // ---- selection bitmask per token, and the workgroup's union of blocks ----
    for (int i = tid; i < 64 * nbw; i += kMThreads) sm.mask[i] = 0u;
    __syncthreads();
    if (tid < 64) {
        const int64_t t = t0 + tid;
        uint32_t* row = sm.mask + tid * nbw;
        if (t < T) {
            if (sel != nullptr) {
                const int64_t r = (static_cast<int64_t>(b) * H + g) * T + t;
                const int n = min(static_cast<int64_t>(n_sel[r]), cap);
                for (int i = 0; i < n; ++i) {
                    const int j = sel[r * cap + i];
                    if (j >= 0 && j < NB) row[j >> 5] |= 1u << (j & 31);
                }
            } else {
                const int64_t jmax = causal ? qb : NB - 1;
                for (int64_t j = 0; j <= jmax; ++j) row[j >> 5] |= 1u << (j & 31);
            }
        }
    }
    __syncthreads();
    if (tid == 0) {
        int n = 0;
        for (int w = 0; w < nbw; ++w) {
            uint32_t u = 0;
            for (int tt = 0; tt < 64; ++tt) u |= sm.mask[tt * nbw + w];
            while (u) {
                const int bit = __builtin_ctz(u);
                sm.list[n++] = static_cast<uint16_t>(w * 32 + bit);
                u &= u - 1;
            }
        }
        sm.n_list = n;
    }

    // ---- Q^T B-operands (registers for the whole kernel) ----
    bf16x8 qb_op[R][2];
    int tok[R];          // token index within the query block for this lane's column, per tile
    int64_t tpos[R];     // absolute position
#pragma unroll
    for (int tt = 0; tt < R; ++tt) {
        const int c = 16 * tt + col16;
        const int tw = c / R;
        const int hh = c % R;
        tok[tt] = 16 * wave + tw;
        tpos[tt] = t0 + tok[tt];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            uint4 raw = make_uint4(0u, 0u, 0u, 0u);
            if (tpos[tt] < T) {
                const uint16_t* p = q + b * q_sb + tpos[tt] * q_st + static_cast<int64_t>(g * R + hh) * q_sh +
                                    32 * kk + 8 * grp;
                raw = *reinterpret_cast<const uint4*>(p);
            }
            qb_op[tt][kk] = __builtin_bit_cast(bf16x8, raw);
        }
    }

    f32x4 o[R][4];
    float m_run[R], l_run[R];
#pragma unroll
    for (int tt = 0; tt < R; ++tt) {
        m_run[tt] = -__builtin_inff();
        l_run[tt] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[tt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // ---- staging of one KV block: thread -> (row pair, 16 B chunk) ----
    const int st_chunk = tid % 8;        // 8 bf16 of d
    const int st_pair = tid / 8;         // rows 2*pair, 2*pair+1 (32 pairs)
    const uint16_t* kbase = k + b * kv_sb + static_cast<int64_t>(g) * kv_sh + st_chunk * 8;
    const uint16_t* vbase = v + b * kv_sb + static_cast<int64_t>(g) * kv_sh + st_chunk * 8;
    uint4 kreg[2], vreg[2];
    auto fetch = [&](int64_t j) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int64_t s = j * kMBs + 2 * st_pair + r;
            if (s < T) {
                kreg[r] = *reinterpret_cast<const uint4*>(kbase + s * kv_st);
                vreg[r] = *reinterpret_cast<const uint4*>(vbase + s * kv_st);
            } else {
                kreg[r] = make_uint4(0u, 0u, 0u, 0u);
                vreg[r] = make_uint4(0u, 0u, 0u, 0u);
            }
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int r = 0; r < 2; ++r)
            *reinterpret_cast<uint4*>(&sm.k[buf][(2 * st_pair + r) * kKRow + st_chunk * 8]) = kreg[r];
        const uint16_t* v0 = reinterpret_cast<const uint16_t*>(&vreg[0]);
        const uint16_t* v1 = reinterpret_cast<const uint16_t*>(&vreg[1]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t w = static_cast<uint32_t>(v0[e]) | (static_cast<uint32_t>(v1[e]) << 16);
            *reinterpret_cast<uint32_t*>(&sm.vt[buf][(st_chunk * 8 + e) * kVRow + 2 * st_pair]) = w;
        }
    };

    __syncthreads();
    const int n_list = sm.n_list;
    if (n_list > 0) {
        fetch(sm.list[0]);
        stash(0);
    }
    __syncthreads();

    for (int u = 0; u < n_list; ++u) {
        const int buf = u & 1;
        const int j = sm.list[u];
        if (u + 1 < n_list) fetch(sm.list[u + 1]);

        // which tiles of this wave need block j
        bool member[R];
        bool any = false;
#pragma unroll
        for (int tt = 0; tt < R; ++tt) {
            member[tt] = (sm.mask[tok[tt] * nbw + (j >> 5)] >> (j & 31)) & 1u;
            const bool tile_any = __ballot(member[tt]) != 0ull;
            any = any || tile_any;
        }
        if (any) {
            bf16x8 ka[4][2];
#pragma unroll
            for (int n = 0; n < 4; ++n)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk)
                    ka[n][kk] = lds_read8(&sm.k[buf][(16 * n + col16) * kKRow + 32 * kk + 8 * grp]);
            bf16x8 va[4][2];
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    const uint16_t* row = &sm.vt[buf][(16 * dt + col16) * kVRow];
                    va[dt][m] = lds_read4x2(row + 32 * m + 4 * grp, row + 32 * m + 16 + 4 * grp);
                }
            const bool diag = (j == qb);
#pragma unroll
            for (int tt = 0; tt < R; ++tt) {
                if (__ballot(member[tt]) == 0ull) continue;
                f32x4 s[4];
#pragma unroll
                for (int n = 0; n < 4; ++n) {
                    s[n] = f32x4{0.f, 0.f, 0.f, 0.f};
                    s[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[n][0], qb_op[tt][0], s[n], 0, 0, 0);
                    s[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[n][1], qb_op[tt][1], s[n], 0, 0, 0);
                }
                // mask: column not selecting j; causal diagonal; keys beyond T
                float mx = -__builtin_inff();
#pragma unroll
                for (int n = 0; n < 4; ++n)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int64_t kp = static_cast<int64_t>(j) * kMBs + 16 * n + 4 * grp + i;
                        bool ok = member[tt];
                        if (causal) ok = ok && (!diag || kp <= tpos[tt]);
                        else ok = ok && kp < T;
                        s[n][i] = ok ? s[n][i] * scale_log2 : -__builtin_inff();
                        mx = fmaxf(mx, s[n][i]);
                    }
                mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
                mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
                const float m_new = fmaxf(m_run[tt], mx);
                const bool live = m_new != -__builtin_inff();
                const float alpha = live ? __builtin_amdgcn_exp2f(m_run[tt] - m_new) : 1.0f;
                float rs = 0.0f;
#pragma unroll
                for (int n = 0; n < 4; ++n)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float p = live ? __builtin_amdgcn_exp2f(s[n][i] - m_new) : 0.0f;
                        s[n][i] = p;
                        rs += p;
                    }
                rs += __shfl_xor(rs, 16, kWave);
                rs += __shfl_xor(rs, 32, kWave);
                l_run[tt] = l_run[tt] * alpha + rs;
                m_run[tt] = m_new;
                bf16x8 pb[2];
#pragma unroll
                for (int m = 0; m < 2; ++m)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        pb[m][i] = static_cast<__bf16>(s[2 * m][i]);
                        pb[m][4 + i] = static_cast<__bf16>(s[2 * m + 1][i]);
                    }
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    o[tt][dt] *= alpha;
                    o[tt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt][0], pb[0], o[tt][dt], 0, 0, 0);
                    o[tt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt][1], pb[1], o[tt][dt], 0, 0, 0);
                }
            }
        }
        if (u + 1 < n_list) stash(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue: out[b, t, h*64 + d] = O / l ----
#pragma unroll
    for (int tt = 0; tt < R; ++tt) {
        if (tpos[tt] >= T) continue;
        const int c = 16 * tt + col16;
        const int hh = c % R;
        const float inv = 1.0f / l_run[tt];
        uint16_t* orow = out + b * out_sb + tpos[tt] * out_st + static_cast<int64_t>(g * R + hh) * kMD;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            bf16x4 w;
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = static_cast<__bf16>(o[tt][dt][i] * inv);
            *reinterpret_cast<bf16x4*>(orow + 16 * dt + 4 * grp) = w;
        }
    }
}

bool prefill_mfma_supported(int dtype, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t bs,
                            int64_t q_sb, int64_t q_st, int64_t q_sh, int64_t kv_sb, int64_t kv_st,
                            int64_t kv_sh, int64_t out_sb, int64_t out_st, const void* q, const void* k,
                            const void* v, const void* out) {
    if (dtype != SPARDA_BF16 || D != kMD || bs != kMBs) return false;
    if (cdiv(T, kMBs) > kMaxNBWords * 32) return false;
    const int64_t R = Hq / Hkv;
    if (R < 1 || R > 4) return false;
    auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!al16(q) || !al16(k) || !al16(v) || (reinterpret_cast<uintptr_t>(out) & 7u)) return false;
    if ((q_sb % 8) || (q_st % 8) || (q_sh % 8) || (kv_sb % 8) || (kv_st % 8) || (kv_sh % 8)) return false;
    if ((out_sb % 4) || (out_st % 4)) return false;
    return true;
}

int launch_prefill_mfma(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k,
                        const void* v, int64_t kv_sb, int64_t kv_st, int64_t kv_sh,
                        const int32_t* sel, const int32_t* n_sel, int64_t cap, int64_t B, int64_t T,
                        int64_t Hq, int64_t Hkv, int64_t bs, int causal, float scale, void* out,
                        int64_t out_sb, int64_t out_st, hipStream_t stream) {
    (void)bs;
    const int64_t NBq = cdiv(T, kMBs);
    const int64_t R = Hq / Hkv;
    dim3 grid(static_cast<unsigned>(B * Hkv * NBq));
    const float sl = scale * kLog2eM;
#define SPARDA_MF(R_)                                                                                     \
    hipLaunchKernelGGL((prefill_mfma_kernel<R_>), grid, dim3(kMThreads), 0, stream,                       \
                       static_cast<const uint16_t*>(q), q_sb, q_st, q_sh, static_cast<const uint16_t*>(k), \
                       static_cast<const uint16_t*>(v), kv_sb, kv_st, kv_sh, sel, n_sel, cap, T,           \
                       static_cast<int>(Hkv), NBq, causal, sl, static_cast<uint16_t*>(out), out_sb, out_st)
    switch (R) {
        case 1: SPARDA_MF(1); break;
        case 2: SPARDA_MF(2); break;
        case 3: SPARDA_MF(3); break;
        default: SPARDA_MF(4); break;
    }
#undef SPARDA_MF
    return check_hip(hipGetLastError(), "prefill_mfma_kernel");
}

}  // namespace sparda
