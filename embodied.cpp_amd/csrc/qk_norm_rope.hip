// Per-head q/k RMSNorm + RoPE on a QKV projection output, with the K and V
// heads appended into the paged cache, gfx950.
//
// Reference: the Cosmos3 language tower runs, after its three W8 projections,
// cosmos3_qwen_head_rmsnorm_f32 on Q and on K, cosmos3_qwen_rope_f32 or
// cosmos3_qwen_mrope_f32 on each, and hands K/V to attention
// (models/cosmos3.cpp:4940-5012; kernels/cosmos3/cosmos3_qwen_language_cuda.cu
// :52-83 head_rmsnorm_kernel, :85-116 rope_kernel, :117-153 mrope_kernel).
// Here one launch does all of it and the paged append: a workgroup per token,
// a wave per head of its bf16 QKV row, lane l holding dims l + 64 e (e < D/64),
// so the RoPE pair (d, d + D/2) is in one lane for D >= 128 (lanes l and l ^ 32
// for D = 64) and the head's sum of squares is one wave reduction.  Arithmetic is
// f32 with the reference's bf16 rounding points: bf16(x * inv), bf16(. *
// gamma), bf16(sin), bf16(cos), bf16(v c + r s).  sin, cos and pow are the
// device library's sincosf and powf; 1/sqrt is rsqrtf.
#include <hip/hip_runtime.h>

#include <cmath>

#include "emb_common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct NRParams {
    const uint16_t *qkv;
    int64_t ld;
    int32_t tokens, q_heads, kv_heads;
    const uint16_t *q_gamma, *k_gamma;
    float eps;
    int32_t rope_kind;
    float theta;
    int32_t first_pos;
    const int32_t *pos_ids;
    uint16_t *q_out;
    int64_t ldq;
    const int32_t *slots, *bt;
    int32_t capacity;
    uint16_t *k_pool, *v_pool, *v16_pool;
};

__device__ __forceinline__ float bf16f(uint32_t b) { return __builtin_bit_cast(float, b << 16); }

__device__ __forceinline__ uint32_t bf16_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ float round_bf16(float f) { return bf16f(bf16_rne(f)); }

// V heads: a thread per (token, head, 8-dim chunk), tokens fastest, so the
// 16 tokens of a page store one 32-byte row of the transposed V page (and of
// its f16 shadow) together (emb_kv_append's order).
template <int D>
__device__ __forceinline__ void append_v(const NRParams &p, int64_t idx) {
    constexpr int CH = D / 8;
    const int32_t s = (int32_t)(idx % p.tokens);
    const int64_t hc = idx / p.tokens;
    const int c = (int)(hc % CH), h = (int)(hc / CH);
    if (h >= p.kv_heads) return;
    const u32x4 w = *reinterpret_cast<const u32x4 *>(p.qkv + (int64_t)s * p.ld +
                                                     (int64_t)(p.q_heads + p.kv_heads + h) * D + c * 8);
    const int32_t slot = p.slots[s];
    if (slot < 0 || slot >= p.capacity) return;
    const int32_t page = p.bt ? p.bt[slot >> 4] : (slot >> 4);
    if (page < 0) return;
    const int32_t t = slot & 15;
    const int64_t pbase = ((int64_t)page * p.kv_heads + h) * 16 * D;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t b = (w[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
        const int d = c * 8 + e;
        p.v_pool[pbase + d * 16 + t] = (uint16_t)b;
        if (p.v16_pool) p.v16_pool[pbase + emb::v16_index(d, t)] = __builtin_bit_cast(uint16_t, (_Float16)bf16f(b));
    }
}

// Workgroups [0, tokens): one per token for its Q and K heads -- each lane
// first takes the bf16 cos / sin of its dims at the token's position (shared
// by every Q and K head of the token, so the transcendental work is per
// token, not per element), then the four waves loop over the heads, a wave a
// head.  Workgroups past that append the V heads (append_v).
template <int D>
__global__ __launch_bounds__(256) void qk_norm_rope_append_kernel(NRParams p) {
    constexpr int E = D / 64 > 0 ? D / 64 : 1;  // elements a lane holds
    constexpr int HALF = D / 2;
    if ((int32_t)blockIdx.x >= p.tokens) {
        append_v<D>(p, (int64_t)(blockIdx.x - p.tokens) * 256 + threadIdx.x);
        return;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int32_t tok = blockIdx.x;
    const int units = p.q_heads + p.kv_heads;
    const bool act = D >= 64 || lane < D;  // lanes holding a dim

    float cs[E], sn[E];
    if (p.rope_kind) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int d = lane + 64 * e;
            const int pd = d < HALF ? d : d - HALF;
            int axis = 0;
            if (p.rope_kind == 2 && pd < 60) axis = pd % 3 == 1 ? 1 : (pd % 3 == 2 ? 2 : 0);
            const float pos = p.rope_kind == 2 ? (float)p.pos_ids[(int64_t)axis * p.tokens + tok]
                                               : (float)(p.first_pos + tok);
            const float f = powf(p.theta, -(float)(2 * pd) / (float)D);
            float s_, c_;
            sincosf(pos * f, &s_, &c_);
            cs[e] = round_bf16(c_);
            sn[e] = round_bf16(s_);
        }
    }

    // cache destination of the token's K rows (a slot outside
    // [0, capacity) or on an unmapped page is skipped, as in emb_kv_append)
    int64_t page_base = -1;
    int32_t trow = 0;
    {
        const int32_t slot = p.slots[tok];
        if (slot >= 0 && slot < p.capacity) {
            const int32_t page = p.bt ? p.bt[slot >> 4] : (slot >> 4);
            if (page >= 0) {
                page_base = (int64_t)page * p.kv_heads * 16 * D;
                trow = slot & 15;
            }
        }
    }

    for (int u = wave; u < units; u += 4) {
        const int kind = u < p.q_heads ? 0 : 1;  // Q, K
        const int h = kind == 0 ? u : u - p.q_heads;
        const uint16_t *row = p.qkv + (int64_t)tok * p.ld + (int64_t)u * D;
        float v[E];
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = act ? bf16f(row[lane + 64 * e]) : 0.0f;
        const int64_t pbase = page_base < 0 ? -1 : page_base + (int64_t)h * 16 * D;
        const uint16_t *gamma = kind == 0 ? p.q_gamma : p.k_gamma;
        if (gamma) {  // head RMSNorm: one wave reduction of the squares
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) ss += v[e] * v[e];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
            const float inv = rsqrtf(ss / (float)D + p.eps);
#pragma unroll
            for (int e = 0; e < E; ++e)
                v[e] = round_bf16(round_bf16(v[e] * inv) * (act ? bf16f(gamma[lane + 64 * e]) : 0.0f));
        }
        if (p.rope_kind) {
            float r[E];  // rotate-half partner: -v[d + D/2] below D/2, v[d - D/2] above
            if constexpr (E >= 2) {
#pragma unroll
                for (int e = 0; e < E; ++e) r[e] = e < E / 2 ? -v[e + E / 2] : v[e - E / 2];
            } else {
                const float o = __shfl_xor(v[0], 32, 64);
                r[0] = lane < 32 ? -o : o;
            }
#pragma unroll
            for (int e = 0; e < E; ++e) v[e] = round_bf16(v[e] * cs[e] + r[e] * sn[e]);
        }
        if (!act) continue;
        if (kind == 0) {
            uint16_t *o = p.q_out + (int64_t)tok * p.ldq + (int64_t)h * D;
#pragma unroll
            for (int e = 0; e < E; ++e) o[lane + 64 * e] = (uint16_t)bf16_rne(v[e]);
        } else if (pbase >= 0) {
#pragma unroll
            for (int e = 0; e < E; ++e) p.k_pool[pbase + trow * D + lane + 64 * e] = (uint16_t)bf16_rne(v[e]);
        }
    }
}

inline bool aligned16(const void *q) { return ((uintptr_t)q & 15u) == 0; }

}  // namespace

extern "C" int emb_qkv_norm_rope_append(const void *qkv, int64_t ld, int32_t tokens, int32_t q_heads,
                                        int32_t kv_heads, int32_t head_dim, const uint16_t *q_gamma,
                                        const uint16_t *k_gamma, float eps, int32_t rope_kind, float rope_theta,
                                        int32_t first_position, const int32_t *position_ids, void *q_out,
                                        int64_t ldq, const int32_t *slots, const int32_t *block_table,
                                        int32_t capacity, void *k_pool, void *v_pool, void *v16_pool,
                                        hipStream_t stream) {
    EMB_CHECK_ARG(qkv && q_out && slots && k_pool && v_pool, "null pointer");
    EMB_CHECK_ARG(tokens > 0 && q_heads > 0 && kv_heads > 0 && capacity > 0, "non-positive size");
    EMB_CHECK_ARG(head_dim == 64 || head_dim == 128 || head_dim == 256, "head_dim must be 64, 128 or 256");
    EMB_CHECK_ARG(ld >= (int64_t)(q_heads + 2 * kv_heads) * head_dim, "ld smaller than a QKV row");
    EMB_CHECK_ARG(ldq >= (int64_t)q_heads * head_dim, "ldq smaller than a Q row");
    EMB_CHECK_ARG(rope_kind >= 0 && rope_kind <= 2, "rope_kind must be 0 (none), 1 (positions) or 2 (MRoPE)");
    EMB_CHECK_ARG(rope_kind != 2 || position_ids, "MRoPE needs position_ids");
    EMB_CHECK_ARG(rope_kind == 0 || (rope_theta > 0.0f && std::isfinite(rope_theta)), "rope_theta must be positive");
    EMB_CHECK_ARG(eps >= 0.0f && std::isfinite(eps), "eps must be finite and non-negative");
    EMB_CHECK_ARG(aligned16(k_pool) && aligned16(v_pool) && aligned16(v16_pool), "pools must be 16-byte aligned");
    NRParams p{(const uint16_t *)qkv, ld, tokens, q_heads, kv_heads, q_gamma, k_gamma, eps, rope_kind,
               rope_theta, first_position, position_ids, (uint16_t *)q_out, ldq, slots, block_table, capacity,
               (uint16_t *)k_pool, (uint16_t *)v_pool, (uint16_t *)v16_pool};
    const int64_t v_threads = (int64_t)tokens * kv_heads * (head_dim / 8);
    EMB_CHECK_ARG(tokens + (v_threads + 255) / 256 < INT32_MAX, "grid too large");
    const dim3 grid((unsigned)(tokens + (v_threads + 255) / 256));
    switch (head_dim) {
        case 64: hipLaunchKernelGGL(qk_norm_rope_append_kernel<64>, grid, dim3(256), 0, stream, p); break;
        case 128: hipLaunchKernelGGL(qk_norm_rope_append_kernel<128>, grid, dim3(256), 0, stream, p); break;
        default: hipLaunchKernelGGL(qk_norm_rope_append_kernel<256>, grid, dim3(256), 0, stream, p); break;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return emb::set_error(EMB_ERR_LAUNCH, "emb_qkv_norm_rope_append: %s", hipGetErrorString(e));
    return EMB_OK;
}
