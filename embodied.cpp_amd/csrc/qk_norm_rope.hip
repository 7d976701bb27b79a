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

#include <algorithm>
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

// ---- LingBot: full-row q/k RMSNorm + Wan RoPE + append (f32 QKV) ----
//
// Reference: build_attention_shape (models/lingbot_va.cpp:1219-1250): q =
// rms_norm(lin(q)) * q_norm_weight over the whole hidden row (all heads at
// once), k the same, v = lin(v); then apply_wan_rope_shape (:1190-1206) on q
// and k: per head, pairs (2i, 2i+1) rotated by the per-token tables
// rope_cos / rope_sin [seq][head_dim/2] (y0 = x0 c - x1 s, y1 = x1 c + x0 s).
// Everything is f32 (ggml's rms_norm: scale = 1 / sqrt(sum(x^2) / n + eps)),
// each node rounded on its own (no fused multiply-add); the outputs are
// rounded to bf16 once, for the bf16 Q buffer and cache.
constexpr int RN_MAXC = 8;  // float4 chunks a thread holds: hidden <= 8192

struct RNParams {
    const float *qkv;
    int64_t ld;
    int32_t tokens, heads, hd, hidden;
    const float *bias, *q_w, *k_w;
    float eps;
    const float *cs, *sn;  // [tokens][hd/2]
    uint16_t *q_out;
    int64_t ldq;
    const int32_t *slots, *bt;
    int32_t capacity;
    uint16_t *k_pool, *v_pool, *v16_pool;
};

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u32x2 pack_bf16x4(const f32x4_t &v) {
    return u32x2{bf16_rne(v[0]) | (bf16_rne(v[1]) << 16), bf16_rne(v[2]) | (bf16_rne(v[3]) << 16)};
}

// Workgroup sum of two values (four waves).
__device__ __forceinline__ void wg_sum2(float &a, float &b, float *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        a += __shfl_xor(a, off, 64);
        b += __shfl_xor(b, off, 64);
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        red[wave * 2] = a;
        red[wave * 2 + 1] = b;
    }
    __syncthreads();
    a = (red[0] + red[2]) + (red[4] + red[6]);
    b = (red[1] + red[3]) + (red[5] + red[7]);
}

// Cache page of a token's slot: the element offset of page row 0 of head 0, or
// -1 when the slot is outside [0, capacity) or on an unmapped page (skipped,
// as in emb_kv_append).
__device__ __forceinline__ int64_t slot_page_base(const int32_t *slots, const int32_t *bt, int32_t capacity,
                                                  int32_t tok, int32_t heads, int32_t hd, int32_t &trow) {
    const int32_t slot = slots[tok];
    trow = slot & 15;
    if (slot < 0 || slot >= capacity) return -1;
    const int32_t page = bt ? bt[slot >> 4] : (slot >> 4);
    return page < 0 ? -1 : (int64_t)page * heads * 16 * hd;
}

// f32 V heads into the transposed V page (and its f16 shadow): a thread per
// (token, head, 8-dim chunk) with tokens fastest, so the 16 tokens of a page
// store one 32-byte row together.  src points at the token-0 V columns of
// head 0; bias (NULL: none) at head 0's V bias.
__device__ __forceinline__ void append_v_f32(int64_t idx, const float *src, int64_t ld, const float *bias,
                                             int32_t tokens, int32_t heads, int32_t hd, const int32_t *slots,
                                             const int32_t *bt, int32_t capacity, uint16_t *v_pool,
                                             uint16_t *v16_pool) {
    const int CH = hd / 8;
    const int32_t s = (int32_t)(idx % tokens);
    const int64_t hc = idx / tokens;
    const int c = (int)(hc % CH), h = (int)(hc / CH);
    if (h >= heads) return;
    int32_t t;
    const int64_t page_base = slot_page_base(slots, bt, capacity, s, heads, hd, t);
    if (page_base < 0) return;
    const int col = h * hd + c * 8;
    const float *x = src + (int64_t)s * ld + col;
    f32x4_t v0 = *reinterpret_cast<const f32x4_t *>(x), v1 = *reinterpret_cast<const f32x4_t *>(x + 4);
    if (bias) {
        v0 = v0 + *reinterpret_cast<const f32x4_t *>(bias + col);
        v1 = v1 + *reinterpret_cast<const f32x4_t *>(bias + col + 4);
    }
    const int64_t pbase = page_base + (int64_t)h * 16 * hd;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t b = bf16_rne(e < 4 ? v0[e] : v1[e - 4]);
        const int d = c * 8 + e;
        v_pool[pbase + d * 16 + t] = (uint16_t)b;
        if (v16_pool) v16_pool[pbase + emb::v16_index(d, t)] = __builtin_bit_cast(uint16_t, (_Float16)bf16f(b));
    }
}

__global__ __launch_bounds__(256) void row_norm_rope_append_kernel(RNParams p) {
#pragma clang fp contract(off)
    __shared__ float red[8];
    if ((int32_t)blockIdx.x >= p.tokens) {
        append_v_f32((int64_t)(blockIdx.x - p.tokens) * 256 + threadIdx.x, p.qkv + 2 * p.hidden, p.ld,
                     p.bias ? p.bias + 2 * p.hidden : nullptr, p.tokens, p.heads, p.hd, p.slots, p.bt, p.capacity,
                     p.v_pool, p.v16_pool);
        return;
    }
    const int32_t tok = blockIdx.x;
    const int nch = p.hidden / 4;
    const float *row = p.qkv + (int64_t)tok * p.ld;
    f32x4_t q[RN_MAXC], k[RN_MAXC];
    float sq = 0.0f, sk = 0.0f;
#pragma unroll
    for (int j = 0; j < RN_MAXC; ++j) {
        const int c = threadIdx.x + 256 * j;
        q[j] = k[j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        if (c < nch) {
            q[j] = *reinterpret_cast<const f32x4_t *>(row + 4 * c);
            k[j] = *reinterpret_cast<const f32x4_t *>(row + p.hidden + 4 * c);
            if (p.bias) {
                q[j] = q[j] + *reinterpret_cast<const f32x4_t *>(p.bias + 4 * c);
                k[j] = k[j] + *reinterpret_cast<const f32x4_t *>(p.bias + p.hidden + 4 * c);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sq += q[j][e] * q[j][e];
                sk += k[j][e] * k[j][e];
            }
        }
    }
    float inv_q = 1.0f, inv_k = 1.0f;
    if (p.q_w || p.k_w) {
        wg_sum2(sq, sk, red);
        inv_q = 1.0f / sqrtf(sq / (float)p.hidden + p.eps);
        inv_k = 1.0f / sqrtf(sk / (float)p.hidden + p.eps);
    }
    int32_t trow;
    const int64_t page_base = slot_page_base(p.slots, p.bt, p.capacity, tok, p.heads, p.hd, trow);
    const int half = p.hd / 2;
#pragma unroll
    for (int j = 0; j < RN_MAXC; ++j) {
        const int c = threadIdx.x + 256 * j;
        if (c >= nch) continue;
        const int e0 = 4 * c;
        if (p.q_w) q[j] = (q[j] * inv_q) * *reinterpret_cast<const f32x4_t *>(p.q_w + e0);
        if (p.k_w) k[j] = (k[j] * inv_k) * *reinterpret_cast<const f32x4_t *>(p.k_w + e0);
        const int h = e0 / p.hd, d = e0 % p.hd;
        if (p.cs) {
            const int pi = d / 2;  // pairs pi, pi + 1 of this chunk
            const float *cr = p.cs + (int64_t)tok * half + pi, *sr = p.sn + (int64_t)tok * half + pi;
            const float c0 = cr[0], c1 = cr[1], s0 = sr[0], s1 = sr[1];
            auto rot = [&](f32x4_t &x) {
#pragma clang fp contract(off)
                const f32x4_t o = x;
                x[0] = o[0] * c0 - o[1] * s0;
                x[1] = o[1] * c0 + o[0] * s0;
                x[2] = o[2] * c1 - o[3] * s1;
                x[3] = o[3] * c1 + o[2] * s1;
            };
            rot(q[j]);
            rot(k[j]);
        }
        *reinterpret_cast<u32x2 *>(p.q_out + (int64_t)tok * p.ldq + e0) = pack_bf16x4(q[j]);
        if (page_base >= 0)
            *reinterpret_cast<u32x2 *>(p.k_pool + page_base + (int64_t)h * 16 * p.hd + trow * p.hd + d) =
                pack_bf16x4(k[j]);
    }
}

// ---- pi0.5: NEOX RoPE (ggml_rope_ext) on f32 Q/K + append ----
//
// Reference: build_adarms_gemma_layer / build_gemma_layer (models/pi05.cpp
// :386-408, :300-325) run q, k, v = mul_mat(W, x_norm) (f32), then
// ggml_rope_ext(t, positions, NULL, n_dims = head_dim, GGML_ROPE_TYPE_NEOX,
// 0, freq_base, freq_scale 1, ext_factor 0, attn_factor 1, 32, 1) on q and k
// (:394-402), and concatenate k_rope / v onto the cached prefix K/V (:405-408).
// ggml (llama.cpp b9016; not vendored) defines that rope for f32 on its CUDA
// backend as: theta_scale = powf(freq_base, -2 / n_dims) on the host; for pair
// i < n_dims / 2 of a row at position pos, theta = pos * powf(theta_scale, i)
// (freq_scale 1 and ext_factor 0 leave it as is, attn_factor 1 scales nothing),
// and the pair (x[i], x[i + n_dims / 2]) becomes
// (x0 cos - x1 sin, x0 sin + x1 cos), cos and sin in f32.  Here each product
// is rounded on its own (no fused multiply-add); cos, sin and pow are the
// device library's.  Q is stored f32 (ggml's result type) or bf16, K and V go
// into the cache in bf16 (round to nearest even).
//
// Blocks [0, qk_blocks) each take tb consecutive tokens and walk their
// (token, Q-or-K head, 4 pairs) items, pairs fastest, so a head's threads read
// the two halves of its row as contiguous 16-byte vectors, up to NX_NI items a
// thread per round.  A thread issues the loads of its items first; meanwhile
// the block puts cos and sin of every (token, pair) it holds into LDS -- one
// powf, cosf and sinf per pair and token, shared by all Q and K heads of the
// token -- and after one barrier the items are rotated and stored.  tb is
// chosen so that tb * head_dim/2 <= 256 (one pair a thread; head_dim > 512:
// one token) and a round covers the block where the head count allows.
// Blocks past those append V (append_v_f32).
constexpr int NX_MAX_PAIRS = 512;  // LDS cos/sin entries: head_dim <= 1024
constexpr int NX_NI = 4;           // items a thread holds per round

struct NXParams {
    const float *q, *k, *v;
    int64_t ldqi, ldk, ldv;
    int32_t tokens, q_heads, kv_heads, hd;
    const int32_t *pos;
    int32_t first_pos;
    float theta_scale;
    void *q_out;
    int32_t q_f32;
    int64_t ldq;
    const int32_t *slots, *bt;
    int32_t capacity;
    uint16_t *k_pool, *v_pool, *v16_pool;
    int32_t tb;  // tokens per block
    int32_t qk_blocks;
};

__global__ __launch_bounds__(256) void neox_rope_append_kernel(NXParams p) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float cs[NX_MAX_PAIRS], sn[NX_MAX_PAIRS];
    if ((int32_t)blockIdx.x >= p.qk_blocks) {
        append_v_f32((int64_t)(blockIdx.x - p.qk_blocks) * 256 + threadIdx.x, p.v, p.ldv, nullptr, p.tokens,
                     p.kv_heads, p.hd, p.slots, p.bt, p.capacity, p.v_pool, p.v16_pool);
        return;
    }
    const int half = p.hd / 2;
    const int CH = p.hd / 8;  // items per head, 4 pairs each
    const int units = p.q_heads + p.kv_heads;
    const int per_tok = units * CH;
    const int32_t tok0 = (int32_t)blockIdx.x * p.tb;
    const int n_tok = min(p.tb, p.tokens - tok0);
    const int n_items = n_tok * per_tok;  // block-uniform
    for (int base = 0; base < n_items; base += 256 * NX_NI) {
        f32x4_t lo[NX_NI], hi[NX_NI];
#pragma unroll
        for (int k = 0; k < NX_NI; ++k) {
            const int w = base + k * 256 + (int)threadIdx.x;
            if (w >= n_items) continue;
            const int tl = w / per_tok, r = w % per_tok;
            const int u = r / CH, j = r % CH;
            const int32_t tok = tok0 + tl;
            const float *row = u < p.q_heads ? p.q + (int64_t)tok * p.ldqi + (int64_t)u * p.hd
                                             : p.k + (int64_t)tok * p.ldk + (int64_t)(u - p.q_heads) * p.hd;
            lo[k] = *reinterpret_cast<const f32x4_t *>(row + 4 * j);
            hi[k] = *reinterpret_cast<const f32x4_t *>(row + half + 4 * j);
        }
        if (base == 0) {
            for (int w = threadIdx.x; w < n_tok * half; w += 256) {
                const int32_t tok = tok0 + w / half;
                const float pos = (float)(p.pos ? p.pos[tok] : p.first_pos + tok);
                const float theta = pos * powf(p.theta_scale, (float)(w % half));
                cs[w] = cosf(theta);
                sn[w] = sinf(theta);
            }
            __syncthreads();
        }
#pragma unroll
        for (int k = 0; k < NX_NI; ++k) {
            const int w = base + k * 256 + (int)threadIdx.x;
            if (w >= n_items) continue;
            const int tl = w / per_tok, r = w % per_tok;
            const int u = r / CH, j = r % CH;
            const int32_t tok = tok0 + tl;
            const f32x4_t c = *reinterpret_cast<const f32x4_t *>(cs + tl * half + 4 * j);
            const f32x4_t s = *reinterpret_cast<const f32x4_t *>(sn + tl * half + 4 * j);
            f32x4_t a = lo[k], b = hi[k];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float x0 = lo[k][e], x1 = hi[k][e];
                a[e] = x0 * c[e] - x1 * s[e];
                b[e] = x0 * s[e] + x1 * c[e];
            }
            if (u < p.q_heads) {
                if (p.q_f32) {
                    float *o = reinterpret_cast<float *>(p.q_out) + (int64_t)tok * p.ldq + (int64_t)u * p.hd;
                    *reinterpret_cast<f32x4_t *>(o + 4 * j) = a;
                    *reinterpret_cast<f32x4_t *>(o + half + 4 * j) = b;
                } else {
                    uint16_t *o = reinterpret_cast<uint16_t *>(p.q_out) + (int64_t)tok * p.ldq + (int64_t)u * p.hd;
                    *reinterpret_cast<u32x2 *>(o + 4 * j) = pack_bf16x4(a);
                    *reinterpret_cast<u32x2 *>(o + half + 4 * j) = pack_bf16x4(b);
                }
                continue;
            }
            int32_t trow;
            const int64_t page_base = slot_page_base(p.slots, p.bt, p.capacity, tok, p.kv_heads, p.hd, trow);
            if (page_base < 0) continue;
            uint16_t *kr = p.k_pool + page_base + (int64_t)(u - p.q_heads) * 16 * p.hd + (int64_t)trow * p.hd;
            *reinterpret_cast<u32x2 *>(kr + 4 * j) = pack_bf16x4(a);
            *reinterpret_cast<u32x2 *>(kr + half + 4 * j) = pack_bf16x4(b);
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

extern "C" int emb_qkv_rownorm_rope_append(const float *qkv, int64_t ld, int32_t tokens, int32_t heads,
                                           int32_t head_dim, const float *qkv_bias, const float *q_weight,
                                           const float *k_weight, float eps, const float *rope_cos,
                                           const float *rope_sin, void *q_out, int64_t ldq, const int32_t *slots,
                                           const int32_t *block_table, int32_t capacity, void *k_pool,
                                           void *v_pool, void *v16_pool, hipStream_t stream) {
    EMB_CHECK_ARG(qkv && q_out && slots && k_pool && v_pool, "null pointer");
    EMB_CHECK_ARG(tokens > 0 && heads > 0 && capacity > 0, "non-positive size");
    EMB_CHECK_ARG(head_dim > 0 && head_dim % 8 == 0, "head_dim must be a positive multiple of 8");
    const int64_t hidden = (int64_t)heads * head_dim;
    EMB_CHECK_ARG(hidden <= 4 * 256 * RN_MAXC, "heads * head_dim must be at most 8192");
    EMB_CHECK_ARG(ld >= 3 * hidden && ld % 4 == 0, "ld must cover a QKV row and be a multiple of 4");
    EMB_CHECK_ARG(ldq >= hidden && ldq % 4 == 0, "ldq must cover a Q row and be a multiple of 4");
    EMB_CHECK_ARG((rope_cos == nullptr) == (rope_sin == nullptr), "rope_cos and rope_sin go together");
    EMB_CHECK_ARG(eps >= 0.0f && std::isfinite(eps), "eps must be finite and non-negative");
    EMB_CHECK_ARG(aligned16(qkv) && aligned16(qkv_bias) && aligned16(q_weight) && aligned16(k_weight),
                  "qkv, bias and norm weights must be 16-byte aligned");
    EMB_CHECK_ARG(((uintptr_t)q_out & 7u) == 0 && ((uintptr_t)k_pool & 7u) == 0, "q_out and k_pool must be 8-byte aligned");
    RNParams p{qkv, ld, tokens, heads, head_dim, (int32_t)hidden, qkv_bias, q_weight, k_weight, eps, rope_cos,
               rope_sin, (uint16_t *)q_out, ldq, slots, block_table, capacity, (uint16_t *)k_pool,
               (uint16_t *)v_pool, (uint16_t *)v16_pool};
    const int64_t v_threads = (int64_t)tokens * heads * (head_dim / 8);
    EMB_CHECK_ARG(tokens + (v_threads + 255) / 256 < INT32_MAX, "grid too large");
    hipLaunchKernelGGL(row_norm_rope_append_kernel, dim3((unsigned)(tokens + (v_threads + 255) / 256)), dim3(256), 0,
                       stream, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return emb::set_error(EMB_ERR_LAUNCH, "emb_qkv_rownorm_rope_append: %s", hipGetErrorString(e));
    return EMB_OK;
}

extern "C" int emb_qkv_neox_rope_append(const float *q, int64_t ld_q, const float *k, int64_t ld_k, const float *v,
                                        int64_t ld_v, int32_t tokens, int32_t q_heads, int32_t kv_heads,
                                        int32_t head_dim, const int32_t *positions, int32_t first_position,
                                        float freq_base, void *q_out, int32_t q_out_f32, int64_t ldq,
                                        const int32_t *slots, const int32_t *block_table, int32_t capacity,
                                        void *k_pool, void *v_pool, void *v16_pool, hipStream_t stream) {
    EMB_CHECK_ARG(q && k && v && q_out && slots && k_pool && v_pool, "null pointer");
    EMB_CHECK_ARG(tokens > 0 && q_heads > 0 && kv_heads > 0 && capacity > 0, "non-positive size");
    EMB_CHECK_ARG(head_dim > 0 && head_dim % 8 == 0 && head_dim <= 1024, "head_dim must be a multiple of 8, at most 1024");
    EMB_CHECK_ARG(ld_q >= (int64_t)q_heads * head_dim && ld_k >= (int64_t)kv_heads * head_dim &&
                      ld_v >= (int64_t)kv_heads * head_dim,
                  "ld_q / ld_k / ld_v smaller than a row of heads");
    EMB_CHECK_ARG(ld_q % 4 == 0 && ld_k % 4 == 0 && ld_v % 4 == 0, "ld_q, ld_k and ld_v must be multiples of 4");
    EMB_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v), "q, k and v must be 16-byte aligned");
    EMB_CHECK_ARG(ldq >= (int64_t)q_heads * head_dim && ldq % 4 == 0, "ldq must cover a Q row and be a multiple of 4");
    EMB_CHECK_ARG(q_out_f32 ? aligned16(q_out) : ((uintptr_t)q_out & 7u) == 0,
                  "q_out must be 16-byte (f32) or 8-byte (bf16) aligned");
    EMB_CHECK_ARG(((uintptr_t)k_pool & 7u) == 0, "k_pool must be 8-byte aligned");
    EMB_CHECK_ARG(freq_base > 0.0f && std::isfinite(freq_base), "freq_base must be positive and finite");
    const float theta_scale = powf(freq_base, -2.0f / (float)head_dim);
    const int64_t per_tok = (int64_t)(q_heads + kv_heads) * (head_dim / 8);
    EMB_CHECK_ARG(per_tok <= (1 << 24), "too many heads");
    const int64_t tb = std::max<int64_t>(1, std::min<int64_t>(256 / (head_dim / 2), 256 * NX_NI / per_tok));
    const int64_t v_threads = (int64_t)tokens * kv_heads * (head_dim / 8);
    const int64_t qk_blocks = (tokens + tb - 1) / tb, v_blocks = (v_threads + 255) / 256;
    EMB_CHECK_ARG(qk_blocks + v_blocks < INT32_MAX, "grid too large");
    NXParams p{q, k, v, ld_q, ld_k, ld_v, tokens, q_heads, kv_heads, head_dim, positions, first_position,
               theta_scale, q_out, q_out_f32, ldq, slots, block_table, capacity, (uint16_t *)k_pool,
               (uint16_t *)v_pool, (uint16_t *)v16_pool, (int32_t)tb, (int32_t)qk_blocks};
    hipLaunchKernelGGL(neox_rope_append_kernel, dim3((unsigned)(qk_blocks + v_blocks)), dim3(256), 0, stream, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return emb::set_error(EMB_ERR_LAUNCH, "emb_qkv_neox_rope_append: %s", hipGetErrorString(e));
    return EMB_OK;
}
