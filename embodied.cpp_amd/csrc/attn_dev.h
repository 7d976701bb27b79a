// Device helpers and constants shared by the two attention kernels of
// libemb_kv.so (paged_attn.hip: row tiles of 128 query rows with optional
// split-K; paged_attn_ks.hip: key-split workgroups of 32 query rows), and the
// parameter block of the key-split kernel.  HIP sources only.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace emb_attn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x2 __attribute__((ext_vector_type(2)));

// The online softmax rescales the accumulators only when a row's max grows by
// more than this many powers of two.
constexpr float RESCALE_TH = 8.0f;
// A row whose largest |O| lies below this (with a non-empty key set) is
// recomputed exactly from the bf16 pool: V reaches the fast P.V product as
// f16, exact only for |v| in [2^-14, 65504].
constexpr float EXACT_TINY = 0x1p-12f;
constexpr float LOG2E = 1.4426950408889634f;

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __builtin_bit_cast(float, b << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// The four values rounded to bf16 precision (nearest even), kept as f32.
__device__ __forceinline__ f32x4 round_bf16x4(const f32x4 &v) {
    return f32x4{__builtin_bit_cast(float, f32_to_bf16_bits(v[0]) << 16),
                 __builtin_bit_cast(float, f32_to_bf16_bits(v[1]) << 16),
                 __builtin_bit_cast(float, f32_to_bf16_bits(v[2]) << 16),
                 __builtin_bit_cast(float, f32_to_bf16_bits(v[3]) << 16)};
}

// Four floats as four f16 (round to nearest even), packed in two dwords.
__device__ __forceinline__ u32x2 f16x4_bits(const f32x4 &v) {
    u32x2 w;
    w[0] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[0]) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[1]) << 16);
    w[1] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2]) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[3]) << 16);
    return w;
}

// Lane l and lane l ^ 32 of x, as a pair, by one VALU lane swap: the first
// element is x of lane l & 31, the second x of lane l | 32 (so their max or
// sum is the same in both halves of the wave).
__device__ __forceinline__ void half_pair(float x, float &a, float &b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                    false, false);
    a = __builtin_bit_cast(float, (uint32_t)r[0]);
    b = __builtin_bit_cast(float, (uint32_t)r[1]);
}

constexpr uint32_t RSRC_W3 = 0x00020000u;  // buffer resource word 3 (raw, 32-bit elements)

// Raw buffer descriptor over [base, base + bytes) (stride 0, 32-bit records),
// its words forced into SGPRs (the arguments are wave-uniform).
__device__ __forceinline__ u32x4 buf_desc(const void *base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a),
                 (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu),
                 (uint32_t)__builtin_amdgcn_readfirstlane(bytes), RSRC_W3};
}

// vmcnt(N) with the other counters left alone.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
}

// One global -> LDS copy of 16 bytes a lane: lane i's 16 bytes at byte offset
// voff of the buffer land at LDS byte m0 + 16 i (bytes past the buffer's end
// land as zeros).  Written as inline asm on purpose: the compiler cannot tell
// the pipeline stages apart, so for its own form of this load it waits for
// every outstanding copy (vmcnt(0)) before the next LDS read of any stage --
// the prefetch included.  The kernel counts these loads itself (wait_vmcnt).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_copy16(const u32x4 &desc, uint32_t m0, uint32_t voff) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"  // SALU write of M0 -> LDS-DMA read of M0: one wait state
        "buffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0),
        "v"(voff), "s"(desc)
        : "memory", "m0");
}
#pragma clang diagnostic pop

// Block-table entries per sequence the key-split kernel holds in LDS (32768
// keys); longer tables take the row-tile kernel.
constexpr int KS_MAX_PAGES = 2048;

// Parameters of the key-split kernel (paged_attn_ks.hip).  Pool layout,
// bounds and zero-row rules are those of emb_paged_attention (emb_kv.h).
struct KsParams {
    const void *q;
    float *out;
    int64_t q_stride, out_stride;
    int32_t round_out;
    const int32_t *cu_q;
    const int32_t *n_keys;
    int32_t nq_single, nk_single;
    const uint16_t *k_pool;
    const uint16_t *v_pool;    // bf16, read only by the exact recompute
    const uint16_t *v16_pool;  // f16 shadow, the fast path's V
    const int32_t *bt;
    int32_t bt_stride;
    int32_t capacity;
    int32_t hkv, G;
    int32_t row_blocks;  // 32-row blocks per (sequence, kv head)
    int32_t total_wg;
    float c_log2;  // scale * log2(e)
    float th_raw;  // RESCALE_TH / c_log2
};

// Launches the key-split kernel (head_dim 128 or 256); returns the launch status.
hipError_t ks_launch(const KsParams &p, int head_dim, bool q_f32, hipStream_t stream);

}  // namespace emb_attn
