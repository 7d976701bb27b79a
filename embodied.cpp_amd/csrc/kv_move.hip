// Paged KV append (scatter of new token rows into pages) and gather (compact
// copy of cache rows in key-list order), gfx950.
//
// Reference semantics: runtime_kv_update_f32_kernel and
// runtime_kv_gather_f32_kernel (kernels/lingbot/lingbot_flex_attn_cuda.cu:626-649,
// :875-898): row s goes to logical slot slots[s]; slots outside [0, capacity)
// are skipped; gather copies slot valid[i] to row i and leaves rows of
// out-of-range slots untouched.  Here the cache is bf16 and paged:
//   K page p, head h, row t, dim d : k_pool[((p*H + h)*16 + t)*D + d]
//   V page p, head h, dim d, row t : v_pool[((p*H + h)*D + d)*16 + t]
// V is stored transposed inside each page so that the attention kernel reads 16
// consecutive keys of one dimension with one 32-byte access.
//
// The kernels are byte movers bound by HBM.  Threads are ordered with the
// token index fastest, so the 16 tokens of one page write (append) or read
// (gather) one 32-byte V row together, while the K rows move as 16-byte vectors;
// large appends read and write whole head rows and turn V through LDS.
#include <hip/hip_runtime.h>

#include "emb_common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct MoveGeom {
    int32_t n;          // tokens
    int32_t heads, head_dim, chunks;  // chunks = head_dim / 8
    int32_t capacity;
    int64_t src_stride; // elements between source tokens (append)
};

__device__ __forceinline__ uint16_t bf16_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Loads 8 consecutive source elements as bf16 bits.
template <typename Src>
__device__ __forceinline__ void load8(const Src *p, uint16_t (&o)[8]);

template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t *p, uint16_t (&o)[8]) {
    const u32x4 w = *reinterpret_cast<const u32x4 *>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        o[2 * i] = (uint16_t)(w[i] & 0xffffu);
        o[2 * i + 1] = (uint16_t)(w[i] >> 16);
    }
}

// Loaded as float vectors: hipcc 7.2 folds __builtin_bit_cast(float, v[i]) of
// an ext-vector element to element 0 for every i, so no element is bit-cast.
template <>
__device__ __forceinline__ void load8<float>(const float *p, uint16_t (&o)[8]) {
    const f32x4 a = *reinterpret_cast<const f32x4 *>(p);
    const f32x4 b = *reinterpret_cast<const f32x4 *>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        o[i] = bf16_rne(a[i]);
        o[4 + i] = bf16_rne(b[i]);
    }
}

__device__ __forceinline__ u32x4 pack8(const uint16_t (&o)[8]) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = (uint32_t)o[2 * i] | ((uint32_t)o[2 * i + 1] << 16);
    return w;
}

// One thread per (token s, head h, 8-wide chunk c), s fastest, so the 16
// tokens of one page write one 32-byte V row together.  Index arithmetic is
// 32-bit (the host checks that n*H*D/8 fits); only addresses are 64-bit.
// With a V shadow, each element is also written as f16 at its position in the
// attention MFMA's key order (emb::v16_index).
template <typename Src>
__global__ __launch_bounds__(256) void kv_append_kernel(const Src *__restrict__ k, const Src *__restrict__ v,
                                                        const int32_t *__restrict__ slots,
                                                        const int32_t *__restrict__ block_table,
                                                        uint16_t *__restrict__ k_pool,
                                                        uint16_t *__restrict__ v_pool,
                                                        uint16_t *__restrict__ v16_pool, MoveGeom g) {
    const int32_t total = g.n * g.heads * g.chunks;
    for (int32_t idx = (int32_t)(blockIdx.x * blockDim.x + threadIdx.x); idx < total;
         idx += (int32_t)(gridDim.x * blockDim.x)) {
        const int32_t s = idx % g.n;
        const int32_t hc = idx / g.n;
        const int32_t c = hc % g.chunks;
        const int32_t h = hc / g.chunks;
        const int32_t slot = slots[s];
        if (slot < 0 || slot >= g.capacity) continue;
        const int32_t page = block_table ? block_table[slot >> 4] : (slot >> 4);
        if (page < 0) continue;
        const int32_t t = slot & 15;
        const int64_t src = (int64_t)s * g.src_stride + h * g.head_dim + c * 8;
        uint16_t kv[8], vv[8];
        load8<Src>(k + src, kv);
        load8<Src>(v + src, vv);
        const int64_t pbase = ((int64_t)page * g.heads + h) * 16 * g.head_dim;  // page element base
        *reinterpret_cast<u32x4 *>(k_pool + pbase + t * g.head_dim + c * 8) = pack8(kv);
#pragma unroll
        for (int e = 0; e < 8; ++e) v_pool[pbase + (c * 8 + e) * 16 + t] = vv[e];
        if (v16_pool) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                v16_pool[pbase + emb::v16_index(c * 8 + e, t)] =
                    __builtin_bit_cast(uint16_t, (_Float16)__builtin_bit_cast(float, (uint32_t)vv[e] << 16));
        }
    }
}

// Large appends: a workgroup per (16 consecutive tokens, head).  Each token's
// head row is read whole (chunk fastest: D*2 contiguous bytes, against 16 bytes
// per row with the token-fastest order) and its K row written whole; V goes
// through LDS and is written token-fastest, so the 16 tokens of a page (with
// consecutive slots) still write each 32-byte V row together.  Same skip rules
// and the same values as kv_append_kernel.
constexpr int ROWS_MAX_D = 256;

template <typename Src>
__global__ __launch_bounds__(256) void kv_append_rows_kernel(const Src *__restrict__ k, const Src *__restrict__ v,
                                                             const int32_t *__restrict__ slots,
                                                             const int32_t *__restrict__ block_table,
                                                             uint16_t *__restrict__ k_pool,
                                                             uint16_t *__restrict__ v_pool,
                                                             uint16_t *__restrict__ v16_pool, MoveGeom g) {
    // V of the 16 tokens, [token][d] with rows of D + 8 (16-byte aligned rows;
    // the 16 tokens of one d fall in 16 different banks)
    __shared__ __attribute__((aligned(16))) uint16_t vt[16 * (ROWS_MAX_D + 8)];
    const int32_t ld = g.head_dim + 8;
    const int32_t h = (int32_t)(blockIdx.x % g.heads);
    const int32_t s0 = (int32_t)(blockIdx.x / g.heads) * 16;
    for (int32_t u = threadIdx.x; u < 16 * g.chunks; u += 256) {
        const int32_t tok = u / g.chunks, c = u % g.chunks;
        const int32_t s = s0 + tok;
        if (s >= g.n) continue;
        const int64_t src = (int64_t)s * g.src_stride + h * g.head_dim + c * 8;
        uint16_t kv[8], vv[8];
        load8<Src>(k + src, kv);
        load8<Src>(v + src, vv);
        *reinterpret_cast<u32x4 *>(vt + tok * ld + c * 8) = pack8(vv);
        const int32_t slot = slots[s];
        if (slot < 0 || slot >= g.capacity) continue;
        const int32_t page = block_table ? block_table[slot >> 4] : (slot >> 4);
        if (page < 0) continue;
        const int64_t pbase = ((int64_t)page * g.heads + h) * 16 * g.head_dim;
        *reinterpret_cast<u32x4 *>(k_pool + pbase + (slot & 15) * g.head_dim + c * 8) = pack8(kv);
    }
    __syncthreads();
    for (int32_t w = threadIdx.x; w < 16 * g.head_dim; w += 256) {
        const int32_t tok = w % 16, d = w / 16;
        const int32_t s = s0 + tok;
        if (s >= g.n) continue;
        const int32_t slot = slots[s];
        if (slot < 0 || slot >= g.capacity) continue;
        const int32_t page = block_table ? block_table[slot >> 4] : (slot >> 4);
        if (page < 0) continue;
        const int32_t t = slot & 15;
        const int64_t pbase = ((int64_t)page * g.heads + h) * 16 * g.head_dim;
        const uint16_t b = vt[tok * ld + d];
        v_pool[pbase + d * 16 + t] = b;
        if (v16_pool)
            v16_pool[pbase + emb::v16_index(d, t)] =
                __builtin_bit_cast(uint16_t, (_Float16)__builtin_bit_cast(float, (uint32_t)b << 16));
    }
}

// One thread per (key i, head h, chunk c), i fastest.  Dst = uint16_t (bf16)
// or float (the f32 face).
template <typename Dst>
__global__ __launch_bounds__(256) void kv_gather_kernel(const uint16_t *__restrict__ k_pool,
                                                        const uint16_t *__restrict__ v_pool,
                                                        const int32_t *__restrict__ valid,
                                                        const int32_t *__restrict__ block_table,
                                                        Dst *__restrict__ k_out, Dst *__restrict__ v_out,
                                                        MoveGeom g) {
    const int64_t total = (int64_t)g.n * g.heads * g.chunks;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int32_t i = (int32_t)(idx % g.n);
        const int64_t hc = idx / g.n;
        const int32_t c = (int32_t)(hc % g.chunks);
        const int32_t h = (int32_t)(hc / g.chunks);
        const int32_t slot = valid[i];
        if (slot < 0 || slot >= g.capacity) continue;
        const int32_t page = block_table ? block_table[slot >> 4] : (slot >> 4);
        if (page < 0) continue;
        const int32_t t = slot & 15;
        const int64_t ksrc = (((int64_t)page * g.heads + h) * 16 + t) * g.head_dim + c * 8;
        const int64_t vsrc = (((int64_t)page * g.heads + h) * g.head_dim + c * 8) * 16 + t;
        uint16_t kv[8], vv[8];
        load8<uint16_t>(k_pool + ksrc, kv);
#pragma unroll
        for (int e = 0; e < 8; ++e) vv[e] = v_pool[vsrc + e * 16];
        const int64_t dst = ((int64_t)i * g.heads + h) * g.head_dim + c * 8;
        if constexpr (sizeof(Dst) == 2) {
            *reinterpret_cast<u32x4 *>(k_out + dst) = pack8(kv);
            *reinterpret_cast<u32x4 *>(v_out + dst) = pack8(vv);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                k_out[dst + e] = __builtin_bit_cast(float, (uint32_t)kv[e] << 16);
                v_out[dst + e] = __builtin_bit_cast(float, (uint32_t)vv[e] << 16);
            }
        }
    }
}

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

inline int grid_for(int64_t total) {
    int64_t g = (total + 255) / 256;
    if (g > 65536) g = 65536;
    return (int)(g < 1 ? 1 : g);
}

template <typename Src>
int launch_append(const Src *k, const Src *v, int64_t src_stride, int32_t n, const int32_t *slots,
                  const int32_t *block_table, int32_t capacity, void *k_pool, void *v_pool, void *v16_pool,
                  int32_t heads, int32_t head_dim, hipStream_t stream) {
    EMB_CHECK_ARG(k && v && slots && k_pool && v_pool, "null pointer");
    EMB_CHECK_ARG(n > 0 && heads > 0 && head_dim > 0 && capacity > 0, "non-positive size");
    EMB_CHECK_ARG(head_dim % 8 == 0, "head_dim must be a multiple of 8");
    EMB_CHECK_ARG(src_stride >= (int64_t)heads * head_dim, "src_stride smaller than a token row");
    EMB_CHECK_ARG((src_stride * (int64_t)sizeof(Src)) % 16 == 0, "source rows must be 16-byte aligned");
    EMB_CHECK_ARG(aligned16(k) && aligned16(v) && aligned16(k_pool) && aligned16(v_pool) && aligned16(v16_pool),
                  "buffers must be 16-byte aligned");
    MoveGeom g{n, heads, head_dim, head_dim / 8, capacity, src_stride};
    const int64_t total = (int64_t)n * heads * g.chunks;
    EMB_CHECK_ARG(total < INT32_MAX, "append too large for one launch");
    const int64_t groups = ((int64_t)n + 15) / 16 * heads;
    if (groups >= 768 && head_dim <= ROWS_MAX_D && groups < INT32_MAX) {
        // enough (16 tokens, head) workgroups to fill the chip (3 a CU).
        // Measured: 1560 x 24 heads x 128 (2352 groups) 20.6 -> 13.2 us and
        // 14688 x 1 x 256 (918) 18.2 -> 12.7 us on this path, while
        // 1040 x 8 x 256 (520 groups) is slower on it (10.9 against 8.4 us) and
        // the pi0.5 step's 918 x 1 x 256 (58 groups) is latency-bound
        hipLaunchKernelGGL(kv_append_rows_kernel<Src>, dim3((unsigned)groups), dim3(256), 0, stream, k, v, slots,
                           block_table, (uint16_t *)k_pool, (uint16_t *)v_pool, (uint16_t *)v16_pool, g);
    } else {
        hipLaunchKernelGGL(kv_append_kernel<Src>, dim3(grid_for(total)), dim3(256), 0, stream, k, v, slots,
                           block_table, (uint16_t *)k_pool, (uint16_t *)v_pool, (uint16_t *)v16_pool, g);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return emb::set_error(EMB_ERR_LAUNCH, "kv_append launch: %s", hipGetErrorString(e));
    return EMB_OK;
}

// Large gathers: the append's row layout in reverse -- a workgroup per (16
// consecutive output rows, head) reads V token-fastest (the 16 keys of a page
// with consecutive slots read one 32-byte V row together) into LDS, and writes
// each output row's K and V whole.  Same skip rules and values as
// kv_gather_kernel.
template <typename Dst>
__global__ __launch_bounds__(256) void kv_gather_rows_kernel(const uint16_t *__restrict__ k_pool,
                                                             const uint16_t *__restrict__ v_pool,
                                                             const int32_t *__restrict__ valid,
                                                             const int32_t *__restrict__ block_table,
                                                             Dst *__restrict__ k_out, Dst *__restrict__ v_out,
                                                             MoveGeom g) {
    __shared__ __attribute__((aligned(16))) uint16_t vt[16 * (ROWS_MAX_D + 8)];
    const int32_t ld = g.head_dim + 8;
    const int32_t h = (int32_t)(blockIdx.x % g.heads);
    const int32_t i0 = (int32_t)(blockIdx.x / g.heads) * 16;
    for (int32_t w = threadIdx.x; w < 16 * g.head_dim; w += 256) {
        const int32_t tok = w % 16, d = w / 16, i = i0 + tok;
        if (i >= g.n) continue;
        const int32_t slot = valid[i];
        if (slot < 0 || slot >= g.capacity) continue;
        const int32_t page = block_table ? block_table[slot >> 4] : (slot >> 4);
        if (page < 0) continue;
        vt[tok * ld + d] = v_pool[(((int64_t)page * g.heads + h) * g.head_dim + d) * 16 + (slot & 15)];
    }
    __syncthreads();
    for (int32_t u = threadIdx.x; u < 16 * g.chunks; u += 256) {
        const int32_t tok = u / g.chunks, c = u % g.chunks, i = i0 + tok;
        if (i >= g.n) continue;
        const int32_t slot = valid[i];
        if (slot < 0 || slot >= g.capacity) continue;
        const int32_t page = block_table ? block_table[slot >> 4] : (slot >> 4);
        if (page < 0) continue;
        uint16_t kv[8], vv[8];
        load8<uint16_t>(k_pool + (((int64_t)page * g.heads + h) * 16 + (slot & 15)) * g.head_dim + c * 8, kv);
        load8<uint16_t>(vt + tok * ld + c * 8, vv);
        const int64_t dst = ((int64_t)i * g.heads + h) * g.head_dim + c * 8;
        if constexpr (sizeof(Dst) == 2) {
            *reinterpret_cast<u32x4 *>(k_out + dst) = pack8(kv);
            *reinterpret_cast<u32x4 *>(v_out + dst) = pack8(vv);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                k_out[dst + e] = __builtin_bit_cast(float, (uint32_t)kv[e] << 16);
                v_out[dst + e] = __builtin_bit_cast(float, (uint32_t)vv[e] << 16);
            }
        }
    }
}

template <typename Dst>
int launch_gather(const void *k_pool, const void *v_pool, const int32_t *valid, int32_t n,
                  const int32_t *block_table, int32_t capacity, Dst *k_out, Dst *v_out, int32_t heads,
                  int32_t head_dim, hipStream_t stream) {
    EMB_CHECK_ARG(k_pool && v_pool && valid && k_out && v_out, "null pointer");
    EMB_CHECK_ARG(n > 0 && heads > 0 && head_dim > 0 && capacity > 0, "non-positive size");
    EMB_CHECK_ARG(head_dim % 8 == 0, "head_dim must be a multiple of 8");
    EMB_CHECK_ARG(aligned16(k_out) && aligned16(v_out) && aligned16(k_pool) && aligned16(v_pool),
                  "buffers must be 16-byte aligned");
    MoveGeom g{n, heads, head_dim, head_dim / 8, capacity, 0};
    const int64_t total = (int64_t)n * heads * g.chunks;
    const int64_t groups = ((int64_t)n + 15) / 16 * heads;
    if (groups >= 768 && head_dim <= ROWS_MAX_D && groups < INT32_MAX) {  // the append's rule
        hipLaunchKernelGGL(kv_gather_rows_kernel<Dst>, dim3((unsigned)groups), dim3(256), 0, stream,
                           (const uint16_t *)k_pool, (const uint16_t *)v_pool, valid, block_table, k_out, v_out, g);
    } else {
        hipLaunchKernelGGL(kv_gather_kernel<Dst>, dim3(grid_for(total)), dim3(256), 0, stream,
                           (const uint16_t *)k_pool, (const uint16_t *)v_pool, valid, block_table, k_out, v_out, g);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return emb::set_error(EMB_ERR_LAUNCH, "kv_gather launch: %s", hipGetErrorString(e));
    return EMB_OK;
}

}  // namespace

extern "C" {

int emb_kv_append(const void *k_new, const void *v_new, int64_t src_stride, int32_t n, const int32_t *slots,
                  const int32_t *block_table, int32_t capacity, void *k_pool, void *v_pool, void *v16_pool,
                  int32_t n_kv_heads, int32_t head_dim, hipStream_t stream) {
    return launch_append<uint16_t>((const uint16_t *)k_new, (const uint16_t *)v_new, src_stride, n, slots,
                                   block_table, capacity, k_pool, v_pool, v16_pool, n_kv_heads, head_dim, stream);
}

int emb_kv_gather(const void *k_pool, const void *v_pool, const int32_t *valid, int32_t n,
                  const int32_t *block_table, int32_t capacity, void *k_out, void *v_out, int32_t n_kv_heads,
                  int32_t head_dim, hipStream_t stream) {
    return launch_gather<uint16_t>(k_pool, v_pool, valid, n, block_table, capacity, (uint16_t *)k_out,
                                   (uint16_t *)v_out, n_kv_heads, head_dim, stream);
}

// Reference-named f32 face (kernels/lingbot/lingbot_flex_attn_cuda.cu:900-919,
// :987-1008): the caller's f32-sized cache buffers hold a bf16 identity-paged
// pool, which needs ceil16(capacity)*H*D*2 <= capacity*H*D*4 bytes.
int lingbot_runtime_kv_update_f32(const float *k, const float *v, float *cache_k, float *cache_v,
                                  const int *slots, int seq, int n_heads, int head_dim, int capacity,
                                  hipStream_t stream) {
    EMB_CHECK_ARG(capacity >= 8, "capacity must be >= 8 for the bf16 paged layout");
    return launch_append<float>(k, v, (int64_t)n_heads * head_dim, seq, slots, nullptr, capacity, cache_k, cache_v,
                                nullptr, n_heads, head_dim, stream);
}

int lingbot_runtime_kv_gather_f32(const float *cache_k, const float *cache_v, const int *valid_slots,
                                  float *compact_k, float *compact_v, int seq_k, int n_heads, int head_dim,
                                  int capacity, hipStream_t stream) {
    EMB_CHECK_ARG(capacity >= 8, "capacity must be >= 8 for the bf16 paged layout");
    return launch_gather<float>(cache_k, cache_v, valid_slots, seq_k, nullptr, capacity, compact_k, compact_v,
                                n_heads, head_dim, stream);
}

}  // extern "C"
