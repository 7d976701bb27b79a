// W8A16 linear for gfx950 (MI355X): bf16 activations x int8 weights stored in
// the Marlin kU8B128 channelwise layout, fp32 accumulate, per-output-channel
// bf16 scale applied to the fp32 accumulator, bf16 result.
//
// Reference semantics: cosmos3_w8a16_linear_* (kernels/cosmos3/
// cosmos3_w8_marlin_cuda.cu:302-501, :651-765) with the layout contract of
// marlin_w8_dst_byte / unpack_marlin_uint8b128 / marlin_scale_index (:50-88,
// kernels/cosmos3/README.md:55-64) and the epilogue order of vLLM Marlin
// (scale on the fp32 accumulator, third_party/vllm_marlin/marlin_template.h:
// 166-174, :1970-1996):
//   y[m][n] = bf16( (sum_k bf16(x[m][k]) * (u8[k][n] - 128)) * s[n] ).
// The Marlin code itself is not used; the kernel reads the packed words by the
// layout formula.
//
// Layout recap.  qweight is int32 [K/16][4N]; band r = k/16 holds 16 k x N
// bytes.  In a band, 64-column group g = n/64 owns words g*256 .. g*256+255,
// and within the group the word index is
//   (n%8)*32 + (n/8)%8 + j*8,   j = (k%8)/2,
// with byte lane (k%2)*2 + (k/8)%2.  So for one column n the 16 k of a band sit
// in the 4 words j = 0..3: word j holds k = 2j, 8+2j, 2j+1, 9+2j (bytes 0..3).
//
// MFMA mapping (32x32x16 bf16, C = X . W), natural k order in both operands:
// lane half h of the A operand (row) and of the B operand (column n) holds k =
// 8h .. 8h+7 of the 16-k step.  The staging thread holding words j = 2h', 2h'+1
// of a column has k = 4h'..4h'+3 (bytes 0 and 2) and 8+4h'..11+4h' (bytes 1
// and 3): it writes them dequantized to element 4h' of half 0 and of half 1.
// x needs no reordering.
//
// Tiling.  With bf16 x, K % 64 == 0 and 256-row tiles, the 256 x 256 kernel
// further down (eight waves, x copied straight into LDS) runs.  Otherwise a
// workgroup of 4 waves (2 x 2) computes a 256 x 128 tile of y; a wave owns
// 128 x 64 (4 x 2 MFMA blocks, 128 accumulator registers).  Where
// 256-row tiles would need no fewer rounds of resident workgroups, the tiles
// are 128 x 128 instead (2 x 2 blocks a wave); each output element sums the
// same k-steps in the same order either way.  K moves
// in tiles of 64.  The next k-tile's x and W words are loaded into registers
// while the current one is multiplied; they are then converted (W: u8 ->
// bf16(u8 - 128), once per workgroup) and written to the single LDS stage.
// Two workgroups share a CU.
//
// Epilogue.  Plain mode writes y (bf16, or f32).  QKV mode splits the columns:
// [0, n_q) go to a bf16 Q buffer, the next n_kv to the K pages and the last
// n_kv to the V pages of a paged KV pool (emb_kv.h layout), at logical slot
// slots[m] of the token -- the append of runtime_kv_update (kernels/lingbot/
// lingbot_flex_attn_cuda.cu:626-649) fused into the projection, and the f16 V
// shadow when one is given.  Gated-residual mode is the projection after
// attention with the block's residual update in the epilogue (the LingBot
// post graph, models/lingbot_va.cpp:11693-11695, with lin() at :1178-1180):
//   out[m][n] = x_in[m][n] + ((acc * s[n]) + bias[n]) * (gate[m][n] + gate_bias[n]),
// each operation rounded to f32 as the graph's separate add/mul nodes do (no
// fused multiply-add), optionally rounded to bf16 (the graph's bf16 boundary).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <type_traits>

#include "emb_common.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int BN = 128, BK = 64;  // tile rows BM (256 or 128) is a template argument
constexpr int AS = BK + 8;  // bf16 elements per staged x row (bank spread)
// A stage: BM x AS bf16; B stage:
constexpr int B_ELEMS = (BK / 16) * BN * 2 * 8;  // [band][n][h][8] bf16

enum { Y_BF16 = 0, Y_F32_ROUNDED = 1, Y_F32_RAW = 2, Y_QKV = 3, Y_GATED = 4, Y_GATED_B16 = 5, Y_GATED_F32 = 6 };
// Y_GATED_B16: bf16 weights (ggml BF16 [N][K] rows), the fp32 accumulator
// rounded to bf16 before the bias; Y_GATED_F32: f32 weights and f32 x, the
// fp32 accumulator as is.  Both use the gated-residual epilogue without scales.

struct GParams {
    const void *x;
    int64_t ldx;
    const uint32_t *qw;   // [K/16][4N] words
    const uint16_t *scales;
    int32_t M, K, N;
    int32_t m_tiles, n_tiles;
    void *y;
    int64_t ldy;
    // QKV mode
    int32_t n_q, n_kv, head_dim, hkv, capacity;
    const int32_t *slots;
    const int32_t *bt;
    uint16_t *k_pool, *v_pool, *v16_pool;
    // gated-residual mode (y is the f32 output)
    const float *bias, *gate, *gate_bias, *res;
    int64_t ldg, ldr;
    int32_t round_out;
    // f32 x: when set, x is first rounded into this bf16 [M][K] buffer and the
    // GEMM reads that (the same bf16 values the in-kernel rounding gives)
    uint16_t *x_ws;
    // dense weights (Y_GATED_B16: bf16, Y_GATED_F32: f32), row n at wd + n * ldw
    const void *wd;
    int64_t ldw;
};

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}


// bf16 bits of (byte - 128) for byte i of w, in the upper half of a dword:
// the integer-to-float conversion by exponent bias (a "magic number"): the
// byte permute builds the f32 bit pattern 0x4B0000bb = 2^23 + b, subtracting
// 2^23 + 128 in f32 is exact, and the integer result (|b - 128| <= 128, at most
// 8 significant bits) is exactly the upper half of its f32 pattern.
__device__ __forceinline__ uint32_t u8_bf16_hi(uint32_t w, int i) {
    constexpr uint32_t MAGIC = 0x4B4B4B4Bu;
    const uint32_t sel = (uint32_t)(4 + i) | (0x0cu << 8) | (0x0cu << 16) | (0x03u << 24);
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(float, __builtin_amdgcn_perm(w, MAGIC, sel)) - 8388736.0f);
}
// two bf16 (upper halves of a and b) -> one dword, a low
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

template <bool XF32, int BM, bool WB16 = false>
struct Stage {
    // x: 4 units of (row, 16-k group); W: two 16-byte runs of one band
    // (WB16: four 16-byte runs of bf16 weight rows).
    u32x4 xa[BM / 64], xb[BM / 64];
    u32x4 w0, w1;
    u32x4 wr[WB16 ? 4 : 1];

    __device__ __forceinline__ void load(const GParams &p, int32_t m0, int32_t n0, int32_t k0) {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < BM / 64; ++i) {
            const int u = tid + i * 256;
            const int row = u >> 2, g = u & 3;
            const int32_t m = m0 + row, k = k0 + g * 16;
            xa[i] = u32x4{0u, 0u, 0u, 0u};
            xb[i] = u32x4{0u, 0u, 0u, 0u};
            if (m < p.M && k < p.K) {
                if (XF32) {
                    const float *src = reinterpret_cast<const float *>(p.x) + (int64_t)m * p.ldx + k;
                    f32x4 f[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) f[q] = *reinterpret_cast<const f32x4 *>(src + 4 * q);
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        xa[i][2 * q] = f32_to_bf16_bits(f[q][0]) | (f32_to_bf16_bits(f[q][1]) << 16);
                        xa[i][2 * q + 1] = f32_to_bf16_bits(f[q][2]) | (f32_to_bf16_bits(f[q][3]) << 16);
                        xb[i][2 * q] = f32_to_bf16_bits(f[q + 2][0]) | (f32_to_bf16_bits(f[q + 2][1]) << 16);
                        xb[i][2 * q + 1] = f32_to_bf16_bits(f[q + 2][2]) | (f32_to_bf16_bits(f[q + 2][3]) << 16);
                    }
                } else {
                    const uint16_t *src = reinterpret_cast<const uint16_t *>(p.x) + (int64_t)m * p.ldx + k;
                    xa[i] = *reinterpret_cast<const u32x4 *>(src);
                    xb[i] = *reinterpret_cast<const u32x4 *>(src + 8);
                }
            }
        }
        if constexpr (WB16) {
            // unit u = t + 256 i: column n = u / 8 of the tile, 8 k (band u%8/2,
            // half u%2) -- eight lanes read one row's 128 contiguous bytes
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int u = tid + i * 256;
                const int n = u >> 3, sub = u & 7;
                const int32_t k = k0 + sub * 8;
                wr[i] = u32x4{0u, 0u, 0u, 0u};
                if (n0 + n < p.N && k < p.K)
                    wr[i] = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const uint16_t *>(p.wd) +
                                                             (int64_t)(n0 + n) * p.ldw + k);
            }
            return;
        }
        // W: thread t takes band t/64 of the tile, 64-column group (t/32)%2,
        // and the two 16-byte runs at word c0 and c0 + 8 of that group, where
        // c0 = (n%8)*32 + (q%2)*4 + (q/2)*16 for n%8 = (t%32)/4, q = t%4:
        // words j = 2h and 2h+1 (h = q/2) of the 4 columns n/8%8 = (q%2)*4 + e.
        const int band = tid >> 6, grp = (tid >> 5) & 1, idx = tid & 31;
        const int n8 = idx >> 2, q = idx & 3;
        const int c0 = n8 * 32 + (q & 1) * 4 + (q >> 1) * 16;
        const int32_t kb = (k0 >> 4) + band;
        const int32_t col64 = (n0 >> 6) + grp;
        w0 = u32x4{0u, 0u, 0u, 0u};
        w1 = u32x4{0u, 0u, 0u, 0u};
        if (kb < (p.K >> 4) && col64 * 64 < p.N) {
            const uint32_t *src = p.qw + (int64_t)kb * (4 * (int64_t)p.N) + col64 * 256 + c0;
            w0 = *reinterpret_cast<const u32x4 *>(src);
            w1 = *reinterpret_cast<const u32x4 *>(src + 8);
        }
    }

    __device__ __forceinline__ void store(uint16_t *as, uint16_t *bs) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < BM / 64; ++i) {
            const int u = tid + i * 256;
            const int row = u >> 2, g = u & 3;
            uint16_t *dst = as + row * AS + g * 16;  // natural k order
            *reinterpret_cast<u32x4 *>(dst) = xa[i];
            *reinterpret_cast<u32x4 *>(dst + 8) = xb[i];
        }
        if constexpr (WB16) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int u = tid + i * 256;
                const int n = u >> 3, sub = u & 7;
                const int band = sub >> 1, h = sub & 1;
                const int sw = (n >> 3) & 1;
                *reinterpret_cast<u32x4 *>(bs + (band * BN + n) * 16 + (h ^ sw) * 8) = wr[i];
            }
            return;
        }
        const int band = tid >> 6, grp = (tid >> 5) & 1, idx = tid & 31;
        const int n8 = idx >> 2, q = idx & 3;
        const int h = q >> 1;
        // natural k order: words 2h and 2h+1 of column n hold k 4h..4h+3
        // (bytes 0, 2 of each) for half 0 and k 8+4h..11+4h (bytes 1, 3) for
        // half 1, both at element 4h of the half
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int n = grp * 64 + ((q & 1) * 4 + e) * 8 + n8;  // column inside the tile
            const uint32_t a0 = u8_bf16_hi(w0[e], 0), a1 = u8_bf16_hi(w0[e], 1), a2 = u8_bf16_hi(w0[e], 2),
                           a3 = u8_bf16_hi(w0[e], 3);
            const uint32_t b0 = u8_bf16_hi(w1[e], 0), b1 = u8_bf16_hi(w1[e], 1), b2 = u8_bf16_hi(w1[e], 2),
                           b3 = u8_bf16_hi(w1[e], 3);
            const int sw = (n >> 3) & 1;  // bank swizzle of the two halves
            uint16_t *col = bs + (band * BN + n) * 16;
            *reinterpret_cast<u32x2 *>(col + (0 ^ sw) * 8 + 4 * h) = u32x2{pack_hi(a0, a2), pack_hi(b0, b2)};
            *reinterpret_cast<u32x2 *>(col + (1 ^ sw) * 8 + 4 * h) = u32x2{pack_hi(a1, a3), pack_hi(b1, b3)};
        }
    }
};

// Epilogue of a wave's 128 (or 64) x 64 block: lane holds column n = n0 + wn*64 + j*32
// + lrow and rows m0 + wm*(BM/2) + i*32 + (r/4)*8 + lhi*4 + r%4.  lds: at least BM*8 bytes
// of LDS no wave reads any more (the QKV row table); NT threads in the workgroup.
template <int MODE, int BM, int NT>
__device__ __forceinline__ void gemm_epilogue(const GParams &p, f32x16 (&acc)[BM / 64][2], int32_t m0,
                                              int32_t n0, int wm, int wn, int lane, uint16_t *lds) {
    constexpr int MI = BM / 64;
    const int lrow = lane & 31, lhi = lane >> 5;
    if constexpr (MODE == Y_QKV) {
        // Row table in the (now free) A tile: for each of the tile's BM rows the
        // element offset of its page (page * hkv * 16 * head_dim) with the
        // in-page token in the low 4 bits, or -1 when the row is past M or its
        // slot is out of range or unmapped.  A page offset is a multiple of 16
        // elements, so its low 4 bits are free.
        int64_t *rowtab = reinterpret_cast<int64_t *>(lds);
        __syncthreads();  // every wave is past its last fragment read of as
        for (int r = threadIdx.x; r < BM; r += NT) {
            const int32_t m = m0 + r;
            int64_t e = -1;
            if (m < p.M) {
                const int32_t slot = p.slots[m];
                if (slot >= 0 && slot < p.capacity) {
                    const int32_t page = p.bt ? p.bt[slot >> 4] : (slot >> 4);
                    if (page >= 0) e = (int64_t)page * p.hkv * 16 * p.head_dim + (slot & 15);
                }
            }
            rowtab[r] = e;
        }
        __syncthreads();
        const int64_t hstride = 16 * (int64_t)p.head_dim;
        // one column block at a time with a compile-time j: the unroller gives
        // up on a two-trip loop around this body, and a runtime j would index
        // the accumulators through scratch memory
        auto store_cols = [&](auto jc) __attribute__((always_inline)) {
            constexpr int j = decltype(jc)::value;
            const int32_t n = n0 + wn * 64 + j * 32 + lrow;
            if (n >= p.N) return;
            const float s = __builtin_bit_cast(float, (uint32_t)p.scales[(n >> 5) * 32 + ((n & 31) >> 3) * 2 +
                                                                        ((n & 7) >> 1) * 8 + (n & 1)]
                                                             << 16);
            if (n < p.n_q) {
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int32_t m = m0 + wm * (BM / 2) + i * 32 + (r >> 2) * 8 + lhi * 4 + (r & 3);
                        if (m < p.M)
                            reinterpret_cast<uint16_t *>(p.y)[(int64_t)m * p.ldy + n] =
                                (uint16_t)f32_to_bf16_bits(acc[i][j][r] * s);
                    }
                return;
            }
            const int32_t c = n - p.n_q;
            const bool is_v = c >= p.n_kv;
            const int32_t cc = is_v ? c - p.n_kv : c;
            const int32_t d = cc % p.head_dim;
            const int64_t hoff = (cc / p.head_dim) * hstride;
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int rl = wm * (BM / 2) + i * 32 + g * 8 + lhi * 4;  // four consecutive rows
                    int64_t e[4];
                    uint32_t b[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        e[k] = rowtab[rl + k];
                        b[k] = f32_to_bf16_bits(acc[i][j][g * 4 + k] * s);
                    }
                    if (!is_v) {
#pragma unroll
                        for (int k = 0; k < 4; ++k)
                            if (e[k] >= 0) p.k_pool[(e[k] & ~15LL) + hoff + (e[k] & 15) * p.head_dim + d] = b[k];
                        continue;
                    }
                    // V: four rows on consecutive slots of one page starting at a
                    // multiple of 4 are contiguous in the [d][16] page rows (and in
                    // the shadow's order, which keeps bits 0-1 of the token)
                    const bool run = e[0] >= 0 && (e[0] & 3) == 0 && e[1] == e[0] + 1 && e[2] == e[0] + 2 &&
                                     e[3] == e[0] + 3;
                    if (run) {
                        const int64_t pb = (e[0] & ~15LL) + hoff;
                        const int t0 = (int)(e[0] & 15);
                        *reinterpret_cast<u32x2 *>(p.v_pool + pb + d * 16 + t0) =
                            u32x2{b[0] | (b[1] << 16), b[2] | (b[3] << 16)};
                        if (p.v16_pool) {
                            uint32_t h16[4];
#pragma unroll
                            for (int k = 0; k < 4; ++k)
                                h16[k] = __builtin_bit_cast(uint16_t, (_Float16)__builtin_bit_cast(float, b[k] << 16));
                            *reinterpret_cast<u32x2 *>(p.v16_pool + pb + emb::v16_index(d, t0)) =
                                u32x2{h16[0] | (h16[1] << 16), h16[2] | (h16[3] << 16)};
                        }
                        continue;
                    }
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        if (e[k] < 0) continue;
                        const int64_t pb = (e[k] & ~15LL) + hoff;
                        const int t = (int)(e[k] & 15);
                        p.v_pool[pb + d * 16 + t] = (uint16_t)b[k];
                        if (p.v16_pool)
                            p.v16_pool[pb + emb::v16_index(d, t)] =
                                __builtin_bit_cast(uint16_t, (_Float16)__builtin_bit_cast(float, b[k] << 16));
                    }
                }
        };
        store_cols(std::integral_constant<int, 0>{});
        store_cols(std::integral_constant<int, 1>{});
        return;
    }
    if constexpr (MODE == Y_GATED || MODE == Y_GATED_B16 || MODE == Y_GATED_F32) {
        // Per (row block i, column j): all 16 residual and gate loads first
        // (rows past M clamped to M - 1, so every load is in bounds and none
        // waits on a branch), then the arithmetic and the stores.  The dense
        // modes have no scale and may have no residual (out = the projection,
        // gated or not).
        auto body = [&](auto gated) __attribute__((always_inline)) {
#pragma clang fp contract(off)
            constexpr bool G = decltype(gated)::value;
            const bool R = p.res != nullptr;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int32_t n = n0 + wn * 64 + j * 32 + lrow;
                if (n >= p.N) continue;
                float s = 1.0f;
                if constexpr (MODE == Y_GATED)
                    s = __builtin_bit_cast(float, (uint32_t)p.scales[(n >> 5) * 32 + ((n & 31) >> 3) * 2 +
                                                                    ((n & 7) >> 1) * 8 + (n & 1)]
                                                      << 16);
                const float bn = p.bias ? p.bias[n] : 0.0f;
                const float gb = G && p.gate_bias ? p.gate_bias[n] : 0.0f;
#pragma unroll
                for (int i = 0; i < MI; ++i) {
                    float rv[16], gv[16];
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int32_t m = min(m0 + wm * (BM / 2) + i * 32 + (r >> 2) * 8 + lhi * 4 + (r & 3), p.M - 1);
                        rv[r] = R ? p.res[(int64_t)m * p.ldr + n] : 0.0f;
                        if constexpr (G) gv[r] = p.gate[(int64_t)m * p.ldg + n];
                    }
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int32_t m = m0 + wm * (BM / 2) + i * 32 + (r >> 2) * 8 + lhi * 4 + (r & 3);
                        float a;
                        if constexpr (MODE == Y_GATED)
                            a = acc[i][j][r] * s;
                        else if constexpr (MODE == Y_GATED_B16)
                            a = __builtin_bit_cast(float, f32_to_bf16_bits(acc[i][j][r]) << 16);
                        else
                            a = acc[i][j][r];
                        if (p.bias) a = a + bn;
                        if constexpr (G) a = a * (gv[r] + gb);
                        float v = R ? rv[r] + a : a;
                        if (p.round_out) v = __builtin_bit_cast(float, f32_to_bf16_bits(v) << 16);
                        if (m < p.M) reinterpret_cast<float *>(p.y)[(int64_t)m * p.ldy + n] = v;
                    }
                }
            }
        };
        if (p.gate)
            body(std::integral_constant<bool, true>{});
        else
            body(std::integral_constant<bool, false>{});
        return;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int32_t n = n0 + wn * 64 + j * 32 + lrow;
        if (n >= p.N) continue;
        const float s = __builtin_bit_cast(float, (uint32_t)p.scales[(n >> 5) * 32 + ((n & 31) >> 3) * 2 +
                                                                    ((n & 7) >> 1) * 8 + (n & 1)]
                                                         << 16);
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int32_t m = m0 + wm * (BM / 2) + i * 32 + (r >> 2) * 8 + lhi * 4 + (r & 3);
                if (m >= p.M) continue;
                const float v = acc[i][j][r] * s;
                if (MODE == Y_F32_RAW) {
                    reinterpret_cast<float *>(p.y)[(int64_t)m * p.ldy + n] = v;
                } else {
                    const uint32_t bits = f32_to_bf16_bits(v);
                    if (MODE == Y_BF16)
                        reinterpret_cast<uint16_t *>(p.y)[(int64_t)m * p.ldy + n] = (uint16_t)bits;
                    else
                        reinterpret_cast<float *>(p.y)[(int64_t)m * p.ldy + n] = __builtin_bit_cast(float, bits << 16);
                }
            }
    }
}

template <bool XF32, int MODE, int BM>
__global__ __launch_bounds__(256, 2) void w8a16_gemm_kernel(GParams p) {
    __shared__ __attribute__((aligned(16))) uint16_t as[BM * AS];
    __shared__ __attribute__((aligned(16))) uint16_t bs[B_ELEMS];

    // XCD-aware order: consecutive logical tiles share an n-tile (the same
    // W columns) and land on one XCD's L2.
    const int nwg = (int)gridDim.x;
    const int lin = (int)(blockIdx.x % 8) * (nwg / 8) + (int)(blockIdx.x / 8);
    if (lin >= p.m_tiles * p.n_tiles) return;
    const int mt = lin % p.m_tiles, nt = lin / p.m_tiles;
    const int32_t m0 = mt * BM, n0 = nt * BN;

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int lrow = lane & 31, lhi = lane >> 5;

    constexpr int MI = BM / 64;  // 32-row MFMA blocks a wave holds
    f32x16 acc[MI][2];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

    Stage<XF32, BM, MODE == Y_GATED_B16> st;
    const int32_t n_kt = (p.K + BK - 1) / BK;
    st.load(p, m0, n0, 0);
    st.store(as, bs);
    __syncthreads();

    for (int32_t kt = 0; kt < n_kt; ++kt) {
        const bool more = kt + 1 < n_kt;
        if (more) st.load(p, m0, n0, (kt + 1) * BK);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            bf16x8 a[4], bfr[2];
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const int row = wm * (BM / 2) + i * 32 + lrow;
                a[i] = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4 *>(as + row * AS + ks * 16 + lhi * 8));
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = wn * 64 + j * 32 + lrow;
                const int slot = lhi ^ ((n >> 3) & 1);
                bfr[j] = __builtin_bit_cast(bf16x8,
                                            *reinterpret_cast<const u32x4 *>(bs + ((ks * BN + n) * 2 + slot) * 8));
            }
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            __syncthreads();
            st.store(as, bs);
            __syncthreads();
        }
    }

    gemm_epilogue<MODE, BM, 256>(p, acc, m0, n0, wm, wn, lane, as);
}

// ---- f32 weights and f32 x: fp32 MFMA (32x32x2) ----
//
// The ggml F32 x F32 product (cublasSgemm in the CUDA backend): products and
// sums in fp32, nothing rounded to a narrower type.  A workgroup of 4 waves
// (2 x 2) computes a 128 x 128 tile, 64 x 64 a wave (2 x 2 blocks), K in tiles
// of 32 staged through registers into one LDS stage.  One MFMA takes a k pair:
// lane (row, h) supplies A[row][k] with k = 2s + h at step s.  Both operands
// read 16 bytes a lane at k = 8q + 4h .. 8q + 4h + 3 and step 4q + t uses the
// t-th of them, so the k sum runs in one fixed permuted order for A and W.
constexpr int FBM = 128, FBK = 32, FLD = FBK + 4;  // rows padded by 16 bytes

template <int MODE>
__global__ __launch_bounds__(256, 2) void f32_gemm_kernel(GParams p) {
    __shared__ __attribute__((aligned(16))) float xs[FBM * FLD];
    __shared__ __attribute__((aligned(16))) float ws[FBM * FLD];
    const int nwg = (int)gridDim.x;
    const int lin = (int)(blockIdx.x % 8) * (nwg / 8) + (int)(blockIdx.x / 8);
    if (lin >= p.m_tiles * p.n_tiles) return;
    const int mt = lin % p.m_tiles, nt = lin / p.m_tiles;
    const int32_t m0 = mt * FBM, n0 = nt * FBM;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int lrow = lane & 31, lhi = lane >> 5;
    const float *xg = reinterpret_cast<const float *>(p.x);
    const float *wg = reinterpret_cast<const float *>(p.wd);

    // unit u = t + 256 i: row u / 8 of the tile, k = 4 (u % 8) of the k-tile
    f32x4 rx[4], rw[4];
    auto load = [&](int32_t k0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int u = tid + i * 256;
            const int row = u >> 3;
            const int32_t k = k0 + (u & 7) * 4;
            rx[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            rw[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (m0 + row < p.M && k < p.K) rx[i] = *reinterpret_cast<const f32x4 *>(xg + (int64_t)(m0 + row) * p.ldx + k);
            if (n0 + row < p.N && k < p.K) rw[i] = *reinterpret_cast<const f32x4 *>(wg + (int64_t)(n0 + row) * p.ldw + k);
        }
    };
    auto store = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int u = tid + i * 256;
            const int off = (u >> 3) * FLD + (u & 7) * 4;
            *reinterpret_cast<f32x4 *>(xs + off) = rx[i];
            *reinterpret_cast<f32x4 *>(ws + off) = rw[i];
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
    const int32_t n_kt = (p.K + FBK - 1) / FBK;
    load(0);
    store();
    __syncthreads();
    for (int32_t kt = 0; kt < n_kt; ++kt) {
        const bool more = kt + 1 < n_kt;
        if (more) load((kt + 1) * FBK);
#pragma unroll
        for (int q = 0; q < FBK / 8; ++q) {
            f32x4 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = *reinterpret_cast<const f32x4 *>(xs + (wm * 64 + i * 32 + lrow) * FLD + 8 * q + 4 * lhi);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = *reinterpret_cast<const f32x4 *>(ws + (wn * 64 + j * 32 + lrow) * FLD + 8 * q + 4 * lhi);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][t], b[j][t], acc[i][j], 0, 0, 0);
        }
        if (more) {
            __syncthreads();
            store();
            __syncthreads();
        }
    }
    gemm_epilogue<MODE, FBM, 256>(p, acc, m0, n0, wm, wn, lane, reinterpret_cast<uint16_t *>(xs));
}

// ---- 256 x 256 tiles with x copied straight into LDS (bf16 x, K % 64 == 0) ----
//
// Eight waves (2 x 4), each the same 128 x 64 block as above, share a 256-row
// x tile and a 256-column W tile, so each byte staged feeds twice the MFMAs of
// the 256 x 128 tile.  Two LDS stages of 64 KB: while tile kt is multiplied,
// tile kt + 1 is staged into the other one -- x by DMA (buffer_load ... lds,
// no registers), W from registers loaded one tile earlier and dequantized on
// the way.  W goes to LDS in natural k order ([band][n][half][8]: half h of
// column n holds k = 8h .. 8h + 7), so x keeps its own order and needs no
// permutation: lane (row, h) reads k-chunk 2 ks + h of its row, lane (n, h)
// the same k of column n.  x rows are 128 bytes; the 16-byte chunk c of row r
// sits at granule c ^ ((r >> 1) & 7) of the row, so the 16 rows a quarter-wave
// reads hit 16 different bank groups (W: half h at slot h ^ ((n >> 3) & 1)).
constexpr uint32_t RSRC_W3 = 0x00020000u;       // raw buffer, 32-bit elements

__device__ __forceinline__ u32x4 buf_desc(const void *base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a),
                 (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu),
                 (uint32_t)__builtin_amdgcn_readfirstlane(bytes), RSRC_W3};
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
}

// Lane i's 16 bytes at byte offset voff of the buffer land at LDS byte m0 + 16 i
// (bytes past the buffer's end land as zeros).  The kernel counts these loads
// itself (wait_vmcnt).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_copy16(const u32x4 &d, uint32_t m0, uint32_t voff) {
    // every operand but voff is wave-uniform: pin it to SGPRs
    const u32x4 desc = {(uint32_t)__builtin_amdgcn_readfirstlane(d[0]), (uint32_t)__builtin_amdgcn_readfirstlane(d[1]),
                        (uint32_t)__builtin_amdgcn_readfirstlane(d[2]), (uint32_t)__builtin_amdgcn_readfirstlane(d[3])};
    m0 = (uint32_t)__builtin_amdgcn_readfirstlane(m0);
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"  // SALU write of M0 -> LDS-DMA read of M0: one wait state
        "buffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0),
        "v"(voff), "s"(desc)
        : "memory", "m0");
}
#pragma clang diagnostic pop


// One thread's W words of a k-tile (NG 64-column groups in the tile): thread t
// takes band t / (32 NG) of the tile, 64-column group (t / 32) % NG, and in it
// the words j = 2h, 2h + 1 (h = q / 2)
// of the 4 columns with n % 8 = (t % 32) / 4 and (n / 8) % 8 = (q % 2) * 4 + e,
// q = t % 4 (the layout recap at the top).  Loaded by inline asm, so the
// kernel counts them with its copies (the compiler would wait for them with
// vmcnt(0), i.e. for every copy issued after them too).
struct WRegs {
    u32x4 w0, w1;
};

template <int NG>
__device__ __forceinline__ void load_w(WRegs &r, const GParams &p, int32_t n0, int32_t k0, int tid) {
    const int band = tid / (32 * NG), grp = (tid >> 5) % NG, idx = tid & 31;
    const int n8 = idx >> 2, q = idx & 3;
    const int c0 = n8 * 32 + (q & 1) * 4 + (q >> 1) * 16;
    // bands past K (the loads issued beyond the last k-tile) read the last band
    const int32_t kb = min((k0 >> 4) + band, (p.K >> 4) - 1);
    // a group past N reads the last one instead (its columns are never stored)
    const int32_t col64 = min((n0 >> 6) + grp, p.N / 64 - 1);
    const uint32_t *src = p.qw + (int64_t)kb * (4 * (int64_t)p.N) + col64 * 256 + c0;
    asm volatile(
        "global_load_dwordx4 %0, %2, off\n\t"
        "global_load_dwordx4 %1, %2, off offset:32"
        : "=&v"(r.w0), "=&v"(r.w1)
        : "v"(src)
        : "memory");
}

// Column n holds, in word 2h, k = 4h, 8+4h, 4h+1, 9+4h and in word 2h+1
// k = 4h+2, 10+4h, 4h+3, 11+4h (bytes 0..3): k 4h..4h+3 go to half 0 at
// element 4h, k 8+4h..11+4h to half 1 at element 4h.  Part e: the e-th of the
// thread's four columns.
template <int NG>
__device__ __forceinline__ void store_w_part(const WRegs &r, uint16_t *ws, int tid, int e) {
    const int band = tid / (32 * NG), grp = (tid >> 5) % NG, idx = tid & 31;
    const int n8 = idx >> 2, q = idx & 3;
    const int h = q >> 1;
    const int n = grp * 64 + ((q & 1) * 4 + e) * 8 + n8;  // column inside the tile
    const uint32_t a0 = u8_bf16_hi(r.w0[e], 0), a1 = u8_bf16_hi(r.w0[e], 1), a2 = u8_bf16_hi(r.w0[e], 2),
                   a3 = u8_bf16_hi(r.w0[e], 3);
    const uint32_t b0 = u8_bf16_hi(r.w1[e], 0), b1 = u8_bf16_hi(r.w1[e], 1), b2 = u8_bf16_hi(r.w1[e], 2),
                   b3 = u8_bf16_hi(r.w1[e], 3);
    const u32x2 lo = {pack_hi(a0, a2), pack_hi(b0, b2)};  // k 4h, 4h+1, 4h+2, 4h+3
    const u32x2 hi = {pack_hi(a1, a3), pack_hi(b1, b3)};  // k 8+4h .. 11+4h
    const int sw = (n >> 3) & 1;
    uint16_t *col = ws + (band * NG * 64 + n) * 16;
    *reinterpret_cast<u32x2 *>(col + (0 ^ sw) * 8 + 4 * h) = lo;
    *reinterpret_cast<u32x2 *>(col + (1 ^ sw) * 8 + 4 * h) = hi;
}

// vmcnt(N) that also re-defines the W registers, so no use of them is
// scheduled before the wait.
template <int N>
__device__ __forceinline__ void wait_w(WRegs &r) {
    static_assert(N >= 0 && N < 16, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%2)" : "+v"(r.w0), "+v"(r.w1) : "n"(N));
}

// Pipeline, per k-tile kt: three x stages and two W stages.  At the top of
// iteration kt the copies of x(kt+2) and the loads of W(kt+2) go out (into
// the x stage and the register set nothing reads any more); the MFMAs of
// tile kt run with the dequantized stores of W(kt+1) -- loaded a whole
// iteration earlier -- between their k-steps; one counted wait for x(kt+1)
// and W(kt+1), one barrier.
//
// The W loads are inline asm the compiler cannot see in flight: any copy of
// their registers placed between a load and its wait would read stale data,
// and the compiler places such copies where control flow merges.  So nothing
// between a load and its wait branches: every iteration issues its copies and
// loads (past the last k-tile they reread the last band and fill a stage no
// one reads), every wait has the same count, K is a multiple of two k-tiles
// (the loop body is two iterations with no test between them), and the last
// loads are waited for, by a wait that names their registers, before the
// epilogue reuses LDS and registers.
constexpr int NXS = 3;

// TM x TM tiles: TM = 256 with eight waves (2 x 4, 128 x 64 a wave, 160 KB of
// LDS, one workgroup a CU); TM = 128 with four (2 x 2, 64 x 64 a wave, 80 KB,
// two a CU).  A thread issues four x copies and two W loads a k-tile in both.
template <int TM>
struct Pipe {
    static constexpr int NT = TM == 256 ? 512 : 256;  // threads
    static constexpr int WN = NT / 128;               // waves along n (2 along m)
    static constexpr int NG = TM / 64;                // 64-column groups
    static constexpr int TX = TM * BK;                // bf16 elements of one x image
    static constexpr int TW = (BK / 16) * TM * 16;    // bf16 elements of one W image
    static constexpr int WG_PER_CU = TM == 256 ? 1 : 2;
};

template <int MODE, int TM>
__global__ __launch_bounds__(Pipe<TM>::NT, Pipe<TM>::WG_PER_CU) void w8a16_gemm_pipe_kernel(GParams p) {
    using PP = Pipe<TM>;
    constexpr int NT = PP::NT, NG = PP::NG, TX = PP::TX, TW = PP::TW, TBN = TM;
    __shared__ __attribute__((aligned(16))) uint16_t smem[NXS * TX + 2 * TW];
    constexpr int BM = TM, MI = BM / 64;
    static_assert(BM * 8 == 4 * NT && (BK / 16) * TM * 16 == 32 * NT, "four x copies and two W loads a thread");
    const int nwg = (int)gridDim.x;
    const int lin = (int)(blockIdx.x % 8) * (nwg / 8) + (int)(blockIdx.x / 8);
    if (lin >= p.m_tiles * p.n_tiles) return;
    const int mt = lin % p.m_tiles, nt = lin / p.m_tiles;
    const int32_t m0 = mt * BM, n0 = nt * TBN;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wm = wave / PP::WN, wn = wave % PP::WN;
    const int lrow = lane & 31, lhi = lane >> 5;

    // x rows [m0, M) as one buffer: rows past M read as zeros
    const uint16_t *xb = reinterpret_cast<const uint16_t *>(p.x) + (int64_t)m0 * p.ldx;
    const uint32_t xbytes = (uint32_t)min<int64_t>((int64_t)(p.M - m0) * p.ldx * 2, 0xffffffffLL);
    const u32x4 xdesc = buf_desc(xb, xbytes);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t *)smem;
    // copy i of this wave: granules (i*NT + wave*64 + lane) of the x image
    uint32_t xoff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int g = i * NT + wave * 64 + lane;
        const int row = g >> 3, slot = g & 7;
        const int c = slot ^ ((row >> 1) & 7);
        xoff[i] = (uint32_t)((row * p.ldx + c * 8) * 2);
    }
    auto copy_x = [&](int stage, int32_t k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            lds_copy16(xdesc, lds0 + (uint32_t)(stage * TX + i * NT * 8 + wave * 64 * 8) * 2,
                       xoff[i] + (uint32_t)k0 * 2);
    };
    uint16_t *const wst = smem + NXS * TX;  // the two W images

    f32x16 acc[MI][2];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

    const int32_t n_kt = p.K / BK;  // even
    WRegs wr[2];
    copy_x(0, 0);
    load_w<NG>(wr[0], p, n0, 0, tid);
    copy_x(1, BK);
    load_w<NG>(wr[1], p, n0, BK, tid);
    wait_w<6>(wr[0]);
#pragma unroll
    for (int e = 0; e < 4; ++e) store_w_part<NG>(wr[0], wst, tid, e);
    __syncthreads();

    // two iterations per trip so the W register set is a compile-time index
    auto iteration = [&](int32_t kt, auto par) __attribute__((always_inline)) {
        constexpr int P = decltype(par)::value;  // kt & 1
        const int xs_cur = kt % NXS;
        const bool more = kt + 1 < n_kt;
        copy_x((kt + 2) % NXS, (kt + 2) * BK);
        load_w<NG>(wr[P], p, n0, (kt + 2) * BK, tid);  // set P held W(kt), stored last iteration
        const uint16_t *xs = smem + xs_cur * TX;
        const uint16_t *ws = wst + P * TW;
        uint16_t *ws_next = wst + (P ^ 1) * TW;
        // fragments of k-step ks + 1 are read while the MFMAs of step ks run
        bf16x8 fa[2][MI], fb[2][2];
        auto read_frags = [&](int ks, int buf) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const int row = wm * (BM / 2) + i * 32 + lrow;
                const int c = ks * 2 + lhi;
                fa[buf][i] = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4 *>(xs + (row * 8 + (c ^ ((row >> 1) & 7))) * 8));
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = wn * 64 + j * 32 + lrow;
                fb[buf][j] = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4 *>(ws + ((ks * TBN + n) * 2 + (lhi ^ ((n >> 3) & 1))) * 8));
            }
        };
        read_frags(0, 0);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int cb = ks & 1;
            if (ks + 1 < BK / 16) read_frags(ks + 1, cb ^ 1);
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[cb][i], fb[cb][j], acc[i][j], 0, 0, 0);
            // x(kt+1) and W(kt+1) (issued before this iteration's copies) have landed
            if (ks == 0) wait_w<6>(wr[P ^ 1]);
            if (more) store_w_part<NG>(wr[P ^ 1], ws_next, tid, ks);
        }
        __syncthreads();
    };
    for (int32_t kt = 0; kt < n_kt; kt += 2) {
        iteration(kt, std::integral_constant<int, 0>{});
        iteration(kt + 1, std::integral_constant<int, 1>{});
    }
    // The copies and W loads issued past the last k-tile land here.  The wait
    // names both W register sets: until it, they stay reserved for their
    // loads (a plain wait would let the epilogue's address arithmetic take
    // those registers while the loads could still overwrite them).
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(wr[0].w0), "+v"(wr[0].w1), "+v"(wr[1].w0), "+v"(wr[1].w1));
    __syncthreads();
    gemm_epilogue<MODE, BM, NT>(p, acc, m0, n0, wm, wn, lane, smem);
}

// ---- Dense bf16 weights: both operands copied straight into LDS ----
//
// ggml BF16 weights are [N][K] rows, the layout of x, so a W tile is staged
// like an x tile: DMA copies into a two-stage ring (x keeps its three), B
// fragments read with the same granule swizzle.  Per k-tile kt: the copies of
// W(kt+1) and then of x(kt+2) go out; the MFMAs of tile kt run; vmcnt(4)
// (everything but the x copies just issued) and one barrier.  No register
// loads, so nothing is in flight in registers.
template <int TM>
__global__ __launch_bounds__(Pipe<TM>::NT, Pipe<TM>::WG_PER_CU) void dense_gemm_pipe_kernel(GParams p) {
    using PP = Pipe<TM>;
    constexpr int NT = PP::NT, TX = PP::TX;  // a W image is TM rows x BK too
    constexpr int NWS = 2;
    __shared__ __attribute__((aligned(16))) uint16_t smem[NXS * TX + NWS * TX];
    constexpr int BM = TM, MI = BM / 64;
    static_assert(BM * 8 == 4 * NT, "four copies a thread for each operand");
    const int nwg = (int)gridDim.x;
    const int lin = (int)(blockIdx.x % 8) * (nwg / 8) + (int)(blockIdx.x / 8);
    if (lin >= p.m_tiles * p.n_tiles) return;
    const int mt = lin % p.m_tiles, nt = lin / p.m_tiles;
    const int32_t m0 = mt * BM, n0 = nt * TM;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wm = wave / PP::WN, wn = wave % PP::WN;
    const int lrow = lane & 31, lhi = lane >> 5;

    // rows past M (x) or N (W) read as zeros
    const uint16_t *xb = reinterpret_cast<const uint16_t *>(p.x) + (int64_t)m0 * p.ldx;
    const u32x4 xdesc = buf_desc(xb, (uint32_t)min<int64_t>((int64_t)(p.M - m0) * p.ldx * 2, 0xffffffffLL));
    const uint16_t *wb = reinterpret_cast<const uint16_t *>(p.wd) + (int64_t)n0 * p.ldw;
    const u32x4 wdesc = buf_desc(wb, (uint32_t)min<int64_t>((int64_t)(p.N - n0) * p.ldw * 2, 0xffffffffLL));
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t *)smem;
    uint32_t xoff[4], woff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int g = i * NT + wave * 64 + lane;
        const int row = g >> 3, c = (g & 7) ^ ((row >> 1) & 7);
        xoff[i] = (uint32_t)((row * p.ldx + c * 8) * 2);
        woff[i] = (uint32_t)((row * p.ldw + c * 8) * 2);
    }
    auto copy = [&](const u32x4 &desc, const uint32_t (&off)[4], int base, int32_t k0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            lds_copy16(desc, lds0 + (uint32_t)(base + i * NT * 8 + wave * 64 * 8) * 2, off[i] + (uint32_t)k0 * 2);
    };
    auto copy_x = [&](int stage, int32_t k0) { copy(xdesc, xoff, stage * TX, k0); };
    auto copy_w = [&](int stage, int32_t k0) { copy(wdesc, woff, (NXS + stage) * TX, k0); };

    f32x16 acc[MI][2];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

    const int32_t n_kt = p.K / BK;
    copy_w(0, 0);
    copy_x(0, 0);
    if (n_kt > 1) copy_x(1, BK);
    wait_vmcnt<0>();
    __syncthreads();
    for (int32_t kt = 0; kt < n_kt; ++kt) {
        const bool more = kt + 1 < n_kt, more2 = kt + 2 < n_kt;
        if (more) copy_w((kt + 1) % NWS, (kt + 1) * BK);
        if (more2) copy_x((kt + 2) % NXS, (kt + 2) * BK);
        const uint16_t *xs = smem + (kt % NXS) * TX;
        const uint16_t *ws = smem + (NXS + kt % NWS) * TX;
        bf16x8 fa[2][MI], fb[2][2];
        auto read_frags = [&](int ks, int buf) __attribute__((always_inline)) {
            const int c = ks * 2 + lhi;
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const int row = wm * (BM / 2) + i * 32 + lrow;
                fa[buf][i] = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4 *>(xs + (row * 8 + (c ^ ((row >> 1) & 7))) * 8));
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = wn * 64 + j * 32 + lrow;
                fb[buf][j] = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4 *>(ws + (n * 8 + (c ^ ((n >> 1) & 7))) * 8));
            }
        };
        read_frags(0, 0);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int cb = ks & 1;
            if (ks + 1 < BK / 16) read_frags(ks + 1, cb ^ 1);
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[cb][i], fb[cb][j], acc[i][j], 0, 0, 0);
        }
        // W(kt+1) and x(kt+1) have landed (only the x(kt+2) copies may fly)
        if (more2)
            wait_vmcnt<4>();
        else
            wait_vmcnt<0>();
        __syncthreads();
    }
    gemm_epilogue<Y_GATED_B16, BM, NT>(p, acc, m0, n0, wm, wn, lane, smem);
}

template <int TM>
hipError_t launch_dense_pipe(const GParams &p, hipStream_t stream) {
    const int total = p.m_tiles * p.n_tiles;
    hipLaunchKernelGGL((dense_gemm_pipe_kernel<TM>), dim3((total + 7) / 8 * 8), dim3(Pipe<TM>::NT), 0, stream, p);
    return hipGetLastError();
}

template <int MODE, int TM>
hipError_t launch_pipe(const GParams &p, hipStream_t stream) {
    const int total = p.m_tiles * p.n_tiles;
    const int grid = (total + 7) / 8 * 8;
    hipLaunchKernelGGL((w8a16_gemm_pipe_kernel<MODE, TM>), dim3(grid), dim3(Pipe<TM>::NT), 0, stream, p);
    return hipGetLastError();
}

template <int TM>
hipError_t dispatch_pipe(const GParams &p, int mode, hipStream_t stream) {
    switch (mode) {
        case Y_BF16: return launch_pipe<Y_BF16, TM>(p, stream);
        case Y_F32_ROUNDED: return launch_pipe<Y_F32_ROUNDED, TM>(p, stream);
        case Y_F32_RAW: return launch_pipe<Y_F32_RAW, TM>(p, stream);
        case Y_GATED: return launch_pipe<Y_GATED, TM>(p, stream);
        default: return launch_pipe<Y_QKV, TM>(p, stream);
    }
}

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// f32 [M][ldx] -> bf16 [M][K] (round to nearest even), four elements a thread.
// Rounding once here instead of while staging keeps the GEMM's prefetch of
// the next k-tile in flight: the staging path has to wait for its f32 loads
// before it can convert them, inside the loop.
__global__ void rows_to_bf16_kernel(const float *x, int64_t ldx, int32_t M, int32_t K, uint16_t *y) {
    const int32_t q = K / 4;
    const int64_t total = (int64_t)M * q;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t m = i / q, c = (i % q) * 4;
        const f32x4 v = *reinterpret_cast<const f32x4 *>(x + m * ldx + c);
        *reinterpret_cast<u32x2 *>(y + m * K + c) =
            u32x2{f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16),
                  f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16)};
    }
}

template <bool XF32, int MODE, int BM>
hipError_t launch(const GParams &p, hipStream_t stream) {
    const int total = p.m_tiles * p.n_tiles;
    const int grid = (total + 7) / 8 * 8;
    hipLaunchKernelGGL((w8a16_gemm_kernel<XF32, MODE, BM>), dim3(grid), dim3(256), 0, stream, p);
    return hipGetLastError();
}

template <int BM>
hipError_t dispatch(const GParams &p, bool xf32, int mode, hipStream_t stream) {
    if (xf32) {
        switch (mode) {
            case Y_BF16: return launch<true, Y_BF16, BM>(p, stream);
            case Y_F32_ROUNDED: return launch<true, Y_F32_ROUNDED, BM>(p, stream);
            case Y_F32_RAW: return launch<true, Y_F32_RAW, BM>(p, stream);
            case Y_GATED: return launch<true, Y_GATED, BM>(p, stream);
            case Y_GATED_B16: return launch<true, Y_GATED_B16, BM>(p, stream);
            default: return launch<true, Y_QKV, BM>(p, stream);
        }
    }
    switch (mode) {
        case Y_BF16: return launch<false, Y_BF16, BM>(p, stream);
        case Y_F32_ROUNDED: return launch<false, Y_F32_ROUNDED, BM>(p, stream);
        case Y_F32_RAW: return launch<false, Y_F32_RAW, BM>(p, stream);
        case Y_GATED: return launch<false, Y_GATED, BM>(p, stream);
        case Y_GATED_B16: return launch<false, Y_GATED_B16, BM>(p, stream);
        default: return launch<false, Y_QKV, BM>(p, stream);
    }
}

// f32 weights: 128 x 128 tiles of the fp32 MFMA kernel
int run_gemm_f32(GParams p, hipStream_t stream) {
    EMB_CHECK_ARG(p.x && p.wd, "null x/weight");
    EMB_CHECK_ARG(p.M > 0 && p.K > 0 && p.N > 0, "non-positive size");
    if (p.K % 4 != 0)
        return emb::set_error(EMB_ERR_UNSUPPORTED, "f32 weights need in_features %% 4 == 0 (got %d)", p.K);
    EMB_CHECK_ARG(p.ldx >= p.K && p.ldx % 4 == 0 && p.ldw >= p.K && p.ldw % 4 == 0,
                  "x and weight row strides must cover K, 16-byte aligned");
    EMB_CHECK_ARG(aligned16(p.x) && aligned16(p.wd), "x and weight must be 16-byte aligned");
    p.m_tiles = (p.M + FBM - 1) / FBM;
    p.n_tiles = (p.N + FBM - 1) / FBM;
    EMB_CHECK_ARG((int64_t)p.m_tiles * p.n_tiles < INT_MAX / 2, "problem too large");
    const int total = p.m_tiles * p.n_tiles;
    hipLaunchKernelGGL((f32_gemm_kernel<Y_GATED_F32>), dim3((total + 7) / 8 * 8), dim3(256), 0, stream, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return emb::set_error(EMB_ERR_LAUNCH, "f32 GEMM launch: %s", hipGetErrorString(e));
    return EMB_OK;
}

int run_gemm(GParams p, bool xf32, int mode, hipStream_t stream) {
    const bool dense = mode == Y_GATED_B16;
    EMB_CHECK_ARG(p.x && (dense ? p.wd != nullptr : p.qw && p.scales), "null x/weights/scales");
    EMB_CHECK_ARG(p.M > 0 && p.K > 0 && p.N > 0, "non-positive size");
    if (dense) {
        if (p.K % 16 != 0)
            return emb::set_error(EMB_ERR_UNSUPPORTED, "bf16 weights need in_features %% 16 == 0 (got %d)", p.K);
        EMB_CHECK_ARG(p.ldw >= p.K && p.ldw % 8 == 0 && aligned16(p.wd),
                      "weight rows must cover K, 16-byte aligned");
    } else if (p.K % 16 != 0 || p.N % 64 != 0)
        return emb::set_error(EMB_ERR_UNSUPPORTED, "W8A16 needs in_features %% 16 == 0 and out_features %% 64 == 0 "
                                                   "(got %d, %d)", p.K, p.N);
    EMB_CHECK_ARG(p.ldx >= p.K && (p.ldx * (xf32 ? 4 : 2)) % 16 == 0, "x row stride must cover K, 16-byte aligned");
    EMB_CHECK_ARG(aligned16(p.x) && (dense || aligned16(p.qw)), "x and qweight must be 16-byte aligned");
    EMB_CHECK_ARG((int64_t)p.M * (p.N / 64) < INT_MAX, "problem too large");
    // Tile height by rounds of resident workgroups on MI355X's 256 CUs: two
    // 256-row workgroups fit a CU (VGPRs), three 128-row ones.  A 128-row
    // tile costs about 0.77 of a 256-row one (its B-tile dequant is not
    // halved), so 128-row tiles win unless they need more rounds (measured:
    // 1560 x 3072 -> 3072 and 3200 x 4096 -> 6144 run faster with 128 rows,
    // 1560 x 3072 -> 9216 with 256).
    p.n_tiles = (p.N + BN - 1) / BN;
    const int64_t rounds256 = ((int64_t)((p.M + 255) / 256) * p.n_tiles + 511) / 512;
    const int64_t rounds128 = ((int64_t)((p.M + 127) / 128) * p.n_tiles + 767) / 768;
    const bool narrow = rounds128 <= rounds256;
    p.m_tiles = narrow ? (p.M + 127) / 128 : (p.M + 255) / 256;
    hipError_t e;
    if (xf32 && p.x_ws) {
        EMB_CHECK_ARG(aligned16(p.x_ws), "x_bf16_workspace must be 16-byte aligned");
        const int64_t units = (int64_t)p.M * (p.K / 4);
        const int64_t g = std::min<int64_t>((units + 255) / 256, 8192);
        hipLaunchKernelGGL(rows_to_bf16_kernel, dim3((unsigned)g), dim3(256), 0, stream, (const float *)p.x, p.ldx,
                           p.M, p.K, p.x_ws);
        e = hipGetLastError();
        if (e != hipSuccess) return emb::set_error(EMB_ERR_LAUNCH, "x rounding launch: %s", hipGetErrorString(e));
        p.x = p.x_ws;
        p.ldx = p.K;
        xf32 = false;
    }
    if (dense && !xf32 && p.K % BK == 0 && p.ldw % 8 == 0 && aligned16(p.x) && aligned16(p.wd)) {
        // both operands copied straight into LDS (tile size as below)
        const int64_t t256 = (int64_t)((p.M + 255) / 256) * ((p.N + 255) / 256);
        const int tm = t256 >= 192 ? 256 : 128;
        p.n_tiles = (p.N + tm - 1) / tm;
        p.m_tiles = (p.M + tm - 1) / tm;
        e = tm == 256 ? launch_dense_pipe<256>(p, stream) : launch_dense_pipe<128>(p, stream);
    } else if (!dense && !xf32 && p.K % (2 * BK) == 0 && aligned16(p.x)) {
        // x copied straight into LDS: 256 x 256 tiles when they fill at least
        // three quarters of MI355X's 256 CUs (one a CU), 128 x 128 otherwise
        // (two a CU)
        const int64_t t256 = (int64_t)((p.M + 255) / 256) * ((p.N + 255) / 256);
        const int tm = t256 >= 192 ? 256 : 128;
        p.n_tiles = (p.N + tm - 1) / tm;
        p.m_tiles = (p.M + tm - 1) / tm;
        e = tm == 256 ? dispatch_pipe<256>(p, mode, stream) : dispatch_pipe<128>(p, mode, stream);
    } else {
        e = narrow ? dispatch<128>(p, xf32, mode, stream) : dispatch<256>(p, xf32, mode, stream);
    }
    if (e != hipSuccess) return emb::set_error(EMB_ERR_LAUNCH, "w8a16 launch: %s", hipGetErrorString(e));
    return EMB_OK;
}

// The reference's shape contract (cosmos3_w8_marlin_cuda.cu:302-330, :651-703):
// qweight [in/16][out*4] int32, scales [1][out] or [out][1] bf16.
int check_ref_shapes(int batch, int in_features, int out_features, int qweight_rows, int qweight_cols, int scale_rows,
                     int scale_cols) {
    EMB_CHECK_ARG(batch > 0 && in_features > 0 && out_features > 0, "non-positive size");
    EMB_CHECK_ARG(qweight_rows == in_features / 16 && qweight_cols == out_features * 4,
                  "qweight must be [in/16][out*4] (got [%d][%d])", qweight_rows, qweight_cols);
    EMB_CHECK_ARG((scale_rows == 1 && scale_cols == out_features) || (scale_rows == out_features && scale_cols == 1),
                  "scales must be [1][out] or [out][1]");
    return EMB_OK;
}

__global__ void f32_to_bf16_kernel(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = (uint16_t)f32_to_bf16_bits(x[i]);
}

// Argument checks and parameters shared by the gated-residual entry points.
// residual may be NULL here (the dense entry's plain projection); out may be
// the residual itself (each element is read, then written, by one thread);
// any other overlap of out with an input is rejected, and so is a bf16
// workspace that overlaps anything the GEMM reads or writes after filling it.
int gated_params(GParams &p, const void *x, int32_t x_is_f32, int64_t ldx, int32_t M, int32_t K, int32_t N,
                 const float *bias, const float *gate, int64_t ldg, const float *gate_bias, const float *residual,
                 int64_t ldr, float *out, int64_t ldo, int32_t round_bf16, void *x_bf16_workspace) {
    EMB_CHECK_ARG(out, "null out");
    EMB_CHECK_ARG(M > 0 && K > 0 && N > 0, "non-positive size");
    EMB_CHECK_ARG((!residual || ldr >= N) && ldo >= N, "ldr and ldo must cover N");
    EMB_CHECK_ARG(!gate || ldg >= N, "ldg must cover N");
    EMB_CHECK_ARG(gate || !gate_bias, "gate_bias needs a gate");
    const float *olo = out, *ohi = out + (int64_t)(M - 1) * ldo + N;
    auto overlaps = [&](const void *q, int64_t bytes) {
        const char *a = (const char *)q, *b = a + bytes;
        return q && a < (const char *)ohi && (const char *)olo < b;
    };
    EMB_CHECK_ARG(!residual || residual == out || !overlaps(residual, ((int64_t)(M - 1) * ldr + N) * 4),
                  "out overlaps residual without being it");
    EMB_CHECK_ARG(!overlaps(gate, gate ? ((int64_t)(M - 1) * ldg + N) * 4 : 0) && !overlaps(bias, (int64_t)N * 4) &&
                      !overlaps(gate_bias, (int64_t)N * 4),
                  "out overlaps gate or bias");
    EMB_CHECK_ARG(residual != out || ldr == ldo, "in-place update needs ldr == ldo");
    if (x_is_f32 && x_bf16_workspace) {  // the workspace is written before the GEMM reads the others
        const char *w0 = (const char *)x_bf16_workspace, *w1 = w0 + (int64_t)M * K * 2;
        auto hits = [&](const void *q, int64_t bytes) {
            return q && (const char *)q < w1 && w0 < (const char *)q + bytes;
        };
        EMB_CHECK_ARG(!hits(out, ((int64_t)(M - 1) * ldo + N) * 4) &&
                          !hits(residual, residual ? ((int64_t)(M - 1) * ldr + N) * 4 : 0) &&
                          !hits(gate, gate ? ((int64_t)(M - 1) * ldg + N) * 4 : 0) && !hits(bias, (int64_t)N * 4) &&
                          !hits(gate_bias, (int64_t)N * 4) && !hits(x, ((int64_t)(M - 1) * ldx + K) * 4),
                      "x_bf16_workspace overlaps an input or out");
    }
    p.x = x;
    p.ldx = ldx;
    p.M = M;
    p.K = K;
    p.N = N;
    p.y = out;
    p.ldy = ldo;
    p.bias = bias;
    p.gate = gate;
    p.gate_bias = gate_bias;
    p.res = residual;
    p.ldg = ldg;
    p.ldr = ldr;
    p.round_out = round_bf16 != 0;
    p.x_ws = (uint16_t *)x_bf16_workspace;
    return EMB_OK;
}

}  // namespace

extern "C" {

int emb_w8a16_gemm(const void *x, int32_t x_is_f32, int64_t ldx, const int32_t *qweight, const uint16_t *scales,
                   int32_t M, int32_t K, int32_t N, void *y, int64_t ldy, int32_t y_kind, hipStream_t stream) {
    EMB_CHECK_ARG(y, "null y");
    EMB_CHECK_ARG(y_kind >= EMB_W8_Y_BF16 && y_kind <= EMB_W8_Y_F32_RAW, "unknown y_kind");
    EMB_CHECK_ARG(ldy >= N, "ldy must cover N");
    GParams p{};
    p.x = x;
    p.ldx = ldx;
    p.qw = reinterpret_cast<const uint32_t *>(qweight);
    p.scales = scales;
    p.M = M;
    p.K = K;
    p.N = N;
    p.y = y;
    p.ldy = ldy;
    return run_gemm(p, x_is_f32 != 0, y_kind, stream);
}

int emb_w8a16_qkv_append(const void *x, int32_t x_is_f32, int64_t ldx, const int32_t *qweight,
                         const uint16_t *scales, int32_t M, int32_t K, int32_t n_q, void *q_out, int64_t ldq,
                         const int32_t *slots, const int32_t *block_table, int32_t capacity, void *k_pool,
                         void *v_pool, void *v16_pool, int32_t n_kv_heads, int32_t head_dim, hipStream_t stream) {
    EMB_CHECK_ARG(slots && k_pool && v_pool, "null slots/pool");
    EMB_CHECK_ARG(n_q >= 0 && n_kv_heads > 0 && head_dim > 0 && capacity > 0, "bad sizes");
    EMB_CHECK_ARG(n_q == 0 || (q_out && ldq >= n_q), "q_out and ldq >= n_q required when n_q > 0");
    EMB_CHECK_ARG(aligned16(v_pool) && aligned16(v16_pool), "v_pool and v16_pool must be 16-byte aligned");
    GParams p{};
    p.x = x;
    p.ldx = ldx;
    p.qw = reinterpret_cast<const uint32_t *>(qweight);
    p.scales = scales;
    p.M = M;
    p.K = K;
    p.n_q = n_q;
    p.n_kv = n_kv_heads * head_dim;
    p.N = n_q + 2 * p.n_kv;
    p.y = q_out;
    p.ldy = ldq;
    p.head_dim = head_dim;
    p.hkv = n_kv_heads;
    p.capacity = capacity;
    p.slots = slots;
    p.bt = block_table;
    p.k_pool = (uint16_t *)k_pool;
    p.v_pool = (uint16_t *)v_pool;
    p.v16_pool = (uint16_t *)v16_pool;
    return run_gemm(p, x_is_f32 != 0, Y_QKV, stream);
}

int emb_w8a16_gated_residual(const void *x, int32_t x_is_f32, int64_t ldx, const int32_t *qweight,
                             const uint16_t *scales, int32_t M, int32_t K, int32_t N, const float *bias,
                             const float *gate, int64_t ldg, const float *gate_bias, const float *residual,
                             int64_t ldr, float *out, int64_t ldo, int32_t round_bf16, void *x_bf16_workspace,
                             hipStream_t stream) {
    EMB_CHECK_ARG(residual, "null residual");
    GParams p{};
    const int rc = gated_params(p, x, x_is_f32, ldx, M, K, N, bias, gate, ldg, gate_bias, residual, ldr, out, ldo,
                                round_bf16, x_bf16_workspace);
    if (rc) return rc;
    p.qw = reinterpret_cast<const uint32_t *>(qweight);
    p.scales = scales;
    return run_gemm(p, x_is_f32 != 0, Y_GATED, stream);
}

int emb_dense_gated_residual(const void *x, int32_t x_is_f32, int64_t ldx, const void *weight, int32_t weight_type,
                             int64_t ldw, int32_t M, int32_t K, int32_t N, const float *bias, const float *gate,
                             int64_t ldg, const float *gate_bias, const float *residual, int64_t ldr, float *out,
                             int64_t ldo, int32_t round_bf16, void *x_bf16_workspace, hipStream_t stream) {
    EMB_CHECK_ARG(weight, "null weight");
    if (weight_type != EMB_GGML_BF16 && weight_type != EMB_GGML_F32)
        return emb::set_error(EMB_ERR_UNSUPPORTED, "weight_type must be ggml BF16 (30) or F32 (0), got %d",
                              weight_type);
    if (weight_type == EMB_GGML_F32 && !x_is_f32)
        return emb::set_error(EMB_ERR_UNSUPPORTED, "f32 weights take f32 x");
    const bool f32w = weight_type == EMB_GGML_F32;
    EMB_CHECK_ARG(ldw >= K, "ldw must cover K");
    // the weights are read while out is written: no overlap
    if (out && M > 0 && N > 0 && ldo >= N) {
        const char *w0 = (const char *)weight, *w1 = w0 + ((int64_t)(N - 1) * ldw + K) * (f32w ? 4 : 2);
        const char *o0 = (const char *)out, *o1 = (const char *)(out + (int64_t)(M - 1) * ldo + N);
        EMB_CHECK_ARG(!(w0 < o1 && o0 < w1), "out overlaps the weights");
    }
    GParams p{};
    const int rc = gated_params(p, x, x_is_f32, ldx, M, K, N, bias, gate, ldg, gate_bias, residual, ldr, out, ldo,
                                round_bf16, f32w ? nullptr : x_bf16_workspace);
    if (rc) return rc;
    p.wd = weight;
    p.ldw = ldw;
    if (f32w) return run_gemm_f32(p, stream);
    return run_gemm(p, x_is_f32 != 0, Y_GATED_B16, stream);
}

// ---- reference-named face (kernels/cosmos3/cosmos3_w8_marlin_cuda.h:24-84) ----
// y is f32 holding the bf16-rounded result, as the reference's bf16 -> f32
// widening (cosmos3_w8_marlin_cuda.cu:407) leaves it.  linear_f32_ws rounds x
// into x_bf16_workspace first (as the reference does, :446-455) and runs the
// bf16 GEMM; linear_f32 has no workspace and rounds x while staging it.  The
// other workspaces are accepted and unused: no split-K reduction buffer is
// needed.

int cosmos3_w8a16_linear_f32(const float *x, const int *qweight, const unsigned short *scales_bf16, float *y,
                             int batch, int in_features, int out_features, int qweight_rows, int qweight_cols,
                             int scale_rows, int scale_cols, hipStream_t stream) {
    const int rc = check_ref_shapes(batch, in_features, out_features, qweight_rows, qweight_cols, scale_rows,
                                    scale_cols);
    if (rc) return rc;
    return emb_w8a16_gemm(x, 1, in_features, qweight, scales_bf16, batch, in_features, out_features, y, out_features,
                          EMB_W8_Y_F32_ROUNDED, stream);
}

int cosmos3_w8a16_linear_f32_ws(const float *x, const int *qweight, const unsigned short *scales_bf16, float *y,
                                unsigned short *x_bf16_workspace, unsigned short *y_bf16_workspace,
                                float *c_tmp_workspace, int *int_workspace, int batch, int in_features,
                                int out_features, int qweight_rows, int qweight_cols, int scale_rows, int scale_cols,
                                hipStream_t stream) {
    (void)y_bf16_workspace;
    (void)c_tmp_workspace;
    (void)int_workspace;
    const int rc = check_ref_shapes(batch, in_features, out_features, qweight_rows, qweight_cols, scale_rows,
                                    scale_cols);
    if (rc) return rc;
    EMB_CHECK_ARG(y, "null y");
    GParams p{};
    p.x = x;
    p.ldx = in_features;
    p.qw = reinterpret_cast<const uint32_t *>(qweight);
    p.scales = scales_bf16;
    p.M = batch;
    p.K = in_features;
    p.N = out_features;
    p.y = y;
    p.ldy = out_features;
    p.x_ws = x_bf16_workspace;  // rounded once into it, then the bf16 GEMM
    return run_gemm(p, true, Y_F32_ROUNDED, stream);
}

int cosmos3_w8a16_linear_bf16_ws(const unsigned short *x_bf16, const int *qweight, const unsigned short *scales_bf16,
                                 float *y, unsigned short *y_bf16_workspace, float *c_tmp_workspace,
                                 int *int_workspace, int batch, int in_features, int out_features, int qweight_rows,
                                 int qweight_cols, int scale_rows, int scale_cols, hipStream_t stream) {
    (void)y_bf16_workspace;
    (void)c_tmp_workspace;
    (void)int_workspace;
    const int rc = check_ref_shapes(batch, in_features, out_features, qweight_rows, qweight_cols, scale_rows,
                                    scale_cols);
    if (rc) return rc;
    return emb_w8a16_gemm(x_bf16, 0, in_features, qweight, scales_bf16, batch, in_features, out_features, y,
                          out_features, EMB_W8_Y_F32_ROUNDED, stream);
}

int cosmos3_w8a16_f32_to_bf16_ws(const float *x, unsigned short *x_bf16_workspace, int count, hipStream_t stream) {
    EMB_CHECK_ARG(x && x_bf16_workspace && count > 0, "bad arguments");
    int64_t g = ((int64_t)count + 255) / 256;
    if (g > 65536) g = 65536;
    hipLaunchKernelGGL(f32_to_bf16_kernel, dim3((int)g), dim3(256), 0, stream, x, (uint16_t *)x_bf16_workspace,
                       (int64_t)count);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return emb::set_error(EMB_ERR_LAUNCH, "f32_to_bf16 launch: %s", hipGetErrorString(e));
    return EMB_OK;
}

}  // extern "C"
