// Paged block-masked attention for gfx950 (MI355X).
//
// out[q, h] = sum_j softmax_j(scale * q.k_j + mask) v_j over the keys of one
// sequence, the keys living in 16-slot pages of a bf16 pool (layout in
// emb_kv.h).  Reference semantics: runtime_kv_attn_* over valid slots
// (kernels/lingbot/lingbot_flex_attn_cuda.cu:651-873), flex_attn with a CSR
// block table and token mask (:502-582), and the ggml attention the VLA
// experts call (models/pi05.cpp:405-418, models/hy_vla.cpp:1066-1076) with
// GQA broadcast (q head h reads kv head h / (hq/hkv)).
//
// Work decomposition.  A workgroup of 4 waves owns 128 query rows of one
// (sequence, kv head); a row is (token, q head of the GQA group), so all query
// heads that share a kv head also share every K/V tile the workgroup stages in
// LDS.  Each wave owns 32 rows.  Keys stream in tiles of KT = 32 keys (64 at
// head_dim 64).
//
// Per wave and key tile the math is done transposed, with MFMA 32x32x16:
//   S^T[32 keys x 32 rows] = K[keys x D] . Q^T       (bf16 x bf16 -> f32)
//   O^T[D x 32 rows]      += V^T[D x keys] . P^T      (f16 x f16 -> f32)
// so that lane l owns query row l%32: its scores and its D/2 output
// accumulators all belong to the same row, the row max needs one cross-lane
// step (lanes l and l^32), and rescaling needs no shuffles.  P and V go through
// f16 rather than bf16 because P in bf16 (8 significant bits) alone would put
// the mean relative error near 1.1e-3; f16 keeps it near 2e-4.  V in f16 is
// exact for |v| in [2^-14, 65504].
//
// LDS image of a key tile (one pipeline stage):
//   K: row r (key), 16-byte chunk c (dims 8c..8c+7) at r*D + ((c ^ swz(r))*8),
//      swz(r) = r & min(D/8 - 1, 15): the XOR keeps the 16 rows one MFMA
//      operand read touches on distinct banks without padding.
//   V: page p of the tile, dim d: 16 f16 keys at (p*D + d)*16, in the key
//      order the P.V MFMA consumes (key t at position t with bits 2 and 3
//      swapped), the two 8-key halves exchanged when bit 3 of d is set.
// Tiles reach LDS in one of three ways:
//   * DMA: with an f16 V shadow pool (written by the append in exactly the
//     V image above), K rows and V pages are copied by buffer loads that write
//     LDS directly (16 bytes a lane); no registers, no conversion.
//   * REG: bf16 V is loaded into registers, converted to f16 and permuted,
//     then written; K goes the same way.
//   * VALID: like REG, but key j is the slot valid[j] of an arbitrary list.
// Page ids come from an LDS copy of the block-table segment; each page is read
// through a buffer resource sized to its valid rows, so the end of the key
// list reads as zeros without branches.
//
// Pipeline over three LDS stages: at tile t, one stage holds tile t (its V
// feeds P.V), one tile t+1 (its K feeds the next S) and one receives tile t+2,
// whose loads are in flight for the whole iteration.  The S MFMAs of tile t+1
// overlap the softmax VALU work of tile t, and the P.V MFMAs of tile t overlap
// the staging of tile t+2.  One barrier a tile.
//
// The online softmax keeps the running max in raw score units and rescales
// the accumulators only when some row's max grows by more than 2^8 in the
// exponent; the decision is taken per wave (ballot), so the rescale is a
// uniform branch that most tiles skip.
//
// Split-K: with splits > 1 each workgroup handles one key range and writes
// unnormalised partials (O, m, l) that attn_merge_kernel combines.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <mutex>
#include <type_traits>

#include "attn_dev.h"
#include "emb_common.h"

// Split-K scratch of emb_paged_attention_noalloc: the partials of a call live
// here instead of in a caller workspace.  One copy per device the library
// runs on, held until the process ends; every call on a device shares it.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)48 << 20;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {

using namespace emb_attn;
typedef __attribute__((address_space(3))) void lds_void;

constexpr int WAVES = 4;
constexpr int ROWS_PER_WAVE = 32;
constexpr int ROWS_PER_WG = WAVES * ROWS_PER_WAVE;
constexpr int SEG_PAGES = 1024;  // block-table entries held in LDS at a time (16384 keys)
// Block-table entries every wave of the DMA path holds in registers from the start.
constexpr int WIN_PAGES = 128;
// LDS fragment reads kept in flight ahead of the MFMA that consumes them: the
// LDS latency is several MFMA issue slots, and the compiler's own schedule
// issues each read just one MFMA ahead.
constexpr int AHEAD = 4;

enum { LD_DMA = 0, LD_REG = 1, LD_VALID = 2 };

template <int D>
struct Geo {
    // keys per tile: two pages at D >= 128 (three stages of 32 keys fit two
    // workgroups a CU at D = 128), four at D = 64
    static constexpr int KT = D >= 128 ? 32 : 64;
    static constexpr int KB = KT / 32;          // 32-key MFMA blocks per tile
    static constexpr int PAGES = KT / 16;
    static constexpr int CH = D / 8;            // 16-byte chunks per key row
    static constexpr int SWZ = (CH < 16 ? CH : 16) - 1;
    static constexpr int K_ELEMS = KT * D;      // bf16 K image
    static constexpr int V_ELEMS = KT * D;      // f16 V image
    static constexpr int STAGE = K_ELEMS + V_ELEMS;
    static constexpr int BLOCKS = K_ELEMS * 2 / 1024;  // 1 KB DMA blocks per image
    static constexpr int KPT = KT * CH / 256;   // register path: K chunks per thread
    static constexpr int VPT = D * KT / 8 / 256;
    static constexpr int MIN_WG = D >= 256 ? 1 : 2;
    static_assert(KPT >= 1 && VPT >= 1 && BLOCKS % 4 == 0, "tile too small for 256 threads");
};

struct KParams {
    const void *q;
    float *out;
    int64_t q_stride, out_stride;
    int32_t round_out;  // store every output value rounded to bf16 precision
    const int32_t *cu_q;
    const int32_t *n_keys;
    const int32_t *q_pos0;
    int32_t nq_single, nk_single;  // per-sequence bounds when cu_q / n_keys are null
    const uint16_t *k_pool;
    const uint16_t *v_pool;
    const uint16_t *v16_pool;
    const int32_t *bt;
    int32_t bt_stride;
    const int32_t *valid;
    int32_t valid_stride;
    int32_t capacity;
    int32_t batch, hq, hkv, G;
    int32_t max_q;
    int32_t row_tiles;
    int32_t splits;
    int32_t split_keys;  // > 0: a sequence of n keys takes min(splits, ceil(n / split_keys)) splits
    int32_t total_wg;
    float scale;
    float c_log2;     // scale * log2(e)
    float th_raw;     // RESCALE_TH / c_log2
    float inv_scale;  // 1 / scale (additive masks are added in raw score units)
    int32_t chunk, window;
    const void *mask;
    int64_t mask_q_stride, mask_b_stride;
    const uint8_t *bmap;
    int32_t bsize, bmap_cols;
    int64_t bmap_b_stride;
    // [batch*hkv][splits][row_tiles*128][D] f16: the split's O / l, each
    // 32-row block in the MFMA accumulator order (element ((c*64 + lane)*4 + e)
    // of a block is dims c*8 + (lane/32)*4 + e of row lane%32)
    uint16_t *ws_o;
    // [batch*hkv][splits][row_tiles*128][4]: m (log2 units), l, k0, k1 (dims
    // [0, D/2) of O/l stored as O/l * 2^-k0, dims [D/2, D) with 2^-k1)
    float *ws_ml;
};

// Two bf16 (packed in a dword) -> two f16 (packed in a dword), round to nearest even.
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t w) {
    const _Float16 lo = (_Float16)bf16_to_f32(w & 0xffffu);
    const _Float16 hi = (_Float16)bf16_to_f32(w >> 16);
    return (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

// Page of logical slot `slot` of sequence b (identity map without a table).
__device__ __forceinline__ int32_t page_of(const int32_t *bt_b, int32_t slot) {
    return bt_b ? bt_b[slot >> 4] : (slot >> 4);
}

// Element offsets inside a stage (see the header comment).
// Splits a sequence with nk keys takes (the merge kernel reads the same count).
__device__ __forceinline__ int32_t seq_splits(const KParams &p, int32_t nk) {
    if (p.split_keys <= 0) return p.splits;
    return min(p.splits, max(1, (nk + p.split_keys - 1) / p.split_keys));
}

template <int D>
__device__ __forceinline__ int k_off(int row, int chunk) {
    return row * D + ((chunk ^ (row & Geo<D>::SWZ)) << 3);
}
template <int D>
__device__ __forceinline__ int v_off(int page, int d, int half) {
    return Geo<D>::K_ELEMS + (page * D + d) * 16 + ((half ^ ((d >> 3) & 1)) << 3);
}

// The tile's page ids (uniform over the workgroup) from the LDS block table.
template <int D>
__device__ __forceinline__ void tile_pages(const int32_t *pt, int32_t (&pid)[Geo<D>::PAGES]) {
    if constexpr (Geo<D>::PAGES == 4) {
        const i32x4 w = *reinterpret_cast<const i32x4 *>(pt);
#pragma unroll
        for (int i = 0; i < 4; ++i) pid[i] = __builtin_amdgcn_readfirstlane(w[i]);
    } else {
        const i32x2 w = *reinterpret_cast<const i32x2 *>(pt);
        pid[0] = __builtin_amdgcn_readfirstlane(w[0]);
        pid[1] = __builtin_amdgcn_readfirstlane(w[1]);
    }
}

// Tile keys k0 + [0, KT), key j = logical slot j.  Buffer resources of the
// tile's pages: K covers only the rows below lim = min(n_keys, capacity), V
// the whole page (nothing for an unmapped page).
template <int D>
__device__ __forceinline__ void page_rsrc(const KParams &p, const uint16_t *vbase, const int32_t (&pid)[Geo<D>::PAGES],
                                          int32_t k0, int32_t lim, int32_t kvh,
                                          __amdgpu_buffer_rsrc_t (&kr)[Geo<D>::PAGES],
                                          __amdgpu_buffer_rsrc_t (&vr)[Geo<D>::PAGES]) {
#pragma unroll
    for (int pg = 0; pg < Geo<D>::PAGES; ++pg) {
        const int32_t page = pid[pg];
        // readfirstlane: the clamp may be selected as a VALU op, and a
        // descriptor word in a VGPR turns every load into a waterfall loop
        const int32_t rows =
            __builtin_amdgcn_readfirstlane(page < 0 ? 0 : min(max(lim - (k0 + pg * 16), 0), 16));
        const int64_t off = page < 0 ? 0 : ((int64_t)page * p.hkv + kvh) * (16 * D);
        kr[pg] = __builtin_amdgcn_make_buffer_rsrc((void *)(p.k_pool + off), 0, rows * D * 2, RSRC_W3);
        vr[pg] = __builtin_amdgcn_make_buffer_rsrc((void *)(vbase + off), 0, rows > 0 ? 16 * D * 2 : 0, RSRC_W3);
    }
}


// DMA path: the tile's K rows and f16 V-shadow pages go straight into the
// stage.  Wave w copies 1 KB blocks b = 4j + w of each image; block b of the
// K image holds key rows [b*64/CH, (b+1)*64/CH), so lane i loads the global
// chunk that the XOR swizzle puts at slot (b*64 + i) % CH of its row.  A block
// never crosses a page, so one descriptor serves all 64 lanes.  The per-lane
// byte offsets do not depend on the tile and are computed once.
template <int D>
struct DmaPlan {
    using G = Geo<D>;
    static constexpr int NB = G::BLOCKS / 4;  // blocks per wave and image
    static constexpr int PER_TILE = 2 * NB;   // copies per wave and tile
    static constexpr int RB = 64 / G::CH;     // key rows per K block
    uint32_t koff[NB], voff[NB];
    int wave;

    __device__ __forceinline__ void init() {
        const int lane = threadIdx.x & 63;
        wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int b = j * 4 + wave;
            const int q = b * 64 + lane;
            const int r = q / G::CH, sl = q % G::CH;
            const int c = sl ^ (r & G::SWZ);
            koff[j] = ((r & 15) * D + c * 8) * 2;
            // V image: page pp covers blocks [pp*D/32, (pp+1)*D/32)
            const int pp = D >= 128 ? (j * 4 * 32) / D : 2 * j + (wave >> 1);
            voff[j] = b * 1024 - pp * D * 32 + lane * 16;
        }
    }

    // Descriptors of one tile's pages: K covers the rows below lim =
    // min(n_keys, capacity), V the whole page of a mapped page.
    struct Descs {
        u32x4 kd[G::PAGES], vd[G::PAGES];
    };
    __device__ __forceinline__ void prepare(const KParams &p, const int32_t *pt, int32_t k0, int32_t lim, int32_t kvh,
                                            Descs &ds) const {
        int32_t pid[G::PAGES];
        tile_pages<D>(pt, pid);
        prepare_ids(p, pid, k0, lim, kvh, ds);
    }
    __device__ __forceinline__ void prepare_ids(const KParams &p, const int32_t (&pid)[G::PAGES], int32_t k0,
                                                int32_t lim, int32_t kvh, Descs &ds) const {
#pragma unroll
        for (int pg = 0; pg < G::PAGES; ++pg) {
            const int32_t page = pid[pg];
            const int32_t rows = page < 0 ? 0 : min(max(lim - (k0 + pg * 16), 0), 16);
            const int64_t off = page < 0 ? 0 : ((int64_t)page * p.hkv + kvh) * (16 * D);
            ds.kd[pg] = buf_desc(p.k_pool + off, rows * D * 2);
            ds.vd[pg] = buf_desc(p.v16_pool + off, rows > 0 ? 16 * D * 2 : 0);
        }
        // The descriptors may come from VALU writes of SGPRs (readfirstlane);
        // a VMEM read of such an SGPR needs 5 wait states, which the compiler
        // does not insert for inline-asm operands.
        asm volatile("s_nop 4");
    }

    // Descriptors with no records: copies through them write zeros.
    __device__ __forceinline__ void empty(Descs &ds) const {
        const u32x4 z = {0u, 0u, 0u, RSRC_W3};
#pragma unroll
        for (int pg = 0; pg < G::PAGES; ++pg) ds.kd[pg] = ds.vd[pg] = z;
    }

    // Copy n of this wave's PER_TILE copies of a tile into the stage at LDS
    // byte address st: n < NB is K block 4n + w, the rest V blocks.
    __device__ __forceinline__ void copy(const Descs &ds, uint32_t st, int n) const {
        if (n < NB) {
            const int j = n, b = j * 4 + wave;
            u32x4 dk;
            // page of K block b = (4j + w) * RB / 16: j*RB/4 for RB <= 4 (w < 4),
            // 2j + w/2 for RB = 8 (D = 64)
            if constexpr (RB <= 4)
                dk = ds.kd[(j * RB) / 4];
            else
                dk = (wave >> 1) ? ds.kd[2 * j + 1] : ds.kd[2 * j];
            lds_copy16(dk, __builtin_amdgcn_readfirstlane(st + b * 1024), koff[j]);
        } else {
            const int j = n - NB, b = j * 4 + wave;
            u32x4 dv;
            if constexpr (D >= 128)
                dv = ds.vd[(j * 4 * 32) / D];
            else
                dv = (wave >> 1) ? ds.vd[2 * j + 1] : ds.vd[2 * j];
            lds_copy16(dv, __builtin_amdgcn_readfirstlane(st + G::K_ELEMS * 2 + b * 1024), voff[j]);
        }
    }

    // All copies of tile keys [k0, k0 + KT), pages pid, into the stage at LDS
    // byte address st.
    __device__ __forceinline__ void issue_ids(const KParams &p, const int32_t (&pid)[G::PAGES], int32_t k0,
                                              int32_t lim, int32_t kvh, uint32_t st) const {
        Descs ds;
        prepare_ids(p, pid, k0, lim, kvh, ds);
#pragma unroll
        for (int n = 0; n < PER_TILE; ++n) copy(ds, st, n);
    }
};

// Register paths: global -> registers (in flight during the compute of the
// previous tile) -> converted and written into the stage image.
template <int D, bool VALID>
struct RegLoader {
    using G = Geo<D>;
    u32x4 k[G::KPT];
    u32x4 v[G::VPT];

    __device__ __forceinline__ void issue_direct(const KParams &p, const int32_t *pt, int32_t k0, int32_t lim,
                                                 int32_t kvh) {
        const int tid = threadIdx.x;
        int32_t pid[G::PAGES];
        tile_pages<D>(pt, pid);
        __amdgpu_buffer_rsrc_t kr[G::PAGES], vr[G::PAGES];
        page_rsrc<D>(p, p.v_pool, pid, k0, lim, kvh, kr, vr);
        // Page of a chunk.  A page holds 16*CH K chunks and 2*D V chunks; at
        // D >= 128 that is >= 256, so chunk i of every thread lies in page
        // i*256/(page chunks), a constant.  At D = 64 a page is 128 chunks and
        // the lower and upper 128 threads read consecutive pages (a choice
        // between two descriptors on a wave-uniform condition).
        const bool upper = __builtin_amdgcn_readfirstlane(tid >> 7) != 0;
#pragma unroll
        for (int i = 0; i < G::KPT; ++i) {
            const int c = tid + i * 256;
            const int key = c / G::CH, dc = c % G::CH;
            __amdgpu_buffer_rsrc_t r;
            if constexpr (16 * G::CH >= 256)
                r = kr[i * 256 / (16 * G::CH)];
            else
                r = upper ? kr[2 * i + 1] : kr[2 * i];
            k[i] = __builtin_bit_cast(u32x4,
                                      __builtin_amdgcn_raw_buffer_load_b128(r, ((key & 15) * D + dc * 8) * 2, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < G::VPT; ++i) {
            const int c = tid + i * 256;
            const int rem = c % (2 * D);
            const int d = rem >> 1, half = rem & 1;
            __amdgpu_buffer_rsrc_t r;
            if constexpr (2 * D >= 256)
                r = vr[i * 256 / (2 * D)];
            else
                r = upper ? vr[2 * i + 1] : vr[2 * i];
            v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (d * 16 + half * 8) * 2, 0, 0));
        }
        if (k0 + G::KT > lim) {  // last tile: zero V of the keys past the end
#pragma unroll
            for (int i = 0; i < G::VPT; ++i) {
                const int c = tid + i * 256;
                const int pg = c / (2 * D);
                const int half = (c % (2 * D)) & 1;
                const int32_t jb = k0 + pg * 16 + half * 8;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (jb + e >= lim) v[i][e >> 1] &= (e & 1) ? 0x0000ffffu : 0xffff0000u;
            }
        }
    }

    // With a valid-slot list key j is logical slot valid[j] (a negative or
    // out-of-range slot is a zero row).
    __device__ __forceinline__ void issue_valid(const KParams &p, const int32_t *valid_b, const int32_t *bt_b,
                                                int32_t k0, int32_t nk, int32_t kvh) {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < G::KPT; ++i) {
            const int c = tid + i * 256;
            const int key = c / G::CH, dc = c % G::CH;
            const int32_t j = k0 + key;
            k[i] = u32x4{0u, 0u, 0u, 0u};
            const int32_t s = j < nk ? valid_b[j] : -1;
            if (s >= 0 && s < p.capacity) {
                const int32_t page = page_of(bt_b, s);
                if (page >= 0)
                    k[i] = *reinterpret_cast<const u32x4 *>(
                        p.k_pool + (((int64_t)page * p.hkv + kvh) * 16 + (s & 15)) * D + dc * 8);
            }
        }
#pragma unroll
        for (int i = 0; i < G::VPT; ++i) {
            const int c = tid + i * 256;
            const int pg = c / (2 * D);
            const int rem = c % (2 * D);
            const int d = rem >> 1, half = rem & 1;
            const int32_t jb = k0 + pg * 16 + half * 8;
            int32_t s[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) s[e] = jb + e < nk ? valid_b[jb + e] : -1;
            bool run = s[0] >= 0 && (s[0] & 7) == 0 && s[0] + 7 < p.capacity;
#pragma unroll
            for (int e = 1; e < 8; ++e) run = run && s[e] == s[0] + e;
            u32x4 w = {0u, 0u, 0u, 0u};
            if (run) {
                const int32_t page = page_of(bt_b, s[0]);
                if (page >= 0)
                    w = *reinterpret_cast<const u32x4 *>(p.v_pool + (((int64_t)page * p.hkv + kvh) * D + d) * 16 +
                                                         (s[0] & 15));
            } else {
                uint32_t hv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    hv[e] = 0u;
                    if (s[e] >= 0 && s[e] < p.capacity) {
                        const int32_t page = page_of(bt_b, s[e]);
                        if (page >= 0) hv[e] = p.v_pool[(((int64_t)page * p.hkv + kvh) * D + d) * 16 + (s[e] & 15)];
                    }
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = hv[2 * e] | (hv[2 * e + 1] << 16);
            }
            v[i] = w;
        }
    }

    // Registers -> stage image: K chunks to their swizzled slots; V to f16, keys
    // +0..3 of the 8-key half to permuted positions half*4.. of image half 0,
    // keys +4..7 to image half 1.
    __device__ __forceinline__ void store(uint16_t *stage) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < G::KPT; ++i) {
            const int c = tid + i * 256;
            const int key = c / G::CH, dc = c % G::CH;
            *reinterpret_cast<u32x4 *>(&stage[k_off<D>(key, dc)]) = k[i];
        }
#pragma unroll
        for (int i = 0; i < G::VPT; ++i) {
            const int c = tid + i * 256;
            const int pg = c / (2 * D);
            const int rem = c % (2 * D);
            const int d = rem >> 1, half = rem & 1;
            const u32x2 lo = {bf16x2_to_f16x2(v[i][0]), bf16x2_to_f16x2(v[i][1])};  // keys +0..3
            const u32x2 hi = {bf16x2_to_f16x2(v[i][2]), bf16x2_to_f16x2(v[i][3])};  // keys +4..7
            *reinterpret_cast<u32x2 *>(&stage[v_off<D>(pg, d, 0) + half * 4]) = lo;
            *reinterpret_cast<u32x2 *>(&stage[v_off<D>(pg, d, 1) + half * 4]) = hi;
        }
    }
};

// pt[i] = page id of page index seg_p0 + i, or -1 at and past p_end.
// (All loads first, then all LDS writes: one memory round trip, not four.)
__device__ __forceinline__ void load_segment(const int32_t *bt_b, int32_t seg_p0, int32_t p_end, int32_t *pt) {
    static_assert(SEG_PAGES % 256 == 0, "segment must split evenly over the workgroup");
    int32_t v[SEG_PAGES / 256];
#pragma unroll
    for (int k = 0; k < SEG_PAGES / 256; ++k) {
        const int32_t pi = seg_p0 + (int)threadIdx.x + k * 256;
        v[k] = pi < p_end ? page_of(bt_b, pi * 16) : -1;
    }
#pragma unroll
    for (int k = 0; k < SEG_PAGES / 256; ++k) pt[threadIdx.x + k * 256] = v[k];
}

// Workgroups a CU holds.  At head_dim 128 the unmasked DMA kernel runs three
// (a three-stage ring, 52 KB of LDS and at most 168 VGPRs each; the few
// values that do not fit live outside the key loop): a third wave per SIMD
// hides more of each tile's latency.  The masked and register-staged
// variants would spill inside the loop there, so they keep two.
template <int D, int MASK, int LD>
constexpr int wg_per_cu() {
    return D == 128 && LD == LD_DMA && MASK == EMB_MASK_FULL ? 3 : Geo<D>::MIN_WG;
}

template <int D, int MASK, int LD, bool QF32>
__global__ __launch_bounds__(256, (wg_per_cu<D, MASK, LD>())) void paged_attn_kernel(KParams p) {
    using G = Geo<D>;
    constexpr bool VALID = LD == LD_VALID;
    // four stages when the copies bypass registers (a tile's loads get two
    // iterations to land), three otherwise and where three workgroups share a CU
    constexpr int NST = LD == LD_DMA && wg_per_cu<D, MASK, LD>() < 3 ? 4 : 3;
    __shared__ __attribute__((aligned(16))) uint16_t smem[NST * G::STAGE];
    __shared__ __attribute__((aligned(16))) int32_t pt[VALID ? 4 : SEG_PAGES];

    // XCD-aware order: hardware ids go round-robin over the 8 XCDs, so logical
    // work ids are handed out in contiguous runs per XCD, keeping the row tiles
    // of one (sequence, kv head) -- which read the same K/V -- on one L2.
    const int nwg_pad = (int)gridDim.x;
    const int lin = (int)(blockIdx.x % 8) * (nwg_pad / 8) + (int)(blockIdx.x / 8);
    if (lin >= p.total_wg) return;
    const int row_tile = lin % p.row_tiles;
    int rest = lin / p.row_tiles;
    const int split = rest % p.splits;
    rest /= p.splits;
    const int kvh = rest % p.hkv;
    const int b = rest / p.hkv;

    // bounds of sequence b (without cu_q / n_keys every sequence has nq_single
    // queries and nk_single keys, known before any load)
    const int32_t q_begin = p.cu_q ? p.cu_q[b] : b * p.nq_single;
    const int32_t nq = p.cu_q ? p.cu_q[b + 1] - q_begin : p.nq_single;
    const int32_t nk = p.n_keys ? p.n_keys[b] : p.nk_single;
    const int32_t rows = nq * p.G;
    const int32_t row0 = row_tile * ROWS_PER_WG;
    if (row0 >= rows) return;
    const int32_t qpos0 = p.q_pos0 ? p.q_pos0[b] : nk - nq;

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int lrow = lane & 31;
    const int lhi = lane >> 5;
    const int32_t my_row = row0 + wave * ROWS_PER_WAVE + lrow;
    const bool row_ok = my_row < rows;
    // a wave past the last row only helps stage tiles (and meets the barriers)
    const bool wave_live = __builtin_amdgcn_readfirstlane(row0 + wave * ROWS_PER_WAVE) < rows;
    const int32_t tok = row_ok ? my_row / p.G : 0;
    const int32_t head = kvh * p.G + (row_ok ? my_row % p.G : 0);
    const int32_t qpos = qpos0 + tok;

    const int32_t *valid_b = VALID ? p.valid + (int64_t)b * p.valid_stride : nullptr;
    const int32_t *bt_b = p.bt ? p.bt + (int64_t)b * p.bt_stride : nullptr;
    // Block-table window: every wave loads entries [0, WIN_PAGES) of the
    // sequence's row into registers (entry 64k + lane in win[k]) while the
    // sequence bounds are read.  The prologue takes its page ids from it by
    // lane reads -- no dependent load, LDS round trip or barrier before the
    // first copies -- and it becomes the LDS table the loop starts with.
    // (Entries past the sequence's keys need no mask: a page's copy size
    // comes from n_keys.)
    int32_t win[WIN_PAGES / 64];
    if constexpr (LD == LD_DMA) {
#pragma unroll
        for (int k = 0; k < WIN_PAGES / 64; ++k) {
            const int32_t pi = lane + k * 64;
            win[k] = bt_b && pi < p.bt_stride ? bt_b[pi] : -1;
        }
    }

    // Query fragment: B operand of S^T = K Q^T.  Lane l holds row l%32,
    // dims kk*16 + (l/32)*8 + [0, 8).
    bf16x8 qf[D / 16];
    auto load_q = [&]() {
        const int64_t qoff = (int64_t)(q_begin + tok) * p.q_stride + (int64_t)head * D + lhi * 8;
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
            u32x4 w = {0u, 0u, 0u, 0u};
            if (row_ok) {
                if (QF32) {
                    const float *qp = reinterpret_cast<const float *>(p.q) + qoff + kk * 16;
                    const f32x4 a = *reinterpret_cast<const f32x4 *>(qp);
                    const f32x4 c = *reinterpret_cast<const f32x4 *>(qp + 4);
                    w[0] = f32_to_bf16_bits(a[0]) | (f32_to_bf16_bits(a[1]) << 16);
                    w[1] = f32_to_bf16_bits(a[2]) | (f32_to_bf16_bits(a[3]) << 16);
                    w[2] = f32_to_bf16_bits(c[0]) | (f32_to_bf16_bits(c[1]) << 16);
                    w[3] = f32_to_bf16_bits(c[2]) | (f32_to_bf16_bits(c[3]) << 16);
                } else {
                    w = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const uint16_t *>(p.q) + qoff + kk * 16);
                }
            }
            qf[kk] = __builtin_bit_cast(bf16x8, w);
        }
    };
    // At D = 256 the accumulators (128) and the rest of the loop fill the 256
    // arch VGPRs; the read-only query fragment moves to AGPRs, which MFMA reads
    // directly.  (Done once the loads have landed, so the move does not wait.)
    auto pin_q = [&]() {
        if constexpr (D >= 256) {
#pragma unroll
            for (int kk = 0; kk < D / 16; ++kk) {
                u32x4 w = __builtin_bit_cast(u32x4, qf[kk]);
                asm volatile("" : "+a"(w));
                qf[kk] = __builtin_bit_cast(bf16x8, w);
            }
        }
    };

    // Key range of this workgroup: mask bounds, then this split's share.
    const int32_t last_row = min(row0 + ROWS_PER_WG, rows) - 1;
    const int32_t qp_min = qpos0 + row0 / p.G, qp_max = qpos0 + last_row / p.G;
    int32_t k_lo = 0, k_hi = nk;
    if (MASK == EMB_MASK_CHUNK) {
        k_hi = min(nk, (qp_max / p.chunk + 1) * p.chunk);
        if (p.window >= 0) k_lo = max(0, (qp_min / p.chunk - p.window) * p.chunk);
    }
    int32_t t_lo = k_lo / G::KT, t_hi = (max(k_hi, k_lo) + G::KT - 1) / G::KT;
    // splits of this sequence: with one (a short sequence of a ragged batch
    // under split_keys) the workgroup writes its output rows itself, and the
    // merge kernel skips the sequence
    const int32_t ns_seq = p.splits > 1 ? seq_splits(p, nk) : 1;
    if (p.splits > 1) {
        const int32_t ns = ns_seq;
        if (split >= ns) return;  // a short sequence of a ragged batch: fewer splits (uniform per workgroup)
        const int32_t nt = t_hi - t_lo;
        const int32_t per = (nt + ns - 1) / ns;
        const int32_t a = t_lo + split * per;
        t_hi = min(t_hi, a + per);
        t_lo = min(a, t_hi);
    }
    // Keys every row of the workgroup sees under a chunk mask (no per-key test needed there).
    int32_t full_lo = 0, full_hi = nk;
    if (MASK == EMB_MASK_CHUNK) {
        full_hi = min(nk, (qp_min / p.chunk + 1) * p.chunk);
        full_lo = p.window >= 0 ? max(0, (qp_max / p.chunk - p.window) * p.chunk) : 0;
    }

    f32x16 acc_o[D / 32];
#pragma unroll
    for (int i = 0; i < D / 32; ++i) acc_o[i] = f32x16{};
    float m_run = -INFINITY, l_run = 0.0f;

    const int32_t lim = min(nk, p.capacity);  // slots at or past the capacity are zero rows
    // pages this workgroup reads: up to its last tile, within the table row
    const int32_t p_end = min((min(lim, t_hi * G::KT) + 15) / 16, bt_b ? p.bt_stride : INT32_MAX);
    // LDS table segment [seg_p0, seg_p0 + seg_len) of page indices (the
    // register window, when there is one, starts at page 0)
    const bool windowed = LD == LD_DMA && bt_b != nullptr;
    int32_t seg_p0 = windowed ? 0 : t_lo * G::PAGES;
    int32_t seg_len = windowed ? WIN_PAGES : SEG_PAGES;

    // DMA staging: copies straight into a stage (the lane offsets are fixed).
    DmaPlan<D> dma;
    if constexpr (LD == LD_DMA) dma.init();
    const uint32_t smem_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t *)smem;
    // LDS table offset of tile tt's page ids, reloading the next segment when
    // tt leaves the current one (a uniform call with a barrier; every wave is
    // past its last read of the old segment: the previous tile ended with a
    // barrier).
    auto seg_index = [&](int32_t tt) {
        int32_t pi = tt * G::PAGES - seg_p0;
        if (pi + G::PAGES > seg_len) {
            seg_p0 = tt * G::PAGES;
            seg_len = SEG_PAGES;
            load_segment(bt_b, seg_p0, p_end, pt);
            __syncthreads();
            pi = 0;
        }
        return pi;
    };
    // Register paths: starts the loads of tile tt into l (a uniform call),
    // which l.store() writes into a stage.
    auto issue = [&](RegLoader<D, VALID> &l, int32_t tt) {
        if constexpr (LD == LD_VALID) {
            l.issue_valid(p, valid_b, bt_b, tt * G::KT, nk, kvh);
        } else {
            const int32_t pi = seg_index(tt);
            l.issue_direct(p, pt + pi, tt * G::KT, lim, kvh);
        }
    };

    // S^T = K Q^T of the tile in stage st: in block kb, lane holds keys
    // kb*32 + (r/4)*8 + lhi*4 + r%4 of row lrow.
    auto qk = [&](const uint16_t *st, f32x16(&s)[G::KB]) {
#pragma unroll
        for (int kb = 0; kb < G::KB; ++kb) {
            s[kb] = f32x16{};
#pragma unroll
            for (int kk = 0; kk < D / 16; ++kk) {
                const u32x4 kw = *reinterpret_cast<const u32x4 *>(&st[k_off<D>(kb * 32 + lrow, kk * 2 + lhi)]);
                s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kw), qf[kk], s[kb], 0, 0, 0);
            }
        }
    };

    // Mask of the tile starting at key k0 (raw score units).
    auto apply_mask = [&](f32x16(&sv)[G::KB], int32_t k0) {
        bool tile_full = k0 + G::KT <= nk;
        if (MASK == EMB_MASK_CHUNK) tile_full = tile_full && k0 >= full_lo && k0 + G::KT <= full_hi;
        if (MASK == EMB_MASK_TOKEN || MASK == EMB_MASK_ADD || MASK == EMB_MASK_BLOCKMAP) tile_full = false;
        if (!tile_full) {  // one uniform branch around the whole per-key mask
#pragma unroll
            for (int kb = 0; kb < G::KB; ++kb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float x = sv[kb][r];
                    const int32_t j = k0 + kb * 32 + (r >> 2) * 8 + lhi * 4 + (r & 3);
                    bool vis = row_ok && j < nk;
                    if (MASK == EMB_MASK_CHUNK) {
                        const int32_t qc = qpos / p.chunk, kc = j / p.chunk;
                        vis = vis && kc <= qc && (p.window < 0 || qc - kc <= p.window);
                    } else if (MASK == EMB_MASK_TOKEN) {
                        vis = vis && reinterpret_cast<const uint8_t *>(p.mask)[(int64_t)b * p.mask_b_stride +
                                                                              (int64_t)tok * p.mask_q_stride + j] != 0;
                    } else if (MASK == EMB_MASK_ADD) {
                        if (vis)
                            x += p.inv_scale * reinterpret_cast<const float *>(p.mask)[(int64_t)b * p.mask_b_stride +
                                                                                      (int64_t)tok * p.mask_q_stride + j];
                    } else if (MASK == EMB_MASK_BLOCKMAP) {
                        vis = vis && p.bmap[(int64_t)b * p.bmap_b_stride + (int64_t)(tok / p.bsize) * p.bmap_cols +
                                            j / p.bsize] != 0;
                        if (vis && p.mask)
                            vis = reinterpret_cast<const uint8_t *>(p.mask)[(int64_t)b * p.mask_b_stride +
                                                                            (int64_t)tok * p.mask_q_stride + j] != 0;
                    }
                    sv[kb][r] = vis ? x : -INFINITY;
                }
            }
        }
    };
    // Row max of a tile (both half-waves hold the row's max).
    auto tile_max = [&](const f32x16(&sv)[G::KB]) {
        float mt = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < G::KB; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sv[kb][r]);
        float a, c;
        half_pair(mt, a, c);
        return fmaxf(a, c);
    };

    // Prologue: the first NST-1 tiles staged, S of tile t_lo computed.
    RegLoader<D, VALID> ld;
    if constexpr (LD == LD_DMA) {
        // The first NST-1 tiles' copies go out first, their page ids read
        // straight from the table (uniform loads, no LDS round trip and no
        // barrier); then the query loads, which land while the copies stream
        // in.  The LDS table serves the loop (the barrier below publishes it).
        static_assert(WIN_PAGES == 128, "two window registers");
        // (all ids first: each copy is a compiler memory barrier)
        int32_t pid[NST - 1][G::PAGES];
#pragma unroll
        for (int i = 0; i < NST - 1; ++i)
#pragma unroll
            for (int pg = 0; pg < G::PAGES; ++pg) {
                const int32_t pi = (t_lo + i) * G::PAGES + pg;
                int32_t id = -1;
                if (pi < p_end) {
                    id = pi;  // identity table
                    if (windowed) {
                        const int32_t w0 = __builtin_amdgcn_readlane(win[0], pi & 63);
                        const int32_t w1 = __builtin_amdgcn_readlane(win[1], pi & 63);
                        id = pi < 64 ? w0 : pi < WIN_PAGES ? w1 : __builtin_amdgcn_readfirstlane(bt_b[pi]);
                    }
                }
                pid[i][pg] = id;
            }
        if (windowed) {
            if (wave < WIN_PAGES / 64) pt[wave * 64 + lane] = wave == 0 ? win[0] : win[1];
        } else if (t_lo < t_hi) {
            load_segment(bt_b, seg_p0, p_end, pt);
        }
#pragma unroll
        for (int i = 0; i < NST - 1; ++i)
            if (t_lo + i < t_hi) dma.issue_ids(p, pid[i], (t_lo + i) * G::KT, lim, kvh, smem_lds + i * (G::STAGE * 2));
        load_q();
    } else {
        load_q();
        if (t_lo < t_hi) {
            if (LD != LD_VALID) {
                load_segment(bt_b, seg_p0, p_end, pt);
                __syncthreads();
            }
            RegLoader<D, VALID> l1;
            issue(ld, t_lo);
            if (t_lo + 1 < t_hi) issue(l1, t_lo + 1);
            ld.store(smem);
            if (t_lo + 1 < t_hi) l1.store(smem + G::STAGE);
        }
    }
    // Every load issued so far (the query fragment included) has landed.
    // Without this the compiler, merging the path that skips the prologue,
    // treats the query registers as possibly in flight inside the loop and
    // waits for all outstanding loads -- the prefetch included -- before the
    // first MFMA of every tile.
    wait_vmcnt<0>();
    pin_q();
    __syncthreads();
    f32x16 s_cur[G::KB];
    if (wave_live) qk(smem, s_cur);
    float mt_cur = -INFINITY;  // row max of the current tile (masked)
    if (wave_live && t_lo < t_hi) {
        apply_mask(s_cur, t_lo * G::KT);
        mt_cur = tile_max(s_cur);
    }

    // Stage `cur` holds tile t, nx1 tile t+1, and stage nxl receives tile
    // t + NST - 1.  Past the end, the extra S and the stores work on stale
    // stage contents that nothing reads.
    //
    // One key tile, per wave: the lazy rescale check on the row max of tile t;
    // then the S MFMAs of tile t+1 with the softmax VALU work of tile t between
    // them; then the P.V MFMAs of tile t with, between them, the copies of
    // tile t+3 (DMA) and the mask and row max of tile t+1.  The order is fixed
    // step by step (sched_barrier): each step issues one MFMA and the LDS read
    // AHEAD steps later, so the MFMAs never wait out the LDS latency, and the
    // copies trickle into the address unit instead of stalling all waves at
    // once at the top of the tile.
    constexpr int KS = D / 16;                 // k-steps of one 32-key S block
    constexpr int NS = G::KB * KS;             // S MFMAs a tile
    constexpr int NPV = G::KB * 2 * (D / 32);  // P.V MFMAs a tile
    constexpr int EPM = G::KB * 16 / NS;       // score elements per step (both phases)
    static_assert(NPV * EPM == G::KB * 16 && 2 * DmaPlan<D>::PER_TILE <= NPV, "tile schedule");
    //
    // The loop runs NST tiles an iteration (tile t_lo + i sits in stage i %
    // NST), so every stage index is a compile-time constant: LDS addresses
    // take the stage as an immediate offset, and the scores of consecutive
    // tiles alternate between two register sets instead of being copied.
    for (int32_t t0 = t_lo; t0 < t_hi; t0 += NST) {
#pragma unroll
      for (int cur = 0; cur < NST; ++cur) {
        const int32_t t = t0 + cur;
        if (t >= t_hi) break;
        const int nx1 = cur + 1 == NST ? 0 : cur + 1;
        const int nxl = cur == 0 ? NST - 1 : cur - 1;  // receives tile t + NST - 1
        const bool more = t + NST - 1 < t_hi;
        typename DmaPlan<D>::Descs dsc;
        const uint32_t st_l = smem_lds + nxl * (G::STAGE * 2);
        if constexpr (LD == LD_DMA) {
            // Past the last tile the copies still run, through empty
            // descriptors: they write zeros into stage nxl, which no later
            // tile reads, and keep the schedule free of branches.
            if (more)
                dma.prepare(p, pt + seg_index(t + NST - 1), (t + NST - 1) * G::KT, lim, kvh, dsc);
            else
                dma.empty(dsc);
        } else {
            if (more) issue(ld, t + NST - 1);
        }

        if (wave_live) {
            // wave-uniform lazy rescale
            if (__builtin_amdgcn_ballot_w64(mt_cur > m_run + p.th_raw) != 0) {
                const float m_new = fmaxf(m_run, mt_cur);
                const float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m_run - m_new) * p.c_log2);
#pragma unroll
                for (int i = 0; i < D / 32; ++i) acc_o[i] *= alpha;
                l_run *= alpha;
                m_run = m_new;
            }

            const uint16_t *stk = smem + nx1 * G::STAGE;
            const uint16_t *stv = smem + cur * G::STAGE;
            auto read_k = [&](int i) {
                return *reinterpret_cast<const u32x4 *>(&stk[k_off<D>((i / KS) * 32 + lrow, (i % KS) * 2 + lhi)]);
            };
            auto read_v = [&](int i) {  // i = (kb*2 + pg) * (D/32) + dt
                return *reinterpret_cast<const u32x4 *>(
                    &stv[v_off<D>(i / (D / 32), (i % (D / 32)) * 32 + lrow, lhi)]);
            };
            f32x16 s_nxt[G::KB];
            const float neg_mc = m_run == -INFINITY ? 0.0f : -m_run * p.c_log2;
            f16x8 pf[G::KB][2];
            u32x4 kbuf[AHEAD];
#pragma unroll
            for (int i = 0; i < AHEAD; ++i) kbuf[i] = read_k(i);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < NS; ++i) {
                const int kb = i / KS, kk = i % KS;
                s_nxt[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kbuf[i % AHEAD]), qf[kk],
                                                                   kk == 0 ? f32x16{} : s_nxt[kb], 0, 0, 0);
                if (i + AHEAD < NS) kbuf[i % AHEAD] = read_k(i + AHEAD);
#pragma unroll
                for (int u = 0; u < EPM; ++u) {
                    const int el = i * EPM + u, eb = el / 16, r = el % 16;
                    const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[eb][r], p.c_log2, neg_mc));
                    pf[eb][r >> 3][r & 7] = (_Float16)e;
                    // row sum of exactly the f16 weights the P.V product uses
                    if (r & 1)
                        l_run = __builtin_amdgcn_fdot2(f16x2{pf[eb][r >> 3][(r & 7) - 1], pf[eb][r >> 3][r & 7]},
                                                       f16x2{(_Float16)1.0f, (_Float16)1.0f}, l_run, false);
                }
                // keep this step's softmax here: without a use, IR passes sink
                // the whole softmax below the S MFMAs (sched_barrier only binds
                // the machine scheduler)
                asm volatile("" : "+v"(l_run));
                __builtin_amdgcn_sched_barrier(0);
            }
            if (t + 1 < t_hi) apply_mask(s_nxt, (t + 1) * G::KT);
            float mt_nxt = -INFINITY;
            u32x4 vbuf[AHEAD];
#pragma unroll
            for (int i = 0; i < AHEAD; ++i) vbuf[i] = read_v(i);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < NPV; ++i) {
                const int kp = i / (D / 32), dt = i % (D / 32);
                acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, vbuf[i % AHEAD]),
                                                                  pf[kp >> 1][kp & 1], acc_o[dt], 0, 0, 0);
                if (i + AHEAD < NPV) vbuf[i % AHEAD] = read_v(i + AHEAD);
                if constexpr (LD == LD_DMA)
                    if ((i & 1) && (i >> 1) < DmaPlan<D>::PER_TILE) dma.copy(dsc, st_l, i >> 1);
#pragma unroll
                for (int u = 0; u < EPM; ++u) {
                    const int el = i * EPM + u;
                    mt_nxt = fmaxf(mt_nxt, s_nxt[el / 16][el % 16]);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            {
                float a, c;
                half_pair(mt_nxt, a, c);
                mt_cur = fmaxf(a, c);
            }
#pragma unroll
            for (int kb = 0; kb < G::KB; ++kb) s_cur[kb] = s_nxt[kb];
        } else if constexpr (LD == LD_DMA) {
#pragma unroll
            for (int n = 0; n < DmaPlan<D>::PER_TILE; ++n) dma.copy(dsc, st_l, n);
        }
        if constexpr (LD == LD_DMA) {
            // tile t+2 (needed by the next S) has landed; with four stages
            // tile t+3, issued this tile, may still fly; after the last tile
            // nothing may (the epilogue reuses the stages)
            if (t + 1 < t_hi)
                wait_vmcnt<(NST - 3) * DmaPlan<D>::PER_TILE>();
            else
                wait_vmcnt<0>();
        } else if (more) {
            ld.store(smem + nxl * G::STAGE);
        }
        __syncthreads();
      }
    }
    {
        float a, c;
        half_pair(l_run, a, c);
        l_run = a + c;
    }

    // Exactness.  V reaches the loop's P.V product as f16, which is exact
    // only for |v| in [2^-14, 65504]: a larger value turns the row into
    // inf/NaN, and when every visible value is far below 2^-14 the f16
    // subnormals lose the row's precision.  A wave any of whose rows ended
    // non-finite, or with a largest |O| below 2^-12 over a non-empty key set
    // (|O| <= max |v|, so all its weight sat on values the f16 path cannot
    // hold), recomputes its rows here from the bf16 pool: K and V read
    // straight into the MFMA operands, P in f32 split into two bf16 parts
    // (P_hi + P_lo carries 16 bits), P.V as two bf16 MFMAs.  No LDS, no
    // barrier: the other waves of the workgroup go on to the epilogue.
    if (wave_live) {
        float amax = 0.0f;
        bool fin = true;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                fin = fin && __builtin_isfinite(acc_o[dt][e]);
                amax = fmaxf(amax, fabsf(acc_o[dt][e]));
            }
        float a, c;
        half_pair(amax, a, c);
        amax = fmaxf(a, c);
        const bool bad = row_ok && l_run > 0.0f && (!fin || amax < EXACT_TINY * l_run);
        if (__builtin_amdgcn_ballot_w64(bad) != 0) {
            // the query fragment again (reloaded rather than kept live past the
            // loop, where it would cost the loop registers)
            load_q();
            pin_q();
#pragma unroll
            for (int i = 0; i < D / 32; ++i) acc_o[i] = f32x16{};
            float m_x = -INFINITY, l_x = 0.0f;
            // logical slot of key j (-1: a zero row), and its page
            auto slot_of = [&](int32_t j) {
                int32_t sl;
                if constexpr (VALID) {
                    sl = j < nk ? valid_b[j] : -1;
                    if (sl >= p.capacity) sl = -1;
                } else {
                    sl = j < lim ? j : -1;
                }
                if (sl >= 0 && bt_b && (sl >> 4) >= p.bt_stride) sl = -1;
                return sl;
            };
            auto page_row = [&](int32_t sl) -> int32_t {  // (page, kv head) index of slot sl, or -1
                if (sl < 0) return -1;
                const int32_t page = page_of(bt_b, sl);
                return page < 0 ? -1 : page * p.hkv + kvh;
            };
            for (int32_t t = t_lo; t < t_hi; ++t) {
                const int32_t k0 = t * G::KT;
                f32x16 sx[G::KB];
#pragma unroll
                for (int kb = 0; kb < G::KB; ++kb) {
                    const int32_t sl = slot_of(k0 + kb * 32 + lrow);
                    const int32_t pr = page_row(sl);
                    const uint16_t *krow = p.k_pool + ((int64_t)(pr < 0 ? 0 : pr) * 16 + (sl & 15)) * D + lhi * 8;
                    sx[kb] = f32x16{};
#pragma unroll
                    for (int kk = 0; kk < D / 16; ++kk) {
                        u32x4 w = {0u, 0u, 0u, 0u};
                        if (pr >= 0) w = *reinterpret_cast<const u32x4 *>(krow + kk * 16);
                        sx[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, w), qf[kk], sx[kb],
                                                                         0, 0, 0);
                    }
                }
                apply_mask(sx, k0);
                const float m_new = fmaxf(m_x, tile_max(sx));
                const float alpha = m_x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m_x - m_new) * p.c_log2);
#pragma unroll
                for (int i = 0; i < D / 32; ++i) acc_o[i] *= alpha;
                l_x *= alpha;
                m_x = m_new;
                const float neg = m_new == -INFINITY ? 0.0f : -m_new * p.c_log2;
#pragma unroll
                for (int kb = 0; kb < G::KB; ++kb) {
                    // k-step ks of the block: lane holds S elements 8ks..8ks+7,
                    // keys 16ks + (m/4)*8 + lhi*4 + m%4 (m = 0..7); V supplies
                    // the same keys for dim dt*32 + lrow.
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        u32x4 ph, pl;
#pragma unroll
                        for (int m = 0; m < 8; m += 2) {
                            uint32_t h[2], lo[2];
#pragma unroll
                            for (int u = 0; u < 2; ++u) {
                                const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sx[kb][ks * 8 + m + u], p.c_log2, neg));
                                l_x += pv;
                                h[u] = f32_to_bf16_bits(pv);
                                lo[u] = f32_to_bf16_bits(pv - bf16_to_f32(h[u]));
                            }
                            ph[m / 2] = h[0] | (h[1] << 16);
                            pl[m / 2] = lo[0] | (lo[1] << 16);
                        }
                        int32_t vs[8], vr[8];
#pragma unroll
                        for (int m = 0; m < 8; ++m) {
                            vs[m] = slot_of(k0 + kb * 32 + ks * 16 + (m >> 2) * 8 + lhi * 4 + (m & 3));
                            vr[m] = page_row(vs[m]);
                        }
#pragma unroll
                        for (int dt = 0; dt < D / 32; ++dt) {
                            const int d = dt * 32 + lrow;
                            u32x4 vw;
#pragma unroll
                            for (int m = 0; m < 8; m += 2) {
                                uint32_t e0 = 0u, e1 = 0u;
                                if (vr[m] >= 0) e0 = p.v_pool[((int64_t)vr[m] * D + d) * 16 + (vs[m] & 15)];
                                if (vr[m + 1] >= 0) e1 = p.v_pool[((int64_t)vr[m + 1] * D + d) * 16 + (vs[m + 1] & 15)];
                                vw[m / 2] = e0 | (e1 << 16);
                            }
                            acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                                __builtin_bit_cast(bf16x8, vw), __builtin_bit_cast(bf16x8, ph), acc_o[dt], 0, 0, 0);
                            acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                                __builtin_bit_cast(bf16x8, vw), __builtin_bit_cast(bf16x8, pl), acc_o[dt], 0, 0, 0);
                        }
                    }
                }
            }
            half_pair(l_x, a, c);
            l_run = a + c;
            m_run = m_x;
        }
    }

    const float sc = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    // Split partials: O / l in f16 with a per-row power-of-two scale 2^k that
    // puts the row's largest |O/l| in [2^14, 2^15) (O/l of a split is a
    // weighted mean of V rows, so f16 keeps 11 bits relative to the row's
    // largest element, whatever its magnitude; the merge reweights the splits
    // by l), and (m, l, k) per row.  Only the merge kernel reads them, so each
    // wave stores its 32-row block in the accumulator order: every store
    // instruction writes 512 contiguous bytes, with no staging through LDS.
    // (Rows past the end carry values nothing reads.)
    if (ns_seq > 1) {
        const int64_t unit_row0 = ((int64_t)(b * p.hkv + kvh) * p.splits + split) * ((int64_t)p.row_tiles * ROWS_PER_WG);
        // A power-of-two scale per half of the dims (dims [0, D/2) and
        // [D/2, D)), from that half's largest |O/l|: a half whose values are
        // far below the other's keeps its own 11 bits.
        constexpr int HB = D / 64;  // 32-dim blocks in a half
        float om[2] = {0.0f, 0.0f};
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int e = 0; e < 16; ++e) om[dt >= HB ? 1 : 0] = fmaxf(om[dt >= HB ? 1 : 0], fabsf(acc_o[dt][e]));
        int kh[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float a, c;
            half_pair(om[h], a, c);
            const float omax = fmaxf(a, c) * sc;
            int ex = 0;
            if (omax > 0.0f && __builtin_isfinite(omax)) frexpf(omax, &ex);
            kh[h] = omax > 0.0f ? min(max(ex - 15, -100), 100) : 0;  // omax * 2^-k in [2^14, 2^15)
        }
        if (row_ok && lhi == 0) {
            const int64_t rowi = unit_row0 + my_row;
            *reinterpret_cast<f32x4 *>(p.ws_ml + rowi * 4) =
                f32x4{m_run == -INFINITY ? -INFINITY : m_run * p.c_log2, l_run, (float)kh[0], (float)kh[1]};
        }
        if (wave_live) {
            const float scs[2] = {ldexpf(sc, -kh[0]), ldexpf(sc, -kh[1])};
            uint16_t *blk = p.ws_o + (unit_row0 + row0 + wave * ROWS_PER_WAVE) * D + lane * 4;
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
                const float f = scs[dt >= HB ? 1 : 0];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x4 v = {acc_o[dt][j * 4] * f, acc_o[dt][j * 4 + 1] * f, acc_o[dt][j * 4 + 2] * f,
                                     acc_o[dt][j * 4 + 3] * f};
                    *reinterpret_cast<u32x2 *>(blk + (dt * 4 + j) * 256) = f16x4_bits(v);
                }
            }
        }
        return;
    }
    // Output rows, the normalised O (f32).  Lane l holds dims dt*32 + j*8 +
    // (l/32)*4 + [0,4) of row l%32, so a direct 16-byte store touches 64 rows
    // (cache lines) per instruction.  Where the stages have room, each wave
    // instead writes its 32 rows x D block into LDS (16-byte chunk c of row r
    // at chunk c ^ (r & 31), which spreads the 32 rows of one write over the
    // banks) and stores whole rows: D*4 contiguous bytes per row, 1024/D rows
    // an instruction.
    constexpr int CHR = D / 4;  // 16-byte chunks in a row of D floats
    if constexpr (NST * G::STAGE * 2 >= WAVES * ROWS_PER_WAVE * D * 4) {
        // every wave is past its last stage read (the loop ended with a barrier)
        float *ob = reinterpret_cast<float *>(smem) + wave * (ROWS_PER_WAVE * D);
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = dt * 8 + j * 2 + lhi;
                const f32x4 v = {acc_o[dt][j * 4] * sc, acc_o[dt][j * 4 + 1] * sc, acc_o[dt][j * 4 + 2] * sc,
                                 acc_o[dt][j * 4 + 3] * sc};
                *reinterpret_cast<f32x4 *>(ob + lrow * D + ((c ^ (lrow & (CHR - 1) & 31)) << 2)) = v;
            }
        constexpr int RPI = 64 / CHR;  // rows per store instruction
        constexpr int NI = ROWS_PER_WAVE / RPI;
        const int sub = lane / CHR, c = lane % CHR;
        // all reads first (the accumulators are dead), then the stores back to back
        f32x4 rv[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int r = i * RPI + sub;
            rv[i] = *reinterpret_cast<const f32x4 *>(ob + r * D + ((c ^ (r & (CHR - 1) & 31)) << 2));
        }
        __builtin_amdgcn_sched_barrier(0);
        // lane r < 32 holds the destination (element offset) of row r of the
        // wave, -1 past the last row; a store takes its rows' offsets by lane
        // reads (scalar when one row fills the instruction)
        int64_t dst_off = -1;
        if (row_ok) dst_off = (int64_t)(q_begin + tok) * p.out_stride + (int64_t)head * D;
        const uint32_t off_lo = (uint32_t)dst_off, off_hi = (uint32_t)((uint64_t)dst_off >> 32);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            int64_t off;
            if constexpr (RPI == 1) {
                off = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane(off_hi, i) << 32) |
                                (uint32_t)__builtin_amdgcn_readlane(off_lo, i));
            } else {
                int64_t cand[RPI];
#pragma unroll
                for (int u = 0; u < RPI; ++u)
                    cand[u] = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane(off_hi, i * RPI + u) << 32) |
                                        (uint32_t)__builtin_amdgcn_readlane(off_lo, i * RPI + u));
                off = cand[0];
#pragma unroll
                for (int u = 1; u < RPI; ++u) off = sub == u ? cand[u] : off;
            }
            if (off < 0) continue;
            *reinterpret_cast<f32x4 *>(p.out + off + c * 4) = p.round_out ? round_bf16x4(rv[i]) : rv[i];
        }
    } else {
        if (!row_ok) return;
        const int64_t off = (int64_t)(q_begin + tok) * p.out_stride + (int64_t)head * D;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f32x4 v = {acc_o[dt][j * 4] * sc, acc_o[dt][j * 4 + 1] * sc, acc_o[dt][j * 4 + 2] * sc,
                                 acc_o[dt][j * 4 + 3] * sc};
                *reinterpret_cast<f32x4 *>(p.out + off + dt * 32 + j * 8 + lhi * 4) = p.round_out ? round_bf16x4(v) : v;
            }
    }
}

// Combines split partials (m in log2 units, O_s already divided by l_s):
// m = max m_s, w_s = l_s 2^(m_s - m), out = sum w_s O_s / sum w_s.  A wave
// takes NCH 8-dim chunks of a 32-row block, lane l of chunk c the four dims
// that lane l of the producing wave stored there (row l%32, dims c*8 +
// (l/32)*4 + [0,4)), so each split's partial of a chunk arrives as one
// contiguous 512-byte read.  Every load of the wave (all splits, all its
// chunks) is issued before any is used, and the grid is small enough that
// every wave is resident at once: the kernel costs about one memory latency.
template <int D, int MS, int NCH>
__global__ __launch_bounds__(256) void attn_merge_kernel(KParams p) {
    constexpr int NC = D / 8;      // 8-dim chunks of a row
    constexpr int NG = NC / NCH;   // chunk groups, one wave each
    static_assert(NC % NCH == 0, "chunk groups");
    const int32_t blocks_per_unit = p.row_tiles * (ROWS_PER_WG / 32);
    const int64_t total = (int64_t)p.batch * p.hkv * blocks_per_unit * NG * 64;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int lane = (int)(idx & 63);
        int64_t w = idx >> 6;
        const int cg = (int)(w % NG);
        w /= NG;
        const int32_t blk = (int32_t)(w % blocks_per_unit);
        w /= blocks_per_unit;
        const int kvh = (int)(w % p.hkv);
        const int b = (int)(w / p.hkv);
        const int32_t row = blk * 32 + (lane & 31);
        const int32_t q_begin = p.cu_q ? p.cu_q[b] : b * p.nq_single;
        const int32_t nq = p.cu_q ? p.cu_q[b + 1] - q_begin : p.nq_single;
        if (row >= nq * p.G) continue;
        const int64_t rows_per_unit = (int64_t)blocks_per_unit * 32;
        const int64_t unit0 = (int64_t)(b * p.hkv + kvh) * p.splits;
        const int32_t ns = seq_splits(p, p.n_keys ? p.n_keys[b] : p.nk_single);
        if (ns <= 1) continue;  // one split: the attention kernel wrote the rows itself
        float ms[MS], ls[MS];
        int ks[MS];
        u32x2 os[MS][NCH];
#pragma unroll
        for (int s = 0; s < MS; ++s) {
            ms[s] = -INFINITY;
            ls[s] = 0.0f;
            ks[s] = 0;
#pragma unroll
            for (int j = 0; j < NCH; ++j) os[s][j] = u32x2{0u, 0u};
            if (s < ns) {
                const int64_t u = (unit0 + s) * rows_per_unit;
                const f32x4 ml = *reinterpret_cast<const f32x4 *>(p.ws_ml + (u + row) * 4);
                ms[s] = ml[0];
                ls[s] = ml[1];
                ks[s] = (int)ml[2 + (cg * NCH * 8 >= D / 2 ? 1 : 0)];  // the scale of this chunk's half
                const uint16_t *src = p.ws_o + (u + blk * 32) * D + (cg * NCH * 64 + lane) * 4;
#pragma unroll
                for (int j = 0; j < NCH; ++j) os[s][j] = *reinterpret_cast<const u32x2 *>(src + j * 256);
            }
        }
        float m = -INFINITY;
#pragma unroll
        for (int s = 0; s < MS; ++s) m = fmaxf(m, ms[s]);
        float wgt[MS], l = 0.0f;
#pragma unroll
        for (int s = 0; s < MS; ++s) {
            wgt[s] = ms[s] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms[s] - m) * ls[s];
            l += wgt[s];
        }
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int s = 0; s < MS; ++s) wgt[s] = ldexpf(wgt[s], ks[s]);  // the partial's stored scale
        const int32_t tok = row / p.G;
        const int32_t head = kvh * p.G + row % p.G;
        float *dst = p.out + (int64_t)(q_begin + tok) * p.out_stride + (int64_t)head * D + cg * NCH * 8 + (lane >> 5) * 4;
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
            float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < MS; ++s)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    o[e] += wgt[s] * (float)__builtin_bit_cast(_Float16, (uint16_t)(os[s][j][e >> 1] >> ((e & 1) * 16)));
            const f32x4 r = {o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv};
            *reinterpret_cast<f32x4 *>(dst + j * 8) = p.round_out ? round_bf16x4(r) : r;
        }
    }
}


// ---- Attention with bf16 probabilities (SmolVLA's rounding) ----
//
// Reference: build_self_attn_layer and build_cross_attn_layer
// (models/smolvla.cpp:255-266, :309-318): kq = mul_mat(K, Q) in f32, attn =
// bf16_round(soft_max_ext(kq, mask, 1/sqrt(hd))), kqv = mul_mat(V, attn) -- the
// probabilities are normalised, then rounded to bf16, then multiplied with V.
// Normalised probabilities need the row's max and sum before any P.V term, so
// this path makes two passes over the keys, a wave per (query token, head) row:
//   pass 1: a lane per key computes s = (q . k) * scale (+ additive mask, or
//           -inf where hidden), keeping a per-lane running max and sum of
//           exp; one wave reduction gives the row's m and l;
//   pass 2: per 64 keys, a lane per key recomputes s and stores
//           p = bf16(exp(s - m) * (1/l)) in LDS; then the lanes, over dims,
//           accumulate p * v in f32 -- on the paged path 16 keys of a page per
//           32-byte V load.
// The query row is rounded to bf16 (as on the MFMA path) and broadcast from
// LDS.  K/V addressing, zero rows and masks are the main kernel's.  Not tuned:
// it serves the small SmolVLA shapes, where it is latency-bound.
template <int D, int MASK, bool VALID, bool QF32>
__global__ __launch_bounds__(256) void attn_pbf16_kernel(KParams p) {
    constexpr int E = D / 64;  // dims a lane accumulates
    __shared__ __attribute__((aligned(16))) float qs[4][D];
    __shared__ float ps[4][64];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + wave;
    const int64_t per_b = (int64_t)p.max_q * p.hq;
    const int32_t b = (int32_t)min(r / per_b, (int64_t)p.batch - 1);
    const int32_t qi = (int32_t)((r % per_b) / p.hq), h = (int32_t)(r % p.hq);
    const int32_t q_begin = p.cu_q ? p.cu_q[b] : b * p.nq_single;
    const int32_t nq = p.cu_q ? p.cu_q[b + 1] - q_begin : p.nq_single;
    const int32_t nk = p.n_keys ? p.n_keys[b] : p.nk_single;
    const bool live = r < (int64_t)p.batch * per_b && qi < nq;  // wave-uniform
    const int32_t tok = qi;
    const int32_t qpos = (p.q_pos0 ? p.q_pos0[b] : nk - nq) + tok;
    const int32_t kvh = h / p.G;
    const int32_t *valid_b = VALID ? p.valid + (int64_t)b * p.valid_stride : nullptr;
    const int32_t *bt_b = p.bt ? p.bt + (int64_t)b * p.bt_stride : nullptr;
    const int32_t lim = VALID ? p.capacity : min(p.capacity, p.bt ? p.bt_stride * 16 : p.capacity);

    for (int d = lane; d < D; d += 64) {
        float x = 0.0f;
        if (live) {
            const int64_t off = (int64_t)(q_begin + tok) * p.q_stride + (int64_t)h * D + d;
            x = QF32 ? bf16_to_f32(f32_to_bf16_bits(reinterpret_cast<const float *>(p.q)[off]))
                     : bf16_to_f32(reinterpret_cast<const uint16_t *>(p.q)[off]);
        }
        qs[wave][d] = x;
    }
    __syncthreads();

    // page of key j's slot, or -1 for a zero row
    auto key_page = [&](int32_t j, int32_t &t) -> int32_t {
        const int32_t sl = VALID ? valid_b[j] : j;
        t = sl & 15;
        if (sl < 0 || sl >= lim) return -1;
        return page_of(bt_b, sl);
    };
    // masked, scaled score of key j (-inf when hidden)
    auto score = [&](int32_t j) -> float {
        int32_t t;
        const int32_t pg = key_page(j, t);
        float dot = 0.0f;
        if (pg >= 0) {
            const uint16_t *kr = p.k_pool + (((int64_t)pg * p.hkv + kvh) * 16 + t) * D;
#pragma unroll 4
            for (int c = 0; c < D / 8; ++c) {
                const u32x4 w = *reinterpret_cast<const u32x4 *>(kr + c * 8);
                const f32x4 qa = *reinterpret_cast<const f32x4 *>(&qs[wave][c * 8]);
                const f32x4 qb = *reinterpret_cast<const f32x4 *>(&qs[wave][c * 8 + 4]);
                dot += qa[0] * bf16_to_f32(w[0] & 0xffffu) + qa[1] * bf16_to_f32(w[0] >> 16) +
                       qa[2] * bf16_to_f32(w[1] & 0xffffu) + qa[3] * bf16_to_f32(w[1] >> 16) +
                       qb[0] * bf16_to_f32(w[2] & 0xffffu) + qb[1] * bf16_to_f32(w[2] >> 16) +
                       qb[2] * bf16_to_f32(w[3] & 0xffffu) + qb[3] * bf16_to_f32(w[3] >> 16);
            }
        }
        float x = dot * p.scale;
        bool vis = true;
        if (MASK == EMB_MASK_CHUNK) {
            const int32_t qc = qpos / p.chunk, kc = j / p.chunk;
            vis = kc <= qc && (p.window < 0 || qc - kc <= p.window);
        } else if (MASK == EMB_MASK_TOKEN) {
            vis = reinterpret_cast<const uint8_t *>(p.mask)[(int64_t)b * p.mask_b_stride + (int64_t)tok * p.mask_q_stride +
                                                            j] != 0;
        } else if (MASK == EMB_MASK_ADD) {
            x += reinterpret_cast<const float *>(p.mask)[(int64_t)b * p.mask_b_stride + (int64_t)tok * p.mask_q_stride +
                                                         j];
        }
        return vis ? x : -INFINITY;
    };

    // pass 1: row max and sum of exp
    float m = -INFINITY, l = 0.0f;
    if (live) {
        for (int32_t j = lane; j < nk; j += 64) {
            const float x = score(j);
            if (x > m) {
                l = l * expf(m - x) + 1.0f;
                m = x;
            } else if (x > -INFINITY) {
                l += expf(x - m);
            }
        }
    }
    float mr = m;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mr = fmaxf(mr, __shfl_xor(mr, off, 64));
    float lr = mr > -INFINITY && m > -INFINITY ? l * expf(m - mr) : 0.0f;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) lr += __shfl_xor(lr, off, 64);
    const bool any = mr > -INFINITY;  // a row with no visible key stores zeros
    const float inv_l = any ? 1.0f / lr : 0.0f;

    // pass 2: P.V with P = bf16(exp(s - m) / l)
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = 0.0f;
    const int32_t kend = live && any ? nk : 0;
    for (int32_t j0 = 0; j0 < kend; j0 += 64) {
        const int32_t j = j0 + lane;
        float pj = 0.0f;
        if (j < nk) {
            const float x = score(j);
            pj = x > -INFINITY ? bf16_to_f32(f32_to_bf16_bits(expf(x - mr) * inv_l)) : 0.0f;
        }
        ps[wave][lane] = pj;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int n = min(64, nk - j0);
        if (!VALID) {
            // keys j0 .. j0+n-1 are slots j0.. : 16 keys of a page per V load
            for (int pg0 = 0; pg0 < n; pg0 += 16) {
                const int32_t sl = j0 + pg0;
                int32_t page = sl < lim ? page_of(bt_b, sl) : -1;
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const int d = lane + 64 * e;
                    u32x4 w0 = {0u, 0u, 0u, 0u}, w1 = w0;
                    if (page >= 0) {
                        const uint16_t *vr = p.v_pool + (((int64_t)page * p.hkv + kvh) * D + d) * 16;
                        w0 = *reinterpret_cast<const u32x4 *>(vr);
                        w1 = *reinterpret_cast<const u32x4 *>(vr + 8);
                    }
#pragma unroll
                    for (int t = 0; t < 16; ++t) {
                        if (pg0 + t >= n || sl + t >= lim) break;
                        const uint32_t wd = t < 8 ? w0[t >> 1] : w1[(t - 8) >> 1];
                        acc[e] += ps[wave][pg0 + t] * bf16_to_f32((t & 1) ? wd >> 16 : wd & 0xffffu);
                    }
                }
            }
        } else {
            for (int jj = 0; jj < n; ++jj) {
                int32_t t;
                const int32_t pg = key_page(j0 + jj, t);
                if (pg < 0) continue;
                const float pv = ps[wave][jj];
#pragma unroll
                for (int e = 0; e < E; ++e)
                    acc[e] += pv * bf16_to_f32(p.v_pool[(((int64_t)pg * p.hkv + kvh) * D + lane + 64 * e) * 16 + t]);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (!live) return;
    float *dst = p.out + (int64_t)(q_begin + tok) * p.out_stride + (int64_t)h * D;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const float o = acc[e];
        dst[lane + 64 * e] = p.round_out ? bf16_to_f32(f32_to_bf16_bits(o)) : o;
    }
}

template <int D, int MASK>
hipError_t launch_pbf16(const KParams &kp, bool valid, bool qf32, hipStream_t stream) {
    const int64_t rows = (int64_t)kp.batch * kp.max_q * kp.hq;
    const dim3 grid((unsigned)((rows + 3) / 4));
    if (valid && qf32)
        hipLaunchKernelGGL((attn_pbf16_kernel<D, MASK, true, true>), grid, dim3(256), 0, stream, kp);
    else if (valid)
        hipLaunchKernelGGL((attn_pbf16_kernel<D, MASK, true, false>), grid, dim3(256), 0, stream, kp);
    else if (qf32)
        hipLaunchKernelGGL((attn_pbf16_kernel<D, MASK, false, true>), grid, dim3(256), 0, stream, kp);
    else
        hipLaunchKernelGGL((attn_pbf16_kernel<D, MASK, false, false>), grid, dim3(256), 0, stream, kp);
    return hipGetLastError();
}

template <int D>
hipError_t dispatch_pbf16(const KParams &kp, int mask, bool valid, bool qf32, hipStream_t stream) {
    switch (mask) {
        case EMB_MASK_FULL: return launch_pbf16<D, EMB_MASK_FULL>(kp, valid, qf32, stream);
        case EMB_MASK_CHUNK: return launch_pbf16<D, EMB_MASK_CHUNK>(kp, valid, qf32, stream);
        case EMB_MASK_TOKEN: return launch_pbf16<D, EMB_MASK_TOKEN>(kp, valid, qf32, stream);
        default: return launch_pbf16<D, EMB_MASK_ADD>(kp, valid, qf32, stream);
    }
}

template <int D, int MASK, int LD, bool QF32>
hipError_t launch_kernel(const KParams &kp, hipStream_t stream) {
    const int grid = (kp.total_wg + 7) / 8 * 8;
    hipLaunchKernelGGL((paged_attn_kernel<D, MASK, LD, QF32>), dim3(grid), dim3(256), 0, stream, kp);
    return hipGetLastError();
}

template <int D, int MASK>
hipError_t dispatch_lq(const KParams &kp, int ld, bool qf32, hipStream_t stream) {
    switch (ld) {
        case LD_DMA:
            return qf32 ? launch_kernel<D, MASK, LD_DMA, true>(kp, stream) : launch_kernel<D, MASK, LD_DMA, false>(kp, stream);
        case LD_REG:
            return qf32 ? launch_kernel<D, MASK, LD_REG, true>(kp, stream) : launch_kernel<D, MASK, LD_REG, false>(kp, stream);
        default:
            return qf32 ? launch_kernel<D, MASK, LD_VALID, true>(kp, stream)
                        : launch_kernel<D, MASK, LD_VALID, false>(kp, stream);
    }
}

template <int D>
hipError_t dispatch_mask(const KParams &kp, int mask, int ld, bool qf32, hipStream_t stream) {
    switch (mask) {
        case EMB_MASK_FULL: return dispatch_lq<D, EMB_MASK_FULL>(kp, ld, qf32, stream);
        case EMB_MASK_CHUNK: return dispatch_lq<D, EMB_MASK_CHUNK>(kp, ld, qf32, stream);
        case EMB_MASK_TOKEN: return dispatch_lq<D, EMB_MASK_TOKEN>(kp, ld, qf32, stream);
        case EMB_MASK_ADD: return dispatch_lq<D, EMB_MASK_ADD>(kp, ld, qf32, stream);
        default: return dispatch_lq<D, EMB_MASK_BLOCKMAP>(kp, ld, qf32, stream);
    }
}

template <int D>
hipError_t launch_merge(const KParams &kp, hipStream_t stream) {
    // four chunks a wave up to 8 splits, fewer past that (registers)
    const int64_t rows = (int64_t)kp.batch * kp.hkv * kp.row_tiles * ROWS_PER_WG;
    auto grid = [&](int nch) {
        const int64_t g = (rows * (D / 8) / nch * 2 + 255) / 256;  // 64 lanes per 32 rows
        return dim3((unsigned)(g > 65536 ? 65536 : g));
    };
    if (kp.splits <= 4)
        hipLaunchKernelGGL((attn_merge_kernel<D, 4, 4>), grid(4), dim3(256), 0, stream, kp);
    else if (kp.splits <= 8)
        hipLaunchKernelGGL((attn_merge_kernel<D, 8, 4>), grid(4), dim3(256), 0, stream, kp);
    else if (kp.splits <= 16)
        hipLaunchKernelGGL((attn_merge_kernel<D, 16, 2>), grid(2), dim3(256), 0, stream, kp);
    else
        hipLaunchKernelGGL((attn_merge_kernel<D, 64, 1>), grid(1), dim3(256), 0, stream, kp);
    return hipGetLastError();
}

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

int run_attention(const emb_attn_args *a, int32_t nq_single, int32_t nk_single, hipStream_t stream) {
    EMB_CHECK_ARG(a, "null args");
    EMB_CHECK_ARG(a->q && a->out && a->k_pool && a->v_pool, "null q/out/pool");
    EMB_CHECK_ARG(a->batch > 0 && a->hq > 0 && a->hkv > 0 && a->hq % a->hkv == 0, "bad head counts");
    EMB_CHECK_ARG(a->head_dim == 64 || a->head_dim == 128 || a->head_dim == 256, "head_dim must be 64, 128 or 256");
    EMB_CHECK_ARG(a->max_q > 0, "max_q must be positive");
    EMB_CHECK_ARG((a->cu_q != nullptr) == (a->n_keys != nullptr), "cu_q and n_keys go together");
    if (!a->cu_q && nk_single == 0) {
        // uniform batch: max_q queries and n_keys_uniform keys per sequence
        EMB_CHECK_ARG(a->n_keys_uniform > 0, "n_keys_uniform must be positive when cu_q and n_keys are NULL");
        nq_single = a->max_q;
        nk_single = a->n_keys_uniform;
    }
    EMB_CHECK_ARG(a->capacity > 0, "capacity must be positive");
    EMB_CHECK_ARG(!a->valid_slots || a->valid_stride >= 0, "bad valid_stride");
    EMB_CHECK_ARG(!a->block_tables || a->bt_stride > 0, "bad bt_stride");
    EMB_CHECK_ARG(a->scale > 0.0f && std::isfinite(a->scale), "scale must be positive and finite");
    const int64_t esz = a->q_is_f32 ? 4 : 2;
    EMB_CHECK_ARG(a->q_stride >= (int64_t)a->hq * a->head_dim && (a->q_stride * esz) % 16 == 0,
                  "q_stride must cover a token and keep 16-byte alignment");
    EMB_CHECK_ARG(a->out_stride >= (int64_t)a->hq * a->head_dim && a->out_stride % 4 == 0, "bad out_stride");
    EMB_CHECK_ARG(aligned16(a->q) && aligned16(a->out) && aligned16(a->k_pool) && aligned16(a->v_pool) &&
                      aligned16(a->v16_pool),
                  "buffers must be 16-byte aligned");
    EMB_CHECK_ARG(a->mask_kind >= EMB_MASK_FULL && a->mask_kind <= EMB_MASK_BLOCKMAP, "unknown mask kind");
    if (a->mask_kind == EMB_MASK_CHUNK) EMB_CHECK_ARG(a->chunk > 0, "chunk must be positive");
    if (a->mask_kind == EMB_MASK_TOKEN || a->mask_kind == EMB_MASK_ADD) EMB_CHECK_ARG(a->mask, "mask pointer required");
    if (a->mask_kind == EMB_MASK_BLOCKMAP)
        EMB_CHECK_ARG(a->block_map && a->block_size > 0 && a->block_map_cols > 0, "block map required");
    const int splits = a->splits > 1 ? a->splits : 1;
    EMB_CHECK_ARG(splits <= 64, "splits must be <= 64");
    if (splits > 1) EMB_CHECK_ARG(a->workspace && aligned16(a->workspace), "split-K needs an aligned workspace");

    KParams kp{};
    kp.q = a->q;
    kp.out = a->out;
    kp.q_stride = a->q_stride;
    kp.out_stride = a->out_stride;
    kp.round_out = a->out_bf16_round != 0;
    kp.cu_q = a->cu_q;
    kp.n_keys = a->n_keys;
    kp.q_pos0 = a->q_pos0;
    kp.nq_single = nq_single;
    kp.nk_single = nk_single;
    kp.k_pool = (const uint16_t *)a->k_pool;
    kp.v_pool = (const uint16_t *)a->v_pool;
    kp.v16_pool = (const uint16_t *)a->v16_pool;
    kp.bt = a->block_tables;
    kp.bt_stride = a->bt_stride;
    kp.valid = a->valid_slots;
    kp.valid_stride = a->valid_stride;
    kp.capacity = a->capacity;
    kp.batch = a->batch;
    kp.hq = a->hq;
    kp.hkv = a->hkv;
    kp.G = a->hq / a->hkv;
    kp.row_tiles = (int32_t)(((int64_t)a->max_q * kp.G + ROWS_PER_WG - 1) / ROWS_PER_WG);
    kp.splits = splits;
    EMB_CHECK_ARG(a->split_keys >= 0, "split_keys must be >= 0");
    kp.split_keys = splits > 1 ? a->split_keys : 0;
    const int64_t total = (int64_t)a->batch * a->hkv * splits * kp.row_tiles;
    EMB_CHECK_ARG(total < INT_MAX / 2, "grid too large");
    kp.total_wg = (int32_t)total;
    kp.scale = a->scale;
    kp.max_q = a->max_q;
    kp.c_log2 = a->scale * LOG2E;
    kp.th_raw = RESCALE_TH / kp.c_log2;
    kp.inv_scale = 1.0f / a->scale;
    kp.chunk = a->chunk;
    kp.window = a->window;
    kp.mask = a->mask;
    kp.mask_q_stride = a->mask_q_stride;
    kp.mask_b_stride = a->mask_batch_stride;
    kp.bmap = a->block_map;
    kp.bsize = a->block_size;
    kp.bmap_cols = a->block_map_cols;
    kp.bmap_b_stride = a->block_map_batch_stride;
    if (splits > 1) {
        const int64_t rows_all = (int64_t)a->batch * a->hkv * splits * kp.row_tiles * ROWS_PER_WG;
        kp.ws_o = (uint16_t *)a->workspace;
        kp.ws_ml = reinterpret_cast<float *>(kp.ws_o + rows_all * a->head_dim);
    }
    const bool qf32 = a->q_is_f32 != 0;
    hipError_t e;
    EMB_CHECK_ARG(a->kernel >= EMB_ATTN_AUTO && a->kernel <= EMB_ATTN_KEY_SPLIT, "unknown kernel choice");
    const bool ks_ok = a->mask_kind == EMB_MASK_FULL && a->v16_pool && !a->valid_slots && !a->p_bf16 &&
                       (a->head_dim == 128 || a->head_dim == 256) && splits == 1 &&
                       (!a->block_tables || a->bt_stride <= KS_MAX_PAGES) &&
                       (int64_t)a->max_q * a->q_stride * esz < ((int64_t)1 << 31);  // 32-bit query offsets
    if (a->kernel == EMB_ATTN_KEY_SPLIT && !ks_ok)
        return emb::set_error(EMB_ERR_UNSUPPORTED,
                              "the key-split kernel takes the FULL mask, an f16 V shadow, no valid-slot list, "
                              "head_dim 128 or 256, no split-K, no p_bf16, at most %d block-table entries "
                              "and a query block under 2 GiB",
                              KS_MAX_PAGES);
    if (a->p_bf16) {
        EMB_CHECK_ARG(splits == 1, "p_bf16 runs unsplit (splits must be 0 or 1)");
        EMB_CHECK_ARG(a->mask_kind != EMB_MASK_BLOCKMAP, "p_bf16 takes no block map");
        EMB_CHECK_ARG((int64_t)a->batch * a->max_q * a->hq / 4 < INT_MAX, "grid too large");
        const bool valid = a->valid_slots != nullptr;
        switch (a->head_dim) {
            case 64: e = dispatch_pbf16<64>(kp, a->mask_kind, valid, qf32, stream); break;
            case 128: e = dispatch_pbf16<128>(kp, a->mask_kind, valid, qf32, stream); break;
            default: e = dispatch_pbf16<256>(kp, a->mask_kind, valid, qf32, stream); break;
        }
        if (e != hipSuccess) return emb::set_error(EMB_ERR_LAUNCH, "p_bf16 attention launch: %s", hipGetErrorString(e));
        return EMB_OK;
    }
    const int64_t rows_per_unit = (int64_t)a->max_q * kp.G;
    // Automatic choice: the key-split kernel reads every K/V tile once per 32
    // rows instead of once per 128, so it pays off only while the row tiles
    // would leave most of the GPU idle (at most half the CUs busy unsplit).
    bool ks_auto = false;
    if (ks_ok && a->kernel == EMB_ATTN_AUTO && rows_per_unit <= 512) {
        int dev = 0, n_cu = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
            ks_auto = 2 * (int64_t)a->batch * a->hkv * kp.row_tiles <= n_cu;
    }
    if (ks_ok && (a->kernel == EMB_ATTN_KEY_SPLIT || ks_auto)) {
        KsParams ks{};
        ks.q = kp.q;
        ks.out = kp.out;
        ks.q_stride = kp.q_stride;
        ks.out_stride = kp.out_stride;
        ks.round_out = kp.round_out;
        ks.cu_q = kp.cu_q;
        ks.n_keys = kp.n_keys;
        ks.nq_single = kp.nq_single;
        ks.nk_single = kp.nk_single;
        ks.k_pool = kp.k_pool;
        ks.v_pool = kp.v_pool;
        ks.v16_pool = kp.v16_pool;
        ks.bt = kp.bt;
        ks.bt_stride = kp.bt_stride;
        ks.capacity = kp.capacity;
        ks.hkv = kp.hkv;
        ks.G = kp.G;
        ks.row_blocks = (int32_t)((rows_per_unit + 31) / 32);
        const int64_t wgs = (int64_t)a->batch * a->hkv * ks.row_blocks;
        EMB_CHECK_ARG(wgs < INT_MAX / 2, "grid too large");
        ks.total_wg = (int32_t)wgs;
        ks.c_log2 = kp.c_log2;
        ks.th_raw = kp.th_raw;
        e = ks_launch(ks, a->head_dim, qf32, stream);
        if (e != hipSuccess) return emb::set_error(EMB_ERR_LAUNCH, "key-split attention launch: %s", hipGetErrorString(e));
        return EMB_OK;
    }
    const int ld = a->valid_slots ? LD_VALID : (a->v16_pool ? LD_DMA : LD_REG);
    switch (a->head_dim) {
        case 64: e = dispatch_mask<64>(kp, a->mask_kind, ld, qf32, stream); break;
        case 128: e = dispatch_mask<128>(kp, a->mask_kind, ld, qf32, stream); break;
        default: e = dispatch_mask<256>(kp, a->mask_kind, ld, qf32, stream); break;
    }
    if (e == hipSuccess && splits > 1) {
        switch (a->head_dim) {
            case 64: e = launch_merge<64>(kp, stream); break;
            case 128: e = launch_merge<128>(kp, stream); break;
            default: e = launch_merge<256>(kp, stream); break;
        }
    }
    if (e != hipSuccess) return emb::set_error(EMB_ERR_LAUNCH, "paged attention launch: %s", hipGetErrorString(e));
    return EMB_OK;
}

// Reference-named face: q/out f32 [seq][H][D], cache buffers hold the bf16
// identity-paged pool written by lingbot_runtime_kv_update_f32, MHA.
int runtime_kv_attn(const float *q, const float *cache_k, const float *cache_v, const int *valid_slots, float *out,
                    int seq_q, int seq_k, int n_heads, int head_dim, int capacity, float scale, hipStream_t stream) {
    EMB_CHECK_ARG(q && cache_k && cache_v && valid_slots && out, "null pointer");
    EMB_CHECK_ARG(seq_q > 0 && seq_k > 0 && n_heads > 0 && head_dim > 0, "non-positive size");
    emb_attn_args a{};
    a.q = q;
    a.q_is_f32 = 1;
    a.q_stride = (int64_t)n_heads * head_dim;
    a.out = out;
    a.out_stride = a.q_stride;
    a.k_pool = cache_k;
    a.v_pool = cache_v;
    a.valid_slots = valid_slots;
    a.valid_stride = 0;
    a.capacity = capacity;
    a.batch = 1;
    a.hq = a.hkv = n_heads;
    a.head_dim = head_dim;
    a.max_q = seq_q;
    a.scale = scale;
    a.mask_kind = EMB_MASK_FULL;
    return run_attention(&a, seq_q, seq_k, stream);
}

// Device address of `scratch` on the current device, looked up on the first
// call there (hipGetSymbolAddress with that device current) and kept.
std::mutex g_scratch_mu;
constexpr int MAX_DEVICES = 64;
void *g_scratch_ptr[MAX_DEVICES] = {};

int scratch_on_current_device(void **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return emb::set_error(EMB_ERR_LAUNCH, "hipGetDevice failed");
    if (dev < 0 || dev >= MAX_DEVICES) return emb::set_error(EMB_ERR_UNSUPPORTED, "device ordinal %d", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return emb::set_error(EMB_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return EMB_OK;
}

}  // namespace

extern "C" {

int emb_paged_attention_noalloc(const emb_attn_args *a, hipStream_t stream) {
    EMB_CHECK_ARG(a, "null args");
    EMB_CHECK_ARG(!a->workspace, "workspace must be NULL: the split-K partials go to the library's scratch");
    if (a->splits <= 1) return run_attention(a, 0, 0, stream);
    const size_t need = emb_attn_workspace_bytes(a->batch, a->max_q, a->hq, a->hkv, a->head_dim, a->splits);
    if (need > NOALLOC_SCRATCH_BYTES)
        return emb::set_error(EMB_ERR_CAPACITY,
                              "split-K partials of this call need %zu bytes; the no-allocation scratch holds %zu "
                              "(fewer splits, or emb_paged_attention with a workspace)",
                              need, NOALLOC_SCRATCH_BYTES);
    void *ptr = nullptr;
    const int rc = scratch_on_current_device(&ptr);
    if (rc) return rc;
    emb_attn_args b = *a;
    b.workspace = ptr;
    return run_attention(&b, 0, 0, stream);
}

size_t emb_attn_workspace_bytes(int32_t batch, int32_t max_q, int32_t hq, int32_t hkv, int32_t head_dim,
                                int32_t splits) {
    if (batch <= 0 || max_q <= 0 || hq <= 0 || hkv <= 0 || hq % hkv || head_dim <= 0 || splits <= 1) return 0;
    const int64_t row_tiles = ((int64_t)max_q * (hq / hkv) + ROWS_PER_WG - 1) / ROWS_PER_WG;
    const int64_t rows_all = (int64_t)batch * hkv * splits * row_tiles * ROWS_PER_WG;
    return (size_t)rows_all * ((size_t)head_dim * sizeof(uint16_t) + 4 * sizeof(float));
}

int emb_paged_attention(const emb_attn_args *a, hipStream_t stream) {
    EMB_CHECK_ARG(a, "null args");
    return run_attention(a, 0, 0, stream);
}

int lingbot_runtime_kv_attn_f32(const float *q, const float *cache_k, const float *cache_v, const int *valid_slots,
                                float *out, int seq_q, int seq_k, int n_heads, int head_dim, float scale,
                                hipStream_t stream) {
    return runtime_kv_attn(q, cache_k, cache_v, valid_slots, out, seq_q, seq_k, n_heads, head_dim, INT_MAX, scale,
                           stream);
}

int lingbot_runtime_kv_attn_online_f32(const float *q, const float *cache_k, const float *cache_v,
                                       const int *valid_slots, float *out, int seq_q, int seq_k, int n_heads,
                                       int head_dim, float scale, hipStream_t stream) {
    return runtime_kv_attn(q, cache_k, cache_v, valid_slots, out, seq_q, seq_k, n_heads, head_dim, INT_MAX, scale,
                           stream);
}

int lingbot_runtime_kv_attn_warp_f32(const float *q, const float *cache_k, const float *cache_v,
                                     const int *valid_slots, float *out, int seq_q, int seq_k, int n_heads,
                                     int head_dim, float scale, hipStream_t stream) {
    return runtime_kv_attn(q, cache_k, cache_v, valid_slots, out, seq_q, seq_k, n_heads, head_dim, INT_MAX, scale,
                           stream);
}

int lingbot_runtime_kv_attn_cublas_f32(const float *q, const float *cache_k, const float *cache_v,
                                       const int *valid_slots, float *out, int seq_q, int seq_k, int n_heads,
                                       int head_dim, int capacity, float scale, hipStream_t stream) {
    EMB_CHECK_ARG(capacity > 0, "capacity must be positive");
    return runtime_kv_attn(q, cache_k, cache_v, valid_slots, out, seq_q, seq_k, n_heads, head_dim, capacity, scale,
                           stream);
}

}  // extern "C"
