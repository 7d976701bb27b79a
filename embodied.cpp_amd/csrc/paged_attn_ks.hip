// Key-split paged attention for gfx950 (MI355X): few query rows per
// (sequence, kv head), all keys visible.
//
// Same result contract as paged_attn_kernel with the FULL mask and the f16 V
// shadow (emb_kv.h): out[q, h] = sum_j softmax_j(scale * q.k_j) v_j over keys
// j < n_keys of the sequence, key j = logical slot j of the block table, keys
// at or past min(capacity, bt_stride*16) and keys in unmapped pages are zero
// K/V rows (score 0, zero value).  Reference semantics: the VLA experts'
// attention over the cached prefix (models/pi05.cpp:405-418) and the runtime
// KV attention (kernels/lingbot/lingbot_flex_attn_cuda.cu:651-720).
//
// Why a second kernel.  The row-tile kernel shares every staged K/V tile
// between 128 query rows.  A pi0.5 expert step has 408 rows (51 tokens x 8
// q-heads) per layer and kv head: four row tiles, the last a fifth full, and
// 72 workgroups for 18 layers -- so the keys have to be split over
// workgroups, with partials written out and merged by a second launch.  Here
// a workgroup owns one 32-row block and ALL its keys, and its four waves split
// the keys among themselves:
//   * wave w takes key tiles w, w+4, w+8, ... (32 keys each);
//   * each wave stages its own tiles: K rows are copied into two LDS stages
//     of the wave (buffer loads that write LDS, whole rows, 1 KB a copy), the
//     f16 V-shadow chunks are loaded straight into the P.V operand registers;
//     no barrier inside the key loop, the four waves of a CU run
//     independently;
//   * the four partial (O, m, l) merge through LDS at the end and the
//     workgroup writes its 32 output rows once.
// 18 x 13 = 234 workgroups for the pi0.5 step: no merge launch, no partials
// in HBM, 416 rows computed for 408 (the row-tile kernel computes 512).  The
// price: every CU streams a whole layer's K/V (888 KB at pi0.5 shape), 3.25x
// the row tiles' L2 -> CU traffic.  Measured on MI355X, one CU streams at most
// 70-90 GB/s and the L2s together 10-15 TB/s, so the key loop takes about as
// long as the streaming alone; the kernel wins while the row tiles would
// leave most CUs idle (the host's automatic choice, emb_kv.h).
//
// Per wave and key tile the MFMA math is the row-tile kernel's, transposed:
//   S^T[32 keys x 32 rows] = K . Q^T   (bf16 32x32x16, f32 accumulation)
//   O^T[D x 32 rows]      += V^T . P^T  (f16 32x32x16, P and V in f16)
// lane l owns query row l%32; the 16 scores a lane holds for a tile are keys
// (r/4)*8 + (l/32)*4 + r%4 (r = 0..15), so the row max is one lane swap.
//
// Operands:
//   K: fragment kk of the S product is row l%32, 16-byte chunk kk*2 + l/32
//      of the LDS stage (chunks XOR-swizzled by row: conflict-free reads).
//   V: the f16 shadow page holds each dim's 16 keys in the order the P.V
//      MFMA consumes them (emb_common.h v16_index), so the A operand of page
//      kp, dims dt*32 + [0,32), is one 16-byte read a lane: 1 KB contiguous
//      per instruction.
// Missing keys (past the limit, unmapped pages): K copies through a
// descriptor that ends at the page's last valid row read zeros; V reads from
// a zero block, and V of keys past the limit inside the last page is masked
// to zero; keys past n_keys are masked (score -inf).
//
// Pipeline per wave: while the S MFMAs of tile i+1 run, the softmax VALU work
// of tile i is interleaved between them; while the P.V MFMAs of tile i run,
// the mask and row max of tile i+1, the V loads of tile i+1 (each into the
// register its MFMA has just read) and the K copies of tile i+3 are.  K is
// two tiles ahead, V one.  Past the wave's last tile the loads read zeros
// and one extra S is computed and dropped: measured, this branch-free form
// is faster than a peeled last tile (25.9 vs 26.8 us at config 1).  The
// online softmax is the row-tile kernel's: running max in raw score units,
// accumulators rescaled only when a row's max grows by more than 2^8 (a
// wave-uniform branch most tiles skip).
//
// Exactness: as in the row-tile kernel, a workgroup any of whose waves ended
// with a non-finite partial, or a partial whose largest |O| is below 2^-12
// of its weight, recomputes all four partials from the bf16 pool (P split in
// two bf16 parts, bf16 V) before the merge.
#include <hip/hip_runtime.h>

#include <cmath>

#include "attn_dev.h"

namespace emb_attn {
namespace {

typedef __attribute__((address_space(1))) uint16_t gu16;  // global memory
typedef __attribute__((address_space(1))) u32x4 gu32x4;

constexpr int KS_WAVES = 4;
constexpr int KS_MAXD = 256;

// Zero K rows and V-shadow chunks: loads of missing keys read here.  A V
// source address is a lane offset below 16*D plus dt*512 elements.
__device__ __attribute__((aligned(16))) uint16_t ks_zero[16 * KS_MAXD];

template <int D, bool QF32>
__global__ __launch_bounds__(256, D >= 256 ? 1 : 2) void attn_ks_kernel(KsParams p) {
    constexpr int KS = D / 16;   // k-steps of S (one MFMA each)
    constexpr int DT = D / 32;   // 32-dim blocks of O^T
    constexpr int NV = 2 * DT;   // P.V MFMAs (and V operand chunks) per tile: two 16-key pages
    constexpr int EPM = 16 / KS; // score elements handled per S step
    constexpr int EPV = 16 / NV; // and per P.V step
    static_assert(D == 128 || D == 256, "head_dim 128 or 256");
    // K stages of the key loop, one LDS object each (see the fast path); after
    // the loop they hold the four waves' scaled partial O^T for the merge:
    // rows 0-15 of wave w in ks_k0[w], rows 16-31 in ks_k1[w], row r's 16-byte
    // chunk c at chunk c ^ (r & 31)
    __shared__ __attribute__((aligned(16))) uint16_t ks_k0[KS_WAVES][32 * D];
    __shared__ __attribute__((aligned(16))) uint16_t ks_k1[KS_WAVES][32 * D];
    __shared__ float mlb[KS_WAVES][32][2];
    __shared__ int32_t tbl[KS_MAX_PAGES];  // the sequence's block-table row
    // At head_dim 256 with bf16 Q the workgroup's 32 query rows are copied
    // into LDS once (1 KB copies of two whole rows, the K image's swizzle) and
    // every wave reads its fragments from there: one 16 KB stream instead of
    // four waves each loading the rows in 32-byte pieces.  (At head_dim 128
    // the buffer would cost the second workgroup per CU its LDS.)
    constexpr bool QLDS = D == 256 && !QF32;
    __shared__ __attribute__((aligned(16))) uint16_t ks_q[QLDS ? 32 * D : 8];

    const int nwg = (int)gridDim.x;
    // XCD-aware order: hardware ids go round-robin over the 8 XCDs; logical ids
    // are handed out in contiguous runs per XCD, so the row blocks of one
    // (sequence, kv head) -- which read the same K/V -- share one L2.
    const int lin = (int)(blockIdx.x % 8) * (nwg / 8) + (int)(blockIdx.x / 8);
    if (lin >= p.total_wg) return;
    const int rb = lin % p.row_blocks;
    const int rest = lin / p.row_blocks;
    const int kvh = rest % p.hkv;
    const int b = rest / p.hkv;

    // (bounds read through readfirstlane: they are uniform, and values the
    // compiler must treat as per-lane would turn the copies' buffer
    // descriptors into per-lane loops)
    const int32_t q_begin = __builtin_amdgcn_readfirstlane(p.cu_q ? p.cu_q[b] : b * p.nq_single);
    const int32_t nq = __builtin_amdgcn_readfirstlane(p.cu_q ? p.cu_q[b + 1] - q_begin : p.nq_single);
    const int32_t nk = __builtin_amdgcn_readfirstlane(p.n_keys ? p.n_keys[b] : p.nk_single);
    const int32_t rows = nq * p.G;
    const int32_t row0 = rb * 32;
    if (row0 >= rows) return;  // uniform over the workgroup

    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int lrow = lane & 31;
    const int lhi = lane >> 5;
    const int32_t my_row = row0 + lrow;
    const bool row_ok = my_row < rows;
    const int32_t tok = row_ok ? my_row / p.G : 0;
    const int32_t head = kvh * p.G + (row_ok ? my_row % p.G : 0);
    const int32_t *bt_b = p.bt ? p.bt + (int64_t)b * p.bt_stride : nullptr;
    // keys at or past lim are zero rows; past nk they do not exist
    int32_t lim = min(nk, p.capacity);
    if (bt_b) lim = min(lim, p.bt_stride * 16);
    const int32_t nt = (nk + 31) >> 5;

    // The block-table row goes into LDS at the start of the fast path (the
    // host admits at most KS_MAX_PAGES entries); the page id of page index pi
    // (wave-uniform) is then one broadcast LDS read, -1 for none.
    auto page_id = [&](int32_t pi) -> int32_t {
        if (!bt_b) return pi;
        const int32_t id = tbl[min(pi, KS_MAX_PAGES - 1)];  // read unconditionally, then selected (no branch)
        return __builtin_amdgcn_readfirstlane(pi < p.bt_stride ? id : -1);
    };
    // Page ids of key tile t's two pages (2t, 2t+1) and of tile u's, as one
    // 8-byte LDS read each and a single wait: straight-line code, so the
    // reads of both tiles are in flight together.
    const bool has_bt = bt_b != nullptr;
    auto page_ids2 = [&](int32_t t, int32_t u, int32_t &t0id, int32_t &t1id, int32_t &u0id, int32_t &u1id) {
        const i32x2 wt = *reinterpret_cast<const i32x2 *>(&tbl[min(2 * t, KS_MAX_PAGES - 2)]);
        const i32x2 wu = *reinterpret_cast<const i32x2 *>(&tbl[min(2 * u, KS_MAX_PAGES - 2)]);
        auto pick = [&](int32_t pi, int32_t id) {
            return __builtin_amdgcn_readfirstlane(has_bt ? (pi < p.bt_stride ? id : -1) : pi);
        };
        t0id = pick(2 * t, wt[0]);
        t1id = pick(2 * t + 1, wt[1]);
        u0id = pick(2 * u, wu[0]);
        u1id = pick(2 * u + 1, wu[1]);
    };
    // Uniform 64-bit address, its halves forced into SGPRs, as a global
    // (address space 1) pointer, so loads through it are global loads.
    auto uniform_ptr = [](const void *q) {
        const uint64_t a = reinterpret_cast<uint64_t>(q);
        return reinterpret_cast<const gu16 *>(
            ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) << 32) |
            (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a));
    };
    // Exact path: source of this lane's K operand for tile t (key t*32 + lrow,
    // dims lhi*8 + kk*16), read straight into registers.
    auto k_src = [&](int32_t t, int32_t pid0, int32_t pid1) -> const uint16_t * {
        const int32_t key = t * 32 + lrow;
        const int32_t pid = lrow < 16 ? pid0 : pid1;
        if (key < lim && pid >= 0) return p.k_pool + (((int64_t)pid * p.hkv + kvh) * 16 + (lrow & 15)) * D + lhi * 8;
        return ks_zero + lhi * 8;
    };
    // Source of this lane's V operand for page kp of tile t: dim dt*32 + lrow at + dt*512.
    const int vlane = lrow * 16 + ((lhi ^ ((lrow >> 3) & 1)) << 3);
    auto v_src = [&](int32_t t, int kp, int32_t pid) -> const uint16_t * {
        if (t * 32 + kp * 16 < lim && pid >= 0) return p.v16_pool + ((int64_t)pid * p.hkv + kvh) * (16 * D) + vlane;
        return ks_zero + vlane;
    };
    auto load_k = [&](u32x4(&kr)[KS], const uint16_t *src) {
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) kr[kk] = *reinterpret_cast<const u32x4 *>(src + kk * 16);
    };
    auto load_v = [&](u32x4(&vr)[NV], const uint16_t *s0, const uint16_t *s1) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            vr[dt] = *reinterpret_cast<const u32x4 *>(s0 + dt * 512);
            vr[DT + dt] = *reinterpret_cast<const u32x4 *>(s1 + dt * 512);
        }
    };
    // Keys at or past nk do not exist: score -inf.
    auto mask_tail = [&](f32x16 &s, int32_t t) {
        if (t * 32 + 32 > nk) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int32_t key = t * 32 + (r >> 2) * 8 + lhi * 4 + (r & 3);
                if (key >= nk) s[r] = -INFINITY;
            }
        }
    };
    auto tile_max = [&](const f32x16 &s) {
        float mt = s[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
        float a, c;
        half_pair(mt, a, c);
        return fmaxf(a, c);
    };

    // Query fragment (B operand of S^T): row lrow, dims kk*16 + lhi*8 + [0, 8).
    bf16x8 qf[KS];
    auto load_q = [&]() {
        const int64_t qoff = (int64_t)(q_begin + tok) * p.q_stride + (int64_t)head * D + lhi * 8;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
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
    auto qk = [&](const u32x4(&kr)[KS]) {
        f32x16 s = {};
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
            s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kr[kk]), qf[kk], s, 0, 0, 0);
        return s;
    };

    f32x16 acc[DT];
#pragma unroll
    for (int i = 0; i < DT; ++i) acc[i] = f32x16{};
    float m_run = -INFINITY, l_run = 0.0f;

    // ---- fast path: f16 P.V from the shadow ----
    {
        // K rows reach LDS by buffer loads that write it directly (whole
        // 16-byte chunks of two rows per 1 KB copy, XOR-swizzled so the
        // fragment reads below are bank-conflict free), in two stages per wave
        // that are separate LDS objects: the compiler then tracks each stage's
        // copies and waits for exactly the ones a read needs.  V goes into
        // registers: each V operand register is reloaded with the next tile's
        // V as soon as its P.V MFMA has read it.  Tile i of the wave (key tile
        // t0 + 4i) uses K stage i % 2.
        constexpr int CH = D / 8;     // 16-byte chunks of a K row
        constexpr int RB = 64 / CH;   // K rows per 1 KB copy
        constexpr int NKC = 32 / RB;  // copies per K tile
        constexpr int NKP = NKC / 2;  // copies per page
        static_assert(NKC <= NV, "one K copy per P.V step at most");
        constexpr int KAHEAD = 2;     // K fragment reads in flight ahead of their MFMA
        // byte offset in the page of this lane's chunk of copy j (the same for
        // both pages of a tile): row r = (j % NKP)*RB + lane/CH, slot lane%CH
        // holds chunk slot ^ (r & 15)
        auto koff = [&](int j) {
            const int r = (j % NKP) * RB + lane / CH;
            return (uint32_t)((r * D + (((lane % CH) ^ (r & 15)) << 3)) * 2);
        };
        struct KDesc {
            u32x4 r[2];
        };
        // descriptors of tile t's two pages: K rows below lim only (the rest,
        // and unmapped pages, read as zeros)
        auto k_desc = [&](int32_t t, int32_t pid0, int32_t pid1) {
            KDesc kd;
#pragma unroll
            for (int kp = 0; kp < 2; ++kp) {
                const int32_t pid = kp ? pid1 : pid0;
                const int32_t rows = pid < 0 ? 0 : min(max(lim - (t * 32 + kp * 16), 0), 16);
                const int64_t off = pid < 0 ? 0 : ((int64_t)pid * p.hkv + kvh) * (16 * D);
                kd.r[kp] = buf_desc(p.k_pool + off, (uint32_t)(rows * D * 2));
            }
            // VALU-written descriptor SGPRs read by a VMEM instruction: five
            // wait states, which the compiler does not count for asm operands
            asm volatile("s_nop 4");
            return kd;
        };
        // The copies are inline asm (lds_copy16), invisible to the compiler's
        // wait counting; the kernel waits for them itself (wait_vmcnt before
        // each S phase).  The compiler's own waits for the V loads may retire
        // copies issued after those loads earlier than needed, never later.
        auto k_copy = [&](const uint16_t *stage, const KDesc &kd, int j) {
            lds_copy16(kd.r[j / NKP],
                       (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t *)(stage + j * 512),
                       koff(j));
        };
        uint16_t *kst0 = ks_k0[wave];
        uint16_t *kst1 = ks_k1[wave];
        // fragment kk of S: row lrow, chunk kk*2 + lhi
        auto read_k = [&](const uint16_t *stage, int kk) {
            return *reinterpret_cast<const u32x4 *>(&stage[lrow * D + (((kk * 2 + lhi) ^ (lrow & 15)) << 3)]);
        };
        auto qk_lds = [&](const uint16_t *stage) {
            f32x16 s = {};
#pragma unroll
            for (int kk = 0; kk < KS; ++kk)
                s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, read_k(stage, kk)), qf[kk], s, 0,
                                                            0, 0);
            return s;
        };

        const int32_t t0 = wave;
        u32x4 vb[NV];
        if constexpr (QLDS) {
            // copy j (wave w issues j = w, w+4, ...): rows 2j, 2j+1 of the
            // block; rows past the sequence's queries fall outside the
            // descriptor and land as zeros
            const u32x4 qd = buf_desc(reinterpret_cast<const uint16_t *>(p.q) + (int64_t)q_begin * p.q_stride,
                                      (uint32_t)((int64_t)nq * p.q_stride * 2));
            asm volatile("s_nop 4");  // VALU-written descriptor SGPRs read by VMEM
            const uint32_t qlds = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t *)ks_q;
#pragma unroll
            for (int j = wave; j < 16; j += 4) {
                const int r = 2 * j + lhi;
                const int32_t row = row0 + r;
                const int32_t tk = row / p.G, hd = kvh * p.G + row % p.G;
                const int c = lrow ^ (r & 15);
                lds_copy16(qd, qlds + j * 1024, (uint32_t)(((int64_t)tk * p.q_stride + (int64_t)hd * D + c * 8) * 2));
            }
        } else {
            load_q();  // in flight while the table is read
        }
        if (bt_b)
            for (int i = threadIdx.x; i < p.bt_stride; i += 256) tbl[i] = bt_b[i];
        if constexpr (QLDS) wait_vmcnt<0>();  // the query copies (and the table loads) have landed
        if (QLDS || bt_b) __syncthreads();
        if constexpr (QLDS) {
#pragma unroll
            for (int kk = 0; kk < KS; ++kk)
                qf[kk] = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4 *>(&ks_q[lrow * D + (((kk * 2 + lhi) ^ (lrow & 15)) << 3)]));
        }
        {
            const int32_t t1 = t0 + 4;
            int32_t a0, a1, b0, b1;
            page_ids2(t0, t1, a0, a1, b0, b1);
            const KDesc ka = k_desc(t0, a0, a1);
#pragma unroll
            for (int j = 0; j < NKC; ++j) k_copy(kst0, ka, j);
            const KDesc kb = k_desc(t1, b0, b1);
#pragma unroll
            for (int j = 0; j < NKC; ++j) k_copy(kst1, kb, j);
            load_v(vb, v_src(t0, 0, a0), v_src(t0, 1, a1));
        }
        // The read-only query fragment lives in AGPRs (MFMA reads them
        // directly), leaving the arch VGPRs to the softmax and the V operands.
        if constexpr (D >= 256) {
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) {
                u32x4 w = __builtin_bit_cast(u32x4, qf[kk]);
                asm volatile("" : "+a"(w));
                qf[kk] = __builtin_bit_cast(bf16x8, w);
            }
        }
        // K of tile t0 has landed (after it: the copies of t0+4 and the V loads of t0)
        wait_vmcnt<NKC + NV>();
        f32x16 s_cur = qk_lds(kst0);
        {  // K of tile t0+8 into stage 0, which S of tile t0 has read
            const int32_t t2 = t0 + 8;
            const int32_t c0 = page_id(2 * t2), c1 = page_id(2 * t2 + 1);
            const KDesc kc = k_desc(t2, c0, c1);
#pragma unroll
            for (int j = 0; j < NKC; ++j) k_copy(kst0, kc, j);
        }
        mask_tail(s_cur, t0);
        float mt_cur = tile_max(s_cur);
        m_run = mt_cur;  // the first tile sets the running max (no rescale needed)

        // One tile t of the wave.  On entry: s_cur = S of tile t (masked),
        // mt_cur its row max; V of t in vb; K of t+4 in stage kn (in flight),
        // K of t+8 in the other stage (in flight).  The S MFMAs of tile t+4
        // run with the softmax of tile t between them; the P.V MFMAs of tile t
        // with the mask and row max of t+4, the V loads of t+4 (each into the
        // register its MFMA has just read) and the K copies of t+12 (into
        // stage kn, just read) between them.  Past the end the loads read
        // zeros: the extra S of the last tile is computed and dropped.  The
        // tile has no branch but the (rare) rescale: masks and zeroing are
        // selects, so no register is copied at a merge while a load into it
        // is in flight.
        // The zero block's address, opaque to the compiler so that it stays in
        // two SGPRs: otherwise it is reloaded from the GOT on every tile, a
        // scalar load and a wait in the middle of the loop.
        uint64_t zero_addr = reinterpret_cast<uint64_t>(ks_zero);
        asm volatile("" : "+s"(zero_addr));
        const uint16_t *zero_blk = reinterpret_cast<const uint16_t *>(zero_addr);
        auto tile = [&](int32_t t, int32_t tn, int32_t tc, uint16_t *kn) {
            // K of tile t+4 has landed: after its last copy (at the end of the
            // P.V phase two tiles back) the previous tile issued NV V loads and
            // NKC copies
            wait_vmcnt<NKC + NV>();
            u32x4 kbuf[KAHEAD];
#pragma unroll
            for (int i = 0; i < KAHEAD; ++i) kbuf[i] = read_k(kn, i);
            // page ids of tile tn (its V, loaded below) and tile tc (its K copies)
            int32_t n0, n1, c0, c1;
            page_ids2(tn, tc, n0, n1, c0, c1);
            if (__builtin_amdgcn_ballot_w64(mt_cur > m_run + p.th_raw) != 0) {
                const float m_new = fmaxf(m_run, mt_cur);
                const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * p.c_log2);
#pragma unroll
                for (int i = 0; i < DT; ++i) acc[i] *= alpha;
                l_run *= alpha;
                m_run = m_new;
            }
            const float neg_mc = m_run == -INFINITY ? 0.0f : -m_run * p.c_log2;
            f16x8 pf[2];
            f32x16 s_nxt = {};
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < KS; ++i) {
                s_nxt = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kbuf[i % KAHEAD]), qf[i],
                                                                s_nxt, 0, 0, 0);
                if (i + KAHEAD < KS) kbuf[i % KAHEAD] = read_k(kn, i + KAHEAD);
#pragma unroll
                for (int u = 0; u < EPM; ++u) {
                    const int r = i * EPM + u;
                    const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[r], p.c_log2, neg_mc));
                    pf[r >> 3][r & 7] = (_Float16)e;
                    // row sum of exactly the f16 weights the P.V product uses
                    if (r & 1)
                        l_run = __builtin_amdgcn_fdot2(f16x2{pf[r >> 3][(r & 7) - 1], pf[r >> 3][r & 7]},
                                                       f16x2{(_Float16)1.0f, (_Float16)1.0f}, l_run, false);
                }
                // keep this step's softmax here (IR passes would sink it below the MFMAs)
                asm volatile("" : "+v"(l_run));
                __builtin_amdgcn_sched_barrier(0);
            }
            // V elements of tile t at or past lim are zeroed (element e of the
            // chunk of page kp is key t*32 + kp*16 + (e/4)*8 + lhi*4 + e%4):
            // masks all-ones on every tile but the last
            const int32_t vrel = lim - t * 32 - lhi * 4;
            uint32_t keep[2][4];
#pragma unroll
            for (int kp = 0; kp < 2; ++kp)
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const int e0 = 2 * w, e1 = 2 * w + 1;
                    const int o0 = kp * 16 + (e0 >> 2) * 8 + (e0 & 3), o1 = kp * 16 + (e1 >> 2) * 8 + (e1 & 3);
                    keep[kp][w] = (o0 < vrel ? 0x0000ffffu : 0u) | (o1 < vrel ? 0xffff0000u : 0u);
                }
            const KDesc kc = k_desc(tc, c0, c1);
            const gu16 *vs0 = uniform_ptr(tn * 32 < lim && n0 >= 0
                                                  ? p.v16_pool + ((int64_t)n0 * p.hkv + kvh) * (16 * D)
                                                  : zero_blk) + vlane;
            const gu16 *vs1 = uniform_ptr(tn * 32 + 16 < lim && n1 >= 0
                                                  ? p.v16_pool + ((int64_t)n1 * p.hkv + kvh) * (16 * D)
                                                  : zero_blk) + vlane;
            // keys at or past nk do not exist: score -inf (selects; all kept
            // on every tile but the last)
            const int32_t srel = nk - tn * 32 - lhi * 4;
            float mt_nxt = -INFINITY;
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                u32x4 v = vb[i];
#pragma unroll
                for (int w = 0; w < 4; ++w) v[w] &= keep[i / DT][w];
                acc[i % DT] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, v), pf[i / DT],
                                                                     acc[i % DT], 0, 0, 0);
                // V of tile t+4, dims (i % DT)*32 of page i / DT
                vb[i] = *reinterpret_cast<const gu32x4 *>((i < DT ? vs0 : vs1) + (i % DT) * 512);
                if (i < NKC) k_copy(kn, kc, i);
#pragma unroll
                for (int u = 0; u < EPV; ++u) {
                    const int r = i * EPV + u;
                    const float x = ((r >> 2) * 8 + (r & 3)) < srel ? s_nxt[r] : -INFINITY;
                    s_nxt[r] = x;
                    mt_nxt = fmaxf(mt_nxt, x);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            float a, c;
            half_pair(mt_nxt, a, c);
            mt_cur = fmaxf(a, c);
            s_cur = s_nxt;
        };
        // Tiles alternate between the two K stages.  One tile per iteration:
        // the V registers stay the same registers across the back edge (an
        // unrolled pair of tiles let the allocator rename them, and the copies
        // at the back edge waited for loads still in flight).
        for (int32_t t = t0, i = 0; t < nt; t += 4, ++i) tile(t, t + 4, t + 12, (i & 1) ? kst0 : kst1);
    }

    // every copy into this wave's stages has landed (they become its merge buffer)
    wait_vmcnt<0>();

    // ---- merge of the four partials ----
    // Each wave publishes its rows' (m, l), then writes its partial O scaled
    // by its weight 2^(m_w - M) / L into its own stages, checking it on the
    // way: a partial that is non-finite, or whose largest |O| is below 2^-12
    // of its weight (all the weight on values the f16 path cannot hold
    // exactly), sends the workgroup to the exact path, which recomputes all
    // four partials from the bf16 pool and writes them again.
    auto row_part = [&](int w, int r) {  // row r of wave w's partial (its K stages, free after its loop)
        return reinterpret_cast<float *>(r < 16 ? ks_k0[w] : ks_k1[w]) + (r & 15) * D;
    };
    auto publish_and_write = [&]() {
        float a, c;
        half_pair(l_run, a, c);
        const float l_w = a + c;
        if (lhi == 0) {
            mlb[wave][lrow][0] = m_run;
            mlb[wave][lrow][1] = l_w;
        }
        __syncthreads();
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < KS_WAVES; ++w) M = fmaxf(M, mlb[w][lrow][0]);
        float L = 0.0f, own = 0.0f;
#pragma unroll
        for (int w = 0; w < KS_WAVES; ++w) {
            const float mw = mlb[w][lrow][0];
            const float sw = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((mw - M) * p.c_log2);
            L += mlb[w][lrow][1] * sw;
            if (w == wave) own = sw;
        }
        const float f = L > 0.0f ? own / L : 0.0f;
        float amax = 0.0f;
        bool fin = true;
        float *ob = row_part(wave, lrow);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f32x4 o = {acc[dt][j * 4], acc[dt][j * 4 + 1], acc[dt][j * 4 + 2], acc[dt][j * 4 + 3]};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    fin = fin && __builtin_isfinite(o[e]);
                    amax = fmaxf(amax, fabsf(o[e]));
                }
                const int cch = dt * 8 + j * 2 + lhi;  // chunk of dims dt*32 + j*8 + lhi*4 + [0,4)
                // a zero weight drops the partial (and any non-finite value in it)
                const f32x4 v = f == 0.0f ? f32x4{0.f, 0.f, 0.f, 0.f} : o * f;
                *reinterpret_cast<f32x4 *>(ob + ((cch ^ lrow) << 2)) = v;
            }
        half_pair(amax, a, c);
        amax = fmaxf(a, c);
        return row_ok && f > 0.0f && l_w > 0.0f && (!fin || amax < EXACT_TINY * l_w);
    };
    if (__syncthreads_or(publish_and_write())) {
        // ---- exact path: every wave recomputes its partial from the bf16 pool ----
        load_q();
#pragma unroll
        for (int i = 0; i < DT; ++i) acc[i] = f32x16{};
        float m_x = -INFINITY, l_x = 0.0f;
        for (int32_t t = wave; t < nt; t += 4) {
            const int32_t a0 = page_id(2 * t), a1 = page_id(2 * t + 1);
            u32x4 kr[KS];
            load_k(kr, k_src(t, a0, a1));
            f32x16 s = qk(kr);
            mask_tail(s, t);
            const float m_new = fmaxf(m_x, tile_max(s));
            const float alpha = m_x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m_x - m_new) * p.c_log2);
#pragma unroll
            for (int i = 0; i < DT; ++i) acc[i] *= alpha;
            l_x *= alpha;
            m_x = m_new;
            const float neg = m_new == -INFINITY ? 0.0f : -m_new * p.c_log2;
#pragma unroll
            for (int kp = 0; kp < 2; ++kp) {
                // P of the page's 8 keys of this lane (k-index e <-> key
                // kp*16 + (e/4)*8 + lhi*4 + e%4) as two bf16 parts
                u32x4 ph, pl;
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    uint32_t h[2], lo[2];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kp * 8 + e + u], p.c_log2, neg));
                        l_x += pv;
                        h[u] = f32_to_bf16_bits(pv);
                        lo[u] = f32_to_bf16_bits(pv - bf16_to_f32(h[u]));
                    }
                    ph[e / 2] = h[0] | (h[1] << 16);
                    pl[e / 2] = lo[0] | (lo[1] << 16);
                }
                const int32_t pid = kp ? a1 : a0;
                const int32_t kb = t * 32 + kp * 16;
                const bool page_ok = kb < lim && pid >= 0;
                // bf16 page rows: v_pool[((page*hkv + kvh)*D + d)*16 + key%16]
                const uint16_t *vp = page_ok ? p.v_pool + ((int64_t)pid * p.hkv + kvh) * (16 * D) : ks_zero;
                uint32_t keep[4];
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const int e0 = 2 * w, e1 = 2 * w + 1;
                    const int32_t k0 = kb + (e0 >> 2) * 8 + lhi * 4 + (e0 & 3);
                    const int32_t k1 = kb + (e1 >> 2) * 8 + lhi * 4 + (e1 & 3);
                    keep[w] = (page_ok && k0 < lim ? 0x0000ffffu : 0u) | (page_ok && k1 < lim ? 0xffff0000u : 0u);
                }
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    const uint16_t *row = vp + (dt * 32 + lrow) * 16 + lhi * 4;
                    const u32x2 lo4 = *reinterpret_cast<const u32x2 *>(row);
                    const u32x2 hi4 = *reinterpret_cast<const u32x2 *>(row + 8);
                    const u32x4 vw = {lo4[0] & keep[0], lo4[1] & keep[1], hi4[0] & keep[2], hi4[1] & keep[3]};
                    acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, vw),
                                                                      __builtin_bit_cast(bf16x8, ph), acc[dt], 0, 0, 0);
                    acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, vw),
                                                                      __builtin_bit_cast(bf16x8, pl), acc[dt], 0, 0, 0);
                }
            }
        }
        l_run = l_x;  // per-lane partial sums, as on the fast path
        m_run = m_x;
        // every wave is past its reads of the first write (the barrier
        // above); this barrier also orders the rewrite before the reads below
        __syncthreads_or(publish_and_write());
    }
    // (the barrier of the last __syncthreads_or orders every partial write
    // before the reads below)

    // Wave w stores rows w*8 .. w*8+7: a row is D/4 16-byte chunks, 64/(D/4)
    // rows per store instruction.
    constexpr int CHR = D / 4;
    constexpr int RPI = 64 / CHR;
    const int sub = lane / CHR, cc = lane % CHR;
#pragma unroll
    for (int i = 0; i < 8 / RPI; ++i) {
        const int r = wave * 8 + i * RPI + sub;
        const int32_t row = row0 + r;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < KS_WAVES; ++w) v += *reinterpret_cast<const f32x4 *>(row_part(w, r) + ((cc ^ r) << 2));
        if (row < rows) {
            const int32_t tk = row / p.G, hd = kvh * p.G + row % p.G;
            float *dst = p.out + (int64_t)(q_begin + tk) * p.out_stride + (int64_t)hd * D + cc * 4;
            *reinterpret_cast<f32x4 *>(dst) = p.round_out ? round_bf16x4(v) : v;
        }
    }
}

template <int D, bool QF32>
hipError_t launch(const KsParams &p, hipStream_t stream) {
    const int grid = (p.total_wg + 7) / 8 * 8;
    hipLaunchKernelGGL((attn_ks_kernel<D, QF32>), dim3(grid), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace

hipError_t ks_launch(const KsParams &p, int head_dim, bool q_f32, hipStream_t stream) {
    if (head_dim == 256) return q_f32 ? launch<256, true>(p, stream) : launch<256, false>(p, stream);
    return q_f32 ? launch<128, true>(p, stream) : launch<128, false>(p, stream);
}

}  // namespace emb_attn
