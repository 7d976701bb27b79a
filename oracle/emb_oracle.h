/*
 * emb_oracle.h -- CPU oracle for the KV-cached attention step.
 *
 * TEST INFRASTRUCTURE ONLY.  This library restates, in plain C, the
 * reference's semantics for the hot path (slot cache + eviction, paged
 * append/gather, flex masks and block tables, masked attention, Marlin W8
 * layout and W8A16 numerics).  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker.  The
 * product library (embodied.cpp_amd/libemb_kv.so) never links or calls it.
 *
 * Every function cites the reference file:line it follows (paths relative to
 * the reference repository root).  Where the reference leaves a choice open
 * (std::sort is not stable) the oracle states the rule it uses.
 */
#ifndef EMB_ORACLE_H
#define EMB_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- bf16 / random generation ---------------- */
float    orc_bf16_to_f32(uint16_t b);
uint16_t orc_f32_to_bf16(float f); /* round to nearest even, NaN kept quiet */

typedef struct { uint64_t mt[312]; int idx; } orc_mt64;
void     orc_mt64_seed(orc_mt64 *g, uint64_t seed);
uint64_t orc_mt64_next(orc_mt64 *g);
/* n bf16 values ~ N(0,1): Box-Muller on pairs of 53-bit uniforms, RNE to bf16 */
void     orc_fill_normal_bf16(uint64_t seed, int64_t n, uint16_t *out);
uint64_t orc_mt64_nth(uint64_t seed, int64_t n); /* n-th output (1-based) */

/* ---------------- slot cache (models/lingbot_va.cpp:8740-8997) ---------------- */
typedef struct {
    int64_t total;     /* capacity in token slots */
    int64_t *id;       /* insertion epoch, -1 = never/evicted */
    uint8_t *mask;     /* 1 = valid (visible) */
    uint8_t *is_pred;  /* 1 = prediction slot (mode 1) */
    int legacy_clear_pred;
} orc_slot_cache;

orc_slot_cache *orc_cache_new(int64_t total, int legacy_clear_pred);
void    orc_cache_free(orc_slot_cache *c);
int64_t orc_cache_used_count(const orc_slot_cache *c);
int64_t orc_cache_pred_count(const orc_slot_cache *c);
int64_t orc_cache_next_id(const orc_slot_cache *c);
int     orc_cache_allocate(orc_slot_cache *c, int64_t key_size, int64_t *slots);
int     orc_cache_update_meta(orc_slot_cache *c, int64_t key_size, int pred, int64_t *slots);
int     orc_cache_prepare_mode0(orc_slot_cache *c, int64_t key_size, int64_t *slots,
                                int64_t *valid, int64_t *n_valid);
void    orc_cache_restore(orc_slot_cache *c, const int64_t *slots, int64_t n);
void    orc_cache_clear_pred(orc_slot_cache *c);
int64_t orc_cache_collect_valid(const orc_slot_cache *c, int64_t *valid);
int64_t *orc_cache_id_ptr(orc_slot_cache *c);
uint8_t *orc_cache_mask_ptr(orc_slot_cache *c);
uint8_t *orc_cache_is_pred_ptr(orc_slot_cache *c);

int64_t orc_lingbot_capacity(int64_t override_tokens, int64_t frame_chunk_size,
                             int64_t action_per_frame, int64_t n_suffix, int64_t attn_window,
                             int64_t latent_h, int64_t latent_w, int64_t patch_t,
                             int64_t patch_h, int64_t patch_w, int64_t seq);

/* ---------------- token-slot cache data movement (kernels/lingbot/lingbot_flex_attn_cuda.cu) ---- */
void orc_slot_update(const uint16_t *k, const uint16_t *v, uint16_t *cache_k, uint16_t *cache_v,
                     const int32_t *slots, int64_t seq, int64_t heads, int64_t head_dim,
                     int64_t capacity);
void orc_slot_gather(const uint16_t *cache_k, const uint16_t *cache_v, const int32_t *valid,
                     uint16_t *out_k, uint16_t *out_v, int64_t seq_k, int64_t heads,
                     int64_t head_dim, int64_t capacity);

/* ---------------- paged pool movement (the build's page layout) ---------------- */
/* K page: [page][h][16][d]; V page: [page][h][d][16]; block_table NULL = identity. */
void orc_paged_append(const uint16_t *k, const uint16_t *v, int64_t src_stride, int64_t n,
                      int64_t heads, int64_t head_dim, const int32_t *slots,
                      const int32_t *block_table, int64_t capacity, uint16_t *k_pool,
                      uint16_t *v_pool);
void orc_paged_gather(const uint16_t *k_pool, const uint16_t *v_pool, const int32_t *valid,
                      int64_t n, int64_t heads, int64_t head_dim, const int32_t *block_table,
                      int64_t capacity, uint16_t *k_out, uint16_t *v_out);

/* ---------------- flex masks (models/lingbot_va.cpp:9274-9465) ---------------- */
typedef struct {
    int64_t n, n_text;
    int64_t *seq_ids, *frame_ids, *noise_ids, *text_seq_ids;
    int64_t window_size, block_size;
} orc_flex_meta;

orc_flex_meta *orc_flex_meta_build(int64_t lat_b, int64_t lat_f, int64_t lat_h, int64_t lat_w,
                                   int64_t act_b, int64_t act_f, int64_t act_h, int64_t act_w,
                                   int64_t padded_length, int64_t chunk_size, int64_t window_size,
                                   int64_t pt, int64_t ph, int64_t pw, int64_t text_seq,
                                   int64_t block_size);
void    orc_flex_meta_free(orc_flex_meta *m);
int     orc_flex_self_allowed(const orc_flex_meta *m, int64_t q, int64_t k);
int     orc_flex_cross_allowed(const orc_flex_meta *m, int64_t q, int64_t k);
/* CSR builders: return nnz; row_ptr must hold q_blocks+1, col_idx q_blocks*kv_blocks */
int64_t orc_dense_block_table(int64_t seq_q, int64_t seq_k, int64_t bs, int64_t *row_ptr,
                              int64_t *col_idx);
int64_t orc_self_block_table(const orc_flex_meta *m, int64_t *row_ptr, int64_t *col_idx);
int64_t orc_cross_block_table(const orc_flex_meta *m, int64_t *row_ptr, int64_t *col_idx);
void    orc_self_token_mask(const orc_flex_meta *m, uint8_t *mask);
int64_t orc_max_row_nnz(const int64_t *row_ptr, int64_t q_blocks);

/* ---------------- attention ---------------- */
void orc_dense_masked_attention(const float *q, const float *k, const float *v,
                                const uint8_t *mask, int64_t seq, int64_t heads,
                                int64_t head_dim, float *out);
void orc_flex_attention(const float *q, const float *k, const float *v, const int32_t *row_ptr,
                        const int32_t *col_idx, const uint8_t *token_mask, float *out,
                        int64_t seq_q, int64_t seq_k, int64_t heads, int64_t head_dim,
                        int64_t block_size, float scale);
void orc_runtime_kv_attn(const float *q, const float *cache_k, const float *cache_v,
                         const int32_t *valid, float *out, int64_t seq_q, int64_t seq_k,
                         int64_t heads, int64_t head_dim, float scale, int online_quirk);

/* GQA attention with ggml soft_max_ext / flash_attn_ext semantics.
 * q [n_q][hq][d], k/v [n_k][hkv][d] (bf16), out [n_q][hq][d] f32.
 * allow: optional u8 [n_q][n_k] (0 = -inf); add: optional f32 [n_q][n_k].
 * chunk > 0 adds a chunk-causal rule on positions (q_pos0 + i vs j).
 * rows: optional list of query token indices to evaluate (n_rows of them);
 * threads: OpenMP threads (<=0 = default). */
void orc_gqa_attention_bf16(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                            int64_t n_q, int64_t n_k, int64_t hq, int64_t hkv, int64_t d,
                            float scale, const uint8_t *allow, const float *add, int64_t chunk,
                            int64_t window, int64_t q_pos0, const int64_t *rows, int64_t n_rows,
                            int threads, float *out);

/* CPU baseline (bench.py cpu_baseline leg): f32 ggml op order, OpenMP threads.
 * Returns the number of threads used. */
int orc_cpu_attention_f32(const float *q, const float *k, const float *v, int64_t n_q, int64_t n_k,
                          int64_t hq, int64_t hkv, int64_t d, float scale, int threads, float *out);

/* ---------------- W8 Marlin (kernels/cosmos3/cosmos3_w8_marlin_cuda.cu:50-88) ---------------- */
int64_t orc_marlin_dst_byte(int64_t k, int64_t n, int64_t out_features);
int64_t orc_marlin_scale_index(int64_t n);
void    orc_marlin_pack_w8(const int8_t *w, int64_t K, int64_t N, int32_t *qweight);
int     orc_marlin_unpack_w8(const int32_t *qweight, int64_t K, int64_t N, int64_t k, int64_t n);
void    orc_marlin_pack_scales(const uint16_t *s_logical, int64_t N, uint16_t *s_stored);
/* y = bf16( sum_k x[m][k] * w[k][n] * s[n] ), fp32 accumulate; y_bf16 and y_f32 (pre-round) */
void    orc_w8a16_gemm(const uint16_t *x, const int32_t *qweight, const uint16_t *s_stored,
                       int64_t M, int64_t K, int64_t N, const int64_t *rows, int64_t n_rows,
                       int threads, uint16_t *y_bf16, float *y_f32);

/* ---------------- Qwen per-head q/k RMSNorm + RoPE (Cosmos3 language tower) ----------------
 * One part (Q or K) of a projection output x, bf16 [tokens][width] with
 * `heads` heads of head_dim d starting at column 0 of each row.
 *   norm  (kernels/cosmos3/cosmos3_qwen_language_cuda.cu:52-83), when gamma != NULL:
 *     inv = 1/sqrt(sum_d x^2 / d + eps); v = bf16(bf16(x * inv) * gamma)
 *   rope  (:85-116 simple, position first_pos + token; :117-153 MRoPE, position
 *     pos_ids[axis * tokens + token] with axis 1 / 2 for pair dims p < 60 with
 *     p % 3 == 1 / 2, else axis 0), when rope_kind != 0:
 *     p = d' mod (d/2), f = theta^(-2p/d), a = pos * f, s = bf16(sin a),
 *     c = bf16(cos a), y = bf16(v * c + r * s), r = -v[d' + d/2] below d/2,
 *     v[d' - d/2] above.
 * Output bf16 [tokens][heads][d] (row stride out_ld). */
void orc_head_norm_rope(const uint16_t *x, int64_t ld, int64_t tokens, int64_t heads, int64_t d,
                        const uint16_t *gamma, float eps, int rope_kind, float theta, int64_t first_pos,
                        const int32_t *pos_ids, uint16_t *out, int64_t out_ld);
/* pi0.5 NEOX RoPE in f32 (ggml_rope_ext at models/pi05.cpp:308-314,394-400):
 * x f32 [tokens][ld] (heads * d columns) -> out f32 [tokens][out_ld];
 * position of token t: pos[t], or first_pos + t when pos is NULL. */
void orc_neox_rope_f32(const float *x, int64_t ld, int64_t tokens, int64_t heads, int64_t d,
                       const int32_t *pos, int64_t first_pos, float freq_base, float *out, int64_t out_ld);

#ifdef __cplusplus
}
#endif
#endif
