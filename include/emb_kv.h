/*
 * emb_kv.h -- C ABI of the MI355X (gfx950) KV-cached attention step.
 *
 * One shared library, libemb_kv.so, built from embodied.cpp_amd/csrc/.
 * Conventions (same as the reference's kernel-level face,
 * kernels/lingbot/lingbot_flex_attn_cuda.h:9-105 and
 * kernels/cosmos3/cosmos3_w8_marlin_cuda.h:9-124):
 *   - every device entry point is asynchronous on the hipStream_t it takes;
 *   - it returns 0 on success and a negative code otherwise (-1 for bad
 *     arguments, checked on the host before any launch), and
 *     emb_last_error() returns a message for the calling thread;
 *   - all device buffers are owned by the caller; no entry point listed here
 *     allocates device memory unless its comment says so.
 *
 * Page layout of the KV pool (bf16, EMB_PAGE_TOKENS = 16 token slots a page):
 *   K page p, kv head h, slot row t, dim d : k_pool[((p*H + h)*16 + t)*D + d]
 *   V page p, kv head h, dim d, slot row t : v_pool[((p*H + h)*D + d)*16 + t]
 * A sequence's logical slot s lives in page block_table[s / 16], row s % 16;
 * block_table == NULL means the identity map (page = s / 16).
 *
 * Optional f16 V shadow (same page count and element count as v_pool): page
 * p, head h, dim d holds the 16 keys of the page as f16 in the order the
 * attention MFMA reads them,
 *   v16_pool[((p*H + h)*D + d)*16 + (((P(t) >> 3) ^ ((d >> 3) & 1)) << 3) + (P(t) & 7)]
 * where P(t) is row t with bits 2 and 3 swapped.  The append writes it when
 * given; attention given one copies its pages into LDS as they are.  The bf16
 * pool stays the bit-exact store (gather reads it).  A shadow must start
 * zero-filled (rows never appended are read, multiplied by zero weights).
 *
 * Value range.  Attention is exact for any finite bf16 V (the reference's
 * f32 range): its fast P.V product takes V as f16 (from the shadow, or
 * converted in registers), and a query row whose output comes out non-finite
 * (some visible |v| > 65504) or whose largest |out| is below 2^-12 over a
 * non-empty key set (its weight sits on values below f16's normal range) is
 * recomputed by the kernel from the bf16 pool with a bf16 P.V product (P kept
 * to 16 bits as two bf16 parts).  Split-K partials carry a per-row
 * power-of-two scale, so they hold any finite magnitude too.
 */
#ifndef EMB_KV_H
#define EMB_KV_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EMB_PAGE_TOKENS 16

enum {
    EMB_OK = 0,
    EMB_ERR_ARG = -1,        /* null pointer / bad size (reference convention) */
    EMB_ERR_LAUNCH = -2,     /* hipGetLastError after a launch */
    EMB_ERR_CAPACITY = -3,   /* slot cache / page pool could not satisfy a request */
    EMB_ERR_UNSUPPORTED = -4 /* shape outside what the kernels are built for */
};

const char *emb_last_error(void);
const char *emb_version(void);

/* ============================================================
 * Host-side slot cache: LingBotKVCache semantics
 * (models/lingbot_va.cpp:8740-8997), one per (model, session, layer, branch)
 * key (LingBotRuntimeKVKey, :9066-9089).  Logical slots are backed by pages of
 * a shared pool once a page pool is bound.
 * ============================================================ */
typedef struct emb_slot_cache emb_slot_cache;
typedef struct emb_page_pool emb_page_pool;

/* LingBotKVCache::init (:8751-8763) for batch 1; legacy_clear_pred plays the
 * VLA_LINGBOT_RUNTIME_KV_LEGACY_CLEAR_PRED flag (:153-155). */
emb_slot_cache *emb_slot_cache_create(int64_t capacity, int legacy_clear_pred);
void emb_slot_cache_destroy(emb_slot_cache *c);
int64_t emb_slot_cache_capacity(const emb_slot_cache *c);
int64_t emb_slot_cache_used_count(const emb_slot_cache *c);   /* :8774-8776 */
int64_t emb_slot_cache_pred_count(const emb_slot_cache *c);   /* :8778-8784 */
int64_t emb_slot_cache_next_id(const emb_slot_cache *c);      /* :8786-8792 */
/* allocate_slots_into (:8793-8831): returns 0 and fills slots[key_size]. */
int emb_slot_cache_allocate(emb_slot_cache *c, int64_t key_size, int64_t *slots);
/* update_meta_only (:8888-8902): cache modes 1 (pred) and 2 (update). */
int emb_slot_cache_update_meta(emb_slot_cache *c, int64_t key_size, int pred, int64_t *slots);
/* prepare_mode0_temp_slots_no_insert (:8904-8944): cache mode 0.
 * valid must hold capacity entries; *n_valid receives the count. */
int emb_slot_cache_prepare_mode0(emb_slot_cache *c, int64_t key_size, int64_t *slots,
                                 int64_t *valid, int64_t *n_valid);
void emb_slot_cache_restore(emb_slot_cache *c, const int64_t *slots, int64_t n); /* :8946-8952 */
void emb_slot_cache_clear_pred(emb_slot_cache *c);                                /* :8954-8965 */
int64_t emb_slot_cache_collect_valid(const emb_slot_cache *c, int64_t *valid);    /* :8967-8972 */
/* Snapshot of the per-slot metadata (each array has capacity entries). */
int emb_slot_cache_export(const emb_slot_cache *c, int64_t *id, uint8_t *mask, uint8_t *is_pred);

/* Page pool: host allocator of physical page ids in [0, n_pages).  seed == 0
 * hands pages out in ascending order, otherwise in a seeded random order. */
emb_page_pool *emb_page_pool_create(int32_t n_pages, uint64_t seed);
void emb_page_pool_destroy(emb_page_pool *p);
int32_t emb_page_pool_free_count(const emb_page_pool *p);
/* Bind a pool: every slot a later call hands out gets its page mapped. */
int emb_slot_cache_bind_pool(emb_slot_cache *c, emb_page_pool *p);
/* Map pages for logical slots [0, n_slots) now (e.g. for a prefix). */
int emb_slot_cache_map_range(emb_slot_cache *c, int64_t n_slots);
/* Block table of ceil(capacity/16) entries; unmapped pages are -1. */
int emb_slot_cache_block_table(const emb_slot_cache *c, int32_t *bt, int64_t n);
/* Return every mapped page to the pool (session reset). */
int emb_slot_cache_release_pages(emb_slot_cache *c);

/* lingbot_runtime_kv_capacity (:9217-9249) with the environment lookups made
 * arguments; override_tokens > 0 plays VLA_LINGBOT_KV_CACHE_TOKENS. */
int64_t emb_lingbot_kv_capacity(int64_t override_tokens, int64_t frame_chunk_size,
                                int64_t action_per_frame, int64_t n_suffix,
                                int64_t attn_window, int64_t latent_h, int64_t latent_w,
                                int64_t patch_t, int64_t patch_h, int64_t patch_w, int64_t seq);

/* Flex-mask metadata and block tables (models/lingbot_va.cpp:9274-9465). */
typedef struct emb_flex_meta emb_flex_meta;
emb_flex_meta *emb_flex_meta_build(int64_t lat_b, int64_t lat_f, int64_t lat_h, int64_t lat_w,
                                   int64_t act_b, int64_t act_f, int64_t act_h, int64_t act_w,
                                   int64_t padded_length, int64_t chunk_size,
                                   int64_t window_size, int64_t pt, int64_t ph, int64_t pw,
                                   int64_t text_seq, int64_t block_size);
void emb_flex_meta_destroy(emb_flex_meta *m);
int64_t emb_flex_meta_len(const emb_flex_meta *m);
int emb_flex_meta_ids(const emb_flex_meta *m, int64_t *seq_ids, int64_t *frame_ids,
                      int64_t *noise_ids);
int emb_flex_self_allowed(const emb_flex_meta *m, int64_t q, int64_t k);  /* :9330-9340 */
int emb_flex_cross_allowed(const emb_flex_meta *m, int64_t q, int64_t k); /* :9342-9344 */
/* CSR tables; row_ptr holds q_blocks+1 entries, col_idx q_blocks*kv_blocks.
 * Return nnz, or a negative error. */
int64_t emb_dense_block_table(int64_t seq_q, int64_t seq_k, int64_t block_size,
                              int32_t *row_ptr, int32_t *col_idx);             /* :9354-9372 */
int64_t emb_self_block_table(const emb_flex_meta *m, int32_t *row_ptr, int32_t *col_idx);
int64_t emb_cross_block_table(const emb_flex_meta *m, int32_t *row_ptr, int32_t *col_idx);
int emb_self_token_mask(const emb_flex_meta *m, uint8_t *mask);                /* :9456-9465 */

/* ============================================================
 * Call-site masks and positions (host): what the reference's model graphs
 * build before ggml's attention ops, as u8 "visible" masks for
 * EMB_MASK_TOKEN / f32 additive masks for EMB_MASK_ADD, and in the
 * reference's own additive form (0 / -inf) for emb_ggml_flash_attn_ext.
 * Row = query, column = key.
 * ============================================================ */
/* HY-VLA make_visual_patch_groups (models/hy_vla.cpp:1251-1277): runs of
 * nonzero modality flags, a single zero not ending a group; group_of[i] = the
 * group of token i or -1.  Returns the group count. */
int32_t emb_hy_patch_groups(const int32_t *modality_mask, int32_t n, int32_t *group_of);
/* HY-VLA make_prefix_mask (models/hy_vla.cpp:1279-1306) [n][n]: causal, but
 * among patch-group tokens a key is visible iff it is in the query's group
 * (bidirectional inside a group, cross-group pairs hidden); group_of NULL =
 * plain causal (:2131).  allow: u8 1 = visible; mask_f16: the reference's F16
 * bits (0x0000 / 0xFC00).  Either may be NULL. */
int emb_hy_prefix_mask(int64_t n, const int32_t *group_of, uint8_t *allow, uint16_t *mask_f16);
/* HY-VLA expert-with-prefix mask (models/hy_vla.cpp:2831-2843)
 * [n_suf][n_pref + n_suf]: all prefix keys; suffix row 0 (state) sees only
 * itself among the suffix, other rows the whole suffix. */
int emb_hy_suffix_mask(int64_t n_pref, int64_t n_suf, uint8_t *allow, uint16_t *mask_f16);
/* GR00T DiT (models/groot_n1.cpp:656-661): 0 = self-attention layer (no
 * mask), 1 = cross-attention with the text mask, 2 = with the image mask. */
int emb_groot_layer_mask_kind(int32_t layer, int32_t attend_text_every_n_blocks);
/* GR00T cross-attention masks (models/groot_n1.cpp:708-716), f32 additive
 * [n_q][n_keys]: text = valid and not image, image = valid and image.  Either
 * output may be NULL. */
int emb_groot_cross_masks(const int32_t *attention_mask, const int32_t *image_flags, int64_t n_keys, int64_t n_q,
                          float *text_mask, float *image_mask);
/* SmolVLA masks (models/smolvla.cpp:696-725), f32 additive; any may be NULL:
 * prefix [n_prefix][n_prefix] (invalid keys hidden; the last prefix token,
 * the state, hidden from the other queries), full [n_suf][n_prefix + n_suf]
 * (invalid prefix keys hidden, causal inside the suffix), cross
 * [n_suf][n_prefix] (invalid prefix keys hidden). */
int emb_smolvla_masks(const uint8_t *prefix_valid, int64_t n_prefix, int64_t n_suf, float *prefix_mask,
                      float *full_mask, float *cross_mask);
/* SmolVLA RoPE positions (models/smolvla.cpp:680-688): prefix i at
 * max(valid tokens in [0, i] - 1, 0), suffix i at (valid prefix tokens) + i,
 * cross-attention queries at i.  Any output may be NULL. */
int emb_smolvla_positions(const uint8_t *prefix_valid, int64_t n_prefix, int64_t n_suf, int32_t *prefix_pos,
                          int32_t *suffix_pos, int32_t *cross_pos);

/* ============================================================
 * Device data movement (bf16 pool)
 * ============================================================ */

/* Append n new token rows into the pool: runtime_kv_update (a9,
 * kernels/lingbot/lingbot_flex_attn_cuda.cu:626-649) made paged.
 * k_new/v_new: bf16 rows of n_kv_heads*head_dim elements, row stride src_stride
 * (elements).  slots: int32 [n] logical slots (device); a slot outside
 * [0, capacity) or on an unmapped page (-1) is skipped, as the reference skips
 * out-of-range slots.  v16_pool (may be NULL): the f16 V shadow, written too. */
int emb_kv_append(const void *k_new, const void *v_new, int64_t src_stride, int32_t n,
                  const int32_t *slots, const int32_t *block_table, int32_t capacity,
                  void *k_pool, void *v_pool, void *v16_pool, int32_t n_kv_heads,
                  int32_t head_dim, hipStream_t stream);

/* Gather rows valid[0..n) into compact [n][H][D] bf16 (reference layout):
 * runtime_kv_gather (a10, :875-898).  Out-of-range slots leave the row as is. */
int emb_kv_gather(const void *k_pool, const void *v_pool, const int32_t *valid, int32_t n,
                  const int32_t *block_table, int32_t capacity, void *k_out, void *v_out,
                  int32_t n_kv_heads, int32_t head_dim, hipStream_t stream);

/* ============================================================
 * Device-resident slot metadata: the same LingBotKVCache semantics as the
 * host cache above, kept in device memory and updated by kernels, so the
 * slots and the valid-slot list reach the append and the attention on the
 * stream with no host scan and no synchronous copy.  Replaces, per layer and
 * call, the host metadata update under the global runtime-KV mutex plus the
 * cudaMemcpy of slots and valid_slots in
 * run_lingbot_runtime_kv_device_attention (models/lingbot_va.cpp:9568-9650,
 * :9697-9767).  The arrays are caller-owned device memory of `capacity`
 * entries; emb_dev_cache_init sets every slot empty (id -1, mask 0, is_pred 0).
 * Eviction ties (equal ids) go in ascending slot order, as in the host cache.
 * Calls on one cache are stream-ordered; concurrent calls on one cache race.
 * ============================================================ */
typedef struct emb_dev_slot_cache {
    int64_t *id;          /* device [capacity]: insertion id, -1 = empty */
    uint8_t *mask;        /* device [capacity]: 1 = visible */
    uint8_t *is_pred;     /* device [capacity]: inserted in mode 1 */
    int32_t capacity;
    int32_t legacy_clear_pred; /* VLA_LINGBOT_RUNTIME_KV_LEGACY_CLEAR_PRED semantics */
} emb_dev_slot_cache;

int emb_dev_cache_init(const emb_dev_slot_cache *c, hipStream_t stream);
/* One runtime-KV metadata call with key_size new keys.  mode 1 / 2:
 * update_meta_only (:8887-8902) with pred = (mode == 1), then
 * collect_valid_slots (:8967-8972); mode 0: prepare_mode0_temp_slots_no_insert
 * (:8904-8944).  Device outputs: slots[key_size] (ascending), valid[capacity]
 * (may be NULL) and *n_valid (may be NULL), *status = 0, or EMB_ERR_CAPACITY
 * when even evicting every visible slot leaves fewer than key_size free, i.e.
 * key_size > capacity: the evictions stay, as in allocate_slots_into
 * (:8793-8831), slots[] is set to -1 and *n_valid to 0 (so an append and an
 * attention queued after it see no keys), and the call itself also returns
 * EMB_ERR_CAPACITY. */
int emb_dev_cache_update(const emb_dev_slot_cache *c, int32_t key_size, int32_t mode, int32_t *slots,
                         int32_t *valid, int32_t *n_valid, int32_t *status, hipStream_t stream);
int emb_dev_cache_restore(const emb_dev_slot_cache *c, const int32_t *slots, int32_t n,
                          hipStream_t stream);                                   /* :8946-8952 */
int emb_dev_cache_clear_pred(const emb_dev_slot_cache *c, hipStream_t stream);   /* :8954-8965 */

/* ============================================================
 * Per-head q/k RMSNorm + RoPE + paged append, one launch after the QKV
 * projection: replaces cosmos3_qwen_head_rmsnorm_f32 (Q and K),
 * cosmos3_qwen_rope_f32 / cosmos3_qwen_mrope_f32 (Q and K) and the cache
 * update (models/cosmos3.cpp:4967-5012; kernels/cosmos3/
 * cosmos3_qwen_language_cuda.h:21-52, .cu:52-153).
 * qkv: bf16 [tokens][ld], per row q_heads Q heads, then kv_heads K heads, then
 * kv_heads V heads, head_dim each (the layout emb_w8a16_gemm writes for a
 * concatenated [Wq | Wk | Wv]).  Q and K: RMSNorm over each head with bf16
 * gamma[head_dim] (NULL gamma: no norm), then RoPE: rope_kind 0 none, 1
 * position first_position + token, 2 MRoPE with position_ids [3][tokens]
 * (int32).  Q goes to q_out (bf16 [tokens][ldq]); K and V go into the paged
 * cache at slots[token] (same rules and layout as emb_kv_append, f16 V shadow
 * when v16_pool is given).  bf16 rounding points as the reference.
 * ============================================================ */
int emb_qkv_norm_rope_append(const void *qkv, int64_t ld, int32_t tokens, int32_t q_heads,
                             int32_t kv_heads, int32_t head_dim, const uint16_t *q_gamma,
                             const uint16_t *k_gamma, float eps, int32_t rope_kind, float rope_theta,
                             int32_t first_position, const int32_t *position_ids, void *q_out,
                             int64_t ldq, const int32_t *slots, const int32_t *block_table,
                             int32_t capacity, void *k_pool, void *v_pool, void *v16_pool,
                             hipStream_t stream);

/* LingBot form of the same step: full-row q/k RMSNorm (over all heads of the
 * row at once) and Wan RoPE from per-token tables, with the K/V append --
 * build_attention_shape's q/k/v path (models/lingbot_va.cpp:1219-1250;
 * apply_wan_rope_shape :1190-1206; lin() :1178-1180) on the f32 projection
 * output of the QKV graph (:11795-11875), ahead of
 * lingbot_runtime_kv_update_f32's append (lingbot_flex_attn_cuda.cu:626-649).
 * qkv: f32 [tokens][ld], columns [0, H*D) q, [H*D, 2H*D) k, [2H*D, 3H*D) v
 * (H = heads for q and k/v alike); qkv_bias f32 [3*H*D] or NULL, added first
 * (lin's bias).  q = rms_norm(q) * q_weight, k likewise (f32 [H*D] weights;
 * NULL skips that norm), scale = 1 / sqrt(sum(x^2) / (H*D) + eps).  RoPE:
 * rope_cos / rope_sin f32 [tokens][D/2] (both or neither); in each head pair
 * (2i, 2i+1) becomes (x0 c - x1 s, x1 c + x0 s) with c, s at [token][i].
 * Every step is an f32 operation of its own; Q goes to q_out bf16
 * [tokens][ldq], K and V bf16 into the cache at slots[token] (skip rules of
 * emb_kv_append), f16 V shadow if v16_pool.  Needs D % 8 == 0 and
 * H*D <= 8192; qkv, bias and weights 16-byte aligned, ld and ldq multiples
 * of 4. */
int emb_qkv_rownorm_rope_append(const float *qkv, int64_t ld, int32_t tokens, int32_t heads,
                                int32_t head_dim, const float *qkv_bias, const float *q_weight,
                                const float *k_weight, float eps, const float *rope_cos,
                                const float *rope_sin, void *q_out, int64_t ldq,
                                const int32_t *slots, const int32_t *block_table, int32_t capacity,
                                void *k_pool, void *v_pool, void *v16_pool, hipStream_t stream);

/* pi0.5 form: NEOX RoPE on the f32 Q and K projections and the K/V append, in
 * one launch -- replaces build_adarms_gemma_layer's (and build_gemma_layer's)
 * ggml_rope_ext(t, positions, NULL, head_dim, GGML_ROPE_TYPE_NEOX, 0,
 * freq_base, 1, 0, 1, 32, 1) on q and k and the ggml_concat of k_rope / v onto
 * the cached prefix (models/pi05.cpp:394-408, :308-325; suffix positions
 * n_prefix + i at :876-878, prefix positions i at :872-874).
 * q: f32 [tokens][ld_q] (q_heads heads of head_dim), k and v: f32
 * [tokens][ld_k] / [tokens][ld_v] (kv_heads heads) -- three mul_mat outputs,
 * or column ranges of one fused row.  Position of token i: positions[i]
 * (device int32 [tokens]) or, with positions NULL, first_position + i.
 * For pair i < head_dim/2 of a head, theta = pos * theta_scale^i with
 * theta_scale = freq_base^(-2/head_dim) (f32, ggml's rule), and
 * (x[i], x[i + head_dim/2]) -> (x0 cos - x1 sin, x0 sin + x1 cos) in f32.
 * Q goes to q_out [tokens][ldq], f32 (q_out_f32 nonzero) or bf16; K and V go
 * into the cache in bf16 at slots[token] (skip rules and layout of
 * emb_kv_append; f16 V shadow when v16_pool).  head_dim % 8 == 0; q, k, v 16-byte
 * aligned, ld_q / ld_k / ld_v / ldq multiples of 4. */
int emb_qkv_neox_rope_append(const float *q, int64_t ld_q, const float *k, int64_t ld_k, const float *v,
                             int64_t ld_v, int32_t tokens, int32_t q_heads, int32_t kv_heads,
                             int32_t head_dim, const int32_t *positions, int32_t first_position,
                             float freq_base, void *q_out, int32_t q_out_f32, int64_t ldq,
                             const int32_t *slots, const int32_t *block_table, int32_t capacity,
                             void *k_pool, void *v_pool, void *v16_pool, hipStream_t stream);

/* Reference-named Cosmos3 language-tower attention faces
 * (kernels/cosmos3/cosmos3_qwen_language_cuda.h:77-112, called from
 * models/cosmos3.cpp:5032,7889,8187): f32 q [tokens][hidden], k/v
 * [tokens][kv], GQA (query head h reads kv head h / (q_heads / kv_heads)),
 * scale 1/sqrt(head_dim), output f32 rounded to bf16 values.  causal: key j
 * visible to query i iff j <= i; gen_full: every generated token sees all
 * all_tokens keys.  head_dim <= 256.  The K/V staging of the two faces
 * without a workspace argument is a stream-ordered allocation of the call
 * (hipMallocAsync, released by hipFreeAsync on the same stream). */
int cosmos3_qwen_causal_gqa_attention_f32(const float *q, const float *k, const float *v, float *y,
                                          int tokens, int hidden, int kv, int q_heads, int kv_heads,
                                          int head_dim, hipStream_t stream);
int cosmos3_qwen_gen_full_gqa_attention_f32(const float *q_gen, const float *k_all, const float *v_all,
                                            float *y_gen, int gen_tokens, int all_tokens, int hidden,
                                            int kv, int q_heads, int kv_heads, int head_dim,
                                            hipStream_t stream);
/* The generated-token faces the MoT denoise calls (models/cosmos3.cpp:7889,
 * :8187; cosmos3_qwen_language_cuda.h:105-134), with caller workspaces sized
 * as the model sizes them (:7221-7227): scores_workspace gen_tokens *
 * all_tokens * (q_heads / kv_heads) floats, bf16_workspace gen_tokens *
 * hidden + 2 * all_tokens * kv halfwords.  The staged K/V go into one of them
 * when it is large enough (at the model's shapes both are), else into a
 * stream-ordered allocation of the call.  Same arithmetic and output as
 * cosmos3_qwen_gen_full_gqa_attention_f32; -1 for a null pointer or
 * inconsistent sizes. */
int cosmos3_qwen_gen_full_gqa_attention_workspace_f32(const float *q_gen, const float *k_all,
                                                      const float *v_all, float *y_gen,
                                                      float *scores_workspace, int gen_tokens,
                                                      int all_tokens, int hidden, int kv, int q_heads,
                                                      int kv_heads, int head_dim, hipStream_t stream);
int cosmos3_qwen_gen_full_gqa_attention_workspace_bf16tc_f32(
    const float *q_gen, const float *k_all, const float *v_all, float *y_gen, float *scores_workspace,
    unsigned short *bf16_workspace, int gen_tokens, int all_tokens, int hidden, int kv, int q_heads,
    int kv_heads, int head_dim, hipStream_t stream);

/* ============================================================
 * Paged block-masked attention (one launch for a batch of sequences)
 * ============================================================ */
enum {
    EMB_MASK_FULL = 0,    /* every key visible (pi0.5 prefix-LM from the suffix; prefill) */
    EMB_MASK_CHUNK = 1,   /* chunk-causal: key j visible to query position p iff
                             j/chunk <= p/chunk and p/chunk - j/chunk <= window
                             (window < 0: unlimited); chunk = 1 is causal */
    EMB_MASK_TOKEN = 2,   /* u8 [n_q][n_k] per sequence, 0 = hidden */
    EMB_MASK_ADD = 3,     /* f32 [n_q][n_k] per sequence added to scaled scores */
    EMB_MASK_BLOCKMAP = 4 /* u8 block map [q_blocks][k_blocks] (flex CSR) and an
                             optional u8 token mask */
};

typedef struct emb_attn_args {
    /* queries: bf16 (q_is_f32 == 0) or f32, [total_q tokens][hq][d] with token
     * stride q_stride elements; sequence b owns tokens cu_q[b]..cu_q[b+1]. */
    const void *q;
    int32_t q_is_f32;
    int64_t q_stride;
    /* output f32 [total_q][hq][d], token stride out_stride elements */
    float *out;
    int64_t out_stride;
    /* cu_q and n_keys are both given, or both NULL: then every sequence has
     * max_q query tokens (sequence b owns tokens b*max_q..) and
     * n_keys_uniform keys, and the kernels read no per-sequence bounds */
    const int32_t *cu_q;       /* device [batch+1] */
    const int32_t *n_keys;     /* device [batch]: keys per sequence */
    const int32_t *q_pos0;     /* device [batch] or NULL: position of query 0 in
                                  key index space (NULL: n_keys - n_q) */
    /* pool; v16_pool (may be NULL) is the f16 V shadow: when given (and no
     * valid-slot list), tiles are copied into LDS without conversion */
    const void *k_pool, *v_pool;
    const void *v16_pool;
    const int32_t *block_tables; /* device [batch][bt_stride] or NULL (identity); keys
                                    past bt_stride*16 read as zero rows */
    int32_t bt_stride;
    const int32_t *valid_slots;  /* device [batch][valid_stride] or NULL: key j is
                                    logical slot j; else key j is slot valid[j]
                                    (a negative entry is a zero K/V row, the
                                    online-kernel behaviour of :722-792) */
    int32_t valid_stride;
    int32_t capacity;            /* logical slots per sequence (bounds check) */
    int32_t batch, hq, hkv, head_dim;
    int32_t max_q;               /* max query tokens over the batch (host) */
    float scale;
    /* mask */
    int32_t mask_kind;
    int32_t chunk, window;             /* EMB_MASK_CHUNK */
    const void *mask;                  /* TOKEN: u8, ADD: f32 */
    int64_t mask_q_stride;             /* elements between query rows */
    int64_t mask_batch_stride;         /* elements between sequences */
    const uint8_t *block_map;          /* BLOCKMAP: [q_blocks][k_blocks] per sequence */
    int32_t block_size, block_map_cols;
    int64_t block_map_batch_stride;
    /* split-K over keys: 0/1 = none.  With splits > 1, workspace must hold
     * emb_attn_workspace_bytes(...) bytes of device memory: per row tile of
     * 128 rows and split, the partial O/l (f16, row-scaled by 2^k) and
     * (m, l, k, 0) as four floats. */
    int32_t splits;
    void *workspace;
    int32_t n_keys_uniform;            /* keys per sequence when cu_q and n_keys are NULL */
    int32_t out_bf16_round;            /* nonzero: every output value is stored rounded to
                                          bf16 precision (nearest even), still as f32 -- the
                                          Cosmos3 kernels' output rounding, done in the store */
    int32_t p_bf16;                    /* nonzero: the softmax probabilities are normalised and
                                          rounded to bf16 before P.V, f32 accumulation
                                          (SmolVLA's bf16_round(soft_max_ext(...)),
                                          models/smolvla.cpp:264-266, :317-318); a two-pass
                                          kernel, unsplit (splits 0 or 1), masks FULL, CHUNK,
                                          TOKEN or ADD; the f16 V shadow is not read */
    int32_t split_keys;                /* with splits > 1: 0 = every sequence takes `splits`
                                          splits; > 0 = a sequence of n keys takes
                                          min(splits, ceil(n / split_keys)) (at least 1), so
                                          short sequences of a ragged batch are not cut into
                                          splits that cost more than they save; a sequence
                                          left with one split writes its output directly
                                          (no partials, no merge work) */
    int32_t kernel;                    /* EMB_ATTN_AUTO (0), EMB_ATTN_ROW_TILES (1) or
                                          EMB_ATTN_KEY_SPLIT (2), below */
} emb_attn_args;

/* emb_attn_args.kernel.  Both kernels compute the same attention; they differ
 * in how the work is cut.
 *   ROW_TILES: a workgroup owns 128 query rows of one (sequence, kv head) and
 *     shares every K/V tile among them; every mask kind, the valid-slot list,
 *     register or shadow staging, split-K (register and shadow staging give
 *     the same output bit for bit).
 *   KEY_SPLIT: a workgroup owns 32 query rows and all their keys; its four
 *     waves split the keys and merge their partials in the kernel (no split-K
 *     workspace, no second launch).  FULL mask, f16 V shadow given, no
 *     valid-slot list, head_dim 128 or 256, splits 0 or 1, p_bf16 off,
 *     bt_stride <= 2048 (tables of up to 32768 keys); anything else returns
 *     EMB_ERR_UNSUPPORTED.  For few rows per kv head (the pi0.5 / GR00T /
 *     HY-VLA action experts: 51 tokens x 8 q-heads) over few sequences: it
 *     reads each K/V tile once per 32 rows (the row tiles once per 128), so
 *     it wins only while the row tiles would leave the GPU mostly idle.
 *   AUTO: KEY_SPLIT where it applies, max_q * (hq / hkv) <= 512 and the
 *     unsplit row tiles (batch * hkv * ceil(max_q * hq / hkv / 128)) would
 *     occupy at most half the device's compute units; else ROW_TILES.
 * The two kernels add the same terms in different orders, so their outputs
 * agree within rounding, not bit for bit. */
#define EMB_ATTN_AUTO 0
#define EMB_ATTN_ROW_TILES 1
#define EMB_ATTN_KEY_SPLIT 2

size_t emb_attn_workspace_bytes(int32_t batch, int32_t max_q, int32_t hq, int32_t hkv,
                                int32_t head_dim, int32_t splits);
int emb_paged_attention(const emb_attn_args *a, hipStream_t stream);
/* No counterpart in the reference: emb_paged_attention for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, except that workspace
 * must be NULL: the split-K partials go to a scratch array the library holds
 * on each device (48 MiB, for as long as the process runs; at most
 * emb_attn_workspace_bytes() of it per call: config 1's 18-layer launch at 3
 * splits takes 14.6 MB, config 3's layer at 4 splits 43.3 MB).  A call whose
 * partials need more returns EMB_ERR_CAPACITY before any launch.  Calls no
 * hipMalloc / hipFree; the first call on a device looks the scratch address
 * up.  Every call on one device shares the scratch (nothing in it must start
 * zeroed; each split writes its rows before the merge reads them), so calls
 * that overlap on one device -- several streams, or several threads -- race. */
int emb_paged_attention_noalloc(const emb_attn_args *a, hipStream_t stream);

/* ============================================================
 * Reference-named kernel-level face (same signatures as
 * kernels/lingbot/lingbot_flex_attn_cuda.h:13-105 with hipStream_t).
 * cache_k/cache_v are device buffers the caller sized for the reference's f32
 * cache (capacity*n_heads*head_dim floats); this library keeps them as a bf16
 * identity-paged pool inside that space, which needs capacity >= 8.  f32
 * inputs are rounded to bf16 (round to nearest even) on append.
 * ============================================================ */
int lingbot_runtime_kv_update_f32(const float *k, const float *v, float *cache_k, float *cache_v,
                                  const int *slots, int seq, int n_heads, int head_dim,
                                  int capacity, hipStream_t stream);
int lingbot_runtime_kv_gather_f32(const float *cache_k, const float *cache_v,
                                  const int *valid_slots, float *compact_k, float *compact_v,
                                  int seq_k, int n_heads, int head_dim, int capacity,
                                  hipStream_t stream);
int lingbot_runtime_kv_attn_f32(const float *q, const float *cache_k, const float *cache_v,
                                const int *valid_slots, float *out, int seq_q, int seq_k,
                                int n_heads, int head_dim, float scale, hipStream_t stream);
int lingbot_runtime_kv_attn_online_f32(const float *q, const float *cache_k,
                                       const float *cache_v, const int *valid_slots, float *out,
                                       int seq_q, int seq_k, int n_heads, int head_dim,
                                       float scale, hipStream_t stream);
int lingbot_runtime_kv_attn_warp_f32(const float *q, const float *cache_k, const float *cache_v,
                                     const int *valid_slots, float *out, int seq_q, int seq_k,
                                     int n_heads, int head_dim, float scale, hipStream_t stream);
/* Called at models/lingbot_va.cpp:9622 but defined nowhere in the reference. */
int lingbot_runtime_kv_attn_cublas_f32(const float *q, const float *cache_k,
                                       const float *cache_v, const int *valid_slots, float *out,
                                       int seq_q, int seq_k, int n_heads, int head_dim,
                                       int capacity, float scale, hipStream_t stream);

/* ============================================================
 * Whole-tensor faces: K/V given as tensors are staged by the library into an
 * identity-paged bf16 pool with its f16 V shadow, then attended with
 * emb_paged_attention.  Head sizes up to 256 other than 64/128/256 run padded
 * with zero dimensions (which change no score and no kept output).
 * ============================================================ */

/* Block-sparse attention, same signatures as
 * kernels/lingbot/lingbot_flex_attn_cuda.h:13-43 with hipStream_t: query q of
 * block qb = q / block_size sees the keys of the key blocks listed in
 * col_idx[row_ptr[qb] .. row_ptr[qb+1]) (device CSR), filtered by token_mask
 * (u8 [seq_q][seq_k], masked variant); out = softmax(scale q.k) v, 0 for a
 * row with no visible key.  q/k/v/out: f32 [seq][n_heads][head_dim], device.
 * A key block listed twice counts once (the reference would count it twice).
 * Q, K and V round to bf16 (fp32 accumulation; V of any finite magnitude: see
 * "Value range" above).  The K/V staging is a stream-ordered allocation of
 * the call (hipMallocAsync, released by hipFreeAsync on the same stream):
 * calls on different streams do not share memory. */
int lingbot_flex_attn_f32(const float *q, const float *k, const float *v, const int *row_ptr,
                          const int *col_idx, float *out, int seq_q, int seq_k, int n_heads,
                          int head_dim, int block_size, float scale, hipStream_t stream);
int lingbot_flex_attn_f32_masked(const float *q, const float *k, const float *v,
                                 const int *row_ptr, const int *col_idx,
                                 const unsigned char *token_mask, float *out, int seq_q,
                                 int seq_k, int n_heads, int head_dim, int block_size,
                                 float scale, hipStream_t stream);
/* The reference's in-source known-answer test (lingbot_flex_attn_cuda.cu:
 * 1010-1076): its 8-token, 2-head, head-size-8 inputs, causal window-4 mask
 * and CSR {0,1,3}/{0,0,1}, checked against a dense host loop.  Returns 0 when
 * the max abs difference is below 2e-2 (the reference's own bound is 1e-5
 * for its all-f32 kernel) and prints it.  Allocates its small device inputs. */
int lingbot_flex_attn_cuda_smoke(hipStream_t stream);

/* ggml tensor descriptor (the fields a ggml-hip backend forwards). */
enum { EMB_GGML_F32 = 0, EMB_GGML_F16 = 1, EMB_GGML_BF16 = 30 }; /* ggml_type values */
typedef struct emb_ggml_tensor {
    int32_t type;      /* EMB_GGML_F32 / F16 / BF16 */
    int64_t ne[4];     /* elements per dimension, ne[0] innermost */
    size_t nb[4];      /* byte strides */
    void *data;        /* device memory */
} emb_ggml_tensor;

/* ggml_flash_attn_ext(q, k, v, mask, scale, max_bias, logit_softcap) with
 * F32 precision, as the VLA experts call it (models/hy_vla.cpp:1066-1076;
 * the MUL_MAT -> SOFT_MAX_EXT -> MUL_MAT pattern of models/pi05.cpp:405-418
 * is the same computation with dst strides [D, n_q, H_q]):
 *   q [D, n_q, H_q, B], k/v [D, n_kv, H_kv, B or 1] (v not transposed),
 *   mask (may be NULL) additive [n_kv, >= n_q, 1, 1 or B], F16 or F32,
 *   dst F32 [D, H_q, n_q, B] at any strides,
 *   dst = softmax(scale * q.k + mask) v, q head h reading kv head
 *   h / (H_q / H_kv).  max_bias and logit_softcap must be 0 (-4 otherwise).
 * Q.K^T runs as bf16 MFMA: f32/f16 q and k round to bf16 (f16 v is kept
 * exactly for P.V), so the result is that of the reference on bf16-rounded q
 * and k, within the attention tolerance. 
 * workspace: device memory of emb_ggml_flash_attn_ext_workspace() bytes (16-
 * byte aligned); nothing is allocated.  The workspace query returns 0 for
 * descriptors the entry would reject. */
size_t emb_ggml_flash_attn_ext_workspace(const emb_ggml_tensor *q, const emb_ggml_tensor *k,
                                         const emb_ggml_tensor *v, const emb_ggml_tensor *mask,
                                         const emb_ggml_tensor *dst);
int emb_ggml_flash_attn_ext(const emb_ggml_tensor *q, const emb_ggml_tensor *k,
                            const emb_ggml_tensor *v, const emb_ggml_tensor *mask, float scale,
                            float max_bias, float logit_softcap, emb_ggml_tensor *dst,
                            void *workspace, size_t workspace_bytes, hipStream_t stream);

/* ============================================================
 * W8A16 linear (int8 weight-only, Marlin kU8B128 channelwise layout)
 * y[m][n] = bf16( (sum_k bf16(x[m][k]) * (u8[k][n] - 128)) * s[n] ), fp32
 * accumulate, the scale applied to the fp32 accumulator -- the numerics of
 * cosmos3_w8a16_linear_* over vllm Marlin
 * (kernels/cosmos3/cosmos3_w8_marlin_cuda.cu:302-501,651-765).
 * qweight: int32 [K/16][4N] in the layout of marlin_w8_dst_byte
 * (cosmos3_w8_marlin_cuda.cu:50-58, kernels/cosmos3/README.md:55-64);
 * scales: bf16 [N] in the order of marlin_scale_index (:79-88).
 * Needs K % 16 == 0 and N % 64 == 0 (else EMB_ERR_UNSUPPORTED).
 * ============================================================ */
enum {
    EMB_W8_Y_BF16 = 0,        /* y: bf16 [M][ldy] */
    EMB_W8_Y_F32_ROUNDED = 1, /* y: f32 [M][ldy] holding the bf16-rounded value
                                 (the reference's bf16 -> f32 widening, :407) */
    EMB_W8_Y_F32_RAW = 2      /* y: f32 [M][ldy], the fp32 epilogue value before
                                 the bf16 round (for numerics checks) */
};
/* x: bf16 (x_is_f32 == 0) or f32 (rounded to bf16 on load) [M][ldx]. */
int emb_w8a16_gemm(const void *x, int32_t x_is_f32, int64_t ldx, const int32_t *qweight,
                   const uint16_t *scales, int32_t M, int32_t K, int32_t N, void *y, int64_t ldy,
                   int32_t y_kind, hipStream_t stream);

/* The QKV projection that feeds the cache, with the append fused into its
 * epilogue (no reference counterpart as one call: models/cosmos3.cpp:4941-4943
 * makes three W8 calls and lingbot_runtime_kv_update_f32 then scatters K/V).
 * Output columns: [0, n_q) -> q_out bf16 [M][ldq]; the next
 * n_kv_heads*head_dim -> K and the last n_kv_heads*head_dim -> V, written as
 * bf16 into the pool pages of logical slot slots[m] (same skip rules as
 * emb_kv_append).  N = n_q + 2*n_kv_heads*head_dim. */
int emb_w8a16_qkv_append(const void *x, int32_t x_is_f32, int64_t ldx, const int32_t *qweight,
                         const uint16_t *scales, int32_t M, int32_t K, int32_t n_q, void *q_out,
                         int64_t ldq, const int32_t *slots, const int32_t *block_table,
                         int32_t capacity, void *k_pool, void *v_pool, void *v16_pool,
                         int32_t n_kv_heads, int32_t head_dim, hipStream_t stream);

/* The projection after attention with the block's gated residual update in
 * its epilogue: replaces lin(o, self_ctx) and x = x_in + a1 * gate_msa of the
 * LingBot post graph (models/lingbot_va.cpp:11693-11695; lin() :1178-1180;
 * gate_msa = timestep_proj chunk 2 + scale_shift chunk 2, :11679-11681), with
 * the O weights in the W8 layout above.
 *   out[m][n] = residual[m][n] + ((acc[m][n] * s[n]) + bias[n])
 *                                * (gate[m][n] + gate_bias[n])
 * acc as in emb_w8a16_gemm (fp32, not rounded to bf16).  Each operation is
 * rounded to f32 separately (no fused multiply-add), as the graph's add and
 * mul nodes are.  bias, gate_bias: f32 [N] or NULL (0); gate: f32 [M][ldg]
 * or NULL (no gate: a plain residual add, gate_bias must then be NULL);
 * residual f32 [M][ldr]; out f32 [M][ldo], which may be the residual itself
 * (in place, ldo == ldr) but must not otherwise overlap an input.
 * round_bf16 != 0 rounds out to bf16 precision (the graph's bf16 boundary,
 * :11676-11678).  x_bf16_workspace (bf16 [M][K], 16-byte aligned, or NULL):
 * with f32 x, x is rounded into it first and the GEMM reads it -- the same
 * values as without it, and faster (the in-kernel rounding stalls the k-tile
 * prefetch); ignored for bf16 x. */
int emb_w8a16_gated_residual(const void *x, int32_t x_is_f32, int64_t ldx, const int32_t *qweight,
                             const uint16_t *scales, int32_t M, int32_t K, int32_t N,
                             const float *bias, const float *gate, int64_t ldg,
                             const float *gate_bias, const float *residual, int64_t ldr, float *out,
                             int64_t ldo, int32_t round_bf16, void *x_bf16_workspace,
                             hipStream_t stream);

/* The same projection with the block's resident weights in ggml's dense
 * layouts (models/lingbot_va.cpp:1808-1851: F32 by default, BF16 by
 * VLA_LINGBOT_RESIDENT_BLOCK_DTYPE), replacing lin(o, self_ctx) =
 * ggml_add(ggml_mul_mat(W, x), bias) (:1178-1180) and the gated residual
 * (:11693-11695) with the product in the numerics of ggml's CUDA mul_mat:
 *   weight_type EMB_GGML_BF16: W bf16 [N][ldw]; x (f32, rounded to bf16, or
 *     bf16) times W with fp32 accumulation, the result rounded to bf16 and
 *     widened (the cuBLAS bf16 GEMM and its bf16 -> f32 conversion), then
 *     + bias; x_bf16_workspace as for emb_w8a16_gated_residual;
 *   weight_type EMB_GGML_F32: W f32 [N][ldw], x f32; an fp32 product (the
 *     reference's cublasSgemm), + bias; no workspace.
 *   out[m][n] = residual[m][n] + lin[m][n] * (gate[m][n] + gate_bias[n])
 * with each operation rounded to f32 separately.  residual NULL: out = lin *
 * (gate + gate_bias), or out = lin with no gate (the plain lin() of any
 * LingBot projection).  Other arguments as emb_w8a16_gated_residual; W must
 * not overlap out.  Needs K % 16 == 0 (BF16) or K % 4 == 0 (F32), rows
 * 16-byte aligned.  ggml's quantized block types are not taken
 * (EMB_ERR_UNSUPPORTED). */
int emb_dense_gated_residual(const void *x, int32_t x_is_f32, int64_t ldx, const void *weight,
                             int32_t weight_type, int64_t ldw, int32_t M, int32_t K, int32_t N,
                             const float *bias, const float *gate, int64_t ldg,
                             const float *gate_bias, const float *residual, int64_t ldr, float *out,
                             int64_t ldo, int32_t round_bf16, void *x_bf16_workspace,
                             hipStream_t stream);

/* Reference-named W8 face (kernels/cosmos3/cosmos3_w8_marlin_cuda.h:24-84 with
 * hipStream_t).  y is f32 holding the bf16-rounded result.  linear_f32_ws
 * rounds x into x_bf16_workspace (batch * in_features bf16, or NULL: rounded
 * while staged) before the GEMM, as the reference does; the other workspaces
 * are accepted and not used. */
int cosmos3_w8a16_linear_f32(const float *x, const int *qweight, const unsigned short *scales_bf16,
                             float *y, int batch, int in_features, int out_features,
                             int qweight_rows, int qweight_cols, int scale_rows, int scale_cols,
                             hipStream_t stream);
int cosmos3_w8a16_linear_f32_ws(const float *x, const int *qweight,
                                const unsigned short *scales_bf16, float *y,
                                unsigned short *x_bf16_workspace, unsigned short *y_bf16_workspace,
                                float *c_tmp_workspace, int *int_workspace, int batch,
                                int in_features, int out_features, int qweight_rows,
                                int qweight_cols, int scale_rows, int scale_cols, hipStream_t stream);
int cosmos3_w8a16_linear_bf16_ws(const unsigned short *x_bf16, const int *qweight,
                                 const unsigned short *scales_bf16, float *y,
                                 unsigned short *y_bf16_workspace, float *c_tmp_workspace,
                                 int *int_workspace, int batch, int in_features, int out_features,
                                 int qweight_rows, int qweight_cols, int scale_rows, int scale_cols,
                                 hipStream_t stream);
int cosmos3_w8a16_f32_to_bf16_ws(const float *x, unsigned short *x_bf16_workspace, int count,
                                 hipStream_t stream);

/* Synthetic inputs for the bench: N(0,1) bf16 from std::mt19937_64(seed)
 * (Box-Muller on 53-bit uniforms), written to host memory. */
int emb_synth_normal_bf16(uint64_t seed, int64_t n, uint16_t *out);

#ifdef __cplusplus
}
#endif
#endif
