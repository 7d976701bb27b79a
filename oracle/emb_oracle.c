/*
 * emb_oracle.c -- CPU oracle (TEST INFRASTRUCTURE ONLY; see emb_oracle.h).
 *
 * Plain C11 restatement of the reference's algorithms for the KV-cached
 * attention step.  Citations are file:line in the reference repository.
 * Accumulations in the attention and GEMM oracles use double so that the
 * oracle sits closer to exact arithmetic than any fp32 implementation under
 * test; the reference's own CPU references accumulate in float, which is
 * within fp32 rounding of this.
 */
#include "emb_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ================= bf16 ================= */

float orc_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

/* ================= mt19937_64 (the C++ std::mt19937_64 engine) ================= */

void orc_mt64_seed(orc_mt64 *g, uint64_t seed) {
    g->mt[0] = seed;
    for (int i = 1; i < 312; ++i)
        g->mt[i] = 6364136223846793005ULL * (g->mt[i - 1] ^ (g->mt[i - 1] >> 62)) + (uint64_t)i;
    g->idx = 312;
}

uint64_t orc_mt64_next(orc_mt64 *g) {
    const uint64_t UM = 0xFFFFFFFF80000000ULL, LM = 0x7FFFFFFFULL;
    if (g->idx >= 312) {
        for (int i = 0; i < 312; ++i) {
            uint64_t x = (g->mt[i] & UM) | (g->mt[(i + 1) % 312] & LM);
            uint64_t xa = x >> 1;
            if (x & 1ULL) xa ^= 0xB5026F5AA96619E9ULL;
            g->mt[i] = g->mt[(i + 156) % 312] ^ xa;
        }
        g->idx = 0;
    }
    uint64_t x = g->mt[g->idx++];
    x ^= (x >> 29) & 0x5555555555555555ULL;
    x ^= (x << 17) & 0x71D67FFFEDA60000ULL;
    x ^= (x << 37) & 0xFFF7EEE000000000ULL;
    x ^= x >> 43;
    return x;
}

uint64_t orc_mt64_nth(uint64_t seed, int64_t n) {
    orc_mt64 g;
    orc_mt64_seed(&g, seed);
    uint64_t x = 0;
    for (int64_t i = 0; i < n; ++i) x = orc_mt64_next(&g);
    return x;
}

void orc_fill_normal_bf16(uint64_t seed, int64_t n, uint16_t *out) {
    orc_mt64 g;
    orc_mt64_seed(&g, seed);
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        uint64_t a = orc_mt64_next(&g), b = orc_mt64_next(&g);
        double u1 = ((double)(a >> 11) + 0.5) * (1.0 / 9007199254740992.0);
        double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
        double r = sqrt(-2.0 * log(u1));
        out[i] = orc_f32_to_bf16((float)(r * cos(two_pi * u2)));
        if (i + 1 < n) out[i + 1] = orc_f32_to_bf16((float)(r * sin(two_pi * u2)));
    }
}

/* ================= slot cache: models/lingbot_va.cpp:8740-8997 ================= */

orc_slot_cache *orc_cache_new(int64_t total, int legacy_clear_pred) {
    /* LingBotKVCache::init, :8751-8763 (meta part; K/V rows live elsewhere) */
    orc_slot_cache *c = (orc_slot_cache *)calloc(1, sizeof(*c));
    c->total = total;
    c->id = (int64_t *)malloc(sizeof(int64_t) * (size_t)(total > 0 ? total : 1));
    c->mask = (uint8_t *)calloc((size_t)(total > 0 ? total : 1), 1);
    c->is_pred = (uint8_t *)calloc((size_t)(total > 0 ? total : 1), 1);
    for (int64_t i = 0; i < total; ++i) c->id[i] = -1;
    c->legacy_clear_pred = legacy_clear_pred;
    return c;
}

void orc_cache_free(orc_slot_cache *c) {
    if (!c) return;
    free(c->id);
    free(c->mask);
    free(c->is_pred);
    free(c);
}

int64_t *orc_cache_id_ptr(orc_slot_cache *c) { return c->id; }
uint8_t *orc_cache_mask_ptr(orc_slot_cache *c) { return c->mask; }
uint8_t *orc_cache_is_pred_ptr(orc_slot_cache *c) { return c->is_pred; }

int64_t orc_cache_used_count(const orc_slot_cache *c) { /* :8774-8776 */
    int64_t n = 0;
    for (int64_t i = 0; i < c->total; ++i) n += c->mask[i] == 1;
    return n;
}

int64_t orc_cache_pred_count(const orc_slot_cache *c) { /* :8778-8784 */
    int64_t n = 0;
    for (int64_t i = 0; i < c->total; ++i) n += (c->mask[i] && c->is_pred[i]);
    return n;
}

int64_t orc_cache_next_id(const orc_slot_cache *c) { /* :8786-8792 */
    int64_t out = -1;
    for (int64_t i = 0; i < c->total; ++i)
        if (c->mask[i] && c->id[i] > out) out = c->id[i];
    return out + 1;
}

static const int64_t *g_sort_ids; /* comparator context (single-threaded use) */
static int cmp_by_id_then_slot(const void *a, const void *b) {
    int64_t sa = *(const int64_t *)a, sb = *(const int64_t *)b;
    int64_t ia = g_sort_ids[sa], ib = g_sort_ids[sb];
    if (ia != ib) return ia < ib ? -1 : 1;
    return sa < sb ? -1 : (sa > sb);
}
static int cmp_i64(const void *a, const void *b) {
    int64_t x = *(const int64_t *)a, y = *(const int64_t *)b;
    return x < y ? -1 : (x > y);
}

/* allocate_slots_into, :8793-8831.  Free slots ascending; if short, evict the
 * `need` used slots with the lowest id.  The reference sorts with std::sort
 * (not stable), so the victims among equal ids are unspecified there; this
 * oracle breaks ties by ascending slot.  Evictions persist on failure. */
int orc_cache_allocate(orc_slot_cache *c, int64_t key_size, int64_t *slots) {
    if (key_size <= 0) return 0;
    int64_t T = c->total;
    int64_t *fr = (int64_t *)malloc(sizeof(int64_t) * (size_t)(T + 1));
    int64_t nf = 0;
    for (int64_t i = 0; i < T; ++i)
        if (!c->mask[i]) fr[nf++] = i;
    if (nf < key_size) {
        int64_t *used = (int64_t *)malloc(sizeof(int64_t) * (size_t)(T + 1));
        int64_t nu = 0;
        for (int64_t i = 0; i < T; ++i)
            if (c->mask[i]) used[nu++] = i;
        g_sort_ids = c->id;
        qsort(used, (size_t)nu, sizeof(int64_t), cmp_by_id_then_slot);
        int64_t need = key_size - nf;
        for (int64_t i = 0; i < need && i < nu; ++i) {
            int64_t s = used[i];
            c->mask[s] = 0;
            c->id[s] = -1;
            if (c->legacy_clear_pred) c->is_pred[s] = 0;
            fr[nf++] = s;
        }
        qsort(fr, (size_t)nf, sizeof(int64_t), cmp_i64);
        free(used);
    }
    int ok = nf >= key_size;
    if (ok) memcpy(slots, fr, sizeof(int64_t) * (size_t)key_size);
    free(fr);
    return ok;
}

/* update_meta_only, :8888-8902 (batch == 1).  next_id is taken after eviction. */
int orc_cache_update_meta(orc_slot_cache *c, int64_t key_size, int pred, int64_t *slots) {
    if (key_size <= 0) return 0;
    if (!orc_cache_allocate(c, key_size, slots)) return 0;
    int64_t nid = orc_cache_next_id(c);
    for (int64_t i = 0; i < key_size; ++i) {
        c->mask[slots[i]] = 1;
        c->id[slots[i]] = nid;
        c->is_pred[slots[i]] = pred ? 1 : 0;
    }
    return 1;
}

/* prepare_mode0_temp_slots_no_insert, :8904-8944 */
int orc_cache_prepare_mode0(orc_slot_cache *c, int64_t key_size, int64_t *slots, int64_t *valid,
                            int64_t *n_valid) {
    *n_valid = 0;
    if (key_size <= 0) return 0;
    if (!orc_cache_allocate(c, key_size, slots)) return 0;
    for (int64_t i = 0; i < key_size; ++i) {
        if (i > 0 && slots[i] <= slots[i - 1]) return 0;
        if (slots[i] < 0 || slots[i] >= c->total || c->mask[slots[i]]) return 0;
    }
    int64_t history_used = orc_cache_used_count(c);
    int64_t nid = orc_cache_next_id(c);
    for (int64_t i = 0; i < key_size; ++i) {
        c->id[slots[i]] = nid;
        c->is_pred[slots[i]] = 0;
    }
    int64_t nv = 0, j = 0;
    for (int64_t i = 0; i < c->total; ++i) {
        while (j < key_size && slots[j] < i) ++j;
        if (c->mask[i] || (j < key_size && slots[j] == i)) valid[nv++] = i;
    }
    *n_valid = nv;
    return nv == history_used + key_size;
}

void orc_cache_restore(orc_slot_cache *c, const int64_t *slots, int64_t n) { /* :8946-8952 */
    for (int64_t i = 0; i < n; ++i)
        if (slots[i] >= 0 && slots[i] < c->total) c->mask[slots[i]] = 0;
}

void orc_cache_clear_pred(orc_slot_cache *c) { /* :8954-8965 */
    for (int64_t i = 0; i < c->total; ++i) {
        if (c->is_pred[i]) {
            c->mask[i] = 0;
            if (c->legacy_clear_pred) {
                c->is_pred[i] = 0;
                c->id[i] = -1;
            }
        }
    }
}

int64_t orc_cache_collect_valid(const orc_slot_cache *c, int64_t *valid) { /* :8967-8972 */
    int64_t n = 0;
    for (int64_t i = 0; i < c->total; ++i)
        if (c->mask[i]) valid[n++] = i;
    return n;
}

/* lingbot_runtime_kv_capacity, :9217-9249, with the environment replaced by
 * explicit arguments (override_tokens > 0 plays VLA_LINGBOT_KV_CACHE_TOKENS). */
int64_t orc_lingbot_capacity(int64_t override_tokens, int64_t frame_chunk_size,
                             int64_t action_per_frame, int64_t n_suffix, int64_t attn_window,
                             int64_t latent_h, int64_t latent_w, int64_t patch_t,
                             int64_t patch_h, int64_t patch_w, int64_t seq) {
    if (override_tokens > 0) return override_tokens > seq ? override_tokens : seq;
    int64_t latent_tokens = (patch_t > 0 && patch_h > 0 && patch_w > 0)
                                ? (frame_chunk_size * latent_h * latent_w) / (patch_t * patch_h * patch_w)
                                : 128;
    int64_t action_tokens = n_suffix > 0 ? n_suffix : frame_chunk_size * action_per_frame;
    int64_t cap = (attn_window / 2) * latent_tokens + (attn_window / 2) * action_tokens;
    return cap > seq ? cap : seq;
}

/* ================= token-slot movement: lingbot_flex_attn_cuda.cu ================= */

/* runtime_kv_update_f32_kernel, :626-649 (on bf16 payloads) */
void orc_slot_update(const uint16_t *k, const uint16_t *v, uint16_t *cache_k, uint16_t *cache_v,
                     const int32_t *slots, int64_t seq, int64_t heads, int64_t head_dim,
                     int64_t capacity) {
    int64_t hd = heads * head_dim;
    for (int64_t s = 0; s < seq; ++s) {
        int64_t slot = slots[s];
        if (slot < 0 || slot >= capacity) continue;
        memcpy(cache_k + slot * hd, k + s * hd, sizeof(uint16_t) * (size_t)hd);
        memcpy(cache_v + slot * hd, v + s * hd, sizeof(uint16_t) * (size_t)hd);
    }
}

/* runtime_kv_gather_f32_kernel, :875-898 */
void orc_slot_gather(const uint16_t *cache_k, const uint16_t *cache_v, const int32_t *valid,
                     uint16_t *out_k, uint16_t *out_v, int64_t seq_k, int64_t heads,
                     int64_t head_dim, int64_t capacity) {
    int64_t hd = heads * head_dim;
    for (int64_t i = 0; i < seq_k; ++i) {
        int64_t slot = valid[i];
        if (slot < 0 || slot >= capacity) continue;
        memcpy(out_k + i * hd, cache_k + slot * hd, sizeof(uint16_t) * (size_t)hd);
        memcpy(out_v + i * hd, cache_v + slot * hd, sizeof(uint16_t) * (size_t)hd);
    }
}

/* ================= paged pool (logical slot s -> page bt[s/16], row s%16) ================= */

void orc_paged_append(const uint16_t *k, const uint16_t *v, int64_t src_stride, int64_t n,
                      int64_t heads, int64_t head_dim, const int32_t *slots,
                      const int32_t *block_table, int64_t capacity, uint16_t *k_pool,
                      uint16_t *v_pool) {
    for (int64_t s = 0; s < n; ++s) {
        int64_t slot = slots[s];
        if (slot < 0 || slot >= capacity) continue;
        int64_t page = block_table ? block_table[slot / 16] : slot / 16;
        if (page < 0) continue;
        int64_t t = slot % 16;
        for (int64_t h = 0; h < heads; ++h)
            for (int64_t d = 0; d < head_dim; ++d) {
                int64_t src = s * src_stride + h * head_dim + d;
                k_pool[((page * heads + h) * 16 + t) * head_dim + d] = k[src];
                v_pool[((page * heads + h) * head_dim + d) * 16 + t] = v[src];
            }
    }
}

void orc_paged_gather(const uint16_t *k_pool, const uint16_t *v_pool, const int32_t *valid,
                      int64_t n, int64_t heads, int64_t head_dim, const int32_t *block_table,
                      int64_t capacity, uint16_t *k_out, uint16_t *v_out) {
    for (int64_t i = 0; i < n; ++i) {
        int64_t slot = valid[i];
        if (slot < 0 || slot >= capacity) continue;
        int64_t page = block_table ? block_table[slot / 16] : slot / 16;
        if (page < 0) continue;
        int64_t t = slot % 16;
        for (int64_t h = 0; h < heads; ++h)
            for (int64_t d = 0; d < head_dim; ++d) {
                int64_t dst = (i * heads + h) * head_dim + d;
                k_out[dst] = k_pool[((page * heads + h) * 16 + t) * head_dim + d];
                v_out[dst] = v_pool[((page * heads + h) * head_dim + d) * 16 + t];
            }
    }
}

/* ================= flex masks: models/lingbot_va.cpp:9274-9465 ================= */

/* build_flex_mask_meta, :9283-9328.  Channel counts do not enter the ids. */
orc_flex_meta *orc_flex_meta_build(int64_t lat_b, int64_t lat_f, int64_t lat_h, int64_t lat_w,
                                   int64_t act_b, int64_t act_f, int64_t act_h, int64_t act_w,
                                   int64_t padded_length, int64_t chunk_size, int64_t window_size,
                                   int64_t pt, int64_t ph, int64_t pw, int64_t text_seq,
                                   int64_t block_size) {
    (void)act_b; /* the action loop runs inside the latent batch loop (:9298-9316) */
    int64_t nl_per_b = (lat_f / pt) * (lat_h / ph) * (lat_w / pw);
    int64_t na_per_b = act_f * act_h * act_w;
    int64_t nl = lat_b * nl_per_b, na = lat_b * na_per_b;
    int64_t n = 2 * nl + 2 * na + padded_length;
    orc_flex_meta *m = (orc_flex_meta *)calloc(1, sizeof(*m));
    m->n = n;
    m->n_text = lat_b * text_seq;
    m->seq_ids = (int64_t *)malloc(sizeof(int64_t) * (size_t)(n + 1));
    m->frame_ids = (int64_t *)malloc(sizeof(int64_t) * (size_t)(n + 1));
    m->noise_ids = (int64_t *)malloc(sizeof(int64_t) * (size_t)(n + 1));
    m->text_seq_ids = (int64_t *)malloc(sizeof(int64_t) * (size_t)(m->n_text + 1));
    m->window_size = window_size;
    m->block_size = block_size;
    int64_t *ls = (int64_t *)malloc(sizeof(int64_t) * (size_t)(nl + 1));
    int64_t *lf = (int64_t *)malloc(sizeof(int64_t) * (size_t)(nl + 1));
    int64_t *as = (int64_t *)malloc(sizeof(int64_t) * (size_t)(na + 1));
    int64_t *af = (int64_t *)malloc(sizeof(int64_t) * (size_t)(na + 1));
    int64_t il = 0, ia = 0;
    for (int64_t b = 0; b < lat_b; ++b) {
        for (int64_t f = 0; f < lat_f / pt; ++f)
            for (int64_t h = 0; h < lat_h / ph; ++h)
                for (int64_t w = 0; w < lat_w / pw; ++w) {
                    ls[il] = b;
                    lf[il++] = (f * pt) / chunk_size * 2;
                }
        for (int64_t f = 0; f < act_f; ++f)
            for (int64_t h = 0; h < act_h; ++h)
                for (int64_t w = 0; w < act_w; ++w) {
                    as[ia] = b;
                    af[ia++] = f / chunk_size * 2 + 1;
                }
    }
    int64_t p = 0;
    for (int64_t i = 0; i < nl; ++i, ++p) { m->seq_ids[p] = ls[i]; m->frame_ids[p] = lf[i]; m->noise_ids[p] = 0; }
    for (int64_t i = 0; i < nl; ++i, ++p) { m->seq_ids[p] = ls[i]; m->frame_ids[p] = lf[i]; m->noise_ids[p] = 1; }
    for (int64_t i = 0; i < na; ++i, ++p) { m->seq_ids[p] = as[i]; m->frame_ids[p] = af[i]; m->noise_ids[p] = 0; }
    for (int64_t i = 0; i < na; ++i, ++p) { m->seq_ids[p] = as[i]; m->frame_ids[p] = af[i]; m->noise_ids[p] = 1; }
    for (int64_t i = 0; i < padded_length; ++i, ++p) { m->seq_ids[p] = -1; m->frame_ids[p] = -1; m->noise_ids[p] = -1; }
    for (int64_t b = 0, t = 0; b < lat_b; ++b)
        for (int64_t i = 0; i < text_seq; ++i) m->text_seq_ids[t++] = b;
    free(ls); free(lf); free(as); free(af);
    return m;
}

void orc_flex_meta_free(orc_flex_meta *m) {
    if (!m) return;
    free(m->seq_ids); free(m->frame_ids); free(m->noise_ids); free(m->text_seq_ids);
    free(m);
}

int orc_flex_self_allowed(const orc_flex_meta *m, int64_t q, int64_t k) { /* :9330-9340 */
    if (m->seq_ids[q] < 0 || m->seq_ids[q] != m->seq_ids[k]) return 0;
    int64_t qf = m->frame_ids[q], kf = m->frame_ids[k];
    int64_t qn = m->noise_ids[q], kn = m->noise_ids[k];
    int c2c = qn == 1 && kn == 1 && kf <= qf;
    int n2c = qn == 0 && kn == 1 && kf < qf;
    int n2n = qn == 0 && kn == 0 && kf == qf;
    int64_t df = qf - kf;
    if (df < 0) df = -df;
    return (c2c || n2c || n2n) && df <= m->window_size;
}

int orc_flex_cross_allowed(const orc_flex_meta *m, int64_t q, int64_t k) { /* :9342-9344 */
    return m->seq_ids[q] >= 0 && m->seq_ids[q] == m->text_seq_ids[k];
}

int64_t orc_dense_block_table(int64_t seq_q, int64_t seq_k, int64_t bs, int64_t *row_ptr,
                              int64_t *col_idx) { /* build_dense_block_table, :9354-9372 */
    int64_t qb = (seq_q + bs - 1) / bs, kb = (seq_k + bs - 1) / bs, nnz = 0;
    row_ptr[0] = 0;
    for (int64_t r = 0; r < qb; ++r) {
        for (int64_t c = 0; c < kb; ++c) col_idx[nnz++] = c;
        row_ptr[r + 1] = nnz;
    }
    return nnz;
}

typedef int (*orc_pred_fn)(const orc_flex_meta *, int64_t, int64_t);

static int64_t block_table_brute(const orc_flex_meta *m, int64_t qn, int64_t kn, orc_pred_fn fn,
                                 int64_t *row_ptr, int64_t *col_idx) {
    int64_t bs = m->block_size;
    int64_t qb = (qn + bs - 1) / bs, kb = (kn + bs - 1) / bs, nnz = 0;
    row_ptr[0] = 0;
    for (int64_t r = 0; r < qb; ++r) {
        int64_t q0 = r * bs, q1 = q0 + bs < qn ? q0 + bs : qn;
        for (int64_t c = 0; c < kb; ++c) {
            int64_t k0 = c * bs, k1 = k0 + bs < kn ? k0 + bs : kn;
            int any = 0;
            for (int64_t q = q0; q < q1 && !any; ++q)
                for (int64_t k = k0; k < k1; ++k)
                    if (fn(m, q, k)) { any = 1; break; }
            if (any) col_idx[nnz++] = c;
        }
        row_ptr[r + 1] = nnz;
    }
    return nnz;
}

int64_t orc_self_block_table(const orc_flex_meta *m, int64_t *row_ptr, int64_t *col_idx) {
    return block_table_brute(m, m->n, m->n, orc_flex_self_allowed, row_ptr, col_idx); /* :9374-9403 */
}

int64_t orc_cross_block_table(const orc_flex_meta *m, int64_t *row_ptr, int64_t *col_idx) {
    return block_table_brute(m, m->n, m->n_text, orc_flex_cross_allowed, row_ptr, col_idx); /* :9405-9433 */
}

void orc_self_token_mask(const orc_flex_meta *m, uint8_t *mask) { /* :9456-9465 */
    for (int64_t q = 0; q < m->n; ++q)
        for (int64_t k = 0; k < m->n; ++k) mask[q * m->n + k] = (uint8_t)orc_flex_self_allowed(m, q, k);
}

int64_t orc_max_row_nnz(const int64_t *row_ptr, int64_t q_blocks) { /* :9442-9448 */
    int64_t out = 0;
    for (int64_t r = 0; r < q_blocks; ++r)
        if (row_ptr[r + 1] - row_ptr[r] > out) out = row_ptr[r + 1] - row_ptr[r];
    return out;
}

/* ================= attention ================= */

/* dense_masked_attention_ref, models/lingbot_va.cpp:9467-9511 (also dense_ref,
 * kernels/lingbot/lingbot_flex_attn_cuda.cu:1010-1031): two passes, divide at
 * the end, an empty row gives 0. */
void orc_dense_masked_attention(const float *q, const float *k, const float *v,
                                const uint8_t *mask, int64_t seq, int64_t heads,
                                int64_t head_dim, float *out) {
    const double scale = 1.0 / sqrt((double)head_dim);
    for (int64_t s = 0; s < seq; ++s)
        for (int64_t h = 0; h < heads; ++h) {
            const float *qr = q + (s * heads + h) * head_dim;
            double mx = -INFINITY;
            for (int64_t t = 0; t < seq; ++t) {
                if (!mask[s * seq + t]) continue;
                double dot = 0;
                const float *kr = k + (t * heads + h) * head_dim;
                for (int64_t d = 0; d < head_dim; ++d) dot += (double)qr[d] * kr[d];
                if (dot * scale > mx) mx = dot * scale;
            }
            double sum = 0;
            double *acc = (double *)calloc((size_t)head_dim, sizeof(double));
            for (int64_t t = 0; t < seq; ++t) {
                if (!mask[s * seq + t]) continue;
                double dot = 0;
                const float *kr = k + (t * heads + h) * head_dim;
                for (int64_t d = 0; d < head_dim; ++d) dot += (double)qr[d] * kr[d];
                double w = exp(dot * scale - mx);
                sum += w;
                const float *vr = v + (t * heads + h) * head_dim;
                for (int64_t d = 0; d < head_dim; ++d) acc[d] += w * vr[d];
            }
            for (int64_t d = 0; d < head_dim; ++d)
                out[(s * heads + h) * head_dim + d] = sum > 0 ? (float)(acc[d] / sum) : 0.0f;
            free(acc);
        }
}

/* flex_attn_f32_kernel, lingbot_flex_attn_cuda.cu:502-582: keys come from the
 * CSR row of the query's block (each listed block once per listing), then the
 * optional dense token mask filters them. */
void orc_flex_attention(const float *q, const float *k, const float *v, const int32_t *row_ptr,
                        const int32_t *col_idx, const uint8_t *token_mask, float *out,
                        int64_t seq_q, int64_t seq_k, int64_t heads, int64_t head_dim,
                        int64_t block_size, float scale) {
    double *acc = (double *)malloc(sizeof(double) * (size_t)head_dim);
    for (int64_t qi = 0; qi < seq_q; ++qi)
        for (int64_t h = 0; h < heads; ++h) {
            const float *qr = q + (qi * heads + h) * head_dim;
            int64_t qb = qi / block_size;
            double mx = -INFINITY, sum = 0;
            for (int pass = 0; pass < 2; ++pass) {
                if (pass == 1) memset(acc, 0, sizeof(double) * (size_t)head_dim);
                for (int64_t p = row_ptr[qb]; p < row_ptr[qb + 1]; ++p) {
                    int64_t k0 = (int64_t)col_idx[p] * block_size;
                    int64_t k1 = k0 + block_size < seq_k ? k0 + block_size : seq_k;
                    for (int64_t kid = k0; kid < k1; ++kid) {
                        if (token_mask && !token_mask[qi * seq_k + kid]) continue;
                        double dot = 0;
                        const float *kr = k + (kid * heads + h) * head_dim;
                        for (int64_t d = 0; d < head_dim; ++d) dot += (double)qr[d] * kr[d];
                        double s = dot * scale;
                        if (pass == 0) {
                            if (s > mx) mx = s;
                        } else {
                            double w = exp(s - mx);
                            sum += w;
                            const float *vr = v + (kid * heads + h) * head_dim;
                            for (int64_t d = 0; d < head_dim; ++d) acc[d] += w * vr[d];
                        }
                    }
                }
            }
            for (int64_t d = 0; d < head_dim; ++d)
                out[(qi * heads + h) * head_dim + d] = sum > 0 ? (float)(acc[d] / sum) : 0.0f;
        }
    free(acc);
}

/* runtime_kv_attn_{f32,online_f32,warp_f32}, lingbot_flex_attn_cuda.cu:651-873:
 * attention of q over cache rows valid[0..seq_k).  online_quirk = 1 keeps the
 * online/warp behaviour for a negative slot (dot = 0, so exp(0 - max) joins the
 * denominator, and no V row); online_quirk = 0 skips such keys. */
void orc_runtime_kv_attn(const float *q, const float *cache_k, const float *cache_v,
                         const int32_t *valid, float *out, int64_t seq_q, int64_t seq_k,
                         int64_t heads, int64_t head_dim, float scale, int online_quirk) {
    double *acc = (double *)malloc(sizeof(double) * (size_t)head_dim);
    for (int64_t qi = 0; qi < seq_q; ++qi)
        for (int64_t h = 0; h < heads; ++h) {
            const float *qr = q + (qi * heads + h) * head_dim;
            double mx = -INFINITY, sum = 0;
            for (int pass = 0; pass < 2; ++pass) {
                if (pass == 1) memset(acc, 0, sizeof(double) * (size_t)head_dim);
                for (int64_t j = 0; j < seq_k; ++j) {
                    int64_t slot = valid[j];
                    if (slot < 0 && !online_quirk) continue;
                    double dot = 0;
                    if (slot >= 0) {
                        const float *kr = cache_k + (slot * heads + h) * head_dim;
                        for (int64_t d = 0; d < head_dim; ++d) dot += (double)qr[d] * kr[d];
                    }
                    double s = dot * scale;
                    if (pass == 0) {
                        if (s > mx) mx = s;
                    } else {
                        double w = exp(s - mx);
                        sum += w;
                        if (slot >= 0) {
                            const float *vr = cache_v + (slot * heads + h) * head_dim;
                            for (int64_t d = 0; d < head_dim; ++d) acc[d] += w * vr[d];
                        }
                    }
                }
            }
            for (int64_t d = 0; d < head_dim; ++d)
                out[(qi * heads + h) * head_dim + d] = sum > 0 ? (float)(acc[d] / sum) : 0.0f;
        }
    free(acc);
}

/* ggml attention as called by models/pi05.cpp:405-418 (mul_mat F32 -> soft_max_ext
 * (mask, scale) -> mul_mat) and models/hy_vla.cpp:1066-1076 (flash_attn_ext with an
 * additive mask): q head h reads kv head h / (hq/hkv).  A row whose keys are all
 * masked gives 0 (as dense_masked_attention_ref does). */
void orc_gqa_attention_bf16(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                            int64_t n_q, int64_t n_k, int64_t hq, int64_t hkv, int64_t d,
                            float scale, const uint8_t *allow, const float *add, int64_t chunk,
                            int64_t window, int64_t q_pos0, const int64_t *rows, int64_t n_rows,
                            int threads, float *out) {
    if (!rows) n_rows = n_q;
    int64_t G = hq / hkv;
    int64_t total = n_rows * hq;
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#else
    (void)threads;
#endif
    {
        float *kf = (float *)malloc(sizeof(float) * (size_t)d);
        double *acc = (double *)malloc(sizeof(double) * (size_t)d);
        double *sc = (double *)malloc(sizeof(double) * (size_t)(n_k + 1));
        float *qf = (float *)malloc(sizeof(float) * (size_t)d);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
        for (int64_t w = 0; w < total; ++w) {
            int64_t ri = w / hq, h = w % hq;
            int64_t i = rows ? rows[ri] : ri;
            int64_t kvh = h / G;
            for (int64_t x = 0; x < d; ++x) qf[x] = orc_bf16_to_f32(q[(i * hq + h) * d + x]);
            int64_t qpos = q_pos0 + i;
            double mx = -INFINITY;
            for (int64_t j = 0; j < n_k; ++j) {
                int ok = allow ? allow[i * n_k + j] != 0 : 1;
                if (ok && chunk > 0) {
                    int64_t qc = qpos / chunk, kc = j / chunk;
                    ok = kc <= qc && (window < 0 || qc - kc <= window);
                }
                if (!ok) { sc[j] = -INFINITY; continue; }
                const uint16_t *kr = k + (j * hkv + kvh) * d;
                double dot = 0;
                for (int64_t x = 0; x < d; ++x) dot += (double)qf[x] * orc_bf16_to_f32(kr[x]);
                double s = dot * scale + (add ? (double)add[i * n_k + j] : 0.0);
                sc[j] = s;
                if (s > mx) mx = s;
            }
            double sum = 0;
            for (int64_t x = 0; x < d; ++x) acc[x] = 0;
            if (mx > -INFINITY) {
                for (int64_t j = 0; j < n_k; ++j) {
                    if (sc[j] == -INFINITY) continue;
                    double p = exp(sc[j] - mx);
                    sum += p;
                    const uint16_t *vr = v + (j * hkv + kvh) * d;
                    for (int64_t x = 0; x < d; ++x) acc[x] += p * orc_bf16_to_f32(vr[x]);
                }
            }
            float *o = out + (i * hq + h) * d;
            for (int64_t x = 0; x < d; ++x) o[x] = sum > 0 ? (float)(acc[x] / sum) : 0.0f;
        }
        free(kf); free(acc); free(sc); free(qf);
    }
}

/* ================= W8 Marlin: kernels/cosmos3/cosmos3_w8_marlin_cuda.cu:50-88 ================= */

int64_t orc_marlin_dst_byte(int64_t k, int64_t n, int64_t out_features) { /* :50-58, README:55-64 */
    int64_t row = k / 16;
    int64_t col = (n / 64) * 256 + (n % 8) * 32 + ((n / 8) % 8) + ((k % 8) / 2) * 8;
    int64_t lane = (k % 2) * 2 + ((k / 8) % 2);
    return ((row * (out_features * 4) + col) * 4) + lane;
}

int64_t orc_marlin_scale_index(int64_t n) { /* marlin_scale_index, :79-88 */
    static const int inv[32] = {0, 1, 8,  9,  16, 17, 24, 25, 2, 3, 10, 11, 18, 19, 26, 27,
                                4, 5, 12, 13, 20, 21, 28, 29, 6, 7, 14, 15, 22, 23, 30, 31};
    return (n / 32) * 32 + inv[n & 31];
}

void orc_marlin_pack_w8(const int8_t *w, int64_t K, int64_t N, int32_t *qweight) {
    uint8_t *bytes = (uint8_t *)qweight; /* little-endian lanes, as unpack reads them */
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n) bytes[orc_marlin_dst_byte(k, n, N)] = (uint8_t)(w[k * N + n] + 128);
}

int orc_marlin_unpack_w8(const int32_t *qweight, int64_t K, int64_t N, int64_t k, int64_t n) {
    /* unpack_marlin_uint8b128, :60-77 */
    if (k < 0 || k >= K || n < 0 || n >= N) return 0;
    int64_t b = orc_marlin_dst_byte(k, n, N);
    uint32_t word = (uint32_t)qweight[b / 4];
    return (int)((word >> ((b & 3) * 8)) & 0xffu) - 128;
}

void orc_marlin_pack_scales(const uint16_t *s_logical, int64_t N, uint16_t *s_stored) {
    for (int64_t n = 0; n < N; ++n) s_stored[orc_marlin_scale_index(n)] = s_logical[n];
}

/* Numerics of the Marlin channelwise path: bf16(x) * (u8 - 128) accumulated in
 * fp32, the fp32 accumulator multiplied by the fp32 channel scale
 * (third_party/vllm_marlin/marlin_template.h:166-174, :1974-1993), then rounded to
 * bf16 (cosmos3_w8_marlin_cuda.cu:371-406) and widened to f32 (:407). */
void orc_w8a16_gemm(const uint16_t *x, const int32_t *qweight, const uint16_t *s_stored,
                    int64_t M, int64_t K, int64_t N, const int64_t *rows, int64_t n_rows,
                    int threads, uint16_t *y_bf16, float *y_f32) {
    if (!rows) n_rows = M;
    /* dequantise once: wT[n][k] */
    int8_t *wT = (int8_t *)malloc((size_t)(K * N));
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n) wT[n * K + k] = (int8_t)orc_marlin_unpack_w8(qweight, K, N, k, n);
    float *sf = (float *)malloc(sizeof(float) * (size_t)N);
    for (int64_t n = 0; n < N; ++n) sf[n] = orc_bf16_to_f32(s_stored[orc_marlin_scale_index(n)]);
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#else
    (void)threads;
#endif
    {
        float *xf = (float *)malloc(sizeof(float) * (size_t)K);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int64_t r = 0; r < n_rows; ++r) {
            int64_t m = rows ? rows[r] : r;
            for (int64_t k = 0; k < K; ++k) xf[k] = orc_bf16_to_f32(x[m * K + k]);
            for (int64_t n = 0; n < N; ++n) {
                const int8_t *wr = wT + n * K;
                double acc = 0;
                for (int64_t k = 0; k < K; ++k) acc += (double)xf[k] * (double)wr[k];
                float y = (float)acc * sf[n];
                if (y_f32) y_f32[r * N + n] = y;
                if (y_bf16) y_bf16[r * N + n] = orc_f32_to_bf16(y);
            }
        }
        free(xf);
    }
    free(wT);
    free(sf);
}

/* ================= CPU baseline (timed by bench.py, not a checker) ================= */

/* fp32 restatement of the reference's CPU op order for the action-expert
 * attention (models/pi05.cpp:414-418: kq = mul_mat(K, Q) in F32,
 * soft_max_ext(kq, mask = 0, scale), kqv = mul_mat(V, softmax)), threaded over
 * (query, head) rows with OpenMP.  q [n_q][hq][d], k/v [n_k][hkv][d] already
 * widened to f32, as ggml holds them. */
__attribute__((target("avx2,fma"))) static void cpu_attn_row_avx2(const float *qr, const float *k,
                                                                   const float *v, int64_t n_k,
                                                                   int64_t hkv, int64_t kvh, int64_t d,
                                                                   float scale, float *sc, float *o) {
    float mx = -INFINITY;
    for (int64_t j = 0; j < n_k; ++j) {
        const float *kr = k + (j * hkv + kvh) * d;
        float dot = 0.0f;
#pragma omp simd reduction(+ : dot)
        for (int64_t x = 0; x < d; ++x) dot += qr[x] * kr[x];
        sc[j] = dot * scale;
        if (sc[j] > mx) mx = sc[j];
    }
    float sum = 0.0f;
    for (int64_t j = 0; j < n_k; ++j) {
        sc[j] = expf(sc[j] - mx);
        sum += sc[j];
    }
    for (int64_t x = 0; x < d; ++x) o[x] = 0.0f;
    for (int64_t j = 0; j < n_k; ++j) {
        const float *vr = v + (j * hkv + kvh) * d;
        const float p = sc[j];
#pragma omp simd
        for (int64_t x = 0; x < d; ++x) o[x] += p * vr[x];
    }
    const float inv = 1.0f / sum;
    for (int64_t x = 0; x < d; ++x) o[x] *= inv;
}

static void cpu_attn_row_generic(const float *qr, const float *k, const float *v, int64_t n_k,
                                 int64_t hkv, int64_t kvh, int64_t d, float scale, float *sc, float *o) {
    float mx = -INFINITY;
    for (int64_t j = 0; j < n_k; ++j) {
        const float *kr = k + (j * hkv + kvh) * d;
        float dot = 0.0f;
        for (int64_t x = 0; x < d; ++x) dot += qr[x] * kr[x];
        sc[j] = dot * scale;
        if (sc[j] > mx) mx = sc[j];
    }
    float sum = 0.0f;
    for (int64_t j = 0; j < n_k; ++j) {
        sc[j] = expf(sc[j] - mx);
        sum += sc[j];
    }
    for (int64_t x = 0; x < d; ++x) o[x] = 0.0f;
    for (int64_t j = 0; j < n_k; ++j) {
        const float *vr = v + (j * hkv + kvh) * d;
        for (int64_t x = 0; x < d; ++x) o[x] += sc[j] * vr[x];
    }
    for (int64_t x = 0; x < d; ++x) o[x] /= sum;
}

int orc_cpu_attention_f32(const float *q, const float *k, const float *v, int64_t n_q, int64_t n_k,
                          int64_t hq, int64_t hkv, int64_t d, float scale, int threads, float *out) {
    const int avx2 = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    const int64_t G = hq / hkv;
    int used = 1;
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#else
    (void)threads;
#endif
    {
        float *sc = (float *)malloc(sizeof(float) * (size_t)(n_k + 1));
#ifdef _OPENMP
#pragma omp single
        used = omp_get_num_threads();
#pragma omp for schedule(static)
#endif
        for (int64_t w = 0; w < n_q * hq; ++w) {
            const int64_t i = w / hq, h = w % hq;
            const float *qr = q + (i * hq + h) * d;
            float *o = out + (i * hq + h) * d;
            if (avx2)
                cpu_attn_row_avx2(qr, k, v, n_k, hkv, h / G, d, scale, sc, o);
            else
                cpu_attn_row_generic(qr, k, v, n_k, hkv, h / G, d, scale, sc, o);
        }
        free(sc);
    }
    return used;
}

/* ---------------- Qwen per-head q/k RMSNorm + RoPE ----------------
 * kernels/cosmos3/cosmos3_qwen_language_cuda.cu:52-83 (head_rmsnorm_kernel),
 * :85-116 (rope_kernel), :117-153 (mrope_kernel).  f32 arithmetic with the
 * reference's bf16 rounding points; sin/cos/pow from libm in f32. */
static float orc_round_bf16(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }

void orc_head_norm_rope(const uint16_t *x, int64_t ld, int64_t tokens, int64_t heads, int64_t d,
                        const uint16_t *gamma, float eps, int rope_kind, float theta, int64_t first_pos,
                        const int32_t *pos_ids, uint16_t *out, int64_t out_ld) {
    float *v = (float *)malloc(sizeof(float) * (size_t)d);
    const int64_t half = d / 2;
    for (int64_t t = 0; t < tokens; ++t) {
        for (int64_t h = 0; h < heads; ++h) {
            const uint16_t *xr = x + t * ld + h * d;
            if (gamma) {
                float sum = 0.0f;
                for (int64_t i = 0; i < d; ++i) {
                    const float a = orc_bf16_to_f32(xr[i]);
                    sum += a * a;
                }
                const float inv = 1.0f / sqrtf(sum / (float)d + eps);
                for (int64_t i = 0; i < d; ++i)
                    v[i] = orc_round_bf16(orc_round_bf16(orc_bf16_to_f32(xr[i]) * inv) * orc_bf16_to_f32(gamma[i]));
            } else {
                for (int64_t i = 0; i < d; ++i) v[i] = orc_bf16_to_f32(xr[i]);
            }
            uint16_t *o = out + t * out_ld + h * d;
            for (int64_t i = 0; i < d; ++i) {
                if (!rope_kind) {
                    o[i] = orc_f32_to_bf16(v[i]);
                    continue;
                }
                const int64_t p = i < half ? i : i - half;
                int axis = 0;
                if (rope_kind == 2 && p < 60) axis = p % 3 == 1 ? 1 : (p % 3 == 2 ? 2 : 0);
                const float pos = rope_kind == 2 ? (float)pos_ids[axis * tokens + t] : (float)(first_pos + t);
                const float f = powf(theta, -(float)(2 * p) / (float)d);
                const float a = pos * f;
                const float sn = orc_round_bf16(sinf(a)), cs = orc_round_bf16(cosf(a));
                const float r = i < half ? -v[i + half] : v[i - half];
                o[i] = orc_f32_to_bf16(v[i] * cs + r * sn);
            }
        }
    }
    free(v);
}

/* ---------------- pi0.5 NEOX RoPE (ggml_rope_ext, GGML_ROPE_TYPE_NEOX) ----------------
 * Call sites: models/pi05.cpp:308-314 (prefix layers) and :394-400 (expert
 * layers), n_dims = head_dim, freq_scale 1, ext_factor 0, attn_factor 1,
 * positions from :872-878.  ggml itself (llama.cpp b9016) is not vendored; this
 * restates its published f32 rope for its CUDA backend: theta_scale =
 * powf(freq_base, -2 / n_dims); pair i of a row at position pos turns by
 * theta = pos * powf(theta_scale, i) (freq_scale 1 and ext_factor 0 leave
 * theta as is; attn_factor 1 scales cos/sin by 1), and (x[i], x[i + n/2])
 * -> (x0 cos - x1 sin, x0 sin + x1 cos).  f32 throughout, each product rounded
 * on its own (the build uses -ffp-contract=off); libm powf/cosf/sinf. */
void orc_neox_rope_f32(const float *x, int64_t ld, int64_t tokens, int64_t heads, int64_t d,
                       const int32_t *pos, int64_t first_pos, float freq_base, float *out, int64_t out_ld) {
    const int64_t half = d / 2;
    const float theta_scale = powf(freq_base, -2.0f / (float)d);
    for (int64_t t = 0; t < tokens; ++t) {
        const float p = (float)(pos ? (int64_t)pos[t] : first_pos + t);
        for (int64_t h = 0; h < heads; ++h) {
            const float *xr = x + t * ld + h * d;
            float *o = out + t * out_ld + h * d;
            for (int64_t i = 0; i < half; ++i) {
                const float theta = p * powf(theta_scale, (float)i);
                const float c = cosf(theta), s = sinf(theta);
                const float x0 = xr[i], x1 = xr[i + half];
                o[i] = x0 * c - x1 * s;
                o[i + half] = x0 * s + x1 * c;
            }
        }
    }
}
