// Host side of the KV-cached attention step: slot cache with the reference's
// LingBotKVCache semantics, the page pool behind it, the capacity formula and
// the flex-mask builders.
//
// Semantics follow models/lingbot_va.cpp:8740-8997 (cache), :9217-9249
// (capacity) and :9274-9465 (flex masks).  The bookkeeping differs: the
// reference rescans all `capacity` slots on every call under a global mutex;
// here the free slots and the valid slots grouped by insertion id are kept in
// ordered sets, so allocation and eviction touch only the slots they hand out.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstring>
#include <map>
#include <mutex>
#include <set>
#include <vector>

#include "emb_common.h"

namespace emb {

static thread_local std::string g_last_error;

int set_error(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

void clear_error() { g_last_error.clear(); }

}  // namespace emb

struct emb_page_pool {
    int32_t n_pages = 0;
    std::vector<int32_t> free_stack;  // next page handed out is free_stack.back()
    std::set<emb_slot_cache *> caches;  // bound caches, unbound when the pool goes away
    std::mutex mu;                    // caches of several threads may share one pool
};

struct emb_slot_cache {
    int64_t total = 0;
    bool legacy = false;
    std::vector<int64_t> id;
    std::vector<uint8_t> mask, is_pred;
    std::set<int64_t> free_slots;                   // mask == 0, ascending
    std::map<int64_t, std::set<int64_t>> valid_by_id;  // mask == 1 grouped by id
    int64_t used = 0;
    emb_page_pool *pool = nullptr;
    std::vector<int32_t> pages;  // logical page -> physical page, -1 unmapped

    void mark_valid(int64_t s, int64_t nid, bool pred) {
        if (mask[s]) {
            auto it = valid_by_id.find(id[s]);
            it->second.erase(s);
            if (it->second.empty()) valid_by_id.erase(it);
        } else {
            free_slots.erase(s);
            ++used;
        }
        mask[s] = 1;
        id[s] = nid;
        is_pred[s] = pred ? 1 : 0;
        valid_by_id[nid].insert(s);
    }

    void mark_free(int64_t s) {
        if (!mask[s]) return;
        auto it = valid_by_id.find(id[s]);
        it->second.erase(s);
        if (it->second.empty()) valid_by_id.erase(it);
        mask[s] = 0;
        free_slots.insert(s);
        --used;
    }

    int64_t next_id() const { return valid_by_id.empty() ? 0 : valid_by_id.rbegin()->first + 1; }

    int ensure_page(int64_t slot) {
        if (!pool) return EMB_OK;
        int64_t lp = slot / EMB_PAGE_TOKENS;
        if (pages[lp] >= 0) return EMB_OK;
        std::lock_guard<std::mutex> g(pool->mu);
        if (pool->free_stack.empty())
            return emb::set_error(EMB_ERR_CAPACITY, "page pool exhausted (%d pages)", pool->n_pages);
        pages[lp] = pool->free_stack.back();
        pool->free_stack.pop_back();
        return EMB_OK;
    }

    // allocate_slots_into (:8793-8831).  Victims are the `need` valid slots of
    // lowest id; the reference sorts them with std::sort (unstable), this picks
    // ties in ascending slot order.  Evictions persist when the call fails.
    int allocate(int64_t key_size, int64_t *slots) {
        if (key_size <= 0) return emb::set_error(EMB_ERR_ARG, "key_size must be positive");
        int64_t nfree = (int64_t)free_slots.size();
        if (nfree < key_size) {
            int64_t need = key_size - nfree;
            while (need > 0 && !valid_by_id.empty()) {
                auto it = valid_by_id.begin();
                while (need > 0 && !it->second.empty()) {
                    int64_t s = *it->second.begin();
                    it->second.erase(it->second.begin());
                    mask[s] = 0;
                    id[s] = -1;
                    if (legacy) is_pred[s] = 0;
                    free_slots.insert(s);
                    --used;
                    --need;
                }
                if (it->second.empty()) valid_by_id.erase(it);
            }
        }
        if ((int64_t)free_slots.size() < key_size)
            return emb::set_error(EMB_ERR_CAPACITY, "slot cache capacity %lld < request %lld",
                                  (long long)total, (long long)key_size);
        auto it = free_slots.begin();
        for (int64_t i = 0; i < key_size; ++i, ++it) slots[i] = *it;
        for (int64_t i = 0; i < key_size; ++i) {
            int rc = ensure_page(slots[i]);
            if (rc) return rc;
        }
        return EMB_OK;
    }
};

extern "C" {

const char *emb_last_error(void) { return emb::g_last_error.c_str(); }
const char *emb_version(void) { return "emb_kv 0.1 gfx950"; }

emb_slot_cache *emb_slot_cache_create(int64_t capacity, int legacy_clear_pred) {
    if (capacity <= 0 || capacity > (int64_t)1 << 31) {
        emb::set_error(EMB_ERR_ARG, "capacity must be in (0, 2^31]");
        return nullptr;
    }
    auto *c = new emb_slot_cache();
    c->total = capacity;
    c->legacy = legacy_clear_pred != 0;
    c->id.assign((size_t)capacity, -1);
    c->mask.assign((size_t)capacity, 0);
    c->is_pred.assign((size_t)capacity, 0);
    for (int64_t i = 0; i < capacity; ++i) c->free_slots.insert(c->free_slots.end(), i);
    c->pages.assign((size_t)((capacity + EMB_PAGE_TOKENS - 1) / EMB_PAGE_TOKENS), -1);
    return c;
}

void emb_slot_cache_destroy(emb_slot_cache *c) {
    if (!c) return;
    emb_slot_cache_release_pages(c);
    if (c->pool) {
        std::lock_guard<std::mutex> g(c->pool->mu);
        c->pool->caches.erase(c);
    }
    delete c;
}

int64_t emb_slot_cache_capacity(const emb_slot_cache *c) { return c ? c->total : -1; }
int64_t emb_slot_cache_used_count(const emb_slot_cache *c) { return c ? c->used : -1; }

int64_t emb_slot_cache_pred_count(const emb_slot_cache *c) {
    if (!c) return -1;
    int64_t n = 0;
    for (const auto &kv : c->valid_by_id)
        for (int64_t s : kv.second) n += c->is_pred[s] != 0;
    return n;
}

int64_t emb_slot_cache_next_id(const emb_slot_cache *c) { return c ? c->next_id() : -1; }

int emb_slot_cache_allocate(emb_slot_cache *c, int64_t key_size, int64_t *slots) {
    EMB_CHECK_ARG(c && slots, "null argument");
    return c->allocate(key_size, slots);
}

// update_meta_only (:8888-8902): the new id is taken after eviction.
int emb_slot_cache_update_meta(emb_slot_cache *c, int64_t key_size, int pred, int64_t *slots) {
    EMB_CHECK_ARG(c && slots, "null argument");
    int rc = c->allocate(key_size, slots);
    if (rc) return rc;
    const int64_t nid = c->next_id();
    for (int64_t i = 0; i < key_size; ++i) c->mark_valid(slots[i], nid, pred != 0);
    return EMB_OK;
}

// prepare_mode0_temp_slots_no_insert (:8904-8944): the temporary slots get the
// next id and is_pred = 0 but stay invisible (mask 0) to later calls.
int emb_slot_cache_prepare_mode0(emb_slot_cache *c, int64_t key_size, int64_t *slots,
                                 int64_t *valid, int64_t *n_valid) {
    EMB_CHECK_ARG(c && slots && valid && n_valid, "null argument");
    *n_valid = 0;
    int rc = c->allocate(key_size, slots);
    if (rc) return rc;
    const int64_t nid = c->next_id();
    for (int64_t i = 0; i < key_size; ++i) {
        c->id[slots[i]] = nid;
        c->is_pred[slots[i]] = 0;
    }
    // valid = used slots U temp slots, ascending (a merge of two sorted lists)
    int64_t nv = 0, j = 0;
    auto fit = c->free_slots.begin();
    for (int64_t s = 0; s < c->total; ++s) {
        bool is_free = fit != c->free_slots.end() && *fit == s;
        if (is_free) ++fit;
        while (j < key_size && slots[j] < s) ++j;
        if (!is_free || (j < key_size && slots[j] == s)) valid[nv++] = s;
    }
    *n_valid = nv;
    if (nv != c->used + key_size)
        return emb::set_error(EMB_ERR_CAPACITY, "mode-0 valid list size mismatch");
    return EMB_OK;
}

void emb_slot_cache_restore(emb_slot_cache *c, const int64_t *slots, int64_t n) {
    if (!c || !slots) return;
    for (int64_t i = 0; i < n; ++i)
        if (slots[i] >= 0 && slots[i] < c->total) c->mark_free(slots[i]);
}

void emb_slot_cache_clear_pred(emb_slot_cache *c) {
    if (!c) return;
    for (int64_t s = 0; s < c->total; ++s) {
        if (!c->is_pred[s]) continue;
        c->mark_free(s);
        if (c->legacy) {
            c->is_pred[s] = 0;
            c->id[s] = -1;
        }
    }
}

int64_t emb_slot_cache_collect_valid(const emb_slot_cache *c, int64_t *valid) {
    if (!c || !valid) return emb::set_error(EMB_ERR_ARG, "null argument");
    int64_t n = 0;
    for (int64_t s = 0; s < c->total; ++s)
        if (c->mask[s]) valid[n++] = s;
    return n;
}

int emb_slot_cache_export(const emb_slot_cache *c, int64_t *id, uint8_t *mask, uint8_t *is_pred) {
    EMB_CHECK_ARG(c, "null cache");
    if (id) std::memcpy(id, c->id.data(), sizeof(int64_t) * c->id.size());
    if (mask) std::memcpy(mask, c->mask.data(), c->mask.size());
    if (is_pred) std::memcpy(is_pred, c->is_pred.data(), c->is_pred.size());
    return EMB_OK;
}

emb_page_pool *emb_page_pool_create(int32_t n_pages, uint64_t seed) {
    if (n_pages <= 0) {
        emb::set_error(EMB_ERR_ARG, "n_pages must be positive");
        return nullptr;
    }
    auto *p = new emb_page_pool();
    p->n_pages = n_pages;
    std::vector<int32_t> order((size_t)n_pages);
    for (int32_t i = 0; i < n_pages; ++i) order[(size_t)i] = i;
    if (seed != 0) {  // Fisher-Yates with mt19937_64
        emb::Mt64 g(seed);
        for (int32_t i = n_pages - 1; i > 0; --i) {
            int32_t j = (int32_t)(g.next() % (uint64_t)(i + 1));
            std::swap(order[(size_t)i], order[(size_t)j]);
        }
    }
    p->free_stack.assign(order.rbegin(), order.rend());
    return p;
}

// Caches still bound lose their pool: their pages read as unmapped (-1).
void emb_page_pool_destroy(emb_page_pool *p) {
    if (!p) return;
    for (emb_slot_cache *c : p->caches) {
        c->pool = nullptr;
        std::fill(c->pages.begin(), c->pages.end(), -1);
    }
    delete p;
}

int32_t emb_page_pool_free_count(const emb_page_pool *p) {
    return p ? (int32_t)p->free_stack.size() : -1;
}

int emb_slot_cache_bind_pool(emb_slot_cache *c, emb_page_pool *p) {
    EMB_CHECK_ARG(c && p, "null argument");
    EMB_CHECK_ARG(!c->pool || c->pool == p, "cache already bound to another pool");
    c->pool = p;
    {
        std::lock_guard<std::mutex> g(p->mu);
        p->caches.insert(c);
    }
    for (int64_t s = 0; s < c->total; ++s)
        if (c->mask[s]) {
            int rc = c->ensure_page(s);
            if (rc) return rc;
        }
    return EMB_OK;
}

int emb_slot_cache_map_range(emb_slot_cache *c, int64_t n_slots) {
    EMB_CHECK_ARG(c && c->pool, "cache has no page pool");
    EMB_CHECK_ARG(n_slots >= 0 && n_slots <= c->total, "n_slots out of range");
    for (int64_t s = 0; s < n_slots; s += EMB_PAGE_TOKENS) {
        int rc = c->ensure_page(s);
        if (rc) return rc;
    }
    return EMB_OK;
}

int emb_slot_cache_block_table(const emb_slot_cache *c, int32_t *bt, int64_t n) {
    EMB_CHECK_ARG(c && bt, "null argument");
    EMB_CHECK_ARG(n >= (int64_t)c->pages.size(), "block table needs %zu entries", c->pages.size());
    std::memcpy(bt, c->pages.data(), sizeof(int32_t) * c->pages.size());
    for (int64_t i = (int64_t)c->pages.size(); i < n; ++i) bt[i] = -1;
    return EMB_OK;
}

int emb_slot_cache_release_pages(emb_slot_cache *c) {
    EMB_CHECK_ARG(c, "null cache");
    if (!c->pool) return EMB_OK;
    std::lock_guard<std::mutex> g(c->pool->mu);
    for (auto &p : c->pages)
        if (p >= 0) {
            c->pool->free_stack.push_back(p);
            p = -1;
        }
    return EMB_OK;
}

int64_t emb_lingbot_kv_capacity(int64_t override_tokens, int64_t frame_chunk_size,
                                int64_t action_per_frame, int64_t n_suffix, int64_t attn_window,
                                int64_t latent_h, int64_t latent_w, int64_t patch_t,
                                int64_t patch_h, int64_t patch_w, int64_t seq) {
    if (override_tokens > 0) return std::max(override_tokens, seq);
    const int64_t latent_tokens =
        (patch_t > 0 && patch_h > 0 && patch_w > 0)
            ? (frame_chunk_size * latent_h * latent_w) / (patch_t * patch_h * patch_w)
            : 128;
    const int64_t action_tokens = n_suffix > 0 ? n_suffix : frame_chunk_size * action_per_frame;
    return std::max((attn_window / 2) * latent_tokens + (attn_window / 2) * action_tokens, seq);
}

int emb_synth_normal_bf16(uint64_t seed, int64_t n, uint16_t *out) {
    EMB_CHECK_ARG(out && n >= 0, "bad argument");
    emb::Mt64 g(seed);
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        const uint64_t a = g.next(), b = g.next();
        const double u1 = ((double)(a >> 11) + 0.5) * (1.0 / 9007199254740992.0);
        const double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
        const double r = std::sqrt(-2.0 * std::log(u1));
        out[i] = emb::f32_to_bf16_rne((float)(r * std::cos(two_pi * u2)));
        if (i + 1 < n) out[i + 1] = emb::f32_to_bf16_rne((float)(r * std::sin(two_pi * u2)));
    }
    return EMB_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Flex masks: models/lingbot_va.cpp:9274-9465.
// ---------------------------------------------------------------------------
struct emb_flex_meta {
    std::vector<int64_t> seq_ids, frame_ids, noise_ids, text_seq_ids;
    int64_t window_size = 0, block_size = 64;

    bool self_allowed(int64_t q, int64_t k) const {
        if (seq_ids[(size_t)q] < 0 || seq_ids[(size_t)q] != seq_ids[(size_t)k]) return false;
        const int64_t qf = frame_ids[(size_t)q], kf = frame_ids[(size_t)k];
        const int64_t qn = noise_ids[(size_t)q], kn = noise_ids[(size_t)k];
        const bool c2c = qn == 1 && kn == 1 && kf <= qf;
        const bool n2c = qn == 0 && kn == 1 && kf < qf;
        const bool n2n = qn == 0 && kn == 0 && kf == qf;
        return (c2c || n2c || n2n) && std::llabs(qf - kf) <= window_size;
    }
    bool cross_allowed(int64_t q, int64_t k) const {
        return seq_ids[(size_t)q] >= 0 && seq_ids[(size_t)q] == text_seq_ids[(size_t)k];
    }
};

template <typename Pred>
static int64_t brute_block_table(int64_t qn, int64_t kn, int64_t bs, Pred allowed, int32_t *row_ptr,
                                 int32_t *col_idx) {
    const int64_t qb = (qn + bs - 1) / bs, kb = (kn + bs - 1) / bs;
    int64_t nnz = 0;
    row_ptr[0] = 0;
    for (int64_t r = 0; r < qb; ++r) {
        const int64_t q0 = r * bs, q1 = std::min(q0 + bs, qn);
        for (int64_t c = 0; c < kb; ++c) {
            const int64_t k0 = c * bs, k1 = std::min(k0 + bs, kn);
            bool any = false;
            for (int64_t q = q0; q < q1 && !any; ++q)
                for (int64_t k = k0; k < k1 && !any; ++k) any = allowed(q, k);
            if (any) col_idx[nnz++] = (int32_t)c;
        }
        row_ptr[r + 1] = (int32_t)nnz;
    }
    return nnz;
}

extern "C" {

emb_flex_meta *emb_flex_meta_build(int64_t lat_b, int64_t lat_f, int64_t lat_h, int64_t lat_w,
                                   int64_t act_b, int64_t act_f, int64_t act_h, int64_t act_w,
                                   int64_t padded_length, int64_t chunk_size, int64_t window_size,
                                   int64_t pt, int64_t ph, int64_t pw, int64_t text_seq,
                                   int64_t block_size) {
    (void)act_b;  // the action loop runs inside the latent batch loop (:9298-9316)
    if (pt <= 0 || ph <= 0 || pw <= 0 || chunk_size <= 0 || block_size <= 0 || padded_length < 0) {
        emb::set_error(EMB_ERR_ARG, "bad flex meta shape");
        return nullptr;
    }
    auto *m = new emb_flex_meta();
    m->window_size = window_size;
    m->block_size = block_size;
    std::vector<int64_t> ls, lf, as, af;
    for (int64_t b = 0; b < lat_b; ++b) {
        for (int64_t f = 0; f < lat_f / pt; ++f)
            for (int64_t h = 0; h < lat_h / ph; ++h)
                for (int64_t w = 0; w < lat_w / pw; ++w) {
                    ls.push_back(b);
                    lf.push_back((f * pt) / chunk_size * 2);
                }
        for (int64_t f = 0; f < act_f; ++f)
            for (int64_t h = 0; h < act_h; ++h)
                for (int64_t w = 0; w < act_w; ++w) {
                    as.push_back(b);
                    af.push_back(f / chunk_size * 2 + 1);
                }
    }
    auto put = [&](const std::vector<int64_t> &s, const std::vector<int64_t> &f, int64_t noise) {
        m->seq_ids.insert(m->seq_ids.end(), s.begin(), s.end());
        m->frame_ids.insert(m->frame_ids.end(), f.begin(), f.end());
        m->noise_ids.insert(m->noise_ids.end(), s.size(), noise);
    };
    put(ls, lf, 0);
    put(ls, lf, 1);
    put(as, af, 0);
    put(as, af, 1);
    m->seq_ids.insert(m->seq_ids.end(), (size_t)padded_length, -1);
    m->frame_ids.insert(m->frame_ids.end(), (size_t)padded_length, -1);
    m->noise_ids.insert(m->noise_ids.end(), (size_t)padded_length, -1);
    for (int64_t b = 0; b < lat_b; ++b) m->text_seq_ids.insert(m->text_seq_ids.end(), (size_t)text_seq, b);
    return m;
}

void emb_flex_meta_destroy(emb_flex_meta *m) { delete m; }
int64_t emb_flex_meta_len(const emb_flex_meta *m) { return m ? (int64_t)m->seq_ids.size() : -1; }

int emb_flex_meta_ids(const emb_flex_meta *m, int64_t *seq_ids, int64_t *frame_ids, int64_t *noise_ids) {
    EMB_CHECK_ARG(m, "null meta");
    const size_t n = m->seq_ids.size() * sizeof(int64_t);
    if (seq_ids) std::memcpy(seq_ids, m->seq_ids.data(), n);
    if (frame_ids) std::memcpy(frame_ids, m->frame_ids.data(), n);
    if (noise_ids) std::memcpy(noise_ids, m->noise_ids.data(), n);
    return EMB_OK;
}

int emb_flex_self_allowed(const emb_flex_meta *m, int64_t q, int64_t k) {
    const int64_t n = emb_flex_meta_len(m);
    if (!m || q < 0 || k < 0 || q >= n || k >= n) return 0;
    return m->self_allowed(q, k) ? 1 : 0;
}

int emb_flex_cross_allowed(const emb_flex_meta *m, int64_t q, int64_t k) {
    if (!m || q < 0 || k < 0 || q >= (int64_t)m->seq_ids.size() || k >= (int64_t)m->text_seq_ids.size())
        return 0;
    return m->cross_allowed(q, k) ? 1 : 0;
}

int64_t emb_dense_block_table(int64_t seq_q, int64_t seq_k, int64_t block_size, int32_t *row_ptr,
                              int32_t *col_idx) {
    EMB_CHECK_ARG(row_ptr && col_idx && seq_q > 0 && seq_k > 0 && block_size > 0, "bad argument");
    return brute_block_table(seq_q, seq_k, block_size, [](int64_t, int64_t) { return true; }, row_ptr,
                             col_idx);
}

int64_t emb_self_block_table(const emb_flex_meta *m, int32_t *row_ptr, int32_t *col_idx) {
    EMB_CHECK_ARG(m && row_ptr && col_idx, "null argument");
    const int64_t n = (int64_t)m->seq_ids.size();
    return brute_block_table(n, n, m->block_size, [m](int64_t q, int64_t k) { return m->self_allowed(q, k); },
                             row_ptr, col_idx);
}

int64_t emb_cross_block_table(const emb_flex_meta *m, int32_t *row_ptr, int32_t *col_idx) {
    EMB_CHECK_ARG(m && row_ptr && col_idx, "null argument");
    return brute_block_table((int64_t)m->seq_ids.size(), (int64_t)m->text_seq_ids.size(), m->block_size,
                             [m](int64_t q, int64_t k) { return m->cross_allowed(q, k); }, row_ptr, col_idx);
}

int emb_self_token_mask(const emb_flex_meta *m, uint8_t *mask) {
    EMB_CHECK_ARG(m && mask, "null argument");
    const int64_t n = (int64_t)m->seq_ids.size();
    for (int64_t q = 0; q < n; ++q)
        for (int64_t k = 0; k < n; ++k) mask[q * n + k] = m->self_allowed(q, k) ? 1 : 0;
    return EMB_OK;
}

}  // extern "C"
