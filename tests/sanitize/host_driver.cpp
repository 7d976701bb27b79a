// Exercises the library's host code (slot cache, page pool, capacity, flex
// masks, call-site masks, the synthetic generator) under AddressSanitizer and
// UndefinedBehaviorSanitizer: every entry point with valid arguments,
// eviction cycles, and the error paths.  Exits nonzero on a failed check; the
// sanitizers abort on their own findings.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "emb_kv.h"

#define CHECK(x)                                                   \
    do {                                                           \
        if (!(x)) {                                                \
            std::fprintf(stderr, "check failed: %s (line %d)\n", #x, __LINE__); \
            std::exit(1);                                          \
        }                                                          \
    } while (0)

static void slot_cache_cycles() {
    const int64_t cap = 200;
    for (int legacy = 0; legacy < 2; ++legacy) {
        emb_slot_cache *c = emb_slot_cache_create(cap, legacy);
        CHECK(c && emb_slot_cache_capacity(c) == cap);
        emb_page_pool *pool = emb_page_pool_create(64, 7);
        CHECK(pool && emb_slot_cache_bind_pool(c, pool) == EMB_OK);
        CHECK(emb_slot_cache_map_range(c, 48) == EMB_OK);
        std::vector<int64_t> slots(cap), valid(cap), ids(cap);
        std::vector<uint8_t> mask(cap), pred(cap);
        std::vector<int32_t> bt((cap + 15) / 16);
        for (int round = 0; round < 40; ++round) {
            const int64_t k = 13 + round % 29;
            const int mode = round % 3;
            if (mode == 0) {
                int64_t n_valid = 0;
                CHECK(emb_slot_cache_prepare_mode0(c, k, slots.data(), valid.data(), &n_valid) == EMB_OK);
                CHECK(n_valid >= 0 && n_valid <= cap);
                emb_slot_cache_restore(c, slots.data(), k);
            } else {
                CHECK(emb_slot_cache_update_meta(c, k, mode == 1, slots.data()) == EMB_OK);
            }
            if (round % 7 == 6) emb_slot_cache_clear_pred(c);
            const int64_t nv = emb_slot_cache_collect_valid(c, valid.data());
            CHECK(nv >= 0 && nv <= cap);
            CHECK(emb_slot_cache_used_count(c) >= 0 && emb_slot_cache_pred_count(c) >= 0);
            CHECK(emb_slot_cache_export(c, ids.data(), mask.data(), pred.data()) == EMB_OK);
            CHECK(emb_slot_cache_block_table(c, bt.data(), (int64_t)bt.size()) == EMB_OK);
            (void)emb_slot_cache_next_id(c);
        }
        int64_t s1[1];
        CHECK(emb_slot_cache_allocate(c, cap + 1, s1) != EMB_OK);  // more than the capacity
        CHECK(emb_slot_cache_release_pages(c) == EMB_OK);
        CHECK(emb_page_pool_free_count(pool) == 64);
        emb_slot_cache_destroy(c);
        emb_page_pool_destroy(pool);
    }
    CHECK(emb_slot_cache_create(0, 0) == nullptr);
    CHECK(emb_lingbot_kv_capacity(0, 4, 4, 0, 30, 8, 16, 1, 2, 2, 0) > 0);
}

static void flex_tables() {
    const int64_t args[3][16] = {{1, 2, 2, 2, 1, 2, 1, 1, 1, 1, 4, 1, 1, 1, 5, 4},
                                 {1, 4, 4, 4, 1, 4, 2, 1, 3, 2, 1, 2, 2, 2, 7, 8},
                                 {2, 2, 2, 4, 1, 2, 2, 1, 0, 1, 0, 1, 1, 2, 3, 4}};
    for (const auto &a : args) {
        emb_flex_meta *m = emb_flex_meta_build(a[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7], a[8], a[9], a[10],
                                               a[11], a[12], a[13], a[14], a[15]);
        CHECK(m);
        const int64_t n = emb_flex_meta_len(m);
        std::vector<int64_t> s(n), f(n), z(n);
        CHECK(emb_flex_meta_ids(m, s.data(), f.data(), z.data()) == EMB_OK);
        for (int64_t q = 0; q < n; ++q)
            for (int64_t k = 0; k < n; ++k) {
                (void)emb_flex_self_allowed(m, q, k);
                (void)emb_flex_cross_allowed(m, q, k);
            }
        const int64_t qb = (n + a[15] - 1) / a[15];
        std::vector<int32_t> rp(qb + 1), ci(qb * qb + qb * 64);
        CHECK(emb_self_block_table(m, rp.data(), ci.data()) >= 0);
        CHECK(emb_cross_block_table(m, rp.data(), ci.data()) >= 0);
        std::vector<uint8_t> tm(n * n);
        CHECK(emb_self_token_mask(m, tm.data()) == EMB_OK);
        emb_flex_meta_destroy(m);
    }
    std::vector<int32_t> rp(4), ci(16);
    CHECK(emb_dense_block_table(10, 12, 4, rp.data(), ci.data()) == 9);
    CHECK(emb_dense_block_table(0, 12, 4, rp.data(), ci.data()) == EMB_ERR_ARG);
}

static void call_masks() {
    std::vector<int32_t> mod = {0, 1, 1, 0, 1, 1, 0, 0, 1, 0, 1};
    std::vector<int32_t> group_of(mod.size());
    CHECK(emb_hy_patch_groups(mod.data(), (int32_t)mod.size(), group_of.data()) == 2);
    const int64_t n = (int64_t)mod.size();
    std::vector<uint8_t> allow(n * n);
    std::vector<uint16_t> f16(n * n);
    CHECK(emb_hy_prefix_mask(n, group_of.data(), allow.data(), f16.data()) == EMB_OK);
    CHECK(emb_hy_prefix_mask(n, nullptr, allow.data(), nullptr) == EMB_OK);
    std::vector<uint8_t> sa(5 * (n + 5));
    CHECK(emb_hy_suffix_mask(n, 5, sa.data(), nullptr) == EMB_OK);
    CHECK(emb_groot_layer_mask_kind(4, 2) == 1 && emb_groot_layer_mask_kind(2, 2) == 2);
    std::vector<int32_t> valid = {1, 1, 1, 0}, img = {0, 1, 1, 1};
    std::vector<float> tmask(3 * 4), imask(3 * 4);
    CHECK(emb_groot_cross_masks(valid.data(), img.data(), 4, 3, tmask.data(), imask.data()) == EMB_OK);
    std::vector<uint8_t> pv = {1, 1, 0, 1, 1};
    std::vector<float> pm(25), fm(2 * 7), cm(2 * 5);
    CHECK(emb_smolvla_masks(pv.data(), 5, 2, pm.data(), fm.data(), cm.data()) == EMB_OK);
    std::vector<int32_t> pp(5), sp(2), cp(2);
    CHECK(emb_smolvla_positions(pv.data(), 5, 2, pp.data(), sp.data(), cp.data()) == EMB_OK);
    CHECK(pp[4] == 3 && sp[0] == 4 && cp[1] == 1);
    CHECK(emb_hy_patch_groups(nullptr, 3, group_of.data()) == EMB_ERR_ARG);
    CHECK(emb_smolvla_masks(pv.data(), 0, 2, nullptr, nullptr, nullptr) == EMB_ERR_ARG);
}

int main() {
    slot_cache_cycles();
    flex_tables();
    call_masks();
    std::vector<uint16_t> r(1001);
    CHECK(emb_synth_normal_bf16(5, 1001, r.data()) == EMB_OK);
    std::printf("host driver ok\n");
    return 0;
}
