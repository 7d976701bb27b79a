/* Exercises the CPU oracle (oracle/emb_oracle.c) under AddressSanitizer and
 * UndefinedBehaviorSanitizer at small sizes: slot cache cycles, paged
 * append/gather, flex tables and attentions, GQA attention with masks, the CPU
 * baseline attention, Marlin packing and the W8 GEMM, and both RoPE forms. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "emb_oracle.h"

#define CHECK(x)                                                         \
    do {                                                                 \
        if (!(x)) {                                                      \
            fprintf(stderr, "check failed: %s (line %d)\n", #x, __LINE__); \
            exit(1);                                                     \
        }                                                                \
    } while (0)

static void *xcalloc(size_t n, size_t sz) {
    void *p = calloc(n, sz);
    CHECK(p);
    return p;
}

int main(void) {
    /* slot cache */
    for (int legacy = 0; legacy < 2; ++legacy) {
        orc_slot_cache *c = orc_cache_new(100, legacy);
        int64_t *slots = xcalloc(100, sizeof(int64_t)), *valid = xcalloc(100, sizeof(int64_t));
        for (int r = 0; r < 30; ++r) {
            const int64_t k = 7 + r % 19;
            int64_t nv = 0;
            if (r % 3 == 0) {
                CHECK(orc_cache_prepare_mode0(c, k, slots, valid, &nv));
                orc_cache_restore(c, slots, k);
            } else {
                CHECK(orc_cache_update_meta(c, k, r % 3 == 1, slots));
            }
            if (r % 5 == 4) orc_cache_clear_pred(c);
            CHECK(orc_cache_collect_valid(c, valid) <= 100);
            (void)orc_cache_used_count(c);
            (void)orc_cache_pred_count(c);
            (void)orc_cache_next_id(c);
        }
        CHECK(!orc_cache_allocate(c, 101, slots));
        free(slots);
        free(valid);
        orc_cache_free(c);
    }
    (void)orc_lingbot_capacity(0, 4, 4, 0, 30, 8, 16, 1, 2, 2, 0);

    /* paged movement */
    const int64_t H = 2, D = 64, n = 40, cap = 64;
    uint16_t *k = xcalloc(n * H * D, 2), *v = xcalloc(n * H * D, 2);
    orc_fill_normal_bf16(1, n * H * D, k);
    orc_fill_normal_bf16(2, n * H * D, v);
    int32_t bt[4] = {3, -1, 0, 2}, sl[40], val[40];
    for (int i = 0; i < n; ++i) sl[i] = (i * 7) % (int)cap;
    for (int i = 0; i < n; ++i) val[i] = i % 3 == 0 ? -1 : sl[i];
    uint16_t *kp = xcalloc(4 * H * 16 * D, 2), *vp = xcalloc(4 * H * 16 * D, 2);
    orc_paged_append(k, v, H * D, n, H, D, sl, bt, cap, kp, vp);
    uint16_t *ko = xcalloc(n * H * D, 2), *vo = xcalloc(n * H * D, 2);
    orc_paged_gather(kp, vp, val, n, H, D, bt, cap, ko, vo);
    uint16_t *ck = xcalloc(cap * H * D, 2), *cv = xcalloc(cap * H * D, 2);
    orc_slot_update(k, v, ck, cv, sl, n, H, D, cap);
    orc_slot_gather(ck, cv, val, ko, vo, n, H, D, cap);

    /* flex tables and attentions */
    orc_flex_meta *m = orc_flex_meta_build(1, 4, 4, 4, 1, 4, 2, 1, 3, 2, 1, 2, 2, 2, 7, 8);
    CHECK(m);
    const int64_t L = m->n, qb = (L + 7) / 8, tb = (m->n_text + 7) / 8;
    int64_t *rp = xcalloc(qb + 1, sizeof(int64_t)), *ci = xcalloc(qb * (qb > tb ? qb : tb) + 1, sizeof(int64_t));
    CHECK(orc_self_block_table(m, rp, ci) >= 0);
    (void)orc_max_row_nnz(rp, qb);
    CHECK(orc_cross_block_table(m, rp, ci) >= 0);
    uint8_t *tm = xcalloc(L * L, 1);
    orc_self_token_mask(m, tm);
    float *qf = xcalloc(L * H * D, 4), *kf = xcalloc(L * H * D, 4), *vf = xcalloc(L * H * D, 4), *of = xcalloc(L * H * D, 4);
    for (int64_t i = 0; i < L * H * D; ++i) {
        qf[i] = (float)((i * 37) % 11) / 11.0f - 0.5f;
        kf[i] = (float)((i * 17) % 13) / 13.0f - 0.5f;
        vf[i] = (float)((i * 7) % 5) / 5.0f;
    }
    orc_dense_masked_attention(qf, kf, vf, tm, L, H, D, of);
    int64_t *drp = xcalloc(qb + 1, sizeof(int64_t)), *dci = xcalloc(qb * qb + 1, sizeof(int64_t));
    CHECK(orc_dense_block_table(L, L, 8, drp, dci) == qb * qb);
    int32_t *rp32 = xcalloc(qb + 1, 4), *ci32 = xcalloc(qb * qb + 1, 4);
    for (int64_t i = 0; i <= qb; ++i) rp32[i] = (int32_t)drp[i];
    for (int64_t i = 0; i < qb * qb; ++i) ci32[i] = (int32_t)dci[i];
    orc_flex_attention(qf, kf, vf, rp32, ci32, tm, of, L, L, H, D, 8, 0.125f);
    int32_t *vs = xcalloc(L, 4);
    for (int64_t i = 0; i < L; ++i) vs[i] = i % 4 == 0 ? -1 : (int32_t)i;
    orc_runtime_kv_attn(qf, kf, vf, vs, of, L, L, H, D, 0.125f, 1);
    orc_flex_meta_free(m);

    /* GQA attention with every mask form, rows, and the CPU baseline */
    const int64_t nq = 9, nk = 33, hq = 4, hkv = 2;
    uint16_t *qb16 = xcalloc(nq * hq * D, 2), *kb16 = xcalloc(nk * hkv * D, 2), *vb16 = xcalloc(nk * hkv * D, 2);
    orc_fill_normal_bf16(3, nq * hq * D, qb16);
    orc_fill_normal_bf16(4, nk * hkv * D, kb16);
    orc_fill_normal_bf16(5, nk * hkv * D, vb16);
    uint8_t *allow = xcalloc(nq * nk, 1);
    float *add = xcalloc(nq * nk, 4), *out = xcalloc(nq * hq * D, 4);
    for (int64_t i = 0; i < nq * nk; ++i) {
        allow[i] = i % 5 != 0;
        add[i] = (float)(i % 3) - 1.0f;
    }
    int64_t rows[3] = {0, 4, 8};
    orc_gqa_attention_bf16(qb16, kb16, vb16, nq, nk, hq, hkv, D, 0.125f, allow, add, 0, -1, nk - nq, NULL, 0, 2, out);
    orc_gqa_attention_bf16(qb16, kb16, vb16, nq, nk, hq, hkv, D, 0.125f, NULL, NULL, 4, 2, 10, rows, 3, 1, out);
    float *q32 = xcalloc(nq * hq * D, 4), *k32 = xcalloc(nk * hkv * D, 4), *v32 = xcalloc(nk * hkv * D, 4);
    for (int64_t i = 0; i < nq * hq * D; ++i) q32[i] = orc_bf16_to_f32(qb16[i]);
    for (int64_t i = 0; i < nk * hkv * D; ++i) {
        k32[i] = orc_bf16_to_f32(kb16[i]);
        v32[i] = orc_bf16_to_f32(vb16[i]);
    }
    CHECK(orc_cpu_attention_f32(q32, k32, v32, nq, nk, hq, hkv, D, 0.125f, 2, out) == 2);

    /* Marlin packing and the W8 GEMM */
    const int64_t K = 32, N = 128, M = 5;
    int8_t *w = xcalloc(K * N, 1);
    for (int64_t i = 0; i < K * N; ++i) w[i] = (int8_t)((i * 29) % 255 - 127);
    int32_t *qw = xcalloc(K * N / 4, 4);
    orc_marlin_pack_w8(w, K, N, qw);
    CHECK(orc_marlin_unpack_w8(qw, K, N, 3, 77) == w[3 * N + 77]);
    (void)orc_marlin_dst_byte(5, 9, N);
    (void)orc_marlin_scale_index(9);
    uint16_t *s = xcalloc(N, 2), *ss = xcalloc(N, 2);
    orc_fill_normal_bf16(6, N, s);
    orc_marlin_pack_scales(s, N, ss);
    uint16_t *x = xcalloc(M * K, 2), *yb = xcalloc(M * N, 2);
    float *yf = xcalloc(M * N, 4);
    orc_fill_normal_bf16(7, M * K, x);
    orc_w8a16_gemm(x, qw, ss, M, K, N, NULL, 0, 2, yb, yf);
    int64_t r2[2] = {1, 4};
    orc_w8a16_gemm(x, qw, ss, M, K, N, r2, 2, 1, yb, yf);

    /* RoPE forms */
    const int64_t T = 6, HH = 3;
    uint16_t *xr = xcalloc(T * HH * D, 2), *g = xcalloc(D, 2), *yr = xcalloc(T * HH * D, 2);
    orc_fill_normal_bf16(8, T * HH * D, xr);
    orc_fill_normal_bf16(9, D, g);
    int32_t pids[3 * 6] = {0, 1, 2, 3, 4, 5, 5, 4, 3, 2, 1, 0, 2, 2, 2, 2, 2, 2};
    for (int kind = 0; kind < 3; ++kind) orc_head_norm_rope(xr, HH * D, T, HH, D, g, 1e-6f, kind, 1e6f, 3, pids, yr, HH * D);
    float *xf = xcalloc(T * HH * D, 4), *yf2 = xcalloc(T * HH * D, 4);
    for (int64_t i = 0; i < T * HH * D; ++i) xf[i] = orc_bf16_to_f32(xr[i]);
    orc_neox_rope_f32(xf, HH * D, T, HH, D, NULL, 816, 10000.0f, yf2, HH * D);
    orc_neox_rope_f32(xf, HH * D, T, HH, D, pids, 0, 10000.0f, yf2, HH * D);

    free(k); free(v); free(kp); free(vp); free(ko); free(vo); free(ck); free(cv);
    free(rp); free(ci); free(tm); free(qf); free(kf); free(vf); free(of); free(drp); free(dci); free(rp32); free(ci32); free(vs);
    free(qb16); free(kb16); free(vb16); free(allow); free(add); free(out); free(q32); free(k32); free(v32);
    free(w); free(qw); free(s); free(ss); free(x); free(yb); free(yf); free(xr); free(g); free(yr); free(xf); free(yf2);
    printf("oracle driver ok\n");
    return 0;
}
