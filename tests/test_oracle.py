"""Pins the CPU oracle (oracle/emb_oracle.c) before it is trusted as the checker.

Each test is a known answer derived by hand from the reference's documented
semantics, a known answer the reference itself holds, an invariant, or a
reduction to a library routine (numpy) -- chosen so that a plausible slip
(wrong index, swapped operand, dropped term) fails.
"""
from __future__ import annotations

import math

import numpy as np
import pytest


# ---------------- random generation ----------------
def test_mt19937_64_known_answer(orc):
    # C++ standard [rand.predef]: the 10000th output of a default-constructed
    # std::mt19937_64 (seed 5489) is 9981545732273789042.
    assert orc.lib().orc_mt64_nth(5489, 10000) == 9981545732273789042


def test_bf16_round_to_nearest_even(orc):
    import torch
    L = orc.lib()
    assert L.orc_f32_to_bf16(1.0) == 0x3F80
    assert L.orc_f32_to_bf16(1.0 + 2.0 ** -8) == 0x3F80          # tie -> even
    assert L.orc_f32_to_bf16(1.0 + 3 * 2.0 ** -8) == 0x3F82      # tie -> even (up)
    assert L.orc_f32_to_bf16(-2.5) == 0xC020
    x = np.random.default_rng(1).standard_normal(20000).astype(np.float32) * 37
    ours = orc.f32_to_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    assert np.array_equal(np.array([L.orc_f32_to_bf16(float(v)) for v in x[:500]], np.uint16), ref[:500])


def test_normal_generator_statistics(orc):
    z = orc.bf16_to_f32(orc.normal_bf16(0xE3BD0001, 400000)).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    assert abs(np.mean(np.abs(z) < 1.0) - 0.6827) < 0.005  # one-sigma mass


# ---------------- slot cache: hand-derived scenarios ----------------
def test_slot_cache_fill_and_whole_chunk_eviction(orc):
    c = orc.Cache(6)
    assert list(c.update_meta(2, 0)) == [0, 1] and c.next_id() == 1
    assert list(c.update_meta(2, 1)) == [2, 3]
    assert list(c.update_meta(2, 0)) == [4, 5]
    ids, m, pr = c.state()
    assert list(ids) == [0, 0, 1, 1, 2, 2] and list(m) == [1] * 6 and list(pr) == [0, 0, 1, 1, 0, 0]
    # full: the oldest chunk (id 0, slots 0-1) is evicted; the new id is max+1
    assert list(c.update_meta(2, 0)) == [0, 1]
    ids, m, pr = c.state()
    assert list(ids) == [3, 3, 1, 1, 2, 2]
    # valid slots are in ascending slot order, not age order
    assert list(c.collect_valid()) == [0, 1, 2, 3, 4, 5]
    assert c.used_count() == 6 and c.pred_count() == 2


def test_slot_cache_clear_pred_and_mode0(orc):
    c = orc.Cache(8)
    c.update_meta(3, 0)      # slots 0-2 id 0
    c.update_meta(2, 1)      # slots 3-4 id 1 (pred)
    c.clear_pred()           # non-legacy: mask 0, id/is_pred kept
    ids, m, pr = c.state()
    assert list(m) == [1, 1, 1, 0, 0, 0, 0, 0]
    assert list(ids[:5]) == [0, 0, 0, 1, 1] and list(pr[:5]) == [0, 0, 0, 1, 1]
    assert c.pred_count() == 0 and c.next_id() == 1
    s, v = c.prepare_mode0(2)  # temp slots 3-4, id 1, invisible afterwards
    assert list(s) == [3, 4] and list(v) == [0, 1, 2, 3, 4]
    ids, m, pr = c.state()
    assert list(m) == [1, 1, 1, 0, 0, 0, 0, 0] and list(ids[3:5]) == [1, 1] and list(pr[3:5]) == [0, 0]
    assert list(c.collect_valid()) == [0, 1, 2]


def test_slot_cache_legacy_clear_pred(orc):
    c = orc.Cache(4, legacy=True)
    c.update_meta(2, 1)
    c.clear_pred()
    ids, m, pr = c.state()
    assert list(ids) == [-1] * 4 and list(m) == [0] * 4 and list(pr) == [0] * 4


def test_slot_cache_eviction_tie_rule_and_failure(orc):
    c = orc.Cache(4)
    c.update_meta(3, 0)  # slots 0-2 id 0
    # need 2 more with 1 free: evict ONE of the id-0 slots.  std::sort leaves the
    # choice open in the reference; the oracle takes the lowest slot.
    assert list(c.update_meta(2, 0)) == [0, 3]
    ids, m, _ = c.state()
    assert list(ids) == [1, 0, 0, 1]
    # a request larger than capacity fails, after evicting everything
    assert c.update_meta(5, 0) is None
    assert c.used_count() == 0


def test_slot_cache_mode0_restore_keeps_ids(orc):
    c = orc.Cache(4)
    c.update_meta(2, 0)
    s = c.update_meta(2, 0)   # mode-0 without the fast path: insert then restore
    c.restore(s)
    ids, m, _ = c.state()
    assert list(m) == [1, 1, 0, 0] and list(ids) == [0, 0, 1, 1]
    assert c.next_id() == 1


def test_lingbot_capacity_known_answers(orc):
    # LIBERO defaults (models/lingbot_va.cpp:9231-9248): window 30, 4 frames a
    # chunk, 4 actions a frame, latent 8x16, patch (1,2,2):
    # latent tokens 4*8*16/4 = 128, action tokens 16 -> 15*128 + 15*16 = 2160.
    assert orc.lingbot_capacity(seq=100) == 2160
    # robotwin_tshape: window 72, 2 frames, 16 actions, latent 24x20:
    # latent 2*24*20/4 = 240, action 32 -> 36*240 + 36*32 = 9792
    assert orc.lingbot_capacity(frame_chunk_size=2, action_per_frame=16, attn_window=72,
                                latent_h=24, latent_w=20, seq=10) == 9792
    assert orc.lingbot_capacity(seq=5000) == 5000                    # never below seq
    assert orc.lingbot_capacity(override_tokens=14040, seq=1560) == 14040
    assert orc.lingbot_capacity(override_tokens=100, seq=1560) == 1560
    assert orc.lingbot_capacity(patch_t=0, seq=1) == 15 * 128 + 15 * 16  # 128-token default


# ---------------- paged layout == token-slot layout (bit-exact chain) ----------------
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_paged_matches_slot_semantics(orc, seed):
    rng = np.random.default_rng(seed)
    H, D, cap = 3, 16, 70
    n = 40
    k = rng.integers(0, 65535, (n, H, D), dtype=np.uint16)
    v = rng.integers(0, 65535, (n, H, D), dtype=np.uint16)
    slots = rng.choice(np.arange(-3, cap + 3), n, replace=False).astype(np.int32)
    n_pages = (cap + 15) // 16
    bt = rng.permutation(n_pages + 5)[:n_pages].astype(np.int32)
    ck = np.zeros((cap, H, D), np.uint16)
    cv = np.zeros((cap, H, D), np.uint16)
    orc.slot_update(k, v, ck, cv, slots, H, D, cap)
    kp = np.zeros(((n_pages + 5) * H * 16 * D,), np.uint16)
    vpool = np.zeros_like(kp)
    orc.paged_append(k, v, H * D, slots, bt, H, D, cap, kp, vpool)
    valid = np.sort(slots[(slots >= 0) & (slots < cap)])
    valid = np.concatenate([valid, [-1, cap]]).astype(np.int32)  # out-of-range rows untouched
    g1k = np.full((len(valid), H, D), 7, np.uint16); g1v = g1k.copy()
    g2k = g1k.copy(); g2v = g1k.copy()
    orc.slot_gather(ck, cv, valid, H, D, cap, g1k, g1v)
    orc.paged_gather(kp, vpool, valid, bt, H, D, cap, g2k, g2v)
    assert np.array_equal(g1k, g2k) and np.array_equal(g1v, g2v)
    # the gathered rows are exactly the appended source rows
    src_of = {int(s): i for i, s in enumerate(slots)}
    for i, s in enumerate(valid[:-2]):
        assert np.array_equal(g2k[i], k[src_of[int(s)]]) and np.array_equal(g2v[i], v[src_of[int(s)]])
    assert np.all(g2k[-2:] == 7)
    # layout: K row t of page p is contiguous; V is stored [d][t]
    s0 = int(valid[0]); p0 = int(bt[s0 // 16]); t0 = s0 % 16
    base = (p0 * H + 1) * 16 * D
    assert np.array_equal(kp[base + t0 * D: base + (t0 + 1) * D], k[src_of[s0], 1])
    assert vpool[(p0 * H + 1) * D * 16 + 5 * 16 + t0] == v[src_of[s0], 1, 5]


# ---------------- flex masks ----------------
def _small_meta(orc, window=4):
    # latent (b=1, f=2, h=2, w=2), patch 1 -> 8 tokens a copy, frames (f*1)/1*2 = {0, 2};
    # action (f=2, h=1, w=1) -> frames f*2+1 = {1, 3}; padding 1.
    # order: latent noisy [0,8), latent clean [8,16), action noisy 16-17,
    # action clean 18-19, pad 20.
    return orc.FlexMeta(1, 2, 2, 2, 1, 2, 1, 1, 1, 1, window, 1, 1, 1, 5, 4)


def test_flex_predicate_known_answers(orc):
    m = _small_meta(orc)
    A = lambda q, k: orc.lib().orc_flex_self_allowed(m.h, q, k)
    assert A(4, 8) == 1      # noisy f2 -> clean f0: noise2clean needs kf < qf
    assert A(4, 12) == 0     # noisy f2 -> clean f2: not strictly earlier
    assert A(4, 5) == 1      # noisy f2 -> noisy f2: same frame
    assert A(4, 0) == 0      # noisy f2 -> noisy f0
    assert A(12, 8) == 1     # clean f2 -> clean f0: clean2clean kf <= qf
    assert A(12, 13) == 1    # clean -> clean same frame
    assert A(8, 12) == 0     # clean f0 -> clean f2: future
    assert A(8, 0) == 0      # clean never sees noisy
    assert A(16, 8) == 1     # action noisy f1 -> latent clean f0
    assert A(16, 12) == 0    # action noisy f1 -> latent clean f2 (future)
    assert A(18, 19) == 0    # action clean f1 -> action clean f3
    assert A(19, 18) == 1
    assert A(20, 20) == 0 and A(3, 20) == 0   # padding sees and is seen by nothing
    m1 = _small_meta(orc, window=1)
    assert orc.lib().orc_flex_self_allowed(m1.h, 12, 8) == 0  # |2-0| > window
    assert orc.lib().orc_flex_cross_allowed(m.h, 3, 4) == 1
    assert orc.lib().orc_flex_cross_allowed(m.h, 20, 0) == 0


def test_flex_block_tables_brute_force(orc):
    m = _small_meta(orc)
    n, bs = 21, 4
    tm = orc.self_token_mask(m, n)
    rp, ci = orc.self_block_table(m, n, bs)
    qb = (n + bs - 1) // bs
    for r in range(qb):
        want = [c for c in range(qb) if tm[r * bs:(r + 1) * bs, c * bs:(c + 1) * bs].any()]
        assert list(ci[rp[r]:rp[r + 1]]) == want
    rp, ci = orc.dense_block_table(9, 13, 4)
    assert list(rp) == [0, 4, 8, 12] and list(ci) == [0, 1, 2, 3] * 3
    rp, ci = orc.cross_block_table(m, n, 5, bs)
    assert list(ci[rp[5]:rp[6]]) == []         # block 5 holds only the pad token
    assert orc.lib().orc_max_row_nnz(rp.ctypes.data_as(orc.i64p), qb) == 2


# ---------------- attention ----------------
def _smoke_inputs():
    # lingbot_flex_attn_cuda_smoke, kernels/lingbot/lingbot_flex_attn_cuda.cu:1033-1048
    S, H, D = 8, 2, 8
    i = np.arange(S * H * D, dtype=np.float32)
    q = (np.sin(i * np.float32(0.017)) * np.float32(0.2)).astype(np.float32)
    k = (np.cos(i * np.float32(0.019)) * np.float32(0.15)).astype(np.float32)
    v = (np.sin(i * np.float32(0.023)) * np.float32(0.3)).astype(np.float32)
    s, t = np.meshgrid(np.arange(S), np.arange(S), indexing="ij")
    mask = ((t <= s) & (s - t <= 4)).astype(np.uint8)
    return S, H, D, q, k, v, mask


def test_reference_flex_smoke_known_answer(orc):
    S, H, D, q, k, v, mask = _smoke_inputs()
    scale = 1.0 / math.sqrt(D)
    dense = orc.dense_masked_attention(q, k, v, mask, S, H, D)
    flex = orc.flex_attention(q, k, v, [0, 1, 3], [0, 0, 1], mask, S, S, H, D, 4, scale)
    assert np.abs(flex - dense).max() < 1e-5  # the reference's own pass criterion
    # and the same numbers from numpy's softmax over a masked score matrix
    qh, kh, vh = (x.reshape(S, H, D).astype(np.float64) for x in (q, k, v))
    sc = np.einsum("shd,thd->hst", qh, kh) * scale
    sc = np.where(mask[None].astype(bool), sc, -np.inf)
    p = np.exp(sc - sc.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ref = np.einsum("hst,thd->shd", p, vh).reshape(-1)
    assert np.abs(dense - ref).max() < 1e-6


def _np_attention(q, k, v, hq, hkv, scale, allow=None, add=None):
    """softmax(q k^T * scale + add) v with numpy matmul; q [nq,hq,d], k/v [nk,hkv,d]."""
    G = hq // hkv
    qh = q.astype(np.float64).transpose(1, 0, 2)
    kh = np.repeat(k.astype(np.float64).transpose(1, 0, 2), G, axis=0)
    vh = np.repeat(v.astype(np.float64).transpose(1, 0, 2), G, axis=0)
    s = qh @ kh.transpose(0, 2, 1) * scale
    if add is not None:
        s = s + add[None]
    if allow is not None:
        s = np.where(allow[None].astype(bool), s, -np.inf)
    mx = s.max(-1, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0)
    p = np.exp(s - mx)
    den = p.sum(-1, keepdims=True)
    o = (p @ vh) / np.where(den > 0, den, 1)
    o = np.where(den > 0, o, 0)
    return o.transpose(1, 0, 2)


@pytest.mark.parametrize("hq,hkv", [(8, 1), (8, 2), (4, 4)])
def test_gqa_oracle_matches_numpy(orc, hq, hkv):
    rng = np.random.default_rng(hq * 10 + hkv)
    nq, nk, d = 5, 23, 32
    qb = orc.f32_to_bf16(rng.standard_normal((nq, hq, d)).astype(np.float32))
    kb = orc.f32_to_bf16(rng.standard_normal((nk, hkv, d)).astype(np.float32))
    vb = orc.f32_to_bf16(rng.standard_normal((nk, hkv, d)).astype(np.float32))
    allow = (rng.random((nq, nk)) < 0.7).astype(np.uint8)
    allow[2] = 0  # an empty row gives 0
    add = rng.standard_normal((nq, nk)).astype(np.float32)
    scale = 1 / math.sqrt(d)
    out = orc.gqa_attention(qb, kb, vb, nq, nk, hq, hkv, d, scale, allow=allow, add=add)
    ref = _np_attention(orc.bf16_to_f32(qb), orc.bf16_to_f32(kb), orc.bf16_to_f32(vb), hq, hkv,
                        scale, allow=allow, add=add)
    assert np.abs(out - ref).max() < 1e-5
    assert np.all(out[2] == 0)


def test_gqa_head_mapping_and_special_cases(orc):
    # q = 0 gives uniform weights: each q head returns the mean V of its kv head,
    # and q head h must read kv head h // (hq/hkv).
    nq, nk, hq, hkv, d = 3, 6, 8, 2, 16
    q = np.zeros((nq, hq, d), np.uint16)
    v = np.zeros((nk, hkv, d), np.float32)
    v[:, 0] = np.arange(nk)[:, None]          # mean 2.5
    v[:, 1] = -np.arange(nk)[:, None] * 2     # mean -5
    k = orc.f32_to_bf16(np.random.default_rng(0).standard_normal((nk, hkv, d)).astype(np.float32))
    out = orc.gqa_attention(q, k, orc.f32_to_bf16(v), nq, nk, hq, hkv, d, 0.1)
    assert np.allclose(out[:, :4], 2.5) and np.allclose(out[:, 4:], -5.0)
    # a single visible key returns that key's V row exactly
    allow = np.zeros((nq, nk), np.uint8)
    allow[:, 3] = 1
    out = orc.gqa_attention(q, k, orc.f32_to_bf16(v), nq, nk, hq, hkv, d, 0.1, allow=allow)
    assert np.all(out[:, :4] == 3.0) and np.all(out[:, 4:] == -6.0)
    # chunk-causal rule on positions: chunk 2, queries at positions 4..6 of 6 keys
    # (q_pos0 = nk - nq = 3): position p sees keys j with j//2 <= p//2.
    out_c = orc.gqa_attention(q, k, orc.f32_to_bf16(v), nq, nk, hq, hkv, d, 0.1, chunk=2)
    vis = [[j for j in range(nk) if j // 2 <= (3 + i) // 2] for i in range(nq)]
    for i in range(nq):
        assert np.allclose(out_c[i, 0], np.mean(vis[i])), (i, out_c[i, 0, 0])


def test_runtime_kv_attention_quirk(orc):
    # online/warp kernels: a negative slot adds exp(0 - max) to the denominator
    # and no V row.  With q = 0 every score is 0: out = sum(v_valid) / n_all.
    H, D, cap = 2, 8, 5
    q = np.zeros(1 * H * D, np.float32)
    ck = np.random.default_rng(3).standard_normal(cap * H * D).astype(np.float32)
    cv = np.arange(cap * H * D, dtype=np.float32) % 7
    valid = [4, -1, 1]
    out = orc.runtime_kv_attn(q, ck, cv, valid, 1, H, D, 0.3).reshape(H, D)
    cvr = cv.reshape(cap, H, D)
    assert np.allclose(out, (cvr[4] + cvr[1]) / 3)
    out2 = orc.runtime_kv_attn(q, ck, cv, valid, 1, H, D, 0.3, online_quirk=False).reshape(H, D)
    assert np.allclose(out2, (cvr[4] + cvr[1]) / 2)


# ---------------- W8 Marlin layout and numerics ----------------
def test_marlin_dst_byte_known_answers(orc):
    f = lambda k, n, N=128: orc.lib().orc_marlin_dst_byte(k, n, N)
    # kernels/cosmos3/README.md:55-64 evaluated by hand
    assert f(0, 0) == 0
    assert f(1, 0) == 2          # lane (k%2)*2
    assert f(8, 0) == 1          # lane (k/8)%2
    assert f(9, 0) == 3
    assert f(2, 0) == 32         # col ((k%8)/2)*8 = 8 -> byte 32
    assert f(0, 1) == 128        # col (n%8)*32 = 32
    assert f(0, 8) == 4          # col (n/8)%8 = 1
    assert f(0, 64) == 1024      # col (n/64)*256
    assert f(16, 0) == 16 * 128  # next 16-row band: row*(N*4) words
    K, N = 32, 128
    bytes_ = sorted(f(k, n, N) for k in range(K) for n in range(N))
    assert bytes_ == list(range(K * N))  # a bijection onto the packed payload


def test_marlin_scale_permutation(orc):
    si = orc.lib().orc_marlin_scale_index
    assert [si(n) for n in (0, 1, 2, 8, 9, 31, 32, 34)] == [0, 1, 8, 2, 3, 31, 32, 40]
    assert sorted(si(n) for n in range(96)) == list(range(96))


def test_marlin_pack_unpack_and_gemm(orc):
    rng = np.random.default_rng(5)
    K, N, M = 64, 128, 7
    w = rng.integers(-127, 128, (K, N), dtype=np.int8)
    q = orc.marlin_pack_w8(w)
    assert q.shape == (K // 16, 4 * N)
    for k, n in [(0, 0), (5, 77), (63, 127), (17, 64)]:
        assert orc.marlin_unpack_w8(q, K, N, k, n) == w[k, n]
    s = orc.f32_to_bf16(rng.uniform(0.001, 0.01, N).astype(np.float32))
    s_st = orc.marlin_pack_scales(s)
    x = orc.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    yb, yf = orc.w8a16_gemm(x, q, s_st, M, K, N)
    ref = (orc.bf16_to_f32(x).astype(np.float64) @ w.astype(np.float64)) * orc.bf16_to_f32(s)[None].astype(np.float64)
    assert np.allclose(yf, ref, rtol=1e-6, atol=1e-5)
    assert np.array_equal(yb, orc.f32_to_bf16(yf))


# ---------------- Qwen per-head q/k RMSNorm + RoPE ----------------
def _bf(orc, rng, shape, scale=1.0):
    return orc.f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def test_head_norm_invariants(orc):
    rng = np.random.default_rng(31)
    T, H, D = 5, 3, 128
    x = _bf(orc, rng, (T, H * D))
    one = orc.f32_to_bf16(np.ones(D, np.float32))
    y = orc.bf16_to_f32(orc.head_norm_rope(x, T, H, D, gamma=one, eps=0.0)).astype(np.float64)
    assert np.allclose(np.sqrt((y ** 2).mean(-1)), 1.0, atol=4e-3)  # unit RMS per head
    # scaling a head by a power of two leaves the normalised head unchanged (eps 0: exact)
    x4 = orc.f32_to_bf16(orc.bf16_to_f32(x) * np.float32(4.0))
    assert np.array_equal(orc.head_norm_rope(x4, T, H, D, gamma=one, eps=0.0),
                          orc.head_norm_rope(x, T, H, D, gamma=one, eps=0.0))
    # gamma multiplies after the normalisation: gamma = 2 doubles the unit-gamma result exactly
    two = orc.f32_to_bf16(np.full(D, 2.0, np.float32))
    assert np.array_equal(orc.bf16_to_f32(orc.head_norm_rope(x, T, H, D, gamma=two, eps=0.0)),
                          2 * orc.bf16_to_f32(orc.head_norm_rope(x, T, H, D, gamma=one, eps=0.0)))


def test_rope_invariants_and_axis_rule(orc):
    rng = np.random.default_rng(32)
    T, H, D = 6, 2, 128
    x = _bf(orc, rng, (T, H * D))
    xr = x.reshape(T, H, D)
    # position 0 is the identity; the rotation keeps each (d, d + D/2) pair's length
    y = orc.head_norm_rope(x, T, H, D, rope_kind=1, first_pos=0)
    assert np.array_equal(y[0], xr[0])
    y = orc.bf16_to_f32(orc.head_norm_rope(x, T, H, D, rope_kind=1, theta=10000.0, first_pos=7)).astype(np.float64)
    xf = orc.bf16_to_f32(xr).astype(np.float64)
    n_in = np.hypot(xf[..., :D // 2], xf[..., D // 2:])
    n_out = np.hypot(y[..., :D // 2], y[..., D // 2:])
    assert np.allclose(n_out, n_in, rtol=2e-2, atol=2e-2)
    # pair p rotates by pos * theta^(-2p/D): p = 0 by pos radians (float64 check, bf16 sin/cos)
    pos = 7 + np.arange(T)
    c0, s0 = np.cos(pos), np.sin(pos)
    want = xf[:, :, 0] * c0[:, None] - xf[:, :, D // 2] * s0[:, None]
    assert np.allclose(y[:, :, 0], want, atol=3e-2)
    # MRoPE with the same positions on all three axes is the plain RoPE
    ids = np.tile(7 + np.arange(T, dtype=np.int32), 3)
    assert np.array_equal(orc.head_norm_rope(x, T, H, D, rope_kind=2, theta=10000.0, pos_ids=ids),
                          orc.head_norm_rope(x, T, H, D, rope_kind=1, theta=10000.0, first_pos=7))
    # axis rule (cosmos3_qwen_language_cuda.cu:131-136): only axis 1 nonzero ->
    # exactly the pairs p < 60 with p % 3 == 1 rotate
    ids = np.zeros(3 * T, np.int32)
    ids[T:2 * T] = 5
    y = orc.head_norm_rope(x, T, H, D, rope_kind=2, theta=10000.0, pos_ids=ids)
    p = np.arange(D) % (D // 2)
    moved = (y != xr).any(axis=(0, 1))
    assert np.array_equal(moved, (p < 60) & (p % 3 == 1))


def test_head_norm_rope_matches_numpy(orc):
    """float64 numpy of the same formula with the reference's bf16 rounding points: within 1 bf16 ulp."""
    rng = np.random.default_rng(33)
    T, H, D, eps, theta = 4, 2, 64, 1e-6, 5e5
    x = _bf(orc, rng, (T, H * D), 3.0)
    g = _bf(orc, rng, (D,), 0.5)
    got = orc.bf16_to_f32(orc.head_norm_rope(x, T, H, D, gamma=g, eps=eps, rope_kind=1, theta=theta, first_pos=3))
    rb = lambda a: orc.bf16_to_f32(orc.f32_to_bf16(np.asarray(a, np.float32)))
    xf = orc.bf16_to_f32(x).reshape(T, H, D).astype(np.float64)
    inv = 1.0 / np.sqrt((xf ** 2).mean(-1, keepdims=True) + eps)
    v = rb(rb(xf * inv) * orc.bf16_to_f32(g)).astype(np.float64)
    pidx = np.arange(D) % (D // 2)
    a = (3 + np.arange(T))[:, None] * theta ** (-2.0 * pidx / D)[None, :]
    c, s = rb(np.cos(a)).astype(np.float64), rb(np.sin(a)).astype(np.float64)
    r = np.concatenate([-v[..., D // 2:], v[..., :D // 2]], axis=-1)
    want = rb(v * c[:, None, :] + r * s[:, None, :])
    ulp = np.abs(want) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(got - want) <= ulp)


# ---------------- gated residual (post-attention projection epilogue) ----------------
def test_gated_residual_special_cases(orc):
    """No gate and no bias: a plain f32 residual add; gate 1: the same; gate 0
    with gate_bias 0: the residual unchanged; gate 0 with gate_bias g: the
    same as gate g; bias shifts y before the gate (not after)."""
    rng = np.random.default_rng(11)
    M, N = 7, 64
    y = rng.standard_normal((M, N)).astype(np.float32)
    r = rng.standard_normal((M, N)).astype(np.float32) * 3
    g = rng.standard_normal((M, N)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    assert np.array_equal(orc.gated_residual(y, r), r + y)
    assert np.array_equal(orc.gated_residual(y, r, gate=np.ones((M, N), np.float32)), r + y)
    assert np.array_equal(orc.gated_residual(y, r, gate=np.zeros((M, N), np.float32),
                                             gate_bias=np.zeros(N, np.float32)), r)
    gb = rng.standard_normal(N).astype(np.float32)
    assert np.array_equal(orc.gated_residual(y, r, gate=np.zeros((M, N), np.float32), gate_bias=gb),
                          orc.gated_residual(y, r, gate=np.broadcast_to(gb, (M, N)).copy()))
    # exact small integers: (y + b) * (g + gb) + r by hand
    yi = np.array([[3.0, -2.0]], np.float32)
    out = orc.gated_residual(yi, np.array([[10.0, 1.0]], np.float32), bias=np.array([1.0, 4.0], np.float32),
                             gate=np.array([[2.0, 0.5]], np.float32), gate_bias=np.array([1.0, 0.5], np.float32))
    assert np.array_equal(out, np.array([[10.0 + 4.0 * 3.0, 1.0 + 2.0 * 1.0]], np.float32))


def test_gated_residual_separate_roundings_and_bf16(orc):
    """Each node rounds to f32: the result equals the float64 value of the
    same expression rounded after every step, and differs from a single
    final rounding somewhere on random data (so a fused form would fail);
    round_bf16 rounds the f32 result to nearest-even bf16."""
    rng = np.random.default_rng(12)
    M, N = 64, 128
    y, r, g = (rng.standard_normal((M, N)).astype(np.float32) for _ in range(3))
    b, gb = (rng.standard_normal(N).astype(np.float32) for _ in range(2))
    out = orc.gated_residual(y, r, bias=b, gate=g, gate_bias=gb)
    f32 = lambda v: np.float32(v)
    a1 = f32(y.astype(np.float64) + b)
    gg = f32(g.astype(np.float64) + gb)
    want = f32(r.astype(np.float64) + f32(a1.astype(np.float64) * gg))
    assert np.array_equal(out, want)
    once = f32(r.astype(np.float64) + (y.astype(np.float64) + b) * (g.astype(np.float64) + gb))
    assert not np.array_equal(out, once)
    ob = orc.gated_residual(y, r, bias=b, gate=g, gate_bias=gb, round_bf16=True)
    import torch
    assert np.array_equal(ob, torch.from_numpy(out).to(torch.bfloat16).float().numpy())


# ---------------- LingBot full-row RMSNorm + Wan RoPE ----------------
def test_lingbot_row_norm_invariants(orc):
    """Unit weight: every row comes out with mean square 1 / (1 + eps / ms)
    (ms = the input row's mean square), the row's direction unchanged; a
    per-column weight multiplies column-wise; scaling a row (eps = 0) leaves
    the result unchanged up to f32 rounding."""
    rng = np.random.default_rng(41)
    x = (rng.standard_normal((9, 3072)) * rng.uniform(0.1, 30, (9, 1))).astype(np.float32)
    y = orc.lingbot_row_norm(x, np.ones(3072, np.float32), eps=1e-6).astype(np.float64)
    ms = (x.astype(np.float64) ** 2).mean(axis=1)
    np.testing.assert_allclose((y ** 2).mean(axis=1), ms / (ms + 1e-6), rtol=1e-5)
    cosang = (y * x).sum(1) / np.linalg.norm(y, axis=1) / np.linalg.norm(x.astype(np.float64), axis=1)
    np.testing.assert_allclose(cosang, 1.0, rtol=1e-6)
    w = rng.uniform(0.5, 2, 3072).astype(np.float32)
    np.testing.assert_allclose(orc.lingbot_row_norm(x, w), y * w, rtol=3e-7, atol=1e-7)
    np.testing.assert_allclose(orc.lingbot_row_norm(x * np.float32(8), w, eps=0.0),
                               orc.lingbot_row_norm(x, w, eps=0.0), rtol=1e-6)


def test_wan_rope_is_a_complex_rotation(orc):
    """Each (x0, x1) pair times (c + i s) as a complex product, to f32
    rounding; c = 1, s = 0 is the identity and c = 0, s = 1 maps a pair to
    (-x1, x0) exactly; the tables are indexed by token and pair, shared by
    every head."""
    rng = np.random.default_rng(42)
    T, H, D = 5, 3, 16
    x = rng.standard_normal((T, H * D)).astype(np.float32)
    ang = rng.uniform(-np.pi, np.pi, (T, D // 2))
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    y = orc.wan_rope(x, H, D, c, s)
    z = x.astype(np.float64).reshape(T, H, D // 2, 2)
    zc = (z[..., 0] + 1j * z[..., 1]) * (c.astype(np.float64) + 1j * s.astype(np.float64))[:, None, :]
    want = np.stack([zc.real, zc.imag], -1).reshape(T, H * D)
    np.testing.assert_allclose(y, want, rtol=0, atol=4e-7 * np.abs(x).max())
    one, zero = np.ones((T, D // 2), np.float32), np.zeros((T, D // 2), np.float32)
    assert np.array_equal(orc.wan_rope(x, H, D, one, zero), x)
    r = orc.wan_rope(x, H, D, zero, one).reshape(T, H, D // 2, 2)
    xp = x.reshape(T, H, D // 2, 2)
    assert np.array_equal(r[..., 0], -xp[..., 1]) and np.array_equal(r[..., 1], xp[..., 0])


def test_lingbot_qkv_bias_then_norm(orc):
    """The bias is added before the norm (lin() then rms_norm); v only gets its
    bias; with no weights and no tables q and k are the biased projections."""
    rng = np.random.default_rng(43)
    T, H, D = 4, 2, 8
    x = rng.standard_normal((T, 3 * H * D + 5)).astype(np.float32)
    b = rng.standard_normal(3 * H * D).astype(np.float32)
    q, k, v = orc.lingbot_qkv(x, H, D, bias=b)
    xb = x[:, :3 * H * D] + b
    assert np.array_equal(q, xb[:, :H * D]) and np.array_equal(k, xb[:, H * D:2 * H * D])
    assert np.array_equal(v, xb[:, 2 * H * D:])
    w = np.ones(H * D, np.float32)
    q2, _, _ = orc.lingbot_qkv(x, H, D, bias=b, q_w=w)
    assert np.array_equal(q2, orc.lingbot_row_norm(xb[:, :H * D], w))


# ---------------- pi0.5 NEOX RoPE (ggml_rope_ext, models/pi05.cpp:394-400) ----------------
def _neox64(x, pos, d, base=10000.0):
    """float64 rotation of the f32 input: pair (i, i + d/2) by pos * base^(-2i/d)."""
    x = x.astype(np.float64)
    half = d // 2
    th = np.asarray(pos, np.float64)[:, None] * base ** (-2.0 * np.arange(half) / d)[None, :]
    c, s = np.cos(th)[:, None, :], np.sin(th)[:, None, :]
    x0, x1 = x[..., :half], x[..., half:]
    return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1), th


def test_neox_rope_identity_onehots_and_known_answer(orc):
    rng = np.random.default_rng(41)
    T, H, D = 5, 3, 256
    x = rng.standard_normal((T, H * D)).astype(np.float32)
    # position 0 turns nothing: cos 0 = 1 and sin 0 = 0 leave every value exact
    assert np.array_equal(orc.neox_rope(x, T, H, D, first_pos=0)[0], x.reshape(T, H, D)[0])
    # NEOX pairs dim i with i + D/2 (not 2i with 2i + 1): a one-hot at i lands on
    # i (cos) and i + D/2 (sin) only; a one-hot at i + D/2 on i (-sin) and i + D/2 (cos)
    pos = 5
    for i in (0, 1, 7, D // 2 - 1):
        th = pos * 10000.0 ** (-2.0 * i / D)
        for src, (a, b) in ((i, (math.cos(th), math.sin(th))), (i + D // 2, (-math.sin(th), math.cos(th)))):
            e = np.zeros((1, D), np.float32)
            e[0, src] = 1.0
            y = orc.neox_rope(e, 1, 1, D, first_pos=pos)[0, 0].astype(np.float64)
            nz = set(np.flatnonzero(y).tolist())
            assert nz <= {i, i + D // 2}, (i, src, sorted(nz))
            assert abs(y[i] - a) < 1e-5 and abs(y[i + D // 2] - b) < 1e-5, (i, src, y[i], y[i + D // 2])
    # pair 0 turns by exactly pos radians (theta_scale^0 = 1): position 1 is a turn by 1 rad
    e = np.zeros((1, D), np.float32)
    e[0, 0] = 1.0
    y = orc.neox_rope(e, 1, 1, D, first_pos=1)[0, 0]
    assert y[0] == np.float32(math.cos(1.0)) and y[D // 2] == np.float32(math.sin(1.0))


def test_neox_rope_float64_and_pair_lengths(orc):
    # against float64 at the config-1 suffix positions (n_prefix 816 + i): the
    # only gap is f32 theta, whose relative error grows with the power i of the
    # rounded theta_scale (about (i + 4) ulp), plus the f32 sin/cos/products
    rng = np.random.default_rng(42)
    T, H, D = 51, 9, 256
    x = (rng.standard_normal((T, H * D)) * 3).astype(np.float32)
    pos = 816 + np.arange(T)
    y = orc.neox_rope(x, T, H, D, first_pos=816).astype(np.float64)
    want, th = _neox64(x.reshape(T, H, D), pos, D)
    half = D // 2
    n_in = np.hypot(x.reshape(T, H, D)[..., :half].astype(np.float64), x.reshape(T, H, D)[..., half:])
    dth = th * (np.arange(half) + 4) * 2.0 ** -24 + 4 * 2.0 ** -24  # angle error bound [T][half]
    tol = np.concatenate([n_in * dth[:, None, :]] * 2, axis=-1) + 1e-6
    err = np.abs(y - want)
    assert np.all(err <= tol), float(np.max(err / tol))
    # a rotation: each (i, i + D/2) pair keeps its length
    n_out = np.hypot(y[..., :half], y[..., half:])
    assert np.allclose(n_out, n_in, rtol=2e-6, atol=1e-6)
    # the explicit positions array reads the same as first_pos + t
    assert np.array_equal(orc.neox_rope(x, T, H, D, positions=pos.astype(np.int32)), y.astype(np.float32))


def test_neox_rope_relative_position_and_cpu_rule(orc):
    # RoPE's defining property: <rope(q, m), rope(k, n)> depends on m - n only
    rng = np.random.default_rng(43)
    D = 256
    q = rng.standard_normal((1, D)).astype(np.float32)
    k = rng.standard_normal((1, D)).astype(np.float32)
    dots = []
    for m, n in ((820, 816), (4, 0), (104, 100)):
        a = orc.neox_rope(q, 1, 1, D, first_pos=m)[0, 0].astype(np.float64)
        b = orc.neox_rope(k, 1, 1, D, first_pos=n)[0, 0].astype(np.float64)
        dots.append(a @ b)
    assert max(dots) - min(dots) < 1e-5 * np.linalg.norm(q) * np.linalg.norm(k), dots
    # ggml's CPU backend builds theta by repeated multiplication (theta *=
    # theta_scale per pair) instead of one power per pair; the two f32 rules
    # agree within the f32 theta error bound above
    T, H = 51, 1
    x = rng.standard_normal((T, D)).astype(np.float32)
    ts = np.float32(np.float32(10000.0) ** np.float32(-2.0 / D))
    th = np.zeros((T, D // 2), np.float32)
    for t in range(T):
        v = np.float32(816 + t)
        for i in range(D // 2):
            th[t, i] = v
            v = np.float32(v * ts)
    c, s = np.cos(th.astype(np.float64)), np.sin(th.astype(np.float64))
    x0, x1 = x[:, :D // 2].astype(np.float64), x[:, D // 2:].astype(np.float64)
    cpu = np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)
    y = orc.neox_rope(x, T, H, D, first_pos=816)[:, 0].astype(np.float64)
    assert np.max(np.abs(y - cpu)) < 5e-3 * np.max(np.abs(x)), np.max(np.abs(y - cpu))


# ---------------- call-site masks (hand-derived known answers) ----------------
I = float("-inf")


def test_hy_patch_groups_known_answers(orc):
    # runs of nonzero flags; one zero keeps the group open, two or more close it
    assert orc.hy_patch_groups([0, 1, 1, 0, 1, 1, 0, 0, 1, 0]) == [[1, 2, 4, 5], [8]]
    assert orc.hy_patch_groups([1, 1, 0, 0, 1]) == [[0, 1], [4]]
    assert orc.hy_patch_groups([1, 0, 1, 0, 1]) == [[0, 2, 4]]
    assert orc.hy_patch_groups([0, 0, 0]) == []
    assert orc.hy_patch_groups([0, 0, 1, 1, 1]) == [[2, 3, 4]]
    assert orc.hy_patch_groups([]) == []


def test_hy_prefix_and_suffix_masks_known_answers(orc):
    # n = 5, groups {1, 2} and {4}: causal outside the groups, a group sees
    # itself both ways, the two groups never see each other
    want = np.array([[0, I, I, I, I],
                     [0, 0, 0, I, I],
                     [0, 0, 0, I, I],
                     [0, 0, 0, 0, I],
                     [0, I, I, 0, 0]], np.float32)
    assert np.array_equal(orc.hy_prefix_mask(5, [[1, 2], [4]]), want)
    assert np.array_equal(orc.hy_prefix_mask(4), np.triu(np.full((4, 4), I, np.float32), 1))
    # suffix (n_pref 2, n_suf 3): all prefix keys; row 0 sees only suffix key 0
    want = np.array([[0, 0, 0, I, I],
                     [0, 0, 0, 0, 0],
                     [0, 0, 0, 0, 0]], np.float32)
    assert np.array_equal(orc.hy_suffix_mask(2, 3), want)


def test_groot_and_smolvla_masks_known_answers(orc):
    # GR00T layers with attend_text_every_n_blocks 2: 0 text, 1 self, 2 image, 3 self, 4 text
    assert [orc.groot_layer_mask_kind(i, 2) for i in range(6)] == [1, 0, 2, 0, 1, 0]
    assert [orc.groot_layer_mask_kind(i, 1) for i in range(4)] == [1, 0, 1, 0]
    text, image = orc.groot_cross_masks([1, 1, 1, 0], [0, 1, 1, 1], 2)
    assert np.array_equal(text, np.array([[0, I, I, I]] * 2, np.float32))
    assert np.array_equal(image, np.array([[I, 0, 0, I]] * 2, np.float32))
    # SmolVLA: prefix [img, img, pad, lang, state], suffix of 2
    pm, fm, cm = orc.smolvla_masks([1, 1, 0, 1, 1], 2)
    want_pm = np.array([[0, 0, I, 0, I]] * 4 + [[0, 0, I, 0, 0]], np.float32)
    assert np.array_equal(pm, want_pm)
    assert np.array_equal(fm, np.array([[0, 0, I, 0, 0, 0, I],
                                        [0, 0, I, 0, 0, 0, 0]], np.float32))
    assert np.array_equal(cm, np.array([[0, 0, I, 0, 0]] * 2, np.float32))
    pp, sp, cp = orc.smolvla_positions([1, 1, 0, 1, 1], 2)
    assert pp.tolist() == [0, 1, 1, 2, 3] and sp.tolist() == [4, 5] and cp.tolist() == [0, 1]
    pp, _, _ = orc.smolvla_positions([0, 0, 1], 1)
    assert pp.tolist() == [0, 0, 0]


def test_pbf16_attention_known_answers(orc):
    D = 64
    rng = np.random.default_rng(61)
    one = orc.f32_to_bf16(np.ones(1, np.float32))[0]
    # three equal scores: p = bf16(1/3) = 0x3EAB (0.333984375), so a V of ones
    # gives 3 * 0.333984375 = 1.001953125, not 1
    q = np.zeros((1, 1, D), np.uint16)
    k = np.zeros((3, 1, D), np.uint16)
    v = np.full((3, 1, D), one, np.uint16)
    out = orc.pbf16_attention(q, k, v, 1, 3, 1, 1, D, 0.125)
    assert np.all(out == 1.001953125)
    third = np.float64(np.float32(1) / np.float32(3))  # f32 p without the bf16 rounding
    assert np.all(orc.pbf16_attention(q, k, v, 1, 3, 1, 1, D, 0.125, round_p=False) == 3 * third)
    # two equal scores: p = 0.5 exactly; one visible key: p = 1 (output = v)
    vv = orc.f32_to_bf16(rng.standard_normal((3, 1, D)).astype(np.float32))
    vf = orc.bf16_to_f32(vv).astype(np.float64)
    add = np.array([[0, 0, I]], np.float32)
    assert np.array_equal(orc.pbf16_attention(q, k, vv, 1, 3, 1, 1, D, 0.125, add=add)[0, 0],
                          (vf[0, 0] + vf[1, 0]) / 2)
    add = np.array([[I, 0, I]], np.float32)
    assert np.array_equal(orc.pbf16_attention(q, k, vv, 1, 3, 1, 1, D, 0.125, add=add)[0, 0], vf[1, 0])
    # without the rounding it is the (pinned) f32 attention oracle
    n_q, n_k, hq, hkv = 7, 40, 4, 2
    qb = orc.f32_to_bf16(rng.standard_normal((n_q, hq, D)).astype(np.float32))
    kb = orc.f32_to_bf16(rng.standard_normal((n_k, hkv, D)).astype(np.float32))
    vb = orc.f32_to_bf16(rng.standard_normal((n_k, hkv, D)).astype(np.float32))
    a = orc.pbf16_attention(qb, kb, vb, n_q, n_k, hq, hkv, D, 0.125, round_p=False)
    b = orc.gqa_attention(qb, kb, vb, n_q, n_k, hq, hkv, D, 0.125, q_pos0=0)
    assert np.allclose(a, b, atol=2e-6), np.max(np.abs(a - b))
    # and the rounding moves it by about bf16's precision of p (2^-9 relative)
    r = orc.pbf16_attention(qb, kb, vb, n_q, n_k, hq, hkv, D, 0.125)
    rel = np.abs(r - a).sum() / np.abs(a).sum()
    assert 1e-4 < rel < 3e-3, rel


# ---------------- the CPU baseline's attention (bench.py cpu_baseline) ----------------
@pytest.mark.parametrize("threads", [1, 4])
def test_cpu_baseline_attention_matches_oracle(orc, threads):
    # config-1 layer problem: 51 queries x 8 heads over 867 keys, one kv head, d 256
    n_q, n_k, hq, hkv, d = 51, 867, 8, 1, 256
    k = orc.normal_bf16(0xE3BD0001, n_k * hkv * d)
    v = orc.normal_bf16(0xE3BD0002, n_k * hkv * d)
    q = orc.normal_bf16(0xE3BD000A, n_q * hq * d)
    got, used = orc.cpu_attention_f32(orc.bf16_to_f32(q), orc.bf16_to_f32(k), orc.bf16_to_f32(v), n_q, n_k, hq, hkv,
                                      d, 1 / 16, threads)
    assert used == threads
    want = orc.gqa_attention(q, k, v, n_q, n_k, hq, hkv, d, 1 / 16)
    assert np.allclose(got, want, rtol=0, atol=2e-5), np.max(np.abs(got - want))
    # GQA: heads 0..3 read kv head 0, heads 4..7 kv head 1
    n_k2, hkv2 = 100, 2
    k2 = orc.normal_bf16(7, n_k2 * hkv2 * d)
    v2 = orc.normal_bf16(8, n_k2 * hkv2 * d)
    got2, _ = orc.cpu_attention_f32(orc.bf16_to_f32(q), orc.bf16_to_f32(k2), orc.bf16_to_f32(v2), n_q, n_k2, hq,
                                    hkv2, d, 1 / 16, threads)
    want2 = orc.gqa_attention(q, k2, v2, n_q, n_k2, hq, hkv2, d, 1 / 16)
    assert np.allclose(got2, want2, rtol=0, atol=2e-5)


# ---------------- dense-weight lin() (ggml CUDA mul_mat numerics) ----------------
def test_dense_linear_known_answers(orc):
    f = np.float32
    # 257 ones: exact sum 257, which bf16 rounds to 256 (tie to even); f32 keeps it
    x = np.ones((1, 257), f)
    w = np.ones((1, 257), f)
    assert orc.dense_linear(x, w, False)[0, 0] == 257.0
    assert orc.dense_linear(x, orc.f32_to_bf16(w), True)[0, 0] == 256.0
    # the bias is added after the bf16 rounding, as its own f32 node
    b = np.array([0.5], f)
    assert orc.dense_linear(x, w, False, bias=b)[0, 0] == 257.5
    assert orc.dense_linear(x, orc.f32_to_bf16(w), True, bias=b)[0, 0] == 256.5
    # x is rounded to bf16 first with bf16 weights (1 + 2^-9 -> 1), not with f32 ones
    x1 = np.array([[1 + 2.0 ** -9]], f)
    w1 = np.array([[1.0]], f)
    assert orc.dense_linear(x1, w1, False)[0, 0] == f(1 + 2.0 ** -9)
    assert orc.dense_linear(x1, orc.f32_to_bf16(w1), True)[0, 0] == 1.0
    # and one rounding of the exact sum, not a rounding per partial sum:
    # 2^24 + 1 + 1 is 2^24 + 2 exactly, which sequential f32 adds would lose
    x3 = np.array([[2.0 ** 24, 1.0, 1.0]], f)
    w3 = np.ones((1, 3), f)
    assert orc.dense_linear(x3, w3, False)[0, 0] == f(2.0 ** 24 + 2)


def test_dense_linear_index_order_brute_force(orc):
    # w is [N][K] (ggml ne0 = K); a transposed operand or swapped index fails here
    rng = np.random.default_rng(5)
    M, K, N = 3, 5, 4
    x = rng.integers(-8, 9, (M, K)).astype(np.float32)
    w = rng.integers(-8, 9, (N, K)).astype(np.float32)
    bias = rng.integers(-4, 5, N).astype(np.float32)
    want = np.zeros((M, N), np.float32)
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                acc += float(x[m, k]) * float(w[n, k])
            want[m, n] = acc + bias[n]
    assert np.array_equal(orc.dense_linear(x, w, False, bias=bias), want)
    assert np.array_equal(orc.dense_linear(x, orc.f32_to_bf16(w), True, bias=bias), want)  # small integers: exact
    # bf16 x given as bits equals f32 x rounded by the oracle
    xb = orc.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    assert np.array_equal(orc.dense_linear(xb, orc.f32_to_bf16(w), True),
                          orc.dense_linear(orc.bf16_to_f32(xb), orc.f32_to_bf16(w), True))
    # rows= picks rows of x
    assert np.array_equal(orc.dense_linear(x, w, False, rows=[2, 0]), orc.dense_linear(x, w, False)[[2, 0]])


def test_gated_residual_without_residual(orc):
    f = np.float32
    y = np.array([[1.5, -0.0]], f)
    g = np.array([[2.0, 3.0]], f)
    out = orc.gated_residual(y, None, gate=g)
    assert out[0, 0] == 3.0 and out[0, 1] == 0.0 and np.signbit(out[0, 1])  # -0 * 3 stays -0: no residual add
    assert np.array_equal(orc.gated_residual(y, None), y)
