"""CPU tests of libemb_kv.so: exports, host-side cache/page/flex logic vs the
oracle, and argument checks that return before any GPU work."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest


def test_library_exports_every_header_symbol(emb):
    syms = emb.header_symbols()
    assert len(syms) > 40
    missing = [s for s in syms if not hasattr(emb.lib(), s)]
    assert not missing, missing
    assert b"gfx950" in emb.lib().emb_version()


def _ops(rng, n_ops, cap):
    ops = []
    for _ in range(n_ops):
        r = rng.random()
        k = int(rng.integers(1, max(2, cap // 3)))
        if r < 0.45:
            ops.append(("update", k, int(rng.random() < 0.3)))
        elif r < 0.7:
            ops.append(("mode0", k, 0))
        elif r < 0.8:
            ops.append(("clear_pred", 0, 0))
        elif r < 0.9:
            ops.append(("update_restore", k, 0))
        else:
            ops.append(("chunk", cap // 4, 0))
    return ops


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("legacy", [False, True])
def test_slot_cache_matches_oracle(emb, orc, seed, legacy):
    rng = np.random.default_rng(seed)
    cap = int(rng.integers(8, 60))
    a = emb.SlotCache(cap, legacy)
    b = orc.Cache(cap, legacy)
    for op, k, pred in _ops(rng, 60, cap):
        if op in ("update", "chunk"):
            sa, rc = a.update_meta(k, pred)
            sb = b.update_meta(k, pred)
            assert (rc == 0) == (sb is not None)
            if sb is not None:
                assert np.array_equal(sa, sb)
        elif op == "update_restore":
            sa, rc = a.update_meta(k, 0)
            sb = b.update_meta(k, 0)
            assert (rc == 0) == (sb is not None)
            if sb is not None:
                a.restore(sa)
                b.restore(sb)
        elif op == "mode0":
            sa, va, rc = a.prepare_mode0(k)
            sb, vb = b.prepare_mode0(k)
            assert (rc == 0) == (sb is not None)
            if sb is not None:
                assert np.array_equal(sa, sb) and np.array_equal(va, vb)
        else:
            a.clear_pred()
            b.clear_pred()
        ia, ma, pa = a.state()
        ib, mb, pb = b.state()
        assert np.array_equal(ia, ib) and np.array_equal(ma, mb) and np.array_equal(pa, pb), op
        assert a.used_count() == b.used_count() and a.pred_count() == b.pred_count()
        assert a.next_id() == b.next_id()
        assert np.array_equal(a.collect_valid(), b.collect_valid())


def test_page_pool_and_block_table(emb):
    pool = emb.PagePool(20, seed=7)
    c = emb.SlotCache(64)
    c.bind_pool(pool)
    assert pool.free_count() == 20
    s, rc = c.update_meta(20, 0)          # slots 0..19 -> pages for logical pages 0, 1
    assert rc == 0 and list(s) == list(range(20))
    bt = c.block_table()
    assert bt.shape == (4,) and bt[0] >= 0 and bt[1] >= 0 and bt[2] == -1 and bt[3] == -1
    assert pool.free_count() == 18 and bt[0] != bt[1]
    c.map_range(64)
    bt = c.block_table()
    assert np.all(bt >= 0) and len(set(bt.tolist())) == 4 and pool.free_count() == 16
    c2 = emb.SlotCache(300)
    c2.bind_pool(pool)
    _, rc = c2.update_meta(300, 0)          # needs 19 pages, 16 left
    assert rc == -3 and "exhausted" in emb.last_error()
    assert c2.used_count() == 0 and pool.free_count() == 0  # mapped pages stay with c2
    c.release_pages()
    assert pool.free_count() == 4
    c2.release_pages()
    assert pool.free_count() == 20
    # a seeded pool hands out a permutation; seed 0 hands out 0, 1, 2, ...
    p0 = emb.PagePool(8, seed=0)
    c3 = emb.SlotCache(128)
    c3.bind_pool(p0)
    c3.map_range(128)
    assert list(c3.block_table()) == list(range(8))


def test_capacity_matches_oracle(emb, orc):
    for kw in [dict(seq=100), dict(frame_chunk_size=2, action_per_frame=16, attn_window=72,
                                   latent_h=24, latent_w=20, seq=10),
               dict(override_tokens=14040, seq=1560), dict(patch_t=0, seq=1), dict(seq=99999),
               dict(n_suffix=7, attn_window=9, seq=3)]:
        assert emb.lingbot_kv_capacity(**kw) == orc.lingbot_capacity(**kw), kw


def test_flex_meta_tables_match_oracle(emb, orc):
    L = emb.lib()
    for args in [(1, 2, 2, 2, 1, 2, 1, 1, 1, 1, 4, 1, 1, 1, 5, 4),
                 (1, 4, 4, 4, 1, 4, 2, 1, 3, 2, 1, 2, 2, 2, 7, 8),
                 (2, 2, 2, 4, 1, 2, 2, 1, 0, 1, 0, 1, 1, 2, 3, 4)]:
        m = L.emb_flex_meta_build(*args)
        om = orc.FlexMeta(*args)
        n = L.emb_flex_meta_len(m)
        for q in range(n):
            for k in range(n):
                assert L.emb_flex_self_allowed(m, q, k) == orc.lib().orc_flex_self_allowed(om.h, q, k)
        bs = args[-1]
        qb = (n + bs - 1) // bs
        rp = np.zeros(qb + 1, np.int32)
        ci = np.zeros(qb * qb, np.int32)
        nnz = L.emb_self_block_table(m, rp.ctypes.data_as(emb.i32p), ci.ctypes.data_as(emb.i32p))
        orp, oci = orc.self_block_table(om, n, bs)
        assert np.array_equal(rp, orp) and np.array_equal(ci[:nnz], oci)
        tm = np.zeros(n * n, np.uint8)
        L.emb_self_token_mask(m, tm.ctypes.data_as(emb.u8p))
        assert np.array_equal(tm.reshape(n, n), orc.self_token_mask(om, n))
        L.emb_flex_meta_destroy(m)
    rp = np.zeros(4, np.int32)
    ci = np.zeros(12, np.int32)
    assert L.emb_dense_block_table(9, 13, 4, rp.ctypes.data_as(emb.i32p), ci.ctypes.data_as(emb.i32p)) == 12


def test_synthetic_generator_matches_oracle(emb, orc):
    for seed, n in [(0xE3BD0001, 1001), (0xE3BD0003, 4096)]:
        assert np.array_equal(emb.synth_normal_bf16(seed, n), orc.normal_bf16(seed, n))


def test_device_entry_points_reject_bad_arguments(emb):
    L = emb.lib()
    # every check below returns before any HIP call, so it runs without a GPU
    assert L.emb_kv_append(None, None, 0, 1, None, None, 16, None, None, None, 1, 128, None) == -1
    assert "null" in emb.last_error()
    buf = C.c_void_p(256)  # aligned, never dereferenced: rejected on shape first
    assert L.emb_kv_append(buf, buf, 100, 4, buf, None, 16, buf, buf, None, 1, 100, None) == -1
    assert "multiple of 8" in emb.last_error()
    assert L.emb_kv_append(buf, buf, 128, 4, buf, None, 16, buf, buf, C.c_void_p(264), 1, 128, None) == -1
    assert "aligned" in emb.last_error()
    # W8: shapes outside the Marlin contract are refused before any launch
    assert L.emb_w8a16_gemm(buf, 0, 96, buf, buf, 4, 96, 96, buf, 96, 0, None) == -4
    assert "out_features" in emb.last_error()
    assert L.cosmos3_w8a16_linear_f32(buf, buf, buf, buf, 4, 128, 128, 9, 512, 1, 128, None) == -1
    assert L.emb_w8a16_gemm(buf, 0, 128, buf, buf, 4, 128, 128, buf, 128, 7, None) == -1
    # LingBot row norm + RoPE: head_dim, row size and table pairing are checked first
    R = L.emb_qkv_rownorm_rope_append
    assert R(buf, 384, 4, 1, 124, None, None, None, 1e-6, None, None, buf, 128, buf, None, 16, buf, buf, None,
             None) == -1 and "multiple of 8" in emb.last_error()
    assert R(buf, 3 * 8448, 4, 66, 128, None, None, None, 1e-6, None, None, buf, 8448, buf, None, 16, buf, buf,
             None, None) == -1 and "8192" in emb.last_error()
    assert R(buf, 384, 4, 1, 128, None, None, None, 1e-6, buf, None, buf, 128, buf, None, 16, buf, buf, None,
             None) == -1 and "go together" in emb.last_error()
    assert R(buf, 380, 4, 1, 128, None, None, None, 1e-6, None, None, buf, 128, buf, None, 16, buf, buf, None,
             None) == -1 and "ld" in emb.last_error()
    # gated residual: overlaps, strides and gate_bias without a gate are refused
    G = lambda *a: L.emb_w8a16_gated_residual(*a[:-1], None, a[-1])  # no x workspace
    o, r = C.c_void_p(1 << 20), C.c_void_p(1 << 24)
    assert G(buf, 0, 128, buf, buf, 4, 128, 128, None, None, 128, None, None, 128, o, 128, 0, None) == -1
    assert "null" in emb.last_error()
    assert G(buf, 0, 128, buf, buf, 4, 128, 128, None, None, 128, buf, r, 128, o, 128, 0, None) == -1
    assert "gate_bias needs a gate" in emb.last_error()
    assert G(buf, 0, 128, buf, buf, 4, 128, 128, None, None, 128, None, C.c_void_p((1 << 20) + 512), 128, o, 128,
             0, None) == -1
    assert "overlaps residual" in emb.last_error()
    assert G(buf, 0, 128, buf, buf, 4, 128, 128, None, C.c_void_p((1 << 20) + 64), 768, None, r, 128, o, 128,
             0, None) == -1
    assert "overlaps gate" in emb.last_error()
    assert G(buf, 0, 128, buf, buf, 4, 128, 128, None, None, 128, None, o, 256, o, 128, 0, None) == -1
    assert "ldr == ldo" in emb.last_error()
    assert G(buf, 0, 128, buf, buf, 4, 128, 128, None, r, 64, None, r, 128, o, 128, 0, None) == -1
    assert "ldg" in emb.last_error()
    assert G(buf, 0, 96, buf, buf, 4, 96, 96, None, None, 96, None, r, 96, o, 96, 0, None) == -4
    # an f32 x workspace that overlaps out is refused
    assert L.emb_w8a16_gated_residual(buf, 1, 128, buf, buf, 4, 128, 128, None, None, 128, None, r, 128, o, 128, 0,
                                      C.c_void_p((1 << 20) + 256), None) == -1
    assert "workspace overlaps" in emb.last_error()
    # dense weights: weight type, x type, K, ldw and a weight/out overlap are refused first
    D = L.emb_dense_gated_residual
    w = C.c_void_p(1 << 26)
    args = lambda x32, K, wp, wt, ldw, out: (buf, x32, K, wp, wt, ldw, 4, K, 128, None, None, 128, None, r, 128, out,
                                             128, 0, None, None)
    assert D(*args(1, 128, w, emb.EMB_GGML_F16, 128, o)) == -4 and "weight_type" in emb.last_error()
    assert D(*args(0, 128, w, emb.EMB_GGML_F32, 128, o)) == -4 and "f32 x" in emb.last_error()
    assert D(*args(1, 120, w, emb.EMB_GGML_BF16, 120, o)) == -4 and "% 16" in emb.last_error()
    assert D(*args(1, 130, w, emb.EMB_GGML_F32, 132, o)) == -4 and "% 4" in emb.last_error()
    assert D(*args(1, 128, w, emb.EMB_GGML_BF16, 64, o)) == -1 and "ldw" in emb.last_error()
    assert D(*args(1, 128, o, emb.EMB_GGML_BF16, 128, C.c_void_p((1 << 20) + 4096))) == -1
    assert "overlaps the weights" in emb.last_error()
    assert D(*args(1, 128, None, emb.EMB_GGML_BF16, 128, o)) == -1 and "null weight" in emb.last_error()
    assert L.emb_kv_gather(buf, buf, buf, 0, None, 16, buf, buf, 1, 128, None) == -1
    assert L.lingbot_runtime_kv_update_f32(buf, buf, buf, buf, buf, 4, 1, 64, 4, None) == -1
    assert "capacity" in emb.last_error()
    with pytest.raises(RuntimeError, match="head_dim"):
        emb.paged_attention(q=256, out=256, k_pool=256, v_pool=256, batch=1, hq=8, hkv=1, d=96,
                            max_q=4, scale=0.1, capacity=64)
    with pytest.raises(RuntimeError, match="split_keys"):
        emb.paged_attention(q=256, out=256, k_pool=256, v_pool=256, batch=1, hq=8, hkv=1, d=256,
                            max_q=4, scale=0.1, capacity=64, n_keys_uniform=64, splits=2, workspace=256,
                            split_keys=-1)
    with pytest.raises(RuntimeError, match="head counts"):
        emb.paged_attention(q=256, out=256, k_pool=256, v_pool=256, batch=1, hq=6, hkv=4, d=128,
                            max_q=4, scale=0.1, capacity=64)
    with pytest.raises(RuntimeError, match="cu_q"):
        emb.paged_attention(q=256, out=256, k_pool=256, v_pool=256, batch=2, hq=8, hkv=1, d=128,
                            max_q=4, scale=0.1, capacity=64)
    with pytest.raises(RuntimeError, match="go together"):
        emb.paged_attention(q=256, out=256, k_pool=256, v_pool=256, batch=2, hq=8, hkv=1, d=128,
                            max_q=4, scale=0.1, capacity=64, cu_q=256)
    with pytest.raises(RuntimeError, match="workspace"):
        emb.paged_attention(q=256, out=256, k_pool=256, v_pool=256, batch=1, hq=8, hkv=1, d=128,
                            max_q=4, scale=0.1, capacity=64, splits=4, n_keys_uniform=40)
    assert L.lingbot_runtime_kv_attn_f32(None, None, None, None, None, 1, 1, 1, 64, 0.1, None) == -1
    # device slot metadata: descriptor and call arguments are checked before any launch
    dc = emb.DevCacheDesc(256, 256, 256, 0, 0)
    assert L.emb_dev_cache_init(C.byref(dc), None) == -1 and "capacity" in emb.last_error()
    dc = emb.DevCacheDesc(256, 256, 256, 64, 0)
    assert L.emb_dev_cache_update(C.byref(dc), 0, 2, buf, None, None, buf, None) == -1
    assert L.emb_dev_cache_update(C.byref(dc), 4, 3, buf, None, None, buf, None) == -1
    assert "mode" in emb.last_error()
    assert L.emb_dev_cache_update(C.byref(dc), 4, 1, None, None, None, buf, None) == -1
    assert L.emb_dev_cache_restore(C.byref(dc), None, 4, None) == -1
    assert L.emb_dev_cache_clear_pred(None, None) == -1
    # f16 partial rows (O/l) plus f32 (m, l) per row
    assert emb.attn_workspace_bytes(1, 51, 8, 1, 256, 4) == 4 * 512 * (256 * 2 + 4 * 4)  # f16 O + (m, l, k, 0)
    # whole-tensor faces: null pointers, head sizes past 256, ggml descriptors
    assert L.lingbot_flex_attn_f32(None, buf, buf, buf, buf, buf, 8, 8, 2, 64, 4, 0.1, None) == -1
    assert L.lingbot_flex_attn_f32(buf, buf, buf, buf, buf, buf, 8, 8, 2, 320, 4, 0.1, None) == -4
    assert L.lingbot_flex_attn_f32_masked(buf, buf, buf, buf, buf, None, buf, 8, 8, 2, 64, 4, 0.1, None) == -1
    q = emb.ggml_tensor(256, emb.EMB_GGML_F32, [128, 5, 8, 2])
    k = emb.ggml_tensor(256, emb.EMB_GGML_F16, [128, 40, 2, 2])
    o = emb.ggml_tensor(256, emb.EMB_GGML_F32, [128, 8, 5, 2])
    ws = L.emb_ggml_flash_attn_ext_workspace(C.byref(q), C.byref(k), C.byref(k), None, C.byref(o))
    pages = (40 + 15) // 16
    assert ws >= 3 * 2 * pages * 2 * 16 * 128 * 2  # three pools of two sequences
    o_bad = emb.ggml_tensor(256, emb.EMB_GGML_F32, [128, 5, 8, 2])  # not [D, H_q, n_q, B]
    assert L.emb_ggml_flash_attn_ext_workspace(C.byref(q), C.byref(k), C.byref(k), None, C.byref(o_bad)) == 0
    q_big = emb.ggml_tensor(256, emb.EMB_GGML_F32, [320, 5, 8, 2])
    k_big = emb.ggml_tensor(256, emb.EMB_GGML_F16, [320, 40, 2, 2])
    assert L.emb_ggml_flash_attn_ext_workspace(C.byref(q_big), C.byref(k_big), C.byref(k_big), None, None) == 0
    assert L.emb_ggml_flash_attn_ext(C.byref(q), C.byref(k), C.byref(k), None, 0.1, 0.0, 0.0, C.byref(o),
                                     None, ws, None) == -1  # no workspace
    assert "workspace" in emb.last_error()


def test_gated_residual_wrapper_refuses_short_buffers(emb):
    """The Python face checks tensor extents the C-ABI cannot see: a Marlin
    weight of [K/16][N] words instead of [K/16][4N] is refused before launch."""
    import torch
    M, K, N = 8, 64, 64
    x = torch.zeros((M, K), dtype=torch.int16)
    s = torch.zeros(N, dtype=torch.int16)
    r = torch.zeros((M, N))
    with pytest.raises(ValueError, match="qweight"):
        emb.w8a16_gated_residual(x, torch.zeros((K // 16, N), dtype=torch.int32), s, M, K, N, r, r)
    tp = torch.zeros((M, 6 * N))
    with pytest.raises(ValueError, match="gate"):  # a gate view at column 5N has too few columns left
        emb.w8a16_gated_residual(x, torch.zeros((K // 16, 4 * N), dtype=torch.int32), s, M, K, N, r, r,
                                 gate=tp[:, 5 * N + 1:], ldg=6 * N)


def test_reference_f32_faces_reject_like_the_reference(emb):
    """lingbot_runtime_kv_update_f32 / _gather_f32 return -1 for a null pointer
    or a non-positive seq, n_heads, head_dim or capacity, before any launch, as
    the reference's wrappers do (kernels/lingbot/lingbot_flex_attn_cuda.cu:911-913,
    :998-1001)."""
    L = emb.lib()
    b = C.c_void_p(256)
    U, G = L.lingbot_runtime_kv_update_f32, L.lingbot_runtime_kv_gather_f32
    for seq, h, d, cap in [(0, 2, 64, 64), (4, 0, 64, 64), (4, 2, 0, 64), (4, 2, 64, 0), (-1, 2, 64, 64)]:
        assert U(b, b, b, b, b, seq, h, d, cap, None) == -1
        assert G(b, b, b, b, b, seq, h, d, cap, None) == -1
    assert U(None, b, b, b, b, 4, 2, 64, 64, None) == -1
    assert G(b, b, None, b, b, 4, 2, 64, 64, None) == -1


# ---------------- call-site mask builders against the oracle's step-by-step restatement ----------------
def _f16_bits(m):
    return np.asarray(m, np.float32).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_hy_masks_match_oracle(emb, orc, seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 90))
    # modality flags with runs and isolated / double zeros
    mod = (rng.random(n) < 0.6).astype(np.int32)
    n_groups, group_of = emb.hy_patch_groups(mod)
    groups = orc.hy_patch_groups(mod.tolist())
    assert n_groups == len(groups)
    want_of = np.full(n, -1, np.int32)
    for g, members in enumerate(groups):
        want_of[members] = g
    assert np.array_equal(group_of, want_of)
    for with_groups in (False, True):
        allow, f16 = emb.hy_prefix_mask(n, group_of if with_groups else None)
        ref = orc.hy_prefix_mask(n, groups if with_groups else None)
        assert np.array_equal(f16, _f16_bits(ref)), "F16 bits"
        assert np.array_equal(allow, (ref == 0).astype(np.uint8))
    n_suf = int(rng.integers(1, 60))
    allow, f16 = emb.hy_suffix_mask(n, n_suf)
    ref = orc.hy_suffix_mask(n, n_suf)
    assert np.array_equal(f16, _f16_bits(ref)) and np.array_equal(allow, (ref == 0).astype(np.uint8))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_groot_and_smolvla_masks_match_oracle(emb, orc, seed):
    rng = np.random.default_rng(10 + seed)
    nk, nq = int(rng.integers(1, 300)), int(rng.integers(1, 20))
    valid = (rng.random(nk) < 0.8).astype(np.int32)
    img = (rng.random(nk) < 0.5).astype(np.int32)
    for a, b in zip(emb.groot_cross_masks(valid, img, nq), orc.groot_cross_masks(valid, img, nq)):
        assert np.array_equal(a, b)
    for every in (1, 2, 3):
        assert [emb.groot_layer_mask_kind(i, every) for i in range(16)] == \
               [orc.groot_layer_mask_kind(i, every) for i in range(16)]
    npre, nsuf = int(rng.integers(1, 200)), int(rng.integers(1, 60))
    pv = (rng.random(npre) < 0.85).astype(np.uint8)
    for a, b in zip(emb.smolvla_masks(pv, nsuf), orc.smolvla_masks(pv.tolist(), nsuf)):
        assert np.array_equal(a, b)
    for a, b in zip(emb.smolvla_positions(pv, nsuf), orc.smolvla_positions(pv.tolist(), nsuf)):
        assert np.array_equal(a, b)


def test_mask_builders_refuse_bad_arguments(emb):
    L = emb.lib()
    assert L.emb_hy_prefix_mask(0, None, None, None) == emb.EMB_ERR_ARG
    assert L.emb_hy_suffix_mask(4, 0, None, None) == emb.EMB_ERR_ARG
    assert L.emb_groot_layer_mask_kind(-1, 2) == emb.EMB_ERR_ARG
    assert L.emb_smolvla_masks(None, 4, 2, None, None, None) == emb.EMB_ERR_ARG
