"""GPU parity of paged KV append / gather / eviction: bit-exact against the
oracle's restatement of the reference's slot semantics
(models/lingbot_va.cpp:8740-8997, kernels/lingbot/lingbot_flex_attn_cuda.cu:626-649,875-898)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import v16_shadow

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch, torch.device("cuda")


def _t(torch, dev, a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to(dev)


def _np(t):
    a = t.cpu().numpy()
    return a.view(np.uint16) if a.dtype == np.int16 else a


@pytest.mark.parametrize("H,D,extra,n", [(24, 128, 0, 120), (1, 256, 64, 120), (2, 64, 8, 120),
                                         # 768 (16 tokens, head) groups and more: a workgroup each
                                         (24, 128, 0, 700), (8, 256, 64, 2048), (16, 64, 8, 1030)])
def test_append_gather_bit_exact(emb, orc, torch_dev, H, D, extra, n):
    torch, dev = torch_dev
    rng = np.random.default_rng(H * 1000 + D + n)
    cap = max(200, n + 80)
    n_pages_seq = (cap + 15) // 16
    pool_pages = n_pages_seq + 7
    bt = rng.permutation(pool_pages)[:n_pages_seq].astype(np.int32)
    bt[3] = -1                                       # an unmapped page: its slots are skipped
    stride = H * D + extra                           # rows read from a wider fused buffer
    k = rng.integers(0, 65536, (n, stride), dtype=np.uint16)
    v = rng.integers(0, 65536, (n, stride), dtype=np.uint16)
    slots = rng.choice(np.arange(-5, cap + 5), n, replace=False).astype(np.int32)
    kp0 = rng.integers(0, 65536, pool_pages * H * 16 * D, dtype=np.uint16)
    vp0 = rng.integers(0, 65536, pool_pages * H * 16 * D, dtype=np.uint16)
    # oracle
    kp_ref, vp_ref = kp0.copy(), vp0.copy()
    orc.paged_append(k, v, stride, slots, bt, H, D, cap, kp_ref, vp_ref)
    # device, with the f16 V shadow written alongside
    kp, vpl = _t(torch, dev, kp0), _t(torch, dev, vp0)
    v16 = _t(torch, dev, v16_shadow(vp0, D))
    emb.kv_append(_t(torch, dev, k), _t(torch, dev, v), stride, n, _t(torch, dev, slots),
                  _t(torch, dev, bt), cap, kp, vpl, H, D, v16_pool=v16)
    torch.cuda.synchronize()
    assert np.array_equal(_np(kp), kp_ref) and np.array_equal(_np(vpl), vp_ref)
    # shadow = f16 of the bf16 pool in the documented order (NaN sources: payloads not compared)
    exp16 = v16_shadow(vp_ref, D)
    src_nan = np.isnan(v16_shadow(vp_ref, D).view(np.float16))
    got16 = _np(v16)
    assert np.array_equal(got16[~src_nan], exp16[~src_nan]), "V shadow differs"
    assert np.isnan(got16.view(np.float16)[src_nan]).all()
    # gather: valid list in arbitrary order with out-of-range entries
    valid = np.concatenate([rng.permutation(slots[(slots >= 0) & (slots < cap)]), [-1, cap, 7]]).astype(np.int32)
    gk0 = rng.integers(0, 65536, (len(valid), H, D), dtype=np.uint16)
    gk_ref, gv_ref = gk0.copy(), gk0.copy()
    orc.paged_gather(kp_ref, vp_ref, valid, bt, H, D, cap, gk_ref, gv_ref)
    gk, gv = _t(torch, dev, gk0), _t(torch, dev, gk0)
    emb.kv_gather(kp, vpl, _t(torch, dev, valid), len(valid), _t(torch, dev, bt), cap, gk, gv, H, D)
    torch.cuda.synchronize()
    assert np.array_equal(_np(gk), gk_ref) and np.array_equal(_np(gv), gv_ref)


def test_chunk_eviction_sequence_bit_exact(emb, orc, torch_dev):
    """LingBot-style sliding window: capacity = 9 chunks, one chunk appended per
    step, the oldest chunk evicted once full.  Every step the gathered K/V (in
    valid-slot order) must equal the reference's token-slot cache."""
    torch, dev = torch_dev
    H, D, C, W = 4, 128, 40, 9
    cap = C * W
    rng = np.random.default_rng(11)
    pool = emb.PagePool((cap + 15) // 16 + 3, seed=0xE3BD0003)
    cache = emb.SlotCache(cap)
    cache.bind_pool(pool)
    ocache = orc.Cache(cap)
    ref_k = np.zeros((cap, H, D), np.uint16)
    ref_v = np.zeros((cap, H, D), np.uint16)
    n_pages = (cap + 15) // 16 + 3
    kp = torch.zeros(n_pages * H * 16 * D, dtype=torch.int16, device=dev)
    vpl = torch.zeros_like(kp)
    for step in range(W + 5):
        pred = step % 4 == 3
        ks = rng.integers(0, 65536, (C, H, D), dtype=np.uint16)
        vs = rng.integers(0, 65536, (C, H, D), dtype=np.uint16)
        slots, rc = cache.update_meta(C, pred)
        assert rc == 0
        oslots = ocache.update_meta(C, pred)
        assert np.array_equal(slots, oslots)
        orc.slot_update(ks, vs, ref_k, ref_v, oslots.astype(np.int32), H, D, cap)
        bt = cache.block_table()
        emb.kv_append(_t(torch, dev, ks), _t(torch, dev, vs), H * D, C,
                      _t(torch, dev, slots.astype(np.int32)), _t(torch, dev, bt), cap, kp, vpl, H, D)
        if step == W + 2:
            cache.clear_pred()
            ocache.clear_pred()
        valid = cache.collect_valid()
        assert np.array_equal(valid, ocache.collect_valid())
        gk = torch.empty((len(valid), H, D), dtype=torch.int16, device=dev)
        gv = torch.empty_like(gk)
        emb.kv_gather(kp, vpl, _t(torch, dev, valid.astype(np.int32)), len(valid), _t(torch, dev, bt), cap,
                      gk, gv, H, D)
        torch.cuda.synchronize()
        ok = np.zeros((len(valid), H, D), np.uint16)
        ov = np.zeros_like(ok)
        orc.slot_gather(ref_k, ref_v, valid.astype(np.int32), H, D, cap, ok, ov)
        assert np.array_equal(_np(gk), ok) and np.array_equal(_np(gv), ov), step


@pytest.mark.parametrize("cap,n", [(50, 30), (5600, 5500)])  # 5500 tokens: the (16 tokens, head) workgroups
def test_reference_named_f32_update_gather(emb, orc, torch_dev, cap, n):
    torch, dev = torch_dev
    H, D = 3, 64
    rng = np.random.default_rng(2 + n)
    kb = orc.f32_to_bf16(rng.standard_normal((n, H, D)).astype(np.float32))
    vb = orc.f32_to_bf16(rng.standard_normal((n, H, D)).astype(np.float32))
    kf, vf = orc.bf16_to_f32(kb), orc.bf16_to_f32(vb)
    slots = rng.permutation(cap)[:n].astype(np.int32)
    slots[0] = -1
    ck = torch.zeros(cap * H * D, dtype=torch.float32, device=dev)
    cv = torch.zeros_like(ck)
    L = emb.lib()
    assert L.lingbot_runtime_kv_update_f32(_t(torch, dev, kf).data_ptr(), _t(torch, dev, vf).data_ptr(),
                                           ck.data_ptr(), cv.data_ptr(), _t(torch, dev, slots).data_ptr(),
                                           n, H, D, cap, None) == 0
    valid = np.sort(slots[1:]).astype(np.int32)
    gk = torch.zeros((len(valid), H, D), dtype=torch.float32, device=dev)
    gv = torch.zeros_like(gk)
    assert L.lingbot_runtime_kv_gather_f32(ck.data_ptr(), cv.data_ptr(), _t(torch, dev, valid).data_ptr(),
                                           gk.data_ptr(), gv.data_ptr(), len(valid), H, D, cap, None) == 0
    torch.cuda.synchronize()
    src = {int(s): i for i, s in enumerate(slots)}
    idx = [src[int(s)] for s in valid]
    assert np.array_equal(gk.cpu().numpy(), kf[idx]) and np.array_equal(gv.cpu().numpy(), vf[idx])


def test_reference_named_f32_update_narrows_general_f32(emb, orc, torch_dev):
    """lingbot_runtime_kv_update_f32 on general f32 K/V (not bf16-representable,
    RNE ties included, large and tiny magnitudes): the cache holds bf16, so the
    gather returns bf16_rne(x) widened to f32 -- bit-exact to that rounding, not
    to the f32 input (the reference's own f32 cache would return x itself;
    kernels/lingbot/lingbot_flex_attn_cuda.cu:626-649)."""
    torch, dev = torch_dev
    H, D, cap, n = 2, 64, 64, 48
    rng = np.random.default_rng(91)
    k = rng.standard_normal((n, H, D)).astype(np.float32)
    v = (rng.standard_normal((n, H, D)) * np.float32(1e30)).astype(np.float32)
    kb = k.view(np.uint32)
    kb[0, 0, :8] = (kb[0, 0, :8] & 0xFFFE0000) | 0x8000  # exact halfway, even bf16 LSB: rounds down
    kb[1, 0, :8] = (kb[1, 0, :8] & 0xFFFE0000) | 0x18000  # exact halfway, odd bf16 LSB: rounds up
    v[2, 1, :4] = np.float32(1e-30)
    v[3, 1, :4] = np.float32(-7.1e-7)
    slots = np.arange(n, dtype=np.int32)
    ck = torch.zeros(cap * H * D, dtype=torch.float32, device=dev)
    cv = torch.zeros_like(ck)
    L = emb.lib()
    assert L.lingbot_runtime_kv_update_f32(_t(torch, dev, k).data_ptr(), _t(torch, dev, v).data_ptr(),
                                           ck.data_ptr(), cv.data_ptr(), _t(torch, dev, slots).data_ptr(),
                                           n, H, D, cap, None) == 0
    gk = torch.zeros((n, H, D), dtype=torch.float32, device=dev)
    gv = torch.zeros_like(gk)
    assert L.lingbot_runtime_kv_gather_f32(ck.data_ptr(), cv.data_ptr(), _t(torch, dev, slots).data_ptr(),
                                           gk.data_ptr(), gv.data_ptr(), n, H, D, cap, None) == 0
    torch.cuda.synchronize()
    want_k = orc.bf16_to_f32(orc.f32_to_bf16(k))
    want_v = orc.bf16_to_f32(orc.f32_to_bf16(v))
    assert np.array_equal(gk.cpu().numpy(), want_k)
    assert np.array_equal(gv.cpu().numpy(), want_v)
    assert not np.array_equal(want_k, k)  # the inputs really needed rounding
