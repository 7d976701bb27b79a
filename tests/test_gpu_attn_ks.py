"""GPU parity of the key-split attention kernel (emb_attn_args.kernel =
EMB_ATTN_KEY_SPLIT: a workgroup per 32 query rows, its four waves splitting the
keys, partials merged in the kernel) against the oracle.

Bar: max |gpu - oracle| <= 2e-2 and sum|gpu - oracle| / sum|oracle| <= 1e-3 on
identical seeded bf16 inputs.  The cases here are
the kernel's own edges: the zero-row rules (unmapped pages, keys at or past the
capacity or the table), tables longer than the 128 entries a wave holds in
registers, empty sequences, Q in f32, bf16 output rounding, the automatic
kernel choice and the calls the kernel refuses.  The shapes the bench times
(pi0.5 step, multi-session batches) are checked in test_gpu_attn.py, whose
Seqs.run runs this kernel next to the row-tile kernel wherever it applies.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import assert_close
from test_gpu_attn import Seqs, _t

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch, torch.device("cuda")


def _launch(emb, torch, dev, s, scale, kernel, q=None, q_is_f32=False, capacity=None, bt=None, bt_stride=None,
            uniform=False, **kw):
    """One launch over the Seqs pool (its f16 shadow given); per-sequence outputs."""
    from conftest import v16_shadow
    q = np.concatenate(s.q) if q is None else q
    bt = s.bt if bt is None else bt
    keep = [_t(torch, dev, q), _t(torch, dev, s.kp), _t(torch, dev, s.vp), _t(torch, dev, v16_shadow(s.vp, s.d)),
            _t(torch, dev, np.ascontiguousarray(bt)), _t(torch, dev, s.cu_q),
            _t(torch, dev, np.array(s.n_keys, np.int32))]
    out = torch.full((int(s.cu_q[-1]), s.hq, s.d), float("nan"), dtype=torch.float32, device=dev)
    emb.paged_attention(q=keep[0], q_is_f32=q_is_f32, out=out, k_pool=keep[1], v_pool=keep[2], v16_pool=keep[3],
                        batch=len(s.n_q), hq=s.hq, hkv=s.hkv, d=s.d, max_q=max(s.n_q), scale=scale,
                        capacity=s.cap if capacity is None else capacity,
                        cu_q=None if uniform else keep[5], n_keys=None if uniform else keep[6],
                        n_keys_uniform=s.n_keys[0] if uniform else 0,
                        block_tables=keep[4], bt_stride=s.bt_stride if bt_stride is None else bt_stride,
                        kernel=kernel, **kw)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    return [o[s.cu_q[b]:s.cu_q[b + 1]] for b in range(len(s.n_q))]


def _zeroed(s, b, keys):
    """K and V of sequence b with the given key rows zeroed (what the kernels
    read for missing keys)."""
    k, v = s.k[b].copy(), s.v[b].copy()
    k[keys] = 0
    v[keys] = 0
    return k, v


@pytest.mark.parametrize("d", [128, 256])
def test_zero_rows_unmapped_page_and_capacity(emb, orc, torch_dev, d):
    """An unmapped page inside a sequence (table entry -1) and a capacity below
    the key count: those keys are zero K/V rows -- score 0, inside the softmax,
    value 0 -- in both kernels, as in the oracle fed zeroed rows."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0xE3BD0100 + d)
    s = Seqs(orc, rng, [300, 867, 45], [51, 20, 3], 8, 1, d)
    bt = s.bt.copy()
    bt[1, 5] = -1                 # keys 80..95 of sequence 1
    cap = 800                     # keys 800..866 of sequence 1
    scale = 1 / math.sqrt(d)
    for kernel in (emb.EMB_ATTN_KEY_SPLIT, emb.EMB_ATTN_ROW_TILES):
        got = _launch(emb, torch, dev, s, scale, kernel, capacity=cap, bt=bt)
        for b in range(3):
            missing = list(range(80, 96)) + list(range(800, 867)) if b == 1 else []
            k, v = _zeroed(s, b, missing)
            ref = orc.gqa_attention(s.q[b], k, v, s.n_q[b], s.n_keys[b], s.hq, s.hkv, d, scale)
            assert_close(got[b], ref, f"kernel {kernel} d {d} seq {b}")


def test_table_shorter_than_keys(emb, orc, torch_dev):
    """bt_stride * 16 below n_keys: keys past the table are zero rows."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0xE3BD0101)
    s = Seqs(orc, rng, [867], [51], 8, 1, 256)
    stride = 40  # 640 keys covered
    got = _launch(emb, torch, dev, s, 1 / 16, emb.EMB_ATTN_KEY_SPLIT, bt=s.bt[:, :stride], bt_stride=stride)[0]
    k, v = _zeroed(s, 0, list(range(640, 867)))
    assert_close(got, orc.gqa_attention(s.q[0], k, v, 51, 867, 8, 1, 256, 1 / 16), "table of 40 pages")


def test_long_tables_and_empty_sequences(emb, orc, torch_dev):
    """Tables past the 128 entries each wave holds in registers (2100 keys:
    132 pages), a sequence without queries, one with a single key, one with
    no keys (its rows are zeros), D 256, G 8; then the uniform form."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0xE3BD0102)
    s = Seqs(orc, rng, [2100, 40, 1, 0, 97], [51, 0, 7, 5, 1], 8, 1, 256)
    got = _launch(emb, torch, dev, s, 1 / 16, emb.EMB_ATTN_KEY_SPLIT)
    for b in range(5):
        if s.n_q[b] == 0:
            assert got[b].size == 0
            continue
        ref = s.oracle(orc, b, 1 / 16)
        if s.n_keys[b] == 0:
            assert np.array_equal(got[b], np.zeros_like(got[b])), "no keys: zero rows"
        assert_close(got[b], ref, f"seq {b} ({s.n_keys[b]} keys, {s.n_q[b]} queries)")
    u = Seqs(orc, rng, [2100] * 3, [51] * 3, 8, 1, 256)
    a = _launch(emb, torch, dev, u, 1 / 16, emb.EMB_ATTN_KEY_SPLIT)
    b = _launch(emb, torch, dev, u, 1 / 16, emb.EMB_ATTN_KEY_SPLIT, uniform=True)
    for i in range(3):
        assert np.array_equal(a[i], b[i]), f"uniform form differs, seq {i}"
        assert_close(b[i], u.oracle(orc, i, 1 / 16), f"uniform seq {i}")


@pytest.mark.parametrize("d,hq,hkv", [(256, 8, 1), (128, 4, 2), (128, 2, 2)])
def test_q_f32_and_bf16_output(emb, orc, torch_dev, d, hq, hkv):
    """Q given as f32 is rounded to bf16 (nearest even) in the kernel: equal to
    the bf16 Q bit for bit when the f32 values are bf16 values, within the bar
    of the oracle on the rounded Q otherwise; out_bf16_round stores exactly
    the bf16 rounding of the plain output."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0xE3BD0103 + d + hq)
    s = Seqs(orc, rng, [300, 77], [40, 13], hq, hkv, d)
    sc = 1 / math.sqrt(d)
    plain = _launch(emb, torch, dev, s, sc, emb.EMB_ATTN_KEY_SPLIT)
    q32 = orc.bf16_to_f32(np.concatenate(s.q)).astype(np.float32)
    same = _launch(emb, torch, dev, s, sc, emb.EMB_ATTN_KEY_SPLIT, q=q32, q_is_f32=True)
    for b in range(2):
        assert np.array_equal(plain[b], same[b]), f"f32 Q of bf16 values, seq {b}"
    qn = (q32 + rng.standard_normal(q32.shape).astype(np.float32) * 1e-3).astype(np.float32)
    got = _launch(emb, torch, dev, s, sc, emb.EMB_ATTN_KEY_SPLIT, q=qn, q_is_f32=True)
    qr = orc.f32_to_bf16(qn)
    for b in range(2):
        qb = qr[s.cu_q[b]:s.cu_q[b + 1]]
        ref = orc.gqa_attention(qb, s.k[b], s.v[b], s.n_q[b], s.n_keys[b], hq, hkv, d, sc)
        assert_close(got[b], ref, f"general f32 Q seq {b}")
    rnd = _launch(emb, torch, dev, s, sc, emb.EMB_ATTN_KEY_SPLIT, out_bf16_round=True)
    for b in range(2):
        want = orc.bf16_to_f32(orc.f32_to_bf16(np.ascontiguousarray(plain[b])))
        assert np.array_equal(rnd[b], want), f"bf16 output seq {b}"


def test_auto_choice_and_determinism(emb, orc, torch_dev):
    """kernel 0 (automatic) runs the key-split kernel for at most 512 rows per
    kv head and the row tiles above; repeated launches are bit-identical."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0xE3BD0104)
    small = Seqs(orc, rng, [867, 500], [51, 64], 8, 1, 256)   # 408 / 512 rows
    big = Seqs(orc, rng, [300], [65], 8, 1, 256)               # 520 rows
    ks = _launch(emb, torch, dev, small, 1 / 16, emb.EMB_ATTN_KEY_SPLIT)
    ks2 = _launch(emb, torch, dev, small, 1 / 16, emb.EMB_ATTN_KEY_SPLIT)
    auto = _launch(emb, torch, dev, small, 1 / 16, emb.EMB_ATTN_AUTO)
    for b in range(2):
        assert np.array_equal(ks[b], ks2[b]), "repeat differs"
        assert np.array_equal(ks[b], auto[b]), "auto did not take the key-split kernel at <= 512 rows"
        assert_close(ks[b], small.oracle(orc, b, 1 / 16), f"seq {b}")
    rt = _launch(emb, torch, dev, big, 1 / 16, emb.EMB_ATTN_ROW_TILES)
    auto = _launch(emb, torch, dev, big, 1 / 16, emb.EMB_ATTN_AUTO)
    assert np.array_equal(rt[0], auto[0]), "auto did not take the row tiles above 512 rows"


def test_refused_calls(emb, orc, torch_dev):
    """The key-split kernel refuses what it does not implement, before any
    launch: a mask other than FULL, split-K, no f16 shadow, head_dim 64."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0xE3BD0105)
    s = Seqs(orc, rng, [100], [4], 4, 2, 128)
    cases = [dict(mask_kind=emb.EMB_MASK_CHUNK, chunk=16), dict(splits=2, workspace=None)]
    for kw in cases:
        with pytest.raises(RuntimeError, match="rc=-4"):
            if "workspace" in kw:
                ws = torch.zeros(emb.attn_workspace_bytes(1, 4, 4, 2, 128, 2) // 4 + 4, device=dev)
                kw = dict(kw, workspace=ws)
            _launch(emb, torch, dev, s, 0.1, emb.EMB_ATTN_KEY_SPLIT, **kw)
    q = torch.zeros(4 * 4 * 128, dtype=torch.int16, device=dev)
    out = torch.zeros(4 * 4 * 128, dtype=torch.float32, device=dev)
    pool = torch.zeros(16 * 2 * 128 * 8, dtype=torch.int16, device=dev)
    with pytest.raises(RuntimeError, match="rc=-4"):
        emb.paged_attention(q=q, out=out, k_pool=pool, v_pool=pool, batch=1, hq=4, hkv=2, d=128, max_q=4,
                            scale=0.1, capacity=16, n_keys_uniform=16, kernel=emb.EMB_ATTN_KEY_SPLIT)
    q64 = torch.zeros(4 * 4 * 64, dtype=torch.int16, device=dev)
    with pytest.raises(RuntimeError, match="rc=-4"):
        emb.paged_attention(q=q64, out=out, k_pool=pool, v_pool=pool, v16_pool=pool, batch=1, hq=4, hkv=2, d=64,
                            max_q=4, scale=0.1, capacity=16, n_keys_uniform=16, kernel=emb.EMB_ATTN_KEY_SPLIT)
