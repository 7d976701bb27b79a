"""Device-resident slot metadata (emb_dev_cache_*) against the oracle's
LingBotKVCache restatement, bit for bit: the slots each call returns, the
valid-slot list, its length, the failure status, and the (id, mask, is_pred)
state after every call; then a LingBot step whose slots and valid list never
leave the device, against the same step driven from the host cache."""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import assert_close

pytestmark = pytest.mark.gpu

CAPACITY_ERR = -3  # EMB_ERR_CAPACITY


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch, torch.device("cuda")


def _ops(rng, n_ops, cap):
    ops = []
    for _ in range(n_ops):
        r = rng.random()
        k = int(rng.integers(1, max(2, cap // 3)))
        if r < 0.4:
            ops.append(("update", k, int(rng.random() < 0.3)))
        elif r < 0.65:
            ops.append(("mode0", k, 0))
        elif r < 0.75:
            ops.append(("clear_pred", 0, 0))
        elif r < 0.85:
            ops.append(("update_restore", k, 0))
        elif r < 0.97:
            ops.append(("chunk", max(1, cap // 4), 0))
        else:
            ops.append(("update", cap + 1, 0))  # fails after evicting everything
    return ops


def _check_state(torch, dev_cache, orc_cache, what):
    torch.cuda.synchronize()
    ia, ma, pa = dev_cache.state()
    ib, mb, pb = orc_cache.state()
    assert np.array_equal(ia, ib), f"{what}: id"
    assert np.array_equal(ma, mb), f"{what}: mask"
    assert np.array_equal(pa, pb), f"{what}: is_pred"


def _replay(emb, orc, torch, dev, cap, ops, legacy):
    d = emb.DevSlotCache(cap, dev, legacy_clear_pred=legacy)
    o = orc.Cache(cap, legacy)
    for i, (op, k, pred) in enumerate(ops):
        what = f"op {i} {op} k={k}"
        if op in ("update", "chunk", "update_restore"):
            mode = 1 if pred else 2
            slots, valid, nv, st = d.update(k, mode)
            sb = o.update_meta(k, pred)
            torch.cuda.synchronize()
            if sb is None:
                # failure (k > capacity): status and return code say so, and what
                # a queued append / attention would read lists no key
                assert int(st.item()) == CAPACITY_ERR and d.last_rc == CAPACITY_ERR, what
                assert np.all(slots.cpu().numpy() == -1) and int(nv.item()) == 0, what
            else:
                assert d.last_rc == 0, what
                assert int(st.item()) == 0, what
                assert np.array_equal(slots.cpu().numpy(), sb), what
                vb = o.collect_valid()
                assert int(nv.item()) == len(vb), what
                assert np.array_equal(valid[:len(vb)].cpu().numpy(), vb), what
                if op == "update_restore":  # the mode-0 path without the fast path
                    d.restore(slots, k)
                    o.restore(sb)
        elif op == "mode0":
            slots, valid, nv, st = d.update(k, 0)
            sb, vb = o.prepare_mode0(k)
            torch.cuda.synchronize()
            if sb is None:
                assert int(st.item()) == CAPACITY_ERR and d.last_rc == CAPACITY_ERR, what
                assert np.all(slots.cpu().numpy() == -1) and int(nv.item()) == 0, what
            else:
                assert int(st.item()) == 0, what
                assert np.array_equal(slots.cpu().numpy(), sb), what
                assert int(nv.item()) == len(vb), what
                assert np.array_equal(valid[:len(vb)].cpu().numpy(), vb), what
        else:
            d.clear_pred()
            o.clear_pred()
        _check_state(torch, d, o, what)


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("legacy", [False, True])
def test_dev_cache_random_sequences(emb, orc, torch_dev, seed, legacy):
    torch, dev = torch_dev
    rng = np.random.default_rng(100 + seed)
    # seeds 0-2 stage the metadata in LDS; seed 3 is past that limit (14336 slots)
    cap = [int(rng.integers(8, 60)), int(rng.integers(8, 60)), int(rng.integers(900, 3000)),
           int(rng.integers(15000, 20000))][seed]
    _replay(emb, orc, torch, dev, cap, _ops(rng, 40, cap), legacy)


def test_dev_cache_lingbot_window(emb, orc, torch_dev):
    """Config-3 metadata: 9-chunk window of 1560-token chunks (14040 slots): clean
    chunk inserts past the point where the oldest chunk is evicted, prediction
    chunks cleared, mode-0 denoise queries in between."""
    torch, dev = torch_dev
    cap, C = 14040, 1560
    ops = []
    for step in range(14):
        ops.append(("mode0", C, 0))
        ops.append(("update", C, 1))
        ops.append(("clear_pred", 0, 0))
        ops.append(("update", C, 0))
    _replay(emb, orc, torch, dev, cap, ops, False)


def test_dev_cache_golden_fixture(emb, torch_dev):
    """The committed LingBot metadata sequence (tests/golden/slot_cache.json)."""
    import json
    from pathlib import Path
    torch, dev = torch_dev
    fx = json.loads((Path(__file__).resolve().parent / "golden" / "slot_cache.json").read_text())
    d = emb.DevSlotCache(fx["capacity"], dev)
    last = None
    for i, st in enumerate(fx["steps"]):
        what = f"step {i} {st['op']}"
        if st["op"] == "update":
            slots, _, _, status = d.update(st["n"], 1 if st["pred"] else 2)
            torch.cuda.synchronize()
            if st["slots"] is None:
                assert int(status.item()) == CAPACITY_ERR, what
            else:
                assert list(slots.cpu().numpy()) == st["slots"], what
        elif st["op"] == "mode0":
            slots, valid, nv, _ = d.update(st["n"], 0)
            torch.cuda.synchronize()
            last = slots.clone()
            assert list(slots.cpu().numpy()) == st["slots"], what
            assert list(valid[:int(nv.item())].cpu().numpy()) == st["valid"], what
        elif st["op"] == "restore":
            d.restore(last, len(last))
        else:
            d.clear_pred()
        ids, m, pr = d.state()
        assert list(ids) == st["id"] and list(m) == st["mask"] and list(pr) == st["is_pred"], what


def test_device_resident_lingbot_step(emb, orc, torch_dev):
    """Two chunk steps (append a chunk, attend over the valid slots) with the
    metadata, slots and valid list kept on the device, against the same steps
    with the host cache and host-to-device copies: identical cache bytes and
    identical attention output; the output also within the bar of the oracle."""
    torch, dev = torch_dev
    H, D, C, W = 4, 128, 96, 3
    cap = C * W
    pages = cap // 16
    rng = np.random.default_rng(7)
    bt = torch.from_numpy(rng.permutation(pages).astype(np.int32)).to(dev)
    bf = lambda shape: orc.f32_to_bf16(rng.standard_normal(shape).astype(np.float32))
    chunks = [(bf((C, H, D)), bf((C, H, D)), bf((C, H, D))) for _ in range(W + 1)]
    t = lambda a: torch.from_numpy(a.view(np.int16)).to(dev)
    outs = {}
    for path in ("device", "host"):
        kp = torch.zeros(pages * H * 16 * D, dtype=torch.int16, device=dev)
        vp = torch.zeros_like(kp)
        if path == "device":
            dc = emb.DevSlotCache(cap, dev)
        else:
            hc = emb.SlotCache(cap)
        res = []
        for q, k, v in chunks:
            out = torch.zeros((C, H, D), dtype=torch.float32, device=dev)
            if path == "device":
                slots, valid, nv, st = dc.update(C, 2)
                n_keys = nv
            else:
                sl, rc = hc.update_meta(C, 0)
                assert rc == 0
                slots = torch.from_numpy(sl.astype(np.int32)).to(dev)
                vl = hc.collect_valid()
                valid = torch.from_numpy(vl.astype(np.int32)).to(dev)
                n_keys = torch.tensor([len(vl)], dtype=torch.int32, device=dev)
            emb.kv_append(t(k), t(v), H * D, C, slots, bt, cap, kp, vp, H, D)
            emb.paged_attention(q=t(q), out=out, k_pool=kp, v_pool=vp, batch=1, hq=H, hkv=H, d=D, max_q=C,
                                scale=1 / math.sqrt(D), capacity=cap,
                                cu_q=torch.tensor([0, C], dtype=torch.int32, device=dev), n_keys=n_keys,
                                block_tables=bt, bt_stride=pages, valid_slots=valid, valid_stride=cap)
            torch.cuda.synchronize()
            res.append(out.cpu().numpy())
        outs[path] = (res, kp.cpu().numpy(), vp.cpu().numpy())
    for i in range(len(chunks)):
        assert np.array_equal(outs["device"][0][i], outs["host"][0][i]), f"step {i}"
    assert np.array_equal(outs["device"][1], outs["host"][1]) and np.array_equal(outs["device"][2], outs["host"][2])
    # the last step attends over chunks 1..3 (chunk 0 evicted) in slot order
    o = orc.Cache(cap)
    for _ in chunks:
        o.update_meta(C, 0)
    valid = o.collect_valid()
    ks = np.zeros((cap, H, D), np.uint16)
    vs = np.zeros((cap, H, D), np.uint16)
    hist = orc.Cache(cap)
    for q, k, v in chunks:
        s = hist.update_meta(C, 0)
        ks[s], vs[s] = k, v
    q = chunks[-1][0]
    ref = orc.gqa_attention(q, ks[valid], vs[valid], C, len(valid), H, H, D, 1 / math.sqrt(D))
    assert_close(outs["device"][0][-1], ref, "device-resident step")
