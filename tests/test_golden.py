"""The committed golden fixtures (tests/golden/, written by make_golden.py with
numpy alone) against the CPU oracle, the host slot cache, and -- marked gpu --
the HIP kernels through the C ABI."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from conftest import assert_close, v16_shadow

GOLDEN = Path(__file__).resolve().parent / "golden"
ATT = np.load(GOLDEN / "attention.npz")
FLEX = np.load(GOLDEN / "flex_smoke.npz")
W8 = np.load(GOLDEN / "marlin_w8.npz")
SLOTS = json.loads((GOLDEN / "slot_cache.json").read_text())
CASES = ["pi05", "chunk", "addmask"]


def _case(name):
    nq, nk, hq, hkv, d = (int(x) for x in ATT[f"{name}_dims"])
    kw = {}
    if f"{name}_chunk" in ATT:
        kw = dict(chunk=int(ATT[f"{name}_chunk"]), window=int(ATT[f"{name}_window"]))
    if f"{name}_add" in ATT:
        kw = dict(add=ATT[f"{name}_add"])
    return (ATT[f"{name}_q"], ATT[f"{name}_k"], ATT[f"{name}_v"], nq, nk, hq, hkv, d,
            float(ATT[f"{name}_scale"]), kw, ATT[f"{name}_out"])


# ---------------- CPU: the oracle and the host library ----------------
def test_oracle_matches_flex_smoke_fixture(orc):
    S, H, D, BS = (int(FLEX[x]) for x in ("S", "H", "D", "BS"))
    got = orc.flex_attention(FLEX["q"], FLEX["k"], FLEX["v"], FLEX["row_ptr"], FLEX["col_idx"], FLEX["mask"],
                             S, S, H, D, BS, float(FLEX["scale"]))
    assert np.abs(got - FLEX["out"]).max() < 1e-5  # the reference smoke's own bar


@pytest.mark.parametrize("name", CASES)
def test_oracle_matches_attention_fixture(orc, name):
    q, k, v, nq, nk, hq, hkv, d, scale, kw, out = _case(name)
    got = orc.gqa_attention(q, k, v, nq, nk, hq, hkv, d, scale, **kw)
    assert np.abs(got - out).max() < 1e-5, name


def test_oracle_matches_marlin_fixture(orc):
    M, K, N = int(W8["M"]), int(W8["K"]), int(W8["N"])
    assert np.array_equal(orc.marlin_pack_w8(W8["w"]), W8["qweight"])
    yb, _ = orc.w8a16_gemm(W8["x"], W8["qweight"], W8["s_stored"], M, K, N)
    assert np.array_equal(yb, W8["y"])


def _replay_slots(cache):
    last = None
    for i, st in enumerate(SLOTS["steps"]):
        what = f"step {i} ({st['op']})"
        if st["op"] == "update":
            got = cache.update_meta(st["n"], st["pred"])
            assert (got is None if st["slots"] is None else list(got) == st["slots"]), what
        elif st["op"] == "mode0":
            last, valid = cache.prepare_mode0(st["n"])
            assert list(last) == st["slots"] and list(valid) == st["valid"], what
        elif st["op"] == "restore":
            cache.restore(last)
        else:
            cache.clear_pred()
        ids, m, pr = cache.state()
        assert list(ids) == st["id"] and list(m) == st["mask"] and list(pr) == st["is_pred"], what
        assert cache.next_id() == st["next_id"] and list(cache.collect_valid()) == st["valid_after"], what


def test_oracle_matches_slot_cache_fixture(orc):
    _replay_slots(orc.Cache(SLOTS["capacity"]))


class _HostCache:
    """The host library's slot cache with the oracle's return conventions."""

    def __init__(self, emb, capacity):
        self.c = emb.SlotCache(capacity)

    def update_meta(self, n, pred):
        return self.c.update_meta(n, pred)[0]

    def prepare_mode0(self, n):
        return self.c.prepare_mode0(n)[:2]

    def __getattr__(self, name):
        return getattr(self.c, name)


def test_host_slot_cache_matches_fixture(emb):
    _replay_slots(_HostCache(emb, SLOTS["capacity"]))


# ---------------- GPU: the kernels through the C ABI ----------------
@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch, torch.device("cuda")


def _dev(torch, dev, a):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to(dev)


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_paged_attention_matches_fixture(emb, torch_dev, name):
    """Keys appended through emb_kv_append into a reversed page order, then the
    attention through the f16-shadow (DMA) path, split 1 and 2."""
    torch, dev = torch_dev
    q, k, v, nq, nk, hq, hkv, d, scale, kw, out = _case(name)
    pages = (nk + 15) // 16
    bt = np.arange(pages)[::-1].astype(np.int32).copy()
    n_el = pages * hkv * 16 * d
    kp = torch.zeros(n_el, dtype=torch.int16, device=dev)
    vp, v16 = torch.zeros_like(kp), torch.zeros_like(kp)
    emb.kv_append(_dev(torch, dev, k), _dev(torch, dev, v), hkv * d, nk, _dev(torch, dev, np.arange(nk, dtype=np.int32)),
                  _dev(torch, dev, bt), pages * 16, kp, vp, hkv, d, v16_pool=v16)
    mask = {}
    if "chunk" in kw:
        mask = dict(mask_kind=emb.EMB_MASK_CHUNK, chunk=kw["chunk"], window=kw["window"])
    elif "add" in kw:
        mask = dict(mask_kind=emb.EMB_MASK_ADD, mask=_dev(torch, dev, kw["add"]), mask_q_stride=nk)
    torch.cuda.synchronize()
    # the f16 shadow the append wrote is the one the layout defines
    assert np.array_equal(v16.cpu().numpy().view(np.uint16), v16_shadow(vp.cpu().numpy().view(np.uint16), d))
    for splits in (1, 2):
        ws = None
        if splits > 1:
            ws = torch.zeros(emb.attn_workspace_bytes(1, nq, hq, hkv, d, splits) // 4 + 4, dtype=torch.float32,
                             device=dev)
        o = torch.full((nq, hq, d), float("nan"), dtype=torch.float32, device=dev)
        emb.paged_attention(q=_dev(torch, dev, q), out=o, k_pool=kp, v_pool=vp, v16_pool=v16, batch=1, hq=hq,
                            hkv=hkv, d=d, max_q=nq, scale=scale, capacity=pages * 16, n_keys_uniform=nk,
                            block_tables=_dev(torch, dev, bt), bt_stride=pages, splits=splits, workspace=ws, **mask)
        torch.cuda.synchronize()
        assert_close(o.cpu().numpy(), out, f"{name} splits {splits}")


@pytest.mark.gpu
def test_flex_face_matches_smoke_fixture(emb, torch_dev):
    torch, dev = torch_dev
    S, H, D, BS = (int(FLEX[x]) for x in ("S", "H", "D", "BS"))
    o = torch.full((S * H * D,), float("nan"), dtype=torch.float32, device=dev)
    emb.flex_attention(_dev(torch, dev, FLEX["q"]), _dev(torch, dev, FLEX["k"]), _dev(torch, dev, FLEX["v"]),
                       _dev(torch, dev, FLEX["row_ptr"]), _dev(torch, dev, FLEX["col_idx"]), o, S, S, H, D, BS,
                       float(FLEX["scale"]), token_mask=_dev(torch, dev, FLEX["mask"]))
    torch.cuda.synchronize()
    # q and k are rounded to bf16 for the MFMA: the bar is the attention tolerance
    assert_close(o.cpu().numpy(), FLEX["out"], "flex smoke")


@pytest.mark.gpu
def test_w8a16_gemm_matches_fixture(emb, torch_dev):
    torch, dev = torch_dev
    M, K, N = int(W8["M"]), int(W8["K"]), int(W8["N"])
    y = torch.zeros((M, N), dtype=torch.int16, device=dev)
    emb.w8a16_gemm(_dev(torch, dev, W8["x"]), _dev(torch, dev, W8["qweight"]), _dev(torch, dev, W8["s_stored"]),
                   M, K, N, y)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint16), W8["y"])
