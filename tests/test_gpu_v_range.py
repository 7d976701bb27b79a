"""V of any finite magnitude through every attention path.

The kernels' fast P.V product takes V as f16, which holds |v| up to 65504 and
keeps full precision down to 2^-14.  Rows whose output comes out non-finite,
or whose largest |O| is below 2^-12 over a non-empty key set, are recomputed
by the kernel from the bf16 pool with bf16 P.V (P split into two bf16 parts),
and split-K partials carry a per-row power-of-two scale.  These tests feed V
scaled by 1e30, 3e5 (just past the f16 range), 6e4 (inside it), 1e-7 and a mix
of page magnitudes, through the register, shadow (LDS copy) and valid-list
paths, split-K, and the reference-named faces, against the oracle (reference
semantics: lingbot_flex_attn_cuda.cu:651-720 and :502-582, all f32).  The bar
(max-abs 2e-2, mean-rel 1e-3) is applied to the output divided by the V scale,
i.e. relative to the data's own magnitude.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import assert_close
from test_gpu_attn import Seqs, _bf16, _t

pytestmark = pytest.mark.gpu

SCALES = [("huge", 1e30), ("past_f16", 3e5), ("near_f16_max", 6e4), ("tiny", 1e-7)]


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch, torch.device("cuda")


def _close_rows(got, ref, what):
    """The bar per row, relative to that row's magnitude (rows mixing V scales)."""
    g = np.asarray(got, np.float64).reshape(-1, got.shape[-1])
    r = np.asarray(ref, np.float64).reshape(-1, ref.shape[-1])
    s = np.maximum(np.abs(r).max(axis=1, keepdims=True), 1e-300)
    assert_close(g / s, r / s, what)


@pytest.mark.parametrize("d,hq,hkv", [(256, 8, 1), (128, 4, 2), (64, 2, 2)])
@pytest.mark.parametrize("name,vs", SCALES)
def test_paged_paths_any_v_range(emb, orc, torch_dev, d, hq, hkv, name, vs):
    """Register and shadow staging (required bit-identical by Seqs.run), with
    and without split-K, a ragged two-sequence batch."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0x5EED + d + hq)
    s = Seqs(orc, rng, [300, 77], [40, 13], hq, hkv, d, v_scale=vs)
    sc = 1 / math.sqrt(d)
    for splits in (1, 3):
        got = s.run(emb, torch, dev, sc, splits=splits)
        for b in range(2):
            ref = s.oracle(orc, b, sc)
            assert np.all(np.isfinite(got[b])), f"{name} d={d} splits={splits} b={b}: non-finite"
            assert_close(got[b] / vs, ref / vs, f"{name} d={d} splits={splits} b={b}")
            if s.ks_out is not None:
                assert_close(s.ks_out[b] / vs, ref / vs, f"{name} d={d} b={b} key-split")


def test_mixed_page_magnitudes(emb, orc, torch_dev):
    """Keys 96..159 carry V scaled by 1e5 (past f16), keys 400.. by 1e-6, the
    rest N(0,1): rows lean on different ranges; cfg1-like shape, split-K 3."""
    torch, dev = torch_dev
    rng = np.random.default_rng(77)

    def vscale(k):
        f = np.ones((k, 1, 1))
        f[96:160] = 1e5
        f[400:] = 1e-6
        return f
    s = Seqs(orc, rng, [867], [51], 8, 1, 256, v_scale=vscale)
    for splits in (1, 3):
        got = s.run(emb, torch, dev, 1 / 16, splits=splits)[0]
        _close_rows(got, s.oracle(orc, 0, 1 / 16), f"mixed splits={splits}")
        if splits == 1:
            _close_rows(s.ks_out[0], s.oracle(orc, 0, 1 / 16), "mixed key-split")


@pytest.mark.parametrize("name,vs", SCALES)
def test_valid_list_any_v_range(emb, orc, torch_dev, name, vs):
    """The valid-slot-list path (LingBot runtime KV) through emb_paged_attention
    and through the reference-named f32 faces."""
    torch, dev = torch_dev
    rng = np.random.default_rng(31)
    H, D, cap, nq = 4, 128, 200, 21
    ck = _bf16(orc, rng, (cap, H, D))
    cv = orc.f32_to_bf16((rng.standard_normal((cap, H, D)) * vs).astype(np.float32))
    q = _bf16(orc, rng, (nq, H, D))
    valid = np.concatenate([np.arange(16, 48), rng.choice(np.arange(48, cap), 90, replace=False), [-1],
                            np.arange(0, 7)]).astype(np.int32)
    n_pages = cap // 16 + 1
    bt = rng.permutation(n_pages + 2)[:n_pages].astype(np.int32)
    kp = np.zeros((n_pages + 2) * H * 16 * D, np.uint16)
    vp = np.zeros_like(kp)
    orc.paged_append(ck, cv, H * D, np.arange(cap, dtype=np.int32), bt, H, D, cap, kp, vp)
    ref = orc.runtime_kv_attn(orc.bf16_to_f32(q).reshape(-1), orc.bf16_to_f32(ck).reshape(-1),
                              orc.bf16_to_f32(cv).reshape(-1), valid, nq, H, D, 0.1).reshape(nq, H, D)
    out = torch.zeros((nq, H, D), dtype=torch.float32, device=dev)
    keep = [_t(torch, dev, x) for x in (q, kp, vp, bt, valid)]
    emb.paged_attention(q=keep[0], out=out, k_pool=keep[1], v_pool=keep[2], batch=1, hq=H, hkv=H, d=D,
                        max_q=nq, scale=0.1, capacity=cap, cu_q=_t(torch, dev, np.array([0, nq], np.int32)),
                        n_keys=_t(torch, dev, np.array([len(valid)], np.int32)), block_tables=keep[3],
                        bt_stride=n_pages, valid_slots=keep[4], valid_stride=len(valid))
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy() / vs, ref / vs, f"valid list {name}")
    # reference-named faces over an f32 cache the update face fills
    L = emb.lib()
    cfk = torch.zeros(cap * H * D, dtype=torch.float32, device=dev)
    cfv = torch.zeros_like(cfk)
    tk = _t(torch, dev, orc.bf16_to_f32(ck))
    tv = _t(torch, dev, orc.bf16_to_f32(cv))
    tq = _t(torch, dev, orc.bf16_to_f32(q))
    slots = _t(torch, dev, np.arange(cap, dtype=np.int32))
    assert L.lingbot_runtime_kv_update_f32(tk.data_ptr(), tv.data_ptr(), cfk.data_ptr(), cfv.data_ptr(),
                                           slots.data_ptr(), cap, H, D, cap, None) == 0
    o2 = torch.zeros((nq, H, D), dtype=torch.float32, device=dev)
    assert L.lingbot_runtime_kv_attn_f32(tq.data_ptr(), cfk.data_ptr(), cfv.data_ptr(), keep[4].data_ptr(),
                                         o2.data_ptr(), nq, len(valid), H, D, 0.1, None) == 0, emb.last_error()
    torch.cuda.synchronize()
    assert_close(o2.cpu().numpy() / vs, ref / vs, f"lingbot_runtime_kv_attn_f32 {name}")


@pytest.mark.parametrize("name,vs", SCALES)
def test_faces_any_v_range(emb, orc, torch_dev, name, vs):
    """lingbot_flex_attn_f32, the Cosmos3 GQA faces and the ggml entry with f32 V."""
    torch, dev = torch_dev
    rng = np.random.default_rng(47)
    bfv = lambda shape, s=1.0: orc.bf16_to_f32(orc.f32_to_bf16((rng.standard_normal(shape) * s).astype(np.float32)))
    # flex: 70 queries, 93 keys, 3 heads, D 128, a random CSR
    sq, sk, H, D, bs = 70, 93, 3, 128, 16
    q, k, v = bfv((sq, H, D)), bfv((sk, H, D)), bfv((sk, H, D), vs)
    qb, kb = (sq + bs - 1) // bs, (sk + bs - 1) // bs
    rp, ci = [0], []
    for r in range(qb):
        ci += [c for c in range(kb) if rng.random() < 0.7 or c == 0]
        rp.append(len(ci))
    rp, ci = np.array(rp, np.int32), np.array(ci, np.int32)
    scale = 1 / math.sqrt(D)
    ref = orc.flex_attention(q, k, v, rp, ci, None, sq, sk, H, D, bs, scale).reshape(sq, H, D)
    out = torch.full((sq, H, D), float("nan"), dtype=torch.float32, device=dev)
    d_ = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    emb.flex_attention(d_(q), d_(k), d_(v), d_(rp), d_(ci), out, sq, sk, H, D, bs, scale)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy() / vs, ref / vs, f"flex {name}")

    # Cosmos3 causal GQA (output rounded to bf16 values, as the reference rounds it)
    T, hq, hkv, Dc = 160, 8, 2, 128
    qc, kc, vc = (orc.f32_to_bf16((rng.standard_normal(sh) * s).astype(np.float32))
                  for sh, s in (((T, hq, Dc), 1.0), ((T, hkv, Dc), 1.0), ((T, hkv, Dc), vs)))
    f = lambda a: torch.from_numpy(orc.bf16_to_f32(a).reshape(a.shape[0], -1).copy()).to(dev)
    qd, kd, vd = f(qc), f(kc), f(vc)
    y = torch.full((T, hq * Dc), float("nan"), dtype=torch.float32, device=dev)
    L = emb.lib()
    assert L.cosmos3_qwen_causal_gqa_attention_f32(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), y.data_ptr(),
                                                   T, hq * Dc, hkv * Dc, hq, hkv, Dc, None) == 0, emb.last_error()
    torch.cuda.synchronize()
    rb = lambda a: orc.bf16_to_f32(orc.f32_to_bf16(a))
    ref = rb(orc.gqa_attention(qc, kc, vc, T, T, hq, hkv, Dc, 1 / math.sqrt(Dc), chunk=1))
    assert_close(y.cpu().numpy().reshape(T, hq, Dc) / vs, ref / vs, f"cosmos3 causal {name}")

    # ggml flash_attn_ext with F32 K/V (staged to bf16) and no mask
    n_q, n_kv, hq, hkv, Dg = 19, 70, 4, 2, 64
    qg = bfv((1, n_q, hq, Dg))
    kg, vg = bfv((1, n_kv, hkv, Dg)), bfv((1, n_kv, hkv, Dg), vs)
    G = hq // hkv
    refg = np.zeros((n_q, hq, Dg))
    for h in range(hq):
        s_ = qg[0, :, h, :].astype(np.float64) @ kg[0, :, h // G, :].astype(np.float64).T * 0.125
        p_ = np.exp(s_ - s_.max(axis=1, keepdims=True))
        refg[:, h, :] = (p_ / p_.sum(axis=1, keepdims=True)) @ vg[0, :, h // G, :].astype(np.float64)
    tq, tk, tv = d_(qg), d_(kg), d_(vg)
    qdd = emb.ggml_tensor(tq, emb.EMB_GGML_F32, [Dg, n_q, hq, 1], [1, hq * Dg, Dg, n_q * hq * Dg])
    kdd = emb.ggml_tensor(tk, emb.EMB_GGML_F32, [Dg, n_kv, hkv, 1], [1, hkv * Dg, Dg, n_kv * hkv * Dg])
    vdd = emb.ggml_tensor(tv, emb.EMB_GGML_F32, [Dg, n_kv, hkv, 1], [1, hkv * Dg, Dg, n_kv * hkv * Dg])
    og = torch.full((n_q, hq, Dg), float("nan"), dtype=torch.float32, device=dev)
    odd = emb.ggml_tensor(og, emb.EMB_GGML_F32, [Dg, hq, n_q, 1])
    emb.ggml_flash_attn_ext(qdd, kdd, vdd, None, odd, 0.125)
    torch.cuda.synchronize()
    assert_close(og.cpu().numpy() / vs, refg / vs, f"ggml {name}")


def test_dim_halves_of_different_magnitude(emb, orc, torch_dev):
    """V dims [0, 128) scaled by 1e-2 and dims [128, 256) by 1e3 (cfg1-like
    shape, split-K 1 and 3).  Split partials carry a power-of-two scale per
    half of the dims (2^17 apart here): each half is held to the bar relative
    to its own magnitude, so a half merged with the other half's scale would
    fail."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0xD1A5)
    dscale = np.concatenate([np.full(128, 1e-2), np.full(128, 1e3)])[None, None, :]
    s = Seqs(orc, rng, [867, 300], [51, 20], 8, 1, 256, v_scale=lambda k: dscale)
    for splits in (1, 3):
        got = s.run(emb, torch, dev, 1 / 16, splits=splits)
        for b in range(2):
            ref = s.oracle(orc, b, 1 / 16)
            for h, sl in enumerate((slice(0, 128), slice(128, 256))):
                mag = float(np.abs(ref[..., sl]).max())
                assert_close(got[b][..., sl] / mag, ref[..., sl] / mag, f"splits={splits} b={b} dims half {h}")
                if s.ks_out is not None:
                    assert_close(s.ks_out[b][..., sl] / mag, ref[..., sl] / mag, f"key-split b={b} dims half {h}")
