"""GPU parity of attention under the masks the reference's model graphs build
(HY-VLA, GR00T, SmolVLA), each mask made by the library's host builder (pinned
against the oracle's step-by-step restatement in test_host.py) and the result
checked against the oracle at the model's shape.

Shapes: SmolVLA 15/5 heads of 64 (scripts/convert_smolvla_to_gguf.py:212-214),
chunk 50.  HY-VLA and GR00T take their head counts from the GGUF; the tests
use 16/8 heads of 128 (HY-VLA) and 32 heads of 48 (GR00T's DiT) as stand-ins,
with the sequence structure of the call sites.  Bar
(max-abs 2e-2, mean-rel 1e-3).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import assert_close, rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch, torch.device("cuda")


def _t(torch, dev, a):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to(dev)


def _bf16(orc, rng, shape, scale=1.0):
    return orc.f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


class Pool:
    """One sequence of n_k keys in a randomly permuted page pool (appended by the oracle)."""

    def __init__(self, orc, rng, n_k, hkv, d):
        pages = (n_k + 15) // 16
        self.bt = rng.permutation(pages + 3)[:pages].astype(np.int32)
        total = pages + 3
        self.cap = pages * 16
        self.k = _bf16(orc, rng, (n_k, hkv, d))
        self.v = _bf16(orc, rng, (n_k, hkv, d))
        self.kp = np.zeros(total * hkv * 16 * d, np.uint16)
        self.vp = np.zeros_like(self.kp)
        orc.paged_append(self.k, self.v, hkv * d, np.arange(n_k, dtype=np.int32), self.bt, hkv, d, self.cap,
                         self.kp, self.vp)
        self.n_k, self.hkv, self.d = n_k, hkv, d

    def attend(self, emb, torch, dev, q, hq, n_q, q_pos0=None, **kw):
        out = torch.full((n_q, hq, self.d), float("nan"), dtype=torch.float32, device=dev)
        keep = [_t(torch, dev, x) for x in (q, self.kp, self.vp, self.bt)]
        qp0 = None if q_pos0 is None else _t(torch, dev, np.array([q_pos0], np.int32))
        nk = _t(torch, dev, np.array([self.n_k], np.int32))
        cu = _t(torch, dev, np.array([0, n_q], np.int32))
        emb.paged_attention(q=keep[0], out=out, k_pool=keep[1], v_pool=keep[2], batch=1, hq=hq, hkv=self.hkv,
                            d=self.d, max_q=n_q, scale=1.0 / math.sqrt(self.d), capacity=self.cap, cu_q=cu,
                            n_keys=nk, q_pos0=qp0, block_tables=keep[3], bt_stride=len(self.bt), **kw)
        torch.cuda.synchronize()
        return out.cpu().numpy()


# ---------------- HY-VLA ----------------
def _hy_modality(rng):
    """48 text tokens, then three 64-patch images (one with a single zero inside,
    which keeps its group open), separated by two-token runs of zeros."""
    parts = [np.zeros(48, np.int32)]
    for im in range(3):
        img = np.ones(64, np.int32)
        if im == 1:
            img[20] = 0
        parts += [img, np.zeros(2, np.int32)]
    return np.concatenate(parts)


def test_hy_vla_routed_prefix_attention(emb, orc, torch_dev):
    """Prefix self-attention under make_prefix_mask with patch groups
    (models/hy_vla.cpp:1279-1306, :2801), TOKEN mask on the paged path."""
    torch, dev = torch_dev
    rng = np.random.default_rng(71)
    hq, hkv, d = 16, 8, 128
    mod = _hy_modality(rng)
    n = len(mod)
    n_groups, group_of = emb.hy_patch_groups(mod)
    assert n_groups == 3
    allow, _ = emb.hy_prefix_mask(n, group_of)
    pool = Pool(orc, rng, n, hkv, d)
    q = _bf16(orc, rng, (n, hq, d))
    got = pool.attend(emb, torch, dev, q, hq, n, q_pos0=0, mask_kind=emb.EMB_MASK_TOKEN, mask=_t(torch, dev, allow),
                      mask_q_stride=n)
    want = orc.gqa_attention(q, pool.k, pool.v, n, n, hq, hkv, d, 1.0 / math.sqrt(d), allow=allow, q_pos0=0)
    assert_close(got, want, "HY-VLA prefix")
    # the same mask through the ggml-descriptor face in the reference's F16 form
    _, f16 = emb.hy_prefix_mask(n, group_of)
    got_f = _ggml_face(emb, torch, dev, orc.bf16_to_f32(q), orc.bf16_to_f32(pool.k), orc.bf16_to_f32(pool.v),
                       f16, emb.EMB_GGML_F16, 1.0 / math.sqrt(d))
    assert_close(got_f, want, "HY-VLA prefix, ggml face F16 mask")


def test_hy_vla_expert_with_prefix_attention(emb, orc, torch_dev):
    """Suffix (state + 50 actions) over prefix + suffix keys under full_mask
    (models/hy_vla.cpp:2831-2843): row 0 sees the prefix and itself only."""
    torch, dev = torch_dev
    rng = np.random.default_rng(72)
    hq, hkv, d = 16, 8, 128
    n_pref, n_suf = len(_hy_modality(rng)), 51
    allow, _ = emb.hy_suffix_mask(n_pref, n_suf)
    pool = Pool(orc, rng, n_pref + n_suf, hkv, d)
    q = _bf16(orc, rng, (n_suf, hq, d))
    for splits in (1, 3):
        ws = None
        if splits > 1:
            ws = torch.empty(emb.attn_workspace_bytes(1, n_suf, hq, hkv, d, splits) // 4 + 4, dtype=torch.float32,
                             device=dev)
        got = pool.attend(emb, torch, dev, q, hq, n_suf, mask_kind=emb.EMB_MASK_TOKEN,
                          mask=_t(torch, dev, allow), mask_q_stride=n_pref + n_suf, splits=splits, workspace=ws)
        want = orc.gqa_attention(q, pool.k, pool.v, n_suf, n_pref + n_suf, hq, hkv, d, 1.0 / math.sqrt(d),
                                 allow=allow)
        assert_close(got, want, f"HY-VLA expert with prefix, splits {splits}")


# ---------------- GR00T ----------------
def _ggml_face(emb, torch, dev, q, k, v, mask, mask_type, scale):
    """emb_ggml_flash_attn_ext on f32 q [n_q][hq][D], k/v [n_kv][hkv][D] and a
    mask [n_q][n_kv] of mask_type; returns f32 [n_q][hq][D]."""
    n_q, hq, D = q.shape
    n_kv, hkv = k.shape[0], k.shape[1]
    q_store = _t(torch, dev, np.ascontiguousarray(q.transpose(1, 0, 2), np.float32))
    qd = emb.ggml_tensor(q_store, emb.EMB_GGML_F32, [D, n_q, hq, 1], [1, D, n_q * D, hq * n_q * D])
    kt = _t(torch, dev, np.ascontiguousarray(k, np.float32))
    vt = _t(torch, dev, np.ascontiguousarray(v, np.float32))
    kd = emb.ggml_tensor(kt, emb.EMB_GGML_F32, [D, n_kv, hkv, 1], [1, hkv * D, D, n_kv * hkv * D])
    vd = emb.ggml_tensor(vt, emb.EMB_GGML_F32, [D, n_kv, hkv, 1], [1, hkv * D, D, n_kv * hkv * D])
    mt = _t(torch, dev, np.ascontiguousarray(mask))
    md = emb.ggml_tensor(mt, mask_type, [n_kv, n_q, 1, 1])
    out = torch.full((n_q, hq, D), float("nan"), dtype=torch.float32, device=dev)
    od = emb.ggml_tensor(out, emb.EMB_GGML_F32, [D, hq, n_q, 1])
    emb.ggml_flash_attn_ext(qd, kd, vd, md, od, scale)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_groot_dit_cross_attention_masks(emb, orc, torch_dev):
    """DiT cross-attention of state + 16 action tokens over backbone features
    (models/groot_n1.cpp:328-364) with the text and image masks
    (:708-716), chosen per layer (:656-661); K/V re-projected every step, so
    the whole-tensor face (head_dim 48, run padded)."""
    torch, dev = torch_dev
    rng = np.random.default_rng(73)
    heads, D, n_q = 32, 48, 17
    # backbone: 40 text tokens, 256 image tokens, 24 more text, 8 padding
    valid = np.concatenate([np.ones(320, np.int32), np.zeros(8, np.int32)])
    img = np.concatenate([np.zeros(40, np.int32), np.ones(256, np.int32), np.zeros(32, np.int32)])
    n_kv = len(valid)
    text_m, image_m = emb.groot_cross_masks(valid, img, n_q)
    kinds = [emb.groot_layer_mask_kind(layer, 2) for layer in range(4)]
    assert kinds == [1, 0, 2, 0]
    rb = lambda a: orc.bf16_to_f32(orc.f32_to_bf16(a.astype(np.float32)))
    q = rb(rng.standard_normal((n_q, heads, D)))
    k = rb(rng.standard_normal((n_kv, heads, D)))
    v = rb(rng.standard_normal((n_kv, heads, D)))
    for kind, m in ((1, text_m), (2, image_m)):
        got = _ggml_face(emb, torch, dev, q, k, v, m, emb.EMB_GGML_F32, 1.0 / math.sqrt(D))
        want = orc.gqa_attention(orc.f32_to_bf16(q), orc.f32_to_bf16(k), orc.f32_to_bf16(v), n_q, n_kv, heads,
                                 heads, D, 1.0 / math.sqrt(D), allow=(m == 0).astype(np.uint8), q_pos0=0)
        assert_close(got, want, f"GR00T cross-attention, mask kind {kind}")


# ---------------- SmolVLA ----------------
SMOL_HQ, SMOL_HKV, SMOL_D, SMOL_SUF = 15, 5, 64, 50


def _smol_prefix_valid():
    # two 64-token images, 48 language slots of which the last 13 are padding, the state
    return np.concatenate([np.ones(128 + 35, np.uint8), np.zeros(13, np.uint8), np.ones(1, np.uint8)])


def _round_out(orc, a):
    return orc.bf16_to_f32(orc.f32_to_bf16(np.asarray(a, np.float32))).astype(np.float64)


@pytest.mark.parametrize("q_f32,valid_list", [(False, False), (True, False), (False, True)])
def test_smolvla_expert_self_attention_bf16_p(emb, orc, torch_dev, q_f32, valid_list):
    """Expert self-attention of the 50-token chunk over the cached prefix plus
    itself under full_mask (padding hidden, causal in the chunk;
    models/smolvla.cpp:711-722), with the probabilities rounded to bf16
    before P.V and the output rounded to bf16 (:264-266)."""
    torch, dev = torch_dev
    rng = np.random.default_rng(74 + 2 * q_f32 + valid_list)
    pv = _smol_prefix_valid()
    n_pref = len(pv)
    n_total = n_pref + SMOL_SUF
    _, fm, _ = emb.smolvla_masks(pv, SMOL_SUF)
    pool = Pool(orc, rng, n_total, SMOL_HKV, SMOL_D)
    q = _bf16(orc, rng, (SMOL_SUF, SMOL_HQ, SMOL_D))
    qin = orc.bf16_to_f32(q) if q_f32 else q
    kw = dict(mask_kind=emb.EMB_MASK_ADD, mask=_t(torch, dev, fm), mask_q_stride=n_total, p_bf16=True,
              q_is_f32=q_f32, out_bf16_round=True)
    if valid_list:  # key j read through the valid list (here slot j)
        kw["valid_slots"] = _t(torch, dev, np.arange(n_total, dtype=np.int32))
        kw["valid_stride"] = n_total
    got = pool.attend(emb, torch, dev, qin, SMOL_HQ, SMOL_SUF, **kw)
    scale = 1.0 / math.sqrt(SMOL_D)
    want = _round_out(orc, orc.pbf16_attention(q, pool.k, pool.v, SMOL_SUF, n_total, SMOL_HQ, SMOL_HKV, SMOL_D,
                                               scale, add=fm))
    assert_close(got, want, "SmolVLA expert self-attention (bf16 P)")
    # the same rounding points make it far closer than the bar
    mx, mr = rel_err(got, want)
    assert mr <= 2e-4, mr


def test_smolvla_prefix_and_cross_attention_bf16_p(emb, orc, torch_dev):
    """The prefix pass under prefix_mask (state hidden from the other tokens)
    and the expert's cross-attention over re-projected prefix K/V under
    cross_mask (models/smolvla.cpp:698-723), both with bf16 P.  Also records
    how far the f16-P path lands from this bf16-P reference."""
    torch, dev = torch_dev
    rng = np.random.default_rng(77)
    pv = _smol_prefix_valid()
    n_pref = len(pv)
    pm, _, cm = emb.smolvla_masks(pv, SMOL_SUF)
    scale = 1.0 / math.sqrt(SMOL_D)
    pool = Pool(orc, rng, n_pref, SMOL_HKV, SMOL_D)
    # prefix self-attention: n_pref queries over n_pref keys
    q = _bf16(orc, rng, (n_pref, SMOL_HQ, SMOL_D))
    got = pool.attend(emb, torch, dev, q, SMOL_HQ, n_pref, q_pos0=0, mask_kind=emb.EMB_MASK_ADD,
                      mask=_t(torch, dev, pm), mask_q_stride=n_pref, p_bf16=True, out_bf16_round=True)
    want = _round_out(orc, orc.pbf16_attention(q, pool.k, pool.v, n_pref, n_pref, SMOL_HQ, SMOL_HKV, SMOL_D, scale,
                                               add=pm))
    assert_close(got, want, "SmolVLA prefix (bf16 P)")
    # cross-attention: 50 queries over the prefix keys
    q = _bf16(orc, rng, (SMOL_SUF, SMOL_HQ, SMOL_D))
    got = pool.attend(emb, torch, dev, q, SMOL_HQ, SMOL_SUF, q_pos0=0, mask_kind=emb.EMB_MASK_ADD,
                      mask=_t(torch, dev, cm), mask_q_stride=n_pref, p_bf16=True)
    want = orc.pbf16_attention(q, pool.k, pool.v, SMOL_SUF, n_pref, SMOL_HQ, SMOL_HKV, SMOL_D, scale, add=cm)
    assert_close(got, want, "SmolVLA cross-attention (bf16 P)")
    # the default (f16 P, unnormalised) path against the same bf16-P reference
    got16 = pool.attend(emb, torch, dev, q, SMOL_HQ, SMOL_SUF, q_pos0=0, mask_kind=emb.EMB_MASK_ADD,
                        mask=_t(torch, dev, cm), mask_q_stride=n_pref)
    mx16, mr16 = rel_err(got16, want)
    mx, mr = rel_err(got, want)
    print(f"SmolVLA cross-attention vs bf16-P reference: p_bf16 path mean-rel {mr:.2e}, "
          f"f16-P path mean-rel {mr16:.2e} (max-abs {mx16:.2e})")
    assert mr < mr16


def test_p_bf16_refusals(emb, torch_dev):
    torch, dev = torch_dev
    buf = torch.zeros(1 << 16, dtype=torch.int16, device=dev)
    out = torch.zeros(1 << 14, dtype=torch.float32, device=dev)
    common = dict(q=buf, out=out, k_pool=buf, v_pool=buf, batch=1, hq=2, hkv=1, d=64, max_q=4, scale=0.125,
                  capacity=64, n_keys_uniform=16, p_bf16=True)
    with pytest.raises(RuntimeError):
        emb.paged_attention(**common, splits=2, workspace=out)
    with pytest.raises(RuntimeError):
        emb.paged_attention(**common, mask_kind=emb.EMB_MASK_BLOCKMAP, block_map=buf, block_size=16,
                            block_map_cols=1)
