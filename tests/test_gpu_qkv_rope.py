"""GPU parity of emb_qkv_norm_rope_append (per-head q/k RMSNorm + RoPE + paged
append) against the oracle's restatement of the Cosmos3 kernels
(kernels/cosmos3/cosmos3_qwen_language_cuda.cu:52-153).

Q and K are bf16 results of f32 arithmetic whose transcendental functions
(sin, cos, pow, 1/sqrt) come from the device library here and libm in the
oracle, so a value on a bf16 rounding boundary may land one ulp apart: the
bar is the north-star tolerance (max-abs 2e-2, mean-rel 1e-3) with at least
99% of the elements bit-identical.  V and every cache position are bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_close, v16_shadow

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch, torch.device("cuda")


def _t(torch, dev, a):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to(dev)


def _close_bf16(got, want, what):
    gf, wf = (x.astype(np.uint16) for x in (got, want))
    same = np.mean(gf == wf)
    import oracle
    assert_close(oracle.bf16_to_f32(gf), oracle.bf16_to_f32(wf).astype(np.float64), what)
    assert same >= 0.99, f"{what}: only {same:.4f} of the elements bit-identical"


@pytest.mark.parametrize("D,hq,hkv,rope_kind,norm", [
    (128, 8, 2, 1, True),    # Qwen GQA 4:1, plain RoPE
    (128, 4, 4, 2, True),    # MRoPE
    (128, 6, 2, 0, True),    # norm only
    (64, 4, 2, 1, False),    # RoPE only, pairs across lanes l and l ^ 32
    (256, 2, 1, 2, True),
])
def test_qkv_norm_rope_append(emb, orc, torch_dev, D, hq, hkv, rope_kind, norm):
    torch, dev = torch_dev
    rng = np.random.default_rng(D + hq + 10 * rope_kind)
    T = 37
    width = (hq + 2 * hkv) * D
    ld = width + 24  # padded rows
    qkv = orc.f32_to_bf16((rng.standard_normal((T, ld)) * 2.5).astype(np.float32))
    qg = orc.f32_to_bf16(rng.uniform(0.5, 1.5, D).astype(np.float32)) if norm else None
    kg = orc.f32_to_bf16(rng.uniform(0.5, 1.5, D).astype(np.float32)) if norm else None
    pos = rng.integers(0, 4000, 3 * T).astype(np.int32)
    theta, first = 1e6, 123
    # slots: a permuted page table, one unmapped page and one out-of-range slot
    cap = 64
    pages = cap // 16
    bt = np.array([2, -1, 0, 3], np.int32)
    slots = rng.permutation(cap)[:T].astype(np.int32)
    slots[5] = cap + 3  # skipped
    n_el = pages * hkv * 16 * D
    kp = torch.zeros(n_el, dtype=torch.int16, device=dev)
    vp, v16 = torch.zeros_like(kp), torch.zeros_like(kp)
    qo = torch.zeros((T, hq * D), dtype=torch.int16, device=dev)
    emb.qkv_norm_rope_append(_t(torch, dev, qkv), ld, T, hq, hkv, D, qo, _t(torch, dev, slots),
                             _t(torch, dev, bt), cap, kp, vp, v16_pool=v16,
                             q_gamma=None if qg is None else _t(torch, dev, qg),
                             k_gamma=None if kg is None else _t(torch, dev, kg), eps=1e-6,
                             rope_kind=rope_kind, rope_theta=theta, first_position=first,
                             position_ids=_t(torch, dev, pos))
    torch.cuda.synchronize()
    kw = dict(gamma=None, eps=1e-6, rope_kind=rope_kind, theta=theta, first_pos=first, pos_ids=pos, ld=ld)
    q_ref = orc.head_norm_rope(qkv, T, hq, D, **{**kw, "gamma": qg})
    k_ref = orc.head_norm_rope(np.ascontiguousarray(qkv[:, hq * D:]), T, hkv, D,
                               **{**kw, "gamma": kg, "ld": ld - hq * D})
    _close_bf16(qo.cpu().numpy().view(np.uint16).reshape(T, hq, D), q_ref, "Q")
    # expected cache: K and V rows of every appended token at its page row
    kpool = np.zeros(n_el, np.uint16)
    vpool = np.zeros(n_el, np.uint16)
    v_in = qkv[:, (hq + hkv) * D:(hq + 2 * hkv) * D].reshape(T, hkv, D)
    got_k = kp.cpu().numpy().view(np.uint16)
    kmask = np.zeros(n_el, bool)
    for i, s in enumerate(slots):
        if s < 0 or s >= cap or bt[s // 16] < 0:
            continue
        for h in range(hkv):
            base = (bt[s // 16] * hkv + h) * 16 * D
            kpool[base + (s % 16) * D: base + (s % 16) * D + D] = k_ref[i, h]
            kmask[base + (s % 16) * D: base + (s % 16) * D + D] = True
            vpool[base + np.arange(D) * 16 + s % 16] = v_in[i, h]
    assert np.all(got_k[~kmask] == 0), "K written outside the appended rows"
    _close_bf16(got_k[kmask], kpool[kmask], "K in the cache")
    assert np.array_equal(vp.cpu().numpy().view(np.uint16), vpool), "V pool not bit-exact"
    assert np.array_equal(v16.cpu().numpy().view(np.uint16), v16_shadow(vpool, D)), "V shadow not bit-exact"
