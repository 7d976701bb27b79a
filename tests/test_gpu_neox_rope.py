"""GPU parity of emb_qkv_neox_rope_append -- pi0.5's NEOX RoPE on the f32 Q/K
projections plus the paged K/V append (models/pi05.cpp:394-408) -- against the
oracle's restatement of ggml_rope_ext (orc_neox_rope_f32).

The device and the oracle both compute theta = pos * theta_scale^i, cos, sin
and the two rotated values in f32, but powf/cosf/sinf come from the device
library on one side and libm on the other, so a value may differ by a few ulp
of theta.  The bar for f32 Q: within the f32 theta error bound of the oracle
test (|err| <= |pair| * (theta * (i + 4) + 4) * 2^-23 per pair) and the
north-star tolerance (max-abs 2e-2, mean-rel 1e-3).  bf16 Q and K: every
element within one bf16 ulp of the bf16 of the oracle's f32 value (a value
whose f32 result lies next to a bf16 rounding boundary may round the other
way) and at least 99% of them bit-identical.  V, its f16 shadow and every cache position
are bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_close, v16_shadow

pytestmark = pytest.mark.gpu

N_PREFIX = 816  # config 1: 816 prefix keys, 51 suffix queries at positions 816 + i


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch, torch.device("cuda")


def _t(torch, dev, a):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to(dev)


def _close_bf16(got, want_f32, bound, what, orc):
    """got: bf16 bits; want_f32: the oracle's f32 values; bound: the f32 theta
    error bound per element.  Each got must be the bf16 rounding of a value
    within bound of the oracle's, and 99% must equal the oracle's own rounding."""
    want = orc.f32_to_bf16(np.ascontiguousarray(want_f32, np.float32))
    g = orc.bf16_to_f32(got).astype(np.float64)
    half_ulp = np.ldexp(1.0, np.frexp(np.abs(g))[1] - 9)  # bf16 keeps 8 significant bits
    err = np.abs(g - want_f32)
    assert np.all(err <= half_ulp + bound), f"{what}: worst excess {np.max(err - half_ulp - bound):.3e}"
    same = np.mean(got == want)
    assert same >= 0.99, f"{what}: only {same:.4f} of the elements bit-identical"


def _theta_bound(x, pos, d):
    """Per-element bound on |device - oracle| for f32 rotated rows x [T][H][d]."""
    half = d // 2
    th = np.asarray(pos, np.float64)[:, None] * 10000.0 ** (-2.0 * np.arange(half) / d)[None, :]
    x = x.astype(np.float64)
    n = np.hypot(x[..., :half], x[..., half:])
    b = n * (th * (np.arange(half) + 4) + 4)[:, None, :] * 2.0 ** -23
    return np.concatenate([b, b], axis=-1) + 1e-6


@pytest.mark.parametrize("D,hq,hkv,fused,q_f32,explicit_pos", [
    (256, 8, 1, False, True, False),   # config 1: three mul_mat outputs, positions 816 + i
    (256, 8, 1, True, False, True),    # one fused row, bf16 Q, positions array
    (128, 8, 2, True, True, True),     # GQA 4:1
    (64, 4, 4, False, False, False),
])
def test_neox_rope_append(emb, orc, torch_dev, D, hq, hkv, fused, q_f32, explicit_pos):
    torch, dev = torch_dev
    rng = np.random.default_rng(D + hq + 3 * hkv + 7 * fused)
    T = 51
    if explicit_pos:
        pos = rng.integers(0, 3000, T).astype(np.int32)
    else:
        pos = (N_PREFIX + np.arange(T)).astype(np.int32)
    if fused:
        ld = (hq + 2 * hkv) * D + 12  # padded [q | k | v] rows
        qkv = (rng.standard_normal((T, ld)) * 2).astype(np.float32)
        q_in, k_in, v_in = qkv[:, :hq * D], qkv[:, hq * D:(hq + hkv) * D], qkv[:, (hq + hkv) * D:(hq + 2 * hkv) * D]
        g = _t(torch, dev, qkv)
        qa, ka, va = g, g[:, hq * D:], g[:, (hq + hkv) * D:]
        ldq_in = ldk = ldv = ld
    else:
        q_in = (rng.standard_normal((T, hq * D)) * 2).astype(np.float32)
        k_in = (rng.standard_normal((T, hkv * D)) * 2).astype(np.float32)
        v_in = (rng.standard_normal((T, hkv * D)) * 2).astype(np.float32)
        qa, ka, va = (_t(torch, dev, a) for a in (q_in, k_in, v_in))
        ldq_in, ldk, ldv = hq * D, hkv * D, hkv * D
    # slots: a permuted page table with one unmapped page, one slot past capacity
    cap = 128
    pages = cap // 16
    bt = rng.permutation(pages).astype(np.int32)
    bt[3] = -1
    slots = rng.permutation(cap)[:T].astype(np.int32)
    slots[5] = cap + 9
    n_el = pages * hkv * 16 * D
    kp = torch.zeros(n_el, dtype=torch.int16, device=dev)
    vp, v16 = torch.zeros_like(kp), torch.zeros_like(kp)
    qo = torch.zeros((T, hq * D), dtype=torch.float32 if q_f32 else torch.int16, device=dev)
    emb.qkv_neox_rope_append(qa, ldq_in, ka, ldk, va, ldv, T, hq, hkv, D, qo, _t(torch, dev, slots),
                             _t(torch, dev, bt), cap, kp, vp, v16_pool=v16,
                             positions=_t(torch, dev, pos) if explicit_pos else None,
                             first_position=0 if explicit_pos else N_PREFIX, freq_base=10000.0, q_out_f32=q_f32)
    torch.cuda.synchronize()
    q_ref = orc.neox_rope(q_in, T, hq, D, positions=pos)
    k_ref = orc.neox_rope(k_in, T, hkv, D, positions=pos)
    if q_f32:
        got = qo.cpu().numpy().reshape(T, hq, D)
        err = np.abs(got.astype(np.float64) - q_ref)
        bound = _theta_bound(q_in.reshape(T, hq, D), pos, D)
        assert np.all(err <= bound), f"Q: worst err/bound {np.max(err / bound):.3f}"
        assert_close(got, q_ref.astype(np.float64), "Q f32")
    else:
        _close_bf16(qo.cpu().numpy().view(np.uint16).reshape(T, hq, D), q_ref,
                    _theta_bound(q_in.reshape(T, hq, D), pos, D), "Q bf16", orc)
    # expected cache: K and V rows of every appended token at its page row
    got_k = kp.cpu().numpy().view(np.uint16)
    kmask = np.zeros(n_el, bool)
    vpool = np.zeros(n_el, np.uint16)
    v_bits = orc.f32_to_bf16(np.ascontiguousarray(v_in, np.float32)).reshape(T, hkv, D)
    k_bound = _theta_bound(k_in.reshape(T, hkv, D), pos, D)
    rows = []  # (got bits, oracle f32, bound) of every appended K row
    for i, s in enumerate(slots):
        if s < 0 or s >= cap or bt[s // 16] < 0:
            continue
        for h in range(hkv):
            base = (bt[s // 16] * hkv + h) * 16 * D + (s % 16) * D
            rows.append((got_k[base:base + D], k_ref[i, h], k_bound[i, h]))
            kmask[base:base + D] = True
            vpool[(bt[s // 16] * hkv + h) * 16 * D + np.arange(D) * 16 + s % 16] = v_bits[i, h]
    assert np.all(got_k[~kmask] == 0), "K written outside the appended rows"
    _close_bf16(*(np.concatenate(c) for c in zip(*rows)), "K in the cache", orc)
    assert np.array_equal(vp.cpu().numpy().view(np.uint16), vpool), "V pool not bit-exact"
    assert np.array_equal(v16.cpu().numpy().view(np.uint16), v16_shadow(vpool, D)), "V shadow not bit-exact"


def test_pi05_layer_produce_then_attend(emb, orc, torch_dev):
    """One pi0.5 expert layer at config-1 shape (8/1 heads, D 256): the prefix
    K/V (positions 0..815) and the suffix Q/K/V (positions 816 + i) go through
    the producer, then attention over the 867 keys with the f32 Q the producer
    wrote (models/pi05.cpp:394-418).  Oracle: ggml's rope (orc_neox_rope_f32)
    on the same inputs, K/V/Q rounded to bf16, then orc_gqa_attention_bf16."""
    torch, dev = torch_dev
    rng = np.random.default_rng(5)
    hq, hkv, D, T = 8, 1, 256, 51
    n_k = N_PREFIX + T
    pages = (n_k + 15) // 16 + 2
    cap = pages * 16
    bt = rng.permutation(pages).astype(np.int32)
    n_el = pages * hkv * 16 * D
    kp = torch.zeros(n_el, dtype=torch.int16, device=dev)
    vp, v16 = torch.zeros_like(kp), torch.zeros_like(kp)
    btd = _t(torch, dev, bt)
    # prefix layer: rope at positions 0..815, K/V into slots 0..815 (its Q is the
    # prefix's own attention input, not used here)
    kpre = rng.standard_normal((N_PREFIX, D)).astype(np.float32)
    vpre = rng.standard_normal((N_PREFIX, D)).astype(np.float32)
    qpre = torch.zeros((N_PREFIX, hq * D), dtype=torch.int16, device=dev)
    qpre_in = torch.zeros((N_PREFIX, hq * D), dtype=torch.float32, device=dev)
    emb.qkv_neox_rope_append(qpre_in, hq * D, _t(torch, dev, kpre), D, _t(torch, dev, vpre), D, N_PREFIX, hq,
                             hkv, D, qpre, _t(torch, dev, np.arange(N_PREFIX, dtype=np.int32)), btd, cap, kp, vp,
                             v16_pool=v16, first_position=0, q_out_f32=False)
    # expert layer: suffix at positions 816 + i, slots 816..866
    qs = rng.standard_normal((T, hq * D)).astype(np.float32)
    ks = rng.standard_normal((T, D)).astype(np.float32)
    vs = rng.standard_normal((T, D)).astype(np.float32)
    qo = torch.zeros((T, hq * D), dtype=torch.float32, device=dev)
    emb.qkv_neox_rope_append(_t(torch, dev, qs), hq * D, _t(torch, dev, ks), D, _t(torch, dev, vs), D, T, hq, hkv,
                             D, qo, _t(torch, dev, (N_PREFIX + np.arange(T)).astype(np.int32)), btd, cap, kp, vp,
                             v16_pool=v16, first_position=N_PREFIX)
    out = torch.zeros((T, hq * D), dtype=torch.float32, device=dev)
    ws = torch.empty(emb.lib().emb_attn_workspace_bytes(1, T, hq, hkv, D, 3), dtype=torch.uint8, device=dev)
    emb.paged_attention(q=qo, q_is_f32=True, out=out, k_pool=kp, v_pool=vp, v16_pool=v16, batch=1, hq=hq,
                        hkv=hkv, d=D, max_q=T, scale=1.0 / 16, capacity=cap, block_tables=btd,
                        bt_stride=pages, n_keys_uniform=n_k, splits=3, workspace=ws)
    torch.cuda.synchronize()
    k_all = np.concatenate([orc.neox_rope(kpre, N_PREFIX, hkv, D, first_pos=0),
                            orc.neox_rope(ks, T, hkv, D, first_pos=N_PREFIX)])
    v_all = np.concatenate([vpre, vs]).reshape(n_k, hkv, D)
    q_ref = orc.neox_rope(qs, T, hq, D, first_pos=N_PREFIX)
    want = orc.gqa_attention(orc.f32_to_bf16(q_ref), orc.f32_to_bf16(k_all), orc.f32_to_bf16(v_all), T, n_k,
                             hq, hkv, D, 1.0 / 16)
    assert_close(out.cpu().numpy().reshape(T, hq, D), want.astype(np.float64), "pi0.5 layer attention")
    # the appended cache reads back as the oracle's rows (logical slot j -> page bt[j // 16])
    got_k = kp.cpu().numpy().view(np.uint16).reshape(pages, 16, D)
    k_rows = got_k[bt[np.arange(n_k) // 16], np.arange(n_k) % 16]
    same = np.mean(k_rows == orc.f32_to_bf16(np.ascontiguousarray(k_all.reshape(n_k, D))))
    assert same >= 0.99, f"K cache: only {same:.4f} bit-identical"
