"""GPU parity of the whole-tensor faces: the reference-named block-sparse
attention (kernels/lingbot/lingbot_flex_attn_cuda.cu:502-624) against the
oracle's restatement of it, its in-source known-answer smoke (:1010-1076), and
the ggml flash_attn_ext descriptor entry against a float64 evaluation of
softmax(scale q.k + mask) v with GQA broadcast."""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch, torch.device("cuda")


def _dev(torch, dev, a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _bf16_valued(orc, rng, shape, scale=1.0):
    """f32 values exactly representable in bf16 (so the kernel's bf16 rounding of Q/K is exact)."""
    return orc.bf16_to_f32(orc.f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32)))


def test_flex_smoke_known_answer(emb):
    assert emb.lib().lingbot_flex_attn_cuda_smoke(None) == 0, emb.last_error()


def _random_csr(rng, qb, kb, p_keep):
    rp, ci = [0], []
    for r in range(qb):
        cols = [c for c in range(kb) if rng.random() < p_keep]
        if r == 1:
            cols = []  # a query block that sees nothing: its rows give 0
        ci += cols
        rp.append(len(ci))
    return np.array(rp, np.int32), np.array(ci if ci else [0], np.int32)


@pytest.mark.parametrize("D", [64, 128, 256, 8, 96])
@pytest.mark.parametrize("masked", [False, True])
def test_flex_matches_oracle(emb, orc, torch_dev, D, masked):
    torch, dev = torch_dev
    rng = np.random.default_rng(D * 10 + masked)
    sq, sk, H, bs = 70, 93, 3, 16
    q = _bf16_valued(orc, rng, (sq, H, D))
    k = _bf16_valued(orc, rng, (sk, H, D))
    v = _bf16_valued(orc, rng, (sk, H, D))
    rp, ci = _random_csr(rng, (sq + bs - 1) // bs, (sk + bs - 1) // bs, 0.6)
    tm = None
    if masked:
        tm = (rng.random((sq, sk)) < 0.7).astype(np.uint8)
        tm[5, :] = 0  # a row whose listed blocks are all masked out
    scale = 1.0 / math.sqrt(D)
    ref = orc.flex_attention(q, k, v, rp, ci, tm, sq, sk, H, D, bs, scale).reshape(sq, H, D)
    out = torch.full((sq, H, D), float("nan"), dtype=torch.float32, device=dev)
    emb.flex_attention(_dev(torch, dev, q), _dev(torch, dev, k), _dev(torch, dev, v), _dev(torch, dev, rp),
                       _dev(torch, dev, ci), out, sq, sk, H, D, bs, scale,
                       token_mask=None if tm is None else _dev(torch, dev, tm))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.all(got[bs:2 * bs] == 0.0)  # the empty query block
    assert_close(got, ref, f"flex D={D} masked={masked}")


def _ggml_ref(q, k, v, mask, scale):
    """q [B][n_q][hq][D], k/v [Bk][n_kv][hkv][D], mask [Bm][n_q][n_kv] or None -> [B][n_q][hq][D] (float64)."""
    B, n_q, hq, D = q.shape
    hkv = k.shape[2]
    G = hq // hkv
    out = np.zeros((B, n_q, hq, D))
    for b in range(B):
        kb = k[b if k.shape[0] > 1 else 0].astype(np.float64)
        vb = v[b if v.shape[0] > 1 else 0].astype(np.float64)
        for h in range(hq):
            s = q[b, :, h, :].astype(np.float64) @ kb[:, h // G, :].T * scale
            if mask is not None:
                s = s + mask[b if mask.shape[0] > 1 else 0].astype(np.float64)
            s = s - s.max(axis=1, keepdims=True)
            p = np.exp(s)
            out[b, :, h, :] = (p / p.sum(axis=1, keepdims=True)) @ vb[:, h // G, :]
    return out


@pytest.mark.parametrize("D,hq,hkv,B,kvb,exact", [(128, 8, 2, 2, 2, True), (64, 4, 4, 1, 1, True),
                                                  (256, 8, 1, 2, 1, True), (80, 6, 3, 1, 1, True),
                                                  (128, 8, 2, 2, 2, False)])
def test_ggml_flash_attn_ext(emb, orc, torch_dev, D, hq, hkv, B, kvb, exact):
    torch, dev = torch_dev
    rng = np.random.default_rng(D + hq + B)
    n_q, n_kv, pad = 37, 150, 64
    if exact:  # values bf16 can hold: only the P -> f16 step is rounded
        q = _bf16_valued(orc, rng, (B, n_q, hq, D))
        k = _bf16_valued(orc, rng, (kvb, n_kv, hkv, D)).astype(np.float16)
        v = _bf16_valued(orc, rng, (kvb, n_kv, hkv, D)).astype(np.float16)
    else:  # general f16 K/V and f32 Q (the kernel rounds Q and K to bf16)
        q = rng.standard_normal((B, n_q, hq, D)).astype(np.float32)
        k = rng.standard_normal((kvb, n_kv, hkv, D)).astype(np.float16)
        v = rng.standard_normal((kvb, n_kv, hkv, D)).astype(np.float16)
    # additive F16 mask [B][n_q_pad][n_kv]: causal-ish with a finite bias, padded rows garbage
    m = np.zeros((B, pad, n_kv), np.float32)
    for b in range(B):
        for i in range(n_q):
            m[b, i, n_kv - n_q + i + 1 + b:] = -np.inf
            m[b, i, : 7 * (b + 1)] -= 2.5
    m[:, n_q:, :] = 123.0
    m16 = m.astype(np.float16)
    scale = 1.0 / math.sqrt(D)
    ref = _ggml_ref(q, k.astype(np.float32), v.astype(np.float32), m16[:, :n_q].astype(np.float32), scale)

    # q stored as [B][hq][n_q][D] and described permuted as [D, n_q, hq, B] (ggml's permute(q, 0, 2, 1, 3))
    q_store = _dev(torch, dev, np.ascontiguousarray(q.transpose(0, 2, 1, 3)))
    qd = emb.ggml_tensor(q_store, emb.EMB_GGML_F32, [D, n_q, hq, B], [1, D, n_q * D, hq * n_q * D])
    kt, vt = _dev(torch, dev, k), _dev(torch, dev, v)
    kd = emb.ggml_tensor(kt, emb.EMB_GGML_F16, [D, n_kv, hkv, kvb], [1, hkv * D, D, n_kv * hkv * D])
    vd = emb.ggml_tensor(vt, emb.EMB_GGML_F16, [D, n_kv, hkv, kvb], [1, hkv * D, D, n_kv * hkv * D])
    mt = _dev(torch, dev, m16)
    md = emb.ggml_tensor(mt, emb.EMB_GGML_F16, [n_kv, pad, 1, B])
    # flash_attn_ext's own result layout [D, hq, n_q, B]
    out = torch.full((B, n_q, hq, D), float("nan"), dtype=torch.float32, device=dev)
    od = emb.ggml_tensor(out, emb.EMB_GGML_F32, [D, hq, n_q, B])
    emb.ggml_flash_attn_ext(qd, kd, vd, md, od, scale)
    # the MUL_MAT -> SOFT_MAX -> MUL_MAT layout [D, n_q, hq, B] written through dst strides
    out2 = torch.full((B, hq, n_q, D), float("nan"), dtype=torch.float32, device=dev)
    od2 = emb.ggml_tensor(out2, emb.EMB_GGML_F32, [D, hq, n_q, B], [1, n_q * D, D, hq * n_q * D])
    emb.ggml_flash_attn_ext(qd, kd, vd, md, od2, scale)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    got2 = out2.cpu().numpy().transpose(0, 2, 1, 3)
    assert np.array_equal(got, got2)
    if exact:
        assert_close(got, ref, f"ggml D={D} hq={hq} hkv={hkv} B={B}")
    else:
        # The path computes Q.K^T in bf16 (the tolerance contract is stated on
        # bf16 inputs): against the reference on bf16-rounded Q and K it meets
        # the contract; against the unrounded reference only that rounding
        # remains (a few 1e-3 relative).
        rb = lambda a: orc.bf16_to_f32(orc.f32_to_bf16(np.asarray(a, np.float32)))
        ref_b = _ggml_ref(rb(q), rb(k.astype(np.float32)), v.astype(np.float32),
                          m16[:, :n_q].astype(np.float32), scale)
        assert_close(got, ref_b, f"ggml (bf16 Q/K) D={D} hq={hq} hkv={hkv} B={B}")
        assert_close(got, ref, "ggml (unrounded reference)", max_abs=2e-2, mean_rel=5e-3)


def test_ggml_rejects_unsupported(emb, torch_dev):
    torch, dev = torch_dev
    buf = torch.zeros(4096, dtype=torch.float32, device=dev)
    q = emb.ggml_tensor(buf, emb.EMB_GGML_F32, [64, 4, 2, 1])
    k = emb.ggml_tensor(buf, emb.EMB_GGML_F16, [64, 8, 1, 1])
    o = emb.ggml_tensor(buf, emb.EMB_GGML_F32, [64, 2, 4, 1])
    L = emb.lib()
    import ctypes as C
    nb = L.emb_ggml_flash_attn_ext_workspace(C.byref(q), C.byref(k), C.byref(k), None, C.byref(o))
    assert nb > 0
    assert L.emb_ggml_flash_attn_ext(C.byref(q), C.byref(k), C.byref(k), None, 0.125, 1.0, 0.0, C.byref(o),
                                     emb.ptr(buf), nb, None) == -4  # ALiBi
    kbad = emb.ggml_tensor(buf, emb.EMB_GGML_F16, [64, 8, 3, 1])  # 2 q heads over 3 kv heads
    assert L.emb_ggml_flash_attn_ext_workspace(C.byref(q), C.byref(kbad), C.byref(kbad), None, C.byref(o)) == 0


@pytest.mark.parametrize("D,hq,hkv", [(128, 8, 2), (64, 4, 4), (96, 6, 3)])
def test_cosmos3_gqa_faces(emb, orc, torch_dev, D, hq, hkv):
    """cosmos3_qwen_causal_gqa_attention_f32 and cosmos3_qwen_gen_full_gqa_attention_f32
    (kernels/cosmos3/cosmos3_qwen_language_cuda.cu:246-298, :371-425): f32 tensors,
    GQA, causal or full, output rounded to bf16 values."""
    torch, dev = torch_dev
    rng = np.random.default_rng(D * 7 + hq)
    T, G = 300, 51
    bf = lambda shape: orc.f32_to_bf16(rng.standard_normal(shape).astype(np.float32))
    q, k, v = bf((T, hq, D)), bf((T, hkv, D)), bf((T, hkv, D))
    f = lambda a: torch.from_numpy(orc.bf16_to_f32(a).reshape(a.shape[0], -1).copy()).to(dev)
    L = emb.lib()
    qd, kd, vd = f(q), f(k), f(v)  # kept alive while the launches run
    y = torch.full((T, hq * D), float("nan"), dtype=torch.float32, device=dev)
    rc = L.cosmos3_qwen_causal_gqa_attention_f32(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), y.data_ptr(),
                                                 T, hq * D, hkv * D, hq, hkv, D, None)
    assert rc == 0, emb.last_error()
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.array_equal(got, orc.bf16_to_f32(orc.f32_to_bf16(got))), "output not rounded to bf16"
    # the reference rounds its output to bf16 values: so is the oracle's here
    rb = lambda a: orc.bf16_to_f32(orc.f32_to_bf16(a))
    ref = rb(orc.gqa_attention(q, k, v, T, T, hq, hkv, D, 1 / math.sqrt(D), chunk=1))
    assert_close(got.reshape(T, hq, D), ref, "causal")
    # generated tokens (the last G) over every key
    yg = torch.full((G, hq * D), float("nan"), dtype=torch.float32, device=dev)
    qg = q[T - G:]
    qgd = f(qg)
    rc = L.cosmos3_qwen_gen_full_gqa_attention_f32(qgd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                                   yg.data_ptr(), G, T, hq * D, hkv * D, hq, hkv, D, None)
    assert rc == 0, emb.last_error()
    torch.cuda.synchronize()
    ref = rb(orc.gqa_attention(qg, k, v, G, T, hq, hkv, D, 1 / math.sqrt(D)))
    assert_close(yg.cpu().numpy().reshape(G, hq, D), ref, "gen full")
    assert L.cosmos3_qwen_causal_gqa_attention_f32(None, None, None, None, T, hq * D, hkv * D, hq, hkv, D, None) == -1
    assert L.cosmos3_qwen_causal_gqa_attention_f32(y.data_ptr(), y.data_ptr(), y.data_ptr(), y.data_ptr(), T,
                                                   hq * D + 1, hkv * D, hq, hkv, D, None) == -1


@pytest.mark.parametrize("G,T,hq,hkv,D", [(51, 300, 8, 2, 128), (1, 64, 4, 1, 64)])
def test_cosmos3_gen_full_workspace_faces(emb, orc, torch_dev, G, T, hq, hkv, D):
    """cosmos3_qwen_gen_full_gqa_attention_workspace_f32 and _workspace_bf16tc_f32
    (kernels/cosmos3/cosmos3_qwen_language_cuda.h:105-134), the symbols the MoT
    denoise calls (models/cosmos3.cpp:7889, :8187), with caller workspaces of
    the model's sizes: bit-identical to the workspace-free face (same
    arithmetic), within the bar of the oracle rounded to bf16, and the
    workspaces' contents are scratch.  The second shape's workspaces are too
    small for the staging (one generated token): the call allocates instead."""
    torch, dev = torch_dev
    rng = np.random.default_rng(G * 3 + D)
    bf = lambda shape: orc.f32_to_bf16(rng.standard_normal(shape).astype(np.float32))
    q, k, v = bf((G, hq, D)), bf((T, hkv, D)), bf((T, hkv, D))
    f = lambda a: torch.from_numpy(orc.bf16_to_f32(a).reshape(a.shape[0], -1).copy()).to(dev)
    qd, kd, vd = f(q), f(k), f(v)
    L = emb.lib()
    args = (G, T, hq * D, hkv * D, hq, hkv, D)
    y0 = torch.full((G, hq * D), float("nan"), dtype=torch.float32, device=dev)
    assert L.cosmos3_qwen_gen_full_gqa_attention_f32(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), y0.data_ptr(),
                                                     *args, None) == 0, emb.last_error()
    scores = torch.full((G * T * (hq // hkv),), 7.0, dtype=torch.float32, device=dev)
    bfw = torch.zeros(G * hq * D + 2 * T * hkv * D, dtype=torch.int16, device=dev)
    y1 = torch.full_like(y0, float("nan"))
    assert L.cosmos3_qwen_gen_full_gqa_attention_workspace_f32(
        qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), y1.data_ptr(), scores.data_ptr(), *args, None) == 0, \
        emb.last_error()
    y2 = torch.full_like(y0, float("nan"))
    assert L.cosmos3_qwen_gen_full_gqa_attention_workspace_bf16tc_f32(
        qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), y2.data_ptr(), scores.data_ptr(), bfw.data_ptr(), *args,
        None) == 0, emb.last_error()
    torch.cuda.synchronize()
    a0, a1, a2 = (t.cpu().numpy() for t in (y0, y1, y2))
    assert np.array_equal(a0, a1) and np.array_equal(a0, a2)
    rb = lambda a: orc.bf16_to_f32(orc.f32_to_bf16(a))
    ref = rb(orc.gqa_attention(q, k, v, G, T, hq, hkv, D, 1 / math.sqrt(D)))
    assert_close(a1.reshape(G, hq, D), ref, "gen full workspace")
    # the reference's argument checks (:1152-1158, :1190-1196)
    assert L.cosmos3_qwen_gen_full_gqa_attention_workspace_f32(
        qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), y1.data_ptr(), None, *args, None) == -1
    assert L.cosmos3_qwen_gen_full_gqa_attention_workspace_bf16tc_f32(
        qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), y2.data_ptr(), scores.data_ptr(), None, *args, None) == -1
    bad = (G, T, hq * D + 1, hkv * D, hq, hkv, D)
    assert L.cosmos3_qwen_gen_full_gqa_attention_workspace_f32(
        qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), y1.data_ptr(), scores.data_ptr(), *bad, None) == -1


def test_faces_on_two_streams(emb, orc, torch_dev):
    """Two flex calls of different sizes in flight on two streams at once: each
    call stages into its own stream-ordered allocation, so neither result is
    disturbed by the other (both bit-identical to the same calls run alone)."""
    torch, dev = torch_dev
    rng = np.random.default_rng(5)
    cases = []
    for sq, sk in ((64, 400), (40, 90)):
        H, D, bs = 2, 64, 16
        q = _bf16_valued(orc, rng, (sq, H, D))
        k = _bf16_valued(orc, rng, (sk, H, D))
        v = _bf16_valued(orc, rng, (sk, H, D))
        rp, ci = _random_csr(rng, (sq + bs - 1) // bs, (sk + bs - 1) // bs, 0.8)
        cases.append([_dev(torch, dev, x) for x in (q, k, v, rp, ci)] + [sq, sk, H, D, bs])
    def run(c, out, stream):
        q, k, v, rp, ci, sq, sk, H, D, bs = c
        emb.flex_attention(q, k, v, rp, ci, out, sq, sk, H, D, bs, 0.125, stream=stream)
    alone = []
    for c in cases:
        o = torch.zeros((c[5], c[7], c[8]), dtype=torch.float32, device=dev)
        run(c, o, None)
        torch.cuda.synchronize()
        alone.append(o.cpu().numpy())
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = [torch.zeros((c[5], c[7], c[8]), dtype=torch.float32, device=dev) for c in cases]
    torch.cuda.synchronize()
    for _ in range(3):
        run(cases[0], outs[0], s1)
        run(cases[1], outs[1], s2)
    torch.cuda.synchronize()
    for a, o in zip(alone, outs):
        assert np.array_equal(a, o.cpu().numpy())
