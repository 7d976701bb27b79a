"""GPU parity of emb_dense_gated_residual: LingBot's lin() on its dense resident
block weights (models/lingbot_va.cpp:1808-1851: F32, or BF16) with the gated
residual of the post graph (:11693-11695, lin() :1178-1180), against the
oracle's dense_linear (ggml's CUDA mul_mat numerics) and gated_residual.

Bars:
  * projection, BF16 weights: the result is bf16(fp32 accumulation), whose
    order cuBLAS leaves unspecified.  Each element is within one bf16 ulp plus
    the fp32 accumulation bound E = K * 2^-24 * sum_k |x_k w_k| of the oracle's
    bf16(exact sum), and at least 99% of them are identical to it;
  * projection, F32 weights: within E + 2^-24 |exact| of the exact sum;
  * epilogue: bit-identical to the oracle's epilogue applied to the same
    kernel's own projection (the call with no bias, gate or residual), for
    every combination of bias, strided gate, gate bias, residual, in-place
    residual and the bf16 boundary;
  * f32 x rounded while staged, through the bf16 workspace, or given as bf16:
    bit-identical results.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


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


def _problem(orc, rng, M, K, N, bf16w):
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    if bf16w:
        w = orc.f32_to_bf16(w)
    return x, w


def _check_projection(orc, got, x, w, bf16w, rows):
    want = orc.dense_linear(x, w, bf16w, rows=rows)
    xs = x[rows]
    xe = orc.bf16_to_f32(orc.f32_to_bf16(xs)) if bf16w else xs
    we = orc.bf16_to_f32(w) if bf16w else w
    mag = np.abs(xe.astype(np.float64)) @ np.abs(we.astype(np.float64)).T
    E = x.shape[1] * U * mag * 1.01 + 1e-30
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    if bf16w:
        big = np.maximum(np.abs(got), np.abs(want)).astype(np.float64)
        ulp = np.exp2(np.floor(np.log2(np.maximum(big, 1e-30))) - 7)
        assert np.all(diff <= E + ulp), f"max excess {np.max(diff - E - ulp)}"
        same = np.mean(got == want)
        assert same >= 0.99, f"only {same:.4f} identical"
    else:
        assert np.all(diff <= E + U * np.abs(want)), f"max excess {np.max(diff - E - U * np.abs(want))}"


def _lin(emb, torch, dev, xt, wt, wtype, M, K, N, x_is_f32=True, ldx=None, ws=None):
    out = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    emb.dense_gated_residual(xt, wt, wtype, M, K, N, out, x_is_f32=x_is_f32, ldx=ldx, x_bf16_workspace=ws)
    return out


@pytest.mark.parametrize("bf16w,xform", [(True, "f32"), (True, "bf16"), (False, "f32")],
                         ids=["bf16-staged", "bf16-copied", "f32"])
@pytest.mark.parametrize("M,K,N,sample", [
    (300, 512, 384, None),
    (129, 384, 200, None),       # N not a multiple of the tile width
    (37, 1024, 64, None),
    (1560, 3072, 3072, 96),      # LingBot O-projection shape, sampled rows
])
def test_dense_projection(emb, orc, torch_dev, bf16w, xform, M, K, N, sample):
    """xform "f32": x rounded while staged (the single-stage kernel); "bf16":
    x given as bf16 rows, both operands copied straight into LDS."""
    torch, dev = torch_dev
    rng = np.random.default_rng(M * 7 + K + N + bf16w)
    x, w = _problem(orc, rng, M, K, N, bf16w)
    wtype = emb.EMB_GGML_BF16 if bf16w else emb.EMB_GGML_F32
    if xform == "bf16":
        x = orc.bf16_to_f32(orc.f32_to_bf16(x))  # the oracle rounds it the same way
        out = _lin(emb, torch, dev, _t(torch, dev, orc.f32_to_bf16(x)), _t(torch, dev, w), wtype, M, K, N,
                   x_is_f32=False)
    else:
        out = _lin(emb, torch, dev, _t(torch, dev, x), _t(torch, dev, w), wtype, M, K, N)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    rows = np.arange(M) if sample is None else np.sort(rng.choice(M, sample, replace=False))
    _check_projection(orc, got[rows], x, w, bf16w, rows)
    assert np.isfinite(got).all()


def test_dense_projection_bf16_wide(emb, orc, torch_dev):
    """1560 x 3072 -> 9216 (the QKV / FFN width), where the 256-row tile runs."""
    torch, dev = torch_dev
    rng = np.random.default_rng(9216)
    M, K, N = 1560, 3072, 9216
    x, w = _problem(orc, rng, M, K, N, True)
    xb = orc.f32_to_bf16(x)
    staged = _lin(emb, torch, dev, _t(torch, dev, x), _t(torch, dev, w), emb.EMB_GGML_BF16, M, K, N)
    copied = _lin(emb, torch, dev, _t(torch, dev, xb), _t(torch, dev, w), emb.EMB_GGML_BF16, M, K, N,
                  x_is_f32=False)
    torch.cuda.synchronize()
    rows = np.sort(rng.choice(M, 32, replace=False))
    rows[-1] = M - 1  # the last, partial row tile
    _check_projection(orc, staged.cpu().numpy()[rows], x, w, True, rows)
    # the 256 x 256 copied-operand kernel sums the same k-steps in the same order
    assert torch.equal(staged, copied), "staged and copied kernels differ"


@pytest.mark.parametrize("bf16w", [True, False], ids=["bf16", "f32"])
@pytest.mark.parametrize("gated,bias,res,rnd", [
    (True, True, True, False),
    (True, False, True, True),    # bf16 boundary
    (False, True, True, False),   # plain residual add
    (True, True, False, False),   # lin * gate, no residual
    (False, True, False, False),  # the plain lin()
])
def test_dense_epilogue_exact(emb, orc, torch_dev, bf16w, gated, bias, res, rnd):
    torch, dev = torch_dev
    M, K, N = 261, 256, 320
    rng = np.random.default_rng(M + 3 * gated + 5 * bias + 7 * res + 11 * rnd + bf16w)
    x, w = _problem(orc, rng, M, K, N, bf16w)
    wtype = emb.EMB_GGML_BF16 if bf16w else emb.EMB_GGML_F32
    tproj = rng.standard_normal((M, 6 * N)).astype(np.float32)  # gate at column 2N of a [M][6N] projection
    ss = rng.standard_normal(6 * N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    r = (rng.standard_normal((M, N)) * 4).astype(np.float32) if res else None
    xt, wt = _t(torch, dev, x), _t(torch, dev, w)
    lin = _lin(emb, torch, dev, xt, wt, wtype, M, K, N)
    tp, sst = _t(torch, dev, tproj), _t(torch, dev, ss)
    out = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    emb.dense_gated_residual(xt, wt, wtype, M, K, N, out, residual=None if r is None else _t(torch, dev, r),
                             bias=None if b is None else _t(torch, dev, b),
                             gate=tp[:, 2 * N:] if gated else None, ldg=6 * N,
                             gate_bias=sst[2 * N:3 * N] if gated else None, round_bf16=rnd)
    torch.cuda.synchronize()
    want = orc.gated_residual(lin.cpu().numpy(), r, bias=b, gate=tproj[:, 2 * N:3 * N] if gated else None,
                              gate_bias=ss[2 * N:3 * N] if gated else None, round_bf16=rnd)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"epilogue differs at {np.argwhere(got != want)[:5].tolist()}"


def test_dense_exact_integers_in_place(emb, orc, torch_dev):
    """Small dyadic values everywhere, out = the residual tensor: every
    intermediate is exact, so both weight types equal the oracle bit for bit."""
    torch, dev = torch_dev
    rng = np.random.default_rng(44)
    M, K, N = 200, 256, 256
    x = rng.integers(-4, 5, (M, K)).astype(np.float32)
    wf = (rng.integers(-3, 4, (N, K)) / 8).astype(np.float32)
    gate = (rng.integers(-8, 9, (M, N)) / 8).astype(np.float32)
    gb = (rng.integers(-8, 9, N) / 8).astype(np.float32)
    b = (rng.integers(-8, 9, N) / 4).astype(np.float32)
    res = rng.integers(-100, 100, (M, N)).astype(np.float32)
    for bf16w in (True, False):
        w = orc.f32_to_bf16(wf) if bf16w else wf
        rt = _t(torch, dev, res)
        emb.dense_gated_residual(_t(torch, dev, x), _t(torch, dev, w),
                                 emb.EMB_GGML_BF16 if bf16w else emb.EMB_GGML_F32, M, K, N, rt, residual=rt,
                                 bias=_t(torch, dev, b), gate=_t(torch, dev, gate), gate_bias=_t(torch, dev, gb))
        torch.cuda.synchronize()
        lin = orc.dense_linear(x, w, bf16w, bias=b)
        assert np.array_equal(rt.cpu().numpy(), orc.gated_residual(lin, res, gate=gate, gate_bias=gb))


def test_dense_bf16_x_forms_agree(emb, orc, torch_dev):
    """f32 x rounded while staged, rounded into the workspace first, or given
    as bf16 rows: the same bf16 values, so bit-identical results."""
    torch, dev = torch_dev
    rng = np.random.default_rng(55)
    M, K, N = 301, 320, 192
    ldx = K + 12
    xf = rng.standard_normal((M, ldx)).astype(np.float32)
    xb = orc.f32_to_bf16(np.ascontiguousarray(xf[:, :K]))
    w = orc.f32_to_bf16((rng.standard_normal((N, K)) / 16).astype(np.float32))
    wt, xft = _t(torch, dev, w), _t(torch, dev, xf)
    outs = []
    for how in ("staged", "workspace", "bf16"):
        if how == "bf16":
            out = _lin(emb, torch, dev, _t(torch, dev, xb), wt, emb.EMB_GGML_BF16, M, K, N, x_is_f32=False)
        else:
            ws = torch.full((M * K,), -1, dtype=torch.int16, device=dev) if how == "workspace" else None
            out = _lin(emb, torch, dev, xft, wt, emb.EMB_GGML_BF16, M, K, N, ldx=ldx, ws=ws)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    _check_projection(orc, outs[0], np.ascontiguousarray(xf[:, :K]), w, True, np.arange(M))


def test_dense_weight_row_stride(emb, orc, torch_dev):
    """Weights as a view with padded rows (ldw > K), both types."""
    torch, dev = torch_dev
    rng = np.random.default_rng(66)
    M, K, N, ldw = 96, 256, 128, 264
    x = rng.standard_normal((M, K)).astype(np.float32)
    wpad = (rng.standard_normal((N, ldw)) / 16).astype(np.float32)
    for bf16w in (True, False):
        w = orc.f32_to_bf16(wpad) if bf16w else wpad
        out = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        emb.dense_gated_residual(_t(torch, dev, x), _t(torch, dev, w),
                                 emb.EMB_GGML_BF16 if bf16w else emb.EMB_GGML_F32, M, K, N, out, ldw=ldw)
        torch.cuda.synchronize()
        _check_projection(orc, out.cpu().numpy(), x, np.ascontiguousarray(w[:, :K]), bf16w, np.arange(M))
