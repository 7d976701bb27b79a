"""GPU parity of emb_w8a16_gated_residual (the projection after attention with
the LingBot gated residual in its epilogue, models/lingbot_va.cpp:11693-11695)
against the oracle.

Bars:
  * epilogue: bit-identical to the oracle's epilogue applied to the same
    kernel's own fp32 projection value (EMB_W8_Y_F32_RAW), so the order of the
    f32 operations, the column/row indexing of bias, gate and residual, the
    strides and the bf16 boundary round are exact;
  * end to end: within the north-star tolerance (max-abs 2e-2, mean-rel 1e-3)
    of the oracle's W8 projection plus the same epilogue, and bit-exact where
    every value is a small dyadic number (exact in any summation order).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_close

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


def _weights(orc, rng, K, N):
    w = rng.integers(-127, 128, (K, N), dtype=np.int8)
    s = orc.f32_to_bf16(rng.uniform(0.001, 0.01, N).astype(np.float32))
    return orc.marlin_pack_w8(w), orc.marlin_pack_scales(s)


@pytest.mark.parametrize("M,K,N,gated,bias,rnd", [
    (300, 512, 384, True, True, False),
    (37, 256, 128, False, True, False),   # plain residual add
    (129, 384, 256, True, False, True),   # bf16 boundary
])
def test_gated_residual_epilogue_exact(emb, orc, torch_dev, M, K, N, gated, bias, rnd):
    torch, dev = torch_dev
    rng = np.random.default_rng(M + K + N)
    q, s_st = _weights(orc, rng, K, N)
    x = orc.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    # gate read from a [M][6N] timestep projection at column 2N (the LingBot layout)
    tproj = rng.standard_normal((M, 6 * N)).astype(np.float32)
    ss = rng.standard_normal(6 * N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    res = (rng.standard_normal((M, N)) * 4).astype(np.float32)
    xt, qt, st = _t(torch, dev, x), _t(torch, dev, q), _t(torch, dev, s_st)
    raw = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    emb.w8a16_gemm(xt, qt, st, M, K, N, raw, y_kind=emb.EMB_W8_Y_F32_RAW)
    tp = _t(torch, dev, tproj)
    sst = _t(torch, dev, ss)
    out = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    emb.w8a16_gated_residual(xt, qt, st, M, K, N, _t(torch, dev, res), out,
                             bias=None if b is None else _t(torch, dev, b),
                             gate=tp[:, 2 * N:] if gated else None, ldg=6 * N,
                             gate_bias=sst[2 * N:3 * N] if gated else None, round_bf16=rnd)
    torch.cuda.synchronize()
    want = orc.gated_residual(raw.cpu().numpy(), res, bias=b, gate=tproj[:, 2 * N:3 * N] if gated else None,
                              gate_bias=ss[2 * N:3 * N] if gated else None, round_bf16=rnd)
    got = out.cpu().numpy()
    assert np.array_equal(got, want), f"epilogue differs at {np.argwhere(got != want)[:5].tolist()}"
    # end to end against the oracle's own projection
    _, yf_ref = orc.w8a16_gemm(x, q, s_st, M, K, N)
    ref = orc.gated_residual(yf_ref, res, bias=b, gate=tproj[:, 2 * N:3 * N] if gated else None,
                             gate_bias=ss[2 * N:3 * N] if gated else None, round_bf16=rnd)
    if rnd:  # one bf16 ulp where accumulation order moves a value across a rounding boundary
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
        assert np.all(np.abs(got - ref) <= ulp + 1e-5 * np.abs(ref).max())
    else:
        assert_close(got, ref, "gated residual vs oracle")


def test_gated_residual_exact_integers_in_place(emb, orc, torch_dev):
    """Small dyadic values everywhere: every intermediate is exact, so the
    result is bit-identical to the oracle; out is the residual tensor itself."""
    torch, dev = torch_dev
    rng = np.random.default_rng(21)
    M, K, N = 200, 256, 256
    w = rng.integers(-3, 4, (K, N), dtype=np.int8)
    s = orc.f32_to_bf16(np.full(N, 0.125, np.float32))
    q, s_st = orc.marlin_pack_w8(w), orc.marlin_pack_scales(s)
    x = orc.f32_to_bf16(rng.integers(-4, 5, (M, K)).astype(np.float32))
    gate = (rng.integers(-8, 9, (M, N)) / 8).astype(np.float32)
    gb = (rng.integers(-8, 9, N) / 8).astype(np.float32)
    b = (rng.integers(-8, 9, N) / 4).astype(np.float32)
    res = rng.integers(-100, 100, (M, N)).astype(np.float32)
    rt = _t(torch, dev, res)
    emb.w8a16_gated_residual(_t(torch, dev, x), _t(torch, dev, q), _t(torch, dev, s_st), M, K, N, rt, rt,
                             bias=_t(torch, dev, b), gate=_t(torch, dev, gate), gate_bias=_t(torch, dev, gb))
    torch.cuda.synchronize()
    _, yf = orc.w8a16_gemm(x, q, s_st, M, K, N)
    assert np.array_equal(rt.cpu().numpy(), orc.gated_residual(yf, res, bias=b, gate=gate, gate_bias=gb))


def test_gated_residual_f32_x_with_and_without_workspace(emb, orc, torch_dev):
    """f32 activations (the attention output): rounded while staged, rounded
    first into a bf16 workspace, or handed over already rounded -- the same
    bf16 values, so the three results are bit-identical."""
    torch, dev = torch_dev
    rng = np.random.default_rng(33)
    M, K, N = 301, 320, 192
    q, s_st = _weights(orc, rng, K, N)
    ldx = K + 12  # padded rows
    xf = rng.standard_normal((M, ldx)).astype(np.float32)
    xb = orc.f32_to_bf16(np.ascontiguousarray(xf[:, :K]))
    gate = rng.standard_normal((M, N)).astype(np.float32)
    res = rng.standard_normal((M, N)).astype(np.float32)
    qt, st, gt, rt = (_t(torch, dev, a) for a in (q, s_st, gate, res))
    xft = _t(torch, dev, xf)
    outs = []
    for how in ("staged", "workspace", "bf16"):
        out = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        if how == "bf16":
            emb.w8a16_gated_residual(_t(torch, dev, xb), qt, st, M, K, N, rt, out, gate=gt)
        else:
            ws = torch.full((M * K,), -1, dtype=torch.int16, device=dev) if how == "workspace" else None
            emb.w8a16_gated_residual(xft, qt, st, M, K, N, rt, out, gate=gt, x_is_f32=True, ldx=ldx,
                                     x_bf16_workspace=ws)
            if ws is not None:
                torch.cuda.synchronize()
                assert np.array_equal(ws.cpu().numpy().view(np.uint16), xb.reshape(-1)), "workspace bf16 rows"
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
