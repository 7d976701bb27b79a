"""emb_paged_attention_noalloc (the entry point for callers that cannot
allocate): split-K partials in the library's per-device scratch instead of a
caller workspace.  Checked through the C ABI against emb_paged_attention with
a workspace -- the same kernels, so bit-identical -- on two calls in a row,
the second smaller (the scratch keeps the first call's contents), and against
the oracle; oversized requests and a passed workspace are refused before any
launch."""
from __future__ import annotations

import ctypes as C
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


def _both(emb, torch, dev, s, scale, splits):
    """(with a caller workspace, through the scratch) outputs of one launch."""
    q = _t(torch, dev, np.concatenate(s.q))
    kp, vp, bt = _t(torch, dev, s.kp), _t(torch, dev, s.vp), _t(torch, dev, s.bt)
    cu = _t(torch, dev, s.cu_q)
    nk = _t(torch, dev, np.array(s.n_keys, np.int32))
    outs = []
    for noalloc in (False, True):
        ws = None
        if splits > 1 and not noalloc:
            nb = emb.attn_workspace_bytes(len(s.n_q), max(s.n_q), s.hq, s.hkv, s.d, splits)
            ws = torch.empty(nb // 4 + 4, dtype=torch.float32, device=dev)
        out = torch.full((int(s.cu_q[-1]), s.hq, s.d), float("nan"), dtype=torch.float32, device=dev)
        emb.paged_attention(q=q, out=out, k_pool=kp, v_pool=vp, batch=len(s.n_q), hq=s.hq, hkv=s.hkv, d=s.d,
                            max_q=max(s.n_q), scale=scale, capacity=s.cap, cu_q=cu, n_keys=nk, block_tables=bt,
                            bt_stride=s.bt_stride, splits=splits, workspace=ws, noalloc=noalloc)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    return outs


def test_noalloc_matches_workspace_entry(emb, orc, torch_dev):
    torch, dev = torch_dev
    rng = np.random.default_rng(0xA110C)
    # call 1: six config-1 layers (51 x 8 heads over 867 keys, D 256), split-K 3
    big = Seqs(orc, rng, [867] * 6, [51] * 6, 8, 1, 256)
    ref_ws, got = _both(emb, torch, dev, big, 1 / 16, 3)
    assert np.array_equal(ref_ws, got), "noalloc differs from the workspace entry (call 1)"
    for b in (0, 5):
        assert_close(got[big.cu_q[b]:big.cu_q[b + 1]], big.oracle(orc, b, 1 / 16), f"call 1 seq {b}")
    # call 2, smaller: a ragged GQA batch at D 128, split-K 2, over the scratch
    # the first call left behind
    small = Seqs(orc, rng, [300, 77], [40, 13], 4, 2, 128)
    ref_ws, got = _both(emb, torch, dev, small, 1 / math.sqrt(128), 2)
    assert np.array_equal(ref_ws, got), "noalloc differs from the workspace entry (call 2)"
    for b in range(2):
        assert_close(got[small.cu_q[b]:small.cu_q[b + 1]], small.oracle(orc, b, 1 / math.sqrt(128)),
                     f"call 2 seq {b}")
    # no split: no scratch involved, same result
    ref_ws, got = _both(emb, torch, dev, small, 1 / math.sqrt(128), 1)
    assert np.array_equal(ref_ws, got)


def test_noalloc_refusals(emb, torch_dev):
    torch, dev = torch_dev
    L = emb.lib()
    buf = torch.zeros(1 << 16, dtype=torch.float32, device=dev)
    a = emb.AttnArgs()
    a.q = a.out = a.k_pool = a.v_pool = emb.ptr(buf)
    a.q_stride = a.out_stride = 8 * 256
    a.batch, a.hq, a.hkv, a.head_dim, a.max_q = 64, 8, 1, 256, 51
    a.n_keys_uniform, a.capacity, a.scale = 867, 880, 0.0625
    a.splits = 16  # 64 x 4 row tiles x 16 splits of partials: about 277 MB, over the 48 MiB scratch
    assert L.emb_paged_attention_noalloc(C.byref(a), None) == -3
    assert "scratch" in emb.last_error()
    a.splits = 3
    a.workspace = emb.ptr(buf)
    assert L.emb_paged_attention_noalloc(C.byref(a), None) == -1
    assert "workspace must be NULL" in emb.last_error()
    torch.cuda.synchronize()
    assert float(buf.abs().sum()) == 0.0  # nothing launched
