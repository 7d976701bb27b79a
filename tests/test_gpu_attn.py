"""GPU parity of the paged block-masked attention against the oracle.

Bar: max |gpu - oracle| <= 2e-2 and sum|gpu - oracle| / sum|oracle| <= 1e-3 on
identical seeded bf16 inputs.  The pool is built
on the host by the oracle's paged append, so these tests isolate the
attention kernel from the append kernel.
"""
from __future__ import annotations

import math

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
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to(dev)


def _bf16(orc, rng, shape):
    return orc.f32_to_bf16(rng.standard_normal(shape).astype(np.float32))


class Seqs:
    """A batch of sequences whose keys live in one shared, randomly permuted page pool."""

    def __init__(self, orc, rng, n_keys, n_q, hq, hkv, d, extra_pages=5, v_scale=1.0):
        self.n_keys, self.n_q = list(n_keys), list(n_q)
        self.hq, self.hkv, self.d = hq, hkv, d
        pages = [(k + 15) // 16 for k in n_keys]
        self.bt_stride = max(pages)
        total = sum(pages) + extra_pages
        perm = rng.permutation(total).astype(np.int32)
        self.bt = np.full((len(n_keys), self.bt_stride), -1, np.int32)
        o = 0
        for b, p in enumerate(pages):
            self.bt[b, :p] = perm[o:o + p]
            o += p
        self.k = [_bf16(orc, rng, (k, hkv, d)) for k in n_keys]
        # v_scale: a number, or a function of the key count giving per-key scales [k][1][1]
        vsc = v_scale if callable(v_scale) else (lambda k: v_scale)
        self.v = [orc.f32_to_bf16((rng.standard_normal((k, hkv, d)) * vsc(k)).astype(np.float32)) for k in n_keys]
        self.q = [_bf16(orc, rng, (q, hq, d)) for q in n_q]
        self.kp = rng.integers(0, 65536, total * hkv * 16 * d, dtype=np.uint16)  # garbage elsewhere
        self.vp = rng.integers(0, 65536, total * hkv * 16 * d, dtype=np.uint16)
        # keep garbage finite-free of NaN/Inf so a stray read would show as error, not NaN
        for a in (self.kp, self.vp):
            a &= np.uint16(0xBFFF)
        self.cap = self.bt_stride * 16
        for b, k in enumerate(n_keys):
            orc.paged_append(self.k[b], self.v[b], hkv * d, np.arange(k, dtype=np.int32), self.bt[b],
                             hkv, d, self.cap, self.kp, self.vp)
        self.cu_q = np.concatenate([[0], np.cumsum(n_q)]).astype(np.int32)

    def run(self, emb, torch, dev, scale, splits=1, uniform=False, **kw):
        """Runs the row-tile kernel twice -- tiles staged through registers from the
        bf16 V pool, and copied into LDS from the f16 V shadow -- and requires the
        two to agree bit for bit (same arithmetic, same conversions).  Where the
        key-split kernel applies (FULL mask, no split-K, D 128/256) it runs too:
        its output is kept in ks_out (the callers check it against the oracle
        with ks_check) and must agree with the row-tile output within the bar.
        uniform: the batch goes in the form without bounds arrays (equal
        sequences only)."""
        if uniform:
            assert len(set(self.n_keys)) == 1 and len(set(self.n_q)) == 1
        ws = None
        if splits > 1:
            nb = emb.attn_workspace_bytes(len(self.n_q), max(self.n_q), self.hq, self.hkv, self.d, splits)
            ws = torch.empty(nb // 4 + 4, dtype=torch.float32, device=dev)
        keep = dict(q=_t(torch, dev, np.concatenate(self.q)), kp=_t(torch, dev, self.kp),
                    vp=_t(torch, dev, self.vp), v16=_t(torch, dev, v16_shadow(self.vp, self.d)),
                    bt=_t(torch, dev, self.bt), cu=_t(torch, dev, self.cu_q),
                    nk=_t(torch, dev, np.array(self.n_keys, np.int32)))
        def launch(v16, kernel):
            out = torch.full((int(self.cu_q[-1]), self.hq, self.d), float("nan"), dtype=torch.float32, device=dev)
            emb.paged_attention(q=keep["q"], out=out, k_pool=keep["kp"], v_pool=keep["vp"], v16_pool=v16,
                                batch=len(self.n_q), hq=self.hq, hkv=self.hkv, d=self.d, max_q=max(self.n_q),
                                scale=scale, capacity=self.cap, cu_q=None if uniform else keep["cu"],
                                n_keys=None if uniform else keep["nk"],
                                n_keys_uniform=self.n_keys[0] if uniform else 0,
                                block_tables=keep["bt"], bt_stride=self.bt_stride, splits=splits, workspace=ws,
                                kernel=kernel, **kw)
            torch.cuda.synchronize()
            return out.cpu().numpy()

        outs = [launch(None, emb.EMB_ATTN_ROW_TILES), launch(keep["v16"], emb.EMB_ATTN_ROW_TILES)]
        assert np.array_equal(outs[0], outs[1], equal_nan=True), "register and LDS-copy paths differ"
        per_seq = lambda o: [o[self.cu_q[b]:self.cu_q[b + 1]] for b in range(len(self.n_q))]
        self.reg_out = per_seq(outs[0])
        self.ks_out = None
        if (splits <= 1 and kw.get("mask_kind", emb.EMB_MASK_FULL) == emb.EMB_MASK_FULL and self.d in (128, 256)
                and not kw.get("p_bf16") and kw.get("valid_slots") is None):
            ks = launch(keep["v16"], emb.EMB_ATTN_KEY_SPLIT)
            for b in range(len(self.n_q)):
                sl = slice(self.cu_q[b], self.cu_q[b + 1])
                mag = max(float(np.abs(outs[1][sl]).max(initial=0.0)), 1e-30)  # the bar relative to the data's scale
                assert_close(ks[sl] / mag, outs[1][sl] / mag, f"key-split vs row tiles, seq {b}")
            self.ks_out = per_seq(ks)
        return per_seq(outs[1])

    def ks_check(self, orc, scale, what, rows=None, **kw):
        """The key-split output of the last run against the oracle (all rows, or
        the given rows of every sequence); the last run must have run it."""
        assert self.ks_out is not None, f"{what}: the key-split kernel did not run"
        for b in range(len(self.n_q)):
            ref = self.oracle(orc, b, scale, rows=rows, **kw)
            got = self.ks_out[b]
            if rows is not None:
                got, ref = got[rows], ref[rows]
            assert_close(got, ref, f"{what} key-split seq {b}")

    def oracle(self, orc, b, scale, rows=None, **kw):
        return orc.gqa_attention(self.q[b], self.k[b], self.v[b], self.n_q[b], self.n_keys[b], self.hq, self.hkv,
                                 self.d, scale, rows=rows, **kw)


def test_pi05_action_expert_shape(emb, orc, torch_dev):
    """cfg1: prefix 816 + 51 new keys, 51 queries x 8 heads over 1 kv head, D=256, all visible."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0xE3BD0000)
    s = Seqs(orc, rng, [867], [51], 8, 1, 256)
    scale = 1 / 16
    got = s.run(emb, torch, dev, scale)[0]
    assert_close(got, s.oracle(orc, 0, scale), "pi05 cfg1")
    s.ks_check(orc, scale, "pi05 cfg1")
    got4 = s.run(emb, torch, dev, scale, splits=4)[0]
    assert_close(got4, s.oracle(orc, 0, scale), "pi05 cfg1 split-K 4")
    got6 = s.run(emb, torch, dev, scale, splits=6)[0]
    assert_close(got6, s.oracle(orc, 0, scale), "pi05 cfg1 split-K 6")


def test_pi05_register_path_against_oracle(emb, orc, torch_dev):
    """cfg1 shape with a second, shorter sequence: the register-staged path (no
    V shadow) and the shadow path, each against the oracle, with and without
    split-K (5 splits leave the last split of the short sequence empty)."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0xE3BD0010)
    s = Seqs(orc, rng, [867, 300], [51, 40], 8, 1, 256)
    scale = 1 / 16
    for splits in (1, 3, 5):
        got = s.run(emb, torch, dev, scale, splits=splits)
        for b in range(2):
            ref = s.oracle(orc, b, scale)
            assert_close(got[b], ref, f"shadow path b={b} splits={splits}")
            assert_close(s.reg_out[b], ref, f"register path b={b} splits={splits}")
        if splits == 1:
            s.ks_check(orc, scale, "pi05 two sequences")


def test_uniform_batch_form(emb, orc, torch_dev):
    """cfg1 layers batched in one launch without bounds arrays (every sequence 51 queries
    over 867 keys): bit-identical to the launch with cu_q / n_keys, and within the bar."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0xE3BD0010)
    s = Seqs(orc, rng, [867] * 3, [51] * 3, 8, 1, 256)
    for splits in (1, 3):
        arr = s.run(emb, torch, dev, 1 / 16, splits=splits)
        uni = s.run(emb, torch, dev, 1 / 16, splits=splits, uniform=True)
        for b in range(3):
            assert np.array_equal(arr[b], uni[b]), f"uniform form differs, splits {splits} seq {b}"
            assert_close(uni[b], s.oracle(orc, b, 1 / 16), f"uniform seq {b} splits {splits}")
        if splits == 1:
            s.ks_check(orc, 1 / 16, "uniform form")


@pytest.mark.parametrize("d,hq,hkv", [(256, 8, 1), (128, 4, 2), (64, 2, 2)])
def test_out_bf16_round(emb, orc, torch_dev, d, hq, hkv):
    """out_bf16_round stores every output value rounded to bf16 (nearest even):
    exactly the rounding of the unrounded output, through both output paths
    (staged through LDS at D = 256, direct below) and through the split-K merge."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0xE3BD0011 + d)
    s = Seqs(orc, rng, [300, 77], [40, 13], hq, hkv, d)
    for splits in (1, 3):
        plain = s.run(emb, torch, dev, 1 / math.sqrt(d), splits=splits)
        rnd = s.run(emb, torch, dev, 1 / math.sqrt(d), splits=splits, out_bf16_round=True)
        for b in range(2):
            want = orc.bf16_to_f32(orc.f32_to_bf16(np.ascontiguousarray(plain[b])))
            assert np.array_equal(rnd[b], want), f"d {d} splits {splits} seq {b}"


@pytest.mark.parametrize("d,hq,hkv,mask", [(256, 8, 1, "full"), (128, 8, 2, "chunk"), (64, 4, 4, "full")])
def test_null_block_tables_are_identity(emb, orc, torch_dev, d, hq, hkv, mask):
    """NULL block tables map slot s to page s / 16 (the faces pass them for
    K/V shared by every sequence): bit-identical to explicit identity tables,
    for two sequences over the same pages, split-K 1 and 3, and within the bar
    of the oracle."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0xE3BD0012 + d)
    nk, nq, B = 300, 40, 2
    pages = (nk + 15) // 16
    k = orc.f32_to_bf16(rng.standard_normal((nk, hkv, d)).astype(np.float32))
    v = orc.f32_to_bf16(rng.standard_normal((nk, hkv, d)).astype(np.float32))
    q = orc.f32_to_bf16(rng.standard_normal((B * nq, hq, d)).astype(np.float32))
    kp = np.zeros(pages * hkv * 16 * d, np.uint16)
    vp = np.zeros_like(kp)
    orc.paged_append(k.reshape(nk, -1), v.reshape(nk, -1), hkv * d, np.arange(nk, dtype=np.int32),
                     np.arange(pages, dtype=np.int32), hkv, d, pages * 16, kp, vp)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16) if a.dtype == np.uint16 else a).to(dev)
    kpt, vpt, v16 = t(kp), t(vp), t(v16_shadow(vp, d))
    kw = dict(chunk=16, window=-1, mask_kind=emb.EMB_MASK_CHUNK) if mask == "chunk" else {}
    outs = {}
    for splits in (1, 3):
        ws = None
        if splits > 1:
            ws = torch.empty(emb.attn_workspace_bytes(B, nq, hq, hkv, d, splits) // 4 + 4, dtype=torch.float32,
                             device=dev)
        for how in ("tables", "null"):
            out = torch.full((B * nq, hq, d), float("nan"), dtype=torch.float32, device=dev)
            bt = t(np.tile(np.arange(pages, dtype=np.int32), B)) if how == "tables" else None
            emb.paged_attention(q=t(q), out=out, k_pool=kpt, v_pool=vpt, v16_pool=v16, batch=B, hq=hq, hkv=hkv, d=d,
                                max_q=nq, scale=1 / math.sqrt(d), capacity=pages * 16, n_keys_uniform=nk,
                                block_tables=bt, bt_stride=pages if bt is not None else 0, splits=splits,
                                workspace=ws, **kw)
            torch.cuda.synchronize()
            outs[(splits, how)] = out.cpu().numpy()
        assert np.array_equal(outs[(splits, "tables")], outs[(splits, "null")]), f"splits {splits}"
    okw = dict(chunk=16, window=-1) if mask == "chunk" else {}
    for b in range(B):
        ref = orc.gqa_attention(q[b * nq:(b + 1) * nq], k, v, nq, nk, hq, hkv, d, 1 / math.sqrt(d), **okw)
        assert_close(outs[(1, "null")][b * nq:(b + 1) * nq], ref, f"null tables seq {b}")


@pytest.mark.parametrize("B,splits,split_keys", [(1, 8, 0), (8, 8, 0), (32, 2, 0), (64, 1, 0), (64, 2, 0),
                                                   (8, 8, 128), (32, 4, 384), (64, 4, 320), (64, 3, 512),
                                                   (32, 2, 640), (64, 2, 768)])
def test_multi_session_sweep(emb, orc, torch_dev, B, splits, split_keys):
    """cfg4 at every batch the bench times, with its prefix lengths and split
    choices: session b's prefix is 300 + x_b % 901, x_b the b-th output of
    std::mt19937_64(0xE3BD0004); 51 queries x 8 heads over prefix + 51 keys,
    pages scattered in one pool.  All rows of every session at B <= 8; 24
    sampled rows of every session at B = 32 and 64.  split_keys > 0: each
    session takes min(splits, ceil(keys / split_keys)) splits, so sessions of
    one batch are cut differently and the merge reads a count per session;
    a session with one split is written by its own workgroups (no partials)
    and skipped by the merge (split_keys 640 / 768 leave about half the
    sessions unsplit)."""
    torch, dev = torch_dev
    lens = [300 + orc.lib().orc_mt64_nth(0xE3BD0004, b + 1) % 901 for b in range(B)]
    assert 300 <= min(lens) and max(lens) <= 1200
    rng = np.random.default_rng(0xE3BD0004 + B)
    s = Seqs(orc, rng, [int(x) + 51 for x in lens], [51] * B, 8, 1, 256)
    got = s.run(emb, torch, dev, 1 / 16, splits=splits, split_keys=split_keys)
    for b in range(B):
        rows = None if B <= 8 else np.sort(rng.choice(51, 3, replace=False))
        ref = s.oracle(orc, b, 1 / 16, rows=rows)
        if rows is None:
            assert_close(got[b], ref, f"B={B} session {b}")
        else:
            assert_close(got[b][rows], ref[rows], f"B={B} session {b} rows {rows.tolist()}")
        if s.ks_out is not None:
            ks = s.ks_out[b] if rows is None else s.ks_out[b][rows]
            assert_close(ks, ref if rows is None else ref[rows], f"B={B} session {b} key-split")


def test_split_keys_uniform_batch(emb, orc, torch_dev):
    """split_keys on the bounds-free form (every sequence n_keys_uniform keys):
    867 keys with splits 8 and split_keys 300 run 3 splits; the result equals
    the same call with splits 3 bit for bit, and the oracle within the bar."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0xE3BD0000 + 7)
    s = Seqs(orc, rng, [867, 867], [51, 51], 8, 1, 256)
    a = s.run(emb, torch, dev, 1 / 16, splits=8, uniform=True, split_keys=300)
    b = s.run(emb, torch, dev, 1 / 16, splits=3, uniform=True)
    for i in range(2):
        assert np.array_equal(a[i], b[i]), f"sequence {i}: split_keys 300 of 8 differs from 3 splits"
        assert_close(a[i], s.oracle(orc, i, 1 / 16), f"sequence {i}")


def test_prefill_prefix_lm_rows(emb, orc, torch_dev):
    """cfg2: 816-token bidirectional prefix prefill, 8 q heads / 1 kv head, D=256 (row sample)."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0xE3BD0001)
    s = Seqs(orc, rng, [816], [816], 8, 1, 256)
    got = s.run(emb, torch, dev, 1 / 16)[0]
    rows = np.concatenate([np.arange(0, 20), np.arange(400, 420), np.arange(796, 816)])
    ref = s.oracle(orc, 0, 1 / 16, rows=rows)
    assert_close(got[rows], ref[rows], "prefill rows")
    assert_close(s.ks_out[0][rows], ref[rows], "prefill rows key-split")


def test_lingbot_chunk_step_rows(emb, orc, torch_dev):
    """cfg3: 1560 queries x 24 heads (MHA) over 8 prior chunks + the current one (14040 keys), D=128."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0xE3BD0002)
    s = Seqs(orc, rng, [14040], [1560], 24, 24, 128)
    got = s.run(emb, torch, dev, 1 / math.sqrt(128))[0]
    rows = np.array([0, 1, 31, 32, 777, 1023, 1500, 1559])
    ref = s.oracle(orc, 0, 1 / math.sqrt(128), rows=rows)
    assert_close(got[rows], ref[rows], "lingbot rows")
    assert_close(s.ks_out[0][rows], ref[rows], "lingbot rows key-split (878 pages: table entries past 128)")


@pytest.mark.parametrize("window", [-1, 1])
def test_chunk_causal_prefill(emb, orc, torch_dev, window):
    """Multi-chunk prefill under the chunk-causal mask (bidirectional inside a chunk)."""
    torch, dev = torch_dev
    rng = np.random.default_rng(5 + window)
    s = Seqs(orc, rng, [390], [390], 4, 4, 128)
    got = s.run(emb, torch, dev, 0.09, mask_kind=emb.EMB_MASK_CHUNK, chunk=130, window=window)[0]
    ref = s.oracle(orc, 0, 0.09, chunk=130, window=window)
    assert_close(got, ref, f"chunk-causal window={window}")


def test_token_mask_hy_vla_suffix(emb, orc, torch_dev):
    """HY-VLA expert mask (models/hy_vla.cpp:2831-2843): every row sees the prefix;
    suffix row 0 (state) sees only itself among the suffix."""
    torch, dev = torch_dev
    rng = np.random.default_rng(9)
    n_pref, n_suf = 100, 51
    s = Seqs(orc, rng, [n_pref + n_suf], [n_suf], 8, 2, 128)
    allow = np.ones((n_suf, n_pref + n_suf), np.uint8)
    allow[0, n_pref + 1:] = 0
    m = _t(*torch_dev, allow)
    got = s.run(emb, torch, dev, 0.088, mask_kind=emb.EMB_MASK_TOKEN, mask=m,
                mask_q_stride=n_pref + n_suf)[0]
    assert_close(got, s.oracle(orc, 0, 0.088, allow=allow), "hy_vla token mask")


def test_additive_mask(emb, orc, torch_dev):
    """ggml soft_max_ext / flash_attn_ext additive mask, with -inf entries and an empty row."""
    torch, dev = torch_dev
    rng = np.random.default_rng(10)
    nq, nk = 37, 200
    s = Seqs(orc, rng, [nk], [nq], 8, 1, 64)
    add = rng.standard_normal((nq, nk)).astype(np.float32)
    add[rng.random((nq, nk)) < 0.3] = -np.inf
    add[5] = -np.inf
    got = s.run(emb, torch, dev, 0.125, mask_kind=emb.EMB_MASK_ADD, mask=_t(torch, dev, add),
                mask_q_stride=nk)[0]
    ref = s.oracle(orc, 0, 0.125, add=add)
    assert np.all(got[5] == 0)
    assert_close(got, ref, "additive mask")


def test_flex_block_map_and_token_mask(emb, orc, torch_dev):
    """Flex attention (lingbot_flex_attn_cuda.cu:502-582): CSR block table as a block map plus the
    LingBot chunk-causal token mask from build_flex_mask_meta."""
    torch, dev = torch_dev
    meta = orc.FlexMeta(1, 4, 4, 4, 1, 4, 2, 1, 3, 2, 1, 2, 2, 2, 7, 8)
    # meta length: 2*latent + 2*action + pad = 2*(2*2*2) + 2*(4*2*1) + 3 = 35
    n = 35
    tm = orc.self_token_mask(meta, n)
    bs = 8
    rp, ci = orc.self_block_table(meta, n, bs)
    qb = (n + bs - 1) // bs
    bmap = np.zeros((qb, qb), np.uint8)
    for r in range(qb):
        bmap[r, ci[rp[r]:rp[r + 1]]] = 1
    rng = np.random.default_rng(12)
    H, D = 2, 64
    s = Seqs(orc, rng, [n], [n], H, H, D)
    got = s.run(emb, torch, dev, 0.125, mask_kind=emb.EMB_MASK_BLOCKMAP, block_map=_t(torch, dev, bmap),
                block_size=bs, block_map_cols=qb, mask=_t(torch, dev, tm), mask_q_stride=n)[0]
    qf, kf, vf = (orc.bf16_to_f32(x).reshape(-1) for x in (s.q[0], s.k[0], s.v[0]))
    ref = orc.flex_attention(qf, kf, vf, rp, ci, tm, n, n, H, D, bs, 0.125).reshape(n, H, D)
    assert_close(got, ref, "flex block map")


def test_valid_slot_list_with_gaps_and_negative_slots(emb, orc, torch_dev):
    """runtime_kv_attn over an arbitrary valid-slot list (LingBot after eviction and mode 0):
    a negative slot is a zero K/V row, as in the online/warp reference kernels."""
    torch, dev = torch_dev
    rng = np.random.default_rng(13)
    H, D, cap, nq = 4, 128, 300, 33
    ck = _bf16(orc, rng, (cap, H, D))
    cv = _bf16(orc, rng, (cap, H, D))
    q = _bf16(orc, rng, (nq, H, D))
    valid = np.concatenate([np.arange(16, 48), rng.choice(np.arange(48, cap), 150, replace=False), [-1, -1],
                            np.arange(0, 7)]).astype(np.int32)
    n_pages = cap // 16 + 1
    bt = rng.permutation(n_pages + 2)[:n_pages].astype(np.int32)
    kp = np.zeros((n_pages + 2) * H * 16 * D, np.uint16)
    vp = np.zeros_like(kp)
    orc.paged_append(ck, cv, H * D, np.arange(cap, dtype=np.int32), bt, H, D, cap, kp, vp)
    out = torch.zeros((nq, H, D), dtype=torch.float32, device=dev)
    keep = [_t(torch, dev, x) for x in (q, kp, vp, bt, valid)]
    emb.paged_attention(q=keep[0], out=out, k_pool=keep[1], v_pool=keep[2], batch=1, hq=H, hkv=H, d=D,
                        max_q=nq, scale=0.1, capacity=cap, cu_q=_t(torch, dev, np.array([0, nq], np.int32)),
                        n_keys=_t(torch, dev, np.array([len(valid)], np.int32)), block_tables=keep[3],
                        bt_stride=n_pages, valid_slots=keep[4], valid_stride=len(valid))
    torch.cuda.synchronize()
    ref = orc.runtime_kv_attn(orc.bf16_to_f32(q).reshape(-1), orc.bf16_to_f32(ck).reshape(-1),
                              orc.bf16_to_f32(cv).reshape(-1), valid, nq, H, D, 0.1).reshape(nq, H, D)
    assert_close(out.cpu().numpy(), ref, "valid list")


def test_reference_named_runtime_kv_attention(emb, orc, torch_dev):
    """lingbot_runtime_kv_{update,attn,attn_online,attn_warp,attn_cublas}_f32 with the
    reference's signatures (kernels/lingbot/lingbot_flex_attn_cuda.h:46-93)."""
    torch, dev = torch_dev
    rng = np.random.default_rng(14)
    H, D, cap, nq = 3, 128, 96, 20
    kb, vb, qb = _bf16(orc, rng, (cap, H, D)), _bf16(orc, rng, (cap, H, D)), _bf16(orc, rng, (nq, H, D))
    kf, vf, qf = orc.bf16_to_f32(kb), orc.bf16_to_f32(vb), orc.bf16_to_f32(qb)
    ck = torch.zeros(cap * H * D, dtype=torch.float32, device=dev)
    cv = torch.zeros_like(ck)
    L = emb.lib()
    tk, tv, tq = _t(torch, dev, kf), _t(torch, dev, vf), _t(torch, dev, qf)
    slots = _t(torch, dev, np.arange(cap, dtype=np.int32))
    assert L.lingbot_runtime_kv_update_f32(tk.data_ptr(), tv.data_ptr(), ck.data_ptr(), cv.data_ptr(),
                                           slots.data_ptr(), cap, H, D, cap, None) == 0
    valid = np.array(list(range(0, 40)) + list(range(50, 96)), np.int32)
    tvld = _t(torch, dev, valid)
    ref = orc.runtime_kv_attn(qf.reshape(-1), kf.reshape(-1), vf.reshape(-1), valid, nq, H, D,
                              1 / math.sqrt(D)).reshape(nq, H, D)
    for name in ("lingbot_runtime_kv_attn_f32", "lingbot_runtime_kv_attn_online_f32",
                 "lingbot_runtime_kv_attn_warp_f32", "lingbot_runtime_kv_attn_cublas_f32"):
        out = torch.zeros((nq, H, D), dtype=torch.float32, device=dev)
        args = [tq.data_ptr(), ck.data_ptr(), cv.data_ptr(), tvld.data_ptr(), out.data_ptr(), nq, len(valid), H, D]
        if name.endswith("cublas_f32"):
            args.append(cap)
        rc = getattr(L, name)(*args, 1 / math.sqrt(D), None)
        assert rc == 0, emb.last_error()
        torch.cuda.synchronize()
        assert_close(out.cpu().numpy(), ref, name)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_head_dims_and_ragged_batch(emb, orc, torch_dev, d):
    """Ragged batch: query counts 1..70 (partial row tiles), key counts not multiples of 16."""
    torch, dev = torch_dev
    rng = np.random.default_rng(d)
    nq = [1, 17, 70, 33]
    nk = [5, 77, 300, 129]
    s = Seqs(orc, rng, nk, nq, 4, 2, d)
    got = s.run(emb, torch, dev, 1 / math.sqrt(d))
    for b in range(len(nq)):
        assert_close(got[b], s.oracle(orc, b, 1 / math.sqrt(d)), f"d={d} b={b}")
    if d >= 128:
        s.ks_check(orc, 1 / math.sqrt(d), f"d={d}")
    got3 = s.run(emb, torch, dev, 1 / math.sqrt(d), splits=3)
    for b in range(len(nq)):
        assert_close(got3[b], s.oracle(orc, b, 1 / math.sqrt(d)), f"d={d} b={b} split 3")
