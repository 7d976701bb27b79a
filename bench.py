"""Benchmark of the KV-cached attention step on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs cfg1,cfg2,cfg3,cfg4]
                    [--no-cpu] [--only cfg1_attn]

Headline (the JSON line's `value`): BASELINE.json configs[0] -- the pi0.5
action-expert denoise step: 18 layers, each with an 816-token cached prefix
(1 kv head, head_dim 256, bf16) in 16-token pages scattered over one pool,
fresh Q [51 tokens x 8 heads] and fresh action K/V [51] per layer per step.
One step = one append launch (51 new K/V rows into every layer's temporary
slots 816..866) + one attention launch over the 18 layers' (51x8) x 867
problems, replayed from a HIP graph.  Unit: microseconds per denoise step.

Other configs run as extra measurements in the same JSON object ("extra").
All inputs are synthetic N(0,1) bf16 from the library's std::mt19937_64
generator (seed 0xE3BD0000 + config index), uploaded before timing starts.
The CPU baseline times the oracle's fp32 restatement of the ggml op order on
host cores (bounded sample, see `cpu_baseline.sample`).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "embodied.cpp_amd"))

PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0
PEAK_FP32_TFLOPS = 157.3  # MI355X dense fp32 MFMA


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


class Ctx:
    def __init__(self):
        import torch

        import embkv

        self.torch = torch
        self.emb = embkv
        embkv.lib()
        self.dev = torch.device("cuda:0")
        self.stream = torch.cuda.current_stream()

    def synth(self, seed, n):
        """N(0,1) bf16 from the library generator, as an int16 device tensor."""
        return self.torch.from_numpy(self.emb.synth_normal_bf16(seed, n).view(np.int16)).to(self.dev)

    def i32(self, a):
        return self.torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(self.dev)

    def time_graph(self, fn, steps, warmup):
        """Captures fn() once into a HIP graph; replays warmup + steps times.
        Returns (ms per replay, graph) measured with events on the replay stream."""
        torch = self.torch
        fn(torch.cuda.current_stream())  # eager once (also validates arguments)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                fn(s)
        torch.cuda.synchronize()
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        cur = torch.cuda.current_stream()
        e0.record(cur)
        for _ in range(steps):
            g.replay()
        e1.record(cur)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps, g


# ---------------------------------------------------------------------------
# cfg1: pi0.5 action expert over the cached prefix (denoise steps)
# ---------------------------------------------------------------------------
class PagedLayers:
    """L independent caches (layers or sessions) sharing one permuted page pool.
    Cache b holds n_keys[b] slots: a prefix plus n_new temporary slots."""

    def __init__(self, c: Ctx, seed, n_prefix, n_new, hq, hkv, d, n_steps, extra_pages=64):
        torch, emb = c.torch, c.emb
        self.c = c
        self.L = len(n_prefix)
        self.n_prefix = [int(x) for x in n_prefix]
        self.n_new, self.hq, self.hkv, self.d = n_new, hq, hkv, d
        self.n_keys = [p + n_new for p in self.n_prefix]
        pages = [(k + 15) // 16 for k in self.n_keys]
        self.bt_stride = max(pages)
        self.cap = self.bt_stride * 16
        total_pages = sum(pages) + extra_pages
        g = np.random.default_rng(seed)
        perm = g.permutation(total_pages).astype(np.int32)
        bt = np.full((self.L, self.bt_stride), -1, np.int32)
        o = 0
        for b, p in enumerate(pages):
            bt[b, :p] = perm[o:o + p]
            o += p
        self.bt_np = bt
        self.bt = c.i32(bt)
        self.total_pages = total_pages
        page_elems = hkv * 16 * d
        self.k_pool = torch.zeros(total_pages * page_elems, dtype=torch.int16, device=c.dev)
        self.v_pool = torch.zeros_like(self.k_pool)
        self.v16_pool = torch.zeros_like(self.k_pool)  # f16 V shadow (zero-filled)
        # prefix K/V appended through the library (one combined slot space:
        # cache b's slot s is logical slot b*cap + s of one concatenated table)
        tot_pref = sum(self.n_prefix)
        if tot_pref:
            kpre = c.synth(seed + 1, tot_pref * hkv * d)
            vpre = c.synth(seed + 2, tot_pref * hkv * d)
            slots = np.concatenate([b * self.cap + np.arange(p) for b, p in enumerate(self.n_prefix)])
            emb.kv_append(kpre, vpre, hkv * d, tot_pref, c.i32(slots), self.bt, self.L * self.cap,
                          self.k_pool, self.v_pool, hkv, d, v16_pool=self.v16_pool)
        # per-step new K/V and Q
        self.new_slots = c.i32(np.concatenate([b * self.cap + p + np.arange(n_new)
                                               for b, p in enumerate(self.n_prefix)]))
        self.n_steps = n_steps
        self.q = [c.synth(seed + 10 + s, self.L * n_new * hq * d) for s in range(n_steps)]
        self.knew = [c.synth(seed + 100 + s, self.L * n_new * hkv * d) for s in range(n_steps)]
        self.vnew = [c.synth(seed + 200 + s, self.L * n_new * hkv * d) for s in range(n_steps)]
        self.cu_q = c.i32(np.arange(self.L + 1) * n_new)
        self.nk = c.i32(self.n_keys)
        # equal caches launch in the uniform form (no bounds arrays to read)
        self.uniform = len(set(self.n_keys)) == 1
        self.out = torch.zeros((self.L * n_new, hq, d), dtype=torch.float32, device=c.dev)
        self.ws = None
        torch.cuda.synchronize()

    def set_splits(self, splits, split_keys=0, kernel=None):
        """Split-K factor and kernel (embkv.EMB_ATTN_*; None: the row tiles, which
        every split factor runs on)."""
        self.splits = splits
        self.split_keys = split_keys
        self.kernel = self.c.emb.EMB_ATTN_ROW_TILES if kernel is None else kernel
        if splits > 1:
            nb = self.c.emb.attn_workspace_bytes(self.L, self.n_new, self.hq, self.hkv, self.d, splits)
            self.ws = self.c.torch.zeros(nb // 4 + 64, dtype=self.c.torch.float32, device=self.c.dev)

    def append(self, step, stream):
        s = step % self.n_steps
        self.c.emb.kv_append(self.knew[s], self.vnew[s], self.hkv * self.d, self.L * self.n_new,
                             self.new_slots, self.bt, self.L * self.cap, self.k_pool, self.v_pool,
                             self.hkv, self.d, stream=stream, v16_pool=self.v16_pool)

    def attend(self, step, stream, scale, q=None):
        s = step % self.n_steps
        self.c.emb.paged_attention(q=self.q[s] if q is None else q, out=self.out, k_pool=self.k_pool, v_pool=self.v_pool,
                                   v16_pool=self.v16_pool,
                                   batch=self.L, hq=self.hq, hkv=self.hkv, d=self.d, max_q=self.n_new,
                                   scale=scale, capacity=self.cap,
                                   cu_q=None if self.uniform else self.cu_q,
                                   n_keys=None if self.uniform else self.nk,
                                   n_keys_uniform=self.n_keys[0] if self.uniform else 0,
                                   block_tables=self.bt, bt_stride=self.bt_stride, splits=self.splits,
                                   workspace=self.ws, stream=stream, split_keys=getattr(self, "split_keys", 0),
                                   kernel=getattr(self, "kernel", 0))

    # algorithmic bytes of one attention launch: K/V of every key once, Q, O (f32), tables
    def attn_bytes(self):
        kv = sum(self.n_keys) * self.hkv * self.d * 2 * 2
        q = self.L * self.n_new * self.hq * self.d * 2
        o = self.L * self.n_new * self.hq * self.d * 4
        return kv + q + o + self.L * self.bt_stride * 4

    def attn_flops(self):
        return sum(4.0 * self.n_new * self.hq * k * self.d for k in self.n_keys)

    def survey_step_bytes(self):
        """Per-unit algorithmic bytes as defined for configs 1/4: prefix K/V,
        new K/V read + written, Q and O at bf16, block table."""
        b = 0
        for p, k in zip(self.n_prefix, self.n_keys):
            b += p * self.hkv * self.d * 4 + 2 * self.n_new * self.hkv * self.d * 4
            b += 2 * self.n_new * self.hq * self.d * 2 + 4 * ((k + 15) // 16)
        return b


def kernel_choices(c: Ctx, splits_list):
    """(label, kernel, splits) candidates: the key-split kernel, then the row
    tiles at each split factor."""
    emb = c.emb
    return [("key_split", emb.EMB_ATTN_KEY_SPLIT, 1)] + [(f"row_tiles_split{sp}", emb.EMB_ATTN_ROW_TILES, sp)
                                                          for sp in splits_list]


def bench_cfg1(c: Ctx, steps, warmup, splits_list=(1, 2, 3, 4, 8)):
    n_layers, n_pref, n_new, hq, hkv, d = 18, 816, 51, 8, 1, 256
    P = PagedLayers(c, 0xE3BD0000, [n_pref] * n_layers, n_new, hq, hkv, d, n_steps=10)
    scale = 1.0 / math.sqrt(d)
    best = None
    sweep = {}
    # each candidate timed as 10 launches in one graph (a launch alone is
    # dominated by the graph launch itself, which the denoise-step graph pays
    # once for all its launches)
    def ten(st):
        for i in range(10):
            P.attend(i, st, scale)
    for label, kern, sp in kernel_choices(c, splits_list):
        P.set_splits(sp, kernel=kern)
        ms10, _ = c.time_graph(ten, max(2, steps // 4), 2)
        ms = ms10 / 10
        sweep[label] = ms * 1e3
        if best is None or ms < best[1]:
            best = ((sp, kern, label), ms)
    P.set_splits(best[0][0], kernel=best[0][1])
    attn_us = best[1] * 1e3
    # K consecutive attention launches in one graph: the kernel's average duration
    k_launch = 20

    def attn_many(st):
        for i in range(k_launch):
            P.attend(i, st, scale)
    ms_many, _ = c.time_graph(attn_many, max(2, steps // 4), 2)
    attn_avg_us = ms_many * 1e3 / k_launch

    step_counter = [0]

    def one_step(st):
        P.append(step_counter[0], st)
        P.attend(step_counter[0], st, scale)
    # one step per graph replay: adds a graph launch to every step
    ms_step1, _ = c.time_graph(one_step, steps, warmup)

    # The headline: `steps` consecutive denoise steps (each an append and an
    # attention launch, fresh Q and new K/V per step, the cached prefix shared)
    # captured in one graph and timed as one replay -- a pi0.5 predict() runs
    # its denoise steps in one graph_compute (models/pi05.cpp:797-894).  The
    # warmup replays the same graph (at least once).
    def k_steps(st):
        for s in range(steps):
            P.append(s, st)
            P.attend(s, st, scale)
    ms_k, _ = c.time_graph(k_steps, 1, max(1, -(-warmup // steps)))
    ms_step = ms_k / steps

    # ten denoise steps (the whole config-1 workload) captured as one graph
    def ten_steps(st):
        for s in range(10):
            P.append(s, st)
            P.attend(s, st, scale)
    ms_ten, _ = c.time_graph(ten_steps, max(2, steps // 4), 2)

    # one layer's attention alone (what a model that runs its layers in order sees
    # per layer): average launch time of k_launch launches in one graph, by split
    single = PagedLayers(c, 0xE3BD0000, [n_pref], n_new, hq, hkv, d, n_steps=1)

    def single_many(st):
        for _ in range(k_launch):
            single.attend(0, st, scale)
    sweep1 = {}
    choices1 = {lab: (kern, sp) for lab, kern, sp in kernel_choices(c, (1, 2, 4, 8, 16))}
    for lab, (kern, sp) in choices1.items():
        single.set_splits(sp, kernel=kern)
        ms1, _ = c.time_graph(single_many, max(2, steps // 4), 2)
        sweep1[lab] = ms1 * 1e3 / k_launch
    best1 = min(sweep1, key=sweep1.get)
    single.set_splits(choices1[best1][1], kernel=choices1[best1][0])

    # dependent per-layer launches (model-realistic ordering): 18 x (append, attention)
    layers = [single] * n_layers  # same shapes; the graph holds 36 dependent launches

    def per_layer(st):
        for lp in layers:
            lp.append(0, st)
            lp.attend(0, st, scale)
    ms_layer, _ = c.time_graph(per_layer, max(2, steps // 2), 2)

    # the pi0.5 producer in place of the plain append: the expert's f32 Q/K/V
    # projection outputs go through NEOX RoPE at positions 816 + i
    # (models/pi05.cpp:394-402) into a bf16 Q and the cache, then attention
    # reads that Q -- one producer launch for the 18 layers' 51 tokens
    torch, emb = c.torch, c.emb
    T = n_layers * n_new
    q32 = c.synth(0xE3BD0300, T * hq * d).view(torch.bfloat16).float()
    k32 = c.synth(0xE3BD0301, T * hkv * d).view(torch.bfloat16).float()
    v32 = c.synth(0xE3BD0302, T * hkv * d).view(torch.bfloat16).float()
    q_roped = torch.zeros(T * hq * d, dtype=torch.int16, device=c.dev)
    positions = c.i32(np.tile(n_pref + np.arange(n_new), n_layers))

    def produce(st):
        emb.qkv_neox_rope_append(q32, hq * d, k32, hkv * d, v32, hkv * d, T, hq, hkv, d, q_roped, P.new_slots,
                                 P.bt, P.L * P.cap, P.k_pool, P.v_pool, v16_pool=P.v16_pool, positions=positions,
                                 q_out_f32=False, stream=st)
    ms_prod, _ = c.time_graph(produce, steps, warmup)

    def produce_attend(st):
        produce(st)
        P.attend(0, st, scale, q=q_roped)
    ms_prod_step, _ = c.time_graph(produce_attend, steps, warmup)
    prod_bytes = T * (hq + 2 * hkv) * d * 4 + T * hq * d * 2 + 3 * T * hkv * d * 2 + T * 4 * 2

    # cold vs warm: eager steps, each after 1 GiB is rewritten on the stream
    # (flushes the 256 MB MALL and the L2s; outside the timed region) or not
    cold_us, warm_us = cold_warm_steps(c, one_step, n=max(5, steps // 4))

    ab = P.attn_bytes()
    return dict(
        us_per_step=ms_step * 1e3,
        us_per_step_one_step_graph=ms_step1 * 1e3,
        us_per_step_cold=cold_us,
        us_per_step_warm_eager=warm_us,
        us_per_step_10step_graph=ms_ten * 1e3 / 10,
        us_per_step_dependent_layers=ms_layer * 1e3,
        attn_us_single_layer=sweep1[best1],
        single_layer_kernel=best1,
        single_layer_split_sweep_us=sweep1,
        us_per_step_with_neox_producer=ms_prod_step * 1e3,
        neox_producer_us=ms_prod * 1e3,
        neox_producer_bytes=prod_bytes,
        neox_producer_gbs=prod_bytes / (ms_prod * 1e-3) / 1e9,
        attn_us_in_sweep=attn_us,
        attn_us_avg_in_graph=attn_avg_us,
        splits=best[0][0],
        kernel=best[0][2],
        kernel_sweep_us=sweep,
        attn_bytes_per_launch=ab,
        attn_flops_per_launch=P.attn_flops(),
        survey_bytes_per_step=P.survey_step_bytes(),
    )


def cold_warm_steps(c: Ctx, fn, n):
    """Median GPU time (us) of fn(stream) run eagerly: cold = right after 1 GiB
    is written on the stream (flushes the 256 MB MALL and the L2s; the write
    also gives the host time to enqueue the step), warm = the second of two
    back-to-back runs."""
    torch = c.torch
    flush = torch.empty(1 << 28, dtype=torch.float32, device=c.dev)
    Ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    cold, warm = [], []
    for _ in range(n):
        e0, e1, e2 = Ev(), Ev(), Ev()
        with torch.cuda.stream(c.stream):
            flush.fill_(1.0)
            e0.record(c.stream)
            fn(c.stream)
            e1.record(c.stream)
            fn(c.stream)
            e2.record(c.stream)
        torch.cuda.synchronize()
        cold.append(e0.elapsed_time(e1) * 1e3)
        warm.append(e1.elapsed_time(e2) * 1e3)
    del flush
    return float(np.median(cold)), float(np.median(warm))


def bench_cfg4(c: Ctx, steps, warmup):
    from embkv import lib  # noqa: F401  (library loaded by Ctx)
    res = {}
    # L_b ~ U[300, 1200] from std::mt19937_64(0xE3BD0004): L_b = 300 + x % 901
    g = MT64(0xE3BD0004)
    lens_all = [300 + g.next() % 901 for _ in range(64)]
    for B in (1, 8, 32, 64):
        P = PagedLayers(c, 0xE3BD0004 + B, lens_all[:B], 51, 8, 1, 256, n_steps=2)
        # (splits, split_keys): uniform splits, and per-session splits sized
        # by each session's key count (split_keys > 0)
        # and the key-split kernel (one workgroup per 32 rows, no split)
        best = None
        sweep = {}
        ks = c.emb.EMB_ATTN_KEY_SPLIT
        # (2, 640..896): only the long sessions split in two, the short ones
        # written by their own workgroups (no partials, skipped by the merge)
        for sp, sk, kern in ((1, 0, ks), (1, 0, None), (2, 0, None), (4, 0, None), (8, 0, None), (3, 384, None),
                             (4, 256, None), (4, 320, None), (6, 192, None), (8, 128, None), (2, 640, None),
                             (2, 768, None), (2, 896, None)):
            if B >= 32 and sk == 0 and sp > 2:
                continue
            P.set_splits(sp, sk, kernel=kern)
            ms, _ = c.time_graph(lambda st: P.attend(0, st, 1 / 16), steps, warmup)
            label = "key_split" if kern == ks else f"{sp}/{sk}"
            sweep[label] = ms * 1e3
            if best is None or ms < best[1]:
                best = ((sp, sk, kern, label), ms)
        P.set_splits(best[0][0], best[0][1], kernel=best[0][2])

        def one(st):
            P.append(0, st)
            P.attend(0, st, 1 / 16)
        ms_all, _ = c.time_graph(one, steps, warmup)
        ab = P.attn_bytes()
        res[f"B{B}"] = dict(attn_us=best[1] * 1e3, append_plus_attn_us=ms_all * 1e3, splits=best[0][0],
                            split_keys=best[0][1], kernel=best[0][3], split_sweep_us=sweep,
                            attn_gbs=ab / (best[1] * 1e-3) / 1e9,
                            attn_hbm_frac=ab / (best[1] * 1e-3) / 1e9 / PEAK_HBM_GBS,
                            survey_bytes=P.survey_step_bytes(),
                            survey_gbs=P.survey_step_bytes() / (ms_all * 1e-3) / 1e9,
                            attn_tflops=P.attn_flops() / (best[1] * 1e-3) / 1e12,
                            mean_prefix=float(np.mean(lens_all[:B])))
        del P
        c.torch.cuda.empty_cache()
    return res


def bench_cfg2(c: Ctx, steps, warmup):
    """Prefix prefill + cache build: 18 layers x (append 816 tokens into pages, bidirectional
    prefix attention 816 x 8 heads over 816 keys), one launch each for all layers."""
    torch, emb = c.torch, c.emb
    L, n, hq, hkv, d = 18, 816, 8, 1, 256
    P = PagedLayers(c, 0xE3BD0001, [0] * L, n, hq, hkv, d, n_steps=1)
    # the prefix K/V first: over the zero-filled pool every output row is zero
    # and the kernel takes its exact recompute path, which the sweep must not time
    P.append(0, torch.cuda.current_stream())
    torch.cuda.synchronize()
    sweep = {}
    for sp in (1, 2):
        P.set_splits(sp)
        ms_s, _ = c.time_graph(lambda st: P.attend(0, st, 1 / 16), steps, warmup)
        sweep[sp] = ms_s * 1e3
    best = min(sweep, key=sweep.get)
    P.set_splits(best)

    def one(st):
        P.append(0, st)
        P.attend(0, st, 1 / 16)
    ms, _ = c.time_graph(one, steps, warmup)
    ms_a, _ = c.time_graph(lambda st: P.attend(0, st, 1 / 16), steps, warmup)
    fl = P.attn_flops()
    return dict(us_per_prefill=ms * 1e3, attn_us=ms_a * 1e3, attn_tflops=fl / (ms_a * 1e-3) / 1e12,
                mfma_frac=fl / (ms_a * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, flops=fl, splits=best, split_sweep_us=sweep)


def bench_cfg3(c: Ctx, steps, warmup, n_layers=30, eager_only=False):
    """LingBot-VA chunk step: 24 heads (MHA), head_dim 128, chunk 1560 tokens, 9-chunk window
    (14040 slots).  Steady state: each step appends one chunk into the slots the evicted
    oldest chunk held and attends over all 14040 keys; 30 dependent layers per step."""
    torch, emb = c.torch, c.emb
    H, d, C, W = 24, 128, 1560, 9
    cap = C * W
    pages = cap // 16 + (1 if cap % 16 else 0)
    page_elems = H * 16 * d
    base_k = c.synth(0xE3BD0002 + 1, cap * H * d)
    base_v = c.synth(0xE3BD0002 + 2, cap * H * d)
    q = c.synth(0xE3BD0002 + 3, C * H * d)
    knew = c.synth(0xE3BD0002 + 4, C * H * d)
    vnew = c.synth(0xE3BD0002 + 5, C * H * d)
    pools = []
    g = np.random.default_rng(3)
    for l in range(n_layers):
        bt = g.permutation(pages).astype(np.int32)
        kp = torch.empty(pages * page_elems, dtype=torch.int16, device=c.dev)
        vp = torch.empty_like(kp)
        v16 = torch.zeros_like(kp)
        bt_d = c.i32(bt)
        emb.kv_append(base_k, base_v, H * d, cap, c.i32(np.arange(cap)), bt_d, cap, kp, vp, H, d, v16_pool=v16)
        pools.append((kp, vp, v16, bt_d))
    out = torch.empty((C, H, d), dtype=torch.float32, device=c.dev)
    # the slot range the evicted oldest chunk held (chunk 0), reused by the new chunk
    new_slots = c.i32(np.arange(C))
    scale = 1 / math.sqrt(d)
    cur_split = [1, None]  # splits, workspace

    def set_split(sp):
        cur_split[0] = sp
        cur_split[1] = None
        if sp > 1:
            nb = emb.attn_workspace_bytes(1, C, H, H, d, sp)
            cur_split[1] = torch.zeros(nb // 4 + 64, dtype=torch.float32, device=c.dev)

    def layer(l, st, append=True):
        kp, vp, v16, bt = pools[l]
        if append:
            emb.kv_append(knew, vnew, H * d, C, new_slots, bt, cap, kp, vp, H, d, stream=st, v16_pool=v16)
        emb.paged_attention(q=q, out=out, k_pool=kp, v_pool=vp, v16_pool=v16, batch=1, hq=H, hkv=H, d=d, max_q=C,
                            scale=scale, capacity=cap, n_keys_uniform=cap, block_tables=bt, bt_stride=pages,
                            splits=cur_split[0], workspace=cur_split[1], stream=st)

    if eager_only:  # profiling: plain launches of the attention kernel
        set_split(4)
        for i in range(warmup + steps):
            layer(i % n_layers, c.stream, False)
        torch.cuda.synchronize()
        return {}
    sweep = {}
    for sp in (1, 2, 3, 4, 6):
        set_split(sp)
        ms_s, _ = c.time_graph(lambda st: [layer(l, st, False) for l in range(min(4, n_layers))], 3, 1)
        sweep[sp] = ms_s * 1e3 / min(4, n_layers)
    best = min(sweep, key=sweep.get)
    set_split(best)
    ms_step, _ = c.time_graph(lambda st: [layer(l, st) for l in range(n_layers)], max(2, steps // 4), 1)
    ms_attn, _ = c.time_graph(lambda st: [layer(l, st, False) for l in range(n_layers)], max(2, steps // 4), 1)
    # the chunk append alone (1560 tokens x 24 heads into the evicted chunk's
    # slots, with the f16 shadow), 30 layers' pools in one graph
    ms_app, _ = c.time_graph(lambda st: [emb.kv_append(knew, vnew, H * d, C, new_slots, pools[l][3], cap, pools[l][0],
                                                       pools[l][1], H, d, stream=st, v16_pool=pools[l][2])
                                         for l in range(n_layers)], max(2, steps // 4), 1)
    app_us = ms_app * 1e3 / n_layers
    # the compact copy of all 14040 cached rows in valid-slot order that the
    # reference makes before its attention (runtime_kv_gather); the paged
    # attention reads the pages in place instead
    gk = torch.empty((cap, H, d), dtype=torch.int16, device=c.dev)
    gv = torch.empty_like(gk)
    valid_all = c.i32(np.arange(cap, dtype=np.int32))
    ms_g, _ = c.time_graph(lambda st: [emb.kv_gather(pools[l][0], pools[l][1], valid_all, cap, pools[l][3], cap, gk,
                                                     gv, H, d, stream=st) for l in range(4)], max(2, steps // 4), 1)
    gather_us = ms_g * 1e3 / 4
    gather_bytes = cap * H * d * 2 * 4 + cap * 4  # read K, V; write K, V; the slot list
    del gk, gv
    app_bytes = C * H * d * 2 * 2 + C * H * d * 2 * 3 + C * 4  # read K, V; write K, V, shadow; slots
    fl_layer = 4.0 * C * H * cap * d
    attn_layer_us = ms_attn * 1e3 / n_layers
    del pools
    torch.cuda.empty_cache()
    return dict(ms_per_step=ms_step, attn_ms_per_step=ms_attn, attn_us_per_layer=attn_layer_us,
                attn_tflops=fl_layer / (attn_layer_us * 1e-6) / 1e12,
                mfma_frac=fl_layer / (attn_layer_us * 1e-6) / 1e12 / PEAK_BF16_TFLOPS,
                flops_per_layer=fl_layer, layers=n_layers, splits=best, split_sweep_us_per_layer=sweep,
                append_chunk_us=app_us, append_chunk_gbs=app_bytes / (app_us * 1e-6) / 1e9,
                gather_window_us=gather_us, gather_window_gbs=gather_bytes / (gather_us * 1e-6) / 1e9)


def bench_meta(c: Ctx, steps, n_layers=30):
    """Runtime-KV slot metadata per layer call at the config-3 shape (14040 slots,
    1560-token chunks, steady state: every call evicts the oldest chunk).
    Device: one emb_dev_cache_update (mode 2, slots + valid list in device
    memory) per layer, 30 layers' caches, graph-timed.  Host: the reference's
    order per layer -- the host cache's update_meta_only and
    collect_valid_slots, then synchronous host-to-device copies of the slots
    and the valid list (models/lingbot_va.cpp:9568-9650, :9697-9767) --
    wall-clock timed."""
    torch, emb = c.torch, c.emb
    cap, C = 14040, 1560
    dev = [emb.DevSlotCache(cap, c.dev) for _ in range(n_layers)]
    host = [emb.SlotCache(cap) for _ in range(n_layers)]
    for _ in range(10):  # past the point where the window is full
        for d in dev:
            d.update(C, 2)
        for h in host:
            h.update_meta(C, 0)
    torch.cuda.synchronize()

    def dev_step(st):
        for d in dev:
            d.update(C, 2, stream=st)
    ms, _ = c.time_graph(dev_step, max(2, steps // 4), 2)
    dev_us = ms * 1e3 / n_layers
    slots_d = torch.empty(C, dtype=torch.int32, device=c.dev)
    valid_d = torch.empty(cap, dtype=torch.int32, device=c.dev)
    reps = max(2, steps // 4)
    t0 = time.perf_counter()
    for _ in range(reps):
        for h in host:
            sl, rc = h.update_meta(C, 0)
            vl = h.collect_valid()
            slots_d.copy_(torch.from_numpy(sl.astype(np.int32)))
            valid_d.copy_(torch.from_numpy(vl.astype(np.int32)))
            torch.cuda.synchronize()
    host_us = (time.perf_counter() - t0) * 1e6 / (reps * n_layers)
    return dict(dev_us_per_layer_call=dev_us, host_us_per_layer_call=host_us, capacity=cap, chunk=C,
                layers=n_layers)


def bench_cosmos3_gqa(c: Ctx, steps, warmup):
    """Cosmos3 language-tower causal GQA attention through the reference-named face
    (cosmos3_qwen_causal_gqa_attention_f32): 3200 packed text + vision + action tokens,
    32 query heads over 8 kv heads, head_dim 128, f32 in and out (staging of the f32
    K/V into the paged pool and the bf16 rounding of the output included)."""
    torch, emb = c.torch, c.emb
    T, HQ, HKV, D = 3200, 32, 8, 128
    q = torch.randn((T, HQ * D), dtype=torch.float32, device=c.dev, generator=torch.Generator(c.dev).manual_seed(5))
    k = torch.randn((T, HKV * D), dtype=torch.float32, device=c.dev, generator=torch.Generator(c.dev).manual_seed(6))
    v = torch.randn((T, HKV * D), dtype=torch.float32, device=c.dev, generator=torch.Generator(c.dev).manual_seed(7))
    y = torch.empty((T, HQ * D), dtype=torch.float32, device=c.dev)
    L = emb.lib()

    def run(st):
        emb.check(L.cosmos3_qwen_causal_gqa_attention_f32(q.data_ptr(), k.data_ptr(), v.data_ptr(), y.data_ptr(),
                                                          T, HQ * D, HKV * D, HQ, HKV, D, emb.stream_ptr(st)),
                  "cosmos3_qwen_causal_gqa_attention_f32")
    ms, _ = c.time_graph(run, steps, warmup)
    flops = 4.0 * HQ * D * T * (T + 1) / 2  # causal: key j <= query i
    return dict(us=ms * 1e3, tflops=flops / (ms * 1e-3) / 1e12, mfma_frac=flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                tokens=T, q_heads=HQ, kv_heads=HKV, head_dim=D)


def _bf16_bits(f: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(f, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bench_cfg5(c: Ctx, steps, warmup):
    """W8A16 QKV projection (1560 x 3072 -> 3 x 3072, int8 Marlin layout, bf16 scales) alone, and
    fused with the append of its K/V slices into a config-3 paged cache followed by the config-3
    attention over 14040 keys (one layer)."""
    torch, emb = c.torch, c.emb
    M, K, H, d, C, W = 1560, 3072, 24, 128, 1560, 9
    N = 3 * H * d
    x = c.synth(0xE3BD0004 + 1, M * K)
    g = np.random.default_rng(0xE3BD0004)
    # u8 = w + 128 with w ~ U[-127, 127]: uniform random bytes in [1, 255] are a uniform random
    # weight in any byte order, so the Marlin payload is drawn directly
    qw = torch.from_numpy(g.integers(1, 256, (K // 16, 16 * N), dtype=np.uint8).view(np.int32)).to(c.dev)
    sc = torch.from_numpy(_bf16_bits(g.uniform(0.001, 0.01, N).astype(np.float32)).view(np.int16)).to(c.dev)
    y = torch.empty((M, N), dtype=torch.int16, device=c.dev)
    flops = 2.0 * M * K * N

    def gemm(st):
        emb.w8a16_gemm(x, qw, sc, M, K, N, y, stream=st)
    ms_g, _ = c.time_graph(gemm, steps, warmup)
    k_launch = 10

    def gemm_many(st):
        for _ in range(k_launch):
            emb.w8a16_gemm(x, qw, sc, M, K, N, y, stream=st)
    ms_many, _ = c.time_graph(gemm_many, max(2, steps // 4), 2)
    gemm_us = ms_many * 1e3 / k_launch

    cap = C * W
    pages = (cap + 15) // 16
    bt = c.i32(g.permutation(pages))
    page_elems = H * 16 * d
    kp = torch.zeros(pages * page_elems, dtype=torch.int16, device=c.dev)
    vp = torch.zeros_like(kp)
    v16 = torch.zeros_like(kp)
    kv0 = c.synth(0xE3BD0004 + 2, cap * H * d)
    emb.kv_append(kv0, kv0, H * d, cap, c.i32(np.arange(cap)), bt, cap, kp, vp, H, d, v16_pool=v16)
    qo = torch.empty((M, H * d), dtype=torch.int16, device=c.dev)
    slots = c.i32(np.arange(C))  # the new chunk takes the slots of the evicted oldest chunk
    out = torch.empty((C, H, d), dtype=torch.float32, device=c.dev)

    def fused(st):
        emb.w8a16_qkv_append(x, qw, sc, M, K, H * d, qo, slots, bt, cap, kp, vp, H, d, stream=st, v16_pool=v16)

    att_splits = 4  # the config-3 attention's best split on MI355X
    ws = torch.zeros(emb.attn_workspace_bytes(1, C, H, H, d, att_splits) // 4 + 64, dtype=torch.float32, device=c.dev)

    def step(st):
        fused(st)
        emb.paged_attention(q=qo, out=out, k_pool=kp, v_pool=vp, v16_pool=v16, batch=1, hq=H, hkv=H, d=d, max_q=C,
                            scale=1 / math.sqrt(d), capacity=cap, n_keys_uniform=cap, block_tables=bt,
                            bt_stride=pages, splits=att_splits, workspace=ws, stream=st)
    ms_f, _ = c.time_graph(fused, steps, warmup)
    ms_s, _ = c.time_graph(step, max(2, steps // 4), 2)

    # Cosmos3-style producer: the plain GEMM, then per-head q/k RMSNorm + RoPE
    # (positions 0..M-1) with the K/V append, one launch (emb_qkv_norm_rope_append)
    qg = torch.from_numpy(_bf16_bits(g.uniform(0.5, 1.5, d).astype(np.float32)).view(np.int16)).to(c.dev)
    kg = torch.from_numpy(_bf16_bits(g.uniform(0.5, 1.5, d).astype(np.float32)).view(np.int16)).to(c.dev)

    def norm_rope(st):
        emb.qkv_norm_rope_append(y, N, M, H, H, d, qo, slots, bt, cap, kp, vp, v16_pool=v16, q_gamma=qg,
                                 k_gamma=kg, eps=1e-6, rope_kind=1, rope_theta=1e6, first_position=0, stream=st)

    def norm_rope_many(st):
        for _ in range(k_launch):
            norm_rope(st)
    ms_nr, _ = c.time_graph(norm_rope_many, max(2, steps // 4), 2)

    def gemm_norm_rope(st):
        gemm(st)
        norm_rope(st)
    ms_gnr, _ = c.time_graph(gemm_norm_rope, steps, warmup)
    # LingBot producer: full-row q/k RMSNorm + Wan RoPE (per-token tables) +
    # append on the f32 QKV projection row (emb_qkv_rownorm_rope_append)
    qkv32 = torch.randn((M, N), dtype=torch.float32, device=c.dev)
    qkb = torch.randn(N, dtype=torch.float32, device=c.dev)
    qnw = torch.rand(H * d, dtype=torch.float32, device=c.dev) + 0.5
    knw = torch.rand(H * d, dtype=torch.float32, device=c.dev) + 0.5
    ang = torch.rand((M, d // 2), dtype=torch.float32, device=c.dev) * 100
    rc, rs = torch.cos(ang), torch.sin(ang)

    def rownorm_many(st):
        for _ in range(k_launch):
            emb.qkv_rownorm_rope_append(qkv32, N, M, H, d, qo, slots, bt, cap, kp, vp, v16_pool=v16, qkv_bias=qkb,
                                        q_weight=qnw, k_weight=knw, eps=1e-6, rope_cos=rc, rope_sin=rs, stream=st)
    ms_rn, _ = c.time_graph(rownorm_many, max(2, steps // 4), 2)
    rn_us = ms_rn * 1e3 / k_launch
    # read QKV f32, bias, weights, tables; write Q, K, V, V shadow (bf16)
    rn_bytes = M * N * 4 + N * 4 + 2 * H * d * 4 + 2 * M * (d // 2) * 4 + 4 * M * H * d * 2

    # LingBot post-attention projection with the gated residual in its epilogue
    # (emb_w8a16_gated_residual): f32 attention output [1560][3072] in, W8 O
    # weights, gate from a [1560][6*3072] timestep projection, in place on x
    No = H * d
    qwo = torch.from_numpy(g.integers(1, 256, (K // 16, 16 * No), dtype=np.uint8).view(np.int32)).to(c.dev)
    sco = torch.from_numpy(_bf16_bits(g.uniform(0.001, 0.01, No).astype(np.float32)).view(np.int16)).to(c.dev)
    tproj = torch.randn((M, 6 * No), dtype=torch.float32, device=c.dev)
    ssh = torch.randn(6 * No, dtype=torch.float32, device=c.dev)
    ob = torch.randn(No, dtype=torch.float32, device=c.dev)
    xres = torch.randn((M, No), dtype=torch.float32, device=c.dev)
    actx = out.view(M, No)
    xws = torch.empty(M * K, dtype=torch.int16, device=c.dev)

    def oproj_many(st):
        for _ in range(k_launch):
            emb.w8a16_gated_residual(actx, qwo, sco, M, K, No, xres, xres, bias=ob, gate=tproj[:, 2 * No:],
                                     ldg=6 * No, gate_bias=ssh[2 * No:3 * No], x_is_f32=True,
                                     x_bf16_workspace=xws, stream=st)
    ms_op, _ = c.time_graph(oproj_many, max(2, steps // 4), 2)
    op_us = ms_op * 1e3 / k_launch
    op_flops = 2.0 * M * K * No
    # the same O-projection on LingBot's dense resident weights (BF16, F32)
    wb16 = torch.randn((No, K), dtype=torch.float32, device=c.dev).mul_(K ** -0.5).to(torch.bfloat16)
    wf32 = wb16.float()
    dense_us = {}
    for name, wt, wty in (("bf16", wb16, emb.EMB_GGML_BF16), ("f32", wf32, emb.EMB_GGML_F32)):
        def dense_many(st, wt=wt, wty=wty):
            for _ in range(k_launch):
                emb.dense_gated_residual(actx, wt, wty, M, K, No, xres, residual=xres, bias=ob,
                                         gate=tproj[:, 2 * No:], ldg=6 * No, gate_bias=ssh[2 * No:3 * No],
                                         x_bf16_workspace=xws if wty == emb.EMB_GGML_BF16 else None, stream=st)
        ms_d, _ = c.time_graph(dense_many, max(2, steps // 4), 2)
        dense_us[name] = ms_d * 1e3 / k_launch
    del wb16, wf32
    nr_bytes = M * N * 2 + M * H * d * 2 + 2 * M * H * d * 2 + M * H * d * 2  # read QKV; write Q, K, V, V shadow
    gemm_bytes = M * K * 2 + K * N + N * 2 + M * N * 2
    return dict(norm_rope_append_us=ms_nr * 1e3 / k_launch,
                norm_rope_append_gbs=nr_bytes / (ms_nr * 1e-3 / k_launch) / 1e9,
                gemm_plus_norm_rope_append_us=ms_gnr * 1e3,
                gemm_us=gemm_us, gemm_us_single_launch=ms_g * 1e3, gemm_tflops=flops / (gemm_us * 1e-6) / 1e12,
                gemm_mfma_frac=flops / (gemm_us * 1e-6) / 1e12 / PEAK_BF16_TFLOPS, gemm_flops=flops,
                gemm_bytes=gemm_bytes, fused_qkv_append_us=ms_f * 1e3,
                fused_plus_attention_us_per_layer=ms_s * 1e3,
                lingbot_rownorm_rope_append_us=rn_us,
                lingbot_rownorm_rope_append_gbs=rn_bytes / (rn_us * 1e-6) / 1e9,
                oproj_gated_residual_us=op_us, oproj_gated_residual_tflops=op_flops / (op_us * 1e-6) / 1e12,
                oproj_gated_residual_mfma_frac=op_flops / (op_us * 1e-6) / 1e12 / PEAK_BF16_TFLOPS,
                oproj_dense_bf16_us=dense_us["bf16"],
                oproj_dense_bf16_tflops=op_flops / (dense_us["bf16"] * 1e-6) / 1e12,
                oproj_dense_bf16_mfma_frac=op_flops / (dense_us["bf16"] * 1e-6) / 1e12 / PEAK_BF16_TFLOPS,
                oproj_dense_f32_us=dense_us["f32"],
                oproj_dense_f32_tflops=op_flops / (dense_us["f32"] * 1e-6) / 1e12,
                oproj_dense_f32_mfma_frac=op_flops / (dense_us["f32"] * 1e-6) / 1e12 / PEAK_FP32_TFLOPS)


class MT64:
    """std::mt19937_64 (for drawing config-4 prefix lengths)."""

    def __init__(self, seed):
        self.mt = [0] * 312
        self.mt[0] = seed & (2 ** 64 - 1)
        for i in range(1, 312):
            self.mt[i] = (6364136223846793005 * (self.mt[i - 1] ^ (self.mt[i - 1] >> 62)) + i) & (2 ** 64 - 1)
        self.idx = 312

    def next(self):
        M = 2 ** 64 - 1
        if self.idx >= 312:
            for i in range(312):
                x = (self.mt[i] & 0xFFFFFFFF80000000) | (self.mt[(i + 1) % 312] & 0x7FFFFFFF)
                xa = x >> 1
                if x & 1:
                    xa ^= 0xB5026F5AA96619E9
                self.mt[i] = self.mt[(i + 156) % 312] ^ xa
            self.idx = 0
        x = self.mt[self.idx]
        self.idx += 1
        x ^= (x >> 29) & 0x5555555555555555
        x ^= (x << 17) & 0x71D67FFFEDA60000 & M
        x ^= (x << 37) & 0xFFF7EEE000000000 & M
        x ^= x >> 43
        return x & M


def cpu_baseline(target_s=10.0):
    """Oracle fp32 restatement of the reference ggml CPU op order (pi05.cpp:414-418) over
    config-1 layer problems on the host cores; whole denoise steps until ~target_s elapse."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    threads = _box_threads()
    n_pref, n_new, hq, hkv, d = 816, 51, 8, 1, 256
    nk = n_pref + n_new
    k = oracle.bf16_to_f32(oracle.normal_bf16(0xE3BD0000 + 1, nk * hkv * d))
    v = oracle.bf16_to_f32(oracle.normal_bf16(0xE3BD0000 + 2, nk * hkv * d))
    q = oracle.bf16_to_f32(oracle.normal_bf16(0xE3BD0000 + 10, n_new * hq * d))

    def step(th):
        used = 0
        for _ in range(18):
            _, used = oracle.cpu_attention_f32(q, k, v, n_new, nk, hq, hkv, d, 1 / 16, th)
        return used

    # the baseline computes the right thing: its output against the oracle on sampled rows
    got, _ = oracle.cpu_attention_f32(q, k, v, n_new, nk, hq, hkv, d, 1 / 16, threads)
    rows = np.arange(0, n_new, 7)  # query tokens
    want = oracle.gqa_attention(oracle.f32_to_bf16(q), oracle.f32_to_bf16(k), oracle.f32_to_bf16(v), n_new, nk, hq,
                                hkv, d, 1 / 16, rows=rows)
    err = float(np.max(np.abs(got[rows] - want[rows])))
    if err > 1e-4:
        raise RuntimeError(f"CPU baseline output differs from the oracle by {err}")
    res = {}
    for th in sorted({threads, min(8, threads)}):
        step(th)  # warm
        t0 = time.perf_counter()
        n = 0
        used = th
        while True:
            used = step(th)
            n += 1
            if time.perf_counter() - t0 >= target_s / 2 or n >= 200:
                break
        res[th] = ((time.perf_counter() - t0) / n * 1e6, n, used)
    th_main = max(res)
    us, n, used = res[th_main]
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": us,
        "unit": "us/denoise-step",
        "cores": used,
        "kind": "port",
        "sample": (f"{n} config-1 denoise steps (18 layers of 51x8 queries over 867 keys, d=256) "
                   f"with the oracle's fp32 ggml-order restatement on {used} OpenMP threads "
                   f"(nproc={os.cpu_count()}, the box's CPU share is 16 threads per GPU; {cpu_model}); "
                   f"reference ggml b9016 is not available offline; min(hw,8)={min(res)} threads: "
                   f"{res[min(res)][0]:.0f} us/step; output checked against the oracle on sampled rows "
                   f"(max abs {err:.1e})"),
    }


def _box_threads():
    """Threads for the CPU baselines: the GPU box's CPU share is 16 threads per
    GPU whatever nproc reports, so min(16, nproc)."""
    return max(1, min(16, os.cpu_count() or 1))


def cpu_baselines_other(cfgs, target_s=3.0):
    """CPU restatements, in the reference's op order, of configs 2, 3 and 5 on the
    host cores (each a bounded sample scaled to the full workload):
      cfg2: 18 prefix layers of bidirectional 816x8 over 816 keys attention
            (pi05.cpp:287-348: mul_mat -> soft_max_ext -> mul_mat, f32);
      cfg3: one LingBot layer: slot allocation (LingBotKVCache update_meta_only,
            lingbot_va.cpp:8793-8831, :8888-8902), scatter of the 1560-token chunk into the f32
            [capacity][24][128] cache, gather of the 14040-slot window
            (lingbot_flex_attn_cuda.cu:626-649, :875-898), dense attention of the
            chunk over the window (:651-720) -- the attention on a sample of
            query tokens, scaled;
      cfg5: the W8 fallback order (cosmos3_w8_marlin_cuda.cu:157-186, :222-300):
            dequantise the 3072x9216 int8 weight with its per-channel scale to f32,
            then an f32 GEMM of the 1560x3072 activations."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    from threadpoolctl import threadpool_limits

    th = _box_threads()
    out = {}

    def timed(fn, budget):
        fn()
        t0 = time.perf_counter()
        n = 0
        while True:
            fn()
            n += 1
            if time.perf_counter() - t0 >= budget or n >= 50:
                return (time.perf_counter() - t0) / n, n

    if "cfg2" in cfgs:
        n, hq, hkv, d, layers = 816, 8, 1, 256, 18
        k = oracle.bf16_to_f32(oracle.normal_bf16(0xE3BD0002 + 1, n * hkv * d))
        v = oracle.bf16_to_f32(oracle.normal_bf16(0xE3BD0002 + 2, n * hkv * d))
        q = oracle.bf16_to_f32(oracle.normal_bf16(0xE3BD0002 + 10, n * hq * d))
        sample_layers = 3
        sec, reps = timed(lambda: [oracle.cpu_attention_f32(q, k, v, n, n, hq, hkv, d, 1 / 16, th)
                                   for _ in range(sample_layers)], target_s)
        out["cfg2"] = {"value": sec / sample_layers * layers * 1e6, "unit": "us per 18-layer prefill attention",
                       "cores": th, "kind": "port",
                       "sample": f"{reps} x {sample_layers} layers of 816x8 queries over 816 keys (d 256), "
                                 f"fp32 oracle attention, scaled to 18 layers"}
    if "cfg3" in cfgs:
        cap, C_, H, d = 14040, 1560, 24, 128
        g = np.random.default_rng(3)
        cache_k = np.zeros((cap, H, d), np.float32)
        cache_v = np.zeros_like(cache_k)
        knew = g.standard_normal((C_, H, d), dtype=np.float32)
        vnew = g.standard_normal((C_, H, d), dtype=np.float32)
        sc = oracle.Cache(cap)
        for _ in range(cap // C_):  # fill the window (cache mode 2: update_meta_only, :8888-8902)
            sc.update_meta(C_, False)
        slots_state = {}

        def move():
            slots = sc.update_meta(C_, False)  # evicts the oldest chunk
            cache_k[slots] = knew
            cache_v[slots] = vnew
            valid = sc.collect_valid()
            slots_state["k"] = cache_k[valid]
            slots_state["v"] = cache_v[valid]
        sec_move, reps_m = timed(move, target_s / 3)
        kw, vw = slots_state["k"], slots_state["v"]
        if kw.shape[0] != cap:
            raise RuntimeError(f"cfg3 CPU baseline: window of {kw.shape[0]} slots, expected {cap}")
        qs = 26  # query tokens sampled of the 1560
        qq = g.standard_normal((qs, H, d), dtype=np.float32)
        sec_att, reps_a = timed(lambda: oracle.cpu_attention_f32(qq, kw, vw, qs, cap, H, H, d, d ** -0.5, th),
                                target_s * 2 / 3)
        per_layer = sec_move + sec_att * C_ / qs
        out["cfg3"] = {"value": per_layer * 1e6, "unit": "us per layer", "cores": th, "kind": "port",
                       "sample": (f"slot allocation + f32 scatter of 1560x24x128 + gather of the 14040-slot window "
                                  f"({sec_move * 1e6:.0f} us, {reps_m} runs, numpy single thread) + dense fp32 "
                                  f"attention of {qs} of the 1560 query tokens over 14040 keys ({reps_a} runs), "
                                  f"scaled by 1560/{qs}")}
    if "cfg5" in cfgs:
        M, K, N = 1560, 3072, 9216
        g = np.random.default_rng(5)
        w8 = g.integers(-127, 128, (K, N), dtype=np.int8)
        scale = (g.random(N, dtype=np.float32) * 0.02 + 0.001).astype(np.float32)
        x = oracle.bf16_to_f32(oracle.normal_bf16(0xE3BD0005, M * K)).reshape(M, K)

        def gemm():
            w = w8.astype(np.float32) * scale[None, :]  # dequantise to f32
            return x @ w
        with threadpool_limits(th):
            sec, reps = timed(gemm, target_s)
        out["cfg5"] = {"value": sec * 1e6, "unit": "us per 1560x3072->9216 projection", "cores": th,
                       "kind": "port",
                       "sample": f"{reps} full runs: numpy int8->f32 dequantisation with per-channel scales, "
                                 f"then an f32 BLAS GEMM on {th} threads"}
    return out


TRAFFIC_FILE = "paged_attn_cfg1_traffic.md"
COPY_CALIB_BYTES = 256 << 20


def _pmc_kib_per_dispatch(path: Path, kernel_sub: str, counter: str) -> float:
    """Mean per-dispatch value of one counter over the dispatches of kernels whose name contains kernel_sub."""
    import csv
    f = next(path.rglob("*counter_collection.csv"))
    vals = [float(r["Counter_Value"]) for r in csv.DictReader(open(f))
            if kernel_sub in r["Kernel_Name"] and r["Counter_Name"] == counter]
    if not vals:
        raise RuntimeError(f"{f}: no {counter} rows for {kernel_sub}")
    return sum(vals) / len(vals)


def traffic_summary(root: Path):
    """HBM bytes per launch of the config-1 attention kernel from FETCH_SIZE / WRITE_SIZE (KiB per
    dispatch), each scaled by what the same counter reads for a plain device copy of known size."""
    ksub = "attn_ks_kernel"  # the key-split kernel, the config-1 choice (bench --only cfg1_attn default)
    fa = _pmc_kib_per_dispatch(root / "pmc_fetch_attn", ksub, "FETCH_SIZE")
    wa = _pmc_kib_per_dispatch(root / "pmc_write_attn", ksub, "WRITE_SIZE")
    fc = _pmc_kib_per_dispatch(root / "pmc_fetch_copy", "copyBuffer", "FETCH_SIZE")
    wc = _pmc_kib_per_dispatch(root / "pmc_write_copy", "copyBuffer", "WRITE_SIZE")
    kf, kw = fc * 1024 / COPY_CALIB_BYTES, wc * 1024 / COPY_CALIB_BYTES
    traffic = fa * 1024 / kf + wa * 1024 / kw
    cmd = ("cd /tmp && timeout -s KILL 90 rocprofv3 --pmc {C} --output-format csv -d <dir>/pmc_{c}_{w} -o run "
           "-- python3 /root/repo/bench.py --only {W} --steps 20 --warmup 2")
    text = f"""# Config-1 attention kernel: HBM traffic per launch (rocprofv3 PMC)

Kernel: `attn_ks_kernel<256>` (the key-split kernel; config 1: 18 layers x 51 queries x 8 heads over
867 keys, head_dim 256, one launch, no split-K), launched by `bench.py --only cfg1_attn`.

| pass | command | mean per dispatch |
|---|---|---|
| FETCH_SIZE, attention | `{cmd.format(C="FETCH_SIZE", c="fetch", w="attn", W="cfg1_attn")}` | {fa:.1f} KiB |
| WRITE_SIZE, attention | `{cmd.format(C="WRITE_SIZE", c="write", w="attn", W="cfg1_attn")}` | {wa:.1f} KiB |
| FETCH_SIZE, copy | `{cmd.format(C="FETCH_SIZE", c="fetch", w="copy", W="copy_calib")}` | {fc:.1f} KiB |
| WRITE_SIZE, copy | `{cmd.format(C="WRITE_SIZE", c="write", w="copy", W="copy_calib")}` | {wc:.1f} KiB |

Calibration: the copy moves {COPY_CALIB_BYTES >> 20} MiB each way, so FETCH_SIZE reads {kf:.4f}x and
WRITE_SIZE {kw:.4f}x the true bytes.

traffic_bytes_per_launch: {traffic:.0f}

(Fetch {fa * 1024 / kf:.0f} B + write {wa * 1024 / kw:.0f} B after calibration; summary written by
`python bench.py --traffic-summary <dir>`.)
"""
    out = ROOT / "profiles" / TRAFFIC_FILE
    out.write_text(text)
    print(text)


def read_traffic(kernel_sub):
    """HBM bytes per launch from the committed PMC summary, or None when the
    summary does not cover kernel_sub (the kernel the headline ran)."""
    f = ROOT / "profiles" / TRAFFIC_FILE
    try:
        text = f.read_text()
        if kernel_sub not in text:
            return None
        for line in text.splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="cfg1,cfg2,cfg3,cfg4,cfg5")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="",
                    help="profiling targets: cfg1_attn (the headline kernel loop), cfg2_attn, cfg3_attn, cfg3_meta, cfg4_attn, cfg5_gemm, "
                         "copy_calib (a plain 256 MiB device copy, the PMC byte-counter calibration)")
    ap.add_argument("--traffic-summary", default="", metavar="DIR",
                    help="write profiles/" + TRAFFIC_FILE + " from the four rocprofv3 --pmc runs under DIR "
                         "(pmc_fetch_attn, pmc_write_attn, pmc_fetch_copy, pmc_write_copy) and exit")
    args = ap.parse_args()
    if args.traffic_summary:
        traffic_summary(Path(args.traffic_summary))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the attention step has no multi-GPU path here; it would shard by session or by kv head)",
              file=sys.stderr)
        sys.exit(2)

    c = Ctx()
    if args.only == "copy_calib":
        src = c.torch.ones(COPY_CALIB_BYTES // 4, dtype=c.torch.float32, device=c.dev)
        dst = c.torch.empty_like(src)
        for _ in range(args.warmup + args.steps):
            dst.copy_(src)
        c.torch.cuda.synchronize()
        log("profile loop done")
        return
    if args.only == "cfg1_attn":
        # EMB_KERNEL=key_split (default) or row_tiles (with EMB_SPLITS, default 3)
        P = PagedLayers(c, 0xE3BD0000, [816] * 18, 51, 8, 1, 256, n_steps=10)
        if os.environ.get("EMB_KERNEL", "key_split") == "key_split":
            P.set_splits(1, kernel=c.emb.EMB_ATTN_KEY_SPLIT)
        else:
            P.set_splits(int(os.environ.get("EMB_SPLITS", "3")))
        for i in range(args.warmup + args.steps):
            P.attend(i, c.stream, 1 / 16)
        c.torch.cuda.synchronize()
        log("profile loop done")
        return
    if args.only == "cfg2_attn":  # prefill attention, 18 layers, split 1
        P = PagedLayers(c, 0xE3BD0001, [0] * 18, 816, 8, 1, 256, n_steps=1)
        P.append(0, c.stream)  # the prefix K/V (a zero pool would take the exact recompute path)
        P.set_splits(1)
        for _ in range(args.warmup + args.steps):
            P.attend(0, c.stream, 1 / 16)
        c.torch.cuda.synchronize()
        log("profile loop done")
        return
    if args.only == "cfg4_attn":  # B = 64 sessions, one layer, unsplit (EMB_KERNEL as for cfg1_attn)
        g = MT64(0xE3BD0004)
        lens = [300 + g.next() % 901 for _ in range(64)]
        P = PagedLayers(c, 0xE3BD0004 + 64, lens, 51, 8, 1, 256, n_steps=2)
        P.set_splits(1, kernel=c.emb.EMB_ATTN_KEY_SPLIT
                     if os.environ.get("EMB_KERNEL", "key_split") == "key_split" else None)
        for _ in range(args.warmup + args.steps):
            P.attend(0, c.stream, 1 / 16)
        c.torch.cuda.synchronize()
        log("profile loop done")
        return
    if args.only == "cfg5_gemm":
        bench_cfg5(c, args.steps, args.warmup)
        log("profile loop done")
        return
    if args.only == "cfg3_meta":  # device slot metadata, 30 layer caches at the config-3 shape
        log("cfg3_meta " + json.dumps(bench_meta(c, args.steps)))
        log("profile loop done")
        return
    if args.only == "cfg3_attn":
        bench_cfg3(c, args.steps, args.warmup, n_layers=2, eager_only=True)
        log("profile loop done")
        return

    cfgs = set(args.configs.split(","))
    extra = {}
    log("cfg1 ...")
    r1 = bench_cfg1(c, args.steps, args.warmup)
    extra["cfg1"] = r1
    log("cfg1", json.dumps(r1))
    if "cfg4" in cfgs:
        log("cfg4 ...")
        extra["cfg4"] = bench_cfg4(c, args.steps, args.warmup)
        log("cfg4", json.dumps(extra["cfg4"]))
    if "cfg2" in cfgs:
        log("cfg2 ...")
        extra["cfg2"] = bench_cfg2(c, args.steps, args.warmup)
        log("cfg2", json.dumps(extra["cfg2"]))
    if "cfg3" in cfgs:
        log("cfg3 ...")
        extra["cfg3"] = bench_cfg3(c, args.steps, args.warmup)
        extra["cfg3"]["slot_metadata"] = bench_meta(c, args.steps)
        log("cfg3", json.dumps(extra["cfg3"]))
    if "cfg5" in cfgs:
        log("cfg5 ...")
        extra["cfg5"] = bench_cfg5(c, args.steps, args.warmup)
        log("cfg5", json.dumps(extra["cfg5"]))
        # the Cosmos3 language tower's causal GQA attention face (models/cosmos3.cpp:5032)
        extra["cosmos3_causal_gqa"] = bench_cosmos3_gqa(c, args.steps, args.warmup)
        log("cosmos3_causal_gqa", json.dumps(extra["cosmos3_causal_gqa"]))

    cpu = None
    if not args.no_cpu:
        log("cpu baseline ...")
        cpu = cpu_baseline()
        log("cpu", json.dumps(cpu))
        others = cpu_baselines_other(cfgs)
        for name, r in others.items():
            extra.setdefault(name, {})["cpu_baseline"] = r
        log("cpu (other configs)", json.dumps(others))

    kern_us = r1["attn_us_avg_in_graph"]
    achieved = r1["attn_bytes_per_launch"] / (kern_us * 1e-6) / 1e9
    line = {
        "metric": "us/denoise-step attention (pi0.5 action expert over cached prefix, 18 layers)",
        "value": r1["us_per_step"],
        "unit": "us/denoise-step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r1["us_per_step"] / 1e3,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) bf16 from std::mt19937_64(0xE3BD0000+cfg), random-permuted page pool",
        "config": {"workload": "BASELINE.json configs[0]: pi0.5 action-expert attention over an 816-token "
                               "cached prefix, 18 layers, 51 queries x 8 heads / 1 kv head, head_dim 256, "
                               "one denoise step = paged append of 51 new K/V + attention per layer, "
                               "layers batched in one launch; `steps` consecutive steps timed as one "
                               "HIP-graph replay",
                   "layers": 18, "prefix": 816, "queries": 51, "hq": 8, "hkv": 1, "head_dim": 256,
                   "page_tokens": 16, "kernel": r1["kernel"], "splits": r1["splits"]},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS, "traffic": read_traffic("attn_ks_kernel" if r1["kernel"] == "key_split"
                                                                        else "paged_attn_kernel"),
                     "kernel": ("attn_ks_kernel<256> (key-split workgroups, one launch)"
                                if r1["kernel"] == "key_split" else
                                "paged_attn_kernel<256,FULL,DMA>" +
                                (f" + attn_merge_kernel<256> (one split-K {r1['splits']} attention launch)"
                                 if r1["splits"] > 1 else "")),
                     "kernel_us": kern_us,
                     "bytes_per_launch": r1["attn_bytes_per_launch"]},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
