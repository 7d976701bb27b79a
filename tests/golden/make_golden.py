"""Writes the golden fixtures under tests/golden/ (numpy only; neither the
oracle nor the library is imported, so the fixtures are an independent check
of both).

    python tests/golden/make_golden.py

Fixtures (inputs and expected outputs):
  flex_smoke.npz      the reference's own flex-attention known answer
                      (kernels/lingbot/lingbot_flex_attn_cuda.cu:1033-1048:
                      closed-form q/k/v, the causal-window token mask, CSR
                      {0,1,3}/{0,0,1}, block size 4); expected output in
                      float64, computed over the token mask restricted to the
                      CSR's block pairs (:502-582).
  attention.npz       three seeded cases of softmax(q.k*scale + mask).v on
                      bf16-valued inputs, expected in float64: the pi0.5
                      action-expert shape (GQA 8/1, D 256, all keys visible,
                      models/pi05.cpp:405-418), chunk-causal MHA with a window
                      (models/lingbot_va.cpp:9336-9344 at chunk granularity),
                      and GQA 8/2 with an additive f32 mask (ggml
                      soft_max_ext / flash_attn_ext mask semantics).
  marlin_w8.npz       a W8A16 product on integer-exact operands: weights in
                      the Marlin byte layout (kernels/cosmos3/README.md:55-64,
                      cosmos3_w8_marlin_cuda.cu:50-58), scales in the Marlin
                      order (:78-88); every partial sum is exact in fp32, so
                      the bf16 result does not depend on summation order.
  slot_cache.json     a LingBot runtime-KV metadata sequence (modes 0/1/2,
                      restore, clear_pred, eviction, a failing request) with
                      the slots returned and the (id, mask, is_pred) state
                      after every operation, from a restatement of
                      models/lingbot_va.cpp:8784-8996.  Eviction ties (equal
                      ids) go in ascending slot order; with at most 16 used
                      slots, as here, that is also what libstdc++'s std::sort
                      (insertion sort below 16 elements) gives the reference.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent


def bf16_bits(f: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even."""
    u = np.ascontiguousarray(f, np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def bf16_val(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def attention64(q, k, v, hq, hkv, scale, allow=None, add=None):
    """softmax(q k^T scale + add) v per head in float64; q [nq,hq,d], k/v
    [nk,hkv,d]; query head h reads kv head h // (hq // hkv); a row with no
    visible key is 0."""
    G = hq // hkv
    nq, _, d = q.shape
    out = np.zeros((nq, hq, d))
    for h in range(hq):
        kh, vh = k[:, h // G].astype(np.float64), v[:, h // G].astype(np.float64)
        s = q[:, h].astype(np.float64) @ kh.T * scale
        if add is not None:
            s = s + add
        if allow is not None:
            s = np.where(allow, s, -np.inf)
        for i in range(nq):
            if not np.isfinite(s[i]).any():
                continue
            p = np.exp(s[i] - s[i].max())
            out[i, h] = p @ vh / p.sum()
    return out


def flex_smoke():
    S, H, D, BS = 8, 2, 8, 4
    i = np.arange(S * H * D, dtype=np.float32)
    q = (np.sin(i * np.float32(0.017)) * np.float32(0.2)).astype(np.float32)
    k = (np.cos(i * np.float32(0.019)) * np.float32(0.15)).astype(np.float32)
    v = (np.sin(i * np.float32(0.023)) * np.float32(0.3)).astype(np.float32)
    s, t = np.meshgrid(np.arange(S), np.arange(S), indexing="ij")
    mask = ((t <= s) & (s - t <= 4)).astype(np.uint8)
    row_ptr = np.array([0, 1, 3], np.int32)
    col_idx = np.array([0, 0, 1], np.int32)
    blocks = np.zeros((S // BS, S // BS), bool)
    for qb in range(S // BS):
        for e in range(row_ptr[qb], row_ptr[qb + 1]):
            blocks[qb, col_idx[e]] = True
    allow = mask.astype(bool) & blocks[s // BS, t // BS]
    scale = 1.0 / math.sqrt(D)
    out = attention64(q.reshape(S, H, D), k.reshape(S, H, D), v.reshape(S, H, D), H, H, scale, allow=allow)
    np.savez(OUT / "flex_smoke.npz", S=S, H=H, D=D, BS=BS, scale=scale, q=q, k=k, v=v, mask=mask,
             row_ptr=row_ptr, col_idx=col_idx, out=out.reshape(-1))


def attention_cases():
    rng = np.random.default_rng(0x60DE)
    arrays = {}

    def case(name, nq, nk, hq, hkv, d, scale, allow=None, add=None, **meta):
        qb = bf16_bits(rng.standard_normal((nq, hq, d)).astype(np.float32))
        kb = bf16_bits(rng.standard_normal((nk, hkv, d)).astype(np.float32))
        vb = bf16_bits(rng.standard_normal((nk, hkv, d)).astype(np.float32))
        out = attention64(bf16_val(qb), bf16_val(kb), bf16_val(vb), hq, hkv, scale, allow=allow, add=add)
        arrays.update({f"{name}_q": qb, f"{name}_k": kb, f"{name}_v": vb, f"{name}_out": out,
                       f"{name}_dims": np.array([nq, nk, hq, hkv, d], np.int64),
                       f"{name}_scale": np.float64(scale)})
        if add is not None:
            arrays[f"{name}_add"] = add.astype(np.float32)
        for key, val in meta.items():
            arrays[f"{name}_{key}"] = np.int64(val)

    # pi0.5 action expert: 38 cached prefix keys + 7 new, every key visible
    case("pi05", 7, 45, 8, 1, 256, 1 / 16)
    # chunk-causal MHA: queries at positions 16..39 (the last 24 of 40 keys),
    # chunk 8, window 2: key j visible to position p iff j/8 <= p/8 and p/8 - j/8 <= 2
    nq, nk, chunk, window = 24, 40, 8, 2
    p = (nk - nq) + np.arange(nq)[:, None]
    j = np.arange(nk)[None, :]
    allow = (j // chunk <= p // chunk) & (p // chunk - j // chunk <= window)
    case("chunk", nq, nk, 2, 2, 128, 1 / math.sqrt(128), allow=allow, chunk=chunk, window=window)
    # GQA 8/2 with an additive mask (a few keys hidden by -inf, the rest biased)
    add = rng.uniform(-2, 2, (5, 29)).astype(np.float32)
    add[rng.random((5, 29)) < 0.2] = -np.inf
    add[:, 0] = 0.0  # every row keeps a key
    case("addmask", 5, 29, 8, 2, 64, 0.125, add=add.astype(np.float64))
    np.savez(OUT / "attention.npz", **arrays)


INV_SCALE_PERM = [0, 1, 8, 9, 16, 17, 24, 25, 2, 3, 10, 11, 18, 19, 26, 27,
                  4, 5, 12, 13, 20, 21, 28, 29, 6, 7, 14, 15, 22, 23, 30, 31]


def marlin_w8():
    rng = np.random.default_rng(0x3A81)
    M, K, N = 20, 128, 128
    w = rng.integers(-127, 128, (K, N)).astype(np.int32)
    qbytes = np.zeros(K // 16 * 4 * N * 4, np.uint8)
    for kk in range(K):
        for n in range(N):
            row, col = kk // 16, (n // 64) * 256 + (n % 8) * 32 + ((n // 8) % 8) + ((kk % 8) // 2) * 8
            lane = (kk % 2) * 2 + ((kk // 8) % 2)
            qbytes[(row * (N * 4) + col) * 4 + lane] = w[kk, n] + 128
    qweight = qbytes.view(np.int32).reshape(K // 16, 4 * N)
    x = rng.integers(-2, 3, (M, K)).astype(np.float32)            # exact in bf16
    s = (2.0 ** -rng.integers(6, 10, N)).astype(np.float32)      # powers of two
    s_stored = np.zeros(N, np.uint16)
    for n in range(N):
        s_stored[(n // 32) * 32 + INV_SCALE_PERM[n % 32]] = bf16_bits(s[n:n + 1])[0]
    exact = (x.astype(np.float64) @ w.astype(np.float64)) * s.astype(np.float64)  # |x@w| < 2^24
    y = bf16_bits(exact.astype(np.float32))
    np.savez(OUT / "marlin_w8.npz", M=M, K=K, N=N, x=bf16_bits(x), qweight=qweight, s_stored=s_stored,
             w=w.astype(np.int8), y=y)


class RefCache:
    """models/lingbot_va.cpp:8740-8996, metadata only (ties in ascending slot)."""

    def __init__(self, total):
        self.total = total
        self.id = [-1] * total
        self.mask = [0] * total
        self.pred = [0] * total

    def next_id(self):
        return max([self.id[i] for i in range(self.total) if self.mask[i]], default=-1) + 1

    def allocate(self, n):
        free = [i for i in range(self.total) if not self.mask[i]]
        if len(free) < n:
            used = sorted((i for i in range(self.total) if self.mask[i]), key=lambda i: self.id[i])
            for slot in used[:n - len(free)]:
                self.mask[slot], self.id[slot] = 0, -1
                free.append(slot)
            free.sort()
        return free[:n] if len(free) >= n else None

    def update(self, n, pred):
        slots = self.allocate(n)
        if slots is None:
            return None
        new_id = self.next_id()
        for s in slots:
            self.mask[s], self.id[s], self.pred[s] = 1, new_id, int(pred)
        return slots

    def prepare_mode0(self, n):
        slots = self.allocate(n)
        if slots is None:
            return None, None
        new_id = self.next_id()
        for s in slots:
            self.id[s], self.pred[s] = new_id, 0
        return slots, [i for i in range(self.total) if self.mask[i] or i in slots]

    def restore(self, slots):
        for s in slots:
            self.mask[s] = 0

    def clear_pred(self):
        for i in range(self.total):
            if self.pred[i]:
                self.mask[i] = 0


def slot_cache():
    c = RefCache(14)
    ops = [("update", 4, 0), ("update", 3, 1), ("update", 4, 0), ("mode0", 3), ("restore",),
           ("update", 4, 0), ("clear_pred",), ("update", 5, 1), ("mode0", 6), ("restore",),
           ("update", 2, 0), ("update", 15, 0)]
    steps, last = [], None
    for op in ops:
        rec = {"op": op[0]}
        if op[0] == "update":
            rec.update(n=op[1], pred=op[2])
            rec["slots"] = c.update(op[1], op[2])
        elif op[0] == "mode0":
            rec["n"] = op[1]
            last, valid = c.prepare_mode0(op[1])
            rec.update(slots=last, valid=valid)
        elif op[0] == "restore":
            rec["slots"] = last
            c.restore(last)
        else:
            c.clear_pred()
        rec.update(id=list(c.id), mask=list(c.mask), is_pred=list(c.pred), next_id=c.next_id(),
                   valid_after=[i for i in range(c.total) if c.mask[i]])
        steps.append(rec)
    (OUT / "slot_cache.json").write_text(json.dumps({"capacity": c.total, "steps": steps}, indent=1) + "\n")


if __name__ == "__main__":
    flex_smoke()
    attention_cases()
    marlin_w8()
    slot_cache()
    for f in sorted(OUT.iterdir()):
        if f.suffix in (".npz", ".json"):
            print(f"{f.name}: {f.stat().st_size} bytes")
