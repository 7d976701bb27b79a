"""Python binding of the CPU oracle (oracle/build/libemb_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU baseline,
never by the product library.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "build" / "libemb_oracle.so"

i32p = C.POINTER(C.c_int32)
i64p = C.POINTER(C.c_int64)
u8p = C.POINTER(C.c_uint8)
i8p = C.POINTER(C.c_int8)
u16p = C.POINTER(C.c_uint16)
f32p = C.POINTER(C.c_float)
vp = C.c_void_p

_SIGS = {
    "orc_bf16_to_f32": (C.c_float, [C.c_uint16]),
    "orc_f32_to_bf16": (C.c_uint16, [C.c_float]),
    "orc_fill_normal_bf16": (None, [C.c_uint64, C.c_int64, u16p]),
    "orc_mt64_nth": (C.c_uint64, [C.c_uint64, C.c_int64]),
    "orc_cache_new": (vp, [C.c_int64, C.c_int]),
    "orc_cache_free": (None, [vp]),
    "orc_cache_used_count": (C.c_int64, [vp]),
    "orc_cache_pred_count": (C.c_int64, [vp]),
    "orc_cache_next_id": (C.c_int64, [vp]),
    "orc_cache_allocate": (C.c_int, [vp, C.c_int64, i64p]),
    "orc_cache_update_meta": (C.c_int, [vp, C.c_int64, C.c_int, i64p]),
    "orc_cache_prepare_mode0": (C.c_int, [vp, C.c_int64, i64p, i64p, i64p]),
    "orc_cache_restore": (None, [vp, i64p, C.c_int64]),
    "orc_cache_clear_pred": (None, [vp]),
    "orc_cache_collect_valid": (C.c_int64, [vp, i64p]),
    "orc_cache_id_ptr": (i64p, [vp]),
    "orc_cache_mask_ptr": (u8p, [vp]),
    "orc_cache_is_pred_ptr": (u8p, [vp]),
    "orc_lingbot_capacity": (C.c_int64, [C.c_int64] * 11),
    "orc_slot_update": (None, [u16p, u16p, u16p, u16p, i32p, C.c_int64, C.c_int64, C.c_int64,
                               C.c_int64]),
    "orc_slot_gather": (None, [u16p, u16p, i32p, u16p, u16p, C.c_int64, C.c_int64, C.c_int64,
                               C.c_int64]),
    "orc_paged_append": (None, [u16p, u16p, C.c_int64, C.c_int64, C.c_int64, C.c_int64, i32p,
                                i32p, C.c_int64, u16p, u16p]),
    "orc_paged_gather": (None, [u16p, u16p, i32p, C.c_int64, C.c_int64, C.c_int64, i32p,
                                C.c_int64, u16p, u16p]),
    "orc_flex_meta_build": (vp, [C.c_int64] * 16),
    "orc_flex_meta_free": (None, [vp]),
    "orc_flex_self_allowed": (C.c_int, [vp, C.c_int64, C.c_int64]),
    "orc_flex_cross_allowed": (C.c_int, [vp, C.c_int64, C.c_int64]),
    "orc_dense_block_table": (C.c_int64, [C.c_int64, C.c_int64, C.c_int64, i64p, i64p]),
    "orc_self_block_table": (C.c_int64, [vp, i64p, i64p]),
    "orc_cross_block_table": (C.c_int64, [vp, i64p, i64p]),
    "orc_self_token_mask": (None, [vp, u8p]),
    "orc_max_row_nnz": (C.c_int64, [i64p, C.c_int64]),
    "orc_dense_masked_attention": (None, [f32p, f32p, f32p, u8p, C.c_int64, C.c_int64, C.c_int64,
                                          f32p]),
    "orc_flex_attention": (None, [f32p, f32p, f32p, i32p, i32p, u8p, f32p, C.c_int64, C.c_int64,
                                  C.c_int64, C.c_int64, C.c_int64, C.c_float]),
    "orc_runtime_kv_attn": (None, [f32p, f32p, f32p, i32p, f32p, C.c_int64, C.c_int64, C.c_int64,
                                   C.c_int64, C.c_float, C.c_int]),
    "orc_head_norm_rope": (None, [u16p, C.c_int64, C.c_int64, C.c_int64, C.c_int64, u16p, C.c_float, C.c_int,
                                  C.c_float, C.c_int64, i32p, u16p, C.c_int64]),
    "orc_neox_rope_f32": (None, [f32p, C.c_int64, C.c_int64, C.c_int64, C.c_int64, i32p, C.c_int64, C.c_float,
                                 f32p, C.c_int64]),
    "orc_gqa_attention_bf16": (None, [u16p, u16p, u16p, C.c_int64, C.c_int64, C.c_int64,
                                      C.c_int64, C.c_int64, C.c_float, u8p, f32p, C.c_int64,
                                      C.c_int64, C.c_int64, i64p, C.c_int64, C.c_int, f32p]),
    "orc_cpu_attention_f32": (C.c_int, [f32p, f32p, f32p, C.c_int64, C.c_int64, C.c_int64,
                                        C.c_int64, C.c_int64, C.c_float, C.c_int, f32p]),
    "orc_marlin_dst_byte": (C.c_int64, [C.c_int64, C.c_int64, C.c_int64]),
    "orc_marlin_scale_index": (C.c_int64, [C.c_int64]),
    "orc_marlin_pack_w8": (None, [i8p, C.c_int64, C.c_int64, i32p]),
    "orc_marlin_unpack_w8": (C.c_int, [i32p, C.c_int64, C.c_int64, C.c_int64, C.c_int64]),
    "orc_marlin_pack_scales": (None, [u16p, C.c_int64, u16p]),
    "orc_w8a16_gemm": (None, [u16p, i32p, u16p, C.c_int64, C.c_int64, C.c_int64, i64p, C.c_int64,
                              C.c_int, u16p, f32p]),
}

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing; run `make -C oracle`")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def P(a: np.ndarray, t):
    return None if a is None else a.ctypes.data_as(t)


# ---------------- bf16 helpers (numpy, vectorised, RNE) ----------------
def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    return (u16.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(f, np.float32))
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def normal_bf16(seed: int, n: int) -> np.ndarray:
    out = np.zeros(n, np.uint16)
    lib().orc_fill_normal_bf16(seed, n, P(out, u16p))
    return out


# ---------------- slot cache ----------------
class Cache:
    def __init__(self, total, legacy=False):
        self.h = lib().orc_cache_new(total, int(legacy))
        self.total = total

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.orc_cache_free(self.h)
            self.h = None

    def used_count(self): return lib().orc_cache_used_count(self.h)
    def pred_count(self): return lib().orc_cache_pred_count(self.h)
    def next_id(self): return lib().orc_cache_next_id(self.h)

    def allocate(self, k):
        a = np.zeros(max(k, 1), np.int64)
        ok = lib().orc_cache_allocate(self.h, k, P(a, i64p))
        return a[:k] if ok else None

    def update_meta(self, k, pred):
        a = np.zeros(max(k, 1), np.int64)
        ok = lib().orc_cache_update_meta(self.h, k, int(pred), P(a, i64p))
        return a[:k] if ok else None

    def prepare_mode0(self, k):
        s = np.zeros(max(k, 1), np.int64)
        v = np.zeros(self.total, np.int64)
        n = C.c_int64(0)
        ok = lib().orc_cache_prepare_mode0(self.h, k, P(s, i64p), P(v, i64p), C.byref(n))
        return (s[:k], v[: n.value]) if ok else (None, None)

    def restore(self, slots):
        a = np.ascontiguousarray(slots, np.int64)
        lib().orc_cache_restore(self.h, P(a, i64p), len(a))

    def clear_pred(self): lib().orc_cache_clear_pred(self.h)

    def collect_valid(self):
        v = np.zeros(self.total, np.int64)
        n = lib().orc_cache_collect_valid(self.h, P(v, i64p))
        return v[:n]

    def state(self):
        L = lib()
        ids = np.ctypeslib.as_array(L.orc_cache_id_ptr(self.h), (self.total,)).copy()
        m = np.ctypeslib.as_array(L.orc_cache_mask_ptr(self.h), (self.total,)).copy()
        pr = np.ctypeslib.as_array(L.orc_cache_is_pred_ptr(self.h), (self.total,)).copy()
        return ids, m, pr


def lingbot_capacity(override_tokens=0, frame_chunk_size=4, action_per_frame=4, n_suffix=0,
                     attn_window=30, latent_h=8, latent_w=16, patch_t=1, patch_h=2, patch_w=2,
                     seq=0):
    return lib().orc_lingbot_capacity(override_tokens, frame_chunk_size, action_per_frame,
                                      n_suffix, attn_window, latent_h, latent_w, patch_t, patch_h,
                                      patch_w, seq)


# ---------------- movement ----------------
def slot_update(k, v, cache_k, cache_v, slots, heads, d, capacity):
    s = np.ascontiguousarray(slots, np.int32)
    lib().orc_slot_update(P(k, u16p), P(v, u16p), P(cache_k, u16p), P(cache_v, u16p), P(s, i32p),
                          len(s), heads, d, capacity)


def slot_gather(cache_k, cache_v, valid, heads, d, capacity, out_k, out_v):
    s = np.ascontiguousarray(valid, np.int32)
    lib().orc_slot_gather(P(cache_k, u16p), P(cache_v, u16p), P(s, i32p), P(out_k, u16p),
                          P(out_v, u16p), len(s), heads, d, capacity)


def paged_append(k, v, src_stride, slots, block_table, heads, d, capacity, k_pool, v_pool):
    s = np.ascontiguousarray(slots, np.int32)
    bt = None if block_table is None else np.ascontiguousarray(block_table, np.int32)
    lib().orc_paged_append(P(k, u16p), P(v, u16p), src_stride, len(s), heads, d, P(s, i32p),
                           P(bt, i32p), capacity, P(k_pool, u16p), P(v_pool, u16p))


def paged_gather(k_pool, v_pool, valid, block_table, heads, d, capacity, k_out, v_out):
    s = np.ascontiguousarray(valid, np.int32)
    bt = None if block_table is None else np.ascontiguousarray(block_table, np.int32)
    lib().orc_paged_gather(P(k_pool, u16p), P(v_pool, u16p), P(s, i32p), len(s), heads, d,
                           P(bt, i32p), capacity, P(k_out, u16p), P(v_out, u16p))


# ---------------- flex ----------------
class FlexMeta:
    def __init__(self, *args):
        self.h = lib().orc_flex_meta_build(*args)

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.orc_flex_meta_free(self.h)
            self.h = None


def self_block_table(meta, n, bs):
    qb = (n + bs - 1) // bs
    rp = np.zeros(qb + 1, np.int64)
    ci = np.zeros(max(qb * qb, 1), np.int64)
    nnz = lib().orc_self_block_table(meta.h, P(rp, i64p), P(ci, i64p))
    return rp, ci[:nnz]


def cross_block_table(meta, n, n_text, bs):
    qb, kb = (n + bs - 1) // bs, (n_text + bs - 1) // bs
    rp = np.zeros(qb + 1, np.int64)
    ci = np.zeros(max(qb * kb, 1), np.int64)
    nnz = lib().orc_cross_block_table(meta.h, P(rp, i64p), P(ci, i64p))
    return rp, ci[:nnz]


def dense_block_table(sq, sk, bs):
    qb, kb = (sq + bs - 1) // bs, (sk + bs - 1) // bs
    rp = np.zeros(qb + 1, np.int64)
    ci = np.zeros(max(qb * kb, 1), np.int64)
    nnz = lib().orc_dense_block_table(sq, sk, bs, P(rp, i64p), P(ci, i64p))
    return rp, ci[:nnz]


def self_token_mask(meta, n):
    m = np.zeros(n * n, np.uint8)
    lib().orc_self_token_mask(meta.h, P(m, u8p))
    return m.reshape(n, n)


# ---------------- attention ----------------
def dense_masked_attention(q, k, v, mask, seq, heads, d):
    out = np.zeros(seq * heads * d, np.float32)
    lib().orc_dense_masked_attention(P(q, f32p), P(k, f32p), P(v, f32p), P(mask, u8p), seq, heads,
                                     d, P(out, f32p))
    return out


def flex_attention(q, k, v, row_ptr, col_idx, token_mask, sq, sk, heads, d, bs, scale):
    out = np.zeros(sq * heads * d, np.float32)
    rp = np.ascontiguousarray(row_ptr, np.int32)
    ci = np.ascontiguousarray(col_idx, np.int32)
    tm = None if token_mask is None else np.ascontiguousarray(token_mask, np.uint8)
    lib().orc_flex_attention(P(q, f32p), P(k, f32p), P(v, f32p), P(rp, i32p), P(ci, i32p),
                             P(tm, u8p), P(out, f32p), sq, sk, heads, d, bs, scale)
    return out


def runtime_kv_attn(q, cache_k, cache_v, valid, sq, heads, d, scale, online_quirk=True):
    vs = np.ascontiguousarray(valid, np.int32)
    out = np.zeros(sq * heads * d, np.float32)
    lib().orc_runtime_kv_attn(P(q, f32p), P(cache_k, f32p), P(cache_v, f32p), P(vs, i32p),
                              P(out, f32p), sq, len(vs), heads, d, scale, int(online_quirk))
    return out


def gqa_attention(q, k, v, n_q, n_k, hq, hkv, d, scale, allow=None, add=None, chunk=0,
                  window=-1, q_pos0=None, rows=None, threads=0):
    """q/k/v: uint16 bf16 bits ([n_q][hq][d], [n_k][hkv][d]); returns f32 [n_q][hq][d]
    (rows not evaluated are zero)."""
    out = np.zeros(n_q * hq * d, np.float32)
    if q_pos0 is None:
        q_pos0 = n_k - n_q
    r = None if rows is None else np.ascontiguousarray(rows, np.int64)
    al = None if allow is None else np.ascontiguousarray(allow, np.uint8)
    ad = None if add is None else np.ascontiguousarray(add, np.float32)
    lib().orc_gqa_attention_bf16(P(q, u16p), P(k, u16p), P(v, u16p), n_q, n_k, hq, hkv, d, scale,
                                 P(al, u8p), P(ad, f32p), chunk, window, q_pos0, P(r, i64p),
                                 0 if r is None else len(r), threads, P(out, f32p))
    return out.reshape(n_q, hq, d)


def cpu_attention_f32(q, k, v, n_q, n_k, hq, hkv, d, scale, threads=0):
    """CPU baseline: f32 arrays in, (out f32 [n_q][hq][d], threads used) back."""
    out = np.zeros(n_q * hq * d, np.float32)
    used = lib().orc_cpu_attention_f32(P(np.ascontiguousarray(q, np.float32), f32p),
                                       P(np.ascontiguousarray(k, np.float32), f32p),
                                       P(np.ascontiguousarray(v, np.float32), f32p), n_q, n_k, hq,
                                       hkv, d, scale, threads, P(out, f32p))
    return out.reshape(n_q, hq, d), used


# ---------------- W8 ----------------
def marlin_pack_w8(w: np.ndarray) -> np.ndarray:
    K, N = w.shape
    q = np.zeros((K // 16, 4 * N), np.int32)
    lib().orc_marlin_pack_w8(P(np.ascontiguousarray(w, np.int8), i8p), K, N, P(q, i32p))
    return q


def marlin_unpack_w8(q, K, N, k, n):
    return lib().orc_marlin_unpack_w8(P(q, i32p), K, N, k, n)


def marlin_pack_scales(s: np.ndarray) -> np.ndarray:
    out = np.zeros_like(s, dtype=np.uint16)
    lib().orc_marlin_pack_scales(P(np.ascontiguousarray(s, np.uint16), u16p), len(s),
                                 P(out, u16p))
    return out


def w8a16_gemm(x, qweight, s_stored, M, K, N, rows=None, threads=0):
    r = None if rows is None else np.ascontiguousarray(rows, np.int64)
    nr = M if r is None else len(r)
    yb = np.zeros(nr * N, np.uint16)
    yf = np.zeros(nr * N, np.float32)
    lib().orc_w8a16_gemm(P(x, u16p), P(qweight, i32p), P(s_stored, u16p), M, K, N, P(r, i64p),
                         nr, threads, P(yb, u16p), P(yf, f32p))
    return yb.reshape(nr, N), yf.reshape(nr, N)


def gated_residual(y, residual, bias=None, gate=None, gate_bias=None, round_bf16=False):
    """Epilogue of the projection after attention in the LingBot post graph
    (models/lingbot_va.cpp:11693-11695, lin() :1178-1180, bf16 boundary
    :11676-11678): a1 = y + bias; x = residual + a1 * (gate + gate_bias), every
    node an f32 operation of its own.  y is the projection's f32 value ([M][N],
    e.g. the second result of w8a16_gemm); gate [M][N] or None; residual None
    leaves x = a1 * (gate + gate_bias) (or a1)."""
    f = np.float32
    a = np.asarray(y, f)
    if bias is not None:
        a = (a + np.asarray(bias, f)[None, :]).astype(f)
    if gate is not None:
        g = np.asarray(gate, f)
        if gate_bias is not None:
            g = (g + np.asarray(gate_bias, f)[None, :]).astype(f)
        a = (a * g).astype(f)
    out = a if residual is None else (np.asarray(residual, f) + a).astype(f)
    if round_bf16:
        out = bf16_to_f32(f32_to_bf16(out))
    return out


def dense_linear(x, w, bf16_weights, bias=None, rows=None):
    """lin(w, x) = ggml_add(ggml_mul_mat(w, x), bias) of the LingBot graph
    (models/lingbot_va.cpp:1178-1180) for its dense resident weight types
    (:1808-1851), in the numerics of ggml's CUDA mul_mat (ggml b9016, a
    dependency not vendored in the reference: ggml_cuda_op_mul_mat_cublas).
      bf16_weights: x rounded to bf16 (RNE), times the bf16 weights with an
        fp32 accumulator (cublasGemmEx, CUBLAS_COMPUTE_32F) into a bf16
        result, widened to f32;
      otherwise: an f32 product (cublasSgemm).
    The accumulation order of cuBLAS is unspecified; the exact sum stands for
    it, taken in float64 (bf16 and f32 products are exact there), rounded to
    f32, then (bf16 weights) to bf16.  x f32 [M][K] (or bf16 bits with
    bf16 weights), w [N][K] (ggml row order: ne0 = K) as f32 or bf16 bits;
    bias f32 [N] added as its own f32 node.  rows: the x rows to evaluate."""
    f = np.float32
    x = np.asarray(x)
    if rows is not None:
        x = x[np.asarray(rows)]
    if bf16_weights:
        xb = bf16_to_f32(x) if x.dtype == np.uint16 else bf16_to_f32(f32_to_bf16(np.asarray(x, f)))
        wf = bf16_to_f32(w) if np.asarray(w).dtype == np.uint16 else np.asarray(w, f)
    else:
        xb, wf = np.asarray(x, f), np.asarray(w, f)
    y = (xb.astype(np.float64) @ wf.astype(np.float64).T).astype(f)
    if bf16_weights:
        y = bf16_to_f32(f32_to_bf16(y))
    if bias is not None:
        y = (y + np.asarray(bias, f)[None, :]).astype(f)
    return y


# ---------------- LingBot full-row q/k RMSNorm + Wan RoPE ----------------
def lingbot_row_norm(x, weight, eps=1e-6):
    """ggml_rms_norm over the whole row then * weight (models/lingbot_va.cpp:
    1233-1234): scale = 1 / sqrt(sum(x^2) / n + eps) in f32 (the sum taken in
    float64), y = (x * scale) * weight, f32 [tokens][n]."""
    f = np.float32
    x = np.asarray(x, f)
    ss = (x.astype(np.float64) ** 2).sum(axis=1)
    scale = (f(1.0) / np.sqrt((ss.astype(f) / f(x.shape[1]) + f(eps)).astype(f))).astype(f)
    return ((x * scale[:, None]).astype(f) * np.asarray(weight, f)[None, :]).astype(f)


def wan_rope(x, heads, d, cos, sin):
    """apply_wan_rope_shape (models/lingbot_va.cpp:1190-1206): x f32
    [tokens][heads*d]; in each head pair (2i, 2i+1) -> (x0 c - x1 s, x1 c + x0 s),
    c = cos[token][i], s = sin[token][i], every product and sum an f32 op."""
    f = np.float32
    t = x.shape[0]
    xp = np.asarray(x, f).reshape(t, heads, d // 2, 2)
    c = np.asarray(cos, f).reshape(t, 1, d // 2)
    s = np.asarray(sin, f).reshape(t, 1, d // 2)
    x0, x1 = xp[..., 0], xp[..., 1]
    y0 = ((x0 * c).astype(f) - (x1 * s).astype(f)).astype(f)
    y1 = ((x1 * c).astype(f) + (x0 * s).astype(f)).astype(f)
    return np.stack([y0, y1], axis=-1).reshape(t, heads * d)


def lingbot_qkv(qkv, heads, d, bias=None, q_w=None, k_w=None, eps=1e-6, cos=None, sin=None):
    """build_attention_shape's q/k/v (models/lingbot_va.cpp:1219-1250) from an
    f32 projection row [tokens][>= 3*heads*d]: (q, k, v) f32 [tokens][heads*d]."""
    f = np.float32
    hid = heads * d
    x = np.asarray(qkv, f)[:, :3 * hid]
    if bias is not None:
        x = (x + np.asarray(bias, f)[None, :]).astype(f)
    q, k, v = x[:, :hid], x[:, hid:2 * hid], x[:, 2 * hid:]
    if q_w is not None:
        q = lingbot_row_norm(q, q_w, eps)
    if k_w is not None:
        k = lingbot_row_norm(k, k_w, eps)
    if cos is not None:
        q, k = wan_rope(q, heads, d, cos, sin), wan_rope(k, heads, d, cos, sin)
    return q, k, v


# ---------------- Qwen per-head q/k RMSNorm + RoPE ----------------
def head_norm_rope(x, tokens, heads, d, gamma=None, eps=1e-6, rope_kind=0, theta=1e6, first_pos=0,
                   pos_ids=None, ld=None):
    """bf16 bits x [tokens][ld] (heads*d columns used) -> bf16 bits [tokens][heads][d]."""
    x = np.ascontiguousarray(x, np.uint16)
    ld = ld or heads * d
    out = np.zeros(tokens * heads * d, np.uint16)
    g = None if gamma is None else np.ascontiguousarray(gamma, np.uint16)
    pid = None if pos_ids is None else np.ascontiguousarray(pos_ids, np.int32)
    lib().orc_head_norm_rope(P(x, u16p), ld, tokens, heads, d, P(g, u16p), C.c_float(eps), rope_kind,
                             C.c_float(theta), first_pos, P(pid, i32p), P(out, u16p), heads * d)
    return out.reshape(tokens, heads, d)


def neox_rope(x, tokens, heads, d, positions=None, first_pos=0, freq_base=10000.0, ld=None):
    """pi0.5 NEOX RoPE (orc_neox_rope_f32): f32 x [tokens][ld] (heads*d columns
    used) -> f32 [tokens][heads][d]."""
    x = np.ascontiguousarray(x, np.float32)
    ld = ld or heads * d
    out = np.zeros(tokens * heads * d, np.float32)
    pos = None if positions is None else np.ascontiguousarray(positions, np.int32)
    lib().orc_neox_rope_f32(P(x, f32p), ld, tokens, heads, d, P(pos, i32p), first_pos, C.c_float(freq_base),
                            P(out, f32p), heads * d)
    return out.reshape(tokens, heads, d)


# ---------------- call-site masks (restated step by step, pure Python) ----------------
NEG_INF = float("-inf")


def hy_patch_groups(modality_mask):
    """make_visual_patch_groups (models/hy_vla.cpp:1251-1277): list of groups
    (lists of token indices), following the reference's scan."""
    groups, cur, i, n = [], [], 0, len(modality_mask)
    while i < n:
        if modality_mask[i] == 0:
            z0 = i
            while i < n and modality_mask[i] == 0:
                i += 1
            if i - z0 >= 2 and cur:
                groups.append(cur)
                cur = []
            continue
        while i < n and modality_mask[i] != 0:
            cur.append(i)
            i += 1
    if cur:
        groups.append(cur)
    return groups


def hy_prefix_mask(n, groups=None):
    """make_prefix_mask (models/hy_vla.cpp:1279-1306): f32 additive [n][n] built
    in the reference's three passes (causal; every patch pair -inf; each
    group's pairs 0)."""
    m = np.array([[0.0 if c <= r else NEG_INF for c in range(n)] for r in range(n)], np.float32)
    if groups is not None:
        every = [t for g in groups for t in g]
        for r in every:
            for c in every:
                m[r, c] = NEG_INF
        for g in groups:
            for r in g:
                for c in g:
                    m[r, c] = 0.0
    return m


def hy_suffix_mask(n_pref, n_suf):
    """full_mask of the routed predict path (models/hy_vla.cpp:2831-2843)."""
    n_total = n_pref + n_suf
    m = np.zeros((n_suf, n_total), np.float32)
    for r in range(n_suf):
        for c in range(n_total):
            allowed = c < n_pref
            if not allowed:
                s = c - n_pref
                allowed = (s == 0) if r == 0 else True
            m[r, c] = 0.0 if allowed else NEG_INF
    return m


def groot_layer_mask_kind(layer, attend_text_every_n_blocks=2):
    """models/groot_n1.cpp:656-661: 0 self-attention, 1 text mask, 2 image mask."""
    if layer % 2 == 1:
        return 0
    return 1 if layer % (2 * attend_text_every_n_blocks) == 0 else 2


def groot_cross_masks(attention_mask, image_flags, n_q):
    """models/groot_n1.cpp:708-716: (text, image) f32 additive [n_q][n_keys]."""
    nk = len(attention_mask)
    text = np.zeros((n_q, nk), np.float32)
    image = np.zeros((n_q, nk), np.float32)
    for q in range(n_q):
        for k in range(nk):
            valid = attention_mask[k] != 0
            is_image = image_flags[k] != 0
            text[q, k] = 0.0 if valid and not is_image else NEG_INF
            image[q, k] = 0.0 if valid and is_image else NEG_INF
    return text, image


def smolvla_masks(prefix_valid, n_suf):
    """models/smolvla.cpp:696-725: (prefix [n][n], full [n_suf][n+n_suf],
    cross [n_suf][n]) f32 additive."""
    n = len(prefix_valid)
    pm = np.zeros((n, n), np.float32)
    for q in range(n):
        for k in range(n):
            if not prefix_valid[k] or (q < n - 1 and k == n - 1):
                pm[q, k] = NEG_INF
    fm = np.zeros((n_suf, n + n_suf), np.float32)
    cm = np.zeros((n_suf, n), np.float32)
    for q in range(n_suf):
        for k in range(n):
            if not prefix_valid[k]:
                fm[q, k] = NEG_INF
                cm[q, k] = NEG_INF
        for k in range(q + 1, n_suf):
            fm[q, n + k] = NEG_INF
    return pm, fm, cm


def smolvla_positions(prefix_valid, n_suf):
    """models/smolvla.cpp:680-688: (prefix, suffix, cross) int32 positions."""
    pp, pos = [], -1
    for v in prefix_valid:
        if v:
            pos += 1
        pp.append(max(pos, 0))
    off = pos + 1
    return (np.array(pp, np.int32), np.array([off + i for i in range(n_suf)], np.int32),
            np.arange(n_suf, dtype=np.int32))


def pbf16_attention(q, k, v, n_q, n_k, hq, hkv, d, scale, add=None, round_p=True):
    """SmolVLA's attention numerics (models/smolvla.cpp:255-266): scores
    kq = K.Q as f32 (computed in float64, rounded to f32), x = kq * scale +
    mask (f32), softmax with the row max (f32 exp), p = e * (1/sum) rounded to
    bf16 (round_p), out = sum_j p_j v_j (float64).  q/k/v: bf16 bits
    [n_q][hq][d] / [n_k][hkv][d]; add: f32 [n_q][n_k] or None.  A row with no
    visible key is 0."""
    qf = bf16_to_f32(np.asarray(q, np.uint16)).astype(np.float64).reshape(n_q, hq, d)
    kf = bf16_to_f32(np.asarray(k, np.uint16)).astype(np.float64).reshape(n_k, hkv, d)
    vf = bf16_to_f32(np.asarray(v, np.uint16)).astype(np.float64).reshape(n_k, hkv, d)
    G = hq // hkv
    out = np.zeros((n_q, hq, d))
    for h in range(hq):
        kk, vv = kf[:, h // G], vf[:, h // G]
        kq = (qf[:, h] @ kk.T).astype(np.float32)
        x = (kq * np.float32(scale)).astype(np.float32)
        if add is not None:
            x = (x + np.asarray(add, np.float32)).astype(np.float32)
        m = np.max(x, axis=1, keepdims=True)
        ok = np.isfinite(m[:, 0])
        with np.errstate(invalid="ignore", over="ignore"):
            e = np.exp((x - np.where(np.isfinite(m), m, 0)).astype(np.float64)).astype(np.float32)
        e[~ok] = 0
        ssum = e.astype(np.float64).sum(axis=1, keepdims=True).astype(np.float32)
        inv = np.where(ssum > 0, np.float32(1) / np.where(ssum > 0, ssum, 1), 0).astype(np.float32)
        p = (e * inv).astype(np.float32)
        if round_p:
            p = bf16_to_f32(f32_to_bf16(p))
        out[:, h] = p.astype(np.float64) @ vv
    return out
