"""ctypes binding of libemb_kv.so (the C ABI in include/emb_kv.h).

Device buffers are passed as raw pointers; torch tensors are accepted
wherever a pointer is expected (their data_ptr() is used), which is how the
tests and bench.py hold device memory.  Loading fails loudly when the library
has not been built: there is no fallback implementation.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libemb_kv.so"

_lib = None

EMB_MASK_FULL, EMB_MASK_CHUNK, EMB_MASK_TOKEN, EMB_MASK_ADD, EMB_MASK_BLOCKMAP = range(5)
EMB_ATTN_AUTO, EMB_ATTN_ROW_TILES, EMB_ATTN_KEY_SPLIT = range(3)
EMB_ERR_ARG, EMB_ERR_LAUNCH, EMB_ERR_CAPACITY, EMB_ERR_UNSUPPORTED = -1, -2, -3, -4

i32p = C.POINTER(C.c_int32)
i64p = C.POINTER(C.c_int64)
u8p = C.POINTER(C.c_uint8)
u16p = C.POINTER(C.c_uint16)
vp = C.c_void_p


class AttnArgs(C.Structure):
    _fields_ = [
        ("q", vp), ("q_is_f32", C.c_int32), ("q_stride", C.c_int64),
        ("out", vp), ("out_stride", C.c_int64),
        ("cu_q", vp), ("n_keys", vp), ("q_pos0", vp),
        ("k_pool", vp), ("v_pool", vp), ("v16_pool", vp),
        ("block_tables", vp), ("bt_stride", C.c_int32),
        ("valid_slots", vp), ("valid_stride", C.c_int32),
        ("capacity", C.c_int32), ("batch", C.c_int32), ("hq", C.c_int32), ("hkv", C.c_int32),
        ("head_dim", C.c_int32), ("max_q", C.c_int32), ("scale", C.c_float),
        ("mask_kind", C.c_int32), ("chunk", C.c_int32), ("window", C.c_int32),
        ("mask", vp), ("mask_q_stride", C.c_int64), ("mask_batch_stride", C.c_int64),
        ("block_map", vp), ("block_size", C.c_int32), ("block_map_cols", C.c_int32),
        ("block_map_batch_stride", C.c_int64),
        ("splits", C.c_int32), ("workspace", vp),
        ("n_keys_uniform", C.c_int32),
        ("out_bf16_round", C.c_int32),
        ("p_bf16", C.c_int32),
        ("split_keys", C.c_int32),
        ("kernel", C.c_int32),
    ]


EMB_GGML_F32, EMB_GGML_F16, EMB_GGML_BF16 = 0, 1, 30


class DevCacheDesc(C.Structure):
    _fields_ = [("id", vp), ("mask", vp), ("is_pred", vp), ("capacity", C.c_int32),
                ("legacy_clear_pred", C.c_int32)]


class GgmlTensor(C.Structure):
    _fields_ = [("type", C.c_int32), ("ne", C.c_int64 * 4), ("nb", C.c_size_t * 4), ("data", vp)]


_SIGS = {
    "emb_last_error": (C.c_char_p, []),
    "emb_version": (C.c_char_p, []),
    "emb_slot_cache_create": (vp, [C.c_int64, C.c_int]),
    "emb_slot_cache_destroy": (None, [vp]),
    "emb_slot_cache_capacity": (C.c_int64, [vp]),
    "emb_slot_cache_used_count": (C.c_int64, [vp]),
    "emb_slot_cache_pred_count": (C.c_int64, [vp]),
    "emb_slot_cache_next_id": (C.c_int64, [vp]),
    "emb_slot_cache_allocate": (C.c_int, [vp, C.c_int64, i64p]),
    "emb_slot_cache_update_meta": (C.c_int, [vp, C.c_int64, C.c_int, i64p]),
    "emb_slot_cache_prepare_mode0": (C.c_int, [vp, C.c_int64, i64p, i64p, i64p]),
    "emb_slot_cache_restore": (None, [vp, i64p, C.c_int64]),
    "emb_slot_cache_clear_pred": (None, [vp]),
    "emb_dev_cache_init": (C.c_int, [C.POINTER(DevCacheDesc), vp]),
    "emb_dev_cache_update": (C.c_int, [C.POINTER(DevCacheDesc), C.c_int32, C.c_int32, vp, vp, vp, vp, vp]),
    "emb_dev_cache_restore": (C.c_int, [C.POINTER(DevCacheDesc), vp, C.c_int32, vp]),
    "emb_dev_cache_clear_pred": (C.c_int, [C.POINTER(DevCacheDesc), vp]),
    "emb_slot_cache_collect_valid": (C.c_int64, [vp, i64p]),
    "emb_slot_cache_export": (C.c_int, [vp, i64p, u8p, u8p]),
    "emb_page_pool_create": (vp, [C.c_int32, C.c_uint64]),
    "emb_page_pool_destroy": (None, [vp]),
    "emb_page_pool_free_count": (C.c_int32, [vp]),
    "emb_slot_cache_bind_pool": (C.c_int, [vp, vp]),
    "emb_slot_cache_map_range": (C.c_int, [vp, C.c_int64]),
    "emb_slot_cache_block_table": (C.c_int, [vp, i32p, C.c_int64]),
    "emb_slot_cache_release_pages": (C.c_int, [vp]),
    "emb_lingbot_kv_capacity": (C.c_int64, [C.c_int64] * 11),
    "emb_flex_meta_build": (vp, [C.c_int64] * 16),
    "emb_flex_meta_destroy": (None, [vp]),
    "emb_flex_meta_len": (C.c_int64, [vp]),
    "emb_flex_meta_ids": (C.c_int, [vp, i64p, i64p, i64p]),
    "emb_flex_self_allowed": (C.c_int, [vp, C.c_int64, C.c_int64]),
    "emb_flex_cross_allowed": (C.c_int, [vp, C.c_int64, C.c_int64]),
    "emb_dense_block_table": (C.c_int64, [C.c_int64, C.c_int64, C.c_int64, i32p, i32p]),
    "emb_self_block_table": (C.c_int64, [vp, i32p, i32p]),
    "emb_cross_block_table": (C.c_int64, [vp, i32p, i32p]),
    "emb_self_token_mask": (C.c_int, [vp, u8p]),
    "emb_kv_append": (C.c_int, [vp, vp, C.c_int64, C.c_int32, vp, vp, C.c_int32, vp, vp, vp,
                                C.c_int32, C.c_int32, vp]),
    "emb_qkv_rownorm_rope_append": (C.c_int, [vp, C.c_int64, C.c_int32, C.c_int32, C.c_int32, vp, vp, vp,
                                              C.c_float, vp, vp, vp, C.c_int64, vp, vp, C.c_int32, vp, vp,
                                              vp, vp]),
    "emb_hy_patch_groups": (C.c_int32, [vp, C.c_int32, vp]),
    "emb_hy_prefix_mask": (C.c_int, [C.c_int64, vp, vp, vp]),
    "emb_hy_suffix_mask": (C.c_int, [C.c_int64, C.c_int64, vp, vp]),
    "emb_groot_layer_mask_kind": (C.c_int, [C.c_int32, C.c_int32]),
    "emb_groot_cross_masks": (C.c_int, [vp, vp, C.c_int64, C.c_int64, vp, vp]),
    "emb_smolvla_masks": (C.c_int, [vp, C.c_int64, C.c_int64, vp, vp, vp]),
    "emb_smolvla_positions": (C.c_int, [vp, C.c_int64, C.c_int64, vp, vp, vp]),
    "emb_qkv_neox_rope_append": (C.c_int, [vp, C.c_int64, vp, C.c_int64, vp, C.c_int64, C.c_int32, C.c_int32,
                                           C.c_int32, C.c_int32, vp, C.c_int32, C.c_float, vp, C.c_int32,
                                           C.c_int64, vp, vp, C.c_int32, vp, vp, vp, vp]),
    "emb_qkv_norm_rope_append": (C.c_int, [vp, C.c_int64, C.c_int32, C.c_int32, C.c_int32, C.c_int32, vp, vp,
                                           C.c_float, C.c_int32, C.c_float, C.c_int32, vp, vp, C.c_int64, vp,
                                           vp, C.c_int32, vp, vp, vp, vp]),
    "emb_kv_gather": (C.c_int, [vp, vp, vp, C.c_int32, vp, C.c_int32, vp, vp, C.c_int32,
                                C.c_int32, vp]),
    "emb_attn_workspace_bytes": (C.c_size_t, [C.c_int32] * 6),
    "emb_paged_attention": (C.c_int, [C.POINTER(AttnArgs), vp]),
    "emb_paged_attention_noalloc": (C.c_int, [C.POINTER(AttnArgs), vp]),
    "lingbot_runtime_kv_update_f32": (C.c_int, [vp, vp, vp, vp, vp, C.c_int, C.c_int, C.c_int,
                                                C.c_int, vp]),
    "lingbot_runtime_kv_gather_f32": (C.c_int, [vp, vp, vp, vp, vp, C.c_int, C.c_int, C.c_int,
                                                C.c_int, vp]),
    "lingbot_runtime_kv_attn_f32": (C.c_int, [vp, vp, vp, vp, vp, C.c_int, C.c_int, C.c_int,
                                              C.c_int, C.c_float, vp]),
    "lingbot_runtime_kv_attn_online_f32": (C.c_int, [vp, vp, vp, vp, vp, C.c_int, C.c_int,
                                                     C.c_int, C.c_int, C.c_float, vp]),
    "lingbot_runtime_kv_attn_warp_f32": (C.c_int, [vp, vp, vp, vp, vp, C.c_int, C.c_int,
                                                   C.c_int, C.c_int, C.c_float, vp]),
    "lingbot_runtime_kv_attn_cublas_f32": (C.c_int, [vp, vp, vp, vp, vp, C.c_int, C.c_int,
                                                     C.c_int, C.c_int, C.c_int, C.c_float, vp]),
    "emb_synth_normal_bf16": (C.c_int, [C.c_uint64, C.c_int64, u16p]),
    "lingbot_flex_attn_f32": (C.c_int, [vp, vp, vp, vp, vp, vp] + [C.c_int] * 5 + [C.c_float, vp]),
    "lingbot_flex_attn_f32_masked": (C.c_int, [vp, vp, vp, vp, vp, vp, vp] + [C.c_int] * 5 + [C.c_float, vp]),
    "lingbot_flex_attn_cuda_smoke": (C.c_int, [vp]),
    "cosmos3_qwen_causal_gqa_attention_f32": (C.c_int, [vp, vp, vp, vp] + [C.c_int] * 6 + [vp]),
    "cosmos3_qwen_gen_full_gqa_attention_f32": (C.c_int, [vp, vp, vp, vp] + [C.c_int] * 7 + [vp]),
    "cosmos3_qwen_gen_full_gqa_attention_workspace_f32": (C.c_int, [vp, vp, vp, vp, vp] + [C.c_int] * 7 + [vp]),
    "cosmos3_qwen_gen_full_gqa_attention_workspace_bf16tc_f32": (C.c_int, [vp] * 6 + [C.c_int] * 7 + [vp]),
    "emb_ggml_flash_attn_ext_workspace": (C.c_size_t, [C.POINTER(GgmlTensor)] * 5),
    "emb_ggml_flash_attn_ext": (C.c_int, [C.POINTER(GgmlTensor)] * 4 + [C.c_float] * 3 +
                                [C.POINTER(GgmlTensor), vp, C.c_size_t, vp]),
    "emb_w8a16_gemm": (C.c_int, [vp, C.c_int32, C.c_int64, vp, vp, C.c_int32, C.c_int32, C.c_int32,
                                 vp, C.c_int64, C.c_int32, vp]),
    "emb_w8a16_qkv_append": (C.c_int, [vp, C.c_int32, C.c_int64, vp, vp, C.c_int32, C.c_int32,
                                       C.c_int32, vp, C.c_int64, vp, vp, C.c_int32, vp, vp, vp,
                                       C.c_int32, C.c_int32, vp]),
    "emb_w8a16_gated_residual": (C.c_int, [vp, C.c_int32, C.c_int64, vp, vp, C.c_int32, C.c_int32,
                                           C.c_int32, vp, vp, C.c_int64, vp, vp, C.c_int64, vp,
                                           C.c_int64, C.c_int32, vp, vp]),
    "emb_dense_gated_residual": (C.c_int, [vp, C.c_int32, C.c_int64, vp, C.c_int32, C.c_int64, C.c_int32,
                                           C.c_int32, C.c_int32, vp, vp, C.c_int64, vp, vp, C.c_int64, vp,
                                           C.c_int64, C.c_int32, vp, vp]),
    "cosmos3_w8a16_linear_f32": (C.c_int, [vp, vp, vp, vp] + [C.c_int] * 7 + [vp]),
    "cosmos3_w8a16_linear_f32_ws": (C.c_int, [vp] * 8 + [C.c_int] * 7 + [vp]),
    "cosmos3_w8a16_linear_bf16_ws": (C.c_int, [vp] * 7 + [C.c_int] * 7 + [vp]),
    "cosmos3_w8a16_f32_to_bf16_ws": (C.c_int, [vp, vp, C.c_int, vp]),
}

EMB_W8_Y_BF16, EMB_W8_Y_F32_ROUNDED, EMB_W8_Y_F32_RAW = range(3)


def header_symbols() -> list[str]:
    """Function names declared in include/emb_kv.h."""
    import re
    text = (PKG.parent / "include" / "emb_kv.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:emb|lingbot|cosmos3)_\w+)\s*\(", text)))


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        # torch ships its own libamdhip64.so.7.  Loading torch first makes this
        # library bind to that same runtime (the dynamic linker matches the
        # soname), so device pointers and streams from torch are valid here; a
        # second HIP runtime in the process would not see the device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return lib().emb_last_error().decode()


def check(rc: int, what: str = "") -> int:
    if rc < 0:
        raise RuntimeError(f"{what} failed rc={rc}: {last_error()}")
    return rc


def ptr(x) -> int | None:
    """Device/host pointer of a torch tensor, a numpy array or an int (None -> NULL)."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    if isinstance(x, np.ndarray):
        return x.ctypes.data
    raise TypeError(type(x))


def stream_ptr(stream=None) -> int | None:
    if stream is None:
        return None
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def _np_i64(n):
    a = np.zeros(max(int(n), 1), dtype=np.int64)
    return a, a.ctypes.data_as(i64p)


class DevSlotCache:
    """emb_dev_cache_*: slot metadata in device memory (torch tensors on `device`).
    update() returns device tensors (slots, valid, n_valid, status); nothing
    is synchronised."""

    def __init__(self, capacity: int, device, legacy_clear_pred: bool = False, stream=None):
        import torch
        self.capacity = capacity
        self.id = torch.empty(capacity, dtype=torch.int64, device=device)
        self.mask = torch.empty(capacity, dtype=torch.uint8, device=device)
        self.is_pred = torch.empty(capacity, dtype=torch.uint8, device=device)
        self.slots = torch.empty(capacity, dtype=torch.int32, device=device)
        self.valid = torch.empty(capacity, dtype=torch.int32, device=device)
        self.n_valid = torch.empty(1, dtype=torch.int32, device=device)
        self.status = torch.empty(1, dtype=torch.int32, device=device)
        self.desc = DevCacheDesc(ptr(self.id), ptr(self.mask), ptr(self.is_pred), capacity, int(legacy_clear_pred))
        check(lib().emb_dev_cache_init(C.byref(self.desc), stream_ptr(stream)), "emb_dev_cache_init")

    def update(self, key_size, mode, stream=None, with_valid=True):
        """The returned status is the device's; last_rc the call's own return
        code (EMB_ERR_CAPACITY, not raised, when key_size > capacity)."""
        if key_size > self.slots.numel():  # slots[key_size] is written even on failure (all -1)
            import torch
            self.slots = torch.empty(key_size, dtype=torch.int32, device=self.slots.device)
        rc = lib().emb_dev_cache_update(C.byref(self.desc), key_size, mode, ptr(self.slots),
                                        ptr(self.valid) if with_valid else None,
                                        ptr(self.n_valid) if with_valid else None, ptr(self.status),
                                        stream_ptr(stream))
        self.last_rc = rc
        if rc != EMB_ERR_CAPACITY:
            check(rc, "emb_dev_cache_update")
        return self.slots[:key_size], self.valid, self.n_valid, self.status

    def restore(self, slots, n, stream=None):
        check(lib().emb_dev_cache_restore(C.byref(self.desc), ptr(slots), n, stream_ptr(stream)),
              "emb_dev_cache_restore")

    def clear_pred(self, stream=None):
        check(lib().emb_dev_cache_clear_pred(C.byref(self.desc), stream_ptr(stream)), "emb_dev_cache_clear_pred")

    def state(self):
        return self.id.cpu().numpy(), self.mask.cpu().numpy(), self.is_pred.cpu().numpy()


class SlotCache:
    """LingBotKVCache semantics (models/lingbot_va.cpp:8740-8997) over libemb_kv."""

    def __init__(self, capacity: int, legacy_clear_pred: bool = False):
        self.h = lib().emb_slot_cache_create(capacity, int(legacy_clear_pred))
        if not self.h:
            raise RuntimeError(last_error())
        self.capacity = capacity

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.emb_slot_cache_destroy(self.h)
            self.h = None

    def used_count(self): return lib().emb_slot_cache_used_count(self.h)
    def pred_count(self): return lib().emb_slot_cache_pred_count(self.h)
    def next_id(self): return lib().emb_slot_cache_next_id(self.h)

    def allocate(self, key_size):
        a, p = _np_i64(key_size)
        rc = lib().emb_slot_cache_allocate(self.h, key_size, p)
        return (a[:key_size] if rc == 0 else None), rc

    def update_meta(self, key_size, pred):
        a, p = _np_i64(key_size)
        rc = lib().emb_slot_cache_update_meta(self.h, key_size, int(pred), p)
        return (a[:key_size] if rc == 0 else None), rc

    def prepare_mode0(self, key_size):
        s, sp = _np_i64(key_size)
        v, vpp = _np_i64(self.capacity)
        n = C.c_int64(0)
        rc = lib().emb_slot_cache_prepare_mode0(self.h, key_size, sp, vpp, C.byref(n))
        if rc != 0:
            return None, None, rc
        return s[:key_size], v[: n.value], rc

    def restore(self, slots):
        a = np.ascontiguousarray(slots, dtype=np.int64)
        lib().emb_slot_cache_restore(self.h, a.ctypes.data_as(i64p), len(a))

    def clear_pred(self): lib().emb_slot_cache_clear_pred(self.h)

    def collect_valid(self):
        v, p = _np_i64(self.capacity)
        n = lib().emb_slot_cache_collect_valid(self.h, p)
        return v[:n]

    def state(self):
        idv = np.zeros(self.capacity, np.int64)
        m = np.zeros(self.capacity, np.uint8)
        pr = np.zeros(self.capacity, np.uint8)
        check(lib().emb_slot_cache_export(self.h, idv.ctypes.data_as(i64p), m.ctypes.data_as(u8p),
                                          pr.ctypes.data_as(u8p)), "export")
        return idv, m, pr

    def bind_pool(self, pool):
        check(lib().emb_slot_cache_bind_pool(self.h, pool.h), "bind_pool")
        self._pool = pool  # the pool must outlive the cache
    def map_range(self, n): check(lib().emb_slot_cache_map_range(self.h, n), "map_range")
    def release_pages(self): check(lib().emb_slot_cache_release_pages(self.h), "release_pages")

    def block_table(self, n=None):
        n = n or (self.capacity + 15) // 16
        bt = np.zeros(n, np.int32)
        check(lib().emb_slot_cache_block_table(self.h, bt.ctypes.data_as(i32p), n), "block_table")
        return bt


class PagePool:
    def __init__(self, n_pages: int, seed: int = 0):
        self.h = lib().emb_page_pool_create(n_pages, seed)
        if not self.h:
            raise RuntimeError(last_error())

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.emb_page_pool_destroy(self.h)
            self.h = None

    def free_count(self): return lib().emb_page_pool_free_count(self.h)


def lingbot_kv_capacity(override_tokens=0, frame_chunk_size=4, action_per_frame=4, n_suffix=0,
                        attn_window=30, latent_h=8, latent_w=16, patch_t=1, patch_h=2, patch_w=2,
                        seq=0):
    return lib().emb_lingbot_kv_capacity(override_tokens, frame_chunk_size, action_per_frame,
                                         n_suffix, attn_window, latent_h, latent_w, patch_t,
                                         patch_h, patch_w, seq)


def synth_normal_bf16(seed: int, n: int) -> np.ndarray:
    out = np.zeros(n, np.uint16)
    check(lib().emb_synth_normal_bf16(seed, n, out.ctypes.data_as(u16p)), "synth")
    return out


# ---- call-site masks (host; numpy in, numpy out) ----
def hy_patch_groups(modality_mask):
    m = np.ascontiguousarray(modality_mask, np.int32)
    g = np.full(max(len(m), 1), -1, np.int32)
    n = check(lib().emb_hy_patch_groups(ptr(m), len(m), ptr(g)), "emb_hy_patch_groups")
    return n, g[:len(m)]


def hy_prefix_mask(n, group_of=None):
    """(u8 allow [n][n], f16 bits [n][n]) of HY-VLA's prefix mask."""
    allow = np.zeros((n, n), np.uint8)
    f16 = np.zeros((n, n), np.uint16)
    g = None if group_of is None else np.ascontiguousarray(group_of, np.int32)
    check(lib().emb_hy_prefix_mask(n, ptr(g), ptr(allow), ptr(f16)), "emb_hy_prefix_mask")
    return allow, f16


def hy_suffix_mask(n_pref, n_suf):
    allow = np.zeros((n_suf, n_pref + n_suf), np.uint8)
    f16 = np.zeros((n_suf, n_pref + n_suf), np.uint16)
    check(lib().emb_hy_suffix_mask(n_pref, n_suf, ptr(allow), ptr(f16)), "emb_hy_suffix_mask")
    return allow, f16


def groot_layer_mask_kind(layer, attend_text_every_n_blocks=2):
    return check(lib().emb_groot_layer_mask_kind(layer, attend_text_every_n_blocks), "emb_groot_layer_mask_kind")


def groot_cross_masks(attention_mask, image_flags, n_q):
    a = np.ascontiguousarray(attention_mask, np.int32)
    im = np.ascontiguousarray(image_flags, np.int32)
    text = np.zeros((n_q, len(a)), np.float32)
    image = np.zeros((n_q, len(a)), np.float32)
    check(lib().emb_groot_cross_masks(ptr(a), ptr(im), len(a), n_q, ptr(text), ptr(image)), "emb_groot_cross_masks")
    return text, image


def smolvla_masks(prefix_valid, n_suf):
    v = np.ascontiguousarray(prefix_valid, np.uint8)
    n = len(v)
    pm = np.zeros((n, n), np.float32)
    fm = np.zeros((n_suf, n + n_suf), np.float32)
    cm = np.zeros((n_suf, n), np.float32)
    check(lib().emb_smolvla_masks(ptr(v), n, n_suf, ptr(pm), ptr(fm), ptr(cm)), "emb_smolvla_masks")
    return pm, fm, cm


def smolvla_positions(prefix_valid, n_suf):
    v = np.ascontiguousarray(prefix_valid, np.uint8)
    pp = np.zeros(len(v), np.int32)
    sp = np.zeros(max(n_suf, 1), np.int32)
    cp = np.zeros(max(n_suf, 1), np.int32)
    check(lib().emb_smolvla_positions(ptr(v), len(v), n_suf, ptr(pp), ptr(sp), ptr(cp)), "emb_smolvla_positions")
    return pp, sp[:n_suf], cp[:n_suf]


def kv_append(k_new, v_new, src_stride, n, slots, block_table, capacity, k_pool, v_pool, hkv, d,
              stream=None, v16_pool=None):
    return check(lib().emb_kv_append(ptr(k_new), ptr(v_new), src_stride, n, ptr(slots),
                                     ptr(block_table), capacity, ptr(k_pool), ptr(v_pool),
                                     ptr(v16_pool), hkv, d, stream_ptr(stream)), "emb_kv_append")


def qkv_norm_rope_append(qkv, ld, tokens, q_heads, kv_heads, d, q_out, slots, block_table, capacity, k_pool,
                         v_pool, v16_pool=None, q_gamma=None, k_gamma=None, eps=1e-6, rope_kind=0,
                         rope_theta=1e6, first_position=0, position_ids=None, ldq=None, stream=None):
    return check(lib().emb_qkv_norm_rope_append(ptr(qkv), ld, tokens, q_heads, kv_heads, d, ptr(q_gamma),
                                                 ptr(k_gamma), eps, rope_kind, rope_theta, first_position,
                                                 ptr(position_ids), ptr(q_out), ldq or q_heads * d, ptr(slots),
                                                 ptr(block_table), capacity, ptr(k_pool), ptr(v_pool),
                                                 ptr(v16_pool), stream_ptr(stream)), "emb_qkv_norm_rope_append")


def qkv_rownorm_rope_append(qkv, ld, tokens, heads, d, q_out, slots, block_table, capacity, k_pool, v_pool,
                            v16_pool=None, qkv_bias=None, q_weight=None, k_weight=None, eps=1e-6,
                            rope_cos=None, rope_sin=None, ldq=None, stream=None):
    """LingBot full-row q/k RMSNorm + Wan RoPE (per-token cos/sin tables) + paged
    K/V append on an f32 QKV row (emb_qkv_rownorm_rope_append)."""
    hid = heads * d
    _need_rows(qkv, tokens, ld, 3 * hid, 4, "qkv")
    _need_rows(q_out, tokens, ldq or hid, hid, 2, "q_out")
    _need_bytes(qkv_bias, 3 * hid * 4, "qkv_bias")
    _need_bytes(q_weight, hid * 4, "q_weight")
    _need_bytes(k_weight, hid * 4, "k_weight")
    _need_bytes(rope_cos, tokens * (d // 2) * 4, "rope_cos")
    _need_bytes(rope_sin, tokens * (d // 2) * 4, "rope_sin")
    _need_bytes(slots, tokens * 4, "slots")
    return check(lib().emb_qkv_rownorm_rope_append(ptr(qkv), ld, tokens, heads, d, ptr(qkv_bias),
                                                    ptr(q_weight), ptr(k_weight), eps, ptr(rope_cos),
                                                    ptr(rope_sin), ptr(q_out), ldq or hid, ptr(slots),
                                                    ptr(block_table), capacity, ptr(k_pool), ptr(v_pool),
                                                    ptr(v16_pool), stream_ptr(stream)),
                 "emb_qkv_rownorm_rope_append")


def qkv_neox_rope_append(q, ld_q, k, ld_k, v, ld_v, tokens, q_heads, kv_heads, d, q_out, slots, block_table,
                         capacity, k_pool, v_pool, v16_pool=None, positions=None, first_position=0,
                         freq_base=10000.0, q_out_f32=True, ldq=None, stream=None):
    """pi0.5 NEOX RoPE (ggml_rope_ext, mode NEOX, n_dims = d) on f32 Q and K plus
    the paged K/V append (emb_qkv_neox_rope_append)."""
    _need_rows(q, tokens, ld_q, q_heads * d, 4, "q")
    _need_rows(k, tokens, ld_k, kv_heads * d, 4, "k")
    _need_rows(v, tokens, ld_v, kv_heads * d, 4, "v")
    _need_rows(q_out, tokens, ldq or q_heads * d, q_heads * d, 4 if q_out_f32 else 2, "q_out")
    _need_bytes(positions, tokens * 4, "positions")
    _need_bytes(slots, tokens * 4, "slots")
    return check(lib().emb_qkv_neox_rope_append(ptr(q), ld_q, ptr(k), ld_k, ptr(v), ld_v, tokens, q_heads,
                                                 kv_heads, d, ptr(positions), first_position, freq_base,
                                                 ptr(q_out), int(bool(q_out_f32)), ldq or q_heads * d,
                                                 ptr(slots), ptr(block_table), capacity, ptr(k_pool),
                                                 ptr(v_pool), ptr(v16_pool), stream_ptr(stream)),
                 "emb_qkv_neox_rope_append")


def kv_gather(k_pool, v_pool, valid, n, block_table, capacity, k_out, v_out, hkv, d, stream=None):
    return check(lib().emb_kv_gather(ptr(k_pool), ptr(v_pool), ptr(valid), n, ptr(block_table),
                                     capacity, ptr(k_out), ptr(v_out), hkv, d, stream_ptr(stream)),
                 "emb_kv_gather")


def w8a16_gemm(x, qweight, scales, M, K, N, y, y_kind=EMB_W8_Y_BF16, x_is_f32=False, ldx=None,
               ldy=None, stream=None):
    return check(lib().emb_w8a16_gemm(ptr(x), int(x_is_f32), ldx or K, ptr(qweight), ptr(scales),
                                       M, K, N, ptr(y), ldy or N, y_kind, stream_ptr(stream)),
                 "emb_w8a16_gemm")


def w8a16_qkv_append(x, qweight, scales, M, K, n_q, q_out, slots, block_table, capacity, k_pool,
                     v_pool, hkv, d, x_is_f32=False, ldx=None, ldq=None, stream=None, v16_pool=None):
    return check(lib().emb_w8a16_qkv_append(ptr(x), int(x_is_f32), ldx or K, ptr(qweight),
                                            ptr(scales), M, K, n_q, ptr(q_out), ldq or n_q,
                                            ptr(slots), ptr(block_table), capacity, ptr(k_pool),
                                            ptr(v_pool), ptr(v16_pool), hkv, d, stream_ptr(stream)),
                 "emb_w8a16_qkv_append")


def _need_bytes(t, nbytes, what):
    """Refuse a torch tensor smaller than the extent a kernel will read or write
    (a C-ABI call cannot see buffer sizes)."""
    if t is None or not hasattr(t, "untyped_storage"):
        return
    have = t.untyped_storage().nbytes() - t.storage_offset() * t.element_size()  # from data_ptr to the end
    if have < nbytes:
        raise ValueError(f"{what}: {have} bytes from its start, {nbytes} needed")


def _need_rows(t, rows, ld, cols, esize, what):
    """Same for a [rows][ld] view: the last row ends at (rows - 1) * ld + cols."""
    _need_bytes(t, ((rows - 1) * ld + cols) * esize, what)


def w8a16_gated_residual(x, qweight, scales, M, K, N, residual, out, bias=None, gate=None,
                         gate_bias=None, ldg=None, ldr=None, ldo=None, round_bf16=False,
                         x_is_f32=False, ldx=None, x_bf16_workspace=None, stream=None):
    """out = residual + ((W8 projection of x) + bias) * (gate + gate_bias), f32
    (emb_w8a16_gated_residual); out may be the residual tensor itself."""
    _need_rows(x, M, ldx or K, K, 4 if x_is_f32 else 2, "x")
    _need_bytes(qweight, (K // 16) * 4 * N * 4, "qweight ([K/16][4N] int32)")
    _need_bytes(scales, N * 2, "scales")
    _need_rows(residual, M, ldr or N, N, 4, "residual")
    _need_rows(out, M, ldo or N, N, 4, "out")
    _need_rows(gate, M, ldg or N, N, 4, "gate")
    _need_bytes(bias, N * 4, "bias")
    _need_bytes(gate_bias, N * 4, "gate_bias")
    if x_is_f32:
        _need_bytes(x_bf16_workspace, M * K * 2, "x_bf16_workspace")
    return check(lib().emb_w8a16_gated_residual(ptr(x), int(x_is_f32), ldx or K, ptr(qweight),
                                                ptr(scales), M, K, N, ptr(bias), ptr(gate),
                                                ldg or N, ptr(gate_bias), ptr(residual), ldr or N,
                                                ptr(out), ldo or N, int(round_bf16),
                                                ptr(x_bf16_workspace), stream_ptr(stream)),
                 "emb_w8a16_gated_residual")


def dense_gated_residual(x, weight, weight_type, M, K, N, out, residual=None, bias=None, gate=None,
                         gate_bias=None, ldw=None, ldg=None, ldr=None, ldo=None, round_bf16=False,
                         x_is_f32=True, ldx=None, x_bf16_workspace=None, stream=None):
    """out = [residual +] (lin(x) [* (gate + gate_bias)]) with ggml dense
    weights, lin = W x + bias in ggml's CUDA mul_mat numerics
    (emb_dense_gated_residual); weight_type EMB_GGML_BF16 or EMB_GGML_F32."""
    wsz = 4 if weight_type == EMB_GGML_F32 else 2
    _need_rows(x, M, ldx or K, K, 4 if x_is_f32 else 2, "x")
    _need_rows(weight, N, ldw or K, K, wsz, "weight")
    _need_rows(residual, M, ldr or N, N, 4, "residual")
    _need_rows(out, M, ldo or N, N, 4, "out")
    _need_rows(gate, M, ldg or N, N, 4, "gate")
    _need_bytes(bias, N * 4, "bias")
    _need_bytes(gate_bias, N * 4, "gate_bias")
    if x_is_f32:
        _need_bytes(x_bf16_workspace, M * K * 2, "x_bf16_workspace")
    return check(lib().emb_dense_gated_residual(ptr(x), int(x_is_f32), ldx or K, ptr(weight), int(weight_type),
                                                ldw or K, M, K, N, ptr(bias), ptr(gate), ldg or N,
                                                ptr(gate_bias), ptr(residual), ldr or N, ptr(out), ldo or N,
                                                int(round_bf16), ptr(x_bf16_workspace), stream_ptr(stream)),
                 "emb_dense_gated_residual")


def attn_workspace_bytes(batch, max_q, hq, hkv, d, splits):
    return lib().emb_attn_workspace_bytes(batch, max_q, hq, hkv, d, splits)


def paged_attention(*, q, out, k_pool, v_pool, batch, hq, hkv, d, max_q, scale, capacity, v16_pool=None,
                    cu_q=None, n_keys=None, q_pos0=None, q_is_f32=False, q_stride=None,
                    out_stride=None, block_tables=None, bt_stride=0, valid_slots=None,
                    valid_stride=0, mask_kind=EMB_MASK_FULL, chunk=0, window=-1, mask=None,
                    mask_q_stride=0, mask_batch_stride=0, block_map=None, block_size=0,
                    block_map_cols=0, block_map_batch_stride=0, splits=1, workspace=None,
                    n_keys_uniform=0, out_bf16_round=False, stream=None, noalloc=False, p_bf16=False,
                    split_keys=0, kernel=0):
    a = AttnArgs()
    a.q = ptr(q); a.q_is_f32 = int(q_is_f32)
    a.q_stride = q_stride if q_stride is not None else hq * d
    a.out = ptr(out); a.out_stride = out_stride if out_stride is not None else hq * d
    a.cu_q = ptr(cu_q); a.n_keys = ptr(n_keys); a.q_pos0 = ptr(q_pos0)
    a.k_pool = ptr(k_pool); a.v_pool = ptr(v_pool); a.v16_pool = ptr(v16_pool)
    a.block_tables = ptr(block_tables); a.bt_stride = bt_stride
    a.valid_slots = ptr(valid_slots); a.valid_stride = valid_stride
    a.capacity = capacity; a.batch = batch; a.hq = hq; a.hkv = hkv; a.head_dim = d
    a.max_q = max_q; a.scale = scale
    a.mask_kind = mask_kind; a.chunk = chunk; a.window = window
    a.mask = ptr(mask); a.mask_q_stride = mask_q_stride; a.mask_batch_stride = mask_batch_stride
    a.block_map = ptr(block_map); a.block_size = block_size; a.block_map_cols = block_map_cols
    a.block_map_batch_stride = block_map_batch_stride
    a.splits = splits; a.workspace = ptr(workspace); a.n_keys_uniform = n_keys_uniform
    a.out_bf16_round = int(out_bf16_round)
    a.p_bf16 = int(p_bf16)
    a.split_keys = int(split_keys)
    a.kernel = int(kernel)
    if noalloc:  # split-K partials in the library's scratch (workspace must be None)
        return check(lib().emb_paged_attention_noalloc(C.byref(a), stream_ptr(stream)), "emb_paged_attention_noalloc")
    return check(lib().emb_paged_attention(C.byref(a), stream_ptr(stream)), "emb_paged_attention")


def flex_attention(q, k, v, row_ptr, col_idx, out, seq_q, seq_k, n_heads, head_dim, block_size, scale,
                   token_mask=None, stream=None):
    """lingbot_flex_attn_f32[_masked]: f32 [seq][H][D] device tensors, device CSR."""
    L = lib()
    if token_mask is None:
        rc = L.lingbot_flex_attn_f32(ptr(q), ptr(k), ptr(v), ptr(row_ptr), ptr(col_idx), ptr(out), seq_q, seq_k,
                                     n_heads, head_dim, block_size, scale, stream_ptr(stream))
    else:
        rc = L.lingbot_flex_attn_f32_masked(ptr(q), ptr(k), ptr(v), ptr(row_ptr), ptr(col_idx), ptr(token_mask),
                                            ptr(out), seq_q, seq_k, n_heads, head_dim, block_size, scale,
                                            stream_ptr(stream))
    return check(rc, "lingbot_flex_attn_f32")


def ggml_tensor(t, ggml_type, ne, nb_elems=None):
    """Descriptor of a device tensor: ne innermost-first; nb_elems (element
    strides, innermost first) default to the contiguous ones."""
    es = 4 if ggml_type == EMB_GGML_F32 else 2
    ne = list(ne) + [1] * (4 - len(ne))
    if nb_elems is None:
        nb_elems = [1, ne[0], ne[0] * ne[1], ne[0] * ne[1] * ne[2]]
    d = GgmlTensor()
    d.type = ggml_type
    for i in range(4):
        d.ne[i] = int(ne[i])
        d.nb[i] = int(nb_elems[i]) * es
    d.data = ptr(t)
    return d


def ggml_flash_attn_ext(q, k, v, mask, dst, scale, workspace=None, max_bias=0.0, logit_softcap=0.0,
                        stream=None):
    """emb_ggml_flash_attn_ext over GgmlTensor descriptors (mask may be None).
    Allocates the workspace with torch when none is given."""
    L = lib()
    mp = C.byref(mask) if mask is not None else None
    nbytes = L.emb_ggml_flash_attn_ext_workspace(C.byref(q), C.byref(k), C.byref(v), mp, C.byref(dst))
    if nbytes == 0:
        raise RuntimeError("emb_ggml_flash_attn_ext: descriptors rejected")
    if workspace is None:
        import torch
        workspace = torch.empty(nbytes // 4 + 64, dtype=torch.float32, device="cuda")
    rc = L.emb_ggml_flash_attn_ext(C.byref(q), C.byref(k), C.byref(v), mp, scale, max_bias, logit_softcap,
                                   C.byref(dst), ptr(workspace), nbytes, stream_ptr(stream))
    return check(rc, "emb_ggml_flash_attn_ext")
