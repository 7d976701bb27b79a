"""Shared test setup: markers, library handles and comparison helpers."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "embodied.cpp_amd", ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

# Tolerances for floating-point outputs.
MAX_ABS = 2e-2
MEAN_REL = 1e-3


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu)")


@pytest.fixture(scope="session")
def orc():
    import oracle
    return oracle


@pytest.fixture(scope="session")
def emb():
    import embkv
    embkv.lib()
    return embkv


def v16_shadow(v_pool: np.ndarray, d: int) -> np.ndarray:
    """f16 V shadow of a bf16 V pool (uint16 bits, [pages*H][d][16] rows), as
    include/emb_kv.h specifies it: row t of dim d at position P = t with bits 2
    and 3 swapped, the two 8-key halves exchanged when bit 3 of d is set."""
    v = v_pool.reshape(-1, d, 16)
    with np.errstate(over="ignore", invalid="ignore"):  # random bit patterns: out of f16 range is inf, as on the GPU
        f = (v.astype(np.uint32) << 16).view(np.float32).astype(np.float16).view(np.uint16)
    t = np.arange(16)
    P = (t & 3) | ((t >> 1) & 4) | ((t << 1) & 8)
    dd = np.arange(d)[:, None]
    pos = (((P[None, :] >> 3) ^ ((dd >> 3) & 1)) << 3) + (P[None, :] & 7)  # [d][16]
    out = np.zeros_like(f)
    out[:, dd, pos] = f[:, dd, np.broadcast_to(t, (d, 16))]
    return out.reshape(-1)


def rel_err(a: np.ndarray, b: np.ndarray) -> tuple[float, float]:
    """(max |a-b|, sum|a-b| / sum|b|) -- mean-rel is the relative L1 error."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    d = np.abs(a - b)
    return float(d.max(initial=0.0)), float(d.sum() / max(np.abs(b).sum(), 1e-30))


def assert_close(a, b, what="", max_abs=MAX_ABS, mean_rel=MEAN_REL):
    assert np.all(np.isfinite(a)), f"{what}: non-finite output"
    mx, mr = rel_err(a, b)
    assert mx <= max_abs and mr <= mean_rel, f"{what}: max_abs={mx:.3e} mean_rel={mr:.3e}"
    return mx, mr
