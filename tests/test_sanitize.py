"""AddressSanitizer + UndefinedBehaviorSanitizer runs of the library's host
code (slot cache, page pool, flex masks, call-site masks) and of the CPU
oracle, through the drivers in tests/sanitize/ (CPU only)."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent / "sanitize"


@pytest.fixture(scope="module")
def built():
    r = subprocess.run(["make", "-s", "-C", str(HERE)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return HERE / "build"


@pytest.mark.parametrize("driver", ["host_driver", "oracle_driver"])
def test_sanitized_driver(built, driver):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1",
               OMP_NUM_THREADS="2")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([str(built / driver)], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr
    assert "driver ok" in r.stdout
