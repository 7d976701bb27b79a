"""Builds libemb_kv.so (HIP kernels + C ABI + host C++) for gfx950, in-tree.

    python embodied.cpp_amd/build.py            # build
    python embodied.cpp_amd/build.py --asm      # also keep gfx950 assembly in _build/

The library lands at embodied.cpp_amd/libemb_kv.so.  Every .hip file is
compiled with -Xclang -target-feature -Xclang -packed-fp32-ops so that hipcc
never emits packed fp32 arithmetic (the host pass warns that it does not know
the feature; that warning is harmless).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libemb_kv.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = ["-O3", "-fPIC", "-std=c++17", f"-I{ROOT / 'include'}", f"-I{CSRC}", "-Wall",
          "-Wno-unused-function"]
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-munsafe-fp-atomics"]
# Per-file extras.  -amdgpu-mfma-vgpr-form: MFMA accumulators stay in arch
# VGPRs.  Left to its heuristic the compiler keeps the attention accumulators in
# AGPRs and, because the (rarely taken) online-softmax rescale multiplies them
# with VALU ops, copies all of them AGPR -> VGPR at the top of every key tile.
# The GEMM must not get it: its 128 accumulators plus staging registers only fit
# in the arch + accumulation file together (with it, the QKV epilogue spills).
# The key-split kernel takes it too (accumulators and scores in arch VGPRs, the
# query fragment in AGPRs, 364 registers with no spill): config 1 23.0 ->
# 22.6 us per launch on one box.
EXTRA = {"paged_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
         "paged_attn_ks.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _compile(src: Path, asm: bool) -> Path:
    obj = BUILD / (src.name + ".o")
    cmd = [HIPCC, *COMMON, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".hip":
        cmd[1:1] = DEVICE + EXTRA.get(src.name, [])
        cmd.insert(1, "-xhip")
    if asm and src.suffix == ".hip":
        cmd += ["-save-temps=obj"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(asm: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, asm), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(asm="--asm" in sys.argv))
