"""The pipelined W8A16 GEMM issues its W loads as inline asm and waits for them
with its own counted s_waitcnt, so the compiler does not know those registers
are in flight.  Any instruction that names them between a load and its wait
would read (or be overwritten by) a load that has not landed: results wrong
with no error.  This test compiles the kernels to gfx950 assembly and walks
from every such load, through the loop's back edge, to the next counted
wait, failing on any instruction that names a destination register."""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SRC = ROOT / "embodied.cpp_amd" / "csrc" / "w8a16_gemm.hip"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _regs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _named(ins):
    out = set()
    for tok in re.findall(r"v\[\d+:\d+\]|\bv\d+\b", ins.split(";")[0]):
        out |= _regs(tok)
    return out


VMEM = re.compile(r"^\s*(buffer_|global_|flat_|scratch_)\w+")
WAIT = re.compile(r"s_waitcnt\s+vmcnt\((\d+)\)")


def violations(asm_lines, kernel_re):
    """(kernel starts, asm loads seen, [(kernel, load line, line, instruction)]).
    From each asm load, every path is followed (both ways at a conditional
    branch) with a count of the vector-memory operations issued after the
    load; an s_waitcnt vmcnt(N) retires the load only once that count is at
    least N (vmcnt counts loads and stores in issue order)."""
    starts = [i for i, l in enumerate(asm_lines) if re.match(kernel_re, l)]
    found, n_loads = [], 0
    for k0 in starts:
        k1 = next(i for i in range(k0, len(asm_lines)) if asm_lines[i].startswith(".Lfunc_end"))
        body = asm_lines[k0:k1]
        labels = {l.split(":")[0]: i for i, l in enumerate(body) if re.match(r"^\.LBB\w+:", l)}
        in_asm, state = [False] * len(body), False
        for i, line in enumerate(body):
            if "ASMSTART" in line:
                state = True
            elif "ASMEND" in line:
                state = False
            in_asm[i] = state
        for i, line in enumerate(body):
            if not (in_asm[i] and "global_load_dwordx4" in line):
                continue
            n_loads += 1
            dst = _regs(line.split()[1].rstrip(","))
            stack, seen, hit = [(i + 1, 0)], set(), None
            while stack and hit is None:
                j, cnt = stack.pop()
                while j < len(body):
                    if (j, min(cnt, 64)) in seen:
                        break
                    seen.add((j, min(cnt, 64)))
                    lj = body[j]
                    w = WAIT.search(lj)
                    if w and cnt >= int(w.group(1)):
                        break  # this load has landed on this path
                    if "s_endpgm" in lj:
                        break
                    ins = lj.strip()
                    if (ins and not ins.startswith((";", ".", "s_")) and not (in_asm[j] and "global_load" in ins)
                            and (_named(ins) & dst)):
                        hit = (j, ins)
                        break
                    if VMEM.match(lj):
                        cnt += 1
                    m = re.match(r"\s*s_cbranch_\w+\s+(\.LBB\w+)", lj)
                    if m:
                        stack.append((labels[m.group(1)], cnt))
                    m = re.match(r"\s*s_branch\s+(\.LBB\w+)", lj)
                    if m:
                        j = labels[m.group(1)]
                        continue
                    j += 1
            if hit:
                found.append((body[0][:70], i, hit[0], hit[1]))
    return starts, n_loads, found


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")
def test_w8_pipeline_loads_untouched_until_waited(tmp_path):
    out = tmp_path / "w8.s"
    subprocess.run([HIPCC, "-xhip", "--offload-arch=gfx950", "--cuda-device-only", "-S", "-Xclang",
                    "-target-feature", "-Xclang", "-packed-fp32-ops", "-O3", "-std=c++17",
                    f"-I{ROOT / 'include'}", f"-I{ROOT / 'embodied.cpp_amd' / 'csrc'}", str(SRC), "-o", str(out)],
                   check=True, stderr=subprocess.DEVNULL)
    starts, n_loads, found = violations(out.read_text().split("\n"),
                                        r"^_ZN12_GLOBAL__N_122w8a16_gemm_pipe_kernel\S*:")
    assert len(starts) >= 10 and n_loads >= 6 * len(starts), (len(starts), n_loads)
    assert not found, found[:4]


def _kernel(lines):
    return ["_ZN12_GLOBAL__N_122w8a16_gemm_pipe_kernelX:"] + lines + [".Lfunc_end0:"]


PAT = r"^_ZN12_GLOBAL__N_122w8a16_gemm_pipe_kernel\S*:"
LOAD = ["\t;;#ASMSTART", "\tglobal_load_dwordx4 v[6:9], v[16:17], off", "\t;;#ASMEND"]
COPIES = ["\t;;#ASMSTART", "\tbuffer_load_dwordx4 v20, s[4:7], 0 offen lds", "\t;;#ASMEND"]


def _wait(n):
    return ["\t;;#ASMSTART", f"\ts_waitcnt vmcnt({n})", "\t;;#ASMEND"]


def test_checker_flags_in_flight_use():
    # a copy of the loaded registers ahead of the wait (where two paths merged)
    _, n, found = violations(_kernel(LOAD + ["\tv_mov_b64_e32 v[72:73], v[8:9]"] + _wait(0)), PAT)
    assert n == 1 and len(found) == 1
    # the same copy after the wait is fine
    assert not violations(_kernel(LOAD + _wait(0) + ["\tv_mov_b64_e32 v[72:73], v[8:9]"]), PAT)[2]
    # a wait that still allows this load in flight (vmcnt(1) with nothing newer)
    # does not cover a write of its registers (the epilogue arithmetic that faulted)
    assert violations(_kernel(LOAD + _wait(1) + ["\tv_or_b32_e32 v7, s9, v180", "\ts_endpgm"]), PAT)[2]
    # ... and it does once a newer operation is counted
    assert not violations(_kernel(LOAD + COPIES + _wait(1) + ["\tv_or_b32_e32 v7, s9, v180", "\ts_endpgm"]),
                          PAT)[2]
    # both ways of a conditional branch are followed
    br = LOAD + ["\ts_cbranch_scc1 .LBB0_2", "\ts_nop 0"] + _wait(0) + ["\ts_endpgm", ".LBB0_2:",
                                                                        "\tv_mov_b32_e32 v9, 0", "\ts_endpgm"]
    assert violations(_kernel(br), PAT)[2]
