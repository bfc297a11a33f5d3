"""Invariants of the dK/dV kernel's inline-assembly loads, checked on the
compiled gfx950 code (CPU: hipcc cross-compiles; no GPU needed).

The kernel loads the next (item, head)'s K | Rk and V rows with inline
assembly into the registers that hold the current ones
(``load16_inplace`` in fna2_amd/csrc/fna2_tile.h), and the next step's ring
barrier (``s_waitcnt vmcnt(N); s_barrier``) is what waits for them.  The
compiler does not know these loads exist, so correctness rests on one
property of the code it emits: on every control-flow path from such a load
to the next ``s_barrier``, no instruction outside inline assembly reads or
writes the load's destination registers (a copy or spill there would see
the register before the data lands).  This test rebuilds the kernel to
assembly with the library's own flags and walks every path.
"""
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


def _regs(tok: str) -> set:
    out = set()
    for a, b in re.findall(r"v\[(\d+):(\d+)\]", tok):
        out |= set(range(int(a), int(b) + 1))
    for a in re.findall(r"\bv(\d+)\b", tok):
        out.add(int(a))
    return out


def inplace_violations(asm: str):
    """(load line, touching line) pairs for every path that breaks the rule."""
    lines = asm.split("\n")
    labels = {}
    for i, l in enumerate(lines):
        m = re.match(r"^(\.LBB[0-9_]+):", l)
        if m:
            labels[m.group(1)] = i
    bad, loads, in_asm = [], 0, False
    for i, l in enumerate(lines):
        if "ASMSTART" in l:
            in_asm = True
            continue
        if "ASMEND" in l:
            in_asm = False
            continue
        if not (in_asm and "buffer_load_dwordx4 v[" in l and " lds" not in l):
            continue
        loads += 1
        dst = _regs(l.split(",")[0])
        stack, seen, found = [(i + 1, True)], set(), None
        while stack and not found:
            j, inside = stack.pop()
            while j < len(lines):
                if (j, inside) in seen:
                    break
                seen.add((j, inside))
                t = lines[j].strip()
                if "ASMSTART" in t:
                    inside = True
                elif "ASMEND" in t:
                    inside = False
                elif "s_barrier" in t or t.startswith("s_endpgm"):
                    break
                elif not inside and t and not t.startswith((";", ".")):
                    if _regs(t) & dst:
                        found = (j + 1, t)
                        break
                    m = re.match(r"s_branch (\S+)", t)
                    if m:
                        j = labels[m.group(1)]
                        continue
                    m = re.match(r"s_cbranch_\w+ (\S+)", t)
                    if m:
                        stack.append((labels[m.group(1)], inside))
                j += 1
        if found:
            bad.append((i + 1, found))
    return loads, bad


def test_checker_catches_a_planted_copy():
    asm = "\n".join([
        ";;#ASMSTART", "\tbuffer_load_dwordx4 v[8:11], v1, s[0:3], 0 offen", ";;#ASMEND",
        "\tv_mov_b32_e32 v20, v9", "\ts_barrier", "\ts_endpgm"])
    assert inplace_violations(asm)[1]
    ok = asm.replace("v_mov_b32_e32 v20, v9", "v_mov_b32_e32 v20, v12")
    assert not inplace_violations(ok)[1]


@pytest.mark.skipif(not (shutil.which("hipcc") or os.path.exists("/opt/rocm/bin/hipcc")),
                    reason="hipcc not available")
def test_dkdv_inplace_row_loads_untouched_until_barrier(tmp_path):
    from fna2_amd import build as B
    out = tmp_path / "dkdv.s"
    cmd = [B.HIPCC, *B.COMMON, "--cuda-device-only", "-S", str(B.CSRC / "fna2_bwd_dkdv.hip"),
           "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    loads, bad = inplace_violations(out.read_text())
    assert loads >= 6 * 18, loads  # every kernel variant has its row loads
    assert not bad, bad[:5]
