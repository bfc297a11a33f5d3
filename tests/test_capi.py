"""The C ABI (include/fna2.h, libfna2_hip.so) on the CPU: no GPU calls.

* the library loads and exports every function the header declares;
* the ctypes structs match the C layout (gcc compiles a probe of the header);
* host-side validation returns the documented status codes (fna2_check_* and
  fna2_fwd/fna2_bwd reject bad arguments before any GPU work).
"""
import ctypes
import re
import subprocess
import sys
from pathlib import Path

import pytest

from fna2_amd import _capi

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "fna2.h"


@pytest.fixture(scope="module")
def lib():
    if not _capi.LIB_PATH.exists():
        from fna2_amd import build
        build.build()
    return _capi.lib()


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*[\w\s\*]+?\b(fna2_\w+)\s*\(", text, flags=re.M)))


def test_exports_every_declared_symbol(lib):
    names = header_functions()
    assert set(names) == set(_capi.SIGNATURES), "ctypes signatures out of sync with fna2.h"
    out = subprocess.run(["nm", "-D", "--defined-only", str(_capi.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (fna2_\w+)", out))
    for n in names:
        assert n in exported, f"{n} not exported"
        assert getattr(lib, n) is not None


def test_version_and_status_strings(lib):
    assert lib.fna2_version() == 3
    for code in _capi.STATUS:
        assert lib.fna2_status_string(code)
    assert lib.fna2_status_string(12345) == b"unknown status"


def _c_layout(tmp_path):
    fields = {
        "fna2_tensor": ["ptr", "stride_b", "stride_s", "stride_h"],
        "fna2_problem": [f for f, _ in _capi.Problem._fields_],
        "fna2_fwd_args": [f for f, _ in _capi.FwdArgs._fields_],
        "fna2_bwd_args": [f for f, _ in _capi.BwdArgs._fields_],
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "fna2.h"', "int main(void){"]
    for st, fs in fields.items():
        lines.append(f'printf("{st} size %zu\\n", sizeof({st}));')
        for f in fs:
            lines.append(f'printf("{st} {f} %zu\\n", offsetof({st}, {f}));')
    lines.append("return 0;}")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c99", f"-I{HEADER.parent}", str(src), "-o", str(exe)], check=True)
    res = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        st, f, v = line.split()
        res[(st, f)] = int(v)
    return res


def test_struct_layout_matches_header(tmp_path):
    c = _c_layout(tmp_path)
    for st, cls in (("fna2_tensor", _capi.Tensor), ("fna2_problem", _capi.Problem),
                    ("fna2_fwd_args", _capi.FwdArgs), ("fna2_bwd_args", _capi.BwdArgs)):
        assert c[(st, "size")] == ctypes.sizeof(cls), st
        for f, _ in cls._fields_:
            assert c[(st, f)] == getattr(cls, f).offset, (st, f)


# ── validation ───────────────────────────────────────────────────────────────

FAKE = 0x10000  # 16-byte aligned, never dereferenced by the host checks


def _t(ptr=FAKE, sb=0, ss=128, sh=64):
    return _capi.Tensor(ptr, sb, ss, sh)


def _fwd(**over):
    p = dict(dtype=1, varlen=0, batch=2, seqlen_q=64, seqlen_k=64, total_q=0, total_k=0,
             heads=4, heads_kv=2, heads_graph=2, head_dim=64, rank=32, causal=1,
             softmax_scale=0.125, cu_seqlens_q=None, cu_seqlens_k=None)
    p.update({k: v for k, v in over.items() if k in p})
    prob = _capi.Problem(**p)
    a = _capi.FwdArgs()
    a.p = prob
    for name in ("q", "k", "v", "out"):
        setattr(a, name, _t(sb=4 * 64 * 64, ss=64, sh=64 * 64))
    a.r_q = _t(sb=2 * 64 * 32, ss=32, sh=64 * 32)
    a.r_k = _t(sb=2 * 64 * 32, ss=32, sh=64 * 32)
    a.lse = _t(sb=4 * 64, ss=1, sh=64)
    a.graph_scale = FAKE
    for k, v in over.items():
        if k not in p:
            setattr(a, k, v)
    return a


def check_fwd(lib, a):
    return _capi.STATUS[lib.fna2_check_fwd(ctypes.byref(a))]


def test_check_fwd_accepts_valid_dense(lib):
    assert check_fwd(lib, _fwd()) == "FNA2_OK"


def test_check_fwd_accepts_fp16(lib):
    # fp16 q/k/v (FNA2_F16), as the reference's kernels are generic over it
    assert check_fwd(lib, _fwd(dtype=_capi.FNA2_F16)) == "FNA2_OK"


@pytest.mark.parametrize("over,code", [
    (dict(dtype=3), "FNA2_E_DTYPE"),
    (dict(dtype=0), "FNA2_E_DTYPE"),
    (dict(head_dim=96), "FNA2_E_HEAD_DIM"),
    (dict(rank=12), "FNA2_E_RANK"),
    (dict(rank=72), "FNA2_E_RANK"),
    (dict(heads=5), "FNA2_E_HEADS"),
    (dict(heads_graph=9), "FNA2_E_HEADS"),
    (dict(batch=-1), "FNA2_E_SHAPE"),
    (dict(softmax_scale=float("nan")), "FNA2_E_SCALE"),
    (dict(varlen=1, total_q=64, total_k=64), "FNA2_E_SEQLENS"),
    (dict(q=_capi.Tensor(FAKE + 2, 0, 64, 64)), "FNA2_E_STRIDE"),
    (dict(k=_capi.Tensor(FAKE, 0, 60, 64)), "FNA2_E_STRIDE"),
    (dict(q=_capi.Tensor(None, 0, 64, 64)), "FNA2_E_NULL"),
    (dict(graph_scale=None), "FNA2_E_NULL"),
])
def test_check_fwd_rejects(lib, over, code):
    assert check_fwd(lib, _fwd(**over)) == code


def test_no_graph_heads_needs_no_rank_pointers(lib):
    a = _fwd(heads_graph=0, rank=0)
    a.r_q = _capi.Tensor(None, 0, 0, 0)
    a.r_k = _capi.Tensor(None, 0, 0, 0)
    a.graph_scale = None
    assert check_fwd(lib, a) == "FNA2_OK"


def test_varlen_workspace_required(lib):
    a = _fwd(varlen=1, batch=3, total_q=200, total_k=200, cu_seqlens_q=FAKE, cu_seqlens_k=FAKE)
    need = lib.fna2_fwd_workspace_bytes(ctypes.byref(a.p))
    assert need > 0
    assert check_fwd(lib, a) == "FNA2_E_WORKSPACE"
    a.workspace, a.workspace_bytes = FAKE, need
    assert check_fwd(lib, a) == "FNA2_OK"


def test_plan_replaces_the_forward_workspace(lib):
    """A varlen forward given a plan of fna2_plan_bytes needs no workspace of
    its own; a short or misaligned plan is rejected; dense problems have no
    plan."""
    assert lib.fna2_plan_bytes(ctypes.byref(_fwd().p)) == 0
    a = _fwd(varlen=1, batch=3, total_q=200, total_k=200, cu_seqlens_q=FAKE, cu_seqlens_k=FAKE)
    need = lib.fna2_plan_bytes(ctypes.byref(a.p))
    assert need > lib.fna2_fwd_workspace_bytes(ctypes.byref(a.p)) > 0  # plus the key tiles
    a.plan, a.plan_bytes = FAKE, need - 1
    assert check_fwd(lib, a) == "FNA2_E_WORKSPACE"
    a.plan, a.plan_bytes = FAKE + 16, need
    assert check_fwd(lib, a) == "FNA2_E_WORKSPACE"
    a.plan, a.plan_bytes = FAKE, need
    assert check_fwd(lib, a) == "FNA2_OK"


def test_fwd_and_bwd_entry_points_reject_before_gpu_work(lib):
    a = _fwd(head_dim=80)
    assert _capi.STATUS[lib.fna2_fwd(ctypes.byref(a), None)] == "FNA2_E_HEAD_DIM"
    b = _capi.BwdArgs()
    b.p = _fwd().p
    assert _capi.STATUS[lib.fna2_bwd(ctypes.byref(b), None)] == "FNA2_E_NULL"


def test_bwd_workspace_layout(lib):
    base = dict(dtype=1, varlen=0, batch=2, seqlen_q=256, seqlen_k=256, total_q=0, total_k=0,
                heads=8, heads_kv=8, heads_graph=8, head_dim=128, causal=1, softmax_scale=0.1,
                cu_seqlens_q=None, cu_seqlens_k=None)
    w32 = lib.fna2_bwd_workspace_bytes(ctypes.byref(_capi.Problem(rank=32, **base)))
    w64 = lib.fna2_bwd_workspace_bytes(ctypes.byref(_capi.Problem(rank=64, **base)))
    w0 = lib.fna2_bwd_workspace_bytes(ctypes.byref(_capi.Problem(**{**base, "heads_graph": 0},
                                                                 rank=0)))
    rows = 2 * 256
    partials = 4 * (2 * 2) * 4 * 8   # fp32 [query tiles][waves][graph heads]
    nlse = rows * 8 * 4              # fp32 -LSE log2(e) per (row, head)
    assert w32 == partials + nlse  # the rank does not change the layout
    assert w64 == partials + nlse
    assert w0 == 256 + nlse        # no graph heads: one aligned partial slot


def test_python_errors_map_to_assertion(lib):
    with pytest.raises(AssertionError, match="FNA2_E_RANK"):
        _capi.raise_for(-4, "x")
    with pytest.raises(_capi.FNA2Error):
        _capi.raise_for(-10, "x")


def _bwd_varlen(total_q, q_row, **over):
    """A varlen backward call whose q / dout rows are q_row elements apart
    (e.g. views into one fused projection), 4 heads of 128, rank 32."""
    p = dict(dtype=1, varlen=1, batch=2, seqlen_q=0, seqlen_k=0, total_q=total_q,
             total_k=total_q, heads=4, heads_kv=4, heads_graph=4, head_dim=128, rank=32,
             causal=1, softmax_scale=0.1, cu_seqlens_q=FAKE, cu_seqlens_k=FAKE)
    p.update(over)
    b = _capi.BwdArgs()
    b.p = _capi.Problem(**p)
    for name in ("q", "k", "v", "out", "dout", "dq", "dk", "dv"):
        setattr(b, name, _t(ss=q_row, sh=128))
    for name in ("r_q", "r_k", "dr_q", "dr_k"):
        setattr(b, name, _t(ss=q_row, sh=32))
    b.lse = _t(ss=4, sh=1)
    b.delta = _t(ss=1, sh=total_q)
    b.graph_scale = FAKE
    b.d_graph_scale = FAKE
    need = _capi.lib().fna2_bwd_workspace_bytes(ctypes.byref(b.p))
    assert need > 0
    b.workspace, b.workspace_bytes = FAKE, need
    return b


def test_check_bwd_bounds_varlen_span_by_total_q(lib):
    """In varlen mode max_seqlen_q is only a hint (0 here): a sequence may
    span every token, so the dK/dV kernel's 32-bit buffer offsets are bounded
    with total_q.  28 KB rows (a fused q | k | v | R projection) x 80,000
    tokens pass 2^31 bytes and must be refused; 70,000 tokens fit."""
    row = 14336  # elements (28 KB)
    assert 80000 * row * 2 >= 1 << 31 > 70000 * row * 2
    big = _bwd_varlen(80000, row)
    assert _capi.STATUS[lib.fna2_check_bwd(ctypes.byref(big))] == "FNA2_E_SHAPE"
    assert _capi.STATUS[lib.fna2_bwd(ctypes.byref(big), None)] == "FNA2_E_SHAPE"
    ok = _bwd_varlen(70000, row)
    assert _capi.STATUS[lib.fna2_check_bwd(ctypes.byref(ok))] == "FNA2_OK"
