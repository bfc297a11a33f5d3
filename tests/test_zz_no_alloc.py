"""The allocation-free forward (fna2_fwd_noalloc) against fna2_fwd.

fna2_fwd_noalloc keeps the varlen tile list in a static 1 MiB device array
instead of the caller's workspace.  On the GPU, two calls in a row through
the C ABI (the second with a smaller input) must equal fna2_fwd bit for bit
(the same kernels); on the CPU, a problem whose tile list would not fit is
refused before any GPU work.
"""
import ctypes
import math

import pytest
import torch

from fna2_amd import _capi
from tests import helpers as H


def _fwd_args(F, q, k, v, rq, rk, gs, cu, max_len, out, lse):
    prob = F._problem(True, cu.shape[0] - 1, max_len, max_len, q.shape[0], k.shape[0], q.shape[1],
                      k.shape[1], rq.shape[1], q.shape[2], rq.shape[2], True,
                      1.0 / math.sqrt(q.shape[2]), cu, cu)
    return prob, _capi.FwdArgs(prob, F._view3(q), F._view3(k), F._view3(v), F._view3(rq),
                               F._view3(rk), gs.data_ptr(), F._view3(out), F._view3(lse), None, 0,
                               None, None, 0)


def _run(gpu, lengths, seed):
    import importlib
    F = importlib.import_module("fna2_amd.flash_naylis_attn")
    lib = _capi.lib()
    (q, k, v, rq, rk, gs, _, cu, _) = H.make_varlen(lengths, 4, 128, 2, 4, 32, seed=seed,
                                                    device=gpu)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    outs = []
    for noalloc in (False, True):
        out = torch.full_like(q, float("nan"))
        lse = torch.full(q.shape[:2], float("nan"), device=gpu)
        prob, args = _fwd_args(F, q, k, v, rq, rk, gs, cu, max(lengths), out, lse)
        if noalloc:
            st = lib.fna2_fwd_noalloc(ctypes.byref(args), stream)
        else:
            nbytes = lib.fna2_fwd_workspace_bytes(ctypes.byref(prob))
            ws = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
            args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes
            st = lib.fna2_fwd(ctypes.byref(args), stream)
        _capi.raise_for(st, "fna2_fwd_noalloc" if noalloc else "fna2_fwd")
        torch.cuda.synchronize()
        outs.append((out, lse))
    (o0, l0), (o1, l1) = outs
    assert torch.equal(o0, o1), "out differs from fna2_fwd"
    assert torch.equal(l0, l1), "lse differs from fna2_fwd"
    assert torch.isfinite(o1.float()).all()


@pytest.mark.gpu
def test_noalloc_forward_equals_fna2_fwd(gpu):
    print("fna2_fwd_noalloc: 5 sequences, then a smaller pack of 3", flush=True)
    _run(gpu, [300, 17, 129, 64, 500], seed=51)
    _run(gpu, [40, 128, 9], seed=52)


def test_noalloc_refuses_problems_beyond_its_scratch():
    """A pack whose tile list exceeds the static scratch is refused with
    FNA2_E_SCRATCH before any GPU call (fake pointers, host-only checks)."""
    if not _capi.available():
        pytest.skip("libfna2_hip.so not built")
    lib = _capi.lib()
    cap = lib.fna2_fwd_noalloc_max_bytes()
    assert cap == 1 << 20
    fake = 0x10000
    t = _capi.Tensor(fake, 0, 1024, 128)
    for total, ok in ((2_000_000, True), (8_000_000, False)):
        prob = _capi.Problem(1, 1, 1000, 0, 0, total, total, 8, 8, 0, 128, 0, 1, 0.088, fake, fake)
        need = lib.fna2_fwd_workspace_bytes(ctypes.byref(prob))
        assert (need <= cap) == ok
        if ok:
            continue
        args = _capi.FwdArgs(prob, t, t, t, _capi.empty_tensor(), _capi.empty_tensor(), None, t,
                             _capi.Tensor(fake, 0, 8, 1), None, 0, None, None, 0)
        st = lib.fna2_fwd_noalloc(ctypes.byref(args), None)
        assert _capi.STATUS[st] == "FNA2_E_SCRATCH"
        assert b"allocation-free" in lib.fna2_status_string(st)
