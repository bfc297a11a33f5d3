"""The custom operators fna2::fwd / fna2::bwd (fna2_amd/ops.py).

CPU: the plan size the fake implementation computes equals the library's
fna2_plan_bytes; fake tensors (no kernel runs) give the outputs' shapes,
dtypes and strides: out in q's layout (also a [B, L, H, D] memory seen as
[B, H, L, D]), fp32 LSE, the plan; make_fx traces flash_naylis_attn into one
fna2.fwd node.
GPU: torch.library.opcheck of both ops; torch.compile(fullgraph=True) of the
forward and backward (no graph break) against the fp64 oracle, dense and
varlen, on the aot_eager backend (tracing, fake tensors and the autograd
registration, without generated kernels).
"""
import ctypes
import importlib
import math

import numpy as np
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import fna2_amd  # noqa: F401  (registers the ops)
from fna2_amd import _capi, ops
from tests import helpers as H

F = importlib.import_module("fna2_amd.flash_naylis_attn")


def test_plan_size_closed_form_matches_library():
    if not _capi.available():
        pytest.skip("libfna2_hip.so not built")
    lib = _capi.lib()
    for tq, tk, n in [(16384, 16384, 64), (1, 5, 1), (32768, 32768, 385), (0, 10, 2),
                      (1000, 2000, 7), (5, 0, 3), (128, 128, 1), (129, 257, 2), (300, 513, 2)]:
        for D, HG, R in [(128, 16, 32), (64, 8, 16), (64, 8, 64), (64, 0, 0), (128, 4, 64)]:
            prob = F._problem(True, n, 0, 0, tq, tk, 16, 16, HG, D, R, True, 0.1)
            prob.cu_seqlens_q = prob.cu_seqlens_k = 0x1000
            assert lib.fna2_plan_bytes(ctypes.byref(prob)) == ops.plan_nbytes(tq, tk, n, D, HG, R), \
                (tq, tk, n, D, HG, R)
    assert ops.plan_nbytes(100, 100, 0) == 0


def test_fake_forward_metadata():
    with FakeTensorMode():
        B, L, Hq, D, R = 2, 300, 4, 128, 32
        mk = lambda *s: torch.empty(*s, device="cuda", dtype=torch.bfloat16)
        # dense, [B, L, H, D] memory as [B, H, L, D] views
        q, k, v = (mk(B, L, Hq, D).transpose(1, 2) for _ in range(3))
        rq, rk = (mk(B, L, Hq, R).transpose(1, 2) for _ in range(2))
        gs = torch.empty(Hq, device="cuda")
        out, lse, plan = torch.ops.fna2.fwd(q, k, v, rq, rk, gs, 0.088, True, None, None, 0, 0)
        assert out.shape == q.shape and out.stride() == q.stride() and out.dtype == q.dtype
        assert lse.shape == (B, Hq, L) and lse.dtype == torch.float32
        assert plan.numel() == 0
        # varlen
        T, N = 700, 5
        qv, kv, vv = mk(T, Hq, D), mk(T, 2, D), mk(T, 2, D)
        rqv, rkv = mk(T, Hq, R), mk(T, Hq, R)
        cu = torch.empty(N + 1, dtype=torch.int32, device="cuda")
        out, lse, plan = torch.ops.fna2.fwd(qv, kv, vv, rqv, rkv, gs, 0.088, True, cu, cu, 300,
                                            300)
        assert out.shape == qv.shape and lse.shape == (T, Hq)
        assert plan.dtype == torch.uint8 and plan.numel() == ops.plan_nbytes(T, T, N, D, Hq, R)
        g = torch.ops.fna2.bwd(mk(T, Hq, D), qv, kv, vv, rqv, rkv, gs, out, lse, plan, 0.088,
                               True, cu, cu, 300, 300)
        assert [tuple(t.shape) for t in g] == [tuple(qv.shape), tuple(kv.shape), tuple(vv.shape),
                                               tuple(rqv.shape), tuple(rkv.shape), (Hq,)]
        g0 = torch.ops.fna2.bwd(mk(T, Hq, D), qv, kv, vv, None, None, None, out, lse, plan,
                                0.088, True, cu, cu, 300, 300)
        assert [t.numel() for t in g0[3:]] == [0, 0, 0]


def test_make_fx_traces_one_fwd_node():
    from torch.fx.experimental.proxy_tensor import make_fx

    def f(q, k, v, rq, rk, gs, cu):
        return F.flash_naylis_attn(q, k, v, rq, rk, gs, None, True, cu, cu, 64, 64)

    with FakeTensorMode():
        mk = lambda *s: torch.empty(*s, device="cuda", dtype=torch.bfloat16)
        args = (mk(100, 2, 64), mk(100, 2, 64), mk(100, 2, 64), mk(100, 2, 16), mk(100, 2, 16),
                torch.empty(2, device="cuda"), torch.empty(3, dtype=torch.int32, device="cuda"))
        gm = make_fx(f, tracing_mode="fake")(*args)
    targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    assert targets.count("fna2.fwd.default") == 1, targets


def _inputs(gpu, varlen):
    if varlen:
        lengths = [130, 1, 64, 257]
        (q, k, v, rq, rk, gs, dout, cu, _) = H.make_varlen(lengths, 4, 128, 2, 4, 32, seed=61)
        return (q, k, v, rq, rk, gs, dout), cu, max(lengths)
    q, k, v, rq, rk, gs, dout = H.make_dense(2, 4, 200, 64, 2, 3, 16, seed=62, layout="bshd")
    return (q, k, v, rq, rk, gs, dout), None, 0


@pytest.mark.gpu
@pytest.mark.parametrize("varlen", [False, True])
def test_opcheck(gpu, varlen):
    (q, k, v, rq, rk, gs, dout), cu, mx = _inputs(gpu, varlen)
    d = lambda t: None if t is None else t.to(gpu)
    cu_g = d(cu)
    args = (d(q), d(k), d(v), d(rq), d(rk), d(gs), 1 / 8, True, cu_g, cu_g, mx, mx)
    print(f"opcheck fna2::fwd varlen={varlen}", flush=True)
    torch.library.opcheck(torch.ops.fna2.fwd.default, args,
                          test_utils=("test_schema", "test_faketensor"))
    out, lse, plan = torch.ops.fna2.fwd(*args)
    bargs = (d(dout), *args[:6], out, lse, plan, 1 / 8, True, cu_g, cu_g, mx, mx)
    torch.library.opcheck(torch.ops.fna2.bwd.default, bargs,
                          test_utils=("test_schema", "test_faketensor"))


@pytest.mark.gpu
@pytest.mark.parametrize("varlen", [False, True])
def test_torch_compile_fullgraph_matches_oracle(gpu, varlen):
    (q, k, v, rq, rk, gs, dout), cu, mx = _inputs(gpu, varlen)
    scale = 1.0 / math.sqrt(q.shape[-1])
    leaves = [t.to(gpu).requires_grad_(True) for t in (q, k, v, rq, rk, gs)]
    cu_g = None if cu is None else cu.to(gpu)

    def fwd(q_, k_, v_, rq_, rk_, gs_):
        return F.flash_naylis_attn(q_, k_, v_, rq_, rk_, gs_, softmax_scale=scale, is_causal=True,
                                   cu_seqlens_q=cu_g, cu_seqlens_k=cu_g, max_seqlen_q=mx,
                                   max_seqlen_k=mx)

    def step(fn):
        out = fn(*leaves)
        return (out.detach(), *torch.autograd.grad(out, leaves, dout.to(gpu)))

    print(f"torch.compile fullgraph varlen={varlen}", flush=True)
    torch._dynamo.reset()
    compiled = torch.compile(fwd, fullgraph=True, backend="aot_eager")
    res = step(compiled)  # the backward runs AOTAutograd's graph (fna2::bwd)
    torch.cuda.synchronize()
    cu_np = None if cu is None else cu.numpy()
    ref_out, _, ref_g = H.oracle_fwd_bwd(q, k, v, rq, rk, gs, dout, scale, True, cu_np, cu_np)
    assert H.max_abs(res[0], ref_out) < H.TOL_OUT
    H.check_grads(res[1:], ref_g)
    # and equal to the eager call bit for bit
    eager = step(fwd)
    for a, b in zip(res, eager):
        assert torch.equal(a, b)
