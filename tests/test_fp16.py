"""fp16 q/k/v through the drop-in API (GPU).

The reference's kernels are generic over the q/k/v dtype: P is cast to
v.dtype (FNA2/flash_naylis_attn.py:187), the output to Out's dtype (:201),
dO to v.dtype and dS to q.dtype in the backward (:522-529); only the ranks
must be bf16 (:1419-1420).  Here the head-dim chain, P and dS run on the
fp16 MFMA and the rank chain on the bf16 one, into the same fp32
accumulators.

Each case draws fp32 inputs from a seed and rounds q, k, v and dO to fp16
(r_q, r_k to bf16).  The fp16 path is checked against the fp64 oracle on
those same fp16 inputs, within the north-star bars (out 2e-2 max abs,
gradients 5e-2 relative norm).  Because a kernel that rounded P, dS or its
outputs to bf16 would also pass those bars, each case also runs the bf16
path on the same draws rounded to bf16 and requires the fp16 path's error
to be at most half the bf16 path's: fp16 keeps 3 more mantissa bits, so its
rounding error is about 8 times smaller.
"""
import importlib
import math

import numpy as np
import pytest
import torch

from tests import helpers as H

pytestmark = pytest.mark.gpu


def _fna2():
    return importlib.import_module("fna2_amd.flash_naylis_attn")


def _draw_dense(B, Hq, S, D, H_KV, H_G, R, seed):
    g = torch.Generator().manual_seed(seed)
    r_std = 1.0 / math.sqrt(R) if R else 1.0
    base = dict(q=torch.randn(B, Hq, S, D, generator=g),
                k=torch.randn(B, H_KV, S, D, generator=g),
                v=torch.randn(B, H_KV, S, D, generator=g))
    rq = (torch.randn(B, H_G, S, R, generator=g) * r_std).bfloat16() if H_G else None
    rk = (torch.randn(B, H_G, S, R, generator=g) * r_std).bfloat16() if H_G else None
    gs = torch.randn(H_G, generator=g).float() if H_G else None
    base["dout"] = torch.randn(B, Hq, S, D, generator=g)
    return base, rq, rk, gs


def _draw_varlen(lengths, Hq, D, H_KV, H_G, R, seed):
    g = torch.Generator().manual_seed(seed)
    T = sum(lengths)
    r_std = 1.0 / math.sqrt(R) if R else 1.0
    base = dict(q=torch.randn(T, Hq, D, generator=g), k=torch.randn(T, H_KV, D, generator=g),
                v=torch.randn(T, H_KV, D, generator=g))
    rq = (torch.randn(T, H_G, R, generator=g) * r_std).bfloat16() if H_G else None
    rk = (torch.randn(T, H_G, R, generator=g) * r_std).bfloat16() if H_G else None
    gs = torch.randn(H_G, generator=g).float() if H_G else None
    base["dout"] = torch.randn(T, Hq, D, generator=g)
    cu = torch.tensor([0] + list(np.cumsum(lengths)), dtype=torch.int32)
    return base, rq, rk, gs, cu


def _errors(gpu, run, base, rq, rk, gs, dtype, scale, causal, cu=None):
    """Run one path on `base` rounded to `dtype`; return (out err, {grad: err})."""
    q, k, v, dout = (base[n].to(dtype) for n in ("q", "k", "v", "dout"))
    dev = [t.to(gpu) if t is not None else None for t in (q, k, v, rq, rk, gs, dout)]
    out, lse, grads = run(dev)
    torch.cuda.synchronize()
    assert out.dtype == dtype and all(g.dtype == dtype for g in grads[:3])
    if rq is not None:
        assert grads[3].dtype == torch.bfloat16 and grads[4].dtype == torch.bfloat16
    cu_np = None if cu is None else cu.numpy()
    ref_out, ref_lse, ref_g = H.oracle_fwd_bwd(q, k, v, rq, rk, gs, dout, scale, causal,
                                               cu_np, cu_np)
    e_out = H.check_out(out, lse, ref_out, ref_lse)
    e_g = H.check_grads(grads, ref_g)
    return e_out, e_g


def _compare(e16, e_bf):
    (o16, g16), (obf, gbf) = e16, e_bf
    print(f"fp16 out {o16:.2e} (bf16 {obf:.2e}); grads " +
          ", ".join(f"{k} {g16[k]:.2e} ({gbf[k]:.2e})" for k in g16), flush=True)
    assert o16 <= 0.5 * obf, (o16, obf)
    for name in ("dq", "dk", "dv"):
        assert g16[name] <= 0.5 * gbf[name], (name, g16[name], gbf[name])


@pytest.mark.parametrize("D,R,H_KV,H_G,causal", [(128, 32, 4, 4, True), (64, 16, 2, 3, True),
                                                (64, 64, 4, 4, False), (128, 0, 2, 0, True)])
def test_fp16_dense_against_oracle(gpu, D, R, H_KV, H_G, causal):
    F = _fna2()
    B, Hq, S = 2, 4, 200
    base, rq, rk, gs = _draw_dense(B, Hq, S, D, H_KV, H_G, R, seed=D + R + H_G)
    scale = 1.0 / math.sqrt(D)
    print(f"fp16 dense D{D} R{R} HKV{H_KV} HG{H_G} causal={causal}", flush=True)

    def run(t):
        q, k, v, rq_, rk_, gs_, dout = t
        out, lse = F._fna2_forward(q, k, v, rq_, rk_, gs_, scale, causal)
        grads = F._fna2_backward(dout, q, k, v, rq_, rk_, gs_, out, lse, scale, causal)
        return out, lse, grads

    e16 = _errors(gpu, run, base, rq, rk, gs, torch.float16, scale, causal)
    ebf = _errors(gpu, run, base, rq, rk, gs, torch.bfloat16, scale, causal)
    _compare(e16, ebf)


@pytest.mark.parametrize("D,R,causal", [(128, 32, True), (128, 32, False), (64, 16, True),
                                        (64, 64, False)])
def test_fp16_varlen_against_oracle(gpu, D, R, causal):
    F = _fna2()
    lengths = [300, 1, 0, 129, 513, 64]
    Hq, H_KV, H_G = 4, 2, 3
    base, rq, rk, gs, cu = _draw_varlen(lengths, Hq, D, H_KV, H_G, R, seed=7 * D + R)
    scale = 1.0 / math.sqrt(D)
    mx = max(lengths)
    print(f"fp16 varlen D{D} R{R} causal={causal} lengths={lengths}", flush=True)

    def run(t):
        q, k, v, rq_, rk_, gs_, dout = t
        c = cu.to(gpu)
        out, lse = F._fna2_forward_varlen(q, k, v, rq_, rk_, gs_, c, c, mx, mx, scale, causal)
        grads = F._fna2_backward_varlen(dout, q, k, v, rq_, rk_, gs_, out, lse, c, c, mx, mx,
                                        scale, causal)
        return out, lse, grads

    e16 = _errors(gpu, run, base, rq, rk, gs, torch.float16, scale, causal, cu)
    ebf = _errors(gpu, run, base, rq, rk, gs, torch.bfloat16, scale, causal, cu)
    _compare(e16, ebf)


def test_fp16_through_the_autograd_api(gpu):
    """flash_naylis_attn with fp16 leaves: fp16 output and q/k/v gradients,
    bf16 rank gradients, graph_scale's gradient in its dtype; the values equal
    the launchers' (varlen, plan path)."""
    F = _fna2()
    lengths = [77, 256, 31]
    base, rq, rk, gs, cu = _draw_varlen(lengths, 4, 128, 4, 4, 32, seed=3)
    c = cu.to(gpu)
    leaves = [base["q"].half(), base["k"].half(), base["v"].half(), rq, rk, gs]
    leaves = [t.to(gpu).requires_grad_(True) for t in leaves]
    dout = base["dout"].half().to(gpu)
    print("fp16 autograd varlen", flush=True)
    out = F.flash_naylis_attn(*leaves, softmax_scale=0.08, is_causal=True, cu_seqlens_q=c,
                              cu_seqlens_k=c, max_seqlen_q=256, max_seqlen_k=256)
    grads = torch.autograd.grad(out, leaves, dout)
    assert out.dtype == torch.float16
    assert [g.dtype for g in grads] == [torch.float16] * 3 + [torch.bfloat16] * 2 + [torch.float32]
    o2, lse = F._fna2_forward_varlen(*[t.detach() for t in leaves], c, c, 256, 256, 0.08, True)
    g2 = F._fna2_backward_varlen(dout, *[t.detach() for t in leaves], o2, lse, c, c, 256, 256,
                                 0.08, True)
    torch.cuda.synchronize()
    assert torch.equal(out, o2)
    for a, b in zip(grads, g2):
        assert torch.equal(a, b)


def test_fp16_rejects_mixed_dtypes(gpu):
    F = _fna2()
    q = torch.zeros(1, 2, 64, 64, dtype=torch.float16, device=gpu)
    k = torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(AssertionError):
        F._fna2_forward(q, k, k, None, None, None, 0.125, True)
    rq = torch.zeros(1, 2, 64, 32, dtype=torch.float16, device=gpu)
    gs = torch.ones(2, device=gpu)
    with pytest.raises(AssertionError):
        F._fna2_forward(q, q, q, rq, rq, gs, 0.125, True)
