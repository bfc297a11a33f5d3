"""GPU parity at the benchmark configurations themselves (BASELINE.json c2-c5)
and the reference's own ``large_seq`` validation shape.

Each test runs ``flash_naylis_attn`` forward and backward (through
``torch.autograd``, so the drop-in API and the plan path are the ones
exercised) on the exact inputs ``fna2_amd.configs.make_inputs`` draws for
the config, and compares out, LSE and all six gradients with the fp64
oracle on the same bf16 inputs:

* out: 2e-2 max abs; LSE: 1e-2 max abs (natural-log units);
* dQ, dK, dV, dR_q, dR_k, d_graph_scale: 5e-2 relative norm.

c4 (B1 H32 L16384 d128 r64) runs all 32 heads on the GPU; its heads are
independent (H_KV = H_G = H), so the oracle checks a full-length subset of
them (heads 0 and 31, every one of the 16,384 rows) exactly.  c1 is the
CPU-only fp32 case (tests/test_oracle.py::test_c1_fp32_within_1e4_of_fp64).

The reference validates at its own shapes in validate_fna2.py:129-173
(configs :44-57); ``large_seq`` is B1 H8 S512 D64 H_KV4 H_G4 R32 with R
drawn at std 1 (:67-81).
"""
import importlib
import math

import numpy as np
import pytest
import torch

from fna2_amd import configs
from tests import helpers as H

pytestmark = pytest.mark.gpu


def _fna2():
    return importlib.import_module("fna2_amd.flash_naylis_attn")


def _run_gpu(inp, causal, gpu):
    """flash_naylis_attn forward + autograd backward on the GPU."""
    F = _fna2()
    leaves = [t.to(gpu).detach().requires_grad_(True)
              for t in (inp.q, inp.k, inp.v, inp.r_q, inp.r_k, inp.graph_scale)]
    cu = None if inp.cu_seqlens is None else inp.cu_seqlens.to(gpu)
    kw = {}
    if cu is not None:
        kw = dict(cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=inp.max_seqlen,
                  max_seqlen_k=inp.max_seqlen)
    out = F.flash_naylis_attn(*leaves, softmax_scale=inp.scale, is_causal=causal, **kw)
    grads = torch.autograd.grad(out, leaves, inp.dout.to(gpu))
    # LSE of the same call: the launcher the autograd function runs
    with torch.no_grad():
        if cu is None:
            _, lse = F._fna2_forward(*[t.detach() for t in leaves], inp.scale, causal)
        else:
            _, lse = F._fna2_forward_varlen(*[t.detach() for t in leaves], cu, cu,
                                            inp.max_seqlen, inp.max_seqlen, inp.scale, causal)
    torch.cuda.synchronize()
    return out.detach(), lse, [g.detach() for g in grads]


def _check_config(name, gpu, heads=None):
    cfg = configs.get(name)
    inp = configs.make_inputs(cfg)
    print(f"config {name}: {cfg.desc}; tokens {cfg.total}, seqs {len(cfg.seq_lengths())}",
          flush=True)
    out, lse, grads = _run_gpu(inp, cfg.causal, gpu)
    cu = None if inp.cu_seqlens is None else inp.cu_seqlens.numpy()
    args = [inp.q, inp.k, inp.v, inp.r_q, inp.r_k, inp.graph_scale, inp.dout]
    if heads is not None:  # dense [B, H, S, *] views: a head subset, every row
        sel = lambda t: t[:, heads]
        args = [sel(t) for t in args[:5]] + [inp.graph_scale[heads], sel(inp.dout)]
        out, lse = out[:, heads], lse[:, heads]
        grads = [sel(g) for g in grads[:5]] + [grads[5][heads]]
    q, k, v, rq, rk, gs, dout = args
    ref_out, ref_lse, ref_g = H.oracle_fwd_bwd(q, k, v, rq, rk, gs, dout, inp.scale, cfg.causal,
                                               cu, cu)
    e_out = H.check_out(out, lse, ref_out, ref_lse)
    errs = H.check_grads(grads, ref_g)
    print(f"config {name}: out max abs {e_out:.2e}; grad rel-norm "
          + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)


def test_config_c2_dense_causal(gpu):
    _check_config("c2", gpu)


def test_config_c3_varlen_causal(gpu):
    _check_config("c3", gpu)


def test_config_c4_long_context_heads_0_and_31(gpu):
    _check_config("c4", gpu, heads=[0, 31])


def test_config_c5_skewed_varlen_noncausal(gpu):
    _check_config("c5", gpu)


def test_reference_large_seq_config(gpu):
    """validate_fna2.py:53-56: B1 H8 S512 D64 H_KV4 H_G4 R32, R ~ N(0, 1)."""
    F = _fna2()
    q, k, v, rq, rk, gs, dout = H.make_dense(1, 8, 512, 64, 4, 4, 32, seed=42, r_std=1.0)
    scale = 1.0 / math.sqrt(64)
    print("large_seq B1 H8 S512 D64 HKV4 HG4 R32", flush=True)
    leaves = [t.to(gpu).requires_grad_(True) for t in (q, k, v, rq, rk, gs)]
    out = F.flash_naylis_attn(*leaves, softmax_scale=scale, is_causal=True)
    grads = torch.autograd.grad(out, leaves, dout.to(gpu))
    _, lse = F._fna2_forward(*[t.detach() for t in leaves], scale, True)
    torch.cuda.synchronize()
    ref_out, ref_lse, ref_g = H.oracle_fwd_bwd(q, k, v, rq, rk, gs, dout, scale, True)
    H.check_out(out, lse, ref_out, ref_lse)
    H.check_grads(grads, ref_g)
