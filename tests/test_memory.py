"""The reference's memory test (T5, FNA2/validate_fna2.py:376-418) on the GPU.

The reference asserts that FNA2's peak memory (torch.cuda.max_memory_allocated)
is below that of the eager path with a materialised [B, H, S, S] bias, at its
validation configurations (60m, 220m, large_seq: validate_fna2.py:44-57).
Here the same comparison runs for the forward and for forward + backward,
as the peak allocated on top of the inputs during the call.

The eager side restates the reference's materialised-bias path
(validate_fna2.py:84-112: repeat K/V per group, bias gs * Rq Rk^T in fp32
cast to bf16, causal -inf, softmax attention) in bf16 with every matmul on
contiguous operands, and its backward by hand (dP = dO V^T, dS = P (dP -
delta), dV = P^T dO, dQ = scale dS K, dK = scale dS^T Q, dRq / dRk from dS):
the [B, H, S, S] scores, probabilities, dP and dS it holds are what the
reference's eager path allocates.  (torch's own bf16 attention and autograd
would run batched products on transposed views, which this GPU pool has seen
fault.)
"""
import math

import pytest
import torch

from tests import helpers as H

pytestmark = pytest.mark.gpu

# validate_fna2.py:44-57
CONFIGS = {
    "60m": dict(B=2, H=8, S=128, D=64, H_KV=4, H_G=4, R=32),
    "220m": dict(B=2, H=12, S=256, D=64, H_KV=4, H_G=8, R=32),
    "large_seq": dict(B=1, H=8, S=512, D=64, H_KV=4, H_G=4, R=32),
}


def _eager_forward(q, k, v, rq, rk, gs, scale):
    B, Hq, S, D = q.shape
    G = Hq // k.shape[1]
    ke = k.repeat_interleave(G, dim=1)
    ve = v.repeat_interleave(G, dim=1)
    H_G = rq.shape[1]
    bias = torch.zeros(B, Hq, S, S, dtype=torch.float32, device=q.device)
    bias[:, :H_G] = torch.matmul(rq.float(), rk.float().transpose(-2, -1).contiguous()) * \
        gs.float().view(1, H_G, 1, 1)
    bias = bias.to(q.dtype)
    bias = bias + torch.triu(torch.full((S, S), float("-inf"), device=q.device, dtype=q.dtype),
                             diagonal=1)
    s = torch.matmul(q, ke.transpose(-2, -1).contiguous()) * scale + bias
    p = torch.softmax(s.float(), dim=-1).to(q.dtype)
    return torch.matmul(p, ve), (ke, ve, p)


def _eager_backward(dout, q, k, rq, rk, gs, out, saved, scale):
    ke, ve, p = saved
    G = q.shape[1] // k.shape[1]
    H_G = rq.shape[1]
    dp = torch.matmul(dout, ve.transpose(-2, -1).contiguous())
    delta = (dout.float() * out.float()).sum(-1, keepdim=True)
    ds = (p.float() * (dp.float() - delta)).to(q.dtype)
    dv = torch.matmul(p.transpose(-2, -1).contiguous(), dout)
    dq = torch.matmul(ds, ke) * scale
    dk = torch.matmul(ds.transpose(-2, -1).contiguous(), q) * scale
    dsg = ds[:, :H_G].float()
    drq = torch.matmul(dsg, rk.float()) * gs.float().view(1, H_G, 1, 1)
    drk = torch.matmul(dsg.transpose(-2, -1).contiguous(), rq.float()) * gs.float().view(1, H_G, 1, 1)
    B, Hkv, S, D = k.shape
    dk = dk.view(B, Hkv, G, S, D).sum(2)
    dv = dv.view(B, Hkv, G, S, D).sum(2)
    return dq, dk, dv, drq.to(q.dtype), drk.to(q.dtype)


def _peak_over_base(fn):
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    res = fn()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - base
    del res
    return peak


@pytest.mark.parametrize("name", list(CONFIGS))
def test_fna2_peak_memory_below_materialised_bias(gpu, name):
    import importlib
    F = importlib.import_module("fna2_amd.flash_naylis_attn")
    c = CONFIGS[name]
    # R ~ N(0, 1) and graph_scale ~ N(0, 1) as validate_fna2.py:67-81 draws them
    q, k, v, rq, rk, gs, dout = H.make_dense(c["B"], c["H"], c["S"], c["D"], c["H_KV"], c["H_G"],
                                             c["R"], seed=42, r_std=1.0, device=gpu)
    scale = 1.0 / math.sqrt(c["D"])
    print(f"T5 {name}: {c}", flush=True)

    def eager_fwd():
        with torch.no_grad():
            return _eager_forward(q, k, v, rq, rk, gs, scale)[0]

    def eager_fwd_bwd():
        with torch.no_grad():
            out, saved = _eager_forward(q, k, v, rq, rk, gs, scale)
            return _eager_backward(dout, q, k, rq, rk, gs, out, saved, scale)

    def fna2_fwd():
        with torch.no_grad():
            return F.flash_naylis_attn(q, k, v, rq, rk, gs, softmax_scale=scale, is_causal=True)

    def fna2_fwd_bwd():
        leaves = [t.detach().requires_grad_(True) for t in (q, k, v, rq, rk, gs)]
        out = F.flash_naylis_attn(*leaves, softmax_scale=scale, is_causal=True)
        return torch.autograd.grad(out, leaves, dout)

    m = {key: _peak_over_base(fn) / 2**20 for key, fn in
         (("eager_fwd", eager_fwd), ("fna2_fwd", fna2_fwd), ("eager_fwd_bwd", eager_fwd_bwd),
          ("fna2_fwd_bwd", fna2_fwd_bwd))}
    bias_mb = c["B"] * c["H"] * c["S"] ** 2 * 2 / 2**20
    print(f"T5 {name}: peak MB above the inputs " +
          ", ".join(f"{k_} {v_:.2f}" for k_, v_ in m.items()) +
          f"; one bf16 [B, H, S, S] tensor = {bias_mb:.2f} MB", flush=True)
    assert m["fna2_fwd"] < m["eager_fwd"], m
    assert m["fna2_fwd_bwd"] < m["eager_fwd_bwd"], m
    # FNA2 holds no O(S^2) tensor: its forward peak stays below one [B, H, S, S]
    # bf16 tensor once that tensor outweighs the O(S) outputs.
    if c["S"] >= 512:
        assert m["fna2_fwd"] < bias_mb, m
