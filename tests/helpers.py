"""Shared helpers for the parity tests (not collected by pytest)."""
from __future__ import annotations

import math

import numpy as np
import torch

from oracle import fna2_oracle as oracle

# Tolerances stated by the north star (bf16 path) against the fp64 oracle
# evaluated on the same bf16 inputs.
TOL_OUT = 2e-2        # max abs, bf16 outputs
TOL_GRAD = 5e-2       # relative norm, bf16 gradients
TOL_LSE = 1e-2        # max abs, fp32 LSE (natural log units)


def max_abs(a, b) -> float:
    a = a.detach().double().cpu().numpy() if hasattr(a, "detach") else np.asarray(a, np.float64)
    b = b.detach().double().cpu().numpy() if hasattr(b, "detach") else np.asarray(b, np.float64)
    if a.size == 0:
        return 0.0
    return float(np.max(np.abs(a - b)))


def rel_norm(got, ref, floor: float = 1e-3) -> float:
    """||got - ref|| / max(||ref||, floor * sqrt(n)).

    The floor keeps the measure meaningful where the exact gradient vanishes
    (e.g. dQ of a one-token causal sequence is exactly 0 up to the 1e-6
    normaliser): there it bounds the RMS error by ``floor * tol``.
    """
    got = got.detach().double().cpu().numpy() if hasattr(got, "detach") else np.asarray(got, np.float64)
    ref = ref.detach().double().cpu().numpy() if hasattr(ref, "detach") else np.asarray(ref, np.float64)
    if ref.size == 0:
        return 0.0
    den = max(np.linalg.norm(ref.ravel()), floor * np.sqrt(ref.size))
    num = np.linalg.norm((got - ref).ravel())
    return float(num / den)


def make_dense(B, H, S, D, H_KV, H_G, R, seed=0, Sk=None, r_std=None, gs=None, device="cpu",
               layout="bhsd"):
    """Seeded bf16 dense inputs [B,H,S,D]; layout 'bshd' returns transposed views."""
    g = torch.Generator().manual_seed(seed)
    Sk = S if Sk is None else Sk
    r_std = 1.0 / math.sqrt(max(R, 1)) if r_std is None else r_std

    def draw(b, h, s, f, std=1.0):
        if layout == "bshd":
            return (torch.randn(b, s, h, f, generator=g) * std).bfloat16().transpose(1, 2)
        return (torch.randn(b, h, s, f, generator=g) * std).bfloat16()

    q = draw(B, H, S, D)
    k = draw(B, H_KV, Sk, D)
    v = draw(B, H_KV, Sk, D)
    rq = draw(B, H_G, S, R, r_std) if H_G else None
    rk = draw(B, H_G, Sk, R, r_std) if H_G else None
    if gs is None:
        gsv = torch.randn(H_G, generator=g).float() if H_G else None
    else:
        gsv = torch.full((H_G,), float(gs)) if H_G else None
    dout = draw(B, H, S, D)
    f = (lambda t: None if t is None else t.to(device))
    return tuple(f(t) for t in (q, k, v, rq, rk, gsv, dout))


def make_varlen(lengths, H, D, H_KV, H_G, R, seed=0, lengths_k=None, r_std=None, gs=None,
                device="cpu"):
    g = torch.Generator().manual_seed(seed)
    lengths_k = lengths if lengths_k is None else lengths_k
    T, Tk = sum(lengths), sum(lengths_k)
    r_std = 1.0 / math.sqrt(max(R, 1)) if r_std is None else r_std
    draw = lambda *s, std=1.0: (torch.randn(*s, generator=g) * std).bfloat16()
    q = draw(T, H, D)
    k = draw(Tk, H_KV, D)
    v = draw(Tk, H_KV, D)
    rq = draw(T, H_G, R, std=r_std) if H_G else None
    rk = draw(Tk, H_G, R, std=r_std) if H_G else None
    if gs is None:
        gsv = torch.randn(H_G, generator=g).float() if H_G else None
    else:
        gsv = torch.full((H_G,), float(gs)) if H_G else None
    dout = draw(T, H, D)
    cu_q = torch.tensor([0] + list(np.cumsum(lengths)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(lengths_k)), dtype=torch.int32)
    f = (lambda t: None if t is None else t.to(device))
    return tuple(f(t) for t in (q, k, v, rq, rk, gsv, dout, cu_q, cu_k))


def oracle_fwd_bwd(q, k, v, rq, rk, gs, dout, scale, causal, cu_q=None, cu_k=None,
                   backward=True):
    out, lse = oracle.forward(q, k, v, rq, rk, gs, scale, causal, cu_q, cu_k)
    if not backward:
        return out, lse, None
    grads = oracle.backward(dout, q, k, v, rq, rk, gs, out, lse, scale, causal, cu_q, cu_k)
    return out, lse, grads


def check_out(out, lse, ref_out, ref_lse, tol=TOL_OUT, tol_lse=TOL_LSE):
    e_out = max_abs(out, ref_out)
    assert e_out < tol, f"out max abs err {e_out:.3e} >= {tol}"
    if lse is not None:
        l = lse.detach().double().cpu().numpy()
        r = np.asarray(ref_lse, np.float64)
        fin = np.isfinite(r)
        assert np.array_equal(np.isfinite(l), fin), "LSE finiteness differs"
        e_lse = float(np.max(np.abs(l[fin] - r[fin]))) if fin.any() else 0.0
        assert e_lse < tol_lse, f"lse max abs err {e_lse:.3e} >= {tol_lse}"
    return e_out


def check_grads(got, ref, tol=TOL_GRAD):
    names = ("dq", "dk", "dv", "drq", "drk", "dgs")
    errs = {}
    for name, g, r in zip(names, got, ref):
        if r is None or np.asarray(r).size == 0:
            assert g is None or g.numel() == 0, f"{name}: expected no gradient"
            continue
        assert g is not None, f"{name}: missing gradient"
        e = rel_norm(g, r)
        errs[name] = e
        assert e < tol, f"{name} rel-norm err {e:.3e} >= {tol}"
    return errs
