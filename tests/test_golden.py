"""Committed fixtures (tests/golden, written by tests/golden/make_golden.py).

CPU: the c3/c5 packings that fna2_amd.configs draws equal the committed
cu_seqlens (the length rules are pinned), and the oracle reproduces the
committed vectors.  GPU: the HIP kernels against the committed vectors at the
bf16 tolerances.
"""
import importlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from fna2_amd import configs
from oracle import fna2_oracle as O

from . import helpers as H

GOLD = Path(__file__).resolve().parent / "golden"
CASES = ("dense_gqa", "varlen_nc")
GRADS = ("dq", "dk", "dv", "drq", "drk", "dgs")


def load(name):
    z = np.load(GOLD / f"vectors_{name}.npz")  # allow_pickle stays False
    t = {k: z[k] for k in z.files}
    for k in ("q", "k", "v", "rq", "rk", "dout"):
        t[k] = torch.from_numpy(t[k].view(np.int16).copy()).view(torch.bfloat16)
    t["gs"] = torch.from_numpy(t["gs"])
    t["cu"] = torch.from_numpy(t["cu_seqlens"]) if "cu_seqlens" in t else None
    return t


def test_packings_match_fixture():
    packs = json.loads((GOLD / "cu_seqlens.json").read_text())
    for name, total, n in (("c3", 16384, 64), ("c5", 32768, 385)):
        cu = configs.get(name).cu_seqlens().tolist()
        assert cu == packs[name]["cu_seqlens"], name
        assert cu[0] == 0 and cu[-1] == total and len(cu) == n + 1
        lens = np.diff(cu)
        if name == "c3":
            assert lens.min() >= 64 and lens.max() <= 512
        else:
            assert lens[0] == 8192 and lens[1:].min() >= 16 and lens[1:].max() <= 128


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_vectors(name):
    t = load(name)
    s, c = float(t["scale"]), bool(t["causal"])
    out, lse = O.forward(t["q"], t["k"], t["v"], t["rq"], t["rk"], t["gs"], s, c, t["cu"], t["cu"])
    np.testing.assert_allclose(np.asarray(out, np.float32), t["out"], atol=1e-6, rtol=1e-5)
    np.testing.assert_allclose(np.asarray(lse, np.float32), t["lse"], atol=1e-5, rtol=1e-6)
    grads = O.backward(t["dout"], t["q"], t["k"], t["v"], t["rq"], t["rk"], t["gs"], out, lse,
                       s, c, t["cu"], t["cu"])
    for g, name_g in zip(grads, GRADS):
        np.testing.assert_allclose(np.asarray(g, np.float32), t[name_g], atol=1e-5, rtol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_kernels_match_vectors(gpu, name):
    F = importlib.import_module("fna2_amd.flash_naylis_attn")
    t = load(name)
    s, c = float(t["scale"]), bool(t["causal"])
    d = {k: t[k].to(gpu) for k in ("q", "k", "v", "rq", "rk", "dout", "gs")}
    if t["cu"] is not None:
        cu = t["cu"].to(gpu)
        mx = int(np.diff(t["cu_seqlens"]).max())
        out, lse = F._fna2_forward_varlen(d["q"], d["k"], d["v"], d["rq"], d["rk"], d["gs"], cu,
                                          cu, mx, mx, s, is_causal=c)
        grads = F._fna2_backward_varlen(d["dout"], d["q"], d["k"], d["v"], d["rq"], d["rk"],
                                        d["gs"], out, lse, cu, cu, mx, mx, s, is_causal=c)
    else:
        out, lse = F._fna2_forward(d["q"], d["k"], d["v"], d["rq"], d["rk"], d["gs"], s, c)
        grads = F._fna2_backward(d["dout"], d["q"], d["k"], d["v"], d["rq"], d["rk"], d["gs"],
                                 out, lse, s, c)
    H.check_out(out, lse, t["out"], t["lse"])
    H.check_grads(grads, [t[g] for g in GRADS])
