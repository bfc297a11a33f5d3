"""Writes the committed fixtures in tests/golden (run: python tests/golden/make_golden.py).

* cu_seqlens.json -- the c3 and c5 sequence packings drawn by
  fna2_amd.configs (seed 42) with the length rules the bench records;
* vectors_<case>.npz -- small seeded cases: bf16 inputs (stored as uint16 bit
  patterns), scale / causal / cu_seqlens, and the fp64 CPU oracle's O, LSE and
  the six gradients (float32).  The kernels are checked against these on the
  GPU and the oracle against them on the CPU (a regression guard: the oracle
  itself is pinned by tests/test_oracle.py).

The reference (myAiByMe/FNA2) ships no golden vectors or fixtures: every one
of its tests is a live differential (validate_fna2.py:129-369).
"""
import json
import math
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from fna2_amd import configs  # noqa: E402
from oracle import fna2_oracle as O  # noqa: E402

CASES = {
    # dense causal GQA with a vanilla head, odd length
    "dense_gqa": dict(varlen=False, B=1, H=4, H_KV=2, H_G=3, S=80, D=64, R=16, causal=True,
                      scale=0.125, seed=101),
    # varlen non-causal, ragged, with an empty sequence, d = 128
    "varlen_nc": dict(varlen=True, lengths=[33, 0, 70, 1], H=2, H_KV=2, H_G=2, D=128, R=32,
                      causal=False, scale=1 / math.sqrt(128), seed=202),
}


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def make_case(c):
    g = torch.Generator().manual_seed(c["seed"])
    bf = lambda *s, std=1.0: (torch.randn(*s, generator=g) * std).bfloat16()
    rs = 1 / math.sqrt(c["R"])
    if c["varlen"]:
        T = sum(c["lengths"])
        q, k, v = bf(T, c["H"], c["D"]), bf(T, c["H_KV"], c["D"]), bf(T, c["H_KV"], c["D"])
        rq, rk = bf(T, c["H_G"], c["R"], std=rs), bf(T, c["H_G"], c["R"], std=rs)
        dout = bf(T, c["H"], c["D"])
        cu = torch.tensor([0] + list(np.cumsum(c["lengths"])), dtype=torch.int32)
    else:
        B, S = c["B"], c["S"]
        q, k, v = bf(B, c["H"], S, c["D"]), bf(B, c["H_KV"], S, c["D"]), bf(B, c["H_KV"], S, c["D"])
        rq, rk = bf(B, c["H_G"], S, c["R"], std=rs), bf(B, c["H_G"], S, c["R"], std=rs)
        dout = bf(B, c["H"], S, c["D"])
        cu = None
    gs = torch.randn(c["H_G"], generator=g).float()
    out, lse = O.forward(q, k, v, rq, rk, gs, c["scale"], c["causal"], cu, cu)
    grads = O.backward(dout, q, k, v, rq, rk, gs, out, lse, c["scale"], c["causal"], cu, cu)
    arrs = dict(q=bits(q), k=bits(k), v=bits(v), rq=bits(rq), rk=bits(rk), dout=bits(dout),
                gs=gs.numpy(), scale=np.float64(c["scale"]), causal=np.int32(c["causal"]),
                out=np.asarray(out, np.float32), lse=np.asarray(lse, np.float32))
    for name, x in zip(("dq", "dk", "dv", "drq", "drk", "dgs"), grads):
        arrs[name] = np.asarray(x, np.float32)
    if cu is not None:
        arrs["cu_seqlens"] = cu.numpy()
    return arrs


def main():
    packs = {}
    for name in ("c3", "c5"):
        cfg = configs.get(name)
        packs[name] = {"cu_seqlens": cfg.cu_seqlens().tolist(),
                       "rule": configs.__doc__.split("Length rules")[1].strip()}
    (HERE / "cu_seqlens.json").write_text(json.dumps(packs, indent=1) + "\n")
    for name, c in CASES.items():
        np.savez_compressed(HERE / f"vectors_{name}.npz", **make_case(c))
    print("written:", sorted(p.name for p in HERE.iterdir() if p.suffix in (".json", ".npz")))


if __name__ == "__main__":
    main()
