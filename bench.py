#!/usr/bin/env python3
"""bench.py — FlashNaylisAttention-2 forward+backward on one MI355X.

Default workload (the headline metric of BASELINE.json): config c3, a varlen
pack of 16384 tokens in 64 causal sequences, H=16, d=128, r=32, bf16.  One
"step" is one pass of the hot path over that batch: ``flash_naylis_attn``
forward, then ``torch.autograd.grad`` of the output against dO (dQ, dK, dV,
dR_q, dR_k, d_graph_scale).  Inputs are resident in HBM before timing starts.

Printed: ONE JSON line with the fwd+bwd throughput (``value``, TFLOP/s of
algorithmic FLOPs: 4d+2r forward and 10d+6r backward per visible
(query, key) pair per head), the forward-only throughput, fractions of the
bf16 dense MFMA peak, a ``roofline`` object for the kernel that takes the
most time per step (per-launch durations from HIP events recorded by the
library on the launch stream during the timed steps), and a ``cpu_baseline``
object: the reference's eager path (SDPA + materialised bias, restated in
``oracle/eager_reference.py``) timed on this host's cores on a bounded
sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3]
"""
from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import statistics
import sys
import time

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA (256 CUs x 2.4 GHz x 4096 FLOP/clk)
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
METRIC = "fwd+bwd TFLOP/s & % bf16 MFMA peak, varlen 16k-token pack H=16 d=128 r=32"


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c3", choices=["c2", "c3", "c4", "c5"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="approximate CPU-baseline budget (seconds)")
    ap.add_argument("--no-flush", action="store_true",
                    help="skip the cache-flushed measurement")
    return ap.parse_args()


def kernel_bytes(cfg, name):
    """Compulsory HBM bytes one launch of kernel `name` must move (each tensor once)."""
    T, H, D, R = cfg.total, cfg.H, cfg.D, cfg.R
    H_KV = H  # configs: H_KV = H_G = H
    row = lambda heads, feat, es=2: T * heads * feat * es
    q = row(H, D)
    kv = row(H_KV, D)
    r = row(H, R)
    lse = row(H, 1, 4)
    if name == "fwd":   # read Q K V Rq Rk, write O LSE
        return q + 2 * kv + 2 * r + q + lse
    if name == "dkdv":  # read Q K V dO Rq Rk LSE delta, write dK dV dRk
        return q + 2 * kv + q + 2 * r + 2 * lse + 2 * kv + r
    if name == "dq":    # read Q K V O dO Rq Rk LSE, write dQ dRq delta
        return q + 2 * kv + 2 * q + 2 * r + 2 * lse + q + r
    raise KeyError(name)


def kernel_flops(cfg, name):
    """Algorithmic FLOPs of one launch: fwd 4d+2r; dK/dV kernel 8d+4r (S, dP, dV, dK,
    dRk); dQ kernel 2d+2r (dQ, dRq) per visible pair per head (sum = bwd 10d+6r)."""
    pairs = sum(n * (n + 1) // 2 if cfg.causal else n * n for n in cfg.seq_lengths()) * cfg.H
    per = {"fwd": 4 * cfg.D + 2 * cfg.R, "dkdv": 8 * cfg.D + 4 * cfg.R,
           "dq": 2 * cfg.D + 2 * cfg.R}[name]
    return pairs * per


def cpu_baseline(cfg, inp, budget_s):
    """Time the eager restatement (fwd+bwd) on a bounded sample on the host cores."""
    import torch

    from oracle import eager_reference as ER

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    lengths = cfg.seq_lengths()
    q, k, v, rq, rk, gs, dout = (t.detach().cpu() for t in (inp.q, inp.k, inp.v, inp.r_q,
                                                             inp.r_k, inp.graph_scale, inp.dout))

    def run(nseq):
        if cfg.varlen:
            T = sum(lengths[:nseq])
            leaves = [t[:T].clone().requires_grad_(True) for t in (q, k, v, rq, rk)]
            g = gs.clone().requires_grad_(True)
            cu = torch.tensor([0] + list(__import__("itertools").accumulate(lengths[:nseq])))
            out = ER.sdpa_reference_varlen(*leaves, g, cu, cu, inp.scale, cfg.causal)
            torch.autograd.grad(out, leaves + [g], dout[:T])
        else:
            leaves = [t[:nseq].clone().requires_grad_(True) for t in (q, k, v, rq, rk)]
            g = gs.clone().requires_grad_(True)
            out = ER.sdpa_reference(*leaves, g, inp.scale, cfg.causal)
            torch.autograd.grad(out, leaves + [g], dout[:nseq])

    # Size the sample: grow the sequence count until one pass takes ~budget/4.
    n, t1 = 1, 0.0
    nmax = len(lengths)
    while True:
        t0 = time.perf_counter()
        run(n)
        t1 = time.perf_counter() - t0
        if t1 >= budget_s / 4 or n >= nmax:
            break
        n = min(nmax, max(n + 1, int(n * min(4.0, (budget_s / 4) / max(t1, 1e-3)))))
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run(n)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    sub = type(cfg)(**{**cfg.__dict__})
    if cfg.varlen:
        sub.lengths = lengths[:n]
    else:
        sub.B = n
    f, b = sub.flops()
    try:
        model = [l for l in open("/proc/cpuinfo") if l.startswith("model name")][0].split(":")[1].strip()
    except (OSError, IndexError):
        model = "unknown"
    what = (f"first {n} of {len(lengths)} sequences ({sum(lengths[:n])} tokens)" if cfg.varlen
            else f"{n} of {cfg.B} batch rows")
    return {
        "value": (f + b) / med / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{what}, all {cfg.H} heads, fwd+bwd eager SDPA + materialised bias in "
                  f"{str(cfg.dtype).replace('torch.', '')}, median of 3 after 1 warm pass; "
                  f"{med * 1e3:.1f} ms per pass; host CPU: {model}",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): this build runs the "
              "kernels on a single MI355X; multi-GPU sharding is described in DESIGN.md and "
              "is not run.", file=sys.stderr)
        sys.exit(2)

    import torch

    from fna2_amd import _capi, configs

    F = importlib.import_module("fna2_amd.flash_naylis_attn")
    _capi.lib()  # fail loudly without the HIP library
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    cfg = configs.get(args.config)
    inp = configs.make_inputs(cfg).to(dev)
    leaves = [t.detach().requires_grad_(True) for t in (inp.q, inp.k, inp.v, inp.r_q, inp.r_k,
                                                         inp.graph_scale)]
    cu, mx = inp.cu_seqlens, inp.max_seqlen
    fwd_flops, bwd_flops = cfg.flops()

    def fwd():
        return F.flash_naylis_attn(*leaves, softmax_scale=inp.scale, is_causal=cfg.causal,
                                   cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=mx,
                                   max_seqlen_k=mx)

    def step():
        out = fwd()
        torch.autograd.grad(out, leaves, inp.dout)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # fwd+bwd, timed on the current stream with per-kernel events
    timer = F.KernelTimer(args.steps, args.steps)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with F.kernel_timing(timer):
        e0.record()
        for _ in range(args.steps):
            step()
        e1.record()
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / args.steps
    kdur = {k: statistics.mean(v) for k, v in timer.durations_ms().items()}

    # forward only
    with torch.no_grad():
        for _ in range(args.warmup):
            fwd()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(args.steps):
            fwd()
        e1.record()
        torch.cuda.synchronize()
    ms_fwd = e0.elapsed_time(e1) / args.steps

    # cache-flushed step (256 MB MALL): 512 MB written between timed steps
    ms_flushed = None
    if not args.no_flush:
        scratch = torch.empty(512 * 2**20, dtype=torch.uint8, device=dev)
        ts = []
        for _ in range(min(args.steps, 10)):
            scratch.fill_(1)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            step()
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b))
        ms_flushed = statistics.median(ts)
        del scratch

    tflops = (fwd_flops + bwd_flops) / (ms_step * 1e-3) / 1e12
    fwd_tflops = fwd_flops / (ms_fwd * 1e-3) / 1e12

    # roofline of the kernel with the largest time per step
    dom = max(("fwd", "dkdv", "dq"), key=lambda k: kdur.get(k, 0.0))
    dur_s = kdur[dom] * 1e-3
    nbytes, nflops = kernel_bytes(cfg, dom), kernel_flops(cfg, dom)
    ridge = PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
    if nflops / nbytes < ridge:
        ach = nbytes / dur_s / 1e9
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(ach / PEAK_HBM_GBS, 4)}
    else:
        ach = nflops / dur_s / 1e12
        roof = {"bound": "mfma", "achieved": round(ach, 1), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(ach / PEAK_BF16_TFLOPS, 4)}
    roof["traffic"] = None
    roof["kernel"] = dom
    roof["algorithmic_bytes"] = nbytes
    roof["algorithmic_flops"] = nflops
    roof["kernel_us"] = round(kdur[dom] * 1e3, 2)

    line = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v/dO, R ~ N(0, r_std), graph_scale = 1)",
        "config": {
            "workload": f"{cfg.name}: {cfg.desc}",
            "tokens": cfg.total,
            "n_seqs": len(cfg.seq_lengths()),
            "H": cfg.H, "d": cfg.D, "r": cfg.R, "causal": cfg.causal,
            "length_rule": "c3: 63 lengths ~U{64..512}, redrawn until the 64th "
                           "(16384 - sum) lies in [64, 512], seed 42" if cfg.name == "c3"
                           else None,
        },
        "frac_peak_fwd_bwd": round(tflops / PEAK_BF16_TFLOPS, 4),
        "fwd_tflops": round(fwd_tflops, 2),
        "frac_peak_fwd": round(fwd_tflops / PEAK_BF16_TFLOPS, 4),
        "ms_fwd": round(ms_fwd, 4),
        "ms_per_step_flushed": None if ms_flushed is None else round(ms_flushed, 4),
        "tflops_flushed": None if ms_flushed is None else
        round((fwd_flops + bwd_flops) / (ms_flushed * 1e-3) / 1e12, 2),
        "kernel_us": {k: round(v * 1e3, 2) for k, v in kdur.items()},
        "roofline": roof,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(cfg, inp, args.cpu_seconds)
        line["cpu_baseline"]["gpu_over_cpu"] = round(tflops / line["cpu_baseline"]["value"], 1)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
