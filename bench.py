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
most time per step (per-launch durations from HIP events that the library
records on its launch stream, in a separate pass of the same steps: event
records between dependent kernels add a few microseconds each, so the timed
steps run without them), the durations of the warmup steps and of the
kernels in a first per-kernel pass (the device's clock ramp after the idle
start: that pass and the forward-only one run before the W warmup and K
timed steps), and a ``cpu_baseline``
object: the reference's eager path (SDPA + materialised bias, restated in
``oracle/eager_reference.py``) timed on this host's cores on a bounded
sample of the same workload.

``--rope`` measures the varlen rotary embedding kernel instead (q and k of
the c3 pack: 16384 tokens, 16 + 16 heads, d = 128, bf16): its HBM rate and
roofline fraction, the reference's per-sequence eager loop on the same GPU,
and the oracle on the host.

``--producer`` measures the projection that produces the kernels' operands
(q, k, v, R_q, R_k from x: one GEMM over the stacked weights, forward and
backward) against the reference's five separate projections.

``--module`` measures one NaylisAttention layer's packed forward + backward
on the c3 pack (projection, QK-RMSNorm + RoPE, attention, output
projection), with the projection's gradients written into one buffer and,
for comparison, into separate tensors.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3]
                       [--rope|--producer|--module|--decode]
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

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA, AMD's figure (256 CUs x 2.4 GHz x 4096 FLOP/clk)
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E, AMD's figure
BF16_FLOP_PER_CLK_CU = 4096  # v_mfma_f32_32x32x16_bf16: 32,768 FLOP per 32 clocks on each of 4 SIMDs
# hipDeviceAttribute_t values of hip_runtime_api.h (ROCm 7)
_HIP_ATTR_CLOCK_RATE_KHZ = 5
_HIP_ATTR_MULTIPROCESSOR_COUNT = 63
METRIC = "fwd+bwd TFLOP/s & % bf16 MFMA peak, varlen 16k-token pack H=16 d=128 r=32"


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c3", choices=["c2", "c3", "c4", "c5"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--rope", action="store_true",
                    help="measure the varlen RoPE kernel (c3 pack) instead of attention")
    ap.add_argument("--decode", action="store_true",
                    help="bench the KV-cache decode kernel instead of the training step")
    ap.add_argument("--leg", choices=["all", "fused", "separate"], default="all",
                    help="--producer: run only the one-GEMM legs or only the five projections "
                         "(e.g. to trace one of them alone)")
    ap.add_argument("--producer", action="store_true",
                    help="measure the fused operand projection (c3-sized module) instead")
    ap.add_argument("--module", action="store_true",
                    help="measure one NaylisAttention layer's packed forward + backward "
                         "(c3 pack, E = 2048) instead")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="approximate CPU-baseline budget (seconds)")
    ap.add_argument("--no-flush", action="store_true",
                    help="skip the cache-flushed measurement")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device-to-device copy (the known-size kernel that "
                         "calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE) and print its rate")
    ap.add_argument("--summarize-pmc", nargs="+", metavar="DIR",
                    help="WORKLOAD_DIR COPY_DIR [NAME]: turn rocprofv3 --pmc FETCH_SIZE / "
                         "WRITE_SIZE runs of this bench and of --copy-calibration into "
                         "profiles/traffic_<NAME>.json (NAME defaults to --config)")
    ap.add_argument("--summarize-trace", nargs=3, metavar=("DB_DIR", "OUT_MD", "COMMAND"),
                    help="write the rocprofv3 --kernel-trace --stats table of DB_DIR to OUT_MD")
    ap.add_argument("--summarize-counters", nargs=3, metavar=("DB_DIR", "OUT_MD", "COMMAND"),
                    help="write the per-kernel means of a rocprofv3 --pmc pass to OUT_MD")
    return ap.parse_args()


def device_peak(dev_index: int = 0) -> dict:
    """The bf16 dense MFMA peak of the device the bench runs on, derived from
    its compute-unit count and peak clock (the HIP runtime's attributes),
    next to AMD's published figure that every fraction in the line uses."""
    import ctypes
    import torch
    cus = torch.cuda.get_device_properties(dev_index).multi_processor_count
    khz = None
    for name in ("libamdhip64.so", "libamdhip64.so.7", "libamdhip64.so.6"):
        try:
            hip = ctypes.CDLL(name)
        except OSError:
            continue
        v = ctypes.c_int(0)
        if hip.hipDeviceGetAttribute(ctypes.byref(v), _HIP_ATTR_CLOCK_RATE_KHZ, dev_index) == 0:
            khz = v.value
        c = ctypes.c_int(0)
        if hip.hipDeviceGetAttribute(ctypes.byref(c), _HIP_ATTR_MULTIPROCESSOR_COUNT, dev_index) == 0:
            cus = c.value or cus
        break
    derived = None if not khz else cus * khz * 1e3 * BF16_FLOP_PER_CLK_CU / 1e12
    return {"published_tflops": PEAK_BF16_TFLOPS, "derived_tflops":
            None if derived is None else round(derived, 1), "cus": cus,
            "clock_mhz": None if not khz else khz / 1000.0,
            "flop_per_clk_cu": BF16_FLOP_PER_CLK_CU}


def copy_rate_gbs(nbytes: int = 512 << 20, reps: int = 5) -> float:
    """Read + write GB/s of a device-to-device copy of nbytes, timed in this
    run: the practical HBM ceiling next to the 8 TB/s sheet figure."""
    import torch
    x = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    y = torch.empty_like(x)
    y.copy_(x)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        y.copy_(x)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del x, y
    return 2 * nbytes / (ms * 1e-3) / 1e9


COPY_BYTES = 1 << 30
TRAFFIC_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")


def copy_calibration():
    """1 GiB device copy, 10 times: reads and writes exactly COPY_BYTES per launch."""
    import torch

    x = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        y.copy_(x)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 10
    print(json.dumps({"copy_bytes": COPY_BYTES, "ms": round(ms, 4),
                      "GBps_read_plus_write": round(2 * COPY_BYTES / ms / 1e6, 1)}), flush=True)


def _profiler_rows(d, query):
    """Rows of `query` over every rocprofv3 database (*_results.db) under d."""
    import glob
    import sqlite3
    rows = []
    for fn in sorted(glob.glob(os.path.join(d, "**", "*_results.db"), recursive=True)):
        con = sqlite3.connect(fn)
        try:
            rows += con.execute(query).fetchall()
        finally:
            con.close()
    return rows


def _short(name):
    return name.replace("(anonymous namespace)::", "").split("(")[0]


def _pmc_means(d):
    """Mean counter value (KiB per dispatch, summed over XCDs) per kernel name."""
    acc = {}
    for name, ctr, v in _profiler_rows(
            d, "select kernel_name, counter_name, value from counters_collection"):
        acc.setdefault((_short(name), ctr), []).append(float(v))
    return {k: sum(v) / len(v) for k, v in acc.items()}


def summarize_trace(d, out_md, command):
    """Markdown table of rocprofv3 --kernel-trace --stats (the top_kernels view)."""
    rows = _profiler_rows(d, "select name, total_calls, total_duration, average, percentage "
                             "from top_kernels order by total_duration desc")
    lines = [f"Command: `{command}`", "",
             "| kernel | calls | total (us) | average (us) | % of GPU time |",
             "|---|---|---|---|---|"]
    for name, calls, tot, avg, pct in rows:
        lines.append(f"| `{_short(name)}` | {calls} | {tot:.1f} | {avg:.2f} | {pct:.1f} |")
    with open(out_md, "w") as fh:
        fh.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def summarize_counters(d, out_md, command):
    """Markdown table of the mean counter values per kernel (one --pmc pass)."""
    m = _pmc_means(d)
    ctrs = sorted({c for _, c in m})
    kernels = sorted({k for k, _ in m if k.startswith("fna2::")})
    lines = [f"Command: `{command}`", "", "Mean per dispatch (summed over the XCDs).", "",
             "| kernel | " + " | ".join(ctrs) + " |", "|---" * (len(ctrs) + 1) + "|"]
    for k in kernels:
        lines.append(f"| `{k}` | " + " | ".join(f"{m.get((k, c), float('nan')):.4g}"
                                                for c in ctrs) + " |")
    with open(out_md, "w") as fh:
        fh.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def summarize_pmc(work_dir, copy_dir, config):
    """Calibrated HBM bytes per launch.  Each counter is scaled by the factor
    that makes the copy kernel's reading equal its known size (1 GiB read and
    1 GiB written per launch)."""
    w, c = _pmc_means(work_dir), _pmc_means(copy_dir)
    copy_fetch = max(v for (n, k), v in c.items() if k == "FETCH_SIZE" and "copyBuffer" in n)
    copy_write = max(v for (n, k), v in c.items() if k == "WRITE_SIZE" and "copyBuffer" in n)
    f_fetch = COPY_BYTES / (copy_fetch * 1024.0)
    f_write = COPY_BYTES / (copy_write * 1024.0)
    kernels = {}
    for (name, ctr), v in w.items():
        if not name.startswith("fna2::"):
            continue
        short = name.split("::")[-1]
        e = kernels.setdefault(short, {})
        if ctr == "FETCH_SIZE":
            e["fetch_bytes"] = round(v * 1024.0 * f_fetch)
        elif ctr == "WRITE_SIZE":
            e["write_bytes"] = round(v * 1024.0 * f_write)
    out = {"config": config, "calibration": {"fetch_factor": round(f_fetch, 4),
                                             "write_factor": round(f_write, 4),
                                             "copy_bytes": COPY_BYTES},
           "kernels": kernels}
    path = os.path.join(TRAFFIC_DIR, f"traffic_{config}.json")
    with open(path, "w") as fh:
        json.dump(out, fh, indent=1)
        fh.write("\n")
    print(json.dumps(out), flush=True)


def measured_traffic(config, kernel):
    """HBM bytes per launch of `kernel` from profiles/traffic_<config>.json, or None."""
    key = {"fwd": "fwd_kernel", "dkdv": "dkdv_kernel", "dq": "dq_kernel"}.get(kernel, kernel)
    try:
        with open(os.path.join(TRAFFIC_DIR, f"traffic_{config}.json")) as fh:
            ks = json.load(fh)["kernels"]
    except (OSError, ValueError, KeyError):
        return None
    for name, e in ks.items():
        if name.startswith(key) and "fetch_bytes" in e and "write_bytes" in e:
            return e["fetch_bytes"] + e["write_bytes"]
    return None


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


def rope_bench(args):
    """Varlen RoPE of q [T, 16, 128] and k [T, 16, 128] (bf16, the c3 pack)."""
    import numpy as np
    import torch

    from fna2_amd import _capi, attention_fna2, configs
    from fna2_amd.rope import rope_varlen, rope_varlen_raw

    _capi.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = configs.get("c3")
    lengths = cfg.seq_lengths()
    cu_list = [0] + list(np.cumsum(lengths))
    T, H, D = cu_list[-1], 16, 128
    g = torch.Generator().manual_seed(42)
    q = torch.randn(T, H, D, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(T, H, D, generator=g).to(torch.bfloat16).to(dev)
    cu = torch.tensor(cu_list, dtype=torch.int32, device=dev)
    rope = attention_fna2.RotaryPositionalEmbedding(D, max_seq_len=1024).to(dev)
    inv = rope.inv_freq

    for _ in range(args.warmup):
        rope_varlen_raw(q, k, cu, inv)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        rope_varlen_raw(q, k, cu, inv)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    nbytes = 2 * (q.numel() + k.numel()) * q.element_size() + cu.numel() * 4 + inv.numel() * 4
    gbs = nbytes / (ms * 1e-3) / 1e9

    # the reference's algorithm on the same GPU: a host loop over the sequences
    # (cu_seqlens.tolist()) applying the dense RoPE (attention_fna2.py:620-647)
    def eager():
        qo, ko = torch.empty_like(q), torch.empty_like(k)
        off = 0
        for n in (cu[1:] - cu[:-1]).tolist():
            qs = q[off:off + n].transpose(0, 1).unsqueeze(0)
            ks = k[off:off + n].transpose(0, 1).unsqueeze(0)
            qr, kr = rope(qs, ks, position_offset=0)
            qo[off:off + n] = qr.squeeze(0).transpose(0, 1)
            ko[off:off + n] = kr.squeeze(0).transpose(0, 1)
            off += n
        return qo, ko
    for _ in range(3):
        eager()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(10):
        eager()
    torch.cuda.synchronize()
    ms_eager = (time.perf_counter() - t0) / 10 * 1e3

    # QK-RMSNorm + RoPE in one launch, forward + backward (fp32 norm weights),
    # against the eager chain the reference runs (q_norm / k_norm then the
    # per-sequence RoPE, attention_fna2.py:558-566)
    wq = torch.ones(D, device=dev, requires_grad=True)
    wk = torch.ones(D, device=dev, requires_grad=True)
    qg, kg = q.detach().requires_grad_(True), k.detach().requires_grad_(True)
    gq, gk = torch.randn_like(q), torch.randn_like(k)

    def timed(fn, n):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n

    def norm_fwd():
        return rope_varlen(qg, kg, cu, inv, wq, wk, 1e-6)

    def norm_fwd_bwd():
        yq, yk = norm_fwd()
        torch.autograd.grad([yq, yk], [qg, kg, wq, wk], [gq, gk])
    ms_norm_fwd = timed(lambda: rope_varlen_raw(q, k, cu, inv, 1, wq, wk, 1e-6), args.steps)
    ms_norm_fb = timed(norm_fwd_bwd, args.steps)
    qn, kn = attention_fna2.RMSNorm(D).to(dev), attention_fna2.RMSNorm(D).to(dev)

    def eager_norm_fwd_bwd():
        a, b = qn(qg), kn(kg)
        qo, ko = torch.empty_like(a), torch.empty_like(b)
        off = 0
        for n in (cu[1:] - cu[:-1]).tolist():
            qr, kr = rope(a[off:off + n].transpose(0, 1).unsqueeze(0),
                          b[off:off + n].transpose(0, 1).unsqueeze(0))
            qo[off:off + n] = qr.squeeze(0).transpose(0, 1)
            ko[off:off + n] = kr.squeeze(0).transpose(0, 1)
            off += n
        torch.autograd.grad([qo, ko], [qg, kg, qn.weight, kn.weight], [gq, gk])
    ms_eager_norm_fb = timed(eager_norm_fwd_bwd, 5)

    line = {
        "metric": "varlen RoPE HBM GB/s (q and k read + written once)",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k)",
        "config": {"workload": f"rope_varlen: c3 pack, {T} tokens / {len(lengths)} seqs, "
                               f"q and k {H} heads each, d={D}"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "rope_kernel", "algorithmic_bytes": nbytes},
        "eager_reference_ms": round(ms_eager, 3),
        "speedup_over_eager": round(ms_eager / ms, 1),
        "qk_norm_rope": {
            "fwd_ms": round(ms_norm_fwd, 4),
            "fwd_GBps": round(nbytes / (ms_norm_fwd * 1e-3) / 1e9, 1),
            "fwd_bwd_ms": round(ms_norm_fb, 4),
            "eager_fwd_bwd_ms": round(ms_eager_norm_fb, 3),
            "speedup_over_eager": round(ms_eager_norm_fb / ms_norm_fb, 1),
        },
    }
    if not args.no_cpu:
        from oracle import rope_oracle as RO
        n = 2048  # leading tokens of the pack
        qc = q[:n].float().cpu().numpy()
        kc = k[:n].float().cpu().numpy()
        cuc = [c for c in cu_list if c <= n] + ([n] if cu_list[-1] > n else [])
        RO.rope_varlen(qc, kc, cuc, inv.cpu().numpy(), "bf16")
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            RO.rope_varlen(qc, kc, cuc, inv.cpu().numpy(), "bf16")
            ts.append(time.perf_counter() - t0)
        med = statistics.median(ts)
        line["cpu_baseline"] = {"value": round(nbytes * n / T / med / 1e9, 3), "unit": "GB/s",
                                "cores": 1, "kind": "port",
                                "sample": f"oracle (numpy) on the first {n} of {T} tokens, "
                                          f"median of 3: {med * 1e3:.1f} ms"}
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


def producer_bench(args):
    """q, k, v, R_q, R_k of a c3-sized NaylisAttention (T = 16384, E = 2048,
    16 heads of 128, 16 graph heads of rank 32, bf16), forward + backward:
    the module's one-GEMM projection over the stacked weights, with separate
    cotangents (``value``: per-block dW / dx GEMMs, no concatenation) and with
    cotangents that are column blocks of one buffer (``ms_stacked_grads``: one
    dx and one dW GEMM), against the reference's five projections."""
    import torch

    from fna2_amd import attention_fna2 as A

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    T, E = 16384, 2048
    torch.manual_seed(0)
    m = A.NaylisAttention(E, 16, rel_rank=32, use_fna2=False).to(dev).to(torch.bfloat16)
    x = torch.randn(T, E, device=dev, dtype=torch.bfloat16, requires_grad=True)
    params = [m.q_proj.weight, m.k_proj.weight, m.v_proj.weight, m.rel_q_proj.weight,
              m.rel_k_proj.weight]
    H, D, HG, R = 16, 128, 16, 32
    grads = [torch.randn(T, H, D, device=dev, dtype=torch.bfloat16) for _ in range(3)] + \
            [torch.randn(T, HG, R, device=dev, dtype=torch.bfloat16) for _ in range(2)]

    def separate():  # attention_fna2.py:554-556, :326-334
        q = m.q_proj(x).view(T, H, D)
        k = m.k_proj(x).view(T, H, D)
        v = m.v_proj(x).view(T, H, D)
        rq = m.rel_q_proj(x).view(T, HG, R).to(torch.bfloat16).contiguous()
        rk = m.rel_k_proj(x).view(T, HG, R).to(torch.bfloat16).contiguous()
        return q, k, v, rq, rk

    # Cotangents as consecutive column blocks of one [T, E + 2 kv + 2 R]
    # buffer (what a caller whose gradient producers write one buffer hands
    # back): the projection's backward is then one dx and one dW GEMM.
    g_all = torch.randn(T, E + 2 * H * D + 2 * HG * R, device=dev, dtype=torch.bfloat16)
    stacked = list(torch.split(g_all, [H * D, H * D, H * D, HG * R, HG * R], dim=-1))
    stacked = [g.view(T, H, D) for g in stacked[:3]] + [g.view(T, HG, R) for g in stacked[3:]]

    def run(fn, cot=grads):
        outs = fn()
        torch.autograd.grad(outs, [x] + params, cot)

    res = {}
    legs = (("separate", separate, grads), ("fused", lambda: m._project(x), grads),
            ("fused_stacked_grads", lambda: m._project(x), stacked))
    if args.leg != "all":
        legs = [leg for leg in legs if leg[0].startswith(args.leg)]
    for name, fn, cot in legs:
        run_ = lambda: run(fn, cot)
        for _ in range(args.warmup):
            run_()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            run_()
        e1.record()
        torch.cuda.synchronize()
        res[name] = e0.elapsed_time(e1) / args.steps
    n_all = E + 2 * H * D + 2 * HG * R
    flops = 3 * 2 * T * E * n_all  # forward GEMM, dX and dW GEMMs
    if "fused" not in res:  # --leg separate
        print(json.dumps({"separate_ms": round(res["separate"], 4)}), flush=True)
        return
    tf = flops / (res["fused"] * 1e-3) / 1e12
    print(json.dumps({
        "metric": "operand producer fwd+bwd TFLOP/s (one GEMM over stacked q/k/v/R weights)",
        "value": round(tf, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(res["fused"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) x and upstream gradients)",
        "config": {"workload": f"producer: T={T}, E={E}, q/k/v 16x128, R_q/R_k 16x32"},
        "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4),
                     "traffic": None, "kernel": "hipBLASLt GEMMs"},
        "separate_ms": round(res["separate"], 4) if "separate" in res else None,
        "speedup_over_separate": (round(res["separate"] / res["fused"], 3)
                                  if "separate" in res else None),
        "ms_stacked_grads": round(res["fused_stacked_grads"], 4),
        "cpu_baseline": None,
    }), flush=True)


def module_bench(args):
    """One NaylisAttention layer on the c3 pack (16384 tokens / 64 sequences,
    E = 2048, 16 heads of 128, 16 graph heads of rank 32, QK-RMSNorm, RoPE,
    bf16), forward + backward of the packed path: the one-GEMM projection,
    the norm + RoPE launch, the attention kernels and the output projection.
    ``value``: with the projection's gradients written into one buffer
    (GradSlab: one dx and one dW GEMM); ``separate_ms``: with separate
    gradient tensors; ``dense_ms``: a dense layer of c2's geometry ([4, 2048,
    1024] input, 16 heads of 64, 16 graph heads of rank 16), forward +
    backward, whose QK-norm and RoPE run in the same launch."""
    import numpy as np
    import torch

    from fna2_amd import attention_fna2 as A
    from fna2_amd import configs

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = configs.get("c3")
    lens = cfg.seq_lengths()
    T, E = sum(lens), 2048
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32, device=dev)
    torch.manual_seed(0)
    m = A.NaylisAttention(E, 16, rel_rank=32, max_seq_len=1024).to(device=dev,
                                                                   dtype=torch.bfloat16)
    assert A._FNA2_AVAILABLE, "the HIP library and a gfx950 device are needed"
    m._use_fna2 = True
    x = torch.randn(T, E, device=dev, dtype=torch.bfloat16, requires_grad=True)
    g = torch.randn(T, E, device=dev, dtype=torch.bfloat16)

    def step():
        # gradients set to None first, as a training step's zero_grad does
        # (else every backward adds into the previous step's)
        x.grad = None
        for p_ in m.parameters():
            p_.grad = None
        y, _ = m(x, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=max(lens),
                 max_seqlen_k=max(lens))
        y.backward(g)

    torch.manual_seed(0)
    md = A.NaylisAttention(1024, 16, rel_rank=16, max_seq_len=2048).to(device=dev,
                                                                       dtype=torch.bfloat16)
    md._use_fna2 = True
    xd = torch.randn(4, 2048, 1024, device=dev, dtype=torch.bfloat16, requires_grad=True)
    gd = torch.randn(4, 2048, 1024, device=dev, dtype=torch.bfloat16)

    def dense_step():
        xd.grad = None
        for p_ in md.parameters():
            p_.grad = None
        y, _ = md(xd)
        y.backward(gd)

    res = {}
    try:
        for slab in (True, False):
            A.NaylisAttention._grad_slab = slab
            for _ in range(args.warmup):
                step()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(args.steps):
                step()
            e1.record()
            torch.cuda.synchronize()
            res[slab] = e0.elapsed_time(e1) / args.steps
    finally:
        A.NaylisAttention._grad_slab = True
    for _ in range(max(args.warmup, 10)):
        dense_step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        dense_step()
    e1.record()
    torch.cuda.synchronize()
    res["dense"] = e0.elapsed_time(e1) / args.steps
    print(json.dumps({
        "metric": "NaylisAttention packed layer fwd+bwd tokens/s (c3 pack, E=2048)",
        "value": round(T / (res[True] * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(res[True], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) x and output gradient, random-init weights)",
        "config": {"workload": f"NaylisAttention(2048, 16, rel_rank=32): {T} tokens / "
                               f"{len(lens)} seqs, QK-RMSNorm + RoPE, causal"},
        "separate_grads_ms": round(res[False], 4),
        "speedup_over_separate_grads": round(res[False] / res[True], 3),
        "dense_ms": round(res["dense"], 4),
        "dense_workload": "NaylisAttention(1024, 16, rel_rank=16) on [4, 2048, 1024], causal",
    }), flush=True)


def decode_bench(args):
    """One-token decode against a KV cache, with c3's attention geometry
    (16 heads of 128, all graph heads of rank 32), 64 sequences x 4096
    cached rows, bf16; plus a grouped-query variant (32 query heads on 8 KV
    heads)."""
    import ctypes

    import torch
    import torch.nn.functional as Fn

    from fna2_amd import _capi
    from fna2_amd.decode import decode_args

    lib = _capi.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    def inputs(B, H, HKV, HG, D, R, L, seed=42):
        g = torch.Generator().manual_seed(seed)
        draw = lambda *s, std=1.0: (torch.randn(*s, generator=g) * std).bfloat16().to(dev)
        return (draw(B, H, D), draw(B, HKV, L, D), draw(B, HKV, L, D), draw(B, HG, R, std=R ** -0.5),
                draw(B, HG, L, R, std=R ** -0.5), torch.randn(HG, generator=g).float().to(dev))

    def measure(shape, bias, steps, warmup):
        B, H, HKV, HG, D, R, L = shape
        q, k, v, rq, rk, gs = inputs(*shape)
        scale = D ** -0.5
        a, keep, out, lse = decode_args(q, k, v, rq if bias else None, rk if bias else None,
                                        gs if bias else None, scale)
        nws = lib.fna2_decode_workspace_bytes(ctypes.byref(a))
        ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=dev)
        a.workspace, a.workspace_bytes = ws.data_ptr(), nws
        call = lambda: _capi.raise_for(lib.fna2_decode(ctypes.byref(a), stream), "fna2_decode")
        for _ in range(warmup):
            call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            call()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        # the split kernel alone: events the library records around it
        pool = [torch.cuda.Event(enable_timing=True) for _ in range(2 * steps)]
        for ev in pool:
            ev.record()
        torch.cuda.synchronize()
        for i in range(steps):
            evs = (ctypes.c_void_p * 2)(pool[2 * i].cuda_event, pool[2 * i + 1].cuda_event)
            a.events = ctypes.cast(evs, ctypes.c_void_p)
            call()
        torch.cuda.synchronize()
        a.events = None
        k_ms = statistics.mean(pool[2 * i].elapsed_time(pool[2 * i + 1]) for i in range(steps))
        nbytes = B * HKV * L * D * 2 * 2 + (B * HG * L * R * 2 if bias else 0) \
            + 2 * B * H * D * 2 + (B * HG * R * 2 if bias else 0)
        # the reference's decode step on the same cache: SDPA over the cached
        # rows (attention_fna2.py:445-473, torch.cat of the cache not timed),
        # and the same with the graph bias as an explicit mask
        G = H // HKV
        ke = k.repeat_interleave(G, dim=1) if G > 1 else k
        ve = v.repeat_interleave(G, dim=1) if G > 1 else v
        q4 = q[:, :, None]

        def eager():
            if G > 1:  # the reference expands K / V every step
                kk, vv = k.repeat_interleave(G, dim=1), v.repeat_interleave(G, dim=1)
            else:
                kk, vv = ke, ve
            mask = None
            if bias:
                b = torch.matmul(rq[:, :, None].float(), rk.float().transpose(-2, -1).contiguous())
                mask = (gs.view(1, -1, 1, 1) * b).to(torch.bfloat16)
                if HG < H:
                    mask = torch.cat([mask, mask.new_zeros(B, H - HG, 1, L)], dim=1)
            return Fn.scaled_dot_product_attention(q4, kk, vv, attn_mask=mask, scale=scale)
        for _ in range(3):
            eager()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        n_e = max(steps // 4, 5)
        for _ in range(n_e):
            eager()
        torch.cuda.synchronize()
        ms_eager = (time.perf_counter() - t0) / n_e * 1e3
        del keep
        return dict(ms=ms, kernel_ms=k_ms, bytes=nbytes, eager_ms=ms_eager,
                    splits=lib.fna2_decode_num_splits(ctypes.byref(a)),
                    inputs=(q, k, v, rq, rk, gs, scale))

    def module_steps(steps):
        """One NaylisAttention decode step (E = 2048, 16 heads of 128, all
        graph heads, rank 32; bf16) for 64 sequences against 4095 cached
        rows: the reference's pattern (tuple cache grown by torch.cat, SDPA
        without the bias: the module built with use_fna2=False), the tuple
        cache on the decode kernel, and a StaticKVCache (written in place),
        with and without the bias."""
        from fna2_amd import attention_fna2 as A
        B, L, E = 64, 4095, 2048
        torch.manual_seed(0)
        res = {}
        x = torch.randn(B, 1, E, device=dev, dtype=torch.bfloat16)
        for name, fna2, bias, static in (("reference_eager", False, False, False),
                                         ("tuple_cache", True, False, False),
                                         ("static_cache", True, False, True),
                                         ("static_cache_bias", True, True, True)):
            m = A.NaylisAttention(E, 16, rel_rank=32, use_fna2=fna2,
                                  decode_graph_bias=bias).to(dev).to(torch.bfloat16).eval()
            if fna2 and not m._use_fna2:
                raise RuntimeError("decode bench: the FNA2 kernels are not available")
            g = torch.Generator(device=dev).manual_seed(1)
            rows = [torch.randn(B, 16, L, 128, device=dev, dtype=torch.bfloat16, generator=g)
                    for _ in range(2)]
            if bias:
                rows.append(torch.randn(B, 16, L, 32, device=dev, dtype=torch.bfloat16,
                                        generator=g) * 32 ** -0.5)
            if static:
                cache = A.StaticKVCache.empty(B, 16, L + steps + 8, 128, 16 if bias else 0, 32,
                                              device=dev)
                cache.append(*rows)
                step = lambda: m(x, past_kv=cache, use_kv_cache=True)
                reset = lambda: setattr(cache, "length", L)
            else:
                past = tuple(rows)
                step = lambda: m(x, past_kv=past, use_kv_cache=True)
                reset = lambda: None
            with torch.no_grad():
                for _ in range(3):
                    step()
                    reset()
                torch.cuda.synchronize()
                ts = []
                for _ in range(steps):
                    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    a.record()
                    step()
                    b.record()
                    torch.cuda.synchronize()
                    reset()
                    ts.append(a.elapsed_time(b))
            res[name] = round(statistics.median(ts), 4)
            del m, rows
        return res

    main_shape = (64, 16, 16, 16, 128, 32, 4096)
    gqa_shape = (64, 32, 8, 32, 128, 32, 4096)
    r = measure(main_shape, True, args.steps, args.warmup)
    r0 = measure(main_shape, False, args.steps, args.warmup)
    rg = measure(gqa_shape, True, args.steps, args.warmup)
    mod = module_steps(max(args.steps // 5, 5))
    gbs = r["bytes"] / (r["ms"] * 1e-3) / 1e9
    kgbs = r["bytes"] / (r["kernel_ms"] * 1e-3) / 1e9
    line = {
        "metric": "decode HBM GB/s (K, V and Rk cache read once per step)",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(r["ms"], 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q and caches, R ~ N(0, 1/R))",
        "config": {"workload": "decode: 64 sequences x 4096 cached rows, 16 heads (all graph "
                               "heads, R=32), 16 KV heads, d=128 (c3's attention geometry)",
                   "num_splits": r["splits"]},
        "roofline": {"bound": "hbm", "achieved": round(kgbs, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(kgbs / PEAK_HBM_GBS, 4),
                     "traffic": measured_traffic("decode", "decode_kernel_d128_c4"),
                     "traffic_source": "profiles/traffic_decode.json (rocprofv3 FETCH_SIZE + "
                                       "WRITE_SIZE per dispatch, copy-calibrated)",
                     "kernel": "decode_kernel_d128_c4", "algorithmic_bytes": r["bytes"],
                     "kernel_ms": round(r["kernel_ms"], 5)},
        "eager_reference_ms": {"with_bias": round(r["eager_ms"], 4),
                               "without_bias": round(r0["eager_ms"], 4)},
        "speedup_over_eager": round(r["eager_ms"] / r["ms"], 2),
        "without_bias": {"ms": round(r0["ms"], 5),
                         "GBps": round(r0["bytes"] / (r0["ms"] * 1e-3) / 1e9, 1),
                         "speedup_over_reference_sdpa": round(r0["eager_ms"] / r0["ms"], 2)},
        "module_step_ms": mod,
        "gqa_32q_8kv": {"ms": round(rg["ms"], 5), "kernel_ms": round(rg["kernel_ms"], 5),
                        "GBps": round(rg["bytes"] / (rg["ms"] * 1e-3) / 1e9, 1),
                        "kernel_GBps": round(rg["bytes"] / (rg["kernel_ms"] * 1e-3) / 1e9, 1),
                        "eager_ms": round(rg["eager_ms"], 4), "num_splits": rg["splits"]},
    }
    if not args.no_cpu:
        from oracle import fna2_oracle as O
        q, k, v, rq, rk, gs, scale = r["inputs"]
        n = 4  # leading sequences
        host = [t[:n].float().cpu().numpy() for t in (q, k, v, rq, rk)]
        gsh = gs.cpu().numpy()
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            O.decode(*host[:3], host[3], host[4], gsh, scale)
            ts.append(time.perf_counter() - t0)
        med = statistics.median(ts)
        line["cpu_baseline"] = {"value": round(r["bytes"] * n / 64 / med / 1e9, 3),
                                "unit": "GB/s", "cores": 1, "kind": "port",
                                "sample": f"oracle.decode (numpy, fp64) on the first {n} of 64 "
                                          f"sequences, median of 3: {med * 1e3:.1f} ms"}
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


def main():
    args = parse()
    if args.decode:
        decode_bench(args)
        return
    if args.producer:
        producer_bench(args)
        return
    if args.module:
        module_bench(args)
        return
    if args.rope:
        rope_bench(args)
        return
    if args.copy_calibration:
        copy_calibration()
        return
    if args.summarize_pmc:
        if len(args.summarize_pmc) not in (2, 3):
            sys.exit("--summarize-pmc takes WORKLOAD_DIR COPY_DIR [NAME]")
        summarize_pmc(*args.summarize_pmc[:2],
                      args.summarize_pmc[2] if len(args.summarize_pmc) == 3 else args.config)
        return
    if args.summarize_trace:
        summarize_trace(*args.summarize_trace)
        return
    if args.summarize_counters:
        summarize_counters(*args.summarize_counters)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): this build runs the "
              "kernels on a single MI355X; sharding over several GPUs is not built.",
              file=sys.stderr)
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

    # Passes, in this order (the device idles while the process starts, and
    # its clocks come up only over the first few dozen steps):
    #  1. W warmup steps, each bracketed by events ("warmup_step_ms");
    #  2. K steps with HIP events around every kernel ("first_pass_kernel_us":
    #     the kernels during that ramp);
    #  3. the forward alone: W warmup + K timed forwards;
    #  4. W warmup + K timed fwd+bwd steps: `value`;
    #  5. K steps with HIP events around every kernel again: the per-kernel
    #     durations of the roofline, on a device at its working clocks (event
    #     records between dependent kernels add a few microseconds each, so
    #     the timed steps run without them).
    def kernel_pass():
        timer = F.KernelTimer(args.steps, args.steps)
        torch.cuda.synchronize()
        with F.kernel_timing(timer):
            for _ in range(args.steps):
                step()
        torch.cuda.synchronize()
        return {k: statistics.mean(v) for k, v in timer.durations_ms().items()}

    ramp = []
    for _ in range(args.warmup):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        step()
        b.record()
        torch.cuda.synchronize()
        ramp.append(round(a.elapsed_time(b), 4))
    kdur_first = kernel_pass()

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
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

    # fwd+bwd, timed on the current stream
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / args.steps

    kdur = kernel_pass()

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
    copy_gbs = copy_rate_gbs()
    roof["copy_GBps"] = round(copy_gbs, 1)
    roof["frac_of_copy"] = (round(roof["achieved"] / copy_gbs, 4) if roof["unit"] == "GB/s"
                            else None)
    roof["traffic"] = measured_traffic(cfg.name, dom)
    roof["traffic_source"] = (f"profiles/traffic_{cfg.name}.json (rocprofv3 FETCH_SIZE + "
                              "WRITE_SIZE per dispatch, copy-calibrated)"
                              if roof["traffic"] is not None else None)
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
        "peak_bf16": device_peak(),
        "frac_peak_fwd_bwd": round(tflops / PEAK_BF16_TFLOPS, 4),
        "fwd_tflops": round(fwd_tflops, 2),
        "frac_peak_fwd": round(fwd_tflops / PEAK_BF16_TFLOPS, 4),
        "ms_fwd": round(ms_fwd, 4),
        "ms_per_step_flushed": None if ms_flushed is None else round(ms_flushed, 4),
        "tflops_flushed": None if ms_flushed is None else
        round((fwd_flops + bwd_flops) / (ms_flushed * 1e-3) / 1e12, 2),
        "kernel_us": {k: round(v * 1e3, 2) for k, v in kdur.items()},
        "warmup_step_ms": ramp,
        "first_pass_kernel_us": {k: round(v * 1e3, 2) for k, v in kdur_first.items()},
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
