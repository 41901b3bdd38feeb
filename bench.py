"""Benchmark of the quantized GEMV hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload: the Q6_K-style symmetric int6 GEMV set
at batch 1 -- RWKV-7 1.5B channel-mix key 2048->8192 and value 8192->2048
in sym@6 (superblocks of 256 = 16 blocks of 16, int8 block scales, fp16 d),
plus the int8 per-row-scaled head 2048->65536; weights N(0, 0.02) with
0.1% of input columns scaled x20, x bf16 N(0, 1).  A step is one pass over
the set (three GEMV launches).  Four device copies of the set (650 MB) are
visited in turn so that every step streams its weights from HBM rather than
the 256 MB Infinity Cache.

metric: algorithmic bytes of the set (canonical .rwkvq buffers + x + y) per
second of step time, in GB/s.  roofline: the dominant kernel (the int8
head GEMV) -- algorithmic bytes per launch over its mean launch time,
measured with HIP events on the launch stream, against the 8 TB/s HBM
peak.  cpu_baseline: the CPU oracle (numpy dequant + fp32 GEMV) on a
bounded sample of the same set, timed on this host.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "rwkv-quant_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
SHAPES = {"cmix_key": (8192, 2048), "cmix_value": (2048, 8192),
          "head": (65536, 2048)}


def build_set():
    """Quantize the three matrices once (CPU), return QuantizedTensors."""
    import torch
    from rwkv_quant.formats import writer
    out = {}
    for i, (name, (rows, cols)) in enumerate(SHAPES.items()):
        g = torch.Generator().manual_seed(i)
        w = torch.randn(rows, cols, generator=g) * 0.02
        n_out = max(1, round(cols * 0.001))
        idx = torch.randperm(cols, generator=g)[:n_out]
        w[:, idx] *= 20.0
        if name == "head":
            codes, scale = writer.rtn_quantize(w, 8)
            out[name] = writer.make_rtn("head.weight", "head", 8, w.shape,
                                        codes, scale)
        else:
            out[name] = writer.pack_sym(f"blocks.0.ffn.{name[5:]}.weight",
                                        "cmix", 6, w, 16, 16, search=True)
        del w
    return out


def algorithmic_bytes(qts):
    """Canonical .rwkvq buffer bytes + fp32 x in + fp32 y out per matrix
    (x is bf16 in the config; the kernel reads it as fp32 -- counted as
    bf16, the smaller figure, so `achieved` is not inflated)."""
    per = {}
    for name, qt in qts.items():
        b = 0
        for f in ("codes", "codes_packed", "scale", "gw_qs", "gw_d", "gw_qh",
                  "gw_qh2"):
            t = getattr(qt, f)
            if t is not None:
                b += t.numel() * t.element_size()
        rows, cols = qt.shape
        per[name] = b + cols * 2 + rows * 4
    return per


def cpu_baseline(qts, budget_s=15.0):
    """Reference-faithful CPU path: oracle dequant to fp32 + fp32 GEMV."""
    import numpy as np
    from oracle import codec_ref as cr
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:                                  # pragma: no cover
        threadpool_limits = None
    cores = len(os.sched_getaffinity(0))
    cores = min(cores, 16)
    per = algorithmic_bytes(qts)
    rng = np.random.default_rng(1)
    xs = {n: rng.standard_normal((1, qt.shape[1])).astype(np.float32)
          for n, qt in qts.items()}
    import contextlib
    ctx = (threadpool_limits(limits=cores) if threadpool_limits
           else contextlib.nullcontext())
    done_bytes, t_total, reps = 0, 0.0, 0
    with ctx:
        while t_total < budget_s and reps < 8:
            for n, qt in qts.items():
                t0 = time.perf_counter()
                w = cr.dequant_qt(qt)
                y = xs[n] @ w.T
                t_total += time.perf_counter() - t0
                done_bytes += per[n]
                del w, y
            reps += 1
    return {"value": round(done_bytes / t_total / 1e9, 4), "unit": "GB/s",
            "cores": cores, "kind": "port",
            "sample": f"{reps} pass(es) over the 3-matrix set "
                      f"({sum(per.values()) / 1e6:.1f} MB each): oracle "
                      f"numpy dequant to fp32 + fp32 GEMV, {t_total:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=4)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for "
              f"--gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    from rwkv_quant.backends.hip import _lib
    from rwkv_quant.backends.hip.quant_linear import (QuantLinearV2,
                                                      SymQuantLinear)
    _lib.load()
    qts = build_set()
    per = algorithmic_bytes(qts)
    set_bytes = sum(per.values())
    dev = torch.device("cuda:0")

    base = {n: (QuantLinearV2(qt) if n == "head" else SymQuantLinear(qt))
            for n, qt in qts.items()}
    # distinct device copies of every buffer
    copies = []
    for c in range(args.copies):
        cp = {}
        for n, lin in base.items():
            if c == 0:
                cp[n] = lin
                continue
            new = lin.__class__.__new__(lin.__class__)
            new.__dict__.update({k: (v.clone() if torch.is_tensor(v) else v)
                                 for k, v in lin.__dict__.items()})
            cp[n] = new
        copies.append(cp)
    g = torch.Generator().manual_seed(1)
    x = {n: torch.randn(1, qt.shape[1], generator=g).to(torch.bfloat16)
         .float().to(dev) for n, qt in qts.items()}
    y = {n: torch.empty(1, qt.shape[0], device=dev) for n, qt in qts.items()}

    def step(i):
        cp = copies[i % len(copies)]
        for n in SHAPES:
            cp[n].gemv_into(x[n], y[n])

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(
        enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for i in range(args.steps):
        step(i)
    t1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / args.steps

    # per-kernel mean launch time (events on the launch stream)
    kern = {}
    for n in SHAPES:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(
            enable_timing=True)
        reps = args.steps
        torch.cuda.synchronize()
        e0.record(stream)
        for i in range(reps):
            copies[i % len(copies)][n].gemv_into(x[n], y[n])
        e1.record(stream)
        torch.cuda.synchronize()
        kern[n] = e0.elapsed_time(e1) / reps
    head_us = kern["head"] * 1e3
    achieved = per["head"] / (kern["head"] * 1e-3) / 1e9

    out = {
        "metric": "quant GEMV GB/s (% HBM peak)",
        "value": round(set_bytes / (ms_per_step * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8/u8 codes, fp16 x pairs, fp32 accumulate",
        "data": "synthetic (seeded N(0,0.02) weights, 0.1% x20 outlier "
                "columns, bf16 N(0,1) x)",
        "config": {"workload": "configs[1]: sym@6 cmix key 2048->8192 + "
                               "value 8192->2048 + rtn@8 head 2048->65536, "
                               "batch 1",
                   "set_bytes": set_bytes, "copies": args.copies},
        "pct_hbm_peak": round(100 * set_bytes / (ms_per_step * 1e-3) / 1e9
                              / HBM_PEAK_GBS, 2),
        "kernels_us": {n: round(v * 1e3, 3) for n, v in kern.items()},
        "roofline": {"bound": "hbm", "kernel": "gemv_kernel<F_RTN8> (head)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None, "launch_us": round(head_us, 3),
                     "bytes_per_launch": per["head"]},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(qts)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
