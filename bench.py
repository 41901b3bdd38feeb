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
peak and against the stream-read ceiling measured in the same run
(stream_ceiling).  Decode lines carry their HBM roofline (algorithmic bytes
per step / step time), prefill lines the GEMM kernels' FLOP rate against
the MFMA peak.  cpu_baseline: the CPU oracle (numpy dequant + fp32 GEMV)
on a bounded sample of the same set at the host's thread share and at one
thread, a torch-CPU GEMV on pre-dequantized weights, and the oracle's
decode / prefill of the 1.5B model, timed on this host.
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


# The GPU box gives one GPU a share of 16 host threads, whatever the
# visible core count; the n-thread CPU runs use min(affinity, 16).
CPU_SHARE = 16


def cpu_baseline(qts, budget_s=15.0, cores=None):
    """Reference-faithful CPU path: oracle dequant to fp32 + fp32 GEMV."""
    import numpy as np
    from oracle import codec_ref as cr
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:                                  # pragma: no cover
        threadpool_limits = None
    if cores is None:
        cores = min(len(os.sched_getaffinity(0)), CPU_SHARE)
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


def gemv_set_bench(args, qts, dev):
    """Time the 3-GEMV set on rotating device copies, replayed from a HIP
    graph (launch gaps as a serving loop sees them)."""
    import torch
    from rwkv_quant.backends.hip.quant_linear import (QuantLinearV2,
                                                      SymQuantLinear)
    base = {n: (QuantLinearV2(qt) if n == "head" else SymQuantLinear(qt))
            for n, qt in qts.items()}
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

    def one_pass(names=SHAPES):
        for cp in copies:
            for n in names:
                cp[n].gemv_into(x[n], y[n])

    def graph_of(names=SHAPES):
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            one_pass(names)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize()
        gph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gph):
            one_pass(names)
        return gph

    set_graph = graph_of()
    reps = max(1, args.steps // args.copies)
    for _ in range(max(1, args.warmup // args.copies)):
        set_graph.replay()
    _mark()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    t0, t1 = (torch.cuda.Event(enable_timing=True) for _ in range(2))
    t0.record(stream)
    for _ in range(reps):
        set_graph.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    steps = reps * args.copies
    ms_per_step = t0.elapsed_time(t1) / steps

    # mean launch time of each kernel on its own (graph of that kernel only)
    kern = {}
    for n in SHAPES:
        gk = graph_of((n,))
        gk.replay()
        torch.cuda.synchronize()
        e0, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(2))
        e0.record(stream)
        for _ in range(reps):
            gk.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        kern[n] = e0.elapsed_time(e1) / (reps * args.copies)
    return ms_per_step, steps, kern


MARK_KERNEL = "spin_kernel"


def _mark():
    """A ~1 us spin kernel launched just before a timed region, so that a
    kernel trace of the run can be cut at it (--trace-summary)."""
    import torch
    torch.cuda._sleep(1000)


def trace_summary(path, top=40):
    """Per-kernel table of a rocprofv3 kernel_trace.csv, over the dispatches
    after the last marker kernel (the last timed region of the run)."""
    import csv
    import re
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    cut = max((i for i, r in enumerate(rows) if MARK_KERNEL in
               r["Kernel_Name"]), default=-1)
    rows = rows[cut + 1:]
    agg = {}
    for r in rows:
        name = re.sub(r"\(.*", "", r["Kernel_Name"].replace(
            "(anonymous namespace)::", "").replace("void ", ""))
        key = (name[:72], r.get("Grid_Size", r.get("Grid_Size_X")),
               r.get("Workgroup_Size", r.get("Workgroup_Size_X")))
        d = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        a = agg.setdefault(key, [0, 0, 1 << 62, 0])
        a[0] += 1
        a[1] += d
        a[2] = min(a[2], d)
        a[3] = max(a[3], d)
    total = sum(a[1] for a in agg.values())
    span = (int(rows[-1]["End_Timestamp"]) - int(rows[0]["Start_Timestamp"])
            if rows else 0)
    print(f"dispatches after the marker: {len(rows)}; kernel time "
          f"{total / 1e3:.1f} us; span first start -> last end "
          f"{span / 1e3:.1f} us")
    print(f"{'kernel':72s} {'grid':>8s} {'wg':>4s} {'calls':>6s} "
          f"{'avg_us':>8s} {'min_us':>8s} {'max_us':>8s} {'share':>6s}")
    for (name, grid, wg), (n, tot, mn, mx) in sorted(
            agg.items(), key=lambda kv: -kv[1][1])[:top]:
        print(f"{name:72s} {grid:>8s} {wg:>4s} {n:6d} {tot / n / 1e3:8.2f} "
              f"{mn / 1e3:8.2f} {mx / 1e3:8.2f} {100 * tot / total:5.1f}%")


def decode_bench(preset, batches, n_tok, dev, shape="1.5b", ceiling=None):
    """ms per decode step of the 1.5B- (or 2.9B-) shaped model (graph
    replay, state carried between steps, fresh uniform-random token ids
    each step), with the HBM roofline of each batch (algorithmic bytes per
    step from the checkpoint's stored tensors, decode_step_bytes)."""
    import torch
    from rwkv_quant.backends.hip.quant_model import QuantRWKV7
    from rwkv_quant.models.synthetic import SHAPES as MS, quantized_model
    t0 = time.time()
    ck = quantized_model(preset, seed=0, device=dev, **{
        k: v for k, v in MS[shape].items() if k != "vocab"},
        vocab=MS[shape]["vocab"])
    model = QuantRWKV7(ck, device=dev)
    step_bytes = {B: decode_step_bytes(ck, B) for B in batches}
    del ck
    build_s = time.time() - t0
    out = {"build_s": round(build_s, 1)}
    g = torch.Generator(device=dev).manual_seed(2)
    for B in batches:
        ids = torch.randint(0, 65536, (n_tok, B), generator=g, device=dev)
        for t in range(4):                     # warm-up + capture
            model.decode_replay(B, ids[t])
        model.reset_replay_state(B)
        _mark()
        torch.cuda.synchronize()
        e0, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(2))
        e0.record()
        for t in range(n_tok):
            model.decode_replay(B, ids[t])
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / n_tok
        out[f"b{B}_ms_per_step"] = round(ms, 4)
        out[f"b{B}_tok_s"] = round(B * 1e3 / ms, 1)
    add_decode_roofline(out, step_bytes, ceiling)
    if 1 in batches:
        # batch 1 runs every layer in one persistent launch where the shape
        # and formats allow it (rwkvq_decode_mk), else one launch per kernel
        out["b1_path"] = ("persistent" if model._persistent(1, 1) is not None
                          else "per-kernel")
    return model, out


def prefill_bench(model, T, dev, reps=5):
    """pp512: full logits, fresh state; the graph captured for this shape is
    replayed after the ids are copied into its input buffer."""
    import torch
    g = torch.Generator(device=dev).manual_seed(3)
    idx = torch.randint(0, 65536, (1, T), generator=g, device=dev)
    st = model.init_state(1)
    model.forward_stateful(idx, st)              # capture + warm-up
    gr = model._seq_graphs[(1, T, False, 0)]
    _mark()
    torch.cuda.synchronize()
    e0, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(2))
    e0.record()
    for _ in range(reps):
        gr["idx"].copy_(idx)
        gr["graph"].replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    return {"T": T, "ms": round(ms, 3), "tok_s": round(T * 1e3 / ms, 1)}


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_head_rtn8_traffic.md")


def measured_traffic():
    """HBM bytes per launch of the head GEMV, from the two rocprofv3 --pmc
    passes (FETCH_SIZE, WRITE_SIZE) summarised in profiles/ -- counters are
    not readable from inside a run, so the figure is the committed one.
    Returns (bytes or None, source)."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1]), os.path.relpath(
                        TRAFFIC_FILE, ROOT)
    except OSError:
        pass
    return None, None


def pmc_pass(args, dev):
    """Small eager workloads for rocprofv3 --pmc passes (one dispatch per
    kernel launch, no graphs): 'set' = the 3-GEMV set, 'copy' = a plain
    fp32 copy kernel of 256 MiB (the counter calibration)."""
    import torch
    if args.pmc_pass == "copy":
        n = 64 << 20
        src = torch.ones(n, device=dev)
        dst = torch.empty(n, device=dev)
        for _ in range(args.steps):
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        print(f"pmc copy pass: {args.steps} x {n * 4} B read + {n * 4} B "
              f"written", flush=True)
        return
    from rwkv_quant.backends.hip.quant_linear import (QuantLinearV2,
                                                      SymQuantLinear)
    qts = build_set()
    lins = {n: (QuantLinearV2(qt) if n == "head" else SymQuantLinear(qt))
            for n, qt in qts.items()}
    x = {n: torch.randn(1, qt.shape[1], device=dev) for n, qt in qts.items()}
    y = {n: torch.empty(1, qt.shape[0], device=dev) for n, qt in qts.items()}
    for _ in range(args.steps):
        for n, lin in lins.items():
            lin.gemv_into(x[n], y[n])
    torch.cuda.synchronize()
    per = algorithmic_bytes(qts)
    print(f"pmc set pass: {args.steps} passes, algorithmic bytes per launch "
          f"{per}", flush=True)


def weight_elems(shape):
    """Matmul weight elements one token meets in the forward of the shape:
    r/k/v/o, channel-mix key/value, the LoRA factors (no v branch in layer
    0) and the head (1.39e9 for 1.5B, 2.78e9 for 2.9B)."""
    from rwkv_quant.models.synthetic import SHAPES as MS, lora_ranks
    sh = MS[shape]
    D, F, L = sh["n_embd"], sh["ffn"], sh["n_layer"]
    rk = lora_ranks(D)
    per = 4 * D * D + 2 * D * F + 2 * D * sum(rk.values())
    return L * per - 2 * D * rk["v"] + sh["vocab"] * D


MFMA_PEAK_TFLOPS = 2500.0        # dense fp16 / bf16, MI355X datasheet


def pp512(model, dev, T=512, shape="1.5b"):
    """Prefill of T tokens with the projection FLOP rate
    (2 * weight_elems(shape) per token): end to end, and over the GEMM
    kernels alone (gemm_only_ms) against the dense fp16 MFMA peak."""
    pf = prefill_bench(model, T, dev)
    flop = 2 * weight_elems(shape) * T
    pf["flop"] = flop
    pf["tflop_s"] = round(flop / (pf["ms"] * 1e-3) / 1e12, 2)
    gm = gemm_only_ms(model, T, dev)
    pf["gemm_ms"] = round(gm, 3)
    pf["gemm_tflop_s"] = round(flop / (gm * 1e-3) / 1e12, 1)
    pf["gemm_frac_mfma_peak"] = round(pf["gemm_tflop_s"] / MFMA_PEAK_TFLOPS,
                                      4)
    return pf


def stream_ceiling(dev, gib=2, blocks=(512, 1024, 2048, 4096, 8192),
                   reps=10):
    """Measured HBM read ceiling: rwkvq_probe_stream_read (16-byte loads,
    the GEMVs' access pattern) over a 2 GiB buffer, the best rate over a
    sweep of workgroup counts, HIP events on the launch stream."""
    import torch
    from rwkv_quant.backends.hip import _lib
    nbytes = gib << 30
    buf = torch.ones(nbytes, dtype=torch.uint8, device=dev)
    out = torch.empty(max(blocks), dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream()
    rates = {}
    for nb in blocks:
        for _ in range(2):
            _lib.call("rwkvq_probe_stream_read", _lib.ptr(buf), nbytes,
                      _lib.ptr(out), nb, _lib.stream_handle(st))
        e0, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(2))
        e0.record(st)
        for _ in range(reps):
            _lib.call("rwkvq_probe_stream_read", _lib.ptr(buf), nbytes,
                      _lib.ptr(out), nb, _lib.stream_handle(st))
        e1.record(st)
        torch.cuda.synchronize()
        rates[nb] = nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del buf
    torch.cuda.empty_cache()
    best = max(rates, key=rates.get)
    return {"gbs": round(rates[best], 1), "workgroups": best,
            "bytes": nbytes,
            "sweep_gbs": {str(k): round(v, 1) for k, v in rates.items()},
            "kernel": "rwkvq_probe_stream_read (16-byte loads, 256 threads "
                      "per workgroup)"}


def qt_bytes(qt):
    """Canonical `.rwkvq` bytes of one stored tensor (every field)."""
    import torch
    b = 0
    for v in vars(qt).values():
        if torch.is_tensor(v):
            b += v.numel() * v.element_size()
    return b


def decode_step_bytes(ck, B):
    """Algorithmic HBM bytes of one decode step of B sequences: every
    stored tensor once (canonical file bytes; the embedding table only for
    the B rows gathered), the fp32 WKV state read and written, the two
    token-shift rows read and written per layer, the fp32 logits out."""
    H, N = ck.n_embd // ck.head_size, ck.head_size
    w = 0
    for key, qt in ck.tensors.items():
        if key == "emb.weight":
            w += B * qt_bytes(qt) // qt.shape[0]
        else:
            w += qt_bytes(qt)
    state = ck.n_layer * B * (H * N * N * 4 * 2 + 2 * ck.n_embd * 4 * 2)
    return w + state + B * ck.vocab_size * 4


def add_decode_roofline(out, step_bytes, ceiling):
    """Per batch: achieved GB/s = algorithmic bytes per step / step time,
    against the 8 TB/s datasheet peak and the measured stream ceiling."""
    for key in list(out):
        if key.endswith("_ms_per_step"):
            b = key[:-len("_ms_per_step")]
            byt = step_bytes[int(b[1:])]
            gbs = byt / (out[key] * 1e-3) / 1e9
            out[f"{b}_bytes_per_step"] = byt
            out[f"{b}_gbs"] = round(gbs, 1)
            out[f"{b}_frac_hbm_peak"] = round(gbs / HBM_PEAK_GBS, 4)
            if ceiling:
                out[f"{b}_frac_stream_ceiling"] = round(gbs / ceiling, 4)


def gemm_only_ms(model, T, dev, reps=5):
    """Time of the prefill's GEMM kernels alone (every projection GEMM of
    every layer, the LoRA GEMMs and the head, on fp16 inputs of the right
    shapes), replayed from a HIP graph: the denominator of the prefill
    MFMA roofline."""
    import torch
    from rwkv_quant.backends.hip import _lib, quant_model as qm
    N = T
    wk = model._work_for(N)
    for t in (wk.xs16, wk.o16, wk.xk16, wk.hk16, wk.h16):
        t.zero_()
    wk.x.zero_()
    wk.xo.zero_()
    logits = torch.empty(N, model.vocab_size, device=dev)

    def run():
        for blk in model.blocks:
            orders = qm._x16_orders(blk)
            if orders is None:
                raise RuntimeError("layer without the fp16 GEMM path")
            tm, cm = blk.tmix, blk.cmix
            o_r, o_o, o_k, o_v = orders
            tm.run_rkv_lora_x16(wk, o_r)
            tm.o_proj.apply_into(wk.o16, wk.x, mode=_lib.EPI_ADD | _lib.X_F16,
                                 n=N)
            cm.key.apply_into(wk.xk16, wk.hk16, n=N,
                              mode=(_lib.EPI_RELU2 | _lib.X_F16 | _lib.Y_F16
                                    | (o_v << _lib.Y_ORDER_SHIFT)))
            cm.value.apply_into(wk.hk16, wk.x, mode=_lib.EPI_ADD | _lib.X_F16,
                                n=N)
        model.head.apply_into(wk.xo, logits, n=N)

    run()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(2))
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def cpu_info():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "cpus_visible": os.cpu_count(),
            "cpus_affinity": len(os.sched_getaffinity(0))}


def cpu_model_baseline(dev, budget_s=20.0):
    """The CPU oracle (numpy float64 restatement of the forward) on the
    1.5B compression model: ms per decode token at batch 1 and prefill
    tok/s on a 16-token prompt, on the host's cores."""
    import numpy as np
    from oracle.rwkv7_ref import RWKV7Oracle
    from rwkv_quant.models.synthetic import (SHAPES as MS, checkpoint_to,
                                             quantized_model)
    ck = quantized_model("compression", seed=0, device=dev, **{
        k: v for k, v in MS["1.5b"].items() if k != "vocab"},
        vocab=MS["1.5b"]["vocab"])
    ck = checkpoint_to(ck, "cpu")
    t0 = time.perf_counter()
    orc = RWKV7Oracle(ck)
    build = time.perf_counter() - t0
    del ck
    ids = np.random.default_rng(5).integers(0, 65536, size=(1, 18))
    st = orc.init_state(1)
    t0 = time.perf_counter()
    _, st = orc.forward_stateful(ids[:, :16], st)
    pf = time.perf_counter() - t0
    dec, n = 0.0, 0
    for t in range(16, 18):
        t0 = time.perf_counter()
        _, st = orc.forward_stateful(ids[:, t:t + 1], st)
        dec += time.perf_counter() - t0
        n += 1
        if dec > budget_s:
            break
    return {"decode_ms_per_token_b1": round(1e3 * dec / n, 1),
            "prefill_tok_s_t16": round(16 / pf, 2),
            "sample": f"oracle (numpy float64) forward of the 1.5B "
                      f"compression model: a 16-token prompt then {n} "
                      f"decode token(s); weights dequantized once "
                      f"({build:.0f} s, untimed)"}


def torch_cpu_ceiling(qts, cores, reps=3):
    """fp32 GEMV on weights dequantized once (untimed), torch CPU: what a
    CPU reaches when it does not dequantize per call."""
    import torch
    from oracle import codec_ref as cr
    per = algorithmic_bytes(qts)
    old = torch.get_num_threads()
    torch.set_num_threads(cores)
    try:
        Ws = {n: torch.from_numpy(cr.dequant_qt(qt)) for n, qt in qts.items()}
        xs = {n: torch.randn(1, qt.shape[1]) for n, qt in qts.items()}
        for n in Ws:
            xs[n] @ Ws[n].T
        t0 = time.perf_counter()
        for _ in range(reps):
            for n in Ws:
                xs[n] @ Ws[n].T
        t = (time.perf_counter() - t0) / reps
    finally:
        torch.set_num_threads(old)
    f32 = sum(w.numel() * 4 for w in Ws.values())
    return {"ms_per_set": round(t * 1e3, 2),
            "set_gbs_algorithmic": round(sum(per.values()) / t / 1e9, 2),
            "fp32_weight_gbs": round(f32 / t / 1e9, 2), "threads": cores}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=4)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-model", action="store_true",
                    help="skip the 1.5B decode / pp512 measurements")
    ap.add_argument("--decode-tokens", type=int, default=128)
    ap.add_argument("--only", choices=("decode", "prefill", "decode2.9b",
                                       "prefill2.9b"), default=None,
                    help="run one model workload alone (for a per-workload "
                         "rocprofv3 profile); prints that section only")
    ap.add_argument("--decode-batches", default=None,
                    help="decode batch sizes for --only decode (default 1,8; "
                         "1,32 for decode2.9b)")
    ap.add_argument("--no-2p9b", action="store_true",
                    help="skip the 2.9B decode / pp2048 measurements")
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="print the per-kernel table of a rocprofv3 kernel "
                         "trace after its last marker kernel and exit")
    ap.add_argument("--pmc-pass", choices=("set", "copy"), default=None,
                    help="run a short eager workload for a rocprofv3 --pmc "
                         "pass and exit (no JSON line)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for "
              f"--gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.trace_summary:
        trace_summary(args.trace_summary)
        return

    import torch
    from rwkv_quant.backends.hip import _lib
    _lib.load()
    dev = torch.device("cuda:0")
    if args.pmc_pass:
        pmc_pass(args, dev)
        return
    if args.only in ("decode", "decode2.9b"):
        big = args.only == "decode2.9b"
        bs = tuple(int(b) for b in (args.decode_batches or (
            "1,32" if big else "1,8")).split(","))
        _, dec = decode_bench("compression", bs, args.decode_tokens, dev,
                              "2.9b" if big else "1.5b",
                              stream_ceiling(dev)["gbs"])
        key = "decode_2p9b_compression" if big else "decode_1p5b_compression"
        print(json.dumps({key: dec}), flush=True)
        return
    if args.only == "prefill":
        model, _ = decode_bench("reduction", (), 0, dev)
        print(json.dumps({"pp512_1p5b_reduction":
                          pp512(model, dev)}), flush=True)
        return
    if args.only == "prefill2.9b":
        model, _ = decode_bench("reduction", (), 0, dev, "2.9b")
        print(json.dumps({"pp2048_2p9b_reduction":
                          pp512(model, dev, 2048, "2.9b")}), flush=True)
        return
    ceiling = stream_ceiling(dev)
    qts = build_set()
    per = algorithmic_bytes(qts)
    set_bytes = sum(per.values())
    ms_per_step, steps, kern = gemv_set_bench(args, qts, dev)
    achieved = per["head"] / (kern["head"] * 1e-3) / 1e9
    value = set_bytes / (ms_per_step * 1e-3) / 1e9
    traffic, traffic_src = measured_traffic()

    out = {
        "metric": "quant GEMV GB/s (% HBM peak)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8/u8 codes, x as fp16 hi+lo (about 22 bits), fp32 accumulate",
        "data": "synthetic (seeded N(0,0.02) weights, 0.1% x20 outlier "
                "columns, bf16 N(0,1) x)",
        "config": {"workload": "configs[1]: sym@6 cmix key 2048->8192 + "
                               "value 8192->2048 + rtn@8 head 2048->65536, "
                               "batch 1, HIP-graph replay over 4 device "
                               "copies (650 MB)",
                   "set_bytes": set_bytes, "copies": args.copies},
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "kernels_us": {n: round(v * 1e3, 3) for n, v in kern.items()},
        "roofline": {"bound": "hbm", "kernel": "gemv_kernel<F_RTN8> (head)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "traffic_source": traffic_src,
                     "launch_us": round(kern["head"] * 1e3, 3),
                     "bytes_per_launch": per["head"],
                     "frac_stream_ceiling": round(achieved / ceiling["gbs"],
                                                  4)},
        "stream_ceiling": ceiling,
        "cpu_baseline": None,
    }
    if not args.no_model:
        model, dec = decode_bench("compression", (1, 8), args.decode_tokens,
                                  dev, ceiling=ceiling["gbs"])
        out["decode_1p5b_compression"] = dec
        del model
        torch.cuda.empty_cache()
        model, dec_r = decode_bench("reduction", (1,), 32, dev,
                                    ceiling=ceiling["gbs"])
        out["decode_1p5b_reduction"] = dec_r
        out["pp512_1p5b_reduction"] = pp512(model, dev)
        del model
        torch.cuda.empty_cache()
    if not args.no_model and not args.no_2p9b:
        # 2.9B shape, decode at batch 1 and 32, prefill T=2048
        model, dec = decode_bench("compression", (1, 32), 64, dev, "2.9b",
                                  ceiling["gbs"])
        out["decode_2p9b_compression"] = dec
        del model
        torch.cuda.empty_cache()
        model, dec_r = decode_bench("reduction", (1,), 32, dev, "2.9b",
                                    ceiling["gbs"])
        out["decode_2p9b_reduction"] = dec_r
        out["pp2048_2p9b_reduction"] = pp512(model, dev, 2048, "2.9b")
        del model
        torch.cuda.empty_cache()
    if not args.no_cpu:
        info = cpu_info()
        cores = min(info["cpus_affinity"], CPU_SHARE)
        cb = cpu_baseline(qts, cores=cores)
        one = cpu_baseline(qts, budget_s=6.0, cores=1)
        cb.update(info)
        cb["cores_note"] = (f"{cores} threads: the GPU box's host share for "
                            f"one GPU ({info['cpus_affinity']} visible in "
                            f"the affinity mask)")
        cb["one_thread"] = {"value": one["value"], "sample": one["sample"]}
        cb["torch_f32_predequantized"] = torch_cpu_ceiling(qts, cores)
        if not args.no_model:
            cb["model_1p5b_compression"] = cpu_model_baseline(dev)
        out["cpu_baseline"] = cb
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
