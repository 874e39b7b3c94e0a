"""Benchmark of the bf16 matrix-multiplication path on one MI355X.

The step (the metric's M=2048 case): the four
prefill GEMMs of one layer of a 4B-class dense model at M=2048 rows --
QKV 2560->4608 (Out::Bf16), O 4096->2560 (Out::Residual), gate|up
2560->18432 (Out::Bf16), down 9216->2560 (Out::Residual) -- with bf16
inputs ~N(0,1) / N(0,0.02) from the seeded generator, f32 accumulation and
one rounding at the output, each GEMM on the kernel the selection layer
picked at load (QwenEngine::gemm with gemm.auto, src/metal/qwen.rs:2200).
`value` = the step's algorithmic flops (2*M*N*K summed) / its GPU time,
inputs resident in HBM, timed with HIP events on the library's stream, after
W warmup steps and HEAT_S seconds of the step (the GPU's sustained clocks).

Also reported (not part of `value`): BASELINE config 1 (one GEMM, M=512),
config 2 at M=512 and 1024, config 4 (27B-class shapes and lm_head at
M=2048) under "prefill_more"; the decode steps at M=4 and 8; BASELINE config 5's MoE layer (the grouped expert GEMMs
against HBM, and as TFLOP/s), and (the metric's second half) the decode matvec, M=1, over
four layers of the same weights plus the lm_head (K=2560, N=151936), 2.2 GB
streamed per step, as GB/s of algorithmic bytes (2*N*K + 2*M*K + 2*M*N per
projection, + 2*M*N for Residual) against HBM's 8 TB/s.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--tune key=value,...]

roofline.traffic (HBM bytes per launch of the dominant kernel) comes from
profiles/traffic.json, written from two counter runs of this file:

    rocprofv3 --pmc FETCH_SIZE -d F -o run --output-format csv -- python3 bench.py --traffic-run
    rocprofv3 --pmc WRITE_SIZE -d W -o run --output-format csv -- python3 bench.py --traffic-run
    python3 bench.py --traffic-summary F/run_counter_collection.csv W/run_counter_collection.csv

The kernel-trace summary in profiles/ comes from

    rocprofv3 --kernel-trace --stats -d P -o bench --output-format csv -- python3 bench.py --steps 20 > B
    python3 bench.py --trace-summary P/bench_kernel_trace.csv B '<that rocprofv3 command>'

--traffic-run selects the step's kernels (every candidate is dispatched, so
every candidate gets counters) and copies COPY_BYTES device to device; the
summary scales each kernel's FETCH_SIZE and WRITE_SIZE (KiB per dispatch)
by what the same counter reads for that copy (COPY_BYTES read, COPY_BYTES
written).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "herbert-metal-bf16_amd"))

import numpy as np  # noqa: E402

MFMA_BF16_PEAK = 2500.0  # TFLOP/s, dense bf16 MFMA, MI355X
HBM_PEAK = 8000.0  # GB/s
M = 2048
LAYER = [("qkv", 2560, 4608, 0), ("o", 4096, 2560, 2), ("gate_up", 2560, 18432, 0),
         ("down", 9216, 2560, 2)]
LM_HEAD = ("lm_head", 2560, 151936, 0)
QKV_REAL = [("qkv10240", 2560, 10240, 0)]
CONFIG1 = [("gemm", 1024, 3584, 0)]
CONFIG4 = [("qkv", 5120, 7168, 0), ("gate_up", 5120, 34816, 0), ("down", 17408, 5120, 2),
           ("lm_head", 5120, 151936, 0)]
DECODE_LAYERS = 4
SEED = 0x5EED0002  # config 2's seeds: X = SEED + 2i, W = SEED + 2i + 1
COPY_BYTES = 1 << 28  # the calibration copy of the traffic counters
MARK_BYTES = 7 * 4096  # the trace marker fill: 7 workgroups of 256 threads
# Seconds of continuous load before each timed region (after the W warmup
# steps): the reference's auto.heat (qwen.rs:2575-2591), which brings the GPU
# to its sustained regime.  On MI355X that regime is the faster one: the
# M=2048 step measured 410-418 us right after a start or 3-5 s idle against
# 355-359 us after 1-15 s of load (the clocks ramp up under load); without a
# heat, K=20 steps (8 ms) are timed mostly before the ramp.
HEAT_S = 1.0
COUNTER_RUN = False
GRAPH = False  # --graph: the decode steps also timed as recorded graphs


# Named regions of the run: each timed region is bracketed by two marker
# fills (a dispatch of MARK_BYTES / 16 threads that a kernel trace or a
# counter run tells apart by its grid), and its name appended here in the
# order the regions ran; the JSON line carries the list ("regions"), so the
# trace and counter summaries attribute each dispatch to its case.
REGIONS = []
_MARK = {}


class region:
    def __init__(self, g, name):
        self.g, self.name = g, name

    def __enter__(self):
        if self.g not in _MARK:
            _MARK[self.g] = self.g.alloc(MARK_BYTES)
        self.g.zero(_MARK[self.g])
        return self

    def __exit__(self, *a):
        self.g.zero(_MARK[self.g])
        REGIONS.append(self.name)


def heat(g, ops, seconds=None):
    """The ops run back to back, ~50 ms a submission, until `seconds` (HEAT_S
    by default) of GPU time have passed (untimed)."""
    seconds = HEAT_S if seconds is None else seconds
    if seconds <= 0:
        return
    one = g.time_ops(ops, 1)
    reps = int(max(1, min(4096, 0.05 / max(one, 1e-6))))
    total = 0.0
    while total < seconds:
        total += g.time_ops(ops, reps)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _median3(fn):
    ts = []
    for _ in range(3):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return sorted(ts)[1]


def cpu_baseline(rows):
    """The contract's scalar CPU restatement (oracle/hb_oracle.c: f32 sums
    in increasing k, one rounding) on the host's cores, each figure the
    median of 3 runs: the metric's GEMMs over `rows` rows of each of the
    step's four (the headline `value`), and beside it config 1 whole, the
    decode step at M=1 (four layers + lm_head) and the MoE layer's grouped
    GEMMs over a sample of tokens."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import hb_oracle as orc
    import herbert_hip as hb
    host = os.cpu_count() or 1
    # The GPU box gives one GPU's job a share of 16 host CPUs, whatever
    # os.cpu_count() reports there; this build's container has 8.
    threads = min(16, host)
    flops, secs = 0.0, 0.0
    for i, (name, k, n, out) in enumerate(LAYER):
        x = hb.normal_bf16(SEED + 2 * i, 1.0, (rows, k))
        w = hb.normal_bf16(SEED + 2 * i + 1, 0.02, (n, k))
        y0 = hb.normal_bf16(SEED + 100 + i, 1.0, (rows, n)) if out == 2 else None
        secs += _median3(lambda: orc.gemm(x, w, out, y0, threads=threads))
        flops += 2.0 * rows * n * k
    res = {"value": flops / secs / 1e12, "unit": "TFLOP/s", "cores": threads, "host_cpus": host,
           "kind": "port", "median_of": 3,
           "sample": "%d of the %d rows of each of the 4 GEMMs (oracle/hb_oracle.c, scalar f32 in k "
                     "order, %d threads: the box's CPU share for one GPU), %.1f s per run" % (
                         rows, M, threads, secs)}
    # config 1, whole
    k, n = CONFIG1[0][1], CONFIG1[0][2]
    x = hb.normal_bf16(0x5EED0001, 1.0, (512, k))
    w = hb.normal_bf16(0x5EED0002, 0.02, (n, k))
    t = _median3(lambda: orc.gemm(x, w, 0, threads=threads))
    res["config1"] = {"value": round(2.0 * 512 * n * k / t / 1e12, 4), "unit": "TFLOP/s", "s": round(t, 3)}
    # decode M=1: the step's weights (4 layers + lm_head) streamed once
    nbytes, t = 0.0, 0.0
    for name, k, n, o in LAYER + [LM_HEAD]:
        layers = 1 if name == "lm_head" else DECODE_LAYERS
        w = hb.normal_bf16(0x5EED0003 + n, 0.02, (n, k))
        x = hb.normal_bf16(0x5EED0003, 1.0, (1, k))
        y0 = hb.normal_bf16(5, 1.0, (1, n)) if o == 2 else None
        t += layers * _median3(lambda: orc.gemm(x, w, o, y0, threads=threads))
        nbytes += layers * (2.0 * n * k + 2.0 * k + 2.0 * n * (2 if o == 2 else 1))
    res["decode_m1"] = {"value": round(nbytes / t / 1e9, 2), "unit": "GB/s", "s": round(t, 3)}
    # MoE (config 5): the grouped gate|up and down over 256 of the 2048
    # tokens (their route from the seeded logits), all 256 experts' weights
    T5, E, TOPK, H, MI = 256, 256, 8, 2048, 512
    scores = hb.normal_bf16(0x5EED0005, 1.0, (T5, E))
    route = orc.route(scores, TOPK)
    lst, tiles = orc.moe_sort(route, TOPK, E, 64)
    wgu = hb.normal_bf16(0x5EED0006, 0.02, (E * 2 * MI, H))
    wdn = hb.normal_bf16(0x5EED0007, 0.02, (E * H, MI))
    xx = hb.normal_bf16(0x5EED0008, 1.0, (T5, H))
    P = T5 * TOPK
    hh = hb.normal_bf16(0x5EED0009, 1.0, (P, MI))
    t = _median3(lambda: (orc.experts_gemm(xx, wgu, lst, tiles, H, 2 * MI, 1, TOPK, P, threads=threads),
                          orc.experts_gemm(hh, wdn, lst, tiles, MI, H, 2, TOPK, P, threads=threads)))
    res["moe"] = {"value": round(2.0 * P * 3 * MI * H / t / 1e12, 4), "unit": "TFLOP/s", "s": round(t, 3),
                  "sample": "%d tokens x top %d, the grouped gate|up and down" % (T5, TOPK)}
    return res


def yardstick(steps):
    """hipBLASLt through torch.matmul (bf16, the same shapes and seeds) as a
    yardstick for the prefill GEMMs: each shape alone, warm, and the four
    of the step back to back.  Printed as text (profiles/); torch is used
    here only, never by the library."""
    import torch
    import herbert_hip as hb
    dev = torch.device("cuda:0")

    def t_of(fn, reps):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / 1e3 / reps

    lines = ["hipBLASLt (torch %s, torch.matmul bf16 -> bf16) on %s" % (torch.__version__,
                                                                         torch.cuda.get_device_name(0))]
    mats = []
    for i, (name, k, n, out) in enumerate(LAYER):
        x = torch.from_numpy(hb.normal_bf16(SEED + 2 * i, 1.0, (M, k)).view(np.int16)).view(torch.bfloat16).to(dev)
        w = torch.from_numpy(hb.normal_bf16(SEED + 2 * i + 1, 0.02, (n, k)).view(np.int16)).view(torch.bfloat16).to(dev)
        mats.append((name, k, n, x, w))
        t = t_of(lambda: torch.matmul(x, w.t()), steps)
        lines.append("  %-8s M=%d K=%d N=%d alone: %8.2f us %7.1f TFLOP/s" % (name, M, k, n, t * 1e6,
                                                                             2.0 * M * n * k / t / 1e12))
    step = lambda: [torch.matmul(x, w.t()) for _, _, _, x, w in mats]  # noqa: E731
    t = t_of(step, steps)
    fl = sum(2.0 * M * n * k for _, k, n, _, _ in mats)
    lines.append("  step (qkv, o, gate_up, down back to back): %8.2f us %7.1f TFLOP/s" % (t * 1e6, fl / t / 1e12))
    # config 1 and config 2 at M=512 and 1024, the same seeds as the bench's sets
    x1 = torch.from_numpy(hb.normal_bf16(0x5EED0001, 1.0, (512, 1024)).view(np.int16)).view(torch.bfloat16).to(dev)
    w1 = torch.from_numpy(hb.normal_bf16(0x5EED0002, 0.02, (3584, 1024)).view(np.int16)).view(torch.bfloat16).to(dev)
    t = t_of(lambda: torch.matmul(x1, w1.t()), steps)
    lines.append("  config 1 (M=512 K=1024 N=3584): %8.2f us %7.1f TFLOP/s" % (t * 1e6, 2.0 * 512 * 1024 * 3584 / t / 1e12))
    for mm in (512, 1024):
        sub = [(name, k, n, x[:mm].contiguous(), w) for name, k, n, x, w in mats]
        t = t_of(lambda: [torch.matmul(x, w.t()) for _, _, _, x, w in sub], steps)
        fl = sum(2.0 * mm * n * k for _, k, n, _, _ in sub)
        lines.append("  config 2 at M=%d, the four back to back: %8.2f us %7.1f TFLOP/s" % (mm, t * 1e6, fl / t / 1e12))
    s = 8192
    a = torch.randn(s, s, device=dev, dtype=torch.bfloat16)
    bmat = torch.randn(s, s, device=dev, dtype=torch.bfloat16)
    t = t_of(lambda: torch.matmul(a, bmat.t()), 10)
    lines.append("  8192^3: %8.2f us %7.1f TFLOP/s" % (t * 1e6, 2.0 * s ** 3 / t / 1e12))
    print("\n".join(lines), flush=True)


def main():
    global HEAT_S, COUNTER_RUN, GRAPH
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--tune", default="")
    ap.add_argument("--heat", type=float, default=HEAT_S,
                    help="seconds of load before each timed region (0: none, the cold-clock figures)")
    ap.add_argument("--cpu-rows", type=int, default=512)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-matvec", action="store_true")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="also time each decode step recorded as one HIP graph (not under a profiler)")
    ap.add_argument("--traffic-run", action="store_true")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"))
    ap.add_argument("--counter-run", action="store_true",
                    help="the bench's regions with --heat 0 and then the calibration copy, for rocprofv3 --pmc")
    ap.add_argument("--picks-out", metavar="FILE", help="write the engine's choices (hb_engine_picks) to FILE")
    ap.add_argument("--picks-in", metavar="FILE",
                    help="seed the engine's choices from FILE (hb_engine_pin): the same kernels as that run")
    ap.add_argument("--counter-summary", nargs="+", metavar="BENCH_OUT CSV",
                    help="that run's stdout, then one counter_collection.csv per counter pass")
    ap.add_argument("--trace-summary", nargs=3, metavar=("TRACE_CSV", "BENCH_OUT", "COMMAND"))
    ap.add_argument("--yardstick", action="store_true",
                    help="time hipBLASLt (torch.matmul) on the step's shapes instead")
    args = ap.parse_args()
    if args.traffic_summary:
        traffic_summary(*args.traffic_summary)
        return
    if args.counter_summary:
        counter_summary(args.counter_summary[0], args.counter_summary[1:])
        return
    if args.trace_summary:
        trace_summary(*args.trace_summary)
        return
    if args.yardstick:
        yardstick(args.steps)
        return
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only (--gpus %d asked); the path would shard "
              "each GEMM by N across GPUs, which is not built" % args.gpus, file=sys.stderr)
        sys.exit(2)

    HEAT_S = 0.0 if args.counter_run else max(0.0, args.heat)
    COUNTER_RUN = args.counter_run
    GRAPH = args.graph
    import herbert_hip as hb
    g = hb.Gpu(0)
    log("[gpu]", g.summary())
    e = hb.Engine(g, args.tune)
    if args.picks_in:
        e.pin(open(args.picks_in).read())
    state = g.alloc_with(np.array([0, 0, 0, M], np.uint32))
    bufs, ops, flops, per_gemm = [], [], 0.0, {}
    t0 = time.time()
    for i, (name, k, n, out) in enumerate(LAYER):
        X = g.alloc_with(hb.normal_bf16(SEED + 2 * i, 1.0, (M, k)))
        W = g.alloc_with(hb.normal_bf16(SEED + 2 * i + 1, 0.02, (n, k)))
        Y = g.alloc_with(hb.normal_bf16(SEED + 100 + i, 1.0, (M, n)))
        bufs += [X, W, Y]
        kern = e.gemm(k, n, out, hb.r(state), hb.r(W), hb.r(X), hb.r(Y), M)
        op = hb.Op(kern, [hb.r(state), hb.r(W), hb.r(X), hb.r(Y), hb.r(state), hb.r(state)], M)
        ops.append(op)
        f = 2.0 * M * n * k
        flops += f
        per_gemm[name] = {"kernel": g.kernel_name(kern), "flops": f, "op": op}
    log("[bench] selection done in %.1f s" % (time.time() - t0))
    if args.traffic_run:
        traffic_run(g, e, ops, per_gemm)
        return

    # Warmup, then exactly K steps between two synchronisations (events at
    # the ends only): the step time.  Then K more steps with an event after
    # every launch: each GEMM's mean launch time (the gap an event adds
    # between launches counts in it, so these are upper bounds).
    g.time_ops(ops, max(args.warmup, 0)) if args.warmup > 0 else None
    heat(g, ops)
    g.sync()
    with region(g, "step_m2048"):
        t = g.time_ops(ops, args.steps)
        g.sync()
        t_ev, each = g.time_each(ops, args.steps)
        g.sync()
    ms = t / args.steps * 1e3
    value = flops / (t / args.steps) / 1e12

    # The dominant kernel's roofline.
    for (name, d), s in zip(per_gemm.items(), each):
        d["us"] = s * 1e6
        d["tflops"] = d["flops"] / s / 1e12
    dom = max(per_gemm, key=lambda nm: per_gemm[nm]["us"])
    dd = per_gemm[dom]
    roofline = {"bound": "mfma", "achieved": round(dd["tflops"], 1), "peak": MFMA_BF16_PEAK,
                "unit": "TFLOP/s", "frac": round(dd["tflops"] / MFMA_BF16_PEAK, 4), "traffic": None,
                "kernel": dd["kernel"], "gemm": dom, "launch_us": round(dd["us"], 2)}
    tr = traffic_of(dd["kernel"])
    if tr:
        roofline["traffic"] = tr["bytes"]

    result = {
        "metric": "bf16 GEMM TFLOP/s + % MFMA peak (M=2048); decode matvec HBM GB/s + % peak",
        "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "4B-class layer prefill GEMMs (qkv, o, gate_up, down) at M=2048 "
                               "(BASELINE configs[1])", "m": M,
                   "gemms": {nm: {"k": k, "n": n, "out": ["Bf16", "F32", "Residual"][o],
                                  "kernel": per_gemm[nm]["kernel"],
                                  "us": round(per_gemm[nm]["us"], 2),
                                  "tflops": round(per_gemm[nm]["tflops"], 1)}
                             for nm, k, n, o in LAYER}},
        "roofline": roofline,
        "ms_per_step_launch_events": round(t_ev / args.steps * 1e3, 4),
        "heat_s": HEAT_S,
    }
    for b in bufs:
        g.free(b)

    if not args.no_extra:
        result["prefill_more"] = bench_prefill_more(g, e, hb, args.steps)

    if not args.no_matvec:
        result["matvec"] = bench_matvec(g, e, hb)
    if not args.no_moe:
        result["moe"] = bench_moe(g, e, hb)
    e.log_summary()
    if args.picks_out:
        with open(args.picks_out, "w") as fh:
            fh.write(e.picks())
    if args.counter_run:
        counter_run(g, hb)
    e.close()
    g.close()
    if not args.no_cpu and not args.counter_run:
        result["cpu_baseline"] = cpu_baseline(args.cpu_rows)
    result["regions"] = REGIONS
    print(json.dumps(result), flush=True)


def traffic_of(kernel, where="step_m2048"):
    """The kernel's HBM bytes per launch in region `where` from
    profiles/counters.json (FETCH_SIZE + WRITE_SIZE of its full-size
    dispatches, scaled), else from profiles/traffic.json, or None."""
    path = os.path.join(ROOT, "profiles", "counters.json")
    if os.path.exists(path):
        c = json.load(open(path)).get(where, {}).get(kernel)
        if c and "bytes" in c:
            return {"bytes": c["bytes"], "fetch_bytes": c["fetch_bytes"], "write_bytes": c["write_bytes"]}
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    return json.load(open(path)).get(kernel)


def gemm_set(g, e, hb, shapes, m, steps, seed, tag):
    """The GEMMs `shapes` [(name, K, N, out)] over m rows, each on the kernel
    the selection layer picks, run back to back: the set's TFLOP/s and each
    GEMM's (launch-event) time."""
    state = g.alloc_with(np.array([0, 0, 0, m], np.uint32))
    bufs, ops, flops = [state], [], []
    for i, (name, k, n, out) in enumerate(shapes):
        X = g.alloc_with(hb.normal_bf16(seed + 2 * i, 1.0, (m, k)))
        W = g.alloc_with(hb.normal_bf16(seed + 2 * i + 1, 0.02, (n, k)))
        Y = g.alloc_with(hb.normal_bf16(seed + 100 + i, 1.0, (m, n)))
        bufs += [X, W, Y]
        kern = e.gemm(k, n, out, hb.r(state), hb.r(W), hb.r(X), hb.r(Y), m)
        ops.append(hb.Op(kern, [hb.r(state), hb.r(W), hb.r(X), hb.r(Y), hb.r(state), hb.r(state)], m))
        flops.append(2.0 * m * n * k)
    g.time_ops(ops, 2)
    heat(g, ops)
    with region(g, tag):
        t = g.time_ops(ops, steps)
        _, each = g.time_each(ops, steps)
    g.sync()
    out = {"m": m, "tflops": round(sum(flops) / (t / steps) / 1e12, 1),
           "frac": round(sum(flops) / (t / steps) / 1e12 / MFMA_BF16_PEAK, 4),
           "us": round(t / steps * 1e6, 2), "gemms": {}}
    for (name, k, n, o), op, f, s in zip(shapes, ops, flops, each):
        out["gemms"][name] = {"k": k, "n": n, "kernel": g.kernel_name(op.kernel), "us": round(s * 1e6, 2),
                              "tflops": round(f / s / 1e12, 1), "frac": round(f / s / 1e12 / MFMA_BF16_PEAK, 4)}
    for b in bufs:
        g.free(b)
    return out


def bench_prefill_more(g, e, hb, steps):
    """The other prefill cases of BASELINE.json: config 1 (one GEMM, M=512,
    K=1024, N=3584), config 2 at M=512 and 1024 (the step above is M=2048),
    config 4 (27B-class shapes at M=2048, lm_head included), and the
    reference's real 4B fused QKV (2560 -> 10240) at M=512, 1024, 2048."""
    steps = max(3, min(steps, 10))
    res = {"config1": gemm_set(g, e, hb, CONFIG1, 512, steps, 0x5EED0001, "config1")}
    # config 1's kernel name is its own (no other case has 1024 x 3584), so
    # its traffic counters are config 1's: HBM bytes per launch against the
    # algorithmic 2*(M*K + N*K + M*N).
    c1 = res["config1"]["gemms"]["gemm"]
    tr = traffic_of(c1["kernel"], "config1")
    k, n = CONFIG1[0][1], CONFIG1[0][2]
    c1["algorithmic_bytes"] = 2 * (512 * k + n * k + 512 * n)
    c1["traffic"] = tr["bytes"] if tr else None
    for m in (512, 1024):
        res["config2_m%d" % m] = gemm_set(g, e, hb, LAYER, m, steps, SEED, "config2_m%d" % m)
    # The reference's real Qwen3.5-4B fused QKV width: q_width = 2 * heads *
    # head_dim carries the output gate, 8192 + 2 * 1024 = 10240 columns
    # (qwen_kernels.rs:41-51, probe.rs:738-741), where BASELINE's config 2
    # names 2560 + 2 * 1024: reported beside it, at each block size.
    for m in (512, 1024, 2048):
        res["qkv10240_m%d" % m] = gemm_set(g, e, hb, QKV_REAL, m, steps, SEED + 40, "qkv10240_m%d" % m)
    res["config4_m2048"] = gemm_set(g, e, hb, CONFIG4, M, steps, 0x5EED0004, "config4_m2048")
    return res


def traffic_run(g, e, ops, per_gemm):
    """The picked kernels a few times, config 1's GEMM (its selection and
    pick), then the calibration copy (a device to device copy of
    COPY_BYTES, HIP's blit kernel)."""
    import herbert_hip as hb
    g.time_ops(ops, 3)
    g.sync()
    c1 = gemm_set(g, e, hb, CONFIG1, 512, 3, 0x5EED0001, "config1")
    g.sync()
    a, b = g.alloc(COPY_BYTES), g.alloc(COPY_BYTES)
    g.zero(a)
    for _ in range(5):
        g.copy(hb.r(b), hb.r(a))
    g.sync()
    g.free(a)
    g.free(b)
    print(json.dumps({"picked": {nm: d["kernel"] for nm, d in per_gemm.items()},
                      "config1": c1["gemms"]["gemm"]["kernel"], "copy_bytes": COPY_BYTES}), flush=True)


def counter_run(g, hb):
    """After the bench's regions (run with --counter-run: heat 0, few
    steps), the calibration copy in a region of its own: COPY_BYTES read
    and COPY_BYTES written by HIP's blit kernel."""
    a, b = g.alloc(COPY_BYTES), g.alloc(COPY_BYTES)
    g.zero(a)
    g.sync()
    with region(g, "calibration"):
        for _ in range(5):
            g.copy(hb.r(b), hb.r(a))
    g.sync()
    g.free(a)
    g.free(b)


# Derived columns of the counter summary: FETCH_SIZE / WRITE_SIZE scaled by
# what they read for the calibration copy; the L2 hit rate; the MFMA pipes'
# busy cycles per SIMD (1024 SIMDs), as microseconds at 2.4 GHz, to set
# beside the kernel's own duration.
SIMDS, CLOCK_MHZ = 1024, 2400.0
# How profiles/counters.json and counters_summary.txt are made (P = picks
# file, from a plain run; the three counter passes run on those picks, so
# every pass measures the same kernels).
COUNTER_COMMANDS = [
    "commands (cd /tmp && export TMPDIR=/tmp first; R = the repository):",
    "  python3 R/bench.py --no-cpu --picks-out P",
    "  rocprofv3 --pmc FETCH_SIZE -d C1 -o run --output-format csv -- "
    "python3 R/bench.py --counter-run --picks-in P --steps 3 --warmup 1 --no-cpu > B",
    "  rocprofv3 --pmc WRITE_SIZE TCC_HIT_sum TCC_MISS_sum -d C2 -o run --output-format csv -- "
    "python3 R/bench.py --counter-run --picks-in P --steps 3 --warmup 1 --no-cpu",
    "  rocprofv3 --pmc SQ_INSTS_MFMA SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_WAIT_INST_ANY SQ_WAVE_CYCLES "
    "-d C3 -o run --output-format csv -- python3 R/bench.py --counter-run --picks-in P --steps 3 --warmup 1 --no-cpu",
    "  python3 R/bench.py --counter-summary B C1/run_counter_collection.csv C2/run_counter_collection.csv "
    "C3/run_counter_collection.csv",
    ""]


def counter_summary(bench_out, csvs):
    """profiles/counters.json and profiles/counters_summary.txt from
    `rocprofv3 --pmc ... --output-format csv` runs of `bench.py
    --counter-run` (one per counter pass) and that run's stdout: each
    dispatch attributed to the region it ran in (between the marker fills,
    named by the JSON line's "regions"), then per region and kernel the
    median of each counter over its full-size dispatches."""
    import csv
    import statistics
    b = None
    for ln in open(bench_out):
        if ln.startswith("{") and '"regions"' in ln:
            b = json.loads(ln)
    if b is None:
        sys.exit("counter summary: no JSON line with regions in %s" % bench_out)
    names = b["regions"]
    acc = {}
    for path in csvs:
        disp = {}
        for r in csv.DictReader(open(path)):
            d = disp.setdefault(int(r["Dispatch_Id"]), {"k": r["Kernel_Name"], "grid": int(r["Grid_Size"]), "c": {}})
            d["c"][r["Counter_Name"]] = d["c"].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        seq = [disp[i] for i in sorted(disp)]
        marks = [i for i, d in enumerate(seq) if d["k"].startswith("fill_zero") and d["grid"] == MARK_BYTES // 16]
        if len(marks) != 2 * len(names):
            sys.exit("counter summary: %s holds %d markers for %d regions" % (path, len(marks), len(names)))
        for ri, nm in enumerate(names):
            for d in seq[marks[2 * ri] + 1:marks[2 * ri + 1]]:
                acc.setdefault(nm, {}).setdefault(d["k"], []).append((d["grid"], d["c"]))
    out = {}
    for nm, kern in acc.items():
        for k, v in kern.items():
            top = max(gs for gs, _ in v)
            full = [c for gs, c in v if gs == top]
            cnames = sorted({cn for c in full for cn in c})
            out.setdefault(nm, {})[k] = {"dispatches": len(full), "grid": top}
            out[nm][k].update({cn: statistics.median(c[cn] for c in full if cn in c) for cn in cnames})
    cal = out.get("calibration", {})
    copy = next((v for k, v in cal.items() if "copyBuffer" in k), None)
    if not copy or "FETCH_SIZE" not in copy or "WRITE_SIZE" not in copy:
        sys.exit("counter summary: no calibration copy with FETCH_SIZE and WRITE_SIZE")
    kib = COPY_BYTES / 1024.0
    sf, sw = kib / copy["FETCH_SIZE"], kib / copy["WRITE_SIZE"]
    for nm, kern in out.items():
        for k, c in kern.items():
            if "FETCH_SIZE" in c:
                c["fetch_bytes"] = round(c["FETCH_SIZE"] * sf * 1024.0)
            if "WRITE_SIZE" in c:
                c["write_bytes"] = round(c["WRITE_SIZE"] * sw * 1024.0)
            if "fetch_bytes" in c and "write_bytes" in c:
                c["bytes"] = c["fetch_bytes"] + c["write_bytes"]
            if c.get("TCC_HIT_sum", 0) + c.get("TCC_MISS_sum", 0) > 0:
                c["l2_hit_rate"] = round(c["TCC_HIT_sum"] / (c["TCC_HIT_sum"] + c["TCC_MISS_sum"]), 4)
            if "SQ_VALU_MFMA_BUSY_CYCLES" in c:
                c["mfma_busy_us_per_simd"] = round(c["SQ_VALU_MFMA_BUSY_CYCLES"] / SIMDS / CLOCK_MHZ, 3)
    out["_calibration"] = {"copy_bytes": COPY_BYTES, "fetch_scale": round(sf, 4), "write_scale": round(sw, 4),
                           "simds": SIMDS, "clock_mhz": CLOCK_MHZ}
    path = os.path.join(ROOT, "profiles", "counters.json")
    with open(path, "w") as fh:
        json.dump(out, fh, indent=1, sort_keys=True)
    lines = COUNTER_COMMANDS + [
        "per region and kernel, medians over its full-size dispatches (bytes scaled by the calibration "
        "copy: fetch x%.4f, write x%.4f); mfma_us = SQ_VALU_MFMA_BUSY_CYCLES / %d SIMDs / %.0f MHz"
        % (sf, sw, SIMDS, CLOCK_MHZ), ""]
    for nm in names:
        if nm == "calibration" or nm not in out:
            continue
        lines.append(nm)
        for k, c in sorted(out[nm].items()):
            if k.startswith("fill_zero"):
                continue
            f = lambda key, sc=1.0, fmt="%.1f": (fmt % (c[key] * sc)) if key in c else "-"  # noqa: E731
            lines.append("  %-72s fetch %8s MB write %7s MB l2hit %6s mfma_us %7s wait_any %10s mfma_insts %10s"
                         % (k[:72], f("fetch_bytes", 1e-6), f("write_bytes", 1e-6), f("l2_hit_rate", 1.0, "%.3f"),
                            f("mfma_busy_us_per_simd", 1.0, "%.2f"), f("SQ_WAIT_INST_ANY", 1.0, "%.0f"),
                            f("SQ_INSTS_MFMA", 1.0, "%.0f")))
    with open(os.path.join(ROOT, "profiles", "counters_summary.txt"), "w") as fh:
        fh.write("\n".join(lines) + "\n")
    print("wrote %s and counters_summary.txt: %d regions" % (path, len(out) - 1))


def trace_summary(trace_csv, bench_json, cmd):
    """The profiles/ summary of a `rocprofv3 --kernel-trace --stats` run of
    this file (its kernel_trace CSV; kernel_stats beside it) and the JSON
    line that run printed: the step's four GEMMs in the timed regions (the
    last 2*steps consecutive steps of them in the trace) against the bench's
    own times, the decode and MoE kernels, the top kernels by total time."""
    import csv
    import statistics
    b = json.loads([ln for ln in open(bench_json) if ln.startswith("{")][-1])
    rows = sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Start_Timestamp"]))
    # A split-K GEMM (name "..._ks<s>") is two dispatches, the parts and
    # their reduce: one launch from the first's start to the second's end.
    merged = []
    for r in rows:
        if r["Kernel_Name"].startswith("gemm_splitk_") and merged and "_ks" in merged[-1]["Kernel_Name"]:
            merged[-1] = dict(merged[-1], End_Timestamp=r["End_Timestamp"])
        else:
            merged.append(r)
    rows = merged

    def dur(r):
        return (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3

    gem = ("qkv", "o", "gate_up", "down")
    names = [b["config"]["gemms"][g]["kernel"] for g in gem]
    seq = [r["Kernel_Name"] for r in rows]
    best, bi, i = 0, 0, 0
    while i < len(seq):
        j = i
        while j + 3 < len(seq) and seq[j:j + 4] == names:
            j += 4
        if (j - i) // 4 > best:
            best, bi = (j - i) // 4, i
        i = j + 1 if j == i else j
    steps = b["steps"]
    last = rows[bi + 4 * (best - steps):bi + 4 * best]  # the per-launch event region
    first = rows[bi + 4 * (best - 2 * steps):bi + 4 * (best - steps)]  # the step-time region

    def span(rr):
        return (int(rr[-1]["End_Timestamp"]) - int(rr[0]["Start_Timestamp"])) / 1e3 / steps

    def avg_of(nm, n=40):
        d = [dur(r) for r in rows if r["Kernel_Name"] == nm]
        return len(d), statistics.mean(d[-n:]) if d else float("nan")

    out = ["command: cd /tmp && TMPDIR=/tmp " + cmd,
           "summary: python3 bench.py --trace-summary <the run's kernel_trace.csv> <its stdout> '<command>'",
           "bench line (same run): value %.1f TFLOP/s, ms_per_step %.4f, roofline.frac %.4f (%s)" % (
               b["value"], b["ms_per_step"], b["roofline"]["frac"], b["roofline"]["gemm"]), "",
           "main step (configs[1], M=2048): %d consecutive steps of the 4 GEMMs found in the trace" % best,
           "  step-time region (%d steps, events at the ends only): rocprof first-start..last-end %.1f "
           "us/step, bench %.1f us/step" % (steps, span(first), b["ms_per_step"] * 1e3)]
    for g, nm in zip(gem, names):
        d1 = [dur(r) for r in first if r["Kernel_Name"] == nm]
        d2 = [dur(r) for r in last if r["Kernel_Name"] == nm]
        out.append("  %-8s %-66s rocprof avg %7.2f us (step region) %7.2f us (event region) | bench event "
                   "avg %7.2f us" % (g, nm, statistics.mean(d1), statistics.mean(d2), b["config"]["gemms"][g]["us"]))
    pm = b.get("prefill_more")
    if pm:
        out += ["", "other prefill cases (bench per-launch event times; rocprof averages over the set's timed "
                    "region, a split-K GEMM with its reduce):"]
        # Each set's timed region lies between two marker fills (grid of
        # MARK_BYTES / 16 threads), the sets in the bench's order.
        marks = [i for i, r in enumerate(rows) if r["Kernel_Name"] == "fill_zero"
                 and int(r.get("Grid_Size_X", r.get("Grid_Size", 0))) == MARK_BYTES // 16]
        regions = [rows[marks[2 * i] + 1:marks[2 * i + 1]] for i in range(len(marks) // 2)]
        names_r = b.get("regions") or list(pm)
        for case, st in pm.items():
            ci = names_r.index(case) if case in names_r else -1
            reg = regions[ci] if 0 <= ci < len(regions) else []
            out.append("  %s: %.1f TFLOP/s (%.1f%% of 2.5 PFLOP/s), %.2f us a set; rocprof first-start..last-end "
                       "%.2f us a set" % (case, st["tflops"], 100 * st["frac"], st["us"],
                                          (int(reg[-1]["End_Timestamp"]) - int(reg[0]["Start_Timestamp"])) / 1e3
                                          / (len(reg) / len(st["gemms"])) if reg else float("nan")))
            for g, d in st["gemms"].items():
                dd = [dur(r) for r in reg if r["Kernel_Name"] == d["kernel"]]
                out.append("    %-8s %-70s bench %7.2f us | rocprof avg %7.2f us (%d in the timed region)" % (
                    g, d["kernel"], d["us"], statistics.mean(dd) if dd else float("nan"), len(dd)))
    mv = b.get("matvec")
    if mv:
        out += ["", "decode (M=1) kernels, rocprof average of their last 40 dispatches:"]
        for g, nm in mv["kernels"].items():
            n, a = avg_of(nm)
            out.append("  %-8s %-52s calls %5d  avg %7.2f us" % (g, nm, n, a))
        for mk in ("m4", "m8"):
            if mk in mv:
                out += ["decode (M=%s) kernels, the same averages; step %.1f GB/s (%.1f%% of HBM):" % (
                    mk[1:], mv[mk]["value"], 100 * mv[mk]["frac"])]
                for g, nm in mv[mk]["kernels"].items():
                    n, a = avg_of(nm)
                    out.append("  %-8s %-52s calls %5d  avg %7.2f us" % (g, nm, n, a))
    moe = b.get("moe")
    if moe:
        out += ["", "MoE layer (config 5): bench per-op times, and the grouped GEMMs' rocprof averages:"]
        out.append("  " + ", ".join("%s %.2f us" % kv for kv in moe["ops_us"].items()))
        for g in ("gate_up", "down"):
            n, a = avg_of(moe[g]["kernel"])
            out.append("  %-8s %-80s calls %5d  avg %7.2f us" % (g, moe[g]["kernel"], n, a))
    stats = list(csv.DictReader(open(trace_csv.replace("kernel_trace", "kernel_stats"))))
    out += ["", "top kernels by total time (the load-time selection's candidates included):"]
    for r in stats[:15]:
        out.append("  %-70s calls %6s avg %9.2f us %5.1f%%" % (r["Name"][:70], r["Calls"],
                                                             float(r["AverageNs"]) / 1e3, float(r["Percentage"])))
    print("\n".join(out))


def traffic_summary(fetch_csv, write_csv):
    """profiles/traffic.json: per kernel (its dispatches over the most
    workgroups, i.e. the full M=2048 block), the median FETCH_SIZE and
    WRITE_SIZE scaled by the calibration copy, in bytes per launch."""
    import csv
    import statistics

    def per_kernel(path, counter):
        rows = {}
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] != counter:
                continue
            rows.setdefault(r["Kernel_Name"], []).append((int(r["Grid_Size"]), float(r["Counter_Value"])))
        out = {}
        for name, v in rows.items():
            top = max(gs for gs, _ in v)
            out[name] = (statistics.median(c for gs, c in v if gs == top), len(v))
        return out

    f, w = per_kernel(fetch_csv, "FETCH_SIZE"), per_kernel(write_csv, "WRITE_SIZE")
    copies = [n for n in f if "copyBuffer" in n]
    if not copies:
        sys.exit("traffic summary: no copyBuffer dispatch in %s" % fetch_csv)
    cf, cw = f[copies[0]][0], w[copies[0]][0]
    kib = COPY_BYTES / 1024.0
    sf, sw = kib / cf, kib / cw
    out = {"_calibration": {"copy_bytes": COPY_BYTES, "copy_kernel": copies[0],
                            "fetch_kib": cf, "write_kib": cw, "fetch_scale": round(sf, 4),
                            "write_scale": round(sw, 4)}}
    for name in sorted(f):
        if not name.startswith("gemm_") or name not in w:
            continue
        out[name] = {"bytes": round((f[name][0] * sf + w[name][0] * sw) * 1024.0),
                     "fetch_bytes": round(f[name][0] * sf * 1024.0),
                     "write_bytes": round(w[name][0] * sw * 1024.0)}
    path = os.path.join(ROOT, "profiles", "traffic.json")
    with open(path, "w") as fh:
        json.dump(out, fh, indent=1, sort_keys=True)
    print("wrote %s: %d kernels, fetch scale %.4f, write scale %.4f" % (path, len(out) - 1, sf, sw))


def bench_moe(g, e, hb):
    """one MoE layer's routed experts over T=2048 tokens,
    256 experts, top 8 (16384 pairs), hidden 2048, expert intermediate 512,
    on the kernels expert_pipes picked: route -> sort -> [gather] -> grouped
    gate|up -> SwiGLU -> grouped down -> combine.  The grouped GEMMs are
    HBM-bound (1.07 GB + 0.54 GB of expert weights); their algorithmic bytes
    are 2*(experts with rows)*N*K + 2*P*K + 2*P*N, flops 2*P*N*K."""
    T, E, TOPK, H, MI = 2048, 256, 8, 2048, 512
    seed = 0x5EED0005
    wgu = g.alloc_with(hb.normal_bf16(seed + 1, 0.02, (E * 2 * MI, H)))
    wdn = g.alloc_with(hb.normal_bf16(seed + 2, 0.02, (E * H, MI)))
    layer = hb.MoeLayer(g, e, E, TOPK, H, MI, T, wgu, wdn, scores=hb.normal_bf16(seed, 1.0, (T, E)),
                        x=hb.normal_bf16(seed + 3, 1.0, (T, H)))
    ops = layer.ops()
    g.time_ops(ops, 3)
    heat(g, ops)
    reps = 20
    with region(g, "moe_layer"):
        t, each = g.time_each(ops, reps)
    route = g.download(layer.buf["route"], np.uint32, T * 2 * TOPK).reshape(T, 2 * TOPK)
    used = len(np.unique(route[:, :TOPK]))
    P = T * TOPK
    names = ["route", "sort"] + (["gather"] if layer.kernels[3] >= 0 else []) + \
        ["gate_up"] + ([] if layer.fused else ["swiglu"]) + ["down", "combine"]
    per = dict(zip(names, each))
    # gate_up writes EGU (2*MI per pair), or EHB (MI per pair) with the SwiGLU fused.
    gu_b = 2.0 * used * 2 * MI * H + 2.0 * P * H + 2.0 * P * (MI if layer.fused else 2 * MI)
    dn_b = 2.0 * used * H * MI + 2.0 * P * MI + 2.0 * P * H
    gu_f, dn_f = 2.0 * P * 2 * MI * H, 2.0 * P * H * MI
    out = {"unit": "GB/s", "peak": HBM_PEAK, "layer_us": round(t / reps * 1e6, 2),
           "experts_with_rows": used, "rows_per_tile": layer.bm,
           "gate_up": {"us": round(per["gate_up"] * 1e6, 2), "gbs": round(gu_b / per["gate_up"] / 1e9, 1),
                       "frac": round(gu_b / per["gate_up"] / 1e9 / HBM_PEAK, 4),
                       "tflops": round(gu_f / per["gate_up"] / 1e12, 1),
                       "kernel": g.kernel_name(layer.kernels[1]), "swiglu_fused": layer.fused},
           "down": {"us": round(per["down"] * 1e6, 2), "gbs": round(dn_b / per["down"] / 1e9, 1),
                    "frac": round(dn_b / per["down"] / 1e9 / HBM_PEAK, 4),
                    "tflops": round(dn_f / per["down"] / 1e12, 1),
                    "kernel": g.kernel_name(layer.kernels[2])},
           "ops_us": {nm: round(v * 1e6, 2) for nm, v in per.items()}}
    out["value"] = round((gu_b + dn_b) / (per["gate_up"] + per["down"]) / 1e9, 1)
    out["frac"] = round(out["value"] / HBM_PEAK, 4)
    layer.free()
    # The tile rows the config names (16, 32, 64; moe.tile, qwen.rs:161-164
    # publishes the reference's layer rate per tile size): the layer on
    # each, the rest of its selection timed as above.
    out["tiles"] = {}
    if COUNTER_RUN:  # the counter passes cover the layer above, on pinned picks
        g.free(wgu)
        g.free(wdn)
        return out
    for bm in (16, 32, 64):
        with hb.Engine(g, "moe.tile=%d" % bm) as et:
            lt = hb.MoeLayer(g, et, E, TOPK, H, MI, T, wgu, wdn, scores=hb.normal_bf16(seed, 1.0, (T, E)),
                             x=hb.normal_bf16(seed + 3, 1.0, (T, H)))
        lops = lt.ops()
        g.time_ops(lops, 3)
        heat(g, lops, HEAT_S / 2)
        tt, ee = g.time_each(lops, reps)
        nm_t = ["route", "sort"] + (["gather"] if lt.kernels[3] >= 0 else []) + \
            ["gate_up"] + ([] if lt.fused else ["swiglu"]) + ["down", "combine"]
        pt = dict(zip(nm_t, ee))
        out["tiles"][str(bm)] = {"layer_us": round(tt / reps * 1e6, 2), "gate_up_us": round(pt["gate_up"] * 1e6, 2),
                                 "down_us": round(pt["down"] * 1e6, 2),
                                 "gate_up_kernel": g.kernel_name(lt.kernels[1]),
                                 "down_kernel": g.kernel_name(lt.kernels[2])}
        lt.free()
    # The whole sparse MLP (qwen.rs:2691-2732): post norm, shared expert
    # (inter 512), router GEMM, the routed experts above, moe_out.
    SI = 512
    w = {"post_norm": g.alloc_with(hb.normal_bf16(seed + 4, 0.1, (H,))),
         "router": g.alloc_with(hb.normal_bf16(seed + 5, 0.02, (E, H))),
         "w_gate_up": wgu, "w_down": wdn,
         "s_gate_up": g.alloc_with(hb.normal_bf16(seed + 6, 0.02, (2 * SI, H))),
         "s_down": g.alloc_with(hb.normal_bf16(seed + 7, 0.02, (H, SI))),
         "shared_gate": g.alloc_with(hb.normal_bf16(seed + 8, 0.05, (H,)))}
    blk = hb.MoeBlock(g, e, E, TOPK, H, MI, SI, T, w, hb.normal_bf16(seed + 9, 1.0, (T, H)))
    bops = blk.ops()
    g.time_ops(bops, 3)
    heat(g, bops, HEAT_S / 2)
    tb = g.time_ops(bops, reps) / reps
    wbytes = 2.0 * used * 3 * MI * H + 2.0 * (E * H + 3 * SI * H + 2 * H)
    out["block"] = {"us": round(tb * 1e6, 2), "weight_gbs": round(wbytes / tb / 1e9, 1),
                    "ops": len(bops), "note": "post norm, shared expert, router, routed experts, moe_out"}
    blk.free()
    for nm in ("post_norm", "router", "s_gate_up", "s_down", "shared_gate"):
        g.free(w[nm])
    g.free(wgu)
    g.free(wdn)
    return out


def decode_fused(g, e, hb, ws):
    """The same M=1 decode step with the reference's decode fusions
    (kernels.rs:236-290; qwen.rs:1311-1336): qkv reads the RMSNorm of the
    residual stream (XSrc::Norm), gate|up too and writes the SwiGLU
    (Out::Swiglu: nf outputs instead of 2*nf), down reads that, lm_head
    reads the final norm: the norms and the SwiGLU cost no launch.  Bytes
    as the plain step's, plus the norm weights, with gate|up's output nf
    wide."""
    eps = 1e-6
    shape = {nm: (k, n, o) for nm, k, n, o in LAYER + [LM_HEAD]}
    K = LAYER[0][1]
    resid = g.alloc_with(hb.normal_bf16(0x5EED0021, 1.0, (1, K)))
    nw = g.alloc_with(hb.normal_bf16(0x5EED0022, 0.1, (K,)))
    attn = g.alloc_with(hb.normal_bf16(0x5EED0023, 1.0, (1, shape["o"][0])))
    nf = shape["gate_up"][1] // 2
    bufs = {"qkv": g.alloc(2 * shape["qkv"][1]), "o": g.alloc_with(hb.normal_bf16(7, 1.0, (1, K))),
            "h": g.alloc(2 * nf), "down": g.alloc_with(hb.normal_bf16(8, 1.0, (1, K))),
            "lm": g.alloc(2 * shape["lm_head"][1])}
    r = hb.r
    kq = e.mv_fused(K, shape["qkv"][1], hb.Out.Bf16, 1, [r(w) for w in ws["qkv"]], r(resid), r(bufs["qkv"]),
                    xsrc=hb.XSrc.Norm, eps=eps, plus_one=True, norm_w=r(nw))
    ko = e.mv(shape["o"][0], K, 2, 1, [r(w) for w in ws["o"]], r(attn), r(bufs["o"]))
    kg = e.mv_fused(K, shape["gate_up"][1], hb.Out.Swiglu, 1, [r(w) for w in ws["gate_up"]], r(resid),
                    r(bufs["h"]), xsrc=hb.XSrc.Norm, eps=eps, plus_one=True, norm_w=r(nw))
    kd = e.mv(nf, K, 2, 1, [r(w) for w in ws["down"]], r(bufs["h"]), r(bufs["down"]))
    kl = e.mv_fused(K, shape["lm_head"][1], hb.Out.Bf16, 1, [r(ws["lm_head"][0])], r(resid), r(bufs["lm"]),
                    xsrc=hb.XSrc.Norm, eps=eps, plus_one=True, norm_w=r(nw))
    ops, nbytes = [], 0.0
    for L in range(DECODE_LAYERS):
        ops.append(hb.Op(kq, [r(ws["qkv"][L]), r(resid), r(bufs["qkv"]), r(nw)], 1))
        ops.append(hb.Op(ko, [r(ws["o"][L]), r(attn), r(bufs["o"])], 1))
        ops.append(hb.Op(kg, [r(ws["gate_up"][L]), r(resid), r(bufs["h"]), r(nw)], 1))
        ops.append(hb.Op(kd, [r(ws["down"][L]), r(bufs["h"]), r(bufs["down"])], 1))
    ops.append(hb.Op(kl, [r(ws["lm_head"][0]), r(resid), r(bufs["lm"]), r(nw)], 1))
    for nm, k, n, o in LAYER:
        nout = n // 2 if nm == "gate_up" else n
        per = 2.0 * n * k + 2.0 * k + 2.0 * nout * (2 if o == 2 else 1)
        if nm in ("qkv", "gate_up"):
            per += 2.0 * k  # the norm weights
        nbytes += DECODE_LAYERS * per
    k, n = LM_HEAD[1], LM_HEAD[2]
    nbytes += 2.0 * n * k + 4.0 * k + 2.0 * n
    g.time_ops(ops, 3)
    heat(g, ops)
    reps = 20
    t = g.time_ops(ops, reps) / reps
    for b in [resid, nw, attn] + list(bufs.values()):
        g.free(b)
    gbs = nbytes / t / 1e9
    return {"value": round(gbs, 1), "frac": round(gbs / HBM_PEAK, 4), "ms_per_step": round(t * 1e3, 4),
            "kernels": {"qkv": g.kernel_name(kq), "gate_up": g.kernel_name(kg), "lm_head": g.kernel_name(kl)}}


def bench_matvec(g, e, hb):
    """Decode steps: DECODE_LAYERS layers of the 4
    projections then the lm_head, in layer order, each weight read once from
    HBM per step, at M = 1 (the reported value), 4 and 8 rows; the same
    weights serve the three."""
    ws = {}
    for name, k, n, o in LAYER + [LM_HEAD]:
        layers = 1 if name == "lm_head" else DECODE_LAYERS
        ws[name] = [g.alloc_with(hb.normal_bf16(0x5EED0003 + 17 * i + n, 0.02, (n, k)))
                    for i in range(layers)]
    tmp = [b for v in ws.values() for b in v]
    res = {}
    for mv_m in (1, 4, 8):
        x_bufs, kern, ys = {}, {}, {}
        for name, k, n, o in LAYER + [LM_HEAD]:
            if k not in x_bufs:
                x_bufs[k] = g.alloc_with(hb.normal_bf16(0x5EED0003, 1.0, (mv_m, k)))
            ys[name] = g.alloc_with(hb.normal_bf16(5, 1.0, (mv_m, n)))
            kern[name] = e.mv(k, n, o, mv_m, [hb.r(w) for w in ws[name]], hb.r(x_bufs[k]), hb.r(ys[name]))
        ops, nbytes = [], 0.0
        seq = [(nm, L) for L in range(DECODE_LAYERS) for nm in ("qkv", "o", "gate_up", "down")]
        seq.append(("lm_head", 0))
        shape = {nm: (k, n, o) for nm, k, n, o in LAYER + [LM_HEAD]}
        for nm, L in seq:
            k, n, o = shape[nm]
            ops.append(hb.Op(kern[nm], [hb.r(ws[nm][L]), hb.r(x_bufs[k]), hb.r(ys[nm])], mv_m))
            nbytes += 2.0 * n * k + 2.0 * mv_m * k + 2.0 * mv_m * n * (2 if o == 2 else 1)
        g.time_ops(ops, 3)
        heat(g, ops)
        reps = 20
        with region(g, "decode_m%d" % mv_m):
            t = g.time_ops(ops, reps) / reps
        forms = {"stream": t}
        if GRAPH:
            # The same step recorded as one HIP graph (the reference encodes a
            # step's ops in one command buffer, qwen.rs:3177), timed the same
            # way (--graph; measured no faster than the stream, and the
            # profiler's kernel trace does not survive a graph launch).
            gr = g.graph(ops)
            try:
                gr.time(3)
                heat(g, ops)
                gr.time(50)
                forms["graph"] = gr.time(reps) / reps
            finally:
                gr.free()
        best = min(forms, key=forms.get)
        best_gbs = nbytes / forms[best] / 1e9
        r = {"value": round(best_gbs, 1), "unit": "GB/s", "frac": round(best_gbs / HBM_PEAK, 4), "peak": HBM_PEAK,
             "form": best,
             "ms_per_step": round(forms[best] * 1e3, 4), "m": mv_m, "layers": DECODE_LAYERS,
             "bytes_per_step": nbytes, "kernels": {nm: g.kernel_name(kern[nm]) for nm in kern}}
        if len(forms) > 1:
            for nm, tt in forms.items():
                r[nm] = {"ms_per_step": round(tt * 1e3, 4), "gbs": round(nbytes / tt / 1e9, 1),
                         "frac": round(nbytes / tt / 1e9 / HBM_PEAK, 4)}
        if mv_m == 1:
            # the lm_head alone, two copies in turn (2 x 778 MB: no copy is
            # still in the 256 MB last-level cache when it is read again)
            k, n = LM_HEAD[1], LM_HEAD[2]
            w2 = g.alloc_with(hb.normal_bf16(0x5EED0099, 0.02, (n, k)))
            tmp.append(w2)
            head2 = hb.Op(ops[-1].kernel, [hb.r(w2), ops[-1].bind[1], ops[-1].bind[2]], mv_m)
            heat(g, [ops[-1], head2], HEAT_S / 4)
            th = g.time_ops([ops[-1], head2], reps) / reps / 2
            hb_bytes = 2.0 * k * n + 2.0 * mv_m * k + 2.0 * mv_m * n
            r["lm_head"] = {"gbs": round(hb_bytes / th / 1e9, 1), "us": round(th * 1e6, 2),
                            "frac": round(hb_bytes / th / 1e9 / HBM_PEAK, 4)}
        res[mv_m] = r
        for b in list(x_bufs.values()) + list(ys.values()):
            g.free(b)
    res["fused"] = decode_fused(g, e, hb, ws)
    for b in tmp:
        g.free(b)
    out = res[1]
    out["fused"] = res["fused"]
    keys = ("value", "frac", "form", "stream", "graph", "ms_per_step", "kernels")
    out["m4"] = {kk: res[4][kk] for kk in keys if kk in res[4]}
    out["m8"] = {kk: res[8][kk] for kk in keys if kk in res[8]}
    return out


if __name__ == "__main__":
    main()
