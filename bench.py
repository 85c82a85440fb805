"""Benchmark: Q4_K GEMV HBM GB/s (% of peak) + ms/layer at Llama-3.3-70B shapes, batch 1.

One step = one decoder layer's seven GEMVs of a Llama-3.3-70B Q4_K_M model at batch 1 (hidden
8192, FFN 28672, 64 query / 8 KV heads of 128): q, k (Q4_K) and v (Q6_K) in one fused launch,
o (Q4_K), gate+up (Q4_K) in one launch with the SiLU epilogue, down (Q6_K). Synthetic seeded
blocks (fp16 d, dmin = |N(0,1)|*0.01; uniform 6-bit scales and 4/6-bit quants), random x. The
weights of 4 distinct layer copies rotate (2.2 GB) so the 256 MB Infinity Cache cannot serve a
repeat; activations stay in HBM for the whole timed region.

Prints one JSON line. value = algorithmic bytes of the layer (weights + 4*T*(cols+rows) per
GEMV) / measured time per layer, in GB/s.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

PEAK_HBM_GBS = 8000.0
METRIC = "Q4_K GEMV HBM GB/s (% of peak) + ms/layer at 70B shapes, batch 1"

HIDDEN, FFN, HEADS, KV_HEADS, HEAD_DIM, LAYERS = 8192, 28672, 64, 8, 128, 80
Q4_K, Q6_K = 12, 14
# name, type, rows, cols
LAYER = [("q", Q4_K, HEADS * HEAD_DIM, HIDDEN), ("k", Q4_K, KV_HEADS * HEAD_DIM, HIDDEN),
         ("v", Q6_K, KV_HEADS * HEAD_DIM, HIDDEN), ("o", Q4_K, HIDDEN, HEADS * HEAD_DIM),
         ("gate", Q4_K, FFN, HIDDEN), ("up", Q4_K, FFN, HIDDEN), ("down", Q6_K, HIDDEN, FFN)]


def row_bytes(t, cols):
    return cols // 256 * (144 if t == Q4_K else 210)


def algo_bytes(mats, T):
    return sum(r * row_bytes(t, c) + 4 * T * (c + r) for _, t, r, c in mats)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--prewarm", type=float, default=0.3,
                    help="seconds of untimed layer steps before the --warmup steps (the clocks' settling)")
    ap.add_argument("--batch", type=int, default=1,
                    help="tokens per step (1..8); with --decode, sequences decoding together (any N)")
    ap.add_argument("--copies", type=int, default=4, help="distinct layer copies to rotate")
    ap.add_argument("--cpu-seconds", type=float, default=6.0, help="CPU-baseline time budget")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--int-dot", action="store_true",
                    help="the integer-dot kernels (Transformer.IntDot, --int-dot): 8-bit activations, "
                         "FastMath.IntDot per row; no CPU baseline")
    ap.add_argument("--graph", action="store_true",
                    help="replay the layer's four calls as a recorded graph (one host call per step) instead "
                         "of enqueueing them one by one")
    ap.add_argument("--float-mma", action="store_true",
                    help="the float products on the matrix cores (wl_set_float_mma: fp16 MFMA on an "
                         "exact two-part split of x, as an engine started with --batch N runs them)")
    ap.add_argument("--formats", action="store_true",
                    help="instead of the layer: the decode GEMV of every GGUF format at the 70B FFN "
                         "shapes (28672x8192 and 8192x28672), one token and eight, one JSON line")
    ap.add_argument("--only", default="", help="with --formats: comma-separated format names")
    ap.add_argument("--stream", action="store_true",
                    help="instead of the resident layer: the layer streamed from pinned host memory "
                         "through two HBM stage slots (copy of layer N+1 beside the compute of N)")
    ap.add_argument("--decode", action="store_true",
                    help="instead of the layer: whole-token greedy decode of the 70B model with every "
                         "layer, the embedding, the head and the KV cache resident in HBM")
    ap.add_argument("--layers", type=int, default=LAYERS, help="with --decode: decoder layers")
    ap.add_argument("--prompt", type=int, default=128, help="with --decode: prompt tokens before decoding")
    ap.add_argument("--tokens", type=int, default=64, help="with --decode: timed greedy tokens")
    ap.add_argument("--no-workloads", action="store_true",
                    help="skip the other workloads (Q8_0 4096^2, 8B layer, 70B layer at 8 tokens, prefill GEMMs, "
                         "I-quant GEMVs, qwen3moe experts) and the copy peak")
    ap.add_argument("--only-workloads", default="",
                    help="comma-separated workload keys to run (default: all)")
    ap.add_argument("--calibrate", type=int, default=0, metavar="MIB",
                    help="before warm-up, run a plain elementwise copy (torch.neg) of MIB MiB three "
                         "times, untimed: the HBM counters of a kernel of known traffic")
    return ap.parse_args()


class Layer:
    def __init__(self, ctx, host):
        self.w = {n: ctx.upload(t, host[n], r, c, name=n) for n, t, r, c in LAYER}

    def free(self):
        for w in self.w.values():
            w.free()


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build runs the hot path on a single MI355X "
              "(--gpus %d requested)" % args.gpus, file=sys.stderr)
        sys.exit(2)
    if args.formats:
        return run_formats(args)
    if args.stream:
        return run_stream(args)
    if args.decode:
        return run_decode_batch(args) if args.batch > 1 else run_decode(args)
    T = args.batch
    if not 1 <= T <= 8:
        sys.exit("--batch must be 1..8")

    import torch
    import windlass_amd
    from windlass_amd import synth
    from windlass_amd._lib import check
    from windlass_amd.backend import Context

    L = windlass_amd.load()
    rng = np.random.default_rng(0x57494E44 + 3000)
    host = {n: synth.blocks(t, r, c, rng) for n, t, r, c in LAYER}
    ctx = Context(0)
    ctx.IntDot = args.int_dot
    ctx.FloatMma = args.float_mma
    layers = [Layer(ctx, host) for _ in range(args.copies)]
    dev = torch.device("cuda:0")
    x = torch.from_numpy(synth.activations(rng, T, HIDDEN)).to(dev)
    yq = torch.empty((T, HEADS * HEAD_DIM), device=dev)
    yk = torch.empty((T, KV_HEADS * HEAD_DIM), device=dev)
    yv = torch.empty((T, KV_HEADS * HEAD_DIM), device=dev)
    yo = torch.empty((T, HIDDEN), device=dev)
    h = torch.empty((T, FFN), device=dev)
    out = torch.empty((T, HIDDEN), device=dev)
    stream = torch.cuda.ExternalStream(ctx.stream, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    # every call's arguments built once, outside the timed loop: the host only enqueues
    hc, px, pq, po, ph, pout = ctx.handle, P(x), P(yq), P(yo), P(h), P(out)
    ys = (ctypes.c_void_p * 3)(yq.data_ptr(), yk.data_ptr(), yv.data_ptr())
    for ly in layers:
        ly.qkv = (ctypes.c_void_p * 3)(ly.w["q"].handle.value, ly.w["k"].handle.value, ly.w["v"].handle.value)
    mm_multi, mm, gu = L.wl_matmul_multi_dev, L.wl_matmul_dev, L.wl_gate_up_dev

    def qkv(ly):
        check(mm_multi(hc, 3, ly.qkv, px, T, ys))

    def o_proj(ly):   # the attention output stands in as yq (attention is not on this path)
        check(mm(hc, ly.w["o"].handle, -1, pq, T, po))

    def gate_up(ly):
        check(gu(hc, ly.w["gate"].handle, ly.w["up"].handle, -1, po, T, ph))

    def down(ly):
        check(mm(hc, ly.w["down"].handle, -1, ph, T, pout))

    def step(i):
        ly = layers[i % len(layers)]
        qkv(ly); o_proj(ly); gate_up(ly); down(ly)

    if args.calibrate > 0:
        src = torch.ones(args.calibrate << 18, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst

    # the other workloads first (GPU parts only; their CPU baselines run after the timed region)
    work, work_cpu = {}, []
    if not args.no_workloads and not args.int_dot and not args.float_mma and T == 1:
        only = [k for k in args.only_workloads.split(",") if k]
        work, work_cpu = run_workloads(ctx, L, stream, layers, host, only)

    # Untimed steady-state warm-up: after the workloads (and their host-side set-up, when the GPU
    # idles) the clocks need about a quarter second of sustained load to settle. Measured with 5
    # warmup and 20 timed steps: 132.5-134.9 us per layer right after the workloads, 120.0 us after
    # 0.25 s of these steps, the same as over 500 timed steps. The --warmup steps and exactly
    # --steps timed steps follow as before.
    t_pre, n_pre = time.time(), 0
    while time.time() - t_pre < args.prewarm:
        for _ in range(100):
            step(n_pre)
            n_pre += 1
        ctx.sync()
    # warmup, then exactly K timed steps between events on the launch stream. A step enqueues the
    # four calls; with --graph it is one replay of them recorded once per layer copy
    # (wl_capture_begin/_end: the same kernels on the same buffers, one host call per step).
    for i in range(args.warmup):
        step(i)
    ctx.sync()
    graphs = [] if not args.graph else [ctx.capture(lambda ly=ly: (qkv(ly), o_proj(ly), gate_up(ly), down(ly)))
                                    for ly in layers]
    run_step = (lambda i: graphs[i % len(graphs)].launch()) if graphs else step
    for i in range(args.warmup):
        run_step(i)
    ctx.sync()
    torch.cuda.synchronize()

    def timed(fn, n):
        with torch.cuda.stream(stream):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for i in range(n):
                fn(i)
            e1.record(stream)
        e1.synchronize()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    ms_layer = timed(run_step, args.steps)
    ms_eager = timed(step, args.steps) if graphs else ms_layer
    for g in graphs:
        g.free()
    layer_bytes = algo_bytes(LAYER, T)
    gbs = layer_bytes / (ms_layer * 1e-3) / 1e9

    # per-launch durations (HIP events on the launch stream around 200 back-to-back calls of one
    # launch, rotating the copies). Events between the calls of a step would add 4-7 us to each
    # bracketed launch. Alone, the gate/up pair (264 MB per copy) streams from HBM as in a step;
    # the four copies of q/k/v (198 MB) and o (151 MB) fit in the 256 MB Infinity Cache, so their
    # figures here are optimistic, and the step time above is what the layer takes.
    def time_launch(fn, reps=200):
        with torch.cuda.stream(stream):
            for i in range(10):
                fn(layers[i % len(layers)])
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for i in range(reps):
                fn(layers[i % len(layers)])
            b.record(stream)
        b.synchronize()
        return a.elapsed_time(b) / reps

    per = {"qkv": time_launch(qkv), "o": time_launch(o_proj), "gate_up": time_launch(gate_up),
           "down": time_launch(down)}
    launch_bytes = {"qkv": algo_bytes(LAYER[0:3], T), "o": algo_bytes(LAYER[3:4], T),
                    "gate_up": algo_bytes(LAYER[4:6], T), "down": algo_bytes(LAYER[6:7], T)}
    dom = max(per, key=per.get)
    ach = launch_bytes[dom] / (per[dom] * 1e-3) / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        kind = "_int" if args.int_dot else "_fmma" if args.float_mma else ""
        traffic = json.load(open(tpath)).get("%s_T%d%s" % (dom, T, kind))

    for ly in layers:
        ly.free()
    ctx.close()

    cpu = None
    if not args.no_cpu and not args.int_dot:
        cpu = cpu_baseline(host, T, rng, args.cpu_seconds)
        for key, fn in work_cpu:
            work[key]["cpu_baseline"] = fn()

    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "prewarm_steps": n_pre,
        "ms_per_step": round(ms_layer, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 x q-blocks -> int32, f32 terms" if args.int_dot else "f32",
        "data": "synthetic seeded GGUF blocks (Q4_K/Q6_K), x ~ N(0,1)",
        "config": {"workload": "Llama-3.3-70B Q4_K_M decoder layer, 7 GEMVs (q,k,o,gate,up Q4_K; v,down Q6_K)",
                   "hidden": HIDDEN, "ffn": FFN, "heads": HEADS, "kv_heads": KV_HEADS, "head_dim": HEAD_DIM,
                   "batch": T, "layer_copies": args.copies, "matrix_calls_per_layer": 4,
                   "kernels": "int-dot (8-bit activations)" if args.int_dot else
                   "fp32 decode GEMV on fp16 MFMA (x in two exact fp16 parts)" if args.float_mma else
                   "fp32 decode GEMV"},
        "pct_of_peak_hbm": round(100 * gbs / PEAK_HBM_GBS, 2),
        "ms_per_layer": round(ms_layer, 5),
        "step_enqueue": "eager calls" if not graphs else "one graph replay per step (the four calls recorded once "
                                                         "per layer copy)",
        "tokens_per_s_80_layers": round(1000.0 * T / (LAYERS * ms_layer), 2),
        "layer_algorithmic_bytes": layer_bytes,
        "per_launch_ms": {k: round(v, 5) for k, v in per.items()},
        "per_launch_note": "each launch timed alone over the 4 rotating copies: q/k/v and o then partly hit the "
                           "256 MB Infinity Cache; ms_per_step is the layer",
        "per_launch_gbs": {k: round(launch_bytes[k] / (per[k] * 1e-3) / 1e9, 1) for k in per},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": traffic,
                     "traffic_source": "profiles/traffic.json: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of "
                                       "this launch, scaled by a 1 GiB copy's counters (not measured in this run)"},
        "cpu_baseline": cpu,
    }
    if graphs:
        line["ms_per_layer_eager_calls"] = round(ms_eager, 5)
    if "copy_peak" in work:
        line["roofline"]["measured_peak"] = work.pop("copy_peak")
        line["roofline"]["frac_of_measured_read_peak"] = round(ach / line["roofline"]["measured_peak"]["read_gbs"], 4)
    if work:
        line["workloads"] = work
    print(json.dumps(line), flush=True)


PEAK_BF16_TFLOPS = 2500.0
WORKING_SET = 1 << 30  # bytes of distinct weights a GEMV workload rotates through (> the 256 MB Infinity Cache)
LLAMA8B = [("q", Q4_K, 4096, 4096), ("k", Q4_K, 1024, 4096), ("v", Q4_K, 1024, 4096), ("o", Q4_K, 4096, 4096),
           ("gate", Q4_K, 14336, 4096), ("up", Q4_K, 14336, 4096), ("down", Q4_K, 4096, 14336)]
Q8_0, IQ2_XXS, IQ4_XS = 8, 16, 23
WBYTES = {Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), IQ2_XXS: (256, 66), IQ4_XS: (256, 136)}


def mat_bytes(t, r, c):
    be, bb = WBYTES[t]
    return r * (c // be) * bb


def gemv_bytes(mats, T):
    return sum(mat_bytes(t, r, c) + 4 * T * (c + r) for _, t, r, c in mats)


def time_events(stream, fn, reps, warm=5, settle=0.2):
    """Average ms per fn(i) call, HIP events on the library's stream around reps calls, after
    `settle` seconds of untimed calls (the clocks settle under sustained load; a workload's
    host-side set-up leaves the GPU idle before it) and `warm` more."""
    import torch
    with torch.cuda.stream(stream):
        t0, n = time.time(), 0
        while time.time() - t0 < settle:
            for _ in range(20):
                fn(n)
                n += 1
            stream.synchronize()
        for i in range(warm):
            fn(i)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(reps):
            fn(i)
        b.record(stream)
    b.synchronize()
    return a.elapsed_time(b) / reps


def best_of(fn, budget_s, min_reps=3, max_reps=50):
    best, reps, t_start = float("inf"), 0, time.perf_counter()
    while reps < min_reps or (time.perf_counter() - t_start < budget_s and reps < max_reps):
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
        reps += 1
    return best, reps


def cpu_threads():
    return int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count()


def cpu_info():
    """The host the CPU baselines run on: model, logical CPUs, SMT state."""
    model = "unknown"
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    smt = None
    try:
        smt = open("/sys/devices/system/cpu/smt/active").read().strip() == "1"
    except OSError:
        pass
    return {"cpu_model": model, "logical_cpus": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
            "smt_active": smt}


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    return oracle


def gemv_cpu(mats, host, T, budget_s, what):
    """The oracle's MatMul (DotRow per row, MatMulEach for T > 1; decode + Block for the
    I-quants) over every matrix of a workload, best of repeated passes."""
    oracle = _oracle()
    rng = np.random.default_rng(99)
    xs = {c: rng.standard_normal((T, c), dtype=np.float32) for _, _, _, c in mats}
    thr = cpu_threads()

    def one():
        for n, t, r, c in mats:
            oracle.matmul(t, host[n], r, c, xs[c], T, each_token=True, threads=thr)
    best, reps = best_of(one, budget_s)
    b = gemv_bytes(mats, T)
    return {"value": round(b / best / 1e9, 3), "unit": "GB/s", "cores": thr, "kind": "port",
            "ms": round(best * 1e3, 3),
            "sample": "%s, best of %d passes, C restatement of Transformer.MatMul (-O2 scalar), %d threads"
                      % (what, reps, thr)}


def intdot_cpu(mats, host, T, budget_s, what):
    """The oracle's integer branch of Transformer.MatMul (FastMath.Quantize per token, then
    FastMath.IntDot per row and token) over every matrix of a workload, best of repeated passes."""
    oracle = _oracle()
    rng = np.random.default_rng(98)
    xs = {c: rng.standard_normal((T, c), dtype=np.float32) for _, _, _, c in mats}
    thr = cpu_threads()

    def one():
        for n, t, r, c in mats:
            oracle.int_matmul(t, host[n], r, c, xs[c], threads=thr)
    best, reps = best_of(one, budget_s)
    b = gemv_bytes(mats, T)
    return {"value": round(b / best / 1e9, 3), "unit": "GB/s", "cores": thr, "kind": "port",
            "ms": round(best * 1e3, 3),
            "sample": "%s, best of %d passes, C restatement of Transformer.MatMul's integer branch "
                      "(FastMath.Quantize + IntDot, -O2 scalar), %d threads" % (what, reps, thr)}


def run_workloads(ctx, L, stream, layers, host70, only):
    """The other measured workloads (GPU legs), each with algorithmic bytes or flops, µs per
    launch set, achieved rate and fraction of peak. Returns the results and the CPU-baseline
    closures to run after the GPU work."""
    import torch
    from windlass_amd import synth
    from windlass_amd._lib import check
    dev = torch.device("cuda:0")
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    out, cpu = {}, []

    def want(k):
        return not only or k in only

    def copies_for(nbytes, cap=64):
        return max(2, min(cap, -(-WORKING_SET // max(nbytes, 1))))

    # device streaming read ceiling: wl_read_peak_dev (loads only) over 4 GiB at several grid
    # sizes, best taken; torch's copy beside it for reference
    if want("copy_peak"):
        n = 1 << 30
        a = torch.ones(n, device=dev)
        sink = torch.zeros(4, dtype=torch.int32, device=dev)
        reads = {}
        for wgs in (1024, 2048, 4096, 8192, 16384):
            ms = time_events(stream, lambda i, w=wgs: check(L.wl_read_peak_dev(ctx.handle, P(a), 4 * n, w, P(sink))),
                             10, warm=2)
            reads[wgs] = round(4 * n / (ms * 1e-3) / 1e9, 1)
        b = torch.empty_like(a)
        cur = torch.cuda.current_stream(dev)
        ms_copy = time_events(cur, lambda i: b.copy_(a), 10, warm=2)
        out["copy_peak"] = {"read_gbs": max(reads.values()), "read_gbs_by_workgroups": reads,
                            "torch_copy_gbs": round(8 * n / (ms_copy * 1e-3) / 1e9, 1),
                            "method": "wl_read_peak_dev: nontemporal 16-byte loads only over 4 GiB, each 256-thread "
                                      "workgroup over one contiguous chunk with eight loads in flight per thread, best "
                                      "of five grid sizes, HIP events over 10 launches each; torch copy_ counts read + "
                                      "write"}
        del a, b, sink
        torch.cuda.empty_cache()

    def layer_set(mats, seed):
        rng = np.random.default_rng(seed)
        host = {n: synth.blocks(t, r, c, rng) for n, t, r, c in mats}
        ncp = copies_for(gemv_bytes(mats, 1))
        ws = [{n: ctx.upload(t, host[n], r, c, name=n) for n, t, r, c in mats} for _ in range(ncp)]
        return host, ws

    def layer_fns(mats, ws, T):
        shape = {n: (r, c) for n, _, r, c in mats}
        x = torch.from_numpy(np.random.default_rng(T).standard_normal((T, shape["q"][1]), dtype=np.float32)).to(dev)
        ys = {n: torch.empty((T, shape[n][0]), device=dev) for n in shape}
        h = torch.empty((T, shape["gate"][0]), device=dev)

        def step(i):
            w = ws[i % len(ws)]
            arr_w = (ctypes.c_void_p * 3)(*[w[n].handle.value for n in "qkv"])
            arr_y = (ctypes.c_void_p * 3)(*[ys[n].data_ptr() for n in "qkv"])
            check(L.wl_matmul_multi_dev(ctx.handle, 3, arr_w, P(x), T, arr_y))
            check(L.wl_matmul_dev(ctx.handle, w["o"].handle, -1, P(ys["q"]), T, P(ys["o"])))
            check(L.wl_gate_up_dev(ctx.handle, w["gate"].handle, w["up"].handle, -1, P(ys["o"]), T, P(h)))
            check(L.wl_matmul_dev(ctx.handle, w["down"].handle, -1, P(h), T, P(ys["down"])))
        return step

    def gemv_entry(mats, T, ms, ncopies):
        b = gemv_bytes(mats, T)
        return {"us": round(ms * 1e3, 2), "algorithmic_bytes": b, "gbs": round(b / (ms * 1e-3) / 1e9, 1),
                "frac_hbm": round(b / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "batch": T, "copies_rotated": ncopies}

    if want("q8_0_4096x4096"):
        mats = [("w", Q8_0, 4096, 4096)]
        rng = np.random.default_rng(0x57494E44 + 1000)
        host = {"w": synth.blocks(Q8_0, 4096, 4096, rng)}
        ncp = copies_for(mat_bytes(Q8_0, 4096, 4096))
        ws = [ctx.upload(Q8_0, host["w"], 4096, 4096) for _ in range(ncp)]
        x = torch.from_numpy(synth.activations(rng, 1, 4096)).to(dev)
        y = torch.empty((1, 4096), device=dev)
        ms = time_events(stream, lambda i: check(L.wl_matmul_dev(ctx.handle, ws[i % ncp].handle, -1, P(x), 1, P(y))),
                         400)
        out["q8_0_4096x4096"] = dict(gemv_entry(mats, 1, ms, ncp), workload="Q8_0 GEMV 4096 x 4096, batch 1")
        for w in ws:
            w.free()
        cpu.append(("q8_0_4096x4096", lambda h=host, m=mats: gemv_cpu(m, h, 1, 1.5, "Q8_0 4096 x 4096 at batch 1")))

    if want("llama8b_q4k_layer"):
        host, ws = layer_set(LLAMA8B, 0x57494E44 + 2000)
        ms = time_events(stream, layer_fns(LLAMA8B, ws, 1), 200)
        out["llama8b_q4k_layer"] = dict(gemv_entry(LLAMA8B, 1, ms, len(ws)),
                                        workload="Llama-3-8B layer, Q4_K: q/o 4096x4096, k/v 1024x4096, gate/up "
                                                 "14336x4096, down 4096x14336, as 4 launches (q/k/v, o, gate+up, down)")
        for w in ws:
            for v in w.values():
                v.free()
        cpu.append(("llama8b_q4k_layer", lambda h=host: gemv_cpu(LLAMA8B, h, 1, 2.0, "8B layer (7 GEMVs) at batch 1")))

    if want("llama70b_q4km_layer_T8"):
        ws = [ly.w for ly in layers]
        ms = time_events(stream, layer_fns(LAYER, ws, 8), 100)
        e = gemv_entry(LAYER, 8, ms, len(ws))
        e["tokens_per_s_per_layer"] = round(8 / (ms * 1e-3), 1)
        out["llama70b_q4km_layer_T8"] = dict(e, workload="Llama-3.3-70B Q4_K_M layer, 8 tokens per launch "
                                                         "(MatMulEach: each token's bits equal its one-token result)")
        cpu.append(("llama70b_q4km_layer_T8", lambda: gemv_cpu(LAYER, host70, 8, 3.0, "70B layer (7 GEMVs) at 8 tokens")))

    if want("llama70b_q4km_layer_T8_intdot"):
        # Transformer.IntDot (--int-dot) at 8 tokens: activations quantized once per call, the
        # products on the int8 matrix cores, every result FastMath.IntDot's bits
        ws = [ly.w for ly in layers]
        ctx.IntDot = True
        try:
            ms = time_events(stream, layer_fns(LAYER, ws, 8), 100)
        finally:
            ctx.IntDot = False
        e = gemv_entry(LAYER, 8, ms, len(ws))
        e["tokens_per_s_per_layer"] = round(8 / (ms * 1e-3), 1)
        out["llama70b_q4km_layer_T8_intdot"] = dict(e, workload="Llama-3.3-70B Q4_K_M layer, 8 tokens, integer-dot "
                                                                "path (Q8_K activations, v_mfma_i32_16x16x32_i8)")
        cpu.append(("llama70b_q4km_layer_T8_intdot",
                    lambda: intdot_cpu(LAYER, host70, 8, 3.0, "70B layer (7 GEMVs) at 8 tokens, integer dot")))

    if want("llama70b_q4km_layer_T8_fmma"):
        # ForwardBatch's float products on the matrix cores (wl_set_float_mma): fp16 MFMA on the
        # exact two-part split of x, each token's bits independent of the batch
        ws = [ly.w for ly in layers]
        ctx.FloatMma = True
        try:
            ms = time_events(stream, layer_fns(LAYER, ws, 8), 100)
        finally:
            ctx.FloatMma = False
        e = gemv_entry(LAYER, 8, ms, len(ws))
        e["tokens_per_s_per_layer"] = round(8 / (ms * 1e-3), 1)
        out["llama70b_q4km_layer_T8_fmma"] = dict(e, workload="Llama-3.3-70B Q4_K_M layer, 8 tokens, float products "
                                                              "on the matrix cores (v_mfma_f32_16x16x32_f16, x split "
                                                              "into two fp16 parts)")
        cpu.append(("llama70b_q4km_layer_T8_fmma",
                    lambda: gemv_cpu(LAYER, host70, 8, 3.0, "70B layer (7 GEMVs) at 8 tokens")))

    for key, t, rows, cols in (("prefill_512_q4k_28672x8192", Q4_K, 28672, 8192),
                               ("prefill_512_q6k_8192x28672", Q6_K, 8192, 28672)):
        if not want(key):
            continue
        T = 512
        rng = np.random.default_rng(0x57494E44 + 4000 + rows)
        host = synth.blocks(t, rows, cols, rng)
        ws = [ctx.upload(t, host, rows, cols) for _ in range(2)]
        x = torch.from_numpy(synth.activations(rng, T, cols)).to(dev)
        y = torch.empty((T, rows), device=dev)
        ms = time_events(stream, lambda i: check(L.wl_matmul_dev(ctx.handle, ws[i % 2].handle, -1, P(x), T, P(y))),
                         20, warm=3)
        flops = 2 * T * rows * cols
        tf = flops / (ms * 1e-3) / 1e12
        out[key] = {"us": round(ms * 1e3, 1), "flops": flops, "tflops": round(tf, 1),
                    "frac_mfma_bf16": round(tf / PEAK_BF16_TFLOPS, 4), "tokens": T,
                    "workload": "prefill GEMM, %s W %dx%d times X [512 x %d] fp32 (bf16 MFMA, fp32 accumulate)"
                                % ("Q4_K" if t == Q4_K else "Q6_K", rows, cols, cols)}
        for w in ws:
            w.free()
        # the vendor library on the same product with dense bf16 operands already in HBM (no
        # decode, no fp32 x): W [rows x cols] @ X^T [cols x T], both contiguous
        wb = torch.randn(rows, cols, device=dev, dtype=torch.bfloat16)
        xt = x.t().contiguous().to(torch.bfloat16)
        ms_v = time_events(stream, lambda i: torch.matmul(wb, xt), 20, warm=3)
        out[key]["vendor_bf16_gemm"] = {
            "us": round(ms_v * 1e3, 1), "tflops": round(flops / (ms_v * 1e-3) / 1e12, 1),
            "what": "torch.matmul (hipBLASLt) of dense bf16 W [%d x %d] and X^T [%d x 512], same stream and "
                    "timing" % (rows, cols, cols)}
        del wb, xt

        def pre_cpu(t=t, rows=rows, cols=cols, host=host):
            oracle = _oracle()
            sub = rows // 8  # one rep over 1/8 of the rows, scaled to the whole matrix
            rb = mat_bytes(t, 1, cols)
            xs = np.random.default_rng(5).standard_normal((512, cols), dtype=np.float32)
            thr = cpu_threads()
            t0 = time.perf_counter()
            oracle.matmul(t, host[:sub * rb], sub, cols, xs, 512, threads=thr)
            s = time.perf_counter() - t0
            fl = 2 * 512 * sub * cols
            return {"value": round(fl / s / 1e9, 2), "unit": "GFLOP/s", "cores": thr, "kind": "port",
                    "s_whole_matrix_est": round(s * rows / sub, 2),
                    "sample": "%d of %d rows x 512 tokens, one rep: decode 32-row tiles + FastMath.Block "
                              "(C restatement, -O2 scalar), %d threads" % (sub, rows, thr)}
        cpu.append((key, pre_cpu))

    for key, t in (("iq4_xs_8192x28672", IQ4_XS), ("iq2_xxs_8192x28672", IQ2_XXS)):
        if not want(key):
            continue
        rows, cols = 8192, 28672
        rng = np.random.default_rng(0x57494E44 + 5000 + t)
        host = synth.blocks(t, rows, cols, rng)
        ncp = copies_for(mat_bytes(t, rows, cols))
        ws = [ctx.upload(t, host, rows, cols) for _ in range(ncp)]
        for T in (1, 8):
            x = torch.from_numpy(synth.activations(rng, T, cols)).to(dev)
            y = torch.empty((T, rows), device=dev)
            ms = time_events(stream, lambda i: check(L.wl_matmul_dev(ctx.handle, ws[i % ncp].handle, -1, P(x), T,
                                                                     P(y))), 200)
            out["%s_T%d" % (key, T)] = dict(gemv_entry([("w", t, rows, cols)], T, ms, ncp),
                                             workload="%s GEMV %dx%d, batch %d" % (
                                                 "IQ4_XS" if t == IQ4_XS else "IQ2_XXS", rows, cols, T))
        for w in ws:
            w.free()
        cpu.append(("%s_T1" % key, lambda h=host, t=t: gemv_cpu(
            [("w", t, 8192, 28672)], {"w": h}, 1, 1.5, "8192 x 28672 at batch 1 (decode + Block)")))
        cpu.append(("%s_T8" % key, lambda h=host, t=t: gemv_cpu(
            [("w", t, 8192, 28672)], {"w": h}, 8, 2.0, "8192 x 28672 at 8 tokens (decode + Block)")))

    if want("qwen3moe_experts"):
        ne, k, embd, ff = 128, 8, 2048, 768
        rng = np.random.default_rng(0x57494E44 + 6000)
        eb = mat_bytes(Q4_K, ff, embd)  # one expert's matrix
        ncp = copies_for(3 * ne * eb, cap=4)
        hosts = [[synth.blocks(Q4_K, ne * ff, embd, rng), synth.blocks(Q4_K, ne * ff, embd, rng),
                  synth.blocks(Q4_K, ne * embd, ff, rng)] for _ in range(ncp)]
        ws = [(ctx.upload(Q4_K, g, ff, embd, experts=ne), ctx.upload(Q4_K, u, ff, embd, experts=ne),
               ctx.upload(Q4_K, d, embd, ff, experts=ne)) for g, u, d in hosts]
        oracle = _oracle()
        for T in (1, 8):
            lg = [rng.standard_normal((T, ne), dtype=np.float32) for _ in range(ncp)]
            dlg = [torch.from_numpy(a).to(dev) for a in lg]
            x = torch.from_numpy(synth.activations(rng, T, embd)).to(dev)
            y = torch.empty((T, embd), device=dev)
            ms = time_events(stream, lambda i: check(L.wl_moe_ffn_dev(
                ctx.handle, P(dlg[i % ncp]), k, 1, ws[i % ncp][0].handle, ws[i % ncp][1].handle, ws[i % ncp][2].handle,
                P(x), T, P(y))), 200)
            # distinct experts the copies' routings touch, averaged
            touched = [len({int(e) for tt in range(T) for e in oracle.route(a[tt], k, True)[0]}) for a in lg]
            nexp = sum(touched) / len(touched)
            b = int(nexp * 3 * eb + 4 * T * (2 * embd + ne))
            out["qwen3moe_experts_T%d" % T] = {
                "us": round(ms * 1e3, 2), "algorithmic_bytes": b, "distinct_experts": nexp,
                "gbs": round(b / (ms * 1e-3) / 1e9, 1), "frac_hbm": round(b / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                "batch": T, "copies_rotated": ncp,
                "workload": "qwen3moe-style experts: hidden 2048, 128 experts FFN 768 Q4_K, top-8 of softmax over "
                            "N(0,1) router logits, route + gate/up + down + weighted combine"}

            def moe_cpu(T=T, hs=hosts[0], lg=lg[0]):
                xs = np.random.default_rng(3).standard_normal((T, embd), dtype=np.float32)
                thr = cpu_threads()
                best, reps = best_of(lambda: oracle.moe_ffn(lg, k, True, Q4_K, hs[0], Q4_K, hs[1], Q4_K, hs[2], ff,
                                                            embd, xs, T, each_token=True, threads=thr), 1.0)
                nx = len({int(e) for tt in range(T) for e in oracle.route(lg[tt], k, True)[0]})
                bb = nx * 3 * eb + 4 * T * (2 * embd + ne)
                return {"value": round(bb / best / 1e9, 3), "unit": "GB/s", "cores": thr, "kind": "port",
                        "ms": round(best * 1e3, 3),
                        "sample": "MoeFfn (route, SwiGLU per chosen expert, weighted sum) at batch %d, best of %d, "
                                  "C restatement (-O2 scalar), %d threads" % (T, reps, thr)}
            cpu.append(("qwen3moe_experts_T%d" % T, moe_cpu))
        for tri in ws:
            for w in tri:
                w.free()
    torch.cuda.synchronize()
    return out, cpu


def run_stream(args):
    """LayerStream's streaming mode on the GPU (src/LayerStream.cs:127-181): four distinct
    70B layers in pinned host memory, two stage slots in HBM; each step waits for its slot
    (Acquire), queues the next layer's copy into the other slot (StartPrefetch), runs the
    layer's seven GEMVs and releases its slot. Reports the copy bandwidth alone, the compute
    alone (resident) and the streamed time per layer."""
    import torch
    import windlass_amd
    from windlass_amd import synth
    from windlass_amd._lib import check
    from windlass_amd.backend import Context, HostBuffer

    L = windlass_amd.load()
    rng = np.random.default_rng(0x57494E44 + 3000)
    offs, total = {}, 0
    for n, t, r, c in LAYER:
        offs[n] = total
        total += (r * row_bytes(t, c) + 63) // 64 * 64
    nhost = 4
    hosts = []
    for _ in range(nhost):
        hb = HostBuffer(total)
        for n, t, r, c in LAYER:
            d = synth.blocks(t, r, c, rng)
            hb.array[offs[n]:offs[n] + d.size] = d
        hosts.append(hb)
    ctx = Context(0)
    slots = [ctx.stage(total) for _ in range(2)]
    views = [{n: s.weight(offs[n], t, r, c, name=n) for n, t, r, c in LAYER} for s in slots]
    dev = torch.device("cuda:0")
    T = args.batch
    x = torch.from_numpy(synth.activations(rng, T, HIDDEN)).to(dev)
    yq = torch.empty((T, HEADS * HEAD_DIM), device=dev)
    yk = torch.empty((T, KV_HEADS * HEAD_DIM), device=dev)
    yv = torch.empty((T, KV_HEADS * HEAD_DIM), device=dev)
    yo = torch.empty((T, HIDDEN), device=dev)
    h = torch.empty((T, FFN), device=dev)
    out = torch.empty((T, HIDDEN), device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def layer(v):
        ws = (ctypes.c_void_p * 3)(v["q"].handle.value, v["k"].handle.value, v["v"].handle.value)
        ys = (ctypes.c_void_p * 3)(yq.data_ptr(), yk.data_ptr(), yv.data_ptr())
        check(L.wl_matmul_multi_dev(ctx.handle, 3, ws, P(x), T, ys))
        check(L.wl_matmul_dev(ctx.handle, v["o"].handle, -1, P(yq), T, P(yo)))
        check(L.wl_gate_up_dev(ctx.handle, v["gate"].handle, v["up"].handle, -1, P(yo), T, P(h)))
        check(L.wl_matmul_dev(ctx.handle, v["down"].handle, -1, P(h), T, P(out)))

    # copies alone: one stage after another into alternating slots
    for i in range(2):
        slots[i % 2].upload_async(hosts[i].array, 0)
    for s in slots:
        s.sync()
    reps = 8
    t0 = time.perf_counter()
    for i in range(reps):
        slots[i % 2].upload_async(hosts[i % nhost].array, 0)
    for s in slots:
        s.sync()
    copy_s = (time.perf_counter() - t0) / reps
    # compute alone: the layer resident in a slot
    slots[0].ready()
    ctx.sync()
    steps = 50
    t0 = time.perf_counter()
    for _ in range(steps):
        layer(views[0])
    ctx.sync()
    compute_s = (time.perf_counter() - t0) / steps
    # streamed: copy of layer i+1 beside the compute of layer i
    slots[0].upload_async(hosts[0].array, 0)
    nstream = 16
    t0 = time.perf_counter()
    for i in range(nstream):
        s = i % 2
        slots[s].ready()
        if i + 1 < nstream:
            slots[1 - s].upload_async(hosts[(i + 1) % nhost].array, 0)
        layer(views[s])
        slots[s].release()
    ctx.sync()
    stream_s = (time.perf_counter() - t0) / nstream
    for vs in views:
        for v in vs.values():
            v.free()
    for s in slots:
        s.free()
    ctx.close()
    for hb in hosts:
        hb.free()
    h2d = total / copy_s / 1e9
    line = {"metric": "70B Q4_K_M layer streamed from pinned host memory: host-to-HBM GB/s and ms/layer",
            "value": round(h2d, 2), "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
            "data": "synthetic seeded GGUF blocks (Q4_K/Q6_K), x ~ N(0,1)",
            "config": {"workload": "Llama-3.3-70B Q4_K_M decoder layer as one stage (%d bytes), 2 HBM slots, "
                                   "4 distinct layers in pinned host memory" % total, "batch": T},
            "stage_bytes": total, "copy_ms_per_layer": round(copy_s * 1e3, 3),
            "compute_ms_per_layer": round(compute_s * 1e3, 4), "streamed_ms_per_layer": round(stream_s * 1e3, 3),
            "overlap": round(max(copy_s, compute_s) / stream_s, 3),
            "resident_note": "with every stage resident (288 GB HBM holds the 42.5 GB file) a layer takes the compute time"}
    print(json.dumps(line), flush=True)


VOCAB = 128256


def run_decode(args):
    """Whole-token greedy decode of Llama-3.3-70B Q4_K_M on one GPU with every tensor resident
    (windlass_amd.DeviceTransformer: Transformer.Forward, src/Transformer.cs:83-125, and the greedy
    loop, src/Engine.cs:356-360). 80 distinct layers in HBM (each its own copy of one synthetic
    layer's blocks), a Q4_K embedding and a Q6_K head of 128256 rows, fp16 KV caches. The prompt
    runs as one prefill pass (the MFMA GEMMs), then --warmup greedy tokens untimed and --tokens
    timed with each sampled id fed to the next step on the device (value); then 16 tokens with
    the host reading every id before the next step (host_synced_tokens_per_s)."""
    import torch
    import windlass_amd
    from windlass_amd import DeviceTransformer, ModelConfig, synth
    from windlass_amd.backend import Context

    rng = np.random.default_rng(0x57494E44 + 4000)
    host = {n: synth.blocks(t, r, c, rng) for n, t, r, c in LAYER}
    names = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate",
             "up": "ffn_up", "down": "ffn_down"}
    windlass_amd.load()
    ctx = Context(0)
    dev = torch.device("cuda:0")

    def vocab_blocks(t):  # 1/8 of the rows synthesised, repeated (content does not change the timing)
        return np.tile(synth.blocks(t, VOCAB // 8, HIDDEN, rng), 8)

    def norm():
        return torch.from_numpy((1 + 0.2 * rng.standard_normal(HIDDEN)).astype(np.float32)).to(dev)

    t0 = time.perf_counter()
    weights = {"token_embd": ctx.upload(Q4_K, vocab_blocks(Q4_K), VOCAB, HIDDEN, name="token_embd"),
               "output": ctx.upload(Q6_K, vocab_blocks(Q6_K), VOCAB, HIDDEN, name="output")}
    vectors = {"output_norm": norm()}
    for l in range(args.layers):
        for n, t, r, c in LAYER:
            key = "blk.%d.%s" % (l, names[n])
            weights[key] = ctx.upload(t, host[n], r, c, name=key)
        vectors["blk.%d.attn_norm" % l], vectors["blk.%d.ffn_norm" % l] = norm(), norm()
    load_s = time.perf_counter() - t0
    cfg = ModelConfig(layers=args.layers, embd=HIDDEN, heads=HEADS, kv_heads=KV_HEADS, head_dim=HEAD_DIM,
                      rope_base=500000.0, eps=1e-5)
    host_tokens = 16
    ctxlen = args.prompt + args.warmup + args.tokens + host_tokens + 1
    m = DeviceTransformer(ctx, cfg, weights, vectors, ctxlen)
    prompt = [int(v) for v in rng.integers(0, VOCAB, args.prompt)]
    ctx.sync()
    t0 = time.perf_counter()
    m.forward(prompt, 0)
    ctx.sync()
    prefill_s = time.perf_counter() - t0
    # the greedy loop with each id fed back on the device (the host queues ahead)
    ids = torch.empty(args.warmup + args.tokens + 1, dtype=torch.int32, device=dev)
    m.sample_into(ids[0:1])
    pos = args.prompt
    for i in range(args.warmup):
        m.forward_ids(ids[i:i + 1], pos)
        m.sample_into(ids[i + 1:i + 2])
        pos += 1
    ctx.sync()
    t0 = time.perf_counter()
    for i in range(args.warmup, args.warmup + args.tokens):
        m.forward_ids(ids[i:i + 1], pos)
        m.sample_into(ids[i + 1:i + 2])
        pos += 1
    ctx.sync()
    decode_s = time.perf_counter() - t0
    # the same with the host reading every id before the next step (the engine's loop)
    tok = int(ids[-1].item())
    t0 = time.perf_counter()
    for _ in range(host_tokens):
        m.forward([tok], pos)
        tok = m.sample()
        pos += 1
    host_s = (time.perf_counter() - t0) / host_tokens
    per_tok = decode_s / args.tokens
    wbytes = sum(w.Rows * w.RowBytes for k, w in weights.items() if k != "token_embd") + HIDDEN * 2 * 4 * args.layers
    emb_row = HIDDEN // 256 * 144
    kv_bytes = args.layers * 2 * 2 * KV_HEADS * HEAD_DIM * (args.prompt + args.warmup + args.tokens / 2)
    line = {"metric": "70B Q4_K_M whole-token greedy decode, every tensor resident in HBM",
            "value": round(1.0 / per_tok, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.tokens,
            "warmup": args.warmup, "ms_per_step": round(per_tok * 1e3, 3), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "fp32 accumulate over Q4_K/Q6_K blocks",
            "data": "synthetic seeded GGUF blocks; random prompt ids; random-init norms",
            "config": {"workload": "Llama-3.3-70B Q4_K_M: %d layers (hidden 8192, FFN 28672, 64/8 heads of 128), "
                                   "vocab 128256, prompt %d then %d timed tokens"
                                   % (args.layers, args.prompt, args.tokens), "batch": 1},
            "ms_per_layer": round(per_tok * 1e3 / args.layers, 4),
            "weights_read_per_token_bytes": int(wbytes + emb_row),
            "kv_read_per_token_bytes_mean": int(kv_bytes),
            "effective_GBps": round((wbytes + emb_row + kv_bytes) / per_tok / 1e9, 1),
            "host_synced_tokens_per_s": round(1.0 / host_s, 2),
            "prefill_tokens_per_s": round(args.prompt / prefill_s, 1), "prefill_s": round(prefill_s, 4),
            "load_s": round(load_s, 2)}
    print(json.dumps(line), flush=True)
    for w in weights.values():
        w.free()
    ctx.close()


def run_decode_batch(args):
    """--decode with --batch N: N sequences decoding together on the resident 70B model
    (DeviceBatch: ForwardBatch's stacked step, src/Transformer.cs:127-170). Each sequence's
    prompt runs into its own KV slot, then --warmup untimed and --tokens timed stacked steps with
    the ids fed back on the device. value = tokens of all sequences per second."""
    import torch
    import windlass_amd
    from windlass_amd import DeviceBatch, DeviceTransformer, ModelConfig, synth
    from windlass_amd._lib import check
    from windlass_amd.backend import Context

    N = args.batch
    rng = np.random.default_rng(0x57494E44 + 4000)
    host = {n: synth.blocks(t, r, c, rng) for n, t, r, c in LAYER}
    names = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate",
             "up": "ffn_up", "down": "ffn_down"}
    L = windlass_amd.load()
    ctx = Context(0)
    ctx.FloatMma = args.float_mma
    dev = torch.device("cuda:0")

    def norm():
        return torch.from_numpy((1 + 0.2 * rng.standard_normal(HIDDEN)).astype(np.float32)).to(dev)

    weights = {"token_embd": ctx.upload(Q4_K, np.tile(synth.blocks(Q4_K, VOCAB // 8, HIDDEN, rng), 8), VOCAB, HIDDEN),
               "output": ctx.upload(Q6_K, np.tile(synth.blocks(Q6_K, VOCAB // 8, HIDDEN, rng), 8), VOCAB, HIDDEN)}
    vectors = {"output_norm": norm()}
    for l in range(args.layers):
        for n, t, r, c in LAYER:
            key = "blk.%d.%s" % (l, names[n])
            weights[key] = ctx.upload(t, host[n], r, c, name=key)
        vectors["blk.%d.attn_norm" % l], vectors["blk.%d.ffn_norm" % l] = norm(), norm()
    cfg = ModelConfig(layers=args.layers, embd=HIDDEN, heads=HEADS, kv_heads=KV_HEADS, head_dim=HEAD_DIM,
                      rope_base=500000.0, eps=1e-5)
    cap = args.prompt + args.warmup + args.tokens + 1
    m = DeviceTransformer(ctx, cfg, weights, vectors, 1)
    b = DeviceBatch(m, N, cap)
    ids = torch.empty((args.warmup + args.tokens + 1, N), dtype=torch.int32, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    for i in range(N):
        lg = b.prefill(i, [int(v) for v in rng.integers(0, VOCAB, args.prompt)])
        check(L.wl_argmax_dev(ctx.handle, P(lg), 1, VOCAB, P(ids[0, i:])))
    seqs = list(range(N))
    for s in range(args.warmup):
        lg = b.step(seqs, ids[s])
        check(L.wl_argmax_dev(ctx.handle, P(lg), N, VOCAB, P(ids[s + 1])))
    ctx.sync()
    t0 = time.perf_counter()
    for s in range(args.warmup, args.warmup + args.tokens):
        lg = b.step(seqs, ids[s])
        check(L.wl_argmax_dev(ctx.handle, P(lg), N, VOCAB, P(ids[s + 1])))
    ctx.sync()
    per_step = (time.perf_counter() - t0) / args.tokens
    line = {"metric": "70B Q4_K_M greedy decode of N sequences together, every tensor resident in HBM",
            "value": round(N / per_step, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.tokens,
            "warmup": args.warmup, "ms_per_step": round(per_step * 1e3, 3), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "fp32 accumulate over Q4_K/Q6_K blocks",
            "data": "synthetic seeded GGUF blocks; random prompt ids; random-init norms",
            "config": {"workload": "Llama-3.3-70B Q4_K_M: %d layers, vocab 128256, %d sequences, prompt %d each, "
                                   "then %d timed stacked steps" % (args.layers, N, args.prompt, args.tokens),
                       "batch": N, "float_mma": bool(args.float_mma)},
            "tokens_per_s_per_sequence": round(1.0 / per_step, 2), "ms_per_layer": round(per_step * 1e3 / args.layers, 4)}
    print(json.dumps(line), flush=True)
    for w in weights.values():
        w.free()
    ctx.close()


# ggml type id -> name, for --formats
FORMATS = {12: "q4_K", 13: "q5_K", 14: "q6_K", 10: "q2_K", 11: "q3_K", 2: "q4_0", 3: "q4_1", 6: "q5_0",
           7: "q5_1", 8: "q8_0", 20: "iq4_nl", 23: "iq4_xs", 16: "iq2_xxs", 21: "iq3_s", 22: "iq2_s", 1: "f16",
           30: "bf16", 0: "f32"}


def run_formats(args):
    """The decode GEMV of every format at the 70B FFN shapes: gate/up-shaped 28672 x 8192 and
    down-shaped 8192 x 28672, at one token and eight. Four weight copies rotate (each at least
    117 MB for the 2-bit formats), HIP events on the library's stream, 200 launches per figure."""
    import torch
    import windlass_amd
    from windlass_amd import synth
    from windlass_amd._lib import check
    from windlass_amd.backend import Context, layout

    L = windlass_amd.load()
    ctx = Context(0)
    dev = torch.device("cuda:0")
    stream = torch.cuda.ExternalStream(ctx.stream, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    rng = np.random.default_rng(0x57494E44 + 5000)
    results = {}
    only = [n for n in args.only.split(",") if n]
    for t, name in FORMATS.items():
        if only and name not in only:
            continue
        be, bb = layout(t)
        for rows, cols in ((FFN, HIDDEN), (HIDDEN, FFN)):
            host = synth.blocks(t, rows, cols, rng)
            ws = [ctx.upload(t, host, rows, cols) for _ in range(args.copies)]
            for T in (1, 8):
                x = torch.from_numpy(synth.activations(rng, T, cols)).to(dev)
                y = torch.empty((T, rows), device=dev)

                def run(i):
                    check(L.wl_matmul_dev(ctx.handle, ws[i % len(ws)].handle, -1, P(x), T, P(y)))

                with torch.cuda.stream(stream):
                    for i in range(10):
                        run(i)
                    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    a.record(stream)
                    for i in range(200):
                        run(i)
                    b.record(stream)
                b.synchronize()
                ms = a.elapsed_time(b) / 200
                byt = rows * (cols // be * bb) + 4 * T * (rows + cols)
                results["%s_%dx%d_T%d" % (name, rows, cols, T)] = {
                    "us": round(ms * 1e3, 2), "gbs": round(byt / (ms * 1e-3) / 1e9, 1)}
            for w in ws:
                w.free()
    ctx.close()
    q4 = results.get("q4_K_%dx%d_T1" % (FFN, HIDDEN), {}).get("gbs")
    line = {"metric": "decode GEMV HBM GB/s per GGUF format at 70B FFN shapes", "value": q4, "unit": "GB/s",
            "n_gpus": 1, "higher_is_better": True, "dtype": "f32", "data": "synthetic seeded blocks, x ~ N(0,1)",
            "config": {"workload": "one matrix per launch: 28672x8192 and 8192x28672, batch 1 and 8",
                       "layer_copies": args.copies},
            "value_is": "q4_K 28672x8192 at batch 1", "per_format": results}
    print(json.dumps(line), flush=True)


def cpu_baseline(host, T, rng, budget_s):
    """The oracle (C restatement of the reference's CPU MatMul: DotRow per row in a parallel
    loop over 32-row tiles) on the host cores: best of repeated whole layers within budget,
    built -O2 scalar (the reference's RyuJIT code) and, as an upper bound, -O3 -march=native."""
    oracle = _oracle()
    threads = cpu_threads()
    x = rng.standard_normal((T, HIDDEN), dtype=np.float32)
    xf = rng.standard_normal((T, FFN), dtype=np.float32)

    def layer():
        for n, t, r, c in LAYER:
            oracle.matmul(t, host[n], r, c, xf if c == FFN else x, T, each_token=True, threads=threads)
    best, reps = best_of(layer, budget_s)
    gbs = algo_bytes(LAYER, T) / best / 1e9
    out = {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
           "ms_per_layer": round(best * 1e3, 2),
           "sample": "whole 70B layer (7 GEMVs) at batch %d, best of %d reps, C restatement of "
                     "Transformer.MatMul/DotRow (-O2, scalar, -ffp-contract=off), %d threads" % (T, reps, threads)}
    out.update(cpu_info())
    try:
        oracle.use("native")
        nbest, nreps = best_of(layer, budget_s / 2)
        out["native_O3_march_native"] = {"value": round(algo_bytes(LAYER, T) / nbest / 1e9, 2), "unit": "GB/s",
                                         "ms_per_layer": round(nbest * 1e3, 2), "reps": nreps,
                                         "build": "gcc -O3 -march=native -ffp-contract=off on this host"}
    except Exception as e:  # a host without a compiler keeps the scalar figure
        out["native_O3_march_native"] = {"error": str(e)[:200]}
    finally:
        oracle.use("scalar")
    return out


if __name__ == "__main__":
    main()
