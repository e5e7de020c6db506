"""Throughput of the MI355X token sampler on its headline workload.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload peaked] [--cpu-budget 10]

A step is one vsmp_pick_batch call over one batch of device-resident logits: the full sampler
pipeline (penalty, top-k, softmax numerators, min-p, top-p, counter-RNG draw) for every row.
Default workload ("peaked"): B=256 x V=151936 fp32, see verbo_amd/workloads.py. The logits are
replicated into enough buffers (> 600 MB) that consecutive steps never find their input in the
256 MB Infinity Cache. Prints one JSON line (stdout); progress goes to stderr.

Fields: value = rows/s over the timed steps; roofline.achieved = algorithmic bytes per call /
mean call duration (two HIP events around the timed steps, on the launch stream);
config.replays_ms_per_step = the median, least and greatest per-step time over 20 further replays
of the same graph, each between its own events (the run-to-run spread); cpu_baseline = the reference sampler
compiled from its sources (oracle/_ref), or the oracle restatement when that is not built, timed
on this host for a bounded sample of the same rows: one thread (value, cores) and every host
thread (value_all_cores, cores_all).
"""
import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
HBM_PEAK_GBS = 8000.0
# how oracle/Makefile compiles the reference's sources for the CPU baseline (its flags, stated)
REF_BUILD = ("the reference's src/*.cpp compiled by oracle/Makefile: g++ -std=c++17 -O3 -march=x86-64-v3 -fPIC "
             "-pthread -fvisibility=hidden -fno-math-errno (the reference's CMake flags, with x86-64-v3 for "
             "-march=native since the library is built on another host than the one it runs on)")
METRIC = "sampled rows/s + % HBM peak, full sampler, B=256 x V=151936 fp32 logits"
DESCR = {
    "single": "single: 1 x 49152 fp32 N(0,2.5^2)+8 spikes, H=64, repeat 1.1, temp .7, top-k 40, top-p .9",
    "greedy": "greedy: 64 x 151936 fp32 N(0,3^2), H=256, repeat 1.15, temp 0, 10% rows with an exact max tie",
    "peaked": ("peaked: 256 x 151936 fp32, 2*Gumbel + 12*rank^-1.1 on 2000 ids, H=512 (half boosted, "
               "repeat_last=0), repeat 1.1, temp .8, top-k 50, top-p .95, min-p .05, per-row seeds 0..255, "
               "counter-RNG draws"),
    "wide": "wide: 512 x 151936 fp32 N(0,0.5^2), top-k 0, top-p .99, temp 1, no penalty",
    "mixed": ("mixed: 1024 x 128256 fp32 N(0,2^2)+spikes, per-row temp/top-k/top-p/min-p/repeat, H U[0,2048], "
              "25% greedy"),
    "head": ("head: LM head 256 x 896 bf16 hidden states against a 151936 x 896 bf16 head (Qwen2.5-0.5B's "
             "shape), fp32 logits, then the peaked workload's sampler (temp .8, top-k 50, top-p .95, min-p .05, "
             "repeat 1.1 over H=512), counter-RNG draws"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_threads():
    """CPU threads this process may use: its affinity set, capped by OMP_NUM_THREADS when set."""
    import os

    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def cpu_baseline(w, budget):
    """Time the reference sampler's pick() on this host over the workload's rows: one thread for
    `budget` seconds (the reported value), then every host thread (rows statically partitioned, one
    sampler per row) for half of it. Uses oracle/_ref when built, else the oracle restatement (one
    thread only)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import numpy as np

    import oracle as O

    params = w.params.copy()
    params["repeat_last"] = 0
    kind = "reference" if O.ref_available() else "port"
    res = {}
    if kind == "reference":
        secs, picks = O.ref_time_rows(w.logits, params, w.hist, w.hist_off, threads=1, budget_s=budget)
        nt = min(host_threads(), w.B)
        secs_all, picks_all = O.ref_time_rows(w.logits, params, w.hist, w.hist_off, threads=nt, budget_s=budget / 2)
        res = {"value_all_cores": picks_all / secs_all, "cores_all": nt}
    else:
        lib = O.load_oracle()
        u = np.full(w.B, 0.5)
        picks, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget:
            O.pick_rows(w.logits, params, w.hist, w.hist_off, u, threads=1)
            picks += w.B
        secs = time.perf_counter() - t0
        del lib
    out = {"value": picks / secs, "unit": "rows/s", "cores": 1, "kind": kind,
           "sample": f"{picks} pick() calls cycling over the {w.B} rows of the same workload for {secs:.1f} s, "
                     f"1 thread, pick only (history accepted beforehand)",
           "build": REF_BUILD if kind == "reference" else "oracle/vsmp_oracle.c, gcc -O2"}
    out.update(res)
    return out


def bench_single(args):
    """The single-row decode workload: 10,000 consecutive draws on one fixed
    1 x 49152 row and history (seed 42, no accept between draws). Reports microseconds per draw for
    the device-resident calls (value: draws/s), the same calls replayed from a HIP graph (100 per
    graph), the drop-in verbo::Sampler::pick on a host row (the path verbo's generate takes: the row
    copied to the device, the id copied back, one synchronisation per pick, plus the ctypes call from
    Python), and the reference's pick on the host CPU (oracle/_ref) on the same row."""
    import numpy as np
    import torch

    import verbo_amd as V
    from verbo_amd import workloads as W

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O

    w = W.make("single")
    p0 = w.params[0]
    prm = V.Params(*[p0[f].item() for f in V.SAMPLING_DTYPE.names])
    dev = torch.device("cuda:0")
    d = torch.from_numpy(w.logits).to(dev)
    h, ho = torch.from_numpy(w.hist).to(dev), torch.from_numpy(w.hist_off).to(dev)
    st0 = O.rng_seed(int(p0["seed"]))
    rng = torch.from_numpy(np.array([st0[0], st0[1]], np.uint64).view(np.int64)).to(dev)
    n = args.draws
    out = torch.empty(n, dtype=torch.int32, device=dev)
    ctx = V.Context(0)
    stream = torch.cuda.current_stream(dev)

    def eager(k):
        for i in range(k):
            ctx.pick_batch(d, prm, h, ho, V.U_XORSHIFT, rng_state=rng, out=out[i:i + 1], stream=stream)

    eager(args.warmup)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    eager(n)
    e1.record(stream)
    torch.cuda.synchronize()
    us_eager = e0.elapsed_time(e1) * 1e3 / n
    log(f"[bench] single: {n} device-resident calls, {us_eager:.2f} us per draw")
    per = 100
    g = torch.cuda.CUDAGraph()
    gs = torch.cuda.Stream()
    with torch.cuda.stream(gs):
        with torch.cuda.graph(g, stream=gs):
            for i in range(per):
                ctx.pick_batch(d, prm, h, ho, V.U_XORSHIFT, rng_state=rng, out=out[i:i + 1], stream=gs)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(n // per):
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    us_graph = e0.elapsed_time(e1) * 1e3 / (n // per * per)
    log(f"[bench] single: graph replays, {us_graph:.2f} us per draw")
    s = V.Sampler(prm)
    for t in w.hist:
        s.accept(int(t))
    row = np.ascontiguousarray(w.logits[0])
    for _ in range(args.warmup):
        s.pick(row)
    k = min(n, 2000)
    t0 = time.perf_counter()
    for _ in range(k):
        s.pick(row)
    us_host = (time.perf_counter() - t0) * 1e6 / k
    log(f"[bench] single: drop-in Sampler::pick on a host row, {us_host:.2f} us per draw")
    cpu = None
    if args.cpu_budget > 0 and O.ref_available():
        c = O.Sampling(*[p0[f].item() for f in O.SAMPLING_DTYPE.names])
        m = 2000
        t0 = time.perf_counter()
        O.ref_sampler_run(w.logits[0], c, w.hist, n_picks=m)
        secs = time.perf_counter() - t0
        cpu = {"value": m / secs, "unit": "draws/s", "cores": 1, "kind": "reference",
               "sample": f"{m} consecutive pick() calls of one reference Sampler on the same row, 1 thread",
               "build": REF_BUILD}
    return {
        "metric": "single-row draws/s, " + DESCR["single"] + ", 10,000 consecutive draws",
        "value": 1e6 / us_eager,
        "unit": "draws/s",
        "n_gpus": 1,
        "steps": n,
        "warmup": args.warmup,
        "ms_per_step": us_eager * 1e-3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": DESCR["single"], "B": 1, "V": w.V, "draw_stream": "the reference's xorshift128+ "
                   "on the device (VSMP_U_XORSHIFT)", "epilogue_dtype": "f64"},
        "us_per_draw": {"device_resident": us_eager, "graph_replay": us_graph, "drop_in_host_row": us_host},
        "roofline": None,
        "cpu_baseline": cpu,
    }


def settle(graph, stream, ms=20.0):
    """Untimed replays of a captured graph until the GPU has run it for about `ms` milliseconds: the
    first replays after the capture run slower (2-4% on the sampler's steps, measured on MI355X),
    as the GPU's clocks settle."""
    import torch

    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    for _ in range(max(0, math.ceil(ms / max(e0.elapsed_time(e1), 1e-3)) - 1)):
        graph.replay()
    torch.cuda.synchronize()


def bench_head(args):
    """The LM head and the pick in one call (vsmp_head_pick, its route by batch size), the fused
    route pinned, the same work unfused (the head's logits written by vsmp_head_logits, then
    vsmp_pick_batch over them), and the head's product alone. Each variant: K steps captured into a
    HIP graph and replayed, timed by two events on the launch stream; the head rotates over three
    copies (816 MB) so that no step finds it in the 256 MB Infinity Cache. value = rows/s of
    vsmp_head_pick."""
    import numpy as np
    import torch

    import verbo_amd as V

    B, Vv, D, H = args.head_rows, 151936, 896, 512
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    hidden = torch.randn(B, D, device=dev, generator=g).to(torch.bfloat16)
    heads = [(torch.randn(Vv, D, device=dev, generator=g) * (3.0 / D ** 0.5)).to(torch.bfloat16) for _ in range(3)]
    rng = np.random.default_rng(7)
    hist = torch.from_numpy(rng.integers(0, Vv, B * H).astype(np.int32)).to(dev)
    hoff = torch.from_numpy(np.arange(0, B * H + 1, H, dtype=np.int32)).to(dev)
    prm = V.Params(temp=0.8, top_k=50, top_p=0.95, min_p=0.05, repeat=1.1, repeat_last=0, seed=0)
    out = torch.empty(B, dtype=torch.int32, device=dev)
    lg = torch.empty(B, Vv, dtype=torch.float32, device=dev)
    ctx = V.Context(0)
    saved = os.environ.get("VSMP_HEAD_ROUTE")
    os.environ["VSMP_HEAD_ROUTE"] = "fused"
    try:
        ctx_fused = V.Context(0)  # the switch is read when a context is created
    finally:
        os.environ.pop("VSMP_HEAD_ROUTE")
        if saved is not None:
            os.environ["VSMP_HEAD_ROUTE"] = saved
    stream = torch.cuda.current_stream(dev)

    def pick(i, st):
        ctx.head_pick(hidden, heads[i % 3], prm, hist, hoff, V.U_COUNTER, counter=i, out=out, stream=st)

    def fused(i, st):
        ctx_fused.head_pick(hidden, heads[i % 3], prm, hist, hoff, V.U_COUNTER, counter=i, out=out, stream=st)

    def unfused(i, st):
        ctx.head_logits(hidden, heads[i % 3], logits=lg, stream=st)
        ctx.pick_batch(lg, prm, hist, hoff, V.U_COUNTER, counter=i, out=out, stream=st)

    def product(i, st):
        ctx.head_logits(hidden, heads[i % 3], logits=lg, stream=st)

    def timed(fn):
        for i in range(args.warmup):
            fn(i, stream)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream(dev)
        cap.wait_stream(stream)
        with torch.cuda.graph(graph, stream=cap):
            for i in range(args.steps):
                fn(args.warmup + i, cap)
        torch.cuda.synchronize()
        graph.replay()
        settle(graph, stream)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps

    def library(i, st):  # the vendor library's product of the same operands (bf16 out), for reference
        with torch.cuda.stream(st):
            torch.nn.functional.linear(hidden, heads[i % 3])

    ms = {name: timed(fn) for name, fn in (("pick", pick), ("fused", fused), ("unfused", unfused),
                                           ("product", product), ("library", library))}
    for k_, v in ms.items():
        log(f"[bench] head: {k_} {v * 1e3:.1f} us/step")
    head_bytes = Vv * D * 2
    alg = head_bytes + B * D * 2 + B * 64 * 4 + B * 4  # head, hidden, the penalised ids read, ids out
    achieved = alg / (ms["pick"] * 1e-3) / 1e9
    flops = 2.0 * B * Vv * D
    return {
        "metric": f"sampled rows/s, {DESCR['head']}".replace("256 x 896", f"{B} x 896"),
        "value": B / (ms["pick"] * 1e-3),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms["pick"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": DESCR["head"].replace("256 x 896", f"{B} x 896"), "B": B, "V": Vv, "D": D,
                   "head_copies": 3,
                   "algorithmic_bytes_per_step": alg, "issue": "hip_graph",
                   "route": "fused" if 16 <= B <= 64 else "whole",
                   "fused_ms_per_step": ms["fused"],
                   "unfused_ms_per_step": ms["unfused"], "product_ms_per_step": ms["product"],
                   "library_product_bf16_ms_per_step": ms["library"],
                   "mfma_tflops_pick": flops / (ms["pick"] * 1e-3) / 1e12,
                   "mfma_tflops_product": flops / (ms["product"] * 1e-3) / 1e12},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None},
        "cpu_baseline": None,
    }


def traffic_from_profiles(name):
    """HBM bytes per call measured by rocprofv3 PMC runs (profiles/<workload>_traffic.json)."""
    p = ROOT / "profiles" / f"{name}_traffic.json"
    if not p.is_file():
        return None
    try:
        return float(json.loads(p.read_text())["bytes_per_call"])
    except (ValueError, KeyError):
        return None


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="peaked", choices=sorted(DESCR))
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU-baseline timing (0: skip)")
    ap.add_argument("--min-buffer-mb", type=float, default=640.0)
    ap.add_argument("--draws", type=int, default=10000, help="single workload: consecutive draws timed")
    ap.add_argument("--head-rows", type=int, default=256, help="head workload: rows (hidden states) per call")
    ap.add_argument("--eager", action="store_true", help="issue the timed calls one by one instead of from a HIP graph")
    ap.add_argument("--copy", action="store_true",
                    help="time a plain device copy of one logits buffer per step instead (the known-size kernel "
                         "that calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the sampler has no multi-GPU path (asked for --gpus {args.gpus}). "
              f"Rows are independent, so each GPU would take its own share of the batch's rows.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import verbo_amd as V
    from verbo_amd import workloads as W

    assert torch.cuda.is_available(), "bench.py needs a ROCm device"
    if args.workload == "single":
        print(json.dumps(bench_single(args)), flush=True)
        return
    if args.workload == "head":
        print(json.dumps(bench_head(args)), flush=True)
        return
    dev = torch.device("cuda:0")
    t0 = time.perf_counter()
    w = W.make(args.workload)
    log(f"[bench] workload {args.workload} {w.B}x{w.V} generated in {time.perf_counter() - t0:.1f}s")
    nbytes = w.logits.nbytes
    nbuf = max(1, math.ceil(args.min_buffer_mb * 1e6 / nbytes))
    host = torch.from_numpy(w.logits)
    bufs = [host.to(dev) for _ in range(nbuf)]
    params = V.to_device_params(w.params, dev) if w.per_row else \
        V.Params(*[w.params[0][f].item() for f in V.SAMPLING_DTYPE.names])
    hist = torch.from_numpy(w.hist if w.hist.size else np.zeros(1, np.int32)).to(dev)
    hoff = torch.from_numpy(w.hist_off).to(dev)
    out = torch.empty(w.B, dtype=torch.int32, device=dev)
    ctx = V.Context(0)
    stream = torch.cuda.current_stream(dev)

    def step(i, st=stream):
        ctx.pick_batch(bufs[i % nbuf], params, hist, hoff, V.U_COUNTER, counter=i, out=out, stream=st)

    if args.copy:
        dst = torch.empty_like(bufs[0])

        def step(i, st=stream):  # noqa: F811 - the calibration step replaces the sampler step
            dst.copy_(bufs[i % nbuf])

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    log(f"[bench] warmup {args.warmup} done, {nbuf} buffers x {nbytes / 1e6:.1f} MB")
    # The K timed steps are issued from a HIP graph that holds them (captured once, replayed once):
    # the GPU then runs them back to back, and the figure is the sampler's, not the Python loop's
    # launch rate (each call costs the host tens of microseconds in ctypes and planning). Two
    # events bracket the replay on the launch stream. --eager times the calls issued one by one.
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    use_graph = not (args.eager or args.copy)
    if use_graph:
        graph = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream(dev)
        cap.wait_stream(stream)
        with torch.cuda.graph(graph, stream=cap):
            for i in range(args.steps):
                step(args.warmup + i, cap)
        torch.cuda.synchronize()
        graph.replay()  # untimed: the first replay uploads the graph
        settle(graph, stream)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    e0.record(stream)
    if use_graph:
        graph.replay()
    else:
        for i in range(args.steps):
            step(args.warmup + i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    total_ms = e0.elapsed_time(e1)
    ms_per_step = total_ms / args.steps
    eager_ms = None
    if use_graph:  # the same steps issued one by one, for comparison
        torch.cuda.synchronize()
        e0.record(stream)
        for i in range(args.steps):
            step(args.warmup + i)
        e1.record(stream)
        torch.cuda.synchronize()
        eager_ms = e0.elapsed_time(e1) / args.steps
    # run-to-run spread: 20 more replays of the same graph, each between its own two events
    reps_ms = []
    if use_graph:
        for _ in range(20):
            e0.record(stream)
            graph.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            reps_ms.append(e0.elapsed_time(e1) / args.steps)
        reps_ms.sort()
    log(f"[bench] {args.steps} steps: {ms_per_step * 1e3:.1f} us/step (wall {wall * 1e3:.2f} ms)")
    if args.copy:
        gbs = 2 * nbytes / (ms_per_step * 1e-3) / 1e9
        print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "us_per_copy": ms_per_step * 1e3,
                          "GB_per_s_read_plus_write": gbs}), flush=True)
        return
    # attainable read bandwidth on this box: the library's plain streaming-read kernel over the same
    # buffers, from a graph as the steps are (issued one by one from Python, the reads would wait on
    # the host's launch rate: each takes about 23 us on the GPU)
    for i in range(nbuf):
        ctx.read_probe(bufs[i], stream=stream)
    torch.cuda.synchronize()
    r0, r1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 8 * nbuf
    rgraph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream(dev)
    cap.wait_stream(stream)
    with torch.cuda.graph(rgraph, stream=cap):
        for i in range(reps):
            ctx.read_probe(bufs[i % nbuf], stream=cap)
    torch.cuda.synchronize()
    rgraph.replay()
    settle(rgraph, stream)
    r0.record(stream)
    rgraph.replay()
    r1.record(stream)
    torch.cuda.synchronize()
    attainable = reps * nbytes / (r0.elapsed_time(r1) * 1e-3) / 1e9
    log(f"[bench] attainable streaming read (plain read kernel over the same buffers): {attainable:.0f} GB/s")
    alg = w.algorithmic_bytes()
    achieved = alg / (ms_per_step * 1e-3) / 1e9
    traffic = traffic_from_profiles(args.workload)
    res = {
        "metric": METRIC if args.workload == "peaked" else f"sampled rows/s, {DESCR[args.workload]}",
        "value": w.B / (ms_per_step * 1e-3),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": DESCR[args.workload], "B": w.B, "V": w.V, "buffers": nbuf,
                   "algorithmic_bytes_per_step": alg, "epilogue_dtype": "f64",
                   "issue": "hip_graph" if use_graph else "eager",
                   "eager_ms_per_step": eager_ms,
                   "replays_ms_per_step": {"n": len(reps_ms), "median": reps_ms[len(reps_ms) // 2],
                                           "min": reps_ms[0], "max": reps_ms[-1]} if reps_ms else None},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic, "attainable_read": attainable},
    }
    if args.cpu_budget > 0:
        log(f"[bench] cpu baseline ({args.cpu_budget:.0f}s budget)")
        res["cpu_baseline"] = cpu_baseline(w, args.cpu_budget)
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
