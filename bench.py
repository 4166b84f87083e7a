"""Benchmark of the MI355X packed-weight hot path: one MoE block (router,
top-8 routing, stable dispatch, trellis-packed SwiGLU experts, route-order
combine, gated shared expert) at ubatch 1, 4, 16, 128 and 512 tokens, plus the
packed projections (2048x2048 non-expert, 151936x2048 int5 output head), the
token side of decoding (embedding rows, greedy and top-p choice), the
attention half of a decode step (full GQA attention, Gated DeltaNet, a whole
decoder layer) and the full 40-layer hybrid stack (256-token prefill at
ubatch 128, 64 greedy decode steps).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Prints one JSON line. `value` is MoE-layer tokens/s at ubatch 1 (decode);
the other ubatches and the projections are reported under `per_ubatch` and
`projections`. Each figure is the median of 7 runs of K timed steps after W
warm-up steps (the reference reports medians of 7, docs/benchmarks.md:262-265).
Weights are synthetic (seeded, reference codec formats); the steps cycle
through 8 layers and a pool of input batches, so each step routes to experts
the recent steps did not touch and the 256 MB Infinity Cache does not hold
the working set. Inputs are resident in HBM before the timed region.
The roofline object is for the kernel with the largest share of the headline
step time; its launch times come from start/stop events the runtime stamps
from each launch's own dispatch (the kernel's execution, as a kernel trace
reports it) over a separate pass of the same steps, and its `traffic` is the
measured HBM bytes per launch from the committed counter summary
(profiles/moe_layer_hbm_traffic.md), or null without one. `checksum` holds
the FNV-1a digests of the output bits of one layer call on each side
(src/main.cpp:90-103) and their largest relative difference.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16/bf16

HIDDEN, EXPERT_HIDDEN, EXPERTS = 2048, 512, 256
EXPERT_TILES = (EXPERT_HIDDEN // 16) * (HIDDEN // 16)           # per projection
EXPERT_TRELLIS_BYTES = EXPERT_TILES * 24 * 2                      # 196,608
EXPERT_GAMMA_BYTES = (EXPERT_HIDDEN // 16 + HIDDEN // 16) * 2     # 320
PER_EXPERT_BYTES = 3 * (EXPERT_TRELLIS_BYTES + EXPERT_GAMMA_BYTES) + 15360  # 606,144 incl. su/sv
NE_TRELLIS_BYTES = EXPERT_TILES * 64 * 2                          # 524,288 per shared matrix
ROUTER_BYTES = EXPERTS * HIDDEN * 2
SHARED_BYTES = 3 * NE_TRELLIS_BYTES + 3 * (HIDDEN + EXPERT_HIDDEN) + 3 * 4
FIXED_LAYER_BYTES = ROUTER_BYTES + SHARED_BYTES + HIDDEN * 2      # 2,633,228
FLOP_PER_TOKEN = 2 * (8 * 3 * EXPERT_HIDDEN * HIDDEN + 3 * EXPERT_HIDDEN * HIDDEN
                      + EXPERTS * HIDDEN + HIDDEN)
HEAD_ROWS, HEAD_COLUMNS = 151936, 2048
HEAD_BYTES = HEAD_ROWS * HEAD_COLUMNS // 8 * 5 + HEAD_ROWS * HEAD_COLUMNS // 64 * 2


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--layers", type=int, default=8, help="distinct layers in the weight rotation")
    p.add_argument("--ubatch", type=str, default="1,4,16,128,512")
    p.add_argument("--runs", type=int, default=7, help="timed runs per figure (median reported)")
    p.add_argument("--no-stack", action="store_true", help="skip the 40-layer stack")
    p.add_argument("--cpu-seconds", type=float, default=8.0, help="CPU baseline budget per ubatch")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--cpu-child", action="store_true", help=argparse.SUPPRESS)
    p.add_argument("--cpu-projections", action="store_true", help=argparse.SUPPRESS)
    p.add_argument("--projection-cpu-seconds", type=float, default=2.0,
                   help="CPU baseline budget per projection figure")
    p.add_argument("--no-projections", action="store_true")
    p.add_argument("--no-graph", action="store_true",
                   help="skip the graph-replay timing of the projections (counter runs)")
    p.add_argument("--projections-only", type=str, default="",
                   help="run only these packed projections (comma list of head_b1, head_b4, ne_b1, "
                        "ne_b4) and print their figures: one workload per profiler run")
    p.add_argument("--copy-bytes", type=int, default=0,
                   help="first run a plain device-to-device copy of this many bytes three times "
                        "(the calibration launch for the HBM byte counters)")
    return p.parse_args()


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def kernel_bytes(name, active):
    """Algorithmic packed bytes one launch of `name` reads, or None."""
    if name in ("moe_decode_one", "moe_decode_few"):
        # the whole layer in one launch (1 row, or 2-12 rows): router, shared
        # expert, and the active experts' gate, up and down with their scales
        return FIXED_LAYER_BYTES + active * PER_EXPERT_BYTES
    if name == "moe_gemv":
        # two launches per step: gate+up (2 expert + 2 shared matrices), down
        # (1 + 1); the mean launch reads half the step's GEMV packed bytes
        return (3 * active * (EXPERT_TRELLIS_BYTES + EXPERT_GAMMA_BYTES) + 3 * NE_TRELLIS_BYTES) / 2
    if name == "expert_mfma":
        # gate+up (2 matrices of every active expert) and down (1): the mean
        # launch decodes 1.5 matrices of each active expert
        return 1.5 * active * (EXPERT_TRELLIS_BYTES + EXPERT_GAMMA_BYTES)
    if name == "ne_mfma":
        return 1.5 * NE_TRELLIS_BYTES
    if name == "expert_gemv":
        return active * (EXPERT_TRELLIS_BYTES + EXPERT_GAMMA_BYTES)
    if name == "ne_gemv":
        return NE_TRELLIS_BYTES
    if name == "bf16_ordered":
        return None  # router (1 MiB) and shared gate (4 KiB) share the name
    return None


def input_pool_size(ubatch):
    """Distinct input batches a run cycles through. Step s runs layer s % L on
    batch (s // L) % X, so consecutive visits of a layer route different
    tokens and touch different experts: at ubatch 1 a step reads about 7.5 MB
    of weights that the previous ~30 steps did not, so the 256 MB Infinity
    Cache does not hold the working set."""
    return 64 if ubatch < 16 else (4 if ubatch < 256 else 2)


def moe_bench(torch, hip, ctx, layers, xs, biases, steps, warmup, runs):
    """Median wall time of `runs` runs of `steps` timed steps, the distinct
    experts per step, and a per-kernel timing pass over the same steps."""
    batch = xs[0].shape[0]
    out = torch.empty((batch, HIDDEN), dtype=torch.float32, device="cuda")
    routes = torch.empty(batch * 8, dtype=torch.int32, device="cuda")
    nl, nx = len(layers), len(xs)

    def step(s):
        j = (s // nl) % nx
        hip.moe_forward(ctx, layers[s % nl], xs[j], batch, biases[j], out, routes, None)

    for s in range(warmup):
        step(s)
    ctx.synchronize()
    walls = []
    for r in range(runs):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for s in range(warmup + r * steps, warmup + (r + 1) * steps):
            step(s)
        torch.cuda.synchronize()
        walls.append(time.perf_counter() - t0)
        # the library's own check after each run: a one-launch MoE wait that
        # ran out (its outputs invalid) fails the benchmark here
        ctx.synchronize()
    # distinct experts per step for the byte count
    active = []
    for s in range(warmup, warmup + steps):
        step(s)
        ctx.synchronize()
        active.append(len(np.unique(routes.cpu().numpy())))
    # per-kernel timing in a separate pass over the same steps
    ctx.profiling(True)
    for s in range(warmup, warmup + steps):
        step(s)
    prof = ctx.profile()
    ctx.profiling(False)
    ctx.synchronize()
    return walls, float(np.mean(active)), prof


def fnv1a64(data: bytes, h: int = 0xCBF29CE484222325) -> int:
    """FNV-1a over raw bytes (hash_bytes, src/main.cpp:90-103)."""
    for b in data:
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def copy_calibration(torch, nbytes):
    """Three plain device-to-device copies of `nbytes` (hipMemcpyAsync's blit
    kernel): the known-size launch the FETCH_SIZE / WRITE_SIZE counters of the
    hot-path kernels are scaled by."""
    n = nbytes // 4
    src = torch.arange(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy calibration: 3 copies of {nbytes} bytes")
    del src, dst


MOE_STATS = os.path.join(ROOT, "profiles", "moe_layer_kernel_stats.md")
MOE_TRAFFIC = os.path.join(ROOT, "profiles", "moe_layer_hbm_traffic.md")
PROJ_STATS = os.path.join(ROOT, "profiles", "projections_kernel_stats.md")
PROJ_TRAFFIC = os.path.join(ROOT, "profiles", "projections_hbm_traffic.md")


def traffic_from_profile(kernel, key, path=MOE_TRAFFIC):
    """Measured HBM bytes per launch of `kernel` in the workload `key` (an
    ubatch, or a projection's name), from a committed counter summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by the same counter's
    reading for a copy of known size), or None."""
    if not os.path.exists(path):
        return None
    for row in open(path):
        cells = [c.strip() for c in row.strip().strip("|").split("|")]
        if len(cells) >= 6 and cells[0] == str(key) and cells[1] == kernel:
            try:
                return int(float(cells[5]))
            except ValueError:
                return None
    return None


def kernel_flops(name, ubatch):
    """Algorithmic flops of the mean launch of `name` (2 x rows x columns per
    routed position), or None. expert_mfma runs twice per step: gate+up
    (2 x 512 x 2048 per position) and down (2048 x 512); the mean launch is
    1.5 projections of 8 * ubatch routed positions. ne_mfma likewise for the
    shared expert's ubatch rows."""
    if name in ("expert_mfma", "moe_gemv"):
        return 1.5 * 2.0 * 8 * ubatch * EXPERT_HIDDEN * HIDDEN
    if name == "ne_mfma":
        return 1.5 * 2.0 * ubatch * EXPERT_HIDDEN * HIDDEN
    if name in ("moe_decode_one", "moe_decode_few"):
        return FLOP_PER_TOKEN * ubatch
    return None


RIDGE_FLOP_PER_BYTE = MFMA_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)  # 312.5


ROCPROF_NAMES = {"moe_decode_one": "k_moe_decode_one", "moe_decode_few": "k_moe_decode_few",
                 "moe_gemv": "k_trellis_gemv",
                 "expert_mfma": "k_expert_mfma", "ne_fused": "k_ne_fused", "head": "k_head_mfma"}


def rocprof_avg_us(kernel, key, path=MOE_STATS):
    """Average duration (us) of `kernel` in the section `## <key>` of a
    committed rocprofv3 --kernel-trace --stats summary ("ubatch 4", or a
    projection's name), or None."""
    want = ROCPROF_NAMES.get(kernel)
    if want is None or not os.path.exists(path):
        return None
    section = None
    for row in open(path):
        if row.startswith("## "):
            section = row[3:].strip()
            continue
        cells = [c.strip().strip("`") for c in row.strip().strip("|").split("|")]
        if section == str(key) and len(cells) >= 3 and cells[0].split("<")[0] == want:
            return float(cells[2])
    return None


def roofline_for(prof, steps, active, ubatch, wall_ms_per_step):
    r = roofline_kernel(prof, active, ubatch)
    if r is None:
        return None
    name = r["kernel"]
    launches, ms = prof[name]
    r["event_avg_us"] = r["avg_launch_us"]
    r["timing"] = "per-launch HIP events"
    if launches == steps and r["share_of_step"] == 1.0:
        # the step is this one launch: the timed region (bracketed by device
        # synchronisation) per step bounds its duration from above without the
        # per-launch event overhead
        us = min(wall_ms_per_step * 1e3, r["avg_launch_us"])
        scale = r["avg_launch_us"] / us
        r["avg_launch_us"] = round(us, 2)
        r["achieved"] = round(r["achieved"] * scale, 2)
        r["frac"] = round(r["frac"] * scale, 4)
        r["timing"] = "timed region / launches (one launch per step)"
    r["rocprof_avg_us"] = rocprof_avg_us(name, f"ubatch {ubatch}")
    r["traffic"] = traffic_from_profile(name, ubatch)
    return r


def roofline_kernel(prof, active, ubatch):
    """The roofline of the launch kind with the largest share of the step
    that has an algorithmic count. Its bound follows its algorithmic
    intensity: MFMA at or above the ridge (312.5 FLOP per packed byte on
    MI355X), HBM below it."""
    total = sum(ms for _, ms in prof.values())
    ranked = sorted(prof.items(), key=lambda kv: -kv[1][1])
    for name, (launches, ms) in ranked:
        nbytes = kernel_bytes(name, active)
        flops = kernel_flops(name, ubatch)
        if nbytes is None and flops is None:
            continue
        avg_ms = ms / launches
        intensity = None if nbytes is None or flops is None else flops / nbytes
        r = {"kernel": name, "avg_launch_us": round(avg_ms * 1e3, 2),
             "share_of_step": round(ms / total, 3),
             "intensity_flop_per_byte": None if intensity is None else round(intensity, 1)}
        if nbytes is None or (intensity is not None and intensity >= RIDGE_FLOP_PER_BYTE):
            achieved = flops / (avg_ms * 1e-3) / 1e12
            r.update({"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_PEAK_TFLOPS,
                      "unit": "TFLOP/s", "frac": round(achieved / MFMA_PEAK_TFLOPS, 4),
                      "traffic": None, "flops_per_launch": int(flops)})
        else:
            achieved = nbytes / (avg_ms * 1e-3) / 1e9
            r.update({"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                      "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                      "bytes_per_launch": int(nbytes)})
            if flops is not None:
                r["flops_per_launch"] = int(flops)
        return r
    return None


# The reference's kernel kinds (include/adi/profiling.hpp:9-40) of this
# library's MoE launches. The routing, Hadamard, SwiGLU and combine launches
# are work the reference does inside moe_forward(_batch) outside any kernel
# timer: they count under "moe" only. At one row the whole layer is one
# launch, so its kinds are not separable on the device.
KIND_OF_LAUNCH = {"router": "bf16_projection", "expert_mfma": "expert_batch",
                  "ne_mfma": "non_expert_batch", "moe_gemv": "expert_batch+non_expert_batch"}


def kind_report(prof, steps, ubatch, cpu_kinds, cpu_ms):
    """The step by the reference's kernel kinds, device beside CPU: calls,
    milliseconds and the reference's work items per step."""
    gpu = {}
    total_ms, total_launches = 0.0, 0
    for name, (launches, ms) in prof.items():
        total_ms += ms
        total_launches += launches
        kind = KIND_OF_LAUNCH.get(name)
        if kind is not None:
            k = gpu.setdefault(kind, [0, 0.0])
            k[0] += launches
            k[1] += ms
    report = {"moe": {"gpu_launches_per_step": round(total_launches / steps, 2),
                      "gpu_ms_per_step": round(total_ms / steps, 4),
                      "cpu_ms_per_step": cpu_ms,
                      "work_items_per_step": ubatch * HIDDEN}}
    for kind, (launches, ms) in gpu.items():
        report[kind] = {"gpu_launches_per_step": round(launches / steps, 2),
                        "gpu_ms_per_step": round(ms / steps, 4)}
    for kind, v in (cpu_kinds or {}).items():
        entry = report.setdefault(kind, {})
        entry["cpu_calls_per_step"] = v["calls_per_step"]
        entry["cpu_ms_per_step"] = v["ms_per_step"]
        entry["work_items_per_step"] = v["work_items_per_step"]
        if "gpu_ms_per_step" not in entry:
            entry["gpu_ms_per_step"] = None
            entry["gpu_note"] = ("inside the one-launch layer" if ("moe_decode_one" in prof or
                                                                    "moe_decode_few" in prof) else
                                 "inside " + next((k for k in gpu if kind in k.split("+")), "moe"))
    return report


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(layer_host, xs, biases, seconds):
    """The reference's own CPU layer (compiled from its sources, its worker
    pool at ADI_THREADS threads) on the bench's first layer and inputs: one
    warm call, then timed calls for about `seconds` per ubatch. Returns the
    warm call's outputs too, for the checksum."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle
    if pyoracle.ref_available():
        lib = pyoracle.load_ref()
        ref_layer = pyoracle.RefMoeLayer(lib, layer_host)
        kind, cores = "reference", int(lib.ref_worker_threads())
        isa = {1: "scalar", 8: "avx2", 16: "avx512"}[lib.ref_selected_isa_lanes()]
        run = lambda x, b: ref_layer.forward(x, b)
    else:
        lib = pyoracle.load_oracle()
        kind, cores, isa = "port", os.cpu_count() or 1, "scalar-order C"
        run = lambda x, b: pyoracle.moe_forward(lib, layer_host, x, isa=16, logit_bias=b)
    results, outputs = {}, {}
    for u, x in xs.items():
        outputs[u] = run(x, biases[u])[0]  # warm call
        n, t0 = 0, time.perf_counter()
        while True:
            run(x, biases[u])
            n += 1
            if time.perf_counter() - t0 >= seconds or n >= 2000:
                break
        dt = (time.perf_counter() - t0) / n
        results[u] = {"tokens_per_s": round(u / dt, 1), "ms_per_step": round(dt * 1e3, 3),
                      "calls": n}
        if kind == "reference":
            # the reference's per-kind kernel profile over a few more calls
            calls = max(1, min(n, 20))
            lib.ref_kernel_profiling(1)
            for _ in range(calls):
                run(x, biases[u])
            lib.ref_kernel_profiling(0)
            results[u]["kinds"] = {k: {"calls_per_step": round(c / calls, 2),
                                       "ms_per_step": round(ms / calls, 4),
                                       "work_items_per_step": int(w // calls)}
                                   for k, (c, ms, w) in pyoracle.ref_kernel_profiles(lib).items()}
    return kind, cores, isa, results, outputs


def cpu_child(args):
    """--cpu-child: the CPU baseline alone, in a process of its own (started
    with ADI_THREADS=1 for the single-thread figure; it never touches the GPU)."""
    if args.cpu_projections:
        print(json.dumps(projection_cpu_baseline(args.cpu_seconds)))
        return
    from adi_amd import synthetic as syn
    layer_host = syn.moe_layer(syn.rng_for(2, 0))
    xs, biases = {}, {}
    for u in [int(v) for v in args.ubatch.split(",")]:
        r = syn.rng_for(3 if u >= 64 else 2, u)
        xs[u] = syn.hidden_states(r, u, HIDDEN)
        biases[u] = syn.zipf_bias(r, EXPERTS) if u >= 64 else None
    kind, cores, isa, results, _ = cpu_baseline(layer_host, xs, biases, args.cpu_seconds)
    print(json.dumps({"kind": kind, "cores": cores, "isa": isa,
                      "per_ubatch": {str(k): v for k, v in results.items()}}))


def cpu_single_thread_projections(seconds):
    import subprocess
    env = dict(os.environ, ADI_THREADS="1", OMP_NUM_THREADS="1")
    cmd = [sys.executable, os.path.abspath(__file__), "--cpu-child", "--cpu-projections",
           "--cpu-seconds", str(seconds)]
    proc = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=900)
    if proc.returncode != 0:
        log(f"single-thread projection baseline failed: {proc.stderr[-400:]}")
        return None
    return json.loads(proc.stdout.strip().splitlines()[-1])


def cpu_single_thread(args):
    import subprocess
    env = dict(os.environ, ADI_THREADS="1", OMP_NUM_THREADS="1")
    cmd = [sys.executable, os.path.abspath(__file__), "--cpu-child", "--ubatch", args.ubatch,
           "--cpu-seconds", str(args.cpu_seconds / 2)]
    proc = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=600)
    if proc.returncode != 0:
        log(f"single-thread CPU baseline failed: {proc.stderr[-400:]}")
        return None
    return json.loads(proc.stdout.strip().splitlines()[-1])


def median_seconds(torch, fn, steps, runs, warm=3):
    """Median over `runs` runs of the mean time of `steps` calls of fn."""
    for _ in range(warm):
        fn(0)
    times = []
    for r in range(runs):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            fn(r * steps + i)
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) / steps)
    return float(np.median(times))


def graph_us(torch, ctx, fn, calls, replays=7):
    """Device time of one call of fn, back to back without host gaps: `calls`
    calls captured in one graph on a side stream, the median of `replays`
    replays timed with events. A Python loop issues about one small call per
    13 us, so a call shorter than that is host-bound in wall time."""
    side = torch.cuda.Stream()
    ctx.use_stream(side)
    try:
        with torch.cuda.stream(side):
            for i in range(3):  # workspaces grown before the capture
                fn(i)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            for i in range(calls):
                fn(i)
        graph.replay()
        torch.cuda.synchronize()
        times = []
        for _ in range(replays):
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            graph.replay()
            stop.record()
            torch.cuda.synchronize()
            times.append(start.elapsed_time(stop) / calls * 1e3)
        del graph
        return float(np.median(times))
    finally:
        torch.cuda.synchronize()
        ctx.use_stream(torch.cuda.current_stream())


def projection_cpu_inputs():
    """Host inputs of the CPU figures for the two packed projections: the
    151,936 x 2048 int5 head and a 2048 x 2048 NE matrix (seeded, the same
    shapes and generators as the device runs) and their input rows."""
    from adi_amd import synthetic as syn
    head = syn.head_chunk(syn.rng_for(1, 0), HEAD_ROWS, HEAD_COLUMNS)
    r = syn.rng_for(1, 1)
    ne = syn.ne_matrix(r, 2048, 2048, syn.ne_tlut(r))
    xs = {b: syn.hidden_states(syn.rng_for(1, 100 + b), b, 2048) for b in (1, 4)}
    heads_x = {b: syn.rms_normalized(x) for b, x in xs.items()}
    return head, ne, xs, heads_x


def projection_cpu_baseline(seconds):
    """mach_ne_matmul and mach_head_matmul of the reference (compiled from
    its sources, oracle/_ref; its worker pool at ADI_THREADS threads, the
    bench-ne / bench-head commands of src/main.cpp:376-461): one warm call,
    then timed calls for about `seconds` each. Returns {name: figures} or
    None without the reference library."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle
    if not pyoracle.ref_available():
        return None
    lib = pyoracle.load_ref()
    head, ne, xs, heads_x = projection_cpu_inputs()
    out = {}
    for b in (1, 4):
        for name, fn in ((f"ne_2048x2048_b{b}", lambda: pyoracle.ne_matmul(lib, ne, xs[b], prefix="ref")),
                         (f"head_151936x2048_b{b}",
                          lambda: pyoracle.head_matmul(lib, head, heads_x[b], prefix="ref"))):
            fn()  # warm call
            n, t0 = 0, time.perf_counter()
            while n < 3 or time.perf_counter() - t0 < seconds:
                fn()
                n += 1
            dt = (time.perf_counter() - t0) / n
            out[name] = {"ms_per_call": round(dt * 1e3, 4), "vectors_per_s": round(b / dt, 1),
                         "calls": n}
    return {"threads": int(lib.ref_worker_threads()),
            "isa": {1: "scalar", 8: "avx2", 16: "avx512"}[lib.ref_selected_isa_lanes()],
            "per_call": out}


def projections(torch, hip, ctx, steps, runs, cpu_seconds, only=None, graphs=True):
    from adi_amd import synthetic as syn
    res = {}
    want = lambda name: only is None or name in only
    rng = syn.rng_for(1, 0)
    copies = 3  # 3 x 204 MB heads exceed the 256 MB Infinity Cache
    heads = [hip.upload_head(ctx, syn.head_chunk(rng, HEAD_ROWS, HEAD_COLUMNS)) for _ in range(copies)]
    for batch in (1, 4):
        if not want(f"head_b{batch}"):
            syn.hidden_states(rng, batch, HEAD_COLUMNS)  # the later draws stay those of a full run
            continue
        x = ctx.to_device(syn.rms_normalized(syn.hidden_states(rng, batch, HEAD_COLUMNS)))
        out = torch.empty((batch, HEAD_ROWS), dtype=torch.float32, device="cuda")
        call = lambda i: hip.head_matmul(ctx, heads[i % copies], x, batch, out)
        dt = median_seconds(torch, call, steps, runs)
        ctx.synchronize()
        us = graph_us(torch, ctx, call, 30) if graphs else float("nan")
        key = f"head_151936x2048_b{batch}"
        res[key] = {
            "ms_per_call": round(dt * 1e3, 4), "vectors_per_s": round(batch / dt, 1),
            "packed_gbs": round(HEAD_BYTES / dt / 1e9, 1),
            "hbm_frac": round(HEAD_BYTES / dt / 1e9 / HBM_PEAK_GBS, 4),
            "graph_us_per_call": round(us, 2),
            "graph_hbm_frac": round(HEAD_BYTES / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "bytes_per_call": HEAD_BYTES,
            "rocprof_kernel": ROCPROF_NAMES["head"],
            "rocprof_avg_us": rocprof_avg_us("head", key, PROJ_STATS),
            "traffic": traffic_from_profile("head", key, PROJ_TRAFFIC)}
    del heads
    tlut = syn.ne_tlut(rng)
    book = ctx.ne_codebook(tlut)
    count = 256  # 256 x 2 MiB rotation
    base = syn.ne_matrix(rng, 2048, 2048, tlut)
    trellis = torch.randint(-32768, 32768, (count, base.trellis.size), dtype=torch.int16, device="cuda")
    su, sv = ctx.to_device(base.su), ctx.to_device(base.sv)
    mats = [hip.NeMatrix(2048, 2048, trellis[i].data_ptr(), su.data_ptr(), sv.data_ptr(),
                         base.weight_scale, book) for i in range(count)]
    nbytes = base.trellis.size * 2 + 4096
    for batch in (1, 4):
        if not want(f"ne_b{batch}"):
            continue
        x = ctx.to_device(syn.hidden_states(rng, batch, 2048))
        out = torch.empty((batch, 2048), dtype=torch.float32, device="cuda")
        call = lambda i: ctx.check(ctx.lib.adi_hip_ne_matmul(
            ctx.handle, hip.C.byref(mats[i % count]), x.data_ptr(), batch, out.data_ptr()))
        dt = median_seconds(torch, call, max(steps, count), runs)
        ctx.synchronize()
        us = graph_us(torch, ctx, call, count) if graphs else float("nan")
        key = f"ne_2048x2048_b{batch}"
        res[key] = {
            "ms_per_call": round(dt * 1e3, 4), "vectors_per_s": round(batch / dt, 1),
            "packed_gbs": round(nbytes / dt / 1e9, 1),
            "hbm_frac": round(nbytes / dt / 1e9 / HBM_PEAK_GBS, 4),
            "graph_us_per_call": round(us, 2),
            "graph_hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "bytes_per_call": nbytes,
            "rocprof_kernel": ROCPROF_NAMES["ne_fused"],
            "rocprof_avg_us": rocprof_avg_us("ne_fused", key, PROJ_STATS),
            "traffic": traffic_from_profile("ne_fused", key, PROJ_TRAFFIC)}
    del trellis, mats
    if only is not None:
        return res
    if cpu_seconds > 0:
        log("projections: cpu baseline")
        cpu = projection_cpu_baseline(cpu_seconds)
        single = cpu_single_thread_projections(cpu_seconds)
        for key, entry in res.items():
            if cpu is not None and key in cpu["per_call"]:
                entry["cpu_baseline"] = {
                    "kind": "reference", "threads": cpu["threads"], "isa": cpu["isa"],
                    **cpu["per_call"][key],
                    "single_thread": None if single is None else single["per_call"].get(key)}
    res.update(decode_side(torch, hip, ctx, steps))
    res.update(attention_side(torch, hip, ctx, steps))
    return res


def decode_side(torch, hip, ctx, steps):
    """The token side of a decode step at the checkpoint's vocabulary
    (248,320 x 2048): the embedding row of a device-resident token, the greedy
    choice, and top-p sampling (temperature 0.7, top_p 0.9) over logits shaped
    like an LM's (a few dominant tokens over a normal tail)."""
    from adi_amd import synthetic as syn
    res = {}
    vocab, hidden = 248320, 2048
    rng = syn.rng_for(4, 0)
    e = syn.embedding(rng, vocab, hidden, exceptions=20000)
    emb = hip.upload_embedding(ctx, e)
    tokens = torch.tensor(rng.integers(0, vocab, 64).astype(np.int32), device="cuda")
    out = torch.empty((64, hidden), dtype=torch.float32, device="cuda")
    logits_host = rng.normal(0.0, 2.0, (4, vocab)).astype(np.float32)
    logits_host[:, rng.integers(0, vocab, 16)] += 12.0
    logits = torch.from_numpy(logits_host).cuda()
    words = torch.tensor(rng.integers(0, 2**62, 4).astype(np.int64), device="cuda")
    picked = torch.empty(4, dtype=torch.int32, device="cuda")

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps * 1e6

    for batch in (1, 64):
        us = timed(lambda: hip.embedding_rows(ctx, emb, tokens, batch, out))
        res[f"embedding_{vocab}x{hidden}_b{batch}"] = {"us_per_call": round(us, 2)}
    for rows in (1, 4):
        us = timed(lambda: hip.argmax_rows(ctx, logits, rows, vocab, picked))
        res[f"greedy_{vocab}_rows{rows}"] = {"us_per_call": round(us, 2)}
        us = timed(lambda: hip.sample_rows(ctx, logits, rows, vocab, 0.7, 0.9, words, picked))
        res[f"top_p_{vocab}_rows{rows}"] = {"us_per_call": round(us, 2)}
    return res


def attention_side(torch, hip, ctx, steps):
    """The attention half of a decode step at hidden 2048: full GQA attention
    at history positions 255 and 4095 (KV cache resident), one Gated DeltaNet
    token, and a whole decoder layer (linear attention + the 256-expert MoE
    block)."""
    from adi_amd import synthetic as syn
    res = {}
    rng = syn.rng_for(5, 0)
    etlut, ntlut = syn.expert_tlut(rng), syn.ne_tlut(rng)
    nbook, ebook = ctx.ne_codebook(ntlut), ctx.expert_codebook(etlut)
    full = hip.upload_full_attention(ctx, syn.full_attention(rng, 2048, ntlut), nbook)
    x = torch.from_numpy(syn.rms_normalized(syn.hidden_states(rng, 1, 2048))[0]).cuda()
    out = torch.empty(2048, dtype=torch.float32, device="cuda")

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return round((time.perf_counter() - t0) / steps * 1e6, 2)

    for position in (255, 4095):
        keys = torch.randn((position + 1, 2, 256), dtype=torch.float32, device="cuda")
        values = torch.randn_like(keys)
        res[f"full_attention_2048_pos{position}"] = {"us_per_call": timed(
            lambda: hip.full_attention_forward(ctx, full, position, x, out, keys, values, position + 1))}
    linear = hip.upload_linear_attention(ctx, syn.linear_attention(rng, 2048, ntlut), nbook)
    conv = torch.zeros(8192 * 3, dtype=torch.float32, device="cuda")
    rec = torch.zeros(32 * 128 * 128, dtype=torch.float32, device="cuda")
    res["linear_attention_2048"] = {"us_per_call": timed(
        lambda: hip.linear_attention_forward(ctx, linear, x, out, conv, rec))}
    layer = hip.upload_decoder_layer(
        ctx, syn.decoder_layer(rng, False, 2048, 512, 256, etlut, ntlut), ebook, nbook)
    state, keep = hip.layer_state(False)
    hidden = x.clone().reshape(1, 2048)
    res["decoder_layer_linear_2048"] = {"us_per_call": timed(
        lambda: hip.decode_layer(ctx, layer, 0, hidden, state))}
    return res


def stack40(torch, hip, ctx, runs, sequences=16):
    """The full hybrid stack of synthetic.StackGeometry: 40 layers at hidden
    2048 (every fourth full GQA attention, the others Gated DeltaNet, each
    with the 256-expert MoE block), the 151,936-token embedding and int5 head,
    driven through the model-level entry points. One sequence: a 256-token
    prompt prefilled in chunks of 128 (adi_hip_prefill), then 64 greedy steps
    (the device's choice read back, adi_hip_decode_batch of one sequence).
    Then `sequences` sequences, each prefilled with the prompt, take 64
    greedy steps together as one decode_batch per step. The weights are drawn
    layer by layer and uploaded (about 7 GB)."""
    from adi_amd import synthetic as syn
    g = syn.StackGeometry()
    etlut, ntlut = syn.stack_codebooks()
    ebook, nbook = ctx.expert_codebook(etlut), ctx.ne_codebook(ntlut)
    layers = []
    for i in range(g.layers):
        layers.append(hip.upload_decoder_layer(ctx, syn.stack_layer(g, i, etlut, ntlut), ebook, nbook))
    emb_host, head_host, norm_host, prompt_host = syn.stack_token_side(g)
    emb, head = hip.upload_embedding(ctx, emb_host), hip.upload_head(ctx, head_host)
    final_norm = ctx.to_device(norm_host)
    del emb_host, head_host
    model = hip.Model(layers, emb, final_norm, [head])
    capacity = g.prompt + g.greedy_steps
    prompt = [int(t) for t in prompt_host]
    logits = torch.empty((sequences, g.vocab), dtype=torch.float32, device="cuda")
    chosen = torch.empty(sequences, dtype=torch.int32, device="cuda")
    seqs = [hip.Sequence(model, capacity) for _ in range(sequences)]

    def greedy(active, replay):
        """64 greedy steps; with `replay` the step is recorded once (in the
        timed region) and replayed, its tokens read from the device."""
        n = len(active)
        graph = hip.DecodeGraph(ctx, model, active, chosen[:n], logits) if replay else None
        for step in range(g.greedy_steps):
            hip.argmax_rows(ctx, logits, n, g.vocab, chosen)
            if graph is not None:
                graph.launch()
            else:
                hip.decode_batch(ctx, model, chosen[:n].tolist(), active, logits)
        torch.cuda.synchronize()
        ctx.synchronize()
        if graph is not None:
            graph.close()

    def run_one(replay=False):
        seqs[0].reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        hip.prefill(ctx, model, prompt, seqs[0], logits[0], ubatch=g.ubatch)
        torch.cuda.synchronize()
        ctx.synchronize()
        t1 = time.perf_counter()
        greedy(seqs[:1], replay)
        return t1 - t0, time.perf_counter() - t1

    def run_batch(replay=False):
        for k, s in enumerate(seqs):
            s.reset()
            hip.prefill(ctx, model, prompt, s, logits[k], ubatch=g.ubatch)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        greedy(seqs, replay)
        return time.perf_counter() - t0

    run_one()  # warm-up: workspaces, kernels
    times = [run_one() for _ in range(runs)]
    prefill_s = float(np.median([t[0] for t in times]))
    decode_s = float(np.median([t[1] for t in times]))
    run_one(True)
    decode_graph_s = float(np.median([run_one(True)[1] for _ in range(runs)]))
    run_batch()
    batch_s = float(np.median([run_batch() for _ in range(runs)]))
    run_batch(True)
    batch_graph_s = float(np.median([run_batch(True) for _ in range(runs)]))
    del layers, seqs, model
    torch.cuda.empty_cache()
    steps = g.greedy_steps
    return {"stack40": {
        "prefill_tokens_per_s": round(g.prompt / prefill_s, 1),
        "prefill_ms": round(prefill_s * 1e3, 2),
        "decode_ms_per_token": round(decode_s / steps * 1e3, 3),
        "decode_tokens_per_s": round(steps / decode_s, 1),
        "decode_replayed_ms_per_token": round(decode_graph_s / steps * 1e3, 3),
        "decode_replayed_tokens_per_s": round(steps / decode_graph_s, 1),
        f"decode_batch{sequences}_ms_per_step": round(batch_s / steps * 1e3, 3),
        f"decode_batch{sequences}_tokens_per_s": round(sequences * steps / batch_s, 1),
        f"decode_batch{sequences}_replayed_ms_per_step": round(batch_graph_s / steps * 1e3, 3),
        f"decode_batch{sequences}_replayed_tokens_per_s":
            round(sequences * steps / batch_graph_s, 1),
        "replay": "one decode step recorded as a HIP graph (adi_hip_decode_graph) per run, "
                  "the recording inside the timed region; tokens chosen on the device",
        "layers": g.layers, "hidden": g.hidden, "vocab": g.vocab, "prompt": g.prompt,
        "ubatch": g.ubatch, "greedy_steps": g.greedy_steps}}


def main():
    args = parse()
    if args.cpu_child:
        cpu_child(args)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU; sharding across GPUs is "
                          "designed but not built", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    from adi_amd import hip
    from adi_amd import synthetic as syn

    ubatches = [int(u) for u in args.ubatch.split(",")]
    ctx = hip.Context(0)
    if args.copy_bytes > 0:
        copy_calibration(torch, args.copy_bytes)
    if args.projections_only:
        only = set(args.projections_only.split(","))
        print(json.dumps({"projections": projections(torch, hip, ctx, args.steps, args.runs, 0.0, only,
                                                     graphs=not args.no_graph)}))
        ctx.close()
        return
    log("generating weights")
    rng = syn.rng_for(2, 0)
    layer_host = syn.moe_layer(rng)
    ebook = ctx.expert_codebook(layer_host.expert_tlut)
    nbook = ctx.ne_codebook(layer_host.ne_tlut)
    layers = [hip.upload_moe_layer(ctx, layer_host, ebook, nbook)]
    for i in range(1, args.layers):
        layers.append(hip.random_device_moe_layer(ctx, 1000 + i, HIDDEN, EXPERT_HIDDEN, EXPERTS,
                                                  ebook, nbook))
    torch.cuda.synchronize()
    xs_host, biases_host = {}, {}
    for u in ubatches:
        r = syn.rng_for(3 if u >= 64 else 2, u)
        xs_host[u] = [syn.hidden_states(r, u, HIDDEN) for _ in range(input_pool_size(u))]
        biases_host[u] = syn.zipf_bias(r, EXPERTS) if u >= 64 else None

    per = {}
    gpu_out = {}
    profiles = {}
    headline = None
    for u in ubatches:
        log(f"moe layer ubatch {u}")
        xs = [ctx.to_device(x) for x in xs_host[u]]
        bias = None if biases_host[u] is None else ctx.to_device(biases_host[u])
        walls, active, prof = moe_bench(torch, hip, ctx, layers, xs, [bias] * len(xs), args.steps,
                                        args.warmup, args.runs)
        wall = float(np.median(walls))
        ms = wall / args.steps * 1e3
        layer_bytes = FIXED_LAYER_BYTES + PER_EXPERT_BYTES * active
        profiles[u] = prof
        entry = {
            "tokens_per_s": round(u / (wall / args.steps), 1), "ms_per_step": round(ms, 4),
            "runs_ms_per_step": [round(w / args.steps * 1e3, 4) for w in walls],
            "active_experts": round(active, 1),
            "layer_packed_bytes": int(layer_bytes),
            "layer_hbm_frac": round(layer_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "mfma_frac_equiv": round(FLOP_PER_TOKEN * u / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 5),
            "roofline": roofline_for(prof, args.steps, active, u, ms),
            "kernels_us_per_step": {k: round(v[1] * 1e3 / args.steps, 2) for k, v in
                                    sorted(prof.items(), key=lambda kv: -kv[1][1])},
        }
        # one call of layer 0 on the first input: the checksum's GPU side
        out = torch.empty((u, HIDDEN), dtype=torch.float32, device="cuda")
        hip.moe_forward(ctx, layers[0], xs[0], u, bias, out, None, None)
        gpu_out[u] = out.cpu().numpy()
        per[str(u)] = entry
        if headline is None:
            headline = (u, entry)
        del xs

    proj = {} if args.no_projections else projections(
        torch, hip, ctx, args.steps, args.runs, 0.0 if args.no_cpu else args.projection_cpu_seconds)
    if not args.no_stack:
        log("40-layer stack")
        del layers
        torch.cuda.empty_cache()
        proj.update(stack40(torch, hip, ctx, min(args.runs, 3)))

    cpu = None
    checksum = None
    if not args.no_cpu:
        log("cpu baseline")
        kind, cores, isa, results, cpu_out = cpu_baseline(
            layer_host, {u: v[0] for u, v in xs_host.items()}, biases_host, args.cpu_seconds)
        single = cpu_single_thread(args)
        u0 = headline[0]
        cpu = {"value": results[u0]["tokens_per_s"], "unit": "tokens/s", "cores": cores,
               "kind": kind, "isa": isa, "cpu_model": cpu_model(),
               "sample": f"one MoE layer (2048 hidden, 256 experts, top-8 + shared) at ubatch "
                         f"{u0}, {results[u0]['calls']} calls after one warm call; other "
                         f"ubatches in per_ubatch",
               "per_ubatch": {str(k): v for k, v in results.items()},
               "single_thread": None if single is None else single["per_ubatch"]}
        for k, v in results.items():
            per[str(k)]["cpu_tokens_per_s"] = v["tokens_per_s"]
            per[str(k)]["kernel_profile"] = kind_report(profiles[k], args.steps, k, v.get("kinds"),
                                                        v["ms_per_step"])
        checksum = {}
        for u in ubatches:
            g, c = gpu_out[u], cpu_out[u]
            err = float(np.max(np.abs(g - c).max(axis=1) / np.abs(c).max(axis=1)))
            checksum[str(u)] = {"gpu_fnv1a": f"{fnv1a64(g.tobytes()):#018x}",
                                "cpu_fnv1a": f"{fnv1a64(c.tobytes()):#018x}",
                                "max_rel_error": float(f"{err:.3g}")}

    u0, e0 = headline
    line = {
        "metric": "MoE-layer + projection tokens/s at ubatch 1/128/512; % of HBM/MFMA peak",
        "value": e0["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "runs": args.runs,
        "ms_per_step": e0["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (seeded reference codecs: 1.5 bpw expert trellis, 4 bpw NE trellis, "
                "int5_g64 head; random-init)",
        "config": {"workload": "moe_layer", "ubatch": u0, "hidden": HIDDEN,
                   "expert_hidden": EXPERT_HIDDEN, "experts": EXPERTS, "top_k": 8,
                   "shared_experts": 1, "weight_rotation_layers": args.layers,
                   "zipf_bias_at_ubatch_ge": 64},
        "roofline": e0["roofline"],
        "cpu_baseline": cpu,
        "checksum": checksum,
        "per_ubatch": per,
        "projections": proj,
    }
    print(json.dumps(line))
    ctx.close()


if __name__ == "__main__":
    main()
