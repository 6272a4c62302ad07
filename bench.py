"""Benchmark of the MI355X Gated DeltaNet operators (one JSON line on stdout).

Headline workload (BASELINE.json configs[1] at its quoted point): one decode
step at B=64 -- state [64, 8, 128, 128] f32 read and written once.  A "step"
is one call of the decode DPS entry point.  Inputs are synthetic (numpy
default_rng, the configs[1] recipe) and resident in HBM before timing starts.
The state pairs rotate over 8 distinct (state, new_state) buffers (512 MiB,
twice the 256 MB Infinity Cache) so no step reads a state that is still cached.

Reported beside it: decode kernel time and achieved HBM bandwidth (the
roofline of the dominant kernel, from HIP events around each launch on the
launch stream), the decode batch sweep of configs[1], the prefill at 1x8192
(ms and tokens/s) and at configs[2..4] -- replaying one input set, and
cache-honestly over rotating input/output/workspace sets larger than three
Infinity Caches -- the reference's other published points (prefill of one
sequence of 64..4096 tokens, decode at B = 128 and 512) beside its B200
figures, and the CPU baseline (the reference's loops restated: in C with
OpenMP on every usable host core and on one thread, and the decode loop nest
in numpy on one thread; bounded samples).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--sweep]
"""

import argparse
import hashlib
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "gated-delta-network_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "decode µs/step + HBM GB/s at B=64; prefill tokens/s + ms at 1×8192"
HBM_PEAK_GBPS = 8000.0
# Published B200 decode latency at B=64 (reference README.md:49): 0.023 ms/step.
B200_DECODE_MS_B64 = 0.023
ROTATE = 8
# The reference's other published points on B200 (/root/reference paths):
# prefill of one sequence, tensors reused (README.md:86-87 for 1x128,
# README.md:102-107 otherwise) and in FlashInfer-Bench clone mode
# (README.md:115-120); decode device time in µs (OPTIMIZATION_LOG.md:51-57).
B200_PREFILL_REUSE_MS = {64: 0.191, 128: 0.268, 256: 0.192, 512: 0.190, 1024: 0.185,
                         2048: 0.229, 4096: 0.420}
B200_PREFILL_CLONE_MS = {64: 0.492, 256: 0.507, 512: 0.525, 1024: 0.546, 2048: 0.639,
                         4096: 0.805}
B200_DECODE_DEVICE_US = {1: 7.76, 8: 9.22, 32: 13.16, 128: 27.90, 512: 86.79}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# Every reported time is the median of TRIALS timed trials, with the min and
# max beside it (the reference's harness reports the median,
# scripts/benchmark.py:23-39).
TRIALS = 5


class Timing(tuple):
    """Per-call time over trials, in ms: (median, min, max, trials)."""

    def __new__(cls, times_ms):
        import statistics
        return super().__new__(cls, (statistics.median(times_ms), min(times_ms), max(times_ms),
                                     len(times_ms)))

    ms = property(lambda self: self[0])
    lo = property(lambda self: self[1])
    hi = property(lambda self: self[2])
    n = property(lambda self: self[3])

    def js(self, scale=1.0, digits=4):
        """{"median", "min", "max", "trials"} in ms (scale=1e3: µs)."""
        return {"median": round(self.ms * scale, digits), "min": round(self.lo * scale, digits),
                "max": round(self.hi * scale, digits), "trials": self.n}


def _event_ms(fn):
    """Milliseconds between HIP events recorded before and after fn() on
    torch's current stream (the stream every call here launches on)."""
    import torch
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    fn()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1)


def _trials(fn, calls, trials=TRIALS):
    """Timing per call of `calls` calls made by each fn(), over `trials` runs."""
    return Timing([_event_ms(fn) / calls for _ in range(trials)])


def _graph_trials(graph, calls, trials=TRIALS):
    """Timing per call of a captured graph of `calls` calls: each trial
    synchronizes, then HIP events on the replay stream bracket one replay
    (exactly `calls` calls) and it synchronizes again."""
    return _trials(graph.replay, calls, trials)


def _dev_inputs(inp, dev):
    import numpy as np
    import torch
    d = {}
    for name in ("q", "k", "v", "a", "b"):
        d[name] = torch.from_numpy(np.ascontiguousarray(inp[name])).to(dev).to(torch.bfloat16)
    for name in ("A_log", "dt_bias"):
        d[name] = torch.from_numpy(inp[name]).to(dev)
    d["state"] = None if inp["state"] is None else torch.from_numpy(inp["state"]).to(dev)
    return d


# Single workloads for `--only` (profiling): decode (batch, tokens per row)
# or prefill sequence lengths.
ONLY_WORKLOADS = {
    "decode_b64": ("decode", (64, 1)),
    "decode_b64_t4": ("decode", (64, 4)),
    "decode_b64_t16": ("decode", (64, 16)),
    "prefill_1x8192": ("prefill", [8192]),
    "prefill_4x8192": ("prefill", [8192] * 4),
    "prefill_1x1024": ("prefill", [1024]),
    "prefill_64x16": ("prefill", [16] * 64),
    "prefill_256x1": ("prefill", [1] * 256),
    "prefill_64x256": ("prefill", [256] * 64),
    "prefill_configs3": ("prefill", [6, 49, 294, 1800, 2040, 61]),
    "prefill_8x2048": ("prefill", [2048] * 8),
}


def bench_decode(B, steps, warmup, dev, variant=-1, tokens=1):
    """Times `steps` decode calls at batch B (`tokens` tokens per row; 1 is the
    plain decode step) two ways and returns (eager, graph) Timings per call.

    eager: back-to-back calls of the DPS entry point (validation, ctypes call
    and launch on the host each time).  graph: the same `steps` launches
    captured once in a HIP graph and replayed, i.e. the serving set-up in which
    the decode step is captured; its per-step time is the kernel's duration
    plus the dispatch gap between consecutive graph nodes.  Both are bracketed
    by HIP events on the launch stream.
    """
    import torch
    from gdn_amd import decode
    from oracle import gdn_oracle as O  # input recipe only

    if tokens == 1:
        inp = O.make_decode_inputs(B, seed=1)
    else:  # B sequences of `tokens` tokens, viewed as [B, T, ...]
        inp = O.make_prefill_inputs([tokens] * B, seed=1)
        for n, tail in (("q", (4, 128)), ("k", (4, 128)), ("v", (8, 128)), ("a", (8,)),
                        ("b", (8,))):
            inp[n] = inp[n].reshape((B, tokens) + tail)
    d = _dev_inputs(inp, dev)
    states = [d["state"].clone() for _ in range(ROTATE)]
    new_states = [torch.empty_like(d["state"]) for _ in range(ROTATE)]
    out = torch.empty((B, tokens, 8, 128), dtype=torch.bfloat16, device=dev)
    args = (d["q"], d["k"], d["v"])
    tail = (d["A_log"], d["a"], d["dt_bias"], d["b"], inp["scale"], out)

    def step(i):
        decode.kernel(*args, states[i % ROTATE], *tail, new_states[i % ROTATE], variant=variant)

    for i in range(warmup):
        step(i)
    eager = _trials(lambda: [step(i) for i in range(steps)], steps)

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        step(0)
    torch.cuda.current_stream(dev).wait_stream(side)
    with torch.cuda.graph(graph):
        for i in range(steps):
            step(i)
    graph.replay()
    return eager, _graph_trials(graph, steps)


def bench_prefill(lens, steps, warmup, dev, variant=-1, slow_decay_heads=None):
    """Times `steps` prefill calls on a packed batch with sequence lengths
    `lens` (the configs[2..4] recipe, zero initial state for one sequence)
    and returns (eager, graph) Timings per call."""
    import numpy as np
    import torch
    from gdn_amd import prefill
    from oracle import gdn_oracle as O  # input recipe only

    kw = {} if slow_decay_heads is None else {"slow_decay_heads": slow_decay_heads}
    inp = O.make_prefill_inputs(lens, seed=2, with_state=len(lens) > 1, **kw)
    d = _dev_inputs(inp, dev)
    cu = torch.from_numpy(inp["cu_seqlens"]).to(dev)
    T, N = sum(lens), len(lens)
    out = torch.empty((T, 8, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((N, 8, 128, 128), dtype=torch.float32, device=dev)

    def step():
        prefill.kernel(d["q"], d["k"], d["v"], d["state"], d["A_log"], d["a"], d["dt_bias"],
                       d["b"], cu, inp["scale"], out, ns, variant=variant)

    for _ in range(warmup):
        step()
    eager = _trials(lambda: [step() for _ in range(steps)], steps)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream(dev).wait_stream(side)
    with torch.cuda.graph(graph):
        for _ in range(steps):
            step()
    graph.replay()
    return eager, _graph_trials(graph, steps)


def bench_prefill_rotated(lens, dev, min_bytes=768 << 20, steps=None):
    """Cache-honest prefill time: `steps` calls captured in one HIP graph that
    cycle over S distinct sets of inputs, outputs and workspace, S chosen so
    that the sets together exceed `min_bytes` (three times the 256 MB Infinity
    Cache), so no call finds its operands left in the MALL by the previous
    call on the same set.  Returns (Timing per call, S, bytes per set)."""
    import torch
    from gdn_amd import prefill
    from oracle import gdn_oracle as O  # input recipe only

    inp = O.make_prefill_inputs(lens, seed=2, with_state=len(lens) > 1)
    base = _dev_inputs(inp, dev)
    base["cu_seqlens"] = torch.from_numpy(inp["cu_seqlens"]).to(dev)
    T, N = sum(lens), len(lens)
    per_set = (sum(t.numel() * t.element_size() for t in base.values() if t is not None)
               + T * 8 * 128 * 2 + N * 8 * 128 * 128 * 4 + prefill.workspace_bytes(T, N))
    S = max(3, -(-min_bytes // per_set))
    steps = steps or max(2 * S, 20)
    sets = []
    for _ in range(S):
        c = {n: (None if t is None else t.clone()) for n, t in base.items()}
        c["out"] = torch.empty((T, 8, 128), dtype=torch.bfloat16, device=dev)
        c["ns"] = torch.empty((N, 8, 128, 128), dtype=torch.float32, device=dev)
        c["ws"] = prefill.alloc_workspace(T, N, dev)
        sets.append(c)

    def step(i):
        c = sets[i % S]
        prefill.kernel(c["q"], c["k"], c["v"], c["state"], c["A_log"], c["a"], c["dt_bias"],
                       c["b"], c["cu_seqlens"], inp["scale"], c["out"], c["ns"], workspace=c["ws"])

    for i in range(S):
        step(i)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        step(0)
    torch.cuda.current_stream(dev).wait_stream(side)
    with torch.cuda.graph(graph):
        for i in range(steps):
            step(i)
    graph.replay()
    timing = _graph_trials(graph, steps)
    del graph, sets
    torch.cuda.empty_cache()
    return timing, S, per_set


def bench_prefill_clone(lens, reps, dev):
    """FlashInfer-Bench's clone mode (OPTIMIZATION_LOG.md:263-300): before each
    timed call every argument is cloned into fresh memory and the device is
    idle; the timed region is one DPS call from the host (validation, ctypes,
    launches) to the end of its last kernel.  Returns the Timing over the
    `reps` calls after three untimed ones."""
    import torch
    from gdn_amd import prefill
    from oracle import gdn_oracle as O  # input recipe only

    inp = O.make_prefill_inputs(lens, seed=2, with_state=len(lens) > 1)
    d = _dev_inputs(inp, dev)
    d["cu_seqlens"] = torch.from_numpy(inp["cu_seqlens"]).to(dev)
    T, N = sum(lens), len(lens)
    names = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")
    times = []
    for i in range(reps + 3):
        c = {n: (None if d[n] is None else d[n].clone()) for n in names}
        out = torch.empty((T, 8, 128), dtype=torch.bfloat16, device=dev)
        ns = torch.empty((N, 8, 128, 128), dtype=torch.float32, device=dev)
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record()
        prefill.kernel(*(c[n] for n in names), inp["scale"], out, ns)
        t1.record()
        torch.cuda.synchronize()
        if i >= 3:
            times.append(t0.elapsed_time(t1))
    return Timing(times)


def bench_copy(nbytes, steps, warmup, dev):
    """The streaming ceiling of the decode step: `steps` calls of the library's
    gdn_stream_copy (the decode kernel's access pattern, nbytes read and
    nbytes written per call) over 8 rotating buffer pairs, captured in a HIP
    graph as bench_decode's steps are; returns the Timing per call."""
    import torch
    from gdn_amd import _lib
    from gdn_amd._common import stream_of

    lib = _lib.load()
    srcs = [torch.ones(nbytes // 4, dtype=torch.float32, device=dev) for _ in range(ROTATE)]
    dsts = [torch.empty_like(srcs[0]) for _ in range(ROTATE)]

    def step(i):
        rc = lib.gdn_stream_copy(srcs[i % ROTATE].data_ptr(), dsts[i % ROTATE].data_ptr(), nbytes,
                                 stream_of(dev))
        _lib.check(rc, "gdn_stream_copy")

    for i in range(warmup):
        step(i)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        step(0)
    torch.cuda.current_stream(dev).wait_stream(side)
    with torch.cuda.graph(graph):
        for i in range(steps):
            step(i)
    graph.replay()
    return _graph_trials(graph, steps)


KERNEL_SOURCE_DIRS = ("gated-delta-network_amd/csrc", "include")


def kernel_sources_sha16(root=ROOT):
    """The first 16 hex digits of a SHA-256 over the kernel and C-ABI sources
    (the .hip, .h and .cpp files and the Makefile of the directories above,
    by name).  The committed counter summaries name the value they were
    measured on ("kernel_sources_sha16: ..."), so that a summary left behind
    by a kernel change is not read as current."""
    h = hashlib.sha256()
    for d in KERNEL_SOURCE_DIRS:
        base = os.path.join(root, d)
        for name in sorted(os.listdir(base)):
            path = os.path.join(base, name)
            if os.path.isfile(path) and (name.endswith((".hip", ".h", ".cpp")) or name == "Makefile"):
                h.update(f"{d}/{name}\0".encode())
                with open(path, "rb") as f:
                    h.update(f.read())
    return h.hexdigest()[:16]


def _current_summary_lines(path, sources=None):
    """The lines of a committed counter summary, or None when it is absent
    or was measured on other kernel sources than the tree's."""
    try:
        with open(path) as f:
            lines = f.readlines()
    except OSError:
        return None
    stamp = [ln.split(":", 1)[1].strip() for ln in lines if ln.startswith("kernel_sources_sha16:")]
    if not stamp or stamp[0] != (sources or kernel_sources_sha16()):
        return None
    return lines


def measured_traffic(path=os.path.join(ROOT, "profiles", "decode_b64_hbm_traffic.md"), sources=None):
    """HBM bytes per decode launch at B=64 from the committed rocprofv3 PMC
    summary (FETCH_SIZE + WRITE_SIZE, scaled by a plain copy of known size);
    None when the summary is absent or stale (other kernel sources)."""
    for line in _current_summary_lines(path, sources) or ():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1])
    return None


def measured_mfma(path=os.path.join(ROOT, "profiles", "prefill_mfma_counters.md"), sources=None):
    """The prefill kernels' MFMA counters from the committed rocprofv3 PMC
    summary: lines "mfma_util.<workload>.<kernel>: <fraction of time the
    matrix cores are busy>" and "mfma_executed_over_algorithmic.<workload>:
    <ratio>", keyed by the line's name; None when the summary is absent or
    stale (other kernel sources)."""
    out = {}
    for line in _current_summary_lines(path, sources) or ():
        if line.startswith(("mfma_util.", "mfma_executed_over_algorithmic.")):
            key, val = line.split(":", 1)
            out[key.strip()] = float(val)
    return out or None


def host_cores():
    """The host CPUs this process may use: os.cpu_count(), the affinity mask,
    and the OpenMP share the box grants (OMP_NUM_THREADS, when set)."""
    aff = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    usable = min(aff, int(omp)) if omp.isdigit() and int(omp) > 0 else aff
    return {"cpu_count": os.cpu_count(), "affinity": aff,
            "omp_num_threads": int(omp) if omp.isdigit() else None, "used": usable}


def _repeat(fn, seconds):
    reps = 0
    t = time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t
        if el >= seconds:
            return el / reps, reps


def cpu_baseline_decode_loop(B, seconds):
    """The reference's decode loop nest (gdn_decode_ref.py:63-80) restated in
    numpy (oracle decode_loop), one thread, repeated for `seconds`; returns
    (seconds per step, steps)."""
    from threadpoolctl import threadpool_limits
    from oracle import gdn_oracle as O

    inp = O.make_decode_inputs(B, seed=1)
    with threadpool_limits(limits=1):
        return _repeat(lambda: O.decode_loop(**inp), seconds)


def cpu_baseline_decode_c(B, threads, seconds):
    """One decode step at batch B as B one-token sequences through the C
    recurrence (oracle/gdn_seq.c, the reference's per-token loop in f32),
    OpenMP over the B x 8 (row, v-head) pairs on `threads` threads, repeated
    for `seconds`; returns (seconds per step, steps)."""
    import numpy as np
    from oracle import gdn_oracle as O

    inp = O.make_decode_inputs(B, seed=1)
    pre = dict(q=inp["q"][:, 0], k=inp["k"][:, 0], v=inp["v"][:, 0], state=inp["state"],
               A_log=inp["A_log"], a=inp["a"][:, 0], dt_bias=inp["dt_bias"], b=inp["b"][:, 0],
               cu_seqlens=np.arange(B + 1, dtype=np.int64), scale=inp["scale"])
    O.set_c_threads(threads)
    try:
        return _repeat(lambda: O.prefill_seq_c(**pre), seconds)
    finally:
        O.set_c_threads(0)


def cpu_baseline_prefill(lens, threads, seconds=0.0):
    """Prefill of `lens` through the C recurrence (the reference's per-token
    loop, f32), OpenMP over the (sequence, v-head) pairs on `threads` threads;
    at least one call, repeated for `seconds`; returns (seconds per call,
    calls)."""
    from oracle import gdn_oracle as O

    inp = O.make_prefill_inputs(lens, seed=2, with_state=len(lens) > 1)
    O.set_c_threads(threads)
    try:
        return _repeat(lambda: O.prefill_seq_c(**inp), seconds)
    finally:
        O.set_c_threads(0)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--variant", type=int, default=-1, help="decode tiling (-1 = built-in)")
    ap.add_argument("--sweep", action="store_true",
                    help="also time every decode batch size of configs[1] and every tiling")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", choices=sorted(ONLY_WORKLOADS),
                    help="profiling mode: time only this workload (eager and graph) and "
                         "print one line; for rocprofv3 summaries of single workloads")
    ap.add_argument("--rotated", action="store_true",
                    help="with --only and a prefill workload: time the calls over rotating "
                         "sets of inputs, outputs and workspace (cache-cold, as "
                         "prefill_ms_*_rotated) instead of one set")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 64 MiB device copy 10 times (the known-size "
                         "reference for rocprofv3 FETCH_SIZE / WRITE_SIZE scaling)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus}: this build measures one GPU only (the operators "
              "are per-GPU shards: decode splits over batch rows or heads and prefill over "
              "sequences or heads, with no cross-GPU exchange).", file=sys.stderr)
        sys.exit(2)

    import torch
    from oracle import gdn_oracle as O

    dev = torch.device("cuda", 0)
    if args.calibrate_copy:
        nbytes = 64 << 20
        src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": nbytes, "copies": 10}), flush=True)
        return
    log(f"device: {torch.cuda.get_device_name(dev)}")
    B = args.batch
    if args.only:
        kind, arg = ONLY_WORKLOADS[args.only]
        if kind == "decode":
            te, tg = bench_decode(arg[0], args.steps, args.warmup, dev, tokens=arg[1])
        elif args.rotated:
            tg, sets, per_set = bench_prefill_rotated(arg, dev)
            log(f"{args.only}: graph {tg.ms * 1e3:.2f} us per call over {sets} rotating sets of "
                f"{per_set / 2**20:.1f} MiB (median of {tg.n}; min {tg.lo * 1e3:.2f}, "
                f"max {tg.hi * 1e3:.2f})")
            return
        else:
            te, tg = bench_prefill(arg, args.steps, args.warmup, dev)
        log(f"{args.only}: eager {te.ms * 1e3:.2f} us, graph {tg.ms * 1e3:.2f} us per call "
            f"(median of {tg.n}; graph min {tg.lo * 1e3:.2f}, max {tg.hi * 1e3:.2f})")
        return

    if args.sweep:
        for b in (1, 2, 4, 8, 16, 32, 48, 64):
            for var in [-1] + list(range(10)) + [16 + i for i in range(10)]:
                te, tg = bench_decode(b, args.steps, args.warmup, dev, var)
                gbs = O.decode_bytes(b) / (tg.ms * 1e-3) / 1e9
                log(f"sweep decode B={b:3d} variant={var:3d}: eager {te.ms * 1e3:8.2f} us/step, "
                    f"graph {tg.ms * 1e3:8.2f} us/step, {gbs:8.1f} GB/s")

    # The headline: one decode step at B, K steps per graph replay, the median
    # of TRIALS replays.
    eager, graph = bench_decode(B, args.steps, args.warmup, dev, args.variant)
    ms_step = graph.ms
    nbytes = O.decode_bytes(B)
    gbs = lambda ms: nbytes / (ms * 1e-3) / 1e9
    gbs_step = gbs(ms_step)
    log(f"decode B={B}: graph {ms_step * 1e3:.2f} us/step median of {graph.n} "
        f"(min {graph.lo * 1e3:.2f}, max {graph.hi * 1e3:.2f}; {gbs_step:.1f} GB/s, "
        f"{gbs_step / HBM_PEAK_GBPS:.1%} of peak); eager {eager.ms * 1e3:.2f} us/step")
    state_bytes = B * 8 * 128 * 128 * 4
    copy = bench_copy(state_bytes, args.steps, args.warmup, dev)
    copy_gbs = 2 * state_bytes / (copy.ms * 1e-3) / 1e9
    log(f"copy of the decode state (read + write {2 * state_bytes >> 20} MiB, the decode "
        f"kernel's access pattern): {copy.ms * 1e3:.2f} us/call ({copy_gbs:.1f} GB/s); decode "
        f"step / copy = {ms_step / copy.ms:.3f}")

    if args.sweep:
        for lens in ([1024], [6, 49, 294, 1800, 2040, 61], [8192], [8192] * 4, [64], [256]):
            for var in (-1, 0, 1):
                pe, pg = bench_prefill(lens, max(5, args.steps // 10), 3, dev, var)
                T = sum(lens)
                log(f"sweep prefill lens={lens if len(lens) < 5 else f'{len(lens)}x{lens[0]}'} "
                    f"variant={var}: eager {pe.ms:.3f} ms, graph {pg.ms:.3f} ms, "
                    f"{T / (pg.ms * 1e-3) / 1e6:.2f} M tok/s")

    pre_lens = [8192]
    pre_eager, pre = bench_prefill(pre_lens, max(10, args.steps // 10), 3, dev)
    pre_ms = pre.ms
    T8 = sum(pre_lens)
    nt8 = sum(-(-L // 64) for L in pre_lens)
    pre_tflops = O.prefill_flops(nt8) / (pre_ms * 1e-3) / 1e12
    pre_gbs = O.prefill_bytes(T8, len(pre_lens)) / (pre_ms * 1e-3) / 1e9
    log(f"prefill 1x8192: graph {pre_ms:.4f} ms median (min {pre.lo:.4f}, max {pre.hi:.4f}; "
        f"{T8 / (pre_ms * 1e-3) / 1e6:.2f} M tok/s, {pre_tflops:.1f} TFLOP/s, {pre_gbs:.0f} GB/s); "
        f"eager {pre_eager.ms:.4f} ms")

    pre_clone = bench_prefill_clone(pre_lens, 20, dev)
    pre1k_eager, pre1k = bench_prefill([1024], max(10, args.steps // 10), 3, dev)
    pre1k_clone = bench_prefill_clone([1024], 20, dev)
    log(f"prefill clone mode: 1x8192 {pre_clone.ms:.3f} ms, 1x1024 {pre1k_clone.ms:.3f} ms; "
        f"1x1024 graph {pre1k.ms:.3f} ms, eager {pre1k_eager.ms:.3f} ms")
    rotated = {}
    for name, lens in (("1x8192", pre_lens), ("1x1024", [1024])):
        t, sets, per_set = bench_prefill_rotated(lens, dev)
        rotated[name] = {"ms": t.js(), "sets": sets, "bytes_per_set": per_set}
    log(f"prefill over rotating input/output/workspace sets (> 768 MiB in all): {rotated}")

    # The reference's other published points: prefill of one sequence of
    # 64..4096 tokens (graph replay, eager calls with tensors reused, clone
    # mode) and decode at B = 128 and 512 (graph replay, 8 rotating states).
    ref_points = {"prefill": {}, "decode": {}}
    for L in (64, 128, 256, 512, 1024, 2048, 4096):
        pe, pg = bench_prefill([L], 20, 3, dev)
        pc = bench_prefill_clone([L], 10, dev)
        ref_points["prefill"][f"1x{L}"] = {
            "graph_ms": pg.js(), "eager_ms": pe.js(), "clone_ms": pc.js(),
            "b200_reuse_ms": B200_PREFILL_REUSE_MS.get(L),
            "b200_clone_ms": B200_PREFILL_CLONE_MS.get(L)}
    for b in (128, 512):
        te, tg = bench_decode(b, 50, 5, dev)
        ref_points["decode"][f"B{b}"] = {
            "us": tg.js(1e3, 3), "us_eager": te.js(1e3, 3),
            "GBps": round(O.decode_bytes(b) / (tg.ms * 1e-3) / 1e9, 1),
            "b200_device_us": B200_DECODE_DEVICE_US[b]}
    log(f"reference points: {ref_points}")

    mtp = {}
    for T in (2, 4, 8, 16):
        _, tg = bench_decode(64, 50, 5, dev, tokens=T)
        mtp[f"B64_T{T}"] = tg.js(1e3, 2)
    log(f"multi-token decode B=64 (us per call): {mtp}")
    # Short batches: one input set replayed (warm in the Infinity Cache, as
    # the other single-set lines) and over rotating sets (cache-cold, as a
    # serving loop meets each request's state).
    short, short_rot = {}, {}
    for name, lens in (("256x1", [1] * 256), ("64x16", [16] * 64), ("1x64", [64]),
                       ("32x64", [64] * 32), ("64x256", [256] * 64)):
        _, pg = bench_prefill(lens, 20, 3, dev)
        short[name] = pg.js()
        if len(lens) > 1:  # (one 64-token sequence would need ~1000 sets)
            short_rot[name] = bench_prefill_rotated(lens, dev)[0].js()
    log(f"short-sequence prefill (ms per call): {short}, over rotating sets {short_rot}")

    # the decode batch sweep (one step in graph replay per B), and
    # the prefill configurations configs[3] and configs[4] (configs[2] is
    # the 1x1024 line above); the 4x8192 recipe skews heads 6-7 to near-unit
    # decay.
    sweep = {}
    for b in (1, 2, 4, 8, 16, 32, 48, 64):
        _, tg = bench_decode(b, 100, 10, dev)
        sweep[f"B{b}"] = {"us": tg.js(1e3, 3),
                          "GBps": round(O.decode_bytes(b) / (tg.ms * 1e-3) / 1e9, 1)}
    log(f"decode sweep (graph us/step, GB/s): {sweep}")
    cfg_detail = {}

    def detail(lens, t):
        T, N = sum(lens), len(lens)
        nt = sum(-(-L // 64) for L in lens)
        tflops = O.prefill_flops(nt) / (t.ms * 1e-3) / 1e12
        return {"ms": t.js(), "tokens_per_s": round(T / (t.ms * 1e-3), 1),
                "tflops": round(tflops, 2), "mfma_frac": round(tflops / 2500.0, 5),
                "hbm_gbps": round(O.prefill_bytes(T, N) / (t.ms * 1e-3) / 1e9, 1)}

    for name, lens, kw in (("configs3_varlen6", [6, 49, 294, 1800, 2040, 61], {}),
                           ("configs4_4x8192", [8192] * 4, {"slow_decay_heads": (6, 7)})):
        _, pg = bench_prefill(lens, 10, 2, dev, **kw)
        cfg_detail[name] = detail(lens, pg)
    cfg_detail["configs2_1x1024"] = detail([1024], pre1k)
    cfg_detail["north_star_1x8192"] = detail(pre_lens, pre)
    log(f"prefill configs: {cfg_detail}")

    # CPU baseline (the reference's loops restated; a reported baseline, not a
    # target): about --cpu-seconds of CPU work in all.
    hc = host_cores()
    slice_s = args.cpu_seconds / 4
    cpu_all_s, reps_all = cpu_baseline_decode_c(B, hc["used"], slice_s)
    cpu_one_s, reps_one = cpu_baseline_decode_c(B, 1, slice_s)
    cpu_loop_s, reps_loop = cpu_baseline_decode_loop(B, slice_s)
    log(f"cpu baseline decode B={B}: C recurrence {cpu_all_s * 1e3:.1f} ms/step on "
        f"{hc['used']} threads, {cpu_one_s * 1e3:.1f} ms/step on 1; numpy loop nest "
        f"{cpu_loop_s * 1e3:.1f} ms/step ({hc})")
    cpu_pre_all, _ = cpu_baseline_prefill(pre_lens, hc["used"], slice_s / 2)
    cpu_pre_one, _ = cpu_baseline_prefill(pre_lens, 1)
    cpu_pre4_all, _ = cpu_baseline_prefill([8192] * 4, hc["used"])
    log(f"cpu baseline prefill 1x8192: {cpu_pre_all:.3f} s on {min(hc['used'], 8)} threads, "
        f"{cpu_pre_one:.3f} s on 1; 4x8192 {cpu_pre4_all:.3f} s on {min(hc['used'], 32)}")

    b200_gbs = O.decode_bytes(64) / (B200_DECODE_MS_B64 * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(gbs_step, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(gbs_step / b200_gbs, 4) if B == 64 else None,
        "dtype": "f32",
        "data": "synthetic: numpy default_rng(seed=1), configs[1] recipe; 8 rotating state buffers",
        "config": {"workload": f"decode step, B={B} (configs[1]), k-last f32 state",
                   "batch": B, "heads_qk": 4, "heads_v": 8, "head_dim": 128},
        "statistic": f"median of {graph.n} HIP-graph replays of the {args.steps} steps; "
                     "every other time in this line: median, min and max of its trials",
        "decode_us_per_step": graph.js(1e3, 3),
        "decode_GBps_min_max": [round(gbs(graph.hi), 1), round(gbs(graph.lo), 1)],
        "decode_us_per_step_eager": eager.js(1e3, 3),
        "decode_copy_ceiling": {"us": copy.js(1e3, 3), "GBps": round(copy_gbs, 1),
                                "bytes_moved": 2 * state_bytes,
                                "decode_time_over_copy": round(ms_step / copy.ms, 4)},
        "prefill_ms_1x8192": round(pre_ms, 4),
        "prefill_ms_1x8192_trials": pre.js(),
        "prefill_ms_1x8192_eager": pre_eager.js(),
        "prefill_tokens_per_s": round(T8 / (pre_ms * 1e-3), 1),
        "prefill_ms_1x8192_clone": pre_clone.js(),
        "prefill_ms_1x1024": pre1k.js(),
        "prefill_ms_1x1024_clone": pre1k_clone.js(),
        "prefill_ms_1x8192_rotated": rotated["1x8192"]["ms"],
        "prefill_ms_1x1024_rotated": rotated["1x1024"]["ms"],
        "prefill_rotated_sets": rotated,
        "reference_points": ref_points,
        "decode_sweep": sweep,
        "prefill_configs": cfg_detail,
        "decode_multi_token_us": mtp,
        "prefill_ms_short_batches": short,
        "prefill_ms_short_batches_rotated": short_rot,
        "prefill_roofline": {"bound": "mfma", "achieved": round(pre_tflops, 2), "peak": 2500.0,
                             "unit": "TFLOP/s", "frac": round(pre_tflops / 2500.0, 5),
                             "hbm_gbs": round(pre_gbs, 1),
                             "flops_per_call": O.prefill_flops(nt8),
                             "bytes_per_call": O.prefill_bytes(T8, len(pre_lens)),
                             "counters": measured_mfma()},
        "roofline": {"bound": "hbm", "achieved": round(gbs_step, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gbs_step / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic() if (B == 64 and args.variant == -1) else None,
                     "traffic_source": "profiles/decode_b64_hbm_traffic.md (rocprofv3 PMC; "
                                       "null when measured on other kernel sources than "
                                       f"these, sha16 {kernel_sources_sha16()})",
                     "kernel": "gdn::decode_kernel",
                     "bytes_per_launch": nbytes},
        "cpu_baseline": {
            "value": round(nbytes / cpu_all_s / 1e9, 4), "unit": "GB/s", "cores": hc["used"],
            "kind": "port",
            "sample": f"{reps_all} decode steps at B={B} ({cpu_all_s * 1e3:.2f} ms/step): the "
                      f"reference's per-token loop in C (oracle/gdn_seq.c, f32), OpenMP over "
                      f"the {B * 8} (row, v-head) pairs on {hc['used']} threads of {cpu_model()}",
            "one_thread": {"value": round(nbytes / cpu_one_s / 1e9, 4), "unit": "GB/s",
                           "ms_per_step": round(cpu_one_s * 1e3, 3), "steps": reps_one},
            "numpy_loop_one_thread": {
                "value": round(nbytes / cpu_loop_s / 1e9, 4), "unit": "GB/s",
                "ms_per_step": round(cpu_loop_s * 1e3, 3), "steps": reps_loop,
                "what": "oracle decode_loop: gdn_decode_ref.py:63-80's loop nest in numpy"},
            "host_cores": hc, "cpu_model": cpu_model()},
        "cpu_baseline_prefill": {
            "value": round(T8 / cpu_pre_all, 1), "unit": "tokens/s", "cores": min(hc["used"], 8),
            "kind": "port",
            "sample": f"1x8192 prefill in {cpu_pre_all:.3f} s: the reference's per-token loop "
                      f"in C (oracle/gdn_seq.c, f32), OpenMP over the 8 v-heads (the "
                      f"parallelism one sequence has) of {cpu_model()}",
            "one_thread": {"value": round(T8 / cpu_pre_one, 1), "unit": "tokens/s",
                           "seconds": round(cpu_pre_one, 3)},
            "configs4_4x8192_all_cores": {"value": round(4 * 8192 / cpu_pre4_all, 1),
                                          "unit": "tokens/s", "cores": min(hc["used"], 32),
                                          "seconds": round(cpu_pre4_all, 3)},
            "host_cores": hc, "cpu_model": cpu_model()},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
