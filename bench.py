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
(ms and tokens/s) and at configs[2..4], and the CPU baseline (the reference's
loop nest restated in numpy, oracle/gdn_oracle.py:decode_loop, single thread,
on a bounded sample).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--sweep]
"""

import argparse
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


def log(msg):
    print(msg, file=sys.stderr, flush=True)


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
    "prefill_64x256": ("prefill", [256] * 64),
    "prefill_configs3": ("prefill", [6, 49, 294, 1800, 2040, 61]),
    "prefill_8x2048": ("prefill", [2048] * 8),
}


def bench_decode(B, steps, warmup, dev, variant=-1, tokens=1):
    """Times `steps` decode calls at batch B (`tokens` tokens per row; 1 is the
    plain decode step) two ways and returns (eager ms/call, graph ms/call).

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

    def timed(fn):
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record()
        fn()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1)

    for i in range(warmup):
        step(i)
    ms_eager = timed(lambda: [step(i) for i in range(steps)]) / steps

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
    ms_graph = min(timed(graph.replay) for _ in range(3)) / steps
    return ms_eager, ms_graph


def bench_prefill(lens, steps, warmup, dev, variant=-1, slow_decay_heads=None):
    """Times `steps` prefill calls on a packed batch with sequence lengths
    `lens` (the configs[2..4] recipe, zero initial state for one sequence)
    and returns (eager ms/call, graph ms/call)."""
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

    def timed(fn):
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record()
        fn()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1)

    for _ in range(warmup):
        step()
    ms_eager = timed(lambda: [step() for _ in range(steps)]) / steps
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
    ms_graph = min(timed(graph.replay) for _ in range(3)) / steps
    return ms_eager, ms_graph


def bench_prefill_clone(lens, reps, dev):
    """FlashInfer-Bench's clone mode (OPTIMIZATION_LOG.md:263-300): before each
    timed call every argument is cloned into fresh memory and the device is
    idle; the timed region is one DPS call from the host (validation, ctypes,
    launches) to the end of its last kernel.  Returns the median ms/call."""
    import statistics
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
    return statistics.median(times)


def bench_copy(nbytes, steps, warmup, dev):
    """The streaming ceiling of the decode step: `steps` calls of the library's
    gdn_stream_copy (the decode kernel's access pattern, nbytes read and
    nbytes written per call) over 8 rotating buffer pairs, captured in a HIP
    graph as bench_decode's steps are; returns ms per call."""
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
    best = None
    for _ in range(3):
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record()
        graph.replay()
        t1.record()
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / steps
        best = ms if best is None else min(best, ms)
    return best


def measured_traffic(path=os.path.join(ROOT, "profiles", "decode_b64_hbm_traffic.md")):
    """HBM bytes per decode launch at B=64 from the committed rocprofv3 PMC
    summary (FETCH_SIZE + WRITE_SIZE, scaled by a plain copy of known size);
    None when the summary is absent."""
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_baseline_decode(B, seconds):
    """The reference's decode loop nest restated in numpy (oracle decode_loop),
    one thread, repeated until `seconds` of CPU time have passed."""
    from threadpoolctl import threadpool_limits
    from oracle import gdn_oracle as O

    inp = O.make_decode_inputs(B, seed=1)
    reps = 0
    with threadpool_limits(limits=1):
        t = time.perf_counter()
        while True:
            O.decode_loop(**inp)
            reps += 1
            el = time.perf_counter() - t
            if el >= seconds:
                break
    return el / reps, reps


def cpu_baseline_prefill(lens):
    """One prefill of `lens` through the sequential recurrence restated in C
    (oracle/gdn_seq.c: the reference's per-token loop, f32, one OpenMP thread
    per (sequence, v-head) pair); returns (seconds, threads used)."""
    from oracle import gdn_oracle as O

    inp = O.make_prefill_inputs(lens, seed=2, with_state=len(lens) > 1)
    threads = min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "64")),
                  len(lens) * 8)
    t = time.perf_counter()
    O.prefill_seq_c(**inp)
    return time.perf_counter() - t, threads


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
            me, mg = bench_decode(arg[0], args.steps, args.warmup, dev, tokens=arg[1])
        else:
            me, mg = bench_prefill(arg, args.steps, args.warmup, dev)
        log(f"{args.only}: eager {me * 1e3:.2f} us, graph {mg * 1e3:.2f} us per call")
        return

    if args.sweep:
        for b in (1, 2, 4, 8, 16, 32, 48, 64):
            for var in [-1] + list(range(10)) + [16 + i for i in range(10)]:
                me, mg = bench_decode(b, args.steps, args.warmup, dev, var)
                gbs = O.decode_bytes(b) / (mg * 1e-3) / 1e9
                log(f"sweep decode B={b:3d} variant={var:3d}: eager {me * 1e3:8.2f} us/step, "
                    f"graph {mg * 1e3:8.2f} us/step, {gbs:8.1f} GB/s")

    ms_eager, ms_step = bench_decode(B, args.steps, args.warmup, dev, args.variant)
    nbytes = O.decode_bytes(B)
    gbs_step = nbytes / (ms_step * 1e-3) / 1e9
    log(f"decode B={B}: graph {ms_step * 1e3:.2f} us/step ({gbs_step:.1f} GB/s, "
        f"{gbs_step / HBM_PEAK_GBPS:.1%} of peak); eager {ms_eager * 1e3:.2f} us/step")
    state_bytes = B * 8 * 128 * 128 * 4
    copy_ms = bench_copy(state_bytes, args.steps, args.warmup, dev)
    copy_gbs = 2 * state_bytes / (copy_ms * 1e-3) / 1e9
    log(f"copy of the decode state (read + write {2 * state_bytes >> 20} MiB, the decode "
        f"kernel's access pattern): {copy_ms * 1e3:.2f} us/call ({copy_gbs:.1f} GB/s); decode "
        f"step / copy = {ms_step / copy_ms:.3f}")

    if args.sweep:
        for lens in ([1024], [6, 49, 294, 1800, 2040, 61], [8192], [8192] * 4, [64], [256]):
            for var in (-1, 0, 1):
                pe, pg = bench_prefill(lens, max(5, args.steps // 10), 3, dev, var)
                T = sum(lens)
                log(f"sweep prefill lens={lens if len(lens) < 5 else f'{len(lens)}x{lens[0]}'} "
                    f"variant={var}: eager {pe:.3f} ms, graph {pg:.3f} ms, "
                    f"{T / (pg * 1e-3) / 1e6:.2f} M tok/s")

    pre_lens = [8192]
    pre_eager, pre_ms = bench_prefill(pre_lens, max(10, args.steps // 10), 3, dev)
    T8 = sum(pre_lens)
    nt8 = sum(-(-L // 64) for L in pre_lens)
    pre_tflops = O.prefill_flops(nt8) / (pre_ms * 1e-3) / 1e12
    pre_gbs = O.prefill_bytes(T8, len(pre_lens)) / (pre_ms * 1e-3) / 1e9
    log(f"prefill 1x8192: graph {pre_ms:.3f} ms ({T8 / (pre_ms * 1e-3) / 1e6:.2f} M tok/s, "
        f"{pre_tflops:.1f} TFLOP/s, {pre_gbs:.0f} GB/s); eager {pre_eager:.3f} ms")

    pre_clone = bench_prefill_clone(pre_lens, 20, dev)
    pre1k_eager, pre1k_ms = bench_prefill([1024], max(10, args.steps // 10), 3, dev)
    pre1k_clone = bench_prefill_clone([1024], 20, dev)
    log(f"prefill clone mode: 1x8192 {pre_clone:.3f} ms, 1x1024 {pre1k_clone:.3f} ms; "
        f"1x1024 graph {pre1k_ms:.3f} ms, eager {pre1k_eager:.3f} ms")

    mtp = {}
    for T in (2, 4, 8, 16):
        _, mg = bench_decode(64, 50, 5, dev, tokens=T)
        mtp[f"B64_T{T}"] = round(mg * 1e3, 2)
    log(f"multi-token decode B=64 (us per call): {mtp}")
    short = {}
    for name, lens in (("256x1", [1] * 256), ("64x16", [16] * 64), ("1x64", [64]),
                       ("32x64", [64] * 32), ("64x256", [256] * 64)):
        _, pg = bench_prefill(lens, 20, 3, dev)
        short[name] = round(pg, 4)
    log(f"short-sequence prefill (ms per call): {short}")

    # the decode batch sweep (one step in graph replay per B), and
    # the prefill configurations configs[3] and configs[4] (configs[2] is
    # the 1x1024 line above); the 4x8192 recipe skews heads 6-7 to near-unit
    # decay.
    sweep = {}
    for b in (1, 2, 4, 8, 16, 32, 48, 64):
        _, mg = bench_decode(b, 100, 10, dev)
        sweep[f"B{b}"] = {"us": round(mg * 1e3, 3),
                          "GBps": round(O.decode_bytes(b) / (mg * 1e-3) / 1e9, 1)}
    log(f"decode sweep (graph us/step, GB/s): {sweep}")
    cfg_ms = {}
    cfg_detail = {}

    def detail(lens, ms):
        T, N = sum(lens), len(lens)
        nt = sum(-(-L // 64) for L in lens)
        tflops = O.prefill_flops(nt) / (ms * 1e-3) / 1e12
        return {"ms": round(ms, 4), "tokens_per_s": round(T / (ms * 1e-3), 1),
                "tflops": round(tflops, 2), "mfma_frac": round(tflops / 2500.0, 5),
                "hbm_gbps": round(O.prefill_bytes(T, N) / (ms * 1e-3) / 1e9, 1)}

    for name, lens, kw in (("configs3_varlen6", [6, 49, 294, 1800, 2040, 61], {}),
                           ("configs4_4x8192", [8192] * 4, {"slow_decay_heads": (6, 7)})):
        _, pg = bench_prefill(lens, 10, 2, dev, **kw)
        cfg_ms[name] = round(pg, 4)
        cfg_detail[name] = detail(lens, pg)
    cfg_detail["configs2_1x1024"] = detail([1024], pre1k_ms)
    cfg_detail["north_star_1x8192"] = detail(pre_lens, pre_ms)
    log(f"prefill configs (graph ms per call): {cfg_ms}")

    cpu_s, reps = cpu_baseline_decode(B, args.cpu_seconds)
    cpu_gbs = nbytes / cpu_s / 1e9
    log(f"cpu baseline decode B={B}: {cpu_s * 1e3:.1f} ms/step over {reps} steps")
    cpu_pre_s, cpu_pre_threads = cpu_baseline_prefill(pre_lens)
    log(f"cpu baseline prefill 1x8192: {cpu_pre_s:.2f} s ({cpu_pre_threads} threads)")

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
        "decode_us_per_step": round(ms_step * 1e3, 3),
        "decode_us_per_step_eager": round(ms_eager * 1e3, 3),
        "decode_copy_ceiling": {"us": round(copy_ms * 1e3, 3), "GBps": round(copy_gbs, 1),
                                "bytes_moved": 2 * state_bytes,
                                "decode_time_over_copy": round(ms_step / copy_ms, 4)},
        "prefill_ms_1x8192": round(pre_ms, 4),
        "prefill_ms_1x8192_eager": round(pre_eager, 4),
        "prefill_tokens_per_s": round(T8 / (pre_ms * 1e-3), 1),
        "prefill_ms_1x8192_clone": round(pre_clone, 4),
        "prefill_ms_1x1024": round(pre1k_ms, 4),
        "prefill_ms_1x1024_clone": round(pre1k_clone, 4),
        "decode_sweep": sweep,
        "prefill_ms_configs": cfg_ms,
        "prefill_configs": cfg_detail,
        "decode_multi_token_us": mtp,
        "prefill_ms_short_batches": short,
        "prefill_roofline": {"bound": "mfma", "achieved": round(pre_tflops, 2), "peak": 2500.0,
                             "unit": "TFLOP/s", "frac": round(pre_tflops / 2500.0, 5),
                             "hbm_gbs": round(pre_gbs, 1),
                             "flops_per_call": O.prefill_flops(nt8),
                             "bytes_per_call": O.prefill_bytes(T8, len(pre_lens))},
        "roofline": {"bound": "hbm", "achieved": round(gbs_step, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gbs_step / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic() if (B == 64 and args.variant == -1) else None,
                     "kernel": "gdn::decode_kernel",
                     "bytes_per_launch": nbytes},
        "cpu_baseline": {"value": round(cpu_gbs, 4), "unit": "GB/s", "cores": 1, "kind": "port",
                         "sample": f"{reps} decode steps at B={B} "
                                   f"({cpu_s * 1e3:.1f} ms/step), oracle decode_loop (numpy), "
                                   f"1 thread of {cpu_model()}"},
        "cpu_baseline_prefill": {"value": round(T8 / cpu_pre_s, 1), "unit": "tokens/s",
                                 "cores": cpu_pre_threads, "kind": "port",
                                 "sample": f"one 1x8192 prefill in {cpu_pre_s:.2f} s, oracle "
                                           f"gdn_seq.c (per-token loop, f32), OpenMP over the "
                                           f"8 v-heads, {cpu_model()}"},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
