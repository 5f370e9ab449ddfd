"""Benchmark of the decode hot path on one MI355X.

Default workload: the 36-layer decode sweep at the Qwen3-4B GQA shape at
10240 tokens — every layer its own K/V cache [1, 8, 10240, 128] fp16 (1.5 GB
in total, past the 256 MB Infinity Cache) and its own query [1, 32, 1, 128].
One step is one decode token through the model's attention: 36 sequential
calls, each the split-KV partial kernel plus the LSE combine kernel, replayed
as one HIP graph. Inputs are resident in HBM before the timed region.

Printed JSON line:
- value: algorithmic GB/s of the whole step (K+V read, Q read, O written:
  10240*4096 + 16384 bytes per call), us_per_call next to it;
- roofline: the partial kernel alone with the tile schedule of the timed call
  (tiles dealt round-robin over the splits), algorithmic bytes per launch
  over its mean duration from HIP events around a graph of 36 partial
  launches; the partial + combine fraction beside it;
- yardstick: the partial kernel's loads alone (same grid, schedule and loads
  in flight, no compute, nothing written) over the same 36 layers, the
  streaming floor of that access pattern;
- cpu_baseline: the reference's CPU decode path (torch SDPA with the query
  heads folded, fp16, threadcut/attention.py:40-42) on os.cpu_count() host
  threads, the fp32 form of the same call beside it, and the host's core
  counts and CPU model;
- splice: the 36-layer suffix splice (Split(2048, 8668, 5668), 14336-token
  caches, theta 1e6) in one launch, algorithmic GB/s (C of K and V read and
  written), with the reference's CPU splice (torch ops per layer) timed on the
  host beside it;
- prefill: the GQA-native prefill attention on a 2048-token chunk over the
  7716 tokens that splice keeps, a 300-token chunk over 9700, and a causal
  2048-token prompt, in TFLOP/s of the matrix cores next to the reference's
  GPU route (repeat_kv + SDPA).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "flash-decode µs/call & HBM GB/s (% of peak), Qwen3-4B GQA shape, 10k ctx"
PEAK_GBS = 8000.0
LAYERS, HQ, HKV, D = 36, 32, 8, 128


def decode_bytes(n, batch=1):
    return batch * (2 * HKV * n * D * 2 + 2 * HQ * D * 2)


def splice_bytes(c, layers=LAYERS):
    return 4 * layers * HKV * c * D * 2


def read_traffic(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/<name>), or None."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def time_graph(graph, steps, warmup, min_warm_ms=0.0):
    """ms per replay over `steps` replays after `warmup` untimed ones; with min_warm_ms,
    untimed replays continue until that much time has passed (the clocks of this part
    take milliseconds to ramp up after the device idled, e.g. during input generation)."""
    import torch

    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < min_warm_ms:
        graph.replay()
        torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps  # ms per replay


WARM_MS = 250.0  # untimed work before each report that times eager calls or its own inputs


def warm_eager(fn, ms=WARM_MS):
    """Calls fn (enqueued work) until `ms` of wall time has passed, synchronizing each
    time: the device then runs at its steady speed when the timed calls start."""
    import torch

    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        fn()
        torch.cuda.synchronize()


def capture(fn):
    import torch

    fn()  # eager warm-up outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def host_info():
    """The host the CPU baselines run on: core counts as the OS and the cgroup report them, and
    the CPU model from lscpu."""
    import subprocess

    info = {"os_cpu_count": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0))}
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()
        info["cgroup_cpus"] = None if quota == "max" else round(int(quota) / int(period), 2)
    except (OSError, ValueError):
        info["cgroup_cpus"] = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        info["model"] = next((l.split(":", 1)[1].strip() for l in out.splitlines() if l.startswith("Model name")),
                             None)
    except (OSError, subprocess.SubprocessError):
        info["model"] = None
    return info


def _median_time(fn, seconds, min_runs=5):
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < min_runs:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_baseline(n, seconds):
    """The reference's CPU decode path on one call of the workload (fp16, torch SDPA with the
    query heads folded, threadcut/attention.py:40-42), and the fp32 oracle form of the same
    call beside it, each bounded to about `seconds`; os.cpu_count() threads."""
    import torch

    from oracle.decode import folded_sdpa
    from threadcut_amd import workloads

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    q, k, v, _ = workloads.decode_inputs(2, n=n)
    scale = D ** -0.5
    for _ in range(3):
        folded_sdpa(q, k, v, scale)
    t, runs = _median_time(lambda: folded_sdpa(q, k, v, scale), seconds)
    q32, k32, v32 = q.float(), k.float(), v.float()
    for _ in range(2):
        folded_sdpa(q32, k32, v32, scale)
    t32, runs32 = _median_time(lambda: folded_sdpa(q32, k32, v32, scale), seconds / 2)
    return {"value": round(decode_bytes(n) / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{runs} single decode calls (q [1,32,1,128], K/V [1,8,{n},128] fp16) of the reference's "
                      f"CPU path (torch SDPA, query heads folded), median {t * 1e6:.1f} us/call",
            "us_per_call": round(t * 1e6, 2),
            "fp32_oracle_us_per_call": round(t32 * 1e6, 2), "fp32_oracle_runs": runs32,
            "host": host_info()}


def cpu_ragged_baseline(seconds):
    """The ragged batch of 16 on the host: the reference's CPU decode (fp16 folded SDPA) once per
    sequence over its own lengths, the whole batch per sample, bounded to about `seconds`."""
    import torch

    from oracle.decode import folded_sdpa

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    lens = torch.randint(1024, 32769, (16,), generator=torch.Generator().manual_seed(3)).tolist()
    g = torch.Generator().manual_seed(3)
    seqs = [(torch.randn((1, HQ, 1, D), generator=g).half(), torch.randn((1, HKV, m, D), generator=g).half(),
             torch.randn((1, HKV, m, D), generator=g).half()) for m in lens]
    scale = D ** -0.5

    def batch():
        for q, k, v in seqs:
            folded_sdpa(q, k, v, scale)

    batch()
    t, runs = _median_time(batch, seconds, min_runs=3)
    nbytes = sum(lens) * 2 * HKV * D * 2 + 16 * 2 * HQ * D * 2
    return {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "us_per_call": round(t * 1e6, 1),
            "sample": f"{runs} passes over the 16 sequences (lengths U[1024, 32768], seed 3), one fp16 folded "
                      f"SDPA per sequence, median per pass"}


def cpu_splice_baseline(seconds, layers=LAYERS):
    """The reference's CPU splice (torch ops per layer, threadcut/kv.py:20-25,83-92) over all
    36 layers of the config (2.1 GB of host K/V), timed for about `seconds`, median."""
    import torch

    from oracle.splice import splice_growing_torch
    from threadcut_amd import workloads

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    s = workloads.SPLICE_SPLIT
    ks, vs = workloads.layer_caches(1, layers, workloads.SPLICE_TOKENS)
    inv = workloads.inv_freq(1e6)
    splice_growing_torch(ks, vs, s.a, s.c0, s.c, inv)  # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        splice_growing_torch(ks, vs, s.a, s.c0, s.c, inv)
        times.append(time.perf_counter() - t0)
    times.sort()
    t = times[len(times) // 2]
    return {"value": round(splice_bytes(s.c, layers) / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "us_per_splice": round(t * 1e6, 1),
            "sample": f"{len(times)} splices of {layers} layers ([1,8,{workloads.SPLICE_TOKENS},128] fp16, {s}) with "
                      f"the reference's torch ops on the host, median"}


def bench_splice(dev, steps, warmup):
    import torch

    from threadcut_amd import _lib, kv, workloads
    from threadcut_amd.match import Split

    s = workloads.SPLICE_SPLIT
    n = workloads.SPLICE_TOKENS
    ks, vs = workloads.layer_caches(1, LAYERS, n, device=dev)
    lib = _lib.load()
    kp = _lib.ptr_array([t.data_ptr() for t in ks])
    vp = _lib.ptr_array([t.data_ptr() for t in vs])
    st = _lib.i64x3(*ks[0].stride()[:3])

    def timed(sp, reps, warm):
        tab = _lib.float_array(kv.rope_table(-sp.gap, workloads.inv_freq(1e6)))

        def run():
            # The same move every time: the buffers' contents change, the work does not.
            _lib.check(lib.tc_splice_rope(kp, vp, LAYERS, st, 1, HKV, n, D, _lib.TC_DTYPE_F16, sp.a, sp.c0, sp.c,
                                          tab, _lib.stream_of(dev)), "tc_splice_rope")

        for _ in range(warm):
            run()
        torch.cuda.synchronize()
        warm_eager(run)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            run()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    ms = timed(s, steps, warmup)
    gbs = splice_bytes(s.c) / (ms * 1e-3) / 1e9
    # Overlapping moves whose gap is under 48 rows (the row walk), 12188 rows per strip.
    short = {}
    for gap in (1, 17, 32, 47):
        sp = Split(2048, 2048 + gap, 12188)
        t = timed(sp, max(4, steps // 10), 2)
        g = splice_bytes(sp.c) / (t * 1e-3) / 1e9
        short[str(gap)] = {"us_per_splice": round(t * 1e3, 1), "GB/s": round(g, 1), "frac": round(g / PEAK_GBS, 4)}
    return {"us_per_splice": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4),
            "bytes": splice_bytes(s.c), "config": {"layers": LAYERS, "tokens": n, "split": [s.a, s.c0, s.c],
                                                   "theta": 1e6},
            "short_gap_walk": {"split": "Split(2048, 2048 + gap, 12188)", "by_gap": short}}


SWEEP = (1536, 4096, 10240, 14336)


def summarize(r, nbytes):
    us = r["ms"] * 1e3 / LAYERS
    pus = r["ms_partial"] * 1e3 / LAYERS
    yus = r["ms_yardstick"] * 1e3 / LAYERS
    return {"us_per_call": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
            "partial_us": round(pus, 3), "partial_GB/s": round(nbytes / pus / 1e3, 1),
            "yardstick_us": round(yus, 3), "partial_over_yardstick": round(pus / yus, 4),
            "splits": r["splits"], "split_tokens": r["split_tokens"]}


def stream_read_lib():
    """The measurement library (threadcut_amd/csrc/bench): the streaming-read yardstick of
    the decode and the matrix-core ceiling of the prefill."""
    import ctypes

    from threadcut_amd import build

    lib = ctypes.CDLL(build.BENCH_LIB)
    lib.tc_bench_mfma_ceiling.restype = ctypes.c_int
    lib.tc_bench_mfma_ceiling.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.tc_bench_empty_launch.restype = ctypes.c_int
    lib.tc_bench_empty_launch.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.tc_bench_stream_read.restype = ctypes.c_int
    lib.tc_bench_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64),
                                         ctypes.POINTER(ctypes.c_int64), ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_void_p, ctypes.c_void_p]
    return lib


def layer_plans(qs, ks, vs, outs, split=None):
    """One DecodePlan per layer, all on one workspace: the layers of a decode step run one
    after another, so each layer's partials are written over the previous layer's (as the
    eager path's per-call workspace from torch's caching allocator also is)."""
    from threadcut_amd import flash_decode

    plans, ws = [], None
    for q, k, v, o in zip(qs, ks, vs, outs):
        plans.append(flash_decode.DecodePlan(q, k, v, D ** -0.5, o, split=split, workspace=ws))
        ws = plans[-1].workspace
    return plans


def measure_sweep(dev, n, steps, warmup, split, only, min_warm_ms=0.0):
    """36 sequential decode calls at n tokens (own K/V per layer) as one HIP graph; the
    partial pass alone and the streaming-read yardstick as graphs over the same layers."""
    import torch

    from threadcut_amd import _lib, workloads

    qs, ks, vs = workloads.sweep_layers(n, LAYERS, 2, device=dev)
    outs = [torch.empty_like(q) for q in qs]
    plans = layer_plans(qs, ks, vs, outs, split=split or None)
    S = plans[0].splits

    def step():
        for p in plans:
            p.run()

    def step_partial():
        for p in plans:
            p.run_partial()

    result = {"splits": S, "split_tokens": plans[0].split_tokens}
    if only in (None, "decode"):
        result["ms"] = time_graph(capture(step), steps, warmup, min_warm_ms)
    if only in (None, "partial"):
        result["ms_partial"] = time_graph(capture(step_partial), steps, warmup, min_warm_ms)
    if only in (None, "yardstick"):
        ylib = stream_read_lib()
        sink = torch.zeros(S * HKV, dtype=torch.int32, device=dev)
        st = [(_lib.i64x2(k.stride(1), k.stride(2)), _lib.i64x2(v.stride(1), v.stride(2))) for k, v in zip(ks, vs)]

        def step_read():
            s_ = _lib.stream_of(dev)
            for (k, v), (kst, vst) in zip(zip(ks, vs), st):
                if ylib.tc_bench_stream_read(k.data_ptr(), v.data_ptr(), kst, vst, n, HKV, S, sink.data_ptr(), s_):
                    raise RuntimeError("tc_bench_stream_read failed")

        result["ms_yardstick"] = time_graph(capture(step_read), steps, warmup, min_warm_ms)

        def step_empty():
            s_ = _lib.stream_of(dev)
            for _ in range(LAYERS):
                if ylib.tc_bench_empty_launch(S * HKV, sink.data_ptr(), s_):
                    raise RuntimeError("tc_bench_empty_launch failed")

        result["ms_empty"] = time_graph(capture(step_empty), steps, warmup, min_warm_ms)
    del plans, ks, vs
    torch.cuda.empty_cache()
    return result


def _time_plan(plan, steps, reps=10):
    def step():
        for _ in range(reps):
            plan.run()
    ms = time_graph(capture(step), steps, 3, min_warm_ms=WARM_MS)
    return ms * 1e3 / reps


def measure_ragged(dev, steps):
    """16 sequences, lengths U[1024, 32768] (seed 3), one padded cache + int32 lengths."""
    import torch

    from threadcut_amd import flash_decode, workloads

    gen = torch.Generator().manual_seed(3)
    lens = torch.randint(1024, 32769, (16,), generator=gen).to(torch.int32)
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    k = torch.randn((16, HKV, 32768, D), generator=g, device=dev).half()
    v = torch.randn((16, HKV, 32768, D), generator=g, device=dev).half()
    q = torch.randn((16, HKV, HQ // HKV, D), generator=g, device=dev).half()
    out = torch.empty_like(q)
    plan = flash_decode.DecodePlan(q, k, v, D ** -0.5, out, lens=lens.to(dev))
    us = _time_plan(plan, steps)
    nbytes = int(lens.sum()) * 2 * HKV * D * 2 + 16 * 2 * HQ * D * 2
    del k, v
    torch.cuda.empty_cache()
    return {"us_per_call": round(us, 2), "GB/s": round(nbytes / us / 1e3, 1), "bytes": nbytes,
            "lens_sum": int(lens.sum()), "splits": plan.splits, "split_tokens": plan.split_tokens}


def measure_long(dev, batch, steps):
    """One decode call over 131072 cached tokens per sequence (seed 4)."""
    import torch

    from threadcut_amd import flash_decode

    n = 131072
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    k = torch.randn((batch, HKV, n, D), generator=g, device=dev).half()
    v = torch.randn((batch, HKV, n, D), generator=g, device=dev).half()
    q = torch.randn((batch, HKV, HQ // HKV, D), generator=g, device=dev).half()
    out = torch.empty_like(q)
    plan = flash_decode.DecodePlan(q, k, v, D ** -0.5, out)
    us = _time_plan(plan, steps)
    nbytes = decode_bytes(n, batch)
    r = {"us_per_call": round(us, 2), "GB/s": round(nbytes / us / 1e3, 1), "bytes": nbytes,
         "splits": plan.splits, "split_tokens": plan.split_tokens}
    if batch == 1:
        # The partial pass alone and its loads alone (the streaming-read yardstick).
        from threadcut_amd import _lib

        reps = 10
        ylib = stream_read_lib()
        sink = torch.zeros(plan.splits * HKV, dtype=torch.int32, device=dev)
        kst, vst = _lib.i64x2(k.stride(1), k.stride(2)), _lib.i64x2(v.stride(1), v.stride(2))

        def partial():
            for _ in range(reps):
                plan.run_partial()

        def loads():
            for _ in range(reps):
                if ylib.tc_bench_stream_read(k.data_ptr(), v.data_ptr(), kst, vst, n, HKV, plan.splits,
                                             sink.data_ptr(), _lib.stream_of(dev)):
                    raise RuntimeError("tc_bench_stream_read failed")

        pus = time_graph(capture(partial), steps, 3, min_warm_ms=WARM_MS) * 1e3 / reps
        yus = time_graph(capture(loads), steps, 3, min_warm_ms=WARM_MS) * 1e3 / reps
        r.update({"partial_us": round(pus, 2), "yardstick_us": round(yus, 2),
                  "partial_over_yardstick": round(pus / yus, 4)})
    del k, v
    torch.cuda.empty_cache()
    return r


def measure_append(dev, n, steps):
    """One decode token over 36 layers at n tokens, cache append included: the
    reference's order (two strided copies into the cache, then attention) vs
    the fused append-and-attend launch."""
    import torch

    from threadcut_amd import _lib

    g = torch.Generator(device=dev)
    g.manual_seed(5)
    cap = n + 64
    ks = [torch.randn((1, HKV, cap, D), generator=g, device=dev).half() for _ in range(LAYERS)]
    vs = [torch.randn((1, HKV, cap, D), generator=g, device=dev).half() for _ in range(LAYERS)]
    kn = [torch.randn((1, HKV, 1, D), generator=g, device=dev).half() for _ in range(LAYERS)]
    vn = [torch.randn((1, HKV, 1, D), generator=g, device=dev).half() for _ in range(LAYERS)]
    qs = [torch.randn((1, HKV, HQ // HKV, D), generator=g, device=dev).half() for _ in range(LAYERS)]
    outs = [torch.empty_like(q) for q in qs]
    plans = layer_plans(qs, [k[:, :, :n] for k in ks], [v[:, :, :n] for v in vs], outs)
    lib = _lib.load()
    ws = plans[0].workspace
    st = _lib.i64x3(*ks[0].stride()[:3])
    nst = _lib.i64x2(0, kn[0].stride(1))
    qst = _lib.i64x3(0, qs[0].stride(1), qs[0].stride(2))

    def plain():
        for k, v, a, b_, p in zip(ks, vs, kn, vn, plans):
            k[:, :, n - 1:n] = a
            v[:, :, n - 1:n] = b_
            p.run()

    def fused():
        s = _lib.stream_of(dev)
        for k, v, a, b_, q, o in zip(ks, vs, kn, vn, qs, outs):
            _lib.check(lib.tc_decode_append_attention(
                q.data_ptr(), qst, k.data_ptr(), st, v.data_ptr(), st, a.data_ptr(), nst, b_.data_ptr(), nst,
                n, 1, HKV, HQ // HKV, D, _lib.TC_DTYPE_F16, D ** -0.5, plans[0].split_tokens,
                ws.data_ptr(), ws.numel(), o.data_ptr(), qst, s), "tc_decode_append_attention")

    ms_plain = time_graph(capture(plain), steps, 5)
    ms_fused = time_graph(capture(fused), steps, 5)
    del ks, vs
    torch.cuda.empty_cache()
    return {"kv_tokens": n, "us_per_layer_copy_then_attend": round(ms_plain * 1e3 / LAYERS, 3),
            "us_per_layer_fused_append": round(ms_fused * 1e3 / LAYERS, 3)}


PEAK_MFMA_F16 = 2500.0  # dense fp16 matrix-core TFLOP/s of one MI355X


def prefill_flops(q_len, n, causal_like, hq=HQ, d=D):
    """Algorithmic FLOPs of one prefill attention call: 2*d each for QK^T and PV per
    visible (query head, query, key) triple; a causal chunk sees n - q_len + t + 1 keys."""
    pairs = q_len * n - (q_len * (q_len - 1) // 2 if causal_like else 0)
    return 4 * pairs * d * hq


def measure_mfma_ceiling(dev, iters=2000):
    """Back-to-back 32x32x16 fp16 MFMAs at the prefill's occupancy (two 256-thread
    work-groups per CU), with constant and with random operand bits: PFLOP/s."""
    import torch

    lib = stream_read_lib()
    wgs = 2 * torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.zeros(wgs * 256, dtype=torch.float32, device=dev)
    out = {}
    for name, rnd in (("constant_operands_pflops", 0), ("random_operands_pflops", 1)):
        def run():
            if lib.tc_bench_mfma_ceiling(rnd, wgs, iters, sink.data_ptr(), _stream(dev)):
                raise RuntimeError("tc_bench_mfma_ceiling failed")
        run()
        torch.cuda.synchronize()
        warm_eager(run)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(3):
            run()
        b.record()
        torch.cuda.synchronize()
        sec = a.elapsed_time(b) / 3 * 1e-3
        out[name] = round(wgs * 4 * iters * 16 * 32768 / sec / 1e15, 3)
    return out


def _stream(dev):
    from threadcut_amd import _lib

    return _lib.stream_of(dev)


def measure_prefill(dev, steps, only_case=None):
    """Prefill attention at the Qwen3-4B shape (32 q / 8 kv heads, D=128, fp16, the reference
    engine's dtype; the engine chunk also in bf16, the checkpoint's): the GQA-native kernel vs
    the reference's GPU route (repeat_kv + SDPA with the same mask)."""
    import torch

    from threadcut_amd import attention, prefill, workloads

    def timed(fn, iters):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        warm_eager(fn)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / iters * 1e3

    chunk_n = workloads.PREFILL_PAST + workloads.PREFILL_CHUNK
    cases = [("chunk_2048_on_7716", workloads.PREFILL_CHUNK, chunk_n, True),
             ("chunk_300_on_9700", 300, 10000, True),
             ("prompt_2048_causal", 2048, 2048, False),
             ("chunk_2048_on_7716_bf16", workloads.PREFILL_CHUNK, chunk_n, True)]
    if only_case is not None:
        # One workload alone (for counter runs); "nomask_2048_on_9764" is the chunk shape without a mask.
        cases = [c for c in cases + [("nomask_2048_on_9764", 2048, 9764, None),
                                     ("holes_2048_on_9764", 2048, 9764, "holes")] if c[0] == only_case]
        if not cases:
            raise SystemExit(f"unknown prefill case {only_case}")
    out = {}
    for name, L, n, masked in cases:
        dtype = torch.bfloat16 if name.endswith("_bf16") else torch.float16
        q, k, v = workloads.prefill_inputs(7, q_len=L, n=n, dtype=dtype, device=dev)
        mask = workloads.causal_mask(L, n, device=dev) if masked else None
        if masked == "holes":
            # Causal with one key in ten hidden at random: every active tile is
            # tested per element against the mask bytes.
            holes = torch.rand(L, n, generator=torch.Generator(device=dev).manual_seed(11), device=dev) < 0.1
            mask = mask & ~holes[None, None]
        causal = masked is False
        scale = D ** -0.5
        iters = max(5, steps // 10)
        prefill.prefill_attention(q, k, v, mask, scale, causal)  # builds the mask's tile map once
        us = timed(lambda: prefill.prefill_attention(q, k, v, mask, scale, causal), iters)
        ref = timed(lambda: torch.nn.functional.scaled_dot_product_attention(
            q, attention.repeat_kv(k, HQ // HKV), attention.repeat_kv(v, HQ // HKV), attn_mask=mask, scale=scale,
            is_causal=causal).transpose(1, 2).contiguous(), iters)
        tflops = prefill_flops(L, n, masked is not None) / (us * 1e-6) / 1e12
        r = {"q_len": L, "kv_tokens": n, "dtype": "bf16" if dtype == torch.bfloat16 else "f16",
             "mask": {True: "bool [1,1,q,n] causal", False: "is_causal", None: "none",
                      "holes": "bool [1,1,q,n] causal, 10% of keys hidden at random"}[masked],
             "splits": prefill.num_splits(1, L, n, HQ, HKV), "us_per_call": round(us, 1),
             "tflops": round(tflops, 1), "frac_of_mfma_peak": round(tflops / PEAK_MFMA_F16, 4),
             "reference_route_us": round(ref, 1), "speedup": round(ref / us, 2)}
        if masked:
            prefill._tile_cache = None
            r["mask_tile_map_us_once_per_forward"] = round(timed(
                lambda: (setattr(prefill, "_tile_cache", None), prefill.mask_tiles(mask, HQ, HKV)), iters), 1)
        out[name] = r
        del q, k, v, mask
    torch.cuda.empty_cache()
    if only_case is None:
        # What the matrix core sustains on data like these (its clock drops under
        # toggling operands), and each workload against it.
        ceil = measure_mfma_ceiling(dev)
        for r in out.values():
            r["frac_of_random_operand_ceiling"] = round(r["tflops"] / 1e3 / ceil["random_operands_pflops"], 4)
        out["mfma_ceiling"] = {**ceil, "what": "v_mfma_f32_32x32x16_f16 back to back, 8 accumulators per wave, "
                                              "two 256-thread work-groups per CU (libthreadcut_bench.so)"}
    return out


QWEN3_4B_CONFIG = dict(vocab_size=151936, hidden_size=2560, intermediate_size=9728, num_hidden_layers=LAYERS,
                       num_attention_heads=HQ, num_key_value_heads=HKV, head_dim=D, max_position_embeddings=40960,
                       rope_theta=1e6, tie_word_embeddings=True)


def measure_timeline(dev, n, steps, paged=False):
    """Per-wave timeline of the decode partial kernel at n tokens (36 layers in one graph, as the
    headline): the measurement build libthreadcut_stamps.so has every partial wave record the
    realtime clock (100 MHz) at its start, after its first tile's step, at its loop's end,
    after the merge barrier and after its partial stores are issued. Times are microseconds
    from the first wave start of the same launch; percentiles over all waves of all layers.
    The gap is from a launch's last store issue to the next launch's first wave start: the
    partial's drain, the combine launch and its work, and the next launch. With `paged` the
    layers are read through a PagedKV's tile table (64-token pages from a shuffled free list)."""
    import ctypes

    import numpy as np
    import torch

    from threadcut_amd import _lib, build, workloads

    lib = _lib.bind(build.STAMPS_LIB)
    lib.tc_decode_set_stamps.restype = None
    lib.tc_decode_set_stamps.argtypes = [ctypes.c_void_p]
    if paged:
        cache = paged_cache(dev, n, 5)
        gq = torch.Generator(device=dev)
        gq.manual_seed(6)
        qs = [torch.randn((1, HKV, HQ // HKV, D), generator=gq, device=dev).half() for _ in range(LAYERS)]
        outs = [torch.empty_like(q) for q in qs]
        runs = [lambda i=i: cache.decode(i, qs[i], D ** -0.5, out=outs[i]) for i in range(LAYERS)]
        S = lib.tc_decode_num_splits(1, HKV, 16 * cache.device_table()[2], 0, 0)
    else:
        qs, ks, vs = workloads.sweep_layers(n, LAYERS, 2, device=dev)
        outs = [torch.empty_like(q) for q in qs]
        plans = layer_plans(qs, ks, vs, outs)
        for p in plans:
            p.lib = lib
        runs = [p.run for p in plans]
        S = plans[0].splits
    waves = 2 if (n <= _lib.TC_DECODE_SHORT_TOKENS and not paged) else 4  # partial work-group shape
    stamps = torch.zeros(LAYERS, HKV * S * waves * 8, dtype=torch.int64, device=dev)

    def step(record):
        with _lib.using(lib):
            for i, run in enumerate(runs):
                lib.tc_decode_set_stamps(stamps[i].data_ptr() if record else None)
                run()
        lib.tc_decode_set_stamps(None)

    g_plain = capture(lambda: step(False))
    g_rec = capture(lambda: step(True))
    ms_plain = time_graph(g_plain, steps, 20, WARM_MS)
    ms_rec = time_graph(g_rec, steps, 20, WARM_MS)
    stamps.zero_()
    g_rec.replay()
    torch.cuda.synchronize()
    raw = stamps.view(LAYERS, HKV, S, waves, 8).cpu().numpy()
    t = raw[..., :5].astype(np.float64) * 0.01  # 100 MHz ticks -> us
    first = t[..., 0].reshape(LAYERS, -1).min(axis=1)
    rel = t - first[:, None, None, None, None]
    names = ["start", "first_step_done", "loop_end", "after_barrier", "stores_issued"]

    def pct(x):
        x = x.ravel()
        return {"p10": round(float(np.percentile(x, 10)), 3), "median": round(float(np.median(x)), 3),
                "p90": round(float(np.percentile(x, 90)), 3), "max": round(float(x.max()), 3)}

    last = t[..., 4].reshape(LAYERS, -1).max(axis=1)
    xcc = (raw[..., 6] & 15).astype(int)
    return {
        "kv_tokens": n, "splits": S, "layers": LAYERS, "cache": "paged" if paged else "contiguous",
        "us_per_call": round(ms_plain * 1e3 / LAYERS, 3),
        "us_per_call_recording": round(ms_rec * 1e3 / LAYERS, 3),
        "events_us_from_launch_start": {nm: pct(rel[..., k]) for k, nm in enumerate(names)},
        "per_wave_us": {"start_to_first_step_done": pct(rel[..., 1] - rel[..., 0]),
                        "loop_end_to_barrier": pct(rel[..., 3] - rel[..., 2]),
                        "barrier_to_stores_issued": pct(rel[..., 4] - rel[..., 3])},
        "launch_span_us_median": round(float(np.median(last - first)), 3),
        "gap_to_next_launch_us_median": round(float(np.median(first[1:] - last[:-1])), 3),
        "loop_end_median_by_kv_head": [round(float(np.median(rel[:, h, :, :, 2])), 3) for h in range(HKV)],
        "xcd_of_kv_head": [int(np.bincount(xcc[:, h].ravel()).argmax()) for h in range(HKV)],
    }


def measure_prefill_sweep(dev, iters=10):
    """The prefill kernel across chunk lengths and cached contexts (Qwen3-4B heads, fp16, a bool
    causal chunk mask; past 0 is a causal prompt through is_causal), each call timed in steady
    state beside the reference's GPU route (repeat_kv + SDPA with the same mask)."""
    import torch

    from threadcut_amd import attention, prefill, workloads

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        warm_eager(fn)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / iters * 1e3

    rows = []
    for q_len in (256, 512, 1024, 2048, 4096):
        for past in (0, 2048, 8192, 16384):
            n = past + q_len
            q, k, v = workloads.prefill_inputs(q_len + past, q_len=q_len, n=n, device=dev)
            causal = past == 0
            mask = None if causal else workloads.causal_mask(q_len, n, device=dev)
            scale = D ** -0.5
            us = timed(lambda: prefill.prefill_attention(q, k, v, mask, scale, causal))
            ref = timed(lambda: torch.nn.functional.scaled_dot_product_attention(
                q, attention.repeat_kv(k, HQ // HKV), attention.repeat_kv(v, HQ // HKV), attn_mask=mask,
                scale=scale, is_causal=causal))
            tflops = prefill_flops(q_len, n, True) / (us * 1e-6) / 1e12
            rows.append({"q_len": q_len, "past": past, "splits": prefill.num_splits(1, q_len, n, HQ, HKV),
                         "us_per_call": round(us, 1), "tflops": round(tflops, 1),
                         "frac_of_mfma_peak": round(tflops / PEAK_MFMA_F16, 4),
                         "reference_route_us": round(ref, 1), "speedup": round(ref / us, 2)})
            del q, k, v, mask
    return {"what": "prefill_attention, Qwen3-4B heads (32 q / 8 kv, D=128), fp16, batch 1", "rows": rows}


def measure_prefill_timeline(dev, iters=20):
    """Per-tile phase times of the prefill kernel on the engine chunk (2048 queries over 7716
    cached tokens, bool causal mask): the measurement build libthreadcut_stamps.so has every
    prefill wave record the shader clock at each tile's start, after its QK^T MFMAs are issued,
    after the softmax, after its P.V MFMAs are issued and once the next tile's loads into LDS
    have landed (the barrier follows). A tile's phases are: QK^T (the next tile's load burst
    included), softmax, P.V, load wait and barrier (its end to the next tile's start).
    Percentiles over every wave's tiles but its first two and last two, in shader-clock
    cycles; the clock is the ratio of the shader clock to the 100 MHz realtime clock over each
    wave's run."""
    import ctypes

    import numpy as np
    import torch

    from threadcut_amd import _lib, build, prefill, workloads

    lib = _lib.bind(build.STAMPS_LIB)
    lib.tc_prefill_set_stamps.restype = None
    lib.tc_prefill_set_stamps.argtypes = [ctypes.c_void_p]
    L, n = workloads.PREFILL_CHUNK, workloads.PREFILL_PAST + workloads.PREFILL_CHUNK
    q, k, v = workloads.prefill_inputs(7, q_len=L, n=n, device=dev)
    mask = workloads.causal_mask(L, n, device=dev)
    g = HQ // HKV
    splits = prefill.num_splits(1, L, n, HQ, HKV)
    groups = -(-L * g // 128) * HKV * splits
    words = 8 + 5 * 256
    stamps = torch.zeros(groups * 4 * words, dtype=torch.int64, device=dev)

    def timed(fn):
        warm_eager(fn)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / iters * 1e3

    with _lib.using(lib):  # the prefill wrapper calls the measurement build in this block
        try:
            call = lambda: prefill.prefill_attention(q, k, v, mask, D ** -0.5, False)
            call()
            us_plain = timed(call)
            lib.tc_prefill_set_stamps(ctypes.c_void_p(stamps.data_ptr()))
            us_rec = timed(call)
            stamps.zero_()
            call()
            torch.cuda.synchronize()
        finally:
            lib.tc_prefill_set_stamps(None)
    raw = stamps.view(groups, 4, words).cpu().numpy().astype(np.int64)
    head = raw[..., :8]
    tiles = head[..., 5]
    clock_ghz = np.median((head[..., 2] - head[..., 0]) / ((head[..., 3] - head[..., 1]) * 10.0))
    phases = {"qk_with_load_burst": [], "softmax": [], "pv": [], "load_wait": [], "barrier": [], "tile": []}
    for w in range(groups):
        for wave in range(4):
            nt = int(tiles[w, wave])
            t = raw[w, wave, 8:8 + 5 * nt].reshape(nt, 5)
            for i in range(2, nt - 2):
                phases["qk_with_load_burst"].append(t[i, 1] - t[i, 0])
                phases["softmax"].append(t[i, 2] - t[i, 1])
                phases["pv"].append(t[i, 3] - t[i, 2])
                phases["load_wait"].append(t[i, 4] - t[i, 3])
                phases["barrier"].append(t[i + 1, 0] - t[i, 4])
                phases["tile"].append(t[i + 1, 0] - t[i, 0])

    def pct(x):
        x = np.asarray(x, dtype=np.float64)
        return {"p10": int(np.percentile(x, 10)), "median": int(np.median(x)), "p90": int(np.percentile(x, 90))}

    span_us = (head[..., 3] - head[..., 1]).max(axis=1) / 100.0
    # Work-groups i and i + groups/2 share a CU (the dispatcher's placement at two per CU): the
    # tile times of the one with more tiles while its partner runs, and after the partner ended.
    shared, alone = [], []
    half = groups // 2
    for w in range(half):
        pair = (w, w + half)
        long_w, short_w = (pair if tiles[pair[0], 0] >= tiles[pair[1], 0] else pair[::-1])
        end_short = head[short_w, :, 2].max()
        for wave in range(4):
            nt = int(tiles[long_w, wave])
            t = raw[long_w, wave, 8:8 + 5 * nt].reshape(nt, 5)[:, 0]
            d = np.diff(t)
            for i in range(2, nt - 2):
                (alone if t[i] > end_short else shared).append(d[i])
    # By XCD (HW_REG_XCC_ID; with 8 KV heads each XCD runs one head's work-groups): its shader clock
    # and when its work-groups with the most tiles end, from the launch's first wave start.
    t0 = head[..., 1].min()
    end_us = (head[..., 3].max(axis=1) - t0) / 100.0
    xcc = (head[:, 0, 4] >> 32) & 0xF
    wg_clock = (head[..., 2] - head[..., 0]).max(axis=1) / ((head[..., 3] - head[..., 1]).max(axis=1) * 10.0)
    longest = tiles[:, 0] >= tiles[:, 0].max() - 8
    by_xcd = {}
    for x in sorted(set(int(v) for v in xcc)):
        m = xcc == x
        by_xcd[str(x)] = {"clock_ghz": round(float(np.median(wg_clock[m])), 3),
                          "longest_work_groups_end_us": {"median": round(float(np.median(end_us[m & longest])), 1),
                                                         "max": round(float(end_us[m].max()), 1)}}
    return {
        "workload": "prefill engine chunk: 2048 queries over 9764 keys (7716 cached), bool causal mask, fp16",
        "work_groups": int(groups), "us_per_call": round(us_plain, 1), "us_per_call_recording": round(us_rec, 1),
        "shader_clock_ghz_median": round(float(clock_ghz), 3),
        "tile_phase_cycles": {k: pct(x) for k, x in phases.items()},
        "tiles_per_work_group": {"min": int(tiles[:, 0].min()), "max": int(tiles[:, 0].max())},
        "work_group_span_us": {"min": round(float(span_us.min()), 1), "median": round(float(np.median(span_us)), 1),
                               "max": round(float(span_us.max()), 1)},
        "longer_of_a_cu_pair_tile_cycles": {"partner_running": pct(shared) if shared else None,
                                            "partner_done": pct(alone) if alone else None},
        "by_xcd": by_xcd,
    }


def measure_decode_step(dev, n=10240, steps=40):
    """Whole-model decode step at the Qwen3-4B shape (random fp16 weights, 36 layers) at n
    cached tokens: the reference's eager per-token loop (engine.py:88-95) with the "threadcut"
    attention and fused cache append, against the same step captured once and replayed
    (graph.DecodeGraph)."""
    import torch
    from transformers import AutoModelForCausalLM, Qwen3Config

    from threadcut_amd import attention, kv, paged
    from threadcut_amd.graph import DecodeGraph

    torch.manual_seed(8)
    cfg = Qwen3Config(**QWEN3_4B_CONFIG)
    with torch.device(dev):
        model = AutoModelForCausalLM.from_config(cfg, dtype=torch.float16, attn_implementation=attention.NAME)
    model.eval()
    g = torch.Generator(device=dev)
    g.manual_seed(8)
    prompt = torch.randint(0, cfg.vocab_size, (1, n), generator=g, device=dev)
    caches = [kv.new_cache(cfg, fused_append=True) for _ in range(2)]
    with torch.no_grad():
        for c in caches:
            for i in range(0, n, 2048):
                model(input_ids=prompt[:, i:i + 2048], past_key_values=c, use_cache=True, logits_to_keep=1)
        tok = torch.randint(0, cfg.vocab_size, (1, 1), generator=g, device=dev)

        def eager_step():
            return model(input_ids=tok, past_key_values=caches[0], use_cache=True, logits_to_keep=1).logits

        for _ in range(3):
            eager_step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            eager_step()
        torch.cuda.synchronize()
        eager_ms = (time.perf_counter() - t0) * 1e3 / steps
        dg = DecodeGraph(model, caches[1], max_new_tokens=steps + 8)
        for _ in range(3):
            dg.step(tok)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            dg.step(tok)
        torch.cuda.synchronize()
        graph_ms = (time.perf_counter() - t0) * 1e3 / steps
        dg.close()
        del caches, dg
        # The same step over the paged cache (64-token pages), prefilled the same way.
        pcache = paged.new_paged_cache(cfg, num_pages=n // 64 + steps // 64 + 8, page_tokens=64)
        for i in range(0, n, 2048):
            model(input_ids=prompt[:, i:i + 2048], past_key_values=pcache, use_cache=True, logits_to_keep=1)
        pg = DecodeGraph(model, pcache, max_new_tokens=steps + 8)
        for _ in range(3):
            pg.step(tok)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            pg.step(tok)
        torch.cuda.synchronize()
        paged_ms = (time.perf_counter() - t0) * 1e3 / steps
        pg.close()
        del pcache, pg
    weights = sum(p.numel() * p.element_size() for p in model.parameters())
    del model
    torch.cuda.empty_cache()
    return {"kv_tokens": n, "layers": LAYERS, "weights_GB": round(weights / 1e9, 2),
            "eager_ms_per_token": round(eager_ms, 3), "graph_ms_per_token": round(graph_ms, 3),
            "speedup": round(eager_ms / graph_ms, 2),
            "graph_ms_per_token_paged_cache": round(paged_ms, 3),
            "graph_weight_read_GB/s": round(weights / (graph_ms * 1e-3) / 1e9, 1),
            "note": "random-init weights; the step includes every layer's projections, MLP and the LM head"}


def measure_torch_reads(dev, n, reps=50):
    """What torch's own kernels achieve on one layer's K/V at n tokens ([2, 8, n, 128] fp16, 36 distinct
    buffers, each sequence captured as one graph): a device copy (reads and writes the bytes) and an
    fp32-accumulating sum (reads them). A yardstick for the decode's streaming rate at this size."""
    import torch

    bufs = [torch.randn((2, HKV, n, D), device=dev, dtype=torch.float16) for _ in range(LAYERS)]
    dsts = [torch.empty_like(b) for b in bufs]
    sums = [torch.empty((), device=dev, dtype=torch.float32) for _ in range(LAYERS)]
    nbytes = bufs[0].numel() * 2
    out = {}
    for name, fn, moved in (("copy", lambda: [d.copy_(b) for d, b in zip(dsts, bufs)], 2 * nbytes),
                            ("sum", lambda: [o.copy_(torch.sum(b, dtype=torch.float32))
                                             for o, b in zip(sums, bufs)], nbytes)):
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            for _ in range(3):
                fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            fn()
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / reps / LAYERS
        out[name] = {"us_per_layer": round(us, 2), "GB/s": round(moved / us / 1e3, 1),
                     "frac": round(moved / us / 1e3 / PEAK_GBS, 4)}
    out["bytes_read_per_layer"] = nbytes
    del bufs, dsts, sums
    torch.cuda.empty_cache()
    return out


def paged_cache(dev, tokens, seed, page_tokens=64):
    """A 36-layer PagedKV holding `tokens` random fp16 K/V rows of sequence 0, its pages
    handed out from a shuffled free list (neighbouring tiles sit on scattered pages)."""
    import random

    import torch

    from threadcut_amd.paged import PagedKV

    cache = PagedKV(LAYERS, HKV, -(-tokens // page_tokens) + 4, page_tokens, device=dev)
    random.Random(seed).shuffle(cache.table.free)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    cache.append(0, [torch.randn((HKV, tokens, D), generator=g, device=dev).half() for _ in range(LAYERS)],
                 [torch.randn((HKV, tokens, D), generator=g, device=dev).half() for _ in range(LAYERS)])
    return cache


def measure_paged(dev, n, steps, page_tokens=64):
    """The paged cache (threadcut_amd.paged): a 36-layer decode sweep at n tokens read
    through the tile table, and the prune of the splice workload (Split(2048, 8668, 5668)
    on 14336 tokens), whose device work is the kept keys' in-place rotation. Pages are
    handed out from a shuffled free list, so neighbouring tiles sit on scattered pages."""
    import time

    import torch

    from threadcut_amd import _lib, kv, workloads
    from threadcut_amd.paged import PageTable, _cut, tiles_of

    out = {"page_tokens": page_tokens}
    cache = paged_cache(dev, n, 5, page_tokens)
    gq = torch.Generator(device=dev)
    gq.manual_seed(6)
    qs = [torch.randn((1, HKV, HQ // HKV, D), generator=gq, device=dev).half() for _ in range(LAYERS)]
    outs = [torch.empty_like(q) for q in qs]

    def step():
        for layer in range(LAYERS):
            cache.decode(layer, qs[layer], D ** -0.5, out=outs[layer])

    ms = time_graph(capture(step), steps, 5, WARM_MS)
    # Beside it, the contiguous decode of the same keys (gathered into [1, Hkv, n, D]
    # per layer), timed the same way in the same run.
    gathered = [cache.gather(layer, 0) for layer in range(LAYERS)]
    outs_c = [torch.empty_like(q) for q in qs]
    plans = layer_plans(qs, [k[None] for k, _ in gathered], [v[None] for _, v in gathered], outs_c)

    def step_contiguous():
        for p in plans:
            p.run()

    ms_c = time_graph(capture(step_contiguous), steps, 5, WARM_MS)
    out[f"decode_{n}"] = {"us_per_call": round(ms * 1e3 / LAYERS, 3),
                          "GB/s": round(LAYERS * decode_bytes(n) / (ms * 1e-3) / 1e9, 1),
                          "contiguous_us_per_call": round(ms_c * 1e3 / LAYERS, 3)}
    del plans, gathered, outs_c

    # One decode step with the new token's K/V: written into its reserved slot by
    # two torch row copies per layer and then attended, against the fused call.
    # The step is completed once eagerly (write_step), so decode() reads the slot.
    kns = [torch.randn((1, HKV, D), generator=gq, device=dev).half() for _ in range(LAYERS)]
    vns = [torch.randn((1, HKV, D), generator=gq, device=dev).half() for _ in range(LAYERS)]
    cache.reserve_step()
    for layer in range(LAYERS):
        cache.write_step(layer, kns[layer], vns[layer])
    page, slot = (int(x) for x in cache.table.token_slots(0)[-1])
    tab, cnt, mt = cache.device_table()
    lib = _lib.load()
    S = lib.tc_decode_num_splits(1, HKV, 16 * mt, 0, 0)
    ws = torch.empty(lib.tc_decode_workspace_bytes(1, HKV, HQ // HKV, D, S), dtype=torch.uint8, device=dev)
    pst = _lib.i64x3(*cache.k_pools[0].stride()[:3])
    nst = _lib.i64x2(HKV * D, D)

    def write_then_attend():
        for layer in range(LAYERS):
            cache.k_pools[layer][page, :, slot] = kns[layer][0]
            cache.v_pools[layer][page, :, slot] = vns[layer][0]
            cache.decode(layer, qs[layer], D ** -0.5, out=outs[layer])

    def fused():
        for layer in range(LAYERS):
            kp, vp = cache.k_pools[layer], cache.v_pools[layer]
            _lib.check(lib.tc_decode_paged_append_attention(
                qs[layer].data_ptr(), _lib.i64x3(*qs[layer].stride()[:3]), kp.data_ptr(), vp.data_ptr(), pst,
                kp.shape[0], kp.shape[2], tab.data_ptr(), cnt.data_ptr(), mt, kns[layer].data_ptr(), nst,
                vns[layer].data_ptr(), nst, 1, HKV, HQ // HKV, D, _lib.TC_DTYPE_F16, D ** -0.5, 0, ws.data_ptr(),
                ws.numel(), outs[layer].data_ptr(), _lib.i64x3(*outs[layer].stride()[:3]), _lib.stream_of(dev)),
                "tc_decode_paged_append_attention")

    ms_plain = time_graph(capture(write_then_attend), steps, 5)
    ms_fused = time_graph(capture(fused), steps, 5)
    out["append_step"] = {"kv_tokens": n + 1, "us_per_layer_write_then_attend": round(ms_plain * 1e3 / LAYERS, 3),
                          "us_per_layer_fused_append": round(ms_fused * 1e3 / LAYERS, 3)}
    del cache, qs, outs, ws
    torch.cuda.empty_cache()

    s = workloads.SPLICE_SPLIT
    cache = paged_cache(dev, workloads.SPLICE_TOKENS, 7, page_tokens)
    suffix = _cut(cache.table.frags[0], s.c0, s.c0 + s.c)
    tiles = tiles_of(suffix, page_tokens)
    t = torch.zeros((len(tiles), 4), dtype=torch.int32)
    t[:, :3] = torch.from_numpy(tiles)
    td = t.to(dev)
    table = _lib.float_array(kv.rope_table(-s.gap, workloads.inv_freq(1e6)))
    lib = _lib.load()
    kp = _lib.ptr_array([p.data_ptr() for p in cache.k_pools])
    st = _lib.i64x3(*cache.k_pools[0].stride()[:3])
    pages = cache.k_pools[0].shape[0]

    def rotate():
        _lib.check(lib.tc_paged_rotate_keys(kp, LAYERS, st, pages, page_tokens, td.data_ptr(), len(tiles), HKV, D,
                                            _lib.TC_DTYPE_F16, table, _lib.stream_of(dev)), "tc_paged_rotate_keys")

    ms = time_graph(capture(rotate), max(5, steps // 10), 3)
    nbytes = 2 * LAYERS * HKV * s.c * D * 2  # K of the kept suffix, read and written
    # Host bookkeeping of one prune (fragment cut, free list, tile list), on copies of the table.
    reps, t0 = 50, time.perf_counter()
    for _ in range(reps):
        pt = PageTable(pages, page_tokens)
        pt.frags = [cache.table.frags[0].copy()]
        pt.free = list(cache.table.free)
        suf, freed = pt.prune(0, s.a, s.c0, s.c)
        tiles_of(suf, page_tokens)
    host_us = (time.perf_counter() - t0) * 1e6 / reps
    out["prune_splice_split"] = {
        "split": [s.a, s.c0, s.c], "tokens": workloads.SPLICE_TOKENS, "layers": LAYERS,
        "us_device": round(ms * 1e3, 2), "bytes": nbytes, "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
        "frac": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_GBS, 4), "tiles": len(tiles),
        "pages_freed": len(freed), "host_us_bookkeeping": round(host_us, 1)}
    del cache, td
    torch.cuda.empty_cache()
    out["prefill_chunk_2048_on_7716"] = measure_paged_prefill(dev, page_tokens)
    return out


def measure_paged_prefill(dev, page_tokens, iters=10):
    """The engine's prefill chunk (2048 queries over 7716 cached keys, bool causal mask, Qwen3-4B
    heads, fp16) through the page pools (per-token row offsets, pages from a shuffled free list)
    against the contiguous prefill kernel on the same keys gathered into one buffer."""
    import random

    import torch

    from threadcut_amd import prefill, workloads
    from threadcut_amd.paged import PagedKV

    L, n = workloads.PREFILL_CHUNK, workloads.PREFILL_PAST + workloads.PREFILL_CHUNK
    q, k, v = workloads.prefill_inputs(7, q_len=L, n=n, device=dev)
    mask = workloads.causal_mask(L, n, device=dev)
    cache = PagedKV(1, HKV, -(-n // page_tokens) + 4, page_tokens, device=dev)
    random.Random(9).shuffle(cache.table.free)
    cache.append(0, [k[0]], [v[0]])

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        warm_eager(fn)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / iters * 1e3

    us_paged = timed(lambda: cache.prefill(0, q, D ** -0.5, mask))
    us_contig = timed(lambda: prefill.prefill_attention(q, k, v, mask, D ** -0.5))
    tflops = prefill_flops(L, n, True) / (us_paged * 1e-6) / 1e12
    del cache, q, k, v, mask
    torch.cuda.empty_cache()
    return {"page_tokens": page_tokens, "us_per_call": round(us_paged, 1), "tflops": round(tflops, 1),
            "contiguous_us_per_call": round(us_contig, 1)}


def measure_match(seconds=2.0):
    """Request split at a 131072-token cache: the native matcher vs the reference's numpy windows."""
    import numpy as np

    from oracle.match import split_windows
    from threadcut_amd.match import split

    rng = np.random.default_rng(6)
    cached = rng.integers(0, 151936, 131072).astype(np.int64)
    new = np.concatenate((cached[:20000], cached[60000:], rng.integers(0, 151936, 100)))

    def timed(fn):
        times, t_end = [], time.perf_counter() + seconds
        while time.perf_counter() < t_end or len(times) < 3:
            t0 = time.perf_counter()
            r = fn(cached, new, 32)
            times.append(time.perf_counter() - t0)
        times.sort()
        return times[len(times) // 2], r

    t_native, r_native = timed(split)
    t_numpy, r_numpy = timed(split_windows)
    assert tuple(r_native.__dict__.values()) == tuple(r_numpy), (r_native, r_numpy)
    return {"cached_tokens": len(cached), "split": [r_native.a, r_native.c0, r_native.c],
            "native_us": round(t_native * 1e6, 1), "reference_numpy_us": round(t_numpy * 1e6, 1)}


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--n", type=int, default=10240, help="KV tokens per layer")
    ap.add_argument("--split", type=int, default=0, help="tokens per KV split (0: tuned)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-splice", action="store_true")
    ap.add_argument("--no-reports", action="store_true",
                    help="skip the other lengths, the ragged batch and the 131072-token calls")
    ap.add_argument("--only", choices=["decode", "partial", "yardstick", "splice", "copy", "prefill", "decode-step",
                                       "paged", "decode-timeline", "decode-timeline-paged", "prefill-timeline",
                                       "prefill-sweep"],
                    default=None,
                    help="run one measurement only (for profiling); copy: a plain 256 MiB device copy, "
                         "the calibration kernel of the HBM byte counters")
    ap.add_argument("--prefill-case", default=None,
                    help="with --only prefill: one workload (chunk_2048_on_7716, chunk_300_on_9700, "
                         "prompt_2048_causal, chunk_2048_on_7716_bf16, nomask_2048_on_9764, holes_2048_on_9764)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the decode path is measured on a single MI355X "
              f"(got --gpus {args.gpus}, WORLD_SIZE {world}); multi-GPU sharding is not part of this build.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import threadcut_amd  # noqa: F401  (fails loudly here if the package is broken)

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.only == "splice":
        print(json.dumps(bench_splice(dev, args.steps, args.warmup)))
        return
    if args.only == "prefill":
        print(json.dumps(measure_prefill(dev, args.steps, args.prefill_case)))
        return
    if args.only == "paged":
        print(json.dumps(measure_paged(dev, args.n, max(20, args.steps // 4))))
        return
    if args.only == "decode-timeline":
        print(json.dumps({str(m): measure_timeline(dev, m, args.steps) for m in
                          ([args.n] if args.n != 10240 else [1536, 10240])}))
        return
    if args.only == "decode-timeline-paged":
        print(json.dumps({"contiguous": measure_timeline(dev, args.n, args.steps),
                          "paged": measure_timeline(dev, args.n, args.steps, paged=True)}))
        return
    if args.only == "prefill-sweep":
        print(json.dumps(measure_prefill_sweep(dev)))
        return
    if args.only == "prefill-timeline":
        print(json.dumps(measure_prefill_timeline(dev)))
        return
    if args.only == "decode-step":
        print(json.dumps(measure_decode_step(dev, args.n)))
        return
    if args.only == "copy":
        src = torch.empty(128 << 20, dtype=torch.float16, device=dev).normal_()
        dst = torch.empty_like(src)
        for _ in range(args.warmup + args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_each_way": src.numel() * 2, "launches": args.warmup + args.steps}))
        return

    n = args.n
    result = measure_sweep(dev, n, args.steps, args.warmup, args.split, args.only)
    if args.only is not None:
        print(json.dumps({k: round(v, 5) for k, v in result.items() if isinstance(v, float)}))
        return

    ms = result["ms"]
    per_call_bytes = decode_bytes(n)
    value = LAYERS * per_call_bytes / (ms * 1e-3) / 1e9
    partial_us = result["ms_partial"] * 1e3 / LAYERS
    achieved = per_call_bytes / (partial_us * 1e-6) / 1e9
    yard_us = result["ms_yardstick"] * 1e3 / LAYERS
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "us_per_call": round(ms * 1e3 / LAYERS, 3),
        "frac_of_peak": round(value / PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 storage, f32 accumulate",
        "data": "synthetic N(0,1) fp16 K/V/Q drawn on the device (seed 2)",
        "config": {"workload": f"36-layer decode sweep at {n} tokens, Qwen3-4B GQA (32 q / 8 kv heads, D=128), "
                               f"batch 1, one HIP graph per step",
                   "layers": LAYERS, "kv_tokens": n, "batch": 1, "q_heads": HQ, "kv_heads": HKV,
                   "head_dim": D, "splits": result["splits"], "split_tokens": result["split_tokens"]},
        "roofline": {"bound": "hbm",
                     "kernel": "decode_partial_kernel<f16, g=4>, tiles dealt round-robin over the splits "
                               "(the schedule of tc_decode_attention)",
                     "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "us_per_launch": round(partial_us, 3),
                     "bytes_per_launch": per_call_bytes,
                     "traffic": read_traffic(f"decode_partial_rr_n{n}_traffic.txt"),
                     "frac_partial_plus_combine": round(value / PEAK_GBS, 4),
                     "combine_us_per_call": round(ms * 1e3 / LAYERS - partial_us, 3)},
        "yardstick": {"what": "the partial kernel's loads alone (same grid, tile schedule, loads in flight), "
                              "36 distinct layers in one graph",
                      "us_per_launch": round(yard_us, 3),
                      "GB/s": round(per_call_bytes / (yard_us * 1e-6) / 1e9, 1),
                      "frac": round(per_call_bytes / (yard_us * 1e-6) / 1e9 / PEAK_GBS, 4),
                      "partial_over_yardstick": round(partial_us / yard_us, 4),
                      "empty_launch_us": round(result["ms_empty"] * 1e3 / LAYERS, 3),
                      "empty_launch_what": "an empty kernel of the partial's grid size, 36 dependent launches in "
                                           "one graph: what one launch costs in the chain before any work"},
    }
    if not args.no_reports:
        sweep = {}
        for m in SWEEP:
            r = result if m == n else measure_sweep(dev, m, max(20, args.steps // 4), 5, args.split, None, WARM_MS)
            sweep[str(m)] = summarize(r, decode_bytes(m))
        line["sweep_36_layers"] = sweep
        line["ragged_16"] = measure_ragged(dev, max(10, args.steps // 10))
        line["long_131072"] = {f"B{b}": measure_long(dev, b, max(10, args.steps // 10)) for b in (1, 4)}
        line["decode_append"] = measure_append(dev, n, max(20, args.steps // 4))
        line["torch_kernels_same_bytes"] = measure_torch_reads(dev, n)
        line["match_split"] = measure_match()
        line["prefill"] = measure_prefill(dev, args.steps)
        line["decode_step_model"] = measure_decode_step(dev, n)
        line["paged"] = measure_paged(dev, n, max(20, args.steps // 4))
    if not args.no_splice:
        line["splice"] = bench_splice(dev, max(5, args.steps // 10), 3)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(n, args.cpu_seconds)
        if "splice" in line:
            line["splice"]["cpu_baseline"] = cpu_splice_baseline(min(5.0, args.cpu_seconds))
        if "ragged_16" in line:
            line["ragged_16"]["cpu_baseline"] = cpu_ragged_baseline(min(5.0, args.cpu_seconds))
    print(json.dumps(line))


if __name__ == "__main__":
    main()
