"""Benchmark of the MI355X quantized decode hot path.

Default line: the Q6_K output-head GEMV (W 128256 x 4096 Q6_K, batch 1) --
algorithmic GB/s and fraction of the 8 TB/s HBM roofline -- plus, in
"workloads", the Q4_K 4096 x 4096 GEMV (cold and hot), the Qwen3Next-shaped
MoE layer at batch 1 and 256, the Nemotron-H-shaped MoE layer at batch 1024
(tokens/s) and the Llama-3.1-8B-layout decode token at position 4096.  Inputs are resident in HBM when timing starts; times are
HIP events around K launches on the stream the kernels run on.

The CPU baseline is the oracle (a C restatement of the reference's CPU
loops, not the reference itself) on the host cores, over a bounded sample.
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

from llambda_amd import ggml, native, synthetic  # noqa: E402
from llambda_amd.hip_backend import make_hip_session_packed  # noqa: E402
from llambda_amd.moe import HipMoeSession, synthetic_nemotron_h, synthetic_qwen3next  # noqa: E402

METRIC = "Dequant-GEMV GB/s (% HBM peak) + MoE layer tokens/s, 1 MI355X"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16 MFMA, MI355X
DTYPE = "f32 via bf16 hi+lo MFMA"  # x split into two bf16, exact bf16 codes, fp32 accumulation


def _cpu_facts():
    """Host cores, the CPU model, and the cores this process may use: its
    affinity set, capped by a cgroup CPU quota when one is set."""
    host = os.cpu_count() or 1
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else host
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as fh:
            q, period = fh.read().split()[:2]
            if q != "max":
                quota = max(1, int(int(q) / int(period)))
    except (OSError, ValueError):
        pass
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    threads = min(usable, quota) if quota else usable
    return {"host_cores": host, "usable_cores": usable, "cgroup_cpus": quota,
            "cpu_model": model, "threads": threads}


CPU = _cpu_facts()
CPU_THREADS = CPU["threads"]


def cpu_entry(value, unit, sample, kind="port"):
    """A cpu_baseline object: the oracle (a C restatement of the reference's
    CPU loops) on every core this process may use."""
    return {"value": value, "unit": unit, "cores": CPU_THREADS, "kind": kind, "sample": sample,
            "host_cores": CPU["host_cores"], "usable_cores": CPU["usable_cores"],
            "cgroup_cpus": CPU["cgroup_cpus"], "cpu_model": CPU["cpu_model"]}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _torch():
    import torch
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU (torch.cuda.is_available() is False)")
    return torch


class Timer:
    """HIP events on the stream the kernels are launched on: a dedicated
    (default-priority) stream, passed to the library by handle."""

    def __init__(self, torch):
        self.torch = torch
        self.stream = torch.cuda.Stream()
        self.handle = self.stream.cuda_stream
        assert self.handle, "a dedicated stream has a non-null handle"

    def time(self, fn, steps: int, warmup: int) -> float:
        torch = self.torch
        torch.cuda.synchronize()
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record(self.stream)
        for _ in range(steps):
            fn()
        stop.record(self.stream)
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / steps  # ms per step


def gemv_bytes(type_tag, rows, columns, tokens=1):
    return rows * ggml.row_bytes(type_tag, columns) + 4 * columns * tokens + 4 * rows * tokens


def bench_gemv(torch, timer, type_tag, rows, columns, steps, warmup, seed=1, copies=1,
               sustained=None, graph=False):
    """One GEMV; with copies > 1 each launch reads a different weight copy
    (rotation), so the 256 MB MALL cannot serve them.  sustained = (settle,
    launches): after the timed steps, `settle` more launches untimed, then
    `launches` timed ones (ms per launch in state["sustained_ms"]).  graph:
    the `steps` launches are captured into one HIP graph and the graph is
    replayed (a launch of a few microseconds otherwise waits on the host's
    enqueue of the next)."""
    rng = np.random.default_rng(seed)
    log(f"generating {copies} x {ggml.NAMES[type_tag]} {rows}x{columns}")
    sessions = []
    w = synthetic.packed(type_tag, rng, rows, columns)
    for c in range(copies):
        if c:
            w = synthetic.packed(type_tag, rng, rows, columns) if c < 4 else np.roll(w, 144 * 7)
        sessions.append(make_hip_session_packed(w, type_tag, rows, columns))
    x = torch.randn(columns, device="cuda", dtype=torch.float32)
    y = torch.empty(rows, device="cuda", dtype=torch.float32)
    state = {"i": 0}

    def step():
        s = sessions[state["i"] % copies]
        state["i"] += 1
        s.run_device(x.data_ptr(), y.data_ptr(), 1, timer.handle)

    if graph:
        timer.time(step, 1, warmup)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=timer.stream, capture_error_mode="relaxed"):
            for _ in range(steps):
                step()
        reps = 5
        with torch.cuda.stream(timer.stream):  # replays go to the current stream
            ms = timer.time(g.replay, reps, 2) / steps
    else:
        ms = timer.time(step, steps, warmup)
    if sustained:
        settle, launches = sustained
        state["sustained_ms"] = timer.time(step, launches, settle)
    for s in sessions:
        s.close()
    nbytes = gemv_bytes(type_tag, rows, columns)
    if sustained:
        return ms, nbytes, state["sustained_ms"]
    return ms, nbytes


def bench_stream_read(torch, timer, nbytes, steps, warmup, sustained):
    """llambda_hip_stream_read over one nbytes buffer: the read rate the device
    sustains, timed exactly as the GEMV beside it (ms per launch, then the
    sustained figure)."""
    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(7)
    out = torch.empty(native.STREAM_READ_WORDS, dtype=torch.int32, device="cuda")
    lib = native.lib()

    def step():
        if lib.llambda_hip_stream_read(buf.data_ptr(), nbytes, out.data_ptr(), timer.handle):
            raise RuntimeError(native.last_error())

    ms = timer.time(step, steps, warmup)
    settle, launches = sustained
    ms_sus = timer.time(step, launches, settle)
    del buf, out
    return ms, ms_sus


REPORT_WARMUP, REPORT_RUNS = 3, 20  # benchmark-gguf-projection-backends' defaults


def projection_report(torch, timer, name, type_tag, rows, columns, seed):
    """benchmark-gguf-projection-backends (llambda.lisp:4825-4949) for one
    synthetic tensor: the reference's deterministic input x[i] = ((17 i + 11)
    mod 257)/128 - 1 (:4870-4874), 3 warm-up and 20 timed runs per backend,
    ms per run, GFLOP/s = 2 N K / time, speedup over the CPU and the maximum
    absolute difference from the CPU output (:4752-4787).  Backends: the CPU
    oracle on the host's cores; the HIP session on device-resident x and y
    (HIP events); the HIP session through the synchronous host-pointer entry
    point the Lisp adapter calls (wall clock)."""
    import oracle
    rng = np.random.default_rng(seed)
    w = synthetic.packed(type_tag, rng, rows, columns)
    x_host = synthetic.reference_input(columns)
    flops = 2.0 * rows * columns
    y_cpu = np.empty(rows, np.float32)

    def cpu():
        y_cpu[:] = oracle.gemv(type_tag, w, rows, columns, x_host, threads=CPU_THREADS)

    ms_cpu = _per_call_us(cpu, REPORT_RUNS, REPORT_WARMUP) / 1e3
    sess = make_hip_session_packed(w, type_tag, rows, columns)
    x = torch.from_numpy(x_host).cuda()
    y = torch.empty(rows, device="cuda", dtype=torch.float32)
    ms_dev = timer.time(lambda: sess.run_device(x.data_ptr(), y.data_ptr(), 1, timer.handle),
                        REPORT_RUNS, REPORT_WARMUP)
    y_dev = y.cpu().numpy()
    y_host = np.empty(rows, np.float32)
    ms_host = _per_call_us(lambda: sess.run_into(y_host, x_host), REPORT_RUNS, REPORT_WARMUP) / 1e3
    sess.close()

    def row(backend, ms, out, **extra):
        r = {"backend": backend, "ms_per_run": round(ms, 4), "gflops": round(flops / ms / 1e6, 2),
             "speedup_vs_cpu": round(ms_cpu / ms, 2),
             "max_absolute_error": float(np.max(np.abs(out - y_cpu)))}
        r.update(extra)
        return r

    results = [row("CPU", ms_cpu, y_cpu, threads=CPU_THREADS, kind="oracle (C restatement)"),
               row("HIP", ms_dev, y_dev, pointers="device"),
               row("HIP", ms_host, y_host, pointers="host (synchronous, as run-hip-session-into)")]
    log(f"Projection {name!r} ({rows} x {columns}), {REPORT_WARMUP} warmup and "
        f"{REPORT_RUNS} timed runs")
    log(f"{'Backend':<12} {'ms/run':<12} {'GFLOP/s':<12} {'speedup':<10} max abs error")
    for r in results:
        label = r["backend"] + ("" if r["backend"] == "CPU" else
                                "/dev" if r["pointers"] == "device" else "/host")
        log(f"{label:<12} {r['ms_per_run']:<12.3f} {r['gflops']:<12.3f} "
            f"{r['speedup_vs_cpu']:<9.2f}x {r['max_absolute_error']:<14.6g}")
    return {"tensor": name, "type": ggml.NAMES[type_tag], "rows": rows, "columns": columns,
            "input": "x[i] = ((17 i + 11) mod 257) / 128 - 1", "warmup_runs": REPORT_WARMUP,
            "timed_runs": REPORT_RUNS, "results": results}


def bench_head_sampling(torch, timer, rows, columns, steps, warmup):
    """Output head then sample-token-id-from-logits on the device (top-k 40,
    top-p 0.9, temperature 1, repetition penalty over a 64-token history,
    random values from a seeded stream), one token per step, synchronous
    (the token reaches the host each step)."""
    from llambda_amd.sampling import HipSampler
    rng = np.random.default_rng(3)
    w = synthetic.packed(ggml.Q6_K, rng, rows, columns)
    sess = make_hip_session_packed(w, ggml.Q6_K, rows, columns)
    sampler = HipSampler(rows)
    x = torch.randn(columns, device="cuda", dtype=torch.float32)
    y = torch.empty(rows, device="cuda", dtype=torch.float32)
    history = rng.integers(0, rows, size=64).tolist()
    rolls = rng.random(steps + warmup).astype(np.float32)
    state = {"i": 0}

    def one(with_gemv):
        if with_gemv:
            sess.run_device(x.data_ptr(), y.data_ptr(), 1, timer.handle)
            timer.stream.synchronize()
        roll = float(rolls[state["i"] % len(rolls)])
        state["i"] += 1
        return sampler.sample(y.data_ptr(), device_count=rows, history=history, top_k=40,
                              top_p=0.9, temperature=1.0, random_value=roll)

    res = {}
    for with_gemv in (True, False):
        for _ in range(warmup):
            one(with_gemv)
        t0 = time.perf_counter()
        for _ in range(steps):
            one(with_gemv)
        res[with_gemv] = (time.perf_counter() - t0) / steps * 1e6
    sampler.close()
    sess.close()
    return {"workload": "Q6_K output head 128256x4096 + sampling (top-k 40, top-p 0.9, "
                        "temperature 1, 64-token repetition history, seeded random values), "
                        "token returned to the host every step",
            "us_per_token": round(res[True], 1), "us_sampling": round(res[False], 1),
            "tokens_per_s": round(1e6 / res[True], 1)}


def _per_call_us(fn, calls, warmup=5):
    for _ in range(warmup):
        fn()
    t0 = time.perf_counter()
    for _ in range(calls):
        fn()
    return (time.perf_counter() - t0) / calls * 1e6


def bench_boundary_gemv(rows, columns, calls):
    """The synchronous host-pointer entry point as the Lisp adapter calls it
    (run-hip-session-into: x copied in, the GEMV, y copied out, stream
    synchronised), Q4_K rows x columns."""
    rng = np.random.default_rng(5)
    sess = make_hip_session_packed(synthetic.packed(ggml.Q4_K, rng, rows, columns), ggml.Q4_K,
                                   rows, columns)
    x = synthetic.activations(rng, 1, columns)[0]
    y = np.empty(rows, dtype=np.float32)
    us = _per_call_us(lambda: sess.run_into(y, x), calls)
    sess.close()
    return us


def bench_boundary_moe(layer, calls):
    """llambda_hip_moe_session_run for one token from host memory, as the
    MoE hook calls it (synchronous)."""
    rng = np.random.default_rng(6)
    sess = HipMoeSession(layer)
    x = synthetic.activations(rng, 1, layer.hidden)[0]
    y = np.empty(layer.hidden, dtype=np.float32)
    us = _per_call_us(lambda: sess.run_into(y, x), calls)
    sess.close()
    return us


def cpu_gemv_baseline(type_tag, rows, columns, seconds):
    import oracle
    rng = np.random.default_rng(99)
    w = synthetic.packed(type_tag, rng, rows, columns)
    x = synthetic.activations(rng, 1, columns)[0]
    oracle.gemv(type_tag, w, rows, columns, x, threads=CPU_THREADS)  # warm the pool
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.gemv(type_tag, w, rows, columns, x, threads=CPU_THREADS)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return gemv_bytes(type_tag, rows, columns) * n / el / 1e9, n


def bench_moe(torch, timer, layer, tokens, steps, warmup, seed):
    rng = np.random.default_rng(seed)
    x_host = synthetic.activations(rng, tokens, layer.hidden)
    session = HipMoeSession(layer)
    x = torch.from_numpy(x_host).to("cuda")
    y = torch.empty_like(x)
    _, idx, _, _ = session.run(x_host, with_routing=True)

    def step():
        session.run_device(x.data_ptr(), y.data_ptr(), tokens, timer.handle)

    # the layer's upload leaves the GPU idle, and the first ~30 ms of launches
    # after idling run slower while the clocks come back: warm up for at
    # least 60 ms whatever the step count asks
    probe = timer.time(step, 3, 1)
    warmup = max(warmup, min(4000, int(60.0 / max(probe, 1e-3))))
    ms = timer.time(step, steps, warmup)
    session.sync(timer.handle)
    session.close()
    distinct = len(np.unique(idx))
    nbytes = (distinct * layer.expert_bytes() + layer.shared_bytes() + layer.router.nbytes
              + (layer.router_bias.nbytes if layer.router_bias is not None else 0)
              + 8 * tokens * layer.hidden)
    return ms, nbytes, distinct


def cpu_moe_baseline(layer, tokens_sample, seconds):
    import oracle
    rng = np.random.default_rng(5)
    x = synthetic.activations(rng, tokens_sample, layer.hidden)
    oracle.moe_forward(layer, x[:1], threads=CPU_THREADS)
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.moe_forward(layer, x[n % tokens_sample:n % tokens_sample + 1], threads=CPU_THREADS)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return n / el, n


LLAMA_CONTEXT = 4224  # cache slots: 4096 prefilled + the decoded token, rounded up


def bench_llama(torch, timer, steps, warmup):
    """Llama-3.1-8B-layout decode token at position 4096: random-init weights
    drawn on the device (Q4_K_M mix), fp32 cache slots 0..4095 ~ N(0, 1)."""
    from llambda_amd.llama import (LLAMA31_8B, HipLlamaSession, synthetic_llama_device,
                                   weight_bytes)
    c = LLAMA31_8B
    log("generating Llama-3.1-8B-layout weights on the device")
    w = synthetic_llama_device(31, c, np.random.default_rng(31))
    wbytes = weight_bytes(w)
    sess = HipLlamaSession(w, context=LLAMA_CONTEXT)
    del w
    torch.cuda.empty_cache()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(32)
    for layer in range(c.layer_count):
        k = torch.randn((c.kv_head_count, 4096, c.head_dim), device="cuda", generator=gen)
        v = torch.randn((c.kv_head_count, 4096, c.head_dim), device="cuda", generator=gen)
        torch.cuda.synchronize()
        sess.write_kv_device(layer, 0, 4096, k.data_ptr(), v.data_ptr())
    del k, v
    logits = torch.empty(c.vocab, device="cuda", dtype=torch.float32)
    pos, token = 4096, 1234
    res = {}
    for graph in (True, False):
        def step():
            sess.step_device(token, pos, logits.data_ptr(), timer.handle, graph=graph)
        # at least 60 ms of warm-up tokens, past the clocks' ramp after the
        # host-side set-up (the same rule as the MoE layers)
        probe = timer.time(step, 3, 1)
        res[graph] = timer.time(step, steps, max(warmup, min(400, int(60.0 / max(probe, 1e-3)))))
    sess.close()
    kv_bytes = 2 * c.layer_count * c.kv_head_count * (pos + 1) * c.head_dim * 4
    return res[True], res[False], wbytes, kv_bytes


def cpu_llama_baseline(seconds):
    """Oracle step of one 8B-shaped layer (cache at 4096) plus the head GEMV
    rate of the head workload: per-token = 32 layers + head."""
    import oracle
    from llambda_amd.llama import LLAMA31_8B, LlamaConfig, synthetic_llama
    c = LLAMA31_8B
    one = LlamaConfig(hidden=c.hidden, layer_count=1, head_count=c.head_count,
                      kv_head_count=c.kv_head_count, ffn=c.ffn, vocab=256,
                      rope_dimension=c.rope_dimension, context=4097)
    rng = np.random.default_rng(33)
    w = synthetic_llama(rng, one)
    kv = np.zeros((1, 2, c.kv_head_count, 4097, c.head_dim), dtype=np.float32)
    kv[:, :, :, :4096] = rng.standard_normal(size=kv[:, :, :, :4096].shape, dtype=np.float32)
    oracle.llama_step(w, kv, 5, 4096, threads=CPU_THREADS)
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.llama_step(w, kv, 5, 4096, threads=CPU_THREADS)
        n += 1
        if time.perf_counter() - t0 >= seconds:
            break
    t_layer = (time.perf_counter() - t0) / n
    head = synthetic.packed(ggml.Q6_K, rng, c.vocab, c.hidden)
    x = synthetic.activations(rng, 1, c.hidden)[0]
    t0 = time.perf_counter()
    oracle.gemv(ggml.Q6_K, head, c.vocab, c.hidden, x, threads=CPU_THREADS)
    t_head = time.perf_counter() - t0
    return 1.0 / (c.layer_count * t_layer + t_head), n


def load_traffic(name):
    """HBM bytes per launch measured with rocprofv3 counters (profiles/)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as fh:
            return json.load(fh).get(name)
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # (the default warmup covers the box's power-management transient: in a
    # fresh process, head launches 26-75 run ~15% slower than the settled
    # rate reached ~30 ms in)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--only", choices=["head", "report", "q4k", "moe", "llama", "copy", "none"],
                    default=None,
                    help="run one workload group only (profiling)")
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="bound on each CPU-baseline sample (0 disables)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              f"(the library runs on one GPU; sharding across GPUs is not implemented)", file=sys.stderr)
        return 2
    torch = _torch()
    if native.lib().llambda_hip_probe() != 1:
        raise SystemExit(f"no usable gfx950 device: {native.last_error()}")
    timer = Timer(torch)
    steps, warmup = args.steps, args.warmup
    workloads = []
    line = None

    if args.only in (None, "head"):
        rows, cols = 128256, 4096
        # the timed steps, then a sustained figure: a fresh process's first
        # ~100 ms of launches carry a power-management transient (launches
        # 26-75 run ~15% slower), so 800 launches are timed after 300 more
        ms, nbytes, ms_sus = bench_gemv(torch, timer, ggml.Q6_K, rows, cols, steps, warmup,
                                        sustained=(300, 800))
        gbs = nbytes / (ms * 1e-3) / 1e9
        gbs_sus = nbytes / (ms_sus * 1e-3) / 1e9
        log(f"Q6_K head: {ms * 1e3:.1f} us/launch, {gbs:.0f} GB/s; sustained "
            f"{ms_sus * 1e3:.1f} us/launch, {gbs_sus:.0f} GB/s")
        # the device's own ceiling: a plain read of as many bytes, timed alike
        rd_ms, rd_ms_sus = bench_stream_read(torch, timer, nbytes, steps, warmup, (300, 800))
        rd_gbs = nbytes / (rd_ms * 1e-3) / 1e9
        rd_gbs_sus = nbytes / (rd_ms_sus * 1e-3) / 1e9
        log(f"streaming read of {nbytes} B: {rd_ms * 1e3:.1f} us/launch, {rd_gbs:.0f} GB/s; "
            f"sustained {rd_ms_sus * 1e3:.1f} us, {rd_gbs_sus:.0f} GB/s")
        cpu = None
        if args.cpu_seconds > 0:
            cpu_gbs, n = cpu_gemv_baseline(ggml.Q6_K, rows, cols, args.cpu_seconds)
            cpu = cpu_entry(round(cpu_gbs, 3), "GB/s",
                            f"{n} full Q6_K 128256x4096 GEMVs, C restatement of the reference "
                            f"CPU loop (8-lane fma accumulator, row partition over "
                            f"{CPU_THREADS} threads); not the Lisp reference itself")
            log(f"CPU baseline: {cpu_gbs:.2f} GB/s over {n} runs")
        samp = bench_head_sampling(torch, timer, rows, cols, max(20, steps // 4), min(warmup, 5))
        workloads.append(samp)
        log(f"Q6_K head + sampling: {samp['us_per_token']} us per token "
            f"(sampling alone {samp['us_sampling']} us)")
        traffic = load_traffic("q6k_head")
        line = {
            "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1,
            "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": DTYPE,
            "data": "synthetic (seeded random Q6_K blocks, x ~ N(0,1))",
            "config": {"workload": "Q6_K output-head GEMV, W 128256x4096, batch 1",
                       "rows": rows, "columns": cols, "algorithmic_bytes": nbytes},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": traffic,
                         "ceiling": {"kernel": "llambda_hip_stream_read (each of 4096 waves "
                                               "streams one contiguous slice, 16-byte loads)",
                                     "bytes": nbytes, "GB/s": round(rd_gbs, 1),
                                     "frac_of_peak": round(rd_gbs / HBM_PEAK_GBS, 4),
                                     "gemv_frac_of_ceiling": round(gbs / rd_gbs, 4),
                                     "sustained_GB/s": round(rd_gbs_sus, 1),
                                     "gemv_sustained_frac_of_ceiling":
                                         round(gbs_sus / rd_gbs_sus, 4)}},
            "sustained": {"launches": 800, "after_launches": steps + warmup + 300,
                          "us_per_launch": round(ms_sus * 1e3, 2), "GB/s": round(gbs_sus, 1),
                          "frac": round(gbs_sus / HBM_PEAK_GBS, 4)},
            "cpu_baseline": cpu,
        }

    if args.only in (None, "report") and args.cpu_seconds > 0:
        reports = [projection_report(torch, timer, "output.weight", ggml.Q6_K, 128256, 4096, 41),
                   projection_report(torch, timer, "blk.0.attn_q.weight", ggml.Q4_K, 4096, 4096,
                                     42),
                   projection_report(torch, timer, "blk.0.ffn_down.weight", ggml.Q6_K, 4096,
                                     14336, 43)]
        if line is not None:
            line["projection_report"] = reports
        else:
            workloads.append({"workload": "projection report", "projection_report": reports})

    if args.only in (None, "q4k"):
        # launches of a few microseconds: timed as a replayed graph of 224
        # launches (two passes over the 112 cold copies), after ~60 ms of
        # warm-up launches (this follows the CPU baseline's seconds of host work)
        q4k_warm = max(warmup, 10000)
        ms_hot, nbytes = bench_gemv(torch, timer, ggml.Q4_K, 4096, 4096, 224, q4k_warm, graph=True)
        ms_cold, _ = bench_gemv(torch, timer, ggml.Q4_K, 4096, 4096, 224, q4k_warm, copies=112,
                                graph=True)
        for label, ms in (("hot (one weight copy, MALL-resident)", ms_hot),
                          ("cold (112 rotating copies, 1.06 GB)", ms_cold)):
            gbs = nbytes / (ms * 1e-3) / 1e9
            workloads.append({"workload": f"Q4_K GEMV 4096x4096 batch 1, {label}, timed as a "
                                          f"replayed graph of 224 launches",
                              "us_per_launch": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                              "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)})
            log(f"Q4_K 4096^2 {label}: {ms * 1e3:.2f} us, {gbs:.0f} GB/s")
        us = bench_boundary_gemv(4096, 4096, max(50, steps))
        workloads.append({"workload": "boundary: llambda_hip_session_run, Q4_K 4096x4096, host x "
                                      "and y (pinned copy in, GEMV storing into mapped host "
                                      "memory, synchronise), as run-hip-session-into calls it",
                          "us_per_call": round(us, 2),
                          "GB/s_incl_pcie": round(nbytes / (us * 1e-6) / 1e9, 1)})
        log(f"boundary session_run Q4_K 4096^2: {us:.1f} us per call")

    if args.only in (None, "moe"):
        rng = np.random.default_rng(2024)
        qwen = synthetic_qwen3next(rng)
        for tokens in (1, 256):
            ms, nbytes, distinct = bench_moe(torch, timer, qwen, tokens,
                                             max(10, steps // (8 if tokens > 1 else 1)),
                                             min(warmup, 10), 7 + tokens)
            entry = {"workload": f"Qwen3Next MoE layer (H2048, E512 top-10, ffn 512, shared 512, "
                                 f"Q4_K/Q6_K), batch {tokens}",
                     "ms_per_step": round(ms, 4), "tokens_per_s": round(tokens / (ms * 1e-3), 1),
                     "distinct_experts": distinct, "algorithmic_bytes": nbytes,
                     "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1)}
            if args.cpu_seconds > 0:
                tps, n = cpu_moe_baseline(qwen, 8, args.cpu_seconds / 2)
                entry["cpu_baseline"] = cpu_entry(round(tps, 2), "tokens/s",
                                                  f"{n} tokens, one at a time")
                entry["speedup_vs_cpu"] = round(entry["tokens_per_s"] / tps, 1)
            workloads.append(entry)
            log(f"qwen3next B={tokens}: {ms:.3f} ms, {entry['tokens_per_s']} tok/s")
        us = bench_boundary_moe(qwen, max(50, steps // 2))
        workloads.append({"workload": "boundary: llambda_hip_moe_session_run, Qwen3Next layer, "
                                      "one token from host memory (synchronous), as the MoE "
                                      "hook calls it",
                          "us_per_call": round(us, 2), "tokens_per_s": round(1e6 / us, 1)})
        log(f"boundary moe_session_run B=1: {us:.1f} us per call")
        del qwen
        rng = np.random.default_rng(2025)
        nem = synthetic_nemotron_h(rng)
        ms, nbytes, distinct = bench_moe(torch, timer, nem, 1024, max(5, steps // 20),
                                         min(warmup, 3), 11)
        entry = {"workload": "Nemotron-H MoE layer (H2688, E128 top-6 Zipf-biased, ffn 1856, "
                             "shared 3712, Q5_0), batch 1024",
                 "ms_per_step": round(ms, 3), "tokens_per_s": round(1024 / (ms * 1e-3), 1),
                 "distinct_experts": distinct, "algorithmic_bytes": nbytes,
                 "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1)}
        flops = 1024 * nem.flops_per_token()
        entry["algorithmic_flops"] = flops
        entry["TFLOP/s"] = round(flops / (ms * 1e-3) / 1e12, 1)
        entry["frac_mfma_bf16"] = round(flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)
        entry["frac_hbm"] = round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        if args.cpu_seconds > 0:
            tps, n = cpu_moe_baseline(nem, 8, args.cpu_seconds / 2)
            entry["cpu_baseline"] = cpu_entry(round(tps, 2), "tokens/s",
                                              f"{n} tokens, one at a time")
            entry["speedup_vs_cpu"] = round(entry["tokens_per_s"] / tps, 1)
        workloads.append(entry)
        log(f"nemotron B=1024: {ms:.3f} ms, {entry['tokens_per_s']} tok/s")

    if args.only in (None, "llama"):
        ms_g, ms_e, wbytes, kv_bytes = bench_llama(torch, timer, max(20, steps // 4), min(warmup, 5))
        total = wbytes + kv_bytes
        entry = {"workload": "Llama-3.1-8B-layout decode token at position 4096 (32 layers, "
                             "hidden 4096, 32/8 heads x 128, SwiGLU 14336, Q4_K_M mix, fp32 KV "
                             "cache), random-init, one HIP graph per token",
                 "ms_per_token": round(ms_g, 4), "tokens_per_s": round(1000.0 / ms_g, 1),
                 "ms_per_token_eager": round(ms_e, 4),
                 "weight_bytes": wbytes, "kv_bytes": kv_bytes,
                 "GB/s": round(total / (ms_g * 1e-3) / 1e9, 1),
                 "frac_hbm": round(total / (ms_g * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        if args.cpu_seconds > 0:
            tps, n = cpu_llama_baseline(args.cpu_seconds)
            entry["cpu_baseline"] = cpu_entry(round(tps, 3), "tokens/s",
                                              f"{n} oracle steps of one 8B-shaped layer at "
                                              f"position 4096, x32, plus one Q6_K head GEMV")
            entry["speedup_vs_cpu"] = round(entry["tokens_per_s"] / tps, 1)
        workloads.append(entry)
        log(f"llama 8B token: {ms_g:.3f} ms (graph), {ms_e:.3f} ms (eager), "
            f"{entry['GB/s']} GB/s")

    if args.only == "copy":
        # a plain device copy of known size: the HBM reference and the
        # calibration of the FETCH_SIZE / WRITE_SIZE counters
        n = 1 << 28  # floats (1 GiB)
        a = torch.empty(n, device="cuda", dtype=torch.float32).fill_(1.0)
        b = torch.empty_like(a)
        with torch.cuda.stream(timer.stream):
            ms = timer.time(lambda: b.copy_(a), max(5, steps // 20), 2)
        gbs = 2 * 4 * n / (ms * 1e-3) / 1e9
        workloads.append({"workload": "device copy 1 GiB -> 1 GiB (torch)", "ms_per_step": round(ms, 4),
                          "GB/s (read+write)": round(gbs, 1)})
        log(f"copy 1 GiB: {ms:.3f} ms, {gbs:.0f} GB/s read+write")

    if line is None:
        line = {"metric": METRIC, "value": None, "unit": "GB/s", "n_gpus": 1, "steps": steps,
                "warmup": warmup, "higher_is_better": True, "scaling": "weak",
                "vs_baseline": None, "dtype": DTYPE, "data": "synthetic",
                "config": {"workload": f"partial run ({args.only})"}}
    line["workloads"] = workloads
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
