#!/usr/bin/env python3
"""Benchmark of the LeVo2 elementwise / reduction / broadcast kernels on one MI355X.

Headline workload (one "step"): the SnakeBeta ladder of one 10.08 s Oobleck
VAE window, F32 (C, T) = (2048,252), (1024,504), (512,2016), (256,8064),
(128,48384), (128,483840), all six shapes in one batched launch
(levo_hip_snake_beta_batch; six single launches are timed beside it),
x ~ N(0,1), per-channel log-parameters ~ U(-0.5, 0.5), inputs resident in
HBM. `value` = ladder algorithmic bytes (read x + write y + parameters) per
step / time per step.

Also reported, per op (rotated buffer sets so that every timed launch reads
data untouched for >= 512 MB of traffic, i.e. from HBM, not the 256 MB
Infinity Cache): SnakeBeta 1 s config, Flow CFG+Euler (50 steps), residual +
RMSNorm / LayerNorm F16, CFG + softmax + argmax / top-50, Q8_0 / Q4_0
quantize / dequantize. Kernel durations come from HIP events recorded on the
stream the kernels run on (torch's current stream); a bounded spin kernel
queued first keeps the GPU busy while the host enqueues each timed region, so
the timed launches run back to back.

The CPU baseline is the CPU oracle (a port of the reference's ggml-cpu op
chains; ggml itself is not available) on this host's cores: the whole ladder
at every thread of the process's CPU share, a 32-channel slice of one rung at
one thread, and each other op at 1 and all threads.

The last stdout line is the JSON result: headline, roofline, the CPU leg and
a one-entry-per-op summary, kept under LINE_BUDGET bytes; the full per-op and
CPU tables go to --ops-out.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import importlib.util
import json
import math
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "achieved HBM GB/s & % of 8 TB/s peak per op; ms per 10.08 s VAE Snake ladder"
PEAK_GBPS = 8000.0
LADDER = [(2048, 252), (1024, 504), (512, 2016), (256, 8064), (128, 48384), (128, 483840)]
ROTATE_BYTES = 512 << 20


def load_binding():
    path = os.path.join(ROOT, "levo2.cpp_amd", "levo_hip.py")
    spec = importlib.util.spec_from_file_location("levo_hip_binding", path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules["levo_hip_binding"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg: str) -> None:
    sys.stderr.write(msg + "\n")
    sys.stderr.flush()


def snake_bytes(C, T):
    return 8 * C * T + 8 * C


class HeadStart:
    """Keeps the GPU busy with a bounded spin kernel while the host enqueues a
    timed region, so the timed launches run back-to-back and HIP events time
    the GPU, not the Python launch rate."""

    def __init__(self, torch):
        self.torch = torch
        torch.cuda._sleep(1000)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        cycles = 2_000_000
        a.record()
        torch.cuda._sleep(cycles)
        b.record()
        torch.cuda.synchronize()
        self.cycles_per_ms = cycles / max(a.elapsed_time(b), 1e-3)

    def __call__(self, ms: float):
        self.torch.cuda._sleep(int(self.cycles_per_ms * ms))


def time_region(torch, head, enqueue, host_ms_estimate):
    """Time enqueue() between two events after a spin head start."""
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    head(min(200.0, 2.0 * host_ms_estimate + 1.0))
    start.record()
    t0 = time.perf_counter()
    enqueue()
    host_ms = (time.perf_counter() - t0) * 1e3
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end), host_ms


def time_op(torch, head, launch, n_sets, warmup, steps):
    """Mean ms per launch of launch(set_index) over `steps` back-to-back launches
    cycling through n_sets buffer sets (>= 512 MB of traffic between reuses)."""
    t0 = time.perf_counter()
    for i in range(warmup):
        launch(i % n_sets)
    host_ms = (time.perf_counter() - t0) * 1e3 / max(warmup, 1) * steps
    torch.cuda.synchronize()

    def run():
        for i in range(steps):
            launch(i % n_sets)

    ms, host = time_region(torch, head, run, host_ms)
    if host > ms:  # the head start was too short: the GPU waited on the host
        ms, host = time_region(torch, head, run, host)
    return ms / steps


def op_entry(bytes_per_launch, ms, read=None, write=None, **extra):
    """One op's figures; read / write split the algorithmic bytes for the
    streaming ceiling of the same mix (default: all read)."""
    gbps = bytes_per_launch / (ms * 1e-3) / 1e9
    e = {"bytes_per_launch": int(bytes_per_launch), "us_per_launch": round(ms * 1e3, 3),
         "GB/s": round(gbps, 1), "frac": round(gbps / PEAK_GBPS, 4)}
    r = int(bytes_per_launch if read is None else read)
    e["read_bytes"], e["write_bytes"] = r, int(bytes_per_launch - r if write is None else write)
    e.update(extra)
    return e


_CEIL_CACHE = {}


def load_stream_lib():
    import ctypes
    path = os.path.join(ROOT, "levo2.cpp_amd", "liblevo_bench_stream.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(path)
    lib.levo_bench_stream.restype = ctypes.c_int
    lib.levo_bench_stream.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                      ctypes.c_void_p]
    return lib


def stream_ceiling(torch, head, dev, read_bytes, write_bytes, warmup, steps):
    """GB/s (read + write) of the best plain streaming launch moving the same
    bytes in the same mix: dwordx4 loads and stores, one, two or four vectors
    per thread (levo2.cpp_amd/bench/stream_ceiling.hip), rotated over >= 512 MB
    like the ops. What one launch of this size and mix reaches on this GPU."""
    rb, wb = int(read_bytes) // 16 * 16, int(write_bytes) // 16 * 16
    key = (rb, wb)
    if key in _CEIL_CACHE:
        return _CEIL_CACHE[key]
    lib = load_stream_lib()
    n = math.ceil(ROTATE_BYTES / max(rb + wb, 16)) + 1
    src = [torch.ones(max(rb, 16) // 4, dtype=torch.float32, device=dev) for _ in range(n)]
    dst = [torch.empty(max(wb, 16) // 4, dtype=torch.float32, device=dev) for _ in range(n)]
    stream = torch.cuda.current_stream().cuda_stream
    best = (0.0, 1)
    for vpt in (1, 2, 4):
        def launch(i, vpt=vpt):
            if lib.levo_bench_stream(src[i].data_ptr(), dst[i].data_ptr(), rb, wb, vpt, stream) != 0:
                raise RuntimeError("levo_bench_stream failed")
        ms = time_op(torch, head, launch, n, warmup, max(steps, 50))
        gbps = (rb + wb) / (ms * 1e-3) / 1e9
        if gbps > best[0]:
            best = (round(gbps, 1), vpt)
    del src, dst
    torch.cuda.empty_cache()
    _CEIL_CACHE[key] = best
    return best


def add_ceilings(torch, head, dev, ops, warmup, steps):
    """Annotate every HBM-bound op entry with the streaming ceiling of its byte
    count and read / write mix (ceiling_GB/s) and its fraction of it."""
    for entry in ops.values():
        entries = entry.values() if "bytes_per_launch" not in entry else [entry]
        for e in entries:
            if isinstance(e, dict) and "bytes_per_launch" in e and e.get("bound") not in ("mfma", "latency", "valu"):
                c, vpt = stream_ceiling(torch, head, dev, e.get("read_bytes", e["bytes_per_launch"]),
                                        e.get("write_bytes", 0), warmup, steps)
                e["ceiling_GB/s"] = c
                e["ceiling_vectors_per_thread"] = vpt
                e["of_ceiling"] = round(e["GB/s"] / c, 3)


def cpu_share():
    """Threads of the CPU share this process may use: its affinity set,
    narrowed by OMP_NUM_THREADS when the environment sets one (a host that
    shares its cores between GPUs sets it to one GPU's share)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    try:
        omp = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        omp = 0
    return max(1, min(n, omp) if omp > 0 else n)


def cpu_model():
    """The host CPU as lscpu names it (model, sockets, cores, threads)."""
    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    model = info.get("Model name")
    if not model and os.path.exists("/proc/cpuinfo"):
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    return {"model": model, "sockets": info.get("Socket(s)"), "cores_per_socket": info.get("Core(s) per socket"),
            "threads_per_core": info.get("Thread(s) per core"), "nproc": os.cpu_count()}


class pinned:
    """Runs the block on the first `threads` CPUs of the allowed set (the
    reference pins its CPU runs with taskset)."""

    def __init__(self, threads):
        self.threads = threads

    def __enter__(self):
        try:
            self.saved = os.sched_getaffinity(0)
            os.sched_setaffinity(0, sorted(self.saved)[: self.threads])
        except (AttributeError, OSError):
            self.saved = None
        return self

    def __exit__(self, *exc):
        if self.saved is not None:
            os.sched_setaffinity(0, self.saved)


def median_seconds(fn, warmup=3, runs=10):
    """3 warm-ups, then the median wall time of `runs` timed calls."""
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times))


def split_rows(n, parts):
    step = -(-n // parts)
    return [(i, min(n, i + step)) for i in range(0, n, step)]


# ---------------------------------------------------------------------------------------
def bench_ladder(torch, hip, head, dev, warmup, steps):
    g = torch.Generator(device=dev)
    g.manual_seed(20250101)
    rng = np.random.default_rng(7)
    per_set = sum(snake_bytes(C, T) for C, T in LADDER)
    n_sets = max(2, math.ceil(ROTATE_BYTES / per_set) + 1)
    sets = []
    for s in range(n_sets):
        tensors = []
        for C, T in LADDER:
            x = torch.randn((C, T), generator=g, device=dev, dtype=torch.float32)
            a = torch.from_numpy(rng.uniform(-0.5, 0.5, C).astype(np.float32)).to(dev)
            b = torch.from_numpy(rng.uniform(-0.5, 0.5, C).astype(np.float32)).to(dev)
            tensors.append((x, a, b, torch.empty_like(x)))
        sets.append(tensors)
    torch.cuda.synchronize()

    def ladder_batch(s):  # the headline: one launch over the six shapes
        hip.snake_beta_batch(sets[s])

    def ladder_six(s):  # one launch per shape
        for x, a, b, y in sets[s]:
            hip.snake_beta(x, a, b, y)

    def timed(ladder):
        t0 = time.perf_counter()
        for i in range(warmup):
            ladder(i % n_sets)
        host_ms = (time.perf_counter() - t0) * 1e3 / max(warmup, 1) * steps
        torch.cuda.synchronize()

        def run():
            for i in range(steps):
                ladder(i % n_sets)

        # timed region: K ladder steps back to back, events on the kernels' stream
        ms, host = time_region(torch, head, run, host_ms)
        if host > ms:
            ms, host = time_region(torch, head, run, host)
        return ms

    ms_six = timed(ladder_six)
    wall0 = time.perf_counter()
    ms_total = timed(ladder_batch)
    wall_ms = (time.perf_counter() - wall0) * 1e3
    host = [(t[0].cpu().numpy(), t[1].cpu().numpy(), t[2].cpu().numpy()) for t in sets[0]]
    # per-shape launch durations: each shape K times back to back over its own
    # rotation (>= 512 MB between reuses of a buffer)
    per_shape = {}
    shape_ms = []
    for j, (C, T) in enumerate(LADDER):
        n = max(2, math.ceil(ROTATE_BYTES / snake_bytes(C, T)) + 1)
        xs = [sets[0][j][0]] + [torch.randn((C, T), generator=g, device=dev) for _ in range(n - 1)]
        ys = [torch.empty((C, T), device=dev) for _ in range(n)]
        a, b = sets[0][j][1], sets[0][j][2]
        ms = time_op(torch, head, lambda i: hip.snake_beta(xs[i], a, b, ys[i]), n, warmup, max(steps, n))
        per_shape[f"{C}x{T}"] = op_entry(snake_bytes(C, T), ms, read=4 * C * T + 8 * C, rotated_sets=n)
        shape_ms.append(ms)
        del xs, ys
    del sets
    torch.cuda.empty_cache()
    return dict(ms_per_step=ms_total / steps, ms_per_step_six=ms_six / steps, wall_ms=wall_ms, per_shape=per_shape,
                ladder_bytes=per_set, host=host, n_sets=n_sets, dominant=(LADDER[-1], shape_ms[-1]))


def bench_snake_1s(torch, hip, head, dev, warmup, steps):
    C, T = 128, 48000
    per = snake_bytes(C, T)
    n = math.ceil(ROTATE_BYTES / per) + 1
    rng = np.random.default_rng(11)
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    bufs = [(torch.randn((C, T), generator=g, device=dev), torch.from_numpy(rng.uniform(-0.5, 0.5, C).astype(np.float32)).to(dev),
             torch.from_numpy(rng.uniform(-0.5, 0.5, C).astype(np.float32)).to(dev)) for _ in range(n)]
    outs = [torch.empty((C, T), device=dev) for _ in range(n)]
    ms = time_op(torch, head, lambda i: hip.snake_beta(bufs[i][0], bufs[i][1], bufs[i][2], outs[i]), n, warmup, steps)
    return op_entry(per, ms, read=4 * C * T + 8 * C, shape=[C, T], dtype="f32")


def bench_flow(torch, hip, head, dev, warmup, steps):
    n_el, nsteps = 64 * 2520, 50
    per = 16 * n_el
    n_sets = math.ceil(ROTATE_BYTES / (per * nsteps)) + 1
    g = torch.Generator(device=dev)
    g.manual_seed(50)
    xs = [torch.randn(n_el, generator=g, device=dev) for _ in range(n_sets)]
    vs = [[(torch.randn(n_el, generator=g, device=dev), torch.randn(n_el, generator=g, device=dev))
           for _ in range(nsteps)] for _ in range(n_sets)]
    dt = float(np.float32(1) / np.float32(nsteps))

    def solve(s):
        for k in range(nsteps):
            hip.flow_cfg_euler(xs[s], vs[s][k][0], vs[s][k][1], n_el, 1.5, dt)

    # one launch per Euler step: mean kernel time over back-to-back launches
    step_ms = time_op(torch, head, lambda i: hip.flow_cfg_euler(xs[i % n_sets], vs[i % n_sets][i % nsteps][0],
                                                                 vs[i % n_sets][i % nsteps][1], n_el, 1.5, dt),
                      n_sets * nsteps, warmup, max(steps, 50))
    reps = max(1, steps // 5)
    solve_ms = time_op(torch, head, solve, n_sets, 1, reps)
    # the same 50 launches captured into a HIP graph per buffer set and
    # replayed with the sets rotated as above, so both figures see the same
    # cache state
    graph_ms = None
    try:
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        graphs = []
        for s_ in range(n_sets):
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                solve(s_)
            graphs.append(graph)
        torch.cuda.synchronize()
        for graph in graphs:
            graph.replay()
        torch.cuda.synchronize()
        graph_ms = time_op(torch, head, lambda i: graphs[i].replay(), n_sets, 1, reps)
    except Exception as e:  # graph capture is an extra measurement only
        log(f"flow graph capture skipped: {e}")
    e = op_entry(per, step_ms, read=12 * n_el, shape=[1, 64, 2520], dtype="f32",
                 solve_50_steps_ms=round(solve_ms, 4),
                 solve_50_steps_GBps=round(per * nsteps / (solve_ms * 1e-3) / 1e9, 1))
    if graph_ms is not None:
        e["solve_50_steps_graph_ms"] = round(graph_ms, 4)
        e["solve_50_steps_graph_GBps"] = round(per * nsteps / (graph_ms * 1e-3) / 1e9, 1)
    return e


def bench_flow_window(torch, hip, binding, head, dev, warmup, steps):
    """Device-resident Flow step at LeVo's window: estimator rows of
    24 | 64 | 2048 | 64 = 2200 floats, 1000 frames, 250 in-context frames,
    batch 2 (CFG 1.5). `us_per_launch`: levo_hip_flow_step (a middle step:
    velocity slice + CFG + Euler + next state columns), buffers rotated over
    >= 512 MB. `assemble_us`: levo_hip_flow_assemble_input, once per window.
    `replaced_copies_us`: the 17.6 MB host-to-device + 17.6 MB device-to-host
    pinned copies the reference makes per step instead."""
    F, L, M, C, P = 1000, 64, 24, 2048, 250
    H = M + 2 * L + C
    step_bytes = 4 * L * (2 * F + (F - P) + 2 * P + F + 2 * F)
    n_step = math.ceil(ROTATE_BYTES / step_bytes) + 1
    big = torch.empty((n_step, 2, 2, F, H), dtype=torch.float32, device=dev)  # [set][mi|out][batch][frame][col]
    big[:, :, :, :, H - L:].normal_()
    g = torch.Generator(device=dev)
    g.manual_seed(2200)
    mk = lambda *shape: torch.randn(shape, generator=g, device=dev)
    noise, ctx, mask, cond = mk(F, L), mk(F, L), mk(F, M), mk(F, C)
    states = [mk(F, L) for _ in range(n_step)]
    args = []
    for i in range(n_step):
        a = binding.FlowStepArgs()
        a.state, a.output, a.out_pitch, a.vel_col = states[i].data_ptr(), big[i, 1].data_ptr(), H, H - L
        a.batch, a.guidance, a.frames, a.latent, a.step, a.steps = 2, 1.5, F, L, 20, 50
        a.noise, a.context, a.prefix_frames, a.sigma_min = noise.data_ptr(), ctx.data_ptr(), P, 1e-4
        a.next_input, a.in_pitch, a.state_col = big[i, 0].data_ptr(), H, H - L
        args.append(a)
    step_ms = time_op(torch, head, lambda i: hip.flow_step(args[i]), n_step, warmup, max(steps, 100))

    asm_bytes = 4 * (2 * F * H + F * M + 2 * F * L + F * C + F * L + 2 * P * L)
    n_asm = math.ceil(ROTATE_BYTES / asm_bytes) + 1
    mis = torch.empty((n_asm, 2, F, H), dtype=torch.float32, device=dev)
    asm = []
    for i in range(n_asm):
        a = binding.FlowInputArgs()
        a.model_input, a.batch, a.frames = mis[i].data_ptr(), 2, F
        a.mask_embedding, a.mask_dim, a.context, a.latent = mask.data_ptr(), M, ctx.data_ptr(), L
        a.conditioning, a.condition_width = cond.data_ptr(), C
        a.state, a.noise, a.prefix_frames = states[i % n_step].data_ptr(), noise.data_ptr(), P
        a.step, a.steps, a.sigma_min = 0, 50, 1e-4
        asm.append(a)
    asm_ms = time_op(torch, head, lambda i: hip.flow_assemble_input(asm[i]), n_asm, warmup, max(steps, 50))
    del mis

    host = torch.empty((2, F, H), dtype=torch.float32).pin_memory()
    dbuf = big[0, 0]
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 10
    a.record()
    for _ in range(reps):
        dbuf.copy_(host, non_blocking=True)
        host.copy_(big[0, 1], non_blocking=True)
    b.record()
    torch.cuda.synchronize()
    copies_ms = a.elapsed_time(b) / reps
    del big
    return op_entry(step_bytes, step_ms, shape=[2, F, H], dtype="f32", prefix_frames=P, guidance=1.5,
                    assemble_us=round(asm_ms * 1e3, 3),
                    assemble_GBps=round(asm_bytes / (asm_ms * 1e-3) / 1e9, 1), assemble_bytes=asm_bytes,
                    window_50_steps_us=round((asm_ms + 50 * step_ms) * 1e3, 2),
                    replaced_copies_us=round(copies_ms * 1e3, 1), bound="latency")


def bench_norm(torch, hip, head, dev, warmup, steps, layer, rows, D, f16=True):
    """Residual + RMS / LayerNorm over [rows, D]: F16 activations and
    parameters (the LeLM norms), or F32 (f16=False: the Flow estimator's
    LayerNorm, [2 x 1000 frames, 2200])."""
    es = 2 if f16 else 4
    per = 4 * es * rows * D + ((2 if layer else 1) * es * D)
    n = max(2, math.ceil(ROTATE_BYTES / per) + 1) if rows > 2 else 64
    g = torch.Generator(device=dev)
    g.manual_seed(rows * D + layer)
    dt = torch.float16 if f16 else torch.float32
    mk = lambda shape, s=1.0, m=0.0: (torch.randn(shape, generator=g, device=dev) * s + m).to(dt)
    w, b = mk(D, 0.02, 1.0), mk(D, 0.02)
    sets = [(mk((rows, D)), mk((rows, D)), torch.empty((rows, D), device=dev, dtype=dt),
             torch.empty((rows, D), device=dev, dtype=dt)) for _ in range(n)]
    t = 1 if f16 else 0
    eps = 1e-6 if f16 else 1e-5  # the LeLM's and the Flow estimator's
    if layer:
        fn = lambda i: hip.layer_norm(t, sets[i][0], sets[i][1], w, b, t, sets[i][2], sets[i][3], rows, D, eps)
    else:
        fn = lambda i: hip.rms_norm(t, sets[i][0], sets[i][1], w, t, sets[i][2], sets[i][3], rows, D, eps)
    ms = time_op(torch, head, fn, n, warmup, max(steps, 50))
    return op_entry(per, ms, read=per - 2 * es * rows * D, shape=[rows, D],
                    dtype=("f16" if f16 else "f32") + " io / f32 accumulate")


def modulated_norm_args(torch, binding, dev, g, rows, D, rpb, x, d, h, y, keep):
    """levo_hip_modulated_norm_args of a Flow estimator block boundary: gate /
    scale / shift are chunks 2 / 4 / 3 of a [batch][6 D] time modulation plus
    the block's learned [6 D] table (modulation_chunk)."""
    batches = rows // rpb
    tm = torch.randn((batches, 6 * D), generator=g, device=dev) * 0.3
    table = torch.randn(6 * D, generator=g, device=dev) * 0.3
    gamma = torch.randn(D, generator=g, device=dev) * 0.02 + 1
    beta = torch.randn(D, generator=g, device=dev) * 0.02
    keep.extend([tm, table, gamma, beta])
    vec = lambda k: binding.BatchVector(tm.data_ptr() + 4 * k * D, 6 * D, table.data_ptr() + 4 * k * D)
    a = binding.ModulatedNormArgs()
    a.x, a.delta, a.gate = x.data_ptr(), d.data_ptr(), vec(2)
    a.gamma, a.beta, a.param_type = gamma.data_ptr(), beta.data_ptr(), 0
    a.scale, a.shift = vec(4), vec(3)
    a.h_out, a.y = h.data_ptr(), y.data_ptr()
    a.rows, a.rows_per_batch, a.dim, a.eps = rows, rpb, D, 1e-5
    return a


def bench_norm_modulated(torch, hip, binding, head, dev, warmup, steps):
    """The Flow estimator's block boundary, [2 x 1000 frames, 2200] F32: gated
    residual + LayerNorm + AdaLN modulation in one launch
    (levo_hip_residual_layer_norm_modulated)."""
    rows, D, rpb = 2000, 2200, 1000
    row_bytes = 16 * rows * D                 # read x, delta; write h, y
    vec_bytes = 8 * D + 3 * (2 * D * 4 + D * 4)  # gamma, beta; 3 x (2 dynamic rows + learned)
    per = row_bytes + vec_bytes
    n = math.ceil(ROTATE_BYTES / per) + 1
    g = torch.Generator(device=dev)
    g.manual_seed(2200)
    keep = []
    args = []
    for _ in range(n):
        x, d = torch.randn((rows, D), generator=g, device=dev), torch.randn((rows, D), generator=g, device=dev)
        h, y = torch.empty_like(x), torch.empty_like(x)
        keep.extend([x, d, h, y])
        args.append(modulated_norm_args(torch, binding, dev, g, rows, D, rpb, x, d, h, y, keep))
    ms = time_op(torch, head, lambda i: hip.layer_norm_modulated(args[i]), n, warmup, max(steps, 50))
    e = op_entry(per, ms, read=per - 8 * rows * D, shape=[rows, D], dtype="f32 io / f32 accumulate")
    e["replaces"] = ("ggml_mul(out, gate), ggml_add(., residual), ggml_norm, ggml_mul(gamma), ggml_add(beta), "
                     "ggml_mul(1 + scale), ggml_add(shift): 3 full-tensor passes with the plain fused LayerNorm")
    return e


def bench_sample(torch, hip, binding, head, dev, warmup, steps):
    P, S, V, cap = 750, 3, 16384, 64
    rows = P * S
    reads = 2 * rows * V * 4
    writes = rows * (4 + 4 + 4 + 4 + 50 * (4 + 4))  # best, count, max, lse, 50 x (id, prob)
    per = reads + writes
    n = math.ceil(ROTATE_BYTES / reads) + 1
    g = torch.Generator(device=dev)
    g.manual_seed(750)
    sets = [(torch.randn((rows, V), generator=g, device=dev) * 3, torch.randn((rows, V), generator=g, device=dev) * 3)
            for _ in range(n)]
    best = torch.empty(rows, dtype=torch.int32, device=dev)
    count = torch.empty(rows, dtype=torch.int32, device=dev)
    ids = torch.empty((rows, cap), dtype=torch.int32, device=dev)
    probs = torch.empty((rows, cap), dtype=torch.float32, device=dev)
    mx = torch.empty(rows, dtype=torch.float32, device=dev)
    lse = torch.empty(rows, dtype=torch.float32, device=dev)
    args = []
    for c, u in sets:
        a = binding.SampleArgs()
        a.cond, a.uncond, a.rows, a.vocab, a.row_pitch = c.data_ptr(), u.data_ptr(), rows, V, V
        a.cfg_scale, a.temperature, a.n_streams = 1.5, 0.9, 3
        for s in range(3):
            a.top_k[s] = 50
        a.best, a.count, a.cand_ids, a.cand_probs = best.data_ptr(), count.data_ptr(), ids.data_ptr(), probs.data_ptr()
        a.row_max, a.row_lse, a.capacity = mx.data_ptr(), lse.data_ptr(), cap
        args.append(a)
    ms = time_op(torch, head, lambda i: hip.cfg_sample(args[i]), n, warmup, steps)
    return op_entry(per, ms, read=reads, shape=[P, 2, S, V], dtype="f32", top_k=50, temperature=0.9)


def bench_decode_step(torch, hip, binding, head, dev, warmup, steps):
    """Sampling of one LeLM decode step on the device: 1 position x 3 streams
    x 16385 ids, CFG s = 1.5, penalty window 50, a 3-id ignore list, top-k
    50/1/1, T = 0.9, through levo_hip_sample_step (rows split into one-wave
    parts of 512 ids, then one join-and-draw workgroup per row), the path the
    C++ Sampler takes. Latency-bound (393 KB per step). `us_per_launch`: the
    step; `cfg_sample_plus_draw_us`: the same step as levo_hip_cfg_sample +
    levo_hip_sample_draw back to back; `roundtrip_us`: median wall time from
    the first launch until the 3 ids and draw counts are in pinned host memory
    (Python launch overhead included); `graph_roundtrip_us`: the same with the
    step and both copies captured once into a HIP graph and replayed."""
    S, V, cap = 3, 16385, 64
    n = 64
    g = torch.Generator(device=dev)
    g.manual_seed(V)
    sets = [(torch.randn((S, V), generator=g, device=dev) * 3, torch.randn((S, V), generator=g, device=dev) * 3)
            for _ in range(n)]
    recent = torch.randint(0, V - 1, (S, 50), generator=g, device=dev, dtype=torch.int64)
    ignore = torch.tensor([0, 1, 2], dtype=torch.int64, device=dev)
    bits = torch.randint(-2 ** 62, 2 ** 62, (S,), generator=g, device=dev, dtype=torch.int64)
    best = torch.empty(S, dtype=torch.int32, device=dev)
    count = torch.empty(S, dtype=torch.int32, device=dev)
    ids = torch.empty((S, cap), dtype=torch.int32, device=dev)
    lg = torch.empty((S, cap), dtype=torch.float32, device=dev)
    mx = torch.empty(S, dtype=torch.float32, device=dev)
    tokens = torch.empty(S, dtype=torch.int64, device=dev)
    draws = torch.empty(S, dtype=torch.int32, device=dev)
    sargs = []
    for c, u in sets:
        a = binding.SampleArgs()
        a.cond, a.uncond, a.rows, a.vocab, a.row_pitch = c.data_ptr(), u.data_ptr(), S, V, V
        a.cfg_scale, a.temperature, a.n_streams = 1.5, 0.9, S
        a.top_k[0], a.top_k[1], a.top_k[2] = 50, 1, 1
        a.recent, a.n_recent, a.repetition_penalty, a.penalty_limit = recent.data_ptr(), 50, 1.1, V - 1
        a.ignore, a.n_ignore = ignore.data_ptr(), 3
        a.best, a.count, a.cand_ids, a.cand_logits = best.data_ptr(), count.data_ptr(), ids.data_ptr(), lg.data_ptr()
        a.row_max, a.capacity = mx.data_ptr(), cap
        sargs.append(a)
    d = binding.DrawArgs()
    d.best, d.count, d.cand_ids, d.cand_logits, d.row_max = (best.data_ptr(), count.data_ptr(), ids.data_ptr(),
                                                             lg.data_ptr(), mx.data_ptr())
    d.rows, d.capacity, d.temperature, d.use_sampling = S, cap, 0.9, 1
    d.bits, d.tokens, d.draws = bits.data_ptr(), tokens.data_ptr(), draws.data_ptr()

    def two_launches(i):
        hip.cfg_sample(sargs[i])
        hip.sample_draw(d)

    device_ms = time_op(torch, head, two_launches, n, warmup, max(steps, 200))
    sample_ms = time_op(torch, head, lambda i: hip.cfg_sample(sargs[i]), n, warmup, max(steps, 200))
    # the step through levo_hip_sample_step (part launch + join-and-draw launch)
    ws_bytes = hip.sample_step_workspace_bytes(S, V)
    ws = torch.empty((ws_bytes + 15) // 16 * 4, dtype=torch.float32, device=dev)

    def step(i):
        hip.sample_step(sargs[i], d, ws, ws_bytes)

    split_ms = time_op(torch, head, step, n, warmup, max(steps, 200))
    h_tok = torch.empty(S, dtype=torch.int64, pin_memory=True)
    h_draws = torch.empty(S, dtype=torch.int32, pin_memory=True)
    stream = torch.cuda.current_stream()
    walls = []
    for i in range(warmup + 200):
        stream.synchronize()
        t0 = time.perf_counter()
        step(i % n)
        h_tok.copy_(tokens, non_blocking=True)
        h_draws.copy_(draws, non_blocking=True)
        stream.synchronize()
        walls.append(time.perf_counter() - t0)
    roundtrip_ms = float(np.median(walls[warmup:])) * 1e3
    # the same step and copies captured once into a HIP graph and replayed
    graph_rt_ms = None
    try:
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            step(0)
            h_tok.copy_(tokens, non_blocking=True)
            h_draws.copy_(draws, non_blocking=True)
        torch.cuda.synchronize()
        gwalls = []
        for i in range(warmup + 200):
            stream.synchronize()
            t0 = time.perf_counter()
            graph.replay()
            stream.synchronize()
            gwalls.append(time.perf_counter() - t0)
        graph_rt_ms = float(np.median(gwalls[warmup:])) * 1e3
    except Exception as e:  # graph capture is an extra measurement only
        log(f"decode-step graph capture skipped: {e}")
    per = 2 * S * V * 4 + S * 50 * 8 + 3 * 8 + S * (4 + 4 + 4 + cap * 8 + 8 + 8 + 4)
    return op_entry(per, split_ms, shape=[1, 2, S, V], dtype="f32 logits / f64 weights", top_k=[50, 1, 1],
                    temperature=0.9, cfg_sample_plus_draw_us=round(device_ms * 1e3, 3),
                    cfg_sample_us=round(sample_ms * 1e3, 3), sample_draw_us=round((device_ms - sample_ms) * 1e3, 3),
                    roundtrip_us=round(roundtrip_ms * 1e3, 2),
                    graph_roundtrip_us=None if graph_rt_ms is None else round(graph_rt_ms * 1e3, 2),
                    bytes_to_host=S * (8 + 4),
                    bound="latency")


def bench_mul_mat(torch, hip, head, dev, warmup, steps):
    """Q8_0 decode mat-vec at LeLM medium's matrices (hidden 1536, FFN 8960,
    codebook head 16385) with the CFG pair of activation columns, already
    quantized to Q8_0; weights rotated over >= 512 MB. `layer`: one decoder
    layer's decode step as it runs: the 4 activation quantizations
    (levo_hip_quantize_chunk: attention input, attention output, FFN input,
    FFN hidden) and the 7 matrices (q, k, v, o, gate, up, down); then the
    same work in 5 launches (levo_hip_mul_mat_q8_0_multi). `*_packed`: the
    same matrices repacked once at load (levo_hip_repack_q8_0) with the
    activations as columns (levo_hip_quantize_q8_0_columns)."""
    shapes = {"attn_1536x1536": (1536, 1536), "ffn_up_8960x1536": (8960, 1536),
              "ffn_down_1536x8960": (1536, 8960), "head_16385x1536": (16385, 1536)}
    n_vec = 2
    out = {}
    g = torch.Generator(device=dev)
    g.manual_seed(34)

    def mk(rows, k, n):
        nbytes = rows * (k // 32) * 34
        stride = (nbytes + 255) // 256 * 256
        w = torch.randint(-127, 128, (n, stride), generator=g, device=dev, dtype=torch.int8).view(torch.uint8)
        scale = torch.full((rows * (k // 32),), 0x2000, dtype=torch.int16, device=dev)  # F16 2^-7 scales
        for i in range(n):
            w[i, :nbytes].view(rows * (k // 32), 34)[:, :2] = scale.view(torch.uint8).view(-1, 2)
        return w

    def quantized(k):
        x = torch.randn((n_vec, k), generator=g, device=dev)
        xb = torch.empty(n_vec * (k // 32) * 34 + 16, dtype=torch.uint8, device=dev)
        hip.quantize_chunk(8, x, xb, 0, n_vec, k)
        return x, xb

    def columns(x, k):
        xc = torch.empty(n_vec * (k // 32) * 36, dtype=torch.uint8, device=dev)
        hip.quantize_q8_0_columns(x, k, xc, n_vec, k)
        return xc

    def repacked(w, rows, k):
        p = torch.empty_like(w)
        for i in range(w.shape[0]):
            hip.repack_q8_0(w[i], p[i], rows, k)
        return p

    for name, (rows, k) in shapes.items():
        nbytes = rows * (k // 32) * 34
        per = nbytes + n_vec * (k // 32) * 34 + n_vec * rows * 4
        n = math.ceil(ROTATE_BYTES / nbytes) + 1
        w = mk(rows, k, n)
        x, xb = quantized(k)
        y = torch.empty((n_vec, rows), device=dev)
        ms = time_op(torch, head, lambda i: hip.mul_mat_q8_0(w[i].data_ptr(), xb, y, rows, rows, k, n_vec),
                     n, warmup, max(steps, 50))
        out[name] = op_entry(per, ms, read=per - n_vec * rows * 4, shape=[rows, k], n_vec=n_vec,
                             dtype="q8_0 weights / q8_0 activations")
        # the same matrix repacked once at load (levo_hip_repack_q8_0), the
        # activations as columns (levo_hip_quantize_q8_0_columns)
        p = repacked(w, rows, k)
        del w
        xc = columns(x, k)
        per_p = nbytes + xc.numel() + n_vec * rows * 4
        ms = time_op(torch, head, lambda i: hip.mul_mat_q8_0_packed(p[i].data_ptr(), xc, y, rows, rows, k, n_vec),
                     n, warmup, max(steps, 50))
        out[name + "_packed"] = op_entry(per_p, ms, read=per_p - n_vec * rows * 4, shape=[rows, k], n_vec=n_vec,
                                         dtype="q8_0 weights (packed) / q8_0 activation columns")
        del p
    layer = [(1536, 1536)] * 4 + [(8960, 1536)] * 2 + [(1536, 8960)]
    layer_bytes = sum(r * (k // 32) * 34 + n_vec * (k // 32) * 34 + n_vec * r * 4 for r, k in layer)
    layer_bytes += 3 * n_vec * 1536 * (4 + 34 / 32) + n_vec * 8960 * (4 + 34 / 32)
    n = math.ceil(ROTATE_BYTES / layer_bytes) + 1
    mats = [[mk(r, k, 1)[0] for r, k in layer] for _ in range(n)]
    x_attn, xb_attn = quantized(1536)
    x_out, xb_out = quantized(1536)
    x_ffn, xb_ffn = quantized(1536)
    x_hid, xb_hid = quantized(8960)
    ys = {r: torch.empty((n_vec, r), device=dev) for r in (1536, 8960)}
    plan = [(xb_attn, 1536, 1536)] * 3 + [(xb_out, 1536, 1536)] + [(xb_ffn, 8960, 1536)] * 2 + [(xb_hid, 1536, 8960)]

    def run_layer(i):
        hip.quantize_chunk(8, x_attn, xb_attn, 0, n_vec, 1536)
        for j in range(3):
            hip.mul_mat_q8_0(mats[i][j].data_ptr(), xb_attn, ys[1536], 1536, 1536, 1536, n_vec)
        hip.quantize_chunk(8, x_out, xb_out, 0, n_vec, 1536)
        hip.mul_mat_q8_0(mats[i][3].data_ptr(), xb_out, ys[1536], 1536, 1536, 1536, n_vec)
        hip.quantize_chunk(8, x_ffn, xb_ffn, 0, n_vec, 1536)
        for j in (4, 5):
            hip.mul_mat_q8_0(mats[i][j].data_ptr(), xb_ffn, ys[8960], 8960, 8960, 1536, n_vec)
        hip.quantize_chunk(8, x_hid, xb_hid, 0, n_vec, 8960)
        hip.mul_mat_q8_0(mats[i][6].data_ptr(), xb_hid, ys[1536], 1536, 1536, 8960, n_vec)

    ms = time_op(torch, head, run_layer, n, warmup, max(steps, 20))
    out["layer_4_quantize_7_matrices"] = op_entry(layer_bytes, ms, n_vec=n_vec,
                                                  dtype="q8_0 weights / q8_0 activations",
                                                  us_per_token_28_layers=round(28 * ms * 1e3, 1))
    # the same layer with the matrices that share an input in one launch each
    # (levo_hip_mul_mat_q8_0_multi: q / k / v, o, gate / up with the F32
    # activations quantized inside the launch), ffn_down as before: 5 launches
    yq = [torch.empty((n_vec, 1536), device=dev) for _ in range(4)]
    yf = [torch.empty((n_vec, 8960), device=dev) for _ in range(2)]

    def run_layer_multi(i):
        hip.mul_mat_q8_0_multi([(mats[i][j], yq[j], 1536, 1536) for j in range(3)], 1536, n_vec,
                               x=x_attn, x_pitch=1536)
        hip.mul_mat_q8_0_multi([(mats[i][3], yq[3], 1536, 1536)], 1536, n_vec, x=x_out, x_pitch=1536)
        hip.mul_mat_q8_0_multi([(mats[i][4], yf[0], 8960, 8960), (mats[i][5], yf[1], 8960, 8960)], 1536, n_vec,
                               x=x_ffn, x_pitch=1536)
        hip.quantize_chunk(8, x_hid, xb_hid, 0, n_vec, 8960)
        hip.mul_mat_q8_0(mats[i][6].data_ptr(), xb_hid, ys[1536], 1536, 1536, 8960, n_vec)

    ms = time_op(torch, head, run_layer_multi, n, warmup, max(steps, 20))
    out["layer_5_launches"] = op_entry(layer_bytes, ms, n_vec=n_vec, dtype="q8_0 weights / q8_0 activations",
                                       us_per_token_28_layers=round(28 * ms * 1e3, 1))
    # the 5-launch layer on packed matrices (repacked once, outside the
    # timing), ffn_down's input quantized to columns
    pmats = [[repacked(m.view(1, -1), r, k)[0] for m, (r, k) in zip(mats[i], layer)] for i in range(n)]
    del mats
    xc_hid = torch.empty(n_vec * (8960 // 32) * 36, dtype=torch.uint8, device=dev)

    def run_layer_packed(i):
        hip.mul_mat_q8_0_multi([(pmats[i][j], yq[j], 1536, 1536) for j in range(3)], 1536, n_vec,
                               x=x_attn, x_pitch=1536, packed=True)
        hip.mul_mat_q8_0_multi([(pmats[i][3], yq[3], 1536, 1536)], 1536, n_vec, x=x_out, x_pitch=1536, packed=True)
        hip.mul_mat_q8_0_multi([(pmats[i][4], yf[0], 8960, 8960), (pmats[i][5], yf[1], 8960, 8960)], 1536, n_vec,
                               x=x_ffn, x_pitch=1536, packed=True)
        hip.quantize_q8_0_columns(x_hid, 8960, xc_hid, n_vec, 8960)
        hip.mul_mat_q8_0_packed(pmats[i][6].data_ptr(), xc_hid, ys[1536], 1536, 1536, 8960, n_vec)

    ms = time_op(torch, head, run_layer_packed, n, warmup, max(steps, 20))
    out["layer_5_launches_packed"] = op_entry(layer_bytes, ms, n_vec=n_vec,
                                              dtype="q8_0 weights (packed) / q8_0 activation columns",
                                              us_per_token_28_layers=round(28 * ms * 1e3, 1))
    return out


PEAK_F32_MFMA_TFLOPS = 157.3


def bench_mul_mat_kquant(torch, hip, head, dev, warmup, steps):
    """K-quant decode mat-vec (levo_hip_mul_mat_kquant: Q4_K, Q5_K, Q6_K
    weights, the Q4_K_M / Q5_K_M / Q6_K profiles' matrices) at LeLM medium's
    matrices with the CFG pair of activation columns already quantized to
    Q8_K; weights rotated over >= 512 MB. Bytes: weights + Q8_K activations + y."""
    shapes = {"attn_1536x1536": (1536, 1536), "ffn_up_8960x1536": (8960, 1536),
              "ffn_down_1536x8960": (1536, 8960), "head_16385x1536": (16385, 1536)}
    n_vec = 2
    out = {}
    g = torch.Generator(device=dev)
    g.manual_seed(35)
    for qtype, tname, bb in ((12, "q4_K", 144), (13, "q5_K", 176), (14, "q6_K", 210)):
        for name, (rows, k) in shapes.items():
            nb = rows * (k // 256)
            nbytes = nb * bb
            stride = (nbytes + 255) // 256 * 256
            n = math.ceil(ROTATE_BYTES / nbytes) + 1
            w = torch.randint(0, 256, (n, stride), generator=g, device=dev, dtype=torch.uint8)
            scale = torch.full((nb, 1), 0x1400, dtype=torch.int16, device=dev).view(torch.uint8)  # F16 2^-10
            for i in range(n):
                blocks = w[i, :nbytes].view(nb, bb)
                if qtype == 14:
                    blocks[:, 208:210] = scale
                else:
                    blocks[:, 0:2] = scale
                    blocks[:, 2:4] = scale
            x = torch.randn((n_vec, k), generator=g, device=dev)
            xb = torch.empty(n_vec * (k // 256) * 292, dtype=torch.uint8, device=dev)
            hip.quantize_q8_K(x, xb, n_vec * k)
            y = torch.empty((n_vec, rows), device=dev)
            per = nbytes + n_vec * (k // 256) * 292 + n_vec * rows * 4
            ms = time_op(torch, head, lambda i: hip.mul_mat_kquant(qtype, w[i].data_ptr(), xb, y, rows, rows, k,
                                                                    n_vec), n, warmup, max(steps, 50))
            out[f"{tname}_{name}"] = op_entry(per, ms, read=per - n_vec * rows * 4, shape=[rows, k], n_vec=n_vec,
                                              dtype=f"{tname} weights / q8_K activations")
            del w
        torch.cuda.empty_cache()
    out.update(bench_kquant_layer(torch, hip, head, dev, warmup, steps, g))
    return out


def bench_kquant_layer(torch, hip, head, dev, warmup, steps, g):
    """One LeLM medium decode layer's seven matrices under the Q4_K_M profile
    (q, k, gate, up Q4_K; v, o, down promoted to Q6_K,
    src/levo-quantization.h:75-95), CFG pair of activation columns: as 4 Q8_K
    quantizations + 7 mat-vecs, and with the matrices that share an input in
    one levo_hip_mul_mat_kquant_multi launch each (q / k / v, o, gate / up,
    the F32 activations quantized inside the launch) + ffn_down's
    quantization and mat-vec: 5 launches."""
    n_vec = 2
    Q4, Q6 = 12, 14
    layer = [(Q4, 1536, 1536), (Q4, 1536, 1536), (Q6, 1536, 1536), (Q6, 1536, 1536), (Q4, 8960, 1536),
             (Q4, 8960, 1536), (Q6, 1536, 8960)]
    bb = {Q4: 144, Q6: 210}
    wbytes = [r * (k // 256) * bb[t] for t, r, k in layer]
    layer_bytes = sum(wbytes) + sum(n_vec * r * 4 for _, r, _ in layer) + n_vec * 4 * (3 * 1536 + 8960)
    n = math.ceil(ROTATE_BYTES / layer_bytes) + 1
    mats = []
    for _ in range(n):
        ms_ = []
        for (t, r, k), nb_ in zip(layer, wbytes):
            w = torch.randint(0, 256, (nb_,), generator=g, device=dev, dtype=torch.uint8)
            blocks = w.view(-1, bb[t])
            scale = torch.full((blocks.shape[0], 1), 0x1400, dtype=torch.int16, device=dev).view(torch.uint8)
            if t == Q6:
                blocks[:, 208:210] = scale
            else:
                blocks[:, 0:2] = scale
                blocks[:, 2:4] = scale
            ms_.append(w)
        mats.append(ms_)
    xs = {name: torch.randn((n_vec, k), generator=g, device=dev) for name, k in
          (("attn", 1536), ("out", 1536), ("ffn", 1536), ("hid", 8960))}
    xbs = {name: torch.empty(n_vec * (x.shape[1] // 256) * 292, dtype=torch.uint8, device=dev)
           for name, x in xs.items()}
    y1 = [torch.empty((n_vec, 1536), device=dev) for _ in range(5)]
    y8 = [torch.empty((n_vec, 8960), device=dev) for _ in range(2)]
    ys = [y1[0], y1[1], y1[2], y1[3], y8[0], y8[1], y1[4]]
    src = ["attn", "attn", "attn", "out", "ffn", "ffn", "hid"]

    def run_layer(i):
        for name in ("attn", "out", "ffn", "hid"):
            hip.quantize_q8_K(xs[name], xbs[name], xs[name].numel())
        for j, (t, r, k) in enumerate(layer):
            hip.mul_mat_kquant(t, mats[i][j].data_ptr(), xbs[src[j]], ys[j], r, r, k, n_vec)

    def run_layer_multi(i):
        m = lambda j: (layer[j][0], mats[i][j], ys[j], layer[j][1], layer[j][1])
        hip.mul_mat_kquant_multi([m(0), m(1), m(2)], 1536, n_vec, x=xs["attn"], x_pitch=1536)
        hip.mul_mat_kquant_multi([m(3)], 1536, n_vec, x=xs["out"], x_pitch=1536)
        hip.mul_mat_kquant_multi([m(4), m(5)], 1536, n_vec, x=xs["ffn"], x_pitch=1536)
        hip.quantize_q8_K(xs["hid"], xbs["hid"], xs["hid"].numel())
        hip.mul_mat_kquant(Q6, mats[i][6].data_ptr(), xbs["hid"], ys[6], 1536, 1536, 8960, n_vec)

    out = {}
    for name, fn in (("q4_K_M_layer_11_launches", run_layer), ("q4_K_M_layer_5_launches", run_layer_multi)):
        ms = time_op(torch, head, fn, n, warmup, max(steps, 20))
        out[name] = op_entry(layer_bytes, ms, n_vec=n_vec, dtype="q4_K / q6_K weights / q8_K activations",
                             us_per_token_28_layers=round(28 * ms * 1e3, 1))
    return out


def bench_snake_conv(torch, hip, head, dev, warmup, steps):
    """Fused SnakeBeta + Conv1d (+ bias, + residual) of the VAE decoder's
    residual units at a 10.08 s window's real stage lengths: stage 5
    (128 channels x 483840 samples; k = 7 at dilation 1 / 3 / 9, k = 1 with
    the residual add), stage 3 (256 x 60480) and stage 1 (1024 x 2520).
    Every case runs levo_hip_snake_conv1d_split with a workspace, as the
    decoder does: stage 1's 160 output tiles (fewer than the 256 CUs) split
    their input channels three ways plus the combine launch (both timed);
    the larger grids run unsplit. Stage 1 is also timed without the
    workspace (`stage1_k7_d9_unsplit`). Matrix-core bound: `TFLOP/s` is
    2 * C_out * C_in * k * T_out per call over the call's time, against the
    F32 MFMA peak; bytes are x, y (and the residual) once."""
    out = {}
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    cases = [("stage5_k7_d1", 128, 483840, 7, 1), ("stage5_k7_d9", 128, 483840, 7, 9),
             ("stage5_k1_residual", 128, 483840, 1, 1), ("stage3_k7_d3", 256, 60480, 7, 3),
             ("stage1_k7_d9", 1024, 2520, 7, 9), ("stage1_k7_d9_unsplit", 1024, 2520, 7, 9),
             ("stage1_k1_residual", 1024, 2520, 1, 1)]
    for name, c, t, kw, dil in cases:
        pad = 3 * dil if kw == 7 else 0
        x = torch.randn((c, t), generator=g, device=dev)
        w = torch.randn((c, c, kw), generator=g, device=dev) / math.sqrt(c * kw)
        b = torch.randn(c, generator=g, device=dev) * 0.1
        a = torch.randn(c, generator=g, device=dev) * 0.5
        bl = torch.randn(c, generator=g, device=dev) * 0.5
        r = torch.randn((c, t), generator=g, device=dev) if kw == 1 else None
        y = torch.empty((c, t), device=dev)
        if name.endswith("_unsplit"):
            fn = lambda i: hip.snake_conv1d(x, c, t, w, c, kw, alpha_log=a, beta_log=bl, bias=b, padding=pad,
                                            dilation=dil, residual=r, y=y)
        else:
            nws = hip.snake_conv1d_split_workspace_floats(c, t)
            ws = torch.empty(nws, device=dev)
            fn = lambda i: hip.snake_conv1d_split(x, c, t, w, c, kw, workspace=ws, workspace_floats=nws,
                                                  alpha_log=a, beta_log=bl, bias=b, padding=pad, dilation=dil,
                                                  residual=r, y=y)
        ms = time_op(torch, head, fn, 1, warmup, max(steps // 4, 5))
        flops = 2.0 * c * c * kw * t
        tflops = flops / (ms * 1e-3) / 1e12
        nbytes = 4 * c * t * (3 if r is not None else 2)
        out[name] = {"shape": [c, t, kw, dil], "us_per_launch": round(ms * 1e3, 1), "TFLOP/s": round(tflops, 1),
                     "frac_f32_mfma": round(tflops / PEAK_F32_MFMA_TFLOPS, 4), "bytes_per_launch": nbytes,
                     "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1), "bound": "mfma"}
        del x, w, y, r
    # stage 1's upsampler (SnakeBeta + ConvTranspose1d 2048 -> 1024, stride 10) at the same window:
    # 252 input frames, 160 workgroups over the ten stride phases, split three ways
    ci, co, t_in, s = 2048, 1024, 252, 10
    pad = (s + 1) // 2
    t_out = (t_in + 1) * s - 2 * pad
    x = torch.randn((ci, t_in), generator=g, device=dev)
    packed = torch.randn(s * co * ci * 2, generator=g, device=dev) / math.sqrt(2 * ci)
    b = torch.randn(co, generator=g, device=dev) * 0.1
    a = torch.randn(ci, generator=g, device=dev) * 0.5
    bl = torch.randn(ci, generator=g, device=dev) * 0.5
    y = torch.empty((co, t_out), device=dev)
    nws = hip.snake_conv_transpose1d_split_workspace_floats(co, t_in, s)
    ws = torch.empty(nws, device=dev)
    for name, split in (("stage1_upsample_x10", True), ("stage1_upsample_x10_unsplit", False)):
        if split:
            fn = lambda i: hip.snake_conv_transpose1d_split(x, ci, t_in, packed, co, s, workspace=ws,
                                                            workspace_floats=nws, alpha_log=a, beta_log=bl, bias=b,
                                                            padding=pad, y=y)
        else:
            fn = lambda i: hip.snake_conv_transpose1d(x, ci, t_in, packed, co, s, alpha_log=a, beta_log=bl, bias=b,
                                                      padding=pad, y=y)
        ms = time_op(torch, head, fn, 1, warmup, max(steps // 4, 5))
        tflops = 2.0 * ci * co * 2 * s * (t_in + 1) / (ms * 1e-3) / 1e12  # two taps per phase column
        nbytes = 4 * (ci * t_in + co * t_out)
        out[name] = {"shape": [ci, co, t_in, s], "us_per_launch": round(ms * 1e3, 1), "TFLOP/s": round(tflops, 1),
                     "frac_f32_mfma": round(tflops / PEAK_F32_MFMA_TFLOPS, 4), "bytes_per_launch": nbytes,
                     "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1), "bound": "mfma"}
    return out


def vae_decode_flops(frames):
    """2 * C_out * C_in * taps * T_out summed over the decoder's 37 convolutions
    (each transposed-conv output sample takes 2 taps per input channel)."""
    f = 2.0 * 2048 * 64 * 7 * frames
    t = frames
    for s, (ci, co) in enumerate(zip((2048, 1024, 512, 256, 128), (1024, 512, 256, 128, 128))):
        t *= (10, 6, 4, 4, 2)[s]
        f += 2.0 * ci * co * 2 * t + 3 * (2.0 * co * co * 7 * t + 2.0 * co * co * t)
    return f + 2.0 * 2 * 128 * 7 * t


def bench_vae_decode(torch, hip, binding, head, dev, warmup, steps, frames=252):
    """The whole Oobleck VAE decoder (levo_hip_vae_decode: 37 SnakeBeta +
    convolution steps in 31 launches, the six 128-channel residual units one
    launch each, plus a combine launch for each convolution whose grid is
    split over its input channels) on one window: latent [64][frames] to stereo audio
    [2][frames * 1920], random weights of the decoder's shapes. 252 frames is
    10.08 s of audio; 1000 frames is the renderer's decode window
    (renderer_window_frames, src/levo-renderer-pattern.h:11)."""
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    keep = []

    def put(*shape, scale):
        t = torch.randn(shape, generator=g, device=dev) * scale
        keep.append(t)
        return t.data_ptr()

    w = binding.VaeDecoderWeights()
    w.input.weight, w.input.bias = put(2048, 64, 7, scale=0.5 / math.sqrt(64 * 7)), put(2048, scale=0.05)
    for s in range(5):
        ci, co, st = binding.VAE_IN_WIDTH[s], binding.VAE_OUT_WIDTH[s], binding.VAE_STRIDES[s]
        sg = w.stage[s]
        sg.activation.alpha_log, sg.activation.beta_log = put(ci, scale=0.3), put(ci, scale=0.3)
        raw = torch.randn((ci, co, 2 * st), generator=g, device=dev) * (0.5 / math.sqrt(2 * ci))
        packed = torch.empty(st * co * ci * 2, device=dev)
        hip.conv_transpose1d_pack_weights(raw, packed, ci, co, st)
        keep.append(packed)
        sg.upsample.weight, sg.upsample.bias = packed.data_ptr(), put(co, scale=0.05)
        for r in range(3):
            ru = sg.residual[r]
            ru.pre.alpha_log, ru.pre.beta_log = put(co, scale=0.3), put(co, scale=0.3)
            ru.conv_0.weight, ru.conv_0.bias = put(co, co, 7, scale=0.5 / math.sqrt(co * 7)), put(co, scale=0.05)
            ru.post.alpha_log, ru.post.beta_log = put(co, scale=0.3), put(co, scale=0.3)
            ru.conv_1.weight, ru.conv_1.bias = put(co, co, 1, scale=0.3 / math.sqrt(co)), put(co, scale=0.05)
    w.output_activation.alpha_log, w.output_activation.beta_log = put(128, scale=0.3), put(128, scale=0.3)
    w.output_weight = put(2, 128, 7, scale=0.5 / math.sqrt(128 * 7))
    w.param_type = 0
    latent = torch.randn((64, frames), generator=g, device=dev)
    audio = torch.empty((2, frames * 1920), device=dev)
    nbytes = hip.vae_decode_workspace_bytes(frames)
    ws = torch.empty(nbytes // 4, device=dev)
    ms = time_op(torch, head, lambda i: hip.vae_decode(w, latent, frames, audio, ws, nbytes), 1,
                 max(warmup // 10, 2), max(steps // 10, 5))
    assert bool(torch.isfinite(audio).all())
    flops = vae_decode_flops(frames)
    tflops = flops / (ms * 1e-3) / 1e12
    seconds = frames * 1920 / 48000
    del keep, ws
    torch.cuda.empty_cache()
    return {"frames": frames, "audio_seconds": seconds, "ms_per_window": round(ms, 3),
            "realtime_factor": round(seconds / (ms * 1e-3), 1), "steps": 31, "flops_per_window": flops,
            "TFLOP/s": round(tflops, 1), "frac_f32_mfma": round(tflops / PEAK_F32_MFMA_TFLOPS, 4), "bound": "mfma"}


def bench_quant(torch, hip, head, dev, warmup, steps):
    R, Cc = 4096, 1536
    out = {}
    for qt, name, bb in ((8, "q8_0", 34), (2, "q4_0", 18)):
        qbytes = R * Cc // 32 * bb
        per_q = 2 * R * Cc + qbytes
        per_d = qbytes + 4 * R * Cc
        n = math.ceil(ROTATE_BYTES / min(per_q, per_d)) + 1
        g = torch.Generator(device=dev)
        g.manual_seed(qt)
        src = [(torch.randn((R, Cc), generator=g, device=dev) * 0.02).half() for _ in range(n)]
        q = [torch.empty(qbytes, dtype=torch.uint8, device=dev) for _ in range(n)]
        deq = [torch.empty((R, Cc), dtype=torch.float32, device=dev) for _ in range(n)]
        ms = time_op(torch, head, lambda i: hip.quantize_rows(qt, src[i], 1, Cc, Cc, q[i], R, Cc), n, warmup,
                     max(steps, 50))
        out[f"{name}_quantize_f16"] = op_entry(per_q, ms, read=2 * R * Cc, shape=[R, Cc])
        ms = time_op(torch, head, lambda i: hip.dequantize(qt, q[i], deq[i], 0, R * Cc), n, warmup, max(steps, 50))
        out[f"{name}_dequantize_f32"] = op_entry(per_d, ms, read=qbytes, shape=[R, Cc])
        del src, q, deq
        torch.cuda.empty_cache()
    # the K-quant profiles' quantizers (quantize_row_q{4,5,6}_K_ref) on the same F16 matrix: a scale search
    # per 32- (16-) value sub-block, VALU-bound
    for qt, name, bb in ((12, "q4_K", 144), (13, "q5_K", 176), (14, "q6_K", 210)):
        qbytes = R * Cc // 256 * bb
        per_q = 2 * R * Cc + qbytes
        n = math.ceil(ROTATE_BYTES / per_q) + 1
        g = torch.Generator(device=dev)
        g.manual_seed(qt)
        src = [(torch.randn((R, Cc), generator=g, device=dev) * 0.02).half() for _ in range(n)]
        q = [torch.empty(qbytes, dtype=torch.uint8, device=dev) for _ in range(n)]
        ms = time_op(torch, head, lambda i: hip.quantize_rows(qt, src[i], 1, Cc, Cc, q[i], R, Cc), n, warmup,
                     max(steps, 20))
        out[f"{name}_quantize_f16"] = op_entry(per_q, ms, read=2 * R * Cc, shape=[R, Cc], bound="valu",
                                               sub_blocks_per_s=round(R * Cc / (32 if qt != 14 else 16) / (ms * 1e-3)))
        del src, q
        torch.cuda.empty_cache()
    # the converter's F16 <-> F32 rows (ggml_fp32_to_fp16_row / ggml_fp16_to_fp32_row) at the same shape
    per = 6 * R * Cc
    n = math.ceil(ROTATE_BYTES / per) + 1
    g = torch.Generator(device=dev)
    g.manual_seed(12)
    f32 = [torch.randn((R, Cc), generator=g, device=dev) * 0.02 for _ in range(n)]
    f16 = [torch.empty((R, Cc), dtype=torch.float16, device=dev) for _ in range(n)]
    ms = time_op(torch, head, lambda i: hip.fp32_to_fp16_row(f32[i], f16[i], R * Cc), n, warmup, max(steps, 50))
    out["fp32_to_fp16_row"] = op_entry(per, ms, read=4 * R * Cc, shape=[R, Cc])
    ms = time_op(torch, head, lambda i: hip.fp16_to_fp32_row(f16[i], f32[i], R * Cc), n, warmup, max(steps, 50))
    out["fp16_to_fp32_row"] = op_entry(per, ms, read=2 * R * Cc, shape=[R, Cc])
    del f32, f16
    torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------------------
def cpu_baseline(host_ladder, with_ops=True):
    """The CPU leg, timed as the reference times its CPU runs: pinned to 1
    thread and to every thread of the process's CPU share, 3 warm-ups and the
    median of 10 runs, with the host CPU named. The headline is the oracle's
    five-pass ggml-cpu SnakeBeta chain (mul, sin, sqr, div, add; rows split
    over threads as ggml-cpu does) on the whole ladder at all threads; the
    1-thread figure runs the first 32 channels of the 128 x 48384 rung (the
    five passes over 1.5M elements take about 0.2 s on one core)."""
    from oracle.levo_oracle import Oracle
    orc = Oracle()
    threads = cpu_share()
    total_bytes = sum(snake_bytes(x.shape[0], x.shape[1]) for x, _, _ in host_ladder)

    def ladder(t):
        for x, a, b in host_ladder:
            orc.snake_beta(x, a, b, threads=t)

    with pinned(threads):
        secs = median_seconds(lambda: ladder(threads))
    x1, a1, b1 = next(t for t in host_ladder if t[0].shape == (128, 48384))
    xs, as_, bs = np.ascontiguousarray(x1[:32]), a1[:32].copy(), b1[:32].copy()
    with pinned(1):
        secs1 = median_seconds(lambda: orc.snake_beta(xs, as_, bs, threads=1))
    one = {"value": round(snake_bytes(32, 48384) / secs1 / 1e9, 4), "unit": "GB/s", "cores": 1,
           "sample": "SnakeBeta 32 x 48384 (the first 32 channels of the 128 x 48384 rung), F32"}
    out = {"value": round(total_bytes / secs / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
           "ms_per_step": round(secs * 1e3, 2), "one_thread": one, "cpu": cpu_model(),
           "method": "pinned (sched_setaffinity) to 1 and to all threads of the CPU share; 3 warm-ups, "
                     "median of 10 runs; oracle C restatement built with -O3",
           "sample": f"the full ladder (72,253,440 elements) per run through the oracle's five-pass ggml-cpu "
                     f"chain, {threads} threads"}
    if with_ops:
        out["ops"] = cpu_ops_baselines(orc, threads)
    return out


def cpu_ops_baselines(orc, threads):
    """Every other op of the table on the CPU at 1 thread and at `threads`
    (3 warm-ups, median of 10), in the GPU figures' algorithmic bytes. Ops
    whose oracle function is single-threaded run as `threads` row chunks on a
    thread pool (ctypes drops the GIL for the C call)."""
    from oracle.levo_oracle import Reference, have_reference
    res = {}
    pool = cf.ThreadPoolExecutor(threads)

    def both(name, nbytes, one_fn, all_fn, sample, kind="port"):
        with pinned(1):
            t1 = median_seconds(one_fn)
        with pinned(threads):
            tn = median_seconds(all_fn)
        res[name] = {"1_thread_GB/s": round(nbytes / t1 / 1e9, 3), f"{threads}_threads_GB/s": round(nbytes / tn / 1e9, 3),
                     "1_thread_ms": round(t1 * 1e3, 3), f"{threads}_threads_ms": round(tn * 1e3, 3),
                     "bytes": int(nbytes), "kind": kind, "sample": sample}

    def chunked(fn, n):
        parts = split_rows(n, threads)
        return lambda: list(pool.map(lambda r: fn(*r), parts))

    # SnakeBeta, one second of audio at 128 channels
    x = orc.gaussian(128 * 48000, 11).reshape(128, 48000)
    a = (orc.gaussian(128, 12) * 0.1).astype(np.float32)
    both("snake_beta_128x48000", snake_bytes(128, 48000), lambda: orc.snake_beta(x, a, a, threads=1),
         lambda: orc.snake_beta(x, a, a, threads=threads), "the five-pass ggml-cpu chain, rows split over threads")
    # residual norms, F16 activations and parameters
    rows, D = 756, 2048
    xh = orc.f32_to_f16(orc.gaussian(rows * D, 1).reshape(rows, D))
    dh = orc.f32_to_f16(orc.gaussian(rows * D, 2).reshape(rows, D))
    w = orc.f32_to_f16(orc.gaussian(D, 3) * 0.02 + 1)
    bb = orc.f32_to_f16(orc.gaussian(D, 4) * 0.02)
    both(f"residual_rmsnorm_f16_{rows}x{D}", 8 * rows * D + 2 * D,
         lambda: orc.rms_norm(xh, dh, w, 1e-6, threads=1), lambda: orc.rms_norm(xh, dh, w, 1e-6, threads=threads),
         "add, cast, rms_norm, cast, mul (ggml-cpu chain), rows split over threads")
    both(f"residual_layernorm_f16_{rows}x{D}", 8 * rows * D + 4 * D,
         lambda: orc.layer_norm(xh, dh, w, bb, 1e-6, threads=1),
         lambda: orc.layer_norm(xh, dh, w, bb, 1e-6, threads=threads),
         "add, norm, mul, add (ggml-cpu chain), rows split over threads")
    # Flow CFG + Euler, one step of the 64 x 2520 latent
    n = 64 * 2520
    st, vu, vc = orc.gaussian(n, 4), orc.gaussian(n, 5), orc.gaussian(n, 6)
    both("flow_cfg_euler_64x2520", 16 * n, lambda: orc.flow_cfg_euler(st, vu, vc, 1.5, 0.02),
         chunked(lambda i, j: orc.flow_cfg_euler(st[i:j], vu[i:j], vc[i:j], 1.5, 0.02), n),
         "the renderer's host CFG + Euler loop (src/levo-flow-renderer.cpp), one step")
    # Q8_0 / Q4_0 blocks and F16 <-> F32 rows at [4096, 1536]
    R, C = 4096, 1536
    xq = orc.f32_to_f16((orc.gaussian(R * C, 7) * 0.02).reshape(R, C))
    for qt, name, bsz in ((8, "q8_0", 34), (2, "q4_0", 18)):
        q = orc.quantize_f16_padded(qt, xq, C)
        both(f"{name}_quantize_f16", 2 * R * C + R * C // 32 * bsz, lambda: orc.quantize_f16_padded(qt, xq, C),
             chunked(lambda i, j: orc.quantize_f16_padded(qt, xq[i:j], C), R),
             "ggml's reference block quantizer over F16 rows (ggml_quantize_chunk's path)")
        qb = q.reshape(R, -1)
        both(f"{name}_dequantize_f32", R * C // 32 * bsz + 4 * R * C, lambda: orc.dequantize(qt, q, R * C),
             chunked(lambda i, j: orc.dequantize(qt, np.ascontiguousarray(qb[i:j]), (j - i) * C), R),
             "ggml's dequantize_row to F32")
    for qt, name, bsz in ((12, "q4_K", 144), (13, "q5_K", 176), (14, "q6_K", 210)):
        rows_k = 256  # a 256-row slice of the matrix: the scale search costs ~0.1 s per slice on one core
        xk = np.ascontiguousarray(xq[:rows_k])
        both(f"{name}_quantize_f16", 2 * rows_k * C + rows_k * C // 256 * bsz,
             lambda: orc.quantize_f16_padded(qt, xk, C),
             chunked(lambda i, j: orc.quantize_f16_padded(qt, xk[i:j], C), rows_k),
             f"ggml's quantize_row_{name}_ref over {rows_k} F16 rows of 1536 (GB/s of the same bytes)")
    f = orc.gaussian(R * C, 9)
    h = orc.f32_to_f16(f)
    both("fp32_to_fp16_row", 6 * R * C, lambda: orc.f32_to_f16(f),
         chunked(lambda i, j: orc.f32_to_f16(f[i * C:j * C]), R), "ggml_fp32_to_fp16_row (RNE)")
    both("fp16_to_fp32_row", 6 * R * C, lambda: orc.f16_to_f32(h),
         chunked(lambda i, j: orc.f16_to_f32(h[i * C:j * C]), R), "ggml_fp16_to_fp32_row")
    if have_reference():
        ref = Reference()
        V, per = 16384, 60
        c = orc.gaussian(per * V, 8) * 3
        u = orc.gaussian(per * V, 9) * 3
        samplers = [ref.sampler(1 + t) for t in range(threads)]

        def rows_on(t, lo, hi):
            for r in range(lo, hi):
                logit = ref.apply_cfg(c[r * V:(r + 1) * V], u[r * V:(r + 1) * V], 1.5)
                samplers[t].sample(logit, 50, 0.9, True)

        with pinned(1):
            t1 = median_seconds(lambda: rows_on(0, 0, per))
        with pinned(threads):
            tn = median_seconds(lambda: list(pool.map(lambda t: rows_on(t, 0, per), range(threads))))
        res["cfg_softmax_top50"] = {
            "1_thread_GB/s": round(per * 2 * V * 4 / t1 / 1e9, 3),
            f"{threads}_threads_GB/s": round(threads * per * 2 * V * 4 / tn / 1e9, 3),
            "1_thread_rows_per_s": round(per / t1, 1), f"{threads}_threads_rows_per_s": round(threads * per / tn, 1),
            "kind": "reference",
            "sample": f"{per} rows of 16384 per thread: levo::apply_cfg + Sampler::sample(top-50, T=0.9), "
                      f"each thread its own Sampler"}
        V2 = 16385
        streams = (orc.gaussian(3 * V2, 10) * 3).reshape(3, V2)
        recent = (np.arange(150, dtype=np.int64) * 97 % (V2 - 1)).reshape(3, 50)
        s2 = ref.sampler(2)
        with pinned(1):
            t1 = median_seconds(lambda: s2.sample_streams(streams, use_sampling=True, temperature=0.9,
                                                          top_k_mixed=50, top_k_detail=1, repetition_penalty=1.1,
                                                          recent=recent, ignore=(0, 1, 2)))
        res["decode_step_sample"] = {
            "1_thread_us_per_step": round(t1 * 1e6, 1), "kind": "reference",
            "sample": "Sampler::sample_streams over 3 host rows of 16385 (penalty window 50, 3 ignored ids, "
                      "top-k 50/1/1, T = 0.9), one step at a time (a decode step is serial); the reference "
                      "first copies 2 x 196 KB of logits to the host"}
    pool.shutdown()
    return res


def traffic_probe(torch, hip, binding, dev) -> None:
    """One launch of each hot-path kernel at its config shape plus a plain
    256 MiB device-to-device copy (the calibration kernel of known size), for
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes. Prints the launch order."""
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    order = []
    src = torch.randn(64 << 20, generator=g, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    order.append(("copy_256MiB", 2 * src.numel() * 4))
    for C, T in ((128, 483840), (128, 48000)):
        x = torch.randn((C, T), generator=g, device=dev)
        a = torch.rand(C, generator=g, device=dev) - 0.5
        y = torch.empty_like(x)
        hip.snake_beta(x, a, a, y)
        order.append((f"snake_beta_{C}x{T}", snake_bytes(C, T)))
    jobs = []
    for C, T in LADDER:
        x = torch.randn((C, T), generator=g, device=dev)
        a = torch.rand(C, generator=g, device=dev) - 0.5
        jobs.append((x, a, a, torch.empty_like(x)))
    hip.snake_beta_batch(jobs)
    order.append(("snake_beta_batch_ladder", sum(snake_bytes(C, T) for C, T in LADDER)))
    del jobs
    for rows, D in ((756, 2048), (756, 1536)):
        xh = torch.randn((rows, D), generator=g, device=dev).half()
        dh = torch.randn((rows, D), generator=g, device=dev).half()
        w = torch.ones(D, device=dev).half()
        hh, yh = torch.empty_like(xh), torch.empty_like(xh)
        hip.rms_norm(1, xh, dh, w, 1, hh, yh, rows, D, 1e-6)
        order.append((f"rmsnorm_f16_{rows}x{D}", 8 * rows * D + 2 * D))
        hip.layer_norm(1, xh, dh, w, w, 1, hh, yh, rows, D, 1e-6)
        order.append((f"layernorm_f16_{rows}x{D}", 8 * rows * D + 4 * D))
        del xh, dh, hh, yh
    rows, D = 2000, 2200  # the Flow estimator's F32 LayerNorm
    xf = torch.randn((rows, D), generator=g, device=dev)
    df = torch.randn((rows, D), generator=g, device=dev)
    wf = torch.ones(D, device=dev)
    hf, yf = torch.empty_like(xf), torch.empty_like(xf)
    hip.layer_norm(0, xf, df, wf, wf, 0, hf, yf, rows, D, 1e-5)
    order.append(("layernorm_f32_2000x2200", 16 * rows * D + 8 * D))
    keep = []
    a = modulated_norm_args(torch, binding, dev, g, rows, D, 1000, xf, df, hf, yf, keep)
    hip.layer_norm_modulated(a)
    order.append(("gated_layernorm_adaln_f32_2000x2200", 16 * rows * D + 8 * D + 3 * 12 * D))
    del xf, df, hf, yf, keep
    n = 64 * 2520
    st, vu, vc = (torch.randn(n, generator=g, device=dev) for _ in range(3))
    hip.flow_cfg_euler(st, vu, vc, n, 1.5, 0.02)
    order.append(("flow_cfg_euler_64x2520", 16 * n))
    R, Cc = 4096, 1536
    wq = (torch.randn((R, Cc), generator=g, device=dev) * 0.02).half()
    q = torch.empty(R * Cc // 32 * 34, dtype=torch.uint8, device=dev)
    hip.quantize_rows(8, wq, 1, Cc, Cc, q, R, Cc)
    order.append(("q8_0_quantize_f16", 2 * R * Cc + q.numel()))
    deq = torch.empty((R, Cc), device=dev)
    hip.dequantize(8, q, deq, 0, R * Cc)
    order.append(("q8_0_dequantize_f32", q.numel() + 4 * R * Cc))
    q4 = torch.empty(R * Cc // 32 * 18, dtype=torch.uint8, device=dev)
    hip.quantize_rows(2, wq, 1, Cc, Cc, q4, R, Cc)
    order.append(("q4_0_quantize_f16", 2 * R * Cc + q4.numel()))
    hip.dequantize(2, q4, deq, 0, R * Cc)
    order.append(("q4_0_dequantize_f32", q4.numel() + 4 * R * Cc))
    for qt, name, bb in ((12, "q4_K", 144), (13, "q5_K", 176), (14, "q6_K", 210)):
        qk = torch.empty(R * Cc // 256 * bb, dtype=torch.uint8, device=dev)
        hip.quantize_rows(qt, wq, 1, Cc, Cc, qk, R, Cc)
        order.append((f"{name}_quantize_f16", 2 * R * Cc + qk.numel()))
        del qk
    # decode mat-vecs at LeLM's ffn_down (1536 x 8960), two activation columns,
    # with their weight and activation quantizations
    Rw, Kw, NV = 1536, 8960, 2
    wf = (torch.randn((Rw, Kw), generator=g, device=dev) * 0.02).half()
    xf = torch.randn((NV, Kw), generator=g, device=dev)
    yv = torch.empty((NV, Rw), device=dev)
    wq8 = torch.empty(Rw * Kw // 32 * 34, dtype=torch.uint8, device=dev)
    hip.quantize_rows(8, wf, 1, Kw, Kw, wq8, Rw, Kw)
    order.append(("prep_q8_0_weights", 2 * Rw * Kw + wq8.numel()))
    xq8 = torch.empty(NV * Kw // 32 * 34, dtype=torch.uint8, device=dev)
    hip.quantize_chunk(8, xf, xq8, 0, NV, Kw)
    order.append(("prep_q8_0_activations", 4 * NV * Kw + xq8.numel()))
    hip.mul_mat_q8_0(wq8, xq8, yv, Rw, Rw, Kw, NV)
    order.append(("mul_mat_q8_0_ffn_down_1536x8960", wq8.numel() + xq8.numel() + 4 * NV * Rw))
    wp8 = torch.empty_like(wq8)
    hip.repack_q8_0(wq8, wp8, Rw, Kw)
    order.append(("repack_q8_0_weights", 2 * wq8.numel()))
    xc8 = torch.empty(NV * Kw // 32 * 36, dtype=torch.uint8, device=dev)
    hip.quantize_q8_0_columns(xf, Kw, xc8, NV, Kw)
    order.append(("prep_q8_0_columns", 4 * NV * Kw + xc8.numel()))
    hip.mul_mat_q8_0_packed(wp8, xc8, yv, Rw, Rw, Kw, NV)
    order.append(("mul_mat_q8_0_packed_ffn_down_1536x8960", wp8.numel() + xc8.numel() + 4 * NV * Rw))
    del wp8, xc8
    wq4k = torch.empty(Rw * Kw // 256 * 144, dtype=torch.uint8, device=dev)
    hip.quantize_rows(12, wf, 1, Kw, Kw, wq4k, Rw, Kw)
    order.append(("prep_q4_K_weights", 2 * Rw * Kw + wq4k.numel()))
    xq8k = torch.empty(NV * (Kw // 256) * 292, dtype=torch.uint8, device=dev)
    hip.quantize_q8_K(xf, xq8k, NV * Kw)
    order.append(("prep_q8_K_activations", 4 * NV * Kw + xq8k.numel()))
    hip.mul_mat_kquant(12, wq4k, xq8k, yv, Rw, Rw, Kw, NV)
    order.append(("mul_mat_q4_K_ffn_down_1536x8960", wq4k.numel() + xq8k.numel() + 4 * NV * Rw))
    del wf, xf, yv, wq8, xq8, wq4k, xq8k
    P, S, V = 750, 3, 16384
    c = torch.randn((P * S, V), generator=g, device=dev) * 3
    u = torch.randn((P * S, V), generator=g, device=dev) * 3
    out_i = torch.empty((P * S, 64), dtype=torch.int32, device=dev)
    out_f = torch.empty((P * S, 64), device=dev)
    small_i = torch.empty((2, P * S), dtype=torch.int32, device=dev)
    small_f = torch.empty((2, P * S), device=dev)
    a = binding.SampleArgs()
    a.cond, a.uncond, a.rows, a.vocab, a.row_pitch = c.data_ptr(), u.data_ptr(), P * S, V, V
    a.cfg_scale, a.temperature, a.n_streams = 1.5, 0.9, 3
    for k in range(3):
        a.top_k[k] = 50
    a.best, a.count = small_i[0].data_ptr(), small_i[1].data_ptr()
    a.cand_ids, a.cand_probs, a.capacity = out_i.data_ptr(), out_f.data_ptr(), 64
    a.row_max, a.row_lse = small_f[0].data_ptr(), small_f[1].data_ptr()
    hip.cfg_sample(a)
    order.append(("cfg_softmax_top50_750x3x16384", 2 * P * S * V * 4 + P * S * 416))
    torch.cuda.synchronize()
    print(json.dumps({"traffic_probe_launch_order": order}))


def run_host_dropins():
    """The C++ drop-ins that keep the reference's host-vector signatures
    (levo2.cpp_amd/bench/host_dropins.cpp: Sampler::sample_streams on host
    logits, flow::solve_flow_euler with a host velocity callback, a host F32
    chunk quantized to Q8_0), timed wall-clock with their PCIe transfers. Run
    as a child process before this one touches the GPU."""
    exe = os.path.join(ROOT, "levo2.cpp_amd", "bench", "host_dropins")
    if not os.path.exists(exe):
        return {"error": f"{exe} is not built"}
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        return {"error": f"host_dropins rc={r.returncode}: {r.stderr[-400:]}"}
    return json.loads(r.stdout.strip().splitlines()[-1])


def host_dropin_references(gpu):
    """The reference side of the host drop-ins on one host core: the
    reference's own Sampler::sample_streams (oracle/_ref), the oracle port of
    solve_flow_euler's loop (src/levo-flow-renderer.cpp:57-120: in-context
    rows, callback, require_finite, Euler update, require_finite) with the
    same fixed-velocity callback, and the oracle port of ggml_quantize_chunk
    to Q8_0 on the same [4096, 1536] F32 chunk (3 warm-ups, median of 10)."""
    from oracle.levo_oracle import Oracle, Reference, have_reference
    orc = Oracle()
    out = {}
    with pinned(1):
        if have_reference():
            ref = Reference()
            V = 16385
            streams = (orc.gaussian(3 * V, 10) * 3).reshape(3, V)
            recent = (np.arange(150, dtype=np.int64) * 97 % (V - 1)).reshape(3, 50)
            s2 = ref.sampler(2)
            t = median_seconds(lambda: s2.sample_streams(streams, use_sampling=True, temperature=0.9, top_k_mixed=50,
                                                         top_k_detail=1, repetition_penalty=1.1, recent=recent,
                                                         ignore=(0, 1, 2)))
            out["sample_streams_3x16385"] = {"gpu_dropin_us": gpu.get("sample_streams_3x16385_us"),
                                             "reference_cpu_us": round(t * 1e6, 1), "kind": "reference"}
        F, L, P, steps = 1000, 64, 250, 50
        noise, ctx, vel = orc.gaussian(F * L, 20), orc.gaussian(F * L, 21), orc.gaussian(F * L, 22) * 0.1

        def solve():
            state = noise.copy()
            dt = np.float32(1.0) / np.float32(steps)
            for step in range(steps):
                t_ = np.float32(step) * dt
                orc.flow_incontext(state, noise, ctx, P * L, t_, 1e-4)
                v = vel  # the callback's fixed velocity
                if not np.isfinite(v).all():
                    raise ValueError
                orc.flow_cfg_euler(state, v, v, 1.0, dt)
                if not np.isfinite(state).all():
                    raise ValueError
            state[:P * L] = ctx[:P * L]
            return state

        t = median_seconds(solve)
        out["solve_flow_euler_1000x64_50_steps"] = {"gpu_dropin_us": gpu.get("solve_flow_euler_1000x64_50_steps_us"),
                                                    "reference_cpu_us": round(t * 1e6, 1), "kind": "port"}
        x = (orc.gaussian(4096 * 1536, 30) * 0.02).reshape(4096, 1536)
        t = median_seconds(lambda: orc.quantize(8, x))
        out["quantize_chunk_q8_0_4096x1536"] = {"gpu_dropin_us": gpu.get("quantize_chunk_q8_0_4096x1536_host_us"),
                                                "reference_cpu_us": round(t * 1e6, 1), "kind": "port"}
    for e in out.values():
        if e.get("gpu_dropin_us"):
            e["speedup"] = round(e["reference_cpu_us"] / e["gpu_dropin_us"], 2)
    out["note"] = ("wall-clock per call, host buffers in and out (PCIe transfers included); reference side on one "
                   "pinned host core")
    return out


OP_GROUPS = ("snake", "flow", "norm", "sample", "quant", "gemv", "conv", "vae")

# The result line is the last line of stdout and has to stay small enough for
# a log tail to hold it whole; the full per-op tables go to a file instead.
LINE_BUDGET = 7168


def ops_summary(ops):
    """One [us per launch, GB/s, fraction of 8 TB/s, fraction of the streaming
    ceiling] entry per timed op ("group/name" for nested tables). Entries
    without an HBM figure (MFMA-bound convolutions, whole decoder windows)
    carry [us, TFLOP/s, fraction of the F32 MFMA peak, null]."""
    out = {}

    def num(v, nd):
        return None if v is None else round(float(v), nd)

    def visit(name, e):
        if not isinstance(e, dict):
            return
        us = e.get("us_per_launch")
        if us is None and "ms_per_step" in e:
            us = e["ms_per_step"] * 1e3
        if us is None and "ms_per_window" in e:
            us = e["ms_per_window"] * 1e3
        if us is not None and ("GB/s" in e or "TFLOP/s" in e):
            if e.get("bound") == "mfma" or ("GB/s" not in e):
                out[name] = [num(us, 2), num(e.get("TFLOP/s"), 1), num(e.get("frac_f32_mfma"), 3), None]
            else:
                out[name] = [num(us, 2), num(e["GB/s"], 1), num(e.get("frac"), 3), num(e.get("of_ceiling"), 3)]
            return
        for k, v in e.items():
            visit(f"{name}/{k}" if name else k, v)

    visit("", {k: v for k, v in ops.items() if k != "host_dropins"})
    return out


def compact_cpu(cpu):
    """The CPU leg without its per-op sample descriptions: headline keys plus
    [1-thread GB/s, all-threads GB/s] per op."""
    if not cpu:
        return cpu
    keep = ("value", "unit", "cores", "kind", "sample", "ms_per_step", "method")
    out = {k: cpu[k] for k in keep if k in cpu}
    if "one_thread" in cpu:
        out["one_thread"] = {k: cpu["one_thread"][k] for k in ("value", "unit", "cores", "sample")
                             if k in cpu["one_thread"]}
    if "cpu" in cpu:
        out["cpu_model"] = cpu["cpu"].get("model")
    if "ops" in cpu:
        per = {}
        for name, e in cpu["ops"].items():
            if not isinstance(e, dict):
                continue
            all_key = next((k for k in e if k.endswith("_threads_GB/s")), None)
            per[name] = [e.get("1_thread_GB/s"), e.get(all_key) if all_key else None]
        out["ops_GBps_1_and_all_threads"] = per
    return out


def final_line(full, ops_file=None):
    """The JSON result line: headline keys, config, roofline, the compact CPU
    leg and one short entry per op. Falls back to dropping the op summary if
    the line would exceed LINE_BUDGET bytes, so the headline always fits."""
    line = {k: v for k, v in full.items() if k not in ("ops", "cpu_baseline")}
    line["cpu_baseline"] = compact_cpu(full.get("cpu_baseline"))
    if full.get("ops"):
        line["ops_summary_fields"] = ["us", "GB/s (TFLOP/s if MFMA-bound)", "frac of 8 TB/s (of F32 MFMA peak)",
                                      "of streaming ceiling"]
        line["ops_summary"] = ops_summary(full["ops"])
        if ops_file:
            line["ops_full_table"] = os.path.relpath(ops_file, ROOT)
    text = json.dumps(line, separators=(",", ":"))
    if len(text.encode()) > LINE_BUDGET:
        log(f"result line {len(text)} B exceeds {LINE_BUDGET} B: op summary left to the full table")
        line.pop("ops_summary", None)
        line.pop("ops_summary_fields", None)
        line["ops_summary_dropped"] = True
        text = json.dumps(line, separators=(",", ":"))
    if len(text.encode()) > LINE_BUDGET:
        raise SystemExit(f"bench.py: result line of {len(text)} B exceeds {LINE_BUDGET} B")
    return text


def run_ops(torch, hip, binding, head, dev, args, groups):
    """The op table: every group in `groups`, the same shapes whether run
    alone (--only) or after the headline."""
    w, k = args.warmup, args.steps
    ops = {}
    if "snake" in groups:
        log("ops: snake 1 s")
        ops["snake_beta_128x48000"] = bench_snake_1s(torch, hip, head, dev, w, k)
    if "flow" in groups:
        log("ops: flow")
        ops["flow_cfg_euler_64x2520"] = bench_flow(torch, hip, head, dev, w, k)
        log("ops: flow window step")
        ops["flow_window_step_1000x64_rows2200"] = bench_flow_window(torch, hip, binding, head, dev, w, k)
    if "norm" in groups:
        for layer, name in ((False, "rmsnorm"), (True, "layernorm")):
            for rows, D in ((756, 2048), (756, 1536), (1, 2048), (2, 2048)):
                log(f"ops: {name} {rows}x{D}")
                ops[f"residual_{name}_f16_{rows}x{D}"] = bench_norm(torch, hip, head, dev, w, k, layer, rows, D)
        log("ops: layernorm f32 2000x2200 (Flow estimator)")
        ops["residual_layernorm_f32_2000x2200"] = bench_norm(torch, hip, head, dev, w, k, True, 2000, 2200, f16=False)
        log("ops: gated residual + layernorm + modulation f32 2000x2200 (Flow estimator block boundary)")
        ops["gated_residual_layernorm_adaln_f32_2000x2200"] = bench_norm_modulated(torch, hip, binding, head, dev,
                                                                                   w, k)
    if "sample" in groups:
        log("ops: cfg sample")
        ops["cfg_softmax_top50_750x3x16384"] = bench_sample(torch, hip, binding, head, dev, w, k)
        log("ops: decode-step sampling")
        ops["decode_step_sample_1x3x16385"] = bench_decode_step(torch, hip, binding, head, dev, w, k)
    if "quant" in groups:
        log("ops: quant")
        ops.update(bench_quant(torch, hip, head, dev, w, k))
    if "gemv" in groups:
        log("ops: q8_0 mat-vec")
        ops["mul_mat_q8_0"] = bench_mul_mat(torch, hip, head, dev, w, k)
        log("ops: k-quant mat-vec")
        ops["mul_mat_kquant"] = bench_mul_mat_kquant(torch, hip, head, dev, w, k)
    if "conv" in groups:
        log("ops: snake conv1d")
        ops["snake_conv1d"] = bench_snake_conv(torch, hip, head, dev, w, k)
    if "vae" in groups:
        for frames in (252, 1000):
            log(f"ops: vae decoder window of {frames} frames")
            ops[f"vae_decode_{frames}_frames"] = bench_vae_decode(torch, hip, binding, head, dev, w, k, frames)
    return ops


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-ops", action="store_true", help="only the headline ladder")
    p.add_argument("--only", default="",
                   help="comma-separated op groups to run alone (snake,flow,norm,sample,quant,gemv,conv,vae); "
                        "prints the op table without the headline ladder")
    p.add_argument("--ceiling", action="store_true",
                   help="with --only: annotate each op with the plain streaming ceiling of its bytes and mix")
    p.add_argument("--traffic-probe", action="store_true",
                   help="one launch per kernel + a 256 MiB copy, for rocprofv3 --pmc runs")
    p.add_argument("--ops-out", default=os.path.join(ROOT, "gpurun_out", "bench_ops.json"),
                   help="file for the full per-op and CPU tables (the result line carries a summary); "
                        "empty to skip")
    args = p.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        sys.stderr.write("bench.py measures one MI355X: this build has no multi-GPU path "
                         "(every op shards without exchange; see the sharding notes). Run with --gpus 1.\n")
        return 2

    host_dropins = None if (args.no_ops or args.only or args.traffic_probe) else run_host_dropins()
    import torch
    if not torch.cuda.is_available():
        sys.stderr.write("bench.py needs a GPU\n")
        return 1
    binding = load_binding()
    hip = binding.LevoHip()
    dev = torch.device("cuda:0")
    log(f"device: {torch.cuda.get_device_name(0)}")
    if args.traffic_probe:
        traffic_probe(torch, hip, binding, dev)
        return 0

    head = HeadStart(torch)
    if args.only:
        ops = run_ops(torch, hip, binding, head, dev, args, set(args.only.split(",")))
        if args.ceiling:
            add_ceilings(torch, head, dev, ops, args.warmup, args.steps)
        print(json.dumps({"ops": ops}))
        return 0
    log("ladder: start")
    lad = bench_ladder(torch, hip, head, dev, args.warmup, args.steps)
    log(f"ladder: {lad['ms_per_step']:.4f} ms/step (six launches: {lad['ms_per_step_six']:.4f})")
    # the headline's kernel: one levo_hip_snake_beta_batch launch moves the whole ladder
    achieved = lad["ladder_bytes"] / (lad["ms_per_step"] * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS, "unit": "GB/s",
                "frac": round(achieved / PEAK_GBPS, 4), "traffic": None,
                "kernel": "snake_beta_batch_kernel", "shape": LADDER,
                "algorithmic_bytes_per_launch": lad["ladder_bytes"], "us_per_launch": round(lad["ms_per_step"] * 1e3, 3)}
    traffic_file = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(traffic_file):
        try:
            tr = json.load(open(traffic_file)).get("snake_beta_batch_ladder")
            if tr:
                roofline["traffic"] = tr["hbm_bytes_per_launch"]
        except (ValueError, KeyError):
            pass
    (C, T), dom_ms = lad["dominant"]
    largest = {"kernel": "snake_beta_vec<float, 2>", "shape": [C, T], "us_per_launch": round(dom_ms * 1e3, 3),
               "GB/s": round(snake_bytes(C, T) / (dom_ms * 1e-3) / 1e9, 1)}

    ops = {"snake_beta_ladder_shapes": lad["per_shape"], "snake_beta_largest_shape_alone": largest,
           "snake_beta_ladder_six_launches": {"ms_per_step": round(lad["ms_per_step_six"], 5),
                                              "GB/s": round(lad["ladder_bytes"] / (lad["ms_per_step_six"] * 1e-3) / 1e9,
                                                            1)}}
    if not args.no_ops:
        ops.update(run_ops(torch, hip, binding, head, dev, args, OP_GROUPS))
        log("ops: host-vector drop-ins (reference side)")
        ops["host_dropins"] = (host_dropin_references(host_dropins) if "error" not in host_dropins
                               else host_dropins)
        log("ops: streaming ceilings")
        add_ceilings(torch, head, dev, ops, args.warmup, args.steps)

    cpu = None
    if not args.no_cpu:
        log("cpu baseline: start")
        cpu = cpu_baseline(lad["host"], with_ops=not args.no_ops)
        log("cpu baseline: done")

    value = lad["ladder_bytes"] / (lad["ms_per_step"] * 1e-3) / 1e9
    full = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(lad["ms_per_step"], 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "SnakeBeta ladder of one 10.08 s Oobleck VAE window, F32, one batched launch over "
                               "the six shapes (levo_hip_snake_beta_batch)",
                   "shapes_CxT": LADDER, "elements_per_step": 72253440,
                   "algorithmic_bytes_per_step": lad["ladder_bytes"], "frac_of_8TBps": round(value / PEAK_GBPS, 4),
                   "rotated_buffer_sets": lad["n_sets"]},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "ops": ops,
    }
    if args.ops_out:
        os.makedirs(os.path.dirname(os.path.abspath(args.ops_out)), exist_ok=True)
        with open(args.ops_out, "w") as fh:
            json.dump(full, fh, indent=1)
        log(f"full op and CPU tables: {args.ops_out}")
    print(final_line(full, ops_file=args.ops_out or None))
    return 0


if __name__ == "__main__":
    sys.exit(main())
