#!/usr/bin/env python3
"""Benchmark of the LeVo2 elementwise / reduction / broadcast kernels on one MI355X.

Headline workload (one "step"): the SnakeBeta ladder of one 10.08 s Oobleck
VAE window, F32 (C, T) = (2048,252), (1024,504), (512,2016), (256,8064),
(128,48384), (128,483840), one kernel launch per shape as the decoder issues
them, x ~ N(0,1), per-channel log-parameters ~ U(-0.5, 0.5), inputs resident
in HBM. `value` = ladder algorithmic bytes (read x + write y + parameters) per
step / wall time per step.

Also reported, per op (rotated buffer sets so that every timed launch reads
data untouched for >= 512 MB of traffic, i.e. from HBM, not the 256 MB
Infinity Cache): SnakeBeta 1 s config, Flow CFG+Euler (50 steps), residual +
RMSNorm / LayerNorm F16, CFG + softmax + argmax / top-50, Q8_0 / Q4_0
quantize / dequantize. Kernel durations come from HIP events recorded on the
stream the kernels run on (torch's current stream).

The CPU baseline is the CPU oracle (a port of the reference's ggml-cpu op
chains; ggml itself is not available) run on a bounded sample on this host.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import math
import os
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


class Timer:
    """Per-launch HIP events on torch's current stream."""

    def __init__(self, torch, n):
        self.ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
        self.i = 0

    def mark(self):
        self.ev[self.i].record()
        self.i += 1

    def durations_ms(self):
        return [self.ev[k].elapsed_time(self.ev[k + 1]) for k in range(self.i - 1)]


def time_op(torch, launch, n_sets, warmup, steps):
    """launch(set_index) enqueues one launch; returns mean ms per launch from
    back-to-back per-launch events (>= 512 MB between reuses of a set)."""
    for i in range(warmup):
        launch(i % n_sets)
    torch.cuda.synchronize()
    t = Timer(torch, steps)
    for i in range(steps):
        t.mark()
        launch(i % n_sets)
    t.mark()
    torch.cuda.synchronize()
    d = t.durations_ms()
    return float(np.mean(d)), float(np.min(d))


def op_entry(bytes_per_launch, ms, ms_min, **extra):
    gbps = bytes_per_launch / (ms * 1e-3) / 1e9
    e = {"bytes_per_launch": int(bytes_per_launch), "us_per_launch": round(ms * 1e3, 3),
         "us_min": round(ms_min * 1e3, 3), "GB/s": round(gbps, 1), "frac": round(gbps / PEAK_GBPS, 4)}
    e.update(extra)
    return e


def cpu_threads():
    try:
        return max(1, min(16, len(os.sched_getaffinity(0))))
    except AttributeError:
        return max(1, min(16, os.cpu_count() or 1))


# ---------------------------------------------------------------------------------------
def bench_ladder(torch, hip, dev, warmup, steps):
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

    def ladder(s, timer=None):
        for (C, T), (x, a, b, y) in zip(LADDER, sets[s]):
            if timer:
                timer.mark()
            hip.snake_beta(x, a, b, y)

    for i in range(warmup):
        ladder(i % n_sets)
    torch.cuda.synchronize()
    # timed region: K ladder steps, one event before every launch and one at the end
    timer = Timer(torch, steps * len(LADDER))
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        ladder(i % n_sets, timer)
    timer.mark()
    end.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms_total = start.elapsed_time(end)
    d = np.array(timer.durations_ms()).reshape(steps, len(LADDER))
    per_shape = {}
    for j, (C, T) in enumerate(LADDER):
        per_shape[f"{C}x{T}"] = op_entry(snake_bytes(C, T), float(d[:, j].mean()), float(d[:, j].min()))
    host = [(t[0].cpu().numpy(), t[1].cpu().numpy(), t[2].cpu().numpy()) for t in sets[0]]
    return dict(ms_per_step=ms_total / steps, wall_ms=wall_ms, per_shape=per_shape,
                ladder_bytes=per_set, host=host, n_sets=n_sets,
                dominant=(LADDER[-1], float(d[:, -1].mean())))


def bench_snake_1s(torch, hip, dev, warmup, steps):
    C, T = 128, 48000
    per = snake_bytes(C, T)
    n = math.ceil(ROTATE_BYTES / per) + 1
    rng = np.random.default_rng(11)
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    bufs = [(torch.randn((C, T), generator=g, device=dev), torch.from_numpy(rng.uniform(-0.5, 0.5, C).astype(np.float32)).to(dev),
             torch.from_numpy(rng.uniform(-0.5, 0.5, C).astype(np.float32)).to(dev)) for _ in range(n)]
    outs = [torch.empty((C, T), device=dev) for _ in range(n)]
    ms, mn = time_op(torch, lambda i: hip.snake_beta(bufs[i][0], bufs[i][1], bufs[i][2], outs[i]), n, warmup, steps)
    return op_entry(per, ms, mn, shape=[C, T], dtype="f32")


def bench_flow(torch, hip, dev, warmup, steps):
    n_el, nsteps = 64 * 2520, 50
    per = 16 * n_el
    n_sets = math.ceil(ROTATE_BYTES / (per * nsteps)) + 1
    g = torch.Generator(device=dev)
    g.manual_seed(50)
    xs = [torch.randn(n_el, generator=g, device=dev) for _ in range(n_sets)]
    vs = [[(torch.randn(n_el, generator=g, device=dev), torch.randn(n_el, generator=g, device=dev))
           for _ in range(nsteps)] for _ in range(n_sets)]
    dt = float(np.float32(1) / np.float32(nsteps))

    def solve(s, timer=None):
        for k in range(nsteps):
            if timer:
                timer.mark()
            hip.flow_cfg_euler(xs[s], vs[s][k][0], vs[s][k][1], n_el, 1.5, dt)

    for i in range(warmup):
        solve(i % n_sets)
    torch.cuda.synchronize()
    reps = max(1, steps // 5)
    timer = Timer(torch, reps * nsteps)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(reps):
        solve(i % n_sets, timer)
    timer.mark()
    end.record()
    torch.cuda.synchronize()
    d = np.array(timer.durations_ms())
    solve_ms = start.elapsed_time(end) / reps
    # the same 50 launches captured once into a HIP graph and replayed
    graph_ms = None
    try:
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            solve(0)
        torch.cuda.synchronize()
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        gs, ge = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        gs.record()
        for _ in range(reps):
            graph.replay()
        ge.record()
        torch.cuda.synchronize()
        graph_ms = gs.elapsed_time(ge) / reps
    except Exception as e:  # graph capture is an extra measurement only
        log(f"flow graph capture skipped: {e}")
    e = op_entry(per, float(d.mean()), float(d.min()), shape=[1, 64, 2520], dtype="f32",
                 solve_50_steps_ms=round(solve_ms, 4), solve_50_steps_GBps=round(per * nsteps / (solve_ms * 1e-3) / 1e9, 1))
    if graph_ms is not None:
        e["solve_50_steps_graph_ms"] = round(graph_ms, 4)
    return e


def bench_norm(torch, hip, dev, warmup, steps, layer, rows, D):
    per = 8 * rows * D + (4 * D if layer else 2 * D)
    n = max(2, math.ceil(ROTATE_BYTES / per) + 1) if rows > 2 else 64
    g = torch.Generator(device=dev)
    g.manual_seed(rows * D + layer)
    mk = lambda shape, s=1.0, m=0.0: (torch.randn(shape, generator=g, device=dev) * s + m).half()
    w, b = mk(D, 0.02, 1.0), mk(D, 0.02)
    sets = [(mk((rows, D)), mk((rows, D)), torch.empty((rows, D), device=dev, dtype=torch.float16),
             torch.empty((rows, D), device=dev, dtype=torch.float16)) for _ in range(n)]
    if layer:
        fn = lambda i: hip.layer_norm(1, sets[i][0], sets[i][1], w, b, 1, sets[i][2], sets[i][3], rows, D, 1e-6)
    else:
        fn = lambda i: hip.rms_norm(1, sets[i][0], sets[i][1], w, 1, sets[i][2], sets[i][3], rows, D, 1e-6)
    ms, mn = time_op(torch, fn, n, warmup, max(steps, 20))
    return op_entry(per, ms, mn, shape=[rows, D], dtype="f16 io / f32 accumulate")


def bench_sample(torch, hip, binding, dev, warmup, steps):
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
    ms, mn = time_op(torch, lambda i: hip.cfg_sample(args[i]), n, warmup, steps)
    return op_entry(per, ms, mn, shape=[P, 2, S, V], dtype="f32", top_k=50, temperature=0.9)


def bench_quant(torch, hip, dev, warmup, steps):
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
        ms, mn = time_op(torch, lambda i: hip.quantize_rows(qt, src[i], 1, Cc, Cc, q[i], R, Cc), n, warmup, steps)
        out[f"{name}_quantize_f16"] = op_entry(per_q, ms, mn, shape=[R, Cc])
        ms, mn = time_op(torch, lambda i: hip.dequantize(qt, q[i], deq[i], 0, R * Cc), n, warmup, steps)
        out[f"{name}_dequantize_f32"] = op_entry(per_d, ms, mn, shape=[R, Cc])
        del src, q, deq
        torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------------------
def cpu_baseline(host_ladder, budget_s=12.0):
    """The oracle's five-pass ggml-cpu SnakeBeta chain on the ladder, all host threads."""
    from oracle.levo_oracle import Oracle
    orc = Oracle()
    threads = cpu_threads()
    total_bytes = sum(snake_bytes(x.shape[0], x.shape[1]) for x, _, _ in host_ladder)
    done, t0 = 0, time.perf_counter()
    while True:
        for x, a, b in host_ladder:
            orc.snake_beta(x, a, b, threads=threads)
        done += 1
        if time.perf_counter() - t0 > budget_s or done >= 50:
            break
    secs = time.perf_counter() - t0
    return {"value": round(total_bytes * done / secs / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "ms_per_step": round(secs / done * 1e3, 2),
            "sample": f"{done} full ladders (72,253,440 elements each) through the oracle's five-pass "
                      f"ggml-cpu chain (mul, sin, sqr, div, add), {threads} threads, rows split as ggml-cpu"}


def cpu_ops_baselines():
    """Bounded CPU timings of the other ops (single sample each)."""
    from oracle.levo_oracle import Oracle, Reference, have_reference
    orc = Oracle()
    threads = cpu_threads()
    res = {}
    rows, D = 756, 2048
    x = orc.f32_to_f16(orc.gaussian(rows * D, 1).reshape(rows, D))
    d = orc.f32_to_f16(orc.gaussian(rows * D, 2).reshape(rows, D))
    w = orc.f32_to_f16(orc.gaussian(D, 3) * 0.02 + 1)
    t0 = time.perf_counter()
    reps = 0
    while time.perf_counter() - t0 < 1.0:
        orc.rms_norm(x, d, w, 1e-6, threads=threads)
        reps += 1
    res["rmsnorm_f16_756x2048"] = {"GB/s": round(8 * rows * D * reps / (time.perf_counter() - t0) / 1e9, 3),
                                   "cores": threads, "kind": "port"}
    n = 64 * 2520
    st, vu, vc = orc.gaussian(n, 4), orc.gaussian(n, 5), orc.gaussian(n, 6)
    t0 = time.perf_counter()
    reps = 0
    while time.perf_counter() - t0 < 0.5:
        orc.flow_cfg_euler(st, vu, vc, 1.5, 0.02)
        reps += 1
    res["flow_cfg_euler"] = {"GB/s": round(16 * n * reps / (time.perf_counter() - t0) / 1e9, 3), "cores": 1,
                             "kind": "port"}
    xq = orc.f32_to_f16((orc.gaussian(4096 * 1536, 7) * 0.02).reshape(4096, 1536))
    t0 = time.perf_counter()
    orc.quantize_f16_padded(8, xq, 1536)
    secs = time.perf_counter() - t0
    res["q8_0_quantize_f16"] = {"GB/s": round((2 + 34 / 32) * xq.size / secs / 1e9, 3), "cores": 1, "kind": "port"}
    if have_reference():
        ref = Reference()
        V = 16384
        c = orc.gaussian(60 * V, 8) * 3
        u = orc.gaussian(60 * V, 9) * 3
        s = ref.sampler(1)
        t0 = time.perf_counter()
        for r in range(60):
            l = ref.apply_cfg(c[r * V:(r + 1) * V], u[r * V:(r + 1) * V], 1.5)
            s.sample(l, 50, 0.9, True)
        secs = time.perf_counter() - t0
        res["cfg_sample_top50"] = {"GB/s": round(60 * 2 * V * 4 / secs / 1e9, 3), "rows_per_s": round(60 / secs, 1),
                                   "cores": 1, "kind": "reference",
                                   "sample": "60 rows of 16384: levo::apply_cfg + Sampler::sample(top-50, T=0.9)"}
    return res


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-ops", action="store_true", help="only the headline ladder")
    args = p.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        sys.stderr.write("bench.py measures one MI355X: this build has no multi-GPU path "
                         "(every op shards without exchange; see the sharding notes). Run with --gpus 1.\n")
        return 2

    import torch
    if not torch.cuda.is_available():
        sys.stderr.write("bench.py needs a GPU\n")
        return 1
    binding = load_binding()
    hip = binding.LevoHip()
    dev = torch.device("cuda:0")
    log(f"device: {torch.cuda.get_device_name(0)}")

    log("ladder: start")
    lad = bench_ladder(torch, hip, dev, args.warmup, args.steps)
    log(f"ladder: {lad['ms_per_step']:.4f} ms/step")
    (C, T), dom_ms = lad["dominant"]
    dom_bytes = snake_bytes(C, T)
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS, "unit": "GB/s",
                "frac": round(achieved / PEAK_GBPS, 4), "traffic": None,
                "kernel": "snake_beta_vec<float,4>", "shape": [C, T], "algorithmic_bytes_per_launch": dom_bytes,
                "us_per_launch": round(dom_ms * 1e3, 3)}
    traffic_file = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(traffic_file):
        try:
            tr = json.load(open(traffic_file)).get("snake_beta_128x483840")
            if tr:
                roofline["traffic"] = tr["hbm_bytes_per_launch"]
        except (ValueError, KeyError):
            pass

    ops = {"snake_beta_ladder_shapes": lad["per_shape"]}
    if not args.no_ops:
        log("ops: snake 1 s")
        ops["snake_beta_128x48000"] = bench_snake_1s(torch, hip, dev, args.warmup, args.steps)
        log("ops: flow")
        ops["flow_cfg_euler_64x2520"] = bench_flow(torch, hip, dev, args.warmup, args.steps)
        for layer, name in ((False, "rmsnorm"), (True, "layernorm")):
            for rows, D in ((756, 2048), (756, 1536), (1, 2048), (2, 2048)):
                log(f"ops: {name} {rows}x{D}")
                ops[f"residual_{name}_f16_{rows}x{D}"] = bench_norm(torch, hip, dev, args.warmup, args.steps, layer, rows, D)
        log("ops: cfg sample")
        ops["cfg_softmax_top50_750x3x16384"] = bench_sample(torch, hip, binding, dev, args.warmup, args.steps)
        log("ops: quant")
        ops.update(bench_quant(torch, hip, dev, args.warmup, args.steps))

    cpu = None
    if not args.no_cpu:
        log("cpu baseline: start")
        cpu = cpu_baseline(lad["host"])
        if not args.no_ops:
            cpu["ops"] = cpu_ops_baselines()
        log("cpu baseline: done")

    value = lad["ladder_bytes"] / (lad["ms_per_step"] * 1e-3) / 1e9
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(lad["ms_per_step"], 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "SnakeBeta ladder of one 10.08 s Oobleck VAE window, F32, one launch per shape",
                   "shapes_CxT": LADDER, "elements_per_step": 72253440,
                   "algorithmic_bytes_per_step": lad["ladder_bytes"], "frac_of_8TBps": round(value / PEAK_GBPS, 4),
                   "rotated_buffer_sets": lad["n_sets"]},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "ops": ops,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
