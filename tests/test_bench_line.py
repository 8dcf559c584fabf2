"""bench.py's result line: built from a synthetic result shaped like a full
run (every op group, nested mat-vec / conv tables, the CPU leg with per-op
figures) it parses as JSON, keeps the headline keys, the roofline and the CPU
baseline, and stays within the byte budget a log tail holds whole."""
from __future__ import annotations

import importlib.util
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    argv, sys.argv = sys.argv, ["bench.py"]
    try:
        spec.loader.exec_module(mod)
    finally:
        sys.argv = argv
    return mod


def _hbm(us, gbps):
    return {"bytes_per_launch": 123456789, "us_per_launch": us, "GB/s": gbps, "frac": round(gbps / 8000, 4),
            "read_bytes": 98765432, "write_bytes": 24691357, "dtype": "f16 io / f32 accumulate",
            "ceiling_GB/s": 4321.0, "ceiling_vectors_per_thread": 4, "of_ceiling": 0.876,
            "rotated_sets": 12, "shape": [4096, 1536]}


def _mfma(us):
    return {"us_per_launch": us, "TFLOP/s": 97.7, "frac_f32_mfma": 0.6212, "bytes_per_launch": 495452160,
            "GB/s": 436.2, "bound": "mfma", "shape": [1024, 2520, 7, 9]}


def synthetic_full(n_flat=36, n_nested=32):
    ops = {f"residual_layernorm_f32_gate_adaln_{i:03d}x2200": _hbm(15.663, 4495.8) for i in range(n_flat)}
    ops["mul_mat_kquant"] = {f"q6_K_ffn_down_1536x8960_{i:02d}": _hbm(10.407, 1088.0) for i in range(n_nested // 2)}
    ops["snake_conv1d"] = {f"stage5_k7_d{i:02d}": _mfma(1135.8) for i in range(n_nested // 2)}
    ops["vae_decode_1000_frames"] = {"frames": 1000, "ms_per_window": 52.395, "TFLOP/s": 93.0,
                                     "frac_f32_mfma": 0.591, "bound": "mfma", "launches": 31}
    ops["host_dropins"] = {"solve_flow_euler_1000x64_50_steps": {"gpu_dropin_us": 3456.0,
                                                                 "reference_cpu_us": 1206.0, "kind": "reference"}}
    cpu_ops = {f"op_{i:02d}": {"1_thread_GB/s": 1.398, "16_threads_GB/s": 16.115, "1_thread_ms": 35.157,
                               "16_threads_ms": 3.05, "bytes": 49153024, "kind": "port",
                               "sample": "the five-pass ggml-cpu chain, rows split over threads " * 2}
               for i in range(20)}
    ladder = [[2048, 252], [1024, 504], [512, 2016], [256, 8064], [128, 48384], [128, 483840]]
    return {
        "metric": "achieved HBM GB/s & % of 8 TB/s peak per op; ms per 10.08 s VAE Snake ladder",
        "value": 6251.0, "unit": "GB/s", "n_gpus": 1, "steps": 20, "warmup": 5, "ms_per_step": 0.09248,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "SnakeBeta ladder of one 10.08 s Oobleck VAE window, F32, one batched launch",
                   "shapes_CxT": ladder, "elements_per_step": 72253440},
        "roofline": {"bound": "hbm", "achieved": 6251.0, "peak": 8000.0, "unit": "GB/s", "frac": 0.7814,
                     "traffic": 578377457, "kernel": "snake_beta_batch_kernel", "shape": ladder},
        "cpu_baseline": {"value": 12.142, "unit": "GB/s", "cores": 16, "kind": "port", "ms_per_step": 47.61,
                         "sample": "the full ladder through the oracle's five-pass ggml-cpu chain, 16 threads",
                         "one_thread": {"value": 1.544, "unit": "GB/s", "cores": 1, "sample": "32 x 48384"},
                         "cpu": {"model": "AMD EPYC", "nproc": 16}, "method": "pinned; median of 10",
                         "ops": cpu_ops},
        "ops": ops,
    }


def test_line_fits_with_a_full_op_table():
    b = _bench()
    text = b.final_line(synthetic_full(), ops_file=os.path.join(ROOT, "gpurun_out", "bench_ops.json"))
    assert len(text.encode()) <= b.LINE_BUDGET
    assert "\n" not in text
    line = json.loads(text)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config"):
        assert key in line, key
    assert line["roofline"]["frac"] == 0.7814 and line["roofline"]["bound"] == "hbm"
    cpu = line["cpu_baseline"]
    assert (cpu["value"], cpu["cores"], cpu["kind"]) == (12.142, 16, "port") and cpu["sample"]
    assert cpu["ops_GBps_1_and_all_threads"]["op_00"] == [1.398, 16.115]
    s = line["ops_summary"]
    assert s["residual_layernorm_f32_gate_adaln_000x2200"] == [15.66, 4495.8, 0.562, 0.876]
    assert s["mul_mat_kquant/q6_K_ffn_down_1536x8960_00"][0] == 10.41
    assert s["snake_conv1d/stage5_k7_d00"] == [1135.8, 97.7, 0.621, None]
    assert s["vae_decode_1000_frames"] == [52395.0, 93.0, 0.591, None]
    assert not any(k.startswith("host_dropins") for k in s)
    assert line["ops_full_table"] == "gpurun_out/bench_ops.json"


def test_oversized_table_keeps_the_headline():
    b = _bench()
    text = b.final_line(synthetic_full(n_flat=400, n_nested=200))
    assert len(text.encode()) <= b.LINE_BUDGET
    line = json.loads(text)
    assert line["ops_summary_dropped"] is True and "ops_summary" not in line
    assert line["roofline"]["achieved"] == 6251.0 and line["cpu_baseline"]["value"] == 12.142


def test_headline_only_run():
    b = _bench()
    full = synthetic_full()
    full["ops"] = {}
    full["cpu_baseline"] = None
    line = json.loads(b.final_line(full))
    assert line["cpu_baseline"] is None and "ops_summary" not in line
