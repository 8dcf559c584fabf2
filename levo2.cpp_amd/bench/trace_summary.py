"""Summarize a rocprofv3 kernel trace (CSV) of bench.py per kernel and launch
shape: one row per (kernel, grid, workgroup) with the dispatch count and the
average / min / max duration, so that the ops that share a kernel at several
shapes (the ladder rungs, the norm row counts, the mat-vec matrices) each get
their own row. Library kernels only (levo_hip:: and the streaming-ceiling
kernels of bench.py); torch's own kernels (input generation, the timing head
start) and HIP's copies are left out.

    python3 levo2.cpp_amd/bench/trace_summary.py <kernel_trace.csv> > table.md

With --vae, the HBM bytes of each of the 31 steps of the last VAE decode (a
split-K convolution's combine launch counted with its split launch)
in two rocprofv3 --pmc runs of `bench.py --only vae` (FETCH_SIZE, then
WRITE_SIZE), scaled by the copy factors in traffic.json, beside the bytes of
the launch's activations (inputs and outputs once) and weights:

    python3 levo2.cpp_amd/bench/trace_summary.py --vae <fetch_counter_collection.csv>
        <write_counter_collection.csv> profiles/traffic.json <frames> > table.md

With --vae-trace, each step of the last decode of each window size in a
kernel trace of `bench.py --only vae` (a split-K convolution and its combine
launch as one step), with its duration and TFLOP/s:

    python3 levo2.cpp_amd/bench/trace_summary.py --vae-trace <kernel_trace.csv> > table.md

With --traffic, the HBM bytes per launch of bench.py --traffic-probe from two
rocprofv3 --pmc runs (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each
scaled by what the counter reads for the probe's first launch, a plain
device-to-device copy of known size; writes traffic.json (read by bench.py)
and prints the table:

    python3 levo2.cpp_amd/bench/trace_summary.py --traffic <fetch_counter_collection.csv>
        <write_counter_collection.csv> <probe stdout> <traffic.json> > traffic.md

With --issue, per launch of the same probe from one rocprofv3 --pmc run of SQ
counters: waves, instructions per wave by kind, wave lifetime and the share
of it spent issuing VALU work:

    python3 levo2.cpp_amd/bench/trace_summary.py --issue <sq_counter_collection.csv> <probe stdout> > issue.md
"""
from __future__ import annotations

import csv
import json
import re
import sys
from collections import defaultdict


N_SIMDS = 256 * 4     # MI355X: 256 CUs of 4 SIMDs
CLOCK_MHZ = 2400.0    # engine clock (cycles per microsecond)
N_SE = 32             # shader engines (8 XCDs of 4) that SQ_BUSY_CYCLES is summed over


def short_name(name: str) -> str | None:
    if "levo_hip::" in name or "stream_kernel" in name:
        n = re.sub(r"^void ", "", name)
        n = re.sub(r"levo_hip::(\(anonymous namespace\)::)?", "", n)
        n = re.sub(r"\(anonymous namespace\)::", "", n)
        return re.sub(r"\(.*\)$", "", n).strip()
    return None


def summarize(path: str) -> list[str]:
    groups = defaultdict(list)
    for r in csv.DictReader(open(path)):
        n = short_name(r["Kernel_Name"])
        if n is None:
            continue
        wg = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"])
        grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        groups[(n, grid // max(wg, 1), wg)].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    rows = ["| kernel | workgroups | threads | calls | avg us | min us | max us |",
            "|---|---:|---:|---:|---:|---:|---:|"]
    for (n, wgs, wg), d in sorted(groups.items(), key=lambda kv: (kv[0][0], kv[0][1])):
        rows.append(f"| `{n}` | {wgs} | {wg} | {len(d)} | {sum(d) / len(d) / 1e3:.3f} | {min(d) / 1e3:.3f} | "
                    f"{max(d) / 1e3:.3f} |")
    return rows


def counters(path: str, counter: str) -> list[tuple[int, str, float]]:
    out = []
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] != counter:
            continue
        n = r["Kernel_Name"]
        if "levo_hip::" in n or "copyBuffer" in n:
            out.append((int(r["Dispatch_Id"]), n, float(r["Counter_Value"])))
    return sorted(out)


def traffic(fetch_csv: str, write_csv: str, probe_log: str, json_out: str) -> list[str]:
    order = None
    for line in open(probe_log):
        if "traffic_probe_launch_order" in line:
            order = json.loads(line[line.index("{"):])["traffic_probe_launch_order"]
    fe = counters(fetch_csv, "FETCH_SIZE")
    wr = counters(write_csv, "WRITE_SIZE")
    if order is None or not (len(fe) == len(order) == len(wr)):
        raise SystemExit(f"launch counts differ: order {None if order is None else len(order)}, "
                         f"fetch {len(fe)}, write {len(wr)}")
    copy_bytes = order[0][1]  # the copy reads and writes copy_bytes / 2 each
    fscale = (copy_bytes / 2) / (fe[0][2] * 1024)
    wscale = (copy_bytes / 2) / (wr[0][2] * 1024)
    res = {"fetch_scale": fscale, "write_scale": wscale}
    rows = [f"Counter scale (bytes per counted byte, from the {copy_bytes // 2:,}-byte copy): "
            f"FETCH_SIZE {fscale:.4f}, WRITE_SIZE {wscale:.4f}", "",
            "| launch | kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes (scaled) | algorithmic bytes | ratio |",
            "|---|---|---:|---:|---:|---:|---:|"]
    for (name, alg), (_, kn, f), (_, kn2, w) in zip(order, fe, wr):
        assert kn == kn2
        hbm = f * 1024 * fscale + w * 1024 * wscale
        res[name] = {"hbm_bytes_per_launch": int(round(hbm)), "algorithmic_bytes": alg, "fetch_kib": f,
                     "write_kib": w}
        kname = short_name(kn) or kn.split("(")[0].strip()
        rows.append(f"| {name} | `{kname}` | {f:.1f} | {w:.1f} | {int(round(hbm)):,} | {alg:,} | {hbm / alg:.4f} |")
    json.dump(res, open(json_out, "w"), indent=1)
    return rows


def vae_flops(frames: int) -> list[float]:
    """2 * C_out * C_in * taps * T_out of each of the 31 launches (both convs
    of a one-launch residual unit; a transposed-conv output sample takes 2
    taps per input channel)."""
    out = [2.0 * 2048 * 64 * 7 * frames]
    t = frames
    for ci, co, st in zip((2048, 1024, 512, 256, 128), (1024, 512, 256, 128, 128), (10, 6, 4, 4, 2)):
        t *= st
        out.append(2.0 * co * ci * 2 * t)
        for _ in range(3):
            k7, k1 = 2.0 * co * co * 7 * t, 2.0 * co * co * t
            out += [k7, k1] if co > 128 else [k7 + k1]
    return out + [2.0 * 2 * 128 * 7 * t]


def is_combine(name: str) -> bool:
    return "split_combine" in name


def vae_trace(path: str) -> list[str]:
    launches = []
    for r in csv.DictReader(open(path)):
        n = short_name(r["Kernel_Name"])
        if n is None or "pack_transpose" in n or "stream_kernel" in n:
            continue
        wg = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"])
        grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        launches.append((int(r["Start_Timestamp"]), n, grid // max(wg, 1),
                         int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
    launches.sort()
    # a split-K convolution is two launches, the split one and its combine:
    # one step of the decode, timed from the first's start to the second's end
    steps = []
    for start, n, wgs, ns in launches:
        if is_combine(n) and steps:
            s0, n0, w0, _ = steps[-1]
            steps[-1] = (s0, n0 + " + combine", w0, start + ns - s0)
        else:
            steps.append((start, n, wgs, ns))
    per = len(vae_launches(1))
    decodes = [steps[i:i + per] for i in range(0, len(steps) - per + 1, per)]
    rows = []
    for frames in (252, 1000):
        # the output conv's grid tells the window size: 1024 of the frames * 1920 samples per workgroup
        mine = [d for d in decodes if d[-1][2] == -(-frames * 1920 // 1024)]
        if not mine:
            continue
        d = mine[-1]
        labels = [lab for lab, _, _ in vae_launches(frames)]
        flops = vae_flops(frames)
        rows += [f"#### {frames} frames ({frames * 1920 / 48000:.2f} s of audio)", "",
                 "| step | kernel | grid (WGs) | µs | TFLOP/s |", "|---|---|---:|---:|---:|"]
        for lab, (_, n, wgs, ns), fl in zip(labels, d, flops):
            rows.append(f"| {lab} | `{n}` | {wgs} | {ns / 1e3:.1f} | {fl / ns / 1e3:.1f} |")
        tot = d[-1][0] + d[-1][3] - d[0][0]
        busy = sum(x[3] for x in d)
        rows += [f"| **total** (first start to last end; {busy / 1e3:.1f} µs inside the steps) | | | "
                 f"**{tot / 1e3:.1f}** | **{sum(flops) / tot / 1e3:.1f}** |", ""]
    return rows


def vae_launches(frames: int) -> list[tuple[str, int, int]]:
    """(label, activation bytes, weight bytes) of the decoder's 31 launches in
    order: the input conv; per stage the SnakeBeta + upsampler, then three
    residual units (two launches at 256-1024 channels, k = 7 then k = 1 with
    the residual add; one at 128); the SnakeBeta + output conv."""
    f4 = 4
    out = [("input conv 64->2048 k7", (64 + 2048) * frames * f4, (2048 * 64 * 7 + 2048) * f4)]
    t = frames
    for s, (ci, co, st) in enumerate(zip((2048, 1024, 512, 256, 128), (1024, 512, 256, 128, 128),
                                         (10, 6, 4, 4, 2))):
        t_in, t = t, t * st
        out.append((f"stage {s + 1} snake+upsample {ci}->{co} x{st}", (ci * t_in + co * t) * f4,
                    (ci * co * 2 * st + co + 2 * ci) * f4))
        for d in (1, 3, 9):
            if co > 128:
                out.append((f"stage {s + 1} snake+conv k7 d{d} {co}", 2 * co * t * f4, (co * co * 7 + 3 * co) * f4))
                out.append((f"stage {s + 1} snake+conv k1 +res {co}", 3 * co * t * f4, (co * co + 3 * co) * f4))
            else:
                out.append((f"stage {s + 1} residual unit d{d} {co} (one launch)", 2 * co * t * f4,
                            (co * co * 8 + 6 * co) * f4))
    out.append(("snake+output conv 128->2 k7", (128 + 2) * t * f4, (2 * 128 * 7 + 2 * 128) * f4))
    return out


def vae_traffic(fetch_csv: str, write_csv: str, traffic_json: str, frames: str) -> list[str]:
    scales = json.load(open(traffic_json))
    labels = vae_launches(int(frames))
    def lib(rows):
        # HIP's copies left out; a split-K convolution's combine counted with its split launch
        steps = []
        for r in rows:
            if "levo_hip::" not in r[1]:
                continue
            if is_combine(r[1]) and steps:
                steps[-1] = (steps[-1][0], steps[-1][1], steps[-1][2] + r[2])
            else:
                steps.append(r)
        return steps[-len(labels):]
    fe = lib(counters(fetch_csv, "FETCH_SIZE"))
    wr = lib(counters(write_csv, "WRITE_SIZE"))
    rows = [f"FETCH_SIZE x {scales['fetch_scale']:.4f}, WRITE_SIZE x {scales['write_scale']:.4f} (the copy factors "
            f"of traffic.json); the last {len(labels)} launches of each run, the {frames}-frame decode.", "",
            "| launch | activations (MB) | weights (MB) | FETCH (MB) | WRITE (MB) | HBM ÷ (activations + weights) |",
            "|---|---:|---:|---:|---:|---:|"]
    tot = [0.0] * 4
    for (label, act, wts), (_, _, f), (_, _, w) in zip(labels, fe, wr):
        fb = f * 1024 * scales["fetch_scale"]
        wb = w * 1024 * scales["write_scale"]
        for i, v in enumerate((act, wts, fb, wb)):
            tot[i] += v
        rows.append(f"| {label} | {act / 1e6:.1f} | {wts / 1e6:.1f} | {fb / 1e6:.1f} | {wb / 1e6:.1f} | "
                    f"{(fb + wb) / (act + wts):.2f} |")
    rows.append(f"| **total** | **{tot[0] / 1e6:.0f}** | **{tot[1] / 1e6:.0f}** | **{tot[2] / 1e6:.0f}** | "
                f"**{tot[3] / 1e6:.0f}** | **{(tot[2] + tot[3]) / (tot[0] + tot[1]):.2f}** |")
    return rows


def issue(sq_csv: str, probe_log: str) -> list[str]:
    """Per launch of bench.py --traffic-probe, from one rocprofv3 --pmc run of
    SQ_WAVES, SQ_INSTS_VALU, SQ_INSTS_SALU, SQ_INSTS_VMEM_RD, SQ_INSTS_LDS,
    SQ_WAVE_CYCLES, SQ_ACTIVE_INST_VALU, SQ_BUSY_CYCLES (+ GRBM_GUI_ACTIVE):
    instructions per wave, a wave's average lifetime and the share of it spent
    issuing VALU work (SQ_ACTIVE_INST_VALU / SQ_WAVE_CYCLES, both in the same
    per-wave cycle units)."""
    order = None
    for line in open(probe_log):
        if "traffic_probe_launch_order" in line:
            order = json.loads(line[line.index("{"):])["traffic_probe_launch_order"]
    per = defaultdict(dict)
    names = {}
    for r in csv.DictReader(open(sq_csv)):
        n = r["Kernel_Name"]
        if not ("levo_hip::" in n or "copyBuffer" in n):
            continue
        did = int(r["Dispatch_Id"])
        per[did][r["Counter_Name"]] = per[did].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        names[did] = n
    ids = sorted(per)
    if order is None or len(ids) != len(order):
        raise SystemExit(f"launch counts differ: order {None if order is None else len(order)}, counted {len(ids)}")
    rows = ["| launch | kernel | waves | VALU / wave | SALU / wave | VMEM rd / wave | LDS / wave | "
            "wave lifetime (cycles) | VALU-active share of lifetime | VALU busy per SIMD (us) | "
            "VALU share of SQ-busy cycles |",
            "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for (name, _), did in zip(order, ids):
        c = per[did]
        waves = c.get("SQ_WAVES", 0.0) or 1.0
        life = c.get("SQ_WAVE_CYCLES", 0.0) / waves
        act = c.get("SQ_ACTIVE_INST_VALU", 0.0) / max(c.get("SQ_WAVE_CYCLES", 0.0), 1.0)
        # the launch's VALU issue cycles (4-cycle units) spread over the
        # GPU's SIMDs, at the 2.4 GHz engine clock: the shortest time the
        # launch's VALU work can take
        busy_us = c.get("SQ_ACTIVE_INST_VALU", 0.0) * 4.0 / N_SIMDS / CLOCK_MHZ
        # the same VALU cycles per SIMD over the launch's SQ-busy cycles per
        # shader engine (SQ_BUSY_CYCLES sums the engines): near 1 when every
        # SIMD issues VALU work for the whole launch
        se_busy = c.get("SQ_BUSY_CYCLES", 0.0) / N_SE
        share = c.get("SQ_ACTIVE_INST_VALU", 0.0) * 4.0 / N_SIMDS / se_busy if se_busy > 0 else 0.0
        kname = short_name(names[did]) or names[did].split("(")[0].strip()
        rows.append(f"| {name} | `{kname}` | {int(waves):,} | {c.get('SQ_INSTS_VALU', 0) / waves:.1f} | "
                    f"{c.get('SQ_INSTS_SALU', 0) / waves:.1f} | {c.get('SQ_INSTS_VMEM_RD', 0) / waves:.1f} | "
                    f"{c.get('SQ_INSTS_LDS', 0) / waves:.1f} | {life:.0f} | {act:.3f} | {busy_us:.2f} | "
                    f"{share:.2f} |")
    return rows


if __name__ == "__main__":
    if sys.argv[1] == "--issue":
        print("\n".join(issue(sys.argv[2], sys.argv[3])))
    elif sys.argv[1] == "--traffic":
        print("\n".join(traffic(*sys.argv[2:6])))
    elif sys.argv[1] == "--vae-trace":
        print("\n".join(vae_trace(sys.argv[2])))
    elif sys.argv[1] == "--vae":
        print("\n".join(vae_traffic(*sys.argv[2:6])))
    else:
        print("\n".join(summarize(sys.argv[1])))
