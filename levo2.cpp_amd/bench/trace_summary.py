"""Summarize a rocprofv3 kernel trace (CSV) of bench.py per kernel and launch
shape: one row per (kernel, grid, workgroup) with the dispatch count and the
average / min / max duration, so that the ops that share a kernel at several
shapes (the ladder rungs, the norm row counts, the mat-vec matrices) each get
their own row. Library kernels only (levo_hip:: and the streaming-ceiling
kernels of bench.py); torch's own kernels (input generation, the timing head
start) and HIP's copies are left out.

    python3 levo2.cpp_amd/bench/trace_summary.py <kernel_trace.csv> > table.md

With --traffic, the HBM bytes per launch of bench.py --traffic-probe from two
rocprofv3 --pmc runs (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each
scaled by what the counter reads for the probe's first launch, a plain
device-to-device copy of known size; writes traffic.json (read by bench.py)
and prints the table:

    python3 levo2.cpp_amd/bench/trace_summary.py --traffic <fetch_counter_collection.csv>
        <write_counter_collection.csv> <probe stdout> <traffic.json> > traffic.md
"""
from __future__ import annotations

import csv
import json
import re
import sys
from collections import defaultdict


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


if __name__ == "__main__":
    if sys.argv[1] == "--traffic":
        print("\n".join(traffic(*sys.argv[2:6])))
    else:
        print("\n".join(summarize(sys.argv[1])))
