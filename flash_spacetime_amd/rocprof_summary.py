"""Summarise rocprofv3 CSV output of `bench.py` into the figures the bench reports.

Reads a `--kernel-trace --stats` run (kernel_stats.csv) and two counter runs
(`--pmc FETCH_SIZE`, `--pmc WRITE_SIZE`, counter_collection.csv), all made with
`--output-format csv`, of the same bench command with `--calibrate-copy`. The
calibration kernel (an fp32 multiply by 1.0 over a buffer of known size, one
read and one write per element) gives the factor between each counter's
reading (KiB per dispatch) and the bytes actually moved; the library kernels'
readings are scaled by it.

Writes a markdown summary (stdout or --md) and a JSON file (--json) with the
per-launch HBM bytes of each library kernel, which bench.py reports as the
roofline's `traffic`.

Usage:
  python -m flash_spacetime_amd.rocprof_summary --trace DIR --fetch DIR --write DIR \
      [--md OUT.md] [--json OUT.json] [--command "..."]
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import os
from collections import defaultdict

CALIB_TAG = "MulFunctor"           # torch's elementwise multiply kernel
# Kernel-name fragments of each phase: the bf16 kernels (fwd2/bwd_rows2/bwd_cols2)
# and the fp32 ones (fwd/bwd_rows/bwd_cols) share a phase.
PHASES = {"fwd2_kernel": "fwd", "fwd_kernel": "fwd",
          "bwd_rows2_kernel": "bwd_rows", "bwd_rows_kernel": "bwd_rows",
          "bwd_cols2_kernel": "bwd_cols", "bwd_cols_kernel": "bwd_cols",
          "dw_reduce_seg_kernel": "bwd_reduce_seg", "dw_reduce_final_kernel": "bwd_reduce_final",
          "blkcum_kernel": "worklist", "sort_events_kernel": "worklist_sort"}


def _find(directory: str, suffix: str) -> str:
    hits = sorted(glob.glob(os.path.join(directory, "**", f"*{suffix}"), recursive=True))
    if not hits:
        raise FileNotFoundError(f"no *{suffix} under {directory}")
    return hits[0]


def phase_of(kernel_name: str) -> str | None:
    for tag, phase in PHASES.items():
        if tag in kernel_name:
            return phase
    if CALIB_TAG in kernel_name:
        return "calibration_copy"
    return None


def read_stats(directory: str):
    rows = {}
    with open(_find(directory, "kernel_stats.csv")) as f:
        for r in csv.DictReader(f):
            ph = phase_of(r["Name"])
            if ph:
                rows.setdefault(ph, []).append(r)
    out = {}
    for ph, rs in rows.items():
        calls = sum(int(r["Calls"]) for r in rs)
        total = sum(float(r["TotalDurationNs"]) for r in rs)
        out[ph] = {"calls": calls, "avg_us": total / calls / 1e3, "names": [r["Name"] for r in rs]}
    return out


def read_trace_loop(directory: str, n: int = 10):
    """Mean duration (us) of each phase's last n dispatches in the kernel
    trace: the per-phase timing loop that bench.py runs after its steps (n
    back-to-back launches of one kernel), i.e. the launches the bench's own
    HIP-event figure covers. Empty when the trace file is absent."""
    try:
        path = _find(directory, "kernel_trace.csv")
    except FileNotFoundError:
        return {}
    durs = defaultdict(list)
    with open(path) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    for r in rows:
        ph = phase_of(r["Kernel_Name"])
        if ph:
            durs[ph].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    return {ph: sum(v[-n:]) / len(v[-n:]) for ph, v in durs.items() if len(v) >= n}


def read_counter(directory: str, counter: str):
    vals = defaultdict(list)
    meta = {}
    with open(_find(directory, "counter_collection.csv")) as f:
        for r in csv.DictReader(f):
            if r.get("Counter_Name") != counter:
                continue
            ph = phase_of(r["Kernel_Name"])
            if not ph:
                continue
            vals[ph].append(float(r["Counter_Value"]))
            meta[ph] = {k: r.get(k) for k in ("Grid_Size", "Workgroup_Size", "LDS_Block_Size", "VGPR_Count",
                                              "Accum_VGPR_Count", "SGPR_Count")}
    return {ph: sum(v) / len(v) for ph, v in vals.items()}, meta


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--trace", required=True)
    ap.add_argument("--fetch", required=True)
    ap.add_argument("--write", required=True)
    ap.add_argument("--calib-bytes", type=float, default=float(2 ** 30),
                    help="bytes the calibration kernel reads (and writes) per dispatch")
    ap.add_argument("--md")
    ap.add_argument("--json")
    ap.add_argument("--command", default="")
    args = ap.parse_args()

    stats = read_stats(args.trace)
    loop = read_trace_loop(args.trace)
    fetch, meta = read_counter(args.fetch, "FETCH_SIZE")
    write, _ = read_counter(args.write, "WRITE_SIZE")
    if "calibration_copy" not in fetch or "calibration_copy" not in write:
        raise SystemExit("calibration kernel missing: run bench.py with --calibrate-copy")
    f_scale = args.calib_bytes / (fetch["calibration_copy"] * 1024.0)
    w_scale = args.calib_bytes / (write["calibration_copy"] * 1024.0)

    traffic = {}
    lines = ["| kernel | launches | avg duration (us) | timing-loop avg (us) | FETCH_SIZE (KiB) | WRITE_SIZE (KiB) "
             "| HBM bytes / launch (scaled) | grid | VGPR | AGPR | LDS (B) |",
             "|---|---|---|---|---|---|---|---|---|---|---|"]
    for ph in ("fwd", "bwd_rows", "bwd_cols", "bwd_reduce_seg", "bwd_reduce_final", "worklist", "worklist_sort"):
        if ph not in stats:
            continue
        fk, wk = fetch.get(ph), write.get(ph)
        nbytes = None
        if fk is not None and wk is not None:
            nbytes = fk * 1024.0 * f_scale + wk * 1024.0 * w_scale
            traffic[ph] = {"bytes": nbytes, "fetch_kib": fk, "write_kib": wk, "avg_us": stats[ph]["avg_us"]}
            if ph in loop:
                traffic[ph]["loop_avg_us"] = loop[ph]
        m = meta.get(ph, {})
        lp = f"{loop[ph]:.1f}" if ph in loop else ""
        lines.append(f"| {ph} | {stats[ph]['calls']} | {stats[ph]['avg_us']:.1f} | {lp} | "
                     f"{'' if fk is None else f'{fk:.0f}'} | {'' if wk is None else f'{wk:.0f}'} | "
                     f"{'' if nbytes is None else f'{nbytes:.4g}'} | {m.get('Grid_Size', '')} | "
                     f"{m.get('VGPR_Count', '')} | {m.get('Accum_VGPR_Count', '')} | {m.get('LDS_Block_Size', '')} |")
    md = "\n".join([
        *(["Command:", "", "```", args.command, "```", ""] if args.command else []),
        f"Calibration: fp32 multiply-by-1 over {args.calib_bytes / 2 ** 30:.2f} GiB read + the same written: "
        f"FETCH_SIZE {fetch['calibration_copy']:.0f} KiB (scale {f_scale:.3f}), "
        f"WRITE_SIZE {write['calibration_copy']:.0f} KiB (scale {w_scale:.3f}).",
        "",
        *lines,
        "",
    ])
    if args.md:
        with open(args.md, "w") as f:
            f.write(md)
    else:
        print(md)
    if args.json:
        with open(args.json, "w") as f:
            json.dump({"fetch_scale": f_scale, "write_scale": w_scale, "kernels": traffic}, f, indent=1)


if __name__ == "__main__":
    main()
