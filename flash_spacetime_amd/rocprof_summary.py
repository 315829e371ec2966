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
  python -m flash_spacetime_amd.rocprof_summary --counters DIR [DIR ...] [--trace DIR] \
      [--md OUT.md] [--command "..."]

The second form summarises any counter passes (`--pmc ...`, csv output) of
the library kernels: the mean reading per launch, and utilisation figures
derived with the GPU's own geometry from rocprofv3's agent_info.csv
(`GRBM_GUI_ACTIVE` counts cycles on every XCD, `SQ_VALU_MFMA_BUSY_CYCLES`
on every SIMD, `SQ_LDS_BANK_CONFLICT` on every CU; `SQ_ACTIVE_INST_*` and
`SQ_WAVE_CYCLES` / `SQ_WAIT_*` are in units of four cycles).
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
          "worklist_kernel": "worklist"}


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


def read_agent(directory: str):
    """(XCDs, CUs, SIMDs) of the GPU agent in rocprofv3's agent_info.csv."""
    with open(_find(directory, "agent_info.csv")) as f:
        for r in csv.DictReader(f):
            if r.get("Agent_Type") == "GPU":
                return int(r["Num_Xcc"]), int(r["Cu_Count"]), int(r["Simd_Count"])
    raise SystemExit("no GPU agent in agent_info.csv")


def read_all_counters(directories):
    vals = defaultdict(lambda: defaultdict(list))
    for d in directories:
        with open(_find(d, "counter_collection.csv")) as f:
            for r in csv.DictReader(f):
                ph = phase_of(r["Kernel_Name"])
                if ph in ("fwd", "bwd_rows", "bwd_cols"):
                    vals[ph][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return {ph: {c: sum(v) / len(v) for c, v in cs.items()} for ph, cs in vals.items()}


def counters_main(args):
    xcc, cus, simds = read_agent(args.counters[0])
    data = read_all_counters(args.counters)
    loop = read_trace_loop(args.trace) if args.trace else {}
    phases = [ph for ph in ("fwd", "bwd_rows", "bwd_cols") if ph in data]

    def derived(c):
        out = {}
        if "GRBM_GUI_ACTIVE" in c:
            cyc = c["GRBM_GUI_ACTIVE"] / xcc  # cycles of one XCD over the launch
            out["cycles"] = cyc
            if "SQ_VALU_MFMA_BUSY_CYCLES" in c:
                out["MFMA busy (per SIMD)"] = c["SQ_VALU_MFMA_BUSY_CYCLES"] / (cyc * simds)
            if "SQ_ACTIVE_INST_VALU" in c:
                out["VALU issue (per SIMD)"] = 4 * c["SQ_ACTIVE_INST_VALU"] / (cyc * simds)
            if "SQ_ACTIVE_INST_LDS" in c:
                out["LDS issue (per SIMD)"] = 4 * c["SQ_ACTIVE_INST_LDS"] / (cyc * simds)
            if "SQ_LDS_BANK_CONFLICT" in c:
                out["LDS bank-conflict stall (per CU)"] = c["SQ_LDS_BANK_CONFLICT"] / (cyc * cus)
        if "SQ_WAVE_CYCLES" in c:
            for k, name in (("SQ_WAIT_INST_ANY", "waves waiting on a dependency"),
                            ("SQ_WAIT_ANY", "waves waiting (any)"),
                            ("SQ_ACTIVE_INST_ANY", "waves issuing")):
                if k in c:
                    out[name] = c[k] / c["SQ_WAVE_CYCLES"]
        if "SQ_VALU_MFMA_BUSY_CYCLES" in c and c.get("SQ_INSTS_MFMA"):
            out["cycles per MFMA"] = c["SQ_VALU_MFMA_BUSY_CYCLES"] / c["SQ_INSTS_MFMA"]
        return out

    der = {ph: derived(data[ph]) for ph in phases}
    names = []
    for ph in phases:
        for k in der[ph]:
            if k not in names:
                names.append(k)
    lines = ["| | " + " | ".join(phases) + " |", "|---|" + "---|" * len(phases)]
    if loop:
        lines.append("| timing-loop avg (us, kernel trace) | " + " | ".join(
            f"{loop[ph]:.1f}" if ph in loop else "" for ph in phases) + " |")
    for k in names:
        cells = []
        for ph in phases:
            v = der[ph].get(k)
            cells.append("" if v is None else (f"{v:.4g}" if k in ("cycles", "cycles per MFMA") else f"{100 * v:.1f} %"))
        lines.append(f"| {k} | " + " | ".join(cells) + " |")
    raw = ["| counter (mean per launch) | " + " | ".join(phases) + " |", "|---|" + "---|" * len(phases)]
    counters = sorted({c for ph in phases for c in data[ph]})
    for c in counters:
        raw.append(f"| {c} | " + " | ".join(f"{data[ph].get(c, float('nan')):.4g}" for ph in phases) + " |")
    md = "\n".join([
        *(["Command:", "", "```", args.command, "```", ""] if args.command else []),
        f"GPU: {xcc} XCDs, {cus} CUs, {simds} SIMDs (rocprofv3 agent_info).", "",
        *lines, "", *raw, "",
    ])
    if args.md:
        with open(args.md, "w") as f:
            f.write(md)
    else:
        print(md)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--trace")
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--counters", nargs="+",
                    help="counter-pass directories to summarise (second form); --trace optional")
    ap.add_argument("--calib-bytes", type=float, default=float(2 ** 30),
                    help="bytes the calibration kernel reads (and writes) per dispatch")
    ap.add_argument("--md")
    ap.add_argument("--json")
    ap.add_argument("--command", default="")
    args = ap.parse_args()
    if args.counters:
        counters_main(args)
        return
    if not (args.trace and args.fetch and args.write):
        ap.error("--trace, --fetch and --write are required (or --counters)")

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
             "| HBM bytes / launch (scaled) | grid | LDS (B) |",
             "|---|---|---|---|---|---|---|---|---|"]
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
                     f"{m.get('LDS_Block_Size', '')} |")
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
