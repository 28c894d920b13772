"""Turns rocprofv3 CSV output into the summaries kept under ``profiles/``.

    # per-kernel duration table from a --kernel-trace --stats run
    python -m tensors_amd.profiling stats <dir>/run_kernel_stats.csv --title "..." --cmd "..."

    # per-launch HBM traffic from two --pmc runs (FETCH_SIZE, then WRITE_SIZE)
    # of ``bench.py --probe``, calibrated against the probe's copy kernel
    python -m tensors_amd.profiling traffic --fetch <dir>/run_counter_collection.csv \
        --write <dir>/run_counter_collection.csv --json profiles/<name>.json --cmd "..."

FETCH_SIZE / WRITE_SIZE are L2 <-> memory kilobytes per dispatch.  The
calibration kernel is ``tf_add`` over ``bench.PROBE_CAL_N`` floats (reads
2 x 4 x N bytes, writes 4 x N bytes): the factor measured/known for it is
divided out of every other kernel's reading.
"""
from __future__ import annotations

import argparse
import csv
import json
import sys
from collections import defaultdict
from pathlib import Path

# Kernels of bench.py --probe (C2 step): label -> (name substring, algorithmic bytes per launch)
N2 = 2048
C2_KERNELS = {
    "gemm_f32_fwd_c2": ("gemm_f32_dl_kernel<true, true>", 4 * (3 * N2 * N2 + N2)),
    "gemm_f32_bwd_dx_c2": ("gemm_f32_dl_kernel<true, false>", 4 * 3 * N2 * N2),
    "gemm_f32_bwd_dw_c2": ("gemm_f32_dl_kernel<false, false>", 4 * 3 * N2 * N2),
}
CAL_NAME = "binary_kernel"


def per_dispatch(path: str | Path, counter: str) -> dict[str, list[float]]:
    """kernel name -> per-dispatch value of `counter` (summed over instances)."""
    sums: dict[tuple[str, str], float] = defaultdict(float)
    names: dict[str, str] = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            sums[(r["Dispatch_Id"], r["Counter_Name"])] += float(r["Counter_Value"])
            names[r["Dispatch_Id"]] = r["Kernel_Name"]
    out: dict[str, list[float]] = defaultdict(list)
    for (disp, _), v in sums.items():
        out[names[disp]].append(v)
    return out


def _match(table: dict[str, list[float]], sub: str) -> list[float]:
    vals = [v for name, vs in table.items() if sub in name for v in vs]
    if not vals:
        raise SystemExit(f"no dispatch of a kernel matching {sub!r}")
    return vals


def traffic(fetch_csv, write_csv, cal_n: int) -> dict:
    fetch = per_dispatch(fetch_csv, "FETCH_SIZE")
    write = per_dispatch(write_csv, "WRITE_SIZE")
    cal_read, cal_write = 2 * 4 * cal_n, 4 * cal_n
    cal_f = sum(_match(fetch, CAL_NAME)) / len(_match(fetch, CAL_NAME)) * 1024.0
    cal_w = sum(_match(write, CAL_NAME)) / len(_match(write, CAL_NAME)) * 1024.0
    f_scale, w_scale = cal_read / cal_f, cal_write / cal_w
    res = {"calibration": {"kernel": f"tf_add over {cal_n} floats", "known_read_bytes": cal_read,
                           "known_write_bytes": cal_write, "measured_fetch_bytes": round(cal_f),
                           "measured_write_bytes": round(cal_w), "fetch_scale": round(f_scale, 4),
                           "write_scale": round(w_scale, 4)}}
    for label, (sub, algo) in C2_KERNELS.items():
        fv, wv = _match(fetch, sub), _match(write, sub)
        fb = sum(fv) / len(fv) * 1024.0 * f_scale
        wb = sum(wv) / len(wv) * 1024.0 * w_scale
        res[label] = {"kernel": sub, "fetch_bytes": round(fb), "write_bytes": round(wb),
                      "traffic_bytes": round(fb + wb), "algorithmic_bytes": algo,
                      "traffic_over_algorithmic": round((fb + wb) / algo, 3), "dispatches": len(fv)}
    bwd = [res["gemm_f32_bwd_dx_c2"], res["gemm_f32_bwd_dw_c2"]]
    res["gemm_f32_bwd_c2"] = round(sum(r["traffic_bytes"] for r in bwd) / 2)  # bench.py roofline.traffic
    return res


def stats_table(path: str | Path, top: int = 25) -> str:
    rows = list(csv.DictReader(open(path, newline="")))
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    lines = ["| kernel | calls | total ms | avg us | min us | max us | % |", "|---|---:|---:|---:|---:|---:|---:|"]
    for r in rows[:top]:
        name = r["Name"].replace("(anonymous namespace)::", "").replace("|", "\\|")
        if len(name) > 110:
            name = name[:107] + "..."
        lines.append(f"| `{name}` | {r['Calls']} | {float(r['TotalDurationNs']) / 1e6:.3f} | "
                     f"{float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                     f"{float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.1f} |")
    return "\n".join(lines)


def phase_table(trace_csv: str | Path, phases: list[tuple[str, int]], match: list[str]) -> str:
    """Mean duration per bench phase of each kernel matching a substring in
    `match`: its dispatches in launch order are split into consecutive groups
    of the given sizes (e.g. warmup, timed, per-kernel events)."""
    per: dict[str, list[tuple[int, int]]] = defaultdict(list)
    with open(trace_csv, newline="") as f:
        for r in csv.DictReader(f):
            per[r["Kernel_Name"]].append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    head = "| kernel | " + " | ".join(f"{p} (n={n}) avg us" for p, n in phases) + " |"
    lines = [head, "|---|" + "---:|" * len(phases)]
    for sub in match:
        for kname in sorted(n for n in per if sub in n):
            spans = sorted(per[kname])
            cells, i = [], 0
            for _, n in phases:
                group = spans[i:i + n]
                i += n
                cells.append(f"{sum(e - s for s, e in group) / len(group) / 1e3:.2f}" if group else "—")
            name = kname.replace("(anonymous namespace)::", "").replace("|", "\\|")
            lines.append(f"| `{name[:110]}` | " + " | ".join(cells) + " |")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m tensors_amd.profiling")
    sub = ap.add_subparsers(dest="action", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("--title", required=True)
    s.add_argument("--cmd", required=True, help="the rocprofv3 command that produced the CSV")
    s.add_argument("--out")
    s.add_argument("--trace", help="the run's kernel_trace.csv, for a per-phase table")
    s.add_argument("--phases", help="phase sizes in dispatches per kernel, e.g. warmup=50,timed=100,events=100")
    s.add_argument("--match", nargs="*", default=[], help="kernel-name substrings for the per-phase table")
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--cal-n", type=int, default=1 << 26)
    t.add_argument("--json", required=True)
    t.add_argument("--cmd", required=True, nargs="+", help="the two rocprofv3 commands")
    a = ap.parse_args(argv)
    if a.action == "stats":
        text = f"# {a.title}\n\nCommand (repo root):\n\n```\n{a.cmd}\n```\n\n{stats_table(a.csv)}\n"
        if a.trace and a.phases:
            phases = [(p.split("=")[0], int(p.split("=")[1])) for p in a.phases.split(",")]
            text += ("\nPer phase (each kernel's dispatches in launch order, split into the bench's phases):\n\n"
                     f"{phase_table(a.trace, phases, a.match)}\n")
        if a.out:
            Path(a.out).write_text(text)
        else:
            sys.stdout.write(text)
    else:
        res = traffic(a.fetch, a.write, a.cal_n)
        res["commands"] = a.cmd
        Path(a.json).write_text(json.dumps(res, indent=2) + "\n")
        print(json.dumps(res, indent=2))
    return 0


if __name__ == "__main__":
    sys.exit(main())
