"""Turns rocprofv3 CSV output into the summaries kept under ``profiles/``.

    # per-kernel duration table from a --kernel-trace --stats run
    python -m tensors_amd.profiling stats <dir>/run_kernel_stats.csv --title "..." --cmd "..."

    # per-launch HBM traffic from two --pmc runs (FETCH_SIZE, then WRITE_SIZE)
    # of ``bench.py --probe c2`` (or ``--probe c5`` with ``--config c5``, or
    # ``--probe bw`` with ``--config bw``: the bandwidth kernels),
    # calibrated against the probe's tf_add kernel
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
CAL_NAME = "binary_kernel<float, AddOp>"

C5_DIMS = [4096, 8192, 8192, 4096, 1000]
C5_B = 4096
C5_PARAMS = sum(C5_DIMS[i + 1] * C5_DIMS[i] + C5_DIMS[i + 1] for i in range(4))   # 138,286,056

# The path's bandwidth kernels at their configurations' shapes (launched by
# ``bench.py --probe bw``): label -> (kernel-name substring, algorithmic
# bytes per launch).  Algorithmic bytes count each operand once: what a
# launch must read and write, not what its caches re-fetch.
R3, C3 = 4096, 1024                  # C3a / C3b: [4096 x 1024] fp32
L3 = 1024                            # C3c: LayerNorm [1024 x 1024]
CONV2 = (128, 32, 32, 32, 3, 16)     # C4 conv2: N, C, H, W, k, output side (stride 2, pad 1)
_conv_x = CONV2[0] * CONV2[1] * CONV2[2] * CONV2[3] * 4
_conv_col = CONV2[0] * CONV2[1] * CONV2[4] ** 2 * CONV2[5] ** 2 * 4
BW_KERNELS = {
    # logits read, dlogits written, int64 targets and the saved logsumexp read
    "ce_bwd_c3a": ("ce_kernel<float, 4, 1>", 2 * R3 * C3 * 4 + R3 * 8 + R3 * 4),
    # one pass: logits and targets read, dlogits and the per-row nll written
    "ce_fused_fwd_bwd_c3a": ("ce_kernel<float, 4, 2>", 2 * R3 * C3 * 4 + R3 * 8 + R3 * 4),
    "relu_bwd_c3b": ("binary_kernel<float, ReluBwdOp>", 3 * R3 * C3 * 4),
    # the whole op in one launch: dy, x read, dx written; gamma, mean, rstd
    # read; dgamma, dbeta written (the column blocks' read of x and dy and
    # their partials are not part of it)
    "layernorm_bwd_op_c3c": ("ln_bwd_onepass_kernel<4>", 3 * L3 * L3 * 4 + 3 * L3 * 4 + 2 * L3 * 4),
    # dy read, db written; the (strip, chunk) partials written and read back
    "colsum_c2": ("colsum_tile_kernel<float>", N2 * N2 * 4 + N2 * 4),
    # p, g, v read; p, v written (W and b in one launch)
    "sgd_c2": ("sgd_multi_kernel<false>", 20 * (N2 * N2 + N2)),
    # as above plus the bf16 copy of every parameter
    "sgd_c5": ("sgd_multi_kernel<true>", 22 * C5_PARAMS),
    "im2col_conv2_c4": ("im2col_plane4_kernel", _conv_x + _conv_col),
    "col2im_conv2_c4": ("col2im_plane_kernel<float, 2>", _conv_col + _conv_x),
    # C5 layer 1's ReLU backward with the next Linear's bias gradient
    # (bf16 [4096 x 8192]): dy, x read, dz written, db (fp32) written
    "relu_bwd_colsum_c5": ("relu_bwd_colsum_kernel<unsigned short>", 3 * C5_B * C5_DIMS[1] * 2 + C5_DIMS[1] * 4),
}
# Config 4's five implicit convolution launches (bench.py --probe c4):
# label -> (kernel-name substring, algorithmic bytes per launch: each
# operand read or written once).  conv1 (3 -> 32, 32 x 32, stride 1) and
# conv2 (32 -> 64, stride 2), batch 128, 3 x 3, pad 1.
_c4x1, _c4y1 = 128 * 3 * 32 * 32 * 4, 128 * 32 * 32 * 32 * 4
_c4x2, _c4y2 = 128 * 32 * 32 * 32 * 4, 128 * 64 * 16 * 16 * 4
_c4w1, _c4w2 = 32 * 27 * 4 + 32 * 4, 64 * 288 * 4 + 64 * 4
C4_KERNELS = {
    "conv1_fwd": ("conv_fwd_implicit_kernel<32>", _c4x1 + _c4y1 + _c4w1),
    "conv2_fwd": ("conv_fwd_implicit_kernel<64>", _c4x2 + _c4y2 + _c4w2),
    "conv1_dw_db": ("conv_bwd_weight_stream_kernel<true, true, false>", _c4x1 + _c4y1 + _c4w1),
    "conv2_dw_db": ("conv_bwd_weight_implicit_kernel<64>", _c4x2 + _c4y2 + _c4w2),
    "conv2_dx": ("conv_bwd_data_lds_kernel", _c4x2 + _c4y2 + _c4w2),
}
# The streaming-ceiling row (bench.py --hbm-ceiling: mix, non-temporal,
# MB per array) each kernel is read against: the mix of its reads and writes
# at the nearest array size.
BW_CEILING = {
    "ce_bwd_c3a": ("copy (1R+1W)", True, 16),
    "ce_fused_fwd_bwd_c3a": ("copy (1R+1W)", True, 16),
    "relu_bwd_c3b": ("2R+1W", True, 16),
    "layernorm_bwd_op_c3c": ("2R+1W", True, 4),
    "colsum_c2": ("read only (1R)", True, 16),
    "sgd_c2": ("3R+2W (SGD mix)", False, 16),
    "sgd_c5": ("3R+2W (SGD mix)", True, 512),
    "im2col_conv2_c4": ("copy (1R+1W)", True, 16),
    "col2im_conv2_c4": ("copy (1R+1W)", True, 16),
    "relu_bwd_colsum_c5": ("2R+1W", True, 64),
}
# The LayerNorm backward op as a whole (C3c): dy, x, dx, gamma, dgamma,
# dbeta, mean, rstd -- the block partials are not part of it.
LN_OP_BYTES = 3 * L3 * L3 * 4 + 3 * L3 * 4 + 2 * L3 * 4


def _kname(name: str) -> str:
    """Kernel name as the stats tables print it (no anonymous-namespace
    qualifiers), which the label tables' substrings are written against."""
    return name.replace("(anonymous namespace)::", "")


def per_dispatch(path: str | Path, counter: str) -> dict[str, list[float]]:
    """kernel name -> per-dispatch value of `counter` (summed over instances)."""
    sums: dict[tuple[str, str], float] = defaultdict(float)
    names: dict[str, str] = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            sums[(r["Dispatch_Id"], r["Counter_Name"])] += float(r["Counter_Value"])
            names[r["Dispatch_Id"]] = _kname(r["Kernel_Name"])
    out: dict[str, list[float]] = defaultdict(list)
    for (disp, _), v in sums.items():
        out[names[disp]].append(v)
    return out


def _match(table: dict[str, list[float]], sub: str) -> list[float]:
    vals = [v for name, vs in table.items() if sub in name for v in vs]
    if not vals:
        raise SystemExit(f"no dispatch of a kernel matching {sub!r}")
    return vals


def traffic(fetch_csv, write_csv, cal_n: int, kernels: dict | None = None) -> dict:
    """Calibrated HBM bytes per launch of each kernel in `kernels` (label ->
    (name substring, algorithmic bytes)); C2's GEMMs by default."""
    kernels = C2_KERNELS if kernels is None else kernels
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
    for label, (sub, algo) in kernels.items():
        fv, wv = _match(fetch, sub), _match(write, sub)
        fb = sum(fv) / len(fv) * 1024.0 * f_scale
        wb = sum(wv) / len(wv) * 1024.0 * w_scale
        res[label] = {"kernel": sub, "fetch_bytes": round(fb), "write_bytes": round(wb),
                      "traffic_bytes": round(fb + wb), "algorithmic_bytes": algo,
                      "traffic_over_algorithmic": round((fb + wb) / algo, 3), "dispatches": len(fv)}
    if kernels is C2_KERNELS:
        bwd = [res["gemm_f32_bwd_dx_c2"], res["gemm_f32_bwd_dw_c2"]]
        res["gemm_f32_bwd_c2"] = round(sum(r["traffic_bytes"] for r in bwd) / 2)  # bench.py roofline.traffic
    return res


# Config 5 (bench.py --probe c5): the step's GEMMs in launch order per step,
# (kind, M, N, K, output bytes per element): forward L1..L4, then per layer
# from the last: dW, dX (no dX for layer 1).  A split-K reduction dispatch
# belongs to the GEMM launched right before it.
def c5_gemm_order() -> list[tuple[str, int, int, int, int]]:
    d, B = C5_DIMS, C5_B
    seq = [("fwd", B, d[i + 1], d[i], 2) for i in range(4)]
    for i in range(3, -1, -1):
        seq.append(("dW", d[i + 1], d[i], B, 4))
        if i > 0:
            seq.append(("dX", B, d[i], d[i + 1], 2))
    return seq


def _ordered(path: str | Path, counter: str) -> list[tuple[str, float]]:
    """(kernel name, value of `counter` summed over instances) per dispatch, in
    dispatch order."""
    sums: dict[int, float] = defaultdict(float)
    names: dict[int, str] = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            d = int(r["Dispatch_Id"])
            sums[d] += float(r["Counter_Value"])
            names[d] = _kname(r["Kernel_Name"])
    return [(names[d], sums[d]) for d in sorted(sums)]


def traffic_c5(fetch_csv, write_csv, cal_n: int) -> dict:
    """Calibrated HBM bytes of config 5's GEMMs, by kind (fwd / dX / dW) per
    step and per launch, from two counter runs of ``bench.py --probe c5``."""
    fetch, write = _ordered(fetch_csv, "FETCH_SIZE"), _ordered(write_csv, "WRITE_SIZE")
    cal_read, cal_write = 2 * 4 * cal_n, 4 * cal_n
    cal_f = [v for n, v in fetch if CAL_NAME in n]
    cal_w = [v for n, v in write if CAL_NAME in n]
    if not cal_f or not cal_w:
        raise SystemExit("no calibration dispatch")
    f_scale = cal_read / (sum(cal_f) / len(cal_f) * 1024.0)
    w_scale = cal_write / (sum(cal_w) / len(cal_w) * 1024.0)
    order = c5_gemm_order()
    totals = {k: {"fetch_bytes": 0.0, "write_bytes": 0.0, "algorithmic_bytes": 0, "launches": 0}
              for k in ("fwd", "dX", "dW")}
    steps = 0
    for stream, key, scale in ((fetch, "fetch_bytes", f_scale), (write, "write_bytes", w_scale)):
        pos, count = -1, 0
        for name, v in stream:
            if "gemm_" in name:
                pos += 1
                count += 1
                kind, M, N, K, ob = order[pos % len(order)]
                totals[kind][key] += v * 1024.0 * scale
                if key == "fetch_bytes":
                    totals[kind]["algorithmic_bytes"] += 2 * (M * K + K * N) + ob * M * N
                    totals[kind]["launches"] += 1
            elif "splitk_reduce" in name and pos >= 0:
                totals[order[pos % len(order)][0]][key] += v * 1024.0 * scale
        if count % len(order):
            raise SystemExit(f"{count} GEMM dispatches is not a whole number of C5 steps")
        steps = count // len(order)
    res = {"calibration": {"kernel": f"tf_add over {cal_n} floats", "known_read_bytes": cal_read,
                           "known_write_bytes": cal_write, "fetch_scale": round(f_scale, 4),
                           "write_scale": round(w_scale, 4)},
           "steps": steps}
    for kind, t in totals.items():
        tb = t["fetch_bytes"] + t["write_bytes"]
        res[f"gemm_bf16_{kind}_c5"] = {
            "launches_per_step": t["launches"] // steps,
            "fetch_bytes_per_step": round(t["fetch_bytes"] / steps),
            "write_bytes_per_step": round(t["write_bytes"] / steps),
            "traffic_bytes_per_step": round(tb / steps),
            "algorithmic_bytes_per_step": t["algorithmic_bytes"] // steps,
            "traffic_over_algorithmic": round(tb / t["algorithmic_bytes"], 3)}
    bwd = [res["gemm_bf16_dX_c5"], res["gemm_bf16_dW_c5"]]
    n_bwd = sum(r["launches_per_step"] for r in bwd)
    res["gemm_bf16_bwd_c5"] = round(sum(r["traffic_bytes_per_step"] for r in bwd) / n_bwd)  # bench roofline.traffic
    return res


def _gemm_positions(rows: list[tuple[str, float]]) -> list[list[float]]:
    """Values of the GEMM dispatches of ``bench.py --probe c5`` grouped by
    position in c5_gemm_order (one entry per step)."""
    order = c5_gemm_order()
    vals = [v for n, v in rows if "gemm_" in n]
    if len(vals) % len(order):
        raise SystemExit(f"{len(vals)} GEMM dispatches is not a whole number of C5 steps")
    return [[vals[i] for i in range(pos, len(vals), len(order))] for pos in range(len(order))]


def _trace_ordered(trace_csv: str | Path) -> list[tuple[str, float]]:
    rows = []
    with open(trace_csv, newline="") as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), _kname(r["Kernel_Name"]),
                         (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
    rows.sort()
    return [(n, d) for _, n, d in rows]


def mfma_table(runs: list[tuple[str, str, str]]) -> str:
    """Per C5 GEMM shape: MFMA busy (the derived counter MfmaUtil: MFMA busy
    cycles over GPU-active cycles x SIMDs) and kernel duration, for each run
    (label, counter CSV of --pmc MfmaUtil, kernel_trace.csv), both of
    ``bench.py --probe c5``."""
    cols = []
    for label, pmc, trace in runs:
        util = _gemm_positions(_ordered(pmc, "MfmaUtil"))
        dur = _gemm_positions(_trace_ordered(trace))
        names = [n for n, _ in _trace_ordered(trace) if "gemm_" in n][:len(c5_gemm_order())]
        cols.append((label, util, dur, names))
    head = "| GEMM | M x N x K | " + " | ".join(
        f"{lab}: kernel | {lab}: MFMA busy | {lab}: us | {lab}: TF/s" for lab, *_ in cols) + " |"
    lines = [head, "|---|---|" + "---|---:|---:|---:|" * len(cols)]
    tot = [[0.0, 0.0, 0.0] for _ in cols]        # bwd: flop, us, busy x us
    for pos, (kind, M, N, K, _) in enumerate(c5_gemm_order()):
        cells = []
        for ci, (lab, util, dur, names) in enumerate(cols):
            u = sum(util[pos]) / len(util[pos])
            d = sum(dur[pos]) / len(dur[pos])
            flop = 2.0 * M * N * K
            k = names[pos].split("(")[0].replace("void ", "")
            cells.append(f"`{k}` | {u:.1f} % | {d:.1f} | {flop / d / 1e6:.0f}")
            if kind != "fwd":
                tot[ci][0] += flop
                tot[ci][1] += d
                tot[ci][2] += u * d
        lines.append(f"| {kind} | {M} x {N} x {K} | " + " | ".join(cells) + " |")
    cells = [f"backward | {t[2] / t[1]:.1f} % (time-weighted) | {t[1]:.1f} | {t[0] / t[1] / 1e6:.0f}" for t in tot]
    lines.append("| all dW + dX | | " + " | ".join(cells) + " |")
    return "\n".join(lines)


def c5_api_order() -> list[tuple[str, int, int, int]]:
    """The config-5 step's GEMMs in the order the C++ API launches them:
    forward L1..L4, then the engine's backward from the last layer, each
    LinearBackward computing dX before dW (no dX for layer 1)."""
    d, B = C5_DIMS, C5_B
    seq = [("fwd", B, d[i + 1], d[i]) for i in range(4)]
    for i in range(3, -1, -1):
        if i > 0:
            seq.append(("dX", B, d[i], d[i + 1]))
        seq.append(("dW", d[i + 1], d[i], B))
    return seq


def c5_gemm_table(trace_csv: str | Path, bench_line: dict | None = None, tail_steps: int = 0) -> str:
    """Mean kernel time of each GEMM of the config-5 step from a kernel trace
    of the C++ API step (GEMM dispatches in launch order, 11 per step; a
    split-K reduction counts with the GEMM before it: from the GEMM's start
    to the reduction's end), over all steps and over the last `tail_steps`
    (the bench's event-timed steps), beside the bench's event timing of the
    same GEMM when its JSON line is given."""
    rows = []
    with open(trace_csv, newline="") as f:
        for r in csv.DictReader(f):
            n = r["Kernel_Name"]
            if "gemm_" in n or "splitk_reduce" in n:
                rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), "splitk_reduce" in n))
    rows.sort()
    order = c5_api_order()
    spans: list[list[float]] = []      # per GEMM dispatch: [start, end]
    for start, end, is_reduce in rows:
        if not is_reduce:
            spans.append([start, end])
        elif spans:
            spans[-1][1] = end
    if len(spans) % len(order):
        raise SystemExit(f"{len(spans)} GEMM dispatches is not a whole number of config-5 steps")
    nsteps = len(spans) // len(order)
    tail = min(tail_steps, nsteps)

    def avg(i, first):
        v = [(spans[s * len(order) + i][1] - spans[s * len(order) + i][0]) / 1e3 for s in range(first, nsteps)]
        return sum(v) / len(v)

    ev = {}
    if bench_line:
        for g in bench_line.get("per_gemm", []):
            ev[(g["kind"], g["M"], g["N"], g["K"])] = g["us"]
    lines = [f"| GEMM | M x N x K | kernel avg us, all {nsteps} steps | kernel avg us, last {tail} steps | "
             "event avg us (bench) | TFLOP/s (all steps) |", "|---|---|---:|---:|---:|---:|"]
    tot = {"fwd": [0.0, 0.0, 0.0, 0.0], "bwd": [0.0, 0.0, 0.0, 0.0]}
    for i, (kind, M, N, K) in enumerate(order):
        a_all = avg(i, 0)
        a_tail = avg(i, nsteps - tail) if tail else float("nan")
        flop = 2.0 * M * N * K
        e = ev.get((kind, M, N, K))
        lines.append(f"| {kind} | {M} x {N} x {K} | {a_all:.1f} | {a_tail:.1f} | "
                     f"{'' if e is None else f'{e:.1f}'} | {flop / (a_all * 1e-6) / 1e12:.0f} |")
        t = tot["fwd" if kind == "fwd" else "bwd"]
        t[0] += a_all
        t[1] += a_tail
        t[2] += e if e is not None else float("nan")
        t[3] += flop
    for name, n in (("bwd", 7), ("fwd", 4)):
        t = tot[name]
        lines.append(f"| {name} sum ({n}) | | {t[0]:.1f} | {t[1]:.1f} | {t[2]:.1f} | "
                     f"{t[3] / (t[0] * 1e-6) / 1e12:.0f} |")
    return "\n".join(lines)


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


def _json_line(path: str | Path, key: str) -> dict:
    for ln in Path(path).read_text().splitlines():
        if ln.startswith("{") and f'"{key}"' in ln:
            return json.loads(ln)[key]
    raise SystemExit(f"no JSON line with {key!r} in {path}")


def ceiling_table(ceiling_log: str | Path) -> str:
    rows = _json_line(ceiling_log, "hbm_ceiling")["rows"]
    sizes = sorted({r["mb_per_array"] for r in rows})
    lines = ["| mix | loads/stores | " + " | ".join(f"{m} MB/array" for m in sizes) + " |",
             "|---|---|" + "---:|" * len(sizes)]
    for mix in dict.fromkeys(r["mix"] for r in rows):
        for nt in (False, True):
            cells = []
            for m in sizes:
                r = next((r for r in rows if r["mix"] == mix and r["nt"] == nt and r["mb_per_array"] == m), None)
                if r is None:
                    cells.append("")
                    continue
                cell = f"{r['gbps'] / 1e3:.2f} TB/s ({r['us']:.1f} us)"
                if "gbps_by_form" in r:
                    cell += " [" + " / ".join(f"{v / 1e3:.2f}" for v in r["gbps_by_form"].values()) + "]"
                cells.append(cell)
            lines.append(f"| {mix} | {'non-temporal' if nt else 'cached'} | " + " | ".join(cells) + " |")
    if rows and "gbps_by_form" in rows[0]:
        lines.append("")
        lines.append("Each cell: the best form's rate and time; in brackets the rate of every form, in the order "
                     + ", ".join(rows[0]["gbps_by_form"]) + ".")
    return "\n".join(lines)


def bw_table(stats_csv: str | Path, traffic_json: str | Path, events_log: str | Path,
             ceiling_log: str | Path) -> str:
    """One row per bandwidth kernel: event-timed and rocprof durations,
    algorithmic bytes and rate, the matching streaming ceiling, and the
    counters' HBM bytes."""
    stats = {_kname(r["Name"]): r for r in csv.DictReader(open(stats_csv, newline=""))}
    traffic_res = json.loads(Path(traffic_json).read_text())
    events = _json_line(events_log, "bw_events_us")
    ceil = _json_line(ceiling_log, "hbm_ceiling")["rows"]
    lines = ["| kernel | config shape | event us | rocprof avg us | algorithmic MB | GB/s (event) | of 8 TB/s | "
             "ceiling (mix, us) | of ceiling | FETCH+WRITE MB | traffic / algorithmic |",
             "|---|---|---:|---:|---:|---:|---:|---|---:|---:|---:|"]
    for label, (sub, algo) in BW_KERNELS.items():
        st = [r for n, r in stats.items() if sub in n]
        avg = sum(float(r["TotalDurationNs"]) for r in st) / max(1, sum(int(r["Calls"]) for r in st)) / 1e3
        ev = events.get(label)
        t = traffic_res.get(label, {})
        mix, nt, mb = BW_CEILING[label]
        c = next((r for r in ceil if r["mix"] == mix and r["nt"] == nt and r["mb_per_array"] == mb), None)
        us = ev if ev is not None else avg
        gbps = algo / us / 1e3
        cell_c = f"{mix}{' nt' if nt else ''} {mb} MB: {c['gbps'] / 1e3:.2f} TB/s" if c else "-"
        of_c = f"{gbps / c['gbps']:.0%}" if c else "-"
        lines.append(f"| `{sub}` | {label} | {ev if ev is not None else '-'} | {avg:.2f} | {algo / 1e6:.2f} | "
                     f"{gbps:.0f} | {gbps / 8000:.0%} | {cell_c} | {of_c} | "
                     f"{t.get('traffic_bytes', 0) / 1e6:.2f} | {t.get('traffic_over_algorithmic', '-')} |")
    return "\n".join(lines)


def _stats_rows(stats_csv: str | Path) -> dict[str, tuple[int, float]]:
    """kernel name -> (calls, average us) from a kernel_stats.csv."""
    out = {}
    with open(stats_csv, newline="") as f:
        for r in csv.DictReader(f):
            out[_kname(r["Name"])] = (int(r["Calls"]), float(r["AverageNs"]) / 1e3)
    return out


C4_CONV_FLOP = {"conv1_fwd": 226492416, "conv2_fwd": 1207959552, "conv1_dw_db": 226492416,
                "conv2_dw_db": 1207959552, "conv2_dx": 1207959552}


def conv_table(stats_csv, traffic_json, mfma_csv, insts_csv, events_log) -> str:
    """Config 4's five convolution kernels (bench.py --probe c4): trace
    duration, event time, FLOP rate against fp32 MFMA, calibrated HBM bytes
    against the algorithmic bytes, MFMA busy and instruction mix per MFMA."""
    stats = _stats_rows(stats_csv)
    tr = json.loads(Path(traffic_json).read_text())
    ev = _json_line(events_log, "conv_events_us")
    util = per_dispatch(mfma_csv, "MfmaUtil")
    ins = {c: per_dispatch(insts_csv, c) for c in ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_LDS")}
    avg = lambda v: sum(v) / len(v)
    lines = ["| launch | kernel | trace avg us | event us | GFLOP | TF/s | of fp32 MFMA peak | HBM bytes (x algorithmic) "
             "| GB/s | of 8 TB/s | MFMA busy | VALU / MFMA | LDS / MFMA |",
             "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for label, (sub, algo) in C4_KERNELS.items():
        name = next((n for n in stats if sub in n), None)
        if name is None:
            continue
        calls, us = stats[name]
        flop = C4_CONV_FLOP[label]
        t = tr.get(label, {})
        tb = t.get("traffic_bytes")
        u = avg(_match(util, sub))
        valu, mfma, lds = (avg(_match(ins[c], sub)) for c in ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_LDS"))
        short = name.split("(")[0].replace("void ", "")
        lines.append(f"| {label} | `{short}` | {us:.1f} | {ev.get(label, float('nan')):.1f} | {flop / 1e9:.3f} | "
                     f"{flop / us / 1e6:.1f} | {flop / us / 1e6 / 157.3:.1%} | "
                     f"{tb / 1e6:.1f} MB ({tb / algo:.2f}x) | {tb / us / 1e3:.0f} | {tb / us / 1e3 / 8000:.1%} | "
                     f"{u:.1f} % | {(valu - mfma) / max(mfma, 1):.1f} | {lds / max(mfma, 1):.2f} |")
    ps = next((n for n in stats if "conv_partial_sum_kernel" in n), None)
    if ps:
        lines.append(f"| weight-gradient partial sums | `conv_partial_sum_kernel` | {stats[ps][1]:.1f} | | | | | | | | | | |")
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
    s.add_argument("--c5-gemms", help="the run's kernel_trace.csv: add the per-GEMM table of the config-5 step")
    s.add_argument("--bench-log", help="file holding the bench's JSON line (event timings for that table)")
    s.add_argument("--tail-steps", type=int, default=7, help="steps of the bench's event-timed pass")
    s.add_argument("--events-log", help="log of an unprofiled run of the same command: its JSON line is appended")
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--cal-n", type=int, default=1 << 26)
    t.add_argument("--config", choices=["c2", "c4", "c5", "bw"], default="c2")
    t.add_argument("--json", required=True)
    t.add_argument("--cmd", required=True, nargs="+", help="the two rocprofv3 commands")
    b = sub.add_parser("bw-summary", help="markdown table of the bandwidth kernels (bench.py --probe bw)")
    b.add_argument("--stats", required=True, help="kernel_stats.csv of a --kernel-trace --stats run of --probe bw")
    b.add_argument("--traffic", required=True, help="the traffic JSON (--config bw)")
    b.add_argument("--events", required=True, help="log of an unprofiled --probe bw run")
    b.add_argument("--ceiling", required=True, help="log of bench.py --hbm-ceiling")
    b.add_argument("--cmd", required=True, nargs="+", help="the commands that produced the inputs")
    b.add_argument("--out", required=True)
    c = sub.add_parser("ceiling-summary", help="markdown table of bench.py --hbm-ceiling")
    c.add_argument("--ceiling", required=True)
    c.add_argument("--stats", help="kernel_stats.csv of a --kernel-trace run of the same command")
    c.add_argument("--cmd", required=True, nargs="+")
    c.add_argument("--out", required=True)
    cs = sub.add_parser("conv-summary", help="config 4's convolution kernels (bench.py --probe c4)")
    cs.add_argument("--stats", required=True, help="kernel_stats.csv of a --kernel-trace --stats run of --probe c4")
    cs.add_argument("--traffic", required=True, help="the traffic JSON (--config c4)")
    cs.add_argument("--mfma", required=True, help="counter CSV of a --pmc MfmaUtil run")
    cs.add_argument("--insts", required=True, help="counter CSV of a --pmc SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS run")
    cs.add_argument("--events", required=True, help="log of an unprofiled --probe c4 run")
    cs.add_argument("--cmd", required=True, nargs="+")
    cs.add_argument("--out", required=True)
    m = sub.add_parser("mfma-summary", help="MFMA busy per config-5 GEMM shape (bench.py --probe c5)")
    m.add_argument("--run", nargs=3, action="append", required=True, metavar=("LABEL", "PMC_CSV", "TRACE_CSV"))
    m.add_argument("--cmd", required=True, nargs="+")
    m.add_argument("--out", required=True)
    a = ap.parse_args(argv)
    if a.action == "conv-summary":
        cmds = "\n".join(a.cmd)
        text = (f"# Config 4 (CNN, batch 128): the five convolution launches\n\nCommands (repo root):\n\n```\n{cmds}\n"
                f"```\n\n{conv_table(a.stats, a.traffic, a.mfma, a.insts, a.events)}\n\nFLOP and algorithmic bytes per "
                f"launch as in bench.py (each operand read or written once; conv1 is bound by HBM, conv2 by fp32 "
                f"MFMA).  HBM bytes: FETCH_SIZE and WRITE_SIZE scaled by what they read for the probe's tf_add launches "
                f"of known traffic.  "
                f"VALU / MFMA: non-MFMA vector instructions per MFMA instruction (SQ_INSTS_VALU counts both).\n"
                f"\nKernel trace of the same command:\n\n{stats_table(a.stats)}\n")
        Path(a.out).write_text(text)
        sys.stdout.write(text)
        return 0
    if a.action == "mfma-summary":
        cmds = "\n".join(a.cmd)
        text = (f"# MFMA busy per config-5 GEMM shape (bf16 in, fp32 accumulate; 3 steps of GEMMs, averaged)\n\n"
                f"Commands (repo root):\n\n```\n{cmds}\n```\n\n{mfma_table(a.run)}\n")
        Path(a.out).write_text(text)
        sys.stdout.write(text)
        return 0
    if a.action == "bw-summary":
        cmds = "\n".join(a.cmd)
        text = (f"# Bandwidth kernels of the path at their configurations' shapes\n\nCommands (repo root):\n\n"
                f"```\n{cmds}\n```\n\n{bw_table(a.stats, a.traffic, a.events, a.ceiling)}\n")
        Path(a.out).write_text(text)
        sys.stdout.write(text)
        return 0
    if a.action == "ceiling-summary":
        cmds = "\n".join(a.cmd)
        text = (f"# HBM streaming ceilings (one MI355X)\n\nCommands (repo root):\n\n```\n{cmds}\n```\n\n"
                f"Event-timed, buffers rotated past the 256 MB last-level cache:\n\n{ceiling_table(a.ceiling)}\n")
        if a.stats:
            text += f"\nKernel trace of the same command:\n\n{stats_table(a.stats)}\n"
        Path(a.out).write_text(text)
        sys.stdout.write(text)
        return 0
    if a.action == "stats":
        text = f"# {a.title}\n\nCommand (repo root):\n\n```\n{a.cmd}\n```\n\n{stats_table(a.csv)}\n"
        if a.trace and a.phases:
            phases = [(p.split("=")[0], int(p.split("=")[1])) for p in a.phases.split(",")]
            text += ("\nPer phase (each kernel's dispatches in launch order, split into the bench's phases):\n\n"
                     f"{phase_table(a.trace, phases, a.match)}\n")
        if a.c5_gemms:
            line = None
            if a.bench_log:
                for ln in Path(a.bench_log).read_text().splitlines():
                    if ln.startswith("{") and '"metric"' in ln:
                        line = json.loads(ln)
            text += ("\nConfig-5 GEMMs (dispatches of the C++ API step in launch order; split-K reductions "
                     "counted with their GEMM):\n\n" + c5_gemm_table(a.c5_gemms, line, a.tail_steps) + "\n")
        if a.events_log:
            ev = [ln for ln in Path(a.events_log).read_text().splitlines() if ln.startswith("{")]
            if ev:
                body = json.dumps(json.loads(ev[-1]), indent=1)
                text += f"\nEvent timings of an unprofiled run of the same command:\n\n```json\n{body}\n```\n"
        if a.out:
            Path(a.out).write_text(text)
        else:
            sys.stdout.write(text)
    else:
        if a.config == "c5":
            res = traffic_c5(a.fetch, a.write, a.cal_n)
        else:
            res = traffic(a.fetch, a.write, a.cal_n,
                          {"bw": BW_KERNELS, "c4": C4_KERNELS}.get(a.config))
        res["commands"] = a.cmd
        Path(a.json).write_text(json.dumps(res, indent=2) + "\n")
        print(json.dumps(res, indent=2))
    return 0


if __name__ == "__main__":
    sys.exit(main())
