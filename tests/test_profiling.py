"""Host logic of tensors_amd.profiling (the summaries under profiles/): the
traffic calibration arithmetic, the stats table and the per-phase split, on
synthetic rocprofv3 CSV files."""
from __future__ import annotations

import csv
import json

from tensors_amd import profiling


def _write_counters(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for r in rows:
            w.writerow(r)


def test_traffic_calibration(tmp_path):
    # The copy kernel reads 2 x 4 x N and writes 4 x N bytes; the counter
    # reports half the fetch bytes (scale 2) and the exact write bytes.  A GEMM
    # dispatch whose raw FETCH_SIZE is 50,000 KiB must come out as 100,000 KiB.
    n = 1 << 20
    cal_f_kib = 2 * 4 * n / 1024 / 2
    cal_w_kib = 4 * n / 1024
    fetch, write = [], []
    d = 0
    for name, f_kib, w_kib in [("binary_kernel<float, AddOp>", cal_f_kib, cal_w_kib)] + \
            [(k, 50000.0, 16384.0) for k, _ in profiling.C2_KERNELS.values()]:
        d += 1
        # two counter instances per dispatch (summed by per_dispatch)
        for part in (0.25, 0.75):
            fetch.append({"Dispatch_Id": d, "Kernel_Name": name, "Counter_Name": "FETCH_SIZE",
                          "Counter_Value": f_kib * part})
            write.append({"Dispatch_Id": d, "Kernel_Name": name, "Counter_Name": "WRITE_SIZE",
                          "Counter_Value": w_kib * part})
    fp, wp = tmp_path / "f.csv", tmp_path / "w.csv"
    _write_counters(fp, fetch)
    _write_counters(wp, write)
    res = profiling.traffic(fp, wp, n)
    assert abs(res["calibration"]["fetch_scale"] - 2.0) < 1e-6
    assert abs(res["calibration"]["write_scale"] - 1.0) < 1e-6
    dx = res["gemm_f32_bwd_dx_c2"]
    assert dx["fetch_bytes"] == 100000 * 1024 and dx["write_bytes"] == 16384 * 1024
    assert dx["traffic_bytes"] == dx["fetch_bytes"] + dx["write_bytes"]
    assert res["gemm_f32_bwd_c2"] == dx["traffic_bytes"]
    json.dumps(res)


def test_stats_and_phase_tables(tmp_path):
    stats = tmp_path / "s.csv"
    with open(stats, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Name", "Calls", "TotalDurationNs", "AverageNs", "MinNs", "MaxNs",
                                          "Percentage"])
        w.writeheader()
        w.writerow({"Name": "void (anonymous namespace)::k_a<1>(int)", "Calls": 6, "TotalDurationNs": 6000,
                    "AverageNs": 1000, "MinNs": 500, "MaxNs": 2000, "Percentage": 75.0})
        w.writerow({"Name": "k_b(float|int)", "Calls": 2, "TotalDurationNs": 2000, "AverageNs": 1000,
                    "MinNs": 1000, "MaxNs": 1000, "Percentage": 25.0})
    table = profiling.stats_table(stats)
    assert table.splitlines()[2].startswith("| `void k_a<1>(int)` | 6 | 0.006 | 1.00 |")
    assert "k_b(float\\|int)" in table          # pipes escaped for markdown
    trace = tmp_path / "t.csv"
    with open(trace, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        # k_a: durations 4, 4 (warmup), 2, 2 (timed), 1, 1 (events) microseconds, written out of order
        t = 0
        rows = []
        for dur in (4000, 4000, 2000, 2000, 1000, 1000):
            rows.append({"Kernel_Name": "k_a<1>", "Start_Timestamp": t, "End_Timestamp": t + dur})
            t += 10000
        for r in reversed(rows):
            w.writerow(r)
    out = profiling.phase_table(trace, [("warmup", 2), ("timed", 2), ("events", 2)], ["k_a"])
    assert out.splitlines()[-1] == "| `k_a<1>` | 4.00 | 2.00 | 1.00 |"


def test_traffic_c5_attributes_split_reductions_to_their_gemm(tmp_path):
    """Two probe steps: each GEMM dispatch reads 1000 KiB and writes 100 KiB
    (raw); the split-K reductions after the L4 forward and L4 dW add 10 KiB
    each to those GEMMs' kinds.  The copy kernel calibrates fetch x2, write x1."""
    n = 1 << 20
    order = profiling.c5_gemm_order()
    rows_f, rows_w = [], []
    d = 0

    def add(name, f, w):
        nonlocal d
        d += 1
        rows_f.append({"Dispatch_Id": d, "Kernel_Name": name, "Counter_Name": "FETCH_SIZE", "Counter_Value": f})
        rows_w.append({"Dispatch_Id": d, "Kernel_Name": name, "Counter_Name": "WRITE_SIZE", "Counter_Value": w})

    for _ in range(2):
        for i, (kind, M, N, K, ob) in enumerate(order):
            add("gemm_bf16_dl8_kernel<...>", 1000.0, 100.0)
            if i in (3, 4):           # L4 forward, L4 dW
                add("splitk_reduce_kernel(GemmParams, int)", 10.0, 10.0)
    add("binary_kernel<float, AddOp>", 2 * 4 * n / 1024 / 2, 4 * n / 1024)
    fp, wp = tmp_path / "f.csv", tmp_path / "w.csv"
    _write_counters(fp, rows_f)
    _write_counters(wp, rows_w)
    res = profiling.traffic_c5(fp, wp, n)
    assert res["steps"] == 2
    fwd, dx, dw = res["gemm_bf16_fwd_c5"], res["gemm_bf16_dX_c5"], res["gemm_bf16_dW_c5"]
    assert (fwd["launches_per_step"], dx["launches_per_step"], dw["launches_per_step"]) == (4, 3, 4)
    assert fwd["fetch_bytes_per_step"] == (4 * 1000 + 10) * 2 * 1024
    assert dw["write_bytes_per_step"] == (4 * 100 + 10) * 1024
    assert dx["traffic_bytes_per_step"] == 3 * (2000 + 100) * 1024
    assert res["gemm_bf16_bwd_c5"] == round((dx["traffic_bytes_per_step"] + dw["traffic_bytes_per_step"]) / 7)
    # algorithmic bytes of the L2 dW (8192 x 8192 x 4096, bf16 in, fp32 out) are part of dW's total
    assert dw["algorithmic_bytes_per_step"] >= 2 * (8192 * 4096 * 2) + 4 * 8192 * 8192


def test_bandwidth_traffic_matches_qualified_names(tmp_path):
    # rocprofv3's counter CSV names kernels with their anonymous-namespace
    # qualifiers; the label table's substrings are written without them.
    n = 1 << 20
    fetch, write = [], []
    kernels = [("void (anonymous namespace)::binary_kernel<float, (anonymous namespace)::AddOp>(float const*)",
                2 * 4 * n / 1024 / 2, 4 * n / 1024)]
    for label, (sub, algo) in profiling.BW_KERNELS.items():
        # every kernel's raw reading is exactly its algorithmic bytes once the
        # fetch scale of 2 is applied (reads = all but the 1/4 that is written)
        kernels.append((f"void (anonymous namespace)::{sub}(float const*)", algo * 0.75 / 1024 / 2,
                        algo * 0.25 / 1024))
    for d, (name, f_kib, w_kib) in enumerate(kernels, 1):
        fetch.append({"Dispatch_Id": d, "Kernel_Name": name, "Counter_Name": "FETCH_SIZE", "Counter_Value": f_kib})
        write.append({"Dispatch_Id": d, "Kernel_Name": name, "Counter_Name": "WRITE_SIZE", "Counter_Value": w_kib})
    fp, wp = tmp_path / "f.csv", tmp_path / "w.csv"
    _write_counters(fp, fetch)
    _write_counters(wp, write)
    res = profiling.traffic(fp, wp, n, profiling.BW_KERNELS)
    for label, (_, algo) in profiling.BW_KERNELS.items():
        assert abs(res[label]["traffic_over_algorithmic"] - 1.0) < 1e-3, label
    assert "gemm_f32_bwd_c2" not in res
    # the LayerNorm backward op is one launch; its algorithmic bytes are the
    # op's operands and results
    op = res["layernorm_bwd_op_c3c"]
    assert op["algorithmic_bytes"] == profiling.LN_OP_BYTES == 12603392


def test_ceiling_and_bandwidth_tables(tmp_path):
    ceil = {"hbm_ceiling": {"rows": [
        {"mix": m, "nt": nt, "mb_per_array": mb, "us": 10.0, "bytes": 40_000_000, "gbps": 4000.0}
        for m in ("copy (1R+1W)", "2R+1W", "3R+2W (SGD mix)", "read only (1R)")
        for nt in (False, True) for mb in (4, 16, 512)]}}
    clog = tmp_path / "hbm.log"
    clog.write_text("hbm ceiling: progress line\n" + json.dumps(ceil) + "\n")
    table = profiling.ceiling_table(clog)
    assert table.count("\n") == 1 + 8 and "4.00 TB/s (10.0 us)" in table
    events = {label: 20.0 for label in profiling.BW_KERNELS}
    events["layernorm_bwd_op_c3c"] = 10.0
    elog = tmp_path / "ev.log"
    elog.write_text(json.dumps({"bw_events_us": events}) + "\n")
    stats = tmp_path / "s.csv"
    with open(stats, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Name", "Calls", "TotalDurationNs"])
        w.writeheader()
        for label, (sub, _) in profiling.BW_KERNELS.items():
            w.writerow({"Name": f"void (anonymous namespace)::{sub}(int)", "Calls": 4, "TotalDurationNs": 80000})
    tj = tmp_path / "t.json"
    tj.write_text(json.dumps({"layernorm_bwd_op_c3c": {"traffic_bytes": 17_000_000, "algorithmic_bytes": 12603392,
                                                        "traffic_over_algorithmic": 1.349}}))
    bw = profiling.bw_table(stats, tj, elog, clog)
    lines = bw.splitlines()
    assert len(lines) == 2 + len(profiling.BW_KERNELS)
    relu = next(ln for ln in lines if "relu_bwd_c3b" in ln)
    # 50,331,648 B in 20 us = 2517 GB/s; 20 us rocprof average
    assert "| 20.0 | 20.00 | 50.33 | 2517 |" in relu
    assert "layernorm_bwd_op_c3c | 10.0 |" in next(ln for ln in lines if "layernorm" in ln)


def test_mfma_table_groups_dispatches_by_c5_position(tmp_path):
    order = profiling.c5_gemm_order()
    steps = 2
    pmc, trace = [], []
    t = 0
    d = 0
    for s in range(steps):
        for pos, (kind, M, N, K, _) in enumerate(order):
            d += 1
            name = f"void (anonymous namespace)::gemm_bf16_pp_kernel<{kind}>(GemmParams)"
            pmc.append({"Dispatch_Id": d, "Kernel_Name": name, "Counter_Name": "MfmaUtil",
                        "Counter_Value": 50.0 + pos + 10 * s})
            dur = 1000 * (pos + 1)              # ns
            trace.append({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + dur})
            t += dur + 100
            if kind != "fwd":                   # a split-K reduction between GEMMs is skipped
                d += 1
                pmc.append({"Dispatch_Id": d, "Kernel_Name": "splitk_reduce_kernel(GemmParams, int)",
                            "Counter_Name": "MfmaUtil", "Counter_Value": 0.0})
                trace.append({"Kernel_Name": "splitk_reduce_kernel(GemmParams, int)", "Start_Timestamp": t,
                              "End_Timestamp": t + 50})
                t += 150
    pp, tp = tmp_path / "p.csv", tmp_path / "t.csv"
    _write_counters(pp, pmc)
    with open(tp, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        trace.reverse()                         # rows out of time order are sorted
        for r in trace:
            w.writerow(r)
    table = profiling.mfma_table([("pp", str(pp), str(tp))])
    lines = table.splitlines()
    assert len(lines) == 2 + len(order) + 1
    first = lines[2]
    # position 0: MfmaUtil 50 and 60 over the two steps -> 55 %, 1 us each
    assert "| 55.0 % | 1.0 |" in first
    M, N, K = order[0][1:4]
    assert f"{M} x {N} x {K}" in first
