#!/usr/bin/env python3
"""Benchmark of the training hot path on one MI355X.

Headline workload, config 5 (the largest configuration, which fits one GPU):
the wide MLP 4096-8192-8192-4096-1000 at batch 4096, bf16 weights and
activations with fp32 accumulation and fp32 master weights, ReLU,
CrossEntropy over 1000 labels, SGD with momentum.  One step is the whole
fwd + bwd + SGD step through the C++20 tensorforge API (nn::Linear,
nn::CrossEntropyLoss, Tensor::backward, optim::SGD) on device-resident
inputs, host launch work included.  Prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

`value` is the wall time of the K timed steps (the device drained before and
after) divided by K.  The roofline entry is for the backward GEMMs (the
dominant kernels): a second pass of the same step with the library's launch
timing on (tf_hip_timing_*: a HIP event before and after every GEMM on the
stream it runs on) gives each GEMM's duration; `achieved` is the backward
GEMMs' 2*M*N*K FLOP per step over their summed duration, against the
2.5 PFLOP/s dense bf16 MFMA peak.  ``traffic`` is read from the committed
rocprofv3 counter summary when present.  The other configurations (C2's
isolated fp32 Linear step with its own fp32 roofline, the C3 bandwidth
kernels, the C1 and C4 training steps) are reported under `other_configs`.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_FP32_TFLOPS = 157.3
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBPS = 8000.0
C5_DIMS = [4096, 8192, 8192, 4096, 1000]
C5_BATCH = 4096
N2 = 2048
GEMM_FLOP = 2 * N2 * N2 * N2          # 17,179,869,184


def _median(x):
    return float(np.median(np.asarray(x, dtype=np.float64)))


def bench_c2(steps: int, warmup: int):
    import tensors_amd as ta
    from tensors_amd import ops, synth

    ctx = ta.Context(0)
    X = ctx.array(synth.normal(synth.seed(2, 0), (N2, N2)))
    W = ctx.array(synth.normal(synth.seed(2, 1), (N2, N2)))
    dY = ctx.array(synth.normal(synth.seed(2, 2), (N2, N2)))
    b = ctx.array(synth.normal(synth.seed(2, 3), (N2,)))
    Y, dX, dW, db = ctx.empty((N2, N2)), ctx.empty((N2, N2)), ctx.empty((N2, N2)), ctx.empty((N2,))
    vW, vb = ctx.zeros((N2, N2)), ctx.zeros((N2,))
    lr, mu = 1e-3, 0.9

    n_ev = 6
    events = [[ctx.event() for _ in range(n_ev)] for _ in range(max(steps, 1))]

    def step(ev=None):
        rec = (lambda i: ev[i].record()) if ev is not None else (lambda i: None)
        rec(0)
        ops.gemm(X, W, Y, trans_b=True, bias=b)
        rec(1)
        ops.gemm(dY, W, dX)
        rec(2)
        ops.gemm(dY, X, dW, trans_a=True)
        rec(3)
        ops.colsum(dY, db)
        rec(4)
        ops.sgd_momentum_multi([W, b], [dW, db], [vW, vb], lr, mu)
        rec(5)

    for _ in range(warmup):
        step()
    # Timed region: exactly `steps` steps with nothing else on the stream.
    ctx.sync()
    t0 = time.perf_counter()
    for s in range(steps):
        step()
    ctx.sync()
    wall_ms = (time.perf_counter() - t0) * 1e3
    # Per-kernel breakdown (and the roofline figure) from a second, untimed
    # pass with an event between consecutive kernels.
    for s in range(steps):
        step(events[s])
    ctx.sync()

    per = {"fwd_gemm": [], "bwd_gemm_dx": [], "bwd_gemm_dw": [], "colsum": [], "sgd": [], "step_dev": []}
    for s in range(steps):
        ev = events[s]
        per["fwd_gemm"].append(ev[0].elapsed_ms(ev[1]))
        per["bwd_gemm_dx"].append(ev[1].elapsed_ms(ev[2]))
        per["bwd_gemm_dw"].append(ev[2].elapsed_ms(ev[3]))
        per["colsum"].append(ev[3].elapsed_ms(ev[4]))
        per["sgd"].append(ev[4].elapsed_ms(ev[5]))
        per["step_dev"].append(ev[0].elapsed_ms(ev[5]))
    mean = {k: float(np.mean(v)) for k, v in per.items()}
    ctx.close()
    return wall_ms / steps, mean, per


def _rotating_bench(ctx, n_sets, launch, reps=60):
    """Average device time of `launch(i)` cycling over n_sets buffer sets (the
    sets together exceed the 256 MB Infinity Cache, so every launch streams
    from HBM).  Event pair around `reps` back-to-back launches."""
    for i in range(n_sets):
        launch(i)
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    e0.record()
    for r in range(reps):
        launch(r % n_sets)
    e1.record()
    return e0.elapsed_ms(e1) / reps


def _bw_entry(label: str, ms: float) -> dict:
    from tensors_amd.profiling import BW_KERNELS
    algo = BW_KERNELS[label][1]
    return {"us": round(ms * 1e3, 2), "bytes": algo, "gbps": round(algo / ms / 1e6, 1),
            "frac_hbm": round(algo / ms / 1e6 / PEAK_HBM_GBPS, 3)}


def bench_c3(more: bool = True, reps: int = 60):
    """Config 3 bandwidth kernels: fused LogSoftmax+NLL backward [4096 x 1024],
    ReLU backward [4096 x 1024], LayerNorm backward [1024 x 1024]; with
    `more`, the other backward kernels of the path at C3b's shape."""
    import tensors_amd as ta
    from tensors_amd import ops, synth
    from tensors_amd.profiling import LN_OP_BYTES

    ctx = ta.Context(0)
    out = {}
    R, Cc = 4096, 1024
    sets = 10
    logits = [ctx.array(synth.normal(synth.seed(3, 0) + i, (R, Cc), std=3.0)) for i in range(sets)]
    tg = ctx.array(synth.uniform_int(synth.seed(3, 1), (R,), Cc))
    lse = [ctx.empty((R,)) for _ in range(sets)]
    loss = ctx.empty((1,))
    for i in range(sets):
        ops.ce_fwd(logits[i], tg, loss, lse[i])
    dl = [ctx.empty((R, Cc)) for _ in range(sets)]
    ms = _rotating_bench(ctx, sets, lambda i: ops.ce_bwd(logits[i], tg, dl[i], lse=lse[i]), reps)
    out["c3a_logsoftmax_nll_bwd"] = _bw_entry("ce_bwd_c3a", ms)
    ms = _rotating_bench(ctx, sets, lambda i: ops.ce_fwd_bwd(logits[i], tg, loss, dl[i]), reps)
    out["c3a_ce_fused_fwd_bwd"] = _bw_entry("ce_fused_fwd_bwd_c3a", ms)
    del logits, dl, lse
    sets = 6
    xs = [ctx.array(synth.normal(synth.seed(3, 2) + i, (R, Cc))) for i in range(sets)]
    dys = [ctx.array(synth.normal(synth.seed(3, 3) + i, (R, Cc))) for i in range(sets)]
    dxs = [ctx.empty((R, Cc)) for _ in range(sets)]
    ms = _rotating_bench(ctx, sets, lambda i: ops.relu_bwd(dys[i], xs[i], dxs[i]), reps)
    out["c3b_relu_bwd"] = _bw_entry("relu_bwd_c3b", ms)
    # The other backward kernels of the path at the same shape (two reads and
    # one write of 16 MB each); the values do not affect their speed.
    algo = R * Cc * 4 * 3
    for name, fn in (("sigmoid_bwd", lambda i: ops.sigmoid_bwd(dys[i], xs[i], dxs[i])),
                     ("tanh_bwd", lambda i: ops.tanh_bwd(dys[i], xs[i], dxs[i])),
                     ("softmax_bwd", lambda i: ops.softmax_bwd(xs[i], dys[i], dxs[i])),
                     ("mul", lambda i: ops.mul(dys[i], xs[i], dxs[i])),
                     ("add", lambda i: ops.add(dys[i], xs[i], dxs[i]))) if more else ():
        ms = _rotating_bench(ctx, sets, fn, reps)
        out[f"c3_more_{name}"] = {"us": round(ms * 1e3, 2), "bytes": algo, "gbps": round(algo / ms / 1e6, 1),
                                  "frac_hbm": round(algo / ms / 1e6 / PEAK_HBM_GBPS, 3)}
    del xs, dys, dxs
    R = Cc = 1024
    sets = 24
    g = ctx.array(np.ones(Cc, np.float32))
    xs = [ctx.array(synth.normal(synth.seed(3, 4) + i, (R, Cc))) for i in range(sets)]
    dys = [ctx.array(synth.normal(synth.seed(3, 5) + i, (R, Cc))) for i in range(sets)]
    means = [ctx.empty((R,)) for _ in range(sets)]
    rstds = [ctx.empty((R,)) for _ in range(sets)]
    ys = ctx.empty((R, Cc))
    beta = ctx.zeros((Cc,))
    for i in range(sets):
        ops.layernorm_fwd(xs[i], g, beta, ys, means[i], rstds[i])
    dxs = [ctx.empty((R, Cc)) for _ in range(sets)]
    dg, db = ctx.empty((Cc,)), ctx.empty((Cc,))
    ms = _rotating_bench(ctx, sets, lambda i: ops.layernorm_bwd(dys[i], xs[i], g, means[i], rstds[i], dxs[i], dg, db),
                         reps)
    out["c3c_layernorm_bwd"] = {"us": round(ms * 1e3, 2), "bytes": LN_OP_BYTES,
                                "gbps": round(LN_OP_BYTES / ms / 1e6, 1),
                                "frac_hbm": round(LN_OP_BYTES / ms / 1e6 / PEAK_HBM_GBPS, 3)}
    ctx.close()
    return out


def bench_bandwidth_rotated(reps: int = 60):
    """The other bandwidth kernels of the path at their configurations'
    shapes, each launch on a buffer set not touched since the cache last held
    it (sets together > 256 MB): C2's bias column sum and SGD-momentum step
    (W and b in one launch), C5's SGD step over its 138 M parameters with the
    bf16 copies, C4 conv2's im2col and col2im (N 128, C 32, 32 x 32, k 3,
    stride 2, pad 1), and C5's fused ReLU backward + bias gradient."""
    import tensors_amd as ta
    from tensors_amd import ops, synth
    from tensors_amd.profiling import CONV2

    ctx = ta.Context(0)
    out = {}
    sets = 20                                         # 20 x 16 MB
    dys = [ctx.array(synth.normal(synth.seed(6, 0) + i, (N2, N2))) for i in range(sets)]
    db = ctx.empty((N2,))
    out["colsum_c2"] = _bw_entry("colsum_c2", _rotating_bench(ctx, sets, lambda i: ops.colsum(dys[i], db), reps))
    del dys
    sets = 6                                          # 6 x 3 x 16 MB
    Ws = [ctx.array(synth.normal(synth.seed(6, 1) + i, (N2, N2))) for i in range(sets)]
    bs = [ctx.zeros((N2,)) for _ in range(sets)]
    dWs = [ctx.array(synth.normal(synth.seed(6, 2) + i, (N2, N2), std=1e-3)) for i in range(sets)]
    dbs = [ctx.zeros((N2,)) for _ in range(sets)]
    vWs, vbs = [ctx.zeros((N2, N2)) for _ in range(sets)], [ctx.zeros((N2,)) for _ in range(sets)]
    out["sgd_c2"] = _bw_entry("sgd_c2", _rotating_bench(
        ctx, sets, lambda i: ops.sgd_momentum_multi([Ws[i], bs[i]], [dWs[i], dbs[i]], [vWs[i], vbs[i]], 1e-3, 0.9),
        reps))
    del Ws, bs, dWs, dbs, vWs, vbs
    # C5: one set of 1.9 GB, far past the cache.
    shapes = [s for i in range(4) for s in ((C5_DIMS[i + 1], C5_DIMS[i]), (C5_DIMS[i + 1],))]
    ps = [ctx.zeros(s) for s in shapes]
    gs = [ctx.zeros(s) for s in shapes]
    vs = [ctx.zeros(s) for s in shapes]
    sh = [ctx.empty(s, ta.BF16) for s in shapes]
    out["sgd_c5"] = _bw_entry("sgd_c5", _rotating_bench(
        ctx, 1, lambda i: ops.sgd_momentum_multi(ps, gs, vs, 1e-2, 0.9, sh), max(3, reps // 6)))
    del ps, gs, vs, sh
    N, C, H, W, k, oh = CONV2
    sets = 6                                          # 6 x (16.8 + 37.7) MB
    xs = [ctx.array(synth.normal(synth.seed(6, 3) + i, (N, C, H, W))) for i in range(sets)]
    cols = [ctx.empty((N, C * k * k, oh * oh)) for _ in range(sets)]
    out["im2col_conv2_c4"] = _bw_entry("im2col_conv2_c4", _rotating_bench(
        ctx, sets, lambda i: ops.im2col(xs[i], cols[i], k, k, (2, 2), (1, 1)), reps))
    out["col2im_conv2_c4"] = _bw_entry("col2im_conv2_c4", _rotating_bench(
        ctx, sets, lambda i: ops.col2im(cols[i], xs[i], k, k, (2, 2), (1, 1)), reps))
    del xs, cols
    # C5 layer 1's ReLU backward + the next Linear's bias gradient, bf16
    # [4096 x 8192]; 4 x 3 x 64 MB.
    R5, C5w = C5_BATCH, C5_DIMS[1]
    sets = 4
    gs = [ctx.array(ta.f32_to_bf16_bits(synth.normal(synth.seed(6, 4) + i, (R5, C5w))), ta.BF16) for i in range(sets)]
    xs = [ctx.array(ta.f32_to_bf16_bits(synth.normal(synth.seed(6, 5) + i, (R5, C5w))), ta.BF16) for i in range(sets)]
    dzs = [ctx.empty((R5, C5w), ta.BF16) for _ in range(sets)]
    db5 = ctx.empty((C5w,))
    out["relu_bwd_colsum_c5"] = _bw_entry("relu_bwd_colsum_c5", _rotating_bench(
        ctx, sets, lambda i: ops.relu_bwd_colsum(gs[i], xs[i], dzs[i], db5), reps))
    ctx.close()
    return out


HBM_PROBE_MB = (4, 16, 64, 256, 512)
HBM_PROBE_KINDS = ("copy (1R+1W)", "2R+1W", "3R+2W (SGD mix)", "read only (1R)")


HBM_PROBE_FORMS = ("elementwise loop", "persistent, 1 block per CU, 16 loads in flight",
                   "persistent, 2 blocks per CU, 8 loads in flight")


def hbm_ceiling() -> dict:
    """Streaming rate of plain copy / 2R+1W / 3R+2W / read-only kernels over
    arrays of 4 to 512 MB, buffers rotated past the 256 MB cache, cached and
    non-temporal, each in three loop forms (libtf_hbm_probe.so): the
    elementwise kernels' own loop and grid, and two persistent forms that
    share nothing with it (one or two blocks per CU, each walking one
    contiguous range with 16 or 8 16-byte loads per input in flight per
    thread).  The ceiling of a row is the best of its forms."""
    import ctypes as C
    lib = C.CDLL(str(ROOT / "tensors_amd" / "lib" / "libtf_hbm_probe.so"))
    lib.tf_hbm_probe_form.argtypes = [C.c_int, C.c_int, C.c_int64, C.c_int, C.c_int, C.POINTER(C.c_double)]
    lib.tf_hbm_probe_form.restype = C.c_int
    lib.tf_hbm_probe_bytes.argtypes = [C.c_int, C.c_int64]
    lib.tf_hbm_probe_bytes.restype = C.c_int64
    rows = []
    for kind, kname in enumerate(HBM_PROBE_KINDS):
        for nt in (0, 1):
            for mb in HBM_PROBE_MB:
                moved = lib.tf_hbm_probe_bytes(kind, mb << 20)
                per_form = {}
                for form, fname in enumerate(HBM_PROBE_FORMS):
                    us = C.c_double()
                    rc = lib.tf_hbm_probe_form(kind, nt, mb << 20, max(10, 2048 // mb), form, C.byref(us))
                    if rc != 0:
                        raise RuntimeError(f"tf_hbm_probe_form({kind}, {nt}, {mb} MB, {form}) failed: {rc}")
                    per_form[fname] = round(moved / us.value / 1e3, 1)
                best = max(per_form, key=per_form.get)
                rows.append({"mix": kname, "nt": bool(nt), "mb_per_array": mb, "bytes": moved,
                             "gbps": per_form[best], "best_form": best, "gbps_by_form": per_form,
                             "us": round(moved / per_form[best] / 1e3, 2)})
                print(f"hbm ceiling: {kname} nt={nt} {mb} MB: " +
                      ", ".join(f"{k} {v:.0f} GB/s" for k, v in per_form.items()), flush=True)
    return {"rows": rows}


def bench_c1():
    """Config 1: the MLP step through the C++ API (host launch work
    included), eagerly and as a replayed HIP graph of the step."""
    from tensors_amd import api, synth
    xs = synth.mnist_like(synth.seed(1, 0), (100, 64, 784))
    ys = synth.uniform_int(synth.seed(1, 1), (100, 64), 10)
    _, _, ms = api.mlp_train([784, 256, 128, 10], xs, ys, steps=100, warmup=10, lr=0.1, mu=0.9, on_gpu=True,
                             reference_compat=True)
    # The same loop with its step captured once in a HIP graph and replayed
    # (batch selection and loss recording on the device).
    _, _, ms_g = api.mlp_train([784, 256, 128, 10], xs, ys, steps=100, warmup=10, lr=0.1, mu=0.9, on_gpu=True,
                               reference_compat=True, graph=1)
    return {"workload": "C1 MLP 784-256-128-10 fp32, batch 64, Linear+ReLU, CE chain, SGD momentum (lr 0.1, "
                        "mu 0.9), the reference's bias-free Linear; whole step through the C++ API",
            "ms_per_step": round(ms, 4), "ms_per_step_graph": round(ms_g, 4),
            "flop_per_step": C1_FLOP, "bound": "launch latency (11 dependent kernels of 4-9 us)"}


# Config 4: the convolutions at batch 128 (N, Cin, H, Cout, stride); FLOP
# and algorithmic bytes (each operand once) per launch.
C4_B = 128
C4_CONV1 = dict(cin=3, h=32, cout=32, stride=1, oh=32)
C4_CONV2 = dict(cin=32, h=32, cout=64, stride=2, oh=16)


def _conv_flop(c):
    return 2 * C4_B * c["cout"] * c["oh"] ** 2 * c["cin"] * 9


def _conv_bytes(c, kind):
    x = C4_B * c["cin"] * c["h"] ** 2 * 4
    y = C4_B * c["cout"] * c["oh"] ** 2 * 4
    w = c["cout"] * c["cin"] * 9 * 4 + c["cout"] * 4
    return x + y + w      # fwd: x, w, b in, y out; dW: x, dy in, dw, db out; dX: dy, w in, dx out


C4_STEP_FLOP = 1476395008 + 2726297600     # fwd + bwd (conv1's data gradient is not needed)
C1_FLOP = 30048256 + 34406400


def bench_c4(reps: int = 40):
    """Config 4: the CNN step through the C++ API, then its five convolution
    launches at their batch-128 shapes (conv1 3 -> 32, 32 x 32, stride 1;
    conv2 32 -> 64, stride 2; both 3 x 3, pad 1), `reps` event-timed
    launches each over 4 buffer sets, each against its roofline: conv1
    (27-deep products) against HBM, conv2 against fp32 MFMA."""
    import tensors_amd as ta
    from tensors_amd import api, ops, synth
    xs = synth.normal(synth.seed(4, 0), (1, C4_B, 3, 32, 32))
    ys = synth.uniform_int(synth.seed(4, 1), (1, C4_B), 10)
    # 100 timed steps after 50 untimed ones: 20 steps after 3 varied by
    # +-3 % from run to run.
    _, step_ms = api.cnn_train(xs, ys, steps=150, warmup=50, lr=0.01, mu=0.9, on_gpu=True)
    events = _conv_events(reps)
    kernels = {}
    for name, us in events.items():
        c = C4_CONV1 if name.startswith("conv1") else C4_CONV2
        flop, nbytes = _conv_flop(c), _conv_bytes(c, name)
        kernels[name] = {"us": us, "flop": flop, "tflops": round(flop / us / 1e6, 2),
                         "frac_fp32": round(flop / us / 1e6 / PEAK_FP32_TFLOPS, 3), "bytes": nbytes,
                         "gbps": round(nbytes / us / 1e3, 1), "frac_hbm": round(nbytes / us / 1e3 / PEAK_HBM_GBPS, 3),
                         "bound": "hbm" if c is C4_CONV1 else "mfma"}
    step_tf = C4_STEP_FLOP / (step_ms * 1e-3) / 1e12
    return {"workload": "C4 CNN fp32, batch 128: Conv(3->32, 3x3, s1 p1)+ReLU, Conv(32->64, 3x3, s2 p1)+ReLU, "
                        "flatten, Linear(16384->10), CE, SGD momentum (lr 0.01, mu 0.9); whole step through the "
                        "C++ API",
            "ms_per_step": round(step_ms, 4),
            "roofline": {"bound": "mfma", "kernel": "whole step (4 convolution GEMMs + classifier), FLOP / step time",
                         "achieved": round(step_tf, 2), "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(step_tf / PEAK_FP32_TFLOPS, 4), "traffic": None,
                         "algorithmic_flop_per_step": C4_STEP_FLOP},
            "conv_kernels": kernels}


def _conv_events(reps):
    """Event-timed launches (us) of the five implicit convolution kernels at
    their config-4 shapes, over 4 buffer sets."""
    import tensors_amd as ta
    from tensors_amd import ops, synth
    ctx = ta.Context(0)
    B, S = C4_B, 4
    x1 = [ctx.array(synth.normal(synth.seed(7, i), (B, 3, 32, 32))) for i in range(S)]
    h1 = [ctx.array(synth.normal(synth.seed(7, 10 + i), (B, 32, 32, 32))) for i in range(S)]
    w1, b1 = ctx.array(synth.normal(synth.seed(7, 20), (32, 3, 3, 3), std=0.2)), ctx.zeros((32,))
    w2, b2 = ctx.array(synth.normal(synth.seed(7, 21), (64, 32, 3, 3), std=0.06)), ctx.zeros((64,))
    y1 = [ctx.empty((B, 32, 32, 32)) for _ in range(S)]
    y2 = [ctx.empty((B, 64, 16, 16)) for _ in range(S)]
    dy1 = [ctx.array(synth.normal(synth.seed(7, 30 + i), (B, 32, 32, 32))) for i in range(S)]
    dy2 = [ctx.array(synth.normal(synth.seed(7, 40 + i), (B, 64, 16, 16))) for i in range(S)]
    dh1 = [ctx.empty((B, 32, 32, 32)) for _ in range(S)]
    gw1, gw2, gb1, gb2 = ctx.empty((32, 3, 3, 3)), ctx.empty((64, 32, 3, 3)), ctx.empty((32,)), ctx.empty((64,))
    cases = {
        "conv1_fwd": lambda i: ops.conv2d_fwd(x1[i], w1, y1[i], b1, (1, 1), (1, 1), (1, 1), True),
        "conv2_fwd": lambda i: ops.conv2d_fwd(h1[i], w2, y2[i], b2, (2, 2), (1, 1), (1, 1), True),
        "conv1_dw_db": lambda i: ops.conv2d_bwd_weight(x1[i], dy1[i], gw1, (1, 1), (1, 1), db=gb1),
        "conv2_dw_db": lambda i: ops.conv2d_bwd_weight(h1[i], dy2[i], gw2, (2, 2), (1, 1), db=gb2),
        "conv2_dx": lambda i: ops.conv2d_bwd_data(dy2[i], w2, dh1[i], (2, 2), (1, 1)),
    }
    out = {name: round(_rotating_bench(ctx, S, f, reps) * 1e3, 2) for name, f in cases.items()}
    ctx.close()
    return out


def _c5_inputs():
    from tensors_amd import synth
    xs = synth.normal(synth.seed(5, 0), (1, C5_BATCH, C5_DIMS[0]))
    ys = synth.uniform_int(synth.seed(5, 1), (1, C5_BATCH), C5_DIMS[-1])
    return xs, ys


def _gemm_kind(ta, tb):
    return {(0, 1): "fwd", (0, 0): "dX", (1, 0): "dW"}.get((ta, tb), f"ta{ta}tb{tb}")


def bench_c5(steps: int, warmup: int, timing_steps: int = 12, timing_warmup: int = 5):
    """Config-5 step through the C++ API: timed steps, then a second pass with
    the launch timing on for the per-GEMM durations.  The second pass builds
    its model anew (a second or two of host work, while the GPU idles and its
    clocks drop), so its first `timing_warmup` steps (16 ms) are not used."""
    from tensors_amd import api
    from tensors_amd._lib import call
    import ctypes as C

    xs, ys = _c5_inputs()
    kw = dict(lr=0.01, mu=0.9, on_gpu=True, bf16=True)
    losses, _, ms = api.mlp_train(C5_DIMS, xs, ys, steps=warmup + steps, warmup=warmup, **kw)
    per_step = 3 * (len(C5_DIMS) - 1) - 1     # 4 forward, 4 dW, 3 dX (the input needs no gradient)
    call("tf_hip_timing_start", per_step * timing_steps + 64)
    try:
        api.mlp_train(C5_DIMS, xs, ys, steps=timing_steps, warmup=0, **kw)
    finally:
        n = C.c_int(0)
        call("tf_hip_timing_stop", C.byref(n))
    shape = (C.c_int64 * 4)()
    meta = (C.c_int * 4)()
    t = C.c_float()
    recs = []
    for i in range(n.value):
        call("tf_hip_timing_record", i, shape, meta, C.byref(t))
        recs.append((tuple(shape), tuple(meta), t.value))
    if len(recs) != per_step * timing_steps:
        raise RuntimeError(f"C5 timing pass: {len(recs)} GEMM records, expected {per_step * timing_steps}")
    recs = recs[per_step * timing_warmup:]
    nsteps = timing_steps - timing_warmup
    gemms = {}
    for (M, N, K, _), (ta, tb, _, _), ms_k in recs:
        key = (_gemm_kind(ta, tb), M, N, K)
        g = gemms.setdefault(key, {"ms": [], "flop": 2 * M * N * K})
        g["ms"].append(ms_k)
    per_gemm = []
    bwd_flop = bwd_ms = fwd_flop = fwd_ms = 0.0
    for (kind, M, N, K), g in gemms.items():
        mean = float(np.mean(g["ms"]))
        calls = len(g["ms"]) / nsteps
        per_gemm.append({"kind": kind, "M": M, "N": N, "K": K, "per_step": calls, "us": round(mean * 1e3, 1),
                         "tflops": round(g["flop"] / (mean * 1e-3) / 1e12, 1)})
        if kind == "fwd":
            fwd_flop += g["flop"] * calls
            fwd_ms += mean * calls
        else:
            bwd_flop += g["flop"] * calls
            bwd_ms += mean * calls
    return {"ms_step": ms, "losses_finite": bool(np.all(np.isfinite(losses))), "per_gemm": per_gemm,
            "bwd_flop_step": bwd_flop, "bwd_ms_step": bwd_ms, "fwd_flop_step": fwd_flop, "fwd_ms_step": fwd_ms,
            "bwd_launches_step": int(round(sum(p["per_step"] for p in per_gemm if p["kind"] != "fwd")))}


def _host_info():
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, os.cpu_count()


def cpu_baseline_c5():
    """Reference CPU path on a bounded sample of config 5, extrapolated.

    The reference has no bf16 path and no threads; its fp32 nn::Linear
    forward + engine backward (naive GEMMs plus transpose copies of W) is
    timed for the middle layer shape 4096 -> 8192 at batch rows B = 2 and 6
    (the module constructor timed apart and removed).  Time is linear in B
    plus a fixed part (the copies of W); both scale with in*out, so the
    step estimate is (fixed + slope * 4096) * sum(in*out) / (4096*8192).
    Uses oracle/_ref (the reference compiled from its sources) when present,
    else the C restatement.
    """
    import oracle
    inn, out = 4096, 8192
    rng = np.random.default_rng(0x7E45)
    W = rng.standard_normal((out, inn), dtype=np.float32) * np.float32(inn ** -0.5)
    kind = "reference" if oracle.ref_available() else "port"
    times = {}
    init_s = 0.0
    if kind == "reference":
        w0 = np.empty((out, inn), np.float32)
        t0 = time.perf_counter()
        oracle.ref_call("ref_linear_init", inn, out, w0)
        init_s = time.perf_counter() - t0
    for B in (2, 6):
        X = rng.standard_normal((B, inn), dtype=np.float32)
        dY = rng.standard_normal((B, out), dtype=np.float32)
        t0 = time.perf_counter()
        if kind == "reference":
            y = np.empty((B, out), np.float32)
            dx = np.empty((B, inn), np.float32)
            dw = np.empty((out, inn), np.float32)
            oracle.ref_call("ref_linear", X, W, dY, y, dx, dw, B, inn, out)
        else:
            oracle.linear_fwd(X, W)
            oracle.linear_bwd(X, W, dY)
        times[B] = time.perf_counter() - t0 - init_s
    slope = (times[6] - times[2]) / 4.0
    fixed = max(times[2] - 2 * slope, 0.0)
    layer_ms = (fixed + slope * C5_BATCH) * 1e3
    scale = sum(C5_DIMS[i] * C5_DIMS[i + 1] for i in range(len(C5_DIMS) - 1)) / (inn * out)
    model, ncpu = _host_info()
    return {
        "value": round(layer_ms * scale, 1),
        "unit": "ms/step",
        "cores": 1,
        "kind": kind,
        "extrapolated": True,
        "host": f"{model}, {ncpu} logical CPUs visible; the reference is single-threaded",
        "sample": (f"fp32 Linear 4096->8192 fwd+bwd (reference order) at batch 2 and 6 rows "
                   f"({times[2]:.2f} s, {times[6]:.2f} s after {init_s:.2f} s of module init), extrapolated "
                   f"linearly to 4096 rows and by weight count to the 4 layers (x{scale:.3f}); "
                   f"fp32 stands in for bf16, which the reference lacks"),
    }


def cpu_baseline_c2():
    """Reference CPU path on a bounded sample of config 2.

    nn::Linear forward + engine backward (reference order: transpose copies +
    naive GEMMs) at batch rows B = 32 and 96; the time is linear in B plus a
    fixed part (the 2048 x 2048 transposes of W), so the full-batch step time
    is the fit evaluated at B = 2048.  Uses oracle/_ref (the reference compiled
    from its sources) when present, else the C restatement.
    """
    import oracle
    from tensors_amd import synth

    inn = out = N2
    W = synth.normal(synth.seed(2, 1), (out, inn))
    times = {}
    kind = "reference" if oracle.ref_available() else "port"
    for B in (32, 96):
        X = synth.normal(synth.seed(2, 0), (N2, inn))[:B].copy()
        dY = synth.normal(synth.seed(2, 2), (N2, out))[:B].copy()
        t0 = time.perf_counter()
        if kind == "reference":
            y = np.empty((B, out), np.float32)
            dx = np.empty((B, inn), np.float32)
            dw = np.empty((out, inn), np.float32)
            oracle.ref_call("ref_linear", X, W, dY, y, dx, dw, B, inn, out)
        else:
            oracle.linear_fwd(X, W)
            oracle.linear_bwd(X, W, dY)
        times[B] = time.perf_counter() - t0
    slope = (times[96] - times[32]) / 64.0
    fixed = max(times[32] - 32 * slope, 0.0)
    full_ms = (fixed + slope * N2) * 1e3
    return {
        "value": full_ms,
        "unit": "ms/step",
        "cores": 1,
        "kind": kind,
        "sample": (f"Linear 2048->2048 fwd+bwd at batch 32 and 96 rows ({times[32]:.2f} s, {times[96]:.2f} s), "
                   f"extrapolated linearly to 2048 rows; single thread"),
    }


def _ref_seconds(name, *args):
    """Mean seconds of one of oracle/_ref's timed runs (ref_time_*)."""
    import ctypes as C
    import oracle
    sec = C.c_double(0.0)
    oracle.ref_call(name, *args, C.byref(sec))
    return sec.value


def cpu_baseline_c1():
    """The compiled reference's config-1 step: Linear(784,256)-ReLU-
    Linear(256,128)-ReLU-Linear(128,10), the train_mlp cross-entropy chain,
    loss.backward() and the manual momentum loop (examples/train_mlp.cpp:
    54-76, 145-159), batch 64, through oracle/_ref's ref_mlp_train; 2 and 12
    steps, the difference over 10 steps (the modules' construction cancels).
    Without oracle/_ref: the C restatement of the same step."""
    import oracle
    from tensors_amd import synth
    xs = synth.mnist_like(synth.seed(1, 0), (12, 64, 784))
    ys = synth.uniform_int(synth.seed(1, 1), (12, 64), 10)
    dims = np.array([784, 256, 128, 10], np.int32)
    kind = "reference" if oracle.ref_available() else "port"
    t = {}
    for steps in (2, 12):
        t0 = time.perf_counter()
        if kind == "reference":
            losses = np.empty(steps, np.float32)
            oracle.ref_call("ref_mlp_train", xs, ys, steps, 64, 0.1, 0.9, losses, dims, 4, None)
        else:
            ws = [np.zeros((dims[i + 1], dims[i]), np.float32) + np.float32(0.01) for i in range(3)]
            vs = [np.zeros_like(w) for w in ws]
            for s_ in range(steps):
                oracle.mlp_step(ws, vs, xs[s_], ys[s_], 0.1, 0.9)
        t[steps] = time.perf_counter() - t0
    model, ncpu = _host_info()
    return {"value": round((t[12] - t[2]) / 10 * 1e3, 2), "unit": "ms/step", "cores": 1, "kind": kind,
            "host": f"{model}, {ncpu} logical CPUs visible; the reference is single-threaded",
            "sample": f"config-1 steps at batch 64: 12 steps {t[12]:.2f} s, 2 steps {t[2]:.2f} s; per step = "
                      "the difference over 10 steps (fwd + loss.backward() + momentum loop)"}


def cpu_baseline_c3():
    """The compiled reference's backward nodes at config 3's shapes, each
    timed alone (oracle/_ref ref_time_*, inputs and forward graphs built
    outside the timed part): the whole train_mlp cross-entropy chain's
    backward (loss.backward(), what the fused LogSoftmax+NLL kernel
    replaces) and LogSoftmaxBackward::apply by itself at [4096 x 1024];
    ReluBackward::apply at [4096 x 1024]; the LayerNorm backward through the
    engine at [1024 x 1024] (the reference's stub, dX = dY * gamma), and the
    true LayerNorm gradient's C restatement (oracle.layernorm_bwd), which
    the GPU kernel computes.  Returns {c3 entry name: cpu_baseline}."""
    import oracle
    from tensors_amd import synth
    model, ncpu = _host_info()
    host = f"{model}, {ncpu} logical CPUs visible; the reference is single-threaded"
    R, Cc = 4096, 1024
    logits = synth.normal(synth.seed(3, 0), (R, Cc), std=3.0)
    tg = synth.uniform_int(synth.seed(3, 1), (R,), Cc)
    x = synth.normal(synth.seed(3, 2), (R, Cc))
    dy = synth.normal(synth.seed(3, 3), (R, Cc))
    L = 1024
    lx, ldy = synth.normal(synth.seed(3, 4), (L, L)), synth.normal(synth.seed(3, 5), (L, L))
    g, b = np.ones(L, np.float32), np.zeros(L, np.float32)
    out = {}
    if not oracle.ref_available():
        return out
    import ctypes as C
    chain = _ref_seconds("ref_time_ce_chain_bwd", logits, tg, R, Cc, C.c_int32(3))
    node = _ref_seconds("ref_time_log_softmax_bwd", logits, tg, R, Cc, C.c_int32(3))
    out["c3a_logsoftmax_nll_bwd"] = {
        "value": round(chain * 1e3, 2), "unit": "ms", "cores": 1, "kind": "reference", "host": host,
        "sample": f"the cross-entropy chain's loss.backward() at [4096 x 1024], mean of 3 (LogSoftmaxBackward::apply "
                  f"alone: {node * 1e3:.2f} ms)"}
    relu = _ref_seconds("ref_time_relu_bwd", dy, x, R * Cc, C.c_int32(5))
    out["c3b_relu_bwd"] = {"value": round(relu * 1e3, 2), "unit": "ms", "cores": 1, "kind": "reference",
                           "host": host, "sample": "ReluBackward::apply at [4096 x 1024], mean of 5"}
    stub = _ref_seconds("ref_time_layernorm_bwd", lx, g, b, ldy, L, L, 1e-5, C.c_int32(10))
    _, mean, rstd = oracle.layernorm_fwd(lx, g, b)
    t0 = time.perf_counter()
    for _ in range(5):
        oracle.layernorm_bwd(lx, ldy, g, mean, rstd)
    true_ms = (time.perf_counter() - t0) / 5 * 1e3
    out["c3c_layernorm_bwd"] = {
        "value": round(stub * 1e3, 2), "unit": "ms", "cores": 1, "kind": "reference", "host": host,
        "sample": f"the reference's LayerNorm backward (its stub, dX = dY * gamma) through the engine at "
                  f"[1024 x 1024], mean of 10; the true gradient, which the GPU computes, in the C restatement: "
                  f"{true_ms:.2f} ms"}
    return out


def cpu_baseline_c4():
    """Config 4's step on the CPU, restated: the reference has no CPU
    convolution backward.  The forward convolutions are the compiled
    reference's Conv2dModule::forward (oracle/_ref ref_conv2d_fwd), the
    backward convolutions the reference test's loop (nn/conv2d_backward_test
    .cpp:50-106, restated in oracle.conv2d_bwd), the rest the restated
    reference ops (oracle: ReLU, Linear, the CE chain, momentum SGD), all
    single-threaded; batch 16 and 48 timed, extrapolated linearly to 128.
    Labelled a port: its largest part, the backward loop, is the restated
    one."""
    import oracle
    from tensors_amd import synth
    ref = oracle.ref_available()
    params = [synth.normal(synth.seed(4, 10 + i), s, std=sd) for i, (s, sd) in
              enumerate(zip([(32, 3, 3, 3), (32,), (64, 32, 3, 3), (64,), (10, 16384), (10,)],
                            [0.2, 0.1, 0.06, 0.1, 0.01, 0.1]))]
    x_all = synth.normal(synth.seed(4, 0), (C4_B, 3, 32, 32))
    y_all = synth.uniform_int(synth.seed(4, 1), (C4_B,), 10)

    def conv_fwd(x, w, bb, stride):
        if not ref:
            return oracle.conv2d_fwd(x, w, bb, stride, 1)
        N, Cin, H, _ = x.shape
        Cout = w.shape[0]
        oh = (H + 2 - 3) // stride + 1
        yv = np.empty((N, Cout, oh, oh), np.float32)
        oracle.ref_call("ref_conv2d_fwd", np.ascontiguousarray(x), w, bb, yv, N, Cin, H, H, Cout, 3, stride, 1)
        return yv

    t = {}
    for B in (16, 48):
        x, y = np.ascontiguousarray(x_all[:B]), y_all[:B].copy()
        ps = [p.copy() for p in params]
        vs = [np.zeros_like(p) for p in ps]
        w1, b1, w2, b2, wf, bfc = ps
        t0 = time.perf_counter()
        z1 = conv_fwd(x, w1, b1, 1)
        h1 = oracle.relu(z1)
        z2 = conv_fwd(h1, w2, b2, 2)
        h2 = oracle.relu(z2)
        f = h2.reshape(B, -1)
        logits = oracle.add(oracle.linear_fwd(f, wf), np.broadcast_to(bfc, (B, 10)))
        _, gl = oracle.ce_chain(logits, y)
        df, dwf = oracle.linear_bwd(f, wf, gl)
        dbf = oracle.colsum(gl)
        dz2 = oracle.relu_bwd(df.reshape(h2.shape), z2)
        dh1, dw2, db2 = oracle.conv2d_bwd(h1, w2, dz2, (2, 2), (1, 1), (1, 1))
        dz1 = oracle.relu_bwd(dh1, z1)
        _, dw1, db1 = oracle.conv2d_bwd(x, w1, dz1, (1, 1), (1, 1), (1, 1))
        for i, gr in enumerate((dw1, db1, dw2, db2, dwf, dbf)):
            oracle.sgd_momentum(ps[i], gr, vs[i], 0.01, 0.9)
        t[B] = time.perf_counter() - t0
    slope = (t[48] - t[16]) / 32.0
    fixed = max(t[16] - 16 * slope, 0.0)
    model, ncpu = _host_info()
    return {"value": round((fixed + slope * C4_B) * 1e3, 1), "unit": "ms/step", "cores": 1,
            "kind": "port", "restated": True, "extrapolated": True,
            "host": f"{model}, {ncpu} logical CPUs visible; single-threaded",
            "sample": f"config-4 step at batch 16 and 48 ({t[16]:.2f} s, {t[48]:.2f} s), extrapolated linearly to "
                      f"128; forward convolutions by {'the compiled reference' if ref else 'the C restatement of'} "
                      f"Conv2dModule::forward, their "
                      f"backward by the reference test's loop restated (the reference has no CPU conv backward)"}


TRAFFIC_JSON = {"c2": ROOT / "profiles" / "gemm_f32_c2_traffic.json",
                "c5": ROOT / "profiles" / "gemm_bf16_c5_traffic.json"}
PROBE_CAL_N = 1 << 26      # calibration tf_add: reads 2 x 256 MB, writes 256 MB


def load_traffic(config: str, name: str):
    """Calibrated HBM bytes per launch from the committed counter summary
    (tensors_amd.profiling traffic), or None when it is absent."""
    path = TRAFFIC_JSON[config]
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get(name)
    except Exception:
        return None


def _probe_calibration(ctx):
    from tensors_amd import ops
    ca, cb, cc = ctx.zeros((PROBE_CAL_N,)), ctx.zeros((PROBE_CAL_N,)), ctx.empty((PROBE_CAL_N,))
    for _ in range(3):
        ops.add(ca, cb, cc)
    ctx.sync()


def probe_c2(steps: int = 5) -> None:
    """Launches for rocprofv3 counter runs: `steps` C2 steps (fwd GEMM, dX,
    dW, colsum, SGD) and 3 calibration tf_add launches over PROBE_CAL_N
    floats whose traffic is known.  No timing, no output but one line."""
    import tensors_amd as ta
    from tensors_amd import ops, synth

    ctx = ta.Context(0)
    X = ctx.array(synth.normal(synth.seed(2, 0), (N2, N2)))
    W = ctx.array(synth.normal(synth.seed(2, 1), (N2, N2)))
    dY = ctx.array(synth.normal(synth.seed(2, 2), (N2, N2)))
    b = ctx.array(synth.normal(synth.seed(2, 3), (N2,)))
    Y, dX, dW, db = ctx.empty((N2, N2)), ctx.empty((N2, N2)), ctx.empty((N2, N2)), ctx.empty((N2,))
    vW, vb = ctx.zeros((N2, N2)), ctx.zeros((N2,))
    for _ in range(steps):
        ops.gemm(X, W, Y, trans_b=True, bias=b)
        ops.gemm(dY, W, dX)
        ops.gemm(dY, X, dW, trans_a=True)
        ops.colsum(dY, db)
        ops.sgd_momentum_multi([W, b], [dW, db], [vW, vb], 1e-3, 0.9)
    ctx.sync()
    _probe_calibration(ctx)
    ctx.close()
    print(f"probe: {steps} C2 steps, 3 calibration launches", flush=True)


def probe_c5(steps: int = 3) -> None:
    """Launches for rocprofv3 counter runs: the config-5 step's GEMMs at their
    shapes, layouts and output types (forward with bias + ReLU in bf16, dX in
    bf16, dW in fp32), `steps` times over, then the calibration launches."""
    import tensors_amd as ta
    from tensors_amd import ops

    ctx = ta.Context(0)
    rng = np.random.default_rng(0x7E45)
    B, d = C5_BATCH, C5_DIMS
    bf = lambda shape, sd=1.0: ctx.array(ta.f32_to_bf16_bits(rng.standard_normal(shape, dtype=np.float32)
                                                             * np.float32(sd)), ta.BF16)
    acts = [bf((B, d[i])) for i in range(4)]
    ws = [bf((d[i + 1], d[i]), d[i] ** -0.5) for i in range(4)]
    grads = [bf((B, d[i + 1]), 1e-3) for i in range(4)]
    biases = [ctx.zeros((d[i + 1],)) for i in range(4)]
    outs = [ctx.empty((B, d[i + 1]), ta.BF16) for i in range(4)]
    dxs = [ctx.empty((B, d[i]), ta.BF16) for i in range(4)]
    dws = [ctx.empty((d[i + 1], d[i])) for i in range(4)]
    for _ in range(steps):
        for i in range(4):
            ops.gemm(acts[i], ws[i], outs[i], trans_b=True, bias=biases[i], relu=i < 3)
        for i in range(3, -1, -1):
            ops.gemm(grads[i], acts[i], dws[i], trans_a=True)
            if i > 0:
                ops.gemm(grads[i], ws[i], dxs[i])
    ctx.sync()
    _probe_calibration(ctx)
    ctx.close()
    print(f"probe: {steps} x the C5 step's GEMMs, 3 calibration launches", flush=True)


def probe_bw() -> None:
    """Launches for rocprofv3 runs: every bandwidth kernel of the path at its
    configuration's shape (bench_c3 without the extra kernels, then
    bench_bandwidth_rotated), 20 timed launches each over rotated buffers,
    then the calibration launches.  Prints the event timings (us per launch,
    keyed by the labels of tensors_amd.profiling.BW_KERNELS) as one JSON
    line; run unprofiled, they are the figures a --kernel-trace run of the
    same command is set beside."""
    c3 = bench_c3(more=False, reps=20)
    out = {"ce_bwd_c3a": c3["c3a_logsoftmax_nll_bwd"]["us"],
           "ce_fused_fwd_bwd_c3a": c3["c3a_ce_fused_fwd_bwd"]["us"],
           "relu_bwd_c3b": c3["c3b_relu_bwd"]["us"],
           "layernorm_bwd_op_c3c": c3["c3c_layernorm_bwd"]["us"]}
    out.update({k: v["us"] for k, v in bench_bandwidth_rotated(reps=20).items()})
    import tensors_amd as ta
    ctx = ta.Context(0)
    _probe_calibration(ctx)
    ctx.close()
    print(json.dumps({"bw_events_us": out}), flush=True)


def probe_c4() -> None:
    """Launches for rocprofv3 runs of config 4: 13 API training steps (3
    warmup), then its five implicit-GEMM convolution launches at their C4
    shapes, 40 event-timed launches each over 4 buffer sets (_conv_events),
    then the calibration launches.  Prints the step time and the per-launch
    event timings (us) as one JSON line."""
    import tensors_amd as ta
    from tensors_amd import api, synth
    xs = synth.normal(synth.seed(4, 0), (1, C4_B, 3, 32, 32))
    ys = synth.uniform_int(synth.seed(4, 1), (1, C4_B), 10)
    _, step_ms = api.cnn_train(xs, ys, steps=13, warmup=3, lr=0.01, mu=0.9, on_gpu=True)
    out = _conv_events(40)
    ctx = ta.Context(0)
    _probe_calibration(ctx)
    ctx.close()
    print(json.dumps({"c4_step_ms": round(step_ms, 4), "conv_events_us": out}), flush=True)


def c2_report(steps: int, warmup: int) -> dict:
    ms_step, mean, per = bench_c2(steps, warmup)
    bwd_ms = 0.5 * (mean["bwd_gemm_dx"] + mean["bwd_gemm_dw"])
    bwd_tflops = GEMM_FLOP / (bwd_ms * 1e-3) / 1e12
    fwd_tflops = GEMM_FLOP / (mean["fwd_gemm"] * 1e-3) / 1e12
    colsum_gbps = (N2 * N2 * 4 + N2 * 4) / (mean["colsum"] * 1e-3) / 1e9
    sgd_gbps = (N2 * N2 + N2) * 20 / (mean["sgd"] * 1e-3) / 1e9
    return {
        "workload": "C2 isolated Linear 2048x2048 fp32: fwd GEMM+bias, bwd dX/dW GEMMs, bias colsum, "
                    "fused SGD-momentum on W and b (ops level, device-resident)",
        "ms_per_step": round(ms_step, 4),
        "steps": steps,
        "warmup": warmup,
        "dtype": "f32",
        "roofline": {
            "bound": "mfma",
            "kernel": "gemm_f32 (bwd dX NN + dW TN, mean of both)",
            "achieved": round(bwd_tflops, 2),
            "peak": PEAK_FP32_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(bwd_tflops / PEAK_FP32_TFLOPS, 4),
            "traffic": load_traffic("c2", "gemm_f32_bwd_c2"),
            "algorithmic_flop_per_launch": GEMM_FLOP,
        },
        "kernels_ms": {k: round(v, 5) for k, v in mean.items()},
        "fwd_gemm_tflops": round(fwd_tflops, 2),
        "colsum_gbps": round(colsum_gbps, 1),
        "sgd_gbps": round(sgd_gbps, 1),
        "step_ms_device_median": round(_median(per["step_dev"]), 4),
    }


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # The GPU's clocks need more than ~10 ms of load to settle after the
    # host-side input generation: 5 warmup steps of config 5 are ~16 ms.
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--only-headline", action="store_true", help="skip the other configurations' measurements")
    ap.add_argument("--probe", choices=["c2", "c4", "c5", "bw"],
                    help="launch a config's kernels (bw: the bandwidth kernels) for a profiler, then exit")
    ap.add_argument("--hbm-ceiling", action="store_true",
                    help="run the HBM streaming-ceiling microbenchmark, print its JSON line, then exit")
    ap.add_argument("--config", choices=["c1", "c2", "c3", "c4", "bw"],
                    help="run only this entry of other_configs (as the full run measures it, without its CPU "
                         "baseline), print it as one JSON line, then exit: the command a profiler wraps to "
                         "reproduce that entry's figures")
    args = ap.parse_args(argv)
    if args.probe:
        {"c2": probe_c2, "c4": probe_c4, "c5": probe_c5, "bw": probe_bw}[args.probe]()
        return 0
    if args.config:
        run = {"c1": bench_c1, "c2": lambda: c2_report(100, 50), "c3": bench_c3, "c4": bench_c4,
               "bw": bench_bandwidth_rotated}[args.config]
        print(json.dumps({"config": args.config, "report": run()}), flush=True)
        return 0
    if args.hbm_ceiling:
        print(json.dumps({"hbm_ceiling": hbm_ceiling()}), flush=True)
        return 0

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the path's multi-GPU sharding is a design note, not a measured configuration.", file=sys.stderr)
        return 2
    rank = int(os.environ.get("RANK", "0"))

    c5 = bench_c5(args.steps, args.warmup)
    ms_step = c5["ms_step"]
    bwd_tflops = c5["bwd_flop_step"] / (c5["bwd_ms_step"] * 1e-3) / 1e12
    step_flop = c5["fwd_flop_step"] + c5["bwd_flop_step"]
    line = {
        "metric": "fwd+bwd+SGD step ms; bwd GEMM TFLOPS & bwd kernel GB/s as % MI355X peak",
        "value": round(ms_step, 4),
        "unit": "ms/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) inputs, uniform labels; Kaiming-uniform init from the reference's seed)",
        "config": {"workload": "C5 wide MLP 4096-8192-8192-4096-1000, batch 4096, bf16 weights/activations with "
                               "fp32 accumulate and fp32 master weights, ReLU, CrossEntropy over 1000 labels, "
                               "SGD momentum (lr 0.01, mu 0.9); full fwd+bwd+SGD step through the C++ API",
                   "dims": C5_DIMS, "batch": C5_BATCH},
        "roofline": {
            "bound": "mfma",
            "kernel": f"bf16 backward GEMMs ({c5['bwd_launches_step']} launches per step: 4 dW, 3 dX), "
                      "FLOP over summed event-timed durations",
            "achieved": round(bwd_tflops, 1),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(bwd_tflops / PEAK_BF16_TFLOPS, 4),
            "traffic": load_traffic("c5", "gemm_bf16_bwd_c5"),
            "algorithmic_flop_per_step": int(c5["bwd_flop_step"]),
        },
        "step_tflops": round(step_flop / (ms_step * 1e-3) / 1e12, 1),
        "gemm_ms_per_step": {"fwd": round(c5["fwd_ms_step"], 4), "bwd": round(c5["bwd_ms_step"], 4)},
        "fwd_gemm_tflops": round(c5["fwd_flop_step"] / (c5["fwd_ms_step"] * 1e-3) / 1e12, 1),
        "per_gemm": c5["per_gemm"],
        "losses_finite": c5["losses_finite"],
    }
    if not args.only_headline:
        # Each configuration starts from an empty memory pool, as in a process
        # of its own: after C5's and C2's gigabytes were pooled, conv1's
        # ReLU-masked weight gradient in the C4 step ran 12.3 -> 16.9 us.
        from tensors_amd import api
        oc = {}
        for name, run in (("c2", lambda: c2_report(100, 50)), ("c3", bench_c3),
                          ("bandwidth_rotated", bench_bandwidth_rotated), ("c1", bench_c1), ("c4", bench_c4)):
            api.release_memory()
            oc[name] = run()
        line["other_configs"] = oc
    if rank == 0 and not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_c5()
        if "other_configs" in line:
            oc = line["other_configs"]
            oc["c2"]["cpu_baseline"] = cpu_baseline_c2()
            oc["c1"]["cpu_baseline"] = cpu_baseline_c1()
            for name, cb in cpu_baseline_c3().items():
                oc["c3"][name]["cpu_baseline"] = cb
            oc["c4"]["cpu_baseline"] = cpu_baseline_c4()
    if rank == 0:
        print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
