"""The cross-block reductions that finish in their last-arriving block, run
many times over, each result compared bit for bit with the first.

Six kernels publish per-block partial sums with agent-scope atomic stores,
wait until those stores have landed, and count themselves in on a
per-output counter; the block that draws the last ticket adds the partials
in a fixed order (tfd::wait_stores_landed in csrc/common.hpp states why
this is ordered on gfx950).  A partial read before it landed, or a counter
left non-zero by an earlier launch, would show as a result that differs
from one launch to the next on the same inputs.  Each case runs at the
configuration shape that takes the ticket path:

* colsum_tile_kernel: config 2's bias gradient (2048 x 2048, fp32) and
  config 5's 1000-wide output bias (4096 x 1000, bf16, a ragged last strip);
* relu_bwd_colsum_kernel: config 5's layer-1 ReLU backward + bias gradient
  (4096 x 8192, bf16);
* ln_bwd_onepass_kernel: config 3c's LayerNorm backward (1024 x 1024);
* gemm_f32_small_kernel: config 1's first layer forward (64 x 256 x 784,
  13 K chunk groups per tile);
* gemm_f32_narrow_mfma_kernel: config 4's classifier forward (128 x 10 x 16384);
* ce_kernel's in-kernel loss mean: config 1's and config 4's cross entropy
  (64 x 10 and 128 x 10 logits: 16 and 32 blocks, a grid small enough for
  the last block to form the mean), and larger grids whose mean is a
  separate one-block launch (4096 x 1024, 8000 and 8100 rows).

A mismatch fails at the first repetition that differs (named in the
message); the first result is also checked against float64.
"""
from __future__ import annotations

import numpy as np
import pytest

import tensors_amd as ta
from tensors_amd import ops, synth
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu

REPS = 200


def _bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    return a.view(np.uint16 if a.dtype.itemsize == 2 else np.uint32)


def _repeat(what, launch, outputs):
    """launch() REPS times; after each, every array in `outputs` must equal
    its value after the first launch bit for bit."""
    first = None
    for rep in range(REPS):
        launch()
        got = [_bits(o.numpy()).copy() for o in outputs]
        if first is None:
            first = got
            continue
        for k, (g, f) in enumerate(zip(got, first)):
            if not np.array_equal(g, f):
                bad = int(np.flatnonzero(g.ravel() != f.ravel())[0])
                pytest.fail(f"{what}: output {k} of repetition {rep} differs from the first at element {bad}")
    return first


def test_colsum_tile_repeats_bit_for_bit(ctx):
    dy = synth.normal(5101, (2048, 2048))
    d_dy, db = ctx.array(dy), ctx.empty((2048,))
    _repeat("colsum C2", lambda: ops.colsum(d_dy, db), [db])
    assert_close(db.numpy(), dy.astype(np.float64).sum(0), 1e-4, "colsum C2 vs float64")
    h = ta.f32_to_bf16_bits(synth.normal(5102, (4096, 1000)))
    d_h, db2 = ctx.array(h, ta.BF16), ctx.empty((1000,))
    _repeat("colsum bf16 C5 output layer", lambda: ops.colsum(d_h, db2), [db2])
    assert_close(db2.numpy(), ta.bf16_bits_to_f32(h).astype(np.float64).sum(0), 1e-4, "colsum bf16 vs float64")


def test_relu_bwd_colsum_repeats_bit_for_bit(ctx):
    R, Cc = 4096, 8192
    g = ta.f32_to_bf16_bits(synth.normal(5103, (R, Cc)))
    x = ta.f32_to_bf16_bits(synth.normal(5104, (R, Cc)))
    dg, dx_, dz, db = ctx.array(g, ta.BF16), ctx.array(x, ta.BF16), ctx.empty((R, Cc), ta.BF16), ctx.empty((Cc,))
    _repeat("relu_bwd_colsum C5", lambda: ops.relu_bwd_colsum(dg, dx_, dz, db), [db])
    masked = np.where(ta.bf16_bits_to_f32(x) > 0, ta.bf16_bits_to_f32(g), 0.0).astype(np.float64)
    assert_close(db.numpy(), masked.sum(0), 1e-4, "relu_bwd_colsum db vs float64")


def test_layernorm_bwd_onepass_repeats_bit_for_bit(ctx):
    R = Cc = 1024
    x, dy = synth.normal(5105, (R, Cc)), synth.normal(5106, (R, Cc))
    gamma = synth.normal(5107, (Cc,), std=0.1) + np.float32(1.0)
    dx_, ddy, dgam = ctx.array(x), ctx.array(dy), ctx.array(gamma)
    y, mean, rstd = ctx.empty((R, Cc)), ctx.empty((R,)), ctx.empty((R,))
    ops.layernorm_fwd(dx_, dgam, ctx.zeros((Cc,)), y, mean, rstd)
    dxo, dg, dbt = ctx.empty((R, Cc)), ctx.empty((Cc,)), ctx.empty((Cc,))
    _repeat("layernorm_bwd C3c", lambda: ops.layernorm_bwd(ddy, dx_, dgam, mean, rstd, dxo, dg, dbt), [dg, dbt, dxo])
    assert_close(dbt.numpy(), dy.astype(np.float64).sum(0), 1e-4, "dbeta vs float64")


def test_small_and_narrow_gemm_repeat_bit_for_bit(ctx):
    a, w = synth.normal(5108, (64, 784)), synth.normal(5109, (256, 784), std=0.05)
    da, dw, c = ctx.array(a), ctx.array(w), ctx.empty((64, 256))
    _repeat("gemm_f32_small C1 layer 1", lambda: ops.gemm(da, dw, c, trans_b=True), [c])
    assert_close(c.numpy(), a.astype(np.float64) @ w.astype(np.float64).T, 1e-4, "small GEMM vs float64")
    x, wf = synth.normal(5110, (128, 16384)), synth.normal(5111, (10, 16384), std=0.01)
    dxf, dwf, cf = ctx.array(x), ctx.array(wf), ctx.empty((128, 10))
    _repeat("gemm_f32_narrow_mfma C4 classifier", lambda: ops.gemm(dxf, dwf, cf, trans_b=True), [cf])
    assert_close(cf.numpy(), x.astype(np.float64) @ wf.astype(np.float64).T, 1e-4, "narrow GEMM vs float64")


@pytest.mark.parametrize("R,Cc", [(64, 10), (128, 10), (4096, 1024), (8000, 16), (8100, 16)])
def test_ce_loss_mean_repeats_bit_for_bit(ctx, R, Cc):
    """The in-kernel mean up to 64 blocks (C1's and C4's 16 and 32 blocks);
    the separate one-block mean launch after the kernel for larger grids
    (C3a's 4096 x 1024: 1024 blocks; 8000 and 8100 rows)."""
    logits = synth.normal(5112 + R, (R, Cc), std=3.0)
    labels = synth.uniform_int(5113 + R, (R,), Cc)
    dl_, dt = ctx.array(logits), ctx.array(labels)
    loss, dlog = ctx.empty((1,)), ctx.empty((R, Cc))
    _repeat(f"ce loss mean {R} x {Cc}", lambda: ops.ce_fwd_bwd(dl_, dt, loss, dlog), [loss, dlog])
    lg = logits.astype(np.float64)
    lse = np.log(np.exp(lg - lg.max(1, keepdims=True)).sum(1)) + lg.max(1)
    want = float(np.mean(lse - lg[np.arange(R), labels]))
    assert abs(float(loss.numpy()[0]) - want) <= 1e-5 * max(1.0, abs(want))
