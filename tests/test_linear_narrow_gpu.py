"""tf_linear_bwd_narrow: the backward of a Linear layer with few outputs
(dx = dy W, dw = dy^T x, db = column sums of dy) in one launch, against
float64 of the same fp32 inputs (rtol 1e-4 relative to the largest
magnitude, as the other fp32 GEMM tests).  The reference forms these as
MatmulBackward's two products (autograd/ops/MatmulBackward.hpp:26-34) behind
nn/Linear.cpp:60-63 plus the transpose of the weight gradient.

Shapes: config 4's classifier (128 x 10 x 16384), 16 outputs, a ragged last
column block (K = 1028), row counts that are not multiples of 16 and more
rows than one batch of a thread's loads (300), and a single row.  Each
output is checked with the others switched off, every output is written
once (the buffers start as 7.0), and a second call is bit-identical.
"""
from __future__ import annotations

import numpy as np
import pytest

from tensors_amd import ops, synth
from tests.conftest import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu

RTOL32 = 1e-4

CASES = [
    (128, 10, 16384),   # config 4's classifier
    (64, 16, 2048),     # 16 outputs
    (300, 3, 1028),     # ragged last column block, 300 rows (three row batches)
    (1, 7, 1024),       # one row
    (64, 10, 128),      # config 1's last layer (two column blocks)
]


@pytest.mark.parametrize("M,N,K", CASES)
def test_linear_bwd_narrow_vs_float64(ctx, M, N, K):
    dy = synth.normal(611 + M, (M, N))
    x = synth.normal(612 + N, (M, K))
    w = synth.normal(613 + K, (N, K), std=0.05)
    want = {"dx": dy.astype(np.float64) @ w.astype(np.float64),
            "dw": dy.astype(np.float64).T @ x.astype(np.float64),
            "db": dy.astype(np.float64).sum(0)}
    shapes = {"dx": (M, K), "dw": (N, K), "db": (N,)}
    d_dy, d_x, d_w = ctx.array(dy), ctx.array(x), ctx.array(w)
    outs = {k: ctx.array(np.full(s, 7.0, np.float32)) for k, s in shapes.items()}
    ops.linear_bwd_narrow(d_dy, d_x, d_w, outs["dx"], outs["dw"], outs["db"])
    first = {k: v.numpy() for k, v in outs.items()}
    for k in shapes:
        assert_close(first[k], want[k], RTOL32, f"{k} {M}x{N}x{K}")
    ops.linear_bwd_narrow(d_dy, d_x, d_w, outs["dx"], outs["dw"], outs["db"])
    for k in shapes:
        assert_bitexact(outs[k].numpy(), first[k], f"second call {k}")
    # One output at a time: the same values (x is not needed without dw).
    for only in shapes:
        o = ctx.array(np.full(shapes[only], 7.0, np.float32))
        ops.linear_bwd_narrow(d_dy, d_x if only == "dw" else None, d_w, **{only: o})
        assert_bitexact(o.numpy(), first[only], f"{only} alone")


def test_linear_bwd_narrow_rejects_unsupported(ctx):
    """More than 16 outputs, or K not a multiple of 4, is refused with an
    error (the Linear backward then takes the two GEMMs)."""
    dy, w = ctx.array(np.ones((4, 17), np.float32)), ctx.array(np.ones((17, 1024), np.float32))
    with pytest.raises(Exception, match="16"):
        ops.linear_bwd_narrow(dy, None, w, dx=ctx.empty((4, 1024)))
    dy2, w2 = ctx.array(np.ones((4, 3), np.float32)), ctx.array(np.ones((3, 1026), np.float32))
    with pytest.raises(Exception, match="K % 4"):
        ops.linear_bwd_narrow(dy2, None, w2, dx=ctx.empty((4, 1026)))
