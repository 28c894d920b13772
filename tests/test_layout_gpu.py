"""Row a9's layout and elementwise kernels at multi-block shapes, LeakyReLU
(the registry's sixth slot) and the device argmax, through the C ABI.

Bars: kernels whose arithmetic order equals the reference's are bit-exact
against the oracle (sum along a non-final dim walks the reduced dim in
order, as Tensor::sum does; broadcast, transpose, casts, sub, scale,
LeakyReLU and argmax are exact); the other reductions are within rtol 1e-4
of float64 with atol = rtol * rms.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tensors_amd import _lib, synth
from tensors_amd._lib import TFError, call
from tests.conftest import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu


# ---------------------------------------------------------------------------
# Tensor::sum along one dim and SumBackward's broadcast
# (tensor/Tensor.cpp:513-561, autograd/ops/SumBackward.hpp:27-39)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("outer,reduce,inner", [(1, 4096, 1024), (4096, 1024, 1), (8, 513, 257), (3, 1, 5),
                                                (2, 4097, 3), (1, 7, 1)])
def test_sum_dim(ctx, outer, reduce, inner):
    x = synth.normal(900 + outer + reduce + inner, (outer, reduce, inner))
    dx = ctx.array(x)
    out = ctx.empty((outer, inner))
    call("tf_sum_dim", ctx.handle, dx.ptr, out.ptr, outer, reduce, inner)
    got = out.numpy()
    if outer > 1 and inner > 1:
        # general path: one thread per output, reduced dim in order = Tensor::sum
        assert_bitexact(got, oracle.sum_dim(x, outer, reduce, inner), "sum_dim (reference order)")
    else:
        assert_close(got, x.astype(np.float64).sum(1), 1e-4, f"sum_dim {outer}x{reduce}x{inner}")


@pytest.mark.parametrize("outer,reduce,inner", [(1, 4096, 1024), (4096, 1024, 1), (8, 513, 257), (2, 1, 3)])
def test_expand_dim_is_sum_backward(ctx, outer, reduce, inner):
    up = synth.normal(920 + outer + inner, (outer, inner))
    dup = ctx.array(up)
    out = ctx.empty((outer, reduce, inner))
    call("tf_expand_dim", ctx.handle, dup.ptr, out.ptr, outer, reduce, inner)
    assert_bitexact(out.numpy(), np.broadcast_to(up[:, None, :], (outer, reduce, inner)), "expand_dim")


# ---------------------------------------------------------------------------
# Tensor::transpose of the last two dims (tensor/Tensor.cpp:579-619)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("batch,rows,cols,dt", [(1, 2049, 3001, "f32"), (3, 130, 67, "bf16"), (2, 65, 64, "i64"),
                                                (1, 1, 1000, "f32"), (1, 4096, 1024, "f32")])
def test_transpose2d(ctx, batch, rows, cols, dt):
    import tensors_amd as ta
    if dt == "f32":
        x, tf, dtype = synth.normal(930 + rows, (batch, rows, cols)), _lib.TF_F32, np.float32
    elif dt == "bf16":
        x, tf, dtype = ta.f32_to_bf16_bits(synth.normal(931, (batch, rows, cols))), _lib.TF_BF16, ta.BF16
    else:
        x = synth.uniform_int(932, (batch, rows, cols), 1 << 30) << 20
        tf, dtype = _lib.TF_I64, np.int64
    dx = ctx.array(x, dtype)
    out = ctx.empty((batch, cols, rows), dtype)
    call("tf_transpose2d", ctx.handle, dx.ptr, out.ptr, batch, rows, cols, tf)
    got = out.numpy()
    want = np.ascontiguousarray(np.swapaxes(x, 1, 2))
    assert_bitexact(got.view(want.dtype) if dt == "bf16" else got, want, f"transpose {dt}")
    oref = np.stack([oracle.transpose2d(x[b]) for b in range(batch)]) if dt == "f32" else None
    if oref is not None:
        assert_bitexact(got, oref, "transpose vs oracle")


# ---------------------------------------------------------------------------
# sub, scale by a device scalar, bf16 -> f32 widening
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n", [4096 * 1024, 1000003, 3])
def test_sub_and_scale_by(ctx, n):
    a, b = synth.normal(940, (n,)), synth.normal(941, (n,))
    da, db, out = ctx.array(a), ctx.array(b), ctx.empty((n,))
    call("tf_sub", ctx.handle, da.ptr, db.ptr, out.ptr, n, _lib.TF_F32)
    assert_bitexact(out.numpy(), (a - b).astype(np.float32), "sub")
    s = np.array([-0.37], np.float32)
    ds = ctx.array(s)
    call("tf_scale_by", ctx.handle, da.ptr, ds.ptr, out.ptr, n, _lib.TF_F32)
    assert_bitexact(out.numpy(), (a * s[0]).astype(np.float32), "scale_by")


@pytest.mark.parametrize("n", [4096 * 1024 + 5, 7])
def test_cast_round_trip(ctx, n):
    import tensors_amd as ta
    x = synth.normal(950, (n,), std=100.0)
    dx = ctx.array(x)
    h = ctx.empty((n,), ta.BF16)
    back = ctx.empty((n,))
    call("tf_cast_f32_bf16", ctx.handle, dx.ptr, h.ptr, n)
    call("tf_cast_bf16_f32", ctx.handle, h.ptr, back.ptr, n)
    bits = h.numpy()
    assert_bitexact(bits, ta.f32_to_bf16_bits(x), "f32 -> bf16")
    assert_bitexact(back.numpy(), oracle.bf16_round(x), "bf16 -> f32 is exact widening")


# ---------------------------------------------------------------------------
# LeakyReLU (cuda/CudaKernelRegistry.hpp:17,24; tensor/Tensor.cpp:303-327)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n", [4096 * 1024, 1001, 4])
@pytest.mark.parametrize("alpha", [0.01, 0.2, 0.0])
def test_leaky_relu_bitexact(ctx, n, alpha):
    from tensors_amd import ops
    x = synth.normal(960 + n, (n,))
    x[:4] = np.array([0.0, -0.0, -1e-45, 3e38], np.float32)[:min(4, n)]
    dx, y = ctx.array(x), ctx.empty((n,))
    ops.leaky_relu(dx, y, alpha)
    assert_bitexact(y.numpy(), oracle.leaky_relu(x, alpha), f"leaky_relu alpha={alpha}")


def test_leaky_relu_bf16(ctx):
    import tensors_amd as ta
    from tensors_amd import ops
    x16 = ta.f32_to_bf16_bits(synth.normal(965, (100003,)))
    dx, y = ctx.array(x16, ta.BF16), ctx.empty((100003,), ta.BF16)
    ops.leaky_relu(dx, y, 0.1)
    want = ta.f32_to_bf16_bits(oracle.leaky_relu(ta.bf16_bits_to_f32(x16), 0.1))
    assert_bitexact(y.numpy(), want, "leaky_relu bf16")


# ---------------------------------------------------------------------------
# argmax (examples/train_mlp.cpp:95-101)
# ---------------------------------------------------------------------------
def _argmax_case(rows, cols, seed):
    x = synth.normal(seed, (rows, cols))
    # ties inside rows (first column must win), equal maxima far apart
    q = np.round(x * 2) / 2
    x[: rows // 3] = q[: rows // 3]
    if rows >= 8 and cols >= 4:
        nan = np.float32(np.nan)
        x[0, :] = -1e30                         # nothing exceeds the start value -> 0
        x[1, :] = nan
        x[1, cols // 2] = 1.0                   # NaNs never win
        x[2, :] = -np.inf
        x[3, :] = -2e30
        x[3, cols - 1] = -1e29                  # the last column wins
        x[4, :] = 0.0
        x[4, ::2] = -0.0                        # -0 / +0 tie: first stays
        x[5, :] = 3.0                           # all equal -> 0
        x[6, :] = -5.0
        x[6, cols - 1] = 7.0
        x[7, 1] = x[7, cols - 1] = 99.0         # first of two maxima
    return x


@pytest.mark.parametrize("rows,cols", [(4096, 1000), (64, 10), (128, 10), (13, 2049), (9, 1001), (8, 4), (3, 1),
                                       (1, 4096)])
def test_argmax_rows_bitexact(ctx, rows, cols):
    from tensors_amd import ops
    x = _argmax_case(rows, cols, 970 + rows + cols)
    labels = synth.uniform_int(971, (rows,), cols)
    want = oracle.argmax_rows(x)
    labels[: rows // 2] = want[: rows // 2]
    dx, pred = ctx.array(x), ctx.empty((rows,), np.int64)
    dl, corr = ctx.array(labels), ctx.empty((1,), np.int64)
    ops.argmax_rows(dx, pred, dl, corr)
    assert_bitexact(pred.numpy(), want, f"argmax {rows}x{cols}")
    assert int(corr.numpy()[0]) == int(np.sum(want == labels))
    ops.argmax_rows(dx, pred)                   # without the count
    assert_bitexact(pred.numpy(), want, "argmax without count")


def test_argmax_rejects_half_a_count(ctx):
    dx, pred = ctx.array(np.zeros((4, 3), np.float32)), ctx.empty((4,), np.int64)
    with pytest.raises(TFError):
        call("tf_argmax_rows", ctx.handle, dx.ptr, pred.ptr, pred.ptr, None, 4, 3)
    corr = ctx.array(np.full(1, 5, np.int64))
    call("tf_argmax_rows", ctx.handle, dx.ptr, pred.ptr, pred.ptr, corr.ptr, 0, 3)
    assert int(corr.numpy()[0]) == 0
