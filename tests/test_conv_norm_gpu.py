"""LayerNorm forward/backward, im2col/col2im and the Conv2d backward built from
them (batched / batch-reduced MFMA GEMMs), against the CPU oracle."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tensors_amd import synth
from tests.conftest import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu
RTOL32 = 1e-4


def _ops():
    from tensors_amd import ops
    return ops


# Backward paths: one launch with per-block column strips (16-byte rows of
# up to 2048 columns: 1024, 64 x 1000 with a partly filled last strip,
# 2048 x 1024 with two rows per wave, 96 x 256 and 1024 x 4 with strips past
# the last column, 256 x 2048, grids of 8k blocks and not); rows cached in
# registers with column partials (odd widths, few rows: 1001, 1, 520, 264,
# 40 x 2048); streamed wide rows (3000).
@pytest.mark.parametrize("R,Cc", [(1024, 1024), (64, 128), (7, 3000), (33, 1001), (1, 1), (300, 2048), (4096, 1024),
                                  (2, 520), (5, 264), (1000, 1536), (64, 1000), (2048, 1024), (96, 256), (1024, 4),
                                  (40, 2048), (256, 2048), (12, 1024)])
def test_layernorm_fwd_bwd(ctx, R, Cc):
    ops = _ops()
    x = synth.normal(201 + Cc, (R, Cc))
    dy = synth.normal(202 + Cc, (R, Cc))
    gamma = synth.normal(203, (Cc,), mean=1.0, std=0.1)
    beta = synth.normal(204, (Cc,))
    y_ref, m_ref, r_ref = oracle.layernorm_fwd(x, gamma, beta)
    dx_, dg_, db_ = ctx.array(x), ctx.array(gamma), ctx.array(beta)
    y, mean, rstd = ctx.empty((R, Cc)), ctx.empty((R,)), ctx.empty((R,))
    ops.layernorm_fwd(dx_, dg_, db_, y, mean, rstd)
    assert_close(y.numpy(), y_ref, RTOL32, "ln fwd")
    assert_close(mean.numpy(), m_ref, RTOL32, "ln mean", atol=1e-6)
    assert_close(rstd.numpy(), r_ref, RTOL32, "ln rstd")
    dx, dgam, dbet = ctx.empty((R, Cc)), ctx.empty((Cc,)), ctx.empty((Cc,))
    ops.layernorm_bwd(ctx.array(dy), dx_, dg_, mean, rstd, dx, dgam, dbet)
    want_dx, want_dg, want_db = oracle.layernorm_bwd(x, dy, gamma, m_ref, r_ref)
    assert_close(dx.numpy(), want_dx, RTOL32, "ln dx")
    assert_close(dgam.numpy(), want_dg, RTOL32, "ln dgamma")
    assert_close(dbet.numpy(), want_db, RTOL32, "ln dbeta")


def test_layernorm_bwd_reference_stub_bitexact(ctx):
    ops = _ops()
    R, Cc = 1024, 1024
    dy = synth.normal(211, (R, Cc))
    gamma = synth.normal(212, (Cc,), mean=1.0, std=0.1)
    dx, dgam, dbet = ctx.empty((R, Cc)), ctx.array(np.ones(Cc, np.float32)), ctx.array(np.ones(Cc, np.float32))
    ops.layernorm_bwd(ctx.array(dy), None, ctx.array(gamma), None, None, dx, dgam, dbet, reference_compat=True)
    want_dx, want_dg, want_db = oracle.layernorm_bwd_stub(dy, gamma)
    assert_bitexact(dx.numpy(), want_dx, "stub dx")
    assert_bitexact(dgam.numpy(), want_dg, "stub dgamma")
    assert_bitexact(dbet.numpy(), want_db, "stub dbeta")


IM2COL_CASES = [
    # N, C, H, W, k, stride, pad, dil
    (2, 3, 8, 8, 3, 1, 1, 1),
    (2, 4, 9, 7, 3, 2, 1, 1),
    (1, 2, 10, 10, 3, 1, 2, 2),
    (3, 1, 5, 6, 1, 1, 0, 1),
    (128, 3, 32, 32, 3, 1, 1, 1),       # C4 conv1
    (16, 32, 32, 32, 3, 2, 1, 1),       # C4 conv2 geometry (reduced batch)
    # >= 256 planes: the LDS plane forms (im2col in row groups, col2im per plane)
    (128, 32, 32, 32, 3, 2, 1, 1),      # C4 conv2 at full size
    (64, 8, 9, 7, 3, 2, 1, 1),          # odd plane, stride 2
    (32, 16, 10, 10, 3, 1, 2, 2),       # dilation 2
    (256, 1, 5, 6, 1, 1, 0, 1),         # 1x1
    (32, 8, 13, 11, 5, 3, 2, 1),        # stride 3, 5x5
    (16, 16, 64, 64, 5, 1, 2, 1),       # im2col in 25 row groups; col2im column chunk too big for LDS
    (2, 128, 130, 130, 3, 1, 1, 1),     # plane too big for LDS: element forms
    (64, 4, 16, 16, 7, 2, 3, 1),        # 7x7 stride 2: col2im plane form with up to 4 x 4 taps per pixel
    (64, 4, 12, 12, 9, 1, 4, 1),        # 9x9 stride 1: col2im plane form, 9 taps per axis (the per-tap loop)
]


@pytest.mark.parametrize("case", IM2COL_CASES)
def test_im2col_bitexact_and_col2im_adjoint(ctx, case):
    ops = _ops()
    N, Cc, H, W, k, s, p, d = case
    x = synth.normal(221 + N * Cc, (N, Cc, H, W))
    col_ref = oracle.im2col(x, k, k, s, s, p, p, d, d)
    col = ctx.empty(col_ref.shape)
    ops.im2col(ctx.array(x), col, k, k, (s, s), (p, p), (d, d))
    assert_bitexact(col.numpy(), col_ref, f"im2col {case}")
    c = synth.normal(222 + N, col_ref.shape)
    dx = ctx.empty(x.shape)
    ops.col2im(ctx.array(c), dx, k, k, (s, s), (p, p), (d, d))
    assert_close(dx.numpy(), oracle.col2im(c, x.shape, k, k, s, s, p, p, d, d), 1e-5, "col2im vs scatter")
    # adjoint: <im2col x, c> == <x, col2im c>
    lhs = float(np.dot(col_ref.astype(np.float64).ravel(), c.astype(np.float64).ravel()))
    rhs = float(np.dot(x.astype(np.float64).ravel(), dx.numpy().astype(np.float64).ravel()))
    assert abs(lhs - rhs) <= 1e-4 * (abs(lhs) + 1.0)


@pytest.mark.parametrize("case", [IM2COL_CASES[0], IM2COL_CASES[1], IM2COL_CASES[6], IM2COL_CASES[8],
                                  IM2COL_CASES[12]])
def test_im2col_col2im_float16(ctx, case):
    # Float16, which the reference's im2col / col2im also take
    # (cuda/kernels/im2col.cu:133-150, col2im.cu:163-185): im2col copies, so
    # bit for bit; col2im sums the taps in fp32 in the element form's order
    # and rounds once to f16 (to nearest even), so within one f16 step of the
    # oracle's fp32 scatter rounded the same way.  Covers the plane forms,
    # the element forms and the strided / dilated maps.
    ops = _ops()
    N, Cc, H, W, k, s, p, d = case
    x16 = oracle.f32_to_f16_bits(synth.normal(231 + N * Cc, (N, Cc, H, W), std=3.0))
    x = oracle.f16_bits_to_f32(x16)
    col_ref = oracle.im2col(x, k, k, s, s, p, p, d, d)
    col = ctx.empty(col_ref.shape, np.float16)
    ops.im2col(ctx.array(x16.view(np.float16)), col, k, k, (s, s), (p, p), (d, d))
    assert_bitexact(col.numpy().view(np.uint16), oracle.f32_to_f16_bits(col_ref), f"f16 im2col {case}")
    c16 = oracle.f32_to_f16_bits(synth.normal(232 + N, col_ref.shape))
    dx = ctx.empty(x.shape, np.float16)
    ops.col2im(ctx.array(c16.view(np.float16)), dx, k, k, (s, s), (p, p), (d, d))
    want = oracle.f16_bits_to_f32(oracle.f32_to_f16_bits(
        oracle.col2im(oracle.f16_bits_to_f32(c16), x.shape, k, k, s, s, p, p, d, d)))
    assert_close(dx.numpy().astype(np.float32), want, 2.0 ** -10, f"f16 col2im {case}")


def _conv_bwd_gpu(ctx, x, w, gout, stride, pad, need_dx=True):
    """Conv2d backward from the C-ABI pieces, as the Conv2dModule backward node runs it."""
    from tensors_amd._lib import TF_EPI_NONE
    ops = _ops()
    N, Cin, H, W = x.shape
    Cout, _, kH, kW = w.shape
    oh, ow = ops.conv_out(H, kH, stride, pad, 1), ops.conv_out(W, kW, stride, pad, 1)
    P, KK = oh * ow, Cin * kH * kW
    dx_, dw_, dg_ = ctx.array(x), ctx.array(w), ctx.array(gout)
    col = ctx.empty((N, KK, P))
    ops.im2col(dx_, col, kH, kW, (stride, stride), (pad, pad))
    gw = ctx.empty((Cout, KK))
    # dW = sum_n dY[n] (Cout x P) @ col[n]^T (P x KK)
    ops.gemm_ex(dg_, col, gw, Cout, KK, P, lda=P, ldb=P, ldc=KK, trans_b=True, stride_a=Cout * P,
                stride_b=KK * P, batch=N, reduce_batch=True, epilogue=TF_EPI_NONE)
    gb = ctx.empty((Cout,))
    ops.chansum_nchw(dg_, gb)
    gin = None
    if need_dx:
        dcol = ctx.empty((N, KK, P))
        # dcol[n] = W^T (KK x Cout) @ dY[n] (Cout x P)
        ops.gemm_ex(dw_, dg_, dcol, KK, P, Cout, lda=KK, ldb=P, ldc=P, trans_a=True, stride_a=0,
                    stride_b=Cout * P, stride_c=KK * P, batch=N)
        gin = ctx.empty(x.shape)
        ops.col2im(dcol, gin, kH, kW, (stride, stride), (pad, pad))
    return gin, gw, gb


CONV_CASES = [(2, 3, 8, 8, 4, 3, 1, 1), (4, 5, 9, 9, 6, 3, 2, 1), (2, 2, 6, 6, 3, 1, 1, 0),
              (8, 3, 32, 32, 32, 3, 1, 1), (4, 32, 32, 32, 64, 3, 2, 1)]


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv2d_backward_vs_reference_loop(ctx, case):
    N, Cin, H, W, Cout, k, s, p = case
    x = synth.normal(231 + N, (N, Cin, H, W))
    w = synth.normal(232 + Cout, (Cout, Cin, k, k), std=0.2)
    oh = (H + 2 * p - k) // s + 1
    gout = synth.normal(233, (N, Cout, oh, oh))
    gin, gw, gb = _conv_bwd_gpu(ctx, x, w, gout, s, p)
    rin, rw, rb = oracle.conv2d_bwd(x, w, gout, (s, s), (p, p), (1, 1))
    assert_close(gin.numpy(), rin, RTOL32, f"conv dX {case}")
    assert_close(gw.numpy().reshape(rw.shape), rw, RTOL32, f"conv dW {case}")
    assert_close(gb.numpy(), rb, RTOL32, f"conv db {case}")


def test_conv2d_backward_golden_1x1(ctx):
    # nn/conv2d_backward_test.cpp:110-160: 1x1 kernel golden values.
    x = np.array([1, 2, 3, 4], np.float32).reshape(1, 1, 2, 2)
    w = np.array([2.0], np.float32).reshape(1, 1, 1, 1)
    gout = np.array([0.1, 0.2, 0.3, 0.4], np.float32).reshape(1, 1, 2, 2)
    gin, gw, gb = _conv_bwd_gpu(ctx, x, w, gout, 1, 0)
    assert_close(gin.numpy().ravel(), [0.2, 0.4, 0.6, 0.8], 1e-6, "golden dX", atol=1e-7)
    assert_close(gw.numpy().ravel(), [3.0], 1e-6, "golden dW", atol=1e-7)
    rin, rw, rb = oracle.conv2d_bwd(x, w, gout, (1, 1), (0, 0), (1, 1))
    assert_close(gin.numpy(), rin, 1e-6, "1x1 dX", atol=1e-7)
    assert_close(gw.numpy().reshape(rw.shape), rw, 1e-6, "1x1 dW", atol=1e-7)
    assert_close(gb.numpy(), rb, 1e-6, "1x1 db", atol=1e-7)


@pytest.mark.parametrize("relu", [False, True])
def test_conv2d_forward_row_bias(ctx, relu):
    from tensors_amd._lib import TF_EPI_ROW_BIAS, TF_EPI_ROW_BIAS_RELU
    ops = _ops()
    N, Cin, H, W, Cout, k, s, p = 4, 3, 16, 16, 8, 3, 1, 1
    x = synth.normal(241, (N, Cin, H, W))
    w = synth.normal(242, (Cout, Cin, k, k), std=0.2)
    b = synth.normal(243, (Cout,))
    P, KK = H * W, Cin * k * k
    col = ctx.empty((N, KK, P))
    ops.im2col(ctx.array(x), col, k, k, (s, s), (p, p))
    y = ctx.empty((N, Cout, H, W))
    ops.gemm_ex(ctx.array(w), col, y, Cout, P, KK, lda=KK, ldb=P, ldc=P, stride_b=KK * P, stride_c=Cout * P,
                batch=N, epilogue=TF_EPI_ROW_BIAS_RELU if relu else TF_EPI_ROW_BIAS, bias=ctx.array(b))
    want = oracle.conv2d_fwd(x, w, b, s, p)
    assert_close(y.numpy(), np.maximum(want, 0) if relu else want, RTOL32, "conv fwd")


IMPLICIT_CASES = [
    # N, C, H, W, Cout, k, stride, pad, dil
    (128, 3, 32, 32, 32, 3, 1, 1, 1),      # C4 conv1
    (128, 32, 32, 32, 64, 3, 2, 1, 1),     # C4 conv2
    (3, 5, 13, 17, 40, 3, 2, 0, 1),        # odd extents, partial pixel tiles and channel block
    (2, 4, 12, 11, 70, 3, 1, 2, 2),        # dilation 2, two channel blocks (64 + 6)
    (2, 6, 19, 23, 8, 5, 3, 2, 1),         # 5 x 5, stride 3
    (4, 7, 9, 9, 3, 1, 1, 0, 1),           # 1 x 1, odd K
    (1, 2, 40, 200, 33, 3, 1, 1, 1),       # output rows wider than a pixel tile
    # few taps with stride, dilation and several 32-channel blocks
    (5, 2, 15, 13, 20, 3, 2, 1, 2),        # K = 18, stride 2, dilation 2, a partial last pixel tile
    (3, 1, 11, 9, 70, 5, 3, 2, 1),         # K = 25, stride 3, three channel blocks (32 + 32 + 6)
    (2, 39, 16, 16, 24, 3, 1, 1, 1),       # K = 351: 11 weight-gradient tiles, the last 3 split in 2 pixel slices
    (2, 60, 8, 8, 20, 3, 1, 1, 1),         # K = 540: 17 weight-gradient tiles, the last one unpaired
]


def _conv_truth(x, w, b, s, p, d, relu):
    """float64 from the bit-exact im2col restatement: y[n] = W @ col[n]."""
    N = x.shape[0]
    Cout, _, kH, kW = w.shape
    col = oracle.im2col(x, kH, kW, s, s, p, p, d, d).astype(np.float64)
    y = np.einsum("ok,nkp->nop", w.reshape(Cout, -1).astype(np.float64), col)
    if b is not None:
        y += b.astype(np.float64)[None, :, None]
    if relu:
        y = np.maximum(y, 0.0)
    H, W = x.shape[2:]
    oh, ow = (H + 2 * p - d * (kH - 1) - 1) // s + 1, (W + 2 * p - d * (kW - 1) - 1) // s + 1
    return y.reshape(N, Cout, oh, ow)


@pytest.mark.parametrize("case", IMPLICIT_CASES)
@pytest.mark.parametrize("bias_relu", [(True, True), (False, False)])
def test_conv2d_fwd_implicit_vs_float64(ctx, case, bias_relu):
    """tf_conv2d_fwd (implicit GEMM: filter rows and input patch in LDS, no
    col buffer) against float64 on the bit-exact im2col restatement."""
    ops = _ops()
    N, C, H, W, Cout, k, s, p, d = case
    use_bias, relu = bias_relu
    x = synth.normal(251 + N + C, (N, C, H, W))
    w = synth.normal(252 + Cout, (Cout, C, k, k), std=0.2)
    b = synth.normal(253, (Cout,)) if use_bias else None
    oh, ow = ops.conv_out(H, k, s, p, d), ops.conv_out(W, k, s, p, d)
    y = ctx.empty((N, Cout, oh, ow))
    ops.conv2d_fwd(ctx.array(x), ctx.array(w), y, ctx.array(b) if b is not None else None, (s, s), (p, p), (d, d),
                   relu)
    assert_close(y.numpy(), _conv_truth(x, w, b, s, p, d, relu), RTOL32, f"implicit conv {case}")


@pytest.mark.parametrize("case", IMPLICIT_CASES)
def test_conv2d_bwd_weight_implicit_vs_float64(ctx, case):
    """tf_conv2d_bwd_weight (implicit GEMM over each block's pixels, then a
    fixed-order sum of the per-block partials) against float64 on the
    bit-exact im2col restatement, with and without the bias gradient it forms
    from the same dy tiles; bit-identical on a second call."""
    ops = _ops()
    N, C, H, W, Cout, k, s, p, d = case
    x = synth.normal(261 + N + C, (N, C, H, W))
    oh, ow = ops.conv_out(H, k, s, p, d), ops.conv_out(W, k, s, p, d)
    gy = synth.normal(262 + Cout, (N, Cout, oh, ow))
    col = oracle.im2col(x, k, k, s, s, p, p, d, d).astype(np.float64)
    want = np.einsum("nop,nkp->ok", gy.astype(np.float64).reshape(N, Cout, -1), col).reshape(Cout, C, k, k)
    dxx, dgy = ctx.array(x), ctx.array(gy)
    gw = ctx.empty((Cout, C, k, k))
    ops.conv2d_bwd_weight(dxx, dgy, gw, (s, s), (p, p), (d, d))
    first = gw.numpy()
    assert_close(first, want, RTOL32, f"implicit dW {case}")
    gb = ctx.array(np.full((Cout,), 7.0, np.float32))
    ops.conv2d_bwd_weight(dxx, dgy, gw, (s, s), (p, p), (d, d), db=gb)
    assert_bitexact(gw.numpy(), first, "second call, with db")
    assert_close(gb.numpy(), gy.astype(np.float64).sum(axis=(0, 2, 3)), RTOL32, f"implicit db {case}")


DX_EXTRA_CASES = [
    # N, C, H, W, Cout, k, stride, pad, dil: phases that no tap reaches
    (2, 3, 9, 10, 5, 1, 2, 0, 1),          # 1 x 1, stride 2: odd rows / columns get nothing
    (2, 4, 11, 12, 6, 3, 2, 1, 2),         # dilation 2 = stride: every tap in one residue class
    (1, 3, 10, 10, 4, 2, 3, 0, 1),         # stride 3 > kernel 2, trailing row beyond the last window
    (3, 70, 8, 8, 16, 3, 1, 1, 1),         # 64 + 6 input channels: two channel blocks
    (1, 2, 40, 200, 8, 3, 1, 1, 1),        # rows wider than a pixel tile (the dy patch holds Cout channels)
    # strided, >= 128 (image, channel group) blocks: dcol per image in LDS, col2im from LDS
    (160, 5, 13, 17, 12, 5, 3, 2, 1),      # 5 x 5, stride 3: 5 channels x 25 taps = 125 dcol rows, 56 pixels
    (128, 3, 9, 10, 5, 1, 2, 0, 1),        # 1 x 1, stride 2: odd rows / columns get nothing
    (64, 40, 12, 11, 70, 3, 2, 2, 2),      # dilation 2, 40 channels in groups of 16, 70 co (two K chunks)
    (128, 2, 20, 21, 6, 9, 2, 4, 1),       # 9 x 9, stride 2: five column taps, the per-element col2im loop
    # strided, two blocks per CU; col2im with at most 2 x 2 taps per pixel
    # (stride-2 3 x 3) or at most 4 x 4 (5 x 5)
    (128, 30, 24, 24, 40, 3, 2, 1, 1),     # 144 pixels, groups 8 + 8 + 8 + 6, filter by plain loads, 40 co
    (130, 32, 16, 16, 24, 3, 2, 1, 1),     # 64 pixels, 24 co (a partly filled K chunk)
    (256, 6, 16, 16, 16, 5, 2, 2, 1),      # 5 x 5: groups of 3 channels (75 dcol rows), up to 3 x 3 taps
]
# The forward cases whose dy patch (Cout channels) fits the LDS.
DX_CASES = [c for c in IMPLICIT_CASES if c[3] <= 64] + DX_EXTRA_CASES


def _dx_truth(gy, w, x_shape, s, p, d):
    """float64 adjoint of the bit-exact im2col map: dcol[n] = W^T dy[n], then
    each col element adds into the input pixel im2col copied it from (found by
    running im2col on the pixel index + 1; 0 marks padding)."""
    N, C, H, W = x_shape
    Cout, _, kH, kW = w.shape
    src = (np.arange(N * C * H * W, dtype=np.float64) + 1).reshape(x_shape).astype(np.float32)
    assert src.size < (1 << 24)                       # exact in float32
    idx = oracle.im2col(src, kH, kW, s, s, p, p, d, d).astype(np.int64)
    dcol = np.einsum("ok,nop->nkp", w.reshape(Cout, -1).astype(np.float64),
                     gy.astype(np.float64).reshape(N, Cout, -1))
    keep = idx > 0
    return np.bincount(idx[keep] - 1, weights=dcol[keep], minlength=N * C * H * W).reshape(x_shape)


@pytest.mark.parametrize("case", DX_CASES)
def test_conv2d_bwd_data_implicit_vs_float64(ctx, case):
    """tf_conv2d_bwd_data (implicit GEMM per sub-pixel phase, or for strided
    layers with enough blocks the column gradient per image in LDS gathered
    from there; no dcol buffer in memory, no col2im launch) against the
    float64 adjoint of the bit-exact im2col map; every dx element is written
    (dx starts as 7.0); bit-identical on a second call."""
    ops = _ops()
    N, C, H, W, Cout, k, s, p, d = case
    oh, ow = ops.conv_out(H, k, s, p, d), ops.conv_out(W, k, s, p, d)
    w = synth.normal(271 + Cout, (Cout, C, k, k), std=0.2)
    gy = synth.normal(272 + N + C, (N, Cout, oh, ow))
    want = _dx_truth(gy, w, (N, C, H, W), s, p, d)
    dw_, dgy = ctx.array(w), ctx.array(gy)
    dx = ctx.array(np.full((N, C, H, W), 7.0, np.float32))
    ops.conv2d_bwd_data(dgy, dw_, dx, (s, s), (p, p), (d, d))
    first = dx.numpy()
    assert_close(first, want, RTOL32, f"implicit dX {case}")
    ops.conv2d_bwd_data(dgy, dw_, dx, (s, s), (p, p), (d, d))
    assert_bitexact(dx.numpy(), first, "second call")


class _Offset:
    """A view of a device array starting one float in (4-byte aligned, not
    16-byte aligned), with `shape` elements."""

    def __init__(self, base, shape):
        self.base = base                   # keeps the allocation alive
        self.ctx, self.shape, self.dtype = base.ctx, tuple(shape), base.dtype
        self.size = int(np.prod(self.shape))
        self.ptr = base.ptr + 4


@pytest.mark.parametrize("case", [(128, 32, 32, 32, 64, 3, 2, 1, 1), (3, 5, 13, 16, 40, 3, 1, 1, 1),
                                  (4, 3, 16, 20, 24, 3, 1, 1, 1), (2, 2, 9, 9, 40, 3, 1, 1, 1)])
def test_conv2d_implicit_unaligned_operands_match_aligned(ctx, case):
    """Operands that are not 16-byte aligned take the scalar staging loads of
    the implicit kernels (forward, weight + bias gradient, both data-gradient
    forms) and the element-wise loads of the streaming weight gradient (the
    last two shapes, K <= 31); the results equal the aligned calls bit for bit (same values,
    same summation order)."""
    ops = _ops()
    N, C, H, W, Cout, k, s, p, d = case
    oh, ow = ops.conv_out(H, k, s, p, d), ops.conv_out(W, k, s, p, d)
    x = synth.normal(281, (N, C, H, W))
    w = synth.normal(282, (Cout, C, k, k), std=0.2)
    gy = synth.normal(283, (N, Cout, oh, ow))
    pad = np.zeros(1, np.float32)

    def both(a):
        return ctx.array(a), _Offset(ctx.array(np.concatenate([pad, a.ravel()])), a.shape)

    (xa, xu), (wa, wu), (ga, gu) = both(x), both(w), both(gy)
    outs = []
    for xx, ww, gg in ((xa, wa, ga), (xu, wu, gu)):
        y = ctx.empty((N, Cout, oh, ow))
        ops.conv2d_fwd(xx, ww, y, None, (s, s), (p, p), (d, d), False)
        gw, gb = ctx.empty((Cout, C, k, k)), ctx.empty((Cout,))
        ops.conv2d_bwd_weight(xx, gg, gw, (s, s), (p, p), (d, d), db=gb)
        gx = ctx.empty((N, C, H, W))
        ops.conv2d_bwd_data(gg, ww, gx, (s, s), (p, p), (d, d))
        outs.append([t.numpy() for t in (y, gw, gb, gx)])
    for name, a, b in zip(("y", "dw", "db", "dx"), outs[0], outs[1]):
        assert_bitexact(b, a, f"unaligned {name} {case}")


def test_conv2d_bwd_data_implicit_reports_unsupported(ctx):
    """Filter columns plus dy patch over 160 KB of LDS: TF_ERR_UNSUPPORTED,
    nothing written (the API then takes the dcol GEMM + col2im)."""
    from tensors_amd._lib import TF_ERR_UNSUPPORTED, TFError
    ops = _ops()
    dy = ctx.zeros((1, 256, 40, 40))
    w = ctx.zeros((256, 64, 3, 3))
    dx = ctx.array(np.full((1, 64, 40, 40), 7.0, np.float32))
    with pytest.raises(TFError) as e:
        ops.conv2d_bwd_data(dy, w, dx, (1, 1), (1, 1))
    assert e.value.status == TF_ERR_UNSUPPORTED
    assert np.all(dx.numpy() == 7.0)


def test_conv2d_fwd_implicit_reports_unsupported(ctx):
    """Filter rows plus input patch over 160 KB of LDS: TF_ERR_UNSUPPORTED,
    nothing written (the API then takes im2col + GEMM)."""
    from tensors_amd._lib import TF_ERR_UNSUPPORTED, TFError
    ops = _ops()
    x = ctx.zeros((1, 64, 70, 70))
    w = ctx.zeros((64, 64, 3, 3))
    y = ctx.array(np.full((1, 64, 70, 70), 7.0, np.float32))
    with pytest.raises(TFError) as e:
        ops.conv2d_fwd(x, w, y, None, (1, 1), (1, 1))
    assert e.value.status == TF_ERR_UNSUPPORTED
    assert np.all(y.numpy() == 7.0)


def test_gemm_row_bias_relu_splitk(ctx):
    from tensors_amd._lib import TF_EPI_ROW_BIAS_RELU
    ops = _ops()
    M, N, K = 40, 24, 9000
    a = synth.normal(251, (M, K))
    b = synth.normal(252, (K, N))
    bias = synth.normal(253, (M,))
    c = ctx.empty((M, N))
    ops.gemm_ex(ctx.array(a), ctx.array(b), c, M, N, K, lda=K, ldb=N, ldc=N, epilogue=TF_EPI_ROW_BIAS_RELU,
                bias=ctx.array(bias))
    want = np.maximum(a.astype(np.float64) @ b.astype(np.float64) + bias[:, None], 0)
    assert_close(c.numpy(), want, RTOL32, "row bias relu split-K")


def test_col2im_checks_out_extent(ctx):
    """tf_col2im takes launch_col2im's outH/outW (cuda/kernels/col2im.cuh:22-29)
    and rejects values that disagree with the geometry."""
    from tensors_amd._lib import TFError, call, TF_F32
    col = ctx.zeros((1, 9, 16))
    dx = ctx.empty((1, 1, 4, 4))
    call("tf_col2im", ctx.handle, col.ptr, dx.ptr, 1, 1, 4, 4, 3, 3, 1, 1, 1, 1, 1, 1, 4, 4, TF_F32)
    with pytest.raises(TFError, match="outH"):
        call("tf_col2im", ctx.handle, col.ptr, dx.ptr, 1, 1, 4, 4, 3, 3, 1, 1, 1, 1, 1, 1, 4, 3, TF_F32)



RELU_CASES = [
    (128, 3, 32, 32, 32, 3, 1, 1, 1),      # C4 conv1
    (128, 32, 32, 32, 64, 3, 2, 1, 1),     # C4 conv2
    (3, 5, 13, 17, 40, 3, 2, 0, 1),        # odd extents: partial pixel tiles and channel block
    (2, 4, 12, 11, 70, 3, 1, 2, 2),        # two channel blocks (64 + 6), dilation 2
    (5, 2, 15, 13, 20, 3, 2, 1, 2),        # slices of one tile over several waves
    (3, 2, 9, 9, 40, 3, 1, 1, 1),          # 81 pixels (not a multiple of 4): element-wise dy, y and dz
]


@pytest.mark.parametrize("case", RELU_CASES)
def test_conv2d_bwd_weight_relu_equals_explicit_relu(ctx, case):
    """tf_conv2d_bwd_weight_relu (the mask y > 0 of a following ReLU applied to
    the staged dy tiles) equals tf_relu_bwd then tf_conv2d_bwd_weight, bit for
    bit: dw, db, and the masked gradient it writes (every element once; the
    buffer starts as 7.0).  y holds exact zeros (about half) and dy negative
    values where y == 0 (ReluBackward's dy * 0 is -0 there)."""
    ops = _ops()
    N, C, H, W, Cout, k, s, p, d = case
    oh, ow = ops.conv_out(H, k, s, p, d), ops.conv_out(W, k, s, p, d)
    x = synth.normal(291, (N, C, H, W))
    y = np.maximum(synth.normal(293, (N, Cout, oh, ow)), np.float32(0.0))
    gy = synth.normal(294, (N, Cout, oh, ow))
    dx_, dy_, gy_ = ctx.array(x), ctx.array(y), ctx.array(gy)
    dz = ctx.empty((N, Cout, oh, ow))
    ops.relu_bwd(gy_, dy_, dz)
    want_w, want_b = ctx.empty((Cout, C, k, k)), ctx.empty((Cout,))
    ops.conv2d_bwd_weight(dx_, dz, want_w, (s, s), (p, p), (d, d), db=want_b)
    got_w, got_b = ctx.empty((Cout, C, k, k)), ctx.empty((Cout,))
    got_z = ctx.array(np.full((N, Cout, oh, ow), 7.0, np.float32))
    ops.conv2d_bwd_weight(dx_, gy_, got_w, (s, s), (p, p), (d, d), db=got_b, relu_y=dy_, dz=got_z)
    assert_bitexact(got_w.numpy(), want_w.numpy(), f"dw with ReLU mask {case}")
    assert_bitexact(got_b.numpy(), want_b.numpy(), f"db with ReLU mask {case}")
    assert_bitexact(got_z.numpy(), dz.numpy(), f"masked gradient {case}")
    # Without dz and without db: the same dw.
    got_w2 = ctx.empty((Cout, C, k, k))
    ops.conv2d_bwd_weight(dx_, gy_, got_w2, (s, s), (p, p), (d, d), relu_y=dy_)
    assert_bitexact(got_w2.numpy(), want_w.numpy(), f"dw with ReLU mask, no db {case}")
