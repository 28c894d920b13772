"""Parity of every hot-path kernel against the CPU oracle, through the C ABI.

Bars: integer/index work and kernels whose arithmetic order equals the
reference's (ReLU backward, add/mul, SGD) are bit-exact; floating-point
reductions are within rtol 1e-4 (fp32) / 2e-2 (bf16) of float64 truth with
atol = rtol * rms(truth).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tensors_amd import synth
from tests.conftest import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu

RTOL32 = 1e-4
RTOL16 = 2e-2


def _ops():
    from tensors_amd import ops
    return ops


# ---------------------------------------------------------------------------
# runtime
# ---------------------------------------------------------------------------
def test_memcpy_roundtrip_and_fill(ctx):
    x = synth.normal(1, (1000, 3))
    d = ctx.array(x)
    assert_bitexact(d.numpy(), x, "H2D/D2H round trip")
    from tensors_amd._lib import call
    call("tf_hip_fill_f32", ctx.handle, d.ptr, 2.5, 2999)
    got = d.numpy().reshape(-1)
    assert np.all(got[:2999] == 2.5) and got[2999] == x.reshape(-1)[2999]
    z = ctx.zeros((37,), np.float32)
    assert np.all(z.numpy() == 0)
    r, u = ctx.pool_stats()
    assert r >= u > 0


def test_block_cache_reuse_and_errors(ctx):
    import ctypes as C
    from tensors_amd._lib import TFError, call
    def alloc(n):
        p = C.c_void_p()
        call("tf_hip_alloc", ctx.handle, n, C.byref(p))
        return p.value
    a = alloc(3000)                  # size class 3072
    call("tf_hip_free", ctx.handle, a)
    assert alloc(3001) == a          # same class: the cached block comes back
    b = alloc(3 << 20)               # 4 MB class
    call("tf_hip_free", ctx.handle, b)
    c = alloc(5 << 20)               # 6 MB class: not the cached 4 MB block
    assert c != b
    with pytest.raises(TFError):
        call("tf_hip_free", ctx.handle, b)   # already freed (it sits in the cache)
    call("tf_hip_free", ctx.handle, c)
    call("tf_hip_free", ctx.handle, a)
    call("tf_hip_trim", ctx.handle, 0)       # hands the cache back to the pool
    d = alloc(1 << 20)
    x = np.arange(1 << 18, dtype=np.float32)
    from tensors_amd import _lib
    call("tf_hip_memcpy", ctx.handle, d, x.ctypes.data, x.nbytes, _lib.TF_COPY_H2D)
    y = np.empty_like(x)
    call("tf_hip_memcpy", ctx.handle, y.ctypes.data, d, x.nbytes, _lib.TF_COPY_D2H)
    assert_bitexact(y, x, "round trip through a block after trim")
    call("tf_hip_free", ctx.handle, d)


def test_zero_size_alloc_and_event_timing(ctx):
    e = ctx.empty((0,), np.float32)
    assert e.ptr is not None            # zero bytes allocates 1 byte
    a, b = ctx.event(), ctx.event()
    a.record()
    b.record()
    assert b is not None and a.elapsed_ms(b) >= 0.0


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------
def _gemm_truth(a, b, ta, tb, alpha=1.0, beta=0.0, c0=None, bias=None, relu=False):
    A = a.astype(np.float64).T if ta else a.astype(np.float64)
    B = b.astype(np.float64).T if tb else b.astype(np.float64)
    out = alpha * (A @ B)
    if beta != 0.0:
        out += beta * c0.astype(np.float64)
    if bias is not None:
        out += bias.astype(np.float64)[None, :]
    if relu:
        out = np.maximum(out, 0.0)
    return out


def _run_gemm(ctx, a, b, ta, tb, M, N, **kw):
    ops = _ops()
    da, db = ctx.array(a), ctx.array(b)
    c0 = kw.pop("c0", None)
    dc = ctx.array(c0) if c0 is not None else ctx.zeros((M, N), np.float32)
    bias = kw.pop("bias", None)
    dbias = ctx.array(bias) if bias is not None else None
    ops.gemm(da, db, dc, trans_a=ta, trans_b=tb, bias=dbias, **kw)
    return dc.numpy()


def test_gemm_known_answers(ctx):
    # autograd/ops/autograd_all_ops_test.cpp:281-328: arange A[2x3] @ B[3x2]
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    b = np.arange(6, dtype=np.float32).reshape(3, 2)
    got = _run_gemm(ctx, a, b, False, False, 2, 2)
    assert np.array_equal(got, np.array([[10, 13], [28, 40]], np.float32))
    # cuda/kernels/gemm_optimized_test.cpp:109-125: [[1,2],[3,4]] @ [[5,6],[7,8]]
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[5, 6], [7, 8]], np.float32)
    assert np.array_equal(_run_gemm(ctx, a, b, False, False, 2, 2), np.array([[19, 22], [43, 50]], np.float32))


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", [(64, 256, 784), (17, 19, 23), (128, 128, 128), (300, 200, 100),
                                   (1, 1, 1), (129, 257, 65), (64, 10, 128), (256, 784, 64)])
def test_gemm_layouts_vs_truth(ctx, ta, tb, M, N, K):
    rng_seed = synth.seed(2, 7) + M * 131 + N * 17 + K
    a = synth.normal(rng_seed, (K, M) if ta else (M, K))
    b = synth.normal(rng_seed + 1, (N, K) if tb else (K, N))
    got = _run_gemm(ctx, a, b, ta, tb, M, N)
    assert_close(got, _gemm_truth(a, b, ta, tb), RTOL32, f"gemm ta={ta} tb={tb} {M}x{N}x{K}")


def test_gemm_matches_reference_order_oracle(ctx):
    # The oracle reproduces Tensor::matmul's sequential loop; the MFMA kernel
    # sums in another order, so the bar is the fp32 tolerance, not bits.
    a = synth.normal(11, (64, 784))
    b = synth.normal(12, (784, 256))
    got = _run_gemm(ctx, a, b, False, False, 64, 256)
    assert_close(got, oracle.matmul(a, b), RTOL32, "gemm vs ref-order oracle")


def test_gemm_splitk_long_k(ctx):
    # C4's classifier: [128 x 16384] @ [16384 x 10] (the narrow-output kernel's k chunks).
    a = synth.normal(21, (128, 16384))
    w = synth.normal(22, (10, 16384))
    got = _run_gemm(ctx, a, w, False, True, 128, 10)
    assert_close(got, _gemm_truth(a, w, False, True), RTOL32, "split-K gemm")


@pytest.mark.parametrize("M,N,K", [(128, 10, 16384), (13, 1, 2051), (64, 16, 4096), (8, 7, 2048), (300, 3, 9001),
                                   (100, 10, 4100), (64, 10, 128)])
def test_gemm_narrow_output_long_k(ctx, M, N, K):
    """Outputs of at most 16 columns over K >= 2048 (A row-major, B as
    [N x K]): the MFMA narrow-output kernel when K % 4 == 0 (128 x 10 x
    16384, 64 x 16 x 4096, 8 x 7 x 2048, 100 x 10 x 4100: a ragged last
    512-deep chunk and a row count off the 16-row groups, and config 1's last
    layer 64 x 10 x 128: one chunk, no partials), the
    butterfly form otherwise (13 x 1 x 2051, 300 x 3 x 9001: ragged 1024-deep
    chunks, rows off its 8-row groups); bias and bias + ReLU; bit-identical on
    a second call (each row group's arrival counter back at zero)."""
    ops = _ops()
    seed = synth.seed(2, 11) + M + N + K
    a = synth.normal(seed, (M, K))
    w = synth.normal(seed + 1, (N, K))
    bias = synth.normal(seed + 2, (N,))
    da, dw, db = ctx.array(a), ctx.array(w), ctx.array(bias)
    c = ctx.empty((M, N))
    ops.gemm(da, dw, c, trans_b=True, bias=db)
    first = c.numpy()
    assert_close(first, _gemm_truth(a, w, False, True, bias=bias), RTOL32, f"narrow gemm {M}x{N}x{K}")
    ops.gemm(da, dw, c, trans_b=True, bias=db)
    assert_bitexact(c.numpy(), first, f"narrow gemm {M}x{N}x{K} repeat")
    ops.gemm(da, dw, c, trans_b=True, bias=db, relu=True, alpha=0.5)
    assert_close(c.numpy(), _gemm_truth(a, w, False, True, alpha=0.5, bias=bias, relu=True), RTOL32,
                 f"narrow gemm {M}x{N}x{K} bias+relu")


@pytest.mark.parametrize("M,N,K", [(128, 16384, 10), (200, 300, 7), (64, 1024, 32), (256, 257, 1), (77, 1027, 32),
                                   (300, 2049, 5)])
def test_gemm_short_k_wide_output(ctx, M, N, K):
    """K <= 32 and at least 256 output columns (A and B row-major: a
    classifier's data gradient), with a bias, against float64."""
    seed = synth.seed(2, 12) + M + N + K
    a = synth.normal(seed, (M, K))
    b = synth.normal(seed + 1, (K, N))
    bias = synth.normal(seed + 2, (N,))
    got = _run_gemm(ctx, a, b, False, False, M, N, bias=bias)
    assert_close(got, _gemm_truth(a, b, False, False, bias=bias), RTOL32, f"short-K gemm {M}x{N}x{K}")


def test_gemm_epilogues(ctx):
    M, N, K = 96, 200, 150
    a = synth.normal(31, (M, K))
    b = synth.normal(32, (K, N))
    c0 = synth.normal(33, (M, N))
    bias = synth.normal(34, (N,))
    got = _run_gemm(ctx, a, b, False, False, M, N, alpha=0.5, beta=0.25, c0=c0)
    assert_close(got, _gemm_truth(a, b, False, False, 0.5, 0.25, c0), RTOL32, "alpha/beta")
    got = _run_gemm(ctx, a, b, False, False, M, N, bias=bias, relu=True)
    assert_close(got, _gemm_truth(a, b, False, False, bias=bias, relu=True), RTOL32, "bias+relu")
    # K == 0: C = beta*C + bias
    z = np.zeros((M, 0), np.float32)
    got = _run_gemm(ctx, z, np.zeros((0, N), np.float32), False, False, M, N, bias=bias)
    assert_close(got, np.broadcast_to(bias, (M, N)), RTOL32, "K=0")


@pytest.mark.parametrize("ta,tb", [(False, True), (True, False), (False, False)])
@pytest.mark.parametrize("M,N,K", [(33, 65, 2048), (31, 1, 1000), (128, 1024, 1024), (64, 256, 784), (5, 7, 129)])
def test_gemm_small_path_repeatable(ctx, ta, tb, M, N, K):
    """Products of the small fp32 path (32 x 32 tiles, K over up to 32 chunk
    groups whose partials the tile's last-arriving block adds in chunk
    order): within fp32 tolerance of float64, and bit-identical across calls
    interleaved with another product that reuses the tiles' arrival counters
    (each tile's counter must be back at zero after every call)."""
    ops = _ops()
    seed = synth.seed(2, 9) + M + N + K
    a = synth.normal(seed, (K, M) if ta else (M, K))
    b = synth.normal(seed + 1, (N, K) if tb else (K, N))
    o = synth.normal(seed + 2, (48, 700))
    da, db, dc = ctx.array(a), ctx.array(b), ctx.empty((M, N))
    do, dw, dz = ctx.array(o), ctx.array(synth.normal(seed + 3, (700, 96))), ctx.empty((48, 96))
    outs = []
    for _ in range(3):
        ops.gemm(da, db, dc, trans_a=ta, trans_b=tb)
        outs.append(dc.numpy())
        ops.gemm(do, dw, dz)
    assert_close(outs[0], _gemm_truth(a, b, ta, tb), RTOL32, f"small gemm {M}x{N}x{K}")
    for r in (1, 2):
        assert_bitexact(outs[r], outs[0], f"call {r} vs call 0")
    assert_close(dz.numpy(), _gemm_truth(o, synth.normal(seed + 3, (700, 96)), False, False), RTOL32, "other")


def test_gemm_splitk_with_epilogue(ctx):
    # 64 x 320 over K = 8192: too large for the small path, few tiles, so
    # split-K with the bias and ReLU applied by the reduction.
    a = synth.normal(41, (64, 8192))
    b = synth.normal(42, (8192, 320))
    bias = synth.normal(43, (320,))
    got = _run_gemm(ctx, a, b, False, False, 64, 320, bias=bias, relu=True)
    assert_close(got, _gemm_truth(a, b, False, False, bias=bias, relu=True), RTOL32, "split-K + bias/relu")


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False)])
def test_gemm_bf16_fp32_accumulate(ctx, ta, tb):
    import tensors_amd as ta_mod
    from tensors_amd import ops
    M, N, K = 192, 160, 320
    a32 = synth.normal(51, (K, M) if ta else (M, K))
    b32 = synth.normal(52, (N, K) if tb else (K, N))
    a16, b16 = ta_mod.f32_to_bf16_bits(a32), ta_mod.f32_to_bf16_bits(b32)
    truth = _gemm_truth(ta_mod.bf16_bits_to_f32(a16), ta_mod.bf16_bits_to_f32(b16), ta, tb)
    da, db = ctx.array(a16, ta_mod.BF16), ctx.array(b16, ta_mod.BF16)
    dc = ctx.zeros((M, N), np.float32)
    ops.gemm(da, db, dc, trans_a=ta, trans_b=tb)
    assert_close(dc.numpy(), truth, RTOL32, "bf16 in / fp32 out")   # exact products, fp32 sums
    dc16 = ctx.zeros((M, N), ta_mod.BF16)
    ops.gemm(da, db, dc16, trans_a=ta, trans_b=tb)
    assert_close(ta_mod.bf16_bits_to_f32(dc16.numpy()), truth, RTOL16, "bf16 in / bf16 out")


# Shapes that select the 256 x 256 bf16 kernel: all-interior tiles; ragged
# M/N edges with K a multiple of 64 (interior + guarded tiles in one grid);
# ragged K (every tile guarded); few tiles with K split over 4 slices.
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", [(4096, 4096, 384), (4000, 4100, 256), (3900, 4352, 200), (2048, 2048, 2048),
                                   (2048, 1000, 4096)])
def test_gemm_bf16_large_tile(ctx, ta, tb, M, N, K):
    import tensors_amd as ta_mod
    from tensors_amd import ops
    seed = synth.seed(2, 9) + M + N + K
    a16 = ta_mod.f32_to_bf16_bits(synth.normal(seed, (K, M) if ta else (M, K)))
    b16 = ta_mod.f32_to_bf16_bits(synth.normal(seed + 1, (N, K) if tb else (K, N)))
    truth = _gemm_truth(ta_mod.bf16_bits_to_f32(a16), ta_mod.bf16_bits_to_f32(b16), ta, tb)
    da, db = ctx.array(a16, ta_mod.BF16), ctx.array(b16, ta_mod.BF16)
    dc = ctx.zeros((M, N), np.float32)
    ops.gemm(da, db, dc, trans_a=ta, trans_b=tb)
    assert_close(dc.numpy(), truth, RTOL32, f"bf16 256-tile ta={ta} tb={tb} {M}x{N}x{K}")


def test_gemm_bf16_large_tile_epilogues(ctx):
    import tensors_amd as ta_mod
    from tensors_amd import ops
    M, N, K = 4096, 4000, 320
    a16 = ta_mod.f32_to_bf16_bits(synth.normal(71, (M, K)))
    b16 = ta_mod.f32_to_bf16_bits(synth.normal(72, (N, K)))
    a, b = ta_mod.bf16_bits_to_f32(a16), ta_mod.bf16_bits_to_f32(b16)
    bias = synth.normal(73, (N,))
    c0 = synth.normal(74, (M, N))
    da, db, dbias = ctx.array(a16, ta_mod.BF16), ctx.array(b16, ta_mod.BF16), ctx.array(bias)
    # bf16 output with bias + ReLU (Linear forward in bf16 compute)
    dc16 = ctx.zeros((M, N), ta_mod.BF16)
    ops.gemm(da, db, dc16, trans_a=False, trans_b=True, bias=dbias, relu=True)
    truth = _gemm_truth(a, b, False, True, bias=bias, relu=True)
    assert_close(ta_mod.bf16_bits_to_f32(dc16.numpy()), truth, RTOL16, "bf16 out, bias+relu")
    # fp32 output with alpha / beta
    dc = ctx.array(c0)
    ops.gemm(da, db, dc, trans_a=False, trans_b=True, alpha=0.5, beta=0.25)
    assert_close(dc.numpy(), _gemm_truth(a, b, False, True, 0.5, 0.25, c0), RTOL32, "alpha/beta")


# Shapes that select the fp32 128 x 128 tiles with the direct-to-LDS kernel:
# all-interior tiles; ragged M/N that are multiples of 4 (partial tiles in the
# direct kernel); ragged M/N that are not (the register-staged kernel takes
# the edge tiles of MN-major operands); K not a multiple of 32 (no direct
# path).
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", [(2048, 2048, 2048), (2000, 2100, 256), (2046, 2050, 96), (2048, 2304, 200)])
def test_gemm_f32_large_tile(ctx, ta, tb, M, N, K):
    seed = synth.seed(2, 10) + M + N + K
    a = synth.normal(seed, (K, M) if ta else (M, K))
    b = synth.normal(seed + 1, (N, K) if tb else (K, N))
    got = _run_gemm(ctx, a, b, ta, tb, M, N)
    assert_close(got, _gemm_truth(a, b, ta, tb), RTOL32, f"fp32 128-tile ta={ta} tb={tb} {M}x{N}x{K}")


def test_gemm_f32_large_tile_epilogues(ctx):
    M, N, K = 2048, 2176, 64
    a = synth.normal(81, (M, K))
    b = synth.normal(82, (N, K))
    bias = synth.normal(83, (N,))
    c0 = synth.normal(84, (M, N))
    got = _run_gemm(ctx, a, b, False, True, M, N, bias=bias, relu=True)
    assert_close(got, _gemm_truth(a, b, False, True, bias=bias, relu=True), RTOL32, "fp32 128-tile bias+relu")
    got = _run_gemm(ctx, a, b, False, True, M, N, alpha=0.5, beta=0.25, c0=c0)
    assert_close(got, _gemm_truth(a, b, False, True, 0.5, 0.25, c0), RTOL32, "fp32 128-tile alpha/beta")


# Every epilogue form the large-tile kernels compile separately (copy, alpha,
# bias, bias + ReLU, ReLU alone) with fp32 and bf16 outputs, on shapes whose
# blocks are all interior (the staged whole-row store path), split over K
# (split-K partials), and ragged (the bounds-checked path).  The product is
# computed once per shape in float64; each form is applied to it.
_EPI_FORMS = [("plain", 1.0, False, False), ("alpha", 0.75, False, False), ("bias", 1.0, True, False),
              ("bias_relu", 1.0, True, True), ("relu", 1.0, False, True), ("alpha_bias_relu", -1.5, True, True)]


@pytest.mark.parametrize("dt,M,N,K,ta,tb", [
    ("f32", 2048, 2048, 128, False, True), ("f32", 2048, 2048, 96, True, False), ("f32", 512, 512, 8192, False, False),
    ("f32", 2000, 2052, 96, False, True),
    ("bf16", 4096, 4096, 256, False, True), ("bf16", 4096, 4096, 192, True, False),
    ("bf16", 1024, 1024, 8192, False, False), ("bf16", 3900, 4100, 128, False, True)])
def test_gemm_large_tile_epilogue_forms(ctx, dt, M, N, K, ta, tb):
    import tensors_amd as ta_mod
    from tensors_amd import ops
    seed = synth.seed(2, 30) + M + K
    a = synth.normal(seed, (K, M) if ta else (M, K))
    b = synth.normal(seed + 1, (N, K) if tb else (K, N))
    if dt == "bf16":
        a16, b16 = ta_mod.f32_to_bf16_bits(a), ta_mod.f32_to_bf16_bits(b)
        a, b = ta_mod.bf16_bits_to_f32(a16), ta_mod.bf16_bits_to_f32(b16)
        da, db = ctx.array(a16, ta_mod.BF16), ctx.array(b16, ta_mod.BF16)
    else:
        da, db = ctx.array(a), ctx.array(b)
    prod = _gemm_truth(a, b, ta, tb)
    bias = synth.normal(seed + 2, (N,))
    dbias = ctx.array(bias)
    for name, alpha, use_bias, relu in _EPI_FORMS:
        want = alpha * prod + (bias.astype(np.float64) if use_bias else 0.0)
        if relu:
            want = np.maximum(want, 0.0)
        for out in ("f32", "bf16"):
            dc = ctx.zeros((M, N), np.float32 if out == "f32" else ta_mod.BF16)
            ops.gemm(da, db, dc, trans_a=ta, trans_b=tb, alpha=alpha, bias=dbias if use_bias else None, relu=relu)
            got = dc.numpy() if out == "f32" else ta_mod.bf16_bits_to_f32(dc.numpy())
            tol = RTOL16 if (dt == "bf16" or out == "bf16") else RTOL32
            assert_close(got, want, tol, f"{dt} in, {out} out, {name}, {M}x{N}x{K} ta={ta} tb={tb}")


def _row_bias_truth(a, b, ta, tb, bias, relu):
    out = _gemm_truth(a, b, ta, tb) + bias.astype(np.float64)[:, None]
    return np.maximum(out, 0.0) if relu else out


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_gemm_large_tile_row_bias(ctx, dt):
    # Row-bias epilogue (conv-forward form) on the large-tile kernels: the
    # fp32 direct kernel, and the general copy path of the 256 x 256 bf16
    # kernel with bf16 and fp32 output; ragged N for the edge tiles.
    import tensors_amd as ta_mod
    from tensors_amd import ops
    from tensors_amd._lib import TF_EPI_ROW_BIAS_RELU
    M, N, K = (2048, 2052, 128) if dt == "f32" else (4096, 4100, 128)
    a = synth.normal(101, (M, K))
    b = synth.normal(102, (N, K))
    bias = synth.normal(103, (M,))
    if dt == "bf16":
        a16, b16 = ta_mod.f32_to_bf16_bits(a), ta_mod.f32_to_bf16_bits(b)
        a, b = ta_mod.bf16_bits_to_f32(a16), ta_mod.bf16_bits_to_f32(b16)
        da, db = ctx.array(a16, ta_mod.BF16), ctx.array(b16, ta_mod.BF16)
        outs = [np.float32, ta_mod.BF16]
    else:
        da, db = ctx.array(a), ctx.array(b)
        outs = [np.float32]
    dbias = ctx.array(bias)
    truth = _row_bias_truth(a, b, False, True, bias, True)
    for odt in outs:
        dc = ctx.zeros((M, N), odt)
        ops.gemm_ex(da, db, dc, M, N, K, lda=K, ldb=K, ldc=N, trans_b=True, epilogue=TF_EPI_ROW_BIAS_RELU,
                    bias=dbias)
        f32_out = odt is np.float32
        got = dc.numpy() if f32_out else ta_mod.bf16_bits_to_f32(dc.numpy())
        assert_close(got, truth, RTOL32 if f32_out else RTOL16,
                     f"{dt} in, {'fp32' if f32_out else 'bf16'} out, row bias + relu")


def test_gemm_bf16_large_tile_beta_split(ctx):
    # alpha / beta with an fp32 C on the 256 x 256 kernel when K is split
    # (few tiles, long K): partial sums, then the reduction's epilogue.
    import tensors_amd as ta_mod
    from tensors_amd import ops
    M, N, K = 512, 512, 8192
    a16 = ta_mod.f32_to_bf16_bits(synth.normal(111, (M, K)))
    b16 = ta_mod.f32_to_bf16_bits(synth.normal(112, (K, N)))
    a, b = ta_mod.bf16_bits_to_f32(a16), ta_mod.bf16_bits_to_f32(b16)
    c0 = synth.normal(113, (M, N))
    dc = ctx.array(c0)
    ops.gemm(ctx.array(a16, ta_mod.BF16), ctx.array(b16, ta_mod.BF16), dc, alpha=0.5, beta=0.25)
    assert_close(dc.numpy(), _gemm_truth(a, b, False, False, 0.5, 0.25, c0), RTOL32, "bf16 split-K alpha/beta")


def test_gemm_f32_large_tile_reduce_batch(ctx):
    # C = sum_b A_b^T B_b (weight-gradient form) with 128 x 128 tiles.
    from tensors_amd import ops
    nb, M, N, K = 3, 2048, 2048, 96
    a = synth.normal(91, (nb, K, M))
    b = synth.normal(92, (nb, K, N))
    da, db = ctx.array(a), ctx.array(b)
    dc = ctx.zeros((M, N))
    ops.gemm_ex(da, db, dc, M, N, K, lda=M, ldb=N, ldc=N, trans_a=True, stride_a=K * M, stride_b=K * N,
                batch=nb, reduce_batch=True)
    truth = np.einsum("bkm,bkn->mn", a.astype(np.float64), b.astype(np.float64))
    assert_close(dc.numpy(), truth, RTOL32, "fp32 128-tile batch reduction")


@pytest.mark.parametrize("dt,nb,M,N,K", [("bf16", 3, 4096, 4096, 128), ("f32", 8, 512, 512, 96),
                                         ("bf16", 8, 512, 512, 128), ("f32", 5, 256, 384, 64)])
def test_gemm_reduce_batch_walk(ctx, dt, nb, M, N, K):
    # C = sum_b A_b^T B_b through the direct kernels' k-block walk: the walk
    # crosses batch elements (wraps) and, where few tiles make the GEMM split
    # over K, starts and ends inside an element.
    import tensors_amd as ta_mod
    from tensors_amd import ops
    a = synth.normal(231 + nb, (nb, K, M))
    b = synth.normal(232 + nb, (nb, K, N))
    if dt == "bf16":
        a16, b16 = ta_mod.f32_to_bf16_bits(a), ta_mod.f32_to_bf16_bits(b)
        a, b = ta_mod.bf16_bits_to_f32(a16), ta_mod.bf16_bits_to_f32(b16)
        da, db = ctx.array(a16, ta_mod.BF16), ctx.array(b16, ta_mod.BF16)
    else:
        da, db = ctx.array(a), ctx.array(b)
    dc = ctx.zeros((M, N))
    ops.gemm_ex(da, db, dc, M, N, K, lda=M, ldb=N, ldc=N, trans_a=True, stride_a=K * M, stride_b=K * N,
                batch=nb, reduce_batch=True)
    truth = np.einsum("bkm,bkn->mn", a.astype(np.float64), b.astype(np.float64))
    assert_close(dc.numpy(), truth, RTOL16 if dt == "bf16" else RTOL32, f"{dt} batch reduction {nb}x{M}x{N}x{K}")


@pytest.mark.parametrize("ta,tb,nb,M,N,K,pad", [
    (False, False, 1, 4096, 4096, 1000, 0),   # last 32-deep block holds 8 of K
    (False, True, 1, 4096, 2048, 968, 8),     # whole last block past K; split in two; padded rows
    (True, False, 1, 4096, 4096, 200, 0),
    (True, True, 1, 4096, 4096, 8, 0),        # one 64-deep block, 56 of it masked
    (True, False, 3, 4096, 4096, 200, 0),     # batch reduction: the walk wraps after a partial block
    (False, False, 2, 2048, 2048, 1000, 8),   # batch reduction split over K, slices start mid-element
])
def test_gemm_bf16_direct_k_tail(ctx, ta, tb, nb, M, N, K, pad):
    # K % 64 != 0 on the direct large-tile kernel: the loads of k >= K must
    # read zero.  Past K lie the padding of K-major rows (random here), the
    # next row, or the next batch element, so a leak changes the result.
    import tensors_amd as ta_mod
    from tensors_amd import ops
    lda = (M if ta else K) + pad
    ldb = (K if tb else N) + pad
    a_shape = (nb, K, lda) if ta else (nb, M, lda)
    b_shape = (nb, N, ldb) if tb else (nb, K, ldb)
    a16 = ta_mod.f32_to_bf16_bits(synth.normal(241 + K, a_shape))
    b16 = ta_mod.f32_to_bf16_bits(synth.normal(242 + K, b_shape))
    a, b = ta_mod.bf16_bits_to_f32(a16), ta_mod.bf16_bits_to_f32(b16)
    dc = ctx.zeros((M, N))
    ops.gemm_ex(ctx.array(a16, ta_mod.BF16), ctx.array(b16, ta_mod.BF16), dc, M, N, K, lda=lda, ldb=ldb, ldc=N,
                trans_a=ta, trans_b=tb, stride_a=a_shape[1] * lda, stride_b=b_shape[1] * ldb, batch=nb,
                reduce_batch=nb > 1)
    truth = np.zeros((M, N))
    for e in range(nb):
        ae = a[e][:, :M] if ta else a[e][:, :K]
        be = b[e][:, :K] if tb else b[e][:, :N]
        truth += _gemm_truth(ae, be, ta, tb)
    assert_close(dc.numpy(), truth, RTOL16, f"bf16 K tail ta={ta} tb={tb} {nb}x{M}x{N}x{K} pad={pad}")


@pytest.mark.parametrize("M,N,K,nb,shared_a,epi,out_bf16,beta", [
    (32, 1024, 27, 4, True, "row_bias_relu", False, 0.0),   # convolution over 3 channels, 3x3
    (64, 300, 32, 2, False, "bias", False, 0.0),            # ragged N, column bias, A per element
    (1, 256, 1, 1, True, "none", False, 0.0),
    (17, 777, 9, 3, True, "relu", True, 0.0),               # bf16 output
    (8, 512, 16, 2, False, "none", False, 0.5),             # beta * C
    (64, 4096, 32, 1, True, "row_bias", False, 0.0),
])
def test_gemm_f32_short_k(ctx, M, N, K, nb, shared_a, epi, out_bf16, beta):
    # K <= 32, M <= 64, N >= 256, A K-major, B MN-major: the VALU path.
    import tensors_amd as ta_mod
    from tensors_amd import ops
    from tensors_amd._lib import TF_EPI_BIAS, TF_EPI_NONE, TF_EPI_RELU, TF_EPI_ROW_BIAS, TF_EPI_ROW_BIAS_RELU
    codes = {"none": TF_EPI_NONE, "bias": TF_EPI_BIAS, "relu": TF_EPI_RELU, "row_bias": TF_EPI_ROW_BIAS,
             "row_bias_relu": TF_EPI_ROW_BIAS_RELU}
    a = synth.normal(261 + K, (1 if shared_a else nb, M, K))
    b = synth.normal(262 + K, (nb, K, N))
    c0 = synth.normal(263 + K, (nb, M, N))
    bias = synth.normal(264 + K, (M if epi.startswith("row") else N,))
    dc = ctx.empty((nb, M, N), ta_mod.BF16) if out_bf16 else ctx.array(c0)
    ops.gemm_ex(ctx.array(a), ctx.array(b), dc, M, N, K, lda=K, ldb=N, ldc=N, stride_a=0 if shared_a else M * K,
                stride_b=K * N, stride_c=M * N, batch=nb, beta=beta, epilogue=codes[epi],
                bias=ctx.array(bias) if epi in ("bias", "row_bias", "row_bias_relu") else None)
    truth = np.einsum("bmk,bkn->bmn", np.broadcast_to(a, (nb, M, K)).astype(np.float64), b.astype(np.float64))
    truth += beta * c0.astype(np.float64)
    if epi == "bias":
        truth += bias.astype(np.float64)[None, None, :]
    if epi.startswith("row"):
        truth += bias.astype(np.float64)[None, :, None]
    if epi in ("relu", "row_bias_relu"):
        truth = np.maximum(truth, 0.0)
    got = ta_mod.bf16_bits_to_f32(dc.numpy()) if out_bf16 else dc.numpy()
    assert_close(got, truth, RTOL16 if out_bf16 else RTOL32, f"short-K GEMM {M}x{N}x{K} b{nb} {epi}")


def test_gemm_strided_batched(ctx):
    from tensors_amd._lib import TF_F32, call
    B, M, N, K = 5, 33, 47, 29
    a = synth.normal(61, (B, M, K))
    b = synth.normal(62, (B, K, N))
    da, db = ctx.array(a), ctx.array(b)
    dc = ctx.zeros((B, M, N))
    call("tf_gemm_strided_batched", ctx.handle, 0, 0, M, N, K, 1.0, da.ptr, K, M * K, db.ptr, N, K * N,
         0.0, dc.ptr, N, M * N, B, TF_F32, TF_F32)
    truth = np.einsum("bmk,bkn->bmn", a.astype(np.float64), b.astype(np.float64))
    assert_close(dc.numpy(), truth, RTOL32, "strided batched")


def test_gemm_rejects_bad_shapes(ctx):
    from tensors_amd._lib import TF_F32, TFError, call
    d = ctx.zeros((4, 4))
    with pytest.raises(TFError):
        call("tf_gemm", ctx.handle, 0, 0, 4, 4, 4, 1.0, d.ptr, 2, d.ptr, 4, 0.0, d.ptr, 4, TF_F32, TF_F32, 0, None)
    with pytest.raises(TFError):
        call("tf_gemm", ctx.handle, 0, 0, 4, 4, 4, 1.0, d.ptr, 4, d.ptr, 4, 0.0, d.ptr, 4, TF_F32, TF_F32, 1, None)


def test_c2_linear_full_size(ctx):
    """Config 2 at full size: Y = X W^T + b, dX = dY W, dW = dY^T X, db = colsum(dY)."""
    ops = _ops()
    n = 2048
    X = synth.normal(synth.seed(2, 0), (n, n))
    W = synth.normal(synth.seed(2, 1), (n, n))
    dY = synth.normal(synth.seed(2, 2), (n, n))
    b = synth.normal(synth.seed(2, 3), (n,))
    dX_, dW_, dY_, dB_ = ctx.array(X), ctx.array(W), ctx.array(dY), ctx.array(b)
    Y, dXo, dWo, db = ctx.empty((n, n)), ctx.empty((n, n)), ctx.empty((n, n)), ctx.empty((n,))
    ops.gemm(dX_, dW_, Y, trans_b=True, bias=dB_)
    ops.gemm(dY_, dW_, dXo)
    ops.gemm(dY_, dX_, dWo, trans_a=True)
    ops.colsum(dY_, db)
    X64, W64, dY64 = X.astype(np.float64), W.astype(np.float64), dY.astype(np.float64)
    assert_close(Y.numpy(), X64 @ W64.T + b, RTOL32, "C2 Y")
    assert_close(dXo.numpy(), dY64 @ W64, RTOL32, "C2 dX")
    assert_close(dWo.numpy(), dY64.T @ X64, RTOL32, "C2 dW")
    assert_close(db.numpy(), dY64.sum(0), RTOL32, "C2 db")


# ---------------------------------------------------------------------------
# elementwise backward
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("ta,tb,M,N,K", [
    (False, False, 64, 256, 128),    # config 1: second layer's dX = (dY * [y > 0]) W2
    (True, False, 128, 256, 64),     # config 1: second layer's dW = (dY * [y > 0])^T X
    (True, False, 256, 784, 64),     # config 1: first layer's dW
    (False, True, 17, 19, 23), (True, True, 33, 65, 2048), (True, False, 5, 40, 129),
])
def test_gemm_relu_masked_equals_mask_then_gemm(ctx, ta, tb, M, N, K):
    """tf_gemm_relu_masked (the ReLU backward applied as the small kernel
    loads A) equals tf_relu_bwd followed by tf_gemm bit for bit: the masked
    element is the same product dy * (y > 0 ? 1 : 0) and the GEMM the same
    kernel.  The mask holds 0, -0 and +-1e-38 (strict > 0), and the product
    is checked against float64 too."""
    ops = _ops()
    seed = synth.seed(2, 11) + M + N + K
    shape_a = (K, M) if ta else (M, K)
    a = synth.normal(seed, shape_a)
    y = np.maximum(synth.normal(seed + 1, shape_a), 0.0).astype(np.float32)
    y.flat[:4] = [0.0, -0.0, 1e-38, -1e-38]
    b = synth.normal(seed + 2, (N, K) if tb else (K, N))
    da, dy_, db = ctx.array(a), ctx.array(y), ctx.array(b)
    got = ops.gemm_relu_masked(da, dy_, db, ctx.array(np.full((M, N), 7.0, np.float32)), trans_a=ta, trans_b=tb)
    dz = ops.relu_bwd(da, dy_, ctx.empty(shape_a))
    want = ops.gemm(dz, db, ctx.empty((M, N)), trans_a=ta, trans_b=tb)
    assert_bitexact(got.numpy(), want.numpy(), f"masked gemm {M}x{N}x{K}")
    assert_close(got.numpy(), _gemm_truth(oracle.relu_bwd(a, y), b, ta, tb), RTOL32, "masked gemm vs float64")
    again = ops.gemm_relu_masked(da, dy_, db, ctx.empty((M, N)), trans_a=ta, trans_b=tb)
    assert_bitexact(again.numpy(), got.numpy(), "second call")


@pytest.mark.parametrize("M,N,K,masked", [
    (64, 128, 256, True),      # config 1: the second layer's backward (dX 64 x 256, dW 128 x 256)
    (64, 128, 256, False),
    (50, 40, 70, True),        # ragged tiles in both products
    (3, 300, 33, False),       # one row group; dW over a 3-deep batch
])
def test_linear_bwd_small_equals_two_products(ctx, M, N, K, masked):
    """tf_linear_bwd_small (dX = dZ W and dW = dZ^T X in one launch, dZ = dY
    masked by y > 0 or dY itself) equals the two products launched alone bit
    for bit, twice in a row (the arrival counters are back at zero after each
    call), and float64 within the fp32 tolerance."""
    ops = _ops()
    seed = synth.seed(2, 13) + M + N + K
    dy = synth.normal(seed, (M, N))
    y = np.maximum(synth.normal(seed + 1, (M, N)), 0.0).astype(np.float32)
    x = synth.normal(seed + 2, (M, K))
    w = synth.normal(seed + 3, (N, K), std=0.1)
    d_dy, d_y, d_x, d_w = ctx.array(dy), ctx.array(y), ctx.array(x), ctx.array(w)
    mask = d_y if masked else None
    if masked:
        want_dx = ops.gemm_relu_masked(d_dy, d_y, d_w, ctx.empty((M, K))).numpy()
        want_dw = ops.gemm_relu_masked(d_dy, d_y, d_x, ctx.empty((N, K)), trans_a=True).numpy()
    else:
        want_dx = ops.gemm(d_dy, d_w, ctx.empty((M, K))).numpy()
        want_dw = ops.gemm(d_dy, d_x, ctx.empty((N, K)), trans_a=True).numpy()
    dz = oracle.relu_bwd(dy, y) if masked else dy
    for call in range(2):
        dx = ctx.array(np.full((M, K), 7.0, np.float32))
        dw = ctx.array(np.full((N, K), 7.0, np.float32))
        ops.linear_bwd_small(d_dy, d_x, d_w, dx, dw, mask=mask)
        assert_bitexact(dx.numpy(), want_dx, f"dx call {call}")
        assert_bitexact(dw.numpy(), want_dw, f"dw call {call}")
    assert_close(want_dx, _gemm_truth(dz, w, False, False), RTOL32, "dx vs float64")
    assert_close(want_dw, _gemm_truth(dz, x, True, False), RTOL32, "dw vs float64")


def test_linear_bwd_small_rejects_large_products(ctx):
    """A product whose inner extent exceeds the small kernel's 2048 is
    refused with TF_ERR_UNSUPPORTED (the Linear backward then launches the
    products separately)."""
    from tensors_amd._lib import TF_ERR_UNSUPPORTED, TFError
    ops = _ops()
    dy, x, w = ctx.zeros((4, 3000)), ctx.zeros((4, 8)), ctx.zeros((3000, 8))
    with pytest.raises(TFError) as e:
        ops.linear_bwd_small(dy, x, w, ctx.empty((4, 8)), ctx.empty((3000, 8)))
    assert e.value.status == TF_ERR_UNSUPPORTED


def test_gemm_relu_masked_outside_small_path(ctx):
    """A product the small kernel does not take (K > 2048) is refused with
    TF_ERR_UNSUPPORTED, and a narrow one (N <= 16, which plain tf_gemm sends
    to another kernel) still takes the small kernel with the mask."""
    ops = _ops()
    a, y = ctx.array(np.ones((8, 4096), np.float32)), ctx.array(np.ones((8, 4096), np.float32))
    with pytest.raises(Exception, match="small-product"):
        ops.gemm_relu_masked(a, y, ctx.array(np.ones((4096, 40), np.float32)), ctx.empty((8, 40)))
    a = synth.normal(901, (64, 256))
    y = np.maximum(synth.normal(902, (64, 256)), 0.0).astype(np.float32)
    b = synth.normal(903, (10, 256))
    got = ops.gemm_relu_masked(ctx.array(a), ctx.array(y), ctx.array(b), ctx.empty((64, 10)), trans_b=True)
    assert_close(got.numpy(), _gemm_truth(oracle.relu_bwd(a, y), b, False, True), RTOL32, "narrow masked")


SIZES = [0, 1, 17, 1000, 4096 * 1024 + 3]


@pytest.mark.parametrize("n", SIZES)
def test_relu_bwd_bitexact(ctx, n):
    ops = _ops()
    x = synth.normal(71, (n,))
    dy = synth.normal(72, (n,))
    if n >= 4:
        x[:4] = [0.0, -0.0, 1e-38, -1e-38]     # x == 0 masks to 0 (strict >)
    d = ctx.empty((n,))
    ops.relu_bwd(ctx.array(dy), ctx.array(x), d)
    assert_bitexact(d.numpy(), oracle.relu_bwd(dy, x), f"relu_bwd n={n}")


@pytest.mark.parametrize("n", [1, 1000, 1 << 20])
def test_sigmoid_tanh_bwd(ctx, n):
    ops = _ops()
    x = synth.normal(81, (n,))
    dy = synth.normal(82, (n,))
    ys, yt = oracle.sigmoid(x), oracle.tanh(x)
    d = ctx.empty((n,))
    ops.sigmoid_bwd(ctx.array(dy), ctx.array(ys), d)
    assert_close(d.numpy(), oracle.sigmoid_bwd(dy, ys), 1e-6, "sigmoid_bwd", atol=1e-7)
    ops.tanh_bwd(ctx.array(dy), ctx.array(yt), d)
    assert_close(d.numpy(), oracle.tanh_bwd(dy, yt), 1e-6, "tanh_bwd", atol=1e-7)


def test_forward_activations(ctx):
    ops = _ops()
    x = synth.normal(91, (5000,), std=3.0)
    d = ctx.empty((5000,))
    ops.relu(ctx.array(x), d)
    assert_bitexact(d.numpy(), oracle.relu(x), "relu fwd")
    ops.sigmoid(ctx.array(x), d)
    assert_close(d.numpy(), oracle.sigmoid(x), 1e-6, "sigmoid fwd", atol=1e-7)
    ops.tanh(ctx.array(x), d)
    assert_close(d.numpy(), oracle.tanh(x), 1e-6, "tanh fwd", atol=1e-7)


@pytest.mark.parametrize("n", [3, 4096, 1 << 20])
def test_add_mul_bitexact(ctx, n):
    ops = _ops()
    a, b = synth.normal(101, (n,)), synth.normal(102, (n,))
    d = ctx.empty((n,))
    ops.add(ctx.array(a), ctx.array(b), d)
    assert_bitexact(d.numpy(), oracle.add(a, b), "add")
    ops.mul(ctx.array(a), ctx.array(b), d)
    assert_bitexact(d.numpy(), a * b, "mul")


def test_relu_bwd_bf16(ctx):
    import tensors_amd as ta_mod
    ops = _ops()
    n = 4099
    x16 = ta_mod.f32_to_bf16_bits(synth.normal(111, (n,)))
    dy16 = ta_mod.f32_to_bf16_bits(synth.normal(112, (n,)))
    d = ctx.empty((n,), ta_mod.BF16)
    ops.relu_bwd(ctx.array(dy16, ta_mod.BF16), ctx.array(x16, ta_mod.BF16), d)
    want = ta_mod.f32_to_bf16_bits(oracle.relu_bwd(ta_mod.bf16_bits_to_f32(dy16), ta_mod.bf16_bits_to_f32(x16)))
    assert_bitexact(d.numpy(), want, "relu_bwd bf16")


# Float16 through the slots the reference's registry fills for Float16
# (cuda/kernels/elementwise.cu:185-245: widen with __half2float, compute in
# fp32, round with __float2half): the expected values are the oracle's fp32
# loop on the widened inputs, rounded by the oracle's round-to-nearest-even.
def _f16(x):
    return oracle.f32_to_f16_bits(x)


def _w16(h):
    return oracle.f16_bits_to_f32(h)


def _f16_inputs(seed, n, std=4.0):
    h = _f16(synth.normal(seed, (n,), std=std))
    if n >= 8:
        h[:8] = [0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x7BFF, 0xFBFF, 0x3C00]   # +-0, subnormals, +-max, 1
    return h


@pytest.mark.parametrize("n", [1, 17, 4099, (1 << 20) + 5])
def test_f16_add_mul_relu_leaky_bitexact(ctx, n):
    ops = _ops()
    a16, b16 = _f16_inputs(131, n), _f16_inputs(132, n)
    if n >= 16:
        b16[8:16] = [0x7BFF, 0x7BFF, 0x0001, 0x8001, 0x3C00, 0x3555, 0x7800, 0x0400]   # overflow, subnormal sums
    a, b = _w16(a16), _w16(b16)
    da, db = ctx.array(a16.view(np.float16)), ctx.array(b16.view(np.float16))
    out = ctx.empty((n,), np.float16)
    for name, fn, want in (("add", ops.add, oracle.add(a, b)), ("mul", ops.mul, a * b)):
        fn(da, db, out)
        assert_bitexact(out.numpy().view(np.uint16), _f16(want), f"f16 {name} n={n}")
    ops.relu(da, out)
    assert_bitexact(out.numpy().view(np.uint16), _f16(oracle.relu(a)), f"f16 relu n={n}")
    ops.leaky_relu(da, out, 0.1)
    assert_bitexact(out.numpy().view(np.uint16), _f16(oracle.leaky_relu(a, 0.1)), f"f16 leaky_relu n={n}")


@pytest.mark.parametrize("n", [5, 4099, 1 << 20])
def test_f16_sigmoid_tanh_and_backward(ctx, n):
    # The device's expf / tanhf differ from the host's by a few fp32 ulp; after
    # rounding to f16 that is at most one f16 step (2^-10 relative, 2^-24
    # absolute near zero), so the bar is written in those units.
    ops = _ops()
    x16, dy16 = _f16_inputs(141, n), _f16_inputs(142, n, std=1.0)
    x, dy = _w16(x16), _w16(dy16)
    dx_, ddy = ctx.array(x16.view(np.float16)), ctx.array(dy16.view(np.float16))
    out = ctx.empty((n,), np.float16)
    rtol, atol = 2.0 ** -10, 2.0 ** -24
    for name, fn, want in (("sigmoid", ops.sigmoid, oracle.sigmoid(x)), ("tanh", ops.tanh, oracle.tanh(x))):
        fn(dx_, out)
        assert_close(out.numpy().astype(np.float32), _w16(_f16(want)), rtol, f"f16 {name}", atol=atol)
    # backward on f16 saved outputs: dy * y * (1 - y) and dy * (1 - y^2) may
    # round differently in fp32 where the compiler fuses a multiply-add (as
    # for fp32, where the bar is 1e-6), so within one f16 step; dy * [x > 0]
    # is one exact selection, so bit for bit.
    ys16, yt16 = _f16(oracle.sigmoid(x)), _f16(oracle.tanh(x))
    for name, fn, y16, ref in (("sigmoid_bwd", ops.sigmoid_bwd, ys16, oracle.sigmoid_bwd),
                               ("tanh_bwd", ops.tanh_bwd, yt16, oracle.tanh_bwd)):
        fn(ddy, ctx.array(y16.view(np.float16)), out)
        assert_close(out.numpy().astype(np.float32), _w16(_f16(ref(dy, _w16(y16)))), rtol, f"f16 {name}", atol=atol)
    ops.relu_bwd(ddy, dx_, out)
    assert_bitexact(out.numpy().view(np.uint16), _f16(oracle.relu_bwd(dy, x)), "f16 relu_bwd")


# ---------------------------------------------------------------------------
# cross entropy / softmax rows
# ---------------------------------------------------------------------------
CE_SHAPES = [(64, 10), (128, 10), (4096, 1024), (4096, 1000), (33, 1023), (7, 3000), (5, 9000), (1, 1)]


@pytest.mark.parametrize("R,Cc", CE_SHAPES)
def test_ce_fwd_bwd_vs_chain(ctx, R, Cc):
    ops = _ops()
    logits = synth.normal(121 + R, (R, Cc), std=3.0)
    labels = synth.uniform_int(122 + Cc, (R,), Cc)
    loss_ref, d_ref = oracle.ce_chain(logits, labels)
    dl, dt = ctx.array(logits), ctx.array(labels)
    loss, lse, d = ctx.empty((1,)), ctx.empty((R,)), ctx.empty((R, Cc))
    ops.ce_fwd(dl, dt, loss, lse)
    assert_close(loss.numpy(), [loss_ref], RTOL32, "ce loss")
    ops.ce_bwd(dl, dt, d, lse=lse)
    assert_close(d.numpy(), d_ref, RTOL32, "ce bwd (saved lse)")
    ops.ce_bwd(dl, dt, d)
    assert_close(d.numpy(), d_ref, RTOL32, "ce bwd (recomputed lse)")
    loss2 = ctx.empty((1,))
    ops.ce_fwd_bwd(dl, dt, loss2, d)
    assert_close(loss2.numpy(), [loss_ref], RTOL32, "fused loss")
    assert_close(d.numpy(), d_ref, RTOL32, "fused dlogits")


@pytest.mark.parametrize("R,Cc", CE_SHAPES + [(4096, 1004), (9, 1001)])
def test_ce_fwd_bwd_bf16(ctx, R, Cc):
    """tf_ce_fwd_bwd_bf16 equals tf_ce_fwd_bwd on the widened logits followed
    by a round to bf16: bit for bit where both take the same element mapping
    (widths that are multiples of 4: the loss, and dlogits after rounding),
    within fp32 tolerance otherwise; and the oracle's chain within tolerance.
    Module flags, with a bad target making the loss NaN."""
    import tensors_amd as ta_mod
    from tensors_amd import _lib
    ops = _ops()
    bits = ta_mod.f32_to_bf16_bits(synth.normal(141 + R, (R, Cc), std=3.0))
    wide = ta_mod.bf16_bits_to_f32(bits)
    labels = synth.uniform_int(142 + Cc, (R,), Cc)
    dt = ctx.array(labels)
    loss16, d16 = ctx.empty((1,)), ctx.empty((R, Cc), ta_mod.BF16)
    loss32, d32 = ctx.empty((1,)), ctx.empty((R, Cc))
    ops.ce_fwd_bwd_bf16(ctx.array(bits, ta_mod.BF16), dt, loss16, d16, flags=_lib.TF_CE_MODULE)
    ops.ce_fwd_bwd(ctx.array(wide), dt, loss32, d32, flags=_lib.TF_CE_MODULE)
    want = ta_mod.f32_to_bf16_bits(d32.numpy())
    if Cc % 4 == 0:
        assert_bitexact(loss16.numpy(), loss32.numpy(), f"ce bf16 loss {R}x{Cc}")
        assert_bitexact(d16.numpy(), want, f"ce bf16 dlogits {R}x{Cc}")
    else:
        assert_close(loss16.numpy(), loss32.numpy(), RTOL32, f"ce bf16 loss {R}x{Cc}")
        assert_close(ta_mod.bf16_bits_to_f32(d16.numpy()), ta_mod.bf16_bits_to_f32(want), RTOL16,
                     f"ce bf16 dlogits {R}x{Cc}")
    assert_close(loss16.numpy(), [oracle.ce_module(wide, labels)], RTOL32, "ce bf16 loss vs oracle")
    _, d_ref = oracle.ce_chain(wide, labels)
    assert_close(ta_mod.bf16_bits_to_f32(d16.numpy()), d_ref, RTOL16, "ce bf16 dlogits vs oracle")
    if R > 1:
        labels[R // 2] = Cc
        ops.ce_fwd_bwd_bf16(ctx.array(bits, ta_mod.BF16), ctx.array(labels), loss16, d16, flags=_lib.TF_CE_MODULE)
        assert np.isnan(loss16.numpy()[0])
        assert np.all(d16.numpy()[R // 2] == 0)


def test_ce_upstream_scale_and_bad_labels(ctx):
    ops = _ops()
    R, Cc = 16, 10
    logits = synth.normal(131, (R, Cc))
    labels = synth.uniform_int(132, (R,), Cc)
    labels[3], labels[7] = -1, Cc          # skipped by the chain's one-hot mask
    loss_ref, d_ref = oracle.ce_chain(logits, labels)
    g = ctx.array(np.array([0.75], np.float32))
    d = ctx.empty((R, Cc))
    ops.ce_bwd(ctx.array(logits), ctx.array(labels), d, grad_loss=g)
    assert_close(d.numpy(), 0.75 * d_ref, RTOL32, "ce bwd * upstream")
    assert np.all(d.numpy()[[3, 7]] == 0.0)
    loss = ctx.empty((1,))
    ops.ce_fwd(ctx.array(logits), ctx.array(labels), loss)
    assert_close(loss.numpy(), [loss_ref], RTOL32, "loss with skipped labels")


def test_ce_module_flags_clamp_and_nan(ctx):
    """TF_CE_MODULE gives nn::CrossEntropyLoss's loss (probability clamped at
    1e-9, oracle.ce_module pinned to the reference); a bad target makes the
    loss NaN instead of a plausible value; the gradient is unchanged."""
    from tensors_amd import _lib
    ops = _ops()
    R, Cc = 64, 10
    logits = synth.normal(133, (R, Cc), std=3.0)
    labels = synth.uniform_int(134, (R,), Cc)
    logits[5] = np.array([0, 0, 0, 0, 0, 0, 0, 0, 0, 40], np.float32)
    labels[5] = 0
    dl, dt = ctx.array(logits), ctx.array(labels)
    loss, d = ctx.empty((1,)), ctx.empty((R, Cc))
    ops.ce_fwd(dl, dt, loss, flags=_lib.TF_CE_MODULE)
    assert_close(loss.numpy(), [oracle.ce_module(logits, labels)], RTOL32, "module loss with clamp")
    ops.ce_fwd(dl, dt, loss)                       # the chain: no clamp (row 5 contributes 40)
    assert float(loss.numpy()[0]) > oracle.ce_module(logits, labels) + 15.0 / R
    ops.ce_fwd_bwd(dl, dt, loss, d, flags=_lib.TF_CE_MODULE)
    assert_close(loss.numpy(), [oracle.ce_module(logits, labels)], RTOL32, "fused module loss")
    _, d_ref = oracle.ce_chain(logits, labels)
    assert_close(d.numpy(), d_ref, RTOL32, "gradient unchanged by the flags")
    labels[9] = Cc
    dt = ctx.array(labels)
    ops.ce_fwd(dl, dt, loss, flags=_lib.TF_CE_MODULE)
    assert np.isnan(loss.numpy()[0])
    ops.ce_fwd(dl, dt, loss, flags=_lib.TF_CE_CHAIN)
    assert np.isfinite(loss.numpy()[0])


@pytest.mark.parametrize("R,Cc", [(64, 10), (256, 1024), (3, 777), (2, 5000)])
def test_softmax_family(ctx, R, Cc):
    ops = _ops()
    x = synth.normal(141 + Cc, (R, Cc), std=2.0)
    dy = synth.normal(142 + Cc, (R, Cc))
    dx, dy_d, y = ctx.array(x), ctx.array(dy), ctx.empty((R, Cc))
    ops.log_softmax(dx, y)
    ly = oracle.log_softmax(x)
    assert_close(y.numpy(), ly, RTOL32, "log_softmax fwd")
    ops.softmax(dx, y)
    sy = oracle.softmax(x)
    assert_close(y.numpy(), sy, RTOL32, "softmax fwd")
    g = ctx.empty((R, Cc))
    ops.log_softmax_bwd(ctx.array(ly), dy_d, g)
    assert_close(g.numpy(), oracle.log_softmax_bwd(ly, dy), RTOL32, "log_softmax bwd")
    ops.softmax_bwd(ctx.array(sy), dy_d, g)
    assert_close(g.numpy(), oracle.softmax_bwd(sy, dy), RTOL32, "softmax bwd")


def test_softmax_bwd_uniform_is_zero(ctx):
    # autograd/ops/autograd_all_ops_test.cpp:108-121: uniform input, grad 0.
    ops = _ops()
    R, Cc = 4, 8
    y = np.full((R, Cc), 1.0 / Cc, np.float32)
    g = ctx.empty((R, Cc))
    ops.softmax_bwd(ctx.array(y), ctx.array(np.ones((R, Cc), np.float32)), g)
    assert np.max(np.abs(g.numpy())) < 1e-7


# ---------------------------------------------------------------------------
# reductions
# ---------------------------------------------------------------------------
# Multiples of 4 columns take the one-launch tile kernel: (2048, 2048),
# (4096, 8192), (7, 4096), (3001, 16384), (64, 256), (33, 64) (a short last
# chunk), (5000, 96) (157 chunks added by each strip's last block), and with
# a ragged last 32-column strip (100, 2056), (4096, 1000), (9, 4); small ones
# ((17, 19), (1, 5), (4096, 10)) take one block, (3, 1001) the two stages.
@pytest.mark.parametrize("R,Cc", [(2048, 2048), (64, 256), (17, 19), (1, 5), (4096, 10), (3, 1001), (4096, 8192),
                                  (7, 4096), (3001, 16384), (100, 2056), (33, 64), (5000, 96), (4096, 1000), (9, 4)])
def test_colsum(ctx, R, Cc):
    ops = _ops()
    dy = synth.normal(151 + R, (R, Cc))
    db = ctx.empty((Cc,))
    ops.colsum(ctx.array(dy), db)
    assert_close(db.numpy(), dy.astype(np.float64).sum(0), RTOL32, f"colsum {R}x{Cc}")
    assert_close(db.numpy(), oracle.colsum(dy), RTOL32, "colsum vs oracle")


@pytest.mark.parametrize("R,Cc", [(2048, 2048), (4096, 8192), (17, 19), (1, 5), (3, 1001), (64, 258), (7, 4096),
                                  (3001, 16384), (5000, 96), (4096, 1000), (100, 2056)])
def test_colsum_bf16(ctx, R, Cc):
    # bf16 dy summed in fp32: bit-exact against the fp32 colsum of the widened
    # tensor (same order; widening is exact), and within fp32 tolerance of
    # float64.
    import tensors_amd as ta_mod
    ops = _ops()
    bits = ta_mod.f32_to_bf16_bits(synth.normal(171 + R, (R, Cc)))
    wide = ta_mod.bf16_bits_to_f32(bits)
    db16, db32 = ctx.empty((Cc,)), ctx.empty((Cc,))
    ops.colsum(ctx.array(bits, ta_mod.BF16), db16)
    ops.colsum(ctx.array(wide), db32)
    assert np.array_equal(db16.numpy(), db32.numpy()), f"colsum_bf16 {R}x{Cc}"
    assert_close(db16.numpy(), wide.astype(np.float64).sum(0), RTOL32, f"colsum_bf16 {R}x{Cc} vs float64")


# tf_relu_bwd_colsum: one pass for widths that are multiples of 4
# ((4096, 1024) over several row chunks, (64, 8192), (33, 64), (5000, 96),
# (3, 1000) and (9, 1004) with a partial last 256-column strip), the two
# separate kernels otherwise ((17, 19)).  dz must equal tf_relu_bwd bit for bit (and the
# oracle's rule); db must be within fp32 tolerance of float64 and of the
# colsum of that dz, and bit-identical on a second call.  Special values:
# x = +-0 and NaN mask to 0, dy = +-inf under a zero mask gives NaN, dy = -0.
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("R,Cc", [(4096, 1024), (33, 64), (5000, 96), (64, 8192), (17, 19), (3, 1000), (9, 1004)])
def test_relu_bwd_colsum(ctx, dtype, R, Cc):
    import tensors_amd as ta_mod
    ops = _ops()
    x = synth.normal(181 + R, (R, Cc))
    dy = synth.normal(182 + Cc, (R, Cc))
    x[0, :6] = [0.0, -0.0, np.nan, 1e-30, -1e-30, 2.0]
    dy[0, :6] = [np.inf, -np.inf, 3.0, -0.0, -0.0, -0.0]
    if dtype == "bf16":
        xb, dyb = ta_mod.f32_to_bf16_bits(x), ta_mod.f32_to_bf16_bits(dy)
        dt = ta_mod.BF16
        want_dz = ta_mod.f32_to_bf16_bits(oracle.relu_bwd(ta_mod.bf16_bits_to_f32(dyb), ta_mod.bf16_bits_to_f32(xb)))
    else:
        xb, dyb, dt = x, dy, np.float32
        want_dz = oracle.relu_bwd(dy, x)
    dy_d, x_d = ctx.array(dyb, dt), ctx.array(xb, dt)
    dz, dz2 = ctx.empty((R, Cc), dt), ctx.empty((R, Cc), dt)
    db, db2 = ctx.empty((Cc,)), ctx.empty((Cc,))
    ops.relu_bwd_colsum(dy_d, x_d, dz, db)
    ops.relu_bwd(dy_d, x_d, dz2)
    ops.colsum(dz2, db2)
    got = dz.numpy()
    assert_bitexact(got, dz2.numpy(), f"relu_bwd_colsum dz {dtype} {R}x{Cc} vs tf_relu_bwd")
    # inf * 0 is NaN on both sides, with the host's and the GPU's own default
    # NaN bits: compare NaN positions as NaN, the rest bit for bit.
    gw = ta_mod.bf16_bits_to_f32(got) if dtype == "bf16" else got
    ww = ta_mod.bf16_bits_to_f32(want_dz) if dtype == "bf16" else want_dz
    nan = np.isnan(ww)
    assert np.array_equal(np.isnan(gw), nan) and nan[0, :2].all(), f"relu_bwd_colsum NaN positions {dtype}"
    assert_bitexact(got[~nan], want_dz[~nan], f"relu_bwd_colsum dz {dtype} {R}x{Cc} vs oracle")
    db1 = db.numpy()
    ops.relu_bwd_colsum(dy_d, x_d, dz, db)
    assert np.array_equal(db.numpy(), db1, equal_nan=True), f"relu_bwd_colsum db {dtype} {R}x{Cc} repeat"
    assert np.array_equal(np.isnan(db1), np.isnan(db2.numpy())), f"relu_bwd_colsum db NaNs {dtype} {R}x{Cc}"
    fin = ~np.isnan(db1)
    assert_close(db1[fin], db2.numpy()[fin], RTOL32, f"relu_bwd_colsum db {dtype} {R}x{Cc} vs colsum")
    wide = ta_mod.bf16_bits_to_f32(got) if dtype == "bf16" else got
    # Row 0 holds the NaN of inf * 0: compare the other columns to float64.
    truth = wide.astype(np.float64).sum(0)
    ok = np.isfinite(truth)
    assert np.isnan(db.numpy()[~ok]).all()
    assert_close(db.numpy()[ok], truth[ok], RTOL32, f"relu_bwd_colsum db {dtype} {R}x{Cc} vs float64")


def test_colsum_zero_rows(ctx):
    ops = _ops()
    db = ctx.array(np.full(7, 3.0, np.float32))
    ops.colsum(ctx.empty((0, 7)), db)
    assert np.all(db.numpy() == 0.0)


@pytest.mark.parametrize("shape", [(128, 32, 32, 32), (128, 64, 16, 16), (2, 3, 5, 7), (1, 1, 1, 1)])
def test_chansum_nchw(ctx, shape):
    ops = _ops()
    dy = synth.normal(161 + shape[1], shape)
    db = ctx.empty((shape[1],))
    ops.chansum_nchw(ctx.array(dy), db)
    assert_close(db.numpy(), dy.astype(np.float64).sum((0, 2, 3)), RTOL32, f"chansum {shape}")
    assert_close(db.numpy(), oracle.chansum_nchw(dy), RTOL32, "chansum vs oracle")


# ---------------------------------------------------------------------------
# SGD
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n", [1, 7, 235146, 1 << 20])
@pytest.mark.parametrize("mu", [0.9, 0.0])
def test_sgd_momentum_bitexact(ctx, n, mu):
    import tensors_amd as ta_mod
    ops = _ops()
    p, g, v = synth.normal(171, (n,)), synth.normal(172, (n,)), synth.normal(173, (n,))
    dp, dg, dv = ctx.array(p), ctx.array(g), ctx.array(v)
    sh = ctx.empty((n,), ta_mod.BF16)
    for _ in range(3):
        ops.sgd_momentum(dp, dg, dv, 0.1, mu, p_bf16=sh)
        p, v = oracle.sgd_momentum(p, g, v, 0.1, mu)
    assert_bitexact(dp.numpy(), p, "sgd p")
    assert_bitexact(dv.numpy(), v, "sgd v")
    assert_bitexact(sh.numpy(), ta_mod.f32_to_bf16_bits(p), "bf16 shadow")


class _OffsetView:
    """n float32 elements `offset` elements into a DeviceArray (not owned)."""

    def __init__(self, base, offset, n):
        from tensors_amd.device import DeviceArray
        self._base = base
        self.ctx, self.shape, self.dtype, self.size = base.ctx, (n,), np.float32, n
        self.nbytes = 4 * n
        self.ptr = base.ptr + 4 * offset
        self.tf_dtype = base.tf_dtype
        self.numpy = lambda: DeviceArray.numpy(self)


@pytest.mark.parametrize("mu", [0.9, 0.0])
def test_sgd_momentum_multi_bitexact(ctx, mu):
    # One launch over several parameters (ragged sizes, an unaligned one,
    # with and without a bf16 shadow) equals the oracle step of each.
    import tensors_amd as ta_mod
    ops = _ops()
    sizes = [2048, 7, 1, 235146, 2049, 1 << 20, 0]
    ps = [synth.normal(181 + i, (n,)) for i, n in enumerate(sizes)]
    gs = [synth.normal(191 + i, (n,)) for i, n in enumerate(sizes)]
    vs = [synth.normal(201 + i, (n,)) for i, n in enumerate(sizes)]
    dps = [ctx.array(x) for x in ps]
    dgs = [ctx.array(x) for x in gs]
    dvs = [ctx.array(x) for x in vs]
    # An unaligned parameter: a view one float into a larger buffer.
    base = ctx.array(np.concatenate([np.zeros(1, np.float32), ps[1]]))
    dps[1] = _OffsetView(base, 1, sizes[1])
    shs = [ctx.empty((n,), ta_mod.BF16) if i % 2 == 0 else None for i, n in enumerate(sizes)]
    for _ in range(3):
        ops.sgd_momentum_multi(dps, dgs, dvs if mu != 0.0 else None, 0.1, mu, shadows=shs)
        for i in range(len(sizes)):
            ps[i], vs[i] = oracle.sgd_momentum(ps[i], gs[i], vs[i], 0.1, mu)
    for i, n in enumerate(sizes):
        assert_bitexact(dps[i].numpy(), ps[i], f"multi sgd p[{i}] n={n}")
        if mu != 0.0:
            assert_bitexact(dvs[i].numpy(), vs[i], f"multi sgd v[{i}] n={n}")
        if shs[i] is not None:
            assert_bitexact(shs[i].numpy(), ta_mod.f32_to_bf16_bits(ps[i]), f"multi sgd shadow[{i}]")


def _bf16_special_inputs():
    """float32 bit patterns that exercise every branch of round-to-nearest-even
    to bf16: signed zeros, denormals, exact ties with even and odd kept bits,
    values just above and below a tie, the largest finite values (some round
    to infinity), infinities, and NaNs whose payload lies in the kept bits,
    only in the dropped bits, or both."""
    pats = [0x00000000, 0x80000000, 0x00000001, 0x807FFFFF, 0x00008000, 0x00018000, 0x00400000,
            0x3F808000, 0x3F818000, 0x3F807FFF, 0x3F808001, 0x3F800000, 0xBF808000, 0xBF818000,
            0x7F7F7FFF, 0x7F7F8000, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F800000, 0xFF800000,
            0x7FC00000, 0xFFC00000, 0x7F800001, 0xFF800001, 0x7FA00000, 0x7F80FFFF, 0x7FFFFFFF, 0xFFFFFFFF]
    rnd = synth.uniform_int(221, (4096,), 1 << 31).astype(np.uint32) * 2 + 1
    u = np.concatenate([np.array(pats, np.uint32), rnd, np.arange(0x3F800000, 0x3F800000 + 4096, dtype=np.uint32)])
    return u[: (u.size // 8) * 8 + 5]   # a scalar tail as well as the vector body


def test_cast_f32_bf16_hw_rounding(ctx):
    # Every f32 -> bf16 store in the library goes through the hardware
    # conversion (v_cvt_pk_bf16_f32: the cast's vector body converts pairs,
    # its scalar tail single values).  Both must equal the oracle's rule bit
    # for bit: round to nearest even, and a NaN keeps its sign and top
    # payload bits with the quiet bit set.
    import tensors_amd as ta_mod
    from tensors_amd._lib import call
    u = _bf16_special_inputs()
    x = u.view(np.float32)
    dx = ctx.array(x)
    dy = ctx.empty(x.shape, ta_mod.BF16)
    call("tf_cast_f32_bf16", ctx.handle, dx.ptr, dy.ptr, x.size)
    assert_bitexact(dy.numpy(), ta_mod.f32_to_bf16_bits(x), "bf16 rounding (incl. NaN payloads)")
