"""tf_gemm_noalloc (the GEMM entry point that allocates nothing) against
tf_gemm through the C ABI: the same kernels and split choices, so the outputs
must be bit-identical.  Two calls in a row on the shared scratch array, the
second smaller than the first, products that use no partials at all, then
shapes whose partials exceed the fixed scratch on the tiled split-K path and
on the narrow-output path, which must be rejected without touching the
output."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from tensors_amd import _lib, synth
from tensors_amd._lib import TFError, call
from tests.conftest import assert_bitexact

pytestmark = pytest.mark.gpu


def _gemm(ctx, entry, a, b, c, trans_a, trans_b, bias=None, relu=False):
    M, N = c.shape
    K = a.shape[0] if trans_a else a.shape[1]
    epi = (_lib.TF_EPI_BIAS_RELU if relu else _lib.TF_EPI_BIAS) if bias is not None else _lib.TF_EPI_NONE
    call(entry, ctx.handle, int(trans_a), int(trans_b), M, N, K, 1.0, a.ptr, a.shape[1], b.ptr, b.shape[1], 0.0,
         c.ptr, c.shape[1], a.tf_dtype, c.tf_dtype, epi, bias.ptr if bias is not None else None)


def _pair(ctx, a, b, shape, out_dtype, trans_a, trans_b, bias=None, relu=False):
    c_ref, c_new = ctx.zeros(shape, out_dtype), ctx.zeros(shape, out_dtype)
    _gemm(ctx, "tf_gemm", a, b, c_ref, trans_a, trans_b, bias, relu)
    _gemm(ctx, "tf_gemm_noalloc", a, b, c_new, trans_a, trans_b, bias, relu)
    return c_ref.numpy(), c_new.numpy()


def test_gemm_noalloc_matches_tf_gemm(ctx):
    import tensors_amd as ta
    # 1) config 5's last-layer forward: bf16 4096 x 1000 x 4096, 4 K slices
    #    (65.5 MB of partials, the largest split the benchmarks make).
    rng = np.random.default_rng(9100)
    a = ctx.array(ta.f32_to_bf16_bits(rng.standard_normal((4096, 4096), dtype=np.float32)), ta.BF16)
    w = ctx.array(ta.f32_to_bf16_bits(rng.standard_normal((1000, 4096), dtype=np.float32) * np.float32(0.02)),
                  ta.BF16)
    bias = ctx.array(synth.normal(9101, (1000,)))
    ref, got = _pair(ctx, a, w, (4096, 1000), ta.BF16, False, True, bias=bias)
    assert_bitexact(got, ref, "bf16 4096x1000x4096 split-K")
    del a, w
    # 2) a smaller call right after, on the same scratch: config 4's
    #    classifier [128 x 16384] @ [10 x 16384]^T in fp32 (128 K slices).
    x = ctx.array(synth.normal(9102, (128, 16384)))
    wf = ctx.array(synth.normal(9103, (10, 16384), std=0.01))
    ref, got = _pair(ctx, x, wf, (128, 10), np.float32, False, True)
    assert_bitexact(got, ref, "fp32 128x10x16384 split-K")
    # 3) a small fp32 product (40 tiles of 32 x 32): its four K chunk groups
    #    add their partials through the scratch too (gemm_f32_small_kernel).
    p = ctx.array(synth.normal(9104, (300, 200)))
    q = ctx.array(synth.normal(9105, (200, 100)))
    ref, got = _pair(ctx, p, q, (300, 100), np.float32, False, False, relu=True, bias=ctx.array(synth.normal(9106, (100,))))
    assert_bitexact(got, ref, "fp32 300x100x200")
    # 4) products without any partials (one tile per CU or more, no split):
    #    bf16 4096 x 4096 x 512 (256 tiles of 256 x 256) and config 2's
    #    fp32 2048^3 (256 tiles of 128 x 128).
    a = ctx.array(ta.f32_to_bf16_bits(rng.standard_normal((4096, 512), dtype=np.float32)), ta.BF16)
    b = ctx.array(ta.f32_to_bf16_bits(rng.standard_normal((4096, 512), dtype=np.float32)), ta.BF16)
    ref, got = _pair(ctx, a, b, (4096, 4096), np.float32, False, True)
    assert_bitexact(got, ref, "bf16 4096x4096x512 (no split)")
    del a, b
    x2 = ctx.array(synth.normal(9107, (2048, 2048)))
    w2 = ctx.array(synth.normal(9108, (2048, 2048)))
    ref, got = _pair(ctx, x2, w2, (2048, 2048), np.float32, False, False)
    assert_bitexact(got, ref, "fp32 2048^3 (no split)")
    ctx.sync()


def test_gemm_noalloc_rejects_partials_beyond_scratch(ctx):
    import tensors_amd as ta
    # bf16 4096 x 1536 x 2048: 16 x 6 tiles of 256, split over 3 K slices
    # -> 3 * 4096 * 1536 * 4 = 75.5 MB of partials > 64 MiB.
    a = ctx.zeros((4096, 2048), ta.BF16)
    b = ctx.zeros((2048, 1536), ta.BF16)
    c = ctx.array(np.full((4096, 1536), 7.0, np.float32))
    with pytest.raises(TFError, match="scratch"):
        _gemm(ctx, "tf_gemm_noalloc", a, b, c, False, False)
    assert np.all(c.numpy() == 7.0)
    # tf_gemm takes the same shape (its workspace grows from the pool).
    _gemm(ctx, "tf_gemm", a, b, c, False, False)
    assert np.all(c.numpy() == 0.0)
    ctx.sync()


def test_gemm_noalloc_rejects_narrow_output_partials_beyond_scratch(ctx):
    # The narrow-output fp32 path (<= 16 columns, K >= 2048): 32768 x 16 over
    # K = 33792 is 66 chunks of 512 (the MFMA form), whose partials need
    # 66 * 32768 * 16 * 4 = 138 MB > 64 MiB.  Rejected before any launch, so
    # the output keeps its contents; the operands are real allocations of
    # the stated shapes all the same (A is 4.4 GB).
    M, N, K = 32768, 16, 33792
    a = ctx.zeros((M, K))
    b = ctx.zeros((N, K))
    c = ctx.array(np.full((M, N), 3.0, np.float32))
    with pytest.raises(TFError, match="scratch"):
        _gemm(ctx, "tf_gemm_noalloc", a, b, c, False, True)
    assert np.all(c.numpy() == 3.0)
    del a
    ctx.sync()
