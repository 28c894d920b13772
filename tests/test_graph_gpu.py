"""HIP-graph capture through the C ABI (tf_graph_*), and the two device-side
step helpers (tf_gather_indexed, tf_record_step).

A captured sequence of library calls is replayed several times with the
program's own eager work (new inputs uploaded, the outputs read back) and
synchronisations between the replays, and every replay is checked bit for
bit against the same calls run eagerly on the same inputs.  The capture's
rules are checked from the host: a block-cache miss and a synchronising call
during capture fail, the capture then yields no graph, and the context keeps
working; a block allocated during capture and freed while its graph exists
is not handed to other allocations.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from tensors_amd import ops, synth
from tensors_amd._lib import TFError, call, lib
from tests.conftest import assert_bitexact

pytestmark = pytest.mark.gpu


def _end(ctx):
    g = C.c_void_p()
    call("tf_graph_end", ctx.handle, C.byref(g))
    return g


def test_graph_replays_match_eager_calls(ctx):
    B, K, N = 64, 256, 128
    a = ctx.array(synth.normal(1001, (B, K)))
    w = ctx.array(synth.normal(1002, (N, K), std=0.06))
    z, h, c = ctx.empty((B, N)), ctx.empty((B, N)), ctx.empty((N,))
    z2, h2, c2 = ctx.empty((B, N)), ctx.empty((B, N)), ctx.empty((N,))

    def seq(zz, hh, cc):
        ops.gemm(a, w, zz, trans_b=True)
        ops.relu(zz, hh)
        ops.colsum(hh, cc)

    seq(z2, h2, c2)                    # eager once: any workspace is grown now
    ctx.sync()
    call("tf_graph_begin", ctx.handle)
    seq(z, h, c)
    g = _end(ctx)
    try:
        for r in range(4):
            a.upload(synth.normal(1100 + r, (B, K)))      # eager work between replays
            call("tf_graph_launch", ctx.handle, g)
            seq(z2, h2, c2)                               # the same calls, eagerly
            ctx.sync()
            for got, want, what in ((z, z2, "gemm"), (h, h2, "relu"), (c, c2, "colsum")):
                assert_bitexact(got.numpy(), want.numpy(), f"replay {r}: {what}")
    finally:
        call("tf_graph_destroy", g)


def test_capture_fails_on_a_cache_miss_and_on_sync(ctx):
    call("tf_graph_begin", ctx.handle)
    p = C.c_void_p()
    with pytest.raises(TFError):
        call("tf_hip_alloc", ctx.handle, C.c_size_t((3 << 30) + 12345), C.byref(p))   # no such cached block
    with pytest.raises(TFError):
        _end(ctx)
    call("tf_graph_begin", ctx.handle)
    with pytest.raises(TFError):
        call("tf_hip_sync", ctx.handle)
    with pytest.raises(TFError):
        _end(ctx)
    # The context is usable afterwards.
    x = ctx.array(synth.normal(1200, (1000,)))
    y = ctx.empty((1000,))
    ops.relu(x, y)
    assert_bitexact(y.numpy(), np.maximum(x.numpy(), 0).astype(np.float32), "relu after failed captures")


def test_gather_and_record_in_a_replayed_graph(ctx):
    n, bytes_ = 3, 4096 * 4 + 8
    srcs = [ctx.array(synth.normal(1300 + i, (bytes_ // 4,))) for i in range(n)]
    table = ctx.array(np.array([s.ptr for s in srcs], np.uint64), np.uint64)
    counter = ctx.array(np.array([0], np.int64))
    dst = ctx.empty((bytes_ // 4,))
    ring = ctx.zeros((8,))
    call("tf_gather_indexed", ctx.handle, dst.ptr, table.ptr, n, counter.ptr, bytes_)
    call("tf_record_step", ctx.handle, dst.ptr, ring.ptr, 8, counter.ptr)     # eager: step 0
    ctx.sync()
    assert_bitexact(dst.numpy(), srcs[0].numpy(), "gather step 0")
    call("tf_graph_begin", ctx.handle)
    call("tf_gather_indexed", ctx.handle, dst.ptr, table.ptr, n, counter.ptr, bytes_)
    call("tf_record_step", ctx.handle, dst.ptr, ring.ptr, 8, counter.ptr)
    g = _end(ctx)
    try:
        for step in range(1, 10):                         # the ring holds 8: later steps only count
            call("tf_graph_launch", ctx.handle, g)
            ctx.sync()
            assert_bitexact(dst.numpy(), srcs[step % n].numpy(), f"gather step {step}")
            assert int(counter.numpy()[0]) == step + 1
    finally:
        call("tf_graph_destroy", g)
    want = np.array([srcs[s % n].numpy()[0] for s in range(8)], np.float32)
    assert_bitexact(ring.numpy(), want, "recorded values")


def test_block_allocated_during_capture_stays_with_its_graph(ctx):
    # A size class no other test uses (2 MB steps above 1 MB: 38.1 MB -> 40 MB).
    n = 10_000_000
    x = ctx.array(synth.normal(1400, (n,)))
    first = ctx.empty((n,))
    first.free()                                   # the cache now holds one block of the class
    call("tf_graph_begin", ctx.handle)
    inside = ctx.empty((n,))                       # served from the cache during capture
    ops.relu(x, inside)
    g = _end(ctx)
    try:
        held = inside.ptr
        inside.free()                              # freed while the graph exists
        other = ctx.empty((n,))
        assert other.ptr != held, "a block the graph writes was handed to another allocation"
        call("tf_hip_fill_f32", ctx.handle, other.ptr, 5.0, n)
        call("tf_graph_launch", ctx.handle, g)     # writes relu(x) into the held block
        ctx.sync()
        assert np.all(other.numpy() == 5.0), "a replay wrote into another allocation's memory"
    finally:
        call("tf_graph_destroy", g)
    other.free()
    ctx.sync()
