"""The C++20 tensorforge API on GPU 0 (libtensorforge.so over libtf_hip.so):
self-tests, the config-1 100-step loss trajectory against the compiled
reference, the config-4 CNN step against the reference-order oracle, and the
config-5 bf16 mixed-precision MLP."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from tensors_amd import api, synth
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"
FIX = np.load(GOLD / "reference_outputs.npz")
META = json.loads((GOLD / "reference_outputs.json").read_text())
C1 = [784, 256, 128, 10]


def sample_idx(n):
    return np.unique(synth.uniform_int(0xF1C5, (4096,), n)) if n > 4096 else np.arange(n)


@pytest.mark.parametrize("name", api.selftest_names())
def test_selftest_gpu(name, ctx):
    api.selftest(name, on_gpu=True)


def _c1_inputs(steps):
    xs = synth.mnist_like(synth.seed(1, 0), (100, 64, 784))[:steps]
    ys = synth.uniform_int(synth.seed(1, 1), (100, 64), 10)[:steps]
    return xs, ys


def test_c1_loss_trajectory_matches_reference(ctx):
    """100 fwd+bwd+momentum-SGD steps on the GPU (fused Linear / CE nodes, MFMA
    GEMMs) follow the compiled reference's trajectory within 1e-3."""
    xs, ys = _c1_inputs(100)
    losses, fw, _ = api.mlp_train(C1, xs, ys, steps=100, lr=0.1, mu=0.9, on_gpu=True, reference_compat=True,
                                  want_weights=True)
    ref = FIX["c1_losses_100"]
    err = np.max(np.abs(losses.astype(np.float64) - ref))
    assert err <= 1e-3, f"max |loss - reference| = {err}"
    got = fw[sample_idx(fw.size)]
    want = FIX["c1_weights_after_100:sample"]
    assert_close(got, want, 1e-3, "weights after 100 steps")


@pytest.mark.parametrize("graph", [1, 2])
def test_c1_graph_replay_matches_eager_and_reference(ctx, graph):
    """The config-1 loop with its step captured in a HIP graph after 10 eager
    steps: the 90 replays reproduce the eager loop bit for bit (same kernels,
    same order, same buffers' contents) and so follow the reference's
    trajectory within 1e-3.  graph=2 waits for every replay and reads its
    loss before launching the next (eager work and synchronisations between
    replays; the harness also checks that no later replay changed an earlier
    replay's recorded loss)."""
    xs, ys = _c1_inputs(100)
    kw = dict(steps=100, warmup=10, lr=0.1, mu=0.9, on_gpu=True, reference_compat=True, want_weights=True)
    eager, fw_e, _ = api.mlp_train(C1, xs, ys, **kw)
    print(f"graph mode {graph}", flush=True)
    replay, fw_g, _ = api.mlp_train(C1, xs, ys, graph=graph, **kw)
    assert np.array_equal(replay.view(np.uint32), eager.view(np.uint32)), \
        f"first differing step {int(np.argmax(replay != eager))}"
    assert np.array_equal(fw_g.view(np.uint32), fw_e.view(np.uint32))
    err = np.max(np.abs(replay.astype(np.float64) - FIX["c1_losses_100"]))
    assert err <= 1e-3, f"max |loss - reference| = {err}"


def test_c1_graph_replay_with_fewer_batches_than_steps(ctx):
    """Batch selection on the device wraps around the batch table (step s
    uses batch s % n_batches), as the eager loop does."""
    xs, ys = _c1_inputs(7)
    kw = dict(steps=30, warmup=3, lr=0.1, mu=0.9, on_gpu=True, reference_compat=True)
    eager, _, _ = api.mlp_train(C1, xs, ys, **kw)
    replay, _, _ = api.mlp_train(C1, xs, ys, graph=1, **kw)
    assert np.array_equal(replay.view(np.uint32), eager.view(np.uint32))


def test_c1_graph_mode_rejects_bad_arguments(ctx):
    xs, ys = _c1_inputs(2)
    with pytest.raises(api.HarnessError):
        api.mlp_train(C1, xs, ys, steps=4, warmup=0, lr=0.1, mu=0.9, on_gpu=True, graph=1)
    with pytest.raises(api.HarnessError):
        api.mlp_train(C1, xs, ys, steps=4, warmup=1, lr=0.1, mu=0.9, on_gpu=False, graph=1)


def test_c1_first_step_update_matches_reference(ctx):
    """The first SGD update (= -lr * gradient) of every weight matches the
    reference's within rtol 1e-4 (atol 1e-4 * rms of the update)."""
    xs, ys = _c1_inputs(1)
    _, w0, _ = api.mlp_train(C1, xs, ys, steps=0, lr=0.1, mu=0.9, on_gpu=False, reference_compat=True,
                             want_weights=True)
    _, w1, _ = api.mlp_train(C1, xs, ys, steps=1, lr=0.1, mu=0.9, on_gpu=True, reference_compat=True,
                             want_weights=True)
    idx = sample_idx(w0.size)
    upd_gpu = w1[idx].astype(np.float64) - w0[idx]
    upd_ref = FIX["c1_weights_after_1:sample"].astype(np.float64) - w0[idx]
    assert_close(upd_gpu, upd_ref, 1e-4, "first update")


def test_c1_bias_mode_trains(ctx):
    """With the bias enabled (this backend's default) the step runs and the
    loss stays in the ln(10) band on random labels."""
    xs, ys = _c1_inputs(20)
    losses, _, _ = api.mlp_train(C1, xs, ys, steps=20, lr=0.1, mu=0.9, on_gpu=True)
    assert np.all(np.isfinite(losses)) and abs(float(losses[-1]) - np.log(10)) < 0.2


def _cnn_params(H):
    flat = 64 * (H // 2) * (H // 2)
    shapes = [(32, 3, 3, 3), (32,), (64, 32, 3, 3), (64,), (10, flat), (10,)]
    stds = [0.2, 0.1, 0.06, 0.1, 0.01, 0.1]
    return [synth.normal(synth.seed(4, 10 + i), s, std=sd) for i, (s, sd) in enumerate(zip(shapes, stds))]


def test_c4_cnn_steps_match_reference_loop(ctx):
    """3 steps of the config-4 CNN (reduced batch 8) through Conv2dModule /
    Linear / CrossEntropyLoss / SGD on the GPU vs the restated reference loop."""
    B, H, steps = 8, 32, 3
    xs = synth.normal(synth.seed(4, 0), (steps, B, 3, H, H))
    ys = synth.uniform_int(synth.seed(4, 1), (steps, B), 10)
    params = _cnn_params(H)
    init = np.concatenate([p.ravel() for p in params])
    losses, _ = api.cnn_train(xs, ys, steps=steps, lr=0.01, mu=0.9, on_gpu=True, init_params=init)
    ps = [p.copy() for p in params]
    vs = [np.zeros_like(p) for p in ps]
    ref = [oracle.cnn_step(ps, vs, xs[s], ys[s], 0.01, 0.9) for s in range(steps)]
    assert_close(losses, ref, 1e-4, "cnn losses", atol=1e-5)


def test_c4_cnn_full_batch_runs(ctx):
    B, H = 128, 32
    xs = synth.normal(synth.seed(4, 0), (1, B, 3, H, H))
    ys = synth.uniform_int(synth.seed(4, 1), (1, B), 10)
    losses, ms = api.cnn_train(xs, ys, steps=5, lr=0.01, mu=0.9, on_gpu=True, warmup=1)
    assert np.all(np.isfinite(losses)) and ms > 0


def test_c5_bf16_mlp_tracks_fp32(ctx):
    """Reduced config 5 (bf16 weights/activations, fp32 accumulate and master
    weights): the loss trajectory stays within 2e-2 of the same model in fp32."""
    dims = [512, 1024, 1024, 512, 100]
    B, steps = 256, 5
    xs = synth.normal(synth.seed(5, 0), (steps, B, dims[0]))
    ys = synth.uniform_int(synth.seed(5, 1), (steps, B), dims[-1])
    l32, _, _ = api.mlp_train(dims, xs, ys, steps=steps, lr=0.01, mu=0.9, on_gpu=True)
    l16, _, _ = api.mlp_train(dims, xs, ys, steps=steps, lr=0.01, mu=0.9, on_gpu=True, bf16=True)
    assert np.all(np.isfinite(l16))
    assert_close(l16, l32, 2e-2, "bf16 vs fp32 losses", atol=1e-2)


@pytest.mark.parametrize("cfg", ["c1", "c5"])
def test_pool_use_is_flat_across_steps(ctx, cfg):
    """Storage is released when its last reference goes (the reference never
    frees, tensor/Storage.hpp:27): the device pool's bytes in use after each
    step stop growing after the first steps (C1: steps 10 and 100 equal; C5
    at full size: steps 4 and 12 equal)."""
    if cfg == "c1":
        dims, steps, early = C1, 100, 9
        xs, ys = _c1_inputs(100)
        kw = dict(lr=0.1, mu=0.9, reference_compat=True)
    else:
        dims, steps, early = [4096, 8192, 8192, 4096, 1000], 12, 3
        xs = np.random.default_rng(5500).standard_normal((1, 4096, 4096), dtype=np.float32)
        ys = np.random.default_rng(5501).integers(0, 1000, (1, 4096)).astype(np.int64)
        kw = dict(lr=0.01, mu=0.9, bf16=True)
    trace = np.zeros(steps, np.uint64)
    losses, _, _ = api.mlp_train(dims, xs, ys, steps=steps, on_gpu=True, pool_trace=trace, **kw)
    assert np.all(np.isfinite(losses))
    assert trace[early] > 0
    assert np.all(trace[early:] == trace[early]), f"pool bytes in use grow: {trace.tolist()}"


def test_release_memory_returns_pool_memory(ctx):
    """tfa_release_memory hands the harness's cached blocks and the pool's
    free memory back to the driver: after a C1 run the device pool holds no
    more than before (the pool is shared with this test's context, whose own
    allocations stay), and training afterwards gives the same losses."""
    xs, ys = _c1_inputs(20)
    kw = dict(lr=0.1, mu=0.9, reference_compat=True)
    before, _, _ = api.mlp_train(C1, xs, ys, steps=20, on_gpu=True, **kw)
    ctx.sync()
    reserved0, _ = ctx.pool_stats()
    api.release_memory()
    api.release_memory()                          # nothing left to release: still fine
    ctx.sync()
    reserved1, used1 = ctx.pool_stats()
    assert used1 <= reserved1 <= reserved0, (reserved0, reserved1, used1)
    after, _, _ = api.mlp_train(C1, xs, ys, steps=20, on_gpu=True, **kw)
    assert np.array_equal(before, after)

