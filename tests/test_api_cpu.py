"""The C++20 tensorforge API (libtensorforge.so) on CPU tensors: the
self-tests that restate the reference's unit tests, the reference weight
init, and a short training run against the reference-order oracle."""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from tensors_amd import api, synth
from tests.conftest import assert_close

META = json.loads((Path(__file__).resolve().parent / "golden" / "reference_outputs.json").read_text())
FIX = np.load(Path(__file__).resolve().parent / "golden" / "reference_outputs.npz")
C1 = [784, 256, 128, 10]


@pytest.mark.parametrize("name", api.selftest_names())
def test_selftest_cpu(name):
    api.selftest(name, on_gpu=False)


def test_unknown_selftest_reports_error():
    with pytest.raises(api.HarnessError, match="unknown self-test"):
        api.selftest("no_such_test", on_gpu=False)


def _init_weights():
    _, fw, _ = api.mlp_train(C1, np.zeros((1, 1, 784), np.float32), np.zeros((1, 1), np.int64), steps=0, lr=0.1,
                             mu=0.9, on_gpu=False, reference_compat=True, want_weights=True)
    offs = np.cumsum([0] + [C1[k] * C1[k + 1] for k in range(3)])
    return [fw[offs[i]:offs[i + 1]].reshape(C1[i + 1], C1[i]) for i in range(3)]


def test_linear_init_equals_reference_init():
    """nn::Linear's Kaiming-uniform init reproduces the reference's weights bit for bit."""
    for i, w in enumerate(_init_weights()):
        key = f"c1_init_w{i}"
        if key in FIX.files:
            assert np.array_equal(w.view(np.uint32), FIX[key].view(np.uint32))
        else:
            assert hashlib.sha256(np.ascontiguousarray(w).tobytes()).hexdigest() == META[f"{key}:sha256"]


def test_cpu_training_tracks_oracle():
    """5 steps of the config-1 MLP on CPU tensors through the C++ API vs the
    reference-order oracle (the API's CE module computes softmax then log,
    the chain log_softmax, so equality is to tolerance)."""
    steps = 5
    xs = synth.mnist_like(synth.seed(1, 0), (steps, 64, 784))
    ys = synth.uniform_int(synth.seed(1, 1), (steps, 64), 10)
    losses, fw, _ = api.mlp_train(C1, xs, ys, steps=steps, lr=0.1, mu=0.9, on_gpu=False, reference_compat=True,
                                  want_weights=True)
    ws = [w.copy() for w in _init_weights()]
    vs = [np.zeros_like(w) for w in ws]
    ref = [oracle.mlp_step(ws, vs, xs[s], ys[s], 0.1, 0.9) for s in range(steps)]
    assert_close(losses, ref, 1e-5, "losses", atol=1e-5)
    assert_close(fw, np.concatenate([w.ravel() for w in ws]), 1e-4, "weights")


def test_release_memory_without_gpu_context_is_a_no_op():
    """tfa_release_memory before any GPU context exists (here: no GPU)."""
    api.release_memory()


def test_cpu_errors_are_reported():
    with pytest.raises(api.HarnessError):
        api.mlp_train([784, 10], np.zeros((1, 2, 784), np.float32), np.zeros((1, 2), np.int64), steps=1, lr=-1.0,
                      mu=0.0, on_gpu=False)
    with pytest.raises(api.HarnessError, match="bf16"):
        api.mlp_train([784, 10], np.zeros((1, 2, 784), np.float32), np.zeros((1, 2), np.int64), steps=1, lr=0.1,
                      mu=0.0, on_gpu=False, bf16=True)


def test_mlp_step_trace_on_cpu_matches_float64():
    """tfa_mlp_step_trace on CPU tensors (fp32, reference loop order): the
    stored outputs, gradients and updated parameters of one step of a small
    MLP with biases against float64."""
    dims, B = [20, 16, 12, 5], 9
    rng = np.random.default_rng(77)
    x = rng.standard_normal((B, dims[0])).astype(np.float32)
    y = rng.integers(0, dims[-1], B).astype(np.int64)
    w0 = [(rng.standard_normal((dims[i + 1], dims[i])) * 0.3).astype(np.float32) for i in range(3)]
    loss, acts, grads, fw, fb = api.mlp_step_trace(dims, x, y, lr=1.0, mu=0.0, on_gpu=False,
                                                   init_weights=np.concatenate([w.ravel() for w in w0]))
    a = [x.astype(np.float64)]
    for i in range(3):
        z = a[-1] @ w0[i].T.astype(np.float64)
        a.append(np.maximum(z, 0) if i < 2 else z)
    for l in range(4):
        np.testing.assert_allclose(acts[l], a[l], rtol=1e-5, atol=1e-6)
    m = a[3].max(1, keepdims=True)
    e = np.exp(a[3] - m)
    p = e / e.sum(1, keepdims=True)
    assert abs(loss - np.mean(-np.log(p[np.arange(B), y]))) < 1e-5
    p[np.arange(B), y] -= 1
    g = p / B
    for l in range(3, 0, -1):
        np.testing.assert_allclose(grads[l - 1], g, rtol=1e-4, atol=1e-7)
        dz = g if l == 3 else g * (a[l] > 0)
        np.testing.assert_allclose(w0[l - 1] - fw[l - 1], dz.T @ a[l - 1], rtol=1e-4, atol=1e-6)
        np.testing.assert_allclose(-fb[l - 1].ravel(), dz.sum(0), rtol=1e-4, atol=1e-7)
        g = dz @ w0[l - 1].astype(np.float64)
