"""Shared pytest setup: repo root on sys.path, the `gpu` marker, a device
context fixture and tolerance helpers."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def ctx():
    """One tf_ctx for the whole GPU session (fails, never skips, without a GPU)."""
    import tensors_amd as ta
    if ta.device_count() < 1:
        pytest.fail("GPU test selected but no HIP device is visible")
    c = ta.Context(0)
    yield c
    c.sync()
    c.close()


def assert_close(got, truth, rtol, what="", atol=None):
    """|got - truth| <= atol + rtol*|truth| with atol = rtol * rms(truth) by default
    (so near-zero entries of long sums are not judged on relative error alone)."""
    got = np.asarray(got, dtype=np.float64)
    truth = np.asarray(truth, dtype=np.float64)
    assert got.shape == truth.shape, f"{what}: shape {got.shape} vs {truth.shape}"
    if atol is None:
        rms = float(np.sqrt(np.mean(truth * truth))) if truth.size else 0.0
        atol = rtol * rms
    err = np.abs(got - truth)
    bound = atol + rtol * np.abs(truth)
    bad = ~(err <= bound)
    if bad.any():
        i = int(np.argmax(np.where(bad, err - bound, -np.inf)))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{got.size} outside rtol={rtol} atol={atol:.3g}; "
            f"worst flat index {i}: got {got.flat[i]!r} truth {truth.flat[i]!r}")


def assert_bitexact(got, ref, what=""):
    got = np.ascontiguousarray(got)
    ref = np.ascontiguousarray(ref)
    assert got.shape == ref.shape and got.dtype == ref.dtype, f"{what}: {got.shape}/{got.dtype} vs {ref.shape}/{ref.dtype}"
    gv = got.view(np.uint8).reshape(-1)
    rv = ref.view(np.uint8).reshape(-1)
    if not np.array_equal(gv, rv):
        diff = np.nonzero(got.reshape(-1).view(np.uint8 if got.dtype.itemsize == 1 else
                                               {2: np.uint16, 4: np.uint32, 8: np.uint64}[got.dtype.itemsize])
                          != ref.reshape(-1).view(np.uint8 if ref.dtype.itemsize == 1 else
                                                  {2: np.uint16, 4: np.uint32, 8: np.uint64}[ref.dtype.itemsize]))[0]
        i = int(diff[0])
        raise AssertionError(f"{what}: {diff.size} elements differ bitwise; first at {i}: "
                             f"{got.reshape(-1)[i]!r} vs {ref.reshape(-1)[i]!r}")
