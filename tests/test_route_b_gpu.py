"""Route B on the GPU: the reference's own Tensor code (compiled from its
sources into oracle/_ref/route_b_check with the INTEGRATION.md registrar and
libtf_hip.so, by ``make -C oracle routeb``) runs add, mul, relu, leaky_relu,
sigmoid and tanh on device tensors; the program compares each with the
reference's CPU loops on the same inputs (bit-exact for add, mul, relu and
leaky_relu; sigmoid and tanh within 1e-6 relative + 1e-7 absolute).

The binary is built in the container that holds the reference tree and
travels with the repository; where it was not built the test is skipped.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "route_b_check"


@pytest.mark.skipif(not EXE.exists(), reason="oracle/_ref/route_b_check was not built (needs the reference tree)")
def test_route_b_elementwise_slots_on_device():
    print("route_b_check gpu", flush=True)
    r = subprocess.run([str(EXE), "gpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "route B gpu ok" in r.stdout, r.stdout[-4000:] + r.stderr[-2000:]
