"""The reference's own doctest suites, compiled unchanged against this build's
C++ API (the headers under tensors_amd/cpp, lib/libtensorforge.so), once
plain and once under AddressSanitizer + UndefinedBehaviorSanitizer (with a
sanitized build of libtensorforge.so made from the same sources); and the
route-B registrar of INTEGRATION.md, compiled as written against the
reference's own headers and linked with the reference's objects and
libtf_hip.so (oracle/_ref/route_b_check).

CPU only; skipped where /root/reference is absent (the GPU box).  The suites
are every ``*_test.cpp`` under the reference's tensor/, autograd/, nn/,
data/ and tests/ except those that include the CUDA toolkit's
``cuda_runtime.h`` (tensor/tensor_to_test.cpp, nn/conv2d_forward_test.cpp,
nn/conv2d_backward_test.cpp: they drive CUDA directly); the reference's
cuda/ suites test its CUDA kernels, which this build replaces.  The
reference's two example programs (examples/train_mlp.cpp, train_cnn.cpp)
are also built unchanged and run on small synthetic MNIST / CIFAR-10 files.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
REF = Path("/root/reference")
CPP = ROOT / "tensors_amd" / "cpp"
LIB = ROOT / "tensors_amd" / "lib"
SAN = ["-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-fno-sanitize-recover=undefined"]
SAN_ENV = {"ASAN_OPTIONS": "detect_leaks=1:verify_asan_link_order=0",
           "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"}


def _suites() -> list[Path]:
    if not (REF / "third_party" / "doctest" / "doctest.h").exists():
        return []
    out = []
    for top in ("tensor", "autograd", "nn", "data", "tests"):
        for f in sorted((REF / top).rglob("*_test.cpp")):
            if "cuda_runtime.h" not in f.read_text(errors="replace"):
                out.append(f)
    return out


SUITES = _suites()
pytestmark = pytest.mark.skipif(not SUITES, reason="the reference tree is not present")


def _name(f: Path) -> str:
    return str(f.relative_to(REF).with_suffix(""))


def _run(cmd, **kw):
    return subprocess.run(cmd, capture_output=True, text=True, **kw)


@pytest.fixture(scope="module")
def doctest_include(tmp_path_factory):
    # The suites include <doctest/doctest.h>; the reference keeps the header
    # at third_party/doctest/doctest.h (its build adds the prefix).
    d = tmp_path_factory.mktemp("doctest_inc")
    (d / "doctest").mkdir()
    (d / "doctest" / "doctest.h").symlink_to(REF / "third_party" / "doctest" / "doctest.h")
    return d


def _compile_all(out_dir: Path, inc: Path, libdir: Path, extra: list[str]) -> dict[str, tuple[Path, str]]:
    def one(f: Path):
        exe = out_dir / _name(f).replace("/", "__")
        r = _run(["g++", "-std=c++20", "-O1", "-g", *extra, f"-I{inc}", f"-I{CPP}", str(f), f"-L{libdir}",
                  "-ltensorforge", f"-Wl,-rpath,{libdir}", f"-Wl,-rpath,{LIB}", "-o", str(exe)])
        return _name(f), (exe if r.returncode == 0 else None, r.stderr[-3000:])
    with cf.ThreadPoolExecutor(max_workers=8) as ex:
        return dict(ex.map(one, SUITES))


@pytest.fixture(scope="module")
def plain_bins(tmp_path_factory, doctest_include):
    if not (LIB / "libtensorforge.so").exists():
        pytest.fail("libtensorforge.so is not built")
    return _compile_all(tmp_path_factory.mktemp("suites_plain"), doctest_include, LIB, [])


@pytest.fixture(scope="module")
def sanitized_bins(tmp_path_factory, doctest_include):
    """A sanitized libtensorforge.so from tensors_amd/cpp (the flags of
    tensors_amd/build.py plus the sanitizers), then every suite against it."""
    d = tmp_path_factory.mktemp("suites_san")
    srcs = sorted(CPP.rglob("*.cpp"))
    inc = [f"-I{ROOT / 'include'}", f"-I{CPP}"]

    def obj(s: Path):
        o = d / ("_".join(s.relative_to(CPP).with_suffix("").parts) + ".o")
        r = _run(["g++", "-std=c++20", "-O1", "-g", "-fPIC", *SAN, *inc, "-c", str(s), "-o", str(o)])
        assert r.returncode == 0, f"sanitized build of {s.name} failed:\n{r.stderr[-3000:]}"
        return str(o)
    with cf.ThreadPoolExecutor(max_workers=8) as ex:
        objs = list(ex.map(obj, srcs))
    r = _run(["g++", "-shared", *SAN, "-Wl,-Bsymbolic", "-o", str(d / "libtensorforge.so"), *objs, f"-L{LIB}",
              "-ltf_hip", f"-Wl,-rpath,{LIB}"])
    assert r.returncode == 0, r.stderr[-3000:]
    return _compile_all(d, doctest_include, d, SAN)


def _check(bins, name, env=None):
    exe, err = bins[name]
    assert exe is not None, f"{name} does not compile against tensors_amd/cpp:\n{err}"
    r = _run([str(exe)], timeout=300, env={**os.environ, **(env or {})})
    tail = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0 and "Status: SUCCESS" in r.stdout, f"{name} failed (rc {r.returncode}):\n{tail}"


@pytest.mark.parametrize("name", [_name(f) for f in SUITES])
def test_reference_suite_plain(plain_bins, name):
    _check(plain_bins, name)


@pytest.mark.parametrize("name", [_name(f) for f in SUITES])
def test_reference_suite_sanitized(sanitized_bins, name):
    _check(sanitized_bins, name, SAN_ENV)


def test_route_b_registrar_builds_against_the_reference_and_registers():
    """make -C oracle routeb: the INTEGRATION.md registrar block, the
    reference's objects, tests/route_b/route_b_check.cpp and libtf_hip.so.
    Run without a GPU, the check sees the registrar's static initialiser
    install the CUDA allocator and copy callback in the reference's
    allocator_dispatch."""
    r = _run(["make", "-s", "-C", str(ROOT / "oracle"), f"REF={REF}", "routeb"])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-3000:]
    exe = ROOT / "oracle" / "_ref" / "route_b_check"
    r = _run([str(exe), "registry"], timeout=60)
    assert r.returncode == 0 and "route B registry ok" in r.stdout, r.stdout + r.stderr
    reg = (ROOT / "oracle" / "_ref" / "tf_hip_registrar.cpp").read_text()
    for slot in ("register_cuda_add", "register_cuda_mul", "register_cuda_relu", "register_cuda_sigmoid",
                 "register_cuda_tanh", "register_cuda_leaky_relu", "register_allocator", "register_cuda_copy"):
        assert f"{slot}(" in reg, f"the registrar does not call {slot}"


def _write_mnist(d, n_train, n_test, seed):
    """Learnable synthetic MNIST: each image is its class's fixed random
    prototype plus noise, so the example's 95 % test-accuracy exit check
    (examples/train_mlp.cpp) can pass."""
    rng = np.random.default_rng(seed)
    proto = rng.integers(0, 256, (10, 784))
    for split, n in (("train", n_train), ("t10k", n_test)):
        y = rng.integers(0, 10, n)
        x = np.clip(proto[y] + rng.integers(-24, 25, (n, 784)), 0, 255).astype(np.uint8)
        hdr = np.array([0x803, n, 28, 28], ">u4").tobytes()
        (d / f"{split}-images-idx3-ubyte").write_bytes(hdr + x.tobytes())
        (d / f"{split}-labels-idx1-ubyte").write_bytes(np.array([0x801, n], ">u4").tobytes() +
                                                       y.astype(np.uint8).tobytes())


def _write_cifar(d, per_batch, seed):
    rng = np.random.default_rng(seed)
    for f in [f"data_batch_{i}.bin" for i in range(1, 6)] + ["test_batch.bin"]:
        recs = rng.integers(0, 256, (per_batch, 3073), dtype=np.uint8)
        recs[:, 0] = rng.integers(0, 10, per_batch)
        (d / f).write_bytes(recs.tobytes())


@pytest.mark.parametrize("example,env,writer", [
    ("train_mlp", "TENSORFORGE_MNIST_DIR", lambda d: _write_mnist(d, 256, 64, 5)),
    ("train_cnn", "TENSORFORGE_CIFAR_DIR", lambda d: _write_cifar(d, 16, 6)),
])
def test_reference_example_builds_and_runs(tmp_path, doctest_include, example, env, writer):
    """examples/<example>.cpp compiled unchanged against tensors_amd/cpp and
    libtensorforge.so, run on CPU tensors (as written) over small synthetic
    files in the on-disk formats.  train_mlp must train to its own 95 %
    test-accuracy exit check.  train_cnn loads the files and then stops, as
    it does against the reference itself: with padding 0 (the reference's
    Conv2dModule default, nn/Conv2dModule.hpp:17-19) its 32 x 32 inputs reach
    the flatten as [bs, 32, 14, 14], which it reshapes to [bs, 32 * 7 * 7]
    (examples/train_cnn.cpp:65-68, 96), and reshape throws
    std::invalid_argument on the element count (tensor/shape_ops.cpp)."""
    if not (LIB / "libtensorforge.so").exists():
        pytest.fail("libtensorforge.so is not built")
    src = REF / "examples" / f"{example}.cpp"
    exe = tmp_path / example
    r = _run(["g++", "-std=c++20", "-O2", f"-I{CPP}", str(src), f"-L{LIB}", "-ltensorforge", f"-Wl,-rpath,{LIB}",
              "-o", str(exe)])
    assert r.returncode == 0, r.stderr[-3000:]
    data = tmp_path / "data"
    data.mkdir()
    writer(data)
    r = _run([str(exe)], timeout=600, env={**os.environ, env: str(data)})
    if example == "train_mlp":
        assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-2000:])
        assert "final_test_acc=" in r.stdout
    else:
        assert "[train_cnn] train=80 test=16" in r.stdout, r.stdout[-2000:]
        assert r.returncode != 0 and "invalid_argument" in r.stderr and "reshape" in r.stderr, r.stderr[-2000:]
