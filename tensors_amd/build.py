"""Build the in-tree native libraries.

* ``tensors_amd/lib/libtf_hip.so`` — the HIP kernels and the C ABI declared in
  ``include/tf_hip.h``, compiled for gfx950 only with ``hipcc``.
* ``tensors_amd/lib/libtf_hbm_probe.so`` — the HBM streaming-ceiling
  microbenchmark (``csrc/probe/hbm_ceiling.hip``), used by ``bench.py
  --hbm-ceiling``.
* ``tensors_amd/lib/libtensorforge.so`` — the C++20 tensorforge API
  (Tensor / autograd Engine / nn / optim) that dispatches device tensors to
  libtf_hip.so; compiled with ``g++`` (no HIP headers involved).

Objects are built in parallel into ``tensors_amd/_build/`` and every call
rebuilds (the driver's "does it build" check relies on that).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
CPP = PKG / "cpp"
LIB = PKG / "lib"
BUILD = PKG / "_build"
INCLUDE = ROOT / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-FP32 instructions are disabled: some of their forms have produced
# silently wrong results on these GPUs.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Private arrays stay in registers or scratch; never silently in LDS (the
    # GEMM kernels size their LDS to one workgroup per CU).
    "-mllvm", "-disable-promote-alloca-to-lds",
    "-Wno-unused-command-line-argument", "-Wno-inline-asm",
    f"-I{INCLUDE}", f"-I{CSRC}",
]

CXX = os.environ.get("CXX", "g++")
CXX_FLAGS = ["-std=c++20", "-O2", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
             f"-I{INCLUDE}", f"-I{CPP}"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {cmd[0]} ... {cmd[-1]}")


def build_hip(jobs: int = 8, defines: tuple[str, ...] = (), out: Path | None = None,
              build_dir: Path = BUILD) -> Path:
    build_dir.mkdir(parents=True, exist_ok=True)
    LIB.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    objs = [build_dir / (s.stem + ".hip.o") for s in srcs]
    dflags = [f"-D{d}" for d in defines]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, [HIPCC, *HIP_FLAGS, *dflags, "-c", str(s), "-o", str(o)]) for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    out = out or LIB / "libtf_hip.so"
    out.parent.mkdir(parents=True, exist_ok=True)
    tmp = out.with_name(out.name + ".tmp")
    # Every build is named libtf_hip.so to the loader, so a variant loaded
    # first (TF_HIP_LIBRARY) also serves libtensorforge.so's dependency.
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-soname,libtf_hip.so", "-o", str(tmp),
          *map(str, objs)])
    os.replace(tmp, out)
    return out


def build_cpp(jobs: int = 8) -> Path | None:
    srcs = sorted(CPP.rglob("*.cpp"))
    if not srcs:
        return None
    BUILD.mkdir(exist_ok=True)
    objs = [BUILD / ("cpp_" + "_".join(s.relative_to(CPP).with_suffix("").parts) + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, [CXX, *CXX_FLAGS, "-c", str(s), "-o", str(o)]) for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    out = LIB / "libtensorforge.so"
    tmp = LIB / "libtensorforge.so.tmp"
    # -Bsymbolic: internal calls bind to this library's own definitions.
    _run([CXX, "-shared", "-fPIC", "-Wl,-Bsymbolic", "-o", str(tmp), *map(str, objs),
          f"-L{LIB}", "-ltf_hip", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)
    return out


def build_probe() -> Path:
    """libtf_hbm_probe.so: the HBM streaming-ceiling microbenchmark
    (csrc/probe/), a measuring instrument kept out of libtf_hip.so."""
    LIB.mkdir(exist_ok=True)
    out = LIB / "libtf_hbm_probe.so"
    tmp = LIB / "libtf_hbm_probe.so.tmp"
    _run([HIPCC, *HIP_FLAGS, "-shared", "-o", str(tmp), str(CSRC / "probe" / "hbm_ceiling.hip")])
    os.replace(tmp, out)
    return out


def build(jobs: int = 8) -> None:
    with cf.ThreadPoolExecutor(max_workers=2) as ex:
        probe = ex.submit(build_probe)
        build_hip(jobs)
        probe.result()
    build_cpp(jobs)


def build_variant(define: str) -> Path:
    """A kernel-variant build of libtf_hip.so with one extra -D (e.g.
    TF_BF16_KERNEL=1), at lib/variants/libtf_hip_<NAME>_<VALUE>.so; load it
    with TF_HIP_LIBRARY=<that path>."""
    tag = define.replace("=", "_").lower()
    return build_hip(defines=(define,), out=LIB / "variants" / f"libtf_hip_{tag}.so",
                     build_dir=BUILD / f"variant_{tag}")


if __name__ == "__main__":
    import argparse
    ap = argparse.ArgumentParser(prog="python -m tensors_amd.build")
    ap.add_argument("--variant", help="build only a kernel-variant libtf_hip.so with this -D (NAME=VALUE)")
    a = ap.parse_args()
    if a.variant:
        print("built:", build_variant(a.variant))
    else:
        build()
        print("built:", *sorted(p.name for p in LIB.glob("*.so")))
