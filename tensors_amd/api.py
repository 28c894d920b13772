"""ctypes binding of ``lib/libtensorforge.so``'s harness entry points
(``include/tfa_harness.h``), which drive the C++20 tensorforge API —
nn::Linear / Conv2dModule / CrossEntropyLoss, Tensor::backward through the
Engine, optim::SGD — on CPU tensors or on GPU 0.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from ._lib import LIB_DIR, lib as _hip_lib  # noqa: F401  (libtf_hip must load first)

TF_LIB_PATH = LIB_DIR / "libtensorforge.so"


class HarnessError(RuntimeError):
    pass


def _load() -> C.CDLL:
    if not TF_LIB_PATH.exists():
        raise ImportError(f"{TF_LIB_PATH} is missing: run __graft_entry__.build()")
    lib = C.CDLL(str(TF_LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
    lib.tfa_last_error.restype = C.c_char_p
    lib.tfa_selftest_names.restype = C.c_char_p
    lib.tfa_selftest.argtypes = [C.c_char_p, C.c_int32]
    lib.tfa_selftest.restype = C.c_int
    p, i64, i32, f = C.c_void_p, C.c_int64, C.c_int32, C.c_float
    lib.tfa_mlp_train.argtypes = [p, i32, i64, i64, i64, i64, p, p, f, f, i32, i32, i32, p, p, p, p, p, i32]
    lib.tfa_mlp_train.restype = C.c_int
    lib.tfa_mlp_step_trace.argtypes = [p, i32, i64, p, p, f, f, i32, i32, p, p, p, p, p, p]
    lib.tfa_mlp_step_trace.restype = C.c_int
    lib.tfa_cnn_train.argtypes = [i64, i64, i64, i64, i64, i64, p, p, f, f, i32, p, p, p, p]
    lib.tfa_cnn_train.restype = C.c_int
    lib.tfa_release_memory.argtypes = []
    lib.tfa_release_memory.restype = C.c_int
    return lib


lib = _load()


def _check(rc: int) -> None:
    if rc != 0:
        raise HarnessError(lib.tfa_last_error().decode(errors="replace"))


def _ptr(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def selftest_names() -> list[str]:
    return lib.tfa_selftest_names().decode().split()


def selftest(name: str, on_gpu: bool) -> None:
    _check(lib.tfa_selftest(name.encode(), int(on_gpu)))


def mlp_train(dims, xs, ys, *, steps, lr, mu, on_gpu, reference_compat=False, bf16=False, init_weights=None,
              warmup=0, want_weights=False, pool_trace=None, graph=0):
    """Returns (losses[steps], final_weights or None, ms_per_step).  With
    pool_trace a uint64 array [steps], it receives the device pool's bytes in
    use after each step (GPU only).  graph=1 replays a HIP graph of one step
    after the warmup steps (warmup >= 1, GPU only); graph=2 also waits for and
    reads every replay's loss before the next."""
    dims_a = np.ascontiguousarray(dims, dtype=np.int32)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    ys = np.ascontiguousarray(ys, dtype=np.int64)
    n_batches, batch = ys.shape
    assert xs.shape == (n_batches, batch, dims_a[0])
    losses = np.zeros(steps, np.float32)
    nw = int(sum(int(dims_a[i]) * int(dims_a[i + 1]) for i in range(len(dims_a) - 1)))
    fw = np.zeros(nw, np.float32) if want_weights else None
    iw = None if init_weights is None else np.ascontiguousarray(init_weights, dtype=np.float32)
    if iw is not None:
        assert iw.size == nw
    ms = C.c_double(0.0)
    if pool_trace is not None:
        assert pool_trace.dtype == np.uint64 and pool_trace.size == steps and pool_trace.flags["C_CONTIGUOUS"]
    _check(lib.tfa_mlp_train(_ptr(dims_a), len(dims_a), batch, steps, warmup, n_batches, _ptr(xs), _ptr(ys), lr, mu,
                             int(on_gpu), int(reference_compat), int(bf16), _ptr(iw), _ptr(losses), _ptr(fw),
                             C.byref(ms), _ptr(pool_trace), int(graph)))
    return losses, fw, ms.value


def mlp_step_trace(dims, x, y, *, lr, mu, on_gpu, bf16=False, init_weights=None):
    """One step of the MLP with biases (tfa_mlp_step_trace).  Returns
    (loss, acts, grads, weights, biases): acts[l] is layer l's input as its
    GEMM read it for l = 0 and layer l-1's output otherwise (l = 0 .. L),
    grads[l - 1] the gradient of acts[l] (l = 1 .. L), weights / biases the
    parameters after the SGD step; all float32 arrays."""
    dims_a = np.ascontiguousarray(dims, dtype=np.int32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.ascontiguousarray(y, dtype=np.int64)
    B = y.shape[0]
    assert x.shape == (B, dims_a[0])
    L = len(dims_a) - 1
    acts = np.empty(B * int(dims_a.astype(np.int64).sum()), np.float32)
    grads = np.empty(B * int(dims_a[1:].astype(np.int64).sum()), np.float32)
    nw = int(sum(int(dims_a[i]) * int(dims_a[i + 1]) for i in range(L)))
    fw, fb = np.empty(nw, np.float32), np.empty(int(dims_a[1:].astype(np.int64).sum()), np.float32)
    iw = None if init_weights is None else np.ascontiguousarray(init_weights, dtype=np.float32)
    loss = np.zeros(1, np.float32)
    _check(lib.tfa_mlp_step_trace(_ptr(dims_a), len(dims_a), B, _ptr(x), _ptr(y), lr, mu, int(on_gpu), int(bf16),
                                  _ptr(iw), _ptr(loss), _ptr(acts), _ptr(grads), _ptr(fw), _ptr(fb)))

    def split(flat, rows_of, cols_of, n):
        out, o = [], 0
        for i in range(n):
            k = rows_of(i) * cols_of(i)
            out.append(flat[o:o + k].reshape(rows_of(i), cols_of(i)))
            o += k
        return out

    d = [int(v) for v in dims_a]
    return (float(loss[0]), split(acts, lambda i: B, lambda i: d[i], L + 1),
            split(grads, lambda i: B, lambda i: d[i + 1], L),
            split(fw, lambda i: d[i + 1], lambda i: d[i], L), split(fb, lambda i: d[i + 1], lambda i: 1, L))


def release_memory():
    """Returns the GPU memory the harness holds unused (its block cache and
    the memory pool's free memory) to the driver (tfa_release_memory)."""
    _check(lib.tfa_release_memory())


def cnn_train(xs, ys, *, steps, lr, mu, on_gpu, init_params=None, warmup=0, want_params=False):
    """xs [n_batches, B, 3, H, W]; returns (losses, ms_per_step), or
    (losses, final_params, ms_per_step) with want_params (the six parameters
    concatenated: conv1.w, conv1.b, conv2.w, conv2.b, fc.w, fc.b)."""
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    ys = np.ascontiguousarray(ys, dtype=np.int64)
    n_batches, batch, _, H, W = xs.shape
    losses = np.zeros(steps, np.float32)
    ip = None if init_params is None else np.ascontiguousarray(init_params, dtype=np.float32)
    flat = 64 * (H // 2) * (W // 2)
    n_params = 32 * 27 + 32 + 64 * 288 + 64 + 10 * flat + 10
    fp = np.zeros(n_params, np.float32) if want_params else None
    if ip is not None:
        assert ip.size == n_params
    ms = C.c_double(0.0)
    _check(lib.tfa_cnn_train(batch, H, W, steps, warmup, n_batches, _ptr(xs), _ptr(ys), lr, mu, int(on_gpu), _ptr(ip),
                             _ptr(losses), _ptr(fp), C.byref(ms)))
    return (losses, fp, ms.value) if want_params else (losses, ms.value)
