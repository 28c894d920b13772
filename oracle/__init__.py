"""CPU oracle for tensorforge's training hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this package, and only as the checker (or the timed CPU
baseline); the product path never does.

* ``liboracle.so`` (``tf_oracle.c``): the C restatement of each reference
  function in the reference's own loop order and float32 arithmetic.
* ``_ref/libtfref.so`` (optional): the reference's own CPU implementation
  compiled from its sources by ``oracle/Makefile`` with ``ref_shim.cpp``; only
  present where the reference tree was available at build time.

How each function is pinned is described in oracle/README.md and tested in
tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "liboracle.so"
REF_SO = HERE / "_ref" / "libtfref.so"

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i64 = C.c_int64
_f = C.c_float


def build(ref: str = "/root/reference") -> None:
    """Compile liboracle.so (and _ref/libtfref.so when the reference exists)."""
    subprocess.run(["make", "-s", "-C", str(HERE), f"REF={ref}", "-j8"], check=True)


def _load_oracle() -> C.CDLL:
    if not ORACLE_SO.exists():
        build()
    lib = C.CDLL(str(ORACLE_SO))
    sig = {
        "orc_matmul": [_f32p, _f32p, _f32p, _i64, _i64, _i64],
        "orc_transpose2d": [_f32p, _f32p, _i64, _i64],
        "orc_add": [_f32p, _f32p, _f32p, _i64],
        "orc_mul": [_f32p, _f32p, _f32p, _i64],
        "orc_relu_fwd": [_f32p, _f32p, _i64],
        "orc_leaky_relu_fwd": [_f32p, _f32p, _i64, _f],
        "orc_sigmoid_fwd": [_f32p, _f32p, _i64],
        "orc_tanh_fwd": [_f32p, _f32p, _i64],
        "orc_relu_bwd": [_f32p, _f32p, _f32p, _i64],
        "orc_sigmoid_bwd": [_f32p, _f32p, _f32p, _i64],
        "orc_tanh_bwd": [_f32p, _f32p, _f32p, _i64],
        "orc_softmax_fwd": [_f32p, _f32p, _i64, _i64],
        "orc_log_softmax_fwd": [_f32p, _f32p, _i64, _i64],
        "orc_log_softmax_bwd": [_f32p, _f32p, _f32p, _i64, _i64],
        "orc_softmax_bwd": [_f32p, _f32p, _f32p, _i64, _i64],
        "orc_ce_chain": [_f32p, _i64p, _i64, _i64, _f32p, _f32p, C.c_void_p],
        "orc_colsum": [_f32p, _f32p, _i64, _i64],
        "orc_chansum_nchw": [_f32p, _f32p, _i64, _i64, _i64],
        "orc_sgd_momentum": [_f32p, _f32p, _f32p, _i64, _f, _f],
        "orc_layernorm_fwd": [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i64, _i64, _f],
        "orc_layernorm_bwd_stub": [_f32p, _f32p, _f32p, _f32p, _f32p, _i64, _i64],
        "orc_layernorm_bwd": [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i64, _i64],
        "orc_im2col": [_f32p, _f32p] + [_i64] * 12,
        "orc_col2im": [_f32p, _f32p] + [_i64] * 12,
        "orc_conv2d_fwd": [_f32p, _f32p, C.c_void_p, _f32p] + [_i64] * 10,
        "orc_conv2d_bwd": [_f32p, _f32p, C.c_int, _f32p, _f32p, _f32p, _f32p] + [_i64] * 13,
        "orc_argmax_rows": [_f32p, _i64p, _i64, _i64],
        "orc_sum_dim": [_f32p, _f32p, _i64, _i64, _i64],
        "orc_f32_to_f16": [_f32p, _u16p, _i64],
        "orc_f16_to_f32": [_u16p, _f32p, _i64],
    }
    lib.orc_ce_module.argtypes = [_f32p, _i64p, _i64, _i64, _f32p, _f32p]
    lib.orc_ce_module.restype = C.c_int
    for name, args in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = None
    return lib


lib = _load_oracle()


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32)


# --------------------------------------------------------------------------
# Reference-order float32 functions (tf_oracle.c)
# --------------------------------------------------------------------------
def matmul(a, b):
    a, b = _f32(a), _f32(b)
    M, K = a.shape
    K2, N = b.shape
    assert K == K2
    c = np.empty((M, N), np.float32)
    lib.orc_matmul(a, b, c, M, K, N)
    return c


def transpose2d(x):
    x = _f32(x)
    out = np.empty((x.shape[1], x.shape[0]), np.float32)
    lib.orc_transpose2d(x, out, x.shape[0], x.shape[1])
    return out


def linear_fwd(x, w):
    """nn::Linear forward y = x @ transpose(W) (nn/Linear.cpp:60-63)."""
    return matmul(x, transpose2d(w))


def linear_bwd(x, w, dy):
    """MatmulBackward + TransposeBackward of Linear: dX = dY @ W, dW = (X^T @ dY)^T."""
    dx = matmul(dy, w)
    dw = transpose2d(matmul(transpose2d(x), dy))
    return dx, dw


def f32_to_f16_bits(x):
    """IEEE binary16 bit patterns of float32 values, round to nearest even
    (the reference's __float2half)."""
    x = _f32(x)
    h = np.empty(x.shape, np.uint16)
    lib.orc_f32_to_f16(x.reshape(-1), h.reshape(-1), x.size)
    return h


def f16_bits_to_f32(h):
    """float32 values of IEEE binary16 bit patterns (exact)."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    x = np.empty(h.shape, np.float32)
    lib.orc_f16_to_f32(h.reshape(-1), x.reshape(-1), h.size)
    return x


def _unary(fn, x):
    x = _f32(x)
    y = np.empty_like(x)
    fn(x.reshape(-1), y.reshape(-1), x.size)
    return y


def relu(x):
    return _unary(lib.orc_relu_fwd, x)


def leaky_relu(x, alpha):
    x = _f32(x)
    y = np.empty_like(x)
    lib.orc_leaky_relu_fwd(x.reshape(-1), y.reshape(-1), x.size, alpha)
    return y


def sigmoid(x):
    return _unary(lib.orc_sigmoid_fwd, x)


def tanh(x):
    return _unary(lib.orc_tanh_fwd, x)


def _binary(fn, a, b):
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    fn(a.reshape(-1), b.reshape(-1), out.reshape(-1), a.size)
    return out


def add(a, b):
    return _binary(lib.orc_add, a, b)


def relu_bwd(dy, x):
    return _binary(lib.orc_relu_bwd, dy, x)


def sigmoid_bwd(dy, y):
    return _binary(lib.orc_sigmoid_bwd, dy, y)


def tanh_bwd(dy, y):
    return _binary(lib.orc_tanh_bwd, dy, y)


def _rows(fn, x):
    x = _f32(x)
    y = np.empty_like(x)
    fn(x, y, x.shape[0], x.shape[1])
    return y


def log_softmax(x):
    return _rows(lib.orc_log_softmax_fwd, x)


def softmax(x):
    return _rows(lib.orc_softmax_fwd, x)


def log_softmax_bwd(y, dy):
    y, dy = _f32(y), _f32(dy)
    dx = np.empty_like(y)
    lib.orc_log_softmax_bwd(y, dy, dx, y.shape[0], y.shape[1])
    return dx


def softmax_bwd(y, dy):
    y, dy = _f32(y), _f32(dy)
    dx = np.empty_like(y)
    lib.orc_softmax_bwd(y, dy, dx, y.shape[0], y.shape[1])
    return dx


def ce_chain(logits, labels):
    """(loss, dlogits) of the train_mlp cross-entropy chain and its backward."""
    logits = _f32(logits)
    labels = np.ascontiguousarray(labels, dtype=np.int64)
    loss = np.zeros(1, np.float32)
    d = np.empty_like(logits)
    lib.orc_ce_chain(logits, labels, logits.shape[0], logits.shape[1], loss, d, None)
    return float(loss[0]), d


def ce_module(logits, labels):
    """Loss of nn::CrossEntropyLoss::forward (probability clamped at 1e-9);
    raises IndexError for a target outside [0, C), as the reference throws."""
    logits = _f32(logits)
    labels = np.ascontiguousarray(labels, dtype=np.int64)
    loss = np.zeros(1, np.float32)
    probs = np.empty_like(logits)
    if lib.orc_ce_module(logits, labels, logits.shape[0], logits.shape[1], loss, probs) != 0:
        raise IndexError("CrossEntropyLoss: target index out of range")
    return float(loss[0])


def colsum(dy):
    dy = _f32(dy)
    db = np.empty(dy.shape[1], np.float32)
    lib.orc_colsum(dy, db, dy.shape[0], dy.shape[1])
    return db


def chansum_nchw(dy):
    dy = _f32(dy)
    N, Cc, H, W = dy.shape
    db = np.empty(Cc, np.float32)
    lib.orc_chansum_nchw(dy, db, N, Cc, H * W)
    return db


def sgd_momentum(p, g, v, lr, mu):
    """Returns updated (p, v) copies."""
    p, g, v = _f32(p).copy(), _f32(g), _f32(v).copy()
    lib.orc_sgd_momentum(p.reshape(-1), g.reshape(-1), v.reshape(-1), p.size, lr, mu)
    return p, v


def layernorm_fwd(x, gamma, beta, eps=1e-5):
    x, gamma, beta = _f32(x), _f32(gamma), _f32(beta)
    R, Cc = x.shape
    y = np.empty_like(x)
    mean = np.empty(R, np.float32)
    rstd = np.empty(R, np.float32)
    lib.orc_layernorm_fwd(x, gamma, beta, y, mean, rstd, R, Cc, eps)
    return y, mean, rstd


def layernorm_bwd_stub(dy, gamma):
    dy, gamma = _f32(dy), _f32(gamma)
    R, Cc = dy.shape
    dx = np.empty_like(dy)
    dg = np.empty(Cc, np.float32)
    db = np.empty(Cc, np.float32)
    lib.orc_layernorm_bwd_stub(dy, gamma, dx, dg, db, R, Cc)
    return dx, dg, db


def layernorm_bwd(x, dy, gamma, mean, rstd):
    x, dy, gamma, mean, rstd = map(_f32, (x, dy, gamma, mean, rstd))
    R, Cc = x.shape
    dx = np.empty_like(x)
    dg = np.empty(Cc, np.float32)
    db = np.empty(Cc, np.float32)
    lib.orc_layernorm_bwd(x, dy, gamma, mean, rstd, dx, dg, db, R, Cc)
    return dx, dg, db


def conv_out(H, k, s, p, d):
    return (H + 2 * p - d * (k - 1) - 1) // s + 1


def im2col(x, kH, kW, sh=1, sw=1, ph=0, pw=0, dh=1, dw=1):
    x = _f32(x)
    N, Cc, H, W = x.shape
    oh, ow = conv_out(H, kH, sh, ph, dh), conv_out(W, kW, sw, pw, dw)
    col = np.empty((N, Cc * kH * kW, oh * ow), np.float32)
    lib.orc_im2col(x, col, N, Cc, H, W, kH, kW, sh, sw, ph, pw, dh, dw)
    return col


def col2im(col, shape, kH, kW, sh=1, sw=1, ph=0, pw=0, dh=1, dw=1):
    col = _f32(col)
    N, Cc, H, W = shape
    dx = np.empty(shape, np.float32)
    lib.orc_col2im(col, dx, N, Cc, H, W, kH, kW, sh, sw, ph, pw, dh, dw)
    return dx


def conv2d_fwd(x, w, b=None, stride=1, pad=0, dil=1):
    x, w = _f32(x), _f32(w)
    N, Cin, H, W = x.shape
    Cout, _, kH, kW = w.shape
    oh = (H + 2 * pad - (dil * (kH - 1) + 1)) // stride + 1
    ow = (W + 2 * pad - (dil * (kW - 1) + 1)) // stride + 1
    y = np.empty((N, Cout, oh, ow), np.float32)
    bb = _f32(b) if b is not None else None
    lib.orc_conv2d_fwd(x, w, bb.ctypes.data if bb is not None else None, y, N, Cin, H, W, Cout, kH, kW,
                       stride, pad, dil)
    return y


def conv2d_bwd(x, w, gout, stride=(1, 1), pad=(0, 0), dil=(1, 1), has_bias=True):
    x, w, gout = _f32(x), _f32(w), _f32(gout)
    N, Cin, H, W = x.shape
    Cout, _, kH, kW = w.shape
    gin = np.empty_like(x)
    gw = np.empty_like(w)
    gb = np.empty(Cout, np.float32)
    lib.orc_conv2d_bwd(x, w, int(has_bias), gout, gin, gw, gb, N, Cin, H, W, Cout, kH, kW,
                       stride[0], stride[1], pad[0], pad[1], dil[0], dil[1])
    return gin, gw, gb


def sum_dim(x, outer, reduce, inner):
    """Tensor::sum along the middle dim of x viewed as [outer][reduce][inner]."""
    x = _f32(x).reshape(-1)
    assert x.size == outer * reduce * inner
    out = np.empty(outer * inner, np.float32)
    lib.orc_sum_dim(x, out, outer, reduce, inner)
    return out.reshape(outer, inner)


def argmax_rows(x):
    x = _f32(x)
    out = np.empty(x.shape[0], np.int64)
    lib.orc_argmax_rows(x, out, x.shape[0], x.shape[1])
    return out


# --------------------------------------------------------------------------
# Composite: one config-1 style training step in reference order.
# --------------------------------------------------------------------------
def mlp_step(weights, vels, x, labels, lr, mu):
    """Forward (Linear-ReLU-...-Linear), chain CE, backward, momentum SGD.

    Mirrors the reference graph: per layer Wt = transpose(W), h = x @ Wt,
    ReLU between layers; backward dX = dY @ W, dW = transpose(X^T @ dY),
    ReluBackward dy * mask.  Updates weights/vels in place; returns the loss.
    """
    acts = [_f32(x)]
    pre = []
    h = acts[0]
    for li, w in enumerate(weights):
        z = linear_fwd(h, w)
        pre.append(z)
        h = relu(z) if li + 1 < len(weights) else z
        acts.append(h)
    loss, g = ce_chain(h, labels)
    grads = [None] * len(weights)
    for li in range(len(weights) - 1, -1, -1):
        if li + 1 < len(weights):
            g = relu_bwd(g, pre[li])
        dx, dw = linear_bwd(acts[li], weights[li], g)
        grads[li] = dw
        g = dx
    for li in range(len(weights)):
        p, v = sgd_momentum(weights[li], grads[li], vels[li], lr, mu)
        weights[li][...] = p
        vels[li][...] = v
    return loss


def bf16_round(x):
    """Nearest bfloat16 value of each float32 (ties to even), as float32.

    bfloat16 keeps the top 16 bits of a float32; rounding adds 0x7FFF plus
    the lowest kept bit and truncates.  Finite inputs only: a finite value
    never carries past +/-inf (0x7F7FFFFF + 0x8000 = 0x7F807FFF -> inf).
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    with np.errstate(over="ignore"):
        r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    return r.view(np.float32)


def _no_round(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def mlp_step_mixed(weights, biases, vels, bvels, x, labels, lr, mu, rounding=True, trace=None):
    """One step of the mixed-precision MLP (config 5): bf16 operands and
    activations, float32 accumulation, float32 master weights.

    The reference has no bf16 path (tensor/Tensor.cpp:344-346); this restates
    its graph (nn/Linear.cpp:45-64 forward, Linear+ReLU layers, the
    cross-entropy of examples/train_mlp.cpp:54-76, the momentum rule of
    nn/optim/SGD.hpp:3-6) with a bf16 rounding at each point where the mixed
    precision step stores a bf16 tensor:
      * the input and each weight's working copy: bf16(x), bf16(W);
      * each layer's output: bf16(relu(acc + b)) (the last layer without
        the ReLU); acc is the float32 sum over bf16 products;
      * the loss gradient: dlogits = (softmax - onehot)/N in float32, then
        bf16 for the backward GEMMs;
      * dX = bf16(dY16 @ W16), masked by the layer input's ReLU (y > 0);
      * dW = dY16^T @ X16 and db = colsum(dY16), both kept in float32;
      * SGD on the float32 masters: v = mu*v + g, p = p - lr*v, each
        operation rounded to float32.
    `rounding=False` turns every bf16 rounding into the identity, which
    leaves the float32 step (then equal to mlp_step up to summation order).
    Products run through numpy's float32 BLAS (float32 accumulation, in
    another order than the GPU).  weights/biases/vels/bvels are updated in
    place (biases[l] may be None: no bias); returns the loss.  With `trace` a
    dict, the step's stored tensors go into it: "w16" (working weights),
    "acts" (the input and every layer's output), "dlogits", "dx" (each
    layer's data gradient before the mask, layers 1 .. L-1), "dw" and "db"
    (each layer's parameter gradients), all float32.
    """
    rnd = bf16_round if rounding else _no_round
    L = len(weights)
    w16 = [rnd(w) for w in weights]
    h = rnd(x)
    acts = [h]
    for li in range(L):
        z = h @ w16[li].T
        if biases[li] is not None:
            z = z + _f32(biases[li])
        if li + 1 < L:
            z = np.maximum(z, np.float32(0))
        h = rnd(z)
        acts.append(h)
    logits = acts[-1].astype(np.float64)
    labels = np.asarray(labels, dtype=np.int64)
    N = logits.shape[0]
    rows = np.arange(N)
    mx = logits.max(axis=1, keepdims=True)
    e = np.exp(logits - mx)
    s = e.sum(axis=1, keepdims=True)
    lse = mx[:, 0] + np.log(s[:, 0])
    loss = float(np.mean(lse - logits[rows, labels]))
    g = e / s
    g[rows, labels] -= 1.0
    g /= N
    g = rnd(g.astype(np.float32))
    if trace is not None:
        trace.update(w16=w16, acts=acts, dlogits=g, dx=[None] * L, dw=[None] * L, db=[None] * L)
    f_lr, f_mu = np.float32(lr), np.float32(mu)

    def sgd(p, grad, v):
        if mu != 0.0:
            v[...] = f_mu * v + grad
            p[...] = p - f_lr * v
        else:
            p[...] = p - f_lr * grad

    for li in range(L - 1, -1, -1):
        dw = (g.T @ acts[li]).astype(np.float32)
        db = g.astype(np.float64).sum(axis=0).astype(np.float32)
        if trace is not None:
            trace["dw"][li], trace["db"][li] = dw, db
        if li > 0:
            dh = rnd(g @ w16[li])
            if trace is not None:
                trace["dx"][li] = dh
            g = np.where(acts[li] > 0, dh, np.float32(0)).astype(np.float32)
        sgd(weights[li], dw, vels[li])
        if biases[li] is not None:
            sgd(biases[li], db, bvels[li])
    return loss


def cnn_step(params, vels, x, labels, lr, mu):
    """One config-4 training step in reference order: Conv(3->32, s1 p1) +
    ReLU, Conv(32->64, s2 p1) + ReLU, flatten, Linear(+bias), CE chain;
    backward through the reference's conv loop (nn/conv2d_backward_test.cpp:
    50-106), Linear backward and ReluBackward; momentum SGD on all six
    parameters (updated in place).  params = [w1, b1, w2, b2, wf, bf]."""
    w1, b1, w2, b2, wf, bfc = params
    x = _f32(x)
    B = x.shape[0]
    z1 = conv2d_fwd(x, w1, b1, 1, 1)
    h1 = relu(z1)
    z2 = conv2d_fwd(h1, w2, b2, 2, 1)
    h2 = relu(z2)
    f = h2.reshape(B, -1)
    logits = add(linear_fwd(f, wf), np.broadcast_to(bfc, (B, bfc.size)))
    loss, g = ce_chain(logits, labels)
    df, dwf = linear_bwd(f, wf, g)
    dbf = colsum(g)
    dz2 = relu_bwd(df.reshape(h2.shape), z2)
    dh1, dw2, db2 = conv2d_bwd(h1, w2, dz2, (2, 2), (1, 1), (1, 1))
    dz1 = relu_bwd(dh1, z1)
    _, dw1, db1 = conv2d_bwd(x, w1, dz1, (1, 1), (1, 1), (1, 1))
    for i, gr in enumerate((dw1, db1, dw2, db2, dwf, dbf)):
        p, v = sgd_momentum(params[i], gr, vels[i], lr, mu)
        params[i][...] = p
        vels[i][...] = v
    return loss


# --------------------------------------------------------------------------
# The compiled reference (optional)
# --------------------------------------------------------------------------
_ref = None


def ref_available() -> bool:
    return REF_SO.exists()


def ref():
    """ctypes handle on _ref/libtfref.so (raises if it was not built)."""
    global _ref
    if _ref is None:
        if not REF_SO.exists():
            raise FileNotFoundError(f"{REF_SO} not built (needs the reference tree)")
        r = C.CDLL(str(REF_SO), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        r.ref_last_error.restype = C.c_char_p
        for name in ("ref_matmul", "ref_transpose2d", "ref_matmul_backward", "ref_linear", "ref_linear_init",
                     "ref_conv2d_init", "ref_relu_fwd", "ref_leaky_relu_fwd", "ref_sigmoid_fwd", "ref_tanh_fwd", "ref_relu_bwd",
                     "ref_log_softmax_fwd", "ref_softmax_fwd", "ref_log_softmax_bwd", "ref_softmax_bwd",
                     "ref_sum", "ref_add", "ref_layernorm_fwd", "ref_layernorm_bwd", "ref_ce_chain",
                     "ref_ce_module", "ref_conv2d_fwd", "ref_mlp_train"):
            getattr(r, name).restype = C.c_int
        _ref = r
    return _ref


def ref_call(name: str, *args) -> None:
    """Call ref_<name> with numpy arrays as pointers, ints as int64, floats as float."""
    r = ref()
    final = []
    for a in args:
        if isinstance(a, np.ndarray):
            assert a.flags["C_CONTIGUOUS"]
            final.append(C.c_void_p(a.ctypes.data))
        elif isinstance(a, (bool, np.bool_)):
            raise TypeError("bool argument")
        elif isinstance(a, (int, np.integer)):
            final.append(C.c_int64(int(a)))
        elif isinstance(a, (float, np.floating)):
            final.append(C.c_float(float(a)))
        else:
            final.append(a)
    if getattr(r, name)(*final) != 0:
        raise RuntimeError(f"{name}: {r.ref_last_error().decode()}")
