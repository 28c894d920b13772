"""Full-size parity of the two largest configurations on GPU 0.

Config 5 (wide MLP, bf16 operands and activations, fp32 accumulation and
fp32 master weights, through the C++ API) is checked three ways:
  * reduced dims, three steps, against the mixed-precision oracle
    (oracle.mlp_step_mixed: the reference's graph with bf16 roundings where
    the GPU stores bf16), losses and weight updates within the bf16 bar;
  * the full 4096-8192-8192-4096-1000 step at batch 4096 against the same
    oracle run at full size (float32 BLAS on the host);
  * the full step elementwise: every layer's output, weight gradient (on
    sampled rows), whole bias gradient, data gradient and the logits'
    gradient against float64 recomputed from the step's own stored bf16
    operands (check_step_trace), so each GEMM and sum of the step is judged
    at fp32 accuracy or one bf16 rounding, not by a norm;
  * every GEMM of the full step, at its exact shape, layout and epilogue,
    against float64 on sampled output rows.
Config 4 (CNN, batch 128) runs a full-batch step against the reference-order
oracle step (the reference's own conv backward loop, restated).

Bars: rtol 2e-2 for bf16 results, 1e-4 for fp32 results, atol = rtol * rms,
elementwise wherever GPU and oracle see the same inputs (each GEMM, the
losses, the step trace, whose bf16 bar is one rounding).  Against the
host-side oracle's own step, a whole bf16 training step is judged per layer
by the relative
Frobenius norm of the weight update (<= 2e-2): bf16 storage turns the
different float32 summation orders of GPU and host into occasional
one-ulp differences of logits and activations (0.4-0.8 %) and rare ReLU
mask differences, which move single gradient entries by a large fraction of
the update's rms.  Measured on the host with the oracle alone: perturbing
the reduced config's input by a relative 1e-7 moves single entries of the
one-step update by up to 0.84 rms but the update as a whole by 0.8 % (2.6 %
after three steps, hence one step for the update and three for the loss).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tensors_amd import api, synth
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu

RTOL16 = 2e-2
RTOL32 = 1e-4
C5 = [4096, 8192, 8192, 4096, 1000]


def _rng_normal(seed, shape, std=1.0):
    """Fast seeded N(0, std) float32 (numpy PCG64) for multi-GB test inputs."""
    return (np.random.default_rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(std))


def _mlp_init(dims, seed):
    return [_rng_normal(seed + i, (dims[i + 1], dims[i]), std=float(dims[i]) ** -0.5) for i in range(len(dims) - 1)]


def _split(flat, dims):
    out, off = [], 0
    for i in range(len(dims) - 1):
        n = dims[i] * dims[i + 1]
        out.append(flat[off:off + n].reshape(dims[i + 1], dims[i]))
        off += n
    return out


def assert_rel_norm(got, want, tol, what):
    """||got - want|| <= tol * ||want|| (Frobenius, float64)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    rel = float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-300))
    assert rel <= tol, f"{what}: relative norm error {rel:.3g} > {tol}"


def _sample(n, count, seed):
    return np.unique(np.random.default_rng(seed).integers(0, n, count))


# ---------------------------------------------------------------------------
# config 5
# ---------------------------------------------------------------------------
def test_c5_reduced_bf16_steps_match_mixed_oracle(ctx):
    """[512, 1024, 1024, 512, 100], batch 256, biases on (zero init): three
    bf16 steps through nn::Linear / CrossEntropyLoss / SGD on the GPU against
    the mixed-precision oracle: every step's loss, and each layer's weight
    update after the first step."""
    dims = [512, 1024, 1024, 512, 100]
    B, steps = 256, 3
    xs = synth.normal(synth.seed(5, 0), (steps, B, dims[0]))
    ys = synth.uniform_int(synth.seed(5, 1), (steps, B), dims[-1])
    w0 = _mlp_init(dims, 5100)
    init = np.concatenate([w.ravel() for w in w0])
    lr, mu = 0.1, 0.9
    losses, _, _ = api.mlp_train(dims, xs, ys, steps=steps, lr=lr, mu=mu, on_gpu=True, bf16=True,
                                 init_weights=init)
    _, fw1, _ = api.mlp_train(dims, xs, ys, steps=1, lr=lr, mu=mu, on_gpu=True, bf16=True, init_weights=init,
                              want_weights=True)
    ws = [w.copy() for w in w0]
    bs = [np.zeros(dims[i + 1], np.float32) for i in range(len(dims) - 1)]
    vs = [np.zeros_like(w) for w in ws]
    bv = [np.zeros_like(b) for b in bs]
    ref = []
    for s in range(steps):
        ref.append(oracle.mlp_step_mixed(ws, bs, vs, bv, xs[s], ys[s], lr, mu))
        if s == 0:
            for i, (g, w) in enumerate(zip(_split(fw1, dims), ws)):
                assert_rel_norm(g.astype(np.float64) - w0[i], w.astype(np.float64) - w0[i], RTOL16,
                                f"layer {i} update after one step")
    assert np.all(np.isfinite(losses))
    assert_close(losses, ref, RTOL16, "losses")


def test_c5_full_size_step_matches_mixed_oracle(ctx):
    """The benchmark's config-5 step at full size (4096-8192-8192-4096-1000,
    batch 4096, 138 M weights) on the GPU against the mixed-precision oracle
    run at full size on the host: the loss (near ln 1000 at this init) and
    every layer's weight update.  lr = 1, mu = 0, so the update is the
    gradient itself."""
    B = 4096
    x = _rng_normal(5200, (1, B, C5[0]))
    y = np.random.default_rng(5201).integers(0, C5[-1], (1, B)).astype(np.int64)
    w0 = _mlp_init(C5, 5210)
    init = np.concatenate([w.ravel() for w in w0])
    losses, fw, _ = api.mlp_train(C5, x, y, steps=1, lr=1.0, mu=0.0, on_gpu=True, bf16=True, init_weights=init,
                                  want_weights=True)
    del init
    ws = [w.copy() for w in w0]
    bs = [np.zeros(C5[i + 1], np.float32) for i in range(4)]
    ref = oracle.mlp_step_mixed(ws, bs, [np.zeros(1, np.float32)] * 4, [np.zeros(1, np.float32)] * 4, x[0], y[0],
                                1.0, 0.0)
    assert np.isfinite(losses[0]) and abs(float(losses[0]) - np.log(1000.0)) < 0.5, losses[0]
    assert abs(float(losses[0]) - ref) <= RTOL16 * abs(ref), (float(losses[0]), ref)
    for i, (g, w) in enumerate(zip(_split(fw, C5), ws)):
        assert_rel_norm(g.astype(np.float64) - w0[i], w.astype(np.float64) - w0[i], RTOL16, f"layer {i} gradient")


def check_step_trace(dims, B, bf16, seed):
    """One step through the C++ API (tfa_mlp_step_trace: biases on, lr = 1,
    mu = 0, so each parameter's change is its gradient), judged elementwise
    against float64 computed from the step's own stored operands: each
    layer's output on sampled rows, its weight gradient on sampled rows, its
    whole bias gradient, the data gradient it passes down on sampled rows,
    the logits' gradient and the loss.  Because the truth starts from the
    same (bf16) operands the GPU multiplied, the GEMMs' and sums' own errors
    are judged, not bf16 rounding chaos upstream:
      * fp32 results (dW, db, and all of an fp32 step): rtol 1e-4,
        atol = 1e-4 * rms;
      * bf16 results (layer outputs, dX, dlogits): one rounding to bf16,
        |err| <= 2^-8 |truth| (a bf16 step at most) + 1e-4 * rms."""
    import tensors_amd as ta
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, dims[0]), dtype=np.float32)
    y = rng.integers(0, dims[-1], B).astype(np.int64)
    w0 = _mlp_init(dims, seed + 1)
    init = np.concatenate([w.ravel() for w in w0])
    loss, acts, grads, fw, fb = api.mlp_step_trace(dims, x, y, lr=1.0, mu=0.0, on_gpu=True, bf16=bf16,
                                                   init_weights=init)
    del init
    L = len(dims) - 1
    rnd = (lambda a: ta.bf16_bits_to_f32(ta.f32_to_bf16_bits(a))) if bf16 else (lambda a: a)

    def close16(got, truth, what):
        if not bf16:
            assert_close(got, truth, RTOL32, what)
            return
        got, truth = np.asarray(got, np.float64), np.asarray(truth, np.float64)
        atol = RTOL32 * np.sqrt(np.mean(truth ** 2))
        bad = np.abs(got - truth) > 2.0 ** -8 * np.abs(truth) + atol
        assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} beyond one bf16 rounding"

    if bf16:
        np.testing.assert_array_equal(acts[0], rnd(x))           # the input as the first GEMM read it
    else:
        np.testing.assert_array_equal(acts[0], x)
    # logits' gradient and the loss, from the stored logits
    lg = acts[L].astype(np.float64)
    m = lg.max(1, keepdims=True)
    e = np.exp(lg - m)
    lse = m[:, 0] + np.log(e.sum(1))
    assert abs(loss - float(np.mean(lse - lg[np.arange(B), y]))) <= RTOL32 * abs(loss)
    p_ = e / e.sum(1, keepdims=True)
    p_[np.arange(B), y] -= 1.0
    close16(grads[L - 1], p_ / B, "dlogits")
    del lg, e, p_
    for l in range(L, 0, -1):
        i = l - 1
        a_in = acts[i].astype(np.float64)
        wq = rnd(w0[i]).astype(np.float64)                       # the weight as the GEMMs read it
        dz = grads[l - 1] if l == L else np.where(acts[l] > 0, grads[l - 1], np.float32(0))
        rows = np.unique(np.concatenate([[0, B - 1], _sample(B, 62, seed + 10 * l)]))
        z = a_in[rows] @ wq.T
        close16(acts[l][rows], np.maximum(z, 0.0) if l < L else z, f"layer {l} output, sampled rows")
        orows = np.unique(np.concatenate([[0, dims[l] - 1], _sample(dims[l], 62, seed + 10 * l + 1)]))
        dw = w0[i][orows].astype(np.float64) - fw[i][orows]
        assert_close(dw, dz[:, orows].T.astype(np.float64) @ a_in, RTOL32, f"layer {l} dW, sampled rows")
        assert_close(-fb[i].ravel(), dz.astype(np.float64).sum(0), RTOL32, f"layer {l} db")
        if i >= 1:
            close16(grads[i - 1][rows], dz[rows].astype(np.float64) @ wq, f"layer {l} dX, sampled rows")
        del a_in, dz


def test_c5_full_size_step_elementwise_vs_float64(ctx):
    """Config 5's step at full size (4096-8192-8192-4096-1000, batch 4096,
    bf16 compute, biases on): every GEMM output, weight and bias gradient of
    the step elementwise against float64 of the step's own operands."""
    check_step_trace(C5, 4096, True, 5300)


def test_c2_like_fp32_step_elementwise_vs_float64(ctx):
    """The same check on an fp32 step (one 2048 -> 2048 layer before a
    2048 -> 10 output layer, batch 2048: config 2's Linear inside a step)."""
    check_step_trace([2048, 2048, 10], 2048, False, 5310)


# (M, N, K, trans_a, trans_b, out, epilogue) of every GEMM in the config-5
# step: y = x W^T (+b, ReLU) in bf16, dX = dY W in bf16, dW = dY^T X in fp32.
# Layer 1's dX is not computed (the input needs no gradient).
C5_GEMMS = {
    "L1_fwd": (4096, 8192, 4096, False, True, "bf16", "bias_relu"),
    "L1_dW": (8192, 4096, 4096, True, False, "f32", None),
    "L2_fwd": (4096, 8192, 8192, False, True, "bf16", "bias_relu"),
    "L2_dX": (4096, 8192, 8192, False, False, "bf16", None),
    "L2_dW": (8192, 8192, 4096, True, False, "f32", None),
    "L3_fwd": (4096, 4096, 8192, False, True, "bf16", "bias_relu"),
    "L3_dX": (4096, 8192, 4096, False, False, "bf16", None),
    "L3_dW": (4096, 8192, 4096, True, False, "f32", None),
    "L4_fwd": (4096, 1000, 4096, False, True, "bf16", "bias"),
    "L4_dX": (4096, 4096, 1000, False, False, "bf16", None),
    "L4_dW": (1000, 4096, 4096, True, False, "f32", None),
}


@pytest.mark.parametrize("name", list(C5_GEMMS))
def test_c5_gemm_at_full_shape_vs_float64(ctx, name):
    import tensors_amd as ta
    from tensors_amd import ops
    M, N, K, tra, trb, out, epi = C5_GEMMS[name]
    seed = 5400 + 7 * list(C5_GEMMS).index(name)
    a16 = ta.f32_to_bf16_bits(_rng_normal(seed, (K, M) if tra else (M, K)))
    b16 = ta.f32_to_bf16_bits(_rng_normal(seed + 1, (N, K) if trb else (K, N)))
    bias = _rng_normal(seed + 2, (N,)) if epi else None
    da, db = ctx.array(a16, ta.BF16), ctx.array(b16, ta.BF16)
    dc = ctx.empty((M, N), ta.BF16 if out == "bf16" else np.float32)
    dbias = ctx.array(bias) if bias is not None else None
    ops.gemm(da, db, dc, trans_a=tra, trans_b=trb, bias=dbias, relu=(epi == "bias_relu"))
    got = dc.numpy()
    got = ta.bf16_bits_to_f32(got) if out == "bf16" else got
    del da, db, dc
    # 64 output rows: the first and last of the matrix, both sides of 256-row
    # tile boundaries, and random rows.
    rows = np.unique(np.concatenate([[0, 255, 256, M - 1], _sample(M, 60, seed + 3)]))
    a = ta.bf16_bits_to_f32(a16)
    b = ta.bf16_bits_to_f32(b16)
    a_rows = (a[:, rows].T if tra else a[rows]).astype(np.float64)
    del a
    b_op = (b.T if trb else b).astype(np.float64)
    truth = a_rows @ b_op
    if bias is not None:
        truth += bias.astype(np.float64)
    if epi == "bias_relu":
        truth = np.maximum(truth, 0.0)
    assert_close(got[rows], truth, RTOL16 if out == "bf16" else RTOL32, f"{name} {M}x{N}x{K} sampled rows")


# ---------------------------------------------------------------------------
# config 4
# ---------------------------------------------------------------------------
def _im2col64(x, k, s, p):
    """[N, C, H, W] -> [N, C*k*k, OH*OW] in float64 (the index map of
    cuda/kernels/im2col.cu:66-98: ih = oh*s + ki - p, zero outside)."""
    N, Cc, H, W = x.shape
    xp = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (p, p), (p, p)))
    oh, ow = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    col = np.empty((N, Cc, k, k, oh, ow))
    for ki in range(k):
        for kj in range(k):
            col[:, :, ki, kj] = xp[:, :, ki:ki + s * oh:s, kj:kj + s * ow:s]
    return col.reshape(N, Cc * k * k, oh * ow), oh, ow


def _col2im64(col, shape, k, s, p):
    N, Cc, H, W = shape
    oh, ow = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    col = col.reshape(N, Cc, k, k, oh, ow)
    dxp = np.zeros((N, Cc, H + 2 * p, W + 2 * p))
    for ki in range(k):
        for kj in range(k):
            dxp[:, :, ki:ki + s * oh:s, kj:kj + s * ow:s] += col[:, :, ki, kj]
    return dxp[:, :, p:p + H, p:p + W]


def _cnn_step64(params, x, y, keep=None):
    """Loss and gradients of the config-4 network in float64: the same math
    as the reference's conv loop (nn/conv2d_backward_test.cpp:50-106), the
    Linear backward and the CE chain, summed exactly enough to judge fp32.
    With `keep` a dict, the intermediates go into it."""
    w1, b1, w2, b2, wf, bf = [p.astype(np.float64) for p in params]
    B = x.shape[0]
    col1, oh1, ow1 = _im2col64(x, 3, 1, 1)
    z1 = np.einsum("ok,nkp->nop", w1.reshape(32, -1), col1) + b1[None, :, None]
    h1 = np.maximum(z1, 0).reshape(B, 32, oh1, ow1)
    col2, oh2, ow2 = _im2col64(h1, 3, 2, 1)
    z2 = np.einsum("ok,nkp->nop", w2.reshape(64, -1), col2) + b2[None, :, None]
    f = np.maximum(z2, 0).reshape(B, -1)
    logits = f @ wf.T + bf
    m = logits.max(1, keepdims=True)
    e = np.exp(logits - m)
    lse = m[:, 0] + np.log(e.sum(1))
    loss = float(np.mean(lse - logits[np.arange(B), y]))
    g = e / e.sum(1, keepdims=True)
    g[np.arange(B), y] -= 1
    g /= B
    dwf, dbf = g.T @ f, g.sum(0)
    dh2 = (g @ wf).reshape(z2.shape)
    dz2 = dh2 * (z2 > 0)
    dw2 = np.einsum("nop,nkp->ok", dz2, col2).reshape(w2.shape)
    db2 = dz2.sum((0, 2))
    dh1 = _col2im64(np.einsum("ok,nop->nkp", w2.reshape(64, -1), dz2), h1.shape, 3, 2, 1)
    dz1 = dh1.reshape(z1.shape) * (z1 > 0)
    dw1 = np.einsum("nop,nkp->ok", dz1, col1).reshape(w1.shape)
    db1 = dz1.sum((0, 2))
    if keep is not None:
        keep.update(col1=col1, z1=z1, col2=col2, z2=z2, dh2=dh2, dh1=dh1.reshape(z1.shape), w1=w1, b1=b1, w2=w2,
                    b2=b2, h1_shape=h1.shape)
    return loss, [dw1, db1, dw2, db2, dwf, dbf]


U32 = 2.0 ** -24          # fp32 unit roundoff (round to nearest)


def _gamma(n):
    """gamma_n = n u / (1 - n u): the bound on the relative error of any fp32
    evaluation of a sum of n + 1 terms (in any order and bracketing), relative
    to the sum of the terms' magnitudes (Higham, Accuracy and Stability of
    Numerical Algorithms, 2nd ed., section 3.1)."""
    return n * U32 / (1.0 - n * U32)


def _fp32_preactivation_bounds(k):
    """Per pre-activation bound on |fp32 z - z| for any fp32 evaluation of the
    two convolutions, from the error model above.  conv1: 27 products plus
    the bias, e1 = gamma_28 (sum |w1| |x| + |b1|).  conv2 reads relu(z1)
    computed in fp32, which is off by at most e1 at each tap (ReLU is
    1-Lipschitz), and sums 288 products plus the bias:
    e2 = gamma_289 (sum |w2| (|h1| + e1) + |b2|) + sum |w2| e1."""
    w1a, w2a = np.abs(k["w1"].reshape(32, -1)), np.abs(k["w2"].reshape(64, -1))
    e1 = _gamma(28) * (np.einsum("ok,nkp->nop", w1a, np.abs(k["col1"])) + np.abs(k["b1"])[None, :, None])
    e1col, _, _ = _im2col64(e1.reshape(k["h1_shape"]), 3, 2, 1)
    carried = np.einsum("ok,nkp->nop", w2a, e1col)
    e2 = _gamma(289) * (np.einsum("ok,nkp->nop", w2a, np.abs(k["col2"]) + e1col)
                        + np.abs(k["b2"])[None, :, None]) + carried
    return e1, e2


def _relu_tie_envelope(k):
    """Bound on how far an fp32 step's conv gradients may sit from the
    float64 ones because a ReLU mask differs: only where a pre-activation is
    within its fp32 error bound of zero (_fp32_preactivation_bounds) can an
    fp32 forward put it on the other side of zero from float64.  Flipping
    the mask at (n, c, p) moves dz by dh there: db by |dh|, dW row c by
    |dh| |col[n, :, p]|, and, for conv2, conv1's upstream gradient by
    |dh| |W2[c, :]| at that column's taps (then through conv1's mask into
    its dW and db).  Returns per-element bounds for [dw1, db1, dw2, db2] and
    the numbers of such sites in conv1 and conv2."""
    col1, z1, col2, z2, dh2, dh1, w2 = (k[n] for n in ("col1", "z1", "col2", "z2", "dh2", "dh1", "w2"))
    e1, e2 = _fp32_preactivation_bounds(k)
    env_dw1 = np.zeros((32, col1.shape[1]))
    env_db1 = np.zeros(32)
    env_dw2 = np.zeros((64, col2.shape[1]))
    env_db2 = np.zeros(64)
    t2 = np.argwhere(np.abs(z2) <= e2)
    spread = np.zeros_like(col2)                  # |change of dcol2| from conv2's ties
    for n, c, p_ in t2:
        a = abs(dh2[n, c, p_])
        env_db2[c] += a
        env_dw2[c] += a * np.abs(col2[n, :, p_])
        spread[n, :, p_] += a * np.abs(w2.reshape(64, -1)[c])
    if len(t2):
        d1 = _col2im64(spread, k["h1_shape"], 3, 2, 1).reshape(z1.shape) * (z1 > 0)
        env_dw1 += np.einsum("nop,nkp->ok", d1, np.abs(col1))
        env_db1 += d1.sum((0, 2))
    t1 = np.argwhere(np.abs(z1) <= e1)
    for n, c, p_ in t1:
        a = abs(dh1[n, c, p_])
        env_db1[c] += a
        env_dw1[c] += a * np.abs(col1[n, :, p_])
    return [env_dw1, env_db1, env_dw2, env_db2], len(t1), len(t2)


def test_c4_full_batch_step_vs_float64(ctx):
    """One full config-4 step (batch 128) on the GPU: the loss against the
    restated reference loop (oracle.cnn_step), and every parameter's gradient
    against the same step in float64 (lr = 1, mu = 0, so p_old - p_new is
    the gradient).  This covers the batch-reduced weight-gradient GEMMs over
    128 images, the plane im2col/col2im kernels at 384 and 4096 planes and
    the split-K choices that only the full batch selects.  The reference
    loop's own sequential fp32 sums (131,072 terms per conv1 weight, 32,768
    per conv2 weight) are themselves off float64 by up to 0.2 % (conv1) and
    0.9 % (conv2) of the gradient's rms here, far above rtol 1e-4, so the
    gradients are judged against float64, as every other fp32 reduction.
    The conv gradients get, on top of rtol 1e-4, the bound that ReLU ties
    allow (_relu_tie_envelope): an fp32 forward may put a pre-activation
    that lies within its fp32 error bound (gamma_K sum |w| |x|, per site) of
    zero on the other side from float64 (one such flip moves a conv2 bias
    gradient by ~1e-3 of its rms), whichever kernel computes the
    convolution."""
    B, H = 128, 32
    xs = synth.normal(synth.seed(4, 0), (1, B, 3, H, H))
    ys = synth.uniform_int(synth.seed(4, 1), (1, B), 10)
    flat = 64 * (H // 2) * (H // 2)
    shapes = [(32, 3, 3, 3), (32,), (64, 32, 3, 3), (64,), (10, flat), (10,)]
    stds = [0.2, 0.1, 0.06, 0.1, 0.01, 0.1]
    params = [synth.normal(synth.seed(4, 10 + i), s, std=sd) for i, (s, sd) in enumerate(zip(shapes, stds))]
    init = np.concatenate([p.ravel() for p in params])
    losses, fp, _ = api.cnn_train(xs, ys, steps=1, lr=1.0, mu=0.0, on_gpu=True, init_params=init, want_params=True)
    ps = [p.copy() for p in params]
    ref = oracle.cnn_step(ps, [np.zeros_like(p) for p in ps], xs[0], ys[0], 1.0, 0.0)
    assert abs(float(losses[0]) - ref) <= RTOL32 * max(1.0, abs(ref)), (float(losses[0]), ref)
    keep = {}
    loss64, grads = _cnn_step64(params, xs[0], ys[0], keep)
    assert abs(float(losses[0]) - loss64) <= RTOL32 * max(1.0, abs(loss64))
    env, n_t1, n_t2 = _relu_tie_envelope(keep)
    # sites within their fp32 bound of zero are rare among the 6.3 M
    # pre-activations, so the envelope covers few gradient entries
    assert n_t1 + n_t2 < 2000, (n_t1, n_t2)
    off = 0
    names = ["conv1.w", "conv1.b", "conv2.w", "conv2.b", "fc.w", "fc.b"]
    for i, (name, p0, g64) in enumerate(zip(names, params, grads)):
        n = p0.size
        got = p0.ravel().astype(np.float64) - fp[off:off + n]
        off += n
        truth = g64.ravel()
        atol = RTOL32 * np.sqrt(np.mean(truth ** 2))
        slack = env[i].ravel() if i < 4 else 0.0
        err = np.abs(got - truth)
        bad = err > atol + RTOL32 * np.abs(truth) + slack
        assert not bad.any(), (f"{name} gradient: {int(bad.sum())}/{n} outside rtol 1e-4 + ReLU-tie bound; worst "
                               f"err {float(err.max()):.3g}, rms {float(np.sqrt(np.mean(truth ** 2))):.3g}")
