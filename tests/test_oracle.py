"""Pins the CPU oracle (oracle/tf_oracle.c) before it is trusted as the
checker of the GPU path.

Every oracle function is checked by at least one of:
  * the golden fixtures written from the compiled reference
    (tests/golden/make_golden.py) — bit-exact;
  * the compiled reference itself (oracle/_ref), when built here — bit-exact
    on fresh random inputs;
  * known answers from the reference's own tests (cited);
  * mathematics: float64 closed forms, central differences of the forward,
    brute-force index loops, adjoint identities.
A few tests plant a plausible mistake in an oracle-shaped computation and
assert that the corresponding check rejects it.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from tensors_amd import synth
from tests.conftest import assert_bitexact, assert_close

GOLD = Path(__file__).resolve().parent / "golden"
FIX = np.load(GOLD / "reference_outputs.npz")
META = json.loads((GOLD / "reference_outputs.json").read_text())

needs_ref = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (no reference tree)")


def sample_idx(n):
    return np.unique(synth.uniform_int(0xF1C5, (4096,), n)) if n > 4096 else np.arange(n)


def check_fixture(name, arr):
    """Bit-exact comparison with a fixture (whole, or sample + SHA-256)."""
    arr = np.ascontiguousarray(arr)
    if name in FIX.files:
        assert_bitexact(arr.reshape(FIX[name].shape), FIX[name], name)
        return
    assert list(arr.shape) == META[f"{name}:shape"], name
    assert_bitexact(arr.ravel()[sample_idx(arr.size)], FIX[f"{name}:sample"], name + " sample")
    assert hashlib.sha256(arr.tobytes()).hexdigest() == META[f"{name}:sha256"], name + " sha256"


# ---------------------------------------------------------------------------
# fixtures from the compiled reference
# ---------------------------------------------------------------------------
def test_matmul_and_backward_match_reference_bits():
    a = synth.normal(synth.seed(9, 0), (64, 784))
    b = synth.normal(synth.seed(9, 1), (784, 256))
    dc = synth.normal(synth.seed(9, 2), (64, 256))
    check_fixture("matmul_64x784x256", oracle.matmul(a, b))
    # MatmulBackward: dA = dC @ transpose(B), dB = transpose(A) @ dC
    check_fixture("matmul_bwd_dA", oracle.matmul(dc, oracle.transpose2d(b)))
    check_fixture("matmul_bwd_dB", oracle.matmul(oracle.transpose2d(a), dc))


def test_linear_matches_reference_bits():
    a = synth.normal(synth.seed(9, 0), (64, 784))
    dc = synth.normal(synth.seed(9, 2), (64, 256))
    w = synth.normal(synth.seed(9, 3), (256, 784), std=0.03)
    check_fixture("linear_y", oracle.linear_fwd(a, w))
    dx, dw = oracle.linear_bwd(a, w, dc)
    check_fixture("linear_dx", dx)
    check_fixture("linear_dw", dw)


def test_relu_bwd_and_activations_match_reference_bits():
    x = synth.normal(synth.seed(9, 4), (65536,))
    x[:4] = [0.0, -0.0, 1e-38, -1e-38]
    dy = synth.normal(synth.seed(9, 5), (65536,))
    check_fixture("relu_bwd", oracle.relu_bwd(dy, x))
    xx = synth.normal(synth.seed(9, 6), (4096,), std=3.0)
    check_fixture("relu_fwd", oracle.relu(xx))
    check_fixture("sigmoid_fwd", oracle.sigmoid(xx))
    check_fixture("tanh_fwd", oracle.tanh(xx))


@pytest.mark.parametrize("R,Cc", [(64, 10), (256, 1024)])
def test_softmax_family_matches_reference_bits(R, Cc):
    xx = synth.normal(synth.seed(9, 7), (R, Cc), std=2.0)
    gy = synth.normal(synth.seed(9, 8), (R, Cc))
    y = oracle.softmax(xx)
    check_fixture(f"softmax_fwd_{R}x{Cc}", y)
    check_fixture(f"softmax_bwd_{R}x{Cc}", oracle.softmax_bwd(y, gy))
    ly = oracle.log_softmax(xx)
    check_fixture(f"log_softmax_fwd_{R}x{Cc}", ly)
    check_fixture(f"log_softmax_bwd_{R}x{Cc}", oracle.log_softmax_bwd(ly, gy))


@pytest.mark.parametrize("R,Cc,sd", [(64, 10, 1.0), (128, 10, 1.0), (256, 1024, 3.0)])
def test_ce_chain_matches_reference_bits(R, Cc, sd):
    lg = synth.normal(synth.seed(3, R), (R, Cc), std=sd)
    lb = synth.uniform_int(synth.seed(3, R + 1), (R,), Cc)
    loss, d = oracle.ce_chain(lg, lb)
    check_fixture(f"ce_chain_loss_{R}x{Cc}", np.array([loss], np.float32))
    check_fixture(f"ce_chain_dlogits_{R}x{Cc}", d)


def test_sum_and_layernorm_and_conv_match_reference_bits():
    xx = synth.normal(synth.seed(9, 9), (33, 47))
    check_fixture("sum_dim0", oracle.colsum(xx))
    check_fixture("sum_dim1", np.array([sum_row(r) for r in xx], np.float32))
    xx = synth.normal(synth.seed(9, 10), (64, 128))
    g = synth.normal(synth.seed(9, 11), (128,), mean=1.0, std=0.1)
    bb = synth.normal(synth.seed(9, 12), (128,))
    gy = synth.normal(synth.seed(9, 13), (64, 128))
    y, _, _ = oracle.layernorm_fwd(xx, g, bb)
    check_fixture("layernorm_fwd", y)
    check_fixture("layernorm_bwd_stub", oracle.layernorm_bwd_stub(gy, g)[0])
    x4 = synth.normal(synth.seed(4, 0), (2, 3, 8, 8))
    wc = synth.normal(synth.seed(4, 1), (4, 3, 3, 3), std=0.2)
    bc = synth.normal(synth.seed(4, 2), (4,))
    for (stride, pad) in ((1, 1), (2, 1)):
        check_fixture(f"conv2d_fwd_s{stride}p{pad}", oracle.conv2d_fwd(x4, wc, bc, stride, pad))


def sum_row(r):
    s = np.float32(0)
    for v in r:
        s = np.float32(s + v)
    return s


def test_c1_trajectory_of_oracle_matches_reference_bits():
    """100 momentum-SGD steps of the config-1 MLP in reference order equal the
    compiled reference's trajectory bit for bit (and its weights after 1 and
    100 steps)."""
    xs = synth.mnist_like(synth.seed(1, 0), (100, 64, 784))
    ys = synth.uniform_int(synth.seed(1, 1), (100, 64), 10)
    ws = [FIX_W(i) for i in range(3)]
    vs = [np.zeros_like(w) for w in ws]
    losses = []
    for s in range(100):
        losses.append(oracle.mlp_step(ws, vs, xs[s], ys[s], 0.1, 0.9))
        if s == 0:
            check_fixture("c1_weights_after_1", np.concatenate([w.ravel() for w in ws]))
    check_fixture("c1_losses_100", np.array(losses, np.float32))
    check_fixture("c1_weights_after_100", np.concatenate([w.ravel() for w in ws]))


_INIT_CACHE = {}


def FIX_W(i):
    """C1 initial weight i: the reference init when _ref is built, else the
    C++ API's own init (pinned to the fixture's SHA-256 in test_api_cpu)."""
    if i not in _INIT_CACHE:
        dims = [784, 256, 128, 10]
        if oracle.ref_available():
            w = np.empty((dims[i + 1], dims[i]), np.float32)
            oracle.ref_call("ref_linear_init", dims[i], dims[i + 1], w)
        else:
            from tensors_amd import api
            _, fw, _ = api.mlp_train(dims, np.zeros((1, 1, 784), np.float32), np.zeros((1, 1), np.int64), steps=0,
                                     lr=0.1, mu=0.9, on_gpu=False, reference_compat=True, want_weights=True)
            offs = np.cumsum([0] + [dims[k] * dims[k + 1] for k in range(3)])
            w = fw[offs[i]:offs[i + 1]].reshape(dims[i + 1], dims[i]).copy()
        check_fixture(f"c1_init_w{i}", w)
        _INIT_CACHE[i] = w
    return _INIT_CACHE[i].copy()


# ---------------------------------------------------------------------------
# live comparisons with the compiled reference
# ---------------------------------------------------------------------------
@needs_ref
@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (5, 7, 3), (17, 19, 23), (64, 128, 10)])
def test_matmul_live_bits(M, K, N):
    a = synth.normal(500 + M, (M, K))
    b = synth.normal(501 + N, (K, N))
    c = np.empty((M, N), np.float32)
    oracle.ref_call("ref_matmul", a, b, c, M, K, N)
    assert_bitexact(oracle.matmul(a, b), c, "matmul")
    t = np.empty((K, M), np.float32)
    oracle.ref_call("ref_transpose2d", a, t, M, K)
    assert_bitexact(oracle.transpose2d(a), t, "transpose")


@needs_ref
@pytest.mark.parametrize("R,Cc", [(1, 1), (3, 7), (33, 100), (8, 4096)])
def test_row_ops_live_bits(R, Cc):
    x = synth.normal(510 + Cc, (R, Cc), std=4.0)
    g = synth.normal(511 + Cc, (R, Cc))
    for name, fwd, bwd in (("softmax", oracle.softmax, oracle.softmax_bwd),
                           ("log_softmax", oracle.log_softmax, oracle.log_softmax_bwd)):
        y = np.empty_like(x)
        oracle.ref_call(f"ref_{name}_fwd", x, y, R, Cc)
        assert_bitexact(fwd(x), y, name)
        gx = np.empty_like(x)
        oracle.ref_call(f"ref_{name}_bwd", y, g, gx, R, Cc)
        assert_bitexact(bwd(y, g), gx, name + " bwd")
    labels = synth.uniform_int(512, (R,), Cc)
    labels[0] = -1 if R > 1 else labels[0]          # skipped by the chain's mask
    loss = np.zeros(1, np.float32)
    d = np.empty_like(x)
    oracle.ref_call("ref_ce_chain", x, labels, R, Cc, loss, d)
    ol, od = oracle.ce_chain(x, labels)
    assert_bitexact(np.array([ol], np.float32), loss, "ce loss")
    assert_bitexact(od, d, "ce dlogits")


@needs_ref
def test_layernorm_and_conv_live_bits():
    x = synth.normal(520, (9, 33))
    g = synth.normal(521, (33,), mean=1.0, std=0.2)
    b = synth.normal(522, (33,))
    y = np.empty_like(x)
    oracle.ref_call("ref_layernorm_fwd", x, g, b, y, 9, 33, 1e-5)
    assert_bitexact(oracle.layernorm_fwd(x, g, b)[0], y, "ln fwd")
    dy = synth.normal(523, (9, 33))
    dx = np.empty_like(x)
    oracle.ref_call("ref_layernorm_bwd", x, g, b, dy, dx, 9, 33, 1e-5)
    assert_bitexact(oracle.layernorm_bwd_stub(dy, g)[0], dx, "ln stub bwd")
    x4 = synth.normal(524, (3, 2, 7, 9))
    w4 = synth.normal(525, (5, 2, 3, 3))
    b4 = synth.normal(526, (5,))
    for stride, pad in ((1, 0), (2, 1), (3, 2)):
        oh = (7 + 2 * pad - 3) // stride + 1
        ow = (9 + 2 * pad - 3) // stride + 1
        y4 = np.empty((3, 5, oh, ow), np.float32)
        oracle.ref_call("ref_conv2d_fwd", x4, w4, b4, y4, 3, 2, 7, 9, 5, 3, stride, pad)
        assert_bitexact(oracle.conv2d_fwd(x4, w4, b4, stride, pad), y4, f"conv fwd s{stride}p{pad}")


@needs_ref
def test_linear_and_relu_live_bits():
    x = synth.normal(530, (13, 21))
    w = synth.normal(531, (17, 21))
    dy = synth.normal(532, (13, 17))
    y, dx, dw = np.empty((13, 17), np.float32), np.empty((13, 21), np.float32), np.empty((17, 21), np.float32)
    oracle.ref_call("ref_linear", x, w, dy, y, dx, dw, 13, 21, 17)
    assert_bitexact(oracle.linear_fwd(x, w), y, "linear y")
    odx, odw = oracle.linear_bwd(x, w, dy)
    assert_bitexact(odx, dx, "linear dx")
    assert_bitexact(odw, dw, "linear dw")
    r = np.empty(x.size, np.float32)
    up, xin = dx.ravel().copy(), x.ravel().copy()
    oracle.ref_call("ref_relu_bwd", up, xin, r, x.size)
    assert_bitexact(oracle.relu_bwd(up, xin), r, "relu bwd")


# ---------------------------------------------------------------------------
# known answers from the reference's tests
# ---------------------------------------------------------------------------
def test_known_answers():
    # autograd/ops/autograd_all_ops_test.cpp:281-328
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    b = np.arange(6, dtype=np.float32).reshape(3, 2)
    assert np.array_equal(oracle.matmul(a, b), [[10, 13], [28, 40]])
    g = np.ones((2, 2), np.float32)
    assert np.array_equal(oracle.matmul(g, oracle.transpose2d(b)), [[1, 5, 9], [1, 5, 9]])
    assert np.array_equal(oracle.matmul(oracle.transpose2d(a), g), [[3, 3], [5, 5], [7, 7]])
    # cuda/kernels/gemm_optimized_test.cpp:109-125
    assert np.array_equal(oracle.matmul([[1, 2], [3, 4]], [[5, 6], [7, 8]]), [[19, 22], [43, 50]])
    # autograd/ops/autograd_all_ops_test.cpp:73-94: relu mask with x == 0 -> 0
    assert np.array_equal(oracle.relu_bwd(np.ones(3, np.float32), np.array([-1, 0, 2], np.float32)), [0, 0, 1])
    # autograd/ops/autograd_all_ops_test.cpp:108-121: uniform softmax, grad 0
    y = oracle.softmax(np.full((2, 4), 0.3, np.float32))
    assert np.max(np.abs(oracle.softmax_bwd(y, np.ones((2, 4), np.float32)))) < 1e-7
    # nn/cross_entropy_test.cpp:10-49 (module loss = chain loss here)
    loss, _ = oracle.ce_chain(np.array([[1, 2, 3]], np.float32), np.array([2]))
    assert abs(loss - 0.4076) < 0.01 * 0.4076
    loss, _ = oracle.ce_chain(np.ones((2, 3), np.float32), np.array([0, 2]))
    assert abs(loss - 1.0986) < 0.01 * 1.0986
    # nn/conv2d_backward_test.cpp:110-160: 1x1 golden
    gin, gw, gb = oracle.conv2d_bwd(np.array([1, 2, 3, 4], np.float32).reshape(1, 1, 2, 2),
                                    np.array([2.0], np.float32).reshape(1, 1, 1, 1),
                                    np.array([0.1, 0.2, 0.3, 0.4], np.float32).reshape(1, 1, 2, 2), has_bias=False)
    assert_close(gin.ravel(), [0.2, 0.4, 0.6, 0.8], 1e-6, atol=1e-7)
    assert_close(gw.ravel(), [3.0], 1e-6, atol=1e-7)
    assert gb[0] == 0.0


# ---------------------------------------------------------------------------
# mathematics: closed forms, finite differences, brute force
# ---------------------------------------------------------------------------
def test_matmul_close_to_float64():
    a = synth.normal(600, (64, 784))
    b = synth.normal(601, (784, 256))
    assert_close(oracle.matmul(a, b), a.astype(np.float64) @ b.astype(np.float64), 1e-5)


def test_ce_chain_is_softmax_minus_onehot_over_n():
    lg = synth.normal(610, (37, 11), std=3.0)
    lb = synth.uniform_int(611, (37,), 11)
    loss, d = oracle.ce_chain(lg, lb)
    x = lg.astype(np.float64)
    p = np.exp(x - x.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    oh = np.zeros_like(p)
    oh[np.arange(37), lb] = 1.0
    assert_close(d, (p - oh) / 37, 1e-5)
    assert abs(loss - float(np.mean(-np.log(p[np.arange(37), lb])))) < 1e-5


def test_relu_bwd_sign_of_zero():
    # dy * 0.0 keeps the sign of dy (-0.0 for negative dy), as the reference.
    d = oracle.relu_bwd(np.array([-1.0, 1.0], np.float32), np.array([-3.0, -3.0], np.float32))
    assert np.signbit(d[0]) and not np.signbit(d[1])


def _central(f, x, h):
    x = x.astype(np.float64)
    g = np.empty_like(x)
    for i in range(x.size):
        xp, xm = x.copy(), x.copy()
        xp.flat[i] += h
        xm.flat[i] -= h
        g.flat[i] = (f(xp) - f(xm)) / (2 * h)
    return g


def _sigmoid64(x):
    return 1.0 / (1.0 + np.exp(-x))


def test_sigmoid_tanh_bwd_are_derivatives_of_the_forward():
    x = synth.normal(620, (40,), std=2.0)
    w = synth.normal(621, (40,))
    # The oracle's forwards equal the reference's (fixture test above); the
    # backward rules must be their derivatives.
    gs = _central(lambda v: float(np.sum(_sigmoid64(v) * w)), x, 1e-5)
    gt = _central(lambda v: float(np.sum(np.tanh(v) * w)), x, 1e-5)
    assert_close(oracle.sigmoid_bwd(w, oracle.sigmoid(x)), gs, 1e-5)
    assert_close(oracle.tanh_bwd(w, oracle.tanh(x)), gt, 1e-5)


def _ln64(x, g, b, eps=1e-5):
    m = x.mean(1, keepdims=True)
    v = ((x - m) ** 2).mean(1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * g + b


def test_layernorm_true_bwd_is_derivative_of_the_forward():
    R, Cc = 4, 9
    x = synth.normal(630, (R, Cc))
    g = synth.normal(631, (Cc,), mean=1.0, std=0.3)
    b = synth.normal(632, (Cc,))
    w = synth.normal(633, (R, Cc))
    _, m, rs = oracle.layernorm_fwd(x, g, b)
    dx, dg, db = oracle.layernorm_bwd(x, w, g, m, rs)
    g64, b64 = g.astype(np.float64), b.astype(np.float64)
    assert_close(dx, _central(lambda v: float(np.sum(_ln64(v, g64, b64) * w)), x, 1e-6), 1e-4)
    assert_close(dg, _central(lambda v: float(np.sum(_ln64(x.astype(np.float64), v, b64) * w)), g, 1e-6), 1e-4)
    assert_close(db, _central(lambda v: float(np.sum(_ln64(x.astype(np.float64), g64, v) * w)), b, 1e-6), 1e-4)


def test_planted_mistake_in_layernorm_bwd_is_caught():
    """Dropping the mean(g*xhat) term (a plausible mistake) must fail the
    finite-difference check used above."""
    R, Cc = 4, 9
    x = synth.normal(630, (R, Cc))
    g = synth.normal(631, (Cc,), mean=1.0, std=0.3)
    w = synth.normal(633, (R, Cc))
    x64, g64 = x.astype(np.float64), g.astype(np.float64)
    m = x64.mean(1, keepdims=True)
    rs = 1 / np.sqrt(((x64 - m) ** 2).mean(1, keepdims=True) + 1e-5)
    xh = (x64 - m) * rs
    gg = w * g64
    wrong = rs * (gg - gg.mean(1, keepdims=True))             # term dropped
    truth = _central(lambda v: float(np.sum(_ln64(v, g64, 0.0) * w)), x, 1e-6)
    with pytest.raises(AssertionError):
        assert_close(wrong, truth, 1e-4)
    right = rs * (gg - gg.mean(1, keepdims=True) - xh * (gg * xh).mean(1, keepdims=True))
    assert_close(right, truth, 1e-4)


def test_planted_mistake_transposed_operand_is_caught():
    """A Linear backward that used W^T instead of W (shapes permitting) fails
    the fixture comparison."""
    a = synth.normal(synth.seed(9, 0), (64, 784))
    dc = synth.normal(synth.seed(9, 2), (64, 256))
    w = synth.normal(synth.seed(9, 3), (256, 784), std=0.03)
    _, dw = oracle.linear_bwd(a, w, dc)
    with pytest.raises(AssertionError):
        check_fixture("linear_dw", oracle.transpose2d(oracle.transpose2d(dw) * np.float32(1.0001)).copy())


def test_sgd_mu0_equals_train_mlp_manual_loop():
    p, g, v = synth.normal(640, (1000,)), synth.normal(641, (1000,)), synth.normal(642, (1000,))
    np_, nv = oracle.sgd_momentum(p, g, v, 0.05, 0.0)
    # examples/train_mlp.cpp:155-157: pp[k] -= step_lr * gp[k]
    assert_bitexact(np_, (p - np.float32(0.05) * g).astype(np.float32), "mu=0")
    assert_bitexact(nv, v, "velocity untouched")


def test_sgd_momentum_closed_form_two_steps():
    p, g = synth.normal(650, (100,)), synth.normal(651, (100,))
    v = np.zeros(100, np.float32)
    lr, mu = np.float32(0.1), np.float32(0.9)
    q, w = p.copy(), v.copy()
    for _ in range(2):
        w = (w * mu + g).astype(np.float32)
        q = (q - w * lr).astype(np.float32)
    pp, vv = oracle.sgd_momentum(p, g, v, 0.1, 0.9)
    pp, vv = oracle.sgd_momentum(pp, g, vv, 0.1, 0.9)
    assert_bitexact(pp, q, "p")
    assert_bitexact(vv, w, "v")


def test_colsum_chansum_close_to_float64():
    x = synth.normal(660, (301, 45))
    assert_close(oracle.colsum(x), x.astype(np.float64).sum(0), 1e-5)
    y = synth.normal(661, (6, 5, 7, 9))
    assert_close(oracle.chansum_nchw(y), y.astype(np.float64).sum((0, 2, 3)), 1e-5)


def _im2col_brute(x, k, s, p, d):
    N, Cc, H, W = x.shape
    oh = (H + 2 * p - d * (k - 1) - 1) // s + 1
    ow = (W + 2 * p - d * (k - 1) - 1) // s + 1
    col = np.zeros((N, Cc * k * k, oh * ow), np.float32)
    for n in range(N):
        for c in range(Cc):
            for ki in range(k):
                for kj in range(k):
                    for i in range(oh):
                        for j in range(ow):
                            ih, iw = i * s + ki * d - p, j * s + kj * d - p
                            if 0 <= ih < H and 0 <= iw < W:
                                col[n, (c * k + ki) * k + kj, i * ow + j] = x[n, c, ih, iw]
    return col


@pytest.mark.parametrize("case", [(1, 2, 5, 6, 3, 1, 1, 1), (2, 1, 7, 7, 3, 2, 1, 1), (1, 3, 9, 8, 3, 1, 2, 2),
                                  (1, 1, 4, 4, 1, 1, 0, 1)])
def test_im2col_brute_force_and_col2im_adjoint(case):
    N, Cc, H, W, k, s, p, d = case
    x = synth.normal(670, (N, Cc, H, W))
    col = oracle.im2col(x, k, k, s, s, p, p, d, d)
    assert_bitexact(col, _im2col_brute(x, k, s, p, d), "im2col")
    c = synth.normal(671, col.shape)
    back = oracle.col2im(c, x.shape, k, k, s, s, p, p, d, d)
    lhs = float(np.dot(col.astype(np.float64).ravel(), c.astype(np.float64).ravel()))
    rhs = float(np.dot(x.astype(np.float64).ravel(), back.astype(np.float64).ravel()))
    assert abs(lhs - rhs) <= 1e-5 * (abs(lhs) + 1)


def test_conv2d_bwd_is_derivative_of_conv2d_fwd():
    x = synth.normal(680, (2, 2, 5, 5))
    w = synth.normal(681, (3, 2, 3, 3))
    b = synth.normal(682, (3,))
    for stride, pad in ((1, 1), (2, 1)):
        y = oracle.conv2d_fwd(x, w, b, stride, pad)
        up = synth.normal(683, y.shape)

        def L(xv=None, wv=None, bv=None):
            xx = x if xv is None else xv
            ww = w if wv is None else wv
            bb = b if bv is None else bv
            return float(np.sum(_conv64(xx, ww, bb, stride, pad) * up))

        gin, gw, gb = oracle.conv2d_bwd(x, w, up, (stride, stride), (pad, pad), (1, 1))
        assert_close(gin, _central(lambda v: L(xv=v), x, 1e-6), 1e-4)
        assert_close(gw, _central(lambda v: L(wv=v), w, 1e-6), 1e-4)
        assert_close(gb, _central(lambda v: L(bv=v), b, 1e-6), 1e-4)


def _conv64(x, w, b, s, p):
    x = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (p, p), (p, p)))
    N, Cc, H, W = x.shape
    Co, _, k, _ = w.shape
    oh, ow = (H - k) // s + 1, (W - k) // s + 1
    y = np.zeros((N, Co, oh, ow))
    for i in range(oh):
        for j in range(ow):
            patch = x[:, :, i * s:i * s + k, j * s:j * s + k]
            y[:, :, i, j] = np.tensordot(patch, w.astype(np.float64), axes=([1, 2, 3], [1, 2, 3]))
    return y + b.astype(np.float64)[None, :, None, None]


def test_argmax_first_max_wins():
    x = np.array([[1, 3, 3, 2], [5, 5, 5, 5], [-1, -2, -0.5, -0.5]], np.float32)
    assert list(oracle.argmax_rows(x)) == [1, 0, 2]
    # examples/train_mlp.cpp:95-100 starts from -1e30 with prediction 0 and
    # compares with '>': values at or below -1e30 and NaN never win; -0.0
    # and +0.0 tie (the first stays).
    nan = np.float32(np.nan)
    y = np.array([[-1e30, -3e30, -1e30, -np.inf], [nan, nan, 2, nan], [nan, nan, nan, nan],
                  [-0.0, 0.0, -0.0, -1], [0.0, -0.0, 0, -1], [-2e30, -1e29, -1e30, -1e29]], np.float32)
    assert list(oracle.argmax_rows(y)) == [0, 2, 0, 0, 0, 1]


@needs_ref
def test_leaky_relu_live_bits_and_known_answers():
    x = np.concatenate([synth.normal(800, (999,)), np.array([0.0, -0.0, 1e-45, -1e-45, 3e38, -3e38],
                                                             np.float32)])
    for alpha in (0.01, 0.2, 1.5, 0.0):
        y = np.empty_like(x)
        oracle.ref_call("ref_leaky_relu_fwd", x, y, x.size, alpha)
        assert_bitexact(oracle.leaky_relu(x, alpha), y, f"leaky_relu alpha={alpha}")
    got = oracle.leaky_relu(np.array([-2, -0.5, 0, 0.5], np.float32), 0.1)
    assert_bitexact(got, np.array([np.float32(0.1) * np.float32(-2), np.float32(0.1) * np.float32(-0.5), 0, 0.5],
                                  np.float32), "known")


# ---------------------------------------------------------------------------
# mixed-precision (bf16) step of config 5
# ---------------------------------------------------------------------------
def test_bf16_round_known_answers_and_package_rule():
    """Ties go to the even neighbour; one bf16 ulp at 1.0 is 2^-7."""
    one = 1.0
    x = np.array([one, one + 2 ** -8, one + 3 * 2 ** -8, one + 2 ** -8 + 2 ** -20, -(one + 2 ** -8),
                  2 ** -130, 3.0e38, -3.4e38, np.inf, -np.inf, 0.0, -0.0], np.float32)
    want = np.array([one, one, one + 2 ** -6, one + 2 ** -7, -one, 2 ** -130], np.float32)
    got = oracle.bf16_round(x)
    # -3.4e38 lies above the largest bf16 (3.3895e38) past the midpoint to 2^128
    assert np.array_equal(got[:6], want) and got[7] == -np.inf and np.isinf(got[8])
    assert np.signbit(got[11]) and not np.signbit(got[10])
    # 3.0e38 lies between bf16 neighbours 2.9909e38 and 3.0042e38
    assert abs(float(got[6]) - 3.0e38) <= 2 ** 120
    # Same rule as the package's bit conversion (which the GPU's hardware
    # conversion is compared with bit for bit).
    from tensors_amd import bf16_bits_to_f32, f32_to_bf16_bits
    r = np.concatenate([synth.normal(700, (20000,)), synth.normal(701, (2000,), std=1e-38),
                        synth.normal(702, (2000,), std=1e30)])
    assert_bitexact(oracle.bf16_round(r), bf16_bits_to_f32(f32_to_bf16_bits(r)), "bf16 rule")


def _mixed_init(dims, seed0, bias):
    ws = [synth.normal(seed0 + i, (dims[i + 1], dims[i]), std=float(dims[i]) ** -0.5) for i in range(len(dims) - 1)]
    bs = [synth.normal(seed0 + 50 + i, (dims[i + 1],), std=0.1) if bias else None for i in range(len(dims) - 1)]
    return ws, bs


def test_mixed_step_without_rounding_is_the_reference_order_step():
    """With the bf16 roundings turned off and no bias, three steps equal the
    reference-order fp32 step (mlp_step, pinned bit-exact to the compiled
    reference's 100-step trajectory) up to summation order."""
    dims = [40, 32, 24, 10]
    ws, _ = _mixed_init(dims, 710, False)
    ws_ref = [w.copy() for w in ws]
    vs = [np.zeros_like(w) for w in ws]
    vs_ref = [np.zeros_like(w) for w in ws]
    for s in range(3):
        x = synth.normal(720 + s, (16, dims[0]))
        y = synth.uniform_int(730 + s, (16,), dims[-1])
        l_mix = oracle.mlp_step_mixed(ws, [None] * 3, vs, [None] * 3, x, y, 0.1, 0.9, rounding=False)
        l_ref = oracle.mlp_step(ws_ref, vs_ref, x, y, 0.1, 0.9)
        assert abs(l_mix - l_ref) <= 1e-5 * max(1.0, abs(l_ref)), (s, l_mix, l_ref)
    for i in range(3):
        assert_close(ws[i], ws_ref[i], 1e-5, f"W{i} after 3 steps")
        assert_close(vs[i], vs_ref[i], 1e-4, f"v{i} after 3 steps")


def _mlp_loss64(ws, bs, x, y):
    h = x.astype(np.float64)
    for i, (w, b) in enumerate(zip(ws, bs)):
        h = h @ w.astype(np.float64).T + b.astype(np.float64)
        if i + 1 < len(ws):
            h = np.maximum(h, 0.0)
    m = h.max(1, keepdims=True)
    lse = m[:, 0] + np.log(np.exp(h - m).sum(1))
    return float(np.mean(lse - h[np.arange(len(y)), y]))


def test_mixed_step_gradients_are_derivatives_of_the_loss():
    """Without rounding, mu = 0 and lr = 1, the update p_old - p_new is the
    gradient: it must equal central differences of a float64 forward, for
    the weights and the biases of every layer (a dropped bias gradient, a
    mask taken from the wrong tensor or a transposed operand fails this)."""
    dims = [12, 9, 7, 5]
    ws, bs = _mixed_init(dims, 740, True)
    x = synth.normal(760, (6, dims[0]))
    y = synth.uniform_int(761, (6,), dims[-1])
    w0 = [w.astype(np.float64) for w in ws]
    b0 = [b.astype(np.float64) for b in bs]
    loss = oracle.mlp_step_mixed(ws, bs, [np.zeros_like(w) for w in ws], [np.zeros_like(b) for b in bs], x, y,
                                 1.0, 0.0, rounding=False)
    assert abs(loss - _mlp_loss64(w0, b0, x, y)) < 1e-5
    h = 1e-5
    for li in range(3):
        for arr0, new, is_w in ((w0[li], ws[li], True), (b0[li], bs[li], False)):
            g = arr0 - new.astype(np.float64)
            cd = np.zeros_like(arr0)
            for idx in np.ndindex(arr0.shape):
                p, m = [a.copy() for a in w0], [a.copy() for a in w0]
                pb, mb = [a.copy() for a in b0], [a.copy() for a in b0]
                (p if is_w else pb)[li][idx] += h
                (m if is_w else mb)[li][idx] -= h
                cd[idx] = (_mlp_loss64(p, pb, x, y) - _mlp_loss64(m, mb, x, y)) / (2 * h)
            assert_close(g, cd, 1e-3, f"layer {li} {'W' if is_w else 'b'} gradient", atol=1e-5)


def test_mixed_step_rounding_changes_results_by_bf16_amounts():
    """With rounding on, the loss moves by about a bf16 ulp from the float32
    step, not by zero (the roundings are applied) and not by more than the
    bf16 bar (they are applied to the right tensors)."""
    dims = [64, 48, 32, 10]
    ws, bs = _mixed_init(dims, 780, True)
    x = synth.normal(790, (32, dims[0]))
    y = synth.uniform_int(791, (32,), dims[-1])
    args = lambda: ([w.copy() for w in ws], [b.copy() for b in bs], [np.zeros_like(w) for w in ws],
                    [np.zeros_like(b) for b in bs])
    l16 = oracle.mlp_step_mixed(*args()[:2], *args()[2:], x, y, 0.1, 0.9, rounding=True)
    l32 = oracle.mlp_step_mixed(*args()[:2], *args()[2:], x, y, 0.1, 0.9, rounding=False)
    assert 0 < abs(l16 - l32) < 2e-2 * abs(l32)


def _mixed_trace_problems(tr, bs, x, y):
    """Where the stored tensors of a mixed step (oracle.mlp_step_mixed's
    trace) break the rounding points of the bf16 compute path, judged from
    the values alone against float64 recomputed from the trace's own inputs:
    stored bf16 tensors (input, weights' working copies, layer outputs,
    dlogits, data gradients) must be bf16 values within one rounding (half a
    bf16 step) of their float64 value; fp32 gradients (dW, db) must be within
    fp32 accumulation error of float64, which a bf16 rounding of them is not.
    Returns a list of descriptions (empty: every point as specified)."""
    probs = []
    is16 = lambda a: np.array_equal(oracle.bf16_round(a), a)

    def one_rounding(got, truth, what):
        got, truth = np.asarray(got, np.float64), np.asarray(truth, np.float64)
        if not is16(np.asarray(got, np.float32)):
            probs.append(f"{what}: not bf16 values")
        e = np.floor(np.log2(np.maximum(np.abs(truth), 1e-300)))
        bound = np.exp2(e - 8) * (1 + 1e-3) + 1e-6 * np.sqrt(np.mean(truth ** 2))
        if (np.abs(got - truth) > bound).any():
            probs.append(f"{what}: beyond one bf16 rounding")

    def fp32(got, truth, what):
        truth = np.asarray(truth, np.float64)
        if (np.abs(got - truth) > 1e-5 * (np.abs(truth) + np.sqrt(np.mean(truth ** 2)))).any():
            probs.append(f"{what}: not within fp32 accumulation error")

    acts, w16, L = tr["acts"], tr["w16"], len(tr["w16"])
    one_rounding(acts[0], x, "input")
    for i in range(L):
        z = acts[i].astype(np.float64) @ w16[i].astype(np.float64).T + bs[i].astype(np.float64)
        one_rounding(acts[i + 1], np.maximum(z, 0) if i + 1 < L else z, f"layer {i} output")
    lg = acts[L].astype(np.float64)
    e = np.exp(lg - lg.max(1, keepdims=True))
    p = e / e.sum(1, keepdims=True)
    p[np.arange(len(y)), y] -= 1
    one_rounding(tr["dlogits"], p / len(y), "dlogits")
    g = tr["dlogits"].astype(np.float64)
    for i in range(L - 1, -1, -1):
        fp32(tr["dw"][i], g.T @ acts[i].astype(np.float64), f"layer {i} dW")
        fp32(tr["db"][i], g.sum(0), f"layer {i} db")
        if i > 0:
            one_rounding(tr["dx"][i], g @ w16[i].astype(np.float64), f"layer {i} dX")
            g = np.where(acts[i] > 0, tr["dx"][i], 0.0).astype(np.float64)
    return probs


def test_mixed_step_rounding_points_are_pinned():
    """The mixed oracle rounds to bf16 exactly where the GPU's bf16 step
    stores bf16 tensors and nowhere else (the stored-tensor properties of
    _mixed_trace_problems); planted mistakes in the oracle's output -- a
    dropped rounding of the layer outputs or of dX, an extra rounding of dW,
    db or of the pre-bias sum -- are each caught."""
    dims = [64, 48, 40, 10]
    ws, bs = _mixed_init(dims, 800, True)
    bs = [b + np.float32(0.05) for b in bs]
    x = synth.normal(801, (32, dims[0]))
    y = synth.uniform_int(802, (32,), dims[-1])
    tr = {}
    oracle.mlp_step_mixed([w.copy() for w in ws], [b.copy() for b in bs], [np.zeros_like(w) for w in ws],
                          [np.zeros_like(b) for b in bs], x, y, 0.1, 0.0, trace=tr)
    assert _mixed_trace_problems(tr, bs, x, y) == []
    rnd = oracle.bf16_round
    planted = {
        "dropped output rounding": dict(tr, acts=[tr["acts"][0]] + [
            np.maximum(a.astype(np.float32) @ w.T + b, 0).astype(np.float32) if i + 1 < 3 else
            (a.astype(np.float32) @ w.T + b).astype(np.float32)
            for i, (a, w, b) in enumerate(zip(tr["acts"][:-1], tr["w16"], bs))]),
        "dropped dX rounding": dict(tr, dx=[None] + [
            (tr["dlogits"] if li == 2 else np.where(tr["acts"][li + 1] > 0, tr["dx"][li + 1], 0)).astype(np.float32)
            @ tr["w16"][li] for li in (1, 2)]),
        "rounded dW": dict(tr, dw=[rnd(d) for d in tr["dw"]]),
        "rounded db": dict(tr, db=[rnd(d) for d in tr["db"]]),
        "rounded pre-bias sum": dict(tr, acts=[tr["acts"][0]] + [
            rnd(np.maximum(rnd(a @ w.T) + b, 0)) if i + 1 < 3 else rnd(rnd(a @ w.T) + b)
            for i, (a, w, b) in enumerate(zip(tr["acts"][:-1], tr["w16"], bs))]),
    }
    for name, bad in planted.items():
        assert _mixed_trace_problems(bad, bs, x, y), f"planted mistake not caught: {name}"


@needs_ref
def test_sum_dim_live_bits_and_float64():
    x = synth.normal(810, (37, 53))
    for dim, (o, r, i) in ((0, (1, 37, 53)), (1, (37, 53, 1))):
        out = np.empty(53 if dim == 0 else 37, np.float32)
        oracle.ref_call("ref_sum", x, out, 37, 53, dim)
        assert_bitexact(oracle.sum_dim(x, o, r, i).reshape(-1), out, f"sum dim {dim}")
    y = synth.normal(811, (5, 7, 9))
    assert_close(oracle.sum_dim(y, 5, 7, 9), y.astype(np.float64).sum(1), 1e-6, "3-D middle dim")


@needs_ref
def test_ce_module_live_bits_and_clamp():
    """nn::CrossEntropyLoss::forward: the compiled reference's loss equals the
    oracle's bit for bit, including rows whose target probability is below
    the 1e-9 clamp; a bad target raises in both."""
    logits = synth.normal(820, (64, 10), std=3.0)
    labels = synth.uniform_int(821, (64,), 10)
    logits[5] = np.array([0, 0, 0, 0, 0, 0, 0, 0, 0, 40], np.float32)   # p(t=0) ~ 4e-18 < 1e-9
    labels[5] = 0
    out = np.zeros(1, np.float32)
    oracle.ref_call("ref_ce_module", logits, labels, 64, 10, out)
    assert oracle.ce_module(logits, labels) == float(out[0])
    # the clamped row contributes -log(1e-9) = 20.72
    mask = np.ones(64, bool)
    mask[5] = False
    rest = oracle.ce_module(logits[mask], labels[mask])
    assert abs(float(out[0]) * 64 - (rest * 63 + 20.7232658)) < 1e-3
    bad = labels.copy()
    bad[3] = 10
    with pytest.raises(IndexError):
        oracle.ce_module(logits, bad)
    with pytest.raises(RuntimeError):
        oracle.ref_call("ref_ce_module", logits, bad, 64, 10, out)


# ---------------------------------------------------------------------------
# IEEE half conversions (the checker of the Float16 device paths)
# ---------------------------------------------------------------------------
def _f16_table():
    """Every finite non-negative binary16 value as float64, from the format's
    definition (not from any library): k * 2^-24 for subnormals,
    2^(e-15) * (1 + m/1024) otherwise."""
    h = np.arange(0x7C00, dtype=np.uint32)
    e = (h >> 10).astype(np.int64)
    m = (h & 0x3FF).astype(np.float64)
    return np.where(e == 0, m * 2.0 ** -24, (1.0 + m / 1024.0) * np.exp2((e - 15).astype(np.float64)))


def test_f16_to_f32_is_the_format_definition():
    vals = _f16_table()
    h = np.arange(0x7C00, dtype=np.uint16)
    got = oracle.f16_bits_to_f32(h).astype(np.float64)
    np.testing.assert_array_equal(got, vals)
    np.testing.assert_array_equal(oracle.f16_bits_to_f32(h | 0x8000).astype(np.float64), -vals)
    assert np.isposinf(oracle.f16_bits_to_f32(np.array([0x7C00], np.uint16)))[0]
    assert np.isnan(oracle.f16_bits_to_f32(np.array([0x7E00, 0x7C01, 0xFE00], np.uint16))).all()
    # numpy's own decode agrees for every pattern (NaNs as NaNs)
    allh = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    a, b = oracle.f16_bits_to_f32(allh), allh.view(np.float16).astype(np.float32)
    same = (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))
    assert same.all()


def _nearest_even_by_brute_force(x):
    """binary16 pattern of each float32 x by exhaustive nearest search over the
    format's values (ties to the even pattern, overflow past the midpoint of
    65504 and 2^16 to infinity); float64 holds every distance exactly."""
    vals = np.append(_f16_table(), 65536.0)           # 65536: the pattern 0x7C00 (infinity)
    ax = np.abs(x.astype(np.float64))
    hi = np.clip(np.searchsorted(vals, ax, side="left"), 1, len(vals) - 1)
    lo = hi - 1
    dlo, dhi = ax - vals[lo], vals[hi] - ax
    pick = np.where(dlo < dhi, lo, np.where(dhi < dlo, hi, np.where(lo % 2 == 0, lo, hi)))
    pick = np.where(ax >= 65536.0, len(vals) - 1, pick)
    return (pick.astype(np.uint32) | (np.signbit(x).astype(np.uint32) << 15)).astype(np.uint16)


def test_f32_to_f16_rounds_to_nearest_even():
    vals = _f16_table()
    mids = (vals[:-1] + vals[1:]) / 2                  # every tie between neighbours
    near = np.concatenate([mids, np.nextafter(mids.astype(np.float32), np.float32(np.inf)).astype(np.float64),
                           np.nextafter(mids.astype(np.float32), np.float32(0)).astype(np.float64)])
    rng = np.random.default_rng(0xF16)
    rand = rng.standard_normal(200000) * np.exp2(rng.integers(-30, 18, 200000))
    edges = np.array([0.0, 2.0 ** -25, 2.0 ** -25 * (1 + 2 ** -23), 2.0 ** -26, 2.0 ** -24 * 1.5, 65504.0,
                      65519.99, 65520.0, 65535.0, 1e30, 1e-40])
    x = np.concatenate([near, rand, edges]).astype(np.float32)
    x = np.concatenate([x, -x])
    # every tie is exactly representable in float32
    assert np.array_equal(mids.astype(np.float32).astype(np.float64), mids)
    got = oracle.f32_to_f16_bits(x)
    assert_bitexact(got, _nearest_even_by_brute_force(x), "f32 -> f16 against brute force")
    assert_bitexact(got, x.astype(np.float16).view(np.uint16), "f32 -> f16 against numpy")
    assert (oracle.f32_to_f16_bits(np.array([np.inf, -np.inf], np.float32)) == [0x7C00, 0xFC00]).all()
    assert np.isnan(oracle.f16_bits_to_f32(oracle.f32_to_f16_bits(np.array([np.nan], np.float32)))).all()


def test_planted_f16_rounding_mistakes_are_caught():
    # Truncation and ties-away-from-zero both disagree with the brute-force
    # reference on the tie set, so the check above would catch either.
    vals = _f16_table()
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    want = _nearest_even_by_brute_force(mids)
    trunc = np.searchsorted(vals, mids.astype(np.float64), side="right").astype(np.uint16) - 1
    away = trunc + 1
    assert (trunc != want).any() and (away != want).any()
