"""Python-level calls of the hot-path kernels on DeviceArrays.

Each function checks shapes on the host (so a kernel is never launched on a
shape it does not assume), then calls the C ABI.  Names follow the reference
operations they implement; the reference file each one mirrors is cited in
``include/tf_hip.h``.
"""
from __future__ import annotations

from . import _lib
from ._lib import call
from .device import DeviceArray


def _ctx(*arrays: DeviceArray):
    return arrays[0].ctx.handle


def _same(*arrays: DeviceArray) -> int:
    n = arrays[0].size
    for a in arrays[1:]:
        if a.size != n:
            raise ValueError(f"size mismatch: {[x.shape for x in arrays]}")
    return n


def gemm(a: DeviceArray, b: DeviceArray, c: DeviceArray, *, trans_a=False, trans_b=False, alpha=1.0,
         beta=0.0, bias: DeviceArray | None = None, relu=False) -> DeviceArray:
    """c = epi(alpha * op(a) @ op(b) + beta * c) for 2-D row-major arrays."""
    if len(a.shape) != 2 or len(b.shape) != 2 or len(c.shape) != 2:
        raise ValueError("gemm expects 2-D arrays")
    M, K = (a.shape[1], a.shape[0]) if trans_a else a.shape
    Kb, N = (b.shape[1], b.shape[0]) if trans_b else b.shape
    if K != Kb or c.shape != (M, N):
        raise ValueError(f"gemm shape mismatch: op(a) {M}x{K}, op(b) {Kb}x{N}, c {c.shape}")
    if bias is not None and bias.size != N:
        raise ValueError("gemm: bias must have N elements")
    epi = (_lib.TF_EPI_BIAS_RELU if relu else _lib.TF_EPI_BIAS) if bias is not None else \
        (_lib.TF_EPI_RELU if relu else _lib.TF_EPI_NONE)
    call("tf_gemm", _ctx(a), int(trans_a), int(trans_b), M, N, K, alpha, a.ptr, a.shape[1], b.ptr, b.shape[1],
         beta, c.ptr, c.shape[1], a.tf_dtype, c.tf_dtype, epi, bias.ptr if bias is not None else None)
    return c


def gemm_relu_masked(a, mask, b, c, *, trans_a=False, trans_b=False):
    """c = (a * (mask > 0)) as op(a), times op(b), fp32 (tf_gemm_relu_masked);
    mask has a's shape and layout."""
    if len(a.shape) != 2 or len(b.shape) != 2 or len(c.shape) != 2 or tuple(mask.shape) != tuple(a.shape):
        raise ValueError("gemm_relu_masked expects 2-D arrays and a mask shaped as a")
    M, K = (a.shape[1], a.shape[0]) if trans_a else a.shape
    Kb, N = (b.shape[1], b.shape[0]) if trans_b else b.shape
    if K != Kb or c.shape != (M, N):
        raise ValueError(f"gemm_relu_masked shape mismatch: op(a) {M}x{K}, op(b) {Kb}x{N}, c {c.shape}")
    call("tf_gemm_relu_masked", _ctx(a), int(trans_a), int(trans_b), M, N, K, a.ptr, a.shape[1], mask.ptr, b.ptr,
         b.shape[1], c.ptr, c.shape[1])
    return c


def relu_bwd(dy, x, dx):
    call("tf_relu_bwd", _ctx(dy), dy.ptr, x.ptr, dx.ptr, _same(dy, x, dx), dy.tf_dtype)
    return dx


def sigmoid_bwd(dy, y, dx):
    call("tf_sigmoid_bwd", _ctx(dy), dy.ptr, y.ptr, dx.ptr, _same(dy, y, dx), dy.tf_dtype)
    return dx


def tanh_bwd(dy, y, dx):
    call("tf_tanh_bwd", _ctx(dy), dy.ptr, y.ptr, dx.ptr, _same(dy, y, dx), dy.tf_dtype)
    return dx


def relu(x, y):
    call("tf_relu_fwd", _ctx(x), x.ptr, y.ptr, _same(x, y), x.tf_dtype)
    return y


def leaky_relu(x, y, alpha):
    call("tf_leaky_relu_fwd", _ctx(x), x.ptr, y.ptr, _same(x, y), float(alpha), x.tf_dtype)
    return y


def argmax_rows(x, pred, labels=None, correct=None):
    """pred[r] = argmax of row r (int64), the reference's first-max rule;
    with labels and correct, also correct[0] = number of matches."""
    if len(x.shape) != 2 or pred.size != x.shape[0]:
        raise ValueError("argmax_rows: x must be 2-D and pred hold one entry per row")
    if (labels is None) != (correct is None) or (labels is not None and labels.size != x.shape[0]):
        raise ValueError("argmax_rows: labels (one per row) and correct go together")
    call("tf_argmax_rows", _ctx(x), x.ptr, pred.ptr, labels.ptr if labels is not None else None,
         correct.ptr if correct is not None else None, x.shape[0], x.shape[1])
    return pred


def sigmoid(x, y):
    call("tf_sigmoid_fwd", _ctx(x), x.ptr, y.ptr, _same(x, y), x.tf_dtype)
    return y


def tanh(x, y):
    call("tf_tanh_fwd", _ctx(x), x.ptr, y.ptr, _same(x, y), x.tf_dtype)
    return y


def add(a, b, out):
    call("tf_add", _ctx(a), a.ptr, b.ptr, out.ptr, _same(a, b, out), a.tf_dtype)
    return out


def mul(a, b, out):
    call("tf_mul", _ctx(a), a.ptr, b.ptr, out.ptr, _same(a, b, out), a.tf_dtype)
    return out


def _rows_cols(x: DeviceArray):
    if len(x.shape) != 2:
        raise ValueError("row kernels expect 2-D arrays")
    return x.shape


def _check_targets(logits, targets):
    rows, _ = _rows_cols(logits)
    if targets.size != rows or targets.tf_dtype != _lib.TF_I64:
        raise ValueError("targets must be int64 with one entry per row")


def ce_fwd(logits, targets, loss, lse=None, flags=_lib.TF_CE_CHAIN):
    """loss[0] = mean cross-entropy; flags TF_CE_* (0: the train_mlp chain)."""
    rows, cols = _rows_cols(logits)
    _check_targets(logits, targets)
    if lse is not None and lse.size != rows:
        raise ValueError("lse must have one entry per row")
    call("tf_ce_fwd", _ctx(logits), logits.ptr, targets.ptr, loss.ptr, lse.ptr if lse is not None else None,
         rows, cols, flags)
    return loss


def ce_bwd(logits, targets, dlogits, lse=None, grad_loss=None):
    rows, cols = _rows_cols(logits)
    _check_targets(logits, targets)
    _same(logits, dlogits)
    call("tf_ce_bwd", _ctx(logits), logits.ptr, targets.ptr, lse.ptr if lse is not None else None,
         grad_loss.ptr if grad_loss is not None else None, dlogits.ptr, rows, cols)
    return dlogits


def ce_fwd_bwd(logits, targets, loss, dlogits, flags=_lib.TF_CE_CHAIN):
    rows, cols = _rows_cols(logits)
    _check_targets(logits, targets)
    _same(logits, dlogits)
    call("tf_ce_fwd_bwd", _ctx(logits), logits.ptr, targets.ptr, loss.ptr, dlogits.ptr, rows, cols, flags)
    return loss, dlogits


def ce_fwd_bwd_bf16(logits, targets, loss, dlogits, flags=_lib.TF_CE_CHAIN):
    """tf_ce_fwd_bwd on bf16 logits (dlogits in bf16)."""
    rows, cols = _rows_cols(logits)
    _check_targets(logits, targets)
    _same(logits, dlogits)
    if logits.tf_dtype != _lib.TF_BF16 or dlogits.tf_dtype != _lib.TF_BF16:
        raise ValueError("ce_fwd_bwd_bf16: logits and dlogits must be bf16")
    call("tf_ce_fwd_bwd_bf16", _ctx(logits), logits.ptr, targets.ptr, loss.ptr, dlogits.ptr, rows, cols, flags)
    return loss, dlogits


def log_softmax(x, y):
    rows, cols = _rows_cols(x)
    _same(x, y)
    call("tf_log_softmax_fwd", _ctx(x), x.ptr, y.ptr, rows, cols)
    return y


def softmax(x, y):
    rows, cols = _rows_cols(x)
    _same(x, y)
    call("tf_softmax_fwd", _ctx(x), x.ptr, y.ptr, rows, cols)
    return y


def log_softmax_bwd(y, dy, dx):
    rows, cols = _rows_cols(y)
    _same(y, dy, dx)
    call("tf_log_softmax_bwd", _ctx(y), y.ptr, dy.ptr, dx.ptr, rows, cols)
    return dx


def softmax_bwd(y, dy, dx):
    rows, cols = _rows_cols(y)
    _same(y, dy, dx)
    call("tf_softmax_bwd", _ctx(y), y.ptr, dy.ptr, dx.ptr, rows, cols)
    return dx


def colsum(dy, db):
    rows, cols = _rows_cols(dy)
    if db.size != cols:
        raise ValueError("colsum: db must have one entry per column")
    fn = "tf_colsum_bf16" if dy.tf_dtype == _lib.TF_BF16 else "tf_colsum"
    call(fn, _ctx(dy), dy.ptr, db.ptr, rows, cols)
    return db


def relu_bwd_colsum(dy, x, dz, db):
    """dz = relu_bwd(dy, x) and db = colsum(dz) in one call (tf_relu_bwd_colsum)."""
    rows, cols = _rows_cols(dy)
    _same(dy, x, dz)
    if not dy.tf_dtype == x.tf_dtype == dz.tf_dtype:
        raise ValueError("relu_bwd_colsum: dy, x and dz must share a dtype")
    if db.size != cols:
        raise ValueError("relu_bwd_colsum: db must have one entry per column")
    call("tf_relu_bwd_colsum", _ctx(dy), dy.ptr, x.ptr, dz.ptr, db.ptr, rows, cols, dy.tf_dtype)
    return dz, db


def linear_bwd_small(dy, x, w, dx, dw, mask=None):
    """dx = dz w and dw = dz^T x in one launch (tf_linear_bwd_small), dz = dy
    masked by mask > 0 when a mask is given.  dy [M, N], x [M, K], w [N, K]."""
    M, N = dy.shape
    K = w.shape[1]
    if tuple(w.shape) != (N, K) or tuple(x.shape) != (M, K) or tuple(dx.shape) != (M, K) or \
            tuple(dw.shape) != (N, K) or (mask is not None and tuple(mask.shape) != (M, N)):
        raise ValueError("linear_bwd_small: shape mismatch")
    call("tf_linear_bwd_small", _ctx(dy), dy.ptr, mask.ptr if mask is not None else None, x.ptr, w.ptr, dx.ptr,
         dw.ptr, M, N, K)
    return dx, dw


def linear_bwd_narrow(dy, x, w, dx=None, dw=None, db=None):
    """The backward of a Linear layer with at most 16 outputs in one launch
    (tf_linear_bwd_narrow): dx = dy w, dw = dy^T x, db = column sums of dy;
    each output is written when given.  dy [M, N], x [M, K], w [N, K], fp32."""
    M, N = dy.shape
    Nw, K = w.shape
    if Nw != N or (dw is not None and tuple(x.shape) != (M, K)):
        raise ValueError("linear_bwd_narrow: shape mismatch")
    for t, shape in ((dx, (M, K)), (dw, (N, K)), (db, (N,))):
        if t is not None and tuple(t.shape) != shape:
            raise ValueError(f"linear_bwd_narrow: output shape {tuple(t.shape)} != {shape}")
    ptr = lambda t: t.ptr if t is not None else None
    call("tf_linear_bwd_narrow", _ctx(dy), dy.ptr, ptr(x), w.ptr, ptr(dx), ptr(dw), ptr(db), M, N, K)
    return dx, dw, db


def chansum_nchw(dy, db):
    if len(dy.shape) != 4:
        raise ValueError("chansum expects NCHW")
    N, Cc, H, W = dy.shape
    if db.size != Cc:
        raise ValueError("chansum: db must have C entries")
    call("tf_chansum_nchw", _ctx(dy), dy.ptr, db.ptr, N, Cc, H * W)
    return db


def sgd_momentum(p, g, v, lr, mu, p_bf16=None):
    n = _same(p, g) if v is None else _same(p, g, v)
    call("tf_sgd_momentum", _ctx(p), p.ptr, g.ptr, v.ptr if v is not None else None,
         p_bf16.ptr if p_bf16 is not None else None, n, lr, mu)
    return p


SGD_MULTI_MAX = 32


def sgd_momentum_multi(ps, gs, vs, lr, mu, shadows=None):
    """One launch for several parameters: entry i as sgd_momentum(ps[i], gs[i],
    vs[i], lr, mu, shadows[i]); vs / shadows may be None or hold None."""
    import ctypes as C
    count = len(ps)
    if count > SGD_MULTI_MAX or len(gs) != count or (vs is not None and len(vs) != count) or \
            (shadows is not None and len(shadows) != count):
        raise ValueError("sgd_momentum_multi: mismatched or too many parameter lists")
    if count == 0:
        return ps
    ns = [(_same(p, g) if vs is None or vs[i] is None else _same(p, g, vs[i])) for i, (p, g) in enumerate(zip(ps, gs))]
    arr = lambda xs: (C.c_void_p * count)(*[x.ptr if x is not None else None for x in xs])
    p_arr, g_arr = arr(ps), arr(gs)
    v_arr = arr(vs) if vs is not None else None
    s_arr = arr(shadows) if shadows is not None else None
    n_arr = (C.c_int64 * count)(*ns)
    call("tf_sgd_momentum_multi", _ctx(ps[0]), count, C.cast(p_arr, C.c_void_p), C.cast(g_arr, C.c_void_p),
         C.cast(v_arr, C.c_void_p) if v_arr is not None else None,
         C.cast(s_arr, C.c_void_p) if s_arr is not None else None, C.cast(n_arr, C.c_void_p), lr, mu)
    return ps


def gemm_ex(a, b, c, M, N, K, *, lda, ldb, ldc, trans_a=False, trans_b=False, stride_a=0, stride_b=0, stride_c=0,
            batch=1, reduce_batch=False, alpha=1.0, beta=0.0, epilogue=_lib.TF_EPI_NONE, bias=None):
    """Raw tf_gemm_ex on DeviceArrays (extents and strides in elements; the
    caller is responsible for them fitting the arrays — checked here)."""
    def need(rows, ld, stride, nb):
        return (nb - 1) * stride + (rows - 1) * ld if rows > 0 else 0
    a_rows, a_w = (K, M) if trans_a else (M, K)
    b_rows, b_w = (N, K) if trans_b else (K, N)
    nb = batch
    if K > 0 and need(a_rows, lda, stride_a, nb) + a_w > a.size:
        raise ValueError("gemm_ex: A extents exceed the array")
    if K > 0 and need(b_rows, ldb, stride_b, nb) + b_w > b.size:
        raise ValueError("gemm_ex: B extents exceed the array")
    if need(M, ldc, 0 if reduce_batch else stride_c, 1 if reduce_batch else nb) + N > c.size:
        raise ValueError("gemm_ex: C extents exceed the array")
    call("tf_gemm_ex", _ctx(a), int(trans_a), int(trans_b), M, N, K, alpha, a.ptr, lda, stride_a, b.ptr, ldb,
         stride_b, beta, c.ptr, ldc, stride_c, batch, int(reduce_batch), a.tf_dtype, c.tf_dtype, epilogue,
         bias.ptr if bias is not None else None)
    return c


def layernorm_fwd(x, gamma, beta, y, mean, rstd, eps=1e-5):
    rows, cols = _rows_cols(x)
    if gamma.size != cols or beta.size != cols or mean.size != rows or rstd.size != rows:
        raise ValueError("layernorm_fwd: parameter sizes")
    _same(x, y)
    call("tf_layernorm_fwd", _ctx(x), x.ptr, gamma.ptr, beta.ptr, y.ptr, mean.ptr, rstd.ptr, rows, cols, eps)
    return y


def layernorm_bwd(dy, x, gamma, mean, rstd, dx, dgamma, dbeta, reference_compat=False):
    rows, cols = _rows_cols(dy)
    _same(dy, dx)
    if gamma.size != cols or dgamma.size != cols or dbeta.size != cols:
        raise ValueError("layernorm_bwd: parameter sizes")
    if not reference_compat:
        _same(dy, x)
        if mean.size != rows or rstd.size != rows:
            raise ValueError("layernorm_bwd: mean/rstd sizes")
    call("tf_layernorm_bwd", _ctx(dy), dy.ptr, x.ptr if x is not None else None, gamma.ptr,
         mean.ptr if mean is not None else None, rstd.ptr if rstd is not None else None, dx.ptr, dgamma.ptr,
         dbeta.ptr, rows, cols, int(reference_compat))
    return dx


def conv_out(H, k, s, p, d):
    return (H + 2 * p - d * (k - 1) - 1) // s + 1


def im2col(x, col, kH, kW, stride=(1, 1), pad=(0, 0), dil=(1, 1)):
    N, Cc, H, W = x.shape
    oh, ow = conv_out(H, kH, stride[0], pad[0], dil[0]), conv_out(W, kW, stride[1], pad[1], dil[1])
    if col.size != N * Cc * kH * kW * oh * ow:
        raise ValueError("im2col: col has the wrong size")
    call("tf_im2col", _ctx(x), x.ptr, col.ptr, N, Cc, H, W, kH, kW, stride[0], stride[1], pad[0], pad[1],
         dil[0], dil[1], x.tf_dtype)
    return col


def conv2d_fwd(x, w, y, bias=None, stride=(1, 1), pad=(0, 0), dil=(1, 1), relu=False):
    """y = conv(x, w) (+ bias, ReLU) by the implicit-GEMM kernel (no col
    buffer); TFError with TF_ERR_UNSUPPORTED when the shape does not fit it."""
    N, Cc, H, W = x.shape
    Cout, Cw, kH, kW = w.shape
    if Cw != Cc:
        raise ValueError("conv2d_fwd: weight and input channel counts differ")
    oh, ow = conv_out(H, kH, stride[0], pad[0], dil[0]), conv_out(W, kW, stride[1], pad[1], dil[1])
    if tuple(y.shape) != (N, Cout, oh, ow):
        raise ValueError("conv2d_fwd: y has the wrong shape")
    if bias is not None and bias.size != Cout:
        raise ValueError("conv2d_fwd: bias must have one entry per output channel")
    call("tf_conv2d_fwd", _ctx(x), x.ptr, w.ptr, bias.ptr if bias is not None else None, y.ptr, N, Cc, H, W, Cout,
         kH, kW, stride[0], stride[1], pad[0], pad[1], dil[0], dil[1], int(relu))
    return y


def conv2d_bwd_weight(x, dy, dw, stride=(1, 1), pad=(0, 0), dil=(1, 1), db=None, relu_y=None, dz=None):
    """dw = sum over images and pixels of dy (x) col(x), and (db given) the
    bias gradient db = sum of dy over images and pixels, by the implicit-GEMM
    kernel (no col buffer); TFError with TF_ERR_UNSUPPORTED when the shape
    does not fit it.  relu_y given: dy is the gradient of a ReLU's output
    relu_y and dy * (relu_y > 0) is used, and written to dz when given
    (tf_conv2d_bwd_weight_relu)."""
    N, Cc, H, W = x.shape
    Cout, Cw, kH, kW = dw.shape
    if Cw != Cc:
        raise ValueError("conv2d_bwd_weight: dw and input channel counts differ")
    oh, ow = conv_out(H, kH, stride[0], pad[0], dil[0]), conv_out(W, kW, stride[1], pad[1], dil[1])
    if tuple(dy.shape) != (N, Cout, oh, ow):
        raise ValueError("conv2d_bwd_weight: dy has the wrong shape")
    if db is not None and db.size != Cout:
        raise ValueError("conv2d_bwd_weight: db must have one entry per output channel")
    if relu_y is not None:
        if tuple(relu_y.shape) != tuple(dy.shape):
            raise ValueError("conv2d_bwd_weight: relu_y must have dy's shape")
        if dz is not None and tuple(dz.shape) != tuple(dy.shape):
            raise ValueError("conv2d_bwd_weight: dz must have dy's shape")
        call("tf_conv2d_bwd_weight_relu", _ctx(x), x.ptr, dy.ptr, relu_y.ptr, dz.ptr if dz is not None else None,
             dw.ptr, db.ptr if db is not None else None, N, Cc, H, W, Cout, kH, kW, stride[0], stride[1], pad[0],
             pad[1], dil[0], dil[1])
        return dw
    call("tf_conv2d_bwd_weight", _ctx(x), x.ptr, dy.ptr, dw.ptr, db.ptr if db is not None else None, N, Cc, H, W,
         Cout, kH, kW, stride[0], stride[1],
         pad[0], pad[1], dil[0], dil[1])
    return dw


def conv2d_bwd_data(dy, w, dx, stride=(1, 1), pad=(0, 0), dil=(1, 1)):
    """dx = the data gradient of conv(x, w) for upstream dy, by the implicit-GEMM
    kernel over the stride's sub-pixel phases (no dcol buffer, no col2im);
    TFError with TF_ERR_UNSUPPORTED when the shape does not fit it."""
    N, Cc, H, W = dx.shape
    Cout, Cw, kH, kW = w.shape
    if Cw != Cc:
        raise ValueError("conv2d_bwd_data: weight and dx channel counts differ")
    oh, ow = conv_out(H, kH, stride[0], pad[0], dil[0]), conv_out(W, kW, stride[1], pad[1], dil[1])
    if tuple(dy.shape) != (N, Cout, oh, ow):
        raise ValueError("conv2d_bwd_data: dy has the wrong shape")
    call("tf_conv2d_bwd_data", _ctx(dy), dy.ptr, w.ptr, dx.ptr, N, Cc, H, W, Cout, kH, kW, stride[0], stride[1],
         pad[0], pad[1], dil[0], dil[1])
    return dx


def col2im(col, dx, kH, kW, stride=(1, 1), pad=(0, 0), dil=(1, 1)):
    N, Cc, H, W = dx.shape
    oh, ow = conv_out(H, kH, stride[0], pad[0], dil[0]), conv_out(W, kW, stride[1], pad[1], dil[1])
    if col.size != N * Cc * kH * kW * oh * ow:
        raise ValueError("col2im: col has the wrong size")
    call("tf_col2im", _ctx(col), col.ptr, dx.ptr, N, Cc, H, W, kH, kW, stride[0], stride[1], pad[0], pad[1],
         dil[0], dil[1], oh, ow, col.tf_dtype)
    return dx
