// apply() of every backward node, plus the raw (non-wiring) primitives they
// use.  GPU tensors go to libtf_hip kernels through hip/HipBackend; CPU
// tensors run loops in the reference's order.
#include "autograd/ops/AddBackward.hpp"
#include "autograd/ops/Conv2dBackward.hpp"
#include "autograd/ops/CrossEntropyBackward.hpp"
#include "autograd/ops/LayerNormBackward.hpp"
#include "autograd/ops/LinearBackward.hpp"
#include "autograd/ops/LogSoftmaxBackward.hpp"
#include "autograd/ops/MatmulBackward.hpp"
#include "autograd/ops/MulBackward.hpp"
#include "autograd/ops/ReluBackward.hpp"
#include "autograd/ops/ReshapeBackward.hpp"
#include "autograd/ops/SigmoidBackward.hpp"
#include "autograd/ops/SoftmaxBackward.hpp"
#include "autograd/ops/SumBackward.hpp"
#include "autograd/ops/TanhBackward.hpp"
#include "autograd/ops/TransposeBackward.hpp"
#include "autograd/ops/raw.hpp"
#include "hip/HipBackend.hpp"
#include "tensor/Compat.hpp"
#include "tensor/factory.hpp"
#include "tensor/shape_ops.hpp"
#include "tf_hip.h"

#include <cmath>
#include <cstring>
#include <stdexcept>
#include <string>

namespace tensorforge {

namespace {

bool gpu(const Tensor& t) { return t.device().type == DeviceType::CUDA; }
const float* cf(const Tensor& t) { return static_cast<const float*>(t.data()); }
float* mf(Tensor& t) { return static_cast<float*>(t.data()); }

void cpu_f32(const Tensor& t, const char* what) {
    if (t.dtype() != Dtype::Float32) throw std::invalid_argument(std::string(what) + ": CPU path supports Float32 only");
}

bool wants(const Node& n, size_t i) { return i < n.next_edges_.size() && n.next_edges_[i].function != nullptr; }

// Rows / last-dim width of a tensor viewed as [rows x cols].
void as_rows(const Tensor& t, int64_t& rows, int64_t& cols) {
    cols = t.shape().ndim() ? t.shape()[t.shape().ndim() - 1] : 0;
    rows = cols ? t.numel() / cols : 0;
}

}  // namespace

// ---------------------------------------------------------------------------
// raw primitives
// ---------------------------------------------------------------------------
namespace raw {

Tensor empty_like(const Tensor& t) { return Tensor::empty(t.shape(), t.dtype(), t.device()); }

Tensor zeros_like(const Tensor& t) { return zeros(t.shape(), t.dtype(), t.device()); }

Tensor mul(const Tensor& a, const Tensor& b) {
    if (a.numel() != b.numel()) throw std::invalid_argument("raw::mul: size mismatch");
    Tensor out = empty_like(a);
    if (gpu(a)) {
        hip::mul(a, b, out);
        return out;
    }
    cpu_f32(a, "mul");
    for (int64_t i = 0; i < a.numel(); ++i) mf(out)[i] = cf(a)[i] * cf(b)[i];
    return out;
}

Tensor gemm(const Tensor& A, bool ta, const Tensor& B, bool tb) {
    const int64_t M = ta ? A.shape()[1] : A.shape()[0];
    const int64_t K = ta ? A.shape()[0] : A.shape()[1];
    const int64_t N = tb ? B.shape()[0] : B.shape()[1];
    if ((tb ? B.shape()[1] : B.shape()[0]) != K) throw std::invalid_argument("raw::gemm: inner dimensions differ");
    Tensor C = Tensor::empty(Shape{M, N}, A.dtype(), A.device());
    if (gpu(A)) {
        hip::gemm(A, ta, B, tb, C);
        return C;
    }
    cpu_f32(A, "gemm");
    const float* a = cf(A);
    const float* b = cf(B);
    float* c = mf(C);
    const int64_t lda = A.shape()[1], ldb = B.shape()[1];
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            float acc = 0.0f;
            for (int64_t k = 0; k < K; ++k) {
                const float av = ta ? a[k * lda + i] : a[i * lda + k];
                const float bv = tb ? b[j * ldb + k] : b[k * ldb + j];
                acc += av * bv;
            }
            c[i * N + j] = acc;
        }
    return C;
}

Tensor relu_backward(const Tensor& dy, const Tensor& x) {
    Tensor dx = empty_like(dy);
    if (gpu(dy)) {
        hip::relu_backward(dy, x, dx);
        return dx;
    }
    cpu_f32(dy, "relu_backward");
    for (int64_t i = 0; i < dy.numel(); ++i) {
        const float mask = cf(x)[i] > 0.0f ? 1.0f : 0.0f;
        mf(dx)[i] = cf(dy)[i] * mask;
    }
    return dx;
}

Tensor sigmoid_backward(const Tensor& dy, const Tensor& y) {
    Tensor dx = empty_like(dy);
    if (gpu(dy)) {
        hip::sigmoid_backward(dy, y, dx);
        return dx;
    }
    cpu_f32(dy, "sigmoid_backward");
    for (int64_t i = 0; i < dy.numel(); ++i) mf(dx)[i] = cf(dy)[i] * (cf(y)[i] * (1.0f - cf(y)[i]));
    return dx;
}

Tensor tanh_backward(const Tensor& dy, const Tensor& y) {
    Tensor dx = empty_like(dy);
    if (gpu(dy)) {
        hip::tanh_backward(dy, y, dx);
        return dx;
    }
    cpu_f32(dy, "tanh_backward");
    for (int64_t i = 0; i < dy.numel(); ++i) mf(dx)[i] = cf(dy)[i] * (1.0f - cf(y)[i] * cf(y)[i]);
    return dx;
}

Tensor softmax_backward(const Tensor& y, const Tensor& dy) {
    Tensor dx = empty_like(y);
    if (gpu(y)) {
        hip::softmax_backward(y, dy, dx);
        return dx;
    }
    cpu_f32(y, "softmax_backward");
    int64_t R, C;
    as_rows(y, R, C);
    for (int64_t r = 0; r < R; ++r) {
        float s = 0.0f;
        for (int64_t j = 0; j < C; ++j) s += cf(dy)[r * C + j] * cf(y)[r * C + j];
        for (int64_t j = 0; j < C; ++j) {
            const float d = cf(dy)[r * C + j] - s;
            mf(dx)[r * C + j] = cf(y)[r * C + j] * d;
        }
    }
    return dx;
}

Tensor log_softmax_backward(const Tensor& y, const Tensor& dy) {
    Tensor dx = empty_like(y);
    if (gpu(y)) {
        hip::log_softmax_backward(y, dy, dx);
        return dx;
    }
    cpu_f32(y, "log_softmax_backward");
    int64_t R, C;
    as_rows(y, R, C);
    for (int64_t r = 0; r < R; ++r) {
        float s = 0.0f;
        for (int64_t j = 0; j < C; ++j) s += cf(dy)[r * C + j];
        for (int64_t j = 0; j < C; ++j) mf(dx)[r * C + j] = cf(dy)[r * C + j] - std::exp(cf(y)[r * C + j]) * s;
    }
    return dx;
}

Tensor transpose(const Tensor& x, int64_t dim0, int64_t dim1) {
    // The gradient tensor carries no autograd state, so Tensor::transpose's
    // wirer does not attach anything.
    return x.transpose(dim0, dim1);
}

Tensor expand(const Tensor& up, const Tensor& like, int64_t outer, int64_t reduce, int64_t inner) {
    Tensor out = Tensor::empty(like.shape(), up.dtype(), up.device());
    if (gpu(up)) {
        hip::expand_dim(up, out, outer, reduce, inner);
        return out;
    }
    cpu_f32(up, "expand");
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t r = 0; r < reduce; ++r)
            for (int64_t i = 0; i < inner; ++i) mf(out)[(o * reduce + r) * inner + i] = cf(up)[o * inner + i];
    return out;
}

Tensor colsum(const Tensor& dy) {
    int64_t R, C;
    as_rows(dy, R, C);
    Tensor db = Tensor::empty(Shape{C}, Dtype::Float32, dy.device());
    if (gpu(dy)) {
        hip::colsum(dy, db);  // Float32 or BFloat16 dy, fp32 sums
        return db;
    }
    cpu_f32(dy, "colsum");
    for (int64_t c = 0; c < C; ++c) {
        float s = 0.0f;
        for (int64_t r = 0; r < R; ++r) s += cf(dy)[r * C + c];
        mf(db)[c] = s;
    }
    return db;
}

}  // namespace raw

// ---------------------------------------------------------------------------
// nodes
// ---------------------------------------------------------------------------
std::vector<Tensor> MulBackward::apply(std::vector<Tensor>&& grads) {
    const Tensor& a = a_.unpack();
    const Tensor& b = b_.unpack();
    Tensor ga = wants(*this, 0) ? raw::mul(grads[0], b) : Tensor();
    Tensor gb = wants(*this, 1) ? raw::mul(a, grads[0]) : Tensor();
    return {std::move(ga), std::move(gb)};
}

std::vector<Tensor> MatmulBackward::apply(std::vector<Tensor>&& grads) {
    const Tensor& a = a_.unpack();
    const Tensor& b = b_.unpack();
    Tensor ga = wants(*this, 0) ? raw::gemm(grads[0], false, b, true) : Tensor();
    Tensor gb = wants(*this, 1) ? raw::gemm(a, true, grads[0], false) : Tensor();
    return {std::move(ga), std::move(gb)};
}

std::vector<Tensor> ReluBackward::apply(std::vector<Tensor>&& grads) {
    const Tensor& x = input_.unpack();
    const Tensor& g = grads[0];
    auto* linear = fuse_bias_grad_ && !next_edges_.empty()
                       ? dynamic_cast<LinearBackward*>(next_edges_[0].function.get())
                       : nullptr;
    if (linear && gpu(g) && g.dtype() == x.dtype() && g.shape() == x.shape() && g.shape().ndim() >= 1 &&
        g.stride() == Stride::compute_row_major(g.shape()) && linear->sums_bias_grad_of(g.dtype())) {
        // The masked gradient's column sums are the Linear's bias gradient:
        // both in one pass over g and x.
        Tensor dz = raw::empty_like(g);
        Tensor db = Tensor::empty(Shape{g.shape()[g.shape().ndim() - 1]}, Dtype::Float32, g.device());
        hip::relu_backward_colsum(g, x, dz, db);
        linear->set_bias_grad(std::move(db));
        return {std::move(dz)};
    }
    return {raw::relu_backward(g, x)};
}

std::vector<Tensor> SigmoidBackward::apply(std::vector<Tensor>&& grads) {
    return {raw::sigmoid_backward(grads[0], y_.unpack())};
}

std::vector<Tensor> TanhBackward::apply(std::vector<Tensor>&& grads) {
    return {raw::tanh_backward(grads[0], y_.unpack())};
}

std::vector<Tensor> SoftmaxBackward::apply(std::vector<Tensor>&& grads) {
    return {raw::softmax_backward(y_.unpack(), grads[0])};
}

std::vector<Tensor> LogSoftmaxBackward::apply(std::vector<Tensor>&& grads) {
    return {raw::log_softmax_backward(y_.unpack(), grads[0])};
}

std::vector<Tensor> SumBackward::apply(std::vector<Tensor>&& grads) {
    const int64_t nd = static_cast<int64_t>(in_shape_.ndim());
    int64_t outer = 1, inner = 1;
    for (int64_t i = 0; i < nd; ++i) {
        if (i < dim_) outer *= in_shape_[i];
        if (i > dim_) inner *= in_shape_[i];
    }
    Tensor like = Tensor(nullptr, 0, in_shape_, Stride::compute_row_major(in_shape_));
    return {raw::expand(grads[0], like, outer, in_shape_[dim_], inner)};
}

std::vector<Tensor> ReshapeBackward::apply(std::vector<Tensor>&& grads) {
    const Tensor& g = grads[0];
    if (g.stride() == Stride::compute_row_major(g.shape())) return {reshape(g, in_shape_)};
    Tensor c = g.to(g.device());  // contiguous copy
    return {reshape(c, in_shape_)};
}

std::vector<Tensor> TransposeBackward::apply(std::vector<Tensor>&& grads) {
    return {raw::transpose(grads[0], dim0_, dim1_)};
}

std::vector<Tensor> LayerNormBackward::apply(std::vector<Tensor>&& grads) {
    const Tensor& x = x_.unpack();
    const Tensor& mean = mean_.unpack();
    const Tensor& rstd = rstd_.unpack();
    const Tensor& gamma = gamma_.unpack();
    const Tensor& dy = grads[0];
    const bool stub = compat::layernorm_stub_backward();
    Tensor dx = raw::empty_like(dy);
    Tensor dgamma = Tensor::empty(gamma.shape(), Dtype::Float32, gamma.device());
    Tensor dbeta = Tensor::empty(gamma.shape(), Dtype::Float32, gamma.device());
    if (gpu(dy)) {
        hip::layernorm_backward(dy, x, gamma, mean, rstd, dx, dgamma, dbeta, stub);
        return {std::move(dx), std::move(dgamma), std::move(dbeta)};
    }
    cpu_f32(dy, "layer_norm backward");
    int64_t R, C;
    as_rows(dy, R, C);
    const float* g = cf(gamma);
    if (stub) {
        for (int64_t r = 0; r < R; ++r)
            for (int64_t j = 0; j < C; ++j) mf(dx)[r * C + j] = cf(dy)[r * C + j] * g[j];
        std::memset(dgamma.data(), 0, sizeof(float) * C);
        std::memset(dbeta.data(), 0, sizeof(float) * C);
        return {std::move(dx), std::move(dgamma), std::move(dbeta)};
    }
    std::memset(dgamma.data(), 0, sizeof(float) * C);
    std::memset(dbeta.data(), 0, sizeof(float) * C);
    for (int64_t r = 0; r < R; ++r) {
        const float m = cf(mean)[r], rs = cf(rstd)[r];
        float s1 = 0.0f, s2 = 0.0f;
        for (int64_t j = 0; j < C; ++j) {
            const float xh = (cf(x)[r * C + j] - m) * rs;
            const float gg = cf(dy)[r * C + j] * g[j];
            s1 += gg;
            s2 += gg * xh;
            mf(dgamma)[j] += cf(dy)[r * C + j] * xh;
            mf(dbeta)[j] += cf(dy)[r * C + j];
        }
        s1 /= static_cast<float>(C);
        s2 /= static_cast<float>(C);
        for (int64_t j = 0; j < C; ++j) {
            const float xh = (cf(x)[r * C + j] - m) * rs;
            mf(dx)[r * C + j] = rs * (cf(dy)[r * C + j] * g[j] - s1 - xh * s2);
        }
    }
    return {std::move(dx), std::move(dgamma), std::move(dbeta)};
}

std::vector<Tensor> LinearBackward::apply(std::vector<Tensor>&& grads) {
    const Tensor& x = x_.unpack();
    const Tensor& w = w_.unpack();
    Tensor dy = grads[0];
    // Mixed precision: activations/weights in bf16, the upstream gradient
    // arrives in fp32 from the loss — both GEMM operands must share a dtype.
    if (gpu(dy) && dy.dtype() != x.dtype()) {
        Tensor c = Tensor::empty(dy.shape(), x.dtype(), dy.device());
        hip::cast(dy, c);
        dy = c;
    }
    Tensor dx, dw, db;
    bool dx_done = false, dw_done = false;
    const bool gpu32 = gpu(dy) && dy.dtype() == Dtype::Float32 && grad_dtype_ == Dtype::Float32;
    // Both products of a small layer in one launch (with the ReLU mask on
    // dy's load when this node carries the ReLU); a head of at most 16
    // outputs without ReLU takes the narrow kernel below instead, which also
    // forms db.
    if (gpu32 && wants(*this, 0) && wants(*this, 1) && (relu_ || w.shape()[0] > 16) &&
        hip::linear_backward_small(dy, relu_ ? &relu_y_.unpack() : nullptr, x, w, dx, dw))
        dx_done = dw_done = true;
    if (relu_ && !(dx_done && dw_done && !(has_bias_ && wants(*this, 2)))) {
        // dz = dy * (y > 0) folded into the products' load of dy where the
        // kernel takes it; whatever remains gets the explicit masked dz.
        const Tensor& y = relu_y_.unpack();
        if (gpu32) {
            if (wants(*this, 0) && !dx_done) {
                Tensor t = Tensor::empty(Shape{dy.shape()[0], w.shape()[1]}, Dtype::Float32, dy.device());
                if (hip::gemm_relu_masked(dy, false, y, w, false, t)) {
                    dx = std::move(t);
                    dx_done = true;
                }
            }
            if (wants(*this, 1) && !dw_done) {
                Tensor t = Tensor::empty(w.shape(), Dtype::Float32, dy.device());
                if (hip::gemm_relu_masked(dy, true, y, x, false, t)) {
                    dw = std::move(t);
                    dw_done = true;
                }
            }
        }
        if ((wants(*this, 0) && !dx_done) || (wants(*this, 1) && !dw_done) || (has_bias_ && wants(*this, 2)))
            dy = raw::relu_backward(dy, y);
    }
    // Few outputs (a classifier head): dX, dW and db in one launch.
    const bool want_db = has_bias_ && wants(*this, 2) && !pending_db_.storage();
    if (!dx_done && !dw_done && gpu(dy) && grad_dtype_ == Dtype::Float32 && (wants(*this, 0) || wants(*this, 1)) &&
        hip::linear_backward_narrow(dy, x, w, wants(*this, 0) ? &dx : nullptr, wants(*this, 1) ? &dw : nullptr,
                                    want_db ? &db : nullptr)) {
        if (has_bias_ && wants(*this, 2) && !want_db) db = std::move(pending_db_);
        pending_db_ = Tensor();
        return {std::move(dx), std::move(dw), std::move(db)};
    }
    if (wants(*this, 0) && !dx_done) dx = raw::gemm(dy, false, w, false);   // [B x in]
    if (wants(*this, 1) && !dw_done) {
        const int64_t out = w.shape()[0], in = w.shape()[1];
        if (gpu(dy)) {
            dw = Tensor::empty(Shape{out, in}, grad_dtype_, dy.device());
            hip::gemm(dy, true, x, false, dw);                            // dY^T X, fp32 out
        } else {
            dw = raw::gemm(dy, true, x, false);
        }
    }
    if (has_bias_ && wants(*this, 2)) db = pending_db_.storage() ? std::move(pending_db_) : raw::colsum(dy);
    pending_db_ = Tensor();
    return {std::move(dx), std::move(dw), std::move(db)};
}

bool LinearBackward::sums_bias_grad_of(Dtype dt) const {
    return has_bias_ && wants(*this, 2) && x_.data_.storage() && x_.data_.dtype() == dt;
}

std::vector<Tensor> CrossEntropyBackward::apply(std::vector<Tensor>&& grads) {
    if (precomputed_) {
        // dlogits for g = 1; an undefined gradient is the unit seed.
        const Tensor& dl = stats_.unpack();
        if (!grads[0].storage()) return {dl};
        if (dl.dtype() == Dtype::Float32) {
            // A non-unit upstream gradient: g * dl in fp32.
            Tensor d = raw::empty_like(dl);
            hip::scale_by(dl, grads[0], d);
            return {std::move(d)};
        }
        // BFloat16 dlogits hold a rounding already: recompute
        // g * (softmax - onehot) / N in fp32 from the widened logits.
        const Tensor lf = logits_.unpack().to(Dtype::Float32);
        Tensor d = raw::empty_like(lf);
        hip::cross_entropy_backward(lf, targets_.unpack(), nullptr, &grads[0], d);
        return {std::move(d)};
    }
    const Tensor& logits = logits_.unpack();
    const Tensor& targets = targets_.unpack();
    const Tensor& stats = stats_.unpack();
    const Tensor& g = grads[0];
    Tensor d = raw::empty_like(logits);
    if (gpu(logits)) {
        hip::cross_entropy_backward(logits, targets, &stats, &g, d);
        return {std::move(d)};
    }
    // CPU: stats holds softmax probabilities.
    const int64_t N = logits.shape()[0], C = logits.shape()[1];
    const float scale = cf(g)[0] * static_cast<float>(1.0 / static_cast<double>(N));
    const auto* t = static_cast<const int64_t*>(targets.data());
    for (int64_t r = 0; r < N; ++r) {
        const bool ok = t[r] >= 0 && t[r] < C;
        for (int64_t j = 0; j < C; ++j) {
            const float p = cf(stats)[r * C + j];
            mf(d)[r * C + j] = ok ? p * scale - (j == t[r] ? scale : 0.0f) : 0.0f;
        }
    }
    return {std::move(d)};
}

std::vector<Tensor> Conv2dBackward::apply(std::vector<Tensor>&& grads) {
    const Tensor& saved = saved_.unpack();
    const Tensor& w = w_.unpack();
    // With a fused ReLU the incoming gradient is that of the ReLU's output y:
    // the implicit weight gradient applies dy * (y > 0) to its staged tiles
    // (and writes that masked gradient when dX is wanted); every other path
    // uses masked(), ReluBackward's result formed once.
    const Tensor* relu_y = relu_ ? &relu_y_.unpack() : nullptr;
    Tensor dz;
    auto masked = [&]() -> const Tensor& {
        if (!relu_y) return grads[0];
        if (!dz.storage()) dz = raw::relu_backward(grads[0], *relu_y);
        return dz;
    };
    const Tensor& dy_in = grads[0];
    const int64_t P = g_.outH * g_.outW, KK = g_.Cin * g_.kH * g_.kW;
    Tensor dx, dw, db;
    if (gpu(dy_in)) {
        const int dev = dy_in.device().index;
        const bool want_db = has_bias_ && wants(*this, 2);
        bool implicit_dw = false;
        if (wants(*this, 1)) {
            dw = Tensor::empty(w.shape(), Dtype::Float32, dy_in.device());
            if (want_db) db = Tensor::empty(Shape{g_.Cout}, Dtype::Float32, dy_in.device());
            // With the input saved (implicit forward): the implicit weight
            // gradient, which also forms the bias gradient from its dy tiles;
            // else col is formed here for the GEMM.
            // With the ReLU fused and dX wanted, the kernel also writes the
            // masked gradient for the data gradient below.
            Tensor dz_try;
            if (relu_y && wants(*this, 0)) dz_try = raw::empty_like(dy_in);
            implicit_dw = saved_input_ && dy_in.dtype() == Dtype::Float32 &&
                          hip::conv2d_backward_weight_implicit(saved, dy_in, dw, want_db ? &db : nullptr, g_.sh, g_.sw,
                                                               g_.ph, g_.pw, g_.dh, g_.dw, relu_y,
                                                               dz_try.storage() ? &dz_try : nullptr);
            if (implicit_dw && dz_try.storage()) dz = std::move(dz_try);
            if (!implicit_dw) {
                const Tensor& dy = masked();
                Tensor col = saved;
                if (saved_input_) {
                    col = Tensor::empty(Shape{g_.N, KK, P}, Dtype::Float32, dy.device());
                    hip::im2col(saved, col, g_.kH, g_.kW, g_.sh, g_.sw, g_.ph, g_.pw, g_.dh, g_.dw);
                }
                hip::gemm_ex(dev, false, true, g_.Cout, KK, P, dy.data(), P, g_.Cout * P, col.data(), P, KK * P,
                             dw.data(), KK, 0, g_.N, true, dy.dtype(), Dtype::Float32, TF_EPI_NONE, nullptr);
            }
        }
        if (want_db && !implicit_dw) {
            db = Tensor::empty(Shape{g_.Cout}, Dtype::Float32, dy_in.device());
            hip::chansum_nchw(masked(), db);
        }
        if (wants(*this, 0)) {
            dx = Tensor::empty(Shape{g_.N, g_.Cin, g_.H, g_.W}, dy_in.dtype(), dy_in.device());
            // The implicit data gradient (no dcol buffer, no col2im) when the
            // shape fits it, else dcol = W^T dy per image and col2im.
            const bool f32 = dy_in.dtype() == Dtype::Float32 && w.dtype() == Dtype::Float32;
            if (!f32 || !hip::conv2d_backward_data_implicit(masked(), w, dx, g_.sh, g_.sw, g_.ph, g_.pw, g_.dh, g_.dw)) {
                const Tensor& dy = masked();
                Tensor dcol = Tensor::empty(Shape{g_.N, KK, P}, dy.dtype(), dy.device());
                hip::gemm_ex(dev, true, false, KK, P, g_.Cout, w.data(), KK, 0, dy.data(), P, g_.Cout * P, dcol.data(),
                             P, KK * P, g_.N, false, dy.dtype(), dy.dtype(), TF_EPI_NONE, nullptr);
                hip::col2im(dcol, dx, g_.kH, g_.kW, g_.sh, g_.sw, g_.ph, g_.pw, g_.dh, g_.dw);
            }
        }
        return {std::move(dx), std::move(dw), std::move(db)};
    }
    // CPU: the reference's host loop (nn/conv2d_backward_test.cpp:50-106).
    const Tensor& dy = masked();
    cpu_f32(dy, "conv2d backward");
    dx = zeros(Shape{g_.N, g_.Cin, g_.H, g_.W}, Dtype::Float32, Device::cpu());
    dw = zeros(w.shape(), Dtype::Float32, Device::cpu());
    db = zeros(Shape{g_.Cout}, Dtype::Float32, Device::cpu());
    const float* in = cf(saved);
    const float* wt = cf(w);
    const float* go = cf(dy);
    for (int64_t n = 0; n < g_.N; ++n)
        for (int64_t co = 0; co < g_.Cout; ++co)
            for (int64_t oh = 0; oh < g_.outH; ++oh)
                for (int64_t ow = 0; ow < g_.outW; ++ow) {
                    const float gv = go[((n * g_.Cout + co) * g_.outH + oh) * g_.outW + ow];
                    mf(db)[co] += gv;
                    for (int64_t ci = 0; ci < g_.Cin; ++ci)
                        for (int64_t ki = 0; ki < g_.kH; ++ki)
                            for (int64_t kj = 0; kj < g_.kW; ++kj) {
                                const int64_t ih = oh * g_.sh + ki * g_.dh - g_.ph;
                                const int64_t iw = ow * g_.sw + kj * g_.dw - g_.pw;
                                if (ih < 0 || ih >= g_.H || iw < 0 || iw >= g_.W) continue;
                                const int64_t widx = ((co * g_.Cin + ci) * g_.kH + ki) * g_.kW + kj;
                                const int64_t xidx = ((n * g_.Cin + ci) * g_.H + ih) * g_.W + iw;
                                mf(dx)[xidx] += gv * wt[widx];
                                mf(dw)[widx] += gv * in[xidx];
                            }
                }
    if (!has_bias_) db = Tensor();
    return {std::move(dx), std::move(dw), std::move(db)};
}

}  // namespace tensorforge
