// Tensor's autograd surface (requires_grad / grad / backward) and the wirers
// that attach a backward node to each op's output.  Conventions follow
// reference autograd/TensorAutograd.cpp:31-332; sigmoid and tanh are wired
// (the reference leaves them as no-ops) and SumBackward broadcasts along the
// reduced dimension.
#include "autograd/AccumulateGrad.hpp"
#include "autograd/AutogradMeta.hpp"
#include "autograd/Engine.hpp"
#include "autograd/Wiring.hpp"
#include "autograd/ops/AddBackward.hpp"
#include "autograd/ops/LayerNormBackward.hpp"
#include "autograd/ops/LogSoftmaxBackward.hpp"
#include "autograd/ops/MatmulBackward.hpp"
#include "autograd/ops/MulBackward.hpp"
#include "autograd/ops/ReluBackward.hpp"
#include "autograd/ops/SigmoidBackward.hpp"
#include "autograd/ops/SoftmaxBackward.hpp"
#include "autograd/ops/SumBackward.hpp"
#include "autograd/ops/TanhBackward.hpp"
#include "autograd/ops/TransposeBackward.hpp"
#include "hip/HipBackend.hpp"
#include "tensor/AutogradWirer.hpp"
#include "tensor/factory.hpp"

#include <cmath>
#include <memory>
#include <stdexcept>

namespace tensorforge {

std::shared_ptr<AutogradMeta>& Tensor::autograd_meta() noexcept { return autograd_meta_; }
const std::shared_ptr<AutogradMeta>& Tensor::autograd_meta() const noexcept { return autograd_meta_; }

void Tensor::requires_grad(bool req) {
    if (!autograd_meta_) autograd_meta_ = std::make_shared<AutogradMeta>();
    autograd_meta_->requires_grad_ = req;
    if (req && !autograd_meta_->grad_accumulator_)
        autograd_meta_->grad_accumulator_ = std::make_shared<AccumulateGrad>(autograd_meta_);
}

bool Tensor::requires_grad() const noexcept { return autograd_meta_ && autograd_meta_->requires_grad_; }

Tensor Tensor::grad() const { return autograd_meta_ ? autograd_meta_->grad_ : Tensor(); }

void Tensor::backward() {
    if (!autograd_meta_ || !autograd_meta_->grad_fn_)
        throw std::runtime_error("backward() called on tensor without grad_fn");
    // Seed dL/dL = 1 (a fill kernel for GPU tensors), or an undefined tensor
    // meaning ones for a node that takes it so.
    Shape s = numel() == 0 ? Shape{1} : shape();
    Tensor seed;
    if (!autograd_meta_->grad_fn_->accepts_unit_seed())
        seed = dtype() == Dtype::Float32 ? ones(s, Dtype::Float32, device()) : Tensor::empty(s, dtype(), device());
    Engine engine;
    engine.execute(autograd_meta_->grad_fn_, seed, false);
}

namespace wiring {

Edge accumulator_edge(const Tensor& t) {
    const auto& m = t.autograd_meta();
    return Edge(m ? m->grad_accumulator_ : nullptr, 0);
}

Edge source_edge(const Tensor& t) {
    const auto& m = t.autograd_meta();
    if (!m) return Edge(nullptr, 0);
    return Edge(m->grad_fn_ ? m->grad_fn_ : m->grad_accumulator_, 0);
}

void attach(Tensor& out, const NodePtr<Node>& grad_fn, std::vector<Edge> edges) {
    out.requires_grad(true);
    grad_fn->next_edges_ = std::move(edges);
    out.autograd_meta()->grad_fn_ = grad_fn;
    if (auto& acc = out.autograd_meta()->grad_accumulator_) acc->next_edges_ = {Edge(grad_fn, 0)};
}

}  // namespace wiring

namespace {

using wiring::accumulator_edge;
using wiring::attach;
using wiring::source_edge;

void wire_add(Tensor& out, const Tensor& a, const Tensor& b) {
    if (!(a.requires_grad() || b.requires_grad())) return;
    attach(out, std::make_shared<AddBackward>(), {accumulator_edge(a), accumulator_edge(b)});
}

void wire_mul(Tensor& out, const Tensor& a, const Tensor& b) {
    if (!(a.requires_grad() || b.requires_grad())) return;
    attach(out, std::make_shared<MulBackward>(a, b), {accumulator_edge(a), accumulator_edge(b)});
}

void wire_matmul(Tensor& out, const Tensor& a, const Tensor& b) {
    if (!(a.requires_grad() || b.requires_grad())) return;
    attach(out, std::make_shared<MatmulBackward>(a, b), {accumulator_edge(a), accumulator_edge(b)});
}

template <typename NodeT, typename Saved>
void wire_unary(Tensor& out, const Tensor& x, const Saved& saved) {
    if (!x.requires_grad()) return;
    attach(out, std::make_shared<NodeT>(saved), {source_edge(x)});
}

void wire_relu(Tensor& out, const Tensor& x) { wire_unary<ReluBackward>(out, x, x); }
void wire_sigmoid(Tensor& out, const Tensor& x) { wire_unary<SigmoidBackward>(out, x, out); }
void wire_tanh(Tensor& out, const Tensor& x) { wire_unary<TanhBackward>(out, x, out); }
void wire_leaky_relu(Tensor&, const Tensor&) {}  // not on the training path (as in the reference)
void wire_log(Tensor&, const Tensor&) {}          // idem

void wire_softmax(Tensor& out, const Tensor& x, int64_t) {
    if (!x.requires_grad()) return;
    attach(out, std::make_shared<SoftmaxBackward>(out), {accumulator_edge(x)});
}

void wire_log_softmax(Tensor& out, const Tensor& x, int64_t) {
    if (!x.requires_grad()) return;
    attach(out, std::make_shared<LogSoftmaxBackward>(out), {accumulator_edge(x)});
}

void wire_layernorm(Tensor& out, const Tensor& x, const Tensor& gamma, const Tensor& beta, float eps) {
    if (!(x.requires_grad() || gamma.requires_grad() || beta.requires_grad())) return;
    const int64_t rows = x.shape()[0], cols = x.shape()[1];
    Tensor mean = Tensor::empty(Shape{rows}, Dtype::Float32, x.device());
    Tensor rstd = Tensor::empty(Shape{rows}, Dtype::Float32, x.device());
    if (x.device().type == DeviceType::CUDA) {
        Tensor scratch = Tensor::empty(x.shape(), x.dtype(), x.device());
        hip::layernorm_forward(x, gamma, beta, scratch, mean, rstd, eps);
    } else {
        const float* xp = static_cast<const float*>(x.data());
        for (int64_t r = 0; r < rows; ++r) {
            float s = 0.0f;
            for (int64_t j = 0; j < cols; ++j) s += xp[r * cols + j];
            const float m = s / static_cast<float>(cols);
            float v = 0.0f;
            for (int64_t j = 0; j < cols; ++j) {
                const float d = xp[r * cols + j] - m;
                v += d * d;
            }
            static_cast<float*>(mean.data())[r] = m;
            static_cast<float*>(rstd.data())[r] = 1.0f / std::sqrt(v / static_cast<float>(cols) + eps);
        }
    }
    attach(out, std::make_shared<LayerNormBackward>(x, mean, rstd, gamma),
           {accumulator_edge(x), accumulator_edge(gamma), accumulator_edge(beta)});
}

void wire_sum(Tensor& out, const Tensor& x, int64_t dim, bool) {
    if (!x.requires_grad()) return;
    attach(out, std::make_shared<SumBackward>(x, dim), {source_edge(x)});
}

void wire_transpose(Tensor& out, const Tensor& x, int64_t dim0, int64_t dim1) {
    if (!x.requires_grad()) return;
    attach(out, std::make_shared<TransposeBackward>(dim0, dim1), {source_edge(x)});
}

struct WirerRegistrar {
    WirerRegistrar() { init_tensor_autograd(); }
} g_registrar;

}  // namespace

void init_tensor_autograd() {
    register_add_wirer(&wire_add);
    register_mul_wirer(&wire_mul);
    register_matmul_wirer(&wire_matmul);
    register_relu_wirer(&wire_relu);
    register_sigmoid_wirer(&wire_sigmoid);
    register_tanh_wirer(&wire_tanh);
    register_leaky_relu_wirer(&wire_leaky_relu);
    register_log_wirer(&wire_log);
    register_softmax_wirer(&wire_softmax);
    register_log_softmax_wirer(&wire_log_softmax);
    register_layernorm_wirer(&wire_layernorm);
    register_sum_wirer(&wire_sum);
    register_transpose_wirer(&wire_transpose);
}

}  // namespace tensorforge
