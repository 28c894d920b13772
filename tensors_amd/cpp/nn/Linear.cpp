#include "nn/Linear.hpp"

#include "autograd/Wiring.hpp"
#include "autograd/ops/LinearBackward.hpp"
#include "autograd/ops/ReluBackward.hpp"
#include "hip/HipBackend.hpp"
#include "hip/Shadow.hpp"
#include "tensor/Compat.hpp"
#include "tensor/factory.hpp"

#include <cmath>
#include <random>
#include <stdexcept>

namespace tensorforge::nn {

Linear::Linear(int in_features, int out_features, bool bias)
    : in_features_(in_features), out_features_(out_features), bias_enabled_(bias) {
    // Kaiming-uniform, fan_in: U(-sqrt(1/in), sqrt(1/in)) from a fixed-seed
    // mt19937 — the same draw as the reference (nn/Linear.cpp:21-29) so
    // models start from identical weights.
    Tensor w = Tensor::empty(Shape{out_features, in_features}, Dtype::Float32, Device::cpu());
    const float bound = std::sqrt(1.0f / static_cast<float>(in_features));
    std::mt19937 gen(0xC0FFEEu);
    std::uniform_real_distribution<float> u(-bound, bound);
    float* wp = static_cast<float*>(w.data());
    for (int64_t i = 0; i < w.numel(); ++i) wp[i] = u(gen);
    register_parameter("weight", Parameter(std::move(w)));
    if (bias_enabled_) register_parameter("bias", Parameter(zeros(Shape{out_features}, Dtype::Float32, Device::cpu())));
}

void Linear::set_compute_dtype(Dtype dtype) {
    if (dtype != Dtype::Float32 && dtype != Dtype::BFloat16)
        throw std::invalid_argument("Linear: compute dtype must be Float32 or BFloat16");
    compute_dtype_ = dtype;
}

Tensor Linear::forward(Tensor x) { return forward_impl(std::move(x), false); }

Tensor Linear::forward_relu(Tensor x) {
    if (x.device().type != DeviceType::CUDA) return forward_impl(std::move(x), false).relu();
    return forward_impl(std::move(x), true);
}

Tensor Linear::forward_impl(Tensor x, bool relu) {
    if (x.shape().ndim() != 2) throw std::invalid_argument("Linear.forward expects 2D input [N, in_features]");
    if (x.shape()[1] != in_features_) throw std::invalid_argument("Linear.forward: in_features mismatch");
    const Tensor& W = parameters_.at("weight").data_;
    if (x.device() != W.device()) throw std::invalid_argument("Linear.forward: input and weight on different devices");
    const bool use_bias = bias_enabled_ && !compat::linear_drops_bias();
    const Tensor* b = use_bias ? &parameters_.at("bias").data_ : nullptr;
    const int64_t B = x.shape()[0];

    Tensor y;
    NodePtr<LinearBackward> node;
    if (x.device().type == DeviceType::CUDA) {
        if (compute_dtype_ == Dtype::BFloat16) {
            if (x.dtype() != Dtype::BFloat16) x = x.to(Dtype::BFloat16);
            Tensor w16 = hip::shadow_for(W);
            y = Tensor::empty(Shape{B, out_features_}, Dtype::BFloat16, x.device());
            hip::gemm(x, false, w16, true, y, 1.0f, 0.0f, b, relu);
            if (x.requires_grad() || W.requires_grad() || (b && b->requires_grad()))
                node = std::make_shared<LinearBackward>(x, w16, use_bias, Dtype::Float32);
        } else {
            if (x.dtype() != Dtype::Float32) throw std::invalid_argument("Linear.forward: Float32 input expected");
            y = Tensor::empty(Shape{B, out_features_}, Dtype::Float32, x.device());
            hip::gemm(x, false, W, true, y, 1.0f, 0.0f, b, relu);
            if (x.requires_grad() || W.requires_grad() || (b && b->requires_grad()))
                node = std::make_shared<LinearBackward>(x, W, use_bias, Dtype::Float32);
        }
    } else {
        if (x.dtype() != Dtype::Float32) throw std::invalid_argument("Linear.forward: only Float32 supported on CPU");
        // y[n][o] = sum_i x[n][i] W[o][i], i ascending (the reference's
        // x.matmul(W^T) loop order), then + b[o].
        y = Tensor::empty(Shape{B, out_features_}, Dtype::Float32, Device::cpu());
        const float* xp = static_cast<const float*>(x.data());
        const float* wp = static_cast<const float*>(W.data());
        float* yp = static_cast<float*>(y.data());
        for (int64_t n = 0; n < B; ++n)
            for (int64_t o = 0; o < out_features_; ++o) {
                float acc = 0.0f;
                for (int64_t i = 0; i < in_features_; ++i) acc += xp[n * in_features_ + i] * wp[o * in_features_ + i];
                yp[n * out_features_ + o] = acc;
            }
        if (b) {
            const float* bp = static_cast<const float*>(b->data());
            for (int64_t n = 0; n < B; ++n)
                for (int64_t o = 0; o < out_features_; ++o) yp[n * out_features_ + o] += bp[o];
        }
        if (x.requires_grad() || W.requires_grad() || (b && b->requires_grad()))
            node = std::make_shared<LinearBackward>(x, W, use_bias, Dtype::Float32);
    }
    if (node) {
        std::vector<Edge> edges = {wiring::accumulator_edge(x), wiring::accumulator_edge(W),
                                   b ? wiring::accumulator_edge(*b) : Edge(nullptr, 0)};
        if (relu && !b && x.device().type == DeviceType::CUDA && compute_dtype_ == Dtype::Float32) {
            // Bias-free fp32: the Linear's node takes the ReLU's backward
            // itself (its products apply the mask as they load dy), so the
            // masked gradient is never written.
            node->fuse_relu(y);
            wiring::attach(y, node, std::move(edges));
        } else if (relu) {
            // The graph of forward() then relu(): ReluBackward -> LinearBackward,
            // without the pre-activation tensor.  The ReLU node's mask is taken
            // from y (y > 0 exactly where the pre-activation is > 0).
            node->next_edges_ = std::move(edges);
            auto relu_node = std::make_shared<ReluBackward>(y);
            relu_node->fuse_bias_grad();
            wiring::attach(y, relu_node, {Edge(node, 0)});
        } else {
            wiring::attach(y, node, std::move(edges));
        }
    }
    return y;
}

}  // namespace tensorforge::nn
