#include "nn/Conv2dModule.hpp"

#include "autograd/Wiring.hpp"
#include "hip/HipBackend.hpp"
#include "nn/ConvCommon.hpp"
#include "tensor/factory.hpp"
#include "tf_hip.h"

#include <cmath>
#include <random>
#include <stdexcept>

namespace tensorforge::nn {

namespace detail {

Tensor conv2d_forward(const Tensor& x, const Tensor& w, const Tensor* bias, int64_t sh, int64_t sw, int64_t ph,
                      int64_t pw, int64_t dh, int64_t dw, bool relu) {
    if (x.shape().ndim() != 4) throw std::invalid_argument("Conv2d.forward expects [N, Cin, H, W]");
    if (x.dtype() != Dtype::Float32) throw std::invalid_argument("Conv2d.forward: only Float32 supported");
    if (x.device() != w.device()) throw std::invalid_argument("Conv2d.forward: input and weight on different devices");
    ConvGeometry g{};
    g.N = x.shape()[0];
    g.Cin = x.shape()[1];
    g.H = x.shape()[2];
    g.W = x.shape()[3];
    g.Cout = w.shape()[0];
    g.kH = w.shape()[2];
    g.kW = w.shape()[3];
    g.sh = sh; g.sw = sw; g.ph = ph; g.pw = pw; g.dh = dh; g.dw = dw;
    if (w.shape()[1] != g.Cin) throw std::invalid_argument("Conv2d.forward: Cin mismatch");
    if (sh <= 0 || sw <= 0 || dh <= 0 || dw <= 0) throw std::invalid_argument("Conv2d.forward: non-positive stride/dilation");
    g.outH = (g.H + 2 * ph - (dh * (g.kH - 1) + 1)) / sh + 1;
    g.outW = (g.W + 2 * pw - (dw * (g.kW - 1) + 1)) / sw + 1;
    if (g.outH <= 0 || g.outW <= 0) throw std::invalid_argument("Conv2d.forward: empty output");
    const int64_t P = g.outH * g.outW, KK = g.Cin * g.kH * g.kW;

    Tensor y = Tensor::empty(Shape{g.N, g.Cout, g.outH, g.outW}, Dtype::Float32, x.device());
    Tensor saved = x;
    bool saved_input = false;
    if (x.device().type == DeviceType::CUDA &&
        hip::conv2d_forward_implicit(x, w, bias, y, sh, sw, ph, pw, dh, dw, relu)) {
        // Implicit GEMM: no col buffer; the backward forms col from x if it
        // needs dW.
        saved_input = true;
    } else if (x.device().type == DeviceType::CUDA) {
        Tensor col = Tensor::empty(Shape{g.N, KK, P}, Dtype::Float32, x.device());
        hip::im2col(x, col, g.kH, g.kW, sh, sw, ph, pw, dh, dw);
        hip::gemm_ex(x.device().index, false, false, g.Cout, P, KK, w.data(), KK, 0, col.data(), P, KK * P, y.data(), P,
                     g.Cout * P, g.N, false, Dtype::Float32, Dtype::Float32,
                     bias ? (relu ? TF_EPI_ROW_BIAS_RELU : TF_EPI_ROW_BIAS) : (relu ? TF_EPI_RELU : TF_EPI_NONE),
                     bias ? static_cast<const float*>(bias->data()) : nullptr);
        saved = col;
    } else {
        if (relu) throw std::invalid_argument("conv2d_forward: fused ReLU is a GPU path");
        // Direct loop in the reference's order (nn/Conv2dModule.cpp:26-70).
        const float* in = static_cast<const float*>(x.data());
        const float* wt = static_cast<const float*>(w.data());
        const float* bp = bias ? static_cast<const float*>(bias->data()) : nullptr;
        float* out = static_cast<float*>(y.data());
        for (int64_t n = 0; n < g.N; ++n)
            for (int64_t co = 0; co < g.Cout; ++co)
                for (int64_t oh = 0; oh < g.outH; ++oh)
                    for (int64_t ow = 0; ow < g.outW; ++ow) {
                        float acc = 0.0f;
                        for (int64_t ci = 0; ci < g.Cin; ++ci)
                            for (int64_t kh = 0; kh < g.kH; ++kh)
                                for (int64_t kw = 0; kw < g.kW; ++kw) {
                                    const int64_t ih = oh * sh - ph + kh * dh;
                                    const int64_t iw = ow * sw - pw + kw * dw;
                                    if (ih < 0 || ih >= g.H || iw < 0 || iw >= g.W) continue;
                                    acc += in[((n * g.Cin + ci) * g.H + ih) * g.W + iw] *
                                           wt[((co * g.Cin + ci) * g.kH + kh) * g.kW + kw];
                                }
                        if (bp) acc += bp[co];
                        out[((n * g.Cout + co) * g.outH + oh) * g.outW + ow] = acc;
                    }
    }
    if (x.requires_grad() || w.requires_grad() || (bias && bias->requires_grad())) {
        auto node = std::make_shared<Conv2dBackward>(saved, w, bias != nullptr, g, saved_input);
        std::vector<Edge> edges = {wiring::accumulator_edge(x), wiring::accumulator_edge(w),
                                   bias ? wiring::accumulator_edge(*bias) : Edge(nullptr, 0)};
        // With relu: the gradient of the convolution then relu(), without the
        // pre-activation tensor (the ReLU mask is y > 0), formed by the
        // convolution's node itself (Conv2dBackward::fuse_relu), so the
        // masked gradient needs no pass of its own.
        if (relu) node->fuse_relu(y);
        wiring::attach(y, node, std::move(edges));
    }
    return y;
}

}  // namespace detail

Conv2dModule::Conv2dModule(int in_channels, int out_channels, int kernel_size, int stride, int padding, int dilation,
                           bool bias)
    : in_channels_(in_channels), out_channels_(out_channels), kernel_size_(kernel_size), stride_(stride),
      padding_(padding), dilation_(dilation), bias_enabled_(bias) {
    // Kaiming-uniform with fan_in = Cin * k * k from the fixed-seed mt19937
    // the reference uses (nn/Conv2dModule.cpp:88-97), so weights match it.
    Tensor w = Tensor::empty(Shape{out_channels, in_channels, kernel_size, kernel_size}, Dtype::Float32, Device::cpu());
    const float bound = std::sqrt(1.0f / static_cast<float>(in_channels * kernel_size * kernel_size));
    std::mt19937 gen(0xC0FFEEu);
    std::uniform_real_distribution<float> u(-bound, bound);
    float* wp = static_cast<float*>(w.data());
    for (int64_t i = 0; i < w.numel(); ++i) wp[i] = u(gen);
    register_parameter("weight", Parameter(std::move(w)));
    if (bias_enabled_) register_parameter("bias", Parameter(zeros(Shape{out_channels}, Dtype::Float32, Device::cpu())));
}

Tensor Conv2dModule::forward(Tensor x) { return forward_impl(std::move(x), false); }

Tensor Conv2dModule::forward_relu(Tensor x) {
    if (x.device().type != DeviceType::CUDA) return forward_impl(std::move(x), false).relu();
    return forward_impl(std::move(x), true);
}

Tensor Conv2dModule::forward_impl(Tensor x, bool relu) {
    if (x.shape().ndim() != 4) throw std::invalid_argument("Conv2dModule.forward expects [N, Cin, H, W]");
    if (x.shape()[1] != in_channels_) throw std::invalid_argument("Conv2dModule.forward: Cin mismatch");
    if (kernel_size_ <= 0 || stride_ <= 0 || dilation_ <= 0)
        throw std::invalid_argument("Conv2dModule.forward: non-positive stride/dilation/kernel");
    const Tensor& w = parameters_.at("weight").data_;
    const Tensor* b = bias_enabled_ ? &parameters_.at("bias").data_ : nullptr;
    return detail::conv2d_forward(x, w, b, stride_, stride_, padding_, padding_, dilation_, dilation_, relu);
}

}  // namespace tensorforge::nn
