// GPU Conv2d with an explicit backward (reference nn/Conv2d.hpp:32-95, same
// API).  Weights start at 0.1 and bias at 0.05 on GPU 0, as in the reference
// constructor.  forward: im2col + one batched MFMA GEMM (bias in the
// epilogue); backward: batch-reduced GEMM for dW, batched GEMM + gather
// col2im for dX and a deterministic channel sum for db — no per-sample
// launches, host synchronisation or host accumulation.
#pragma once

#include "nn/Module.hpp"
#include "tensor/Tensor.hpp"

#include <cstdint>

namespace tensorforge::nn {

struct Conv2dGrad {
    Tensor grad_input;
    Tensor grad_weight;
    Tensor grad_bias;
};

class Conv2d : public Module {
public:
    Conv2d(int64_t in_channels, int64_t out_channels, int64_t kernel_h, int64_t kernel_w, int64_t stride_h = 1,
           int64_t stride_w = 1, int64_t pad_h = 0, int64_t pad_w = 0, int64_t dilation_h = 1, int64_t dilation_w = 1,
           bool bias_enabled = true);

    Tensor forward(Tensor input) override;
    Conv2dGrad backward(Tensor grad_output, Tensor input);

    [[nodiscard]] Parameter& weight() { return parameters_.at("weight"); }
    [[nodiscard]] Parameter& bias() { return parameters_.at("bias"); }

    int64_t in_channels() const noexcept { return in_channels_; }
    int64_t out_channels() const noexcept { return out_channels_; }
    int64_t kernel_h() const noexcept { return kernel_h_; }
    int64_t kernel_w() const noexcept { return kernel_w_; }
    int64_t stride_h() const noexcept { return stride_h_; }
    int64_t stride_w() const noexcept { return stride_w_; }
    int64_t pad_h() const noexcept { return pad_h_; }
    int64_t pad_w() const noexcept { return pad_w_; }
    int64_t dilation_h() const noexcept { return dilation_h_; }
    int64_t dilation_w() const noexcept { return dilation_w_; }
    bool bias_enabled() const noexcept { return bias_enabled_; }

    [[nodiscard]] int64_t out_h(int64_t H) const;
    [[nodiscard]] int64_t out_w(int64_t W) const;

private:
    int64_t in_channels_, out_channels_, kernel_h_, kernel_w_, stride_h_, stride_w_, pad_h_, pad_w_, dilation_h_,
        dilation_w_;
    bool bias_enabled_;
};

}  // namespace tensorforge::nn
