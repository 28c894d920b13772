// Fully connected layer y = x W^T + b (reference nn/Linear.hpp:24-37, same
// API).  Weight [out, in] with the reference's Kaiming-uniform init, bias
// zeros.  Unlike the reference (which never adds its bias,
// nn/Linear.cpp:60-63) the bias is used, unless
// compat::set_linear_drops_bias(true).  Forward is one MFMA GEMM with the
// bias in its epilogue; backward is one LinearBackward node.
//
// set_compute_dtype(BFloat16): the fp32 weight stays the parameter (master);
// forward and backward use its bf16 shadow with fp32 accumulation and the
// weight gradient comes out in fp32.
#pragma once

#include "nn/Module.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge::nn {

class Linear : public Module {
public:
    Linear(int in_features, int out_features, bool bias = true);

    [[nodiscard]] Tensor forward(Tensor x) override;
    // relu(forward(x)) with the ReLU in the GEMM epilogue on the GPU (one
    // launch, no pre-activation tensor).  Same values and gradients as the
    // two calls; the backward graph is ReluBackward -> LinearBackward, or,
    // for a bias-free fp32 layer, one LinearBackward that applies the ReLU
    // mask as its products load dy.  No counterpart in the reference, which
    // has only the separate modules.
    [[nodiscard]] Tensor forward_relu(Tensor x);

    [[nodiscard]] int in_features() const noexcept { return in_features_; }
    [[nodiscard]] int out_features() const noexcept { return out_features_; }

    void set_compute_dtype(Dtype dtype);
    [[nodiscard]] Dtype compute_dtype() const noexcept { return compute_dtype_; }

private:
    [[nodiscard]] Tensor forward_impl(Tensor x, bool relu);

    int in_features_;
    int out_features_;
    bool bias_enabled_;
    Dtype compute_dtype_ = Dtype::Float32;
};

}  // namespace tensorforge::nn
