// 2-D convolution module (reference nn/Conv2dModule.hpp, same API): weight
// [Cout, Cin, k, k] with the reference's Kaiming-uniform init, bias zeros.
// CPU: the reference's direct loop.  GPU: im2col + one batched MFMA GEMM with
// the bias in its epilogue.  Unlike the reference (forward only) the output is
// wired to a Conv2dBackward node.
#pragma once

#include "nn/Module.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge::nn {

class Conv2dModule : public Module {
public:
    Conv2dModule(int in_channels, int out_channels, int kernel_size, int stride = 1, int padding = 0,
                 int dilation = 1, bool bias = true);

    [[nodiscard]] Tensor forward(Tensor x) override;
    // relu(forward(x)) with the ReLU in the GEMM epilogue on the GPU; same
    // values and backward graph as the two calls (no counterpart in the
    // reference, which has only the separate modules).
    [[nodiscard]] Tensor forward_relu(Tensor x);

private:
    [[nodiscard]] Tensor forward_impl(Tensor x, bool relu);

    int in_channels_;
    int out_channels_;
    int kernel_size_;
    int stride_;
    int padding_;
    int dilation_;
    bool bias_enabled_;
};

}  // namespace tensorforge::nn
