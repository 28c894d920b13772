// Conv2d backward (reference nn/Conv2d.cpp:140-260, without its per-sample
// launches and host accumulation):
//   dW = sum_n dY[n] col[n]^T     one batch-reduced MFMA GEMM
//   dcol[n] = W^T dY[n]           one batched GEMM, then dX = col2im(dcol)
//   db = sum_{n,h,w} dY           deterministic channel reduction
// The forward saves col = im2col(x) when it built one (im2col + GEMM), or x
// when it ran the implicit-GEMM kernel (no col buffer); then the backward
// forms col for dW itself.  Outputs follow
// next_edges_ = {x, W, b}; an empty edge skips that gradient (e.g. dX of the
// network input).
#pragma once

#include "autograd/Node.hpp"
#include "autograd/SavedTensor.hpp"
#include "tensor/Tensor.hpp"

#include <cstdint>

namespace tensorforge {

struct ConvGeometry {
    int64_t N, Cin, H, W, Cout, kH, kW, sh, sw, ph, pw, dh, dw, outH, outW;
};

class Conv2dBackward : public Node {
public:
    // GPU: `x_or_col` is the im2col matrix [N, Cin*kH*kW, outH*outW], or the
    // input when `saved_input` (implicit forward); CPU: the input itself.
    Conv2dBackward(const Tensor& x_or_col, const Tensor& weight, bool has_bias, ConvGeometry g, bool saved_input = false)
        : saved_(x_or_col), w_(weight), has_bias_(has_bias), g_(g), saved_input_(saved_input) {}
    std::vector<Tensor> apply(std::vector<Tensor>&& grads) override;
    void release_saved() override { saved_.reset(); w_.reset(); relu_y_.reset(); }
    // The convolution is followed by a ReLU whose output y this node is then
    // attached to (Conv2dModule::forward_relu): the incoming gradient is the
    // ReLU output's, and dy * (y > 0), ReluBackward's result, is formed
    // inside the gradient kernels where they take it, else explicitly.
    void fuse_relu(const Tensor& y) {
        relu_y_ = SavedTensor(y);
        relu_ = true;
    }

private:
    SavedTensor saved_, w_, relu_y_{Tensor()};
    bool relu_ = false;
    bool has_bias_;
    ConvGeometry g_;
    bool saved_input_ = false;
};

}  // namespace tensorforge
