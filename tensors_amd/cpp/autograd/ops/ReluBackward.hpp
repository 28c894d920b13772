// y = max(x, 0): dx = dy * (x > 0 ? 1 : 0) (reference
// autograd/ops/ReluBackward.hpp:17-36), one fused kernel on the GPU.
#pragma once

#include "autograd/Node.hpp"
#include "autograd/SavedTensor.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge {

class ReluBackward : public Node {
public:
    explicit ReluBackward(const Tensor& input) : input_(input) {}
    std::vector<Tensor> apply(std::vector<Tensor>&& grads) override;
    void release_saved() override { input_.reset(); }
    // Set by nn::Linear::forward_relu, whose ReLU output is the only use of
    // the Linear's output: on the GPU apply() then also computes that
    // LinearBackward's bias gradient (the column sums of the masked
    // gradient) in the same pass and hands it over.
    void fuse_bias_grad() { fuse_bias_grad_ = true; }

private:
    SavedTensor input_;
    bool fuse_bias_grad_ = false;
};

}  // namespace tensorforge
