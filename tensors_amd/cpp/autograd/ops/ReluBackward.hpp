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

private:
    SavedTensor input_;
};

}  // namespace tensorforge
