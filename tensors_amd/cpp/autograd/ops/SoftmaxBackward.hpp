// y = softmax(x): dx = y * (dy - sum_j dy*y) (reference
// autograd/ops/SoftmaxBackward.hpp:22-59), one row kernel on the GPU.
#pragma once

#include "autograd/Node.hpp"
#include "autograd/SavedTensor.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge {

class SoftmaxBackward : public Node {
public:
    explicit SoftmaxBackward(const Tensor& y) : y_(y) {}
    std::vector<Tensor> apply(std::vector<Tensor>&& grads) override;
    void release_saved() override { y_.reset(); }

private:
    SavedTensor y_;
};

}  // namespace tensorforge
