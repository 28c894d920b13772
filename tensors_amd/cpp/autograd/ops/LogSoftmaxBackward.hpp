// y = log_softmax(x): dx = dy - exp(y) * sum_j dy (reference
// autograd/ops/LogSoftmaxBackward.hpp:21-62), one row kernel on the GPU.
#pragma once

#include "autograd/Node.hpp"
#include "autograd/SavedTensor.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge {

class LogSoftmaxBackward : public Node {
public:
    explicit LogSoftmaxBackward(const Tensor& y) : y_(y) {}
    std::vector<Tensor> apply(std::vector<Tensor>&& grads) override;
    void release_saved() override { y_.reset(); }

private:
    SavedTensor y_;
};

}  // namespace tensorforge
