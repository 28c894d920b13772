// y = sigmoid(x): dx = dy * y * (1 - y) on the saved output.  The reference
// leaves sigmoid unwired (autograd/TensorAutograd.cpp:152-156); this node
// implements the derivative stated there.
#pragma once

#include "autograd/Node.hpp"
#include "autograd/SavedTensor.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge {

class SigmoidBackward : public Node {
public:
    explicit SigmoidBackward(const Tensor& output) : y_(output) {}
    std::vector<Tensor> apply(std::vector<Tensor>&& grads) override;
    void release_saved() override { y_.reset(); }

private:
    SavedTensor y_;
};

}  // namespace tensorforge
