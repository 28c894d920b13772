// y = tanh(x): dx = dy * (1 - y^2) on the saved output (unwired in the
// reference, autograd/TensorAutograd.cpp:158-164).
#pragma once

#include "autograd/Node.hpp"
#include "autograd/SavedTensor.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge {

class TanhBackward : public Node {
public:
    explicit TanhBackward(const Tensor& output) : y_(output) {}
    std::vector<Tensor> apply(std::vector<Tensor>&& grads) override;
    void release_saved() override { y_.reset(); }

private:
    SavedTensor y_;
};

}  // namespace tensorforge
