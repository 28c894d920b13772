// z = a * b: {dz * b, a * dz} (reference autograd/ops/MulBackward.hpp:15-31).
#pragma once

#include "autograd/Node.hpp"
#include "autograd/SavedTensor.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge {

class MulBackward : public Node {
public:
    MulBackward(const Tensor& a, const Tensor& b) : a_(a), b_(b) {}
    std::vector<Tensor> apply(std::vector<Tensor>&& grads) override;
    void release_saved() override { a_.reset(); b_.reset(); }

private:
    SavedTensor a_, b_;
};

}  // namespace tensorforge
