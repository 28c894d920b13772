// z = a + b: both inputs receive the upstream gradient
// (reference autograd/ops/AddBackward.hpp:16-25).
#pragma once

#include "autograd/Node.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge {

class AddBackward : public Node {
public:
    AddBackward() = default;
    std::vector<Tensor> apply(std::vector<Tensor>&& grads) override { return {grads[0], grads[0]}; }
};

}  // namespace tensorforge
