// y = sum(x, dim): dx = dy broadcast back along `dim`.  The reference copies
// dy[0] everywhere (autograd/ops/SumBackward.hpp:35-37), which is right only
// for a uniform upstream gradient; this node broadcasts along the reduced
// dimension, equal to the reference wherever the reference is right.
#pragma once

#include "autograd/Node.hpp"
#include "tensor/Shape.hpp"
#include "tensor/Tensor.hpp"

#include <cstdint>

namespace tensorforge {

class SumBackward : public Node {
public:
    SumBackward(const Tensor& input, int64_t dim) : in_shape_(input.shape()), dim_(dim) {}
    std::vector<Tensor> apply(std::vector<Tensor>&& grads) override;

private:
    Shape in_shape_;
    int64_t dim_;
};

}  // namespace tensorforge
