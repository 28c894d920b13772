// y = reshape(x): dx = dy viewed with x's shape (no copy).  The reference's
// reshape is not wired into autograd; wiring it lets a flattened conv output
// feed nn::Linear inside one graph.
#pragma once

#include "autograd/Node.hpp"
#include "tensor/Shape.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge {

class ReshapeBackward : public Node {
public:
    explicit ReshapeBackward(Shape in_shape) : in_shape_(std::move(in_shape)) {}
    std::vector<Tensor> apply(std::vector<Tensor>&& grads) override;

private:
    Shape in_shape_;
};

}  // namespace tensorforge
