// y = x.transpose(d0, d1): dx = dy.transpose(d0, d1) (reference
// autograd/ops/TransposeBackward.hpp:21-33).
#pragma once

#include "autograd/Node.hpp"
#include "tensor/Tensor.hpp"

#include <cstdint>

namespace tensorforge {

class TransposeBackward : public Node {
public:
    TransposeBackward(int64_t dim0, int64_t dim1) : dim0_(dim0), dim1_(dim1) {}
    std::vector<Tensor> apply(std::vector<Tensor>&& grads) override;

private:
    int64_t dim0_, dim1_;
};

}  // namespace tensorforge
