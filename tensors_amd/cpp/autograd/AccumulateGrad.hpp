// Leaf sink (reference autograd/AccumulateGrad.hpp): stores the incoming
// gradient in the tensor's AutogradMeta::grad_ (overwrite, as the reference
// does) and passes it on to the chained grad_fn of an intermediate tensor.
#pragma once

#include "autograd/Node.hpp"
#include "tensor/Tensor.hpp"

#include <memory>
#include <vector>

namespace tensorforge {

struct AutogradMeta;

class AccumulateGrad : public Node {
public:
    explicit AccumulateGrad(std::weak_ptr<AutogradMeta> meta);
    std::vector<Tensor> apply(std::vector<Tensor>&& grads) override;

private:
    std::weak_ptr<AutogradMeta> meta_;
};

}  // namespace tensorforge
