// SGD with momentum (reference nn/optim/SGD.hpp:29-53, same API):
//   v <- mu * v + g;  p <- p - lr * v        (mu == 0: p <- p - lr * g)
// GPU parameters are updated in place by one fused kernel per parameter
// (p, g, v read once; p, v written once; a registered bf16 shadow of p is
// written in the same pass).  The reference's step() throws for every
// non-scalar parameter (its lr/momentum are Shape{1} tensors and operator*
// does not broadcast, nn/optim/SGD.cpp:50-56); this one implements the
// documented rule.
#pragma once

#include "tensor/Tensor.hpp"

#include <cstddef>
#include <vector>

namespace tensorforge::nn::optim {

class SGD {
public:
    SGD(std::vector<Tensor*> parameters, float lr, float momentum = 0.0f);

    void step();
    void zero_grad();

    [[nodiscard]] std::size_t size() const noexcept { return parameters_.size(); }
    [[nodiscard]] const std::vector<Tensor*>& parameters() const noexcept { return parameters_; }

private:
    std::vector<Tensor*> parameters_;
    float lr_;
    float momentum_;
    std::vector<Tensor> velocity_;
};

}  // namespace tensorforge::nn::optim
