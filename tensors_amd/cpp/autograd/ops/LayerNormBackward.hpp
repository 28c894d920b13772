// Row LayerNorm backward.  True gradient by default:
//   dx = rstd (g - mean(g) - xhat mean(g xhat)), g = dy gamma,
//   dgamma = sum_rows dy xhat, dbeta = sum_rows dy.
// With compat::layernorm_stub_backward() it reproduces the reference stub
// (autograd/ops/LayerNormBackward.hpp:39-59: dx = dy gamma, zero dgamma/dbeta).
#pragma once

#include "autograd/Node.hpp"
#include "autograd/SavedTensor.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge {

class LayerNormBackward : public Node {
public:
    LayerNormBackward(const Tensor& x, const Tensor& mean, const Tensor& rstd, const Tensor& gamma)
        : x_(x), mean_(mean), rstd_(rstd), gamma_(gamma) {}
    std::vector<Tensor> apply(std::vector<Tensor>&& grads) override;
    void release_saved() override { x_.reset(); mean_.reset(); rstd_.reset(); gamma_.reset(); }

private:
    SavedTensor x_, mean_, rstd_, gamma_;
};

}  // namespace tensorforge
