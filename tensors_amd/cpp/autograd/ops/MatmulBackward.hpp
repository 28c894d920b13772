// C = A B: dA = dC B^T, dB = A^T dC (reference
// autograd/ops/MatmulBackward.hpp:21-39).  On the GPU both are single MFMA
// GEMM launches with transpose flags (no transpose copies); a gradient whose
// edge is empty (input without grad) is not computed.
#pragma once

#include "autograd/Node.hpp"
#include "autograd/SavedTensor.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge {

class MatmulBackward : public Node {
public:
    MatmulBackward(const Tensor& a, const Tensor& b) : a_(a), b_(b) {}
    std::vector<Tensor> apply(std::vector<Tensor>&& grads) override;
    void release_saved() override { a_.reset(); b_.reset(); }

private:
    SavedTensor a_, b_;
};

}  // namespace tensorforge
