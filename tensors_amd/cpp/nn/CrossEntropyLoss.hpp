// Cross-entropy over class logits (reference nn/CrossEntropyLoss.hpp:23,
// same API): forward(logits [N, C], targets [N] Int64) -> mean loss [1].
// The reference module is forward-only; here the loss is wired into autograd
// through one CrossEntropyBackward node (dlogits = g (softmax - onehot) / N).
// GPU: one row kernel computes the loss and saves each row's
// log-sum-exp; BFloat16 logits are promoted to Float32 first.
#pragma once

#include "nn/Module.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge::nn {

class CrossEntropyLoss : public Module {
public:
    CrossEntropyLoss() = default;
    [[nodiscard]] Tensor forward(Tensor logits, Tensor targets);
    [[nodiscard]] Tensor forward(Tensor logits) override;  // throws: targets required
};

}  // namespace tensorforge::nn
