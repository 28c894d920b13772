// loss = mean_r (logsumexp(logits_r) - logits_r[t_r]):
//   dlogits = g * (softmax(logits) - onehot(t)) / N
// One node in place of the train_mlp chain's LogSoftmax + Mul + 2 x Sum +
// 2 x scalar Mul backward nodes (examples/train_mlp.cpp:54-76); on the GPU a
// single streaming kernel using the saved row log-sum-exp.
#pragma once

#include "autograd/Node.hpp"
#include "autograd/SavedTensor.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge {

class CrossEntropyBackward : public Node {
public:
    // lse: saved row log-sum-exp (GPU) or softmax probabilities (CPU).
    CrossEntropyBackward(const Tensor& logits, const Tensor& targets, const Tensor& row_stats)
        : logits_(logits), targets_(targets), stats_(row_stats) {}
    // GPU, fused with the forward: dlogits for an upstream gradient of 1,
    // computed in the forward's pass over the logits.  For BFloat16 logits
    // the dlogits are BFloat16 and the node also keeps the logits and
    // targets: a non-unit upstream gradient g then recomputes g * dlogits in
    // fp32 from the logits, so they are rounded to bf16 once (by the
    // consumer), not once before and once after the scaling.
    struct Precomputed {};
    CrossEntropyBackward(Precomputed, const Tensor& dlogits, const Tensor& logits = Tensor(),
                         const Tensor& targets = Tensor())
        : logits_(logits), targets_(targets), stats_(dlogits), precomputed_(true) {}
    std::vector<Tensor> apply(std::vector<Tensor>&& grads) override;
    void release_saved() override { logits_.reset(); targets_.reset(); stats_.reset(); }
    // The precomputed dlogits are the answer for a unit seed as they are.
    bool accepts_unit_seed() const override { return precomputed_; }

private:
    SavedTensor logits_, targets_, stats_;
    bool precomputed_ = false;
};

}  // namespace tensorforge
