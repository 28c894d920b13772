// y = x W^T (+ b), one node for nn::Linear: dX = dY W, dW = dY^T X,
// db = sum_rows dY.  The reference reaches the same dW through
// MatmulBackward + TransposeBackward with two transpose copies
// (nn/Linear.cpp:61-63, autograd/ops/TransposeBackward.hpp:26-28); here
// each gradient is one GEMM written directly in W's layout.  Outputs follow
// next_edges_ = {x, W, b}; an empty edge skips that gradient.
#pragma once

#include "autograd/Node.hpp"
#include "autograd/SavedTensor.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge {

class LinearBackward : public Node {
public:
    // `weight` is the tensor the forward multiplied with (the bf16 shadow in
    // mixed precision); dW is produced in `grad_dtype` on its device.
    LinearBackward(const Tensor& x, const Tensor& weight, bool has_bias, Dtype grad_dtype)
        : x_(x), w_(weight), has_bias_(has_bias), grad_dtype_(grad_dtype) {}
    std::vector<Tensor> apply(std::vector<Tensor>&& grads) override;
    void release_saved() override { x_.reset(); w_.reset(); relu_y_.reset(); pending_db_ = Tensor(); }
    // The layer is followed by a ReLU whose output y this node is then
    // attached to (Linear::forward_relu without bias): the incoming gradient
    // is the ReLU output's, and ReluBackward's dy * (y > 0) is applied by the
    // products as they load dy, else formed explicitly first.
    void fuse_relu(const Tensor& y) {
        relu_y_ = SavedTensor(y);
        relu_ = true;
    }
    // True when apply() will sum an upstream gradient of dtype `dt` into a
    // bias gradient as it arrives (no cast first).
    bool sums_bias_grad_of(Dtype dt) const;
    // A bias gradient already computed from the upstream gradient this node
    // is about to receive (by the ReluBackward in front of it); apply() uses
    // it instead of summing the columns again.
    void set_bias_grad(Tensor db) { pending_db_ = std::move(db); }

private:
    SavedTensor x_, w_, relu_y_{Tensor()};
    bool relu_ = false;
    bool has_bias_;
    Dtype grad_dtype_;
    Tensor pending_db_;
};

}  // namespace tensorforge
