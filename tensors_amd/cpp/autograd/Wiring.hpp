// Helpers for attaching backward nodes to op outputs (used by the Tensor op
// wirers and by the nn modules' fused nodes).
#pragma once

#include "autograd/Node.hpp"
#include "tensor/Tensor.hpp"

#include <vector>

namespace tensorforge::wiring {

// Edge to `t`'s AccumulateGrad (which chains on to t's grad_fn when t is an
// intermediate), or an empty edge when t does not require grad.  This is the
// reference's convention for binary ops (autograd/TensorAutograd.cpp:86-126).
[[nodiscard]] Edge accumulator_edge(const Tensor& t);
// Edge to t's grad_fn when it has one, else to its AccumulateGrad (the
// reference's convention for unary ops, autograd/TensorAutograd.cpp:131-150).
[[nodiscard]] Edge source_edge(const Tensor& t);
// Make `out` require grad, set its grad_fn and chain out's own accumulator to it.
void attach(Tensor& out, const NodePtr<Node>& grad_fn, std::vector<Edge> edges);

}  // namespace tensorforge::wiring
