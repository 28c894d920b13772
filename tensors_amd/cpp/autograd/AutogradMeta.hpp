// Per-tensor autograd state (reference autograd/AutogradMeta.hpp:15-20).
#pragma once

#include "autograd/IntrusivePtr.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge {

class Node;

struct AutogradMeta {
    NodePtr<Node> grad_fn_;
    NodePtr<Node> grad_accumulator_;
    Tensor grad_;
    bool requires_grad_ = false;
};

}  // namespace tensorforge
