// Backward-graph vertex and edge (reference autograd/Node.hpp:17-47, same API).
#pragma once

#include "autograd/IntrusivePtr.hpp"

#include <cstdint>
#include <memory>
#include <vector>

namespace tensorforge {

class Tensor;
class Node;

// An input of a node: the node that produced it and which of that node's
// outputs was used.
struct Edge {
    NodePtr<Node> function;
    uint32_t input_nr = 0;

    Edge() = default;
    Edge(NodePtr<Node> fn, uint32_t nr) : function(std::move(fn)), input_nr(nr) {}
};

// A backward function: given the gradients of its outputs, apply() returns
// the gradients of its inputs, one per entry of next_edges_.
class Node : public std::enable_shared_from_this<Node> {
public:
    std::vector<Edge> next_edges_;
    uint64_t sequence_nr_ = 0;

    Node() = default;
    explicit Node(std::vector<Edge> next_edges) : next_edges_(std::move(next_edges)) {}
    virtual ~Node() = default;

    virtual std::vector<Tensor> apply(std::vector<Tensor>&& grads) = 0;
    // Drop saved tensors once the node has run (keep_graph == false).
    virtual void release_saved() {}
    // True when apply() takes an undefined gradient as "all ones", so that
    // Tensor::backward() on this node's output can skip filling the seed.
    virtual bool accepts_unit_seed() const { return false; }
};

}  // namespace tensorforge
