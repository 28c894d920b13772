// Single-threaded backward executor (reference autograd/Engine.hpp:14-31,
// same API): count each reachable node's inbound edges, then run nodes in
// FIFO order as their counts reach zero, routing outputs to InputBuffers.
// GPU nodes only enqueue kernels, so the host walk overlaps device work.
#pragma once

#include "autograd/InputBuffer.hpp"
#include "autograd/Node.hpp"
#include "tensor/Tensor.hpp"

#include <unordered_map>

namespace tensorforge {

class GraphTask {
public:
    std::unordered_map<Node*, int> dependencies_;
    std::unordered_map<Node*, InputBuffer> input_buffers_;
    bool keep_graph_;

    explicit GraphTask(bool keep_graph) : keep_graph_(keep_graph) {}
};

class Engine {
public:
    void execute(NodePtr<Node> root, const Tensor& initial_grad, bool keep_graph);

private:
    void compute_dependencies(Node* root, GraphTask& task);
};

}  // namespace tensorforge
