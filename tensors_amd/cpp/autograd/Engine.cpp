// Engine::execute / compute_dependencies (algorithm of reference
// autograd/Engine.cpp:5-71: BFS dependency counts, FIFO ready queue).
#include "autograd/Engine.hpp"

#include <algorithm>
#include <deque>

namespace tensorforge {

void Engine::compute_dependencies(Node* root, GraphTask& task) {
    std::deque<Node*> frontier{root};
    task.dependencies_[root] = 0;
    while (!frontier.empty()) {
        Node* n = frontier.front();
        frontier.pop_front();
        for (const Edge& e : n->next_edges_) {
            Node* next = e.function.get();
            if (!next) continue;
            auto [it, inserted] = task.dependencies_.try_emplace(next, 0);
            if (inserted) frontier.push_back(next);
            ++it->second;
        }
    }
}

void Engine::execute(NodePtr<Node> root, const Tensor& initial_grad, bool keep_graph) {
    GraphTask task(keep_graph);
    compute_dependencies(root.get(), task);
    task.input_buffers_[root.get()] = InputBuffer(1);
    task.input_buffers_[root.get()].add(0, initial_grad);

    std::deque<Node*> ready{root.get()};
    while (!ready.empty()) {
        Node* node = ready.front();
        ready.pop_front();
        auto buf = task.input_buffers_.find(node);
        std::vector<Tensor> outs;
        if (buf != task.input_buffers_.end()) {
            outs = node->apply(buf->second.take());
            task.input_buffers_.erase(buf);
        }
        // A node that received nothing still releases its successors, so a
        // successor that also has a live path is not left waiting.
        const size_t n = std::min(node->next_edges_.size(), outs.size());
        for (size_t i = 0; i < node->next_edges_.size(); ++i) {
            const Edge& e = node->next_edges_[i];
            Node* next = e.function.get();
            if (!next) continue;
            // A skipped gradient (no storage) still counts as delivered.
            if (i < n && outs[i].storage()) {
                auto [it, inserted] = task.input_buffers_.try_emplace(next, InputBuffer(1));
                it->second.add(e.input_nr, std::move(outs[i]));
            }
            if (--task.dependencies_[next] == 0) ready.push_back(next);
        }
        if (!keep_graph) node->release_saved();
    }
}

}  // namespace tensorforge
