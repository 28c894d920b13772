// Collects the gradients flowing into one node from several paths
// (reference autograd/InputBuffer.hpp); fan-in is summed on the tensors'
// device.
#pragma once

#include "tensor/Tensor.hpp"

#include <cstddef>
#include <optional>
#include <vector>

namespace tensorforge {

class InputBuffer {
public:
    InputBuffer() = default;
    explicit InputBuffer(size_t num_outputs);
    void add(size_t pos, Tensor grad);
    std::vector<Tensor> take();

private:
    std::vector<std::optional<Tensor>> buffer_;
};

}  // namespace tensorforge
