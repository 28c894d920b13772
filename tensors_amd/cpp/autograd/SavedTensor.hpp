// A forward tensor saved for backward plus its version at save time
// (reference autograd/SavedTensor.hpp): unpack() throws if the storage was
// modified in place afterwards.
#pragma once

#include "tensor/Tensor.hpp"

#include <cstdint>

namespace tensorforge {

class SavedTensor {
public:
    Tensor data_;
    uint32_t version_at_save_;

    explicit SavedTensor(Tensor t) : data_(std::move(t)), version_at_save_(data_.version()) {}
    const Tensor& unpack() const;
    // Drop the reference (after the node ran).
    void reset() { data_ = Tensor(); }
};

}  // namespace tensorforge
