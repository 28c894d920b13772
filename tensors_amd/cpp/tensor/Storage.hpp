// tensorforge StorageImpl / Storage (reference tensor/Storage.hpp:13-57).
//
// Same public surface; one addition that fixes the reference's leak (its
// destructor is defaulted and drops the raw pointer, so no storage is ever
// freed): the allocator that created the block installs a release callback,
// run once when the last Storage reference goes away.  For GPU storage that
// is tf_hip_free: the block goes to its context's cache of freed blocks,
// from which the next allocation of its size class on the same stream takes
// it (stream-ordered, like the pool's own reuse).
#pragma once

#include "tensor/Device.hpp"
#include "tensor/Dtype.hpp"

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <memory>

namespace tensorforge {

class StorageImpl {
public:
    using ReleaseFn = void (*)(void* data, Device device);

    StorageImpl(void* data, size_t size_bytes, Device device, Dtype dtype, ReleaseFn release_fn = nullptr)
        : data_(data), size_bytes_(size_bytes), device_(device), dtype_(dtype), release_fn_(release_fn) {}

    StorageImpl(const StorageImpl&) = delete;
    StorageImpl& operator=(const StorageImpl&) = delete;
    StorageImpl(StorageImpl&&) = delete;
    StorageImpl& operator=(StorageImpl&&) = delete;

    ~StorageImpl() {
        if (data_ != nullptr && release_fn_ != nullptr) release_fn_(data_, device_);
    }

    [[nodiscard]] void* data() noexcept { return data_; }
    [[nodiscard]] const void* data() const noexcept { return data_; }
    [[nodiscard]] size_t size_bytes() const noexcept { return size_bytes_; }
    [[nodiscard]] Device device() const noexcept { return device_; }
    [[nodiscard]] Dtype dtype() const noexcept { return dtype_; }

    [[nodiscard]] uint32_t bump_version() noexcept { return version_.fetch_add(1, std::memory_order_relaxed) + 1; }
    [[nodiscard]] uint32_t current_version() const noexcept { return version_.load(std::memory_order_relaxed); }

    // Forget the block without releasing it (its owner frees it).
    void release() noexcept { data_ = nullptr; }

private:
    void* data_;
    size_t size_bytes_;
    Device device_;
    Dtype dtype_;
    ReleaseFn release_fn_;
    std::atomic<uint32_t> version_{0};
};

using Storage = std::shared_ptr<StorageImpl>;

}  // namespace tensorforge
