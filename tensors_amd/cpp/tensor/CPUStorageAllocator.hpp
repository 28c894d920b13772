// Storage allocators and the per-device allocator / copy dispatch
// (reference tensor/CPUStorageAllocator.hpp:11-85, same API).  The GPU
// allocator registered by the HIP backend serves blocks from the device's
// stream-ordered memory pool.
#pragma once

#include "tensor/Device.hpp"
#include "tensor/Dtype.hpp"
#include "tensor/Storage.hpp"

#include <cstddef>

namespace tensorforge {

class StorageAllocator {
public:
    virtual ~StorageAllocator() = default;
    [[nodiscard]] virtual Storage allocate(size_t size_bytes, Device device, Dtype dtype) = 0;
    virtual void free(Storage storage) = 0;
};

class CPUStorageAllocator : public StorageAllocator {
public:
    [[nodiscard]] Storage allocate(size_t size_bytes, Device device, Dtype dtype) override;
    void free(Storage storage) override;
    static CPUStorageAllocator& instance();
};

namespace allocator_dispatch {

using AllocateFn = Storage (*)(size_t size_bytes, Device device, Dtype dtype);
using FreeFn = void (*)(Storage storage);

void register_allocator(DeviceType type, AllocateFn alloc_fn, FreeFn free_fn);
AllocateFn get_allocator(DeviceType type);
FreeFn get_deallocator(DeviceType type);
[[nodiscard]] Storage allocate(size_t size_bytes, Device device, Dtype dtype);
void free_storage(Storage storage);

enum class CudaCopyKind : int { HostToHost = 0, HostToDevice = 1, DeviceToHost = 2, DeviceToDevice = 3 };
using CudaCopyFn = void (*)(void* dst, const void* src, size_t bytes, CudaCopyKind kind);

void register_cuda_copy(CudaCopyFn fn);
CudaCopyFn get_cuda_copy();
bool cuda_copy_available();

}  // namespace allocator_dispatch

}  // namespace tensorforge
