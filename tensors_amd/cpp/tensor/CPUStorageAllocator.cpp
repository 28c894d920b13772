// CPU allocator (64-byte aligned blocks, released with std::free when the
// last Storage reference goes away) and the per-device allocator / copy
// registry (reference tensor/CPUStorageAllocator.cpp:30-158).
#include "tensor/CPUStorageAllocator.hpp"

#include <cstdlib>
#include <mutex>
#include <new>
#include <stdexcept>

namespace tensorforge {

namespace {

constexpr size_t kAlignment = 64;

struct Slot {
    allocator_dispatch::AllocateFn alloc = nullptr;
    allocator_dispatch::FreeFn free = nullptr;
};

std::mutex& registry_mutex() {
    static std::mutex m;
    return m;
}

Slot& slot(DeviceType t) {
    static Slot slots[4];
    return slots[static_cast<size_t>(t) & 3];
}

allocator_dispatch::CudaCopyFn& copy_slot() {
    static allocator_dispatch::CudaCopyFn fn = nullptr;
    return fn;
}

void host_release(void* p, Device) { std::free(p); }

Storage cpu_alloc(size_t bytes, Device d, Dtype t) { return CPUStorageAllocator::instance().allocate(bytes, d, t); }
void cpu_free(Storage s) { CPUStorageAllocator::instance().free(std::move(s)); }

struct RegisterCpu {
    RegisterCpu() { allocator_dispatch::register_allocator(DeviceType::CPU, cpu_alloc, cpu_free); }
} g_register_cpu;

}  // namespace

Storage CPUStorageAllocator::allocate(size_t size_bytes, Device device, Dtype dtype) {
    if (device.type != DeviceType::CPU) throw std::invalid_argument("CPUStorageAllocator can only allocate CPU storage");
    size_t rounded = ((size_bytes + kAlignment - 1) / kAlignment) * kAlignment;
    if (rounded == 0) rounded = kAlignment;
    void* p = std::aligned_alloc(kAlignment, rounded);
    if (!p) throw std::bad_alloc();
    return std::make_shared<StorageImpl>(p, size_bytes, device, dtype, &host_release);
}

void CPUStorageAllocator::free(Storage storage) {
    if (!storage) return;
    void* p = storage->data();
    storage->release();
    std::free(p);
}

CPUStorageAllocator& CPUStorageAllocator::instance() {
    static CPUStorageAllocator a;
    return a;
}

namespace allocator_dispatch {

void register_allocator(DeviceType type, AllocateFn alloc_fn, FreeFn free_fn) {
    std::lock_guard<std::mutex> lock(registry_mutex());
    slot(type) = Slot{alloc_fn, free_fn};
}

AllocateFn get_allocator(DeviceType type) {
    std::lock_guard<std::mutex> lock(registry_mutex());
    return slot(type).alloc;
}

FreeFn get_deallocator(DeviceType type) {
    std::lock_guard<std::mutex> lock(registry_mutex());
    return slot(type).free;
}

Storage allocate(size_t size_bytes, Device device, Dtype dtype) {
    AllocateFn fn = get_allocator(device.type);
    if (!fn) throw std::runtime_error("No allocator registered for this device type");
    return fn(size_bytes, device, dtype);
}

void free_storage(Storage storage) {
    if (!storage) return;
    if (FreeFn fn = get_deallocator(storage->device().type)) fn(std::move(storage));
}

void register_cuda_copy(CudaCopyFn fn) {
    std::lock_guard<std::mutex> lock(registry_mutex());
    copy_slot() = fn;
}

CudaCopyFn get_cuda_copy() {
    std::lock_guard<std::mutex> lock(registry_mutex());
    return copy_slot();
}

bool cuda_copy_available() { return get_cuda_copy() != nullptr; }

}  // namespace allocator_dispatch

}  // namespace tensorforge
