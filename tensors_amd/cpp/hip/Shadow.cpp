#include "hip/Shadow.hpp"

#include "hip/HipBackend.hpp"

#include <mutex>
#include <stdexcept>
#include <unordered_map>

namespace tensorforge::hip {

namespace {

struct Entry {
    std::weak_ptr<StorageImpl> master;
    Tensor shadow;
    uint32_t version;
};

std::mutex g_mutex;
std::unordered_map<const StorageImpl*, Entry> g_shadows;

}  // namespace

Tensor find_shadow(const Tensor& master) {
    std::lock_guard<std::mutex> lock(g_mutex);
    auto it = g_shadows.find(master.storage().get());
    if (it == g_shadows.end() || it->second.master.expired()) return Tensor();
    return it->second.shadow;
}

Tensor shadow_for(const Tensor& master) {
    if (master.device().type != DeviceType::CUDA || master.dtype() != Dtype::Float32)
        throw std::invalid_argument("shadow_for: master must be a Float32 GPU tensor");
    std::lock_guard<std::mutex> lock(g_mutex);
    // Drop entries whose master is gone.
    for (auto it = g_shadows.begin(); it != g_shadows.end();) {
        it = it->second.master.expired() ? g_shadows.erase(it) : std::next(it);
    }
    auto& e = g_shadows[master.storage().get()];
    if (e.master.expired() || e.shadow.numel() != master.numel()) {
        e.master = master.storage();
        e.shadow = Tensor::empty(master.shape(), Dtype::BFloat16, master.device());
        e.version = master.version() + 1;  // force the cast below
    }
    if (e.version != master.version()) {
        cast(master, e.shadow);
        e.version = master.version();
    }
    return e.shadow;
}

void mark_shadow_current(const Tensor& master) {
    std::lock_guard<std::mutex> lock(g_mutex);
    auto it = g_shadows.find(master.storage().get());
    if (it != g_shadows.end()) it->second.version = master.version();
}

}  // namespace tensorforge::hip
