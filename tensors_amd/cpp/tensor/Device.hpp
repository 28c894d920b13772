// tensorforge Device (reference tensor/Device.hpp:8-28).  DeviceType::CUDA is
// kept as the name of "the GPU": on this backend it is an MI355X reached
// through libtf_hip.
#pragma once

#include <cstdint>
#include <ostream>

namespace tensorforge {

enum class DeviceType : uint8_t { CPU, CUDA };

struct Device {
    DeviceType type = DeviceType::CPU;
    int32_t index = 0;

    [[nodiscard]] static Device cpu() noexcept { return {DeviceType::CPU, 0}; }
    [[nodiscard]] static Device cuda(int32_t i = 0) noexcept { return {DeviceType::CUDA, i}; }

    [[nodiscard]] bool operator==(const Device& o) const noexcept { return type == o.type && index == o.index; }
    [[nodiscard]] bool operator!=(const Device& o) const noexcept { return !(*this == o); }
};

inline std::ostream& operator<<(std::ostream& os, const Device& d) {
    if (d.type == DeviceType::CPU) return os << "CPU";
    return os << "CUDA:" << d.index;
}

}  // namespace tensorforge
