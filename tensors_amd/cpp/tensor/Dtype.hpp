// tensorforge Dtype: same enumerators and values as the reference
// (tensor/Dtype.hpp:9-16), which the C ABI's TF_* codes also use.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string_view>

namespace tensorforge {

enum class Dtype : uint8_t { Float32, Float16, BFloat16, Int32, Int64, Bool };

[[nodiscard]] constexpr size_t dtype_size(Dtype d) noexcept {
    switch (d) {
    case Dtype::Float32: case Dtype::Int32: return 4;
    case Dtype::Float16: case Dtype::BFloat16: return 2;
    case Dtype::Int64: return 8;
    case Dtype::Bool: return 1;
    }
    return 0;
}

[[nodiscard]] constexpr std::string_view dtype_name(Dtype d) noexcept {
    constexpr std::string_view names[] = {"Float32", "Float16", "BFloat16", "Int32", "Int64", "Bool"};
    auto i = static_cast<size_t>(d);
    return i < 6 ? names[i] : std::string_view("Unknown");
}

}  // namespace tensorforge
