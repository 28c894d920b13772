// tensorforge Stride (reference tensor/Stride.hpp:13-54): element strides.
#pragma once

#include "tensor/Shape.hpp"

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <ostream>
#include <vector>

namespace tensorforge {

class Stride {
public:
    Stride() = default;
    Stride(std::initializer_list<int64_t> s) : strides_(s) {}
    explicit Stride(std::vector<int64_t> s) : strides_(std::move(s)) {}

    [[nodiscard]] int64_t operator[](size_t i) const { return strides_[i]; }
    [[nodiscard]] int64_t& operator[](size_t i) { return strides_[i]; }
    [[nodiscard]] size_t ndim() const noexcept { return strides_.size(); }
    [[nodiscard]] const std::vector<int64_t>& data() const noexcept { return strides_; }
    [[nodiscard]] std::vector<int64_t>& data() noexcept { return strides_; }
    [[nodiscard]] bool operator==(const Stride& o) const noexcept { return strides_ == o.strides_; }
    [[nodiscard]] bool operator!=(const Stride& o) const noexcept { return strides_ != o.strides_; }

    // Row-major (C order) strides of `shape`: the last dimension is contiguous.
    [[nodiscard]] static Stride compute_row_major(const Shape& shape) {
        std::vector<int64_t> s(shape.ndim());
        int64_t acc = 1;
        for (size_t i = shape.ndim(); i-- > 0;) {
            s[i] = acc;
            acc *= shape[i];
        }
        return Stride(std::move(s));
    }

private:
    std::vector<int64_t> strides_;
};

inline std::ostream& operator<<(std::ostream& os, const Stride& s) {
    os << "Stride(";
    for (size_t i = 0; i < s.ndim(); ++i) os << (i ? ", " : "") << s[i];
    return os << ")";
}

}  // namespace tensorforge
