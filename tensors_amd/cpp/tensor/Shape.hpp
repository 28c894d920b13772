// tensorforge Shape (reference tensor/Shape.hpp:12-47): a list of extents.
// numel() of a 0-d shape is 0, as in the reference.
#pragma once

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <ostream>
#include <vector>

namespace tensorforge {

class Shape {
public:
    Shape() = default;
    Shape(std::initializer_list<int64_t> dims) : dims_(dims) {}
    explicit Shape(std::vector<int64_t> dims) : dims_(std::move(dims)) {}

    [[nodiscard]] int64_t operator[](size_t i) const { return dims_[i]; }
    [[nodiscard]] int64_t& operator[](size_t i) { return dims_[i]; }
    [[nodiscard]] size_t ndim() const noexcept { return dims_.size(); }
    [[nodiscard]] int64_t numel() const {
        if (dims_.empty()) return 0;
        int64_t n = 1;
        for (int64_t d : dims_) n *= d;
        return n;
    }
    [[nodiscard]] const std::vector<int64_t>& data() const noexcept { return dims_; }
    [[nodiscard]] std::vector<int64_t>& data() noexcept { return dims_; }
    [[nodiscard]] bool operator==(const Shape& o) const noexcept { return dims_ == o.dims_; }
    [[nodiscard]] bool operator!=(const Shape& o) const noexcept { return dims_ != o.dims_; }

private:
    std::vector<int64_t> dims_;
};

inline std::ostream& operator<<(std::ostream& os, const Shape& s) {
    os << "Shape(";
    for (size_t i = 0; i < s.ndim(); ++i) os << (i ? ", " : "") << s[i];
    return os << ")";
}

}  // namespace tensorforge
