// Slicing views along one dimension (share storage with the input).
#include "tensor/slicing.hpp"

#include <stdexcept>

namespace tensorforge {

Tensor slice(const Tensor& t, size_t dim, int64_t start, int64_t end) {
    if (dim >= t.shape().ndim()) throw std::out_of_range("slice: dim out of range");
    const int64_t n = t.shape()[dim];
    if (start < 0) start += n;
    if (end < 0) end += n;
    if (start < 0 || end > n || start > end) throw std::out_of_range("slice: bounds out of range");
    Shape sh = t.shape();
    sh[dim] = end - start;
    const size_t off = t.storage_offset() + static_cast<size_t>(start * t.stride()[dim]);
    return Tensor(t.storage(), off, std::move(sh), t.stride());
}

Tensor narrow(const Tensor& t, size_t dim, int64_t start, int64_t length) {
    return slice(t, dim, start, start + length);
}

Tensor select(const Tensor& t, size_t dim, int64_t index) {
    if (dim >= t.shape().ndim()) throw std::out_of_range("select: dim out of range");
    const int64_t n = t.shape()[dim];
    if (index < 0) index += n;
    if (index < 0 || index >= n) throw std::out_of_range("select: index out of range");
    std::vector<int64_t> sh, st;
    for (size_t i = 0; i < t.shape().ndim(); ++i) {
        if (i == dim) continue;
        sh.push_back(t.shape()[i]);
        st.push_back(t.stride()[i]);
    }
    const size_t off = t.storage_offset() + static_cast<size_t>(index * t.stride()[dim]);
    return Tensor(t.storage(), off, Shape(std::move(sh)), Stride(std::move(st)));
}

}  // namespace tensorforge
