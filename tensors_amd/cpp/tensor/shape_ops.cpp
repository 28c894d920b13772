// View reshaping: the result shares the input's storage.
#include "tensor/shape_ops.hpp"

#include "autograd/Wiring.hpp"
#include "autograd/ops/ReshapeBackward.hpp"

#include <stdexcept>

namespace tensorforge {

Tensor reshape(const Tensor& t, Shape new_shape) {
    if (new_shape.numel() != t.numel()) throw std::invalid_argument("reshape: element count mismatch");
    if (t.stride() != Stride::compute_row_major(t.shape()))
        throw std::invalid_argument("reshape: input must be contiguous");
    Stride s = Stride::compute_row_major(new_shape);
    Tensor out(t.storage(), t.storage_offset(), std::move(new_shape), std::move(s));
    if (t.requires_grad())
        wiring::attach(out, std::make_shared<ReshapeBackward>(t.shape()), {wiring::source_edge(t)});
    return out;
}

Tensor transpose(const Tensor& t, size_t dim0, size_t dim1) {
    if (dim0 >= t.shape().ndim() || dim1 >= t.shape().ndim()) throw std::out_of_range("transpose: dim out of range");
    Shape sh = t.shape();
    Stride st = t.stride();
    std::swap(sh.data()[dim0], sh.data()[dim1]);
    std::swap(st.data()[dim0], st.data()[dim1]);
    return Tensor(t.storage(), t.storage_offset(), std::move(sh), std::move(st));
}

Tensor permute(const Tensor& t, std::vector<size_t> dims) {
    if (dims.size() != t.shape().ndim()) throw std::invalid_argument("permute: wrong number of dims");
    std::vector<int64_t> sh(dims.size()), st(dims.size());
    std::vector<bool> seen(dims.size(), false);
    for (size_t i = 0; i < dims.size(); ++i) {
        if (dims[i] >= dims.size() || seen[dims[i]]) throw std::invalid_argument("permute: not a permutation");
        seen[dims[i]] = true;
        sh[i] = t.shape()[dims[i]];
        st[i] = t.stride()[dims[i]];
    }
    return Tensor(t.storage(), t.storage_offset(), Shape(std::move(sh)), Stride(std::move(st)));
}

}  // namespace tensorforge
