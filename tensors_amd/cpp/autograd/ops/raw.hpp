// Device-dispatching tensor primitives for backward nodes.  Unlike the
// Tensor methods they never call an autograd wirer, so running a node does
// not grow the graph (the reference builds throw-away nodes there, e.g.
// autograd/ops/MatmulBackward.hpp:29-32).  CPU variants keep the
// reference's loop order.
#pragma once

#include "tensor/Tensor.hpp"

#include <cstdint>

namespace tensorforge::raw {

[[nodiscard]] Tensor empty_like(const Tensor& t);
[[nodiscard]] Tensor zeros_like(const Tensor& t);
[[nodiscard]] Tensor mul(const Tensor& a, const Tensor& b);
// C = op(A) op(B); CPU sums k ascending with a single accumulator.
[[nodiscard]] Tensor gemm(const Tensor& A, bool trans_a, const Tensor& B, bool trans_b);
[[nodiscard]] Tensor relu_backward(const Tensor& dy, const Tensor& x);
[[nodiscard]] Tensor sigmoid_backward(const Tensor& dy, const Tensor& y);
[[nodiscard]] Tensor tanh_backward(const Tensor& dy, const Tensor& y);
[[nodiscard]] Tensor softmax_backward(const Tensor& y, const Tensor& dy);
[[nodiscard]] Tensor log_softmax_backward(const Tensor& y, const Tensor& dy);
[[nodiscard]] Tensor transpose(const Tensor& x, int64_t dim0, int64_t dim1);
// out[o][r][i] = up[o][i] with out shaped like `like`.
[[nodiscard]] Tensor expand(const Tensor& up, const Tensor& like, int64_t outer, int64_t reduce, int64_t inner);
// db[c] = sum_r dy[r][c] over a [rows x cols] view of dy.
[[nodiscard]] Tensor colsum(const Tensor& dy);

}  // namespace tensorforge::raw
