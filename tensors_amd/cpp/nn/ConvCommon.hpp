// Shared forward of Conv2dModule and Conv2d: computes y and attaches the
// Conv2dBackward node.  relu (GPU only): y = relu(conv) from the GEMM
// epilogue, with a ReluBackward node (mask y > 0) in front of Conv2dBackward.
#pragma once

#include "autograd/ops/Conv2dBackward.hpp"
#include "tensor/Tensor.hpp"

namespace tensorforge::nn::detail {

Tensor conv2d_forward(const Tensor& x, const Tensor& w, const Tensor* bias, int64_t sh, int64_t sw, int64_t ph,
                      int64_t pw, int64_t dh, int64_t dw, bool relu = false);

}  // namespace tensorforge::nn::detail
