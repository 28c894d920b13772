// Autograd wirer slots (reference tensor/AutogradWirer.hpp:29-76, same API):
// Tensor ops call the registered wirer after computing their output so the
// autograd library can attach a backward node without tensor/ depending on
// autograd/.
#pragma once

#include "tensor/Tensor.hpp"

namespace tensorforge {

using AutogradWirerFn = void (*)(Tensor& out, const Tensor& a, const Tensor& b);
using AutogradUnaryWirerFn = void (*)(Tensor& out, const Tensor& x);
using AutogradSoftmaxWirerFn = void (*)(Tensor& out, const Tensor& x, int64_t dim);
using AutogradLayerNormWirerFn = void (*)(Tensor& out, const Tensor& x, const Tensor& gamma, const Tensor& beta,
                                          float eps);
using AutogradReduceWirerFn = void (*)(Tensor& out, const Tensor& x, int64_t dim, bool keepdim);
using AutogradTransposeWirerFn = void (*)(Tensor& out, const Tensor& x, int64_t dim0, int64_t dim1);

void register_add_wirer(AutogradWirerFn fn);
void register_mul_wirer(AutogradWirerFn fn);
void register_matmul_wirer(AutogradWirerFn fn);
void register_relu_wirer(AutogradUnaryWirerFn fn);
void register_sigmoid_wirer(AutogradUnaryWirerFn fn);
void register_tanh_wirer(AutogradUnaryWirerFn fn);
void register_leaky_relu_wirer(AutogradUnaryWirerFn fn);
void register_log_wirer(AutogradUnaryWirerFn fn);
void register_softmax_wirer(AutogradSoftmaxWirerFn fn);
void register_log_softmax_wirer(AutogradSoftmaxWirerFn fn);
void register_layernorm_wirer(AutogradLayerNormWirerFn fn);
void register_sum_wirer(AutogradReduceWirerFn fn);
void register_transpose_wirer(AutogradTransposeWirerFn fn);

// Registers every wirer above; idempotent.
void init_tensor_autograd();

}  // namespace tensorforge
