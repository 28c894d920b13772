#include "nn/Conv2d.hpp"

#include "hip/HipBackend.hpp"
#include "nn/ConvCommon.hpp"
#include "tensor/factory.hpp"
#include "tf_hip.h"

#include <stdexcept>

namespace tensorforge::nn {

Conv2d::Conv2d(int64_t in_channels, int64_t out_channels, int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
               int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t dilation_h, int64_t dilation_w,
               bool bias_enabled)
    : in_channels_(in_channels), out_channels_(out_channels), kernel_h_(kernel_h), kernel_w_(kernel_w),
      stride_h_(stride_h), stride_w_(stride_w), pad_h_(pad_h), pad_w_(pad_w), dilation_h_(dilation_h),
      dilation_w_(dilation_w), bias_enabled_(bias_enabled) {
    register_parameter("weight",
                       Parameter(full(Shape{out_channels, in_channels, kernel_h, kernel_w}, 0.1, Dtype::Float32,
                                      Device::cuda(0))));
    if (bias_enabled) register_parameter("bias", Parameter(full(Shape{out_channels}, 0.05, Dtype::Float32, Device::cuda(0))));
}

int64_t Conv2d::out_h(int64_t H) const { return (H + 2 * pad_h_ - dilation_h_ * (kernel_h_ - 1) - 1) / stride_h_ + 1; }
int64_t Conv2d::out_w(int64_t W) const { return (W + 2 * pad_w_ - dilation_w_ * (kernel_w_ - 1) - 1) / stride_w_ + 1; }

Tensor Conv2d::forward(Tensor input) {
    if (input.shape().ndim() != 4) throw std::invalid_argument("Conv2d.forward expects [N, Cin, H, W]");
    if (input.shape()[1] != in_channels_) throw std::invalid_argument("Conv2d.forward: Cin mismatch");
    const Tensor* b = bias_enabled_ ? &bias().data_ : nullptr;
    return detail::conv2d_forward(input, weight().data_, b, stride_h_, stride_w_, pad_h_, pad_w_, dilation_h_,
                                  dilation_w_);
}

Conv2dGrad Conv2d::backward(Tensor grad_output, Tensor input) {
    if (input.device().type != DeviceType::CUDA || grad_output.device().type != DeviceType::CUDA)
        throw std::invalid_argument("Conv2d.backward: tensors must be on the GPU");
    if (input.shape().ndim() != 4 || grad_output.shape().ndim() != 4)
        throw std::invalid_argument("Conv2d.backward expects 4-D tensors");
    const int64_t N = input.shape()[0], Cin = input.shape()[1], H = input.shape()[2], W = input.shape()[3];
    const int64_t oh = out_h(H), ow = out_w(W);
    if (grad_output.shape() != Shape{N, out_channels_, oh, ow})
        throw std::invalid_argument("Conv2d.backward: grad_output shape mismatch");
    const int64_t P = oh * ow, KK = Cin * kernel_h_ * kernel_w_;
    const int dev = input.device().index;
    const Tensor& w = weight().data_;

    // Implicit-GEMM weight and data gradients (no col / dcol buffers) when
    // the shape fits their LDS layouts; else the im2col / col2im forms.
    Conv2dGrad g;
    g.grad_weight = Tensor::empty(w.shape(), Dtype::Float32, input.device());
    g.grad_bias = bias_enabled_ ? Tensor::empty(Shape{out_channels_}, Dtype::Float32, input.device())
                                : zeros(Shape{out_channels_}, Dtype::Float32, input.device());
    const bool db_done = hip::conv2d_backward_weight_implicit(input, grad_output, g.grad_weight,
                                                              bias_enabled_ ? &g.grad_bias : nullptr, stride_h_,
                                                              stride_w_, pad_h_, pad_w_, dilation_h_, dilation_w_);
    if (!db_done) {
        Tensor col = Tensor::empty(Shape{N, KK, P}, Dtype::Float32, input.device());
        hip::im2col(input, col, kernel_h_, kernel_w_, stride_h_, stride_w_, pad_h_, pad_w_, dilation_h_, dilation_w_);
        hip::gemm_ex(dev, false, true, out_channels_, KK, P, grad_output.data(), P, out_channels_ * P, col.data(), P,
                     KK * P, g.grad_weight.data(), KK, 0, N, true, Dtype::Float32, Dtype::Float32, TF_EPI_NONE, nullptr);
    }
    g.grad_input = Tensor::empty(input.shape(), Dtype::Float32, input.device());
    if (!hip::conv2d_backward_data_implicit(grad_output, w, g.grad_input, stride_h_, stride_w_, pad_h_, pad_w_,
                                            dilation_h_, dilation_w_)) {
        Tensor dcol = Tensor::empty(Shape{N, KK, P}, Dtype::Float32, input.device());
        hip::gemm_ex(dev, true, false, KK, P, out_channels_, w.data(), KK, 0, grad_output.data(), P,
                     out_channels_ * P, dcol.data(), P, KK * P, N, false, Dtype::Float32, Dtype::Float32, TF_EPI_NONE,
                     nullptr);
        hip::col2im(dcol, g.grad_input, kernel_h_, kernel_w_, stride_h_, stride_w_, pad_h_, pad_w_, dilation_h_,
                    dilation_w_);
    }
    if (bias_enabled_ && !db_done) hip::chansum_nchw(grad_output, g.grad_bias);
    return g;
}

}  // namespace tensorforge::nn
