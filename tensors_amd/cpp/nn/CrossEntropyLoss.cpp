#include "nn/CrossEntropyLoss.hpp"

#include "autograd/Wiring.hpp"
#include "autograd/ops/CrossEntropyBackward.hpp"
#include "hip/HipBackend.hpp"
#include "tf_hip.h"

#include <cmath>
#include <stdexcept>

namespace tensorforge::nn {

Tensor CrossEntropyLoss::forward(Tensor logits, Tensor targets) {
    const bool on_gpu = logits.device().type == DeviceType::CUDA;
    if (logits.dtype() != Dtype::Float32 && !(on_gpu && logits.dtype() == Dtype::BFloat16))
        throw std::invalid_argument("CrossEntropyLoss: logits must be Float32 (or BFloat16 on the GPU)");
    if (logits.shape().ndim() != 2) throw std::invalid_argument("CrossEntropyLoss: logits must be 2D (N, C)");
    if (targets.dtype() != Dtype::Int64) throw std::invalid_argument("CrossEntropyLoss: targets must be Int64");
    const int64_t N = logits.shape()[0], C = logits.shape()[1];
    if (targets.numel() != N) throw std::invalid_argument("CrossEntropyLoss: targets.numel() must equal logits.shape()[0]");
    if (targets.device() != logits.device()) targets = targets.to(logits.device());

    Tensor loss = Tensor::empty(Shape{1}, Dtype::Float32, logits.device());
    NodePtr<CrossEntropyBackward> node;
    if (on_gpu) {
        // The module's loss (nn/CrossEntropyLoss.cpp:47-58 of the reference):
        // the probability clamped at 1e-9, and a target outside [0, C) makes
        // the loss NaN instead of throwing (a host check would need a
        // device->host copy per step); such a row gets a zero gradient.
        // With a gradient to come, dlogits (for an upstream gradient of 1)
        // are computed in the same pass over the logits as the loss, and the
        // loss mean in the same kernel; the backward node returns them, or
        // scales them by a non-unit upstream gradient.  BFloat16 logits (a
        // bf16 Linear's output) are read as they are and their dlogits come
        // out in BFloat16, the dtype that Linear's backward multiplies in.
        if (logits.dtype() == Dtype::BFloat16 && logits.requires_grad()) {
            Tensor dl = Tensor::empty(logits.shape(), Dtype::BFloat16, logits.device());
            hip::cross_entropy_forward_backward_bf16(logits, targets, loss, dl, TF_CE_MODULE);
            node = std::make_shared<CrossEntropyBackward>(CrossEntropyBackward::Precomputed{}, dl, logits, targets);
            wiring::attach(loss, node, {wiring::accumulator_edge(logits)});
            return loss;
        }
        Tensor lf = logits.dtype() == Dtype::Float32 ? logits : logits.to(Dtype::Float32);
        if (logits.requires_grad()) {
            Tensor dl = Tensor::empty(lf.shape(), Dtype::Float32, logits.device());
            hip::cross_entropy_forward_backward(lf, targets, loss, dl, TF_CE_MODULE);
            node = std::make_shared<CrossEntropyBackward>(CrossEntropyBackward::Precomputed{}, dl);
        } else {
            hip::cross_entropy_forward(lf, targets, loss, nullptr, TF_CE_MODULE);
        }
    } else {
        // softmax -> gather -> clamp(1e-9) -> -log -> mean, as
        // reference nn/CrossEntropyLoss.cpp:36-62.
        Tensor probs = Tensor::empty(logits.shape(), Dtype::Float32, Device::cpu());
        const float* x = static_cast<const float*>(logits.data());
        float* p = static_cast<float*>(probs.data());
        for (int64_t r = 0; r < N; ++r) {
            float mx = x[r * C];
            for (int64_t j = 1; j < C; ++j) mx = x[r * C + j] > mx ? x[r * C + j] : mx;
            float s = 0.0f;
            for (int64_t j = 0; j < C; ++j) {
                p[r * C + j] = std::exp(x[r * C + j] - mx);
                s += p[r * C + j];
            }
            const float inv = 1.0f / s;
            for (int64_t j = 0; j < C; ++j) p[r * C + j] *= inv;
        }
        const int64_t* t = static_cast<const int64_t*>(targets.data());
        float total = 0.0f;
        for (int64_t r = 0; r < N; ++r) {
            if (t[r] < 0 || t[r] >= C) throw std::out_of_range("CrossEntropyLoss: target index out of range");
            const float pt = p[r * C + t[r]];
            total += -std::log(pt < 1e-9f ? 1e-9f : pt);
        }
        static_cast<float*>(loss.data())[0] = total / static_cast<float>(N);
        if (logits.requires_grad()) node = std::make_shared<CrossEntropyBackward>(logits, targets, probs);
    }
    if (node) wiring::attach(loss, node, {wiring::accumulator_edge(logits)});
    return loss;
}

Tensor CrossEntropyLoss::forward(Tensor) {
    throw std::logic_error(
        "CrossEntropyLoss::forward(logits) requires targets; call forward(logits, targets) instead.");
}

}  // namespace tensorforge::nn
