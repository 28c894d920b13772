// Fan-in accumulation (reference autograd/InputBuffer.cpp:11-55): a second
// gradient for the same slot is added elementwise into a new tensor — on the
// GPU by the add kernel.
#include "autograd/InputBuffer.hpp"

#include "hip/HipBackend.hpp"

#include <stdexcept>

namespace tensorforge {

namespace {

Tensor add_grads(const Tensor& a, const Tensor& b) {
    if (a.shape() != b.shape()) throw std::runtime_error("InputBuffer: shape mismatch during gradient accumulation");
    if (a.dtype() != b.dtype() || a.device() != b.device())
        throw std::runtime_error("InputBuffer: dtype/device mismatch during gradient accumulation");
    Tensor r = Tensor::empty(a.shape(), a.dtype(), a.device());
    if (a.device().type == DeviceType::CUDA) {
        hip::add(a, b, r);
        return r;
    }
    if (a.dtype() != Dtype::Float32) throw std::runtime_error("InputBuffer: CPU accumulation supports Float32 only");
    const float* pa = static_cast<const float*>(a.data());
    const float* pb = static_cast<const float*>(b.data());
    float* pr = static_cast<float*>(r.data());
    for (int64_t i = 0; i < a.numel(); ++i) pr[i] = pa[i] + pb[i];
    return r;
}

}  // namespace

InputBuffer::InputBuffer(size_t num_outputs) : buffer_(num_outputs) {}

void InputBuffer::add(size_t pos, Tensor grad) {
    if (pos >= buffer_.size()) buffer_.resize(pos + 1);
    if (!buffer_[pos]) buffer_[pos] = std::move(grad);
    else buffer_[pos] = add_grads(*buffer_[pos], grad);
}

std::vector<Tensor> InputBuffer::take() {
    std::vector<Tensor> out;
    out.reserve(buffer_.size());
    for (auto& g : buffer_) out.push_back(g ? std::move(*g) : Tensor());
    buffer_.clear();
    return out;
}

}  // namespace tensorforge
