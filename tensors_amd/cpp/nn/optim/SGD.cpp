#include "nn/optim/SGD.hpp"

#include "hip/HipBackend.hpp"
#include "hip/Shadow.hpp"
#include "tensor/factory.hpp"

#include <cstring>
#include <stdexcept>

namespace tensorforge::nn::optim {

SGD::SGD(std::vector<Tensor*> parameters, float lr, float momentum)
    : parameters_(std::move(parameters)), lr_(lr), momentum_(momentum) {
    if (lr_ <= 0.0f) throw std::invalid_argument("SGD: lr must be positive");
    if (momentum_ < 0.0f || momentum_ >= 1.0f) throw std::invalid_argument("SGD: momentum must lie in [0, 1)");
    velocity_.resize(parameters_.size());
    if (momentum_ > 0.0f)
        for (size_t i = 0; i < parameters_.size(); ++i)
            velocity_[i] = zeros(parameters_[i]->shape(), Dtype::Float32, parameters_[i]->device());
}

void SGD::step() {
    // GPU parameters are updated together (one launch per 32 parameters of a
    // device, hip::sgd_momentum_multi); nn/optim/SGD.cpp:50-56 updates them one
    // by one, and each ends up the same either way.
    std::vector<hip::SgdItem> batch;
    batch.reserve(parameters_.size());
    for (size_t i = 0; i < parameters_.size(); ++i) {
        Tensor& p = *parameters_[i];
        Tensor g = p.grad();
        if (g.numel() == 0) continue;  // no gradient yet
        if (g.device() != p.device()) g = g.to(p.device());
        if (p.dtype() != Dtype::Float32 || g.dtype() != Dtype::Float32)
            throw std::invalid_argument("SGD: parameters and gradients must be Float32");
        Tensor* v = nullptr;
        if (momentum_ > 0.0f) {
            if (velocity_[i].device() != p.device() || velocity_[i].numel() != p.numel())
                velocity_[i] = zeros(p.shape(), Dtype::Float32, p.device());
            v = &velocity_[i];
        }
        if (p.device().type == DeviceType::CUDA) {
            batch.push_back(hip::SgdItem{&p, g, v, hip::find_shadow(p)});
        } else {
            float* pp = static_cast<float*>(p.data());
            const float* gp = static_cast<const float*>(g.data());
            float* vp = v ? static_cast<float*>(v->data()) : nullptr;
            for (int64_t k = 0; k < p.numel(); ++k) {
                if (vp) {
                    const float vm = vp[k] * momentum_;
                    vp[k] = vm + gp[k];
                    const float s = vp[k] * lr_;
                    pp[k] = pp[k] - s;
                } else {
                    const float s = gp[k] * lr_;
                    pp[k] = pp[k] - s;
                }
            }
            (void)p.bump_version();
        }
    }
    if (!batch.empty()) {
        hip::sgd_momentum_multi(batch, lr_, momentum_);
        for (const hip::SgdItem& it : batch) {
            (void)it.p->bump_version();
            if (it.shadow.numel()) hip::mark_shadow_current(*it.p);
        }
    }
}

void SGD::zero_grad() {
    for (Tensor* p : parameters_) {
        if (!p) continue;
        Tensor g = p->grad();
        if (g.numel() == 0) continue;
        if (g.device().type == DeviceType::CUDA) {
            hip::zero(g);
        } else {
            std::memset(g.data(), 0, static_cast<size_t>(g.numel()) * dtype_size(g.dtype()));
        }
    }
}

}  // namespace tensorforge::nn::optim
