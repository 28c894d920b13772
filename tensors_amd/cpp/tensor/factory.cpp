// Tensor factories.  Float32 GPU tensors are filled by a device kernel;
// other dtypes are built on the host and copied.
#include "tensor/factory.hpp"

#include "hip/HipBackend.hpp"

#include <cstring>
#include <stdexcept>
#include <vector>

namespace tensorforge {

namespace {

void host_fill(void* p, int64_t n, double v, Dtype d) {
    switch (d) {
    case Dtype::Float32: { auto* q = static_cast<float*>(p); for (int64_t i = 0; i < n; ++i) q[i] = static_cast<float>(v); break; }
    case Dtype::Int32: { auto* q = static_cast<int32_t*>(p); for (int64_t i = 0; i < n; ++i) q[i] = static_cast<int32_t>(v); break; }
    case Dtype::Int64: { auto* q = static_cast<int64_t*>(p); for (int64_t i = 0; i < n; ++i) q[i] = static_cast<int64_t>(v); break; }
    case Dtype::Bool: { auto* q = static_cast<uint8_t*>(p); for (int64_t i = 0; i < n; ++i) q[i] = v != 0.0; break; }
    case Dtype::BFloat16: {
        // Proper bf16 encoding of v (the reference stores an int16 cast,
        // tensor/factory.cpp:23-34, which is not a bf16 value).
        float f = static_cast<float>(v);
        uint32_t u;
        std::memcpy(&u, &f, 4);
        u += 0x7fffu + ((u >> 16) & 1u);
        auto h = static_cast<uint16_t>(u >> 16);
        auto* q = static_cast<uint16_t*>(p);
        for (int64_t i = 0; i < n; ++i) q[i] = h;
        break;
    }
    case Dtype::Float16:
        throw std::invalid_argument("full: Float16 fill is not implemented");
    }
}

}  // namespace

Tensor full(Shape shape, double value, Dtype dtype, Device device) {
    Tensor t = Tensor::empty(std::move(shape), dtype, device);
    if (t.numel() == 0) return t;
    if (device.type == DeviceType::CUDA) {
        if (dtype == Dtype::Float32) {
            hip::fill(t, static_cast<float>(value));
            return t;
        }
        if (value == 0.0) {
            hip::zero(t);
            return t;
        }
        Tensor h = Tensor::empty(t.shape(), dtype, Device::cpu());
        host_fill(h.data(), h.numel(), value, dtype);
        return h.to(device);
    }
    host_fill(t.data(), t.numel(), value, dtype);
    return t;
}

Tensor zeros(Shape shape, Dtype dtype, Device device) { return full(std::move(shape), 0.0, dtype, device); }
Tensor ones(Shape shape, Dtype dtype, Device device) { return full(std::move(shape), 1.0, dtype, device); }

Tensor arange(int64_t start, int64_t end, int64_t step, Dtype dtype, Device device) {
    if (step == 0) throw std::invalid_argument("arange: step must be non-zero");
    int64_t n = (end - start + step + (step > 0 ? -1 : 1)) / step;
    if (n < 0) n = 0;
    Tensor h = Tensor::empty(Shape{n}, dtype, Device::cpu());
    for (int64_t i = 0; i < n; ++i) {
        const int64_t v = start + i * step;
        switch (dtype) {
        case Dtype::Float32: static_cast<float*>(h.data())[i] = static_cast<float>(v); break;
        case Dtype::Int32: static_cast<int32_t*>(h.data())[i] = static_cast<int32_t>(v); break;
        case Dtype::Int64: static_cast<int64_t*>(h.data())[i] = v; break;
        default: throw std::invalid_argument("arange: dtype must be Float32, Int32 or Int64");
        }
    }
    return device.type == DeviceType::CPU ? h : h.to(device);
}

Tensor copy(const Tensor& src, Device dst_device) { return src.to(dst_device); }

}  // namespace tensorforge
