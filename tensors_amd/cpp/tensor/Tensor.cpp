// Tensor operations.  CPU tensors: scalar loops with the reference's
// semantics (tensor/Tensor.cpp:97-619).  GPU tensors: libtf_hip kernels via
// hip/HipBackend — never a host fallback.  After computing, each op calls its
// autograd wirer slot (tensor/AutogradWirer.hpp) so autograd can attach the
// backward node.
#include "tensor/Tensor.hpp"

#include "cuda/CudaKernelRegistry.hpp"
#include "hip/HipBackend.hpp"
#include "tensor/AutogradWirer.hpp"
#include "tensor/CPUStorageAllocator.hpp"
#include "tensor/factory.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace tensorforge {

namespace {

// Kernel slots (filled by the HIP backend when libtensorforge loads).
BinaryOpFn g_add_fn = nullptr;
BinaryOpFn g_mul_fn = nullptr;
UnaryOpFn g_relu_fn = nullptr;
UnaryOpFn g_sigmoid_fn = nullptr;
UnaryOpFn g_tanh_fn = nullptr;
LeakyReluFn g_leaky_relu_fn = nullptr;
void* g_current_stream = nullptr;

// Autograd wirer slots.
AutogradWirerFn g_wire_add = nullptr;
AutogradWirerFn g_wire_mul = nullptr;
AutogradWirerFn g_wire_matmul = nullptr;
AutogradUnaryWirerFn g_wire_relu = nullptr;
AutogradUnaryWirerFn g_wire_sigmoid = nullptr;
AutogradUnaryWirerFn g_wire_tanh = nullptr;
AutogradUnaryWirerFn g_wire_leaky_relu = nullptr;
AutogradUnaryWirerFn g_wire_log = nullptr;
AutogradSoftmaxWirerFn g_wire_softmax = nullptr;
AutogradSoftmaxWirerFn g_wire_log_softmax = nullptr;
AutogradLayerNormWirerFn g_wire_layernorm = nullptr;
AutogradReduceWirerFn g_wire_sum = nullptr;
AutogradTransposeWirerFn g_wire_transpose = nullptr;

bool on_gpu(const Tensor& t) { return t.device().type == DeviceType::CUDA; }

void require_f32_cpu(const Tensor& t, const char* what) {
    if (t.dtype() != Dtype::Float32) throw std::invalid_argument(std::string(what) + ": Float32 only on the CPU");
}

int64_t norm_dim(int64_t dim, int64_t ndim, const char* what) {
    if (dim < 0) dim += ndim;
    if (dim < 0 || dim >= ndim) throw std::out_of_range(std::string(what) + ": dim out of range");
    return dim;
}

const float* fp(const Tensor& t) { return static_cast<const float*>(t.data()); }
float* fp(Tensor& t) { return static_cast<float*>(t.data()); }

template <typename Op>
Tensor binary_op(const Tensor& a, const Tensor& b, Op op, const char* name, BinaryOpFn slot,
                 void (*gpu)(const Tensor&, const Tensor&, Tensor&)) {
    if (a.shape() != b.shape()) throw std::invalid_argument(std::string("Tensor::") + name + " shape mismatch");
    if (a.dtype() != b.dtype()) throw std::invalid_argument(std::string("Tensor::") + name + " dtype mismatch");
    if (a.device() != b.device()) throw std::invalid_argument(std::string("Tensor::") + name + " device mismatch");
    Tensor out = Tensor::empty(a.shape(), a.dtype(), a.device());
    if (!on_gpu(a)) {
        require_f32_cpu(a, name);
        const float* pa = fp(a);
        const float* pb = fp(b);
        float* po = fp(out);
        for (int64_t i = 0; i < a.numel(); ++i) po[i] = op(pa[i], pb[i]);
    } else if (slot != nullptr) {
        slot(a.data(), b.data(), out.data(), a.numel(), a.dtype(), g_current_stream);
    } else {
        gpu(a, b, out);
    }
    return out;
}

template <typename Op>
Tensor unary_op(const Tensor& x, Op op, const char* name, UnaryOpFn slot, void (*gpu)(const Tensor&, Tensor&)) {
    Tensor out = Tensor::empty(x.shape(), x.dtype(), x.device());
    if (!on_gpu(x)) {
        require_f32_cpu(x, name);
        const float* px = fp(x);
        float* po = fp(out);
        for (int64_t i = 0; i < x.numel(); ++i) po[i] = op(px[i]);
    } else if (slot != nullptr) {
        slot(x.data(), out.data(), x.numel(), x.dtype(), g_current_stream);
    } else {
        gpu(x, out);
    }
    return out;
}

// Round-to-nearest-even float -> bf16 bits, NaN kept quiet.
uint16_t host_f32_to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}
float host_bf16_to_f32(uint16_t h) {
    uint32_t u = static_cast<uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

}  // namespace

Tensor Tensor::empty(Shape shape, Dtype dtype, Device device) {
    // A 0-d shape has numel() == 0 (reference convention) yet holds one value
    // (e.g. a full reduction): give it room for one element.
    const int64_t slots = shape.ndim() == 0 ? 1 : shape.numel();
    const size_t bytes = static_cast<size_t>(slots) * dtype_size(dtype);
    Storage storage = allocator_dispatch::allocate(bytes, device, dtype);
    Stride stride = Stride::compute_row_major(shape);
    return Tensor(std::move(storage), 0, std::move(shape), std::move(stride));
}

Tensor Tensor::operator+(const Tensor& other) const {
    Tensor out = binary_op(*this, other, [](float a, float b) { return a + b; }, "operator+", g_add_fn, &hip::add);
    if (g_wire_add) g_wire_add(out, *this, other);
    return out;
}

Tensor Tensor::operator*(const Tensor& other) const {
    Tensor out = binary_op(*this, other, [](float a, float b) { return a * b; }, "operator*", g_mul_fn, &hip::mul);
    if (g_wire_mul) g_wire_mul(out, *this, other);
    return out;
}

Tensor Tensor::operator-(const Tensor& other) const {
    // As in the reference, subtraction is not wired into autograd.
    return binary_op(*this, other, [](float a, float b) { return a - b; }, "operator-", nullptr, &hip::sub);
}

Tensor Tensor::to(Device device, Dtype dtype) const {
    const Device src_dev = this->device();
    const Dtype src_dt = this->dtype();
    const size_t n = static_cast<size_t>(numel());
    if (src_dt == dtype) {
        Tensor out = Tensor::empty(shape_, dtype, device);
        const size_t bytes = n * dtype_size(dtype);
        if (bytes == 0) return out;
        if (src_dev.type == DeviceType::CPU && device.type == DeviceType::CPU) {
            std::memcpy(out.data(), data(), bytes);
            return out;
        }
        auto fn = allocator_dispatch::get_cuda_copy();
        if (!fn) throw std::runtime_error("Tensor::to: no GPU copy callback registered");
        using K = allocator_dispatch::CudaCopyKind;
        K kind = src_dev.type == DeviceType::CPU ? K::HostToDevice
                 : device.type == DeviceType::CPU ? K::DeviceToHost
                                                  : K::DeviceToDevice;
        hip::copy_bytes(out.data(), data(), bytes, kind, src_dev.type == DeviceType::CUDA ? src_dev.index : device.index);
        return out;
    }
    const bool f32_bf16 = (src_dt == Dtype::Float32 && dtype == Dtype::BFloat16) ||
                          (src_dt == Dtype::BFloat16 && dtype == Dtype::Float32);
    if (!f32_bf16) throw std::invalid_argument("Tensor::to: only Float32 <-> BFloat16 dtype conversions");
    if (src_dev.type == DeviceType::CUDA) {
        Tensor cast_t = Tensor::empty(shape_, dtype, src_dev);
        hip::cast(*this, cast_t);
        return device == src_dev ? cast_t : cast_t.to(device);
    }
    Tensor cast_t = Tensor::empty(shape_, dtype, Device::cpu());
    if (dtype == Dtype::BFloat16) {
        const float* s = fp(*this);
        auto* d = static_cast<uint16_t*>(cast_t.data());
        for (size_t i = 0; i < n; ++i) d[i] = host_f32_to_bf16(s[i]);
    } else {
        const auto* s = static_cast<const uint16_t*>(data());
        float* d = fp(cast_t);
        for (size_t i = 0; i < n; ++i) d[i] = host_bf16_to_f32(s[i]);
    }
    return device.type == DeviceType::CPU ? cast_t : cast_t.to(device);
}

Tensor Tensor::to(Device device) const { return to(device, dtype()); }
Tensor Tensor::to(Dtype dtype) const { return to(device(), dtype); }

Tensor Tensor::relu() const {
    Tensor out = unary_op(*this, [](float x) { return x > 0.0f ? x : 0.0f; }, "relu", g_relu_fn, &hip::relu);
    if (g_wire_relu) g_wire_relu(out, *this);
    return out;
}

Tensor Tensor::sigmoid() const {
    Tensor out = unary_op(*this, [](float x) { return 1.0f / (1.0f + std::exp(-x)); }, "sigmoid", g_sigmoid_fn,
                          &hip::sigmoid);
    if (g_wire_sigmoid) g_wire_sigmoid(out, *this);
    return out;
}

Tensor Tensor::tanh() const {
    Tensor out = unary_op(*this, [](float x) { return std::tanh(x); }, "tanh", g_tanh_fn, &hip::tanh);
    if (g_wire_tanh) g_wire_tanh(out, *this);
    return out;
}

Tensor Tensor::leaky_relu(float alpha) const {
    Tensor out = Tensor::empty(shape_, dtype(), device());
    if (on_gpu(*this)) {
        if (!g_leaky_relu_fn) throw std::runtime_error("Tensor::leaky_relu: no GPU kernel registered");
        g_leaky_relu_fn(data(), out.data(), numel(), dtype(), alpha, g_current_stream);
    } else {
        require_f32_cpu(*this, "leaky_relu");
        const float* x = fp(*this);
        float* y = fp(out);
        for (int64_t i = 0; i < numel(); ++i) y[i] = x[i] > 0.0f ? x[i] : alpha * x[i];
    }
    if (g_wire_leaky_relu) g_wire_leaky_relu(out, *this);
    return out;
}

Tensor Tensor::matmul(const Tensor& other) const {
    if (shape_.ndim() != 2 || other.shape_.ndim() != 2)
        throw std::invalid_argument("Tensor::matmul: both operands must be 2D");
    if (shape_[1] != other.shape_[0]) throw std::invalid_argument("Tensor::matmul: shape mismatch (a.cols != b.rows)");
    if (device() != other.device()) throw std::invalid_argument("Tensor::matmul: operands on different devices");
    if (dtype() != other.dtype()) throw std::invalid_argument("Tensor::matmul: dtype mismatch");
    const int64_t M = shape_[0], K = shape_[1], N = other.shape_[1];
    Tensor out = Tensor::empty(Shape{M, N}, dtype(), device());
    if (on_gpu(*this)) {
        hip::gemm(*this, false, other, false, out);
    } else {
        require_f32_cpu(*this, "matmul");
        const float* a = fp(*this);
        const float* b = fp(other);
        float* c = fp(out);
        for (int64_t i = 0; i < M; ++i)
            for (int64_t j = 0; j < N; ++j) {
                float acc = 0.0f;
                for (int64_t k = 0; k < K; ++k) acc += a[i * K + k] * b[k * N + j];
                c[i * N + j] = acc;
            }
    }
    if (g_wire_matmul) g_wire_matmul(out, *this, other);
    return out;
}

namespace {

// Shared softmax / log_softmax over the last dim (the only one supported, as
// in the reference).
Tensor softmax_like(const Tensor& x, int64_t dim, bool log_variant) {
    const char* name = log_variant ? "Tensor::log_softmax" : "Tensor::softmax";
    const int64_t nd = static_cast<int64_t>(x.shape().ndim());
    dim = norm_dim(dim, nd, name);
    if (dim != nd - 1) throw std::invalid_argument(std::string(name) + ": only last-dim in v1");
    Tensor out = Tensor::empty(x.shape(), x.dtype(), x.device());
    if (on_gpu(x)) {
        if (log_variant) hip::log_softmax(x, out);
        else hip::softmax(x, out);
        return out;
    }
    require_f32_cpu(x, name);
    const int64_t inner = x.shape()[nd - 1];
    const int64_t outer = inner ? x.numel() / inner : 0;
    const float* px = fp(x);
    float* py = fp(out);
    for (int64_t r = 0; r < outer; ++r) {
        const float* row = px + r * inner;
        float* yr = py + r * inner;
        float mx = row[0];
        for (int64_t j = 1; j < inner; ++j) mx = row[j] > mx ? row[j] : mx;
        float s = 0.0f;
        if (log_variant) {
            for (int64_t j = 0; j < inner; ++j) s += std::exp(row[j] - mx);
            const float lz = std::log(s) + mx;
            for (int64_t j = 0; j < inner; ++j) yr[j] = row[j] - lz;
        } else {
            for (int64_t j = 0; j < inner; ++j) {
                yr[j] = std::exp(row[j] - mx);
                s += yr[j];
            }
            const float inv = 1.0f / s;
            for (int64_t j = 0; j < inner; ++j) yr[j] *= inv;
        }
    }
    return out;
}

}  // namespace

Tensor Tensor::softmax(int64_t dim) const {
    Tensor out = softmax_like(*this, dim, false);
    if (g_wire_softmax) g_wire_softmax(out, *this, dim);
    return out;
}

Tensor Tensor::log_softmax(int64_t dim) const {
    Tensor out = softmax_like(*this, dim, true);
    if (g_wire_log_softmax) g_wire_log_softmax(out, *this, dim);
    return out;
}

Tensor Tensor::layer_norm(const Tensor& gamma, const Tensor& beta, float eps) const {
    if (shape_.ndim() != 2) throw std::invalid_argument("Tensor::layer_norm: only 2D rows in v1");
    const int64_t rows = shape_[0], cols = shape_[1];
    if (gamma.numel() != cols || beta.numel() != cols)
        throw std::invalid_argument("Tensor::layer_norm: gamma/beta must be [cols]");
    Tensor out = Tensor::empty(shape_, dtype(), device());
    if (on_gpu(*this)) {
        // Row statistics are recomputed by the wirer for the backward node
        // (as the reference wirer does); here they are scratch.
        Tensor mean = Tensor::empty(Shape{rows}, Dtype::Float32, device());
        Tensor rstd = Tensor::empty(Shape{rows}, Dtype::Float32, device());
        hip::layernorm_forward(*this, gamma, beta, out, mean, rstd, eps);
    } else {
        require_f32_cpu(*this, "layer_norm");
        const float* x = fp(*this);
        const float* g = fp(gamma);
        const float* b = fp(beta);
        float* y = fp(out);
        for (int64_t r = 0; r < rows; ++r) {
            const float* row = x + r * cols;
            float s = 0.0f;
            for (int64_t j = 0; j < cols; ++j) s += row[j];
            const float m = s / static_cast<float>(cols);
            float vs = 0.0f;
            for (int64_t j = 0; j < cols; ++j) {
                const float d = row[j] - m;
                vs += d * d;
            }
            const float rs = 1.0f / std::sqrt(vs / static_cast<float>(cols) + eps);
            for (int64_t j = 0; j < cols; ++j) y[r * cols + j] = (row[j] - m) * rs * g[j] + b[j];
        }
    }
    if (g_wire_layernorm) g_wire_layernorm(out, *this, gamma, beta, eps);
    return out;
}

Tensor Tensor::log() const {
    if (on_gpu(*this)) throw std::runtime_error("Tensor::log: GPU kernel not implemented (not on the training path)");
    require_f32_cpu(*this, "log");
    Tensor out = Tensor::empty(shape_, dtype(), device());
    const float* x = fp(*this);
    float* y = fp(out);
    for (int64_t i = 0; i < numel(); ++i) y[i] = std::log(x[i]);
    if (g_wire_log) g_wire_log(out, *this);
    return out;
}

Tensor Tensor::sum(int64_t dim, bool keepdim) const {
    const int64_t nd = static_cast<int64_t>(shape_.ndim());
    dim = norm_dim(dim, nd, "Tensor::sum");
    std::vector<int64_t> od;
    int64_t outer = 1, inner = 1;
    for (int64_t i = 0; i < nd; ++i) {
        if (i < dim) outer *= shape_[i];
        if (i > dim) inner *= shape_[i];
        if (i != dim) od.push_back(shape_[i]);
        else if (keepdim) od.push_back(1);
    }
    const int64_t reduce = shape_[dim];
    Tensor out = Tensor::empty(Shape(od), dtype(), device());
    if (on_gpu(*this)) {
        hip::sum_dim(*this, out, outer, reduce, inner);
    } else {
        require_f32_cpu(*this, "sum");
        const float* x = fp(*this);
        float* y = fp(out);
        for (int64_t o = 0; o < outer; ++o)
            for (int64_t i = 0; i < inner; ++i) {
                float s = 0.0f;
                for (int64_t r = 0; r < reduce; ++r) s += x[(o * reduce + r) * inner + i];
                y[o * inner + i] = s;
            }
    }
    if (g_wire_sum) g_wire_sum(out, *this, dim, keepdim);
    return out;
}

Tensor Tensor::mean() const {
    // Scalar mean over all elements (not wired into autograd, as in the reference).
    const int64_t n = numel();
    if (on_gpu(*this)) {
        Tensor flat(storage_, storage_offset_, Shape{n}, Stride{1});
        Tensor s = Tensor::empty(Shape{1}, Dtype::Float32, device());
        hip::sum_dim(flat, s, 1, n, 1);
        Tensor scale = full(Shape{1}, 1.0 / static_cast<double>(n), Dtype::Float32, device());
        Tensor out = Tensor::empty(Shape{1}, Dtype::Float32, device());
        // mean = sum * (1/n): the reference divides (s / n); within one ulp.
        hip::mul(s, scale, out);
        return out;
    }
    require_f32_cpu(*this, "mean");
    const float* x = fp(*this);
    float s = 0.0f;
    for (int64_t i = 0; i < n; ++i) s += x[i];
    Tensor out = Tensor::empty(Shape{1}, Dtype::Float32, device());
    fp(out)[0] = s / static_cast<float>(n);
    return out;
}

Tensor Tensor::transpose(int64_t dim0, int64_t dim1) const {
    const int64_t nd = static_cast<int64_t>(shape_.ndim());
    dim0 = norm_dim(dim0, nd, "Tensor::transpose");
    dim1 = norm_dim(dim1, nd, "Tensor::transpose");
    Shape ns = shape_;
    std::swap(ns.data()[dim0], ns.data()[dim1]);
    Tensor out = Tensor::empty(ns, dtype(), device());
    if (on_gpu(*this)) {
        const int64_t lo = std::min(dim0, dim1), hi = std::max(dim0, dim1);
        if (dim0 == dim1) {
            hip::cast(*this, out);  // same dtype: device copy
        } else if (hi == nd - 1 && lo == nd - 2) {
            const int64_t rows = shape_[lo], cols = shape_[hi];
            hip::transpose2d(*this, out, rows * cols ? numel() / (rows * cols) : 0, rows, cols);
        } else {
            throw std::invalid_argument("Tensor::transpose: on the GPU only the last two dims can be swapped");
        }
    } else {
        const size_t es = dtype_size(dtype());
        Stride is = Stride::compute_row_major(shape_);
        std::vector<int64_t> coord(nd);
        const char* src = static_cast<const char*>(data());
        char* dst = static_cast<char*>(out.data());
        for (int64_t flat = 0; flat < out.numel(); ++flat) {
            int64_t rem = flat;
            for (int64_t d = nd - 1; d >= 0; --d) {
                coord[d] = rem % ns[d];
                rem /= ns[d];
            }
            std::swap(coord[dim0], coord[dim1]);
            int64_t off = 0;
            for (int64_t d = 0; d < nd; ++d) off += coord[d] * is[d];
            std::memcpy(dst + flat * es, src + off * es, es);
        }
    }
    if (g_wire_transpose) g_wire_transpose(out, *this, dim0, dim1);
    return out;
}

void register_cuda_add(BinaryOpFn fn) { g_add_fn = fn; }
void register_cuda_mul(BinaryOpFn fn) { g_mul_fn = fn; }
void register_cuda_relu(UnaryOpFn fn) { g_relu_fn = fn; }
void register_cuda_sigmoid(UnaryOpFn fn) { g_sigmoid_fn = fn; }
void register_cuda_tanh(UnaryOpFn fn) { g_tanh_fn = fn; }
void register_cuda_leaky_relu(LeakyReluFn fn) { g_leaky_relu_fn = fn; }
void register_current_stream(void* stream) {
    g_current_stream = stream;
    hip::set_stream(stream, 0);
}

void register_add_wirer(AutogradWirerFn fn) { g_wire_add = fn; }
void register_mul_wirer(AutogradWirerFn fn) { g_wire_mul = fn; }
void register_matmul_wirer(AutogradWirerFn fn) { g_wire_matmul = fn; }
void register_relu_wirer(AutogradUnaryWirerFn fn) { g_wire_relu = fn; }
void register_sigmoid_wirer(AutogradUnaryWirerFn fn) { g_wire_sigmoid = fn; }
void register_tanh_wirer(AutogradUnaryWirerFn fn) { g_wire_tanh = fn; }
void register_leaky_relu_wirer(AutogradUnaryWirerFn fn) { g_wire_leaky_relu = fn; }
void register_log_wirer(AutogradUnaryWirerFn fn) { g_wire_log = fn; }
void register_softmax_wirer(AutogradSoftmaxWirerFn fn) { g_wire_softmax = fn; }
void register_log_softmax_wirer(AutogradSoftmaxWirerFn fn) { g_wire_log_softmax = fn; }
void register_layernorm_wirer(AutogradLayerNormWirerFn fn) { g_wire_layernorm = fn; }
void register_sum_wirer(AutogradReduceWirerFn fn) { g_wire_sum = fn; }
void register_transpose_wirer(AutogradTransposeWirerFn fn) { g_wire_transpose = fn; }

}  // namespace tensorforge
