// C entry points that drive the C++ API end to end (include/tfa_harness.h):
// training loops shaped like the reference's examples and self-tests that
// restate the reference's own unit tests (each cites the test it restates).
// Every self-test runs on CPU tensors or on GPU 0.
#include "tfa_harness.h"

#include "data/CifarLoader.hpp"
#include "data/MnistLoader.hpp"
#include "autograd/AccumulateGrad.hpp"
#include "autograd/AutogradMeta.hpp"
#include "autograd/Engine.hpp"
#include "autograd/ops/AddBackward.hpp"
#include "hip/HipBackend.hpp"
#include "nn/Activations.hpp"
#include "nn/Conv2d.hpp"
#include "nn/Conv2dModule.hpp"
#include "nn/CrossEntropyLoss.hpp"
#include "nn/Linear.hpp"
#include "nn/optim/SGD.hpp"
#include "tensor/AutogradWirer.hpp"
#include "tensor/Compat.hpp"
#include "tensor/factory.hpp"
#include "tensor/shape_ops.hpp"

#include <chrono>
#include <unistd.h>
#include <fstream>
#include <filesystem>
#include <cmath>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

using namespace tensorforge;

namespace {

thread_local std::string g_err;

template <typename F>
int guarded(F&& f) {
    try {
        init_tensor_autograd();
        f();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 1;
    } catch (...) {
        g_err = "unknown exception";
        return 1;
    }
}

// Restores the reference-compat switches when a harness call returns.
struct CompatScope {
    bool bias, ln;
    explicit CompatScope(bool on) : bias(compat::linear_drops_bias()), ln(compat::layernorm_stub_backward()) {
        compat::set_reference_compat(on);
    }
    ~CompatScope() {
        compat::set_linear_drops_bias(bias);
        compat::set_layernorm_stub_backward(ln);
    }
};

Device dev_of(int on_gpu) { return on_gpu ? Device::cuda(0) : Device::cpu(); }

Tensor host_f32(const float* src, Shape s) {
    Tensor t = Tensor::empty(std::move(s), Dtype::Float32, Device::cpu());
    if (src) std::memcpy(t.data(), src, sizeof(float) * static_cast<size_t>(t.numel()));
    return t;
}

Tensor host_i64(const int64_t* src, Shape s) {
    Tensor t = Tensor::empty(std::move(s), Dtype::Int64, Device::cpu());
    std::memcpy(t.data(), src, sizeof(int64_t) * static_cast<size_t>(t.numel()));
    return t;
}

std::vector<float> to_host(const Tensor& t) {
    Tensor h = t.device().type == DeviceType::CPU ? t : t.to(Device::cpu());
    if (h.dtype() != Dtype::Float32) h = h.to(Dtype::Float32);
    const float* p = static_cast<const float*>(h.data());
    return std::vector<float>(p, p + h.numel());
}

void sync_if_gpu(int on_gpu) {
    if (on_gpu) hip::synchronize(0);
}

// ---------------------------------------------------------------------------
// self-tests
// ---------------------------------------------------------------------------
#define TFA_CHECK(cond)                                                                          \
    do {                                                                                         \
        if (!(cond)) throw std::runtime_error(std::string("check failed: ") + #cond);            \
    } while (0)

void check_near(float got, float want, float tol, const std::string& what) {
    if (!(std::fabs(got - want) <= tol * std::max(1.0f, std::fabs(want)))) {
        std::ostringstream os;
        os << what << ": got " << got << " want " << want;
        throw std::runtime_error(os.str());
    }
}

void check_all(const Tensor& t, float want, const std::string& what, float tol = 1e-6f) {
    auto v = to_host(t);
    TFA_CHECK(!v.empty());
    for (size_t i = 0; i < v.size(); ++i) check_near(v[i], want, tol, what + "[" + std::to_string(i) + "]");
}

void check_vec(const Tensor& t, const std::vector<float>& want, const std::string& what, float tol = 1e-5f) {
    auto v = to_host(t);
    if (v.size() != want.size()) throw std::runtime_error(what + ": size mismatch");
    for (size_t i = 0; i < v.size(); ++i) check_near(v[i], want[i], tol, what + "[" + std::to_string(i) + "]");
}

Tensor filled(Shape s, float v, Device d) { return full(std::move(s), v, Dtype::Float32, d); }

Tensor from_vals(const std::vector<float>& v, Shape s, Device d) { return host_f32(v.data(), std::move(s)).to(d); }

// autograd/engine_test.cpp:65-100 — a.grad == 2 through fan-in of a hand-built graph.
void t_engine_fan_in(Device d) {
    Tensor a = filled({2, 3}, 1.0f, d), b = filled({2, 3}, 1.0f, d), c = filled({2, 3}, 1.0f, d);
    a.requires_grad(true);
    b.requires_grad(true);
    c.requires_grad(true);
    auto e = std::make_shared<AddBackward>();
    e->next_edges_ = {Edge(a.autograd_meta()->grad_accumulator_, 0), Edge(b.autograd_meta()->grad_accumulator_, 0)};
    auto f = std::make_shared<AddBackward>();
    f->next_edges_ = {Edge(a.autograd_meta()->grad_accumulator_, 0), Edge(c.autograd_meta()->grad_accumulator_, 0)};
    auto loss = std::make_shared<AddBackward>();
    loss->next_edges_ = {Edge(e, 0), Edge(f, 0)};
    Engine().execute(loss, filled({2, 3}, 1.0f, d), false);
    check_all(a.grad(), 2.0f, "a.grad");
    check_all(b.grad(), 1.0f, "b.grad");
    check_all(c.grad(), 1.0f, "c.grad");
}

// autograd/engine_test.cpp:126-152 — a deep chain of adds reaches the leaf.
void t_engine_deep_chain(Device d) {
    Tensor a = filled({4}, 1.0f, d);
    a.requires_grad(true);
    Tensor z = filled({4}, 0.0f, d);
    Tensor h = a;
    for (int i = 0; i < 64; ++i) h = h + z;
    h.backward();
    check_all(a.grad(), 1.0f, "a.grad");
}

// tests/autograd/chain_autograd_test.cpp:25-54 — d = (a+b)*a, e = d.sum(0).
void t_chain_add_mul_sum(Device d) {
    Tensor a = filled({2, 3}, 2.0f, d), b = filled({2, 3}, 3.0f, d);
    a.requires_grad(true);
    b.requires_grad(true);
    Tensor c = a + b;
    Tensor dd = c * a;
    Tensor e = dd.sum(0);
    TFA_CHECK(e.requires_grad() && e.autograd_meta()->grad_fn_ != nullptr);
    e.backward();
    check_all(a.grad(), 7.0f, "a.grad");
    check_all(b.grad(), 2.0f, "b.grad");
}

// tests/autograd/chain_autograd_test.cpp:56-68 — transpose reaches the leaf.
void t_transpose_grad(Device d) {
    Tensor W = filled({3, 4}, 0.5f, d);
    W.requires_grad(true);
    Tensor Wt = W.transpose(0, 1);
    TFA_CHECK(Wt.shape() == (Shape{4, 3}));
    Tensor s = Wt.sum(0).sum(0);
    s.backward();
    check_all(W.grad(), 1.0f, "W.grad");
    TFA_CHECK(W.grad().shape() == (Shape{3, 4}));
}

// autograd/ops/autograd_all_ops_test.cpp:281-328 — matmul arange known answers.
void t_matmul_known_answer(Device d) {
    Tensor a = from_vals({0, 1, 2, 3, 4, 5}, {2, 3}, d);
    Tensor b = from_vals({0, 1, 2, 3, 4, 5}, {3, 2}, d);
    a.requires_grad(true);
    b.requires_grad(true);
    Tensor c = a.matmul(b);
    check_vec(c, {10, 13, 28, 40}, "C");
    c.backward();
    check_vec(a.grad(), {1, 5, 9, 1, 5, 9}, "dA");
    check_vec(b.grad(), {3, 3, 5, 5, 7, 7}, "dB");
}

// autograd/ops/autograd_all_ops_test.cpp:253-268 — ones @ ones, grads 2.
void t_matmul_ones(Device d) {
    Tensor a = filled({2, 2}, 1.0f, d), b = filled({2, 2}, 1.0f, d);
    a.requires_grad(true);
    b.requires_grad(true);
    a.matmul(b).backward();
    check_all(a.grad(), 2.0f, "dA");
    check_all(b.grad(), 2.0f, "dB");
}

// autograd/ops/autograd_all_ops_test.cpp:73-94 — relu mask, x == 0 -> 0.
void t_relu_mask(Device d) {
    Tensor x = from_vals({-2, -0.5f, 0, 0.5f, 2, 3}, {6}, d);
    x.requires_grad(true);
    Tensor y = x.relu();
    check_vec(y, {0, 0, 0, 0.5f, 2, 3}, "relu");
    y.backward();
    check_vec(x.grad(), {0, 0, 0, 1, 1, 1}, "relu grad");
}

// Tensor::leaky_relu through the registry's LeakyReluFn slot on the GPU
// (tensor/Tensor.cpp:303-327): x > 0 ? x : alpha * x.
void t_leaky_relu(Device d) {
    Tensor x = from_vals({-2, -0.5f, 0, 0.5f, 3}, {5}, d);
    check_vec(x.leaky_relu(0.1f), {0.1f * -2.0f, 0.1f * -0.5f, 0, 0.5f, 3}, "leaky_relu", 0.0f);
}

// autograd/ops/autograd_all_ops_test.cpp:108-121 — uniform softmax, grad 0.
void t_softmax_uniform(Device d) {
    Tensor x = filled({2, 4}, 0.3f, d);
    x.requires_grad(true);
    Tensor y = x.softmax(-1);
    check_all(y, 0.25f, "softmax");
    y.backward();
    check_all(x.grad(), 0.0f, "softmax grad", 1e-6f);
}

// autograd/ops/autograd_all_ops_test.cpp:164-177 — log_softmax closed form.
void t_log_softmax_closed_form(Device d) {
    Tensor x = from_vals({1, 2, 3}, {1, 3}, d);
    Tensor y = x.log_softmax(-1);
    const double lz = std::log(std::exp(1.0) + std::exp(2.0) + std::exp(3.0));
    check_vec(y, {float(1 - lz), float(2 - lz), float(3 - lz)}, "log_softmax");
}

// autograd/ops/autograd_add_mul_test.cpp:122-143 — c = a * b arange grads.
void t_mul_arange(Device d) {
    Tensor a = from_vals({0, 1, 2, 3}, {4}, d), b = from_vals({4, 5, 6, 7}, {4}, d);
    a.requires_grad(true);
    b.requires_grad(true);
    (a * b).backward();
    check_vec(a.grad(), {4, 5, 6, 7}, "da");
    check_vec(b.grad(), {0, 1, 2, 3}, "db");
}

// autograd/ops/autograd_add_mul_test.cpp:145-162 — mutating a saved input throws.
void t_saved_tensor_version(Device d) {
    Tensor a = filled({3}, 2.0f, d), b = filled({3}, 3.0f, d);
    a.requires_grad(true);
    b.requires_grad(true);
    Tensor c = a * b;
    (void)b.bump_version();
    bool threw = false;
    try {
        c.backward();
    } catch (const std::runtime_error&) {
        threw = true;
    }
    TFA_CHECK(threw);
}

// nn/cross_entropy_test.cpp:10-49 — CE known answers 0.4076 and 1.0986.
void t_cross_entropy_known(Device d) {
    nn::CrossEntropyLoss ce;
    Tensor logits = from_vals({1, 2, 3}, {1, 3}, d);
    int64_t t2 = 2;
    Tensor tg = host_i64(&t2, {1}).to(d);
    check_near(to_host(ce.forward(logits, tg))[0], 0.4076f, 1e-3f, "single");
    Tensor l2 = filled({2, 3}, 1.0f, d);
    int64_t tt[2] = {0, 2};
    check_near(to_host(ce.forward(l2, host_i64(tt, {2}).to(d)))[0], 1.0986f, 1e-3f, "batch");
}

// CE gradient = (softmax - onehot) / N (no reference test covers it).
void t_cross_entropy_grad(Device d) {
    nn::CrossEntropyLoss ce;
    Tensor logits = from_vals({1, 2, 3, 0, 0, 0}, {2, 3}, d);
    logits.requires_grad(true);
    int64_t tt[2] = {2, 0};
    ce.forward(logits, host_i64(tt, {2}).to(d)).backward();
    const double z = std::exp(1.0) + std::exp(2.0) + std::exp(3.0);
    std::vector<float> want = {float(std::exp(1.0) / z / 2), float(std::exp(2.0) / z / 2),
                               float((std::exp(3.0) / z - 1) / 2), float((1.0 / 3 - 1) / 2), float(1.0 / 6),
                               float(1.0 / 6)};
    check_vec(logits.grad(), want, "dlogits", 1e-5f);
}

// nn::CrossEntropyLoss under a non-unit upstream gradient: (loss * 0.3)
// and the sum of two losses (different targets) on the same logits, fp32
// and (on the GPU) BFloat16 logits from a Linear.  logits.grad against
// g * (softmax - onehot) / N in double (from the logits as stored), within
// fp32 rounding: for bf16 logits this shows the scaled gradient is formed in
// fp32 from the logits, not from dlogits already rounded to bf16.  W.grad
// against double dlogits^T x, at the compute dtype's tolerance.  With a unit
// seed the bf16 dlogits must be the double value rounded once (within half a
// bf16 step).
void t_cross_entropy_scaled_upstream(Device d) {
    const int R = 37, I = 24, C = 13;
    std::vector<float> xv(R * I), wv(C * I);
    for (int i = 0; i < R * I; ++i) xv[i] = std::sin(0.31f * i + 0.2f);
    for (int i = 0; i < C * I; ++i) wv[i] = 0.4f * std::cos(0.17f * i);
    std::vector<int64_t> t1(R), t2(R);
    for (int r = 0; r < R; ++r) {
        t1[r] = (r * 7) % C;
        t2[r] = (r * 5 + 3) % C;
    }
    const bool gpu = d.type == DeviceType::CUDA;
    for (int bf16 = 0; bf16 <= (gpu ? 1 : 0); ++bf16) {
        for (int mode = 0; mode < 3; ++mode) {   // 0: loss * 0.3, 1: loss1 + loss2, 2: loss (unit seed)
            nn::Linear fc(I, C);
            fc.to(d);
            if (bf16) fc.set_compute_dtype(Dtype::BFloat16);
            for (auto& np : fc.named_parameters()) {
                np.second->data_ = np.first == "weight" ? from_vals(wv, {C, I}, d) : filled({C}, 0.0f, d);
                np.second->data_.requires_grad(true);
            }
            Tensor x = from_vals(xv, {R, I}, d);
            Tensor logits = fc.forward(x);
            nn::CrossEntropyLoss ce;
            Tensor l1 = ce.forward(logits, host_i64(t1.data(), {R}).to(d));
            const float g = 0.3f;
            if (mode == 0) (l1 * filled({1}, g, d)).backward();
            else if (mode == 1) (l1 + ce.forward(logits, host_i64(t2.data(), {R}).to(d))).backward();
            else l1.backward();
            // Truth in double from the stored logits and inputs.
            const std::vector<float> lg = to_host(logits);
            const std::vector<float> xs = bf16 ? to_host(x.to(Dtype::BFloat16)) : xv;
            std::vector<double> dl(R * C, 0.0);
            for (int r = 0; r < R; ++r) {
                double mx = lg[r * C];
                for (int j = 1; j < C; ++j) mx = std::max(mx, (double)lg[r * C + j]);
                double z = 0.0;
                for (int j = 0; j < C; ++j) z += std::exp(lg[r * C + j] - mx);
                for (int j = 0; j < C; ++j) {
                    const double p = std::exp(lg[r * C + j] - mx) / z;
                    if (mode == 0) dl[r * C + j] = g * (p - (j == t1[r])) / R;
                    else if (mode == 1) dl[r * C + j] = (2 * p - (j == t1[r]) - (j == t2[r])) / R;
                    else dl[r * C + j] = (p - (j == t1[r])) / R;
                }
            }
            const std::string tag = std::string(bf16 ? " (bf16 logits" : " (fp32 logits") +
                                    (mode == 0 ? ", loss * 0.3)" : mode == 1 ? ", loss1 + loss2)" : ", unit seed)");
            const std::vector<float> gl = to_host(logits.grad());
            TFA_CHECK(gl.size() == dl.size());
            double rms = 0.0;
            for (double v : dl) rms += v * v;
            rms = std::sqrt(rms / dl.size());
            for (size_t i = 0; i < dl.size(); ++i) {
                double bound;
                if (bf16 && mode == 2) {
                    // bf16 dlogits: half a bf16 step of the value (2^(e-8)
                    // for 2^e <= |v| < 2^(e+1)) plus fp32 noise.
                    const double a = std::fabs(dl[i]);
                    bound = (a > 0 ? std::ldexp(1.0, (int)std::floor(std::log2(a)) - 8) : 0.0) + 4e-6 * a + 1e-9;
                } else {
                    bound = 1e-5 * (std::fabs(dl[i]) + rms);
                }
                if (!(std::fabs(gl[i] - dl[i]) <= bound)) {
                    std::ostringstream os;
                    os << "dlogits" << tag << "[" << i << "]: got " << gl[i] << " want " << dl[i];
                    throw std::runtime_error(os.str());
                }
            }
            // W.grad = dlogits^T x (as the backward's GEMM sees dlogits: in
            // the compute dtype).
            std::vector<float> gw;
            for (auto& np : fc.named_parameters())
                if (np.first == "weight") gw = to_host(np.second->data_.grad());
            TFA_CHECK(gw.size() == (size_t)C * I);
            std::vector<double> tw(C * I, 0.0);
            double wrms = 0.0;
            for (int o = 0; o < C; ++o)
                for (int k = 0; k < I; ++k) {
                    double acc = 0.0;
                    for (int r = 0; r < R; ++r) acc += dl[r * C + o] * xs[r * I + k];
                    tw[o * I + k] = acc;
                    wrms += acc * acc;
                }
            wrms = std::sqrt(wrms / tw.size());
            const double rt = bf16 ? 2e-2 : 1e-4;
            for (size_t i = 0; i < tw.size(); ++i)
                if (!(std::fabs(gw[i] - tw[i]) <= rt * (std::fabs(tw[i]) + wrms))) {
                    std::ostringstream os;
                    os << "dW" << tag << "[" << i << "]: got " << gw[i] << " want " << tw[i];
                    throw std::runtime_error(os.str());
                }
        }
    }
}

// Sigmoid / tanh backward (wired here; the reference leaves them unwired).
void t_sigmoid_tanh_grad(Device d) {
    Tensor x = from_vals({-1.5f, 0.0f, 0.7f}, {3}, d);
    x.requires_grad(true);
    x.sigmoid().backward();
    std::vector<float> ws, wt;
    for (float v : {-1.5f, 0.0f, 0.7f}) {
        double s = 1.0 / (1.0 + std::exp(-double(v)));
        ws.push_back(float(s * (1 - s)));
        double t = std::tanh(double(v));
        wt.push_back(float(1 - t * t));
    }
    check_vec(x.grad(), ws, "sigmoid'");
    Tensor x2 = from_vals({-1.5f, 0.0f, 0.7f}, {3}, d);
    x2.requires_grad(true);
    x2.tanh().backward();
    check_vec(x2.grad(), wt, "tanh'");
}

// LayerNorm: true gradient of sum(y * w) vs double-precision finite differences;
// stub mode reproduces dx = dy * gamma.
void t_layernorm_grad(Device d) {
    const int R = 3, C = 5;
    std::vector<float> xv = {0.3f, -1.2f, 0.8f, 2.0f, -0.4f, 1.1f, 0.0f, -0.7f, 0.5f, 0.9f,
                             -2.0f, 0.25f, 1.5f, -0.1f, 0.6f};
    std::vector<float> gv = {1.0f, 0.5f, 2.0f, -1.0f, 1.5f};
    std::vector<float> bv = {0.1f, 0.0f, -0.2f, 0.3f, 0.0f};
    auto loss_at = [&](const std::vector<float>& xs) {
        double tot = 0.0;
        for (int r = 0; r < R; ++r) {
            double m = 0, v = 0;
            for (int j = 0; j < C; ++j) m += xs[r * C + j];
            m /= C;
            for (int j = 0; j < C; ++j) v += (xs[r * C + j] - m) * (xs[r * C + j] - m);
            v /= C;
            const double rs = 1.0 / std::sqrt(v + 1e-5);
            for (int j = 0; j < C; ++j) tot += ((xs[r * C + j] - m) * rs * gv[j] + bv[j]) * (j + 1);
        }
        return tot;
    };
    Tensor x = from_vals(xv, {R, C}, d), g = from_vals(gv, {C}, d), b = from_vals(bv, {C}, d);
    x.requires_grad(true);
    g.requires_grad(true);
    b.requires_grad(true);
    Tensor y = x.layer_norm(g, b, 1e-5f);
    std::vector<float> wv;
    for (int r = 0; r < R; ++r)
        for (int j = 0; j < C; ++j) wv.push_back(float(j + 1));
    Tensor w = from_vals(wv, {R, C}, d);
    Engine().execute(y.autograd_meta()->grad_fn_, w, false);
    std::vector<float> want;
    for (int i = 0; i < R * C; ++i) {
        auto xp = xv, xm = xv;
        const double h = 1e-3;
        xp[i] += float(h);
        xm[i] -= float(h);
        want.push_back(float((loss_at(xp) - loss_at(xm)) / (2 * h)));
    }
    check_vec(x.grad(), want, "ln dx", 5e-3f);
    std::vector<float> wb(C, 0.0f);
    for (int j = 0; j < C; ++j) wb[j] = float(R * (j + 1));
    check_vec(b.grad(), wb, "ln dbeta", 1e-5f);

    compat::set_layernorm_stub_backward(true);
    Tensor x2 = from_vals(xv, {R, C}, d);
    x2.requires_grad(true);
    Tensor y2 = x2.layer_norm(g, b, 1e-5f);
    Engine().execute(y2.autograd_meta()->grad_fn_, w, false);
    compat::set_layernorm_stub_backward(false);
    std::vector<float> stub;
    for (int r = 0; r < R; ++r)
        for (int j = 0; j < C; ++j) stub.push_back(float(j + 1) * gv[j]);
    check_vec(x2.grad(), stub, "stub dx", 0.0f);
}

// nn/conv2d_backward_test.cpp:110-160 — 1x1 kernel golden gradients
// (weight 2, grad_out 0.1..0.4: dX = 0.2..0.8, dW = 3.0), through
// Conv2dModule's autograd node on either device.
void t_conv_1x1_golden(Device d) {
    Tensor x = from_vals({1, 2, 3, 4}, {1, 1, 2, 2}, d);
    x.requires_grad(true);
    nn::Conv2dModule conv(1, 1, 1);
    conv.to(d);
    for (auto& np : conv.named_parameters()) {
        if (np.first == "weight") np.second->data_ = from_vals({2.0f}, {1, 1, 1, 1}, d);
        np.second->data_.requires_grad(true);
    }
    Tensor y = conv.forward(x);
    check_vec(y, {2, 4, 6, 8}, "y");
    Tensor up = from_vals({0.1f, 0.2f, 0.3f, 0.4f}, {1, 1, 2, 2}, d);
    Engine().execute(y.autograd_meta()->grad_fn_, up, false);
    check_vec(x.grad(), {0.2f, 0.4f, 0.6f, 0.8f}, "dX");
    for (auto& np : conv.named_parameters()) {
        if (np.first == "weight") check_vec(np.second->data_.grad(), {3.0f}, "dW");
        if (np.first == "bias") check_vec(np.second->data_.grad(), {1.0f}, "db");
    }
}

// The same golden case through nn::Conv2d's explicit backward (GPU module,
// bias disabled -> zero bias gradient).
void t_conv2d_module_explicit_backward(Device d) {
    if (d.type != DeviceType::CUDA) return;  // nn::Conv2d lives on the GPU, as in the reference
    nn::Conv2d conv(1, 1, 1, 1, 1, 1, 0, 0, 1, 1, false);
    conv.weight().data_ = from_vals({2.0f}, {1, 1, 1, 1}, d);
    Tensor x = from_vals({1, 2, 3, 4}, {1, 1, 2, 2}, d);
    Tensor go = from_vals({0.1f, 0.2f, 0.3f, 0.4f}, {1, 1, 2, 2}, d);
    nn::Conv2dGrad g = conv.backward(go, x);
    check_vec(g.grad_input, {0.2f, 0.4f, 0.6f, 0.8f}, "dX");
    check_vec(g.grad_weight, {3.0f}, "dW");
    check_vec(g.grad_bias, {0.0f}, "db");
}

// Linear: y = x W^T + b, dX = dY W, dW = dY^T X, db = colsum dY.
void t_linear_grads(Device d) {
    nn::Linear fc(3, 2);
    fc.to(d);
    Tensor W = from_vals({1, 2, 3, 4, 5, 6}, {2, 3}, d);
    Tensor b = from_vals({0.5f, -1.0f}, {2}, d);
    for (auto& np : fc.named_parameters()) {
        np.second->data_ = np.first == "weight" ? W : b;
        np.second->data_.requires_grad(true);
    }
    Tensor x = from_vals({1, 0, -1, 2, 1, 0}, {2, 3}, d);
    x.requires_grad(true);
    Tensor y = fc.forward(x);
    check_vec(y, {-1.5f, -3.0f, 4.5f, 12.0f}, "y");
    Tensor up = from_vals({1, 2, 3, 4}, {2, 2}, d);
    Engine().execute(y.autograd_meta()->grad_fn_, up, false);
    check_vec(x.grad(), {9, 12, 15, 19, 26, 33}, "dX");
    for (auto& np : fc.named_parameters()) {
        if (np.first == "weight") check_vec(np.second->data_.grad(), {7, 3, -1, 10, 4, -2}, "dW");
        if (np.first == "bias") check_vec(np.second->data_.grad(), {4, 6}, "db");
    }
}

// Linear::forward_relu = relu(Linear::forward): the same layer and upstream
// as t_linear_grads, rows with a negative pre-activation masked out.
void t_linear_relu_fused(Device d) {
    nn::Linear fc(3, 2);
    fc.to(d);
    Tensor W = from_vals({1, 2, 3, 4, 5, 6}, {2, 3}, d);
    Tensor b = from_vals({0.5f, -1.0f}, {2}, d);
    for (auto& np : fc.named_parameters()) {
        np.second->data_ = np.first == "weight" ? W : b;
        np.second->data_.requires_grad(true);
    }
    Tensor x = from_vals({1, 0, -1, 2, 1, 0}, {2, 3}, d);
    x.requires_grad(true);
    Tensor y = fc.forward_relu(x);
    check_vec(y, {0.0f, 0.0f, 4.5f, 12.0f}, "y");
    Tensor up = from_vals({1, 2, 3, 4}, {2, 2}, d);
    Engine().execute(y.autograd_meta()->grad_fn_, up, false);
    // dZ = up * (y > 0) = [[0, 0], [3, 4]].
    check_vec(x.grad(), {0, 0, 0, 19, 26, 33}, "dX");
    for (auto& np : fc.named_parameters()) {
        if (np.first == "weight") check_vec(np.second->data_.grad(), {6, 3, 0, 8, 4, 0}, "dW");
        if (np.first == "bias") check_vec(np.second->data_.grad(), {3, 4}, "db");
    }
}

// Linear::forward_relu on a layer wide enough for the one-pass ReLU backward
// + bias gradient (300 rows x 256 outputs, three row chunks), fp32 and (on
// the GPU) bf16 compute: dX and dW equal those of forward() then relu(), db
// within fp32 summation tolerance of it and of a double-precision sum of the
// masked upstream gradient.
void t_linear_relu_bias_wide(Device d) {
    const int R = 300, I = 96, O = 256;
    std::vector<float> xv(R * I), wv(O * I), bv(O), uv(R * O);
    for (int i = 0; i < R * I; ++i) xv[i] = std::sin(0.37f * i);
    for (int i = 0; i < O * I; ++i) wv[i] = 0.1f * std::cos(0.11f * i);
    for (int i = 0; i < O; ++i) bv[i] = 0.5f * std::sin(1.3f * i);
    for (int i = 0; i < R * O; ++i) uv[i] = std::cos(0.07f * i);
    const bool gpu = d.type == DeviceType::CUDA;
    for (int bf16 = 0; bf16 <= (gpu ? 1 : 0); ++bf16) {
        std::vector<float> got[2][4];   // [fused?][y, dX, dW, db]
        for (int fused = 0; fused < 2; ++fused) {
            nn::Linear fc(I, O);
            fc.to(d);
            if (bf16) fc.set_compute_dtype(Dtype::BFloat16);
            Tensor W = from_vals(wv, {O, I}, d), b = from_vals(bv, {O}, d);
            for (auto& np : fc.named_parameters()) {
                np.second->data_ = np.first == "weight" ? W : b;
                np.second->data_.requires_grad(true);
            }
            Tensor x = from_vals(xv, {R, I}, d);
            x.requires_grad(true);
            Tensor y = fused ? fc.forward_relu(x) : fc.forward(x).relu();
            Tensor up = from_vals(uv, {R, O}, d);
            if (bf16) up = up.to(Dtype::BFloat16);
            Engine().execute(y.autograd_meta()->grad_fn_, up, false);
            got[fused][0] = to_host(y);
            got[fused][1] = to_host(x.grad());
            for (auto& np : fc.named_parameters())
                got[fused][np.first == "weight" ? 2 : 3] = to_host(np.second->data_.grad());
            TFA_CHECK(got[fused][2].size() == (size_t)O * I && got[fused][3].size() == (size_t)O);
        }
        const std::string tag = bf16 ? " (bf16)" : " (fp32)";
        for (int k = 0; k < 3; ++k)
            for (size_t i = 0; i < got[0][k].size(); ++i)
                check_near(got[1][k][i], got[0][k][i], 1e-6f, "fused vs relu(forward)" + tag + " output " +
                                                               std::to_string(k) + "[" + std::to_string(i) + "]");
        for (int o = 0; o < O; ++o) {
            // The masked upstream gradient as the backward sees it (bf16 up
            // in bf16 compute), summed in double.
            double s = 0.0;
            for (int r = 0; r < R; ++r) {
                float u = uv[r * O + o];
                if (bf16) u = to_host(from_vals({u}, {1}, Device::cpu()).to(Dtype::BFloat16))[0];
                if (got[0][0][r * O + o] > 0.0f) s += u;
            }
            check_near(got[1][3][o], got[0][3][o], 1e-5f, "db fused vs relu(forward)" + tag + "[" + std::to_string(o) + "]");
            check_near(got[1][3][o], (float)s, 1e-4f, "db vs double sum" + tag + "[" + std::to_string(o) + "]");
        }
    }
}

// Linear::forward_relu on a bias-free fp32 layer, whose backward node takes
// the ReLU itself (on the GPU its products apply the mask as they load dy):
// y, dX and dW equal those of forward() then relu() bit for bit, with and
// without dX wanted (a first layer), and the upstream gradient of y is left
// unmasked.
void t_linear_relu_nobias(Device d) {
    const int R = 64, I = 96, O = 256;
    std::vector<float> xv(R * I), wv(O * I), uv(R * O);
    for (int i = 0; i < R * I; ++i) xv[i] = std::sin(0.37f * i);
    for (int i = 0; i < O * I; ++i) wv[i] = 0.1f * std::cos(0.11f * i);
    for (int i = 0; i < R * O; ++i) uv[i] = std::cos(0.07f * i);
    for (int want_dx = 0; want_dx < 2; ++want_dx) {
        std::vector<float> got[2][3];   // [fused?][y, dX, dW]
        for (int fused = 0; fused < 2; ++fused) {
            nn::Linear fc(I, O, false);
            fc.to(d);
            Tensor W = from_vals(wv, {O, I}, d);
            for (auto& np : fc.named_parameters()) {
                np.second->data_ = W;
                np.second->data_.requires_grad(true);
            }
            Tensor x = from_vals(xv, {R, I}, d);
            x.requires_grad(want_dx != 0);
            Tensor y = fused ? fc.forward_relu(x) : fc.forward(x).relu();
            Tensor up = from_vals(uv, {R, O}, d);
            Engine().execute(y.autograd_meta()->grad_fn_, up, false);
            got[fused][0] = to_host(y);
            if (want_dx) got[fused][1] = to_host(x.grad());
            else TFA_CHECK(!x.grad().storage());
            got[fused][2] = to_host(fc.named_parameters().at(0).second->data_.grad());
            TFA_CHECK(got[fused][2].size() == (size_t)O * I);
            TFA_CHECK(to_host(up) == uv);
        }
        for (int k = 0; k < 3; ++k) {
            TFA_CHECK(got[0][k].size() == got[1][k].size());
            for (size_t i = 0; i < got[0][k].size(); ++i)
                if (!(got[1][k][i] == got[0][k][i]))
                    check_near(got[1][k][i], got[0][k][i], 0.0f, "bias-free fused vs relu(forward) output " +
                                                                    std::to_string(k) + "[" + std::to_string(i) + "]");
        }
    }
}

// Conv2dModule::forward_relu on a 1x1 convolution (w = 2, b = 0).
void t_conv_relu_fused(Device d) {
    Tensor x = from_vals({1, -2, 3, -4}, {1, 1, 2, 2}, d);
    x.requires_grad(true);
    nn::Conv2dModule conv(1, 1, 1);
    conv.to(d);
    for (auto& np : conv.named_parameters()) {
        if (np.first == "weight") np.second->data_ = from_vals({2.0f}, {1, 1, 1, 1}, d);
        np.second->data_.requires_grad(true);
    }
    Tensor y = conv.forward_relu(x);
    check_vec(y, {2, 0, 6, 0}, "y");
    Tensor up = from_vals({0.1f, 0.2f, 0.3f, 0.4f}, {1, 1, 2, 2}, d);
    Engine().execute(y.autograd_meta()->grad_fn_, up, false);
    check_vec(x.grad(), {0.2f, 0.0f, 0.6f, 0.0f}, "dX");
    for (auto& np : conv.named_parameters()) {
        if (np.first == "weight") check_vec(np.second->data_.grad(), {1.0f}, "dW");
        if (np.first == "bias") check_vec(np.second->data_.grad(), {0.4f}, "db");
    }
}

// optim::SGD momentum rule v = mu v + g; p = p - lr v (nn/optim/SGD.hpp:3-6).
void t_sgd_momentum_rule(Device d) {
    Tensor p = from_vals({1.0f, -2.0f}, {2}, d);
    p.requires_grad(true);
    nn::optim::SGD opt({&p}, 0.5f, 0.9f);
    for (int s = 0; s < 2; ++s) {
        Tensor g = from_vals({0.2f, 0.4f}, {2}, d);
        p.autograd_meta()->grad_ = g;
        opt.step();
    }
    // v1 = g, p1 = p0 - 0.5 g; v2 = 0.9 g + g = 1.9 g; p2 = p1 - 0.95 g.
    check_vec(p, {1.0f - 0.5f * 0.2f - 0.95f * 0.2f, -2.0f - 0.5f * 0.4f - 0.95f * 0.4f}, "p", 1e-6f);
}

// Reshape is wired: a flatten feeding a Linear reaches the conv output.
void t_reshape_grad(Device d) {
    Tensor x = filled({2, 3, 2}, 1.0f, d);
    x.requires_grad(true);
    Tensor f = reshape(x, Shape{2, 6});
    f.sum(1).sum(0).backward();
    check_all(x.grad(), 1.0f, "dx");
    TFA_CHECK(x.grad().shape() == (Shape{2, 3, 2}));
}

// Sum over a non-final dim with a non-uniform upstream: true broadcast.
void t_sum_broadcast(Device d) {
    Tensor x = filled({2, 3}, 1.0f, d);
    x.requires_grad(true);
    Tensor s = x.sum(1);  // [2]
    Engine().execute(s.autograd_meta()->grad_fn_, from_vals({1.0f, 5.0f}, {2}, d), false);
    check_vec(x.grad(), {1, 1, 1, 5, 5, 5}, "dx");
}

// The file loaders on synthetic files (3 MNIST images and labels, 4 CIFAR
// records in two batches): shapes, the reference's normalisation of known
// bytes, and -- on the GPU -- the device decode bit for bit equal to the
// host decode.
void t_data_loaders(Device d) {
    namespace fs = std::filesystem;
    const fs::path dir = fs::temp_directory_path() / ("tfa_data_" + std::to_string(::getpid()));
    fs::create_directories(dir);
    auto put = [&](const char* name, const std::vector<uint8_t>& bytes) {
        std::ofstream(dir / name, std::ios::binary).write(reinterpret_cast<const char*>(bytes.data()),
                                                          static_cast<std::streamsize>(bytes.size()));
    };
    auto be = [](std::vector<uint8_t>& v, uint32_t x) {
        for (int s = 24; s >= 0; s -= 8) v.push_back(static_cast<uint8_t>(x >> s));
    };
    std::vector<uint8_t> img, lab;
    be(img, 0x803); be(img, 3); be(img, 28); be(img, 28);
    for (int i = 0; i < 3 * 784; ++i) img.push_back(static_cast<uint8_t>((i * 37 + 11) & 255));
    be(lab, 0x801); be(lab, 3);
    for (uint8_t v : {7, 0, 9}) lab.push_back(v);
    for (const char* f : {"train-images-idx3-ubyte", "t10k-images-idx3-ubyte"}) put(f, img);
    for (const char* f : {"train-labels-idx1-ubyte", "t10k-labels-idx1-ubyte"}) put(f, lab);
    std::vector<uint8_t> rec;
    for (int r = 0; r < 2; ++r) {
        rec.push_back(static_cast<uint8_t>(3 + r));
        for (int i = 0; i < 3072; ++i) rec.push_back(static_cast<uint8_t>((i * 13 + 7 * r) & 255));
    }
    for (const char* f : {"data_batch_1.bin", "data_batch_2.bin", "data_batch_3.bin", "data_batch_4.bin",
                          "data_batch_5.bin", "test_batch.bin"})
        put(f, rec);
    auto [mx, my] = data::load_mnist_train(dir.string());
    TFA_CHECK(mx.shape() == (Shape{3, 1, 28, 28}) && my.shape() == (Shape{3}));
    const float* px = static_cast<const float*>(mx.data());
    for (int i : {0, 1, 783, 2351}) {
        const float want = (static_cast<float>((i * 37 + 11) & 255) * (1.0f / 255.0f) - 0.1307f) * (1.0f / 0.3081f);
        TFA_CHECK(px[i] == want);
    }
    TFA_CHECK(static_cast<const int64_t*>(my.data())[2] == 9);
    auto [cx, cy] = data::load_cifar10_train(dir.string());
    TFA_CHECK(cx.shape() == (Shape{10, 3, 32, 32}) && cy.shape() == (Shape{10}));
    const float* pc = static_cast<const float*>(cx.data());
    const float want_g = (static_cast<float>((1024 * 13 + 5 * 0) & 255) * (1.0f / 255.0f) - 0.4822f) / 0.2435f;
    TFA_CHECK(pc[1024] == want_g && static_cast<const int64_t*>(cy.data())[1] == 4);
    if (d.type == DeviceType::CUDA) {
        auto [gx, gy] = data::load_mnist_test(dir.string(), d);
        auto [hx, hy] = data::load_cifar10_test(dir.string(), d);
        auto bits_equal = [](const Tensor& dev, const Tensor& host) {
            Tensor back = dev.to(Device::cpu());
            return back.numel() == host.numel() &&
                   std::memcmp(back.data(), host.data(), static_cast<size_t>(host.numel()) * dtype_size(host.dtype())) == 0;
        };
        auto [tx, ty] = data::load_mnist_test(dir.string());
        auto [ux, uy] = data::load_cifar10_test(dir.string());
        TFA_CHECK(gx.device() == d && bits_equal(gx, tx) && bits_equal(gy, ty));
        TFA_CHECK(hx.device() == d && bits_equal(hx, ux) && bits_equal(hy, uy));
    }
    fs::remove_all(dir);
}

const std::map<std::string, std::function<void(Device)>>& registry() {
    static const std::map<std::string, std::function<void(Device)>> r = {
        {"engine_fan_in", t_engine_fan_in},
        {"data_loaders", t_data_loaders},
        {"engine_deep_chain", t_engine_deep_chain},
        {"chain_add_mul_sum", t_chain_add_mul_sum},
        {"transpose_grad", t_transpose_grad},
        {"matmul_known_answer", t_matmul_known_answer},
        {"matmul_ones", t_matmul_ones},
        {"relu_mask", t_relu_mask},
        {"softmax_uniform", t_softmax_uniform},
        {"log_softmax_closed_form", t_log_softmax_closed_form},
        {"mul_arange", t_mul_arange},
        {"saved_tensor_version", t_saved_tensor_version},
        {"cross_entropy_known", t_cross_entropy_known},
        {"cross_entropy_grad", t_cross_entropy_grad},
        {"cross_entropy_scaled_upstream", t_cross_entropy_scaled_upstream},
        {"sigmoid_tanh_grad", t_sigmoid_tanh_grad},
        {"layernorm_grad", t_layernorm_grad},
        {"conv_1x1_golden", t_conv_1x1_golden},
        {"conv2d_explicit_backward", t_conv2d_module_explicit_backward},
        {"linear_grads", t_linear_grads},
        {"linear_relu_fused", t_linear_relu_fused},
        {"linear_relu_bias_wide", t_linear_relu_bias_wide},
        {"linear_relu_nobias", t_linear_relu_nobias},
        {"conv_relu_fused", t_conv_relu_fused},
        {"sgd_momentum_rule", t_sgd_momentum_rule},
        {"reshape_grad", t_reshape_grad},
        {"sum_broadcast", t_sum_broadcast},
        {"leaky_relu", t_leaky_relu},
    };
    return r;
}

}  // namespace

extern "C" {

const char* tfa_last_error(void) { return g_err.c_str(); }

const char* tfa_selftest_names(void) {
    static std::string names;
    if (names.empty())
        for (const auto& kv : registry()) names += (names.empty() ? "" : " ") + kv.first;
    return names.c_str();
}

int tfa_selftest(const char* name, int32_t on_gpu) {
    return guarded([&] {
        auto it = registry().find(name ? name : "");
        if (it == registry().end()) throw std::invalid_argument(std::string("unknown self-test ") + (name ? name : ""));
        CompatScope scope(false);
        it->second(dev_of(on_gpu));
        sync_if_gpu(on_gpu);
    });
}

int tfa_mlp_train(const int32_t* dims, int32_t ndims, int64_t batch, int64_t steps, int64_t warmup, int64_t n_batches,
                  const float* xs, const int64_t* ys, float lr, float mu, int32_t on_gpu, int32_t reference_compat,
                  int32_t bf16, const float* init_weights, float* losses, float* final_weights, double* ms_per_step,
                  uint64_t* pool_used, int32_t graph) {
    return guarded([&] {
        if (ndims < 2 || batch <= 0 || steps < 0 || n_batches <= 0 || warmup < 0 || warmup > steps)
            throw std::invalid_argument("tfa_mlp_train: bad sizes");
        if (bf16 && !on_gpu) throw std::invalid_argument("tfa_mlp_train: bf16 needs the GPU");
        if (pool_used && !on_gpu) throw std::invalid_argument("tfa_mlp_train: pool_used needs the GPU");
        if (graph < 0 || graph > 2) throw std::invalid_argument("tfa_mlp_train: graph must be 0, 1 or 2");
        if (graph && (!on_gpu || pool_used || warmup < 1))
            throw std::invalid_argument("tfa_mlp_train: graph needs the GPU, warmup >= 1 and no pool_used");
        CompatScope scope(reference_compat != 0);
        const Device d = dev_of(on_gpu);
        std::vector<std::shared_ptr<nn::Linear>> layers;
        size_t off = 0;
        for (int32_t l = 0; l + 1 < ndims; ++l) {
            auto fc = std::make_shared<nn::Linear>(dims[l], dims[l + 1]);
            if (init_weights) {
                for (auto& np : fc->named_parameters())
                    if (np.first == "weight")
                        std::memcpy(np.second->data_.data(), init_weights + off, sizeof(float) * np.second->data_.numel());
            }
            off += static_cast<size_t>(dims[l]) * dims[l + 1];
            fc->to(d);
            if (bf16) fc->set_compute_dtype(Dtype::BFloat16);
            layers.push_back(fc);
        }
        std::vector<Tensor*> params;
        for (auto& fc : layers)
            for (auto* p : fc->parameters()) params.push_back(&p->data_);
        nn::optim::SGD opt(params, lr, mu);
        nn::CrossEntropyLoss ce;

        std::vector<Tensor> xb, yb;
        for (int64_t i = 0; i < n_batches; ++i) {
            xb.push_back(host_f32(xs + i * batch * dims[0], Shape{batch, dims[0]}).to(d));
            yb.push_back(host_i64(ys + i * batch, Shape{batch}).to(d));
        }
        std::vector<Tensor> loss_t;
        loss_t.reserve(static_cast<size_t>(steps));
        auto run_step = [&](int64_t s) {
            Tensor h = xb[s % n_batches];
            // Hidden layers: Linear then ReLU, fused into one GEMM on the GPU.
            for (size_t l = 0; l < layers.size(); ++l)
                h = l + 1 < layers.size() ? layers[l]->forward_relu(h) : layers[l]->forward(h);
            Tensor loss = ce.forward(h, yb[s % n_batches]);
            loss.backward();
            opt.step();
            // Keep the value only: the step's autograd graph (nodes, edges)
            // is released with `loss` instead of living until the end.
            Tensor kept = loss;
            kept.autograd_meta().reset();
            loss_t.push_back(kept);
            if (pool_used) {
                hip::synchronize(0);
                hip::pool_stats(0, nullptr, &pool_used[s]);
            }
        };
        if (!graph) {
            for (int64_t s = 0; s < warmup; ++s) run_step(s);
            sync_if_gpu(on_gpu);
            auto t0 = std::chrono::steady_clock::now();
            for (int64_t s = warmup; s < steps; ++s) run_step(s);
            sync_if_gpu(on_gpu);
            auto t1 = std::chrono::steady_clock::now();
            if (ms_per_step)
                *ms_per_step = steps > warmup ? std::chrono::duration<double, std::milli>(t1 - t0).count() / double(steps - warmup) : 0.0;
            if (losses)
                for (int64_t s = 0; s < steps; ++s) losses[s] = to_host(loss_t[static_cast<size_t>(s)])[0];
        } else {
            // One HIP graph per step: the step reads its batch through a
            // device table indexed by a device step counter and records its
            // loss in a device ring (which advances the counter), so a replay
            // needs no host work but its launch.  The warmup steps run the
            // same step eagerly, which also fills the block cache that the
            // capture allocates from.
            std::vector<int64_t> xt, yt;
            for (int64_t i = 0; i < n_batches; ++i) {
                xt.push_back(static_cast<int64_t>(reinterpret_cast<uintptr_t>(xb[i].data())));
                yt.push_back(static_cast<int64_t>(reinterpret_cast<uintptr_t>(yb[i].data())));
            }
            const Tensor xtab = host_i64(xt.data(), Shape{n_batches}).to(d);
            const Tensor ytab = host_i64(yt.data(), Shape{n_batches}).to(d);
            const int64_t zero = 0;
            Tensor counter = host_i64(&zero, Shape{1}).to(d);
            Tensor ring = Tensor::empty(Shape{steps}, Dtype::Float32, d);
            Tensor xs_dev = Tensor::empty(Shape{batch, dims[0]}, Dtype::Float32, d);
            Tensor ys_dev = Tensor::empty(Shape{batch}, Dtype::Int64, d);
            auto graph_step = [&] {
                hip::gather_indexed(xs_dev.data(), static_cast<const uint64_t*>(xtab.data()), n_batches,
                                    static_cast<const int64_t*>(counter.data()), batch * dims[0] * 4);
                hip::gather_indexed(ys_dev.data(), static_cast<const uint64_t*>(ytab.data()), n_batches,
                                    static_cast<const int64_t*>(counter.data()), batch * 8);
                Tensor h = xs_dev;
                for (size_t l = 0; l < layers.size(); ++l)
                    h = l + 1 < layers.size() ? layers[l]->forward_relu(h) : layers[l]->forward(h);
                Tensor loss = ce.forward(h, ys_dev);
                loss.backward();
                opt.step();
                hip::record_step(static_cast<const float*>(loss.data()), static_cast<float*>(ring.data()), steps,
                                 static_cast<int64_t*>(counter.data()));
            };
            for (int64_t s = 0; s < warmup; ++s) graph_step();
            sync_if_gpu(on_gpu);
            hip::CapturedGraph g = hip::capture(graph_step);
            std::vector<float> seen;
            auto t0 = std::chrono::steady_clock::now();
            for (int64_t s = warmup; s < steps; ++s) {
                g.launch();
                if (graph == 2) {
                    // Checked replay: the host waits for each replay and reads
                    // its loss (eager work and a synchronisation between
                    // replays), then the ring is compared with these reads.
                    seen.push_back(to_host(ring)[static_cast<size_t>(s)]);
                }
            }
            sync_if_gpu(on_gpu);
            auto t1 = std::chrono::steady_clock::now();
            if (ms_per_step)
                *ms_per_step = steps > warmup ? std::chrono::duration<double, std::milli>(t1 - t0).count() / double(steps - warmup) : 0.0;
            const std::vector<float> ring_h = to_host(ring);
            for (size_t i = 0; i < seen.size(); ++i)
                if (std::memcmp(&seen[i], &ring_h[static_cast<size_t>(warmup) + i], sizeof(float)) != 0)
                    throw std::runtime_error("tfa_mlp_train: a replay's loss changed after later replays");
            if (losses)
                for (int64_t s = 0; s < steps; ++s) losses[s] = ring_h[static_cast<size_t>(s)];
        }
        if (final_weights) {
            size_t o = 0;
            for (auto& fc : layers)
                for (auto& np : fc->named_parameters())
                    if (np.first == "weight") {
                        auto v = to_host(np.second->data_);
                        std::memcpy(final_weights + o, v.data(), sizeof(float) * v.size());
                        o += v.size();
                    }
        }
    });
}

int tfa_mlp_step_trace(const int32_t* dims, int32_t ndims, int64_t batch, const float* x, const int64_t* y, float lr,
                       float mu, int32_t on_gpu, int32_t bf16, const float* init_weights, float* loss, float* acts,
                       float* grads, float* final_weights, float* final_biases) {
    return guarded([&] {
        if (ndims < 2 || batch <= 0) throw std::invalid_argument("tfa_mlp_step_trace: bad sizes");
        if (bf16 && !on_gpu) throw std::invalid_argument("tfa_mlp_step_trace: bf16 needs the GPU");
        CompatScope scope(false);
        const Device d = dev_of(on_gpu);
        std::vector<std::shared_ptr<nn::Linear>> layers;
        size_t off = 0;
        for (int32_t l = 0; l + 1 < ndims; ++l) {
            auto fc = std::make_shared<nn::Linear>(dims[l], dims[l + 1]);
            if (init_weights)
                for (auto& np : fc->named_parameters())
                    if (np.first == "weight")
                        std::memcpy(np.second->data_.data(), init_weights + off, sizeof(float) * np.second->data_.numel());
            off += static_cast<size_t>(dims[l]) * dims[l + 1];
            fc->to(d);
            if (bf16) fc->set_compute_dtype(Dtype::BFloat16);
            layers.push_back(fc);
        }
        std::vector<Tensor*> params;
        for (auto& fc : layers)
            for (auto* p : fc->parameters()) params.push_back(&p->data_);
        nn::optim::SGD opt(params, lr, mu);
        nn::CrossEntropyLoss ce;
        // The step of tfa_mlp_train, keeping every layer's output.
        std::vector<Tensor> outs;
        Tensor h = host_f32(x, Shape{batch, dims[0]}).to(d);
        Tensor in = h;
        for (size_t l = 0; l < layers.size(); ++l) {
            h = l + 1 < layers.size() ? layers[l]->forward_relu(h) : layers[l]->forward(h);
            outs.push_back(h);
        }
        Tensor lt = ce.forward(h, host_i64(y, Shape{batch}).to(d));
        lt.backward();
        opt.step();
        *loss = to_host(lt)[0];
        // The first layer's input as its GEMM read it (bf16 compute rounds it).
        std::vector<float> a0 = to_host(bf16 ? in.to(Dtype::BFloat16) : in);
        std::memcpy(acts, a0.data(), sizeof(float) * a0.size());
        size_t ao = a0.size(), go = 0;
        for (auto& t : outs) {
            const std::vector<float> a = to_host(t), g = to_host(t.grad());
            if (a.size() != g.size()) throw std::runtime_error("tfa_mlp_step_trace: a layer output has no gradient");
            std::memcpy(acts + ao, a.data(), sizeof(float) * a.size());
            std::memcpy(grads + go, g.data(), sizeof(float) * g.size());
            ao += a.size();
            go += g.size();
        }
        size_t wo = 0, bo = 0;
        for (auto& fc : layers)
            for (auto& np : fc->named_parameters()) {
                const std::vector<float> v = to_host(np.second->data_);
                if (np.first == "weight") {
                    if (final_weights) std::memcpy(final_weights + wo, v.data(), sizeof(float) * v.size());
                    wo += v.size();
                } else {
                    if (final_biases) std::memcpy(final_biases + bo, v.data(), sizeof(float) * v.size());
                    bo += v.size();
                }
            }
    });
}

int tfa_release_memory(void) {
    return guarded([&] { hip::trim(0); });
}

int tfa_cnn_train(int64_t batch, int64_t H, int64_t W, int64_t steps, int64_t warmup, int64_t n_batches, const float* xs,
                  const int64_t* ys, float lr, float mu, int32_t on_gpu, const float* init_params, float* losses,
                  float* final_params, double* ms_per_step) {
    return guarded([&] {
        if (batch <= 0 || steps < 0 || n_batches <= 0 || warmup < 0 || warmup > steps || H % 2 || W % 2)
            throw std::invalid_argument("tfa_cnn_train: bad sizes");
        CompatScope scope(false);
        const Device d = dev_of(on_gpu);
        nn::Conv2dModule conv1(3, 32, 3, 1, 1), conv2(32, 64, 3, 2, 1);
        const int64_t flat = 64 * (H / 2) * (W / 2);
        nn::Linear fc(static_cast<int>(flat), 10);
        // The six parameters in the order of init_params / final_params.
        const std::pair<nn::Module*, const char*> order[6] = {{&conv1, "weight"}, {&conv1, "bias"}, {&conv2, "weight"},
                                                              {&conv2, "bias"},   {&fc, "weight"},    {&fc, "bias"}};
        auto param = [](nn::Module* m, const char* name) -> Tensor& {
            for (auto& np : m->named_parameters())
                if (np.first == name) return np.second->data_;
            throw std::logic_error(std::string("tfa_cnn_train: no parameter ") + name);
        };
        if (init_params) {
            size_t off = 0;
            for (const auto& o : order) {
                Tensor& t = param(o.first, o.second);
                std::memcpy(t.data(), init_params + off, sizeof(float) * static_cast<size_t>(t.numel()));
                off += static_cast<size_t>(t.numel());
            }
        }
        conv1.to(d);
        conv2.to(d);
        fc.to(d);
        std::vector<Tensor*> params;
        for (nn::Module* m : std::initializer_list<nn::Module*>{&conv1, &conv2, &fc})
            for (auto* p : m->parameters()) params.push_back(&p->data_);
        nn::optim::SGD opt(params, lr, mu);
        nn::CrossEntropyLoss ce;
        std::vector<Tensor> xb, yb;
        for (int64_t i = 0; i < n_batches; ++i) {
            xb.push_back(host_f32(xs + i * batch * 3 * H * W, Shape{batch, 3, H, W}).to(d));
            yb.push_back(host_i64(ys + i * batch, Shape{batch}).to(d));
        }
        std::vector<Tensor> loss_t;
        auto run_step = [&](int64_t s) {
            // Conv then ReLU, fused into one GEMM on the GPU.
            Tensor h = conv1.forward_relu(xb[s % n_batches]);
            h = conv2.forward_relu(h);
            h = reshape(h, Shape{batch, flat});
            Tensor loss = ce.forward(fc.forward(h), yb[s % n_batches]);
            loss.backward();
            opt.step();
            // Keep the value only: the step's autograd graph (nodes, edges)
            // is released with `loss` instead of living until the end.
            Tensor kept = loss;
            kept.autograd_meta().reset();
            loss_t.push_back(kept);
        };
        for (int64_t s = 0; s < warmup; ++s) run_step(s);
        sync_if_gpu(on_gpu);
        auto t0 = std::chrono::steady_clock::now();
        for (int64_t s = warmup; s < steps; ++s) run_step(s);
        sync_if_gpu(on_gpu);
        auto t1 = std::chrono::steady_clock::now();
        if (ms_per_step)
            *ms_per_step = steps > warmup ? std::chrono::duration<double, std::milli>(t1 - t0).count() / double(steps - warmup) : 0.0;
        if (losses)
            for (int64_t s = 0; s < steps; ++s) losses[s] = to_host(loss_t[static_cast<size_t>(s)])[0];
        if (final_params) {
            size_t off = 0;
            for (const auto& o : order) {
                auto v = to_host(param(o.first, o.second));
                std::memcpy(final_params + off, v.data(), sizeof(float) * v.size());
                off += v.size();
            }
        }
    });
}

}  // extern "C"
