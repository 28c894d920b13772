// ref_shim.cpp — C entry points over the reference's own CPU implementation,
// compiled together with the reference sources (oracle/Makefile) into
// oracle/_ref/libtfref.so.  TEST INFRASTRUCTURE ONLY: used to pin the C
// restatement (oracle/tf_oracle.c) and to write golden fixtures
// (tests/golden/make_golden.py); never loaded by the product path.
//
// Each function drives the reference's public API exactly as its own tests
// and examples do; citations are relative to the reference repository root.
#include "autograd/AutogradMeta.hpp"
#include "autograd/Engine.hpp"
#include "autograd/ops/LogSoftmaxBackward.hpp"
#include "autograd/ops/ReluBackward.hpp"
#include "autograd/ops/SoftmaxBackward.hpp"
#include "nn/Activations.hpp"
#include "nn/Conv2dModule.hpp"
#include "nn/CrossEntropyLoss.hpp"
#include "nn/Linear.hpp"
#include "tensor/Tensor.hpp"
#include "tensor/factory.hpp"

#include <chrono>
#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

namespace tensorforge {
void init_tensor_autograd();
}

using namespace tensorforge;

namespace {

std::string g_err;

Tensor host_tensor(const float* src, Shape shape) {
    Tensor t = Tensor::empty(std::move(shape), Dtype::Float32, Device::cpu());
    if (src) std::memcpy(t.data(), src, sizeof(float) * static_cast<size_t>(t.numel()));
    return t;
}

void copy_out(const Tensor& t, float* dst) {
    std::memcpy(dst, t.data(), sizeof(float) * static_cast<size_t>(t.numel()));
}

// Run the engine from `out` with upstream gradient `grad` (the reference
// Tensor::backward always seeds ones, autograd/TensorAutograd.cpp:53-71).
void run_backward(const Tensor& out, const Tensor& grad) {
    Engine engine;
    engine.execute(out.autograd_meta()->grad_fn_, grad, false);
}

// examples/train_mlp.cpp:54-76, verbatim in behaviour.
Tensor chain_cross_entropy(const Tensor& logits, const Tensor& labels) {
    const int64_t N = logits.shape()[0];
    const int64_t C = logits.shape()[1];
    Tensor log_probs = logits.log_softmax(-1);
    Tensor mask = zeros(Shape{N, C}, Dtype::Float32, Device::cpu());
    const int64_t* lp = static_cast<const int64_t*>(labels.data());
    float* mp = static_cast<float*>(mask.data());
    for (int64_t i = 0; i < N; ++i) {
        const int64_t t = lp[i];
        if (t >= 0 && t < C) mp[i * C + t] = 1.0f;
    }
    Tensor picked = log_probs * mask;
    Tensor row_sum = picked.sum(1);
    Tensor total = row_sum.sum(0, true);
    Tensor neg_one = full(Shape{1}, -1.0, Dtype::Float32, Device::cpu());
    Tensor total_nll = neg_one * total;
    Tensor n_inv = full(Shape{1}, 1.0 / static_cast<double>(N), Dtype::Float32, Device::cpu());
    return total_nll * n_inv;
}

template <typename F>
int guarded(F&& f) {
    try {
        init_tensor_autograd();
        f();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 1;
    }
}

}  // namespace

extern "C" {

const char* ref_last_error() { return g_err.c_str(); }

int ref_matmul(const float* a, const float* b, float* c, int64_t M, int64_t K, int64_t N) {
    return guarded([&] { copy_out(host_tensor(a, Shape{M, K}).matmul(host_tensor(b, Shape{K, N})), c); });
}

int ref_transpose2d(const float* in, float* out, int64_t R, int64_t C) {
    return guarded([&] { copy_out(host_tensor(in, Shape{R, C}).transpose(0, 1), out); });
}

// MatmulBackward through the engine: c = a.matmul(b), upstream dc.
int ref_matmul_backward(const float* a, const float* b, const float* dc, float* da, float* db, int64_t M,
                        int64_t K, int64_t N) {
    return guarded([&] {
        Tensor ta = host_tensor(a, Shape{M, K}), tb = host_tensor(b, Shape{K, N});
        ta.requires_grad(true);
        tb.requires_grad(true);
        Tensor c = ta.matmul(tb);
        run_backward(c, host_tensor(dc, Shape{M, N}));
        copy_out(ta.grad(), da);
        copy_out(tb.grad(), db);
    });
}

// nn::Linear with a given weight: y = x @ W^T (nn/Linear.cpp:45-64) and its
// backward for upstream dy.  Bias is registered but unused by the reference.
int ref_linear(const float* x, const float* w, const float* dy, float* y, float* dx, float* dw, int64_t B,
               int64_t in, int64_t out) {
    return guarded([&] {
        nn::Linear fc(static_cast<int>(in), static_cast<int>(out));
        for (auto& np : fc.named_parameters())
            if (np.first == "weight") std::memcpy(np.second->data_.data(), w, sizeof(float) * in * out);
        Tensor tx = host_tensor(x, Shape{B, in});
        tx.requires_grad(true);
        Tensor ty = fc.forward(tx);
        copy_out(ty, y);
        run_backward(ty, host_tensor(dy, Shape{B, out}));
        copy_out(tx.grad(), dx);
        for (auto& np : fc.named_parameters())
            if (np.first == "weight") copy_out(np.second->data_.grad(), dw);
    });
}

// Initial weight of nn::Linear(in, out) (nn/Linear.cpp:21-29).
int ref_linear_init(int64_t in, int64_t out, float* w) {
    return guarded([&] {
        nn::Linear fc(static_cast<int>(in), static_cast<int>(out));
        for (auto& np : fc.named_parameters())
            if (np.first == "weight") copy_out(np.second->data_, w);
    });
}

// Initial weight of nn::Conv2dModule (nn/Conv2dModule.cpp:72-102).
int ref_conv2d_init(int64_t cin, int64_t cout, int64_t k, float* w) {
    return guarded([&] {
        nn::Conv2dModule conv(static_cast<int>(cin), static_cast<int>(cout), static_cast<int>(k));
        for (auto& np : conv.named_parameters())
            if (np.first == "weight") copy_out(np.second->data_, w);
    });
}

int ref_relu_fwd(const float* x, float* y, int64_t n) {
    return guarded([&] { copy_out(host_tensor(x, Shape{n}).relu(), y); });
}
int ref_leaky_relu_fwd(const float* x, float* y, int64_t n, float alpha) {
    return guarded([&] { copy_out(host_tensor(x, Shape{n}).leaky_relu(alpha), y); });
}
int ref_sigmoid_fwd(const float* x, float* y, int64_t n) {
    return guarded([&] { copy_out(host_tensor(x, Shape{n}).sigmoid(), y); });
}
int ref_tanh_fwd(const float* x, float* y, int64_t n) {
    return guarded([&] { copy_out(host_tensor(x, Shape{n}).tanh(), y); });
}

int ref_relu_bwd(const float* dy, const float* x, float* dx, int64_t n) {
    return guarded([&] {
        ReluBackward node(host_tensor(x, Shape{n}));
        std::vector<Tensor> g{host_tensor(dy, Shape{n})};
        copy_out(node.apply(std::move(g))[0], dx);
    });
}

int ref_log_softmax_fwd(const float* x, float* y, int64_t R, int64_t C) {
    return guarded([&] { copy_out(host_tensor(x, Shape{R, C}).log_softmax(-1), y); });
}
int ref_softmax_fwd(const float* x, float* y, int64_t R, int64_t C) {
    return guarded([&] { copy_out(host_tensor(x, Shape{R, C}).softmax(-1), y); });
}
int ref_log_softmax_bwd(const float* y, const float* gy, float* gx, int64_t R, int64_t C) {
    return guarded([&] {
        LogSoftmaxBackward node(host_tensor(y, Shape{R, C}));
        std::vector<Tensor> g{host_tensor(gy, Shape{R, C})};
        copy_out(node.apply(std::move(g))[0], gx);
    });
}
int ref_softmax_bwd(const float* y, const float* gy, float* gx, int64_t R, int64_t C) {
    return guarded([&] {
        SoftmaxBackward node(host_tensor(y, Shape{R, C}));
        std::vector<Tensor> g{host_tensor(gy, Shape{R, C})};
        copy_out(node.apply(std::move(g))[0], gx);
    });
}

int ref_sum(const float* x, float* out, int64_t R, int64_t C, int64_t dim) {
    return guarded([&] { copy_out(host_tensor(x, Shape{R, C}).sum(dim), out); });
}

int ref_add(const float* a, const float* b, float* out, int64_t n) {
    return guarded([&] { copy_out(host_tensor(a, Shape{n}) + host_tensor(b, Shape{n}), out); });
}

int ref_layernorm_fwd(const float* x, const float* g, const float* b, float* y, int64_t R, int64_t C, float eps) {
    return guarded([&] {
        copy_out(host_tensor(x, Shape{R, C}).layer_norm(host_tensor(g, Shape{C}), host_tensor(b, Shape{C}), eps), y);
    });
}

// LayerNormBackward through the engine (the reference's stub gradient).
int ref_layernorm_bwd(const float* x, const float* g, const float* b, const float* dy, float* dx, int64_t R,
                      int64_t C, float eps) {
    return guarded([&] {
        Tensor tx = host_tensor(x, Shape{R, C});
        tx.requires_grad(true);
        Tensor y = tx.layer_norm(host_tensor(g, Shape{C}), host_tensor(b, Shape{C}), eps);
        run_backward(y, host_tensor(dy, Shape{R, C}));
        copy_out(tx.grad(), dx);
    });
}

// The train_mlp cross-entropy chain: loss and dL/dlogits via loss.backward().
int ref_ce_chain(const float* logits, const int64_t* labels, int64_t R, int64_t C, float* loss, float* dlogits) {
    return guarded([&] {
        Tensor tl = host_tensor(logits, Shape{R, C});
        tl.requires_grad(true);
        Tensor lab = Tensor::empty(Shape{R}, Dtype::Int64, Device::cpu());
        std::memcpy(lab.data(), labels, sizeof(int64_t) * R);
        Tensor l = chain_cross_entropy(tl, lab);
        loss[0] = static_cast<const float*>(l.data())[0];
        l.backward();
        copy_out(tl.grad(), dlogits);
    });
}

// nn::CrossEntropyLoss::forward (nn/CrossEntropyLoss.cpp:11-63): softmax,
// gather, clamp(1e-9), -log, mean.
int ref_ce_module(const float* logits, const int64_t* labels, int64_t R, int64_t C, float* loss) {
    return guarded([&] {
        Tensor lab = Tensor::empty(Shape{R}, Dtype::Int64, Device::cpu());
        std::memcpy(lab.data(), labels, sizeof(int64_t) * R);
        nn::CrossEntropyLoss ce;
        Tensor l = ce.forward(host_tensor(logits, Shape{R, C}), lab);
        loss[0] = static_cast<const float*>(l.data())[0];
    });
}

// Conv2dModule::forward with a given weight/bias (nn/Conv2dModule.cpp:104-154).
int ref_conv2d_fwd(const float* x, const float* w, const float* b, float* y, int64_t N, int64_t Cin, int64_t H,
                   int64_t W, int64_t Cout, int64_t k, int64_t stride, int64_t pad) {
    return guarded([&] {
        nn::Conv2dModule conv(static_cast<int>(Cin), static_cast<int>(Cout), static_cast<int>(k),
                              static_cast<int>(stride), static_cast<int>(pad));
        for (auto& np : conv.named_parameters()) {
            if (np.first == "weight") std::memcpy(np.second->data_.data(), w, sizeof(float) * Cout * Cin * k * k);
            if (np.first == "bias") std::memcpy(np.second->data_.data(), b, sizeof(float) * Cout);
        }
        copy_out(conv.forward(host_tensor(x, Shape{N, Cin, H, W})), y);
    });
}

// Config-1 training: Linear(784,256)-ReLU-Linear(256,128)-ReLU-Linear(128,10),
// the train_mlp chain loss, loss.backward(), then momentum SGD applied by a
// host loop in the documented order (v = v*mu + g; p = p - v*lr;
// nn/optim/SGD.cpp:50-54) since SGD::step throws for mu > 0.  Weights start
// from the reference init.  xs: [steps][B][784], ys: [steps][B].
int ref_mlp_train(const float* xs, const int64_t* ys, int64_t steps, int64_t B, float lr, float mu, float* losses,
                  const int32_t* dims, int64_t ndims, float* final_weights) {
    return guarded([&] {
        std::vector<std::shared_ptr<nn::Linear>> layers;
        for (int64_t l = 0; l + 1 < ndims; ++l)
            layers.push_back(std::make_shared<nn::Linear>(dims[l], dims[l + 1]));
        nn::ReLU relu;
        std::vector<Tensor*> params;
        for (auto& fc : layers)
            for (auto& np : fc->named_parameters())
                if (np.first == "weight") params.push_back(&np.second->data_);
        std::vector<std::vector<float>> vel;
        for (Tensor* p : params) vel.emplace_back(static_cast<size_t>(p->numel()), 0.0f);
        const int64_t in = dims[0];
        for (int64_t s = 0; s < steps; ++s) {
            Tensor x = host_tensor(xs + s * B * in, Shape{B, in});
            Tensor lab = Tensor::empty(Shape{B}, Dtype::Int64, Device::cpu());
            std::memcpy(lab.data(), ys + s * B, sizeof(int64_t) * B);
            Tensor h = x;
            for (size_t l = 0; l < layers.size(); ++l) {
                h = layers[l]->forward(h);
                if (l + 1 < layers.size()) h = relu.forward(h);
            }
            Tensor loss = chain_cross_entropy(h, lab);
            losses[s] = static_cast<const float*>(loss.data())[0];
            loss.backward();
            for (size_t i = 0; i < params.size(); ++i) {
                Tensor g = params[i]->grad();
                float* pp = static_cast<float*>(params[i]->data());
                const float* gp = static_cast<const float*>(g.data());
                float* vp = vel[i].data();
                for (int64_t k = 0; k < params[i]->numel(); ++k) {
                    float vm = vp[k] * mu;
                    vp[k] = vm + gp[k];
                    float step = vp[k] * lr;
                    pp[k] = pp[k] - step;
                }
            }
        }
        if (final_weights) {
            size_t off = 0;
            for (Tensor* p : params) {
                copy_out(*p, final_weights + off);
                off += static_cast<size_t>(p->numel());
            }
        }
    });
}

// ---------------------------------------------------------------------------
// Timed runs for bench.py's CPU baselines: each builds its inputs and graph
// outside the timed part, runs the reference's operation `reps` times and
// stores the mean wall seconds of the operation alone in *sec.
// ---------------------------------------------------------------------------
namespace {
double seconds_since(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}
}  // namespace

// LogSoftmaxBackward::apply on y = log_softmax(logits) with the chain's
// upstream gradient -onehot/N (autograd/ops/LogSoftmaxBackward.hpp:26-58).
int ref_time_log_softmax_bwd(const float* logits, const int64_t* labels, int64_t R, int64_t C, int32_t reps,
                             double* sec) {
    return guarded([&] {
        Tensor y = host_tensor(logits, Shape{R, C}).log_softmax(-1);
        Tensor gy = zeros(Shape{R, C}, Dtype::Float32, Device::cpu());
        float* gp = static_cast<float*>(gy.data());
        for (int64_t r = 0; r < R; ++r)
            if (labels[r] >= 0 && labels[r] < C) gp[r * C + labels[r]] = -1.0f / static_cast<float>(R);
        double t = 0.0;
        for (int32_t i = 0; i < reps; ++i) {
            LogSoftmaxBackward node(y);
            std::vector<Tensor> g{gy};
            auto t0 = std::chrono::steady_clock::now();
            Tensor gx = node.apply(std::move(g))[0];
            t += seconds_since(t0);
        }
        *sec = t / reps;
    });
}

// The whole backward of the train_mlp cross-entropy chain, loss.backward()
// (examples/train_mlp.cpp:54-76); the forward chain is rebuilt untimed for
// every repetition.
int ref_time_ce_chain_bwd(const float* logits, const int64_t* labels, int64_t R, int64_t C, int32_t reps, double* sec) {
    return guarded([&] {
        Tensor lab = Tensor::empty(Shape{R}, Dtype::Int64, Device::cpu());
        std::memcpy(lab.data(), labels, sizeof(int64_t) * R);
        double t = 0.0;
        for (int32_t i = 0; i < reps; ++i) {
            Tensor tl = host_tensor(logits, Shape{R, C});
            tl.requires_grad(true);
            Tensor l = chain_cross_entropy(tl, lab);
            auto t0 = std::chrono::steady_clock::now();
            l.backward();
            t += seconds_since(t0);
        }
        *sec = t / reps;
    });
}

// ReluBackward::apply (autograd/ops/ReluBackward.hpp:22-32).
int ref_time_relu_bwd(const float* dy, const float* x, int64_t n, int32_t reps, double* sec) {
    return guarded([&] {
        Tensor tx = host_tensor(x, Shape{n}), tdy = host_tensor(dy, Shape{n});
        double t = 0.0;
        for (int32_t i = 0; i < reps; ++i) {
            ReluBackward node(tx);
            std::vector<Tensor> g{tdy};
            auto t0 = std::chrono::steady_clock::now();
            Tensor dx = node.apply(std::move(g))[0];
            t += seconds_since(t0);
        }
        *sec = t / reps;
    });
}

// The backward of Tensor::layer_norm through the engine (its
// LayerNormBackward stub, autograd/ops/LayerNormBackward.hpp:33-60); the
// forward is rebuilt untimed for every repetition.
int ref_time_layernorm_bwd(const float* x, const float* g, const float* b, const float* dy, int64_t R, int64_t C,
                           float eps, int32_t reps, double* sec) {
    return guarded([&] {
        Tensor tg = host_tensor(g, Shape{C}), tb = host_tensor(b, Shape{C}), tdy = host_tensor(dy, Shape{R, C});
        double t = 0.0;
        for (int32_t i = 0; i < reps; ++i) {
            Tensor tx = host_tensor(x, Shape{R, C});
            tx.requires_grad(true);
            Tensor y = tx.layer_norm(tg, tb, eps);
            auto t0 = std::chrono::steady_clock::now();
            run_backward(y, tdy);
            t += seconds_since(t0);
        }
        *sec = t / reps;
    });
}

}  // extern "C"
