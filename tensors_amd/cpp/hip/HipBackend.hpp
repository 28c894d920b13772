// HIP backend of the C++ API: replaces the reference's DeviceContext
// (cuda/CudaContext.{hpp,cpp}), CudaStorageAllocator
// (cuda/memory/CudaStorageAllocator.cpp) and the kernel registrations
// (cuda/kernels/elementwise.cu:318-336).  Everything goes through the C ABI
// of libtf_hip (include/tf_hip.h); a failing call throws std::runtime_error
// carrying tf_last_error().
//
// The device-op wrappers below take Tensors, check shapes / dtypes / devices
// on the host and launch on the device's stream.  Operands must be
// contiguous; outputs are caller-allocated.
#pragma once

#include "tensor/CPUStorageAllocator.hpp"
#include "tensor/Tensor.hpp"

#include <functional>
#include <vector>

#include <cstddef>
#include <cstdint>

struct tf_ctx;
struct tf_graph;

namespace tensorforge::hip {

// The context of GPU `device` (created on first use; one stream and the
// device's memory pool).  Throws when no GPU is visible.
tf_ctx* context(int device = 0);
// Pool bytes reserved and in use on `device` (tf_hip_pool_stats).
void pool_stats(int device, uint64_t* reserved, uint64_t* used);
// Throws std::runtime_error("<what>: <tf_last_error()>") when status != 0.
void check(int status, const char* what);
// Registers the GPU allocator, copy callback and elementwise slots (idempotent;
// also runs when libtensorforge is loaded).
void register_backend();
// Blocks until the device's stream has drained.
void synchronize(int device = 0);
// Hands the device's cached blocks and the pool's unused memory back to the
// driver (tf_hip_trim with nothing kept); a no-op before the context exists.
void trim(int device = 0);
// Launch on a caller-owned hipStream_t from now on (nullptr: the context's own).
void set_stream(void* stream, int device = 0);

// ---- HIP graphs (tf_graph_*) ----------------------------------------------
// The device work that `record` enqueues on `device`, captured once and
// replayed with one launch.  Under capture the block cache serves every
// allocation (run the same work eagerly once first), and nothing may wait for
// the device or copy from / to the host.  Tensors created during the capture
// that outlive it must stay alive while the graph is replayed.
class CapturedGraph {
public:
    CapturedGraph() = default;
    CapturedGraph(tf_graph* g, int device) : g_(g), device_(device) {}
    ~CapturedGraph();
    CapturedGraph(const CapturedGraph&) = delete;
    CapturedGraph& operator=(const CapturedGraph&) = delete;
    CapturedGraph(CapturedGraph&& o) noexcept : g_(o.g_), device_(o.device_) { o.g_ = nullptr; }
    CapturedGraph& operator=(CapturedGraph&& o) noexcept;
    // Enqueues one replay on the device's stream.
    void launch() const;

private:
    tf_graph* g_ = nullptr;
    int device_ = 0;
};
CapturedGraph capture(const std::function<void()>& record, int device = 0);
// dst[0:bytes) = table[*counter % n][0:bytes) on the device (tf_gather_indexed).
void gather_indexed(void* dst, const uint64_t* table, int64_t n, const int64_t* counter, int64_t bytes,
                    int device = 0);
// ring[*counter] = *src, then ++*counter, on the device (tf_record_step).
void record_step(const float* src, float* ring, int64_t ring_len, int64_t* counter, int device = 0);

// ---- memory --------------------------------------------------------------
Storage allocate(size_t size_bytes, Device device, Dtype dtype);
void copy_bytes(void* dst, const void* src, size_t bytes, allocator_dispatch::CudaCopyKind kind, int device = 0);
void fill(Tensor& t, float value);
void zero(Tensor& t);

// ---- elementwise ---------------------------------------------------------
void add(const Tensor& a, const Tensor& b, Tensor& out);
void sub(const Tensor& a, const Tensor& b, Tensor& out);
void mul(const Tensor& a, const Tensor& b, Tensor& out);
void relu(const Tensor& x, Tensor& y);
void sigmoid(const Tensor& x, Tensor& y);
void tanh(const Tensor& x, Tensor& y);
void relu_backward(const Tensor& dy, const Tensor& x, Tensor& dx);
void sigmoid_backward(const Tensor& dy, const Tensor& y, Tensor& dx);
void tanh_backward(const Tensor& dy, const Tensor& y, Tensor& dx);
void cast(const Tensor& x, Tensor& y);  // Float32 <-> BFloat16

// ---- GEMM ----------------------------------------------------------------
// C (M x N) = epi(alpha * op(A) op(B) + beta * C) on 2-D row-major tensors;
// op(X) = X^T when the flag is set.  bias: Float32 [N] or nullptr.
void gemm(const Tensor& A, bool trans_a, const Tensor& B, bool trans_b, Tensor& C, float alpha = 1.0f,
          float beta = 0.0f, const Tensor* bias = nullptr, bool relu = false);
// C = (A * [mask > 0]) op(B), Float32, mask shaped as A (tf_gemm_relu_masked):
// a ReLU's backward folded into the product's left operand.  False (nothing
// launched) when the product does not fit the kernel that takes the mask.
bool gemm_relu_masked(const Tensor& A, bool trans_a, const Tensor& mask, const Tensor& B, bool trans_b, Tensor& C);
// Raw tf_gemm_ex on device pointers (conv layers).
void gemm_ex(int device, bool trans_a, bool trans_b, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
             int64_t stride_a, const void* B, int64_t ldb, int64_t stride_b, void* C, int64_t ldc, int64_t stride_c,
             int64_t batch, bool reduce_batch, Dtype in_dtype, Dtype out_dtype, int epilogue, const float* bias,
             float beta = 0.0f);

// ---- rows ----------------------------------------------------------------
void softmax(const Tensor& x, Tensor& y);
void log_softmax(const Tensor& x, Tensor& y);
void softmax_backward(const Tensor& y, const Tensor& dy, Tensor& dx);
void log_softmax_backward(const Tensor& y, const Tensor& dy, Tensor& dx);
// flags: TF_CE_* of tf_ce_fwd (TF_CE_MODULE for nn::CrossEntropyLoss).
void cross_entropy_forward(const Tensor& logits, const Tensor& targets, Tensor& loss, Tensor* lse, int flags);
void cross_entropy_backward(const Tensor& logits, const Tensor& targets, const Tensor* lse, const Tensor* grad_loss,
                            Tensor& dlogits);
// Loss and dlogits = (softmax - onehot) / N in one pass (tf_ce_fwd_bwd).
void cross_entropy_forward_backward(const Tensor& logits, const Tensor& targets, Tensor& loss, Tensor& dlogits,
                                    int flags);
// The same for BFloat16 logits: dlogits in BFloat16 (tf_ce_fwd_bwd_bf16).
void cross_entropy_forward_backward_bf16(const Tensor& logits, const Tensor& targets, Tensor& loss, Tensor& dlogits,
                                         int flags);
// out = x * s[0] for a device scalar s (tf_scale_by).
void scale_by(const Tensor& x, const Tensor& s, Tensor& out);
void layernorm_forward(const Tensor& x, const Tensor& gamma, const Tensor& beta, Tensor& y, Tensor& mean,
                       Tensor& rstd, float eps);
void layernorm_backward(const Tensor& dy, const Tensor& x, const Tensor& gamma, const Tensor& mean, const Tensor& rstd,
                        Tensor& dx, Tensor& dgamma, Tensor& dbeta, bool reference_compat);

// ---- reductions / layout ---------------------------------------------------
void sum_dim(const Tensor& x, Tensor& out, int64_t outer, int64_t reduce, int64_t inner);
void expand_dim(const Tensor& up, Tensor& out, int64_t outer, int64_t reduce, int64_t inner);
void transpose2d(const Tensor& x, Tensor& out, int64_t batch, int64_t rows, int64_t cols);
void colsum(const Tensor& dy, Tensor& db);
// dz = dy * (x > 0 ? 1 : 0) and db = the column sums of dz over the last
// dimension, in one pass (tf_relu_bwd_colsum); dy, x, dz share shape and dtype.
void relu_backward_colsum(const Tensor& dy, const Tensor& x, Tensor& dz, Tensor& db);
// The backward of a Linear layer with at most 16 outputs in one launch
// (tf_linear_bwd_narrow): dx = dy W, dw = dy^T x, db = column sums of dy,
// each written when its pointer is given.  False (nothing launched) when
// the shapes, dtypes or alignment do not fit that kernel.
bool linear_backward_narrow(const Tensor& dy, const Tensor& x, const Tensor& w, Tensor* dx, Tensor* dw, Tensor* db);
// dx = dz w and dw = dz^T x of a small Float32 Linear layer in one launch
// (tf_linear_bwd_small), dz = dy * (mask > 0) when mask is given.  False
// (nothing launched) when a product does not fit the small-product kernel.
bool linear_backward_small(const Tensor& dy, const Tensor* mask, const Tensor& x, const Tensor& w, Tensor& dx,
                           Tensor& dw);
void chansum_nchw(const Tensor& dy, Tensor& db);
// Implicit-GEMM convolution forward (tf_conv2d_fwd): false when the shape
// does not fit the kernel's LDS (nothing was launched), else y is written.
bool conv2d_forward_implicit(const Tensor& x, const Tensor& w, const Tensor* bias, Tensor& y, int64_t sh, int64_t sw,
                             int64_t ph, int64_t pw, int64_t dh, int64_t dw, bool relu);
// Implicit-GEMM weight gradient (tf_conv2d_bwd_weight): false when the shape
// does not fit the kernel's LDS (nothing was launched), else dw is written,
// and db (the bias gradient) too when it is not nullptr.  relu_y: dy is the
// gradient of a ReLU's output relu_y; the gradient used is
// dy * (relu_y > 0), which is also written to *dz_out when that is given
// (tf_conv2d_bwd_weight_relu).
bool conv2d_backward_weight_implicit(const Tensor& x, const Tensor& dy, Tensor& dw, Tensor* db, int64_t sh, int64_t sw,
                                     int64_t ph, int64_t pw, int64_t dh, int64_t dwl, const Tensor* relu_y = nullptr,
                                     Tensor* dz_out = nullptr);

// Implicit-GEMM data gradient (tf_conv2d_bwd_data): false when the shape does
// not fit the kernel's LDS (nothing was launched), else dx is written.
bool conv2d_backward_data_implicit(const Tensor& dy, const Tensor& w, Tensor& dx, int64_t sh, int64_t sw, int64_t ph,
                                   int64_t pw, int64_t dh, int64_t dwl);

// ---- conv index maps -----------------------------------------------------
void im2col(const Tensor& x, Tensor& col, int64_t kH, int64_t kW, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
            int64_t dh, int64_t dw);
void col2im(const Tensor& col, Tensor& dx, int64_t kH, int64_t kW, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
            int64_t dh, int64_t dw);

// ---- optimiser -----------------------------------------------------------
// Fused v = mu*v + g; p -= lr*v (mu == 0: p -= lr*g); shadow (BFloat16, may
// be nullptr) receives bf16(p).
void sgd_momentum(Tensor& p, const Tensor& g, Tensor* v, Tensor* shadow, float lr, float mu);
// The same update for several parameters, one launch per 32 parameters of
// one device (tf_sgd_momentum_multi).  v / shadow: nullptr or as above.
struct SgdItem {
    Tensor* p;
    Tensor g;
    Tensor* v;
    Tensor shadow;  // empty: none
};
void sgd_momentum_multi(std::vector<SgdItem>& items, float lr, float mu);

}  // namespace tensorforge::hip
