#include "hip/HipBackend.hpp"

#include "cuda/CudaKernelRegistry.hpp"
#include "tf_hip.h"

#include <atomic>
#include <cstdlib>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

namespace tensorforge::hip {

namespace {

constexpr int kMaxDevices = 16;
std::mutex g_ctx_mutex;
tf_ctx* g_ctx[kMaxDevices] = {};
// Set at process exit: storages destroyed after it must not call into a
// runtime that may already be torn down.
std::atomic<bool> g_exiting{false};

int tf_code(Dtype d) { return static_cast<int>(d); }  // TF_* codes equal Dtype values

void require(bool cond, const std::string& msg) {
    if (!cond) throw std::invalid_argument(msg);
}

void require_gpu(const Tensor& t, const char* what) {
    require(t.device().type == DeviceType::CUDA, std::string(what) + ": tensor is not on the GPU");
    require(t.data() != nullptr || t.numel() == 0, std::string(what) + ": tensor has no storage");
}

void require_contig(const Tensor& t, const char* what) {
    require(t.stride() == Stride::compute_row_major(t.shape()), std::string(what) + ": tensor must be contiguous");
}

tf_ctx* ctx_of(const Tensor& t) { return context(t.device().index); }

// Elements a tensor's storage holds: a 0-d tensor holds one value.
int64_t slots(const Tensor& t) { return t.shape().ndim() == 0 ? 1 : t.numel(); }

void release_gpu(void* data, Device device) {
    if (g_exiting.load()) return;
    tf_ctx* c = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_ctx_mutex);
        c = g_ctx[device.index];
    }
    if (c) (void)tf_hip_free(c, data);
}

Storage gpu_allocate_dispatch(size_t bytes, Device device, Dtype dtype) { return allocate(bytes, device, dtype); }
void gpu_free_dispatch(Storage storage) {
    if (storage && storage->data()) {
        release_gpu(storage->data(), storage->device());
        storage->release();
    }
}
void copy_dispatch(void* dst, const void* src, size_t bytes, allocator_dispatch::CudaCopyKind kind) {
    copy_bytes(dst, src, bytes, kind, 0);
}

// Elementwise launchers in the reference's slot signatures.
void slot_add(const void* a, const void* b, void* o, int64_t n, Dtype d, void*) {
    check(tf_add(context(0), a, b, o, n, tf_code(d)), "add");
}
void slot_mul(const void* a, const void* b, void* o, int64_t n, Dtype d, void*) {
    check(tf_mul(context(0), a, b, o, n, tf_code(d)), "mul");
}
void slot_relu(const void* x, void* y, int64_t n, Dtype d, void*) { check(tf_relu_fwd(context(0), x, y, n, tf_code(d)), "relu"); }
void slot_sigmoid(const void* x, void* y, int64_t n, Dtype d, void*) {
    check(tf_sigmoid_fwd(context(0), x, y, n, tf_code(d)), "sigmoid");
}
void slot_tanh(const void* x, void* y, int64_t n, Dtype d, void*) { check(tf_tanh_fwd(context(0), x, y, n, tf_code(d)), "tanh"); }
void slot_leaky_relu(const void* x, void* y, int64_t n, Dtype d, float alpha, void*) {
    check(tf_leaky_relu_fwd(context(0), x, y, n, alpha, tf_code(d)), "leaky_relu");
}

struct AutoRegister {
    AutoRegister() { register_backend(); }
} g_auto_register;

}  // namespace

void check(int status, const char* what) {
    if (status != TF_OK) throw std::runtime_error(std::string(what) + ": " + tf_last_error());
}

tf_ctx* context(int device) {
    require(device >= 0 && device < kMaxDevices, "hip::context: device index out of range");
    std::lock_guard<std::mutex> lock(g_ctx_mutex);
    if (!g_ctx[device]) {
        tf_ctx* c = nullptr;
        check(tf_hip_init(device, &c), "hip::context");
        g_ctx[device] = c;
        static bool hooked = false;
        if (!hooked) {
            hooked = true;
            std::atexit([] { g_exiting.store(true); });
        }
    }
    return g_ctx[device];
}

void register_backend() {
    static std::once_flag once;
    std::call_once(once, [] {
        allocator_dispatch::register_allocator(DeviceType::CUDA, gpu_allocate_dispatch, gpu_free_dispatch);
        allocator_dispatch::register_cuda_copy(copy_dispatch);
        register_cuda_add(slot_add);
        register_cuda_mul(slot_mul);
        register_cuda_relu(slot_relu);
        register_cuda_sigmoid(slot_sigmoid);
        register_cuda_tanh(slot_tanh);
        register_cuda_leaky_relu(slot_leaky_relu);
    });
}

void synchronize(int device) { check(tf_hip_sync(context(device)), "hip::synchronize"); }

void trim(int device) {
    tf_ctx* c = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_ctx_mutex);
        if (device >= 0 && device < kMaxDevices) c = g_ctx[device];
    }
    if (c) check(tf_hip_trim(c, 0), "hip::trim");
}

void pool_stats(int device, uint64_t* reserved, uint64_t* used) {
    check(tf_hip_pool_stats(context(device), reserved, used), "hip::pool_stats");
}

void set_stream(void* stream, int device) { check(tf_hip_set_stream(context(device), stream), "hip::set_stream"); }

CapturedGraph::~CapturedGraph() {
    if (g_) (void)tf_graph_destroy(g_);
}

CapturedGraph& CapturedGraph::operator=(CapturedGraph&& o) noexcept {
    if (this != &o) {
        if (g_) (void)tf_graph_destroy(g_);
        g_ = o.g_;
        device_ = o.device_;
        o.g_ = nullptr;
    }
    return *this;
}

void CapturedGraph::launch() const {
    if (g_ == nullptr) throw std::logic_error("hip::CapturedGraph::launch: empty graph");
    check(tf_graph_launch(context(device_), g_), "hip::CapturedGraph::launch");
}

CapturedGraph capture(const std::function<void()>& record, int device) {
    tf_ctx* ctx = context(device);
    check(tf_graph_begin(ctx), "hip::capture");
    try {
        record();
    } catch (...) {
        // End the capture (its graph, if any, is dropped) and report the
        // failing call's own error.
        tf_graph* g = nullptr;
        if (tf_graph_end(ctx, &g) == TF_OK && g) (void)tf_graph_destroy(g);
        throw;
    }
    tf_graph* g = nullptr;
    check(tf_graph_end(ctx, &g), "hip::capture");
    return CapturedGraph(g, device);
}

void gather_indexed(void* dst, const uint64_t* table, int64_t n, const int64_t* counter, int64_t bytes, int device) {
    check(tf_gather_indexed(context(device), dst, table, n, counter, bytes), "hip::gather_indexed");
}

void record_step(const float* src, float* ring, int64_t ring_len, int64_t* counter, int device) {
    check(tf_record_step(context(device), src, ring, ring_len, counter), "hip::record_step");
}

Storage allocate(size_t size_bytes, Device device, Dtype dtype) {
    require(device.type == DeviceType::CUDA, "hip::allocate: not a GPU device");
    void* p = nullptr;
    check(tf_hip_alloc(context(device.index), size_bytes, &p), "hip::allocate");
    return std::make_shared<StorageImpl>(p, size_bytes, device, dtype, &release_gpu);
}

void copy_bytes(void* dst, const void* src, size_t bytes, allocator_dispatch::CudaCopyKind kind, int device) {
    check(tf_hip_memcpy(context(device), dst, src, bytes, static_cast<int>(kind)), "hip::copy");
}

void fill(Tensor& t, float value) {
    require_gpu(t, "hip::fill");
    require(t.dtype() == Dtype::Float32, "hip::fill: Float32 only");
    check(tf_hip_fill_f32(ctx_of(t), static_cast<float*>(t.data()), value, t.numel()), "hip::fill");
}

void zero(Tensor& t) {
    require_gpu(t, "hip::zero");
    check(tf_hip_zero(ctx_of(t), t.data(), static_cast<size_t>(t.numel()) * dtype_size(t.dtype())), "hip::zero");
}

namespace {
void check_same(const Tensor& a, const Tensor& b, const char* what) {
    require(a.numel() == b.numel(), std::string(what) + ": element count mismatch");
    require(a.dtype() == b.dtype(), std::string(what) + ": dtype mismatch");
}
}  // namespace

#define TF_BINARY(NAME, FN)                                                                          \
    void NAME(const Tensor& a, const Tensor& b, Tensor& out) {                                       \
        require_gpu(a, #NAME); require_gpu(b, #NAME); require_gpu(out, #NAME);                        \
        check_same(a, b, #NAME); check_same(a, out, #NAME);                                           \
        check(FN(ctx_of(a), a.data(), b.data(), out.data(), a.numel(), tf_code(a.dtype())), #NAME);   \
    }
TF_BINARY(add, tf_add)
TF_BINARY(sub, tf_sub)
TF_BINARY(mul, tf_mul)
TF_BINARY(relu_backward, tf_relu_bwd)
TF_BINARY(sigmoid_backward, tf_sigmoid_bwd)
TF_BINARY(tanh_backward, tf_tanh_bwd)
#undef TF_BINARY

#define TF_UNARY(NAME, FN)                                                                     \
    void NAME(const Tensor& x, Tensor& y) {                                                    \
        require_gpu(x, #NAME); require_gpu(y, #NAME); check_same(x, y, #NAME);                  \
        check(FN(ctx_of(x), x.data(), y.data(), x.numel(), tf_code(x.dtype())), #NAME);         \
    }
TF_UNARY(relu, tf_relu_fwd)
TF_UNARY(sigmoid, tf_sigmoid_fwd)
TF_UNARY(tanh, tf_tanh_fwd)
#undef TF_UNARY

void cast(const Tensor& x, Tensor& y) {
    require_gpu(x, "hip::cast");
    require_gpu(y, "hip::cast");
    require(x.numel() == y.numel(), "hip::cast: element count mismatch");
    if (x.dtype() == Dtype::Float32 && y.dtype() == Dtype::BFloat16) {
        check(tf_cast_f32_bf16(ctx_of(x), static_cast<const float*>(x.data()), y.data(), x.numel()), "hip::cast");
    } else if (x.dtype() == Dtype::BFloat16 && y.dtype() == Dtype::Float32) {
        check(tf_cast_bf16_f32(ctx_of(x), x.data(), static_cast<float*>(y.data()), x.numel()), "hip::cast");
    } else if (x.dtype() == y.dtype()) {
        copy_bytes(y.data(), x.data(), static_cast<size_t>(x.numel()) * dtype_size(x.dtype()),
                   allocator_dispatch::CudaCopyKind::DeviceToDevice, x.device().index);
    } else {
        throw std::invalid_argument("hip::cast: only Float32 <-> BFloat16 conversions are implemented");
    }
}

void gemm(const Tensor& A, bool trans_a, const Tensor& B, bool trans_b, Tensor& C, float alpha, float beta,
          const Tensor* bias, bool relu) {
    require_gpu(A, "hip::gemm");
    require_gpu(B, "hip::gemm");
    require_gpu(C, "hip::gemm");
    require(A.shape().ndim() == 2 && B.shape().ndim() == 2 && C.shape().ndim() == 2, "hip::gemm: 2-D tensors only");
    require_contig(A, "hip::gemm A");
    require_contig(B, "hip::gemm B");
    require_contig(C, "hip::gemm C");
    require(A.dtype() == B.dtype(), "hip::gemm: A and B dtypes differ");
    const int64_t M = trans_a ? A.shape()[1] : A.shape()[0];
    const int64_t K = trans_a ? A.shape()[0] : A.shape()[1];
    const int64_t Kb = trans_b ? B.shape()[1] : B.shape()[0];
    const int64_t N = trans_b ? B.shape()[0] : B.shape()[1];
    require(K == Kb, "hip::gemm: inner dimensions differ");
    require(C.shape()[0] == M && C.shape()[1] == N, "hip::gemm: output shape mismatch");
    int epi = TF_EPI_NONE;
    if (bias) {
        require_gpu(*bias, "hip::gemm bias");
        require(bias->dtype() == Dtype::Float32 && bias->numel() == N, "hip::gemm: bias must be Float32 [N]");
        epi = relu ? TF_EPI_BIAS_RELU : TF_EPI_BIAS;
    } else if (relu) {
        epi = TF_EPI_RELU;
    }
    check(tf_gemm(ctx_of(A), trans_a, trans_b, M, N, K, alpha, A.data(), A.shape()[1], B.data(), B.shape()[1], beta,
                  C.data(), C.shape()[1], tf_code(A.dtype()), tf_code(C.dtype()), epi,
                  bias ? static_cast<const float*>(bias->data()) : nullptr),
          "hip::gemm");
}

bool gemm_relu_masked(const Tensor& A, bool trans_a, const Tensor& mask, const Tensor& B, bool trans_b, Tensor& C) {
    const auto f32 = [](const Tensor& t) {
        return t.device().type == DeviceType::CUDA && t.dtype() == Dtype::Float32 && t.shape().ndim() == 2 &&
               t.stride() == Stride::compute_row_major(t.shape());
    };
    if (!f32(A) || !f32(mask) || !f32(B) || !f32(C) || mask.shape() != A.shape()) return false;
    if (mask.device() != A.device() || B.device() != A.device() || C.device() != A.device()) return false;
    const int64_t M = trans_a ? A.shape()[1] : A.shape()[0];
    const int64_t K = trans_a ? A.shape()[0] : A.shape()[1];
    const int64_t N = trans_b ? B.shape()[0] : B.shape()[1];
    require((trans_b ? B.shape()[1] : B.shape()[0]) == K, "hip::gemm_relu_masked: inner dimensions differ");
    require(C.shape()[0] == M && C.shape()[1] == N, "hip::gemm_relu_masked: output shape mismatch");
    const int st = tf_gemm_relu_masked(ctx_of(A), trans_a, trans_b, M, N, K, static_cast<const float*>(A.data()),
                                       A.shape()[1], static_cast<const float*>(mask.data()),
                                       static_cast<const float*>(B.data()), B.shape()[1], static_cast<float*>(C.data()),
                                       C.shape()[1]);
    if (st == TF_ERR_UNSUPPORTED) return false;
    check(st, "hip::gemm_relu_masked");
    return true;
}

void gemm_ex(int device, bool trans_a, bool trans_b, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
             int64_t stride_a, const void* B, int64_t ldb, int64_t stride_b, void* C, int64_t ldc, int64_t stride_c,
             int64_t batch, bool reduce_batch, Dtype in_dtype, Dtype out_dtype, int epilogue, const float* bias,
             float beta) {
    check(tf_gemm_ex(context(device), trans_a, trans_b, M, N, K, 1.0f, A, lda, stride_a, B, ldb, stride_b, beta, C,
                     ldc, stride_c, batch, reduce_batch, tf_code(in_dtype), tf_code(out_dtype), epilogue, bias),
          "hip::gemm_ex");
}

namespace {
// [rows, cols] view of a contiguous tensor (cols = last dimension), any dtype.
void rows_cols_any(const Tensor& t, int64_t& rows, int64_t& cols, const char* what) {
    require(t.shape().ndim() >= 1, std::string(what) + ": needs at least 1-D");
    require_contig(t, what);
    cols = t.shape()[t.shape().ndim() - 1];
    rows = cols ? t.numel() / cols : 0;
}

void rows_cols(const Tensor& t, int64_t& rows, int64_t& cols, const char* what) {
    require(t.dtype() == Dtype::Float32, std::string(what) + ": Float32 only");
    rows_cols_any(t, rows, cols, what);
}
}  // namespace

void softmax(const Tensor& x, Tensor& y) {
    require_gpu(x, "hip::softmax"); require_gpu(y, "hip::softmax"); check_same(x, y, "hip::softmax");
    int64_t r, c; rows_cols(x, r, c, "hip::softmax");
    check(tf_softmax_fwd(ctx_of(x), static_cast<const float*>(x.data()), static_cast<float*>(y.data()), r, c), "hip::softmax");
}

void log_softmax(const Tensor& x, Tensor& y) {
    require_gpu(x, "hip::log_softmax"); require_gpu(y, "hip::log_softmax"); check_same(x, y, "hip::log_softmax");
    int64_t r, c; rows_cols(x, r, c, "hip::log_softmax");
    check(tf_log_softmax_fwd(ctx_of(x), static_cast<const float*>(x.data()), static_cast<float*>(y.data()), r, c),
          "hip::log_softmax");
}

void softmax_backward(const Tensor& y, const Tensor& dy, Tensor& dx) {
    require_gpu(y, "hip::softmax_backward"); check_same(y, dy, "hip::softmax_backward"); check_same(y, dx, "hip::softmax_backward");
    int64_t r, c; rows_cols(y, r, c, "hip::softmax_backward");
    check(tf_softmax_bwd(ctx_of(y), static_cast<const float*>(y.data()), static_cast<const float*>(dy.data()),
                         static_cast<float*>(dx.data()), r, c), "hip::softmax_backward");
}

void log_softmax_backward(const Tensor& y, const Tensor& dy, Tensor& dx) {
    require_gpu(y, "hip::log_softmax_backward"); check_same(y, dy, "hip::log_softmax_backward");
    check_same(y, dx, "hip::log_softmax_backward");
    int64_t r, c; rows_cols(y, r, c, "hip::log_softmax_backward");
    check(tf_log_softmax_bwd(ctx_of(y), static_cast<const float*>(y.data()), static_cast<const float*>(dy.data()),
                             static_cast<float*>(dx.data()), r, c), "hip::log_softmax_backward");
}

void cross_entropy_forward(const Tensor& logits, const Tensor& targets, Tensor& loss, Tensor* lse, int flags) {
    require_gpu(logits, "hip::cross_entropy"); require_gpu(targets, "hip::cross_entropy"); require_gpu(loss, "hip::cross_entropy");
    require(logits.shape().ndim() == 2, "hip::cross_entropy: logits must be 2-D");
    int64_t r, c; rows_cols(logits, r, c, "hip::cross_entropy");
    require(targets.dtype() == Dtype::Int64 && targets.numel() == r, "hip::cross_entropy: targets must be Int64 [N]");
    require(loss.dtype() == Dtype::Float32 && loss.numel() >= 1, "hip::cross_entropy: loss must be Float32");
    if (lse) require(lse->numel() == r && lse->dtype() == Dtype::Float32, "hip::cross_entropy: lse must be Float32 [N]");
    check(tf_ce_fwd(ctx_of(logits), static_cast<const float*>(logits.data()), static_cast<const int64_t*>(targets.data()),
                    static_cast<float*>(loss.data()), lse ? static_cast<float*>(lse->data()) : nullptr, r, c, flags),
          "hip::cross_entropy");
}

void cross_entropy_backward(const Tensor& logits, const Tensor& targets, const Tensor* lse, const Tensor* grad_loss,
                            Tensor& dlogits) {
    require_gpu(logits, "hip::cross_entropy_backward"); check_same(logits, dlogits, "hip::cross_entropy_backward");
    int64_t r, c; rows_cols(logits, r, c, "hip::cross_entropy_backward");
    require(targets.dtype() == Dtype::Int64 && targets.numel() == r, "hip::cross_entropy_backward: targets");
    if (grad_loss) require_gpu(*grad_loss, "hip::cross_entropy_backward grad");
    check(tf_ce_bwd(ctx_of(logits), static_cast<const float*>(logits.data()), static_cast<const int64_t*>(targets.data()),
                    lse ? static_cast<const float*>(lse->data()) : nullptr,
                    grad_loss ? static_cast<const float*>(grad_loss->data()) : nullptr,
                    static_cast<float*>(dlogits.data()), r, c),
          "hip::cross_entropy_backward");
}

void cross_entropy_forward_backward(const Tensor& logits, const Tensor& targets, Tensor& loss, Tensor& dlogits,
                                    int flags) {
    require_gpu(logits, "hip::cross_entropy_forward_backward"); require_gpu(targets, "hip::cross_entropy_forward_backward");
    require_gpu(loss, "hip::cross_entropy_forward_backward");
    check_same(logits, dlogits, "hip::cross_entropy_forward_backward");
    int64_t r, c; rows_cols(logits, r, c, "hip::cross_entropy_forward_backward");
    require(targets.dtype() == Dtype::Int64 && targets.numel() == r, "hip::cross_entropy_forward_backward: targets");
    require(loss.dtype() == Dtype::Float32 && loss.numel() >= 1, "hip::cross_entropy_forward_backward: loss");
    check(tf_ce_fwd_bwd(ctx_of(logits), static_cast<const float*>(logits.data()),
                        static_cast<const int64_t*>(targets.data()), static_cast<float*>(loss.data()),
                        static_cast<float*>(dlogits.data()), r, c, flags),
          "hip::cross_entropy_forward_backward");
}

void cross_entropy_forward_backward_bf16(const Tensor& logits, const Tensor& targets, Tensor& loss, Tensor& dlogits,
                                         int flags) {
    const char* what = "hip::cross_entropy_forward_backward_bf16";
    require_gpu(logits, what); require_gpu(targets, what); require_gpu(loss, what);
    check_same(logits, dlogits, what);
    require(logits.dtype() == Dtype::BFloat16, std::string(what) + ": BFloat16 logits");
    int64_t r, c; rows_cols_any(logits, r, c, what);
    require(logits.shape().ndim() == 2, std::string(what) + ": 2-D logits");
    require(targets.dtype() == Dtype::Int64 && targets.numel() == r, std::string(what) + ": targets");
    require(loss.dtype() == Dtype::Float32 && loss.numel() >= 1, std::string(what) + ": loss");
    check(tf_ce_fwd_bwd_bf16(ctx_of(logits), logits.data(), static_cast<const int64_t*>(targets.data()),
                             static_cast<float*>(loss.data()), dlogits.data(), r, c, flags),
          what);
}

void scale_by(const Tensor& x, const Tensor& s, Tensor& out) {
    require_gpu(x, "hip::scale_by"); require_gpu(s, "hip::scale_by");
    check_same(x, out, "hip::scale_by");
    require(s.dtype() == Dtype::Float32 && s.numel() >= 1, "hip::scale_by: the scale must be Float32");
    check(tf_scale_by(ctx_of(x), x.data(), static_cast<const float*>(s.data()), out.data(), x.numel(),
                      static_cast<int>(x.dtype())),
          "hip::scale_by");
}

void layernorm_forward(const Tensor& x, const Tensor& gamma, const Tensor& beta, Tensor& y, Tensor& mean,
                       Tensor& rstd, float eps) {
    require_gpu(x, "hip::layer_norm"); check_same(x, y, "hip::layer_norm");
    int64_t r, c; rows_cols(x, r, c, "hip::layer_norm");
    require(gamma.numel() == c && beta.numel() == c && mean.numel() == r && rstd.numel() == r,
            "hip::layer_norm: parameter sizes");
    check(tf_layernorm_fwd(ctx_of(x), static_cast<const float*>(x.data()), static_cast<const float*>(gamma.data()),
                           static_cast<const float*>(beta.data()), static_cast<float*>(y.data()),
                           static_cast<float*>(mean.data()), static_cast<float*>(rstd.data()), r, c, eps),
          "hip::layer_norm");
}

void layernorm_backward(const Tensor& dy, const Tensor& x, const Tensor& gamma, const Tensor& mean, const Tensor& rstd,
                        Tensor& dx, Tensor& dgamma, Tensor& dbeta, bool reference_compat) {
    require_gpu(dy, "hip::layer_norm_backward"); check_same(dy, dx, "hip::layer_norm_backward");
    int64_t r, c; rows_cols(dy, r, c, "hip::layer_norm_backward");
    require(gamma.numel() == c && dgamma.numel() == c && dbeta.numel() == c, "hip::layer_norm_backward: sizes");
    check(tf_layernorm_bwd(ctx_of(dy), static_cast<const float*>(dy.data()), static_cast<const float*>(x.data()),
                           static_cast<const float*>(gamma.data()), static_cast<const float*>(mean.data()),
                           static_cast<const float*>(rstd.data()), static_cast<float*>(dx.data()),
                           static_cast<float*>(dgamma.data()), static_cast<float*>(dbeta.data()), r, c,
                           reference_compat ? 1 : 0),
          "hip::layer_norm_backward");
}

void sum_dim(const Tensor& x, Tensor& out, int64_t outer, int64_t reduce, int64_t inner) {
    require_gpu(x, "hip::sum"); require_gpu(out, "hip::sum");
    require(slots(x) == outer * reduce * inner && slots(out) == outer * inner, "hip::sum: extents");
    require(x.dtype() == Dtype::Float32, "hip::sum: Float32 only");
    check(tf_sum_dim(ctx_of(x), static_cast<const float*>(x.data()), static_cast<float*>(out.data()), outer, reduce, inner),
          "hip::sum");
}

void expand_dim(const Tensor& up, Tensor& out, int64_t outer, int64_t reduce, int64_t inner) {
    require_gpu(up, "hip::expand"); require_gpu(out, "hip::expand");
    require(slots(up) == outer * inner && slots(out) == outer * reduce * inner, "hip::expand: extents");
    check(tf_expand_dim(ctx_of(up), static_cast<const float*>(up.data()), static_cast<float*>(out.data()), outer,
                        reduce, inner),
          "hip::expand");
}

void transpose2d(const Tensor& x, Tensor& out, int64_t batch, int64_t rows, int64_t cols) {
    require_gpu(x, "hip::transpose"); require_gpu(out, "hip::transpose");
    require(x.numel() == batch * rows * cols && out.numel() == x.numel(), "hip::transpose: extents");
    check(tf_transpose2d(ctx_of(x), x.data(), out.data(), batch, rows, cols, tf_code(x.dtype())), "hip::transpose");
}

void colsum(const Tensor& dy, Tensor& db) {
    require_gpu(dy, "hip::colsum");
    int64_t r, c; rows_cols_any(dy, r, c, "hip::colsum");
    require(db.numel() == c && db.dtype() == Dtype::Float32, "hip::colsum: db size");
    if (dy.dtype() == Dtype::BFloat16) {
        check(tf_colsum_bf16(ctx_of(dy), dy.data(), static_cast<float*>(db.data()), r, c), "hip::colsum");
        return;
    }
    require(dy.dtype() == Dtype::Float32, "hip::colsum: dy must be Float32 or BFloat16");
    check(tf_colsum(ctx_of(dy), static_cast<const float*>(dy.data()), static_cast<float*>(db.data()), r, c), "hip::colsum");
}

void relu_backward_colsum(const Tensor& dy, const Tensor& x, Tensor& dz, Tensor& db) {
    const char* what = "hip::relu_backward_colsum";
    require_gpu(dy, what); require_gpu(x, what); require_gpu(dz, what); require_gpu(db, what);
    check_same(dy, x, what); check_same(dy, dz, what);
    require(dy.shape() == x.shape() && dy.shape() == dz.shape(), std::string(what) + ": shape mismatch");
    require_contig(x, what); require_contig(dz, what);
    int64_t r, c; rows_cols_any(dy, r, c, what);
    require(db.numel() == c && db.dtype() == Dtype::Float32, std::string(what) + ": db size");
    check(tf_relu_bwd_colsum(ctx_of(dy), dy.data(), x.data(), dz.data(), static_cast<float*>(db.data()), r, c,
                             tf_code(dy.dtype())), what);
}

bool linear_backward_narrow(const Tensor& dy, const Tensor& x, const Tensor& w, Tensor* dx, Tensor* dw, Tensor* db) {
    const auto f32 = [](const Tensor& t) {
        return t.device().type == DeviceType::CUDA && t.dtype() == Dtype::Float32 && t.shape().ndim() == 2 &&
               t.stride() == Stride::compute_row_major(t.shape());
    };
    if (!f32(dy) || !f32(w) || (dw && !f32(x))) return false;
    const int64_t M = dy.shape()[0], N = dy.shape()[1], K = w.shape()[1];
    if (w.shape()[0] != N || N > 16 || K % 4 != 0 || K < 64) return false;
    if (dw && (x.shape()[0] != M || x.shape()[1] != K)) return false;
    const auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    if (!a16(w.data()) || (dw && !a16(x.data()))) return false;
    if (dx) *dx = Tensor::empty(Shape{M, K}, Dtype::Float32, dy.device());
    if (dw) *dw = Tensor::empty(Shape{N, K}, Dtype::Float32, dy.device());
    if (db) *db = Tensor::empty(Shape{N}, Dtype::Float32, dy.device());
    check(tf_linear_bwd_narrow(ctx_of(dy), static_cast<const float*>(dy.data()),
                               dw ? static_cast<const float*>(x.data()) : nullptr, static_cast<const float*>(w.data()),
                               dx ? static_cast<float*>(dx->data()) : nullptr, dw ? static_cast<float*>(dw->data()) : nullptr,
                               db ? static_cast<float*>(db->data()) : nullptr, M, N, K),
          "hip::linear_backward_narrow");
    return true;
}

bool linear_backward_small(const Tensor& dy, const Tensor* mask, const Tensor& x, const Tensor& w, Tensor& dx,
                           Tensor& dw) {
    const auto f32 = [](const Tensor& t) {
        return t.device().type == DeviceType::CUDA && t.dtype() == Dtype::Float32 && t.shape().ndim() == 2 &&
               t.stride() == Stride::compute_row_major(t.shape());
    };
    if (!f32(dy) || !f32(x) || !f32(w) || (mask && (!f32(*mask) || mask->shape() != dy.shape()))) return false;
    const int64_t M = dy.shape()[0], N = dy.shape()[1], K = w.shape()[1];
    if (M == 0 || N == 0 || K == 0 || w.shape()[0] != N || x.shape()[0] != M || x.shape()[1] != K) return false;
    if (x.device() != dy.device() || w.device() != dy.device() || (mask && mask->device() != dy.device())) return false;
    Tensor tdx = Tensor::empty(Shape{M, K}, Dtype::Float32, dy.device());
    Tensor tdw = Tensor::empty(Shape{N, K}, Dtype::Float32, dy.device());
    const int st = tf_linear_bwd_small(ctx_of(dy), static_cast<const float*>(dy.data()),
                                       mask ? static_cast<const float*>(mask->data()) : nullptr,
                                       static_cast<const float*>(x.data()), static_cast<const float*>(w.data()),
                                       static_cast<float*>(tdx.data()), static_cast<float*>(tdw.data()), M, N, K);
    if (st == TF_ERR_UNSUPPORTED) return false;
    check(st, "hip::linear_backward_small");
    dx = std::move(tdx);
    dw = std::move(tdw);
    return true;
}

bool conv2d_forward_implicit(const Tensor& x, const Tensor& w, const Tensor* bias, Tensor& y, int64_t sh, int64_t sw,
                             int64_t ph, int64_t pw, int64_t dh, int64_t dw, bool relu) {
    require_gpu(x, "hip::conv2d_forward"); require_gpu(w, "hip::conv2d_forward"); require_gpu(y, "hip::conv2d_forward");
    require(x.dtype() == Dtype::Float32 && w.dtype() == Dtype::Float32 && y.dtype() == Dtype::Float32,
            "hip::conv2d_forward: Float32 only");
    const auto& xs = x.shape();
    const auto& ws = w.shape();
    const int st = tf_conv2d_fwd(ctx_of(x), static_cast<const float*>(x.data()), static_cast<const float*>(w.data()),
                                 bias ? static_cast<const float*>(bias->data()) : nullptr, static_cast<float*>(y.data()),
                                 xs[0], xs[1], xs[2], xs[3], ws[0], ws[2], ws[3], sh, sw, ph, pw, dh, dw, relu ? 1 : 0);
    if (st == TF_ERR_UNSUPPORTED) return false;
    check(st, "hip::conv2d_forward");
    return true;
}

bool conv2d_backward_weight_implicit(const Tensor& x, const Tensor& dy, Tensor& dw, Tensor* db, int64_t sh, int64_t sw,
                                     int64_t ph, int64_t pw, int64_t dh, int64_t dwl, const Tensor* relu_y,
                                     Tensor* dz_out) {
    require_gpu(x, "hip::conv2d_backward_weight"); require_gpu(dy, "hip::conv2d_backward_weight");
    require_gpu(dw, "hip::conv2d_backward_weight");
    require(x.dtype() == Dtype::Float32 && dy.dtype() == Dtype::Float32 && dw.dtype() == Dtype::Float32,
            "hip::conv2d_backward_weight: Float32 only");
    const auto& xs = x.shape();
    const auto& ws = dw.shape();
    if (db) {
        require_gpu(*db, "hip::conv2d_backward_weight");
        require(db->dtype() == Dtype::Float32 && db->numel() == ws[0], "hip::conv2d_backward_weight: db size");
    }
    float* dbp = db ? static_cast<float*>(db->data()) : nullptr;
    int st;
    if (relu_y) {
        require_gpu(*relu_y, "hip::conv2d_backward_weight");
        require(relu_y->dtype() == Dtype::Float32 && relu_y->shape() == dy.shape(),
                "hip::conv2d_backward_weight: ReLU output must match dy");
        require_contig(*relu_y, "hip::conv2d_backward_weight");
        float* dzp = nullptr;
        if (dz_out) {
            require_gpu(*dz_out, "hip::conv2d_backward_weight");
            require(dz_out->dtype() == Dtype::Float32 && dz_out->shape() == dy.shape(),
                    "hip::conv2d_backward_weight: masked-gradient output must match dy");
            require_contig(*dz_out, "hip::conv2d_backward_weight");
            dzp = static_cast<float*>(dz_out->data());
        }
        st = tf_conv2d_bwd_weight_relu(ctx_of(x), static_cast<const float*>(x.data()),
                                       static_cast<const float*>(dy.data()), static_cast<const float*>(relu_y->data()),
                                       dzp, static_cast<float*>(dw.data()), dbp, xs[0], xs[1], xs[2], xs[3], ws[0],
                                       ws[2], ws[3], sh, sw, ph, pw, dh, dwl);
    } else {
        st = tf_conv2d_bwd_weight(ctx_of(x), static_cast<const float*>(x.data()), static_cast<const float*>(dy.data()),
                                  static_cast<float*>(dw.data()), dbp, xs[0], xs[1], xs[2], xs[3], ws[0], ws[2], ws[3],
                                  sh, sw, ph, pw, dh, dwl);
    }
    if (st == TF_ERR_UNSUPPORTED) return false;
    check(st, "hip::conv2d_backward_weight");
    return true;
}

bool conv2d_backward_data_implicit(const Tensor& dy, const Tensor& w, Tensor& dx, int64_t sh, int64_t sw, int64_t ph,
                                   int64_t pw, int64_t dh, int64_t dwl) {
    require_gpu(dy, "hip::conv2d_backward_data"); require_gpu(w, "hip::conv2d_backward_data");
    require_gpu(dx, "hip::conv2d_backward_data");
    require(dy.dtype() == Dtype::Float32 && w.dtype() == Dtype::Float32 && dx.dtype() == Dtype::Float32,
            "hip::conv2d_backward_data: Float32 only");
    const auto& xs = dx.shape();
    const auto& ws = w.shape();
    const int st = tf_conv2d_bwd_data(ctx_of(dy), static_cast<const float*>(dy.data()),
                                      static_cast<const float*>(w.data()), static_cast<float*>(dx.data()), xs[0], xs[1],
                                      xs[2], xs[3], ws[0], ws[2], ws[3], sh, sw, ph, pw, dh, dwl);
    if (st == TF_ERR_UNSUPPORTED) return false;
    check(st, "hip::conv2d_backward_data");
    return true;
}

void chansum_nchw(const Tensor& dy, Tensor& db) {
    require_gpu(dy, "hip::chansum");
    require(dy.shape().ndim() == 4, "hip::chansum: NCHW");
    const int64_t N = dy.shape()[0], C = dy.shape()[1], HW = dy.shape()[2] * dy.shape()[3];
    require(db.numel() == C, "hip::chansum: db size");
    check(tf_chansum_nchw(ctx_of(dy), static_cast<const float*>(dy.data()), static_cast<float*>(db.data()), N, C, HW),
          "hip::chansum");
}

void im2col(const Tensor& x, Tensor& col, int64_t kH, int64_t kW, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
            int64_t dh, int64_t dw) {
    require_gpu(x, "hip::im2col"); require_gpu(col, "hip::im2col");
    require(x.shape().ndim() == 4, "hip::im2col: NCHW");
    const auto& s = x.shape();
    check(tf_im2col(ctx_of(x), x.data(), col.data(), s[0], s[1], s[2], s[3], kH, kW, sh, sw, ph, pw, dh, dw,
                    tf_code(x.dtype())),
          "hip::im2col");
}

void col2im(const Tensor& col, Tensor& dx, int64_t kH, int64_t kW, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
            int64_t dh, int64_t dw) {
    require_gpu(col, "hip::col2im"); require_gpu(dx, "hip::col2im");
    require(dx.shape().ndim() == 4, "hip::col2im: NCHW");
    const auto& s = dx.shape();
    const int64_t oh = (s[2] + 2 * ph - dh * (kH - 1) - 1) / sh + 1, ow = (s[3] + 2 * pw - dw * (kW - 1) - 1) / sw + 1;
    check(tf_col2im(ctx_of(col), col.data(), dx.data(), s[0], s[1], s[2], s[3], kH, kW, sh, sw, ph, pw, dh, dw, oh, ow,
                    tf_code(col.dtype())),
          "hip::col2im");
}

void sgd_momentum(Tensor& p, const Tensor& g, Tensor* v, Tensor* shadow, float lr, float mu) {
    require_gpu(p, "hip::sgd"); require_gpu(g, "hip::sgd");
    require(p.dtype() == Dtype::Float32 && g.dtype() == Dtype::Float32 && p.numel() == g.numel(),
            "hip::sgd: p and g must be Float32 of equal size");
    if (v) require(v->numel() == p.numel() && v->dtype() == Dtype::Float32, "hip::sgd: velocity size");
    if (shadow) require(shadow->numel() == p.numel() && shadow->dtype() == Dtype::BFloat16, "hip::sgd: shadow");
    check(tf_sgd_momentum(ctx_of(p), static_cast<float*>(p.data()), static_cast<const float*>(g.data()),
                          v ? static_cast<float*>(v->data()) : nullptr, shadow ? shadow->data() : nullptr, p.numel(),
                          lr, mu),
          "hip::sgd");
}

void sgd_momentum_multi(std::vector<SgdItem>& items, float lr, float mu) {
    size_t i = 0;
    while (i < items.size()) {
        // A run of up to TF_SGD_MULTI_MAX parameters on one device.
        tf_ctx* ctx = ctx_of(*items[i].p);
        float* ps[TF_SGD_MULTI_MAX];
        const float* gs[TF_SGD_MULTI_MAX];
        float* vs[TF_SGD_MULTI_MAX];
        void* ss[TF_SGD_MULTI_MAX];
        int64_t ns[TF_SGD_MULTI_MAX];
        int count = 0;
        for (; i < items.size() && count < TF_SGD_MULTI_MAX && ctx_of(*items[i].p) == ctx; ++i, ++count) {
            SgdItem& it = items[i];
            Tensor& p = *it.p;
            require_gpu(p, "hip::sgd"); require_gpu(it.g, "hip::sgd");
            require(p.dtype() == Dtype::Float32 && it.g.dtype() == Dtype::Float32 && p.numel() == it.g.numel(),
                    "hip::sgd: p and g must be Float32 of equal size");
            if (it.v) require(it.v->numel() == p.numel() && it.v->dtype() == Dtype::Float32, "hip::sgd: velocity size");
            if (it.shadow.numel())
                require(it.shadow.numel() == p.numel() && it.shadow.dtype() == Dtype::BFloat16, "hip::sgd: shadow");
            ps[count] = static_cast<float*>(p.data());
            gs[count] = static_cast<const float*>(it.g.data());
            vs[count] = it.v ? static_cast<float*>(it.v->data()) : nullptr;
            ss[count] = it.shadow.numel() ? it.shadow.data() : nullptr;
            ns[count] = p.numel();
        }
        check(tf_sgd_momentum_multi(ctx, count, ps, gs, vs, ss, ns, lr, mu), "hip::sgd");
    }
}

}  // namespace tensorforge::hip
