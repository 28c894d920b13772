/*
 * tf_hip.h — C ABI of the MI355X (gfx950) backend for tensorforge's training
 * hot path: the reverse-mode backward pass, its gradient kernels and the
 * fused SGD-momentum update.
 *
 * Every entry point is extern "C", takes plain pointers and sizes, returns a
 * tf_status (0 = TF_OK) and records a human-readable message retrievable with
 * tf_last_error() (thread-local) on failure.  Kernels are asynchronous on the
 * context's current stream; nothing synchronises implicitly except the calls
 * documented as synchronous (tf_hip_sync, tf_hip_memcpy with D2H/H2H,
 * tf_hip_event_elapsed).
 *
 * All matrices are row-major.  Dtype codes match tensorforge's
 * `enum class Dtype : uint8_t` (reference tensor/Dtype.hpp:9-16).
 *
 * The reference interfaces each group replaces are cited beside it
 * (paths relative to the reference repository root).
 */
#ifndef TF_HIP_H
#define TF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct tf_ctx tf_ctx;
typedef int tf_status;

enum {
    TF_OK = 0,
    TF_ERR_INVALID = 1,     /* bad argument (shape, dtype, null pointer) */
    TF_ERR_HIP = 2,         /* a HIP runtime call failed */
    TF_ERR_UNSUPPORTED = 3, /* dtype/layout combination not implemented */
    TF_ERR_OOM = 4          /* device allocation failed */
};

/* == tensorforge Dtype (tensor/Dtype.hpp:9-16) */
enum {
    TF_F32 = 0,
    TF_F16 = 1,
    TF_BF16 = 2,
    TF_I32 = 3,
    TF_I64 = 4,
    TF_BOOL = 5
};

/* == allocator_dispatch::CudaCopyKind (tensor/CPUStorageAllocator.hpp:69-74) */
enum {
    TF_COPY_H2H = 0,
    TF_COPY_H2D = 1,
    TF_COPY_D2H = 2,
    TF_COPY_D2D = 3
};

/* GEMM epilogues applied after alpha*acc + beta*C. */
enum {
    TF_EPI_NONE = 0,
    TF_EPI_BIAS = 1,      /* + bias[n] */
    TF_EPI_BIAS_RELU = 2, /* max(. + bias[n], 0) */
    TF_EPI_RELU = 3,      /* max(., 0) */
    TF_EPI_ROW_BIAS = 4,  /* + bias[m]          (conv forward: one bias per output channel) */
    TF_EPI_ROW_BIAS_RELU = 5
};

/* ---------------------------------------------------------------------------
 * Errors and version
 * ------------------------------------------------------------------------- */
const char* tf_last_error(void);
const char* tf_version(void);

/* ---------------------------------------------------------------------------
 * Runtime: context, stream, allocator, copies, events.
 * Replaces DeviceContext / CudaStream / CudaEvent (cuda/CudaContext.hpp:23-140,
 * cuda/CudaContext.cpp:18-60) and CudaStorageAllocator
 * (cuda/memory/CudaStorageAllocator.cpp:34-143).
 * ------------------------------------------------------------------------- */

/* Number of visible GPUs (0 when none). Never fails on a GPU-less host. */
tf_status tf_hip_device_count(int* count);

/* Create a context on `device`: one non-blocking stream at default priority
 * and a hipMemPool_t with a raised release threshold (the reference pool keeps
 * 64 MiB, cuda/memory/CudaStorageAllocator.cpp:48-50; this one keeps all freed
 * memory cached until tf_hip_trim). */
tf_status tf_hip_init(int device, tf_ctx** out);
tf_status tf_hip_shutdown(tf_ctx* ctx);

/* The stream kernels are launched on (hipStream_t as void*). */
tf_status tf_hip_stream(tf_ctx* ctx, void** stream);
/* Launch on a caller-owned stream from now on; NULL restores the context's. */
tf_status tf_hip_set_stream(tf_ctx* ctx, void* stream);
/* Block until all work on the current stream has finished. */
tf_status tf_hip_sync(tf_ctx* ctx);

/* Stream-ordered pool allocation (hipMallocAsync on the context's pool).
 * bytes == 0 allocates 1 byte, as the reference does
 * (cuda/memory/storage_allocator_test.cpp:42-48). */
tf_status tf_hip_alloc(tf_ctx* ctx, size_t bytes, void** out);
/* Stream-ordered free: the block waits in the context's cache for the next
 * allocation of its size class (512-byte steps to 1 MB, 2 MB steps above)
 * on the context's stream.  NULL is a no-op; a pointer this context did not
 * allocate (or already freed) is an error. */
tf_status tf_hip_free(tf_ctx* ctx, void* ptr);
/* Hand the context's cached blocks back to the pool and return pool memory
 * above `keep_bytes` to the device. */
tf_status tf_hip_trim(tf_ctx* ctx, size_t keep_bytes);
/* Bytes currently reserved by the pool and in use by live allocations. */
tf_status tf_hip_pool_stats(tf_ctx* ctx, uint64_t* reserved, uint64_t* used);

/* Copy `bytes` (kind = TF_COPY_*). H2D and D2D are stream-ordered; D2H and
 * H2H return after the data has landed.  Replaces cuda_copy_dispatch
 * (cuda/memory/CudaStorageAllocator.cpp:67-87). */
tf_status tf_hip_memcpy(tf_ctx* ctx, void* dst, const void* src, size_t bytes, int kind);

/* p[i] = value for i < n (float32) — a kernel, safe under graph capture. */
tf_status tf_hip_fill_f32(tf_ctx* ctx, float* p, float value, int64_t n);
/* Byte fill through a kernel (no hipMemsetAsync). */
tf_status tf_hip_zero(tf_ctx* ctx, void* p, size_t bytes);

/* Events on the current stream, for timing. */
tf_status tf_hip_event_create(tf_ctx* ctx, void** event);
tf_status tf_hip_event_record(tf_ctx* ctx, void* event);
/* Waits for `end`, then returns the elapsed milliseconds start -> end. */
tf_status tf_hip_event_elapsed(void* start, void* end, float* ms);
tf_status tf_hip_event_destroy(void* event);

/* HIP-graph capture (no counterpart in the reference, which launches every
 * kernel of a step from the host, examples/train_mlp.cpp:141-199).  For
 * callers whose step is launch-bound: capture it once, then replay it with
 * one tf_graph_launch per step.
 *   tf_graph_begin  starts capturing the context's stream: every library call
 *                   on the context until tf_graph_end is recorded, not run.
 *                   While capturing, tf_hip_alloc serves only from blocks
 *                   freed earlier in the capture or from the block cache (a
 *                   miss is TF_ERR_INVALID: run the step once eagerly first,
 *                   which fills the cache), the workspace may not grow, and
 *                   tf_hip_sync, tf_hip_set_stream, tf_hip_trim and copies
 *                   other than TF_COPY_D2D are errors.
 *   tf_graph_end    ends the capture and instantiates the graph; after a
 *                   failed call during capture it returns that error and no
 *                   graph.  Blocks freed during capture belong to the graph
 *                   until tf_graph_destroy (so no other allocation receives a
 *                   replay's temporaries), and so do blocks allocated during
 *                   capture that the caller frees while the graph exists:
 *                   tf_hip_free hands them to the graph, not to the cache.
 *                   Blocks allocated before the capture that the graph reads
 *                   or writes must stay live while it is replayed.
 *   tf_graph_launch enqueues one replay on the context's stream (the context
 *                   must be the capturing one, its workspace unmoved).
 *   tf_graph_destroy returns the graph's blocks to the context's cache;
 *                   destroy graphs before tf_hip_shutdown of their context.
 * Captured work contains no hipMemsetAsync (fills are kernels). */
typedef struct tf_graph tf_graph;
tf_status tf_graph_begin(tf_ctx* ctx);
tf_status tf_graph_end(tf_ctx* ctx, tf_graph** out);
tf_status tf_graph_launch(tf_ctx* ctx, tf_graph* graph);
tf_status tf_graph_destroy(tf_graph* graph);
/* Device-side step selection for a replayed step (no counterpart in the
 * reference).  tf_gather_indexed: dst[0:bytes) = table[*counter % n][0:bytes),
 * where table holds n device addresses (as uint64), each of a buffer of at
 * least `bytes` bytes.  tf_record_step: ring[*counter] = *src when
 * 0 <= *counter < ring_len, then *counter += 1.  Both read the counter on
 * the device, so a captured step picks a new batch and records its loss on
 * every replay. */
tf_status tf_gather_indexed(tf_ctx* ctx, void* dst, const uint64_t* table, int64_t n, const int64_t* counter,
                            int64_t bytes);
tf_status tf_record_step(tf_ctx* ctx, const float* src, float* ring, int64_t ring_len, int64_t* counter);

/* Launch timing, for measurement (no counterpart in the reference, whose
 * benchmarks time from outside).  tf_hip_timing_start creates `max_records`
 * event pairs and starts recording: from then on every GEMM call
 * (tf_gemm, tf_gemm_noalloc, tf_gemm_strided_batched, tf_gemm_ex) on any
 * context records one event before its kernels and one after them on that
 * context's stream, until the records are used up or tf_hip_timing_stop.
 * The events add two stream packets per GEMM: time a step without them.
 * tf_hip_timing_record returns record i: shape = {M, N, K, batch},
 * meta = {trans_a, trans_b, in_dtype, out_dtype}, and the milliseconds
 * between its events (this waits for the second one). */
tf_status tf_hip_timing_start(int max_records);
tf_status tf_hip_timing_stop(int* count);
tf_status tf_hip_timing_record(int i, int64_t* shape, int* meta, float* ms);

/* ---------------------------------------------------------------------------
 * GEMM on MFMA.  C[m,n] = epi(alpha * sum_k op(A)[m,k] * op(B)[k,n] + beta*C[m,n])
 *   op(A) is M x K: trans_a == 0 -> A[m*lda + k], trans_a == 1 -> A[k*lda + m]
 *   op(B) is K x N: trans_b == 0 -> B[k*ldb + n], trans_b == 1 -> B[n*ldb + k]
 * in_dtype: TF_F32 (v_mfma_f32_32x32x2_f32) or TF_BF16 (bf16 MFMA, fp32
 * accumulate).  out_dtype: TF_F32 or TF_BF16.  bias: float32[N] or NULL.
 * beta != 0 requires out_dtype == TF_F32.
 * Replaces launch_gemm_{naive,tiled_16x16,optimized} (cuda/kernels/gemm.cuh:33-53)
 * and the CPU loops of Tensor::matmul (tensor/Tensor.cpp:334-368) plus the
 * transpose copies of MatmulBackward (autograd/ops/MatmulBackward.hpp:29-32),
 * which become layout flags.
 * ------------------------------------------------------------------------- */
tf_status tf_gemm(tf_ctx* ctx, int trans_a, int trans_b,
                  int64_t M, int64_t N, int64_t K, float alpha,
                  const void* A, int64_t lda, const void* B, int64_t ldb,
                  float beta, void* C, int64_t ldc,
                  int in_dtype, int out_dtype, int epilogue, const float* bias);

/* tf_gemm without any allocation: no counterpart in the reference; for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * kernels and results as tf_gemm; the split-K partials, which tf_gemm keeps
 * in the context's pool-grown workspace, go to a fixed 64 MiB device array
 * instead (one per GPU, held until the process ends).  A shape whose
 * partials need more is rejected with TF_ERR_INVALID.  Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (two streams, two
 * threads) race and must be ordered by the caller. */
tf_status tf_gemm_noalloc(tf_ctx* ctx, int trans_a, int trans_b,
                          int64_t M, int64_t N, int64_t K, float alpha,
                          const void* A, int64_t lda, const void* B, int64_t ldb,
                          float beta, void* C, int64_t ldc,
                          int in_dtype, int out_dtype, int epilogue, const float* bias);

/* Strided-batched GEMM: for b < batch, the same op on A + b*stride_a,
 * B + b*stride_b, C + b*stride_c (strides in elements).  Used by Conv2d
 * forward/backward in place of the reference's per-sample launches
 * (nn/Conv2d.cpp:124-127, 186-198, 213-243). */
tf_status tf_gemm_strided_batched(tf_ctx* ctx, int trans_a, int trans_b,
                                  int64_t M, int64_t N, int64_t K, float alpha,
                                  const void* A, int64_t lda, int64_t stride_a,
                                  const void* B, int64_t ldb, int64_t stride_b,
                                  float beta, void* C, int64_t ldc, int64_t stride_c,
                                  int64_t batch, int in_dtype, int out_dtype);

/* General form.  batch > 1 with reduce_batch == 0: independent products as
 * tf_gemm_strided_batched.  reduce_batch != 0: one output,
 *   C = epi(alpha * sum_b op(A + b*stride_a) op(B + b*stride_b) + beta*C),
 * i.e. a GEMM whose reduction runs over (b, k) — Conv2d's weight gradient
 * dW = sum_n dY[n] col[n]^T without the reference's per-sample host
 * accumulation (nn/Conv2d.cpp:213-243).  stride_c is ignored then. */
tf_status tf_gemm_ex(tf_ctx* ctx, int trans_a, int trans_b,
                     int64_t M, int64_t N, int64_t K, float alpha,
                     const void* A, int64_t lda, int64_t stride_a,
                     const void* B, int64_t ldb, int64_t stride_b,
                     float beta, void* C, int64_t ldc, int64_t stride_c,
                     int64_t batch, int reduce_batch,
                     int in_dtype, int out_dtype, int epilogue, const float* bias);

/* ---------------------------------------------------------------------------
 * Elementwise forward + backward (bandwidth kernels, float32 unless noted).
 * Forward ops replace the registered elementwise launchers
 * (cuda/CudaKernelRegistry.hpp:15-26, cuda/kernels/elementwise.cu:80-173).
 * ------------------------------------------------------------------------- */
tf_status tf_add(tf_ctx* ctx, const void* a, const void* b, void* out, int64_t n, int dtype);
tf_status tf_sub(tf_ctx* ctx, const void* a, const void* b, void* out, int64_t n, int dtype);
tf_status tf_mul(tf_ctx* ctx, const void* a, const void* b, void* out, int64_t n, int dtype);
/* out = a * s[0] where s is a device scalar. */
tf_status tf_scale_by(tf_ctx* ctx, const void* a, const float* s, void* out, int64_t n, int dtype);
tf_status tf_relu_fwd(tf_ctx* ctx, const void* x, void* y, int64_t n, int dtype);
/* y = x > 0 ? x : alpha * x  (the registry's LeakyReluFn slot,
 * cuda/CudaKernelRegistry.hpp:17,24, filled by cuda/kernels/elementwise.cu:299-301,325) */
tf_status tf_leaky_relu_fwd(tf_ctx* ctx, const void* x, void* y, int64_t n, float alpha, int dtype);
tf_status tf_sigmoid_fwd(tf_ctx* ctx, const void* x, void* y, int64_t n, int dtype);
tf_status tf_tanh_fwd(tf_ctx* ctx, const void* x, void* y, int64_t n, int dtype);

/* dx = dy * (x > 0 ? 1 : 0)   (autograd/ops/ReluBackward.hpp:22-32) */
tf_status tf_relu_bwd(tf_ctx* ctx, const void* dy, const void* x, void* dx, int64_t n, int dtype);
/* dx = dy * y * (1 - y), y = sigmoid output (autograd/TensorAutograd.cpp:152-156) */
tf_status tf_sigmoid_bwd(tf_ctx* ctx, const void* dy, const void* y, void* dx, int64_t n, int dtype);
/* dx = dy * (1 - y*y), y = tanh output (autograd/TensorAutograd.cpp:158-164) */
tf_status tf_tanh_bwd(tf_ctx* ctx, const void* dy, const void* y, void* dx, int64_t n, int dtype);

/* ---------------------------------------------------------------------------
 * Row kernels (one wave64 per row).
 * ------------------------------------------------------------------------- */
/* Cross-entropy forward: lse[r] = logsumexp(logits[r,:]) (may be NULL) and
 * loss[0] = mean_r nll[r], nll[r] = lse[r] - logits[r, t_r].  flags:
 *   0 (TF_CE_CHAIN): the train_mlp chain (examples/train_mlp.cpp:54-76): a
 *     target outside [0, cols) contributes nll 0 (its one-hot row is empty);
 *   TF_CE_STRICT: such a target makes its nll, and so the loss, NaN (the
 *     module throws for it, nn/CrossEntropyLoss.cpp:47-53; no host check);
 *   TF_CE_CLAMP: nll[r] <= -logf(1e-9f), the module's clamp of the
 *     probability at 1e-9 (nn/CrossEntropyLoss.cpp:54-55);
 *   TF_CE_MODULE = both: nn::CrossEntropyLoss::forward's loss. */
enum { TF_CE_CHAIN = 0, TF_CE_STRICT = 1, TF_CE_CLAMP = 2, TF_CE_MODULE = 3 };
tf_status tf_ce_fwd(tf_ctx* ctx, const float* logits, const int64_t* targets,
                    float* loss, float* lse, int64_t rows, int64_t cols, int flags);
/* Fused LogSoftmax+NLL backward: dlogits = g * (softmax(logits) - onehot) / rows
 * where g = grad_loss[0] (NULL means 1).  With lse from tf_ce_fwd the kernel
 * is a single streaming pass; with lse == NULL it recomputes row statistics.
 * Replaces LogSoftmaxBackward + MulBackward + 2x SumBackward + 2x scalar
 * MulBackward of the chain (autograd/ops/LogSoftmaxBackward.hpp:26-58). */
tf_status tf_ce_bwd(tf_ctx* ctx, const float* logits, const int64_t* targets,
                    const float* lse, const float* grad_loss, float* dlogits,
                    int64_t rows, int64_t cols);
/* Forward and backward in one pass over logits (upstream gradient 1); flags
 * as tf_ce_fwd's (they change the loss only). */
tf_status tf_ce_fwd_bwd(tf_ctx* ctx, const float* logits, const int64_t* targets,
                        float* loss, float* dlogits, int64_t rows, int64_t cols, int flags);
/* The same for bf16 logits (bit patterns): each value widened to fp32 in the
 * kernel (exact), the loss in fp32, dlogits rounded to bf16 (nearest even).
 * Equal to tf_ce_fwd_bwd on the widened logits followed by a cast of dlogits
 * to bf16, in one pass: the cross entropy of a bf16 Linear's output
 * (nn/CrossEntropyLoss.cpp:13-77 on the bf16 compute path). */
tf_status tf_ce_fwd_bwd_bf16(tf_ctx* ctx, const void* logits, const int64_t* targets,
                             float* loss, void* dlogits, int64_t rows, int64_t cols, int flags);
/* pred[r] = first column of row r holding its largest value, with the
 * reference's scan (examples/train_mlp.cpp:95-100: running maximum from
 * -1e30, strict '>', prediction 0 when no value exceeds it).  With labels
 * (int64[rows]) and correct (int64[1]) both non-NULL, also
 * correct[0] = #{r : pred[r] == labels[r]} (the accuracy count of
 * eval_accuracy, examples/train_mlp.cpp:101), without a host copy. */
tf_status tf_argmax_rows(tf_ctx* ctx, const float* x, int64_t* pred, const int64_t* labels, int64_t* correct,
                         int64_t rows, int64_t cols);
/* Row log_softmax / softmax forward (tensor/Tensor.cpp:370-447). */
tf_status tf_log_softmax_fwd(tf_ctx* ctx, const float* x, float* y, int64_t rows, int64_t cols);
tf_status tf_softmax_fwd(tf_ctx* ctx, const float* x, float* y, int64_t rows, int64_t cols);
/* dx = dy - exp(y) * sum_j dy  (autograd/ops/LogSoftmaxBackward.hpp:26-58) */
tf_status tf_log_softmax_bwd(tf_ctx* ctx, const float* y, const float* dy, float* dx,
                             int64_t rows, int64_t cols);
/* dx = y * (dy - sum_j dy*y)  (autograd/ops/SoftmaxBackward.hpp:27-55) */
tf_status tf_softmax_bwd(tf_ctx* ctx, const float* y, const float* dy, float* dx,
                         int64_t rows, int64_t cols);

/* ---------------------------------------------------------------------------
 * Reductions (deterministic two-stage, no atomics).
 * ------------------------------------------------------------------------- */
/* db[c] = sum_r dy[r, c]  (Linear bias grad; no reference counterpart, the
 * reference Linear drops its bias, nn/Linear.cpp:60-63) */
tf_status tf_colsum(tf_ctx* ctx, const float* dy, float* db, int64_t rows, int64_t cols);
/* The same for bf16 dy (bit patterns), summed in fp32; equal to tf_colsum of
 * the widened tensor (the bf16 compute path's bias grad, no cast pass). */
tf_status tf_colsum_bf16(tf_ctx* ctx, const void* dy, float* db, int64_t rows, int64_t cols);
/* dz = dy * (x > 0 ? 1 : 0) over a [rows x cols] matrix, then
 * db[c] = sum_r dz[r, c]: the ReLU backward (autograd/ops/ReluBackward.hpp:22-32)
 * of a ReLU that follows a Linear with bias, fused with that Linear's bias
 * gradient (nn::Linear::forward_relu's backward).  dtype TF_F32 or TF_BF16
 * (dy, x, dz); db is fp32.  dz is bit-identical to tf_relu_bwd and db to
 * tf_colsum / tf_colsum_bf16 of that dz; one pass over dy and x where the
 * column-strip launch applies, else those two calls. */
tf_status tf_relu_bwd_colsum(tf_ctx* ctx, const void* dy, const void* x, void* dz, float* db, int64_t rows,
                             int64_t cols, int dtype);
/* C = (A * [mask > 0]) B in fp32, the ReLU backward folded into the load of a
 * product's left operand: op(A)[m, k] is taken as op(A)[m, k] *
 * (op(mask)[m, k] > 0 ? 1 : 0), mask laid out as A (same trans_a and lda).
 * Replaces ReluBackward's mask product (autograd/ops/ReluBackward.hpp:22-32)
 * in front of the two products of MatmulBackward
 * (autograd/ops/MatmulBackward.hpp:26-34) when a bias-free Linear is followed
 * by a ReLU: dX = (dY * [y > 0]) W and dW = (dY * [y > 0])^T X without the
 * masked gradient in memory.  Bit-identical to tf_relu_bwd then tf_gemm.
 * Only the small-product kernel takes the mask: K <= 2048 and M*N*K <= 2^27,
 * else TF_ERR_UNSUPPORTED (the caller then masks and multiplies in two
 * calls). */
tf_status tf_gemm_relu_masked(tf_ctx* ctx, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                              const float* A, int64_t lda, const float* mask, const float* B, int64_t ldb, float* C,
                              int64_t ldc);
/* Both weight-side products of a small bias-free Linear layer (y = x w^T,
 * fp32) in one launch: dx = dz w (M x K) and dw = dz^T x (N x K), with
 * dz = dy * (mask > 0 ? 1 : 0) when mask (shaped as dy) is given, else dy.
 * dy and mask are [M x N], x and dx [M x K], w and dw [N x K], row-major.
 * Replaces MatmulBackward's two products (autograd/ops/MatmulBackward.hpp:26-34)
 * behind nn/Linear.cpp:60-63, and with a mask the ReluBackward before them
 * (autograd/ops/ReluBackward.hpp:22-32).  Each block of the launch computes
 * exactly what it computes in the product's own launch, so dx and dw are
 * bit-identical to tf_gemm_relu_masked (tf_gemm without a mask) of each
 * product.  TF_ERR_UNSUPPORTED when either product does not fit the
 * small-product kernel (inner extent <= 2048, M*N*K <= 2^27). */
tf_status tf_linear_bwd_small(tf_ctx* ctx, const float* dy, const float* mask, const float* x, const float* w,
                              float* dx, float* dw, int64_t M, int64_t N, int64_t K);
/* The whole backward of a Linear layer with few outputs (fp32, N <= 16), in
 * one launch: dx[r, k] = sum_n dy[r, n] w[n, k] (M x K), dw[n, k] =
 * sum_r dy[r, n] x[r, k] (N x K), db[n] = sum_r dy[r, n].  Replaces, for such
 * layers, the two products of MatmulBackward (autograd/ops/MatmulBackward.hpp:26-34)
 * behind nn/Linear.cpp:60-63's x.matmul(W^T), the transpose of the weight
 * gradient (autograd/ops/TransposeBackward.hpp) and the bias column sum.
 * dx, dw or db may be NULL (not wanted).  Needs K % 4 == 0 and x, w, dx, dw
 * 16-byte aligned; dy is [M x N] contiguous.  Each block owns 64
 * columns of K for every row, so nothing is summed across blocks:
 * deterministic, every output written once. */
tf_status tf_linear_bwd_narrow(tf_ctx* ctx, const float* dy, const float* x, const float* w, float* dx, float* dw,
                               float* db, int64_t M, int64_t N, int64_t K);
/* db[c] = sum_{n,hw} dy[n, c, hw]  (replaces launch_reduce_sum_axis_nchw,
 * cuda/kernels/reduce_sum_axis.cu:53-120, which is wrong for H*W > 256) */
tf_status tf_chansum_nchw(tf_ctx* ctx, const float* dy, float* db,
                          int64_t N, int64_t C, int64_t HW);

/* ---------------------------------------------------------------------------
 * LayerNorm over the last dimension (tensor/Tensor.cpp:449-494).
 * ------------------------------------------------------------------------- */
/* y = (x - mean) * rstd * gamma + beta; saves mean[rows], rstd[rows]. */
tf_status tf_layernorm_fwd(tf_ctx* ctx, const float* x, const float* gamma, const float* beta,
                           float* y, float* mean, float* rstd, int64_t rows, int64_t cols, float eps);
/* True gradient: dx = rstd * (g - mean(g) - xhat * mean(g * xhat)), g = dy*gamma,
 * dgamma = sum_rows dy*xhat, dbeta = sum_rows dy.  reference_compat != 0
 * reproduces the reference's stub (autograd/ops/LayerNormBackward.hpp:39-59):
 * dx = dy * gamma, dgamma = dbeta = 0 (x, mean, rstd may then be NULL). */
tf_status tf_layernorm_bwd(tf_ctx* ctx, const float* dy, const float* x, const float* gamma,
                           const float* mean, const float* rstd, float* dx, float* dgamma,
                           float* dbeta, int64_t rows, int64_t cols, int reference_compat);

/* ---------------------------------------------------------------------------
 * Conv2d index maps, NCHW, with the parameter lists of launch_im2col
 * (cuda/kernels/im2col.cuh:37-43) and launch_col2im (cuda/kernels/col2im.cuh:22-29,
 * including its outH/outW, which must equal the geometry's) after the
 * context; the dtype is last and the stream is the context's.
 * col is [N][C*kH*kW][outH*outW].  col2im gathers (deterministic).
 * ------------------------------------------------------------------------- */
tf_status tf_im2col(tf_ctx* ctx, const void* x, void* col, int64_t N, int64_t C, int64_t H, int64_t W,
                    int64_t kH, int64_t kW, int64_t stride_h, int64_t stride_w, int64_t pad_h,
                    int64_t pad_w, int64_t dilation_h, int64_t dilation_w, int dtype);
tf_status tf_col2im(tf_ctx* ctx, const void* col, void* dx, int64_t N, int64_t C, int64_t H, int64_t W,
                    int64_t kH, int64_t kW, int64_t stride_h, int64_t stride_w, int64_t pad_h,
                    int64_t pad_w, int64_t dilation_h, int64_t dilation_w, int64_t outH, int64_t outW,
                    int dtype);

/* Conv2d forward without a col buffer (implicit GEMM; replaces
 * nn/Conv2d.cpp:101-139's launch_im2col + per-image launch_gemm_tiled_16x16 +
 * launch_bias_add): y[N][Cout][outH][outW] = conv(x[N][C][H][W],
 * w[Cout][C][kH][kW]) + bias[co] (bias may be NULL), then max(., 0) when
 * relu != 0.  Float32.  TF_ERR_UNSUPPORTED when Cout x C*kH*kW filter rows
 * and the input rows of 128 output pixels (all channels, padded width) do not
 * fit the 160 KB of LDS; the caller then uses tf_im2col + tf_gemm_ex. */
tf_status tf_conv2d_fwd(tf_ctx* ctx, const float* x, const float* w, const float* bias, float* y, int64_t N,
                        int64_t C, int64_t H, int64_t W, int64_t Cout, int64_t kH, int64_t kW, int64_t stride_h,
                        int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t dilation_h, int64_t dilation_w,
                        int relu);
/* Conv2d weight gradient without a col buffer (implicit GEMM; replaces
 * nn/Conv2d.cpp:140-260's launch_im2col + per-sample GEMM + host
 * accumulation): dw[Cout][C][kH][kW] = sum over images and output pixels of
 * dy[n][co][p] * col[n][k][p], col gathered from x; and, when db is not
 * NULL, the bias gradient db[co] = sum over images and pixels of dy[n][co][p]
 * (launch_reduce_sum_axis_nchw, cuda/kernels/reduce_sum_axis.cu:53-120) from
 * the same dy tiles.  Float32; per-block partials are summed in a fixed
 * order (deterministic).  TF_ERR_UNSUPPORTED when the dy tile, tap tables
 * and input patch do not fit the LDS. */
tf_status tf_conv2d_bwd_weight(tf_ctx* ctx, const float* x, const float* dy, float* dw, float* db, int64_t N, int64_t C,
                               int64_t H, int64_t W, int64_t Cout, int64_t kH, int64_t kW, int64_t stride_h,
                               int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t dilation_h,
                               int64_t dilation_w);
/* Conv2d data gradient without the dcol buffer or col2im (implicit GEMM over
 * the stride's sub-pixel phases; replaces nn/Conv2d.cpp:178-204's per-image
 * launch_gemm_tiled_16x16 of W^T x dy into col_grad + launch_col2im):
 * dx[N][C][H][W] = sum over co and the taps reaching each input pixel of
 * w[co][c][ki][kj] * dy[n][co][oh][ow].  Float32, deterministic (a fixed
 * order per geometry), every dx element written (zeros where no tap reaches).
 * TF_ERR_UNSUPPORTED when the filter columns and the dy patch of one phase
 * tile do not fit the LDS; the caller then uses tf_gemm_ex + tf_col2im. */
tf_status tf_conv2d_bwd_data(tf_ctx* ctx, const float* dy, const float* w, float* dx, int64_t N, int64_t C, int64_t H,
                             int64_t W, int64_t Cout, int64_t kH, int64_t kW, int64_t stride_h, int64_t stride_w,
                             int64_t pad_h, int64_t pad_w, int64_t dilation_h, int64_t dilation_w);
/* tf_conv2d_bwd_weight for a convolution followed by a ReLU (tf_conv2d_fwd
 * with relu != 0), taking the gradient through the ReLU on the way: dy is
 * the gradient of the ReLU's output y (same shape as dy), and dw, db are
 * formed from dy * (y > 0 ? 1 : 0), the ReluBackward of
 * autograd/ops/ReluBackward.hpp:22-32, applied to the kernel's staged dy
 * tiles instead of in a pass of its own.  When dz is not NULL that masked
 * gradient is also written there (the kernel's blocks cover dy once), for
 * the data gradient that follows (tf_conv2d_bwd_data on dz).  Results equal
 * tf_relu_bwd (dy, y) followed by tf_conv2d_bwd_weight, bit for bit. */
tf_status tf_conv2d_bwd_weight_relu(tf_ctx* ctx, const float* x, const float* dy, const float* y, float* dz, float* dw,
                                    float* db, int64_t N, int64_t C, int64_t H, int64_t W, int64_t Cout, int64_t kH,
                                    int64_t kW, int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                                    int64_t dilation_h, int64_t dilation_w);

/* Byte -> float decode of the file loaders (data/MnistLoader.cpp:43-80 and
 * data/CifarLoader.cpp:40-75 normalise each pixel on the host):
 * dst[i] = table[(i / plane) % channels][src[i]] for i < n, table being
 * channels x 256 floats (1 to 4 channels) on the device. */
tf_status tf_decode_u8(tf_ctx* ctx, const uint8_t* src, float* dst, int64_t n, int64_t plane, int channels,
                       const float* table);

/* ---------------------------------------------------------------------------
 * Layout kernels over contiguous data viewed as [outer][reduce][inner].
 * ------------------------------------------------------------------------- */
/* out[o][i] = sum_r x[o][r][i]  (Tensor::sum along one dim, tensor/Tensor.cpp:513-561) */
tf_status tf_sum_dim(tf_ctx* ctx, const float* x, float* out, int64_t outer, int64_t reduce, int64_t inner);
/* out[o][r][i] = up[o][i]  (SumBackward's broadcast along the reduced dim;
 * equals the reference's autograd/ops/SumBackward.hpp:35-37 wherever that
 * one is correct, i.e. for uniform upstream gradients) */
tf_status tf_expand_dim(tf_ctx* ctx, const float* up, float* out, int64_t outer, int64_t reduce, int64_t inner);
/* out[b][j][i] = x[b][i][j] for b < batch  (Tensor::transpose of the last two
 * dims, tensor/Tensor.cpp:579-619, which copies) */
tf_status tf_transpose2d(tf_ctx* ctx, const void* x, void* out, int64_t batch, int64_t rows, int64_t cols,
                         int dtype);

/* ---------------------------------------------------------------------------
 * Optimiser: fused SGD with momentum (nn/optim/SGD.hpp:3-6):
 *   v <- mu * v + g ;  p <- p - lr * v        (mu == 0: p <- p - lr * g, v untouched)
 * p, g, v float32[n]; p_bf16 (optional, may be NULL) receives bf16(p).
 * ------------------------------------------------------------------------- */
tf_status tf_sgd_momentum(tf_ctx* ctx, float* p, const float* g, float* v,
                          void* p_bf16, int64_t n, float lr, float mu);
/* The same update for `count` parameters in one launch (the per-parameter
 * loop of nn/optim/SGD.cpp:50-56): entry i is (p[i], g[i], v[i], p_bf16[i],
 * n[i]); v and p_bf16 may be NULL arrays (no velocity / no shadows) or hold
 * NULL entries.  Each parameter ends up as tf_sgd_momentum leaves it. */
#define TF_SGD_MULTI_MAX 32
tf_status tf_sgd_momentum_multi(tf_ctx* ctx, int count, float* const* p, const float* const* g,
                                float* const* v, void* const* p_bf16, const int64_t* n, float lr, float mu);

/* float32 <-> bf16 conversion (round to nearest even). */
tf_status tf_cast_f32_bf16(tf_ctx* ctx, const float* x, void* y, int64_t n);
tf_status tf_cast_bf16_f32(tf_ctx* ctx, const void* x, float* y, int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* TF_HIP_H */
