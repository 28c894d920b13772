/*
 * tfa_harness.h — C entry points of libtensorforge.so that drive the C++20
 * tensorforge API (Tensor / Engine / nn / optim) end to end.  They are the
 * test and benchmark harness of this backend (the reference's equivalents
 * are its example programs, examples/train_mlp.cpp and
 * examples/train_cnn.cpp, and its doctest suites); they are not part of the
 * drop-in kernel boundary, which is include/tf_hip.h.
 *
 * Every function returns 0 on success and non-zero on failure, with a
 * message from tfa_last_error().
 */
#ifndef TFA_HARNESS_H
#define TFA_HARNESS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char* tfa_last_error(void);

/* MLP training through nn::Linear, nn::ReLU, nn::CrossEntropyLoss,
 * Tensor::backward and optim::SGD.
 *   dims[ndims]        layer widths, e.g. {784, 256, 128, 10}
 *   xs                 [n_batches][batch][dims[0]] float32, ys [n_batches][batch] int64;
 *                      step s uses batch s % n_batches
 *   on_gpu             0: CPU tensors, 1: GPU 0
 *   reference_compat   1: Linear drops its bias (as the reference does)
 *   bf16               1: Linear layers compute in bf16 with fp32 master weights (GPU only)
 *   init_weights       NULL (module init) or the concatenated weights [dims[l+1] x dims[l]]
 *   losses[steps]      out: loss of every step (read back after the loop)
 *   final_weights      NULL or out: concatenated weights after the last step
 *   ms_per_step        NULL or out: wall time per timed step (steps after `warmup`),
 *                      host launch work included, device drained at both ends.
 *   pool_used          NULL or out [steps]: the device pool's bytes in use after each
 *                      step (the device drained first; GPU only, and then the steps
 *                      are not timed).
 *   graph              0: every step launched from the host.  1: the warmup steps
 *                      (>= 1) run eagerly, one step is captured in a HIP graph
 *                      (tf_graph_*) and the remaining steps are replays of it, each
 *                      picking its batch and recording its loss on the device.
 *                      2: as 1, with the host waiting for every replay and reading
 *                      its loss before the next (checked replays; not a timing mode).
 *                      GPU only, without pool_used. */
int tfa_mlp_train(const int32_t* dims, int32_t ndims, int64_t batch, int64_t steps, int64_t warmup,
                  int64_t n_batches, const float* xs, const int64_t* ys, float lr, float mu, int32_t on_gpu,
                  int32_t reference_compat, int32_t bf16, const float* init_weights, float* losses,
                  float* final_weights, double* ms_per_step, uint64_t* pool_used, int32_t graph);

/* One training step of tfa_mlp_train's MLP (biases on, zero at the start,
 * as nn::Linear initialises them), keeping what the step stored, so that
 * every GEMM and reduction of the step can be judged against float64 on the
 * step's own operands.  x [batch][dims[0]] float32, y [batch] int64.
 *   loss      out [1]
 *   acts      out: the first layer's input as its GEMM read it (rounded to
 *             bf16 in bf16 compute), then every layer's output (hidden
 *             layers after their ReLU, then the logits): batch x dims[l] for
 *             l = 0 .. ndims-1, concatenated, widened to float32 (exact)
 *   grads     out: the gradient of every layer's output (Tensor::grad of the
 *             intermediates, kept as in the reference), l = 1 .. ndims-1
 *   final_weights, final_biases   NULL or out: parameters after the SGD step */
int tfa_mlp_step_trace(const int32_t* dims, int32_t ndims, int64_t batch, const float* x, const int64_t* y, float lr,
                       float mu, int32_t on_gpu, int32_t bf16, const float* init_weights, float* loss, float* acts,
                       float* grads, float* final_weights, float* final_biases);

/* CNN training (the config-4 network): Conv2dModule(3,32,3,1,1) - ReLU -
 * Conv2dModule(32,64,3,2,1) - ReLU - flatten - Linear(64*(H/2)*(W/2), 10) -
 * CrossEntropyLoss, optim::SGD.  xs [n_batches][batch][3][H][W]; init_params
 * NULL or {conv1.w, conv1.b, conv2.w, conv2.b, fc.w, fc.b} concatenated;
 * final_params NULL or out: the same six tensors after the last step. */
int tfa_cnn_train(int64_t batch, int64_t H, int64_t W, int64_t steps, int64_t warmup, int64_t n_batches,
                  const float* xs, const int64_t* ys, float lr, float mu, int32_t on_gpu, const float* init_params,
                  float* losses, float* final_params, double* ms_per_step);

/* Returns the GPU memory the harness's context holds unused (its block cache
 * and the pool's free memory) to the driver, so that the next run starts
 * from an empty pool as in a fresh process; 0 also when no GPU context
 * exists yet. */
int tfa_release_memory(void);

/* Runs one of the C++ self-tests (`name`, see tfa_selftest_names) on the CPU
 * (on_gpu = 0) or on GPU 0 (on_gpu = 1). */
int tfa_selftest(const char* name, int32_t on_gpu);
/* Space-separated list of self-test names. */
const char* tfa_selftest_names(void);

#ifdef __cplusplus
}
#endif

#endif /* TFA_HARNESS_H */
