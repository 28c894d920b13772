// Shared plumbing for the gfx950 kernels behind include/tf_hip.h:
// the context struct, error recording, argument checks and small device
// helpers (wave64 reductions, bf16 conversion).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "tf_hip.h"

struct tf_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;   // current launch stream
    hipMemPool_t pool = nullptr;
    int num_cus = 0;
    // Scratch for multi-stage kernels (split-K partials, reduction partials,
    // per-row losses).  Grown on demand from the pool; stream-ordered.
    void* ws = nullptr;
    size_t ws_bytes = 0;
};

namespace tfh {

// Record a message for tf_last_error() and return the status.
tf_status set_error(tf_status code, const std::string& msg);
tf_status hip_error(hipError_t e, const char* what);

// Make sure ctx->ws holds at least `bytes`; returns TF_OK or an error.
tf_status ensure_workspace(tf_ctx* ctx, size_t bytes);
// out[j] = sum_k part[k * W + j] (fixed order) for j < W; columns j < split
// go to out_lo[j], the rest to out_hi[j - split].  Launched on ctx->stream.
tf_status partial_rows_sum(tf_ctx* ctx, const float* part, float* out_lo, float* out_hi, int64_t K, int64_t W,
                           int64_t split);

inline bool bad_ctx(tf_ctx* ctx) { return ctx == nullptr || ctx->stream == nullptr; }

// Launch-error check after every <<<>>>: catches bad launch shapes early.
inline tf_status check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, what);
    return TF_OK;
}

}  // namespace tfh

#define TF_REQUIRE(cond, msg)                                              \
    do {                                                                   \
        if (!(cond)) return tfh::set_error(TF_ERR_INVALID, (msg));         \
    } while (0)

#define TF_HIP_CHECK(expr)                                                 \
    do {                                                                   \
        hipError_t _e = (expr);                                            \
        if (_e != hipSuccess) return tfh::hip_error(_e, #expr);            \
    } while (0)

#define TF_CTX_CHECK(ctx)                                                  \
    do {                                                                   \
        if (tfh::bad_ctx(ctx)) return tfh::set_error(TF_ERR_INVALID, "null or shut-down tf_ctx"); \
    } while (0)

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
namespace tfd {

constexpr int kWave = 64;

// Butterfly sum over the 64 lanes of a wave; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

// bf16 <-> f32, round to nearest even; NaN stays NaN (quiet bit forced).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    // Round to nearest even; a NaN keeps its top bits and is made quiet.
    // Written as a select so the compiler emits no branch.
    const uint32_t u = __float_as_uint(f);
    const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    const uint32_t quiet = (u >> 16) | 0x40u;
    return (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? quiet : rounded);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(((uint32_t)h) << 16);
}

// Grid size for a grid-stride elementwise kernel over n items with 256
// threads per block: enough blocks to fill 256 CUs several times over.
inline int grid_for(int64_t n_items, int per_thread = 1, int max_blocks = 8192) {
    int64_t threads = (n_items + per_thread - 1) / per_thread;
    int64_t blocks = (threads + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > max_blocks) blocks = max_blocks;
    return (int)blocks;
}

}  // namespace tfd
