// Reductions and layout kernels behind the Tensor ops the backward pass
// composes: sum along one dimension (Tensor::sum, tensor/Tensor.cpp:513-561),
// its backward broadcast (SumBackward), and a batched 2-D transpose
// (Tensor::transpose copies, tensor/Tensor.cpp:579-619).  All operate on
// contiguous row-major data viewed as [outer][reduce][inner].
#include "common.hpp"

namespace {

// inner == 1: one wave per row, out[o] = sum_r x[o][r].
__global__ __launch_bounds__(256) void rowsum_kernel(const float* __restrict__ x, float* __restrict__ out, int64_t rows,
                                                     int64_t cols) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float* xr = x + r * cols;
    float s = 0.0f;
    for (int64_t j = lane; j < cols; j += 64) s += xr[j];
    s = tfd::wave_sum(s);
    if (lane == 0) out[r] = s;
}

// General: one thread per output element, reduce dimension walked in order.
__global__ void sum_dim_kernel(const float* __restrict__ x, float* __restrict__ out, int64_t outer, int64_t reduce,
                               int64_t inner) {
    const int64_t total = outer * inner;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < total; i += stride) {
        const int64_t o = i / inner, in = i - o * inner;
        const float* p = x + o * reduce * inner + in;
        float s = 0.0f;
        for (int64_t r = 0; r < reduce; ++r) s += p[r * inner];
        out[i] = s;
    }
}

// out[o][r][i] = up[o][i].
__global__ void expand_dim_kernel(const float* __restrict__ up, float* __restrict__ out, int64_t outer, int64_t reduce,
                                  int64_t inner) {
    const int64_t total = outer * reduce * inner;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < total; i += stride) {
        const int64_t in = i % inner;
        const int64_t o = i / (reduce * inner);
        out[i] = up[o * inner + in];
    }
}

// out[b][j][i] = x[b][i][j] through a 64 x 65 LDS tile (conflict-free).
template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(const T* __restrict__ x, T* __restrict__ out, int64_t R,
                                                        int64_t C) {
    __shared__ T tile[64][65];
    const int64_t b = blockIdx.z;
    const T* xb = x + b * R * C;
    T* ob = out + b * R * C;
    const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4) {
        const int64_t r = r0 + i, c = c0 + tx;
        if (r < R && c < C) tile[i][tx] = xb[r * C + c];
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
        const int64_t c = c0 + i, r = r0 + tx;
        if (r < R && c < C) ob[c * R + r] = tile[tx][i];
    }
}

}  // namespace

extern "C" {

tf_status tf_sum_dim(tf_ctx* ctx, const float* x, float* out, int64_t outer, int64_t reduce, int64_t inner) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(outer >= 0 && reduce >= 0 && inner >= 0, "tf_sum_dim: negative extent");
    if (outer == 0 || inner == 0) return TF_OK;
    TF_REQUIRE(out != nullptr && (reduce == 0 || x != nullptr), "tf_sum_dim: null pointer");
    if (reduce == 0) return tf_hip_fill_f32(ctx, out, 0.0f, outer * inner);
    if (inner == 1) {
        rowsum_kernel<<<(unsigned)((outer + 3) / 4), 256, 0, ctx->stream>>>(x, out, outer, reduce);
        return tfh::check_launch("rowsum_kernel");
    }
    if (outer == 1) return tf_colsum(ctx, x, out, reduce, inner);
    sum_dim_kernel<<<tfd::grid_for(outer * inner), 256, 0, ctx->stream>>>(x, out, outer, reduce, inner);
    return tfh::check_launch("sum_dim_kernel");
}

tf_status tf_expand_dim(tf_ctx* ctx, const float* up, float* out, int64_t outer, int64_t reduce, int64_t inner) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(outer >= 0 && reduce >= 0 && inner >= 0, "tf_expand_dim: negative extent");
    const int64_t total = outer * reduce * inner;
    if (total == 0) return TF_OK;
    TF_REQUIRE(up && out, "tf_expand_dim: null pointer");
    expand_dim_kernel<<<tfd::grid_for(total, 4), 256, 0, ctx->stream>>>(up, out, outer, reduce, inner);
    return tfh::check_launch("expand_dim_kernel");
}

tf_status tf_transpose2d(tf_ctx* ctx, const void* x, void* out, int64_t batch, int64_t rows, int64_t cols, int dtype) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(batch >= 0 && rows >= 0 && cols >= 0 && batch < 65536, "tf_transpose2d: bad extent");
    if (batch == 0 || rows == 0 || cols == 0) return TF_OK;
    TF_REQUIRE(x && out && x != out, "tf_transpose2d: null or aliased pointer");
    TF_REQUIRE((rows + 63) / 64 < 65536, "tf_transpose2d: too many rows");
    dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64), (unsigned)batch);
    if (dtype == TF_F32 || dtype == TF_I32) {
        transpose_kernel<uint32_t><<<grid, 256, 0, ctx->stream>>>((const uint32_t*)x, (uint32_t*)out, rows, cols);
    } else if (dtype == TF_BF16 || dtype == TF_F16) {
        transpose_kernel<uint16_t><<<grid, 256, 0, ctx->stream>>>((const uint16_t*)x, (uint16_t*)out, rows, cols);
    } else if (dtype == TF_I64) {
        transpose_kernel<uint64_t><<<grid, 256, 0, ctx->stream>>>((const uint64_t*)x, (uint64_t*)out, rows, cols);
    } else {
        return tfh::set_error(TF_ERR_UNSUPPORTED, "tf_transpose2d: unsupported dtype");
    }
    return tfh::check_launch("transpose_kernel");
}

}  // extern "C"
