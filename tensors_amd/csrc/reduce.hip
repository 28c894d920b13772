// Bias-gradient reductions, deterministic two-stage (no atomics):
//   colsum : db[c] = sum_r dy[r, c]           (Linear bias grad)
//   chansum: db[c] = sum_{n,p} dy[n, c, p]    (Conv2d bias grad, NCHW)
// Stage 1 writes per-chunk partial sums to the context workspace, stage 2
// adds the partials in ascending chunk order.  The reference's conv kernel
// lets every block overwrite out[c] with its own partial
// (cuda/kernels/reduce_sum_axis.cu:60-97); this one reduces all of them.
#include "common.hpp"

#include <algorithm>

namespace {

constexpr int kColsPerBlock = 256;  // 64 lanes x float4

// Stage 1 of colsum: block (strip, chunk) sums rows [chunk*rpc, ...) of the
// 256-column strip.  The four waves take interleaved rows; LDS combines them.
__global__ __launch_bounds__(256) void colsum_stage1(const float* __restrict__ dy, float* __restrict__ part,
                                                     int rows, int cols, int rows_per_chunk, int vec) {
    __shared__ float4 red[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c0 = blockIdx.x * kColsPerBlock + 4 * lane;
    const int r0 = blockIdx.y * rows_per_chunk;
    const int r1 = min(rows, r0 + rows_per_chunk);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (vec && c0 + 4 <= cols) {
        for (int r = r0 + wave; r < r1; r += 4) {
            float4 v = *reinterpret_cast<const float4*>(dy + (int64_t)r * cols + c0);
            acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
        }
    } else {
        for (int r = r0 + wave; r < r1; r += 4) {
            const float* row = dy + (int64_t)r * cols;
            if (c0 + 0 < cols) acc.x += row[c0 + 0];
            if (c0 + 1 < cols) acc.y += row[c0 + 1];
            if (c0 + 2 < cols) acc.z += row[c0 + 2];
            if (c0 + 3 < cols) acc.w += row[c0 + 3];
        }
    }
    red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
        float4 a = red[0][lane], b = red[1][lane], c = red[2][lane], d = red[3][lane];
        float4 s = make_float4((a.x + b.x) + (c.x + d.x), (a.y + b.y) + (c.y + d.y),
                               (a.z + b.z) + (c.z + d.z), (a.w + b.w) + (c.w + d.w));
        float* out = part + (int64_t)blockIdx.y * cols;
        if (c0 + 0 < cols) out[c0 + 0] = s.x;
        if (c0 + 1 < cols) out[c0 + 1] = s.y;
        if (c0 + 2 < cols) out[c0 + 2] = s.z;
        if (c0 + 3 < cols) out[c0 + 3] = s.w;
    }
}

// Stage 2 (shared by colsum and chansum): out[c] = sum_k part[k, c].  A block
// owns 64 columns; its 4 waves take chunks k = w, w + 4, ... and LDS adds the
// four wave sums in a fixed order.
__global__ __launch_bounds__(256) void partial_sum_stage2(const float* __restrict__ part, float* __restrict__ out,
                                                          int chunks, int cols) {
    __shared__ float red[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + lane;
    float s = 0.0f;
    if (c < cols)
        for (int k = wave; k < chunks; k += 4) s += part[(int64_t)k * cols + c];
    red[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && c < cols) out[c] = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
}

// Stage 1 of chansum: block (c, chunk) sums samples [chunk*npc, ...) of
// channel c; each (n, c) plane is HW contiguous floats.
__global__ __launch_bounds__(256) void chansum_stage1(const float* __restrict__ dy, float* __restrict__ part,
                                                      int N, int C, int64_t HW, int n_per_chunk, int vec) {
    __shared__ float red[4];
    const int c = blockIdx.x;
    const int n0 = blockIdx.y * n_per_chunk;
    const int n1 = min(N, n0 + n_per_chunk);
    float acc = 0.0f;
    for (int n = n0; n < n1; ++n) {
        const float* plane = dy + ((int64_t)n * C + c) * HW;
        if (vec) {
            for (int64_t i = threadIdx.x; i < HW / 4; i += 256) {
                float4 v = reinterpret_cast<const float4*>(plane)[i];
                acc += (v.x + v.y) + (v.z + v.w);
            }
        } else {
            for (int64_t i = threadIdx.x; i < HW; i += 256) acc += plane[i];
        }
    }
    acc = tfd::wave_sum(acc);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) part[(int64_t)blockIdx.y * C + c] = (red[0] + red[1]) + (red[2] + red[3]);
}

}  // namespace

extern "C" {

tf_status tf_colsum(tf_ctx* ctx, const float* dy, float* db, int64_t rows, int64_t cols) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(rows >= 0 && cols >= 0 && rows < (1LL << 31) && cols < (1LL << 31), "tf_colsum: bad extent");
    if (cols == 0) return TF_OK;
    TF_REQUIRE(db != nullptr && (rows == 0 || dy != nullptr), "tf_colsum: null pointer");
    if (rows == 0) return tf_hip_fill_f32(ctx, db, 0.0f, cols);
    const int strips = (int)((cols + kColsPerBlock - 1) / kColsPerBlock);
    // Aim for ~512 stage-1 blocks (two per CU) with at least 16 rows each.
    int64_t chunks = (512 + strips - 1) / strips;
    chunks = std::min<int64_t>(chunks, (rows + 15) / 16);
    if (chunks < 1) chunks = 1;
    int rpc = (int)((rows + chunks - 1) / chunks);
    chunks = (rows + rpc - 1) / rpc;
    tf_status st = tfh::ensure_workspace(ctx, (size_t)chunks * cols * sizeof(float));
    if (st != TF_OK) return st;
    float* part = reinterpret_cast<float*>(ctx->ws);
    int vec = (reinterpret_cast<uintptr_t>(dy) & 15) == 0 && cols % 4 == 0;
    colsum_stage1<<<dim3(strips, (unsigned)chunks), 256, 0, ctx->stream>>>(dy, part, (int)rows, (int)cols, rpc, vec);
    st = tfh::check_launch("colsum_stage1");
    if (st != TF_OK) return st;
    partial_sum_stage2<<<(unsigned)((cols + 63) / 64), 256, 0, ctx->stream>>>(part, db, (int)chunks, (int)cols);
    return tfh::check_launch("partial_sum_stage2");
}

tf_status tf_chansum_nchw(tf_ctx* ctx, const float* dy, float* db, int64_t N, int64_t C, int64_t HW) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(N >= 0 && C >= 0 && HW >= 0 && N < (1LL << 31) && C < 65536, "tf_chansum_nchw: bad extent");
    if (C == 0) return TF_OK;
    TF_REQUIRE(db != nullptr && (N * HW == 0 || dy != nullptr), "tf_chansum_nchw: null pointer");
    if (N == 0 || HW == 0) return tf_hip_fill_f32(ctx, db, 0.0f, C);
    // Enough (c, chunk) blocks to fill the GPU; each block reads >= 16 KiB.
    int64_t per_plane = HW * 4;
    int64_t n_per_chunk = std::max<int64_t>(1, (16384 + per_plane - 1) / per_plane);
    int64_t chunks = (N + n_per_chunk - 1) / n_per_chunk;
    tf_status st = tfh::ensure_workspace(ctx, (size_t)chunks * C * sizeof(float));
    if (st != TF_OK) return st;
    float* part = reinterpret_cast<float*>(ctx->ws);
    int vec = (reinterpret_cast<uintptr_t>(dy) & 15) == 0 && HW % 4 == 0;
    chansum_stage1<<<dim3((unsigned)C, (unsigned)chunks), 256, 0, ctx->stream>>>(dy, part, (int)N, (int)C, HW,
                                                                                   (int)n_per_chunk, vec);
    st = tfh::check_launch("chansum_stage1");
    if (st != TF_OK) return st;
    partial_sum_stage2<<<(unsigned)((C + 63) / 64), 256, 0, ctx->stream>>>(part, db, (int)chunks, (int)C);
    return tfh::check_launch("partial_sum_stage2");
}

}  // extern "C"
