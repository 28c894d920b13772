// Bias-gradient reductions, deterministic (no atomics, fixed summation order):
//   colsum : db[c] = sum_r dy[r, c]           (Linear bias grad; fp32 or bf16 dy)
//   chansum: db[c] = sum_{n,p} dy[n, c, p]    (Conv2d bias grad, NCHW)
// Colsums over a multiple of 32 columns run as one launch of (strip, chunk)
// blocks whose last arrival per strip adds the chunks.  The others are
// two-stage: stage 1 writes per-chunk partial sums to the context
// workspace, stage 2 (tfh::partial_rows_sum, also used by the LayerNorm
// backward) adds them in a fixed order.  The reference's conv kernel
// lets every block overwrite out[c] with its own partial
// (cuda/kernels/reduce_sum_axis.cu:60-97); this one reduces all of them.
#include "common.hpp"

#include <algorithm>

namespace {

constexpr int kColsPerBlock = 256;  // 64 lanes x float4

// Element loads as fp32: float, or bf16 bit patterns (uint16_t; widening is
// exact, so the bf16 sums equal those of the cast fp32 tensor).
__device__ __forceinline__ float elem_f32(const float* p, int64_t i) { return p[i]; }
__device__ __forceinline__ float elem_f32(const uint16_t* p, int64_t i) { return __uint_as_float((uint32_t)p[i] << 16); }
// Four consecutive elements (16-byte / 8-byte aligned), read once:
// non-temporal loads.
__device__ __forceinline__ float4 vec4_f32(const float* p) { return tfd::ld_nt(reinterpret_cast<const float4*>(p)); }
__device__ __forceinline__ float4 vec4_f32(const uint16_t* p) {
    const uint2 u = tfd::ld_nt(reinterpret_cast<const uint2*>(p));
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                       __uint_as_float(u.y & 0xffff0000u));
}

// Stage 1 of colsum: block (strip, chunk) sums rows [chunk*rpc, ...) of the
// 256-column strip.  The four waves take interleaved rows; LDS combines them.
template <typename T>
__global__ __launch_bounds__(256) void colsum_stage1(const T* __restrict__ dy, float* __restrict__ part,
                                                     int rows, int cols, int rows_per_chunk, int vec) {
    __shared__ float4 red[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c0 = blockIdx.x * kColsPerBlock + 4 * lane;
    const int r0 = blockIdx.y * rows_per_chunk;
    const int r1 = min(rows, r0 + rows_per_chunk);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (vec && c0 + 4 <= cols) {
#pragma unroll 4
        for (int r = r0 + wave; r < r1; r += 4) {
            float4 v = vec4_f32(dy + (int64_t)r * cols + c0);
            acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
        }
    } else {
        for (int r = r0 + wave; r < r1; r += 4) {
            const T* row = dy + (int64_t)r * cols;
            if (c0 + 0 < cols) acc.x += elem_f32(row, c0 + 0);
            if (c0 + 1 < cols) acc.y += elem_f32(row, c0 + 1);
            if (c0 + 2 < cols) acc.z += elem_f32(row, c0 + 2);
            if (c0 + 3 < cols) acc.w += elem_f32(row, c0 + 3);
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

// One-launch colsum over (strip, chunk) blocks: block (s, c) sums rows
// [c rpc, (c + 1) rpc) of the 32-column strip s (a 128-byte line per fp32
// row): 8 lanes per row, 4 columns per lane, 32 row groups taking rows
// g, g + 32, ... in ascending order with sixteen loads in flight, then a
// butterfly across the lanes of a wave that hold the same columns and the
// four waves in order through LDS.  The block stores its 32 sums to
// part[s][c] and counts itself in on the strip's arrival counter; the block
// that arrives last adds the strip's chunks in order 0, 1, ... into db and
// resets the counter.  Partials and counter use agent-scope relaxed atomics
// (coherent across the XCDs' L2s without cache maintenance), and a block's
// stores have completed (vmcnt 0 in every thread, then the barrier) before it
// counts itself in.  Strips are spread XCD by XCD (see the kernel).  Every
// strip's counter sees only `chunks` arrivals, so
// strips finish independently.  fp32 and bf16 inputs of one shape share the
// grid and the order, so their sums are equal for equal values.
constexpr int kTileCols = 32;
constexpr int kTileU = 16;
#ifndef TF_COLSUM_BLOCKS
#define TF_COLSUM_BLOCKS 256
#endif
constexpr int kTileBlocks = TF_COLSUM_BLOCKS;   // (strip, chunk) blocks aimed for
constexpr int kWaitVm0 = 0x0F70;   // s_waitcnt vmcnt(0), other counters free

template <typename T>
__global__ __launch_bounds__(256) void colsum_tile_kernel(const T* __restrict__ dy, float* __restrict__ db,
                                                          float* __restrict__ part, unsigned* __restrict__ tickets,
                                                          int rows, int cols, int rpc, int chunks) {
    __shared__ float4 red[4][8];
    __shared__ bool last;
    // Workgroups go to the 8 XCDs round-robin (block x of a row of the grid
    // on XCD x % 8 when the row length is a multiple of 8): each XCD takes a
    // contiguous range of strips, so strips sharing a cache line (bf16: two
    // 64-byte strips per 128-byte line) share an L2.
    const int strips = gridDim.x;
    const int strip = strips % 8 == 0 ? (blockIdx.x % 8) * (strips / 8) + blockIdx.x / 8 : blockIdx.x;
    const int chunk = blockIdx.y;
    const int cg = threadIdx.x & 7, rg = threadIdx.x >> 3;
    const int c0 = strip * kTileCols + 4 * cg;
    const int r0 = chunk * rpc, r1 = min(rows, r0 + rpc);
    const T* base = dy + c0;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    int r = r0 + rg;
    for (; r + (kTileU - 1) * 32 < r1; r += kTileU * 32) {
        float4 v[kTileU];
#pragma unroll
        for (int u = 0; u < kTileU; ++u) v[u] = vec4_f32(base + (int64_t)(r + 32 * u) * cols);
#pragma unroll
        for (int u = 0; u < kTileU; ++u) {
            acc.x += v[u].x; acc.y += v[u].y; acc.z += v[u].z; acc.w += v[u].w;
        }
    }
    for (; r < r1; r += 32) {
        const float4 v = vec4_f32(base + (int64_t)r * cols);
        acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
#pragma unroll
    for (int off = 8; off < 64; off <<= 1) {
        acc.x += __shfl_xor(acc.x, off, 64);
        acc.y += __shfl_xor(acc.y, off, 64);
        acc.z += __shfl_xor(acc.z, off, 64);
        acc.w += __shfl_xor(acc.w, off, 64);
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane < 8) red[wave][lane] = acc;
    __syncthreads();
    float* mine = part + ((int64_t)strip * chunks + chunk) * kTileCols;
    if (threadIdx.x < 8) {
        const float4 a = red[0][cg], b1 = red[1][cg], c = red[2][cg], d = red[3][cg];
        const float s[4] = {(a.x + b1.x) + (c.x + d.x), (a.y + b1.y) + (c.y + d.y), (a.z + b1.z) + (c.z + d.z),
                            (a.w + b1.w) + (c.w + d.w)};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // One chunk: the block's sums are the result.
            if (chunks == 1) db[c0 + e] = s[e];
            else __hip_atomic_store(mine + 4 * cg + e, s[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (chunks == 1) return;
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(tickets + strip, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (unsigned)(chunks - 1);
    __syncthreads();
    if (!last) return;
    if (threadIdx.x < kTileCols) {
        // The chunks' loads eight at a time in flight, added in chunk order.
        const float* sp = part + (int64_t)strip * chunks * kTileCols + threadIdx.x;
        float v = 0.0f;
        int k = 0;
        for (; k + 8 <= chunks; k += 8) {
            float t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                t[u] = __hip_atomic_load(sp + (int64_t)(k + u) * kTileCols, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int u = 0; u < 8; ++u) v += t[u];
        }
        for (; k < chunks; ++k)
            v += __hip_atomic_load(sp + (int64_t)k * kTileCols, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        db[strip * kTileCols + threadIdx.x] = v;
    }
    if (threadIdx.x == 0) __hip_atomic_store(tickets + strip, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Stage 2 of every two-stage reduction here (colsum, chansum, LayerNorm
// dgamma/dbeta): out[j] = sum_k part[k][j] over a [K][W] partial matrix, the
// first `split` columns to out_lo, the rest to out_hi.  A block owns 16
// columns; its 256 threads are 16 columns x 16 k-groups (a group of 16 lanes
// reads 64 contiguous bytes of one partial row), each thread adds k = g,
// g + 16, ... in ascending order with its loads in flight together, and the
// 16 group sums are added in a fixed tree order (deterministic).
__global__ __launch_bounds__(256) void partial_rows_sum_kernel(const float* __restrict__ part, float* __restrict__ out_lo,
                                                           float* __restrict__ out_hi, int K, int W, int split) {
    __shared__ float red[16][17];
    const int cl = threadIdx.x & 15, kg = threadIdx.x >> 4;
    const int j = blockIdx.x * 16 + cl;
    float s = 0.0f;
    if (j < W) {
#pragma unroll 8
        for (int k = kg; k < K; k += 16) s += part[(int64_t)k * W + j];
    }
    red[kg][cl] = s;
    __syncthreads();
    if (threadIdx.x < 16 && j < W) {
        float t[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = red[2 * i][cl] + red[2 * i + 1][cl];
        const float v = ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
        if (j < split) out_lo[j] = v;
        else out_hi[j - split] = v;
    }
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

namespace tfh {

tf_status partial_rows_sum(tf_ctx* ctx, const float* part, float* out_lo, float* out_hi, int64_t K, int64_t W,
                           int64_t split) {
    if (W == 0) return TF_OK;
    partial_rows_sum_kernel<<<(unsigned)((W + 15) / 16), 256, 0, ctx->stream>>>(part, out_lo, out_hi, (int)K, (int)W,
                                                                               (int)split);
    return check_launch("partial_rows_sum_kernel");
}

}  // namespace tfh

namespace {

template <typename T>
tf_status colsum_impl(tf_ctx* ctx, const T* dy, float* db, int64_t rows, int64_t cols) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(rows >= 0 && cols >= 0 && rows < (1LL << 31) && cols < (1LL << 31), "tf_colsum: bad extent");
    if (cols == 0) return TF_OK;
    TF_REQUIRE(db != nullptr && (rows == 0 || dy != nullptr), "tf_colsum: null pointer");
    if (rows == 0) return tf_hip_fill_f32(ctx, db, 0.0f, cols);
    const int vec = (reinterpret_cast<uintptr_t>(dy) & (4 * sizeof(T) - 1)) == 0 && cols % 4 == 0;
    // Widths in 32-column strips: one launch of (strip, chunk) blocks, about
    // kTileBlocks of them, with the last block of each strip adding its chunks.
    const int64_t tstrips = cols / kTileCols;
    if (vec && cols % kTileCols == 0 && tstrips <= tfh::kTicketColsumStrips) {
        int64_t chunks = std::max<int64_t>(1, std::min<int64_t>((kTileBlocks + tstrips - 1) / tstrips, (rows + 31) / 32));
        const int rpc = (int)((rows + chunks - 1) / chunks);
        chunks = (rows + rpc - 1) / rpc;
        tf_status st = tfh::ensure_workspace(ctx, (size_t)tstrips * chunks * kTileCols * sizeof(float));
        if (st != TF_OK) return st;
        colsum_tile_kernel<T><<<dim3((unsigned)tstrips, (unsigned)chunks), 256, 0, ctx->stream>>>(
            dy, db, reinterpret_cast<float*>(ctx->ws), ctx->tickets + tfh::kTicketColsum, (int)rows, (int)cols, rpc,
            (int)chunks);
        return tfh::check_launch("colsum_tile_kernel");
    }
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
    colsum_stage1<T><<<dim3(strips, (unsigned)chunks), 256, 0, ctx->stream>>>(dy, part, (int)rows, (int)cols, rpc,
                                                                             vec);
    st = tfh::check_launch("colsum_stage1");
    if (st != TF_OK) return st;
    return tfh::partial_rows_sum(ctx, part, db, nullptr, chunks, cols, cols);
}

}  // namespace

extern "C" {

tf_status tf_colsum(tf_ctx* ctx, const float* dy, float* db, int64_t rows, int64_t cols) {
    return colsum_impl(ctx, dy, db, rows, cols);
}

tf_status tf_colsum_bf16(tf_ctx* ctx, const void* dy, float* db, int64_t rows, int64_t cols) {
    return colsum_impl(ctx, static_cast<const uint16_t*>(dy), db, rows, cols);
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
    return tfh::partial_rows_sum(ctx, part, db, nullptr, chunks, C, C);
}

}  // extern "C"
