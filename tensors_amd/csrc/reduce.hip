// Bias-gradient reductions, deterministic (no atomics, fixed summation order):
//   colsum : db[c] = sum_r dy[r, c]           (Linear bias grad; fp32 or bf16 dy)
//   chansum: db[c] = sum_{n,p} dy[n, c, p]    (Conv2d bias grad, NCHW)
// Colsums over a multiple of 4 columns run as one launch of (strip, chunk)
// blocks whose last arrival per strip adds the chunks; small ones as one
// block.  The others are two-stage: stage 1 writes per-chunk partial sums to the context
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
constexpr int kTileLanes = kTileCols / 4;     // lanes per row segment (4 columns each)
constexpr int kTileRG = 256 / kTileLanes;      // row groups per block
constexpr int kTileU = 16;
#ifndef TF_COLSUM_BLOCKS
#define TF_COLSUM_BLOCKS 256
#endif
constexpr int kTileBlocks = TF_COLSUM_BLOCKS;   // (strip, chunk) blocks aimed for

template <typename T>
__global__ __launch_bounds__(256) void colsum_tile_kernel(const T* __restrict__ dy, float* __restrict__ db,
                                                          float* __restrict__ part, unsigned* __restrict__ tickets,
                                                          int rows, int cols, int rpc, int chunks) {
    __shared__ float4 red[4][kTileLanes];
    __shared__ bool last;
    // Workgroups go to the 8 XCDs round-robin (block x of a row of the grid
    // on XCD x % 8 when the row length is a multiple of 8): each XCD takes a
    // contiguous range of strips, so strips sharing a cache line (bf16: two
    // 64-byte strips per 128-byte line) share an L2.
    const int strips = gridDim.x;
    const int strip = strips % 8 == 0 ? (blockIdx.x % 8) * (strips / 8) + blockIdx.x / 8 : blockIdx.x;
    const int chunk = blockIdx.y;
    const int cg = threadIdx.x % kTileLanes, rg = threadIdx.x / kTileLanes;
    const int c0 = strip * kTileCols + 4 * cg;
    // cols % 4 == 0: a lane's four columns are all inside or all past the
    // last (ragged) strip's end.
    const int r0 = chunk * rpc, r1 = c0 < cols ? min(rows, r0 + rpc) : r0;
    const T* base = dy + c0;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    int r = r0 + rg;
    for (; r + (kTileU - 1) * kTileRG < r1; r += kTileU * kTileRG) {
        float4 v[kTileU];
#pragma unroll
        for (int u = 0; u < kTileU; ++u) v[u] = vec4_f32(base + (int64_t)(r + kTileRG * u) * cols);
#pragma unroll
        for (int u = 0; u < kTileU; ++u) {
            acc.x += v[u].x; acc.y += v[u].y; acc.z += v[u].z; acc.w += v[u].w;
        }
    }
    for (; r < r1; r += kTileRG) {
        const float4 v = vec4_f32(base + (int64_t)r * cols);
        acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
#pragma unroll
    for (int off = kTileLanes; off < 64; off <<= 1) {
        acc.x += __shfl_xor(acc.x, off, 64);
        acc.y += __shfl_xor(acc.y, off, 64);
        acc.z += __shfl_xor(acc.z, off, 64);
        acc.w += __shfl_xor(acc.w, off, 64);
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane < kTileLanes) red[wave][lane] = acc;
    __syncthreads();
    float* mine = part + ((int64_t)strip * chunks + chunk) * kTileCols;
    if (threadIdx.x < kTileLanes) {
        const float4 a = red[0][cg], b1 = red[1][cg], c = red[2][cg], d = red[3][cg];
        const float s[4] = {(a.x + b1.x) + (c.x + d.x), (a.y + b1.y) + (c.y + d.y), (a.z + b1.z) + (c.z + d.z),
                            (a.w + b1.w) + (c.w + d.w)};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // One chunk: the block's sums are the result.
            if (chunks == 1) {
                if (c0 < cols) db[c0 + e] = s[e];
            } else {
                __hip_atomic_store(mine + 4 * cg + e, s[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    if (chunks == 1) return;
    tfd::wait_stores_landed();
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(tickets + strip, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (unsigned)(chunks - 1);
    __syncthreads();
    if (!last) return;
    if (threadIdx.x < kTileCols && strip * kTileCols + (int)threadIdx.x < cols) {
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

// ReLU backward fused with the column sum of its result
// (tf_relu_bwd_colsum): dz = dy * (x > 0 ? 1 : 0) in fp32, rounded to T and
// stored; db[c] = sum_r dz[r, c] over the stored values.  Streaming layout:
// block (s, k) owns the 256-column strip s (a lane per 4 columns, so a wave
// reads and writes 512 / 1024 contiguous bytes of a row) and the kRcRows
// rows of chunk k, which its four waves take interleaved (r0 + w,
// r0 + w + 4, ...), eight rows' loads in flight per wave.  The waves' sums
// are added in order through LDS; with several chunks the block stores its
// 256 sums with agent-scope stores and counts in on the strip's counter, and
// the last block of the strip adds the chunks in order (deterministic) and
// resets the counter, as in colsum_tile_kernel.  Measured at the C5 shapes
// (bf16, buffers past the cache): 4096 x 8192 in 38 us against 51 us for
// tf_relu_bwd + tf_colsum_bf16, 4096 x 4096 in 27 against 29; lanes of 16
// bytes (8 bf16 columns) were slower at 4096 x 8192 (43-52 us).
template <typename T> struct Raw4;   // four consecutive elements as loaded
template <> struct Raw4<float> { using type = float4; };
template <> struct Raw4<uint16_t> { using type = uint2; };
__device__ __forceinline__ float4 ld_raw4(const float* p) { return tfd::ld_nt(reinterpret_cast<const float4*>(p)); }
__device__ __forceinline__ uint2 ld_raw4(const uint16_t* p) { return tfd::ld_nt(reinterpret_cast<const uint2*>(p)); }
__device__ __forceinline__ float4 widen4(const float4 v) { return v; }
__device__ __forceinline__ float4 widen4(const uint2 u) {
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                       __uint_as_float(u.y & 0xffff0000u));
}
__device__ __forceinline__ float relu_mask(float x) { return x > 0.0f ? 1.0f : 0.0f; }
// The rule of tf_relu_bwd on four elements; returns the stored values in fp32.
__device__ __forceinline__ float4 relu_bwd4(const float4 g, const float4 x, float* dz) {
    const float4 o = make_float4(g.x * relu_mask(x.x), g.y * relu_mask(x.y), g.z * relu_mask(x.z), g.w * relu_mask(x.w));
    tfd::st_nt(reinterpret_cast<float4*>(dz), o);
    return o;
}
__device__ __forceinline__ float4 relu_bwd4(const uint2 g16, const uint2 x16, uint16_t* dz) {
    const float4 g = widen4(g16), x = widen4(x16);
    const uint2 o = make_uint2(tfd::bf16x2_rne(g.x * relu_mask(x.x), g.y * relu_mask(x.y)),
                               tfd::bf16x2_rne(g.z * relu_mask(x.z), g.w * relu_mask(x.w)));
    tfd::st_nt(reinterpret_cast<uint2*>(dz), o);
    return widen4(o);
}

constexpr int kRcCols = 256;   // columns per strip (64 lanes x 4)
constexpr int kRcU = 8;        // rows in flight per wave
constexpr int kRcRows = 128;   // rows per chunk (64 and 256 measured slower at the C5 shapes)
constexpr int kRcMaxBlocks = 4096;

template <typename T>
__global__ __launch_bounds__(256) void relu_bwd_colsum_kernel(const T* __restrict__ dy, const T* __restrict__ x,
                                                              T* __restrict__ dz, float* __restrict__ db,
                                                              float* __restrict__ part, unsigned* __restrict__ tickets,
                                                              int rows, int cols, int rpc, int chunks) {
    using R4 = typename Raw4<T>::type;
    __shared__ float4 red[4][64];
    __shared__ bool last;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int strip = blockIdx.x, chunk = blockIdx.y;
    const int c = strip * kRcCols + 4 * lane;
    const bool on = c < cols;   // cols % 4 == 0: a lane's 4 columns are all in or all out
    const int r0 = chunk * rpc, r1 = min(rows, r0 + rpc);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (on) {
        int r = r0 + wave;
        for (; r + 4 * (kRcU - 1) < r1; r += 4 * kRcU) {
            R4 g[kRcU], m[kRcU];
#pragma unroll
            for (int u = 0; u < kRcU; ++u) {
                const int64_t off = (int64_t)(r + 4 * u) * cols + c;
                g[u] = ld_raw4(dy + off);
                m[u] = ld_raw4(x + off);
            }
#pragma unroll
            for (int u = 0; u < kRcU; ++u) {
                const float4 f = relu_bwd4(g[u], m[u], dz + (int64_t)(r + 4 * u) * cols + c);
                acc.x += f.x; acc.y += f.y; acc.z += f.z; acc.w += f.w;
            }
        }
        for (; r < r1; r += 4) {
            const int64_t off = (int64_t)r * cols + c;
            const float4 f = relu_bwd4(ld_raw4(dy + off), ld_raw4(x + off), dz + off);
            acc.x += f.x; acc.y += f.y; acc.z += f.z; acc.w += f.w;
        }
    }
    red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && on) {
        const float4 a = red[0][lane], b1 = red[1][lane], c2 = red[2][lane], d = red[3][lane];
        const float sum[4] = {(a.x + b1.x) + (c2.x + d.x), (a.y + b1.y) + (c2.y + d.y), (a.z + b1.z) + (c2.z + d.z),
                              (a.w + b1.w) + (c2.w + d.w)};
        float* mine = part + ((int64_t)strip * chunks + chunk) * kRcCols + 4 * lane;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (chunks == 1) db[c + e] = sum[e];
            else __hip_atomic_store(mine + e, sum[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (chunks == 1) return;
    tfd::wait_stores_landed();
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(tickets + strip, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (unsigned)(chunks - 1);
    __syncthreads();
    if (!last) return;
    // A thread per column of the strip: the chunks' sums eight loads at a
    // time in flight, added in chunk order.
    const int col = strip * kRcCols + threadIdx.x;
    if (col < cols) {
        const float* sp = part + (int64_t)strip * chunks * kRcCols + threadIdx.x;
        float v = 0.0f;
        int k = 0;
        for (; k + 8 <= chunks; k += 8) {
            float t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                t[u] = __hip_atomic_load(sp + (int64_t)(k + u) * kRcCols, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int u = 0; u < 8; ++u) v += t[u];
        }
        for (; k < chunks; ++k)
            v += __hip_atomic_load(sp + (int64_t)k * kRcCols, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        db[col] = v;
    }
    if (threadIdx.x == 0) __hip_atomic_store(tickets + strip, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Small colsums (cols <= 256, rows * cols <= kSmallColsum) in one block: the
// 256 threads are cols columns x G = 256 / cols row groups; thread (c, g)
// adds rows g, g + G, ... of column c in ascending order (eight loads in
// flight), and thread c adds the G group sums in order.  One launch where
// the two-stage path takes two (C4's 10-wide classifier bias).
constexpr int64_t kSmallColsum = 1 << 16;
template <typename T>
__global__ __launch_bounds__(256) void colsum_small_kernel(const T* __restrict__ dy, float* __restrict__ db, int rows,
                                                           int cols) {
    __shared__ float red[256];
    const int G = 256 / cols;
    const int c = threadIdx.x % cols, g = threadIdx.x / cols;
    float s = 0.0f;
    if (g < G) {
        int r = g;
        for (; r + 7 * G < rows; r += 8 * G) {
            float t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) t[u] = elem_f32(dy, (int64_t)(r + u * G) * cols + c);
#pragma unroll
            for (int u = 0; u < 8; ++u) s += t[u];
        }
        for (; r < rows; r += G) s += elem_f32(dy, (int64_t)r * cols + c);
    }
    red[threadIdx.x] = s;
    __syncthreads();
    if ((int)threadIdx.x < cols) {
        float v = 0.0f;
        for (int k = 0; k < G; ++k) v += red[k * cols + threadIdx.x];
        db[threadIdx.x] = v;
    }
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
    // 32-column strips (the last one ragged): one launch of (strip, chunk)
    // blocks, about kTileBlocks of them, with the last block of each strip
    // adding its chunks.  vec implies cols % 4 == 0.
    const int64_t tstrips = (cols + kTileCols - 1) / kTileCols;
    if (vec && tstrips <= tfh::kTicketColsumStrips) {
        int64_t chunks = std::max<int64_t>(1, std::min<int64_t>((kTileBlocks + tstrips - 1) / tstrips,
                                                                (rows + kTileRG - 1) / kTileRG));
        const int rpc = (int)((rows + chunks - 1) / chunks);
        chunks = (rows + rpc - 1) / rpc;
        tf_status st = tfh::ensure_workspace(ctx, (size_t)tstrips * chunks * kTileCols * sizeof(float));
        if (st != TF_OK) return st;
        colsum_tile_kernel<T><<<dim3((unsigned)tstrips, (unsigned)chunks), 256, 0, ctx->stream>>>(
            dy, db, reinterpret_cast<float*>(ctx->ws), ctx->tickets + tfh::kTicketColsum, (int)rows, (int)cols, rpc,
            (int)chunks);
        return tfh::check_launch("colsum_tile_kernel");
    }
    if (cols <= 256 && rows * cols <= kSmallColsum) {
        colsum_small_kernel<T><<<1, 256, 0, ctx->stream>>>(dy, db, (int)rows, (int)cols);
        return tfh::check_launch("colsum_small_kernel");
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

// dz = relu_bwd(dy, x) and db = colsum(dz): one launch of
// relu_bwd_colsum_kernel where its layout applies, else tf_relu_bwd followed
// by the colsum.
template <typename T>
tf_status relu_bwd_colsum_impl(tf_ctx* ctx, const T* dy, const T* x, T* dz, float* db, int64_t rows, int64_t cols,
                               int dtype) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(rows >= 0 && cols >= 0 && rows < (1LL << 31) && cols < (1LL << 31), "tf_relu_bwd_colsum: bad extent");
    if (cols == 0) return TF_OK;
    TF_REQUIRE(db != nullptr && (rows == 0 || (dy && x && dz)), "tf_relu_bwd_colsum: null pointer");
    if (rows == 0) return tf_hip_fill_f32(ctx, db, 0.0f, cols);
    constexpr uintptr_t amask = 4 * sizeof(T) - 1;   // a lane's 4 elements in one access
    const bool vec = ((reinterpret_cast<uintptr_t>(dy) | reinterpret_cast<uintptr_t>(x) |
                       reinterpret_cast<uintptr_t>(dz)) & amask) == 0 && cols % 4 == 0;
    const int64_t strips = (cols + kRcCols - 1) / kRcCols;
    if (vec && strips <= tfh::kTicketColsumStrips) {
        // Chunks of kRcRows rows, fewer when that would exceed kRcMaxBlocks
        // blocks.
        int64_t chunks = std::max<int64_t>(1, std::min<int64_t>((rows + kRcRows - 1) / kRcRows,
                                                                (kRcMaxBlocks + strips - 1) / strips));
        const int rpc = (int)((rows + chunks - 1) / chunks);
        chunks = (rows + rpc - 1) / rpc;
        TF_REQUIRE(chunks <= 65535, "tf_relu_bwd_colsum: too many row chunks");
        tf_status st = tfh::ensure_workspace(ctx, (size_t)strips * chunks * kRcCols * sizeof(float));
        if (st != TF_OK) return st;
        relu_bwd_colsum_kernel<T><<<dim3((unsigned)strips, (unsigned)chunks), 256, 0, ctx->stream>>>(
            dy, x, dz, db, reinterpret_cast<float*>(ctx->ws), ctx->tickets + tfh::kTicketColsum, (int)rows, (int)cols,
            rpc, (int)chunks);
        return tfh::check_launch("relu_bwd_colsum_kernel");
    }
    tf_status st = tf_relu_bwd(ctx, dy, x, dz, rows * cols, dtype);
    if (st != TF_OK) return st;
    return colsum_impl(ctx, static_cast<const T*>(dz), db, rows, cols);
}

}  // namespace

extern "C" {

tf_status tf_relu_bwd_colsum(tf_ctx* ctx, const void* dy, const void* x, void* dz, float* db, int64_t rows,
                             int64_t cols, int dtype) {
    if (dtype == TF_F32)
        return relu_bwd_colsum_impl(ctx, static_cast<const float*>(dy), static_cast<const float*>(x),
                                    static_cast<float*>(dz), db, rows, cols, dtype);
    if (dtype == TF_BF16)
        return relu_bwd_colsum_impl(ctx, static_cast<const uint16_t*>(dy), static_cast<const uint16_t*>(x),
                                    static_cast<uint16_t*>(dz), db, rows, cols, dtype);
    return tfh::set_error(TF_ERR_UNSUPPORTED, "tf_relu_bwd_colsum: dtype must be Float32 or BFloat16");
}

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
