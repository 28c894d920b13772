// LayerNorm forward and backward over the last dimension.
//
// Forward (tensor/Tensor.cpp:449-494): two-pass mean / variance per row,
// y = (x - mean) * rstd * gamma + beta, saving mean and rstd.
//
// Backward, true gradient (the reference ships only a stub,
// autograd/ops/LayerNormBackward.hpp:39-59):
//   xhat = (x - mean) * rstd,  g = dy * gamma
//   dx   = rstd * (g - mean_j(g) - xhat * mean_j(g * xhat))
//   dgamma[j] = sum_r dy * xhat,  dbeta[j] = sum_r dy
// Reference-compatible mode reproduces the stub exactly: dx = dy * gamma,
// dgamma = dbeta = 0.
//
// Rows of up to 2048 columns whose width is a multiple of 32 (16-byte rows):
// one launch, row blocks for dx beside (strip, chunk) blocks for
// dgamma/dbeta (ln_bwd_onepass_kernel).  Other rows of up to 2048 columns:
// one fused pass (one wave per row, the row held in registers; each wave
// also accumulates its rows' dgamma/dbeta column partials, combined per block
// in LDS and then across blocks by a fixed-order column-strip reduction).
// Wider rows: a streaming row kernel for dx and a column kernel for
// dgamma/dbeta.
#include "common.hpp"

#include <algorithm>
#include <cmath>

namespace {

constexpr int kMaxCached = 8;  // 8 x 256 columns

__device__ __forceinline__ int col_of(int c, int lane, int q, bool vec) {
    return vec ? 256 * c + 4 * lane + q : 256 * c + lane + 64 * q;
}

// Whole rows held in registers, read and written once: non-temporal vector
// accesses.
template <int NC, bool NT = true>
__device__ __forceinline__ void load_row(const float* __restrict__ row, int cols, int lane, bool vec,
                                         float (&v)[NC][4]) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        int base = 256 * c + 4 * lane;
        if (vec && base + 4 <= cols) {
            const float4 t = NT ? tfd::ld_nt(reinterpret_cast<const float4*>(row + base))
                                : *reinterpret_cast<const float4*>(row + base);
            v[c][0] = t.x; v[c][1] = t.y; v[c][2] = t.z; v[c][3] = t.w;
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                int j = col_of(c, lane, q, vec);
                v[c][q] = j < cols ? row[j] : 0.0f;
            }
        }
    }
}

template <int NC>
__device__ __forceinline__ void store_row(float* __restrict__ row, int cols, int lane, bool vec,
                                          const float (&v)[NC][4]) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        int base = 256 * c + 4 * lane;
        if (vec && base + 4 <= cols) {
            tfd::st_nt(reinterpret_cast<float4*>(row + base), make_float4(v[c][0], v[c][1], v[c][2], v[c][3]));
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                int j = col_of(c, lane, q, vec);
                if (j < cols) row[j] = v[c][q];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Forward.  Grid-stride over rows, one wave per row.
// ---------------------------------------------------------------------------
template <int NC>
__global__ __launch_bounds__(256) void ln_fwd_kernel(const float* __restrict__ x, const float* __restrict__ gamma,
                                                     const float* __restrict__ beta, float* __restrict__ y,
                                                     float* __restrict__ mean, float* __restrict__ rstd, int rows,
                                                     int cols, float eps, int vec) {
    const int lane = threadIdx.x & 63;
    const int wave_id = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int n_waves = gridDim.x * 4;
    const float inv_c = 1.0f / (float)cols;
    for (int r = wave_id; r < rows; r += n_waves) {
        const float* xr = x + (int64_t)r * cols;
        float v[NC][4];
        load_row<NC>(xr, cols, lane, vec, v);
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) s += v[c][q];
        const float m = tfd::wave_sum(s) * inv_c;
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int j = col_of(c, lane, q, vec);
                const float d = j < cols ? v[c][q] - m : 0.0f;
                ss += d * d;
            }
        const float var = tfd::wave_sum(ss) * inv_c;
        const float rs = 1.0f / sqrtf(var + eps);
        if (lane == 0) {
            mean[r] = m;
            rstd[r] = rs;
        }
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int j = col_of(c, lane, q, vec);
                v[c][q] = j < cols ? (v[c][q] - m) * rs * gamma[j] + beta[j] : 0.0f;
            }
        store_row<NC>(y + (int64_t)r * cols, cols, lane, vec, v);
    }
}

// Streaming forward for rows wider than the register cache.
__global__ __launch_bounds__(256) void ln_fwd_stream_kernel(const float* __restrict__ x, const float* __restrict__ gamma,
                                                            const float* __restrict__ beta, float* __restrict__ y,
                                                            float* __restrict__ mean, float* __restrict__ rstd,
                                                            int rows, int cols, float eps) {
    const int lane = threadIdx.x & 63;
    const int wave_id = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int n_waves = gridDim.x * 4;
    const float inv_c = 1.0f / (float)cols;
    for (int r = wave_id; r < rows; r += n_waves) {
        const float* xr = x + (int64_t)r * cols;
        float s = 0.0f;
        for (int j = lane; j < cols; j += 64) s += xr[j];
        const float m = tfd::wave_sum(s) * inv_c;
        float ss = 0.0f;
        for (int j = lane; j < cols; j += 64) {
            float d = xr[j] - m;
            ss += d * d;
        }
        const float rs = 1.0f / sqrtf(tfd::wave_sum(ss) * inv_c + eps);
        if (lane == 0) {
            mean[r] = m;
            rstd[r] = rs;
        }
        float* yr = y + (int64_t)r * cols;
        for (int j = lane; j < cols; j += 64) yr[j] = (xr[j] - m) * rs * gamma[j] + beta[j];
    }
}

// ---------------------------------------------------------------------------
// Fused backward for cols <= 256 * NC.  Block b (WAVES waves) handles rows
// [b * rpb, (b+1) * rpb); each wave takes every WAVES-th of them.  Column
// partial sums of dy * xhat and dy go to part[b][0][:] and part[b][1][:].
// ---------------------------------------------------------------------------
template <int NC, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void ln_bwd_fused_kernel(const float* __restrict__ dy,
                                                                  const float* __restrict__ x,
                                                                  const float* __restrict__ gamma,
                                                                  const float* __restrict__ mean,
                                                                  const float* __restrict__ rstd, float* __restrict__ dx,
                                                                  float* __restrict__ part, int rows, int cols,
                                                                  int rows_per_block, int vec) {
    __shared__ float red[WAVES][2][NC * 256];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = blockIdx.x * rows_per_block;
    const int r1 = min(rows, r0 + rows_per_block);
    const float inv_c = 1.0f / (float)cols;
    float gacc[NC][4], bacc[NC][4];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) gacc[c][q] = bacc[c][q] = 0.0f;
    float gm[NC][4];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int j = col_of(c, lane, q, vec);
            gm[c][q] = j < cols ? gamma[j] : 0.0f;
        }
    for (int r = r0 + wave; r < r1; r += WAVES) {
        float xv[NC][4], gv[NC][4];
        load_row<NC>(x + (int64_t)r * cols, cols, lane, vec, xv);
        load_row<NC>(dy + (int64_t)r * cols, cols, lane, vec, gv);
        const float m = mean[r], rs = rstd[r];
        float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float xh = (xv[c][q] - m) * rs;
                const float g = gv[c][q] * gm[c][q];
                s1 += g;
                s2 += g * xh;
                gacc[c][q] += gv[c][q] * xh;
                bacc[c][q] += gv[c][q];
                xv[c][q] = xh;
            }
        s1 = tfd::wave_sum(s1) * inv_c;
        s2 = tfd::wave_sum(s2) * inv_c;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float g = gv[c][q] * gm[c][q];
                xv[c][q] = rs * (g - s1 - xv[c][q] * s2);
            }
        store_row<NC>(dx + (int64_t)r * cols, cols, lane, vec, xv);
    }
    // Block combine of the waves' column partials (fixed order).
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int slot = 256 * c + 4 * lane + q;   // storage slot, not column
            red[wave][0][slot] = gacc[c][q];
            red[wave][1][slot] = bacc[c][q];
        }
    __syncthreads();
    for (int slot = threadIdx.x; slot < NC * 256; slot += WAVES * 64) {
        const int c = slot / 256, rem = slot % 256, l = rem / 4, q = rem % 4;
        const int j = col_of(c, l, q, vec);
        if (j >= cols) continue;
        float* pg = part + (int64_t)blockIdx.x * 2 * cols;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float t = red[0][h][slot];
#pragma unroll
            for (int w = 1; w < WAVES; ++w) t += red[w][h][slot];
            pg[h * cols + j] = t;
        }
    }
}

// ---------------------------------------------------------------------------
// One launch for rows of up to 2048 columns (16-byte rows, cols % 32 == 0).
// dgamma / dbeta need only x, dy and the saved mean / rstd, not the row
// pass, so they are computed beside it instead of after it: blocks
// [0, row_blocks) compute dx (a wave per row, as ln_bwd_fused_kernel, without
// column partials), and each block after them sums a 32-column strip over a
// chunk of rpc rows: 8 lanes x 4 columns per row, 32 row groups taking rows
// g, g + 32, ... in ascending order (four rows' loads in flight), a
// butterfly across the lanes holding the same columns, the four waves in
// order through LDS.  It stores its 2 x 32 sums with agent-scope stores
// and counts in on the strip's counter; the strip's last block adds the
// chunks in order (deterministic) and resets the counter.  Both kinds read
// x and dy with plain loads, so the second reader mostly hits the caches.
// ---------------------------------------------------------------------------
constexpr int kLnStrip = 32;
#ifndef TF_LN_COL_BLOCKS
#define TF_LN_COL_BLOCKS 256
#endif
constexpr int kLnColBlocks = TF_LN_COL_BLOCKS;   // (strip, chunk) blocks aimed for
#ifndef TF_LN_COL_U
#define TF_LN_COL_U 4
#endif

template <int NC>
__global__ __launch_bounds__(256) void ln_bwd_onepass_kernel(const float* __restrict__ dy, const float* __restrict__ x,
                                                             const float* __restrict__ gamma,
                                                             const float* __restrict__ mean,
                                                             const float* __restrict__ rstd, float* __restrict__ dx,
                                                             float* __restrict__ dgamma, float* __restrict__ dbeta,
                                                             float* __restrict__ part, unsigned* __restrict__ tickets,
                                                             int rows, int cols, int rows_per_block, int row_blocks,
                                                             int strips, int rpc, int chunks) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // Workgroups go to the 8 XCDs round-robin (block b to XCD b % 8).  When
    // the counts allow, XCD x gets the row blocks of one contiguous eighth of
    // the rows and the column blocks of the chunks inside that eighth, so a
    // row's second reader finds it in the XCD's own L2.
    const bool xcd_map = (row_blocks & 7) == 0 && (chunks & 7) == 0;
    // The column blocks come first in the grid: their chain (loads, partial
    // stores, the strip counter, the last block's loads) is longer than a
    // row block's, so they are dispatched before the row blocks (6.8 ->
    // 6.6 us at 1024 x 1024).  bidx numbers row blocks from 0, then the
    // column blocks.
    const int ncol = strips * chunks;
    const int bidx = (int)blockIdx.x < ncol ? (int)blockIdx.x + row_blocks : (int)blockIdx.x - ncol;
    if (bidx < row_blocks) {
        const int rb = xcd_map ? (bidx & 7) * (row_blocks >> 3) + (bidx >> 3) : bidx;
        const int r0 = rb * rows_per_block, r1 = min(rows, r0 + rows_per_block);
        const float inv_c = 1.0f / (float)cols;
        float gm[NC][4];
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int j = col_of(c, lane, q, true);
                gm[c][q] = j < cols ? gamma[j] : 0.0f;
            }
        for (int r = r0 + wave; r < r1; r += 4) {
            float xv[NC][4], gv[NC][4];
            load_row<NC, false>(x + (int64_t)r * cols, cols, lane, true, xv);
            load_row<NC, false>(dy + (int64_t)r * cols, cols, lane, true, gv);
            const float m = mean[r], rs = rstd[r];
            float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float xh = (xv[c][q] - m) * rs;
                    const float g = gv[c][q] * gm[c][q];
                    s1 += g;
                    s2 += g * xh;
                    xv[c][q] = xh;
                }
            s1 = tfd::wave_sum(s1) * inv_c;
            s2 = tfd::wave_sum(s2) * inv_c;
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int q = 0; q < 4; ++q) xv[c][q] = rs * (gv[c][q] * gm[c][q] - s1 - xv[c][q] * s2);
            store_row<NC>(dx + (int64_t)r * cols, cols, lane, true, xv);
        }
        return;
    }
    __shared__ float4 red[4][2][8];
    __shared__ bool last;
    const int tb = bidx - row_blocks;
    int strip, chunk;
    if (xcd_map) {
        const int k = chunks >> 3, idx = tb >> 3;
        chunk = (tb & 7) * k + idx % k;
        strip = idx / k;
    } else {
        strip = tb % strips;
        chunk = tb / strips;
    }
    const int cg = threadIdx.x & 7, rg = threadIdx.x >> 3;
    const int c0 = strip * kLnStrip + 4 * cg;
    const int r0 = chunk * rpc, r1 = min(rows, r0 + rpc);
    float4 ag = make_float4(0.f, 0.f, 0.f, 0.f), ab = ag;
    auto add_row = [&](const float4 xv, const float4 dv, float m, float rs) {
        ag.x += dv.x * ((xv.x - m) * rs); ag.y += dv.y * ((xv.y - m) * rs);
        ag.z += dv.z * ((xv.z - m) * rs); ag.w += dv.w * ((xv.w - m) * rs);
        ab.x += dv.x; ab.y += dv.y; ab.z += dv.z; ab.w += dv.w;
    };
    int r = r0 + rg;
    constexpr int CU = TF_LN_COL_U;   // rows' loads in flight per thread
    for (; r + (CU - 1) * 32 < r1; r += CU * 32) {
        float4 xv[CU], dv[CU];
        float m[CU], rs[CU];
#pragma unroll
        for (int u = 0; u < CU; ++u) {
            const int64_t off = (int64_t)(r + 32 * u) * cols + c0;
            xv[u] = *reinterpret_cast<const float4*>(x + off);
            dv[u] = *reinterpret_cast<const float4*>(dy + off);
            m[u] = mean[r + 32 * u];
            rs[u] = rstd[r + 32 * u];
        }
#pragma unroll
        for (int u = 0; u < CU; ++u) add_row(xv[u], dv[u], m[u], rs[u]);
    }
    for (; r < r1; r += 32) {
        const int64_t off = (int64_t)r * cols + c0;
        add_row(*reinterpret_cast<const float4*>(x + off), *reinterpret_cast<const float4*>(dy + off), mean[r],
                rstd[r]);
    }
#pragma unroll
    for (int off = 8; off < 64; off <<= 1) {
        ag.x += __shfl_xor(ag.x, off, 64); ag.y += __shfl_xor(ag.y, off, 64);
        ag.z += __shfl_xor(ag.z, off, 64); ag.w += __shfl_xor(ag.w, off, 64);
        ab.x += __shfl_xor(ab.x, off, 64); ab.y += __shfl_xor(ab.y, off, 64);
        ab.z += __shfl_xor(ab.z, off, 64); ab.w += __shfl_xor(ab.w, off, 64);
    }
    if (lane < 8) {
        red[wave][0][lane] = ag;
        red[wave][1][lane] = ab;
    }
    __syncthreads();
    float* mine = part + ((int64_t)strip * chunks + chunk) * 2 * kLnStrip;
    if (threadIdx.x < 16) {
        const int h = threadIdx.x >> 3, q = threadIdx.x & 7;
        const float4 a = red[0][h][q], b1 = red[1][h][q], c = red[2][h][q], d = red[3][h][q];
        const float v[4] = {(a.x + b1.x) + (c.x + d.x), (a.y + b1.y) + (c.y + d.y), (a.z + b1.z) + (c.z + d.z),
                            (a.w + b1.w) + (c.w + d.w)};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (chunks == 1) (h ? dbeta : dgamma)[strip * kLnStrip + 4 * q + e] = v[e];
            else __hip_atomic_store(mine + h * kLnStrip + 4 * q + e, v[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
    if (threadIdx.x < 2 * kLnStrip) {
        // The chunks' sums eight loads at a time in flight, added in order.
        const float* sp = part + (int64_t)strip * chunks * 2 * kLnStrip + threadIdx.x;
        float v = 0.0f;
        int k = 0;
        for (; k + 8 <= chunks; k += 8) {
            float t8[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                t8[u] = __hip_atomic_load(sp + (int64_t)(k + u) * 2 * kLnStrip, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int u = 0; u < 8; ++u) v += t8[u];
        }
        for (; k < chunks; ++k)
            v += __hip_atomic_load(sp + (int64_t)k * 2 * kLnStrip, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int j = strip * kLnStrip + (threadIdx.x & (kLnStrip - 1));
        if (threadIdx.x < kLnStrip) dgamma[j] = v;
        else dbeta[j] = v;
    }
    if (threadIdx.x == 0) __hip_atomic_store(tickets + strip, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Column sums of the row pass's partials part[K][W] (W = 2 * cols: the
// dgamma columns, then the dbeta columns) in one launch of 32-column
// strips.  Block s owns columns 32s .. 32s + 31 of every partial row: thread
// t adds 16-byte vectors at columns 32s + 4(t % 8) of rows k = t / 8,
// k + 32, ... (a row segment is one whole 128-byte line; the block's loads
// are all in flight together), then the 32 row groups are combined through
// LDS in a fixed order, so the result is deterministic.  (Strips of 16 and
// 64 columns were measured slower at 1024 x 1024.)
__global__ __launch_bounds__(256) void ln_part_strip_kernel(const float* __restrict__ part, float* __restrict__ dgamma,
                                                            float* __restrict__ dbeta, int K, int W, int cols,
                                                            int vec) {
    constexpr int kQuads = 8, kGroups = 32;
    __shared__ float red[kGroups][4 * kQuads + 1];
    const int q = threadIdx.x % kQuads, kg = threadIdx.x / kQuads;
    const int j = blockIdx.x * 4 * kQuads + 4 * q;
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (vec && j + 4 <= W) {
#pragma unroll 8
        for (int k = kg; k < K; k += kGroups) {
            const float4 v = *reinterpret_cast<const float4*>(part + (int64_t)k * W + j);
            a[0] += v.x; a[1] += v.y; a[2] += v.z; a[3] += v.w;
        }
    } else {
        for (int k = kg; k < K; k += kGroups)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (j + e < W) a[e] += part[(int64_t)k * W + j + e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) red[kg][4 * q + e] = a[e];
    __syncthreads();
    if (threadIdx.x < 4 * kQuads) {
        const int c = threadIdx.x, jj = blockIdx.x * 4 * kQuads + c;
        float t[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = (red[4 * i][c] + red[4 * i + 1][c]) + (red[4 * i + 2][c] + red[4 * i + 3][c]);
        const float v = ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
        if (jj < W) {
            if (jj < cols) dgamma[jj] = v;
            else dbeta[jj - cols] = v;
        }
    }
}

// Streaming dx for wide rows (three passes over the row).
__global__ __launch_bounds__(256) void ln_bwd_dx_stream_kernel(const float* __restrict__ dy, const float* __restrict__ x,
                                                               const float* __restrict__ gamma,
                                                               const float* __restrict__ mean,
                                                               const float* __restrict__ rstd, float* __restrict__ dx,
                                                               int rows, int cols) {
    const int lane = threadIdx.x & 63;
    const int wave_id = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int n_waves = gridDim.x * 4;
    const float inv_c = 1.0f / (float)cols;
    for (int r = wave_id; r < rows; r += n_waves) {
        const float* xr = x + (int64_t)r * cols;
        const float* gr = dy + (int64_t)r * cols;
        const float m = mean[r], rs = rstd[r];
        float s1 = 0.0f, s2 = 0.0f;
        for (int j = lane; j < cols; j += 64) {
            const float g = gr[j] * gamma[j];
            s1 += g;
            s2 += g * (xr[j] - m) * rs;
        }
        s1 = tfd::wave_sum(s1) * inv_c;
        s2 = tfd::wave_sum(s2) * inv_c;
        float* dr = dx + (int64_t)r * cols;
        for (int j = lane; j < cols; j += 64) {
            const float g = gr[j] * gamma[j];
            dr[j] = rs * (g - s1 - (xr[j] - m) * rs * s2);
        }
    }
}

// Column partials of dy * xhat and dy for wide rows: block (strip, chunk).
__global__ __launch_bounds__(256) void ln_bwd_cols_kernel(const float* __restrict__ dy, const float* __restrict__ x,
                                                          const float* __restrict__ mean,
                                                          const float* __restrict__ rstd, float* __restrict__ part,
                                                          int rows, int cols, int rows_per_chunk) {
    __shared__ float red[4][2][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = blockIdx.x * 64 + lane;
    const int r0 = blockIdx.y * rows_per_chunk;
    const int r1 = min(rows, r0 + rows_per_chunk);
    float ga = 0.0f, ba = 0.0f;
    if (j < cols)
        for (int r = r0 + wave; r < r1; r += 4) {
            const float g = dy[(int64_t)r * cols + j];
            ga += g * ((x[(int64_t)r * cols + j] - mean[r]) * rstd[r]);
            ba += g;
        }
    red[wave][0][lane] = ga;
    red[wave][1][lane] = ba;
    __syncthreads();
    if (wave == 0 && j < cols) {
        float* pg = part + (int64_t)blockIdx.y * 2 * cols;
        pg[j] = (red[0][0][lane] + red[1][0][lane]) + (red[2][0][lane] + red[3][0][lane]);
        pg[cols + j] = (red[0][1][lane] + red[1][1][lane]) + (red[2][1][lane] + red[3][1][lane]);
    }
}

// Reference-compatible stub: dx = dy * gamma[col].
__global__ void ln_bwd_stub_kernel(const float* __restrict__ dy, const float* __restrict__ gamma,
                                   float* __restrict__ dx, int64_t n, int cols) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) dx[i] = dy[i] * gamma[i % cols];
}

int chunks_for(int64_t cols) {
    int64_t c = (cols + 255) / 256;
    if (c <= 1) return 1;
    if (c <= 2) return 2;
    if (c <= 4) return 4;
    if (c <= kMaxCached) return kMaxCached;
    return 0;
}

bool row_vec(const void* p, int64_t cols) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0 && cols % 4 == 0; }

int row_grid(int64_t rows) { return (int)std::min<int64_t>((rows + 3) / 4, 2048); }

}  // namespace

extern "C" {

tf_status tf_layernorm_fwd(tf_ctx* ctx, const float* x, const float* gamma, const float* beta, float* y,
                           float* mean, float* rstd, int64_t rows, int64_t cols, float eps) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(rows >= 0 && cols >= 0 && rows < (1LL << 31) && cols < (1LL << 31), "tf_layernorm_fwd: bad extent");
    if (rows == 0 || cols == 0) return TF_OK;
    TF_REQUIRE(x && gamma && beta && y && mean && rstd, "tf_layernorm_fwd: null pointer");
    const int vec = row_vec(x, cols) && row_vec(y, cols);
    const dim3 grid(row_grid(rows));
    switch (chunks_for(cols)) {
    case 1: ln_fwd_kernel<1><<<grid, 256, 0, ctx->stream>>>(x, gamma, beta, y, mean, rstd, (int)rows, (int)cols, eps, vec); break;
    case 2: ln_fwd_kernel<2><<<grid, 256, 0, ctx->stream>>>(x, gamma, beta, y, mean, rstd, (int)rows, (int)cols, eps, vec); break;
    case 4: ln_fwd_kernel<4><<<grid, 256, 0, ctx->stream>>>(x, gamma, beta, y, mean, rstd, (int)rows, (int)cols, eps, vec); break;
    case kMaxCached: ln_fwd_kernel<kMaxCached><<<grid, 256, 0, ctx->stream>>>(x, gamma, beta, y, mean, rstd, (int)rows, (int)cols, eps, vec); break;
    default: ln_fwd_stream_kernel<<<grid, 256, 0, ctx->stream>>>(x, gamma, beta, y, mean, rstd, (int)rows, (int)cols, eps); break;
    }
    return tfh::check_launch("ln_fwd_kernel");
}

tf_status tf_layernorm_bwd(tf_ctx* ctx, const float* dy, const float* x, const float* gamma, const float* mean,
                           const float* rstd, float* dx, float* dgamma, float* dbeta, int64_t rows, int64_t cols,
                           int reference_compat) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(rows >= 0 && cols >= 0 && rows < (1LL << 31) && cols < (1LL << 31), "tf_layernorm_bwd: bad extent");
    if (cols == 0) return TF_OK;
    TF_REQUIRE(gamma && (rows == 0 || (dy && dx)), "tf_layernorm_bwd: null pointer");
    if (reference_compat) {
        if (rows > 0) {
            ln_bwd_stub_kernel<<<tfd::grid_for(rows * cols, 4), 256, 0, ctx->stream>>>(dy, gamma, dx, rows * cols, (int)cols);
            tf_status st = tfh::check_launch("ln_bwd_stub_kernel");
            if (st != TF_OK) return st;
        }
        if (dgamma) { tf_status st = tf_hip_fill_f32(ctx, dgamma, 0.0f, cols); if (st != TF_OK) return st; }
        if (dbeta) { tf_status st = tf_hip_fill_f32(ctx, dbeta, 0.0f, cols); if (st != TF_OK) return st; }
        return TF_OK;
    }
    TF_REQUIRE(x && mean && rstd && dgamma && dbeta, "tf_layernorm_bwd: null pointer");
    if (rows == 0) {
        tf_status st = tf_hip_fill_f32(ctx, dgamma, 0.0f, cols);
        if (st != TF_OK) return st;
        return tf_hip_fill_f32(ctx, dbeta, 0.0f, cols);
    }
    const int nc = chunks_for(cols);
    const bool vec = row_vec(x, cols) && row_vec(dy, cols) && row_vec(dx, cols);
    const int64_t tstrips = cols / kLnStrip;
    if (nc > 0 && vec && cols % kLnStrip == 0 && tstrips <= tfh::kTicketColsumStrips) {
        // One launch: row blocks (4 waves, >= 1 row per wave, >= 256 blocks
        // when the rows allow) beside (strip, chunk) blocks for dgamma/dbeta,
        // about 256 of those.  The strip counters are the column sum's
        // (tfh::kTicketColsum): kernels on one stream run in order and each
        // leaves its counters at zero.
        constexpr int waves = 4;
        const int64_t rpb = std::max<int64_t>(waves, (rows + 255) / 256);
        const int64_t row_blocks = (rows + rpb - 1) / rpb;
        int64_t chunks =
            std::max<int64_t>(1, std::min<int64_t>((kLnColBlocks + tstrips - 1) / tstrips, (rows + 31) / 32));
        const int rpc = (int)((rows + chunks - 1) / chunks);
        chunks = (rows + rpc - 1) / rpc;
        tf_status st = tfh::ensure_workspace(ctx, (size_t)tstrips * chunks * 2 * kLnStrip * sizeof(float));
        if (st != TF_OK) return st;
        float* part = reinterpret_cast<float*>(ctx->ws);
        const dim3 grid((unsigned)(row_blocks + tstrips * chunks));
#define TF_LN_ONE(NC) ln_bwd_onepass_kernel<NC><<<grid, 256, 0, ctx->stream>>>(dy, x, gamma, mean, rstd, dx, dgamma, \
                          dbeta, part, ctx->tickets + tfh::kTicketColsum, (int)rows, (int)cols, (int)rpb, (int)row_blocks, \
                          (int)tstrips, rpc, (int)chunks)
        switch (nc) {
        case 1: TF_LN_ONE(1); break;
        case 2: TF_LN_ONE(2); break;
        case 4: TF_LN_ONE(4); break;
        default: TF_LN_ONE(kMaxCached); break;
        }
#undef TF_LN_ONE
        return tfh::check_launch("ln_bwd_onepass_kernel");
    }
    if (nc > 0) {
        // Blocks of 4 waves, >= 1 row per wave, >= 256 blocks when the rows
        // allow (1024 rows: 256 blocks of one row per wave, every CU busy;
        // blocks of 8 waves left half of them idle).
        constexpr int waves = 4;
        const int64_t rpb = std::max<int64_t>(waves, (rows + 255) / 256);
        const int64_t nblocks = (rows + rpb - 1) / rpb;
        tf_status st = tfh::ensure_workspace(ctx, (size_t)nblocks * 2 * cols * sizeof(float));
        if (st != TF_OK) return st;
        float* part = reinterpret_cast<float*>(ctx->ws);
        const dim3 grid((unsigned)nblocks);
#define TF_LN_BWD(NC) ln_bwd_fused_kernel<NC, waves><<<grid, waves * 64, 0, ctx->stream>>>(dy, x, gamma, mean, rstd, \
                                                     dx, part, (int)rows, (int)cols, (int)rpb, vec)
        switch (nc) {
        case 1: TF_LN_BWD(1); break;
        case 2: TF_LN_BWD(2); break;
        case 4: TF_LN_BWD(4); break;
        default: TF_LN_BWD(kMaxCached); break;
        }
#undef TF_LN_BWD
        st = tfh::check_launch("ln_bwd_fused_kernel");
        if (st != TF_OK) return st;
        // part is [nblocks][dgamma cols | dbeta cols]: column sums of a
        // [nblocks][2 cols] matrix, split into the two outputs.
        const int64_t W = 2 * cols;
        ln_part_strip_kernel<<<(unsigned)((W + 31) / 32), 256, 0, ctx->stream>>>(part, dgamma, dbeta, (int)nblocks,
                                                                               (int)W, (int)cols, W % 4 == 0);
        return tfh::check_launch("ln_part_strip_kernel");
    }
    ln_bwd_dx_stream_kernel<<<row_grid(rows), 256, 0, ctx->stream>>>(dy, x, gamma, mean, rstd, dx, (int)rows, (int)cols);
    tf_status st = tfh::check_launch("ln_bwd_dx_stream_kernel");
    if (st != TF_OK) return st;
    const int strips = (int)((cols + 63) / 64);
    int64_t chunks = std::max<int64_t>(1, std::min<int64_t>((512 + strips - 1) / strips, (rows + 15) / 16));
    int rpc = (int)((rows + chunks - 1) / chunks);
    chunks = (rows + rpc - 1) / rpc;
    st = tfh::ensure_workspace(ctx, (size_t)chunks * 2 * cols * sizeof(float));
    if (st != TF_OK) return st;
    float* part = reinterpret_cast<float*>(ctx->ws);
    ln_bwd_cols_kernel<<<dim3(strips, (unsigned)chunks), 256, 0, ctx->stream>>>(dy, x, mean, rstd, part, (int)rows,
                                                                               (int)cols, rpc);
    st = tfh::check_launch("ln_bwd_cols_kernel");
    if (st != TF_OK) return st;
    return tfh::partial_rows_sum(ctx, part, dgamma, dbeta, chunks, 2 * cols, cols);
}

}  // extern "C"
