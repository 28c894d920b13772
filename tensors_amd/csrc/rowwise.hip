// Row kernels: cross-entropy forward/backward (fused LogSoftmax+NLL; the
// fused form also for bf16 logits, widened on load and rounded on store),
// log_softmax / softmax forward and backward.  One wave64 per row, 4 rows per
// 256-thread block.  Rows of up to kMaxCached * 256 columns stay in registers
// (one HBM read per pass); wider rows are streamed twice.
//
// Element mapping inside a row: chunk c covers columns [256c, 256c + 256).
// With 16-byte aligned rows lane l owns columns 256c + 4l .. 4l+3 (one
// float4); otherwise lane l owns 256c + l + 64q, q = 0..3.  Both cover every
// column exactly once, so the same code handles ragged widths.
#include "common.hpp"

#include <cmath>

namespace {

constexpr int kRowsPerBlock = 4;
constexpr int kMaxCached = 8;  // 2048 columns cached in registers

__device__ __forceinline__ int col_of(int c, int lane, int q, bool vec) {
    return vec ? 256 * c + 4 * lane + q : 256 * c + lane + 64 * q;
}

// NT: non-temporal vector accesses, for rows read or written once (the
// register-cached path); the streamed path reads its row twice and keeps the
// default policy so the second read can hit the cache.
template <int NC, bool NT = false>
__device__ __forceinline__ void load_row(const float* __restrict__ row, int cols, int lane, bool vec,
                                         float (&v)[NC][4], float fill) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        int base = 256 * c + 4 * lane;
        if (vec && base + 4 <= cols) {
            const float4* src = reinterpret_cast<const float4*>(row + base);
            float4 t = NT ? tfd::ld_nt(src) : *src;
            v[c][0] = t.x; v[c][1] = t.y; v[c][2] = t.z; v[c][3] = t.w;
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                int j = col_of(c, lane, q, vec);
                v[c][q] = j < cols ? row[j] : fill;
            }
        }
    }
}

template <int NC, bool NT = false>
__device__ __forceinline__ void store_row(float* __restrict__ row, int cols, int lane, bool vec,
                                          const float (&v)[NC][4]) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        int base = 256 * c + 4 * lane;
        if (vec && base + 4 <= cols) {
            float4* dst = reinterpret_cast<float4*>(row + base);
            const float4 t = make_float4(v[c][0], v[c][1], v[c][2], v[c][3]);
            if (NT) tfd::st_nt(dst, t);
            else *dst = t;
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                int j = col_of(c, lane, q, vec);
                if (j < cols) row[j] = v[c][q];
            }
        }
    }
}

// bf16 rows (bit patterns, for the cross entropy of bf16 logits): the same
// element mapping with 8-byte vectors, widened to fp32 on load (exact) and
// rounded to nearest even on store (v_cvt_pk_bf16_f32, as every bf16 store).
template <int NC, bool NT = false>
__device__ __forceinline__ void load_row(const uint16_t* __restrict__ row, int cols, int lane, bool vec,
                                         float (&v)[NC][4], float fill) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        int base = 256 * c + 4 * lane;
        if (vec && base + 4 <= cols) {
            const uint2* src = reinterpret_cast<const uint2*>(row + base);
            const uint2 t = NT ? tfd::ld_nt(src) : *src;
            v[c][0] = __uint_as_float(t.x << 16); v[c][1] = __uint_as_float(t.x & 0xffff0000u);
            v[c][2] = __uint_as_float(t.y << 16); v[c][3] = __uint_as_float(t.y & 0xffff0000u);
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                int j = col_of(c, lane, q, vec);
                v[c][q] = j < cols ? tfd::bf16_to_f32(row[j]) : fill;
            }
        }
    }
}

template <int NC, bool NT = false>
__device__ __forceinline__ void store_row(uint16_t* __restrict__ row, int cols, int lane, bool vec,
                                          const float (&v)[NC][4]) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        int base = 256 * c + 4 * lane;
        if (vec && base + 4 <= cols) {
            uint2* dst = reinterpret_cast<uint2*>(row + base);
            const uint2 t = make_uint2(tfd::bf16x2_rne(v[c][0], v[c][1]), tfd::bf16x2_rne(v[c][2], v[c][3]));
            if (NT) tfd::st_nt(dst, t);
            else *dst = t;
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                int j = col_of(c, lane, q, vec);
                if (j < cols) row[j] = tfd::f32_to_bf16(v[c][q]);
            }
        }
    }
}

__device__ __forceinline__ float elem_f32(const float* p, int64_t i) { return p[i]; }
__device__ __forceinline__ float elem_f32(const uint16_t* p, int64_t i) { return tfd::bf16_to_f32(p[i]); }

// Row statistics of a streamed (uncached) row: max and sum exp(x - max),
// online over 256-column chunks.
template <typename T>
__device__ __forceinline__ void stream_stats(const T* __restrict__ row, int cols, int lane, bool vec,
                                             float& mx, float& sum) {
    float m = -INFINITY, s = 0.0f;
    for (int c = 0; 256 * c < cols; ++c) {
        float v[1][4];
        // load one chunk at offset 256c
        const T* base = row + 256 * c;
        load_row<1>(base, cols - 256 * c, lane, vec, v, -INFINITY);
        float cm = fmaxf(fmaxf(v[0][0], v[0][1]), fmaxf(v[0][2], v[0][3]));
        float nm = fmaxf(m, cm);
        if (nm != -INFINITY) {
            s = s * __expf(m - nm);
#pragma unroll
            for (int q = 0; q < 4; ++q) s += __expf(v[0][q] - nm);
        }
        m = nm;
    }
    // combine lanes: each lane has (m, s); rescale to the wave max.
    float gm = tfd::wave_max(m);
    s = (m == -INFINITY) ? 0.0f : s * __expf(m - gm);
    sum = tfd::wave_sum(s);
    mx = gm;
}

// ---------------------------------------------------------------------------
// Cross entropy.  MODE 0: forward only (lse, per-row nll).  MODE 1: backward
// only (dlogits).  MODE 2: fused forward + backward.
// nll[r] = lse_r - x[r, t_r].  A target outside [0, cols) gives nll 0 and a
// zero gradient row (the train_mlp chain's one-hot mask skips such labels,
// examples/train_mlp.cpp:60-66), or NaN with `strict` (the module throws
// for them, nn/CrossEntropyLoss.cpp:47-53; NaN makes the mean loss NaN
// without a host check).  nll is capped at nll_max (the module's clamp of
// the probability at 1e-9, nn/CrossEntropyLoss.cpp:54-55; +inf: no cap).
// dlogits = scale * (exp(x - lse) - onehot), scale = g / rows.
// ---------------------------------------------------------------------------
// loss[0] = (sum_r nll[r]) * inv_rows by one block of 256 threads in a fixed
// order: thread i adds nll[i], nll[i + 256], ... in turn, then a wave
// butterfly, then the four waves' sums as (w0 + w1) + (w2 + w3).
// The nll values are read with agent-scope atomic loads (coherent across
// XCDs, written by other blocks with agent-scope atomic stores).
__device__ __forceinline__ void block_mean(const float* __restrict__ nll, int rows, float inv_rows,
                                           float* __restrict__ loss) {
    __shared__ float part[4];
    float s = 0.0f;
    int i = threadIdx.x;
    // Sixteen loads in flight, then added in the same order as one at a time.
    for (; i + 15 * 256 < rows; i += 16 * 256) {
        float t[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) t[u] = __hip_atomic_load(nll + i + 256 * u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int u = 0; u < 16; ++u) s += t[u];
    }
    for (; i < rows; i += 256) s += __hip_atomic_load(nll + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s = tfd::wave_sum(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) loss[0] = ((part[0] + part[1]) + (part[2] + part[3])) * inv_rows;
}

// One row of ce_kernel, by one wave.
template <typename T, int NC, int MODE>
__device__ __forceinline__ void ce_row(const T* __restrict__ logits, const int64_t* __restrict__ targets,
                                       const float* __restrict__ lse_in, const float* __restrict__ grad_loss,
                                       float* __restrict__ lse_out, float* __restrict__ nll,
                                       T* __restrict__ dlogits, int r, int cols, float inv_rows, int vec,
                                       float nll_max, int strict, bool nll_atomic) {
    constexpr int NCC = NC > 0 ? NC : 1;
    const int lane = threadIdx.x & 63;
    const T* x = logits + (int64_t)r * cols;
    const int64_t t = targets[r];
    const bool t_ok = t >= 0 && t < cols;

    float lse;
    float v[NCC][4];
    if constexpr (NC > 0) {
        load_row<NCC, true>(x, cols, lane, vec, v, -INFINITY);
    }
    if (MODE == 1 && lse_in != nullptr) {
        lse = lse_in[r];
    } else if constexpr (NC > 0) {
        float m = -INFINITY;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) m = fmaxf(m, v[c][q]);
        m = tfd::wave_max(m);
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) s += __expf(v[c][q] - m);
        s = tfd::wave_sum(s);
        lse = m + __logf(s);
    } else {
        float m, s;
        stream_stats(x, cols, lane, vec, m, s);
        lse = m + __logf(s);
    }

    if (MODE != 1) {
        float xt = 0.0f;
        if constexpr (NC > 0) {
            // The target's logit from the row in registers (no dependent
            // load): the lane holding column t adds it, every other term is
            // +0.0, so the wave sum is that value (a -0.0 logit comes out as
            // +0.0, which gives the same lse - x).
            float h = 0.0f;
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int q = 0; q < 4; ++q) h += col_of(c, lane, q, vec) == t ? v[c][q] : 0.0f;
            xt = tfd::wave_sum(h);
        }
        if (lane == 0) {
            if (lse_out) lse_out[r] = lse;
            float nl = t_ok ? lse - (NC > 0 ? xt : elem_f32(x, t)) : (strict ? __builtin_nanf("") : 0.0f);
            nl = nl > nll_max ? nll_max : nl;   // NaN stays NaN
            // With the in-kernel mean another block reads it: an agent-scope
            // store; otherwise a later launch reads it.
            if (nll_atomic) __hip_atomic_store(nll + r, nl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else nll[r] = nl;
        }
    }
    if (MODE != 0) {
        const float g = grad_loss ? grad_loss[0] : 1.0f;
        const float scale = t_ok ? g * inv_rows : 0.0f;
        T* dx = dlogits + (int64_t)r * cols;
        if constexpr (NC > 0) {
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    int j = col_of(c, lane, q, vec);
                    float pj = __expf(v[c][q] - lse);
                    v[c][q] = pj * scale - (j == t ? scale : 0.0f);
                }
            store_row<NCC, true>(dx, cols, lane, vec, v);
        } else {
            for (int c = 0; 256 * c < cols; ++c) {
                float w[1][4];
                load_row<1>(x + 256 * c, cols - 256 * c, lane, vec, w, -INFINITY);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    int j = 256 * c + col_of(0, lane, q, vec);
                    float pj = __expf(w[0][q] - lse);
                    w[0][q] = pj * scale - (j == t ? scale : 0.0f);
                }
                store_row<1>(dx + 256 * c, cols - 256 * c, lane, vec, w);
            }
        }
    }
}

// With `ticket` (MODE 0 and 2): every block counts itself in once its rows'
// nll are written, and the block that arrives last computes the mean loss
// with block_mean and resets the counter for the next launch.  nll and the
// counter go through agent-scope relaxed atomics (coherent across XCDs, no
// cache maintenance); a block's stores have completed (vmcnt 0 in every
// thread, then the barrier) before it counts itself in.  (A device-scope
// fence instead writes back and invalidates the XCD's L2 in every block.)
template <typename T, int NC, int MODE>
__global__ __launch_bounds__(256) void ce_kernel(const T* __restrict__ logits, const int64_t* __restrict__ targets,
                                                 const float* __restrict__ lse_in, const float* __restrict__ grad_loss,
                                                 float* __restrict__ lse_out, float* __restrict__ nll,
                                                 T* __restrict__ dlogits, int rows, int cols, float inv_rows,
                                                 int vec, float nll_max, int strict, float* __restrict__ loss,
                                                 unsigned* __restrict__ ticket) {
    const int r = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (r < rows) ce_row<T, NC, MODE>(logits, targets, lse_in, grad_loss, lse_out, nll, dlogits, r, cols, inv_rows,
                                   vec, nll_max, strict, ticket != nullptr);
    if (MODE != 1 && ticket != nullptr) {
        __shared__ int last;
        tfd::wait_stores_landed();
        __syncthreads();
        if (threadIdx.x == 0)
            last = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
        __syncthreads();
        if (last) {
            block_mean(nll, rows, inv_rows, loss);
            if (threadIdx.x == 0) __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---------------------------------------------------------------------------
// log_softmax / softmax forward (tensor/Tensor.cpp:370-447) and backward
// (autograd/ops/LogSoftmaxBackward.hpp:26-58, SoftmaxBackward.hpp:27-55).
// KIND 0: y = x - lse.   KIND 1: y = exp(x - max) / sum.
// ---------------------------------------------------------------------------
template <int NC, int KIND>
__global__ __launch_bounds__(256) void softmax_fwd_kernel(const float* __restrict__ xs, float* __restrict__ ys,
                                                          int rows, int cols, int vec) {
    constexpr int NCC = NC > 0 ? NC : 1;
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float* x = xs + (int64_t)r * cols;
    float* y = ys + (int64_t)r * cols;
    if constexpr (NC > 0) {
        float v[NCC][4];
        load_row<NCC, true>(x, cols, lane, vec, v, -INFINITY);
        float m = -INFINITY;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) m = fmaxf(m, v[c][q]);
        m = tfd::wave_max(m);
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) s += __expf(v[c][q] - m);
        s = tfd::wave_sum(s);
        const float lz = m + __logf(s), inv = 1.0f / s;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) v[c][q] = KIND == 0 ? v[c][q] - lz : __expf(v[c][q] - m) * inv;
        store_row<NCC, true>(y, cols, lane, vec, v);
    } else {
        float m, s;
        stream_stats(x, cols, lane, vec, m, s);
        const float lz = m + __logf(s), inv = 1.0f / s;
        for (int c = 0; 256 * c < cols; ++c) {
            float w[1][4];
            load_row<1>(x + 256 * c, cols - 256 * c, lane, vec, w, -INFINITY);
#pragma unroll
            for (int q = 0; q < 4; ++q) w[0][q] = KIND == 0 ? w[0][q] - lz : __expf(w[0][q] - m) * inv;
            store_row<1>(y + 256 * c, cols - 256 * c, lane, vec, w);
        }
    }
}

// KIND 0 (log_softmax): dx = dy - exp(y) * sum(dy).
// KIND 1 (softmax):     dx = y * (dy - sum(dy * y)).
template <int NC, int KIND>
__global__ __launch_bounds__(256) void softmax_bwd_kernel(const float* __restrict__ ys, const float* __restrict__ dys,
                                                          float* __restrict__ dxs, int rows, int cols, int vec) {
    constexpr int NCC = NC > 0 ? NC : 1;
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float* y = ys + (int64_t)r * cols;
    const float* dy = dys + (int64_t)r * cols;
    float* dx = dxs + (int64_t)r * cols;
    if constexpr (NC > 0) {
        float yv[NCC][4], gv[NCC][4];
        load_row<NCC, true>(y, cols, lane, vec, yv, 0.0f);
        load_row<NCC, true>(dy, cols, lane, vec, gv, 0.0f);
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) s += KIND == 0 ? gv[c][q] : gv[c][q] * yv[c][q];
        s = tfd::wave_sum(s);
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                gv[c][q] = KIND == 0 ? gv[c][q] - expf(yv[c][q]) * s : yv[c][q] * (gv[c][q] - s);
        store_row<NCC, true>(dx, cols, lane, vec, gv);
    } else {
        float s = 0.0f;
        for (int c = 0; 256 * c < cols; ++c) {
            float a[1][4], b[1][4];
            load_row<1>(y + 256 * c, cols - 256 * c, lane, vec, a, 0.0f);
            load_row<1>(dy + 256 * c, cols - 256 * c, lane, vec, b, 0.0f);
#pragma unroll
            for (int q = 0; q < 4; ++q) s += KIND == 0 ? b[0][q] : b[0][q] * a[0][q];
        }
        s = tfd::wave_sum(s);
        for (int c = 0; 256 * c < cols; ++c) {
            float a[1][4], b[1][4];
            load_row<1>(y + 256 * c, cols - 256 * c, lane, vec, a, 0.0f);
            load_row<1>(dy + 256 * c, cols - 256 * c, lane, vec, b, 0.0f);
#pragma unroll
            for (int q = 0; q < 4; ++q) b[0][q] = KIND == 0 ? b[0][q] - expf(a[0][q]) * s : a[0][q] * (b[0][q] - s);
            store_row<1>(dx + 256 * c, cols - 256 * c, lane, vec, b);
        }
    }
}

// Four-element vectors of the row helpers: 16 bytes for fp32, 8 for bf16.
bool row_vec_ok(const float* p, int64_t cols) {
    return (reinterpret_cast<uintptr_t>(p) & 15) == 0 && (cols % 4) == 0;
}
bool row_vec_ok(const uint16_t* p, int64_t cols) {
    return (reinterpret_cast<uintptr_t>(p) & 7) == 0 && (cols % 4) == 0;
}

// Number of register-cached 256-column chunks for a row width (0 = stream).
int chunks_for(int64_t cols) {
    int64_t c = (cols + 255) / 256;
    if (c <= 1) return 1;
    if (c <= 2) return 2;
    if (c <= 4) return 4;
    if (c <= kMaxCached) return kMaxCached;
    return 0;
}

// The mean loss by a separate one-block launch: for grids over
// kTicketMaxBlocks blocks, whose arrivals on one counter (one atomic per
// block, serialised) would cost more than the launch (1024 blocks: ~10 us).
constexpr int kTicketMaxBlocks = 64;
__global__ __launch_bounds__(256) void mean_kernel(const float* __restrict__ nll, int rows, float inv_rows,
                                                   float* __restrict__ loss) {
    block_mean(nll, rows, inv_rows, loss);
}

// T is deduced from the logits only (dlogits may be nullptr).
template <typename T> struct Same { using type = T; };
template <int MODE, typename T = float>
tf_status launch_ce(tf_ctx* ctx, const T* logits, const int64_t* targets, const float* lse_in,
                    const float* grad_loss, float* lse_out, float* nll, typename Same<T>::type* dlogits, int64_t rows,
                    int64_t cols,
                    int flags = 0, float* loss = nullptr) {
    // With `loss`: the mean loss too, by the kernel's last block when the
    // grid is small, else by mean_kernel after it.
    const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
    const bool in_kernel = loss != nullptr && blocks <= kTicketMaxBlocks;
    unsigned* ticket = in_kernel ? ctx->tickets + tfh::kTicketCE : nullptr;
    // -log(1e-9f) with the host's logf, as the module computes it.
    const float nll_max = (flags & TF_CE_CLAMP) ? -std::log(1e-9f) : INFINITY;
    const int strict = (flags & TF_CE_STRICT) ? 1 : 0;
    const int vec = row_vec_ok(logits, cols) && (dlogits == nullptr || row_vec_ok(dlogits, cols));
    const float inv_rows = (float)(1.0 / (double)rows);
    dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));
#define TF_CE_LAUNCH(NC)                                                                              \
    ce_kernel<T, NC, MODE><<<grid, 256, 0, ctx->stream>>>(logits, targets, lse_in, grad_loss, lse_out, nll, \
                                                         dlogits, (int)rows, (int)cols, inv_rows, vec, nll_max, \
                                                         strict, loss, ticket)
    switch (chunks_for(cols)) {
    case 1: TF_CE_LAUNCH(1); break;
    case 2: TF_CE_LAUNCH(2); break;
    case 4: TF_CE_LAUNCH(4); break;
    case kMaxCached: TF_CE_LAUNCH(kMaxCached); break;
    default: TF_CE_LAUNCH(0); break;
    }
#undef TF_CE_LAUNCH
    tf_status st = tfh::check_launch("ce_kernel");
    if (st != TF_OK || loss == nullptr || in_kernel) return st;
    mean_kernel<<<1, 256, 0, ctx->stream>>>(nll, (int)rows, inv_rows, loss);
    return tfh::check_launch("mean_kernel");
}

// ---------------------------------------------------------------------------
// Row argmax with the reference's rule (examples/train_mlp.cpp:95-100): scan
// the row in order, take column c when x[c] > the running maximum, which
// starts at -1e30 with prediction 0.  The result is the first column holding
// the row's largest value when that value exceeds -1e30, else 0 (NaN never
// wins a comparison).  One wave per row: each lane scans its columns in
// increasing order under the same strict rule from (-1e30, none), and lanes
// combine by larger value, then smaller column; a row no lane took gets 0.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void argmax_kernel(const float* __restrict__ x, int64_t* __restrict__ pred,
                                                     int rows, int cols, int vec) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float* row = x + (int64_t)r * cols;
    constexpr int kNone = 0x7fffffff;
    float best = -1e30f;
    int idx = kNone;
    for (int c = 0; 256 * c < cols; ++c) {
        float v[1][4];
        load_row<1, true>(row + 256 * c, cols - 256 * c, lane, vec != 0, v, -INFINITY);
#pragma unroll
        for (int q = 0; q < 4; ++q) {   // the lane's columns of this chunk, in increasing order
            if (v[0][q] > best) {
                best = v[0][q];
                idx = col_of(c, lane, q, vec != 0);
            }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ob = __shfl_xor(best, off, tfd::kWave);
        const int oi = __shfl_xor(idx, off, tfd::kWave);
        if (ob > best || (ob == best && oi < idx)) {
            best = ob;
            idx = oi;
        }
    }
    if (lane == 0) pred[r] = idx == kNone ? 0 : idx;
}

// correct[0] = number of rows with pred[r] == labels[r] (one block, fixed order).
__global__ __launch_bounds__(256) void count_equal_kernel(const int64_t* __restrict__ pred,
                                                          const int64_t* __restrict__ labels, int rows,
                                                          int64_t* __restrict__ correct) {
    __shared__ int part[256];
    int n = 0;
    for (int r = threadIdx.x; r < rows; r += 256) n += pred[r] == labels[r] ? 1 : 0;
    part[threadIdx.x] = n;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) part[threadIdx.x] += part[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) correct[0] = part[0];
}

tf_status check_rows(tf_ctx* ctx, int64_t rows, int64_t cols) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(rows >= 0 && cols >= 0, "row kernel: negative extent");
    TF_REQUIRE(rows < (1LL << 31) && cols < (1LL << 31), "row kernel: extent exceeds 2^31");
    return TF_OK;
}

}  // namespace

extern "C" {

tf_status tf_ce_fwd(tf_ctx* ctx, const float* logits, const int64_t* targets, float* loss, float* lse,
                    int64_t rows, int64_t cols, int flags) {
    tf_status st = check_rows(ctx, rows, cols);
    if (st != TF_OK) return st;
    TF_REQUIRE(rows > 0 && cols > 0, "tf_ce_fwd: empty logits");
    TF_REQUIRE(logits && targets && loss, "tf_ce_fwd: null pointer");
    st = tfh::ensure_workspace(ctx, (size_t)rows * sizeof(float));
    if (st != TF_OK) return st;
    float* nll = reinterpret_cast<float*>(ctx->ws);
    TF_REQUIRE((flags & ~TF_CE_MODULE) == 0, "tf_ce_fwd: unknown flags");
    return launch_ce<0>(ctx, logits, targets, nullptr, nullptr, lse, nll, nullptr, rows, cols, flags, loss);
}

tf_status tf_ce_bwd(tf_ctx* ctx, const float* logits, const int64_t* targets, const float* lse,
                    const float* grad_loss, float* dlogits, int64_t rows, int64_t cols) {
    tf_status st = check_rows(ctx, rows, cols);
    if (st != TF_OK) return st;
    if (rows == 0 || cols == 0) return TF_OK;
    TF_REQUIRE(logits && targets && dlogits, "tf_ce_bwd: null pointer");
    return launch_ce<1>(ctx, logits, targets, lse, grad_loss, nullptr, nullptr, dlogits, rows, cols);
}

tf_status tf_ce_fwd_bwd(tf_ctx* ctx, const float* logits, const int64_t* targets, float* loss, float* dlogits,
                        int64_t rows, int64_t cols, int flags) {
    tf_status st = check_rows(ctx, rows, cols);
    if (st != TF_OK) return st;
    TF_REQUIRE(rows > 0 && cols > 0, "tf_ce_fwd_bwd: empty logits");
    TF_REQUIRE(logits && targets && loss && dlogits, "tf_ce_fwd_bwd: null pointer");
    st = tfh::ensure_workspace(ctx, (size_t)rows * sizeof(float));
    if (st != TF_OK) return st;
    float* nll = reinterpret_cast<float*>(ctx->ws);
    TF_REQUIRE((flags & ~TF_CE_MODULE) == 0, "tf_ce_fwd_bwd: unknown flags");
    return launch_ce<2>(ctx, logits, targets, nullptr, nullptr, nullptr, nll, dlogits, rows, cols, flags, loss);
}

tf_status tf_ce_fwd_bwd_bf16(tf_ctx* ctx, const void* logits, const int64_t* targets, float* loss, void* dlogits,
                             int64_t rows, int64_t cols, int flags) {
    tf_status st = check_rows(ctx, rows, cols);
    if (st != TF_OK) return st;
    TF_REQUIRE(rows > 0 && cols > 0, "tf_ce_fwd_bwd_bf16: empty logits");
    TF_REQUIRE(logits && targets && loss && dlogits, "tf_ce_fwd_bwd_bf16: null pointer");
    st = tfh::ensure_workspace(ctx, (size_t)rows * sizeof(float));
    if (st != TF_OK) return st;
    float* nll = reinterpret_cast<float*>(ctx->ws);
    TF_REQUIRE((flags & ~TF_CE_MODULE) == 0, "tf_ce_fwd_bwd_bf16: unknown flags");
    return launch_ce<2>(ctx, static_cast<const uint16_t*>(logits), targets, nullptr, nullptr, nullptr, nll,
                        static_cast<uint16_t*>(dlogits), rows, cols, flags, loss);
}

tf_status tf_argmax_rows(tf_ctx* ctx, const float* x, int64_t* pred, const int64_t* labels, int64_t* correct,
                         int64_t rows, int64_t cols) {
    tf_status st = check_rows(ctx, rows, cols);
    if (st != TF_OK) return st;
    TF_REQUIRE((labels == nullptr) == (correct == nullptr), "tf_argmax_rows: labels and correct go together");
    if (rows == 0) {
        if (correct) return tf_hip_zero(ctx, correct, sizeof(int64_t));
        return TF_OK;
    }
    TF_REQUIRE(x && pred && (cols > 0), "tf_argmax_rows: null pointer or no columns");
    dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    argmax_kernel<<<grid, 256, 0, ctx->stream>>>(x, pred, (int)rows, (int)cols, row_vec_ok(x, cols));
    st = tfh::check_launch("argmax_kernel");
    if (st != TF_OK || correct == nullptr) return st;
    count_equal_kernel<<<1, 256, 0, ctx->stream>>>(pred, labels, (int)rows, correct);
    return tfh::check_launch("count_equal_kernel");
}

#define TF_ROW_LAUNCH(KERNEL, KIND, ...)                                          \
    do {                                                                          \
        dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));        \
        switch (chunks_for(cols)) {                                               \
        case 1: KERNEL<1, KIND><<<grid, 256, 0, ctx->stream>>>(__VA_ARGS__); break; \
        case 2: KERNEL<2, KIND><<<grid, 256, 0, ctx->stream>>>(__VA_ARGS__); break; \
        case 4: KERNEL<4, KIND><<<grid, 256, 0, ctx->stream>>>(__VA_ARGS__); break; \
        case kMaxCached: KERNEL<kMaxCached, KIND><<<grid, 256, 0, ctx->stream>>>(__VA_ARGS__); break; \
        default: KERNEL<0, KIND><<<grid, 256, 0, ctx->stream>>>(__VA_ARGS__); break; \
        }                                                                         \
    } while (0)

tf_status tf_log_softmax_fwd(tf_ctx* ctx, const float* x, float* y, int64_t rows, int64_t cols) {
    tf_status st = check_rows(ctx, rows, cols);
    if (st != TF_OK) return st;
    if (rows == 0 || cols == 0) return TF_OK;
    TF_REQUIRE(x && y, "tf_log_softmax_fwd: null pointer");
    int vec = row_vec_ok(x, cols) && row_vec_ok(y, cols);
    TF_ROW_LAUNCH(softmax_fwd_kernel, 0, x, y, (int)rows, (int)cols, vec);
    return tfh::check_launch("softmax_fwd_kernel");
}

tf_status tf_softmax_fwd(tf_ctx* ctx, const float* x, float* y, int64_t rows, int64_t cols) {
    tf_status st = check_rows(ctx, rows, cols);
    if (st != TF_OK) return st;
    if (rows == 0 || cols == 0) return TF_OK;
    TF_REQUIRE(x && y, "tf_softmax_fwd: null pointer");
    int vec = row_vec_ok(x, cols) && row_vec_ok(y, cols);
    TF_ROW_LAUNCH(softmax_fwd_kernel, 1, x, y, (int)rows, (int)cols, vec);
    return tfh::check_launch("softmax_fwd_kernel");
}

tf_status tf_log_softmax_bwd(tf_ctx* ctx, const float* y, const float* dy, float* dx, int64_t rows, int64_t cols) {
    tf_status st = check_rows(ctx, rows, cols);
    if (st != TF_OK) return st;
    if (rows == 0 || cols == 0) return TF_OK;
    TF_REQUIRE(y && dy && dx, "tf_log_softmax_bwd: null pointer");
    int vec = row_vec_ok(y, cols) && row_vec_ok(dy, cols) && row_vec_ok(dx, cols);
    TF_ROW_LAUNCH(softmax_bwd_kernel, 0, y, dy, dx, (int)rows, (int)cols, vec);
    return tfh::check_launch("softmax_bwd_kernel");
}

tf_status tf_softmax_bwd(tf_ctx* ctx, const float* y, const float* dy, float* dx, int64_t rows, int64_t cols) {
    tf_status st = check_rows(ctx, rows, cols);
    if (st != TF_OK) return st;
    if (rows == 0 || cols == 0) return TF_OK;
    TF_REQUIRE(y && dy && dx, "tf_softmax_bwd: null pointer");
    int vec = row_vec_ok(y, cols) && row_vec_ok(dy, cols) && row_vec_ok(dx, cols);
    TF_ROW_LAUNCH(softmax_bwd_kernel, 1, y, dy, dx, (int)rows, (int)cols, vec);
    return tfh::check_launch("softmax_bwd_kernel");
}

#undef TF_ROW_LAUNCH

}  // extern "C"
