// im2col / col2im index maps for Conv2d (NCHW, float32 or bf16).
//
//   col[n][c*kH*kW + ki*kW + kj][oh*outW + ow] = x[n][c][ih][iw]  (0 outside)
//   ih = oh*sh + ki*dh - ph,  iw = ow*sw + kj*dw - pw
// (cuda/kernels/im2col.cu:57-99).  One thread per column element, writes
// coalesced along the output-pixel index.
//
// col2im is the adjoint.  The reference scatters with atomicAdd
// (cuda/kernels/col2im.cu:50-80; its fp16/bf16 variant races, :111-113);
// here every input pixel gathers its <= kH*kW taps in (ki, kj) order, so the
// result is deterministic and needs no atomics:
//   dx[n][c][ih][iw] = sum_{ki,kj : (ih + ph - ki*dh) % sh == 0, ...} col[...]
#include "common.hpp"

#include <algorithm>

namespace {

struct ConvGeom {
    int64_t N, C, H, W, kH, kW, sh, sw, ph, pw, dh, dw, outH, outW;
};

template <typename T>
__device__ __forceinline__ float ldf(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ldf<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float ldf<uint16_t>(const uint16_t* p, int64_t i) { return tfd::bf16_to_f32(p[i]); }

template <typename T>
__device__ __forceinline__ void stf(T* p, int64_t i, float v);
template <>
__device__ __forceinline__ void stf<float>(float* p, int64_t i, float v) { p[i] = v; }
template <>
__device__ __forceinline__ void stf<uint16_t>(uint16_t* p, int64_t i, float v) { p[i] = tfd::f32_to_bf16(v); }

template <typename T>
__global__ void im2col_kernel(const T* __restrict__ x, T* __restrict__ col, ConvGeom g) {
    const int64_t sp = g.outH * g.outW;
    const int64_t rows = g.C * g.kH * g.kW;
    const int64_t total = g.N * rows * sp;
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; idx < total; idx += stride) {
        const int64_t o = idx % sp;
        const int64_t t = idx / sp;
        const int64_t row = t % rows;
        const int64_t n = t / rows;
        const int64_t kk = g.kH * g.kW;
        const int64_t c = row / kk, rk = row - c * kk;
        const int64_t ki = rk / g.kW, kj = rk - ki * g.kW;
        const int64_t oh = o / g.outW, ow = o - oh * g.outW;
        const int64_t ih = oh * g.sh + ki * g.dh - g.ph;
        const int64_t iw = ow * g.sw + kj * g.dw - g.pw;
        float v = 0.0f;
        if (ih >= 0 && ih < g.H && iw >= 0 && iw < g.W) v = ldf(x, ((n * g.C + c) * g.H + ih) * g.W + iw);
        stf(col, idx, v);
    }
}

template <typename T>
__global__ void col2im_kernel(const T* __restrict__ col, T* __restrict__ dx, ConvGeom g) {
    const int64_t sp = g.outH * g.outW;
    const int64_t rows = g.C * g.kH * g.kW;
    const int64_t total = g.N * g.C * g.H * g.W;
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; idx < total; idx += stride) {
        const int64_t iw = idx % g.W;
        int64_t t = idx / g.W;
        const int64_t ih = t % g.H;
        t /= g.H;
        const int64_t c = t % g.C;
        const int64_t n = t / g.C;
        const T* cn = col + n * rows * sp;
        float acc = 0.0f;
        for (int64_t ki = 0; ki < g.kH; ++ki) {
            const int64_t hh = ih + g.ph - ki * g.dh;
            if (hh < 0 || hh % g.sh != 0) continue;
            const int64_t oh = hh / g.sh;
            if (oh >= g.outH) continue;
            for (int64_t kj = 0; kj < g.kW; ++kj) {
                const int64_t ww = iw + g.pw - kj * g.dw;
                if (ww < 0 || ww % g.sw != 0) continue;
                const int64_t ow = ww / g.sw;
                if (ow >= g.outW) continue;
                const int64_t row = (c * g.kH + ki) * g.kW + kj;
                acc += ldf(cn, row * sp + oh * g.outW + ow);
            }
        }
        stf(dx, idx, acc);
    }
}

// Plane forms, used when a channel plane and its kH*kW column rows fit in
// LDS (the common case): one block per (n, c) plane or part of its rows.
// col[n][c*kH*kW + r][o] for fixed (n, c) is one contiguous run of
// kH*kW*outH*outW elements, so the block's stores (im2col) or loads
// (col2im) are a single coalesced stream, the other side goes through LDS,
// and the index arithmetic is 32-bit.  Same values as the element forms:
// im2col copies, col2im sums the taps in the same (ki, kj) order.
constexpr int kPlaneLdsFloats = 16384;  // 64 KB of LDS per block

// dst[0 .. n) = src[0 .. n) as floats, by the whole block: eight loads in
// flight per thread before their LDS stores (a plain strided loop waits for
// each load in turn).
template <typename T>
__device__ __forceinline__ void stage_to_lds(const T* __restrict__ src, float* dst, int n) {
    int i = threadIdx.x;
    for (; i + 7 * 256 < n; i += 8 * 256) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = ldf(src, i + u * 256);
#pragma unroll
        for (int u = 0; u < 8; ++u) dst[i + u * 256] = v[u];
    }
    for (; i < n; i += 256) dst[i] = ldf(src, i);
}

// Rows r0 .. r0 + rows_per_block - 1 of plane blockIdx.x.
template <typename T>
__global__ __launch_bounds__(256) void im2col_plane_kernel(const T* __restrict__ x, T* __restrict__ col, ConvGeom g64,
                                                           int rows_per_block) {
    extern __shared__ float plane[];
    const int H = (int)g64.H, W = (int)g64.W, kW = (int)g64.kW, outW = (int)g64.outW;
    const int sh = (int)g64.sh, sw = (int)g64.sw, dh = (int)g64.dh, dw = (int)g64.dw;
    const int kk = (int)(g64.kH * g64.kW), sp = (int)(g64.outH * g64.outW), hw = H * W;
    const int64_t nc = blockIdx.x;
    const T* xp = x + nc * hw;
    stage_to_lds(xp, plane, hw);
    __syncthreads();
    const int r0 = blockIdx.y * rows_per_block, r1 = min(kk, r0 + rows_per_block);
    T* cp = col + nc * kk * sp;
    const int ph = (int)g64.ph, pw = (int)g64.pw;
    // Output pixel outer (one division per pixel), rows inner: for each row
    // the wave's lanes still store consecutive pixels.
    for (int o = threadIdx.x; o < sp; o += 256) {
        const int oh = o / outW, ow = o - oh * outW;
        const int ihb = oh * sh - ph, iwb = ow * sw - pw;
        int ki = r0 / kW, kj = r0 - (r0 / kW) * kW;
        for (int r = r0; r < r1; ++r) {
            const int ih = ihb + ki * dh, iw = iwb + kj * dw;
            float v = 0.0f;
            if ((unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W) v = plane[ih * W + iw];
            stf(cp, (int64_t)r * sp + o, v);
            if (++kj == kW) {
                kj = 0;
                ++ki;
            }
        }
    }
}

template <typename T>
__global__ __launch_bounds__(256) void col2im_plane_kernel(const T* __restrict__ col, T* __restrict__ dx, ConvGeom g64) {
    extern __shared__ float cols[];
    const int H = (int)g64.H, W = (int)g64.W, kH = (int)g64.kH, kW = (int)g64.kW;
    const int outH = (int)g64.outH, outW = (int)g64.outW, sh = (int)g64.sh, sw = (int)g64.sw;
    const int ph = (int)g64.ph, pw = (int)g64.pw, dh = (int)g64.dh, dw = (int)g64.dw;
    const int sp = outH * outW, n_col = kH * kW * sp, hw = H * W;
    const int64_t nc = blockIdx.x;
    const T* cp = col + nc * n_col;
    stage_to_lds(cp, cols, n_col);
    __syncthreads();
    T* dp = dx + nc * hw;
    // Tap (ki, kj) reaches output row oh = (ih + ph - ki*dh) / sh when that
    // is a whole number in [0, outH); the quotient and remainder are carried
    // from tap to tap (one division per pixel and axis instead of per tap).
    const int dqh = dh / sh, drh = dh - dqh * sh, dqw = dw / sw, drw = dw - dqw * sw;
    for (int p = threadIdx.x; p < hw; p += 256) {
        const int ih = p / W, iw = p - ih * W;
        const int qw0 = (iw + pw) / sw, rw0 = (iw + pw) - qw0 * sw;
        int qh = (ih + ph) / sh, rh = (ih + ph) - qh * sh;
        float acc = 0.0f;
        for (int ki = 0; ki < kH; ++ki) {
            if (qh < 0) break;  // hh < 0 here and for every later ki
            if (rh == 0 && qh < outH) {
                const float* crow = cols + ki * kW * sp + qh * outW;
                int qw = qw0, rw = rw0;
                for (int kj = 0; kj < kW; ++kj) {
                    if (qw < 0) break;
                    if (rw == 0 && qw < outW) acc += crow[kj * sp + qw];
                    rw -= drw;
                    qw -= dqw;
                    if (rw < 0) {
                        rw += sw;
                        --qw;
                    }
                }
            }
            rh -= drh;
            qh -= dqh;
            if (rh < 0) {
                rh += sh;
                --qh;
            }
        }
        stf(dp, p, acc);
    }
}

// The plane forms' 32-bit index arithmetic stays in range: every input
// coordinate they form lies within +-2^24.
bool plane_indices_fit(const ConvGeom& g) {
    const int64_t lim = 1LL << 24;
    return (g.outH - 1) * g.sh + (g.kH - 1) * g.dh < lim && (g.outW - 1) * g.sw + (g.kW - 1) * g.dw < lim &&
           g.ph < lim && g.pw < lim && g.H < lim && g.W < lim;
}

tf_status make_geom(ConvGeom& g, int64_t N, int64_t C, int64_t H, int64_t W, int64_t kH, int64_t kW, int64_t sh,
                    int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw) {
    TF_REQUIRE(N >= 0 && C >= 0 && H >= 0 && W >= 0, "conv: negative extent");
    TF_REQUIRE(kH > 0 && kW > 0 && sh > 0 && sw > 0 && dh > 0 && dw > 0 && ph >= 0 && pw >= 0,
               "conv: kernel, stride and dilation must be positive, padding non-negative");
    g = ConvGeom{N, C, H, W, kH, kW, sh, sw, ph, pw, dh, dw, 0, 0};
    g.outH = (H + 2 * ph - dh * (kH - 1) - 1) / sh + 1;
    g.outW = (W + 2 * pw - dw * (kW - 1) - 1) / sw + 1;
    TF_REQUIRE(g.outH > 0 && g.outW > 0, "conv: empty output (kernel larger than padded input)");
    return TF_OK;
}

}  // namespace

extern "C" {

tf_status tf_im2col(tf_ctx* ctx, const void* x, void* col, int64_t N, int64_t C, int64_t H, int64_t W, int64_t kH,
                    int64_t kW, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw, int dtype) {
    TF_CTX_CHECK(ctx);
    ConvGeom g;
    tf_status st = make_geom(g, N, C, H, W, kH, kW, sh, sw, ph, pw, dh, dw);
    if (st != TF_OK) return st;
    const int64_t total = N * C * kH * kW * g.outH * g.outW;
    if (total == 0) return TF_OK;
    TF_REQUIRE(x && col, "tf_im2col: null pointer");
    TF_REQUIRE(dtype == TF_F32 || dtype == TF_BF16, "tf_im2col: dtype must be Float32 or BFloat16");
    const int64_t planes = N * C, sp = g.outH * g.outW, kk = kH * kW;
    if (H * W <= kPlaneLdsFloats && kk * sp <= (1LL << 30) && planes >= 256 && planes < (1LL << 31) &&
        plane_indices_fit(g)) {
        // Row groups of about 4096 outputs per block.
        const int64_t groups = std::min<int64_t>({kk, std::max<int64_t>(1, (kk * sp) / 4096), 1024});
        const int rpb = (int)((kk + groups - 1) / groups);
        const dim3 grid((unsigned)planes, (unsigned)((kk + rpb - 1) / rpb));
        const size_t lds = (size_t)(H * W) * sizeof(float);
        if (dtype == TF_F32)
            im2col_plane_kernel<float><<<grid, 256, lds, ctx->stream>>>((const float*)x, (float*)col, g, rpb);
        else
            im2col_plane_kernel<uint16_t><<<grid, 256, lds, ctx->stream>>>((const uint16_t*)x, (uint16_t*)col, g, rpb);
        return tfh::check_launch("im2col_plane_kernel");
    }
    if (dtype == TF_F32) {
        im2col_kernel<float><<<tfd::grid_for(total, 4), 256, 0, ctx->stream>>>((const float*)x, (float*)col, g);
    } else if (dtype == TF_BF16) {
        im2col_kernel<uint16_t><<<tfd::grid_for(total, 4), 256, 0, ctx->stream>>>((const uint16_t*)x, (uint16_t*)col, g);
    } else {
        return tfh::set_error(TF_ERR_UNSUPPORTED, "tf_im2col: dtype must be Float32 or BFloat16");
    }
    return tfh::check_launch("im2col_kernel");
}

tf_status tf_col2im(tf_ctx* ctx, const void* col, void* dx, int64_t N, int64_t C, int64_t H, int64_t W, int64_t kH,
                    int64_t kW, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw, int64_t outH,
                    int64_t outW, int dtype) {
    TF_CTX_CHECK(ctx);
    ConvGeom g;
    tf_status st = make_geom(g, N, C, H, W, kH, kW, sh, sw, ph, pw, dh, dw);
    if (st != TF_OK) return st;
    TF_REQUIRE(outH == g.outH && outW == g.outW,
               "tf_col2im: outH/outW do not match the geometry ((H + 2p - d(k-1) - 1) / s + 1)");
    const int64_t total = N * C * H * W;
    if (total == 0) return TF_OK;
    TF_REQUIRE(col && dx, "tf_col2im: null pointer");
    TF_REQUIRE(dtype == TF_F32 || dtype == TF_BF16, "tf_col2im: dtype must be Float32 or BFloat16");
    const int64_t planes = N * C, n_col = kH * kW * g.outH * g.outW;
    if (n_col <= kPlaneLdsFloats && H * W < (1LL << 30) && planes >= 256 && planes < (1LL << 31) &&
        plane_indices_fit(g)) {
        const size_t lds = (size_t)n_col * sizeof(float);
        if (dtype == TF_F32)
            col2im_plane_kernel<float><<<(unsigned)planes, 256, lds, ctx->stream>>>((const float*)col, (float*)dx, g);
        else
            col2im_plane_kernel<uint16_t><<<(unsigned)planes, 256, lds, ctx->stream>>>((const uint16_t*)col,
                                                                                     (uint16_t*)dx, g);
        return tfh::check_launch("col2im_plane_kernel");
    }
    if (dtype == TF_F32) {
        col2im_kernel<float><<<tfd::grid_for(total, 2), 256, 0, ctx->stream>>>((const float*)col, (float*)dx, g);
    } else if (dtype == TF_BF16) {
        col2im_kernel<uint16_t><<<tfd::grid_for(total, 2), 256, 0, ctx->stream>>>((const uint16_t*)col, (uint16_t*)dx, g);
    } else {
        return tfh::set_error(TF_ERR_UNSUPPORTED, "tf_col2im: dtype must be Float32 or BFloat16");
    }
    return tfh::check_launch("col2im_kernel");
}

}  // extern "C"
