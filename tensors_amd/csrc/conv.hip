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
                    int64_t kW, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw, int dtype) {
    TF_CTX_CHECK(ctx);
    ConvGeom g;
    tf_status st = make_geom(g, N, C, H, W, kH, kW, sh, sw, ph, pw, dh, dw);
    if (st != TF_OK) return st;
    const int64_t total = N * C * H * W;
    if (total == 0) return TF_OK;
    TF_REQUIRE(col && dx, "tf_col2im: null pointer");
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
