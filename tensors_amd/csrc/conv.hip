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


// ---------------------------------------------------------------------------
// Implicit-GEMM convolution forward (fp32, NCHW, MFMA): y[n][co][p] =
// epi(sum_k w[co][k] * col[n][k][p]) with col gathered from x on the fly, so
// no col buffer is written (nn/Conv2d.cpp:101-139 materialises it with
// launch_im2col, cuda/kernels/im2col.cu:57-99, then multiplies per image).
//
// Block (8 waves, two per SIMD) = MT output channels x NP consecutive output
// pixels of one image, NP = 128 (MT = 64) or 256 (MT = 32), so each wave
// owns one 32 x 32 sub-tile.  The block stages in LDS, once:
//   * the MT x K filter rows, split by k parity: wk[row][h][j] = w[row][2j+h]
//     (row stride KH2 + 4 words), so lane half h reads four consecutive k
//     steps' operands with one 16-byte read;
//   * the tap table, split the same way: koff[h][j] = patch offset of tap
//     k = 2j + h = (ci, kh, kw), i.e. (ci PH + kh dh) PW + kw dw;
//   * the input patch its pixels read: every channel, input rows ih_lo ..
//     ih_lo + PH - 1 of its output rows, each padded to PW = W + 2 pw
//     columns with zeros.
// Pixel (oh, ow) then reads tap k at koff + ((oh - oh_lo) sh) PW + ow sw:
// per four k steps one filter read, one tap read and four patch reads feed
// four v_mfma_f32_32x32x2f32 (lane half h supplies k = 2j + h of both
// operands).  K is padded to a multiple of 8 with zero filter columns (their
// taps read a valid offset).  Staged loads are issued 16 at a time into
// registers before their LDS stores.  Epilogue: + bias[co], ReLU.
// ---------------------------------------------------------------------------
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));
constexpr int kIgThreads = 512;
template <int MT>
constexpr int ig_pixels() { return MT == 64 ? 128 : 256; }

template <int MT>
__global__ __launch_bounds__(kIgThreads) void conv_fwd_implicit_kernel(const float* __restrict__ x,
                                                                       const float* __restrict__ w,
                                                                       const float* __restrict__ bias,
                                                                       float* __restrict__ y, ConvGeom g, int Cout,
                                                                       int K, int Kp, int PH, int PW,
                                                                       int tiles_per_image, int relu) {
    extern __shared__ float smem[];
    constexpr int NP = ig_pixels<MT>();
    constexpr int MSUB = MT / 32;
    const int KH2 = Kp / 2;                     // k steps per half
    const int RS = 2 * (KH2 + 4);               // filter row stride (words)
    float* wk = smem;                           // [MT][2][KH2 + 4]
    int* koff = reinterpret_cast<int*>(wk + MT * RS);   // [2][KH2]
    float* patch = reinterpret_cast<float*>(koff + Kp); // [C][PH][PW]
    const int P = (int)(g.outH * g.outW), outW = (int)g.outW;
    const int n = blockIdx.x / tiles_per_image, pt = blockIdx.x - n * tiles_per_image;
    const int p0 = pt * NP, p_end = min(p0 + NP, P);
    const int co0 = blockIdx.y * MT;
    const int oh_lo = p0 / outW;
    const int ih_lo = oh_lo * (int)g.sh - (int)g.ph;
    const int C = (int)g.C, H = (int)g.H, W = (int)g.W, kHW = (int)(g.kH * g.kW), kW = (int)g.kW;
    const int t = threadIdx.x;

    constexpr int kStage = 16;
    for (int base = t; base < MT * Kp; base += kIgThreads * kStage) {
        float v[kStage];
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int i = base + kIgThreads * u;
            const int r = i / Kp, k = i - r * Kp;
            v[u] = (i < MT * Kp && co0 + r < Cout && k < K) ? w[(int64_t)(co0 + r) * K + k] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int i = base + kIgThreads * u;
            if (i < MT * Kp) {
                const int r = i / Kp, k = i - r * Kp;
                wk[r * RS + (k & 1) * (KH2 + 4) + (k >> 1)] = v[u];
            }
        }
    }
    for (int k = t; k < Kp; k += kIgThreads) {
        const int kc = min(k, K - 1);
        const int ci = kc / kHW, rem = kc - ci * kHW, kh = rem / kW, kw = rem - kh * kW;
        koff[(k & 1) * KH2 + (k >> 1)] = (ci * PH + kh * (int)g.dh) * PW + kw * (int)g.dw;
    }
    const float* xn = x + (int64_t)n * C * H * W;
    const int plane = PH * PW;
    for (int base = t; base < C * plane; base += kIgThreads * kStage) {
        float v[kStage];
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int i = base + kIgThreads * u;
            const int ci = i / plane, rr = (i - ci * plane) / PW, cc = i - ci * plane - rr * PW;
            const int ih = ih_lo + rr, iw = cc - (int)g.pw;
            v[u] = (i < C * plane && ih >= 0 && ih < H && iw >= 0 && iw < W) ? xn[((int64_t)ci * H + ih) * W + iw]
                                                                              : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int i = base + kIgThreads * u;
            if (i < C * plane) patch[i] = v[u];
        }
    }
    __syncthreads();

    const int wave = t >> 6, lane = t & 63, l32 = lane & 31, half = lane >> 5;
    const int m_sub = wave % MSUB, n_sub = wave / MSUB;
    const int pp = p0 + n_sub * 32 + l32;
    int pix_off;
    {
        const int q = pp < p_end ? pp : p0;
        const int oh = q / outW, ow = q - oh * outW;
        pix_off = (oh - oh_lo) * (int)g.sh * PW + ow * (int)g.sw;
    }
    v16f acc = v16f{};
    const float* wrow = wk + (m_sub * 32 + l32) * RS + half * (KH2 + 4);
    const int* krow = koff + half * KH2;
    const float* pbase = patch + pix_off;
    // KH2 is a multiple of 4 (Kp a multiple of 8).
    for (int j = 0; j < KH2; j += 4) {
        const v4f a = *reinterpret_cast<const v4f*>(wrow + j);
        const v4i ko = *reinterpret_cast<const v4i*>(krow + j);
        const float b0 = pbase[ko.x], b1 = pbase[ko.y], b2 = pbase[ko.z], b3 = pbase[ko.w];
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b1, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b2, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b3, acc, 0, 0, 0);
    }

    if (pp >= p_end) return;
    float* yn = y + (int64_t)n * Cout * P;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int co = co0 + m_sub * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (co >= Cout) continue;
        float v = acc[r] + (bias ? bias[co] : 0.0f);
        if (relu) v = fmaxf(v, 0.0f);
        yn[(int64_t)co * P + pp] = v;
    }
}

// LDS layout of conv_fwd_implicit_kernel, or 0 when it does not fit.
size_t implicit_lds_bytes(const ConvGeom& g, int MT, int K, int& Kp, int& PH, int& PW) {
    Kp = (K + 7) / 8 * 8;
    const int np = MT == 64 ? ig_pixels<64>() : ig_pixels<32>();
    const int64_t rows_max = (np - 1) / g.outW + 2;               // output rows a pixel run can touch
    const int64_t ph_rows = std::min<int64_t>(rows_max, g.outH) - 1;
    PH = (int)(ph_rows * g.sh + (g.kH - 1) * g.dh + 1);
    PW = (int)(g.W + 2 * g.pw);
    const int64_t floats = (int64_t)MT * 2 * (Kp / 2 + 4) + Kp + g.C * (int64_t)PH * PW;
    const int64_t bytes = floats * 4;
    return bytes <= 160 * 1024 ? (size_t)bytes : 0;
}

// ---------------------------------------------------------------------------
// Implicit-GEMM convolution weight gradient (fp32, NCHW, MFMA):
//   dw[co][k] = sum_n sum_p dy[n][co][p] * col[n][k][p]
// with col gathered from x on the fly (nn/Conv2d.cpp:140-260 builds col with
// launch_im2col and multiplies per image).  Blocks tile the pixels as the
// forward does (MT channels x NP pixels of one image, 8 waves); each block
// stages dy's MT x NP tile (split by pixel parity, like the forward's
// filter rows), the pixel-offset table poff[h][j] of pixel 2j + h, the tap
// table koff[k] and the input patch, then computes its MT x K partial with
// v_mfma_f32_32x32x2f32 over its pixels (lane half h supplies pixel 2j + h
// of both operands: dy[co][p] and patch[koff[k] + poff[p]]).  Work items are
// (32 x 32 output tile, pixel slice): with fewer tiles than waves, each
// tile's pixels are split over several waves and their sums combined in LDS
// in slice order.  The block writes its partial to part[block][co][k]; the
// partials are then summed in a fixed order (tfh::sum_partials).  Pixels
// past the image's end carry dy = 0.
// ---------------------------------------------------------------------------
template <int MT>
__global__ __launch_bounds__(kIgThreads) void conv_bwd_weight_implicit_kernel(const float* __restrict__ x,
                                                                              const float* __restrict__ dy,
                                                                              float* __restrict__ part, ConvGeom g,
                                                                              int Cout, int K, int Kc, int PH, int PW,
                                                                              int tiles_per_image, int slices) {
    extern __shared__ float smem[];
    constexpr int NP = ig_pixels<MT>();
    constexpr int NH = NP / 2;
    constexpr int RS = 2 * (NH + 4);
    float* dyt = smem;                                     // [MT][2][NH + 4]
    int* poff = reinterpret_cast<int*>(dyt + MT * RS);      // [2][NH]
    int* koff = poff + NP;                                  // [Kc]
    float* patch = reinterpret_cast<float*>(koff + Kc);    // [C][PH][PW]
    const int P = (int)(g.outH * g.outW), outW = (int)g.outW;
    const int n = blockIdx.x / tiles_per_image, pt = blockIdx.x - n * tiles_per_image;
    const int p0 = pt * NP, p_end = min(p0 + NP, P);
    const int co0 = blockIdx.y * MT;
    const int oh_lo = p0 / outW;
    const int ih_lo = oh_lo * (int)g.sh - (int)g.ph;
    const int C = (int)g.C, H = (int)g.H, W = (int)g.W, kHW = (int)(g.kH * g.kW), kW = (int)g.kW;
    const int t = threadIdx.x;
    const int plane = PH * PW;
    float* red = patch + C * plane;                         // [8][16][64] when slices > 1

    constexpr int kStage = 16;
    const float* dyn = dy + (int64_t)n * Cout * P;
    for (int base = t; base < MT * NP; base += kIgThreads * kStage) {
        float v[kStage];
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int i = base + kIgThreads * u;
            const int r = i / NP, q = i - r * NP;
            v[u] = (i < MT * NP && co0 + r < Cout && p0 + q < p_end) ? dyn[(int64_t)(co0 + r) * P + p0 + q] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int i = base + kIgThreads * u;
            if (i < MT * NP) {
                const int r = i / NP, q = i - r * NP;
                dyt[r * RS + (q & 1) * (NH + 4) + (q >> 1)] = v[u];
            }
        }
    }
    for (int q = t; q < NP; q += kIgThreads) {
        const int pp = p0 + q < p_end ? p0 + q : p0;
        const int oh = pp / outW, ow = pp - oh * outW;
        poff[(q & 1) * NH + (q >> 1)] = (oh - oh_lo) * (int)g.sh * PW + ow * (int)g.sw;
    }
    for (int k = t; k < Kc; k += kIgThreads) {
        const int kc = min(k, K - 1);
        const int ci = kc / kHW, rem = kc - ci * kHW, kh = rem / kW, kw = rem - kh * kW;
        koff[k] = (ci * PH + kh * (int)g.dh) * PW + kw * (int)g.dw;
    }
    const float* xn = x + (int64_t)n * C * H * W;
    for (int base = t; base < C * plane; base += kIgThreads * kStage) {
        float v[kStage];
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int i = base + kIgThreads * u;
            const int ci = i / plane, rr = (i - ci * plane) / PW, cc = i - ci * plane - rr * PW;
            const int ih = ih_lo + rr, iw = cc - (int)g.pw;
            v[u] = (i < C * plane && ih >= 0 && ih < H && iw >= 0 && iw < W) ? xn[((int64_t)ci * H + ih) * W + iw]
                                                                              : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int i = base + kIgThreads * u;
            if (i < C * plane) patch[i] = v[u];
        }
    }
    __syncthreads();

    const int wave = t >> 6, lane = t & 63, l32 = lane & 31, half = lane >> 5;
    const int TM = MT / 32, TK = Kc / 32, T = TM * TK;
    const int steps = NH / slices;                          // pixel pairs per slice (a multiple of 4)
    float* outp = part + (int64_t)blockIdx.x * Cout * K;
    for (int item = wave; item < T * slices; item += kIgThreads / 64) {
        const int tile = item / slices, sl = item - tile * slices;
        const int tr = tile / TK, tc = tile - tr * TK;
        const float* arow = dyt + (tr * 32 + l32) * RS + half * (NH + 4) + sl * steps;
        const int* prow = poff + half * NH + sl * steps;
        const float* pb = patch + koff[tc * 32 + l32];
        v16f acc = v16f{};
        for (int j = 0; j < steps; j += 4) {
            const v4f a = *reinterpret_cast<const v4f*>(arow + j);
            const v4i po = *reinterpret_cast<const v4i*>(prow + j);
            const float b0 = pb[po.x], b1 = pb[po.y], b2 = pb[po.z], b3 = pb[po.w];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b0, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b1, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b2, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b3, acc, 0, 0, 0);
        }
        if (slices == 1) {
            const int k = tc * 32 + l32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int co = co0 + tr * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (co < Cout && k < K) outp[(int64_t)co * K + k] = acc[r];
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) red[(item * 16 + r) * 64 + lane] = acc[r];
        }
    }
    if (slices > 1) {
        __syncthreads();
        // Combine each tile's slices in slice order: one wave per tile.
        for (int tile = wave; tile < T; tile += kIgThreads / 64) {
            const int tr = tile / TK, tc = tile - tr * TK, k = tc * 32 + l32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float v = red[((tile * slices) * 16 + r) * 64 + lane];
                for (int sl = 1; sl < slices; ++sl) v += red[((tile * slices + sl) * 16 + r) * 64 + lane];
                const int co = co0 + tr * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (co < Cout && k < K) outp[(int64_t)co * K + k] = v;
            }
        }
    }
}

// LDS layout of conv_bwd_weight_implicit_kernel, or 0 when it does not fit.
size_t implicit_dw_lds_bytes(const ConvGeom& g, int MT, int K, int& Kc, int& PH, int& PW, int& slices) {
    Kc = (K + 31) / 32 * 32;
    const int np = MT == 64 ? ig_pixels<64>() : ig_pixels<32>();
    const int64_t rows_max = (np - 1) / g.outW + 2;
    const int64_t ph_rows = std::min<int64_t>(rows_max, g.outH) - 1;
    PH = (int)(ph_rows * g.sh + (g.kH - 1) * g.dh + 1);
    PW = (int)(g.W + 2 * g.pw);
    const int tiles = (MT / 32) * (Kc / 32);
    slices = 1;
    while (tiles * slices * 2 <= kIgThreads / 64 && (np / 2) / (slices * 2) >= 4) slices *= 2;
    const int64_t floats = (int64_t)MT * 2 * (np / 2 + 4) + np + Kc + g.C * (int64_t)PH * PW +
                           (slices > 1 ? (int64_t)tiles * slices * 16 * 64 : 0);
    const int64_t bytes = floats * 4;
    return bytes <= 160 * 1024 ? (size_t)bytes : 0;
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

tf_status tf_conv2d_fwd(tf_ctx* ctx, const float* x, const float* w, const float* bias, float* y, int64_t N,
                        int64_t C, int64_t H, int64_t W, int64_t Cout, int64_t kH, int64_t kW, int64_t sh, int64_t sw,
                        int64_t ph, int64_t pw, int64_t dh, int64_t dw, int relu) {
    TF_CTX_CHECK(ctx);
    ConvGeom g;
    tf_status st = make_geom(g, N, C, H, W, kH, kW, sh, sw, ph, pw, dh, dw);
    if (st != TF_OK) return st;
    TF_REQUIRE(Cout > 0 && C > 0, "tf_conv2d_fwd: empty channel count");
    if (N == 0) return TF_OK;
    TF_REQUIRE(x && w && y, "tf_conv2d_fwd: null pointer");
    const int64_t K = C * kH * kW;
    TF_REQUIRE(K < (1 << 20) && N * C * H * W < (1LL << 31) && N * Cout * g.outH * g.outW < (1LL << 31) &&
                   Cout < (1 << 20),
               "tf_conv2d_fwd: extent beyond this kernel's 32-bit indexing");
    const int MT = Cout <= 32 ? 32 : 64;
    int Kp, PH, PW;
    const size_t lds = implicit_lds_bytes(g, MT, (int)K, Kp, PH, PW);
    if (lds == 0)
        return tfh::set_error(TF_ERR_UNSUPPORTED, "tf_conv2d_fwd: filter rows and input patch exceed the 160 KB of LDS "
                                                  "(use tf_im2col + tf_gemm_ex)");
    const int64_t P = g.outH * g.outW;
    const int np = MT == 64 ? ig_pixels<64>() : ig_pixels<32>();
    const int tpi = (int)((P + np - 1) / np);
    TF_REQUIRE(N * tpi < (1LL << 31), "tf_conv2d_fwd: too many blocks");
    const dim3 grid((unsigned)(N * tpi), (unsigned)((Cout + MT - 1) / MT));
    // Dynamic LDS above 64 KB needs the attribute; set once per kernel to the
    // whole 160 KB, before any launch (and any graph capture) uses it.
    static const bool lds_ok = [] {
        const int all = 160 * 1024;
        return hipFuncSetAttribute(reinterpret_cast<const void*>(conv_fwd_implicit_kernel<32>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, all) == hipSuccess &&
               hipFuncSetAttribute(reinterpret_cast<const void*>(conv_fwd_implicit_kernel<64>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, all) == hipSuccess;
    }();
    if (!lds_ok) {
        (void)hipGetLastError();
        return tfh::set_error(TF_ERR_HIP, "tf_conv2d_fwd: hipFuncSetAttribute (dynamic LDS) failed");
    }
    if (MT == 32) {
        conv_fwd_implicit_kernel<32><<<grid, kIgThreads, lds, ctx->stream>>>(x, w, bias, y, g, (int)Cout, (int)K, Kp, PH, PW,
                                                                      tpi, relu);
    } else {
        conv_fwd_implicit_kernel<64><<<grid, kIgThreads, lds, ctx->stream>>>(x, w, bias, y, g, (int)Cout, (int)K, Kp, PH, PW,
                                                                      tpi, relu);
    }
    return tfh::check_launch("conv_fwd_implicit_kernel");
}

tf_status tf_conv2d_bwd_weight(tf_ctx* ctx, const float* x, const float* dy, float* dw, int64_t N, int64_t C,
                               int64_t H, int64_t W, int64_t Cout, int64_t kH, int64_t kW, int64_t sh, int64_t sw,
                               int64_t ph, int64_t pw, int64_t dh, int64_t dw_) {
    TF_CTX_CHECK(ctx);
    ConvGeom g;
    tf_status st = make_geom(g, N, C, H, W, kH, kW, sh, sw, ph, pw, dh, dw_);
    if (st != TF_OK) return st;
    TF_REQUIRE(Cout > 0 && C > 0, "tf_conv2d_bwd_weight: empty channel count");
    TF_REQUIRE(x && dy && dw, "tf_conv2d_bwd_weight: null pointer");
    const int64_t K = C * kH * kW;
    TF_REQUIRE(K < (1 << 20) && N * C * H * W < (1LL << 31) && N * Cout * g.outH * g.outW < (1LL << 31) &&
                   Cout < (1 << 20),
               "tf_conv2d_bwd_weight: extent beyond this kernel's 32-bit indexing");
    if (N == 0) return tf_hip_fill_f32(ctx, dw, 0.0f, Cout * K);
    const int MT = Cout <= 32 ? 32 : 64;
    int Kc, PH, PW, slices;
    const size_t lds = implicit_dw_lds_bytes(g, MT, (int)K, Kc, PH, PW, slices);
    if (lds == 0)
        return tfh::set_error(TF_ERR_UNSUPPORTED, "tf_conv2d_bwd_weight: dy tile, tap tables and input patch exceed the "
                                                  "160 KB of LDS (use tf_im2col + tf_gemm_ex)");
    const int64_t P = g.outH * g.outW;
    const int np = MT == 64 ? ig_pixels<64>() : ig_pixels<32>();
    const int tpi = (int)((P + np - 1) / np);
    const int64_t blocks = N * tpi;
    TF_REQUIRE(blocks < (1LL << 31), "tf_conv2d_bwd_weight: too many blocks");
    st = tfh::ensure_workspace(ctx, (size_t)blocks * Cout * K * sizeof(float));
    if (st != TF_OK) return st;
    float* part = reinterpret_cast<float*>(ctx->ws);
    static const bool lds_ok = [] {
        const int all = 160 * 1024;
        return hipFuncSetAttribute(reinterpret_cast<const void*>(conv_bwd_weight_implicit_kernel<32>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, all) == hipSuccess &&
               hipFuncSetAttribute(reinterpret_cast<const void*>(conv_bwd_weight_implicit_kernel<64>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, all) == hipSuccess;
    }();
    if (!lds_ok) {
        (void)hipGetLastError();
        return tfh::set_error(TF_ERR_HIP, "tf_conv2d_bwd_weight: hipFuncSetAttribute (dynamic LDS) failed");
    }
    const dim3 grid((unsigned)blocks, (unsigned)((Cout + MT - 1) / MT));
    if (MT == 32)
        conv_bwd_weight_implicit_kernel<32><<<grid, kIgThreads, lds, ctx->stream>>>(x, dy, part, g, (int)Cout, (int)K,
                                                                                   Kc, PH, PW, tpi, slices);
    else
        conv_bwd_weight_implicit_kernel<64><<<grid, kIgThreads, lds, ctx->stream>>>(x, dy, part, g, (int)Cout, (int)K,
                                                                                   Kc, PH, PW, tpi, slices);
    st = tfh::check_launch("conv_bwd_weight_implicit_kernel");
    if (st != TF_OK) return st;
    return tfh::sum_partials(ctx, part, blocks, Cout, K, dw, K);
}

}  // extern "C"
