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
template <>
__device__ __forceinline__ float ldf<_Float16>(const _Float16* p, int64_t i) { return (float)p[i]; }

template <typename T>
__device__ __forceinline__ void stf(T* p, int64_t i, float v);
template <>
__device__ __forceinline__ void stf<float>(float* p, int64_t i, float v) { p[i] = v; }
template <>
__device__ __forceinline__ void stf<uint16_t>(uint16_t* p, int64_t i, float v) { p[i] = tfd::f32_to_bf16(v); }
// Half: round to nearest even (v_cvt_f16_f32), as __float2half in the
// reference's typed col2im (cuda/kernels/col2im.cu:44).
template <>
__device__ __forceinline__ void stf<_Float16>(_Float16* p, int64_t i, float v) { p[i] = tfd::f32_to_f16(v); }

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

// Tap tables of a col2im from LDS (NT threads build them), for column rows
// (ki, kj) of RD words each: per input row ih, rcnt[ih] taps with offsets
// roff[ih kH + a] = ki kW RD + oh outW (ki ascending); per input column iw,
// ccnt[iw] taps with offsets coff[iw kW + b] = kj RD + ow (kj ascending).
template <int NT>
__device__ __forceinline__ void build_tap_tables(const ConvGeom& g, int RD, int* rcnt, int* roff, int* ccnt, int* coff,
                                                 int t) {
    const int H = (int)g.H, W = (int)g.W, kH = (int)g.kH, kW = (int)g.kW, outH = (int)g.outH, outW = (int)g.outW;
    const int sh = (int)g.sh, sw = (int)g.sw, dh = (int)g.dh, dwl = (int)g.dw, ph = (int)g.ph, pw = (int)g.pw;
    for (int ih = t; ih < H; ih += NT) {
        int c = 0;
        for (int ki = 0; ki < kH; ++ki) {
            const int hh = ih + ph - ki * dh;
            if (hh >= 0 && hh % sh == 0 && hh / sh < outH) roff[ih * kH + c++] = ki * kW * RD + (hh / sh) * outW;
        }
        rcnt[ih] = c;
    }
    for (int iw = t; iw < W; iw += NT) {
        int c = 0;
        for (int kj = 0; kj < kW; ++kj) {
            const int ww = iw + pw - kj * dwl;
            if (ww >= 0 && ww % sw == 0 && ww / sw < outW) coff[iw * kW + c++] = kj * RD + ww / sw;
        }
        ccnt[iw] = c;
    }
}

// col2im of one (n, c) plane: its kH kW column rows staged in LDS, the tap
// tables after them.  MT > 0: no input pixel has more than MT row taps or
// MT column taps (2 for stride-2 3 x 3 layers, 3 for stride-1 ones), so a
// pixel reads all MT x MT candidates unconditionally (invalid ones at offset
// 0, a valid address) and adds the valid ones in (ki, kj) order: its LDS
// reads go out together instead of one branch and one wait per tap, and the
// sum equals the tap-by-tap one (adding +0.0 leaves it unchanged, and a sum
// that starts at +0.0 is never -0.0).  MT = 0: the tap-by-tap loop.
template <typename T, int MT>
__global__ __launch_bounds__(256) void col2im_plane_kernel(const T* __restrict__ col, T* __restrict__ dx, ConvGeom g64) {
    extern __shared__ float cols[];
    const int H = (int)g64.H, W = (int)g64.W, kH = (int)g64.kH, kW = (int)g64.kW;
    const int sp = (int)(g64.outH * g64.outW), n_col = kH * kW * sp, hw = H * W;
    int* rcnt = reinterpret_cast<int*>(cols + n_col);   // [H]
    int* roff = rcnt + H;                                // [H][kH]
    int* ccnt = roff + H * kH;                           // [W]
    int* coff = ccnt + W;                                // [W][kW]
    build_tap_tables<256>(g64, sp, rcnt, roff, ccnt, coff, threadIdx.x);
    const int64_t nc = blockIdx.x;
    stage_to_lds(col + nc * n_col, cols, n_col);
    __syncthreads();
    T* dp = dx + nc * hw;
    constexpr int M = MT > 0 ? MT : 1;
    for (int p = threadIdx.x; p < hw; p += 256) {
        const int ih = p / W, iw = p - ih * W;
        const int nr = rcnt[ih], ncl = ccnt[iw];
        float acc = 0.0f;
        if (MT > 0 && nr <= MT && ncl <= MT) {
            int ro[M], co[M];
#pragma unroll
            for (int a = 0; a < M; ++a) ro[a] = a < nr ? roff[ih * kH + a] : 0;
#pragma unroll
            for (int b = 0; b < M; ++b) co[b] = b < ncl ? coff[iw * kW + b] : 0;
            float v[M][M];
#pragma unroll
            for (int a = 0; a < M; ++a)
#pragma unroll
                for (int b = 0; b < M; ++b) v[a][b] = cols[ro[a] + co[b]];
#pragma unroll
            for (int a = 0; a < M; ++a)
#pragma unroll
                for (int b = 0; b < M; ++b) acc += a < nr && b < ncl ? v[a][b] : 0.0f;
        } else {
            for (int a = 0; a < nr; ++a) {
                const float* crow = cols + roff[ih * kH + a];
                for (int b = 0; b < ncl; ++b) acc += crow[coff[iw * kW + b]];
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
//   * the MT x K filter rows, wk[row][k] (row stride Kp + 4 words, Kp = K
//     rounded up to 8, zero past K), copied with 16-byte loads and stores
//     when K % 4 == 0;
//   * the tap table koff[k] = patch offset of tap k = (ci, kh, kw), i.e.
//     (ci PH + kh dh) PWs + kw dw;
//   * the input patch its pixels read: every channel, input rows ih_lo ..
//     ih_lo + PH - 1 of its output rows, each stored as PWs = 4 m columns
//     (column c holds iw = c - L, L = pw rounded up to 4, zeros outside the
//     image), so a row's interior is copied with 16-byte loads and stores
//     when W % 4 == 0.
// Pixel (oh, ow) then reads tap k at koff[k] + (oh - oh_lo) sh PWs + ow sw +
// L - pw.  Lane half h supplies k in [h Kp/2, (h + 1) Kp/2) of both operands:
// per four k steps one 16-byte filter read, one 16-byte tap read and four
// patch reads feed four v_mfma_f32_32x32x2f32; the reads of the next four
// steps are issued before the current four MFMAs (taps two steps ahead), so
// the LDS latency is not on the MFMA chain.  Padded k steps carry zero
// filter values and a valid tap.  Epilogue: + bias[co], ReLU.
// ---------------------------------------------------------------------------
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));
constexpr int kIgThreads = 512;
template <int MT>
constexpr int ig_pixels() { return MT == 64 ? 128 : 256; }

// x / d and x % d for 0 <= x < 2^22, 0 < d, by a float reciprocal and one
// correction step (the rounded product is within one of the quotient): about
// ten instructions instead of a signed division's expansion, in the staging
// loops that split every LDS element's index.
struct FastDiv {
    int d;
    float rcp;
};
__device__ __forceinline__ FastDiv fast_div(int d) { return FastDiv{d, 1.0f / (float)d}; }
__device__ __forceinline__ int divmod(int x, const FastDiv& f, int& r) {
    int q = (int)((float)x * f.rcp);
    r = x - __mul24(q, f.d);
    if (r < 0) {
        --q;
        r += f.d;
    } else if (r >= f.d) {
        ++q;
        r -= f.d;
    }
    return q;
}

// fp32 im2col, plane form, for output rows of whole quads (outW % 4 == 0)
// and a 16-byte aligned col: work item w of the block's rows is col row
// r0 + w / (sp / 4), output pixels 4 q .. 4 q + 3 of one output row, so a
// wave stores 1 KB of one col row per instruction (im2col_plane_kernel: 256
// bytes).  Every tap's LDS read is issued (at offset 0 outside the image)
// and the value selected.  The same values as im2col_plane_kernel.
__global__ __launch_bounds__(256) void im2col_plane4_kernel(const float* __restrict__ x, float* __restrict__ col,
                                                            ConvGeom g64, int rows_per_block) {
    extern __shared__ float plane[];
    const int H = (int)g64.H, W = (int)g64.W, kW = (int)g64.kW, outW = (int)g64.outW;
    const int sh = (int)g64.sh, sw = (int)g64.sw, dh = (int)g64.dh, dw = (int)g64.dw;
    const int ph = (int)g64.ph, pw = (int)g64.pw;
    const int kk = (int)(g64.kH * g64.kW), sp = (int)(g64.outH * g64.outW), hw = H * W;
    const int64_t nc = blockIdx.x;
    stage_to_lds(x + nc * hw, plane, hw);
    __syncthreads();
    const int r0 = blockIdx.y * rows_per_block, r1 = min(kk, r0 + rows_per_block);
    const int q4 = sp >> 2, items = (r1 - r0) * q4;
    const FastDiv fq = fast_div(q4), fw = fast_div(outW), fkw = fast_div(kW);
    float4* cp4 = reinterpret_cast<float4*>(col + nc * kk * sp);
    for (int w = threadIdx.x; w < items; w += 256) {
        int qd, ow, kj;
        const int r = r0 + divmod(w, fq, qd);
        const int oh = divmod(4 * qd, fw, ow);
        const int ki = divmod(r, fkw, kj);
        const int ih = oh * sh - ph + ki * dh, iw0 = ow * sw - pw + kj * dw;
        const bool row_in = (unsigned)ih < (unsigned)H;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int iw = iw0 + e * sw;
            const bool in = row_in && (unsigned)iw < (unsigned)W;
            const float t = plane[in ? ih * W + iw : 0];
            v[e] = in ? t : 0.0f;
        }
        cp4[(int64_t)r * q4 + qd] = make_float4(v[0], v[1], v[2], v[3]);
    }
}

constexpr int kStage4 = 8;  // 16-byte staging loads in flight per thread

// Staging sources: slot i of a source is 16 bytes (4 floats) bound for LDS
// word offset dst(i) (a multiple of 4), read by load(i, dst) with zeros
// outside the operand.

// rows x (slots s0 .. s0 + ns) of a row-major matrix: slot i is row i / ns,
// columns 4 (s0 + i % ns) .. + 3 of src (row stride ld; rows < nrows and
// columns < cols valid); 16-byte global loads when vec (cols and ld
// multiples of 4, src 16-byte aligned).  LDS row stride dst_ld.
struct RowSlots {
    const float* src;
    int ld, nrows, cols, dst_ld, s0, ns;
    bool vec;
    FastDiv fns;
    __device__ __forceinline__ RowSlots(const float* src_, int ld_, int nrows_, int cols_, int dst_ld_, int s0_,
                                        int ns_, bool vec_)
        : src(src_), ld(ld_), nrows(nrows_), cols(cols_), dst_ld(dst_ld_), s0(s0_), ns(ns_), vec(vec_),
          fns(fast_div(ns_)) {}
    __device__ __forceinline__ v4f load(int i, int& dst) const {
        int sl;
        const int r = divmod(i, fns, sl);
        const int c = 4 * (s0 + sl);
        dst = r * dst_ld + c;
        v4f val = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        if (r < nrows) {
            const float* sp = src + r * ld + c;
            if (vec) {
                if (c < cols) val = *reinterpret_cast<const v4f*>(sp);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (c + e < cols) val[e] = sp[e];
            }
        }
        return val;
    }
};

// The zero-padded input patch: slot i (counted from slot g0) of
// patch[ci][rr][c] = x[ci][ih_lo + rr][c - L] (zero outside the image), ci <
// C, rr < PH, c < PWs, 4 floats per slot; xn is the image's first element.
// 16-byte loads when vec (W % 4 == 0 and xn 16-byte aligned; L is a
// multiple of 4, so slots never straddle the image edge).
struct PatchSlots {
    const float* xn;
    int H, W, PH, L, ih_lo, g0;
    bool vec;
    FastDiv fspr, fPH;
    __device__ __forceinline__ PatchSlots(const float* xn_, int H_, int W_, int PH_, int PWs, int L_, int ih_lo_,
                                          int g0_, bool vec_)
        : xn(xn_), H(H_), W(W_), PH(PH_), L(L_), ih_lo(ih_lo_), g0(g0_), vec(vec_), fspr(fast_div(PWs / 4)),
          fPH(fast_div(PH_)) {}
    __device__ __forceinline__ v4f load(int i, int& dst) const {
        const int gi = g0 + i;
        dst = 4 * gi;
        int sl, rr;
        const int row = divmod(gi, fspr, sl);
        const int ci = divmod(row, fPH, rr);
        const int ih = ih_lo + rr, iw = 4 * sl - L;
        v4f val = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        if (ih >= 0 && ih < H) {
            const float* sp = xn + (ci * H + ih) * W + iw;
            if (vec) {
                if (iw >= 0 && iw < W) val = *reinterpret_cast<const v4f*>(sp);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (iw + e >= 0 && iw + e < W) val[e] = sp[e];
            }
        }
        return val;
    }
};

// Slots [first, n) of `src` into LDS at `lds`, by the whole block, kStage4
// loads in flight per thread before their stores.
template <class Src>
__device__ __forceinline__ void stage_slots(const Src& src, float* lds, int first, int n) {
    for (int base = first + threadIdx.x; base < n; base += kIgThreads * kStage4) {
        v4f v[kStage4];
        int d[kStage4];
#pragma unroll
        for (int u = 0; u < kStage4; ++u) {
            const int i = base + kIgThreads * u;
            v[u] = i < n ? src.load(i, d[u]) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int u = 0; u < kStage4; ++u) {
            const int i = base + kIgThreads * u;
            if (i < n) *reinterpret_cast<v4f*>(lds + d[u]) = v[u];
        }
    }
}

// The first R * kIgThreads slots of a source held in registers: load() issues
// them, store() (after other work) writes them to LDS; the remaining slots
// go through stage_slots(src, lds, R * kIgThreads, n).
template <int R>
struct Ahead {
    v4f v[R];
    int d[R];
    template <class Src>
    __device__ __forceinline__ void load(const Src& src, int n) {
#pragma unroll
        for (int u = 0; u < R; ++u) {
            const int i = threadIdx.x + kIgThreads * u;
            v[u] = i < n ? src.load(i, d[u]) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    __device__ __forceinline__ void store(float* lds, int n) const {
#pragma unroll
        for (int u = 0; u < R; ++u)
            if ((int)threadIdx.x + kIgThreads * u < n) *reinterpret_cast<v4f*>(lds + d[u]) = v[u];
    }
};

// rows x cols floats from src (row stride ld, rows < nrows valid, columns
// < cols valid, zero elsewhere) into dst[r][0 .. 4 spr) with row stride
// dst_ld; 16-byte global loads when vec (cols and ld multiples of 4, src
// 16-byte aligned).  rows * spr < 2^22.
__device__ __forceinline__ void stage_rows(const float* __restrict__ src, int ld, int nrows, int cols, float* dst,
                                           int dst_ld, int rows, int spr, bool vec) {
    stage_slots(RowSlots(src, ld, nrows, cols, dst_ld, 0, spr, vec), dst, 0, rows * spr);
}

// The whole patch (C channels) into LDS; see PatchSlots.
__device__ __forceinline__ void stage_patch(const float* __restrict__ xn, float* patch, int C, int H, int W, int PH,
                                            int PWs, int L, int ih_lo, bool vec) {
    stage_slots(PatchSlots(xn, H, W, PH, PWs, L, ih_lo, 0, vec), patch, 0, C * PH * (PWs / 4));
}

// Direct-load staging: slots [0, n) of an LDS region at byte address lds0,
// slot j's 16 bytes read from byte offset off(j) of `rsrc` (zeros for
// tfd::kBufOob).  Wave w issues the 64-slot chunks w, w + 8, ...; every load
// of the region is in flight at once.  The caller waits (vmcnt(0)) and
// synchronises before reading.
template <class Off>
__device__ __forceinline__ void stage_direct(tfd::buf_rsrc_t rsrc, uint32_t lds0, int n, const Off& off) {
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
    for (int c = wave; c * 64 < n; c += kIgThreads / 64) {
        const int j = c * 64 + lane;
        if (j < n) tfd::load16_to_lds(rsrc, off(j), lds0 + (uint32_t)c * 1024u);
    }
}

// Byte offset (from the image's first element) of patch slot j in the
// aligned layout (PatchSlots), or tfd::kBufOob for a slot outside the image.
struct PatchOff {
    int H, W, PH, L, ih_lo;
    FastDiv fspr, fPH;
    __device__ __forceinline__ uint32_t operator()(int j) const {
        int sl, rr;
        const int row = divmod(j, fspr, sl);
        const int ci = divmod(row, fPH, rr);
        const int ih = ih_lo + rr, iw = 4 * sl - L;
        return ih >= 0 && ih < H && iw >= 0 && iw < W ? 4u * (uint32_t)((ci * H + ih) * W + iw) : tfd::kBufOob;
    }
};

// Byte offset of slot j of an LDS block [rows][RS words] (RS / 4 slots a
// row) holding columns c0 .. of `nrows` rows of a row-major matrix with row
// stride ld floats: columns c0 + 4 sl .. + 3 of row r, or tfd::kBufOob for
// columns at or past c0 + cols (padding) and rows past nrows.
struct RowOff {
    int ld, c0, cols, nrows;
    FastDiv fspr;
    __device__ __forceinline__ uint32_t operator()(int j) const {
        int sl;
        const int r = divmod(j, fspr, sl);
        return r < nrows && 4 * sl < cols ? 4u * (uint32_t)(r * ld + c0 + 4 * sl) : tfd::kBufOob;
    }
};

// acc += A (32 rows of wrow, k along the row) x B (32 pixels: pbase[koff[k]])
// over KH2 k steps per lane half (KH2 a multiple of 4, >= 4), with the next
// four steps' reads in flight during the current four MFMAs.
__device__ __forceinline__ v16f mfma_gather_loop(const float* wrow, const int* krow, const float* pbase, int KH2) {
    v16f acc = v16f{};
    v4f a = *reinterpret_cast<const v4f*>(wrow);
    v4i kn = *reinterpret_cast<const v4i*>(krow);
    float b0 = pbase[kn.x], b1 = pbase[kn.y], b2 = pbase[kn.z], b3 = pbase[kn.w];
    kn = *reinterpret_cast<const v4i*>(krow + min(4, KH2 - 4));
    for (int j = 0; j < KH2; j += 4) {
        const v4i kn2 = *reinterpret_cast<const v4i*>(krow + min(j + 8, KH2 - 4));
        const v4f an = *reinterpret_cast<const v4f*>(wrow + min(j + 4, KH2 - 4));
        const float c0 = pbase[kn.x], c1 = pbase[kn.y], c2 = pbase[kn.z], c3 = pbase[kn.w];
        // Keep the reads above the MFMAs (otherwise they are sunk to their use
        // in the next step and each step waits for its own reads).
        __builtin_amdgcn_sched_barrier(0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b1, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b2, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b3, acc, 0, 0, 0);
        a = an;
        b0 = c0;
        b1 = c1;
        b2 = c2;
        b3 = c3;
        kn = kn2;
    }
    return acc;
}

// Two mfma_gather_loop chains at once: A rows wrow0 / wrow1, tap rows
// krow0 / krow1 (the same rows when SAME_K: two tiles over the same
// pixels, read once) and patch bases pbase0 / pbase1.  The two
// accumulators' MFMAs alternate, so each waits on its own chain only and
// the matrix pipe has the other's to run meanwhile; each accumulator sees
// the same MFMAs in the same order as in mfma_gather_loop.
template <bool SAME_K>
__device__ __forceinline__ void mfma_gather_loop2(const float* wrow0, const float* wrow1, const int* krow0,
                                                  const int* krow1, const float* pbase0, const float* pbase1, int KH2,
                                                  v16f& acc0, v16f& acc1) {
    acc0 = v16f{};
    acc1 = v16f{};
    v4f a0 = *reinterpret_cast<const v4f*>(wrow0), a1 = *reinterpret_cast<const v4f*>(wrow1);
    v4i kn = *reinterpret_cast<const v4i*>(krow0);
    v4i km = SAME_K ? kn : *reinterpret_cast<const v4i*>(krow1);
    float b0 = pbase0[kn.x], b1 = pbase0[kn.y], b2 = pbase0[kn.z], b3 = pbase0[kn.w];
    float e0 = pbase1[km.x], e1 = pbase1[km.y], e2 = pbase1[km.z], e3 = pbase1[km.w];
    kn = *reinterpret_cast<const v4i*>(krow0 + min(4, KH2 - 4));
    km = SAME_K ? kn : *reinterpret_cast<const v4i*>(krow1 + min(4, KH2 - 4));
    for (int j = 0; j < KH2; j += 4) {
        const v4i kn2 = *reinterpret_cast<const v4i*>(krow0 + min(j + 8, KH2 - 4));
        const v4i km2 = SAME_K ? kn2 : *reinterpret_cast<const v4i*>(krow1 + min(j + 8, KH2 - 4));
        const v4f an0 = *reinterpret_cast<const v4f*>(wrow0 + min(j + 4, KH2 - 4));
        const v4f an1 = *reinterpret_cast<const v4f*>(wrow1 + min(j + 4, KH2 - 4));
        const float c0 = pbase0[kn.x], c1 = pbase0[kn.y], c2 = pbase0[kn.z], c3 = pbase0[kn.w];
        const float d0 = pbase1[km.x], d1 = pbase1[km.y], d2 = pbase1[km.z], d3 = pbase1[km.w];
        __builtin_amdgcn_sched_barrier(0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.x, b0, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.x, e0, acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.y, b1, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.y, e1, acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.z, b2, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.z, e2, acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.w, b3, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.w, e3, acc1, 0, 0, 0);
        a0 = an0;
        a1 = an1;
        b0 = c0; b1 = c1; b2 = c2; b3 = c3;
        e0 = d0; e1 = d1; e2 = d2; e3 = d3;
        kn = kn2;
        km = km2;
    }
}

// acc += the k steps j0 .. j1 - 1 of 8 k each, lane half h taking k =
// 8 j + 4 h .. 8 j + 4 h + 3 (wrow and krow already offset by 4 h), with the
// next step's reads in flight during the current four MFMAs as above.
__device__ __forceinline__ v16f mfma_gather_steps(v16f acc, const float* wrow, const int* krow, const float* pbase,
                                                  int j0, int j1) {
    if (j0 >= j1) return acc;
    v4f a = *reinterpret_cast<const v4f*>(wrow + 8 * j0);
    v4i kn = *reinterpret_cast<const v4i*>(krow + 8 * j0);
    float b0 = pbase[kn.x], b1 = pbase[kn.y], b2 = pbase[kn.z], b3 = pbase[kn.w];
    kn = *reinterpret_cast<const v4i*>(krow + 8 * min(j0 + 1, j1 - 1));
    for (int j = j0; j < j1; ++j) {
        const v4i kn2 = *reinterpret_cast<const v4i*>(krow + 8 * min(j + 2, j1 - 1));
        const v4f an = *reinterpret_cast<const v4f*>(wrow + 8 * min(j + 1, j1 - 1));
        const float c0 = pbase[kn.x], c1 = pbase[kn.y], c2 = pbase[kn.z], c3 = pbase[kn.w];
        __builtin_amdgcn_sched_barrier(0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b1, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b2, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b3, acc, 0, 0, 0);
        a = an;
        b0 = c0;
        b1 = c1;
        b2 = c2;
        b3 = c3;
        kn = kn2;
    }
    return acc;
}

// mfma_gather_steps with the steps split over two accumulators by the
// parity of j (even steps into acc0, odd into acc1), so consecutive steps'
// MFMAs do not wait on each other; the caller adds acc0 + acc1.  Which
// accumulator a step goes to depends only on j, so splitting a range
// [j0, j1) into several calls gives the same sums.
__device__ __forceinline__ void mfma_gather_steps2(v16f& acc0, v16f& acc1, const float* wrow, const int* krow,
                                                   const float* pbase, int j0, int j1) {
    if (j0 >= j1) return;
    v4f a = *reinterpret_cast<const v4f*>(wrow + 8 * j0);
    v4i kn = *reinterpret_cast<const v4i*>(krow + 8 * j0);
    float b0 = pbase[kn.x], b1 = pbase[kn.y], b2 = pbase[kn.z], b3 = pbase[kn.w];
    kn = *reinterpret_cast<const v4i*>(krow + 8 * min(j0 + 1, j1 - 1));
    int j = j0;
    auto step = [&](v16f& acc) __attribute__((always_inline)) {
        const v4i kn2 = *reinterpret_cast<const v4i*>(krow + 8 * min(j + 2, j1 - 1));
        const v4f an = *reinterpret_cast<const v4f*>(wrow + 8 * min(j + 1, j1 - 1));
        const float c0 = pbase[kn.x], c1 = pbase[kn.y], c2 = pbase[kn.z], c3 = pbase[kn.w];
        __builtin_amdgcn_sched_barrier(0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b1, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b2, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b3, acc, 0, 0, 0);
        a = an;
        b0 = c0;
        b1 = c1;
        b2 = c2;
        b3 = c3;
        kn = kn2;
        ++j;
    };
    if (j & 1) step(acc1);
    while (j + 1 < j1) {
        step(acc0);
        step(acc1);
    }
    if (j < j1) step(acc0);
}

template <int MT>
__global__ __launch_bounds__(kIgThreads) void conv_fwd_implicit_kernel(const float* __restrict__ x,
                                                                       const float* __restrict__ w,
                                                                       const float* __restrict__ bias,
                                                                       float* __restrict__ y, ConvGeom g, int Cout,
                                                                       int K, int Kp, int PH, int PWs, int L,
                                                                       int tiles_per_image, int relu, int vec) {
    extern __shared__ float smem[];
    constexpr int NP = ig_pixels<MT>();
    constexpr int MSUB = MT / 32;
    const int RS = Kp + 4;                      // filter row stride (words): RS / 4 odd, no bank conflicts
    float* wk = smem;                           // [MT][RS]
    int* koff = reinterpret_cast<int*>(wk + MT * RS);   // [Kp]
    float* patch = reinterpret_cast<float*>(koff + Kp); // [C][PH][PWs]
    const int P = (int)(g.outH * g.outW), outW = (int)g.outW;
    const int n = blockIdx.x / tiles_per_image, pt = blockIdx.x - n * tiles_per_image;
    const int p0 = pt * NP, p_end = min(p0 + NP, P);
    const int co0 = blockIdx.y * MT;
    const int oh_lo = p0 / outW;
    const int ih_lo = oh_lo * (int)g.sh - (int)g.ph;
    const int C = (int)g.C, H = (int)g.H, W = (int)g.W, kHW = (int)(g.kH * g.kW), kW = (int)g.kW;
    const int t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63, l32 = lane & 31, half = lane >> 5;
    const int m_sub = wave % MSUB, n_sub = wave / MSUB;
    const int pp = p0 + n_sub * 32 + l32;
    int pix_off;
    {
        const int q = pp < p_end ? pp : p0;
        const int oh = q / outW, ow = q - oh * outW;
        pix_off = (oh - oh_lo) * (int)g.sh * PWs + ow * (int)g.sw + L - (int)g.pw;
    }
    const int KS = Kp / 8;                                  // k steps of 8
    // The block's bias values, read from LDS by the epilogue: a global load
    // in the store loop would make each store wait for the ones before it
    // (loads and stores share one counter), which cost 2 us per launch.
    __shared__ float bias_s[MT];
    if (t < MT) bias_s[t] = bias && co0 + t < Cout ? bias[co0 + t] : 0.0f;
    v16f acc;
    if (vec & 4) {
        // Direct loads (bit 2: aligned patch layout, 16-byte image rows):
        // LDS = filter rows [MT][RS] | input patch | tap table, each of the
        // first two regions rounded up to whole KB.  The patch and (when its
        // rows are 16-byte loadable, bit 1) the filter go global -> LDS in one
        // round trip; otherwise the filter is staged through registers while
        // the patch loads are in flight.
        float* wkd = smem;
        float* patchd = smem + (MT * RS + 255) / 256 * 256;
        int* koffd = reinterpret_cast<int*>(patchd + (C * PH * PWs + 255) / 256 * 256);
        const float* xn = x + (int64_t)n * C * H * W;
        const int nrows = min(MT, Cout - co0);
        stage_direct(tfd::buf_rsrc(xn, (uint32_t)(C * H * W) * 4u), tfd::lds_byte_addr(patchd), C * PH * (PWs / 4),
                     PatchOff{H, W, PH, L, ih_lo, fast_div(PWs / 4), fast_div(PH)});
        if (vec & 2)
            stage_direct(tfd::buf_rsrc(w + (int64_t)co0 * K, (uint32_t)(nrows * K) * 4u), tfd::lds_byte_addr(wkd),
                         MT * (RS / 4), RowOff{K, 0, K, nrows, fast_div(RS / 4)});
        else
            stage_slots(RowSlots(w + (int64_t)co0 * K, K, nrows, K, RS, 0, Kp / 4, false), wkd, 0, MT * (Kp / 4));
        for (int k = t; k < Kp; k += kIgThreads) {
            const int kc = min(k, K - 1);
            const int ci = kc / kHW, rem = kc - ci * kHW, kh = rem / kW, kw = rem - kh * kW;
            koffd[k] = (ci * PH + kh * (int)g.dh) * PWs + kw * (int)g.dw;
        }
        __builtin_amdgcn_s_waitcnt(tfd::waitcnt_vm(0));
        __syncthreads();
        const float* wrow = wkd + (m_sub * 32 + l32) * RS + 4 * half;
        if constexpr (MT == 64) {
            // Two accumulators (a register cost that the 32-channel form,
            // two blocks a CU, cannot pay).
            v16f acc0 = v16f{}, acc1 = v16f{};
            mfma_gather_steps2(acc0, acc1, wrow, koffd + 4 * half, patchd + pix_off, 0, KS);
            acc = acc0 + acc1;
        } else {
            acc = mfma_gather_steps(v16f{}, wrow, koffd + 4 * half, patchd + pix_off, 0, KS);
        }
    } else {

    // Two phases: the k steps whose taps lie in the first CA channels, then
    // the rest.  Phase A's filter columns and channels are staged first;
    // phase B's loads are issued into registers before phase A's MFMAs and
    // stored to LDS after them, so their latency overlaps the arithmetic.
    // (A loop over four such phases measured slower: each phase adds a
    // barrier and a staging tail.)
    const int KA8 = C >= 2 ? max(1, min(KS, ((C + 1) / 2) * kHW / 8)) : KS;
    const int CA = min(C, (8 * KA8 + kHW - 1) / kHW);       // channels phase A reads
    const int spr = PWs / 4;
    const RowSlots w_a(w + (int64_t)co0 * K, K, min(MT, Cout - co0), K, RS, 0, 2 * KA8, (vec & 2) != 0);
    const RowSlots w_b(w + (int64_t)co0 * K, K, min(MT, Cout - co0), K, RS, 2 * KA8, Kp / 4 - 2 * KA8, (vec & 2) != 0);
    const float* xn = x + (int64_t)n * C * H * W;
    const PatchSlots p_a(xn, H, W, PH, PWs, L, ih_lo, 0, (vec & 1) != 0);
    const PatchSlots p_b(xn, H, W, PH, PWs, L, ih_lo, CA * PH * spr, (vec & 1) != 0);
    const int n_wb = MT * (Kp / 4 - 2 * KA8), n_pb = (C - CA) * PH * spr;
    for (int k = t; k < Kp; k += kIgThreads) {
        const int kc = min(k, K - 1);
        const int ci = kc / kHW, rem = kc - ci * kHW, kh = rem / kW, kw = rem - kh * kW;
        koff[k] = (ci * PH + kh * (int)g.dh) * PWs + kw * (int)g.dw;
    }
    stage_slots(w_a, wk, 0, MT * 2 * KA8);
    stage_slots(p_a, patch, 0, CA * PH * spr);
    constexpr int kAhead = 6;
    Ahead<kAhead> ahead_w, ahead_p;
    ahead_w.load(w_b, n_wb);
    ahead_p.load(p_b, n_pb);
    __syncthreads();

    const float* wrow = wk + (m_sub * 32 + l32) * RS + 4 * half;
    const int* krow = koff + 4 * half;
    v16f acc0 = v16f{}, acc1 = v16f{};
    if constexpr (MT == 64) mfma_gather_steps2(acc0, acc1, wrow, krow, patch + pix_off, 0, KA8);
    else acc0 = mfma_gather_steps(acc0, wrow, krow, patch + pix_off, 0, KA8);
    if (KA8 < KS) {
        ahead_w.store(wk, n_wb);
        stage_slots(w_b, wk, kAhead * kIgThreads, n_wb);
        ahead_p.store(patch, n_pb);
        stage_slots(p_b, patch, kAhead * kIgThreads, n_pb);
        __syncthreads();
        if constexpr (MT == 64) mfma_gather_steps2(acc0, acc1, wrow, krow, patch + pix_off, KA8, KS);
        else acc0 = mfma_gather_steps(acc0, wrow, krow, patch + pix_off, KA8, KS);
    }
    acc = MT == 64 ? acc0 + acc1 : acc0;
    }

    if (pp >= p_end) return;
    float* yn = y + (int64_t)n * Cout * P;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int co = co0 + m_sub * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (co >= Cout) continue;
        float v = acc[r] + bias_s[co - co0];
        if (relu) v = fmaxf(v, 0.0f);
        yn[(int64_t)co * P + pp] = v;
    }
}

// Patch columns of the forward and weight-gradient kernels: column c holds
// iw = c - L, L = pw (rounded up to 4 for the aligned layout, whose image
// columns start on 16-byte boundaries), PWs = one past the last column a tap
// reads, rounded up to 4.
void patch_cols(const ConvGeom& g, bool aligned, int& L, int& PWs) {
    L = (int)(aligned ? (g.pw + 3) / 4 * 4 : g.pw);
    PWs = (int)((L + (g.outW - 1) * g.sw + (g.kW - 1) * g.dw - g.pw + 1 + 3) / 4 * 4);
}

// Most rows that a run of np consecutive pixels (starting at multiples of np)
// of a rows x cols grid spans.
int64_t rows_spanned(int64_t rows, int64_t cols, int64_t np) {
    const int64_t total = rows * cols;
    int64_t most = 0;
    // A run's start column p0 mod cols repeats after cols / gcd(np, cols) runs.
    for (int64_t k = 0; k < cols && k * np < total; ++k) {
        const int64_t p0 = k * np;
        most = std::max(most, (std::min(p0 + np, total) - 1) / cols - p0 / cols + 1);
    }
    return most;
}

// Dynamic LDS of conv_fwd_implicit_kernel: the 160 KB of a CU less its
// static 256-byte bias table.
constexpr int64_t kFwdDynLds = 160 * 1024 - 256;

// LDS layout of conv_fwd_implicit_kernel (the aligned patch layout when it
// fits, else the tight one), or 0 when neither fits.
size_t implicit_lds_bytes(const ConvGeom& g, int MT, int K, int& Kp, int& PH, int& PWs, int& L, bool& aligned) {
    Kp = (K + 7) / 8 * 8;
    const int np = MT == 64 ? ig_pixels<64>() : ig_pixels<32>();
    PH = (int)((rows_spanned(g.outH, g.outW, np) - 1) * g.sh + (g.kH - 1) * g.dh + 1);
    for (int a = 1; a >= 0; --a) {
        aligned = a != 0;
        patch_cols(g, aligned, L, PWs);
        const int64_t bytes = ((int64_t)MT * (Kp + 4) + Kp + g.C * (int64_t)PH * PWs) * 4;
        if (bytes <= kFwdDynLds) return (size_t)bytes;
    }
    return 0;
}

// ---------------------------------------------------------------------------
// Implicit-GEMM convolution weight gradient (fp32, NCHW, MFMA):
//   dw[co][k] = sum_n sum_p dy[n][co][p] * col[n][k][p]
// with col gathered from x on the fly (nn/Conv2d.cpp:140-260 builds col with
// launch_im2col and multiplies per image).  Blocks tile the pixels as the
// forward does (MT channels x NP pixels of one image, 8 waves); each block
// stages dy's MT x NP tile (dyt[co][p], row stride NP + 4 words), the
// pixel-offset table poff[p], the tap table koff[k] and the input patch (the
// forward's layout), then computes its MT x K partial with
// v_mfma_f32_32x32x2f32 over its pixels (lane half h supplies the pixels of
// its half of each slice for both operands: dy[co][p] and
// patch[koff[k] + poff[p]]).  Work items are (32 x 32 output tile, pixel
// slice): with fewer tiles than waves, each tile's pixels are split over
// several waves and their sums combined in LDS in slice order.  The block
// writes its partial to part[block][co][k]; the partials are then summed in
// a fixed order (tfh::sum_partials).  Pixels past the image's end carry
// dy = 0.
// ---------------------------------------------------------------------------
template <int MT>
__global__ __launch_bounds__(kIgThreads) void conv_bwd_weight_implicit_kernel(const float* __restrict__ x,
                                                                              const float* __restrict__ dy,
                                                                              float* __restrict__ part, ConvGeom g,
                                                                              int Cout, int K, int Kc, int PH, int PWs,
                                                                              int L, int tiles_per_image, int slices,
                                                                              int vec, int with_db,
                                                                              const float* __restrict__ relu_y,
                                                                              float* __restrict__ dz_out) {
    extern __shared__ float smem[];
    constexpr int NP = ig_pixels<MT>();
    constexpr int NH = NP / 2;
    constexpr int RS = NP + 4;                             // RS / 4 odd: no bank conflicts
    const int P = (int)(g.outH * g.outW), outW = (int)g.outW;
    const int n = blockIdx.x / tiles_per_image, pt = blockIdx.x - n * tiles_per_image;
    const int p0 = pt * NP, p_end = min(p0 + NP, P);
    const int co0 = blockIdx.y * MT;
    const int oh_lo = p0 / outW;
    const int ih_lo = oh_lo * (int)g.sh - (int)g.ph;
    const int C = (int)g.C, H = (int)g.H, W = (int)g.W, kHW = (int)(g.kH * g.kW), kW = (int)g.kW;
    const int t = threadIdx.x;
    const int plane = PH * PWs;
    const int nrows = min(MT, Cout - co0);
    float *dyt, *patch, *red;
    int *poff, *koff;
    if (vec & 4) {
        // Direct loads (bit 2: 16-byte dy rows and the aligned patch layout):
        // LDS = dy tile [MT][RS] | input patch (each rounded up to whole KB) |
        // pixel and tap tables | slice sums.  Both regions go global -> LDS
        // in one round trip while the tables are built.
        dyt = smem;
        patch = smem + (MT * RS + 255) / 256 * 256;
        poff = reinterpret_cast<int*>(patch + (C * plane + 255) / 256 * 256);
        koff = poff + NP;
        red = reinterpret_cast<float*>(koff + Kc);
        const float* xn = x + (int64_t)n * C * H * W;
        stage_direct(tfd::buf_rsrc(xn, (uint32_t)(C * H * W) * 4u), tfd::lds_byte_addr(patch), C * PH * (PWs / 4),
                     PatchOff{H, W, PH, L, ih_lo, fast_div(PWs / 4), fast_div(PH)});
        stage_direct(tfd::buf_rsrc(dy + ((int64_t)n * Cout + co0) * P, (uint32_t)(nrows * P) * 4u),
                     tfd::lds_byte_addr(dyt), MT * (RS / 4), RowOff{P, p0, p_end - p0, nrows, fast_div(RS / 4)});
    } else {
        dyt = smem;                                         // [MT][RS]
        poff = reinterpret_cast<int*>(dyt + MT * RS);       // [NP]
        koff = poff + NP;                                   // [Kc]
        patch = reinterpret_cast<float*>(koff + Kc);        // [C][PH][PWs]
        red = patch + C * plane;                            // [8][16][64] when slices > 1
        stage_rows(dy + ((int64_t)n * Cout + co0) * P + p0, P, nrows, p_end - p0, dyt, RS, MT, NP / 4, (vec & 2) != 0);
    }
    for (int q = t; q < NP; q += kIgThreads) {
        const int pp = p0 + q < p_end ? p0 + q : p0;
        const int oh = pp / outW, ow = pp - oh * outW;
        poff[q] = (oh - oh_lo) * (int)g.sh * PWs + ow * (int)g.sw + L - (int)g.pw;
    }
    for (int k = t; k < Kc; k += kIgThreads) {
        const int kc = min(k, K - 1);
        const int ci = kc / kHW, rem = kc - ci * kHW, kh = rem / kW, kw = rem - kh * kW;
        koff[k] = (ci * PH + kh * (int)g.dh) * PWs + kw * (int)g.dw;
    }
    // relu_y: the gradient is taken through a ReLU whose output is relu_y
    // (same shape as dy): dy * (relu_y > 0 ? 1 : 0), as ReluBackward forms
    // it, applied to the staged tile.  The mask values are loaded before
    // the staging wait, so their latency overlaps it.
    constexpr int kMaskPer = MT * NP / kIgThreads;
    float mv[kMaskPer];
    if (relu_y) {
        const float* yb = relu_y + ((int64_t)n * Cout + co0) * P + p0;
#pragma unroll
        for (int u = 0; u < kMaskPer; ++u) {
            const int i = t + kIgThreads * u, r = i / NP, pc = i - r * NP;
            mv[u] = r < nrows && p0 + pc < p_end ? yb[(int64_t)r * P + pc] : 0.0f;
        }
    }
    if (vec & 4) __builtin_amdgcn_s_waitcnt(tfd::waitcnt_vm(0));
    else stage_patch(x + (int64_t)n * C * H * W, patch, C, H, W, PH, PWs, L, ih_lo, (vec & 1) != 0);
    __syncthreads();
    if (relu_y) {
        // dz_out: the masked gradient itself, for the data gradient that
        // follows (these blocks cover every element of dy exactly once).
        float* zb = dz_out ? dz_out + ((int64_t)n * Cout + co0) * P + p0 : nullptr;
#pragma unroll
        for (int u = 0; u < kMaskPer; ++u) {
            const int i = t + kIgThreads * u, r = i / NP, pc = i - r * NP;
            const float v = dyt[r * RS + pc] * (mv[u] > 0.0f ? 1.0f : 0.0f);
            dyt[r * RS + pc] = v;
            if (zb && r < nrows && p0 + pc < p_end) zb[(int64_t)r * P + pc] = v;
        }
        __syncthreads();
    }

    const int wave = t >> 6, lane = t & 63, l32 = lane & 31, half = lane >> 5;
    const int TM = MT / 32, TK = Kc / 32, T = TM * TK;
    const int steps = NH / slices;                          // pixels per slice and lane half (a multiple of 4)
    const int KD = K + with_db;                             // partial row: dw[co][0 .. K) then db[co]
    float* outp = part + (int64_t)blockIdx.x * Cout * KD;
    if (with_db) {
        // db partial: the block's dy row sums (pixels past the image hold 0),
        // lane pairs then a butterfly in a fixed order.
        for (int r = wave; r < MT; r += kIgThreads / 64) {
            const float* row = dyt + r * RS;
            float v = 0.0f;
            for (int q = lane; q < NP; q += 64) v += row[q];
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
            if (lane == 0 && co0 + r < Cout) outp[(int64_t)(co0 + r) * KD + K] = v;
        }
    }
    auto store_tile = [&](int tile, const v16f& acc) {
        const int tr = tile / TK, tc = tile - tr * TK, k = tc * 32 + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int co = co0 + tr * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
            if (co < Cout && k < K) outp[(int64_t)co * KD + k] = acc[r];
        }
    };
    if (slices == 1) {
        // Tiles wave, wave + 8 as a pair (two MFMA chains), then the next
        // pair: the same tiles per wave as one at a time.
        const int q0 = half * NH;
        for (int tile = wave; tile < T; tile += 2 * (kIgThreads / 64)) {
            const int tile2 = tile + kIgThreads / 64;
            const int tr = tile / TK, tc = tile - tr * TK;
            if (tile2 < T) {
                const int tr2 = tile2 / TK, tc2 = tile2 - tr2 * TK;
                v16f acc0, acc1;
                mfma_gather_loop2<true>(dyt + (tr * 32 + l32) * RS + q0, dyt + (tr2 * 32 + l32) * RS + q0, poff + q0,
                                        poff + q0, patch + koff[tc * 32 + l32], patch + koff[tc2 * 32 + l32], NH, acc0,
                                        acc1);
                store_tile(tile, acc0);
                store_tile(tile2, acc1);
            } else {
                // A tile without a partner: its pixels' two halves as the two
                // chains, added at the end.
                v16f acc0, acc1;
                const float* wrow = dyt + (tr * 32 + l32) * RS + q0;
                const float* pb = patch + koff[tc * 32 + l32];
                mfma_gather_loop2<false>(wrow, wrow + NH / 2, poff + q0, poff + q0 + NH / 2, pb, pb, NH / 2, acc0,
                                         acc1);
                store_tile(tile, acc0 + acc1);
            }
        }
    }
    for (int item = wave; slices > 1 && item < T * slices; item += kIgThreads / 64) {
        const int tile = item / slices, sl = item - tile * slices;
        const int tr = tile / TK, tc = tile - tr * TK;
        const int q0 = half * NH + sl * steps;
        const v16f acc = mfma_gather_loop(dyt + (tr * 32 + l32) * RS + q0, poff + q0, patch + koff[tc * 32 + l32],
                                          steps);
        if (slices == 1) {
            const int k = tc * 32 + l32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int co = co0 + tr * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (co < Cout && k < K) outp[(int64_t)co * KD + k] = acc[r];
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
                if (co < Cout && k < K) outp[(int64_t)co * KD + k] = v;
            }
        }
    }
}

// dw[co][k] (k < K) and db[co] (k == K when KD = K + 1) = the sum over the
// weight-gradient blocks b of part[b][co][k].  A workgroup owns EL
// consecutive partial elements x G = 256 / EL block groups; each thread adds
// blocks g, g + G, ... in ascending order (16 loads in flight) and the G
// group sums are combined in a fixed pairwise tree: deterministic.
constexpr int kPsEl = 32;   // partial elements per workgroup (128-byte rows)
template <int EL>
__global__ __launch_bounds__(256) void conv_partial_sum_kernel(const float* __restrict__ part, int blocks,
                                                               int64_t plane, int K, int KD, float* __restrict__ dw,
                                                               float* __restrict__ db) {
    constexpr int G = 256 / EL;
    __shared__ float red[G][EL + 1];
    const int el = threadIdx.x % EL, g = threadIdx.x / EL;
    const int64_t i = (int64_t)blockIdx.x * EL + el;
    float s = 0.0f;
    if (i < plane) {
        const float* src = part + i;
        int b = g;
        for (; b + 15 * G < blocks; b += 16 * G) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) v[u] = src[(int64_t)(b + u * G) * plane];
#pragma unroll
            for (int u = 0; u < 16; ++u) s += v[u];
        }
        for (; b < blocks; b += G) s += src[(int64_t)b * plane];
    }
    red[g][el] = s;
#pragma unroll
    for (int w = G / 2; w >= 1; w >>= 1) {
        __syncthreads();
        if (g < w) red[g][el] += red[g + w][el];
    }
    if (g != 0 || i >= plane) return;
    const float sum = red[0][el];
    const int64_t co = i / KD;
    const int k = (int)(i - co * KD);
    if (k < K) dw[co * K + k] = sum;
    else db[co] = sum;
}

// ---------------------------------------------------------------------------
// Streaming weight gradient for filters with few taps (K = C kH kW <= 31,
// e.g. a first convolution over 3 input channels), where the implicit kernel
// above waits on its staging round trips with little MFMA work to hide them.
// A block takes kWsPixels consecutive pixels of one image and 32 output
// channels.  The input patch those pixels read (a few KB) goes to LDS; dy
// (and the ReLU output y) are read once, straight into registers, every
// load of a thread issued before the patch is waited for (loads retire in
// issue order, so the patch loads go first).  Lane (c = lane % 32,
// h = lane / 32) of wave w holds dy[c][q .. q + 3] for the pixels
// q = 8 j + 4 h of the wave's 8-pixel groups j and feeds them one pixel at a
// time as the A operand of v_mfma_f32_32x32x2f32 (rows = output channels,
// the two lane halves' pixels summed by the instruction), with B = the
// patch value of tap k = lane % 32 at that pixel.  Column k = K carries
// B = 1, so the same MFMAs form the bias gradient sum_p dy[c][p]; columns
// past it carry 0.  The eight waves' 32 x 32 sums are added in wave order
// through LDS and written as the block's partial (part[block][co][0 .. K],
// db at K), which conv_partial_sum_kernel adds in a fixed order: the result
// is deterministic and does not depend on the operands' alignment.
// ---------------------------------------------------------------------------
constexpr int kWsPixels = 512;                                // pixels per block
constexpr int kWsGroups = kWsPixels / 8 / (kIgThreads / 64);  // 8-pixel groups per wave
constexpr int kWsPatchSlots = 4;                              // 16-byte patch slots per thread
constexpr int kWsMaxPatch = kWsPatchSlots * kIgThreads * 4;   // patch floats

// Every load of the kernel below is unconditional (an address clamped into
// the operand, then a select): a branch around a load makes the compiler
// wait for all loads in flight where the paths join, which would put the
// loads back in sequence.
template <bool XVEC, bool DVEC, bool RELU>
__global__ __launch_bounds__(kIgThreads) void conv_bwd_weight_stream_kernel(
    const float* __restrict__ x, const float* __restrict__ dy, const float* __restrict__ relu_y,
    float* __restrict__ dz_out, float* __restrict__ part, ConvGeom g, int Cout, int K, int with_db, int PH, int PWs,
    int L, int tiles_per_image) {
    extern __shared__ float smem[];
    const int C = (int)g.C, H = (int)g.H, W = (int)g.W, kHW = (int)(g.kH * g.kW), kW = (int)g.kW;
    const int P = (int)(g.outH * g.outW), outW = (int)g.outW;
    const int n = blockIdx.x / tiles_per_image, pt = blockIdx.x - n * tiles_per_image;
    const int p0 = pt * kWsPixels, p_end = min(p0 + kWsPixels, P);
    const int co0 = blockIdx.y * 32, nco = min(32, Cout - co0);
    const int oh_lo = p0 / outW, ih_lo = oh_lo * (int)g.sh - (int)g.ph;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, l32 = lane & 31, half = lane >> 5;
    const int spr = PWs / 4, nslots = C * PH * spr;
    float* patch = smem;                                              // [C][PH][PWs]
    int* poff = reinterpret_cast<int*>(smem + 4 * nslots);            // [kWsPixels]
    float* red = reinterpret_cast<float*>(poff + kWsPixels);          // [8 waves][16][64]

    // Patch slots (16 bytes each): patch[ci][rr][c] = x[ci][ih_lo + rr][c - L],
    // zero outside the image.
    const float* xn = x + (int64_t)n * C * H * W;
    const FastDiv fspr = fast_div(spr), fPH = fast_div(PH);
    v4f pv[kWsPatchSlots];
#pragma unroll
    for (int u = 0; u < kWsPatchSlots; ++u) {
        const int i = min(t + kIgThreads * u, nslots - 1);
        int sl, rr;
        const int prow = divmod(i, fspr, sl);
        const int ci = divmod(prow, fPH, rr);
        const int ih = ih_lo + rr, iw = 4 * sl - L;
        const bool row_ok = ih >= 0 && ih < H;
        const int rbase = (ci * H + (row_ok ? ih : 0)) * W;
        if (XVEC) {
            const bool ok = row_ok && iw >= 0 && iw < W;
            const v4f v = *reinterpret_cast<const v4f*>(xn + rbase + (ok ? iw : 0));
            pv[u] = ok ? v : v4f{0.0f, 0.0f, 0.0f, 0.0f};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bool ok = row_ok && iw + e >= 0 && iw + e < W;
                const float v = xn[rbase + (ok ? iw + e : 0)];
                pv[u][e] = ok ? v : 0.0f;
            }
        }
    }
    // This lane's channel and pixels of dy (and y); zeros past the channels
    // and pixels of the block.
    const bool chan = l32 < nco;
    const int64_t row = ((int64_t)n * Cout + co0 + (chan ? l32 : 0)) * P;
    auto load4 = [&](const float* src, int p) -> v4f {
        v4f v;
        if (DVEC) {
            const bool ok = chan && p < p_end;
            v = *reinterpret_cast<const v4f*>(src + row + (ok ? p : p0));
            if (!ok) v = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bool ok = chan && p + e < p_end;
                const float f = src[row + (ok ? p + e : p0)];
                v[e] = ok ? f : 0.0f;
            }
        }
        return v;
    };
    v4f gy[kWsGroups], gm[kWsGroups];
#pragma unroll
    for (int j = 0; j < kWsGroups; ++j) {
        const int p = p0 + 8 * (wave * kWsGroups + j) + 4 * half;
        gy[j] = load4(dy, p);
        if (RELU) gm[j] = load4(relu_y, p);
    }
#pragma unroll
    for (int u = 0; u < kWsPatchSlots; ++u) {
        const int i = t + kIgThreads * u;
        if (i < nslots) *reinterpret_cast<v4f*>(patch + 4 * i) = pv[u];
    }
    for (int q = t; q < kWsPixels; q += kIgThreads) {
        const int pp = p0 + q < p_end ? p0 + q : p0;
        const int oh = pp / outW, ow = pp - oh * outW;
        poff[q] = (oh - oh_lo) * (int)g.sh * PWs + ow * (int)g.sw + L - (int)g.pw;
    }
    // Tap k = l32 of this lane; taps past K read a valid element and are
    // replaced by bk (1 in the bias column, else 0).
    const int kc = min(l32, K - 1);
    const int ci = kc / kHW, rem = kc - ci * kHW, kh = rem / kW, kw = rem - kh * kW;
    const int koff = (ci * PH + kh * (int)g.dh) * PWs + kw * (int)g.dw;
    const bool tap = l32 < K;
    const float bk = with_db && l32 == K ? 1.0f : 0.0f;
    __syncthreads();

    v16f acc = v16f{};
#pragma unroll
    for (int j = 0; j < kWsGroups; ++j) {
        const int q = 8 * (wave * kWsGroups + j) + 4 * half;
        const v4i po = *reinterpret_cast<const v4i*>(poff + q);
        v4f d = gy[j];
        if (RELU) {
            // ReluBackward's dy * (y > 0 ? 1 : 0), and the masked gradient
            // itself for a data gradient that follows (each element once).
#pragma unroll
            for (int e = 0; e < 4; ++e) d[e] *= gm[j][e] > 0.0f ? 1.0f : 0.0f;
            if (dz_out && chan) {
                const int p = p0 + q;
                if (DVEC) {
                    if (p < p_end) *reinterpret_cast<v4f*>(dz_out + row + p) = d;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (p + e < p_end) dz_out[row + p + e] = d[e];
                }
            }
        }
        const float r0 = patch[koff + po.x], r1 = patch[koff + po.y], r2 = patch[koff + po.z],
                    r3 = patch[koff + po.w];
        const float b0 = tap ? r0 : bk, b1 = tap ? r1 : bk, b2 = tap ? r2 : bk, b3 = tap ? r3 : bk;
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(d.x, b0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(d.y, b1, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(d.z, b2, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(d.w, b3, acc, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) red[(wave * 16 + r) * 64 + lane] = acc[r];
    __syncthreads();
    const int KD = K + with_db;
    float* outp = part + (int64_t)blockIdx.x * Cout * KD;
    for (int e = t; e < 16 * 64; e += kIgThreads) {
        const int r = e >> 6, ln = e & 63;
        float v = red[r * 64 + ln];
        for (int w = 1; w < kIgThreads / 64; ++w) v += red[(w * 16 + r) * 64 + ln];
        const int co = co0 + 8 * (r >> 2) + 4 * (ln >> 5) + (r & 3), k = ln & 31;
        if (co < Cout && k < KD) outp[(int64_t)co * KD + k] = v;
    }
}

// LDS layout of conv_bwd_weight_implicit_kernel, or 0 when it does not fit.
size_t implicit_dw_lds_bytes(const ConvGeom& g, int MT, int K, int& Kc, int& PH, int& PWs, int& L, int& slices,
                             bool& aligned) {
    Kc = (K + 31) / 32 * 32;
    const int np = MT == 64 ? ig_pixels<64>() : ig_pixels<32>();
    PH = (int)((rows_spanned(g.outH, g.outW, np) - 1) * g.sh + (g.kH - 1) * g.dh + 1);
    const int tiles = (MT / 32) * (Kc / 32);
    slices = 1;
    while (tiles * slices * 2 <= kIgThreads / 64 && (np / 2) / (slices * 2) >= 4) slices *= 2;
    for (int a = 1; a >= 0; --a) {
        aligned = a != 0;
        patch_cols(g, aligned, L, PWs);
        const int64_t floats = (int64_t)MT * (np + 4) + np + Kc + g.C * (int64_t)PH * PWs +
                               (slices > 1 ? (int64_t)tiles * slices * 16 * 64 : 0);
        if (floats * 4 <= 160 * 1024) return (size_t)(floats * 4);
    }
    return 0;
}

// ---------------------------------------------------------------------------
// Implicit-GEMM convolution data gradient (fp32, NCHW, MFMA):
//   dx[n][c][ih][iw] = sum_co sum_{ki,kj} w[co][c][ki][kj] dy[n][co][oh][ow],
//   oh = (ih + ph - ki dh) / sh, ow = (iw + pw - kj dw) / sw (whole, in range)
// with neither the dcol buffer nor col2im (nn/Conv2d.cpp:178-204 forms
// dcol = W^T dy per image, then launch_col2im, cuda/kernels/col2im.cu:50-80).
//
// Sub-pixel phases: the taps that reach input row ih depend only on
// (ih + ph) mod sh.  Phase (i0, j0), i0 < sh, j0 < sw, holds the pixels
// ih = i0 + sh a, iw = j0 + sw b; its row taps are the ki with
// ki dh = i0 + ph (mod sh), and each reaches oh = a + e(ki) with the whole
// number e(ki) = (i0 + ph - ki dh) / sh (columns likewise, f(kj)).  Within a
// phase the data gradient is therefore a stride-1 correlation of dy, an
// implicit GEMM with M = C (rows c), N = the phase's pixels, and
// K = Cout x row taps x column taps, k = (co, ti, tj):
//   A[c][k] = w[co][c][ki(ti)][kj(tj)],  B[k][(a, b)] = dy[co][a + e][b + f].
// A block (8 waves, two per SIMD) takes MT input channels x NP consecutive
// pixels of one phase of one image and lays out LDS as the forward kernel
// does: the MT filter rows split by k parity, the tap offset table split the
// same way, and the dy patch [Cout][PH][PW] its pixels read (dy rows
// a_lo + e_min .. , columns f_min .. , zero outside dy).  A phase without
// taps (possible for sh > kH dh, or dilations sharing a residue) has K = 0
// and stores zeros.  The sum for one dx element runs over k in (co, ti, tj)
// order, fixed per geometry: deterministic.
// ---------------------------------------------------------------------------
struct PhaseTaps {
    int n;         // taps of this phase along the axis
    int e_min;     // smallest offset e(k) over them
    int span;      // e_max - e_min (0 without taps)
};

// Taps of phase r0 (< s) along one axis: k in [0, kk) with k d = r0 + p (mod s),
// e(k) = (r0 + p - k d) / s.
__host__ __device__ inline PhaseTaps phase_taps(int r0, int p, int kk, int s, int d) {
    PhaseTaps t{0, 0, 0};
    int e_max = 0;
    for (int k = 0; k < kk; ++k) {
        const int num = r0 + p - k * d;
        if (((num % s) + s) % s != 0) continue;
        const int e = num / s;
        if (t.n == 0 || e < t.e_min) t.e_min = e;
        if (t.n == 0 || e > e_max) e_max = e;
        ++t.n;
    }
    t.span = t.n ? e_max - t.e_min : 0;
    return t;
}

// The ti-th tap (in increasing k) of phase r0 along one axis; ti < its count.
__device__ inline int phase_tap(int r0, int p, int kk, int s, int d, int ti) {
    for (int k = 0; k < kk; ++k) {
        const int num = r0 + p - k * d;
        if (((num % s) + s) % s != 0) continue;
        if (ti-- == 0) return k;
    }
    return 0;
}

template <int MT>
__global__ __launch_bounds__(kIgThreads) void conv_bwd_data_implicit_kernel(const float* __restrict__ dy,
                                                                            const float* __restrict__ w,
                                                                            float* __restrict__ dx, ConvGeom g,
                                                                            int Cout, int PH, int PWs, int L,
                                                                            int tiles_per_phase, int vec) {
    extern __shared__ float smem[];
    constexpr int NP = ig_pixels<MT>();
    constexpr int MSUB = MT / 32;
    const int sh = (int)g.sh, sw = (int)g.sw;
    const int phases = sh * sw;
    // Block b runs on XCD b % 8 and the phases carry different numbers of
    // taps, so consecutive groups of 8 blocks take consecutive phases: each
    // XCD's share cycles through all of them.  Block (q = b / 8, x = b % 8):
    // phase q % phases, image tile r = (q / phases) 8 + x = n tiles + pt.
    const int q8 = blockIdx.x >> 3;
    const int phase = q8 % phases;
    const int r = (q8 / phases) * 8 + (blockIdx.x & 7);
    if (r >= (int)g.N * tiles_per_phase) return;         // uniform per block
    const int n = r / tiles_per_phase, pt = r - n * tiles_per_phase;
    const int i0 = phase / sw, j0 = phase - i0 * sw;
    const int H = (int)g.H, W = (int)g.W;
    const int Ha = i0 < H ? (H - i0 + sh - 1) / sh : 0;
    const int Wb = j0 < W ? (W - j0 + sw - 1) / sw : 0;
    const int Pph = Ha * Wb;
    const int p0 = pt * NP;
    if (p0 >= Pph) return;                               // uniform per block
    const int p_end = min(p0 + NP, Pph);
    const int kH = (int)g.kH, kW = (int)g.kW, dh = (int)g.dh, dwl = (int)g.dw;
    const int ph = (int)g.ph, pw = (int)g.pw;
    const PhaseTaps th = phase_taps(i0, ph, kH, sh, dh), tw = phase_taps(j0, pw, kW, sw, dwl);
    const int taps = th.n * tw.n;
    const int K = Cout * taps;
    const int Kp = max(8, (K + 7) / 8 * 8);
    const int KH2 = Kp / 2;
    const int RS = Kp + 4;                               // RS / 4 odd: no bank conflicts
    const int C = (int)g.C, outH = (int)g.outH, outW = (int)g.outW;
    const int c0 = blockIdx.y * MT;
    const int a_lo = p0 / Wb;
    const int kHW = kH * kW;
    float* wk = smem;                                    // [MT][RS]
    int* koff = reinterpret_cast<int*>(wk + MT * RS);    // [Kp]
    int* tap_w = koff + Kp;                              // [kH kW]: ki kW + kj of tap tt
    int* tap_p = tap_w + kHW;                            // [kH kW]: its dy patch offset
    float* patch = smem + (((MT * RS + Kp + 2 * kHW) + 3) & ~3);  // [Cout][PH][PWs]
    const int t = threadIdx.x;

    // Tap tt = (ti, tj) of this phase: its filter position and patch offset
    // (patch row e - e_min, column b + f + L for pixel column b).
    for (int tt = t; tt < taps; tt += kIgThreads) {
        const int ti = tt / tw.n, tj = tt - ti * tw.n;
        const int ki = phase_tap(i0, ph, kH, sh, dh, ti), kj = phase_tap(j0, pw, kW, sw, dwl, tj);
        tap_w[tt] = ki * kW + kj;
        tap_p[tt] = ((i0 + ph - ki * dh) / sh - th.e_min) * PWs + (j0 + pw - kj * dwl) / sw + L;
    }
    __syncthreads();

    constexpr int kStage = 16;
    const FastDiv ftaps = fast_div(max(taps, 1));
    // Filter columns: i = k MT + r (r fastest: consecutive lanes read
    // consecutive input channels, kH kW floats apart).
    for (int base = t; base < MT * Kp; base += kIgThreads * kStage) {
        float v[kStage];
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int i = base + kIgThreads * u;
            const int r = i & (MT - 1), k = i / MT;
            float val = 0.0f;
            if (i < MT * Kp && c0 + r < C && k < K) {
                int tt;
                const int co = divmod(k, ftaps, tt);
                val = w[((int64_t)co * C + c0 + r) * kHW + tap_w[tt]];
            }
            v[u] = val;
        }
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int i = base + kIgThreads * u;
            if (i < MT * Kp) wk[(i & (MT - 1)) * RS + i / MT] = v[u];
        }
    }
    for (int k = t; k < Kp; k += kIgThreads) {
        int tt = 0, co = 0;
        if (K > 0) co = divmod(min(k, K - 1), ftaps, tt);
        koff[k] = K > 0 ? co * PH * PWs + tap_p[tt] : 0;
    }
    if (K > 0)
        stage_patch(dy + (int64_t)n * Cout * outH * outW, patch, Cout, outH, outW, PH, PWs, L, a_lo + th.e_min,
                    vec != 0);
    __syncthreads();

    const int wave = t >> 6, lane = t & 63, l32 = lane & 31, half = lane >> 5;
    const int m_sub = wave % MSUB, n_sub = wave / MSUB;
    const int pp = p0 + n_sub * 32 + l32;
    int pix_off;
    {
        const int q = pp < p_end ? pp : p0;
        const int a = q / Wb, bb = q - a * Wb;
        pix_off = (a - a_lo) * PWs + bb;
    }
    const v16f acc = K > 0 ? mfma_gather_loop(wk + (m_sub * 32 + l32) * RS + half * KH2, koff + half * KH2,
                                              patch + pix_off, KH2)
                           : v16f{};

    if (pp >= p_end) return;
    const int a = pp / Wb, bb = pp - a * Wb;
    float* dxn = dx + (int64_t)n * C * H * W + (int64_t)(i0 + sh * a) * W + (j0 + sw * bb);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int c = c0 + m_sub * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (c < C) dxn[(int64_t)c * H * W] = acc[r];
    }
}

// ---------------------------------------------------------------------------
// Data gradient for convolutions with at most 256 output pixels per image
// (strided layers): per image, the column gradient of a group of CG input
// channels, dcol[m][p] = sum_co w[co][c0 + m / kk][m % kk] dy[n][co][p]
// (m < CG kk, kk = kH kW), is formed on MFMA straight into LDS, and the
// block then gathers it into dx (col2im from LDS).  nn/Conv2d.cpp:178-204
// writes dcol for the whole batch to memory and launch_col2im reads it back.
//
// Block (8 waves) = one image x one channel group.  The K loop runs over co
// in chunks of KC: LDS holds A[m][k] = w[k0 + k][c0 + m/kk][m%kk] (row stride
// KC + 4) and B[k][p] = dy[n][k0 + k][p] (row stride 272, columns >= P zero);
// wave w owns pixels 32 w .. 32 w + 31 (two 16-column tiles) and all R row
// tiles of 16 (M = CG kk <= 16 R; tiles past M read rows that are never
// stored, within the LDS allocation), with v_mfma_f32_16x16x4f32: per four
// co, the R A reads and two B reads are issued together, then the 2 R
// MFMAs.  Both strides keep the reads free of bank conflicts.  After the K
// loop the accumulators go to LDS as D[m][p] (row stride 260, conflict-free
// for the stores), and each thread sums, for its dx elements, the taps
// reaching them in (ki, kj) order, as col2im does, from two small tables
// built at the start: per input row the D offsets ki kW RD + oh outW of its
// row taps, per input column the offsets kj RD + ow of its column taps.
// ---------------------------------------------------------------------------
constexpr int kDlxRB = 256 + 16;     // B row stride (words)
constexpr int kDlxRD = 256 + 4;      // D row stride (words)

// col2im from LDS with lane <-> input column, MT the most row taps and the
// most column taps of any input pixel (2 for stride-2 3 x 3 layers): a
// thread's column taps sit in registers, each output reads all MT x MT
// candidates unconditionally (invalid ones at offset 0, a valid address)
// and adds the valid ones in (ki, kj) order, so the LDS reads of an output
// go out together instead of one branch and one wait per tap.  Adding +0.0
// for an invalid tap leaves the sum's bits unchanged (a sum that starts at
// +0.0 is never -0.0), so the result equals the tap-by-tap loop.
template <int MT>
__device__ __forceinline__ void col2im_cols(const float* Ds, float* __restrict__ dxn, const int* rcnt,
                                            const int* roff, const int* ccnt, const int* coff, int CGv, int H,
                                            int W, int kH, int kW, int rpp, int slot, int iw) {
    const int HW = H * W, kk = kH * kW;
    const int nc = ccnt[iw];
    int cof[MT];
#pragma unroll
    for (int b = 0; b < MT; ++b) cof[b] = b < nc ? coff[iw * kW + b] : 0;
    if (rpp <= H) {
        // Rows ih = slot, slot + rpp, ...: a row's taps go to registers once
        // and the channel group is walked under them.
        for (int ih = slot; ih < H; ih += rpp) {
            const int nr = rcnt[ih];
            float* out = dxn + ih * W + iw;
            const float* dc = Ds;
            if (nr <= MT) {
                int ro[MT];
#pragma unroll
                for (int a = 0; a < MT; ++a) ro[a] = a < nr ? roff[ih * kH + a] : 0;
#pragma unroll(MT == 2 ? 2 : 1)
                for (int cl = 0; cl < CGv; ++cl, dc += kk * kDlxRD, out += HW) {
                    float v[MT][MT];
#pragma unroll
                    for (int a = 0; a < MT; ++a)
#pragma unroll
                        for (int b = 0; b < MT; ++b) v[a][b] = dc[ro[a] + cof[b]];
                    float sum = 0.0f;
#pragma unroll
                    for (int a = 0; a < MT; ++a)
#pragma unroll
                        for (int b = 0; b < MT; ++b) sum += a < nr && b < nc ? v[a][b] : 0.0f;
                    *out = sum;
                }
            } else {
                for (int cl = 0; cl < CGv; ++cl, dc += kk * kDlxRD, out += HW) {
                    float sum = 0.0f;
                    for (int a = 0; a < nr; ++a) {
                        const float* drow = dc + roff[ih * kH + a];
                        float v[MT];
#pragma unroll
                        for (int b = 0; b < MT; ++b) v[b] = drow[cof[b]];
#pragma unroll
                        for (int b = 0; b < MT; ++b) sum += b < nc ? v[b] : 0.0f;
                    }
                    *out = sum;
                }
            }
        }
        return;
    }
    const int dcl = rpp / H, dih = rpp - dcl * H;
    int cl = slot / H, ih = slot - cl * H;
    for (int r = slot; r < CGv * H; r += rpp) {
        const float* dc = Ds + cl * kk * kDlxRD;
        const int nr = rcnt[ih];
        float sum = 0.0f;
        for (int a = 0; a < nr; ++a) {
            const float* drow = dc + roff[ih * kH + a];
            float v[MT];
#pragma unroll
            for (int b = 0; b < MT; ++b) v[b] = drow[cof[b]];
#pragma unroll
            for (int b = 0; b < MT; ++b) sum += b < nc ? v[b] : 0.0f;
        }
        dxn[cl * HW + ih * W + iw] = sum;
        ih += dih;
        cl += dcl;
        if (ih >= H) {
            ih -= H;
            ++cl;
        }
    }
}

// col2im from LDS, NT threads: dx[cl][ih][iw] (dxn = the group's first
// channel) = sum over its row taps (ki order) and column taps (kj order) of
// D[cl kk + ki kW + kj][oh outW + ow], D with row stride kDlxRD.  taps: 2
// when W <= NT and no input pixel has more than two row or two column taps,
// 4 when W <= NT and none more than four column taps, else 0 (a loop per
// element).
template <int NT>
__device__ __forceinline__ void col2im_from_lds(const float* Ds, float* __restrict__ dxn, const int* rcnt,
                                                const int* roff, const int* ccnt, const int* coff, int CGv, int H,
                                                int W, int kH, int kW, int taps, int t) {
    if (taps) {
        const int rpp = NT / W, slot = t / W, iw = t - slot * W;
        if (slot >= rpp) return;
        if (taps == 2)
            col2im_cols<2>(Ds, dxn, rcnt, roff, ccnt, coff, CGv, H, W, kH, kW, rpp, slot, iw);
        else
            col2im_cols<4>(Ds, dxn, rcnt, roff, ccnt, coff, CGv, H, W, kH, kW, rpp, slot, iw);
        return;
    }
    const int HW = H * W, kk = kH * kW;
    const FastDiv fHW = fast_div(HW), fW = fast_div(W);
    for (int e = t; e < CGv * HW; e += NT) {
        int rem, iw;
        const int cl = divmod(e, fHW, rem);
        const int ih = divmod(rem, fW, iw);
        const float* dc = Ds + cl * kk * kDlxRD;
        const int nr = rcnt[ih], nc = ccnt[iw];
        float sum = 0.0f;
        for (int a = 0; a < nr; ++a) {
            const float* drow = dc + roff[ih * kH + a];
            for (int b = 0; b < nc; ++b) sum += drow[coff[iw * kW + b]];
        }
        dxn[e] = sum;
    }
}

// kDlxR row tiles of 16 (M <= 16 kDlxR), kDlxKC co per K chunk: <9, 64> (one
// block per CU) or <5, 32> (two blocks per CU, whose phases then overlap).
template <int kDlxR, int kDlxKC>
__global__ __launch_bounds__(kIgThreads) void conv_bwd_data_lds_kernel(const float* __restrict__ dy,
                                                                       const float* __restrict__ w,
                                                                       float* __restrict__ dx, ConvGeom g, int Cout,
                                                                       int CG, int RT, int tab_off, int vec,
                                                                       int taps) {
    extern __shared__ float smem[];
    const int C = (int)g.C, H = (int)g.H, W = (int)g.W, outW = (int)g.outW, outH = (int)g.outH;
    const int P = outH * outW, kH = (int)g.kH, kW = (int)g.kW, kk = kH * kW;
    const int groups = (C + CG - 1) / CG;
    // Workgroups go to the 8 XCDs round-robin (block b to XCD b % 8): XCD x
    // takes the x-th contiguous eighth of the (image, group) list, so the
    // groups of one image, which all read that image's dy, run side by side
    // on one XCD and share its L2.
    int wi = (int)blockIdx.x;
    {
        const int nb = (int)gridDim.x, q8 = nb >> 3, r8 = nb & 7, x = wi & 7, s = wi >> 3;
        wi = x < r8 ? x * (q8 + 1) + s : r8 * (q8 + 1) + (x - r8) * q8 + s;
    }
    const int n = wi / groups, c0 = (wi - n * groups) * CG;
    const int CGv = min(CG, C - c0), Mv = CGv * kk, Mp = RT * 16;
    // A is stored k-major, As[k][m] with row stride 16 R words (80 or 144, both
    // 16 mod 64, so the four k rows of one MFMA operand read hit different
    // banks): a k row is CG kk consecutive filter elements, which direct
    // loads copy as they are.
    constexpr int RAk = 16 * kDlxR;
    float* As = smem;                                     // [KC][RAk]
    float* Bs = smem + kDlxKC * RAk;                      // [KC][kDlxRB]
    // Tap tables (after the larger of the two phases' layouts):
    int* rcnt = reinterpret_cast<int*>(smem + tab_off);   // [H]
    int* roff = rcnt + H;                                 // [H][kH]
    int* ccnt = roff + H * kH;                            // [W]
    int* coff = ccnt + W;                                 // [W][kW]
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, l16 = lane & 15, q = lane >> 4;
    build_tap_tables<kIgThreads>(g, kDlxRD, rcnt, roff, ccnt, coff, t);
    v4f acc[kDlxR][2];
#pragma unroll
    for (int r = 0; r < kDlxR; ++r) acc[r][0] = acc[r][1] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    const float* dyn = dy + (int64_t)n * Cout * P;
    for (int k0 = 0; k0 < Cout; k0 += kDlxKC) {
        const int kc = min(kDlxKC, Cout - k0), kcp = (kc + 3) & ~3;
        // Bit 0 of vec: dy rows by direct loads (16-byte rows); bit 1: the
        // filter rows too (C kk and CG kk multiples of 4, w 16-byte aligned).
        // Rows kc .. kcp - 1 and columns past P read as zeros.
        if (vec & 1)
            stage_direct(tfd::buf_rsrc(dyn + (int64_t)k0 * P, (uint32_t)(kc * P) * 4u), tfd::lds_byte_addr(Bs),
                         kcp * (kDlxRB / 4), RowOff{P, 0, P, kc, fast_div(kDlxRB / 4)});
        else
            stage_rows(dyn + (int64_t)k0 * P, P, kc, P, Bs, kDlxRB, kcp, kDlxRB / 4 - 4, false);
        if (vec & 2) {
            stage_direct(tfd::buf_rsrc(w + (int64_t)k0 * C * kk, (uint32_t)(kc * C * kk) * 4u), tfd::lds_byte_addr(As),
                         kcp * (RAk / 4), RowOff{C * kk, c0 * kk, Mv, kc, fast_div(RAk / 4)});
        } else {
            // i = k Mp + m: consecutive m read consecutive filter elements.
            const FastDiv fMp = fast_div(Mp);
            for (int i = t; i < kcp * Mp; i += kIgThreads) {
                int m;
                const int k = divmod(i, fMp, m);
                As[k * RAk + m] = (k < kc && m < Mv) ? w[((int64_t)(k0 + k) * C + c0) * kk + m] : 0.0f;
            }
        }
        if (vec & 3) __builtin_amdgcn_s_waitcnt(tfd::waitcnt_vm(0));
        __syncthreads();
        for (int s = 0; s < kcp; s += 4) {
            const float* brow = Bs + (s + q) * kDlxRB + wave * 32 + l16;
            const float b0 = brow[0], b1 = brow[16];
            float a[kDlxR];
#pragma unroll
            for (int r = 0; r < kDlxR; ++r) a[r] = As[(s + q) * RAk + r * 16 + l16];
#pragma unroll
            for (int r = 0; r < kDlxR; ++r) {
                acc[r][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[r], b0, acc[r][0], 0, 0, 0);
                acc[r][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[r], b1, acc[r][1], 0, 0, 0);
            }
        }
        __syncthreads();
    }
    // D[m][p]: lane holds rows 16 r + 4 q + i, column 32 wave + 16 ct + l16.
    float* Ds = smem;
#pragma unroll
    for (int r = 0; r < kDlxR; ++r) {
        if (r < RT) {
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (r * 16 + 4 * q + i < Mv) Ds[(r * 16 + 4 * q + i) * kDlxRD + wave * 32 + ct * 16 + l16] = acc[r][ct][i];
        }
    }
    __syncthreads();
    col2im_from_lds<kIgThreads>(Ds, dx + ((int64_t)n * C + c0) * H * W, rcnt, roff, ccnt, coff, CGv, H, W, kH, kW,
                                taps, t);
}

// LDS bytes, channel group and tap-table offset (words) of
// conv_bwd_data_lds_kernel<R, KC>, or 0 when the shape is not its kind (more
// than 256 output pixels, or no channel group whose D tile fits `limit`).
size_t dx_lds_bytes(const ConvGeom& g, int R, int KC, int64_t limit, int& CG, int& RT, int& tab_off) {
    const int64_t P = g.outH * g.outW, kk = g.kH * g.kW;
    if (P > 256 || kk > 16 * R) return 0;
    CG = (int)std::min<int64_t>(g.C, 16 * R / kk);
    RT = (int)((CG * kk + 15) / 16);
    if ((int64_t)CG * g.H * g.W >= (1 << 22)) return 0;
    // Phase 1: As [KC][16 R] (row tiles past RT read columns of it that
    // are computed and dropped) and Bs [KC][kDlxRB].  Phase 2 stores the CG kk
    // rows of D.
    const int64_t phase1 = (int64_t)KC * 16 * R + (int64_t)KC * kDlxRB;
    const int64_t phase2 = (int64_t)CG * kk * kDlxRD;
    tab_off = (int)std::max(phase1, phase2);
    const int64_t tables = g.H * (1 + g.kH) + g.W * (1 + g.kW);
    const int64_t bytes = (tab_off + tables) * 4;
    return bytes <= limit ? (size_t)bytes : 0;
}

// LDS layout of conv_bwd_data_implicit_kernel (the largest phase), or 0 when
// it does not fit; tpp = pixel tiles of the largest phase.  Patch columns:
// column c holds dy column c - L, L = the most negative column offset of
// any phase's taps (rounded up to 4 for the aligned layout when that fits).
size_t implicit_dx_lds_bytes(const ConvGeom& g, int MT, int Cout, int& PH, int& PWs, int& L, int& tpp,
                             bool& aligned) {
    const int np = MT == 64 ? ig_pixels<64>() : ig_pixels<32>();
    PH = 1;
    tpp = 1;
    int64_t kmax = 0, neg = 0, right = 1;
    for (int i0 = 0; i0 < g.sh; ++i0) {
        const PhaseTaps th = phase_taps(i0, (int)g.ph, (int)g.kH, (int)g.sh, (int)g.dh);
        const int64_t Ha = i0 < g.H ? (g.H - i0 + g.sh - 1) / g.sh : 0;
        for (int j0 = 0; j0 < g.sw; ++j0) {
            const PhaseTaps tw = phase_taps(j0, (int)g.pw, (int)g.kW, (int)g.sw, (int)g.dw);
            const int64_t Wb = j0 < g.W ? (g.W - j0 + g.sw - 1) / g.sw : 0;
            if (Ha == 0 || Wb == 0) continue;
            tpp = std::max<int>(tpp, (int)((Ha * Wb + np - 1) / np));
            const int64_t rows = rows_spanned(Ha, Wb, np);                  // phase rows a tile touches
            PH = std::max<int>(PH, (int)(rows + th.span));
            kmax = std::max<int64_t>(kmax, (int64_t)Cout * th.n * tw.n);
            if (tw.n) {
                neg = std::max<int64_t>(neg, -(int64_t)tw.e_min);
                right = std::max<int64_t>(right, Wb + tw.e_min + tw.span);   // columns b + f < this
            }
        }
    }
    const int64_t kp = std::max<int64_t>(8, (kmax + 7) / 8 * 8);
    const int64_t head = ((int64_t)MT * (kp + 4) + kp + 2 * g.kH * g.kW + 3) / 4 * 4;
    for (int a = 1; a >= 0; --a) {
        aligned = a != 0;
        L = (int)(aligned ? (neg + 3) / 4 * 4 : neg);
        PWs = (int)((L + right + 3) / 4 * 4);
        const int64_t bytes = (head + (int64_t)Cout * PH * PWs) * 4;
        if (bytes <= 160 * 1024) return (size_t)bytes;
    }
    return 0;
}

// The plane forms' 32-bit index arithmetic stays in range: every input
// coordinate they form lies within +-2^24.
bool plane_indices_fit(const ConvGeom& g) {
    const int64_t lim = 1LL << 24;
    return (g.outH - 1) * g.sh + (g.kH - 1) * g.dh < lim && (g.outW - 1) * g.sw + (g.kW - 1) * g.dw < lim &&
           g.ph < lim && g.pw < lim && g.H < lim && g.W < lim;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

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
    if (dtype != TF_F32 && dtype != TF_BF16 && dtype != TF_F16)
        return tfh::set_error(TF_ERR_UNSUPPORTED, "tf_im2col: dtype must be Float32, Float16 or BFloat16");
    const int64_t planes = N * C, sp = g.outH * g.outW, kk = kH * kW;
    if (H * W <= kPlaneLdsFloats && kk * sp <= (1LL << 30) && planes >= 256 && planes < (1LL << 31) &&
        plane_indices_fit(g)) {
        // Row groups of about 4096 outputs per block.
        const int64_t groups = std::min<int64_t>({kk, std::max<int64_t>(1, (kk * sp) / 4096), 1024});
        const int rpb = (int)((kk + groups - 1) / groups);
        const dim3 grid((unsigned)planes, (unsigned)((kk + rpb - 1) / rpb));
        const size_t lds = (size_t)(H * W) * sizeof(float);
        if (dtype == TF_F32 && g.outW % 4 == 0 && aligned16(col))
            im2col_plane4_kernel<<<grid, 256, lds, ctx->stream>>>((const float*)x, (float*)col, g, rpb);
        else if (dtype == TF_F32)
            im2col_plane_kernel<float><<<grid, 256, lds, ctx->stream>>>((const float*)x, (float*)col, g, rpb);
        else if (dtype == TF_BF16)
            im2col_plane_kernel<uint16_t><<<grid, 256, lds, ctx->stream>>>((const uint16_t*)x, (uint16_t*)col, g, rpb);
        else
            im2col_plane_kernel<_Float16><<<grid, 256, lds, ctx->stream>>>((const _Float16*)x, (_Float16*)col, g, rpb);
        return tfh::check_launch("im2col_plane_kernel");
    }
    if (dtype == TF_F32)
        im2col_kernel<float><<<tfd::grid_for(total, 4), 256, 0, ctx->stream>>>((const float*)x, (float*)col, g);
    else if (dtype == TF_BF16)
        im2col_kernel<uint16_t><<<tfd::grid_for(total, 4), 256, 0, ctx->stream>>>((const uint16_t*)x, (uint16_t*)col, g);
    else
        im2col_kernel<_Float16><<<tfd::grid_for(total, 4), 256, 0, ctx->stream>>>((const _Float16*)x, (_Float16*)col, g);
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
    if (dtype != TF_F32 && dtype != TF_BF16 && dtype != TF_F16)
        return tfh::set_error(TF_ERR_UNSUPPORTED, "tf_col2im: dtype must be Float32, Float16 or BFloat16");
    const int64_t planes = N * C, n_col = kH * kW * g.outH * g.outW;
    const int64_t tables = H * (1 + kH) + W * (1 + kW);
    if (n_col + tables <= kPlaneLdsFloats && H * W < (1LL << 30) && planes >= 256 && planes < (1LL << 31) &&
        plane_indices_fit(g)) {
        // The most row taps and column taps of any input pixel (an upper
        // bound: taps by residue class, before the image edges).
        int mt = 0;
        for (int64_t i0 = 0; i0 < sh; ++i0) mt = std::max(mt, phase_taps((int)i0, (int)ph, (int)kH, (int)sh, (int)dh).n);
        for (int64_t j0 = 0; j0 < sw; ++j0) mt = std::max(mt, phase_taps((int)j0, (int)pw, (int)kW, (int)sw, (int)dw).n);
        const size_t lds = (size_t)(n_col + tables) * sizeof(float);
#define TF_C2I_PLANE(T, MT)                                                                                   \
    col2im_plane_kernel<T, MT><<<(unsigned)planes, 256, lds, ctx->stream>>>((const T*)col, (T*)dx, g)
#define TF_C2I_PLANE_MT(T)                                                                                    \
    do {                                                                                                      \
        if (mt <= 1) TF_C2I_PLANE(T, 1);                                                                      \
        else if (mt == 2) TF_C2I_PLANE(T, 2);                                                                 \
        else if (mt == 3) TF_C2I_PLANE(T, 3);                                                                 \
        else if (mt == 4) TF_C2I_PLANE(T, 4);                                                                 \
        else TF_C2I_PLANE(T, 0);                                                                              \
    } while (0)
        if (dtype == TF_F32)
            TF_C2I_PLANE_MT(float);
        else if (dtype == TF_BF16)
            TF_C2I_PLANE_MT(uint16_t);
        else
            TF_C2I_PLANE_MT(_Float16);
#undef TF_C2I_PLANE_MT
#undef TF_C2I_PLANE
        return tfh::check_launch("col2im_plane_kernel");
    }
    if (dtype == TF_F32)
        col2im_kernel<float><<<tfd::grid_for(total, 2), 256, 0, ctx->stream>>>((const float*)col, (float*)dx, g);
    else if (dtype == TF_BF16)
        col2im_kernel<uint16_t><<<tfd::grid_for(total, 2), 256, 0, ctx->stream>>>((const uint16_t*)col, (uint16_t*)dx, g);
    else
        col2im_kernel<_Float16><<<tfd::grid_for(total, 2), 256, 0, ctx->stream>>>((const _Float16*)col, (_Float16*)dx, g);
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
    int Kp, PH, PWs, L;
    bool aligned;
    const size_t lds = implicit_lds_bytes(g, MT, (int)K, Kp, PH, PWs, L, aligned);
    if (lds == 0)
        return tfh::set_error(TF_ERR_UNSUPPORTED, "tf_conv2d_fwd: filter rows and input patch exceed the 160 KB of LDS "
                                                  "(use tf_im2col + tf_gemm_ex)");
    const int64_t P = g.outH * g.outW;
    const int np = MT == 64 ? ig_pixels<64>() : ig_pixels<32>();
    const int tpi = (int)((P + np - 1) / np);
    TF_REQUIRE(N * tpi < (1LL << 31), "tf_conv2d_fwd: too many blocks");
    // 16-byte staging loads: bit 0 input rows, bit 1 filter rows; bit 2: the
    // direct-load layout (aligned 16-byte input rows, regions in whole KB),
    // when it fits.
    int vec = (aligned && W % 4 == 0 && aligned16(x) ? 1 : 0) | (K % 4 == 0 && aligned16(w) ? 2 : 0);
    size_t lds_launch = lds;
    if (vec & 1) {
        const int64_t direct = ((MT * (int64_t)(Kp + 4) + 255) / 256 * 256 + (C * (int64_t)PH * PWs + 255) / 256 * 256 +
                                Kp) * 4;
        if (direct <= kFwdDynLds) {
            vec |= 4;
            lds_launch = (size_t)direct;
        }
    }
    const dim3 grid((unsigned)(N * tpi), (unsigned)((Cout + MT - 1) / MT));
    // Dynamic LDS above 64 KB needs the attribute; set once per kernel to the
    // whole 160 KB, before any launch (and any graph capture) uses it.
    static const bool lds_ok = [] {
        const int all = (int)kFwdDynLds;
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
        conv_fwd_implicit_kernel<32><<<grid, kIgThreads, lds_launch, ctx->stream>>>(x, w, bias, y, g, (int)Cout, (int)K,
                                                                                    Kp, PH, PWs, L, tpi, relu, vec);
    } else {
        conv_fwd_implicit_kernel<64><<<grid, kIgThreads, lds_launch, ctx->stream>>>(x, w, bias, y, g, (int)Cout, (int)K,
                                                                                    Kp, PH, PWs, L, tpi, relu, vec);
    }
    return tfh::check_launch("conv_fwd_implicit_kernel");
}

}  // extern "C"

namespace {

tf_status conv_bwd_weight_impl(tf_ctx* ctx, const float* x, const float* dy, const float* relu_y, float* dz,
                               float* dw, float* db, int64_t N, int64_t C, int64_t H, int64_t W, int64_t Cout,
                               int64_t kH, int64_t kW, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh,
                               int64_t dw_) {
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
    if (N == 0) {
        st = tf_hip_fill_f32(ctx, dw, 0.0f, Cout * K);
        return st == TF_OK && db ? tf_hip_fill_f32(ctx, db, 0.0f, Cout) : st;
    }
    const int with_db = db ? 1 : 0;
    const int64_t KD = K + with_db;
    const int64_t plane = Cout * KD;
    if (K <= 31) {
        // Few filter taps: conv_bwd_weight_stream_kernel, when its patch fits.
        const bool xal = g.W % 4 == 0 && aligned16(x);
        int Ls, PWss;
        patch_cols(g, xal, Ls, PWss);
        const int PHs = (int)((rows_spanned(g.outH, g.outW, kWsPixels) - 1) * g.sh + (g.kH - 1) * g.dh + 1);
        const int64_t pfl = C * (int64_t)PHs * PWss;
        if (pfl <= kWsMaxPatch) {
            const int64_t P = g.outH * g.outW;
            const bool dvec = P % 4 == 0 && aligned16(dy) && (!relu_y || aligned16(relu_y)) && (!dz || aligned16(dz));
            const int64_t tpi = (P + kWsPixels - 1) / kWsPixels;
            const int64_t blocks = N * tpi;
            TF_REQUIRE(blocks < (1LL << 31), "tf_conv2d_bwd_weight: too many blocks");
            st = tfh::ensure_workspace(ctx, (size_t)blocks * Cout * KD * sizeof(float));
            if (st != TF_OK) return st;
            float* part = reinterpret_cast<float*>(ctx->ws);
            // <= 32 + 2 + 32 KB: within the default dynamic LDS limit.
            const size_t lds = (size_t)(pfl + kWsPixels + (kIgThreads / 64) * 16 * 64) * 4;
            const dim3 grid((unsigned)blocks, (unsigned)((Cout + 31) / 32));
            const int sel = (xal ? 4 : 0) | (dvec ? 2 : 0) | (relu_y ? 1 : 0);
#define TF_WS_LAUNCH(XV, DV, RL)                                                                               \
    conv_bwd_weight_stream_kernel<XV, DV, RL><<<grid, kIgThreads, lds, ctx->stream>>>(                      \
        x, dy, relu_y, dz, part, g, (int)Cout, (int)K, with_db, PHs, PWss, Ls, (int)tpi)
            switch (sel) {
                case 0: TF_WS_LAUNCH(false, false, false); break;
                case 1: TF_WS_LAUNCH(false, false, true); break;
                case 2: TF_WS_LAUNCH(false, true, false); break;
                case 3: TF_WS_LAUNCH(false, true, true); break;
                case 4: TF_WS_LAUNCH(true, false, false); break;
                case 5: TF_WS_LAUNCH(true, false, true); break;
                case 6: TF_WS_LAUNCH(true, true, false); break;
                default: TF_WS_LAUNCH(true, true, true); break;
            }
#undef TF_WS_LAUNCH
            st = tfh::check_launch("conv_bwd_weight_stream_kernel");
            if (st != TF_OK) return st;
            conv_partial_sum_kernel<kPsEl><<<(unsigned)((plane + kPsEl - 1) / kPsEl), 256, 0, ctx->stream>>>(
                part, (int)blocks, plane, (int)K, (int)KD, dw, db);
            return tfh::check_launch("conv_partial_sum_kernel");
        }
    }
    const int MT = Cout <= 32 ? 32 : 64;
    int Kc, PH, PWs, L, slices;
    bool aligned;
    const size_t lds = implicit_dw_lds_bytes(g, MT, (int)K, Kc, PH, PWs, L, slices, aligned);
    if (lds == 0)
        return tfh::set_error(TF_ERR_UNSUPPORTED, "tf_conv2d_bwd_weight: dy tile, tap tables and input patch exceed the "
                                                  "160 KB of LDS (use tf_im2col + tf_gemm_ex)");
    const int64_t P = g.outH * g.outW;
    const int np = MT == 64 ? ig_pixels<64>() : ig_pixels<32>();
    const int tpi = (int)((P + np - 1) / np);
    const int64_t blocks = N * tpi;
    TF_REQUIRE(blocks < (1LL << 31), "tf_conv2d_bwd_weight: too many blocks");
    // 16-byte staging loads: bit 0 input rows, bit 1 dy rows; bit 2: the
    // direct-load layout (both, regions in whole KB), when it fits.
    int vec = (aligned && W % 4 == 0 && aligned16(x) ? 1 : 0) | (P % 4 == 0 && aligned16(dy) ? 2 : 0);
    size_t lds_launch = lds;
    if ((vec & 3) == 3) {
        const int64_t tiles = (MT / 32) * (Kc / 32);
        const int64_t direct = ((MT * (int64_t)(np + 4) + 255) / 256 * 256 + (C * (int64_t)PH * PWs + 255) / 256 * 256 +
                                np + Kc + (slices > 1 ? tiles * slices * 16 * 64 : 0)) * 4;
        if (direct <= 160 * 1024) {
            vec |= 4;
            lds_launch = (size_t)direct;
        }
    }
    st = tfh::ensure_workspace(ctx, (size_t)blocks * Cout * KD * sizeof(float));
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
        conv_bwd_weight_implicit_kernel<32><<<grid, kIgThreads, lds_launch, ctx->stream>>>(
            x, dy, part, g, (int)Cout, (int)K, Kc, PH, PWs, L, tpi, slices, vec, with_db, relu_y, dz);
    else
        conv_bwd_weight_implicit_kernel<64><<<grid, kIgThreads, lds_launch, ctx->stream>>>(
            x, dy, part, g, (int)Cout, (int)K, Kc, PH, PWs, L, tpi, slices, vec, with_db, relu_y, dz);
    st = tfh::check_launch("conv_bwd_weight_implicit_kernel");
    if (st != TF_OK) return st;
    conv_partial_sum_kernel<kPsEl><<<(unsigned)((plane + kPsEl - 1) / kPsEl), 256, 0, ctx->stream>>>(
        part, (int)blocks, plane, (int)K, (int)KD, dw, db);
    return tfh::check_launch("conv_partial_sum_kernel");
}

tf_status conv_bwd_data_impl(tf_ctx* ctx, const float* dy, const float* w, float* dx, int64_t N, int64_t C,
                             int64_t H, int64_t W, int64_t Cout, int64_t kH, int64_t kW, int64_t sh, int64_t sw,
                             int64_t ph, int64_t pw, int64_t dh, int64_t dw_) {
    TF_CTX_CHECK(ctx);
    ConvGeom g;
    tf_status st = make_geom(g, N, C, H, W, kH, kW, sh, sw, ph, pw, dh, dw_);
    if (st != TF_OK) return st;
    TF_REQUIRE(Cout > 0 && C > 0, "tf_conv2d_bwd_data: empty channel count");
    if (N == 0) return TF_OK;
    TF_REQUIRE(dy && w && dx, "tf_conv2d_bwd_data: null pointer");
    TF_REQUIRE(Cout * kH * kW < (1 << 20) && N * C * H * W < (1LL << 31) && N * Cout * g.outH * g.outW < (1LL << 31) &&
                   C * kH * kW < (1 << 20) && sh * sw <= 4096 && kH <= 4096 && kW <= 4096,
               "tf_conv2d_bwd_data: extent beyond this kernel's 32-bit indexing");
    static const bool lds_ok = [] {
        const int all = 160 * 1024;
        return hipFuncSetAttribute(reinterpret_cast<const void*>(conv_bwd_data_implicit_kernel<32>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, all) == hipSuccess &&
               hipFuncSetAttribute(reinterpret_cast<const void*>(conv_bwd_data_implicit_kernel<64>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, all) == hipSuccess &&
               hipFuncSetAttribute(reinterpret_cast<const void*>(conv_bwd_data_lds_kernel<5, 32>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, all) == hipSuccess &&
               hipFuncSetAttribute(reinterpret_cast<const void*>(conv_bwd_data_lds_kernel<9, 64>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, all) == hipSuccess;
    }();
    if (!lds_ok) {
        (void)hipGetLastError();
        return tfh::set_error(TF_ERR_HIP, "tf_conv2d_bwd_data: hipFuncSetAttribute (dynamic LDS) failed");
    }
    // Strided layers with few output pixels and enough (image, channel group)
    // blocks to fill the GPU: dcol per image in LDS, then col2im from LDS;
    // two blocks per CU (small channel groups) when that layout fits.
    if (sh > 1 || sw > 1) {
        int CG, RT, tab_off;
        // Column-per-lane col2im: the most column and row taps of an input
        // pixel.
        int most = 0, most_r = 0;
        for (int j0 = 0; j0 < sw; ++j0) most = std::max(most, phase_taps(j0, (int)pw, (int)kW, (int)sw, (int)dw_).n);
        for (int i0 = 0; i0 < sh; ++i0) most_r = std::max(most_r, phase_taps(i0, (int)ph, (int)kH, (int)sh, (int)dh).n);
        const auto taps_for = [&](int nt) { return W > nt ? 0 : most <= 2 && most_r <= 2 ? 2 : most <= 4 ? 4 : 0; };
        bool two = true;
        size_t lds_b = dx_lds_bytes(g, 5, 32, 80 * 1024, CG, RT, tab_off);
        if (lds_b == 0 || N * ((C + CG - 1) / CG) < 256) {
            two = false;
            lds_b = dx_lds_bytes(g, 9, 64, 160 * 1024, CG, RT, tab_off);
        }
        const int64_t nblk = lds_b ? N * ((C + CG - 1) / CG) : 0;
        if (nblk >= 128 && nblk < (1LL << 31)) {
            const int64_t P = g.outH * g.outW;
            // Direct loads: bit 0 dy rows, bit 1 filter rows.
            const int vec = (P % 4 == 0 && aligned16(dy) ? 1 : 0) |
                            ((C * kH * kW) % 4 == 0 && (CG * kH * kW) % 4 == 0 && aligned16(w) ? 2 : 0);
            const int taps = taps_for(kIgThreads);
            if (two)
                conv_bwd_data_lds_kernel<5, 32><<<(unsigned)nblk, kIgThreads, lds_b, ctx->stream>>>(
                    dy, w, dx, g, (int)Cout, CG, RT, tab_off, vec, taps);
            else
                conv_bwd_data_lds_kernel<9, 64><<<(unsigned)nblk, kIgThreads, lds_b, ctx->stream>>>(
                    dy, w, dx, g, (int)Cout, CG, RT, tab_off, vec, taps);
            return tfh::check_launch("conv_bwd_data_lds_kernel");
        }
    }
    const int MT = C <= 32 ? 32 : 64;
    int PH, PWs, L, tpp;
    bool aligned;
    const size_t lds = implicit_dx_lds_bytes(g, MT, (int)Cout, PH, PWs, L, tpp, aligned);
    if (lds == 0)
        return tfh::set_error(TF_ERR_UNSUPPORTED, "tf_conv2d_bwd_data: filter columns and dy patch exceed the 160 KB "
                                                  "of LDS (use tf_gemm_ex + tf_col2im)");
    const int64_t blocks = (N * tpp + 7) / 8 * 8 * sh * sw;  // see the kernel's block order
    TF_REQUIRE(blocks < (1LL << 31), "tf_conv2d_bwd_data: too many blocks");
    // 16-byte loads of dy rows.
    const int vec = aligned && g.outW % 4 == 0 && aligned16(dy) ? 1 : 0;
    const dim3 grid((unsigned)blocks, (unsigned)((C + MT - 1) / MT));
    if (MT == 32)
        conv_bwd_data_implicit_kernel<32><<<grid, kIgThreads, lds, ctx->stream>>>(dy, w, dx, g, (int)Cout, PH, PWs, L, tpp,
                                                                                 vec);
    else
        conv_bwd_data_implicit_kernel<64><<<grid, kIgThreads, lds, ctx->stream>>>(dy, w, dx, g, (int)Cout, PH, PWs, L, tpp,
                                                                                 vec);
    return tfh::check_launch("conv_bwd_data_implicit_kernel");
}

}  // namespace

extern "C" {

tf_status tf_conv2d_bwd_weight(tf_ctx* ctx, const float* x, const float* dy, float* dw, float* db, int64_t N,
                               int64_t C, int64_t H, int64_t W, int64_t Cout, int64_t kH, int64_t kW, int64_t sh,
                               int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw_) {
    return conv_bwd_weight_impl(ctx, x, dy, nullptr, nullptr, dw, db, N, C, H, W, Cout, kH, kW, sh, sw, ph, pw, dh,
                                dw_);
}

tf_status tf_conv2d_bwd_weight_relu(tf_ctx* ctx, const float* x, const float* dy, const float* y, float* dz, float* dw,
                                    float* db, int64_t N, int64_t C, int64_t H, int64_t W, int64_t Cout, int64_t kH,
                                    int64_t kW, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh,
                                    int64_t dw_) {
    TF_REQUIRE(y, "tf_conv2d_bwd_weight_relu: null ReLU output");
    return conv_bwd_weight_impl(ctx, x, dy, y, dz, dw, db, N, C, H, W, Cout, kH, kW, sh, sw, ph, pw, dh, dw_);
}

tf_status tf_conv2d_bwd_data(tf_ctx* ctx, const float* dy, const float* w, float* dx, int64_t N, int64_t C, int64_t H,
                             int64_t W, int64_t Cout, int64_t kH, int64_t kW, int64_t sh, int64_t sw, int64_t ph,
                             int64_t pw, int64_t dh, int64_t dw_) {
    return conv_bwd_data_impl(ctx, dy, w, dx, N, C, H, W, Cout, kH, kW, sh, sw, ph, pw, dh, dw_);
}

}  // extern "C"
