// Elementwise bandwidth kernels: forward activations, their backward
// (ReLU / Sigmoid / Tanh), gradient accumulation (add), mul, scalar scale,
// the fused SGD-momentum update and f32<->bf16 casts.
//
// Every kernel is a grid-stride loop over 16-byte vectors (4 x f32, or
// 8 x bf16 / f16) with a scalar tail, 256 threads per block; 16-bit types are
// widened to f32 for the arithmetic and rounded once on the way out.  They are HBM-bound:
// the algorithmic traffic per element is listed beside each one.  The
// streaming kernels (activations, their backward, SGD) read and write their
// vectors with non-temporal accesses (tfd::ld_nt / st_nt).
#include "common.hpp"

namespace {

using tfd::bf16_to_f32;
using tfd::f32_to_bf16;
using tfd::ld_nt;
using tfd::st_nt;

// ----- element access for f32 / bf16 storage with f32 math ----------------
template <typename T> struct Elem;
template <> struct Elem<float> {
    static __device__ __forceinline__ float ld(const float* p, int64_t i) { return p[i]; }
    static __device__ __forceinline__ void st(float* p, int64_t i, float v) { p[i] = v; }
};
template <> struct Elem<uint16_t> {
    static __device__ __forceinline__ float ld(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
    static __device__ __forceinline__ void st(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
};
// IEEE half: widened exactly (v_cvt_f32_f16), rounded to nearest even on
// the way back (v_cvt_f16_f32 in the default round mode), as the
// reference's __half2float / __float2half (cuda/kernels/elementwise.cu:42-64).
template <> struct Elem<_Float16> {
    static __device__ __forceinline__ float ld(const _Float16* p, int64_t i) { return (float)p[i]; }
    static __device__ __forceinline__ void st(_Float16* p, int64_t i, float v) { p[i] = tfd::f32_to_f16(v); }
};

// Number of scalars in a 16-byte vector.
template <typename T> constexpr int kVec = 16 / sizeof(T);

// Streaming loops: a block works on chunks of kUnroll x 256 consecutive
// 16-byte vectors (grid-stride over chunks); each thread loads its kUnroll
// vectors of the chunk (256 vectors apart, so each load instruction is one
// contiguous 4 KB piece per block) before any arithmetic or store.
constexpr int kUnroll = 4;
constexpr int kChunk = kUnroll * 256;  // vectors per block chunk

template <typename T, typename Op>
__device__ __forceinline__ uint4 apply2(const uint4& va, const uint4& vb, Op op) {
    constexpr int V = kVec<T>;
    uint4 vo;
    const T* ea = reinterpret_cast<const T*>(&va);
    const T* eb = reinterpret_cast<const T*>(&vb);
    T* eo = reinterpret_cast<T*>(&vo);
#pragma unroll
    for (int j = 0; j < V; ++j) Elem<T>::st(eo, j, op(Elem<T>::ld(ea, j), Elem<T>::ld(eb, j)));
    return vo;
}

template <typename T, typename Op>
__device__ __forceinline__ uint4 apply1(const uint4& vx, Op op) {
    constexpr int V = kVec<T>;
    uint4 vo;
    const T* ex = reinterpret_cast<const T*>(&vx);
    T* eo = reinterpret_cast<T*>(&vo);
#pragma unroll
    for (int j = 0; j < V; ++j) Elem<T>::st(eo, j, op(Elem<T>::ld(ex, j)));
    return vo;
}

// Binary elementwise: out = op(a, b).  Vector body when all three pointers
// are 16-byte aligned, scalar loop otherwise / for the tail.
template <typename T, typename Op>
__global__ __launch_bounds__(256) void binary_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                     T* __restrict__ out, int64_t n, Op op, int vec_ok) {
    constexpr int V = kVec<T>;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t nv = vec_ok ? n / V : 0;
    const uint4* A = reinterpret_cast<const uint4*>(a);
    const uint4* B = reinterpret_cast<const uint4*>(b);
    uint4* O = reinterpret_cast<uint4*>(out);
    const int64_t full = nv / kChunk;
    for (int64_t c = blockIdx.x; c < full; c += gridDim.x) {
        const int64_t i = c * kChunk + threadIdx.x;
        uint4 va[kUnroll], vb[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            va[u] = ld_nt(A + i + u * 256);
            vb[u] = ld_nt(B + i + u * 256);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) st_nt(O + i + u * 256, apply2<T>(va[u], vb[u], op));
    }
    for (int64_t i = full * kChunk + tid; i < nv; i += stride) st_nt(O + i, apply2<T>(ld_nt(A + i), ld_nt(B + i), op));
    for (int64_t j = nv * V + tid; j < n; j += stride)
        Elem<T>::st(out, j, op(Elem<T>::ld(a, j), Elem<T>::ld(b, j)));
}

template <typename T, typename Op>
__global__ __launch_bounds__(256) void unary_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t n, Op op,
                                                    int vec_ok) {
    constexpr int V = kVec<T>;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t nv = vec_ok ? n / V : 0;
    const uint4* X = reinterpret_cast<const uint4*>(x);
    uint4* Y = reinterpret_cast<uint4*>(y);
    const int64_t full = nv / kChunk;
    for (int64_t c = blockIdx.x; c < full; c += gridDim.x) {
        const int64_t i = c * kChunk + threadIdx.x;
        uint4 vx[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) vx[u] = ld_nt(X + i + u * 256);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) st_nt(Y + i + u * 256, apply1<T>(vx[u], op));
    }
    for (int64_t i = full * kChunk + tid; i < nv; i += stride) st_nt(Y + i, apply1<T>(ld_nt(X + i), op));
    for (int64_t j = nv * V + tid; j < n; j += stride) Elem<T>::st(y, j, op(Elem<T>::ld(x, j)));
}

// Operators.  The backward ones reproduce the reference's arithmetic order:
// ReluBackward builds mask = (x > 0 ? 1 : 0) and multiplies dy * mask
// (autograd/ops/ReluBackward.hpp:25-31), so negative dy over a masked
// element yields -0.0 exactly as on the CPU.
struct AddOp { __device__ float operator()(float a, float b) const { return a + b; } };
struct SubOp { __device__ float operator()(float a, float b) const { return a - b; } };
struct MulOp { __device__ float operator()(float a, float b) const { return a * b; } };
struct ReluBwdOp {
    __device__ float operator()(float dy, float x) const { return dy * (x > 0.0f ? 1.0f : 0.0f); }
};
struct SigmoidBwdOp {
    __device__ float operator()(float dy, float y) const { return dy * (y * (1.0f - y)); }
};
struct TanhBwdOp {
    __device__ float operator()(float dy, float y) const { return dy * (1.0f - y * y); }
};
struct ReluOp { __device__ float operator()(float x) const { return x > 0.0f ? x : 0.0f; } };
// x > 0 ? x : alpha * x, one rounding (the reference's LeakyReluOp,
// cuda/kernels/elementwise.cu:116-121, and its CPU loop).
struct LeakyReluOp {
    float alpha;
    __device__ float operator()(float x) const { return x > 0.0f ? x : alpha * x; }
};
struct SigmoidOp { __device__ float operator()(float x) const { return 1.0f / (1.0f + expf(-x)); } };
struct TanhOp { __device__ float operator()(float x) const { return tanhf(x); } };

template <typename T>
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <typename Op>
tf_status launch_binary(tf_ctx* ctx, const void* a, const void* b, void* out, int64_t n, int dtype,
                        Op op, const char* name) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(n >= 0, "negative element count");
    if (n == 0) return TF_OK;
    TF_REQUIRE(a && b && out, "null pointer");
    int vec_ok = aligned16<char>(a) && aligned16<char>(b) && aligned16<char>(out);
    if (dtype == TF_F32) {
        binary_kernel<float, Op><<<tfd::grid_for(n, 4 * kUnroll), 256, 0, ctx->stream>>>(
            (const float*)a, (const float*)b, (float*)out, n, op, vec_ok);
    } else if (dtype == TF_BF16) {
        binary_kernel<uint16_t, Op><<<tfd::grid_for(n, 8 * kUnroll), 256, 0, ctx->stream>>>(
            (const uint16_t*)a, (const uint16_t*)b, (uint16_t*)out, n, op, vec_ok);
    } else if (dtype == TF_F16) {
        binary_kernel<_Float16, Op><<<tfd::grid_for(n, 8 * kUnroll), 256, 0, ctx->stream>>>(
            (const _Float16*)a, (const _Float16*)b, (_Float16*)out, n, op, vec_ok);
    } else {
        return tfh::set_error(TF_ERR_UNSUPPORTED, std::string(name) + ": dtype must be Float32, Float16 or BFloat16");
    }
    return tfh::check_launch(name);
}

template <typename Op>
tf_status launch_unary(tf_ctx* ctx, const void* x, void* y, int64_t n, int dtype, Op op, const char* name) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(n >= 0, "negative element count");
    if (n == 0) return TF_OK;
    TF_REQUIRE(x && y, "null pointer");
    int vec_ok = aligned16<char>(x) && aligned16<char>(y);
    if (dtype == TF_F32) {
        unary_kernel<float, Op><<<tfd::grid_for(n, 4 * kUnroll), 256, 0, ctx->stream>>>(
            (const float*)x, (float*)y, n, op, vec_ok);
    } else if (dtype == TF_BF16) {
        unary_kernel<uint16_t, Op><<<tfd::grid_for(n, 8 * kUnroll), 256, 0, ctx->stream>>>(
            (const uint16_t*)x, (uint16_t*)y, n, op, vec_ok);
    } else if (dtype == TF_F16) {
        unary_kernel<_Float16, Op><<<tfd::grid_for(n, 8 * kUnroll), 256, 0, ctx->stream>>>(
            (const _Float16*)x, (_Float16*)y, n, op, vec_ok);
    } else {
        return tfh::set_error(TF_ERR_UNSUPPORTED, std::string(name) + ": dtype must be Float32, Float16 or BFloat16");
    }
    return tfh::check_launch(name);
}

// out[i] = a[i] * s[0] (device scalar; used for upstream-gradient scaling).
__global__ void scale_by_kernel(const float* __restrict__ a, const float* __restrict__ s,
                                float* __restrict__ out, int64_t n) {
    float k = s[0];
    int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = tid; i < n; i += stride) out[i] = a[i] * k;
}

// Fused SGD with momentum, one pass: reads p, g, v; writes p, v
// (20 B/param; +2 B with the bf16 shadow).  Contraction is disabled so the
// update rounds exactly like the host loop v*mu + g, p - v*lr (two roundings
// each), the order of nn/optim/SGD.cpp:50-54.
// Four bf16 (round to nearest even) packed as they lie in memory.
__device__ __forceinline__ uint2 bf16x4(const float4& v) {
    return make_uint2(tfd::bf16x2_rne(v.x, v.y), tfd::bf16x2_rne(v.z, v.w));
}

__device__ __forceinline__ void sgd4(float4& pp, const float4& gg, float4& vv, bool use_v, float lr, float mu) {
#pragma clang fp contract(off)
    float* pe = reinterpret_cast<float*>(&pp);
    const float* ge = reinterpret_cast<const float*>(&gg);
    float* ve = reinterpret_cast<float*>(&vv);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (use_v) {
            const float vm = ve[j] * mu;
            ve[j] = vm + ge[j];
            const float step = ve[j] * lr;
            pe[j] = pe[j] - step;
        } else {
            const float step = lr * ge[j];
            pe[j] = pe[j] - step;
        }
    }
}

// NT: non-temporal accesses, for parameter sets too large to stay in the
// last-level cache between steps (tfd::kStreamMinBytes).
template <bool NT>
__global__ __launch_bounds__(256) void sgd_momentum_kernel(float* __restrict__ p, const float* __restrict__ g,
                                                           float* __restrict__ v, uint16_t* __restrict__ p_bf16,
                                                           int64_t n, float lr, float mu, int vec_ok) {
#pragma clang fp contract(off)
    constexpr int U = 2;  // iterations in flight (3 input streams)
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t nv = vec_ok ? n / 4 : 0;
    const bool use_v = mu != 0.0f;
    float4* P = reinterpret_cast<float4*>(p);
    const float4* G = reinterpret_cast<const float4*>(g);
    float4* Vv = reinterpret_cast<float4*>(v);
    auto finish = [&](int64_t i, float4& pp, float4& vv) {
        tfd::st_v<NT>(P + i, pp);
        if (use_v) tfd::st_v<NT>(Vv + i, vv);
        if (p_bf16) tfd::st_v<NT>(reinterpret_cast<uint2*>(p_bf16) + i, bf16x4(pp));
    };
    const int64_t full = nv / (U * 256);
    for (int64_t c = blockIdx.x; c < full; c += gridDim.x) {
        const int64_t i = c * (U * 256) + threadIdx.x;
        float4 pp[U], gg[U], vv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            pp[u] = tfd::ld_v<NT>(P + i + u * 256);
            gg[u] = tfd::ld_v<NT>(G + i + u * 256);
            vv[u] = use_v ? tfd::ld_v<NT>(Vv + i + u * 256) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            sgd4(pp[u], gg[u], vv[u], use_v, lr, mu);
            finish(i + u * 256, pp[u], vv[u]);
        }
    }
    for (int64_t i = full * (U * 256) + tid; i < nv; i += stride) {
        float4 pp = P[i], gg = G[i], vv = use_v ? Vv[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        sgd4(pp, gg, vv, use_v, lr, mu);
        finish(i, pp, vv);
    }
    for (int64_t j = nv * 4 + tid; j < n; j += stride) {
        float pv = p[j];
        if (use_v) {
            float vm = v[j] * mu;
            float vn = vm + g[j];
            v[j] = vn;
            float step = vn * lr;
            pv = pv - step;
        } else {
            float step = lr * g[j];
            pv = pv - step;
        }
        p[j] = pv;
        if (p_bf16) p_bf16[j] = f32_to_bf16(pv);
    }
}

// Scalar SGD step of one element (the tail of the vector kernels).
__device__ __forceinline__ float sgd1(float pv, float gv, float* vp, bool use_v, float lr, float mu) {
#pragma clang fp contract(off)
    if (use_v) {
        const float vm = *vp * mu;
        const float vn = vm + gv;
        *vp = vn;
        const float step = vn * lr;
        return pv - step;
    }
    const float step = lr * gv;
    return pv - step;
}

// Several parameters in one launch (an optimiser's whole step).  Work units
// of sgd_unit<NT>() consecutive elements of one tensor; unit u belongs to tensor t
// with unit_start[t] <= u < unit_start[t + 1].  The element update is the
// one of sgd_momentum_kernel (sgd4 / sgd1), so each tensor ends up exactly
// as tf_sgd_momentum would leave it.
// float4 per thread and stream, loaded together: 4 for updates that stream
// past the last-level cache (C5's 138 M parameters: 551 -> 538 us), 2 for
// small warm ones (C2: 16.1 us, against 16.9 with 4).  A work unit is 256
// threads' worth.
template <bool NT> constexpr int sgd_u() { return NT ? 4 : 2; }
template <bool NT> constexpr int sgd_unit() { return 256 * 4 * sgd_u<NT>(); }
struct SgdMultiArgs {
    float* p[TF_SGD_MULTI_MAX];
    const float* g[TF_SGD_MULTI_MAX];
    float* v[TF_SGD_MULTI_MAX];
    uint16_t* s[TF_SGD_MULTI_MAX];
    int64_t n[TF_SGD_MULTI_MAX];
    int64_t unit_start[TF_SGD_MULTI_MAX + 1];
    int vec_ok[TF_SGD_MULTI_MAX];
    int count;
};

template <bool NT>
__global__ __launch_bounds__(256) void sgd_multi_kernel(const SgdMultiArgs a, float lr, float mu) {
#pragma clang fp contract(off)
    const bool use_v = mu != 0.0f;
    const int64_t units = a.unit_start[a.count];
    for (int64_t u = blockIdx.x; u < units; u += gridDim.x) {
        int t = 0;
        while (u >= a.unit_start[t + 1]) ++t;
        constexpr int kU = sgd_u<NT>(), kUnit = sgd_unit<NT>();
        const int64_t e0 = (u - a.unit_start[t]) * kUnit;
        const int64_t e1 = min(a.n[t], e0 + kUnit);
        float* p = a.p[t];
        const float* g = a.g[t];
        float* v = a.v[t];
        uint16_t* s = a.s[t];
        int64_t js = e0;  // first element of the scalar part
        if (a.vec_ok[t]) {
            float4* P = reinterpret_cast<float4*>(p);
            const float4* G = reinterpret_cast<const float4*>(g);
            float4* V = reinterpret_cast<float4*>(v);
            const int64_t vend = e1 / 4;  // e0 is a multiple of 4
            const int64_t i0 = e0 / 4 + threadIdx.x;
            float4 pp[kU], gg[kU], vv[kU];
#pragma unroll
            for (int k = 0; k < kU; ++k) {
                vv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (i0 + 256 * k < vend) {
                    pp[k] = tfd::ld_v<NT>(P + i0 + 256 * k);
                    gg[k] = tfd::ld_v<NT>(G + i0 + 256 * k);
                    if (use_v) vv[k] = tfd::ld_v<NT>(V + i0 + 256 * k);
                }
            }
#pragma unroll
            for (int k = 0; k < kU; ++k) {
                const int64_t i = i0 + 256 * k;
                if (i >= vend) continue;
                sgd4(pp[k], gg[k], vv[k], use_v, lr, mu);
                tfd::st_v<NT>(P + i, pp[k]);
                if (use_v) tfd::st_v<NT>(V + i, vv[k]);
                if (s) tfd::st_v<NT>(reinterpret_cast<uint2*>(s) + i, bf16x4(pp[k]));
            }
            js = vend * 4;
        }
        for (int64_t j = js + threadIdx.x; j < e1; j += 256) {
            const float pv = sgd1(p[j], g[j], use_v ? v + j : nullptr, use_v, lr, mu);
            p[j] = pv;
            if (s) s[j] = f32_to_bf16(pv);
        }
    }
}

// Casts: 8 elements per iteration (two float4 <-> one 16-byte bf16 vector)
// when both pointers are 16-byte aligned; scalar for the rest.
__global__ __launch_bounds__(256) void cast_f32_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y,
                                                            int64_t n, int vec_ok) {
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t nv = vec_ok ? n / 8 : 0;
    for (int64_t i = tid; i < nv; i += stride) {
        const float4 a = reinterpret_cast<const float4*>(x)[2 * i];
        const float4 b = reinterpret_cast<const float4*>(x)[2 * i + 1];
        uint4 o;
        o.x = tfd::bf16x2_rne(a.x, a.y);
        o.y = tfd::bf16x2_rne(a.z, a.w);
        o.z = tfd::bf16x2_rne(b.x, b.y);
        o.w = tfd::bf16x2_rne(b.z, b.w);
        reinterpret_cast<uint4*>(y)[i] = o;
    }
    for (int64_t j = nv * 8 + tid; j < n; j += stride) y[j] = f32_to_bf16(x[j]);
}

__global__ __launch_bounds__(256) void cast_bf16_f32_kernel(const uint16_t* __restrict__ x, float* __restrict__ y,
                                                            int64_t n, int vec_ok) {
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t nv = vec_ok ? n / 8 : 0;
    for (int64_t i = tid; i < nv; i += stride) {
        const uint4 h = reinterpret_cast<const uint4*>(x)[i];
        reinterpret_cast<float4*>(y)[2 * i] = make_float4(bf16_to_f32((uint16_t)h.x), bf16_to_f32((uint16_t)(h.x >> 16)),
                                                          bf16_to_f32((uint16_t)h.y), bf16_to_f32((uint16_t)(h.y >> 16)));
        reinterpret_cast<float4*>(y)[2 * i + 1] =
            make_float4(bf16_to_f32((uint16_t)h.z), bf16_to_f32((uint16_t)(h.z >> 16)), bf16_to_f32((uint16_t)h.w),
                        bf16_to_f32((uint16_t)(h.w >> 16)));
    }
    for (int64_t j = nv * 8 + tid; j < n; j += stride) y[j] = bf16_to_f32(x[j]);
}

}  // namespace

extern "C" {

tf_status tf_add(tf_ctx* ctx, const void* a, const void* b, void* out, int64_t n, int dtype) {
    return launch_binary(ctx, a, b, out, n, dtype, AddOp{}, "tf_add");
}
tf_status tf_sub(tf_ctx* ctx, const void* a, const void* b, void* out, int64_t n, int dtype) {
    return launch_binary(ctx, a, b, out, n, dtype, SubOp{}, "tf_sub");
}
tf_status tf_mul(tf_ctx* ctx, const void* a, const void* b, void* out, int64_t n, int dtype) {
    return launch_binary(ctx, a, b, out, n, dtype, MulOp{}, "tf_mul");
}
tf_status tf_relu_bwd(tf_ctx* ctx, const void* dy, const void* x, void* dx, int64_t n, int dtype) {
    return launch_binary(ctx, dy, x, dx, n, dtype, ReluBwdOp{}, "tf_relu_bwd");
}
tf_status tf_sigmoid_bwd(tf_ctx* ctx, const void* dy, const void* y, void* dx, int64_t n, int dtype) {
    return launch_binary(ctx, dy, y, dx, n, dtype, SigmoidBwdOp{}, "tf_sigmoid_bwd");
}
tf_status tf_tanh_bwd(tf_ctx* ctx, const void* dy, const void* y, void* dx, int64_t n, int dtype) {
    return launch_binary(ctx, dy, y, dx, n, dtype, TanhBwdOp{}, "tf_tanh_bwd");
}
tf_status tf_relu_fwd(tf_ctx* ctx, const void* x, void* y, int64_t n, int dtype) {
    return launch_unary(ctx, x, y, n, dtype, ReluOp{}, "tf_relu_fwd");
}
tf_status tf_leaky_relu_fwd(tf_ctx* ctx, const void* x, void* y, int64_t n, float alpha, int dtype) {
    return launch_unary(ctx, x, y, n, dtype, LeakyReluOp{alpha}, "tf_leaky_relu_fwd");
}
tf_status tf_sigmoid_fwd(tf_ctx* ctx, const void* x, void* y, int64_t n, int dtype) {
    return launch_unary(ctx, x, y, n, dtype, SigmoidOp{}, "tf_sigmoid_fwd");
}
tf_status tf_tanh_fwd(tf_ctx* ctx, const void* x, void* y, int64_t n, int dtype) {
    return launch_unary(ctx, x, y, n, dtype, TanhOp{}, "tf_tanh_fwd");
}

tf_status tf_scale_by(tf_ctx* ctx, const void* a, const float* s, void* out, int64_t n, int dtype) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(dtype == TF_F32, "tf_scale_by: Float32 only");
    TF_REQUIRE(n >= 0, "tf_scale_by: negative n");
    if (n == 0) return TF_OK;
    TF_REQUIRE(a && s && out, "tf_scale_by: null pointer");
    scale_by_kernel<<<tfd::grid_for(n, 4), 256, 0, ctx->stream>>>((const float*)a, s, (float*)out, n);
    return tfh::check_launch("scale_by_kernel");
}

tf_status tf_sgd_momentum(tf_ctx* ctx, float* p, const float* g, float* v, void* p_bf16,
                          int64_t n, float lr, float mu) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(n >= 0, "tf_sgd_momentum: negative n");
    if (n == 0) return TF_OK;
    TF_REQUIRE(p && g, "tf_sgd_momentum: null p or g");
    TF_REQUIRE(mu == 0.0f || v != nullptr, "tf_sgd_momentum: momentum needs a velocity buffer");
    TF_REQUIRE(mu >= 0.0f && mu < 1.0f, "tf_sgd_momentum: momentum must lie in [0, 1)");
    int vec_ok = aligned16<char>(p) && aligned16<char>(g) && (v == nullptr || aligned16<char>(v)) &&
                 (p_bf16 == nullptr || (reinterpret_cast<uintptr_t>(p_bf16) & 7) == 0);
    const int64_t bytes = n * (12 + (mu != 0.0f ? 8 : 0) + (p_bf16 ? 2 : 0));
    auto kernel = bytes > tfd::kStreamMinBytes ? sgd_momentum_kernel<true> : sgd_momentum_kernel<false>;
    kernel<<<tfd::grid_for(n, 4 * 2), 256, 0, ctx->stream>>>(p, g, v, (uint16_t*)p_bf16, n, lr, mu, vec_ok);
    return tfh::check_launch("sgd_momentum_kernel");
}

tf_status tf_sgd_momentum_multi(tf_ctx* ctx, int count, float* const* p, const float* const* g, float* const* v,
                                void* const* p_bf16, const int64_t* n, float lr, float mu) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(count >= 0 && count <= TF_SGD_MULTI_MAX, "tf_sgd_momentum_multi: count must lie in [0, 32]");
    if (count == 0) return TF_OK;
    TF_REQUIRE(p && g && n, "tf_sgd_momentum_multi: null p, g or n array");
    TF_REQUIRE(mu >= 0.0f && mu < 1.0f, "tf_sgd_momentum_multi: momentum must lie in [0, 1)");
    SgdMultiArgs a{};
    int64_t units = 0, bytes = 0;
    int m = 0;
    for (int i = 0; i < count; ++i) {
        TF_REQUIRE(n[i] >= 0, "tf_sgd_momentum_multi: negative n");
        if (n[i] == 0) continue;
        TF_REQUIRE(p[i] && g[i], "tf_sgd_momentum_multi: null p or g");
        float* vi = v ? v[i] : nullptr;
        TF_REQUIRE(mu == 0.0f || vi != nullptr, "tf_sgd_momentum_multi: momentum needs a velocity buffer");
        void* si = p_bf16 ? p_bf16[i] : nullptr;
        a.p[m] = p[i];
        a.g[m] = g[i];
        a.v[m] = vi;
        a.s[m] = static_cast<uint16_t*>(si);
        a.n[m] = n[i];
        a.vec_ok[m] = aligned16<char>(p[i]) && aligned16<char>(g[i]) && (vi == nullptr || aligned16<char>(vi)) &&
                      (si == nullptr || (reinterpret_cast<uintptr_t>(si) & 7) == 0);
        bytes += n[i] * (12 + (mu != 0.0f ? 8 : 0) + (si ? 2 : 0));
        ++m;
    }
    a.count = m;
    const bool nt = bytes > tfd::kStreamMinBytes;
    const int64_t unit = nt ? sgd_unit<true>() : sgd_unit<false>();
    for (int i = 0; i < m; ++i) {
        a.unit_start[i] = units;
        units += (a.n[i] + unit - 1) / unit;
    }
    a.unit_start[m] = units;
    if (units == 0) return TF_OK;
    auto kernel = nt ? sgd_multi_kernel<true> : sgd_multi_kernel<false>;
    kernel<<<(unsigned)std::min<int64_t>(units, 16384), 256, 0, ctx->stream>>>(a, lr, mu);
    return tfh::check_launch("sgd_multi_kernel");
}

tf_status tf_cast_f32_bf16(tf_ctx* ctx, const float* x, void* y, int64_t n) {
    TF_CTX_CHECK(ctx);
    if (n == 0) return TF_OK;
    TF_REQUIRE(x && y && n > 0, "tf_cast_f32_bf16: bad argument");
    cast_f32_bf16_kernel<<<tfd::grid_for(n, 8), 256, 0, ctx->stream>>>(x, (uint16_t*)y, n,
                                                                       aligned16<char>(x) && aligned16<char>(y));
    return tfh::check_launch("cast_f32_bf16_kernel");
}

tf_status tf_cast_bf16_f32(tf_ctx* ctx, const void* x, float* y, int64_t n) {
    TF_CTX_CHECK(ctx);
    if (n == 0) return TF_OK;
    TF_REQUIRE(x && y && n > 0, "tf_cast_bf16_f32: bad argument");
    cast_bf16_f32_kernel<<<tfd::grid_for(n, 8), 256, 0, ctx->stream>>>((const uint16_t*)x, y, n,
                                                                       aligned16<char>(x) && aligned16<char>(y));
    return tfh::check_launch("cast_bf16_f32_kernel");
}

}  // extern "C"

namespace {

// dst[i] = table[(i / plane) % channels][src[i]]: the file loaders' byte ->
// float decode (data/Decode.cpp) through a per-channel table of 256 values
// held in LDS; four bytes per thread per step when plane % 4 == 0 (a quad
// then stays in one channel).
__global__ __launch_bounds__(256) void decode_u8_kernel(const uint8_t* __restrict__ src, float* __restrict__ dst,
                                                        int64_t n, int64_t plane, int channels,
                                                        const float* __restrict__ table, int quads) {
    __shared__ float tab[4 * 256];
    for (int i = threadIdx.x; i < channels * 256; i += 256) tab[i] = table[i];
    __syncthreads();
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    if (quads) {
        for (int64_t q = tid; q < n / 4; q += stride) {
            const uchar4 b = reinterpret_cast<const uchar4*>(src)[q];
            const float* t = tab + 256 * (int)(((4 * q) / plane) % channels);
            reinterpret_cast<float4*>(dst)[q] = make_float4(t[b.x], t[b.y], t[b.z], t[b.w]);
        }
    } else {
        for (int64_t i = tid; i < n; i += stride) dst[i] = tab[256 * (int)((i / plane) % channels) + src[i]];
    }
}

}  // namespace

extern "C" {

tf_status tf_decode_u8(tf_ctx* ctx, const uint8_t* src, float* dst, int64_t n, int64_t plane, int channels,
                       const float* table) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(n >= 0 && plane > 0 && channels >= 1 && channels <= 4, "tf_decode_u8: bad sizes (1 to 4 channels)");
    if (n == 0) return TF_OK;
    TF_REQUIRE(src && dst && table, "tf_decode_u8: null pointer");
    const int quads = (plane % 4 == 0 && n % 4 == 0 && (reinterpret_cast<uintptr_t>(src) & 3) == 0 &&
                       (reinterpret_cast<uintptr_t>(dst) & 15) == 0) ? 1 : 0;
    decode_u8_kernel<<<tfd::grid_for(n, quads ? 16 : 4), 256, 0, ctx->stream>>>(src, dst, n, plane, channels, table,
                                                                                quads);
    return tfh::check_launch("decode_u8_kernel");
}

}  // extern "C"

