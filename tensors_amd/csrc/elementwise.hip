// Elementwise bandwidth kernels: forward activations, their backward
// (ReLU / Sigmoid / Tanh), gradient accumulation (add), mul, scalar scale,
// the fused SGD-momentum update and f32<->bf16 casts.
//
// Every kernel is a grid-stride loop over 16-byte vectors (4 x f32 or
// 8 x bf16) with a scalar tail, 256 threads per block.  They are HBM-bound:
// the algorithmic traffic per element is listed beside each one.
#include "common.hpp"

namespace {

using tfd::bf16_to_f32;
using tfd::f32_to_bf16;

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

// Number of scalars in a 16-byte vector.
template <typename T> constexpr int kVec = 16 / sizeof(T);

// Binary elementwise: out = op(a, b).  Vector body when all three pointers
// are 16-byte aligned, scalar loop otherwise / for the tail.
template <typename T, typename Op>
__global__ void binary_kernel(const T* __restrict__ a, const T* __restrict__ b,
                              T* __restrict__ out, int64_t n, Op op, int vec_ok) {
    constexpr int V = kVec<T>;
    int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t nv = vec_ok ? n / V : 0;
    for (int64_t i = tid; i < nv; i += stride) {
        uint4 va = reinterpret_cast<const uint4*>(a)[i];
        uint4 vb = reinterpret_cast<const uint4*>(b)[i];
        uint4 vo;
        const T* ea = reinterpret_cast<const T*>(&va);
        const T* eb = reinterpret_cast<const T*>(&vb);
        T* eo = reinterpret_cast<T*>(&vo);
#pragma unroll
        for (int j = 0; j < V; ++j)
            Elem<T>::st(eo, j, op(Elem<T>::ld(ea, j), Elem<T>::ld(eb, j)));
        reinterpret_cast<uint4*>(out)[i] = vo;
    }
    for (int64_t i = nv * V + tid; i < n; i += stride)
        Elem<T>::st(out, i, op(Elem<T>::ld(a, i), Elem<T>::ld(b, i)));
}

template <typename T, typename Op>
__global__ void unary_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t n, Op op, int vec_ok) {
    constexpr int V = kVec<T>;
    int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t nv = vec_ok ? n / V : 0;
    for (int64_t i = tid; i < nv; i += stride) {
        uint4 vx = reinterpret_cast<const uint4*>(x)[i];
        uint4 vo;
        const T* ex = reinterpret_cast<const T*>(&vx);
        T* eo = reinterpret_cast<T*>(&vo);
#pragma unroll
        for (int j = 0; j < V; ++j) Elem<T>::st(eo, j, op(Elem<T>::ld(ex, j)));
        reinterpret_cast<uint4*>(y)[i] = vo;
    }
    for (int64_t i = nv * V + tid; i < n; i += stride) Elem<T>::st(y, i, op(Elem<T>::ld(x, i)));
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
        binary_kernel<float, Op><<<tfd::grid_for(n, 4 * 4), 256, 0, ctx->stream>>>(
            (const float*)a, (const float*)b, (float*)out, n, op, vec_ok);
    } else if (dtype == TF_BF16) {
        binary_kernel<uint16_t, Op><<<tfd::grid_for(n, 8 * 4), 256, 0, ctx->stream>>>(
            (const uint16_t*)a, (const uint16_t*)b, (uint16_t*)out, n, op, vec_ok);
    } else {
        return tfh::set_error(TF_ERR_UNSUPPORTED, std::string(name) + ": dtype must be Float32 or BFloat16");
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
        unary_kernel<float, Op><<<tfd::grid_for(n, 4 * 4), 256, 0, ctx->stream>>>(
            (const float*)x, (float*)y, n, op, vec_ok);
    } else if (dtype == TF_BF16) {
        unary_kernel<uint16_t, Op><<<tfd::grid_for(n, 8 * 4), 256, 0, ctx->stream>>>(
            (const uint16_t*)x, (uint16_t*)y, n, op, vec_ok);
    } else {
        return tfh::set_error(TF_ERR_UNSUPPORTED, std::string(name) + ": dtype must be Float32 or BFloat16");
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
__global__ void sgd_momentum_kernel(float* __restrict__ p, const float* __restrict__ g,
                                    float* __restrict__ v, uint16_t* __restrict__ p_bf16,
                                    int64_t n, float lr, float mu, int vec_ok) {
#pragma clang fp contract(off)
    int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t nv = vec_ok ? n / 4 : 0;
    const bool use_v = mu != 0.0f;
    for (int64_t i = tid; i < nv; i += stride) {
        float4 pp = reinterpret_cast<float4*>(p)[i];
        float4 gg = reinterpret_cast<const float4*>(g)[i];
        float* pe = reinterpret_cast<float*>(&pp);
        const float* ge = reinterpret_cast<const float*>(&gg);
        if (use_v) {
            float4 vv = reinterpret_cast<float4*>(v)[i];
            float* ve = reinterpret_cast<float*>(&vv);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float vm = ve[j] * mu;
                ve[j] = vm + ge[j];
                float step = ve[j] * lr;
                pe[j] = pe[j] - step;
            }
            reinterpret_cast<float4*>(v)[i] = vv;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float step = lr * ge[j];
                pe[j] = pe[j] - step;
            }
        }
        reinterpret_cast<float4*>(p)[i] = pp;
        if (p_bf16) {
            ushort4 h;
            h.x = f32_to_bf16(pe[0]);
            h.y = f32_to_bf16(pe[1]);
            h.z = f32_to_bf16(pe[2]);
            h.w = f32_to_bf16(pe[3]);
            reinterpret_cast<ushort4*>(p_bf16)[i] = h;
        }
    }
    for (int64_t i = nv * 4 + tid; i < n; i += stride) {
        float pv = p[i];
        if (use_v) {
            float vm = v[i] * mu;
            float vn = vm + g[i];
            v[i] = vn;
            float step = vn * lr;
            pv = pv - step;
        } else {
            float step = lr * g[i];
            pv = pv - step;
        }
        p[i] = pv;
        if (p_bf16) p_bf16[i] = f32_to_bf16(pv);
    }
}

__global__ void cast_f32_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y, int64_t n) {
    int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = tid; i < n; i += stride) y[i] = f32_to_bf16(x[i]);
}

__global__ void cast_bf16_f32_kernel(const uint16_t* __restrict__ x, float* __restrict__ y, int64_t n) {
    int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = tid; i < n; i += stride) y[i] = bf16_to_f32(x[i]);
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
    sgd_momentum_kernel<<<tfd::grid_for(n, 4 * 4), 256, 0, ctx->stream>>>(
        p, g, v, (uint16_t*)p_bf16, n, lr, mu, vec_ok);
    return tfh::check_launch("sgd_momentum_kernel");
}

tf_status tf_cast_f32_bf16(tf_ctx* ctx, const float* x, void* y, int64_t n) {
    TF_CTX_CHECK(ctx);
    if (n == 0) return TF_OK;
    TF_REQUIRE(x && y && n > 0, "tf_cast_f32_bf16: bad argument");
    cast_f32_bf16_kernel<<<tfd::grid_for(n, 4), 256, 0, ctx->stream>>>(x, (uint16_t*)y, n);
    return tfh::check_launch("cast_f32_bf16_kernel");
}

tf_status tf_cast_bf16_f32(tf_ctx* ctx, const void* x, float* y, int64_t n) {
    TF_CTX_CHECK(ctx);
    if (n == 0) return TF_OK;
    TF_REQUIRE(x && y && n > 0, "tf_cast_bf16_f32: bad argument");
    cast_bf16_f32_kernel<<<tfd::grid_for(n, 4), 256, 0, ctx->stream>>>((const uint16_t*)x, y, n);
    return tfh::check_launch("cast_bf16_f32_kernel");
}

}  // extern "C"
