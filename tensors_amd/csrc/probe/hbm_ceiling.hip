// HBM streaming ceilings of this GPU: the rate a plain streaming kernel
// reaches for the access mixes of the path's bandwidth kernels, so their
// achieved GB/s can be read against what the memory system delivers rather
// than only against the published 8 TB/s.
//
// Built into its own library (libtf_hbm_probe.so), not into libtf_hip.so:
// it is a measuring instrument, not part of the drop-in.
//
// Mixes (16-byte vectors, the elementwise kernels' loop and grid: a block
// takes chunks of 4 x 256 vectors, each thread issues its four loads before
// any store; one block per chunk up to 8192 blocks):
//   kind 0: copy            out0 = in0                 1 read, 1 write
//   kind 1: two reads, one write  out0 = in0 + in1     (ReLU backward, add)
//   kind 2: three reads, two writes  (SGD momentum: p, g, v in; p, v out)
//   kind 3: read only (column sums): the loaded values are summed and the sum
//           is stored only if it equals a value that the zero-filled arrays
//           never produce, which keeps the loads live without a write stream
// each with cached or non-temporal (nt) loads and stores.
//
// Every launch works on one of several buffer sets whose total size is at
// least 1 GiB (four times the 256 MB last-level cache), cycled in order, so
// each launch streams from HBM.
#include "common.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

namespace {

constexpr int kUnroll = 4;
constexpr int kChunk = kUnroll * 256;

template <bool NT>
__device__ __forceinline__ float4 ld(const float4* p) {
    if constexpr (NT) return tfd::ld_nt(p);
    else return *p;
}
template <bool NT>
__device__ __forceinline__ void st(float4* p, const float4& v) {
    if constexpr (NT) tfd::st_nt(p, v);
    else *p = v;
}

__device__ __forceinline__ float4 add4(const float4& a, const float4& b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
__device__ __forceinline__ float4 sub4(const float4& a, const float4& b) {
    return make_float4(a.x - b.x, a.y - b.y, a.z - b.z, a.w - b.w);
}

// nv: number of 16-byte vectors per array, a multiple of kChunk.
template <int NIN, int NOUT, bool NT>
__global__ __launch_bounds__(256) void hbm_stream_kernel(const float4* __restrict__ a, const float4* __restrict__ b,
                                                         const float4* __restrict__ c, float4* __restrict__ o0,
                                                         float4* __restrict__ o1, int64_t nv) {
    const int64_t chunks = nv / kChunk;
    for (int64_t ch = blockIdx.x; ch < chunks; ch += gridDim.x) {
        const int64_t i = ch * kChunk + threadIdx.x;
        float4 va[kUnroll], vb[kUnroll], vc[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            va[u] = ld<NT>(a + i + u * 256);
            if constexpr (NIN > 1) vb[u] = ld<NT>(b + i + u * 256);
            if constexpr (NIN > 2) vc[u] = ld<NT>(c + i + u * 256);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            float4 r = va[u];
            if constexpr (NIN > 1) r = add4(r, vb[u]);
            if constexpr (NIN > 2) r = add4(r, vc[u]);
            if constexpr (NOUT == 0) {
                if (r.x + r.y + r.z + r.w == 1234.5f) o0[i + u * 256] = r;
            } else {
                st<NT>(o0 + i + u * 256, r);
            }
            if constexpr (NOUT > 1) st<NT>(o1 + i + u * 256, sub4(vb[u], vc[u]));
        }
    }
}

// A second, independent streaming form: persistent blocks (gridDim =
// CUs x B), each owning one contiguous 1/gridDim of the arrays (split at
// 256-vector granularity) and walking it with U 16-byte loads per input in
// flight per thread before any arithmetic or store (U = 16 with one block
// per CU, U = 8 with two).  It shares no loop shape with the elementwise
// kernels, so a rate it reaches and they do not is a loss in those kernels.
template <int NIN, int NOUT, bool NT, int U>
__global__ __launch_bounds__(256) void hbm_persistent_kernel(const float4* __restrict__ a, const float4* __restrict__ b,
                                                             const float4* __restrict__ c, float4* __restrict__ o0,
                                                             float4* __restrict__ o1, int64_t nv) {
    const int64_t groups = nv / 256;
    const int64_t v0 = groups * blockIdx.x / gridDim.x * 256, v1 = groups * (blockIdx.x + 1) / gridDim.x * 256;
    for (int64_t i = v0 + threadIdx.x; i < v1; i += (int64_t)U * 256) {
        float4 va[U], vb[U], vc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t j = i + u * 256 < v1 ? i + u * 256 : i;
            va[u] = ld<NT>(a + j);
            if constexpr (NIN > 1) vb[u] = ld<NT>(b + j);
            if constexpr (NIN > 2) vc[u] = ld<NT>(c + j);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (i + u * 256 >= v1) break;
            float4 r = va[u];
            if constexpr (NIN > 1) r = add4(r, vb[u]);
            if constexpr (NIN > 2) r = add4(r, vc[u]);
            if constexpr (NOUT == 0) {
                if (r.x + r.y + r.z + r.w == 1234.5f) o0[i + u * 256] = r;
            } else {
                st<NT>(o0 + i + u * 256, r);
            }
            if constexpr (NOUT > 1) st<NT>(o1 + i + u * 256, sub4(vb[u], vc[u]));
        }
    }
}

struct Mix {
    int nin, nout;
};
constexpr Mix kMixes[4] = {{1, 1}, {2, 1}, {3, 2}, {1, 0}};

// form 0: the elementwise kernels' loop and grid; 1: the persistent form,
// a block per CU (pgrid) with 16 loads per input in flight per thread; 2:
// two blocks per CU with 8.
template <int NIN, int NOUT>
void launch_mix(bool nt, int form, unsigned grid, unsigned pgrid, float4** arr, int64_t nv, hipStream_t s) {
    const float4* a = arr[0];
    const float4* b = NIN > 1 ? arr[1] : nullptr;
    const float4* c = NIN > 2 ? arr[2] : nullptr;
    // The read-only mix has no output array: its guarded store (never taken
    // for zero-filled data) would go to its input.
    float4* o0 = NOUT > 0 ? arr[NIN] : arr[0];
    float4* o1 = NOUT > 1 ? arr[NIN + 1] : nullptr;
    if (form == 1) {
        if (nt) hbm_persistent_kernel<NIN, NOUT, true, 16><<<pgrid, 256, 0, s>>>(a, b, c, o0, o1, nv);
        else hbm_persistent_kernel<NIN, NOUT, false, 16><<<pgrid, 256, 0, s>>>(a, b, c, o0, o1, nv);
    } else if (form == 2) {
        if (nt) hbm_persistent_kernel<NIN, NOUT, true, 8><<<2 * pgrid, 256, 0, s>>>(a, b, c, o0, o1, nv);
        else hbm_persistent_kernel<NIN, NOUT, false, 8><<<2 * pgrid, 256, 0, s>>>(a, b, c, o0, o1, nv);
    } else {
        if (nt) hbm_stream_kernel<NIN, NOUT, true><<<grid, 256, 0, s>>>(a, b, c, o0, o1, nv);
        else hbm_stream_kernel<NIN, NOUT, false><<<grid, 256, 0, s>>>(a, b, c, o0, o1, nv);
    }
}

void launch(int kind, bool nt, int form, unsigned grid, unsigned pgrid, float4** arr, int64_t nv, hipStream_t s) {
    switch (kind) {
    case 0: launch_mix<1, 1>(nt, form, grid, pgrid, arr, nv, s); break;
    case 1: launch_mix<2, 1>(nt, form, grid, pgrid, arr, nv, s); break;
    case 2: launch_mix<3, 2>(nt, form, grid, pgrid, arr, nv, s); break;
    default: launch_mix<1, 0>(nt, form, grid, pgrid, arr, nv, s); break;
    }
}

}  // namespace

extern "C" {

// Average device time of one launch of mix `kind` (0 copy, 1 two reads + one
// write, 2 three reads + two writes, 3 read only) over arrays of `bytes` bytes each
// (rounded down to a multiple of 256 KiB), non-temporal when `nt` is set, in
// streaming form `form` (0: the elementwise kernels' loop and grid, 1 / 2:
// persistent blocks, one per CU with 16 loads per input in flight per
// thread / two per CU with 8):
// `reps` launches cycling over the buffer sets, timed with one event pair on
// a stream of default priority after one untimed pass over every set.
// Returns 0 on success, -1 for bad arguments, else the HIP error code.
int tf_hbm_probe_form(int kind, int nt, int64_t bytes, int reps, int form, double* us_per_launch) {
    if (kind < 0 || kind > 3 || reps < 1 || form < 0 || form > 2 || us_per_launch == nullptr) return -1;
    const int64_t nv = bytes / 16 / (16 * kChunk) * (16 * kChunk);   // a whole number of form 2's steps too
    if (nv <= 0) return -1;
    const Mix m = kMixes[kind];
    const int per_set = m.nin + m.nout;
    const int64_t set_bytes = (int64_t)per_set * nv * 16;
    const int sets = (int)std::max<int64_t>(2, ((int64_t)1 << 30) / set_bytes + 1);
    // One block per chunk up to 8192 blocks, as the elementwise kernels launch;
    // the persistent forms: one or two blocks per CU.
    const unsigned grid = (unsigned)tfd::grid_for(nv, kUnroll);
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return -1;
    const unsigned pgrid = (unsigned)cus;

    std::vector<float4*> bufs((size_t)sets * per_set, nullptr);
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    auto cleanup = [&]() {
        for (float4* p : bufs)
            if (p) (void)hipFree(p);
        if (e0) (void)hipEventDestroy(e0);
        if (e1) (void)hipEventDestroy(e1);
        if (s) (void)hipStreamDestroy(s);
    };
#define TF_PROBE_CHECK(expr)            \
    do {                                \
        hipError_t r_ = (expr);         \
        if (r_ != hipSuccess) {         \
            cleanup();                  \
            return (int)r_;             \
        }                               \
    } while (0)
    for (float4*& p : bufs) {
        TF_PROBE_CHECK(hipMalloc(reinterpret_cast<void**>(&p), (size_t)nv * 16));
        TF_PROBE_CHECK(hipMemset(p, 0, (size_t)nv * 16));
    }
    TF_PROBE_CHECK(hipStreamCreate(&s));
    TF_PROBE_CHECK(hipEventCreate(&e0));
    TF_PROBE_CHECK(hipEventCreate(&e1));
    for (int i = 0; i < sets; ++i) launch(kind, nt != 0, form, grid, pgrid, &bufs[(size_t)i * per_set], nv, s);
    TF_PROBE_CHECK(hipGetLastError());
    TF_PROBE_CHECK(hipEventRecord(e0, s));
    for (int r = 0; r < reps; ++r)
        launch(kind, nt != 0, form, grid, pgrid, &bufs[(size_t)(r % sets) * per_set], nv, s);
    TF_PROBE_CHECK(hipGetLastError());
    TF_PROBE_CHECK(hipEventRecord(e1, s));
    TF_PROBE_CHECK(hipEventSynchronize(e1));
    float ms = 0.0f;
    TF_PROBE_CHECK(hipEventElapsedTime(&ms, e0, e1));
#undef TF_PROBE_CHECK
    cleanup();
    *us_per_launch = (double)ms * 1e3 / reps;
    return 0;
}

// The elementwise kernels' form (form 0).
int tf_hbm_probe(int kind, int nt, int64_t bytes, int reps, double* us_per_launch) {
    return tf_hbm_probe_form(kind, nt, bytes, reps, 0, us_per_launch);
}

// Bytes one launch of `kind` moves for arrays of `bytes` bytes (after the
// same rounding as tf_hbm_probe_form).
int64_t tf_hbm_probe_bytes(int kind, int64_t bytes) {
    if (kind < 0 || kind > 3) return -1;
    const int64_t nv = bytes / 16 / (16 * kChunk) * (16 * kChunk);
    return (int64_t)(kMixes[kind].nin + kMixes[kind].nout) * nv * 16;
}

}  // extern "C"
