// Shared plumbing for the gfx950 kernels behind include/tf_hip.h:
// the context struct, error recording, argument checks and small device
// helpers (wave64 reductions, bf16 conversion).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "tf_hip.h"

// The kernels are written for gfx950 (CDNA4) only.  Beyond instruction
// choice, the cross-block reductions (see tfd::wait_stores_landed below) rely on
// how this GPU's memory system orders and completes agent-scope atomics, so
// a device build for any other target is refused rather than left to run
// with different guarantees.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "tensors_amd kernels target gfx950 only (build with --offload-arch=gfx950)"
#endif

struct tf_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;   // current launch stream
    hipMemPool_t pool = nullptr;
    int num_cus = 0;
    // Scratch for multi-stage kernels (split-K partials, reduction partials,
    // per-row losses).  Grown on demand from the pool; stream-ordered.
    void* ws = nullptr;
    size_t ws_bytes = 0;
    // Block cache in front of the pool (tf_hip_alloc / tf_hip_free): freed
    // blocks wait here by size class and go to the next request of that
    // class, stream-ordered on `stream` like the pool's own reuse.  A pool
    // round trip (hipFreeAsync + hipMallocFromPoolAsync) costs 30-70 us of
    // host time per block on this runtime; a cache hit costs a map lookup.
    std::mutex cache_mu;
    std::unordered_map<size_t, std::vector<void*>> cached;  // size class -> free blocks
    std::unordered_map<void*, size_t> live;                  // block -> size class
    size_t cached_bytes = 0;
    // HIP-graph capture of the stream (tf_graph_begin .. tf_graph_end).
    // While capturing, allocations come from capture_free (blocks freed
    // earlier in the same capture) or the block cache, never from the pool;
    // frees go to capture_free, whose blocks the graph keeps until it is
    // destroyed, so a replay's temporaries are never handed to other work.
    bool capturing = false;
    bool capture_failed = false;  // a call failed while capturing
    std::unordered_map<size_t, std::vector<void*>> capture_free;
    // Blocks allocated during the current capture (the graph's kernels hold
    // their addresses), and, after tf_graph_end, those of them still live,
    // each mapped to its graph's list of held blocks: a tf_hip_free of such a
    // block hands it to the graph instead of the cache, so no other work is
    // given memory that later replays still write.
    std::vector<void*> capture_allocs;
    std::unordered_map<void*, std::vector<std::pair<void*, size_t>>*> graph_owned;
    // Arrival counters of the kernels whose last block to finish does a
    // final step (tfh::kTicket*): zero between launches (that block resets
    // its counter), so captured graphs replay them unchanged.  Launches on
    // one context are stream-ordered, so one counter per kernel suffices.
    unsigned* tickets = nullptr;
};

namespace tfh {

// Record a message for tf_last_error() and return the status.
tf_status set_error(tf_status code, const std::string& msg);
tf_status hip_error(hipError_t e, const char* what);

// Make sure ctx->ws holds at least `bytes`; returns TF_OK or an error.
tf_status ensure_workspace(tf_ctx* ctx, size_t bytes);
// out[m][n] (row stride ldc) = sum over s < splits of part[s][m][n] in a
// fixed order (16 split groups, each ascending, combined in a tree).
tf_status sum_partials(tf_ctx* ctx, const float* part, int64_t splits, int64_t M, int64_t N, float* out, int64_t ldc);
// out[j] = sum_k part[k * W + j] (fixed order) for j < W; columns j < split
// go to out_lo[j], the rest to out_hi[j - split].  Launched on ctx->stream.
tf_status partial_rows_sum(tf_ctx* ctx, const float* part, float* out_lo, float* out_hi, int64_t K, int64_t W,
                           int64_t split);

inline bool bad_ctx(tf_ctx* ctx) { return ctx == nullptr || ctx->stream == nullptr; }

// Slots of tf_ctx::tickets: the CE kernel's, then one per output tile of
// the small fp32 GEMM (at most kTicketGemmTiles tiles), then one per
// 32-column strip of the one-launch colsum.
constexpr int kTicketCE = 0;
constexpr int kTicketGemm = 64;
constexpr int kTicketGemmTiles = 4096;
constexpr int kTicketColsum = kTicketGemm + kTicketGemmTiles;
constexpr int kTicketColsumStrips = 4096;
constexpr int kTickets = kTicketColsum + kTicketColsumStrips;

// Launch timing (tf_hip_timing_*): a GEMM entry point constructs one of
// these around its launches; while recording is on it records an event on
// the context's stream at construction and another at destruction.
class TimedLaunch {
public:
    TimedLaunch(tf_ctx* ctx, int64_t M, int64_t N, int64_t K, int64_t batch, int trans_a, int trans_b, int in_dtype,
                int out_dtype);
    ~TimedLaunch();
    TimedLaunch(const TimedLaunch&) = delete;
    TimedLaunch& operator=(const TimedLaunch&) = delete;

private:
    tf_ctx* ctx_;
    int slot_ = -1;
};

// Launch-error check after every <<<>>>: catches bad launch shapes early.
inline tf_status check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, what);
    return TF_OK;
}

}  // namespace tfh

#define TF_REQUIRE(cond, msg)                                              \
    do {                                                                   \
        if (!(cond)) return tfh::set_error(TF_ERR_INVALID, (msg));         \
    } while (0)

#define TF_HIP_CHECK(expr)                                                 \
    do {                                                                   \
        hipError_t _e = (expr);                                            \
        if (_e != hipSuccess) return tfh::hip_error(_e, #expr);            \
    } while (0)

#define TF_CTX_CHECK(ctx)                                                  \
    do {                                                                   \
        if (tfh::bad_ctx(ctx)) return tfh::set_error(TF_ERR_INVALID, "null or shut-down tf_ctx"); \
    } while (0)

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
namespace tfd {

constexpr int kWave = 64;

// s_waitcnt immediate (gfx9 encoding, which gfx950 keeps) waiting until at
// most n vector memory operations of this wave are outstanding, leaving the
// export and LDS counters unconstrained.
constexpr int waitcnt_vm(int n) { return (n & 0xF) | ((n >> 4) << 14) | 0x0F70; }
// ... and also for all outstanding LDS operations.
constexpr int waitcnt_vm_lds(int n) { return (n & 0xF) | ((n >> 4) << 14) | 0x0070; }

// Cross-block reductions with a last-arriving block ("ticket" pattern):
// every block stores its partial results with agent-scope relaxed atomic
// stores, then counts itself in on a per-output counter with an agent-scope
// relaxed fetch_add; the block that draws the last ticket reads all partials
// with agent-scope relaxed atomic loads and writes the result.
//
// Why this is ordered on gfx950 without release/acquire cache maintenance:
//  * agent-scope atomic stores and loads are issued with the system-coherent
//    cache policy: a store is written through the issuing XCD's L2 to the
//    memory-side coherence point and a load is not served from a (possibly
//    stale) L2 line, so partials are visible to every XCD once they land;
//  * the wave counter vmcnt counts stores as well as loads on this GPU, and
//    a store leaves it only when the coherence point has acknowledged it, so
//    s_waitcnt vmcnt(0) in every thread means every partial of the block has
//    landed;
//  * the workgroup barrier after that wait (with its workgroup-scope fences,
//    which also keep the compiler from moving the atomic stores past it)
//    makes thread 0's ticket fetch_add happen after all of the block's
//    partials landed; the fetch_add is itself performed at the coherence
//    point, so a block that sees count == blocks - 1 runs after every other
//    block's partials landed, and its atomic loads see them.
// The C++/HIP memory model by itself promises this only with a release on
// the ticket and an acquire in the last block; on this GPU those lower to an
// L2 write-back and invalidate per block (buffer_wbl2 / buffer_inv), which
// made a one-launch column sum of 16 MB take 64 us instead of 7.4 us.  The
// pattern is therefore tied to gfx950 (the #error above), and a GPU test
// repeats each such kernel hundreds of times, comparing results bit for bit.
__device__ __forceinline__ void wait_stores_landed() { __builtin_amdgcn_s_waitcnt(waitcnt_vm(0)); }

// Direct global -> LDS loads (buffer_load_dwordx4 ... lds).  One instruction
// moves 16 bytes per active lane: lane l's bytes land at LDS byte M0 + 16 l,
// so a wave fills one contiguous KB per instruction with no registers and no
// LDS store instructions.  The loads count in vmcnt like any other load; the
// caller waits for them (s_waitcnt vmcnt) before a barrier and the reads.
// A lane offset at or past the descriptor's byte count reads zeros (raw
// buffer range check), which is how padding is filled.
typedef int buf_rsrc_t __attribute__((ext_vector_type(4)));
constexpr uint32_t kBufOob = 0x80000000u;   // a lane offset past every descriptor's range
// Descriptor for raw 16-byte loads of `bytes` bytes from `base` (gfx9-family
// word 3: raw dword access).
__device__ __forceinline__ buf_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return buf_rsrc_t{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xffffu), (int)bytes, 0x00020000};
}
// LDS byte address of a pointer into LDS.
__device__ __forceinline__ uint32_t lds_byte_addr(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)const_cast<void*>(p);
}
// One direct load: 16 bytes at byte offset voff of the descriptor's range
// into LDS byte lds_chunk + 16 (lane).  lds_chunk is wave-uniform.  Inline
// assembly so that the compiler's wait-count pass, which cannot track which
// LDS bytes such a load writes, adds no waits of its own; M0 is written here
// and used by nothing else in the kernels that call it.
__device__ __forceinline__ void load16_to_lds(buf_rsrc_t rsrc, uint32_t voff, uint32_t lds_chunk) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_chunk), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
}

// Butterfly sum over the 64 lanes of a wave; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

// f32 -> bf16 with the hardware conversion (v_cvt_pk_bf16_f32): round to
// nearest even; a NaN keeps its sign and top payload bits and is made quiet
// (bf16 bits = (f32 bits >> 16) | 0x40).  That is the rule of
// tensors_amd.f32_to_bf16_bits (the tests' oracle); a GPU test compares the
// two bit for bit over ties, denormals, overflow, infinities and NaN
// payloads.  One instruction per pair instead of about six per value.
typedef float cvt_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 cvt_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16x2_rne(float a, float b) {  // a in the low half
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(cvt_f32x2{a, b}, cvt_bf16x2));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// f32 -> IEEE half, round to nearest even (v_cvt_f16_f32), from a value
// that has been rounded to fp32 first.  The empty asm makes the fp32 value
// opaque: otherwise the compiler folds the producing multiply or add into a
// mixed-precision v_fma_mixlo_f16 (a * b + 0 straight to half), which rounds
// once instead of twice and turns a -0 product into +0 (found by the GPU
// test of the Float16 leaky ReLU on -0.0).
__device__ __forceinline__ _Float16 f32_to_f16(float v) {
    __asm__("" : "+v"(v));
    return (_Float16)v;
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(((uint32_t)h) << 16);
}

// Streaming accesses (global_load / global_store ... nt) for data a kernel
// touches once.  The non-temporal hint lets the caches evict these lines
// first.  On this GPU it raised a 16 MB copy from 4.5 to 4.9 TB/s, two reads
// plus a write from 4.7 to 5.5 TB/s, and three reads plus two writes (SGD)
// from 4.8 to 5.6 TB/s.  The event-timed microbenchmark rotated buffers past
// the 256 MB last-level cache.
typedef unsigned int nt_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int nt_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ld_nt(const uint4* p) {
    const nt_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt(uint4* p, const uint4& v) {
    __builtin_nontemporal_store(nt_u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<nt_u32x4*>(p));
}
__device__ __forceinline__ float4 ld_nt(const float4* p) {
    const nt_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4*>(p));
    return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
__device__ __forceinline__ void st_nt(float4* p, const float4& v) {
    __builtin_nontemporal_store(nt_u32x4{__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z),
                                         __float_as_uint(v.w)},
                                reinterpret_cast<nt_u32x4*>(p));
}
__device__ __forceinline__ uint2 ld_nt(const uint2* p) {
    const nt_u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x2*>(p));
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ void st_nt(uint2* p, const uint2& v) {
    __builtin_nontemporal_store(nt_u32x2{v.x, v.y}, reinterpret_cast<nt_u32x2*>(p));
}
// The same with the hint chosen at compile time.
template <bool NT, typename V>
__device__ __forceinline__ V ld_v(const V* p) {
    if constexpr (NT) return ld_nt(p);
    else return *p;
}
template <bool NT, typename V>
__device__ __forceinline__ void st_v(V* p, const V& v) {
    if constexpr (NT) st_nt(p, v);
    else *p = v;
}
// Launches that move more than this many bytes cannot keep their data in the
// 256 MB last-level cache between uses; below it (e.g. a small model's
// parameters, read again every step) cached accesses are faster: the SGD
// update of 4 M parameters (84 MB) took 12.9 us with warm data and cached
// accesses, 13.5 us with non-temporal ones; 24.2 vs 26.7 us with cold data.
constexpr int64_t kStreamMinBytes = 256ll << 20;

// Grid size for a grid-stride elementwise kernel over n items with 256
// threads per block: enough blocks to fill 256 CUs several times over.
inline int grid_for(int64_t n_items, int per_thread = 1, int max_blocks = 8192) {
    int64_t threads = (n_items + per_thread - 1) / per_thread;
    int64_t blocks = (threads + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > max_blocks) blocks = max_blocks;
    return (int)blocks;
}

}  // namespace tfd
