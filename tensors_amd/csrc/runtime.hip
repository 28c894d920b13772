// Runtime half of the C ABI: context + stream, pool allocator, copies,
// fills and events.  Replaces the reference's DeviceContext/CudaStream/
// CudaEvent (cuda/CudaContext.{hpp,cpp}) and CudaStorageAllocator
// (cuda/memory/CudaStorageAllocator.cpp:34-143).
//
// Design: one context per (caller, device).  Each context owns a
// non-blocking stream at default priority and the device's memory pool with
// an unlimited release threshold, so steady-state training steps never call
// into the driver for memory.  In front of the pool sits a per-context block
// cache: a freed block is kept by size class and handed to the next request
// of that class on the same stream, so steady-state steps make no pool calls
// either (a hipFreeAsync + hipMallocFromPoolAsync pair took 30-70 us of host
// time per block here, which made small training steps host-bound).
#include "alloc_policy.hpp"
#include "common.hpp"

#include <mutex>

namespace {

thread_local std::string g_last_error;

__global__ void fill_f32_kernel(float* __restrict__ p, float v, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    // float4 body over the 16-byte aligned prefix, scalar tail.
    int64_t n4 = ((reinterpret_cast<uintptr_t>(p) & 15) == 0) ? n / 4 : 0;
    float4* p4 = reinterpret_cast<float4*>(p);
    for (int64_t j = i; j < n4; j += stride) p4[j] = make_float4(v, v, v, v);
    for (int64_t j = n4 * 4 + i; j < n; j += stride) p[j] = v;
}

__global__ void zero_bytes_kernel(uint8_t* __restrict__ p, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t n16 = ((reinterpret_cast<uintptr_t>(p) & 15) == 0) ? n / 16 : 0;
    uint4* p16 = reinterpret_cast<uint4*>(p);
    for (size_t j = i; j < n16; j += stride) p16[j] = make_uint4(0, 0, 0, 0);
    for (size_t j = n16 * 16 + i; j < n; j += stride) p[j] = 0;
}

// Allocation sizes of the block cache: 512-byte steps up to 1 MB, 2 MB
// steps above (at most 2 MB, under 6 %, of padding for blocks of 32 MB+).
size_t size_class(size_t bytes) {
    const size_t step = bytes <= (size_t(1) << 20) ? 512 : (size_t(2) << 20);
    return (bytes + step - 1) / step * step;
}

// Hands every cached block back to the pool (stream-ordered); caller holds
// ctx->cache_mu.
tf_status release_cached(tf_ctx* ctx) {
    for (auto& kv : ctx->cached) {
        for (void* p : kv.second) TF_HIP_CHECK(hipFreeAsync(p, ctx->stream));
        kv.second.clear();
    }
    ctx->cached.clear();
    ctx->cached_bytes = 0;
    return TF_OK;
}

// Out-of-memory release: hands the cached blocks and the workspace back to
// the pool (stream-ordered, then waits for the stream so the pool can reuse
// them) and reports whether anything was freed.  Caller holds ctx->cache_mu.
bool release_for_retry(tf_ctx* ctx) {
    const bool any = ctx->cached_bytes > 0 || ctx->ws != nullptr;
    if (!any) return false;
    if (release_cached(ctx) != TF_OK) return false;
    if (ctx->ws) {
        if (hipFreeAsync(ctx->ws, ctx->stream) != hipSuccess) return false;
        ctx->ws = nullptr;
        ctx->ws_bytes = 0;
    }
    return hipStreamSynchronize(ctx->stream) == hipSuccess;
}

tfh::AllocOutcome outcome_of(hipError_t e) {
    if (e == hipSuccess) return tfh::AllocOutcome::Ok;
    (void)hipGetLastError();
    return e == hipErrorOutOfMemory ? tfh::AllocOutcome::OutOfMemory : tfh::AllocOutcome::Failed;
}

// Launch-timing records (tf_hip_timing_*), process-wide.
struct TimingRecord {
    int64_t shape[4];
    int meta[4];
};
struct TimingState {
    std::mutex mu;
    bool on = false;
    std::vector<hipEvent_t> events;   // 2 per record
    std::vector<TimingRecord> records;
    size_t used = 0;
};
TimingState& timing() {
    static TimingState t;
    return t;
}

}  // namespace

namespace tfh {

TimedLaunch::TimedLaunch(tf_ctx* ctx, int64_t M, int64_t N, int64_t K, int64_t batch, int trans_a, int trans_b,
                         int in_dtype, int out_dtype)
    : ctx_(ctx) {
    TimingState& t = timing();
    std::lock_guard<std::mutex> lock(t.mu);
    if (!t.on || ctx == nullptr || ctx->capturing || t.used >= t.records.size()) return;
    slot_ = (int)t.used++;
    t.records[slot_] = TimingRecord{{M, N, K, batch}, {trans_a, trans_b, in_dtype, out_dtype}};
    (void)hipEventRecord(t.events[2 * slot_], ctx->stream);
}

TimedLaunch::~TimedLaunch() {
    if (slot_ < 0) return;
    TimingState& t = timing();
    std::lock_guard<std::mutex> lock(t.mu);
    (void)hipEventRecord(t.events[2 * slot_ + 1], ctx_->stream);
}

tf_status set_error(tf_status code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

tf_status hip_error(hipError_t e, const char* what) {
    g_last_error = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
    return e == hipErrorOutOfMemory ? TF_ERR_OOM : TF_ERR_HIP;
}

tf_status ensure_workspace(tf_ctx* ctx, size_t bytes) {
    if (ctx->ws_bytes >= bytes) return TF_OK;
    if (ctx->capturing) {
        ctx->capture_failed = true;
        return set_error(TF_ERR_INVALID, "ensure_workspace: the workspace would grow while a graph is being captured "
                                         "(run the captured work once eagerly first)");
    }
    if (ctx->ws) {
        TF_HIP_CHECK(hipFreeAsync(ctx->ws, ctx->stream));
        ctx->ws = nullptr;
        ctx->ws_bytes = 0;
    }
    const size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
    hipError_t e = hipSuccess;
    void* p = nullptr;
    std::lock_guard<std::mutex> lock(ctx->cache_mu);
    const AllocOutcome r = allocate_with_retry(
        [&] { return outcome_of(e = hipMallocFromPoolAsync(&p, want, ctx->pool, ctx->stream)); },
        [&] { return release_for_retry(ctx); });
    if (r != AllocOutcome::Ok) return hip_error(e, "ensure_workspace: hipMallocFromPoolAsync");
    ctx->ws = p;
    ctx->ws_bytes = want;
    return TF_OK;
}

}  // namespace tfh

extern "C" {

const char* tf_last_error(void) { return g_last_error.c_str(); }

const char* tf_version(void) { return "tensors_amd 0.1 (gfx950)"; }

tf_status tf_hip_device_count(int* count) {
    TF_REQUIRE(count != nullptr, "tf_hip_device_count: null count");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    *count = (e == hipSuccess) ? n : 0;
    if (e != hipSuccess) (void)hipGetLastError();
    return TF_OK;
}

tf_status tf_hip_init(int device, tf_ctx** out) {
    TF_REQUIRE(out != nullptr, "tf_hip_init: null out");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
        (void)hipGetLastError();
        return tfh::set_error(TF_ERR_HIP, "tf_hip_init: no HIP device visible");
    }
    TF_REQUIRE(device >= 0 && device < n, "tf_hip_init: device index out of range");
    TF_HIP_CHECK(hipSetDevice(device));

    tf_ctx* ctx = new tf_ctx();
    ctx->device = device;
    hipDeviceProp_t prop;
    TF_HIP_CHECK(hipGetDeviceProperties(&prop, device));
    ctx->num_cus = prop.multiProcessorCount;
    // Default priority only: streams of mixed priority have hung these boxes.
    TF_HIP_CHECK(hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking));
    ctx->stream = ctx->own_stream;
    TF_HIP_CHECK(hipDeviceGetDefaultMemPool(&ctx->pool, device));
    uint64_t threshold = UINT64_MAX;  // keep freed blocks cached
    TF_HIP_CHECK(hipMemPoolSetAttribute(ctx->pool, hipMemPoolAttrReleaseThreshold, &threshold));
    TF_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&ctx->tickets), tfh::kTickets * sizeof(unsigned)));
    zero_bytes_kernel<<<1, 256, 0, ctx->stream>>>(reinterpret_cast<uint8_t*>(ctx->tickets),
                                                  tfh::kTickets * sizeof(unsigned));
    TF_HIP_CHECK(hipGetLastError());
    TF_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    *out = ctx;
    return TF_OK;
}

tf_status tf_hip_shutdown(tf_ctx* ctx) {
    if (ctx == nullptr) return TF_OK;
    if (ctx->capturing) {
        // An unfinished capture: end it, drop the graph, keep its blocks.
        hipGraph_t g = nullptr;
        if (hipStreamEndCapture(ctx->stream, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
        (void)hipGetLastError();
        ctx->capturing = false;
        for (auto& kv : ctx->capture_free)
            for (void* p : kv.second) ctx->cached[kv.first].push_back(p);
        ctx->capture_free.clear();
        ctx->capture_allocs.clear();
    }
    if (ctx->own_stream) {
        // Cached blocks go back to the pool once the current stream's work is done.
        if (ctx->stream != ctx->own_stream) (void)hipStreamSynchronize(ctx->stream);
        for (auto& kv : ctx->cached)
            for (void* p : kv.second) (void)hipFreeAsync(p, ctx->own_stream);
        if (ctx->ws) (void)hipFreeAsync(ctx->ws, ctx->own_stream);
        (void)hipStreamSynchronize(ctx->own_stream);
        (void)hipStreamDestroy(ctx->own_stream);
    }
    if (ctx->tickets) (void)hipFree(ctx->tickets);
    delete ctx;
    return TF_OK;
}

tf_status tf_hip_stream(tf_ctx* ctx, void** stream) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(stream != nullptr, "tf_hip_stream: null out");
    *stream = (void*)ctx->stream;
    return TF_OK;
}

tf_status tf_hip_set_stream(tf_ctx* ctx, void* stream) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(!ctx->capturing, "tf_hip_set_stream: a graph is being captured on this context");
    // Workspace frees are stream-ordered on the stream that last used them:
    // order the switch so the workspace is never used on two streams at once.
    hipStream_t next = stream ? (hipStream_t)stream : ctx->own_stream;
    if (next != ctx->stream) TF_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    ctx->stream = next;
    return TF_OK;
}

tf_status tf_hip_sync(tf_ctx* ctx) {
    TF_CTX_CHECK(ctx);
    if (ctx->capturing) {
        ctx->capture_failed = true;
        return tfh::set_error(TF_ERR_INVALID, "tf_hip_sync: a graph is being captured on this context");
    }
    TF_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    return TF_OK;
}

tf_status tf_hip_alloc(tf_ctx* ctx, size_t bytes, void** out) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(out != nullptr, "tf_hip_alloc: null out");
    const size_t cls = size_class(bytes == 0 ? 1 : bytes);
    std::lock_guard<std::mutex> lock(ctx->cache_mu);
    if (ctx->capturing) {
        // Blocks freed earlier in this capture first (stream order inside the
        // graph makes their reuse safe), then the cache; never the pool.
        auto cf = ctx->capture_free.find(cls);
        if (cf != ctx->capture_free.end() && !cf->second.empty()) {
            *out = cf->second.back();
            cf->second.pop_back();
            ctx->live.emplace(*out, cls);
            ctx->capture_allocs.push_back(*out);
            return TF_OK;
        }
    }
    auto it = ctx->cached.find(cls);
    if (it != ctx->cached.end() && !it->second.empty()) {
        // Last freed first (the block likeliest to still be in the caches).
        // Any cached block is safe: its uses were all enqueued on this
        // stream before its free, so they run before the new owner's work.
        *out = it->second.back();
        it->second.pop_back();
        ctx->cached_bytes -= cls;
        ctx->live.emplace(*out, cls);
        if (ctx->capturing) ctx->capture_allocs.push_back(*out);
        return TF_OK;
    }
    if (ctx->capturing) {
        *out = nullptr;
        ctx->capture_failed = true;
        return tfh::set_error(TF_ERR_INVALID, "tf_hip_alloc: no cached block of " + std::to_string(cls) +
                                                  " bytes while a graph is being captured (run the captured work "
                                                  "once eagerly first, so the block cache holds its blocks)");
    }
    hipError_t e = hipSuccess;
    const tfh::AllocOutcome r = tfh::allocate_with_retry(
        [&] { return outcome_of(e = hipMallocFromPoolAsync(out, cls, ctx->pool, ctx->stream)); },
        [&] { return release_for_retry(ctx); });
    if (r != tfh::AllocOutcome::Ok) {
        *out = nullptr;
        return tfh::hip_error(e, "tf_hip_alloc: hipMallocFromPoolAsync");
    }
    ctx->live.emplace(*out, cls);
    return TF_OK;
}

tf_status tf_hip_free(tf_ctx* ctx, void* ptr) {
    TF_CTX_CHECK(ctx);
    if (ptr == nullptr) return TF_OK;
    std::lock_guard<std::mutex> lock(ctx->cache_mu);
    auto it = ctx->live.find(ptr);
    TF_REQUIRE(it != ctx->live.end(), "tf_hip_free: pointer not allocated by this context (or freed twice)");
    if (ctx->capturing) {
        ctx->capture_free[it->second].push_back(ptr);
    } else if (auto g = ctx->graph_owned.find(ptr); g != ctx->graph_owned.end()) {
        // Allocated while a graph was captured that still exists: its
        // replays write this block, so the graph keeps it until destroyed.
        g->second->emplace_back(ptr, it->second);
        ctx->graph_owned.erase(g);
    } else {
        ctx->cached[it->second].push_back(ptr);
        ctx->cached_bytes += it->second;
    }
    ctx->live.erase(it);
    return TF_OK;
}

tf_status tf_hip_trim(tf_ctx* ctx, size_t keep_bytes) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(!ctx->capturing, "tf_hip_trim: a graph is being captured on this context");
    {
        std::lock_guard<std::mutex> lock(ctx->cache_mu);
        tf_status st = release_cached(ctx);
        if (st != TF_OK) return st;
    }
    TF_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    TF_HIP_CHECK(hipMemPoolTrimTo(ctx->pool, keep_bytes));
    return TF_OK;
}

tf_status tf_hip_pool_stats(tf_ctx* ctx, uint64_t* reserved, uint64_t* used) {
    TF_CTX_CHECK(ctx);
    uint64_t r = 0, u = 0;
    TF_HIP_CHECK(hipMemPoolGetAttribute(ctx->pool, hipMemPoolAttrReservedMemCurrent, &r));
    TF_HIP_CHECK(hipMemPoolGetAttribute(ctx->pool, hipMemPoolAttrUsedMemCurrent, &u));
    if (reserved) *reserved = r;
    if (used) *used = u;
    return TF_OK;
}

tf_status tf_hip_memcpy(tf_ctx* ctx, void* dst, const void* src, size_t bytes, int kind) {
    TF_CTX_CHECK(ctx);
    if (bytes == 0) return TF_OK;
    TF_REQUIRE(dst != nullptr && src != nullptr, "tf_hip_memcpy: null pointer");
    hipMemcpyKind k;
    switch (kind) {
    case TF_COPY_H2H: k = hipMemcpyHostToHost; break;
    case TF_COPY_H2D: k = hipMemcpyHostToDevice; break;
    case TF_COPY_D2H: k = hipMemcpyDeviceToHost; break;
    case TF_COPY_D2D: k = hipMemcpyDeviceToDevice; break;
    default: return tfh::set_error(TF_ERR_INVALID, "tf_hip_memcpy: bad copy kind");
    }
    if (ctx->capturing && kind != TF_COPY_D2D) {
        // A host buffer would be read or written at replay time, long after
        // the caller has reused it.
        ctx->capture_failed = true;
        return tfh::set_error(TF_ERR_INVALID, "tf_hip_memcpy: only device-to-device copies can be captured");
    }
    TF_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, k, ctx->stream));
    if (kind == TF_COPY_D2H || kind == TF_COPY_H2H || kind == TF_COPY_H2D) {
        // Host buffers are pageable and caller-owned: finish before returning.
        TF_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    }
    return TF_OK;
}

tf_status tf_hip_fill_f32(tf_ctx* ctx, float* p, float value, int64_t n) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(n >= 0, "tf_hip_fill_f32: negative n");
    if (n == 0) return TF_OK;
    TF_REQUIRE(p != nullptr, "tf_hip_fill_f32: null pointer");
    fill_f32_kernel<<<tfd::grid_for(n, 4), 256, 0, ctx->stream>>>(p, value, n);
    return tfh::check_launch("fill_f32_kernel");
}

tf_status tf_hip_zero(tf_ctx* ctx, void* p, size_t bytes) {
    TF_CTX_CHECK(ctx);
    if (bytes == 0) return TF_OK;
    TF_REQUIRE(p != nullptr, "tf_hip_zero: null pointer");
    zero_bytes_kernel<<<tfd::grid_for((int64_t)bytes, 16), 256, 0, ctx->stream>>>((uint8_t*)p, bytes);
    return tfh::check_launch("zero_bytes_kernel");
}

tf_status tf_hip_timing_start(int max_records) {
    TF_REQUIRE(max_records > 0 && max_records <= (1 << 20), "tf_hip_timing_start: max_records out of range");
    TimingState& t = timing();
    std::lock_guard<std::mutex> lock(t.mu);
    while (t.events.size() < 2 * (size_t)max_records) {
        hipEvent_t e;
        TF_HIP_CHECK(hipEventCreate(&e));
        t.events.push_back(e);
    }
    t.records.assign((size_t)max_records, TimingRecord{});
    t.used = 0;
    t.on = true;
    return TF_OK;
}

tf_status tf_hip_timing_stop(int* count) {
    TimingState& t = timing();
    std::lock_guard<std::mutex> lock(t.mu);
    t.on = false;
    if (count) *count = (int)t.used;
    return TF_OK;
}

tf_status tf_hip_timing_record(int i, int64_t* shape, int* meta, float* ms) {
    TimingState& t = timing();
    std::lock_guard<std::mutex> lock(t.mu);
    TF_REQUIRE(!t.on, "tf_hip_timing_record: stop recording first");
    TF_REQUIRE(i >= 0 && (size_t)i < t.used, "tf_hip_timing_record: no such record");
    if (shape)
        for (int j = 0; j < 4; ++j) shape[j] = t.records[i].shape[j];
    if (meta)
        for (int j = 0; j < 4; ++j) meta[j] = t.records[i].meta[j];
    if (ms) {
        TF_HIP_CHECK(hipEventSynchronize(t.events[2 * i + 1]));
        TF_HIP_CHECK(hipEventElapsedTime(ms, t.events[2 * i], t.events[2 * i + 1]));
    }
    return TF_OK;
}

tf_status tf_hip_event_create(tf_ctx* ctx, void** event) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(event != nullptr, "tf_hip_event_create: null out");
    hipEvent_t e;
    TF_HIP_CHECK(hipEventCreate(&e));
    *event = (void*)e;
    return TF_OK;
}

tf_status tf_hip_event_record(tf_ctx* ctx, void* event) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(event != nullptr, "tf_hip_event_record: null event");
    TF_HIP_CHECK(hipEventRecord((hipEvent_t)event, ctx->stream));
    return TF_OK;
}

tf_status tf_hip_event_elapsed(void* start, void* end, float* ms) {
    TF_REQUIRE(start && end && ms, "tf_hip_event_elapsed: null argument");
    TF_HIP_CHECK(hipEventSynchronize((hipEvent_t)end));
    TF_HIP_CHECK(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end));
    return TF_OK;
}

tf_status tf_hip_event_destroy(void* event) {
    if (event == nullptr) return TF_OK;
    TF_HIP_CHECK(hipEventDestroy((hipEvent_t)event));
    return TF_OK;
}

}  // extern "C"
