// HIP-graph capture of a context's work, and two small kernels that let a
// captured training step pick its batch and record its loss on the device,
// so that one graph launch per step replays the whole step.
//
// The reference launches every kernel of a step from the host
// (examples/train_mlp.cpp:141-199 drives forward, backward and SGD per
// batch); at config 1's sizes (batch 64, 784-256-128-10) the ~17 launches of
// a step cost more host time than their kernels take, so capture turns them
// into one hipGraphLaunch.
//
// Capture rules (enforced in runtime.hip): while a graph is being captured
// the block cache serves every allocation (a miss is an error, as is growing
// the workspace), frees go to a capture-local list that later allocations
// of the same capture reuse, and synchronising calls or host copies are
// errors.  The graph keeps the blocks freed during capture until it is
// destroyed, and so are blocks allocated during capture that are freed while
// the graph exists, so no other work is handed memory a replay writes.
#include "common.hpp"

#include <vector>

struct tf_graph {
    tf_ctx* ctx = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    void* ws = nullptr;                                // the context's workspace at capture
    // Blocks the graph keeps until it is destroyed: those freed during
    // capture, and those allocated during capture and freed since.
    std::vector<std::pair<void*, size_t>> held;
};

namespace {

// dst[0:bytes) = table[*counter % n][0:bytes): the batch of the step the
// counter names.  Grid-stride over 16-byte vectors when all of dst, the
// source and bytes are 16-byte multiples (checked per call on the device,
// since the source is chosen there), else bytes.
__global__ __launch_bounds__(256) void gather_indexed_kernel(uint8_t* __restrict__ dst,
                                                             const uint64_t* __restrict__ table, int64_t n,
                                                             const int64_t* __restrict__ counter, int64_t bytes) {
    const int64_t c = *counter;
    const int64_t k = ((c % n) + n) % n;
    const uint8_t* src = reinterpret_cast<const uint8_t*>(table[k]);
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const bool vec = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) | (uintptr_t)bytes) & 15) == 0;
    if (vec) {
        const uint4* s4 = reinterpret_cast<const uint4*>(src);
        uint4* d4 = reinterpret_cast<uint4*>(dst);
        for (int64_t i = tid; i < bytes / 16; i += stride) d4[i] = s4[i];
    } else {
        for (int64_t i = tid; i < bytes; i += stride) dst[i] = src[i];
    }
}

// ring[*counter] = *src when *counter < ring_len; then ++*counter.  Lane 0
// of one wave: it runs after the step's last kernel, in stream order.
__global__ void record_step_kernel(const float* __restrict__ src, float* __restrict__ ring, int64_t ring_len,
                                   int64_t* __restrict__ counter) {
    if (threadIdx.x != 0) return;
    const int64_t c = *counter;
    if (c >= 0 && c < ring_len) ring[c] = *src;
    *counter = c + 1;
}

}  // namespace

extern "C" {

tf_status tf_graph_begin(tf_ctx* ctx) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(!ctx->capturing, "tf_graph_begin: a graph is already being captured on this context");
    // Thread-local mode: a call on this thread that is unsafe during capture
    // fails instead of silently running.
    TF_HIP_CHECK(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    std::lock_guard<std::mutex> lock(ctx->cache_mu);
    ctx->capturing = true;
    ctx->capture_failed = false;
    ctx->capture_free.clear();
    ctx->capture_allocs.clear();
    return TF_OK;
}

tf_status tf_graph_end(tf_ctx* ctx, tf_graph** out) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(out != nullptr, "tf_graph_end: null out");
    *out = nullptr;
    TF_REQUIRE(ctx->capturing, "tf_graph_end: no graph is being captured on this context");
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
    std::vector<std::pair<void*, size_t>> held;
    std::vector<void*> allocs;
    bool failed;
    {
        std::lock_guard<std::mutex> lock(ctx->cache_mu);
        ctx->capturing = false;
        failed = ctx->capture_failed || e != hipSuccess || graph == nullptr;
        for (auto& kv : ctx->capture_free)
            for (void* p : kv.second) held.emplace_back(p, kv.first);
        ctx->capture_free.clear();
        allocs.swap(ctx->capture_allocs);
        if (failed) {
            // Nothing was run: the blocks go back to the cache as they are.
            for (auto& b : held) {
                ctx->cached[b.second].push_back(b.first);
                ctx->cached_bytes += b.second;
            }
        }
    }
    if (failed) {
        if (graph) (void)hipGraphDestroy(graph);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return tfh::hip_error(e, "tf_graph_end: hipStreamEndCapture");
        }
        // The failing call's own message is kept in tf_last_error().
        return TF_ERR_INVALID;
    }
    hipGraphExec_t exec = nullptr;
    const hipError_t ei = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (ei != hipSuccess) {
        (void)hipGraphDestroy(graph);
        std::lock_guard<std::mutex> lock(ctx->cache_mu);
        for (auto& b : held) {
            ctx->cached[b.second].push_back(b.first);
            ctx->cached_bytes += b.second;
        }
        return tfh::hip_error(ei, "tf_graph_end: hipGraphInstantiate");
    }
    tf_graph* g = new tf_graph();
    g->ctx = ctx;
    g->graph = graph;
    g->exec = exec;
    g->ws = ctx->ws;
    g->held = std::move(held);
    {
        // Blocks allocated during capture and still live: a later free hands
        // them to this graph (tf_hip_free) instead of the cache.
        std::lock_guard<std::mutex> lock(ctx->cache_mu);
        for (void* p : allocs)
            if (ctx->live.count(p)) ctx->graph_owned[p] = &g->held;
    }
    *out = g;
    return TF_OK;
}

tf_status tf_graph_launch(tf_ctx* ctx, tf_graph* g) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(g != nullptr && g->exec != nullptr, "tf_graph_launch: null graph");
    TF_REQUIRE(g->ctx == ctx, "tf_graph_launch: the graph was captured on another context");
    TF_REQUIRE(!ctx->capturing, "tf_graph_launch: a graph is being captured on this context");
    // The graph's kernels hold the workspace address of capture time.
    TF_REQUIRE(ctx->ws == g->ws, "tf_graph_launch: the context's workspace was reallocated since the capture");
    TF_HIP_CHECK(hipGraphLaunch(g->exec, ctx->stream));
    return TF_OK;
}

tf_status tf_graph_destroy(tf_graph* g) {
    if (g == nullptr) return TF_OK;
    tf_ctx* ctx = g->ctx;
    hipError_t e1 = g->exec ? hipGraphExecDestroy(g->exec) : hipSuccess;
    hipError_t e2 = g->graph ? hipGraphDestroy(g->graph) : hipSuccess;
    {
        // Replays were enqueued on ctx->stream before this call, so the
        // blocks follow the cache's stream-ordered reuse like any free.
        std::lock_guard<std::mutex> lock(ctx->cache_mu);
        for (auto& b : g->held) {
            ctx->cached[b.second].push_back(b.first);
            ctx->cached_bytes += b.second;
        }
        // Its still-live blocks become ordinary ones again.
        for (auto it = ctx->graph_owned.begin(); it != ctx->graph_owned.end();)
            it = it->second == &g->held ? ctx->graph_owned.erase(it) : std::next(it);
    }
    delete g;
    if (e1 != hipSuccess) return tfh::hip_error(e1, "tf_graph_destroy: hipGraphExecDestroy");
    if (e2 != hipSuccess) return tfh::hip_error(e2, "tf_graph_destroy: hipGraphDestroy");
    return TF_OK;
}

tf_status tf_gather_indexed(tf_ctx* ctx, void* dst, const uint64_t* table, int64_t n, const int64_t* counter,
                            int64_t bytes) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(dst && table && counter, "tf_gather_indexed: null pointer");
    TF_REQUIRE(n > 0 && bytes >= 0, "tf_gather_indexed: bad sizes");
    if (bytes == 0) return TF_OK;
    gather_indexed_kernel<<<tfd::grid_for(bytes, 64, 1024), 256, 0, ctx->stream>>>((uint8_t*)dst, table, n, counter,
                                                                                    bytes);
    return tfh::check_launch("gather_indexed_kernel");
}

tf_status tf_record_step(tf_ctx* ctx, const float* src, float* ring, int64_t ring_len, int64_t* counter) {
    TF_CTX_CHECK(ctx);
    TF_REQUIRE(src && ring && counter, "tf_record_step: null pointer");
    TF_REQUIRE(ring_len > 0, "tf_record_step: empty ring");
    record_step_kernel<<<1, 64, 0, ctx->stream>>>(src, ring, ring_len, counter);
    return tfh::check_launch("record_step_kernel");
}

}  // extern "C"
