// Out-of-memory policy of the pool allocator (tf_hip_alloc and the split-K /
// reduction workspace), kept free of HIP types so a host-only test can drive
// it with fake allocators.
#pragma once

namespace tfh {

enum class AllocOutcome { Ok, OutOfMemory, Failed };

// One allocation attempt, then, only if it ran out of memory, one release of
// what the context holds back (its cached blocks, its workspace) and one
// more attempt when that release handed anything back.  `attempt()` returns
// an AllocOutcome; `release()` returns true when it freed memory (and has
// waited for the frees to take effect), false when there was nothing to
// free or the release itself failed.
template <class Attempt, class Release>
AllocOutcome allocate_with_retry(Attempt&& attempt, Release&& release) {
    const AllocOutcome first = attempt();
    if (first != AllocOutcome::OutOfMemory) return first;
    if (!release()) return first;
    return attempt();
}

}  // namespace tfh
