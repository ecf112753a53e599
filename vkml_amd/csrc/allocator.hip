// Device memory for vkhip_alloc / vkhip_free: a caching allocator ordered by
// the backend's single stream.
//
// The reference defers a free until the GPU has passed the timeline value of
// the work that used the buffer (retirement queue, vulkan_backend.cpp:921-984).
// Here every launch, copy and fill of the backend is enqueued on ONE stream,
// so a block released by the host can be handed to the next allocation at
// once: whatever uses it next is enqueued later on the same stream and runs
// after every earlier use. Blocks are kept in per-size free lists (sizes
// rounded up, below) and returned to HIP only on an allocation failure, on
// vkhip_release_cached and at shutdown; hipMalloc/hipFree are never on the
// per-node path. (Stream-ordered hipMallocAsync/hipFreeAsync measured about
// 10-90 us per call on MI355X, the larger for larger blocks, which made a
// CIFAR training step mostly host time.)
//
// When the backend is moved to another stream (vkhip_set_stream) the old
// stream is synchronised first, so cached blocks carry no pending work across
// streams.
#include <mutex>
#include <unordered_map>
#include <vector>

#include "common.h"

namespace vkhip {

namespace {

struct Cache {
    std::mutex mu;
    std::unordered_map<size_t, std::vector<void*>> free_lists;  // rounded size -> blocks
    std::unordered_map<void*, size_t> live;                       // block -> rounded size
    size_t bytes_live = 0;
    size_t bytes_cached = 0;
};

Cache& cache() {
    static Cache c;
    return c;
}

// 256-byte steps up to 1 MiB, 64 KiB steps up to 64 MiB, 2 MiB steps above:
// at most ~3% of padding past 1 MiB, and the few sizes a training step uses
// repeat exactly from step to step.
size_t round_size(size_t n) {
    const size_t step = n <= (1u << 20) ? 256 : n <= (64u << 20) ? (64u << 10) : (2u << 20);
    return (n + step - 1) / step * step;
}

// Returns every cached block to HIP. The caller holds the lock.
int release_locked(Cache& c) {
    if (c.bytes_cached == 0) return VKHIP_OK;
    VKHIP_HIP(hipStreamSynchronize(ctx().stream));
    for (auto& kv : c.free_lists)
        for (void* p : kv.second) VKHIP_HIP(hipFree(p));
    c.free_lists.clear();
    c.bytes_cached = 0;
    return VKHIP_OK;
}

}  // namespace

int cached_alloc(size_t nbytes, void** out) {
    Cache& c = cache();
    const size_t sz = round_size(nbytes);
    std::lock_guard<std::mutex> lk(c.mu);
    auto it = c.free_lists.find(sz);
    if (it != c.free_lists.end() && !it->second.empty()) {
        *out = it->second.back();
        it->second.pop_back();
        c.bytes_cached -= sz;
    } else {
        void* p = nullptr;
        if (hipMalloc(&p, sz) != hipSuccess) {
            (void)hipGetLastError();
            publish("allocator.release", "alloc", "release_cached", "",
                    "an allocation failed: cached blocks go back to HIP and it is retried",
                    static_cast<int64_t>(sz), static_cast<int64_t>(c.bytes_cached));
            int st = release_locked(c);
            if (st != VKHIP_OK) return st;
            if (hipMalloc(&p, sz) != hipSuccess) {
                (void)hipGetLastError();
                return fail(VKHIP_ERR_OOM, "alloc: %zu bytes could not be allocated", nbytes);
            }
        }
        *out = p;
    }
    c.live.emplace(*out, sz);
    c.bytes_live += sz;
    return VKHIP_OK;
}

int cached_free(void* ptr) {
    Cache& c = cache();
    std::lock_guard<std::mutex> lk(c.mu);
    auto it = c.live.find(ptr);
    if (it == c.live.end())
        return fail(VKHIP_ERR_INVALID, "free: %p was not allocated by vkhip_alloc (or freed twice)", ptr);
    const size_t sz = it->second;
    c.live.erase(it);
    c.bytes_live -= sz;
    c.free_lists[sz].push_back(ptr);
    c.bytes_cached += sz;
    return VKHIP_OK;
}

int release_cached() {
    Cache& c = cache();
    std::lock_guard<std::mutex> lk(c.mu);
    return release_locked(c);
}

void memory_stats(size_t* live, size_t* cached) {
    Cache& c = cache();
    std::lock_guard<std::mutex> lk(c.mu);
    if (live) *live = c.bytes_live;
    if (cached) *cached = c.bytes_cached;
}

}  // namespace vkhip
