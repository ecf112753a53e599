// Decision facts and per-unit timing (include/vkhip.h, "Observability").
//
// Decision sites call publish() and learn nothing back: whether a subscriber
// exists is this file's business (the reference's rule, observe.h:22-37).
// Units of work (a node of vkhip_compute, or one per-op entry call) get a
// dispatch id when they begin; decisions published inside a unit quote it, and
// when profiling is on the unit's launches are bracketed by a pair of pooled
// HIP events on the backend stream, read back by vkhip_profile_read.
#include <atomic>
#include <cstring>
#include <deque>
#include <mutex>
#include <vector>

#include "common.h"

namespace vkhip {

namespace {

struct Pending {
    char label[48];
    hipEvent_t start, end;
    uint64_t dispatch;
};

struct Observe {
    std::mutex mu;
    vkhip_decision_fn fn = nullptr;
    void* user = nullptr;
    std::atomic<bool> subscribed{false};
    std::atomic<bool> profiling{false};
    uint64_t next_dispatch = 0;
    uint64_t current = 0;
    int depth = 0;  // units do not nest: an inner begin joins the outer unit
    hipEvent_t open_start = nullptr;
    char open_label[48] = {0};
    std::deque<Pending> pending;
    std::vector<hipEvent_t> free_events;
    uint64_t dropped = 0;
};

Observe& obs() {
    static Observe o;
    return o;
}

constexpr size_t kMaxPending = 65536;

hipEvent_t take_event(Observe& o) {
    if (!o.free_events.empty()) {
        hipEvent_t e = o.free_events.back();
        o.free_events.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return e;
}

}  // namespace

void publish(const char* site, const char* op, const char* chose, const char* instead_of,
             const char* because, int64_t required, int64_t available) {
    Observe& o = obs();
    if (!o.subscribed.load(std::memory_order_relaxed)) return;
    vkhip_decision_fn fn;
    void* user;
    vkhip_decision d{site, op, chose, instead_of ? instead_of : "", because ? because : "",
                     required, available, 0};
    {
        std::lock_guard<std::mutex> lk(o.mu);
        fn = o.fn;
        user = o.user;
        d.dispatch = o.current;
    }
    if (fn) fn(&d, user);  // outside the lock: a subscriber may call back in
}

void unit_begin(const char* label) {
    Observe& o = obs();
    std::lock_guard<std::mutex> lk(o.mu);
    if (o.depth++ > 0) return;
    o.current = ++o.next_dispatch;
    if (!o.profiling.load(std::memory_order_relaxed)) return;
    o.open_start = take_event(o);
    snprintf(o.open_label, sizeof o.open_label, "%s", label);
    if (o.open_start && hipEventRecord(o.open_start, ctx().stream) != hipSuccess) {
        (void)hipGetLastError();
        o.free_events.push_back(o.open_start);
        o.open_start = nullptr;
    }
}

void unit_end() {
    Observe& o = obs();
    std::lock_guard<std::mutex> lk(o.mu);
    if (o.depth == 0 || --o.depth > 0) return;
    if (!o.open_start) return;
    hipEvent_t end = take_event(o);
    if (!end || hipEventRecord(end, ctx().stream) != hipSuccess) {
        (void)hipGetLastError();
        o.free_events.push_back(o.open_start);
        if (end) o.free_events.push_back(end);
        o.open_start = nullptr;
        return;
    }
    Pending p;
    memcpy(p.label, o.open_label, sizeof p.label);
    p.start = o.open_start;
    p.end = end;
    p.dispatch = o.current;
    o.open_start = nullptr;
    if (o.pending.size() >= kMaxPending) {
        // Oldest first out; its events are complete or will be by reuse
        // (events recorded again simply move forward on the stream).
        o.free_events.push_back(o.pending.front().start);
        o.free_events.push_back(o.pending.front().end);
        o.pending.pop_front();
        ++o.dropped;
    }
    o.pending.push_back(p);
}

}  // namespace vkhip

using vkhip::ctx;
using vkhip::fail;

extern "C" int vkhip_subscribe_decisions(vkhip_decision_fn fn, void* user) {
    vkhip::Observe& o = vkhip::obs();
    std::lock_guard<std::mutex> lk(o.mu);
    o.fn = fn;
    o.user = user;
    o.subscribed.store(fn != nullptr, std::memory_order_relaxed);
    return VKHIP_OK;
}

namespace vkhip {
bool profiling_on() { return obs().profiling.load(std::memory_order_relaxed); }
}  // namespace vkhip

extern "C" int vkhip_set_profiling(int enabled) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::obs().profiling.store(enabled != 0, std::memory_order_relaxed);
    return VKHIP_OK;
}

extern "C" int vkhip_profile_read(vkhip_profile_record* out, size_t capacity, size_t* count,
                                  uint64_t* dropped) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (!count || (capacity > 0 && !out)) return fail(VKHIP_ERR_INVALID, "profile_read: null output");
    vkhip::Observe& o = vkhip::obs();
    std::lock_guard<std::mutex> lk(o.mu);
    size_t n = 0;
    while (n < capacity && !o.pending.empty()) {
        vkhip::Pending& p = o.pending.front();
        VKHIP_HIP(hipEventSynchronize(p.end));
        float ms = 0.0f;
        VKHIP_HIP(hipEventElapsedTime(&ms, p.start, p.end));
        memcpy(out[n].label, p.label, sizeof out[n].label);
        out[n].gpu_ms = ms;
        out[n].dispatch = p.dispatch;
        o.free_events.push_back(p.start);
        o.free_events.push_back(p.end);
        o.pending.pop_front();
        ++n;
    }
    *count = n;
    if (dropped) *dropped = o.dropped;
    o.dropped = 0;
    return VKHIP_OK;
}
