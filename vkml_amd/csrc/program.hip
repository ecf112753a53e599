// Recorded programs: a training step's device calls, recorded once while the
// step runs and re-enqueued for every later step whose graph repeats.
//
// The reference measured the same idea for its Vulkan submission path ("record
// once, re-submit the same buffer", docs/adr/0012-asynchronous-submission.md
// section 2) and names the host cost it removes (docs/SMALL-STEP-LATENCY.md:
// 44-51: the MLP step is ~200x its arithmetic floor, the difference being
// per-node host work). Here the host core in Python builds and packs a few
// hundred node records per step; a program keeps the packed records of the
// recorded step and replays them from C, so a repeated step costs one call.
//
// Recording captures the three calls that enqueue work on tensors:
// vkhip_compute (the node span of a flush, byte for byte), vkhip_sgd_step and
// vkhip_copy_device_to_device. Host copies are not recorded: a replaying host
// uploads its new inputs into the recorded input buffers first. Every pointer
// is replayed as recorded, so the host keeps every buffer a program touches
// alive and unmoved for the program's life. The split-K and reduction
// workspaces are looked up per call, as they are in eager work.
//
// A replayed SGD step continues from the velocity the recorded step left:
// the "first step" flag of each parameter (velocity = gradient) is recorded
// as 0.
//
// With use_graph, the first run captures the replayed launches into a HIP
// graph on the backend stream and later runs launch that graph: one call per
// step instead of one per kernel. While a graph exists the backend keeps the
// workspace blocks it captured (a workspace that grows later gets a new block;
// the captured one is freed when the last graph is destroyed).
#include <cstring>
#include <memory>
#include <mutex>
#include <vector>

#include "common.h"

namespace vkhip {

int launch_sgd_step(const vkhip_sgd_param* params, size_t count, float lr, float momentum,
                    float weight_decay, int nesterov);

}  // namespace vkhip

struct vkhip_program {
    enum Kind { kCompute, kSgd, kCopy };
    struct Call {
        Kind kind;
        std::vector<vkhip_node> nodes;
        std::vector<vkhip_sgd_param> sgd;
        std::vector<vkhip_copy> copies;
        float lr = 0.0f, momentum = 0.0f, weight_decay = 0.0f;
        int nesterov = 0;
    };
    std::vector<Call> calls;
    size_t node_count = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    hipStream_t graph_stream = nullptr;
    // Early outputs: the declared device spans are copied into `out_host`
    // (pinned, device-visible at `out_dev`) behind calls[out_after - 1] of each
    // plain run, and `out_event` is recorded there.
    std::vector<vkhip_copy> outputs;
    void* out_host = nullptr;
    void* out_dev = nullptr;
    size_t out_bytes = 0;
    size_t out_after = 0;
    hipEvent_t out_event = nullptr;
    bool out_ready = false;  // the latest run was a plain run that recorded out_event
    // Input bindings: each recorded pointer field that lies in a bound input
    // span, with its offset there; vkhip_program_bind_input rewrites them.
    struct Site {
        void** slot;
        uintptr_t offset;
    };
    struct Binding {
        uintptr_t recorded;
        size_t nbytes;
        std::vector<Site> sites;
    };
    std::vector<Binding> bindings;
};

namespace vkhip {

namespace {
std::mutex g_prog_mu;
vkhip_program* g_recording = nullptr;  // the program being recorded, if any
bool g_replaying = false;              // calls made by a replay are not recorded again
}  // namespace

bool program_recording() { return g_recording != nullptr && !g_replaying; }

void program_note_compute(const vkhip_node* nodes, size_t n) {
    std::lock_guard<std::mutex> lk(g_prog_mu);
    if (!g_recording || g_replaying || n == 0) return;
    vkhip_program::Call c;
    c.kind = vkhip_program::kCompute;
    c.nodes.assign(nodes, nodes + n);
    g_recording->node_count += n;
    g_recording->calls.push_back(std::move(c));
}

void program_note_sgd(const vkhip_sgd_param* params, size_t count, float lr, float momentum,
                      float weight_decay, int nesterov) {
    std::lock_guard<std::mutex> lk(g_prog_mu);
    if (!g_recording || g_replaying || count == 0) return;
    vkhip_program::Call c;
    c.kind = vkhip_program::kSgd;
    c.sgd.assign(params, params + count);
    for (vkhip_sgd_param& p : c.sgd) p.first = 0;
    c.lr = lr;
    c.momentum = momentum;
    c.weight_decay = weight_decay;
    c.nesterov = nesterov;
    g_recording->calls.push_back(std::move(c));
}

void program_note_copy(const vkhip_copy* copies, size_t n) {
    std::lock_guard<std::mutex> lk(g_prog_mu);
    if (!g_recording || g_replaying || n == 0) return;
    vkhip_program::Call c;
    c.kind = vkhip_program::kCopy;
    c.copies.assign(copies, copies + n);
    g_recording->calls.push_back(std::move(c));
}

int compute_nodes(const vkhip_node* nodes, size_t n);  // runtime.hip
int copy_pairs(const vkhip_copy* copies, size_t n);     // runtime.hip

static int replay(const vkhip_program& p, bool early_outputs) {
    for (size_t k = 0; k < p.calls.size(); ++k) {
        if (early_outputs && k == p.out_after) {
            int st = copy_pairs(p.outputs.data(), p.outputs.size());
            if (st != VKHIP_OK) return st;
            VKHIP_HIP(hipEventRecord(p.out_event, ctx().stream));
        }
        const vkhip_program::Call& c = p.calls[k];
        int st = VKHIP_OK;
        switch (c.kind) {
            case vkhip_program::kCompute: st = compute_nodes(c.nodes.data(), c.nodes.size()); break;
            case vkhip_program::kSgd:
                st = launch_sgd_step(c.sgd.data(), c.sgd.size(), c.lr, c.momentum, c.weight_decay,
                                     c.nesterov);
                break;
            case vkhip_program::kCopy: st = copy_pairs(c.copies.data(), c.copies.size()); break;
        }
        if (st != VKHIP_OK) return st;
    }
    if (early_outputs && p.out_after == p.calls.size()) {
        const int st = copy_pairs(p.outputs.data(), p.outputs.size());
        if (st != VKHIP_OK) return st;
        VKHIP_HIP(hipEventRecord(p.out_event, ctx().stream));
    }
    return VKHIP_OK;
}

struct ReplayScope {
    ReplayScope() {
        std::lock_guard<std::mutex> lk(g_prog_mu);
        g_replaying = true;
    }
    ~ReplayScope() {
        std::lock_guard<std::mutex> lk(g_prog_mu);
        g_replaying = false;
    }
};

}  // namespace vkhip

using vkhip::ctx;
using vkhip::fail;

extern "C" int vkhip_program_begin(void) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    std::lock_guard<std::mutex> lk(vkhip::g_prog_mu);
    if (vkhip::g_recording) return fail(VKHIP_ERR_INVALID, "program_begin: already recording");
    vkhip::g_recording = new (std::nothrow) vkhip_program();
    if (!vkhip::g_recording) return fail(VKHIP_ERR_OOM, "program_begin: out of host memory");
    return VKHIP_OK;
}

namespace vkhip {
namespace {

// Bytes [lo, hi) a tensor's elements occupy (strides may be negative or 0).
struct Span {
    uintptr_t lo, hi;
};

Span tensor_span(const vkhip_tensor& t) {
    const int64_t item = t.dtype == VKHIP_I64 ? 8 : t.dtype == VKHIP_BOOL ? 1 : t.dtype == VKHIP_F16 ? 2 : 4;
    int64_t lo = 0, hi = 0;
    for (int i = 0; i < t.ndim; ++i) {
        if (t.ne[i] <= 0) return {0, 0};
        const int64_t reach = (t.ne[i] - 1) * t.nb[i];
        if (reach < 0) lo += reach; else hi += reach;
    }
    const uintptr_t base = reinterpret_cast<uintptr_t>(t.data);
    return {base + static_cast<uintptr_t>(lo * item), base + static_cast<uintptr_t>((hi + 1) * item)};
}

bool overlaps(const Span& a, const Span& b) { return a.lo < b.hi && b.lo < a.hi; }

// Constant nodes (FULL, ARANGE: no sources, the value in their params) whose
// output no other recorded call writes keep the value the recording wrote,
// since a program holds every buffer it touches: replays leave them out (the
// seed and 1/count of a mean's gradient, say, one launch per step).
void drop_constant_nodes(vkhip_program& p) {
    std::vector<Span> writes;
    std::vector<size_t> own;  // per node, in call order: its output's index in writes
    for (const vkhip_program::Call& c : p.calls) {
        for (const vkhip_node& nd : c.nodes) {
            own.push_back(writes.size());
            writes.push_back(tensor_span(nd.out));
        }
        for (const vkhip_sgd_param& sp : c.sgd) {
            const uintptr_t pa = reinterpret_cast<uintptr_t>(sp.param), va = reinterpret_cast<uintptr_t>(sp.velocity);
            writes.push_back({pa, pa + sp.n * sizeof(float)});
            if (sp.velocity) writes.push_back({va, va + sp.n * sizeof(float)});
        }
        for (const vkhip_copy& cp : c.copies) {
            const uintptr_t d = reinterpret_cast<uintptr_t>(cp.dst);
            writes.push_back({d, d + cp.nbytes});
        }
    }
    size_t k = 0;
    for (vkhip_program::Call& c : p.calls) {
        std::vector<vkhip_node> kept;
        for (const vkhip_node& nd : c.nodes) {
            const size_t mine = own[k++];
            bool constant = (nd.op == VKHIP_OP_FULL || nd.op == VKHIP_OP_ARANGE) && nd.n_src == 0;
            const Span s = writes[mine];
            for (size_t w = 0; constant && w < writes.size(); ++w)
                if (w != mine && overlaps(s, writes[w])) constant = false;
            if (!constant) kept.push_back(nd);
        }
        p.node_count -= c.nodes.size() - kept.size();
        c.nodes.swap(kept);
    }
}

}  // namespace
}  // namespace vkhip

extern "C" int vkhip_program_end(vkhip_program** out) {
    if (!out) return fail(VKHIP_ERR_INVALID, "program_end: null output");
    std::lock_guard<std::mutex> lk(vkhip::g_prog_mu);
    *out = nullptr;
    if (!vkhip::g_recording) return fail(VKHIP_ERR_INVALID, "program_end: not recording");
    vkhip::drop_constant_nodes(*vkhip::g_recording);
    *out = vkhip::g_recording;
    vkhip::g_recording = nullptr;
    return VKHIP_OK;
}

extern "C" int vkhip_program_run(vkhip_program* p, int use_graph) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (!p) return fail(VKHIP_ERR_INVALID, "program_run: null program");
    if (vkhip::program_recording())
        return fail(VKHIP_ERR_INVALID, "program_run: cannot replay while recording");
    hipStream_t stream = ctx().stream;
    p->out_ready = false;
    if (p->exec) {
        if (stream != p->graph_stream)
            return fail(VKHIP_ERR_INVALID, "program_run: the backend stream changed since the graph was captured");
        VKHIP_HIP(hipGraphLaunch(p->exec, stream));
        return VKHIP_OK;
    }
    vkhip::ReplayScope scope;
    if (!(use_graph & 1)) {
        const bool early = !p->outputs.empty() && !(use_graph & 2);
        st = vkhip::replay(*p, early);
        p->out_ready = early && st == VKHIP_OK;
        return st;
    }
    // First graph run: capture the replayed launches, then launch the graph.
    // Profiling records events per unit of work, which a capture must not do.
    if (vkhip::profiling_on()) return vkhip::replay(*p, false);
    st = vkhip::pin_workspaces(+1);
    if (st != VKHIP_OK) return st;
    VKHIP_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
    st = vkhip::replay(*p, false);
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(stream, &graph);
    if (st != VKHIP_OK || e != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        (void)vkhip::pin_workspaces(-1);
        if (st != VKHIP_OK) return st;
        return fail(VKHIP_ERR_DEVICE, "program_run: graph capture failed: %s", hipGetErrorString(e));
    }
    hipGraphExec_t exec = nullptr;
    const hipError_t ie = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (ie != hipSuccess) {
        (void)hipGraphDestroy(graph);
        (void)vkhip::pin_workspaces(-1);
        return fail(VKHIP_ERR_DEVICE, "program_run: graph instantiation failed: %s", hipGetErrorString(ie));
    }
    p->graph = graph;
    p->exec = exec;
    p->graph_stream = stream;
    VKHIP_HIP(hipGraphLaunch(exec, stream));
    return VKHIP_OK;
}

extern "C" int vkhip_program_destroy(vkhip_program* p) {
    if (!p) return VKHIP_OK;
    int st = VKHIP_OK;
    if (p->exec) {
        // the graph may still be running: wait before its workspaces can go
        if (ctx().ready && hipStreamSynchronize(p->graph_stream) != hipSuccess)
            st = fail(VKHIP_ERR_DEVICE, "program_destroy: stream synchronisation failed");
        (void)hipGraphExecDestroy(p->exec);
        (void)hipGraphDestroy(p->graph);
        const int rc = vkhip::pin_workspaces(-1);
        if (st == VKHIP_OK) st = rc;
    }
    if (p->out_event) {
        // a plain run may still be copying into the pinned block
        if (ctx().ready && hipEventSynchronize(p->out_event) != hipSuccess && st == VKHIP_OK)
            st = fail(VKHIP_ERR_DEVICE, "program_destroy: output event synchronisation failed");
        (void)hipEventDestroy(p->out_event);
    }
    if (p->out_host) (void)hipHostFree(p->out_host);
    delete p;
    return st;
}

extern "C" int vkhip_program_info(const vkhip_program* p, size_t* calls, size_t* nodes,
                                  int* has_graph) {
    if (!p) return fail(VKHIP_ERR_INVALID, "program_info: null program");
    if (calls) *calls = p->calls.size();
    if (nodes) *nodes = p->node_count;
    if (has_graph) *has_graph = p->exec ? 1 : 0;
    return VKHIP_OK;
}

namespace vkhip {
namespace {

// A recorded unit (one node, one SGD call or one copy call) with the byte
// spans it reads and writes.
struct RecordedUnit {
    vkhip_program::Call call;
    std::vector<Span> reads, writes;
};

bool any_overlap(const std::vector<Span>& a, const std::vector<Span>& b) {
    for (const Span& x : a)
        for (const Span& y : b)
            if (overlaps(x, y)) return true;
    return false;
}

// Two units may trade places unless one writes bytes the other reads or writes.
bool hazard(const RecordedUnit& a, const RecordedUnit& b) {
    return any_overlap(a.writes, b.reads) || any_overlap(a.writes, b.writes) || any_overlap(a.reads, b.writes);
}

std::vector<RecordedUnit> units_of(const vkhip_program& p) {
    std::vector<RecordedUnit> units;
    for (const vkhip_program::Call& c : p.calls) {
        if (c.kind == vkhip_program::kCompute) {
            for (const vkhip_node& nd : c.nodes) {
                RecordedUnit u;
                u.call.kind = vkhip_program::kCompute;
                u.call.nodes.push_back(nd);
                for (int i = 0; i < nd.n_src && i < 3; ++i) u.reads.push_back(tensor_span(nd.src[i]));
                u.writes.push_back(tensor_span(nd.out));
                units.push_back(std::move(u));
            }
            continue;
        }
        RecordedUnit u;
        u.call = c;
        for (const vkhip_sgd_param& sp : c.sgd) {
            const uintptr_t pa = reinterpret_cast<uintptr_t>(sp.param), ga = reinterpret_cast<uintptr_t>(sp.grad),
                            va = reinterpret_cast<uintptr_t>(sp.velocity), nb = sp.n * sizeof(float);
            u.reads.push_back({ga, ga + nb});
            u.writes.push_back({pa, pa + nb});
            if (sp.velocity) u.writes.push_back({va, va + nb});
        }
        for (const vkhip_copy& cp : c.copies) {
            const uintptr_t d = reinterpret_cast<uintptr_t>(cp.dst), sa = reinterpret_cast<uintptr_t>(cp.src);
            u.reads.push_back({sa, sa + cp.nbytes});
            u.writes.push_back({d, d + cp.nbytes});
        }
        units.push_back(std::move(u));
    }
    return units;
}

// The order in which `units` run when each unit the outputs depend on moves
// ahead of the later-recorded units it has no hazard with, keeping the order
// among those units: `order[i]` is the recorded index of the i-th unit to
// run. Returns one past the position of the last unit that writes an output
// (0 when none does): the outputs are final behind that many units.
size_t output_order(const std::vector<RecordedUnit>& units, const std::vector<Span>& outs, std::vector<size_t>& order) {
    const size_t n = units.size();
    // The dependence cone: walking back from the end, a unit that writes bytes
    // the outputs (or a unit already in the cone) read joins it.
    std::vector<char> cone(n, 0);
    std::vector<Span> needed = outs;
    for (size_t i = n; i-- > 0;) {
        if (!any_overlap(units[i].writes, needed)) continue;
        cone[i] = 1;
        needed.insert(needed.end(), units[i].reads.begin(), units[i].reads.end());
    }
    order.resize(n);
    for (size_t i = 0; i < n; ++i) order[i] = i;
    for (size_t i = 0; i < n; ++i) {
        if (!cone[order[i]]) continue;
        size_t j = i;
        while (j > 0 && !cone[order[j - 1]] && !hazard(units[order[j - 1]], units[order[j]])) {
            std::swap(order[j - 1], order[j]);
            --j;
        }
    }
    size_t last = 0;
    for (size_t i = 0; i < n; ++i)
        if (any_overlap(units[order[i]].writes, outs)) last = i + 1;
    return last;
}

// Reorders the program's units by output_order and regroups consecutive
// nodes into compute calls, ending a call at the last unit that writes an
// output. Returns the number of calls up to and including that unit.
size_t hoist_outputs(vkhip_program& p, const std::vector<Span>& outs) {
    std::vector<RecordedUnit> units = units_of(p);
    std::vector<size_t> order;
    const size_t last = output_order(units, outs, order);
    std::vector<vkhip_program::Call> calls;
    size_t after = 0;
    for (size_t i = 0; i < order.size(); ++i) {
        RecordedUnit& u = units[order[i]];
        const bool join = u.call.kind == vkhip_program::kCompute && !calls.empty() &&
                          calls.back().kind == vkhip_program::kCompute && i != last;
        if (join)
            calls.back().nodes.push_back(u.call.nodes[0]);
        else
            calls.push_back(std::move(u.call));
        if (i + 1 == last) after = calls.size();
    }
    p.calls.swap(calls);
    return after;
}

}  // namespace
}  // namespace vkhip

extern "C" int vkhip_program_set_outputs(vkhip_program* p, const vkhip_copy* outputs, size_t n) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (!p || (n && !outputs)) return fail(VKHIP_ERR_INVALID, "program_set_outputs: null argument");
    if (!p->outputs.empty()) return fail(VKHIP_ERR_INVALID, "program_set_outputs: outputs already declared");
    if (!p->bindings.empty()) return fail(VKHIP_ERR_INVALID, "program_set_outputs: inputs already bound");
    if (p->exec) return fail(VKHIP_ERR_INVALID, "program_set_outputs: the program has a captured graph");
    if (n == 0) return VKHIP_OK;
    constexpr size_t kMaxOutputBytes = 4096;
    size_t total = 0;
    std::vector<vkhip::Span> spans;
    for (size_t i = 0; i < n; ++i) {
        if (!outputs[i].src || outputs[i].nbytes == 0)
            return fail(VKHIP_ERR_INVALID, "program_set_outputs: output %zu is empty", i);
        total += outputs[i].nbytes;
        const uintptr_t a = reinterpret_cast<uintptr_t>(outputs[i].src);
        spans.push_back({a, a + outputs[i].nbytes});
    }
    if (total > kMaxOutputBytes)
        return fail(VKHIP_ERR_INVALID, "program_set_outputs: %zu bytes of outputs (at most %zu)", total,
                    kMaxOutputBytes);
    void* host = nullptr;
    void* dev = nullptr;
    if (hipHostMalloc(&host, total, hipHostMallocDefault) != hipSuccess || !host)
        return fail(VKHIP_ERR_OOM, "program_set_outputs: %zu bytes of pinned memory", total);
    hipEvent_t ev = nullptr;
    if (hipHostGetDevicePointer(&dev, host, 0) != hipSuccess ||
        hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
        (void)hipHostFree(host);
        return fail(VKHIP_ERR_DEVICE, "program_set_outputs: pinned block or event could not be set up");
    }
    std::lock_guard<std::mutex> lk(vkhip::g_prog_mu);
    p->out_after = vkhip::hoist_outputs(*p, spans);
    size_t off = 0;
    for (size_t i = 0; i < n; ++i) {
        vkhip_copy c = outputs[i];
        c.dst = static_cast<unsigned char*>(dev) + off;
        off += c.nbytes;
        p->outputs.push_back(c);
    }
    p->out_host = host;
    p->out_dev = dev;
    p->out_bytes = total;
    p->out_event = ev;
    p->out_ready = false;
    return VKHIP_OK;
}

extern "C" int vkhip_program_read_outputs(vkhip_program* p, void* host_dst, size_t nbytes) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (!p || !host_dst) return fail(VKHIP_ERR_INVALID, "program_read_outputs: null argument");
    if (p->outputs.empty() || !p->out_ready)
        return fail(VKHIP_ERR_INVALID, "program_read_outputs: no plain run with declared outputs");
    if (nbytes != p->out_bytes)
        return fail(VKHIP_ERR_INVALID, "program_read_outputs: %zu bytes asked, the outputs hold %zu", nbytes,
                    p->out_bytes);
    VKHIP_HIP(hipEventSynchronize(p->out_event));
    memcpy(host_dst, p->out_host, nbytes);
    return VKHIP_OK;
}

extern "C" int vkhip_program_output_order(const vkhip_node* nodes, size_t n, const vkhip_copy* outputs,
                                          size_t n_outputs, size_t* order, size_t* out_after) {
    if ((n && (!nodes || !order)) || (n_outputs && !outputs) || !out_after)
        return fail(VKHIP_ERR_INVALID, "program_output_order: null argument");
    std::vector<vkhip::RecordedUnit> units;
    for (size_t i = 0; i < n; ++i) {
        vkhip::RecordedUnit u;
        u.call.kind = vkhip_program::kCompute;
        u.call.nodes.push_back(nodes[i]);
        for (int k = 0; k < nodes[i].n_src && k < 3; ++k) u.reads.push_back(vkhip::tensor_span(nodes[i].src[k]));
        u.writes.push_back(vkhip::tensor_span(nodes[i].out));
        units.push_back(std::move(u));
    }
    std::vector<vkhip::Span> spans;
    for (size_t i = 0; i < n_outputs; ++i) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(outputs[i].src);
        spans.push_back({a, a + outputs[i].nbytes});
    }
    std::vector<size_t> ord;
    *out_after = vkhip::output_order(units, spans, ord);
    for (size_t i = 0; i < n; ++i) order[i] = ord[i];
    return VKHIP_OK;
}

extern "C" int vkhip_program_bind_input(vkhip_program* p, const void* recorded, const void* now, size_t nbytes) {
    if (!p || !recorded || !now || nbytes == 0) return fail(VKHIP_ERR_INVALID, "program_bind_input: null argument");
    if (p->exec) return fail(VKHIP_ERR_INVALID, "program_bind_input: the program has a captured graph");
    const uintptr_t r = reinterpret_cast<uintptr_t>(recorded);
    vkhip_program::Binding* b = nullptr;
    for (vkhip_program::Binding& x : p->bindings) {
        if (x.recorded == r && x.nbytes == nbytes) b = &x;
        else if (x.recorded < r + nbytes && r < x.recorded + x.nbytes)
            return fail(VKHIP_ERR_INVALID, "program_bind_input: span overlaps another bound input");
    }
    if (!b) {
        // First binding of this span: find every pointer field inside it.
        // A span some recorded call writes is not an input: refused.
        vkhip_program::Binding nb;
        nb.recorded = r;
        nb.nbytes = nbytes;
        bool written = false;
        auto note = [&](void** slot, bool write) {
            const uintptr_t a = reinterpret_cast<uintptr_t>(*slot);
            if (a < r || a >= r + nbytes) return;
            nb.sites.push_back({slot, a - r});
            written = written || write;
        };
        for (vkhip_program::Call& c : p->calls) {
            for (vkhip_node& nd : c.nodes) {
                note(&nd.out.data, true);
                for (int i = 0; i < nd.n_src && i < 3; ++i) note(&nd.src[i].data, false);
            }
            for (vkhip_sgd_param& sp : c.sgd) {
                note(reinterpret_cast<void**>(&sp.param), true);
                note(reinterpret_cast<void**>(const_cast<float**>(&sp.grad)), false);
                note(reinterpret_cast<void**>(&sp.velocity), true);
            }
            for (vkhip_copy& cp : c.copies) {
                note(&cp.dst, true);
                note(const_cast<void**>(&cp.src), false);
            }
        }
        if (written) return fail(VKHIP_ERR_INVALID, "program_bind_input: a recorded call writes the span");
        p->bindings.push_back(std::move(nb));
        b = &p->bindings.back();
    }
    const uintptr_t base = reinterpret_cast<uintptr_t>(now);
    for (const vkhip_program::Site& site : b->sites) *site.slot = reinterpret_cast<void*>(base + site.offset);
    return VKHIP_OK;
}
