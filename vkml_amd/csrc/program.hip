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

static int replay(const vkhip_program& p) {
    for (const vkhip_program::Call& c : p.calls) {
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
    if (p->exec) {
        if (stream != p->graph_stream)
            return fail(VKHIP_ERR_INVALID, "program_run: the backend stream changed since the graph was captured");
        VKHIP_HIP(hipGraphLaunch(p->exec, stream));
        return VKHIP_OK;
    }
    vkhip::ReplayScope scope;
    if (!use_graph) return vkhip::replay(*p);
    // First graph run: capture the replayed launches, then launch the graph.
    // Profiling records events per unit of work, which a capture must not do.
    if (vkhip::profiling_on()) return vkhip::replay(*p);
    st = vkhip::pin_workspaces(+1);
    if (st != VKHIP_OK) return st;
    VKHIP_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
    st = vkhip::replay(*p);
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
