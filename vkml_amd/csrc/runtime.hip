// Backend runtime: device binding, stream, memory, copies, and the
// compute(span<Node*>) dispatcher that turns one graph flush into an ordered
// launch sequence on one HIP stream.
//
// Mirrors the reference Backend contract (include/vkml/backend/api/backend.h:34-125):
// compute() orders work and may return before it completes; host reads
// synchronise; frees are stream-ordered so memory still read by enqueued work
// is not reused early (the reference retires frees behind its timeline,
// vulkan_backend.cpp:921-984; hipFreeAsync gives that ordering directly).
#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>

#include "common.h"

namespace vkhip {

// Launchers defined in the kernel translation units (gemm() in common.h).
int launch_im2col(const float* src, const vkhip_operand& sd, float* dst, const vkhip_unfold& p);
int launch_col2im(const float* cols, float* dst, uint32_t n, uint32_t channels,
                  const vkhip_unfold& p);
int conv2d_forward(const float* x, const vkhip_operand& xd, const float* w,
                   const vkhip_operand& wd, float* out, const vkhip_unfold& p, const float* bias,
                   int64_t bias_stride, bool relu);
int conv2d_weight_grad(const float* x, const vkhip_operand& xd, const float* gr,
                       const vkhip_operand& gd, float* out, const vkhip_unfold& p);
int conv2d_weight_grad_sum(const float* x, const vkhip_operand& xd, const float* gr,
                           const vkhip_operand& gd, float* out, const vkhip_unfold& p);
int launch_max_pool2x2_backward_relu_sums(const float* grad, const float* src, const vkhip_operand& sd,
                                          float* dst, float* bias_out);
int conv2d_pool_weight_bias_grad(const float* x, const vkhip_operand& xd, const float* y, const vkhip_operand& yd,
                                 const float* gp, const vkhip_operand& gpd, float* out, const vkhip_unfold& p);
int conv2d_input_grad(const float* gr, const vkhip_operand& gd, const float* w, int64_t w_row,
                      uint32_t channels, float* out, const vkhip_unfold& p);
int launch_cross_entropy(const float* logits, int64_t row_stride, const int64_t* labels,
                         const float* g_out, float* out, uint32_t rows, uint32_t n, int backward);
int launch_max_pool2d(const float* src, const vkhip_operand& sd, float* dst, uint32_t out_h,
                      uint32_t out_w, const vkhip_unfold& p);
int launch_max_pool2d_backward(const float* grad, const float* src, const vkhip_operand& sd,
                               float* dst, uint32_t out_h, uint32_t out_w, const vkhip_unfold& p,
                               bool relu);
int launch_softmax(const float* src, const vkhip_operand& d, float* dst, int axis, int log_mode);
int launch_reduce(int op, const float* src, const vkhip_operand& d, uint32_t mask, void* dst);
int launch_elementwise(const vkhip_node& nd);
int launch_copy_bytes(void* dst, const void* src, size_t nbytes);
int launch_copy_pairs(const vkhip_copy* copies, size_t n);

static thread_local char g_last_error[512] = "";

void set_error_msg(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
}

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
    return code;
}

Context& ctx() {
    static Context c;
    return c;
}

static std::mutex g_mu;  // guards init/shutdown/workspace (reference allocation-map mutex)

// ---- fixed scratch of the allocation-free GEMM entry point ----------------------
// vkhip_gemm_noalloc keeps its split-K partials here instead of in the grown
// workspace. Every GPU the library runs on holds its own copy of this array
// until the process ends, at its own address. In host code `scratch` is a
// host-side stand-in, not a device address: its device address comes from
// hipGetSymbolAddress, once per device at vkhip_init with that device current,
// and only that address is handed to kernels. Nothing here needs to start at
// zero: every partition writes its whole slice before the fold reads it.
constexpr size_t kScratchBytes = VKHIP_GEMM_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxScratchDevices = 64;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];
static float* g_scratch_ptr[kMaxScratchDevices] = {};

static int resolve_scratch(int device) {
    if (device < 0 || device >= kMaxScratchDevices) return VKHIP_OK;  // entry point unavailable
    if (g_scratch_ptr[device]) return VKHIP_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return fail(VKHIP_ERR_DEVICE, "hipGetSymbolAddress(scratch) on device %d failed: %s", device,
                    hipGetErrorString(e));
    g_scratch_ptr[device] = static_cast<float*>(p);
    return VKHIP_OK;
}
static int release_stage_slots();  // pinned upload/download slots, below

int require_ready() {
    if (!ctx().ready)
        return fail(VKHIP_ERR_NOT_INITIALISED, "vkhip: backend not initialised (call vkhip_init)");
    return VKHIP_OK;
}

int workspace(size_t bytes, float** out, int slot) {
    std::lock_guard<std::mutex> lk(g_mu);
    Context& c = ctx();
    if (slot < 0 || slot > 2) return fail(VKHIP_ERR_INVALID, "workspace: slot %d", slot);
    if (c.ws_bytes[slot] < bytes) {
        if (c.ws[slot] && c.ws_pins > 0) {
            // a captured graph still addresses this block: keep it
            if (c.ws_retired_count == static_cast<int>(sizeof c.ws_retired / sizeof c.ws_retired[0]))
                return fail(VKHIP_ERR_UNSUPPORTED,
                            "workspace: too many blocks held by captured graphs (destroy some programs)");
            c.ws_retired[c.ws_retired_count++] = c.ws[slot];
        } else if (c.ws[slot]) {
            VKHIP_HIP(hipFreeAsync(c.ws[slot], c.stream));
        }
        c.ws[slot] = nullptr;
        c.ws_bytes[slot] = 0;
        void* p = nullptr;
        if (hipMallocAsync(&p, bytes, c.stream) != hipSuccess)
            return fail(VKHIP_ERR_OOM, "workspace of %zu bytes could not be allocated", bytes);
        c.ws[slot] = static_cast<float*>(p);
        c.ws_bytes[slot] = bytes;
    }
    *out = c.ws[slot];
    return VKHIP_OK;
}

int pin_workspaces(int delta) {
    std::lock_guard<std::mutex> lk(g_mu);
    Context& c = ctx();
    c.ws_pins += delta;
    if (c.ws_pins < 0) c.ws_pins = 0;
    if (c.ws_pins == 0 && c.ws_retired_count > 0) {
        for (int i = 0; i < c.ws_retired_count; ++i)
            if (c.ready) VKHIP_HIP(hipFreeAsync(c.ws_retired[i], c.stream));
        c.ws_retired_count = 0;
    }
    return VKHIP_OK;
}

bool workspaces_pinned() {
    std::lock_guard<std::mutex> lk(g_mu);
    return ctx().ws_pins > 0;
}

// ---- node -> descriptor helpers ------------------------------------------------

static vkhip_operand to_operand(const vkhip_tensor& t) {
    vkhip_operand d;
    const int pad = 4 - t.ndim;
    for (int i = 0; i < 4; ++i) {
        d.ne[i] = 1;
        d.nb[i] = 0;
    }
    for (int i = 0; i < t.ndim; ++i) {
        d.ne[pad + i] = static_cast<uint32_t>(t.ne[i]);
        d.nb[pad + i] = t.nb[i];
    }
    return d;
}

static bool contiguous(const vkhip_tensor& t) {
    int64_t expect = 1;
    for (int i = t.ndim - 1; i >= 0; --i) {
        if (t.ne[i] == 1) continue;
        if (t.nb[i] != expect) return false;
        expect *= t.ne[i];
    }
    return true;
}

static bool fits32(const vkhip_tensor& t) {
    if (t.ndim < 0 || t.ndim > 4) return false;
    for (int i = 0; i < t.ndim; ++i)
        if (t.ne[i] < 0 || t.ne[i] > 0xffffffffll) return false;
    return true;
}

static bool is_f32(const vkhip_tensor& t) { return t.dtype == VKHIP_F32; }

// Elementwise nodes write a contiguous output and read sources already
// broadcast to its extents (stride 0 on broadcast axes), as the reference's
// executor hands them over.
static bool elementwise_layout(const vkhip_node& nd) {
    if (!contiguous(nd.out)) return false;
    for (int s = 0; s < nd.n_src; ++s) {
        if (nd.src[s].ndim != nd.out.ndim) return false;
        for (int i = 0; i < nd.out.ndim; ++i)
            if (nd.src[s].ne[i] != nd.out.ne[i]) return false;
    }
    return true;
}

static bool is_elementwise(int op) {
    switch (op) {
        case VKHIP_OP_FULL: case VKHIP_OP_ARANGE: case VKHIP_OP_CONTIGUOUS: case VKHIP_OP_CAST:
        case VKHIP_OP_NEG: case VKHIP_OP_EXP: case VKHIP_OP_LOG: case VKHIP_OP_RELU:
        case VKHIP_OP_ADD: case VKHIP_OP_SUB: case VKHIP_OP_MUL: case VKHIP_OP_DIV:
        case VKHIP_OP_ADD_RELU:
        case VKHIP_OP_SCALED_ADD: case VKHIP_OP_MAXIMUM: case VKHIP_OP_MINIMUM:
        case VKHIP_OP_EQUAL: case VKHIP_OP_LESS: case VKHIP_OP_GREATER: case VKHIP_OP_LESS_EQUAL:
        case VKHIP_OP_GREATER_EQUAL: case VKHIP_OP_NOT_EQUAL: case VKHIP_OP_WHERE:
        case VKHIP_OP_RELU_BACKWARD:
            return true;
        default: return false;
    }
}

static int supports_node(const vkhip_node& nd) {
    if (!fits32(nd.out)) return 0;
    if (nd.n_src < 0 || nd.n_src > 3) return 0;
    for (int s = 0; s < nd.n_src; ++s)
        if (!fits32(nd.src[s])) return 0;
    if (is_elementwise(nd.op) && !elementwise_layout(nd)) return 0;
    const vkhip_tensor& o = nd.out;
    switch (nd.op) {
        case VKHIP_OP_FULL:
            return o.dtype == VKHIP_F32 || o.dtype == VKHIP_I64 || o.dtype == VKHIP_BOOL;
        case VKHIP_OP_ARANGE: return o.dtype == VKHIP_F32 || o.dtype == VKHIP_I64;
        case VKHIP_OP_CONTIGUOUS:
            return nd.n_src == 1 && nd.src[0].dtype == o.dtype &&
                   (o.dtype == VKHIP_F32 || o.dtype == VKHIP_I64 || o.dtype == VKHIP_BOOL);
        case VKHIP_OP_CAST: {
            const int f = nd.src[0].dtype, t = o.dtype;
            return nd.n_src == 1 && ((f == VKHIP_I64 && t == VKHIP_F32) ||
                                     (f == VKHIP_BOOL && t == VKHIP_F32) ||
                                     (f == VKHIP_F32 && t == VKHIP_I64) ||
                                     (f == VKHIP_F32 && t == VKHIP_F32));
        }
        case VKHIP_OP_NEG:
        case VKHIP_OP_EXP:
        case VKHIP_OP_LOG:
        case VKHIP_OP_RELU: return nd.n_src == 1 && is_f32(o) && is_f32(nd.src[0]);
        case VKHIP_OP_ADD:
        case VKHIP_OP_ADD_RELU:
        case VKHIP_OP_SUB:
        case VKHIP_OP_MUL:
        case VKHIP_OP_DIV:
        case VKHIP_OP_SCALED_ADD:
        case VKHIP_OP_MAXIMUM:
        case VKHIP_OP_MINIMUM:
        case VKHIP_OP_RELU_BACKWARD:
            return nd.n_src == 2 && is_f32(o) && is_f32(nd.src[0]) && is_f32(nd.src[1]);
        case VKHIP_OP_EQUAL:
        case VKHIP_OP_LESS:
        case VKHIP_OP_GREATER:
        case VKHIP_OP_LESS_EQUAL:
        case VKHIP_OP_GREATER_EQUAL:
        case VKHIP_OP_NOT_EQUAL:
            return nd.n_src == 2 && o.dtype == VKHIP_BOOL && is_f32(nd.src[0]) && is_f32(nd.src[1]);
        case VKHIP_OP_WHERE:
            return nd.n_src == 3 && nd.src[0].dtype == VKHIP_BOOL && is_f32(o) &&
                   is_f32(nd.src[1]) && is_f32(nd.src[2]);
        case VKHIP_OP_SUM:
        case VKHIP_OP_MEAN:
        case VKHIP_OP_MAX:
        case VKHIP_OP_MIN: return nd.n_src == 1 && is_f32(o) && is_f32(nd.src[0]) && contiguous(o);
        case VKHIP_OP_ARGMAX:
        case VKHIP_OP_ARGMIN:
            return nd.n_src == 1 && o.dtype == VKHIP_I64 && is_f32(nd.src[0]) && contiguous(o);
        case VKHIP_OP_MATMUL:
            return nd.n_src == 2 && is_f32(o) && is_f32(nd.src[0]) && is_f32(nd.src[1]) &&
                   contiguous(o) && nd.src[0].ndim >= 2 && nd.src[1].ndim >= 2;
        case VKHIP_OP_MATMUL_BIAS:
            return nd.n_src == 3 && is_f32(o) && is_f32(nd.src[0]) && is_f32(nd.src[1]) &&
                   is_f32(nd.src[2]) && contiguous(o) && nd.src[0].ndim >= 2 && nd.src[1].ndim >= 2 &&
                   o.ndim >= 2 && nd.src[2].ndim == 1 && nd.src[2].ne[0] == o.ne[o.ndim - 1];
        case VKHIP_OP_MATMUL_RELU_BACKWARD: {
            if (!(nd.n_src == 3 && is_f32(o) && is_f32(nd.src[0]) && is_f32(nd.src[1]) &&
                  is_f32(nd.src[2]) && contiguous(o) && contiguous(nd.src[2]) && nd.src[0].ndim >= 2 &&
                  nd.src[1].ndim >= 2 && o.ndim >= 2 && nd.src[2].ndim == o.ndim))
                return 0;
            for (int i = 0; i < o.ndim; ++i)
                if (nd.src[2].ne[i] != o.ne[i]) return 0;
            return 1;
        }
        case VKHIP_OP_SOFTMAX:
        case VKHIP_OP_LOG_SOFTMAX:
            return nd.n_src == 1 && is_f32(o) && is_f32(nd.src[0]) && contiguous(o) &&
                   nd.src[0].ndim >= 1;
        case VKHIP_OP_IM2COL:
            return nd.n_src == 1 && is_f32(o) && is_f32(nd.src[0]) && nd.src[0].ndim == 4 &&
                   o.ndim == 3 && contiguous(o);
        case VKHIP_OP_COL2IM:
            return nd.n_src == 1 && is_f32(o) && is_f32(nd.src[0]) && nd.src[0].ndim == 3 &&
                   contiguous(nd.src[0]) && o.ndim == 4 && contiguous(o);
        case VKHIP_OP_MAX_POOL2D:
            return nd.n_src == 1 && is_f32(o) && is_f32(nd.src[0]) && nd.src[0].ndim == 4 &&
                   o.ndim == 4 && contiguous(o);
        case VKHIP_OP_CONV2D:
        case VKHIP_OP_CONV2D_BIAS_RELU: {
            const vkhip_tensor& x = nd.src[0];
            const vkhip_tensor& w = nd.src[1];
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            if (nd.op == VKHIP_OP_CONV2D_BIAS_RELU) {
                // the bias: [Cout] or [Cout, 1, 1], any stride along channels
                const vkhip_tensor& b = nd.src[2];
                if (nd.n_src != 3 || !is_f32(b) || b.ndim < 1 || b.ne[0] != w.ne[0]) return 0;
                for (int i = 1; i < b.ndim; ++i)
                    if (b.ne[i] != 1) return 0;
            }
            if (nd.n_src != (nd.op == VKHIP_OP_CONV2D ? 2 : 3) || !is_f32(x) || !is_f32(w) || !is_f32(o) || x.ndim != 4 ||
                o.ndim != 4 || !contiguous(o) || o.ne[0] != x.ne[0] || o.ne[1] != w.ne[0] ||
                static_cast<int64_t>(p.kernel_h) * p.kernel_w > 63)
                return 0;
            if (w.ndim == 4)  // [Cout, C, kh, kw] whose last three axes merge into contiguous rows
                return w.ne[1] == x.ne[1] && w.nb[3] == 1 && w.nb[2] == w.ne[3] &&
                       w.nb[1] == w.ne[2] * w.nb[2];
            return w.ndim == 2 && w.nb[1] == 1;
        }
        case VKHIP_OP_CONV2D_WEIGHT_GRAD: {
            const vkhip_tensor& x = nd.src[0];
            const vkhip_tensor& gr = nd.src[1];
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            return nd.n_src == 2 && is_f32(x) && is_f32(gr) && is_f32(o) && x.ndim == 4 &&
                   gr.ndim == 4 && o.ndim == 3 && contiguous(o) && gr.ne[0] == x.ne[0] &&
                   o.ne[0] == x.ne[0] && o.ne[1] == gr.ne[1] && gr.nb[3] == 1 &&
                   gr.nb[2] == gr.ne[3] &&
                   static_cast<int64_t>(p.kernel_h) * p.kernel_w <= 63;
        }
        case VKHIP_OP_CONV2D_INPUT_GRAD: {
            const vkhip_tensor& gr = nd.src[0];
            const vkhip_tensor& w = nd.src[1];
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            if (nd.n_src != 2 || !is_f32(gr) || !is_f32(w) || !is_f32(o) || gr.ndim != 4 ||
                o.ndim != 4 || !contiguous(o) || o.ne[0] != gr.ne[0] || w.ne[0] != gr.ne[1] ||
                gr.nb[3] != 1 || gr.nb[2] != gr.ne[3] || o.ne[2] != p.image_h || o.ne[3] != p.image_w ||
                static_cast<int64_t>(p.kernel_h) * p.kernel_w > 63)
                return 0;
            if (w.ndim == 4)
                return w.ne[1] == o.ne[1] && w.ne[2] == p.kernel_h && w.ne[3] == p.kernel_w &&
                       w.nb[3] == 1 && w.nb[2] == w.ne[3] && w.nb[1] == w.ne[2] * w.nb[2];
            return w.ndim == 2 && w.nb[1] == 1 &&
                   w.ne[1] == o.ne[1] * static_cast<int64_t>(p.kernel_h) * p.kernel_w;
        }
        case VKHIP_OP_CONV2D_WEIGHT_GRAD_SUM: {
            const vkhip_tensor& x = nd.src[0];
            const vkhip_tensor& gr = nd.src[1];
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            return nd.n_src == 2 && is_f32(x) && is_f32(gr) && is_f32(o) && x.ndim == 4 &&
                   gr.ndim == 4 && o.ndim == 2 && contiguous(o) && gr.ne[0] == x.ne[0] &&
                   o.ne[0] == gr.ne[1] && gr.nb[3] == 1 && gr.nb[2] == gr.ne[3] &&
                   static_cast<int64_t>(p.kernel_h) * p.kernel_w <= 63;
        }
        case VKHIP_OP_CONV2D_POOL_WEIGHT_BIAS_GRAD: {
            const vkhip_tensor& x = nd.src[0];
            const vkhip_tensor& y = nd.src[1];
            const vkhip_tensor& gp = nd.src[2];
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            return nd.n_src == 3 && is_f32(x) && is_f32(y) && is_f32(gp) && is_f32(o) && x.ndim == 4 &&
                   y.ndim == 4 && gp.ndim == 4 && contiguous(y) && contiguous(gp) && o.ndim == 1 && contiguous(o) &&
                   static_cast<int64_t>(p.kernel_h) * p.kernel_w <= 63;
        }
        case VKHIP_OP_CROSS_ENTROPY:
        case VKHIP_OP_CROSS_ENTROPY_BACKWARD: {
            const vkhip_tensor& x = nd.src[0];
            const vkhip_tensor& y = nd.src[1];
            const bool back = nd.op == VKHIP_OP_CROSS_ENTROPY_BACKWARD;
            if (nd.n_src != (back ? 3 : 2) || !is_f32(x) || x.ndim != 2 || x.nb[1] != 1 ||
                x.ne[1] < 1 || x.ne[1] > 2048 || y.dtype != VKHIP_I64 || y.ndim != 1 ||
                y.ne[0] != x.ne[0] || !contiguous(y) || !is_f32(o) || !contiguous(o))
                return 0;
            if (back)
                return nd.src[2].ndim == 1 && nd.src[2].ne[0] == x.ne[0] && is_f32(nd.src[2]) &&
                       contiguous(nd.src[2]) && o.ndim == 2 && o.ne[0] == x.ne[0] &&
                       o.ne[1] == x.ne[1];
            return o.ndim == 1 && o.ne[0] == x.ne[0];
        }
        case VKHIP_OP_MAX_POOL2D_BACKWARD:
        case VKHIP_OP_MAX_POOL2D_BACKWARD_RELU:
            return nd.n_src == 2 && is_f32(o) && is_f32(nd.src[0]) && is_f32(nd.src[1]) &&
                   nd.src[0].ndim == 4 && contiguous(nd.src[0]) && nd.src[1].ndim == 4 &&
                   o.ndim == 4 && contiguous(o);
        case VKHIP_OP_MAX_POOL2D_BACKWARD_RELU_BIAS: {
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            return nd.n_src == 2 && is_f32(o) && is_f32(nd.src[0]) && is_f32(nd.src[1]) && nd.src[0].ndim == 4 &&
                   contiguous(nd.src[0]) && nd.src[1].ndim == 4 && contiguous(nd.src[1]) && o.ndim == 1 &&
                   contiguous(o) && p.kernel_h == 2 && p.kernel_w == 2 && p.stride_h == 2 && p.stride_w == 2 &&
                   p.pad_h == 0 && p.pad_w == 0 && p.dilation_h == 1 && p.dilation_w == 1;
        }
        default: return 0;
    }
}

static const char* op_name(int op);

static int64_t window_span(int64_t extent, int k, int s, int pad, int dil) {
    if (k <= 0 || s <= 0 || dil <= 0 || pad < 0) return -1;
    return (extent + 2LL * pad - (static_cast<int64_t>(dil) * (k - 1) + 1)) / s + 1;
}

static int64_t tensor_numel(const vkhip_tensor& t) {
    int64_t n = 1;
    for (int i = 0; i < t.ndim; ++i) n *= t.ne[i];
    return n;
}

// The extents a node's params and operands imply for its output (and, for
// col2im, its source). The kernels size their writes and reads from params
// and operand descriptors, so a node whose tensors disagree with them is
// refused here instead of reading or writing out of bounds. Returns VKHIP_OK
// or VKHIP_ERR_INVALID with the message set.
static int check_extents(const vkhip_node& nd) {
    const vkhip_tensor& o = nd.out;
    if (nd.n_src < 0 || nd.n_src > 3) return fail(VKHIP_ERR_INVALID, "node with %d sources", nd.n_src);
    if (!fits32(o)) return fail(VKHIP_ERR_INVALID, "%s: output rank or extents out of range", op_name(nd.op));
    for (int s = 0; s < nd.n_src; ++s)
        if (!fits32(nd.src[s]))
            return fail(VKHIP_ERR_INVALID, "%s: source %d rank or extents out of range", op_name(nd.op), s);
    switch (nd.op) {
        case VKHIP_OP_MATMUL:
        case VKHIP_OP_MATMUL_BIAS:
        case VKHIP_OP_MATMUL_RELU_BACKWARD: {
            if (nd.n_src != (nd.op == VKHIP_OP_MATMUL ? 2 : 3) || nd.src[0].ndim < 2 ||
                nd.src[1].ndim < 2 || o.ndim < 2)
                return fail(VKHIP_ERR_INVALID, "matmul: operands and output need rank >= 2");
            if (nd.op == VKHIP_OP_MATMUL_RELU_BACKWARD) {
                bool same = nd.src[2].ndim == o.ndim;
                for (int i = 0; same && i < o.ndim; ++i) same = nd.src[2].ne[i] == o.ne[i];
                if (!same)
                    return fail(VKHIP_ERR_INVALID, "matmul_relu_backward: the mask's extents differ from the output's");
            }
            if (nd.op == VKHIP_OP_MATMUL_BIAS &&
                (nd.src[2].ndim != 1 || nd.src[2].ne[0] != o.ne[o.ndim - 1]))
                return fail(VKHIP_ERR_INVALID, "matmul_bias: the bias needs one value per output column");
            const vkhip_operand a = to_operand(nd.src[0]), b = to_operand(nd.src[1]);
            const vkhip_operand c = to_operand(o);
            if (a.ne[3] != b.ne[2])
                return fail(VKHIP_ERR_INVALID, "matmul: inner extents %u and %u disagree", a.ne[3], b.ne[2]);
            const uint32_t want[4] = {std::max(a.ne[0], b.ne[0]), std::max(a.ne[1], b.ne[1]), a.ne[2],
                                      b.ne[3]};
            for (int i = 0; i < 4; ++i)
                if (c.ne[i] != want[i] || (i < 2 && ((a.ne[i] != 1 && a.ne[i] != want[i]) ||
                                                     (b.ne[i] != 1 && b.ne[i] != want[i]))))
                    return fail(VKHIP_ERR_INVALID,
                                "matmul: output [%u,%u,%u,%u] disagrees with the operands' [%u,%u,%u,%u]",
                                c.ne[0], c.ne[1], c.ne[2], c.ne[3], want[0], want[1], want[2], want[3]);
            return VKHIP_OK;
        }
        case VKHIP_OP_SOFTMAX:
        case VKHIP_OP_LOG_SOFTMAX:
            if (nd.n_src != 1 || o.ndim != nd.src[0].ndim)
                return fail(VKHIP_ERR_INVALID, "softmax: output rank differs from the source's");
            for (int i = 0; i < o.ndim; ++i)
                if (o.ne[i] != nd.src[0].ne[i])
                    return fail(VKHIP_ERR_INVALID, "softmax: output extents differ from the source's");
            return VKHIP_OK;
        case VKHIP_OP_SUM:
        case VKHIP_OP_MEAN:
        case VKHIP_OP_MAX:
        case VKHIP_OP_MIN:
        case VKHIP_OP_ARGMAX:
        case VKHIP_OP_ARGMIN: {
            if (nd.n_src != 1) return fail(VKHIP_ERR_INVALID, "reduction: one source expected");
            uint32_t mask;
            memcpy(&mask, nd.params, sizeof mask);
            const vkhip_tensor& s = nd.src[0];
            if (s.ndim < 0 || s.ndim > 4 || (mask >> std::max(s.ndim, 0)) != 0)
                return fail(VKHIP_ERR_INVALID, "reduction: axes mask 0x%x outside rank %d", mask, s.ndim);
            if (mask == 0) mask = s.ndim <= 0 ? 0u : (1u << s.ndim) - 1u;
            int64_t kept = 1;
            for (int i = 0; i < s.ndim; ++i)
                if (!((mask >> i) & 1u)) kept *= s.ne[i];
            if (tensor_numel(o) != kept)
                return fail(VKHIP_ERR_INVALID, "reduction: output holds %lld values, the kept axes give %lld",
                            static_cast<long long>(tensor_numel(o)), static_cast<long long>(kept));
            return VKHIP_OK;
        }
        case VKHIP_OP_IM2COL:
        case VKHIP_OP_COL2IM: {
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            const int64_t oh = window_span(p.image_h, p.kernel_h, p.stride_h, p.pad_h, p.dilation_h);
            const int64_t ow = window_span(p.image_w, p.kernel_w, p.stride_w, p.pad_w, p.dilation_w);
            if (oh <= 0 || ow <= 0 || p.image_h < 0 || p.image_w < 0)
                return fail(VKHIP_ERR_INVALID, "%s: invalid window geometry", op_name(nd.op));
            const bool fwd = nd.op == VKHIP_OP_IM2COL;
            const vkhip_tensor& img = fwd ? nd.src[0] : o;
            const vkhip_tensor& cols = fwd ? o : nd.src[0];
            if (nd.n_src != 1 || img.ndim != 4 || cols.ndim != 3)
                return fail(VKHIP_ERR_INVALID, "%s: image rank 4 and columns rank 3 expected", op_name(nd.op));
            const int64_t rows = img.ne[1] * static_cast<int64_t>(p.kernel_h) * p.kernel_w;
            if (img.ne[2] != p.image_h || img.ne[3] != p.image_w || cols.ne[0] != img.ne[0] ||
                cols.ne[1] != rows || cols.ne[2] != oh * ow)
                return fail(VKHIP_ERR_INVALID,
                            "%s: columns [%lld,%lld,%lld] and image [%lld,%lld,%lld,%lld] disagree with "
                            "the window geometry (want [%lld,%lld,%lld], image %dx%d)",
                            op_name(nd.op), static_cast<long long>(cols.ne[0]),
                            static_cast<long long>(cols.ne[1]), static_cast<long long>(cols.ne[2]),
                            static_cast<long long>(img.ne[0]), static_cast<long long>(img.ne[1]),
                            static_cast<long long>(img.ne[2]), static_cast<long long>(img.ne[3]),
                            static_cast<long long>(img.ne[0]), static_cast<long long>(rows),
                            static_cast<long long>(oh * ow), p.image_h, p.image_w);
            return VKHIP_OK;
        }
        case VKHIP_OP_MAX_POOL2D_BACKWARD_RELU_BIAS: {
            const vkhip_tensor& g = nd.src[0];
            const vkhip_tensor& y = nd.src[1];
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            if (nd.n_src != 2 || g.ndim != 4 || y.ndim != 4 || o.ndim != 1 || y.ne[2] != p.image_h ||
                y.ne[3] != p.image_w || y.ne[2] % 2 != 0 || y.ne[3] % 2 != 0 || g.ne[0] != y.ne[0] ||
                g.ne[1] != y.ne[1] || g.ne[2] != y.ne[2] / 2 || g.ne[3] != y.ne[3] / 2 ||
                o.ne[0] != y.ne[0] * y.ne[1] * y.ne[2] * y.ne[3] + y.ne[1])
                return fail(VKHIP_ERR_INVALID,
                            "max_pool2d_backward_relu_bias: gradient, pool input and output extents disagree "
                            "with 2x2 windows at stride 2 over even extents");
            return VKHIP_OK;
        }
        case VKHIP_OP_CONV2D_POOL_WEIGHT_BIAS_GRAD: {
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            const int64_t oh = window_span(p.image_h, p.kernel_h, p.stride_h, p.pad_h, p.dilation_h);
            const int64_t ow = window_span(p.image_w, p.kernel_w, p.stride_w, p.pad_w, p.dilation_w);
            const vkhip_tensor& x = nd.src[0];
            const vkhip_tensor& y = nd.src[1];
            const vkhip_tensor& gp = nd.src[2];
            if (nd.n_src != 3 || x.ndim != 4 || y.ndim != 4 || gp.ndim != 4 || o.ndim != 1 || oh <= 0 || ow <= 0 ||
                x.ne[2] != p.image_h || x.ne[3] != p.image_w || y.ne[0] != x.ne[0] || y.ne[2] != oh ||
                y.ne[3] != ow || gp.ne[0] != y.ne[0] || gp.ne[1] != y.ne[1] || gp.ne[2] != oh / 2 ||
                gp.ne[3] != ow / 2 ||
                o.ne[0] != y.ne[1] * (x.ne[1] * static_cast<int64_t>(p.kernel_h) * p.kernel_w + 1))
                return fail(VKHIP_ERR_INVALID,
                            "conv2d_pool_weight_bias_grad: image, layer output, pool gradient and output extents "
                            "disagree with the window geometry");
            return VKHIP_OK;
        }
        case VKHIP_OP_MAX_POOL2D: {
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            const int64_t oh = window_span(p.image_h, p.kernel_h, p.stride_h, p.pad_h, p.dilation_h);
            const int64_t ow = window_span(p.image_w, p.kernel_w, p.stride_w, p.pad_w, p.dilation_w);
            const vkhip_tensor& x = nd.src[0];
            if (nd.n_src != 1 || x.ndim != 4 || o.ndim != 4 || oh <= 0 || ow <= 0 ||
                x.ne[2] != p.image_h || x.ne[3] != p.image_w || o.ne[0] != x.ne[0] ||
                o.ne[1] != x.ne[1] || o.ne[2] != oh || o.ne[3] != ow)
                return fail(VKHIP_ERR_INVALID, "max_pool2d: input/output extents disagree with the window geometry");
            return VKHIP_OK;
        }
        case VKHIP_OP_MAX_POOL2D_BACKWARD:
        case VKHIP_OP_MAX_POOL2D_BACKWARD_RELU: {
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            const int64_t oh = window_span(p.image_h, p.kernel_h, p.stride_h, p.pad_h, p.dilation_h);
            const int64_t ow = window_span(p.image_w, p.kernel_w, p.stride_w, p.pad_w, p.dilation_w);
            const vkhip_tensor& g = nd.src[0];
            const vkhip_tensor& x = nd.src[1];
            if (nd.n_src != 2 || g.ndim != 4 || x.ndim != 4 || o.ndim != 4 || oh <= 0 || ow <= 0 ||
                x.ne[2] != p.image_h || x.ne[3] != p.image_w || g.ne[0] != x.ne[0] ||
                g.ne[1] != x.ne[1] || g.ne[2] != oh || g.ne[3] != ow)
                return fail(VKHIP_ERR_INVALID,
                            "max_pool2d_backward: gradient/input extents disagree with the window geometry");
            for (int i = 0; i < 4; ++i)
                if (o.ne[i] != x.ne[i])
                    return fail(VKHIP_ERR_INVALID, "max_pool2d_backward: output shape differs from the input's");
            return VKHIP_OK;
        }
        default: return VKHIP_OK;  // elementwise (same extents: supports_node), conv, cross-entropy
    }
}

static const char* op_name(int op) {
    switch (op) {
        case VKHIP_OP_MATMUL: return "matmul";
        case VKHIP_OP_MATMUL_BIAS: return "matmul_bias";
        case VKHIP_OP_MATMUL_RELU_BACKWARD: return "matmul_relu_backward";
        case VKHIP_OP_SOFTMAX: return "softmax";
        case VKHIP_OP_LOG_SOFTMAX: return "log_softmax";
        case VKHIP_OP_IM2COL: return "im2col";
        case VKHIP_OP_COL2IM: return "col2im";
        case VKHIP_OP_SUM: return "sum";
        case VKHIP_OP_MEAN: return "mean";
        case VKHIP_OP_MAX: return "max";
        case VKHIP_OP_ARGMAX: return "argmax";
        case VKHIP_OP_MAX_POOL2D: return "max_pool2d";
        case VKHIP_OP_MAX_POOL2D_BACKWARD: return "max_pool2d_backward";
        case VKHIP_OP_MAX_POOL2D_BACKWARD_RELU: return "max_pool2d_backward_relu";
        case VKHIP_OP_CONV2D_POOL_WEIGHT_BIAS_GRAD: return "conv2d_pool_weight_bias_grad";
        case VKHIP_OP_MAX_POOL2D_BACKWARD_RELU_BIAS: return "max_pool2d_backward_relu_bias";
        case VKHIP_OP_CROSS_ENTROPY: return "cross_entropy";
        case VKHIP_OP_CROSS_ENTROPY_BACKWARD: return "cross_entropy_backward";
        case VKHIP_OP_CONV2D: return "conv2d";
        case VKHIP_OP_CONV2D_WEIGHT_GRAD: return "conv2d_weight_grad";
        case VKHIP_OP_CONV2D_WEIGHT_GRAD_SUM: return "conv2d_weight_grad_sum";
        case VKHIP_OP_CONV2D_INPUT_GRAD: return "conv2d_input_grad";
        case VKHIP_OP_CONV2D_BIAS_RELU: return "conv2d_bias_relu";
        case VKHIP_OP_MIN: return "min";
        case VKHIP_OP_ARGMIN: return "argmin";
        case VKHIP_OP_FULL: return "full";
        case VKHIP_OP_ARANGE: return "arange";
        case VKHIP_OP_CONTIGUOUS: return "contiguous";
        case VKHIP_OP_CAST: return "cast";
        case VKHIP_OP_NEG: return "neg";
        case VKHIP_OP_EXP: return "exp";
        case VKHIP_OP_LOG: return "log";
        case VKHIP_OP_RELU: return "relu";
        case VKHIP_OP_RELU_BACKWARD: return "relu_backward";
        case VKHIP_OP_ADD: return "add";
        case VKHIP_OP_ADD_RELU: return "add_relu";
        case VKHIP_OP_SUB: return "sub";
        case VKHIP_OP_MUL: return "mul";
        case VKHIP_OP_DIV: return "div";
        case VKHIP_OP_SCALED_ADD: return "scaled_add";
        case VKHIP_OP_MAXIMUM: return "maximum";
        case VKHIP_OP_MINIMUM: return "minimum";
        case VKHIP_OP_EQUAL: return "equal";
        case VKHIP_OP_LESS: return "less";
        case VKHIP_OP_GREATER: return "greater";
        case VKHIP_OP_LESS_EQUAL: return "less_equal";
        case VKHIP_OP_GREATER_EQUAL: return "greater_equal";
        case VKHIP_OP_NOT_EQUAL: return "not_equal";
        case VKHIP_OP_WHERE: return "where";
        default: return "op";
    }
}

static int compute_node(const vkhip_node& nd) {
    Unit unit(op_name(nd.op));
    {
        const int rc = check_extents(nd);
        if (rc != VKHIP_OK) return rc;
    }
    if (!supports_node(nd))
        return fail(VKHIP_ERR_UNSUPPORTED, "vkhip: %s (op %d) is not supported for these dtypes/layout",
                    op_name(nd.op), nd.op);
    switch (nd.op) {
        case VKHIP_OP_MATMUL:
        case VKHIP_OP_MATMUL_BIAS:
        case VKHIP_OP_MATMUL_RELU_BACKWARD: {
            const vkhip_operand a = to_operand(nd.src[0]);
            const vkhip_operand b = to_operand(nd.src[1]);
            const vkhip_gemm_opts opts{ctx().node_gemm_kernel, 0};
            GemmEpilogue epi{nullptr, 0, false};
            if (nd.op == VKHIP_OP_MATMUL_BIAS) {
                uint32_t relu;
                memcpy(&relu, nd.params, sizeof relu);
                epi = GemmEpilogue{static_cast<const float*>(nd.src[2].data), nd.src[2].nb[0], relu != 0};
            } else if (nd.op == VKHIP_OP_MATMUL_RELU_BACKWARD) {
                epi.mask = static_cast<const float*>(nd.src[2].data);
            }
            return gemm(static_cast<const float*>(nd.src[0].data), a,
                        static_cast<const float*>(nd.src[1].data), b,
                        static_cast<float*>(nd.out.data), &opts, nullptr,
                        nd.op == VKHIP_OP_MATMUL ? nullptr : &epi);
        }
        case VKHIP_OP_SUM:
        case VKHIP_OP_MEAN:
        case VKHIP_OP_MAX:
        case VKHIP_OP_MIN:
        case VKHIP_OP_ARGMAX:
        case VKHIP_OP_ARGMIN: {
            uint32_t mask;
            memcpy(&mask, nd.params, sizeof mask);
            const int ndim = nd.src[0].ndim;
            if (mask == 0) mask = ndim <= 0 ? 0u : (1u << ndim) - 1u;  // reduce-all
            static const int map[] = {VKHIP_REDUCE_SUM, VKHIP_REDUCE_MEAN, VKHIP_REDUCE_MAX,
                                      VKHIP_REDUCE_MIN, -1,                VKHIP_REDUCE_ARGMAX,
                                      VKHIP_REDUCE_ARGMIN};
            const vkhip_operand d = to_operand(nd.src[0]);
            return launch_reduce(map[nd.op - VKHIP_OP_SUM], static_cast<const float*>(nd.src[0].data),
                                 d, (mask << (4 - ndim)) & 0xfu, nd.out.data);
        }
        case VKHIP_OP_SOFTMAX:
        case VKHIP_OP_LOG_SOFTMAX: {
            int32_t axis;
            memcpy(&axis, nd.params, sizeof axis);
            const int ndim = nd.src[0].ndim;
            if (axis < 0) axis += ndim;
            if (axis < 0 || axis >= ndim) return fail(VKHIP_ERR_INVALID, "softmax: bad axis");
            return launch_softmax(static_cast<const float*>(nd.src[0].data), to_operand(nd.src[0]),
                                  static_cast<float*>(nd.out.data), axis + 4 - ndim,
                                  nd.op == VKHIP_OP_LOG_SOFTMAX);
        }
        case VKHIP_OP_IM2COL: {
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            return launch_im2col(static_cast<const float*>(nd.src[0].data), to_operand(nd.src[0]),
                                 static_cast<float*>(nd.out.data), p);
        }
        case VKHIP_OP_COL2IM: {
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            return launch_col2im(static_cast<const float*>(nd.src[0].data),
                                 static_cast<float*>(nd.out.data), static_cast<uint32_t>(nd.out.ne[0]),
                                 static_cast<uint32_t>(nd.out.ne[1]), p);
        }
        case VKHIP_OP_CONV2D:
        case VKHIP_OP_CONV2D_BIAS_RELU: {
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            const vkhip_tensor& w = nd.src[1];
            const int64_t ck = w.ndim == 4 ? w.ne[1] * w.ne[2] * w.ne[3] : w.ne[1];
            if (w.ndim == 4 && (w.ne[2] != p.kernel_h || w.ne[3] != p.kernel_w))
                return fail(VKHIP_ERR_INVALID, "conv2d: weight window %lldx%lld, params %dx%d",
                            static_cast<long long>(w.ne[2]), static_cast<long long>(w.ne[3]),
                            p.kernel_h, p.kernel_w);
            if (ck > 0xffffffffll) return fail(VKHIP_ERR_UNSUPPORTED, "conv2d: weight too large");
            vkhip_operand wd;
            wd.ne[0] = 1;
            wd.ne[1] = 1;
            wd.ne[2] = static_cast<uint32_t>(w.ne[0]);
            wd.ne[3] = static_cast<uint32_t>(ck);
            wd.nb[0] = 0;
            wd.nb[1] = 0;
            wd.nb[2] = w.nb[0];
            wd.nb[3] = w.ndim == 4 ? w.nb[3] : w.nb[1];
            const int64_t oh = (static_cast<int64_t>(p.image_h) + 2 * p.pad_h -
                                (static_cast<int64_t>(p.dilation_h) * (p.kernel_h - 1) + 1)) / std::max(p.stride_h, 1) + 1;
            const int64_t ow = (static_cast<int64_t>(p.image_w) + 2 * p.pad_w -
                                (static_cast<int64_t>(p.dilation_w) * (p.kernel_w - 1) + 1)) / std::max(p.stride_w, 1) + 1;
            if (nd.out.ne[2] != oh || nd.out.ne[3] != ow)
                return fail(VKHIP_ERR_INVALID, "conv2d: output %lldx%lld, geometry gives %lldx%lld",
                            static_cast<long long>(nd.out.ne[2]), static_cast<long long>(nd.out.ne[3]),
                            static_cast<long long>(oh), static_cast<long long>(ow));
            const bool fused = nd.op == VKHIP_OP_CONV2D_BIAS_RELU;
            return conv2d_forward(static_cast<const float*>(nd.src[0].data), to_operand(nd.src[0]),
                                  static_cast<const float*>(w.data), wd,
                                  static_cast<float*>(nd.out.data), p,
                                  fused ? static_cast<const float*>(nd.src[2].data) : nullptr,
                                  fused ? nd.src[2].nb[0] : 0, fused);
        }
        case VKHIP_OP_CONV2D_WEIGHT_GRAD: {
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            const vkhip_tensor& gr = nd.src[1];
            const int64_t L = gr.ne[2] * gr.ne[3];
            const int64_t ck = nd.src[0].ne[1] * static_cast<int64_t>(p.kernel_h) * p.kernel_w;
            if (nd.out.ne[2] != ck)
                return fail(VKHIP_ERR_INVALID, "conv2d weight grad: output has %lld columns, want %lld",
                            static_cast<long long>(nd.out.ne[2]), static_cast<long long>(ck));
            if (L > 0xffffffffll) return fail(VKHIP_ERR_UNSUPPORTED, "conv2d weight grad: too many positions");
            vkhip_operand gd;
            gd.ne[0] = 1;
            gd.ne[1] = static_cast<uint32_t>(gr.ne[0]);
            gd.ne[2] = static_cast<uint32_t>(gr.ne[1]);
            gd.ne[3] = static_cast<uint32_t>(L);
            gd.nb[0] = 0;
            gd.nb[1] = gr.nb[0];
            gd.nb[2] = gr.nb[1];
            gd.nb[3] = 1;
            return conv2d_weight_grad(static_cast<const float*>(nd.src[0].data), to_operand(nd.src[0]),
                                      static_cast<const float*>(gr.data), gd,
                                      static_cast<float*>(nd.out.data), p);
        }
        case VKHIP_OP_CONV2D_INPUT_GRAD: {
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            if (nd.out.ne[1] > 0xffffffffll || nd.src[0].ne[0] > 0xffffffffll || nd.src[0].ne[1] > 0xffffffffll)
                return fail(VKHIP_ERR_UNSUPPORTED, "conv2d input grad: extents too large");
            return conv2d_input_grad(static_cast<const float*>(nd.src[0].data), to_operand(nd.src[0]),
                                     static_cast<const float*>(nd.src[1].data), nd.src[1].nb[0],
                                     static_cast<uint32_t>(nd.out.ne[1]), static_cast<float*>(nd.out.data), p);
        }
        case VKHIP_OP_CONV2D_WEIGHT_GRAD_SUM: {
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            const vkhip_tensor& gr = nd.src[1];
            const int64_t L = gr.ne[2] * gr.ne[3];
            const int64_t ck = nd.src[0].ne[1] * static_cast<int64_t>(p.kernel_h) * p.kernel_w;
            if (nd.out.ne[1] != ck)
                return fail(VKHIP_ERR_INVALID, "conv2d weight grad sum: output has %lld columns, want %lld",
                            static_cast<long long>(nd.out.ne[1]), static_cast<long long>(ck));
            if (L > 0xffffffffll) return fail(VKHIP_ERR_UNSUPPORTED, "conv2d weight grad sum: too many positions");
            vkhip_operand gd;
            gd.ne[0] = 1;
            gd.ne[1] = static_cast<uint32_t>(gr.ne[0]);
            gd.ne[2] = static_cast<uint32_t>(gr.ne[1]);
            gd.ne[3] = static_cast<uint32_t>(L);
            gd.nb[0] = 0;
            gd.nb[1] = gr.nb[0];
            gd.nb[2] = gr.nb[1];
            gd.nb[3] = 1;
            return conv2d_weight_grad_sum(static_cast<const float*>(nd.src[0].data), to_operand(nd.src[0]),
                                          static_cast<const float*>(gr.data), gd,
                                          static_cast<float*>(nd.out.data), p);
        }
        case VKHIP_OP_MAX_POOL2D_BACKWARD_RELU_BIAS: {
            const vkhip_tensor& y = nd.src[1];
            float* out = static_cast<float*>(nd.out.data);
            return launch_max_pool2x2_backward_relu_sums(static_cast<const float*>(nd.src[0].data),
                                                         static_cast<const float*>(y.data), to_operand(y), out,
                                                         out + y.ne[0] * y.ne[1] * y.ne[2] * y.ne[3]);
        }
        case VKHIP_OP_CONV2D_POOL_WEIGHT_BIAS_GRAD: {
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            return conv2d_pool_weight_bias_grad(static_cast<const float*>(nd.src[0].data), to_operand(nd.src[0]),
                                                static_cast<const float*>(nd.src[1].data), to_operand(nd.src[1]),
                                                static_cast<const float*>(nd.src[2].data), to_operand(nd.src[2]),
                                                static_cast<float*>(nd.out.data), p);
        }
        case VKHIP_OP_CROSS_ENTROPY:
        case VKHIP_OP_CROSS_ENTROPY_BACKWARD: {
            const bool back = nd.op == VKHIP_OP_CROSS_ENTROPY_BACKWARD;
            return launch_cross_entropy(
                static_cast<const float*>(nd.src[0].data), nd.src[0].nb[0],
                static_cast<const int64_t*>(nd.src[1].data),
                back ? static_cast<const float*>(nd.src[2].data) : nullptr,
                static_cast<float*>(nd.out.data), static_cast<uint32_t>(nd.src[0].ne[0]),
                static_cast<uint32_t>(nd.src[0].ne[1]), back ? 1 : 0);
        }
        case VKHIP_OP_MAX_POOL2D: {
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            if (nd.out.ne[0] != nd.src[0].ne[0] || nd.out.ne[1] != nd.src[0].ne[1])
                return fail(VKHIP_ERR_INVALID, "max_pool2d: output planes disagree with the input's");
            return launch_max_pool2d(static_cast<const float*>(nd.src[0].data), to_operand(nd.src[0]),
                                     static_cast<float*>(nd.out.data),
                                     static_cast<uint32_t>(nd.out.ne[2]),
                                     static_cast<uint32_t>(nd.out.ne[3]), p);
        }
        case VKHIP_OP_MAX_POOL2D_BACKWARD:
        case VKHIP_OP_MAX_POOL2D_BACKWARD_RELU: {
            vkhip_unfold p;
            memcpy(&p, nd.params, sizeof p);
            for (int i = 0; i < 4; ++i)
                if (nd.out.ne[i] != nd.src[1].ne[i])
                    return fail(VKHIP_ERR_INVALID, "max_pool2d_backward: output shape differs from the input's");
            if (nd.src[0].ne[0] != nd.src[1].ne[0] || nd.src[0].ne[1] != nd.src[1].ne[1])
                return fail(VKHIP_ERR_INVALID, "max_pool2d_backward: gradient planes disagree with the input's");
            return launch_max_pool2d_backward(
                static_cast<const float*>(nd.src[0].data), static_cast<const float*>(nd.src[1].data),
                to_operand(nd.src[1]), static_cast<float*>(nd.out.data),
                static_cast<uint32_t>(nd.src[0].ne[2]), static_cast<uint32_t>(nd.src[0].ne[3]), p,
                nd.op == VKHIP_OP_MAX_POOL2D_BACKWARD_RELU);
        }
        default: return launch_elementwise(nd);
    }
}

}  // namespace vkhip

using vkhip::ctx;
using vkhip::fail;

// ---- lifecycle ---------------------------------------------------------------------

extern "C" int vkhip_init(int device) {
    std::lock_guard<std::mutex> lk(vkhip::g_mu);
    vkhip::Context& c = ctx();
    if (c.ready) {
        if (c.device == device) return VKHIP_OK;
        return fail(VKHIP_ERR_INVALID, "vkhip: already bound to device %d", c.device);
    }
    int count = 0;
    VKHIP_HIP(hipGetDeviceCount(&count));
    if (device < 0 || device >= count)
        return fail(VKHIP_ERR_DEVICE, "vkhip: no device %d (%d visible)", device, count);
    VKHIP_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    VKHIP_HIP(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(VKHIP_ERR_UNSUPPORTED, "vkhip: built for gfx950, device %d is %s", device,
                    prop.gcnArchName);
    // Stream-ordered allocations come from the device's default pool; keep
    // freed blocks in it instead of returning them to the OS at every
    // synchronisation, so a training step's per-node allocations are reused.
    hipMemPool_t pool;
    VKHIP_HIP(hipDeviceGetDefaultMemPool(&pool, device));
    uint64_t keep = ~0ull;
    VKHIP_HIP(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep));
    {
        const int rc = vkhip::resolve_scratch(device);
        if (rc != VKHIP_OK) return rc;
    }
    VKHIP_HIP(hipStreamCreateWithFlags(&c.own_stream, hipStreamNonBlocking));
    c.stream = c.own_stream;
    c.device = device;
    c.scratch = device < vkhip::kMaxScratchDevices ? vkhip::g_scratch_ptr[device] : nullptr;
    c.node_gemm_kernel = VKHIP_GEMM_AUTO;
    c.exact_math = 0;
    if (const char* sel = getenv("VKHIP_NUMERICS"))
        if (strcmp(sel, "exact") == 0) c.exact_math = 1;
    if (const char* sel = getenv("VKHIP_GEMM_KERNEL")) {
        if (strcmp(sel, "exact") == 0) c.node_gemm_kernel = VKHIP_GEMM_EXACT;
        else if (strcmp(sel, "mfma") == 0) c.node_gemm_kernel = VKHIP_GEMM_MFMA;
    }
    memset(&c.caps, 0, sizeof c.caps);
    snprintf(c.caps.name, sizeof c.caps.name, "%s", prop.name);
    c.caps.device_index = device;
    c.caps.compute_units = prop.multiProcessorCount;
    c.caps.wavefront_size = prop.warpSize;
    c.caps.max_threads_per_block = prop.maxThreadsPerBlock;
    c.caps.max_shared_memory = static_cast<int64_t>(prop.sharedMemPerBlock);
    c.caps.total_memory = static_cast<int64_t>(prop.totalGlobalMem);
    c.caps.global_float_atomics = 1;
    c.caps.asynchronous = 1;
    c.ready = true;
    return VKHIP_OK;
}

extern "C" int vkhip_shutdown(void) {
    std::lock_guard<std::mutex> lk(vkhip::g_mu);
    vkhip::Context& c = ctx();
    if (!c.ready) return VKHIP_OK;
    for (int slot = 0; slot < 3; ++slot) {
        if (c.ws[slot]) VKHIP_HIP(hipFreeAsync(c.ws[slot], c.stream));
        c.ws[slot] = nullptr;
        c.ws_bytes[slot] = 0;
    }
    for (int i = 0; i < c.ws_retired_count; ++i) VKHIP_HIP(hipFreeAsync(c.ws_retired[i], c.stream));
    c.ws_retired_count = 0;
    c.ws_pins = 0;
    {
        const int rc = vkhip::release_conv_tables();
        if (rc != VKHIP_OK) return rc;
    }
    VKHIP_HIP(hipStreamSynchronize(c.stream));
    if (c.copy_stream) {
        VKHIP_HIP(hipStreamSynchronize(c.copy_stream));
        VKHIP_HIP(hipStreamDestroy(c.copy_stream));
        c.copy_stream = nullptr;
    }
    {
        const int rc = vkhip::release_stage_slots();
        if (rc != VKHIP_OK) return rc;
    }
    {
        const int rc = vkhip::release_cached();
        if (rc != VKHIP_OK) return rc;
    }
    VKHIP_HIP(hipStreamDestroy(c.own_stream));
    c.own_stream = nullptr;
    c.stream = nullptr;
    c.scratch = nullptr;
    c.ready = false;
    return VKHIP_OK;
}

extern "C" const char* vkhip_last_error(void) { return vkhip::g_last_error; }

extern "C" int vkhip_caps_get(vkhip_caps* out) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (!out) return fail(VKHIP_ERR_INVALID, "caps: null output");
    *out = ctx().caps;
    return VKHIP_OK;
}

extern "C" int vkhip_set_stream(void* stream) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    hipStream_t next = stream ? static_cast<hipStream_t>(stream) : ctx().own_stream;
    // Cached blocks may still be in use by work on the old stream.
    if (next != ctx().stream) VKHIP_HIP(hipStreamSynchronize(ctx().stream));
    ctx().stream = next;
    return VKHIP_OK;
}

extern "C" void* vkhip_get_stream(void) { return ctx().stream; }

extern "C" int vkhip_set_numerics(int mode) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (mode != VKHIP_NUMERICS_FAST && mode != VKHIP_NUMERICS_EXACT)
        return fail(VKHIP_ERR_INVALID, "set_numerics: unknown mode %d", mode);
    ctx().exact_math = mode == VKHIP_NUMERICS_EXACT ? 1 : 0;
    return VKHIP_OK;
}

extern "C" int vkhip_get_numerics(void) {
    return ctx().exact_math ? VKHIP_NUMERICS_EXACT : VKHIP_NUMERICS_FAST;
}

// ---- memory ----------------------------------------------------------------------------

extern "C" int vkhip_alloc(size_t nbytes, void** out_ptr) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (!out_ptr) return fail(VKHIP_ERR_INVALID, "alloc: null output");
    *out_ptr = nullptr;
    if (nbytes == 0) return VKHIP_OK;
    return vkhip::cached_alloc(nbytes, out_ptr);
}

extern "C" int vkhip_free(void* ptr) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (!ptr) return VKHIP_OK;
    return vkhip::cached_free(ptr);
}

extern "C" int vkhip_release_cached(void) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    return vkhip::release_cached();
}

extern "C" int vkhip_memory_stats(size_t* bytes_in_use, size_t* bytes_cached) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::memory_stats(bytes_in_use, bytes_cached);
    return VKHIP_OK;
}

// ---- host copies through pinned staging slots ----------------------------------
// An upload from pageable memory through HIP waits for the DMA and for all work
// queued before it (~90 us for a 200 KB batch of inputs on an idle device).
// Uploads of up to kStagedMax bytes instead go through a ring of pinned slots:
// the bytes are copied on the host into a slot, the slot's DMA is enqueued on
// the stream behind the work already there, and the call returns; the caller's
// buffer is free at once (the reference's copy_from_host contract). A slot is
// reused only after the event recorded behind its previous DMA has completed.
// Small downloads come back through a slot too (DMA, stream sync, host copy).
// Slots are 1 MB and there are 32: every upload takes at least one slot (a
// 512-byte label tensor as much as a 200 KB batch), so the slot count bounds
// how many queued steps the host can run ahead of the device. With 4 slots of
// 4 MB a training loop that does not read its loss back could queue only two
// steps, and waited on a busy device at every upload (config 1's MLP: 0.162
// ms/step queued against 0.109 read back).
namespace vkhip {
constexpr size_t kStageSlotBytes = size_t{1} << 20;
constexpr int kStageSlots = 32;
constexpr size_t kStagedMax = kStageSlotBytes * kStageSlots;
struct StageSlot {
    void* host = nullptr;
    hipEvent_t done = nullptr;
    bool pending = false;  // an event was recorded behind this slot's last DMA
};
static StageSlot g_stage[kStageSlots];
static int g_stage_next = 0;
static std::mutex g_stage_mu;

// The next slot, allocated on first use and idle (its last DMA completed).
static int next_stage_slot(StageSlot** out) {
    StageSlot& s = g_stage[g_stage_next];
    g_stage_next = (g_stage_next + 1) % kStageSlots;
    if (!s.host) {
        if (hipHostMalloc(&s.host, kStageSlotBytes, hipHostMallocDefault) != hipSuccess) {
            s.host = nullptr;
            return fail(VKHIP_ERR_OOM, "pinned staging slot of %zu bytes could not be allocated",
                        kStageSlotBytes);
        }
        VKHIP_HIP(hipEventCreateWithFlags(&s.done, hipEventDisableTiming));
    } else if (s.pending) {
        VKHIP_HIP(hipEventSynchronize(s.done));
        s.pending = false;
    }
    *out = &s;
    return VKHIP_OK;
}

// Waits for and frees the staging slots (shutdown).
static int release_stage_slots() {
    std::lock_guard<std::mutex> lk(g_stage_mu);
    for (StageSlot& s : g_stage) {
        if (s.pending) VKHIP_HIP(hipEventSynchronize(s.done));
        s.pending = false;
        if (s.done) VKHIP_HIP(hipEventDestroy(s.done));
        s.done = nullptr;
        if (s.host) VKHIP_HIP(hipHostFree(s.host));
        s.host = nullptr;
    }
    g_stage_next = 0;
    return VKHIP_OK;
}
}  // namespace vkhip

extern "C" int vkhip_copy_from_host(void* dst, const void* host_src, size_t nbytes) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (nbytes == 0) return VKHIP_OK;
    if (!dst || !host_src) return fail(VKHIP_ERR_INVALID, "copy_from_host: null pointer");
    if (nbytes > vkhip::kStagedMax) {
        VKHIP_HIP(hipMemcpyAsync(dst, host_src, nbytes, hipMemcpyHostToDevice, ctx().stream));
        // The host buffer belongs to the caller once this returns.
        VKHIP_HIP(hipStreamSynchronize(ctx().stream));
        return VKHIP_OK;
    }
    std::lock_guard<std::mutex> lk(vkhip::g_stage_mu);
    for (size_t off = 0; off < nbytes; off += vkhip::kStageSlotBytes) {
        const size_t chunk = std::min(vkhip::kStageSlotBytes, nbytes - off);
        vkhip::StageSlot* slot = nullptr;
        st = vkhip::next_stage_slot(&slot);
        if (st != VKHIP_OK) return st;
        memcpy(slot->host, static_cast<const char*>(host_src) + off, chunk);
        VKHIP_HIP(hipMemcpyAsync(static_cast<char*>(dst) + off, slot->host, chunk,
                                 hipMemcpyHostToDevice, ctx().stream));
        VKHIP_HIP(hipEventRecord(slot->done, ctx().stream));
        slot->pending = true;
    }
    return VKHIP_OK;
}

// Pinned host buffers handed out by vkhip_host_alloc: an upload ahead of the
// stream from inside one is DMA'd from there, without the staging copy.
namespace vkhip {
static std::mutex g_host_mu;
static std::map<uintptr_t, size_t> g_host_blocks;  // start -> bytes

static bool in_host_block(const void* p, size_t nbytes) {
    std::lock_guard<std::mutex> lk(g_host_mu);
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    auto it = g_host_blocks.upper_bound(a);
    if (it == g_host_blocks.begin()) return false;
    --it;
    return a >= it->first && a + nbytes <= it->first + it->second;
}
}  // namespace vkhip

extern "C" int vkhip_host_alloc(size_t nbytes, void** out) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (!out) return fail(VKHIP_ERR_INVALID, "host_alloc: null output");
    *out = nullptr;
    if (nbytes == 0) return VKHIP_OK;
    void* p = nullptr;
    if (hipHostMalloc(&p, nbytes, hipHostMallocDefault) != hipSuccess || !p)
        return fail(VKHIP_ERR_OOM, "host_alloc: %zu bytes of pinned host memory could not be allocated", nbytes);
    std::lock_guard<std::mutex> lk(vkhip::g_host_mu);
    vkhip::g_host_blocks[reinterpret_cast<uintptr_t>(p)] = nbytes;
    *out = p;
    return VKHIP_OK;
}

extern "C" int vkhip_host_free(void* p) {
    if (!p) return VKHIP_OK;
    {
        std::lock_guard<std::mutex> lk(vkhip::g_host_mu);
        auto it = vkhip::g_host_blocks.find(reinterpret_cast<uintptr_t>(p));
        if (it == vkhip::g_host_blocks.end())
            return fail(VKHIP_ERR_INVALID, "host_free: %p was not handed out by vkhip_host_alloc", p);
        vkhip::g_host_blocks.erase(it);
    }
    // a DMA may still read it: free only once the device is done
    if (ctx().ready) {
        VKHIP_HIP(hipStreamSynchronize(ctx().stream));
        if (ctx().copy_stream) VKHIP_HIP(hipStreamSynchronize(ctx().copy_stream));
    }
    VKHIP_HIP(hipHostFree(p));
    return VKHIP_OK;
}

// Uploads ahead of the stream: the same pinned slots, the DMAs on a second
// stream that waits only for `after` (the event the stream recorded once it no
// longer reads dst), so a training loop copies batch i + 1 on the host and over
// PCIe while the device runs step i; `done` is recorded behind the DMAs for the
// stream to wait on (vkhip_stream_wait_event) before it reads dst.
extern "C" int vkhip_copy_from_host_async(void* dst, const void* host_src, size_t nbytes, void* after,
                                          void* done) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (!done) return fail(VKHIP_ERR_INVALID, "copy_from_host_async: null completion event");
    if (nbytes && (!dst || !host_src)) return fail(VKHIP_ERR_INVALID, "copy_from_host_async: null pointer");
    if (nbytes > vkhip::kStagedMax)
        return fail(VKHIP_ERR_UNSUPPORTED, "copy_from_host_async: %zu bytes exceed the %zu bytes of staging slots",
                    nbytes, vkhip::kStagedMax);
    vkhip::Context& c = ctx();
    if (!c.copy_stream) VKHIP_HIP(hipStreamCreateWithFlags(&c.copy_stream, hipStreamNonBlocking));
    if (after) VKHIP_HIP(hipStreamWaitEvent(c.copy_stream, static_cast<hipEvent_t>(after), 0));
    if (nbytes && vkhip::in_host_block(host_src, nbytes)) {
        // pinned by vkhip_host_alloc: the DMA reads the caller's bytes
        VKHIP_HIP(hipMemcpyAsync(dst, host_src, nbytes, hipMemcpyHostToDevice, c.copy_stream));
        VKHIP_HIP(hipEventRecord(static_cast<hipEvent_t>(done), c.copy_stream));
        return VKHIP_OK;
    }
    std::lock_guard<std::mutex> lk(vkhip::g_stage_mu);
    for (size_t off = 0; off < nbytes; off += vkhip::kStageSlotBytes) {
        const size_t chunk = std::min(vkhip::kStageSlotBytes, nbytes - off);
        vkhip::StageSlot* slot = nullptr;
        st = vkhip::next_stage_slot(&slot);
        if (st != VKHIP_OK) return st;
        memcpy(slot->host, static_cast<const char*>(host_src) + off, chunk);
        VKHIP_HIP(hipMemcpyAsync(static_cast<char*>(dst) + off, slot->host, chunk, hipMemcpyHostToDevice,
                                 c.copy_stream));
        VKHIP_HIP(hipEventRecord(slot->done, c.copy_stream));
        slot->pending = true;
    }
    VKHIP_HIP(hipEventRecord(static_cast<hipEvent_t>(done), c.copy_stream));
    return VKHIP_OK;
}

extern "C" int vkhip_stream_wait_event(void* event) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (!event) return fail(VKHIP_ERR_INVALID, "stream_wait_event: null event");
    VKHIP_HIP(hipStreamWaitEvent(ctx().stream, static_cast<hipEvent_t>(event), 0));
    return VKHIP_OK;
}

extern "C" int vkhip_copy_to_host(void* host_dst, const void* src, size_t nbytes) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (nbytes == 0) return VKHIP_OK;
    if (!host_dst || !src) return fail(VKHIP_ERR_INVALID, "copy_to_host: null pointer");
    if (nbytes > vkhip::kStageSlotBytes) {
        VKHIP_HIP(hipMemcpyAsync(host_dst, src, nbytes, hipMemcpyDeviceToHost, ctx().stream));
        VKHIP_HIP(hipStreamSynchronize(ctx().stream));
        return VKHIP_OK;
    }
    std::lock_guard<std::mutex> lk(vkhip::g_stage_mu);
    vkhip::StageSlot* slot = nullptr;
    st = vkhip::next_stage_slot(&slot);
    if (st != VKHIP_OK) return st;
    VKHIP_HIP(hipMemcpyAsync(slot->host, src, nbytes, hipMemcpyDeviceToHost, ctx().stream));
    VKHIP_HIP(hipStreamSynchronize(ctx().stream));
    memcpy(host_dst, slot->host, nbytes);
    return VKHIP_OK;
}

namespace vkhip {
int copy_pairs(const vkhip_copy* copies, size_t n);
}

extern "C" int vkhip_copy_device_to_device(const vkhip_copy* copies, size_t n) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (n && !copies) return fail(VKHIP_ERR_INVALID, "copy_device_to_device: null copy list");
    st = vkhip::copy_pairs(copies, n);
    if (st == VKHIP_OK) vkhip::program_note_copy(copies, n);
    return st;
}

extern "C" int vkhip_synchronize(void) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    VKHIP_HIP(hipStreamSynchronize(ctx().stream));
    return VKHIP_OK;
}

// ---- compute -------------------------------------------------------------------------

extern "C" int vkhip_supports(const vkhip_node* node) {
    return node && vkhip::check_extents(*node) == VKHIP_OK ? vkhip::supports_node(*node) : 0;
}

namespace vkhip {
int compute_nodes(const vkhip_node* nodes, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const int st = compute_node(nodes[i]);
        if (st != VKHIP_OK) return st;
    }
    return VKHIP_OK;
}

int copy_pairs(const vkhip_copy* copies, size_t n) {
    Unit unit("copy_device_to_device");
    return launch_copy_pairs(copies, n);
}
}  // namespace vkhip

extern "C" int vkhip_compute(const vkhip_node* nodes, size_t n) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (n && !nodes) return fail(VKHIP_ERR_INVALID, "compute: null node span");
    st = vkhip::compute_nodes(nodes, n);
    if (st == VKHIP_OK) vkhip::program_note_compute(nodes, n);
    return st;
}

extern "C" int vkhip_max_pool2d(const float* src, float* dst, uint32_t planes, uint32_t out_h,
                                uint32_t out_w, const vkhip_unfold* p) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::Unit unit("max_pool2d");
    if (!p) return fail(VKHIP_ERR_INVALID, "max_pool2d: null params");
    vkhip_operand d;
    const uint32_t ne[4] = {1, planes, static_cast<uint32_t>(p->image_h), static_cast<uint32_t>(p->image_w)};
    int64_t s = 1;
    for (int i = 3; i >= 0; --i) {
        d.ne[i] = ne[i];
        d.nb[i] = s;
        s *= ne[i];
    }
    return vkhip::launch_max_pool2d(src, d, dst, out_h, out_w, *p);
}

extern "C" int vkhip_max_pool2d_backward(const float* grad, const float* src, float* dst,
                                         uint32_t planes, uint32_t out_h, uint32_t out_w,
                                         const vkhip_unfold* p) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::Unit unit("max_pool2d_backward");
    if (!p) return fail(VKHIP_ERR_INVALID, "max_pool2d_backward: null params");
    vkhip_operand d;
    const uint32_t ne[4] = {1, planes, static_cast<uint32_t>(p->image_h), static_cast<uint32_t>(p->image_w)};
    int64_t s = 1;
    for (int i = 3; i >= 0; --i) {
        d.ne[i] = ne[i];
        d.nb[i] = s;
        s *= ne[i];
    }
    return vkhip::launch_max_pool2d_backward(grad, src, d, dst, out_h, out_w, *p, false);
}

// ---- timing ------------------------------------------------------------------------------

extern "C" int vkhip_event_create(void** out_event) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (!out_event) return fail(VKHIP_ERR_INVALID, "event_create: null output");
    hipEvent_t e;
    VKHIP_HIP(hipEventCreate(&e));
    *out_event = e;
    return VKHIP_OK;
}

extern "C" int vkhip_event_destroy(void* event) {
    if (!event) return VKHIP_OK;
    VKHIP_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)));
    return VKHIP_OK;
}

extern "C" int vkhip_event_record(void* event) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    VKHIP_HIP(hipEventRecord(static_cast<hipEvent_t>(event), ctx().stream));
    return VKHIP_OK;
}

extern "C" int vkhip_event_elapsed(void* start, void* end, float* out_ms) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (!out_ms) return fail(VKHIP_ERR_INVALID, "event_elapsed: null output");
    VKHIP_HIP(hipEventSynchronize(static_cast<hipEvent_t>(end)));
    VKHIP_HIP(hipEventElapsedTime(out_ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)));
    return VKHIP_OK;
}

extern "C" int vkhip_event_synchronize(void* event) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (!event) return fail(VKHIP_ERR_INVALID, "event_synchronize: null event");
    VKHIP_HIP(hipEventSynchronize(static_cast<hipEvent_t>(event)));
    return VKHIP_OK;
}

// ---- host-side planning helpers (no device needed) -----------------------------------

extern "C" int vkhip_exact_math(const float* host_x, float* host_y, size_t n, int log_mode) {
    if (n && (!host_x || !host_y)) return fail(VKHIP_ERR_INVALID, "exact_math: null array");
    for (size_t i = 0; i < n; ++i)
        host_y[i] = log_mode ? vkhip::exact_logf(host_x[i]) : vkhip::exact_expf(host_x[i]);
    return VKHIP_OK;
}

extern "C" uint32_t vkhip_fast_divide(uint32_t n, uint32_t d) {
    return d == 0 ? 0xffffffffu : vkhip::FastDiv(d).div(n);
}

extern "C" int vkhip_pairwise_leaf(uint32_t n, uint32_t leaf, uint32_t* out_depth,
                                   uint32_t* out_begin, uint32_t* out_end) {
    const int depth = vkhip::pairwise_depth(n);
    uint32_t b = 0, e = 0;
    if (leaf < (1u << depth)) vkhip::pairwise_leaf(n, depth, leaf, b, e);
    if (out_depth) *out_depth = static_cast<uint32_t>(depth);
    if (out_begin) *out_begin = b;
    if (out_end) *out_end = e;
    return leaf < (1u << depth) ? VKHIP_OK : VKHIP_ERR_INVALID;
}
