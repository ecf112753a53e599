/*
 * vkhip.h -- C ABI of the MI355X (gfx950) device backend for vkML's hot path.
 *
 * This is the drop-in boundary. In the reference, every graph flush reaches a
 * device through one virtual call, `vkml::Backend::compute(span<Node* const>)`
 * (reference: include/vkml/backend/api/backend.h:49-125), made by
 * `dispatch::realize` (src/dispatch/executor.cpp:132). The Vulkan implementation
 * of that call is `VulkanBackend::compute` (src/backend/vulkan/vulkan_backend.cpp:1189-2718).
 * This header replaces that implementation with plain C entry points:
 *
 *   - device/memory/copy/sync entry points mirror the rest of `Backend`
 *     (allocator(), copy_from_host, copy_to_host, copy_device_to_device,
 *     synchronize, capabilities);
 *   - `vkhip_compute` takes an ordered span of node records -- a C struct
 *     rendering of `vkml::Node` (include/vkml/graph/node.h:69-157) -- and
 *     enqueues one launch sequence on the backend's HIP stream;
 *   - one launch entry point per op family (gemm, split-K reduce, gemv,
 *     im2col, col2im, softmax, reduce, max-pool, elementwise) takes device
 *     pointers plus rank-4 operand descriptors, as the reference's push-constant
 *     blocks do (vulkan_backend.cpp:87-115 `GpuOperand`, :472-483 `GemmPush`).
 *
 * Conventions
 *   - No exceptions cross this ABI. Every entry point returns an int status
 *     (VKHIP_OK == 0); `vkhip_last_error()` gives the message of the last
 *     failure on the calling thread. The C++ wrapper maps the codes back to
 *     vkML's exception types (error.h:26-68).
 *   - All pointers are device addresses unless named `host_*`.
 *   - Work is stream-ordered and MAY RETURN BEFORE COMPLETION, exactly as the
 *     reference contract allows (backend.h:72-79). Host reads synchronise.
 *   - Strides are in ELEMENTS, extents are right-aligned to rank 4 and padded
 *     with 1 (reference to_gpu_operand, vulkan_backend.cpp:99-115). A stride of
 *     0 is a broadcast axis.
 */
#ifndef VKHIP_H
#define VKHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
enum vkhip_status {
    VKHIP_OK = 0,
    VKHIP_ERR_DEVICE = 1,        /* HIP runtime failure      -> vkml::DeviceError */
    VKHIP_ERR_UNSUPPORTED = 2,   /* op/dtype/layout not here -> vkml::NotImplementedError */
    VKHIP_ERR_INVALID = 3,       /* bad argument / shape     -> vkml::InternalError */
    VKHIP_ERR_OOM = 4,           /* allocation failed        -> vkml::OutOfMemoryError */
    VKHIP_ERR_NOT_INITIALISED = 5
};

/* ---- dtypes: same numbering as vkml::DType (include/vkml/core/dtype.h:17-23) */
enum vkhip_dtype {
    VKHIP_F32 = 0,
    VKHIP_F16 = 1, /* storage-only in the reference; not supported here */
    VKHIP_I32 = 2,
    VKHIP_I64 = 3,
    VKHIP_BOOL = 4 /* one byte per element, 0 or 1 */
};

/* ---- operand descriptor (reference GpuOperand, vulkan_backend.cpp:87-115) */
typedef struct vkhip_operand {
    uint32_t ne[4]; /* extents, right-aligned, padded with 1 */
    int64_t nb[4];  /* strides in elements; 0 = broadcast */
} vkhip_operand;

/* ---- op params: byte-compatible with the reference's structs ----------- */
typedef struct vkhip_unfold { /* vkml::UnfoldParams, include/vkml/graph/op.h:300-311 */
    int32_t kernel_h, kernel_w;
    int32_t stride_h, stride_w;
    int32_t pad_h, pad_w;
    int32_t dilation_h, dilation_w;
    int32_t image_h, image_w;
} vkhip_unfold;

/* ---- reduce op ids: same order as the reference shader's op_id
 *      (vulkan_backend.cpp:1863-1871) */
enum vkhip_reduce_op {
    VKHIP_REDUCE_SUM = 0,
    VKHIP_REDUCE_MEAN = 1,
    VKHIP_REDUCE_MAX = 2,
    VKHIP_REDUCE_MIN = 3,
    VKHIP_REDUCE_ARGMAX = 4,
    VKHIP_REDUCE_ARGMIN = 5
};

/* ---- node ops handled by vkhip_compute: the hot-path and support subset of
 *      vkml::OpKind (include/vkml/graph/op.h:30-139), numbered with OpKind's
 *      own ordinals so a host passes `static_cast<int>(node.op)` unchanged. */
enum vkhip_op {
    VKHIP_OP_FULL = 2,
    VKHIP_OP_ARANGE = 3,
    VKHIP_OP_CONTIGUOUS = 11,
    VKHIP_OP_CAST = 12,
    VKHIP_OP_ADD = 14,
    VKHIP_OP_SUB = 15,
    VKHIP_OP_MUL = 16,
    VKHIP_OP_SCALED_ADD = 17,
    VKHIP_OP_DIV = 18,
    VKHIP_OP_MAXIMUM = 20,
    VKHIP_OP_MINIMUM = 21,
    VKHIP_OP_EQUAL = 22,
    VKHIP_OP_LESS = 23,
    VKHIP_OP_GREATER = 24,
    VKHIP_OP_LESS_EQUAL = 25,
    VKHIP_OP_GREATER_EQUAL = 26,
    VKHIP_OP_NOT_EQUAL = 27,
    VKHIP_OP_NEG = 28,
    VKHIP_OP_EXP = 35,
    VKHIP_OP_LOG = 36,
    VKHIP_OP_RELU = 43,
    VKHIP_OP_SUM = 47,
    VKHIP_OP_MEAN = 48,
    VKHIP_OP_MAX = 49,
    VKHIP_OP_MIN = 50,
    VKHIP_OP_ARGMAX = 52,
    VKHIP_OP_ARGMIN = 53,
    VKHIP_OP_MATMUL = 54,
    VKHIP_OP_SOFTMAX = 55,
    VKHIP_OP_LOG_SOFTMAX = 56,
    VKHIP_OP_IM2COL = 57,
    VKHIP_OP_COL2IM = 58,
    VKHIP_OP_MAX_POOL2D = 59,
    VKHIP_OP_MAX_POOL2D_BACKWARD = 60,
    VKHIP_OP_WHERE = 64,
    /* Backend extensions (not vkML OpKind ordinals): the reference's
     * cross_entropy composition (ops.cpp:417-441: mean(-sum(log_softmax(x) *
     * one_hot(labels), -1))) fused per row, and its gradient as the reference
     * autograd builds it (neg, sum and mul backward, then log_softmax backward
     * g - exp(out) * sum(g), autograd.cpp). Values are those of the unfused
     * graph, operation for operation; see vkhip_node below. */
    VKHIP_OP_CROSS_ENTROPY = 96,          /* src0 logits [N,C] f32 (unit-stride rows), src1 labels [N] i64 -> out [N] f32: -sum_c(ls*onehot) */
    VKHIP_OP_CROSS_ENTROPY_BACKWARD = 97, /* src0 logits, src1 labels, src2 g [N] f32 -> out [N,C] f32: d(out)/d(logits) */
    /* src0 x [N,C,H,W], src1 weight [Cout,C,kh,kw] (C,kh,kw mergeable) or
     * [Cout,C*kh*kw], params vkhip_unfold -> out [N,Cout,out_h,out_w]: the
     * reference conv2d without bias (ops.cpp:662-705), im2col never written;
     * bit-identical to IM2COL followed by MATMUL with the flat weight. */
    VKHIP_OP_CONV2D = 98,
    /* src0 x [N,C,H,W], src1 grad [N,Cout,out_h,out_w] (positions unit-stride),
     * params vkhip_unfold -> out [N,Cout,C*kh*kw]: per image grad @ im2col(x)^T,
     * the conv2d weight gradient before its batch sum, bit-identical to IM2COL
     * followed by MATMUL(grad, cols^T). */
    VKHIP_OP_CONV2D_WEIGHT_GRAD = 99,
    /* src0 x, src1 g (the relu's input and the gradient of its output, same
     * extents as out) -> out = x <= 0 ? +0 : g: the reference relu gradient
     * where(less_equal(x, zeros_like(x)), zeros_like(g), g) (autograd.cpp:397-408)
     * as one node, value for value (a NaN x passes g through). */
    VKHIP_OP_RELU_BACKWARD = 100,
    /* src0 x [N,C,H,W], src1 grad [N,Cout,out_h,out_w] (positions unit-stride),
     * params vkhip_unfold -> out [Cout, C*kh*kw]: the conv2d weight gradient
     * summed over the batch, the value of CONV2D_WEIGHT_GRAD followed by the
     * batch SUM. FAST numerics fold the batch into the product's K axis (no
     * intermediate, within the GEMM tolerance of the graph); EXACT numerics
     * give the graph's bits. */
    VKHIP_OP_CONV2D_WEIGHT_GRAD_SUM = 101,
    /* src0 grad [N,Cout,out_h,out_w] (positions unit-stride), src1 weight
     * [Cout,C,kh,kw] or [Cout,C*kh*kw] (rows contiguous), params the forward's
     * vkhip_unfold -> out [N,C,H,W] contiguous: the conv2d input gradient,
     * the value of col2im(flat_weight^T @ grad). FAST numerics with unit
     * strides compute it as one convolution of grad with the flipped,
     * transposed weight when C >= 32 (no column matrix; within the GEMM
     * tolerance of the graph); otherwise the TN product and col2im (the
     * graph's bits). */
    VKHIP_OP_CONV2D_INPUT_GRAD = 102,
    /* CONV2D with the bias add and ReLU that follow it in a conv layer: src0
     * x, src1 w (as CONV2D), src2 bias [Cout] or [Cout,1,1] (any stride along
     * channels) -> out = relu(conv2d(x, w) + bias[c]), where relu(v) = v <= 0
     * ? 0 : v: the values of the CONV2D, ADD (bias broadcast) and RELU nodes
     * it replaces, bit for bit, without writing and re-reading the two
     * intermediates. */
    VKHIP_OP_CONV2D_BIAS_RELU = 103,
    /* relu(src0 + src1), sources with the output's extents (broadcast axes
     * stride 0) as for ADD: the ADD and RELU nodes' values in one pass
     * (a Linear layer's bias add and activation). */
    VKHIP_OP_ADD_RELU = 104,
    /* MAX_POOL2D_BACKWARD followed by the RELU_BACKWARD of the relu that
     * produced the pool's input: src0 g [N,C,out_h,out_w], src1 x [N,C,H,W]
     * (the pool's input, the relu's output), params vkhip_unfold as for
     * MAX_POOL2D_BACKWARD -> out = x <= 0 ? +0 : max_pool2d_backward(g, x):
     * the two nodes' values (selects only), in one pass that reads x once. */
    VKHIP_OP_MAX_POOL2D_BACKWARD_RELU = 105,
    /* MATMUL with the bias add (and ReLU) of a Linear layer: src0, src1 as
     * MATMUL, src2 bias [N] (any stride), params uint32 relu -> out =
     * relu?(src0 @ src1 + bias[col]), relu(v) = v <= 0 ? 0 : v: the values of
     * the MATMUL, ADD (bias broadcast over rows) and RELU nodes it replaces,
     * the epilogue applied where the split-K partials are folded (or in a
     * pass after an unsplit product). */
    VKHIP_OP_MATMUL_BIAS = 106,
    /* MATMUL followed by the RELU_BACKWARD it feeds: src0, src1 as MATMUL,
     * src2 x with the output's extents (contiguous; the relu's input or
     * output) -> out = x <= 0 ? +0 : src0 @ src1 (a NaN x passes the product):
     * the two nodes' values, the select applied where the split-K partials
     * are folded (or in a pass after an unsplit product). */
    VKHIP_OP_MATMUL_RELU_BACKWARD = 107,
    /* The weight and bias gradients of a conv layer y = relu(conv2d(x, w) +
     * bias) whose output feeds a 2x2, stride-2 max-pool, from the pool's
     * output gradient: src0 x [N,C,H,W], src1 y [N,Cout,oh,ow] (contiguous),
     * src2 gp [N,Cout,oh/2,ow/2] (contiguous), params the conv's
     * vkhip_unfold -> out [Cout*C*kh*kw + Cout] contiguous: the weight
     * gradient [Cout, C*kh*kw] then the bias gradient [Cout], the values of
     * MAX_POOL2D_BACKWARD_RELU(gp, y) = dz, CONV2D_WEIGHT_GRAD_SUM(x, dz) and
     * SUM(dz, axes 0, 2, 3) that it replaces (the backward of conv2d's bias
     * add, the relu and the pool, autograd.cpp:84-116 and :397-408, and the
     * pool's adjoint). FAST numerics where the small-window kernel takes the
     * layer form dz in the kernel without writing it: the replaced nodes'
     * fast-path bits; otherwise those nodes in turn. */
    VKHIP_OP_CONV2D_POOL_WEIGHT_BIAS_GRAD = 108,
    /* MAX_POOL2D_BACKWARD_RELU of 2x2 windows at stride 2 with the bias
     * gradient of the conv layer whose relu output the pool read: src0 g
     * [N,C,H/2,W/2], src1 y [N,C,H,W] (both contiguous), params the pool's
     * vkhip_unfold (2x2, stride 2, no padding) -> out [N*C*H*W + C]
     * contiguous: the pool gradient dz (105's values) then SUM(dz, axes 0, 2,
     * 3), the broadcast adjoint of the layer's bias (autograd.cpp:84-116), in
     * the pairwise tree's order; one pass over dz where the planes allow it
     * (rows of 16 or 32, power-of-two extents). */
    VKHIP_OP_MAX_POOL2D_BACKWARD_RELU_BIAS = 109
};

/* ---- a tensor as a node sees it (vkml::Node shape + storage) ------------ */
typedef struct vkhip_tensor {
    void* data;      /* device address of element 0 (Node::data()) */
    int32_t dtype;   /* vkhip_dtype */
    int32_t ndim;    /* 0..4 */
    int64_t ne[4];   /* extents, first ndim used (Shape::dim) */
    int64_t nb[4];   /* strides in ELEMENTS, first ndim used (Shape::stride / itemsize) */
} vkhip_tensor;

/* ---- one node of a flush (vkml::Node, node.h:69-157) -------------------- */
typedef struct vkhip_node {
    int32_t op;            /* vkhip_op */
    int32_t n_src;         /* 0..3 */
    vkhip_tensor out;      /* bound, contiguous */
    vkhip_tensor src[3];   /* realised sources; views already resolved to strides */
    uint8_t params[64];    /* vkml::OpParams::raw (op.h:199-221), same payload layout */
} vkhip_node;

/* ---- device description (vkml::DeviceCapabilities, capabilities.h:23-119) */
typedef struct vkhip_caps {
    char name[64];
    int32_t device_index;
    int32_t compute_units;        /* split-K and reduce planning use it */
    int32_t wavefront_size;       /* 64 on CDNA */
    int32_t max_threads_per_block;
    int64_t max_shared_memory;    /* LDS bytes per workgroup */
    int64_t total_memory;
    int32_t global_float_atomics; /* present on gfx950, deliberately unused */
    int32_t asynchronous;         /* 1: compute() returns before completion */
} vkhip_caps;

/* ---- one device-to-device copy (vkml::BufferCopy, backend.h:18-24) ------ */
typedef struct vkhip_copy {
    void* dst;
    const void* src;
    size_t nbytes;
} vkhip_copy;

/* ---- GEMM selection knobs: the reference's VKML_GEMM_* switches
 *      (vulkan_backend.cpp:536-561, 2160-2250) as explicit arguments ------- */
enum vkhip_gemm_kernel {
    VKHIP_GEMM_AUTO = 0,   /* MFMA tiles, split-K / GEMV by the planner */
    VKHIP_GEMM_MFMA = 1,   /* MFMA tiles, never GEMV */
    VKHIP_GEMM_GEMV = 2,   /* force the GEMV path (N == 1 or M == 1 only) */
    /* the comparison arm: each product rounded, the K products summed in the
     * CPU oracle's pairwise order, so C is the oracle's bit for bit (the role
     * of the reference's gemm_naive.comp:56-101, VKML_GEMM_KERNEL=naive,
     * vulkan_backend.cpp:2158-2161). Vector ALU, not matrix cores: slow. */
    VKHIP_GEMM_EXACT = 3
};
typedef struct vkhip_gemm_opts {
    int32_t kernel;        /* vkhip_gemm_kernel */
    int32_t split_k;       /* 0 = AUTO planner, 1 = OFF, >1 = forced partition request */
} vkhip_gemm_opts;

/* ======================================================================== */
/* Backend lifecycle / description  (Backend::name/device/capabilities)     */
/* ======================================================================== */

/* Binds the calling process to GPU `device` and creates the backend stream.
 * Idempotent for the same device. */
int vkhip_init(int device);
/* Releases the stream and the backend's internal workspaces. */
int vkhip_shutdown(void);
/* Message of the last failure on this thread ("" if none). */
const char* vkhip_last_error(void);
int vkhip_caps_get(vkhip_caps* out);
/* Makes the backend enqueue on `stream` (a hipStream_t; NULL = its own).
 * Lets a host that owns the stream (e.g. PyTorch) share stream order. The
 * previous stream is synchronised first (cached blocks carry no pending work
 * across streams). */
int vkhip_set_stream(void* stream);
void* vkhip_get_stream(void);

/* ======================================================================== */
/* Memory (Backend::allocator, copies, synchronize)                          */
/* ======================================================================== */
/* Device memory (Backend::allocator; reference VulkanBackend allocation map,
 * vulkan_backend.cpp:894-919). Served from per-size caches of blocks; the
 * backend's one stream orders every use, so a freed block is reused by later
 * work only (the reference's retirement queue, vulkan_backend.cpp:921-984). */
int vkhip_alloc(size_t nbytes, void** out_ptr);
/* Returns a block from vkhip_alloc to the cache; VKHIP_ERR_INVALID for a
 * pointer it did not hand out. */
int vkhip_free(void* ptr);
/* Synchronises and returns every cached (free) block to HIP. Also done
 * automatically when an allocation fails, then the allocation is retried. */
int vkhip_release_cached(void);
/* Bytes handed out and not freed, and bytes held in the caches. */
int vkhip_memory_stats(size_t* bytes_in_use, size_t* bytes_cached);
/* Returns once the host bytes are copied (uploads up to 16 MB through pinned
 * staging slots, the DMA queued on the stream before any later work): the
 * caller may reuse host_src at once (backend.h copy_from_host). */
int vkhip_copy_from_host(void* dst, const void* host_src, size_t nbytes);
int vkhip_copy_to_host(void* host_dst, const void* src, size_t nbytes); /* synchronises */
/* Pinned host memory (no counterpart in the reference, whose uploads stage
 * through its own buffers): for a data loader that fills its batches where
 * the DMA can read them. vkhip_host_free waits for the device first. */
int vkhip_host_alloc(size_t nbytes, void** out_ptr);
int vkhip_host_free(void* ptr);
/* An upload queued ahead of the stream's work. No counterpart in the
 * reference (its uploads are ordered with its compute queue, backend.h
 * copy_from_host); for a training loop that uploads batch i + 1 while the
 * device runs step i: the separate transfer queue its asynchronous-submission
 * design leaves out (docs/adr/0012-asynchronous-submission.md:223-224), on
 * a HIP stream and events instead of semaphores. The bytes go through the
 * pinned staging slots (at most 32 MB) and return to the caller as
 * vkhip_copy_from_host's do -- except bytes inside a vkhip_host_alloc block,
 * which the DMA reads in place: the caller keeps them unchanged until `done`
 * has completed. The DMAs run on a second stream that first
 * waits for `after` (an event recorded on the backend stream once it no
 * longer reads dst; null: no wait), and `done` is recorded behind them.
 * The backend stream must wait for `done` (vkhip_stream_wait_event) before it
 * reads dst. */
int vkhip_copy_from_host_async(void* dst, const void* host_src, size_t nbytes, void* after, void* done);
/* Later work on the backend stream waits (on the device) for `event`. */
int vkhip_stream_wait_event(void* event);
/* One unit of work for several disjoint copies (backend.h:83-108). */
int vkhip_copy_device_to_device(const vkhip_copy* copies, size_t n);
int vkhip_synchronize(void);

/* ======================================================================== */
/* The Backend::compute boundary                                             */
/* ======================================================================== */
/* 1 if `node` is supported (op, dtype, rank, layout), else 0
 * (VulkanBackend::supports, vulkan_backend.cpp:1012-1187). */
int vkhip_supports(const vkhip_node* node);
/* Enqueues `n` nodes in order on the backend stream (backend.h:72-79). */
int vkhip_compute(const vkhip_node* nodes, size_t n);

/* ======================================================================== */
/* Per-op-family launch entry points (what compute() dispatches to)          */
/* ======================================================================== */

/* C[b0,b1,M,N] (contiguous) = A[b0,b1,M,K] @ B[b0,b1,K,N]; any strides
 * (NN / NT / TN / batch-broadcast). fp32 in, fp32 MFMA accumulate.
 * Reference: Matmul case, vulkan_backend.cpp:2056-2657; CPU oracle
 * kernels_matmul.cpp:34-87. `opts` may be NULL (AUTO). */
int vkhip_gemm(const float* a, const vkhip_operand* a_desc,
               const float* b, const vkhip_operand* b_desc,
               float* c, const vkhip_gemm_opts* opts);

/* vkhip_gemm that allocates nothing. No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments, plan, kernels and bits as vkhip_gemm; the split-K partials go to
 * a fixed per-device scratch array of VKHIP_GEMM_NOALLOC_SCRATCH_BYTES that
 * the library holds until the process ends, instead of the workspace
 * vkhip_gemm grows. A product whose planned split needs more than that is
 * refused with VKHIP_ERR_INVALID (nothing is launched). Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (two streams, two
 * threads) race on it. No profile record is taken for these calls. */
#define VKHIP_GEMM_NOALLOC_SCRATCH_BYTES (32u * 1024u * 1024u)
int vkhip_gemm_noalloc(const float* a, const vkhip_operand* a_desc,
                       const float* b, const vkhip_operand* b_desc,
                       float* c, const vkhip_gemm_opts* opts);

/* The split-K plan the AUTO path would use for this problem
 * (reference plan_split_k, vulkan_backend.cpp:596-647). Writes splits (1 =
 * no split) and chunk (K-tiles per partition, a power of two). */
int vkhip_gemm_plan(uint32_t batch, uint32_t m, uint32_t n, uint32_t k,
                    int32_t split_request, uint32_t* out_splits, uint32_t* out_chunk);

/* dst[i] = carry-stack fold of ws[s*ne + i], s = 0..splits-1
 * (reference gemm_split_k_reduce.comp:48-85). Deterministic, bit-stable. */
int vkhip_split_k_reduce(const float* ws, float* dst, uint64_t ne, uint32_t splits);

/* y[M] = A[M,K] @ x[K] with strided A (row stride lda, unit inner stride
 * required) -- the N == 1 matmul (reference gemv.comp:105-201). Products are
 * rounded, then summed in the CPU oracle's pairwise order: bit-exact. */
int vkhip_gemv(const float* a, int64_t lda, const float* x, int64_t incx, float* y,
               uint32_t m, uint32_t k);

/* cols[N, C*kh*kw, out_h*out_w] from image src[N,C,H,W] (any strides).
 * Reference: ops.cpp:485-512, kernels_movement.cpp:454-483, im2col.comp. */
int vkhip_im2col(const float* src, const vkhip_operand* src_desc, float* dst,
                 const vkhip_unfold* p);

/* image dst[N,C,H,W] (contiguous) from cols[N, C*kh*kw, L] (contiguous);
 * pull with ascending (ki,kj) fold from 0.0f: bit-exact.
 * Reference: ops.cpp:514-541, kernels_movement.cpp:500-542, col2im.comp. */
int vkhip_col2im(const float* cols, float* dst, uint32_t n, uint32_t channels,
                 const vkhip_unfold* p);

/* Softmax / log-softmax of src over `axis` (0..3 of the rank-4 descriptor),
 * out contiguous with src's extents. Reference: ops.cpp:883-900,
 * kernels_reduce.cpp:205-259, softmax.comp. */
int vkhip_softmax(const float* src, const vkhip_operand* src_desc, float* dst, int axis,
                  int log_softmax);

/* Reduction of src over the axes in `axes_mask` (bit i = axis i of the
 * rank-4 descriptor). dst holds prod(kept extents) values, f32 or int64 for
 * argmax/argmin. Reference: ops.cpp:119-130, kernels_reduce.cpp:44-176,
 * reduce.comp. Sum/mean follow the oracle's pairwise association: bit-exact. */
int vkhip_reduce(int op, const float* src, const vkhip_operand* src_desc, uint32_t axes_mask,
                 void* dst);

/* Max-pool forward and backward (pull, first maximum wins). Reference:
 * ops.cpp:611-641, kernels_movement.cpp:556-680, max_pool2d.comp. */
int vkhip_max_pool2d(const float* src, float* dst, uint32_t planes, uint32_t out_h,
                     uint32_t out_w, const vkhip_unfold* p);
int vkhip_max_pool2d_backward(const float* grad, const float* src, float* dst,
                              uint32_t planes, uint32_t out_h, uint32_t out_w,
                              const vkhip_unfold* p);

/* a*alpha + b*beta with two rounded multiplies and one add
 * (reference scaled_add.comp:41-66, kernels_elementwise.cpp:256-259). */
int vkhip_scaled_add(const float* a, const float* b, float* out, uint64_t n, float alpha,
                     float beta);

/* ======================================================================== */
/* Timing (the reference's per-dispatch timestamp pairs, vk_command.h:185-256,
 * exposed as HIP events on the backend stream)                              */
/* ======================================================================== */
int vkhip_event_create(void** out_event);
int vkhip_event_destroy(void* event);
/* Records `event` on the backend stream, after all work enqueued so far. */
int vkhip_event_record(void* event);
/* Milliseconds between two recorded events; waits for `end` to complete. */
int vkhip_event_elapsed(void* start, void* end, float* out_ms);
/* Waits on the host until `event` (recorded) has completed. No counterpart in
 * the reference (its host reads synchronise, tensor.cpp:178-200); for callers
 * that queue work without reading it back and bound how far ahead they run. */
int vkhip_event_synchronize(void* event);

/* Convolution forward as one implicit-im2col GEMM per image:
 * out[n] = w (Cout x C*kh*kw) @ cols(x[n]) with the cols matrix gathered from
 * the image inside the GEMM's tile loads instead of materialised (the
 * reference writes it: im2col then matmul, ops.cpp:662-705). x: [N,C,H,W] any
 * strides; w: [Cout, C*kh*kw] as a rank-4 descriptor [1,1,Cout,CK]; out
 * contiguous [N, Cout, out_h*out_w]. Same plan, tiles and MFMA order as
 * vkhip_gemm on the materialised cols, hence the same bits. */
int vkhip_conv2d(const float* x, const vkhip_operand* x_desc, const float* w,
                 const vkhip_operand* w_desc, float* out, const vkhip_unfold* p);
/* The convolution weight gradient's per-image products without the cols
 * matrix: out[n] = grad[n] (Cout x L) @ im2col(x[n])^T (L x C*kh*kw), the
 * product the reference's conv2d backward takes on the materialised columns
 * (matmul(grad, cols^T), autograd.cpp:548-553 over ops.cpp:662-705; the sum
 * over n stays a separate reduction). x: [N,C,H,W] any strides; grad: rank-4
 * [1, N, Cout, L] with unit stride along L; out contiguous [N, Cout, C*kh*kw].
 * Same plan, K order and split-K fold as vkhip_gemm on the columns, hence the
 * same bits. */
int vkhip_conv2d_weight_grad(const float* x, const vkhip_operand* x_desc, const float* grad,
                             const vkhip_operand* grad_desc, float* out, const vkhip_unfold* p);

/* The weight gradient summed over the batch (VKHIP_OP_CONV2D_WEIGHT_GRAD_SUM):
 * out [Cout, C*kh*kw] contiguous = sum_n grad[n] @ im2col(x[n])^T, what the
 * reference's conv2d backward computes as the per-image products followed by
 * the broadcast adjoint's batch sum (autograd.cpp:548-553, :84-116). grad as
 * for vkhip_conv2d_weight_grad. FAST numerics with out_h*out_w a multiple of
 * 32: one product with the batch folded into K. Otherwise the per-image
 * products and the batch sum (the graph's bits). */
/* The convolution input gradient (VKHIP_OP_CONV2D_INPUT_GRAD): out [N,C,H,W]
 * contiguous = col2im(flat_weight^T @ grad[n]), what the reference's conv2d
 * backward computes for x through the matmul and im2col adjoints
 * (autograd.cpp:548-553, ops.cpp:662-705). grad: rank-4 [N, Cout, out_h,
 * out_w] with unit position strides; w: [1,1,Cout,C*kh*kw] rows contiguous;
 * p: the forward's geometry. FAST numerics with unit strides,
 * dilation*(k-1) >= pad and C >= 32: one implicit-im2col convolution of grad
 * with the weight flipped and transposed (pad dilation*(k-1) - pad).
 * Otherwise the TN product into a column matrix, then col2im. */
int vkhip_conv2d_input_grad(const float* grad, const vkhip_operand* grad_desc, const float* w,
                            const vkhip_operand* w_desc, float* out, const vkhip_unfold* p);
int vkhip_conv2d_weight_grad_sum(const float* x, const vkhip_operand* x_desc, const float* grad,
                                 const vkhip_operand* grad_desc, float* out, const vkhip_unfold* p);

/* ======================================================================== */
/* Fused optimiser step                                                      */
/* ======================================================================== */
/* One parameter of an SGD step: `param` is updated in place, `grad` is
 * contiguous, `velocity` is the momentum buffer (unused when momentum == 0).
 * `first` = 1 on a parameter's first momentum step (no previous velocity). */
typedef struct vkhip_sgd_param {
    float* param;
    const float* grad;
    float* velocity;
    uint64_t n;
    int32_t first;
    int32_t reserved;
} vkhip_sgd_param;
/* The whole SGD step of the reference optimiser (python/vkml/optim.py:
 * 146-199: weight decay g' = g + p*wd, velocity v = m*v + g' (v = g' on the
 * first step), Nesterov direction g' + m*v, p = p - lr*direction) for every
 * parameter in ONE launch, instead of the reference's two ScaledAdd nodes and a
 * copy per parameter (scaled_add.comp:41-66). Each expression is evaluated
 * exactly as those nodes do it: two rounded products and one rounded add, no
 * FMA, so the values are bit-identical to the unfused step. */
int vkhip_sgd_step(const vkhip_sgd_param* params, size_t count, float lr, float momentum,
                   float weight_decay, int nesterov);

/* ======================================================================== */
/* Observability: decision facts and per-dispatch timing                     */
/* ======================================================================== */
/* One choice the backend made, what it rejected, why, and the numbers that
 * forced it (reference vkml::observe::Decision, include/vkml/util/observe.h:
 * 55-93). Sites: "matmul.kernel", "matmul.split_k", "reduce.structure",
 * "softmax.structure", "col2im.kernel", "max_pool2d.kernel",
 * "allocator.release". The strings live for the duration of the callback
 * only. `dispatch` names the unit of work the choice produced: the same id the
 * profile records carry, so a consumer joins the two to learn what a kernel
 * choice cost (vulkan_backend.h:123-131, 174-181). */
typedef struct vkhip_decision {
    const char* site;
    const char* op;          /* the operation in the user's vocabulary */
    const char* chose;
    const char* instead_of;  /* "" when nothing was rejected */
    const char* because;
    int64_t required;        /* the numbers behind the choice; 0 when none */
    int64_t available;
    uint64_t dispatch;
} vkhip_decision;
typedef void (*vkhip_decision_fn)(const vkhip_decision* decision, void* user);
/* Installs the one subscriber (NULL removes it), like observe::subscribe
 * (observe.h:108-119). Decisions are published synchronously on the calling
 * thread, before the work they choose is enqueued. */
int vkhip_subscribe_decisions(vkhip_decision_fn fn, void* user);

/* One measured unit of work: a node of vkhip_compute or one call of a
 * per-op entry point (reference ProfileRecord, vulkan_backend.h:123-131). */
typedef struct vkhip_profile_record {
    char label[48];    /* the op ("matmul", "softmax", ...) */
    double gpu_ms;     /* HIP-event time of the unit's launches on the stream */
    uint64_t dispatch; /* joins with vkhip_decision.dispatch */
} vkhip_profile_record;
/* Enables per-unit event timing (set_profiling, vulkan_backend.h:165-166);
 * zero cost when off. Records accumulate until read (at most 65536 pending;
 * older ones are dropped and counted). */
int vkhip_set_profiling(int enabled);
/* Waits for the recorded work, moves up to `capacity` of the oldest pending
 * records to `out` and sets *count; *dropped (may be NULL) gets the number
 * of records dropped since the last read. */
int vkhip_profile_read(vkhip_profile_record* out, size_t capacity, size_t* count,
                       uint64_t* dropped);

/* ======================================================================== */
/* Numerics mode                                                              */
/* ======================================================================== */
/* FAST (default): matrix-core GEMMs and convolutions, hardware-assisted
 * exp/log; within the north star's tolerances of the CPU oracle (GEMM and
 * softmax 1e-5*sqrt(K)), bit-exact everywhere else. EXACT: every node the
 * CPU oracle's bits: GEMMs (AUTO selection) and convolutions on the exact arm
 * (VKHIP_GEMM_EXACT's arithmetic, convolution columns gathered from the
 * image), softmax / log-softmax / cross-entropy / exp / log with the oracle's
 * exp and log methods (vkhip_exact_math) and true division. The role of the
 * reference's precise comparison arms (gemm_naive.comp:56-101 with
 * VKML_GEMM_KERNEL=naive, vulkan_backend.cpp:2158-2172), extended to the
 * transcendentals so whole training runs can be compared bit for bit. Applies
 * to work enqueued after the call; VKHIP_NUMERICS=exact sets it at init. */
enum vkhip_numerics {
    VKHIP_NUMERICS_FAST = 0,
    VKHIP_NUMERICS_EXACT = 1
};
int vkhip_set_numerics(int mode);
int vkhip_get_numerics(void);

/* ======================================================================== */
/* Recorded programs: replay of a step whose graph repeats                   */
/* ======================================================================== */
/* No single counterpart in the reference; it is the "record once, re-submit"
 * model the reference measured for its submission path
 * (docs/adr/0012-asynchronous-submission.md section 2) applied to the host
 * cost docs/SMALL-STEP-LATENCY.md:44-51 names. While a program records, every
 * vkhip_compute, vkhip_sgd_step and vkhip_copy_device_to_device call runs as
 * usual and is also appended to it with its arguments (node records byte for
 * byte); host copies are not recorded. Replaying enqueues the same calls in
 * the same order with the same device pointers, so the caller keeps every
 * buffer the recorded calls touched alive and in place, and uploads new inputs
 * into the recorded input buffers before each run. A replayed SGD step
 * continues from the recorded step's velocity (its first-step flags are
 * recorded as 0). One program records at a time. */
typedef struct vkhip_program vkhip_program;
int vkhip_program_begin(void);
int vkhip_program_end(vkhip_program** out);
/* use_graph bit 0 set: the first run captures the replayed launches into a
 * HIP graph on the backend stream (not while profiling is on), later runs
 * launch the graph; the backend stream must then stay the same. Bit 0 clear:
 * a plain run, call by call; bit 1 (2) then marks a run whose outputs the
 * caller will not read, which skips the early-output copy below. */
int vkhip_program_run(vkhip_program* program, int use_graph);
/* Waits for a captured graph to finish, then frees the program. */
int vkhip_program_destroy(vkhip_program* program);
int vkhip_program_info(const vkhip_program* program, size_t* calls, size_t* nodes,
                       int* has_graph);
/* Early outputs (no counterpart in the reference; the step-latency target of
 * docs/SMALL-STEP-LATENCY.md:44-51 for a host that reads each step's loss).
 * Declares the program's outputs as n device spans (src, nbytes; dst unused),
 * at most 4096 bytes in all, before its first run. The recorded units (a
 * node, an SGD call, a copy call) are reordered once: each unit that the
 * outputs depend on moves ahead of later-recorded units it shares no buffer
 * hazard with (read/write, write/read, write/write of the bytes their tensors
 * span), so the values of every unit are unchanged. Each plain run (use_graph
 * == 0) then copies the outputs into pinned host memory right behind their
 * last writer and records an event there. Graph runs do not. */
int vkhip_program_set_outputs(vkhip_program* program, const vkhip_copy* outputs, size_t n);
/* Input rebinding (no counterpart in the reference). Points the program's
 * recorded input span [recorded, recorded + nbytes) at `now` for the plain
 * runs enqueued after the call: every pointer field of the recorded calls
 * (node tensors, SGD parameters, copies) that lay inside the span when it was
 * first bound is moved to the same offset from `now`; now == recorded
 * restores it. A host then feeds a step from a batch already in device
 * memory (a resident data set, a staging buffer a DMA filled) without copying
 * it into the recorded input; the bytes at `now` must stay unchanged until
 * the runs that read them have finished. VKHIP_ERR_INVALID once the program
 * has a captured graph, for a span a recorded call writes, or for a span
 * overlapping another bound span. */
int vkhip_program_bind_input(vkhip_program* program, const void* recorded, const void* now, size_t nbytes);
/* Waits for the latest plain run's outputs (not for the rest of its step)
 * and copies their bytes, in declaration order, to host_dst (nbytes: their
 * total). VKHIP_ERR_INVALID when no outputs are declared or the latest run
 * was a graph run or none. */
int vkhip_program_read_outputs(vkhip_program* program, void* host_dst, size_t nbytes);

/* ======================================================================== */
/* Host-side planning helpers (callable without a GPU)                       */
/* ======================================================================== */
/* The order vkhip_program_set_outputs gives n recorded node records (each a
 * unit reading its sources' and writing its output's byte spans) for the
 * declared outputs: order[i] is the recorded index of the i-th node to run,
 * and *out_after the number of nodes after which the outputs are final. No
 * device is touched (pointers are compared, never dereferenced). */
int vkhip_program_output_order(const vkhip_node* nodes, size_t n, const vkhip_copy* outputs,
                               size_t n_outputs, size_t* order, size_t* out_after);
/* Geometry of the CPU oracle's pairwise-summation tree (reference
 * pairwise_sum, src/backend/cpu/reduce.h:55-72) as the device kernels lay it
 * out: depth D and the element range [begin, end) of depth-D leaf `leaf`
 * (0 <= leaf < 2^D; empty for the non-leftmost descendants of a leaf that
 * ended above depth D). Summing each leaf from 0.0f and combining leaves
 * adjacent-first reproduces the oracle's additions. */
int vkhip_pairwise_leaf(uint32_t n, uint32_t leaf, uint32_t* out_depth, uint32_t* out_begin,
                        uint32_t* out_end);
/* The exact numerics mode's exp (log_mode 0) or log (log_mode 1) of n host
 * floats, evaluated on the host by the same source the device kernels use:
 * double-precision Cody-Waite/Taylor exp and atanh-series log, bit for bit
 * the CPU oracle's (which fixes the reference's unpinned std::exp/std::log,
 * kernels_reduce.cpp:227-243, to these methods). */
int vkhip_exact_math(const float* host_x, float* host_y, size_t n, int log_mode);
/* n / d as the device kernels compute it (multiply-high by a precomputed
 * magic number; d = 0 returns 0xffffffff). */
uint32_t vkhip_fast_divide(uint32_t n, uint32_t d);
/* The implicit-im2col map the convolution GEMM gathers with: offset (in
 * elements, from the image of one sample) of cols element (row, pos), given
 * the image's channel/row/column strides x_strides[3], or -1 when it falls in
 * the padding. */
int vkhip_im2col_offset(const vkhip_unfold* p, uint32_t channels, const int64_t* x_strides,
                        uint32_t row, uint32_t pos, int64_t* out_offset);
/* The same map as the weight-gradient gather computes it (the transposed
 * columns gathered by LDS-direct loads: a window row's fixed part plus a
 * position's part, bounds-tested): offset of cols element (row, pos) or -1. */
int vkhip_im2col_offset_t(const vkhip_unfold* p, uint32_t channels, const int64_t* x_strides,
                          uint32_t row, uint32_t pos, int64_t* out_offset);
/* Byte offset the straight-to-LDS (KCD) loader reads for 16-byte slot `slot`
 * of a stage of an operand with row stride s_row (elements), rows from row0,
 * K-tile k0 of kdim; 0x80000000 when the row or k-group is past the operand
 * (read as zeros). The loader requires kdim a multiple of four and 16-byte
 * aligned rows; tests replay it to check every access is aligned and inside
 * the operand. */
uint32_t vkhip_kcd_slot_offset(uint32_t slot, int64_t s_row, uint32_t row0, uint32_t rows,
                               uint32_t k0, uint32_t kdim);

#ifdef __cplusplus
}
#endif

#endif /* VKHIP_H */
