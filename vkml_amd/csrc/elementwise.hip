// Elementwise support ops the training steps need on the device (the
// reference has no CPU fallback, executor.cpp:107-124): unary (neg, exp, log,
// relu, copy), binary (add, sub, mul, div, maximum, minimum, scaled_add),
// comparisons -> bool, where, cast, fill, arange.
//
// Semantics follow the CPU oracle (reference kernels_elementwise.cpp:160-300,
// kernels_movement.cpp:100-200): relu is `x <= 0 ? 0 : x` (NaN propagates);
// maximum/minimum return NaN if either side is NaN; scaled_add is two rounded
// multiplies and one rounded add (never an FMA); arange computes start + i*step
// in double and rounds once. Outputs are contiguous; sources arrive already
// broadcast to the output extents as strides (stride 0 on broadcast axes).
#include "common.h"

namespace vkhip {

// How a source's offset follows the output's linear index.
enum SrcMode : int32_t {
    kContig = 0,  // offset == index
    kScalar = 1,  // every stride 0 (a broadcast scalar)
    kStrided = 2  // sum over the output's rank-4 coordinates times the strides
};

struct Src {
    const void* p;
    int32_t dtype;
    int32_t mode;
    int64_t nb[4];
};

struct EwArgs {
    int32_t op;
    int32_t out_dtype;
    void* out;
    uint64_t n;
    Src s[3];
    float alpha, beta;
    double d0, d1;
    // The output's rank-4 extents and launch-time divisions by the inner three
    // (outputs with 2^32 elements or more decode with 64-bit division).
    uint32_t ne[4];
    FastDiv dv[3];  // by ne[3], ne[2], ne[1]
    int32_t wide;
    int32_t exact;  // exact numerics mode: the oracle's exp and log
};

// Coordinates of output element i (computed once, shared by every source).
struct Coord {
    uint32_t c[4];
};

__device__ __forceinline__ Coord coord_of(const EwArgs& a, uint64_t i) {
    Coord k;
    if (a.wide) {
        uint64_t q = i;
        for (int d = 3; d >= 1; --d) {
            k.c[d] = static_cast<uint32_t>(q % a.ne[d]);
            q /= a.ne[d];
        }
        k.c[0] = static_cast<uint32_t>(q);
        return k;
    }
    uint32_t q = static_cast<uint32_t>(i);
    uint32_t qn = a.dv[0].div(q);
    k.c[3] = q - qn * a.ne[3];
    q = qn;
    qn = a.dv[1].div(q);
    k.c[2] = q - qn * a.ne[2];
    q = qn;
    qn = a.dv[2].div(q);
    k.c[1] = q - qn * a.ne[1];
    k.c[0] = qn;
    return k;
}

__device__ __forceinline__ int64_t src_off(const Src& s, uint64_t i, const Coord& k) {
    if (s.mode == kContig) return static_cast<int64_t>(i);
    if (s.mode == kScalar) return 0;
    return static_cast<int64_t>(k.c[0]) * s.nb[0] + static_cast<int64_t>(k.c[1]) * s.nb[1] +
           static_cast<int64_t>(k.c[2]) * s.nb[2] + static_cast<int64_t>(k.c[3]) * s.nb[3];
}

__device__ __forceinline__ float load_f(const Src& s, uint64_t i, const Coord& k) {
    const int64_t off = src_off(s, i, k);
    switch (s.dtype) {
        case VKHIP_I64: return static_cast<float>(static_cast<const int64_t*>(s.p)[off]);
        case VKHIP_BOOL: return static_cast<const uint8_t*>(s.p)[off] != 0 ? 1.0f : 0.0f;
        case VKHIP_I32: return static_cast<float>(static_cast<const int32_t*>(s.p)[off]);
        default: return static_cast<const float*>(s.p)[off];
    }
}

__device__ __forceinline__ void store_out(const EwArgs& a, uint64_t i, float v) {
    switch (a.out_dtype) {
        case VKHIP_I64: static_cast<int64_t*>(a.out)[i] = static_cast<int64_t>(v); break;
        case VKHIP_BOOL: static_cast<uint8_t*>(a.out)[i] = v != 0.0f ? 1 : 0; break;
        default: static_cast<float*>(a.out)[i] = v; break;
    }
}

__global__ __launch_bounds__(256) void elementwise_kernel(EwArgs a) {
    const uint64_t base = (static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint64_t i = base + j;
        if (i >= a.n) return;
        Coord k{};
        if (a.s[0].mode == kStrided || a.s[1].mode == kStrided || a.s[2].mode == kStrided)
            k = coord_of(a, i);
        switch (a.op) {
            case VKHIP_OP_FULL:
                if (a.out_dtype == VKHIP_I64)
                    static_cast<int64_t*>(a.out)[i] = static_cast<int64_t>(a.d0);
                else if (a.out_dtype == VKHIP_BOOL)
                    static_cast<uint8_t*>(a.out)[i] = a.d0 != 0.0 ? 1 : 0;
                else
                    static_cast<float*>(a.out)[i] = static_cast<float>(a.d0);
                break;
            case VKHIP_OP_ARANGE: {
                const double v = a.d0 + static_cast<double>(i) * a.d1;
                if (a.out_dtype == VKHIP_I64)
                    static_cast<int64_t*>(a.out)[i] = static_cast<int64_t>(v);
                else
                    static_cast<float*>(a.out)[i] = static_cast<float>(v);
                break;
            }
            case VKHIP_OP_CONTIGUOUS:
                if (a.out_dtype == VKHIP_I64)
                    static_cast<int64_t*>(a.out)[i] =
                        static_cast<const int64_t*>(a.s[0].p)[src_off(a.s[0], i, k)];
                else if (a.out_dtype == VKHIP_BOOL)
                    static_cast<uint8_t*>(a.out)[i] =
                        static_cast<const uint8_t*>(a.s[0].p)[src_off(a.s[0], i, k)];
                else
                    static_cast<float*>(a.out)[i] =
                        static_cast<const float*>(a.s[0].p)[src_off(a.s[0], i, k)];
                break;
            case VKHIP_OP_CAST:
                if (a.s[0].dtype == VKHIP_F32 && a.out_dtype == VKHIP_I64)
                    static_cast<int64_t*>(a.out)[i] = static_cast<int64_t>(
                        static_cast<const float*>(a.s[0].p)[src_off(a.s[0], i, k)]);
                else
                    store_out(a, i, load_f(a.s[0], i, k));
                break;
            case VKHIP_OP_NEG: store_out(a, i, -load_f(a.s[0], i, k)); break;
            case VKHIP_OP_EXP: {
                const float x = load_f(a.s[0], i, k);
                store_out(a, i, a.exact ? exact_expf(x) : expf(x));
                break;
            }
            case VKHIP_OP_LOG: {
                const float x = load_f(a.s[0], i, k);
                store_out(a, i, a.exact ? exact_logf(x) : logf(x));
                break;
            }
            case VKHIP_OP_RELU: {
                const float x = load_f(a.s[0], i, k);
                store_out(a, i, x <= 0.0f ? 0.0f : x);
                break;
            }
            case VKHIP_OP_RELU_BACKWARD: {
                const float x = load_f(a.s[0], i, k);
                store_out(a, i, x <= 0.0f ? 0.0f : load_f(a.s[1], i, k));
                break;
            }
            case VKHIP_OP_ADD: store_out(a, i, __fadd_rn(load_f(a.s[0], i, k), load_f(a.s[1], i, k))); break;
            case VKHIP_OP_ADD_RELU: {
                const float v = __fadd_rn(load_f(a.s[0], i, k), load_f(a.s[1], i, k));
                store_out(a, i, v <= 0.0f ? 0.0f : v);
                break;
            }
            case VKHIP_OP_SUB: store_out(a, i, __fsub_rn(load_f(a.s[0], i, k), load_f(a.s[1], i, k))); break;
            case VKHIP_OP_MUL: store_out(a, i, __fmul_rn(load_f(a.s[0], i, k), load_f(a.s[1], i, k))); break;
            case VKHIP_OP_DIV: store_out(a, i, load_f(a.s[0], i, k) / load_f(a.s[1], i, k)); break;
            case VKHIP_OP_SCALED_ADD:
                store_out(a, i,
                          __fadd_rn(__fmul_rn(load_f(a.s[0], i, k), a.alpha),
                                    __fmul_rn(load_f(a.s[1], i, k), a.beta)));
                break;
            case VKHIP_OP_MAXIMUM:
            case VKHIP_OP_MINIMUM: {
                const float x = load_f(a.s[0], i, k), y = load_f(a.s[1], i, k);
                float r;
                if (x != x || y != y)
                    r = __builtin_nanf("");
                else if (a.op == VKHIP_OP_MAXIMUM)
                    r = x > y ? x : y;
                else
                    r = x < y ? x : y;
                store_out(a, i, r);
                break;
            }
            case VKHIP_OP_EQUAL:
            case VKHIP_OP_LESS:
            case VKHIP_OP_GREATER:
            case VKHIP_OP_LESS_EQUAL:
            case VKHIP_OP_GREATER_EQUAL:
            case VKHIP_OP_NOT_EQUAL: {
                const float x = load_f(a.s[0], i, k), y = load_f(a.s[1], i, k);
                bool r = false;
                switch (a.op) {
                    case VKHIP_OP_EQUAL: r = x == y; break;
                    case VKHIP_OP_LESS: r = x < y; break;
                    case VKHIP_OP_GREATER: r = x > y; break;
                    case VKHIP_OP_LESS_EQUAL: r = x <= y; break;
                    case VKHIP_OP_GREATER_EQUAL: r = x >= y; break;
                    default: r = x != y; break;
                }
                static_cast<uint8_t*>(a.out)[i] = r ? 1 : 0;
                break;
            }
            case VKHIP_OP_WHERE: {
                const bool c = static_cast<const uint8_t*>(a.s[0].p)[src_off(a.s[0], i, k)] != 0;
                store_out(a, i, c ? load_f(a.s[1], i, k) : load_f(a.s[2], i, k));
                break;
            }
            default: break;
        }
    }
}

// Contiguous f32 fast path for the ops on the optimiser and activation paths:
// 16-byte loads and stores, no index decoding.
__global__ __launch_bounds__(256) void elementwise_f32_vec_kernel(int op, const float* __restrict__ x,
                                                                  const float* __restrict__ y,
                                                                  float* __restrict__ out,
                                                                  uint64_t n4, float alpha,
                                                                  float beta) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    const f32x4 a = reinterpret_cast<const f32x4*>(x)[i];
    f32x4 b = {0.0f, 0.0f, 0.0f, 0.0f};
    if (y) b = reinterpret_cast<const f32x4*>(y)[i];
    f32x4 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        switch (op) {
            case VKHIP_OP_ADD: r[j] = __fadd_rn(a[j], b[j]); break;
            case VKHIP_OP_ADD_RELU: {
                const float v = __fadd_rn(a[j], b[j]);
                r[j] = v <= 0.0f ? 0.0f : v;
                break;
            }
            case VKHIP_OP_SUB: r[j] = __fsub_rn(a[j], b[j]); break;
            case VKHIP_OP_MUL: r[j] = __fmul_rn(a[j], b[j]); break;
            case VKHIP_OP_SCALED_ADD:
                r[j] = __fadd_rn(__fmul_rn(a[j], alpha), __fmul_rn(b[j], beta));
                break;
            case VKHIP_OP_RELU: r[j] = a[j] <= 0.0f ? 0.0f : a[j]; break;
            case VKHIP_OP_RELU_BACKWARD: r[j] = a[j] <= 0.0f ? 0.0f : b[j]; break;
            case VKHIP_OP_NEG: r[j] = -a[j]; break;
            default: r[j] = a[j]; break;  // contiguous copy
        }
    }
    reinterpret_cast<f32x4*>(out)[i] = r;
}

// Binary f32 ops whose second operand is broadcast in one of the two shapes
// bias adds take, with 16-byte loads and stores of the first operand and the
// output (both contiguous):
//   PERIODIC: y repeats with period `inner` (y's trailing axes contiguous, its
//             leading axes broadcast): y index = i % inner, e.g. [N,F] + [F];
//   RUNS:     y is constant over runs of `inner` elements (its trailing axes
//             broadcast) and indexed by the run number through the leading
//             axes' strides `lead`, e.g. [N,C,H,W] + [C,1,1].
// inner is a multiple of 4, so a thread's four elements share one run (RUNS)
// or read four consecutive y values (PERIODIC).
template <bool RUNS>
__global__ __launch_bounds__(256) void elementwise_bcast_vec_kernel(
    int op, const float* __restrict__ x, const float* __restrict__ y, float* __restrict__ out,
    uint64_t n4, uint32_t inner, FastDiv div_inner, Op4 lead) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    const uint64_t e0 = 4 * i;
    const f32x4 a = reinterpret_cast<const f32x4*>(x)[i];
    f32x4 b;
    if constexpr (RUNS) {
        const uint32_t run = div_inner.div(static_cast<uint32_t>(e0));
        const float v = y[lin_off4(run, lead.ne, lead.nb)];
        b = f32x4{v, v, v, v};
    } else {
        const uint32_t q = div_inner.div(static_cast<uint32_t>(e0));
        const uint32_t r = static_cast<uint32_t>(e0) - q * inner;
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = y[r + j];
    }
    f32x4 res;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        switch (op) {
            case VKHIP_OP_ADD: res[j] = __fadd_rn(a[j], b[j]); break;
            case VKHIP_OP_ADD_RELU: {
                const float v = __fadd_rn(a[j], b[j]);
                res[j] = v <= 0.0f ? 0.0f : v;
                break;
            }
            case VKHIP_OP_SUB: res[j] = __fsub_rn(a[j], b[j]); break;
            default: res[j] = __fmul_rn(a[j], b[j]); break;
        }
    }
    reinterpret_cast<f32x4*>(out)[i] = res;
}

static bool is_contig(const vkhip_tensor& t) {
    int64_t expect = 1;
    for (int i = t.ndim - 1; i >= 0; --i) {
        if (t.ne[i] == 1) continue;
        if (t.nb[i] != expect) return false;
        expect *= t.ne[i];
    }
    return true;
}

static uint64_t tnumel(const vkhip_tensor& t) {
    uint64_t n = 1;
    for (int i = 0; i < t.ndim; ++i) n *= static_cast<uint64_t>(t.ne[i]);
    return n;
}

// Sources arrive with the output's extents (broadcast axes have stride 0).
static Src make_src(const vkhip_tensor& t) {
    Src s{};
    s.p = t.data;
    s.dtype = t.dtype;
    const int pad = 4 - t.ndim;
    bool scalar = true;
    for (int i = 0; i < t.ndim; ++i) {
        s.nb[pad + i] = t.nb[i];
        if (t.ne[i] != 1 && t.nb[i] != 0) scalar = false;
    }
    s.mode = is_contig(t) ? kContig : scalar ? kScalar : kStrided;
    return s;
}

// Materialising a transposed view: out [B0, B1, R, C] contiguous from a
// source whose element (b0, b1, r, c) sits at b0*s0 + b1*s1 + r + c*sc (unit
// stride down the rows: a transpose of the last two axes, as autograd's
// weight gradients of x @ w.T arrive). 64x64 tiles through LDS so that both
// the reads (along r) and the writes (along c) are contiguous; the generic
// strided copy reads a 4-byte element per cache line.
__global__ __launch_bounds__(256) void transpose_copy_kernel(const float* __restrict__ src, int64_t s0,
                                                             int64_t s1, int64_t sc,
                                                             float* __restrict__ dst, uint32_t b1n,
                                                             uint32_t R, uint32_t C, uint32_t tiles_c) {
    __shared__ float tile[64][65];
    const uint32_t t = threadIdx.x;
    const uint32_t tr = blockIdx.x / tiles_c, tc = blockIdx.x - tr * tiles_c;
    const uint32_t r0 = tr * 64, c0 = tc * 64;
    const uint32_t b = blockIdx.y, b0 = b / b1n, b1 = b - b0 * b1n;
    const float* sp = src + static_cast<int64_t>(b0) * s0 + static_cast<int64_t>(b1) * s1;
    float* dp = dst + static_cast<uint64_t>(b) * R * C;
    const uint32_t lr = t & 63, lc = t >> 6;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t c = c0 + lc + 4 * i, r = r0 + lr;
        if (c < C && r < R) tile[lc + 4 * i][lr] = sp[static_cast<int64_t>(c) * sc + r];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t r = r0 + lc + 4 * i, c = c0 + lr;
        if (c < C && r < R) dp[static_cast<uint64_t>(r) * C + c] = tile[lr][lc + 4 * i];
    }
}

int launch_elementwise(const vkhip_node& nd) {
    const uint64_t n = tnumel(nd.out);
    if (n == 0) return VKHIP_OK;
    float ab[2] = {1.0f, 1.0f};
    double dd[2] = {0.0, 0.0};
    memcpy(ab, nd.params, sizeof ab);
    memcpy(dd, nd.params, sizeof dd);
    hipStream_t st = ctx().stream;

    // Vector fast path: f32, everything contiguous and 16-byte aligned.
    const int op = nd.op;
    const bool vec_op = op == VKHIP_OP_ADD || op == VKHIP_OP_ADD_RELU || op == VKHIP_OP_SUB || op == VKHIP_OP_MUL ||
                        op == VKHIP_OP_SCALED_ADD || op == VKHIP_OP_RELU || op == VKHIP_OP_NEG ||
                        op == VKHIP_OP_CONTIGUOUS || op == VKHIP_OP_RELU_BACKWARD;
    if (vec_op && n % 4 == 0 && nd.out.dtype == VKHIP_F32) {
        bool ok = reinterpret_cast<uintptr_t>(nd.out.data) % 16 == 0;
        for (int s = 0; s < nd.n_src && ok; ++s)
            ok = nd.src[s].dtype == VKHIP_F32 && is_contig(nd.src[s]) && tnumel(nd.src[s]) == n &&
                 reinterpret_cast<uintptr_t>(nd.src[s].data) % 16 == 0;
        if (ok) {
            const uint64_t n4 = n / 4;
            hipLaunchKernelGGL(elementwise_f32_vec_kernel, dim3(ceil_div(n4, 256)), dim3(256), 0, st,
                               op, static_cast<const float*>(nd.src[0].data),
                               nd.n_src > 1 ? static_cast<const float*>(nd.src[1].data) : nullptr,
                               static_cast<float*>(nd.out.data), n4, ab[0], ab[1]);
            VKHIP_LAUNCH_CHECK();
            return VKHIP_OK;
        }
    }
    // A transposed view made contiguous (transpose_copy_kernel).
    if (op == VKHIP_OP_CONTIGUOUS && nd.out.dtype == VKHIP_F32 && nd.src[0].dtype == VKHIP_F32 &&
        nd.out.ndim >= 2 && nd.out.ndim <= 4 && is_contig(nd.out)) {
        const vkhip_tensor& x = nd.src[0];
        const int d = x.ndim;
        const int64_t R = x.ne[d - 2], C = x.ne[d - 1];
        if (x.nb[d - 2] == 1 && x.nb[d - 1] != 1 && C > 1 && R > 1 && R < (1ll << 31) && C < (1ll << 31)) {
            int64_t b0n = 1, b1n = 1, s0 = 0, s1 = 0;
            if (d == 3) {
                b1n = x.ne[0];
                s1 = x.nb[0];
            } else if (d == 4) {
                b0n = x.ne[0];
                s0 = x.nb[0];
                b1n = x.ne[1];
                s1 = x.nb[1];
            }
            const uint32_t tiles_c = static_cast<uint32_t>((C + 63) / 64);
            const uint64_t tiles = static_cast<uint64_t>(tiles_c) * ((R + 63) / 64);
            if (tiles <= 0x7fffffffull && b0n * b1n <= 65535) {
                hipLaunchKernelGGL(transpose_copy_kernel, dim3(static_cast<uint32_t>(tiles),
                                                               static_cast<uint32_t>(b0n * b1n)),
                                   dim3(256), 0, st, static_cast<const float*>(x.data), s0, s1,
                                   x.nb[d - 1], static_cast<float*>(nd.out.data),
                                   static_cast<uint32_t>(b1n), static_cast<uint32_t>(R),
                                   static_cast<uint32_t>(C), tiles_c);
                VKHIP_LAUNCH_CHECK();
                return VKHIP_OK;
            }
        }
    }
    // Broadcast second operand of a bias add (see elementwise_bcast_vec_kernel).
    if ((op == VKHIP_OP_ADD || op == VKHIP_OP_ADD_RELU || op == VKHIP_OP_SUB || op == VKHIP_OP_MUL) &&
        nd.n_src == 2 &&
        n % 4 == 0 && n < (1ull << 32) && nd.out.dtype == VKHIP_F32 &&
        nd.src[0].dtype == VKHIP_F32 && nd.src[1].dtype == VKHIP_F32 &&
        is_contig(nd.src[0]) && tnumel(nd.src[0]) == n &&
        reinterpret_cast<uintptr_t>(nd.out.data) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(nd.src[0].data) % 16 == 0) {
        const vkhip_tensor& y = nd.src[1];
        // Trailing axes where y is broadcast (stride 0), then where it is
        // contiguous; extent-1 axes are skipped.
        int axis = y.ndim - 1;
        uint64_t zero_run = 1, contig_run = 1;
        while (axis >= 0 && (y.ne[axis] == 1 || y.nb[axis] == 0)) zero_run *= y.ne[axis--];
        const int lead_end = axis;  // axes [0, lead_end] remain
        if (zero_run > 1 && zero_run % 4 == 0 && lead_end >= 0) {
            // RUNS: y indexed by the run number through its leading axes.
            Op4 lead{};
            for (int i = 0; i < 4; ++i) {
                lead.ne[i] = 1;
                lead.nb[i] = 0;
            }
            const int pad = 3 - lead_end;
            bool fits = pad >= 0;
            for (int i = 0; i <= lead_end && fits; ++i) {
                lead.ne[pad + i] = static_cast<uint32_t>(y.ne[i]);
                lead.nb[pad + i] = y.nb[i];
            }
            if (fits) {
                const uint64_t n4 = n / 4;
                hipLaunchKernelGGL(elementwise_bcast_vec_kernel<true>, dim3(ceil_div(n4, 256)),
                                   dim3(256), 0, st, op, static_cast<const float*>(nd.src[0].data),
                                   static_cast<const float*>(y.data), static_cast<float*>(nd.out.data),
                                   n4, static_cast<uint32_t>(zero_run),
                                   FastDiv(static_cast<uint32_t>(zero_run)), lead);
                VKHIP_LAUNCH_CHECK();
                return VKHIP_OK;
            }
        }
        if (zero_run == 1) {
            // PERIODIC: a contiguous trailing block of y, broadcast over the rest.
            axis = y.ndim - 1;
            while (axis >= 0 && (y.ne[axis] == 1 || static_cast<uint64_t>(y.nb[axis]) == contig_run)) {
                contig_run *= y.ne[axis];
                --axis;
            }
            bool rest_broadcast = true;
            for (int i = 0; i <= axis; ++i)
                if (y.ne[i] != 1 && y.nb[i] != 0) rest_broadcast = false;
            if (rest_broadcast && contig_run % 4 == 0 && contig_run < n) {
                const uint64_t n4 = n / 4;
                hipLaunchKernelGGL(elementwise_bcast_vec_kernel<false>, dim3(ceil_div(n4, 256)),
                                   dim3(256), 0, st, op, static_cast<const float*>(nd.src[0].data),
                                   static_cast<const float*>(y.data), static_cast<float*>(nd.out.data),
                                   n4, static_cast<uint32_t>(contig_run),
                                   FastDiv(static_cast<uint32_t>(contig_run)), Op4{});
                VKHIP_LAUNCH_CHECK();
                return VKHIP_OK;
            }
        }
    }
    EwArgs a{};
    a.op = op;
    a.out_dtype = nd.out.dtype;
    a.exact = ctx().exact_math;
    a.out = nd.out.data;
    a.n = n;
    for (int s = 0; s < nd.n_src && s < 3; ++s) a.s[s] = make_src(nd.src[s]);
    for (int s = nd.n_src; s < 3; ++s) a.s[s].mode = kContig;
    {
        const int pad = 4 - nd.out.ndim;
        for (int i = 0; i < 4; ++i) a.ne[i] = 1;
        for (int i = 0; i < nd.out.ndim; ++i) a.ne[pad + i] = static_cast<uint32_t>(nd.out.ne[i]);
        a.dv[0] = FastDiv(a.ne[3]);
        a.dv[1] = FastDiv(a.ne[2]);
        a.dv[2] = FastDiv(a.ne[1]);
        a.wide = n >= (1ull << 32) ? 1 : 0;
    }
    a.alpha = ab[0];
    a.beta = ab[1];
    a.d0 = dd[0];
    a.d1 = dd[1];
    const uint64_t threads = (n + 3) / 4;
    hipLaunchKernelGGL(elementwise_kernel, dim3(ceil_div(threads, 256)), dim3(256), 0, st, a);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

// Plain 16-byte copy: the batched device-to-device copy, and the kernel whose
// measured bandwidth and HBM byte counters calibrate every other kernel's.
__global__ __launch_bounds__(256) void copy16_kernel(const f32x4_t* __restrict__ src,
                                                     f32x4_t* __restrict__ dst, uint64_t n16) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16;
         i += stride)
        dst[i] = src[i];
}

// Zero-fill of `count` floats: a kernel rather than hipMemsetAsync, so the
// launch sequence stays free of memset nodes when a caller captures the stream
// into a graph.
__global__ __launch_bounds__(256) void zero_f32_kernel(float* __restrict__ dst, uint64_t count) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride)
        dst[i] = 0.0f;
}

int launch_zero_f32(float* dst, uint64_t count) {
    if (count == 0) return VKHIP_OK;
    const uint64_t want = (count + 255) / 256;
    const uint32_t blocks = static_cast<uint32_t>(want < 65536 ? want : 65536);
    hipLaunchKernelGGL(zero_f32_kernel, dim3(blocks), dim3(256), 0, ctx().stream, dst, count);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

// Several disjoint copies in one launch (a training step's batch and labels):
// workgroup w copies 256 units of the pair whose [block_start[i],
// block_start[i+1]) range holds w; a unit is 16 bytes for a pair whose
// addresses and size are 16-byte multiples, else one byte.
constexpr int kCopyBatch = 8;
struct CopyBatch {
    const unsigned char* src[kCopyBatch];
    unsigned char* dst[kCopyBatch];
    uint64_t units[kCopyBatch];
    uint32_t block_start[kCopyBatch + 1];
    uint32_t vec;  // bit i: pair i copies 16-byte units
    int n;
};

__global__ __launch_bounds__(256) void copy_batch_kernel(CopyBatch b) {
    const uint32_t w = blockIdx.x;
    int i = 0;
    while (i + 1 < b.n && w >= b.block_start[i + 1]) ++i;
    const uint64_t u = static_cast<uint64_t>(w - b.block_start[i]) * 256u + threadIdx.x;
    if (u >= b.units[i]) return;
    if ((b.vec >> i) & 1u)
        reinterpret_cast<f32x4_t*>(b.dst[i])[u] = reinterpret_cast<const f32x4_t*>(b.src[i])[u];
    else
        b.dst[i][u] = b.src[i][u];
}

int launch_copy_bytes(void* dst, const void* src, size_t nbytes);

// Copies the pairs: those of up to 64 MB (byte copies: 4 KB) in batches of
// kCopyBatch per launch, any other alone.
int launch_copy_pairs(const vkhip_copy* copies, size_t n) {
    CopyBatch b{};
    uint32_t blocks = 0;
    auto flush = [&]() -> int {
        if (b.n == 0) return VKHIP_OK;
        b.block_start[b.n] = blocks;
        hipLaunchKernelGGL(copy_batch_kernel, dim3(blocks), dim3(256), 0, ctx().stream, b);
        VKHIP_LAUNCH_CHECK();
        b = CopyBatch{};
        blocks = 0;
        return VKHIP_OK;
    };
    for (size_t k = 0; k < n; ++k) {
        const vkhip_copy& c = copies[k];
        if (c.nbytes == 0) continue;
        const bool vec = reinterpret_cast<uintptr_t>(c.dst) % 16 == 0 && reinterpret_cast<uintptr_t>(c.src) % 16 == 0 &&
                         c.nbytes % 16 == 0;
        if (vec ? c.nbytes > (size_t{64} << 20) : c.nbytes > 4096) {
            const int st = launch_copy_bytes(c.dst, c.src, c.nbytes);
            if (st != VKHIP_OK) return st;
            continue;
        }
        const uint64_t units = vec ? c.nbytes / 16 : c.nbytes;
        b.src[b.n] = static_cast<const unsigned char*>(c.src);
        b.dst[b.n] = static_cast<unsigned char*>(c.dst);
        b.units[b.n] = units;
        b.block_start[b.n] = blocks;
        if (vec) b.vec |= 1u << b.n;
        blocks += static_cast<uint32_t>((units + 255) / 256);
        if (++b.n == kCopyBatch) {
            const int st = flush();
            if (st != VKHIP_OK) return st;
        }
    }
    return flush();
}

int launch_copy_bytes(void* dst, const void* src, size_t nbytes) {
    if (nbytes == 0) return VKHIP_OK;
    hipStream_t st = ctx().stream;
    if (reinterpret_cast<uintptr_t>(dst) % 16 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
        nbytes % 16 == 0) {
        // One 16-byte element per thread over a one-shot grid: measured the
        // fastest copy shape on MI355X (6.2 TB/s at 1 GiB vs 4.6-5.5 TB/s for
        // grid-stride loops); the loop only runs for grids past 2^31 threads.
        const uint64_t n16 = nbytes / 16;
        const uint64_t want = (n16 + 255) / 256;
        const uint32_t blocks = static_cast<uint32_t>(want < (1u << 23) ? want : (1u << 23));
        hipLaunchKernelGGL(copy16_kernel, dim3(blocks), dim3(256), 0, st,
                           static_cast<const f32x4_t*>(src), static_cast<f32x4_t*>(dst), n16);
        VKHIP_LAUNCH_CHECK();
        return VKHIP_OK;
    }
    VKHIP_HIP(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToDevice, st));
    return VKHIP_OK;
}

// ---- fused SGD step ----------------------------------------------------------------
// One launch updates up to kSgdBatch parameters: workgroup w belongs to the
// parameter whose [block_start[i], block_start[i+1]) range holds w; each thread
// updates 4 consecutive elements. Every expression is a scaled_add as the
// reference optimiser builds it, a*alpha + b*beta with both products and the
// sum rounded separately (multiplies by 1.0 are exact and left out).
constexpr int kSgdBatch = 64;

struct SgdBatch {
    vkhip_sgd_param p[kSgdBatch];
    uint32_t block_start[kSgdBatch + 1];
    int32_t count;
    float lr, momentum, weight_decay;
    int32_t nesterov;
};

// One parameter element's update (torch.optim.SGD's order of operations).
__device__ __forceinline__ void sgd_update(float& p, float g, float& v, bool first, const SgdBatch& b) {
    if (b.weight_decay != 0.0f) g = __fadd_rn(g, __fmul_rn(p, b.weight_decay));
    float dir = g;
    if (b.momentum != 0.0f) {
        v = first ? g : __fadd_rn(__fmul_rn(v, b.momentum), g);
        dir = b.nesterov ? __fadd_rn(g, __fmul_rn(v, b.momentum)) : v;
    }
    p = __fadd_rn(p, __fmul_rn(dir, -b.lr));
}

// Four consecutive elements per thread: one 16-byte load and store per
// buffer when the parameter's buffers are 16-byte aligned and the four are
// in range, else element by element.
__global__ __launch_bounds__(256) void sgd_step_kernel(SgdBatch b) {
    int i = 0;
    while (i + 1 < b.count && blockIdx.x >= b.block_start[i + 1]) ++i;
    const vkhip_sgd_param& q = b.p[i];
    const uint64_t base = (static_cast<uint64_t>(blockIdx.x - b.block_start[i]) * 256 + threadIdx.x) * 4;
    if (base >= q.n) return;
    const bool mom = b.momentum != 0.0f;
    const bool aligned = ((reinterpret_cast<uintptr_t>(q.param) | reinterpret_cast<uintptr_t>(q.grad) |
                           (mom ? reinterpret_cast<uintptr_t>(q.velocity) : 0)) & 15) == 0;
    if (aligned && base + 4 <= q.n) {
        f32x4_t p = *reinterpret_cast<const f32x4_t*>(q.param + base);
        const f32x4_t g = *reinterpret_cast<const f32x4_t*>(q.grad + base);
        f32x4_t v = {0.0f, 0.0f, 0.0f, 0.0f};
        if (mom && !q.first) v = *reinterpret_cast<const f32x4_t*>(q.velocity + base);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float pj = p[j], vj = v[j];
            sgd_update(pj, g[j], vj, q.first, b);
            p[j] = pj;
            v[j] = vj;
        }
        if (mom) *reinterpret_cast<f32x4_t*>(q.velocity + base) = v;
        *reinterpret_cast<f32x4_t*>(q.param + base) = p;
        return;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint64_t e = base + j;
        if (e >= q.n) return;
        float p = q.param[e];
        float v = mom && !q.first ? q.velocity[e] : 0.0f;
        sgd_update(p, q.grad[e], v, q.first, b);
        if (mom) q.velocity[e] = v;
        q.param[e] = p;
    }
}

int launch_sgd_step(const vkhip_sgd_param* params, size_t count, float lr, float momentum,
                    float weight_decay, int nesterov) {
    for (size_t at = 0; at < count; at += kSgdBatch) {
        SgdBatch b{};
        b.count = static_cast<int32_t>(count - at < kSgdBatch ? count - at : kSgdBatch);
        b.lr = lr;
        b.momentum = momentum;
        b.weight_decay = weight_decay;
        b.nesterov = nesterov ? 1 : 0;
        uint64_t blocks = 0;
        for (int i = 0; i < b.count; ++i) {
            const vkhip_sgd_param& q = params[at + i];
            if (q.n && (!q.param || !q.grad || (momentum != 0.0f && !q.velocity)))
                return fail(VKHIP_ERR_INVALID, "sgd_step: parameter %zu has a null buffer", at + i);
            b.p[i] = q;
            b.block_start[i] = static_cast<uint32_t>(blocks);
            blocks += (q.n + 1023) / 1024;
            if (blocks > 0x7fffffffull) return fail(VKHIP_ERR_UNSUPPORTED, "sgd_step: too many elements");
        }
        b.block_start[b.count] = static_cast<uint32_t>(blocks);
        if (blocks == 0) continue;
        hipLaunchKernelGGL(sgd_step_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                           ctx().stream, b);
        VKHIP_LAUNCH_CHECK();
    }
    return VKHIP_OK;
}

}  // namespace vkhip

extern "C" int vkhip_scaled_add(const float* a, const float* b, float* out, uint64_t n, float alpha,
                                float beta) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::Unit unit("scaled_add");
    vkhip_node nd{};
    nd.op = VKHIP_OP_SCALED_ADD;
    nd.n_src = 2;
    auto flat = [n](vkhip_tensor& t, const void* p) {
        t.data = const_cast<void*>(p);
        t.dtype = VKHIP_F32;
        t.ndim = 1;
        t.ne[0] = static_cast<int64_t>(n);
        t.nb[0] = 1;
    };
    flat(nd.out, out);
    flat(nd.src[0], a);
    flat(nd.src[1], b);
    memcpy(nd.params, &alpha, sizeof alpha);
    memcpy(nd.params + sizeof alpha, &beta, sizeof beta);
    return vkhip::launch_elementwise(nd);
}

extern "C" int vkhip_sgd_step(const vkhip_sgd_param* params, size_t count, float lr,
                              float momentum, float weight_decay, int nesterov) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::Unit unit("sgd_step");
    if (count && !params) return vkhip::fail(VKHIP_ERR_INVALID, "sgd_step: null parameter list");
    st = vkhip::launch_sgd_step(params, count, lr, momentum, weight_decay, nesterov);
    if (st == VKHIP_OK) vkhip::program_note_sgd(params, count, lr, momentum, weight_decay, nesterov);
    return st;
}
