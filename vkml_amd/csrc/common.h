// Shared runtime state and helpers for the vkhip library (gfx950 only).
//
// One process, one device, one HIP stream: a graph flush becomes an ordered
// launch sequence on that stream, which replaces the Vulkan recorder's per-node
// global barrier (reference vulkan_backend.cpp:2667) with stream order.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstring>
#include <cstdint>
#include <cstdio>
#include <string>

#include "vkhip.h"

namespace vkhip {

// Last error message, per host thread (vkhip_last_error).
void set_error_msg(const char* fmt, ...);
int fail(int code, const char* fmt, ...);

struct Context {
    bool ready = false;
    int device = -1;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;  // where launches go: own_stream or a host-provided one
    // Uploads queued ahead of the stream's work (vkhip_copy_from_host_async),
    // created on first use, default priority.
    hipStream_t copy_stream = nullptr;
    vkhip_caps caps{};
    // Split-K partials workspace, grown on demand and released stream-ordered
    // (reference grows its own the same way, vulkan_backend.cpp:899-919).
    // slot 0: split-K partials and reduction partials; slot 1: a node's own
    // temporaries (which may hold data across a GEMM that uses slot 0);
    // slot 2: a fused node's intermediate, held across the nodes it runs
    // (which may use slots 0 and 1)
    float* ws[3] = {nullptr, nullptr, nullptr};
    size_t ws_bytes[3] = {0, 0, 0};
    int ws_pins = 0;               // captured graphs holding the workspace blocks
    void* ws_retired[64] = {};     // blocks replaced while pinned, freed at the last unpin
    int ws_retired_count = 0;
    // Device address of this device's fixed scratch array (runtime.hip), from
    // hipGetSymbolAddress at init; null if it could not be resolved.
    float* scratch = nullptr;
    // GEMM kernel selection for MATMUL nodes, from VKHIP_GEMM_KERNEL at init
    // ("exact" | "mfma" | unset/"auto"), as the reference's VKML_GEMM_KERNEL
    // selects its GEMM for every matmul in the process (vulkan_backend.cpp:2158-2172).
    int node_gemm_kernel = VKHIP_GEMM_AUTO;
    // VKHIP_NUMERICS_EXACT (vkhip_set_numerics, or VKHIP_NUMERICS=exact at
    // init): GEMMs and convolutions on the exact arm, the shared exp/log and
    // true division in softmax, log-softmax, cross-entropy, exp and log.
    int exact_math = 0;
};

Context& ctx();

// Returns VKHIP_OK or a failure code with the message set.
int require_ready();

// Workspace of at least `bytes` on the current stream (slot 0; slot 1 is
// node_temporary's).
int workspace(size_t bytes, float** out, int slot = 0);
// A node's temporary of at least `bytes` (workspace slot 1): valid until the
// next node that asks for one; work using it is ordered on the stream.
inline int node_temporary(size_t bytes, float** out) { return workspace(bytes, out, 1); }
// A fused node's intermediate (workspace slot 2): valid until the next call.
inline int fused_intermediate(size_t bytes, float** out) { return workspace(bytes, out, 2); }
// While pinned (a captured HIP graph holds the current blocks), a workspace
// that must grow gets a new block and keeps the old one until the last pin
// goes, and the implicit-im2col row tables are not evicted.
int pin_workspaces(int delta);
bool workspaces_pinned();

// Recorded programs (program.hip): the calls that enqueue work on tensors
// note themselves after they succeed; no-ops unless a program is recording.
bool program_recording();
void program_note_compute(const vkhip_node* nodes, size_t n);
void program_note_sgd(const vkhip_sgd_param* params, size_t count, float lr, float momentum,
                      float weight_decay, int nesterov);
void program_note_copy(const vkhip_copy* copies, size_t n);
// Per-unit event timing is on (observe.hip).
bool profiling_on();

// A caller-fixed split-K workspace (the allocation-free GEMM entry point's
// per-device scratch array): gemm() uses it instead of growing workspace()
// and refuses a plan that needs more than `bytes`.
struct FixedScratch {
    float* ptr;
    size_t bytes;
};
// A product's epilogue: out[.., col] = relu?(out + bias[col * bias_stride]),
// the values of the ADD of a bias broadcast over rows and the RELU after it;
// or, with mask set (laid out as the output), out = mask <= 0 ? +0 : out, the
// relu gradient of a relu whose output gradient is the product.
struct GemmEpilogue {
    const float* bias;
    int64_t bias_stride;
    bool relu;
    const float* mask = nullptr;
};
int gemm(const float* a, const vkhip_operand& ad, const float* b, const vkhip_operand& bd, float* c,
         const vkhip_gemm_opts* opts, const FixedScratch* scratch = nullptr,
         const GemmEpilogue* epi = nullptr);

// Decision facts and units of work (observe.hip). A unit is a node of
// vkhip_compute or one per-op entry call; decisions published inside it carry
// its dispatch id.
void publish(const char* site, const char* op, const char* chose, const char* instead_of,
             const char* because, int64_t required, int64_t available);
void unit_begin(const char* label);
void unit_end();
struct Unit {
    explicit Unit(const char* label) { unit_begin(label); }
    ~Unit() { unit_end(); }
    Unit(const Unit&) = delete;
    Unit& operator=(const Unit&) = delete;
};

// Zero-fill of `count` floats on the backend stream (elementwise.hip).
int launch_zero_f32(float* dst, uint64_t count);

// The caching allocator behind vkhip_alloc / vkhip_free (allocator.hip).
int cached_alloc(size_t nbytes, void** out);
int cached_free(void* ptr);
int release_cached();
// Frees the cached implicit-im2col row tables (gemm.hip); before release_cached at shutdown.
int release_conv_tables();
void memory_stats(size_t* live, size_t* cached);

#define VKHIP_HIP(expr)                                                                   \
    do {                                                                                  \
        hipError_t e_ = (expr);                                                           \
        if (e_ != hipSuccess)                                                             \
            return ::vkhip::fail(VKHIP_ERR_DEVICE, "%s failed: %s (%s:%d)", #expr,         \
                                 hipGetErrorString(e_), __FILE__, __LINE__);              \
    } while (0)

#define VKHIP_LAUNCH_CHECK()                                                              \
    do {                                                                                  \
        hipError_t e_ = hipGetLastError();                                                \
        if (e_ != hipSuccess)                                                             \
            return ::vkhip::fail(VKHIP_ERR_DEVICE, "kernel launch failed: %s (%s:%d)",    \
                                 hipGetErrorString(e_), __FILE__, __LINE__);              \
    } while (0)

inline uint32_t ceil_div(uint64_t a, uint64_t b) { return static_cast<uint32_t>((a + b - 1) / b); }

// ---- device helpers --------------------------------------------------------

// Offset (elements) of the `linear`-th element, row-major, of a rank-4
// operand (reference linear_to_offset, src/backend/cpu/iterate.h:33-42).
// `linear` < 2^32 at every caller (output counts are checked on the host),
// so 32-bit division suffices; axes of extent 1 (the usual case) are skipped.
__device__ __forceinline__ int64_t lin_off4(uint32_t linear, const uint32_t ne[4],
                                            const int64_t nb[4]) {
    int64_t off = 0;
#pragma unroll
    for (int i = 3; i >= 0; --i) {
        const uint32_t e = ne[i];
        if (e == 1) continue;
        const uint32_t q = linear / e;
        off += static_cast<int64_t>(linear - q * e) * nb[i];
        linear = q;
    }
    return off;
}

// Rank-4 operand passed by value to kernels.
struct Op4 {
    uint32_t ne[4];
    int64_t nb[4];
};

inline Op4 to_op4(const vkhip_operand& d) {
    Op4 o;
    for (int i = 0; i < 4; ++i) {
        o.ne[i] = d.ne[i];
        o.nb[i] = d.nb[i];
    }
    return o;
}

inline uint64_t numel(const vkhip_operand& d) {
    return static_cast<uint64_t>(d.ne[0]) * d.ne[1] * d.ne[2] * d.ne[3];
}

// Pairwise-summation geometry, shared by every kernel that reproduces the CPU
// oracle's association (reference pairwise_sum, src/backend/cpu/reduce.h:55-72:
// split [b,e) at b + n/2 until n <= 32, sum each leaf sequentially from 0).
//
// The recursion tree is laid out as a complete binary tree of depth D, where D
// is the smallest depth at which every range has <= 32 elements. Leaf j (0..2^D-1)
// follows the bits of j from the top; a range that became a leaf at a shallower
// depth is carried whole by its leftmost depth-D descendant, and every other
// descendant carries +0.0. Adding +0.0 is exact for every sum that starts from
// +0.0 (such a sum is never -0.0), so combining the 2^D leaf values pairwise,
// adjacent first, performs exactly the oracle's additions.
__host__ __device__ __forceinline__ int pairwise_depth(uint32_t n) {
    int d = 0;
    // ceil(n / 2^d) is the largest range at depth d.
    while (((static_cast<uint64_t>(n) + (1ull << d) - 1) >> d) > 32u) ++d;
    return d;
}

// Range [begin, end) of depth-D leaf `j` of a length-n pairwise tree; empty
// (begin == end) for descendants of a shallower leaf other than its leftmost.
__host__ __device__ __forceinline__ void pairwise_leaf(uint32_t n, int depth, uint32_t j,
                                                       uint32_t& begin, uint32_t& end) {
    uint32_t b = 0, e = n;
    for (int lvl = depth - 1; lvl >= 0; --lvl) {
        const uint32_t bit = (j >> lvl) & 1u;
        if (e - b <= 32u) {
            // Already a leaf: only the all-zeros path below it carries it.
            if (j & ((2u << lvl) - 1u)) {
                b = e;
            }
            break;
        }
        const uint32_t mid = b + (e - b) / 2;
        if (bit) {
            b = mid;
        } else {
            e = mid;
        }
    }
    begin = b;
    end = e;
}

// ---- division by a runtime-constant divisor -----------------------------------
// Unsigned 32-bit division by a divisor fixed at launch, as one multiply-high,
// a subtract, an add and two shifts (the round-up multiplier method from
// Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994). Exact for every 32-bit numerator.
struct FastDiv {
    uint32_t d, m, s;
    FastDiv() = default;
    __host__ explicit FastDiv(uint32_t divisor) : d(divisor), m(0), s(0) {
        if (d > 1) {
            uint32_t l = 0;
            while ((1ull << l) < d) ++l;  // l = ceil(log2 d)
            s = l;
            m = static_cast<uint32_t>(((1ull << 32) * ((1ull << l) - d)) / d + 1);
        }
    }
    __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
        if (d == 1) return n;
#ifdef __HIP_DEVICE_COMPILE__
        const uint32_t t = __umulhi(m, n);
#else
        const uint32_t t = static_cast<uint32_t>((static_cast<uint64_t>(m) * n) >> 32);
#endif
        return (t + ((n - t) >> 1)) >> (s - 1);
    }
};

// ---- staged rows ------------------------------------------------------------
// A row that is summed in the pairwise order is first staged in LDS with 4
// padding floats after every 32 elements: each full 32-element leaf then starts
// on a 16-byte boundary (read as eight 16-byte loads), and eight consecutive
// leaves start 36 floats apart, which spreads them over distinct LDS banks.
__host__ __device__ __forceinline__ uint32_t stage_index(uint32_t i) { return i + 4u * (i >> 5); }

// Floats one staged row of n elements occupies, rounded to 16 bytes.
__host__ __device__ __forceinline__ uint32_t stage_stride(uint32_t n) {
    return (n + 4u * ((n + 31u) / 32u) + 3u) & ~3u;
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Sequential sum from +0.0 of the leaf [b, e) (e - b <= 32) of a staged row.
// All loads are issued before the additions; absent slots add +0.0, which is
// exact because a sum started from +0.0 is never -0.0.
__device__ __forceinline__ float staged_leaf_sum(const float* st, uint32_t b, uint32_t e) {
    float s = 0.0f;
    if (e - b == 32u && (b & 31u) == 0u) {
        const f32x4_t* p = reinterpret_cast<const f32x4_t*>(st + stage_index(b));
#pragma unroll
        for (int h = 0; h < 8; h += 4) {
            f32x4_t v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = p[h + i];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) s = s + v[i][j];
        }
        return s;
    }
#pragma unroll
    for (int c = 0; c < 32; c += 8) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (b + c + i < e) ? st[stage_index(b + c + i)] : 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) s = s + v[i];
    }
    return s;
}

// Sum of the `per` consecutive depth-D leaves starting at leaf `first` of a
// staged row of n elements, folded with the binary-counter carry stack (per is
// a power of two, so this is the balanced subtree over those leaves).
__device__ __forceinline__ float staged_subtree_sum(const float* st, uint32_t n, int depth,
                                                    uint32_t first, uint32_t per) {
    float stack[9];
#pragma unroll
    for (int l = 0; l < 9; ++l) stack[l] = 0.0f;
    for (uint32_t t = 0; t < per; ++t) {
        uint32_t b, e;
        pairwise_leaf(n, depth, first + t, b, e);
        float s = staged_leaf_sum(st, b, e);
        bool carry = true;
#pragma unroll
        for (int l = 0; l < 9; ++l) {
            if (carry) {
                if ((t >> l) & 1u) {
                    s = stack[l] + s;
                } else {
                    stack[l] = s;
                    carry = false;
                }
            }
        }
    }
    float v = 0.0f;
#pragma unroll
    for (int l = 0; l < 9; ++l)
        if ((1u << l) == per) v = stack[l];
    return v;
}

// ---- exp and log shared with the CPU oracle (the exact numerics mode) ---------
// The reference's CPU softmax calls the platform libm (std::exp / std::log,
// kernels_reduce.cpp:227-243), whose float results are not pinned (glibc's
// expf and logf are within 0.502 ulp and differ from the correctly rounded
// value for about 1e-4 / 1e-3 of inputs). In the exact numerics mode the
// device and the oracle (oracle/vkml_oracle.c) evaluate both with the same
// sequence of IEEE double operations, so they agree bit for bit by
// construction, and each result is the correctly rounded float except when
// exp(x) or log(x) lies within ~2^-27 ulp of a rounding midpoint:
//   exp: Cody-Waite reduction x = k ln2 + r (|r| <= ln2/2, ln2 split in two
//        doubles, fused multiply-adds), the Taylor polynomial of e^r to degree
//        13 in Horner form (truncation below 2^-52), scaled by 2^k;
//   log: x = m 2^e with m in [sqrt(1/2), sqrt(2)), s = (m - 1) / (m + 1)
//        (m - 1 and m + 1 exact), log m = 2 atanh s = 2s (1 + s^2/3 + s^4/5
//        + ... + s^24/25) (truncation below 2^-60), plus e ln2.
// Results below 2^-150 are +0, above FLT_MAX +inf; log(0) = -inf, log of a
// negative number or NaN is NaN.
__host__ __device__ inline float exact_expf(float xf) {
    if (xf != xf) return xf + xf;
    if (xf > 89.0f) return __builtin_inff();
    if (xf < -104.0f) return 0.0f;
    const double x = xf;
    const double kd = __builtin_rint(x * 0x1.71547652b82fep+0);
    double r = __builtin_fma(-kd, 0x1.62e42fefa39efp-1, x);
    r = __builtin_fma(-kd, 0x1.abc9e3b39803fp-56, r);
    double p = 0x1.6124613a86d09p-33;
    p = __builtin_fma(p, r, 0x1.1eed8eff8d898p-29);
    p = __builtin_fma(p, r, 0x1.ae64567f544e4p-26);
    p = __builtin_fma(p, r, 0x1.27e4fb7789f5cp-22);
    p = __builtin_fma(p, r, 0x1.71de3a556c734p-19);
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-16);
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-13);
    p = __builtin_fma(p, r, 0x1.6c16c16c16c17p-10);
    p = __builtin_fma(p, r, 0x1.1111111111111p-7);
    p = __builtin_fma(p, r, 0x1.5555555555555p-5);
    p = __builtin_fma(p, r, 0x1.5555555555555p-3);
    p = __builtin_fma(p, r, 0x1.0000000000000p-1);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    return static_cast<float>(__builtin_ldexp(p, static_cast<int>(kd)));
}

__host__ __device__ inline float exact_logf(float xf) {
    if (xf != xf) return xf + xf;
    if (xf < 0.0f) return __builtin_nanf("");
    if (xf == 0.0f) return -__builtin_inff();
    if (xf == __builtin_inff()) return xf;
    int e = 0;
    double m = __builtin_frexp(static_cast<double>(xf), &e);  // m in [0.5, 1), exact
    if (m < 0x1.6a09e667f3bcdp-1) {
        m = m + m;
        e -= 1;
    }
    const double f = m - 1.0;  // exact: m has at most 24 significant bits
    const double s = f / (2.0 + f);
    const double z = s * s;
    double w = 0x1.47ae147ae147bp-5;
    w = __builtin_fma(w, z, 0x1.642c8590b2164p-5);
    w = __builtin_fma(w, z, 0x1.8618618618618p-5);
    w = __builtin_fma(w, z, 0x1.af286bca1af28p-5);
    w = __builtin_fma(w, z, 0x1.e1e1e1e1e1e1ep-5);
    w = __builtin_fma(w, z, 0x1.1111111111111p-4);
    w = __builtin_fma(w, z, 0x1.3b13b13b13b14p-4);
    w = __builtin_fma(w, z, 0x1.745d1745d1746p-4);
    w = __builtin_fma(w, z, 0x1.c71c71c71c71cp-4);
    w = __builtin_fma(w, z, 0x1.2492492492492p-3);
    w = __builtin_fma(w, z, 0x1.999999999999ap-3);
    w = __builtin_fma(w, z, 0x1.5555555555555p-2);
    const double t = s + s;
    const double lm = __builtin_fma(t * z, w, t);
    const double ed = static_cast<double>(e);
    const double y = __builtin_fma(ed, 0x1.62e42fefa39efp-1, __builtin_fma(ed, 0x1.abc9e3b39803fp-56, lm));
    return static_cast<float>(y);
}

// ---- butterflies across a wave of 64 ----------------------------------------
// Step OFF of a butterfly pairs lane i with lane i ^ OFF. Once the steps
// below OFF have run with a symmetric merge (merge(a, b) == merge(b, a)),
// every aligned group of OFF lanes holds one value, and any exchange that
// lands in the partner group gives the same result. That lets the steps use
// register-speed DPP moves instead of LDS-routed shuffles: xor 1 and xor 2
// are DPP quad permutations, 4 and 8 the half-row and row mirrors (lane
// 7 - i, 15 - i), 16 a ds_swizzle xor within 32 lanes, and the last step
// combines lanes 0 and 32 read into scalars.
template <int OFF>
__device__ __forceinline__ int wave_partner(int v) {
    if constexpr (OFF == 1) return __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false);
    else if constexpr (OFF == 2) return __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false);
    else if constexpr (OFF == 4) return __builtin_amdgcn_update_dpp(v, v, 0x141, 0xF, 0xF, false);
    else if constexpr (OFF == 8) return __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, false);
    else if constexpr (OFF == 16) return __builtin_amdgcn_ds_swizzle(v, 0x401F);
    else return __shfl_xor(v, OFF, 64);
}

template <int OFF>
__device__ __forceinline__ float wave_partner(float v) {
    return __builtin_bit_cast(float, wave_partner<OFF>(__builtin_bit_cast(int, v)));
}

__device__ __forceinline__ float lane_value(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Balanced pairwise sum of the 64 lanes' values (lane order), in every lane.
__device__ __forceinline__ float wave_sum_butterfly(float v) {
    v = v + wave_partner<1>(v);
    v = v + wave_partner<2>(v);
    v = v + wave_partner<4>(v);
    v = v + wave_partner<8>(v);
    v = v + wave_partner<16>(v);
    return lane_value(v, 0) + lane_value(v, 32);
}

// The window scan of a 2x2 max-pool: strict '>' from -inf over a, b, c, d in
// that order (window positions (0,0), (0,1), (1,0), (1,1)); the offset of the
// first maximum, -1 if none wins (all -inf or NaN). Shared by the pool kernels
// and the fused pool-gradient weight-gradient kernel, so both pick alike.
__device__ __forceinline__ int32_t argmax4(float a, float b, float c, float d) {
    float best = -__builtin_inff();
    int32_t off = -1;
    if (a > best) { best = a; off = 0; }
    if (b > best) { best = b; off = 1; }
    if (c > best) { best = c; off = 2; }
    if (d > best) { best = d; off = 3; }
    return off;
}

}  // namespace vkhip
