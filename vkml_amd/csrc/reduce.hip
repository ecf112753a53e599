// Softmax / log-softmax and row/axis reductions (sum, mean, max, min, argmax,
// argmin) for gfx950.
//
// Numerics follow the CPU oracle (reference kernels_reduce.cpp:44-259):
//   - sum and mean are the oracle's pairwise tree (reduce.h:55-72) exactly. The
//     row is staged once in LDS (coalesced 16-byte loads), each thread sums the
//     tree's 32-element leaves sequentially, and leaves combine adjacent-first by
//     a wave64 xor-butterfly and then across waves. Bit-identical to the oracle.
//   - max/min/argmax/argmin are selections, merged with an explicit lowest-index
//     tie-break, so any merge order gives the oracle's sequential answer:
//     first maximum; max/min return the first NaN; argmax/argmin skip NaN.
//   - softmax: peak = max, out = exp(x - peak) / denom or (x - peak) -
//     log(denom). Rows of up to 2048 (one wave each, the cross-entropy rows
//     too) stage exp(x - peak) for the oracle's pairwise tree; longer rows sum
//     it from registers in a fixed order (a different association, a few ulp).
//     exp is a base-2 exponential with a carried rounding term and log is the
//     device library's, so results are within a few ulp of the oracle's libm,
//     not bit-identical.
//
// Bandwidth: one HBM read and (softmax) one write per element; the row never
// leaves the CU between passes.
#include "common.h"

namespace vkhip {

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float max_ignoring_nan(float a, float b) { return (a < b) ? b : a; }

// Peak of a register-held row slice for softmax, as a balanced tree of fmaxf.
// fmaxf ignores a NaN operand and may return either zero when both signs
// meet; neither shows in softmax outputs, so this agrees with the oracle's
// sequential std::max: a row holding a NaN is NaN throughout whatever its
// peak; x - peak depends on the sign of a zero peak only for a zero x, whose
// exp is 1 either way and whose log-softmax value (x - peak) - log(denom) is
// -log(denom) unless denom == 1, which leaves a single zero in the row, and
// that zero is the peak under either rule. Slots with keep[i] false count as
// -inf.
template <int E>
__device__ __forceinline__ float tree_peak(const float (&x)[E], const bool (&keep)[E]) {
    float m[E];
#pragma unroll
    for (int i = 0; i < E; ++i) m[i] = keep[i] ? x[i] : -__builtin_inff();
#pragma unroll
    for (int w = 1; w < E; w <<= 1)
#pragma unroll
        for (int i = 0; i + w < E; i += 2 * w) m[i] = __builtin_fmaxf(m[i], m[i + w]);
    return m[0];
}

// Wave-wide fmaxf (symmetric, NaN-ignoring); used for softmax peaks only,
// where the sign of a zero peak is not observable.
__device__ __forceinline__ float wave_max(float v) {
    v = __builtin_fmaxf(v, wave_partner<1>(v));
    v = __builtin_fmaxf(v, wave_partner<2>(v));
    v = __builtin_fmaxf(v, wave_partner<4>(v));
    v = __builtin_fmaxf(v, wave_partner<8>(v));
    v = __builtin_fmaxf(v, wave_partner<16>(v));
    return __builtin_fmaxf(lane_value(v, 0), lane_value(v, 32));
}

// Pairwise sum of the n values staged in `st` by a group of T threads (t =
// index within the group). Every thread of the group gets the total. `scratch`
// holds T/64 floats for the group. All threads of the BLOCK must call this
// together (it contains block barriers when T > 64).
template <int T>
__device__ float group_pairwise_sum(const float* st, uint32_t n, int depth, int t,
                                    float* scratch) {
    const uint32_t leaves = 1u << depth;
    const uint32_t per = leaves > static_cast<uint32_t>(T) ? leaves / T : 1u;
    float v = 0.0f;
    if (static_cast<uint32_t>(t) * per < leaves) v = staged_subtree_sum(st, n, depth, t * per, per);
    v = wave_sum_butterfly(v);
    if constexpr (T > 64) {
        const int lane = t & 63, wave = t >> 6;
        if (lane == 0) scratch[wave] = v;
        __syncthreads();
        float u = lane < T / 64 ? scratch[lane] : 0.0f;
        v = wave_sum_butterfly(u);
        __syncthreads();
    }
    return v;
}

template <int T>
__device__ float group_max(float v, int t, float* scratch) {
    v = wave_max(v);
    if constexpr (T > 64) {
        const int lane = t & 63, wave = t >> 6;
        if (lane == 0) scratch[wave] = v;
        __syncthreads();
        float u = lane < T / 64 ? scratch[lane] : -__builtin_inff();
        v = wave_max(u);
        __syncthreads();
    }
    return v;
}

// Rows per 256-thread block when a group of T threads owns a row.
template <int T>
struct Rows {
    static constexpr int kPerBlock = T >= 256 ? 1 : 256 / T;
    static constexpr int kThreads = T >= 256 ? T : 256;
};

// Loads this thread's share of a contiguous row: float4 groups 4*(t + T*i)
// (vec) or elements t + T*i (scalar), i < E4 (vec) / 4*E4 (scalar). The
// 16-byte loads are non-temporal (STREAM) for data each workgroup reads once:
// a read-only probe over 67 / 134 MB measured 11.0-11.2 / 20.3-20.6 us with
// them against 11.7 / 22.2 us with ordinary loads. A vector that every
// workgroup reads again (the GEMV's x) keeps ordinary loads. (Loads issued
// unconditionally at clamped addresses, then zeroed, measured slower for the
// softmax rows, 7.6 -> 9.6 us at [4096, 1000], and equal for max.)
template <int T, int E4, bool STREAM = true>
__device__ __forceinline__ void load_row(float (&x)[4 * E4], const float* rs, uint32_t n, int t,
                                         bool live, int vec) {
    if (vec) {
#pragma unroll
        for (int i = 0; i < E4; ++i) {
            const uint32_t e0 = 4u * (t + T * i);
            f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
            if (live && e0 < n) {
                const f32x4* p = reinterpret_cast<const f32x4*>(rs + e0);
                v = STREAM ? __builtin_nontemporal_load(p) : *p;
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) x[4 * i + j] = v[j];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4 * E4; ++i) {
            const uint32_t e = t + T * i;
            x[i] = (live && e < n) ? rs[e] : 0.0f;
        }
    }
}

// load_row for a row that fills every slot (n == 4 * E4 * T, 16-byte
// aligned): no bounds tests, so every load is issued before the first wait.
template <int T, int E4>
__device__ __forceinline__ void load_row_full(float (&x)[4 * E4], const float* rs, int t) {
    f32x4 v[E4];
#pragma unroll
    for (int i = 0; i < E4; ++i)
        v[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(rs) + t + T * i);
#pragma unroll
    for (int i = 0; i < E4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) x[4 * i + j] = v[i][j];
}

__device__ __forceinline__ uint32_t elem_of(int vec, int T, int t, int i) {
    return vec ? 4u * (t + T * (i / 4)) + (i % 4) : static_cast<uint32_t>(t + T * i);
}

// ---- exp for softmax ------------------------------------------------------------
// exp(s) for the softmax shifts s = x - peak <= 0 (or NaN): 2^(s*log2 e) on the
// hardware base-2 exponential (v_exp_f32), with the rounding error of s*log2 e
// carried along. log2 e = kL2eHi + kL2eLo (kL2eHi its float rounding); the
// product's exact remainder comes from one FMA (the 2MultFMA algorithm, Muller
// et al., Handbook of Floating-Point Arithmetic, 2nd ed., sec. 4.4.2), and
// 2^(t + r) = 2^t (1 + r ln 2) to within (r ln 2)^2 / 2 < 2^-41 for |r| < 2^-20.
// The result is within about 2 ulp of exp(s) (against ~1 for the general expf,
// in a third of the instructions: the softmax kernels are instruction-bound at
// 32768-wide rows). Shifts below -150 give 0 (2^t rounds to 0 there); the
// general expf keeps subnormal results down to -103.97, a difference of less
// than 2^-126. s = -inf: 2^t = 0 and r is NaN, which the maximum with -1 (an
// IEEE maxNum: the non-NaN operand) replaces, so the result is +0; for any
// finite s, |r ln 2| < 2^-20 and the maximum leaves it as it is.
__device__ __forceinline__ float softmax_exp(float s) {
    constexpr float kL2eHi = 1.44269502162933349609375f;
    constexpr float kL2eLo = 1.925963033500011e-08f;
    constexpr float kLn2 = 0.6931471805599453f;
    const float t = s * kL2eHi;
    const float r = __builtin_fmaf(s, kL2eLo, __builtin_fmaf(s, kL2eHi, -t));
    const float e = __builtin_amdgcn_exp2f(t);
    return __builtin_fmaf(e, __builtin_fmaxf(r * kLn2, -1.0f), e);
}

// ---- softmax over contiguous rows ------------------------------------------------
// Outputs are exp(x - peak) * (1/denom): one multiply per element by the
// row's correctly rounded reciprocal, within 1.5 ulp of the quotient (the
// exponential above is the larger error term; softmax parity is tolerance-
// based, 1e-5 * sqrt(n) relative).
__device__ __forceinline__ float div_by(float x, float /*d*/, float r) { return x * r; }

// Sum over a group of T threads, in a fixed order (a wave butterfly, then the
// waves' sums in wave order): deterministic, every thread gets the total.
template <int T>
__device__ float group_sum(float v, int t, float* scratch) {
    v = wave_sum_butterfly(v);
    if constexpr (T > 64) {
        const int lane = t & 63, wave = t >> 6;
        if (lane == 0) scratch[wave] = v;
        __syncthreads();
        const float u = lane < T / 64 ? scratch[lane] : 0.0f;
        v = wave_sum_butterfly(u);
        __syncthreads();
    }
    return v;
}

// T threads per row (64: four rows per 256-thread block), rows of n <= 4*E4*T
// contiguous floats at src + row*in_stride; dst rows contiguous. The row is read
// once into registers and exp(x - peak) is computed once and kept there for
// the output. The denominator is summed from the registers (each thread's
// values in order, then group_sum): the row is not staged in LDS for the
// oracle's pairwise tree, which at these widths held one workgroup per CU in
// lockstep phases (256x32768: 18.6 us staged, 15.8 from registers). The
// association differs from the oracle's tree by a few ulp of the
// denominator, inside the softmax tolerance.
template <int T, int E4, bool LOG>
__global__ __launch_bounds__(Rows<T>::kThreads) void softmax_rows_kernel(
    const float* __restrict__ src, int64_t in_stride, float* __restrict__ dst, uint32_t rows,
    uint32_t n, int vec) {
    constexpr int RPB = Rows<T>::kPerBlock;
    constexpr int E = 4 * E4;
    __shared__ float scratch[RPB][T / 64 > 0 ? T / 64 : 1];

    const int slot = threadIdx.x / T;
    const int t = threadIdx.x % T;
    const uint32_t row = blockIdx.x * RPB + slot;
    const bool live = row < rows;
    const float* rs = src + static_cast<int64_t>(live ? row : 0) * in_stride;

    float x[E];
    load_row<T, E4>(x, rs, n, t, live, vec);
    bool keep[E];
#pragma unroll
    for (int i = 0; i < E; ++i) keep[i] = live && elem_of(vec, T, t, i) < n;
    float mx = tree_peak<E>(x, keep);
    mx = group_max<T>(mx, t, scratch[slot]);

    float part = 0.0f;
#pragma unroll
    for (int i = 0; i < E; ++i) {
        const float sh = x[i] - mx;
        const float ex = softmax_exp(sh);
        if (keep[i]) part = part + ex;
        x[i] = LOG ? sh : ex;
    }
    const float denom = group_sum<T>(part, t, scratch[slot]);
    if (!live) return;
    const float ld = logf(denom);
    const float rinv = 1.0f / denom;
    float* ds = dst + static_cast<uint64_t>(row) * n;
    if (vec) {
#pragma unroll
        for (int i = 0; i < E4; ++i) {
            const uint32_t e0 = 4u * (t + T * i);
            if (e0 < n) {
                f32x4 o;
#pragma unroll
                for (int j = 0; j < 4; ++j) o[j] = LOG ? x[4 * i + j] - ld : div_by(x[4 * i + j], denom, rinv);
                __builtin_nontemporal_store(o, reinterpret_cast<f32x4*>(ds + e0));
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < E; ++i) {
            const uint32_t e = t + T * i;
            if (e < n) ds[e] = LOG ? x[i] - ld : div_by(x[i], denom, rinv);
        }
    }
}

// ---- softmax, one workgroup per long row, one pass of statistics ---------------------
// For rows of 1024 threads x 32 floats (up to 32768 elements, e.g. [256, 32768],
// one row per CU): the row's peak and its sum of exponentials are reduced as
// one (peak, sum) pair instead of a peak reduction followed by a sum reduction.
// Each thread sums exp(x - m_t) against its own peak m_t; pairs combine as
// (max(m1, m2), s1 e^(m1 - M) + s2 e^(m2 - M)); the outputs are
// exp(x - m_t) * (e^(m_t - M) / S) (softmax) or x - M - log(S) (log-softmax):
// one block-level exchange and one barrier fewer between the row's loads and
// its stores. The rescaling adds a few roundings (within the fast numerics'
// 1e-5*sqrt(n)); the exact numerics mode has its own kernels. Special values:
// a thread whose elements are all -inf contributes (-inf, 0) and outputs 0; a
// +inf or NaN anywhere makes the sum, and so the row, NaN, as the oracle's.
__device__ __forceinline__ void pair_combine(float& m, float& s, float m2, float s2) {
    const float M = __builtin_fmaxf(m, m2);
    const float a = m == M ? 1.0f : softmax_exp(m - M);
    const float b = m2 == M ? 1.0f : softmax_exp(m2 - M);
    s = s * a + s2 * b;
    m = M;
}

__device__ __forceinline__ void wave_pair(float& m, float& s) {
    pair_combine(m, s, wave_partner<1>(m), wave_partner<1>(s));
    pair_combine(m, s, wave_partner<2>(m), wave_partner<2>(s));
    pair_combine(m, s, wave_partner<4>(m), wave_partner<4>(s));
    pair_combine(m, s, wave_partner<8>(m), wave_partner<8>(s));
    pair_combine(m, s, wave_partner<16>(m), wave_partner<16>(s));
    const float m0 = lane_value(m, 0), s0 = lane_value(s, 0);
    const float m1 = lane_value(m, 32), s1 = lane_value(s, 32);
    m = m0;
    s = s0;
    pair_combine(m, s, m1, s1);
}

// FULL: the row fills every thread's E elements (n == 4 * E4 * 1024): no
// per-element bounds (about a tenth of the kernel's VALU instructions).
template <int E4, bool LOG, bool FULL>
__global__ __launch_bounds__(1024) void softmax_online_rows_kernel(const float* __restrict__ src,
                                                                   int64_t in_stride,
                                                                   float* __restrict__ dst,
                                                                   uint32_t rows, uint32_t n) {
    constexpr int T = 1024, E = 4 * E4;
    __shared__ float sm[T / 64], ss[T / 64];
    const int t = threadIdx.x;
    const uint32_t row = blockIdx.x;
    const float* rs = src + static_cast<int64_t>(row) * in_stride;
    if constexpr (FULL) n = 4u * E4 * T;
    float x[E];
    if constexpr (FULL)
        load_row_full<T, E4>(x, rs, t);
    else
        load_row<T, E4>(x, rs, n, t, true, 1);
    bool keep[E];
#pragma unroll
    for (int i = 0; i < E; ++i) keep[i] = FULL || elem_of(1, T, t, i) < n;
    const float mt = tree_peak<E>(x, keep);
    const float mref = mt == -__builtin_inff() ? 0.0f : mt;  // an all -inf share sums to 0
    float e[E];
    float part = 0.0f;
#pragma unroll
    for (int i = 0; i < E; ++i) {
        e[i] = softmax_exp(x[i] - mref);
        if (keep[i]) part = part + e[i];
    }
    float m = mt, s = part;
    wave_pair(m, s);
    const int lane = t & 63, wave = t >> 6;
    if (lane == 0) {
        sm[wave] = m;
        ss[wave] = s;
    }
    __syncthreads();
    float M = lane < T / 64 ? sm[lane] : -__builtin_inff();
    float S = lane < T / 64 ? ss[lane] : 0.0f;
    wave_pair(M, S);
    float* ds = dst + static_cast<uint64_t>(row) * n;
    if constexpr (LOG) {
        const float ld = logf(S);
#pragma unroll
        for (int i = 0; i < E4; ++i) {
            const uint32_t e0 = 4u * (t + T * i);
            if (e0 < n) {
                f32x4 o;
#pragma unroll
                for (int j = 0; j < 4; ++j) o[j] = (x[4 * i + j] - M) - ld;
                __builtin_nontemporal_store(o, reinterpret_cast<f32x4*>(ds + e0));
            }
        }
    } else {
        // this thread's factor e^(m_t - M) / S (0 for an all -inf share)
        const float f = mt == -__builtin_inff() ? 0.0f : (mt == M ? 1.0f : softmax_exp(mt - M));
        const float scale = f * (1.0f / S);
#pragma unroll
        for (int i = 0; i < E4; ++i) {
            const uint32_t e0 = 4u * (t + T * i);
            if (e0 < n) {
                f32x4 o;
#pragma unroll
                for (int j = 0; j < 4; ++j) o[j] = e[4 * i + j] * scale;
                __builtin_nontemporal_store(o, reinterpret_cast<f32x4*>(ds + e0));
            }
        }
    }
}

// ---- softmax, one wave per row, persistent with prefetch -------------------------------
// Rows of n <= 16*E4 (E4 float4 per lane) contiguous floats. Each wave walks
// rows row0, row0 + stride, ... and issues the next row's loads before it
// works on the current one, so HBM reads of one row overlap the reductions
// and the stores of the previous: the latency-bound phases of the one-shot
// kernel (all loads, then all math, then all stores) interleave instead.
// The wave's LDS stage is private to it; lanes exchange staged values only
// inside the wave, whose LDS operations complete in issue order, so a
// compiler barrier (no s_barrier) orders them.
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
}

template <int E4, bool LOG, bool VEC>
__global__ __launch_bounds__(256) void softmax_wave_rows_kernel(
    const float* __restrict__ src, int64_t in_stride, float* __restrict__ dst, uint32_t rows,
    uint32_t n, int depth, uint32_t sstride) {
    constexpr int vec = VEC ? 1 : 0;
    constexpr int E = 4 * E4;
    extern __shared__ __attribute__((aligned(16))) float dyn[];
    const int wave = threadIdx.x >> 6;
    const int t = threadIdx.x & 63;
    float* stage = dyn + wave * sstride;
    const uint32_t stride = gridDim.x * 4;
    uint32_t row = blockIdx.x * 4 + wave;
    float xn[E];
    load_row<64, E4>(xn, src + static_cast<int64_t>(row < rows ? row : 0) * in_stride, n, t,
                     row < rows, vec);
    // n <= 2048 gives at most 64 leaves: lane t owns leaf t, the same range
    // for every row, so it is computed once.
    uint32_t leaf_b = 0, leaf_e = 0;
    if (static_cast<uint32_t>(t) < (1u << depth)) pairwise_leaf(n, depth, t, leaf_b, leaf_e);
    for (; row < rows; row += stride) {
        float x[E];
#pragma unroll
        for (int i = 0; i < E; ++i) x[i] = xn[i];
        const uint32_t next = row + stride;
        if (next < rows) load_row<64, E4>(xn, src + static_cast<int64_t>(next) * in_stride, n, t, true, vec);
        bool keep[E];
#pragma unroll
        for (int i = 0; i < E; ++i) keep[i] = elem_of(vec, 64, t, i) < n;
        float mx = tree_peak<E>(x, keep);
        mx = wave_max(mx);
#pragma unroll
        for (int i = 0; i < E; ++i) {
            const float sh = x[i] - mx;
            x[i] = LOG ? sh : softmax_exp(sh);
            if (LOG) {
                if (!VEC && elem_of(vec, 64, t, i) < n) stage[stage_index(elem_of(vec, 64, t, i))] = softmax_exp(sh);
            } else if (!VEC) {
                if (elem_of(vec, 64, t, i) < n) stage[stage_index(elem_of(vec, 64, t, i))] = x[i];
            }
        }
        if constexpr (VEC) {
            // Four consecutive elements of one 32-element block: one 16-byte write.
#pragma unroll
            for (int i = 0; i < E4; ++i) {
                const uint32_t e0 = 4u * (t + 64 * i);
                if (e0 < n) {
                    f32x4 w;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        w[j] = LOG ? softmax_exp(x[4 * i + j]) : x[4 * i + j];
                    *reinterpret_cast<f32x4*>(stage + stage_index(e0)) = w;
                }
            }
        }
        wave_lds_fence();
        const float v = leaf_e > leaf_b ? staged_leaf_sum(stage, leaf_b, leaf_e) : 0.0f;
        const float denom = wave_sum_butterfly(v);
        wave_lds_fence();  // every lane's stage reads precede the next row's writes
        const float ld = logf(denom);
        const float rinv = 1.0f / denom;
        float* ds = dst + static_cast<uint64_t>(row) * n;
        if (vec) {
#pragma unroll
            for (int i = 0; i < E4; ++i) {
                const uint32_t e0 = 4u * (t + 64 * i);
                if (e0 < n) {
                    f32x4 o;
#pragma unroll
                    for (int j = 0; j < 4; ++j) o[j] = LOG ? x[4 * i + j] - ld : div_by(x[4 * i + j], denom, rinv);
                    __builtin_nontemporal_store(o, reinterpret_cast<f32x4*>(ds + e0));
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < E; ++i) {
                const uint32_t e = t + 64 * i;
                if (e < n) ds[e] = LOG ? x[i] - ld : div_by(x[i], denom, rinv);
            }
        }
    }
}

// ---- cross-entropy rows (fused) ------------------------------------------------
// One wave per row of C <= 2048 logits. The log-softmax is computed exactly as
// softmax_wave_rows_kernel<.., LOG = true> computes it (fmaxf peak, the same
// exponential staged in the same pairwise tree, logf of the denominator,
// ls = (x - peak) - log(denom)), so ls is bit-identical to the LOG_SOFTMAX
// node's output. Forward: the one-hot row (float(label) == float(c)), the
// rounded products ls*onehot, their pairwise sum over C (the SUM node's tree)
// and its negation. Backward, given g = dL/d(out[r]): the reference autograd's
// chain, neg (-g), sum and mul backward (gl = (-g) * onehot), log-softmax
// backward gl - exp(ls) * pairwise_sum(gl) with the EXP node's expf.
template <int E, bool EXACT>
__global__ __launch_bounds__(256) void cross_entropy_rows_kernel(
    const float* __restrict__ logits, int64_t row_stride, const int64_t* __restrict__ labels,
    const float* __restrict__ g_out, float* __restrict__ out, uint32_t rows, uint32_t n, int depth,
    uint32_t sstride, int backward) {
    extern __shared__ __attribute__((aligned(16))) float dyn[];
    const int wave = threadIdx.x >> 6;
    const int t = threadIdx.x & 63;
    float* stage = dyn + wave * sstride;
    uint32_t leaf_b = 0, leaf_e = 0;
    if (static_cast<uint32_t>(t) < (1u << depth)) pairwise_leaf(n, depth, t, leaf_b, leaf_e);
    for (uint32_t row = blockIdx.x * 4 + wave; row < rows; row += gridDim.x * 4) {
        const float* rs = logits + static_cast<int64_t>(row) * row_stride;
        float x[E];
        bool keep[E];
#pragma unroll
        for (int i = 0; i < E; ++i) {
            const uint32_t e = static_cast<uint32_t>(t) + 64u * i;
            keep[i] = e < n;
            x[i] = keep[i] ? rs[e] : 0.0f;
        }
        const float mx = wave_max(tree_peak<E>(x, keep));
#pragma unroll
        for (int i = 0; i < E; ++i) {
            x[i] = x[i] - mx;
            if (keep[i]) stage[stage_index(t + 64u * i)] = EXACT ? exact_expf(x[i]) : softmax_exp(x[i]);
        }
        wave_lds_fence();
        float v = leaf_e > leaf_b ? staged_leaf_sum(stage, leaf_b, leaf_e) : 0.0f;
        const float denom = wave_sum_butterfly(v);
        wave_lds_fence();
        const float ld = EXACT ? exact_logf(denom) : logf(denom);
        const float label = static_cast<float>(labels[row]);
#pragma unroll
        for (int i = 0; i < E; ++i) x[i] = x[i] - ld;  // log-softmax
        if (!backward) {
#pragma unroll
            for (int i = 0; i < E; ++i) {
                const uint32_t e = static_cast<uint32_t>(t) + 64u * i;
                const float onehot = label == static_cast<float>(e) ? 1.0f : 0.0f;
                if (keep[i]) stage[stage_index(e)] = __fmul_rn(x[i], onehot);
            }
            wave_lds_fence();
            v = leaf_e > leaf_b ? staged_leaf_sum(stage, leaf_b, leaf_e) : 0.0f;
            const float picked = wave_sum_butterfly(v);
            wave_lds_fence();
            if (t == 0) out[row] = -picked;
        } else {
            const float ng = -g_out[row];
            float gl[E];
#pragma unroll
            for (int i = 0; i < E; ++i) {
                const uint32_t e = static_cast<uint32_t>(t) + 64u * i;
                gl[i] = __fmul_rn(ng, label == static_cast<float>(e) ? 1.0f : 0.0f);
                if (keep[i]) stage[stage_index(e)] = gl[i];
            }
            wave_lds_fence();
            v = leaf_e > leaf_b ? staged_leaf_sum(stage, leaf_b, leaf_e) : 0.0f;
            const float total = wave_sum_butterfly(v);
            wave_lds_fence();
            float* ds = out + static_cast<uint64_t>(row) * n;
#pragma unroll
            for (int i = 0; i < E; ++i) {
                const uint32_t e = static_cast<uint32_t>(t) + 64u * i;
                if (keep[i]) ds[e] = __fsub_rn(gl[i], __fmul_rn(EXACT ? exact_expf(x[i]) : expf(x[i]), total));
            }
        }
    }
}

int launch_cross_entropy(const float* logits, int64_t row_stride, const int64_t* labels,
                         const float* g_out, float* out, uint32_t rows, uint32_t n, int backward) {
    if (rows == 0) return VKHIP_OK;
    if (n == 0 || n > 2048)
        return fail(VKHIP_ERR_UNSUPPORTED, "cross_entropy: %u classes (1..2048 supported)", n);
    const int depth = pairwise_depth(n);
    const uint32_t ss = stage_stride(n);
    const size_t lds = 4 * static_cast<size_t>(ss) * sizeof(float);
    const uint32_t cus = ctx().ready ? static_cast<uint32_t>(ctx().caps.compute_units) : 256u;
    const uint32_t want = ceil_div(rows, 4);
    const uint32_t blocks = want < cus * 4 ? want : cus * 4;
    void (*fn)(const float*, int64_t, const int64_t*, const float*, float*, uint32_t, uint32_t, int,
               uint32_t, int);
    const bool ex = ctx().exact_math != 0;
    if (n <= 64) fn = ex ? cross_entropy_rows_kernel<1, true> : cross_entropy_rows_kernel<1, false>;
    else if (n <= 256) fn = ex ? cross_entropy_rows_kernel<4, true> : cross_entropy_rows_kernel<4, false>;
    else if (n <= 1024) fn = ex ? cross_entropy_rows_kernel<16, true> : cross_entropy_rows_kernel<16, false>;
    else fn = ex ? cross_entropy_rows_kernel<32, true> : cross_entropy_rows_kernel<32, false>;
    hipLaunchKernelGGL(fn, dim3(blocks), dim3(256), lds, ctx().stream, logits, row_stride, labels,
                       g_out, out, rows, n, depth, ss, backward);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

// ---- one thread per output: any layout ------------------------------------------------
// The reduced elements of output o are at base(o) + lin_off(i, reduced). Sum and
// mean walk the depth-D leaves in order and fold them with a carry stack (a
// balanced fold over 2^D leaves is the oracle's tree); selections scan in index
// order exactly as the oracle's loops do. Adjacent threads own adjacent outputs,
// so the loads coalesce whenever the kept axis is the contiguous one.
constexpr int kTallLevels = 22;  // 2^21 leaves of <= 32: n < 2^26 elements

// Offset of reduced element i: the reduced axes, merged on the host wherever
// they are contiguous with each other, innermost first; every axis but the
// outermost is split off with a launch-time division (reduced extents are
// below 2^26, so 32-bit quotients suffice).
struct Reader {
    int naxes;         // 1..4
    uint32_t ne[3];    // extents of the inner naxes - 1 axes
    int64_t nb[3];     // their strides
    FastDiv div[3];    // divisions by ne[]
    int64_t nb_outer;  // stride of the outermost axis
    __device__ __forceinline__ int64_t off(uint32_t i) const {
        int64_t o = 0;
        uint32_t q = i;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            if (a + 1 < naxes) {
                const uint32_t qn = div[a].div(q);
                o += static_cast<int64_t>(q - qn * ne[a]) * nb[a];
                q = qn;
            }
        }
        return o + static_cast<int64_t>(q) * nb_outer;
    }
};

// Reader over the reduced axes of `red` (right-aligned rank 4).
static Reader make_reader(const Op4& red) {
    uint32_t ne[4];
    int64_t nb[4];
    int k = 0;  // axes with extent > 1, outermost first, merged when contiguous
    for (int i = 0; i < 4; ++i) {
        if (red.ne[i] == 1) continue;
        if (k > 0 && nb[k - 1] == static_cast<int64_t>(red.ne[i]) * red.nb[i]) {
            ne[k - 1] *= red.ne[i];
            nb[k - 1] = red.nb[i];
        } else {
            ne[k] = red.ne[i];
            nb[k] = red.nb[i];
            ++k;
        }
    }
    Reader r{};
    if (k == 0) {
        r.naxes = 1;
        r.nb_outer = 0;
        return r;
    }
    r.naxes = k;
    for (int a = 0; a + 1 < k; ++a) {  // innermost first
        r.ne[a] = ne[k - 1 - a];
        r.nb[a] = nb[k - 1 - a];
        r.div[a] = FastDiv(ne[k - 1 - a]);
    }
    r.nb_outer = nb[0];
    return r;
}

static Reader single_reader(int64_t step) {
    Reader r{};
    r.naxes = 1;
    r.nb_outer = step;
    return r;
}

// Sum/mean with few pairwise leaves per output (n_red <= 256: at most 8
// leaves of <= 32): a workgroup of 64 x L threads covers 64 consecutive
// outputs, wave w summing leaf w of each (its <= 32 loads in flight at once,
// lanes on consecutive outputs), and lane o of wave 0 then folds the L leaf
// sums in the order the one-thread carry stack of reduce_tall_kernel folds
// them. Same association, so the same bits, in one memory round trip instead
// of one per leaf.
template <int L>
__global__ __launch_bounds__(64 * L) void reduce_tall_leaves_kernel(
    const float* __restrict__ src, Op4 kept, Reader rd, uint32_t n_out, uint32_t n_red, int mean,
    float* __restrict__ dst) {
    static_assert(L == 2 || L == 4 || L == 8, "leaves per output");
    constexpr int D = L == 2 ? 1 : L == 4 ? 2 : 3;
    __shared__ float part[L][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t o = blockIdx.x * 64u + lane;
    if (o < n_out) {
        const float* base = src + lin_off4(o, kept.ne, kept.nb);
        uint32_t b, e;
        pairwise_leaf(n_red, D, static_cast<uint32_t>(w), b, e);
        float v[32];
#pragma unroll
        for (int r = 0; r < 32; ++r) v[r] = b + r < e ? base[rd.off(b + r)] : 0.0f;
        float s = 0.0f;
#pragma unroll
        for (int r = 0; r < 32; ++r)
            if (b + r < e) s = s + v[r];
        part[w][lane] = s;
    }
    __syncthreads();
    if (w != 0 || o >= n_out) return;
    float stack[D + 1];
#pragma unroll
    for (int l = 0; l <= D; ++l) stack[l] = 0.0f;
#pragma unroll
    for (int j = 0; j < L; ++j) {
        float s = part[j][lane];
        bool carry = true;
#pragma unroll
        for (int l = 0; l <= D; ++l) {
            if (carry) {
                if ((j >> l) & 1) {
                    s = stack[l] + s;
                } else {
                    stack[l] = s;
                    carry = false;
                }
            }
        }
    }
    float total = stack[D];
    if (mean) total = total / static_cast<float>(n_red);
    dst[o] = total;
}

__global__ __launch_bounds__(256) void reduce_tall_kernel(int op, const float* __restrict__ src,
                                                          Op4 kept, Reader rd, uint64_t n_out,
                                                          uint32_t n_red, int depth,
                                                          void* __restrict__ dst) {
    const uint64_t o = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (o >= n_out) return;
    const float* base = src + lin_off4(static_cast<uint32_t>(o), kept.ne, kept.nb);
    if (op == VKHIP_REDUCE_SUM || op == VKHIP_REDUCE_MEAN) {
        float stack[kTallLevels];
#pragma unroll
        for (int l = 0; l < kTallLevels; ++l) stack[l] = 0.0f;
        const uint32_t leaves = 1u << depth;
        for (uint32_t j = 0; j < leaves; ++j) {
            uint32_t b, e;
            pairwise_leaf(n_red, depth, j, b, e);
            // All of the leaf's (at most 32) loads are issued before the
            // sequential sum, so a leaf costs one memory round trip.
            float v[32];
#pragma unroll
            for (int r = 0; r < 32; ++r) v[r] = b + r < e ? base[rd.off(b + r)] : 0.0f;
            float s = 0.0f;
#pragma unroll
            for (int r = 0; r < 32; ++r)
                if (b + r < e) s = s + v[r];
            bool carry = true;
#pragma unroll
            for (int l = 0; l < kTallLevels; ++l) {
                if (carry) {
                    if ((j >> l) & 1u) {
                        s = stack[l] + s;
                    } else {
                        stack[l] = s;
                        carry = false;
                    }
                }
            }
        }
        float total = 0.0f;
#pragma unroll
        for (int l = 0; l < kTallLevels; ++l)
            if (l == depth) total = stack[l];
        if (op == VKHIP_REDUCE_MEAN)
            total = n_red == 0 ? __builtin_nanf("") : total / static_cast<float>(n_red);
        static_cast<float*>(dst)[o] = total;
        return;
    }
    // Selections scan in index order, 32 loads in flight at a time.
    if (op == VKHIP_REDUCE_MAX || op == VKHIP_REDUCE_MIN) {
        const bool is_max = op == VKHIP_REDUCE_MAX;
        float best = is_max ? -__builtin_inff() : __builtin_inff();
        bool found_nan = false;
        for (uint32_t i0 = 0; i0 < n_red && !found_nan; i0 += 32) {
            float v[32];
#pragma unroll
            for (int r = 0; r < 32; ++r) v[r] = i0 + r < n_red ? base[rd.off(i0 + r)] : 0.0f;
#pragma unroll
            for (int r = 0; r < 32; ++r) {
                if (found_nan || i0 + r >= n_red) continue;
                if (v[r] != v[r]) {
                    best = v[r];
                    found_nan = true;
                } else if (is_max ? (v[r] > best) : (v[r] < best)) {
                    best = v[r];
                }
            }
        }
        static_cast<float*>(dst)[o] = best;
        return;
    }
    const bool is_max = op == VKHIP_REDUCE_ARGMAX;
    float best = is_max ? -__builtin_inff() : __builtin_inff();
    int64_t best_i = 0;
    for (uint32_t i0 = 0; i0 < n_red; i0 += 32) {
        float v[32];
#pragma unroll
        for (int r = 0; r < 32; ++r) v[r] = i0 + r < n_red ? base[rd.off(i0 + r)] : 0.0f;
#pragma unroll
        for (int r = 0; r < 32; ++r) {
            if (i0 + r < n_red && (is_max ? (v[r] > best) : (v[r] < best))) {
                best = v[r];
                best_i = i0 + r;
            }
        }
    }
    static_cast<int64_t*>(dst)[o] = best_i;
}

// ---- one workgroup per output: contiguous reduced runs ----------------------------------
// Sum / mean: the run is staged in LDS and summed by group_pairwise_sum. With
// PROD, each element is first multiplied by the matching element of a
// contiguous vector x, rounded on its own (no FMA): that is the N == 1 matmul,
// y[o] = sum_k A[o,k] * x[k], in the oracle's order (kernels_matmul.cpp:57-86).
template <int T, int E4, bool PROD>
__global__ __launch_bounds__(Rows<T>::kThreads) void reduce_rows_sum_kernel(
    const float* __restrict__ src, Op4 kept, uint32_t n_out, uint32_t n, int depth, int mean,
    int vec, uint32_t sstride, float* __restrict__ dst, const float* __restrict__ xv) {
    constexpr int RPB = Rows<T>::kPerBlock;
    extern __shared__ __attribute__((aligned(16))) float dyn[];
    __shared__ float scratch[RPB][T / 64 > 0 ? T / 64 : 1];
    const int slot = threadIdx.x / T;
    const int t = threadIdx.x % T;
    const uint32_t o = blockIdx.x * RPB + slot;
    const bool live = o < n_out;
    const float* rs = src + (live ? lin_off4(o, kept.ne, kept.nb) : 0);
    float* stage = dyn + slot * sstride;
    float x[4 * E4];
    load_row<T, E4>(x, rs, n, t, live, vec);
    if constexpr (PROD) {
        float w[4 * E4];
        load_row<T, E4, false>(w, xv, n, t, live, vec);
#pragma unroll
        for (int i = 0; i < 4 * E4; ++i) x[i] = __fmul_rn(x[i], w[i]);
    }
    if (vec) {
#pragma unroll
        for (int i = 0; i < E4; ++i) {
            const uint32_t e0 = 4u * (t + T * i);
            if (live && e0 < n) {
                f32x4 v;
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = x[4 * i + j];
                *reinterpret_cast<f32x4*>(stage + stage_index(e0)) = v;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4 * E4; ++i) {
            const uint32_t e = t + T * i;
            if (live && e < n) stage[stage_index(e)] = x[i];
        }
    }
    __syncthreads();
    float s = group_pairwise_sum<T>(stage, n, depth, t, scratch[slot]);
    if (live && t == 0) dst[o] = mean ? s / static_cast<float>(n) : s;
}

// Row sums (PROD = false) and GEMV rows (PROD = true: the rounded products
// x[k] * A[row, k]) for 2048 < n <= 4096 (at most 128 leaves), two rows per
// 256-thread workgroup: both rows are staged, then threads 0-127 sum row 0's
// leaves and 128-255 row 1's (one row per workgroup leaves half the threads
// idle in the tree). The per-row tree is group_pairwise_sum<256>'s: leaf sums,
// the butterfly over each wave, then the two waves' sums added and 0 + 0
// added, as its four-wave butterfly does (its upper two waves hold no leaves),
// so the bits are the one-row kernel's. Measured (4096 x 4096 GEMV / [8192,
// 4096] sum): 12.8 / 22.2 us, against 14.8 / 24.0 with one row per
// workgroup; a persistent grid of four workgroups per CU that issues its next
// pair's loads while the current pair's tree runs measured 13.4 / 23.8.
//
// FULL: n == 4096, every leaf 32 whole floats (leaf j = [32 j, 32 j + 32)),
// so the loads need no bounds and a thread's leaf needs no range walk.
template <bool PROD, bool FULL>
__global__ __launch_bounds__(256) void rows2_sum_kernel(const float* __restrict__ a, int64_t lda,
                                                        const float* __restrict__ xv,
                                                        float* __restrict__ y, uint32_t m,
                                                        uint32_t n, int depth, uint32_t sstride,
                                                        int mean) {
    extern __shared__ __attribute__((aligned(16))) float dyn[];
    __shared__ float scratch[4];
    if constexpr (FULL) n = 4096u;
    sstride &= ~3u;  // a multiple of four floats (stage_stride): 16-byte LDS stores for row 1
    const int t = threadIdx.x;
    const uint32_t r0 = blockIdx.x * 2;
    const bool live1 = r0 + 1 < m;
    float w[16], x0[16], x1[16];
    const float* a0 = a + static_cast<int64_t>(r0) * lda;
    const float* a1 = a + static_cast<int64_t>(live1 ? r0 + 1 : r0) * lda;
    if constexpr (FULL) {
        // Unconditional loads, the matrix rows' first: bounds tests around
        // each load had the compiler wait for earlier loads between them.
        f32x4 v0[4], v1[4], vw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v0[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(a0) + t + 256 * i);
            v1[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(a1) + t + 256 * i);
        }
        if constexpr (PROD) {
#pragma unroll
            for (int i = 0; i < 4; ++i) vw[i] = reinterpret_cast<const f32x4*>(xv)[t + 256 * i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x0[4 * i + j] = v0[i][j];
                x1[4 * i + j] = v1[i][j];
                if constexpr (PROD) w[4 * i + j] = vw[i][j];
            }
    } else {
        if constexpr (PROD) load_row<256, 4, false>(w, xv, n, t, true, 1);
        load_row<256, 4>(x0, a0, n, t, true, 1);
        load_row<256, 4>(x1, a1, n, t, true, 1);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t e0 = 4u * (t + 256 * i);
        if (FULL || e0 < n) {
            f32x4 v0, v1;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (PROD) {
                    v0[j] = __fmul_rn(x0[4 * i + j], w[4 * i + j]);
                    v1[j] = __fmul_rn(x1[4 * i + j], w[4 * i + j]);
                } else {
                    v0[j] = x0[4 * i + j];
                    v1[j] = x1[4 * i + j];
                }
            }
            *reinterpret_cast<f32x4*>(dyn + stage_index(e0)) = v0;
            *reinterpret_cast<f32x4*>(dyn + sstride + stage_index(e0)) = v1;
        }
    }
    __syncthreads();
    const int row = t >> 7, leaf = t & 127;
    float v = 0.0f;
    if constexpr (FULL)
        v = staged_leaf_sum(dyn + row * sstride, 32u * leaf, 32u * leaf + 32u);
    else if (static_cast<uint32_t>(leaf) < (1u << depth))
        v = staged_subtree_sum(dyn + row * sstride, n, depth, leaf, 1);
    v = wave_sum_butterfly(v);
    const int lane = t & 63, wave = t >> 6;
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    if (lane == 0 && (wave & 1) == 0) {
        const uint32_t o = r0 + row;
        const float s = scratch[wave] + scratch[wave + 1] + (0.0f + 0.0f);
        if (o < m) y[o] = (!PROD && mean) ? s / static_cast<float>(n) : s;
    }
}

// Selections (max/min/argmax/argmin) over contiguous runs that fit the row
// classes: the thread's elements are loaded up front, scanned in index order,
// then merged across threads with the lowest-index tie-break.

// Selections: thread-strided scan, then (value, index) merges with the
// lowest-index tie-break.
struct Sel {
    float v;
    uint32_t i;  // 0xffffffff = no candidate
};

__device__ __forceinline__ Sel sel_merge(int op, Sel a, Sel b) {
    if (b.i == 0xffffffffu) return a;
    if (a.i == 0xffffffffu) return b;
    const bool is_max = op == VKHIP_REDUCE_MAX || op == VKHIP_REDUCE_ARGMAX;
    if (op == VKHIP_REDUCE_MAX || op == VKHIP_REDUCE_MIN) {
        const bool an = a.v != a.v, bn = b.v != b.v;
        if (an || bn) {
            if (an && bn) return a.i < b.i ? a : b;
            return an ? a : b;
        }
    }
    const bool b_better = is_max ? (b.v > a.v) : (b.v < a.v);
    const bool a_better = is_max ? (a.v > b.v) : (a.v < b.v);
    if (b_better) return b;
    if (a_better) return a;
    return a.i < b.i ? a : b;
}

// The same merge with the operation fixed at compile time, so that a lane's
// merge is a handful of compares and selects rather than a branch tree.
template <int OP>
__device__ __forceinline__ Sel sel_merge_t(Sel a, Sel b) {
    constexpr bool is_max = OP == VKHIP_REDUCE_MAX || OP == VKHIP_REDUCE_ARGMAX;
    constexpr bool value_op = OP == VKHIP_REDUCE_MAX || OP == VKHIP_REDUCE_MIN;
    const bool a_none = a.i == 0xffffffffu, b_none = b.i == 0xffffffffu;
    const bool lower = b.i < a.i;  // "none" is the largest index
    bool take_b;
    if constexpr (value_op) {
        const bool an = a.v != a.v, bn = b.v != b.v;
        const bool b_wins = is_max ? b.v > a.v : b.v < a.v;
        const bool tie = !(a.v > b.v) && !(a.v < b.v);
        take_b = (an || bn) ? (bn && (!an || lower)) : (b_wins || (tie && lower));
    } else {
        const bool b_wins = is_max ? b.v > a.v : b.v < a.v;
        const bool tie = a.v == b.v;
        take_b = b_wins || (tie && lower);
    }
    take_b = !b_none && (a_none || take_b);
    return take_b ? b : a;
}

// Selections over rows held in registers: max/min return the first NaN of the
// row if there is one, else the first of the extreme values (which fixes the
// sign of a zero maximum); argmax/argmin skip NaN and return the lowest index
// of a strict improvement, 0 when nothing improves on the initial +-inf.
//
// FULL: every row fills the thread slots exactly (vec, n == 4 * E4 * T), so
// the loads are unconditional and all issued before the first wait
// ([8192, 4096] max: 22.3 -> 21.9-22.2 us).
template <int T, int E4, int OP, bool FULL>
__global__ __launch_bounds__(Rows<T>::kThreads) void reduce_rows_select_reg_kernel(
    const float* __restrict__ src, Op4 kept, uint32_t n_out, uint32_t n, int vec,
    void* __restrict__ dst) {
    constexpr int RPB = Rows<T>::kPerBlock;
    constexpr bool is_max = OP == VKHIP_REDUCE_MAX || OP == VKHIP_REDUCE_ARGMAX;
    constexpr bool value_op = OP == VKHIP_REDUCE_MAX || OP == VKHIP_REDUCE_MIN;
    constexpr uint32_t kNone = 0xffffffffu;
    __shared__ float sv[RPB][T / 64 > 0 ? T / 64 : 1];
    __shared__ uint32_t si[RPB][T / 64 > 0 ? T / 64 : 1];
    const int slot = threadIdx.x / T;
    const int t = threadIdx.x % T;
    const uint32_t o = blockIdx.x * RPB + slot;
    const bool live = o < n_out;
    const float* rs = src + (live ? lin_off4(o, kept.ne, kept.nb) : 0);
    float x[4 * E4];
    if constexpr (FULL)
        load_row_full<T, E4>(x, rs, t);
    else
        load_row<T, E4>(x, rs, n, t, live, vec);
    // One candidate per thread, scanned in increasing index order. For value
    // ops a NaN outranks every number and the first one stays; the first
    // element is taken even when it equals the initial +-inf.
    float bv = is_max ? -__builtin_inff() : __builtin_inff();
    uint32_t bi = kNone;
#pragma unroll
    for (int i = 0; i < 4 * E4; ++i) {
        const uint32_t e = FULL ? 4u * (t + T * (i / 4)) + (i % 4) : elem_of(vec, T, t, i);
        const float v = x[i];
        const bool valid = live && (FULL || e < n);
        const bool improves = is_max ? v > bv : v < bv;
        bool better;
        if constexpr (value_op) {
            const bool b_nan = bv != bv;
            better = valid && (bi == kNone || (!b_nan && (v != v || improves)));
        } else {
            better = valid && improves;
        }
        bv = better ? v : bv;
        bi = better ? e : bi;
    }
    Sel s{bv, bi};
    s = sel_merge_t<OP>(s, Sel{wave_partner<1>(s.v), static_cast<uint32_t>(wave_partner<1>(static_cast<int>(s.i)))});
    s = sel_merge_t<OP>(s, Sel{wave_partner<2>(s.v), static_cast<uint32_t>(wave_partner<2>(static_cast<int>(s.i)))});
    s = sel_merge_t<OP>(s, Sel{wave_partner<4>(s.v), static_cast<uint32_t>(wave_partner<4>(static_cast<int>(s.i)))});
    s = sel_merge_t<OP>(s, Sel{wave_partner<8>(s.v), static_cast<uint32_t>(wave_partner<8>(static_cast<int>(s.i)))});
    s = sel_merge_t<OP>(s, Sel{wave_partner<16>(s.v), static_cast<uint32_t>(wave_partner<16>(static_cast<int>(s.i)))});
    s = sel_merge_t<OP>(Sel{lane_value(s.v, 0), static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(s.i), 0))},
                        Sel{lane_value(s.v, 32), static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(s.i), 32))});
    if constexpr (T > 64) {
        const int lane = t & 63, wave = t >> 6;
        if (lane == 0) {
            sv[slot][wave] = s.v;
            si[slot][wave] = s.i;
        }
        __syncthreads();
        if (t == 0) {
            for (int w = 1; w < T / 64; ++w) s = sel_merge_t<OP>(s, Sel{sv[slot][w], si[slot][w]});
        }
    }
    if (!live || t != 0) return;
    if constexpr (value_op) {
        static_cast<float*>(dst)[o] = s.i == kNone ? (is_max ? -__builtin_inff() : __builtin_inff()) : s.v;
    } else {
        static_cast<int64_t*>(dst)[o] = s.i == kNone ? 0 : static_cast<int64_t>(s.i);
    }
}

template <int T>
__global__ __launch_bounds__(T >= 256 ? T : 256) void reduce_rows_select_kernel(
    int op, const float* __restrict__ src, Op4 kept, uint32_t n_out, uint32_t n, int vec,
    void* __restrict__ dst) {
    constexpr int RPB = T >= 256 ? 1 : 256 / T;
    __shared__ float sv[RPB][T / 64 > 0 ? T / 64 : 1];
    __shared__ uint32_t si[RPB][T / 64 > 0 ? T / 64 : 1];
    const int slot = threadIdx.x / T;
    const int t = threadIdx.x % T;
    const uint32_t o = blockIdx.x * RPB + slot;
    const bool live = o < n_out;
    const float* rs = src + (live ? lin_off4(o, kept.ne, kept.nb) : 0);
    const bool is_max = op == VKHIP_REDUCE_MAX || op == VKHIP_REDUCE_ARGMAX;
    const bool value_op = op == VKHIP_REDUCE_MAX || op == VKHIP_REDUCE_MIN;
    Sel s{is_max ? -__builtin_inff() : __builtin_inff(), 0xffffffffu};
    // Visits this thread's elements in increasing index order, four at a time.
    auto visit = [&](float v, uint32_t e, bool& stop) {
        if (v != v) {
            if (value_op) {
                s = Sel{v, e};  // first NaN of this thread's subsequence
                stop = true;
            }
            return;
        }
        // Value ops take the first element as their candidate even if it is
        // +-inf; index ops need a strict improvement on +-inf, as the
        // oracle's loops do.
        const bool better = is_max ? v > s.v : v < s.v;
        if (better || (value_op && s.i == 0xffffffffu)) s = Sel{v, e};
    };
    if (live) {
        bool stop = false;
        if (vec) {
            for (uint32_t e0 = 4u * t; e0 < n && !stop; e0 += 4u * T) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(rs + e0);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (!stop) visit(v[j], e0 + j, stop);
            }
        } else {
            for (uint32_t e = t; e < n && !stop; e += T) visit(rs[e], e, stop);
        }
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        Sel o2{__shfl_xor(s.v, off, 64), static_cast<uint32_t>(__shfl_xor(static_cast<int>(s.i), off, 64))};
        s = sel_merge(op, s, o2);
    }
    if constexpr (T > 64) {
        const int lane = t & 63, wave = t >> 6;
        if (lane == 0) {
            sv[slot][wave] = s.v;
            si[slot][wave] = s.i;
        }
        __syncthreads();
        if (t == 0) {
            for (int w = 1; w < T / 64; ++w) s = sel_merge(op, s, Sel{sv[slot][w], si[slot][w]});
        }
    }
    if (!live || t != 0) return;
    if (value_op) {
        static_cast<float*>(dst)[o] = s.i == 0xffffffffu ? (is_max ? -__builtin_inff() : __builtin_inff()) : s.v;
    } else {
        static_cast<int64_t*>(dst)[o] = s.i == 0xffffffffu ? 0 : static_cast<int64_t>(s.i);
    }
}

// ---- one workgroup per output: any layout, many reduced elements ---------------------
// Sum / mean over a reduced set that is not one contiguous run (e.g. a conv
// bias gradient, axes {0, 2, 3}), with few outputs: T threads share one
// output, each owning consecutive depth-D leaves read through the reduced
// descriptor, combined by the same butterfly as the staged kernels.
template <int T>
__global__ __launch_bounds__(T) void reduce_wide_strided_kernel(
    const float* __restrict__ src, Op4 kept, Reader rd, uint32_t n, int depth, int mean,
    float* __restrict__ dst) {
    __shared__ float scratch[T / 64];
    const int t = threadIdx.x;
    const uint32_t o = blockIdx.x;
    const float* base = src + lin_off4(o, kept.ne, kept.nb);
    const uint32_t leaves = 1u << depth;
    const uint32_t per = leaves > static_cast<uint32_t>(T) ? leaves / T : 1u;
    float v = 0.0f;
    if (static_cast<uint32_t>(t) * per < leaves) {
        float stack[kTallLevels];
#pragma unroll
        for (int l = 0; l < kTallLevels; ++l) stack[l] = 0.0f;
        for (uint32_t j = 0; j < per; ++j) {
            uint32_t b, e;
            pairwise_leaf(n, depth, t * per + j, b, e);
            float sv = 0.0f;
            for (uint32_t q = b; q < e; ++q) sv = sv + base[rd.off(q)];
            bool carry = true;
#pragma unroll
            for (int l = 0; l < kTallLevels; ++l) {
                if (carry) {
                    if ((j >> l) & 1u) {
                        sv = stack[l] + sv;
                    } else {
                        stack[l] = sv;
                        carry = false;
                    }
                }
            }
        }
#pragma unroll
        for (int l = 0; l < kTallLevels; ++l)
            if ((1u << l) == per) v = stack[l];
    }
    v = wave_sum_butterfly(v);
    const int lane = t & 63, wave = t >> 6;
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float u = lane < T / 64 ? scratch[lane] : 0.0f;
    u = wave_sum_butterfly(u);
    if (t == 0) dst[o] = mean ? u / static_cast<float>(n) : u;
}

// ---- sums with few outputs over many elements: split tree ----------------------
// The oracle's pairwise recursion is self-similar: the node reached from the
// root by the d bits of j (MSB first, midpoint splits) is the pairwise sum of
// its own range, and the top d levels above those nodes only add left + right.
// So a sum over n elements splits exactly into 2^d subtree sums (one workgroup
// each, staged in LDS from coalesced loads and summed with the same leaf
// machinery as the row kernels, depth D - d inside the subtree) and a balanced
// fold of the 2^d partials. A node at depth < d that is already a leaf is
// carried by its leftmost descendant and the others contribute +0.0, which
// leaves every sum unchanged.
constexpr uint32_t kSubtreeMax = 8192;  // elements one workgroup stages

__global__ __launch_bounds__(256) void reduce_subtree_kernel(const float* __restrict__ src,
                                                             Op4 kept, Reader rd, uint32_t n,
                                                             int depth, int split, int vec,
                                                             float* __restrict__ partial) {
    __shared__ __attribute__((aligned(16))) float stage[(kSubtreeMax + 4 * (kSubtreeMax / 32) + 3) & ~3u];
    __shared__ float scratch[4];
    const uint32_t j = blockIdx.x, o = blockIdx.y;
    const float* base = src + lin_off4(o, kept.ne, kept.nb);
    uint32_t b, e;
    pairwise_leaf(n, split, j, b, e);
    const uint32_t m = e - b;
    constexpr int kBatch = kSubtreeMax / 256;
    if (vec && (b & 3u) == 0) {
        // Runs of four consecutive reduced elements are adjacent and 16-byte
        // aligned (host-checked): one offset and one 16-byte load per four,
        // staged as one 16-byte store (stage_index keeps groups of four).
        f32x4_t v[kBatch / 4];
#pragma unroll
        for (int r = 0; r < kBatch / 4; ++r) {
            const uint32_t i = 4u * (threadIdx.x + 256u * r);
            if (i + 3 < m) {
                v[r] = *reinterpret_cast<const f32x4_t*>(base + rd.off(b + i));
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) v[r][q] = i + q < m ? base[rd.off(b + i + q)] : 0.0f;
            }
        }
#pragma unroll
        for (int r = 0; r < kBatch / 4; ++r) {
            const uint32_t i = 4u * (threadIdx.x + 256u * r);
            if (i < m) *reinterpret_cast<f32x4_t*>(stage + stage_index(i)) = v[r];
        }
    } else {
        float v[kBatch];
#pragma unroll
        for (int r = 0; r < kBatch; ++r) {
            const uint32_t i = threadIdx.x + 256u * r;
            v[r] = i < m ? base[rd.off(b + i)] : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < kBatch; ++r) {
            const uint32_t i = threadIdx.x + 256u * r;
            if (i < m) stage[stage_index(i)] = v[r];
        }
    }
    __syncthreads();
    const float sum = group_pairwise_sum<256>(stage, m, depth - split, threadIdx.x, scratch);
    if (threadIdx.x == 0) partial[static_cast<uint64_t>(j) * gridDim.y + o] = sum;
}

// Balanced fold of the 2^split partials of each output (a carry stack over
// 2^split pushes is exactly that tree).
__global__ __launch_bounds__(256) void reduce_subtree_fold_kernel(const float* __restrict__ partial,
                                                                  uint32_t n_out, int split,
                                                                  uint32_t n, int mean,
                                                                  float* __restrict__ dst) {
    const uint32_t o = blockIdx.x * 256 + threadIdx.x;
    if (o >= n_out) return;
    float stack[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) stack[l] = 0.0f;
    const uint32_t parts = 1u << split;
    // The partials of a group of eight are loaded before any is pushed, so
    // their latencies overlap (one dependent load per push took ~5 us for 16).
    for (uint32_t j0 = 0; j0 < parts; j0 += 8) {
        float pv[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
            pv[q] = j0 + q < parts ? partial[static_cast<uint64_t>(j0 + q) * n_out + o] : 0.0f;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const uint32_t j = j0 + q;
            if (j >= parts) break;
            float sv = pv[q];
            bool carry = true;
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                if (carry) {
                    if ((j >> l) & 1u) {
                        sv = stack[l] + sv;
                    } else {
                        stack[l] = sv;
                        carry = false;
                    }
                }
            }
        }
    }
    float total = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; ++l)
        if ((1u << l) == parts) total = stack[l];
    dst[o] = mean ? total / static_cast<float>(n) : total;
}

// ---- host side ----------------------------------------------------------------------

static void split_axes(const vkhip_operand& d, uint32_t mask, Op4& kept, Op4& red) {
    int kc = 0, rc = 0;
    uint32_t kn[4], rn[4];
    int64_t ks[4], rs[4];
    for (int i = 0; i < 4; ++i) {
        if (mask & (1u << i)) {
            rn[rc] = d.ne[i];
            rs[rc++] = d.nb[i];
        } else {
            kn[kc] = d.ne[i];
            ks[kc++] = d.nb[i];
        }
    }
    for (int i = 0; i < 4; ++i) {
        kept.ne[i] = 1;
        kept.nb[i] = 0;
        red.ne[i] = 1;
        red.nb[i] = 0;
    }
    for (int i = 0; i < kc; ++i) {
        kept.ne[4 - kc + i] = kn[i];
        kept.nb[4 - kc + i] = ks[i];
    }
    for (int i = 0; i < rc; ++i) {
        red.ne[4 - rc + i] = rn[i];
        red.nb[4 - rc + i] = rs[i];
    }
}

static uint64_t numel_op4(const Op4& o) {
    return static_cast<uint64_t>(o.ne[0]) * o.ne[1] * o.ne[2] * o.ne[3];
}

// True when the elements of `o` form one contiguous run, row-major, stride 1.
static bool contiguous_run(const Op4& o) {
    int64_t expect = 1;
    for (int i = 3; i >= 0; --i) {
        if (o.ne[i] == 1) continue;
        if (o.nb[i] != expect) return false;
        expect *= o.ne[i];
    }
    return true;
}

// The reduced elements lie on at most one non-unit axis: its stride.
constexpr uint32_t kRowsMax = 32768;  // longest run staged in LDS

// Row size classes: T threads per row and E4 float4 groups per thread.
struct RowClass {
    int T, E4;
};

static RowClass row_class(uint32_t n) {
    if (n <= 256) return {64, 1};
    if (n <= 1024) return {64, 4};
    if (n <= 2048) return {64, 8};
    if (n <= 4096) return {256, 4};
    if (n <= 8192) return {256, 8};
    if (n <= 16384) return {1024, 4};
    return {1024, 8};
}

// Dynamic LDS above 64 KiB must be opted into per kernel.
static int allow_lds(const void* fn, size_t bytes) {
    if (bytes <= 65536) return VKHIP_OK;
    VKHIP_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  static_cast<int>(bytes)));
    return VKHIP_OK;
}

template <int T, int E4>
static int launch_sum_rows(const float* src, const Op4& kept, uint32_t n_out, uint32_t n, int depth,
                           int mean, int vec, float* out, hipStream_t st, const float* xv) {
    constexpr int RPB = Rows<T>::kPerBlock;
    const uint32_t ss = stage_stride(n);
    const size_t lds = static_cast<size_t>(RPB) * ss * sizeof(float);
    if (xv) {
        auto fn = reduce_rows_sum_kernel<T, E4, true>;
        int rc = allow_lds(reinterpret_cast<const void*>(fn), lds);
        if (rc != VKHIP_OK) return rc;
        hipLaunchKernelGGL(fn, dim3(ceil_div(n_out, RPB)), dim3(Rows<T>::kThreads), lds, st, src,
                           kept, n_out, n, depth, mean, vec, ss, out, xv);
    } else {
        auto fn = reduce_rows_sum_kernel<T, E4, false>;
        int rc = allow_lds(reinterpret_cast<const void*>(fn), lds);
        if (rc != VKHIP_OK) return rc;
        hipLaunchKernelGGL(fn, dim3(ceil_div(n_out, RPB)), dim3(Rows<T>::kThreads), lds, st, src,
                           kept, n_out, n, depth, mean, vec, ss, out, xv);
    }
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

template <int T, int E4, bool FULL>
static int launch_select_rows_as(int op, const float* src, const Op4& kept, uint32_t n_out,
                                 uint32_t n, int vec, void* out, hipStream_t st) {
    constexpr int RPB = Rows<T>::kPerBlock;
    const dim3 grid(ceil_div(n_out, RPB)), block(Rows<T>::kThreads);
    switch (op) {
        case VKHIP_REDUCE_MAX:
            hipLaunchKernelGGL((reduce_rows_select_reg_kernel<T, E4, VKHIP_REDUCE_MAX, FULL>), grid,
                               block, 0, st, src, kept, n_out, n, vec, out);
            break;
        case VKHIP_REDUCE_MIN:
            hipLaunchKernelGGL((reduce_rows_select_reg_kernel<T, E4, VKHIP_REDUCE_MIN, FULL>), grid,
                               block, 0, st, src, kept, n_out, n, vec, out);
            break;
        case VKHIP_REDUCE_ARGMAX:
            hipLaunchKernelGGL((reduce_rows_select_reg_kernel<T, E4, VKHIP_REDUCE_ARGMAX, FULL>), grid,
                               block, 0, st, src, kept, n_out, n, vec, out);
            break;
        case VKHIP_REDUCE_ARGMIN:
            hipLaunchKernelGGL((reduce_rows_select_reg_kernel<T, E4, VKHIP_REDUCE_ARGMIN, FULL>), grid,
                               block, 0, st, src, kept, n_out, n, vec, out);
            break;
        default:
            return fail(VKHIP_ERR_INVALID, "select reduce: unknown op %d", op);
    }
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

template <int T, int E4>
static int launch_select_rows(int op, const float* src, const Op4& kept, uint32_t n_out,
                              uint32_t n, int vec, void* out, hipStream_t st) {
    if (vec && n == 4u * E4 * T)
        return launch_select_rows_as<T, E4, true>(op, src, kept, n_out, n, vec, out, st);
    return launch_select_rows_as<T, E4, false>(op, src, kept, n_out, n, vec, out, st);
}

template <int T, int E4>
static int launch_softmax_rows(const float* src, int64_t stride, float* dst, uint32_t rows,
                               uint32_t n, int log_mode, int vec, hipStream_t st) {
    constexpr int RPB = Rows<T>::kPerBlock;
    if constexpr (T == 1024) {
        if (vec) {  // one (peak, sum) reduction per row
            const bool full = n == 4u * E4 * 1024u;
            auto fo = log_mode ? (full ? softmax_online_rows_kernel<E4, true, true> : softmax_online_rows_kernel<E4, true, false>)
                               : (full ? softmax_online_rows_kernel<E4, false, true> : softmax_online_rows_kernel<E4, false, false>);
            hipLaunchKernelGGL(fo, dim3(rows), dim3(1024), 0, st, src, stride, dst, rows, n);
            VKHIP_LAUNCH_CHECK();
            return VKHIP_OK;
        }
    }
    auto fn = log_mode ? softmax_rows_kernel<T, E4, true> : softmax_rows_kernel<T, E4, false>;
    hipLaunchKernelGGL(fn, dim3(ceil_div(rows, RPB)), dim3(Rows<T>::kThreads), 0, st, src,
                       stride, dst, rows, n, vec);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

#define VKHIP_ROW_CLASSES(FN, ...)                                         \
    switch (rc.T * 100 + rc.E4) {                                          \
        case 6401: return FN<64, 1>(__VA_ARGS__);                          \
        case 6404: return FN<64, 4>(__VA_ARGS__);                          \
        case 6408: return FN<64, 8>(__VA_ARGS__);                          \
        case 25604: return FN<256, 4>(__VA_ARGS__);                        \
        case 25608: return FN<256, 8>(__VA_ARGS__);                        \
        case 102404: return FN<1024, 4>(__VA_ARGS__);                      \
        default: return FN<1024, 8>(__VA_ARGS__);                          \
    }

static const char* reduce_name(int op) {
    switch (op) {
        case VKHIP_REDUCE_SUM: return "sum";
        case VKHIP_REDUCE_MEAN: return "mean";
        case VKHIP_REDUCE_MAX: return "max";
        case VKHIP_REDUCE_MIN: return "min";
        case VKHIP_REDUCE_ARGMAX: return "argmax";
        default: return "argmin";
    }
}

int launch_reduce(int op, const float* src, const vkhip_operand& d, uint32_t mask, void* dst) {
    if (op < VKHIP_REDUCE_SUM || op > VKHIP_REDUCE_ARGMIN)
        return fail(VKHIP_ERR_INVALID, "reduce: unknown op %d", op);
    Op4 kept, red;
    split_axes(d, mask & 0xfu, kept, red);
    const uint64_t n_out64 = numel_op4(kept), n_red64 = numel_op4(red);
    if (n_out64 == 0) return VKHIP_OK;
    if (n_red64 >= (1ull << 26) || n_out64 > 0xffffffffull)
        return fail(VKHIP_ERR_UNSUPPORTED, "reduce: extents too large");
    const uint32_t n_out = static_cast<uint32_t>(n_out64), n_red = static_cast<uint32_t>(n_red64);
    hipStream_t st = ctx().stream;
    const bool sum_op = op == VKHIP_REDUCE_SUM || op == VKHIP_REDUCE_MEAN;
    const bool run = contiguous_run(red);
    // Structure rule (reference vulkan_backend.cpp:1912-1920, restated for a
    // 256-CU part): a workgroup per output when the reduced run is contiguous
    // and long enough to feed it; otherwise a lane per output, which coalesces
    // when the kept axis is the contiguous one. Both give identical results.
    const bool wide = run && n_red >= 32 && (!sum_op || n_red <= kRowsMax);
    const char* rname = reduce_name(op);
    if (wide) {
        publish("reduce.structure", rname, "reduce_workgroup_tree", "reduce_lane_per_output",
                "the reduced elements form one contiguous run per output", n_red, n_out);
        const int vec = (reinterpret_cast<uintptr_t>(src) % 16 == 0) && (n_red % 4 == 0) &&
                        (kept.nb[0] % 4 == 0) && (kept.nb[1] % 4 == 0) && (kept.nb[2] % 4 == 0) &&
                        (kept.nb[3] % 4 == 0);
        if (sum_op) {
            const int depth = pairwise_depth(n_red);
            const int mean = op == VKHIP_REDUCE_MEAN;
            float* out = static_cast<float*>(dst);
            const RowClass rc = row_class(n_red);
            if (vec && n_red > 2048 && n_red <= 4096 && n_out >= 2 && kept.ne[0] == 1 &&
                kept.ne[1] == 1 && kept.ne[2] == 1) {
                const uint32_t ss = stage_stride(n_red);
                auto* kern = n_red == 4096 ? rows2_sum_kernel<false, true> : rows2_sum_kernel<false, false>;
                hipLaunchKernelGGL(kern, dim3(ceil_div(n_out, 2u)), dim3(256),
                                   2 * static_cast<size_t>(ss) * sizeof(float), st, src, kept.nb[3],
                                   nullptr, out, n_out, n_red, depth, ss, mean);
                VKHIP_LAUNCH_CHECK();
                return VKHIP_OK;
            }
            VKHIP_ROW_CLASSES(launch_sum_rows, src, kept, n_out, n_red, depth, mean, vec, out, st,
                              nullptr)
        }
        if (n_red <= kRowsMax) {
            const RowClass rc = row_class(n_red);
            VKHIP_ROW_CLASSES(launch_select_rows, op, src, kept, n_out, n_red, vec, dst, st)
        }
        hipLaunchKernelGGL((reduce_rows_select_kernel<256>), dim3(n_out), dim3(256), 0, st, op,
                           src, kept, n_out, n_red, vec, dst);
        VKHIP_LAUNCH_CHECK();
        return VKHIP_OK;
    }
    const Reader rd = make_reader(red);
    const int depth = pairwise_depth(n_red);
    const uint32_t cus = ctx().ready ? static_cast<uint32_t>(ctx().caps.compute_units) : 256u;
    if (sum_op && n_red >= 2048 && n_out < 4 * cus) {
        // Split into 2^split subtrees of at most kSubtreeMax elements, with
        // enough workgroups for two per CU, keeping split <= depth and the
        // partials within 2^7 per output.
        int split = 0;
        while (split < depth && split < 7 &&
               (((static_cast<uint64_t>(n_red) + (1ull << split) - 1) >> split) > kSubtreeMax ||
                (static_cast<uint64_t>(n_out) << split) < 2ull * cus))
            ++split;
        if (((static_cast<uint64_t>(n_red) + (1ull << split) - 1) >> split) <= kSubtreeMax &&
            split > 0) {
            publish("reduce.structure", rname, "reduce_split_tree", "reduce_lane_per_output",
                    "few outputs over many strided elements: one workgroup per subtree",
                    n_red, n_out);
            float* part = nullptr;
            int rc = workspace((static_cast<size_t>(n_out) << split) * sizeof(float), &part);
            if (rc != VKHIP_OK) return rc;
            // 16-byte loads: the innermost reduced axis contiguous in groups of
            // four, every other stride and the base 16-byte aligned.
            bool vec4 = reinterpret_cast<uintptr_t>(src) % 16 == 0;
            if (rd.naxes == 1) {
                vec4 = vec4 && rd.nb_outer == 1;
            } else {
                vec4 = vec4 && rd.nb[0] == 1 && rd.ne[0] % 4 == 0 && rd.nb_outer % 4 == 0;
                for (int a = 1; a + 1 < rd.naxes; ++a) vec4 = vec4 && rd.nb[a] % 4 == 0;
            }
            for (int a = 0; a < 4; ++a) vec4 = vec4 && (kept.ne[a] == 1 || kept.nb[a] % 4 == 0);
            hipLaunchKernelGGL(reduce_subtree_kernel, dim3(1u << split, n_out), dim3(256), 0, st,
                               src, kept, rd, n_red, depth, split, vec4 ? 1 : 0, part);
            VKHIP_LAUNCH_CHECK();
            hipLaunchKernelGGL(reduce_subtree_fold_kernel, dim3(ceil_div(n_out, 256)), dim3(256), 0,
                               st, part, n_out, split, n_red, op == VKHIP_REDUCE_MEAN ? 1 : 0,
                               static_cast<float*>(dst));
            VKHIP_LAUNCH_CHECK();
            return VKHIP_OK;
        }
    }
    if (sum_op && n_red >= 8192 && n_out < 4 * cus) {
        publish("reduce.structure", rname, "reduce_workgroup_strided", "reduce_split_tree",
                "subtrees too long to stage in LDS", n_red, n_out);
        hipLaunchKernelGGL(reduce_wide_strided_kernel<256>, dim3(n_out), dim3(256), 0, st, src,
                           kept, rd, n_red, depth, op == VKHIP_REDUCE_MEAN ? 1 : 0,
                           static_cast<float*>(dst));
        VKHIP_LAUNCH_CHECK();
        return VKHIP_OK;
    }
    if (sum_op && depth >= 1 && depth <= 3 && n_out < (1ull << 32) - 64) {
        publish("reduce.structure", rname, "reduce_wave_per_leaf", "reduce_lane_per_output",
                "the reduced elements are strided, at most 8 pairwise leaves per output",
                n_red, n_out);
        const dim3 grid(ceil_div(n_out, 64));
        const int mean = op == VKHIP_REDUCE_MEAN ? 1 : 0;
        float* out = static_cast<float*>(dst);
        if (depth == 1)
            hipLaunchKernelGGL(reduce_tall_leaves_kernel<2>, grid, dim3(128), 0, st, src, kept, rd,
                               n_out, n_red, mean, out);
        else if (depth == 2)
            hipLaunchKernelGGL(reduce_tall_leaves_kernel<4>, grid, dim3(256), 0, st, src, kept, rd,
                               n_out, n_red, mean, out);
        else
            hipLaunchKernelGGL(reduce_tall_leaves_kernel<8>, grid, dim3(512), 0, st, src, kept, rd,
                               n_out, n_red, mean, out);
        VKHIP_LAUNCH_CHECK();
        return VKHIP_OK;
    }
    publish("reduce.structure", rname, "reduce_lane_per_output", "reduce_workgroup_tree",
            "the reduced elements are strided", n_red, n_out);
    hipLaunchKernelGGL(reduce_tall_kernel, dim3(ceil_div(n_out, 256)), dim3(256), 0, st, op, src,
                       kept, rd, static_cast<uint64_t>(n_out), n_red, depth, dst);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

// ---- softmax host side ------------------------------------------------------------

template <bool EXACT>
__global__ __launch_bounds__(256) void softmax_tall_kernel(const float* __restrict__ src, Op4 kept,
                                                           Reader rd, Op4 okept, Reader ord,
                                                           uint64_t n_out, uint32_t n, int depth,
                                                           int log_mode, float* __restrict__ dst) {
    const uint64_t o = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (o >= n_out) return;
    const float* base = src + lin_off4(static_cast<uint32_t>(o), kept.ne, kept.nb);
    float* obase = dst + lin_off4(static_cast<uint32_t>(o), okept.ne, okept.nb);
    float peak = -__builtin_inff();
    for (uint32_t i = 0; i < n; ++i) peak = max_ignoring_nan(peak, base[rd.off(i)]);
    float stack[kTallLevels];
#pragma unroll
    for (int l = 0; l < kTallLevels; ++l) stack[l] = 0.0f;
    const uint32_t leaves = 1u << depth;
    for (uint32_t j = 0; j < leaves; ++j) {
        uint32_t b, e;
        pairwise_leaf(n, depth, j, b, e);
        float s = 0.0f;
        for (uint32_t q = b; q < e; ++q) {
            const float sh = base[rd.off(q)] - peak;
            s = s + (EXACT ? exact_expf(sh) : softmax_exp(sh));
        }
        bool carry = true;
#pragma unroll
        for (int l = 0; l < kTallLevels; ++l) {
            if (carry) {
                if ((j >> l) & 1u) {
                    s = stack[l] + s;
                } else {
                    stack[l] = s;
                    carry = false;
                }
            }
        }
    }
    float denom = 0.0f;
#pragma unroll
    for (int l = 0; l < kTallLevels; ++l)
        if (l == depth) denom = stack[l];
    const float ld = EXACT ? exact_logf(denom) : logf(denom);
    for (uint32_t i = 0; i < n; ++i) {
        const float sh = base[rd.off(i)] - peak;
        obase[ord.off(i)] = log_mode ? sh - ld : (EXACT ? exact_expf(sh) : softmax_exp(sh)) / denom;
    }
}

// ---- softmax over rows longer than a workgroup holds ------------------------------
// Rows beyond kRowsMax floats are cut into chunks of kSmxChunk floats, one
// workgroup each, in two launches:
//   1. per chunk c: its peak m_c and s_c = sum of exp(x - m_c) over the chunk;
//   2. per chunk: the row's peak M = max_c m_c and denominator
//      d = sum_c s_c * exp(m_c - M), c ascending (the same arithmetic in every
//      workgroup of the row), then the chunk's outputs exp(x - M) / d or
//      (x - M) - log(d).
// The second launch re-reads its chunk, which the first has just pulled
// through the memory-side cache. (For 256x32768 this measured 17.9 us against
// 15.8 for a workgroup per row, so shorter rows keep that path.) The
// denominator is the oracle's sum re-associated (a few ulp; softmax parity is
// tolerance-based). Special values come out as the oracle's: a chunk of -inf
// only contributes 0, a NaN or +inf anywhere in a row makes the row NaN, an
// all -inf row is NaN.
constexpr uint32_t kSmxChunk = 4096;     // floats per workgroup (16 per thread)
constexpr uint32_t kSmxMaxChunks = 256;  // rows up to 2^20 floats

struct SmxStat {
    float peak, sum;
};

template <bool VEC>
__device__ __forceinline__ void load_chunk(float (&x)[16], bool (&keep)[16], const float* rs,
                                           uint32_t b, uint32_t e, int t) {
    if constexpr (VEC) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t e0 = b + 4u * (t + 256 * i);
            f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
            if (e0 < e) v = *reinterpret_cast<const f32x4*>(rs + e0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x[4 * i + j] = v[j];
                keep[4 * i + j] = e0 < e;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t q = b + t + 256u * i;
            keep[i] = q < e;
            x[i] = keep[i] ? rs[q] : 0.0f;
        }
    }
}

template <bool VEC>
__global__ __launch_bounds__(256) void softmax_chunk_stats_kernel(const float* __restrict__ src,
                                                                  int64_t stride, uint32_t n,
                                                                  uint32_t chunks,
                                                                  SmxStat* __restrict__ stats) {
    __shared__ float scratch[4];
    const int t = threadIdx.x;
    const uint32_t row = blockIdx.x / chunks, c = blockIdx.x % chunks;
    const float* rs = src + static_cast<int64_t>(row) * stride;
    const uint32_t b = c * kSmxChunk, e = min(n, b + kSmxChunk);
    float x[16];
    bool keep[16];
    load_chunk<VEC>(x, keep, rs, b, e, t);
    const float m = group_max<256>(tree_peak<16>(x, keep), t, scratch);
    const bool all_ninf = m == -__builtin_inff();
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        // -inf - (-inf) would be NaN: a chunk of -inf only adds zeros (a NaN
        // element still gives NaN).
        const float sh = (all_ninf && x[i] == -__builtin_inff()) ? -__builtin_inff() : x[i] - m;
        if (keep[i]) sum = sum + softmax_exp(sh);
    }
    sum = wave_sum_butterfly(sum);
    if ((t & 63) == 0) scratch[t >> 6] = sum;
    __syncthreads();
    if (t == 0) stats[blockIdx.x] = SmxStat{m, (scratch[0] + scratch[1]) + (scratch[2] + scratch[3])};
}

template <bool VEC, bool LOG>
__global__ __launch_bounds__(256) void softmax_chunk_apply_kernel(const float* __restrict__ src,
                                                                  int64_t stride,
                                                                  float* __restrict__ dst, uint32_t n,
                                                                  uint32_t chunks,
                                                                  const SmxStat* __restrict__ stats) {
    const int t = threadIdx.x;
    const uint32_t row = blockIdx.x / chunks, c = blockIdx.x % chunks;
    const float* rs = src + static_cast<int64_t>(row) * stride;
    const uint32_t b = c * kSmxChunk, e = min(n, b + kSmxChunk);
    float x[16];
    bool keep[16];
    load_chunk<VEC>(x, keep, rs, b, e, t);

    const SmxStat* rstat = stats + static_cast<uint64_t>(row) * chunks;
    float peak = -__builtin_inff();
    for (uint32_t j = 0; j < chunks; ++j) peak = __builtin_fmaxf(peak, rstat[j].peak);
    float denom = 0.0f;
    for (uint32_t j = 0; j < chunks; ++j) denom = denom + rstat[j].sum * softmax_exp(rstat[j].peak - peak);
    const float ld = logf(denom);
    const float rinv = 1.0f / denom;

    float* ds = dst + static_cast<uint64_t>(row) * n;
    if constexpr (VEC) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t e0 = b + 4u * (t + 256 * i);
            if (e0 < e) {
                f32x4 o;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float sh = x[4 * i + j] - peak;
                    o[j] = LOG ? sh - ld : softmax_exp(sh) * rinv;
                }
                __builtin_nontemporal_store(o, reinterpret_cast<f32x4*>(ds + e0));
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t q = b + t + 256u * i;
            if (keep[i]) {
                const float sh = x[i] - peak;
                ds[q] = LOG ? sh - ld : softmax_exp(sh) * rinv;
            }
        }
    }
}

template <bool VEC>
static int launch_softmax_split(const float* src, int64_t row_stride, float* dst, uint32_t rows,
                                uint32_t n, int log_mode, hipStream_t st) {
    const uint32_t chunks = ceil_div(n, kSmxChunk);
    SmxStat* stats = nullptr;
    int rc = workspace(static_cast<size_t>(rows) * chunks * sizeof(SmxStat),
                       reinterpret_cast<float**>(&stats));
    if (rc != VKHIP_OK) return rc;
    const dim3 grid(rows * chunks);
    hipLaunchKernelGGL(softmax_chunk_stats_kernel<VEC>, grid, dim3(256), 0, st, src, row_stride, n,
                       chunks, stats);
    VKHIP_LAUNCH_CHECK();
    if (log_mode)
        hipLaunchKernelGGL((softmax_chunk_apply_kernel<VEC, true>), grid, dim3(256), 0, st, src,
                           row_stride, dst, n, chunks, stats);
    else
        hipLaunchKernelGGL((softmax_chunk_apply_kernel<VEC, false>), grid, dim3(256), 0, st, src,
                           row_stride, dst, n, chunks, stats);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

// Contiguous rows of up to 2048 floats: a wave per row, persistent with
// next-row prefetch when there are more rows than waves. (A variant that kept
// each thread's own 32-float leaves in registers for 4096..32768-wide rows was
// measured and dropped: each lane reading 128 contiguous bytes runs the loads
// at 3.6 TB/s against 5.8 for lane-interleaved 16-byte loads, so the staged
// row-class kernel is faster at those widths: 256x32768 in 18.7 against
// 22.8 us.)
template <bool LOG>
static int launch_softmax_short(const float* src, int64_t row_stride, float* dst, uint32_t rows,
                                uint32_t n, int depth, int vec, hipStream_t st) {
    if (n > 2048) return fail(VKHIP_ERR_INVALID, "softmax: short-row path given n=%u", n);
    const uint32_t ss = stage_stride(n);
    const size_t lds = 4 * static_cast<size_t>(ss) * sizeof(float);
    const uint32_t cus = ctx().ready ? static_cast<uint32_t>(ctx().caps.compute_units) : 256u;
    // Up to four workgroups (16 waves) per CU: on MI355X one row per wave at
    // that occupancy beat two rows per wave at half of it (4096x1000: 10.5 vs
    // 11.3 us); more rows than waves are walked with the next-row prefetch.
    const uint32_t want = ceil_div(rows, 4);
    const uint32_t blocks = want < cus * 4 ? want : cus * 4;
    void (*fn)(const float*, int64_t, float*, uint32_t, uint32_t, int, uint32_t);
    if (n <= 256)
        fn = vec ? softmax_wave_rows_kernel<1, LOG, true> : softmax_wave_rows_kernel<1, LOG, false>;
    else if (n <= 1024)
        fn = vec ? softmax_wave_rows_kernel<4, LOG, true> : softmax_wave_rows_kernel<4, LOG, false>;
    else
        fn = vec ? softmax_wave_rows_kernel<8, LOG, true> : softmax_wave_rows_kernel<8, LOG, false>;
    hipLaunchKernelGGL(fn, dim3(blocks), dim3(256), lds, st, src, row_stride, dst, rows, n, depth, ss);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

int launch_softmax(const float* src, const vkhip_operand& d, float* dst, int axis, int log_mode) {
    if (axis < 0 || axis > 3) return fail(VKHIP_ERR_INVALID, "softmax: axis %d outside 0..3", axis);
    Op4 kept, red;
    split_axes(d, 1u << axis, kept, red);
    const uint64_t n_out64 = numel_op4(kept);
    const uint32_t n = d.ne[axis];
    if (n_out64 == 0 || n == 0) return VKHIP_OK;
    if (n_out64 > 0xffffffffull || n >= (1u << 26))
        return fail(VKHIP_ERR_UNSUPPORTED, "softmax: extents too large");
    const uint32_t rows = static_cast<uint32_t>(n_out64);
    hipStream_t st = ctx().stream;
    const int depth = pairwise_depth(n);
    if (ctx().exact_math) {
        // Exact numerics: one thread per row for every layout, the oracle's
        // sequence (peak, the pairwise sum of exp over the row, log of it or
        // a true division) with the oracle's exp and log.
        publish("softmax.structure", log_mode ? "log_softmax" : "softmax", "softmax_exact_lane_per_row",
                "softmax_wave_per_row", "exact numerics mode", n, rows);
        vkhip_operand od;
        int64_t s = 1;
        for (int i = 3; i >= 0; --i) {
            od.ne[i] = d.ne[i];
            od.nb[i] = s;
            s *= d.ne[i];
        }
        Op4 okept, ored;
        split_axes(od, 1u << axis, okept, ored);
        hipLaunchKernelGGL(softmax_tall_kernel<true>, dim3(ceil_div(rows, 256)), dim3(256), 0, st, src,
                           kept, single_reader(d.nb[axis]), okept, single_reader(od.nb[axis]), n_out64,
                           n, depth, log_mode, dst);
        VKHIP_LAUNCH_CHECK();
        return VKHIP_OK;
    }
    // Fast path: softmax over the innermost, unit-stride axis, rows evenly spaced.
    int64_t row_stride = 0;
    bool rows_regular = true;
    {
        // Kept offsets must be o * row_stride for a single stride.
        int64_t expect = -1;
        int64_t acc = 1;
        for (int i = 3; i >= 0; --i) {
            if (kept.ne[i] == 1) continue;
            if (expect < 0) {
                row_stride = kept.nb[i];
                expect = kept.nb[i];
            }
            if (kept.nb[i] != row_stride * acc) rows_regular = false;
            acc *= kept.ne[i];
        }
        if (expect < 0) row_stride = n;
    }
    const bool split = axis == 3 && d.nb[3] == 1 && rows_regular && n > kRowsMax &&
                       ceil_div(n, kSmxChunk) <= kSmxMaxChunks &&
                       static_cast<uint64_t>(rows) * ceil_div(n, kSmxChunk) < (1ull << 31);
    if (split) {
        const bool vec = (reinterpret_cast<uintptr_t>(src) % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(dst) % 16 == 0) && (n % 4 == 0) &&
                         (row_stride % 4 == 0);
        publish("softmax.structure", log_mode ? "log_softmax" : "softmax", "softmax_split_rows",
                "softmax_workgroup_per_row", "rows longer than one workgroup's registers hold",
                n, rows);
        return vec ? launch_softmax_split<true>(src, row_stride, dst, rows, n, log_mode, st)
                   : launch_softmax_split<false>(src, row_stride, dst, rows, n, log_mode, st);
    }
    if (axis == 3 && d.nb[3] == 1 && rows_regular && n <= kRowsMax) {
        const int vec = (reinterpret_cast<uintptr_t>(src) % 16 == 0) &&
                        (reinterpret_cast<uintptr_t>(dst) % 16 == 0) && (n % 4 == 0) &&
                        (row_stride % 4 == 0);
        publish("softmax.structure", log_mode ? "log_softmax" : "softmax",
                n <= 2048 ? "softmax_wave_per_row" : "softmax_workgroup_per_row",
                "softmax_lane_per_row", n <= 2048 ? "rows of at most 2048 fit one wave's registers"
                                                  : "long contiguous rows",
                n, rows);
        if (n <= 2048)
            return log_mode ? launch_softmax_short<true>(src, row_stride, dst, rows, n, depth, vec, st)
                            : launch_softmax_short<false>(src, row_stride, dst, rows, n, depth, vec, st);
        const RowClass rc = row_class(n);
        VKHIP_ROW_CLASSES(launch_softmax_rows, src, row_stride, dst, rows, n, log_mode, vec, st)
    }
    // General layout: one thread per row.
    publish("softmax.structure", log_mode ? "log_softmax" : "softmax", "softmax_lane_per_row",
            "softmax_workgroup_per_row", "the softmax axis is not the contiguous one", n, rows);
    vkhip_operand od;
    int64_t s = 1;
    for (int i = 3; i >= 0; --i) {
        od.ne[i] = d.ne[i];
        od.nb[i] = s;
        s *= d.ne[i];
    }
    Op4 okept, ored;
    split_axes(od, 1u << axis, okept, ored);
    const Reader rd = single_reader(d.nb[axis]);
    const Reader ord = single_reader(od.nb[axis]);
    hipLaunchKernelGGL(softmax_tall_kernel<false>, dim3(ceil_div(rows, 256)), dim3(256), 0, st, src,
                       kept, rd, okept, ord, n_out64, n, depth, log_mode, dst);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

// y[row] = sum_k A[row, k] * x[k] for a row-major A with unit inner stride and
// a contiguous x: the staged pairwise row sum of rounded products.
int launch_gemv_rows(const float* a, int64_t lda, const float* x, float* y, uint32_t m,
                     uint32_t k) {
    if (m == 0) return VKHIP_OK;
    Op4 kept;
    for (int i = 0; i < 4; ++i) {
        kept.ne[i] = 1;
        kept.nb[i] = 0;
    }
    kept.ne[3] = m;
    kept.nb[3] = lda;
    const int vec = (reinterpret_cast<uintptr_t>(a) % 16 == 0) &&
                    (reinterpret_cast<uintptr_t>(x) % 16 == 0) && (k % 4 == 0) && (lda % 4 == 0);
    const int depth = pairwise_depth(k);
    const RowClass rc = row_class(k);
    hipStream_t st = ctx().stream;
    if (vec && k > 2048 && k <= 4096 && m >= 2) {
        const uint32_t ss = stage_stride(k);
        auto* kern = k == 4096 ? rows2_sum_kernel<true, true> : rows2_sum_kernel<true, false>;
        hipLaunchKernelGGL(kern, dim3(ceil_div(m, 2u)), dim3(256),
                           2 * static_cast<size_t>(ss) * sizeof(float), st, a, lda, x, y, m, k, depth, ss, 0);
        VKHIP_LAUNCH_CHECK();
        return VKHIP_OK;
    }
    VKHIP_ROW_CLASSES(launch_sum_rows, a, kept, m, k, depth, 0, vec, y, st, x)
}

}  // namespace vkhip

extern "C" int vkhip_softmax(const float* src, const vkhip_operand* src_desc, float* dst, int axis,
                             int log_softmax) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::Unit unit("softmax");
    if (!src_desc) return vkhip::fail(VKHIP_ERR_INVALID, "softmax: null descriptor");
    return vkhip::launch_softmax(src, *src_desc, dst, axis, log_softmax);
}

extern "C" int vkhip_reduce(int op, const float* src, const vkhip_operand* src_desc,
                            uint32_t axes_mask, void* dst) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::Unit unit("reduce");
    if (!src_desc) return vkhip::fail(VKHIP_ERR_INVALID, "reduce: null descriptor");
    return vkhip::launch_reduce(op, src, *src_desc, axes_mask, dst);
}
