/*
 * vkml_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of vkML's CPU backend (the parity oracle) for the hot
 * path and the support kernels the training steps need. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only
 * as the checker or as the reported CPU baseline; the product never calls it.
 *
 * Build: -O2 -ffp-contract=off (no FMA contraction, no fast-math), so every
 * product and sum rounds to f32 exactly where the reference's does.
 *
 * Each function cites the reference source it follows. The reference is C++20
 * (templates over a strided Node); here the same loops walk rank-4 operand
 * descriptors (extents right-aligned, strides in elements), and the pairwise
 * recursion is restated over a gathered array, which performs the identical
 * sequence of f32 operations.
 *
 * Threads: functions taking `threads` parallelise over OUTPUT elements only
 * (OpenMP); every output's arithmetic is unchanged, so any thread count gives
 * bit-identical results.
 */
#include "vkhip.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define OR_PAIRWISE_BLOCK 32 /* reference kPairwiseBlock, src/backend/cpu/reduce.h:48 */

/* ------------------------------------------------------------------------ */
/* Pairwise summation: reference pairwise_sum, src/backend/cpu/reduce.h:55-72 */
/* ------------------------------------------------------------------------ */
static float pairwise(const float* v, int64_t begin, int64_t end) {
    const int64_t n = end - begin;
    if (n <= 0) return 0.0f;
    if (n <= OR_PAIRWISE_BLOCK) {
        float acc = 0.0f;
        for (int64_t i = begin; i < end; ++i) acc += v[i];
        return acc;
    }
    const int64_t mid = begin + n / 2; /* midpoint split, reduce.h:69 */
    return pairwise(v, begin, mid) + pairwise(v, mid, end);
}

float or_pairwise_sum(const float* v, int64_t n) { return pairwise(v, 0, n); }

/* ------------------------------------------------------------------------ */
/* exp and log. The reference calls std::exp / std::log on float
 * (kernels_reduce.cpp:227-243), i.e. the platform libm, whose results the
 * reference does not pin (glibc's expf/logf are within 0.502 ulp and miss the
 * correctly rounded value for ~1e-4 / ~1e-3 of inputs). The oracle fixes
 * them to named methods evaluated in IEEE double, so the device's exact
 * numerics mode can reproduce them bit for bit:
 *   exp: Cody-Waite reduction x = k ln2 + r, |r| <= ln2/2 (ln2 as two
 *        doubles, fused multiply-adds), Taylor polynomial of e^r to degree 13
 *        (Horner), times 2^k;
 *   log: x = m 2^e, m in [sqrt(1/2), sqrt(2)), s = (m-1)/(m+1),
 *        log m = 2 atanh s = 2s(1 + s^2/3 + ... + s^24/25), plus e ln2.
 * Each is the correctly rounded float except within ~2^-27 ulp of a rounding
 * midpoint (pinned against mpmath in tests/test_oracle.py).
 *
 * or_set_libm_math(1) switches both to the platform libm's expf / logf, which
 * is what the reference's std::exp / std::log on float call: the oracle then
 * runs the reference's CPU arithmetic as built against this libm. It exists
 * to measure how far two equally valid exp/log choices move a whole training
 * trajectory; parity fixtures use the named methods (the default). */
/* ------------------------------------------------------------------------ */
float or_logf(float xf);

static int or_libm_math = 0;

void or_set_libm_math(int on) { or_libm_math = on != 0; }

int or_get_libm_math(void) { return or_libm_math; }

float or_expf(float xf) {
    if (or_libm_math) return expf(xf);
    if (xf != xf) return xf + xf;
    if (xf > 89.0f) return INFINITY;
    if (xf < -104.0f) return 0.0f;
    const double x = xf;
    const double kd = rint(x * 0x1.71547652b82fep+0);
    double r = fma(-kd, 0x1.62e42fefa39efp-1, x);
    r = fma(-kd, 0x1.abc9e3b39803fp-56, r);
    static const double c[] = {0x1.6124613a86d09p-33, 0x1.1eed8eff8d898p-29, 0x1.ae64567f544e4p-26,
                               0x1.27e4fb7789f5cp-22, 0x1.71de3a556c734p-19, 0x1.a01a01a01a01ap-16,
                               0x1.a01a01a01a01ap-13, 0x1.6c16c16c16c17p-10, 0x1.1111111111111p-7,
                               0x1.5555555555555p-5,  0x1.5555555555555p-3,  0x1.0000000000000p-1,
                               1.0, 1.0};
    double p = c[0];
    for (int i = 1; i < 14; ++i) p = fma(p, r, c[i]);
    return (float)ldexp(p, (int)kd);
}

void or_exp_vec(const float* x, float* y, int64_t n, int log_mode) {
    for (int64_t i = 0; i < n; ++i) y[i] = log_mode ? or_logf(x[i]) : or_expf(x[i]);
}

float or_logf(float xf) {
    if (or_libm_math) return logf(xf);
    if (xf != xf) return xf + xf;
    if (xf < 0.0f) return NAN;
    if (xf == 0.0f) return -INFINITY;
    if (xf == INFINITY) return xf;
    int e = 0;
    double m = frexp((double)xf, &e);
    if (m < 0x1.6a09e667f3bcdp-1) {
        m = m + m;
        e -= 1;
    }
    const double f = m - 1.0;
    const double s = f / (2.0 + f);
    const double z = s * s;
    static const double c[] = {0x1.47ae147ae147bp-5, 0x1.642c8590b2164p-5, 0x1.8618618618618p-5,
                               0x1.af286bca1af28p-5, 0x1.e1e1e1e1e1e1ep-5, 0x1.1111111111111p-4,
                               0x1.3b13b13b13b14p-4, 0x1.745d1745d1746p-4, 0x1.c71c71c71c71cp-4,
                               0x1.2492492492492p-3, 0x1.999999999999ap-3, 0x1.5555555555555p-2};
    double w = c[0];
    for (int i = 1; i < 12; ++i) w = fma(w, z, c[i]);
    const double t = s + s;
    const double lm = fma(t * z, w, t);
    const double ed = (double)e;
    return (float)fma(ed, 0x1.62e42fefa39efp-1, fma(ed, 0x1.abc9e3b39803fp-56, lm));
}

/* Offset (elements) of the `linear`-th element in row-major order of a
 * rank-4 descriptor: reference linear_to_offset, src/backend/cpu/iterate.h:33-42. */
static int64_t lin_off(int64_t linear, const uint32_t ne[4], const int64_t nb[4]) {
    int64_t off = 0;
    for (int i = 3; i >= 0; --i) {
        const int64_t e = ne[i];
        off += (linear % e) * nb[i];
        linear /= e;
    }
    return off;
}

static int64_t numel4(const uint32_t ne[4]) {
    return (int64_t)ne[0] * ne[1] * ne[2] * ne[3];
}

static int nthreads(int threads) { return threads > 0 ? threads : 1; }

/* ------------------------------------------------------------------------ */
/* Matmul: reference matmul_impl<float>, src/backend/cpu/kernels_matmul.cpp:34-87
 * out[b0,b1,M,N] contiguous; per output the K products are rounded to f32
 * (widen(a)*widen(b)) and pairwise-summed. */
/* ------------------------------------------------------------------------ */
void or_matmul(const float* a, const vkhip_operand* ad, const float* b, const vkhip_operand* bd,
               float* out, int threads) {
    const int64_t b0 = ad->ne[0] > bd->ne[0] ? ad->ne[0] : bd->ne[0];
    const int64_t b1 = ad->ne[1] > bd->ne[1] ? ad->ne[1] : bd->ne[1];
    const int64_t m = ad->ne[2], k = ad->ne[3], n = bd->ne[3];
    const int64_t total = b0 * b1 * m * n;
#pragma omp parallel num_threads(nthreads(threads))
    {
        float* prod = (float*)malloc(sizeof(float) * (size_t)(k > 0 ? k : 1));
#pragma omp for schedule(static)
        for (int64_t o = 0; o < total; ++o) {
            const int64_t c = o % n, r = (o / n) % m, i1 = (o / (n * m)) % b1,
                          i0 = o / (n * m * b1);
            const float* ap = a + i0 * ad->nb[0] + i1 * ad->nb[1] + r * ad->nb[2];
            const float* bp = b + i0 * bd->nb[0] + i1 * bd->nb[1] + c * bd->nb[3];
            for (int64_t t = 0; t < k; ++t) prod[t] = ap[t * ad->nb[3]] * bp[t * bd->nb[2]];
            out[o] = pairwise(prod, 0, k);
        }
        free(prod);
    }
}

/* ------------------------------------------------------------------------ */
/* Reductions: reference reduce_generic + k_sum/k_mean/k_max/k_min/k_argmax/
 * k_argmin, src/backend/cpu/kernels_reduce.cpp:44-176, plan from
 * make_reduce_plan (reduce.cpp:11-30). `mask` bit i = axis i of the rank-4
 * descriptor. Output: kept axes, row-major; f32, or int64 for arg ops. */
/* ------------------------------------------------------------------------ */
static void split_plan(const vkhip_operand* d, uint32_t mask, uint32_t kne[4], int64_t knb[4],
                       uint32_t rne[4], int64_t rnb[4]) {
    int kc = 0, rc = 0;
    uint32_t kn[4], rn[4];
    int64_t ks[4], rs[4];
    for (int i = 0; i < 4; ++i) {
        if (mask & (1u << i)) {
            rn[rc] = d->ne[i];
            rs[rc++] = d->nb[i];
        } else {
            kn[kc] = d->ne[i];
            ks[kc++] = d->nb[i];
        }
    }
    for (int i = 0; i < 4; ++i) {
        kne[i] = 1; knb[i] = 0; rne[i] = 1; rnb[i] = 0;
    }
    for (int i = 0; i < kc; ++i) { kne[4 - kc + i] = kn[i]; knb[4 - kc + i] = ks[i]; }
    for (int i = 0; i < rc; ++i) { rne[4 - rc + i] = rn[i]; rnb[4 - rc + i] = rs[i]; }
}

void or_reduce(int op, const float* in, const vkhip_operand* d, uint32_t mask, void* out,
               int threads) {
    uint32_t kne[4], rne[4];
    int64_t knb[4], rnb[4];
    split_plan(d, mask, kne, knb, rne, rnb);
    const int64_t n_out = numel4(kne), n_red = numel4(rne);
#pragma omp parallel num_threads(nthreads(threads))
    {
        float* buf = (float*)malloc(sizeof(float) * (size_t)(n_red > 0 ? n_red : 1));
#pragma omp for schedule(static)
        for (int64_t o = 0; o < n_out; ++o) {
            const float* base = in + lin_off(o, kne, knb);
            for (int64_t i = 0; i < n_red; ++i) buf[i] = base[lin_off(i, rne, rnb)];
            switch (op) {
                case VKHIP_REDUCE_SUM: ((float*)out)[o] = pairwise(buf, 0, n_red); break;
                case VKHIP_REDUCE_MEAN:
                    ((float*)out)[o] = n_red == 0 ? NAN : pairwise(buf, 0, n_red) / (float)n_red;
                    break;
                case VKHIP_REDUCE_MAX:
                case VKHIP_REDUCE_MIN: {
                    /* sequential, NaN returned immediately (kernels_reduce.cpp:124-154) */
                    const int is_max = op == VKHIP_REDUCE_MAX;
                    float best = is_max ? -INFINITY : INFINITY;
                    for (int64_t i = 0; i < n_red; ++i) {
                        const float v = buf[i];
                        if (isnan(v)) { best = v; break; }
                        if (is_max ? (v > best) : (v < best)) best = v;
                    }
                    ((float*)out)[o] = best;
                    break;
                }
                case VKHIP_REDUCE_ARGMAX:
                case VKHIP_REDUCE_ARGMIN: {
                    /* strict comparison keeps the FIRST extremum; NaN never
                     * compares true so it is skipped (kernels_reduce.cpp:156-192) */
                    const int is_max = op == VKHIP_REDUCE_ARGMAX;
                    int64_t best_i = 0;
                    float best = is_max ? -INFINITY : INFINITY;
                    for (int64_t i = 0; i < n_red; ++i) {
                        const float v = buf[i];
                        if (is_max ? (v > best) : (v < best)) { best = v; best_i = i; }
                    }
                    ((int64_t*)out)[o] = best_i;
                    break;
                }
                default: break;
            }
        }
        free(buf);
    }
}

/* ------------------------------------------------------------------------ */
/* Softmax / log-softmax: reference softmax_impl<Log,float>,
 * src/backend/cpu/kernels_reduce.cpp:205-259. peak = running std::max
 * (NaN-ignoring, as std::max(peak, v) is); denom = pairwise sum of
 * exp(x - peak); out = exp(x-peak)/denom or (x-peak) - log(denom).
 * Output contiguous with the input's extents. */
/* ------------------------------------------------------------------------ */
void or_softmax(const float* in, const vkhip_operand* d, float* out, int axis, int log_softmax,
                int threads) {
    const uint32_t mask = 1u << axis;
    uint32_t kne[4], rne[4];
    int64_t knb[4], rnb[4];
    split_plan(d, mask, kne, knb, rne, rnb);
    /* contiguous output strides */
    vkhip_operand od;
    int64_t s = 1;
    for (int i = 3; i >= 0; --i) { od.ne[i] = d->ne[i]; od.nb[i] = s; s *= d->ne[i]; }
    uint32_t okne[4], orne[4];
    int64_t oknb[4], ornb[4];
    split_plan(&od, mask, okne, oknb, orne, ornb);
    const int64_t n_out = numel4(kne), n_axis = numel4(rne);
#pragma omp parallel num_threads(nthreads(threads))
    {
        float* ex = (float*)malloc(sizeof(float) * (size_t)(n_axis > 0 ? n_axis : 1));
#pragma omp for schedule(static)
        for (int64_t o = 0; o < n_out; ++o) {
            const float* base = in + lin_off(o, kne, knb);
            float* obase = out + lin_off(o, okne, oknb);
            float peak = -INFINITY;
            for (int64_t k = 0; k < n_axis; ++k) {
                const float v = base[lin_off(k, rne, rnb)];
                peak = (peak < v) ? v : peak; /* std::max(peak, v) */
            }
            for (int64_t k = 0; k < n_axis; ++k) ex[k] = or_expf(base[lin_off(k, rne, rnb)] - peak);
            const float denom = pairwise(ex, 0, n_axis);
            const float ld = or_logf(denom);
            for (int64_t k = 0; k < n_axis; ++k) {
                const float shifted = base[lin_off(k, rne, rnb)] - peak;
                obase[lin_off(k, orne, ornb)] = log_softmax ? shifted - ld : or_expf(shifted) / denom;
            }
        }
        free(ex);
    }
}

/* ------------------------------------------------------------------------ */
/* im2col / col2im: reference window_of, k_im2col_impl, k_col2im_impl,
 * src/backend/cpu/kernels_movement.cpp:438-542. */
/* ------------------------------------------------------------------------ */
static int64_t span_of(int64_t extent, int k, int s, int pad, int dil) {
    return (extent + 2LL * pad - ((int64_t)dil * (k - 1) + 1)) / s + 1;
}

void or_im2col(const float* src, const vkhip_operand* sd, float* dst, const vkhip_unfold* p,
               int threads) {
    const int64_t nb = sd->ne[0], ch = sd->ne[1];
    const int64_t oh_n = span_of(p->image_h, p->kernel_h, p->stride_h, p->pad_h, p->dilation_h);
    const int64_t ow_n = span_of(p->image_w, p->kernel_w, p->stride_w, p->pad_w, p->dilation_w);
    const int64_t patch = (int64_t)p->kernel_h * p->kernel_w;
    const int64_t rows = ch * patch, L = oh_n * ow_n;
#pragma omp parallel for num_threads(nthreads(threads)) schedule(static) collapse(2)
    for (int64_t n = 0; n < nb; ++n) {
        for (int64_t row = 0; row < rows; ++row) {
            const int64_t c = row / patch, ki = (row % patch) / p->kernel_w,
                          kj = (row % patch) % p->kernel_w;
            for (int64_t pos = 0; pos < L; ++pos) {
                const int64_t oh = pos / ow_n, ow = pos % ow_n;
                const int64_t h = oh * p->stride_h - p->pad_h + ki * p->dilation_h;
                const int64_t x = ow * p->stride_w - p->pad_w + kj * p->dilation_w;
                const int inside = h >= 0 && h < p->image_h && x >= 0 && x < p->image_w;
                dst[(n * rows + row) * L + pos] =
                    inside ? src[n * sd->nb[0] + c * sd->nb[1] + h * sd->nb[2] + x * sd->nb[3]]
                           : 0.0f;
            }
        }
    }
}

void or_col2im(const float* cols, float* dst, uint32_t nbatch, uint32_t channels,
               const vkhip_unfold* p, int threads) {
    const int64_t oh_n = span_of(p->image_h, p->kernel_h, p->stride_h, p->pad_h, p->dilation_h);
    const int64_t ow_n = span_of(p->image_w, p->kernel_w, p->stride_w, p->pad_w, p->dilation_w);
    const int64_t patch = (int64_t)p->kernel_h * p->kernel_w;
    const int64_t rows = (int64_t)channels * patch, L = oh_n * ow_n;
    const int64_t total = (int64_t)nbatch * channels * p->image_h * p->image_w;
#pragma omp parallel for num_threads(nthreads(threads)) schedule(static)
    for (int64_t i = 0; i < total; ++i) {
        const int64_t x = i % p->image_w, h = (i / p->image_w) % p->image_h,
                      c = (i / ((int64_t)p->image_w * p->image_h)) % channels,
                      n = i / ((int64_t)p->image_w * p->image_h * channels);
        float acc = 0.0f;
        for (int64_t ki = 0; ki < p->kernel_h; ++ki) {
            const int64_t top = h + p->pad_h - ki * p->dilation_h;
            if (top < 0 || top % p->stride_h != 0) continue;
            const int64_t oh = top / p->stride_h;
            if (oh >= oh_n) continue;
            for (int64_t kj = 0; kj < p->kernel_w; ++kj) {
                const int64_t left = x + p->pad_w - kj * p->dilation_w;
                if (left < 0 || left % p->stride_w != 0) continue;
                const int64_t ow = left / p->stride_w;
                if (ow >= ow_n) continue;
                const int64_t row = c * patch + ki * p->kernel_w + kj;
                acc += cols[(n * rows + row) * L + oh * ow_n + ow];
            }
        }
        dst[i] = acc;
    }
}

/* ------------------------------------------------------------------------ */
/* Max-pool: reference argmax_in_window, k_max_pool2d_impl,
 * k_max_pool2d_backward_impl, src/backend/cpu/kernels_movement.cpp:556-680.
 * Input and output are contiguous planes [planes, H, W] / [planes, oh, ow]. */
/* ------------------------------------------------------------------------ */
static int64_t window_argmax(const vkhip_unfold* p, int64_t oh, int64_t ow, const float* plane) {
    float best = -INFINITY;
    int64_t best_off = -1;
    for (int64_t ki = 0; ki < p->kernel_h; ++ki) {
        const int64_t h = oh * p->stride_h - p->pad_h + ki * p->dilation_h;
        if (h < 0 || h >= p->image_h) continue;
        for (int64_t kj = 0; kj < p->kernel_w; ++kj) {
            const int64_t x = ow * p->stride_w - p->pad_w + kj * p->dilation_w;
            if (x < 0 || x >= p->image_w) continue;
            const float v = plane[h * p->image_w + x];
            if (v > best) { best = v; best_off = ki * p->kernel_w + kj; }
        }
    }
    return best_off;
}

int or_max_pool2d(const float* src, float* dst, uint32_t planes, uint32_t out_h, uint32_t out_w,
                  const vkhip_unfold* p, int threads) {
    int bad = 0;
#pragma omp parallel for num_threads(nthreads(threads)) schedule(static) reduction(| : bad)
    for (int64_t pl = 0; pl < planes; ++pl) {
        const float* plane = src + pl * (int64_t)p->image_h * p->image_w;
        for (int64_t oh = 0; oh < out_h; ++oh)
            for (int64_t ow = 0; ow < out_w; ++ow) {
                const int64_t off = window_argmax(p, oh, ow, plane);
                if (off < 0) { bad = 1; continue; } /* whole window in padding: VKML_ASSERT */
                const int64_t h = oh * p->stride_h - p->pad_h + (off / p->kernel_w) * p->dilation_h;
                const int64_t x = ow * p->stride_w - p->pad_w + (off % p->kernel_w) * p->dilation_w;
                dst[(pl * out_h + oh) * out_w + ow] = plane[h * p->image_w + x];
            }
    }
    return bad ? VKHIP_ERR_INVALID : VKHIP_OK;
}

void or_max_pool2d_backward(const float* grad, const float* src, float* dst, uint32_t planes,
                            uint32_t out_h, uint32_t out_w, const vkhip_unfold* p, int threads) {
#pragma omp parallel for num_threads(nthreads(threads)) schedule(static)
    for (int64_t pl = 0; pl < planes; ++pl) {
        const float* plane = src + pl * (int64_t)p->image_h * p->image_w;
        for (int64_t h = 0; h < p->image_h; ++h)
            for (int64_t x = 0; x < p->image_w; ++x) {
                float acc = 0.0f;
                for (int64_t ki = 0; ki < p->kernel_h; ++ki) {
                    const int64_t top = h + p->pad_h - ki * p->dilation_h;
                    if (top < 0 || top % p->stride_h != 0) continue;
                    const int64_t oh = top / p->stride_h;
                    if (oh >= out_h) continue;
                    for (int64_t kj = 0; kj < p->kernel_w; ++kj) {
                        const int64_t left = x + p->pad_w - kj * p->dilation_w;
                        if (left < 0 || left % p->stride_w != 0) continue;
                        const int64_t ow = left / p->stride_w;
                        if (ow >= out_w) continue;
                        if (window_argmax(p, oh, ow, plane) == ki * p->kernel_w + kj)
                            acc += grad[(pl * out_h + oh) * out_w + ow];
                    }
                }
                dst[pl * (int64_t)p->image_h * p->image_w + h * p->image_w + x] = acc;
            }
    }
}

/* ------------------------------------------------------------------------ */
/* Split-K carry-stack fold: reference gemm_split_k_reduce.comp:48-85 (the
 * binary-counter push/drain, also restated in tests/python/test_invariants.py:90-107). */
/* ------------------------------------------------------------------------ */
void or_split_k_fold(const float* ws, float* dst, uint64_t ne, uint32_t splits) {
    for (uint64_t i = 0; i < ne; ++i) {
        float stack[32];
        uint32_t count = 0;
        for (uint32_t s = 0; s < splits; ++s) {
            float block = ws[(uint64_t)s * ne + i];
            uint32_t c = count, level = 0;
            while (c & 1u) { block += stack[level]; c >>= 1; ++level; }
            stack[level] = block;
            ++count;
        }
        float total = 0.0f;
        for (uint32_t level = 0; level < 32; ++level)
            if ((count >> level) & 1u) total += stack[level];
        dst[i] = total;
    }
}

/* ------------------------------------------------------------------------ */
/* Elementwise support ops: reference kernels_elementwise.cpp:160-300 and
 * kernels_movement.cpp:100-200 (cast, full, arange). Output contiguous;
 * sources already broadcast to the output extents by strides. */
/* ------------------------------------------------------------------------ */
static float unary_f(int op, float x) {
    switch (op) {
        case VKHIP_OP_NEG: return -x;
        case VKHIP_OP_EXP: return or_expf(x);
        case VKHIP_OP_LOG: return or_logf(x);
        case VKHIP_OP_RELU: return x <= 0.0f ? 0.0f : x; /* NaN propagates, k_relu */
        case VKHIP_OP_CONTIGUOUS: return x;
        default: return NAN;
    }
}

static float binary_f(int op, float x, float y, float alpha, float beta) {
    switch (op) {
        case VKHIP_OP_ADD: return x + y;
        case VKHIP_OP_ADD_RELU: {
            const float v = x + y;
            return v <= 0.0f ? 0.0f : v; /* k_add then k_relu */
        }
        case VKHIP_OP_SUB: return x - y;
        case VKHIP_OP_MUL: return x * y;
        case VKHIP_OP_DIV: return x / y;
        case VKHIP_OP_SCALED_ADD: { const float l = x * alpha; const float r = y * beta; return l + r; }
        case VKHIP_OP_MAXIMUM: return (isnan(x) || isnan(y)) ? NAN : (x > y ? x : y);
        case VKHIP_OP_MINIMUM: return (isnan(x) || isnan(y)) ? NAN : (x < y ? x : y);
        default: return NAN;
    }
}

static int compare_f(int op, float x, float y) {
    switch (op) {
        case VKHIP_OP_EQUAL: return x == y;
        case VKHIP_OP_LESS: return x < y;
        case VKHIP_OP_GREATER: return x > y;
        case VKHIP_OP_LESS_EQUAL: return x <= y;
        case VKHIP_OP_GREATER_EQUAL: return x >= y;
        case VKHIP_OP_NOT_EQUAL: return x != y;
        default: return 0;
    }
}

static void to_desc(const vkhip_tensor* t, vkhip_operand* d) {
    const int pad = 4 - t->ndim;
    for (int i = 0; i < 4; ++i) { d->ne[i] = 1; d->nb[i] = 0; }
    for (int i = 0; i < t->ndim; ++i) { d->ne[pad + i] = (uint32_t)t->ne[i]; d->nb[pad + i] = t->nb[i]; }
}

static int64_t tnumel(const vkhip_tensor* t) {
    int64_t n = 1;
    for (int i = 0; i < t->ndim; ++i) n *= t->ne[i];
    return n;
}

/* ------------------------------------------------------------------------ */
/* Cross-entropy rows: the reference composition (src/api/ops.cpp:417-441)
 * evaluated operation by operation, for the backend's fused
 * VKHIP_OP_CROSS_ENTROPY[_BACKWARD] nodes:
 *   ls     = log_softmax(x) per row (as or_softmax computes it)
 *   onehot = (float)label == (float)c        (Cast, Equal with arange, Cast)
 *   out    = -pairwise_c(ls * onehot)        (Mul, Sum over C, Neg)
 * and the gradient the reference autograd builds for it, given g = dL/dout:
 *   gl = (-g) * onehot                       (Neg, Sum and Mul backward)
 *   dx = gl - expf(ls) * pairwise_c(gl)      (LogSoftmax backward)
 * Rows are x + r*row_stride, C contiguous floats; labels[N] int64. */
/* ------------------------------------------------------------------------ */
void or_cross_entropy(const float* x, int64_t row_stride, const int64_t* labels, const float* g,
                      float* out, int64_t rows, int64_t c, int backward, int threads) {
#pragma omp parallel num_threads(nthreads(threads))
    {
        float* buf = (float*)malloc(sizeof(float) * (size_t)(2 * c + 1));
        float* ls = buf + c;
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            const float* row = x + r * row_stride;
            float peak = -INFINITY;
            for (int64_t k = 0; k < c; ++k) peak = (peak < row[k]) ? row[k] : peak;
            for (int64_t k = 0; k < c; ++k) buf[k] = or_expf(row[k] - peak);
            const float ld = or_logf(pairwise(buf, 0, c));
            for (int64_t k = 0; k < c; ++k) ls[k] = (row[k] - peak) - ld;
            const float label = (float)labels[r];
            if (!backward) {
                for (int64_t k = 0; k < c; ++k) buf[k] = ls[k] * (label == (float)k ? 1.0f : 0.0f);
                out[r] = -pairwise(buf, 0, c);
            } else {
                const float ng = -g[r];
                for (int64_t k = 0; k < c; ++k) buf[k] = ng * (label == (float)k ? 1.0f : 0.0f);
                const float total = pairwise(buf, 0, c);
                for (int64_t k = 0; k < c; ++k) out[r * c + k] = buf[k] - or_expf(ls[k]) * total;
            }
        }
        free(buf);
    }
}

/* ------------------------------------------------------------------------ */
/* or_compute: the CPU backend's compute(span<Node*>) loop over the same node
 * records the device backend takes (reference CpuBackend::compute,
 * src/backend/cpu/cpu_backend.cpp, which looks each op up in its kernel table,
 * kernels.h:15-24). Host pointers. Returns a vkhip_status. */
/* ------------------------------------------------------------------------ */
/* The conv2d weight gradient summed over the batch: the per-image products
 * g[n] [Cout, L] @ im2col(x[n])^T [L, ck], then the broadcast adjoint's batch
 * sum (autograd.cpp:548-553 and :84-116): the graph's value, per element the
 * pairwise sum over the N images. g: [N, Cout, L] with image stride gsn and
 * channel stride gsc (positions contiguous). */
static int weight_grad_sum(const float* x, const vkhip_operand* xd, const float* g, int64_t N, int64_t cout,
                           int64_t L, int64_t gsn, int64_t gsc, int64_t ck, const vkhip_unfold* p, float* out,
                           int threads) {
    float* cols = (float*)malloc(sizeof(float) * (size_t)(N * ck * L + 1));
    float* per = (float*)malloc(sizeof(float) * (size_t)(N * cout * ck + 1));
    if (!cols || !per) { free(cols); free(per); return VKHIP_ERR_OOM; }
    or_im2col(x, xd, cols, p, threads);
    vkhip_operand gd = {{1, (uint32_t)N, (uint32_t)cout, (uint32_t)L}, {0, gsn, gsc, 1}};
    vkhip_operand cd = {{1, (uint32_t)N, (uint32_t)L, (uint32_t)ck}, {0, ck * L, 1, L}};
    or_matmul(g, &gd, cols, &cd, per, threads);
    vkhip_operand pd = {{1, (uint32_t)N, (uint32_t)cout, (uint32_t)ck}, {0, cout * ck, ck, 1}};
    or_reduce(VKHIP_REDUCE_SUM, per, &pd, 0x2u, out, threads);
    free(cols);
    free(per);
    return VKHIP_OK;
}

int or_compute(const vkhip_node* nodes, size_t count, int threads) {
    for (size_t ni = 0; ni < count; ++ni) {
        const vkhip_node* nd = &nodes[ni];
        const vkhip_tensor* o = &nd->out;
        const int64_t n = tnumel(o);
        vkhip_operand s0, s1, s2;
        if (nd->n_src > 0) to_desc(&nd->src[0], &s0);
        if (nd->n_src > 1) to_desc(&nd->src[1], &s1);
        if (nd->n_src > 2) to_desc(&nd->src[2], &s2);
        switch (nd->op) {
            case VKHIP_OP_FULL: {
                double v;
                memcpy(&v, nd->params, sizeof v);
                if (o->dtype == VKHIP_F32) for (int64_t i = 0; i < n; ++i) ((float*)o->data)[i] = (float)v;
                else if (o->dtype == VKHIP_I64) for (int64_t i = 0; i < n; ++i) ((int64_t*)o->data)[i] = (int64_t)v;
                else if (o->dtype == VKHIP_BOOL) memset(o->data, v != 0.0 ? 1 : 0, (size_t)n);
                else return VKHIP_ERR_UNSUPPORTED;
                break;
            }
            case VKHIP_OP_ARANGE: {
                double ar[2];
                memcpy(ar, nd->params, sizeof ar);
                if (o->dtype == VKHIP_F32) for (int64_t i = 0; i < n; ++i) ((float*)o->data)[i] = (float)(ar[0] + (double)i * ar[1]);
                else if (o->dtype == VKHIP_I64) for (int64_t i = 0; i < n; ++i) ((int64_t*)o->data)[i] = (int64_t)(ar[0] + (double)i * ar[1]);
                else return VKHIP_ERR_UNSUPPORTED;
                break;
            }
            case VKHIP_OP_CAST: {
                const int from = nd->src[0].dtype, to = o->dtype;
                for (int64_t i = 0; i < n; ++i) {
                    const int64_t off = lin_off(i, s0.ne, s0.nb);
                    if (from == VKHIP_I64 && to == VKHIP_F32) ((float*)o->data)[i] = (float)((const int64_t*)nd->src[0].data)[off];
                    else if (from == VKHIP_BOOL && to == VKHIP_F32) ((float*)o->data)[i] = ((const uint8_t*)nd->src[0].data)[off] != 0 ? 1.0f : 0.0f;
                    else if (from == VKHIP_F32 && to == VKHIP_I64) ((int64_t*)o->data)[i] = (int64_t)((const float*)nd->src[0].data)[off];
                    else if (from == to && to == VKHIP_F32) ((float*)o->data)[i] = ((const float*)nd->src[0].data)[off];
                    else return VKHIP_ERR_UNSUPPORTED;
                }
                break;
            }
            case VKHIP_OP_CONTIGUOUS:
                if (o->dtype == VKHIP_I64) {
                    for (int64_t i = 0; i < n; ++i) ((int64_t*)o->data)[i] = ((const int64_t*)nd->src[0].data)[lin_off(i, s0.ne, s0.nb)];
                    break;
                }
                /* fall through: f32 copy */
            case VKHIP_OP_NEG: case VKHIP_OP_EXP: case VKHIP_OP_LOG: case VKHIP_OP_RELU: {
                if (o->dtype != VKHIP_F32) return VKHIP_ERR_UNSUPPORTED;
                const float* x = (const float*)nd->src[0].data;
                for (int64_t i = 0; i < n; ++i) ((float*)o->data)[i] = unary_f(nd->op, x[lin_off(i, s0.ne, s0.nb)]);
                break;
            }
            case VKHIP_OP_ADD: case VKHIP_OP_ADD_RELU: case VKHIP_OP_SUB: case VKHIP_OP_MUL: case VKHIP_OP_DIV:
            case VKHIP_OP_SCALED_ADD: case VKHIP_OP_MAXIMUM: case VKHIP_OP_MINIMUM: {
                float ab[2] = {1.0f, 1.0f};
                memcpy(ab, nd->params, sizeof ab);
                const float* x = (const float*)nd->src[0].data;
                const float* y = (const float*)nd->src[1].data;
                for (int64_t i = 0; i < n; ++i)
                    ((float*)o->data)[i] = binary_f(nd->op, x[lin_off(i, s0.ne, s0.nb)], y[lin_off(i, s1.ne, s1.nb)], ab[0], ab[1]);
                break;
            }
            case VKHIP_OP_EQUAL: case VKHIP_OP_LESS: case VKHIP_OP_GREATER: case VKHIP_OP_LESS_EQUAL:
            case VKHIP_OP_GREATER_EQUAL: case VKHIP_OP_NOT_EQUAL: {
                const float* x = (const float*)nd->src[0].data;
                const float* y = (const float*)nd->src[1].data;
                for (int64_t i = 0; i < n; ++i)
                    ((uint8_t*)o->data)[i] = (uint8_t)compare_f(nd->op, x[lin_off(i, s0.ne, s0.nb)], y[lin_off(i, s1.ne, s1.nb)]);
                break;
            }
            case VKHIP_OP_RELU_BACKWARD: {
                /* where(less_equal(x, zeros_like(x)), zeros_like(g), g), autograd.cpp:397-408 */
                const float* x = (const float*)nd->src[0].data;
                const float* g = (const float*)nd->src[1].data;
                for (int64_t i = 0; i < n; ++i) {
                    const float xv = x[lin_off(i, s0.ne, s0.nb)];
                    ((float*)o->data)[i] = compare_f(VKHIP_OP_LESS_EQUAL, xv, 0.0f) ? 0.0f : g[lin_off(i, s1.ne, s1.nb)];
                }
                break;
            }
            case VKHIP_OP_WHERE: {
                const uint8_t* c = (const uint8_t*)nd->src[0].data;
                const float* x = (const float*)nd->src[1].data;
                const float* y = (const float*)nd->src[2].data;
                for (int64_t i = 0; i < n; ++i)
                    ((float*)o->data)[i] = c[lin_off(i, s0.ne, s0.nb)] ? x[lin_off(i, s1.ne, s1.nb)] : y[lin_off(i, s2.ne, s2.nb)];
                break;
            }
            case VKHIP_OP_SUM: case VKHIP_OP_MEAN: case VKHIP_OP_MAX: case VKHIP_OP_MIN:
            case VKHIP_OP_ARGMAX: case VKHIP_OP_ARGMIN: {
                uint32_t mask;
                memcpy(&mask, nd->params, sizeof mask);
                const int nd0 = nd->src[0].ndim;
                if (mask == 0) mask = nd0 <= 0 ? 0u : (1u << nd0) - 1u; /* all_axes_mask */
                const uint32_t mask4 = mask << (4 - nd0);
                static const int map[] = {VKHIP_REDUCE_SUM, VKHIP_REDUCE_MEAN, VKHIP_REDUCE_MAX, VKHIP_REDUCE_MIN, -1, VKHIP_REDUCE_ARGMAX, VKHIP_REDUCE_ARGMIN};
                or_reduce(map[nd->op - VKHIP_OP_SUM], (const float*)nd->src[0].data, &s0, mask4, o->data, threads);
                break;
            }
            case VKHIP_OP_MATMUL:
                or_matmul((const float*)nd->src[0].data, &s0, (const float*)nd->src[1].data, &s1, (float*)o->data, threads);
                break;
            case VKHIP_OP_MATMUL_BIAS: {
                /* MATMUL, then the ADD of the bias broadcast over rows and the
                 * RELU (relu flag in params), element by element in f32 */
                uint32_t relu;
                memcpy(&relu, nd->params, sizeof relu);
                or_matmul((const float*)nd->src[0].data, &s0, (const float*)nd->src[1].data, &s1, (float*)o->data, threads);
                const float* bias = (const float*)nd->src[2].data;
                const int64_t ncols = o->ne[o->ndim - 1], bs = nd->src[2].nb[0];
                float* out = (float*)o->data;
                for (int64_t i = 0; i < n; ++i) {
                    float v = out[i] + bias[(i % ncols) * bs];
                    if (relu) v = unary_f(VKHIP_OP_RELU, v);
                    out[i] = v;
                }
                break;
            }
            case VKHIP_OP_MATMUL_RELU_BACKWARD: {
                /* MATMUL, then RELU_BACKWARD(x = src2 (contiguous), g = product) */
                or_matmul((const float*)nd->src[0].data, &s0, (const float*)nd->src[1].data, &s1, (float*)o->data, threads);
                const float* x = (const float*)nd->src[2].data;
                float* out = (float*)o->data;
                for (int64_t i = 0; i < n; ++i)
                    if (compare_f(VKHIP_OP_LESS_EQUAL, x[i], 0.0f)) out[i] = 0.0f;
                break;
            }
            case VKHIP_OP_SOFTMAX: case VKHIP_OP_LOG_SOFTMAX: {
                int32_t axis;
                memcpy(&axis, nd->params, sizeof axis);
                if (axis < 0) axis += nd->src[0].ndim;
                or_softmax((const float*)nd->src[0].data, &s0, (float*)o->data, axis + 4 - nd->src[0].ndim,
                           nd->op == VKHIP_OP_LOG_SOFTMAX, threads);
                break;
            }
            case VKHIP_OP_IM2COL: {
                vkhip_unfold p;
                memcpy(&p, nd->params, sizeof p);
                or_im2col((const float*)nd->src[0].data, &s0, (float*)o->data, &p, threads);
                break;
            }
            case VKHIP_OP_CONV2D:
            case VKHIP_OP_CONV2D_BIAS_RELU: {
                /* The reference's conv2d graph (ops.cpp:662-705): im2col, then
                 * flat_weight [Cout, C*kh*kw] @ cols [N, C*kh*kw, L] with the
                 * weight broadcast over the batch; for CONV2D_BIAS_RELU then
                 * the bias ADD (broadcast over N, H, W) and k_relu. */
                vkhip_unfold p;
                memcpy(&p, nd->params, sizeof p);
                const vkhip_tensor* w = &nd->src[1];
                const int64_t ck = w->ndim == 4 ? w->ne[1] * w->ne[2] * w->ne[3] : w->ne[1];
                const int64_t L = o->ne[2] * o->ne[3];
                float* cols = (float*)malloc(sizeof(float) * (size_t)(o->ne[0] * ck * L + 1));
                if (!cols) return VKHIP_ERR_OOM;
                or_im2col((const float*)nd->src[0].data, &s0, cols, &p, threads);
                vkhip_operand wd = {{1, 1, (uint32_t)w->ne[0], (uint32_t)ck},
                                    {0, 0, w->nb[0], w->ndim == 4 ? w->nb[3] : w->nb[1]}};
                vkhip_operand cd = {{1, (uint32_t)o->ne[0], (uint32_t)ck, (uint32_t)L},
                                    {0, ck * L, L, 1}};
                or_matmul((const float*)w->data, &wd, cols, &cd, (float*)o->data, threads);
                free(cols);
                if (nd->op == VKHIP_OP_CONV2D_BIAS_RELU) {
                    const float* bias = (const float*)nd->src[2].data;
                    const int64_t bs = nd->src[2].nb[0], cout = o->ne[1];
                    float* y = (float*)o->data;
                    for (int64_t i = 0; i < o->ne[0] * cout * L; ++i) {
                        const float v = y[i] + bias[((i / L) % cout) * bs];
                        y[i] = unary_f(VKHIP_OP_RELU, v);
                    }
                }
                break;
            }
            case VKHIP_OP_CONV2D_WEIGHT_GRAD: {
                /* The reference conv2d backward's weight product per image
                 * (autograd.cpp:548-553 over ops.cpp:662-705): grad [N, Cout, L]
                 * @ im2col(x)^T [N, L, C*kh*kw]; the batch sum is a separate node. */
                vkhip_unfold p;
                memcpy(&p, nd->params, sizeof p);
                const vkhip_tensor* g = &nd->src[1];
                const int64_t L = g->ne[2] * g->ne[3];
                const int64_t ck = o->ne[2];
                float* cols = (float*)malloc(sizeof(float) * (size_t)(o->ne[0] * ck * L + 1));
                if (!cols) return VKHIP_ERR_OOM;
                or_im2col((const float*)nd->src[0].data, &s0, cols, &p, threads);
                vkhip_operand gd = {{1, (uint32_t)g->ne[0], (uint32_t)g->ne[1], (uint32_t)L},
                                    {0, g->nb[0], g->nb[1], 1}};
                vkhip_operand cd = {{1, (uint32_t)o->ne[0], (uint32_t)L, (uint32_t)ck},
                                    {0, ck * L, 1, L}};
                or_matmul((const float*)g->data, &gd, cols, &cd, (float*)o->data, threads);
                free(cols);
                break;
            }
            case VKHIP_OP_CONV2D_INPUT_GRAD: {
                /* The reference conv2d backward's input gradient
                 * (autograd.cpp:548-553 over ops.cpp:662-705): the TN product
                 * flat_weight^T [C*kh*kw, Cout] @ grad[n] [Cout, L] into the
                 * column matrix, then col2im (the im2col adjoint). */
                vkhip_unfold p;
                memcpy(&p, nd->params, sizeof p);
                const vkhip_tensor* g = &nd->src[0];
                const vkhip_tensor* w = &nd->src[1];
                const int64_t N = g->ne[0], cout = g->ne[1];
                const int64_t L = g->ne[2] * g->ne[3];
                const int64_t ck = o->ne[1] * (int64_t)p.kernel_h * p.kernel_w;
                float* cols = (float*)malloc(sizeof(float) * (size_t)(N * ck * L + 1));
                if (!cols) return VKHIP_ERR_OOM;
                vkhip_operand ad = {{1, (uint32_t)N, (uint32_t)ck, (uint32_t)cout},
                                    {0, 0, 1, w->nb[0]}};
                vkhip_operand bd = {{1, (uint32_t)N, (uint32_t)cout, (uint32_t)L},
                                    {0, g->nb[0], g->nb[1], 1}};
                or_matmul((const float*)w->data, &ad, (const float*)g->data, &bd, cols, threads);
                or_col2im(cols, (float*)o->data, (uint32_t)N, (uint32_t)o->ne[1], &p, threads);
                free(cols);
                break;
            }
            case VKHIP_OP_CONV2D_WEIGHT_GRAD_SUM: {
                vkhip_unfold p;
                memcpy(&p, nd->params, sizeof p);
                const vkhip_tensor* g = &nd->src[1];
                const int st = weight_grad_sum((const float*)nd->src[0].data, &s0, (const float*)g->data, g->ne[0],
                                               g->ne[1], g->ne[2] * g->ne[3], g->nb[0], g->nb[1], o->ne[1], &p,
                                               (float*)o->data, threads);
                if (st != VKHIP_OK) return st;
                break;
            }
            case VKHIP_OP_MAX_POOL2D_BACKWARD_RELU_BIAS: {
                /* The nodes it stands for: dz = MAX_POOL2D_BACKWARD_RELU (2x2
                 * windows at stride 2), then the bias gradient, dz summed
                 * over N, H, W (the broadcast adjoint, autograd.cpp:84-116). */
                vkhip_unfold p;
                memcpy(&p, nd->params, sizeof p);
                const vkhip_tensor* y = &nd->src[1];
                const int64_t N = y->ne[0], C = y->ne[1], plane = y->ne[2] * y->ne[3];
                float* out = (float*)o->data;
                or_max_pool2d_backward((const float*)nd->src[0].data, (const float*)y->data, out, (uint32_t)(N * C),
                                       (uint32_t)nd->src[0].ne[2], (uint32_t)nd->src[0].ne[3], &p, threads);
                const float* yv = (const float*)y->data;
                for (int64_t i = 0; i < N * C * plane; ++i)
                    if (compare_f(VKHIP_OP_LESS_EQUAL, yv[i], 0.0f)) out[i] = 0.0f;
                vkhip_operand rd = {{(uint32_t)N, (uint32_t)C, (uint32_t)y->ne[2], (uint32_t)y->ne[3]},
                                    {C * plane, plane, y->ne[3], 1}};
                or_reduce(VKHIP_REDUCE_SUM, out, &rd, 0xDu, out + N * C * plane, threads);
                break;
            }
            case VKHIP_OP_CONV2D_POOL_WEIGHT_BIAS_GRAD: {
                /* The nodes it stands for, in turn: dz = the pool's adjoint
                 * over y (2x2 windows, stride 2) masked by the relu
                 * (MAX_POOL2D_BACKWARD_RELU), the batch-summed weight
                 * gradient of dz (CONV2D_WEIGHT_GRAD_SUM) and the bias
                 * gradient, dz summed over N, oh, ow (the broadcast adjoint,
                 * autograd.cpp:84-116). */
                vkhip_unfold p;
                memcpy(&p, nd->params, sizeof p);
                const vkhip_tensor* y = &nd->src[1];
                const int64_t N = y->ne[0], cout = y->ne[1], L = y->ne[2] * y->ne[3];
                const int64_t ck = nd->src[0].ne[1] * (int64_t)p.kernel_h * p.kernel_w;
                float* dz = (float*)malloc(sizeof(float) * (size_t)(N * cout * L + 1));
                if (!dz) return VKHIP_ERR_OOM;
                vkhip_unfold pp = {2, 2, 2, 2, 0, 0, 1, 1, (int32_t)y->ne[2], (int32_t)y->ne[3]};
                or_max_pool2d_backward((const float*)nd->src[2].data, (const float*)y->data, dz, (uint32_t)(N * cout),
                                       (uint32_t)nd->src[2].ne[2], (uint32_t)nd->src[2].ne[3], &pp, threads);
                const float* yv = (const float*)y->data;
                for (int64_t i = 0; i < N * cout * L; ++i)
                    if (compare_f(VKHIP_OP_LESS_EQUAL, yv[i], 0.0f)) dz[i] = 0.0f;
                float* out = (float*)o->data;
                int st = weight_grad_sum((const float*)nd->src[0].data, &s0, dz, N, cout, L, cout * L, L, ck, &p,
                                         out, threads);
                if (st == VKHIP_OK) {
                    vkhip_operand rd = {{(uint32_t)N, (uint32_t)cout, (uint32_t)y->ne[2], (uint32_t)y->ne[3]},
                                        {cout * L, L, y->ne[3], 1}};
                    or_reduce(VKHIP_REDUCE_SUM, dz, &rd, 0xDu, out + cout * ck, threads);
                }
                free(dz);
                if (st != VKHIP_OK) return st;
                break;
            }
            case VKHIP_OP_COL2IM: {
                vkhip_unfold p;
                memcpy(&p, nd->params, sizeof p);
                or_col2im((const float*)nd->src[0].data, (float*)o->data, (uint32_t)o->ne[0], (uint32_t)o->ne[1], &p, threads);
                break;
            }
            case VKHIP_OP_MAX_POOL2D: {
                vkhip_unfold p;
                memcpy(&p, nd->params, sizeof p);
                const int st = or_max_pool2d((const float*)nd->src[0].data, (float*)o->data,
                                             (uint32_t)(o->ne[0] * o->ne[1]), (uint32_t)o->ne[2], (uint32_t)o->ne[3], &p, threads);
                if (st != VKHIP_OK) return st;
                break;
            }
            case VKHIP_OP_MAX_POOL2D_BACKWARD:
            case VKHIP_OP_MAX_POOL2D_BACKWARD_RELU: {
                vkhip_unfold p;
                memcpy(&p, nd->params, sizeof p);
                or_max_pool2d_backward((const float*)nd->src[0].data, (const float*)nd->src[1].data, (float*)o->data,
                                       (uint32_t)(o->ne[0] * o->ne[1]), (uint32_t)nd->src[0].ne[2], (uint32_t)nd->src[0].ne[3], &p, threads);
                if (nd->op == VKHIP_OP_MAX_POOL2D_BACKWARD_RELU) {
                    /* the relu gradient on the pool's input, as VKHIP_OP_RELU_BACKWARD */
                    const float* x = (const float*)nd->src[1].data;
                    float* out = (float*)o->data;
                    for (int64_t i = 0; i < n; ++i)
                        if (compare_f(VKHIP_OP_LESS_EQUAL, x[i], 0.0f)) out[i] = 0.0f;
                }
                break;
            }
            case VKHIP_OP_CROSS_ENTROPY:
            case VKHIP_OP_CROSS_ENTROPY_BACKWARD: {
                const int back = nd->op == VKHIP_OP_CROSS_ENTROPY_BACKWARD;
                if (nd->src[0].ndim != 2 || nd->src[0].nb[1] != 1) return VKHIP_ERR_UNSUPPORTED;
                or_cross_entropy((const float*)nd->src[0].data, nd->src[0].nb[0],
                                 (const int64_t*)nd->src[1].data,
                                 back ? (const float*)nd->src[2].data : NULL, (float*)o->data,
                                 nd->src[0].ne[0], nd->src[0].ne[1], back, threads);
                break;
            }
            default: return VKHIP_ERR_UNSUPPORTED;
        }
    }
    return VKHIP_OK;
}
