// Convolution lowering and pooling: im2col, col2im, max-pool forward/backward.
//
// All four are bandwidth kernels whose results must equal the CPU oracle bit
// for bit (reference kernels_movement.cpp:438-680): im2col and max-pool forward
// are pure gathers; col2im and max-pool backward PULL, one thread per image
// element, adding contributions in ascending (ki, kj) order from 0.0f exactly
// as the oracle does, so no accumulation order depends on scheduling.
//
// Launch shape: the (image, row) or (image, plane) index that is uniform across
// a workgroup is decoded once from blockIdx; only the position within the row
// is per-thread, so the per-element integer work is one divide by out_w (or W).
#include "common.h"

namespace vkhip {

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct Geo {
    int32_t kh, kw, sh, sw, ph, pw, dh, dw, H, W;
    int32_t out_h, out_w;
};

static int64_t span_of(int64_t extent, int k, int s, int pad, int dil) {
    return (extent + 2LL * pad - (static_cast<int64_t>(dil) * (k - 1) + 1)) / s + 1;
}

static int make_geo(const vkhip_unfold& p, Geo& g) {
    if (p.kernel_h <= 0 || p.kernel_w <= 0 || p.stride_h <= 0 || p.stride_w <= 0 ||
        p.dilation_h <= 0 || p.dilation_w <= 0 || p.pad_h < 0 || p.pad_w < 0 || p.image_h < 0 ||
        p.image_w < 0)
        return fail(VKHIP_ERR_INVALID, "unfold: invalid window geometry");
    g.kh = p.kernel_h;
    g.kw = p.kernel_w;
    g.sh = p.stride_h;
    g.sw = p.stride_w;
    g.ph = p.pad_h;
    g.pw = p.pad_w;
    g.dh = p.dilation_h;
    g.dw = p.dilation_w;
    g.H = p.image_h;
    g.W = p.image_w;
    const int64_t oh = span_of(p.image_h, p.kernel_h, p.stride_h, p.pad_h, p.dilation_h);
    const int64_t ow = span_of(p.image_w, p.kernel_w, p.stride_w, p.pad_w, p.dilation_w);
    if (oh <= 0 || ow <= 0) return fail(VKHIP_ERR_INVALID, "unfold: window larger than padded image");
    g.out_h = static_cast<int32_t>(oh);
    g.out_w = static_cast<int32_t>(ow);
    return VKHIP_OK;
}

// ---- im2col -------------------------------------------------------------------
// dst[(n*rows + row)*L + pos] = inside ? src[n, c, h, x] : 0   (kernels_movement.cpp:454-483)
__global__ __launch_bounds__(256) void im2col_kernel(const float* __restrict__ src, Op4 sd,
                                                     float* __restrict__ dst, Geo g, uint32_t rows,
                                                     uint32_t L, uint32_t pos_blocks, int vec) {
    const uint32_t nr = blockIdx.x / pos_blocks;  // n*rows + row, uniform
    const uint32_t pb = blockIdx.x % pos_blocks;
    const uint32_t n = nr / rows, row = nr % rows;
    const uint32_t patch = g.kh * g.kw;
    const uint32_t c = row / patch, rem = row % patch;
    const int32_t ki = rem / g.kw, kj = rem % g.kw;
    const float* plane = src + n * sd.nb[0] + c * sd.nb[1];
    const uint32_t pos0 = (pb * 256 + threadIdx.x) * 4;
    if (pos0 >= L) return;
    f32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t pos = pos0 + j;
        float val = 0.0f;
        if (pos < L) {
            const int32_t oh = pos / g.out_w;
            const int32_t ow = pos - oh * g.out_w;
            const int32_t h = oh * g.sh - g.ph + ki * g.dh;
            const int32_t x = ow * g.sw - g.pw + kj * g.dw;
            if (h >= 0 && h < g.H && x >= 0 && x < g.W) val = plane[h * sd.nb[2] + x * sd.nb[3]];
        }
        v[j] = val;
    }
    float* out = dst + static_cast<uint64_t>(nr) * L + pos0;
    if (vec && pos0 + 3 < L) {
        *reinterpret_cast<f32x4*>(out) = v;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (pos0 + j < L) out[j] = v[j];
    }
}

int launch_im2col(const float* src, const vkhip_operand& sd, float* dst, const vkhip_unfold& p) {
    Geo g;
    int st = make_geo(p, g);
    if (st != VKHIP_OK) return st;
    if (static_cast<int64_t>(sd.ne[2]) != p.image_h || static_cast<int64_t>(sd.ne[3]) != p.image_w)
        return fail(VKHIP_ERR_INVALID, "im2col: image extent %ux%u disagrees with params %dx%d",
                    sd.ne[2], sd.ne[3], p.image_h, p.image_w);
    const uint32_t nb = sd.ne[0], ch = sd.ne[1];
    const uint32_t rows = ch * g.kh * g.kw;
    const uint32_t L = static_cast<uint32_t>(g.out_h) * g.out_w;
    const uint64_t nrows = static_cast<uint64_t>(nb) * rows;
    if (nrows == 0 || L == 0) return VKHIP_OK;
    const uint32_t pos_blocks = ceil_div(L, 1024);
    const uint64_t blocks = nrows * pos_blocks;
    if (blocks > 0x7fffffffu) return fail(VKHIP_ERR_UNSUPPORTED, "im2col: grid too large");
    const int vec = (L % 4 == 0) && (reinterpret_cast<uintptr_t>(dst) % 16 == 0);
    hipLaunchKernelGGL(im2col_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                       ctx().stream, src, to_op4(sd), dst, g, rows, L, pos_blocks, vec);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

// ---- col2im ---------------------------------------------------------------------
// image[n,c,h,x] = sum over (ki,kj) ascending of cols[...]   (kernels_movement.cpp:500-542)
__global__ __launch_bounds__(256) void col2im_kernel(const float* __restrict__ cols,
                                                     float* __restrict__ dst, Geo g,
                                                     uint32_t channels, uint32_t hw_blocks) {
    const uint32_t plane = blockIdx.x / hw_blocks;  // n*C + c, uniform
    const uint32_t hb = blockIdx.x % hw_blocks;
    const uint32_t c = plane % channels, n = plane / channels;
    const uint32_t idx = hb * 256 + threadIdx.x;
    const uint32_t hw = static_cast<uint32_t>(g.H) * g.W;
    if (idx >= hw) return;
    const int32_t h = idx / g.W;
    const int32_t x = idx - h * g.W;
    const uint32_t patch = g.kh * g.kw;
    const uint64_t L = static_cast<uint64_t>(g.out_h) * g.out_w;
    const float* cbase = cols + (static_cast<uint64_t>(n) * channels * patch + c * patch) * L;
    float acc = 0.0f;
    for (int32_t ki = 0; ki < g.kh; ++ki) {
        const int32_t top = h + g.ph - ki * g.dh;
        if (top < 0 || top % g.sh != 0) continue;
        const int32_t oh = top / g.sh;
        if (oh >= g.out_h) continue;
        for (int32_t kj = 0; kj < g.kw; ++kj) {
            const int32_t left = x + g.pw - kj * g.dw;
            if (left < 0 || left % g.sw != 0) continue;
            const int32_t ow = left / g.sw;
            if (ow >= g.out_w) continue;
            acc = acc + cbase[(ki * g.kw + kj) * L + oh * g.out_w + ow];
        }
    }
    dst[static_cast<uint64_t>(plane) * hw + idx] = acc;
}

int launch_col2im(const float* cols, float* dst, uint32_t n, uint32_t channels,
                  const vkhip_unfold& p) {
    Geo g;
    int st = make_geo(p, g);
    if (st != VKHIP_OK) return st;
    const uint64_t planes = static_cast<uint64_t>(n) * channels;
    const uint32_t hw = static_cast<uint32_t>(g.H) * g.W;
    if (planes == 0 || hw == 0) return VKHIP_OK;
    const uint32_t hw_blocks = ceil_div(hw, 256);
    const uint64_t blocks = planes * hw_blocks;
    if (blocks > 0x7fffffffu) return fail(VKHIP_ERR_UNSUPPORTED, "col2im: grid too large");
    hipLaunchKernelGGL(col2im_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                       ctx().stream, cols, dst, g, channels, hw_blocks);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

// ---- max-pool -------------------------------------------------------------------
// First maximum in row-major window order with -inf padding
// (reference argmax_in_window, kernels_movement.cpp:556-585).
__device__ __forceinline__ int32_t window_argmax(const Geo& g, int32_t oh, int32_t ow,
                                                 const float* plane, int64_t sh_, int64_t sw_) {
    float best = -__builtin_inff();
    int32_t best_off = -1;
    for (int32_t ki = 0; ki < g.kh; ++ki) {
        const int32_t h = oh * g.sh - g.ph + ki * g.dh;
        if (h < 0 || h >= g.H) continue;
        for (int32_t kj = 0; kj < g.kw; ++kj) {
            const int32_t x = ow * g.sw - g.pw + kj * g.dw;
            if (x < 0 || x >= g.W) continue;
            const float v = plane[h * sh_ + x * sw_];
            if (v > best) {
                best = v;
                best_off = ki * g.kw + kj;
            }
        }
    }
    return best_off;
}

// src: [N, C, H, W] with strides sd; dst contiguous [N, C, out_h, out_w].
__global__ __launch_bounds__(256) void max_pool2d_kernel(const float* __restrict__ src, Op4 sd,
                                                         float* __restrict__ dst, Geo g,
                                                         uint32_t channels, uint32_t blocks_per_plane) {
    const uint32_t plane = blockIdx.x / blocks_per_plane;
    const uint32_t idx = (blockIdx.x % blocks_per_plane) * 256 + threadIdx.x;
    const uint32_t ohw = static_cast<uint32_t>(g.out_h) * g.out_w;
    if (idx >= ohw) return;
    const int32_t oh = idx / g.out_w, ow = idx - (idx / g.out_w) * g.out_w;
    const uint32_t c = plane % channels, n = plane / channels;
    const float* pl = src + n * sd.nb[0] + c * sd.nb[1];
    const int32_t off = window_argmax(g, oh, ow, pl, sd.nb[2], sd.nb[3]);
    // The host has checked that every window reaches the image; a window of
    // NaNs still has no maximum, and then the first in-image position is used.
    int32_t ki = 0, kj = 0;
    if (off >= 0) {
        ki = off / g.kw;
        kj = off % g.kw;
    } else {
        while (oh * g.sh - g.ph + ki * g.dh < 0) ++ki;
        while (ow * g.sw - g.pw + kj * g.dw < 0) ++kj;
    }
    const int32_t h = oh * g.sh - g.ph + ki * g.dh;
    const int32_t x = ow * g.sw - g.pw + kj * g.dw;
    dst[static_cast<uint64_t>(plane) * ohw + idx] = pl[h * sd.nb[2] + x * sd.nb[3]];
}

// grad: contiguous [N, C, out_h, out_w]; src: [N, C, H, W] with strides sd;
// dst contiguous [N, C, H, W]. Pull: each input position adds, in ascending
// window order, the gradient of every window whose first maximum it is
// (kernels_movement.cpp:620-680).
__global__ __launch_bounds__(256) void max_pool2d_backward_kernel(
    const float* __restrict__ grad, const float* __restrict__ src, Op4 sd, float* __restrict__ dst,
    Geo g, uint32_t channels, uint32_t blocks_per_plane) {
    const uint32_t plane = blockIdx.x / blocks_per_plane;
    const uint32_t idx = (blockIdx.x % blocks_per_plane) * 256 + threadIdx.x;
    const uint32_t hw = static_cast<uint32_t>(g.H) * g.W;
    if (idx >= hw) return;
    const int32_t h = idx / g.W, x = idx - (idx / g.W) * g.W;
    const uint32_t c = plane % channels, n = plane / channels;
    const float* pl = src + n * sd.nb[0] + c * sd.nb[1];
    const float* gp = grad + static_cast<uint64_t>(plane) * g.out_h * g.out_w;
    float acc = 0.0f;
    for (int32_t ki = 0; ki < g.kh; ++ki) {
        const int32_t top = h + g.ph - ki * g.dh;
        if (top < 0 || top % g.sh != 0) continue;
        const int32_t oh = top / g.sh;
        if (oh >= g.out_h) continue;
        for (int32_t kj = 0; kj < g.kw; ++kj) {
            const int32_t left = x + g.pw - kj * g.dw;
            if (left < 0 || left % g.sw != 0) continue;
            const int32_t ow = left / g.sw;
            if (ow >= g.out_w) continue;
            if (window_argmax(g, oh, ow, pl, sd.nb[2], sd.nb[3]) == ki * g.kw + kj)
                acc = acc + gp[oh * g.out_w + ow];
        }
    }
    dst[static_cast<uint64_t>(plane) * hw + idx] = acc;
}

// True when every pooling window has at least one position inside the image
// (the oracle asserts this per window, kernels_movement.cpp:604-605).
static bool windows_reach_image(const Geo& g) {
    for (int32_t oh = 0; oh < g.out_h; ++oh) {
        bool hit = false;
        for (int32_t ki = 0; ki < g.kh && !hit; ++ki) {
            const int32_t h = oh * g.sh - g.ph + ki * g.dh;
            hit = h >= 0 && h < g.H;
        }
        if (!hit) return false;
    }
    for (int32_t ow = 0; ow < g.out_w; ++ow) {
        bool hit = false;
        for (int32_t kj = 0; kj < g.kw && !hit; ++kj) {
            const int32_t x = ow * g.sw - g.pw + kj * g.dw;
            hit = x >= 0 && x < g.W;
        }
        if (!hit) return false;
    }
    return true;
}

int launch_max_pool2d(const float* src, const vkhip_operand& sd, float* dst, uint32_t out_h,
                      uint32_t out_w, const vkhip_unfold& p) {
    Geo g;
    int st = make_geo(p, g);
    if (st != VKHIP_OK) return st;
    if (static_cast<uint32_t>(g.out_h) != out_h || static_cast<uint32_t>(g.out_w) != out_w)
        return fail(VKHIP_ERR_INVALID, "max_pool2d: output %ux%u disagrees with geometry %dx%d",
                    out_h, out_w, g.out_h, g.out_w);
    if (!windows_reach_image(g))
        return fail(VKHIP_ERR_INVALID, "max_pool2d: a window lies entirely in the padding");
    const uint64_t planes = static_cast<uint64_t>(sd.ne[0]) * sd.ne[1];
    const uint32_t ohw = out_h * out_w;
    if (planes == 0 || ohw == 0) return VKHIP_OK;
    const uint32_t bpp = ceil_div(ohw, 256);
    hipLaunchKernelGGL(max_pool2d_kernel, dim3(static_cast<uint32_t>(planes * bpp)), dim3(256), 0,
                       ctx().stream, src, to_op4(sd), dst, g, sd.ne[1], bpp);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

int launch_max_pool2d_backward(const float* grad, const float* src, const vkhip_operand& sd,
                               float* dst, uint32_t out_h, uint32_t out_w, const vkhip_unfold& p) {
    Geo g;
    int st = make_geo(p, g);
    if (st != VKHIP_OK) return st;
    if (static_cast<uint32_t>(g.out_h) != out_h || static_cast<uint32_t>(g.out_w) != out_w)
        return fail(VKHIP_ERR_INVALID, "max_pool2d_backward: grad %ux%u disagrees with geometry %dx%d",
                    out_h, out_w, g.out_h, g.out_w);
    const uint64_t planes = static_cast<uint64_t>(sd.ne[0]) * sd.ne[1];
    const uint32_t hw = static_cast<uint32_t>(g.H) * g.W;
    if (planes == 0 || hw == 0) return VKHIP_OK;
    const uint32_t bpp = ceil_div(hw, 256);
    hipLaunchKernelGGL(max_pool2d_backward_kernel, dim3(static_cast<uint32_t>(planes * bpp)),
                       dim3(256), 0, ctx().stream, grad, src, to_op4(sd), dst, g, sd.ne[1], bpp);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

}  // namespace vkhip

extern "C" int vkhip_im2col(const float* src, const vkhip_operand* src_desc, float* dst,
                            const vkhip_unfold* p) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (!src_desc || !p) return vkhip::fail(VKHIP_ERR_INVALID, "im2col: null argument");
    return vkhip::launch_im2col(src, *src_desc, dst, *p);
}

extern "C" int vkhip_col2im(const float* cols, float* dst, uint32_t n, uint32_t channels,
                            const vkhip_unfold* p) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (!p) return vkhip::fail(VKHIP_ERR_INVALID, "col2im: null params");
    return vkhip::launch_col2im(cols, dst, n, channels, *p);
}
