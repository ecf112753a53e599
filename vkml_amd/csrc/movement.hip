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

#include <algorithm>

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
//
// A workgroup covers kRowsPerBlock consecutive (image, row) pairs and 1024
// consecutive positions; each thread decodes its four positions once and writes
// them for every row, as one 16-byte store per row when L allows it. NT selects
// non-temporal stores: the cols tensor is written once here and read once by
// the GEMM that follows.
constexpr int kIm2colRows = 4;

template <bool NT>
__global__ __launch_bounds__(256) void im2col_kernel(const float* __restrict__ src, Op4 sd,
                                                     float* __restrict__ dst, Geo g, uint32_t rows,
                                                     uint32_t nrows, uint32_t L,
                                                     uint32_t pos_blocks, int vec, FastDiv div_w) {
    const uint32_t rb = blockIdx.x / pos_blocks;
    const uint32_t pb = blockIdx.x % pos_blocks;
    const uint32_t pos0 = (pb * 256 + threadIdx.x) * 4;
    if (pos0 >= L) return;
    int32_t hb[4], xb[4];
    bool in[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t pos = pos0 + j;
        in[j] = pos < L;
        const int32_t oh = in[j] ? static_cast<int32_t>(div_w.div(pos)) : 0;
        const int32_t ow = in[j] ? static_cast<int32_t>(pos) - oh * g.out_w : 0;
        hb[j] = oh * g.sh - g.ph;
        xb[j] = ow * g.sw - g.pw;
    }
    const uint32_t patch = g.kh * g.kw;
#pragma unroll
    for (int r = 0; r < kIm2colRows; ++r) {
        const uint32_t nr = rb * kIm2colRows + r;  // n*rows + row, uniform
        if (nr >= nrows) break;
        const uint32_t n = nr / rows, row = nr % rows;
        const uint32_t c = row / patch, rem = row % patch;
        const int32_t dhk = (rem / g.kw) * g.dh, dwk = (rem % g.kw) * g.dw;
        const float* plane = src + n * sd.nb[0] + c * sd.nb[1];
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int32_t h = hb[j] + dhk, x = xb[j] + dwk;
            v[j] = (in[j] && h >= 0 && h < g.H && x >= 0 && x < g.W) ? plane[h * sd.nb[2] + x * sd.nb[3]]
                                                                    : 0.0f;
        }
        float* out = dst + static_cast<uint64_t>(nr) * L + pos0;
        if (vec && pos0 + 3 < L) {
            if (NT)
                __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(out));
            else
                *reinterpret_cast<f32x4*>(out) = v;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (in[j]) out[j] = v[j];
        }
    }
}

// The plane-staged im2col: one workgroup per (image plane, block of R output
// rows). The input rows the block's windows touch are loaded once into LDS,
// zero-padded, so each image element is read from memory once; then each
// thread takes four consecutive positions and writes them for every window
// offset (kh*kw cols rows), gathering from LDS. Measured on conv2
// ([128,64,32,32] -> [128,576,1024]): 52 us (6.4 TB/s) against 79 us for the
// per-row gather above, whose image re-reads through the caches (each element
// nine times) held the writes back.
constexpr uint32_t kIm2colTileBytes = 32768;

template <bool NT>
__global__ __launch_bounds__(256) void im2col_plane_kernel(const float* __restrict__ src, Op4 sd,
                                                           float* __restrict__ dst, Geo g,
                                                           uint32_t channels, uint32_t L,
                                                           uint32_t rows_per_block, uint32_t rblocks,
                                                           uint32_t in_rows, uint32_t pitch, int vec,
                                                           FastDiv div_ow, FastDiv div_rb,
                                                           FastDiv div_c, FastDiv div_pitch) {
    extern __shared__ float tile[];
    // Contiguous block ranges per XCD, so the blocks of one image stay in one L2.
    uint32_t bid = blockIdx.x;
    if ((gridDim.x & 7u) == 0) bid = (bid & 7u) * (gridDim.x >> 3) + (bid >> 3);
    const uint32_t plane = div_rb.div(bid);  // n*C + c
    const uint32_t rb = bid - plane * rblocks;
    const uint32_t n = div_c.div(plane), c = plane - n * channels;
    const int32_t oh0 = static_cast<int32_t>(rb * rows_per_block);
    const int32_t h_first = oh0 * g.sh - g.ph;
    const float* img = src + n * sd.nb[0] + c * sd.nb[1];
    const uint32_t tile_n = in_rows * pitch;
    for (uint32_t i = threadIdx.x; i < tile_n; i += 256) {
        const uint32_t r = div_pitch.div(i), x = i - r * pitch;
        const int32_t h = h_first + static_cast<int32_t>(r), w = static_cast<int32_t>(x) - g.pw;
        const bool ok = static_cast<uint32_t>(h) < static_cast<uint32_t>(g.H) &&
                        static_cast<uint32_t>(w) < static_cast<uint32_t>(g.W);
        const float t = img[ok ? h * sd.nb[2] + w * sd.nb[3] : 0];
        tile[i] = ok ? t : 0.0f;
    }
    __syncthreads();
    const uint32_t rows_here = min(rows_per_block, static_cast<uint32_t>(g.out_h - oh0));
    const uint32_t npos = rows_here * static_cast<uint32_t>(g.out_w);
    const uint32_t kk = static_cast<uint32_t>(g.kh * g.kw);
    float* out0 = dst + static_cast<uint64_t>(plane) * kk * L + static_cast<uint64_t>(oh0) * g.out_w;
    for (uint32_t p0 = threadIdx.x * 4; p0 < npos; p0 += 1024) {
        uint32_t at[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t p = min(p0 + j, npos - 1);
            const uint32_t oh = div_ow.div(p), ow = p - oh * static_cast<uint32_t>(g.out_w);
            at[j] = oh * g.sh * pitch + ow * g.sw;
        }
        for (uint32_t r = 0, ki = 0, kj = 0; r < kk; ++r) {
            const uint32_t d = ki * g.dh * pitch + kj * g.dw;
            f32x4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = tile[at[j] + d];
            float* out = out0 + static_cast<uint64_t>(r) * L + p0;
            if (vec && p0 + 3 < npos) {
                if (NT)
                    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(out));
                else
                    *reinterpret_cast<f32x4*>(out) = v;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (p0 + j < npos) out[j] = v[j];
            }
            if (++kj == static_cast<uint32_t>(g.kw)) {
                kj = 0;
                ++ki;
            }
        }
    }
}

// Non-temporal stores for im2col's output (measured 3.8 vs 2.9 TB/s on conv2):
// the cols tensor is streamed out once and read once by the GEMM after it.
// VKHIP_NT_STORES=0 turns them off.
static int nt_stores() {
    static const int v = [] {
        const char* e = getenv("VKHIP_NT_STORES");
        return e && e[0] == '0' ? 0 : 1;
    }();
    return v;
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
    if (nrows > 0xffffffffull) return fail(VKHIP_ERR_UNSUPPORTED, "im2col: too many rows");
    // Plane-staged when a block of output rows fits the LDS tile: R output
    // rows need (R-1)*stride_h + (kh-1)*dil_h + 1 input rows of W + 2*pad_w.
    {
        const uint64_t pitch = static_cast<uint64_t>(g.W) + 2ull * g.pw;
        const uint64_t halo = static_cast<uint64_t>(g.kh - 1) * g.dh + 1;
        const uint64_t max_in_rows = kIm2colTileBytes / 4 / std::max<uint64_t>(pitch, 1);
        uint64_t R = max_in_rows >= halo ? (max_in_rows - halo) / g.sh + 1 : 0;
        R = std::min<uint64_t>(R, static_cast<uint64_t>(g.out_h));
        // whole blocks of four positions keep the 16-byte stores aligned
        while (R > 1 && (R * g.out_w) % 4 != 0 && R < static_cast<uint64_t>(g.out_h)) --R;
        const uint64_t planes = static_cast<uint64_t>(nb) * ch;
        if (R >= 1 && pitch * ((R - 1) * g.sh + halo) * 4 <= kIm2colTileBytes &&
            planes * ceil_div(static_cast<uint64_t>(g.out_h), R) <= 0x7fffffffull) {
            const uint32_t rblocks = static_cast<uint32_t>(ceil_div(static_cast<uint64_t>(g.out_h), R));
            const uint32_t in_rows = static_cast<uint32_t>((R - 1) * g.sh + halo);
            const int vec_plane = (L % 4 == 0) && ((R * g.out_w) % 4 == 0 || rblocks == 1) &&
                                  (reinterpret_cast<uintptr_t>(dst) % 16 == 0);
            const uint32_t blocks = static_cast<uint32_t>(planes * rblocks);
            const size_t lds = static_cast<size_t>(in_rows) * pitch * 4;
            auto kern = nt_stores() ? im2col_plane_kernel<true> : im2col_plane_kernel<false>;
            hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), lds, ctx().stream, src, to_op4(sd), dst, g,
                               ch, L, static_cast<uint32_t>(R), rblocks, in_rows,
                               static_cast<uint32_t>(pitch), vec_plane,
                               FastDiv(static_cast<uint32_t>(g.out_w)), FastDiv(rblocks), FastDiv(ch),
                               FastDiv(static_cast<uint32_t>(pitch)));
            VKHIP_LAUNCH_CHECK();
            publish("im2col.kernel", "im2col", "plane_staged", "row_gather",
                    "the input rows of a block fit the LDS tile", static_cast<int64_t>(lds),
                    kIm2colTileBytes);
            return VKHIP_OK;
        }
    }
    const uint32_t pos_blocks = ceil_div(L, 1024);
    const uint64_t blocks = static_cast<uint64_t>(ceil_div(nrows, kIm2colRows)) * pos_blocks;
    if (blocks > 0x7fffffffu) return fail(VKHIP_ERR_UNSUPPORTED, "im2col: grid too large");
    const int vec = (L % 4 == 0) && (reinterpret_cast<uintptr_t>(dst) % 16 == 0);
    if (nt_stores())
        hipLaunchKernelGGL(im2col_kernel<true>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                           ctx().stream, src, to_op4(sd), dst, g, rows,
                           static_cast<uint32_t>(nrows), L, pos_blocks, vec,
                           FastDiv(static_cast<uint32_t>(g.out_w)));
    else
        hipLaunchKernelGGL(im2col_kernel<false>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                           ctx().stream, src, to_op4(sd), dst, g, rows,
                           static_cast<uint32_t>(nrows), L, pos_blocks, vec,
                           FastDiv(static_cast<uint32_t>(g.out_w)));
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

// ---- col2im ---------------------------------------------------------------------
// image[n,c,h,x] = sum over (ki,kj) ascending of cols[...]   (kernels_movement.cpp:500-542)
// Each thread owns four consecutive x of one image row.
template <bool NT>
__global__ __launch_bounds__(256) void col2im_kernel(const float* __restrict__ cols,
                                                     float* __restrict__ dst, Geo g,
                                                     uint32_t channels, uint64_t total_q,
                                                     uint32_t xq_n, int vec) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= total_q) return;
    const uint32_t xq = static_cast<uint32_t>(i % xq_n);
    const uint64_t t2 = i / xq_n;
    const int32_t h = static_cast<int32_t>(t2 % static_cast<uint32_t>(g.H));
    const uint64_t plane = t2 / static_cast<uint32_t>(g.H);  // n*C + c
    const uint32_t c = static_cast<uint32_t>(plane % channels);
    const uint64_t n = plane / channels;
    const uint32_t patch = g.kh * g.kw;
    const uint64_t L = static_cast<uint64_t>(g.out_h) * g.out_w;
    const float* cbase = cols + (n * channels * patch + static_cast<uint64_t>(c) * patch) * L;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int32_t ki = 0; ki < g.kh; ++ki) {
        const int32_t top = h + g.ph - ki * g.dh;
        if (top < 0 || top % g.sh != 0) continue;
        const int32_t oh = top / g.sh;
        if (oh >= g.out_h) continue;
        const float* crow = cbase + static_cast<uint64_t>(ki * g.kw) * L + static_cast<uint64_t>(oh) * g.out_w;
        for (int32_t kj = 0; kj < g.kw; ++kj) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int32_t x = 4 * xq + j;
                const int32_t left = x + g.pw - kj * g.dw;
                if (x >= g.W || left < 0 || left % g.sw != 0) continue;
                const int32_t ow = left / g.sw;
                if (ow >= g.out_w) continue;
                acc[j] = acc[j] + crow[static_cast<uint64_t>(kj) * L + ow];
            }
        }
    }
    float* out = dst + (plane * g.H + h) * g.W + 4 * xq;
    if (vec) {
        if (NT)
            __builtin_nontemporal_store(acc, reinterpret_cast<f32x4*>(out));
        else
            *reinterpret_cast<f32x4*>(out) = acc;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (4 * xq + j < static_cast<uint32_t>(g.W)) out[j] = acc[j];
    }
}

// Staged variant: one workgroup per (image, channel) plane. That plane's kh*kw
// cols rows are one contiguous run of kh*kw*L floats, staged once in LDS with
// 16-byte loads; each thread then pulls four consecutive output pixels from LDS
// in the same ascending (ki, kj) order. Every cols byte is read from HBM
// exactly once, fully coalesced.
template <bool UNIT>
__global__ __launch_bounds__(256) void col2im_staged_kernel(const float* __restrict__ cols,
                                                            float* __restrict__ dst, Geo g,
                                                            uint32_t plane_floats, int vec_in,
                                                            int vec_out, FastDiv div_w) {
    extern __shared__ __attribute__((aligned(16))) float stage[];
    const uint64_t plane = blockIdx.x;
    const float* src = cols + plane * plane_floats;
    // Every load of the plane is issued before the first LDS write (the plane
    // is at most 64 KB: sixteen 16-byte loads per thread).
    if (vec_in) {
        const f32x4* s4 = reinterpret_cast<const f32x4*>(src);
        f32x4* d4 = reinterpret_cast<f32x4*>(stage);
        const uint32_t nv = plane_floats / 4;
        f32x4 v[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t i = threadIdx.x + 256u * r;
            if (i < nv) v[r] = __builtin_nontemporal_load(s4 + i);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t i = threadIdx.x + 256u * r;
            if (i < nv) d4[i] = v[r];
        }
    } else {
        for (uint32_t i0 = 0; i0 < plane_floats; i0 += 256u * 16) {
            float v[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t i = i0 + threadIdx.x + 256u * r;
                if (i < plane_floats) v[r] = src[i];
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t i = i0 + threadIdx.x + 256u * r;
                if (i < plane_floats) stage[i] = v[r];
            }
        }
    }
    __syncthreads();
    const int32_t L = g.out_h * g.out_w;
    const uint32_t hw = static_cast<uint32_t>(g.H) * g.W;
    float* out = dst + plane * hw;
    for (uint32_t q = threadIdx.x; 4 * q < hw; q += 256) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        const uint32_t pix0 = 4 * q;
        int32_t h = static_cast<int32_t>(div_w.div(pix0));
        int32_t x = static_cast<int32_t>(pix0) - h * g.W;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (pix0 + j < hw) {
                float a = 0.0f;
                for (int32_t ki = 0; ki < g.kh; ++ki) {
                    int32_t oh;
                    if (UNIT) {
                        oh = h + g.ph - ki;
                        if (oh < 0 || oh >= g.out_h) continue;
                    } else {
                        const int32_t top = h + g.ph - ki * g.dh;
                        if (top < 0 || top % g.sh != 0) continue;
                        oh = top / g.sh;
                        if (oh >= g.out_h) continue;
                    }
                    for (int32_t kj = 0; kj < g.kw; ++kj) {
                        int32_t ow;
                        if (UNIT) {
                            ow = x + g.pw - kj;
                            if (ow < 0 || ow >= g.out_w) continue;
                        } else {
                            const int32_t left = x + g.pw - kj * g.dw;
                            if (left < 0 || left % g.sw != 0) continue;
                            ow = left / g.sw;
                            if (ow >= g.out_w) continue;
                        }
                        a = a + stage[(ki * g.kw + kj) * L + oh * g.out_w + ow];
                    }
                }
                acc[j] = a;
            }
            if (++x == g.W) {
                x = 0;
                ++h;
            }
        }
        if (vec_out && pix0 + 3 < hw) {
            *reinterpret_cast<f32x4*>(out + pix0) = acc;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (pix0 + j < hw) out[pix0 + j] = acc[j];
        }
    }
}

// col2im of a 3x3 window, stride 1, padding 1, dilation 1, out = H x W with
// W a multiple of four and Q = W / 4 dividing 64 (the config geometries).
// Thread (plane, h, q) owns output pixels w = 4q .. 4q + 3 of row h. The
// columns it needs from window row ki all lie in output row oh = h + 1 - ki,
// at ow = w + 1 - kj: for each of the nine cols rows it loads the aligned
// float4 at [oh][4q .. 4q + 3] (every cols element is loaded by exactly one
// thread, 16-byte loads coalesced along the row), and the two values just
// outside it (kj = 0 needs [4q + 4], kj = 2 needs [4q - 1]) come from the
// neighbouring lanes of the same row (0 at the image border). No LDS, so
// occupancy is not held to four planes per CU as in the staged kernel.
// Each pixel adds its nine terms in ascending (ki, kj) from +0.0, an absent
// term as +0.0: the sum is never -0.0, so adding +0.0 changes nothing and the
// result is the pull's bits (kernels_movement.cpp:500-542).
__global__ __launch_bounds__(256) void col2im_3x3_kernel(const float* __restrict__ cols,
                                                         float* __restrict__ dst, uint32_t H,
                                                         uint32_t W, uint64_t total, FastDiv div_q,
                                                         FastDiv div_h) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    const bool live = i < total;
    const uint32_t Q = W >> 2;
    const uint64_t ii = live ? i : 0;
    // i = (plane * H + h) * Q + q; total < 2^32 (checked by the launcher)
    const uint32_t row = div_q.div(static_cast<uint32_t>(ii));
    const uint32_t q = static_cast<uint32_t>(ii) - row * Q;
    const uint32_t plane = div_h.div(row);
    const uint32_t h = row - plane * H;
    const uint64_t L = static_cast<uint64_t>(H) * W;
    const float* cb = cols + static_cast<uint64_t>(plane) * 9u * L + 4u * q;
    f32x4 v[9];
#pragma unroll
    for (int ki = 0; ki < 3; ++ki) {
        const int32_t oh = static_cast<int32_t>(h) + 1 - ki;
        const bool ok = live && oh >= 0 && oh < static_cast<int32_t>(H);
        const uint64_t off = ok ? static_cast<uint64_t>(oh) * W : 0u;
#pragma unroll
        for (int kj = 0; kj < 3; ++kj) {
            const f32x4 t = __builtin_nontemporal_load(
                reinterpret_cast<const f32x4*>(cb + static_cast<uint64_t>(ki * 3 + kj) * L + off));
            const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
            v[ki * 3 + kj] = ok ? t : z;
        }
    }
    float nxt[3], prv[3];  // [4q + 4] of window (ki, 0); [4q - 1] of window (ki, 2)
#pragma unroll
    for (int ki = 0; ki < 3; ++ki) {
        const float a = __shfl_down(v[ki * 3][0], 1);
        const float b = __shfl_up(v[ki * 3 + 2][3], 1);
        nxt[ki] = q + 1 < Q ? a : 0.0f;
        prv[ki] = q > 0 ? b : 0.0f;
    }
    f32x4 acc;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float s = 0.0f;
#pragma unroll
        for (int ki = 0; ki < 3; ++ki) {
            s = s + (j < 3 ? v[ki * 3][j + 1] : nxt[ki]);  // kj = 0: ow = w + 1
            s = s + v[ki * 3 + 1][j];                       // kj = 1: ow = w
            s = s + (j > 0 ? v[ki * 3 + 2][j - 1] : prv[ki]);  // kj = 2: ow = w - 1
        }
        acc[j] = s;
    }
    if (live)
        __builtin_nontemporal_store(acc, reinterpret_cast<f32x4*>(dst + static_cast<uint64_t>(row) * W + 4u * q));
}

int launch_col2im(const float* cols, float* dst, uint32_t n, uint32_t channels,
                  const vkhip_unfold& p) {
    Geo g;
    int st = make_geo(p, g);
    if (st != VKHIP_OK) return st;
    const uint64_t planes = static_cast<uint64_t>(n) * channels;
    if (planes == 0 || g.H == 0 || g.W == 0) return VKHIP_OK;
    const uint64_t L = static_cast<uint64_t>(g.out_h) * g.out_w;
    const uint64_t plane_floats = L * g.kh * g.kw;
    // 3x3, stride 1, padding 1 (same-size output), rows of whole float4s
    // whose lanes stay inside one wave: the register kernel above.
    const uint64_t q_total = planes * static_cast<uint64_t>(g.H) * (g.W / 4);
    if (g.kh == 3 && g.kw == 3 && g.sh == 1 && g.sw == 1 && g.dh == 1 && g.dw == 1 && g.ph == 1 &&
        g.pw == 1 && g.out_h == g.H && g.out_w == g.W && g.W % 4 == 0 && 64 % (g.W / 4) == 0 &&
        reinterpret_cast<uintptr_t>(cols) % 16 == 0 && reinterpret_cast<uintptr_t>(dst) % 16 == 0 &&
        planes * 9 * L < (1ull << 40) && q_total + 255 < (1ull << 32)) {
        publish("col2im.kernel", "col2im", "col2im_3x3", "col2im_staged",
                "3x3 window, stride 1, padding 1, rows of whole float4s",
                static_cast<int64_t>(g.W), 4);
        hipLaunchKernelGGL(col2im_3x3_kernel, dim3(static_cast<uint32_t>((q_total + 255) / 256)),
                           dim3(256), 0, ctx().stream, cols, dst, static_cast<uint32_t>(g.H),
                           static_cast<uint32_t>(g.W), q_total,
                           FastDiv(static_cast<uint32_t>(g.W / 4)), FastDiv(static_cast<uint32_t>(g.H)));
        VKHIP_LAUNCH_CHECK();
        return VKHIP_OK;
    }
    const bool staged = plane_floats * sizeof(float) <= 65536 && planes <= 0x7fffffffull;
    publish("col2im.kernel", "col2im", staged ? "col2im_staged" : "col2im_direct",
            staged ? "col2im_direct" : "col2im_staged",
            staged ? "an image plane's columns fit in 64 KB of LDS" : "a plane's columns exceed 64 KB",
            static_cast<int64_t>(plane_floats * sizeof(float)), 65536);
    if (staged) {
        const int vec_in = (plane_floats % 4 == 0) && (reinterpret_cast<uintptr_t>(cols) % 16 == 0);
        const int vec_out = (static_cast<uint64_t>(g.H) * g.W % 4 == 0) &&
                            (reinterpret_cast<uintptr_t>(dst) % 16 == 0);
        const bool unit = g.sh == 1 && g.sw == 1 && g.dh == 1 && g.dw == 1;
        const FastDiv dw(static_cast<uint32_t>(g.W));
        if (unit)
            hipLaunchKernelGGL(col2im_staged_kernel<true>, dim3(static_cast<uint32_t>(planes)),
                               dim3(256), plane_floats * sizeof(float), ctx().stream, cols, dst, g,
                               static_cast<uint32_t>(plane_floats), vec_in, vec_out, dw);
        else
            hipLaunchKernelGGL(col2im_staged_kernel<false>, dim3(static_cast<uint32_t>(planes)),
                               dim3(256), plane_floats * sizeof(float), ctx().stream, cols, dst, g,
                               static_cast<uint32_t>(plane_floats), vec_in, vec_out, dw);
        VKHIP_LAUNCH_CHECK();
        return VKHIP_OK;
    }
    const uint32_t xq_n = ceil_div(g.W, 4);
    const uint64_t total_q = planes * g.H * xq_n;
    const uint64_t blocks = (total_q + 255) / 256;
    if (blocks > 0x7fffffffu) return fail(VKHIP_ERR_UNSUPPORTED, "col2im: grid too large");
    const int vec = (g.W % 4 == 0) && (reinterpret_cast<uintptr_t>(dst) % 16 == 0);
    if (nt_stores())
        hipLaunchKernelGGL(col2im_kernel<true>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                           ctx().stream, cols, dst, g, channels, total_q, xq_n, vec);
    else
        hipLaunchKernelGGL(col2im_kernel<false>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                           ctx().stream, cols, dst, g, channels, total_q, xq_n, vec);
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
// (kernels_movement.cpp:620-680). RELU: then the gradient of the relu that
// produced src, src <= 0 ? +0 : that value (a NaN src passes it through).
template <bool RELU>
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
    if (RELU && pl[h * sd.nb[2] + x * sd.nb[3]] <= 0.0f) acc = 0.0f;
    dst[static_cast<uint64_t>(plane) * hw + idx] = acc;
}

// ---- 2x2 windows tiling the plane exactly (stride 2, no padding or dilation) ----
// Each thread owns two horizontally adjacent windows: two 16-byte loads (rows
// 2*oh and 2*oh + 1, columns 4j..4j+3) cover both. Output row r of the flat
// [planes*out_h, out_w] output reads input rows 2r and 2r + 1 of the flat
// [planes*H, W] input. The window scan is window_argmax's: strict '>' from
// -inf in the order (0,0), (0,1), (1,0), (1,1) (argmax4, common.h); no winner
// (all -inf or NaN) gives -1, and the forward then takes the first position, as
// the general kernel does.

__device__ __forceinline__ float pick4(int32_t off, float a, float b, float c, float d) {
    return off == 1 ? b : off == 2 ? c : off == 3 ? d : a;
}

__global__ __launch_bounds__(256) void max_pool2x2_kernel(const float* __restrict__ src,
                                                         float* __restrict__ dst, uint32_t W,
                                                         FastDiv pairs_per_row, uint32_t total) {
    const uint32_t q = blockIdx.x * 256 + threadIdx.x;
    if (q >= total) return;
    const uint32_t r = pairs_per_row.div(q);
    const uint32_t j = q - r * pairs_per_row.d;
    const float* r0 = src + static_cast<uint64_t>(2 * r) * W + 4 * j;
    const f32x4_t t = *reinterpret_cast<const f32x4_t*>(r0);
    const f32x4_t u = *reinterpret_cast<const f32x4_t*>(r0 + W);
    float2 o;
    o.x = pick4(argmax4(t[0], t[1], u[0], u[1]), t[0], t[1], u[0], u[1]);
    o.y = pick4(argmax4(t[2], t[3], u[2], u[3]), t[2], t[3], u[2], u[3]);
    reinterpret_cast<float2*>(dst)[q] = o;
}

// Backward of the same tiling: every input position lies in exactly one
// window, so the pull of the general kernel reduces to 0 + g at the window's
// first maximum and +0 elsewhere (0 + g also turns a -0 gradient into +0, as
// the pull's accumulator does). RELU: masked by src <= 0 as above, from the
// src values already loaded for the window scan.
template <bool RELU>
__global__ __launch_bounds__(256) void max_pool2x2_backward_kernel(
    const float* __restrict__ grad, const float* __restrict__ src, float* __restrict__ dst,
    uint32_t W, FastDiv pairs_per_row, uint32_t total) {
    const uint32_t q = blockIdx.x * 256 + threadIdx.x;
    if (q >= total) return;
    const uint32_t r = pairs_per_row.div(q);
    const uint32_t j = q - r * pairs_per_row.d;
    const uint64_t base = static_cast<uint64_t>(2 * r) * W + 4 * j;
    const f32x4_t t = *reinterpret_cast<const f32x4_t*>(src + base);
    const f32x4_t u = *reinterpret_cast<const f32x4_t*>(src + base + W);
    const float2 g = reinterpret_cast<const float2*>(grad)[q];
    const int32_t a0 = argmax4(t[0], t[1], u[0], u[1]);
    const int32_t a1 = argmax4(t[2], t[3], u[2], u[3]);
    const float g0 = 0.0f + g.x, g1 = 0.0f + g.y;
    f32x4_t top, bot;
    top[0] = a0 == 0 ? g0 : 0.0f;
    top[1] = a0 == 1 ? g0 : 0.0f;
    bot[0] = a0 == 2 ? g0 : 0.0f;
    bot[1] = a0 == 3 ? g0 : 0.0f;
    top[2] = a1 == 0 ? g1 : 0.0f;
    top[3] = a1 == 1 ? g1 : 0.0f;
    bot[2] = a1 == 2 ? g1 : 0.0f;
    bot[3] = a1 == 3 ? g1 : 0.0f;
    if (RELU) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (t[i] <= 0.0f) top[i] = 0.0f;
            if (u[i] <= 0.0f) bot[i] = 0.0f;
        }
    }
    // the image gradient streams past the L2 (non-temporal): the next
    // kernels read it, this one never does
    __builtin_nontemporal_store(top, reinterpret_cast<f32x4_t*>(dst + base));
    __builtin_nontemporal_store(bot, reinterpret_cast<f32x4_t*>(dst + base + W));
}

// The 2x2 fast path applies to contiguous planes whose width is a multiple of
// 4, 16-byte aligned, pooled by 2x2 windows at stride 2 with no padding or
// dilation over an even height.
static bool pool2x2_tiles(const Geo& g, const vkhip_operand& sd, const void* a, const void* b,
                          const void* c) {
    const bool geo = g.kh == 2 && g.kw == 2 && g.sh == 2 && g.sw == 2 && g.ph == 0 && g.pw == 0 &&
                     g.dh == 1 && g.dw == 1 && g.H % 2 == 0 && g.W % 4 == 0;
    const bool contiguous = sd.nb[3] == 1 && sd.nb[2] == g.W &&
                            sd.nb[1] == static_cast<int64_t>(g.H) * g.W &&
                            (sd.ne[0] == 1 || sd.nb[0] == static_cast<int64_t>(sd.ne[1]) * g.H * g.W);
    const auto al = [](const void* p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    return geo && contiguous && al(a) && al(b) && al(c);
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
    if (static_cast<int64_t>(sd.ne[2]) != p.image_h || static_cast<int64_t>(sd.ne[3]) != p.image_w)
        return fail(VKHIP_ERR_INVALID, "max_pool2d: input is %ux%u but the geometry says %dx%d",
                    sd.ne[2], sd.ne[3], p.image_h, p.image_w);
    if (static_cast<uint32_t>(g.out_h) != out_h || static_cast<uint32_t>(g.out_w) != out_w)
        return fail(VKHIP_ERR_INVALID, "max_pool2d: output %ux%u disagrees with geometry %dx%d",
                    out_h, out_w, g.out_h, g.out_w);
    if (!windows_reach_image(g))
        return fail(VKHIP_ERR_INVALID, "max_pool2d: a window lies entirely in the padding");
    const uint64_t planes = static_cast<uint64_t>(sd.ne[0]) * sd.ne[1];
    const uint32_t ohw = out_h * out_w;
    if (planes == 0 || ohw == 0) return VKHIP_OK;
    const bool tiled = pool2x2_tiles(g, sd, src, dst, nullptr);
    publish("max_pool2d.kernel", "max_pool2d", tiled ? "max_pool2x2_tiled" : "max_pool2d_general",
            tiled ? "max_pool2d_general" : "max_pool2x2_tiled",
            tiled ? "2x2 windows at stride 2 tile the plane" : "windows overlap, pad or dilate",
            g.kh * g.kw, g.sh * g.sw);
    if (tiled) {
        const uint64_t total = planes * ohw / 2;
        if (total <= 0xffffffffull) {
            hipLaunchKernelGGL(max_pool2x2_kernel, dim3(ceil_div(static_cast<uint32_t>(total), 256)),
                               dim3(256), 0, ctx().stream, src, dst, static_cast<uint32_t>(g.W),
                               FastDiv(out_w / 2), static_cast<uint32_t>(total));
            VKHIP_LAUNCH_CHECK();
            return VKHIP_OK;
        }
    }
    const uint32_t bpp = ceil_div(ohw, 256);
    hipLaunchKernelGGL(max_pool2d_kernel, dim3(static_cast<uint32_t>(planes * bpp)), dim3(256), 0,
                       ctx().stream, src, to_op4(sd), dst, g, sd.ne[1], bpp);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

int launch_max_pool2d_backward(const float* grad, const float* src, const vkhip_operand& sd,
                               float* dst, uint32_t out_h, uint32_t out_w, const vkhip_unfold& p,
                               bool relu) {
    Geo g;
    int st = make_geo(p, g);
    if (st != VKHIP_OK) return st;
    if (static_cast<int64_t>(sd.ne[2]) != p.image_h || static_cast<int64_t>(sd.ne[3]) != p.image_w)
        return fail(VKHIP_ERR_INVALID, "max_pool2d: input is %ux%u but the geometry says %dx%d",
                    sd.ne[2], sd.ne[3], p.image_h, p.image_w);
    if (static_cast<uint32_t>(g.out_h) != out_h || static_cast<uint32_t>(g.out_w) != out_w)
        return fail(VKHIP_ERR_INVALID, "max_pool2d_backward: grad %ux%u disagrees with geometry %dx%d",
                    out_h, out_w, g.out_h, g.out_w);
    const uint64_t planes = static_cast<uint64_t>(sd.ne[0]) * sd.ne[1];
    const uint32_t hw = static_cast<uint32_t>(g.H) * g.W;
    if (planes == 0 || hw == 0) return VKHIP_OK;
    const bool tiled = pool2x2_tiles(g, sd, src, dst, grad);
    publish("max_pool2d.kernel", "max_pool2d_backward",
            tiled ? "max_pool2x2_tiled" : "max_pool2d_general",
            tiled ? "max_pool2d_general" : "max_pool2x2_tiled",
            tiled ? "2x2 windows at stride 2 tile the plane" : "windows overlap, pad or dilate",
            g.kh * g.kw, g.sh * g.sw);
    if (tiled) {
        const uint64_t total = planes * out_h * out_w / 2;
        if (total <= 0xffffffffull) {
            hipLaunchKernelGGL(relu ? max_pool2x2_backward_kernel<true> : max_pool2x2_backward_kernel<false>,
                               dim3(ceil_div(static_cast<uint32_t>(total), 256)), dim3(256), 0,
                               ctx().stream, grad, src, dst, static_cast<uint32_t>(g.W),
                               FastDiv(out_w / 2), static_cast<uint32_t>(total));
            VKHIP_LAUNCH_CHECK();
            return VKHIP_OK;
        }
    }
    const uint32_t bpp = ceil_div(hw, 256);
    hipLaunchKernelGGL(relu ? max_pool2d_backward_kernel<true> : max_pool2d_backward_kernel<false>,
                       dim3(static_cast<uint32_t>(planes * bpp)), dim3(256), 0, ctx().stream, grad,
                       src, to_op4(sd), dst, g, sd.ne[1], bpp);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

// ---- the relu-masked pool gradient with each plane's sum (a conv layer's bias
// gradient) ----------------------------------------------------------------------
// MAX_POOL2D_BACKWARD_RELU's values for 2x2 windows at stride 2 over planes of
// rows W = 16 or 32, H = 2P rows, plus for every plane the sum of those values
// in the pairwise tree's order. A workgroup takes RP = 1024 / W consecutive row
// pairs; W / 4 lanes share one (each the 4 positions 4j..4j+3 of both rows: two
// windows, the tiled kernel's selects, 16-byte loads and stores on consecutive
// addresses), and put its values in LDS. Thread t < RP then sums row pair t in
// position order from +0 (one 32-position leaf for W = 16, two for W = 32),
// and the P row pairs of a plane, adjacent lanes, add their sums level by level
// (xor butterflies: a balanced tree, every lane ends with the same value). With
// the planes' positions a power of two the plane is an aligned subtree of the
// reduction over N, H, W; plane_sums_fold_kernel then adds each channel's
// planes as a balanced tree over the images.
template <int W, int P>
__global__ __launch_bounds__(256) void max_pool2x2_backward_relu_sums_kernel(
    const float* __restrict__ grad, const float* __restrict__ src, float* __restrict__ dst,
    float* __restrict__ psum) {
    static_assert((W == 16 || W == 32) && P >= 1 && P <= 32 && (P & (P - 1)) == 0, "row pairs per plane");
    constexpr int L4 = W / 4;           // lanes per row pair
    constexpr int RP = 256 / L4;        // row pairs per workgroup
    constexpr int PITCH = 2 * W + 4;    // LDS floats per row pair (16-byte rows, spread banks)
    static_assert(P <= RP, "a plane's row pairs in one workgroup");
    __shared__ __attribute__((aligned(16))) float vals[RP * PITCH];
    const int t = threadIdx.x, rp = t / L4, j = t % L4;
    const uint64_t q = static_cast<uint64_t>(blockIdx.x) * RP + rp;  // global row pair
    const uint64_t base = q * (2 * W) + 4 * j;
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(src + base);
    const f32x4_t b = *reinterpret_cast<const f32x4_t*>(src + base + W);
    const float2 g = *reinterpret_cast<const float2*>(grad + q * (W / 2) + 2 * j);
    const int32_t a0 = argmax4(a[0], a[1], b[0], b[1]);
    const int32_t a1 = argmax4(a[2], a[3], b[2], b[3]);
    const float g0 = 0.0f + g.x, g1 = 0.0f + g.y;
    f32x4_t top, bot;
    top[0] = a0 == 0 ? g0 : 0.0f;
    top[1] = a0 == 1 ? g0 : 0.0f;
    bot[0] = a0 == 2 ? g0 : 0.0f;
    bot[1] = a0 == 3 ? g0 : 0.0f;
    top[2] = a1 == 0 ? g1 : 0.0f;
    top[3] = a1 == 1 ? g1 : 0.0f;
    bot[2] = a1 == 2 ? g1 : 0.0f;
    bot[3] = a1 == 3 ? g1 : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (a[i] <= 0.0f) top[i] = 0.0f;
        if (b[i] <= 0.0f) bot[i] = 0.0f;
    }
    __builtin_nontemporal_store(top, reinterpret_cast<f32x4_t*>(dst + base));
    __builtin_nontemporal_store(bot, reinterpret_cast<f32x4_t*>(dst + base + W));
    *reinterpret_cast<f32x4_t*>(vals + rp * PITCH + 4 * j) = top;
    *reinterpret_cast<f32x4_t*>(vals + rp * PITCH + W + 4 * j) = bot;
    __syncthreads();
    if (t >= 64) return;  // wave 0 sums (RP <= 64 row pairs), whole waves leave
    float sum = 0.0f;
    if (t < RP) {
        const float* r = vals + t * PITCH;
        float leaf0 = 0.0f, leaf1 = 0.0f;
#pragma unroll
        for (int i = 0; i < W / 4; ++i) {
            const f32x4_t v = *reinterpret_cast<const f32x4_t*>(r + 4 * i);
#pragma unroll
            for (int k = 0; k < 4; ++k) leaf0 = leaf0 + v[k];
        }
        float& second = W == 16 ? leaf0 : leaf1;
#pragma unroll
        for (int i = 0; i < W / 4; ++i) {
            const f32x4_t v = *reinterpret_cast<const f32x4_t*>(r + W + 4 * i);
#pragma unroll
            for (int k = 0; k < 4; ++k) second = second + v[k];
        }
        sum = W == 16 ? leaf0 : leaf0 + leaf1;
    }
    if constexpr (P >= 2) sum = sum + wave_partner<1>(sum);
    if constexpr (P >= 4) sum = sum + wave_partner<2>(sum);
    if constexpr (P >= 8) sum = sum + wave_partner<4>(sum);
    if constexpr (P >= 16) sum = sum + wave_partner<8>(sum);
    if constexpr (P >= 32) sum = sum + wave_partner<16>(sum);
    if (t < RP && t % P == 0) psum[(static_cast<uint64_t>(blockIdx.x) * RP + t) / P] = sum;
}

// Per channel c, the balanced pairwise tree over the images of the plane sums
// psum[n * C + c] (N a power of two): 16 channels per workgroup, R = min(16, N)
// runs of N / R consecutive images each (a binary-counter carry stack, which
// for a power-of-two count is the balanced tree), then the runs level by level.
__global__ __launch_bounds__(256) void plane_sums_fold_kernel(const float* __restrict__ psum, uint32_t n,
                                                              uint32_t channels, float* __restrict__ out) {
    __shared__ float runs[16][17];
    const int tid = threadIdx.x, cl = tid & 15, run = tid >> 4;
    const uint32_t c = blockIdx.x * 16u + static_cast<uint32_t>(cl);
    const uint32_t nr = n < 16u ? n : 16u, per = n / nr;
    float r = 0.0f;
    if (static_cast<uint32_t>(run) < nr && c < channels) {
        float stack[13];
#pragma unroll
        for (int l = 0; l < 13; ++l) stack[l] = 0.0f;
        for (uint32_t i0 = 0; i0 < per; i0 += 8) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                v[k] = i0 + k < per ? psum[static_cast<uint64_t>(run * per + i0 + k) * channels + c] : 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (i0 + k >= per) break;
                const uint32_t count = i0 + k;
                float b = v[k];
                bool carry = true;
#pragma unroll
                for (int l = 0; l < 13; ++l) {
                    if (carry) {
                        if ((count >> l) & 1u) {
                            b = stack[l] + b;
                        } else {
                            stack[l] = b;
                            carry = false;
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int l = 0; l < 13; ++l)
            if (per == (1u << l)) r = stack[l];
    }
    runs[run][cl] = r;
    __syncthreads();
    if (tid < 16 && c < channels) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = runs[i][tid];
#pragma unroll
        for (int w = 1; w < 16; w *= 2)
#pragma unroll
            for (int i = 0; i + w < 16; i += 2 * w)
                if (static_cast<uint32_t>(i + w) < nr) v[i] = v[i] + v[i + w];
        out[c] = v[0];
    }
}

int launch_reduce(int op, const float* src, const vkhip_operand& d, uint32_t mask, void* dst);

// MAX_POOL2D_BACKWARD_RELU of 2x2 windows at stride 2 into dst [N,C,H,W], and
// dst's sum over N, H, W into bias_out [C] (the pairwise tree's bits): the
// kernel above and the fold where they apply (rows of 16 or 32, 2 to 64 rows,
// N*H*W a power of two, contiguous 16-byte aligned operands), else the pool
// backward and the reduction in turn.
int launch_max_pool2x2_backward_relu_sums(const float* grad, const float* src, const vkhip_operand& sd,
                                          float* dst, float* bias_out) {
    const uint32_t N = sd.ne[0], C = sd.ne[1], H = sd.ne[2], Wd = sd.ne[3];
    const uint64_t hw = static_cast<uint64_t>(H) * Wd, total = static_cast<uint64_t>(N) * hw;
    const bool contiguous = sd.nb[3] == 1 && sd.nb[2] == static_cast<int64_t>(Wd) &&
                            sd.nb[1] == static_cast<int64_t>(hw) && (N == 1 || sd.nb[0] == static_cast<int64_t>(C * hw));
    const auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    const uint32_t P = H / 2;
    const uint64_t pairs = static_cast<uint64_t>(N) * C * P;
    const bool fits = (Wd == 16 || Wd == 32) && H % 2 == 0 && P >= 1 && P <= 32 && (P & (P - 1)) == 0 &&
                      (total & (total - 1)) == 0 && (N & (N - 1)) == 0 && contiguous && al(grad) && al(src) &&
                      al(dst) && pairs % 64 == 0 && pairs <= 0xffffffffull && C > 0;
    publish("max_pool2d.kernel", "max_pool2d_backward_relu_sums", fits ? "pool2x2_relu_plane_sums" : "pool_backward_then_sum",
            fits ? "pool_backward_then_sum" : "pool2x2_relu_plane_sums",
            fits ? "rows of 16 or 32 and power-of-two extents: the sums in the pool kernel"
                 : "the plane sums need rows of 16 or 32 and power-of-two extents",
            static_cast<int64_t>(Wd), static_cast<int64_t>(H));
    if (fits) {
        float* psum = nullptr;
        const int st = workspace(static_cast<size_t>(N) * C * sizeof(float), &psum);
        if (st != VKHIP_OK) return st;
        const uint32_t per_wg = 1024u / Wd;  // row pairs per workgroup (pairs is a multiple of 64)
        const dim3 grid(static_cast<uint32_t>(pairs / per_wg));
#define VKHIP_PRS(WW, PP) \
    hipLaunchKernelGGL((max_pool2x2_backward_relu_sums_kernel<WW, PP>), grid, dim3(256), 0, ctx().stream, grad, src, dst, \
                       psum)
#define VKHIP_PRS_P(WW)                                                                                        \
    do {                                                                                                      \
        switch (P) {                                                                                          \
            case 1: VKHIP_PRS(WW, 1); break;                                                                  \
            case 2: VKHIP_PRS(WW, 2); break;                                                                  \
            case 4: VKHIP_PRS(WW, 4); break;                                                                  \
            case 8: VKHIP_PRS(WW, 8); break;                                                                  \
            case 16: VKHIP_PRS(WW, 16); break;                                                                \
            default: VKHIP_PRS(WW, 32); break;                                                                \
        }                                                                                                     \
    } while (0)
        if (Wd == 16) VKHIP_PRS_P(16); else VKHIP_PRS_P(32);
#undef VKHIP_PRS_P
#undef VKHIP_PRS
        VKHIP_LAUNCH_CHECK();
        hipLaunchKernelGGL(plane_sums_fold_kernel, dim3(ceil_div(C, 16u)), dim3(256), 0, ctx().stream, psum, N, C,
                           bias_out);
        VKHIP_LAUNCH_CHECK();
        return VKHIP_OK;
    }
    vkhip_unfold pp{};
    pp.kernel_h = pp.kernel_w = 2;
    pp.stride_h = pp.stride_w = 2;
    pp.dilation_h = pp.dilation_w = 1;
    pp.image_h = static_cast<int32_t>(H);
    pp.image_w = static_cast<int32_t>(Wd);
    int st = launch_max_pool2d_backward(grad, src, sd, dst, H / 2, Wd / 2, pp, true);
    if (st != VKHIP_OK) return st;
    vkhip_operand dd;
    dd.ne[0] = N;
    dd.ne[1] = C;
    dd.ne[2] = H;
    dd.ne[3] = Wd;
    dd.nb[0] = static_cast<int64_t>(C * hw);
    dd.nb[1] = static_cast<int64_t>(hw);
    dd.nb[2] = Wd;
    dd.nb[3] = 1;
    return launch_reduce(VKHIP_REDUCE_SUM, dst, dd, 0xDu, bias_out);
}


}  // namespace vkhip

extern "C" int vkhip_im2col(const float* src, const vkhip_operand* src_desc, float* dst,
                            const vkhip_unfold* p) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::Unit unit("im2col");
    if (!src_desc || !p) return vkhip::fail(VKHIP_ERR_INVALID, "im2col: null argument");
    return vkhip::launch_im2col(src, *src_desc, dst, *p);
}

extern "C" int vkhip_col2im(const float* cols, float* dst, uint32_t n, uint32_t channels,
                            const vkhip_unfold* p) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::Unit unit("col2im");
    if (!p) return vkhip::fail(VKHIP_ERR_INVALID, "col2im: null params");
    return vkhip::launch_col2im(cols, dst, n, channels, *p);
}
