// Small-window convolutions on gfx950 (CDNA4): layers whose window holds at
// most 32 elements (C*kh*kw <= 32) and whose output has at most 64 channels.
// CIFAR's first layer, [128,3,32,32] -> 64 channels with a 3x3 window (27
// elements), is the case in configs 4 and 5 (reference: conv2d,
// src/api/ops.cpp:662-705, im2col then flat_weight @ cols).
//
// Such a layer is one K-tile of a product: 27 of the 32 k of one MFMA chain.
// Its cost is HBM traffic (the forward writes a 33.5 MB output from a 1.6 MB
// image) and the issue slots around the matrix core, not the matrix core
// itself, so these kernels are laid out for few VALU instructions per output.
//
// Forward (win_fwd_kernel). A workgroup of four waves takes 4*BPW consecutive
// 32-position blocks of one image. It stages the input rows those blocks read,
// zero-bordered by the padding, in LDS, followed by a zero region as long as
// one channel's rows: window elements past K read there, so the gather needs
// neither a bounds check nor a select. Each wave computes every output
// channel (at most 64) of its blocks, with the weights in registers for the
// whole launch. Step t pairs window elements t and 16 + t (lanes 0-31 and
// 32-63), the pairing and order of the GEMM kernels' K-tiles, and the
// accumulator starts at zero: every output is the implicit-im2col GEMM's
// value bit for bit, then the epilogue's bias add and ReLU, one rounding each,
// as the graph's ADD and RELU nodes. The accumulator layout puts 32
// consecutive positions of one channel in the 32 lanes of a half-wave, so
// each store instruction writes two whole 128-byte rows; the stores are
// non-temporal buffer stores whose row offset is a scalar operand. (Measured
// at CIFAR conv1: 9.7 us, against 29 us for the transposed layout whose lanes
// each store four positions as one 16-byte non-temporal store -- 64 partial
// lines per instruction -- and 13.2 us for the same with ordinary stores.)
#include "conv_small.h"

#include <algorithm>

namespace vkhip {
namespace {

typedef float v2f __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kWinWaves = 4;            // waves per workgroup
constexpr int kWinThreads = 64 * kWinWaves;
constexpr int kWinLdsFloats = 16384;    // dynamic LDS per workgroup: 64 KB
constexpr int kWinWpitch = 33;          // weight row pitch in LDS (odd: lanes on distinct banks)

struct WinFwd {
    const float* x;
    int64_t sn, sc, sh, sw;  // image strides (elements)
    const float* w;          // [Cout][K], row stride wrow, k stride 1
    int64_t wrow;
    const float* bias;       // null: no bias
    int64_t bias_stride;
    float* out;              // [N][Cout][L] contiguous
    int32_t C, H, W, padh, padw, strh, strw, OW;
    int32_t Wp, rows, plane, stage;  // staged rows per channel, plane = rows * Wp, stage = C * plane
    uint32_t cout, K, L, nblk, wg_per_image;
    FastDiv div_ow;
    int32_t sc4, sh4;                // channel and row strides in bytes
    int32_t q4, r4;                  // 4 = q4 * rows + r4
    int32_t wave_c[4], wave_r[4];    // staged row w: channel and padded row
    int32_t offs[32];  // window element j's offset in the stage; j >= K: the zero region
};

// T: 32-channel tiles (1 or 2); BPW: blocks per wave; RELU: the epilogue's
// ReLU; FULL: Cout = 32*T and L % 32 == 0 (every store of a block inside the
// image unconditional).
// Without a bias the epilogue adds +0, which leaves every value's bits as
// they are: a chain that starts from +0 never ends at -0.
template <int T, int BPW, bool RELU, bool FULL>
__global__ __launch_bounds__(kWinThreads) void win_fwd_kernel(WinFwd p) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, kh = lane >> 5;
    const uint32_t n = blockIdx.y;
    const uint32_t b0 = blockIdx.x * static_cast<uint32_t>(kWinWaves * BPW);
    float* img = smem;                                    // [C][rows][Wp], then `plane` zeros
    float* wts = smem + ((p.stage + p.plane + 3) & ~3);   // [64][kWinWpitch]
    int32_t* offs_l = reinterpret_cast<int32_t*>(wts + 64 * kWinWpitch);  // [32]
    float* bias_l = wts + 64 * kWinWpitch + 32;  // [64]
    const int32_t row_a = static_cast<int32_t>(p.div_ow.div(32u * b0)) * p.strh;

    // The set-up's global loads in one batch. Buffer loads return 0 past the
    // resource (offsets with bit 31 set): the padding columns and the weight
    // slots past K or Cout are loaded as zeros without a select.
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.x + static_cast<int64_t>(n) * p.sn), 0, static_cast<int32_t>(0x80000000u), 0x00020000);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.w), 0, static_cast<int32_t>(0x80000000u), 0x00020000);
    // weights: thread slot e = tid + 256u is channel (tid >> 5) + 8u, element tid & 31
    const uint32_t wj = static_cast<uint32_t>(tid) & 31u, wc = static_cast<uint32_t>(tid) >> 5;
    const uint32_t wvoff = wj < p.K ? (wc * static_cast<uint32_t>(p.wrow) + wj) * 4u : 0x80000000u;
    float we[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        uint32_t voff = wvoff + static_cast<uint32_t>(u) * (32u * static_cast<uint32_t>(p.wrow));
        if (8u * u + 8u > p.cout) voff = wc + 8u * u < p.cout ? voff : 0x80000000u;
        we[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wr, static_cast<int32_t>(voff), 0, 0));
    }
    const int32_t my_off = p.offs[lane & 31];
    // staged rows: wave-uniform row (channel c, padded row rr), lane = padded column
    const int32_t nrows = p.C * p.rows;
    const int w_in = lane - p.padw;
    const bool col_in = lane < p.Wp && static_cast<uint32_t>(w_in) < static_cast<uint32_t>(p.W);
    const uint32_t xvoff = col_in ? static_cast<uint32_t>(w_in) * static_cast<uint32_t>(p.sw) * 4u : 0x80000000u;
    // row wave + 4u is channel c, padded row rr, walked incrementally
    // (4 = q4 * rows + r4)
    constexpr int U = 16;  // staged rows per wave at most (the launch checks C * rows <= 64)
    float sv[U];
    int32_t c = p.wave_c[wave], rr = p.wave_r[wave];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        sv[u] = 0.0f;
        if (wave + kWinWaves * u >= nrows) break;
        {
            const int32_t h = row_a + rr - p.padh;
            if (static_cast<uint32_t>(h) < static_cast<uint32_t>(p.H))
                sv[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                      xr, static_cast<int32_t>(xvoff), c * p.sc4 + h * p.sh4, 0));
        }
        rr += p.r4;
        c += p.q4;
        if (rr >= p.rows) {
            rr -= p.rows;
            ++c;
        }
    }

    // LDS: the zero region, the weights, the window offsets, the staged rows.
    for (int e = tid; e < p.plane; e += kWinThreads) img[p.stage + e] = 0.0f;
#pragma unroll
    for (int u = 0; u < 8; ++u) wts[(wc + 8u * u) * kWinWpitch + wj] = we[u];
    if (tid < 32) offs_l[tid] = my_off;
    if (tid < 64) bias_l[tid] = p.bias && static_cast<uint32_t>(tid) < p.cout ? p.bias[tid * p.bias_stride] : 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int32_t row = wave + kWinWaves * u;
        if (row >= nrows) break;
        if (lane < p.Wp) img[row * p.Wp + lane] = sv[u];
    }
    __syncthreads();

    // This lane's weights (B: window element t + 16*kh of channel 32i + lrow,
    // zero past K or Cout) and window offsets.
    const float* wl = wts + lrow * kWinWpitch + 16 * kh;
    float bw[T][16];
#pragma unroll
    for (int i = 0; i < T; ++i)
#pragma unroll
        for (int t = 0; t < 16; ++t) bw[i][t] = wl[i * 32 * kWinWpitch + t];
    int32_t off[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) off[t] = offs_l[16 * kh + t];
    float bv[T][16];  // the bias of channel 32i + 8(r/4) + 4kh + r%4
#pragma unroll
    for (int i = 0; i < T; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) bv[i][r] = bias_l[32 * i + 8 * (r / 4) + 4 * kh + r % 4];
    // every set-up read lands before the first block's chain starts
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_sched_barrier(0);
    const __amdgpu_buffer_rsrc_t outr = __builtin_amdgcn_make_buffer_rsrc(
        p.out + static_cast<uint64_t>(n) * p.cout * p.L, 0, static_cast<int32_t>(0x80000000u), 0x00020000);

    // Block u of this wave is b0 + wave + 4u. Blocks are software-pipelined:
    // block u's MFMA chain is issued before block u-1's epilogue, so that one
    // wave keeps the matrix core busy while its previous outputs are biased,
    // rectified and stored. Blocks past the image (a partial last workgroup)
    // are computed on clamped positions and not stored.
    auto gather = [&](uint32_t b, float (&av)[16]) {
        const uint32_t pos = 32u * min(b, p.nblk - 1u) + lrow;
        const uint32_t pc = FULL ? pos : min(pos, p.L - 1u);
        const uint32_t oh = p.div_ow.div(pc), ow = pc - oh * static_cast<uint32_t>(p.OW);
        const int32_t base = (static_cast<int32_t>(oh) * p.strh - row_a) * p.Wp + static_cast<int32_t>(ow) * p.strw;
#pragma unroll
        for (int t = 0; t < 16; ++t) av[t] = img[base + off[t]];
    };
    auto chain = [&](const float (&av)[16], v16f (&acc)[T]) {
#pragma unroll
        for (int i = 0; i < T; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
#pragma unroll
        for (int t = 0; t < 16; ++t)
#pragma unroll
            for (int i = 0; i < T; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(bw[i][t], av[t], acc[i], 0, 0, 0);
    };
    // lane (lrow, kh) holds channel 32i + 8(r/4) + 4kh + r%4 of position
    // 32b + lrow in acc[i][r]: each store instruction writes two whole
    // 128-byte rows of 32 positions
    auto epilogue = [&](uint32_t b, const v16f (&acc)[T]) {
        if (b >= p.nblk) return;  // the last workgroup of an image may run past its blocks
        const uint32_t pos = 32u * b + lrow;
#pragma unroll
        for (int i = 0; i < T; ++i) {
            const uint32_t voff = (pos + (32u * i + 4u * kh) * p.L) * 4u;
            float v[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float x = acc[i][r] + bv[i][r];
                if (RELU) x = x <= 0.0f ? 0.0f : x;
                v[r] = x;
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t co = 32u * i + 8u * (r / 4) + 4u * kh + r % 4;
                if (FULL || (co < p.cout && pos < p.L))
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, v[r]), outr, static_cast<int32_t>(voff),
                                                          static_cast<int32_t>((8 * (r / 4) + r % 4) * p.L * 4u), 2);
            }
        }
    };
    const uint32_t bw0 = b0 + static_cast<uint32_t>(wave);
    v16f acc[2][T];
    float av[2][16];
    gather(bw0, av[0]);
#pragma unroll
    for (int u = 0; u < BPW; ++u) {
        // the next block's window values are read while this block's chain runs
        if (u + 1 < BPW) gather(bw0 + kWinWaves * (u + 1), av[(u + 1) & 1]);
        chain(av[u & 1], acc[u & 1]);
        if (u > 0) epilogue(bw0 + kWinWaves * (u - 1), acc[(u - 1) & 1]);
    }
    epilogue(bw0 + kWinWaves * (BPW - 1), acc[(BPW - 1) & 1]);
}

// Padded input rows per channel that the most demanding workgroup reads when
// each workgroup takes `span` consecutive positions of an image.
int32_t win_rows(uint32_t L, uint32_t ow, int32_t strh, int32_t kh, int32_t dilh, int32_t hp, uint32_t span) {
    int32_t rows = 1;
    for (uint32_t first = 0; first < L; first += span) {
        const uint32_t last = std::min(L, first + span) - 1u;
        rows = std::max(rows, static_cast<int32_t>(last / ow - first / ow) * strh + (kh - 1) * dilh + 1);
    }
    return std::min(rows, hp);
}

// LDS floats of a workgroup: the staged rows, the zero region, the weights,
// the window offsets.
size_t win_lds_floats(int32_t channels, int32_t rows, int32_t wp) {
    return ((static_cast<size_t>(channels + 1) * rows * wp + 3) & ~size_t(3)) + 64 * kWinWpitch + 32 + 64;
}

// Blocks per wave. One, with four waves per SIMD resident: the other
// waves' chains hide each wave's set-up and store waits. Measured at CIFAR
// conv1 (all bit-identical): 9.6 us at one block per wave, 15.0 us at two
// and 12.8 us at four (the pipelined loop below, 2 or 1 waves per SIMD).
constexpr uint32_t kWinBpw = 1;

}  // namespace

bool win_fwd_fits(const vkhip_operand& xd, const vkhip_unfold& pr, uint32_t channels, uint64_t ck,
                  uint32_t cout, const vkhip_operand& wd, uint32_t oh, uint32_t ow) {
    const int64_t hp = static_cast<int64_t>(pr.image_h) + 2 * pr.pad_h;
    const int64_t wp = static_cast<int64_t>(pr.image_w) + 2 * pr.pad_w;
    const uint64_t L = static_cast<uint64_t>(oh) * ow;
    if (!(ck >= 1 && ck <= 32 && cout >= 1 && cout <= 64 && (wd.nb[3] == 1 || ck == 1) && wp <= 64 &&
          hp <= 0x7fffffff && L >= 1 && L <= 0x7fffffffull && ow >= 1 && channels >= 1))
        return false;
    // 32-bit byte offsets below bit 31 for the image and the weights (buffer loads)
    if (xd.nb[1] < 0 || xd.nb[2] < 0 || xd.nb[3] < 0 || wd.nb[2] < 0) return false;
    const int64_t span = (static_cast<int64_t>(channels) - 1) * xd.nb[1] +
                         (static_cast<int64_t>(pr.image_h) - 1) * xd.nb[2] +
                         (static_cast<int64_t>(pr.image_w) - 1) * xd.nb[3] + 1;
    const int64_t wspan = (static_cast<int64_t>(cout) - 1) * wd.nb[2] + static_cast<int64_t>(ck) + 8 * wd.nb[2];
    if (span > (int64_t(1) << 28) || wspan > (int64_t(1) << 28) || static_cast<uint64_t>(cout) * L > (1ull << 28))
        return false;
    const int32_t rows = win_rows(static_cast<uint32_t>(L), ow, pr.stride_h, pr.kernel_h, pr.dilation_h,
                                  static_cast<int32_t>(hp), 32u * kWinWaves * kWinBpw);
    return static_cast<int64_t>(channels) * rows <= 16 * kWinWaves &&
           win_lds_floats(static_cast<int32_t>(channels), rows, static_cast<int32_t>(wp)) <= kWinLdsFloats;
}

int win_conv_forward(const float* x, const vkhip_operand& xd, const float* w, const vkhip_operand& wd,
                     float* out, const vkhip_unfold& pr, uint32_t batch, uint32_t channels, uint32_t cout,
                     uint32_t ck, uint32_t oh, uint32_t ow, const float* bias, int64_t bias_stride,
                     bool relu) {
    WinFwd p{};
    p.x = x;
    p.sn = xd.nb[0];
    p.sc = xd.nb[1];
    p.sh = xd.nb[2];
    p.sw = xd.nb[3];
    p.w = w;
    p.wrow = wd.nb[2];
    p.bias = bias;
    p.bias_stride = bias_stride;
    p.out = out;
    p.C = static_cast<int32_t>(channels);
    p.H = pr.image_h;
    p.W = pr.image_w;
    p.padh = pr.pad_h;
    p.padw = pr.pad_w;
    p.strh = pr.stride_h;
    p.strw = pr.stride_w;
    p.OW = static_cast<int32_t>(ow);
    p.Wp = pr.image_w + 2 * pr.pad_w;
    const int32_t hp = pr.image_h + 2 * pr.pad_h;
    p.cout = cout;
    p.K = ck;
    p.L = oh * ow;
    p.nblk = (p.L + 31u) / 32u;
    p.div_ow = FastDiv(ow);
    constexpr uint32_t bpw = kWinBpw;
    p.rows = win_rows(p.L, ow, p.strh, pr.kernel_h, pr.dilation_h, hp, 32u * kWinWaves * bpw);
    p.plane = p.rows * p.Wp;
    p.stage = p.C * p.plane;
    p.sc4 = static_cast<int32_t>(xd.nb[1] * 4);
    p.sh4 = static_cast<int32_t>(xd.nb[2] * 4);
    p.q4 = kWinWaves / p.rows;
    p.r4 = kWinWaves % p.rows;
    for (int w = 0; w < kWinWaves; ++w) {
        p.wave_c[w] = w / p.rows;
        p.wave_r[w] = w % p.rows;
    }
    const int32_t kk = pr.kernel_h * pr.kernel_w;
    for (uint32_t j = 0; j < 32; ++j) {
        if (j >= ck) {
            p.offs[j] = p.stage;
            continue;
        }
        const int32_t c = static_cast<int32_t>(j) / kk, r = static_cast<int32_t>(j) % kk;
        const int32_t ki = r / pr.kernel_w, kj = r % pr.kernel_w;
        p.offs[j] = c * p.plane + ki * pr.dilation_h * p.Wp + kj * pr.dilation_w;
    }
    const size_t lds = win_lds_floats(p.C, p.rows, p.Wp);
    if (p.C * p.rows > 16 * kWinWaves || lds > kWinLdsFloats)
        return fail(VKHIP_ERR_INVALID, "conv2d: staged rows exceed the small-window stage");
    p.wg_per_image = (p.nblk + kWinWaves * bpw - 1) / (kWinWaves * bpw);
    if (batch > 65535)
        return fail(VKHIP_ERR_UNSUPPORTED, "conv2d: batch %u above the grid's 65535", batch);
    const bool two = cout > 32;
    const bool full = cout == (two ? 64u : 32u) && p.L % 32 == 0;
    const dim3 g(p.wg_per_image, batch), blk(kWinThreads);
    const size_t bytes = lds * sizeof(float);
#define VKHIP_WINF(T, B, R, F) hipLaunchKernelGGL((win_fwd_kernel<T, B, R, F>), g, blk, bytes, ctx().stream, p)
#define VKHIP_WINF_F(T, B, R)                                             \
    do {                                                                  \
        if (full) VKHIP_WINF(T, B, R, true); else VKHIP_WINF(T, B, R, false); \
    } while (0)
#define VKHIP_WINF_R(T, B)                                                \
    do {                                                                  \
        if (relu) VKHIP_WINF_F(T, B, true); else VKHIP_WINF_F(T, B, false);   \
    } while (0)
    static_assert(kWinBpw == 1, "instantiate the launch for other blocks per wave");
    if (two) VKHIP_WINF_R(2, 1); else VKHIP_WINF_R(1, 1);
#undef VKHIP_WINF_R
#undef VKHIP_WINF_F
#undef VKHIP_WINF
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}


// ---- weight gradient summed over the batch ------------------------------------
// dW[co][j] = sum over images n and positions p of g[n][co][p] * window element
// j of image n at p (reference: the per-image products matmul(grad, cols^T)
// and the broadcast adjoint's batch sum, autograd.cpp:548-553 and :84-116).
// At CIFAR conv1 the product is [64 x 27] with K = 128 x 1024 positions: it is
// bound by reading the 33.5 MB gradient once.
//
// win_wgrad_kernel: a workgroup of four waves takes CH chunks of 64 positions
// of one image (512 positions at CIFAR conv1: 256 workgroups). It stages the
// input rows those positions read once (as the forward does, with the zero
// region for window elements past K), and streams the gradient through a ring
// of registers D chunks ahead: each chunk is loaded with 16-byte loads of
// whole 256-byte channel rows (16 consecutive lanes on consecutive
// addresses), and written to one of two LDS buffers in a swizzled layout (the
// 16-byte group p of channel co sits at co*16 + (p ^ (co % 16))), from which a
// lane of the product reads its channel's four consecutive positions without
// bank conflicts. Chunk c + 1 is written and read into registers while chunk
// c's MFMAs run. The product is channels x window elements with the positions
// as K: lanes 0-31 and 32-63 take positions p and p + 4 of each 8-position
// group, four steps per 16-byte read; even and odd steps accumulate
// separately (two chains per tile) and are added at the end. The four waves'
// sums are added in wave order through LDS, and the workgroup's [64 x 32]
// partial goes to the workspace.
//
// Measured at CIFAR conv1: 16.4 us with the fold (against 21.3 for the
// per-workgroup streamed kernel it replaces and 30.5 for the per-image
// products and batch sum). The loads alone, in this pattern at one workgroup
// per CU, take 7.7 us; the 33.5 MB read linearly by many workgroups 5.9 us.
//
// The 256 workgroup partials are folded by win_fold_kernel in a second
// launch: each output's partials in workgroup order, as 16 runs added in
// parallel and then in run order. (Folding inside the same launch -- the last
// workgroup of each group of 16 adding the group's partials, the last group
// adding the group sums, ordered by device-scope atomic counts -- measured 29
// us: its tail is six dependent round trips to the level all XCDs share;
// device-scope fences, which write back the L2, made it 109 us.) Fixed orders
// throughout: the result is the same bits on every run, within the GEMM
// tolerance of the per-image graph.
namespace {

constexpr uint32_t kWgMaxParts = 512;  // workgroup partials at most (the fold's 16 runs of 32)

struct WinWgrad {
    const float* x;
    int64_t sn;                // image stride (elements)
    int32_t sc4, sh4, sw4;     // channel, row and column strides of the image (bytes)
    const float* g;
    int64_t gsn;               // gradient image stride (elements)
    int32_t gsc;               // gradient channel stride (elements; rows 16-byte aligned)
    float* part;               // [nwg][2048] workgroup partials (output co * 32 + j)
    float* out;                // [Cout][K]
    // GM = 1: g is the pool's input y (the layer's relu output) and the
    // gradient is that of a 2x2, stride-2 max-pool of y given the pool's
    // output gradient gp [N][Cout][oh/2][ow/2] (rows contiguous).
    const float* gp;
    int64_t gpsn;              // pool gradient image stride (elements)
    int32_t gpsc;              // pool gradient channel stride (elements, even)
    float* bpart;              // GM = 1: [nwg][64] the bias gradient's span sums
    int32_t C, H, W, padh, padw, strh, strw, OW, Wp, rows, plane, stage;
    uint32_t cout, K, L, wg_per_image, nwg;
    FastDiv div_ow;
    int32_t q_step, r_step;            // waves = q_step * rows + r_step
    int32_t wave_c[8], wave_r[8];      // staged row w: channel and padded row
    int32_t offs[32];
};

template <int T, int NW, int CH, int D, int GM>
__global__ __launch_bounds__(64 * NW) void win_wgrad_kernel(WinWgrad p) {
    static_assert(GM == 0 || (NW == 4 && (CH & (CH - 1)) == 0), "pool-gradient chunks: 64 positions");
    extern __shared__ __attribute__((aligned(16))) float smem[];
    constexpr int NT = 64 * NW;        // threads
    constexpr int PC = 16 * NW;        // positions per chunk: 16 per wave
    constexpr int G = PC / 4;          // 16-byte position groups per channel row of a chunk
    constexpr int CF = 64 * PC;        // floats per chunk buffer
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, kh = lane >> 5;
    const uint32_t n = blockIdx.y;
    const uint32_t pos0 = blockIdx.x * static_cast<uint32_t>(PC * CH);  // first position of the workgroup
    float* img = smem;                                          // [C][rows][Wp], then `plane` zeros
    float* gbuf = smem + ((p.stage + p.plane + 3) & ~3);        // 2 x [64 x PC] swizzled
    int32_t* offs_l = reinterpret_cast<int32_t*>(gbuf + 2 * CF);
    const int32_t row_a = static_cast<int32_t>(p.div_ow.div(pos0)) * p.strh;

    // Gradient chunk c: 64 * G 16-byte slots, thread tid loads slots tid + NT u:
    // channel s / G, position group s % G, stored at group (s % G) ^ (channel
    // % 16) of the channel's row. Channels past Cout load zeros.
    const __amdgpu_buffer_rsrc_t gr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.g + static_cast<int64_t>(n) * p.gsn), 0, static_cast<int32_t>(0x80000000u), 0x00020000);
    uint32_t goff[4];
    int32_t gdst[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const uint32_t sl = static_cast<uint32_t>(tid) + NT * u, co = sl / G, grp = sl % G;
        goff[u] = co < p.cout ? (co * static_cast<uint32_t>(p.gsc) + pos0 + 4u * grp) * 4u : 0x80000000u;
        gdst[u] = static_cast<int32_t>(co * G + (grp ^ (co & 15u))) * 4;
    }
    // GM = 1: the chunk's gradient from the pool. A chunk (64 positions) is
    // 64 / OW whole row pairs, i.e. 512 blocks of 2 rows x 4 positions (two
    // pool windows); thread tid takes blocks tid and tid + 256: channel s / 8,
    // block s % 8 = row pair rp and column group cg. Each block loads y's two
    // rows (16 bytes each) and the two windows' pool gradients (8 bytes), and
    // stores the max-pool backward with the relu mask (the values of
    // max_pool2x2_backward_kernel<true>) as the two 16-byte groups of its rows.
    const __amdgpu_buffer_rsrc_t pr_ = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(GM == 1 ? p.gp + static_cast<int64_t>(n) * p.gpsn : p.g), 0,
        static_cast<int32_t>(0x80000000u), 0x00020000);
    uint32_t poff[2] = {0u, 0u}, row2 = 0u;
    int32_t pdst[2][2] = {{0, 0}, {0, 0}};
    if constexpr (GM == 1) {
        const uint32_t qw = static_cast<uint32_t>(p.OW) / 4u;
        row2 = static_cast<uint32_t>(p.OW) * 4u;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint32_t sl = static_cast<uint32_t>(tid) + NT * u, co = sl >> 3, b = sl & 7u;
            const uint32_t rp = b / qw, cg = b - rp * qw;
            const uint32_t at = 2u * rp * static_cast<uint32_t>(p.OW) + 4u * cg;  // block's first position in the chunk
            goff[u] = co < p.cout ? (co * static_cast<uint32_t>(p.gsc) + pos0 + at) * 4u : 0x80000000u;
            poff[u] = co < p.cout ? (co * static_cast<uint32_t>(p.gpsc) + pos0 / 4u + rp * (p.OW / 2u) + 2u * cg) * 4u
                                  : 0x80000000u;
            const uint32_t gtop = at / 4u, gbot = gtop + qw;
            pdst[u][0] = static_cast<int32_t>(co * G + (gtop ^ (co & 15u))) * 4;
            pdst[u][1] = static_cast<int32_t>(co * G + (gbot ^ (co & 15u))) * 4;
        }
    }
    v4f ring[D][4];
    v2f pring[D][2];
    auto load_chunk = [&](int c, v4f (&r)[4], v2f (&pg)[2]) {
        if constexpr (GM == 1) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                r[2 * u] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(
                                                       gr, static_cast<int32_t>(goff[u]), c * PC * 4, 0));
                r[2 * u + 1] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(
                                                           gr, static_cast<int32_t>(goff[u] + row2), c * PC * 4, 0));
                pg[u] = __builtin_bit_cast(v2f, __builtin_amdgcn_raw_buffer_load_b64(
                                                    pr_, static_cast<int32_t>(poff[u]), c * PC, 0));
            }
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u)
                r[u] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(
                                                   gr, static_cast<int32_t>(goff[u]), c * PC * 4, 0));
        }
    };
    auto store_chunk = [&](int buf, const v4f (&r)[4], const v2f (&pg)[2]) {
        if constexpr (GM == 1) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const v4f t = r[2 * u], b = r[2 * u + 1];
                const int32_t a0 = argmax4(t[0], t[1], b[0], b[1]);
                const int32_t a1 = argmax4(t[2], t[3], b[2], b[3]);
                const float g0 = 0.0f + pg[u][0], g1 = 0.0f + pg[u][1];
                v4f top, bot;
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
                    if (t[i] <= 0.0f) top[i] = 0.0f;
                    if (b[i] <= 0.0f) bot[i] = 0.0f;
                }
                *reinterpret_cast<v4f*>(gbuf + buf * CF + pdst[u][0]) = top;
                *reinterpret_cast<v4f*>(gbuf + buf * CF + pdst[u][1]) = bot;
            }
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) *reinterpret_cast<v4f*>(gbuf + buf * CF + gdst[u]) = r[u];
        }
    };
    // The input rows of the workgroup's positions, staged as the forward does.
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.x + static_cast<int64_t>(n) * p.sn), 0, static_cast<int32_t>(0x80000000u), 0x00020000);
    const int32_t my_off = p.offs[lane & 31];
    const int32_t nrows = p.C * p.rows;
    const int w_in = lane - p.padw;
    const bool col_in = lane < p.Wp && static_cast<uint32_t>(w_in) < static_cast<uint32_t>(p.W);
    const uint32_t xvoff = col_in ? static_cast<uint32_t>(w_in) * static_cast<uint32_t>(p.sw4) : 0x80000000u;
    constexpr int U = 64 / NW;
    float sv[U];
    {
        int32_t c = p.wave_c[wave], rr = p.wave_r[wave];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            sv[u] = 0.0f;
            if (wave + NW * u >= nrows) break;
            const int32_t h = row_a + rr - p.padh;
            if (static_cast<uint32_t>(h) < static_cast<uint32_t>(p.H))
                sv[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                      xr, static_cast<int32_t>(xvoff), c * p.sc4 + h * p.sh4, 0));
            rr += p.r_step;
            c += p.q_step;
            if (rr >= p.rows) {
                rr -= p.rows;
                ++c;
            }
        }
    }
    // the first D chunks' loads go out behind the image's
#pragma unroll
    for (int c = 0; c < D && c < CH; ++c) load_chunk(c, ring[c], pring[c]);
    for (int e = tid; e < p.plane; e += NT) img[p.stage + e] = 0.0f;
    if (tid < 32) offs_l[tid] = my_off;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int32_t row = wave + NW * u;
        if (row >= nrows) break;
        if (lane < p.Wp) img[row * p.Wp + lane] = sv[u];
    }
    store_chunk(0, ring[0], pring[0]);
    __syncthreads();
    const int32_t off = offs_l[lrow];  // this lane's window element (B column lrow)

    // GM = 1, the bias gradient: the sum over the workgroup's span of each
    // channel's gradient as the oracle's pairwise tree takes it (the span is
    // an aligned power-of-two subtree): leaves of 32 positions summed in order
    // from +0, adjacent leaves and then pairs added level by level. A chunk
    // holds two leaves per channel; half the threads (waves 0-1 for even
    // chunks, 2-3 for odd ones) sum one leaf each from the chunk buffer, and
    // the even lane keeps the pair's sum in bl[c][co].
    float* bl = reinterpret_cast<float*>(offs_l + 32);  // [CH][64]
    auto leaves = [&](int c) {
        if constexpr (GM == 1) {
            const int t = (tid + 128 * (c & 1)) & 255;
            if (t < 128) {
                const uint32_t co = static_cast<uint32_t>(t) >> 1, j = static_cast<uint32_t>(t) & 1u;
                const float* gb = gbuf + (c & 1) * CF;
                float sum = 0.0f;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const uint32_t grp = 8u * j + k;
                    const v4f v = *reinterpret_cast<const v4f*>(gb + (co * G + (grp ^ (co & 15u))) * 4u);
                    sum = sum + v[0];
                    sum = sum + v[1];
                    sum = sum + v[2];
                    sum = sum + v[3];
                }
                const float other = wave_partner<1>(sum);
                if (j == 0) bl[c * 64 + co] = sum + other;
            }
        }
    };

    // A chunk's operands of this wave: its 16 positions are the 4-position
    // groups 8gg + 4kh (gg = 0, 1); a[gg][i] = 4 positions of channel 32i +
    // lrow, b[gg][q] = window element lrow at the lane's position q.
    struct Ops {
        v4f a[2][T];
        float b[2][4];
    };
    auto read_ops = [&](int c, Ops& o) {
        const float* gb = gbuf + (c & 1) * CF;
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
            const uint32_t grp = 4u * wave + 2u * gg + kh;
#pragma unroll
            for (int i = 0; i < T; ++i) {
                const uint32_t co = 32u * i + lrow;
                o.a[gg][i] = *reinterpret_cast<const v4f*>(gb + (co * G + (grp ^ (co & 15u))) * 4u);
            }
            const uint32_t pp = pos0 + PC * c + 4u * grp;  // this lane's first position
            const uint32_t oh = p.div_ow.div(pp), ow = pp - oh * static_cast<uint32_t>(p.OW);
            const int32_t base = (static_cast<int32_t>(oh) * p.strh - row_a) * p.Wp +
                                 static_cast<int32_t>(ow) * p.strw + off;
#pragma unroll
            for (int q = 0; q < 4; ++q) o.b[gg][q] = img[base + q * p.strw];
        }
    };
    v16f acc[2][T];
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int i = 0; i < T; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[e][i][r] = 0.0f;
    auto mfma_ops = [&](const Ops& o) {
#pragma unroll
        for (int gg = 0; gg < 2; ++gg)
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int i = 0; i < T; ++i)
                    acc[q & 1][i] = __builtin_amdgcn_mfma_f32_32x32x2f32(o.a[gg][i][q], o.b[gg][q], acc[q & 1][i], 0, 0, 0);
    };

    // Chunk c + 1 is written to LDS and read into registers while chunk c's
    // MFMAs run. Buffer (c + 1) & 1 last held chunk c - 1, whose reads ended
    // before the previous barrier.
    Ops ops[2];
    read_ops(0, ops[0]);
    leaves(0);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        if (c + D < CH) load_chunk(c + D, ring[c % D], pring[c % D]);  // its slot's data is in LDS already
        if (c + 1 < CH) {
            store_chunk((c + 1) & 1, ring[(c + 1) % D], pring[(c + 1) % D]);
            __syncthreads();
            read_ops(c + 1, ops[(c + 1) & 1]);
            leaves(c + 1);
        }
        mfma_ops(ops[c & 1]);
    }
    __syncthreads();  // every wave is done with the chunk buffers

    // The waves' sums in wave order, through the (now idle) gradient buffers.
    float* red = gbuf;  // [NW][T][16][64] <= 2 chunk buffers
#pragma unroll
    for (int i = 0; i < T; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[((wave * T + i) * 16 + r) * 64 + lane] = acc[0][i][r] + acc[1][i][r];
    __syncthreads();
    const uint32_t wg = n * p.wg_per_image + blockIdx.x;
    if constexpr (GM == 1) {
        // the chunk pairs' sums up the balanced tree: the span's sum
        if (tid < 64) {
            float v[CH];
#pragma unroll
            for (int c = 0; c < CH; ++c) v[c] = bl[c * 64 + tid];
#pragma unroll
            for (int w = 1; w < CH; w *= 2)
#pragma unroll
                for (int i = 0; i + w < CH; i += 2 * w) v[i] = v[i] + v[i + w];
            p.bpart[static_cast<uint64_t>(wg) * 64u + tid] = v[0];
        }
    }
    float* mine = p.part + static_cast<uint64_t>(wg) * 2048u;
    // output o = co * 32 + j of the partial; lane l of register r of tile i
    // holds co = 32i + 8(r/4) + 4(l/32) + r%4, j = l%32
#pragma unroll
    for (int k = 0; k < 2048 / NT; ++k) {
        const uint32_t o = static_cast<uint32_t>(tid) + NT * k, co = o >> 5, j = o & 31u;
        if (co >= 32u * T) break;
        const uint32_t i = co >> 5, rem = co & 31u, r = 4u * (rem >> 3) + (rem & 3u), l = j + 32u * ((rem >> 2) & 1u);
        float v = red[((0 * T + i) * 16 + r) * 64 + l];
#pragma unroll
        for (int w = 1; w < NW; ++w) v = v + red[((w * T + i) * 16 + r) * 64 + l];
        mine[o] = v;
    }
}

// dW[co][j] = the sum of the `parts` workgroup partials of output o = co*32 + j
// ([parts][2048] at part), in partial order: 16 threads per output, each
// adding a run of at most 16 consecutive partials, then the 16 run sums in run
// order (at most 32 per run). A workgroup takes 16 outputs.
//
// With bpart (the pool-gradient kernel's span sums, [parts][64], parts a power
// of two >= 4), the last four workgroups fold the bias gradient into
// bout[Cout], 16 channels each: per channel the balanced pairwise tree over
// the span sums, as R = min(16, parts) runs of parts / R consecutive sums (a
// binary-counter carry stack over each, which for a power-of-two count is the
// balanced tree), then the R run sums level by level.
__global__ __launch_bounds__(256) void win_fold_kernel(const float* __restrict__ part, uint32_t parts,
                                                       float* __restrict__ out, uint32_t cout, uint32_t K,
                                                       const float* __restrict__ bpart, float* __restrict__ bout) {
    __shared__ float runs[16][17];
    const int tid = threadIdx.x, oi = tid & 15, run = tid >> 4;
    if (bpart != nullptr && blockIdx.x >= gridDim.x - 4) {
        const uint32_t co = (blockIdx.x - (gridDim.x - 4)) * 16u + static_cast<uint32_t>(oi);
        const uint32_t nr = parts < 16u ? parts : 16u, per = parts / nr;
        float r = 0.0f;
        if (static_cast<uint32_t>(run) < nr) {
            float stack[6];
#pragma unroll
            for (int l = 0; l < 6; ++l) stack[l] = 0.0f;
            for (uint32_t i0 = 0; i0 < per; i0 += 8) {
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    v[u] = i0 + u < per ? bpart[static_cast<uint64_t>(run * per + i0 + u) * 64u + co] : 0.0f;
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    if (i0 + u >= per) break;
                    const uint32_t count = i0 + u;
                    float b = v[u];
                    bool carry = true;
#pragma unroll
                    for (int l = 0; l < 6; ++l) {
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
            for (int l = 0; l < 6; ++l)
                if (per == (1u << l)) r = stack[l];
        }
        runs[run][oi] = r;
        __syncthreads();
        if (tid < 16) {
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = runs[i][tid];
#pragma unroll
            for (int w = 1; w < 16; w *= 2)
#pragma unroll
                for (int i = 0; i + w < 16; i += 2 * w)
                    if (static_cast<uint32_t>(i + w) < nr) v[i] = v[i] + v[i + w];
            if (co < cout) bout[co] = v[0];
        }
        return;
    }
    const uint32_t o = blockIdx.x * 16u + oi;
    const uint32_t per = (parts + 15u) / 16u, first = run * per;
    float x[32];
#pragma unroll
    for (int w = 0; w < 32; ++w) {
        const uint32_t q = first + w;
        x[w] = part[static_cast<uint64_t>(q < parts && static_cast<uint32_t>(w) < per ? q : 0u) * 2048u + o];
    }
    float v = 0.0f;
    bool any = false;
#pragma unroll
    for (int w = 0; w < 32; ++w) {
        const bool in = static_cast<uint32_t>(w) < per && first + w < parts;
        const float t = any ? v + x[w] : x[w];
        v = in ? t : v;
        any = any || in;
    }
    runs[run][oi] = v;
    __syncthreads();
    if (tid < 16) {
        float s = runs[0][tid];
        for (uint32_t r = 1; r < 16 && r * per < parts; ++r) s = s + runs[r][tid];
        const uint32_t oo = blockIdx.x * 16u + tid, co = oo >> 5, j = oo & 31u;
        if (co < cout && j < K) out[co * K + j] = s;
    }
}

// Positions per workgroup: the largest of 512, 256, 128, 64 that divides an
// image's positions and leaves at most kWgMaxParts workgroups; 0 if none does.
uint32_t win_wgrad_span(uint64_t batch, uint32_t L) {
    for (uint32_t span = 512; span >= 64; span /= 2)
        if (L % span == 0 && batch * (L / span) <= kWgMaxParts) return span;
    return 0;
}

// Waves per workgroup: four, chunks of 64 positions (measured at CIFAR conv1:
// 16.4 us with the fold, against 17.3 us for eight waves and chunks of 128).
constexpr uint32_t kWgWaves = 4;

constexpr int kWgLdsFloats = 24576;  // dynamic LDS of the weight-gradient kernel: 96 KB

// LDS floats: the staged rows and zero region, two chunk buffers, the offsets
// and the pool-gradient kernel's chunk pair sums (8 chunks x 64 channels).
size_t win_wgrad_lds(int32_t channels, int32_t plane, uint32_t waves) {
    return ((static_cast<size_t>(channels + 1) * plane + 3) & ~size_t(3)) + 2 * 64 * 16 * waves + 32 + 512;
}

// The pool-gradient variant's arguments (GM = 1).
struct WinPoolGrad {
    const float* gp;  // [N][Cout][oh/2][ow/2]
    int64_t gpsn, gpsc;
    float* bias_out;  // [Cout]
};


}  // namespace

// The batch-summed weight gradient's two launches (pool: the pool-gradient
// variant with the bias gradient).
static int win_weight_grad_launch(const float* x, const vkhip_operand& xd, const float* g, const vkhip_operand& gd,
                                  float* out, const vkhip_unfold& pr, uint32_t batch, uint32_t channels,
                                  uint32_t cout, uint32_t ck, uint32_t oh, uint32_t ow, const WinPoolGrad* pool);

bool win_wgrad_fits(const float* g, const vkhip_operand& gd, const vkhip_operand& xd, const vkhip_unfold& pr,
                    uint32_t channels, uint64_t ck, uint32_t cout, uint64_t batch, uint32_t oh, uint32_t ow) {
    const int64_t hp = static_cast<int64_t>(pr.image_h) + 2 * pr.pad_h;
    const int64_t wp = static_cast<int64_t>(pr.image_w) + 2 * pr.pad_w;
    const uint64_t L = static_cast<uint64_t>(oh) * ow;
    if (!(ck >= 1 && ck <= 32 && cout >= 1 && cout <= 64 && wp <= 64 && hp <= 0x7fffffff && channels >= 1 &&
          L >= 64 && L % 64 == 0 && ow % 4 == 0 && L <= (1u << 24) && batch >= 1 && batch <= 65535))
        return false;
    // 16-byte aligned gradient rows of contiguous positions, 32-bit byte offsets
    if (reinterpret_cast<uintptr_t>(g) % 16 != 0 || gd.nb[3] != 1 || gd.nb[1] < 0 || gd.nb[2] < 0 ||
        gd.nb[1] % 4 != 0 || gd.nb[2] % 4 != 0 || (static_cast<int64_t>(cout) - 1) * gd.nb[2] + L > (int64_t(1) << 28))
        return false;
    if (xd.nb[1] < 0 || xd.nb[2] < 0 || xd.nb[3] < 0) return false;
    const int64_t xspan = (static_cast<int64_t>(channels) - 1) * xd.nb[1] +
                          (static_cast<int64_t>(pr.image_h) - 1) * xd.nb[2] +
                          (static_cast<int64_t>(pr.image_w) - 1) * xd.nb[3] + 1;
    if (xspan > (int64_t(1) << 28)) return false;
    const uint32_t span = win_wgrad_span(batch, static_cast<uint32_t>(L));
    if (span == 0) return false;
    const uint32_t waves = kWgWaves;
    const int32_t r2 = win_rows(static_cast<uint32_t>(L), ow, pr.stride_h, pr.kernel_h, pr.dilation_h,
                                static_cast<int32_t>(hp), span);
    const size_t lds = win_wgrad_lds(static_cast<int32_t>(channels), r2 * static_cast<int32_t>(wp), waves);
    return static_cast<int64_t>(channels) * r2 <= 64 && lds <= kWgLdsFloats;
}

int win_conv_weight_grad_sum(const float* x, const vkhip_operand& xd, const float* g, const vkhip_operand& gd,
                             float* out, const vkhip_unfold& pr, uint32_t batch, uint32_t channels, uint32_t cout,
                             uint32_t ck, uint32_t oh, uint32_t ow) {
    return win_weight_grad_launch(x, xd, g, gd, out, pr, batch, channels, cout, ck, oh, ow, nullptr);
}

bool win_pool_wgrad_fits(const float* y, const vkhip_operand& yd, const float* gp, int64_t gpsn, int64_t gpsc,
                         const vkhip_operand& xd, const vkhip_unfold& pr, uint32_t channels, uint64_t ck,
                         uint32_t cout, uint64_t batch, uint32_t oh, uint32_t ow) {
    if (!win_wgrad_fits(y, yd, xd, pr, channels, ck, cout, batch, oh, ow)) return false;
    // chunks of whole row pairs, a power-of-two reduction (so every span is an
    // aligned subtree of the pairwise tree) and at least four spans
    const uint64_t L = static_cast<uint64_t>(oh) * ow;
    const uint64_t total = batch * L;
    if (!(ow == 4 || ow == 8 || ow == 16 || ow == 32) || oh % 2 != 0 || (total & (total - 1)) != 0) return false;
    const uint32_t span = win_wgrad_span(batch, static_cast<uint32_t>(L));
    if (span == 0 || total / span < 4) return false;
    // 8-byte pool-gradient pairs, rows contiguous, 32-bit byte offsets
    if (reinterpret_cast<uintptr_t>(gp) % 8 != 0 || gpsc % 2 != 0 || gpsc < static_cast<int64_t>(L / 4) ||
        gpsn < 0 || (static_cast<int64_t>(cout) - 1) * gpsc + static_cast<int64_t>(L / 4) > (int64_t(1) << 28))
        return false;
    return true;
}

int win_conv_pool_weight_bias_grad(const float* x, const vkhip_operand& xd, const float* y, const vkhip_operand& yd,
                                   const float* gp, int64_t gpsn, int64_t gpsc, float* out, float* bias_out,
                                   const vkhip_unfold& pr, uint32_t batch, uint32_t channels, uint32_t cout,
                                   uint32_t ck, uint32_t oh, uint32_t ow) {
    const WinPoolGrad pool{gp, gpsn, gpsc, bias_out};
    return win_weight_grad_launch(x, xd, y, yd, out, pr, batch, channels, cout, ck, oh, ow, &pool);
}

static int win_weight_grad_launch(const float* x, const vkhip_operand& xd, const float* g, const vkhip_operand& gd,
                                  float* out, const vkhip_unfold& pr, uint32_t batch, uint32_t channels,
                                  uint32_t cout, uint32_t ck, uint32_t oh, uint32_t ow, const WinPoolGrad* pool) {
    WinWgrad p{};
    p.x = x;
    p.sn = xd.nb[0];
    p.sc4 = static_cast<int32_t>(xd.nb[1] * 4);
    p.sh4 = static_cast<int32_t>(xd.nb[2] * 4);
    p.sw4 = static_cast<int32_t>(xd.nb[3] * 4);
    p.g = g;
    p.gsn = gd.nb[1];
    p.gsc = static_cast<int32_t>(gd.nb[2]);
    p.out = out;
    p.C = static_cast<int32_t>(channels);
    p.H = pr.image_h;
    p.W = pr.image_w;
    p.padh = pr.pad_h;
    p.padw = pr.pad_w;
    p.strh = pr.stride_h;
    p.strw = pr.stride_w;
    p.OW = static_cast<int32_t>(ow);
    p.Wp = pr.image_w + 2 * pr.pad_w;
    const int32_t hp = pr.image_h + 2 * pr.pad_h;
    p.cout = cout;
    p.K = ck;
    p.L = oh * ow;
    p.div_ow = FastDiv(ow);
    const uint32_t span = win_wgrad_span(batch, p.L);
    if (span == 0) return fail(VKHIP_ERR_INVALID, "conv2d weight grad sum: no span for %u positions", p.L);
    const uint32_t waves = kWgWaves, ch = span / (16u * waves);
    p.rows = win_rows(p.L, ow, p.strh, pr.kernel_h, pr.dilation_h, hp, span);
    p.plane = p.rows * p.Wp;
    p.stage = p.C * p.plane;
    p.q_step = static_cast<int32_t>(waves) / p.rows;
    p.r_step = static_cast<int32_t>(waves) % p.rows;
    for (int w = 0; w < 8; ++w) {
        p.wave_c[w] = w / p.rows;
        p.wave_r[w] = w % p.rows;
    }
    const int32_t kk = pr.kernel_h * pr.kernel_w;
    for (uint32_t j = 0; j < 32; ++j) {
        if (j >= ck) {
            p.offs[j] = p.stage;
            continue;
        }
        const int32_t c = static_cast<int32_t>(j) / kk, r = static_cast<int32_t>(j) % kk;
        const int32_t ki = r / pr.kernel_w, kj = r % pr.kernel_w;
        p.offs[j] = c * p.plane + ki * pr.dilation_h * p.Wp + kj * pr.dilation_w;
    }
    p.wg_per_image = p.L / span;
    p.nwg = batch * p.wg_per_image;
    const size_t lds = win_wgrad_lds(p.C, p.plane, waves);
    if (p.C * p.rows > 64 || lds > kWgLdsFloats || p.nwg > kWgMaxParts)
        return fail(VKHIP_ERR_INVALID, "conv2d weight grad sum: the small-window plan does not fit");
    const size_t part_floats = static_cast<size_t>(p.nwg) * (2048u + (pool ? 64u : 0u));
    const int st = workspace(part_floats * sizeof(float), &p.part);
    if (st != VKHIP_OK) return st;
    if (pool) {
        p.gp = pool->gp;
        p.gpsn = pool->gpsn;
        p.gpsc = static_cast<int32_t>(pool->gpsc);
        p.bpart = p.part + static_cast<size_t>(p.nwg) * 2048u;
        if ((p.nwg & (p.nwg - 1)) != 0 || p.nwg < 4 || (ch & (ch - 1)) != 0 || 2 * p.OW > 64 || 64 % (2 * p.OW) != 0)
            return fail(VKHIP_ERR_INVALID, "conv2d pool weight grad: the small-window plan does not fit");
    }
    const dim3 grid(p.wg_per_image, batch);
    const size_t bytes = lds * sizeof(float);
    const bool two = cout > 32;
#define VKHIP_WGR(T, NW, CH, D, GM) \
    hipLaunchKernelGGL((win_wgrad_kernel<T, NW, CH, D, GM>), grid, dim3(64 * NW), bytes, ctx().stream, p)
#define VKHIP_WGR_CH(T, GM)                                      \
    do {                                                         \
        static_assert(kWgWaves == 4, "instantiate other wave counts"); \
        if (ch == 8) VKHIP_WGR(T, 4, 8, 4, GM);                  \
        else if (ch == 4) VKHIP_WGR(T, 4, 4, 3, GM);             \
        else if (ch == 2) VKHIP_WGR(T, 4, 2, 2, GM);             \
        else VKHIP_WGR(T, 4, 1, 1, GM);                          \
    } while (0)
    if (pool) {
        if (two) VKHIP_WGR_CH(2, 1); else VKHIP_WGR_CH(1, 1);
    } else {
        if (two) VKHIP_WGR_CH(2, 0); else VKHIP_WGR_CH(1, 0);
    }
#undef VKHIP_WGR_CH
#undef VKHIP_WGR
    VKHIP_LAUNCH_CHECK();
    const uint32_t fold_wgs = (two ? 128u : 64u) + (pool ? 4u : 0u);
    hipLaunchKernelGGL(win_fold_kernel, dim3(fold_wgs), dim3(256), 0, ctx().stream, p.part, p.nwg, out, cout, ck,
                       pool ? p.bpart : nullptr, pool ? pool->bias_out : nullptr);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}


// ---- input gradient of a thin layer ----------------------------------------------
// dX = col2im(flat_weight^T @ grad) (reference: conv2d's backward through the
// im2col node, autograd.cpp:548-553 and ops.cpp:514-541). With C*kh*kw <= 32
// the column matrix has at most 32 rows (27 at CIFAR conv1, 14 MB), and a
// convolution of the gradient with the flipped weight would have C = 3 output
// rows on a 32-row MFMA tile. win_dx_kernel instead computes the columns
// Z = W^T g for the rows of positions a band of dX rows reads (one MFMA tile
// of rows: the window elements; positions in blocks of 32; K = Cout in K-tiles
// of 32 with step t pairing k and 16 + t, the GEMM kernels' chain: Z is the TN
// product's bits) into LDS, and folds them there in col2im's order (for ki,
// for kj, ascending, from 0): dX is the reference lowering's bits, with no 14
// MB column matrix written and read back. The band's halo rows of Z are
// computed by both bands that read them.
namespace {

struct WinDx {
    const float* g;
    int64_t gsn;                // gradient image stride (elements)
    int32_t gsc4;               // gradient channel stride (bytes)
    const float* w;             // flat weight [Cout][K], row stride wrow
    int32_t wrow4;              // (bytes)
    float* out;                 // dX [N][C][H][W] contiguous
    int32_t C, H, W, OH, OW, kh, kw, padh, padw, dilh, dilw;
    uint32_t cout, K, R, zpitch;  // dX rows per workgroup, Z row pitch in LDS (floats)
    FastDiv div_w, div_rw;      // by W, by R * W
};

template <int KT, int NW>
__global__ __launch_bounds__(64 * NW) void win_dx_kernel(WinDx p) {
    extern __shared__ __attribute__((aligned(16))) float zl[];  // [32 window elements][zpitch]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, kh = lane >> 5;
    const uint32_t n = blockIdx.y;
    const int32_t h0 = static_cast<int32_t>(blockIdx.x * p.R);
    const int32_t h1 = min(h0 + static_cast<int32_t>(p.R), p.H);
    // the gradient rows the band's windows reach
    const int32_t zr0 = max(h0 + p.padh - (p.kh - 1) * p.dilh, 0);
    const int32_t zr1 = min(h1 - 1 + p.padh, p.OH - 1);
    const uint32_t zp0 = static_cast<uint32_t>(zr0) * p.OW;
    const uint32_t npos = zr1 >= zr0 ? static_cast<uint32_t>(zr1 - zr0 + 1) * p.OW : 0u;
    const uint32_t nzb = (npos + 31u) / 32u;
    const uint32_t L = static_cast<uint32_t>(p.OH * p.OW);

    // A = W^T: lane (window element lrow, kh) holds W[32kt + t + 16kh][lrow];
    // zero past Cout or K (the GEMM's padding)
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.w), 0, static_cast<int32_t>(0x80000000u), 0x00020000);
    float a[KT][16];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const uint32_t co = 32u * kt + t + 16u * kh;
            const uint32_t off = co < p.cout && static_cast<uint32_t>(lrow) < p.K
                                     ? co * static_cast<uint32_t>(p.wrow4) + 4u * lrow
                                     : 0x80000000u;
            a[kt][t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wr, static_cast<int32_t>(off), 0, 0));
        }
    // B = g: lane (position lrow of the block, kh) holds g[32kt + t + 16kh][p]
    const __amdgpu_buffer_rsrc_t gr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.g + static_cast<int64_t>(n) * p.gsn), 0, static_cast<int32_t>(0x80000000u), 0x00020000);
    auto load_b = [&](uint32_t zb, float (&b)[KT][16]) {
        const uint32_t pos = zp0 + 32u * zb + lrow;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const uint32_t co = 32u * kt + t + 16u * kh;
                const uint32_t off = co < p.cout && pos < L ? co * static_cast<uint32_t>(p.gsc4) + 4u * pos : 0x80000000u;
                b[kt][t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(gr, static_cast<int32_t>(off), 0, 0));
            }
    };
    // Z block zb into LDS: lane (position lrow, kh) holds window element
    // 8(r/4) + 4kh + r%4 in acc[r]
    auto z_block = [&](uint32_t zb, const float (&b)[KT][16]) {
        v16f acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int t = 0; t < 16; ++t) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[kt][t], b[kt][t], acc, 0, 0, 0);
        const uint32_t col = 32u * zb + lrow;
#pragma unroll
        for (int r = 0; r < 16; ++r) zl[(8 * (r / 4) + 4 * kh + r % 4) * p.zpitch + col] = acc[r];
    };
    // blocks wave + NW i: each round loads MB blocks' B, all before the first
    // of their MFMAs (three blocks while they fit the registers of two waves
    // per SIMD)
    constexpr int MB = KT <= 2 ? 3 : 1;
    for (uint32_t zb0 = static_cast<uint32_t>(wave); zb0 < nzb; zb0 += NW * MB) {
        float bs[MB][KT][16];
#pragma unroll
        for (int i = 0; i < MB; ++i)
            if (zb0 + NW * i < nzb) load_b(zb0 + NW * i, bs[i]);
#pragma unroll
        for (int i = 0; i < MB; ++i)
            if (zb0 + NW * i < nzb) z_block(zb0 + NW * i, bs[i]);
    }
    __syncthreads();

    // col2im of the band from LDS: dX[c][h][x] = sum over the window elements
    // that hit it, for ki, for kj, from 0
    // (o walks C x R x W; the last band of an image may hold fewer than R rows)
    const uint32_t rows = static_cast<uint32_t>(h1 - h0), total = static_cast<uint32_t>(p.C) * p.R * p.W;
    for (uint32_t o = static_cast<uint32_t>(tid); o < total; o += 64u * NW) {
        const uint32_t c = p.div_rw.div(o), rem = o - c * p.R * p.W;
        const uint32_t hh = p.div_w.div(rem), x = rem - hh * p.W;
        if (hh >= rows) continue;
        const int32_t h = h0 + static_cast<int32_t>(hh);
        float accv = 0.0f;
        for (int ki = 0; ki < p.kh; ++ki) {
            const int32_t oh = h + p.padh - ki * p.dilh;
            if (oh < 0 || oh >= p.OH) continue;
            const float* zrow = zl + static_cast<uint32_t>((static_cast<int32_t>(c) * p.kh + ki) * p.kw) * p.zpitch +
                                static_cast<uint32_t>(oh) * p.OW - zp0;
            for (int kj = 0; kj < p.kw; ++kj) {
                const int32_t ow = static_cast<int32_t>(x) + p.padw - kj * p.dilw;
                if (ow < 0 || ow >= p.OW) continue;
                accv += zrow[kj * p.zpitch + ow];
            }
        }
        p.out[((static_cast<uint64_t>(n) * p.C + c) * p.H + h) * p.W + x] = accv;
    }
}

// Z row pitch (floats) for npos positions: whole 32-position blocks, then
// 8 mod 16 so that the two half-waves' rows (4 apart) sit on different banks.
uint32_t win_dx_pitch(uint32_t npos) {
    uint32_t pitch = (npos + 31u) / 32u * 32u;
    while (pitch % 16u != 8u) ++pitch;
    return pitch;
}

// dX rows per workgroup: the largest of 16, 8, 4, 2, 1 whose Z band fits the
// LDS and that gives at least 256 workgroups (or 1). (At CIFAR conv1, 16 rows:
// 15.3 us; 8 rows, 512 workgroups, 19.7 us.)
uint32_t win_dx_rows(uint32_t batch, int32_t H, int32_t OH, int32_t OW, int32_t kh, int32_t dilh) {
    for (uint32_t R = 16; R >= 1; R /= 2) {
        const uint32_t zrows = std::min<uint32_t>(R + (kh - 1) * dilh, OH);
        const uint64_t floats = 32ull * win_dx_pitch(zrows * static_cast<uint32_t>(OW));
        const uint64_t wgs = static_cast<uint64_t>(batch) * ((static_cast<uint32_t>(H) + R - 1) / R);
        if (floats <= 24576 && (wgs >= 256 || R == 1)) return R;
    }
    return 0;
}

}  // namespace

bool win_dx_fits(const vkhip_operand& gd, int64_t w_row, const vkhip_unfold& pr, uint32_t batch, uint32_t channels,
                 uint32_t cout, uint32_t oh, uint32_t ow) {
    const uint64_t ck = static_cast<uint64_t>(channels) * pr.kernel_h * pr.kernel_w;
    if (!(pr.stride_h == 1 && pr.stride_w == 1 && ck >= 1 && ck <= 32 && cout >= 1 && cout <= 128 && batch >= 1 &&
          batch <= 65535 && pr.image_h >= 1 && pr.image_w >= 1))
        return false;
    // 32-bit byte offsets within an image's gradient: channel stride x Cout + positions
    const uint64_t L = static_cast<uint64_t>(oh) * ow;
    if (gd.nb[1] < 0 || (static_cast<uint64_t>(cout) - 1) * static_cast<uint64_t>(gd.nb[1]) + L > (1ull << 29))
        return false;
    // and within the weight: row stride x Cout
    if (w_row < 0 || (static_cast<uint64_t>(cout) - 1) * static_cast<uint64_t>(w_row) + ck > (1ull << 29)) return false;
    return win_dx_rows(batch, pr.image_h, static_cast<int32_t>(oh), static_cast<int32_t>(ow), pr.kernel_h,
                       pr.dilation_h) != 0;
}

int win_conv_input_grad(const float* g, const vkhip_operand& gd, const float* w, int64_t w_row, float* out,
                        const vkhip_unfold& pr, uint32_t batch, uint32_t channels, uint32_t cout, uint32_t oh,
                        uint32_t ow) {
    WinDx p{};
    p.g = g;
    p.gsn = gd.nb[0];
    p.gsc4 = static_cast<int32_t>(gd.nb[1] * 4);
    p.w = w;
    p.wrow4 = static_cast<int32_t>(w_row * 4);
    p.out = out;
    p.C = static_cast<int32_t>(channels);
    p.H = pr.image_h;
    p.W = pr.image_w;
    p.OH = static_cast<int32_t>(oh);
    p.OW = static_cast<int32_t>(ow);
    p.kh = pr.kernel_h;
    p.kw = pr.kernel_w;
    p.padh = pr.pad_h;
    p.padw = pr.pad_w;
    p.dilh = pr.dilation_h;
    p.dilw = pr.dilation_w;
    p.cout = cout;
    p.K = channels * pr.kernel_h * pr.kernel_w;
    p.R = win_dx_rows(batch, pr.image_h, p.OH, p.OW, pr.kernel_h, pr.dilation_h);
    if (p.R == 0) return fail(VKHIP_ERR_INVALID, "conv2d input grad: the small-window band does not fit");
    const uint32_t zrows = std::min<uint32_t>(p.R + (pr.kernel_h - 1) * pr.dilation_h, oh);
    p.zpitch = win_dx_pitch(zrows * ow);
    p.div_w = FastDiv(static_cast<uint32_t>(pr.image_w));
    p.div_rw = FastDiv(p.R * static_cast<uint32_t>(pr.image_w));
    const dim3 grid((static_cast<uint32_t>(pr.image_h) + p.R - 1) / p.R, batch);
    const size_t bytes = 32ull * p.zpitch * sizeof(float);
    const uint32_t kt = (cout + 31u) / 32u;
    // eight waves (two per SIMD): 15.3 us at CIFAR conv1, against 19.5 us for four
    if (kt == 1) hipLaunchKernelGGL((win_dx_kernel<1, 8>), grid, dim3(512), bytes, ctx().stream, p);
    else if (kt == 2) hipLaunchKernelGGL((win_dx_kernel<2, 8>), grid, dim3(512), bytes, ctx().stream, p);
    else if (kt == 3) hipLaunchKernelGGL((win_dx_kernel<3, 8>), grid, dim3(512), bytes, ctx().stream, p);
    else hipLaunchKernelGGL((win_dx_kernel<4, 8>), grid, dim3(512), bytes, ctx().stream, p);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}
}  // namespace vkhip
