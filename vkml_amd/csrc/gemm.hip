// fp32 GEMM family on CDNA4 matrix cores: MFMA tiles, split-K with a
// deterministic carry-stack reduce, and a bandwidth GEMV.
//
// Replaces the reference's gemm_naive/gemm_tiled/gemm_reg/gemm_db shaders and
// their selection (reference vulkan_backend.cpp:2056-2657). The reference folds
// K with a per-accumulator carry stack in rounded (no-FMA) arithmetic; matrix
// cores accumulate in hardware order, so GEMM parity with the CPU oracle is
// tolerance-based (normwise, 1e-5*sqrt(K)), while split-K stays bit-stable for
// a fixed split count.
//
// Tile scheme (v_mfma_f32_32x32x2_f32, wave64):
//   - a 256-thread workgroup owns a BM x BN output tile, 4 waves in a 2x2
//     grid, each wave a WM x WN sub-tile of 32x32 MFMA blocks;
//   - both operands are staged in LDS as [row][k] (k contiguous, row pitch
//     BK+4 floats) so every lane reads its MFMA operands as 16-byte
//     ds_read_b128; the +4 pad spreads 8 consecutive rows over distinct banks;
//   - A K-tile is loaded to registers while the previous one is multiplied,
//     then stored to the other LDS buffer: one barrier per K-tile;
//   - inside a K-tile, lane half h (lanes 32..63) supplies k in the upper half
//     of the tile, so each lane's k values are contiguous in LDS. The sum over
//     k is unchanged; only the order MFMA visits the k values differs.
#include "common.h"
#include "conv_small.h"

#include <mutex>
#include <vector>

namespace vkhip {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// An epilogue adds bias[(i % ncols) * bias_stride] to the folded value and
// then applies relu (v <= 0 ? 0 : v) when asked -- the ADD and RELU nodes'
// arithmetic on the product's output -- or (mask != null) takes the relu
// gradient mask[i] <= 0 ? +0 : v, mask laid out as the output (RELU_BACKWARD
// with the product as its incoming gradient; a NaN mask passes v).
struct FoldEpilogue {
    const float* bias;
    int64_t bias_stride;
    uint32_t ncols, relu;
    const float* mask;
};

__device__ __forceinline__ float apply_epilogue(const FoldEpilogue& epi, uint64_t i, float v) {
    if (epi.bias) {
        v = v + epi.bias[static_cast<int64_t>(i % epi.ncols) * epi.bias_stride];
        if (epi.relu) v = v <= 0.0f ? 0.0f : v;
    }
    if (epi.mask && epi.mask[i] <= 0.0f) v = 0.0f;
    return v;
}

struct GemmArgs {
    const float* a;
    const float* b;
    float* c;
    int64_t sa0, sa1, sam, sak;  // A strides: batch0, batch1, m, k (elements)
    int64_t sb0, sb1, sbk, sbn;  // B strides: batch0, batch1, k, n
    uint32_t b1;                 // extent of batch axis 1
    uint32_t m, n, k;
    uint32_t tiles_m, tiles_n;
    uint32_t ktiles;             // ceil(K / BK)
    uint32_t chunk;              // K-tiles per split partition
    uint64_t split_stride;       // elements between partition slices of c
    uint32_t a_vec, b_vec;       // 16-byte loads along k are legal
    uint32_t flat_splits;        // > 0: split grid launched flat, grid.x = tiles * flat_splits
    uint32_t pairs;              // paired direct kernel: partition pairs per tile
    // Convolution epilogue (unsplit register-path conv kernel only): out =
    // acc + bias[row * bias_stride] when bias is set, then relu (x <= 0 ? 0 :
    // x) when relu is set -- the ADD and RELU nodes' arithmetic.
    const float* bias;
    int64_t bias_stride;
    uint32_t relu;
    // A product's epilogue (MATMUL_BIAS, MATMUL_RELU_BACKWARD) applied by the
    // kernel that writes the output (unsplit plans; split plans: the fold).
    FoldEpilogue epi;
};

// The product epilogue at output (z, row, col), when the launch has one.
__device__ __forceinline__ float product_epilogue(const GemmArgs& g, uint32_t z, uint32_t row,
                                                  uint32_t col, float v) {
    if (!g.epi.bias && !g.epi.mask) return v;
    return apply_epilogue(g.epi, (static_cast<uint64_t>(z) * g.m + row) * g.n + col, v);
}

// Output tile (tm, tn) and K partition of this workgroup.
//  - Unsplit grids (blockIdx.x = tile): the hardware deals workgroups to the
//    8 XCDs round-robin, so the tile index is remapped to give each XCD a
//    contiguous tile range, walked in groups of 8 tile-rows for L2 reuse.
//  - Split grids launched flat (flat_splits > 0, grid.x = tiles * partitions):
//    the workgroups one XCD receives (linear id % 8) take a contiguous range
//    of (partition, tile) pairs, so the tiles of one partition, which read the
//    same K slices of A and B, share that XCD's L2 instead of each fetching
//    them from memory.
//  - Otherwise blockIdx.y is the partition.
// Which workgroup computes what never changes what it computes: same bits.
__device__ __forceinline__ void tile_of(const GemmArgs& g, uint32_t& tm, uint32_t& tn,
                                        uint32_t& split) {
    const uint32_t ntiles = g.tiles_m * g.tiles_n;
    uint32_t bid = blockIdx.x;
    split = blockIdx.y;
    if (g.flat_splits) {
        const uint32_t total = ntiles * g.flat_splits;
        const uint32_t xcd = bid & 7u, slot = bid >> 3, q = total >> 3, r = total & 7u;
        const uint32_t v = xcd * q + min(xcd, r) + slot;
        split = v / ntiles;
        bid = v - split * ntiles;
    } else if ((ntiles & 7u) == 0) {
        bid = (bid & 7u) * (ntiles >> 3) + (bid >> 3);
    }
    const uint32_t group_span = 8u * g.tiles_n;
    const uint32_t first_m = (bid / group_span) * 8u;
    const uint32_t gsize = min(g.tiles_m - first_m, 8u);
    tm = first_m + (bid % group_span) % gsize;
    tn = (bid % group_span) / gsize;
}

// Loads one BK-deep tile of an operand (rows x BK) into registers as groups of
// four consecutive k, then stores each group to LDS [row][k] as 16 bytes.
//   KCV  k-contiguous and 16-byte aligned (A in NN, B in NT): lanes walk k
//        first, one 16-byte load per group.
//   RCV  row-contiguous and aligned (B in NN, A in TN): each thread loads a
//        4-row x 4-k block as four 16-byte loads along the rows and transposes
//        it in registers. Lanes walk k-blocks first, so eight lanes fill one
//        128-byte line per k and their LDS stores land on distinct banks.
//   KCS / RCS  any other layout: four 4-byte loads per group, lanes along k
//        (k-contiguous) or along rows.
// GUARD = false is the interior fast path: the whole tile is in range, so no
// per-element bounds checks are emitted.
//   IMG  the B operand of a convolution, gathered from the image (below).
//   IMGT the B operand of a convolution's weight gradient: the transposed
//        cols matrix (k = output positions), gathered from the image.
//   KCD  k-contiguous, 16-byte aligned, K a multiple of 4: loaded straight
//        into LDS by buffer loads (no registers, no LDS stores), rows of BK
//        floats whose 16-byte groups are XOR-swizzled by row (group g of row r
//        at g ^ kcd_swizzle(r)) so the MFMA operand reads stay conflict-free.
//   IMGTB the weight gradient summed over the batch: IMGT with the batch
//        folded into K (k = n * L + position, L a multiple of BK), as B of one
//        product [Cout, N*L] x [N*L, C*kh*kw] (a kernel-level mode: the tile
//        loader is IMGT's, given image n's resource and positions per K-tile).
enum LoadMode { KCV = 0, RCV = 1, KCS = 2, RCS = 3, IMG = 4, IMGT = 5, KCD = 6, IMGTB = 7 };

// The KCD row swizzle. A 16-byte LDS read is served 16 lanes per pass over
// 64 banks (256 bytes); the sixteen rows of a pass (BK = 32 floats = 128
// bytes each) fall on two bank halves by row parity, so the eight rows of one
// parity must take eight distinct groups: bits 1..3 of the row. (Bits 0..2
// gave rows r and r + 8 the same banks: two-way conflicts on every operand
// read, 1/6 of the LDS cycles by SQ_LDS_BANK_CONFLICT.)
__host__ __device__ constexpr int kcd_swizzle(int row) { return (row >> 1) & 7; }

// The byte offset a KCD loader reads for 16-byte slot `slot` of a stage (row
// slot / 8, k-group (slot % 8) ^ kcd_swizzle(row)), or bit 31 (read as 0) for
// a row or k-group past the operand. The loader needs K a multiple of four
// (a group inside K is inside the row) and 16-byte aligned rows.
__host__ __device__ __forceinline__ uint32_t kcd_slot_offset(int slot, int64_t s_row, uint32_t row0,
                                                            uint32_t rows, uint32_t k0, uint32_t kdim) {
    const int r = slot >> 3;
    const uint32_t gr = row0 + r, gk = k0 + 4 * ((slot & 7) ^ kcd_swizzle(r));
    return gr < rows && gk < kdim ? static_cast<uint32_t>((static_cast<int64_t>(gr) * s_row + gk) * 4)
                                  : 0x80000000u;
}

// The B operand of a convolution read straight from the image (implicit
// im2col): element (row, pos) of image n's cols matrix [C*kh*kw, out_h*out_w]
// is x[n, c, h, w] with row = c*kh*kw + ki*kw + kj, pos = oh*out_w + ow,
// h = oh*stride_h - pad_h + ki*dil_h, w = ow*stride_w - pad_w + kj*dil_w, and
// 0 outside the image (kernels_movement.cpp:438-483, the im2col kernel's map).
struct Im2colB {
    const float* x;  // image 0
    int64_t sn;      // image (batch) stride in elements
    // Within one image every offset fits 32 bits (checked by make_im2col).
    int32_t sc, sh, sw;  // channel, row and column strides in elements
    int32_t H, W, kh, kw, kk, strh, strw, padh, padw, dilh, dilw, ow;
    FastDiv div_kk, div_kw, div_ow;  // by kh*kw, kw, out_w
    const int32_t* rows;             // row table (see below)
    uint32_t L, images;              // IMGTB: positions per image, images
    FastDiv div_L;                   // IMGTB: by L
};

// The map splits into a part that depends only on the output position (one
// per lane, fixed for the whole kernel) and a part that depends only on the
// cols row (the same for every lane of a wave in the loader below). Whether
// an element is inside the image depends on the position and on the row's
// window element r = ki*kw + kj only: each position keeps a bit mask over r
// of the elements that fall in the padding.
constexpr int kMaxWindow = 63;  // kh*kw; bit 63 marks rows past K

struct ImgPos {
    int32_t h0, w0;    // top-left image coordinate of the window
    int32_t base;      // its offset (may lie outside the image)
    uint64_t outside;  // bit r set: window element r lies in the padding
};

__host__ __device__ __forceinline__ ImgPos img_pos(const Im2colB& g, uint32_t pos, bool valid) {
    const uint32_t oh = g.div_ow.div(pos);
    const uint32_t ow = pos - oh * static_cast<uint32_t>(g.ow);
    ImgPos p;
    p.h0 = static_cast<int32_t>(oh) * g.strh - g.padh;
    p.w0 = static_cast<int32_t>(ow) * g.strw - g.padw;
    p.base = p.h0 * g.sh + p.w0 * g.sw;
    p.outside = ~0ull;
    if (valid) {
        for (int ki = 0; ki < g.kh; ++ki) {
            const bool row_in = static_cast<uint32_t>(p.h0 + ki * g.dilh) < static_cast<uint32_t>(g.H);
            for (int kj = 0; kj < g.kw; ++kj) {
                const bool in = row_in && static_cast<uint32_t>(p.w0 + kj * g.dilw) <
                                              static_cast<uint32_t>(g.W);
                if (in) p.outside &= ~(1ull << (ki * g.kw + kj));
            }
        }
    }
    return p;
}

// The row part of cols row `row` (channel c, window element ki, kj): its
// offset and its window element.
struct ImgRow {
    int32_t off, r;
};

__host__ __device__ __forceinline__ ImgRow img_row(const Im2colB& g, uint32_t row) {
    const uint32_t c = g.div_kk.div(row);
    const uint32_t r = row - c * static_cast<uint32_t>(g.kk);
    const uint32_t ki = g.div_kw.div(r);
    const uint32_t kj = r - ki * static_cast<uint32_t>(g.kw);
    ImgRow q;
    q.off = static_cast<int32_t>(c) * g.sc + static_cast<int32_t>(ki) * g.dilh * g.sh +
            static_cast<int32_t>(kj) * g.dilw * g.sw;
    q.r = static_cast<int32_t>(r);
    return q;
}

// The gather reads the row part from a table built once per geometry:
// groups of 16 rows as {4*off[16], r[16]} (byte offsets), padded past K with
// rows whose r = 63 is outside for every position, so the loader needs no K
// bound. The table is read through the constant address space: a wave's rows
// are uniform, so these are scalar loads.
constexpr int kRowGroup = 16;
typedef const int32_t __attribute__((address_space(4)))* RowTable;

template <int R, int BK, int MODE>
struct TileLoader {
    static constexpr bool KMAP = MODE == KCV || MODE == KCS || MODE == IMGT;  // lanes walk k first
    static constexpr int kGroups = R * BK / 4;
    static constexpr int kPer = kGroups / 256;
    static_assert(kGroups % 256 == 0, "tile must split evenly over 256 threads");
    static constexpr int kTiles = R * BK / 16;        // 4x4 blocks
    static constexpr int kTPT = (kTiles + 255) / 256;  // blocks per thread
    static constexpr int kRegs = MODE == RCV ? 4 * kTPT : (MODE == KCD ? 1 : kPer);

    __device__ __forceinline__ static void row_kq(int g, int& r, int& kq) {
        if (KMAP) {
            kq = g % (BK / 4);
            r = g / (BK / 4);
        } else {
            r = g % R;
            kq = g / R;
        }
    }

    template <bool GUARD>
    __device__ __forceinline__ static void load(f32x4 (&v)[kRegs], const float* base, int64_t s_row,
                                                int64_t s_k, uint32_t row0, uint32_t rows,
                                                uint32_t k0, uint32_t kdim, int tid) {
        if constexpr (MODE == RCV) {
#pragma unroll
            for (int tt = 0; tt < kTPT; ++tt) {
                const int tile = tid + 256 * tt;
                const bool active = kTiles % 256 == 0 || tile < kTiles;
                const int kg = tile % (BK / 4), mg = active ? tile / (BK / 4) : 0;
                const uint32_t gr0 = row0 + 4 * mg;
                const uint32_t gk0 = k0 + 4 * kg;
                f32x4 c[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float* p = base + static_cast<int64_t>(gk0 + j) * s_k + gr0;
                    if (!GUARD || (active && gr0 + 3 < rows && gk0 + j < kdim)) {
                        c[j] = *reinterpret_cast<const f32x4*>(p);
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            c[j][i] = (active && gr0 + i < rows && gk0 + j < kdim) ? p[i] : 0.0f;
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    f32x4 t;
#pragma unroll
                    for (int j = 0; j < 4; ++j) t[j] = c[j][i];
                    v[4 * tt + i] = t;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                int r, kq;
                row_kq(tid + 256 * i, r, kq);
                const uint32_t gr = row0 + r;
                const uint32_t gk = k0 + 4 * kq;
                const float* p =
                    base + static_cast<int64_t>(gr) * s_row + static_cast<int64_t>(gk) * s_k;
                if (MODE == KCV && (!GUARD || (gr < rows && gk + 3 < kdim))) {
                    v[i] = *reinterpret_cast<const f32x4*>(p);
                } else {
                    f32x4 t;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        t[j] = (!GUARD || (gr < rows && gk + j < kdim)) ? p[j * s_k] : 0.0f;
                    v[i] = t;
                }
            }
        }
    }

    // KCD: R rows x BK k as R*BK/4 16-byte slots; wave w's i-th load fills
    // slots (4i + w)*64 .. +63 of the stage, one per lane, in order (the load
    // writes lane l's 16 bytes at the instruction's LDS base + 16 l). Slot s
    // holds row s / 8, k-group (s % 8) ^ kcd_swizzle(row). Out-of-range groups read
    // an offset past the buffer's range and land as zeros.
    __device__ __forceinline__ static void load_direct(float* stage, __amdgpu_buffer_rsrc_t src,
                                                       int64_t s_row, uint32_t row0, uint32_t rows,
                                                       uint32_t k0, uint32_t kdim, int tid) {
        static_assert(BK == 32 && (R * BK / 4) % 256 == 0, "KCD tile shape");
        constexpr int kLoads = R * BK / 4 / 256;
        const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int chunk = 4 * i + wave;
            const uint32_t off = kcd_slot_offset(chunk * 64 + lane, s_row, row0, rows, k0, kdim);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                src, (__attribute__((address_space(3))) void*)(stage + chunk * 256), 16, off, 0, 0, 0);
        }
    }

    // The A operand of the convolution GEMM (k-contiguous weights, KCV with
    // K a multiple of four, or KCS): out-of-range groups load a clamped
    // in-range address and keep 0, so the loads need no branch and can be
    // scheduled among the MFMAs.
    __device__ __forceinline__ static void load_clamped(f32x4 (&v)[kRegs], const float* base,
                                                        int64_t s_row, uint32_t row0, uint32_t rows,
                                                        uint32_t k0, uint32_t kdim, int tid) {
        static_assert(MODE == KCV || MODE == KCS, "k-contiguous operand");
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            int r, kq;
            row_kq(tid + 256 * i, r, kq);
            const uint32_t gr = row0 + r;
            const uint32_t gk = k0 + 4 * kq;
            const int64_t at = static_cast<int64_t>(gr) * s_row + gk;
            if constexpr (MODE == KCV) {
                const bool ok = gr < rows && gk < kdim;
                const f32x4 t = *reinterpret_cast<const f32x4*>(base + (ok ? at : 0));
#pragma unroll
                for (int j = 0; j < 4; ++j) v[i][j] = ok ? t[j] : 0.0f;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bool ok = gr < rows && gk + j < kdim;
                    const float t = base[ok ? at + j : 0];
                    v[i][j] = ok ? t : 0.0f;
                }
            }
        }
    }

    // IMG: lanes walk output positions, one tile row each (consecutive image
    // addresses for unit stride), and a thread gathers kImgK consecutive k for
    // its position. A wave's k rows are the same for all its lanes: their
    // table entries are scalar loads. Per element a lane adds the row's
    // offset to its position's and sets bit 31 when the element is in the
    // padding; the buffer load returns 0 for such offsets (beyond the
    // resource's 2^31-byte range), so there is no branch and no select. LDS
    // receives the same [row][k] layout as every other mode.
    static constexpr int kImgGroups = 256 / R;
    static constexpr int kImgK = BK / kImgGroups;
    __device__ __forceinline__ static void load_img(f32x4 (&v)[kRegs], __amdgpu_buffer_rsrc_t img,
                                                    RowTable tab, int32_t base4, uint64_t outside,
                                                    uint32_t k0, int tid) {
        static_assert(R % 64 == 0 && kImgK % 4 == 0 && kImgK / 4 == kRegs &&
                          kRowGroup % kImgK == 0, "IMG tile shape");
        const uint32_t kb = k0 + kImgK * __builtin_amdgcn_readfirstlane(tid / R);
        const RowTable t = tab + (kb / kRowGroup) * (2 * kRowGroup) + kb % kRowGroup;
        int32_t off4[kImgK], r[kImgK];
#pragma unroll
        for (int j = 0; j < kImgK; ++j) {
            off4[j] = t[j];
            r[j] = t[kRowGroup + j];
        }
#pragma unroll
        for (int j = 0; j < kImgK; ++j) {
            const uint32_t pad = static_cast<uint32_t>(outside >> r[j]) & 1u;
            const int32_t at = static_cast<int32_t>((pad << 31) | static_cast<uint32_t>(base4 + off4[j]));
            v[j / 4][j % 4] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(img, at, 0, 0));
        }
    }

    // IMGT: element (row r, k = position p) of the transposed cols matrix,
    // for the weight gradient's B operand. Lanes walk k first (a thread owns
    // four consecutive positions, eight threads a 32-position row), each
    // thread keeps kPer fixed rows for the whole kernel: their offsets and
    // displacements are computed once (ImgRows); per K-tile a thread
    // decomposes its four positions, and per element it adds, bounds-checks
    // and loads without branching (bit 31 of a padded element's offset makes
    // the buffer load return 0; so do positions past K and rows past N).
    struct ImgRows {
        int32_t off4[kPer], dh[kPer], dw[kPer];
        bool valid[kPer];
    };
    __device__ __forceinline__ static void img_rows(ImgRows& rs, const Im2colB& im, uint32_t row0,
                                                    uint32_t rows, int tid) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            int r, kq;
            row_kq(tid + 256 * i, r, kq);
            const uint32_t gr = row0 + r;
            rs.valid[i] = gr < rows;
            const ImgRow q = img_row(im, rs.valid[i] ? gr : 0u);
            const uint32_t ki = im.div_kw.div(static_cast<uint32_t>(q.r));
            rs.dh[i] = static_cast<int32_t>(ki) * im.dilh;
            rs.dw[i] = (q.r - static_cast<int32_t>(ki) * im.kw) * im.dilw;
            rs.off4[i] = q.off * 4;
        }
    }
    __device__ __forceinline__ static void load_imgt(f32x4 (&v)[kRegs], __amdgpu_buffer_rsrc_t img,
                                                     const Im2colB& im, const ImgRows& rs,
                                                     uint32_t k0, uint32_t kdim, int tid) {
        static_assert(KMAP && (256 % (BK / 4)) == 0, "IMGT lane map");
        const uint32_t p0 = k0 + 4u * static_cast<uint32_t>(tid % (BK / 4));
        uint32_t oh = im.div_ow.div(p0);
        uint32_t ow = p0 - oh * static_cast<uint32_t>(im.ow);
        int32_t h0[4], w0[4], base4[4];
        bool pv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            pv[j] = p0 + j < kdim;
            h0[j] = static_cast<int32_t>(oh) * im.strh - im.padh;
            w0[j] = static_cast<int32_t>(ow) * im.strw - im.padw;
            base4[j] = (h0[j] * im.sh + w0[j] * im.sw) * 4;
            const bool wrap = ++ow == static_cast<uint32_t>(im.ow);
            ow = wrap ? 0u : ow;
            oh += wrap ? 1u : 0u;
        }
#pragma unroll
        for (int i = 0; i < kPer; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool inside = pv[j] & rs.valid[i] &
                                    (static_cast<uint32_t>(h0[j] + rs.dh[i]) < static_cast<uint32_t>(im.H)) &
                                    (static_cast<uint32_t>(w0[j] + rs.dw[i]) < static_cast<uint32_t>(im.W));
                const uint32_t at = (inside ? 0u : 0x80000000u) |
                                    static_cast<uint32_t>(base4[j] + rs.off4[i]);
                v[i][j] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(img, static_cast<int32_t>(at), 0, 0));
            }
    }

    __device__ __forceinline__ static void store(const f32x4 (&v)[kRegs], float* lds, int tid) {
        if constexpr (MODE == IMG) {
            const int r = tid % R, grp = tid / R;
#pragma unroll
            for (int q = 0; q < kRegs; ++q)
                *reinterpret_cast<f32x4*>(lds + r * (BK + 4) + grp * kImgK + 4 * q) = v[q];
        } else if constexpr (MODE == RCV) {
#pragma unroll
            for (int tt = 0; tt < kTPT; ++tt) {
                const int tile = tid + 256 * tt;
                if (kTiles % 256 == 0 || tile < kTiles) {
                    const int kg = tile % (BK / 4), mg = tile / (BK / 4);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        *reinterpret_cast<f32x4*>(lds + (4 * mg + i) * (BK + 4) + 4 * kg) =
                            v[4 * tt + i];
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                int r, kq;
                row_kq(tid + 256 * i, r, kq);
                *reinterpret_cast<f32x4*>(lds + r * (BK + 4) + 4 * kq) = v[i];
            }
        }
    }
};

// Straight-to-LDS loads with their addresses computed once per kernel. A
// lane's byte offset within the operand is fixed for the whole K loop except
// for the K-tile's part, which is the same for every lane and goes in the
// loads' scalar offset: per load one M0 write and the load. Rows or columns
// past the operand get bit 31 in the fixed offset and read as zeros. The K
// bound is not checked: a last K-tile that K does not fill takes the checked
// loaders (TileLoader::load_direct, load_b_rows_direct, load_rows_direct),
// which fill the same LDS slots.
//   kcd_offsets   KCD slots (k-contiguous rows of BK = 32, swizzled), R rows;
//                 the K-tile part is k0 * 4 bytes.
//   rows_offsets  rows of k, COLS columns each (B in NN, A in TN); the K-tile
//                 part is k0 * s_k * 4 bytes.
template <int R>
__device__ __forceinline__ void kcd_offsets(uint32_t (&vo)[R / 32], int wv, int lane, int64_t s_row,
                                            uint32_t row0, uint32_t rows) {
#pragma unroll
    for (int i = 0; i < R / 32; ++i) vo[i] = kcd_slot_offset((4 * i + wv) * 64 + lane, s_row, row0, rows, 0, ~0u);
}
template <int COLS>
__device__ __forceinline__ void rows_offsets(uint32_t (&vo)[COLS / 32], int wv, int lane, int64_t s_k,
                                             uint32_t col0, uint32_t cols) {
    constexpr int G = COLS / 4;  // 16-byte groups per k row
#pragma unroll
    for (int i = 0; i < COLS / 32; ++i) {
        const int slot = (4 * i + wv) * 64 + lane;
        const uint32_t gc = col0 + 4 * (slot % G);
        vo[i] = gc < cols ? static_cast<uint32_t>(((slot / G) * s_k + gc) * 4) : 0x80000000u;
    }
}
// Issues the loads: load i fills the 64-lane block (4 i + wave) of the stage.
template <int N>
__device__ __forceinline__ void issue_direct(float* stage, __amdgpu_buffer_rsrc_t src, const uint32_t* vo,
                                             int wv, uint32_t soff) {
#pragma unroll
    for (int i = 0; i < N; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            src, (__attribute__((address_space(3))) void*)(stage + (4 * i + wv) * 256), 16, vo[i], soff, 0, 0);
}

template <int BM, int BN, int BK, int WM, int WN, int AMODE, int BMODE>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(GemmArgs g, Im2colB im_in) {
    static_assert((BM / WM) * (BN / WN) == 4, "four waves per workgroup");
    constexpr int LDK = BK + 4;
    constexpr int MI = WM / 32;
    constexpr int NI = WN / 32;
    constexpr int QN = BK / 8;  // groups of four MFMA k-steps per K-tile
    using LA = TileLoader<BM, BK, AMODE>;
    using LB = TileLoader<BN, BK, BMODE == IMGTB ? IMGT : BMODE>;

    __shared__ __attribute__((aligned(16))) float lds[2][(BM + BN) * LDK];
    // the convolution epilogue's bias rows, read before the K loop so their
    // latency hides behind it
    __shared__ float bias_rows[BMODE == IMG ? BM : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm0 = (wave / (BN / WN)) * WM;
    const int wn0 = (wave % (BN / WN)) * WN;

    // Tile order: contiguous tile ranges per XCD (workgroups are dealt to the
    // 8 XCDs round-robin), and within a range, groups of 8 tile-rows so that
    // co-resident tiles share A and B panels in that XCD's L2.
    uint32_t tm, tn, split;
    tile_of(g, tm, tn, split);
    const uint32_t row0 = tm * BM;
    const uint32_t col0 = tn * BN;

    const uint32_t z = blockIdx.z;
    const uint32_t i0 = z / g.b1, i1 = z % g.b1;
    const float* abase = g.a + i0 * g.sa0 + i1 * g.sa1;
    const float* bbase = g.b + i0 * g.sb0 + i1 * g.sb1;
    // Implicit im2col: this image as a buffer resource of 2^31 bytes (loads
    // at offsets with bit 31 set return 0), the row table, and this lane's
    // position.
    const __amdgpu_buffer_rsrc_t arsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(abase), 0, static_cast<int32_t>(0x80000000u), 0x00020000);
    const __amdgpu_buffer_rsrc_t brsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(bbase), 0, static_cast<int32_t>(0x80000000u), 0x00020000);
    const __amdgpu_buffer_rsrc_t img = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(im_in.x + static_cast<int64_t>(z) * im_in.sn), 0,
        static_cast<int32_t>(0x80000000u), 0x00020000);
    RowTable rows = nullptr;
    int32_t base4 = 0;
    uint64_t outside = 0;
    if constexpr (BMODE == IMG) {
        rows = (RowTable)im_in.rows;
        const uint32_t pos = col0 + tid % BN;
        const ImgPos at = img_pos(im_in, pos < g.n ? pos : 0u, pos < g.n);
        base4 = at.base * 4;
        outside = at.outside;
    }
    typename LB::ImgRows trows;
    if constexpr (BMODE == IMGT || BMODE == IMGTB) LB::img_rows(trows, im_in, col0, g.n, tid);
    float* cbase = g.c + static_cast<uint64_t>(split) * g.split_stride +
                   static_cast<uint64_t>(z) * g.m * g.n;

    const uint32_t kt0 = split * g.chunk;
    const uint32_t kt1 = min(g.ktiles, kt0 + g.chunk);
    // Whole tile inside M x N: K-tiles that are also inside K load unguarded.
    const bool rows_in = row0 + BM <= g.m && col0 + BN <= g.n;

    f32x16 acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // KCD operands: offsets computed once (kcd_offsets)
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    uint32_t voa[AMODE == KCD ? BM / 32 : 1], vob[BMODE == KCD ? BN / 32 : 1];
    if constexpr (AMODE == KCD) kcd_offsets<BM>(voa, wv, lane, g.sam, row0, g.m);
    if constexpr (BMODE == KCD) kcd_offsets<BN>(vob, wv, lane, g.sbn, col0, g.n);
    auto a_direct = [&](uint32_t kt, int dst) {
        if constexpr (AMODE == KCD) {
            if ((kt + 1) * BK <= g.k)
                issue_direct<BM / 32>(lds[dst], arsrc, voa, wv, kt * BK * 4);
            else
                LA::load_direct(lds[dst], arsrc, g.sam, row0, g.m, kt * BK, g.k, tid);
        }
    };
    auto b_direct = [&](uint32_t kt, int dst) {
        if constexpr (BMODE == KCD) {
            if ((kt + 1) * BK <= g.k)
                issue_direct<BN / 32>(lds[dst] + BM * LDK, brsrc, vob, wv, kt * BK * 4);
            else
                LB::load_direct(lds[dst] + BM * LDK, brsrc, g.sbn, col0, g.n, kt * BK, g.k, tid);
        }
    };
    f32x4 ra[LA::kRegs], rb[LB::kRegs];
    auto load_tile = [&](uint32_t kt, int dst) {
        (void)dst;
        // (The order matters for the schedule: with A straight into LDS and
        // B through registers, A's loads go first; measured 4% on NN.)
        constexpr bool kImgB = BMODE == IMG || BMODE == IMGT || BMODE == IMGTB;
        if constexpr (AMODE == KCD && BMODE != KCD && !kImgB) {
            a_direct(kt, dst);
            if (rows_in && (kt + 1) * BK <= g.k)
                LB::template load<false>(rb, bbase, g.sbn, g.sbk, col0, g.n, kt * BK, g.k, tid);
            else
                LB::template load<true>(rb, bbase, g.sbn, g.sbk, col0, g.n, kt * BK, g.k, tid);
        } else if constexpr (BMODE == KCD) {
            if constexpr (AMODE == KCD)
                a_direct(kt, dst);
            else if (rows_in && (kt + 1) * BK <= g.k)
                LA::template load<false>(ra, abase, g.sam, g.sak, row0, g.m, kt * BK, g.k, tid);
            else
                LA::template load<true>(ra, abase, g.sam, g.sak, row0, g.m, kt * BK, g.k, tid);
            b_direct(kt, dst);
        } else if constexpr (BMODE == IMG) {
            if constexpr (AMODE == KCD)
                a_direct(kt, dst);
            else
                LA::load_clamped(ra, abase, g.sam, row0, g.m, kt * BK, g.k, tid);
            LB::load_img(rb, img, rows, base4, outside, kt * BK, tid);
        } else if constexpr (BMODE == IMGT) {
            if constexpr (AMODE == KCD)
                a_direct(kt, dst);
            else
                LA::load_clamped(ra, abase, g.sam, row0, g.m, kt * BK, g.k, tid);
            LB::load_imgt(rb, img, im_in, trows, kt * BK, g.k, tid);
        } else if constexpr (BMODE == IMGTB) {
            static_assert(AMODE != KCD, "IMGTB switches image per K-tile: A on the register path");
            // K-tile kt is positions p0 .. p0 + BK - 1 of image n (L is a
            // multiple of BK). The tile after the last, loaded and unused,
            // stays on the last image with positions past L: every load then
            // reads in range or returns 0.
            const uint32_t k0 = kt * BK;
            uint32_t n = im_in.div_L.div(k0);
            n = n < im_in.images ? n : im_in.images - 1u;
            const uint32_t p0 = k0 - n * im_in.L;
            LA::load_clamped(ra, abase + static_cast<int64_t>(n) * g.sa1, g.sam, row0, g.m, p0, im_in.L,
                             tid);
            const __amdgpu_buffer_rsrc_t imgn = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(im_in.x + static_cast<int64_t>(n) * im_in.sn), 0,
                static_cast<int32_t>(0x80000000u), 0x00020000);
            LB::load_imgt(rb, imgn, im_in, trows, p0, im_in.L, tid);
        } else if (rows_in && (kt + 1) * BK <= g.k) {
            LA::template load<false>(ra, abase, g.sam, g.sak, row0, g.m, kt * BK, g.k, tid);
            LB::template load<false>(rb, bbase, g.sbn, g.sbk, col0, g.n, kt * BK, g.k, tid);
        } else {
            LA::template load<true>(ra, abase, g.sam, g.sak, row0, g.m, kt * BK, g.k, tid);
            LB::template load<true>(rb, bbase, g.sbn, g.sbk, col0, g.n, kt * BK, g.k, tid);
        }
    };
    if constexpr (BMODE == IMG) {
        if (g.bias && tid < BM) {
            const uint32_t row = row0 + tid;
            bias_rows[tid] = g.bias[static_cast<int64_t>(row < g.m ? row : 0) * g.bias_stride];
        }
    }
    if (kt0 < kt1) {
        load_tile(kt0, 0);
        if constexpr (AMODE != KCD) LA::store(ra, lds[0], tid);
        if constexpr (BMODE != KCD) LB::store(rb, lds[0] + BM * LDK, tid);
    }
    __syncthreads();

    const int lrow = lane & 31;
    const int kh = lane >> 5;
    const bool single_tile = kt0 + 1 >= kt1;
    for (uint32_t kt = kt0; kt < kt1; ++kt) {
        const int cur = (kt - kt0) & 1;
        const bool more = kt + 1 < kt1;
        // The implicit-im2col loads have no branches: they are issued every
        // iteration (the last one's are in range and unused) so that they sit
        // in the same block as the MFMAs and interleave with them.
        if constexpr (BMODE == IMG || BMODE == IMGT || BMODE == IMGTB) {
            // (A workgroup with a single K-tile -- K <= 32, as a 3-channel
            // 3x3 convolution's 27 -- has no next tile to load or wait for.)
            if (single_tile) {
            } else {
                load_tile(kt + 1, cur ^ 1);
                // Keep every load of the next tile ahead of this tile's MFMAs,
                // so that their latency hides behind all of them.
                __builtin_amdgcn_sched_barrier(0);
            }
        } else if (more) {
            load_tile(kt + 1, cur ^ 1);
        }
        // KCD rows are BK floats with swizzled groups: group kh*4 + q of row
        // r sits at (kh*4 + q) ^ kcd_swizzle(r); rows 32 apart share it.
        constexpr int APITCH = AMODE == KCD ? BK : LDK;
        const float* As = lds[cur] + (wm0 + lrow) * APITCH + (AMODE == KCD ? 0 : kh * (BK / 2));
        auto a_off = [&](int q) {
            return AMODE == KCD ? 4 * ((kh * 4 + q) ^ kcd_swizzle(lrow)) : 4 * q;
        };
        constexpr int BPITCH = BMODE == KCD ? BK : LDK;
        const float* Bs = lds[cur] + BM * LDK + (wn0 + lrow) * BPITCH + (BMODE == KCD ? 0 : kh * (BK / 2));
        auto b_off = [&](int q) {
            return BMODE == KCD ? 4 * ((kh * 4 + q) ^ kcd_swizzle(lrow)) : 4 * q;
        };
        // MFMA operands for step group q+1 are read from LDS while group q's
        // MFMAs run (two register sets).
        f32x4 av[2][MI], bv[2][NI];
#pragma unroll
        for (int i = 0; i < MI; ++i) av[0][i] = *reinterpret_cast<const f32x4*>(As + 32 * i * APITCH + a_off(0));
#pragma unroll
        for (int j = 0; j < NI; ++j) bv[0][j] = *reinterpret_cast<const f32x4*>(Bs + 32 * j * BPITCH + b_off(0));
#pragma unroll
        for (int q = 0; q < QN; ++q) {
            const int cb = q & 1;
            if (q + 1 < QN) {
#pragma unroll
                for (int i = 0; i < MI; ++i)
                    av[cb ^ 1][i] = *reinterpret_cast<const f32x4*>(As + 32 * i * APITCH + a_off(q + 1));
#pragma unroll
                for (int j = 0; j < NI; ++j)
                    bv[cb ^ 1][j] = *reinterpret_cast<const f32x4*>(Bs + 32 * j * BPITCH + b_off(q + 1));
            }
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < NI; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[cb][i][s], bv[cb][j][s],
                                                                         acc[i][j], 0, 0, 0);
            // Spread the next group's LDS reads over this group's MFMAs, one
            // 16-byte read after every MFMA pair; left to itself the compiler
            // bunches them, which exposes LDS latency between MFMA bursts
            // (measured: 110 -> 116 TFLOP/s on NN 4096^3).
            {
                const int reads = (q + 1 < QN) ? (MI + NI) : 0;
#pragma unroll
                for (int r = 0; r < 4 * MI * NI / 2; ++r) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                    if (r < reads) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
            }
        }
        if (more) {
            if constexpr (AMODE != KCD) LA::store(ra, lds[cur ^ 1], tid);
            if constexpr (BMODE != KCD) LB::store(rb, lds[cur ^ 1] + BM * LDK, tid);
        }
        __syncthreads();
    }

    // 32x32 accumulator layout: register r of lane l holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const uint32_t col = col0 + wn0 + 32 * j + lrow;
            // every epilogue load (a mask) before the first store: the
            // compiler cannot tell the output from the mask, and interleaved
            // it waits out one load round trip per store
            float vo[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = row0 + wm0 + 32 * i + 8 * (r / 4) + 4 * kh + (r % 4);
                float v = acc[i][j][r];
                if constexpr (BMODE == IMG) {
                    if (g.bias) v = v + bias_rows[row - row0];
                    if (g.relu) v = v <= 0.0f ? 0.0f : v;
                }
                vo[r] = row < g.m && col < g.n ? product_epilogue(g, z, row, col, v) : v;
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = row0 + wm0 + 32 * i + 8 * (r / 4) + 4 * kh + (r % 4);
                if (row < g.m && col < g.n) {
                    float* at = cbase + static_cast<uint64_t>(row) * g.n + col;
                    // convolution outputs stream past the L2 (non-temporal):
                    // they are read next by another kernel, not by this one
                    if constexpr (BMODE == IMG)
                        __builtin_nontemporal_store(vo[r], at);
                    else
                        *at = vo[r];
                }
            }
        }
}


// ---- NN with both operands straight into LDS ----------------------------------
// A (k-contiguous) lands in LDS as in load mode KCD. B (row-contiguous, NN)
// lands as it lies in memory, BK rows of BN = 128 floats, which the MFMA's B
// operand cannot read as four consecutive k. Instead a lane reads four
// consecutive columns of one k row with one 16-byte LDS read and feeds them to
// four MFMAs, the s-th of which computes the 32 x 32 block of columns
// {4c + s : c < 32}: a wave owns 32 rows x 128 columns as four such strided
// column sets. Each output element still accumulates the same k pairs in the
// same order as the register-path kernel (step (q, st) adds k = 4q + st and
// 16 + 4q + st), so the results are the same bits.
template <int COLS = 128>
__device__ __forceinline__ void load_b_rows_direct(float* stage, __amdgpu_buffer_rsrc_t src,
                                                   int64_t s_k, uint32_t col0, uint32_t cols,
                                                   uint32_t k0, uint32_t kdim, int tid) {
    // 32 k rows x COLS/4 groups of 4 columns = 8 COLS slots, COLS/32 per thread.
    constexpr int G = COLS / 4;
    const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int i = 0; i < COLS / 32; ++i) {
        const int chunk = 4 * i + wave;
        const int slot = chunk * 64 + lane;
        const int r = slot / G, grp = slot % G;
        const uint32_t gk = k0 + r, gc = col0 + 4 * grp;
        const bool ok = gk < kdim && gc < cols;
        const uint32_t off = ok ? static_cast<uint32_t>((static_cast<int64_t>(gk) * s_k + gc) * 4)
                                : 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            src, (__attribute__((address_space(3))) void*)(stage + chunk * 256), 16, off, 0, 0, 0);
    }
}

// ATR (TN): A is row-contiguous too ([k][m] in memory) and lands the same
// way as B, BK rows of 128; a lane reads its row's one float of a k row per
// MFMA step (the rows of a wave are contiguous, so the 32 lanes of a half
// read 32 adjacent floats).
//
// PAIR: two groups of four waves, each with its own LDS double
// buffer, computing the K partitions 2q and 2q+1 of one tile side by side:
// two independent K streams per CU when the grid gives each CU one
// workgroup. Group 1 hands its accumulators to group 0 through LDS and the
// workgroup writes partial(2q) + partial(2q+1), the node the carry-stack fold
// forms first from those two partials (fp addition commutes), so folding the
// g.pairs pair sums gives the bits of folding all the partitions' partials.
// When the partition count is odd the last pair's second group has no K
// range: its sum is the last partial plus +0.0, which folds to the same bits
// (the fold's drain adds the lone last partial to 0.0 first; every later sum
// is the same). With one pair the fold's drain (0.0 + the pair sum) is applied
// here and the result is the output.
//
// BN = 64: 128x64 tiles, a lane's two adjacent columns per k row (one 8-byte
// LDS read) feeding two MFMAs over the column sets {2c + s}. Twice the tiles
// of 128x128, so a grid that gives each CU one 128x128 workgroup gives it
// two independent ones; each output takes the same MFMAs in the same order,
// so the same bits as 128x128.
template <bool ATR, bool PAIR, int BN = 128>
__global__ __launch_bounds__(PAIR ? 512 : 256) void gemm_nn_direct_kernel(GemmArgs g) {
    static_assert(BN == 128 || (BN == 64 && !PAIR), "128x128 tiles, or unpaired 128x64");
    constexpr int BM = 128, BK = 32, LDK = BK + 4, QN = BK / 8;
    constexpr int NS = BN / 32;  // column sets: adjacent columns per lane
    using BV = float __attribute__((ext_vector_type(NS)));
    constexpr int NG = PAIR ? 2 : 1;  // K streams (groups of four waves)
    using LA = TileLoader<BM, BK, KCD>;
    __shared__ __attribute__((aligned(16))) float lds_all[NG][2][BM * LDK + BK * BN];

    const int tid = PAIR ? threadIdx.x & 255 : threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm0 = wave * 32;
    const int grp = PAIR ? __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 8) : 0;
    auto& lds = lds_all[grp];

    uint32_t tm, tn, split;
    tile_of(g, tm, tn, split);
    const uint32_t row0 = tm * BM;
    const uint32_t col0 = tn * BN;
    const uint32_t part = PAIR ? 2 * split + grp : split;  // this group's K partition

    const uint32_t z = blockIdx.z;
    const uint32_t i0 = z / g.b1, i1 = z % g.b1;
    const float* abase = g.a + i0 * g.sa0 + i1 * g.sa1;
    const float* bbase = g.b + i0 * g.sb0 + i1 * g.sb1;
    const __amdgpu_buffer_rsrc_t arsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(abase), 0, static_cast<int32_t>(0x80000000u), 0x00020000);
    const __amdgpu_buffer_rsrc_t brsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(bbase), 0, static_cast<int32_t>(0x80000000u), 0x00020000);
    float* cbase = g.c + static_cast<uint64_t>(split) * g.split_stride +
                   static_cast<uint64_t>(z) * g.m * g.n;
    const uint32_t kt0 = min(g.ktiles, part * g.chunk);
    const uint32_t kt1 = min(g.ktiles, kt0 + g.chunk);
    // Both groups of a pair run the steps of the pair's first (never
    // shorter) partition; a group past its own range only joins the barriers.
    const uint32_t steps = PAIR ? min(g.ktiles - 2 * split * g.chunk, g.chunk) : kt1 - kt0;

    f32x16 acc[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[s][r] = 0.0f;

    // The K-tile's eight straight-to-LDS loads (four of A, four of B) with
    // their offsets computed once (kcd_offsets / rows_offsets).
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    uint32_t voa[4], vob[BN / 32];
    if constexpr (ATR)
        rows_offsets<BM>(voa, wv, lane, g.sak, row0, g.m);
    else
        kcd_offsets<BM>(voa, wv, lane, g.sam, row0, g.m);
    rows_offsets<BN>(vob, wv, lane, g.sbk, col0, g.n);
    const uint32_t a_step = static_cast<uint32_t>((ATR ? g.sak : 1) * BK * 4);
    const uint32_t b_step = static_cast<uint32_t>(g.sbk * BK * 4);
    auto load_tile = [&](uint32_t kt, int dst) {
        if ((kt + 1) * BK > g.k) {
            if constexpr (ATR)
                load_b_rows_direct(lds[dst], arsrc, g.sak, row0, g.m, kt * BK, g.k, tid);
            else
                LA::load_direct(lds[dst], arsrc, g.sam, row0, g.m, kt * BK, g.k, tid);
            load_b_rows_direct<BN>(lds[dst] + BM * LDK, brsrc, g.sbk, col0, g.n, kt * BK, g.k, tid);
            return;
        }
        issue_direct<BM / 32>(lds[dst], arsrc, voa, wv, kt * a_step);
        issue_direct<BN / 32>(lds[dst] + BM * LDK, brsrc, vob, wv, kt * b_step);
    };
    if (kt0 < kt1) load_tile(kt0, 0);
    __syncthreads();

    const int lrow = lane & 31;
    const int kh = lane >> 5;
    for (uint32_t it = 0; it < steps; ++it) {
        const uint32_t kt = kt0 + it;
        if (PAIR && kt >= kt1) {
            __syncthreads();
            continue;
        }
        const int cur = it & 1;
        if (kt + 1 < kt1) load_tile(kt + 1, cur ^ 1);
        const float* As = ATR ? lds[cur] + kh * 16 * BM + wm0 + lrow : lds[cur] + (wm0 + lrow) * BK;
        const float* Bs = lds[cur] + BM * LDK + kh * 16 * BN + NS * lrow;
        auto a_at = [&](int q) {
            if constexpr (ATR) {
                f32x4 v;
#pragma unroll
                for (int st = 0; st < 4; ++st) v[st] = As[(4 * q + st) * BM];
                return v;
            } else {
                return *reinterpret_cast<const f32x4*>(As + 4 * ((kh * 4 + q) ^ kcd_swizzle(lrow)));
            }
        };
        auto b_at = [&](int q, int st) { return *reinterpret_cast<const BV*>(Bs + (4 * q + st) * BN); };
        // (Left to the compiler's scheduler: the MFMA/read interleave the
        // register-path kernel imposes measured 1-3% slower here.)
        f32x4 av[2];
        BV bv[2][4];
        av[0] = a_at(0);
#pragma unroll
        for (int st = 0; st < 4; ++st) bv[0][st] = b_at(0, st);
#pragma unroll
        for (int q = 0; q < QN; ++q) {
            const int cb = q & 1;
            if (q + 1 < QN) {
                av[cb ^ 1] = a_at(q + 1);
#pragma unroll
                for (int st = 0; st < 4; ++st) bv[cb ^ 1][st] = b_at(q + 1, st);
            }
#pragma unroll
            for (int st = 0; st < 4; ++st)
#pragma unroll
                for (int s = 0; s < NS; ++s)
                    acc[s] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[cb][st], bv[cb][st][s], acc[s],
                                                                  0, 0, 0);
        }
        __syncthreads();
    }

    if constexpr (PAIR) {
        // Group 1's accumulators through its own (now idle) LDS stages, one
        // float per lane per register, lanes consecutive: no bank conflicts.
        float* xch = &lds_all[1][0][0];
        const int wv4 = __builtin_amdgcn_readfirstlane(wave);
        if (grp == 1) {
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int r = 0; r < 16; ++r) xch[((wv4 * 4 + s) * 16 + r) * 64 + lane] = acc[s][r];
        }
        __syncthreads();
        if (grp == 1) return;
        const bool final = g.pairs == 1;
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float v = acc[s][r] + xch[((wv4 * 4 + s) * 16 + r) * 64 + lane];
                acc[s][r] = final ? 0.0f + v : v;
            }
    }

    // acc[s] register r of lane l: row 8*(r/4) + 4*(l/32) + r%4 of the wave's
    // 32, column NS*(l%32) + s of the tile: a lane's NS columns are adjacent
    // (N is a multiple of four, so they are in or out together).
    const uint32_t col = col0 + NS * lrow;
    if (col < g.n) {
        // the epilogue's loads (a mask) before the first store (see
        // gemm_mfma_kernel)
        BV vo[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t row = row0 + wm0 + 8 * (r / 4) + 4 * kh + (r % 4);
#pragma unroll
            for (int s = 0; s < NS; ++s)
                vo[r][s] = row < g.m ? product_epilogue(g, z, row, col + s, acc[s][r]) : acc[s][r];
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t row = row0 + wm0 + 8 * (r / 4) + 4 * kh + (r % 4);
            // streamed past the L2 (non-temporal): outputs and split-K
            // partials are read by later kernels, never by this one
            if (row < g.m)
                __builtin_nontemporal_store(vo[r], reinterpret_cast<BV*>(cbase + static_cast<uint64_t>(row) * g.n + col));
        }
    }
}

// The weight-gradient gather's address arithmetic (conv_direct_kernel), also
// built for the host so tests replay it (vkhip_im2col_offset_t). Column j of
// the transposed columns (a window row: channel, window element) contributes
// a fixed offset and displacement; a position contributes the window's origin;
// an element is inside when both displacements land in the image.
struct GatherCol {
    int32_t fo4, fh, fw;  // 4 * offset, row and column displacement
    bool ok;              // j < C*kh*kw
};
__host__ __device__ __forceinline__ GatherCol gather_col(const Im2colB& im, uint32_t j, uint32_t ncols) {
    GatherCol c;
    c.ok = j < ncols;
    const ImgRow q = img_row(im, c.ok ? j : 0u);
    const uint32_t ki = im.div_kw.div(static_cast<uint32_t>(q.r));
    c.fh = static_cast<int32_t>(ki) * im.dilh;
    c.fw = (q.r - static_cast<int32_t>(ki) * im.kw) * im.dilw;
    c.fo4 = q.off * 4;
    return c;
}
struct GatherPos {
    int32_t sh, sw, so4;  // window origin row, column and 4 * its offset
};
__host__ __device__ __forceinline__ GatherPos gather_pos(const Im2colB& im, uint32_t oh, uint32_t ow) {
    GatherPos q;
    q.sh = static_cast<int32_t>(oh) * im.strh - im.padh;
    q.sw = static_cast<int32_t>(ow) * im.strw - im.padw;
    q.so4 = (q.sh * im.sh + q.sw * im.sw) * 4;
    return q;
}
// byte offset of the element in the image, or bit 31 (read as 0)
__host__ __device__ __forceinline__ uint32_t gather_offset(const Im2colB& im, const GatherCol& c,
                                                           int32_t sh, int32_t sw, int32_t so4, bool kok) {
    const bool inside = kok & c.ok & (static_cast<uint32_t>(sh + c.fh) < static_cast<uint32_t>(im.H)) &
                        (static_cast<uint32_t>(sw + c.fw) < static_cast<uint32_t>(im.W));
    return inside ? static_cast<uint32_t>(so4) + static_cast<uint32_t>(c.fo4) : 0x80000000u;
}

// The convolution weight gradient's products with both operands straight into
// LDS, in gemm_nn_direct_kernel's layouts (A KCD-swizzled [128 rows][32 k],
// B [32 k][128 columns]) and MFMA order, so the same bits as that kernel on
// the materialised columns:
//   CD_WGRAD      out[n] = grad[n] (Cout x L) @ cols(x[n])^T: k = position p,
//                 B column = window row j (channel, window element).
//   CD_WGRAD_FOLD the same summed over n, one product with K = N*L (L a
//                 multiple of 32, so each K-tile lies in image kt*32 / L).
// A is the gradient rows of one image, k-contiguous. B is gathered by
// single-float LDS-direct loads: row k of a K-tile is one position for the
// whole wave, so one load brings 64 consecutive B columns (one per lane) of
// it. An element is x[n][c][h][w] at h = sh_k + fh_lane, w = sw_k + fw_lane,
// offset so_k + fo_lane: the position part is scalar, the window-row part
// fixed for the kernel (a lane owns two columns), both from the im2col map
// (kernels_movement.cpp:438-483). Padding, columns past N and positions past
// L read at an offset with bit 31 set, which the 2^31-byte buffer resource
// returns as 0. (The forward's B operand gathered this way -- k = window row,
// a lane owning two positions -- measured slower than the register-path
// IMG loader: [128,64,32,32] -> 128 channels 0.199 -> 0.215 ms.)
enum ConvDirect { CD_WGRAD = 1, CD_WGRAD_FOLD = 2 };

template <int CD, int BN = 128>
__global__ __launch_bounds__(256) void conv_direct_kernel(GemmArgs g, Im2colB im) {
    static_assert(BN == 128 || BN == 64, "128x128 or 128x64 tiles");
    constexpr int BM = 128, BK = 32, LDK = BK + 4, QN = BK / 8;
    constexpr int NS = BN / 32;  // column sets: adjacent columns per lane
    constexpr int NH = BN / 64;  // gathered B columns per lane
    using BV = float __attribute__((ext_vector_type(NS)));
    using LA = TileLoader<BM, BK, KCD>;
    __shared__ __attribute__((aligned(16))) float lds[2][BM * LDK + BK * BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm0 = wave * 32;

    uint32_t tm, tn, split;
    tile_of(g, tm, tn, split);
    const uint32_t row0 = tm * BM;
    const uint32_t col0 = tn * BN;
    const uint32_t z = blockIdx.z;
    float* cbase = g.c + static_cast<uint64_t>(split) * g.split_stride +
                   static_cast<uint64_t>(z) * g.m * g.n;
    const uint32_t kt0 = split * g.chunk;
    const uint32_t kt1 = min(g.ktiles, kt0 + g.chunk);
    // K of one image (A's k extent per image)
    const uint32_t kimg = CD == CD_WGRAD_FOLD ? im.L : g.k;

    // this lane's B columns j = col0 + 64 h + lane: channel and window element
    GatherCol col_of[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) col_of[h] = gather_col(im, col0 + 64 * h + lane, g.n);

    uint32_t voa[BM / 32];
    kcd_offsets<BM>(voa, wave, lane, g.sam, row0, g.m);

    f32x16 acc[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[s][r] = 0.0f;

    auto load_tile = [&](uint32_t kt, int dst) {
        const uint32_t k0 = kt * BK;
        // one B row of the K-tile: its scalar part, then the two loads
        auto gather_row = [&](__amdgpu_buffer_rsrc_t img, int rr, bool kok, int32_t sh_k, int32_t sw_k,
                              int32_t so4_k) {
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const uint32_t off = gather_offset(im, col_of[h], sh_k, sw_k, so4_k, kok);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    img,
                    (__attribute__((address_space(3))) void*)(lds[dst] + BM * LDK + (8 * wave + rr) * BN +
                                                              64 * h),
                    4, off, 0, 0, 0);
            }
        };
        {
            uint32_t n = z, p0 = k0;
            if constexpr (CD == CD_WGRAD_FOLD) {
                n = im.div_L.div(k0);
                p0 = k0 - n * kimg;
            }
            const __amdgpu_buffer_rsrc_t arsrc = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(g.a + static_cast<int64_t>(n) * g.sa1), 0,
                static_cast<int32_t>(0x80000000u), 0x00020000);
            if (p0 + BK <= kimg)
                issue_direct<BM / 32>(lds[dst], arsrc, voa, wave, p0 * 4);
            else
                LA::load_direct(lds[dst], arsrc, g.sam, row0, g.m, p0, kimg, tid);
            const __amdgpu_buffer_rsrc_t img = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(im.x + static_cast<int64_t>(n) * im.sn), 0,
                static_cast<int32_t>(0x80000000u), 0x00020000);
            // wave w gathers positions p0 + 8w .. + 7, walked incrementally
            uint32_t p = p0 + 8 * wave;
            uint32_t oh = im.div_ow.div(p);
            uint32_t ow = p - oh * static_cast<uint32_t>(im.ow);
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) {
                const GatherPos q = gather_pos(im, oh, ow);
                gather_row(img, rr, p < kimg, q.sh, q.sw, q.so4);
                ++p;
                ++ow;
                const bool wrap = ow == static_cast<uint32_t>(im.ow);
                ow = wrap ? 0u : ow;
                oh += wrap ? 1u : 0u;
            }
        }
    };
    if (kt0 < kt1) load_tile(kt0, 0);
    __syncthreads();

    const int lrow = lane & 31;
    const int kh = lane >> 5;
    for (uint32_t kt = kt0; kt < kt1; ++kt) {
        const int cur = (kt - kt0) & 1;
        if (kt + 1 < kt1) load_tile(kt + 1, cur ^ 1);
        const float* As = lds[cur] + (wm0 + lrow) * BK;
        const float* Bs = lds[cur] + BM * LDK + kh * 16 * BN + NS * lrow;
        auto a_at = [&](int q) {
            return *reinterpret_cast<const f32x4*>(As + 4 * ((kh * 4 + q) ^ kcd_swizzle(lrow)));
        };
        auto b_at = [&](int q, int st) { return *reinterpret_cast<const BV*>(Bs + (4 * q + st) * BN); };
        f32x4 av[2];
        BV bv[2][4];
        av[0] = a_at(0);
#pragma unroll
        for (int st = 0; st < 4; ++st) bv[0][st] = b_at(0, st);
#pragma unroll
        for (int q = 0; q < QN; ++q) {
            const int cb = q & 1;
            if (q + 1 < QN) {
                av[cb ^ 1] = a_at(q + 1);
#pragma unroll
                for (int st = 0; st < 4; ++st) bv[cb ^ 1][st] = b_at(q + 1, st);
            }
#pragma unroll
            for (int st = 0; st < 4; ++st)
#pragma unroll
                for (int s = 0; s < NS; ++s)
                    acc[s] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[cb][st], bv[cb][st][s], acc[s],
                                                                  0, 0, 0);
        }
        __syncthreads();
    }

    const uint32_t col = col0 + NS * lrow;
    if (col < g.n) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t row = row0 + wm0 + 8 * (r / 4) + 4 * kh + (r % 4);
            if (row < g.m) {
                BV v;
#pragma unroll
                for (int s = 0; s < NS; ++s) v[s] = acc[s][r];
                if (g.n % NS == 0) {
                    *reinterpret_cast<BV*>(cbase + static_cast<uint64_t>(row) * g.n + col) = v;
                } else {
#pragma unroll
                    for (int s = 0; s < NS; ++s)
                        if (col + s < g.n) cbase[static_cast<uint64_t>(row) * g.n + col + s] = v[s];
                }
            }
        }
    }
}

// 64x64 tiles with both operands straight into LDS, for outputs that give
// each CU only a workgroup or two of 64x64 tiles. Rows of k (B, and A in TN)
// land as 32 rows of 64 floats; A in NN lands KCD-swizzled. Four waves: two
// row groups of 32 x two strided column sets {2c + s}, one MFMA chain each,
// a lane reading one float of a k row per step. Same k order per output as
// the register-path 64x64 kernel, so the same bits.
template <int COLS>
__device__ __forceinline__ void load_rows_direct(float* stage, __amdgpu_buffer_rsrc_t src, int64_t s_k,
                                                 uint32_t col0, uint32_t cols, uint32_t k0,
                                                 uint32_t kdim, int tid) {
    constexpr int G = COLS / 4;  // 16-byte groups per k row
    const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int i = 0; i < 32 * G / 256; ++i) {
        const int chunk = 4 * i + wave;
        const int slot = chunk * 64 + lane;
        const int r = slot / G, grp = slot % G;
        const uint32_t gk = k0 + r, gc = col0 + 4 * grp;
        const bool ok = gk < kdim && gc < cols;
        const uint32_t off = ok ? static_cast<uint32_t>((static_cast<int64_t>(gk) * s_k + gc) * 4)
                                : 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            src, (__attribute__((address_space(3))) void*)(stage + chunk * 256), 16, off, 0, 0, 0);
    }
}

//
// G K-tiles per stage: the loads of the next stage are issued before the
// current stage's MFMAs and complete at the barrier that ends it, so a stage
// of G = 4 (64 MFMAs per wave, 128 KB of LDS for the two stages) covers the
// memory latency that a single K-tile (16 MFMAs) leaves exposed at one
// workgroup per CU. The tiles of a stage run in K order: the same chain, the
// same bits for every G.
template <bool ATR, int G>
__global__ __launch_bounds__(256) void gemm_direct64_kernel(GemmArgs g) {
    constexpr int BM = 64, BN = 64, BK = 32, QN = BK / 8, TILE = BM * BK + BK * BN;
    using LA = TileLoader<BM, BK, KCD>;
    __shared__ __attribute__((aligned(16))) float lds[2][G * TILE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm0 = (wave & 1) * 32;
    const int s0 = wave >> 1;

    uint32_t tm, tn, split;
    tile_of(g, tm, tn, split);
    const uint32_t row0 = tm * BM;
    const uint32_t col0 = tn * BN;

    const uint32_t z = blockIdx.z;
    const uint32_t i0 = z / g.b1, i1 = z % g.b1;
    const float* abase = g.a + i0 * g.sa0 + i1 * g.sa1;
    const float* bbase = g.b + i0 * g.sb0 + i1 * g.sb1;
    const __amdgpu_buffer_rsrc_t arsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(abase), 0, static_cast<int32_t>(0x80000000u), 0x00020000);
    const __amdgpu_buffer_rsrc_t brsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(bbase), 0, static_cast<int32_t>(0x80000000u), 0x00020000);
    float* cbase = g.c + static_cast<uint64_t>(split) * g.split_stride +
                   static_cast<uint64_t>(z) * g.m * g.n;
    const uint32_t kt0 = split * g.chunk;
    const uint32_t kt1 = min(g.ktiles, kt0 + g.chunk);

    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;

    const int wv = __builtin_amdgcn_readfirstlane(wave);
    uint32_t voa[2], vob[2];
    if constexpr (ATR)
        rows_offsets<BM>(voa, wv, lane, g.sak, row0, g.m);
    else
        kcd_offsets<BM>(voa, wv, lane, g.sam, row0, g.m);
    rows_offsets<BN>(vob, wv, lane, g.sbk, col0, g.n);
    const uint32_t a_step = static_cast<uint32_t>((ATR ? g.sak : 1) * BK * 4);
    const uint32_t b_step = static_cast<uint32_t>(g.sbk * BK * 4);
    auto load_tile = [&](uint32_t kt, float* dst) {
        if ((kt + 1) * BK > g.k) {
            if constexpr (ATR)
                load_rows_direct<BM>(dst, arsrc, g.sak, row0, g.m, kt * BK, g.k, tid);
            else
                LA::load_direct(dst, arsrc, g.sam, row0, g.m, kt * BK, g.k, tid);
            load_rows_direct<BN>(dst + BM * BK, brsrc, g.sbk, col0, g.n, kt * BK, g.k, tid);
            return;
        }
        issue_direct<BM / 32>(dst, arsrc, voa, wv, kt * a_step);
        issue_direct<BN / 32>(dst + BM * BK, brsrc, vob, wv, kt * b_step);
    };
    auto load_stage = [&](uint32_t kt, int buf) {
#pragma unroll
        for (int j = 0; j < G; ++j)
            if (kt + j < kt1) load_tile(kt + j, lds[buf] + j * TILE);
    };
    if (kt0 < kt1) load_stage(kt0, 0);
    __syncthreads();

    const int lrow = lane & 31;
    const int kh = lane >> 5;
    for (uint32_t kt = kt0; kt < kt1; kt += G) {
        const int cur = ((kt - kt0) / G) & 1;
        if (kt + G < kt1) load_stage(kt + G, cur ^ 1);
#pragma unroll
        for (int j = 0; j < G; ++j) {
            if (j > 0 && kt + j >= kt1) break;
            const float* tl = lds[cur] + j * TILE;
            const float* As = ATR ? tl + kh * 16 * BM + wm0 + lrow : tl + (wm0 + lrow) * BK;
            const float* Bs = tl + BM * BK + kh * 16 * BN + 2 * lrow + s0;
            auto a_at = [&](int q) {
                if constexpr (ATR) {
                    f32x4 v;
#pragma unroll
                    for (int st = 0; st < 4; ++st) v[st] = As[(4 * q + st) * BM];
                    return v;
                } else {
                    return *reinterpret_cast<const f32x4*>(As + 4 * ((kh * 4 + q) ^ kcd_swizzle(lrow)));
                }
            };
            f32x4 av[2], bv[2];
            av[0] = a_at(0);
#pragma unroll
            for (int st = 0; st < 4; ++st) bv[0][st] = Bs[st * BN];
#pragma unroll
            for (int q = 0; q < QN; ++q) {
                const int cb = q & 1;
                if (q + 1 < QN) {
                    av[cb ^ 1] = a_at(q + 1);
#pragma unroll
                    for (int st = 0; st < 4; ++st) bv[cb ^ 1][st] = Bs[(4 * (q + 1) + st) * BN];
                }
#pragma unroll
                for (int st = 0; st < 4; ++st)
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[cb][st], bv[cb][st], acc, 0, 0, 0);
            }
        }
        __syncthreads();
    }

    // acc register r of lane l: row 8*(r/4) + 4*(l/32) + r%4 of the wave's 32,
    // column 2*(l%32) + s0 of the tile.
    const uint32_t col = col0 + 2 * lrow + s0;
    if (col < g.n) {
        // the epilogue's loads (a mask) before the first store (see
        // gemm_mfma_kernel)
        float vo[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t row = row0 + wm0 + 8 * (r / 4) + 4 * kh + (r % 4);
            vo[r] = row < g.m ? product_epilogue(g, z, row, col, acc[r]) : acc[r];
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t row = row0 + wm0 + 8 * (r / 4) + 4 * kh + (r % 4);
            if (row < g.m) cbase[static_cast<uint64_t>(row) * g.n + col] = vo[r];
        }
    }
}

// ---- split-K partial fold --------------------------------------------------
// Per output: the binary-counter carry stack over the `splits` partial slices,
// drained in ascending level order from 0.0 (reference
// gemm_split_k_reduce.comp:48-85). Unrolled over a fixed number of levels so
// the stack lives in registers.
constexpr int kSplitLevels = 9;  // up to 511 partitions

// Push of one value onto a carry stack of `count` earlier pushes.
__device__ __forceinline__ void carry_push(float (&stack)[kSplitLevels], uint32_t count, float block) {
    bool carry = true;
#pragma unroll
    for (int l = 0; l < kSplitLevels; ++l) {
        if (carry) {
            if ((count >> l) & 1u) {
                block = block + stack[l];
            } else {
                stack[l] = block;
                carry = false;
            }
        }
    }
}

// G thread groups per block of 256 / G consecutive outputs. The host picks the
// chunk C, the smallest power of two with ceil(splits / C) <= G. Groups
// g < nchunks = splits / C fold the consecutive partials [g*C, (g+1)*C),
// which the carry stack leaves as one balanced subtree at level log2(C);
// group nchunks folds the rem = splits % C trailing partials into a carry
// stack of levels below log2(C) and drains it (0.0 + its lowest level + ...).
// The drain of the whole stack takes those low levels first, so group 0
// continues that total with the carry stack of the nchunks chunk values,
// whose levels are log2(C) and up: the same association as one thread
// pushing all partials and draining from 0.0. With C a template constant
// every push position is known at compile time, so the pushes compile to
// straight-line adds. Partials are read eight at a time so the loads overlap;
// outputs are consecutive across the lanes of a group, so loads coalesce.
// (Measured on 64 x 65536 partials: 8 groups 3.0 us; 16 groups 4.4 us and 32
// groups 11.9 us, where group 0's combine grows; 16-byte loads of four
// outputs per lane 3.75 us.)
template <int G, int C>
__global__ __launch_bounds__(256) void split_k_reduce_kernel(const float* __restrict__ ws,
                                                             float* __restrict__ dst, uint64_t ne,
                                                             uint32_t splits, uint32_t nchunks,
                                                             FoldEpilogue epi) {
    constexpr int kOuts = 256 / G;
    constexpr int kChunkLevel = C >= 64 ? 6 : C >= 32 ? 5 : C >= 16 ? 4 : C >= 8 ? 3 : C >= 4 ? 2 : C >= 2 ? 1 : 0;
    static_assert((1 << kChunkLevel) == C && kChunkLevel < kSplitLevels, "chunk is a power of two");
    __shared__ float part[G][kOuts];
    const int g = threadIdx.x / kOuts, o = threadIdx.x % kOuts;
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * kOuts + o;
    const bool live = i < ne;
    const uint32_t rem = splits - nchunks * C;
    const bool chunk = static_cast<uint32_t>(g) < nchunks;
    float val = 0.0f;
    if (live && (chunk || (static_cast<uint32_t>(g) == nchunks && rem != 0))) {
        const uint32_t count = chunk ? C : rem;
        const float* src = ws + static_cast<uint64_t>(g) * C * ne + i;
        float stack[kSplitLevels];
#pragma unroll
        for (int l = 0; l < kSplitLevels; ++l) stack[l] = 0.0f;
#pragma unroll
        for (int s0 = 0; s0 < C; s0 += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8 && s0 + j < C; ++j)
                if (static_cast<uint32_t>(s0 + j) < count) v[j] = src[static_cast<uint64_t>(s0 + j) * ne];
#pragma unroll
            for (int j = 0; j < 8 && s0 + j < C; ++j)
                if (static_cast<uint32_t>(s0 + j) < count) carry_push(stack, s0 + j, v[j]);
        }
        if (chunk) {
            val = stack[kChunkLevel];
        } else {
#pragma unroll
            for (int l = 0; l < kChunkLevel; ++l)
                if ((rem >> l) & 1u) val = val + stack[l];
        }
    }
    part[g][o] = val;
    __syncthreads();
    if (g != 0 || !live) return;
    // The remainder's drained total (0.0 when rem == 0) continues with the
    // chunk values' carry stack, drained from its lowest level.
    float total = rem != 0 ? part[nchunks][o] : 0.0f;
    float chunks[kSplitLevels];
#pragma unroll
    for (int l = 0; l < kSplitLevels; ++l) chunks[l] = 0.0f;
#pragma unroll
    for (int j = 0; j < G; ++j)
        if (static_cast<uint32_t>(j) < nchunks) carry_push(chunks, j, part[j][o]);
#pragma unroll
    for (int l = 0; l < kSplitLevels; ++l)
        if ((nchunks >> l) & 1u) total = total + chunks[l];
    dst[i] = apply_epilogue(epi, i, total);
}

// The same epilogue over an unsplit product's output, in place.
__global__ __launch_bounds__(256) void bias_cols_kernel(float* __restrict__ c, uint64_t ne,
                                                        FoldEpilogue epi) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= ne) return;
    c[i] = apply_epilogue(epi, i, c[i]);
}

// ---- split-K products folded inside the workgroup ----------------------------
// A product whose plan splits K into S = 2..4 partitions (512^3: 4 of 4
// K-tiles; a Linear(256, 100) layer at batch 128: 4 of 2) ran as the split
// kernel writing S partial slices and split_k_reduce_kernel folding them: two
// launches, the second bound by its launch and the partials' round trip
// (10.4 us at 512^3 for 1.7 us of matrix-core work). Here a workgroup owns a
// 32 x 32 output tile and one wave per partition: wave p stages its own
// K-tiles [p*chunk, min((p+1)*chunk, ktiles)) in LDS (its K-slices of A and
// B, zero outside the operands, with waits within the wave only) and runs the
// 16 MFMA steps per K-tile that every kernel here runs (step t pairs k = t and
// k = 16 + t), from 0, so its partial is the split kernel's. The S partials
// then go through LDS and are folded per output exactly as the fold kernel
// folds them (carry stack in partition order, drained from 0.0), with the
// same epilogue: the product's bits, in one launch.
constexpr int kWgFoldLdk = 33;  // LDS pitch of a staged 32 x 32 slice

template <int S, int KT>
__global__ __launch_bounds__(64 * S) void gemm_wgfold_kernel(GemmArgs g, FoldEpilogue epi, int a_kfast,
                                                             int b_kfast) {
    // KT: K-tiles per partition, all of whose operand slices a wave loads
    // into registers before its first MFMA (16-byte loads for a k-contiguous
    // A and an n-contiguous B, the NN layout; elements otherwise)
    __shared__ float stage[S][2][32 * kWgFoldLdk];  // per wave: A [row][k], B [col][k]
    __shared__ float parts[S][16][64];
    const int lane = threadIdx.x & 63;
    const int p = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lrow = lane & 31, kh = lane >> 5;
    const uint32_t tm = blockIdx.x / g.tiles_n, tn = blockIdx.x - tm * g.tiles_n;
    const uint32_t row0 = 32u * tm, col0 = 32u * tn;
    const uint32_t z = blockIdx.z;
    const uint32_t i0 = z / g.b1, i1 = z - i0 * g.b1;
    const float* a = g.a + static_cast<int64_t>(i0) * g.sa0 + static_cast<int64_t>(i1) * g.sa1;
    const float* b = g.b + static_cast<int64_t>(i0) * g.sb0 + static_cast<int64_t>(i1) * g.sb1;
    float* As = stage[p][0];
    float* Bs = stage[p][1];
    const uint32_t kt0 = static_cast<uint32_t>(p) * g.chunk;
    const uint32_t kt1 = min(g.ktiles, kt0 + g.chunk);
    // the vector path: lane l loads row/k-row l/8 + 8q, 4 floats at 4*(l%8)
    const bool vec = g.a_vec && g.b_vec && g.sak == 1 && g.sbn == 1;
    float va[KT][16], vb[KT][16];
#pragma unroll
    for (int u = 0; u < KT; ++u) {
        const uint32_t k0 = 32u * (kt0 + u);
        const bool live = kt0 + u < kt1;
        if (vec) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t rr = static_cast<uint32_t>(lane / 8 + 8 * q), c4 = 4u * (lane % 8);
                const uint32_t gr = row0 + rr, gk = k0 + c4;
                f32x4 x = {0.0f, 0.0f, 0.0f, 0.0f};
                if (live && gr < g.m && gk + 3 < g.k)
                    x = *reinterpret_cast<const f32x4*>(a + static_cast<int64_t>(gr) * g.sam + gk);
                else if (live && gr < g.m)
                    for (int j = 0; j < 4; ++j)
                        if (gk + j < g.k) x[j] = a[static_cast<int64_t>(gr) * g.sam + gk + j];
                const uint32_t gbk = k0 + rr, gc = col0 + c4;
                f32x4 y = {0.0f, 0.0f, 0.0f, 0.0f};
                if (live && gbk < g.k && gc + 3 < g.n)
                    y = *reinterpret_cast<const f32x4*>(b + static_cast<int64_t>(gbk) * g.sbk + gc);
                else if (live && gbk < g.k)
                    for (int j = 0; j < 4; ++j)
                        if (gc + j < g.n) y[j] = b[static_cast<int64_t>(gbk) * g.sbk + gc + j];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    va[u][4 * q + j] = x[j];
                    vb[u][4 * q + j] = y[j];
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t rr = a_kfast ? static_cast<uint32_t>(2 * i + kh) : static_cast<uint32_t>(lrow);
                const uint32_t kk = a_kfast ? static_cast<uint32_t>(lrow) : static_cast<uint32_t>(2 * i + kh);
                const uint32_t gr = row0 + rr, gk = k0 + kk;
                va[u][i] = (live && gr < g.m && gk < g.k)
                               ? a[static_cast<int64_t>(gr) * g.sam + static_cast<int64_t>(gk) * g.sak]
                               : 0.0f;
                const uint32_t cc = b_kfast ? static_cast<uint32_t>(2 * i + kh) : static_cast<uint32_t>(lrow);
                const uint32_t bk = b_kfast ? static_cast<uint32_t>(lrow) : static_cast<uint32_t>(2 * i + kh);
                const uint32_t gc = col0 + cc, gbk = k0 + bk;
                vb[u][i] = (live && gc < g.n && gbk < g.k)
                               ? b[static_cast<int64_t>(gbk) * g.sbk + static_cast<int64_t>(gc) * g.sbn]
                               : 0.0f;
            }
        }
    }
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int u = 0; u < KT; ++u) {
        if (kt0 + u >= kt1) break;
        // (a wave's LDS operations complete in issue order; the fences keep
        // the compiler from moving this K-tile's stores above the previous
        // K-tile's reads, or its reads above these stores)
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
        if (vec) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int rr = lane / 8 + 8 * q, c = 4 * (lane % 8) + j;
                    As[rr * kWgFoldLdk + c] = va[u][4 * q + j];  // A[row rr][k c]
                    Bs[c * kWgFoldLdk + rr] = vb[u][4 * q + j];  // B[k rr][col c] as [col][k]
                }
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int rr = a_kfast ? 2 * i + kh : lrow, kk = a_kfast ? lrow : 2 * i + kh;
                As[rr * kWgFoldLdk + kk] = va[u][i];
                const int cc = b_kfast ? 2 * i + kh : lrow, bk = b_kfast ? lrow : 2 * i + kh;
                Bs[cc * kWgFoldLdk + bk] = vb[u][i];
            }
        }
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int t = 0; t < 16; ++t)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(As[lrow * kWgFoldLdk + 16 * kh + t],
                                                       Bs[lrow * kWgFoldLdk + 16 * kh + t], acc, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) parts[p][r][lane] = acc[r];
    __syncthreads();
    // fold: output (r, l) of the tile, r = 0..15 register, l = lane
    float* cz = g.c + static_cast<uint64_t>(z) * g.m * g.n;
    for (int e = static_cast<int>(threadIdx.x); e < 1024; e += 64 * S) {
        const int r = e >> 6, l = e & 63;
        const uint32_t row = row0 + 8 * (r / 4) + 4 * (l >> 5) + (r % 4);
        const uint32_t col = col0 + (l & 31);
        float stack[kSplitLevels];
#pragma unroll
        for (int lv = 0; lv < kSplitLevels; ++lv) stack[lv] = 0.0f;
#pragma unroll
        for (int q = 0; q < S; ++q) carry_push(stack, static_cast<uint32_t>(q), parts[q][r][l]);
        float total = 0.0f;
#pragma unroll
        for (int lv = 0; lv < kSplitLevels; ++lv)
            if ((static_cast<uint32_t>(S) >> lv) & 1u) total = total + stack[lv];
        if (row < g.m && col < g.n) {
            const uint64_t i = (static_cast<uint64_t>(z) * g.m + row) * g.n + col;
            cz[static_cast<uint64_t>(row) * g.n + col] = apply_epilogue(epi, i, total);
        }
    }
}

// ---- two K partitions of a 64x64 tile in one workgroup -------------------------
// One round of 64x64 tiles (one workgroup per CU) gives each SIMD one wave and
// one MFMA chain (1024^3 unsplit: matrix cores 54% busy). The plan splits K in
// two there, and this kernel
// runs both partitions of a tile as the two halves of one workgroup: waves
// 0-3 partition 0, waves 4-7 partition 1, each half staging its own K-tiles
// straight into LDS and each wave running gemm_direct64_kernel's quarter and
// step order, from 0, so every partial is the split kernel's; two chains per
// SIMD. Partition 1 then hands its partials to partition 0 through LDS, which
// folds each output as split_k_reduce_kernel folds two slices (carry stack in
// partition order, drained from 0.0) and applies the same epilogue: the split
// plan's bits in one launch, with no workspace. G K-tiles per stage per
// partition (128 KB of LDS at G = 2). Measured 1024^3: 58% of peak, the
// matrix cores waiting on the stages' loads (41% of wave cycles) rather than
// on the chains.
template <bool ATR, int G>
__global__ __launch_bounds__(512) void gemm_pair64_kernel(GemmArgs g, FoldEpilogue epi) {
    constexpr int BM = 64, BN = 64, BK = 32, QN = BK / 8, TILE = BM * BK + BK * BN;
    using LA = TileLoader<BM, BK, KCD>;
    __shared__ __attribute__((aligned(16))) float lds[2][2][G * TILE];  // [buffer][partition]

    const int tid = threadIdx.x & 255;  // within the partition's half
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int part = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 8));
    const int wm0 = (wave & 1) * 32;
    const int s0 = wave >> 1;

    uint32_t tm, tn, split;
    tile_of(g, tm, tn, split);
    const uint32_t row0 = tm * BM;
    const uint32_t col0 = tn * BN;

    const uint32_t z = blockIdx.z;
    const uint32_t i0 = z / g.b1, i1 = z % g.b1;
    const float* abase = g.a + i0 * g.sa0 + i1 * g.sa1;
    const float* bbase = g.b + i0 * g.sb0 + i1 * g.sb1;
    const __amdgpu_buffer_rsrc_t arsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(abase), 0, static_cast<int32_t>(0x80000000u), 0x00020000);
    const __amdgpu_buffer_rsrc_t brsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(bbase), 0, static_cast<int32_t>(0x80000000u), 0x00020000);
    const uint32_t kt0 = static_cast<uint32_t>(part) * g.chunk;
    const uint32_t kt1 = min(g.ktiles, kt0 + g.chunk);
    const uint32_t stages = (g.chunk + G - 1) / G;  // the same count for both halves (barriers)

    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;

    const int wv = __builtin_amdgcn_readfirstlane(wave);
    uint32_t voa[2], vob[2];
    if constexpr (ATR)
        rows_offsets<BM>(voa, wv, lane, g.sak, row0, g.m);
    else
        kcd_offsets<BM>(voa, wv, lane, g.sam, row0, g.m);
    rows_offsets<BN>(vob, wv, lane, g.sbk, col0, g.n);
    const uint32_t a_step = static_cast<uint32_t>((ATR ? g.sak : 1) * BK * 4);
    const uint32_t b_step = static_cast<uint32_t>(g.sbk * BK * 4);
    auto load_tile = [&](uint32_t kt, float* dst) {
        if ((kt + 1) * BK > g.k) {
            if constexpr (ATR)
                load_rows_direct<BM>(dst, arsrc, g.sak, row0, g.m, kt * BK, g.k, tid);
            else
                LA::load_direct(dst, arsrc, g.sam, row0, g.m, kt * BK, g.k, tid);
            load_rows_direct<BN>(dst + BM * BK, brsrc, g.sbk, col0, g.n, kt * BK, g.k, tid);
            return;
        }
        issue_direct<BM / 32>(dst, arsrc, voa, wv, kt * a_step);
        issue_direct<BN / 32>(dst + BM * BK, brsrc, vob, wv, kt * b_step);
    };
    auto load_stage = [&](uint32_t kt, int buf) {
#pragma unroll
        for (int j = 0; j < G; ++j)
            if (kt + j < kt1) load_tile(kt + j, lds[buf][part] + j * TILE);
    };
    if (kt0 < kt1) load_stage(kt0, 0);
    __syncthreads();

    const int lrow = lane & 31;
    const int kh = lane >> 5;
    for (uint32_t s = 0; s < stages; ++s) {
        const uint32_t kt = kt0 + s * G;
        const int cur = s & 1;
        if (kt + G < kt1) load_stage(kt + G, cur ^ 1);
#pragma unroll
        for (int j = 0; j < G; ++j) {
            if (kt + j >= kt1) break;
            const float* tl = lds[cur][part] + j * TILE;
            const float* As = ATR ? tl + kh * 16 * BM + wm0 + lrow : tl + (wm0 + lrow) * BK;
            const float* Bs = tl + BM * BK + kh * 16 * BN + 2 * lrow + s0;
            auto a_at = [&](int q) {
                if constexpr (ATR) {
                    f32x4 v;
#pragma unroll
                    for (int st = 0; st < 4; ++st) v[st] = As[(4 * q + st) * BM];
                    return v;
                } else {
                    return *reinterpret_cast<const f32x4*>(As + 4 * ((kh * 4 + q) ^ kcd_swizzle(lrow)));
                }
            };
            f32x4 av[2], bv[2];
            av[0] = a_at(0);
#pragma unroll
            for (int st = 0; st < 4; ++st) bv[0][st] = Bs[st * BN];
#pragma unroll
            for (int q = 0; q < QN; ++q) {
                const int cb = q & 1;
                if (q + 1 < QN) {
                    av[cb ^ 1] = a_at(q + 1);
#pragma unroll
                    for (int st = 0; st < 4; ++st) bv[cb ^ 1][st] = Bs[(4 * (q + 1) + st) * BN];
                }
#pragma unroll
                for (int st = 0; st < 4; ++st)
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[cb][st], bv[cb][st], acc, 0, 0, 0);
            }
        }
        __syncthreads();
    }

    // The last stage issued no loads and ended at a barrier: the stage
    // buffers are free for partition 1's partials (4 waves x 16 x 64 floats).
    float* parts = &lds[0][0][0];
    if (part == 1) {
#pragma unroll
        for (int r = 0; r < 16; ++r) parts[(wave * 16 + r) * 64 + lane] = acc[r];
    }
    __syncthreads();
    if (part == 1) return;
    // acc register r of lane l: row 8*(r/4) + 4*(l/32) + r%4 of the wave's 32,
    // column 2*(l%32) + s0 of the tile.
    const uint32_t col = col0 + 2 * lrow + s0;
    float* cz = g.c + static_cast<uint64_t>(z) * g.m * g.n;
    float vo[16];  // every epilogue load (a mask) before the first store
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        float stack[kSplitLevels];
#pragma unroll
        for (int lv = 0; lv < kSplitLevels; ++lv) stack[lv] = 0.0f;
        carry_push(stack, 0u, acc[r]);
        carry_push(stack, 1u, parts[(wave * 16 + r) * 64 + lane]);
        float total = 0.0f;
#pragma unroll
        for (int lv = 0; lv < kSplitLevels; ++lv)
            if ((2u >> lv) & 1u) total = total + stack[lv];
        const uint32_t row = row0 + wm0 + 8 * (r / 4) + 4 * kh + (r % 4);
        vo[r] = row < g.m && col < g.n
                    ? apply_epilogue(epi, (static_cast<uint64_t>(z) * g.m + row) * g.n + col, total)
                    : total;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t row = row0 + wm0 + 8 * (r / 4) + 4 * kh + (r % 4);
        if (row < g.m && col < g.n) cz[static_cast<uint64_t>(row) * g.n + col] = vo[r];
    }
}

// ---- GEMV -------------------------------------------------------------------
// y[row] = sum_k A[row,k] * x[k]: one wave per row. The row is streamed once
// with 16-byte loads into LDS, products are rounded to f32 separately (no FMA,
// as the oracle's widen(a)*widen(b)), and summed in the oracle's pairwise tree:
// lanes own depth-D leaves, then adjacent leaves combine by xor-butterfly.
// Bit-exact against the CPU oracle.
constexpr int kGemvMaxK = 4096;  // row length one wave stages in LDS

__global__ __launch_bounds__(256) void gemv_kernel(const float* __restrict__ a, int64_t lda,
                                                   const float* __restrict__ x, int64_t incx,
                                                   float* __restrict__ y, uint32_t m, uint32_t k,
                                                   int depth, int vec) {
    constexpr uint32_t kStage = (kGemvMaxK + 4 * (kGemvMaxK / 32) + 3) & ~3u;
    __shared__ __attribute__((aligned(16))) float prod[4][kStage];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + wave;
    const bool live = row < m;
    float* pr = prod[wave];
    if (live) {
        const float* ar = a + static_cast<int64_t>(row) * lda;
        if (vec) {
            // 16 groups of 4 per lane at most (K <= 4096): issue every load first.
            f32x4 av[kGemvMaxK / 256], xv[kGemvMaxK / 256];
#pragma unroll
            for (int i = 0; i < kGemvMaxK / 256; ++i) {
                const uint32_t c = 4u * lane + 256u * i;
                if (c < k) {
                    av[i] = *reinterpret_cast<const f32x4*>(ar + c);
                    if (incx == 1) {
                        xv[i] = *reinterpret_cast<const f32x4*>(x + c);
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j) xv[i][j] = x[static_cast<int64_t>(c + j) * incx];
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < kGemvMaxK / 256; ++i) {
                const uint32_t c = 4u * lane + 256u * i;
                if (c < k) {
                    f32x4 p;
#pragma unroll
                    for (int j = 0; j < 4; ++j) p[j] = __fmul_rn(av[i][j], xv[i][j]);
                    *reinterpret_cast<f32x4*>(pr + stage_index(c)) = p;
                }
            }
        } else {
            for (uint32_t e = lane; e < k; e += 64)
                pr[stage_index(e)] = __fmul_rn(ar[e], x[static_cast<int64_t>(e) * incx]);
        }
    }
    __syncthreads();
    if (!live) return;
    // Leaves: 2^depth of them; lane l owns leaves [l*per, (l+1)*per).
    const uint32_t leaves = 1u << depth;
    const uint32_t per = leaves > 64 ? leaves / 64 : 1;
    float v = 0.0f;
    if (static_cast<uint32_t>(lane) * per < leaves) v = staged_subtree_sum(pr, k, depth, lane * per, per);
    v = wave_sum_butterfly(v);
    if (lane == 0) y[row] = v;
}

// ---- exact GEMM (comparison arm) --------------------------------------------
// C[b, i, j] = the CPU oracle's sum for that output, bit for bit: each product
// a[i,k] * b[k,j] rounded to f32 on its own (no FMA), the K products summed
// in the oracle's pairwise order (reference matmul_impl,
// kernels_matmul.cpp:34-87, over pairwise_sum, reduce.h:55-72). The role of
// the reference's gemm_naive.comp:56-101, the arm selected with
// VKML_GEMM_KERNEL=naive (vulkan_backend.cpp:2158-2161) to check the fast
// kernels against: here the fast kernels accumulate in the matrix cores'
// order, so this arm is what reproduces the oracle exactly.
//
// A workgroup owns a 32 x 32 output tile, a thread 2 x 2 outputs (rows ty and
// ty + 16, columns tx and tx + 16). The K axis is walked leaf by leaf in the
// pairwise tree's depth-D layout (pairwise_leaf): the leaf's A and B slices
// (at most 32 k each) are staged in LDS through the operands' strides, each
// thread sums its outputs' rounded products over the leaf sequentially from
// 0.0, and pushes each leaf sum onto a per-output carry stack; 2^D pushes of
// a complete tree leave the balanced fold of the leaves on top, which is the
// oracle's recursion (empty leaves carry +0.0, exact).
constexpr int kExactTile = 32;
constexpr int kExactLevels = 28;  // 2^27 leaves of 32 cover every 32-bit K

__device__ __forceinline__ void exact_push(float (&stack)[kExactLevels], uint32_t count,
                                           float block) {
    bool carry = true;
#pragma unroll
    for (int l = 0; l < kExactLevels; ++l) {
        if (carry) {
            if ((count >> l) & 1u) {
                block = __fadd_rn(stack[l], block);
            } else {
                stack[l] = block;
                carry = false;
            }
        }
    }
}

// Convolution operands of the exact arm: element (row, pos) of image n's
// columns, row = c*kh*kw + ki*kw + kj, pos = oh*out_w + ow, is x[n, c, h, w]
// with h = oh*stride_h - pad_h + ki*dil_h, w = ow*stride_w - pad_w + kj*dil_w,
// or 0 outside the image (kernels_movement.cpp:438-483). B_IMG: B = the
// columns (forward: k = row, col = pos); B_IMGT: B = their transpose (weight
// gradient: k = pos, col = row).
enum ExactB { B_PTR = 0, B_IMG = 1, B_IMGT = 2 };
struct ExactImg {
    const float* x;
    int64_t sn, sc, sh, sw;  // image strides (elements)
    int32_t H, W, kh, kw, out_w;
    int32_t st_h, st_w, pad_h, pad_w, dil_h, dil_w;
    uint32_t rows, positions;  // C*kh*kw, out_h*out_w
    FastDiv by_kk, by_kw, by_ow;
};

__device__ __forceinline__ float exact_img_value(const ExactImg& im, const float* xn, uint32_t row,
                                                 uint32_t pos) {
    if (row >= im.rows || pos >= im.positions) return 0.0f;
    const uint32_t c = im.by_kk.div(row);
    const uint32_t rem = row - c * static_cast<uint32_t>(im.kh * im.kw);
    const uint32_t ki = im.by_kw.div(rem), kj = rem - ki * static_cast<uint32_t>(im.kw);
    const uint32_t oh = im.by_ow.div(pos), ow = pos - oh * static_cast<uint32_t>(im.out_w);
    const int64_t h = static_cast<int64_t>(oh) * im.st_h - im.pad_h + static_cast<int64_t>(ki) * im.dil_h;
    const int64_t w = static_cast<int64_t>(ow) * im.st_w - im.pad_w + static_cast<int64_t>(kj) * im.dil_w;
    if (h < 0 || h >= im.H || w < 0 || w >= im.W) return 0.0f;
    return xn[static_cast<int64_t>(c) * im.sc + h * im.sh + w * im.sw];
}

template <int BMODE>
__global__ __launch_bounds__(256) void gemm_exact_kernel(GemmArgs g, int depth, ExactImg im) {
    __shared__ float As[kExactTile][kExactTile + 1];  // [row][k]
    __shared__ float Bs[kExactTile][kExactTile + 1];  // [k][col]
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const uint32_t tm = blockIdx.x / g.tiles_n, tn = blockIdx.x - tm * g.tiles_n;
    const uint32_t row0 = tm * kExactTile, col0 = tn * kExactTile;
    const uint32_t bz = blockIdx.z;
    const uint32_t i0 = bz / g.b1, i1 = bz - i0 * g.b1;
    const float* a = g.a + static_cast<int64_t>(i0) * g.sa0 + static_cast<int64_t>(i1) * g.sa1;
    const float* b = g.b + static_cast<int64_t>(i0) * g.sb0 + static_cast<int64_t>(i1) * g.sb1;
    const float* xn = BMODE == B_PTR ? nullptr : im.x + static_cast<int64_t>(bz) * im.sn;
    float stack[4][kExactLevels];
#pragma unroll
    for (int o = 0; o < 4; ++o)
#pragma unroll
        for (int l = 0; l < kExactLevels; ++l) stack[o][l] = 0.0f;
    const uint32_t leaves = 1u << depth;
    for (uint32_t leaf = 0; leaf < leaves; ++leaf) {
        uint32_t kb, ke;
        pairwise_leaf(g.k, depth, leaf, kb, ke);
        const uint32_t len = ke - kb;
        if (len > 0) {
            // stage A[row0 .. +32][kb .. ke) and B[kb .. ke)[col0 .. +32], zeros outside
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int idx = tid + 256 * q;
                const int r = idx >> 5, kk = idx & 31;
                const uint32_t gr = row0 + r;
                As[r][kk] = (gr < g.m && static_cast<uint32_t>(kk) < len)
                                ? a[static_cast<int64_t>(gr) * g.sam + static_cast<int64_t>(kb + kk) * g.sak]
                                : 0.0f;
                const int bk = idx >> 5, c = idx & 31;
                const uint32_t gc = col0 + c;
                const bool in = gc < g.n && static_cast<uint32_t>(bk) < len;
                if constexpr (BMODE == B_PTR)
                    Bs[bk][c] = in ? b[static_cast<int64_t>(kb + bk) * g.sbk + static_cast<int64_t>(gc) * g.sbn]
                                   : 0.0f;
                else if constexpr (BMODE == B_IMG)
                    Bs[bk][c] = in ? exact_img_value(im, xn, kb + bk, gc) : 0.0f;
                else
                    Bs[bk][c] = in ? exact_img_value(im, xn, gc, kb + bk) : 0.0f;
            }
        }
        __syncthreads();
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (uint32_t kk = 0; kk < len; ++kk) {
            const float a0 = As[ty][kk], a1 = As[ty + 16][kk];
            const float b0 = Bs[kk][tx], b1 = Bs[kk][tx + 16];
            acc[0] = __fadd_rn(acc[0], __fmul_rn(a0, b0));
            acc[1] = __fadd_rn(acc[1], __fmul_rn(a0, b1));
            acc[2] = __fadd_rn(acc[2], __fmul_rn(a1, b0));
            acc[3] = __fadd_rn(acc[3], __fmul_rn(a1, b1));
        }
#pragma unroll
        for (int o = 0; o < 4; ++o) exact_push(stack[o], leaf, acc[o]);
        __syncthreads();
    }
    float* c = g.c + static_cast<uint64_t>(bz) * g.m * g.n;
#pragma unroll
    for (int o = 0; o < 4; ++o) {
        const uint32_t gr = row0 + ty + 16 * (o >> 1), gc = col0 + tx + 16 * (o & 1);
        float v = 0.0f;
#pragma unroll
        for (int l = 0; l < kExactLevels; ++l)
            if (l == depth) v = stack[o][l];
        if (gr < g.m && gc < g.n) c[static_cast<uint64_t>(gr) * g.n + gc] = v;
    }
}

// The exact arm's throughput kernel: the same sums as gemm_exact_kernel (each
// product rounded on its own, each leaf summed sequentially from 0.0, leaf sums
// folded by a carry stack), register-blocked the way the reference's default
// gemm_reg.comp:108-274 is, but for wave64 and a 16-lane-wide VALU:
//  - a 64 x 64 output tile per 256-thread workgroup, thread (tx, ty) owning
//    rows 4ty..4ty+3 and columns 4tx..4tx+3 (16 outputs);
//  - a leaf's A slice is staged k-major ([k][row]) and B's [k][col], so every
//    multiply-add step reads its 4 A and 4 B values as two 16-byte LDS reads
//    (one per 16 rounded multiplies and 16 rounded adds; a wave's A read is 4
//    broadcast addresses, its B read 256 contiguous bytes);
//  - the next leaf's operands are loaded into registers while the current
//    leaf is summed, and stored to the other LDS buffer after it (one barrier
//    per leaf);
//  - the carry stack holds LV levels per output, LV >= depth + 1 chosen at
//    launch from K (the reference sizes its stack from K too,
//    gemm_reg.comp:14-29), instead of enough levels for any 32-bit K.
// Staging reads follow the operands' unit stride: along k (a_kfast / b_kfast)
// or along the rows / columns.
constexpr int kExact4Ld = 68;  // LDS row pitch in floats (16-byte aligned rows)

template <int LV>
__device__ __forceinline__ void exact_push_lv(float (&stack)[LV], uint32_t count, float block) {
    bool carry = true;
#pragma unroll
    for (int l = 0; l < LV; ++l) {
        if (carry) {
            if ((count >> l) & 1u) {
                block = __fadd_rn(stack[l], block);
            } else {
                stack[l] = block;
                carry = false;
            }
        }
    }
}

template <int BMODE>
__device__ __forceinline__ void exact4_load(const GemmArgs& g, const ExactImg& im, const float* a,
                                            const float* b, const float* xn, uint32_t row0,
                                            uint32_t col0, uint32_t kb, uint32_t len, int tid,
                                            bool a_kfast, bool b_kfast, float (&va)[8],
                                            float (&vb)[8]) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const int idx = tid + 256 * q;
        const int r = a_kfast ? (idx >> 5) : (idx & 63);
        const int kk = a_kfast ? (idx & 31) : (idx >> 6);
        const uint32_t gr = row0 + r;
        va[q] = (gr < g.m && static_cast<uint32_t>(kk) < len)
                    ? a[static_cast<int64_t>(gr) * g.sam + static_cast<int64_t>(kb + kk) * g.sak]
                    : 0.0f;
        const int c = b_kfast ? (idx >> 5) : (idx & 63);
        const int bk = b_kfast ? (idx & 31) : (idx >> 6);
        const uint32_t gc = col0 + c;
        const bool in = gc < g.n && static_cast<uint32_t>(bk) < len;
        if constexpr (BMODE == B_PTR)
            vb[q] = in ? b[static_cast<int64_t>(kb + bk) * g.sbk + static_cast<int64_t>(gc) * g.sbn] : 0.0f;
        else if constexpr (BMODE == B_IMG)
            vb[q] = in ? exact_img_value(im, xn, kb + bk, gc) : 0.0f;
        else
            vb[q] = in ? exact_img_value(im, xn, gc, kb + bk) : 0.0f;
    }
}

__device__ __forceinline__ void exact4_store(float (*As)[kExact4Ld], float (*Bs)[kExact4Ld], int tid,
                                             bool a_kfast, bool b_kfast, const float (&va)[8],
                                             const float (&vb)[8]) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const int idx = tid + 256 * q;
        const int r = a_kfast ? (idx >> 5) : (idx & 63);
        const int kk = a_kfast ? (idx & 31) : (idx >> 6);
        As[kk][r] = va[q];
        const int c = b_kfast ? (idx >> 5) : (idx & 63);
        const int bk = b_kfast ? (idx & 31) : (idx >> 6);
        Bs[bk][c] = vb[q];
    }
}

// Split over the K axis (blockIdx.y = s of 2^slog): a product with too few
// output tiles to fill the machine gives each split the complete subtree of
// 2^(depth - slog) consecutive leaves starting at leaf s * 2^(depth - slog),
// and writes that subtree's sum to slice s of g.c (split_stride apart). The
// carry-stack fold of the 2^slog slices (split_k_reduce_kernel) is then the
// tree's upper levels, so the result is the unsplit product's bits.
template <int BMODE, int LV>
__global__ __launch_bounds__(256) void gemm_exact4_kernel(GemmArgs g, int depth, ExactImg im,
                                                          int a_kfast_i, int b_kfast_i, int slog) {
    __shared__ __align__(16) float As[2][32][kExact4Ld];  // [buffer][k][row]
    __shared__ __align__(16) float Bs[2][32][kExact4Ld];  // [buffer][k][col]
    const bool a_kfast = a_kfast_i != 0, b_kfast = b_kfast_i != 0;
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const uint32_t tm = blockIdx.x / g.tiles_n, tn = blockIdx.x - tm * g.tiles_n;
    const uint32_t row0 = tm * 64u, col0 = tn * 64u;
    const uint32_t bz = blockIdx.z;
    const uint32_t i0 = bz / g.b1, i1 = bz - i0 * g.b1;
    const float* a = g.a + static_cast<int64_t>(i0) * g.sa0 + static_cast<int64_t>(i1) * g.sa1;
    const float* b = g.b + static_cast<int64_t>(i0) * g.sb0 + static_cast<int64_t>(i1) * g.sb1;
    const float* xn = BMODE == B_PTR ? nullptr : im.x + static_cast<int64_t>(bz) * im.sn;
    float stack[16][LV];
#pragma unroll
    for (int o = 0; o < 16; ++o)
#pragma unroll
        for (int l = 0; l < LV; ++l) stack[o][l] = 0.0f;
    const int ldepth = depth - slog;  // depth of this split's subtree
    const uint32_t leaves = 1u << ldepth;
    const uint32_t first = blockIdx.y << ldepth;
    float va[8], vb[8];
    uint32_t kb, ke;
    pairwise_leaf(g.k, depth, first, kb, ke);
    exact4_load<BMODE>(g, im, a, b, xn, row0, col0, kb, ke - kb, tid, a_kfast, b_kfast, va, vb);
    exact4_store(As[0], Bs[0], tid, a_kfast, b_kfast, va, vb);
    __syncthreads();
    for (uint32_t leaf = 0; leaf < leaves; ++leaf) {
        const int cur = leaf & 1;
        const uint32_t len = ke - kb;
        uint32_t nkb = 0, nke = 0;
        if (leaf + 1 < leaves) {
            pairwise_leaf(g.k, depth, first + leaf + 1, nkb, nke);
            exact4_load<BMODE>(g, im, a, b, xn, row0, col0, nkb, nke - nkb, tid, a_kfast, b_kfast, va, vb);
        }
        float acc[16];
#pragma unroll
        for (int o = 0; o < 16; ++o) acc[o] = 0.0f;
        for (uint32_t kk = 0; kk < len; ++kk) {
            const f32x4 av = *reinterpret_cast<const f32x4*>(&As[cur][kk][4 * ty]);
            const f32x4 bv = *reinterpret_cast<const f32x4*>(&Bs[cur][kk][4 * tx]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[4 * i + j] = __fadd_rn(acc[4 * i + j], __fmul_rn(av[i], bv[j]));
        }
#pragma unroll
        for (int o = 0; o < 16; ++o) exact_push_lv<LV>(stack[o], leaf, acc[o]);
        if (leaf + 1 < leaves) exact4_store(As[cur ^ 1], Bs[cur ^ 1], tid, a_kfast, b_kfast, va, vb);
        kb = nkb;
        ke = nke;
        __syncthreads();
    }
    float* c = g.c + static_cast<uint64_t>(blockIdx.y) * g.split_stride + static_cast<uint64_t>(bz) * g.m * g.n;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t gr = row0 + 4 * ty + i;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t gc = col0 + 4 * tx + j;
            float v = 0.0f;
#pragma unroll
            for (int l = 0; l < LV; ++l)
                if (l == ldepth) v = stack[4 * i + j][l];
            if (gr < g.m && gc < g.n) c[static_cast<uint64_t>(gr) * g.n + gc] = v;
        }
    }
}

// ---- planning ---------------------------------------------------------------

// Split-K plan (reference plan_split_k, vulkan_backend.cpp:596-647), restated
// for MI355X. Kept from the reference: every partition but the last covers the
// same chunk of K-tiles, a forced request gets the largest power-of-two chunk
// that still yields at least that many partitions, the partial workspace is
// capped at 64 MiB, and the fold of the partials is the carry stack (so the
// result is bit-stable for a given plan). Changed: the reference's
// profitability rule (split iff K-tiles >= output tiles, at most 16
// partitions, power-of-two chunk >= 4) was fitted on a 36-CU RDNA1 part. Here
// the caller splits only products whose output tiles cannot give every one of
// the 256 CUs a workgroup; AUTO takes floor(CUs / tiles) partitions (at most
// 256) and the chunk that covers K in that many, at least two K-tiles, when
// that is two or more; products with more than half a round of tiles keep a
// power-of-two chunk giving ceil(CUs / tiles) partitions.
static void plan_split_k(uint32_t tiles, uint32_t ktiles, uint64_t out_elems, uint32_t slots,
                         uint32_t requested, uint32_t& splits, uint32_t& chunk) {
    splits = 1;
    chunk = ktiles;
    if (ktiles < 2 || tiles == 0) return;
    uint32_t c = 1;
    if (requested == 0) {
        // AUTO never splits K of 4 K-tiles or fewer: the fold's launch costs
        // more than the partitions save (64x10x128 6.3 us unsplit against 6.7
        // as 2 partitions, 128x256x100 5.8 against 6.7; 8 K-tiles split into 4
        // still win, 128x100x256 6.7 against 7.9).
        if (ktiles <= 4) return;
        // AUTO: as many partitions as keep the whole grid in one round of one
        // workgroup per CU (a second, partial round would cost a whole
        // partition's time), with equal chunks of K-tiles: 128x784x16384 (7
        // tiles) runs 35 partitions of 15 K-tiles in one round, not 64 of 8
        // in 1.75 rounds.
        if (tiles >= slots) return;
        if (2 * tiles <= slots) {
            uint32_t target = slots / tiles;
            if (target > 256) target = 256;
            c = (ktiles + target - 1) / target;
        } else {
            // more than half a round of tiles: no split fits one round; the
            // largest power-of-two chunk giving ceil(CUs / tiles) partitions,
            // as measured for 1536^3 (3 partitions of 16 K-tiles)
            const uint32_t target = (slots + tiles - 1) / tiles;
            while (c * 2 <= ktiles / target) c *= 2;
        }
        if (c < 2) c = 2;
    } else {
        while (c * 2 <= ktiles / requested) c *= 2;
    }
    if (c >= ktiles) return;
    const uint32_t s = (ktiles + c - 1) / c;
    if (s < 2 || s > 511) return;
    constexpr uint64_t kMaxWorkspaceBytes = 64ull * 1024 * 1024;
    if (out_elems * s * sizeof(float) > kMaxWorkspaceBytes) return;
    splits = s;
    chunk = c;
}

struct TileChoice {
    int bm, bn;
    const char* why = "";   // the reason, for the matmul.kernel decision fact
    uint64_t tiles = 0;     // output tiles of this tiling
    bool pair = false;      // partitions planned for pairs (two per workgroup)
};

template <int BM, int BN, int WM, int WN, int AM>
static void launch_b(const GemmArgs& g, dim3 grid, hipStream_t st, int bmode) {
    constexpr int BK = 32;
    switch (bmode) {
        case KCV: hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, BK, WM, WN, AM, KCV>), grid, dim3(256), 0, st, g, Im2colB{}); break;
        case KCD: hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, BK, WM, WN, AM, KCD>), grid, dim3(256), 0, st, g, Im2colB{}); break;
        case RCV: hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, BK, WM, WN, AM, RCV>), grid, dim3(256), 0, st, g, Im2colB{}); break;
        case KCS: hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, BK, WM, WN, AM, KCS>), grid, dim3(256), 0, st, g, Im2colB{}); break;
        default: hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, BK, WM, WN, AM, RCS>), grid, dim3(256), 0, st, g, Im2colB{}); break;
    }
}

template <int BM, int BN, int WM, int WN>
static int launch_tiles(const GemmArgs& g, uint32_t batch, uint32_t splits, int amode, int bmode) {
    dim3 grid(g.tiles_m * g.tiles_n, splits, batch);
    hipStream_t st = ctx().stream;
    switch (amode) {
        case KCV: launch_b<BM, BN, WM, WN, KCV>(g, grid, st, bmode); break;
        case KCD: launch_b<BM, BN, WM, WN, KCD>(g, grid, st, bmode); break;
        case RCV: launch_b<BM, BN, WM, WN, RCV>(g, grid, st, bmode); break;
        case KCS: launch_b<BM, BN, WM, WN, KCS>(g, grid, st, bmode); break;
        default: launch_b<BM, BN, WM, WN, RCS>(g, grid, st, bmode); break;
    }
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

template <int BM, int BN, int WM, int WN, int BMODE>
static int launch_conv_tiles(const GemmArgs& g, const Im2colB& im, uint32_t batch, uint32_t splits,
                             int amode) {
    constexpr int BK = 32;
    dim3 grid(g.tiles_m * g.tiles_n, splits, batch);
    hipStream_t st = ctx().stream;
    switch (amode) {
        case KCV: hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, BK, WM, WN, KCV, BMODE>), grid, dim3(256), 0, st, g, im); break;
        case KCS: hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, BK, WM, WN, KCS, BMODE>), grid, dim3(256), 0, st, g, im); break;
        case KCD:
            if constexpr (BMODE != IMGTB) {
                hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, BK, WM, WN, KCD, BMODE>), grid, dim3(256), 0, st, g, im);
                break;
            }
            return fail(VKHIP_ERR_INVALID, "conv2d: the batch-folded product takes no straight-to-LDS A");
        default: return fail(VKHIP_ERR_INVALID, "conv2d: A operand load mode %d", amode);
    }
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

template <int G, int C>
static void launch_split_k_fold(const float* ws, float* dst, uint64_t ne, uint32_t splits,
                                const FoldEpilogue& epi) {
    hipLaunchKernelGGL((split_k_reduce_kernel<G, C>), dim3(ceil_div(ne, 256 / G)), dim3(256), 0,
                       ctx().stream, ws, dst, ne, splits, splits / C, epi);
}

int launch_split_k_reduce(const float* ws, float* dst, uint64_t ne, uint32_t splits,
                          const FoldEpilogue& epi) {
    if (ne == 0) return VKHIP_OK;
    if (splits == 0 || splits >= (1u << kSplitLevels))
        return fail(VKHIP_ERR_INVALID, "split-K reduce: %u partitions outside 1..%u", splits,
                    (1u << kSplitLevels) - 1);
    // Groups: 8, or the power of two at or above a smaller partition count
    // (no idle groups); chunk: the smallest power of two that leaves at most
    // that many groups busy (64 for 511 partitions).
    // Small outputs (a weight gradient's few thousand values over hundreds
    // of partials) take 32 groups: 8 outputs per workgroup, so the fold is
    // spread over more workgroups and each thread folds at most 16 partials
    // (the association, and so the bits, do not depend on the group count).
    if (splits <= 2) {
        launch_split_k_fold<2, 1>(ws, dst, ne, splits, epi);
    } else if (splits <= 4) {
        launch_split_k_fold<4, 1>(ws, dst, ne, splits, epi);
    } else if (ne < 32768 && splits > 32) {
        uint32_t chunk = 1;
        while (ceil_div(splits, chunk) > 32) chunk *= 2;
        switch (chunk) {
            case 2: launch_split_k_fold<32, 2>(ws, dst, ne, splits, epi); break;
            case 4: launch_split_k_fold<32, 4>(ws, dst, ne, splits, epi); break;
            case 8: launch_split_k_fold<32, 8>(ws, dst, ne, splits, epi); break;
            default: launch_split_k_fold<32, 16>(ws, dst, ne, splits, epi); break;
        }
    } else {
        uint32_t chunk = 1;
        while (ceil_div(splits, chunk) > 8) chunk *= 2;
        switch (chunk) {
            case 1: launch_split_k_fold<8, 1>(ws, dst, ne, splits, epi); break;
            case 2: launch_split_k_fold<8, 2>(ws, dst, ne, splits, epi); break;
            case 4: launch_split_k_fold<8, 4>(ws, dst, ne, splits, epi); break;
            case 8: launch_split_k_fold<8, 8>(ws, dst, ne, splits, epi); break;
            case 16: launch_split_k_fold<8, 16>(ws, dst, ne, splits, epi); break;
            case 32: launch_split_k_fold<8, 32>(ws, dst, ne, splits, epi); break;
            default: launch_split_k_fold<8, 64>(ws, dst, ne, splits, epi); break;
        }
    }
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

int launch_split_k_reduce(const float* ws, float* dst, uint64_t ne, uint32_t splits) {
    return launch_split_k_reduce(ws, dst, ne, splits, FoldEpilogue{nullptr, 0, 1, 0, nullptr});
}

static FoldEpilogue fold_epilogue(const GemmEpilogue* epi, uint32_t ncols) {
    if (!epi || (!epi->bias && !epi->mask)) return FoldEpilogue{nullptr, 0, 1, 0, nullptr};
    return FoldEpilogue{epi->bias, epi->bias_stride, ncols, epi->relu ? 1u : 0u, epi->mask};
}

static int launch_bias_cols(float* c, uint64_t ne, const FoldEpilogue& epi) {
    if (ne == 0 || (!epi.bias && !epi.mask)) return VKHIP_OK;
    hipLaunchKernelGGL(bias_cols_kernel, dim3(ceil_div(ne, 256)), dim3(256), 0, ctx().stream, c, ne, epi);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

int launch_gemv_rows(const float* a, int64_t lda, const float* x, float* y, uint32_t m, uint32_t k);

int launch_gemv(const float* a, int64_t lda, const float* x, int64_t incx, float* y, uint32_t m,
                uint32_t k) {
    if (m == 0) return VKHIP_OK;
    // Contiguous x and rows up to 32768: the staged row-sum kernel with
    // products (a whole workgroup per row for long rows). Otherwise the
    // wave-per-row kernel below, which also takes a strided x.
    if (incx == 1 && k <= 32768) return launch_gemv_rows(a, lda, x, y, m, k);
    if (k > static_cast<uint32_t>(kGemvMaxK))
        return fail(VKHIP_ERR_UNSUPPORTED, "gemv: K=%u exceeds the LDS-staged maximum %d", k,
                    kGemvMaxK);
    const bool vec = (reinterpret_cast<uintptr_t>(a) % 16 == 0) && (lda % 4 == 0) && (k % 4 == 0) &&
                     (incx != 1 || reinterpret_cast<uintptr_t>(x) % 16 == 0);
    const int depth = pairwise_depth(k);
    hipLaunchKernelGGL(gemv_kernel, dim3(ceil_div(m, 4)), dim3(256), 0, ctx().stream, a, lda, x,
                       incx, y, m, k, depth, vec ? 1 : 0);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

// Tile and split-K choice, from measurements of both tile kernels on MI355X
// (fp32, 256 CUs):
//  - A 128x128 tile (four 64x64 wave tiles, four independent MFMA chains per
//    wave) keeps the matrix cores busy even at one workgroup per CU; a 64x64
//    tile (one chain per wave) needs several workgroups per CU to do so, and
//    wastes less on outputs narrower than 128.
//  - So: enough 128x128 tiles for every CU -> 128x128, unsplit (2048^3 runs
//    at 108 TFLOP/s unsplit, 101 split in two); else enough 64x64 tiles ->
//    64x64, unsplit (1024^3: 31 us, against 34-48 us for any split).
//  - Otherwise split K: with 128x128 tiles when each partition still gets at
//    least 8 K-tiles (256x256x65536: 88 us as 64 partitions, 102 us as 32
//    partitions of 64x64 tiles), else with 64x64 tiles (512^3: 11 us as 4
//    partitions, 16 us as 8).
int gemm_plan(uint32_t batch, uint32_t m, uint32_t n, uint32_t k, int32_t split_request,
              uint32_t& splits, uint32_t& chunk, TileChoice& tile, bool narrow_split = false) {
    constexpr uint32_t BK = 32;
    const uint32_t cu = ctx().ready ? static_cast<uint32_t>(ctx().caps.compute_units) : 256u;
    const uint64_t t128 = static_cast<uint64_t>(ceil_div(m, 128)) * ceil_div(n, 128) * batch;
    const uint64_t t64 = static_cast<uint64_t>(ceil_div(m, 64)) * ceil_div(n, 64) * batch;
    // 128x128 tiles pad the output more than 25% beyond what 64x64 tiles do
    // (padded areas are 16384*t128 and 4096*t64).
    const bool narrow = 16 * t128 > 5 * t64;
    const uint32_t ktiles = ceil_div(k, BK);
    splits = 1;
    chunk = ktiles > 0 ? ktiles : 1;
    const uint32_t req = split_request > 1 ? static_cast<uint32_t>(split_request) : 0u;
    bool want_split = false;
    // 64x64 tiles run two workgroups per CU. At one workgroup per CU they hide
    // little latency (1024x1024x2048: 69 TFLOP/s), and a short last round
    // (under 60% of its slots filled) idles most CUs (1536^3: 73); 128x128
    // tiles that split K into partitions of at least 16 K-tiles run those
    // faster (86 and 89), provided, for the second case, the partitions give
    // at least 1.5 workgroups per CU (1536x1536x4096 as 288 partitions: 71,
    // against 77 on 64x64 tiles). With 8 K-tiles per partition the 64x64
    // tiles still win (1024^3: 69 against 67).
    const uint64_t slots64 = 2ull * cu;
    const bool poor64 = t64 * 10 < ((t64 + slots64 - 1) / slots64) * slots64 * 6;
    const uint64_t target128 = (cu + t128 - 1) / t128;
    uint64_t c128 = 1;
    while (c128 * 2 <= ktiles / target128) c128 *= 2;
    const uint64_t parts128 = t128 * ((ktiles + c128 - 1) / c128);
    const bool deep_split = !narrow && ktiles / target128 >= 16 &&
                            (t64 < slots64 || (poor64 && 2 * parts128 >= 3ull * cu));
    if (t128 >= cu && !narrow) {
        tile = {128, 128, "128x128 tiles give every CU a workgroup"};
    } else if (t64 >= cu && !deep_split) {
        tile = {64, 64, narrow ? "128x128 tiles would pad the output by more than 25%"
                               : "only 64x64 tiles give every CU a workgroup"};
    } else {
        tile = (!narrow && ktiles / target128 >= 8)
                   ? TileChoice{128, 128, "too few output tiles: K split over 128x128 tiles"}
                   : TileChoice{64, 64, "too few output tiles: K split over 64x64 tiles"};
        want_split = true;
    }
    tile.tiles = tile.bm == 128 ? t128 : t64;
    if (split_request == 1) return VKHIP_OK;  // OFF
    // Exactly one round of 64x64 tiles (one workgroup per CU) and K of at
    // least 16 K-tiles: two partitions, which gemm()'s direct path runs as the
    // two halves of one workgroup (gemm_pair64_kernel: two MFMA chains per
    // SIMD: 1024^3 23.2-24.0 us, against 24.1-25.6 unsplit; 128x128 or
    // 128x64 tiles in four partitions plus the fold ran 35.6).
    if (!want_split && req == 0 && tile.bm == 64 && t64 == cu && batch == 1 && ktiles >= 16) {
        splits = 2;
        chunk = (ktiles + 1) / 2;
        return VKHIP_OK;
    }
    if (!want_split && req == 0) return VKHIP_OK;
    const uint64_t tiles = tile.bm == 128 ? t128 : t64;
    if (tiles > 0xffffffffull) return VKHIP_OK;
    plan_split_k(static_cast<uint32_t>(tiles), ktiles, static_cast<uint64_t>(m) * n * batch, cu,
                 req, splits, chunk);
    // A split over 128x128 tiles that gives each CU at most one workgroup is
    // planned with twice the partitions instead, run as pairs by the direct
    // kernel (two K streams per workgroup, gemm_nn_direct_kernel<.., true>),
    // when every partition keeps at least 8 K-tiles and the pairs still fit
    // one workgroup per CU: 256x256x65536 as 128 partitions in 64 pairs runs
    // 74.8 us against 78.6 as 64 partitions. Other kernels run the same plan
    // unpaired (NT 256x256x65536: 81.2 us against 80.3), so every layout
    // keeps the same partitions and the same bits.
    if (req == 0 && tile.bm == 128 && tiles * splits <= cu) {
        uint32_t s2 = 1, c2 = ktiles;
        plan_split_k(static_cast<uint32_t>(tiles), ktiles, static_cast<uint64_t>(m) * n * batch,
                     2 * cu, 0, s2, c2);
        const bool pair_ok = s2 > splits && c2 >= 8 && tiles * ((s2 + 1) / 2) <= cu;
        // gemm()'s direct kernels also run 128x64 tiles, three workgroups per
        // CU (narrow_split): a split over those pads N less (784 columns: 832
        // against 896) and fills three slots per CU instead of one paired
        // workgroup. Taken when its estimated matrix-core time per CU is
        // lower: 128x64 K-tiles per CU over the fraction of the time the
        // matrix cores do useful work, fold included (paired 128x128 0.75,
        // unpaired one workgroup per CU 0.60, three 128x64 per CU 0.75; the
        // last from 128x784x16384 as 57 partitions of 9 K-tiles, 39.9 us
        // against 44.8 as 32 pairs of 8, and 256x256x65536 as 94 partitions
        // of 22, 79.8 us against 78.3 as 64 pairs of 16, which stays paired).
        // (This tile count, unlike the rest of the plan, depends on which
        // operand is A: M x N and N x M may get different partitions, and so
        // different bits. vkhip_gemm_plan exposes the plan so that a caller
        // that swaps the operands, as the host core's in-place weight
        // gradient does, can check that both orientations agree.)
        const uint64_t t6 = static_cast<uint64_t>(ceil_div(m, 128)) * ceil_div(n, 64) * batch;
        uint32_t s3 = 1, c3 = ktiles;
        if (narrow_split && t6 <= 0xffffffffull)
            plan_split_k(static_cast<uint32_t>(t6), ktiles, static_cast<uint64_t>(m) * n * batch, 3 * cu, 0,
                         s3, c3);
        const double cost_now = pair_ok ? 4.0 * c2 / 0.75 : 2.0 * chunk / 0.60;
        const uint64_t rounds3 = (t6 * s3 + 3ull * cu - 1) / (3ull * cu);
        const double cost3 = static_cast<double>(rounds3) * 3.0 * c3 / 0.75;
        if (narrow_split && s3 > 1 && c3 >= 4 && cost3 < cost_now) {
            splits = s3;
            chunk = c3;
        } else if (pair_ok) {
            splits = s2;
            chunk = c2;
            tile.pair = true;
        }
    }
    if (splits == 1) chunk = ktiles > 0 ? ktiles : 1;
    return VKHIP_OK;
}

template <int BMODE, int LV>
static void launch_exact4_lv(const GemmArgs& g, uint32_t batch, int depth, const ExactImg& im,
                             int a_kfast, int b_kfast, int slog) {
    const dim3 grid(g.tiles_m * g.tiles_n, 1u << slog, batch);
    hipLaunchKernelGGL((gemm_exact4_kernel<BMODE, LV>), grid, dim3(256), 0, ctx().stream, g, depth, im,
                       a_kfast, b_kfast, slog);
}

template <int BMODE>
static void launch_exact4(const GemmArgs& g, uint32_t batch, int depth, const ExactImg& im, int a_kfast,
                          int b_kfast, int slog) {
    const int ldepth = depth - slog;  // the stack holds levels 0..ldepth
    if (ldepth < 4)
        launch_exact4_lv<BMODE, 4>(g, batch, depth, im, a_kfast, b_kfast, slog);
    else if (ldepth < 6)
        launch_exact4_lv<BMODE, 6>(g, batch, depth, im, a_kfast, b_kfast, slog);
    else if (ldepth < 9)
        launch_exact4_lv<BMODE, 9>(g, batch, depth, im, a_kfast, b_kfast, slog);
    else
        launch_exact4_lv<BMODE, 13>(g, batch, depth, im, a_kfast, b_kfast, slog);
}

// Deepest K the register-blocked exact kernel takes (its largest stack has 13
// levels: K up to 2^12 leaves of 32 = 131072); deeper K runs gemm_exact_kernel.
constexpr int kExact4MaxDepth = 12;

// K-splits of the exact arm for a product of `tiles` 64x64 output tiles (all
// batches) and pairwise depth `depth`: 2^slog complete subtrees, enough to
// give the 256 CUs two workgroups each, each subtree keeping at least two
// leaves; 0 when the tiles fill the machine already.
static int exact_split_log(uint64_t tiles, int depth, uint64_t out_elems) {
    const uint64_t cu = ctx().ready ? static_cast<uint64_t>(ctx().caps.compute_units) : 256u;
    int slog = 0;
    while (slog + 1 < depth && (tiles << (slog + 1)) <= 2 * cu && slog + 1 <= 8 &&
           (out_elems << (slog + 1)) * sizeof(float) <= (64ull << 20))
        ++slog;
    return slog;
}

// ws: the caller's partial workspace (nullptr: the backend's own, grown on
// demand), of ws_bytes bytes.
static int launch_exact(GemmArgs& g, uint32_t batch, int bmode, const ExactImg& im,
                        float* ws = nullptr, size_t ws_bytes = 0, bool may_split = false) {
    const int depth4 = pairwise_depth(g.k);
    if (depth4 <= kExact4MaxDepth) {
        g.tiles_m = ceil_div(g.m, 64u);
        g.tiles_n = ceil_div(g.n, 64u);
        const uint64_t tiles4 = static_cast<uint64_t>(g.tiles_m) * g.tiles_n;
        if (tiles4 > 0x7fffffffull)
            return fail(VKHIP_ERR_UNSUPPORTED, "exact gemm: %llu output tiles",
                        static_cast<unsigned long long>(tiles4));
        // stage along whichever axis of each operand is unit-stride
        const int a_kfast = g.sak == 1 || g.sam != 1;
        const int b_kfast = bmode == B_IMGT || (bmode == B_PTR && (g.sbk == 1 || g.sbn != 1));
        const uint64_t out_elems = static_cast<uint64_t>(batch) * g.m * g.n;
        const int slog = may_split ? exact_split_log(tiles4 * batch, depth4, out_elems) : 0;
        float* c = g.c;
        if (slog > 0) {
            const size_t need = (out_elems << slog) * sizeof(float);
            if (ws == nullptr) {
                const int wst = workspace(need, &ws);
                if (wst != VKHIP_OK) return wst;
            } else if (need > ws_bytes) {
                return fail(VKHIP_ERR_INVALID,
                            "exact matmul %ux%ux%u (batch %u) splits K into %d subtrees whose partials "
                            "need %zu bytes; the allocation-free entry point's scratch holds %zu",
                            g.m, g.n, g.k, batch, 1 << slog, need, ws_bytes);
            }
            g.c = ws;
            g.split_stride = out_elems;
        }
        if (bmode == B_IMG)
            launch_exact4<B_IMG>(g, batch, depth4, im, a_kfast, b_kfast, slog);
        else if (bmode == B_IMGT)
            launch_exact4<B_IMGT>(g, batch, depth4, im, a_kfast, b_kfast, slog);
        else
            launch_exact4<B_PTR>(g, batch, depth4, im, a_kfast, b_kfast, slog);
        VKHIP_LAUNCH_CHECK();
        if (slog > 0) return launch_split_k_reduce(ws, c, out_elems, 1u << slog);
        return VKHIP_OK;
    }
    g.tiles_m = ceil_div(g.m, kExactTile);
    g.tiles_n = ceil_div(g.n, kExactTile);
    const uint64_t tiles = static_cast<uint64_t>(g.tiles_m) * g.tiles_n;
    if (tiles > 0x7fffffffull)
        return fail(VKHIP_ERR_UNSUPPORTED, "exact gemm: %llu output tiles",
                    static_cast<unsigned long long>(tiles));
    const int depth = pairwise_depth(g.k);
    if (depth >= kExactLevels) return fail(VKHIP_ERR_UNSUPPORTED, "exact gemm: K=%u too deep", g.k);
    const dim3 grid(static_cast<uint32_t>(tiles), 1, batch);
    if (bmode == B_IMG)
        hipLaunchKernelGGL(gemm_exact_kernel<B_IMG>, grid, dim3(256), 0, ctx().stream, g, depth, im);
    else if (bmode == B_IMGT)
        hipLaunchKernelGGL(gemm_exact_kernel<B_IMGT>, grid, dim3(256), 0, ctx().stream, g, depth, im);
    else
        hipLaunchKernelGGL(gemm_exact_kernel<B_PTR>, grid, dim3(256), 0, ctx().stream, g, depth, im);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

static int launch_gemm_exact(const float* a, const vkhip_operand& ad, const float* b,
                             const vkhip_operand& bd, float* c, uint32_t batch, uint32_t b1,
                             uint32_t m, uint32_t n, uint32_t k, float* ws = nullptr,
                             size_t ws_bytes = 0) {
    GemmArgs g{};
    g.a = a;
    g.b = b;
    g.c = c;
    g.sa0 = ad.ne[0] == 1 ? 0 : ad.nb[0];
    g.sa1 = ad.ne[1] == 1 ? 0 : ad.nb[1];
    g.sam = ad.nb[2];
    g.sak = ad.nb[3];
    g.sb0 = bd.ne[0] == 1 ? 0 : bd.nb[0];
    g.sb1 = bd.ne[1] == 1 ? 0 : bd.nb[1];
    g.sbk = bd.nb[2];
    g.sbn = bd.nb[3];
    g.b1 = b1;
    g.m = m;
    g.n = n;
    g.k = k;
    return launch_exact(g, batch, B_PTR, ExactImg{}, ws, ws_bytes, true);
}

// The exact arm's image geometry for a convolution (see ExactImg).
static int exact_img(const vkhip_unfold& p, const float* x, const vkhip_operand& xd, ExactImg& im) {
    const int64_t oh = (static_cast<int64_t>(p.image_h) + 2 * p.pad_h -
                        (static_cast<int64_t>(p.dilation_h) * (p.kernel_h - 1) + 1)) / p.stride_h + 1;
    const int64_t ow = (static_cast<int64_t>(p.image_w) + 2 * p.pad_w -
                        (static_cast<int64_t>(p.dilation_w) * (p.kernel_w - 1) + 1)) / p.stride_w + 1;
    const uint64_t rows = static_cast<uint64_t>(xd.ne[1]) * p.kernel_h * p.kernel_w;
    if (oh <= 0 || ow <= 0 || rows > 0xffffffffull || static_cast<uint64_t>(oh) * ow > 0xffffffffull)
        return fail(VKHIP_ERR_INVALID, "exact conv: invalid geometry");
    im.x = x;
    im.sn = xd.nb[0];
    im.sc = xd.nb[1];
    im.sh = xd.nb[2];
    im.sw = xd.nb[3];
    im.H = p.image_h;
    im.W = p.image_w;
    im.kh = p.kernel_h;
    im.kw = p.kernel_w;
    im.out_w = static_cast<int32_t>(ow);
    im.st_h = p.stride_h;
    im.st_w = p.stride_w;
    im.pad_h = p.pad_h;
    im.pad_w = p.pad_w;
    im.dil_h = p.dilation_h;
    im.dil_w = p.dilation_w;
    im.rows = static_cast<uint32_t>(rows);
    im.positions = static_cast<uint32_t>(oh * ow);
    im.by_kk = FastDiv(static_cast<uint32_t>(p.kernel_h * p.kernel_w));
    im.by_kw = FastDiv(static_cast<uint32_t>(p.kernel_w));
    im.by_ow = FastDiv(static_cast<uint32_t>(ow));
    return VKHIP_OK;
}

// How full a launch's rounds keep the machine: workgroups / (rounds * slots),
// slots = the workgroups resident at once.
static double round_fill(uint64_t wgs, uint64_t slots) {
    return static_cast<double>(wgs) / static_cast<double>((wgs + slots - 1) / slots * slots);
}

static int gemm_core(const float* a, const vkhip_operand& ad, const float* b, const vkhip_operand& bd,
                     float* c, const vkhip_gemm_opts* opts, const FixedScratch* scratch,
                     const FoldEpilogue& fe, bool* fused) {
    const uint32_t b0 = ad.ne[0] > bd.ne[0] ? ad.ne[0] : bd.ne[0];
    const uint32_t b1 = ad.ne[1] > bd.ne[1] ? ad.ne[1] : bd.ne[1];
    const uint32_t m = ad.ne[2], k = ad.ne[3], n = bd.ne[3];
    if (bd.ne[2] != k)
        return fail(VKHIP_ERR_INVALID, "matmul inner dimensions disagree: %u vs %u", k, bd.ne[2]);
    for (int i = 0; i < 2; ++i) {
        if ((ad.ne[i] != 1 && ad.ne[i] != (i ? b1 : b0)) || (bd.ne[i] != 1 && bd.ne[i] != (i ? b1 : b0)))
            return fail(VKHIP_ERR_INVALID, "matmul batch extents disagree");
    }
    const uint64_t batch = static_cast<uint64_t>(b0) * b1;
    if (batch == 0 || m == 0 || n == 0) return VKHIP_OK;
    if (batch > 65535) return fail(VKHIP_ERR_UNSUPPORTED, "matmul batch %llu > 65535",
                                   static_cast<unsigned long long>(batch));
    int kernel = opts ? opts->kernel : VKHIP_GEMM_AUTO;
    if (kernel == VKHIP_GEMM_AUTO && ctx().exact_math) kernel = VKHIP_GEMM_EXACT;
    const int32_t split_req = opts ? opts->split_k : 0;
    if (k == 0) {
        return launch_zero_f32(c, batch * m * n);
    }

    // GEMV: an N == 1 product with a unit-stride K axis of A is a bandwidth
    // problem, not a matrix-core one. AUTO takes it whenever batch == 1.
    if ((kernel == VKHIP_GEMM_GEMV || kernel == VKHIP_GEMM_AUTO) && n == 1 && batch == 1 &&
        ad.nb[3] == 1 && (k <= static_cast<uint32_t>(kGemvMaxK) || (bd.nb[2] == 1 && k <= 32768))) {
        publish("matmul.kernel", "matmul", "gemv", "gemm_mfma",
                kernel == VKHIP_GEMM_GEMV ? "GEMV requested" : "an N == 1 product is bandwidth-bound",
                static_cast<int64_t>(k), static_cast<int64_t>(m));
        return launch_gemv(a, ad.nb[2], b, bd.nb[2], c, m, k);
    }
    if (kernel == VKHIP_GEMM_GEMV)
        return fail(VKHIP_ERR_UNSUPPORTED, "gemv requested for a %ux%ux%u problem", m, n, k);
    if (kernel == VKHIP_GEMM_EXACT) {
        publish("matmul.kernel", "matmul", "gemm_exact", "gemm_mfma", "exact arm requested",
                static_cast<int64_t>(k), static_cast<int64_t>(m) * n);
        return launch_gemm_exact(a, ad, b, bd, c, static_cast<uint32_t>(batch), b1, m, n, k,
                                 scratch ? scratch->ptr : nullptr, scratch ? scratch->bytes : 0);
    }
    if (kernel != VKHIP_GEMM_AUTO && kernel != VKHIP_GEMM_MFMA)
        return fail(VKHIP_ERR_INVALID, "gemm: unknown kernel selection %d", kernel);

    uint32_t splits, chunk;
    TileChoice tile;
    gemm_plan(static_cast<uint32_t>(batch), m, n, k, split_req, splits, chunk, tile, true);
    {
        const int64_t cus = ctx().ready ? ctx().caps.compute_units : 256;
        publish("matmul.kernel", "matmul", tile.bm == 128 ? "gemm_mfma_128x128" : "gemm_mfma_64x64",
                tile.bm == 128 ? "gemm_mfma_64x64" : "gemm_mfma_128x128", tile.why,
                static_cast<int64_t>(tile.tiles), cus);
        char chose[32] = "unsplit";
        if (splits > 1) snprintf(chose, sizeof chose, "split_k_%u", splits);
        publish("matmul.split_k", "matmul", chose, splits > 1 ? "unsplit" : "split_k",
                split_req > 1    ? "partition count requested"
                : split_req == 1 ? "split-K turned off"
                : splits > 1     ? "output tiles below one workgroup per CU"
                                 : "output tiles fill the CUs",
                static_cast<int64_t>(tile.tiles) * splits, cus);
    }

    GemmArgs g{};
    g.a = a;
    g.b = b;
    g.sa0 = ad.ne[0] == 1 ? 0 : ad.nb[0];
    g.sa1 = ad.ne[1] == 1 ? 0 : ad.nb[1];
    g.sam = ad.nb[2];
    g.sak = ad.nb[3];
    g.sb0 = bd.ne[0] == 1 ? 0 : bd.nb[0];
    g.sb1 = bd.ne[1] == 1 ? 0 : bd.nb[1];
    g.sbk = bd.nb[2];
    g.sbn = bd.nb[3];
    g.b1 = b1;
    g.m = m;
    g.n = n;
    g.k = k;
    g.tiles_m = ceil_div(m, tile.bm);
    g.tiles_n = ceil_div(n, tile.bn);
    g.ktiles = ceil_div(k, 32);
    g.chunk = chunk;
    const bool akc = ad.nb[3] == 1 || k == 1;
    const bool bkc = bd.nb[2] == 1 || k == 1;
    auto aligned = [](const float* p, int64_t s0, int64_t s1, int64_t srow) {
        return reinterpret_cast<uintptr_t>(p) % 16 == 0 && s0 % 4 == 0 && s1 % 4 == 0 && srow % 4 == 0;
    };
    // 16-byte loads: along k for a k-contiguous operand, along rows for a
    // row-contiguous one (then the k stride is the row pitch that must keep
    // 16-byte alignment).
    g.a_vec = akc ? (ad.nb[3] == 1 && aligned(a, g.sa0, g.sa1, g.sam))
                  : (g.sam == 1 && aligned(a, g.sa0, g.sa1, g.sak));
    g.b_vec = bkc ? (bd.nb[2] == 1 && aligned(b, g.sb0, g.sb1, g.sbn))
                  : (g.sbn == 1 && aligned(b, g.sb0, g.sb1, g.sbk));

    const uint64_t out_elems = batch * m * n;
    int amode = akc ? (g.a_vec ? KCV : KCS) : (g.a_vec ? RCV : RCS);
    // The buffer-load paths (straight-to-LDS operands and the direct kernels)
    // address an operand by unsigned 32-bit byte offsets from its base, so
    // they take operands whose strides are all non-negative; a negative
    // stride (a reversed view) stays on the pointer loads.
    const bool a_fwd = g.sa0 >= 0 && g.sa1 >= 0 && g.sam >= 0 && g.sak >= 0;
    const bool b_fwd = g.sb0 >= 0 && g.sb1 >= 0 && g.sbk >= 0 && g.sbn >= 0;
    // Straight-to-LDS operands: unit k stride, K a multiple of four, and every
    // byte offset of one batch's operand within the buffer resource's 2^31 bytes.
    if (a_fwd && amode == KCV && g.sak == 1 && k % 4 == 0 &&
        ((static_cast<int64_t>(m) - 1) * g.sam + k) * 4 < (int64_t{1} << 31))
        amode = KCD;
    int bmode = bkc ? (g.b_vec ? KCV : KCS) : (g.b_vec ? RCV : RCS);
    if (b_fwd && bmode == KCV && g.sbk == 1 && k % 4 == 0 &&
        ((static_cast<int64_t>(n) - 1) * g.sbn + k) * 4 < (int64_t{1} << 31))
        bmode = KCD;
    int st;
    // NN and TN with both operands straight into LDS: 128x128 tiles, B
    // row-contiguous with 16-byte rows and N a multiple of four (a 16-byte
    // group is wholly inside or outside), A in load mode KCD (NN) or
    // row-contiguous like B with M a multiple of four (TN), byte offsets
    // within 2^31.
    const bool b_rows = b_fwd && bmode == RCV && g.sbn == 1 && n % 4 == 0 && g.sbk % 4 == 0 &&
                        ((static_cast<int64_t>(k) - 1) * g.sbk + n) * 4 < (int64_t{1} << 31);
    const bool a_rows = a_fwd && amode == RCV && g.sam == 1 && m % 4 == 0 && g.sak % 4 == 0 &&
                        ((static_cast<int64_t>(k) - 1) * g.sak + m) * 4 < (int64_t{1} << 31);
    // The paired direct kernel writes one slice per pair of partitions (none
    // for a single pair); every other kernel one per partition.
    const bool direct128 = tile.bm == 128 && b_rows && (amode == KCD || a_rows);
    const bool paired = direct128 && tile.pair && splits >= 2 && reinterpret_cast<uintptr_t>(c) % 16 == 0;
    // Two to four partitions on 64x64 tiles: one launch, the partials folded
    // inside the workgroup (gemm_wgfold_kernel), the same bits; for products
    // of at least 64 tiles of 32x32 (512^3: 256). Fewer tiles leave most CUs
    // idle: the 128 x 100 x 256 product of a Linear(256, 100) layer (16
    // tiles) took 10.3 us this way against 4.9 + 4.6 us as two launches.
    const uint64_t t32_all = static_cast<uint64_t>(ceil_div(m, 32u)) * ceil_div(n, 32u) * batch;
    if (splits >= 2 && splits <= 4 && chunk <= 4 && tile.bm == 64 && !tile.pair && t32_all >= 64) {
        g.tiles_m = ceil_div(m, 32u);
        g.tiles_n = ceil_div(n, 32u);
        const uint64_t t32 = static_cast<uint64_t>(g.tiles_m) * g.tiles_n;
        if (t32 <= 0x7fffffffull) {
            g.c = c;
            const int akf = g.sak == 1 || g.sam != 1;
            const int bkf = g.sbk == 1 || g.sbn != 1;
            const dim3 grid(static_cast<uint32_t>(t32), 1, static_cast<uint32_t>(batch));
#define VKHIP_WGF(SS, KT) \
    hipLaunchKernelGGL((gemm_wgfold_kernel<SS, KT>), grid, dim3(64 * SS), 0, ctx().stream, g, fe, akf, bkf)
#define VKHIP_WGF_S(KT) \
    do { if (splits == 2) VKHIP_WGF(2, KT); else if (splits == 3) VKHIP_WGF(3, KT); else VKHIP_WGF(4, KT); } while (0)
            if (chunk <= 2) VKHIP_WGF_S(2); else VKHIP_WGF_S(4);
#undef VKHIP_WGF_S
#undef VKHIP_WGF
            VKHIP_LAUNCH_CHECK();
            *fused = true;
            return VKHIP_OK;
        }
        g.tiles_m = ceil_div(m, tile.bm);
        g.tiles_n = ceil_div(n, tile.bn);
    }
    // Two partitions of a 64x64 tile grid that is one round of one workgroup
    // per CU: both in one workgroup, folded there (gemm_pair64_kernel).
    {
        const uint64_t cus = ctx().ready ? static_cast<uint64_t>(ctx().caps.compute_units) : 256u;
        const uint64_t t64n = static_cast<uint64_t>(g.tiles_m) * g.tiles_n * batch;
        if (splits == 2 && tile.bm == 64 && !tile.pair && t64n <= cus && b_rows && (amode == KCD || a_rows)) {
            g.c = c;
            g.flat_splits = 0;
            const dim3 grid(g.tiles_m * g.tiles_n, 1, static_cast<uint32_t>(batch));
            void (*kern)(GemmArgs, FoldEpilogue) = amode == KCD ? gemm_pair64_kernel<false, 2>
                                                                : gemm_pair64_kernel<true, 2>;
            hipLaunchKernelGGL(kern, grid, dim3(512), 0, ctx().stream, g, fe);
            VKHIP_LAUNCH_CHECK();
            *fused = true;
            return VKHIP_OK;
        }
    }
    const uint32_t slices = paired ? (splits + 1) / 2 : splits;
    float* target = c;
    if (slices > 1) {
        float* ws = nullptr;
        const size_t need = out_elems * slices * sizeof(float);
        if (scratch) {
            if (need > scratch->bytes)
                return fail(VKHIP_ERR_INVALID,
                            "matmul %ux%ux%u (batch %llu) splits K into %u partitions whose partials "
                            "need %zu bytes; the allocation-free entry point's scratch holds %zu",
                            m, n, k, static_cast<unsigned long long>(batch), splits, need,
                            scratch->bytes);
            ws = scratch->ptr;
        } else {
            const int wst = workspace(need, &ws);
            if (wst != VKHIP_OK) return wst;
        }
        target = ws;
        g.split_stride = out_elems;
    }
    g.c = target;
    if (slices == 1 && (fe.bias || fe.mask)) {  // the kernel writes the output: its epilogue
        g.epi = fe;
        *fused = true;
    }
    // Split direct launches run flat, partitions grouped per XCD (tile_of).
    const uint64_t flat = static_cast<uint64_t>(g.tiles_m) * g.tiles_n * splits;
    if (splits > 1 && flat <= 0x7fffffffull) g.flat_splits = splits;
    const dim3 dgrid = g.flat_splits ? dim3(static_cast<uint32_t>(flat), 1, static_cast<uint32_t>(batch))
                                     : dim3(g.tiles_m * g.tiles_n, splits, static_cast<uint32_t>(batch));
    // (paired: c is 16-byte aligned, and so is the workspace)
    if (paired || (direct128 && reinterpret_cast<uintptr_t>(target) % 16 == 0)) {
        if (paired) {
            g.pairs = slices;
            dim3 grid(g.tiles_m * g.tiles_n, 1, static_cast<uint32_t>(batch));
            if (g.pairs == 1) {
                g.flat_splits = 0;
            } else {
                const uint64_t pflat = static_cast<uint64_t>(g.tiles_m) * g.tiles_n * g.pairs;
                g.flat_splits = pflat <= 0x7fffffffull ? g.pairs : 0;
                grid = g.flat_splits ? dim3(static_cast<uint32_t>(pflat), 1, static_cast<uint32_t>(batch))
                                     : dim3(g.tiles_m * g.tiles_n, g.pairs, static_cast<uint32_t>(batch));
            }
            if (amode == KCD)
                hipLaunchKernelGGL((gemm_nn_direct_kernel<false, true>), grid, dim3(512), 0, ctx().stream, g);
            else
                hipLaunchKernelGGL((gemm_nn_direct_kernel<true, true>), grid, dim3(512), 0, ctx().stream, g);
            VKHIP_LAUNCH_CHECK();
            if (g.pairs > 1) { *fused = true; return launch_split_k_reduce(target, c, out_elems, g.pairs, fe); }
            return VKHIP_OK;
        }
        // 128x64 tiles when the last round of 128x128 workgroups would leave
        // more of the machine idle: workgroups resident per CU are two of
        // 128x128 (70 KB of LDS each) or three of 128x64 (53 KB), and a
        // 128x64 tile does 0.94x the work per CU-second (4096^3: 130 against
        // 138 TFLOP/s), so the fill of the launch's rounds decides:
        //   fill = workgroups / (rounds * slots), 128x64's scaled by 0.94.
        // Measured: 3072^3 90 -> 119 TFLOP/s, 2304^3 90 -> 112, 2048x3072x2048
        // 105 -> 127, 2048^3 121 -> 125; 4096^3, 8192x1024x4096, 2560^3 and
        // 4096x2048x2048 keep 128x128 (128x64 measured 3-7% slower there).
        const uint64_t cus = ctx().ready ? static_cast<uint64_t>(ctx().caps.compute_units) : 256u;
        const uint64_t w128 = static_cast<uint64_t>(g.tiles_m) * g.tiles_n * splits * batch;
        const uint64_t w64 = static_cast<uint64_t>(g.tiles_m) * ceil_div(n, 64) * splits * batch;
        if (0.94 * round_fill(w64, 3 * cus) > round_fill(w128, 2 * cus)) {
            g.tiles_n = ceil_div(n, 64);
            const uint64_t f64 = static_cast<uint64_t>(g.tiles_m) * g.tiles_n * splits;
            g.flat_splits = (splits > 1 && f64 <= 0x7fffffffull) ? splits : 0;
            const dim3 grid = g.flat_splits ? dim3(static_cast<uint32_t>(f64), 1, static_cast<uint32_t>(batch))
                                            : dim3(g.tiles_m * g.tiles_n, splits, static_cast<uint32_t>(batch));
            if (amode == KCD)
                hipLaunchKernelGGL((gemm_nn_direct_kernel<false, false, 64>), grid, dim3(256), 0, ctx().stream, g);
            else
                hipLaunchKernelGGL((gemm_nn_direct_kernel<true, false, 64>), grid, dim3(256), 0, ctx().stream, g);
            VKHIP_LAUNCH_CHECK();
            if (splits > 1) { *fused = true; return launch_split_k_reduce(target, c, out_elems, splits, fe); }
            return VKHIP_OK;
        }
        const dim3 grid = dgrid;
        if (amode == KCD)
            hipLaunchKernelGGL((gemm_nn_direct_kernel<false, false>), grid, dim3(256), 0, ctx().stream, g);
        else
            hipLaunchKernelGGL((gemm_nn_direct_kernel<true, false>), grid, dim3(256), 0, ctx().stream, g);
        VKHIP_LAUNCH_CHECK();
        if (splits > 1) { *fused = true; return launch_split_k_reduce(target, c, out_elems, splits, fe); }
        return VKHIP_OK;
    }
    if (tile.bm == 64 && b_rows && (amode == KCD || a_rows)) {
        const dim3 grid = dgrid;
        // Four K-tiles per stage when the grid is one round of one workgroup
        // per CU (its 128 KB of LDS allow no second); one K-tile per stage
        // otherwise, where two workgroups per CU hide each other's waits. With
        // A straight to LDS (NN), a short chunk (2-7 K-tiles: a Linear layer's
        // input gradient at batch 128) loads in one or two stages as well
        // (config 5's fc2 input gradient 13.0 -> 12.4 us); with A transposed
        // the four-tile stage made the fc2 weight gradient slower (5.9 -> 8.5).
        const uint64_t cus = ctx().ready ? static_cast<uint64_t>(ctx().caps.compute_units) : 256u;
        const bool staged = static_cast<uint64_t>(grid.x) * grid.y * grid.z <= cus &&
                            (chunk >= 8 || (chunk >= 2 && amode == KCD));
        void (*kern)(GemmArgs) = amode == KCD ? (staged ? gemm_direct64_kernel<false, 4> : gemm_direct64_kernel<false, 1>)
                                              : (staged ? gemm_direct64_kernel<true, 4> : gemm_direct64_kernel<true, 1>);
        hipLaunchKernelGGL(kern, grid, dim3(256), 0, ctx().stream, g);
        VKHIP_LAUNCH_CHECK();
        if (splits > 1) { *fused = true; return launch_split_k_reduce(target, c, out_elems, splits, fe); }
        return VKHIP_OK;
    }
    g.flat_splits = 0;  // the register-path kernel takes the partition from blockIdx.y
    if (tile.bm == 128)
        st = launch_tiles<128, 128, 64, 64>(g, static_cast<uint32_t>(batch), splits, amode, bmode);
    else
        st = launch_tiles<64, 64, 32, 32>(g, static_cast<uint32_t>(batch), splits, amode, bmode);
    if (st != VKHIP_OK) return st;
    if (splits > 1) { *fused = true; return launch_split_k_reduce(target, c, out_elems, splits, fe); }
    return VKHIP_OK;
}

int gemm(const float* a, const vkhip_operand& ad, const float* b, const vkhip_operand& bd, float* c,
         const vkhip_gemm_opts* opts, const FixedScratch* scratch, const GemmEpilogue* epi) {
    const FoldEpilogue fe = fold_epilogue(epi, bd.ne[3]);
    bool fused = false;
    const int st = gemm_core(a, ad, b, bd, c, opts, scratch, fe, &fused);
    if (st != VKHIP_OK || (!fe.bias && !fe.mask) || fused) return st;
    // no split (or the GEMV, the exact arm, K == 0): the epilogue as a pass
    const uint64_t rows = static_cast<uint64_t>(std::max(ad.ne[0], bd.ne[0])) *
                          std::max(ad.ne[1], bd.ne[1]) * ad.ne[2];
    return launch_bias_cols(c, rows * bd.ne[3], fe);
}

// Convolution forward, out[n] = W_flat (Cout x C*kh*kw) @ cols(x[n]) for every
// image n, as the reference lowers conv2d (ops.cpp:662-705: im2col, then a
// matmul with the flat weight broadcast over the batch), but with the cols
// matrix never written: the B tiles are gathered from the image (Im2colB).
// The plan, tiles, load order into LDS and MFMA sequence are those gemm()
// uses for matmul(flat_weight, cols), so the result is bit-identical to it.
// x: [N, C, H, W] (any strides); w: [Cout, C*kh*kw] as a rank-4 operand
// [1, 1, Cout, CK]; out: contiguous [N, Cout, out_h*out_w].
// ---- implicit-im2col row tables ----------------------------------------------

__global__ __launch_bounds__(256) void conv_row_table_kernel(Im2colB im, int32_t* tab, uint32_t k,
                                                              uint32_t rows) {
    const uint32_t row = blockIdx.x * 256u + threadIdx.x;
    if (row >= rows) return;
    ImgRow q{0, kMaxWindow};
    if (row < k) q = img_row(im, row);
    int32_t* grp = tab + (row / kRowGroup) * (2 * kRowGroup) + row % kRowGroup;
    grp[0] = q.off * 4;
    grp[kRowGroup] = q.r;
}

// Tables depend on K, the window and the image strides only; the most recent
// few are kept (device memory from the caching allocator, stream-ordered like
// every other block) and released at shutdown.
struct RowTableEntry {
    uint32_t k, kh, kw;
    int32_t dilh, dilw, sc, sh, sw;
    int32_t* table;
};
static std::mutex g_tab_mu;
static std::vector<RowTableEntry> g_tabs;
constexpr size_t kMaxRowTables = 32;

// Rows covered: every K-tile plus one, since the loader also reads the tile
// after a partition's last.
static int conv_row_table(Im2colB& im, uint32_t k) {
    std::lock_guard<std::mutex> lk(g_tab_mu);
    for (const RowTableEntry& e : g_tabs)
        if (e.k == k && e.kh == static_cast<uint32_t>(im.kh) && e.kw == static_cast<uint32_t>(im.kw) &&
            e.dilh == im.dilh && e.dilw == im.dilw && e.sc == im.sc && e.sh == im.sh && e.sw == im.sw) {
            im.rows = e.table;
            return VKHIP_OK;
        }
    const uint32_t rows = (ceil_div(k, 32u) + 1) * 32u;
    void* p = nullptr;
    int st = cached_alloc(static_cast<size_t>(rows) * 2 * sizeof(int32_t), &p);
    if (st != VKHIP_OK) return st;
    int32_t* table = static_cast<int32_t*>(p);
    hipLaunchKernelGGL(conv_row_table_kernel, dim3(ceil_div(rows, 256u)), dim3(256), 0, ctx().stream,
                       im, table, k, rows);
    VKHIP_LAUNCH_CHECK();
    // (a captured HIP graph may address every cached table: none is evicted
    // while graphs hold the workspaces)
    if (g_tabs.size() >= kMaxRowTables && !workspaces_pinned()) {
        st = cached_free(g_tabs.front().table);
        g_tabs.erase(g_tabs.begin());
        if (st != VKHIP_OK) return st;
    }
    g_tabs.push_back({k, static_cast<uint32_t>(im.kh), static_cast<uint32_t>(im.kw), im.dilh,
                      im.dilw, im.sc, im.sh, im.sw, table});
    im.rows = table;
    return VKHIP_OK;
}

int release_conv_tables() {
    std::lock_guard<std::mutex> lk(g_tab_mu);
    int st = VKHIP_OK;
    for (const RowTableEntry& e : g_tabs) {
        const int rc = cached_free(e.table);
        if (rc != VKHIP_OK) st = rc;
    }
    g_tabs.clear();
    return st;
}

// Fills the image geometry of an implicit-im2col GEMM; the strides of one
// image must be non-negative and every offset inside it must fit 32 bits.
int make_im2col(const vkhip_unfold& p, uint32_t channels, const int64_t* strides, Im2colB& im) {
    const int64_t oh = (static_cast<int64_t>(p.image_h) + 2 * p.pad_h -
                        (static_cast<int64_t>(p.dilation_h) * (p.kernel_h - 1) + 1)) / p.stride_h + 1;
    const int64_t ow = (static_cast<int64_t>(p.image_w) + 2 * p.pad_w -
                        (static_cast<int64_t>(p.dilation_w) * (p.kernel_w - 1) + 1)) / p.stride_w + 1;
    if (p.kernel_h <= 0 || p.kernel_w <= 0 || p.stride_h <= 0 || p.stride_w <= 0 ||
        p.dilation_h <= 0 || p.dilation_w <= 0 || p.pad_h < 0 || p.pad_w < 0 || oh <= 0 || ow <= 0)
        return fail(VKHIP_ERR_INVALID, "implicit im2col: invalid window geometry");
    const int64_t sc = strides[0], sh = strides[1], sw = strides[2];
    if (sc < 0 || sh < 0 || sw < 0)
        return fail(VKHIP_ERR_UNSUPPORTED, "implicit im2col: negative image strides");
    // The largest magnitude any intermediate offset reaches: window origins
    // run from -pad to (out-1)*stride - pad, displacements up to dil*(k-1).
    const int64_t reach_h = std::max<int64_t>(p.image_h, (oh - 1) * p.stride_h) + p.pad_h +
                            static_cast<int64_t>(p.dilation_h) * p.kernel_h;
    const int64_t reach_w = std::max<int64_t>(p.image_w, (ow - 1) * p.stride_w) + p.pad_w +
                            static_cast<int64_t>(p.dilation_w) * p.kernel_w;
    const int64_t reach = static_cast<int64_t>(channels + 1) * sc + reach_h * sh + reach_w * sw;
    if (reach >= (int64_t{1} << 29))
        return fail(VKHIP_ERR_UNSUPPORTED, "implicit im2col: one image spans 2^29 elements or more");
    if (static_cast<int64_t>(p.kernel_h) * p.kernel_w > kMaxWindow)
        return fail(VKHIP_ERR_UNSUPPORTED, "implicit im2col: window of more than %d elements",
                    kMaxWindow);
    im.sc = static_cast<int32_t>(sc);
    im.sh = static_cast<int32_t>(sh);
    im.sw = static_cast<int32_t>(sw);
    im.H = p.image_h;
    im.W = p.image_w;
    im.kh = p.kernel_h;
    im.kw = p.kernel_w;
    im.kk = p.kernel_h * p.kernel_w;
    im.strh = p.stride_h;
    im.strw = p.stride_w;
    im.padh = p.pad_h;
    im.padw = p.pad_w;
    im.dilh = p.dilation_h;
    im.dilw = p.dilation_w;
    im.ow = static_cast<int32_t>(ow);
    im.div_kk = FastDiv(static_cast<uint32_t>(im.kk));
    im.div_kw = FastDiv(static_cast<uint32_t>(im.kw));
    im.div_ow = FastDiv(static_cast<uint32_t>(ow));
    return VKHIP_OK;
}

// The conv epilogue as its own pass, for plans whose kernel cannot apply it
// (split-K partitions, the exact arm): out[n][c][p] = relu(out + bias[c]).
__global__ __launch_bounds__(256) void conv_bias_relu_kernel(float* __restrict__ out, uint64_t total,
                                                             FastDiv div_l, uint32_t cout,
                                                             const float* __restrict__ bias,
                                                             int64_t bias_stride, uint32_t relu) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        // i / L within 2^32 (checked by the caller), its channel is that mod Cout
        const uint32_t c = div_l.div(static_cast<uint32_t>(i)) % cout;
        float v = out[i];
        if (bias) v = v + bias[static_cast<int64_t>(c) * bias_stride];
        if (relu) v = v <= 0.0f ? 0.0f : v;
        out[i] = v;
    }
}

static int launch_conv_epilogue(float* out, uint64_t total, uint32_t positions, uint32_t cout,
                                const float* bias, int64_t bias_stride, bool relu) {
    if (!bias && !relu) return VKHIP_OK;
    if (total == 0) return VKHIP_OK;
    if (total > 0xffffffffull)
        return fail(VKHIP_ERR_UNSUPPORTED, "conv2d epilogue: output of %llu elements",
                    static_cast<unsigned long long>(total));
    const uint32_t blocks = static_cast<uint32_t>(std::min<uint64_t>((total + 255) / 256, 65536));
    hipLaunchKernelGGL(conv_bias_relu_kernel, dim3(blocks), dim3(256), 0, ctx().stream, out, total,
                       FastDiv(positions), cout, bias, bias_stride, relu ? 1u : 0u);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

// ---- weight gradient of a small window (C*kh*kw <= 32, Cout <= 64) ----------
// The 3-channel first layer's product, [Cout, L] x [L, 27] per image, pads a
// GEMM tile to 6-10% use, and its K (positions) is all there is: the layer is
// bound by the gradient's bytes, not by the matrix cores. Here a workgroup of
// eight waves takes a run of K-tiles (32 positions each) of one image, which
// it first stages whole in LDS (padded pitches, stage_image; at most 8192
// floats); each wave
// owns consecutive K-tiles and both 32-row blocks of Cout: its A operand is
// the gradient rows read straight into registers (16 consecutive positions
// per lane, four 16-byte loads), its B operand the columns' window element of
// that position read from the staged image (0 in the padding or past C*kh*kw),
// shared by the two blocks' MFMAs. Each wave's partial keeps the MFMA order of
// the GEMM kernels over its K-tiles; the eight partials are summed in LDS as a
// balanced tree over consecutive waves ((w0+w1)+(w2+w3))+((w4+w5)+(w6+w7)).
//   FOLD = false: one workgroup per image, out[n] = its sum.
//   FOLD = true:  the batch-summed gradient with K = N*L: workgroup b takes
//                 K-tiles [b*kpw, (b+1)*kpw) (within one image) and writes
//                 partial b; the split-K carry-stack fold sums the partials.
// Deterministic for a given shape (fixed partition and summation order);
// within the GEMM tolerance of the lowering, not its bits.
constexpr int kSmallWgradWaves = 8;
constexpr int kSmallWgradLds = 8192;  // floats: the staged image, then 4 wave partials

// Image n into LDS as [C][H][W] with a row pitch of `wp` and a channel pitch
// of `cp` floats (element (c, h, w) at c*cp + h*wp + w). The pitches spread a
// window's elements over the LDS banks: for a 3x3 window over three channels
// the 27 elements one position reads land on 27 distinct banks (wp = 4 mod 64
// gives rows 0, 36 and 72 = 8; cp = 16 mod 64 moves channels by 16 banks).
// Eight loads per thread are issued before their LDS stores, so a stage of up
// to 8 * blockDim elements waits for memory once.
struct StagePitch {
    int32_t wp, cp;
    FastDiv div_hw, div_w;  // by H*W and W
};
__host__ inline StagePitch stage_pitch(int H, int W) {
    StagePitch s;
    s.wp = ((W + 3) & ~3) + 4;
    const int plane = H * s.wp;
    s.cp = ((plane + 47) / 64) * 64 + 16;  // the first value >= plane that is 16 mod 64
    s.div_hw = FastDiv(static_cast<uint32_t>(H * W));
    s.div_w = FastDiv(static_cast<uint32_t>(W));
    return s;
}
__host__ inline uint64_t stage_floats(const StagePitch& s, int chans) {
    return static_cast<uint64_t>(chans) * static_cast<uint64_t>(s.cp);
}
__device__ __forceinline__ void stage_image(float* lds, const Im2colB& im, uint32_t n, uint32_t elems,
                                            const StagePitch& sp) {
    const float* xn = im.x + static_cast<int64_t>(n) * im.sn;
    for (uint32_t e0 = threadIdx.x; e0 < elems; e0 += 8 * blockDim.x) {
        float v[8];
        int32_t at[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t e = e0 + u * blockDim.x;
            const uint32_t ec = e < elems ? e : 0u;
            const uint32_t c = sp.div_hw.div(ec), r = ec - c * sp.div_hw.d, h = sp.div_w.div(r),
                           w = r - h * sp.div_w.d;
            v[u] = xn[static_cast<int32_t>(c) * im.sc + static_cast<int32_t>(h) * im.sh +
                      static_cast<int32_t>(w) * im.sw];
            at[u] = static_cast<int32_t>(c) * sp.cp + static_cast<int32_t>(h) * sp.wp + static_cast<int32_t>(w);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (e0 + u * blockDim.x < elems) lds[at[u]] = v[u];
    }
}

template <bool FOLD>
__global__ __launch_bounds__(64 * kSmallWgradWaves) void conv_wgrad_small_kernel(GemmArgs g, Im2colB im,
                                                                                 uint32_t kpw,
                                                                                 uint32_t per_wave,
                                                                                 StagePitch sp) {
    __shared__ __attribute__((aligned(16))) float lds[kSmallWgradLds];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, kh = lane >> 5;
    const uint32_t tpi = im.L / 32;  // K-tiles per image
    const uint32_t first = blockIdx.x * kpw;
    const uint32_t n = FOLD ? first / tpi : blockIdx.x;
    const uint32_t t0 = FOLD ? first - n * tpi : 0u;
    const int chans = static_cast<int>(g.n) / im.kk;

    // this lane's column j = lrow: channel c, window element (ki, kj); its
    // element of position (oh, ow) is at off + oh*strh*wp + ow*strw when
    // inside the image
    const uint32_t j = static_cast<uint32_t>(lrow);
    const bool jok = j < g.n;
    const uint32_t jc = jok ? j : 0u;
    const uint32_t c = jc / static_cast<uint32_t>(im.kk);
    const uint32_t r = jc - c * static_cast<uint32_t>(im.kk);
    const uint32_t ki = r / static_cast<uint32_t>(im.kw), kj = r - ki * static_cast<uint32_t>(im.kw);
    // (lanes past C*kh*kw get a row far above the image, so that their 'in'
    // test fails; their offset is not formed from it)
    const int fh = jok ? static_cast<int>(ki) * im.dilh - im.padh : -(1 << 20);
    const int fw = static_cast<int>(kj) * im.dilw - im.padw;
    const int off = jok ? static_cast<int>(c) * sp.cp + fh * sp.wp + fw : 0;
    const int sth = im.strh * sp.wp;

    // the gradient rows of this lane in the two Cout blocks (rows past Cout
    // read the last row: their outputs are never stored)
    const float* gn = g.a + static_cast<int64_t>(n) * g.sa1;
    const float* arow0 = gn + static_cast<int64_t>(min(static_cast<uint32_t>(lrow), g.m - 1)) * g.sam + 16 * kh;
    const float* arow1 = gn + static_cast<int64_t>(min(static_cast<uint32_t>(32 + lrow), g.m - 1)) * g.sam + 16 * kh;

    f32x16 acc0, acc1;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        acc0[i] = 0.0f;
        acc1[i] = 0.0f;
    }
    const uint32_t w0 = t0 + static_cast<uint32_t>(wave) * per_wave;
    const uint32_t w1 = min(t0 + kpw, w0 + per_wave);
    // The gradient rows of K-tile t go one tile ahead of its MFMAs (the first
    // tile's ahead of the image staging), so their memory latency overlaps.
    f32x4 a0[4], a1[4];
    auto load_a = [&](uint32_t t) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            a0[q] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(arow0 + t * 32 + 4 * q));
            a1[q] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(arow1 + t * 32 + 4 * q));
        }
    };
    if (w0 < w1) load_a(w0);
    stage_image(lds, im, n, static_cast<uint32_t>(chans * im.H * im.W), sp);
    __syncthreads();
    for (uint32_t t = w0; t < w1; ++t) {
        const uint32_t p0 = t * 32;
        f32x4 c0[4], c1[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            c0[q] = a0[q];
            c1[q] = a1[q];
        }
        if (t + 1 < w1) load_a(t + 1);
        // the window element of positions p0 + 16*kh + i, i = 0..15
        const uint32_t p = p0 + 16 * kh;
        uint32_t oh = im.div_ow.div(p);
        uint32_t ow = p - oh * static_cast<uint32_t>(im.ow);
        float bv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int h = static_cast<int>(oh) * im.strh + fh, w = static_cast<int>(ow) * im.strw + fw;
            const bool in = (static_cast<uint32_t>(h) < static_cast<uint32_t>(im.H)) &
                            (static_cast<uint32_t>(w) < static_cast<uint32_t>(im.W));
            const float v = lds[in ? off + static_cast<int>(oh) * sth + static_cast<int>(ow) * im.strw : 0];
            bv[i] = in ? v : 0.0f;
            if (++ow == static_cast<uint32_t>(im.ow)) {
                ow = 0;
                ++oh;
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(c0[q][st], bv[4 * q + st], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(c1[q][st], bv[4 * q + st], acc1, 0, 0, 0);
            }
    }

    // balanced tree over consecutive waves: at step s the wave w with
    // w % 2s == s hands its partial to w - s, which adds it to its own
    __syncthreads();  // every wave is done with the staged image
#pragma unroll
    for (int s = 1; s < kSmallWgradWaves; s *= 2) {
        float* slot = lds + (wave / (2 * s)) * 2048;
        if ((wave & (2 * s - 1)) == s) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                slot[i * 64 + lane] = acc0[i];
                slot[1024 + i * 64 + lane] = acc1[i];
            }
        }
        __syncthreads();
        if ((wave & (2 * s - 1)) == 0) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                acc0[i] = acc0[i] + slot[i * 64 + lane];
                acc1[i] = acc1[i] + slot[1024 + i * 64 + lane];
            }
        }
        __syncthreads();
    }
    if (wave != 0 || !jok) return;
    // register i of lane l: row 8*(i/4) + 4*(l/32) + i%4 of its block, column l%32
    float* dst = g.c + static_cast<uint64_t>(blockIdx.x) * g.m * g.n;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t row = 8 * (i / 4) + 4 * kh + (i % 4);
        if (row < g.m) dst[static_cast<uint64_t>(row) * g.n + j] = acc0[i];
        if (row + 32 < g.m) dst[static_cast<uint64_t>(row + 32) * g.n + j] = acc1[i];
    }
}

// Whether conv_wgrad_small_kernel takes a weight gradient: C*kh*kw <= 32,
// Cout <= 64, whole K-tiles per image, the image fits the stage, and the
// gradient rows are 16-byte aligned.
static bool wgrad_small_fits(const float* gr, const vkhip_operand& gd, uint64_t ck, uint32_t cout,
                             uint64_t L, const Im2colB& im, uint32_t chans) {
    return ck >= 1 && ck <= 32 && cout >= 1 && cout <= 64 && L % 32 == 0 && L >= 32 &&
           L <= 0x7fffffffull &&
           stage_floats(stage_pitch(im.H, im.W), static_cast<int>(chans)) <= static_cast<uint64_t>(kSmallWgradLds) &&
           reinterpret_cast<uintptr_t>(gr) % 16 == 0 && gd.nb[1] >= 0 && gd.nb[2] >= 0 &&
           gd.nb[1] % 4 == 0 && gd.nb[2] % 4 == 0;
}

// Launch: FOLD writes `parts` partials of Cout*ck floats to `ws`, else out
// [N][Cout][ck] directly.
static int launch_wgrad_small(bool fold, const float* gr, const vkhip_operand& gd, Im2colB im,
                              uint32_t cout, uint32_t ck, uint32_t batch, uint32_t kpw, float* dst) {
    GemmArgs g{};
    g.a = gr;
    g.sa1 = gd.nb[1];
    g.sam = gd.nb[2];
    g.m = cout;
    g.n = ck;
    g.c = dst;
    const uint32_t tpi = im.L / 32;
    const uint32_t per_wave = ceil_div(kpw, static_cast<uint32_t>(kSmallWgradWaves));
    const uint32_t blocks = fold ? static_cast<uint32_t>(static_cast<uint64_t>(batch) * tpi / kpw) : batch;
    const StagePitch sp = stage_pitch(im.H, im.W);
    if (fold)
        hipLaunchKernelGGL(conv_wgrad_small_kernel<true>, dim3(blocks), dim3(64 * kSmallWgradWaves), 0,
                           ctx().stream, g, im, kpw, per_wave, sp);
    else
        hipLaunchKernelGGL(conv_wgrad_small_kernel<false>, dim3(blocks), dim3(64 * kSmallWgradWaves), 0,
                           ctx().stream, g, im, kpw, per_wave, sp);
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

// ---- small-window convolution staging ---------------------------------------
// The image geometry and LDS staging shared by the small-window weight-gradient
// kernels below (windows of at most 32 elements, at most 64 output channels;
// the forward of such layers runs win_fwd_kernel, conv_small.hip).
constexpr int kSmallFwdLds = 8192;  // floats of staged (zero-bordered) image

struct SmallConvFwd {
    const float* x;
    int64_t sn, sc, sh, sw;  // image strides (elements)
    const float* w;
    int64_t wrow;  // weight row stride (elements; k stride 1)
    const float* bias;
    int64_t bias_stride;
    uint32_t relu;
    float* out;
    int32_t C, H, W, kw, kk, strh, strw, padh, padw, dilh, dilw, OW;
    int32_t Hp, Wp, plane;  // staged plane: (H + 2 padh) x (W + 2 padw), plane = Hp * Wp
    uint32_t cout, K, L, nblk;
    uint32_t wg_per_image, blocks_per_wg;
    FastDiv div_ow, div_plane, div_wp;
    int32_t offs[32];  // staged-image offset of window element j (c*plane + ki*dilh*Wp + kj*dilw)
    uint32_t w_flat4;  // weights [Cout][K] contiguous, 16-byte aligned, Cout*K % 4 == 0
    int32_t rows;      // forward: padded input rows staged per channel (plane = rows * Wp)
};

// Staging of image n, zero-bordered by the padding, into lds[0 .. C*plane),
// plus a zero at lds[C*plane] that masked window elements read. Split into
// the loads (U per thread, NT threads, every one issued before any is used;
// addresses clamped into the image and the border selected afterwards, so the
// sequence has no branches) and the LDS stores, so that a kernel can issue
// other loads in between and wait for the staging alone.
template <int NT, int U>
__device__ __forceinline__ void stage_load(float (&v)[U], const SmallConvFwd& p, uint32_t n, int tid) {
    const float* xn = p.x + static_cast<int64_t>(n) * p.sn;
    const uint32_t staged = static_cast<uint32_t>(p.C * p.plane);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t e = static_cast<uint32_t>(tid) + static_cast<uint32_t>(NT) * u;
        const uint32_t ec = e < staged ? e : 0u;
        const uint32_t c = p.div_plane.div(ec), r = ec - c * p.div_plane.d;
        const uint32_t hh = p.div_wp.div(r), ww = r - hh * p.div_wp.d;
        const int h = static_cast<int>(hh) - p.padh, w = static_cast<int>(ww) - p.padw;
        const bool in = e < staged && static_cast<uint32_t>(h) < static_cast<uint32_t>(p.H) &&
                        static_cast<uint32_t>(w) < static_cast<uint32_t>(p.W);
        const int hc = min(max(h, 0), p.H - 1), wc = min(max(w, 0), p.W - 1);
        const float x = xn[static_cast<int64_t>(c) * p.sc + static_cast<int64_t>(hc) * p.sh +
                           static_cast<int64_t>(wc) * p.sw];
        v[u] = in ? x : 0.0f;
    }
}

template <int NT, int U>
__device__ __forceinline__ void stage_store(float* lds, const float (&v)[U], const SmallConvFwd& p, int tid) {
    const uint32_t staged = static_cast<uint32_t>(p.C * p.plane);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t e = static_cast<uint32_t>(tid) + static_cast<uint32_t>(NT) * u;
        if (e < staged) lds[e] = v[u];
    }
    if (tid == 0) lds[staged] = 0.0f;
}

// ---- small-window convolution weight gradient, summed over the batch ----------
// dW[co][j] = sum over images n and positions p of g[n][co][p] * window
// element j of image n at p, for windows of at most 32 elements and at most 64
// output channels (CIFAR conv1: 64 x 27 outputs, K = 128 images x 1024
// positions). The product is bound by reading the output gradient once
// (33.5 MB), so the kernel streams it: each of a workgroup's 8 waves owns BPW
// 32-position blocks of one image and issues all their gradient loads before
// anything else, then the workgroup stages the image (zero-bordered) in LDS,
// and each wave runs 16 MFMA steps per block and channel tile, the lane of
// window element j gathering j's values from LDS. The 8 waves' sums are added
// in wave order through LDS and each workgroup writes one partial of
// Cout x C*kh*kw; the carry-stack fold (split_k_reduce_kernel) adds the
// partials in workgroup order. Fixed orders throughout: the result is the same
// bits on every run (within the GEMM tolerance of the per-image graph, whose
// sums run in another order).
constexpr int kWgradStreamWaves = 8;
constexpr int kWgradStreamLds = 16384;  // floats: the staged image, then the 8 waves' sums

template <int T, int BPW, int U>
__global__ __launch_bounds__(64 * kWgradStreamWaves) void conv_wgrad_stream_kernel(
    SmallConvFwd p, const float* __restrict__ g, int64_t gsn, int64_t gsc, float* __restrict__ ws) {
    __shared__ __attribute__((aligned(16))) float lds[kWgradStreamLds];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, kh = lane >> 5;
    const uint32_t n = blockIdx.x / p.wg_per_image;
    const uint32_t part = blockIdx.x - n * p.wg_per_image;
    const uint32_t b0 = part * p.blocks_per_wg;
    const uint32_t b1 = min(p.nblk, b0 + p.blocks_per_wg);

    // this lane's window element j = lrow, its offset in the staged image (the
    // staged zero past K), and the image's loads: issued first, so that the
    // staging waits for them alone while the gradient's loads below stay in
    // flight
    const bool jok = static_cast<uint32_t>(lrow) < p.K;
    const int32_t my_off = p.offs[lrow];
    float sv[U];
    stage_load<64 * kWgradStreamWaves, U>(sv, p, n, tid);

    // the gradient rows of this lane's channels (rows past Cout read the last
    // row; their sums are never stored), positions 16*kh .. 16*kh + 15 of each
    // block
    const float* gn = g + static_cast<int64_t>(n) * gsn;
    const float* grow[T];
#pragma unroll
    for (int i = 0; i < T; ++i)
        grow[i] = gn + static_cast<int64_t>(min(32u * i + lrow, p.cout - 1u)) * gsc + 16 * kh;
    f32x4 ga[BPW][T][4];
#pragma unroll
    for (int u = 0; u < BPW; ++u) {
        const uint32_t b = b0 + wave + kWgradStreamWaves * u;
        const uint32_t bc = b < b1 ? b : b0;
#pragma unroll
        for (int i = 0; i < T; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                ga[u][i][q] = __builtin_nontemporal_load(
                    reinterpret_cast<const f32x4*>(grow[i] + 32u * bc + 4 * q));
    }
    stage_store<64 * kWgradStreamWaves, U>(lds, sv, p, tid);
    const int32_t off = jok ? my_off : -1;
    const int32_t zslot = p.C * p.plane;
    __syncthreads();

    f32x16 acc[T];
#pragma unroll
    for (int i = 0; i < T; ++i)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[i][q] = 0.0f;
#pragma unroll
    for (int u = 0; u < BPW; ++u) {
        const uint32_t b = b0 + wave + kWgradStreamWaves * u;
        if (b >= b1) break;
        // positions 32b + 16kh + t, t = 0..15, walked along the output rows
        const uint32_t p0 = 32u * b + 16u * kh;
        uint32_t oh = p.div_ow.div(p0), ow = p0 - oh * static_cast<uint32_t>(p.OW);
        float bv[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const int32_t base = static_cast<int32_t>(oh) * p.strh * p.Wp + static_cast<int32_t>(ow) * p.strw;
            bv[t] = lds[off >= 0 ? base + off : zslot];
            if (++ow == static_cast<uint32_t>(p.OW)) {
                ow = 0;
                ++oh;
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int st = 0; st < 4; ++st)
#pragma unroll
                for (int i = 0; i < T; ++i)
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(ga[u][i][q][st], bv[4 * q + st], acc[i], 0, 0, 0);
    }

    // the 8 waves' sums, added in wave order
    __syncthreads();  // every wave is done with the staged image
#pragma unroll
    for (int i = 0; i < T; ++i)
#pragma unroll
        for (int q = 0; q < 16; ++q) lds[((wave * T + i) * 16 + q) * 64 + lane] = acc[i][q];
    __syncthreads();
    float* dst = ws + static_cast<uint64_t>(blockIdx.x) * p.cout * p.K;
#pragma unroll
    for (int e = tid; e < T * 1024; e += 64 * kWgradStreamWaves) {
        const int i = e >> 10, q = (e >> 6) & 15, ln = e & 63;
        float sum = lds[((0 * T + i) * 16 + q) * 64 + ln];
#pragma unroll
        for (int v = 1; v < kWgradStreamWaves; ++v) sum = sum + lds[((v * T + i) * 16 + q) * 64 + ln];
        const uint32_t co = 32u * i + 8 * (q / 4) + 4 * (ln >> 5) + (q % 4);
        const uint32_t jj = static_cast<uint32_t>(ln & 31);
        if (co < p.cout && jj < p.K) dst[static_cast<uint64_t>(co) * p.K + jj] = sum;
    }
}

// The image geometry of the small-window kernels (weights and epilogue unset).
static SmallConvFwd small_conv_geometry(const float* x, const vkhip_operand& xd, const vkhip_unfold& pr,
                                        uint32_t channels, uint32_t cout, uint32_t ck, uint32_t oh,
                                        uint32_t ow) {
    SmallConvFwd p{};
    p.x = x;
    p.sn = xd.nb[0];
    p.sc = xd.nb[1];
    p.sh = xd.nb[2];
    p.sw = xd.nb[3];
    p.C = static_cast<int32_t>(channels);
    p.H = pr.image_h;
    p.W = pr.image_w;
    p.kw = pr.kernel_w;
    p.kk = pr.kernel_h * pr.kernel_w;
    p.strh = pr.stride_h;
    p.strw = pr.stride_w;
    p.padh = pr.pad_h;
    p.padw = pr.pad_w;
    p.dilh = pr.dilation_h;
    p.dilw = pr.dilation_w;
    p.OW = static_cast<int32_t>(ow);
    p.Hp = pr.image_h + 2 * pr.pad_h;
    p.Wp = pr.image_w + 2 * pr.pad_w;
    p.plane = p.Hp * p.Wp;
    p.cout = cout;
    p.K = ck;
    p.L = oh * ow;
    p.nblk = ceil_div(p.L, 32u);
    p.div_ow = FastDiv(ow);
    p.div_plane = FastDiv(static_cast<uint32_t>(p.plane));
    p.div_wp = FastDiv(static_cast<uint32_t>(p.Wp));
    for (uint32_t j = 0; j < 32; ++j) {
        const uint32_t jc = j < ck ? j : 0u;
        const uint32_t c = jc / static_cast<uint32_t>(p.kk), r = jc % static_cast<uint32_t>(p.kk);
        const uint32_t ki = r / static_cast<uint32_t>(p.kw), kj = r % static_cast<uint32_t>(p.kw);
        p.offs[j] = static_cast<int32_t>(c) * p.plane + static_cast<int32_t>(ki) * p.dilh * p.Wp +
                    static_cast<int32_t>(kj) * p.dilw;
    }
    return p;
}

// Whether conv_wgrad_stream_kernel takes a batch-summed weight gradient:
// C*kh*kw <= 32, Cout <= 64, whole 32-position blocks, unit-stride positions
// with 16-byte aligned gradient rows, the zero-bordered image fits the stage.
static bool wgrad_stream_fits(const float* gr, const vkhip_operand& gd, const vkhip_unfold& pr,
                              uint32_t channels, uint64_t ck, uint32_t cout, uint64_t L) {
    const int64_t hp = static_cast<int64_t>(pr.image_h) + 2 * pr.pad_h;
    const int64_t wp = static_cast<int64_t>(pr.image_w) + 2 * pr.pad_w;
    return ck >= 1 && ck <= 32 && cout >= 1 && cout <= 64 && L % 32 == 0 && L >= 32 &&
           L <= 0x7fffffffull && static_cast<int64_t>(channels) * hp * wp < kSmallFwdLds &&
           reinterpret_cast<uintptr_t>(gr) % 16 == 0 && gd.nb[3] == 1 && gd.nb[1] >= 0 &&
           gd.nb[2] >= 0 && gd.nb[1] % 4 == 0 && gd.nb[2] % 4 == 0;
}

// Partials of the streamed weight gradient: each workgroup 8*BPW blocks of one
// image, BPW the smallest of 1, 2, 4 that keeps the partials at most 511 (the
// fold's limit); 0 when none does.
static uint32_t wgrad_stream_bpw(uint64_t batch, uint32_t nblk, uint64_t& parts) {
    for (uint32_t bpw = 1; bpw <= 4; bpw *= 2) {
        parts = batch * ceil_div(nblk, kWgradStreamWaves * bpw);
        if (parts <= 511) return bpw;
    }
    return 0;
}

static int launch_conv_wgrad_stream(SmallConvFwd p, const float* gr, const vkhip_operand& gd,
                                    uint32_t batch, uint32_t bpw, float* ws) {
    p.blocks_per_wg = kWgradStreamWaves * bpw;
    p.wg_per_image = ceil_div(p.nblk, p.blocks_per_wg);
    const dim3 grid(batch * p.wg_per_image);
    const dim3 block(64 * kWgradStreamWaves);
    const bool two = p.cout > 32;
    const uint32_t rounds = ceil_div(static_cast<uint32_t>(p.C * p.plane), 64u * kWgradStreamWaves);
#define VKHIP_WGS(T, B, U) \
    hipLaunchKernelGGL((conv_wgrad_stream_kernel<T, B, U>), grid, block, 0, ctx().stream, p, gr, gd.nb[1], gd.nb[2], ws)
#define VKHIP_WGS_U(T, B) \
    do { if (rounds <= 4) VKHIP_WGS(T, B, 4); else if (rounds <= 8) VKHIP_WGS(T, B, 8); else VKHIP_WGS(T, B, 16); } while (0)
    if (bpw == 1) {
        if (two) VKHIP_WGS_U(2, 1); else VKHIP_WGS_U(1, 1);
    } else if (bpw == 2) {
        if (two) VKHIP_WGS_U(2, 2); else VKHIP_WGS_U(1, 2);
    } else {
        if (two) VKHIP_WGS_U(2, 4); else VKHIP_WGS_U(1, 4);
    }
#undef VKHIP_WGS_U
#undef VKHIP_WGS
    VKHIP_LAUNCH_CHECK();
    return VKHIP_OK;
}

int conv2d_forward(const float* x, const vkhip_operand& xd, const float* w,
                   const vkhip_operand& wd, float* out, const vkhip_unfold& p, const float* bias,
                   int64_t bias_stride, bool relu) {
    if (p.kernel_h <= 0 || p.kernel_w <= 0 || p.stride_h <= 0 || p.stride_w <= 0 ||
        p.dilation_h <= 0 || p.dilation_w <= 0 || p.pad_h < 0 || p.pad_w < 0)
        return fail(VKHIP_ERR_INVALID, "conv2d: invalid window geometry");
    if (static_cast<int64_t>(xd.ne[2]) != p.image_h || static_cast<int64_t>(xd.ne[3]) != p.image_w)
        return fail(VKHIP_ERR_INVALID, "conv2d: image is %ux%u but the geometry says %dx%d",
                    xd.ne[2], xd.ne[3], p.image_h, p.image_w);
    const int64_t oh = (static_cast<int64_t>(p.image_h) + 2 * p.pad_h -
                        (static_cast<int64_t>(p.dilation_h) * (p.kernel_h - 1) + 1)) / p.stride_h + 1;
    const int64_t ow = (static_cast<int64_t>(p.image_w) + 2 * p.pad_w -
                        (static_cast<int64_t>(p.dilation_w) * (p.kernel_w - 1) + 1)) / p.stride_w + 1;
    if (oh <= 0 || ow <= 0) return fail(VKHIP_ERR_INVALID, "conv2d: window larger than padded image");
    const uint64_t batch = static_cast<uint64_t>(xd.ne[0]);
    const uint32_t channels = xd.ne[1];
    const uint64_t ck = static_cast<uint64_t>(channels) * p.kernel_h * p.kernel_w;
    if (wd.ne[0] != 1 || wd.ne[1] != 1 || static_cast<uint64_t>(wd.ne[3]) != ck)
        return fail(VKHIP_ERR_INVALID, "conv2d: weight must be [Cout, C*kh*kw] with C*kh*kw = %llu",
                    static_cast<unsigned long long>(ck));
    const uint64_t L = static_cast<uint64_t>(oh) * ow;
    if (L > 0xffffffffull || ck > 0xffffffffull || batch > 65535)
        return fail(VKHIP_ERR_UNSUPPORTED, "conv2d: extents too large");
    const uint32_t m = wd.ne[2], n = static_cast<uint32_t>(L), k = static_cast<uint32_t>(ck);
    if (batch == 0 || m == 0 || n == 0) return VKHIP_OK;
    if (k == 0) {
        const int st = launch_zero_f32(out, batch * m * n);
        if (st != VKHIP_OK) return st;
        return launch_conv_epilogue(out, batch * m * n, n, m, bias, bias_stride, relu);
    }
    if (ctx().exact_math) {
        // the exact arm with the columns gathered from the image: the oracle's
        // im2col + matmul, bit for bit
        publish("matmul.kernel", "conv2d", "gemm_exact_implicit_im2col", "gemm_mfma_implicit_im2col",
                "exact numerics mode", static_cast<int64_t>(k), static_cast<int64_t>(m) * n);
        if (wd.nb[3] != 1 && k != 1)
            return fail(VKHIP_ERR_UNSUPPORTED, "conv2d: the weight rows must be contiguous");
        ExactImg im{};
        const int geo = exact_img(p, x, xd, im);
        if (geo != VKHIP_OK) return geo;
        GemmArgs g{};
        g.a = w;
        g.b = x;
        g.sam = wd.nb[2];
        g.sak = 1;
        g.b1 = static_cast<uint32_t>(batch);
        g.m = m;
        g.n = n;
        g.k = k;
        g.c = out;
        const int st = launch_exact(g, static_cast<uint32_t>(batch), B_IMG, im);
        if (st != VKHIP_OK) return st;
        return launch_conv_epilogue(out, batch * m * n, n, m, bias, bias_stride, relu);
    }
    if (win_fwd_fits(xd, p, channels, k, m, wd, static_cast<uint32_t>(oh), static_cast<uint32_t>(ow))) {
        publish("matmul.kernel", "conv2d", "win_fwd", "gemm_mfma_implicit_im2col",
                "a window of at most 32 elements and at most 64 output channels: one K-tile per output",
                static_cast<int64_t>(k), static_cast<int64_t>(m));
        return win_conv_forward(x, xd, w, wd, out, p, static_cast<uint32_t>(batch), channels, m, k,
                                static_cast<uint32_t>(oh), static_cast<uint32_t>(ow), bias, bias_stride, relu);
    }
    uint32_t splits, chunk;
    TileChoice tile;
    gemm_plan(static_cast<uint32_t>(batch), m, n, k, 0, splits, chunk, tile);
    publish("matmul.kernel", "conv2d", tile.bm == 128 ? "gemm_mfma_128x128_implicit_im2col"
                                                      : "gemm_mfma_64x64_implicit_im2col",
            "im2col_then_gemm", "the cols matrix is gathered from the image inside the GEMM",
            static_cast<int64_t>(tile.tiles), ctx().ready ? ctx().caps.compute_units : 256);

    GemmArgs g{};
    g.a = w;
    g.b = nullptr;
    g.sa0 = 0;
    g.sa1 = 0;
    g.sam = wd.nb[2];
    g.sak = wd.nb[3];
    g.b1 = static_cast<uint32_t>(batch);
    g.m = m;
    g.n = n;
    g.k = k;
    g.tiles_m = ceil_div(m, tile.bm);
    g.tiles_n = ceil_div(n, tile.bn);
    g.ktiles = ceil_div(k, 32);
    g.chunk = chunk;
    if (wd.nb[3] != 1 && k != 1)
        return fail(VKHIP_ERR_UNSUPPORTED, "conv2d: the weight rows must be contiguous");
    g.sak = 1;
    // 16-byte weight loads when every row starts 16-byte aligned and holds
    // whole groups of four.
    g.a_vec = reinterpret_cast<uintptr_t>(w) % 16 == 0 && g.sam % 4 == 0 && k % 4 == 0;

    Im2colB im{};
    const int geo = make_im2col(p, channels, xd.nb + 1, im);
    if (geo != VKHIP_OK) return geo;
    im.x = x;
    im.sn = xd.nb[0];
    {
        const int rc = conv_row_table(im, k);
        if (rc != VKHIP_OK) return rc;
    }

    const uint64_t out_elems = batch * m * n;
    float* target = out;
    if (splits > 1) {
        float* ws = nullptr;
        int st = workspace(out_elems * splits * sizeof(float), &ws);
        if (st != VKHIP_OK) return st;
        target = ws;
        g.split_stride = out_elems;
    }
    g.c = target;
    if (splits == 1) {  // the kernel applies the epilogue (split plans: after the fold)
        g.bias = bias;
        g.bias_stride = bias_stride;
        g.relu = relu ? 1u : 0u;
    }
    // The weights or gradient rows straight into LDS when the KCD loader's
    // conditions hold (K a multiple of four, 16-byte aligned rows: a_vec;
    // byte offsets within 2^31), else through registers.
    const bool a_kcd = g.a_vec && g.sam >= 0 &&
                       ((static_cast<int64_t>(m) - 1) * g.sam + k) * 4 < (int64_t{1} << 31);
    const int amode = a_kcd ? KCD : (g.a_vec ? KCV : KCS);
    int st;
    // 128x64 tiles when their rounds fill the machine better (two workgroups
    // per CU either way: 70 and 55 KB of LDS; 0.94 for the narrower tile's
    // work per CU-second, as for the GEMM): the CIFAR conv2 layer's 256 tiles
    // of 128x128 give each CU one workgroup, 512 of 128x64 two (0.0556 ->
    // 0.0493 ms); [128,64,32,32] -> 128 keeps 128x128 (0.172 against 0.190).
    // Tile width never changes the bits.
    const uint64_t cus = ctx().ready ? static_cast<uint64_t>(ctx().caps.compute_units) : 256u;
    const uint64_t w128 = static_cast<uint64_t>(g.tiles_m) * g.tiles_n * splits * batch;
    const uint64_t w64 = static_cast<uint64_t>(g.tiles_m) * ceil_div(n, 64) * splits * batch;
    if (tile.bm == 128 && 0.94 * round_fill(w64, 2 * cus) > round_fill(w128, 2 * cus)) {
        g.tiles_n = ceil_div(n, 64);
        st = launch_conv_tiles<128, 64, 64, 32, IMG>(g, im, static_cast<uint32_t>(batch), splits, amode);
    } else if (tile.bm == 128)
        st = launch_conv_tiles<128, 128, 64, 64, IMG>(g, im, static_cast<uint32_t>(batch), splits, amode);
    else
        st = launch_conv_tiles<64, 64, 32, 32, IMG>(g, im, static_cast<uint32_t>(batch), splits, amode);
    if (st != VKHIP_OK) return st;
    if (splits > 1) {
        st = launch_split_k_reduce(target, out, out_elems, splits);
        if (st != VKHIP_OK) return st;
        return launch_conv_epilogue(out, out_elems, n, m, bias, bias_stride, relu);
    }
    return VKHIP_OK;
}


// The weight gradient's per-image products, dW[n] = g[n] (Cout x L) @
// im2col(x[n])^T (L x C*kh*kw), as one GEMM per image whose B operand is
// gathered from the image (load mode IMGT): what the reference's conv2d
// backward computes as matmul(grad, cols^T) on the materialised columns
// (autograd.cpp:548-553 through ops.cpp:662-705), with the same plan, K order
// and split-K fold, hence the same bits. x: [N,C,H,W] any strides; g: [N,
// Cout, L] with unit position stride; out contiguous [N, Cout, C*kh*kw].
// Whether conv_direct_kernel runs 128x64 tiles: the rule gemm() applies to
// its direct kernels (three 128x64 workgroups per CU against two 128x128,
// 0.94 for the narrower tile's work per CU-second, the fill of the launch's
// rounds deciding). The tile width does not change the bits.
static bool wgrad_narrow_tiles(const GemmArgs& g, uint32_t splits, uint64_t batch) {
    const uint64_t cus = ctx().ready ? static_cast<uint64_t>(ctx().caps.compute_units) : 256u;
    const uint64_t w128 = static_cast<uint64_t>(g.tiles_m) * g.tiles_n * splits * batch;
    const uint64_t w64 = static_cast<uint64_t>(g.tiles_m) * ceil_div(g.n, 64u) * splits * batch;
    return 0.94 * round_fill(w64, 3 * cus) > round_fill(w128, 2 * cus);
}

// Whether conv_direct_kernel takes a weight-gradient product: 128x128
// tiles, the gradient rows 16-byte aligned with whole groups of four
// positions, and every byte offset of one image's gradient within 2^31.
static bool wgrad_direct_fits(const GemmArgs& g, uint32_t positions, const float* target) {
    return reinterpret_cast<uintptr_t>(g.a) % 16 == 0 && reinterpret_cast<uintptr_t>(target) % 16 == 0 &&
           g.sam >= 0 && g.sa1 >= 0 && g.sam % 4 == 0 && g.sa1 % 4 == 0 && positions % 4 == 0 &&
           ((static_cast<int64_t>(g.m) - 1) * g.sam + positions) * 4 < (int64_t{1} << 31);
}

int conv2d_weight_grad(const float* x, const vkhip_operand& xd, const float* gr,
                       const vkhip_operand& gd, float* out, const vkhip_unfold& p) {
    if (static_cast<int64_t>(xd.ne[2]) != p.image_h || static_cast<int64_t>(xd.ne[3]) != p.image_w)
        return fail(VKHIP_ERR_INVALID, "conv2d weight grad: image is %ux%u but the geometry says %dx%d",
                    xd.ne[2], xd.ne[3], p.image_h, p.image_w);
    Im2colB im{};
    const int geo = make_im2col(p, xd.ne[1], xd.nb + 1, im);
    if (geo != VKHIP_OK) return geo;
    const int64_t oh = (static_cast<int64_t>(p.image_h) + 2 * p.pad_h -
                        (static_cast<int64_t>(p.dilation_h) * (p.kernel_h - 1) + 1)) / p.stride_h + 1;
    const uint64_t L = static_cast<uint64_t>(oh) * im.ow;
    const uint64_t batch = xd.ne[0];
    const uint64_t ck = static_cast<uint64_t>(xd.ne[1]) * p.kernel_h * p.kernel_w;
    // gd: [1, N, Cout, L] (rank-4, right-aligned)
    if (gd.ne[0] != 1 || gd.ne[1] != batch || static_cast<uint64_t>(gd.ne[3]) != L)
        return fail(VKHIP_ERR_INVALID, "conv2d weight grad: gradient must be [N, Cout, %llu]",
                    static_cast<unsigned long long>(L));
    if (gd.nb[3] != 1 && L != 1)
        return fail(VKHIP_ERR_UNSUPPORTED, "conv2d weight grad: gradient positions must be contiguous");
    if (L > 0xffffffffull || ck > 0xffffffffull || batch > 65535)
        return fail(VKHIP_ERR_UNSUPPORTED, "conv2d weight grad: extents too large");
    const uint32_t m = gd.ne[2], n = static_cast<uint32_t>(ck), k = static_cast<uint32_t>(L);
    if (batch == 0 || m == 0 || n == 0) return VKHIP_OK;
    if (ctx().exact_math) {
        // the exact arm with the transposed columns gathered from the image:
        // the oracle's matmul(grad, im2col(x)^T), bit for bit
        publish("matmul.kernel", "conv2d_weight_grad", "gemm_exact_implicit_im2col_t",
                "gemm_mfma_implicit_im2col_t", "exact numerics mode", static_cast<int64_t>(k),
                static_cast<int64_t>(m) * n);
        ExactImg im{};
        const int geo = exact_img(p, x, xd, im);
        if (geo != VKHIP_OK) return geo;
        GemmArgs g{};
        g.a = gr;
        g.b = x;
        g.sa1 = gd.nb[1];
        g.sam = gd.nb[2];
        g.sak = gd.nb[3];
        g.b1 = static_cast<uint32_t>(batch);
        g.m = m;
        g.n = n;
        g.k = k;
        g.c = out;
        return launch_exact(g, static_cast<uint32_t>(batch), B_IMGT, im);
    }
    if (wgrad_small_fits(gr, gd, ck, m, L, im, xd.ne[1])) {
        publish("matmul.kernel", "conv2d_weight_grad", "conv_wgrad_small_window",
                "gemm_mfma_implicit_im2col_t", "C*kh*kw <= 32: the image staged in LDS, one workgroup per image",
                static_cast<int64_t>(batch), static_cast<int64_t>(ck));
        im.x = x;
        im.sn = xd.nb[0];
        im.L = static_cast<uint32_t>(L);
        return launch_wgrad_small(false, gr, gd, im, m, n, static_cast<uint32_t>(batch),
                                  static_cast<uint32_t>(L / 32), out);
    }
    uint32_t splits, chunk;
    TileChoice tile;
    gemm_plan(static_cast<uint32_t>(batch), m, n, k, 0, splits, chunk, tile);
    publish("matmul.kernel", "conv2d_weight_grad",
            tile.bm == 128 ? "gemm_mfma_128x128_implicit_im2col_t" : "gemm_mfma_64x64_implicit_im2col_t",
            "im2col_then_gemm", "the transposed cols matrix is gathered from the image inside the GEMM",
            static_cast<int64_t>(tile.tiles), ctx().ready ? ctx().caps.compute_units : 256);
    im.x = x;
    im.sn = xd.nb[0];

    GemmArgs g{};
    g.a = gr;
    g.b = nullptr;
    g.sa0 = 0;
    g.sa1 = gd.nb[1];
    g.sam = gd.nb[2];
    g.sak = 1;
    g.b1 = static_cast<uint32_t>(batch);
    g.m = m;
    g.n = n;
    g.k = k;
    g.tiles_m = ceil_div(m, tile.bm);
    g.tiles_n = ceil_div(n, tile.bn);
    g.ktiles = ceil_div(k, 32);
    g.chunk = chunk;
    g.a_vec = reinterpret_cast<uintptr_t>(gr) % 16 == 0 && g.sam % 4 == 0 && g.sa1 % 4 == 0 &&
              k % 4 == 0;
    // The weights or gradient rows straight into LDS when the KCD loader's
    // conditions hold (K a multiple of four, 16-byte aligned rows: a_vec;
    // byte offsets within 2^31), else through registers.
    const bool a_kcd = g.a_vec && g.sam >= 0 &&
                       ((static_cast<int64_t>(m) - 1) * g.sam + k) * 4 < (int64_t{1} << 31);
    const int amode = a_kcd ? KCD : (g.a_vec ? KCV : KCS);
    const uint64_t out_elems = batch * m * n;
    float* target = out;
    if (splits > 1) {
        float* ws = nullptr;
        int st = workspace(out_elems * splits * sizeof(float), &ws);
        if (st != VKHIP_OK) return st;
        target = ws;
    }
    g.c = target;
    g.split_stride = splits > 1 ? out_elems : 0;
    int st;
    if (tile.bm == 128 && wgrad_direct_fits(g, k, target)) {
        // both operands straight into LDS (same bits as the register path);
        // 128x64 tiles when their rounds fill the machine better (as in gemm())
        const bool narrow = wgrad_narrow_tiles(g, splits, batch);
        if (narrow) g.tiles_n = ceil_div(n, 64u);
        const uint64_t flat = static_cast<uint64_t>(g.tiles_m) * g.tiles_n * splits;
        g.flat_splits = splits > 1 && flat <= 0x7fffffffull ? splits : 0;
        const dim3 grid = g.flat_splits ? dim3(static_cast<uint32_t>(flat), 1, static_cast<uint32_t>(batch))
                                        : dim3(g.tiles_m * g.tiles_n, splits, static_cast<uint32_t>(batch));
        if (narrow)
            hipLaunchKernelGGL((conv_direct_kernel<CD_WGRAD, 64>), grid, dim3(256), 0, ctx().stream, g, im);
        else
            hipLaunchKernelGGL((conv_direct_kernel<CD_WGRAD, 128>), grid, dim3(256), 0, ctx().stream, g, im);
        VKHIP_LAUNCH_CHECK();
        st = VKHIP_OK;
    } else if (tile.bm == 128)
        st = launch_conv_tiles<128, 128, 64, 64, IMGT>(g, im, static_cast<uint32_t>(batch), splits, amode);
    else
        st = launch_conv_tiles<64, 64, 32, 32, IMGT>(g, im, static_cast<uint32_t>(batch), splits, amode);
    if (st != VKHIP_OK) return st;
    if (splits > 1) return launch_split_k_reduce(target, out, out_elems, splits);
    return VKHIP_OK;
}

int launch_reduce(int op, const float* src, const vkhip_operand& d, uint32_t mask, void* dst);
int launch_col2im(const float* cols, float* dst, uint32_t n, uint32_t channels, const vkhip_unfold& p);
int launch_max_pool2d_backward(const float* grad, const float* src, const vkhip_operand& sd, float* dst,
                               uint32_t out_h, uint32_t out_w, const vkhip_unfold& p, bool relu);
int conv2d_weight_grad_sum(const float* x, const vkhip_operand& xd, const float* gr, const vkhip_operand& gd,
                           float* out, const vkhip_unfold& p);

// The weight and bias gradients of a conv layer whose output y = relu(conv2d(x,
// w) + bias) feeds a 2x2, stride-2 max-pool, from the pool's output gradient gp
// (VKHIP_OP_CONV2D_POOL_WEIGHT_BIAS_GRAD): out = [Cout*C*kh*kw weight
// gradient, Cout bias gradient], the values of the MAX_POOL2D_BACKWARD_RELU,
// CONV2D_WEIGHT_GRAD_SUM and SUM (over N, oh, ow) nodes it replaces. yd, gpd:
// [N, Cout, oh, ow] and [N, Cout, oh/2, ow/2] (to_operand's rank-4 layout).
//  - FAST numerics where the small-window kernel takes the layer: one pass
//    over y and gp that forms the relu-masked pool gradient in the kernel
//    (never written) and sums both gradients (win_conv_pool_weight_bias_grad):
//    the replaced nodes' bits on the fast path.
//  - Otherwise those nodes in turn, the pool gradient in the fused
//    intermediate.
int conv2d_pool_weight_bias_grad(const float* x, const vkhip_operand& xd, const float* y, const vkhip_operand& yd,
                                 const float* gp, const vkhip_operand& gpd, float* out, const vkhip_unfold& p) {
    const uint32_t batch = yd.ne[0], cout = yd.ne[1], oh = yd.ne[2], ow = yd.ne[3];
    const uint64_t L = static_cast<uint64_t>(oh) * ow;
    const uint64_t ck = static_cast<uint64_t>(xd.ne[1]) * p.kernel_h * p.kernel_w;
    if (gpd.ne[0] != batch || gpd.ne[1] != cout || gpd.ne[2] != oh / 2 || gpd.ne[3] != ow / 2 || xd.ne[0] != batch)
        return fail(VKHIP_ERR_INVALID, "conv2d pool weight grad: pool gradient [%u,%u,%u,%u] does not pool [%u,%u,%u,%u]",
                    gpd.ne[0], gpd.ne[1], gpd.ne[2], gpd.ne[3], batch, cout, oh, ow);
    float* bias_out = out + static_cast<uint64_t>(cout) * ck;
    vkhip_operand gyd;  // y as a gradient operand [1, N, Cout, L]
    gyd.ne[0] = 1;
    gyd.ne[1] = batch;
    gyd.ne[2] = cout;
    gyd.ne[3] = static_cast<uint32_t>(L);
    gyd.nb[0] = 0;
    gyd.nb[1] = yd.nb[0];
    gyd.nb[2] = yd.nb[1];
    gyd.nb[3] = 1;
    const bool y_rows = yd.nb[3] == 1 && yd.nb[2] == static_cast<int64_t>(ow);
    const bool gp_rows = gpd.nb[3] == 1 && gpd.nb[2] == static_cast<int64_t>(ow / 2);
    if (!ctx().exact_math && y_rows && gp_rows && L <= 0xffffffffull &&
        win_pool_wgrad_fits(y, gyd, gp, gpd.nb[0], gpd.nb[1], xd, p, xd.ne[1], ck, cout, batch, oh, ow)) {
        publish("matmul.kernel", "conv2d_pool_weight_bias_grad", "win_wgrad_pool", "pool_backward_then_products",
                "C*kh*kw <= 32: the relu-masked pool gradient formed in the weight-gradient kernel",
                static_cast<int64_t>(L), static_cast<int64_t>(ck));
        return win_conv_pool_weight_bias_grad(x, xd, y, gyd, gp, gpd.nb[0], gpd.nb[1], out, bias_out, p, batch,
                                              xd.ne[1], cout, static_cast<uint32_t>(ck), oh, ow);
    }
    publish("matmul.kernel", "conv2d_pool_weight_bias_grad", "pool_backward_then_products", "win_wgrad_pool",
            ctx().exact_math ? "exact numerics mode" : "the layer does not fit the small-window kernel",
            static_cast<int64_t>(L), static_cast<int64_t>(ck));
    const uint64_t dz_elems = static_cast<uint64_t>(batch) * cout * L;
    float* dz = nullptr;
    int st = fused_intermediate(dz_elems * sizeof(float), &dz);
    if (st != VKHIP_OK) return st;
    vkhip_unfold pp{};
    pp.kernel_h = pp.kernel_w = 2;
    pp.stride_h = pp.stride_w = 2;
    pp.pad_h = pp.pad_w = 0;
    pp.dilation_h = pp.dilation_w = 1;
    pp.image_h = static_cast<int32_t>(oh);
    pp.image_w = static_cast<int32_t>(ow);
    st = launch_max_pool2d_backward(gp, y, yd, dz, gpd.ne[2], gpd.ne[3], pp, true);
    if (st != VKHIP_OK) return st;
    vkhip_operand dgd;  // dz as the gradient operand [1, N, Cout, L]
    dgd.ne[0] = 1;
    dgd.ne[1] = batch;
    dgd.ne[2] = cout;
    dgd.ne[3] = static_cast<uint32_t>(L);
    dgd.nb[0] = 0;
    dgd.nb[1] = static_cast<int64_t>(cout) * static_cast<int64_t>(L);
    dgd.nb[2] = static_cast<int64_t>(L);
    dgd.nb[3] = 1;
    st = conv2d_weight_grad_sum(x, xd, dz, dgd, out, p);
    if (st != VKHIP_OK) return st;
    vkhip_operand rd;  // dz [N, Cout, oh, ow], summed over axes 0, 2, 3
    rd.ne[0] = batch;
    rd.ne[1] = cout;
    rd.ne[2] = oh;
    rd.ne[3] = ow;
    rd.nb[0] = dgd.nb[1];
    rd.nb[1] = static_cast<int64_t>(L);
    rd.nb[2] = static_cast<int64_t>(ow);
    rd.nb[3] = 1;
    return launch_reduce(VKHIP_REDUCE_SUM, dz, rd, 0xDu, bias_out);
}

// The weight gradient summed over the batch, out [Cout, C*kh*kw] = sum_n
// grad[n] @ im2col(x[n])^T: the reference graph's per-image products and
// batch sum (autograd.cpp:548-553 over ops.cpp:662-705, then the broadcast
// adjoint sum, autograd.cpp:84-116).
//  - FAST numerics with L = out_h*out_w a multiple of 32: ONE product with the
//    batch folded into K (k = n*L + position), [Cout, N*L] x [N*L, C*kh*kw],
//    the columns gathered from each image (load mode IMGTB), split-K planned
//    like any product: no [N, Cout, C*kh*kw] intermediate and no separate
//    batch sum. Its K order differs from the graph's (within the GEMM
//    tolerance, not the same bits).
//  - EXACT numerics, or L not a multiple of 32: the per-image products
//    (conv2d_weight_grad, exact in the exact mode) into a node temporary,
//    then the batch sum's pairwise reduction: the graph's bits.
int conv2d_weight_grad_sum(const float* x, const vkhip_operand& xd, const float* gr,
                           const vkhip_operand& gd, float* out, const vkhip_unfold& p) {
    if (static_cast<int64_t>(xd.ne[2]) != p.image_h || static_cast<int64_t>(xd.ne[3]) != p.image_w)
        return fail(VKHIP_ERR_INVALID, "conv2d weight grad sum: image is %ux%u but the geometry says %dx%d",
                    xd.ne[2], xd.ne[3], p.image_h, p.image_w);
    Im2colB im{};
    const int geo = make_im2col(p, xd.ne[1], xd.nb + 1, im);
    if (geo != VKHIP_OK) return geo;
    const int64_t oh = (static_cast<int64_t>(p.image_h) + 2 * p.pad_h -
                        (static_cast<int64_t>(p.dilation_h) * (p.kernel_h - 1) + 1)) / p.stride_h + 1;
    const uint64_t L = static_cast<uint64_t>(oh) * im.ow;
    const uint64_t batch = xd.ne[0];
    const uint64_t ck = static_cast<uint64_t>(xd.ne[1]) * p.kernel_h * p.kernel_w;
    const uint32_t cout = gd.ne[2];
    if (gd.ne[0] != 1 || gd.ne[1] != batch || static_cast<uint64_t>(gd.ne[3]) != L)
        return fail(VKHIP_ERR_INVALID, "conv2d weight grad sum: gradient must be [N, Cout, %llu]",
                    static_cast<unsigned long long>(L));
    if (gd.nb[3] != 1 && L != 1)
        return fail(VKHIP_ERR_UNSUPPORTED, "conv2d weight grad sum: gradient positions must be contiguous");
    if (cout == 0 || ck == 0) return VKHIP_OK;
    if (batch == 0 || L == 0) return launch_zero_f32(out, static_cast<uint64_t>(cout) * ck);
    const uint64_t k64 = batch * L;
    if (ctx().exact_math || L % 32 != 0 || k64 > 0xffffffffull || ck > 0xffffffffull) {
        publish("matmul.kernel", "conv2d_weight_grad_sum", "per_image_products_then_batch_sum",
                "batch_folded_into_k", ctx().exact_math ? "exact numerics mode"
                                                        : "positions per image not a multiple of 32",
                static_cast<int64_t>(L), static_cast<int64_t>(batch));
        float* tmp = nullptr;
        const uint64_t per = static_cast<uint64_t>(cout) * ck;
        int st = node_temporary(batch * per * sizeof(float), &tmp);
        if (st != VKHIP_OK) return st;
        st = conv2d_weight_grad(x, xd, gr, gd, tmp, p);
        if (st != VKHIP_OK) return st;
        vkhip_operand td;
        td.ne[0] = 1;
        td.ne[1] = static_cast<uint32_t>(batch);
        td.ne[2] = cout;
        td.ne[3] = static_cast<uint32_t>(ck);
        td.nb[0] = 0;
        td.nb[1] = static_cast<int64_t>(per);
        td.nb[2] = static_cast<int64_t>(ck);
        td.nb[3] = 1;
        return launch_reduce(VKHIP_REDUCE_SUM, tmp, td, 0x2u, out);
    }
    {
        const uint32_t ohw = static_cast<uint32_t>(L / static_cast<uint64_t>(im.ow));
        if (win_wgrad_fits(gr, gd, xd, p, xd.ne[1], ck, cout, batch, ohw, static_cast<uint32_t>(im.ow))) {
            publish("matmul.kernel", "conv2d_weight_grad_sum", "win_wgrad", "conv_wgrad_small_window_folded",
                    "C*kh*kw <= 32: the gradient streamed once, partials folded in the same launch",
                    static_cast<int64_t>(L), static_cast<int64_t>(ck));
            return win_conv_weight_grad_sum(x, xd, gr, gd, out, p, static_cast<uint32_t>(batch), xd.ne[1], cout,
                                            static_cast<uint32_t>(ck), ohw, static_cast<uint32_t>(im.ow));
        }
    }
    uint64_t stream_parts = 0;
    const uint32_t stream_bpw = wgrad_stream_fits(gr, gd, p, xd.ne[1], ck, cout, L)
                                    ? wgrad_stream_bpw(batch, static_cast<uint32_t>(L / 32), stream_parts)
                                    : 0u;
    if (stream_bpw != 0) {
        publish("matmul.kernel", "conv2d_weight_grad_sum", "conv_wgrad_stream",
                "conv_wgrad_small_window_folded",
                "C*kh*kw <= 32: the gradient streamed once, partials per workgroup",
                static_cast<int64_t>(stream_parts), static_cast<int64_t>(ck));
        const uint32_t oh = static_cast<uint32_t>(L / static_cast<uint64_t>(im.ow));
        SmallConvFwd sp = small_conv_geometry(x, xd, p, xd.ne[1], cout, static_cast<uint32_t>(ck), oh,
                                              static_cast<uint32_t>(im.ow));
        const uint64_t out_elems = static_cast<uint64_t>(cout) * ck;
        float* target = out;
        if (stream_parts > 1) {
            const int st = workspace(out_elems * stream_parts * sizeof(float), &target);
            if (st != VKHIP_OK) return st;
        }
        const int st = launch_conv_wgrad_stream(sp, gr, gd, static_cast<uint32_t>(batch), stream_bpw, target);
        if (st != VKHIP_OK || stream_parts == 1) return st;
        return launch_split_k_reduce(target, out, out_elems, static_cast<uint32_t>(stream_parts));
    }
    if (wgrad_small_fits(gr, gd, ck, cout, L, im, xd.ne[1])) {
        // K-tiles per workgroup: an image's, halved (keeping whole K-tiles
        // per wave) while that leaves fewer than 256 workgroups; at most 511
        // partials for the fold
        const uint32_t tpi = static_cast<uint32_t>(L / 32);
        uint32_t kpw = tpi;
        while (kpw % 2 == 0 && kpw >= 2 * kSmallWgradWaves && batch * tpi / kpw < 256) kpw /= 2;
        const uint64_t parts = batch * tpi / kpw;
        if (parts <= 511) {
            publish("matmul.kernel", "conv2d_weight_grad_sum", "conv_wgrad_small_window_folded",
                    "batch_folded_into_k", "C*kh*kw <= 32: the image staged in LDS, partials per K range",
                    static_cast<int64_t>(parts), static_cast<int64_t>(ck));
            im.x = x;
            im.sn = xd.nb[0];
            im.L = static_cast<uint32_t>(L);
            const uint64_t out_elems = static_cast<uint64_t>(cout) * ck;
            float* target = out;
            if (parts > 1) {
                const int st = workspace(out_elems * parts * sizeof(float), &target);
                if (st != VKHIP_OK) return st;
            }
            const int st = launch_wgrad_small(true, gr, gd, im, cout, static_cast<uint32_t>(ck),
                                              static_cast<uint32_t>(batch), kpw, target);
            if (st != VKHIP_OK || parts == 1) return st;
            return launch_split_k_reduce(target, out, out_elems, static_cast<uint32_t>(parts));
        }
    }
    const uint32_t m = cout, n = static_cast<uint32_t>(ck), k = static_cast<uint32_t>(k64);
    uint32_t splits, chunk;
    TileChoice tile;
    gemm_plan(1, m, n, k, 0, splits, chunk, tile, true);
    publish("matmul.kernel", "conv2d_weight_grad_sum",
            tile.bm == 128 ? "gemm_mfma_128x128_batch_folded" : "gemm_mfma_64x64_batch_folded",
            "per_image_products_then_batch_sum", "the batch folded into K: one product, no intermediate",
            static_cast<int64_t>(tile.tiles), static_cast<int64_t>(splits));
    im.x = x;
    im.sn = xd.nb[0];
    im.L = static_cast<uint32_t>(L);
    im.images = static_cast<uint32_t>(batch);
    im.div_L = FastDiv(static_cast<uint32_t>(L));

    GemmArgs g{};
    g.a = gr;
    g.b = x;
    g.sa1 = gd.nb[1];  // image stride of the gradient
    g.sam = gd.nb[2];
    g.sak = 1;
    g.b1 = 1;
    g.m = m;
    g.n = n;
    g.k = k;
    g.tiles_m = ceil_div(m, tile.bm);
    g.tiles_n = ceil_div(n, tile.bn);
    g.ktiles = ceil_div(k, 32);
    g.chunk = chunk;
    g.a_vec = reinterpret_cast<uintptr_t>(gr) % 16 == 0 && g.sam % 4 == 0 && g.sa1 % 4 == 0;
    const int amode = g.a_vec ? KCV : KCS;
    const uint64_t out_elems = static_cast<uint64_t>(m) * n;
    float* target = out;
    if (splits > 1) {
        float* ws = nullptr;
        int st = workspace(out_elems * splits * sizeof(float), &ws);
        if (st != VKHIP_OK) return st;
        target = ws;
    }
    g.c = target;
    g.split_stride = splits > 1 ? out_elems : 0;
    int st;
    if (tile.bm == 128 && wgrad_direct_fits(g, static_cast<uint32_t>(L), target)) {
        const bool narrow = wgrad_narrow_tiles(g, splits, 1);
        if (narrow) g.tiles_n = ceil_div(n, 64u);
        const uint64_t flat = static_cast<uint64_t>(g.tiles_m) * g.tiles_n * splits;
        g.flat_splits = splits > 1 && flat <= 0x7fffffffull ? splits : 0;
        const dim3 grid = g.flat_splits ? dim3(static_cast<uint32_t>(flat), 1, 1)
                                        : dim3(g.tiles_m * g.tiles_n, splits, 1);
        if (narrow)
            hipLaunchKernelGGL((conv_direct_kernel<CD_WGRAD_FOLD, 64>), grid, dim3(256), 0, ctx().stream, g, im);
        else
            hipLaunchKernelGGL((conv_direct_kernel<CD_WGRAD_FOLD, 128>), grid, dim3(256), 0, ctx().stream, g, im);
        VKHIP_LAUNCH_CHECK();
        st = VKHIP_OK;
    } else if (tile.bm == 128)
        st = launch_conv_tiles<128, 128, 64, 64, IMGTB>(g, im, 1, splits, amode);
    else
        st = launch_conv_tiles<64, 64, 32, 32, IMGTB>(g, im, 1, splits, amode);
    if (st != VKHIP_OK) return st;
    if (splits > 1) return launch_split_k_reduce(target, out, out_elems, splits);
    return VKHIP_OK;
}

// The flipped, transposed weight of the input gradient's convolution:
// wt[c][o*kk + (kk - 1 - r)] = w[o][c*kk + r] (kk = kh*kw window elements,
// r = ki*kw + kj, so kk - 1 - r is the window rotated by 180 degrees).
// One thread per element of wt (fewer than 2^32, checked by the host), the
// index split by multiply-high divisions.
__global__ void conv_weight_flip_kernel(const float* __restrict__ w, int64_t s_out,
                                        float* __restrict__ wt, uint32_t total, FastDiv div_row,
                                        FastDiv div_kk) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= total) return;
    const uint32_t c = div_row.div(i);
    const uint32_t rest = i - c * div_row.d;
    const uint32_t o = div_kk.div(rest);
    const uint32_t r = div_kk.d - 1 - (rest - o * div_kk.d);
    wt[i] = w[static_cast<int64_t>(o) * s_out + static_cast<int64_t>(c) * div_kk.d + r];
}

// Input gradient of conv2d (forward geometry p, weight rows [Cout, C*kh*kw]
// contiguous with row stride w_row). With unit strides the column adjoint
// col2im(W^T @ g) equals the convolution of g with the 180-degree rotated,
// channel-transposed window under pad' = dilation*(k-1) - pad: dX[c][h][w] =
// sum_{o,ki,kj} W[o][c][ki][kj] g[o][h + pad - ki*d][w + pad - kj*d], and
// with ki' = kh-1-ki the row offset is h - pad' + ki'*d. That runs as the
// implicit-im2col conv kernel on g (no column matrix, no col2im pass), in a
// different summation order than the graph (within the GEMM tolerance for
// K = Cout*kh*kw). Exact numerics, other strides or pad > dilation*(k-1) run
// the graph: the TN product into a column matrix, then col2im.
int conv2d_input_grad(const float* gr, const vkhip_operand& gd, const float* w, int64_t w_row,
                      uint32_t channels, float* out, const vkhip_unfold& p) {
    if (p.kernel_h <= 0 || p.kernel_w <= 0 || p.stride_h <= 0 || p.stride_w <= 0 ||
        p.dilation_h <= 0 || p.dilation_w <= 0 || p.pad_h < 0 || p.pad_w < 0 || p.image_h < 0 ||
        p.image_w < 0)
        return fail(VKHIP_ERR_INVALID, "conv2d input grad: invalid window geometry");
    const int64_t oh = (static_cast<int64_t>(p.image_h) + 2 * p.pad_h -
                        (static_cast<int64_t>(p.dilation_h) * (p.kernel_h - 1) + 1)) / p.stride_h + 1;
    const int64_t ow = (static_cast<int64_t>(p.image_w) + 2 * p.pad_w -
                        (static_cast<int64_t>(p.dilation_w) * (p.kernel_w - 1) + 1)) / p.stride_w + 1;
    if (oh <= 0 || ow <= 0) return fail(VKHIP_ERR_INVALID, "conv2d input grad: window larger than padded image");
    if (static_cast<int64_t>(gd.ne[2]) != oh || static_cast<int64_t>(gd.ne[3]) != ow)
        return fail(VKHIP_ERR_INVALID, "conv2d input grad: gradient is %ux%u, the geometry gives %lldx%lld",
                    gd.ne[2], gd.ne[3], static_cast<long long>(oh), static_cast<long long>(ow));
    if (gd.nb[3] != 1 || gd.nb[2] != static_cast<int64_t>(ow))
        return fail(VKHIP_ERR_UNSUPPORTED, "conv2d input grad: gradient positions must be contiguous");
    const uint32_t batch = gd.ne[0], cout = gd.ne[1];
    const uint32_t kk = static_cast<uint32_t>(p.kernel_h * p.kernel_w);
    const uint64_t ck = static_cast<uint64_t>(channels) * kk;
    const uint64_t L = static_cast<uint64_t>(oh) * ow;
    const uint64_t image = static_cast<uint64_t>(p.image_h) * p.image_w;
    if (batch == 0 || channels == 0 || image == 0) return VKHIP_OK;
    if (cout == 0) return launch_zero_f32(out, static_cast<uint64_t>(batch) * channels * image);
    const int pad2h = p.dilation_h * (p.kernel_h - 1) - p.pad_h;
    const int pad2w = p.dilation_w * (p.kernel_w - 1) - p.pad_w;
    // The convolution's output rows are the C input channels: under 32 they
    // fill too little of a 64-row tile (C = 3: 0.3x the TN product + col2im).
    const bool geometry = p.stride_h == 1 && p.stride_w == 1 && pad2h >= 0 && pad2w >= 0 &&
                          kk <= 63 && static_cast<uint64_t>(cout) * kk <= 0xffffffffull;
    const bool fused = !ctx().exact_math && geometry && channels >= 32;
    if (!ctx().exact_math && ctx().node_gemm_kernel != VKHIP_GEMM_EXACT && ck <= 32 &&
        win_dx_fits(gd, w_row, p, batch, channels, cout, static_cast<uint32_t>(oh), static_cast<uint32_t>(ow))) {
        publish("conv.input_grad", "conv2d_input_grad", "columns_in_lds_then_col2im", "tn_product_then_col2im",
                "C*kh*kw <= 32: the column matrix of a band of rows held in LDS, the lowering's bits",
                static_cast<int64_t>(ck), 32);
        return win_conv_input_grad(gr, gd, w, w_row, out, p, batch, channels, cout, static_cast<uint32_t>(oh),
                                   static_cast<uint32_t>(ow));
    }
    publish("conv.input_grad", "conv2d_input_grad",
            fused ? "implicit_conv_of_grad_with_flipped_weight" : "tn_product_then_col2im",
            fused ? "tn_product_then_col2im" : "implicit_conv_of_grad_with_flipped_weight",
            fused ? "unit strides: the column adjoint is a convolution"
                  : (ctx().exact_math ? "exact numerics mode"
                                      : (geometry ? "fewer than 32 input channels"
                                                  : "strided or over-padded window")),
            static_cast<int64_t>(channels), 32);
    if (fused) {
        const uint64_t wt_elems = static_cast<uint64_t>(channels) * cout * kk;
        float* wt = nullptr;
        int st = node_temporary(wt_elems * sizeof(float), &wt);
        if (st != VKHIP_OK) return st;
        if (wt_elems >= (uint64_t{1} << 32))
            return fail(VKHIP_ERR_UNSUPPORTED, "conv2d input grad: %llu weight elements",
                        static_cast<unsigned long long>(wt_elems));
        hipLaunchKernelGGL(conv_weight_flip_kernel, dim3(ceil_div(wt_elems, 256)), dim3(256), 0,
                           ctx().stream, w, w_row, wt, static_cast<uint32_t>(wt_elems),
                           FastDiv(cout * kk), FastDiv(kk));
        VKHIP_LAUNCH_CHECK();
        vkhip_unfold q = p;
        q.stride_h = 1;
        q.stride_w = 1;
        q.pad_h = pad2h;
        q.pad_w = pad2w;
        q.image_h = static_cast<int32_t>(oh);
        q.image_w = static_cast<int32_t>(ow);
        vkhip_operand wd;
        wd.ne[0] = 1;
        wd.ne[1] = 1;
        wd.ne[2] = channels;
        wd.ne[3] = cout * kk;
        wd.nb[0] = 0;
        wd.nb[1] = 0;
        wd.nb[2] = static_cast<int64_t>(cout) * kk;
        wd.nb[3] = 1;
        return conv2d_forward(gr, gd, wt, wd, out, q, nullptr, 0, false);
    }
    if (ck > 0xffffffffull || L > 0xffffffffull)
        return fail(VKHIP_ERR_UNSUPPORTED, "conv2d input grad: extents too large");
    float* cols = nullptr;
    int st = node_temporary(static_cast<uint64_t>(batch) * ck * L * sizeof(float), &cols);
    if (st != VKHIP_OK) return st;
    // flat_weight^T broadcast over the batch @ grad: the graph's MATMUL node
    vkhip_operand ad, bd;
    ad.ne[0] = 1;
    ad.ne[1] = batch;
    ad.ne[2] = static_cast<uint32_t>(ck);
    ad.ne[3] = cout;
    ad.nb[0] = 0;
    ad.nb[1] = 0;
    ad.nb[2] = 1;
    ad.nb[3] = w_row;
    bd.ne[0] = 1;
    bd.ne[1] = batch;
    bd.ne[2] = cout;
    bd.ne[3] = static_cast<uint32_t>(L);
    bd.nb[0] = 0;
    bd.nb[1] = gd.nb[0];
    bd.nb[2] = gd.nb[1];
    bd.nb[3] = 1;
    const vkhip_gemm_opts opts{ctx().node_gemm_kernel, 0};
    st = gemm(w, ad, gr, bd, cols, &opts);
    if (st != VKHIP_OK) return st;
    return launch_col2im(cols, out, batch, channels, p);
}
}  // namespace vkhip

// ---- C ABI -------------------------------------------------------------------
extern "C" int vkhip_gemm(const float* a, const vkhip_operand* a_desc, const float* b,
                          const vkhip_operand* b_desc, float* c, const vkhip_gemm_opts* opts) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::Unit unit("matmul");
    if (!a_desc || !b_desc) return vkhip::fail(VKHIP_ERR_INVALID, "gemm: null descriptor");
    return vkhip::gemm(a, *a_desc, b, *b_desc, c, opts);
}

extern "C" int vkhip_gemm_noalloc(const float* a, const vkhip_operand* a_desc, const float* b,
                                  const vkhip_operand* b_desc, float* c,
                                  const vkhip_gemm_opts* opts) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    if (!a_desc || !b_desc) return vkhip::fail(VKHIP_ERR_INVALID, "gemm_noalloc: null descriptor");
    if (!vkhip::ctx().scratch)
        return vkhip::fail(VKHIP_ERR_UNSUPPORTED, "gemm_noalloc: no scratch array on device %d",
                           vkhip::ctx().device);
    const vkhip::FixedScratch fixed{vkhip::ctx().scratch, VKHIP_GEMM_NOALLOC_SCRATCH_BYTES};
    return vkhip::gemm(a, *a_desc, b, *b_desc, c, opts, &fixed);
}

extern "C" int vkhip_gemm_plan(uint32_t batch, uint32_t m, uint32_t n, uint32_t k,
                               int32_t split_request, uint32_t* out_splits, uint32_t* out_chunk) {
    uint32_t s, c;
    vkhip::TileChoice t;
    vkhip::gemm_plan(batch, m, n, k, split_request, s, c, t, true);
    if (out_splits) *out_splits = s;
    if (out_chunk) *out_chunk = c;
    return VKHIP_OK;
}

extern "C" int vkhip_split_k_reduce(const float* ws, float* dst, uint64_t ne, uint32_t splits) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::Unit unit("split_k_reduce");
    if (splits == 0 || splits > 511)
        return vkhip::fail(VKHIP_ERR_INVALID, "split_k_reduce: splits=%u outside 1..511", splits);
    return vkhip::launch_split_k_reduce(ws, dst, ne, splits);
}

extern "C" int vkhip_gemv(const float* a, int64_t lda, const float* x, int64_t incx, float* y,
                          uint32_t m, uint32_t k) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::Unit unit("gemv");
    return vkhip::launch_gemv(a, lda, x, incx, y, m, k);
}

extern "C" int vkhip_conv2d(const float* x, const vkhip_operand* x_desc, const float* w,
                            const vkhip_operand* w_desc, float* out, const vkhip_unfold* p) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::Unit unit("conv2d");
    if (!x_desc || !w_desc || !p) return vkhip::fail(VKHIP_ERR_INVALID, "conv2d: null argument");
    return vkhip::conv2d_forward(x, *x_desc, w, *w_desc, out, *p, nullptr, 0, false);
}

extern "C" int vkhip_conv2d_weight_grad(const float* x, const vkhip_operand* x_desc,
                                        const float* grad, const vkhip_operand* grad_desc, float* out,
                                        const vkhip_unfold* p) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::Unit unit("conv2d_weight_grad");
    if (!x_desc || !grad_desc || !p) return vkhip::fail(VKHIP_ERR_INVALID, "conv2d weight grad: null argument");
    return vkhip::conv2d_weight_grad(x, *x_desc, grad, *grad_desc, out, *p);
}

extern "C" int vkhip_conv2d_input_grad(const float* grad, const vkhip_operand* grad_desc,
                                       const float* w, const vkhip_operand* w_desc, float* out,
                                       const vkhip_unfold* p) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::Unit unit("conv2d_input_grad");
    if (!grad_desc || !w_desc || !p) return vkhip::fail(VKHIP_ERR_INVALID, "conv2d_input_grad: null argument");
    const int64_t kk = static_cast<int64_t>(p->kernel_h) * p->kernel_w;
    if (kk <= 0 || w_desc->ne[0] != 1 || w_desc->ne[1] != 1 || w_desc->ne[2] != grad_desc->ne[1] ||
        w_desc->ne[3] % kk != 0 || (w_desc->nb[3] != 1 && w_desc->ne[3] > 1) || w_desc->nb[2] < 0)
        return vkhip::fail(VKHIP_ERR_INVALID,
                           "conv2d_input_grad: weight must be [1,1,Cout,C*kh*kw] with contiguous rows");
    return vkhip::conv2d_input_grad(grad, *grad_desc, w, w_desc->nb[2],
                                    static_cast<uint32_t>(w_desc->ne[3] / kk), out, *p);
}

extern "C" int vkhip_conv2d_weight_grad_sum(const float* x, const vkhip_operand* x_desc,
                                            const float* grad, const vkhip_operand* grad_desc,
                                            float* out, const vkhip_unfold* p) {
    int st = vkhip::require_ready();
    if (st != VKHIP_OK) return st;
    vkhip::Unit unit("conv2d_weight_grad_sum");
    if (!x_desc || !grad_desc || !p) return vkhip::fail(VKHIP_ERR_INVALID, "conv2d_weight_grad_sum: null argument");
    return vkhip::conv2d_weight_grad_sum(x, *x_desc, grad, *grad_desc, out, *p);
}

extern "C" uint32_t vkhip_kcd_slot_offset(uint32_t slot, int64_t s_row, uint32_t row0, uint32_t rows,
                                          uint32_t k0, uint32_t kdim) {
    return vkhip::kcd_slot_offset(static_cast<int>(slot), s_row, row0, rows, k0, kdim);
}

extern "C" int vkhip_im2col_offset_t(const vkhip_unfold* p, uint32_t channels, const int64_t* x_strides,
                                     uint32_t row, uint32_t pos, int64_t* out_offset) {
    if (!p || !x_strides || !out_offset) return vkhip::fail(VKHIP_ERR_INVALID, "im2col_offset_t: null argument");
    vkhip::Im2colB im{};
    const int st = vkhip::make_im2col(*p, channels, x_strides, im);
    if (st != VKHIP_OK) return st;
    // The weight-gradient gather's arithmetic (conv_direct_kernel): the
    // window row's fixed part, the position's scalar part, the bounds test.
    const uint32_t ncols = channels * static_cast<uint32_t>(p->kernel_h * p->kernel_w);
    const vkhip::GatherCol c = vkhip::gather_col(im, row, ncols);
    const uint32_t oh = im.div_ow.div(pos);
    const vkhip::GatherPos q = vkhip::gather_pos(im, oh, pos - oh * static_cast<uint32_t>(im.ow));
    const uint32_t at4 = vkhip::gather_offset(im, c, q.sh, q.sw, q.so4, true);
    *out_offset = (at4 >> 31) ? -1 : static_cast<int64_t>(at4 / 4);
    return VKHIP_OK;
}

extern "C" int vkhip_im2col_offset(const vkhip_unfold* p, uint32_t channels, const int64_t* x_strides,
                                   uint32_t row, uint32_t pos, int64_t* out_offset) {
    if (!p || !x_strides || !out_offset) return vkhip::fail(VKHIP_ERR_INVALID, "im2col_offset: null argument");
    vkhip::Im2colB im{};
    const int st = vkhip::make_im2col(*p, channels, x_strides, im);
    if (st != VKHIP_OK) return st;
    // The loader's arithmetic: the table row's byte offset and window
    // element against the position's padding mask.
    const vkhip::ImgPos at = vkhip::img_pos(im, pos, true);
    const vkhip::ImgRow q = vkhip::img_row(im, row);
    const uint32_t pad = static_cast<uint32_t>(at.outside >> q.r) & 1u;
    const uint32_t at4 = (pad << 31) | static_cast<uint32_t>(at.base * 4 + q.off * 4);
    *out_offset = (at4 >> 31) ? -1 : static_cast<int64_t>(at4 / 4);
    return VKHIP_OK;
}
