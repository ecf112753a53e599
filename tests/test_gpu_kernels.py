"""Device parity: every hot-path kernel through the C ABI against the CPU oracle.

Bars (north star): im2col/col2im, pooling, argmax, sum/mean, GEMV and the
split-K fold are bit-exact; GEMM and softmax are within a normwise relative
error of 1e-5*sqrt(K) of the oracle (and inside the backward-error bound of a
float64 product, the reference's own GEMM policy, conftest.py:145-165).
Shapes are the reference's test geometries plus the BASELINE configs; where the
oracle is too slow at full size, full-size runs are checked on row samples
against float64.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from conftest import SEED, gemm_atol, gemm_tolerance, golden, normwise_rel_err, small_window
from vkml_amd import _lib, ops
from vkml_amd.device import DeviceArray

pytestmark = pytest.mark.gpu


def dev(x: np.ndarray) -> DeviceArray:
    return DeviceArray.from_numpy(x)


def layout_view(x: np.ndarray, transposed: bool) -> tuple[np.ndarray, DeviceArray]:
    """Host array and a device view of the same values; `transposed` stores the
    matrix as its transpose and hands out a strided .T view (NT / TN operands)."""
    if transposed:
        d = dev(np.ascontiguousarray(np.swapaxes(x, -1, -2)))
        return x, d.transpose(-2, -1)
    return x, dev(x)


def check_gemm(a: np.ndarray, b: np.ndarray, got: np.ndarray, want: np.ndarray | None = None):
    k = a.shape[-1]
    if want is None:
        want = O.matmul(a, b)
    err = normwise_rel_err(got, want)
    assert err <= gemm_tolerance(k), f"normwise rel err {err:.3g} > {gemm_tolerance(k):.3g}"
    exact = np.matmul(a.astype(np.float64), b.astype(np.float64))
    assert np.max(np.abs(got - exact)) <= gemm_atol(a, b) + 1e-30


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------

def test_gemm_known_answer(hip):
    """reference test_ops.cpp:266-280, 305-311."""
    f = golden("matmul_2d")
    np.testing.assert_array_equal(ops.matmul(dev(f["a"]), dev(f["b"])).numpy(), f["expected"])
    t = golden("matmul_transposed_operand")
    np.testing.assert_array_equal(ops.matmul(dev(t["a"]), dev(t["b_transposed"]).T).numpy(),
                                  t["expected"])
    bb = golden("matmul_batch_broadcast")
    got = ops.matmul(dev(bb["a"][None]), dev(bb["b"][None]).broadcast_to((1, 2, 2, 2))).numpy()
    np.testing.assert_array_equal(got[0], bb["expected"])


def test_gemm_vector_rules(hip):
    f = golden("matmul_vector_rules")
    np.testing.assert_array_equal(ops.matmul(dev(f["m"]), dev(f["v"])).numpy(), f["m_v"])
    np.testing.assert_array_equal(ops.matmul(dev(f["u"]), dev(f["m"])).numpy(), f["u_m"])


@pytest.mark.parametrize("size", [1, 2, 3, 7, 8, 15, 16, 31, 32, 63, 64, 127, 128, 255, 256, 257])
def test_gemm_edge_sizes(hip, size):
    rng = np.random.default_rng(SEED + 32)
    a = rng.uniform(-2, 2, (size, size)).astype(np.float32)
    b = rng.uniform(-2, 2, (size, size)).astype(np.float32)
    check_gemm(a, b, ops.matmul(dev(a), dev(b)).numpy())


def gemm_cases(count: int):
    rng = np.random.default_rng(SEED + 30)
    for i in range(count):
        m, n, k = (int(v) for v in rng.integers(1, 300, 3))
        yield i, m, n, k, bool(rng.integers(2)), bool(rng.integers(2))


@pytest.mark.parametrize("i,m,n,k,ta,tb", list(gemm_cases(40)))
def test_gemm_random_shapes_and_layouts(hip, i, m, n, k, ta, tb):
    rng = np.random.default_rng(SEED + 100 + i)
    a, da = layout_view(rng.uniform(-2, 2, (m, k)).astype(np.float32), ta)
    b, db = layout_view(rng.uniform(-2, 2, (k, n)).astype(np.float32), tb)
    check_gemm(a, b, ops.matmul(da, db).numpy())


@pytest.mark.parametrize("layout", ["nn", "nt", "tn", "tt"])
def test_gemm_config2_512_layouts(hip, layout):
    """BASELINE config 2 at 512^3 in every layout forward/backward emit."""
    rng = np.random.default_rng(SEED + 2)
    a, da = layout_view(rng.standard_normal((512, 512)).astype(np.float32), layout[0] == "t")
    b, db = layout_view(rng.standard_normal((512, 512)).astype(np.float32), layout[1] == "t")
    check_gemm(a, b, ops.matmul(da, db).numpy())


LAYOUT_SHAPES = [  # (batch, m, n, k): 128x128 tiles, split-K, ragged edges, M or N not 4-aligned
    (1, 2048, 2044, 100),
    (4, 1020, 1024, 70),
    (1, 256, 256, 16384),
    (1, 2046, 2048, 67),
    (1, 2048, 2047, 33),
    (1, 1024, 1024, 256),   # 64x64 tiles, one workgroup per CU
    (2, 1000, 1020, 100),   # 64x64 tiles, ragged edges
    (1, 1022, 1024, 64),    # 64x64 tiles, M not 4-aligned (TN through registers)
    (1, 384, 256, 24000),   # paired partitions (84), two per direct workgroup
    (1, 256, 384, 30000),   # paired partitions, odd count (79): the last pair is one
    (3, 128, 256, 40000),   # paired partitions over a batch (84 per tile)
]


@pytest.mark.parametrize("batch,m,n,k", LAYOUT_SHAPES)
def test_gemm_layouts_give_the_same_bits(hip, batch, m, n, k):
    """NN, NT, TN and TT of the same values take different loaders (straight to
    LDS as k rows or as k-contiguous rows, or through registers) but accumulate
    every output's k pairs in one order, so all four are the same bits."""
    rng = np.random.default_rng(SEED + m + n + k)
    a = rng.uniform(-2, 2, (batch, m, k)).astype(np.float32)
    b = rng.uniform(-2, 2, (batch, k, n)).astype(np.float32)
    outs = {}
    for lay in ("nn", "nt", "tn", "tt"):
        _, da = layout_view(a, lay[0] == "t")
        _, db = layout_view(b, lay[1] == "t")
        outs[lay] = ops.matmul(da, db).numpy()
    check_gemm(a, b, outs["nn"])
    for lay in ("nt", "tn", "tt"):
        np.testing.assert_array_equal(outs[lay], outs["nn"], err_msg=lay)


def test_gemm_batched_broadcast_conv_shape(hip):
    """conv2d's GEMM: flat weight [Cout, CK] broadcast (stride 0) over a batch
    of cols [N, CK, L], plus the dW (NT) and dcols (TN) products of backward."""
    rng = np.random.default_rng(SEED + 3)
    n, cout, ck, L = 4, 64, 27, 1024
    w = rng.uniform(-0.2, 0.2, (cout, ck)).astype(np.float32)
    cols = rng.uniform(-1, 1, (n, ck, L)).astype(np.float32)
    g = rng.standard_normal((n, cout, L)).astype(np.float32)
    dw_, dc_, dg_ = dev(w), dev(cols), dev(g)
    fwd = ops.matmul(dw_.broadcast_to((1, n, cout, ck)), dc_.reshape(1, n, ck, L)).numpy()
    check_gemm(np.broadcast_to(w, (1, n, cout, ck)), cols[None], fwd)
    dwt = ops.matmul(dg_.reshape(1, n, cout, L), dc_.reshape(1, n, ck, L).transpose(-2, -1)).numpy()
    check_gemm(g[None], np.swapaxes(cols, -1, -2)[None], dwt)
    dcols = ops.matmul(dw_.T.broadcast_to((1, n, ck, cout)), dg_.reshape(1, n, cout, L)).numpy()
    check_gemm(np.broadcast_to(w.T, (1, n, ck, cout)), g[None], dcols)


def test_gemm_large_k_cancellation(hip):
    """reference test_gemm_large_k_backward_error: K=4096, sign-mixed."""
    rng = np.random.default_rng(SEED + 34)
    a = rng.uniform(-2, 2, (4, 4096)).astype(np.float32)
    b = rng.uniform(-2, 2, (4096, 4)).astype(np.float32)
    got = ops.matmul(dev(a), dev(b)).numpy()
    exact = a.astype(np.float64) @ b.astype(np.float64)
    assert np.max(np.abs(got - exact)) <= gemm_atol(a, b)


def test_gemm_empty_k_writes_zeros(hip):
    """K == 0: every output is an empty sum, 0 (the reference's CPU loop), written
    by a fill kernel over whatever the output buffer held."""
    for a_shape, b_shape in (((5, 0), (0, 7)), ((2, 3, 0), (2, 0, 4))):
        out_shape = a_shape[:-1] + b_shape[-1:]
        out = dev(np.full(out_shape, np.nan, np.float32))
        got = ops.matmul(dev(np.zeros(a_shape, np.float32)), dev(np.zeros(b_shape, np.float32)),
                         out=out).numpy()
        assert got.shape == out_shape and not np.signbit(got).any() and (got == 0).all()


def test_gemm_is_deterministic(hip):
    rng = np.random.default_rng(SEED + 33)
    a, b = dev(rng.uniform(-2, 2, (64, 128)).astype(np.float32)), \
        dev(rng.uniform(-2, 2, (128, 64)).astype(np.float32))
    first = ops.matmul(a, b).numpy()
    for _ in range(8):
        assert ops.matmul(a, b).numpy().tobytes() == first.tobytes()


@pytest.mark.parametrize("m,n,k", [(256, 256, 65536), (128, 784, 16384), (64, 128, 784)])
def test_split_k_config3_parity_and_bit_stability(hip, m, n, k):
    """BASELINE config 3's split-K shapes: AUTO splits, matches the oracle
    within tolerance, and repeats bit for bit; a forced split count is also
    bit-stable and agrees with the unsplit product within tolerance."""
    splits, _ = ops.gemm_plan(1, m, n, k)
    assert splits > 1
    rng = np.random.default_rng(SEED + 4)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    da, db = dev(a), dev(b)
    got = ops.matmul(da, db).numpy()
    want = O.matmul(a, b) if m * n * k <= (1 << 31) else None
    check_gemm(a, b, got, want)
    for _ in range(3):
        assert ops.matmul(da, db).numpy().tobytes() == got.tobytes()
    forced = ops.matmul(da, db, split_k=8).numpy()
    assert ops.matmul(da, db, split_k=8).numpy().tobytes() == forced.tobytes()
    unsplit = ops.matmul(da, db, split_k=1).numpy()
    assert normwise_rel_err(forced, unsplit) <= gemm_tolerance(k)


def _carry_fold_f32(parts):
    """The split-K fold of partials in partition order: binary-counter carry
    stack (block + stack[l]), drained from 0.0 in ascending level order
    (gemm_split_k_reduce.comp:48-85), in float32."""
    stack = {}
    for count, v in enumerate(parts):
        block, lvl = v, 0
        while (count >> lvl) & 1:
            block = (block + stack[lvl]).astype(np.float32)
            lvl += 1
        stack[lvl] = block
    total = np.zeros_like(parts[0])
    for lvl in sorted(stack):
        if (len(parts) >> lvl) & 1:
            total = (total + stack[lvl]).astype(np.float32)
    return total


@pytest.mark.parametrize("m,n,k", [(512, 512, 512), (384, 512, 500), (320, 288, 230), (256, 256, 200)])
@pytest.mark.parametrize("layout", ["nn", "nt"])
def test_workgroup_folded_split_k_is_the_fold_of_its_partitions(hip, m, n, k, layout):
    """Products whose plan splits K into 2-4 partitions of at most 4 K-tiles
    run one launch that folds the partitions' partials in LDS. Their result
    is, bit for bit, the carry-stack fold of the device's own products over
    each partition's K range (each of at most 4 K-tiles, never split, so the
    same MFMA sequence from 0), in NN (16-byte staging) and NT (element
    staging), ragged K included."""
    splits, chunk = ops.gemm_plan(1, m, n, k)
    assert 2 <= splits <= 4 and chunk <= 4, (splits, chunk)
    rng = np.random.default_rng(SEED + m + n + k)
    a = rng.standard_normal((m, k), dtype=np.float32)
    b = rng.standard_normal((k, n), dtype=np.float32)

    def prod(x, y):
        dy = dev(y) if layout == "nn" else dev(np.ascontiguousarray(y.T)).transpose(-2, -1)
        return ops.matmul(dev(x), dy).numpy()

    full = prod(a, b)
    parts = []
    for p in range(splits):
        k0, k1 = 32 * chunk * p, min(k, 32 * chunk * (p + 1))
        parts.append(prod(np.ascontiguousarray(a[:, k0:k1]), np.ascontiguousarray(b[k0:k1])))
    assert full.tobytes() == _carry_fold_f32(parts).tobytes()
    assert normwise_rel_err(full, O.matmul(a, b)) <= gemm_tolerance(k)


@pytest.mark.parametrize("splits", [1, 2, 3, 4, 7, 16, 17, 33, 35, 64, 128, 511])
@pytest.mark.parametrize("ne", [1000, 1001])
def test_split_k_reduce_bit_exact(hip, splits, ne):
    """Every partition count (chunked groups plus a remainder) and both the
    16-byte (ne % 4 == 0) and the scalar loads give the oracle's fold."""
    rng = np.random.default_rng(splits + ne)
    ws = (rng.standard_normal(splits * ne) * 1e3).astype(np.float32)
    got = ops.split_k_reduce(dev(ws), splits).numpy()
    assert got.tobytes() == O.split_k_fold(ws, splits).tobytes()


@pytest.mark.parametrize("m,k", [(1, 1), (7, 31), (64, 784), (129, 1000), (4096, 4096),
                                 (300, 33), (9, 2500), (1, 3000), (4095, 2052)])
def test_gemv_bit_exact(hip, m, k):
    """GEMV rounds each product and sums in the oracle's pairwise order."""
    rng = np.random.default_rng(SEED + m + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    x = rng.standard_normal(k).astype(np.float32)
    got = ops.gemv(dev(a), dev(x)).numpy()
    want = O.matmul(a, x[:, None]).ravel()
    assert got.tobytes() == want.tobytes()
    # the matmul entry point routes N == 1 to the same kernel
    assert ops.matmul(dev(a), dev(x)).numpy().tobytes() == want.tobytes()


def test_gemm_config2_full_size_row_sample(hip):
    """4096^3 (the bench workload) and 8192x1024x4096, checked on sampled rows
    against float64."""
    rng = np.random.default_rng(SEED + 5)
    for m, n, k in [(4096, 4096, 4096), (8192, 1024, 4096)]:
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        got = ops.matmul(dev(a), dev(b)).numpy()
        rows = rng.choice(m, 64, replace=False)
        exact = a[rows].astype(np.float64) @ b.astype(np.float64)
        assert normwise_rel_err(got[rows], exact) <= gemm_tolerance(k)
        assert np.max(np.abs(got[rows] - exact)) <= gemm_atol(a[rows], b)


# ---------------------------------------------------------------------------
# im2col / col2im
# ---------------------------------------------------------------------------

WINDOWS = [  # reference test_vulkan_kernels.py:1303-1310
    ((1, 1, 4, 4), (2, 2), (1, 1), (0, 0), (1, 1)),
    ((2, 3, 5, 5), (3, 3), (1, 1), (1, 1), (1, 1)),
    ((1, 2, 6, 6), (2, 2), (2, 2), (0, 0), (1, 1)),
    ((2, 1, 7, 5), (3, 2), (2, 1), (1, 0), (1, 1)),
    ((1, 2, 5, 5), (2, 2), (1, 1), (0, 0), (2, 2)),
    ((1, 1, 17, 17), (3, 3), (1, 1), (1, 1), (1, 1)),
    # BASELINE config 4 geometries at full batch
    ((128, 3, 32, 32), (3, 3), (1, 1), (1, 1), (1, 1)),
    ((128, 64, 32, 32), (3, 3), (1, 1), (1, 1), (1, 1)),
    ((128, 64, 16, 16), (3, 3), (1, 1), (1, 1), (1, 1)),
    # several LDS-staged row blocks per plane (odd out_w, stride 2, dilation)
    ((2, 3, 300, 300), (3, 3), (1, 1), (1, 1), (1, 1)),
    ((1, 2, 200, 101), (3, 3), (1, 1), (1, 1), (1, 1)),
    ((1, 2, 301, 157), (5, 3), (2, 2), (2, 1), (1, 2)),
    # rows too wide for the LDS tile: the per-row gather
    ((1, 1, 3, 4000), (3, 3), (1, 1), (1, 1), (1, 1)),
]


@pytest.mark.parametrize("shape,kernel,stride,pad,dil", WINDOWS)
def test_im2col_col2im_bit_exact(hip, shape, kernel, stride, pad, dil):
    x = np.random.default_rng(SEED).uniform(-1, 1, shape).astype(np.float32)
    cols = ops.im2col(dev(x), kernel, stride, pad, dil)
    want = O.im2col(x, kernel, stride, pad, dil)
    assert cols.numpy().tobytes() == want.tobytes()
    img = ops.col2im(cols, shape[2:], kernel, stride, pad, dil).numpy()
    assert img.tobytes() == O.col2im(want, shape[2:], kernel, stride, pad, dil).tobytes()


def test_im2col_strided_input_view(hip):
    """The image may arrive as a strided view (here: a channel-transposed copy)."""
    x = np.random.default_rng(SEED).uniform(-1, 1, (2, 5, 9, 7)).astype(np.float32)
    d = dev(np.ascontiguousarray(np.transpose(x, (0, 1, 3, 2)))).transpose(2, 3)
    got = ops.im2col(d, (3, 3), (2, 1), (1, 1), (1, 1)).numpy()
    assert got.tobytes() == O.im2col(x, (3, 3), (2, 1), (1, 1), (1, 1)).tobytes()


CONVS = [  # (x shape, Cout, kernel, stride, pad, dilation)
    ((1, 1, 4, 4), 1, (2, 2), (1, 1), (0, 0), (1, 1)),
    ((2, 3, 5, 5), 4, (3, 3), (1, 1), (1, 1), (1, 1)),
    ((2, 1, 7, 5), 2, (3, 2), (2, 1), (1, 0), (1, 1)),
    ((1, 2, 5, 5), 5, (2, 2), (1, 1), (0, 0), (2, 2)),
    ((3, 4, 9, 11), 6, (5, 3), (2, 3), (2, 1), (1, 2)),
    ((2, 40, 20, 20), 70, (3, 3), (1, 1), (1, 1), (1, 1)),
    ((1, 16, 64, 64), 32, (1, 1), (1, 1), (0, 0), (1, 1)),
    ((4, 64, 16, 16), 128, (3, 3), (2, 2), (1, 1), (1, 1)),
    # BASELINE config 4/5 layers at full batch: 128x128 tiles, 64x64 tiles and split-K
    ((128, 3, 32, 32), 64, (3, 3), (1, 1), (1, 1), (1, 1)),
    ((128, 64, 32, 32), 64, (3, 3), (1, 1), (1, 1), (1, 1)),
    ((128, 64, 16, 16), 128, (3, 3), (1, 1), (1, 1), (1, 1)),
    ((1, 64, 8, 8), 128, (3, 3), (1, 1), (1, 1), (1, 1)),
    # the small-window forward with whole blocks but fewer than a workgroup's
    # four: the blocks past the image compute and must not store
    ((3, 8, 8, 8), 32, (1, 1), (1, 1), (0, 0), (1, 1)),
    ((2, 3, 8, 12), 64, (3, 3), (1, 1), (1, 1), (1, 1)),
]


@pytest.mark.parametrize("shape,cout,kernel,stride,pad,dil", CONVS)
def test_implicit_conv_is_bit_identical_to_im2col_then_gemm(hip, shape, cout, kernel, stride,
                                                            pad, dil):
    """vkhip_conv2d gathers the columns inside the GEMM's tile loads; with the
    same plan and summation order its output equals the reference lowering
    (im2col, then the batch-broadcast GEMM) bit for bit, and the oracle's to
    the GEMM tolerance."""
    rng = np.random.default_rng(SEED + shape[1])
    x = rng.uniform(-1, 1, shape).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (cout, shape[1]) + kernel).astype(np.float32)
    got = ops.conv2d(dev(x), dev(w), stride, pad, dil).numpy()
    cols = ops.im2col(dev(x), kernel, stride, pad, dil)
    n, ck, L = cols.shape
    wf = dev(w.reshape(1, 1, cout, ck)).broadcast_to((1, n, cout, ck))
    want = ops.matmul(wf, cols.reshape(1, n, ck, L)).numpy().reshape(got.shape)
    assert got.tobytes() == want.tobytes()
    if n * cout * L * ck <= 1 << 27:
        ref = O.matmul(np.broadcast_to(w.reshape(1, cout, ck), (n, cout, ck)),
                       O.im2col(x, kernel, stride, pad, dil)).reshape(got.shape)
        assert normwise_rel_err(got, ref) <= gemm_tolerance(ck)


SMALL_WINDOW_CONVS = [  # conv_wgrad_small_kernel geometries beyond CONVS' 3-channel layer
    ((4, 2, 16, 16), 5, (3, 3), (2, 2), (1, 1), (1, 1)),
    ((2, 2, 16, 16), 3, (3, 3), (1, 1), (2, 2), (2, 2)),
    ((3, 1, 32, 32), 40, (5, 5), (1, 1), (2, 2), (1, 1)),
    ((2, 8, 9, 9), 64, (2, 2), (1, 1), (0, 0), (1, 1)),
]


@pytest.mark.parametrize("shape,cout,kernel,stride,pad,dil", CONVS + SMALL_WINDOW_CONVS)
def test_implicit_weight_grad_is_bit_identical_to_gemm_on_cols(hip, shape, cout, kernel, stride,
                                                               pad, dil):
    """vkhip_conv2d_weight_grad gathers the transposed columns inside the GEMM;
    its per-image products equal the reference lowering's matmul(grad,
    im2col(x)^T) bit for bit (same plan, K order and split-K fold), and the
    oracle's to the GEMM tolerance. Small windows (C*kh*kw <= 32) run the
    image-staged kernel instead: within the GEMM tolerance of the lowering,
    and the same bits on a second run."""
    rng = np.random.default_rng(SEED + 3 * shape[1])
    x = rng.uniform(-1, 1, shape).astype(np.float32)
    cols = ops.im2col(dev(x), kernel, stride, pad, dil)
    n, ck, L = cols.shape
    oh = ops.window_count(shape[2], kernel[0], stride[0], pad[0], dil[0])
    ow = ops.window_count(shape[3], kernel[1], stride[1], pad[1], dil[1])
    g = rng.standard_normal((n, cout, oh, ow)).astype(np.float32)
    print(f"weight_grad x={shape} cout={cout} k={kernel} s={stride} p={pad} d={dil}", flush=True)
    got = ops.conv2d_weight_grad(dev(x), dev(g), kernel, stride, pad, dil).numpy()
    want = ops.matmul(dev(g.reshape(1, n, cout, L)),
                      cols.reshape(1, n, ck, L).transpose(-2, -1)).numpy().reshape(got.shape)
    if small_window(shape, cout, kernel, L):
        assert normwise_rel_err(got, want) <= gemm_tolerance(L)
        again = ops.conv2d_weight_grad(dev(x), dev(g), kernel, stride, pad, dil).numpy()
        assert got.tobytes() == again.tobytes()
    else:
        assert got.tobytes() == want.tobytes()
    if n * cout * L * ck <= 1 << 27:
        ref = O.matmul(g.reshape(n, cout, L),
                       np.ascontiguousarray(np.swapaxes(O.im2col(x, kernel, stride, pad, dil), 1, 2)))
        assert normwise_rel_err(got, ref) <= gemm_tolerance(L)


@pytest.mark.parametrize("shape,cout,kernel,stride,pad,dil",
                         CONVS + SMALL_WINDOW_CONVS +
                         [((8, 16, 16, 16), 24, (3, 3), (1, 1), (1, 1), (1, 1)),
                          ((3, 5, 12, 16), 7, (5, 5), (1, 1), (2, 2), (1, 1)),
                          ((600, 1, 8, 8), 6, (3, 3), (1, 1), (1, 1), (1, 1))])
def test_weight_grad_sum_is_the_batch_sum_of_the_products(hip, shape, cout, kernel, stride, pad,
                                                          dil):
    """vkhip_conv2d_weight_grad_sum: with out_h*out_w a multiple of 32 the batch
    is folded into the product's K axis (K = N*out_h*out_w) -- within the GEMM
    tolerance for that K of the per-image products + batch sum and of the
    oracle, whose graph it replaces; otherwise it runs that graph and gives
    its bits."""
    rng = np.random.default_rng(SEED + 5 * shape[1])
    x = rng.uniform(-1, 1, shape).astype(np.float32)
    n = shape[0]
    oh = ops.window_count(shape[2], kernel[0], stride[0], pad[0], dil[0])
    ow = ops.window_count(shape[3], kernel[1], stride[1], pad[1], dil[1])
    L = oh * ow
    g = rng.standard_normal((n, cout, oh, ow)).astype(np.float32)
    print(f"weight_grad_sum x={shape} cout={cout} L={L}", flush=True)
    got = ops.conv2d_weight_grad_sum(dev(x), dev(g), kernel, stride, pad, dil).numpy()
    per = ops.conv2d_weight_grad(dev(x), dev(g), kernel, stride, pad, dil)
    want = ops.sum(per, [0]).numpy()
    ck = shape[1] * kernel[0] * kernel[1]
    assert got.shape == (cout, ck)
    if L % 32:
        assert got.tobytes() == want.tobytes()
    else:
        assert normwise_rel_err(got, want) <= gemm_tolerance(n * L)
    if n * cout * L * ck <= 1 << 27:
        cols = np.ascontiguousarray(np.swapaxes(O.im2col(x, kernel, stride, pad, dil), 1, 2))
        ref = O.sum(O.matmul(g.reshape(n, cout, L), cols), [0])
        assert normwise_rel_err(got, ref) <= gemm_tolerance(n * L)


@pytest.mark.parametrize("shape,cout,kernel,stride,pad,dil",
                         CONVS + [((8, 16, 16, 16), 24, (3, 3), (1, 1), (1, 1), (1, 1)),
                                  ((2, 3, 9, 9), 4, (3, 3), (1, 1), (3, 3), (1, 1)),
                                  ((3, 5, 12, 16), 7, (5, 5), (1, 1), (2, 2), (1, 1)),
                                  ((2, 40, 12, 10), 16, (5, 3), (1, 1), (2, 1), (1, 2)),
                                  ((2, 32, 8, 8), 8, (1, 1), (1, 1), (0, 0), (1, 1)),
                                  # thin layers: four K-tiles with a partial one, dilation
                                  ((2, 2, 6, 10), 100, (3, 3), (1, 1), (1, 1), (1, 1)),
                                  ((1, 4, 5, 7), 40, (2, 2), (1, 1), (0, 0), (2, 2)),
                                  ((300, 3, 20, 20), 33, (3, 3), (1, 1), (1, 1), (1, 1))])
def test_input_grad_matches_the_tn_product_and_col2im(hip, shape, cout, kernel, stride, pad, dil):
    """vkhip_conv2d_input_grad against the reference lowering on the device
    (the TN product flat_weight^T @ grad into columns, then col2im) and the
    oracle: unit strides with pad <= dilation*(k-1) run the convolution of the
    gradient with the flipped, transposed weight (within the GEMM tolerance
    for K = Cout*kh*kw) when there are at least 32 input channels; thin layers
    (C*kh*kw <= 32, unit strides) fold the columns of a band of rows in LDS,
    and they and the other geometries give the lowering's bits."""
    rng = np.random.default_rng(SEED + 7 * shape[1])
    n, c, h, w = shape
    oh = ops.window_count(h, kernel[0], stride[0], pad[0], dil[0])
    ow = ops.window_count(w, kernel[1], stride[1], pad[1], dil[1])
    g = rng.standard_normal((n, cout, oh, ow)).astype(np.float32)
    wt = rng.uniform(-0.5, 0.5, (cout, c) + kernel).astype(np.float32)
    print(f"input_grad x={shape} cout={cout} k={kernel} s={stride} p={pad} d={dil}", flush=True)
    got = ops.conv2d_input_grad(dev(g), dev(wt), (h, w), stride, pad, dil).numpy()
    ck, L = c * kernel[0] * kernel[1], oh * ow
    wf = dev(wt.reshape(1, 1, cout, ck)).broadcast_to((1, n, cout, ck))
    dcols = ops.matmul(wf.transpose(-2, -1), dev(g.reshape(1, n, cout, L))).reshape(n, ck, L)
    want = ops.col2im(dcols, (h, w), kernel, stride, pad, dil).numpy()
    # C*kh*kw <= 32 with unit strides: the columns of a band of rows in LDS,
    # then col2im there (win_dx_kernel): still the lowering's bits
    thin = stride == (1, 1) and c * kernel[0] * kernel[1] <= 32 and cout <= 128
    fused = (stride == (1, 1) and all(d * (k - 1) >= p for d, k, p in zip(dil, kernel, pad))
             and c >= 32 and not thin)
    if fused:
        assert normwise_rel_err(got, want) <= gemm_tolerance(cout * kernel[0] * kernel[1])
    else:
        assert got.tobytes() == want.tobytes()
    if n * cout * L * ck <= 1 << 27:
        cols = O.matmul(np.ascontiguousarray(np.broadcast_to(wt.reshape(cout, ck).T, (n, ck, cout))),
                        g.reshape(n, cout, L))
        ref = O.col2im(cols, (h, w), kernel, stride, pad, dil)
        assert normwise_rel_err(got, ref) <= gemm_tolerance(cout * kernel[0] * kernel[1])


def test_weight_grad_sum_edges(hip):
    """An empty batch gives zeros; a gradient of the wrong extent is refused."""
    x = np.ones((0, 2, 8, 8), np.float32)
    g = np.ones((0, 3, 8, 8), np.float32)
    got = ops.conv2d_weight_grad_sum(dev(x), dev(g), 3, 1, 1).numpy()
    assert got.shape == (3, 18) and not got.any()
    x = np.ones((2, 2, 8, 8), np.float32)
    with pytest.raises(ValueError):
        ops.conv2d_weight_grad_sum(dev(x), dev(np.ones((2, 3, 7, 8), np.float32)), 3, 1, 1)


def test_implicit_conv_strided_image(hip):
    """A channels-last image handed over as an NCHW view, and an image whose
    batch stride leaves a gap between samples."""
    rng = np.random.default_rng(SEED)
    x = rng.uniform(-1, 1, (3, 6, 9, 7)).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (5, 6, 3, 3)).astype(np.float32)
    want = ops.conv2d(dev(x), dev(w), (2, 1), (1, 1), (1, 1)).numpy()
    nhwc = dev(np.ascontiguousarray(np.transpose(x, (0, 2, 3, 1))))
    view = _view(nhwc, (3, 6, 9, 7), (9 * 7 * 6, 1, 7 * 6, 6))
    assert ops.conv2d(view, dev(w), (2, 1), (1, 1), (1, 1)).numpy().tobytes() == want.tobytes()
    padded = np.zeros((3, 8, 9, 7), np.float32)
    padded[:, :6] = x
    gap = _view(dev(padded), (3, 6, 9, 7), (8 * 63, 63, 7, 1))
    assert ops.conv2d(gap, dev(w), (2, 1), (1, 1), (1, 1)).numpy().tobytes() == want.tobytes()


def test_implicit_conv_window_limit(hip):
    """Windows of more than 63 elements are refused by the gather (the tensor
    layer lowers them through im2col + matmul instead); 63 still works."""
    rng = np.random.default_rng(SEED)
    x = rng.uniform(-1, 1, (1, 2, 12, 12)).astype(np.float32)
    with pytest.raises(Exception, match="window"):
        ops.conv2d(dev(x), dev(np.ones((3, 2, 8, 8), np.float32)))
    w = rng.uniform(-0.5, 0.5, (3, 2, 9, 7)).astype(np.float32)
    got = ops.conv2d(dev(x), dev(w), 1, 2).numpy()
    cols = ops.im2col(dev(x), (9, 7), 1, 2)
    want = ops.matmul(dev(w.reshape(1, 1, 3, -1)).broadcast_to((1, 1, 3, 126)),
                      cols.reshape(1, 1, 126, cols.shape[2])).numpy().reshape(got.shape)
    assert got.tobytes() == want.tobytes()


def _view(base: DeviceArray, shape, strides) -> DeviceArray:
    return DeviceArray(shape, np.float32, strides=strides, buffer=base.buffer, offset=base.offset)


@pytest.mark.parametrize("shape", [(3, 5, 7, 8), (2, 2, 3, 4), (1, 3, 5, 64), (1, 1, 4, 256),
                                   (2, 2, 5, 12), (5, 3, 9, 16)])
def test_col2im_3x3_same_size_bit_exact(hip, shape):
    """3x3 / stride 1 / padding 1 col2im over arbitrary columns (not an im2col
    image): neighbouring pixels' terms, the image border, signed zeros and
    partial waves; widths 4..256 take the register kernel, 12 the staged one."""
    n, c, h, w = shape
    rng = np.random.default_rng(SEED + h * w)
    cols = rng.standard_normal((n, c * 9, h * w)).astype(np.float32)
    cols[..., ::7] = -0.0
    cols[0, :, 1] = np.float32(1e8) * np.sign(rng.standard_normal(c * 9)).astype(np.float32)
    got = ops.col2im(dev(cols), (h, w), (3, 3), (1, 1), (1, 1)).numpy()
    assert got.tobytes() == O.col2im(cols, (h, w), (3, 3), (1, 1), (1, 1)).tobytes()


def test_col2im_fold_order_fixture(hip):
    """reference test_col2im_fold_is_bit_reproducible (test_vulkan_kernels.py:1342-1356)."""
    vals = np.array([1e8, 1.0, -1e8, 1e-8, 1.0, -1.0, 1e7, 1.0, -1e7], np.float32)
    cols = np.zeros((1, 9, 16), np.float32)
    cols[0, :, :] = vals[:, None]
    got = ops.col2im(dev(cols), (4, 4), (3, 3), (1, 1), (1, 1)).numpy()
    assert got.tobytes() == O.col2im(cols, (4, 4), (3, 3), (1, 1), (1, 1)).tobytes()
    again = ops.col2im(dev(cols), (4, 4), (3, 3), (1, 1), (1, 1)).numpy()
    assert again.tobytes() == got.tobytes()


# ---------------------------------------------------------------------------
# softmax
# ---------------------------------------------------------------------------

def check_softmax(got, want, n):
    tol = gemm_tolerance(n)
    big = np.abs(want) > 1e-30
    rel = np.abs(got[big] - want[big]) / np.abs(want[big])
    assert rel.size == 0 or rel.max() <= tol, f"max rel err {rel.max():.3g} > {tol:.3g}"
    assert np.all(np.abs(got[~big] - want[~big]) <= 1e-30)


@pytest.mark.parametrize("shape", [(4096, 1000), (256, 32768), (64, 10), (128, 100),
                                   (3, 1), (5, 4097), (7, 2048), (2, 3000), (33, 8192),
                                   (9, 4096), (5, 16384), (3000, 257), (1025, 64),
                                   (3, 100000), (512, 16384)])
@pytest.mark.parametrize("log", [False, True])
def test_softmax_parity(hip, shape, log):
    x = (np.random.default_rng(SEED + shape[1]).standard_normal(shape) * 2).astype(np.float32)
    got = ops.softmax(dev(x), -1, log).numpy()
    want = O.softmax(x, -1, log)
    if log:
        assert normwise_rel_err(got, want) <= gemm_tolerance(shape[1])
    else:
        check_softmax(got, want, shape[1])


@pytest.mark.parametrize("n,structure", [(40000, "softmax_split_rows"),
                                         (65537, "softmax_split_rows"),
                                         (32769, "softmax_split_rows"),
                                         (131072, "softmax_split_rows"),
                                         (12290, "softmax_workgroup_per_row"),
                                         (8196, "softmax_workgroup_per_row"),
                                         (32768, "softmax_workgroup_per_row")])
@pytest.mark.parametrize("log", [False, True])
def test_softmax_long_rows_special_values(hip, n, structure, log):
    """Rows longer than 2048: a workgroup per row up to 32768 floats, beyond
    that 4096-float chunks on separate workgroups (chunk statistics, then
    outputs), including ragged last chunks and unaligned rows. A chunk of -inf
    only, a NaN, a +inf and an all -inf row give the oracle's values."""
    from vkml_amd.device import DecisionRecorder

    x = (np.random.default_rng(SEED + n).standard_normal((6, n)) * 2).astype(np.float32)
    x[1, :4096] = -np.inf          # a whole chunk of -inf
    x[1, -3:] = -np.inf
    x[2, n // 2] = np.nan
    x[3, 5000] = np.inf
    x[4, :] = -np.inf
    x[5, ::7] = -np.inf
    with DecisionRecorder() as rec:
        got = ops.softmax(dev(x), -1, log).numpy()
    assert [d["chose"] for d in rec.decisions if d["site"] == "softmax.structure"] == [structure]
    want = O.softmax(x, -1, log)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_array_equal(np.isneginf(got), np.isneginf(want))
    for r in (0, 1, 5):
        fin = np.isfinite(want[r])
        if log:
            assert normwise_rel_err(got[r][fin], want[r][fin]) <= gemm_tolerance(n)
        else:
            check_softmax(got[r], want[r], n)


STABILITY_INPUTS = golden("softmax_stability_inputs")["inputs"]  # test_vulkan_kernels.py:808-817


@pytest.mark.parametrize("name", list(STABILITY_INPUTS))
@pytest.mark.parametrize("log", [False, True])
def test_softmax_stability(hip, name, log):
    x = np.array(STABILITY_INPUTS[name], np.float32)
    got = ops.softmax(dev(x), -1, log).numpy()
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, O.softmax(x, -1, log), rtol=1e-5, atol=1e-6)


def test_softmax_exponential_accuracy(hip):
    """The softmax kernels' exponential, read back exactly: for a row [0, s]
    with s < -17, 1 + exp(s) rounds to 1, so the second output IS exp(s).
    Within 2 ulp of the correctly rounded exp for normal results, within
    2^-126 below; rows [0, s] with s in (-17, 0] stay within 4 ulp of
    exp(s) / (1 + exp(s))."""
    s = np.concatenate([np.linspace(-103.0, -17.0, 4001), np.linspace(-17.0, 0.0, 2001)[1:]])
    s = s.astype(np.float32)
    rows = np.stack([np.zeros_like(s), s], axis=1)
    got = ops.softmax(dev(rows), -1).numpy()[:, 1].astype(np.float64)
    e = np.exp(s.astype(np.float64))
    want = np.where(s < -17.0, e, e / (1.0 + e))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    normal = want >= 2.0 ** -126
    deep = s < -17.0
    err = np.abs(got - want) / ulp
    assert err[normal & deep].max() <= 2.0, err[normal & deep].max()
    assert err[normal & ~deep].max() <= 4.0, err[normal & ~deep].max()
    assert np.abs(got - want)[~normal].max() <= 2.0 ** -126


def test_softmax_non_last_axis(hip):
    x = np.random.default_rng(1).standard_normal((6, 37, 5)).astype(np.float32)
    for axis in (0, 1):
        got = ops.softmax(dev(x), axis).numpy()
        check_softmax(got, O.softmax(x, axis), x.shape[axis])


# ---------------------------------------------------------------------------
# reductions
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape,axes", [
    ((8192, 4096), [1]),        # BASELINE config 5 standalone
    ((64, 128), [0]),           # Linear bias gradient
    ((128, 64 * 27), [0]),      # conv weight-gradient batch sum (outer axis)
    ((1024, 1024), [1]),
    ((4096, 256), [1]),
    ((3, 100003), [1]),         # long rows, irregular tree
    ((5, 7, 33), [0, 2]),
    ((2, 3, 4, 5), None),
    ((17, 9), [1]),             # below one leaf per row
    ((128, 64, 32, 32), [0, 2, 3]),  # conv bias gradient: split tree over 131072
    ((4096, 64), [0]),          # strided column sums, split tree
    ((2, 3, 70001), [0, 2]),    # uneven tree over two strided axes
    ((50000, 3), [0]),          # three outputs, 128 subtrees of 390-391
    ((7, 3000), [1]),           # two rows per workgroup, odd row count, uneven tree
    ((6, 5, 2052), [2]),        # two rows per workgroup over two kept axes
    ((2, 3, 600000), [0, 2]),   # subtrees too long to stage: per-output workgroups
    ((256, 100), [0]),          # strided, 8 pairwise leaves: a wave per leaf
    ((100, 77), [0]),           # 4 uneven leaves
    ((33, 5), [0]),             # 2 leaves of 16 and 17
    ((128, 9216), [0]),         # many outputs, 4 leaves each
    ((3, 50, 7), [0, 1]),       # 150 over two strided axes, 8 leaves
])
def test_sum_mean_bit_exact(hip, shape, axes):
    x = (np.random.default_rng(SEED).standard_normal(shape) * 10).astype(np.float32)
    d = dev(x)
    assert ops.sum(d, axes).numpy().tobytes() == O.sum(x, axes).tobytes()
    assert ops.mean(d, axes).numpy().tobytes() == O.mean(x, axes).tobytes()


def test_split_tree_sums_back_to_back(hip):
    """Split-tree reductions (subtree partials, then their balanced fold)
    interleaved with different output and subtree counts (64 x 16, 128 x 4,
    3 x 128, 200 x 4 partials) share the reduction workspace; every result
    stays the oracle's bits."""
    rng = np.random.default_rng(SEED + 5)
    cases = [((128, 64, 32, 32), [0, 2, 3]), ((128, 128, 16, 16), [0, 2, 3]), ((50000, 3), [0]),
             ((4096, 64), [0]), ((16, 200, 8, 32), [0, 2, 3])]
    xs = [(rng.standard_normal(shape) * 4).astype(np.float32) for shape, _ in cases]
    ds = [dev(x) for x in xs]
    want = [O.sum(x, axes).tobytes() for x, (_, axes) in zip(xs, cases)]
    for rep in range(3):
        for i in (0, 2, 1, 4, 3, 0, 0, 1):
            got = ops.sum(ds[i], cases[i][1]).numpy().tobytes()
            assert got == want[i], f"repeat {rep}, case {cases[i][0]}"


@pytest.mark.parametrize("shape,axis", [((8192, 4096), 1), ((1024, 1024), 1), ((64, 10), 1),
                                        ((100, 37), 0), ((3, 5000), 1)])
def test_max_min_argmax_exact(hip, shape, axis):
    x = np.random.default_rng(SEED).standard_normal(shape).astype(np.float32)
    x[..., ::97] = np.float32(2.5)  # planted ties
    d = dev(x)
    assert ops.amax(d, [axis]).numpy().tobytes() == O.amax(x, [axis]).tobytes()
    assert ops.amin(d, [axis]).numpy().tobytes() == O.amin(x, [axis]).tobytes()
    np.testing.assert_array_equal(ops.argmax(d, axis).numpy(), O.argmax(x, axis))
    np.testing.assert_array_equal(ops.argmin(d, axis).numpy(), O.argmin(x, axis))


def special_rows(n: int, seed: int) -> np.ndarray:
    """48 rows of width n: planted NaNs, signed-zero ties, infinities,
    all -inf and all-NaN rows - the cases where selection order shows."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((48, n)).astype(np.float32)
    for r in range(8):
        x[r, rng.integers(0, n, 1 + r % 3)] = np.nan
    x[8:16] = np.where(rng.integers(0, 2, (8, n)) == 1, np.float32(0.0), np.float32(-0.0))
    x[16:24] = -np.abs(x[16:24])
    x[16:24, rng.integers(0, n, 3)] = np.float32(-0.0)
    x[16:24, rng.integers(0, n, 3)] = np.float32(0.0)
    x[24:28] = -np.inf
    x[28:32] = np.nan
    x[32:40, rng.integers(0, n, 4)] = np.inf
    x[32:40, rng.integers(0, n, 2)] = -np.inf
    x[36:40, n - 1] = np.nan
    x[40:48, rng.integers(0, n, 5)] = -np.inf
    return x


@pytest.mark.parametrize("n", [1, 10, 80, 300, 1000, 2500, 4096, 9000, 40000])
def test_select_special_values_exact(hip, n):
    """max/min (first NaN, else first extreme, which fixes a zero's sign) and
    argmax/argmin (NaN skipped, first strict improvement) across every row
    class the device dispatches, along the last axis and along axis 0."""
    x = special_rows(n, SEED + n)
    for arr, axis in ((x, 1), (np.ascontiguousarray(x.T), 0)):
        d = dev(arr)
        assert ops.amax(d, [axis]).numpy().tobytes() == O.amax(arr, [axis]).tobytes(), axis
        assert ops.amin(d, [axis]).numpy().tobytes() == O.amin(arr, [axis]).tobytes(), axis
        np.testing.assert_array_equal(ops.argmax(d, axis).numpy(), O.argmax(arr, axis))
        np.testing.assert_array_equal(ops.argmin(d, axis).numpy(), O.argmin(arr, axis))


def test_reduce_known_answers_and_nan(hip):
    a = np.array([[1, 5, 5], [4, 2, 4]], np.float32)
    np.testing.assert_array_equal(ops.argmax(dev(a), 1).numpy(), [1, 0])
    np.testing.assert_array_equal(ops.argmin(dev(a), 1).numpy(), [0, 1])
    x = np.array([[1.0, np.nan, 3.0, 2.0] * 20, [np.nan, np.nan, -np.inf, -np.inf] * 20],
                 np.float32)
    np.testing.assert_array_equal(ops.argmax(dev(x), 1).numpy(), O.argmax(x, 1))
    assert np.isnan(ops.amax(dev(x), [1]).numpy()).all()


# ---------------------------------------------------------------------------
# max-pool and scaled_add
# ---------------------------------------------------------------------------

POOLS = [
    ((1, 1, 4, 4), (2, 2), (2, 2), (0, 0)),
    ((2, 3, 6, 6), (2, 2), (2, 2), (0, 0)),
    ((1, 2, 5, 5), (3, 3), (1, 1), (1, 1)),
    ((2, 1, 7, 5), (3, 2), (2, 1), (1, 0)),
    ((1, 1, 17, 17), (3, 3), (2, 2), (1, 1)),
    ((128, 64, 32, 32), (2, 2), (2, 2), (0, 0)),  # BASELINE configs 4/5
    ((128, 128, 16, 16), (2, 2), (2, 2), (0, 0)),
]


@pytest.mark.parametrize("shape,kernel,stride,pad", POOLS)
def test_max_pool2d_forward_backward_bit_exact(hip, shape, kernel, stride, pad):
    x = np.random.default_rng(SEED).uniform(-3, 3, shape).astype(np.float32)
    y = ops.max_pool2d(dev(x), kernel, stride, pad).numpy()
    assert y.tobytes() == O.max_pool2d(x, kernel, stride, pad).tobytes()
    g = np.random.default_rng(SEED + 1).uniform(-1, 1, y.shape).astype(np.float32)
    gx = ops.max_pool2d_backward(dev(g), dev(x), kernel, stride, pad).numpy()
    assert gx.tobytes() == O.max_pool2d_backward(g, x, kernel, stride, pad).tobytes()


@pytest.mark.parametrize("shape", [(3, 5, 8, 12), (2, 4, 16, 4), (1, 2, 6, 8), (2, 3, 8, 10)])
def test_max_pool2d_ties_nan_and_signed_zero(hip, shape):
    """2x2/stride-2 windows (the tiled fast path where W % 4 == 0, the general
    kernel otherwise): values from {-1, 0, 1} so most windows tie, planted
    NaNs that the window scan skips, -0 gradients, and for the backward some
    windows with no maximum at all (all -inf / NaN), which route nothing."""
    rng = np.random.default_rng(SEED + sum(shape))
    x = rng.integers(-1, 2, shape).astype(np.float32)
    plant = rng.random(shape) < 0.05
    plant[..., ::2, ::2] = False  # every window keeps a number for the forward
    x[plant] = np.nan
    x[..., 0:2, 0:2] = np.where(rng.random((2, 2)) < 0.5, np.float32(0.0), np.float32(-0.0))
    d = dev(x)
    y = ops.max_pool2d(d, (2, 2), (2, 2)).numpy()
    assert y.tobytes() == O.max_pool2d(x, (2, 2), (2, 2), (0, 0)).tobytes()
    g = rng.uniform(-1, 1, y.shape).astype(np.float32)
    g[rng.random(g.shape) < 0.2] = np.float32(-0.0)
    xb = x.copy()
    xb[0, 0, 2:4, 2:4] = -np.inf
    xb[-1, -1, -2:, -2:] = np.nan
    gx = ops.max_pool2d_backward(dev(g), dev(xb), (2, 2), (2, 2)).numpy()
    assert gx.tobytes() == O.max_pool2d_backward(g, xb, (2, 2), (2, 2), (0, 0)).tobytes()


def test_max_pool2d_tie(hip):
    x = np.array([[[[5.0, 5.0], [1.0, 2.0]]]], np.float32)
    g = ops.max_pool2d_backward(dev(np.ones((1, 1, 1, 1), np.float32)), dev(x), (2, 2)).numpy()
    np.testing.assert_array_equal(g, [[[[1, 0], [0, 0]]]])


def test_scaled_add_is_two_rounded_products(hip):
    rng = np.random.default_rng(6)
    a = rng.standard_normal(10001).astype(np.float32)
    b = rng.standard_normal(10001).astype(np.float32)
    got = ops.scaled_add(dev(a), dev(b), 0.9, -0.1).numpy()
    want = (a * np.float32(0.9)).astype(np.float32) + (b * np.float32(-0.1)).astype(np.float32)
    assert got.tobytes() == want.astype(np.float32).tobytes()


def test_caching_allocator_reuses_and_accounts(hip):
    """vkhip_alloc/vkhip_free: a freed block of the same size is handed out
    again, the byte counts follow, an unknown pointer is refused, and
    release_cached empties the cache."""
    from ctypes import byref, c_void_p

    lib = _lib.load()
    b = hip
    b.synchronize()
    base = b.memory_stats()
    p = c_void_p()
    assert lib.vkhip_alloc(3 << 20, byref(p)) == 0 and p.value
    first = p.value
    assert b.memory_stats()["in_use"] == base["in_use"] + (3 << 20)
    assert lib.vkhip_free(c_void_p(first)) == 0
    assert lib.vkhip_free(c_void_p(first)) == _lib.ERR_INVALID  # already freed
    q = c_void_p()
    assert lib.vkhip_alloc((3 << 20) - 100, byref(q)) == 0  # rounds to the same size
    assert q.value == first
    # A reused block is ordinary memory: write and read it through the stream.
    x = np.arange(1 << 18, dtype=np.float32)
    assert lib.vkhip_copy_from_host(q, x.ctypes.data_as(c_void_p), x.nbytes) == 0
    y = np.empty_like(x)
    assert lib.vkhip_copy_to_host(y.ctypes.data_as(c_void_p), q, x.nbytes) == 0
    assert y.tobytes() == x.tobytes()
    assert lib.vkhip_free(q) == 0
    assert b.memory_stats()["cached"] >= 3 << 20
    b.release_cached()
    assert b.memory_stats()["cached"] == 0
    assert lib.vkhip_free(c_void_p(0x1000)) == _lib.ERR_INVALID


@pytest.mark.parametrize("sizes", [[1 << 10, 3 << 20, 5 << 20, 7, 4 << 20, 1 << 22, 333],
                                   [13 << 20, 9 << 20, 17 << 20, 20 << 20]])
def test_host_copies_through_staging_slots(hip, sizes):
    """vkhip_copy_from_host returns once the caller's bytes are copied (small
    uploads go through pinned slots whose DMA is still queued): overwriting the
    host buffer right away must not change what lands on the device, uploads
    queued behind a running kernel land after it, and a ring's worth of
    uploads (chunked, reusing slots) and the direct path above it all arrive."""
    from ctypes import c_void_p

    lib = _lib.load()
    rng = np.random.default_rng(SEED + 91)
    devs, wants = [], []
    big = dev(rng.standard_normal((4096, 4096)).astype(np.float32))
    for nbytes in sizes:
        n = nbytes // 4 + 1
        x = rng.standard_normal(n).astype(np.float32)
        d = DeviceArray((n,), np.float32)
        ops.matmul(big, big)  # keep the stream busy while the upload is queued
        assert lib.vkhip_copy_from_host(c_void_p(d.ptr), x.ctypes.data_as(c_void_p), x.nbytes) == 0
        wants.append(x.copy())
        x[:] = -1.0  # the caller's buffer is free once the call returns
        devs.append(d)
    for d, want in zip(devs, wants):
        assert d.numpy().tobytes() == want.tobytes()
    # Small downloads through a slot, back to back.
    for d, want in zip(devs, wants):
        head = np.empty(min(want.size, 1000), np.float32)
        assert lib.vkhip_copy_to_host(head.ctypes.data_as(c_void_p), c_void_p(d.ptr), head.nbytes) == 0
        assert head.tobytes() == want[:head.size].tobytes()


def test_decision_facts_join_profile_records(hip):
    """Decision facts name the kernel each op chose with the numbers behind it,
    and their dispatch ids join with the per-unit timing records (reference
    observe::Decision and ProfileRecord)."""
    from vkml_amd.device import DecisionRecorder

    rng = np.random.default_rng(SEED + 77)
    a = dev(rng.standard_normal((256, 65536)).astype(np.float32))
    b = dev(rng.standard_normal((65536, 256)).astype(np.float32))
    x = dev(rng.standard_normal((4096, 1000)).astype(np.float32))
    g = dev(rng.standard_normal((16, 64, 32, 32)).astype(np.float32))
    hip.set_profiling(True)
    hip.profile_records()
    with DecisionRecorder() as rec:
        ops.matmul(a, b)
        ops.softmax(x, -1)
        ops.sum(g, [0, 2, 3])
    records = hip.profile_records()
    hip.set_profiling(False)
    by_site = {}
    for d in rec.decisions:
        by_site.setdefault(d["site"], []).append(d)
    splits, _ = ops.gemm_plan(1, 256, 256, 65536)
    kern = by_site["matmul.kernel"][-1]
    assert kern["chose"] == "gemm_mfma_128x128" and kern["required"] == 4
    assert kern["available"] == hip.capabilities().compute_units
    split = by_site["matmul.split_k"][-1]
    assert split["chose"] == f"split_k_{splits}" and split["dispatch"] == kern["dispatch"]
    soft = by_site["softmax.structure"][-1]
    assert soft["chose"] == "softmax_wave_per_row" and (soft["required"], soft["available"]) == (1000, 4096)
    red = by_site["reduce.structure"][-1]
    assert red["chose"] == "reduce_split_tree" and (red["required"], red["available"]) == (16 * 1024, 64)
    timed = {r["dispatch"]: r for r in records}
    for d, label in ((kern, "matmul"), (soft, "softmax"), (red, "reduce")):
        assert timed[d["dispatch"]]["label"] == label and timed[d["dispatch"]]["gpu_ms"] > 0
    assert len({kern["dispatch"], soft["dispatch"], red["dispatch"]}) == 3
    ops.matmul(a, b)
    assert hip.profile_records() == []  # profiling off again


def test_errors_are_reported_not_crashed(hip):
    a = dev(np.ones((3, 4), np.float32))
    b = dev(np.ones((5, 6), np.float32))
    with pytest.raises(ValueError):
        ops.matmul(a, b)
    lib = _lib.load()
    d = _lib.operand((3, 4), (4, 1))
    e = _lib.operand((5, 6), (6, 1))
    from ctypes import byref, c_void_p
    code = lib.vkhip_gemm(c_void_p(a.ptr), byref(d), c_void_p(b.ptr), byref(e), c_void_p(a.ptr),
                          None)
    assert code == _lib.ERR_INVALID and b"inner dimensions" in lib.vkhip_last_error()


def test_host_provided_stream(hip):
    """vkhip_set_stream: work (an upload through the staging slots, a GEMM, a
    softmax and a download) runs on a stream the host hands over, here one
    made with hipStreamCreate (default priority), in order and with the
    results of the backend's own stream; vkhip_set_stream(NULL) returns to it."""
    import ctypes

    hiprt = ctypes.CDLL("libamdhip64.so")
    rng = np.random.default_rng(SEED + 93)
    a = rng.standard_normal((300, 200)).astype(np.float32)
    b = rng.standard_normal((200, 100)).astype(np.float32)
    want = ops.matmul(dev(a), dev(b)).numpy()
    want_sm = ops.softmax(dev(want), -1).numpy()
    own = hip.stream_handle()
    side = ctypes.c_void_p()
    assert hiprt.hipStreamCreate(ctypes.byref(side)) == 0 and side.value
    try:
        hip.set_stream(side.value)
        assert hip.stream_handle() == side.value
        got = ops.matmul(dev(a), dev(b))
        got_sm = ops.softmax(got, -1).numpy()
        assert got.numpy().tobytes() == want.tobytes()
        assert got_sm.tobytes() == want_sm.tobytes()
    finally:
        hip.set_stream(None)
        assert hiprt.hipStreamDestroy(side) == 0
    assert hip.stream_handle() == own
    assert ops.matmul(dev(a), dev(b)).numpy().tobytes() == want.tobytes()


def test_copy_device_to_device_batch(hip):
    """vkhip_copy_device_to_device: several disjoint copies as one unit of work,
    16-byte multiples and odd sizes, batched up to eight pairs per launch
    (twelve pairs here: two launches; 1001 floats is past the batch's 4 KB of
    byte copies and goes alone, as do 64 MB and more), byte for byte;
    mismatched or strided pairs are refused on the host."""
    rng = np.random.default_rng(SEED + 95)
    sizes = (4096, 1001, 37, 1 << 20, 1, 3, 256, 1023, 5, (16 << 20) + 4, 8, 12)
    srcs = [rng.standard_normal(n).astype(np.float32) for n in sizes]
    src_d = [dev(x) for x in srcs]
    dst_d = [DeviceArray((x.size,), np.float32) for x in srcs]
    hip.copy_device_to_device(list(zip(dst_d, src_d)))
    for d, x in zip(dst_d, srcs):
        assert d.numpy().tobytes() == x.tobytes()
    with pytest.raises(ValueError):
        hip.copy_device_to_device([(DeviceArray((10,), np.float32), dev(np.zeros(11, np.float32)))])
    with pytest.raises(ValueError):
        m = dev(np.zeros((4, 6), np.float32))
        hip.copy_device_to_device([(DeviceArray((6, 4), np.float32), m.transpose(0, 1))])


@pytest.mark.parametrize("shape,perm", [((8192, 256), (1, 0)), ((256, 100), (1, 0)), ((65, 130), (1, 0)),
                                        ((3, 100, 37), (0, 2, 1)), ((2, 3, 65, 130), (0, 1, 3, 2)),
                                        ((2, 3, 5, 7), (1, 0, 3, 2)), ((1, 64), (1, 0))])
def test_contiguous_of_a_transposed_view_is_the_values(hip, shape, perm):
    """CONTIGUOUS of views whose last two axes are transposed (the tiled
    transpose path; the weight gradients of x @ w.T arrive this way) and of
    other permutations: the values, byte for byte."""
    from vkml_amd.device import contiguous

    x = np.random.default_rng(SEED + 96).standard_normal(shape).astype(np.float32)
    base = dev(x)
    d = DeviceArray([base.shape[p] for p in perm], np.float32, [base.strides[p] for p in perm],
                    base.buffer, base.offset)
    got = contiguous(d).numpy()
    assert got.tobytes() == np.ascontiguousarray(np.transpose(x, perm)).tobytes()


def test_supports_predicate_and_unsupported_compute(hip):
    """vkhip_supports reports exactly the implemented (op, dtype) set: a float
    relu node is supported, an op this backend lacks and a relu over int64
    are not, and vkhip_compute refuses such a node with ERR_UNSUPPORTED and a
    message instead of running anything (the reference executor's rule: no
    fallback, executor.cpp:107-124)."""
    x = dev(np.arange(8, dtype=np.float32) - 4)
    out = DeviceArray((8,), np.float32)

    def node(op, dtype):
        nd = _lib.NodeDesc()
        nd.op, nd.n_src = op, 1
        for t, arr in ((nd.out, out), (nd.src[0], x)):
            t.data, t.dtype, t.ndim = arr.ptr, dtype, 1
            t.ne[0], t.nb[0] = 8, 1
        return nd

    relu = node(_lib.OP["RELU"], _lib.F32)
    assert hip.supports(relu)
    hip.compute(relu)
    assert out.numpy().tobytes() == np.maximum(np.arange(8, dtype=np.float32) - 4, 0).tobytes()
    for bad in (node(1, _lib.F32), node(_lib.OP["RELU"], _lib.I64)):
        assert not hip.supports(bad)
        with pytest.raises(_lib.NotImplementedOnDevice):
            hip.compute(bad)
