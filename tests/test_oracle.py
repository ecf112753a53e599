"""Pins the CPU oracle (oracle/vkml_oracle.c) before anything is checked against it.

Each oracle function is tied to something independent of its own code:
the reference's known answers (tests/cpp/test_ops.cpp:234-293), its fixtures
(test_vulkan_kernels.py: STABILITY_INPUTS :808-817, the col2im bit-reproducibility
cols :1347-1352, the pool tie :1440), the carry-stack theorem the reference proves
on the host (test_invariants.py:90-191), torch / float64 closed forms, and brute
force on tiny inputs. Each check is chosen so that a plausible slip -- a split at a
block boundary instead of the midpoint, a dropped term, a transposed operand, an
off-by-one window -- fails it.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from conftest import SEED, gemm_atol, golden, pairwise_gamma


def seq32(v: np.ndarray) -> np.float32:
    """Sequential float32 sum from 0 (numpy's cumsum accumulates in order)."""
    v = np.asarray(v, np.float32)
    return np.float32(0.0) if v.size == 0 else np.cumsum(v, dtype=np.float32)[-1]


def carry_fold(vals) -> np.float32:
    """The reference's binary-counter push/drain (test_invariants.py:90-107)."""
    stack, count = {}, 0
    for v in vals:
        block, c, level = np.float32(v), count, 0
        while c & 1:
            block = np.float32(block + stack[level])
            c >>= 1
            level += 1
        stack[level] = block
        count += 1
    total, level = np.float32(0.0), 0
    while (count >> level) != 0:
        if (count >> level) & 1:
            total = np.float32(total + stack[level])
        level += 1
    return total


# ---------------------------------------------------------------------------
# pairwise summation (reference reduce.h:55-72)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n", [0, 1, 2, 31, 32])
def test_pairwise_base_case_is_sequential(n):
    v = np.random.default_rng(n).standard_normal(n).astype(np.float32) * 1e3
    assert O.pairwise_sum(v).tobytes() == seq32(v).tobytes()


@pytest.mark.parametrize("n", [48, 50, 63])
def test_pairwise_splits_at_the_midpoint(n):
    """n in (32, 64]: one split at n//2, not at the 32-element block boundary."""
    rng = np.random.default_rng(n)
    hits = 0
    for _ in range(40):
        v = (rng.standard_normal(n) * 1e4).astype(np.float32)
        want = np.float32(seq32(v[: n // 2]) + seq32(v[n // 2:]))
        assert O.pairwise_sum(v).tobytes() == want.tobytes()
        block_split = np.float32(seq32(v[:32]) + seq32(v[32:]))
        hits += block_split.tobytes() != want.tobytes()
    assert hits > 10, "test cannot tell a midpoint split from a block split"


@pytest.mark.parametrize("q", [1, 2, 5, 7])
def test_pairwise_equals_carry_stack_over_32_blocks(q):
    """For n = 32 * 2^q the recursion is a balanced tree over 32-element
    sequential blocks, i.e. the carry stack over block sums (the N1 theorem,
    reference test_invariants.py:117-135)."""
    n = 32 << q
    v = (np.random.default_rng(q).standard_normal(n) * 1e3).astype(np.float32)
    blocks = [seq32(v[i:i + 32]) for i in range(0, n, 32)]
    assert O.pairwise_sum(v).tobytes() == carry_fold(blocks).tobytes()


def test_pairwise_is_not_a_flat_sum():
    rng = np.random.default_rng(11)
    differ = 0
    for _ in range(40):
        v = (rng.standard_normal(4096) * 1e3).astype(np.float32)
        differ += O.pairwise_sum(v).tobytes() != seq32(v).tobytes()
    assert differ > 10


@pytest.mark.parametrize("n", [100, 784, 1000, 4096, 32768, 65537])
def test_pairwise_within_backward_bound(n):
    v = np.random.default_rng(n).uniform(-2, 2, n).astype(np.float32)
    exact = float(np.sum(v.astype(np.float64)))
    bound = pairwise_gamma(n) * float(np.sum(np.abs(v.astype(np.float64))))
    assert abs(float(O.pairwise_sum(v)) - exact) <= bound


# ---------------------------------------------------------------------------
# matmul (reference kernels_matmul.cpp:34-87)
# ---------------------------------------------------------------------------

def test_matmul_known_answer():
    """reference test_ops.cpp:266-272."""
    f = golden("matmul_2d")
    np.testing.assert_array_equal(O.matmul(f["a"], f["b"]), f["expected"])


def test_matmul_transposed_operand_known_answer():
    """reference test_ops.cpp:274-280: b given as a transposed (strided) view."""
    f = golden("matmul_transposed_operand")
    np.testing.assert_array_equal(O.matmul(f["a"], f["b_transposed"].T), f["expected"])


def test_matmul_batch_broadcast_known_answer():
    """reference test_ops.cpp:305-311: a [1,2,2] identity broadcast over the batch."""
    f = golden("matmul_batch_broadcast")
    b = np.broadcast_to(f["b"], f["a"].shape)
    np.testing.assert_array_equal(O.matmul(f["a"], b), f["expected"])


def test_matmul_vector_known_answers():
    """reference test_ops.cpp:282-293 (rank-1 promoted to a row / a column)."""
    f = golden("matmul_vector_rules")
    m, v, u = f["m"], f["v"].reshape(3, 1), f["u"].reshape(1, 2)
    np.testing.assert_array_equal(O.matmul(m, v).ravel(), f["m_v"])
    np.testing.assert_array_equal(O.matmul(u, m).ravel(), f["u_m"])
    np.testing.assert_array_equal(O.matmul(v.T, v).ravel(), [f["v_v"]])


def test_matmul_products_are_rounded_then_pairwise_summed():
    """One output = pairwise sum of the individually rounded f32 products."""
    rng = np.random.default_rng(5)
    a = rng.standard_normal((3, 1000)).astype(np.float32)
    b = rng.standard_normal((1000, 4)).astype(np.float32)
    got = O.matmul(a, b)
    for i in range(3):
        for j in range(4):
            prods = (a[i] * b[:, j]).astype(np.float32)
            assert got[i, j].tobytes() == O.pairwise_sum(prods).tobytes()


@pytest.mark.parametrize("layout", ["nn", "nt", "tn", "tt"])
def test_matmul_layouts_and_batch_broadcast_vs_float64(layout):
    rng = np.random.default_rng(SEED + 1)
    m, k, n = 37, 130, 29
    a = rng.uniform(-2, 2, (m, k)).astype(np.float32)
    b = rng.uniform(-2, 2, (k, n)).astype(np.float32)
    av = np.ascontiguousarray(a.T).T if layout[0] == "t" else a
    bv = np.ascontiguousarray(b.T).T if layout[1] == "t" else b
    # batch-broadcast A (stride 0) against a real batch of B, as conv2d does
    bb = np.stack([bv, bv * 2, -bv])
    got = O.matmul(av[None], bb)
    want = np.einsum("mk,bkn->bmn", a.astype(np.float64), bb.astype(np.float64))
    assert np.max(np.abs(got - want)) <= gemm_atol(a, b * 2)


def test_matmul_threads_do_not_change_bits():
    rng = np.random.default_rng(3)
    a = rng.standard_normal((64, 300)).astype(np.float32)
    b = rng.standard_normal((300, 48)).astype(np.float32)
    assert O.matmul(a, b, threads=1).tobytes() == O.matmul(a, b, threads=8).tobytes()


# ---------------------------------------------------------------------------
# reductions (reference kernels_reduce.cpp:44-192)
# ---------------------------------------------------------------------------

def test_argmax_argmin_first_extremum_known_answer():
    """reference test_ops.cpp:225-231."""
    f = golden("argmax_first_extremum")
    np.testing.assert_array_equal(O.argmax(f["a"], 1), f["argmax"])
    np.testing.assert_array_equal(O.argmin(f["a"], 1), f["argmin"])


def test_argmax_skips_nan_and_max_returns_it():
    """The CPU loops: argmax's strict `>` never selects NaN; max returns the
    first NaN it meets (kernels_reduce.cpp:124-176)."""
    x = np.array([[1.0, np.nan, 3.0, 2.0], [np.nan, np.nan, -np.inf, -np.inf]], np.float32)
    np.testing.assert_array_equal(O.argmax(x, 1), [2, 0])
    mx = O.amax(x, 1)
    assert np.isnan(mx).all()


def test_sum_is_pairwise_over_the_reduced_axes():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((6, 5, 40)) * 100).astype(np.float32)
    s = O.sum(x, [0, 2])  # reduced elements in row-major order of the reduced axes
    for j in range(5):
        assert s[j].tobytes() == O.pairwise_sum(x[:, j, :].ravel()).tobytes()
    np.testing.assert_array_equal(O.mean(x, [0, 2]), s / np.float32(240))


def test_max_min_are_exact_selections():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((33, 77)).astype(np.float32)
    np.testing.assert_array_equal(O.amax(x, 1), x.max(1))
    np.testing.assert_array_equal(O.amin(x, 0), x.min(0))
    np.testing.assert_array_equal(O.argmax(x, 0), x.argmax(0))


# ---------------------------------------------------------------------------
# softmax (reference kernels_reduce.cpp:205-259)
# ---------------------------------------------------------------------------

STABILITY_INPUTS = golden("softmax_stability_inputs")["inputs"]  # test_vulkan_kernels.py:808-817


@pytest.mark.parametrize("name", list(STABILITY_INPUTS))
@pytest.mark.parametrize("log", [False, True])
def test_softmax_stability_vs_torch_float64(name, log):
    x = STABILITY_INPUTS[name]
    got = O.softmax(x, -1, log)
    assert np.isfinite(got).all()
    t = torch.from_numpy(x.astype(np.float64))
    want = (torch.log_softmax if log else torch.softmax)(t, -1).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_softmax_known_answers():
    """reference test_ops.cpp:233-264."""
    f = golden("softmax_shift_invariance")
    s = O.softmax(f["rows"], 1)
    np.testing.assert_allclose(s.sum(1), 1.0, rtol=1e-6)
    big, small = O.softmax(f["big"], 0), O.softmax(f["small"], 0)
    np.testing.assert_allclose(big, small, atol=f["tolerance"])
    g = golden("log_softmax_finite")
    ls = O.log_softmax(g["x"], 0)
    assert np.isfinite(ls).all() and abs(ls[2] - g["third"]) <= abs(g["third"]) * g["epsilon"]


def test_softmax_denominator_is_pairwise_and_strided_axes_work():
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((4, 300)) * 2).astype(np.float32)
    got = O.softmax(x, -1)
    for r in range(4):
        peak = x[r].max()
        e = np.exp(x[r] - peak).astype(np.float32)
        denom = O.pairwise_sum(e)
        np.testing.assert_allclose(got[r], e / denom, rtol=3e-7)
    # softmax over axis 0 of a transposed view == softmax over axis -1 transposed
    np.testing.assert_array_equal(O.softmax(np.ascontiguousarray(x.T), 0).T, O.softmax(x, -1))


# ---------------------------------------------------------------------------
# im2col / col2im / max-pool (reference kernels_movement.cpp:438-680)
# ---------------------------------------------------------------------------

WINDOWS = [  # reference test_vulkan_kernels.py:1303-1310
    ((1, 1, 4, 4), (2, 2), (1, 1), (0, 0), (1, 1)),
    ((2, 3, 5, 5), (3, 3), (1, 1), (1, 1), (1, 1)),
    ((1, 2, 6, 6), (2, 2), (2, 2), (0, 0), (1, 1)),
    ((2, 1, 7, 5), (3, 2), (2, 1), (1, 0), (1, 1)),
    ((1, 2, 5, 5), (2, 2), (1, 1), (0, 0), (2, 2)),
    ((1, 1, 17, 17), (3, 3), (1, 1), (1, 1), (1, 1)),
]


@pytest.mark.parametrize("shape,kernel,stride,pad,dil", WINDOWS)
def test_im2col_equals_torch_unfold(shape, kernel, stride, pad, dil):
    x = np.random.default_rng(SEED).uniform(-3, 3, shape).astype(np.float32)
    got = O.im2col(x, kernel, stride, pad, dil)
    want = torch.nn.functional.unfold(torch.from_numpy(x), kernel, dil, pad, stride).numpy()
    assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("shape,kernel,stride,pad,dil", WINDOWS)
def test_col2im_is_the_adjoint_of_im2col(shape, kernel, stride, pad, dil):
    """<im2col(x), y> == <x, col2im(y)> exactly, with small integers so every
    f32 sum is exact."""
    rng = np.random.default_rng(SEED + 2)
    x = rng.integers(-4, 5, shape).astype(np.float32)
    cols_shape = O.im2col(x, kernel, stride, pad, dil).shape
    y = rng.integers(-4, 5, cols_shape).astype(np.float32)
    lhs = float(np.sum(O.im2col(x, kernel, stride, pad, dil).astype(np.float64) * y))
    rhs = float(np.sum(x.astype(np.float64) * O.col2im(y, shape[2:], kernel, stride, pad, dil)))
    assert lhs == rhs
    want = torch.nn.functional.fold(torch.from_numpy(y), shape[2:], kernel, dil, pad, stride)
    np.testing.assert_array_equal(O.col2im(y, shape[2:], kernel, stride, pad, dil), want.numpy())


def test_col2im_fold_order_fixture():
    """reference test_vulkan_kernels.py:1342-1356: wide magnitudes expose the
    ascending (ki, kj) fold; interior positions get all nine contributions."""
    f = golden("col2im_fold_order")
    vals = f["row_values"]
    cols = np.zeros(tuple(int(e) for e in f["cols_shape"]), np.float32)
    cols[0, :, :] = vals[:, None]
    got = O.col2im(cols, tuple(int(e) for e in f["image_hw"]), (3, 3), (1, 1), (1, 1))
    # Position (h, w) receives row ki*3+kj when the window at (h+1-ki, w+1-kj) exists.
    for h in range(4):
        for w in range(4):
            acc = np.float32(0.0)
            for ki in range(3):
                for kj in range(3):
                    if 0 <= h + 1 - ki < 4 and 0 <= w + 1 - kj < 4:
                        acc = np.float32(acc + vals[ki * 3 + kj])
            assert got[0, 0, h, w].tobytes() == acc.tobytes()
    # An order-insensitive float64 sum disagrees at the interior, which is what
    # makes this fixture a test of order.
    assert got[0, 0, 1, 1] != np.float32(np.sum(vals.astype(np.float64)))


POOLS = [  # reference test_vulkan_kernels.py:1386-1392
    ((1, 1, 4, 4), (2, 2), (2, 2), (0, 0)),
    ((2, 3, 6, 6), (2, 2), (2, 2), (0, 0)),
    ((1, 2, 5, 5), (3, 3), (1, 1), (1, 1)),
    ((2, 1, 7, 5), (3, 2), (2, 1), (1, 0)),
    ((1, 1, 17, 17), (3, 3), (2, 2), (1, 1)),
]


@pytest.mark.parametrize("shape,kernel,stride,pad", POOLS)
def test_max_pool2d_and_backward_vs_torch(shape, kernel, stride, pad):
    x = np.random.default_rng(SEED).uniform(-3, 3, shape).astype(np.float32)
    t = torch.from_numpy(x).requires_grad_(True)
    y = torch.nn.functional.max_pool2d(t, kernel, stride, pad)
    got = O.max_pool2d(x, kernel, stride, pad)
    assert got.tobytes() == y.detach().numpy().tobytes()
    g = np.random.default_rng(SEED + 1).uniform(-1, 1, got.shape).astype(np.float32)
    y.backward(torch.from_numpy(g))
    np.testing.assert_allclose(O.max_pool2d_backward(g, x, kernel, stride, pad), t.grad.numpy(),
                               rtol=1e-6, atol=1e-7)


def test_max_pool2d_tie_goes_to_the_first_maximum():
    """reference test_vulkan_kernels.py:1440-1452."""
    f = golden("max_pool2d_tie")
    g = O.max_pool2d_backward(np.ones((1, 1, 1, 1), np.float32), f["x"], (2, 2))
    np.testing.assert_array_equal(g, f["grad_of_sum"])


def test_max_pool2d_pads_with_minus_infinity():
    """reference test_vulkan_kernels.py:1425-1437."""
    x = -np.abs(np.random.default_rng(SEED).uniform(-3, 3, (1, 2, 5, 5))).astype(np.float32) - 1
    got = O.max_pool2d(x, (3, 3), (1, 1), (1, 1))
    assert not np.any(got == 0.0)


# ---------------------------------------------------------------------------
# split-K carry-stack fold (reference gemm_split_k_reduce.comp:48-85)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("tiles", [1, 2, 3, 5, 8, 12, 17, 33, 129])
def test_split_fold_power_of_two_chunks_equal_unsplit(tiles):
    """The alignment theorem (reference test_invariants.py:117-135), on the
    oracle's own fold: folding power-of-two chunks, then the chunk results,
    equals one fold over everything."""
    vals = (np.random.default_rng(tiles).standard_normal(tiles) * 1e3).astype(np.float32)
    whole = O.split_k_fold(vals, tiles)
    assert whole.tobytes() == carry_fold(vals).tobytes()
    chunk = 1
    while chunk <= tiles:
        parts = [O.split_k_fold(vals[i:i + chunk], len(vals[i:i + chunk]))[0]
                 for i in range(0, tiles, chunk)]
        assert O.split_k_fold(np.array(parts, np.float32), len(parts)).tobytes() == whole.tobytes()
        chunk *= 2


def test_split_fold_is_a_balanced_tree_for_four():
    v = (np.random.default_rng(4).standard_normal(4) * 1e3).astype(np.float32)
    want = np.float32(np.float32(v[0] + v[1]) + np.float32(v[2] + v[3]))
    assert O.split_k_fold(v, 4)[0].tobytes() == want.tobytes()


def test_split_fold_non_power_of_two_chunks_break_identity():
    """Negative control (reference test_invariants.py:138-163)."""
    rng = np.random.default_rng(12)
    mismatches = 0
    for _ in range(60):
        vals = (rng.standard_normal(97) * 1e3).astype(np.float32)
        parts = [O.split_k_fold(vals[i:i + 5], len(vals[i:i + 5]))[0] for i in range(0, 97, 5)]
        folded = O.split_k_fold(np.array(parts, np.float32), len(parts))
        mismatches += folded.tobytes() != O.split_k_fold(vals, 97).tobytes()
    assert mismatches > 15


# ---- the oracle's exp and log (vkml_oracle.c or_expf / or_logf) ----

def _cr_float(fn, xs):
    """Correctly rounded float32 of fn over float32 inputs, from mpmath at 100
    bits (the double rounding through float64 is below 2^-47 relative)."""
    import mpmath

    mpmath.mp.prec = 100
    out = np.empty(len(xs), np.float32)
    with np.errstate(over="ignore"):
        for i, x in enumerate(xs):
            out[i] = np.float32(float(fn(mpmath.mpf(float(x)))))
    return out


def _exp_inputs():
    rng = np.random.default_rng(SEED + 101)
    special = np.array([0.0, -0.0, 1.0, -1.0, 88.72283, 88.72284, 89.0, -87.33654, -87.3366,
                        -100.0, -103.97, -103.98, -104.0, 1e-8, -1e-8, 0.5, -0.5, 0.34657359,
                        -0.34657359, 0.34657362, 20.0, -20.0], np.float32)
    return np.concatenate([special, rng.uniform(-104, 89, 3000).astype(np.float32),
                           rng.uniform(-20, 0, 3000).astype(np.float32),
                           rng.uniform(-1e-3, 1e-3, 500).astype(np.float32)])


def _log_inputs():
    rng = np.random.default_rng(SEED + 102)
    special = np.array([1.0, 2.0, 0.5, np.float32(np.sqrt(0.5)), np.float32(np.sqrt(2.0)),
                        1.0000001, 0.99999994, 1e-45, 1e-40, 1.1754944e-38, 3.4028235e38, 10.0,
                        100.0, 4.6, 12800.0], np.float32)
    return np.concatenate([special, np.exp(rng.uniform(-100, 88, 3000)).astype(np.float32),
                           rng.uniform(0.5, 2.0, 3000).astype(np.float32),
                           (1 + rng.uniform(-1e-4, 1e-4, 500)).astype(np.float32)])


def test_oracle_exp_is_correctly_rounded():
    """The oracle fixes the reference's unpinned std::exp (platform libm,
    kernels_reduce.cpp:227-243) to a Cody-Waite + degree-13 Taylor method in
    double: against mpmath it must be the correctly rounded float on every
    sampled input, subnormal results and overflow to +inf included. A dropped
    polynomial term, a wrong ln2 split or a bad reduction breaks this."""
    import mpmath

    x = _exp_inputs()
    got = O.expf(x)
    want = _cr_float(mpmath.exp, x)
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{bad.size} mismatches, e.g. x={x[bad[:3]]} got {got[bad[:3]]} want {want[bad[:3]]}"
    assert np.isposinf(O.expf(np.array([89.5, np.inf], np.float32))).all()
    assert (O.expf(np.array([-104.5, -np.inf], np.float32)) == 0).all()
    assert np.isnan(O.expf(np.array([np.nan], np.float32))).all()


def test_oracle_log_is_correctly_rounded():
    import mpmath

    x = _log_inputs()
    got = O.logf(x)
    want = _cr_float(mpmath.log, x)
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{bad.size} mismatches, e.g. x={x[bad[:3]]} got {got[bad[:3]]} want {want[bad[:3]]}"
    sp = O.logf(np.array([0.0, -0.0, -1.0, np.inf, np.nan, 1.0], np.float32))
    assert np.isneginf(sp[0]) and np.isneginf(sp[1]) and np.isnan(sp[2]) and np.isposinf(sp[3])
    assert np.isnan(sp[4]) and sp[5] == 0.0 and not np.signbit(sp[5])


def test_device_source_exp_log_match_the_oracle():
    """libvkhip's exact-numerics exp/log (the source the device kernels use,
    evaluated on the host through vkhip_exact_math) against the oracle's, bit
    for bit, on a dense sweep of the softmax and log domains."""
    from vkml_amd import _lib

    lib = _lib.load()
    rng = np.random.default_rng(SEED + 103)
    for log_mode, x in ((0, np.concatenate([np.linspace(-104, 89, 400_001, dtype=np.float32),
                                            rng.uniform(-30, 0, 400_000).astype(np.float32)])),
                        (1, np.concatenate([np.exp(np.linspace(-103, 88, 400_001)).astype(np.float32),
                                            rng.uniform(1e-3, 1e3, 400_000).astype(np.float32)]))):
        y = np.empty_like(x)
        assert lib.vkhip_exact_math(x.ctypes.data, y.ctypes.data, x.size, log_mode) == 0
        want = O.logf(x) if log_mode else O.expf(x)
        assert y.tobytes() == want.tobytes()
