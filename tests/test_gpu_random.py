"""Seeded random sweeps of the device paths against the oracle and against
each other: geometries and layouts drawn from fixed seeds, so every run checks
the same cases, but many more of them than the hand-picked tests, crossing the
kernels' structure thresholds (tile sizes, leaf counts, vector/generic paths).

Bars as elsewhere: bit-exact for reductions, selections, broadcast arithmetic
and the implicit-vs-explicit convolution identities; softmax within
1e-5*sqrt(n) of the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from conftest import SEED, gemm_tolerance, normwise_rel_err, small_window
from vkml_amd import ops
from vkml_amd import tensor as T
from vkml_amd.device import DeviceArray

pytestmark = pytest.mark.gpu


def dev(x: np.ndarray) -> DeviceArray:
    return DeviceArray.from_numpy(x)


def same_bits(got: np.ndarray, want: np.ndarray) -> None:
    """Equal NaN positions and equal bits everywhere else (a NaN's payload is
    not part of the contract)."""
    assert got.shape == want.shape
    nan = np.isnan(want)
    np.testing.assert_array_equal(np.isnan(got), nan)
    assert got[~nan].tobytes() == want[~nan].tobytes()


def conv_cases(count: int):
    rng = np.random.default_rng(SEED + 500)
    out = []
    while len(out) < count:
        n, c, cout = (int(v) for v in rng.integers(1, [4, 9, 10]))
        h, w = (int(v) for v in rng.integers(1, 21, 2))
        kernel = tuple(int(v) for v in rng.integers(1, 6, 2))
        stride = tuple(int(v) for v in rng.integers(1, 4, 2))
        pad = tuple(int(v) for v in rng.integers(0, 3, 2))
        dil = tuple(int(v) for v in rng.integers(1, 3, 2))
        oh = ops.window_count(h, kernel[0], stride[0], pad[0], dil[0])
        ow = ops.window_count(w, kernel[1], stride[1], pad[1], dil[1])
        if oh > 0 and ow > 0:
            out.append(((n, c, h, w), cout, kernel, stride, pad, dil))
    return out


@pytest.mark.parametrize("shape,cout,kernel,stride,pad,dil", conv_cases(24))
def test_random_conv_forward_and_weight_grad_match_the_lowering(hip, shape, cout, kernel, stride,
                                                                pad, dil):
    """Implicit-im2col forward and weight gradient against im2col + GEMM on
    the device (bit for bit; small-window weight gradients within the GEMM
    tolerance) and the oracle (GEMM tolerance), and the device im2col against
    the oracle's (bit for bit)."""
    rng = np.random.default_rng(SEED + sum(shape) + cout)
    x = rng.uniform(-1, 1, shape).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (cout, shape[1]) + kernel).astype(np.float32)
    cols = ops.im2col(dev(x), kernel, stride, pad, dil)
    ref_cols = O.im2col(x, kernel, stride, pad, dil)
    assert cols.numpy().tobytes() == ref_cols.tobytes()
    n, ck, L = cols.shape
    got = ops.conv2d(dev(x), dev(w), stride, pad, dil).numpy()
    wf = dev(w.reshape(1, 1, cout, ck)).broadcast_to((1, n, cout, ck))
    want = ops.matmul(wf, cols.reshape(1, n, ck, L)).numpy().reshape(got.shape)
    assert got.tobytes() == want.tobytes()
    ref = O.matmul(np.broadcast_to(w.reshape(1, cout, ck), (n, cout, ck)), ref_cols)
    assert normwise_rel_err(got, ref.reshape(got.shape)) <= gemm_tolerance(ck)
    g = rng.standard_normal(got.shape).astype(np.float32)
    dw = ops.conv2d_weight_grad(dev(x), dev(g), kernel, stride, pad, dil).numpy()
    want_dw = ops.matmul(dev(g.reshape(1, n, cout, L)),
                         cols.reshape(1, n, ck, L).transpose(-2, -1)).numpy().reshape(dw.shape)
    if small_window(shape, cout, kernel, L):  # its own fixed summation order
        assert normwise_rel_err(dw, want_dw) <= gemm_tolerance(L)
    else:
        assert dw.tobytes() == want_dw.tobytes()


def reduce_cases(count: int):
    rng = np.random.default_rng(SEED + 600)
    out = []
    for _ in range(count):
        rank = int(rng.integers(1, 5))
        shape = tuple(int(v) for v in rng.choice([1, 2, 3, 5, 7, 16, 33, 64, 100, 129, 300],
                                                 rank))
        k = int(rng.integers(1, rank + 1))
        axes = sorted(int(a) for a in rng.choice(rank, k, replace=False))
        out.append((shape, axes))
    return out


@pytest.mark.parametrize("shape,axes", reduce_cases(40))
def test_random_reductions_are_bit_exact(hip, shape, axes):
    """sum, mean, max and min over random axis subsets of random shapes, and
    argmax/argmin over each single axis, equal the oracle's bits (whichever
    structure the planner picks), with ties and a NaN planted."""
    rng = np.random.default_rng(SEED + len(shape) * 31 + sum(shape))
    x = (rng.standard_normal(shape) * 4).astype(np.float32)
    flat = x.reshape(-1)
    if flat.size > 8:
        flat[3] = flat[5]  # a tie
        flat[flat.size // 2] = np.nan if flat.size > 64 else flat[flat.size // 2]
    d = dev(x)
    same_bits(ops.sum(d, axes).numpy(), O.sum(x, axes))
    same_bits(ops.mean(d, axes).numpy(), O.mean(x, axes))
    same_bits(ops.amax(d, axes).numpy(), O.amax(x, axes))
    same_bits(ops.amin(d, axes).numpy(), O.amin(x, axes))
    for a in range(len(shape)):
        assert ops.argmax(d, a).numpy().tobytes() == O.argmax(x, a).tobytes()
        assert ops.argmin(d, a).numpy().tobytes() == O.argmin(x, a).tobytes()


def broadcast_cases(count: int):
    rng = np.random.default_rng(SEED + 700)
    out = []
    for _ in range(count):
        rank = int(rng.integers(1, 5))
        xs = tuple(int(v) for v in rng.choice([1, 2, 3, 4, 8, 12, 17, 32], rank))
        ys = tuple(e if rng.random() < 0.5 else 1 for e in xs)
        drop = int(rng.integers(0, rank))  # leading axes the second operand omits
        out.append((xs, ys[drop:]))
    return out


@pytest.mark.parametrize("xs,ys", broadcast_cases(30))
def test_random_broadcast_arithmetic_is_bit_exact(hip, xs, ys):
    """add/sub/mul/div/maximum with a broadcast operand on either side, through
    the tensor layer, equal the oracle's bits."""
    from oracle import OracleBackend

    dev_be, cpu = T.default_backend(), OracleBackend()
    rng = np.random.default_rng(SEED + sum(xs) * 7 + len(ys))
    x = rng.standard_normal(xs).astype(np.float32)
    y = (rng.standard_normal(ys) + 0.5).astype(np.float32)
    for op in (T.add, T.sub, T.mul, T.div, T.maximum):
        for a, b in ((x, y), (y, x)):
            got = op(T.tensor(a, backend=dev_be), T.tensor(b, backend=dev_be)).numpy()
            want = op(T.tensor(a, backend=cpu), T.tensor(b, backend=cpu)).numpy()
            same_bits(got, want)


def softmax_cases(count: int):
    rng = np.random.default_rng(SEED + 800)
    out = []
    for _ in range(count):
        rows = int(rng.integers(1, 600))
        n = int(rng.choice([1, 3, 31, 64, 255, 257, 1000, 2048, 2049, 4096, 5000, 8191, 16384,
                            20000, 32768, 33000, 70000]))
        out.append((rows if n <= 8192 else min(rows, 40), n, bool(rng.integers(2))))
    return out


@pytest.mark.parametrize("rows,n,log", softmax_cases(30))
def test_random_softmax_rows(hip, rows, n, log):
    """Softmax / log-softmax over rows of every structure class (a wave per
    row, a workgroup per row, chunks over two launches), against the oracle."""
    x = (np.random.default_rng(SEED + rows * 13 + n).standard_normal((rows, n)) * 2).astype(
        np.float32)
    got = ops.softmax(dev(x), -1, log).numpy()
    want = O.softmax(x, -1, log)
    if log:
        assert normwise_rel_err(got, want) <= gemm_tolerance(n)
    else:
        big = np.abs(want) > 1e-30
        rel = np.abs(got[big] - want[big]) / np.abs(want[big])
        assert rel.size == 0 or rel.max() <= gemm_tolerance(n)
        assert np.all(np.abs(got[~big]) <= 1e-30)
