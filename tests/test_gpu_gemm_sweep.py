"""BASELINE config 2 at every size and layout the benchmark times, and GEMM
operand layouts the fast paths must not take.

Config 2: M = N = K in {512, 1024, 2048, 4096, 8192} and 8192x1024x4096, in the
NN, NT and TN layouts that forward and backward emit, A and B ~ N(0, 1) fp32.
The full product runs on the device; 64 of its rows (the first and last eight,
so both edge tile rows are covered, and 48 drawn at random; every column) are
checked against the CPU oracle (the restated reference matmul) and against a
float64 product: normwise relative error <= 1e-5*sqrt(K) (north star) and
elementwise within the backward-error bound gamma(K)*sum|a||b| (the
reference's policy, conftest.py:145-165).
"""
from __future__ import annotations

from ctypes import byref, c_void_p

import numpy as np
import pytest

import oracle as O
from conftest import SEED, gemm_atol, gemm_tolerance, normwise_rel_err
from vkml_amd import _lib, ops
from vkml_amd.device import DeviceArray

pytestmark = pytest.mark.gpu

SHAPES = [(512, 512, 512), (1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096),
          (8192, 8192, 8192), (8192, 1024, 4096)]


def _rows(m: int, rng) -> np.ndarray:
    edge = np.r_[np.arange(8), np.arange(m - 8, m)]
    rest = rng.choice(np.arange(8, m - 8), 48, replace=False)
    return np.sort(np.r_[edge, rest])


@pytest.mark.timeout(300)
@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
@pytest.mark.parametrize("m,n,k", SHAPES, ids=lambda v: str(v))
def test_config2_gemm_sizes_and_layouts(hip, m, n, k, layout):
    print(f"config2 gemm {m}x{n}x{k} {layout}", flush=True)
    rng = np.random.default_rng(SEED + m + 3 * n + 7 * k + (layout == "nt") + 2 * (layout == "tn"))
    a = rng.standard_normal((m, k), dtype=np.float32)
    b = rng.standard_normal((k, n), dtype=np.float32)
    # NT stores B as its transpose, TN stores A as its transpose: the device
    # sees a column-strided view, exactly as the backward pass hands it over.
    da = DeviceArray.from_numpy(np.ascontiguousarray(a.T)).T if layout[0] == "t" else \
        DeviceArray.from_numpy(a)
    db = DeviceArray.from_numpy(np.ascontiguousarray(b.T)).T if layout[1] == "t" else \
        DeviceArray.from_numpy(b)
    got = ops.matmul(da, db).numpy()
    del da, db
    rows = _rows(m, rng)
    ar = a[rows]
    exact = ar.astype(np.float64) @ b.astype(np.float64)
    err = normwise_rel_err(got[rows], exact)
    assert err <= gemm_tolerance(k), f"vs float64: {err:.3g}"
    assert np.max(np.abs(got[rows] - exact)) <= gemm_atol(ar, b)
    want = O.matmul(ar, b)
    err = normwise_rel_err(got[rows], want)
    assert err <= gemm_tolerance(k), f"vs the oracle: {err:.3g}"


# ---------------------------------------------------------------------------
# Negative strides: reversed views must stay off the buffer-load paths
# (unsigned 32-bit offsets), and still give the contiguous product's bits.
# ---------------------------------------------------------------------------

def _reversed_rows(x: np.ndarray) -> DeviceArray:
    """A device view of x whose rows are stored last-to-first: the view reads
    x, through a negative row stride."""
    stored = DeviceArray.from_numpy(np.ascontiguousarray(x[::-1]))
    r, c = x.shape
    return DeviceArray((r, c), np.float32, (-c, 1), stored.buffer, (r - 1) * c)


def _reversed_cols(x: np.ndarray) -> DeviceArray:
    stored = DeviceArray.from_numpy(np.ascontiguousarray(x[:, ::-1]))
    r, c = x.shape
    return DeviceArray((r, c), np.float32, (c, -1), stored.buffer, c - 1)


@pytest.mark.parametrize("m,n,k", [(256, 256, 512), (64, 96, 128), (1024, 1024, 1024),
                                   (256, 256, 65536)])
@pytest.mark.parametrize("which", ["a_rows", "b_rows", "b_cols", "a_cols"])
def test_gemm_negative_strides(hip, m, n, k, which):
    rng = np.random.default_rng(SEED + m + n + k + len(which))
    a = rng.standard_normal((m, k), dtype=np.float32)
    b = rng.standard_normal((k, n), dtype=np.float32)
    da = {"a_rows": _reversed_rows, "a_cols": _reversed_cols}.get(which, DeviceArray.from_numpy)(a)
    db = {"b_rows": _reversed_rows, "b_cols": _reversed_cols}.get(which, DeviceArray.from_numpy)(b)
    got = ops.matmul(da, db).numpy()
    plain = ops.matmul(DeviceArray.from_numpy(a), DeviceArray.from_numpy(b)).numpy()
    assert got.tobytes() == plain.tobytes()
    rows = np.arange(0, m, max(1, m // 32))
    exact = a[rows].astype(np.float64) @ b.astype(np.float64)
    assert normwise_rel_err(got[rows], exact) <= gemm_tolerance(k)


# ---------------------------------------------------------------------------
# compute() refuses nodes whose extents disagree with params/operands
# ---------------------------------------------------------------------------

def test_compute_refuses_malformed_nodes_before_launching(hip):
    """Every malformed node of the host-side extent table returns
    VKHIP_ERR_INVALID from vkhip_compute. Each tensor pointer is a separate
    64 KB buffer, larger than anything these tiny nodes could touch, so an
    accepted node would still stay in bounds (the test would then fail, not
    fault)."""
    from test_host import _extent_cases

    lib = _lib.load()
    bufs = []
    for name, good, bad in _extent_cases():
        for nd in [good] + bad:
            for t in [nd.out] + [nd.src[i] for i in range(nd.n_src)]:
                buf = DeviceArray((16384,), np.float32)
                bufs.append(buf)
                t.data = buf.ptr
        for i, nd in enumerate(bad):
            code = lib.vkhip_compute(byref(nd), 1)
            assert code == _lib.ERR_INVALID, (name, i, code, lib.vkhip_last_error())
        assert lib.vkhip_compute(byref(good), 1) == _lib.OK, (name, lib.vkhip_last_error())
    hip.synchronize()


# ---------------------------------------------------------------------------
# The exact comparison arm (VKHIP_GEMM_EXACT): the oracle's bits
# ---------------------------------------------------------------------------

EXACT_CASES = [  # (A shape, B shape): 2-D, ragged, K not a multiple of 32, batch broadcast
    ((5, 7), (7, 3)), ((1, 31), (31, 1)), ((64, 784), (784, 128)), ((64, 128), (128, 10)),
    ((33, 1000), (1000, 65)), ((128, 4097), (4097, 40)), ((3, 48), (48, 5)), ((70, 33), (33, 70)),
    ((2, 3, 17, 100), (3, 100, 9)), ((4, 64, 27), (27, 96)), ((256, 256), (256, 256)),
    ((16, 65536), (65536, 8)),
    # config 5's Linear(8192, 256) forward: 8 output tiles, K split into 64
    # subtrees folded by the carry stack
    ((128, 8192), (8192, 256)),
]


@pytest.mark.parametrize("layout", ["nn", "nt", "tn", "tt"])
@pytest.mark.parametrize("ashape,bshape", EXACT_CASES, ids=lambda v: "x".join(map(str, v)))
def test_exact_gemm_arm_is_the_oracle_bit_for_bit(hip, ashape, bshape, layout):
    rng = np.random.default_rng(SEED + sum(ashape) + 3 * sum(bshape) + len(layout))
    a = rng.standard_normal(ashape, dtype=np.float32)
    b = rng.standard_normal(bshape, dtype=np.float32)
    a.reshape(-1)[:3] = [0.0, -0.0, 1e-40]  # signed zero and a subnormal among the products
    def view(x, t):
        if not t:
            return DeviceArray.from_numpy(x)
        return DeviceArray.from_numpy(np.ascontiguousarray(np.swapaxes(x, -1, -2))).transpose(-2, -1)
    got = ops.matmul(view(a, layout[0] == "t"), view(b, layout[1] == "t"),
                     kernel=_lib.GEMM_EXACT).numpy()
    want = O.matmul(a, b)
    assert got.shape == want.shape
    assert got.tobytes() == want.tobytes()


def test_exact_gemm_arm_agrees_with_the_gemv_path(hip):
    """Both reproduce the oracle, so the N == 1 product is the same bits
    whichever arm runs it (the reference's kernel switches are bit-neutral,
    tests/python/test_invariants.py:207-285)."""
    rng = np.random.default_rng(SEED + 99)
    a = rng.standard_normal((300, 2500), dtype=np.float32)
    x = rng.standard_normal((2500, 1), dtype=np.float32)
    da, dx = DeviceArray.from_numpy(a), DeviceArray.from_numpy(x)
    exact = ops.matmul(da, dx, kernel=_lib.GEMM_EXACT).numpy()
    gemv = ops.matmul(da, dx, kernel=_lib.GEMM_GEMV).numpy()
    assert exact.tobytes() == gemv.tobytes() == O.matmul(a, x).tobytes()
