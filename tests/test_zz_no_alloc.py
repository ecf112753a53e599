"""The allocation-free GEMM entry point, vkhip_gemm_noalloc, against vkhip_gemm.

Both run the same plan and kernels; the only difference is where the split-K
partials live (a fixed per-device scratch array instead of the grown
workspace), so the results must be the same bytes. Two calls in a row, the
second smaller, check that a call does not depend on what the previous one
left in the shared scratch. A plan that needs more scratch than the array
holds is refused before any launch.
"""
from __future__ import annotations

from ctypes import byref, c_void_p

import numpy as np
import pytest

from vkml_amd import _lib
from vkml_amd.device import DeviceArray

pytestmark = pytest.mark.gpu


def _gemm(entry, a: DeviceArray, b: DeviceArray, split: int = 0) -> tuple[int, np.ndarray]:
    c = DeviceArray((a.shape[-2], b.shape[-1]), np.float32)
    opts = _lib.GemmOpts(_lib.GEMM_AUTO, split)
    lib = _lib.load()
    code = getattr(lib, entry)(c_void_p(a.ptr), byref(a.operand()), c_void_p(b.ptr),
                               byref(b.operand()), c_void_p(c.ptr), byref(opts))
    return code, (c.numpy() if code == _lib.OK else None)


def _operands(m, n, k, seed, layout="nn"):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((m, k) if layout[0] == "n" else (k, m), dtype=np.float32)
    b = rng.standard_normal((k, n) if layout[1] == "n" else (n, k), dtype=np.float32)
    da, db = DeviceArray.from_numpy(a), DeviceArray.from_numpy(b)
    return (da if layout[0] == "n" else da.T), (db if layout[1] == "n" else db.T)


# (m, n, k, layout, split request): split-K shapes of BASELINE config 3 first
# (the scratch holds their partials), then smaller ones in a row.
CASES = [
    [(256, 256, 65536, "nn", 0), (128, 784, 16384, "nn", 0)],
    [(128, 784, 16384, "nt", 0), (192, 160, 512, "nn", 4)],
    [(512, 512, 512, "tn", 0), (100, 37, 300, "nn", 3)],
    [(1024, 1024, 1024, "nn", 0), (64, 10, 128, "nt", 0)],
]


@pytest.mark.parametrize("calls", CASES, ids=lambda c: "_then_".join(f"{m}x{n}x{k}{l}" for m, n, k, l, _ in c))
def test_noalloc_gemm_matches_gemm_on_two_calls(hip, calls):
    for i, (m, n, k, layout, split) in enumerate(calls):
        print(f"noalloc call {i}: {m}x{n}x{k} {layout} split={split}", flush=True)
        a, b = _operands(m, n, k, 1000 + 17 * i + m, layout)
        code, got = _gemm("vkhip_gemm_noalloc", a, b, split)
        assert code == _lib.OK, _lib.load().vkhip_last_error()
        code, want = _gemm("vkhip_gemm", a, b, split)
        assert code == _lib.OK, _lib.load().vkhip_last_error()
        assert got.tobytes() == want.tobytes(), f"call {i} ({m}x{n}x{k} {layout})"


def test_noalloc_gemm_refuses_a_split_beyond_its_scratch(hip):
    """256x256x65536 forced into 256 partitions needs 64 MiB of partials, more
    than the 32 MiB scratch: refused with ERR_INVALID and a message; the
    entry point still works afterwards."""
    a, b = _operands(256, 256, 65536, 7)
    from vkml_amd import ops

    splits, _ = ops.gemm_plan(1, 256, 256, 65536, 256)
    assert splits * 256 * 256 * 4 > 32 << 20
    code, _ = _gemm("vkhip_gemm_noalloc", a, b, 256)
    assert code == _lib.ERR_INVALID
    assert b"scratch" in _lib.load().vkhip_last_error()
    code, got = _gemm("vkhip_gemm_noalloc", a, b, 0)
    assert code == _lib.OK
    code, want = _gemm("vkhip_gemm", a, b, 0)
    assert got.tobytes() == want.tobytes()
