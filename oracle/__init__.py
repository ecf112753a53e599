"""CPU parity oracle -- TEST INFRASTRUCTURE ONLY.

A numpy-facing wrapper over oracle/vkml_oracle.c, the plain-C restatement of
vkML's CPU backend (reference src/backend/cpu/*). Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this, and
only as the checker or the reported CPU baseline. The product (vkml_amd) never
imports it and has no CPU fallback.

Every function takes numpy arrays (any strides; broadcast views allowed) and
returns new arrays. `threads` parallelises over outputs only: results are
bit-identical for every thread count.

Pinning: each function is checked in tests/test_oracle.py against the
reference's own known answers and fixtures (test_ops.cpp:234-293, the
STABILITY_INPUTS and col2im/pool fixtures of test_vulkan_kernels.py), against
float64 / torch closed forms, and by brute force on small inputs.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, byref, c_float, c_int, c_int64, c_uint32, c_uint64, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libvkml_oracle.so"

REDUCE_SUM, REDUCE_MEAN, REDUCE_MAX, REDUCE_MIN, REDUCE_ARGMAX, REDUCE_ARGMIN = range(6)


class Operand(ctypes.Structure):
    _fields_ = [("ne", c_uint32 * 4), ("nb", c_int64 * 4)]


class Unfold(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "kernel_h", "kernel_w", "stride_h", "stride_w", "pad_h", "pad_w",
        "dilation_h", "dilation_w", "image_h", "image_w")]


_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    P = POINTER
    sig = {
        "or_pairwise_sum": (c_float, [c_void_p, c_int64]),
        "or_matmul": (None, [c_void_p, P(Operand), c_void_p, P(Operand), c_void_p, c_int]),
        "or_reduce": (None, [c_int, c_void_p, P(Operand), c_uint32, c_void_p, c_int]),
        "or_softmax": (None, [c_void_p, P(Operand), c_void_p, c_int, c_int, c_int]),
        "or_im2col": (None, [c_void_p, P(Operand), c_void_p, P(Unfold), c_int]),
        "or_col2im": (None, [c_void_p, c_void_p, c_uint32, c_uint32, P(Unfold), c_int]),
        "or_max_pool2d": (c_int, [c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, P(Unfold),
                                  c_int]),
        "or_max_pool2d_backward": (None, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32,
                                          c_uint32, P(Unfold), c_int]),
        "or_split_k_fold": (None, [c_void_p, c_void_p, c_uint64, c_uint32]),
        "or_compute": (c_int, [c_void_p, ctypes.c_size_t, c_int]),
        "or_exp_vec": (None, [c_void_p, c_void_p, c_int64, c_int]),
        "or_set_libm_math": (None, [c_int]),
        "or_get_libm_math": (c_int, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def default_threads() -> int:
    return int(os.environ.get("VKML_ORACLE_THREADS", os.cpu_count() or 1))


def _operand(a: np.ndarray) -> Operand:
    if a.ndim > 4:
        raise ValueError("rank > 4")
    d = Operand()
    pad = 4 - a.ndim
    for i in range(4):
        d.ne[i], d.nb[i] = 1, 0
    for i in range(a.ndim):
        d.ne[pad + i] = a.shape[i]
        d.nb[pad + i] = a.strides[i] // a.itemsize
    return d


def _ptr(a: np.ndarray) -> c_void_p:
    # Base address of element 0 of a (possibly strided, possibly broadcast) view.
    return c_void_p(a.__array_interface__["data"][0])


def _f32(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype != np.float32:
        raise TypeError(f"oracle expects float32, got {a.dtype}")
    return a


def pairwise_sum(v: np.ndarray) -> np.float32:
    """reference pairwise_sum over a contiguous f32 vector (reduce.h:55-72)."""
    v = np.ascontiguousarray(_f32(v)).ravel()
    return np.float32(load().or_pairwise_sum(_ptr(v), v.size))


def matmul(a: np.ndarray, b: np.ndarray, threads: int | None = None) -> np.ndarray:
    """reference matmul_impl (kernels_matmul.cpp:34-87); operands rank 2..4, batch broadcast."""
    a, b = _f32(a), _f32(b)
    batch = np.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    m, k, n = a.shape[-2], a.shape[-1], b.shape[-1]
    if b.shape[-2] != k:
        raise ValueError("inner dimensions disagree")
    ab = np.broadcast_to(a, batch + (m, k))
    bb = np.broadcast_to(b, batch + (k, n))
    out = np.empty(batch + (m, n), np.float32)
    load().or_matmul(_ptr(ab), byref(_operand(ab)), _ptr(bb), byref(_operand(bb)),
                     _ptr(out), threads or default_threads())
    return out


def _reduce(op: int, x: np.ndarray, axes, threads) -> np.ndarray:
    x = _f32(x)
    if axes is None:
        axes = list(range(x.ndim))
    elif isinstance(axes, int):
        axes = [axes]
    axes = sorted({a % x.ndim for a in axes})
    mask = 0
    for a in axes:
        mask |= 1 << (a + 4 - x.ndim)
    kept = tuple(e for i, e in enumerate(x.shape) if i not in axes)
    out = np.empty(kept, np.int64 if op >= REDUCE_ARGMAX else np.float32)
    load().or_reduce(op, _ptr(x), byref(_operand(x)), mask, _ptr(out),
                     threads or default_threads())
    return out


def sum(x, axes=None, threads=None):  # noqa: A001
    return _reduce(REDUCE_SUM, x, axes, threads)


def mean(x, axes=None, threads=None):
    return _reduce(REDUCE_MEAN, x, axes, threads)


def amax(x, axes=None, threads=None):
    return _reduce(REDUCE_MAX, x, axes, threads)


def amin(x, axes=None, threads=None):
    return _reduce(REDUCE_MIN, x, axes, threads)


def argmax(x, axis, threads=None):
    return _reduce(REDUCE_ARGMAX, x, [axis], threads)


def argmin(x, axis, threads=None):
    return _reduce(REDUCE_ARGMIN, x, [axis], threads)


def softmax(x: np.ndarray, axis: int = -1, log: bool = False, threads=None) -> np.ndarray:
    """reference softmax_impl (kernels_reduce.cpp:205-259)."""
    x = _f32(x)
    out = np.empty(x.shape, np.float32)
    load().or_softmax(_ptr(x), byref(_operand(x)), _ptr(out), (axis % x.ndim) + 4 - x.ndim,
                      1 if log else 0, threads or default_threads())
    return out


def log_softmax(x, axis=-1, threads=None):
    return softmax(x, axis, True, threads)


def _unfold(kernel, stride, pad, dil, hw) -> Unfold:
    u = Unfold()
    u.kernel_h, u.kernel_w = kernel
    u.stride_h, u.stride_w = stride
    u.pad_h, u.pad_w = pad
    u.dilation_h, u.dilation_w = dil
    u.image_h, u.image_w = hw
    return u


def _pair(v):
    return (int(v[0]), int(v[1])) if isinstance(v, (tuple, list)) else (int(v), int(v))


def _span(e, k, s, p, d):
    return (e + 2 * p - (d * (k - 1) + 1)) // s + 1


def im2col(x, kernel, stride=1, padding=0, dilation=1, threads=None) -> np.ndarray:
    """reference k_im2col_impl (kernels_movement.cpp:454-483)."""
    x = _f32(x)
    kh, kw = _pair(kernel)
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    n, c, h, w = x.shape
    oh, ow = _span(h, kh, sh, ph, dh), _span(w, kw, sw, pw, dw)
    out = np.empty((n, c * kh * kw, oh * ow), np.float32)
    u = _unfold((kh, kw), (sh, sw), (ph, pw), (dh, dw), (h, w))
    load().or_im2col(_ptr(x), byref(_operand(x)), _ptr(out), byref(u),
                     threads or default_threads())
    return out


def col2im(cols, image_hw, kernel, stride=1, padding=0, dilation=1, threads=None) -> np.ndarray:
    """reference k_col2im_impl (kernels_movement.cpp:500-542)."""
    cols = np.ascontiguousarray(_f32(cols))
    kh, kw = _pair(kernel)
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    h, w = _pair(image_hw)
    n, rows, _ = cols.shape
    c = rows // (kh * kw)
    out = np.empty((n, c, h, w), np.float32)
    u = _unfold((kh, kw), (sh, sw), (ph, pw), (dh, dw), (h, w))
    load().or_col2im(_ptr(cols), _ptr(out), n, c, byref(u), threads or default_threads())
    return out


def max_pool2d(x, kernel, stride=None, padding=0, threads=None) -> np.ndarray:
    """reference k_max_pool2d_impl (kernels_movement.cpp:588-615)."""
    x = np.ascontiguousarray(_f32(x))
    kh, kw = _pair(kernel)
    sh, sw = _pair(stride if stride is not None else kernel)
    ph, pw = _pair(padding)
    n, c, h, w = x.shape
    oh, ow = _span(h, kh, sh, ph, 1), _span(w, kw, sw, pw, 1)
    out = np.empty((n, c, oh, ow), np.float32)
    u = _unfold((kh, kw), (sh, sw), (ph, pw), (1, 1), (h, w))
    st = load().or_max_pool2d(_ptr(x), _ptr(out), n * c, oh, ow, byref(u),
                              threads or default_threads())
    if st != 0:
        raise ValueError("max_pool2d: a window lies entirely in the padding")
    return out


def max_pool2d_backward(grad, x, kernel, stride=None, padding=0, threads=None) -> np.ndarray:
    """reference k_max_pool2d_backward_impl (kernels_movement.cpp:630-680)."""
    x = np.ascontiguousarray(_f32(x))
    grad = np.ascontiguousarray(_f32(grad))
    kh, kw = _pair(kernel)
    sh, sw = _pair(stride if stride is not None else kernel)
    ph, pw = _pair(padding)
    n, c, h, w = x.shape
    out = np.empty(x.shape, np.float32)
    u = _unfold((kh, kw), (sh, sw), (ph, pw), (1, 1), (h, w))
    load().or_max_pool2d_backward(_ptr(grad), _ptr(x), _ptr(out), n * c, grad.shape[2],
                                  grad.shape[3], byref(u), threads or default_threads())
    return out


def expf(x: np.ndarray) -> np.ndarray:
    """The oracle's exp on float32 values (the method in vkml_oracle.c or_expf)."""
    x = np.ascontiguousarray(_f32(x))
    y = np.empty_like(x)
    load().or_exp_vec(_ptr(x), _ptr(y), x.size, 0)
    return y


def logf(x: np.ndarray) -> np.ndarray:
    """The oracle's log on float32 values (vkml_oracle.c or_logf)."""
    x = np.ascontiguousarray(_f32(x))
    y = np.empty_like(x)
    load().or_exp_vec(_ptr(x), _ptr(y), x.size, 1)
    return y


class libm_math:
    """Context manager: inside it the oracle's exp and log (softmax,
    log-softmax, cross-entropy, EXP/LOG nodes) call the platform libm's expf /
    logf, as the reference's std::exp / std::log on float do
    (kernels_reduce.cpp:233,240; kernels_elementwise.cpp:192,196), instead of
    the named correctly rounded methods. Used to measure the spread between two
    valid builds of the reference's CPU arithmetic; not for parity fixtures."""

    def __enter__(self):
        self._prev = load().or_get_libm_math()
        load().or_set_libm_math(1)
        return self

    def __exit__(self, *exc):
        load().or_set_libm_math(self._prev)
        return False


def split_k_fold(ws: np.ndarray, splits: int) -> np.ndarray:
    """reference gemm_split_k_reduce.comp:48-85 over a flat [splits * ne] workspace."""
    ws = np.ascontiguousarray(_f32(ws)).ravel()
    ne = ws.size // splits
    out = np.empty(ne, np.float32)
    load().or_split_k_fold(_ptr(ws), _ptr(out), ne, splits)
    return out


def compute(nodes, count: int, threads: int | None = None) -> int:
    """CPU backend compute() over vkhip node records whose pointers are HOST addresses."""
    return load().or_compute(ctypes.cast(nodes, c_void_p), count, threads or default_threads())


class HostStorage:
    """Host memory standing in for a device allocation."""

    __slots__ = ("buf", "ptr", "nbytes")

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.buf = np.zeros(self.nbytes + 64, np.uint8)
        base = self.buf.ctypes.data
        self.ptr = base + (-base) % 64


class OracleBackend:
    """vkML's CPU backend for the host core's executor: the same node records,
    evaluated by or_compute on host memory. Tests use it to run the identical
    graph the device runs (reference CpuBackend, src/backend/cpu/cpu_backend.cpp)."""

    name = "cpu-oracle"

    def __init__(self, threads: int | None = None):
        self.threads = threads or default_threads()
        load()

    def alloc(self, nbytes: int) -> HostStorage:
        return HostStorage(max(int(nbytes), 4))

    def upload(self, storage: HostStorage, offset_bytes: int, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        ctypes.memmove(storage.ptr + offset_bytes, arr.ctypes.data, arr.nbytes)

    def download(self, storage: HostStorage, offset_bytes: int, out: np.ndarray) -> None:
        ctypes.memmove(out.ctypes.data, storage.ptr + offset_bytes, out.nbytes)

    def compute(self, nodes, count: int) -> None:
        st = compute(nodes, count, self.threads)
        if st != 0:
            raise RuntimeError(f"oracle compute failed with status {st}")

    def synchronize(self) -> None:
        pass

    def copy(self, copies) -> None:
        """copy_device_to_device on host memory: (dst storage, dst offset
        bytes, src storage, src offset bytes, nbytes) per pair."""
        for dst, doff, src, soff, nbytes in copies:
            ctypes.memmove(dst.ptr + doff, src.ptr + soff, nbytes)

    def sgd_step(self, entries, lr: float, momentum: float, weight_decay: float,
                 nesterov: bool) -> None:
        """The fused optimiser step on host memory, as the reference's
        ScaledAdd nodes compute it (python/vkml/optim.py:146-199,
        scaled_add.comp:41-66): each a*alpha + b*beta is two float32 products
        and one float32 sum (numpy rounds each operation), products by 1.0
        being exact."""
        f32 = np.float32
        for p_st, g_st, goff, v_st, voff, n, first in entries:
            p = np.ctypeslib.as_array(ctypes.cast(p_st.ptr, ctypes.POINTER(ctypes.c_float)), (n,))
            g = np.ctypeslib.as_array(ctypes.cast(g_st.ptr + goff, ctypes.POINTER(ctypes.c_float)),
                                      (n,)).copy()
            if weight_decay != 0.0:
                g = g + p * f32(weight_decay)
            direction = g
            if momentum != 0.0:
                v = np.ctypeslib.as_array(ctypes.cast(v_st.ptr + voff, ctypes.POINTER(ctypes.c_float)),
                                          (n,))
                v[...] = g if first else v * f32(momentum) + g
                direction = g + v * f32(momentum) if nesterov else v
            p[...] = p + direction * f32(-lr)
