"""Eager op-level API over the device backend: one call, one launch sequence.

Each function mirrors the reference op it replaces (argument meaning, output
shape, error behaviour) and calls the matching C entry point of libvkhip:

  matmul        vkml::matmul (src/api/ops.cpp:906-981) for rank-2..4 operands
  im2col        vkml::im2col (ops.cpp:485-512)
  col2im        vkml::col2im (ops.cpp:514-541)
  softmax       vkml::softmax / log_softmax (ops.cpp:883-900)
  sum/mean/amax/amin/argmax/argmin   vkml reductions (ops.cpp:119-130, 851-879)
  max_pool2d    vkml::max_pool2d (ops.cpp:611-641) and its backward node
  scaled_add    vkml::scaled_add (ops.cpp:144-171)
"""
from __future__ import annotations

from ctypes import byref, c_uint32, c_void_p
from typing import Iterable, Sequence

import numpy as np

from . import _lib
from ._lib import check
from .device import DeviceArray, backend


def _pair(v) -> tuple[int, int]:
    if isinstance(v, (tuple, list)):
        if len(v) != 2:
            raise ValueError(f"expected a pair, got {v}")
        return int(v[0]), int(v[1])
    return int(v), int(v)


def _f32(x: DeviceArray, what: str) -> None:
    if x.dtype != np.float32:
        raise TypeError(f"{what}: expected float32, got {x.dtype}")


# ---- GEMM family --------------------------------------------------------------------

def gemm_plan(batch: int, m: int, n: int, k: int, split_k: int = 0) -> tuple[int, int]:
    """(splits, chunk) the AUTO planner picks (or a forced request gives)."""
    lib = _lib.load()
    s, c = c_uint32(), c_uint32()
    check(lib.vkhip_gemm_plan(batch, m, n, k, split_k, byref(s), byref(c)), "gemm_plan")
    return s.value, c.value


def matmul(a: DeviceArray, b: DeviceArray, *, kernel: int = _lib.GEMM_AUTO,
           split_k: int = 0, out: DeviceArray | None = None) -> DeviceArray:
    """C = A @ B with batch broadcasting; A/B may be transposed or broadcast views.

    Rank-1 operands follow torch.matmul's rules as the reference does
    (ops.cpp:906-981): a vector on the left is a 1xK row, on the right a Kx1
    column, and the added axis is dropped from the result.
    """
    _f32(a, "matmul")
    _f32(b, "matmul")
    drop_m = drop_n = False
    if a.ndim == 1:
        a = DeviceArray((1, a.shape[0]), a.dtype, (0, a.strides[0]), a.buffer, a.offset)
        drop_m = True
    if b.ndim == 1:
        b = DeviceArray((b.shape[0], 1), b.dtype, (b.strides[0], 0), b.buffer, b.offset)
        drop_n = True
    if a.shape[-1] != b.shape[-2]:
        raise ValueError(f"matmul inner dimensions disagree: {a.shape} @ {b.shape}")
    batch = np.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    if len(batch) > 2:
        raise ValueError("matmul supports at most two batch axes (rank 4)")
    m, k, n = a.shape[-2], a.shape[-1], b.shape[-1]
    ab = a.broadcast_to(batch + (m, k))
    bb = b.broadcast_to(batch + (k, n))
    shape = batch + (m, n)
    if out is None:
        out = DeviceArray(shape, np.float32)
    elif out.shape != shape or not out.is_contiguous():
        raise ValueError("matmul: out must be contiguous with the result shape")
    opts = _lib.GemmOpts(kernel, split_k)
    check(_lib.load().vkhip_gemm(c_void_p(ab.ptr), byref(ab.operand()), c_void_p(bb.ptr),
                                 byref(bb.operand()), c_void_p(out.ptr), byref(opts)), "matmul")
    if drop_m or drop_n:
        final = list(shape)
        if drop_n:
            final.pop(-1)
        if drop_m:
            final.pop(-2 if not drop_n else -1)
        out = out.reshape(final)
    return out


def split_k_reduce(ws: DeviceArray, splits: int) -> DeviceArray:
    """Carry-stack fold of `splits` equal slices of a flat f32 workspace."""
    _f32(ws, "split_k_reduce")
    if not ws.is_contiguous() or ws.size % splits:
        raise ValueError("split_k_reduce: workspace must be contiguous, splits * ne elements")
    ne = ws.size // splits
    out = DeviceArray((ne,), np.float32)
    check(_lib.load().vkhip_split_k_reduce(c_void_p(ws.ptr), c_void_p(out.ptr), ne, splits),
          "split_k_reduce")
    return out


def _out(out: DeviceArray | None, shape, dtype=np.float32) -> DeviceArray:
    """The result buffer: `out` if given (contiguous, right shape), else new."""
    shape = tuple(int(e) for e in shape)
    if out is None:
        return DeviceArray(shape, dtype)
    if out.shape != shape or out.dtype != np.dtype(dtype) or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous {np.dtype(dtype)} array of shape {shape}")
    return out


def gemv(a: DeviceArray, x: DeviceArray, out: DeviceArray | None = None) -> DeviceArray:
    """y = A @ x for A [M,K] with unit inner stride (the N == 1 matmul)."""
    _f32(a, "gemv")
    _f32(x, "gemv")
    if a.ndim != 2 or x.ndim != 1 or a.shape[1] != x.shape[0] or a.strides[1] != 1:
        raise ValueError("gemv: expects A [M,K] with unit inner stride and x [K]")
    y = _out(out, (a.shape[0],))
    check(_lib.load().vkhip_gemv(c_void_p(a.ptr), a.strides[0], c_void_p(x.ptr), x.strides[0],
                                 c_void_p(y.ptr), a.shape[0], a.shape[1]), "gemv")
    return y


# ---- convolution lowering -------------------------------------------------------------

def window_count(extent: int, k: int, s: int, p: int, d: int) -> int:
    """Output positions along one axis (reference window_count, ops.cpp:448-452)."""
    return (extent + 2 * p - (d * (k - 1) + 1)) // s + 1


def im2col(x: DeviceArray, kernel, stride=1, padding=0, dilation=1,
           out: DeviceArray | None = None) -> DeviceArray:
    """[N, C, H, W] -> [N, C*kh*kw, out_h*out_w] (reference ops.cpp:485-512)."""
    _f32(x, "im2col")
    if x.ndim != 4:
        raise ValueError("im2col expects a rank-4 NCHW input")
    kh, kw = _pair(kernel)
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    n, c, h, w = x.shape
    oh, ow = window_count(h, kh, sh, ph, dh), window_count(w, kw, sw, pw, dw)
    if oh <= 0 or ow <= 0:
        raise ValueError("im2col: kernel larger than the padded image")
    out = _out(out, (n, c * kh * kw, oh * ow))
    u = _lib.unfold((kh, kw), (sh, sw), (ph, pw), (dh, dw), (h, w))
    check(_lib.load().vkhip_im2col(c_void_p(x.ptr), byref(x.operand()), c_void_p(out.ptr),
                                   byref(u)), "im2col")
    return out


def col2im(cols: DeviceArray, image_hw, kernel, stride=1, padding=0, dilation=1,
           out: DeviceArray | None = None) -> DeviceArray:
    """[N, C*kh*kw, L] -> [N, C, H, W], the adjoint of im2col (reference ops.cpp:514-541)."""
    _f32(cols, "col2im")
    if cols.ndim != 3:
        raise ValueError("col2im expects [N, C*kh*kw, L]")
    if not cols.is_contiguous():
        from .device import contiguous
        cols = contiguous(cols)
    kh, kw = _pair(kernel)
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    h, w = _pair(image_hw)
    n, rows, L = cols.shape
    if rows % (kh * kw):
        raise ValueError("col2im: rows not divisible by the kernel area")
    if window_count(h, kh, sh, ph, dh) * window_count(w, kw, sw, pw, dw) != L:
        raise ValueError("col2im: column count disagrees with the image geometry")
    c = rows // (kh * kw)
    out = _out(out, (n, c, h, w))
    u = _lib.unfold((kh, kw), (sh, sw), (ph, pw), (dh, dw), (h, w))
    check(_lib.load().vkhip_col2im(c_void_p(cols.ptr), c_void_p(out.ptr), n, c, byref(u)),
          "col2im")
    return out


def conv2d(x: DeviceArray, weight: DeviceArray, stride=1, padding=0, dilation=1,
           out: DeviceArray | None = None) -> DeviceArray:
    """[N, C, H, W] * [Cout, C, kh, kw] (or the flat [Cout, C*kh*kw]) ->
    [N, Cout, out_h, out_w]: the reference's im2col -> flat_weight @ cols
    (ops.cpp:662-705) as one GEMM that gathers the columns straight from the
    image, without materialising them. Windows of up to 63 elements (kh*kw);
    larger ones raise the library's UNSUPPORTED error."""
    _f32(x, "conv2d")
    _f32(weight, "conv2d")
    if x.ndim != 4 or weight.ndim != 4:
        raise ValueError("conv2d expects an NCHW input and a [Cout, C, kh, kw] weight")
    cout, cin, kh, kw = weight.shape
    if cin != x.shape[1]:
        raise ValueError(f"conv2d: weight has {cin} input channels, the image {x.shape[1]}")
    if not weight.is_contiguous():
        from .device import contiguous
        weight = contiguous(weight)
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    n, _, h, w = x.shape
    oh, ow = window_count(h, kh, sh, ph, dh), window_count(w, kw, sw, pw, dw)
    if oh <= 0 or ow <= 0:
        raise ValueError("conv2d: kernel larger than the padded image")
    out = _out(out, (n, cout, oh, ow))
    u = _lib.unfold((kh, kw), (sh, sw), (ph, pw), (dh, dw), (h, w))
    wd = _lib.operand((cout, cin * kh * kw), (cin * kh * kw, 1))
    check(_lib.load().vkhip_conv2d(c_void_p(x.ptr), byref(x.operand()), c_void_p(weight.ptr),
                                   byref(wd), c_void_p(out.ptr), byref(u)), "conv2d")
    return out


def conv2d_weight_grad(x: DeviceArray, grad: DeviceArray, kernel, stride=1, padding=0,
                       dilation=1, out: DeviceArray | None = None) -> DeviceArray:
    """Per-image weight-gradient products of a convolution, [N, Cout, C*kh*kw]
    = grad [N, Cout, out_h, out_w] @ im2col(x)^T, without materialising the
    columns (the reference's matmul(grad, cols^T) in conv2d's backward,
    autograd.cpp:548-553 over ops.cpp:662-705); summing over N gives dW."""
    _f32(x, "conv2d_weight_grad")
    _f32(grad, "conv2d_weight_grad")
    if x.ndim != 4 or grad.ndim != 4 or grad.shape[0] != x.shape[0]:
        raise ValueError("conv2d_weight_grad expects an NCHW image and an [N, Cout, oh, ow] gradient")
    kh, kw = _pair(kernel)
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    n, c, h, w = x.shape
    oh, ow = window_count(h, kh, sh, ph, dh), window_count(w, kw, sw, pw, dw)
    if grad.shape[2:] != (oh, ow):
        raise ValueError(f"conv2d_weight_grad: gradient is {grad.shape[2:]}, geometry gives {(oh, ow)}")
    if not grad.is_contiguous():
        from .device import contiguous
        grad = contiguous(grad)
    cout = grad.shape[1]
    out = _out(out, (n, cout, c * kh * kw))
    u = _lib.unfold((kh, kw), (sh, sw), (ph, pw), (dh, dw), (h, w))
    gd = _lib.operand((1, n, cout, oh * ow), (0, cout * oh * ow, oh * ow, 1))
    check(_lib.load().vkhip_conv2d_weight_grad(c_void_p(x.ptr), byref(x.operand()),
                                               c_void_p(grad.ptr), byref(gd), c_void_p(out.ptr),
                                               byref(u)), "conv2d_weight_grad")
    return out


def conv2d_input_grad(grad: DeviceArray, weight: DeviceArray, image_hw, stride=1, padding=0,
                      dilation=1, out: DeviceArray | None = None) -> DeviceArray:
    """The convolution's input gradient [N, C, H, W] = col2im(flat_weight^T @
    grad[n]): conv2d's backward for x (autograd.cpp:548-553 through the matmul
    and im2col adjoints, ops.cpp:662-705). Fast numerics with unit strides run
    one convolution of grad with the flipped, transposed weight; otherwise the
    TN product and col2im."""
    _f32(grad, "conv2d_input_grad")
    _f32(weight, "conv2d_input_grad")
    if grad.ndim != 4 or weight.ndim != 4 or grad.shape[1] != weight.shape[0]:
        raise ValueError("conv2d_input_grad expects an [N, Cout, oh, ow] gradient and a [Cout, C, kh, kw] weight")
    cout, c, kh, kw = weight.shape
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    h, w = _pair(image_hw)
    oh, ow = window_count(h, kh, sh, ph, dh), window_count(w, kw, sw, pw, dw)
    if grad.shape[2:] != (oh, ow):
        raise ValueError(f"conv2d_input_grad: gradient is {grad.shape[2:]}, geometry gives {(oh, ow)}")
    if not grad.is_contiguous():
        from .device import contiguous
        grad = contiguous(grad)
    if not weight.is_contiguous():
        from .device import contiguous
        weight = contiguous(weight)
    n = grad.shape[0]
    out = _out(out, (n, c, h, w))
    u = _lib.unfold((kh, kw), (sh, sw), (ph, pw), (dh, dw), (h, w))
    wd = _lib.operand((1, 1, cout, c * kh * kw), (0, 0, c * kh * kw, 1))
    check(_lib.load().vkhip_conv2d_input_grad(c_void_p(grad.ptr), byref(grad.operand()),
                                              c_void_p(weight.ptr), byref(wd), c_void_p(out.ptr),
                                              byref(u)), "conv2d_input_grad")
    return out


def conv2d_weight_grad_sum(x: DeviceArray, grad: DeviceArray, kernel, stride=1, padding=0,
                           dilation=1, out: DeviceArray | None = None) -> DeviceArray:
    """The convolution's weight gradient summed over the batch, [Cout, C*kh*kw]
    = sum_n grad[n] @ im2col(x[n])^T: conv2d's backward for the weight
    (autograd.cpp:548-553) followed by the broadcast adjoint's batch sum
    (autograd.cpp:84-116). Fast numerics with out_h*out_w a multiple of 32 run
    one product with the batch folded into K; otherwise the per-image products
    and the batch sum."""
    _f32(x, "conv2d_weight_grad_sum")
    _f32(grad, "conv2d_weight_grad_sum")
    if x.ndim != 4 or grad.ndim != 4 or grad.shape[0] != x.shape[0]:
        raise ValueError("conv2d_weight_grad_sum expects an NCHW image and an [N, Cout, oh, ow] gradient")
    kh, kw = _pair(kernel)
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    n, c, h, w = x.shape
    oh, ow = window_count(h, kh, sh, ph, dh), window_count(w, kw, sw, pw, dw)
    if grad.shape[2:] != (oh, ow):
        raise ValueError(f"conv2d_weight_grad_sum: gradient is {grad.shape[2:]}, geometry gives {(oh, ow)}")
    if not grad.is_contiguous():
        from .device import contiguous
        grad = contiguous(grad)
    cout = grad.shape[1]
    out = _out(out, (cout, c * kh * kw))
    u = _lib.unfold((kh, kw), (sh, sw), (ph, pw), (dh, dw), (h, w))
    gd = _lib.operand((1, n, cout, oh * ow), (0, cout * oh * ow, oh * ow, 1))
    check(_lib.load().vkhip_conv2d_weight_grad_sum(c_void_p(x.ptr), byref(x.operand()),
                                                   c_void_p(grad.ptr), byref(gd), c_void_p(out.ptr),
                                                   byref(u)), "conv2d_weight_grad_sum")
    return out


# ---- softmax and reductions --------------------------------------------------------------

def _axis4(x: DeviceArray, axis: int) -> int:
    if not -x.ndim <= axis < x.ndim:
        raise ValueError(f"axis {axis} out of range for rank {x.ndim}")
    return (axis % x.ndim) + 4 - x.ndim


def softmax(x: DeviceArray, axis: int = -1, log: bool = False,
            out: DeviceArray | None = None) -> DeviceArray:
    _f32(x, "softmax")
    out = _out(out, x.shape)
    check(_lib.load().vkhip_softmax(c_void_p(x.ptr), byref(x.operand()), c_void_p(out.ptr),
                                    _axis4(x, axis), 1 if log else 0), "softmax")
    return out


def log_softmax(x: DeviceArray, axis: int = -1) -> DeviceArray:
    return softmax(x, axis, log=True)


def _reduce(op: int, x: DeviceArray, axes, keepdim: bool,
            out: DeviceArray | None = None) -> DeviceArray:
    _f32(x, "reduce")
    if axes is None:
        axes = list(range(x.ndim))
    elif isinstance(axes, int):
        axes = [axes]
    axes = sorted({a % x.ndim for a in axes}) if x.ndim else []
    mask = 0
    for a in axes:
        mask |= 1 << (a + 4 - x.ndim)
    kept = [e for i, e in enumerate(x.shape) if i not in axes]
    shape = [1 if i in axes else e for i, e in enumerate(x.shape)] if keepdim else kept
    dt = np.int64 if op in (_lib.REDUCE_ARGMAX, _lib.REDUCE_ARGMIN) else np.float32
    out = _out(out, shape, dt)
    check(_lib.load().vkhip_reduce(op, c_void_p(x.ptr), byref(x.operand()), mask,
                                   c_void_p(out.ptr)), "reduce")
    return out


def sum(x: DeviceArray, axes=None, keepdim: bool = False,
        out: DeviceArray | None = None) -> DeviceArray:  # noqa: A001
    return _reduce(_lib.REDUCE_SUM, x, axes, keepdim, out)


def mean(x: DeviceArray, axes=None, keepdim: bool = False,
        out: DeviceArray | None = None) -> DeviceArray:
    return _reduce(_lib.REDUCE_MEAN, x, axes, keepdim, out)


def amax(x: DeviceArray, axes=None, keepdim: bool = False,
        out: DeviceArray | None = None) -> DeviceArray:
    return _reduce(_lib.REDUCE_MAX, x, axes, keepdim, out)


def amin(x: DeviceArray, axes=None, keepdim: bool = False,
        out: DeviceArray | None = None) -> DeviceArray:
    return _reduce(_lib.REDUCE_MIN, x, axes, keepdim, out)


def argmax(x: DeviceArray, axis: int, keepdim: bool = False) -> DeviceArray:
    return _reduce(_lib.REDUCE_ARGMAX, x, [axis], keepdim)


def argmin(x: DeviceArray, axis: int, keepdim: bool = False) -> DeviceArray:
    return _reduce(_lib.REDUCE_ARGMIN, x, [axis], keepdim)


# ---- pooling and optimiser arithmetic ------------------------------------------------------

def max_pool2d(x: DeviceArray, kernel, stride=None, padding=0) -> DeviceArray:
    """First-maximum pooling with -inf padding (reference ops.cpp:611-641)."""
    _f32(x, "max_pool2d")
    if x.ndim != 4:
        raise ValueError("max_pool2d expects NCHW")
    if not x.is_contiguous():
        from .device import contiguous
        x = contiguous(x)
    kh, kw = _pair(kernel)
    sh, sw = _pair(stride if stride is not None else kernel)
    ph, pw = _pair(padding)
    n, c, h, w = x.shape
    oh, ow = window_count(h, kh, sh, ph, 1), window_count(w, kw, sw, pw, 1)
    out = DeviceArray((n, c, oh, ow), np.float32)
    u = _lib.unfold((kh, kw), (sh, sw), (ph, pw), (1, 1), (h, w))
    check(_lib.load().vkhip_max_pool2d(c_void_p(x.ptr), c_void_p(out.ptr), n * c, oh, ow,
                                       byref(u)), "max_pool2d")
    return out


def max_pool2d_backward(grad: DeviceArray, x: DeviceArray, kernel, stride=None,
                        padding=0) -> DeviceArray:
    _f32(grad, "max_pool2d_backward")
    from .device import contiguous
    if not x.is_contiguous():
        x = contiguous(x)
    if not grad.is_contiguous():
        grad = contiguous(grad)
    kh, kw = _pair(kernel)
    sh, sw = _pair(stride if stride is not None else kernel)
    ph, pw = _pair(padding)
    n, c, h, w = x.shape
    out = DeviceArray(x.shape, np.float32)
    u = _lib.unfold((kh, kw), (sh, sw), (ph, pw), (1, 1), (h, w))
    check(_lib.load().vkhip_max_pool2d_backward(c_void_p(grad.ptr), c_void_p(x.ptr),
                                                c_void_p(out.ptr), n * c, grad.shape[2],
                                                grad.shape[3], byref(u)), "max_pool2d_backward")
    return out


def scaled_add(a: DeviceArray, b: DeviceArray, alpha: float, beta: float) -> DeviceArray:
    """a*alpha + b*beta, two rounded multiplies and one add (reference ADR 0013)."""
    if a.shape != b.shape or not (a.is_contiguous() and b.is_contiguous()):
        raise ValueError("scaled_add: contiguous operands of one shape")
    out = DeviceArray(a.shape, np.float32)
    check(_lib.load().vkhip_scaled_add(c_void_p(a.ptr), c_void_p(b.ptr), c_void_p(out.ptr),
                                       a.size, alpha, beta), "scaled_add")
    return out


def synchronize() -> None:
    backend().synchronize()
