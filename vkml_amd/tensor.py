"""Lazy tensors, the executor and reverse-mode autograd: the host side that
drives the device backend through `Backend.compute(span of nodes)`.

This restates the parts of vkML's host core that the hot path's callers use,
so that the BASELINE training steps (MNIST MLP, CIFAR CNN) run end to end:

  graph      Node with shape/strides/dtype/params and view aliasing
             (reference include/vkml/graph/node.h:69-157, op.h:30-139)
  executor   realize(): topological order, view resolution by aliasing,
             allocation, then ONE backend.compute() over the span
             (reference src/dispatch/executor.cpp:23-154)
  ops        torch-like constructors with the reference's lowering: rank-4
             matmul with broadcast batch axes (src/api/ops.cpp:906-981),
             conv2d = im2col + matmul (:662-705), cross_entropy (:417-441),
             reductions (:119-130), scaled_add (:144-171)
  autograd   backward() with the reference's rules
             (src/autograd/autograd.cpp:84-116, 160-560, 588-673)

A Tensor lives on a backend: the HIP device backend by default. Anything with
the same five methods (alloc/upload/download/compute/synchronize) can stand in,
which is how the tests run the identical graph on the CPU oracle. There is no
implicit fallback: an op the backend does not support raises.
"""
from __future__ import annotations

import ctypes
import struct
import math
from typing import Iterable, Sequence

import numpy as np

from . import _lib

OP = _lib.OP
# View ops are resolved by aliasing on the host and never reach a backend
# (reference backend.h:34-45). Numbered with the reference's OpKind ordinals.
INPUT, FULL, ARANGE = 0, OP["FULL"], OP["ARANGE"]
RESHAPE, PERMUTE, BROADCAST, UNSQUEEZE = 5, 6, 8, 10
VIEW_OPS = {RESHAPE, PERMUTE, BROADCAST, UNSQUEEZE}
LEAF_OPS = {INPUT, FULL, ARANGE}

_VK_DTYPE = {np.dtype(np.float32): _lib.F32, np.dtype(np.int64): _lib.I64,
             np.dtype(np.bool_): _lib.BOOL}

_grad_enabled = True


class no_grad:
    """Context manager that disables graph recording of requires_grad."""

    def __enter__(self):
        global _grad_enabled
        self.prev = _grad_enabled
        _grad_enabled = False

    def __exit__(self, *exc):
        global _grad_enabled
        _grad_enabled = self.prev


def contiguous_strides(shape: Sequence[int]) -> tuple[int, ...]:
    n = len(shape)
    if n == 0:
        return ()
    out = [1] * n
    s = 1
    for i in range(n - 1, 0, -1):
        s *= int(shape[i])
        out[i - 1] = s
    return tuple(out)


def _numel(shape) -> int:
    n = 1
    for e in shape:
        n *= int(e)
    return n


def broadcast_dims(a: Sequence[int], b: Sequence[int]) -> tuple[int, ...]:
    """torch broadcasting of two shapes (reference broadcast_dims)."""
    a, b = list(a), list(b)
    n = max(len(a), len(b))
    a = [1] * (n - len(a)) + a
    b = [1] * (n - len(b)) + b
    out = []
    for x, y in zip(a, b):
        if x != y and x != 1 and y != 1:
            raise ValueError(f"shapes {a} and {b} do not broadcast")
        out.append(max(x, y))
    return tuple(out)


# ---------------------------------------------------------------------------
# Backends
# ---------------------------------------------------------------------------

class DeviceBackend:
    """The HIP device backend (libvkhip) behind the executor."""

    name = "hip"

    def __init__(self, index: int = 0):
        from .device import backend

        self.hip = backend(index)
        self._plans = {}

    def alloc(self, nbytes: int):
        from .device import Buffer

        buf = Buffer(max(int(nbytes), 4))
        if _KEEP is not None:
            _KEEP.append(buf)
        return buf

    def upload(self, storage, offset_bytes: int, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        if arr.nbytes:
            _lib.check(self.hip.lib.vkhip_copy_from_host(
                ctypes.c_void_p(storage.ptr + offset_bytes), arr.ctypes.data_as(ctypes.c_void_p),
                arr.nbytes), "copy_from_host")

    def download(self, storage, offset_bytes: int, out: np.ndarray) -> None:
        if out.nbytes:
            _lib.check(self.hip.lib.vkhip_copy_to_host(
                out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(storage.ptr + offset_bytes),
                out.nbytes), "copy_to_host")

    def compute(self, nodes, count: int) -> None:
        _lib.check(self.hip.lib.vkhip_compute(nodes, count), "compute")

    def sgd_step(self, entries, lr: float, momentum: float, weight_decay: float,
                 nesterov: bool) -> None:
        """entries: (param storage, grad storage, grad offset bytes, velocity
        storage or None, velocity offset bytes, element count, first) per
        parameter; one launch."""
        arr = (_lib.SgdParam * len(entries))()
        if _KEEP is not None:
            _KEEP.extend(x for e in entries for x in (e[0], e[1], e[3]) if x is not None)
        for d, (p, g, goff, v, voff, n, first) in zip(arr, entries):
            d.param = p.ptr
            d.grad = g.ptr + goff
            d.velocity = v.ptr + voff if v is not None else None
            d.n = n
            d.first = 1 if first else 0
        _lib.check(self.hip.lib.vkhip_sgd_step(arr, len(entries), lr, momentum, weight_decay,
                                               1 if nesterov else 0), "sgd_step")

    def transposed_plans_agree(self, batch: int, m: int, n: int, k: int) -> bool:
        """Whether the M x N and N x M products over the same K get the same
        split-K plan, and so the same bits for the same products (the
        library's kernels sum each output's K range in an order only the
        plan's (splits, chunk) decides)."""
        key = (batch, m, n, k)
        hit = self._plans.get(key)
        if hit is None:
            from . import ops

            hit = ops.gemm_plan(batch, m, n, k) == ops.gemm_plan(batch, n, m, k)
            self._plans[key] = hit
        return hit

    def copy(self, copies) -> None:
        """copies: (dst storage, dst offset bytes, src storage, src offset
        bytes, nbytes); one unit of work (Backend::copy_device_to_device)."""
        cs = (_lib.Copy * len(copies))()
        if _KEEP is not None:
            _KEEP.extend(x for c in copies for x in (c[0], c[2]))
        for d, (dst, doff, src, soff, nbytes) in zip(cs, copies):
            d.dst, d.src, d.nbytes = dst.ptr + doff, src.ptr + soff, nbytes
        _lib.check(self.hip.lib.vkhip_copy_device_to_device(cs, len(copies)),
                   "copy_device_to_device")

    def synchronize(self) -> None:
        self.hip.synchronize()


_DEFAULT_BACKEND = None

# While a CapturedStep records, every device buffer its calls touch is kept
# here (see CapturedStep): the replay addresses them by pointer.
_KEEP: list | None = None


def default_backend():
    global _DEFAULT_BACKEND
    if _DEFAULT_BACKEND is None:
        _DEFAULT_BACKEND = DeviceBackend()
    return _DEFAULT_BACKEND


# ---------------------------------------------------------------------------
# Graph
# ---------------------------------------------------------------------------

class Node:
    __slots__ = ("op", "shape", "strides", "dtype", "src", "params", "view_src", "view_offset",
                 "storage", "offset", "computed", "requires_grad", "grad", "backend", "aux",
                 "rec", "__weakref__")

    def __init__(self, op, shape, dtype, backend, src=(), params=b"", requires_grad=False,
                 strides=None):
        self.op = op
        self.shape = tuple(map(int, shape))
        self.strides = tuple(strides) if strides is not None else contiguous_strides(self.shape)
        self.dtype = dtype if isinstance(dtype, np.dtype) else np.dtype(dtype)
        self.src = list(src)
        self.params = params
        self.view_src = None
        self.view_offset = 0
        self.storage = None
        self.offset = 0  # elements
        self.computed = False
        self.requires_grad = requires_grad
        self.grad = None
        self.backend = backend
        self.aux = None  # op-specific host data (permutation, axis, ...)
        self.rec = None  # packed tensor fields, cached once the storage is bound

    @property
    def is_view(self) -> bool:
        return self.op in VIEW_OPS

    @property
    def itemsize(self) -> int:
        return self.dtype.itemsize

    def is_contiguous(self) -> bool:
        expect = 1
        for e, s in zip(reversed(self.shape), reversed(self.strides)):
            if e == 1:
                continue
            if s != expect:
                return False
            expect *= e
        return True


def _params(*values: tuple[str, object]) -> bytes:
    """Packs op params like the reference's 64-byte OpParams payload."""
    out = bytearray()
    for fmt, v in values:
        import struct

        out += struct.pack("<" + fmt, v)
    return bytes(out)


class Tensor:
    """A lazy tensor (reference include/vkml/api/tensor.h)."""

    __slots__ = ("node",)

    def __init__(self, node: Node):
        self.node = node

    # -- construction ------------------------------------------------------------
    @staticmethod
    def from_numpy(arr, requires_grad: bool = False, backend=None) -> "Tensor":
        backend = backend or default_backend()
        arr = np.asarray(arr)
        if arr.dtype == np.float64:
            arr = arr.astype(np.float32)
        if arr.dtype not in _VK_DTYPE:
            raise TypeError(f"unsupported dtype {arr.dtype}")
        n = Node(INPUT, arr.shape, arr.dtype, backend, requires_grad=requires_grad)
        n.storage = backend.alloc(arr.nbytes)
        host = arr.view(np.uint8) if arr.dtype == np.bool_ else arr
        backend.upload(n.storage, 0, host)
        n.computed = True
        return Tensor(n)

    # -- properties -----------------------------------------------------------------
    @property
    def shape(self) -> tuple[int, ...]:
        return self.node.shape

    @property
    def ndim(self) -> int:
        return len(self.node.shape)

    @property
    def dtype(self):
        return self.node.dtype

    @property
    def requires_grad(self) -> bool:
        return self.node.requires_grad

    @property
    def grad(self):
        return Tensor(self.node.grad) if self.node.grad is not None else None

    @grad.setter
    def grad(self, value):
        self.node.grad = value.node if value is not None else None

    def numel(self) -> int:
        return _numel(self.shape)

    def size(self, i: int) -> int:
        return self.shape[i]

    # -- evaluation -------------------------------------------------------------------
    def realize(self) -> "Tensor":
        realize([self])
        return self

    def numpy(self) -> np.ndarray:
        t = self if self.node.is_contiguous() else self.contiguous()
        t.realize()
        n = t.node
        host = np.empty(n.shape, np.uint8 if n.dtype == np.bool_ else n.dtype)
        n.backend.download(n.storage, n.offset * n.itemsize, host)
        return host.astype(np.bool_) if n.dtype == np.bool_ else host

    def item(self) -> float:
        return self.numpy().reshape(-1)[0].item()

    def detach(self) -> "Tensor":
        self.realize()
        n = Node(INPUT, self.shape, self.dtype, self.node.backend, strides=self.node.strides)
        n.storage, n.offset, n.computed = self.node.storage, self.node.offset, True
        return Tensor(n)

    # -- views -----------------------------------------------------------------------------
    def reshape(self, *shape) -> "Tensor":
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        shape = list(shape)
        if -1 in shape:
            known = _numel([e for e in shape if e != -1])
            shape[shape.index(-1)] = self.numel() // max(known, 1)
        if _numel(shape) != self.numel():
            raise ValueError(f"cannot reshape {self.shape} to {tuple(shape)}")
        if tuple(shape) == self.shape:
            return self
        src = self if self.node.is_contiguous() else self.contiguous()
        return _view(RESHAPE, src, shape, contiguous_strides(shape), 0)

    def permute(self, *perm) -> "Tensor":
        if len(perm) == 1 and isinstance(perm[0], (tuple, list)):
            perm = tuple(perm[0])
        perm = [p % self.ndim for p in perm]
        shape = [self.shape[p] for p in perm]
        strides = [self.node.strides[p] for p in perm]
        t = _view(PERMUTE, self, shape, strides, 0)
        t.node.aux = tuple(perm)
        return t

    def transpose(self, a: int, b: int) -> "Tensor":
        perm = list(range(self.ndim))
        a, b = a % self.ndim, b % self.ndim
        perm[a], perm[b] = perm[b], perm[a]
        return self.permute(perm)

    @property
    def T(self) -> "Tensor":
        return self.transpose(-2, -1)

    def unsqueeze(self, axis: int) -> "Tensor":
        axis = axis % (self.ndim + 1)
        shape = list(self.shape)
        strides = list(self.node.strides)
        shape.insert(axis, 1)
        strides.insert(axis, strides[axis] * shape[axis + 1] if axis < len(strides) else 1)
        return _view(UNSQUEEZE, self, shape, strides, 0)

    def broadcast_to(self, dims) -> "Tensor":
        dims = tuple(int(e) for e in dims)
        if dims == self.shape:
            return self
        pad = len(dims) - self.ndim
        if pad < 0:
            raise ValueError(f"cannot broadcast {self.shape} to {dims}")
        src_shape = (1,) * pad + self.shape
        src_str = (0,) * pad + self.node.strides
        strides = []
        for se, ss, te in zip(src_shape, src_str, dims):
            if se == te:
                strides.append(ss)
            elif se == 1:
                strides.append(0)
            else:
                raise ValueError(f"cannot broadcast {self.shape} to {dims}")
        return _view(BROADCAST, self, dims, strides, 0)

    def contiguous(self) -> "Tensor":
        """Self when the layout is already contiguous, a view included (its data
        pointer carries the offset), else a CONTIGUOUS copy (reference
        tensor.cpp:287-299)."""
        if self.node.is_contiguous():
            return self
        if FOLD_CONSTANTS and not self.requires_grad:
            v = _full_value(self)
            if v is not None:
                return full(self.shape, float(v), np.float32, self.node.backend)
        return _unary(OP["CONTIGUOUS"], self)

    def to(self, dtype) -> "Tensor":
        dtype = np.dtype(dtype)
        if dtype == self.dtype:
            return self
        n = Node(OP["CAST"], self.shape, dtype, self.node.backend, [self.node],
                 requires_grad=_grad_enabled and self.requires_grad and dtype == np.float32)
        return Tensor(n)

    # -- arithmetic -----------------------------------------------------------------------
    def __add__(self, o): return add(self, o)
    def __radd__(self, o): return add(self, o)
    def __sub__(self, o): return sub(self, o)
    def __rsub__(self, o): return sub(_scalar_like(self, o), self)
    def __mul__(self, o): return mul(self, o)
    def __rmul__(self, o): return mul(self, o)
    def __truediv__(self, o): return div(self, o)
    def __neg__(self): return neg(self)
    def __matmul__(self, o): return matmul(self, o)

    def backward(self, seed: "Tensor | None" = None) -> None:
        backward(self, seed)

    def __repr__(self) -> str:
        return f"Tensor(shape={self.shape}, dtype={self.dtype}, backend={self.node.backend.name})"


def tensor(data, requires_grad: bool = False, backend=None) -> Tensor:
    return Tensor.from_numpy(np.asarray(data), requires_grad, backend)


def _view(op, t: Tensor, shape, strides, offset) -> Tensor:
    n = Node(op, shape, t.dtype, t.node.backend, [t.node], strides=strides,
             requires_grad=_grad_enabled and t.requires_grad)
    n.view_src = t.node
    n.view_offset = offset
    return Tensor(n)


# ---------------------------------------------------------------------------
# Creation and elementwise ops
# ---------------------------------------------------------------------------

def full(shape, value: float, dtype=np.float32, backend=None) -> Tensor:
    return Tensor(Node(FULL, shape, dtype, backend or default_backend(),
                       params=_params(("d", float(value)))))


def ones(shape, dtype=np.float32, backend=None) -> Tensor:
    return full(shape, 1.0, dtype, backend)


def zeros_like(t: Tensor) -> Tensor:
    return full(t.shape, 0.0, t.dtype, t.node.backend)


def arange(start: float, stop: float, step: float = 1.0, dtype=np.float32, backend=None) -> Tensor:
    count = max(0, math.ceil((stop - start) / step))
    return Tensor(Node(ARANGE, (count,), dtype, backend or default_backend(),
                       params=_params(("d", float(start)), ("d", float(step)))))


# Arithmetic on FULL constants is evaluated on the host (IEEE single
# precision, as the oracle and the device compute it) and a view of a constant
# made contiguous is a new constant: the seed, 1/count and broadcast chain of
# a mean's gradient is then one FULL node instead of four launches.
FOLD_CONSTANTS = True

# The gradient of a weight used as w.T in a product (nn.Linear) computed in
# w's layout (grad^T @ x) rather than as (x^T @ grad)^T then copied: the same
# values (see the MATMUL rule), applied where the backend plans both
# orientations of the product alike.
WEIGHT_GRAD_IN_PLACE_LAYOUT = True


def _matmul_backward(a: "Node", b: "Node", grad: "Tensor", grads: dict) -> None:
    """The MATMUL rule: d(a) = grad @ b^T, d(b) = a^T @ grad (reference
    autograd.cpp), d(b) taken in w's layout when b is a Linear weight's w.T."""
    if a.requires_grad:
        _accumulate(grads, a, matmul(grad, Tensor(b).transpose(-2, -1)))
    if b.requires_grad:
        w = _transposed_matrix_source(b) if WEIGHT_GRAD_IN_PLACE_LAYOUT else None
        if w is not None and len(w.shape) == 2:
            # the backend's product plan must not depend on the orientation
            # (the device's narrow split-K plan can: 128 x 784 and 784 x 128
            # over K = 16384 split K differently)
            agree = getattr(w.backend, "transposed_plans_agree", None)
            batch = int(np.prod(a.shape[:-2], dtype=np.int64)) if len(a.shape) > 2 else 1
            if agree is not None and not agree(batch, w.shape[0], w.shape[1], a.shape[-2]):
                w = None
        if w is not None:
            # b = w^T (x @ w.T, a Linear layer): d(w) = grad^T @ a is the
            # transpose of d(w^T) = a^T @ grad -- the same products summed
            # in the same k order under the same plan -- in w's own layout,
            # so no transposing copy follows.
            _accumulate(grads, w, matmul(grad.transpose(-2, -1), Tensor(a)).reshape(w.shape))
        else:
            _accumulate(grads, b, matmul(Tensor(a).transpose(-2, -1), grad))


def _transposed_matrix_source(b: "Node"):
    """w when node b is the view w.T of a 2-D w that requires grad, or the
    matmul lowering's rank-4 broadcast of that view (leading axes of 1), else
    None."""
    while (b.op == BROADCAST and b.view_src is not None and len(b.view_src.shape) == 2
           and len(b.shape) == 4 and tuple(b.shape[:2]) == (1, 1)
           and tuple(b.shape[2:]) == tuple(b.view_src.shape)):
        b = b.view_src
    if (b.op == PERMUTE and len(b.shape) == 2 and b.aux is not None and list(b.aux) == [1, 0]
            and b.view_src is not None and b.view_src.requires_grad and b.view_src.dtype == np.float32):
        return b.view_src
    return None
_FOLDABLE = {OP["ADD"]: np.add, OP["SUB"]: np.subtract, OP["MUL"]: np.multiply,
             OP["DIV"]: np.divide}


def _full_value(t: "Tensor"):
    """The value of an uncomputed float32 FULL constant, or of a view of one
    (a broadcast or reshape of it), else None."""
    n = t.node
    while n.view_src is not None and n.op in (RESHAPE, BROADCAST, UNSQUEEZE):
        n = n.view_src
    if (n.op != FULL or n.computed or n.dtype != np.float32 or n.requires_grad
            or len(n.params) < 8):
        return None
    import struct

    return np.float32(struct.unpack_from("<d", n.params, 0)[0])


def _scalar_like(peer: Tensor, value) -> Tensor:
    if isinstance(value, Tensor):
        return value
    return full((), float(value), peer.dtype, peer.node.backend)


# A Linear layer's matmul(x, w.T) + bias (and the ReLU after it) as one
# MATMUL_BIAS node: the bias add (and relu) applied where the product's split-K
# partials are folded, the values of the MATMUL, ADD and RELU nodes. False
# builds those nodes.
FUSED_LINEAR_BIAS = True


def _matmul_bias(a: Tensor, b: Tensor, relu: bool):
    """matmul(...) + b as one MATMUL_BIAS node when a is the (reshaped) output
    of a not yet computed MATMUL and b a float32 vector with one value per
    output column; relu=True instead turns such a node (a, as the reshape of a
    MATMUL_BIAS without relu) into one with it. Else None. The replaced nodes
    stay in the graph, computed only if something else needs them."""
    if not FUSED_LINEAR_BIAS or a.dtype != np.float32:
        return None
    v = a.node
    if v.op != RESHAPE or v.view_src is None or v.view_src.computed:
        return None
    mm = v.view_src
    if relu:
        if mm.op != OP["MATMUL_BIAS"] or mm.aux:
            return None
        srcs = list(mm.src)
    else:
        if (mm.op != OP["MATMUL"] or not isinstance(b, Tensor) or b.ndim != 1 or b.dtype != np.float32
                or b.shape[0] != mm.shape[-1] or a.shape[-1] != b.shape[0]):
            return None
        srcs = [mm.src[0], mm.src[1], b.node]
    node = Node(OP["MATMUL_BIAS"], mm.shape, np.float32, mm.backend, srcs,
                params=_params(("I", 1 if relu else 0)),
                requires_grad=_grad_enabled and any(s.requires_grad for s in srcs))
    node.aux = bool(relu)
    return Tensor(node).reshape(a.shape)


def _binary(op, a: Tensor, b, out_dtype=None, params=b"") -> Tensor:
    if op == OP["ADD"] and FUSED_LINEAR_BIAS:
        fused = _matmul_bias(a, b, False)
        if fused is not None:
            return fused
    b = _scalar_like(a, b)
    dims = broadcast_dims(a.shape, b.shape)
    ba = a if a.shape == dims else a.broadcast_to(dims)
    bb = b if b.shape == dims else b.broadcast_to(dims)
    out_dtype = np.dtype(out_dtype or a.dtype)
    rg = _grad_enabled and (a.requires_grad or b.requires_grad) and out_dtype == np.float32
    if FOLD_CONSTANTS and not rg and op in _FOLDABLE and out_dtype == np.float32:
        va, vb = _full_value(a), _full_value(b)
        if va is not None and vb is not None:
            with np.errstate(all="ignore"):
                r = _FOLDABLE[op](va, vb)
            return full(dims, float(np.float32(r)), np.float32, a.node.backend)
    return Tensor(Node(op, dims, out_dtype, a.node.backend, [ba.node, bb.node], params=params,
                       requires_grad=rg))


def _unary(op, a: Tensor) -> Tensor:
    return Tensor(Node(op, a.shape, a.dtype, a.node.backend, [a.node],
                       requires_grad=_grad_enabled and a.requires_grad))


def add(a, b): return _binary(OP["ADD"], a, b)
def sub(a, b): return _binary(OP["SUB"], a, b)
def mul(a, b): return _binary(OP["MUL"], a, b)
def div(a, b): return _binary(OP["DIV"], a, b)
def maximum(a, b): return _binary(OP["MAXIMUM"], a, b)
def minimum(a, b): return _binary(OP["MINIMUM"], a, b)
def equal(a, b): return _binary(OP["EQUAL"], a, b, np.bool_)
def less(a, b): return _binary(OP["LESS"], a, b, np.bool_)
def greater(a, b): return _binary(OP["GREATER"], a, b, np.bool_)
def less_equal(a, b): return _binary(OP["LESS_EQUAL"], a, b, np.bool_)
def greater_equal(a, b): return _binary(OP["GREATER_EQUAL"], a, b, np.bool_)
def neg(a): return _unary(OP["NEG"], a)
def exp(a): return _unary(OP["EXP"], a)
def log(a): return _unary(OP["LOG"], a)
def relu(a):
    if FUSED_CONV_EPILOGUE:
        fused = _conv_bias_relu(a)
        if fused is not None:
            return fused
    if FUSED_LINEAR_BIAS:
        fused = _matmul_bias(a, None, True)
        if fused is not None:
            return fused
    if FUSED_ADD_RELU and a.node.op == OP["ADD"] and a.dtype == np.float32 and len(a.node.src) == 2:
        # relu(x + y) as one ADD_RELU node over the ADD's sources (the ADD
        # stays in the graph, computed only if something else needs it)
        return Tensor(Node(OP["ADD_RELU"], a.shape, np.float32, a.node.backend, list(a.node.src),
                           requires_grad=_grad_enabled and a.node.requires_grad))
    return _unary(OP["RELU"], a)


def _conv_bias_relu(t: Tensor):
    """relu(conv2d(x, w) + bias) as one CONV2D_BIAS_RELU node when t is the
    ADD of a CONV2D node and its bias broadcast from [Cout, 1, 1] (what
    conv2d(x, w, bias) builds), else None. The CONV2D and ADD nodes stay in
    the graph: computed only if something else needs them."""
    n = t.node
    if n.op != OP["ADD"] or n.dtype != np.float32 or len(n.src) != 2:
        return None
    conv, bb = n.src
    if conv.op != OP["CONV2D"] or bb.op != BROADCAST or len(conv.src) != 2:
        return None
    bias3 = bb.src[0]
    cout = conv.shape[1]
    if tuple(bias3.shape) != (cout, 1, 1) or bias3.dtype != np.float32:
        return None
    node = Node(OP["CONV2D_BIAS_RELU"], conv.shape, np.float32, conv.backend,
                [conv.src[0], conv.src[1], bias3], params=conv.params,
                requires_grad=_grad_enabled and n.requires_grad)
    node.aux = conv.aux
    return Tensor(node)


def scaled_add(a: Tensor, b: Tensor, alpha: float, beta: float) -> Tensor:
    """a*alpha + b*beta as one node (reference ops.cpp:144-171)."""
    return _binary(OP["SCALED_ADD"], a, b, params=_params(("f", alpha), ("f", beta)))


def where(cond: Tensor, a: Tensor, b: Tensor) -> Tensor:
    dims = broadcast_dims(broadcast_dims(cond.shape, a.shape), b.shape)
    c, x, y = cond.broadcast_to(dims), a.broadcast_to(dims), b.broadcast_to(dims)
    rg = _grad_enabled and (a.requires_grad or b.requires_grad)
    return Tensor(Node(OP["WHERE"], dims, a.dtype, a.node.backend, [c.node, x.node, y.node],
                       requires_grad=rg))


# ---------------------------------------------------------------------------
# Reductions, softmax, matmul, convolution, pooling
# ---------------------------------------------------------------------------

def _axes_mask(axes, ndim: int) -> int:
    if axes is None or (isinstance(axes, (list, tuple)) and len(axes) == 0):
        return (1 << ndim) - 1 if ndim > 0 else 0
    if isinstance(axes, int):
        axes = [axes]
    mask = 0
    for a in axes:
        a = a % ndim
        if mask & (1 << a):
            raise ValueError(f"axis {a} given more than once")
        mask |= 1 << a
    return mask


def _reduction(op, a: Tensor, axes, keepdim: bool, out_dtype=None) -> Tensor:
    mask = _axes_mask(axes, a.ndim)
    dims = []
    for i, e in enumerate(a.shape):
        if not mask & (1 << i):
            dims.append(e)
        elif keepdim:
            dims.append(1)
    out_dtype = np.dtype(out_dtype or a.dtype)
    n = Node(op, dims, out_dtype, a.node.backend, [a.node],
             params=_params(("I", mask), ("?", keepdim)),
             requires_grad=_grad_enabled and a.requires_grad and out_dtype == np.float32)
    n.aux = (mask, keepdim)
    return Tensor(n)


def sum(a: Tensor, axes=None, keepdim: bool = False) -> Tensor:  # noqa: A001
    return _reduction(OP["SUM"], a, axes, keepdim)


def mean(a: Tensor, axes=None, keepdim: bool = False) -> Tensor:
    return _reduction(OP["MEAN"], a, axes, keepdim)


def amax(a: Tensor, axes=None, keepdim: bool = False) -> Tensor:
    return _reduction(OP["MAX"], a, axes, keepdim)


def argmax(a: Tensor, axis: int, keepdim: bool = False) -> Tensor:
    return _reduction(OP["ARGMAX"], a, [axis], keepdim, np.int64)


def _softmax_family(op, a: Tensor, axis: int) -> Tensor:
    axis = axis % a.ndim
    n = Node(op, a.shape, a.dtype, a.node.backend, [a.node], params=_params(("i", axis)),
             requires_grad=_grad_enabled and a.requires_grad)
    n.aux = axis
    return Tensor(n)


def softmax(a: Tensor, axis: int = -1) -> Tensor:
    return _softmax_family(OP["SOFTMAX"], a, axis)


def log_softmax(a: Tensor, axis: int = -1) -> Tensor:
    return _softmax_family(OP["LOG_SOFTMAX"], a, axis)


def matmul(a: Tensor, b: Tensor) -> Tensor:
    """torch.matmul semantics lowered to one rank-4 Matmul node over broadcast
    views (reference ops.cpp:906-981)."""
    a_vec, b_vec = a.ndim == 1, b.ndim == 1
    am = a.unsqueeze(0) if a_vec else a
    bm = b.unsqueeze(1) if b_vec else b
    m, k = am.shape[-2], am.shape[-1]
    k2, n = bm.shape[-2], bm.shape[-1]
    if k != k2:
        raise ValueError(f"matmul inner dimensions disagree: {k} vs {k2}")
    real_batch = broadcast_dims(am.shape[:-2], bm.shape[:-2])
    if len(real_batch) > 2:
        raise ValueError("matmul supports at most 2 batch axes")
    batch = (1,) * (2 - len(real_batch)) + real_batch
    a4 = am.broadcast_to(batch + (m, k))
    b4 = bm.broadcast_to(batch + (k, n))
    node = Node(OP["MATMUL"], batch + (m, n), a.dtype, a.node.backend, [a4.node, b4.node],
                requires_grad=_grad_enabled and (a.requires_grad or b.requires_grad))
    out = Tensor(node)
    final = list(real_batch) + ([] if a_vec else [m]) + ([] if b_vec else [n])
    return out.reshape(final)


def _unfold_params(kernel, stride, pad, dil, hw) -> bytes:
    return _params(*[("i", int(v)) for v in (*kernel, *stride, *pad, *dil, *hw)])


def _pair(v):
    return (int(v[0]), int(v[1])) if isinstance(v, (tuple, list)) else (int(v), int(v))


def window_count(extent, k, s, p, d) -> int:
    return (extent + 2 * p - (d * (k - 1) + 1)) // s + 1


def im2col(x: Tensor, kernel, stride=1, padding=0, dilation=1) -> Tensor:
    kernel, stride, padding, dilation = map(_pair, (kernel, stride, padding, dilation))
    n_, c, h, w = x.shape
    oh = window_count(h, kernel[0], stride[0], padding[0], dilation[0])
    ow = window_count(w, kernel[1], stride[1], padding[1], dilation[1])
    node = Node(OP["IM2COL"], (n_, c * kernel[0] * kernel[1], oh * ow), x.dtype, x.node.backend,
                [x.node], params=_unfold_params(kernel, stride, padding, dilation, (h, w)),
                requires_grad=_grad_enabled and x.requires_grad)
    node.aux = (kernel, stride, padding, dilation, (h, w))
    return Tensor(node)


def col2im(cols: Tensor, image_hw, kernel, stride=1, padding=0, dilation=1) -> Tensor:
    kernel, stride, padding, dilation, image_hw = map(_pair, (kernel, stride, padding, dilation,
                                                              image_hw))
    n_, rows, _ = cols.shape
    c = rows // (kernel[0] * kernel[1])
    src = cols.contiguous()
    node = Node(OP["COL2IM"], (n_, c, image_hw[0], image_hw[1]), cols.dtype, cols.node.backend,
                [src.node], params=_unfold_params(kernel, stride, padding, dilation, image_hw),
                requires_grad=_grad_enabled and cols.requires_grad)
    node.aux = (kernel, stride, padding, dilation, image_hw)
    return Tensor(node)


# conv2d evaluates flat_weight @ im2col(x) as one CONV2D node: a GEMM that
# gathers its columns from the image, bit-identical to the IM2COL + MATMUL
# pair it replaces (the same GEMM plan and summation order) without writing
# the C*kh*kw times larger column matrix. Its gradient is the reference
# graph's, built from the same nodes. False builds the reference's graph.
IMPLICIT_CONV = True
IMPLICIT_CONV_MAX_WINDOW = 63  # kh*kw the device gather handles; larger windows use the graph


def conv2d(x: Tensor, weight: Tensor, bias: Tensor | None = None, stride=1, padding=0,
           dilation=1) -> Tensor:
    """im2col -> flat_weight @ cols (batch-broadcast A) -> reshape -> + bias
    (reference ops.cpp:662-705)."""
    stride, padding, dilation = map(_pair, (stride, padding, dilation))
    cout = weight.shape[0]
    kernel = (weight.shape[2], weight.shape[3])
    oh = window_count(x.shape[2], kernel[0], stride[0], padding[0], dilation[0])
    ow = window_count(x.shape[3], kernel[1], stride[1], padding[1], dilation[1])
    if (IMPLICIT_CONV and x.ndim == 4 and weight.ndim == 4 and x.dtype == np.float32
            and weight.dtype == np.float32 and weight.shape[1] == x.shape[1]
            and oh > 0 and ow > 0 and kernel[0] * kernel[1] <= IMPLICIT_CONV_MAX_WINDOW):
        w = weight.contiguous()
        node = Node(OP["CONV2D"], (x.shape[0], cout, oh, ow), np.float32, x.node.backend,
                    [x.node, w.node],
                    params=_unfold_params(kernel, stride, padding, dilation, x.shape[2:]),
                    requires_grad=_grad_enabled and (x.requires_grad or w.requires_grad))
        node.aux = (kernel, stride, padding, dilation, tuple(x.shape[2:]))
        out = Tensor(node)
    else:
        cols = im2col(x, kernel, stride, padding, dilation)
        flat_weight = weight.reshape(cout, cols.shape[1])
        out = matmul(flat_weight, cols).reshape(x.shape[0], cout, oh, ow)
    if bias is not None:
        out = add(out, bias.reshape(cout, 1, 1))
    return out


def max_pool2d(x: Tensor, kernel, stride=None, padding=0) -> Tensor:
    kernel = _pair(kernel)
    stride = _pair(stride) if stride is not None else kernel
    padding = _pair(padding)
    n_, c, h, w = x.shape
    oh = window_count(h, kernel[0], stride[0], padding[0], 1)
    ow = window_count(w, kernel[1], stride[1], padding[1], 1)
    node = Node(OP["MAX_POOL2D"], (n_, c, oh, ow), x.dtype, x.node.backend, [x.node],
                params=_unfold_params(kernel, stride, padding, (1, 1), (h, w)),
                requires_grad=_grad_enabled and x.requires_grad)
    return Tensor(node)


def one_hot_f32(target: Tensor, classes: int) -> Tensor:
    """Cast(Equal(Cast(labels->F32)[:, None], arange(C))) (reference ops.cpp:347-354)."""
    indices = arange(0.0, float(classes), 1.0, np.float32, target.node.backend)
    return equal(target.to(np.float32).unsqueeze(-1), indices).to(np.float32)


# The backends evaluate the per-row part of cross_entropy, -sum(log_softmax(x)
# * one_hot, -1), as one CROSS_ENTROPY node and its gradient as one
# CROSS_ENTROPY_BACKWARD node, operation for operation the values of the
# reference graph below (one kernel each instead of ~8 nodes each way). False
# builds the reference's node graph.
FUSED_CROSS_ENTROPY = True

# The relu gradient where(less_equal(x, zeros_like(x)), zeros_like(g), g)
# (reference autograd.cpp:397-408) as one RELU_BACKWARD node: x <= 0 ? +0 : g,
# the same values (a select, no arithmetic) from one pass over x and g instead
# of four kernels and two materialised zero tensors. False builds the
# reference's nodes.
FUSED_RELU_BACKWARD = True

# A relu gradient whose incoming gradient is that of a max-pool over the
# relu's output (conv -> relu -> pool) as one MAX_POOL2D_BACKWARD_RELU node:
# the pool's gradient routed to each window's first maximum, then masked by
# the pool's input <= 0, the values of the two nodes (selects only) in one
# pass. False keeps MAX_POOL2D_BACKWARD and RELU_BACKWARD.
FUSED_POOL_RELU_GRAD = True

# The weight and bias gradients of a conv layer (conv2d with bias, relu, then a
# 2x2 stride-2 max-pool) whose input needs no gradient, as one
# CONV2D_POOL_WEIGHT_BIAS_GRAD node over the image, the layer's output and the
# pool's output gradient, in place of MAX_POOL2D_BACKWARD_RELU,
# CONV2D_WEIGHT_GRAD_SUM and the bias's SUM: on the device the relu-masked pool
# gradient is formed inside the weight-gradient kernel (never written) and the
# bias gradient summed there in the pairwise tree's order; the nodes' values.
# False keeps the three nodes.
FUSED_CONV_POOL_GRAD = True

# A conv layer's bias gradient, when its relu-masked pool gradient is one
# MAX_POOL2D_BACKWARD_RELU node of 2x2 windows at stride 2, as one
# MAX_POOL2D_BACKWARD_RELU_BIAS node whose output holds the pool gradient and
# the bias gradient (both views of it): the device sums each plane of the pool
# gradient while it writes it, in the pairwise tree's order, instead of a
# reduction re-reading it. False keeps the pool gradient and the bias's SUM.
FUSED_POOL_BIAS_GRAD = True

# A relu gradient whose incoming gradient is a product (a Linear layer's input
# gradient, grad @ w, feeding the relu before it) as one MATMUL_RELU_BACKWARD
# node: the select applied where the product's split-K partials are folded.
# False keeps MATMUL and RELU_BACKWARD.
FUSED_MATMUL_RELU_GRAD = True


def _relu_grad(mask_src: "Node", y: "Node", g: "Tensor") -> "Tensor":
    """RELU_BACKWARD(mask_src, g), where mask_src is the relu's input or its
    output y (relu(v) <= 0 exactly where v <= 0; a NaN stays NaN, so both
    masks select alike). When g is the not yet computed gradient of a max-pool
    whose input is y, and y feeds nothing else (else g would be a sum), one
    MAX_POOL2D_BACKWARD_RELU node over the pool gradient's sources instead;
    when g is (a reshape of) a not yet computed product, one
    MATMUL_RELU_BACKWARD node over its operands."""
    gn = g.node
    if (FUSED_POOL_RELU_GRAD and gn.op == OP["MAX_POOL2D_BACKWARD"] and not gn.computed
            and gn.src[1] is y):
        return Tensor(Node(OP["MAX_POOL2D_BACKWARD_RELU"], gn.shape, np.float32, gn.backend,
                           list(gn.src), params=gn.params))
    mm = gn
    while mm.op == RESHAPE and mm.view_src is not None:
        mm = mm.view_src
    if (FUSED_MATMUL_RELU_GRAD and mm.op == OP["MATMUL"] and not mm.computed
            and mask_src.is_contiguous() and _numel(mm.shape) == _numel(mask_src.shape)):
        mask = Tensor(mask_src).reshape(mm.shape)
        node = Node(OP["MATMUL_RELU_BACKWARD"], mm.shape, np.float32, mm.backend,
                    [mm.src[0], mm.src[1], mask.node])
        return Tensor(node).reshape(g.shape)
    return Tensor(Node(OP["RELU_BACKWARD"], mask_src.shape, np.float32, mask_src.backend,
                       [mask_src, gn]))


def cross_entropy(logits: Tensor, target: Tensor) -> Tensor:
    """mean(-sum(log_softmax(logits) * one_hot, -1)) (reference ops.cpp:417-441)."""
    batched = logits.unsqueeze(0) if logits.ndim == 1 else logits
    labels = target.unsqueeze(0) if logits.ndim == 1 else target
    if (FUSED_CROSS_ENTROPY and batched.ndim == 2 and batched.dtype == np.float32
            and labels.dtype == np.int64 and labels.ndim == 1
            and 1 <= batched.shape[1] <= 2048 and labels.shape[0] == batched.shape[0]):
        x = batched.contiguous()
        y = labels.contiguous()
        node = Node(OP["CROSS_ENTROPY"], (x.shape[0],), np.float32, x.node.backend,
                    [x.node, y.node], requires_grad=_grad_enabled and x.requires_grad)
        return mean(Tensor(node))
    picked = sum(mul(log_softmax(batched, -1), one_hot_f32(labels, batched.shape[1])), [-1])
    return mean(neg(picked))


# ---------------------------------------------------------------------------
# Executor
# ---------------------------------------------------------------------------

# One vkhip_node record (include/vkhip.h): op, n_src, out, src[3], params[64];
# a vkhip_tensor is data, dtype, ndim, ne[4], nb[4] (extents and strides
# left-aligned, unused slots 0). Packed with one struct call per node.
_NODE_RECORD = struct.Struct("<ii" + "Qii4q4q" * 4 + "64s")
_NO_TENSOR = (0,) * 11
_PADS = tuple((0,) * (4 - k) for k in range(5))
assert _NODE_RECORD.size == ctypes.sizeof(_lib.NodeDesc)


def _tensor_fields(n: Node) -> tuple:
    """The vkhip_tensor fields of a node with bound storage, cached on the node
    (storage, offset and strides only change through assign(), which clears it)."""
    rec = n.rec
    if rec is None:
        pad = _PADS[len(n.shape)]
        if n.storage is None:
            return (0, _VK_DTYPE[n.dtype], len(n.shape)) + n.shape + pad + n.strides + pad
        data = n.storage.ptr + n.offset * n.dtype.itemsize
        rec = n.rec = (data, _VK_DTYPE[n.dtype], len(n.shape)) + n.shape + pad + n.strides + pad
    return rec


def realize(tensors: Iterable[Tensor]) -> None:
    """Evaluate every uncomputed node the tensors depend on, as ONE backend
    compute() over the span in dependency order (reference executor.cpp:90-154)."""
    roots = [t.node for t in tensors if t is not None and not t.node.computed]
    if not roots:
        return
    # Post-order walk of the uncomputed subgraph: a node is emitted once all
    # of its sources are computed or emitted (sources in order, so the
    # sequence is the one a recursive walk from the roots would give).
    order: list[Node] = []
    seen: set[int] = set()
    stack = list(reversed(roots))
    push, pop, mark, emit = stack.append, stack.pop, seen.add, order.append
    while stack:
        node = stack[-1]
        nid = id(node)
        if nid in seen:
            pop()
            continue
        waiting = False
        for c in reversed(node.src):
            if not c.computed and id(c) not in seen:
                push(c)
                waiting = True
        if waiting:
            continue
        pop()
        mark(nid)
        emit(node)
    by_backend: dict[int, list[Node]] = {}
    backends = {}
    for node in order:
        if node.is_view:
            src = node.view_src
            node.storage = src.storage
            node.offset = src.offset + node.view_offset
            node.computed = True
            continue
        if node.op == INPUT:
            raise RuntimeError("an input tensor has no storage")
        node.storage = node.backend.alloc(max(_numel(node.shape), 1) * node.itemsize)
        node.offset = 0
        by_backend.setdefault(id(node.backend), []).append(node)
        backends[id(node.backend)] = node.backend
    size = _NODE_RECORD.size
    pack = _NODE_RECORD.pack_into
    for key, nodes in by_backend.items():
        buf = bytearray(size * len(nodes))
        for k, node in enumerate(nodes):
            src = node.src
            ns = len(src)
            pack(buf, k * size, node.op, ns, *_tensor_fields(node),
                 *(_tensor_fields(src[0]) if ns > 0 else _NO_TENSOR),
                 *(_tensor_fields(src[1]) if ns > 1 else _NO_TENSOR),
                 *(_tensor_fields(src[2]) if ns > 2 else _NO_TENSOR),
                 node.params or b"")
        arr = (_lib.NodeDesc * len(nodes)).from_buffer(buf)
        if _KEEP is not None:
            _KEEP.extend(x.storage for node in nodes for x in (node, *node.src) if x is not None)
        backends[key].compute(arr, len(nodes))
        for node in nodes:
            node.computed = True


def assign(params: Sequence[Tensor], values: Sequence[Tensor]) -> None:
    """Copy each value into its parameter's storage, as one unit of work
    (reference python/vkml/__init__.py:153-165, which becomes one
    copy_device_to_device over the pairs). Every alias of a parameter (a
    detach() or view taken earlier) then sees the new values, as it does in
    the reference and under the fused SGD step, which updates in place. A
    parameter without bound contiguous storage of its own is bound to the
    value's storage instead."""
    params, values = list(params), list(values)
    if len(params) != len(values):
        raise ValueError(f"assign: {len(params)} destinations but {len(values)} sources")
    realize(values)
    copies = {}
    for p, v in zip(params, values):
        if p.shape != v.shape or p.dtype != v.dtype:
            raise ValueError(f"assign: {v.shape} {v.dtype} into {p.shape} {p.dtype}")
        pn, vn = p.node, v.node
        if (pn.storage is not None and pn.computed and pn.is_contiguous() and vn.is_contiguous()
                and pn.backend is vn.backend and pn.storage is not vn.storage):
            nbytes = _numel(pn.shape) * pn.itemsize
            if nbytes:
                copies.setdefault(id(pn.backend), (pn.backend, []))[1].append(
                    (pn.storage, pn.offset * pn.itemsize, vn.storage, vn.offset * vn.itemsize,
                     nbytes))
            continue
        pn.storage = vn.storage
        pn.offset = vn.offset
        pn.strides = vn.strides
        pn.rec = None
        pn.computed = True
    for backend, pairs in copies.values():
        backend.copy(pairs)


class CapturedStep:
    """A step (forward, backward, optimiser) recorded once and replayed.

    The Python host core costs several microseconds per node to build, order
    and pack a graph, which at the BASELINE training shapes is more than the
    device work of a step (reference docs/SMALL-STEP-LATENCY.md:44-51 measures
    the same gap for its own host). When a step's graph repeats, only its
    inputs change: `CapturedStep(fn, *example_inputs)` runs `fn` once on device
    tensors holding the example inputs while the backend records every
    compute, SGD and copy call it makes (vkhip_program_begin/end), and each
    later `step(*arrays)` uploads the arrays into those same input tensors,
    replays the recorded calls from C (`vkhip_program_run`) and downloads
    `fn`'s outputs. With graph=True the replay is captured into a HIP graph on
    its first run and launched as one unit afterwards.

    Contract (that of any recorded replay): `fn` builds the same graph every
    call (same shapes and control flow, nothing decided from device values,
    step-varying data only through its arguments); hyper-parameters are those
    of the recording (an optimiser's lr and momentum included); the recording
    step is a real step (it updates the parameters) and every replay continues
    from the state the previous one left. Every device buffer the recorded
    calls touch is held by this object until `close()`, so replays never write
    into memory handed out elsewhere. The recording returns what the eager
    step would; replays return the same bits an eager step would (tested).
    """

    def __init__(self, fn, *example_inputs, graph: bool = False, backend=None, early_outputs: bool = True):
        global _KEEP
        from .device import backend as hip_backend

        self.backend = backend or default_backend()
        if not isinstance(self.backend, DeviceBackend):
            raise TypeError("CapturedStep replays device work: it needs the HIP device backend")
        self.lib = hip_backend().lib
        self.graph = bool(graph)
        self.inputs = [Tensor.from_numpy(np.asarray(a), backend=self.backend) for a in example_inputs]
        self._program = None
        if _KEEP is not None:
            raise RuntimeError("CapturedStep: another step is being recorded")
        keep: list = [t.node.storage for t in self.inputs]
        _KEEP = keep
        try:
            _lib.check(self.lib.vkhip_program_begin(), "program_begin")
            try:
                out = fn(*self.inputs)
                out = list(out) if isinstance(out, (tuple, list)) else [out]
                self.outputs = [t if t.node.is_contiguous() else t.contiguous() for t in out]
                realize(self.outputs)
            finally:
                prog = ctypes.c_void_p()
                code = self.lib.vkhip_program_end(ctypes.byref(prog))
                self._program = prog.value
            _lib.check(code, "program_end")
        finally:
            _KEEP = None
        keep.extend(t.node.storage for t in self.outputs)
        self._keep = keep
        self.first = [t.numpy() for t in self.outputs]
        # Plain replays (graph=False) hand their outputs back from pinned host
        # memory once the units the outputs depend on have run, not after the
        # whole step (vkhip_program_set_outputs hoists those units, a loss's
        # forward tail, ahead of the backward pass): the host reads step i's
        # loss and queues step i + 1 while step i's backward pass and update
        # still run, so the device does not idle between steps.
        self._early = None
        if early_outputs and not self.graph and self.outputs:
            spans = [(t.node.storage.ptr + t.node.offset * t.node.itemsize, t.numel() * t.node.itemsize)
                     for t in self.outputs]
            total = int(np.sum([n for _, n in spans]))  # this module's sum() is the tensor reduction
            if all(n > 0 for _, n in spans) and total <= 4096:
                copies = [_lib.Copy(None, ptr, n) for ptr, n in spans]
                _lib.check(self.lib.vkhip_program_set_outputs(self._program, (_lib.Copy * len(copies))(*copies),
                                                              len(copies)), "program_set_outputs")
                self._early = np.empty(total, np.uint8)

    def info(self) -> dict:
        calls, nodes, has_graph = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_int()
        _lib.check(self.lib.vkhip_program_info(self._program, ctypes.byref(calls), ctypes.byref(nodes),
                                               ctypes.byref(has_graph)), "program_info")
        return {"calls": calls.value, "nodes": nodes.value, "graph": bool(has_graph.value)}

    # Steps queued without reading back (read=False) that may be in flight at
    # once. A deeper queue made every enqueue slower on this runtime (config
    # 1's MLP, graph-launched: 0.43-0.56 ms/step with ~16 steps queued against
    # 0.11 read back); two keep the device busy while the host uploads and
    # launches the next step.
    queue_depth = 2

    def __call__(self, *arrays, read: bool = True, prefetch=None):
        """Copies `arrays` into the recorded inputs, replays the step and
        returns `fn`'s outputs as host arrays. An input is a host array
        (uploaded through the pinned staging slots) or a contiguous
        DeviceArray of the recorded shape and dtype (copied on the device,
        stream-ordered: a data set kept resident in HBM feeds its steps with no
        host copy). read=False returns None without waiting for the step: the
        next call's copies are stream-ordered after this replay, so steps
        queue back to back, at most `queue_depth` of them in flight (the call
        first waits for the oldest); `outputs_now()` reads the latest step's
        outputs and `outputs_to()` copies them on the device.

        prefetch: the next call's host arrays. They are uploaded, once this
        step is queued, into device staging buffers on the backend's copy
        stream (vkhip_copy_from_host_async), so the host copy and the DMA of
        batch i + 1 overlap step i on the device, and copied on the device into
        the recorded inputs right behind this step: the next call given those
        same array objects replays at once (any other arrays are uploaded over
        them, as usual). The host bytes are
        copied when this call returns, so a later change to the arrays is not
        seen.

        A plain replay (graph=False) also reads a DeviceArray input in place
        (vkhip_program_bind_input points the recorded input at it): its bytes
        must stay unchanged until the step has run, and the recorded input
        tensor then no longer holds the latest batch."""
        if self._program is None:
            raise RuntimeError("CapturedStep: closed")
        if not read:
            from .device import Event

            if not hasattr(self, "_events"):
                self._events = [Event() for _ in range(self.queue_depth)]
                self._queued = 0
            if self._queued >= self.queue_depth:
                self._events[self._queued % self.queue_depth].synchronize()
        if len(arrays) != len(self.inputs):
            raise ValueError(f"CapturedStep: {len(arrays)} inputs, recorded with {len(self.inputs)}")
        from .device import DeviceArray

        staged = getattr(self, "_staged", None)
        self._staged = None
        if staged is not None and len(staged) == len(arrays) and all(a is b for a, b in zip(arrays, staged)):
            arrays = ()  # prefetched: already copied into the inputs, stream-ordered
        device_copies = []
        for i, (t, a) in enumerate(zip(self.inputs, arrays)):
            rec = t.node.storage.ptr + t.node.offset * t.node.itemsize
            if isinstance(a, DeviceArray):
                if a.shape != t.shape or a.dtype != t.dtype or not a.is_contiguous():
                    raise ValueError(f"CapturedStep: device input {a.shape} {a.dtype} (contiguous: "
                                     f"{a.is_contiguous()}), recorded {t.shape} {t.dtype}")
                if not self._bind(i, a.ptr):  # read in place, or copied into the recorded input
                    device_copies.append(_lib.Copy(rec, a.ptr, a.nbytes_dense()))
                continue
            a = np.asarray(a)
            if a.shape != t.shape or a.dtype != t.dtype:
                raise ValueError(f"CapturedStep: input {a.shape} {a.dtype}, recorded {t.shape} {t.dtype}")
            host = a.view(np.uint8) if a.dtype == np.bool_ else a
            self._bind(i, rec)
            self.backend.upload(t.node.storage, t.node.offset * t.node.itemsize, host)
        if device_copies:
            _lib.check(self.lib.vkhip_copy_device_to_device(
                (_lib.Copy * len(device_copies))(*device_copies), len(device_copies)), "copy_device_to_device")
        mode = 1 if self.graph else 0 if read else 2  # 2: a plain run nobody reads early
        _lib.check(self.lib.vkhip_program_run(self._program, mode), "program_run")
        if prefetch is not None:
            self.prefetch(*prefetch)
        if read:
            self._queued = 0
            if self._early is None:
                return self.outputs_now()
            _lib.check(self.lib.vkhip_program_read_outputs(
                self._program, self._early.ctypes.data_as(ctypes.c_void_p), self._early.nbytes),
                "program_read_outputs")
            outs, off = [], 0
            for t in self.outputs:
                n = t.node
                size = t.numel() * n.itemsize
                host = self._early[off:off + size].view(np.uint8 if n.dtype == np.bool_ else n.dtype)
                host = host.reshape(n.shape).copy()
                outs.append(host.astype(np.bool_) if n.dtype == np.bool_ else host)
                off += size
            return outs
        self._events[self._queued % self.queue_depth].record()
        self._queued += 1
        return None

    def _recorded_ptr(self, i: int) -> int:
        t = self.inputs[i]
        return t.node.storage.ptr + t.node.offset * t.node.itemsize

    def _binding_state(self) -> None:
        if not hasattr(self, "_bound"):  # every input at its recorded address, rebindable unless a graph
            self._bound = [t.node.storage.ptr + t.node.offset * t.node.itemsize for t in self.inputs]
            self._bindable = [not self.graph] * len(self.inputs)

    def _bind(self, i: int, ptr: int) -> bool:
        """Points recorded input i at device address `ptr` for the plain runs
        that follow (vkhip_program_bind_input); False where the program cannot
        be rebound (a graph, or a recorded call writes the input), the caller
        then copies into the recorded input (which this leaves bound)."""
        t = self.inputs[i]
        self._binding_state()
        if not self._bindable[i]:
            return False
        if self._bound[i] == ptr:
            return True
        rec = t.node.storage.ptr + t.node.offset * t.node.itemsize
        code = self.lib.vkhip_program_bind_input(self._program, ctypes.c_void_p(rec), ctypes.c_void_p(ptr),
                                                 t.numel() * t.node.itemsize)
        if code == _lib.ERR_INVALID:
            self._bindable[i] = False
            if self._bound[i] != rec:
                _lib.check(self.lib.vkhip_program_bind_input(self._program, ctypes.c_void_p(rec),
                                                             ctypes.c_void_p(rec), t.numel() * t.node.itemsize),
                           "program_bind_input")
                self._bound[i] = rec
            return False
        _lib.check(code, "program_bind_input")
        self._bound[i] = ptr
        return True

    def prefetch(self, *arrays) -> None:
        """Uploads host `arrays` (the next call's inputs) into one of two
        staging buffer sets on the copy stream, ahead of the work queued so
        far (the copy stream waits only for that set's last device copy out,
        its `free` event, and records `ready` behind the DMAs), then queues on
        the backend stream, behind that work, the wait for `ready` and the
        device copy into the recorded inputs. The next call given these same
        array objects replays without uploading (see __call__)."""
        from .device import DeviceArray, Event

        if self._program is None:
            raise RuntimeError("CapturedStep: closed")
        if len(arrays) != len(self.inputs) or any(isinstance(a, DeviceArray) for a in arrays):
            raise ValueError("CapturedStep: prefetch takes one host array per recorded input")
        if not hasattr(self, "_stage_bufs"):
            self._stage_bufs = [[DeviceArray(t.shape, np.uint8 if t.dtype == np.bool_ else t.dtype)
                                 for t in self.inputs] for _ in range(2)]
            self._stage_ready = [Event(), Event()]
            self._stage_free = [Event().record(), Event().record()]
            self._stage_next = 0
            # per staging set, built once: its buffers' addresses, its events'
            # handles and the device copies into the recorded inputs
            self._stage_args = []
            for k in range(2):
                copies = [_lib.Copy(t.node.storage.ptr + t.node.offset * t.node.itemsize, buf.ptr, buf.nbytes_dense())
                          for t, buf in zip(self.inputs, self._stage_bufs[k])]
                self._stage_args.append(([ctypes.c_void_p(buf.ptr) for buf in self._stage_bufs[k]],
                                         ctypes.c_void_p(self._stage_free[k].handle),
                                         ctypes.c_void_p(self._stage_ready[k].handle),
                                         (_lib.Copy * len(copies))(*copies), len(copies)))
        k = self._stage_next
        self._stage_next ^= 1
        dsts, free, ready, copies, ncopies = self._stage_args[k]
        for t, a, dst in zip(self.inputs, arrays, dsts):
            a = np.ascontiguousarray(a)
            if a.shape != t.shape or a.dtype != t.dtype:
                raise ValueError(f"CapturedStep: prefetch {a.shape} {a.dtype}, recorded {t.shape} {t.dtype}")
            host = a.view(np.uint8) if a.dtype == np.bool_ else a
            _lib.check(self.lib.vkhip_copy_from_host_async(dst, ctypes.c_void_p(host.ctypes.data), host.nbytes,
                                                           free, ready), "copy_from_host_async")
        # Behind the work queued so far (this step's replay included), the
        # stream waits for the DMAs and copies the staged batch into the
        # recorded inputs; the staging set is free again after that copy.
        # (Reading the staging set in place instead, its inputs rebound to it,
        # measured slower for config 5's replay, 0.348 against 0.341-0.345
        # ms/step: the first convolution then reads the batch cold.)
        _lib.check(self.lib.vkhip_stream_wait_event(ready), "stream_wait_event")
        self._binding_state()
        for i, t in enumerate(self.inputs):
            if self._bound[i] != self._recorded_ptr(i):
                self._bind(i, self._recorded_ptr(i))
        _lib.check(self.lib.vkhip_copy_device_to_device(copies, ncopies), "copy_device_to_device")
        self._stage_free[k].record()
        self._staged = arrays

    def outputs_now(self) -> list:
        """`fn`'s outputs of the latest replay, as host arrays (waits for it)."""
        return [t.numpy() for t in self.outputs]

    def outputs_to(self, *dsts) -> None:
        """Copies `fn`'s outputs of the latest replay into the DeviceArrays
        `dsts` (one per output, contiguous, same byte size), on the device and
        stream-ordered after the replay: a queued loop keeps, say, every
        step's loss in a device log and reads the log once."""
        if len(dsts) != len(self.outputs):
            raise ValueError(f"CapturedStep: {len(dsts)} destinations for {len(self.outputs)} outputs")
        copies = []
        for d, t in zip(dsts, self.outputs):
            nbytes = t.numel() * t.node.itemsize
            if not d.is_contiguous() or d.nbytes_dense() != nbytes:
                raise ValueError(f"CapturedStep: destination of {d.nbytes_dense()} bytes for an output "
                                 f"of {nbytes}")
            copies.append(_lib.Copy(d.ptr, t.node.storage.ptr + t.node.offset * t.node.itemsize, nbytes))
        _lib.check(self.lib.vkhip_copy_device_to_device((_lib.Copy * len(copies))(*copies), len(copies)),
                   "copy_device_to_device")

    def close(self) -> None:
        if self._program is not None:
            _lib.check(self.lib.vkhip_program_destroy(self._program), "program_destroy")
            self._program = None
            self._keep = []

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter teardown
            pass


# ---------------------------------------------------------------------------
# Autograd (reference src/autograd/autograd.cpp)
# ---------------------------------------------------------------------------

def _autograd_order(root: Node) -> list[Node]:
    order, done = [], set()
    stack = [(root, 0)]
    while stack:
        node, i = stack[-1]
        if id(node) in done:
            stack.pop()
            continue
        if i < len(node.src):
            stack[-1] = (node, i + 1)
            child = node.src[i]
            if child is not None and child.requires_grad and id(child) not in done:
                stack.append((child, 0))
            continue
        done.add(id(node))
        order.append(node)
        stack.pop()
    return order


def _accumulate(grads: dict, node: Node, g: Tensor) -> None:
    if node is None or not node.requires_grad:
        return
    key = id(node)
    if key in grads:
        grads[key] = (node, grads[key][1] + g)
    else:
        grads[key] = (node, g)


# The conv2d weight gradient as one CONV2D_WEIGHT_GRAD_SUM node (True) or as
# CONV2D_WEIGHT_GRAD per image followed by the batch SUM node, the reference
# graph's shape (False). The oracle gives both the same bits; the device's
# fast numerics fold the batch into the product's K axis for the former,
# which stays within the GEMM tolerance of the graph, not bit-identical.
FOLD_CONV_WEIGHT_GRAD = True

# The conv2d input gradient as one CONV2D_INPUT_GRAD node (True) or as the
# reference graph's TN product and COL2IM (False). The oracle gives both the
# same bits; the device's fast numerics run the node, for unit strides, as a
# convolution of the gradient with the flipped, transposed weight (within the
# GEMM tolerance of the graph).
FUSED_CONV_INPUT_GRAD = True

# relu(conv2d(x, w, bias)) as one CONV2D_BIAS_RELU node (the conv kernel adds
# the bias and applies the ReLU in its epilogue; the same values as the
# CONV2D, ADD and RELU nodes, bit for bit, on the device and the oracle).
FUSED_CONV_EPILOGUE = True

# relu(a + b) as one ADD_RELU node (a Linear layer's bias add and activation):
# the ADD and RELU nodes' values in one pass.
FUSED_ADD_RELU = True


def reduce_to_shape(g: Tensor, target_dims) -> Tensor:
    """Sums g down to target_dims, undoing a broadcast (autograd.cpp:84-116)."""
    gd = list(g.shape)
    target_dims = list(target_dims)
    if gd == target_dims:
        return g
    lead = len(gd) - len(target_dims)
    axes = []
    for i, e in enumerate(gd):
        if e == 1:
            continue
        absent = i < lead
        stretched = not absent and target_dims[i - lead] == 1
        if absent or stretched:
            axes.append(i)
    r = sum(g, axes, keepdim=True) if axes else g
    return r.reshape(target_dims)


def _conv2d_backward(node: Node, a: Node, b: Node, grad: Tensor, grads: dict) -> None:
    """The CONV2D gradient rule (shared with CONV2D_BIAS_RELU); a = x, b = w."""
    tb = lambda: Tensor(b)  # noqa: E731
    # The reference graph's gradients (ops.cpp:662-705 through the
    # MATMUL, BROADCAST, RESHAPE and IM2COL rules): with the weight
    # broadcast over the batch as flat4 [1, N, Cout, CK] and the columns
    # as cols4 [1, N, CK, L], d(flat) = sum_n g4 @ cols4^T and
    # d(x) = col2im(flat4^T @ g4), value for value.
    kernel, stride, pad, dil, hw = node.aux
    n_, cout, oh, ow = node.shape
    ck = _numel(b.shape[1:])
    g4 = grad.reshape(1, n_, cout, oh * ow)
    if a.requires_grad:
        if FUSED_CONV_INPUT_GRAD:
            # col2im(flat^T @ g4) as one node: with unit strides the device
            # runs it as a convolution of the gradient with the flipped,
            # transposed weight (no column matrix); the oracle computes
            # the product and col2im.
            dx = Node(OP["CONV2D_INPUT_GRAD"], a.shape, np.float32, a.backend,
                      [grad.contiguous().node, b], params=node.params)
            _accumulate(grads, a, Tensor(dx))
        else:
            flat4 = tb().reshape(cout, ck).broadcast_to((1, n_, cout, ck))
            dcols = matmul(flat4.transpose(-2, -1), g4).reshape(n_, ck, oh * ow)
            _accumulate(grads, a, col2im(dcols, hw, kernel, stride, pad, dil))
    if b.requires_grad:
        if FOLD_CONV_WEIGHT_GRAD:
            # sum_n g4 @ cols4^T as one node: the device folds the batch
            # into the product's K axis (no [N, Cout, CK] intermediate);
            # the oracle computes the per-image products and batch sum.
            wg = Node(OP["CONV2D_WEIGHT_GRAD_SUM"], (cout, ck), np.float32, a.backend,
                      [a, grad.contiguous().node], params=node.params)
            dflat = Tensor(wg)
        else:
            # The per-image products g4 @ cols4^T as one CONV2D_WEIGHT_GRAD
            # node (the columns gathered from the image, same bits), then
            # the reference's batch sum.
            wg = Node(OP["CONV2D_WEIGHT_GRAD"], (n_, cout, ck), np.float32, a.backend,
                      [a, grad.contiguous().node], params=node.params)
            prod = Tensor(wg).reshape(1, n_, cout, ck)
            dflat = reduce_to_shape(prod, (cout, ck))
        _accumulate(grads, b, dflat.reshape(b.shape))


def _conv_pool_grads(node: Node, a: Node, b: Node, bias3: Node, dz: Tensor, grads: dict) -> bool:
    """The weight and bias gradients of the CONV2D_BIAS_RELU `node` as one
    CONV2D_POOL_WEIGHT_BIAS_GRAD node when dz is the MAX_POOL2D_BACKWARD_RELU
    of a 2x2, stride-2 pool over the node's output, both gradients are wanted
    and the image's is not (else dz is needed anyway): the weight gradient and
    the bias gradient are views of its output. Returns whether it did."""
    pn = dz.node
    if not (FUSED_CONV_POOL_GRAD and FOLD_CONV_WEIGHT_GRAD and pn.op == OP["MAX_POOL2D_BACKWARD_RELU"]
            and not pn.computed and b.requires_grad and bias3.requires_grad and not a.requires_grad):
        return False
    gp, y = pn.src
    n_, cout, oh, ow = node.shape
    if y is not node or pn.params != _unfold_params((2, 2), (2, 2), (0, 0), (1, 1), (oh, ow)):
        return False
    ck = _numel(b.shape[1:])
    out = Tensor(Node(OP["CONV2D_POOL_WEIGHT_BIAS_GRAD"], (cout * ck + cout,), np.float32, a.backend,
                      [a, y, Tensor(gp).contiguous().node], params=node.params))
    dflat = _view(RESHAPE, out, (cout, ck), (ck, 1), 0)
    dbias = _view(RESHAPE, out, (cout,), (1,), cout * ck)
    _accumulate(grads, b, dflat.reshape(b.shape))
    _accumulate(grads, bias3, dbias.reshape(bias3.shape))
    return True


def _pool_relu_bias_grad(dz: Tensor, bias3: Node, grads: dict):
    """When dz is an uncomputed MAX_POOL2D_BACKWARD_RELU of 2x2 windows at
    stride 2 (over a conv layer's relu output), one MAX_POOL2D_BACKWARD_RELU_BIAS
    node in its place: the bias gradient (dz summed over N, H, W) is accumulated
    from its output's tail and the returned view of its head is dz."""
    pn = dz.node
    if not (FUSED_POOL_BIAS_GRAD and pn.op == OP["MAX_POOL2D_BACKWARD_RELU"] and not pn.computed):
        return None
    y = pn.src[1]
    if len(y.shape) != 4:
        return None
    n_, c, h, w = y.shape
    if h % 2 or w % 2 or pn.params != _unfold_params((2, 2), (2, 2), (0, 0), (1, 1), (h, w)):
        return None
    total = n_ * c * h * w
    out = Tensor(Node(OP["MAX_POOL2D_BACKWARD_RELU_BIAS"], (total + c,), np.float32, pn.backend, list(pn.src),
                      params=pn.params))
    dbias = _view(RESHAPE, out, (c,), (1,), total)
    _accumulate(grads, bias3, dbias.reshape(bias3.shape))
    return _view(RESHAPE, out, tuple(y.shape), contiguous_strides(y.shape), 0)


def _apply_backward(node: Node, grad: Tensor, grads: dict) -> None:
    op = node.op
    a = node.src[0] if node.src else None
    b = node.src[1] if len(node.src) > 1 else None
    ta = lambda: Tensor(a)  # noqa: E731
    tb = lambda: Tensor(b)  # noqa: E731
    out = Tensor(node)
    if op in (OP["CONTIGUOUS"], RESHAPE, UNSQUEEZE):
        _accumulate(grads, a, grad.reshape(a.shape))
    elif op == PERMUTE:
        perm = node.aux
        inverse = [0] * len(perm)
        for i, p in enumerate(perm):
            inverse[p] = i
        _accumulate(grads, a, grad.permute(inverse))
    elif op == BROADCAST:
        _accumulate(grads, a, reduce_to_shape(grad, a.shape))
    elif op == OP["CAST"]:
        _accumulate(grads, a, grad.to(a.dtype))
    elif op == OP["ADD"]:
        _accumulate(grads, a, grad)
        _accumulate(grads, b, grad)
    elif op == OP["SUB"]:
        _accumulate(grads, a, grad)
        _accumulate(grads, b, neg(grad))
    elif op == OP["MUL"]:
        if a.requires_grad:
            _accumulate(grads, a, grad * tb())
        if b.requires_grad:
            _accumulate(grads, b, grad * ta())
    elif op == OP["SCALED_ADD"]:
        import struct

        alpha, beta = struct.unpack("<ff", node.params[:8])
        scale = lambda k: grad if k == 1.0 else scaled_add(grad, grad, k, 0.0)  # noqa: E731
        if a.requires_grad:
            _accumulate(grads, a, scale(alpha))
        if b.requires_grad:
            _accumulate(grads, b, scale(beta))
    elif op == OP["DIV"]:
        if a.requires_grad:
            _accumulate(grads, a, grad / tb())
        if b.requires_grad:
            _accumulate(grads, b, neg(grad * out) / tb())
    elif op == OP["NEG"]:
        _accumulate(grads, a, neg(grad))
    elif op == OP["EXP"]:
        _accumulate(grads, a, grad * out)
    elif op == OP["LOG"]:
        _accumulate(grads, a, grad / ta())
    elif op == OP["RELU"]:
        if FUSED_RELU_BACKWARD:
            x = ta()
            g = grad if grad.shape == x.shape else grad.broadcast_to(x.shape)
            _accumulate(grads, a, _relu_grad(x.node, node, g))
        else:
            _accumulate(grads, a, where(less_equal(ta(), zeros_like(ta())), zeros_like(grad), grad))
    elif op in (OP["SUM"], OP["MEAN"]):
        mask, keepdim = node.aux
        src_dims = list(a.shape)
        g = grad
        if op == OP["MEAN"]:
            count = 1
            for i, e in enumerate(src_dims):
                if mask & (1 << i):
                    count *= e
            g = g / float(count)
        if not keepdim:
            keep = [1 if mask & (1 << i) else e for i, e in enumerate(src_dims)]
            g = g.reshape(keep)
        _accumulate(grads, a, g.broadcast_to(src_dims).contiguous())
    elif op == OP["SOFTMAX"]:
        y = out
        dot = sum(grad * y, [node.aux], keepdim=True)
        _accumulate(grads, a, y * sub(grad, dot.broadcast_to(a.shape)))
    elif op == OP["LOG_SOFTMAX"]:
        total = sum(grad, [node.aux], keepdim=True)
        _accumulate(grads, a, sub(grad, exp(out) * total.broadcast_to(a.shape)))
    elif op == OP["MATMUL"]:
        _matmul_backward(a, b, grad, grads)
    elif op == OP["MATMUL_BIAS"]:
        # the RELU rule (the mask from the output, as for CONV2D_BIAS_RELU)
        # when the node has one, the ADD/BROADCAST rules for the bias (the sum
        # over rows), then the MATMUL rule with that gradient
        g = grad if grad.shape == out.shape else grad.broadcast_to(out.shape)
        dz = _relu_grad(node, node, g) if node.aux else g
        bias = node.src[2]
        if bias.requires_grad:
            _accumulate(grads, bias, reduce_to_shape(dz.reshape((-1, bias.shape[0])), bias.shape))
        _matmul_backward(a, b, dz, grads)
    elif op == OP["ADD_RELU"]:
        # the RELU rule (the mask from the output, as for CONV2D_BIAS_RELU)
        # then the ADD rule: the same gradient to both sources
        g = grad if grad.shape == out.shape else grad.broadcast_to(out.shape)
        dz = _relu_grad(node, node, g)
        if a.requires_grad:
            _accumulate(grads, a, dz)
        if b.requires_grad:
            _accumulate(grads, b, dz)
    elif op == OP["CONV2D_BIAS_RELU"]:
        # relu(conv + bias): the RELU rule (the fused relu gradient, here from
        # the output y: y <= 0 exactly where the pre-activation z <= 0, and a
        # NaN z leaves y NaN, so the select is the one on z), the ADD/BROADCAST
        # rules for the bias (its broadcast adjoint: the sum over N, H, W), then
        # the CONV2D rule with that gradient.
        g = grad if grad.shape == out.shape else grad.broadcast_to(out.shape)
        dz = _relu_grad(node, node, g)
        bias3 = node.src[2]
        if _conv_pool_grads(node, a, b, bias3, dz, grads):
            return
        if bias3.requires_grad:
            with_bias = _pool_relu_bias_grad(dz, bias3, grads)
            if with_bias is not None:
                dz = with_bias
            else:
                _accumulate(grads, bias3, reduce_to_shape(dz, bias3.shape))
        if a.requires_grad or b.requires_grad:
            _conv2d_backward(node, a, b, dz, grads)
    elif op == OP["CONV2D"]:
        _conv2d_backward(node, a, b, grad, grads)
    elif op == OP["CROSS_ENTROPY"]:
        g = Node(OP["CROSS_ENTROPY_BACKWARD"], a.shape, np.float32, a.backend,
                 [a, b, grad.contiguous().node])
        _accumulate(grads, a, Tensor(g))
    elif op == OP["MAX_POOL2D"]:
        inp = ta()
        n = Node(OP["MAX_POOL2D_BACKWARD"], inp.shape, inp.dtype, inp.node.backend,
                 [grad.contiguous().node, inp.contiguous().node], params=node.params)
        _accumulate(grads, a, Tensor(n))
    elif op == OP["IM2COL"]:
        kernel, stride, pad, dil, hw = node.aux
        _accumulate(grads, a, col2im(grad, hw, kernel, stride, pad, dil))
    elif op == OP["COL2IM"]:
        kernel, stride, pad, dil, hw = node.aux
        _accumulate(grads, a, im2col(grad, kernel, stride, pad, dil))
    else:
        raise NotImplementedError(f"no gradient rule for op {op}")


# Backward flushes the gradients built so far after the first rule it applies
# and then after every BACKWARD_FLUSH_EVERY rules, so the device starts on the
# forward pass (which the first gradient needs) while the host is still
# building the rest of the backward graph. Only nodes the final flush would
# compute anyway are computed, each once, so the results are the same; 0 turns
# it off (one flush at the end, as the reference does). Graphs whose
# uncomputed nodes hold less than BACKWARD_FLUSH_MIN_BYTES are flushed once at
# the end: their device work is shorter than a flush's host cost (the config-1
# MLP step: 0.50 ms with one flush, 0.54 with early ones; the config-5 CNN step
# 1.57 -> 1.29 ms with them).
BACKWARD_FLUSH_EVERY = 8
BACKWARD_FLUSH_MIN_BYTES = 8 << 20


# Every switch above that makes the host core build something other than the
# reference's node graph: a rewrite, a fused node, an implicit convolution, an
# early flush. Each computes the reference nodes' values (tested per switch);
# together off, a step's graph is the one vkML's own executor hands its
# backend (src/dispatch/executor.cpp:90-154), node for node, every node a
# reference OpKind.
REFERENCE_GRAPH_SWITCHES = {
    "FOLD_CONSTANTS": False, "WEIGHT_GRAD_IN_PLACE_LAYOUT": False, "FUSED_LINEAR_BIAS": False,
    "IMPLICIT_CONV": False, "FUSED_CROSS_ENTROPY": False, "FUSED_RELU_BACKWARD": False,
    "FUSED_POOL_RELU_GRAD": False, "FUSED_MATMUL_RELU_GRAD": False, "FOLD_CONV_WEIGHT_GRAD": False,
    "FUSED_CONV_INPUT_GRAD": False, "FUSED_CONV_EPILOGUE": False, "FUSED_ADD_RELU": False,
    "FUSED_CONV_POOL_GRAD": False, "FUSED_POOL_BIAS_GRAD": False, "BACKWARD_FLUSH_EVERY": 0,
}


class reference_graph:
    """Context manager: graphs built inside it use the reference's OpKind
    nodes only (REFERENCE_GRAPH_SWITCHES), flushed once per realise, as the
    reference's executor would hand them to a drop-in HipBackend::compute.
    (An optimiser built with SGD(fused=False) keeps its step in ScaledAdd
    nodes as well.)"""

    def __enter__(self):
        mod = globals()
        self._saved = {k: mod[k] for k in REFERENCE_GRAPH_SWITCHES}
        mod.update(REFERENCE_GRAPH_SWITCHES)
        return self

    def __exit__(self, *exc):
        globals().update(self._saved)
        return False


def backward(root: Tensor, seed: Tensor | None = None) -> None:
    """Reverse-mode pass from `root`; leaf gradients are realised in one final
    flush (reference autograd.cpp:588-673), after the early flushes above."""
    if not root.requires_grad:
        raise RuntimeError("backward() called on a tensor that does not require grad")
    if seed is None:
        if root.numel() != 1:
            raise ValueError("backward() without a seed requires a scalar")
        seed = ones(root.shape, root.dtype, root.node.backend)
    order = _autograd_order(root.node)
    grads = {id(root.node): (root.node, seed)}
    every = 0
    if BACKWARD_FLUSH_EVERY > 0:
        pending = 0
        for node in order:
            if not node.computed:
                pending += _numel(node.shape) * node.itemsize
                if pending >= BACKWARD_FLUSH_MIN_BYTES:
                    every = BACKWARD_FLUSH_EVERY
                    break
    with no_grad():
        applied = 0
        for node in reversed(order):
            entry = grads.get(id(node))
            if entry is None or node.op in LEAF_OPS:
                continue
            _apply_backward(node, entry[1], grads)
            if every and applied % every == 0:
                realize([grads[id(s)][1] for s in node.src if id(s) in grads])
            applied += 1
        totals, leaves = [], []
        for node in order:
            if node.op not in LEAF_OPS or not node.requires_grad:
                continue
            entry = grads.get(id(node))
            if entry is None:
                continue
            total = Tensor(node.grad) + entry[1] if node.grad is not None else entry[1]
            totals.append(total)
            leaves.append(node)
    realize(totals)
    for node, t in zip(leaves, totals):
        node.grad = t.node
