"""Device side of the host: the HIP backend object and device arrays.

`HipBackend` mirrors vkML's `Backend` interface (reference
include/vkml/backend/api/backend.h:49-125): name, device, capabilities,
allocate (the allocator), supports, compute(span of nodes), copy_from_host,
copy_to_host, copy_device_to_device (batched) and synchronize. It is a thin
layer over the C ABI in include/vkhip.h; every launch happens in libvkhip.so.

`DeviceArray` is a strided view (extents + element strides, rank <= 4) over a
device allocation, the shape/storage pair a vkML `Node` carries.
"""
from __future__ import annotations

import ctypes
import weakref
from ctypes import c_size_t, byref, c_uint32, c_void_p
from typing import Sequence

import numpy as np

from . import _lib
from ._lib import check

_DTYPES = {np.dtype(np.float32): _lib.F32, np.dtype(np.int64): _lib.I64,
           np.dtype(np.int32): _lib.I32, np.dtype(np.bool_): _lib.BOOL,
           np.dtype(np.uint8): _lib.BOOL}
_NP = {_lib.F32: np.float32, _lib.I64: np.int64, _lib.I32: np.int32, _lib.BOOL: np.bool_}


def vk_dtype(dt) -> int:
    return _DTYPES[np.dtype(dt)]


def contiguous_strides(shape: Sequence[int]) -> tuple[int, ...]:
    out, s = [], 1
    for e in reversed(list(shape)):
        out.append(s)
        s *= int(e)
    return tuple(reversed(out))


class Buffer:
    """One device allocation, returned to the backend's caches when the last
    view dies (the backend's single stream orders every use, so this is safe
    while work is in flight)."""

    __slots__ = ("ptr", "nbytes", "__weakref__")

    def __init__(self, nbytes: int):
        lib = backend().lib
        p = c_void_p()
        check(lib.vkhip_alloc(max(int(nbytes), 0), byref(p)), "alloc")
        self.ptr = p.value or 0
        self.nbytes = int(nbytes)

    def __del__(self):
        if self.ptr:
            try:
                _free(self.ptr)
            except Exception:  # interpreter teardown: the backend is gone already
                pass
            self.ptr = 0


def _free(ptr: int) -> None:
    b = _BACKEND
    if b is not None and b.alive:
        b.lib.vkhip_free(ptr)


class PinnedArray(np.ndarray):
    """A host array in pinned memory (vkhip_host_alloc), for batches that a
    data loader fills where the DMA reads them: an upload ahead of the stream
    (vkhip_copy_from_host_async, CapturedStep.prefetch) reads it in place
    instead of copying it into a staging slot first. Keep its values
    unchanged until the step that consumes the upload has run."""

    _block = None


class _HostBlock:
    __slots__ = ("ptr", "__weakref__")

    def __init__(self, nbytes: int):
        p = c_void_p()
        check(backend().lib.vkhip_host_alloc(max(int(nbytes), 1), byref(p)), "host_alloc")
        self.ptr = p.value or 0

    def __del__(self):
        b = _BACKEND
        if self.ptr and b is not None and b.alive:
            try:
                b.lib.vkhip_host_free(c_void_p(self.ptr))
            except Exception:  # interpreter teardown
                pass
        self.ptr = 0


def pinned_empty(shape, dtype=np.float32) -> PinnedArray:
    """An uninitialised PinnedArray of `shape` and `dtype`."""
    dt = np.dtype(dtype)
    count = int(np.prod(shape)) if len(tuple(shape)) else 1
    block = _HostBlock(count * dt.itemsize)
    raw = (ctypes.c_uint8 * max(count * dt.itemsize, 1)).from_address(block.ptr)
    arr = np.frombuffer(raw, dtype=dt, count=count).reshape(shape).view(PinnedArray)
    arr._block = block
    return arr


def pinned_copy(a) -> PinnedArray:
    """A PinnedArray holding a copy of `a`."""
    a = np.asarray(a)
    out = pinned_empty(a.shape, a.dtype)
    out[...] = a
    return out


class DeviceArray:
    """A strided view over a Buffer: extents, element strides, dtype, offset."""

    __slots__ = ("buffer", "shape", "strides", "dtype", "offset")

    def __init__(self, shape, dtype=np.float32, strides=None, buffer: Buffer | None = None,
                 offset: int = 0):
        self.shape = tuple(int(e) for e in shape)
        self.dtype = np.dtype(dtype)
        self.strides = tuple(int(s) for s in strides) if strides is not None else \
            contiguous_strides(self.shape)
        if buffer is None:
            buffer = Buffer(self.nbytes_dense())
        self.buffer = buffer
        self.offset = int(offset)

    # -- geometry ---------------------------------------------------------------
    @property
    def ndim(self) -> int:
        return len(self.shape)

    @property
    def size(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    @property
    def itemsize(self) -> int:
        return self.dtype.itemsize

    def nbytes_dense(self) -> int:
        return self.size * self.itemsize

    @property
    def ptr(self) -> int:
        return self.buffer.ptr + self.offset * self.itemsize

    def is_contiguous(self) -> bool:
        expect = 1
        for e, s in zip(reversed(self.shape), reversed(self.strides)):
            if e == 1:
                continue
            if s != expect:
                return False
            expect *= e
        return True

    def operand(self) -> _lib.Operand:
        return _lib.operand(self.shape, self.strides)

    def desc(self) -> _lib.TensorDesc:
        d = _lib.TensorDesc()
        d.data = self.ptr
        d.dtype = vk_dtype(self.dtype)
        d.ndim = self.ndim
        for i, (e, s) in enumerate(zip(self.shape, self.strides)):
            d.ne[i], d.nb[i] = e, s
        return d

    # -- views (zero copy, as the reference's view ops are) -------------------------
    def transpose(self, a: int = -2, b: int = -1) -> "DeviceArray":
        a %= self.ndim
        b %= self.ndim
        shape, strides = list(self.shape), list(self.strides)
        shape[a], shape[b] = shape[b], shape[a]
        strides[a], strides[b] = strides[b], strides[a]
        return DeviceArray(shape, self.dtype, strides, self.buffer, self.offset)

    @property
    def T(self) -> "DeviceArray":
        return self.transpose(-2, -1)

    def reshape(self, *shape) -> "DeviceArray":
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        shape = list(shape)
        if -1 in shape:
            known = int(np.prod([e for e in shape if e != -1], dtype=np.int64))
            shape[shape.index(-1)] = self.size // max(known, 1)
        if int(np.prod(shape, dtype=np.int64)) != self.size:
            raise ValueError(f"cannot reshape {self.shape} to {tuple(shape)}")
        if not self.is_contiguous():
            raise ValueError("reshape of a non-contiguous view needs a contiguous copy first")
        return DeviceArray(shape, self.dtype, None, self.buffer, self.offset)

    def broadcast_to(self, shape) -> "DeviceArray":
        shape = tuple(int(e) for e in shape)
        pad = len(shape) - self.ndim
        src_shape = (1,) * pad + self.shape
        src_str = (0,) * pad + self.strides
        strides = []
        for se, ss, te in zip(src_shape, src_str, shape):
            if se == te:
                strides.append(ss)
            elif se == 1:
                strides.append(0)
            else:
                raise ValueError(f"cannot broadcast {self.shape} to {shape}")
        return DeviceArray(shape, self.dtype, strides, self.buffer, self.offset)

    # -- host transfer ------------------------------------------------------------------
    @staticmethod
    def from_numpy(arr: np.ndarray) -> "DeviceArray":
        arr = np.ascontiguousarray(arr)
        if arr.dtype == np.bool_:
            arr = arr.view(np.uint8)
            out = DeviceArray(arr.shape, np.bool_)
        else:
            out = DeviceArray(arr.shape, arr.dtype)
        if arr.nbytes:
            check(backend().lib.vkhip_copy_from_host(c_void_p(out.ptr),
                                                     arr.ctypes.data_as(c_void_p), arr.nbytes),
                  "copy_from_host")
        return out

    def numpy(self) -> np.ndarray:
        src = self if self.is_contiguous() else contiguous(self)
        host = np.empty(src.shape, dtype=np.uint8 if src.dtype == np.bool_ else src.dtype)
        if host.nbytes:
            check(backend().lib.vkhip_copy_to_host(host.ctypes.data_as(c_void_p),
                                                   c_void_p(src.ptr), host.nbytes),
                  "copy_to_host")
        return host.astype(np.bool_) if src.dtype == np.bool_ else host

    def __repr__(self) -> str:
        return f"DeviceArray(shape={self.shape}, strides={self.strides}, dtype={self.dtype})"


class HipBackend:
    """vkML `Backend` over libvkhip (reference backend.h:49-125)."""

    def __init__(self, device_index: int = 0):
        self.lib = _lib.load()
        check(self.lib.vkhip_init(device_index), "init")
        self.device_index = device_index
        caps = _lib.Caps()
        check(self.lib.vkhip_caps_get(byref(caps)), "caps")
        self.caps = caps
        self.alive = True

    # Backend::name / device / capabilities
    def name(self) -> str:
        return "hip"

    def device(self) -> str:
        return f"hip:{self.device_index}"

    def capabilities(self) -> _lib.Caps:
        return self.caps

    # numerics mode (vkhip_set_numerics): "fast" or "exact"
    def set_numerics(self, mode: str) -> None:
        codes = {"fast": _lib.NUMERICS_FAST, "exact": _lib.NUMERICS_EXACT}
        if mode not in codes:
            raise ValueError(f"numerics mode {mode!r}: 'fast' or 'exact'")
        check(self.lib.vkhip_set_numerics(codes[mode]), "set_numerics")

    def numerics(self) -> str:
        return "exact" if self.lib.vkhip_get_numerics() == _lib.NUMERICS_EXACT else "fast"

    # Backend::allocator
    def allocate(self, shape, dtype=np.float32) -> DeviceArray:
        return DeviceArray(shape, dtype)

    # Backend::supports / compute
    def supports(self, node: _lib.NodeDesc) -> bool:
        return bool(self.lib.vkhip_supports(byref(node)))

    def compute(self, nodes) -> None:
        if isinstance(nodes, _lib.NodeDesc):
            nodes = [nodes]
        n = len(nodes)
        if n == 0:
            return
        if isinstance(nodes, ctypes.Array):
            arr = nodes
        else:
            arr = (_lib.NodeDesc * n)(*nodes)
        check(self.lib.vkhip_compute(arr, n), "compute")

    # Backend::copy_*
    def copy_from_host(self, dst: DeviceArray, src: np.ndarray) -> None:
        src = np.ascontiguousarray(src)
        check(self.lib.vkhip_copy_from_host(c_void_p(dst.ptr), src.ctypes.data_as(c_void_p),
                                            src.nbytes), "copy_from_host")

    def copy_to_host(self, src: DeviceArray) -> np.ndarray:
        return src.numpy()

    def copy_device_to_device(self, copies) -> None:
        """copies: iterable of (dst DeviceArray, src DeviceArray) pairs, both
        contiguous and of equal byte size (the reference BufferCopy's bytes)."""
        cs = []
        for d, s in copies:
            if not (d.is_contiguous() and s.is_contiguous()):
                raise ValueError("copy_device_to_device: both arrays must be contiguous")
            if d.nbytes_dense() != s.nbytes_dense():
                raise ValueError(f"copy_device_to_device: {s.nbytes_dense()} source bytes for "
                                 f"{d.nbytes_dense()} destination bytes")
            cs.append(_lib.Copy(d.ptr, s.ptr, d.nbytes_dense()))
        if cs:
            check(self.lib.vkhip_copy_device_to_device((_lib.Copy * len(cs))(*cs), len(cs)),
                  "copy_device_to_device")

    def synchronize(self) -> None:
        check(self.lib.vkhip_synchronize(), "synchronize")

    def memory_stats(self) -> dict:
        """Bytes handed out by the caching allocator and bytes it holds free."""
        live, cached = c_size_t(), c_size_t()
        check(self.lib.vkhip_memory_stats(byref(live), byref(cached)), "memory_stats")
        return {"in_use": live.value, "cached": cached.value}

    def release_cached(self) -> None:
        """Returns every cached free block to HIP (synchronises)."""
        check(self.lib.vkhip_release_cached(), "release_cached")

    # -- observability (reference VulkanBackend::set_profiling /
    #    last_profile_records, vulkan_backend.h:123-198; observe::subscribe) --
    def set_profiling(self, enabled: bool) -> None:
        check(self.lib.vkhip_set_profiling(1 if enabled else 0), "set_profiling")

    def profile_records(self) -> list[dict]:
        """Drains the pending per-unit timing records (waits for their work)."""
        out = []
        buf = (_lib.ProfileRecord * 1024)()
        while True:
            n, dropped = c_size_t(), ctypes.c_uint64()
            check(self.lib.vkhip_profile_read(buf, 1024, byref(n), byref(dropped)), "profile_read")
            out += [{"label": r.label.decode(), "gpu_ms": r.gpu_ms, "dispatch": r.dispatch}
                    for r in buf[:n.value]]
            if n.value < 1024:
                return out

    def set_stream(self, stream_handle: int | None) -> None:
        """Launch on a stream the host provides (None: the backend's own);
        the current stream is synchronised first (vkhip_set_stream)."""
        check(self.lib.vkhip_set_stream(c_void_p(stream_handle or None)), "set_stream")

    def stream_handle(self) -> int:
        return self.lib.vkhip_get_stream() or 0


class DecisionRecorder:
    """Collects the backend's decision facts while active:

        with DecisionRecorder() as rec:
            ops.matmul(a, b)
        rec.decisions  # [{"site": "matmul.kernel", "chose": ..., "dispatch": ...}, ...]

    One subscriber at a time, as in the reference (observe.h:108-119)."""

    def __init__(self):
        self.decisions: list[dict] = []

        def on_decision(d, _user):
            x = d.contents
            self.decisions.append({
                "site": x.site.decode(), "op": x.op.decode(), "chose": x.chose.decode(),
                "instead_of": x.instead_of.decode(), "because": x.because.decode(),
                "required": x.required, "available": x.available, "dispatch": x.dispatch})

        self._fn = _lib.DECISION_FN(on_decision)

    def __enter__(self):
        check(backend().lib.vkhip_subscribe_decisions(self._fn, None), "subscribe_decisions")
        return self

    def __exit__(self, *exc):
        backend().lib.vkhip_subscribe_decisions(_lib.DECISION_FN(0), None)
        return False


class Event:
    """A HIP event recorded on the backend stream (launch timing)."""

    __slots__ = ("handle", "__weakref__")

    def __init__(self):
        h = c_void_p()
        check(backend().lib.vkhip_event_create(byref(h)), "event_create")
        self.handle = h.value
        weakref.finalize(self, _destroy_event, self.handle)

    def record(self) -> "Event":
        check(backend().lib.vkhip_event_record(c_void_p(self.handle)), "event_record")
        return self

    def synchronize(self) -> None:
        """Waits on the host until the recorded event has completed."""
        check(backend().lib.vkhip_event_synchronize(c_void_p(self.handle)), "event_synchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(backend().lib.vkhip_event_elapsed(c_void_p(self.handle), c_void_p(end.handle),
                                                byref(ms)), "event_elapsed")
        return float(ms.value)


def _destroy_event(handle: int) -> None:
    b = _BACKEND
    if b is not None and b.alive:
        b.lib.vkhip_event_destroy(c_void_p(handle))


_BACKEND: HipBackend | None = None


def backend(device_index: int = 0) -> HipBackend:
    """The process-wide HIP backend (created on first use; raises without a GPU)."""
    global _BACKEND
    if _BACKEND is None:
        _BACKEND = HipBackend(device_index)
    return _BACKEND


def contiguous(x: DeviceArray) -> DeviceArray:
    """A dense copy of a strided view (the reference's Contiguous op)."""
    out = DeviceArray(x.shape, x.dtype)
    node = _lib.NodeDesc()
    node.op = _lib.OP["CONTIGUOUS"]
    node.n_src = 1
    node.out = out.desc()
    node.src[0] = x.desc()
    backend().compute([node])
    return out
