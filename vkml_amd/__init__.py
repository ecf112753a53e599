"""vkml_amd -- an MI355X (gfx950) device backend for vkML's data-parallel hot path.

The kernels (fp32 MFMA GEMM with split-K and GEMV, im2col/col2im, softmax,
row/axis reductions, and the support ops a training step needs) live in
libvkhip.so behind the C ABI in include/vkhip.h. This package is the host side:
ctypes bindings (`_lib`), the `Backend`-shaped device object and strided device
arrays (`device`), and the eager op API (`ops`).

Importing the package does not touch the GPU; the first device call does, and
raises if libvkhip.so was not built. There is no CPU fallback.
"""
from . import _lib  # noqa: F401
from .device import DeviceArray, HipBackend, backend, contiguous  # noqa: F401

__all__ = ["DeviceArray", "HipBackend", "backend", "contiguous"]
