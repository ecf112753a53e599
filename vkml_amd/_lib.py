"""ctypes binding of libvkhip.so, the gfx950 device backend (include/vkhip.h).

There is no fallback: if the library is missing or cannot be loaded, importing
the backend raises. Build it with ``python -m vkml_amd.build`` (or
``__graft_entry__.build()``).
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t
from ctypes import c_uint8, c_uint32, c_uint64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libvkhip.so"

# ---- status codes / dtypes / ops: include/vkhip.h ---------------------------------
OK, ERR_DEVICE, ERR_UNSUPPORTED, ERR_INVALID, ERR_OOM, ERR_NOT_INITIALISED = range(6)

F32, F16, I32, I64, BOOL = 0, 1, 2, 3, 4

REDUCE_SUM, REDUCE_MEAN, REDUCE_MAX, REDUCE_MIN, REDUCE_ARGMAX, REDUCE_ARGMIN = range(6)

GEMM_AUTO, GEMM_MFMA, GEMM_GEMV, GEMM_EXACT = 0, 1, 2, 3

NUMERICS_FAST, NUMERICS_EXACT = 0, 1

# vkml::OpKind ordinals (include/vkml/graph/op.h:30-139) for the supported subset.
OP = dict(
    FULL=2, ARANGE=3, CONTIGUOUS=11, CAST=12, ADD=14, SUB=15, MUL=16, SCALED_ADD=17, DIV=18,
    MAXIMUM=20, MINIMUM=21, EQUAL=22, LESS=23, GREATER=24, LESS_EQUAL=25, GREATER_EQUAL=26,
    NOT_EQUAL=27, NEG=28, EXP=35, LOG=36, RELU=43, SUM=47, MEAN=48, MAX=49, MIN=50, ARGMAX=52,
    ARGMIN=53, MATMUL=54, SOFTMAX=55, LOG_SOFTMAX=56, IM2COL=57, COL2IM=58, MAX_POOL2D=59,
    MAX_POOL2D_BACKWARD=60, WHERE=64,
    # backend extensions (include/vkhip.h): the fused cross-entropy rows
    CROSS_ENTROPY=96, CROSS_ENTROPY_BACKWARD=97, CONV2D=98, CONV2D_WEIGHT_GRAD=99,
    RELU_BACKWARD=100, CONV2D_WEIGHT_GRAD_SUM=101, CONV2D_INPUT_GRAD=102, CONV2D_BIAS_RELU=103, ADD_RELU=104,
    MAX_POOL2D_BACKWARD_RELU=105, MATMUL_BIAS=106, MATMUL_RELU_BACKWARD=107, CONV2D_POOL_WEIGHT_BIAS_GRAD=108,
    MAX_POOL2D_BACKWARD_RELU_BIAS=109,
)


class Operand(ctypes.Structure):
    _fields_ = [("ne", c_uint32 * 4), ("nb", c_int64 * 4)]


class Unfold(ctypes.Structure):
    _fields_ = [(n, c_int32) for n in (
        "kernel_h", "kernel_w", "stride_h", "stride_w", "pad_h", "pad_w",
        "dilation_h", "dilation_w", "image_h", "image_w")]


class TensorDesc(ctypes.Structure):
    _fields_ = [("data", c_void_p), ("dtype", c_int32), ("ndim", c_int32),
                ("ne", c_int64 * 4), ("nb", c_int64 * 4)]


class NodeDesc(ctypes.Structure):
    _fields_ = [("op", c_int32), ("n_src", c_int32), ("out", TensorDesc),
                ("src", TensorDesc * 3), ("params", c_uint8 * 64)]


class Caps(ctypes.Structure):
    _fields_ = [("name", c_char * 64), ("device_index", c_int32), ("compute_units", c_int32),
                ("wavefront_size", c_int32), ("max_threads_per_block", c_int32),
                ("max_shared_memory", c_int64), ("total_memory", c_int64),
                ("global_float_atomics", c_int32), ("asynchronous", c_int32)]


class Copy(ctypes.Structure):
    _fields_ = [("dst", c_void_p), ("src", c_void_p), ("nbytes", c_size_t)]


class SgdParam(ctypes.Structure):
    _fields_ = [("param", c_void_p), ("grad", c_void_p), ("velocity", c_void_p),
                ("n", c_uint64), ("first", c_int32), ("reserved", c_int32)]


class Decision(ctypes.Structure):
    _fields_ = [("site", c_char_p), ("op", c_char_p), ("chose", c_char_p),
                ("instead_of", c_char_p), ("because", c_char_p), ("required", c_int64),
                ("available", c_int64), ("dispatch", c_uint64)]


DECISION_FN = ctypes.CFUNCTYPE(None, POINTER(Decision), c_void_p)


class ProfileRecord(ctypes.Structure):
    _fields_ = [("label", c_char * 48), ("gpu_ms", ctypes.c_double), ("dispatch", c_uint64)]


class GemmOpts(ctypes.Structure):
    _fields_ = [("kernel", c_int32), ("split_k", c_int32)]


# Every symbol include/vkhip.h declares, with its ctypes signature.
SIGNATURES = {
    "vkhip_init": (c_int, [c_int]),
    "vkhip_shutdown": (c_int, []),
    "vkhip_last_error": (c_char_p, []),
    "vkhip_caps_get": (c_int, [POINTER(Caps)]),
    "vkhip_set_stream": (c_int, [c_void_p]),
    "vkhip_get_stream": (c_void_p, []),
    "vkhip_alloc": (c_int, [c_size_t, POINTER(c_void_p)]),
    "vkhip_free": (c_int, [c_void_p]),
    "vkhip_release_cached": (c_int, []),
    "vkhip_memory_stats": (c_int, [POINTER(c_size_t), POINTER(c_size_t)]),
    "vkhip_sgd_step": (c_int, [POINTER(SgdParam), c_size_t, c_float, c_float, c_float, c_int]),
    "vkhip_conv2d": (c_int, [c_void_p, POINTER(Operand), c_void_p, POINTER(Operand), c_void_p,
                             POINTER(Unfold)]),
    "vkhip_conv2d_weight_grad": (c_int, [c_void_p, POINTER(Operand), c_void_p, POINTER(Operand), c_void_p, POINTER(Unfold)]),
    "vkhip_conv2d_input_grad": (c_int, [c_void_p, POINTER(Operand), c_void_p, POINTER(Operand), c_void_p,
                                        POINTER(Unfold)]),
    "vkhip_conv2d_weight_grad_sum": (c_int, [c_void_p, POINTER(Operand), c_void_p, POINTER(Operand), c_void_p,
                                             POINTER(Unfold)]),
    "vkhip_im2col_offset": (c_int, [POINTER(Unfold), c_uint32, POINTER(c_int64), c_uint32, c_uint32,
                                    POINTER(c_int64)]),
    "vkhip_im2col_offset_t": (c_int, [POINTER(Unfold), c_uint32, POINTER(c_int64), c_uint32, c_uint32,
                                      POINTER(c_int64)]),
    "vkhip_kcd_slot_offset": (c_uint32, [c_uint32, c_int64, c_uint32, c_uint32, c_uint32, c_uint32]),
    "vkhip_subscribe_decisions": (c_int, [DECISION_FN, c_void_p]),
    "vkhip_set_profiling": (c_int, [c_int]),
    "vkhip_profile_read": (c_int, [POINTER(ProfileRecord), c_size_t, POINTER(c_size_t),
                                   POINTER(c_uint64)]),
    "vkhip_copy_from_host": (c_int, [c_void_p, c_void_p, c_size_t]),
    "vkhip_copy_from_host_async": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p, c_void_p]),
    "vkhip_host_alloc": (c_int, [c_size_t, POINTER(c_void_p)]),
    "vkhip_host_free": (c_int, [c_void_p]),
    "vkhip_stream_wait_event": (c_int, [c_void_p]),
    "vkhip_copy_to_host": (c_int, [c_void_p, c_void_p, c_size_t]),
    "vkhip_copy_device_to_device": (c_int, [POINTER(Copy), c_size_t]),
    "vkhip_synchronize": (c_int, []),
    "vkhip_supports": (c_int, [POINTER(NodeDesc)]),
    "vkhip_compute": (c_int, [POINTER(NodeDesc), c_size_t]),
    "vkhip_gemm": (c_int, [c_void_p, POINTER(Operand), c_void_p, POINTER(Operand), c_void_p,
                           POINTER(GemmOpts)]),
    "vkhip_gemm_noalloc": (c_int, [c_void_p, POINTER(Operand), c_void_p, POINTER(Operand),
                                   c_void_p, POINTER(GemmOpts)]),
    "vkhip_set_numerics": (c_int, [c_int]),
    "vkhip_get_numerics": (c_int, []),
    "vkhip_program_begin": (c_int, []),
    "vkhip_program_end": (c_int, [POINTER(c_void_p)]),
    "vkhip_program_run": (c_int, [c_void_p, c_int]),
    "vkhip_program_destroy": (c_int, [c_void_p]),
    "vkhip_program_info": (c_int, [c_void_p, POINTER(c_size_t), POINTER(c_size_t),
                                   POINTER(c_int)]),
    "vkhip_program_set_outputs": (c_int, [c_void_p, c_void_p, c_size_t]),
    "vkhip_program_read_outputs": (c_int, [c_void_p, c_void_p, c_size_t]),
    "vkhip_program_bind_input": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t]),
    "vkhip_program_output_order": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t, POINTER(c_size_t),
                                           POINTER(c_size_t)]),
    "vkhip_gemm_plan": (c_int, [c_uint32, c_uint32, c_uint32, c_uint32, c_int32,
                                POINTER(c_uint32), POINTER(c_uint32)]),
    "vkhip_split_k_reduce": (c_int, [c_void_p, c_void_p, c_uint64, c_uint32]),
    "vkhip_gemv": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_uint32, c_uint32]),
    "vkhip_im2col": (c_int, [c_void_p, POINTER(Operand), c_void_p, POINTER(Unfold)]),
    "vkhip_col2im": (c_int, [c_void_p, c_void_p, c_uint32, c_uint32, POINTER(Unfold)]),
    "vkhip_softmax": (c_int, [c_void_p, POINTER(Operand), c_void_p, c_int, c_int]),
    "vkhip_reduce": (c_int, [c_int, c_void_p, POINTER(Operand), c_uint32, c_void_p]),
    "vkhip_max_pool2d": (c_int, [c_void_p, c_void_p, c_uint32, c_uint32, c_uint32,
                                 POINTER(Unfold)]),
    "vkhip_max_pool2d_backward": (c_int, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32,
                                          c_uint32, POINTER(Unfold)]),
    "vkhip_scaled_add": (c_int, [c_void_p, c_void_p, c_void_p, c_uint64, c_float, c_float]),
    "vkhip_event_create": (c_int, [POINTER(c_void_p)]),
    "vkhip_event_destroy": (c_int, [c_void_p]),
    "vkhip_event_record": (c_int, [c_void_p]),
    "vkhip_event_elapsed": (c_int, [c_void_p, c_void_p, POINTER(c_float)]),
    "vkhip_event_synchronize": (c_int, [c_void_p]),
    "vkhip_fast_divide": (c_uint32, [c_uint32, c_uint32]),
    "vkhip_exact_math": (c_int, [c_void_p, c_void_p, c_size_t, c_int]),
    "vkhip_pairwise_leaf": (c_int, [c_uint32, c_uint32, POINTER(c_uint32), POINTER(c_uint32),
                                    POINTER(c_uint32)]),
}


class VkhipError(RuntimeError):
    """A failed vkhip call; `code` is the vkhip_status."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class DeviceError(VkhipError):
    pass


class NotImplementedOnDevice(VkhipError, NotImplementedError):
    pass


class OutOfMemory(VkhipError, MemoryError):
    pass


_ERRORS = {ERR_DEVICE: DeviceError, ERR_UNSUPPORTED: NotImplementedOnDevice, ERR_OOM: OutOfMemory}

_lib = None


def load() -> ctypes.CDLL:
    """Loads libvkhip.so (no device is touched). Raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"vkml_amd: {LIB_PATH} is missing -- the gfx950 backend has not been built "
            "(run `python -m vkml_amd.build`). There is no CPU fallback.")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(code: int, what: str = "") -> None:
    if code == OK:
        return
    msg = load().vkhip_last_error().decode(errors="replace")
    raise _ERRORS.get(code, VkhipError)(code, f"{what}: {msg}" if what else msg)


def operand(shape, strides) -> Operand:
    """Rank-4 right-aligned operand descriptor from extents and element strides."""
    shape, strides = list(shape), list(strides)
    if len(shape) > 4:
        raise ValueError("rank > 4 is not supported (reference kMaxDims = 4)")
    pad = 4 - len(shape)
    d = Operand()
    for i in range(4):
        d.ne[i], d.nb[i] = 1, 0
    for i, (e, s) in enumerate(zip(shape, strides)):
        d.ne[pad + i], d.nb[pad + i] = int(e), int(s)
    return d


def unfold(kernel, stride, pad, dilation, image_hw) -> Unfold:
    u = Unfold()
    u.kernel_h, u.kernel_w = kernel
    u.stride_h, u.stride_w = stride
    u.pad_h, u.pad_w = pad
    u.dilation_h, u.dilation_w = dilation
    u.image_h, u.image_w = image_hw
    return u
