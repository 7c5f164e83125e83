"""ctypes binding of libqkern.so (the C ABI declared in include/qkern.h).

Loading fails loudly: there is no CPU fallback for any entry point.
"""

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqkern.so")

# qk_status
OK, INVALID_ARGUMENT, RESOURCE_EXHAUSTED, UNIMPLEMENTED, INTERNAL = 0, 3, 8, 12, 13
STATUS_NAMES = {0: "OK", 3: "INVALID_ARGUMENT", 8: "RESOURCE_EXHAUSTED",
                12: "UNIMPLEMENTED", 13: "INTERNAL"}

# qk_dtype
F32, F16, BF16, U8, S8, U32, S32 = 0, 1, 2, 3, 4, 5, 6

MAX_RANK = 6


class MatrixLayoutC(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("order", ctypes.c_int32),
                ("num_rows", ctypes.c_int64), ("num_cols", ctypes.c_int64),
                ("batch_size", ctypes.c_int64),
                ("leading_dim_stride", ctypes.c_int64),
                ("batch_stride", ctypes.c_int64),
                ("transpose", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class GemmConfigC(ctypes.Structure):
    _fields_ = [("lhs", MatrixLayoutC), ("rhs", MatrixLayoutC),
                ("c", MatrixLayoutC), ("output", MatrixLayoutC),
                ("alpha_re", ctypes.c_double), ("alpha_im", ctypes.c_double),
                ("beta", ctypes.c_double)]


class MemoryArgsC(ctypes.Structure):
    _fields_ = [("a", ctypes.c_void_p), ("a_size", ctypes.c_uint64),
                ("b", ctypes.c_void_p), ("b_size", ctypes.c_uint64),
                ("c", ctypes.c_void_p), ("c_size", ctypes.c_uint64),
                ("d", ctypes.c_void_p), ("d_size", ctypes.c_uint64),
                ("bias", ctypes.c_void_p), ("bias_size", ctypes.c_uint64),
                ("aux", ctypes.c_void_p), ("aux_size", ctypes.c_uint64)]


class BufferC(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32),
                ("rank", ctypes.c_int32),
                ("dims", ctypes.c_int64 * MAX_RANK)]


class QuantAttrsC(ctypes.Structure):
    _fields_ = [("bits", ctypes.c_int32), ("group_size", ctypes.c_int32),
                ("packing", ctypes.c_int32), ("has_bias", ctypes.c_int32)]


class AttentionAttrsC(ctypes.Structure):
    _fields_ = [("scale", ctypes.c_float), ("window", ctypes.c_int32)]


class RownormAttrsC(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("eps", ctypes.c_float),
                ("has_gain", ctypes.c_int32), ("has_beta", ctypes.c_int32)]


# Every symbol include/qkern.h declares, with its ctypes signature.
_P = ctypes.POINTER
SIGNATURES = {
    "qk_gemm_plan_create": (ctypes.c_int, [_P(GemmConfigC), ctypes.c_int32,
                                           _P(ctypes.c_void_p)]),
    "qk_gemm_execute": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p,
                                       _P(MemoryArgsC)]),
    "qk_gemm_plan_destroy": (None, [ctypes.c_void_p]),
    "qk_gemm_plan_describe": (ctypes.c_char_p, [ctypes.c_void_p]),
    "qk_qmatvec": (ctypes.c_int, [ctypes.c_void_p, _P(BufferC), _P(BufferC),
                                  _P(BufferC), _P(BufferC), _P(BufferC),
                                  _P(QuantAttrsC)]),
    "qk_embed": (ctypes.c_int, [ctypes.c_void_p, _P(BufferC), _P(BufferC),
                                _P(BufferC), _P(BufferC), _P(BufferC),
                                _P(QuantAttrsC)]),
    "qk_dequantize": (ctypes.c_int, [ctypes.c_void_p, _P(BufferC), _P(BufferC),
                                     _P(BufferC), _P(BufferC),
                                     _P(QuantAttrsC)]),
    "qk_quantize": (ctypes.c_int, [ctypes.c_void_p, _P(BufferC), _P(BufferC),
                                   _P(BufferC), _P(BufferC),
                                   _P(QuantAttrsC)]),
    "qk_rownorm": (ctypes.c_int, [ctypes.c_void_p, _P(BufferC), _P(BufferC),
                                  _P(BufferC), _P(BufferC),
                                  _P(RownormAttrsC)]),
    "qk_decode_attention_workspace_size": (
        ctypes.c_int, [_P(BufferC), _P(BufferC), _P(AttentionAttrsC),
                       _P(ctypes.c_uint64)]),
    "qk_decode_attention": (ctypes.c_int, [ctypes.c_void_p, _P(BufferC),
                                           _P(BufferC), _P(BufferC),
                                           _P(BufferC), _P(BufferC),
                                           _P(AttentionAttrsC),
                                           ctypes.c_void_p, ctypes.c_uint64]),
    "qk_decode_attention_noalloc": (ctypes.c_int, [
        ctypes.c_void_p, _P(BufferC), _P(BufferC), _P(BufferC), _P(BufferC),
        _P(BufferC), _P(AttentionAttrsC)]),
    "qk_last_error_message": (ctypes.c_char_p, []),
    "qk_device_error": (ctypes.c_int, []),
    "qk_reset_device_error": (None, []),
    "qk_version": (ctypes.c_char_p, []),
}

_lib = None


def lib():
    """The loaded library; raises if libqkern.so has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"qkern: {LIB_PATH} is missing; build it with "
                "`make -C metal-pjrt-plugin_amd` or __graft_entry__.build()")
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


class QkError(RuntimeError):
    """A failed qkern call: `status` is the qk_status code."""

    def __init__(self, status, message):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status
        self.message = message


def check(status):
    if status != OK:
        msg = lib().qk_last_error_message().decode()
        raise QkError(status, msg)
