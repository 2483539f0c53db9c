"""ctypes bindings for libingot_rocm.so (include/ingot_rocm.h).

The library is the product; this module only declares its C ABI for Python
callers (tests, smoke, bench). Loading fails loudly when the library has not
been built: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libingot_rocm.so")

NOALLOC_SCRATCH_BYTES = 32 << 20  # INGOT_NOALLOC_SCRATCH_BYTES
# status codes
OK, EINVAL, EDECLINED, EDEVICE, ENOMEM = 0, 1, 2, 3, 4
# dtypes (tensor/dtype.go:12-23)
DT_F32, DT_F16, DT_BF16, DT_I8, DT_U8, DT_I16, DT_I32, DT_I64, DT_BOOL = 1, 2, 3, 4, 5, 6, 7, 8, 9
PACK_I8G = 100  # INGOT_PACK_I8G: int8 weights, one f32 scale per 64 k of a row
GRAPH_FUSE_BIAS, GRAPH_FUSE_ACT, GRAPH_HALF = 1, 2, 4  # INGOT_GRAPH_* compile flags
# activations
(ACT_NONE, ACT_RELU, ACT_GELU_ERF, ACT_GELU_TANH, ACT_SIGMOID, ACT_SILU, ACT_HARDSWISH, ACT_HARDSIGMOID, ACT_CLIP,
 ACT_LEAKYRELU) = range(10)
# C broadcast modes
C_NONE, C_FULL, C_ROW, C_COL, C_SCALAR = range(5)
# math
MATH_AUTO, MATH_F32, MATH_BF16 = 0, 1, 2


class GemmArgs(C.Structure):
    _fields_ = [
        ("M", C.c_int64), ("N", C.c_int64), ("K", C.c_int64),
        ("d_a", C.c_void_p), ("a_dtype", C.c_int32), ("trans_a", C.c_int32), ("lda", C.c_int64),
        ("w", C.c_void_p),
        ("alpha", C.c_float), ("beta", C.c_float),
        ("d_c", C.c_void_p), ("c_mode", C.c_int32), ("math", C.c_int32), ("ldc", C.c_int64),
        ("act", C.c_int32), ("act_alpha", C.c_float), ("act_beta", C.c_float),
        ("post", C.c_int32), ("post_scale", C.c_float), ("post_shift", C.c_float),
        ("d_y", C.c_void_p), ("ldy", C.c_int64),
        ("batch", C.c_int64), ("stride_a", C.c_int64), ("stride_y", C.c_int64), ("y_dtype", C.c_int32),
    ]


class QconvArgs(C.Structure):
    _fields_ = [
        ("n", C.c_int64), ("c", C.c_int64), ("h", C.c_int64), ("w", C.c_int64),
        ("m", C.c_int64), ("kh", C.c_int64), ("kw", C.c_int64), ("group", C.c_int64),
        ("stride_h", C.c_int64), ("stride_w", C.c_int64), ("dilation_h", C.c_int64), ("dilation_w", C.c_int64),
        ("pad_top", C.c_int64), ("pad_left", C.c_int64), ("pad_bottom", C.c_int64), ("pad_right", C.c_int64),
        ("d_x", C.c_void_p), ("x_dtype", C.c_int32), ("zx", C.c_int32),
        ("d_mult", C.c_void_p), ("d_bias", C.c_void_p),
        ("zy", C.c_int32), ("y_dtype", C.c_int32), ("d_y", C.c_void_p),
    ]


class Tensor(C.Structure):
    _fields_ = [("dtype", C.c_int32), ("rank", C.c_int32), ("dims", C.c_int64 * 8), ("data", C.c_void_p)]


# name → (restype, argtypes); every symbol include/ingot_rocm.h declares
SIGNATURES = {
    "ingot_rocm_open": (C.c_int, [C.c_int, C.POINTER(C.c_void_p)]),
    "ingot_rocm_close": (C.c_int, [C.c_void_p]),
    "ingot_rocm_last_error": (C.c_char_p, []),
    "ingot_rocm_version": (C.c_char_p, []),
    "ingot_rocm_sync": (C.c_int, [C.c_void_p]),
    "ingot_rocm_session_workspace": (C.c_int, [C.c_void_p, C.POINTER(C.c_size_t)]),
    "ingot_rocm_stream": (C.c_int, [C.c_void_p, C.POINTER(C.c_void_p)]),
    "ingot_rocm_device_alloc": (C.c_int, [C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p)]),
    "ingot_rocm_device_free": (C.c_int, [C.c_void_p, C.c_void_p]),
    "ingot_rocm_host_alloc": (C.c_int, [C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p)]),
    "ingot_rocm_host_free": (C.c_int, [C.c_void_p, C.c_void_p]),
    "ingot_rocm_memcpy_h2d": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    "ingot_rocm_memcpy_d2h": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    "ingot_rocm_memcpy_d2d": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    "ingot_rocm_memset": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_size_t]),
    "ingot_rocm_timer_start": (C.c_int, [C.c_void_p]),
    "ingot_rocm_timer_stop": (C.c_int, [C.c_void_p, C.POINTER(C.c_float)]),
    "ingot_rocm_weight_upload": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int64, C.c_int64, C.c_int64, C.c_int,
                                           C.c_void_p, C.POINTER(C.c_void_p)]),
    "ingot_rocm_weight_pack_device": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int64, C.c_int64, C.c_int64,
                                                C.c_int, C.c_void_p, C.POINTER(C.c_void_p)]),
    "ingot_rocm_weight_free": (C.c_int, [C.c_void_p, C.c_void_p]),
    "ingot_rocm_weight_info": (C.c_int, [C.c_void_p, C.POINTER(C.c_int64), C.POINTER(C.c_int64),
                                         C.POINTER(C.c_int)]),
    "ingot_rocm_graph_create": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_void_p)]),
    "ingot_rocm_graph_bind": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(Tensor)]),
    "ingot_rocm_graph_compile": (C.c_int, [C.c_void_p, C.c_int]),
    "ingot_rocm_graph_run": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_char_p), C.POINTER(Tensor), C.c_int,
                                       C.POINTER(Tensor), C.POINTER(C.c_int)]),
    "ingot_rocm_graph_describe": (C.c_int, [C.c_void_p, C.c_int, C.c_char_p, C.c_size_t]),
    "ingot_rocm_graph_free": (C.c_int, [C.c_void_p]),
    "ingot_rocm_gemm": (C.c_int, [C.c_void_p, C.POINTER(GemmArgs)]),
    "ingot_rocm_gemm_noalloc": (C.c_int, [C.c_void_p, C.POINTER(GemmArgs)]),
    "ingot_rocm_gemm_dynamic_b": (C.c_int, [C.c_void_p, C.POINTER(GemmArgs), C.c_void_p, C.c_int32, C.c_int32,
                                            C.c_int64, C.c_int64]),
    "ingot_rocm_gemv_bf16": (C.c_int, [C.c_void_p, C.POINTER(GemmArgs)]),
    "ingot_rocm_qlinear_matmul": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_int32,
                                            C.c_int64, C.c_int32, C.c_void_p, C.c_float, C.c_int32, C.c_int32,
                                            C.c_void_p]),
    "ingot_rocm_matmul_integer": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_int32,
                                            C.c_int64, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64,
                                            C.c_int32, C.c_void_p]),
    "ingot_rocm_qlinear_conv": (C.c_int, [C.c_void_p, C.POINTER(QconvArgs), C.c_void_p]),
    "ingot_rocm_dequantize_linear": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_int64, C.c_void_p, C.c_int64,
                                               C.c_int64, C.c_void_p, C.c_int32, C.c_int64, C.c_void_p]),
    "ingot_rocm_activation": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_void_p,
                                        C.c_int32, C.c_float, C.c_float, C.c_int32, C.c_float, C.c_float]),
    "ingot_rocm_cast_bf16": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64]),
    "ingot_rocm_op_create": (C.c_int, [C.c_void_p, C.c_char_p, C.c_char_p, C.c_int, C.c_char_p,
                                       C.POINTER(C.c_void_p)]),
    "ingot_rocm_op_run": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(Tensor), C.c_int, C.POINTER(Tensor),
                                    C.POINTER(C.c_int)]),
    "ingot_rocm_op_set_const": (C.c_int, [C.c_void_p, C.c_int, C.c_int]),
    "ingot_rocm_op_free": (C.c_int, [C.c_void_p]),
    "ingot_rocm_tensor_release": (C.c_int, [C.c_void_p, C.POINTER(Tensor)]),
}

_lib = None


def load() -> C.CDLL:
    """Loads libingot_rocm.so (no fallback: a missing library is an error)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python ingot_amd/build.py` (the gfx950 library is required)")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class IngotError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def check(rc: int) -> None:
    if rc != OK:
        raise IngotError(rc, load().ingot_rocm_last_error().decode())
