"""CPU oracle of ingot's dense-contraction hot path (TEST INFRASTRUCTURE ONLY).

Loads oracle/liboracle.so (oracle.c: scalar restatements of the reference's
Go functions, each citing its file:line) and oracle/libbaseline.so
(baseline.cpp: the reference's threaded amd64 GEMM algorithm, restated in
C++, for bench.py's cpu_baseline). Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg import this package, and only as the checker.

Parity pinning: every function here is checked in tests/test_oracle.py
against the reference tests' known answers (tests/golden/kats.json) and
independent closed forms; see that file's docstring for the mapping.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F32, BF16, I8, U8, I32 = 1, 3, 4, 5, 7

_P = C.c_void_p
_I64 = C.c_int64

_orc = None
_base = None


def _load(name: str) -> C.CDLL:
    path = os.path.join(HERE, name)
    if not os.path.exists(path):
        raise RuntimeError(f"{path} missing: run `make -C oracle`")
    return C.CDLL(path)


def lib() -> C.CDLL:
    global _orc
    if _orc is None:
        L = _load("liboracle.so")
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_f32_to_bf16.argtypes = [C.c_float]
        L.orc_bf16_to_f32.restype = C.c_float
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_bf16_n.argtypes = [_P, _P, _I64]
        L.orc_act.restype = C.c_double
        L.orc_act.argtypes = [C.c_double, C.c_int, C.c_double, C.c_double]
        L.orc_gemm_ref_f32.argtypes = [_I64, _I64, _I64, C.c_float, _P, _I64, _P, _I64, C.c_float, _P, _I64]
        L.orc_gemm.restype = C.c_int
        L.orc_gemm.argtypes = [_I64, _I64, _I64, _P, _I64, C.c_int, _P, C.c_int, _I64, C.c_int, C.c_float, C.c_float,
                               _P, C.c_int, _I64, C.c_int, C.c_float, C.c_float, C.c_int, C.c_float, C.c_float, _P]
        L.orc_dot_bf16.restype = C.c_float
        L.orc_dot_bf16.argtypes = [_P, _P, _I64]
        L.orc_gemv_bf16.argtypes = [_I64, _I64, _P, _P, _I64, _P]
        L.orc_qgemm_ref.argtypes = [_I64, _I64, _I64, _P, _I64, _P, _I64, _P, _I64]
        L.orc_matmul_integer.argtypes = [_I64, _I64, _I64, _P, C.c_int, C.c_int32, _P, _P]
        L.orc_matmul_integer_shifted.argtypes = [_I64, _I64, _I64, _P, C.c_int, C.c_int32, _P, _P]
        L.orc_dequantize_linear.argtypes = [_P, C.c_int, _I64, _P, _I64, _I64, _P, C.c_int, _I64, _P]
        L.orc_quantize_i8g.argtypes = [_I64, _I64, _P, _I64, _P, _P]
        L.orc_quantize_x16.argtypes = [_I64, _P, _P, _P, _P]
        L.orc_dot_q8.argtypes = [_I64, _P, _P, _P, _P, _P]
        L.orc_dot_q8.restype = C.c_float
        L.orc_gemv_i8g.argtypes = [_I64, _I64, _I64, _P, _I64, _P, _P, C.c_float, C.c_float, _P, _P]
        L.orc_qlinear_mult.argtypes = [C.c_float, C.c_float, C.c_float]
        L.orc_qlinear_mult.restype = C.c_float
        L.orc_qlinear_requant.argtypes = [_I64, _P, C.c_float, C.c_int32, C.c_int, _P]
        L.orc_qlinear_conv.restype = _I64
        L.orc_qlinear_conv.argtypes = [_P, _P, C.c_int, C.c_int32, _P, _P, _P, C.c_int32, C.c_int, _P]
        _orc = L
    return _orc


def baseline() -> C.CDLL:
    global _base
    if _base is None:
        B = _load("libbaseline.so")
        B.base_pack_b_f32.restype = _P
        B.base_pack_b_f32.argtypes = [_I64, _I64, _P, _I64, C.c_int]
        B.base_pack_b_bf16.restype = _P
        B.base_pack_b_bf16.argtypes = [_I64, _I64, _P, _I64, C.c_int]
        B.base_free_packed.argtypes = [_P]
        B.base_sgemm_packed.argtypes = [_I64, _P, _I64, _P, _P, _I64, _P, C.c_int, C.c_int]
        B.base_gemv_bf16.argtypes = [_I64, _I64, _I64, _P, _P, _P, C.c_int]
        B.base_qgemm.argtypes = [_I64, _I64, _I64, _P, C.c_int32, _P, _P, C.c_int]
        B.base_active_kernel.restype = C.c_char_p
        B.base_active_kernel.argtypes = [C.POINTER(C.c_int)]
        _base = B
    return _base


def _p(a):
    return None if a is None else a.ctypes.data


# ---------------- restatements ----------------

def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """F32ToBF16 (kernels/gemm/bgemm.go:20-26) elementwise."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_n(_p(x), _p(y), x.size)
    return y


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint32) << 16).view(np.float32)


def act(x: float, code: int, a: float = 0.0, b: float = 0.0) -> float:
    return lib().orc_act(x, code, a, b)


def gemm_ref_f32(a, b, alpha=1.0, beta=0.0, c=None):
    """Ref (kernels/gemm/ref.go:4-18): C = alpha·A·B + beta·C, f32 accumulation."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    n = b.shape[1]
    out = np.zeros((m, n), np.float32) if c is None else np.array(c, np.float32, order="C", copy=True)
    lib().orc_gemm_ref_f32(m, n, k, alpha, _p(a), k, _p(b), n, beta, _p(out), n)
    return out


def gemm(a, b, *, trans_a=False, trans_b=False, b_dtype=F32, alpha=1.0, beta=0.0, c=None, c_mode=0, ldc=0,
         act_code=0, act_alpha=0.0, act_beta=0.0, post=False, post_scale=1.0, post_shift=0.0) -> np.ndarray:
    """The Gemm op (ops/matmul.go:27-139) + epilogue, float64 accumulation."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.uint16 if b_dtype == BF16 else np.float32)
    M, K = (a.shape[1], a.shape[0]) if trans_a else a.shape
    N = b.shape[0] if trans_b else b.shape[1]
    y = np.empty((M, N), np.float64)
    cc = None if c is None else np.ascontiguousarray(c, np.float32)
    rc = lib().orc_gemm(M, N, K, _p(a), a.shape[1], int(trans_a), _p(b), b_dtype, b.shape[1], int(trans_b), alpha,
                        beta, _p(cc), c_mode, ldc, act_code, act_alpha, act_beta, int(post), post_scale, post_shift,
                        _p(y))
    if rc:
        raise ValueError("orc_gemm: bad arguments")
    return y


def gemv_bf16(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """GemvBF16 per row (kernels/gemm/bgemm.go:201-206), sequential f32 dots."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.uint16)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), np.float32)
    for i in range(m):
        lib().orc_gemv_bf16(n, k, _p(x[i]), _p(w), k, _p(y[i]))
    return y


def qgemm_ref(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """QgemmRef (kernels/gemm/qgemm.go:173-183)."""
    a = np.ascontiguousarray(a, np.uint8)
    b = np.ascontiguousarray(b, np.int8)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.int32)
    lib().orc_qgemm_ref(m, n, k, _p(a), k, _p(b), n, _p(c), n)
    return c


def matmul_integer(a: np.ndarray, b: np.ndarray, za: int, shifted: bool = False) -> np.ndarray:
    """MatMulInteger (ops/quant.go:831-900): closed form, or the reference's u8→s8 route."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b, np.int8)
    m, k = a.shape
    n = b.shape[1]
    y = np.empty((m, n), np.int32)
    fn = lib().orc_matmul_integer_shifted if shifted else lib().orc_matmul_integer
    fn(m, n, k, _p(a), U8 if a.dtype == np.uint8 else I8, za, _p(b), _p(y))
    return y


def quantize_i8g(w: np.ndarray):
    """quantizeI8G (kernels/gemm/i8g.go:33-56): int8 q [n][k] and f32 scales [n][k/64] of an f32 [n][k] weight."""
    w = np.ascontiguousarray(w, np.float32)
    n, k = w.shape
    q = np.empty((n, k), np.int8)
    s = np.empty((n, k // 64), np.float32)
    lib().orc_quantize_i8g(n, k, _p(w), k, _p(q), _p(s))
    return q, s


def quantize_x16(x: np.ndarray):
    """vek.QuantizeX16 (kernels/vek/scalar.go:38-60): xh, xl (int8) and per-group scales of an f32 vector."""
    x = np.ascontiguousarray(x, np.float32)
    k = x.shape[0]
    xh, xl = np.empty(k, np.int8), np.empty(k, np.int8)
    sx = np.empty(k // 64, np.float32)
    lib().orc_quantize_x16(k, _p(x), _p(xh), _p(xl), _p(sx))
    return xh, xl, sx


def dot_q8(w, xh, xl, sx, sw) -> float:
    """dotQ8Ref (kernels/vek/scalar.go:20-32)."""
    w, xh, xl = (np.ascontiguousarray(v, np.int8) for v in (w, xh, xl))
    sx, sw = np.ascontiguousarray(sx, np.float32), np.ascontiguousarray(sw, np.float32)
    return float(lib().orc_dot_q8(w.size, _p(w), _p(xh), _p(xl), _p(sx), _p(sw)))


def gemv_i8g(x: np.ndarray, q: np.ndarray, s: np.ndarray, alpha: float = 1.0, beta: float = 0.0,
             c: np.ndarray = None) -> np.ndarray:
    """GemvI8G per row of x (kernels/gemm/i8g.go:70-86); c: C broadcast to [M][N]."""
    x = np.ascontiguousarray(x, np.float32)
    q, s = np.ascontiguousarray(q, np.int8), np.ascontiguousarray(s, np.float32)
    m, k = x.shape
    n = q.shape[0]
    cc = None if c is None else np.ascontiguousarray(np.broadcast_to(np.asarray(c, np.float32), (m, n)))
    y = np.empty((m, n), np.float32)
    lib().orc_gemv_i8g(m, n, k, _p(x), k, _p(q), _p(s), alpha, beta, _p(cc) if cc is not None else None, _p(y))
    return y


def qlinear_mult(sa: float, sb: float, sy: float) -> float:
    """QLinearMatMul's multiplier fl32(fl32(sa·sb)/sy) (ops/quant.go:911)."""
    return float(lib().orc_qlinear_mult(sa, sb, sy))


def qlinear_requant(v: np.ndarray, mult: float, zy: int, u8: bool) -> np.ndarray:
    """QLinearMatMul requantisation of int32 products (ops/quant.go:902-928, satU8/satI8 :26-46)."""
    v = np.ascontiguousarray(v, np.int32)
    y = np.empty(v.shape, np.uint8 if u8 else np.int8)
    lib().orc_qlinear_requant(v.size, _p(v), mult, zy, 1 if u8 else 0, _p(y))
    return y


def qlinear_matmul(a: np.ndarray, b: np.ndarray, za: int, sa: float, sb: float, sy: float, zy: int,
                   u8: bool) -> np.ndarray:
    """QLinearMatMul (ops/quant.go:791-928): MatMulInteger, then the requantisation."""
    return qlinear_requant(matmul_integer(a, b, za), qlinear_mult(sa, sb, sy), zy, u8)


def conv_out(n: int, k: int, stride: int, dil: int, pad_a: int, pad_b: int) -> int:
    """convOut (ops/conv.go:110-113); Go's division truncates toward zero."""
    num = n + pad_a + pad_b - (dil * (k - 1) + 1)
    q = abs(num) // stride
    return (q if num >= 0 else -q) + 1


def resolve_pads(auto_pad: str, pads, strides, dilations, h: int, w: int, kh: int, kw: int):
    """convOp.resolvePads (ops/conv.go:115-136): (top, left, bottom, right)."""
    pads = list(pads)
    if auto_pad in ("NOTSET", ""):
        return tuple(pads)
    if auto_pad == "VALID":
        return (0, 0, 0, 0)
    if auto_pad not in ("SAME_UPPER", "SAME_LOWER"):
        raise ValueError(f"unsupported auto_pad {auto_pad!r}")
    for d, n in enumerate((h, w)):
        k, s, dl = (kh, kw)[d], strides[d], dilations[d]
        out = (n + s - 1) // s
        total = max(0, (out - 1) * s + dl * (k - 1) + 1 - n)
        a = total // 2 if auto_pad == "SAME_UPPER" else (total + 1) // 2
        pads[d], pads[d + 2] = a, total - a
    return tuple(pads)


def qconv_mult(xs: float, ws: np.ndarray, ys: float, m: int) -> np.ndarray:
    """Per-channel requant multipliers fl32(fl32(xs·ws[m])/ys) (ops/quant.go:380-390)."""
    ws = np.asarray(ws, np.float32).reshape(-1)
    return np.array([qlinear_mult(xs, float(ws[i if ws.size > 1 else 0]), ys) for i in range(m)], np.float32)


def qlinear_conv(x: np.ndarray, zx: int, w: np.ndarray, bias, mult: np.ndarray, zy: int, u8_out: bool, group: int = 1,
                 strides=(1, 1), dilations=(1, 1), pads=(0, 0, 0, 0)) -> np.ndarray:
    """QLinearConv (ops/quant.go:343-420, im2col route :642-706, requant :449-468):
    x [N,C,H,W] u8/s8 with zero point zx, w [M,C/group,KH,KW] s8, bias [M] int32 or None,
    mult [M] f32 (qconv_mult), resolved pads (top, left, bottom, right) → y [N,M,OH,OW]."""
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w, np.int8)
    mult = np.ascontiguousarray(mult, np.float32)
    n, c, h, wd = x.shape
    m, _, kh, kw = w.shape
    oh = conv_out(h, kh, strides[0], dilations[0], pads[0], pads[2])
    ow = conv_out(wd, kw, strides[1], dilations[1], pads[1], pads[3])
    if oh < 0 or ow < 0:
        raise ValueError("invalid conv geometry")
    geom = np.array([n, c, h, wd, m, kh, kw, group, strides[0], strides[1], dilations[0], dilations[1], *pads],
                    np.int64)
    y = np.empty((n, m, oh, ow), np.uint8 if u8_out else np.int8)
    b = None if bias is None else np.ascontiguousarray(bias, np.int32)
    dt = {np.dtype(np.uint8): U8, np.dtype(np.int8): I8}[x.dtype]
    r = lib().orc_qlinear_conv(_p(geom), _p(x), dt, zx, _p(w), _p(b) if b is not None else None, _p(mult), zy,
                               1 if u8_out else 0, _p(y))
    if r < 0:
        raise ValueError("invalid conv geometry")
    return y


def dequantize_linear(x: np.ndarray, scale: np.ndarray, inner: int = 1, zp: np.ndarray = None) -> np.ndarray:
    """DequantizeLinear (ops/quant.go:173-229)."""
    x = np.ascontiguousarray(x)
    scale = np.ascontiguousarray(scale, np.float32)
    dt = {np.dtype(np.uint8): U8, np.dtype(np.int8): I8, np.dtype(np.int32): I32}[x.dtype]
    zdt = 0 if zp is None else {np.dtype(np.uint8): U8, np.dtype(np.int8): I8, np.dtype(np.int32): I32}[zp.dtype]
    y = np.empty(x.shape, np.float32)
    lib().orc_dequantize_linear(_p(x), dt, x.size, _p(scale), scale.size, inner, _p(zp), zdt,
                                1 if zp is None else zp.size, _p(y))
    return y


# ---------------- threaded CPU baseline (bench.py's cpu_baseline leg) ----------------

class PackedB:
    """A weight packed once for base_sgemm_packed (PackB / PackBBF16)."""

    def __init__(self, w: np.ndarray, trans_b: bool, bf16: bool):
        self.k, self.n = (w.shape[1], w.shape[0]) if trans_b else w.shape
        self._w = np.ascontiguousarray(w)
        fn = baseline().base_pack_b_bf16 if bf16 else baseline().base_pack_b_f32
        self.h = fn(self.k, self.n, _p(self._w), self._w.shape[1], int(trans_b))

    def __del__(self):
        if getattr(self, "h", None):
            baseline().base_free_packed(self.h)
            self.h = None


def base_sgemm(a: np.ndarray, pb: PackedB, bias=None, gelu=False, threads=1, out=None) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    m = a.shape[0]
    y = np.empty((m, pb.n), np.float32) if out is None else out
    bb = None if bias is None else np.ascontiguousarray(bias, np.float32)
    baseline().base_sgemm_packed(m, _p(a), a.shape[1], pb.h, _p(y), pb.n, _p(bb), int(gelu), threads)
    return y


def base_gemv_bf16(x: np.ndarray, w: np.ndarray, threads=1) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.uint16)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), np.float32)
    baseline().base_gemv_bf16(m, k, n, _p(x), _p(w), _p(y), threads)
    return y


def base_qgemm(a: np.ndarray, bt: np.ndarray, za: int, threads=1) -> np.ndarray:
    a = np.ascontiguousarray(a, np.uint8)
    bt = np.ascontiguousarray(bt, np.int8)
    m, k = a.shape
    n = bt.shape[0]
    y = np.empty((m, n), np.int32)
    baseline().base_qgemm(m, n, k, _p(a), za, _p(bt), _p(y), threads)
    return y


def base_active_kernel():
    """(micro-kernel name, VNNI int8 kernel in use) as the baseline's start-up probe picked them."""
    v = C.c_int()
    name = baseline().base_active_kernel(C.byref(v)).decode()
    return name, bool(v.value)
