"""Python host wrapper over the C ABI: sessions, device tensors, weights, ops.

Device memory comes from the library itself (ingot_rocm_device_alloc); host
data moves as numpy arrays. Every compute call goes through libingot_rocm.so.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence

import numpy as np

from . import _lib as L

NP_OF = {
    L.DT_F32: np.float32, L.DT_F16: np.float16, L.DT_BF16: np.uint16, L.DT_I8: np.int8, L.DT_U8: np.uint8,
    L.DT_I16: np.int16, L.DT_I32: np.int32, L.DT_I64: np.int64, L.DT_BOOL: np.bool_,
}
DT_OF = {np.dtype(np.float32): L.DT_F32, np.dtype(np.float16): L.DT_F16, np.dtype(np.int8): L.DT_I8,
         np.dtype(np.uint8): L.DT_U8, np.dtype(np.int16): L.DT_I16, np.dtype(np.int32): L.DT_I32,
         np.dtype(np.int64): L.DT_I64, np.dtype(np.bool_): L.DT_BOOL}


class DeviceTensor:
    """A dense row-major tensor in device memory."""

    def __init__(self, sess: "Session", dtype: int, shape: Sequence[int], ptr: int, owned: bool, pooled: bool = False):
        self.sess, self.dtype, self.shape, self.ptr = sess, dtype, tuple(int(d) for d in shape), ptr
        self.owned, self.pooled = owned, pooled

    @property
    def numel(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    @property
    def nbytes(self) -> int:
        return self.numel * np.dtype(NP_OF[self.dtype]).itemsize

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=NP_OF[self.dtype])
        if self.nbytes:
            L.check(self.sess.lib.ingot_rocm_memcpy_d2h(self.sess.h, out.ctypes.data, self.ptr, self.nbytes))
        return out

    def as_c(self) -> L.Tensor:
        t = L.Tensor()
        t.dtype = self.dtype
        t.rank = len(self.shape)
        for i, d in enumerate(self.shape):
            t.dims[i] = d
        t.data = self.ptr
        return t

    def free(self) -> None:
        if self.ptr and self.owned:
            L.check(self.sess.lib.ingot_rocm_device_free(self.sess.h, self.ptr))
        elif self.ptr and self.pooled:
            t = self.as_c()
            L.check(self.sess.lib.ingot_rocm_tensor_release(self.sess.h, C.byref(t)))
        self.ptr = 0


class Weight:
    def __init__(self, sess: "Session", handle: int):
        self.sess, self.h = sess, handle
        n, k, dt = C.c_int64(), C.c_int64(), C.c_int()
        L.check(sess.lib.ingot_rocm_weight_info(handle, C.byref(n), C.byref(k), C.byref(dt)))
        self.n, self.k, self.pack_dtype = n.value, k.value, dt.value

    def free(self) -> None:
        if self.h:
            L.check(self.sess.lib.ingot_rocm_weight_free(self.sess.h, self.h))
            self.h = None


class Op:
    """An op built through the registry (ops.Lookup + Builder) and run like Op.Run."""

    def __init__(self, sess: "Session", op_type: str, opset: int, attrs: Optional[dict] = None, domain: str = ""):
        self.sess = sess
        text = ";".join(_attr(k, v) for k, v in (attrs or {}).items())
        h = C.c_void_p()
        L.check(sess.lib.ingot_rocm_op_create(sess.h, domain.encode(), op_type.encode(), opset, text.encode(),
                                              C.byref(h)))
        self.h = h.value

    def run(self, *inputs: Optional[DeviceTensor], max_out: int = 4) -> list:
        arr = (L.Tensor * max(1, len(inputs)))()
        for i, t in enumerate(inputs):
            if t is None:
                arr[i] = L.Tensor()
            else:
                arr[i] = t.as_c()
        outs = (L.Tensor * max_out)()
        n = C.c_int()
        L.check(self.sess.lib.ingot_rocm_op_run(self.h, len(inputs), arr, max_out, outs, C.byref(n)))
        res = []
        for i in range(n.value):
            o = outs[i]
            res.append(DeviceTensor(self.sess, o.dtype, [o.dims[d] for d in range(o.rank)], o.data, False, True))
        return res

    def set_const(self, *inputs: int) -> "Op":
        """Declares inputs constant (same storage and values every run): the op may pack them once."""
        for i in inputs:
            L.check(self.sess.lib.ingot_rocm_op_set_const(self.h, i, 1))
        return self

    def free(self) -> None:
        if self.h:
            L.check(self.sess.lib.ingot_rocm_op_free(self.h))
            self.h = None


def _attr(k: str, v) -> str:
    if isinstance(v, bool) or isinstance(v, (int, np.integer)):
        return f"i:{k}={int(v)}"
    if isinstance(v, (float, np.floating)):
        return f"f:{k}={float(v)!r}"
    if isinstance(v, (list, tuple)):
        return f"I:{k}=" + ",".join(str(int(x)) for x in v)
    return f"s:{k}={v}"


class Session:
    """One device session: stream, pool, weights (ingot_rocm_open)."""

    def __init__(self, device: int = 0):
        self.lib = L.load()
        h = C.c_void_p()
        L.check(self.lib.ingot_rocm_open(device, C.byref(h)))
        self.h = h.value

    def close(self) -> None:
        if self.h:
            L.check(self.lib.ingot_rocm_close(self.h))
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- memory ----
    def empty(self, dtype: int, shape: Sequence[int]) -> DeviceTensor:
        n = int(np.prod(shape, dtype=np.int64)) if len(shape) else 1
        nbytes = max(1, n * np.dtype(NP_OF[dtype]).itemsize)
        p = C.c_void_p()
        L.check(self.lib.ingot_rocm_device_alloc(self.h, nbytes, C.byref(p)))
        return DeviceTensor(self, dtype, shape, p.value, True)

    def to_device(self, arr: np.ndarray, dtype: Optional[int] = None) -> DeviceTensor:
        arr = np.ascontiguousarray(arr)
        dt = dtype if dtype is not None else DT_OF[arr.dtype]
        t = self.empty(dt, arr.shape)
        if arr.nbytes:
            L.check(self.lib.ingot_rocm_memcpy_h2d(self.h, t.ptr, arr.ctypes.data, arr.nbytes))
        return t

    def memset(self, t: DeviceTensor, value: int) -> None:
        L.check(self.lib.ingot_rocm_memset(self.h, t.ptr, value, t.nbytes))

    def copy_d2d(self, dst: DeviceTensor, src: DeviceTensor) -> None:
        if dst.nbytes != src.nbytes:
            raise ValueError(f"copy_d2d: {dst.nbytes} != {src.nbytes} bytes")
        L.check(self.lib.ingot_rocm_memcpy_d2d(self.h, dst.ptr, src.ptr, src.nbytes))

    def sync(self) -> None:
        L.check(self.lib.ingot_rocm_sync(self.h))

    def workspace_bytes(self) -> int:
        """Device bytes the session's growable workspace holds now (ingot_rocm_session_workspace)."""
        n = C.c_size_t()
        L.check(self.lib.ingot_rocm_session_workspace(self.h, C.byref(n)))
        return n.value

    def timer_start(self) -> None:
        L.check(self.lib.ingot_rocm_timer_start(self.h))

    def timer_stop(self) -> float:
        ms = C.c_float()
        L.check(self.lib.ingot_rocm_timer_stop(self.h, C.byref(ms)))
        return ms.value

    # ---- weights ----
    def upload_weight(self, w: np.ndarray, trans: bool, pack_dtype: int, src_dtype: Optional[int] = None) -> Weight:
        w = np.ascontiguousarray(w)
        sdt = src_dtype if src_dtype is not None else DT_OF[w.dtype]
        h = C.c_void_p()
        L.check(self.lib.ingot_rocm_weight_upload(self.h, sdt, pack_dtype, w.shape[0], w.shape[1], w.shape[1],
                                                  1 if trans else 0, w.ctypes.data, C.byref(h)))
        return Weight(self, h.value)

    # ---- kernel layer ----
    def gemm_args(self, a: DeviceTensor, w: Optional[Weight], y: DeviceTensor, M: int, **kw) -> L.GemmArgs:
        """Argument block; without a weight, N and K come from kw["n"], kw["k"]."""
        g = L.GemmArgs()
        n, k = (w.n, w.k) if w is not None else (kw["n"], kw["k"])
        g.M, g.N, g.K = M, n, k
        g.d_a, g.a_dtype = a.ptr, kw.get("a_dtype", a.dtype)
        g.trans_a = 1 if kw.get("trans_a") else 0
        g.lda = kw.get("lda", M if g.trans_a else k)
        g.w = w.h if w is not None else None
        g.alpha, g.beta = kw.get("alpha", 1.0), kw.get("beta", 0.0)
        c = kw.get("c")
        g.d_c = c.ptr if c is not None else None
        g.c_mode = kw.get("c_mode", L.C_NONE)
        g.math = kw.get("math", L.MATH_AUTO)
        g.ldc = kw.get("ldc", n)
        g.act, g.act_alpha, g.act_beta = kw.get("act", L.ACT_NONE), kw.get("act_alpha", 0.0), kw.get("act_beta", 0.0)
        g.post = 1 if kw.get("post") else 0
        g.post_scale, g.post_shift = kw.get("post_scale", 1.0), kw.get("post_shift", 0.0)
        g.d_y, g.ldy = y.ptr, kw.get("ldy", n)
        g.batch, g.stride_a, g.stride_y = kw.get("batch", 1), kw.get("stride_a", 0), kw.get("stride_y", 0)
        g.y_dtype = y.dtype
        return g

    def gemm(self, a: DeviceTensor, w: Weight, y: DeviceTensor, M: int, **kw) -> None:
        g = self.gemm_args(a, w, y, M, **kw)
        L.check(self.lib.ingot_rocm_gemm(self.h, C.byref(g)))

    def gemm_noalloc(self, a: DeviceTensor, w: Weight, y: DeviceTensor, M: int, **kw) -> None:
        """ingot_rocm_gemm_noalloc: the same product with its scratch in the fixed per-GPU array."""
        g = self.gemm_args(a, w, y, M, **kw)
        L.check(self.lib.ingot_rocm_gemm_noalloc(self.h, C.byref(g)))

    def prepare_gemm(self, a: DeviceTensor, w: Weight, y: DeviceTensor, M: int, **kw):
        """ingot_rocm_gemm with its argument block built once: a callable that
        enqueues the same product again (what a compiled session does per node)."""
        ref = C.byref(self.gemm_args(a, w, y, M, **kw))
        fn, h = self.lib.ingot_rocm_gemm, self.h

        def call() -> None:
            rc = fn(h, ref)
            if rc:
                L.check(rc)
        return call

    def gemm_dynamic_b(self, a: DeviceTensor, b: DeviceTensor, y: DeviceTensor, M: int, N: int, K: int,
                       trans_b: bool, ldb: int, stride_b: int, **kw) -> None:
        """Batched GEMM with a per-item activation B (ingot_rocm_gemm_dynamic_b)."""
        g = self.gemm_args(a, None, y, M, n=N, k=K, **kw)
        L.check(self.lib.ingot_rocm_gemm_dynamic_b(self.h, C.byref(g), b.ptr, b.dtype, 1 if trans_b else 0, ldb,
                                                   stride_b))

    def gemv_bf16(self, a: DeviceTensor, w: Weight, y: DeviceTensor, M: int, **kw) -> None:
        g = self.gemm_args(a, w, y, M, **kw)
        L.check(self.lib.ingot_rocm_gemv_bf16(self.h, C.byref(g)))

    def matmul_integer(self, a: DeviceTensor, w: Weight, M: int, za: int, y_i32: Optional[DeviceTensor] = None,
                       scale: Optional[DeviceTensor] = None, dq_zp: int = 0, y_f32: Optional[DeviceTensor] = None,
                       lda: Optional[int] = None) -> None:
        self.prepare_matmul_integer(a, w, M, za, y_i32, scale, dq_zp, y_f32, lda)()

    def prepare_matmul_integer(self, a: DeviceTensor, w: Weight, M: int, za: int,
                               y_i32: Optional[DeviceTensor] = None, scale: Optional[DeviceTensor] = None,
                               dq_zp: int = 0, y_f32: Optional[DeviceTensor] = None, lda: Optional[int] = None):
        """ingot_rocm_matmul_integer with its arguments converted once (see prepare_gemm)."""
        fn = self.lib.ingot_rocm_matmul_integer
        args = [self.h, M, w.n, w.k, a.ptr, a.dtype, lda if lda is not None else w.k, za, w.h,
                y_i32.ptr if y_i32 is not None else None, scale.ptr if scale is not None else None,
                scale.numel if scale is not None else 1, dq_zp, y_f32.ptr if y_f32 is not None else None]
        cargs = [t(v) if v is not None else None for t, v in zip(fn.argtypes, args)]

        def call() -> None:
            rc = fn(*cargs)
            if rc:
                L.check(rc)
        return call

    def qlinear_matmul(self, a: DeviceTensor, w: Weight, M: int, za: int, mult: float, zy: int, y: DeviceTensor,
                       lda: Optional[int] = None) -> None:
        """QLinearMatMul product requantised to y's dtype (u8 or s8)."""
        L.check(self.lib.ingot_rocm_qlinear_matmul(
            self.h, M, w.n, w.k, a.ptr, a.dtype, lda if lda is not None else w.k, za, w.h, mult, zy, y.dtype, y.ptr))

    def qlinear_conv(self, x: DeviceTensor, zx: int, w: Weight, wshape, mult: DeviceTensor, zy: int,
                     y: DeviceTensor, bias: Optional[DeviceTensor] = None, group: int = 1, strides=(1, 1),
                     dilations=(1, 1), pads=(0, 0, 0, 0)) -> None:
        """QLinearConv (ingot_rocm_qlinear_conv): x [N,C,H,W] u8/s8, w packed from its [M, C/group·KH·KW]
        view (upload_weight(w.reshape(M, -1), trans=True, pack_dtype=DT_I8)), wshape = (M, C/group, KH, KW),
        mult [M] f32 on the device, resolved pads (top, left, bottom, right), y [N,M,OH,OW] u8/s8."""
        a = L.QconvArgs()
        a.n, a.c, a.h, a.w = x.shape
        a.m, _, a.kh, a.kw = wshape
        a.group = group
        a.stride_h, a.stride_w = strides
        a.dilation_h, a.dilation_w = dilations
        a.pad_top, a.pad_left, a.pad_bottom, a.pad_right = pads
        a.d_x, a.x_dtype, a.zx = x.ptr, x.dtype, zx
        a.d_mult = mult.ptr
        a.d_bias = bias.ptr if bias is not None else None
        a.zy, a.y_dtype, a.d_y = zy, y.dtype, y.ptr
        L.check(self.lib.ingot_rocm_qlinear_conv(self.h, C.byref(a), w.h))

    def dequantize_linear(self, x: DeviceTensor, scale: DeviceTensor, y: DeviceTensor, inner: int = 1,
                          zp: Optional[DeviceTensor] = None) -> None:
        L.check(self.lib.ingot_rocm_dequantize_linear(
            self.h, x.ptr, x.dtype, x.numel, scale.ptr, scale.numel, inner, zp.ptr if zp is not None else None,
            zp.dtype if zp is not None else 0, zp.numel if zp is not None else 1, y.ptr))

    def activation(self, x: DeviceTensor, y: DeviceTensor, rows: int, cols: int, act: int, bias=None, a: float = 0.0,
                   b: float = 0.0) -> None:
        L.check(self.lib.ingot_rocm_activation(self.h, x.ptr, y.ptr, rows, cols, bias.ptr if bias is not None else None,
                                               act, a, b, 0, 1.0, 0.0))

    def cast_bf16(self, x: DeviceTensor, y: DeviceTensor) -> None:
        L.check(self.lib.ingot_rocm_cast_bf16(self.h, x.ptr, y.ptr, x.numel))

    def op(self, op_type: str, opset: int, attrs: Optional[dict] = None, domain: str = "") -> Op:
        return Op(self, op_type, opset, attrs, domain)


class Graph:
    """A graph session (ingot_rocm_graph_*): an ONNX node list compiled with the reference's GPU-session planning
    and run through the operator layer. Without a session it can be compiled and described, not run."""

    def __init__(self, sess: Optional[Session], text: str):
        self.sess = sess
        self.lib = sess.lib if sess is not None else L.load()
        h = C.c_void_p()
        L.check(self.lib.ingot_rocm_graph_create(sess.h if sess is not None else None, text.encode(), C.byref(h)))
        self.h = h.value

    def bind(self, name: str, t: DeviceTensor) -> None:
        c = t.as_c()
        L.check(self.lib.ingot_rocm_graph_bind(self.h, name.encode(), C.byref(c)))

    def compile(self, flags: int = 0) -> None:
        L.check(self.lib.ingot_rocm_graph_compile(self.h, flags))

    def _describe(self, what: int) -> str:
        buf = C.create_string_buffer(1 << 16)
        L.check(self.lib.ingot_rocm_graph_describe(self.h, what, buf, len(buf)))
        return buf.value.decode()

    def stats(self) -> dict:
        return {k: int(v) for k, v in (kv.split("=") for kv in self._describe(0).split(";") if kv)}

    def plan(self) -> list:
        return [ln for ln in self._describe(1).split("\n") if ln]

    def run(self, feeds: dict, max_out: int = 8) -> list:
        names = (C.c_char_p * max(1, len(feeds)))(*[n.encode() for n in feeds])
        ins = (L.Tensor * max(1, len(feeds)))(*[t.as_c() for t in feeds.values()])
        outs = (L.Tensor * max_out)()
        n = C.c_int()
        L.check(self.lib.ingot_rocm_graph_run(self.h, len(feeds), names, ins, max_out, outs, C.byref(n)))
        return [DeviceTensor(self.sess, o.dtype, [o.dims[d] for d in range(o.rank)], o.data, False, True)
                for o in outs[:n.value]]

    def free(self) -> None:
        if self.h:
            L.check(self.lib.ingot_rocm_graph_free(self.h))
            self.h = None
