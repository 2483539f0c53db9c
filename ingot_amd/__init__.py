"""ingot_amd — MI355X (gfx950) backend for ingot's dense-contraction hot path.

The product is the C-ABI library ``libingot_rocm.so`` (include/ingot_rocm.h):
hand-written HIP kernels for Gemm / MatMul with fused epilogues, the bf16
GEMM and decode GEMV, and int8 MatMulInteger + DequantizeLinear, behind the
reference's op interface. This package holds its sources (``csrc/``), its
build (``build.py``) and a thin Python host wrapper (``host.py``) over the
C ABI for tests and benchmarks.
"""
from ._lib import IngotError, load  # noqa: F401
from .host import DeviceTensor, Graph, Op, Session, Weight  # noqa: F401

__all__ = ["IngotError", "load", "Session", "Weight", "DeviceTensor", "Op", "Graph"]
