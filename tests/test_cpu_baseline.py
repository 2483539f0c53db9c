"""The CPU baseline (oracle/baseline.cpp, bench.py's cpu_baseline leg) computes what it claims to: the reference's
packed-B f32 / bf16-weight GEMM with bias and GELU, the bf16 GEMV and the exact int8 product, on small shapes
against numpy float64 and the integer oracle, with both micro-kernels and both int8 kernels. Test infrastructure
only (the product never runs it)."""
import math

import numpy as np
import pytest

import oracle


def test_kernel_probe_reports_a_kernel():
    name, vnni = oracle.base_active_kernel()
    assert name in ("avx2", "avx512")
    assert isinstance(vnni, bool)


@pytest.mark.parametrize("m,k,n", [(1, 7, 5), (13, 385, 33), (150, 300, 70), (6, 768, 16)])
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("threads", [1, 3])
def test_base_sgemm(m, k, n, bf16, threads):
    rng = np.random.default_rng(m * 7 + k + n)
    a = rng.normal(0, 1, (m, k)).astype(np.float32)
    w = rng.normal(0, 0.1, (n, k)).astype(np.float32)
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    wb = oracle.f32_to_bf16(w) if bf16 else w
    wide = oracle.bf16_to_f32(wb) if bf16 else w
    pb = oracle.PackedB(wb, trans_b=True, bf16=bf16)
    want = a.astype(np.float64) @ wide.astype(np.float64).T + bias
    got = oracle.base_sgemm(a, pb, bias=bias, threads=threads)
    assert np.max(np.abs(got - want)) <= 1e-5 * math.sqrt(k) * max(1.0, np.abs(want).max())
    erf = np.vectorize(math.erf)
    g = oracle.base_sgemm(a, pb, bias=bias, gelu=True, threads=threads)
    assert np.max(np.abs(g - 0.5 * want * (1 + erf(want / math.sqrt(2))))) <= 1e-4 * max(1.0, np.abs(want).max())


def test_base_gemv_bf16():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (2, 1000)).astype(np.float32)
    w = oracle.f32_to_bf16(rng.normal(0, 0.02, (300, 1000)).astype(np.float32))
    want = x.astype(np.float64) @ oracle.bf16_to_f32(w).astype(np.float64).T
    got = oracle.base_gemv_bf16(x, w, threads=4)
    assert np.max(np.abs(got - want)) <= 1e-5 * math.sqrt(1000) * np.abs(want).max()


@pytest.mark.parametrize("m,n", [(8, 12), (7, 12), (16, 64)])
def test_base_qgemm_exact(m, n):
    """m % 4 == 0 and n % 4 == 0 take the VNNI 4×4 blocks where the CPU has them; m = 7 the AVX2 rows."""
    rng = np.random.default_rng(m + n)
    k = 200
    a = rng.integers(0, 256, (m, k)).astype(np.uint8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    got = oracle.base_qgemm(a, np.ascontiguousarray(b.T), 131, threads=2)
    assert np.array_equal(got, oracle.matmul_integer(a, b, 131))


def test_worker_pool_reuse_across_widths():
    """The persistent worker pool (par_run) is reused by regions of changing width and chunk count, back to
    back: every result stays exact, and no region sees another's work."""
    rng = np.random.default_rng(11)
    a = rng.normal(0, 1, (150, 300)).astype(np.float32)
    w = rng.normal(0, 0.1, (70, 300)).astype(np.float32)
    pb = oracle.PackedB(w, trans_b=True, bf16=False)
    want = oracle.base_sgemm(a, pb, threads=1)
    q = rng.integers(0, 256, (16, 64)).astype(np.uint8)
    qb = rng.integers(-127, 128, (64, 64)).astype(np.int8)
    qwant = oracle.matmul_integer(q, qb, 7)
    for threads in [2, 8, 3, 1, 8, 5, 2, 8] * 25:
        assert np.array_equal(oracle.base_sgemm(a, pb, threads=threads), want)
        assert np.array_equal(oracle.base_qgemm(q, np.ascontiguousarray(qb.T), 7, threads=threads), qwant)
