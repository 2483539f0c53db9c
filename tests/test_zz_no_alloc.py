"""ingot_rocm_gemm_noalloc: the same products as ingot_rocm_gemm with the per-call scratch in the fixed per-GPU
array (no allocation in the call).

Each case calls the no-alloc entry point twice in a row through the C ABI, the second time with a smaller input,
and compares both results with ingot_rocm_gemm's on the same inputs. Both run the same kernels, so the results
must be bit-identical. Cases cover every scratch user: the packed bf16 activations (INGOT_MATH_BF16), the hi/lo
planes of f32 activations, the decode GEMV's x planes (M = 5..16, N < 4096) and the grouped-int8 GEMV's
quantised x; plus a product larger than the scratch array, which fails with INGOT_EINVAL.
"""
import numpy as np
import pytest

from helpers import announce, bf16_weights
from ingot_amd import IngotError
from ingot_amd import _lib as L

pytestmark = pytest.mark.gpu


def both(sess, a, w, M, **kw):
    y0 = sess.empty(L.DT_F32, (M, w.n))
    y1 = sess.empty(L.DT_F32, (M, w.n))
    sess.gemm(a, w, y0, M, **kw)
    sess.gemm_noalloc(a, w, y1, M, **kw)
    r0, r1 = y0.numpy(), y1.numpy()
    y0.free(), y1.free()
    return r0, r1


@pytest.mark.parametrize("case", ["bf16_math", "bf16_hilo", "gemv_rows", "i8g", "f32_strided"])
def test_noalloc_matches_gemm(sess, case):
    announce(f"noalloc {case}")
    rng = np.random.default_rng(sum(map(ord, case)))
    # (M, N, K) of the first call, then a smaller second call
    shapes = {"bf16_math": [(700, 520, 1100), (33, 520, 1100)], "bf16_hilo": [(300, 260, 900), (17, 260, 900)],
              "gemv_rows": [(16, 1000, 2048), (5, 1000, 2048)], "i8g": [(4, 700, 1024), (2, 700, 1024)],
              "f32_strided": [(257, 130, 333), (40, 130, 333)]}[case]
    _, n, k = shapes[0]
    bias = sess.to_device(rng.normal(0, 0.1, n).astype(np.float32))
    if case == "i8g":
        w = sess.upload_weight(rng.normal(0, 0.02, (n, k)).astype(np.float32), trans=True, pack_dtype=L.PACK_I8G)
    elif case == "f32_strided":
        w = sess.upload_weight(rng.uniform(-1, 1, (n, k)).astype(np.float32), trans=True, pack_dtype=L.DT_F32)
    else:
        w = sess.upload_weight(bf16_weights(rng, (n, k), 0.05, "normal"), trans=True, pack_dtype=L.DT_BF16,
                               src_dtype=L.DT_BF16)
    kw = dict(beta=1.0, c=bias, c_mode=L.C_ROW, act=L.ACT_GELU_ERF)
    if case == "bf16_math":
        kw["math"] = L.MATH_BF16
    for call, (m, _, _) in enumerate(shapes):
        if case == "f32_strided":
            # A with a row pitch past K (not 16-byte aligned): packed through the scratch
            lda = k + 3
            a = sess.to_device(rng.normal(0, 1, (m, lda)).astype(np.float32))
            r0, r1 = both(sess, a, w, m, lda=lda, **kw)
        else:
            a = sess.to_device(rng.normal(0, 1, (m, k)).astype(np.float32))
            r0, r1 = both(sess, a, w, m, **kw)
        assert np.isfinite(r0).all()
        assert np.array_equal(r1, r0), f"{case} call {call} (M={m}): no-alloc result differs"
        a.free()
    w.free(), bias.free()


def test_noalloc_rejects_oversized_scratch(sess):
    """bf16 math on f32 A packs M·K bf16 values: beyond the fixed array the call fails with a clear error."""
    announce("noalloc oversized")
    rng = np.random.default_rng(8)
    k, n = 4096, 256
    m = L.NOALLOC_SCRATCH_BYTES // (2 * k) + 64
    w = sess.upload_weight(bf16_weights(rng, (n, k), 0.05, "normal"), trans=True, pack_dtype=L.DT_BF16,
                           src_dtype=L.DT_BF16)
    a = sess.empty(L.DT_F32, (m, k))
    y = sess.empty(L.DT_F32, (m, n))
    with pytest.raises(IngotError, match="fixed maximum") as e:
        sess.gemm_noalloc(a, w, y, m, math=L.MATH_BF16)
    assert e.value.code == L.EINVAL
    a.free(), y.free(), w.free()
