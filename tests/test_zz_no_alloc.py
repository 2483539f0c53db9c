"""ingot_rocm_gemm_noalloc: the same products as ingot_rocm_gemm with the per-call scratch in the fixed per-GPU
array (no allocation in the call).

Each case calls the no-alloc entry point twice in a row through the C ABI, the second time with a smaller input,
and compares both results with ingot_rocm_gemm's on the same inputs. Both run the same kernels, so the results
must be bit-identical. Cases cover every scratch user: the packed bf16 activations (INGOT_MATH_BF16), the hi/lo
planes of f32 activations, the decode GEMV's x planes (M = 5..16, N < 4096) and the grouped-int8 GEMV's
quantised x; plus a product larger than the scratch array, which fails with INGOT_EINVAL. Further cases show that
a no-alloc call on a fresh session leaves the session's workspace unallocated, and that no-alloc calls issued back to
back from two sessions (two streams) run in order instead of overwriting each other's scratch.
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


@pytest.mark.parametrize("case", ["bf16_math", "bf16_hilo", "gemv_rows", "i8g"])
def test_noalloc_leaves_workspace_unused(env_session, case):
    """On a fresh session the no-alloc call takes its scratch from the fixed array: the session's growable
    workspace stays unallocated (so the call neither allocated it nor synchronised the stream to grow it), while
    the ordinary call on the same operands then allocates it."""
    announce(f"noalloc workspace {case}")
    rng = np.random.default_rng(5 + len(case))
    s = env_session()
    m, n, k = {"bf16_math": (300, 260, 900), "bf16_hilo": (300, 260, 900), "gemv_rows": (16, 1000, 2048),
               "i8g": (4, 700, 1024)}[case]
    if case == "i8g":
        w = s.upload_weight(rng.normal(0, 0.02, (n, k)).astype(np.float32), trans=True, pack_dtype=L.PACK_I8G)
    else:
        w = s.upload_weight(bf16_weights(rng, (n, k), 0.05, "normal"), trans=True, pack_dtype=L.DT_BF16,
                            src_dtype=L.DT_BF16)
    kw = {"math": L.MATH_BF16} if case == "bf16_math" else {}
    a = s.to_device(rng.normal(0, 1, (m, k)).astype(np.float32))
    y0, y1 = s.empty(L.DT_F32, (m, n)), s.empty(L.DT_F32, (m, n))
    assert s.workspace_bytes() == 0
    s.gemm_noalloc(a, w, y1, m, **kw)
    s.sync()
    assert s.workspace_bytes() == 0, "the no-alloc call used the session workspace"
    s.gemm(a, w, y0, m, **kw)
    assert s.workspace_bytes() > 0, "the ordinary call should need the workspace (the case exercises scratch)"
    assert np.array_equal(y1.numpy(), y0.numpy())
    a.free(), y0.free(), y1.free(), w.free()


def test_noalloc_calls_from_two_sessions_run_in_order(env_session):
    """Two sessions (two streams) issue no-alloc calls back to back with no host synchronisation between them:
    each call packs its own activations into the one scratch array, so the second call's pack would overwrite the
    first call's operand while the first GEMM still reads it, unless the library orders the calls. Every result
    must equal ingot_rocm_gemm's on the same inputs."""
    announce("noalloc two sessions")
    rng = np.random.default_rng(99)
    m, n, k = 4096, 4096, 4096  # 32 MiB of packed bf16 activations: the whole array
    sa, sb = env_session(), env_session()
    wt = bf16_weights(rng, (n, k), 0.05, "normal")
    wa = sa.upload_weight(wt, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
    wb = sb.upload_weight(wt, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
    xs = [rng.normal(0, 1, (m, k)).astype(np.float32) for _ in range(2)]
    da, db = sa.to_device(xs[0]), sb.to_device(xs[1])
    ya, yb = sa.empty(L.DT_F32, (m, n)), sb.empty(L.DT_F32, (m, n))
    ref_a, ref_b = sa.empty(L.DT_F32, (m, n)), sb.empty(L.DT_F32, (m, n))
    sa.gemm(da, wa, ref_a, m, math=L.MATH_BF16)
    sb.gemm(db, wb, ref_b, m, math=L.MATH_BF16)
    want_a, want_b = ref_a.numpy(), ref_b.numpy()
    for rnd in range(3):
        first, second = ((sa, da, wa, ya), (sb, db, wb, yb)) if rnd % 2 == 0 else ((sb, db, wb, yb), (sa, da, wa, ya))
        for s, d, w, y in (first, second):
            s.gemm_noalloc(d, w, y, m, math=L.MATH_BF16)
        assert np.array_equal(ya.numpy(), want_a), f"round {rnd}: session A's result was overwritten"
        assert np.array_equal(yb.numpy(), want_b), f"round {rnd}: session B's result was overwritten"
    for t in (da, db, ya, yb, ref_a, ref_b):
        t.free()
    wa.free(), wb.free()
