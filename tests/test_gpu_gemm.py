"""GPU parity of the MFMA GEMM and the decode GEMV (kernel layer, C ABI).

Every case compares libingot_rocm.so with the CPU oracle (float64) on the
same seeded inputs. Bound: max-abs error <=
1e-3·sqrt(K)·max|A|·max|B| for f32, bf16 and fused-epilogue outputs. The f32
MFMA path is additionally held to the reference's own f32 tolerance
(relative 1e-5·sqrt(K), kernels/gemm/gemm_test.go:34).
Full-size configs check a sampled subset of rows against the oracle (rows
are independent) plus run-to-run bit identity.
"""
import math

import numpy as np
import pytest

import oracle
from helpers import announce, assert_close, bf16_weights, nstar_tol
from ingot_amd import IngotError
from ingot_amd import _lib as L

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1, 1), (3, 5, 7), (4, 4, 4), (37, 29, 300), (64, 33, 129), (257, 129, 33), (130, 600, 96),
          (300, 17, 1), (1, 200, 64), (200, 1, 64)]


def run_gemm(sess, a, w, M, **kw):
    y = sess.empty(L.DT_F32, (M, w.n))
    sess.gemm(a, w, y, M, **kw)
    return y.numpy()


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_gemm_f32_weights(sess, m, n, k):
    announce(f"gemm f32 m={m} n={n} k={k}")
    rng = np.random.default_rng(m * 7919 + n * 31 + k)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    bt = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    da = sess.to_device(a)
    w = sess.upload_weight(bt, trans=True, pack_dtype=L.DT_F32)
    got = run_gemm(sess, da, w, m)
    want = oracle.gemm(a, bt, trans_b=True)
    assert_close(got, want, nstar_tol(k, a, bt), f"f32 {m}x{n}x{k}")
    rel = np.max(np.abs(got - want) / np.maximum(np.abs(want), 1.0))
    assert rel <= 1e-5 * math.sqrt(k), f"f32 relative error {rel:.3e}"
    # the [K,N] source layout (MatMul / Gemm transB=0) packs to the same product
    w2 = sess.upload_weight(np.ascontiguousarray(bt.T), trans=False, pack_dtype=L.DT_F32)
    assert np.array_equal(run_gemm(sess, da, w2, m), got)
    w.free(), w2.free(), da.free()


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_gemm_bf16_weights(sess, m, n, k):
    """Default math for f32 A × bf16 W: activations as bf16 hi+lo planes (f32-class error)."""
    announce(f"gemm bf16 m={m} n={n} k={k}")
    rng = np.random.default_rng(m * 131 + n * 17 + k)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    wb = bf16_weights(rng, (n, k))
    da = sess.to_device(a)
    w = sess.upload_weight(wb, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
    got = run_gemm(sess, da, w, m)
    want = oracle.gemm(a, wb, trans_b=True, b_dtype=oracle.BF16)
    assert_close(got, want, nstar_tol(k, a, oracle.bf16_to_f32(wb)), f"bf16 {m}x{n}x{k}")
    # the reference's bf16-weight op tolerance (ops/gemm_bf16_optest_test.go:57)
    rel = np.max(np.abs(got - want) / (1 + np.abs(want)))
    assert rel <= 1e-5 * math.sqrt(k), f"bf16x2 relative error {rel:.3e}"
    w.free(), da.free()


@pytest.mark.parametrize("m,n,k", [(70, 197, 300), (1, 1000, 1300), (4, 3001, 2048), (300, 513, 2100)])
def test_bf16_pack_sources_agree(sess, m, n, k):
    """TestPackBBF16's property (kernels/gemm/packbf16_test.go:13: the bf16 pack is bit-identical whatever
    route built it, products included) for this library's pack: the same weight uploaded as f32 (rounded by
    the library, F32ToBF16 RNE) or as bf16 bits rounded on the host by the oracle, each as [N,K] (transB) or
    [K,N], gives bit-identical products in both math modes, through the GEMM and, at M <= 4, the GEMV. A
    fifth of the f32 values sit exactly halfway between two bf16 values, so the library's round-to-nearest-
    even must break ties as F32ToBF16 does."""
    announce(f"bf16 pack sources m={m} n={n} k={k}")
    rng = np.random.default_rng(m * 17 + n * 3 + k)
    w32 = rng.normal(0, 0.05, (n, k)).astype(np.float32)
    bits = w32.view(np.uint32)
    tie = rng.random((n, k)) < 0.2
    bits[tie] = (bits[tie] & np.uint32(0xFFFF0000)) | np.uint32(0x8000)
    w16 = oracle.f32_to_bf16(w32)
    ah = rng.normal(0, 1, (m, k)).astype(np.float32)
    a = sess.to_device(ah)
    uploads = [sess.upload_weight(w32, trans=True, pack_dtype=L.DT_BF16),
               sess.upload_weight(w16, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16),
               sess.upload_weight(np.ascontiguousarray(w32.T), trans=False, pack_dtype=L.DT_BF16),
               sess.upload_weight(np.ascontiguousarray(w16.T), trans=False, pack_dtype=L.DT_BF16,
                                  src_dtype=L.DT_BF16)]
    first = None
    for kw in ({}, {"math": L.MATH_BF16}):
        ys = [run_gemm(sess, a, w, m, **kw) for w in uploads]
        for i, y in enumerate(ys[1:], 1):
            assert np.array_equal(y.view(np.uint32), ys[0].view(np.uint32)), f"upload {i} differs {kw}"
        first = ys[0] if first is None else first
    # and the default-math product against the float64 oracle on the host-rounded weight
    want = oracle.gemm(ah, w16, trans_b=True, b_dtype=oracle.BF16)
    assert_close(first, want, nstar_tol(k, ah, oracle.bf16_to_f32(w16)), "bf16 pack vs oracle")
    for w in uploads:
        w.free()
    a.free()


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_gemm_bf16_math_rounds_activations(sess, m, n, k):
    """INGOT_MATH_BF16 (GPUBF16 semantics): A rounded to bf16 once; exact up to f32 accumulation."""
    announce(f"gemm bf16-math m={m} n={n} k={k}")
    rng = np.random.default_rng(m * 7 + n * 5 + k)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    wb = bf16_weights(rng, (n, k))
    w = sess.upload_weight(wb, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
    got = run_gemm(sess, sess.to_device(a), w, m, math=L.MATH_BF16)
    a16 = oracle.bf16_to_f32(oracle.f32_to_bf16(a))
    want = oracle.gemm(a16, wb, trans_b=True, b_dtype=oracle.BF16)
    rel = np.max(np.abs(got - want) / (1 + np.abs(want)))
    assert rel <= 1e-5 * math.sqrt(k), f"bf16 math relative error {rel:.3e}"
    w.free()


@pytest.mark.parametrize("mode", [L.C_FULL, L.C_ROW, L.C_COL, L.C_SCALAR])
@pytest.mark.parametrize("pack", [L.DT_F32, L.DT_BF16])
def test_gemm_alpha_beta_c_modes(sess, mode, pack):
    announce(f"gemm C mode {mode} pack {pack}")
    rng = np.random.default_rng(100 + mode * 10 + pack)
    m, n, k = 45, 70, 130
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    bt = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    c = {L.C_FULL: rng.normal(size=(m, n)), L.C_ROW: rng.normal(size=n), L.C_COL: rng.normal(size=(m, 1)),
         L.C_SCALAR: np.array([0.75])}[mode].astype(np.float32)
    w = sess.upload_weight(bt, trans=True, pack_dtype=pack)
    got = run_gemm(sess, sess.to_device(a), w, m, alpha=0.5, beta=-2.0, c=sess.to_device(c), c_mode=mode, ldc=n)
    bw = bt if pack == L.DT_F32 else oracle.bf16_to_f32(oracle.f32_to_bf16(bt))
    want = oracle.gemm(a, bw, trans_b=True, alpha=0.5, beta=-2.0, c=c, c_mode=mode, ldc=n)
    assert_close(got, want, nstar_tol(k, a, bw) + 1e-6, f"C mode {mode}")


@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (1.0, 1.0), (0.5, 0.0), (2.0, -0.5)])
@pytest.mark.parametrize("pack", [L.DT_F32, L.DT_BF16])
@pytest.mark.parametrize("m,n,k", [(1, 70, 130), (45, 70, 130), (300, 257, 515)])
def test_gemm_alpha_beta_combos(sess, alpha, beta, pack, m, n, k):
    """TestSgemmMatchesRef's α/β combinations (kernels/gemm/gemm_test.go:47) with a full C operand, held to the
    reference's f32 tolerance (relative 1e-5·sqrt(K), kernels/gemm/gemm_test.go:34) against the float64 oracle,
    on the GEMV (M = 1, bf16) and GEMM routes; β = 0 must ignore C even where it holds NaN."""
    announce(f"gemm alpha={alpha} beta={beta} pack={pack} m={m}")
    rng = np.random.default_rng(int(alpha * 10) + int((beta + 1) * 100) + pack * 7 + m)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    bt = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    c = rng.normal(size=(m, n)).astype(np.float32)
    if beta == 0.0:
        c[::3, ::5] = np.nan
    w = sess.upload_weight(bt, trans=True, pack_dtype=pack)
    got = run_gemm(sess, sess.to_device(a), w, m, alpha=alpha, beta=beta, c=sess.to_device(c), c_mode=L.C_FULL,
                   ldc=n)
    bw = bt if pack == L.DT_F32 else oracle.bf16_to_f32(oracle.f32_to_bf16(bt))
    cz = np.where(np.isnan(c), 0, c).astype(np.float32) if beta == 0.0 else c
    want = oracle.gemm(a, bw, trans_b=True, alpha=alpha, beta=beta, c=cz, c_mode=L.C_FULL, ldc=n)
    assert not np.isnan(got).any()
    rel = np.max(np.abs(got - want) / np.maximum(np.abs(want), 1.0))
    assert rel <= 1e-5 * math.sqrt(k), f"relative error {rel:.3e}"
    w.free()


@pytest.mark.parametrize("act,aa,ab", [(L.ACT_RELU, 0, 0), (L.ACT_GELU_ERF, 0, 0), (L.ACT_GELU_TANH, 0, 0),
                                       (L.ACT_SIGMOID, 0, 0), (L.ACT_SILU, 0, 0), (L.ACT_HARDSWISH, 0, 0),
                                       (L.ACT_HARDSIGMOID, 0.2, 0.5), (L.ACT_CLIP, -0.5, 0.7),
                                       (L.ACT_LEAKYRELU, 0.01, 0)])
@pytest.mark.parametrize("m", [3, 40])
def test_gemm_fused_epilogue(sess, act, aa, ab, m):
    """bias + activation + post scale/shift fused into the store (SgemmPackedBEpi / GemmEp)."""
    announce(f"epilogue act={act} m={m}")
    rng = np.random.default_rng(act * 100 + m)
    n, k = 96, 200
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    bt = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    for pack in (L.DT_F32, L.DT_BF16):
        w = sess.upload_weight(bt, trans=True, pack_dtype=pack)
        got = run_gemm(sess, sess.to_device(a), w, m, beta=1.0, c=sess.to_device(bias), c_mode=L.C_ROW, act=act,
                       act_alpha=aa, act_beta=ab, post=True, post_scale=1.5, post_shift=-0.25)
        bw = bt if pack == L.DT_F32 else oracle.bf16_to_f32(oracle.f32_to_bf16(bt))
        want = oracle.gemm(a, bw, trans_b=True, beta=1.0, c=bias, c_mode=2, act_code=act, act_alpha=aa,
                           act_beta=ab, post=True, post_scale=1.5, post_shift=-0.25)
        assert_close(got, want, 1.5 * nstar_tol(k, a, bw) + 1e-5, f"act {act} pack {pack}")
        w.free()


def test_gemm_trans_a_and_bf16_activations(sess):
    announce("gemm transA / bf16 A")
    rng = np.random.default_rng(77)
    m, n, k = 50, 66, 140
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    bt = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    w = sess.upload_weight(bt, trans=True, pack_dtype=L.DT_F32)
    got = run_gemm(sess, sess.to_device(np.ascontiguousarray(a.T)), w, m, trans_a=True, lda=m)
    assert_close(got, oracle.gemm(a, bt, trans_b=True), nstar_tol(k, a, bt), "transA f32")
    wb = sess.upload_weight(bt, trans=True, pack_dtype=L.DT_BF16)
    a16 = oracle.f32_to_bf16(a)
    got = run_gemm(sess, sess.to_device(a16, L.DT_BF16), wb, m, a_dtype=L.DT_BF16)
    want = oracle.gemm(oracle.bf16_to_f32(a16), oracle.f32_to_bf16(bt), trans_b=True, b_dtype=oracle.BF16)
    assert_close(got, want, nstar_tol(k, a, bt), "bf16 A")


def test_gemm_batched_strided(sess):
    announce("gemm batched")
    rng = np.random.default_rng(78)
    bsz, m, n, k = 3, 20, 40, 64
    a = rng.uniform(-1, 1, (bsz, m, k)).astype(np.float32)
    bt = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    w = sess.upload_weight(bt, trans=True, pack_dtype=L.DT_F32)
    y = sess.empty(L.DT_F32, (bsz, m, n))
    sess.gemm(sess.to_device(a), w, y, m, batch=bsz, stride_a=m * k, stride_y=m * n)
    got = y.numpy()
    for i in range(bsz):
        assert_close(got[i], oracle.gemm(a[i], bt, trans_b=True), nstar_tol(k, a, bt), f"batch {i}")


@pytest.mark.parametrize("trans_b", [1, 0])
@pytest.mark.parametrize("b_dt", ["f32", "bf16"])
@pytest.mark.parametrize("shared", [False, True])
def test_gemm_dynamic_b(sess, trans_b, b_dt, shared):
    """Per-item activation B (ingot_rocm_gemm_dynamic_b): Q·Kᵀ (B items [N,K]) and P·V (B items [K,N])."""
    announce(f"gemm dynamic b trans_b={trans_b} {b_dt} shared={shared}")
    rng = np.random.default_rng(3 + trans_b + 2 * shared)
    bsz, m, n, k, ldb_pad = 5, 70, 50, 37, 3
    a = rng.uniform(-1, 1, (bsz, m, k)).astype(np.float32)
    items = 1 if shared else bsz
    rows, cols = (n, k) if trans_b else (k, n)
    if b_dt == "bf16":
        bb = bf16_weights(rng, (items, rows, cols + ldb_pad), 1.0, "uniform")
        bw = oracle.bf16_to_f32(bb)
        db = sess.to_device(bb, L.DT_BF16)
    else:
        bw = rng.uniform(-1, 1, (items, rows, cols + ldb_pad)).astype(np.float32)
        db = sess.to_device(bw)
    y = sess.empty(L.DT_F32, (bsz, m, n))
    sess.gemm_dynamic_b(sess.to_device(a), db, y, m, n, k, bool(trans_b), cols + ldb_pad,
                        0 if shared else rows * (cols + ldb_pad), batch=bsz, stride_a=m * k, stride_y=m * n)
    got = y.numpy()
    for i in range(bsz):
        bi = bw[0 if shared else i][:, :cols]
        want = oracle.gemm(a[i], np.ascontiguousarray(bi), trans_b=bool(trans_b))
        assert_close(got[i], want, nstar_tol(k, a, bi), f"dynamic b item {i}")


def test_gemm_dynamic_b_decode_route(sess):
    """M <= 16, one item, bf16 B: the per-call packed B takes the GEMV route."""
    announce("gemm dynamic b gemv route")
    rng = np.random.default_rng(21)
    m, n, k = 9, 300, 640
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    wb = bf16_weights(rng, (n, k), 0.02, "normal")
    y = sess.empty(L.DT_F32, (m, n))
    sess.gemm_dynamic_b(sess.to_device(x), sess.to_device(wb, L.DT_BF16), y, m, n, k, True, k, 0)
    want = oracle.gemm(x, wb, trans_b=True, b_dtype=oracle.BF16)
    assert_close(y.numpy(), want, nstar_tol(k, x, oracle.bf16_to_f32(wb)), "dynamic b gemv")


@pytest.mark.parametrize("m", [1, 2, 3, 4, 9, 16])
@pytest.mark.parametrize("src", ["f32_nk", "bf16_nk", "f32_kn"])
@pytest.mark.parametrize("n,k", [(300, 640), (2048, 5632)])
def test_gemv_i8g_exact(sess, m, src, n, k):
    """Grouped-int8 decode GEMV (INGOT_PACK_I8G): weight quantisation, activation split, int32 group sums and the
    in-order f32 chain all equal the oracle's restatement of the reference (GemvI8G) bit for bit."""
    announce(f"i8g m={m} {src} n={n} k={k}")
    rng = np.random.default_rng(m * 7 + n + k)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    if src.startswith("bf16"):
        wb = bf16_weights(rng, (n, k), 0.02, "normal")
        wf = oracle.bf16_to_f32(wb)
        w = sess.upload_weight(wb, trans=True, pack_dtype=L.PACK_I8G, src_dtype=L.DT_BF16)
    else:
        wf = (rng.normal(0, 0.02, (n, k)) * rng.uniform(0.2, 5, (n, 1))).astype(np.float32)
        w = sess.upload_weight(wf if src == "f32_nk" else np.ascontiguousarray(wf.T), trans=src == "f32_nk",
                               pack_dtype=L.PACK_I8G)
    c = rng.normal(0, 1, n).astype(np.float32)
    y = sess.empty(L.DT_F32, (m, n))
    sess.gemm(sess.to_device(x), w, y, m, alpha=0.5, beta=2.0, c=sess.to_device(c), c_mode=L.C_ROW)
    q, sc = oracle.quantize_i8g(wf)
    want = oracle.gemv_i8g(x, q, sc, 0.5, 2.0, c)
    got = y.numpy()
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} of {got.size} differ"
    w.free()


@pytest.mark.parametrize("rows", ["1", "2", "4"])
@pytest.mark.parametrize("m", [1, 2, 4])
def test_gemv_i8g_rows_per_wave(env_session, rows, m):
    """Every rows-per-wave variant of the int8 GEMV (INGOT_I8G_ROWS), ragged N, bit-exact."""
    announce(f"i8g rows={rows} m={m}")
    sess = env_session(INGOT_I8G_ROWS=rows)
    rng = np.random.default_rng(int(rows) * 10 + m)
    n, k = 301, 1216
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    wf = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    w = sess.upload_weight(wf, trans=True, pack_dtype=L.PACK_I8G)
    y = sess.empty(L.DT_F32, (m, n))
    sess.gemm(sess.to_device(x), w, y, m)
    q, sc = oracle.quantize_i8g(wf)
    assert np.array_equal(y.numpy(), oracle.gemv_i8g(x, q, sc))
    w.free()


def test_operands_past_2gib_decline(sess):
    """Every GEMM operand is addressed with 32-bit buffer offsets, so an A operand whose extent reaches 2 GiB is
    declined (INGOT_EDECLINED: the caller runs the CPU op) before anything is launched or allocated; the buffers
    here are real and large enough, so even a launch would stay in bounds. A smaller call on them runs."""
    announce("2 GiB decline")
    k, n = 4096, 8
    m = (1 << 31) // (2 * k) + 1  # bf16 rows of 8 KiB: the extent passes 2^31 bytes
    rng = np.random.default_rng(12)
    w = sess.upload_weight(rng.normal(0, 0.02, (n, k)).astype(np.float32), trans=True, pack_dtype=L.DT_BF16)
    a = sess.empty(L.DT_BF16, (m, k))
    y = sess.empty(L.DT_F32, (m, n))
    with pytest.raises(IngotError) as e:
        sess.gemm(a, w, y, m, a_dtype=L.DT_BF16)
    assert e.value.code == L.EDECLINED and "2 GiB" in str(e.value)
    small = 1024
    sess.memset(a, 0)
    sess.gemm(a, w, y, small, a_dtype=L.DT_BF16)
    assert not y.numpy()[:small].any()
    a.free(), y.free(), w.free()


def test_gemv_i8g_declines_prefill(sess):
    """An int8 (I8G) weight serves decode only: M > 16 is declined (the caller keeps its bf16 path)."""
    announce("i8g declines")
    rng = np.random.default_rng(3)
    w = sess.upload_weight(rng.normal(0, 0.02, (64, 128)).astype(np.float32), trans=True, pack_dtype=L.PACK_I8G)
    y = sess.empty(L.DT_F32, (32, 64))
    with pytest.raises(IngotError) as e:
        sess.gemm(sess.to_device(rng.normal(0, 1, (32, 128)).astype(np.float32)), w, y, 32)
    assert e.value.code == L.EDECLINED
    with pytest.raises(IngotError, match="multiple of the group size"):
        sess.upload_weight(rng.normal(0, 0.02, (64, 100)).astype(np.float32), trans=True, pack_dtype=L.PACK_I8G)
    w.free()


@pytest.mark.parametrize("m", [1, 2, 4, 7, 16])
@pytest.mark.parametrize("n,k", [(64, 256), (200, 300), (2048, 2048), (1000, 5632), (96, 1001), (64, 7000)])
def test_gemv_bf16_decode(sess, m, n, k):
    """K = 1001 (not a multiple of 4) and K = 7000 (longer than the LDS-staged rows) take the row kernels at
    M = 2..4; the other shapes the LDS-DMA kernel."""
    announce(f"gemv m={m} n={n} k={k}")
    rng = np.random.default_rng(m * 1000 + n + k)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    wb = bf16_weights(rng, (n, k), 0.02, "normal")
    w = sess.upload_weight(wb, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
    dx = sess.to_device(x)
    y = sess.empty(L.DT_F32, (m, n))
    sess.gemv_bf16(dx, w, y, m)
    got = y.numpy()
    want = oracle.gemm(x, wb, trans_b=True, b_dtype=oracle.BF16)
    wide = oracle.bf16_to_f32(wb)
    assert_close(got, want, nstar_tol(k, x, wide), f"gemv {m}x{n}x{k}")
    # the hi/lo activation split keeps f32-level accuracy (reference f32 bound)
    rel = np.max(np.abs(got - want)) / max(1.0, np.max(np.abs(want)))
    assert rel <= 1e-5 * math.sqrt(k), f"gemv relative error {rel:.3e}"
    # deterministic split-K: a second run is bit-identical
    sess.gemv_bf16(dx, w, y, m)
    assert np.array_equal(y.numpy(), got)
    w.free()


@pytest.mark.parametrize("m", [3, 9])
def test_gemv_epilogue(sess, m):
    announce(f"gemv epilogue m={m}")
    rng = np.random.default_rng(5)
    n, k = 300, 1024
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    wb = bf16_weights(rng, (n, k), 0.02, "normal")
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    w = sess.upload_weight(wb, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
    y = sess.empty(L.DT_F32, (m, n))
    sess.gemv_bf16(sess.to_device(x), w, y, m, alpha=0.5, beta=2.0, c=sess.to_device(bias), c_mode=L.C_ROW,
                   act=L.ACT_SILU)
    want = oracle.gemm(x, wb, trans_b=True, b_dtype=oracle.BF16, alpha=0.5, beta=2.0, c=bias, c_mode=2,
                       act_code=L.ACT_SILU)
    assert_close(y.numpy(), want, nstar_tol(k, x, oracle.bf16_to_f32(wb)), "gemv epilogue")


# Every tile configuration of every GEMM kind (INGOT_GEMM_CFG), on shapes with
# ragged edges in M, N and K, with a bias and an activation in the epilogue
# (int8: the column-sum correction and fused dequantisation). Indices follow the
# configuration tables of gemm_mfma.hip.
GEMM_CFGS = {"f32": range(6), "bf16": range(10), "bf16x2": range(10), "i8": range(6)}


@pytest.mark.parametrize("kind,cfg", [(k, c) for k, r in GEMM_CFGS.items() for c in r])
@pytest.mark.parametrize("m,n,k", [(70, 197, 300), (257, 100, 1030)])
def test_gemm_forced_tile_configs(env_session, kind, cfg, m, n, k):
    announce(f"gemm forced tile kind={kind} cfg={cfg} m={m} n={n} k={k}")
    sess = env_session(INGOT_GEMM_CFG=cfg)
    rng = np.random.default_rng(cfg * 1009 + m * 7 + n + k)
    if kind == "i8":
        a = rng.integers(0, 256, (m, k)).astype(np.uint8)
        b = rng.integers(-127, 128, (k, n)).astype(np.int8)
        sc = rng.uniform(0.001, 0.01, n).astype(np.float32)
        w = sess.upload_weight(b, trans=False, pack_dtype=L.DT_I8)
        yi, yf = sess.empty(L.DT_I32, (m, n)), sess.empty(L.DT_F32, (m, n))
        sess.matmul_integer(sess.to_device(a, L.DT_U8), w, m, 131, y_i32=yi, scale=sess.to_device(sc), y_f32=yf)
        want = oracle.matmul_integer(a, b, 131)
        assert np.array_equal(yi.numpy(), want), f"int8 cfg {cfg}"
        assert np.array_equal(yf.numpy(), oracle.dequantize_linear(want, sc, inner=1)), f"int8 dequant cfg {cfg}"
        w.free()
        return
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    if kind == "f32":
        bt = rng.uniform(-1, 1, (n, k)).astype(np.float32)
        w = sess.upload_weight(bt, trans=True, pack_dtype=L.DT_F32)
        wide, kw, bdt = bt, {}, None
    else:
        bt = bf16_weights(rng, (n, k))
        w = sess.upload_weight(bt, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
        wide, bdt = oracle.bf16_to_f32(bt), oracle.BF16
        kw = {"math": L.MATH_BF16} if kind == "bf16" else {}
    ain = oracle.bf16_to_f32(oracle.f32_to_bf16(a)) if kind == "bf16" else a
    y = sess.empty(L.DT_F32, (m, n))
    sess.gemm(sess.to_device(a), w, y, m, beta=1.0, c=sess.to_device(bias), c_mode=L.C_ROW, act=L.ACT_GELU_ERF, **kw)
    want = oracle.gemm(np.ascontiguousarray(ain), bt, trans_b=True, c=bias, c_mode=L.C_ROW, beta=1.0,
                       act_code=L.ACT_GELU_ERF, **({"b_dtype": bdt} if bdt is not None else {}))
    assert_close(y.numpy(), want, nstar_tol(k, a, wide), f"{kind} cfg {cfg}")
    w.free()


@pytest.mark.parametrize("cfg", ["10", "11", "12", "13", "14", "15", "16", "17", "18", "19", "20", "21", "22",
                                 "23", "24", "25", "26", "27", "28", "29", "30", "1", "2", "3", "4", "5", "6", "7"])
@pytest.mark.parametrize("m", [1, 2, 4, 6, 9, 16])
def test_gemv_forced_configs(env_session, cfg, m):
    """Every GEMV launch configuration (INGOT_GEMV_CFG) that applies to M, strided x, both math modes."""
    rows_cfg = 10 <= int(cfg) <= 26  # VALU kernels for M <= 4
    mm = {"10": 1, "11": 1, "12": 1, "13": 4, "14": 4, "15": 2, "16": 4, "17": 4, "18": 4, "19": 2,
          "20": 1, "21": 4, "22": 4, "23": 4, "24": 2, "25": 1, "26": 4, "27": 8, "28": 8, "29": 8, "30": 8}.get(cfg, 16)
    if (rows_cfg and m > 4) or (int(cfg) < 10 and m <= 4) or m > mm:
        pytest.skip("configuration does not cover this M")
    announce(f"gemv cfg={cfg} m={m}")
    sess = env_session(INGOT_GEMV_CFG=cfg)
    rng = np.random.default_rng(int(cfg) * 31 + m)
    n, k, lda = 328, 1300, 1309
    xs = rng.normal(0, 1, (m, lda)).astype(np.float32)
    x = xs[:, :k]
    wb = bf16_weights(rng, (n, k), 0.02, "normal")
    w = sess.upload_weight(wb, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
    dx = sess.to_device(xs)
    wide = oracle.bf16_to_f32(wb)
    for math_mode in (L.MATH_AUTO, L.MATH_BF16):
        y = sess.empty(L.DT_F32, (m, n))
        sess.gemv_bf16(dx, w, y, m, lda=lda, math=math_mode)
        xin = x if math_mode == L.MATH_AUTO else oracle.bf16_to_f32(oracle.f32_to_bf16(x))
        want = oracle.gemm(np.ascontiguousarray(xin), wb, trans_b=True, b_dtype=oracle.BF16)
        assert_close(y.numpy(), want, nstar_tol(k, x, wide), f"gemv cfg {cfg} m {m} math {math_mode}")
        if math_mode == L.MATH_AUTO:
            rel = np.max(np.abs(y.numpy() - want)) / max(1.0, np.max(np.abs(want)))
            assert rel <= 1e-5 * math.sqrt(k), f"gemv cfg {cfg} relative error {rel:.3e}"
    w.free()


@pytest.mark.parametrize("wdt", ["bf16", "f32"])
@pytest.mark.parametrize("m", [1, 4, 9, 37])
def test_special_activations_follow_ieee(sess, m, wdt):
    """±Inf, NaN and near-f32-max activations, f32-class math. bf16 weights: the row GEMV (M <= 4), the hi/lo
    MFMA GEMV (M <= 16) and the hi/lo GEMM (M > 16); f32 weights: the f32 MFMA GEMM. All give the float64
    oracle's NaN and ±Inf positions and signs (an Inf activation gives ±Inf as in the reference's f32 dot,
    not the NaN of Inf − Inf in a lo term; a finite 3.4e38 stays finite, not the Inf of its bf16 rounding),
    and the finite values agree."""
    announce(f"special activations m={m} w={wdt}")
    rng = np.random.default_rng(100 + m)
    n, k = 96, 512
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    kinds = [r % 5 for r in range(m)]
    for r, kind in enumerate(kinds):
        if kind == 0:
            x[r, 7] = np.inf
        elif kind == 1:
            x[r, 3], x[r, 100] = -np.inf, np.inf  # per column ±Inf or NaN, by the two weights' signs
        elif kind == 2:
            x[r, 11] = np.nan
        elif kind == 3:
            x[r, 5] = 3.4e38
    if wdt == "bf16":
        wb = bf16_weights(rng, (n, k), 0.02, "normal")
        w = sess.upload_weight(wb, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
        kw = {"b_dtype": oracle.BF16}
    else:
        wb = rng.normal(0, 0.02, (n, k)).astype(np.float32)
        w = sess.upload_weight(wb, trans=True, pack_dtype=L.DT_F32)
        kw = {}
    y = sess.empty(L.DT_F32, (m, n))
    sess.gemm(sess.to_device(x), w, y, m)
    got = y.numpy().astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        want = np.asarray(oracle.gemm(x, wb, trans_b=True, **kw), np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(want)), "NaN positions differ"
    inf = np.isinf(want)
    assert np.array_equal(np.isinf(got), inf), "Inf positions differ"
    assert np.array_equal(np.sign(got[inf]), np.sign(want[inf])), "Inf signs differ"
    assert inf[[r for r, kd in enumerate(kinds) if kd == 0]].all()
    fin = np.isfinite(want)
    err = np.abs(got[fin] - want[fin])
    assert np.all(err <= 1e-5 * np.abs(want[fin]) + 1e-3), f"finite values: max err {err.max():.3e}"
    w.free()


# ---------------- BASELINE configs at full size ----------------

def test_config1_gemm_relu(sess):
    """Y = ReLU(A·Bᵀ + bias), f32, A[128,256], B[512,256], transB."""
    announce("config 1")
    rng = np.random.default_rng(1)
    a = rng.uniform(-1, 1, (128, 256)).astype(np.float32)
    b = rng.uniform(-1, 1, (512, 256)).astype(np.float32)
    bias = rng.normal(0, 0.1, 512).astype(np.float32)
    w = sess.upload_weight(b, trans=True, pack_dtype=L.DT_F32)
    got = run_gemm(sess, sess.to_device(a), w, 128, beta=1.0, c=sess.to_device(bias), c_mode=L.C_ROW,
                   act=L.ACT_RELU)
    want = oracle.gemm(a, b, trans_b=True, beta=1.0, c=bias, c_mode=2, act_code=1)
    assert_close(got, want, nstar_tol(256, a, b), "config 1")


BERT = [(768, 2304, 0), (768, 768, 0), (768, 3072, L.ACT_GELU_ERF), (3072, 768, 0)]


@pytest.mark.parametrize("k,n,act", BERT)
def test_config2_bert_f32(sess, k, n, act):
    """BERT-base projections, M=1024, W [K,N] f32 (MatMul layout) + bias (+GELU)."""
    announce(f"bert k={k} n={n}")
    rng = np.random.default_rng(k + n)
    a = rng.normal(0, 1, (1024, k)).astype(np.float32)
    wkn = rng.normal(0, 0.02, (k, n)).astype(np.float32)
    bias = rng.normal(0, 0.02, n).astype(np.float32)
    w = sess.upload_weight(wkn, trans=False, pack_dtype=L.DT_F32)
    got = run_gemm(sess, sess.to_device(a), w, 1024, beta=1.0, c=sess.to_device(bias), c_mode=L.C_ROW, act=act)
    rows = np.arange(0, 1024, 37)
    want = oracle.gemm(a[rows], wkn, beta=1.0, c=bias, c_mode=2, act_code=act)
    assert_close(got[rows], want, nstar_tol(k, a, wkn), f"bert {k}x{n}")


@pytest.mark.parametrize("k,n,act", [(3072, 9216, 0), (3072, 12288, L.ACT_GELU_ERF), (12288, 3072, 0)])
def test_config5_dit_bf16(sess, k, n, act):
    """DiT GEMMs, M=4096, A f32 → bf16 RNE on load (INGOT_MATH_BF16, the benched path),
    W bf16 [N,K], f32 accumulate; north-star bound against the f32-A oracle."""
    announce(f"dit k={k} n={n}")
    rng = np.random.default_rng(k * 3 + n)
    a = rng.normal(0, 1, (4096, k)).astype(np.float32)
    wb = bf16_weights(rng, (n, k), 0.02, "normal")
    w = sess.upload_weight(wb, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
    da = sess.to_device(a)
    got = run_gemm(sess, da, w, 4096, act=act, math=L.MATH_BF16)
    # 256 rows covering every residue mod 256: every wave row and every 16-row MFMA block of every tile
    rows = (np.arange(256) * 17 + 5) % 4096
    assert len(set(rows % 256)) == 256
    want = oracle.gemm(a[rows], wb, trans_b=True, b_dtype=oracle.BF16, act_code=act)
    assert_close(got[rows], want, nstar_tol(k, a, oracle.bf16_to_f32(wb)), f"dit {k}x{n}")
    assert np.array_equal(run_gemm(sess, da, w, 4096, act=act, math=L.MATH_BF16), got), "run-to-run bit identity"
    # default math (bf16 hi+lo activations) on the same inputs
    got2 = run_gemm(sess, da, w, 4096, act=act)
    assert_close(got2[rows], want, 1e-5 * math.sqrt(k) * (1 + np.abs(want).max()), f"dit x2 {k}x{n}")
    w.free(), da.free()


@pytest.mark.parametrize("m", [1, 4, 16])
@pytest.mark.parametrize("k,n", [(2048, 6144), (2048, 2048), (2048, 11264), (5632, 2048)])
def test_config4_decode_gemv(sess, m, k, n):
    """Llama-style decode, bf16 weights, M in {1,4,16} (M <= 4, and M = 16 with N < 4096, run the
    GEMV; M = 16 with N >= 4096 the hi/lo GEMM)."""
    announce(f"decode m={m} k={k} n={n}")
    rng = np.random.default_rng(m + k + n)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    wb = bf16_weights(rng, (n, k), 0.02, "normal")
    w = sess.upload_weight(wb, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
    got = run_gemm(sess, sess.to_device(x), w, m)
    want = oracle.gemm(x, wb, trans_b=True, b_dtype=oracle.BF16)
    assert_close(got, want, nstar_tol(k, x, oracle.bf16_to_f32(wb)), f"decode {m}x{k}x{n}")
    w.free()


@pytest.mark.parametrize("m", [5, 9, 16])
@pytest.mark.parametrize("n", [4095, 4096, 6144])
def test_decode_rows_gemm_route(sess, m, n):
    """M = 5..16 rows of f32 A against bf16 weights: N < 4096 runs the GEMV, N >= 4096 the hi/lo GEMM of
    four-stage 32x32 tiles. Both sides of the boundary with a per-column bias, GELU, and f32 and bf16 Y; f32 Y
    is held to the reference's bf16-weight bound (relative 1e-5·sqrt(K), ops/gemm_bf16_optest_test.go:57)
    against the float64 oracle, bf16 Y additionally to one bf16 rounding of the result."""
    announce(f"decode rows route m={m} n={n}")
    k = 2048
    rng = np.random.default_rng(m * 10007 + n)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    wb = bf16_weights(rng, (n, k), 0.02, "normal")
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    w = sess.upload_weight(wb, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
    dx, db = sess.to_device(x), sess.to_device(bias)
    want = oracle.gemm(x, wb, trans_b=True, b_dtype=oracle.BF16, beta=1.0, c=bias, c_mode=L.C_ROW,
                       act_code=L.ACT_GELU_ERF)
    y = sess.empty(L.DT_F32, (m, n))
    sess.gemm(dx, w, y, m, beta=1.0, c=db, c_mode=L.C_ROW, act=L.ACT_GELU_ERF)
    got = y.numpy()
    rel = np.max(np.abs(got - want) / (1 + np.abs(want)))
    assert rel <= 1e-5 * math.sqrt(k), f"f32 Y relative error {rel:.3e}"
    yb = sess.empty(L.DT_BF16, (m, n))
    sess.gemm(dx, w, yb, m, beta=1.0, c=db, c_mode=L.C_ROW, act=L.ACT_GELU_ERF)
    gotb = oracle.bf16_to_f32(yb.numpy())
    relb = np.max(np.abs(gotb - want) / (1 + np.abs(want)))
    assert relb <= 2.0 ** -8 + 1e-5 * math.sqrt(k), f"bf16 Y relative error {relb:.3e}"
    # the bf16 store is the RNE rounding of the f32 result of the same route
    assert np.array_equal(yb.numpy(), oracle.f32_to_bf16(got))
    w.free()


SENTINEL = np.float32(1e9)


def dirty_rows(sess, m, n, ldy, dtype=L.DT_F32):
    """A destination of m rows of pitch ldy (>= n), every element set to SENTINEL (bf16: its bf16 bits)."""
    host = np.full((m, ldy), SENTINEL, np.float32)
    if dtype == L.DT_BF16:
        host = oracle.f32_to_bf16(host)
    return sess.to_device(host, dtype), host


def check_padded(got_full, want, n, tol, what, sentinel_bits=None):
    """The first n columns match the oracle; columns n..ldy keep the sentinel."""
    assert_close(got_full[:, :n], want, tol, what)
    pad = got_full[:, n:]
    if sentinel_bits is None:
        assert np.all(pad == SENTINEL), f"{what}: row padding written"
    else:
        assert np.all(pad == sentinel_bits), f"{what}: row padding written"


@pytest.mark.parametrize("pad", [3, 4])
@pytest.mark.parametrize("route", ["f32", "bf16", "bf16x2", "gemv_m2", "gemv_m3", "gemv_m6", "gemv_m9", "gemm_m9",
                                   "bf16_y", "gemv_m6_bf16_y"])
def test_dirty_padded_destination(sess, route, pad):
    """The destination starts dirty (1e9 everywhere, as kernels/metal/gemmep_test.go:45-47) with row pitch
    ldy = N + pad: every output is overwritten and the padding past N stays untouched
    (kernels/metal/gemmep_test.go:22-96, kernels/metal/gemm_test.go:14,45). pad = 3 makes the pitch unaligned
    (scalar stores), pad = 4 keeps 16-byte rows (vector stores). The GEMV routes: M = 2, 3 and 6 the LDS-DMA
    kernel, M = 9 the MFMA kernel."""
    announce(f"dirty padded destination route={route} pad={pad}")
    rng = np.random.default_rng(len(route) * 101 + pad)
    m, n, k = {"gemv_m2": (2, 300, 640), "gemv_m3": (3, 300, 640), "gemv_m6": (6, 300, 640), "gemv_m9": (9, 300, 640),
               "gemm_m9": (9, 4100, 512), "gemv_m6_bf16_y": (6, 300, 640)}.get(route, (70, 197, 300))
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    kw = dict(beta=1.0, c=sess.to_device(bias), c_mode=L.C_ROW, act=L.ACT_GELU_ERF)
    ldy = n + pad
    if route == "f32":
        bt = rng.uniform(-1, 1, (n, k)).astype(np.float32)
        w = sess.upload_weight(bt, trans=True, pack_dtype=L.DT_F32)
        wide, okw = bt, {}
    else:
        bt = bf16_weights(rng, (n, k))
        w = sess.upload_weight(bt, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
        wide, okw = oracle.bf16_to_f32(bt), {"b_dtype": oracle.BF16}
        if route == "bf16":
            kw["math"] = L.MATH_BF16
    ain = oracle.bf16_to_f32(oracle.f32_to_bf16(a)) if route == "bf16" else a
    want = oracle.gemm(np.ascontiguousarray(ain), bt, trans_b=True, c=bias, c_mode=L.C_ROW, beta=1.0,
                       act_code=L.ACT_GELU_ERF, **okw)
    tol = nstar_tol(k, a, wide)
    if route.endswith("bf16_y"):
        y, host = dirty_rows(sess, m, n, ldy, L.DT_BF16)
        sess.gemm(sess.to_device(a), w, y, m, ldy=ldy, **kw)
        got = y.numpy()
        assert np.array_equal(got[:, n:], host[:, n:]), "bf16 Y: row padding written"
        assert_close(oracle.bf16_to_f32(got[:, :n]), want, tol + 2.0 ** -8 * np.abs(want).max(), "bf16 Y")
    else:
        y, _ = dirty_rows(sess, m, n, ldy)
        sess.gemm(sess.to_device(a), w, y, m, ldy=ldy, **kw)
        check_padded(y.numpy(), want, n, tol, route)
    w.free()


def test_dirty_destination_int8(sess):
    """MatMulInteger + fused dequant into dirty outputs (1e9 / 0x7f7f7f7f) followed by guard elements: every
    output overwritten (bit-exact), the guard elements past M·N untouched."""
    announce("dirty destination int8")
    rng = np.random.default_rng(99)
    m, n, k = 70, 197, 300
    a = rng.integers(0, 256, (m, k)).astype(np.uint8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    sc = rng.uniform(0.001, 0.01, n).astype(np.float32)
    w = sess.upload_weight(b, trans=False, pack_dtype=L.DT_I8)
    guard = 37
    yi = sess.to_device(np.full(m * n + guard, 0x7F7F7F7F, np.int32))
    yf = sess.to_device(np.full(m * n + guard, SENTINEL, np.float32))
    sess.matmul_integer(sess.to_device(a, L.DT_U8), w, m, 128, y_i32=yi, scale=sess.to_device(sc), y_f32=yf)
    want = oracle.matmul_integer(a, b, 128)
    gi, gf = yi.numpy(), yf.numpy()
    assert np.array_equal(gi[:m * n].reshape(m, n), want)
    assert np.array_equal(gf[:m * n].reshape(m, n), oracle.dequantize_linear(want, sc, inner=1))
    assert np.all(gi[m * n:] == 0x7F7F7F7F) and np.all(gf[m * n:] == SENTINEL)
    w.free()


def test_m_invariance(sess):
    """Rows are bit-identical whatever M is (kernels/gemm/minvariance_test.go:21), where the same kernel kind runs:
    every GEMM tile configuration of one kind reduces K in the same order (k-tile after k-tile, the same MFMA per
    16-byte k chunk), so the tile choice, which follows M, does not change a row. f32 weights: every M (f32
    weights never take the GEMV). bf16 weights with f32 A: every M >= 17, and M = 5..16 when N >= 4096 (the same
    hi/lo GEMM); the decode GEMV (M <= 4, and M = 5..16 with N < 4096) sums in another order, like the
    reference's exempt M = 1 GEMV. int8 is exact, hence invariant."""
    announce("m invariance")
    rng = np.random.default_rng(2024)
    k = 1100
    a = rng.normal(0, 1, (600, k)).astype(np.float32)
    da = sess.to_device(a)

    def rows_of(w, n, M, **kw):
        y = sess.empty(L.DT_F32, (M, n))
        sess.gemm(da, w, y, M, **kw)
        return y.numpy()

    n = 4200
    wf = sess.upload_weight(rng.normal(0, 0.05, (n, k)).astype(np.float32), trans=True, pack_dtype=L.DT_F32)
    full = rows_of(wf, n, 600)
    for M in (1, 3, 16, 33, 129, 257):
        assert np.array_equal(rows_of(wf, n, M), full[:M]), f"f32 weights M={M}"
    wb = sess.upload_weight(bf16_weights(rng, (n, k), 0.05, "normal"), trans=True, pack_dtype=L.DT_BF16,
                            src_dtype=L.DT_BF16)
    for kw in ({}, {"math": L.MATH_BF16}):
        full = rows_of(wb, n, 600, **kw)
        for M in (5, 9, 16, 17, 40, 129, 300):
            assert np.array_equal(rows_of(wb, n, M, **kw), full[:M]), f"bf16 weights M={M} {kw}"
    wf.free(), wb.free(), da.free()


def test_deep_prefetch_tile_m_invariant(env_session):
    """The 256×192 tile with the weight staged through registers (taken for products whose operands are too large
    to stay in the Infinity Cache) reduces K in the tile kinds' common order: its rows are bit-identical to the rows
    the other tiles give at smaller M, for bf16 A and for the hi/lo split, K over several k-tiles and ragged."""
    announce("deep-prefetch tile m invariance")
    rng = np.random.default_rng(77)
    m, n, k = 600, 1000, 1333
    a = rng.normal(0, 1, (m, k)).astype(np.float32)
    wt = bf16_weights(rng, (n, k), 0.05, "normal")
    deep, plain = env_session(INGOT_GEMM_CFG=9), env_session(INGOT_GEMM_CFG=-1)
    for kw in ({}, {"math": L.MATH_BF16}):
        rows = {}
        for name, s, M in (("deep", deep, m), ("plain", plain, 17), ("plain", plain, 300)):
            w = s.upload_weight(wt, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
            y = s.empty(L.DT_F32, (M, n))
            s.gemm(s.to_device(a[:M]), w, y, M, **kw)
            rows[(name, M)] = y.numpy()
            w.free()
        for M in (17, 300):
            assert np.array_equal(rows[("plain", M)], rows[("deep", m)][:M]), f"deep tile rows differ at M={M} {kw}"


@pytest.mark.parametrize("k", [1, 33, 64, 65, 128, 200])
def test_deep_prefetch_tile_short_and_batched(env_session, k):
    """The register-staged 256×192 tile forced (INGOT_GEMM_CFG=9) where its pipeline runs out early: K of one
    k-tile or less (the loads of k-tiles 1..3 are past the end from the start), K of one and two k-tiles exactly
    and ragged; bf16 A and the hi/lo split (two virtual k-tiles per k-tile), a bias and GELU in the epilogue,
    ragged M and N; and a batched per-item B (ingot_rocm_gemm_dynamic_b) whose items the grid's y index selects."""
    announce(f"deep-prefetch tile short k={k}")
    sess = env_session(INGOT_GEMM_CFG=9)
    rng = np.random.default_rng(1000 + k)
    m, n = 300, 250
    a = rng.normal(0, 1, (m, k)).astype(np.float32)
    bt = bf16_weights(rng, (n, k), 0.05, "normal")
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    w = sess.upload_weight(bt, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
    wide = oracle.bf16_to_f32(bt)
    for kind, kw in (("bf16", {"math": L.MATH_BF16}), ("hilo", {})):
        ain = oracle.bf16_to_f32(oracle.f32_to_bf16(a)) if kind == "bf16" else a
        y = sess.empty(L.DT_F32, (m, n))
        sess.gemm(sess.to_device(a), w, y, m, beta=1.0, c=sess.to_device(bias), c_mode=L.C_ROW, act=L.ACT_GELU_ERF,
                  **kw)
        want = oracle.gemm(np.ascontiguousarray(ain), bt, trans_b=True, b_dtype=oracle.BF16, c=bias, c_mode=L.C_ROW,
                           beta=1.0, act_code=L.ACT_GELU_ERF)
        assert_close(y.numpy(), want, nstar_tol(k, a, wide), f"deep tile {kind} k={k}")
    w.free()
    bsz = 3
    ab = rng.normal(0, 1, (bsz, m, k)).astype(np.float32)
    bb = bf16_weights(rng, (bsz, n, k), 0.05, "normal")
    y = sess.empty(L.DT_F32, (bsz, m, n))
    sess.gemm_dynamic_b(sess.to_device(ab), sess.to_device(bb, L.DT_BF16), y, m, n, k, True, k, n * k, batch=bsz,
                        stride_a=m * k, stride_y=m * n, math=L.MATH_BF16)
    got = y.numpy()
    for i in range(bsz):
        ain = oracle.bf16_to_f32(oracle.f32_to_bf16(ab[i]))
        want = oracle.gemm(np.ascontiguousarray(ain), bb[i], trans_b=True, b_dtype=oracle.BF16)
        assert_close(got[i], want, nstar_tol(k, ab, oracle.bf16_to_f32(bb[i])), f"deep tile batched item {i}")


@pytest.mark.parametrize("seed", range(32))
def test_random_products_against_oracle(sess, seed):
    """Seeded random products through ingot_rocm_gemm against the float64 oracle: shapes from 1 to a few hundred
    rows (so the decode GEMV, the small-tile and the large-tile GEMMs all take part), f32 or bf16 weights in either
    source layout, the default and the bf16 math, transposed A (f32 weights), every C mode with random α and β,
    every activation, the post scale and shift, a Y pitch wider than N and bf16 Y. Bound: the north-star max-abs
    bound scaled by |α|, the activation's slope (at most 2) and the post scale, plus bf16 Y's rounding."""
    rng = np.random.default_rng(9000 + seed)

    def dim(lo, hi):
        return int(np.exp(rng.uniform(np.log(lo), np.log(hi + 1))))

    m, n, k = dim(1, 600), dim(16, 1500), dim(24, 2100)
    wdt = ["f32", "bf16"][rng.integers(2)]
    math_mode = L.MATH_BF16 if wdt == "bf16" and rng.integers(3) == 0 else L.MATH_AUTO
    trans_a = wdt == "f32" and bool(rng.integers(2))
    src_kn = bool(rng.integers(2))
    c_mode = int(rng.integers(5))
    act = int(rng.integers(10))
    aa, ab = {L.ACT_HARDSIGMOID: (0.2, 0.5), L.ACT_CLIP: (-0.4, 0.6), L.ACT_LEAKYRELU: (0.03, 0.0)}.get(act, (0.0, 0.0))
    alpha = float(rng.choice([1.0, 0.5, -1.25]))
    beta = float(rng.choice([0.0, 1.0, -0.75])) if c_mode else 0.0
    post = bool(rng.integers(2))
    ps, pt = (1.5, -0.25) if post else (1.0, 0.0)
    ybf16 = bool(rng.integers(4) == 0)
    ldy = n + int(rng.choice([0, 0, 4, 5]))
    announce(f"random product seed={seed} m={m} n={n} k={k} w={wdt} math={math_mode} transA={trans_a} "
             f"c_mode={c_mode} act={act} ybf16={ybf16} ldy={ldy}")
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    bt = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    if wdt == "bf16":
        bt = oracle.bf16_to_f32(oracle.f32_to_bf16(bt))
    src = np.ascontiguousarray(bt.T) if src_kn else bt
    w = sess.upload_weight(src, trans=not src_kn, pack_dtype=L.DT_F32 if wdt == "f32" else L.DT_BF16)
    c = {L.C_FULL: rng.normal(0, 1, (m, n)), L.C_ROW: rng.normal(0, 1, n), L.C_COL: rng.normal(0, 1, m),
         L.C_SCALAR: rng.normal(0, 1, 1)}.get(c_mode)
    c = None if c is None else c.astype(np.float32)
    da = sess.to_device(np.ascontiguousarray(a.T) if trans_a else a)
    y = sess.empty(L.DT_BF16 if ybf16 else L.DT_F32, (m, ldy))
    kw = dict(trans_a=trans_a, alpha=alpha, beta=beta, act=act, act_alpha=aa, act_beta=ab, post=post,
              post_scale=ps, post_shift=pt, ldy=ldy, math=math_mode)
    if c is not None:
        kw.update(c=sess.to_device(c), c_mode=c_mode)
    sess.gemm(da, w, y, m, **kw)
    got = y.numpy()[:, :n]
    got = oracle.bf16_to_f32(got) if ybf16 else got
    ain = oracle.bf16_to_f32(oracle.f32_to_bf16(a)) if math_mode == L.MATH_BF16 else a
    want = oracle.gemm(ain, bt, trans_b=True, alpha=alpha, beta=beta, c=c, c_mode=c_mode if c is not None else 0,
                       ldc=n if c_mode == L.C_FULL else 0, act_code=act, act_alpha=aa, act_beta=ab, post=post,
                       post_scale=ps, post_shift=pt)
    tol = 2.0 * abs(alpha) * ps * nstar_tol(k, a, bt) + 1e-5
    if ybf16:
        tol += float(np.max(np.abs(want))) * 2.0 ** -8
    assert_close(got, want, tol, f"random product seed {seed}")
    w.free()


@pytest.mark.parametrize("n,k", [(2048, 2048), (6144, 2048), (2048, 5632), (1000, 1300)])
def test_gemv_rows_m_invariant(sess, n, k):
    """The decode GEMV among itself: the M = 1 row kernel and the LDS-DMA kernel (M = 2..4 with K % 4 == 0 and
    K <= 6144, and M = 5..8 with K <= 2048 and N < 4096) run the same FMA sequence per row and the same lane
    butterfly, so a row is bit-identical whichever of these M carries it (the reference's GEMV is exempt at
    M = 1; this keeps decode batches of 1..8 rows consistent with each other), in both math modes."""
    announce(f"gemv rows m-invariance n={n} k={k}")
    rng = np.random.default_rng(n + k)
    x = rng.normal(0, 1, (8, k)).astype(np.float32)
    wb = bf16_weights(rng, (n, k), 0.02, "normal")
    w = sess.upload_weight(wb, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
    dx = sess.to_device(x)
    top = 8 if n < 4096 and k <= 2048 else 4
    for kw in ({}, {"math": L.MATH_BF16}):
        ys = {}
        for m in range(1, top + 1):
            y = sess.empty(L.DT_F32, (m, n))
            sess.gemm(dx, w, y, m, **kw)
            ys[m] = y.numpy()
        for m in range(1, top):
            assert np.array_equal(ys[m].view(np.uint32), ys[top][:m].view(np.uint32)), f"M={m} vs M={top} {kw}"
    w.free(), dx.free()


@pytest.mark.parametrize("seed", range(12))
def test_hilo_random_shapes_and_row_invariance(sess, seed):
    """The default math for f32 A × bf16 W (hi/lo planes) on random shapes: large-tile launches (two
    activation planes as a doubled k-tile sequence) and small-tile ones (both planes per LDS stage) are held
    to the reference's f32-class bound (relative 1e-5·sqrt(K), ops/gemm_bf16_optest_test.go:57) against the
    float64 oracle with a bias and GELU; and the rows the smaller call shares with the larger one are
    bit-identical (both tile families multiply each k-tile hi first half, hi second half, lo first half, lo
    second half), as kernels/gemm/minvariance_test.go:21 asks of a GEMM."""
    rng = np.random.default_rng(9000 + seed)
    m = int(rng.integers(300, 1400))
    n = int(rng.integers(4096, 7000)) if seed % 3 == 0 else int(rng.integers(1, 1500))
    k = int(rng.integers(1, 2100))
    m_small = int(rng.integers(17, 65))
    announce(f"hi/lo random seed={seed} m={m} m_small={m_small} n={n} k={k}")
    a = rng.normal(0, 1, (m, k)).astype(np.float32)
    wb = bf16_weights(rng, (n, k), 0.05, "normal")
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    da, db = sess.to_device(a), sess.to_device(bias)
    w = sess.upload_weight(wb, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
    kw = dict(beta=1.0, c=db, c_mode=L.C_ROW, act=L.ACT_GELU_ERF)
    got = run_gemm(sess, da, w, m, **kw)
    rows = np.unique(np.concatenate([np.arange(min(m, 40)), rng.integers(0, m, 60)]))
    want = oracle.gemm(np.ascontiguousarray(a[rows]), wb, trans_b=True, b_dtype=oracle.BF16, beta=1.0, c=bias,
                       c_mode=L.C_ROW, act_code=L.ACT_GELU_ERF)
    rel = np.max(np.abs(got[rows] - want) / (1 + np.abs(want)))
    assert rel <= 1e-5 * math.sqrt(max(k, 1)), f"relative error {rel:.3e}"
    small = run_gemm(sess, da, w, m_small, **kw)
    assert np.array_equal(small, got[:m_small]), f"rows differ between M={m_small} and M={m}"
    w.free(), da.free(), db.free()


@pytest.mark.parametrize("kind", ["f32", "bf16", "i8"])
@pytest.mark.parametrize("seed", range(8))
def test_random_shapes_all_kinds(sess, kind, seed):
    """Random shapes across every GEMM kind and the tile heuristic's whole range (M from 1 to ~1400, N and K
    ragged): f32 weights held to the reference's relative 1e-5·sqrt(K) (kernels/gemm/gemm_test.go:34), bf16
    math to the north-star bound, int8 MatMulInteger + dequant bit-exact; and, except where the decode GEMV
    takes the small call (bf16, M <= 16), rows shared by a small and a large call are bit-identical
    (kernels/gemm/minvariance_test.go:21)."""
    rng = np.random.default_rng(7100 + 97 * seed + len(kind))
    m = int(rng.integers(1, 1400))
    n = int(rng.integers(1, 3000))
    k = int(rng.integers(1, 2500))
    m_small = int(rng.integers(1, min(m, 200) + 1))
    announce(f"random {kind} seed={seed} m={m} m_small={m_small} n={n} k={k}")
    if kind == "i8":
        a = rng.integers(0, 256, (m, k)).astype(np.uint8)
        b = rng.integers(-127, 128, (k, n)).astype(np.int8)
        za = int(rng.integers(0, 256))
        sc = rng.uniform(0.001, 0.01, n).astype(np.float32)
        w = sess.upload_weight(b, trans=False, pack_dtype=L.DT_I8)
        da, ds = sess.to_device(a, L.DT_U8), sess.to_device(sc)

        def run(mm):
            yi, yf = sess.empty(L.DT_I32, (mm, n)), sess.empty(L.DT_F32, (mm, n))
            sess.matmul_integer(da, w, mm, za, y_i32=yi, scale=ds, y_f32=yf)
            return yi.numpy(), yf.numpy()

        yi, yf = run(m)
        want = oracle.matmul_integer(a, b, za)
        assert np.array_equal(yi, want), "int8 products"
        assert np.array_equal(yf, oracle.dequantize_linear(want, sc, inner=1)), "int8 dequant"
        w.free(), da.free(), ds.free()
        return
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    db = sess.to_device(bias)
    kw = dict(beta=1.0, c=db, c_mode=L.C_ROW, act=L.ACT_RELU)
    if kind == "f32":
        bt = rng.uniform(-1, 1, (n, k)).astype(np.float32)
        w = sess.upload_weight(bt, trans=True, pack_dtype=L.DT_F32)
        wide, okw, ain = bt, {}, a
    else:
        bt = bf16_weights(rng, (n, k))
        w = sess.upload_weight(bt, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
        wide, okw = oracle.bf16_to_f32(bt), {"b_dtype": oracle.BF16}
        kw["math"] = L.MATH_BF16
        ain = oracle.bf16_to_f32(oracle.f32_to_bf16(a))
    da = sess.to_device(a)
    got = run_gemm(sess, da, w, m, **kw)
    rows = np.unique(np.concatenate([np.arange(min(m, 24)), rng.integers(0, m, 40)]))
    want = oracle.gemm(np.ascontiguousarray(ain[rows]), bt, trans_b=True, beta=1.0, c=bias, c_mode=L.C_ROW,
                       act_code=L.ACT_RELU, **okw)
    assert_close(got[rows], want, nstar_tol(k, a, wide), f"{kind} {m}x{n}x{k}")
    if kind == "f32":
        rel = np.max(np.abs(got[rows] - want) / np.maximum(np.abs(want), 1.0))
        assert rel <= 1e-5 * math.sqrt(k), f"f32 relative error {rel:.3e}"
    if kind == "f32" or m_small > 16:
        assert np.array_equal(run_gemm(sess, da, w, m_small, **kw), got[:m_small]), f"rows M={m_small} vs M={m}"
    w.free(), da.free(), db.free()


@pytest.mark.parametrize("seed", range(16))
def test_gemv_random_shapes(sess, seed):
    """The decode routes on random shapes (kernels/gemm/bgemm.go:201-206): M from 1 to 16, N from 1 to ~6000
    (odd included), K from 1 to ~7000 (K % 4 != 0 and rows past the LDS-staged length included), strided x,
    a row bias and an activation, both math modes, through the GEMM entry (the router) and the GEMV entry.
    Held to the north-star bound and, f32-class, the reference's relative 1e-5·sqrt(K); a second call is
    bit-identical."""
    rng = np.random.default_rng(8800 + seed)
    m = int(rng.integers(1, 17))
    n = int(rng.integers(1, 6000)) | (1 if seed % 2 else 0)
    k = int(rng.integers(1, 7100)) if seed % 4 else int(rng.integers(1, 700)) * 4
    lda = k + int(rng.integers(0, 9))
    act = [L.ACT_NONE, L.ACT_RELU, L.ACT_GELU_ERF, L.ACT_SILU][seed % 4]
    announce(f"gemv random seed={seed} m={m} n={n} k={k} lda={lda} act={act}")
    xs = rng.normal(0, 1, (m, lda)).astype(np.float32)
    x = xs[:, :k]
    wb = bf16_weights(rng, (n, k), 0.02, "normal")
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    w = sess.upload_weight(wb, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
    dx, db = sess.to_device(xs), sess.to_device(bias)
    wide = oracle.bf16_to_f32(wb)
    kw = dict(lda=lda, beta=1.0, c=db, c_mode=L.C_ROW, act=act)
    for entry in (sess.gemm, sess.gemv_bf16):
        for math_mode in (L.MATH_AUTO, L.MATH_BF16):
            y = sess.empty(L.DT_F32, (m, n))
            entry(dx, w, y, m, math=math_mode, **kw)
            got = y.numpy()
            xin = x if math_mode == L.MATH_AUTO else oracle.bf16_to_f32(oracle.f32_to_bf16(x))
            want = oracle.gemm(np.ascontiguousarray(xin), wb, trans_b=True, b_dtype=oracle.BF16, c=bias,
                               c_mode=L.C_ROW, beta=1.0, act_code=act)
            what = f"{entry.__name__} math {math_mode}"
            assert_close(got, want, nstar_tol(k, x, wide), what)
            if math_mode == L.MATH_AUTO:
                rel = np.max(np.abs(got - want)) / max(1.0, np.max(np.abs(want)))
                assert rel <= 1e-5 * math.sqrt(k), f"{what}: relative error {rel:.3e}"
            entry(dx, w, y, m, math=math_mode, **kw)
            assert np.array_equal(y.numpy(), got), f"{what}: second call differs"
    w.free(), dx.free(), db.free()


@pytest.mark.parametrize("m", [1, 3, 4])
def test_gemv_two_rows_per_wave_odd_n(env_session, m):
    """The LDS-DMA GEMV with two weight rows per wave (INGOT_GEMV_CFG=26) where N is odd: the last wave's
    second row is past N (its loads fill zeros, its sums are not stored)."""
    announce(f"gemv two rows per wave odd n m={m}")
    sess = env_session(INGOT_GEMV_CFG=26)
    rng = np.random.default_rng(4200 + m)
    n, k = 1001, 2048
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    wb = bf16_weights(rng, (n, k), 0.02, "normal")
    w = sess.upload_weight(wb, trans=True, pack_dtype=L.DT_BF16, src_dtype=L.DT_BF16)
    y = sess.empty(L.DT_F32, (m, n))
    sess.gemv_bf16(sess.to_device(x), w, y, m)
    want = oracle.gemm(x, wb, trans_b=True, b_dtype=oracle.BF16)
    assert_close(y.numpy(), want, nstar_tol(k, x, oracle.bf16_to_f32(wb)), f"cfg 26 m {m}")
    w.free()
