"""The operator layer (op.Op mirror) on the GPU, case for case after the
reference's op tests (ops/compute_optest_test.go, ops/gemm_bf16_optest_test.go,
ops/quant_optest_test.go), checked against the CPU oracle.

Exact known answers are compared bit for bit; floating-point products use the
north-star bound 1e-3·sqrt(K)·max|A|·max|B| (and the reference's own
1e-4 relative eqF32 bound where its test used it on exact inputs).
"""
import json
import os

import numpy as np
import pytest

import oracle
from helpers import announce, assert_close, bf16_weights, nstar_tol
from ingot_amd import IngotError
from ingot_amd import _lib as L

pytestmark = pytest.mark.gpu

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kats.json")))


def dev(sess, arr, code=None):
    return sess.to_device(np.ascontiguousarray(arr), code)


def run(op, *ins):
    outs = op.run(*ins)
    res = [o.numpy() for o in outs]
    for o in outs:
        o.free()
    return res


def test_lookup_errors(sess):
    with pytest.raises(IngotError, match="unsupported op"):
        sess.op("Conv", 11)
    with pytest.raises(IngotError, match="not supported at opset 6"):
        sess.op("Gemm", 6)
    with pytest.raises(IngotError, match="unknown ingot_act"):
        sess.op("MatMul", 13, {"ingot_act": "swish"})


def test_gemm_transb_kat(sess):
    """TestGemmTransB (ops/compute_optest_test.go:232-252), bit-exact."""
    announce("op gemm kat")
    k = KATS["gemm_transb"]
    a = np.array(k["A"], np.float32).reshape(k["A_shape"])
    b = np.array(k["B"], np.float32).reshape(k["B_shape"])
    c = np.array(k["C"], np.float32)
    op = sess.op("Gemm", 7, {"transB": 1, "alpha": 2.0, "beta": 1.0})
    (y,) = run(op, dev(sess, a), dev(sess, b), dev(sess, c))
    assert y.shape == (2, 4)
    assert np.array_equal(y, np.array(k["Y"], np.float32))


def test_matmul_batched_kat(sess):
    """TestMatMulBatched (ops/compute_optest_test.go:254-274), bit-exact."""
    announce("op matmul batched kat")
    k = KATS["matmul_batched"]
    a = np.array(k["A"], np.float32).reshape(k["A_shape"])
    b = np.array(k["B"], np.float32).reshape(k["B_shape"])
    (y,) = run(sess.op("MatMul", 1), dev(sess, a), dev(sess, b))
    assert np.array_equal(y, np.array(k["Y"], np.float32))


@pytest.mark.parametrize("as_,bs", [((2, 2, 3), (3, 2)), ((7, 1, 384), (384, 96)), ((3, 5, 17), (17, 9)),
                                    ((2, 3, 4, 33), (33, 5)), ((33,), (33, 5)), ((4, 33), (33,))])
def test_matmul_broadcast_batch(sess, as_, bs):
    """TestMatMulBroadcastBatch (:280-318) plus the NumPy 1-D promotions."""
    announce(f"op matmul bcast {as_} {bs}")
    rng = np.random.default_rng(7)
    a = rng.uniform(-1, 1, as_).astype(np.float32)
    b = rng.uniform(-1, 1, bs).astype(np.float32)
    (y,) = run(sess.op("MatMul", 13), dev(sess, a), dev(sess, b))
    want = np.matmul(a.astype(np.float64), b.astype(np.float64))
    assert y.shape == want.shape
    assert_close(y, want, nstar_tol(bs[0], a, b), "matmul bcast")


@pytest.mark.parametrize("as_,bs", [((2, 3, 77, 40), (2, 3, 40, 77)), ((2, 3, 77, 77), (2, 3, 77, 40)),
                                    ((96, 128, 64), (96, 64, 128)), ((2, 1, 9, 16), (1, 3, 16, 11)),
                                    ((9, 16), (4, 16, 11)), ((4, 9, 16), (1, 16, 11)), ((3, 1, 5), (3, 5, 1))])
def test_matmul_batched_rhs(sess, as_, bs):
    """Batched right operand (attention Q·Kᵀ and P·V shapes, ops/matmul.go:375-403): equal batch shapes,
    whole-side broadcast and a mixed broadcast that needs per-item products; run 2 bit-identical."""
    announce(f"op matmul batched rhs {as_} {bs}")
    rng = np.random.default_rng(17)
    a = rng.uniform(-1, 1, as_).astype(np.float32)
    b = rng.uniform(-1, 1, bs).astype(np.float32)
    op = sess.op("MatMul", 13)
    da, db = dev(sess, a), dev(sess, b)
    (y,) = run(op, da, db)
    want = np.matmul(a.astype(np.float64), b.astype(np.float64))
    assert y.shape == want.shape
    assert_close(y, want, nstar_tol(bs[-2], a, b), "matmul batched rhs")
    (y2,) = run(op, da, db)
    assert np.array_equal(y, y2), "second run differs"


@pytest.mark.parametrize("as_,bs", [((128, 384), (384, 1152)), ((1, 16, 48), (48, 144)), ((7, 1, 384), (384, 96)),
                                    ((5, 13), (13, 7)), ((2, 3, 4, 33), (33, 5)), ((2, 8, 32), (2, 32, 96))])
def test_matmul_bias(sess, as_, bs):
    """TestMatMulBias (:326-368): fused bias on the packed path and the batched-rhs path; run 2 bit-identical."""
    announce(f"op matmul bias {as_} {bs}")
    rng = np.random.default_rng(9)
    a = rng.uniform(-1, 1, as_).astype(np.float32)
    b = rng.uniform(-1, 1, bs).astype(np.float32)
    n = bs[-1]
    bias = rng.uniform(-1, 1, n).astype(np.float32)
    op = sess.op("MatMul", 1)
    da, db, dbias = dev(sess, a), dev(sess, b), dev(sess, bias)
    (y,) = run(op, da, db, dbias)
    want = np.matmul(a.astype(np.float64), b.astype(np.float64)) + bias
    assert_close(y, want, nstar_tol(bs[-2], a, b) + 1e-6, "matmul bias")
    (y2,) = run(op, da, db, dbias)
    assert np.array_equal(y, y2), "second run differs"


@pytest.mark.parametrize("as_,bs", [((128, 384), (384, 1536)), ((1, 16, 48), (48, 144)), ((2, 8, 32), (2, 32, 96))])
def test_matmul_gelu(sess, as_, bs):
    """TestMatMulGelu (:405-): ingot_act=gelu fused vs MatMul → ingot.Gelu."""
    announce(f"op matmul gelu {as_} {bs}")
    rng = np.random.default_rng(31)
    a = rng.uniform(-1, 1, as_).astype(np.float32)
    b = rng.uniform(-1, 1, bs).astype(np.float32)
    bias = rng.uniform(-1, 1, bs[-1]).astype(np.float32)
    da, db, dbias = dev(sess, a), dev(sess, b), dev(sess, bias)
    (fused,) = run(sess.op("MatMul", 1, {"ingot_act": "gelu"}), da, db, dbias)
    mm = sess.op("MatMul", 1).run(da, db, dbias)[0]
    (sep,) = run(sess.op("Gelu", 1, domain="ingot"), mm)
    mm.free()
    assert_close(fused, sep, 1e-5, "fused vs separate gelu")
    pre = np.matmul(a.astype(np.float64), b.astype(np.float64)) + bias
    want = np.vectorize(lambda v: oracle.act(v, L.ACT_GELU_ERF))(pre)
    assert_close(fused, want, nstar_tol(bs[-2], a, b) + 1e-6, "gelu vs oracle")


@pytest.mark.parametrize("m,trans_b", [(37, 0), (37, 1), (1, 0), (1, 1), (3, 1), (16, 1), (17, 1)])
def test_gemm_bf16_weight(sess, m, trans_b):
    """TestGemmBF16Weight (ops/gemm_bf16_optest_test.go:29-63): K=300, N=29, alpha 0.5, beta 2."""
    announce(f"op gemm bf16 m={m} transB={trans_b}")
    rng = np.random.default_rng(81 + m + trans_b)
    K, N = 300, 29
    a = rng.uniform(-1, 1, (m, K)).astype(np.float32)
    b = bf16_weights(rng, (N, K) if trans_b else (K, N))
    c = rng.uniform(-1, 1, N).astype(np.float32)
    op = sess.op("Gemm", 13, {"transB": trans_b, "alpha": 0.5, "beta": 2.0})
    (y,) = run(op, dev(sess, a), dev(sess, b, L.DT_BF16), dev(sess, c))
    want = oracle.gemm(a, b, trans_b=bool(trans_b), b_dtype=oracle.BF16, alpha=0.5, beta=2.0, c=c, c_mode=2)
    assert_close(y, want, nstar_tol(K, a, oracle.bf16_to_f32(b)), "gemm bf16 weight")


@pytest.mark.parametrize("cshape", [(6, 10), (10,), (1, 10), (6, 1), (1,), ()])
def test_gemm_c_broadcast(sess, cshape):
    announce(f"op gemm C {cshape}")
    rng = np.random.default_rng(3)
    a = rng.uniform(-1, 1, (6, 20)).astype(np.float32)
    b = rng.uniform(-1, 1, (20, 10)).astype(np.float32)
    c = rng.normal(size=cshape).astype(np.float32)
    (y,) = run(sess.op("Gemm", 11, {"beta": 0.5}), dev(sess, a), dev(sess, b), dev(sess, c))
    want = a.astype(np.float64) @ b.astype(np.float64) + 0.5 * np.broadcast_to(c.reshape(
        cshape if len(cshape) == 2 else (-1,)), (6, 10))
    assert_close(y, want, nstar_tol(20, a, b) + 1e-6, f"C {cshape}")


def test_gemm_trans_a_and_errors(sess):
    announce("op gemm transA")
    rng = np.random.default_rng(4)
    a = rng.uniform(-1, 1, (20, 6)).astype(np.float32)
    b = rng.uniform(-1, 1, (10, 20)).astype(np.float32)
    (y,) = run(sess.op("Gemm", 11, {"transA": 1, "transB": 1}), dev(sess, a), dev(sess, b))
    assert_close(y, a.T.astype(np.float64) @ b.T.astype(np.float64), nstar_tol(20, a, b), "transA")
    with pytest.raises(IngotError, match="inner dim mismatch"):
        sess.op("Gemm", 11).run(dev(sess, a), dev(sess, b))
    with pytest.raises(IngotError, match="cannot broadcast C"):
        sess.op("Gemm", 11).run(dev(sess, a.T.copy()), dev(sess, b.T.copy()), dev(sess, np.zeros(7, np.float32)))
    with pytest.raises(IngotError, match="need A and B"):
        sess.op("Gemm", 11).run(dev(sess, a))


@pytest.mark.parametrize("m", [1, 3, 9])
def test_gemm_int8_weight(sess, m):
    """TestGemmInt8Weight (ops/gemm_bf16_optest_test.go:96-136): ingot_weight_quant="int8" at decode shapes
    (M <= 4: the int8 GEMV, bit-exact to the oracle and within the reference's bound of the float64 value over
    the quantised operands); M = 9 stays on the exact bf16 path."""
    announce(f"op gemm int8 weight m={m}")
    rng = np.random.default_rng(85 + m)
    K, N = 256, 29
    a = rng.uniform(-1, 1, (m, K)).astype(np.float32)
    wb = bf16_weights(rng, (N, K), 1.0, "uniform")
    wide = oracle.bf16_to_f32(wb)
    c = rng.uniform(-1, 1, N).astype(np.float32)
    op = sess.op("Gemm", 13, {"transB": 1, "alpha": 0.5, "beta": 2.0, "ingot_weight_quant": "int8"})
    (y,) = run(op, dev(sess, a), dev(sess, wb, L.DT_BF16), dev(sess, c))
    if m <= 4:
        q, sc = oracle.quantize_i8g(wide)
        assert np.array_equal(y, oracle.gemv_i8g(a, q, sc, 0.5, 2.0, c))
        deq = (q.reshape(N, -1, 64).astype(np.float64) * sc[..., None]).reshape(N, K)
        for i in range(m):
            xh, xl, sx = oracle.quantize_x16(a[i])
            xq = np.repeat(sx, 64).astype(np.float64) * (128 * xh.astype(np.float64) + xl)
            want = 0.5 * (deq @ xq) + 2.0 * c.astype(np.float64)
            assert np.all(np.abs(y[i] - want) <= 1e-5 * np.sqrt(K) * (1 + np.abs(want)))
    else:
        want = oracle.gemm(a, wb, trans_b=True, b_dtype=oracle.BF16, alpha=0.5, beta=2.0, c=c, c_mode=2)
        assert_close(y, want, nstar_tol(K, a, wide), "gemm bf16 path")


def test_qlinear_matmul_op(sess):
    """TestQLinearMatMulAndMatMulInteger (ops/quant_optest_test.go:194-223), QLinearMatMul half, bit-exact to the
    oracle's requant; output dtype from y_zero_point; the op's error cases."""
    announce("op qlinear matmul")
    km, kr = KATS["matmul_integer"], KATS["qlinear_ref"]
    a = np.array(km["A"], np.uint8).reshape(km["m"], km["k"])
    b = np.array(km["B"], np.int8).reshape(km["k"], km["n"])
    op = sess.op("QLinearMatMul", 10)
    f32 = lambda v: dev(sess, np.array([v], np.float32))
    ins = [dev(sess, a), f32(kr["sa"]), dev(sess, np.array([km["za"]], np.uint8)), dev(sess, b), f32(kr["sb"]),
           dev(sess, np.array([0], np.int8)), f32(kr["sy"]), dev(sess, np.array([kr["zy"]], np.uint8))]
    (y,) = run(op, *ins)
    assert y.dtype == np.uint8
    assert np.array_equal(y.reshape(-1).astype(np.int64), np.array(kr["Y"], np.int64))
    # s8 output zero point → s8 output
    ins_s8 = ins[:7] + [dev(sess, np.array([-7], np.int8))]
    (y8,) = run(op, *ins_s8)
    assert y8.dtype == np.int8
    want = oracle.qlinear_matmul(a, b, km["za"], kr["sa"], kr["sb"], kr["sy"], -7, False)
    assert np.array_equal(y8, want)
    # absent output zero point → u8, zero point 0
    (y0,) = run(op, *(ins[:7] + [None]))
    assert y0.dtype == np.uint8
    assert np.array_equal(y0, oracle.qlinear_matmul(a, b, km["za"], kr["sa"], kr["sb"], kr["sy"], 0, True))
    with pytest.raises(IngotError, match="non-zero weight zero_point"):
        op.run(*(ins[:5] + [dev(sess, np.array([1], np.int8))] + ins[6:]))
    with pytest.raises(IngotError, match="per-tensor a zero_point only"):
        op.run(*(ins[:2] + [dev(sess, np.array([1, 2], np.uint8))] + ins[3:]))
    with pytest.raises(IngotError, match="unsupported output quantization"):
        op.run(*(ins[:7] + [dev(sess, np.array([1, 2], np.uint8))]))
    with pytest.raises(IngotError, match="need 8 inputs"):
        op.run(*ins[:4])


def test_matmul_integer_op(sess):
    """TestQLinearMatMulAndMatMulInteger's MatMulInteger half (ops/quant_optest_test.go:194-223)."""
    announce("op matmulinteger")
    k = KATS["matmul_integer"]
    a = np.array(k["A"], np.uint8).reshape(k["m"], k["k"])
    b = np.array(k["B"], np.int8).reshape(k["k"], k["n"])
    op = sess.op("MatMulInteger", 10)
    da, db = dev(sess, a, L.DT_U8), dev(sess, b, L.DT_I8)
    (y,) = run(op, da, db, dev(sess, np.array([k["za"]], np.uint8), L.DT_U8), dev(sess, np.zeros(1, np.int8), L.DT_I8))
    assert np.array_equal(y, np.array(k["Y"], np.int32))
    with pytest.raises(IngotError, match="non-zero weight zero_point"):
        op.run(da, db, None, dev(sess, np.array([1], np.int8), L.DT_I8))
    with pytest.raises(IngotError, match="only s8 weights"):
        op.run(da, dev(sess, b.view(np.uint8), L.DT_U8))


def test_dequantize_linear_op(sess):
    """TestDequantizeLinear (ops/quant_optest_test.go:60-73) + per-axis + axis errors."""
    announce("op dequant")
    op = sess.op("DequantizeLinear", 10)
    (y,) = run(op, dev(sess, np.array([0, 128, 255], np.uint8), L.DT_U8), dev(sess, np.array([0.5], np.float32)),
               dev(sess, np.array([128], np.uint8), L.DT_U8))
    assert np.array_equal(y, np.array([-64, 0, 63.5], np.float32))
    (y,) = run(op, dev(sess, np.array([-128, 127], np.int8), L.DT_I8), dev(sess, np.array([2.0], np.float32)),
               dev(sess, np.array([-8], np.int8), L.DT_I8))
    assert np.array_equal(y, np.array([-240, 270], np.float32))
    rng = np.random.default_rng(2)
    x = rng.integers(-1000, 1000, (4, 6, 3)).astype(np.int32)
    sc = rng.uniform(0.01, 0.1, 6).astype(np.float32)
    (y,) = run(op, dev(sess, x, L.DT_I32), dev(sess, sc))
    assert np.array_equal(y, oracle.dequantize_linear(x, sc, inner=3))
    with pytest.raises(IngotError, match="per-axis scale len"):
        op.run(dev(sess, x, L.DT_I32), dev(sess, np.ones(5, np.float32)))


@pytest.mark.parametrize("name,domain,attrs,code", [("Relu", "", {}, L.ACT_RELU), ("Gelu", "ingot", {}, L.ACT_GELU_ERF),
                                                   ("Gelu", "", {"approximate": "tanh"}, L.ACT_GELU_TANH),
                                                   ("Sigmoid", "", {}, L.ACT_SIGMOID)])
def test_activation_nodes(sess, name, domain, attrs, code):
    announce(f"op {name}")
    rng = np.random.default_rng(8)
    x = rng.normal(0, 3, (7, 33)).astype(np.float32)
    (y,) = run(sess.op(name, 20 if domain == "" and name == "Gelu" else 13 if domain == "" else 1, attrs, domain),
               dev(sess, x))
    want = np.vectorize(lambda v: oracle.act(v, code))(x.astype(np.float64))
    assert_close(y, want, 2e-6 * max(1.0, float(np.max(np.abs(want)))), name)


@pytest.mark.parametrize("code,a,b", [(L.ACT_RELU, 0, 0), (L.ACT_GELU_ERF, 0, 0), (L.ACT_GELU_TANH, 0, 0),
                                      (L.ACT_SIGMOID, 0, 0), (L.ACT_SILU, 0, 0), (L.ACT_HARDSWISH, 0, 0),
                                      (L.ACT_HARDSIGMOID, 0.2, 0.5), (L.ACT_CLIP, -1.5, 2.0), (L.ACT_LEAKYRELU, 0.1, 0)])
def test_activation_special_values(sess, code, a, b):
    """Every activation of the epilogue set on NaN, ±Inf, ±0, huge and exp-saturating inputs, against the
    oracle: NaN where it gives NaN, the same ±Inf, and finite values within 2e-6 relative.

    NaN through the clamps (expScalar's, clip, hardsigmoid) is where the reference disagrees with itself across
    platforms: its arm64 vector kernels (FMAX/FMIN, kernels/vek/vek_arm64.s) and its scalar tails (Go's min/max,
    kernels/vek/scalar.go:11-13, kernels/vek/vek_generic.go:48-76) pass a NaN through, while its amd64 vector
    bodies (VMAXPS/VMINPS, kernels/vek/genamd64/main.go:241-256) return the bound: clip(NaN) = lo and
    hardsigmoid(NaN) = 0 there. This library follows arm64 and the scalar code (NaN out), and the oracle pins
    that choice."""
    announce(f"activation special values act={code}")
    special = [np.nan, np.inf, -np.inf, 0.0, -0.0, 1e30, -1e30, 3.4e38, -3.4e38, 100.0, -100.0, 88.5, -88.5,
               87.4, -87.4, 20.0, -20.0, 1e-30, -1e-30, 0.5, -0.5, 3.0, -3.0]
    x = np.array(special, np.float32).reshape(1, -1)
    y = sess.empty(L.DT_F32, x.shape)
    sess.activation(dev(sess, x), y, 1, x.shape[1], code, a=a, b=b)
    got = y.numpy().astype(np.float64)
    want = np.array([oracle.act(float(v), code, a, b) for v in x[0].astype(np.float64)]).reshape(x.shape)
    want = want.astype(np.float32).astype(np.float64)  # the f32 the product would hold
    assert np.array_equal(np.isnan(got), np.isnan(want)), f"NaN positions: got {got}, want {want}"
    inf = np.isinf(want)
    assert np.array_equal(np.isinf(got), inf) and np.array_equal(got[inf], want[inf]), f"Inf: got {got}, want {want}"
    fin = np.isfinite(want)
    err = np.abs(got[fin] - want[fin]) / np.maximum(1.0, np.abs(want[fin]))
    assert err.max() <= 2e-6, f"act {code}: relative error {err.max():.3e} at {x[0][fin][np.argmax(err)]}"


def test_gelu_tanh_negative_tail_relative(sess):
    """GELU-tanh over a dense sweep of x in [-8, -2], where 1 + tanh(v) is tiny (ops/elementwise.go:411-414): the
    activation kernel and the f32 GEMM epilogue (both apply_act; the product is x·1 exactly) hold a bound relative
    to the float64 value, 2e-5·|want| (the float32 evaluation of v moves the result by a few 1e-6 relative
    there). The reference rounds tanh(v) to float32 before adding 1, so its own values in this range are off by up
    to 2^-25·|x| absolute; the bound is far inside that too."""
    announce("gelu-tanh negative tail")
    x = np.linspace(-8.0, -2.0, 20001).astype(np.float32)
    # in float64 through 1 + tanh(v) = 2 / (1 + e^(-2v)): the formula's own 1 + tanh(v) cancels in float64 as
    # well once v < -13 (x below about -5.4), where it returns 0 or one ulp of 1
    xd = x.astype(np.float64)
    want = xd / (1.0 + np.exp(-2.0 * 0.7978845608028654 * (xd + 0.044715 * xd ** 3)))
    mid = np.abs(xd) < 4.5  # where the float64 formula is still accurate, the identity must agree with it
    direct = np.array([oracle.act(float(v), L.ACT_GELU_TANH) for v in xd[mid]])
    assert np.allclose(want[mid], direct, rtol=1e-8, atol=0)
    tol = 2e-5 * np.abs(want)
    y = sess.empty(L.DT_F32, (1, x.size))
    sess.activation(dev(sess, x.reshape(1, -1)), y, 1, x.size, L.ACT_GELU_TANH)
    got = y.numpy()[0].astype(np.float64)
    bad = np.abs(got - want) > tol
    assert not bad.any(), f"activation: {bad.sum()} values off, worst at x={x[np.argmax(np.abs(got - want) / tol)]}"
    # the fused epilogue: A[i] = (x_i, 0, ..., 0), every weight row = e_0 (f32 weights: the product is exact)
    k, n = 64, 16
    a = np.zeros((x.size, k), np.float32)
    a[:, 0] = x
    w = np.zeros((n, k), np.float32)
    w[:, 0] = 1.0
    wt = sess.upload_weight(w, trans=True, pack_dtype=L.DT_F32)
    yg = sess.empty(L.DT_F32, (x.size, n))
    sess.gemm(dev(sess, a), wt, yg, x.size, act=L.ACT_GELU_TANH)
    got = yg.numpy().astype(np.float64)
    bad = np.abs(got - want[:, None]) > tol[:, None]
    assert not bad.any(), f"GEMM epilogue: {bad.sum()} values off"
    wt.free()


def test_refilled_weight_buffer_is_repacked(sess):
    """An operand not declared constant is packed per call: the same device buffer refilled with new values
    between runs gives the new product (Gemm f32 and bf16 B, MatMul, MatMulInteger). A declared-constant B
    (ingot_rocm_op_set_const) is packed once and reused on later runs."""
    announce("op refilled weight buffer")
    rng = np.random.default_rng(17)
    m, k, n = 40, 192, 136
    a = rng.normal(0, 1, (m, k)).astype(np.float32)
    da = dev(sess, a)
    cases = [("Gemm", 13, {"transB": 1}, lambda b: b.T), ("MatMul", 13, {}, lambda b: b)]
    for name, opset, attrs, orient in cases:
        op = sess.op(name, opset, attrs)
        shape = (n, k) if attrs.get("transB") else (k, n)
        db = sess.empty(L.DT_F32, shape)
        for rep in range(2):
            b = rng.normal(0, 1, shape).astype(np.float32)
            L.check(sess.lib.ingot_rocm_memcpy_h2d(sess.h, db.ptr, b.ctypes.data, b.nbytes))
            (y,) = run(op, da, db)
            want = a.astype(np.float64) @ orient(b).astype(np.float64)
            err = np.max(np.abs(y - want)) / max(1.0, np.max(np.abs(want)))
            assert err <= 1e-5 * np.sqrt(k), f"{name} run {rep}: relative error {err:.3e}"
        op.free()
    # bf16 B bits refilled in place (Gemm, transB)
    op = sess.op("Gemm", 13, {"transB": 1})
    db = sess.empty(L.DT_BF16, (n, k))
    for rep in range(2):
        wb = bf16_weights(rng, (n, k), 0.5)
        L.check(sess.lib.ingot_rocm_memcpy_h2d(sess.h, db.ptr, wb.ctypes.data, wb.nbytes))
        (y,) = run(op, da, db)
        want = oracle.gemm(a, wb, trans_b=True, b_dtype=oracle.BF16)
        assert_close(y, want, nstar_tol(k, a, oracle.bf16_to_f32(wb)), f"gemm bf16 B run {rep}")
    op.free()
    # MatMulInteger: int8 B refilled in place
    qa = rng.integers(0, 256, (m, k)).astype(np.uint8)
    op = sess.op("MatMulInteger", 10)
    dqa = dev(sess, qa, L.DT_U8)
    dqb = sess.empty(L.DT_I8, (k, n))
    for rep in range(2):
        qb = rng.integers(-127, 128, (k, n)).astype(np.int8)
        L.check(sess.lib.ingot_rocm_memcpy_h2d(sess.h, dqb.ptr, qb.ctypes.data, qb.nbytes))
        (y,) = run(op, dqa, dqb, dev(sess, np.array([128], np.uint8), L.DT_U8))
        assert np.array_equal(y, oracle.matmul_integer(qa, qb, 128)), f"matmul_integer run {rep}"
    op.free()
    # a declared constant is packed once: refilling its storage afterwards is outside the contract, and the
    # cached pack (the first values) is what later runs multiply by
    op = sess.op("MatMul", 13).set_const(1)
    db = sess.empty(L.DT_F32, (k, n))
    b0 = rng.normal(0, 1, (k, n)).astype(np.float32)
    L.check(sess.lib.ingot_rocm_memcpy_h2d(sess.h, db.ptr, b0.ctypes.data, b0.nbytes))
    (y0,) = run(op, da, db)
    b1 = rng.normal(0, 1, (k, n)).astype(np.float32)
    L.check(sess.lib.ingot_rocm_memcpy_h2d(sess.h, db.ptr, b1.ctypes.data, b1.nbytes))
    (y1,) = run(op, da, db)
    assert np.array_equal(y0, y1)
    op.free()
