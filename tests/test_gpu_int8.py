"""GPU parity of int8 MatMulInteger (+ fused DequantizeLinear) and DequantizeLinear.

Bar: bit-exact. int32 outputs equal the oracle's closed form Σ(a−za)·b
(ops/quant.go:831-900); dequantized f32 outputs equal float32(y − z)·scale
(ops/quant.go:173-229) bit for bit.
"""
import json
import os

import numpy as np
import pytest

import oracle
from helpers import announce
from ingot_amd import _lib as L

pytestmark = pytest.mark.gpu

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kats.json")))


def test_matmul_integer_kat(sess):
    announce("int8 kat")
    k = KATS["matmul_integer"]
    a = np.array(k["A"], np.uint8).reshape(k["m"], k["k"])
    b = np.array(k["B"], np.int8).reshape(k["k"], k["n"])
    w = sess.upload_weight(b, trans=False, pack_dtype=L.DT_I8)
    y = sess.empty(L.DT_I32, (k["m"], k["n"]))
    sess.matmul_integer(sess.to_device(a), w, k["m"], k["za"], y_i32=y)
    assert np.array_equal(y.numpy(), np.array(k["Y"], np.int32))


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (7, 33, 12), (5, 128, 70), (64, 256, 64), (130, 384, 200),
                                   (300, 100, 33)])
@pytest.mark.parametrize("a_dt,za", [(np.uint8, 128), (np.uint8, 0), (np.uint8, 201), (np.int8, 0), (np.int8, -9)])
def test_matmul_integer_exact(sess, m, k, n, a_dt, za):
    announce(f"int8 m={m} k={k} n={n} a={np.dtype(a_dt).name} za={za}")
    rng = np.random.default_rng(m * 17 + k * 3 + n + za)
    lo, hi = (0, 256) if a_dt == np.uint8 else (-128, 128)
    a = rng.integers(lo, hi, (m, k)).astype(a_dt)
    b = rng.integers(-128, 128, (k, n)).astype(np.int8)
    w = sess.upload_weight(b, trans=False, pack_dtype=L.DT_I8)
    y = sess.empty(L.DT_I32, (m, n))
    sess.matmul_integer(sess.to_device(a, L.DT_U8 if a_dt == np.uint8 else L.DT_I8), w, m, za, y_i32=y)
    assert np.array_equal(y.numpy(), oracle.matmul_integer(a, b, za))
    w.free()


def test_config3_matmul_integer_dequant(sess):
    """A u8 [1024,768] za=128, B s8 [768,3072] zp 0, then per-column dequant."""
    announce("config 3 int8")
    rng = np.random.default_rng(3)
    a = rng.integers(0, 256, (1024, 768)).astype(np.uint8)
    b = rng.integers(-127, 128, (768, 3072)).astype(np.int8)
    scale = (rng.uniform(0.001, 0.01, 3072).astype(np.float32) * np.float32(0.02)).astype(np.float32)
    w = sess.upload_weight(b, trans=False, pack_dtype=L.DT_I8)
    da = sess.to_device(a, L.DT_U8)
    yi = sess.empty(L.DT_I32, (1024, 3072))
    yf = sess.empty(L.DT_F32, (1024, 3072))
    ds = sess.to_device(scale)
    sess.matmul_integer(da, w, 1024, 128, y_i32=yi, scale=ds, y_f32=yf)
    want = oracle.matmul_integer(a, b, 128)
    got_i = yi.numpy()
    assert np.array_equal(got_i, want)
    assert np.array_equal(yf.numpy(), oracle.dequantize_linear(want, scale, inner=1))
    # f32-only output (the fused form) matches too
    yf2 = sess.empty(L.DT_F32, (1024, 3072))
    sess.matmul_integer(da, w, 1024, 128, scale=ds, y_f32=yf2)
    assert np.array_equal(yf2.numpy(), yf.numpy())


def test_dequantize_kats(sess):
    announce("dequant kats")
    for name, dt, code in [("dequantize_u8", np.uint8, L.DT_U8), ("dequantize_i8", np.int8, L.DT_I8)]:
        k = KATS[name]
        x = sess.to_device(np.array(k["x"], dt), code)
        y = sess.empty(L.DT_F32, (len(k["x"]),))
        sess.dequantize_linear(x, sess.to_device(np.array(k["scale"], np.float32)), y,
                               zp=sess.to_device(np.array(k["zp"], dt), code))
        assert np.array_equal(y.numpy(), np.array(k["y"], np.float32))


@pytest.mark.parametrize("xdt,code", [(np.uint8, L.DT_U8), (np.int8, L.DT_I8), (np.int32, L.DT_I32)])
def test_dequantize_per_axis_exact(sess, xdt, code):
    announce(f"dequant per-axis {np.dtype(xdt).name}")
    rng = np.random.default_rng(9)
    info = np.iinfo(xdt)
    x = rng.integers(max(info.min, -2**24), min(info.max, 2**24), (6, 5, 7), endpoint=True).astype(xdt)
    sc = rng.uniform(0.001, 0.01, 5).astype(np.float32)
    zp = rng.integers(-3, 4, 5).astype(np.int32) if xdt == np.int32 else rng.integers(0, 100, 5).astype(xdt)
    zcode = L.DT_I32 if xdt == np.int32 else code
    y = sess.empty(L.DT_F32, x.shape)
    sess.dequantize_linear(sess.to_device(x, code), sess.to_device(sc), y, inner=7, zp=sess.to_device(zp, zcode))
    assert np.array_equal(y.numpy(), oracle.dequantize_linear(x, sc, inner=7, zp=zp))


# ---------------- QLinearMatMul (requantised int8 output) ----------------

def test_qlinear_matmul_kats(sess):
    """The golden requant cases: the reference test's scales (u8 out) and exact .5 ties with s8 saturation."""
    announce("qlinear kats")
    km, kr, kt = KATS["matmul_integer"], KATS["qlinear_ref"], KATS["qlinear_ties"]
    for case, src in [(kr, km), (kt, kt)]:
        a = np.array(src["A"], np.uint8).reshape(src["m"], src["k"])
        b = np.array(src["B"], np.int8).reshape(src["k"], src["n"])
        w = sess.upload_weight(b, trans=False, pack_dtype=L.DT_I8)
        y = sess.empty(L.DT_U8 if case["u8"] else L.DT_I8, (src["m"], src["n"]))
        mult = oracle.qlinear_mult(case["sa"], case["sb"], case["sy"])
        sess.qlinear_matmul(sess.to_device(a), w, src["m"], src["za"], mult, case["zy"], y)
        want = np.array(case["Y"][:src["m"] * src["n"]], np.int64).reshape(src["m"], src["n"])
        assert np.array_equal(y.numpy().astype(np.int64), want)
        w.free()


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (7, 33, 12), (64, 256, 64), (130, 384, 203), (1024, 768, 3072)])
@pytest.mark.parametrize("a_dt,za,ydt,zy", [(np.uint8, 128, np.uint8, 3), (np.uint8, 77, np.int8, -5),
                                            (np.int8, -9, np.int8, 0), (np.int8, 0, np.uint8, 128)])
def test_qlinear_matmul_exact(sess, m, k, n, a_dt, za, ydt, zy):
    """Bit-exact against the oracle's restatement of the reference requant, ragged and full sizes."""
    announce(f"qlinear m={m} k={k} n={n} a={np.dtype(a_dt).name} y={np.dtype(ydt).name}")
    rng = np.random.default_rng(m + 7 * k + 3 * n + zy)
    lo, hi = (0, 256) if a_dt == np.uint8 else (-128, 128)
    a = rng.integers(lo, hi, (m, k)).astype(a_dt)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    sa, sb = 0.02, 0.003
    sy = float(np.float32(sa) * np.float32(sb) * np.float32(np.sqrt(k) * 40.0))  # spreads outputs over the range
    mult = oracle.qlinear_mult(sa, sb, sy)
    w = sess.upload_weight(b, trans=False, pack_dtype=L.DT_I8)
    y = sess.empty(L.DT_U8 if ydt == np.uint8 else L.DT_I8, (m, n))
    sess.qlinear_matmul(sess.to_device(a), w, m, za, mult, zy, y)
    want = oracle.qlinear_matmul(a, b, za, sa, sb, sy, zy, ydt == np.uint8)
    got = y.numpy()
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} of {got.size} differ"
    w.free()


@pytest.mark.parametrize("seed", range(24))
def test_random_matmul_integer_exact(sess, seed):
    """Seeded random MatMulInteger calls, bit-exact against the oracle's closed form: shapes from 1 up to
    configs[2] size, u8 or s8 activations with any zero point of their type, the full s8 weight range (−128 too)
    in either source layout, an activation pitch wider than K, and the int32 output, the fused per-column or
    per-tensor dequantisation with a zero point, or both."""
    rng = np.random.default_rng(7000 + seed)

    def dim(lo, hi):
        return int(np.exp(rng.uniform(np.log(lo), np.log(hi + 1))))

    m, k, n = dim(1, 800), dim(1, 1600), dim(1, 2500)
    a_dt = [np.uint8, np.int8][rng.integers(2)]
    info = np.iinfo(a_dt)
    za = int(rng.integers(info.min, info.max, endpoint=True))
    lda = k + int(rng.choice([0, 0, 3, 16]))
    kn = bool(rng.integers(2))
    outs = ["i32", "f32", "both"][rng.integers(3)]
    per_col = bool(rng.integers(2))
    dq_zp = int(rng.integers(-40, 41))
    announce(f"int8 random seed={seed} m={m} k={k} n={n} a={np.dtype(a_dt).name} za={za} lda={lda} "
             f"kn={kn} outs={outs} per_col={per_col}")
    a = rng.integers(info.min, info.max, (m, lda), endpoint=True).astype(a_dt)
    b = rng.integers(-128, 127, (k, n), endpoint=True).astype(np.int8)
    w = sess.upload_weight(b if kn else np.ascontiguousarray(b.T), trans=not kn, pack_dtype=L.DT_I8)
    scale = rng.uniform(0.001, 0.01, n if per_col else 1).astype(np.float32)
    yi = sess.empty(L.DT_I32, (m, n)) if outs in ("i32", "both") else None
    yf = sess.empty(L.DT_F32, (m, n)) if outs in ("f32", "both") else None
    sess.matmul_integer(sess.to_device(a, L.DT_U8 if a_dt == np.uint8 else L.DT_I8), w, m, za, y_i32=yi,
                        scale=sess.to_device(scale) if yf is not None else None, dq_zp=dq_zp, y_f32=yf, lda=lda)
    want = oracle.matmul_integer(np.ascontiguousarray(a[:, :k]), b, za)
    if yi is not None:
        assert np.array_equal(yi.numpy(), want), f"int32 seed {seed}"
    if yf is not None:
        wf = oracle.dequantize_linear(want, scale, inner=1, zp=np.array([dq_zp], np.int32))
        assert np.array_equal(yf.numpy(), wf), f"dequant seed {seed}"
    w.free()
