"""Pins the CPU oracle before it is trusted as the checker.

Each oracle function is checked against something it was not derived from:
the reference tests' known answers (tests/golden/kats.json, generated with
exact Python arithmetic), closed forms, and independent implementations
(numpy float64 matmul, pure-Python integer sums, math.erf). Planted-mistake
checks show the known answers reject a transposed operand, a dropped term and
a wrong zero point.

  orc_f32_to_bf16        bf16_rne KATs (exact rational RNE) + NaN/Inf rules
  orc_gemm_ref_f32       TestGemmTransB / TestMatMulBatched KATs (exact ints)
  orc_gemm               same KATs, numpy float64 on random shapes, every
                         C broadcast mode, alpha/beta, transA/transB, bf16 B
  orc_act                closed forms (math.erf, math.tanh, exp), ReLU exact
  orc_gemv_bf16          numpy float64 dot over widened weights
  orc_qgemm_ref          pure-Python int sums
  orc_matmul_integer(+_shifted)  matmul_integer KAT + int64 numpy, both routes
  orc_dequantize_linear  TestDequantizeLinear KATs + numpy f32 formula
"""
import json
import math
import os

import numpy as np
import pytest

import oracle

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kats.json")))


def test_bf16_rne_kats():
    for x, want in KATS["bf16_rne"]:
        f = np.array([x], np.uint32).view(np.float32)
        got = int(oracle.f32_to_bf16(f)[0])
        assert got == want, f"{x:#010x}: got {got:#06x} want {want:#06x}"


def test_bf16_rne_random_matches_exact_rounding():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=20000, dtype=np.uint64).astype(np.uint32)
    bits = bits[(bits & 0x7F800000) != 0x7F800000]  # finite inputs (NaN/Inf are in the KATs)
    bits = bits[(bits & 0x7FFF0000) < 0x7F7F0000]   # next bf16 step finite
    x = bits.view(np.float32)
    got = oracle.f32_to_bf16(x)
    # float64 midpoint rounding: bf16 keeps 8 significant bits; RNE via numpy's
    # float32 → exact value, choose nearest of truncation / next, ties to even
    lo = (bits >> 16).astype(np.uint32)
    lo_v = (lo << 16).view(np.float32).astype(np.float64)
    hi_v = ((lo + 1) << 16).astype(np.uint32).view(np.float32).astype(np.float64)
    xv = x.astype(np.float64)
    dl, dh = np.abs(xv - lo_v), np.abs(hi_v - xv)
    want = np.where((dl < dh) | ((dl == dh) & (lo % 2 == 0)), lo, lo + 1).astype(np.uint16)
    assert np.array_equal(got, want)


def _kat_gemm():
    k = KATS["gemm_transb"]
    a = np.array(k["A"], np.float32).reshape(k["A_shape"])
    b = np.array(k["B"], np.float32).reshape(k["B_shape"])
    return k, a, b, np.array(k["C"], np.float32)


def test_gemm_transb_kat():
    k, a, b, c = _kat_gemm()
    y = oracle.gemm(a, b, trans_b=True, alpha=k["alpha"], beta=k["beta"], c=c, c_mode=2)
    assert np.array_equal(y, np.array(k["Y"], np.float64))
    # Ref (f32) on the same exact inputs
    y32 = oracle.gemm_ref_f32(a, b.T.copy(), alpha=2.0, beta=1.0, c=np.broadcast_to(c, (2, 4)))
    assert np.array_equal(y32, np.array(k["Y"], np.float32))


def test_gemm_kat_rejects_planted_mistakes():
    k, a, b, c = _kat_gemm()
    want = np.array(k["Y"], np.float64)
    # a transposed operand (B read as [K,N] memory of the wrong shape)
    wrong = oracle.gemm(a, b.reshape(3, 4), trans_b=False, alpha=2.0, beta=1.0, c=c, c_mode=2)
    assert not np.array_equal(wrong, want)
    # a dropped term (beta·C omitted)
    assert not np.array_equal(oracle.gemm(a, b, trans_b=True, alpha=2.0, beta=0.0, c=c, c_mode=2), want)
    # wrong broadcast axis (C applied per row instead of per column)
    c2 = np.array([100, 200], np.float32)
    assert not np.array_equal(oracle.gemm(a, b, trans_b=True, alpha=2.0, beta=1.0, c=c2, c_mode=3), want)


def test_matmul_batched_kat():
    k = KATS["matmul_batched"]
    a = np.array(k["A"], np.float32).reshape(k["A_shape"])
    b = np.array(k["B"], np.float32).reshape(k["B_shape"])
    for bt in range(2):
        assert np.array_equal(oracle.gemm(a[bt], b[bt]), np.array(k["Y"][bt], np.float64))


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (3, 5, 7), (37, 29, 300), (64, 33, 129)])
def test_gemm_matches_numpy_float64(m, n, k):
    rng = np.random.default_rng(m * 1000 + n * 10 + k)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    bt = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    ref = a.astype(np.float64) @ bt.T.astype(np.float64)
    np.testing.assert_allclose(oracle.gemm(a, bt, trans_b=True), ref, rtol=0, atol=1e-12)
    np.testing.assert_allclose(oracle.gemm(a, bt.T.copy()), ref, rtol=0, atol=1e-12)
    np.testing.assert_allclose(oracle.gemm(a.T.copy(), bt, trans_a=True, trans_b=True), ref, rtol=0, atol=1e-12)
    # every C mode, alpha/beta
    c_full = rng.normal(size=(m, n)).astype(np.float32)
    c_row = rng.normal(size=n).astype(np.float32)
    c_col = rng.normal(size=(m, 1)).astype(np.float32)
    c_sc = np.array([0.75], np.float32)
    for mode, c, bc in [(1, c_full, c_full), (2, c_row, c_row[None, :]), (3, c_col, c_col), (4, c_sc, c_sc[0])]:
        got = oracle.gemm(a, bt, trans_b=True, alpha=0.5, beta=-2.0, c=c, c_mode=mode, ldc=n)
        np.testing.assert_allclose(got, 0.5 * ref - 2.0 * np.asarray(bc, np.float64), rtol=0, atol=1e-12)


def test_gemm_bf16_weights_widen_exactly():
    rng = np.random.default_rng(5)
    a = rng.uniform(-1, 1, (9, 40)).astype(np.float32)
    w = oracle.f32_to_bf16(rng.uniform(-1, 1, (13, 40)).astype(np.float32))
    wide = oracle.bf16_to_f32(w).astype(np.float64)
    np.testing.assert_allclose(oracle.gemm(a, w, trans_b=True, b_dtype=oracle.BF16), a.astype(np.float64) @ wide.T,
                               rtol=0, atol=1e-12)


def test_activation_closed_forms():
    for x in [-9.0, -3.5, -1.0, -0.25, 0.0, 0.3, 1.0, 2.5, 7.0]:
        assert oracle.act(x, 1) == max(x, 0.0)
        assert oracle.act(x, 2) == pytest.approx(0.5 * x * (1 + math.erf(x / math.sqrt(2))), abs=1e-15)
        assert oracle.act(x, 3) == pytest.approx(
            0.5 * x * (1 + math.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3))), abs=1e-15)
        assert oracle.act(x, 4) == pytest.approx(1 / (1 + math.exp(-x)), abs=1e-15)
        assert oracle.act(x, 5) == pytest.approx(x / (1 + math.exp(-x)), abs=1e-15)
        assert oracle.act(x, 6) == pytest.approx(x * min(max(x / 6 + 0.5, 0), 1), abs=1e-15)
        assert oracle.act(x, 7, 0.2, 0.5) == pytest.approx(min(max(0.2 * x + 0.5, 0), 1), abs=1e-15)
        assert oracle.act(x, 8, -1.0, 2.0) == min(max(x, -1.0), 2.0)
        assert oracle.act(x, 9, 0.01) == (x * 0.01 if x < 0 else x)
    # GELU's defining values
    assert oracle.act(0.0, 2) == 0.0
    assert oracle.act(1.0, 2) == pytest.approx(0.8413447460685429, abs=1e-15)


def test_gemv_bf16_matches_float64_dot():
    rng = np.random.default_rng(7)
    x = rng.normal(size=(3, 257)).astype(np.float32)
    w = oracle.f32_to_bf16(rng.normal(scale=0.02, size=(31, 257)).astype(np.float32))
    ref = x.astype(np.float64) @ oracle.bf16_to_f32(w).astype(np.float64).T
    np.testing.assert_allclose(oracle.gemv_bf16(x, w), ref, rtol=0, atol=1e-5 * math.sqrt(257))


def test_qgemm_ref_matches_python_ints():
    rng = np.random.default_rng(11)
    a = rng.integers(0, 256, (5, 19), dtype=np.uint8)
    b = rng.integers(-128, 128, (19, 7), dtype=np.int8)
    want = [[sum(int(a[i, p]) * int(b[p, j]) for p in range(19)) for j in range(7)] for i in range(5)]
    assert np.array_equal(oracle.qgemm_ref(a, b), np.array(want, np.int32))


def test_matmul_integer_kat_both_routes():
    k = KATS["matmul_integer"]
    a = np.array(k["A"], np.uint8).reshape(k["m"], k["k"])
    b = np.array(k["B"], np.int8).reshape(k["k"], k["n"])
    want = np.array(k["Y"], np.int32)
    assert np.array_equal(oracle.matmul_integer(a, b, k["za"]), want)
    assert np.array_equal(oracle.matmul_integer(a, b, k["za"], shifted=True), want)
    # planted mistake: a wrong zero point (the -za·colSum correction dropped)
    assert not np.array_equal(oracle.matmul_integer(a, b, 0), want)


def test_matmul_integer_s8_and_int64_brute_force():
    rng = np.random.default_rng(13)
    for dt, za in [(np.uint8, 128), (np.uint8, 3), (np.int8, -7), (np.int8, 0)]:
        lo, hi = (0, 256) if dt == np.uint8 else (-128, 128)
        a = rng.integers(lo, hi, (11, 70)).astype(dt)
        b = rng.integers(-127, 128, (70, 9)).astype(np.int8)
        want = ((a.astype(np.int64) - za) @ b.astype(np.int64)).astype(np.int32)
        assert np.array_equal(oracle.matmul_integer(a, b, za), want)
        assert np.array_equal(oracle.matmul_integer(a, b, za, shifted=True), want)


def test_qlinear_requant_kats():
    """QLinearMatMul requantisation against the golden cases (reference test scales; exact .5 ties, s8 saturation)."""
    kr = KATS["qlinear_ref"]
    mult = oracle.qlinear_mult(kr["sa"], kr["sb"], kr["sy"])
    got = oracle.qlinear_requant(np.array(kr["raw"], np.int32), mult, kr["zy"], kr["u8"])
    assert np.array_equal(got.astype(np.int64), np.array(kr["Y"], np.int64))
    # the same product through the whole op, from the matmul_integer inputs
    km = KATS["matmul_integer"]
    a = np.array(km["A"], np.uint8).reshape(km["m"], km["k"])
    b = np.array(km["B"], np.int8).reshape(km["k"], km["n"])
    full = oracle.qlinear_matmul(a, b, km["za"], kr["sa"], kr["sb"], kr["sy"], kr["zy"], True)
    assert np.array_equal(full.reshape(-1).astype(np.int64), np.array(kr["Y"], np.int64))

    kt = KATS["qlinear_ties"]
    a2 = np.array(kt["A"], np.uint8).reshape(kt["m"], kt["k"])
    b2 = np.array(kt["B"], np.int8).reshape(kt["k"], kt["n"])
    raw = np.array(kt["raw"], np.int32)
    mn = kt["m"] * kt["n"]
    assert np.array_equal(oracle.matmul_integer(a2, b2, kt["za"]).reshape(-1), raw[:mn])
    mult2 = oracle.qlinear_mult(kt["sa"], kt["sb"], kt["sy"])
    assert mult2 == 0.0625
    want = np.array(kt["Y"], np.int64)
    assert np.array_equal(oracle.qlinear_requant(raw, mult2, kt["zy"], kt["u8"]).astype(np.int64), want)

    # planted mistakes the cases must reject: rounding half away from zero, and truncation toward zero
    u = raw.astype(np.float32) * np.float32(mult2) + np.float32(kt["zy"])
    away = np.clip(np.sign(u) * np.floor(np.abs(u) + 0.5), -128, 127).astype(np.int64)
    assert not np.array_equal(away, want)
    trunc = np.clip(np.trunc(u), -128, 127).astype(np.int64)
    assert not np.array_equal(trunc, want)


def _np_quantize_i8g(w):
    """quantizeI8G restated independently with vectorised numpy float32 (IEEE division, rint = half-even)."""
    g = w.reshape(w.shape[0], -1, 64).astype(np.float32)
    s = (np.abs(g).max(axis=2) / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(s[..., None] != 0, np.clip(np.rint(g / s[..., None]), -127, 127), 0)
    return q.astype(np.int8).reshape(w.shape), s


def _np_quantize_x16(x):
    g = x.reshape(-1, 64).astype(np.float32)
    s = (np.abs(g).max(axis=1) / np.float32(16256)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = (np.float32(1) / s).astype(np.float32)
        q = np.where(s[:, None] != 0, np.clip(np.rint((g * inv[:, None]).astype(np.float32)), -16256, 16256), 0)
    q = q.astype(np.int64)
    h = (q + 64) >> 7
    return h.astype(np.int8).reshape(-1), (q - h * 128).astype(np.int8).reshape(-1), s, q.reshape(-1)


def test_quantize_i8g_kats_and_numpy():
    """quantizeI8G: exact-grid groups, .5 ties and a zero group by hand; numpy restatement bit for bit."""
    g1 = np.arange(-63, 65, 2, dtype=np.float32)[:64]          # odd integers, max |w| = 63
    g1[0] = -127.0                                               # max 127 → s = 1, q = w
    g2 = np.array([254.0, 3.0, 5.0, -3.0, -5.0, 7.0] + [2.0] * 58, np.float32)  # s = 2: 1.5→2, 2.5→2, 3.5→4
    w = np.stack([np.concatenate([g1, g2, np.zeros(64, np.float32)])])
    q, s = oracle.quantize_i8g(w)
    assert s.tolist() == [[1.0, 2.0, 0.0]]
    assert np.array_equal(q[0, :64], g1.astype(np.int8))
    assert q[0, 64:70].tolist() == [127, 2, 2, -2, -2, 4]
    assert not q[0, 128:].any()
    rng = np.random.default_rng(41)
    w = (rng.normal(0, 0.02, (37, 256)) * rng.uniform(0.1, 10, (37, 1))).astype(np.float32)
    q, s = oracle.quantize_i8g(w)
    qn, sn = _np_quantize_i8g(w)
    assert np.array_equal(q, qn) and np.array_equal(s, sn)
    assert np.abs(q.astype(np.int32)).max() <= 127
    err = np.abs(w.reshape(37, 4, 64) - s[..., None] * q.reshape(37, 4, 64).astype(np.float32))
    assert np.all(err <= 0.5 * s[..., None] * (1 + 1e-5))


def test_quantize_x16_invariants_and_numpy():
    rng = np.random.default_rng(43)
    x = (rng.normal(0, 1, 512) * np.repeat(rng.uniform(0.01, 100, 8), 64)).astype(np.float32)
    x[64:128] = 0.0                                              # a zero group
    xh, xl, sx = oracle.quantize_x16(x)
    nh, nl, ns, q = _np_quantize_x16(x)
    assert np.array_equal(xh, nh) and np.array_equal(xl, nl) and np.array_equal(sx, ns)
    assert np.array_equal(128 * xh.astype(np.int64) + xl, q)
    assert xl.min() >= -64 and xl.max() <= 63 and np.abs(q).max() <= 16256
    assert sx[1] == 0 and not xh[64:128].any() and not xl[64:128].any()
    # planted mistake: the low part taken against 127·h instead of 128·h breaks the split
    assert not np.array_equal(127 * xh.astype(np.int64) + xl, q)


def test_dot_q8_exact_chain():
    """dotQ8Ref: exact int32 group sums (Python ints), then the f32 chain in group order (numpy float32 scalars)."""
    rng = np.random.default_rng(47)
    k = 384
    w = rng.integers(-127, 128, k).astype(np.int8)
    x = rng.normal(0, 1, k).astype(np.float32)
    xh, xl, sx = oracle.quantize_x16(x)
    sw = rng.uniform(1e-4, 1e-2, k // 64).astype(np.float32)
    acc = np.float32(0)
    for g in range(k // 64):
        p = sum(int(w[i]) * (128 * int(xh[i]) + int(xl[i])) for i in range(g * 64, (g + 1) * 64))
        acc = np.float32(acc + np.float32(np.float32(sx[g] * sw[g]) * np.float32(p)))
    assert oracle.dot_q8(w, xh, xl, sx, sw) == float(acc)
    # planted mistake: the high part without its 128 weight
    bad = sum(float(sx[g] * sw[g]) * sum(int(w[i]) * (int(xh[i]) + int(xl[i])) for i in range(g * 64, g * 64 + 64))
              for g in range(k // 64))
    assert abs(bad - float(acc)) > 1e-3 * abs(float(acc))


def test_gemv_i8g_is_close_to_float64():
    """GemvI8G: the documented approximation (weights' int8 rounding) against the float64 product."""
    rng = np.random.default_rng(53)
    m, n, k = 3, 29, 256
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    c = rng.normal(0, 1, n).astype(np.float32)
    q, s = oracle.quantize_i8g(w)
    y = oracle.gemv_i8g(x, q, s, 0.5, 2.0, c)
    deq = (q.reshape(n, 4, 64).astype(np.float64) * s[..., None]).reshape(n, k)
    rows = []
    for i in range(m):
        xh, xl, sx = oracle.quantize_x16(x[i])
        xq = (np.repeat(sx, 64).astype(np.float64) * (128 * xh.astype(np.float64) + xl))
        rows.append(0.5 * (deq @ xq) + 2.0 * c)
    want = np.array(rows)
    assert np.all(np.abs(y - want) <= 1e-5 * math.sqrt(k) * (1 + np.abs(want)))   # TestGemmInt8Weight's bound
    assert np.max(np.abs(y - (0.5 * x.astype(np.float64) @ w.T.astype(np.float64) + 2.0 * c))) < 0.02


def test_dequantize_kats():
    for name, dt in [("dequantize_u8", np.uint8), ("dequantize_i8", np.int8)]:
        k = KATS[name]
        got = oracle.dequantize_linear(np.array(k["x"], dt), np.array(k["scale"], np.float32),
                                       zp=np.array(k["zp"], dt))
        assert np.array_equal(got, np.array(k["y"], np.float32))


def test_dequantize_per_axis_matches_numpy_f32():
    rng = np.random.default_rng(17)
    x = rng.integers(-2**20, 2**20, (6, 5, 4)).astype(np.int32)
    sc = rng.uniform(0.001, 0.01, 5).astype(np.float32)
    want = (x.astype(np.float32) * sc[None, :, None]).astype(np.float32)
    assert np.array_equal(oracle.dequantize_linear(x, sc, inner=4), want)


def test_bf16_widening_and_scalar_rounding_agree():
    """orc_bf16_to_f32 is the exact widening (bits << 16, every pattern incl. NaN
    payloads and subnormals); the scalar orc_f32_to_bf16 equals the elementwise
    orc_f32_to_bf16_n the tests above pin."""
    lib = oracle.lib()
    hs = np.arange(0, 1 << 16, 97, dtype=np.uint32)
    for h in hs:
        got = np.float32(lib.orc_bf16_to_f32(int(h))).view(np.uint32)
        want = np.uint32(h) << np.uint32(16)
        if np.isnan(np.uint32(want).view(np.float32)):
            assert np.isnan(np.uint32(got).view(np.float32)), hex(int(h))
        else:
            assert got == want, hex(int(h))
    rng = np.random.default_rng(11)
    xs = rng.normal(0, 1e3, 257).astype(np.float32)
    vec = oracle.f32_to_bf16(xs)
    assert all(int(lib.orc_f32_to_bf16(float(x))) == int(v) for x, v in zip(xs, vec))
