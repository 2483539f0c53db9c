"""Pins the oracle's QLinearConv restatement (oracle.qlinear_conv).

The oracle follows the reference's own route (ops/quant.go:343-706): u8
activations shifted to s8, taps outside the image filled with the shifted
zero point, an s8 product, then the −zx′·ΣW + bias correction and the
requantisation. The checks below reach the same numbers by other routes:

* a vectorised numpy closed form, y = requant(Σ w·(x − zx) + bias), where
  padded taps contribute exactly zero (the expectation of the reference's
  qlinearConvRef, ops/quant_optest_test.go:94-131), run over the nine
  geometries of TestQLinearConv (ops/quant_optest_test.go:133-147);
* a 1×1 convolution equals QLinearMatMul of the transposed activations
  (oracle.qlinear_matmul, pinned separately by golden requant cases);
* a one-tap kernel reproduces requant(x − zx + bias) per pixel;
* planted mistakes (padding with 0 instead of the zero point, a transposed
  kernel, a wrong group mapping) fail against the oracle.
"""
import numpy as np
import pytest

import oracle


def _requant(v: np.ndarray, mult: np.ndarray, zy: int, u8: bool) -> np.ndarray:
    # float32(v)·mult and + zy rounded separately, half to even, saturate
    t = v.astype(np.float32) * mult.astype(np.float32)
    u = (t + np.float32(zy)).astype(np.float32)
    r = np.rint(u)
    lo, hi = (0, 255) if u8 else (-128, 127)
    return np.clip(r, lo, hi).astype(np.uint8 if u8 else np.int8)


def closed_form(x, zx, w, bias, mult, zy, u8, group=1, strides=(1, 1), dil=(1, 1), pads=(0, 0, 0, 0),
                pad_value=None, swap_khkw=False, group_shift=0):
    """Σ w·(x − zx) + bias with padded taps at zero, then the requantisation.
    pad_value / swap_khkw / group_shift plant mistakes for the negative checks."""
    n, c, h, wd = x.shape
    m, cg, kh, kw = w.shape
    pt, pl, pb, pr = pads
    oh = oracle.conv_out(h, kh, strides[0], dil[0], pt, pb)
    ow = oracle.conv_out(wd, kw, strides[1], dil[1], pl, pr)
    xd = x.astype(np.int64) - zx
    fill = 0 if pad_value is None else pad_value - zx
    xp = np.full((n, c, h + pt + pb, wd + pl + pr), fill, np.int64)
    xp[:, :, pt:pt + h, pl:pl + wd] = xd
    mg = m // group
    wk = w.astype(np.int64)
    if swap_khkw:
        wk = wk.reshape(m, cg, kw, kh).transpose(0, 1, 3, 2)
    acc = np.zeros((n, m, oh, ow), np.int64)
    for g in range(group):
        gi = (g + group_shift) % group
        xs = xp[:, gi * cg:(gi + 1) * cg]
        for i in range(kh):
            for j in range(kw):
                win = xs[:, :, i * dil[0]:i * dil[0] + (oh - 1) * strides[0] + 1:strides[0],
                         j * dil[1]:j * dil[1] + (ow - 1) * strides[1] + 1:strides[1]]
                acc[:, g * mg:(g + 1) * mg] += np.einsum("nchw,mc->nmhw", win, wk[g * mg:(g + 1) * mg, :, i, j])
    if bias is not None:
        acc += np.asarray(bias, np.int64)[None, :, None, None]
    v = ((acc + 2**31) % 2**32 - 2**31).astype(np.int32)
    return _requant(v, np.asarray(mult, np.float32)[None, :, None, None], zy, u8)


# The geometries of TestQLinearConv (ops/quant_optest_test.go:135-146):
# N, C, H, W, M, KH, KW, G, sh, sw, pt, pl (pads symmetric).
REF_CFGS = [
    (1, 3, 8, 9, 4, 3, 3, 1, 1, 1, 1, 1),
    (2, 4, 7, 7, 6, 3, 3, 1, 2, 2, 0, 0),
    (1, 8, 6, 6, 8, 3, 3, 8, 1, 1, 1, 1),
    (1, 6, 9, 11, 6, 5, 5, 6, 1, 1, 2, 2),
    (2, 8, 10, 9, 8, 3, 3, 8, 2, 2, 1, 1),
    (1, 6, 11, 12, 6, 5, 5, 6, 2, 2, 2, 2),
    (1, 4, 8, 8, 4, 3, 3, 4, 1, 1, 0, 0),
    (1, 6, 5, 5, 4, 1, 1, 2, 1, 1, 0, 0),
    (1, 16, 9, 9, 8, 3, 3, 1, 1, 1, 1, 1),
]


def ref_case(cfg, rng, x_dtype=np.uint8, zx=120, zy=17, with_bias=True):
    n, c, h, w, m, kh, kw, g, sh, sw, pt, pl = cfg
    if x_dtype == np.uint8:
        x = rng.integers(0, 256, (n, c, h, w), dtype=np.uint8)
    else:
        x = rng.integers(-128, 128, (n, c, h, w), dtype=np.int8)
    wt = rng.integers(-128, 128, (m, c // g, kh, kw), dtype=np.int8)
    bias = (rng.integers(0, 2048, m) - 1024).astype(np.int32) if with_bias else None
    xs, ys = np.float32(0.02), np.float32(0.4)
    wsc = (np.float32(0.01) + np.arange(m, dtype=np.float32) * np.float32(0.003)).astype(np.float32)
    mult = oracle.qconv_mult(float(xs), wsc, float(ys), m)
    return dict(x=x, zx=zx, w=wt, bias=bias, mult=mult, zy=zy, group=g, strides=(sh, sw), pads=(pt, pl, pt, pl))


@pytest.mark.parametrize("cfg", REF_CFGS)
@pytest.mark.parametrize("x_dtype,zx", [(np.uint8, 120), (np.int8, -7)])
@pytest.mark.parametrize("u8_out", [True, False])
def test_qlinear_conv_closed_form(cfg, x_dtype, zx, u8_out):
    rng = np.random.default_rng(23 + cfg[1] * 7 + cfg[4])
    k = ref_case(cfg, rng, x_dtype, zx, zy=17 if u8_out else -3)
    got = oracle.qlinear_conv(k["x"], k["zx"], k["w"], k["bias"], k["mult"], k["zy"], u8_out, group=k["group"],
                              strides=k["strides"], pads=k["pads"])
    want = closed_form(k["x"], k["zx"], k["w"], k["bias"], k["mult"], k["zy"], u8_out, k["group"], k["strides"],
                       pads=k["pads"])
    assert got.shape == want.shape
    np.testing.assert_array_equal(got, want)
    # the outputs are not saturated wholesale (the case exercises the requant range)
    assert len(np.unique(got)) > 8


def test_qlinear_conv_dilation_asymmetric_pads_no_bias():
    rng = np.random.default_rng(5)
    x = rng.integers(0, 256, (2, 6, 13, 10), dtype=np.uint8)
    w = rng.integers(-128, 128, (4, 3, 3, 2), dtype=np.int8)
    mult = oracle.qconv_mult(0.03, np.full(4, 0.02, np.float32), 0.5, 4)
    for pads in [(0, 1, 2, 0), (2, 0, 1, 3)]:
        got = oracle.qlinear_conv(x, 131, w, None, mult, 9, True, group=2, strides=(2, 1), dilations=(2, 3),
                                  pads=pads)
        want = closed_form(x, 131, w, None, mult, 9, True, 2, (2, 1), (2, 3), pads)
        np.testing.assert_array_equal(got, want)


def test_qlinear_conv_pointwise_is_qlinear_matmul():
    # 1×1, stride 1, no padding: y[n,m,p] = QLinearMatMul(xᵀ, wᵀ) with per-tensor scales
    rng = np.random.default_rng(11)
    c, h, wd, m = 20, 5, 7, 9
    x = rng.integers(0, 256, (1, c, h, wd), dtype=np.uint8)
    w = rng.integers(-128, 128, (m, c, 1, 1), dtype=np.int8)
    sa, sb, sy, za, zy = 0.1, 0.05, 0.7, 110, 3
    mult = oracle.qconv_mult(sa, np.array([sb], np.float32), sy, m)
    got = oracle.qlinear_conv(x, za, w, None, mult, zy, True)
    a = np.ascontiguousarray(x.reshape(c, h * wd).T)
    b = np.ascontiguousarray(w.reshape(m, c).T)
    want = oracle.qlinear_matmul(a, b, za, sa, sb, sy, zy, True)
    np.testing.assert_array_equal(got.reshape(m, h * wd).T, want)


def test_qlinear_conv_one_tap_kernel():
    # depthwise, only the centre tap set to 1: y = requant(x − zx + bias)
    rng = np.random.default_rng(3)
    c = 5
    x = rng.integers(0, 256, (1, c, 6, 4), dtype=np.uint8)
    w = np.zeros((c, 1, 3, 3), np.int8)
    w[:, 0, 1, 1] = 1
    bias = np.arange(c, dtype=np.int32) * 7 - 10
    mult = np.full(c, np.float32(0.75), np.float32)
    got = oracle.qlinear_conv(x, 100, w, bias, mult, 128, True, group=c, pads=(1, 1, 1, 1))
    v = x.astype(np.int32) - 100 + bias[None, :, None, None]
    want = oracle.qlinear_requant(v.reshape(-1), 0.75, 128, True).reshape(x.shape)
    np.testing.assert_array_equal(got, want)


def test_qlinear_conv_planted_mistakes_fail():
    rng = np.random.default_rng(29)
    k = ref_case((1, 4, 7, 6, 4, 3, 2, 2, 1, 1, 1, 1), rng)
    got = oracle.qlinear_conv(k["x"], k["zx"], k["w"], k["bias"], k["mult"], k["zy"], True, group=2,
                              pads=k["pads"])
    base = dict(group=2, strides=(1, 1), pads=k["pads"])
    ok = closed_form(k["x"], k["zx"], k["w"], k["bias"], k["mult"], k["zy"], True, **base)
    np.testing.assert_array_equal(got, ok)
    for plant in [dict(pad_value=0), dict(swap_khkw=True), dict(group_shift=1)]:
        bad = closed_form(k["x"], k["zx"], k["w"], k["bias"], k["mult"], k["zy"], True, **base, **plant)
        assert not np.array_equal(got, bad), plant


def test_qlinear_conv_int32_wraparound():
    # sums past 2^31 wrap like the reference's int32 accumulators
    x = np.full((1, 1, 1, 1), 255, np.uint8)
    w = np.full((1, 1, 1, 1), -128, np.int8)
    bias = np.array([2**31 - 1], np.int32)
    mult = np.array([1e-9], np.float32)
    got = oracle.qlinear_conv(x, 0, w, bias, mult, 0, False)
    v = np.array([(255 * -128 + 2**31 - 1 + 2**31) % 2**32 - 2**31], np.int64).astype(np.int32)
    np.testing.assert_array_equal(got.reshape(-1), oracle.qlinear_requant(v, 1e-9, 0, False))


def test_conv_out_and_resolve_pads():
    # convOut truncates toward zero (Go division)
    assert oracle.conv_out(5, 3, 1, 1, 0, 0) == 3
    assert oracle.conv_out(7, 3, 2, 1, 1, 1) == 4
    assert oracle.conv_out(2, 5, 2, 1, 0, 0) == 0  # (2 − 5)/2 = −1 → 0
    # SAME_*: ceil(in/stride) outputs; the odd total goes to the end (UPPER) or start (LOWER)
    assert oracle.resolve_pads("SAME_UPPER", (0,) * 4, (1, 1), (1, 1), 4, 4, 2, 2) == (0, 0, 1, 1)
    assert oracle.resolve_pads("SAME_LOWER", (0,) * 4, (1, 1), (1, 1), 4, 4, 2, 2) == (1, 1, 0, 0)
    assert oracle.resolve_pads("SAME_UPPER", (0,) * 4, (2, 2), (1, 1), 5, 5, 3, 3) == (1, 1, 1, 1)
    assert oracle.resolve_pads("VALID", (1, 2, 3, 4), (1, 1), (1, 1), 9, 9, 3, 3) == (0, 0, 0, 0)
    assert oracle.resolve_pads("NOTSET", (1, 2, 3, 4), (1, 1), (1, 1), 9, 9, 3, 3) == (1, 2, 3, 4)
    rng = np.random.default_rng(1)
    for _ in range(200):
        n, k, s, d = (int(v) for v in (rng.integers(1, 40), rng.integers(1, 6), rng.integers(1, 4),
                                        rng.integers(1, 3)))
        for mode in ("SAME_UPPER", "SAME_LOWER"):
            pt, _, pb, _ = oracle.resolve_pads(mode, (0,) * 4, (s, 1), (d, 1), n, 1, k, 1)
            assert abs(pt - pb) <= 1 and (pb >= pt) == (mode == "SAME_UPPER" or pt == pb)
            out = oracle.conv_out(n, k, s, d, pt, pb)
            if (out - 1) * s + d * (k - 1) + 1 >= n:  # the window reaches the last input
                assert out == -(-n // s)
    with pytest.raises(ValueError):
        oracle.resolve_pads("BOGUS", (0,) * 4, (1, 1), (1, 1), 4, 4, 2, 2)
