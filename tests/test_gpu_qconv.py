"""GPU parity of QLinearConv (ingot_rocm_qlinear_conv and the QLinearConv@10 op).

Bar: bit-exact against the oracle's restatement of the reference
(qlinearConvOp.Run, ops/quant.go:343-706), on the geometries of the
reference's TestQLinearConv (ops/quant_optest_test.go:133-192) and on larger
shapes that take the im2col → int8 MFMA GEMM route. Both device routes
(direct, GEMM) run every case: INGOT_QCONV_PATH=1 forces the direct kernel,
2 the GEMM.
"""

import numpy as np
import pytest

import oracle
from helpers import announce
from ingot_amd import IngotError
from ingot_amd import _lib as L
from test_oracle_qconv import REF_CFGS

pytestmark = pytest.mark.gpu

DT = {np.dtype(np.uint8): L.DT_U8, np.dtype(np.int8): L.DT_I8}


ROUTES = {"auto": "0", "direct": "1", "gemm": "2"}


@pytest.fixture(params=list(ROUTES))
def route(request):
    return request.param


@pytest.fixture
def qsess(env_session, route):
    """A session whose QLinearConv route is forced (INGOT_QCONV_PATH, read when the session opens)."""
    return env_session(INGOT_QCONV_PATH=ROUTES[route])


def make_case(rng, n, c, h, w, m, kh, kw, g, x_dtype=np.uint8, zx=120, with_bias=True, per_channel=True):
    if x_dtype == np.uint8:
        x = rng.integers(0, 256, (n, c, h, w), dtype=np.uint8)
    else:
        x = rng.integers(-128, 128, (n, c, h, w), dtype=np.int8)
    wt = rng.integers(-128, 128, (m, c // g, kh, kw), dtype=np.int8)
    bias = (rng.integers(0, 2048, m) - 1024).astype(np.int32) if with_bias else None
    xs, ys = 0.02, 0.4
    wsc = (np.float32(0.01) + np.arange(m, dtype=np.float32) * np.float32(0.003)) if per_channel else \
        np.array([0.013], np.float32)
    # keep outputs inside the requant range for wide reductions
    wsc = (wsc / np.float32(max(1.0, np.sqrt(c // g * kh * kw / 9.0)))).astype(np.float32)
    mult = oracle.qconv_mult(xs, wsc, ys, m)
    return x, zx, wt, bias, mult, xs, wsc, ys


def run_conv(sess, x, zx, wt, bias, mult, zy, y_u8, group=1, strides=(1, 1), dilations=(1, 1), pads=(0, 0, 0, 0)):
    n, c, h, w = x.shape
    m, cg, kh, kw = wt.shape
    oh = oracle.conv_out(h, kh, strides[0], dilations[0], pads[0], pads[2])
    ow = oracle.conv_out(w, kw, strides[1], dilations[1], pads[1], pads[3])
    pw = sess.upload_weight(wt.reshape(m, -1), trans=True, pack_dtype=L.DT_I8)
    dx = sess.to_device(x, DT[x.dtype])
    dm = sess.to_device(np.ascontiguousarray(mult, np.float32))
    db = sess.to_device(bias) if bias is not None else None
    y = sess.empty(L.DT_U8 if y_u8 else L.DT_I8, (n, m, max(oh, 0), max(ow, 0)))
    try:
        sess.qlinear_conv(dx, zx, pw, wt.shape, dm, zy, y, bias=db, group=group, strides=strides,
                          dilations=dilations, pads=pads)
        return y.numpy()
    finally:
        for t in (pw, dx, dm, db, y):
            if t is not None:
                t.free()


@pytest.mark.parametrize("cfg", REF_CFGS, ids=[f"c{i}" for i in range(len(REF_CFGS))])
@pytest.mark.parametrize("x_dtype,zx,y_u8,zy", [(np.uint8, 120, True, 17), (np.int8, -7, False, -3)])
def test_reference_geometries(qsess, route, cfg, x_dtype, zx, y_u8, zy):
    sess = qsess
    n, c, h, w, m, kh, kw, g, sh, sw, pt, pl = cfg
    announce(f"qconv ref cfg {cfg} x={np.dtype(x_dtype).name} route={route}")
    rng = np.random.default_rng(hash(cfg) % 2**32)
    x, zx, wt, bias, mult, *_ = make_case(rng, n, c, h, w, m, kh, kw, g, x_dtype, zx)
    kw_ = dict(group=g, strides=(sh, sw), pads=(pt, pl, pt, pl))
    got = run_conv(sess, x, zx, wt, bias, mult, zy, y_u8, **kw_)
    want = oracle.qlinear_conv(x, zx, wt, bias, mult, zy, y_u8, **kw_)
    np.testing.assert_array_equal(got, want)


# Shapes of the GEMM route: several k-tiles, K off the 128 grid, rows off the
# tile grid, groups with a GEMM each, strides, dilations, asymmetric pads, 1×1.
GEMM_CASES = [
    # n, c, h, w, m, kh, kw, g, strides, dilations, pads
    (1, 64, 28, 28, 64, 3, 3, 1, (1, 1), (1, 1), (1, 1, 1, 1)),
    (2, 32, 17, 13, 48, 3, 3, 1, (2, 2), (2, 2), (2, 0, 1, 3)),
    (1, 32, 15, 15, 64, 3, 3, 2, (1, 1), (1, 1), (1, 1, 1, 1)),
    (2, 256, 14, 14, 128, 1, 1, 1, (1, 1), (1, 1), (0, 0, 0, 0)),
    (1, 3, 33, 31, 32, 7, 7, 1, (2, 2), (1, 1), (3, 3, 3, 3)),
    (3, 48, 9, 10, 96, 5, 3, 3, (1, 2), (1, 1), (2, 1, 2, 1)),
    (1, 130, 6, 5, 20, 1, 2, 1, (1, 1), (1, 1), (0, 0, 0, 1)),
]


@pytest.mark.parametrize("case", GEMM_CASES, ids=[f"g{i}" for i in range(len(GEMM_CASES))])
def test_gemm_shapes(qsess, route, case):
    sess = qsess
    n, c, h, w, m, kh, kw, g, st, dl, pads = case
    if route == "direct" and c * h * w * m * kh * kw // g > 5e7:
        pytest.skip("the direct route is covered on the smaller cases")
    announce(f"qconv gemm case {case} route={route}")
    rng = np.random.default_rng(sum(case[:7]))
    for x_dtype, zx, y_u8, zy, with_bias, per_ch in [(np.uint8, 131, True, 9, True, True),
                                                      (np.int8, 4, False, 0, False, False)]:
        x, zx, wt, bias, mult, *_ = make_case(rng, n, c, h, w, m, kh, kw, g, x_dtype, zx, with_bias, per_ch)
        kw_ = dict(group=g, strides=st, dilations=dl, pads=pads)
        got = run_conv(sess, x, zx, wt, bias, mult, zy, y_u8, **kw_)
        want = oracle.qlinear_conv(x, zx, wt, bias, mult, zy, y_u8, **kw_)
        np.testing.assert_array_equal(got, want)
        assert len(np.unique(got)) > 16  # not saturated wholesale


def test_routes_agree_at_size(env_session):
    """A ResNet-stage conv (1×256×56×56 → 256, 3×3, pad 1): GEMM and direct routes are both exact, so they
    agree bit for bit; a slab of output channels is checked against the oracle."""
    announce("qconv routes at size")
    rng = np.random.default_rng(56)
    x, zx, wt, bias, mult, *_ = make_case(rng, 1, 256, 56, 56, 256, 3, 3, 1)
    pads = (1, 1, 1, 1)
    y_gemm = run_conv(env_session(INGOT_QCONV_PATH=2), x, zx, wt, bias, mult, 17, True, pads=pads)
    y_dir = run_conv(env_session(INGOT_QCONV_PATH=1), x, zx, wt, bias, mult, 17, True, pads=pads)
    np.testing.assert_array_equal(y_gemm, y_dir)
    sl = slice(100, 108)
    want = oracle.qlinear_conv(x, zx, wt[sl], bias[sl], mult[sl], 17, True, pads=pads)
    np.testing.assert_array_equal(y_gemm[:, sl], want)
    assert len(np.unique(y_gemm)) > 64


def test_empty_and_degenerate(sess):
    announce("qconv empty")
    rng = np.random.default_rng(0)
    # no images
    x, zx, wt, bias, mult, *_ = make_case(rng, 1, 4, 5, 5, 8, 3, 3, 1)
    got = run_conv(sess, x[:0], zx, wt, bias, mult, 0, True)
    assert got.shape == (0, 8, 3, 3)
    # kernel one wider than the input: OW = (5 − 6)/1 + 1 = 0
    got = run_conv(sess, x, zx, np.ascontiguousarray(np.pad(wt, ((0, 0), (0, 0), (0, 0), (0, 3)))), bias, mult, 0,
                   True)
    assert got.shape == (1, 8, 3, 0)
    # two wider: a negative output size is an error (the reference cannot allocate it)
    with pytest.raises(IngotError, match="negative output size"):
        run_conv(sess, x, zx, np.ascontiguousarray(np.pad(wt, ((0, 0), (0, 0), (0, 0), (0, 4)))), bias, mult, 0,
                 True)
    # 1×1 image, 1×1 kernel, a single channel
    x1 = np.array([[[[200]]]], np.uint8)
    w1 = np.array([[[[-3]]]], np.int8)
    got = run_conv(sess, x1, 100, w1, None, np.array([0.5], np.float32), 7, True)
    np.testing.assert_array_equal(got, oracle.qlinear_conv(x1, 100, w1, None, np.array([0.5], np.float32), 7, True))


def test_zero_point_outside_dtype_declines(sess):
    announce("qconv decline")
    x = np.zeros((1, 1, 3, 3), np.uint8)
    w = np.ones((1, 1, 1, 1), np.int8)
    with pytest.raises(IngotError, match="outside the range"):
        run_conv(sess, x, -5, w, None, np.ones(1, np.float32), 0, True)


# ---- operator layer ----

def dev(sess, arr, code=None):
    return sess.to_device(np.ascontiguousarray(arr), code)


def op_inputs(sess, x, zx, wt, wsc, xs, ys, zy, y_dtype, bias=None):
    f32 = lambda v: dev(sess, np.asarray(v, np.float32).reshape(-1))
    ins = [dev(sess, x, DT[x.dtype]), f32([xs]), dev(sess, np.array([zx], x.dtype), DT[x.dtype]),
           dev(sess, wt, L.DT_I8), f32(wsc), dev(sess, np.zeros(wt.shape[0], np.int8), L.DT_I8), f32([ys]),
           dev(sess, np.array([zy], y_dtype), DT[np.dtype(y_dtype)])]
    if bias is not None:
        ins.append(dev(sess, bias, L.DT_I32))
    return ins


def run_op(op, *ins):
    outs = op.run(*ins)
    res = [o.numpy() for o in outs]
    for o in outs:
        o.free()
    return res


@pytest.mark.parametrize("cfg", REF_CFGS, ids=[f"c{i}" for i in range(len(REF_CFGS))])
def test_op_reference_geometries(sess, cfg):
    """TestQLinearConv through the op (ops/quant_optest_test.go:133-192): NCHW u8 in, u8 out, per-channel
    w_scale, int32 bias, attributes group/strides/pads/kernel_shape."""
    n, c, h, w, m, kh, kw, g, sh, sw, pt, pl = cfg
    announce(f"qconv op cfg {cfg}")
    rng = np.random.default_rng(7 + sum(cfg))
    x, zx, wt, bias, _, xs, wsc, ys = make_case(rng, n, c, h, w, m, kh, kw, g)
    op = sess.op("QLinearConv", 10, {"group": g, "strides": (sh, sw), "pads": (pt, pl, pt, pl),
                                     "kernel_shape": (kh, kw)})
    (y,) = run_op(op, *op_inputs(sess, x, zx, wt, wsc, xs, ys, 17, np.uint8, bias))
    mult = oracle.qconv_mult(xs, wsc, ys, m)
    want = oracle.qlinear_conv(x, zx, wt, bias, mult, 17, True, group=g, strides=(sh, sw), pads=(pt, pl, pt, pl))
    assert y.dtype == np.uint8
    np.testing.assert_array_equal(y, want)
    op.free()


@pytest.mark.parametrize("auto_pad", ["SAME_UPPER", "SAME_LOWER", "VALID"])
def test_op_auto_pad_and_s8_output(sess, auto_pad):
    announce(f"qconv op auto_pad {auto_pad}")
    rng = np.random.default_rng(99)
    x, zx, wt, _, _, xs, wsc, ys = make_case(rng, 2, 24, 11, 8, 32, 4, 3, 1, np.int8, -9, per_channel=False)
    op = sess.op("QLinearConv", 10, {"auto_pad": auto_pad, "strides": (2, 1), "dilations": (1, 2)})
    (y,) = run_op(op, *op_inputs(sess, x, zx, wt, wsc, xs, ys, -4, np.int8))
    pads = oracle.resolve_pads(auto_pad, (0, 0, 0, 0), (2, 1), (1, 2), 11, 8, 4, 3)
    want = oracle.qlinear_conv(x, zx, wt, None, oracle.qconv_mult(xs, wsc, ys, 32), -4, False, strides=(2, 1),
                               dilations=(1, 2), pads=pads)
    assert y.dtype == np.int8
    np.testing.assert_array_equal(y, want)
    op.free()


def test_op_errors(sess):
    announce("qconv op errors")
    rng = np.random.default_rng(1)
    x, zx, wt, bias, _, xs, wsc, ys = make_case(rng, 1, 4, 6, 6, 4, 3, 3, 1)
    ins = op_inputs(sess, x, zx, wt, wsc, xs, ys, 0, np.uint8, bias)
    op = sess.op("QLinearConv", 10, {"pads": (1, 1, 1, 1)})
    with pytest.raises(IngotError, match="need 8-9 inputs"):
        op.run(*ins[:5])
    with pytest.raises(IngotError, match="non-zero weight zero_point"):
        op.run(*(ins[:5] + [dev(sess, np.ones(4, np.int8), L.DT_I8)] + ins[6:]))
    with pytest.raises(IngotError, match="only s8 weights"):
        op.run(*(ins[:3] + [dev(sess, wt.view(np.uint8), L.DT_U8)] + ins[4:]))
    with pytest.raises(IngotError, match="per-tensor activation/output quantization only"):
        op.run(*(ins[:2] + [dev(sess, np.array([1, 2], np.uint8), L.DT_U8)] + ins[3:]))
    with pytest.raises(IngotError, match="only 2-D conv"):
        op.run(*([dev(sess, x.reshape(1, 4, 36), L.DT_U8)] + ins[1:]))
    op_g = sess.op("QLinearConv", 10, {"group": 3})
    with pytest.raises(IngotError, match="channel mismatch"):
        op_g.run(*ins)
    op_p = sess.op("QLinearConv", 10, {"auto_pad": "BOGUS"})
    with pytest.raises(IngotError, match="unsupported auto_pad"):
        op_p.run(*ins)
    with pytest.raises(IngotError, match="only 1-D and 2-D conv supported"):
        sess.op("QLinearConv", 10, {"strides": (1, 1, 1, 1)})
    for o in (op, op_g, op_p):
        o.free()
