"""GPU graph session: the MLP block of the planning tests run end to end on the device.

Reference behaviour mirrored: TestMatMulBias-style fused bias (graph/fuse_matmul_bias.go), planHalf's epilogue
activations, and GPUBF16's bf16 products with the bound of TestGPUHalfActivations
(graph/gpuhalf_test.go:85-151: 0.03·max|y| against the f32 result, bit-identical across runs).
"""
import math

import numpy as np
import pytest

from helpers import announce
from ingot_amd import Graph, IngotError
from ingot_amd import _lib as L

pytestmark = pytest.mark.gpu

MLP = """
input x f32 {m},{d}
const W1 f32 {d},{h}
const b1 f32 {h}
const W2 f32 {h},{d}
const b2 f32 {d}
node MatMul x,W1 -> h1
node Add h1,b1 -> h2
node ingot.Gelu h2 -> h3
node MatMul h3,W2 -> h4
node Add b2,h4 -> h5
node Relu h5 -> y
output y
"""


def mlp_case(sess, m=128, d=768, h=3072, seed=11):
    rng = np.random.default_rng(seed)
    ws = {"W1": rng.normal(0, 1 / math.sqrt(d), (d, h)), "b1": rng.normal(0, 0.1, h),
          "W2": rng.normal(0, 1 / math.sqrt(h), (h, d)), "b2": rng.normal(0, 0.1, d)}
    ws = {k: v.astype(np.float32) for k, v in ws.items()}
    x = rng.normal(0, 1, (m, d)).astype(np.float32)
    dev = {k: sess.to_device(v) for k, v in ws.items()}
    # float64 chain
    erf = np.vectorize(math.erf)
    t = x.astype(np.float64) @ ws["W1"] + ws["b1"]
    t = 0.5 * t * (1 + erf(t / math.sqrt(2)))
    y = np.maximum(t @ ws["W2"] + ws["b2"], 0)
    return MLP.format(m=m, d=d, h=h), dev, sess.to_device(x), y


def run_graph(sess, text, dev, x, flags, runs=1):
    g = Graph(sess, text)
    for k, v in dev.items():
        g.bind(k, v)
    g.compile(flags)
    outs = []
    for _ in range(runs):
        (y,) = g.run({"x": x})
        assert y.dtype == L.DT_F32
        outs.append(y.numpy())
        y.free()
    st = g.stats()
    g.free()
    return outs, st


def test_graph_mlp_f32_fusions(sess):
    announce("graph mlp f32")
    text, dev, x, want = mlp_case(sess)
    (y_bias,), st = run_graph(sess, text, dev, x, L.GRAPH_FUSE_BIAS)
    assert st["fuse-matmul-bias"] == 2 and st["steps"] == 4
    assert np.max(np.abs(y_bias - want)) <= 1e-4 * max(1.0, np.max(np.abs(want)))
    # the activations in the products' stores: the same f32 values as the separate activation ops
    outs, st = run_graph(sess, text, dev, x, L.GRAPH_FUSE_BIAS | L.GRAPH_FUSE_ACT, runs=3)
    assert st["fuse-act"] == 2 and st["steps"] == 2
    for y in outs:
        assert np.array_equal(y, y_bias)


def test_graph_mlp_gpubf16(sess):
    announce("graph mlp gpubf16")
    text, dev, x, want = mlp_case(sess)
    outs, st = run_graph(sess, text, dev, x, L.GRAPH_FUSE_BIAS | L.GRAPH_FUSE_ACT | L.GRAPH_HALF, runs=3)
    assert st["half-out"] == 1
    d = np.max(np.abs(outs[0] - want))
    assert d <= 0.03 * np.max(np.abs(want)) and not math.isnan(d)
    assert d > 1e-4 * np.max(np.abs(want))  # bf16 operands really used
    assert all(np.array_equal(o, outs[0]) for o in outs[1:])


def test_graph_unfused_add_is_declined(sess):
    announce("graph unsupported op")
    text, dev, x, _ = mlp_case(sess, m=8, d=64, h=128)
    g = Graph(sess, text)
    for k, v in dev.items():
        g.bind(k, v)
    with pytest.raises(IngotError, match="Add"):
        g.compile(0)
    g.free()
    with pytest.raises(IngotError, match="not fed"):
        g2 = Graph(sess, text)
        for k, v in dev.items():
            g2.bind(k, v)
        g2.compile(L.GRAPH_FUSE_BIAS)
        g2.run({})


DYN_RHS = """
input x f32 {m},{k}
input z f32 {k},{n}
node Relu z -> rz
node MatMul x,rz -> y
output y
"""


def test_graph_dynamic_rhs_packed_per_run(sess):
    """MatMul(x, Relu(z)) with a 2-D z that is a graph input, not a constant: the right operand is a pooled
    intermediate that comes back at the same device address with new contents on the next run, so it must be
    packed per run (the reference's GPU session caches only graph constants: graph/gpuops_darwin_arm64.go:610-629).
    Two runs with different z, each against the float64 product (f32 tolerance 1e-5·sqrt(K) relative,
    kernels/gemm/gemm_test.go:34)."""
    announce("graph dynamic rhs")
    m, k, n = 96, 320, 200
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    g = Graph(sess, DYN_RHS.format(m=m, k=k, n=n))
    g.compile(L.GRAPH_FUSE_BIAS | L.GRAPH_FUSE_ACT)
    dx = sess.to_device(x)
    for run in range(2):
        z = rng.normal(0, 1, (k, n)).astype(np.float32)
        dz = sess.to_device(z)
        (y,) = g.run({"x": dx, "z": dz})
        want = x.astype(np.float64) @ np.maximum(z, 0).astype(np.float64)
        got = y.numpy()
        y.free()
        dz.free()
        err = np.max(np.abs(got - want)) / max(1.0, np.max(np.abs(want)))
        assert err <= 1e-5 * math.sqrt(k), f"run {run}: relative error {err:.3e}"
    g.free()


def _session_work(seed, runs):
    """One thread's work on a session of its own: the MLP graph under both plans and a decode GEMV, `runs`
    times each; returns every output."""
    from ingot_amd import Session

    s = Session(0)
    try:
        text, dev, x, _ = mlp_case(s, m=64, seed=seed)
        graphs = []
        for flags in (L.GRAPH_FUSE_BIAS | L.GRAPH_FUSE_ACT, L.GRAPH_FUSE_BIAS | L.GRAPH_FUSE_ACT | L.GRAPH_HALF):
            g = Graph(s, text)
            for k, v in dev.items():
                g.bind(k, v)
            g.compile(flags)
            graphs.append(g)
        rng = np.random.default_rng(seed)
        xv = s.to_device(rng.normal(0, 1, (4, 2048)).astype(np.float32))
        w = s.upload_weight(rng.normal(0, 0.02, (3000, 2048)).astype(np.float32), trans=True, pack_dtype=L.DT_BF16)
        yv = s.empty(L.DT_F32, (4, 3000))
        outs = []
        for _ in range(runs):
            for g in graphs:
                (y,) = g.run({"x": x})
                outs.append(y.numpy())
                y.free()
            s.gemm(xv, w, yv, 4)
            outs.append(yv.numpy())
        for g in graphs:
            g.free()
        w.free()
        return outs
    finally:
        s.close()


def test_sessions_run_concurrently():
    """TestSessionConcurrentRun (graph/concurrent_test.go:18) for this backend: one session serialises its own
    calls (a single stream; GPUSession.runMu, graph/gpu_darwin_arm64.go:308), so concurrency is a session per
    thread. Four threads, each with its own session, compiled MLP graphs (f32 and GPUBF16 plans) and an M = 4
    decode GEMV, run at once (the library calls release the interpreter lock); every output is bit-identical
    to the same work run alone."""
    import threading

    announce("sessions on four threads")
    seeds, runs = [31, 32, 33, 34], 6
    alone = {sd: _session_work(sd, runs) for sd in seeds}
    got, errs = {}, []

    def worker(sd):
        try:
            got[sd] = _session_work(sd, runs)
        except Exception as e:  # reported below, in the test's thread
            errs.append(f"seed {sd}: {e!r}")

    threads = [threading.Thread(target=worker, args=(sd,)) for sd in seeds]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errs, errs
    for sd in seeds:
        assert len(got[sd]) == len(alone[sd])
        for i, (a, b) in enumerate(zip(got[sd], alone[sd])):
            assert a.dtype == b.dtype and a.tobytes() == b.tobytes(), f"seed {sd}: output {i} differs"
