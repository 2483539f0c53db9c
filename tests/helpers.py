"""Shared helpers for the GPU parity tests."""
import math

import numpy as np


def nstar_tol(K: int, a: np.ndarray, b: np.ndarray) -> float:
    """The north-star bound: max-abs error <= 1e-3·sqrt(K)·max|A|·max|B|."""
    ma = float(np.max(np.abs(a))) if a.size else 0.0
    mb = float(np.max(np.abs(b))) if b.size else 0.0
    return 1e-3 * math.sqrt(max(K, 1)) * ma * mb


def assert_close(got: np.ndarray, want: np.ndarray, tol: float, what: str = ""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    err = float(np.max(np.abs(got - want))) if got.size else 0.0
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    assert err <= tol, f"{what}: max-abs error {err:.3e} > tol {tol:.3e}"
    return err


def bf16_weights(rng, shape, scale=1.0, dist="uniform"):
    """Random weights rounded to bf16 bits (F32ToBF16)."""
    import oracle

    if dist == "uniform":
        w = rng.uniform(-scale, scale, shape)
    else:
        w = rng.normal(0, scale, shape)
    return oracle.f32_to_bf16(w.astype(np.float32))


def announce(msg: str):
    """Names the case on stdout (flushed) before a GPU step."""
    print(msg, flush=True)
