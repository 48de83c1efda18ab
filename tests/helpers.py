"""Shared test helpers: seeded synthetic EXL3 weights and the parity bar."""
from __future__ import annotations

import numpy as np

TOL = 2e-3  # max-abs error / max|ref| and relative RMS, fp32 accumulate vs fp64 oracle


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def make_linear(seed: int, K: int, N: int, bits: int):
    """trellis uint16 (K/16, N/16, 16*bits) uniform words, suh = +-1, svh = +-U(0.5, 1.5) (fp16)."""
    r = rng(seed)
    trellis = r.integers(0, 65536, size=(K // 16, N // 16, 16 * bits), dtype=np.uint16)
    suh = r.choice(np.array([-1.0, 1.0]), size=K).astype(np.float16)
    svh = (r.choice(np.array([-1.0, 1.0]), size=N) * r.uniform(0.5, 1.5, size=N)).astype(np.float16)
    return trellis, suh, svh


def make_x(seed: int, M: int, K: int) -> np.ndarray:
    return rng(seed).standard_normal((M, K)).astype(np.float16)


def close(got: np.ndarray, ref: np.ndarray, tol: float = TOL) -> tuple[float, float]:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(float(np.abs(ref).max()), 1e-30)
    max_err = float(np.abs(got - ref).max()) / scale
    rms = float(np.sqrt(np.mean((got - ref) ** 2)) / max(np.sqrt(np.mean(ref ** 2)), 1e-30))
    return max_err, rms


def assert_close(got, ref, tol: float = TOL, what: str = ""):
    m, r = close(got, ref, tol)
    assert m <= tol and r <= tol, f"{what}: max-abs/max|ref| = {m:.3e}, rel RMS = {r:.3e} (tol {tol})"
