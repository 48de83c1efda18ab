"""Shared test helpers: seeded synthetic EXL3 weights and the parity bar."""
from __future__ import annotations

import numpy as np

# The parity bar: max|got - ref| / max|ref| <= TOL and RMS(got - ref) / RMS(ref) <= TOL over the
# compared array (a normalised max-abs error, not a per-element relative bound), fp32 accumulate
# against the fp64 oracle.
TOL = 2e-3


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


def zipf_scores(T: int, E: int, s: float, seed: int) -> np.ndarray:
    """Router logits with Zipf(s)-skewed expert popularity: log of the Zipf
    popularity of a seeded permutation of the experts plus Gumbel noise, as fp16 [T][E].  The same
    generator as bench.py's prefill workload."""
    r = np.random.default_rng(seed)
    perm = r.permutation(E)
    pop = np.empty(E)
    pop[perm] = np.arange(1, E + 1, dtype=np.float64) ** (-s)
    logits = np.log(pop)[None, :] + r.gumbel(size=(T, E))
    return logits.astype(np.float16)
