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


def h16(v):
    """Round to fp16 and back (one fp16 rounding point of the reference arithmetic)."""
    with np.errstate(over="ignore"):   # fp16 overflow to inf is part of the reference arithmetic
        return np.asarray(v, np.float64).astype(np.float16).astype(np.float64)


def silu16(g):
    """fp16 SiLU evaluated with one fp16 rounding per step: e = exp(-g), s = 1 + e, r = 1/s, g.r."""
    with np.errstate(over="ignore"):
        e = h16(np.exp(-g))
    s = h16(1.0 + e)
    return h16(g * h16(1.0 / s))


def had128(v):
    """Row-wise orthonormal Sylvester Hadamard-128 (scipy's matrix / sqrt(128)) in fp64."""
    import scipy.linalg
    H = scipy.linalg.hadamard(128).astype(np.float64) / np.sqrt(128.0)
    return (np.asarray(v, np.float64).reshape(-1, 128) @ H.T).reshape(np.shape(v))


def expert_contrib_numpy(x, Wg, Wu, Wd, su, sv, w, L, act=None):
    """Routed contributions c = H(D) . w . svh_d (fp64) of one expert for the rows x [n][hidden], from
    decoded W_hat matrices [in][out] (fp64) with the fp16 rounding points of the reference expert
    (exl3_moe_kernel.cuh:57-262, hadamard_inner.cuh:284-481): a = fp16(H(fp16(x . suh))); G, U fp16;
    g, u = fp16(fp16(H(G)) . svh); act; clamp; fp16(fp16(g . u) . suh_d); fp16(H(.)); D fp16.
    su / sv: the three projections' suh / svh (fp64); w: routing weights [n] (fp64); act None = SiLU,
    "gelu_erf" = exact GELU (its fp16 rounding), "relu2" = non-gated relu2 (no gate GEMM)."""
    x = np.atleast_2d(np.asarray(x, np.float64))

    def a_in(v, s):
        return h16(had128(h16(v * s)))

    U = a_in(x, su[1]) @ Wu
    u = h16(h16(had128(h16(U))) * sv[1])
    if act == "relu2":
        g = np.maximum(u, 0.0)
    else:
        G = a_in(x, su[0]) @ Wg
        g = h16(h16(had128(h16(G))) * sv[0])
        if act == "gelu_erf":
            import scipy.special
            g = h16(0.5 * g * (1.0 + scipy.special.erf(g / np.sqrt(2.0))))
        else:
            g = silu16(g)
    if L:
        Lh = float(np.float16(L))
        u = np.clip(u, -Lh, Lh)
        g = np.minimum(g, Lh)
    p = h16(h16(g * u) * su[2])
    D = h16(h16(had128(p)) @ Wd)
    return had128(D) * np.asarray(w, np.float64)[:, None] * sv[2]
