"""Seeded synthetic inputs for the tests (numpy Philox streams, bit-reproducible).

Distributions follow the benchmark configurations: weights N(0,0.02),
rho = -5 + N(0,0.1), eps N(0,1), LayerNorm x N(0,1), gamma N(1,0.1),
beta N(0,0.1), upstream gradients N(0,1), tokens uniform or Zipf over [0,V).
"""
import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.Philox(key=seed))


def normal(g: np.random.Generator, shape, mean=0.0, std=1.0) -> np.ndarray:
    return (g.standard_normal(shape, dtype=np.float32) * np.float32(std) + np.float32(mean)).astype(np.float32)


def tokens_uniform(g, n: int, V: int) -> np.ndarray:
    return g.integers(0, V, size=n, dtype=np.int32)


def tokens_zipf(g, n: int, V: int, s: float = 1.1) -> np.ndarray:
    """Zipf(s) truncated to [0, V): P(k) proportional to (k+1)^-s (inverse-CDF sampling)."""
    w = 1.0 / np.arange(1, V + 1, dtype=np.float64) ** s
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    return np.minimum(np.searchsorted(cdf, g.random(n)), V - 1).astype(np.int32)


def special_floats() -> np.ndarray:
    """Values that exercise the branches of the elementwise math."""
    v = [0.0, -0.0, 1e-45, -1e-45, 1e-38, -1e-38, 1e-30, -1e-30, 2.0 ** -55, 2.0 ** -25, 2.0 ** -12,
         0.25, -0.25, 0.34657, -0.34657, 0.5, -0.5, 1.0, -1.0, 1.03972, -1.03972, 2.0, -2.0, 9.0, -9.0,
         11.0, -11.0, 19.99, 20.0, 20.0001, -20.0, 22.0, -22.0, 30.0, -30.0, 88.0, 88.72, 89.0, -88.0,
         -103.0, -103.9, -104.0, -110.0, 1e10, -1e10, 3.4e38, -3.4e38,
         np.inf, -np.inf, np.nan]
    return np.array(v, dtype=np.float32)
