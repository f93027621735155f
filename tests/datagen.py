"""Seeded test inputs for the parity tests: PQ codebooks, codes and queries.

Three families:
  - `pq_fixture`: Gaussian-mixture data, codebooks taken from data points and codes by nearest centroid, so the
    distance distribution looks like a trained PQ index;
  - `random_fixture`: N(0, 1) codebooks and uniform codes, the shape of the 100M-vector configuration;
  - `tie_fixture`: small-integer codebooks and queries, so many distances are exactly equal and the (dist, id)
    tie-break decides the order.
"""
from __future__ import annotations

import numpy as np


def mixture(n: int, d: int, components: int, sigma: float, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    centres = rng.standard_normal((components, d), dtype=np.float32)
    which = rng.integers(0, components, size=n)
    return (centres[which] + sigma * rng.standard_normal((n, d), dtype=np.float32)).astype(np.float32)


def encode(x: np.ndarray, centroids: np.ndarray) -> np.ndarray:
    """Nearest centroid per sub-space (ties to the lowest index), chunked to bound memory."""
    n, d = x.shape
    m, ksub, dsub = centroids.shape
    codes = np.empty((n, m), dtype=np.uint8)
    for s in range(m):
        c = centroids[s]
        cn = (c * c).sum(1)
        for a in range(0, n, 65536):
            xs = x[a:a + 65536, s * dsub:(s + 1) * dsub]
            dist = cn[None, :] - 2.0 * xs @ c.T
            codes[a:a + 65536, s] = np.argmin(dist, axis=1)
    return codes


def pq_fixture(n: int, d: int, m: int, nq: int, seed: int, components: int = 50, sigma: float = 0.3):
    rng = np.random.default_rng(seed + 1000)
    base = mixture(n + nq, d, components, sigma, seed)
    x, queries = base[:n], base[n:]
    dsub = d // m
    pick = rng.choice(n, size=256, replace=False)
    centroids = np.stack([x[pick, s * dsub:(s + 1) * dsub] for s in range(m)]).astype(np.float32)
    return centroids, encode(x, centroids), queries


def random_fixture(n: int, d: int, m: int, nq: int, seed: int):
    rng = np.random.default_rng(seed)
    centroids = rng.standard_normal((m, 256, d // m), dtype=np.float32)
    codes = rng.integers(0, 256, size=(n, m), dtype=np.uint8)
    queries = rng.standard_normal((nq, d), dtype=np.float32)
    return centroids, codes, queries


def tie_fixture(n: int, d: int, m: int, nq: int, seed: int):
    rng = np.random.default_rng(seed)
    centroids = rng.integers(0, 3, size=(m, 256, d // m)).astype(np.float32)
    codes = rng.integers(0, 256, size=(n, m), dtype=np.uint8)
    queries = rng.integers(0, 3, size=(nq, d)).astype(np.float32)
    return centroids, codes, queries
