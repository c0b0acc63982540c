"""Seeded synthetic workloads of the benchmark configurations.

Every generator draws from numpy's PCG64 with the given seed, in f32, so
the GPU path and the CPU baseline see the same arrays.
"""
from __future__ import annotations

import numpy as np


def regression_100k(n=100_000, f=32, seed=0):
    """Dense f32 n x f, N(0,1); y = 2 x0 - x1 + sin(3 x2) + 0.5 x3 x4 + N(0, 0.1)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, f), dtype=np.float32)
    y = (2 * x[:, 0] - x[:, 1] + np.sin(3 * x[:, 2]) + 0.5 * x[:, 3] * x[:, 4]
         + rng.normal(0.0, 0.1, n).astype(np.float32)).astype(np.float32)
    return x, y


def higgs_like(n=10_500_000, seed=0, chunk=1 << 20):
    """Binary logistic, dense f32 n x 28: 21 N(0,1) features, 7 nonlinear
    products / magnitudes of them plus N(0, 0.05); label
    Bernoulli(sigmoid(0.8 x0 - 0.5 x1 x2 + tanh(x3) + 0.3 x21))."""
    rng = np.random.default_rng(seed)
    x = np.empty((n, 28), np.float32)
    y = np.empty(n, np.float32)
    for s in range(0, n, chunk):
        m = min(chunk, n - s)
        b = rng.standard_normal((m, 21), dtype=np.float32)
        e = rng.normal(0.0, 0.05, (m, 7)).astype(np.float32)
        derived = np.stack([b[:, 0] * b[:, 1], np.abs(b[:, 2]), b[:, 3] * b[:, 4], np.abs(b[:, 5] * b[:, 6]),
                            b[:, 7] * b[:, 8], np.abs(b[:, 9]), b[:, 10] * b[:, 11]], axis=1) + e
        x[s:s + m, :21] = b
        x[s:s + m, 21:] = derived
        logit = 0.8 * b[:, 0] - 0.5 * b[:, 1] * b[:, 2] + np.tanh(b[:, 3]) + 0.3 * derived[:, 0]
        p = 1.0 / (1.0 + np.exp(-logit.astype(np.float64)))
        y[s:s + m] = (rng.random(m) < p).astype(np.float32)
    return x, y


def sparse_wide(n=500_000, f=2_000, density=0.1, seed=0):
    """CSR f32 n x f, each cell present with probability `density` (Exp(1)
    values), the rest missing; y = sum of 20 chosen features (0 when
    missing) + N(0, 0.1)."""
    rng = np.random.default_rng(seed)
    counts = rng.binomial(f, density, n)
    row_ptr = np.zeros(n + 1, np.uint64)
    row_ptr[1:] = np.cumsum(counts)
    nnz = int(row_ptr[-1])
    col = np.empty(nnz, np.uint32)
    for r in range(n):
        c = rng.choice(f, size=counts[r], replace=False)
        c.sort()
        col[row_ptr[r]:row_ptr[r + 1]] = c
    val = rng.exponential(1.0, nnz).astype(np.float32)
    chosen = rng.choice(f, size=20, replace=False)
    mask = np.isin(col, chosen)
    rows = np.repeat(np.arange(n), counts)
    y = np.bincount(rows[mask], weights=val[mask], minlength=n).astype(np.float32)
    y += rng.normal(0.0, 0.1, n).astype(np.float32)
    return (row_ptr, col, val), y, f


def multiclass(n=2_000_000, f=50, k=10, seed=0):
    """Dense f32 n x f N(0,1); label = argmax_c (W x + Gumbel), W ~ N(0,1) k x f."""
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((k, f), dtype=np.float32)
    x = rng.standard_normal((n, f), dtype=np.float32)
    g = rng.gumbel(size=(n, k)).astype(np.float32)
    y = np.argmax(x @ w.T + g, axis=1).astype(np.float32)
    return x, y


def forest(n_trees=1000, depth=8, n_features=100, seed=0):
    """Full depth-`depth` trees in the reference's node layout (children of
    node i at 2i+1, 2i+2): split features U{0..n_features-1}, thresholds
    drawn N(0,1), leaves N(0, 0.01), default directions uniform."""
    rng = np.random.default_rng(seed)
    internal = (1 << depth) - 1
    total = (1 << (depth + 1)) - 1
    trees = []
    for _ in range(n_trees):
        i = np.arange(total)
        leaf = i >= internal
        left = np.where(leaf, -1, 2 * i + 1).astype(np.int32)
        right = np.where(leaf, -1, 2 * i + 2).astype(np.int32)
        trees.append(dict(
            split_feature=np.where(leaf, 0, rng.integers(0, n_features, total)).astype(np.uint32),
            split_cond=np.where(leaf, 0.0, rng.standard_normal(total)).astype(np.float32),
            default_left=rng.integers(0, 2, total).astype(np.uint8),
            left=left, right=right,
            leaf_value=np.where(leaf, rng.normal(0.0, 0.01, total), 0.0).astype(np.float32)))
    return trees


def predict_rows(n=10_000_000, f=100, nan_rate=0.02, seed=1, chunk=1 << 20):
    """Dense f32 n x f N(0,1) with a fraction of cells NaN (missing)."""
    rng = np.random.default_rng(seed)
    x = np.empty((n, f), np.float32)
    for s in range(0, n, chunk):
        m = min(chunk, n - s)
        b = rng.standard_normal((m, f), dtype=np.float32)
        b[rng.random((m, f)) < nan_rate] = np.nan
        x[s:s + m] = b
    return x
