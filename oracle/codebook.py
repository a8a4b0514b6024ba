# The Lloyd-Max iteration follows reference/centroids.py (SPDX-License-Identifier:
# Apache-2.0, Copyright contributors to the vLLM project) step for step, so that the
# centroids are bit-identical; the code is written anew.
"""Lloyd-Max codebook and pair LUT (oracle side).

``lloyd_max`` restates ``reference/centroids.py:18-79``: a Lloyd-Max scalar quantiser
for N(0, 1/d), initialised uniformly on +-3.5 sigma, cell integrals by the trapezoid
rule with n=200 panels, outer edges at +-10.5 sigma, at most 200 sweeps, stopping
when no centroid moved by ``tol`` (the centroids of the sweep that detected
convergence are *not* adopted, as in the reference).  Arithmetic is Python
float64 in the reference's operation order, then rounded to float32, so the
result is bit-identical to ``get_centroids(d, bits)`` (``reference/centroids.py:82-86``).

``pair_lut`` restates ``baseline/common.py:232-257`` (= ``reference/soa_decode_v2.py:50-66``):
``lut[lo * n + hi] = (c[lo], c[hi])``.

Parity: pinned by the golden vector ``tests/golden/centroids_d128_b4.json`` written
from the reference function itself, by the odd symmetry ``c[i] = -c[n-1-i]``, by the
Lloyd centroid condition evaluated with scipy's Gaussian integrals, and by Max's
(1960) 16-level Gaussian table scaled by ``1/sqrt(d)``.
"""
from __future__ import annotations

import math

import numpy as np


def _trapezoid(fn, a: float, b: float, panels: int = 200) -> float:
    step = (b - a) / panels
    total = 0.5 * (fn(a) + fn(b))
    for k in range(1, panels):
        total += fn(a + k * step)
    return total * step


def lloyd_max(d: int, bits: int, max_iter: int = 200, tol: float = 1e-10):
    """Return ``(centroids, boundaries)`` as float32 arrays."""
    levels = 2 ** bits
    var = 1.0 / d
    sd = math.sqrt(var)
    norm_const = 1.0 / math.sqrt(2 * math.pi * var)

    def density(x):
        return norm_const * math.exp(-x * x / (2 * var))

    def first_moment(x):
        return x * density(x)

    left, right = -3.5 * sd, 3.5 * sd
    cents = [left + (right - left) * (k + 0.5) / levels for k in range(levels)]
    for _ in range(max_iter):
        mids = [(cents[k] + cents[k + 1]) / 2.0 for k in range(levels - 1)]
        edges = [left * 3] + mids + [right * 3]
        moved = []
        for k in range(levels):
            lo_e, hi_e = edges[k], edges[k + 1]
            num = _trapezoid(first_moment, lo_e, hi_e)
            den = _trapezoid(density, lo_e, hi_e)
            moved.append(num / den if den > 1e-15 else cents[k])
        if max(abs(moved[k] - cents[k]) for k in range(levels)) < tol:
            break
        cents = moved
    mids = [(cents[k] + cents[k + 1]) / 2.0 for k in range(levels - 1)]
    return np.asarray(cents, dtype=np.float32), np.asarray(mids, dtype=np.float32)


def centroids(d: int = 128, bits: int = 4) -> np.ndarray:
    return lloyd_max(d, bits)[0]


def pair_lut(cents: np.ndarray) -> np.ndarray:
    """``float32[n*n, 2]`` with row ``lo*n + hi`` = ``(c[lo], c[hi])``."""
    c = np.asarray(cents, dtype=np.float32)
    n = c.shape[0]
    out = np.empty((n, n, 2), dtype=np.float32)
    out[:, :, 0] = c[:, None]
    out[:, :, 1] = c[None, :]
    return out.reshape(n * n, 2)
