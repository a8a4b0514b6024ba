# The Lloyd-Max iteration follows reference/centroids.py (SPDX-License-Identifier:
# Apache-2.0, Copyright contributors to the vLLM project) step for step, so that the
# centroids are bit-identical; the code is written anew.
"""Lloyd-Max codebook for N(0, 1/d) and the byte-indexed pair LUT (host side).

The codebook is the one the cache writer quantises K against: 2^bits centroids of
the Lloyd-Max quantiser for N(0, 1/d), computed as in ``reference/centroids.py:31-86``
(uniform start on +-3.5 sigma, trapezoid cell integrals with 200 panels over edges
at +-10.5 sigma, at most 200 sweeps, tolerance 1e-10, float64 then float32).  The
result is a one-off host table; it is cached per ``(d, bits)``.

``pair_lut(c)[lo * n + hi] = (c[lo], c[hi])`` (``baseline/common.py:232-257``): one row
per packed K byte.
"""
from __future__ import annotations

import functools
import math

import numpy as np


def _cell_integral(fn, a: float, b: float, panels: int = 200) -> float:
    h = (b - a) / panels
    acc = 0.5 * (fn(a) + fn(b))
    for i in range(1, panels):
        acc += fn(a + i * h)
    return acc * h


@functools.lru_cache(maxsize=16)
def _solve(d: int, bits: int) -> tuple[tuple[float, ...], tuple[float, ...]]:
    n = 1 << bits
    var = 1.0 / d
    sigma = math.sqrt(var)
    coef = 1.0 / math.sqrt(2 * math.pi * var)
    pdf = lambda x: coef * math.exp(-x * x / (2 * var))  # noqa: E731
    xpdf = lambda x: x * pdf(x)  # noqa: E731
    lo, hi = -3.5 * sigma, 3.5 * sigma
    c = [lo + (hi - lo) * (i + 0.5) / n for i in range(n)]
    for _ in range(200):
        edges = [lo * 3] + [(c[i] + c[i + 1]) / 2.0 for i in range(n - 1)] + [hi * 3]
        nxt = []
        for i in range(n):
            den = _cell_integral(pdf, edges[i], edges[i + 1])
            num = _cell_integral(xpdf, edges[i], edges[i + 1])
            nxt.append(num / den if den > 1e-15 else c[i])
        if max(abs(nxt[i] - c[i]) for i in range(n)) < 1e-10:
            break
        c = nxt
    mids = [(c[i] + c[i + 1]) / 2.0 for i in range(n - 1)]
    return tuple(c), tuple(mids)


def centroids(d: int = 128, bits: int = 4) -> np.ndarray:
    return np.asarray(_solve(d, bits)[0], dtype=np.float32)


def midpoints(d: int = 128, bits: int = 4) -> np.ndarray:
    return np.asarray(_solve(d, bits)[1], dtype=np.float32)


def pair_lut(cents) -> np.ndarray:
    c = np.asarray(cents, dtype=np.float32).reshape(-1)
    n = c.size
    lut = np.stack(np.broadcast_arrays(c[:, None], c[None, :]), axis=-1)
    return np.ascontiguousarray(lut.reshape(n * n, 2), dtype=np.float32)
