"""The GPU writer's K-index fast path (the cell table), emulated in float32 on the CPU.

The writer (``csrc/store.h``) finds the 4-bit index -- the number of midpoints <= y, the
reference's bucketize (``reference/soa_store.py:306-316``) -- without 15 compares: 128 cells
of width ``w = span / 124`` centred on ``(K + k) w`` (``K`` an integer) hold the midpoint that
lies inside the cell's window (widened by ``w / 64``) and the count below it; the cell of
``y`` is read from the bits of one biased fma.  A codebook takes this path only when every
window holds at most one midpoint and ``|K| < 2^14``.  This file restates the table build
and the lookup in float32 and checks that the result equals ``searchsorted(midpoints, y,
side="right")`` for every float32 ``y`` within three cells of the midpoints' span (for
codebooks around zero, where those are too many, for a 1.5e-4-cell grid around every
midpoint and cell edge and the float32 neighbours of each point): the Lloyd-Max codebook,
uniform midpoints, and both shifted away from zero up to the ``|K|`` bound.
"""
import numpy as np
import pytest

from tq4_decode import codebook

F = np.float32
CELLS = 128
BIAS = F(12582912.0)  # 1.5 * 2^23


def cell_table(mids):
    """``(K, w, ok, base [128], m_in [128])`` as the writer builds them."""
    mmin, mmax = mids.min(), mids.max()
    w = F((mmax - mmin) / F(CELLS - 4))
    kcell = F(np.floor(F((mmin - F(2.0) * w) / w)))
    y0 = F(kcell * w)
    base = np.zeros(CELLS, np.int64)
    m_in = np.full(CELLS, np.nan, F)
    ok = abs(kcell) < F(2.0 ** 14) and 0 < w < np.inf
    for k in range(CELLS):
        lo = F(y0 + F(F(k) - F(0.5)) * w - w * F(1.0 / 64))
        hi = F(y0 + F(F(k) + F(0.5)) * w + w * F(1.0 / 64))
        base[k] = int((mids < lo).sum())
        inside = (mids >= lo) & (mids <= hi)
        ok = ok and inside.sum() <= 1
        if inside.any():
            m_in[k] = mids[inside][-1]
    return kcell, w, ok, base, m_in


def cell_index(mids, y):
    """Indices of float32 ``y`` through the cell table (the MFMA result is a = 256 y)."""
    kcell, w, ok, base, m_in = cell_table(mids)
    a = (F(256.0) * y).astype(F)
    inv_w = F(F(F(1.0) / w) * F(1.0 / 256))
    c0 = F(BIAS - kcell)
    # one fma: the product is exact in float64, then one rounding to float32
    t = (a.astype(np.float64) * np.float64(inv_w) + np.float64(c0)).astype(F)
    t = np.minimum(np.maximum(t, BIAS), F(BIAS + CELLS - 1))
    cell = t.view(np.int32) - np.array([BIAS], F).view(np.int32)[0]
    return ok, base[cell] + (a >= F(256.0) * m_in[cell])


def every_float(lo, hi, limit=4_000_000):
    """Every float32 in [lo, hi] (None when there are more than ``limit``)."""
    def mag(x):
        return int(np.array([abs(x)], F).view(np.int32)[0])
    parts = []
    if lo < 0:  # negative floats: magnitudes from |min(hi, 0)| to |lo|
        parts.append((mag(min(hi, F(0.0))), mag(lo), -1))
    if hi >= 0:
        parts.append((mag(max(lo, F(0.0))), mag(hi), 1))
    if sum(b - a + 1 for a, b, _ in parts) > limit:
        return None
    return np.concatenate([F(s) * np.arange(a, b + 1, dtype=np.int32).view(F) for a, b, s in parts])


def lloyd_max_mids():
    c = codebook.centroids(128, 4).astype(F)
    return ((c[1:] + c[:-1]) / F(2.0)).astype(F)


@pytest.mark.parametrize("shift", [0.0, 0.5, 3.0, 10.0, 40.0])
@pytest.mark.parametrize("kind", ["lloyd_max", "uniform"])
def test_cell_path_equals_the_count_for_every_float(kind, shift):
    mids = lloyd_max_mids() if kind == "lloyd_max" else (F(0.03) * np.arange(15, dtype=F) - F(0.2)).astype(F)
    mids = (mids + F(shift)).astype(F)
    ok, _ = cell_index(mids, mids[:1])
    assert ok, "these codebooks take the cell path"
    w = F((mids.max() - mids.min()) / F(CELLS - 4))
    ys = every_float(F(mids.min() - 3 * w), F(mids.max() + 3 * w))
    if ys is None:
        # too many floats near zero: each midpoint and cell edge +- 1.5 cells on a 1.5e-4-cell
        # grid, plus the float32 neighbours of every point
        near = (mids[:, None] + w * np.linspace(-1.5, 1.5, 20001, dtype=F)[None, :]).ravel().astype(F)
        ys = np.unique(np.concatenate([near, np.nextafter(near, F(np.inf)), np.nextafter(near, F(-np.inf))]))
    _, got = cell_index(mids, ys)
    ref = np.searchsorted(mids, ys, side="right")
    assert np.array_equal(got, ref), f"{(got != ref).sum()} indices differ"


def test_far_shifted_codebook_takes_the_counting_path():
    """|K| >= 2^14: the lookup's rounding error can exceed the windows' widening."""
    ok, _ = cell_index((lloyd_max_mids() + F(1000.0)).astype(F), np.zeros(1, F))
    assert not ok


def test_two_midpoints_in_one_window_take_the_counting_path():
    mids = lloyd_max_mids().copy()
    mids[7] = F(mids[8] - F(1e-4))
    ok, _ = cell_index(np.sort(mids), np.zeros(1, F))
    assert not ok
