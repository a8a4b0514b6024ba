"""Pins of the codebook / pair LUT restatements (oracle and product)."""
import json
import math

import numpy as np
import pytest
from scipy import stats

from conftest import GOLDEN
from oracle import codebook as oc
from tq4_decode import codebook as pc

GOLD = json.loads((GOLDEN / "centroids_d128_b4.json").read_text())

# Max (1960), "Quantizing for minimum distortion", Table I: 16-level Lloyd-Max
# quantiser for N(0,1), positive output levels.
MAX_16 = [0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6181, 2.0690, 2.7326]


def _bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("case", GOLD["cases"], ids=lambda c: f"d{c['d']}b{c['bits']}")
@pytest.mark.parametrize("impl", [oc.lloyd_max, lambda d, b: (pc.centroids(d, b), pc.midpoints(d, b))],
                         ids=["oracle", "package"])
def test_centroids_bit_exact_vs_reference_golden(case, impl):
    cents, mids = impl(case["d"], case["bits"])
    assert np.array_equal(_bits(cents), np.array([int(h, 16) for h in case["centroids_hex"]], np.uint32))
    assert np.array_equal(_bits(mids), np.array([int(h, 16) for h in case["boundaries_hex"]], np.uint32))


def test_centroids_odd_symmetry_and_order():
    c = oc.centroids(128, 4).astype(np.float64)
    assert np.all(np.diff(c) > 0)
    assert np.allclose(c, -c[::-1], atol=1e-7)


def test_centroid_condition_with_exact_gaussian_integrals():
    """Each centroid is the conditional mean of its cell under N(0, 1/128) (closed form
    via scipy's normal cdf/pdf), to the accuracy of the 200-panel trapezoid rule (coarser
    in the two outer cells, whose panels span up to 10.5 sigma)."""
    d = 128
    s = 1 / math.sqrt(d)
    c = oc.centroids(d, 4).astype(np.float64)
    edges = np.concatenate([[-10.5 * s], (c[:-1] + c[1:]) / 2, [10.5 * s]])
    a, b = edges[:-1] / s, edges[1:] / s
    cond_mean = s * (stats.norm.pdf(a) - stats.norm.pdf(b)) / (stats.norm.cdf(b) - stats.norm.cdf(a))
    err = np.abs(cond_mean - c) / s
    assert np.max(err[1:-1]) < 5e-5
    assert np.max(err) < 1e-3


def test_centroids_match_max_table():
    c = oc.centroids(128, 4).astype(np.float64) * math.sqrt(128)
    assert np.allclose(c[8:], MAX_16, atol=2e-3)


def test_pair_lut_entries():
    c = oc.centroids(128, 4)
    lut = oc.pair_lut(c)
    assert lut.shape == (256, 2) and lut.dtype == np.float32
    # byte 0xA3 stores dim 2j = 3 (low nibble) and dim 2j+1 = 10 (high nibble): row 3*16+10
    assert lut[0x3A, 0] == c[3] and lut[0x3A, 1] == c[10]
    assert lut[0xF0, 0] == c[15] and lut[0xF0, 1] == c[0]
    assert np.array_equal(_bits(pc.pair_lut(c)), _bits(lut))


def test_planted_codebook_mistake_is_caught():
    """A codebook solved with too few Lloyd sweeps differs from the golden bits: the
    golden check is sensitive at the last-bit level."""
    gold = np.array([int(h, 16) for h in GOLD["cases"][0]["centroids_hex"]], np.uint32)
    c = oc.lloyd_max(128, 4, max_iter=3)[0]  # truncated iteration: a plausible slip
    assert not np.array_equal(_bits(c), gold)
