"""The GPU writer's 4-bit V code path, emulated in float32 on the CPU, against the oracle.

The writer (``csrc/store.h``, ``quantize_v``) does not compute the reference's
``int((v - min) / scale + 0.5)`` (``reference/soa_store.py:86-116``) directly: it rounds
``q = fma(v, rs, -min * rs)`` to nearest, with ``rs`` the hardware reciprocal of ``scale``
(1 ulp), and only elements whose ``q`` lies within a per-row window of a half-integer take
the IEEE division.  This file emulates that path (all three reciprocals within 1 ulp) and
checks that its codes equal the oracle's on rows built to stress the window: large offsets
(large ``|min / scale|``), exact ties on a half-step grid, bf16-rounded values, constant
rows (the ``1e-8`` scale floor) and wide ranges.  A narrower window (no per-row term) must
fail on the offset rows, so the test does see the term it pins.
"""
import numpy as np
import pytest

from oracle import store as ostore

F32 = np.float32


def _rcp_variants(scale):
    r = (F32(1.0) / scale).astype(F32)
    return [r, np.nextafter(r, F32(np.inf)), np.nextafter(r, F32(0.0))]


def _writer_codes(v, rs, per_row_term=True):
    """Codes of rows ``v`` [R, 128] by the writer's path with reciprocals ``rs`` [R]."""
    vmin = v.min(-1)
    vmax = v.max(-1)
    scale = ((vmax - vmin) / F32(15.0)).astype(F32)
    scale = np.where(scale > F32(1e-8), scale, F32(1e-8)).astype(F32)
    nb = (-vmin * rs).astype(F32)
    # fma: v * rs is exact in float64 (24 + 24 bits), one rounding of the sum to float32
    q = (v.astype(np.float64) * rs[:, None].astype(np.float64) + nb[:, None].astype(np.float64)).astype(F32)
    win = F32(2.0**-16) + (np.abs(nb) * F32(2.0**-22) if per_row_term else np.zeros_like(nb))
    lim = (F32(0.5) - win).astype(F32)
    fast = np.abs(q - np.rint(q)) < lim[:, None]
    code_fast = np.clip(np.rint(q), 0, 255)
    quot = ((v - vmin[:, None]).astype(F32) / scale[:, None]).astype(F32)
    code_div = np.minimum(np.floor((quot + F32(0.5)).astype(F32)), F32(15.0))
    return np.where(fast, code_fast, code_div).astype(np.int64), fast


def _oracle_codes(v):
    codes, _, _ = ostore.quantize_values(v[:, None, :])
    return codes[:, 0, :]


def _rows(rng):
    n = 4000
    rows = [
        rng.standard_normal((n, 128)),
        1000.0 + rng.standard_normal((n, 128)),  # |min / scale| ~ 2000
        -3.0e4 + 10.0 * rng.standard_normal((n, 128)),
        0.25 * rng.integers(-30, 31, (n, 128)),  # half-step grid: exact ties
        np.round(rng.standard_normal((n, 128)) * 8.0) / 8.0 + 7.0,
        np.full((64, 128), 3.25),  # constant rows: scale floor 1e-8
        1.0 + 1e-7 * rng.standard_normal((64, 128)),
        1e30 * rng.standard_normal((64, 128)),
    ]
    out = [r.astype(F32) for r in rows]
    bf = rng.standard_normal((n, 128)).astype(F32)  # bf16-rounded values
    out.append((bf.view(np.uint32) & np.uint32(0xFFFF0000)).view(F32))
    return out


@pytest.mark.parametrize("variant", [0, 1, 2])
def test_writer_vcode_path_matches_oracle(variant):
    rng = np.random.default_rng(11)
    fallbacks = 0
    total = 0
    for v in _rows(rng):
        vmin, vmax = v.min(-1), v.max(-1)
        scale = ((vmax - vmin) / F32(15.0)).astype(F32)
        scale = np.where(scale > F32(1e-8), scale, F32(1e-8)).astype(F32)
        rs = _rcp_variants(scale)[variant]
        got, fast = _writer_codes(v, rs)
        np.testing.assert_array_equal(got, _oracle_codes(v))
        fallbacks += int((~fast).sum())
        total += fast.size
    # the division stays rare on ordinary rows (the constant and offset rows raise it)
    assert fallbacks < 0.2 * total


def test_narrow_window_is_caught():
    """Without the per-row term the offset rows round some elements the wrong way."""
    rng = np.random.default_rng(12)
    v = (1000.0 + rng.standard_normal((4000, 128))).astype(F32)
    vmin, vmax = v.min(-1), v.max(-1)
    scale = ((vmax - vmin) / F32(15.0)).astype(F32)
    rs = _rcp_variants(scale)[0]
    got, _ = _writer_codes(v, rs, per_row_term=False)
    assert np.any(got != _oracle_codes(v))
