"""Pins of the cache layout, nibble order and store restatements."""
import numpy as np
import pytest

from oracle import codebook, layout, store
from tq4_decode import layout as pl
from tq4_decode import workloads


def test_reference_layout_constants():
    # the reference's own static asserts (baseline/common.py:762-775)
    d, hk, bs = 128, 8, 16
    assert layout.slot_bytes(d) == 134 == pl.slot_bytes(d)
    assert layout.soa_meta_offset(bs, hk, d) == 16384 == pl.meta_offset(bs, hk, d)
    assert hk * 3 * bs * 2 == 768
    assert layout.block_bytes(bs, hk, d) == 17152 == pl.block_bytes(bs, hk, d)
    assert 16384 + 768 == 17152
    assert 4096 // bs == 256 and 64 * 256 == 16384


def test_unpack_low_nibble_first():
    got = layout.unpack_nibbles(np.array([[0xA3, 0x0F, 0xF0]], np.uint8))
    assert got.tolist() == [[3, 10, 15, 0, 0, 15]]
    rnd = np.random.default_rng(0).integers(0, 256, (5, 64), dtype=np.uint8)
    bits = np.unpackbits(rnd[..., None], axis=-1, bitorder="little")  # [5, 64, 8] lsb first
    lo = bits[..., :4] @ (1 << np.arange(4))
    hi = bits[..., 4:] @ (1 << np.arange(4))
    assert np.array_equal(layout.unpack_nibbles(rnd), np.stack([lo, hi], -1).reshape(5, 128))


@pytest.mark.parametrize("split", [(1, 4), (7, 4), (4096, 32), (513, 32), (10000, 64), (5, 16)])
def test_split_partition_tiles_the_sequence(split):
    seq_len, s = split
    covered = []
    for sid in range(s):
        a, b = layout.split_range(seq_len, s, sid)
        assert pl.split_bounds(seq_len, s, sid) == (a, b)
        if a < b:
            covered.extend(range(a, b))
    assert covered == list(range(seq_len))


def test_split_partition_brute_force_small():
    for seq_len in range(1, 300):
        for s in (4, 16, 32, 64):
            sizes = [max(0, b - a) for a, b in (layout.split_range(seq_len, s, i) for i in range(s))]
            assert sum(sizes) == seq_len
            ln = -(-seq_len // s)
            live = [x for x in sizes if x]
            assert sizes[:len(live)] == live  # non-empty splits form a prefix
            assert all(x == ln for x in live[:-1]) and 1 <= live[-1] <= ln


@pytest.mark.parametrize("is_aos", [False, True])
def test_store_then_gather_round_trip(is_aos):
    rng = np.random.default_rng(3)
    d, hk, bs = 128, 4, 16
    c = codebook.centroids(d, 4)
    rot = workloads.random_orthogonal(rng, d)
    key = rng.standard_normal((40, hk, d)).astype(np.float32)
    val = rng.standard_normal((40, hk, d)).astype(np.float32)
    slots = rng.permutation(4 * bs)[:40]
    cache = np.zeros((4, bs, hk, layout.slot_bytes(d)), np.uint8)
    store.store(key, val, slots, rot, c, cache, block_size=bs, is_aos=is_aos)
    idx, norm, folded = store.quantize_keys(key, rot, c)
    codes, scale, vmin = store.quantize_values(val)
    gather = layout.gather_aos if is_aos else layout.gather_soa
    for h in range(hk):
        ki, kn, vc, vs, vz = gather(cache, slots // bs, slots % bs, h, bs, hk, d)
        assert np.array_equal(ki, idx[:, h]) and np.array_equal(vc, codes[:, h])
        want = norm[:, h] if is_aos else folded[:, h]
        assert np.array_equal(kn, want.astype(np.float16).astype(np.float64))
        assert np.array_equal(vs, scale[:, h].astype(np.float16).astype(np.float64))
        assert np.array_equal(vz, vmin[:, h].astype(np.float16).astype(np.float64))


def test_bucketize_is_nearest_centroid():
    rng = np.random.default_rng(4)
    c = codebook.centroids(128, 4)
    key = rng.standard_normal((64, 2, 128)).astype(np.float32)
    rot = workloads.random_orthogonal(rng, 128)
    idx, _, _ = store.quantize_keys(key, rot, c)
    x = key / np.linalg.norm(key, axis=-1, keepdims=True)
    y = x @ rot
    brute = np.abs(y[..., None] - c.astype(np.float64)).argmin(-1)
    assert np.mean(idx == brute) > 0.9999


def test_value_quantisation_bounds():
    rng = np.random.default_rng(5)
    v = rng.standard_normal((32, 3, 128)).astype(np.float32)
    codes, scale, vmin = store.quantize_values(v)
    rec = codes * scale[..., None] + vmin[..., None]
    assert codes.min() == 0 and codes.max() == 15
    assert np.all(np.abs(rec - v) <= scale[..., None] * 0.5 + 1e-6)
