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


def test_norm_correction_keeps_the_key_norm():
    """The _nc writers store fp16(||k|| / ||c[idx]||) (reference/soa_store.py:343-353), so the
    decoded key folded * c[idx] has the raw key's norm, to the fp16 rounding of the scalar
    (2^-11 relative).  Folding the other way (||k|| * ||c||) is off by ||c||^2 (~3-6 %)."""
    rng = np.random.default_rng(6)
    c = codebook.centroids(128, 4)
    key = (rng.standard_normal((400, 4, 128)) * rng.uniform(0.1, 30, (400, 4, 1))).astype(np.float32)
    rot = workloads.random_orthogonal(rng, 128)
    idx, norm, folded = store.quantize_keys(key, rot, c)
    cn = np.sqrt((c[idx].astype(np.float64) ** 2).sum(-1))
    knorm = np.linalg.norm(key.astype(np.float64), axis=-1)
    ratio = cn * folded.astype(np.float16).astype(np.float64) / knorm
    assert np.abs(ratio - 1).max() <= 2.0 ** -11 + 1e-6
    wrong = cn * cn * ratio  # the other fold direction
    assert np.abs(wrong - 1).max() > 0.02


def test_fixture_soa_and_aos_slots_hold_the_same_key():
    """The config-1 fixture's two caches come from the same keys: equal K codes, and the SoA
    folded norm times ||c[idx]|| equals the AoS raw norm within the two fp16 roundings."""
    f = np.load(layout.__file__.replace("oracle/layout.py", "tests/golden/config1_b2_ctx256.npz"))
    soa, aos, c = f["cache_soa"], f["cache_aos"], f["centroids"]
    nb, bs, hk = soa.shape[:3]
    data = soa.reshape(nb, -1)[:, :bs * hk * 128].reshape(nb, bs, hk, 128)
    assert np.array_equal(data[..., :64], aos[..., :64])       # K codes
    assert np.array_equal(data[..., 64:], aos[..., 66:130])    # V codes
    meta = soa.reshape(nb, -1)[:, bs * hk * 128:].copy().view(np.float16).reshape(nb, hk, 3, bs)
    folded = meta[:, :, 0, :].transpose(0, 2, 1).astype(np.float64)       # [nb, bs, hk]
    raw = aos[..., 64:66].copy().view(np.float16)[..., 0].astype(np.float64)
    kb = aos[..., :64]
    cn = np.sqrt((c[kb & 15].astype(np.float64) ** 2 + c[kb >> 4].astype(np.float64) ** 2).sum(-1))
    assert np.abs(folded * cn / raw - 1).max() <= 2 * 2.0 ** -11 + 1e-6
    # V scale and zero are stored identically
    assert np.array_equal(meta[:, :, 1, :].transpose(0, 2, 1), aos[..., 130:132].copy().view(np.float16)[..., 0])
    assert np.array_equal(meta[:, :, 2, :].transpose(0, 2, 1), aos[..., 132:134].copy().view(np.float16)[..., 0])


def test_soa_and_converted_aos_decode_alike():
    """The reference's layout check at its benchmark shape (README.md:146, AoS V1 vs SoA V1
    output max-abs 1.28e-5): the AoS cache converted from the B64 x ctx 4096 SoA cache (raw
    norm = fp16(folded * ||c||), baseline/common.py:651-671) decodes (raw / ||c||) to the SoA
    outputs within 2e-5, the LSE within the fp16 rounding of the norm; a decoder that folded
    the norm the other way would differ by percents.  C oracle (fp32)."""
    from oracle import native

    w = workloads.qwen3_4b_b64_ctx4096()
    aos = workloads.soa_to_aos(w.kv_cache, w.centroids, 8)
    a = native.stage1(w.q_rot, w.kv_cache, w.block_table, w.seq_lens, w.centroids, 32, num_kv_heads=8)
    b = native.stage1(w.q_rot, aos, w.block_table, w.seq_lens, w.centroids, 32, num_kv_heads=8,
                      is_aos=True)
    err = np.abs(a[..., :128] - b[..., :128]).max()  # the output columns, as README.md:146
    lse = np.abs(a[..., 128] - b[..., 128]).max()
    print(f"SoA vs converted AoS output max-abs {err:.3e}, LSE {lse:.3e}")
    assert err <= 2e-5
    assert lse <= 2.0 ** -10 * np.abs(a[..., 128]).max()  # fp16 rounding of the norm
