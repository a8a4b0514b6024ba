"""The bit-width preset oracle (``oracle/bits.py``: 3-bit keys / 3- or 4-bit values) pinned
against independent statements: numpy's bit unpacking, the reference's 24-bit group
formula, the 4-bit oracle (the 4/4 case must give its bytes), the reference's slot sizes,
and attention computed straight from the quantizer outputs."""
import math

import numpy as np
import pytest
import torch

from oracle import bits, codebook, layout as OL, stage1 as OS, store as ostore
from tq4_decode import workloads

D = 128


@pytest.mark.parametrize("b", [3, 4])
def test_pack_matches_numpy_bit_stream(b):
    rng = np.random.default_rng(b)
    codes = rng.integers(0, 1 << b, (7, D))
    packed = bits.pack(codes, b)
    assert packed.shape == (7, D * b // 8)
    stream = np.unpackbits(packed, axis=-1, bitorder="little").astype(np.int64)
    weights = 1 << np.arange(b)
    got = (stream.reshape(7, D, b) * weights).sum(-1)
    assert np.array_equal(got, codes)
    assert np.array_equal(bits.unpack(packed, b, D), codes)


def test_three_bit_groups_are_little_endian_24_bit_words():
    # reference/soa_store.py:319-337: packed_24 = sum(q_j << 3j) over groups of 8, 3 bytes LE
    codes = np.tile(np.arange(8), D // 8)
    word = sum(j << (3 * j) for j in range(8))  # 0xFAC688
    assert word == 0xFAC688
    packed = bits.pack(codes[None], 3)[0]
    assert list(packed[:3]) == [0x88, 0xC6, 0xFA]
    assert np.array_equal(packed.reshape(-1, 3), np.tile([0x88, 0xC6, 0xFA], (D // 8, 1)))


def test_four_bit_pack_is_the_nibble_pack():
    codes = np.random.default_rng(1).integers(0, 16, (5, D))
    assert np.array_equal(bits.pack(codes, 4), ostore.pack_nibbles(codes))


def test_slot_sizes_follow_the_reference_formula():
    # reference/config.py:128-164: ceil(D*kb/8) + 2 + ceil(D*vb/8) + 4, rounded up to even
    for kb, vb, want in ((3, 4, 118), (3, 3, 102), (4, 4, 134)):
        raw = math.ceil(D * kb / 8) + 2 + math.ceil(D * vb / 8) + 4
        assert bits.slot_bytes(D, kb, vb) == raw + raw % 2 == want
    assert bits.slot_bytes(D, 4, 4) == OL.slot_bytes(D)


def make(seed, n_tok=40, hk=2, n_blocks=4, bs=16, kb=3):
    rng = np.random.default_rng(seed)
    key = rng.standard_normal((n_tok, hk, D)).astype(np.float32)
    value = (rng.standard_normal((n_tok, hk, D)) * 0.6 + 0.2).astype(np.float32)
    slots = rng.permutation(n_blocks * bs)[:n_tok].astype(np.int64)
    slots[::7] = -1
    rot_t = workloads.random_orthogonal(rng, D)
    cents = codebook.centroids(D, kb).astype(np.float32)
    return key, value, slots, rot_t, cents


@pytest.mark.parametrize("aos", [False, True])
def test_four_four_writer_gives_the_four_bit_oracle_bytes(aos):
    key, value, slots, rot_t, cents = make(3, kb=4)
    c0 = np.full((4, 16, 2, 134), 0x5A, dtype=np.uint8)
    a = bits.store(key, value, slots, rot_t, cents, c0.copy(), 4, 4, is_aos=aos)
    b = ostore.store(key, value, slots, rot_t, cents, c0.copy(), is_aos=aos)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("vb", [3, 4])
@pytest.mark.parametrize("aos", [False, True])
def test_writer_round_trip(vb, aos):
    key, value, slots, rot_t, cents = make(5)
    slot = bits.slot_bytes(D, 3, vb)
    cache = bits.store(key, value, slots, rot_t, cents, np.zeros((4, 16, 2, slot), np.uint8), 3, vb,
                       is_aos=aos)
    idx, norm, folded = ostore.quantize_keys(key, rot_t, cents)
    codes, scale, vmin = bits.quantize_values(value, vb)
    keep = np.nonzero(slots >= 0)[0]
    for h in range(2):
        k, n, v, s, z = bits.gather(cache, slots[keep] // 16, slots[keep] % 16, h, 16, 2, D, 3, vb, aos)
        assert np.array_equal(k, idx[keep, h]) and k.max() <= 7
        want_n = (norm if aos else folded)[keep, h].astype(np.float16).astype(np.float32)
        assert np.array_equal(n, want_n)
        assert np.array_equal(v, codes[keep, h])
        assert np.array_equal(s, scale[keep, h].astype(np.float16).astype(np.float32))
        assert np.array_equal(z, vmin[keep, h].astype(np.float16).astype(np.float32))


def test_three_bit_keys_are_the_nearest_centroid():
    key, value, slots, rot_t, cents = make(6)
    idx, _, _ = ostore.quantize_keys(key, rot_t, cents)
    k = key.astype(np.float64)
    y = (k / (np.linalg.norm(k, axis=-1, keepdims=True) + 1e-8)) @ rot_t.astype(np.float64)
    brute = np.abs(y[..., None] - cents.astype(np.float64)).argmin(-1)
    mids = (cents[:-1] + cents[1:]) / 2
    tie = np.abs(y[..., None] - mids).min(-1) < 1e-6
    assert np.array_equal(idx[~tie], brute[~tie])


@pytest.mark.parametrize("vb", [3, 4])
def test_value_codes_are_nearest_levels(vb):
    v = np.random.default_rng(8).standard_normal((50, D)).astype(np.float32)
    codes, scale, vmin = bits.quantize_values(v, vb)
    top = (1 << vb) - 1
    assert codes.min() == 0 and codes.max() == top
    assert np.all(codes.min(-1) == 0) and np.all(codes.max(-1) == top)
    err = np.abs(codes * scale[:, None].astype(np.float64) + vmin[:, None] - v)
    assert np.all(err <= scale[:, None] * (0.5 + 1e-5))


@pytest.mark.parametrize("vb", [3, 4])
@pytest.mark.parametrize("aos", [False, True])
def test_stage1_on_three_bit_cache_is_attention_over_the_quantized_rows(vb, aos):
    hk, g, bs = 2, 4, 16
    key, value, _, rot_t, cents = make(9, n_tok=50, hk=hk)
    slots = np.arange(50, dtype=np.int64) + 7  # token t -> slot t + 7
    slot = bits.slot_bytes(D, 3, vb)
    cache = bits.store(key, value, slots, rot_t, cents, np.zeros((5, bs, hk, slot), np.uint8), 3, vb,
                       is_aos=aos)
    bt = np.array([[0, 1, 2, 3, 4]], dtype=np.int32)
    seq_lens = np.array([57], dtype=np.int32)  # slots 0..6 hold zeros: V = 0, K = 0
    q = np.random.default_rng(2).standard_normal((1, hk * g, D))
    mid = OS.stage1(q, cache, bt, seq_lens, cents, 1, num_kv_heads=hk, is_aos=aos, bits=(3, vb))
    # independent: dequantized rows from the quantizer outputs
    idx, norm, folded = ostore.quantize_keys(key, rot_t, cents)
    codes, scale, vmin = bits.quantize_values(value, vb)
    c = cents.astype(np.float64)[idx]
    f16 = lambda a: a.astype(np.float16).astype(np.float64)  # noqa: E731
    if aos:
        c = c / np.sqrt((c * c).sum(-1, keepdims=True) + 1e-16)
        kd = c * f16(norm)[..., None]
    else:
        kd = c * f16(folded)[..., None]
    vd = codes * f16(scale)[..., None] + f16(vmin)[..., None]
    for h in range(hk * g):
        kv = h // g
        K = np.concatenate([np.zeros((7, D)), kd[:, kv]])
        V = np.concatenate([np.zeros((7, D)), vd[:, kv]])
        s = torch.from_numpy(K @ q[0, h] / math.sqrt(D))
        p = torch.softmax(s, 0).numpy()
        assert np.allclose(mid[0, h, 0, :D], p @ V, atol=1e-10)
        assert abs(mid[0, h, 0, D] - torch.logsumexp(s, 0).item()) < 1e-10
