"""Pins of the FP8-key preset's oracle: the E4M3 codec against torch's float8_e4m3fn and
the format's definition, the writer/reader round trip, and Stage1 with FP8 keys against
torch attention over the decoded keys."""
import math

import numpy as np
import torch

from oracle import fp8, layout, stage1
from oracle import store as ostore


def test_decode_table_matches_torch_for_every_byte():
    ref = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    got = fp8.decode_table()
    assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.nanmax(np.abs(got - ref)) == 0
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and np.isnan(got[0x7F])


def test_encode_rounds_to_nearest_even_and_saturates():
    vals = fp8.decode_table()
    finite = vals[~np.isnan(vals)]
    assert np.array_equal(fp8.decode(fp8.encode(finite)), finite)  # exact values survive
    # halfway between 1.0 (0x38) and 1.125 (0x39): ties go to the even code 0x38
    assert fp8.encode([1.0625])[0] == 0x38 and fp8.encode([1.0626])[0] == 0x39
    assert list(fp8.encode([460.0, 1e6, -1e6])) == [0x7E, 0x7E, 0xFE]
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(10000) * 50).astype(np.float32)
    y = fp8.decode(fp8.encode(x))
    # nearest representable: no finite code is strictly closer
    d = np.abs(finite[None, :] - x[:, None]).min(1)
    assert np.allclose(np.abs(y - x), d)


def test_store_then_gather_round_trip():
    rng = np.random.default_rng(1)
    n, hk, d, bs = 40, 8, 128, 16
    key = rng.standard_normal((n, hk, d)).astype(np.float32) * 3
    value = rng.standard_normal((n, hk, d)).astype(np.float32)
    slots = rng.permutation(4 * bs)[:n].astype(np.int32)
    for aos in (False, True):
        cache = np.zeros((4, bs, hk, fp8.slot_bytes(d)), np.uint8)
        ostore.store_fp8(key, value, slots, cache, block_size=bs, is_aos=aos)
        codes, scale, vmin = ostore.quantize_values(value)
        for h in range(hk):
            kb, vc, vs, vz = fp8.gather(cache, slots // bs, slots % bs, h, bs, hk, d, aos)
            assert np.array_equal(kb, fp8.encode(key[:, h]))
            assert np.array_equal(vc, codes[:, h])
            assert np.array_equal(vs, scale[:, h].astype(np.float16).astype(np.float64))
            assert np.array_equal(vz, vmin[:, h].astype(np.float16).astype(np.float64))


def test_stage1_fp8_matches_torch_attention():
    rng = np.random.default_rng(2)
    hk, hq, d, bs = 8, 32, 128, 16
    lens = np.array([1, 40, 200], np.int32)
    need = (lens + bs - 1) // bs
    nb = int(need.sum()) + 2
    bt = np.zeros((3, int(need.max())), np.int32)
    perm = rng.permutation(nb).astype(np.int32)
    pos = 0
    for b in range(3):
        bt[b, :need[b]] = perm[pos:pos + need[b]]
        pos += need[b]
    key = rng.standard_normal((int(lens.sum()), hk, d)).astype(np.float32)
    value = rng.standard_normal((int(lens.sum()), hk, d)).astype(np.float32)
    slots = np.concatenate([bt[b, np.arange(lens[b]) // bs] * bs + np.arange(lens[b]) % bs
                            for b in range(3)]).astype(np.int32)
    cache = np.zeros((nb, bs, hk, fp8.slot_bytes(d)), np.uint8)
    ostore.store_fp8(key, value, slots, cache, block_size=bs)
    q = rng.standard_normal((3, hq, d)).astype(np.float32)
    mid = stage1.stage1(q, cache, bt, lens, None, 4, num_kv_heads=hk, key_fp8=True)
    for b in range(3):
        for sid in range(4):
            a, e = layout.split_range(int(lens[b]), 4, sid)
            if a >= e:
                assert np.isnan(mid[b, :, sid]).all()
                continue
            tok = np.arange(a, e)
            for kvh in range(hk):
                kb, vc, vs, vz = fp8.gather(cache, bt[b, tok // bs], tok % bs, kvh, bs, hk, d, False)
                k = torch.from_numpy(fp8.decode(kb))
                v = torch.from_numpy(vc * vs[:, None] + vz[:, None])
                for h in range(kvh * 4, kvh * 4 + 4):
                    s = torch.from_numpy(q[b, h].astype(np.float64)) @ k.T / math.sqrt(d)
                    o = torch.softmax(s, 0) @ v
                    assert np.abs(mid[b, h, sid, :d] - o.numpy()).max() < 1e-12
                    assert abs(mid[b, h, sid, d] - torch.logsumexp(s, 0).item()) < 1e-12
