"""The preset writers over seeded random shapes: 3-bit K with 4- or 3-bit V (``ops.store_preset``)
and FP8 keys (``ops.store_fp8``), with random token counts (past 1024 tiles too), kv-heads, block
sizes, input dtypes, layouts and skipped slots, against the oracle writers.

Bar: FP8 keys -- every byte equal to the oracle writer's (no rotation: an exact cast).  3-bit K --
as the 4-bit writer: V codes, scale and min bit-exact, a K index off by one bucket only within
1e-6 of a midpoint, the K scalar within one fp16 ulp on rows without such a tie.  Both: bytes
outside the written records keep their fill.
"""
import numpy as np
import pytest
import torch

from conftest import to_dev
from oracle import bits as obits
from oracle import fp8 as ofp8
from oracle import store as ostore
from tq4_decode import codebook, ops, workloads

pytestmark = pytest.mark.gpu
D = 128
TORCH = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _case(i):
    rng = np.random.default_rng(20261602 + i)
    hk = int(rng.choice([1, 2, 4, 8]))
    return dict(seed=20261602 + i, preset=["fp8", (3, 4), (3, 3)][i % 3], hk=hk, bs=int(rng.choice([16, 32, 64])),
                n_tok=int(rng.choice([1, 9, 100, 700, 2100 if hk == 8 else 4200])),
                dtype=str(rng.choice(list(TORCH))), layout=str(rng.choice(["soa", "aos"])),
                skip=float(rng.choice([0.0, 0.2])))


CASES = [_case(i) for i in range(24)] + [  # 128- and 256-token KV blocks
    dict(seed=20261630, preset="fp8", hk=8, bs=256, n_tok=700, dtype="bf16", layout="soa", skip=0.2),
    dict(seed=20261631, preset=(3, 4), hk=2, bs=128, n_tok=1000, dtype="f32", layout="aos", skip=0.0),
    dict(seed=20261632, preset=(3, 3), hk=4, bs=256, n_tok=333, dtype="f16", layout="soa", skip=0.2),
    dict(seed=20261633, preset="fp8", hk=1, bs=128, n_tok=64, dtype="f32", layout="aos", skip=0.2)]


def _id(c):
    name = "fp8" if c["preset"] == "fp8" else "k%dv%d" % c["preset"]
    return f"{name}-N{c['n_tok']}-hk{c['hk']}-bs{c['bs']}-{c['dtype']}-{c['layout']}-skip{c['skip']}"


def _record_spans(size, bs, hk, slot, blocks, offs, aos, rec, n_meta):
    """Bytes of every written (block, offset, kv-head) record: the AoS slot's first rec + 2 *
    n_meta bytes, or the SoA record and its n_meta fp16 metadata fields."""
    stride = bs * hk * slot
    heads = np.arange(hk)
    mask = np.zeros(size, dtype=bool)
    if aos:
        spans = [((blocks[:, None] * stride + (offs[:, None] * hk + heads) * slot).reshape(-1), rec + 2 * n_meta)]
    else:
        start = (blocks[:, None] * stride + (offs[:, None] * hk + heads) * rec).reshape(-1)
        meta = blocks[:, None] * stride + bs * hk * rec + (heads * n_meta * bs + offs[:, None]) * 2
        spans = [(start, rec)] + [((meta + 2 * f * bs).reshape(-1), 2) for f in range(n_meta)]
    for s, n in spans:
        mask[(s[:, None] + np.arange(n)).reshape(-1)] = True
    return mask


@pytest.mark.parametrize("c", CASES, ids=[_id(c) for c in CASES])
def test_preset_store_random_shape(dev, c):
    rng = np.random.default_rng(c["seed"])
    hk, bs, n_tok, aos = c["hk"], c["bs"], c["n_tok"], c["layout"] == "aos"
    n_blocks = (n_tok + bs - 1) // bs + 2
    dt = TORCH[c["dtype"]]
    scale = 30.0 if c["preset"] == "fp8" else 1.0
    key = torch.from_numpy((rng.standard_normal((n_tok, hk, D)) * scale).astype(np.float32)).to(dt)
    value = torch.from_numpy((rng.standard_normal((n_tok, hk, D)) * 0.6).astype(np.float32)).to(dt)
    slots = rng.permutation(n_blocks * bs)[:n_tok].astype(np.int32)
    slots[rng.random(n_tok) < c["skip"]] = -1
    kf, vf = key.float().numpy(), value.float().numpy()
    keep = np.nonzero(slots >= 0)[0]
    blocks, offs = (slots[keep] // bs).astype(np.int64), (slots[keep] % bs).astype(np.int64)
    print(_id(c), flush=True)
    if c["preset"] == "fp8":
        slot = ofp8.slot_bytes(D)
        cache0 = np.full((n_blocks, bs, hk, slot), 0x5A, dtype=np.uint8)
        cache = to_dev(cache0, dev)
        ops.store_fp8(key.to(dev), value.to(dev), cache, to_dev(slots, dev), layout=c["layout"])
        torch.cuda.synchronize()
        got = cache.cpu().numpy()
        ref = ostore.store_fp8(kf, vf, slots, cache0.copy(), block_size=bs, is_aos=aos)
        diff = np.nonzero(got.reshape(-1) != ref.reshape(-1))[0]
        assert diff.size == 0, f"{diff.size} bytes differ, first at {diff[:8]}"
        written = _record_spans(cache0.size, bs, hk, slot, blocks, offs, aos, D + D // 2, 2)
    else:
        kb, vb = c["preset"]
        rot_t = workloads.random_orthogonal(rng, D)
        cents = codebook.centroids(D, kb).astype(np.float32)
        mids = ((cents[:-1] + cents[1:]) * np.float32(0.5)).astype(np.float32)
        slot = obits.slot_bytes(D, kb, vb)
        cache0 = np.full((n_blocks, bs, hk, slot), 0xA5, dtype=np.uint8)
        cache = to_dev(cache0, dev)
        ops.store_preset(key.to(dev), value.to(dev), cache, to_dev(slots, dev), to_dev(rot_t, dev), to_dev(mids, dev),
                         to_dev(cents, dev), key_bits=kb, value_bits=vb, layout=c["layout"], norm_correction=not aos)
        torch.cuda.synchronize()
        got = cache.cpu().numpy()
        ref = obits.store(kf, vf, slots, rot_t, cents, cache0.copy(), kb, vb, block_size=bs, is_aos=aos)
        k64 = kf[keep].astype(np.float64)
        y = (k64 / (np.sqrt((k64 ** 2).sum(-1, keepdims=True)) + 1e-8)) @ rot_t.astype(np.float64)
        near_tie = np.abs(y[..., None] - mids.astype(np.float64)).min(-1) < 1e-6
        ties = 0
        for h in range(hk):
            gk, gn, gv, gs, gz = obits.gather(got, blocks, offs, h, bs, hk, D, kb, vb, aos)
            rk, rn, rv, rs, rz = obits.gather(ref, blocks, offs, h, bs, hk, D, kb, vb, aos)
            assert np.array_equal(gv, rv), "V codes differ"
            assert np.array_equal(gs, rs) and np.array_equal(gz, rz), "V scale / min differ"
            diff = gk != rk
            assert not np.any(diff & ~near_tie[:, h]), "K index differs away from a midpoint"
            assert np.all(np.abs(gk.astype(int) - rk.astype(int))[diff] == 1)
            clean = ~diff.any(-1)
            assert np.all(np.abs(gn - rn)[clean] <= np.abs(rn)[clean] * 2.0 ** -10), "K scalar off by > 1 ulp"
            ties += int(diff.sum())
        print(f"K index ties {ties}")
        written = _record_spans(cache0.size, bs, hk, slot, blocks, offs, aos, 16 * (kb + vb), 3)
    assert np.array_equal(got.reshape(-1)[~written], cache0.reshape(-1)[~written]), "bytes outside the records"
    assert np.array_equal(ref.reshape(-1)[~written], cache0.reshape(-1)[~written])
