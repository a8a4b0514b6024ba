"""The 4-bit cache writer (``ops.store``) over seeded random shapes: token count (a decode step's
few rows up to launches past 1024 tiles, the grid-stride path), kv-heads, block size, input
dtype, layout and skipped slots, against the oracle writer.

Bar (as the fixed-shape writer tests): V codes, V scale and V min bit-exact; a K index may
differ only where the rotated value lies within 1e-6 of a midpoint, and then by one bucket;
the stored K scalar within one fp16 ulp on rows without such a tie; bytes outside the written
records keep their fill.
"""
import numpy as np
import pytest
import torch

from conftest import to_dev
from oracle import layout as OL
from oracle import store as ostore
from tq4_decode import codebook, ops, workloads

pytestmark = pytest.mark.gpu
D = 128
TORCH = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _case(i):
    rng = np.random.default_rng(20261502 + i)
    hk = int(rng.choice([1, 2, 4, 8]))
    bs = int(rng.choice([16, 32, 64]))
    n_tok = int(rng.choice([1, 7, 64, 333, 1000, 2100 if hk == 8 else 4200]))
    return dict(seed=20261502 + i, hk=hk, bs=bs, n_tok=n_tok, dtype=str(rng.choice(list(TORCH))),
                layout=str(rng.choice(["soa", "aos"])), skip=float(rng.choice([0.0, 0.2])))


CASES = [_case(i) for i in range(24)] + [  # 128- and 256-token KV blocks
    dict(seed=20261530, hk=8, bs=128, n_tok=700, dtype="bf16", layout="soa", skip=0.2),
    dict(seed=20261531, hk=2, bs=256, n_tok=1000, dtype="f32", layout="aos", skip=0.0),
    dict(seed=20261532, hk=4, bs=256, n_tok=333, dtype="f16", layout="soa", skip=0.2),
    dict(seed=20261533, hk=1, bs=128, n_tok=64, dtype="bf16", layout="aos", skip=0.2)]


def _id(c):
    return f"N{c['n_tok']}-hk{c['hk']}-bs{c['bs']}-{c['dtype']}-{c['layout']}-skip{c['skip']}"


def _rotated(key, rot_t):
    k = key.astype(np.float64)
    return (k / (np.sqrt((k ** 2).sum(-1, keepdims=True)) + 1e-8)) @ rot_t.astype(np.float64)


@pytest.mark.parametrize("c", CASES, ids=[_id(c) for c in CASES])
def test_store_random_shape(dev, c):
    rng = np.random.default_rng(c["seed"])
    hk, bs, n_tok, aos = c["hk"], c["bs"], c["n_tok"], c["layout"] == "aos"
    n_blocks = (n_tok + bs - 1) // bs + 2
    dt = TORCH[c["dtype"]]
    key = torch.from_numpy((rng.standard_normal((n_tok, hk, D)) * 1.3).astype(np.float32)).to(dt)
    value = torch.from_numpy((rng.standard_normal((n_tok, hk, D)) * 0.7 + 0.1).astype(np.float32)).to(dt)
    slots = rng.permutation(n_blocks * bs)[:n_tok].astype(np.int32)
    slots[rng.random(n_tok) < c["skip"]] = -1
    rot_t = workloads.random_orthogonal(rng, D)
    cents = codebook.centroids(D, 4).astype(np.float32)
    mids = ((cents[:-1] + cents[1:]) * np.float32(0.5)).astype(np.float32)
    cache0 = np.full((n_blocks, bs, hk, 134), 0xA5, dtype=np.uint8)
    print(_id(c), flush=True)
    cache = to_dev(cache0, dev)
    ops.store(key.to(dev), value.to(dev), cache, to_dev(slots, dev), to_dev(rot_t, dev), to_dev(mids, dev),
              to_dev(cents, dev), layout=c["layout"], norm_correction=not aos)
    torch.cuda.synchronize()
    got = cache.cpu().numpy()
    kf, vf = key.float().numpy(), value.float().numpy()
    ref = ostore.store(kf, vf, slots, rot_t, cents, cache0.copy(), block_size=bs, is_aos=aos)

    keep = np.nonzero(slots >= 0)[0]
    blocks, offs = slots[keep] // bs, slots[keep] % bs
    gather = OL.gather_aos if aos else OL.gather_soa
    near_tie = np.abs(_rotated(kf[keep], rot_t)[..., None] - mids.astype(np.float64)).min(-1) < 1e-6
    ties = 0
    for h in range(hk):
        gk, gn, gv, gs, gz = gather(got, blocks, offs, h, bs, hk, D)
        rk, rn, rv, rs, rz = gather(ref, blocks, offs, h, bs, hk, D)
        assert np.array_equal(gv, rv), "V codes differ"
        assert np.array_equal(gs, rs) and np.array_equal(gz, rz), "V scale / min differ"
        diff = gk != rk
        assert not np.any(diff & ~near_tie[:, h]), "K index differs away from a midpoint"
        assert np.all(np.abs(gk.astype(int) - rk.astype(int))[diff] == 1)
        clean = ~diff.any(-1)
        assert np.all(np.abs(gn - rn)[clean] <= np.abs(rn)[clean] * 2.0 ** -10), "K scalar off by > 1 ulp"
        ties += int(diff.sum())
    print(f"K index ties {ties}")
    written = _written(cache0.size, bs, hk, blocks.astype(np.int64), offs.astype(np.int64), aos)
    assert np.array_equal(got.reshape(-1)[~written], cache0.reshape(-1)[~written]), "bytes outside the records"
    assert np.array_equal(ref.reshape(-1)[~written], cache0.reshape(-1)[~written])


def _written(size, bs, hk, blocks, offs, aos):
    """Bytes of the records (SoA: 128-byte record + three fp16 metadata fields; AoS: the
    134-byte slot) of every written (block, offset) and kv-head."""
    stride = bs * hk * 134
    heads = np.arange(hk)
    mask = np.zeros(size, dtype=bool)
    if aos:
        starts = (blocks[:, None] * stride + (offs[:, None] * hk + heads) * 134).reshape(-1)
        spans = [(starts, 134)]
    else:
        rec = (blocks[:, None] * stride + (offs[:, None] * hk + heads) * 128).reshape(-1)
        meta = blocks[:, None] * stride + bs * hk * 128 + (heads * 3 * bs + offs[:, None]) * 2
        spans = [(rec, 128)] + [((meta + 2 * f * bs).reshape(-1), 2) for f in range(3)]
    for starts, n in spans:
        mask[(starts[:, None] + np.arange(n)).reshape(-1)] = True
    return mask
