"""The full decode step (``ops.full_decode``: query rotation, pair LUT, Stage1, Stage2 -- or the
one-launch path when every (sequence, kv-head part) gets one Stage1 wave) over seeded random
shapes: batch (up to 300, so that large batches take the one-launch path), kv-heads, GQA group,
split count, layout, query dtype, output dtype and ragged or equal lengths, against the oracle
(the query rotated in float64, then the C Stage1 and Stage2).

Bar: LSE max-abs <= 2e-4; outputs max-abs <= 2e-4 plus the output dtype's rounding (2^-8 of
|out| for bf16, 2^-10 for fp16); empty sequences give NaN rows and -inf LSE on both sides.
"""
import numpy as np
import pytest
import torch

from conftest import to_dev
from oracle import native
from tq4_decode import ops, workloads

pytestmark = pytest.mark.gpu
DTYPES = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}
ROUND = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -8, torch.float32: 0.0}


def _case(i):
    rng = np.random.default_rng(20261402 + i)
    hk = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([g for g in (1, 2, 3, 4, 6, 8, 16) if hk * g <= 128]))
    big = i % 4 == 0  # batches that fill the device with one wave per (sequence, kv-head part)
    batch = int(rng.integers(200, 301)) if big else int(rng.integers(1, 65))
    splits = int(rng.choice([1, 2, 8, 16, 32]))
    equal = rng.random() < 0.4
    if equal:
        lens = np.full(batch, int(rng.integers(1, 1200 if big else 3000)))
    else:
        lens = rng.integers(0, 1200 if big else 3000, batch)
        lens[rng.random(batch) < 0.1] = 0
    budget = 1_500_000 // hk
    while lens.sum() > budget:
        lens = lens // 2
    return dict(seed=20261402 + i, hk=hk, group=group, batch=batch, splits=splits,
                layout=str(rng.choice(["soa", "aos"])), qdt=str(rng.choice(list(DTYPES))),
                odt=str(rng.choice(["same", "f32"])), lens=lens.astype(np.int32))


CASES = [_case(i) for i in range(32)]


def _id(c):
    return (f"B{c['batch']}-hk{c['hk']}-g{c['group']}-S{c['splits']}-{c['layout']}-q{c['qdt']}"
            f"-o{c['odt']}")


@pytest.mark.parametrize("c", CASES, ids=[_id(c) for c in CASES])
def test_full_decode_random_shape(dev, c):
    hk, layout = c["hk"], c["layout"]
    hq = hk * c["group"]
    rng = np.random.default_rng(c["seed"])
    w = workloads.small(c["seed"], c["batch"], c["lens"], c["splits"], num_q_heads=hq, num_kv_heads=hk)
    cache = workloads.soa_to_aos(w.kv_cache, w.centroids, hk) if layout == "aos" else w.kv_cache
    qdt = DTYPES[c["qdt"]]
    odt = qdt if c["odt"] == "same" else torch.float32
    query = torch.from_numpy(rng.standard_normal((c["batch"], hq, 128)).astype(np.float32)).to(qdt)
    rot = workloads.random_orthogonal(rng, 128)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    print(_id(c), flush=True)
    out, lse = ops.full_decode(query.to(dev), t(rot), t(cache), t(w.block_table), t(w.seq_lens),
                               t(w.centroids), c["splits"], layout=layout, out_dtype=odt)
    torch.cuda.synchronize()
    q_rot = (query.double().numpy() @ rot.astype(np.float64)).astype(np.float32)
    mid = native.stage1(q_rot, cache, w.block_table, w.seq_lens, w.centroids, c["splits"],
                        num_kv_heads=hk, is_aos=layout == "aos")
    ro, rl = native.stage2(mid, w.seq_lens)
    got, gl = out.float().cpu().numpy(), lse.cpu().numpy()
    empty = w.seq_lens == 0
    assert np.isnan(got[empty]).all() and np.isneginf(gl[empty]).all()
    live = ~empty
    if live.any():
        err_o = np.abs(got[live] - ro[live]) - ROUND[odt] * np.abs(ro[live])
        err_l = np.abs(gl[live] - rl[live]).max()
        print(f"out excess {err_o.max():.3e}, lse max-abs {err_l:.3e}")
        assert err_o.max() <= 2e-4
        assert err_l <= 2e-4


@pytest.mark.parametrize("batch", [4, 256])
def test_full_decode_attention_scale(dev, batch):
    """A non-default attn_scale through both paths: the four-launch step (batch 4) and the one
    launch with the rotation inside Stage1 (batch 256, one wave per sequence and kv-head)."""
    rng = np.random.default_rng(20261499 + batch)
    lens = rng.integers(1, 900, batch).astype(np.int32)
    w = workloads.small(20261499 + batch, batch, lens, 16, num_q_heads=32, num_kv_heads=8)
    query = torch.from_numpy(rng.standard_normal((batch, 32, 128)).astype(np.float32)).to(torch.float16)
    rot = workloads.random_orthogonal(rng, 128)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    out, lse = ops.full_decode(query.to(dev), t(rot), t(w.kv_cache), t(w.block_table), t(w.seq_lens),
                               t(w.centroids), 16, out_dtype=torch.float32, attn_scale=0.3)
    torch.cuda.synchronize()
    q_rot = (query.double().numpy() @ rot.astype(np.float64)).astype(np.float32)
    mid = native.stage1(q_rot, w.kv_cache, w.block_table, w.seq_lens, w.centroids, 16, num_kv_heads=8,
                        attn_scale=0.3)
    ro, rl = native.stage2(mid, w.seq_lens)
    err_o, err_l = np.abs(out.cpu().numpy() - ro).max(), np.abs(lse.cpu().numpy() - rl).max()
    print(f"batch {batch}: out max-abs {err_o:.3e}, lse max-abs {err_l:.3e}")
    assert err_o <= 2e-4 and err_l <= 2e-4
