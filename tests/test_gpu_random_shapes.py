"""Stage1 parity over seeded random shapes: batch, kv-heads, GQA group, split count, KV
block size, layout and ragged lengths (empty, one-token, long sequences) drawn together, so
that combinations no hand-written case covers meet the oracle.

Bar: max-abs <= 1e-4 on mid_o (outputs and LSE, fp32) and the same untouched-split pattern
(NaN-prefilled; empty splits stay NaN), for the auto kernel and, where it has an instance
for the group, the VALU kernel.
"""
import numpy as np
import pytest
import torch

from conftest import to_dev
from oracle import native
from tq4_decode import ops, workloads

pytestmark = pytest.mark.gpu
TOL = 1e-4
SIMPLE_GROUPS = (1, 2, 4, 6, 8, 16)


def _case(i):
    rng = np.random.default_rng(20261202 + i)
    hk = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([g for g in (1, 2, 3, 4, 5, 6, 8, 12, 16) if hk * g <= 128]))
    batch = int(rng.integers(1, 81))
    splits = int(rng.choice([1, 2, 3, 5, 8, 16, 32, 33, 64, 70]))
    bs = int(rng.choice([16, 16, 32, 64]))
    layout = str(rng.choice(["soa", "aos"]))
    kind = rng.random(batch)
    lens = np.where(kind < 0.15, 0,
                    np.where(kind < 0.3, rng.integers(1, 50, batch),
                             np.where(kind < 0.9, rng.integers(50, 700, batch),
                                      rng.integers(700, 3000, batch))))
    # bound the cache (tokens x kv-heads) so every case stays small
    budget = 400_000 // hk
    while lens.sum() > budget:
        lens = lens // 2
    return dict(seed=20261202 + i, hk=hk, group=group, batch=batch, splits=splits, bs=bs,
                layout=layout, lens=lens.astype(np.int32))


CASES = [_case(i) for i in range(48)]


def _id(c):
    return f"B{c['batch']}-hk{c['hk']}-g{c['group']}-S{c['splits']}-bs{c['bs']}-{c['layout']}"


@pytest.mark.parametrize("c", CASES, ids=[_id(c) for c in CASES])
def test_random_shape_matches_oracle(dev, c):
    hk, layout, bs = c["hk"], c["layout"], c["bs"]
    w = workloads.small(c["seed"], c["batch"], c["lens"], c["splits"], num_q_heads=hk * c["group"],
                        num_kv_heads=hk, block_size=bs)
    cache = (workloads.soa_to_aos(w.kv_cache, w.centroids, hk, block_size=bs) if layout == "aos"
             else w.kv_cache)
    ref = native.stage1(w.q_rot, cache, w.block_table, w.seq_lens, w.centroids, w.num_kv_splits,
                        num_kv_heads=hk, block_size=bs, is_aos=layout == "aos")
    t = lambda a: to_dev(a, dev)  # noqa: E731
    args = (t(w.q_rot), t(cache), t(w.block_table), t(w.seq_lens), t(w.pair_lut))
    kernels = ["auto"] + (["simple"] if c["group"] in SIMPLE_GROUPS else [])
    for kernel in kernels:
        mid = torch.full((w.batch, w.num_q_heads, w.num_kv_splits, 129), float("nan"), device=dev)
        ops.stage1(*args, mid, layout=layout, kernel=kernel)
        torch.cuda.synchronize()
        got = mid.cpu().numpy()
        assert np.array_equal(np.isnan(got), np.isnan(ref)), f"{kernel}: untouched-split pattern differs"
        err = np.nanmax(np.abs(got - ref)) if np.isfinite(ref).any() else 0.0
        print(f"{_id(c)} {kernel}: max-abs {err:.3e}")
        assert err <= TOL, f"{kernel}: max-abs {err} > {TOL}"
