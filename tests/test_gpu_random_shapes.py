"""Stage1 parity over seeded random shapes: batch, kv-heads, GQA group, split count, KV
block size, layout and ragged lengths (empty, one-token, long sequences) drawn together, so
that combinations no hand-written case covers meet the oracle.

Bar: max-abs <= 1e-4 on mid_o (outputs and LSE, fp32) and the same untouched-split pattern
(NaN-prefilled; empty splits stay NaN), for the auto kernel and, where it has an instance
for the group, the VALU kernel (AoS cases also through the backend's head-major storage and
its transpose(1, 2) view); and the same for the FP8-key and 3-bit presets (caches written by
the oracle writers).
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


CASES = [_case(i) for i in range(160)]


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
    runs = [(kernel, args) for kernel in kernels]
    if layout == "aos":
        # the same slots through the backend's head-major storage and its transpose(1, 2) view
        storage = t(cache).permute(0, 2, 1, 3).contiguous()
        runs.append(("auto/head-major view", (args[0], storage.transpose(1, 2)) + args[2:]))
    for kernel, a in runs:
        mid = torch.full((w.batch, w.num_q_heads, w.num_kv_splits, 129), float("nan"), device=dev)
        ops.stage1(*a, mid, layout=layout, kernel=kernel.split("/")[0])
        torch.cuda.synchronize()
        got = mid.cpu().numpy()
        assert np.array_equal(np.isnan(got), np.isnan(ref)), f"{kernel}: untouched-split pattern differs"
        err = np.nanmax(np.abs(got - ref)) if np.isfinite(ref).any() else 0.0
        print(f"{_id(c)} {kernel}: max-abs {err:.3e}")
        assert err <= TOL, f"{kernel}: max-abs {err} > {TOL}"


# The presets (3-bit K with 4- or 3-bit V, FP8 keys) over seeded random shapes, smaller
# (their oracle is the float64 numpy restatement).
def _preset_case(i):
    rng = np.random.default_rng(20261302 + i)
    preset = [(3, 4), (3, 3), "fp8"][i % 3]
    hk = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([g for g in (1, 2, 3, 4, 6, 8, 16) if hk * g <= 64]))
    batch = int(rng.integers(1, 25))
    splits = int(rng.choice([1, 3, 8, 16, 32]))
    bs = int(rng.choice([16, 16, 32]))
    layout = str(rng.choice(["soa", "aos"]))
    kind = rng.random(batch)
    lens = np.where(kind < 0.15, 0, np.where(kind < 0.3, rng.integers(1, 40, batch),
                                             rng.integers(40, 900, batch)))
    while lens.sum() * hk > 60_000:
        lens = lens // 2
    return dict(seed=20261302 + i, preset=preset, hk=hk, group=group, batch=batch, splits=splits,
                bs=bs, layout=layout, lens=lens.astype(np.int32))


PRESET_CASES = [_preset_case(i) for i in range(72)]


def _pid(c):
    name = "fp8" if c["preset"] == "fp8" else "k%dv%d" % c["preset"]
    return f"{name}-B{c['batch']}-hk{c['hk']}-g{c['group']}-S{c['splits']}-bs{c['bs']}-{c['layout']}"


@pytest.mark.parametrize("c", PRESET_CASES, ids=[_pid(c) for c in PRESET_CASES])
def test_random_shape_preset_matches_oracle(dev, c):
    from oracle import bits as obits
    from oracle import fp8 as ofp8
    from oracle import stage1 as ostage
    from oracle import store as ostore
    from tq4_decode import codebook

    rng = np.random.default_rng(c["seed"])
    hk, bs, layout, lens = c["hk"], c["bs"], c["layout"], c["lens"]
    aos = layout == "aos"
    w = workloads.small(c["seed"], c["batch"], lens, c["splits"], num_q_heads=hk * c["group"],
                        num_kv_heads=hk, block_size=bs)
    nb = w.kv_cache.shape[0]
    key = rng.standard_normal((nb * bs, hk, 128)).astype(np.float32)
    value = (rng.standard_normal((nb * bs, hk, 128)) * 0.8).astype(np.float32)
    q = rng.standard_normal((c["batch"], hk * c["group"], 128)).astype(np.float32)
    mid = torch.full((c["batch"], hk * c["group"], c["splits"], 129), float("nan"), device=dev)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    if c["preset"] == "fp8":
        cache = np.zeros((nb, bs, hk, ofp8.slot_bytes(128)), np.uint8)
        ostore.store_fp8(key, value, np.arange(nb * bs, dtype=np.int32), cache, block_size=bs, is_aos=aos)
        ops.stage1_fp8(t(q), t(cache), t(w.block_table), t(w.seq_lens), mid, layout=layout)
        ref = ostage.stage1(q, cache, w.block_table, w.seq_lens, None, c["splits"], num_kv_heads=hk,
                            block_size=bs, is_aos=aos, key_fp8=True)
    else:
        kb, vb = c["preset"]
        cents = codebook.centroids(128, kb).astype(np.float32)
        cache = np.zeros((nb, bs, hk, obits.slot_bytes(128, kb, vb)), np.uint8)
        obits.store(key, value, np.arange(nb * bs), workloads.random_orthogonal(rng, 128), cents, cache,
                    kb, vb, block_size=bs, is_aos=aos)
        ops.stage1_preset(t(q), t(cache), t(w.block_table), t(w.seq_lens), t(cents), mid, key_bits=kb,
                          value_bits=vb, layout=layout)
        ref = ostage.stage1(q, cache, w.block_table, w.seq_lens, cents, c["splits"], num_kv_heads=hk,
                            block_size=bs, is_aos=aos, bits=(kb, vb))
    torch.cuda.synchronize()
    got = mid.cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "untouched-split pattern differs"
    err = np.nanmax(np.abs(got - ref)) if np.isfinite(ref).any() else 0.0
    print(f"{_pid(c)}: max-abs {err:.3e}")
    assert err <= TOL, f"max-abs {err} > {TOL}"
