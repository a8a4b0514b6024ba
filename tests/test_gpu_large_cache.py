"""Caches past 4 GiB: the block addresses of the Stage1 kernels and of the cache writer.

A pool of blocks 16,000 past the 2^32-byte mark (4-bit slots: 266,407 blocks of 16 tokens x 8
kv-heads x 134 bytes, 4.57 GB; the presets' slots likewise, 4.5-4.7 GB) holds the blocks of
a small ragged workload at block indexes past that mark (every fifth one near the start
instead); the rest of the pool is zero.  Stage1 (4-bit SoA and AoS, both kernels; the FP8-key
and 3-bit presets) over the pool must match the oracle over the compact cache (the same bytes
under the original block table): a block read from a wrapped or truncated address would be
zero bytes there and change the rows.  The writer, given slots in the same blocks, must leave
in them exactly the bytes it writes into a compact cache, and nothing anywhere else.

Bar: Stage1 max-abs <= 1e-4 on mid_o and the same untouched-split pattern (NaN-prefilled);
the writer bit-exact against itself on the compact cache.
"""
import numpy as np
import pytest
import torch

from conftest import to_dev
from oracle import native
from tq4_decode import codebook, ops, workloads

pytestmark = pytest.mark.gpu
TOL = 1e-4
HK, BS, SLOT = 8, 16, 134
LENS = [700, 33, 0, 1500, 16, 2048]


def _first_high(slot):
    """First block index past 4 GiB for blocks of BS tokens x HK kv-heads x slot bytes."""
    return (1 << 32) // (BS * HK * slot) + 1


def _pool_blocks(slot):
    return _first_high(slot) + 16_000


def _placement(n, slot=SLOT):
    """Pool index of compact block i: past 4 GiB, or near the start for every fifth."""
    pool = _pool_blocks(slot)
    idx = np.array([5 * i + 3 if i % 5 == 4 else pool - 2 * n + 2 * i for i in range(n)], np.int64)
    assert len(set(idx.tolist())) == n and idx.max() < pool and (idx[idx > 5 * n] >= _first_high(slot)).all()
    return idx


def _pool(dev, compact, idx):
    pool = torch.zeros((_pool_blocks(compact.shape[-1]),) + tuple(compact.shape[1:]), dtype=torch.uint8,
                       device=dev)
    pool[torch.from_numpy(idx).to(dev)] = to_dev(compact, dev)
    return pool


@pytest.mark.parametrize("layout", ["soa", "aos"])
@pytest.mark.parametrize("kernel", ["auto", "simple"])
def test_stage1_over_a_cache_past_4_gib(dev, layout, kernel):
    w = workloads.small(4096, len(LENS), LENS, 8, num_q_heads=32, num_kv_heads=HK, block_size=BS)
    compact = (workloads.soa_to_aos(w.kv_cache, w.centroids, HK, block_size=BS) if layout == "aos"
               else w.kv_cache)
    idx = _placement(compact.shape[0])
    print(f"{layout} {kernel}: {compact.shape[0]} blocks at pool indexes {idx.min()} .. {idx.max()}", flush=True)
    pool = _pool(dev, compact, idx)
    bt = idx[w.block_table].astype(np.int32)
    ref = native.stage1(w.q_rot, compact, w.block_table, w.seq_lens, w.centroids, w.num_kv_splits,
                        num_kv_heads=HK, block_size=BS, is_aos=layout == "aos")
    mid = torch.full((w.batch, w.num_q_heads, w.num_kv_splits, 129), float("nan"), device=dev)
    ops.stage1(to_dev(w.q_rot, dev), pool, to_dev(bt, dev), to_dev(w.seq_lens, dev), to_dev(w.pair_lut, dev),
               mid, layout=layout, kernel=kernel)
    torch.cuda.synchronize()
    got = mid.cpu().numpy()
    del pool
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "untouched-split pattern differs"
    err = np.nanmax(np.abs(got - ref))
    print(f"max-abs {err:.3e}")
    assert err <= TOL, f"max-abs {err} > {TOL}"


@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_writer_into_a_cache_past_4_gib(dev, layout):
    rng = np.random.default_rng(4097)
    n_blocks, n_tok = 40, 500
    key = rng.standard_normal((n_tok, HK, 128)).astype(np.float32)
    value = (rng.standard_normal((n_tok, HK, 128)) * 0.7).astype(np.float32)
    slots = rng.permutation(n_blocks * BS)[:n_tok].astype(np.int64)
    rot_t = workloads.random_orthogonal(rng, 128)
    cents = codebook.centroids(128, 4)
    mids = ((cents[:-1] + cents[1:]) * np.float32(0.5)).astype(np.float32)
    idx = _placement(n_blocks)
    big_slots = (idx[slots // BS] * BS + slots % BS).astype(np.int32)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    args = (t(rot_t), t(mids), t(cents))
    compact = torch.zeros((n_blocks, BS, HK, SLOT), dtype=torch.uint8, device=dev)
    ops.store(t(key), t(value), compact, t(slots.astype(np.int32)), *args, layout=layout)
    pool = torch.zeros((_pool_blocks(SLOT), BS, HK, SLOT), dtype=torch.uint8, device=dev)
    print(f"{layout}: slots in pool blocks {idx.min()} .. {idx.max()}", flush=True)
    ops.store(t(key), t(value), pool, t(big_slots), *args, layout=layout)
    torch.cuda.synchronize()
    placed = pool[torch.from_numpy(idx).to(dev)]
    assert torch.equal(placed, compact), "bytes written past 4 GiB differ"
    # nothing written outside the placed blocks
    total = pool.sum(dtype=torch.int64).item()
    assert total == placed.sum(dtype=torch.int64).item()


@pytest.mark.parametrize("preset", ["fp8", (3, 4), (3, 3)], ids=["fp8", "k3v4", "k3v3"])
def test_presets_over_a_cache_past_4_gib(dev, preset):
    from oracle import bits as obits
    from oracle import fp8 as ofp8
    from oracle import stage1 as ostage
    from oracle import store as ostore

    rng = np.random.default_rng(4098)
    lens = np.array([300, 0, 700, 45], np.int32)
    w = workloads.small(4098, len(lens), lens, 4, num_q_heads=32, num_kv_heads=HK, block_size=BS)
    nb = w.kv_cache.shape[0]
    key = rng.standard_normal((nb * BS, HK, 128)).astype(np.float32)
    value = (rng.standard_normal((nb * BS, HK, 128)) * 0.8).astype(np.float32)
    q = rng.standard_normal((w.batch, 32, 128)).astype(np.float32)
    every = np.arange(nb * BS, dtype=np.int32)
    if preset == "fp8":
        compact = np.zeros((nb, BS, HK, ofp8.slot_bytes(128)), np.uint8)
        ostore.store_fp8(key, value, every, compact, block_size=BS)
        ref = ostage.stage1(q, compact, w.block_table, w.seq_lens, None, 4, num_kv_heads=HK, block_size=BS,
                            key_fp8=True)
    else:
        kb, vb = preset
        cents = codebook.centroids(128, kb).astype(np.float32)
        compact = np.zeros((nb, BS, HK, obits.slot_bytes(128, kb, vb)), np.uint8)
        obits.store(key, value, every, workloads.random_orthogonal(rng, 128), cents, compact, kb, vb,
                    block_size=BS)
        ref = ostage.stage1(q, compact, w.block_table, w.seq_lens, cents, 4, num_kv_heads=HK, block_size=BS,
                            bits=(kb, vb))
    idx = _placement(nb, compact.shape[-1])
    print(f"{preset}: {nb} blocks of {compact.shape[-1]}-byte slots at pool indexes {idx.min()} .. {idx.max()}",
          flush=True)
    pool = _pool(dev, compact, idx)
    bt = to_dev(idx[w.block_table].astype(np.int32), dev)
    mid = torch.full((w.batch, 32, 4, 129), float("nan"), device=dev)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    if preset == "fp8":
        ops.stage1_fp8(t(q), pool, bt, t(w.seq_lens), mid)
    else:
        ops.stage1_preset(t(q), pool, bt, t(w.seq_lens), t(cents), mid, key_bits=kb, value_bits=vb)
    torch.cuda.synchronize()
    got = mid.cpu().numpy()
    del pool
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "untouched-split pattern differs"
    err = np.nanmax(np.abs(got - ref))
    print(f"max-abs {err:.3e}")
    assert err <= TOL, f"max-abs {err} > {TOL}"
