"""Pins of the Stage1 / Stage2 restatements against torch routines, invariants and
each other (numpy float64 vs C float32)."""
import math

import numpy as np
import pytest
import torch

from oracle import layout, native, stage1, torch_stage1
from tq4_decode import workloads


def _small(seed, seq_lens, splits, hq=32, hk=8):
    return workloads.small(seed, len(seq_lens), seq_lens, splits, num_q_heads=hq, num_kv_heads=hk)


def _torch_split_reference(w, is_aos, cache):
    """Per split: torch SDPA + logsumexp over the decoded K / V (float64)."""
    hq, hk = w.num_q_heads, w.num_kv_heads
    g = hq // hk
    mid = np.full((w.batch, hq, w.num_kv_splits, 129), np.nan)
    for b in range(w.batch):
        for sid in range(w.num_kv_splits):
            a, e = layout.split_range(int(w.seq_lens[b]), w.num_kv_splits, sid)
            if a >= e:
                continue
            tok = np.arange(a, e)
            blocks, offs = w.block_table[b, tok // 16], tok % 16
            for kvh in range(hk):
                k, v = stage1.decode_kv(cache, blocks, offs, kvh, w.centroids, is_aos, 16, hk, 128)
                q = torch.from_numpy(w.q_rot[b, kvh * g:(kvh + 1) * g].astype(np.float64))[None]
                kt = torch.from_numpy(k)[None, None].expand(1, g, -1, -1)
                vt = torch.from_numpy(v)[None, None].expand(1, g, -1, -1)
                o = torch.nn.functional.scaled_dot_product_attention(q[:, :, None], kt, vt)
                s = (q @ torch.from_numpy(k).T) / math.sqrt(128)
                mid[b, kvh * g:(kvh + 1) * g, sid, :128] = o[0, :, 0].numpy()
                mid[b, kvh * g:(kvh + 1) * g, sid, 128] = torch.logsumexp(s[0], -1).numpy()
    return mid


@pytest.mark.parametrize("is_aos", [False, True])
def test_numpy_oracle_matches_torch_attention(is_aos):
    w = _small(11, [1, 37, 130, 64], 8)
    cache = workloads.soa_to_aos(w.kv_cache, w.centroids, 8) if is_aos else w.kv_cache
    ref = _torch_split_reference(w, is_aos, cache)
    got = stage1.stage1(w.q_rot, cache, w.block_table, w.seq_lens, w.centroids, 8,
                        num_kv_heads=8, is_aos=is_aos)
    assert np.array_equal(np.isnan(ref), np.isnan(got))
    assert np.nanmax(np.abs(ref - got)) < 1e-12


@pytest.mark.parametrize("hq,hk,lens,splits", [
    (32, 8, [1, 17, 256, 300], 4),
    (32, 8, [512, 33], 32),
    (64, 8, [700], 16),
    (8, 8, [90, 3], 8),
    (16, 8, [45], 5),
])
@pytest.mark.parametrize("is_aos", [False, True])
def test_c_oracle_matches_numpy_oracle(hq, hk, lens, splits, is_aos):
    w = _small(21, lens, splits, hq, hk)
    cache = workloads.soa_to_aos(w.kv_cache, w.centroids, hk) if is_aos else w.kv_cache
    ref = stage1.stage1(w.q_rot, cache, w.block_table, w.seq_lens, w.centroids, splits,
                        num_kv_heads=hk, is_aos=is_aos)
    got = native.stage1(w.q_rot, cache, w.block_table, w.seq_lens, w.centroids, splits,
                        num_kv_heads=hk, is_aos=is_aos)
    assert np.array_equal(np.isnan(ref), np.isnan(got))
    assert np.nanmax(np.abs(ref - got)) < 2e-6
    o, l = stage1.stage2(ref, w.seq_lens)
    co, cl = native.stage2(got, w.seq_lens)
    assert np.abs(o - co).max() < 2e-6 and np.abs(l - cl).max() < 2e-6


@pytest.mark.parametrize("hq,hk,lens,splits", [
    (32, 8, [1, 17, 256, 300], 4),
    (32, 8, [512, 33, 0], 32),
    (64, 8, [700], 16),
    (8, 8, [90, 3], 8),
    (16, 4, [45, 1000], 5),
])
@pytest.mark.parametrize("is_aos", [False, True])
def test_torch_cpu_restatement_matches_numpy_oracle(hq, hk, lens, splits, is_aos):
    """The vectorized torch fp32 restatement (the CPU baseline) against the float64 oracle,
    including an empty sequence and empty splits."""
    w = _small(23, lens, splits, hq, hk)
    cache = workloads.soa_to_aos(w.kv_cache, w.centroids, hk) if is_aos else w.kv_cache
    ref = stage1.stage1(w.q_rot, cache, w.block_table, w.seq_lens, w.centroids, splits,
                        num_kv_heads=hk, is_aos=is_aos)
    got = torch_stage1.stage1(w.q_rot, cache, w.block_table, w.seq_lens, w.centroids, splits,
                              num_kv_heads=hk, is_aos=is_aos)
    assert np.array_equal(np.isnan(ref), np.isnan(got))
    assert np.nanmax(np.abs(ref - got)) < 2e-6


def test_torch_cpu_restatement_matches_config1_fixture(config1):
    f = config1
    for lay, aos in (("soa", False), ("aos", True)):
        got = torch_stage1.stage1(f["q_rot"], f[f"cache_{lay}"], f["block_table"], f["seq_lens"],
                                  f["centroids"], int(f["num_kv_splits"]),
                                  num_kv_heads=int(f["num_kv_heads"]), is_aos=aos)
        assert np.nanmax(np.abs(got - f[f"mid_{lay}"])) < 2e-6


@pytest.mark.parametrize("splits", [1, 4, 32])
def test_sinks_are_an_extra_logit_with_zero_value(splits):
    """Sinks: split 0's softmax over the scores plus the sink logit (value 0), checked with
    torch.softmax / logsumexp over the concatenated logits; Stage2 of the split rows equals
    unsplit attention with the sink appended once."""
    w = _small(31, [1, 37, 300, 130], splits)
    rng = np.random.default_rng(32)
    sinks = rng.normal(0.0, 3.0, 32)
    sinks[5] = -np.inf  # a head without a sink
    sinks[6] = 40.0     # a sink that dominates every score
    got = stage1.stage1(w.q_rot, w.kv_cache, w.block_table, w.seq_lens, w.centroids, splits,
                        num_kv_heads=8, sinks=sinks)
    for b in range(w.batch):
        a, e = layout.split_range(int(w.seq_lens[b]), splits, 0)
        tok = np.arange(a, e)
        blocks, offs = w.block_table[b, tok // 16], tok % 16
        for kvh in range(8):
            k, v = stage1.decode_kv(w.kv_cache, blocks, offs, kvh, w.centroids, False, 16, 8, 128)
            for h in range(kvh * 4, kvh * 4 + 4):
                logits = torch.from_numpy(np.append(w.q_rot[b, h].astype(np.float64) @ k.T / math.sqrt(128),
                                                    sinks[h]))
                p = torch.softmax(logits, 0)[:-1].numpy()
                assert np.abs(got[b, h, 0, :128] - p @ v).max() < 1e-12
                assert abs(got[b, h, 0, 128] - torch.logsumexp(logits, 0).item()) < 1e-12
    o, lse = stage1.stage2(got, w.seq_lens)
    for b in range(w.batch):
        tok = np.arange(int(w.seq_lens[b]))
        blocks, offs = w.block_table[b, tok // 16], tok % 16
        for kvh in range(8):
            k, v = stage1.decode_kv(w.kv_cache, blocks, offs, kvh, w.centroids, False, 16, 8, 128)
            for h in range(kvh * 4, kvh * 4 + 4):
                logits = torch.from_numpy(np.append(w.q_rot[b, h].astype(np.float64) @ k.T / math.sqrt(128),
                                                    sinks[h]))
                p = torch.softmax(logits, 0)[:-1].numpy()
                assert np.abs(o[b, h] - p @ v).max() < 1e-10
                assert abs(lse[b, h] - torch.logsumexp(logits, 0).item()) < 1e-10


@pytest.mark.parametrize("splits", [1, 3, 4, 16, 32, 64])
def test_stage2_of_stage1_equals_unsplit_attention(splits):
    w = _small(31, [5, 100, 333], splits)
    full_o, full_l = stage1.attention_reference(w.q_rot, w.kv_cache, w.block_table, w.seq_lens,
                                                w.centroids, num_kv_heads=8)
    mid = stage1.stage1(w.q_rot, w.kv_cache, w.block_table, w.seq_lens, w.centroids, splits,
                        num_kv_heads=8)
    o, l = stage1.stage2(mid, w.seq_lens)
    assert np.abs(o - full_o).max() < 1e-12 and np.abs(l - full_l).max() < 1e-12


def test_empty_splits_untouched():
    w = _small(41, [3, 40], 32)
    sentinel = np.full((2, 32, 32, 129), 7.25)
    mid = stage1.stage1(w.q_rot, w.kv_cache, w.block_table, w.seq_lens, w.centroids, 32,
                        num_kv_heads=8, mid_o=sentinel.copy())
    for b, n in enumerate([3, 40]):
        live = -(-n // -(-n // 32))
        assert np.all(mid[b, :, live:] == 7.25)
        assert not np.any(mid[b, :, :live] == 7.25)


def test_full_decode_rotation_matches_matmul():
    rng = np.random.default_rng(51)
    w = _small(52, [64, 10], 4)
    query = rng.standard_normal((2, 32, 128)).astype(np.float16)
    rot = workloads.random_orthogonal(rng, 128)
    out, lse, _ = stage1.full_decode(query, rot, w.kv_cache, w.block_table, w.seq_lens,
                                     w.centroids, 4, num_kv_heads=8)
    q_rot = torch.from_numpy(query).double() @ torch.from_numpy(rot).double()
    o2, l2 = stage1.attention_reference(q_rot.numpy(), w.kv_cache, w.block_table, w.seq_lens,
                                        w.centroids, num_kv_heads=8)
    assert np.abs(out - o2).max() < 1e-12 and np.abs(lse - l2).max() < 1e-12


def test_planted_nibble_swap_is_caught(monkeypatch):
    """An oracle reading the high nibble first disagrees with torch attention."""
    w = _small(61, [48], 4)
    ref = _torch_split_reference(w, False, w.kv_cache)

    def swapped(packed):
        p = packed.astype(np.int64)
        out = np.empty(p.shape[:-1] + (2 * p.shape[-1],), np.int64)
        out[..., 0::2], out[..., 1::2] = (p >> 4) & 0xF, p & 0xF
        return out

    monkeypatch.setattr(layout, "unpack_nibbles", swapped)
    bad = stage1.stage1(w.q_rot, w.kv_cache, w.block_table, w.seq_lens, w.centroids, 4,
                        num_kv_heads=8)
    assert np.nanmax(np.abs(bad - ref)) > 1e-3


def test_planted_missing_norm_is_caught(monkeypatch):
    """An oracle that drops the per-token K norm disagrees with torch attention."""
    w = _small(62, [48], 4)
    ref = _torch_split_reference(w, False, w.kv_cache)
    orig = layout.gather_soa

    def no_norm(*a, **k):
        ki, kn, vc, vs, vz = orig(*a, **k)
        return ki, np.ones_like(kn), vc, vs, vz

    monkeypatch.setattr(layout, "gather_soa", no_norm)
    bad = stage1.stage1(w.q_rot, w.kv_cache, w.block_table, w.seq_lens, w.centroids, 4,
                        num_kv_heads=8)
    assert np.nanmax(np.abs(bad - ref)) > 1e-3
