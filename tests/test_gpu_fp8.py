"""FP8-key preset (turboquant_k8v4) on the GPU: the writer bit-exact against the oracle
writer (K bytes = E4M3 of the raw key, round to nearest even, saturating at +-448; V as
the 4-bit writer), and Stage1 / the decode entry against the oracle (max-abs 1e-4,
fp32)."""
import numpy as np
import pytest
import torch

from conftest import to_dev
from oracle import fp8 as ofp8
from oracle import native
from oracle import stage1 as ostage
from oracle import store as ostore
from tq4_decode import ops, workloads

pytestmark = pytest.mark.gpu
HK, D, BS = 8, 128, 16
SLOT = ofp8.slot_bytes(D)
TORCH = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_store_fp8_matches_oracle_writer(dev, dtype, layout):
    rng = np.random.default_rng(301)
    n_tok, n_blocks = 250, 20
    key = (rng.standard_normal((n_tok, HK, D)) * 40).astype(np.float32)
    key[0, 0, :8] = [460.0, -1e4, 448.0, 1e-3, -2.0 ** -9, 2.0 ** -10, 0.0, -0.0]  # saturation, subnormals
    value = (rng.standard_normal((n_tok, HK, D)) * 0.5).astype(np.float32)
    key = torch.from_numpy(key).to(TORCH[dtype]).float().numpy()
    value = torch.from_numpy(value).to(TORCH[dtype]).float().numpy()
    slots = rng.permutation(n_blocks * BS)[:n_tok].astype(np.int32)  # distinct slots
    slots[1:][rng.random(n_tok - 1) < 0.1] = -1  # token 0 (the special keys) is written
    cache0 = np.full((n_blocks, BS, HK, SLOT), 0x5A, dtype=np.uint8)
    cache = to_dev(cache0, dev)
    ops.store_fp8(to_dev(key, dev).to(TORCH[dtype]), to_dev(value, dev).to(TORCH[dtype]), cache,
                  to_dev(slots, dev), layout=layout)
    torch.cuda.synchronize()
    ref = ostore.store_fp8(key, value, slots, cache0.copy(), block_size=BS, is_aos=layout == "aos")
    got = cache.cpu().numpy()
    diff = np.nonzero(got.reshape(-1) != ref.reshape(-1))[0]
    assert diff.size == 0, f"{diff.size} bytes differ, first at {diff[:8]}"


def _fp8_workload(seed, lens, splits, hq=32, hk=HK, layout="soa"):
    rng = np.random.default_rng(seed)
    w = workloads.small(seed, len(lens), lens, splits, num_q_heads=hq, num_kv_heads=hk)
    nb = w.kv_cache.shape[0]
    n_tok = nb * BS
    key = (rng.standard_normal((n_tok, hk, D)) * 2).astype(np.float32)
    value = rng.standard_normal((n_tok, hk, D)).astype(np.float32)
    cache = np.zeros((nb, BS, hk, SLOT), np.uint8)
    ostore.store_fp8(key, value, np.arange(n_tok, dtype=np.int32), cache, block_size=BS,
                     is_aos=layout == "aos")
    query = rng.standard_normal((len(lens), hq, D)).astype(np.float32)
    return w, cache, query


def _stage1(dev, w, cache, query, splits, layout, sinks=None, kernel="auto"):
    mid = torch.full((w.batch, w.num_q_heads, splits, D + 1), float("nan"), device=dev)
    ops.stage1_fp8(to_dev(query, dev), to_dev(cache, dev), to_dev(w.block_table, dev),
                   to_dev(w.seq_lens, dev), mid, layout=layout,
                   sinks=None if sinks is None else to_dev(sinks, dev), kernel=kernel)
    torch.cuda.synchronize()
    return mid.cpu().numpy()


def _assert_parity(got, ref, tol=1e-4):
    """Max-abs bound 1e-4 on every mid_o value (outputs and LSE, fp32)."""
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "untouched-split pattern differs"
    err = np.nanmax(np.abs(got - ref))
    print(f"max-abs {err:.3e}")
    assert err <= tol


@pytest.mark.parametrize("layout", ["soa", "aos"])
@pytest.mark.parametrize("group,kernel", [(1, "auto"), (1, "simple"), (2, "xdl"), (4, "simple"), (4, "xdl"),
                                          (6, "xdl"), (8, "simple"), (8, "xdl"), (16, "auto"), (16, "simple")])
def test_stage1_fp8_matches_oracle(dev, layout, group, kernel):
    """Every group runs on the 16x16x32 MFMA kernel under auto (1 and 2 in 4-head waves with
    padding heads); both kernels are checked."""
    hk = 4
    w, cache, query = _fp8_workload(302, [1, 37, 600, 1025], 8, hq=hk * group, hk=hk, layout=layout)
    got = _stage1(dev, w, cache, query, 8, layout, kernel=kernel)
    ref = ostage.stage1(query, cache, w.block_table, w.seq_lens, None, 8, num_kv_heads=hk,
                        is_aos=layout == "aos", key_fp8=True)
    _assert_parity(got, ref)


def test_stage1_fp8_every_finite_byte(dev):
    """K bytes cover all 254 finite E4M3 codes (0x7F / 0xFF are NaN): the GPU decode of
    every byte enters the scores."""
    w, cache, query = _fp8_workload(303, [640, 300], 4)
    finite = np.array([b for b in range(256) if b not in (0x7F, 0xFF)], np.uint8)
    rng = np.random.default_rng(304)
    rec = ofp8.record_bytes(D)
    blocks = cache.reshape(cache.shape[0], -1)  # SoA: record (t, h) at (t * Hk + h) * rec
    for blk in range(cache.shape[0]):
        for r in range(BS * HK):
            blocks[blk, r * rec:r * rec + D] = rng.permutation(np.resize(finite, D))
    ref = ostage.stage1(query, cache, w.block_table, w.seq_lens, None, 4, num_kv_heads=HK, key_fp8=True)
    for kernel in ("simple", "xdl"):
        got = _stage1(dev, w, cache, query, 4, "soa", kernel=kernel)
        # E4M3 keys up to +-448 give scores (and LSEs) in the thousands, where one fp32 ulp
        # is above 1e-4: the outputs keep the absolute bound, the LSE column a relative one
        _assert_parity(got[..., :D], ref[..., :D])
        lse_err = np.nanmax(np.abs(got[..., D] - ref[..., D]) / np.maximum(1.0, np.abs(ref[..., D])))
        print(f"LSE relative {lse_err:.3e}")
        assert lse_err <= 1e-4


@pytest.mark.parametrize("kernel", ["simple", "xdl"])
def test_stage1_fp8_with_sinks(dev, kernel):
    w, cache, query = _fp8_workload(305, [200, 1, 999], 8)
    sinks = np.random.default_rng(306).normal(0, 2, 32).astype(np.float32)
    got = _stage1(dev, w, cache, query, 8, "soa", sinks, kernel=kernel)
    ref = ostage.stage1(query, cache, w.block_table, w.seq_lens, None, 8, num_kv_heads=HK,
                        key_fp8=True, sinks=sinks)
    _assert_parity(got, ref)


@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_fp8_store_then_decode_entry(dev, layout):
    """Reference call shapes end to end: the writer with key_fp8=True fills the cache, the
    decode entry with key_fp8=True reads it (query unrotated), against the oracle."""
    from tq4_decode import aos_decode, aos_store, soa_decode, soa_store

    rng = np.random.default_rng(307)
    lens = np.array([700, 5, 1300], np.int32)
    need = (lens + BS - 1) // BS
    nb = int(need.sum()) + 2
    bt = np.zeros((3, int(need.max())), np.int32)
    perm = rng.permutation(nb).astype(np.int32)
    pos = 0
    for b in range(3):
        bt[b, :need[b]] = perm[pos:pos + need[b]]
        pos += need[b]
    n_tok = int(lens.sum())
    key = rng.standard_normal((n_tok, HK, D)).astype(np.float32)
    value = rng.standard_normal((n_tok, HK, D)).astype(np.float32)
    slots = np.concatenate([bt[b, np.arange(lens[b]) // BS] * BS + np.arange(lens[b]) % BS
                            for b in range(3)]).astype(np.int32)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    cache = torch.zeros(nb, BS, HK, SLOT, dtype=torch.uint8, device=dev)
    store_mod = aos_store if layout == "aos" else soa_store
    store_mod.triton_turboquant_store(t(key).half(), t(value).half(), cache, t(slots),
                                      torch.eye(D, device=dev), torch.zeros(15, device=dev),
                                      mse_bits=8, key_packed_size=D, value_quant_bits=4, key_fp8=True)
    query = rng.standard_normal((3, 32, D)).astype(np.float16)
    dec = aos_decode if layout == "aos" else soa_decode
    out = dec.triton_turboquant_decode_attention(
        t(query), cache, t(bt), t(lens), torch.eye(D, device=dev), torch.zeros(16, device=dev),
        D ** -0.5, mse_bits=8, key_packed_size=D, value_quant_bits=4, key_fp8=True,
        max_num_kv_splits=16)
    torch.cuda.synchronize()
    ref_cache = ostore.store_fp8(torch.from_numpy(key).half().float().numpy(),
                                 torch.from_numpy(value).half().float().numpy(), slots,
                                 np.zeros((nb, BS, HK, SLOT), np.uint8), block_size=BS,
                                 is_aos=layout == "aos")
    assert np.array_equal(cache.cpu().numpy(), ref_cache)
    mid = ostage.stage1(query.astype(np.float32), ref_cache, bt, lens, None, 16, num_kv_heads=HK,
                        is_aos=layout == "aos", key_fp8=True)
    ro, _ = ostage.stage2(mid, lens)
    err = np.abs(out.float().cpu().numpy() - ro).max()
    print(f"{layout} fp8 decode entry fp16 max-abs {err:.3e}")
    assert err <= 1e-4 + 2.0 ** -11 * np.abs(ro).max()


@pytest.mark.parametrize("layout", ["soa", "aos"])
@pytest.mark.parametrize("group", [4, 8])
def test_stage1_fp8_xdl_long_and_ragged(dev, layout, group):
    """The MFMA kernel over many splits per wave, a 4096-token sequence, empty and
    one-token sequences, at the head counts of the 4-bit workloads."""
    hk = 8 // (group // 4)
    w, cache, query = _fp8_workload(308, [4096, 0, 1, 333, 2049], 32, hq=hk * group, hk=hk, layout=layout)
    got = _stage1(dev, w, cache, query, 32, layout, kernel="xdl")
    ref = ostage.stage1(query, cache, w.block_table, w.seq_lens, None, 32, num_kv_heads=hk,
                        is_aos=layout == "aos", key_fp8=True)
    _assert_parity(got, ref)


@pytest.mark.parametrize("layout", ["soa", "aos"])
@pytest.mark.parametrize("bs", [32, 64])
def test_stage1_fp8_xdl_larger_blocks(dev, layout, bs):
    """The 16x16x32 kernel at 32 / 64-token KV blocks (piece and metadata offsets of the
    192 / 196-byte records)."""
    rng = np.random.default_rng(309 + bs)
    lens = [130, 511, 64, 2000]
    w = workloads.small(309, len(lens), lens, 8, block_size=bs)
    nb = w.kv_cache.shape[0]
    n_tok = nb * bs
    key = (rng.standard_normal((n_tok, HK, D)) * 2).astype(np.float32)
    value = rng.standard_normal((n_tok, HK, D)).astype(np.float32)
    cache = np.zeros((nb, bs, HK, SLOT), np.uint8)
    ostore.store_fp8(key, value, np.arange(n_tok, dtype=np.int32), cache, block_size=bs,
                     is_aos=layout == "aos")
    query = rng.standard_normal((len(lens), 32, D)).astype(np.float32)
    got = _stage1(dev, w, cache, query, 8, layout, kernel="xdl")
    ref = ostage.stage1(query, cache, w.block_table, w.seq_lens, None, 8, num_kv_heads=HK,
                        block_size=bs, is_aos=layout == "aos", key_fp8=True)
    _assert_parity(got, ref)


@pytest.mark.parametrize("layout", ["soa", "aos"])
@pytest.mark.parametrize("bs", [64, 256])
def test_fp8_larger_kv_blocks(dev, layout, bs):
    """The 16x16x32 kernel at 64 / 256-token KV blocks (several 16-token pieces per block: the
    piece and metadata offsets use the 192-byte FP8 record)."""
    rng = np.random.default_rng(330 + bs)
    lens = [130, 511, 64, 2000]
    w = workloads.small(330 + bs, len(lens), lens, 8, num_q_heads=32, num_kv_heads=HK, block_size=bs)
    nb = w.kv_cache.shape[0]
    key = (rng.standard_normal((nb * bs, HK, D)) * 2).astype(np.float32)
    value = rng.standard_normal((nb * bs, HK, D)).astype(np.float32)
    cache = np.zeros((nb, bs, HK, SLOT), np.uint8)
    ostore.store_fp8(key, value, np.arange(nb * bs, dtype=np.int32), cache, block_size=bs, is_aos=layout == "aos")
    query = rng.standard_normal((len(lens), 32, D)).astype(np.float32)
    mid = torch.full((len(lens), 32, 8, D + 1), float("nan"), device=dev)
    ops.stage1_fp8(to_dev(query, dev), to_dev(cache, dev), to_dev(w.block_table, dev), to_dev(w.seq_lens, dev),
                   mid, layout=layout, kernel="xdl")
    torch.cuda.synchronize()
    ref = ostage.stage1(query, cache, w.block_table, w.seq_lens, None, 8, num_kv_heads=HK, block_size=bs,
                        is_aos=layout == "aos", key_fp8=True)
    _assert_parity(mid.cpu().numpy(), ref)


@pytest.mark.parametrize("kernel", ["xdl", "simple"])
def test_fp8_attention_scale(dev, kernel):
    """A non-default attn_scale (0.03: FP8 keys carry the raw key magnitudes) reaches the scores."""
    w, cache, query = _fp8_workload(340, [700, 33, 1500, 129], 8)
    got = np.asarray(_stage1_scaled(dev, w, cache, query, kernel, 0.03))
    ref = ostage.stage1(query, cache, w.block_table, w.seq_lens, None, 8, num_kv_heads=HK, block_size=BS,
                        key_fp8=True, attn_scale=0.03)
    _assert_parity(got, ref)


def _stage1_scaled(dev, w, cache, query, kernel, scale):
    mid = torch.full((w.batch, w.num_q_heads, 8, D + 1), float("nan"), device=dev)
    ops.stage1_fp8(to_dev(query, dev), to_dev(cache, dev), to_dev(w.block_table, dev), to_dev(w.seq_lens, dev), mid,
                   layout="soa", kernel=kernel, attn_scale=scale)
    torch.cuda.synchronize()
    return mid.cpu().numpy()
