"""Bit-width presets on the GPU (turboquant_k3v4_nc: 3-bit K / 4-bit V, turboquant_3bit_nc:
3-bit K / 3-bit V).  Writer bar as the 4-bit writer's: V codes, scale and min bit-exact
against the oracle writer, a K index off by one bucket only where y lies within float
rounding of a midpoint, the stored K scalar within 1 fp16 ulp, other bytes untouched.
Stage1 / the decode entry against the oracle at max-abs 1e-4 (fp32 mid_o)."""
import math

import numpy as np
import pytest
import torch

from conftest import to_dev
from oracle import bits as obits
from oracle import stage1 as ostage
from oracle import store as ostore
from tq4_decode import codebook, ops, workloads

pytestmark = pytest.mark.gpu
D, BS = 128, 16
PRESETS = [(3, 4), (3, 3)]
TORCH = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _codebook(kb):
    cents = codebook.centroids(D, kb).astype(np.float32)
    return cents, ((cents[:-1] + cents[1:]) * np.float32(0.5)).astype(np.float32)


def _rotated(key, rot_t):
    k = key.astype(np.float64)
    return (k / (np.sqrt((k ** 2).sum(-1, keepdims=True)) + 1e-8)) @ rot_t.astype(np.float64)


@pytest.mark.parametrize("preset", PRESETS)
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_store_preset_matches_oracle_writer(dev, preset, dtype, layout):
    kb, vb = preset
    rng = np.random.default_rng(401 + vb)
    hk, n_tok, n_blocks = 8, 300, 24
    key = torch.from_numpy(rng.standard_normal((n_tok, hk, D)).astype(np.float32)).to(TORCH[dtype]).float().numpy()
    value = torch.from_numpy((rng.standard_normal((n_tok, hk, D)) * 0.7 + 0.1).astype(np.float32)
                             ).to(TORCH[dtype]).float().numpy()
    slots = rng.permutation(n_blocks * BS)[:n_tok].astype(np.int32)
    slots[rng.random(n_tok) < 0.1] = -1
    rot_t = workloads.random_orthogonal(rng, D)
    cents, mids = _codebook(kb)
    aos = layout == "aos"
    slot = obits.slot_bytes(D, kb, vb)
    cache0 = np.full((n_blocks, BS, hk, slot), 0xA5, dtype=np.uint8)
    cache = to_dev(cache0, dev)
    ops.store_preset(to_dev(key, dev).to(TORCH[dtype]), to_dev(value, dev).to(TORCH[dtype]), cache,
                     to_dev(slots, dev), to_dev(rot_t, dev), to_dev(mids, dev), to_dev(cents, dev),
                     key_bits=kb, value_bits=vb, layout=layout, norm_correction=not aos)
    torch.cuda.synchronize()
    got = cache.cpu().numpy()
    ref = obits.store(key, value, slots, rot_t, cents, cache0.copy(), kb, vb, is_aos=aos)
    keep = np.nonzero(slots >= 0)[0]
    blocks, offs = slots[keep] // BS, slots[keep] % BS
    near_tie = np.abs(_rotated(key[keep], rot_t)[..., None] - mids.astype(np.float64)).min(-1) < 1e-6
    for h in range(hk):
        gk, gn, gv, gs, gz = obits.gather(got, blocks, offs, h, BS, hk, D, kb, vb, aos)
        rk, rn, rv, rs, rz = obits.gather(ref, blocks, offs, h, BS, hk, D, kb, vb, aos)
        assert np.array_equal(gv, rv), "V codes differ"
        assert np.array_equal(gs, rs) and np.array_equal(gz, rz), "V scale / min differ"
        diff = gk != rk
        assert not np.any(diff & ~near_tie[:, h]), "K index differs away from a midpoint"
        assert np.all(np.abs(gk - rk)[diff] == 1)
        clean = ~diff.any(-1)
        assert np.all(np.abs(gn - rn)[clean] <= np.abs(rn)[clean] * 2.0 ** -10), "K scalar off by > 1 ulp"
    # bytes outside the written records keep the fill
    written = np.zeros(cache0.size, dtype=bool)
    stride, rec = BS * hk * slot, 16 * (kb + vb)
    for blk, off in zip(blocks.astype(np.int64), offs.astype(np.int64)):
        for h in range(hk):
            if aos:
                b0 = blk * stride + (off * hk + h) * slot
                written[b0:b0 + rec + 6] = True
            else:
                b0 = blk * stride + (off * hk + h) * rec
                written[b0:b0 + rec] = True
                meta = blk * stride + BS * hk * rec + ((h * 3) * BS + off) * 2
                for f in range(3):
                    written[meta + 2 * f * BS:meta + 2 * f * BS + 2] = True
    assert np.array_equal(got.reshape(-1)[~written], cache0.reshape(-1)[~written])
    assert np.array_equal(ref.reshape(-1)[~written], cache0.reshape(-1)[~written])


def _table(rng, lens, bs=BS):
    lens = np.asarray(lens, np.int32)
    need = (lens + bs - 1) // bs
    nb = int(need.sum()) + 2
    bt = np.zeros((len(lens), max(1, int(need.max()))), np.int32)
    perm = rng.permutation(nb).astype(np.int32)
    pos = 0
    for b in range(len(lens)):
        bt[b, :need[b]] = perm[pos:pos + need[b]]
        pos += need[b]
    return bt, lens, nb


def _preset_cache(seed, lens, hk, kb, vb, layout, bs=BS):
    rng = np.random.default_rng(seed)
    bt, lens, nb = _table(rng, lens, bs)
    n_tok = nb * bs
    key = rng.standard_normal((n_tok, hk, D)).astype(np.float32)
    value = (rng.standard_normal((n_tok, hk, D)) * 0.8).astype(np.float32)
    cents, _ = _codebook(kb)
    cache = np.zeros((nb, bs, hk, obits.slot_bytes(D, kb, vb)), np.uint8)
    obits.store(key, value, np.arange(n_tok), workloads.random_orthogonal(rng, D), cents, cache, kb, vb,
                block_size=bs, is_aos=layout == "aos")
    return bt, lens, cache, cents, rng


def _stage1(dev, q_rot, cache, bt, lens, cents, splits, kb, vb, layout, sinks=None, kernel="simple"):
    mid = torch.full((q_rot.shape[0], q_rot.shape[1], splits, D + 1), float("nan"), device=dev)
    ops.stage1_preset(to_dev(q_rot, dev), to_dev(cache, dev), to_dev(bt, dev), to_dev(lens, dev),
                      to_dev(cents, dev), mid, key_bits=kb, value_bits=vb, layout=layout,
                      sinks=None if sinks is None else to_dev(sinks, dev), kernel=kernel)
    torch.cuda.synchronize()
    return mid.cpu().numpy()


def _assert_parity(got, ref, tol=1e-4):
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "untouched-split pattern differs"
    err = np.nanmax(np.abs(got - ref))
    print(f"max-abs {err:.3e}")
    assert err <= tol


@pytest.mark.parametrize("preset", PRESETS)
@pytest.mark.parametrize("layout", ["soa", "aos"])
@pytest.mark.parametrize("group", [1, 4, 8, 16])
def test_stage1_preset_matches_oracle(dev, preset, layout, group):
    kb, vb = preset
    hk = 4
    bt, lens, cache, cents, rng = _preset_cache(410 + group, [1, 37, 600, 1025, 0], hk, kb, vb, layout)
    q = rng.standard_normal((len(lens), hk * group, D)).astype(np.float32)
    got = _stage1(dev, q, cache, bt, lens, cents, 8, kb, vb, layout)
    ref = ostage.stage1(q, cache, bt, lens, cents, 8, num_kv_heads=hk, is_aos=layout == "aos",
                        bits=preset)
    _assert_parity(got, ref)


@pytest.mark.parametrize("preset", PRESETS)
@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_stage1_preset_block32_group2(dev, preset, layout):
    """32-token KV blocks and GQA 2 (block stride 32 x Hk x slot)."""
    kb, vb = preset
    hk = 2
    bt, lens, cache, cents, rng = _preset_cache(450, [33, 700, 64], hk, kb, vb, layout, bs=32)
    q = rng.standard_normal((3, hk * 2, D)).astype(np.float32)
    got = _stage1(dev, q, cache, bt, lens, cents, 5, kb, vb, layout)
    ref = ostage.stage1(q, cache, bt, lens, cents, 5, num_kv_heads=hk, block_size=32,
                        is_aos=layout == "aos", bits=preset)
    _assert_parity(got, ref)


@pytest.mark.parametrize("preset", PRESETS)
def test_stage1_preset_with_sinks(dev, preset):
    kb, vb = preset
    bt, lens, cache, cents, rng = _preset_cache(420, [200, 1, 999], 8, kb, vb, "soa")
    q = rng.standard_normal((3, 32, D)).astype(np.float32)
    sinks = rng.normal(0, 2, 32).astype(np.float32)
    got = _stage1(dev, q, cache, bt, lens, cents, 8, kb, vb, "soa", sinks)
    ref = ostage.stage1(q, cache, bt, lens, cents, 8, num_kv_heads=8, bits=preset, sinks=sinks)
    _assert_parity(got, ref)


@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_generic_four_bit_path_matches_the_four_bit_kernel(dev, layout):
    """The bit-width kernel at 4/4 (centroids read directly) against the 4-bit VALU kernel
    (pair LUT) on the same cache: the same sums in the same order."""
    w = workloads.small(430, 4, [1, 300, 2048, 77], 8)
    cache = workloads.soa_to_aos(w.kv_cache, w.centroids, 8) if layout == "aos" else w.kv_cache
    t = lambda a: to_dev(a, dev)  # noqa: E731
    a = torch.full((4, 32, 8, D + 1), float("nan"), device=dev)
    b = a.clone()
    ops.stage1(t(w.q_rot), t(cache), t(w.block_table), t(w.seq_lens), t(w.pair_lut), a, layout=layout,
               kernel="simple")
    ops.stage1_preset(t(w.q_rot), t(cache), t(w.block_table), t(w.seq_lens), t(w.centroids), b,
                      key_bits=4, value_bits=4, layout=layout)
    torch.cuda.synchronize()
    a, b = a.cpu().numpy(), b.cpu().numpy()
    assert np.array_equal(np.isnan(a), np.isnan(b))
    err = np.nanmax(np.abs(a - b))
    print(f"4/4 generic vs 4-bit kernel max-abs {err:.3e}")
    assert err <= 1e-6


@pytest.mark.parametrize("preset", PRESETS)
@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_preset_store_then_decode_entry(dev, preset, layout):
    """Reference call shapes end to end: the writer with mse_bits=3 fills the cache, the
    decode entry reads it; checked against the oracle decode of the bytes written."""
    from tq4_decode import aos_decode, aos_store, soa_decode, soa_store

    kb, vb = preset
    rng = np.random.default_rng(440 + vb)
    hk = 8
    bt, lens, nb = _table(rng, [700, 5, 1300, 0])
    n_tok = int(lens.sum())
    key = rng.standard_normal((n_tok, hk, D)).astype(np.float32)
    value = rng.standard_normal((n_tok, hk, D)).astype(np.float32)
    slots = np.concatenate([bt[b, np.arange(lens[b]) // BS] * BS + np.arange(lens[b]) % BS
                            for b in range(len(lens))]).astype(np.int32)
    rot_t = workloads.random_orthogonal(rng, D)
    cents, mids = _codebook(kb)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    slot = obits.slot_bytes(D, kb, vb)
    cache = torch.zeros(nb, BS, hk, slot, dtype=torch.uint8, device=dev)
    kps = D * kb // 8 + 2
    if layout == "aos":
        aos_store.triton_turboquant_store(t(key).half(), t(value).half(), cache, t(slots), t(rot_t),
                                          t(mids), mse_bits=kb, key_packed_size=kps, value_quant_bits=vb)
    else:
        soa_store.triton_turboquant_store(t(key).half(), t(value).half(), cache, t(slots), t(rot_t),
                                          t(mids), mse_bits=kb, key_packed_size=kps, value_quant_bits=vb,
                                          centroids=t(cents), norm_correction=True)
    query = rng.standard_normal((len(lens), 32, D)).astype(np.float16)
    dec = aos_decode if layout == "aos" else soa_decode
    out = dec.triton_turboquant_decode_attention(
        t(query), cache, t(bt), t(lens), t(rot_t.T.copy()), t(cents), 1 / math.sqrt(D), mse_bits=kb,
        key_packed_size=kps, value_quant_bits=vb, norm_correction=True, max_num_kv_splits=16)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16 and out.shape == (len(lens), 32, D)
    q_rot = (query.astype(np.float64) @ rot_t.astype(np.float64)).astype(np.float32)
    mid = ostage.stage1(q_rot, cache.cpu().numpy(), bt, lens, cents, 16, num_kv_heads=hk,
                        is_aos=layout == "aos", bits=preset)
    live = lens > 0  # the oracle merge takes the non-empty sequences
    ro, _ = ostage.stage2(mid[live], lens[live])
    diff = np.abs(out.float().cpu().numpy()[live] - ro)
    print(f"{layout} {kb}/{vb} decode entry fp16 max-abs {diff.max():.3e}")
    # fp16 output: rounding to nearest (2^-11 relative) on top of the fp32 Stage1 bound
    assert np.all(diff <= 2.0 ** -11 * np.abs(ro) + 1e-4)
    with pytest.raises(RuntimeError):  # a cache of another slot size is rejected
        dec.triton_turboquant_decode_attention(
            t(query), cache, t(bt), t(lens), t(rot_t.T.copy()), t(cents), 1 / math.sqrt(D),
            mse_bits=kb, key_packed_size=kps, value_quant_bits=7 - vb, norm_correction=True)


@pytest.mark.parametrize("vb", [4, 3])
@pytest.mark.parametrize("layout", ["soa", "aos"])
@pytest.mark.parametrize("group", [1, 2, 4, 6, 8, 16])
def test_stage1_k3_on_the_mfma_kernel(dev, layout, group, vb):
    """3-bit K / 4- or 3-bit V on the 16x16x32 kernel (the auto choice; groups 1 and 2 in
    4-head waves with padding heads): many splits per wave, a 4096-token sequence, empty and
    one-token sequences, sinks.  Bound 1e-4 absolute on every mid_o value."""
    hk = {1: 8, 2: 8, 4: 8, 6: 4, 8: 4, 16: 2}[group]
    bt, lens, cache, cents, rng = _preset_cache(460 + group, [4096, 0, 1, 333, 2049], hk, 3, vb, layout)
    q = rng.standard_normal((len(lens), hk * group, D)).astype(np.float32)
    sinks = rng.normal(0, 2, hk * group).astype(np.float32)
    for sk in (None, sinks):
        got = _stage1(dev, q, cache, bt, lens, cents, 32, 3, vb, layout, sinks=sk, kernel="xdl")
        ref = ostage.stage1(q, cache, bt, lens, cents, 32, num_kv_heads=hk, is_aos=layout == "aos",
                            bits=(3, vb), sinks=sk)
        _assert_parity(got, ref, tol=2e-5)  # inside the 1e-4 bar: fp32-grade on this data
    auto = _stage1(dev, q, cache, bt, lens, cents, 32, 3, vb, layout, kernel="auto")
    xdl = _stage1(dev, q, cache, bt, lens, cents, 32, 3, vb, layout, kernel="xdl")
    assert np.array_equal(auto, xdl, equal_nan=True), "auto runs the 16x16x32 kernel"


@pytest.mark.parametrize("vb", [4, 3])
@pytest.mark.parametrize("layout", ["soa", "aos"])
@pytest.mark.parametrize("bs", [32, 64, 128, 256])
def test_stage1_k3_mfma_larger_blocks(dev, layout, bs, vb):
    """The 16x16x32 kernel at 32 - 256-token KV blocks (several 16-token pieces per block:
    the piece and metadata offsets use the preset's record size)."""
    hk = 8
    bt, lens, cache, cents, rng = _preset_cache(470 + bs, [130, 511, 64, 2000], hk, 3, vb, layout, bs=bs)
    q = rng.standard_normal((len(lens), hk * 4, D)).astype(np.float32)
    got = _stage1(dev, q, cache, bt, lens, cents, 8, 3, vb, layout, kernel="xdl")
    ref = ostage.stage1(q, cache, bt, lens, cents, 8, num_kv_heads=hk, block_size=bs,
                        is_aos=layout == "aos", bits=(3, vb))
    _assert_parity(got, ref)


@pytest.mark.parametrize("preset", PRESETS)
@pytest.mark.parametrize("kernel", ["xdl", "simple"])
def test_stage1_preset_attention_scale(dev, preset, kernel):
    """A non-default attn_scale (0.3 instead of 1 / sqrt(D)) reaches the scores of the presets."""
    kb, vb = preset
    hk = 8
    bt, lens, cache, cents, rng = _preset_cache(480 + vb, [700, 33, 1500, 129], hk, kb, vb, "soa")
    q = rng.standard_normal((len(lens), hk * 4, D)).astype(np.float32)
    mid = torch.full((len(lens), hk * 4, 8, D + 1), float("nan"), device=dev)
    ops.stage1_preset(to_dev(q, dev), to_dev(cache, dev), to_dev(bt, dev), to_dev(lens, dev), to_dev(cents, dev), mid,
                      key_bits=kb, value_bits=vb, layout="soa", attn_scale=0.3, kernel=kernel)
    torch.cuda.synchronize()
    ref = ostage.stage1(q, cache, bt, lens, cents, 8, num_kv_heads=hk, block_size=BS, bits=(kb, vb), attn_scale=0.3)
    _assert_parity(mid.cpu().numpy(), ref)
