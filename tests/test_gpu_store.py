"""Cache writer on the GPU (tq4_store through the C ABI) vs the oracle writer.

Bar: V codes, V scale and V min are bit-exact (the same fp32 operations in the same
order); a K index may differ from the oracle's only where y lies within float rounding
of a midpoint (the rotation sums in a different order), and then by one bucket; the
stored K scalar within 1 fp16 ulp; bytes of slots not written stay untouched.  Round
trip: decoding a cache this writer filled matches the oracle's decode of the same bytes.
"""
import numpy as np
import pytest
import torch

from conftest import to_dev
from oracle import layout as OL
from oracle import native
from oracle import store as ostore
from tq4_decode import codebook, ops, workloads

pytestmark = pytest.mark.gpu
HK, D, BS = 8, 128, 16
TORCH = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def make_inputs(seed, n_tok, n_blocks, dtype, scale=1.0):
    rng = np.random.default_rng(seed)
    key = (rng.standard_normal((n_tok, HK, D)) * scale).astype(np.float32)
    value = (rng.standard_normal((n_tok, HK, D)) * 0.7 + 0.1).astype(np.float32)
    # round to the input dtype so both sides quantize the same numbers
    key = torch.from_numpy(key).to(TORCH[dtype]).float().numpy()
    value = torch.from_numpy(value).to(TORCH[dtype]).float().numpy()
    slots = rng.permutation(n_blocks * BS)[:n_tok].astype(np.int32)
    slots[rng.random(n_tok) < 0.1] = -1  # skipped tokens
    rot_t = workloads.random_orthogonal(rng, D)
    cents = codebook.centroids(D, 4)
    mids = ((cents[:-1] + cents[1:]) * np.float32(0.5)).astype(np.float32)
    return key, value, slots, rot_t, cents, mids


def gpu_store(dev, key, value, slots, rot_t, cents, mids, cache0, dtype, layout, nc):
    cache = to_dev(cache0, dev)
    ops.store(to_dev(key, dev).to(TORCH[dtype]), to_dev(value, dev).to(TORCH[dtype]), cache,
              to_dev(slots, dev), to_dev(rot_t, dev), to_dev(mids, dev), to_dev(cents, dev),
              layout=layout, norm_correction=nc)
    torch.cuda.synchronize()
    return cache.cpu().numpy()


def rotated(key, rot_t):
    k = key.astype(np.float64)
    norm = np.sqrt((k ** 2).sum(-1, keepdims=True))
    return (k / (norm + 1e-8)) @ rot_t.astype(np.float64)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_store_matches_oracle_writer(dev, dtype, layout):
    n_tok, n_blocks = 300, 24
    key, value, slots, rot_t, cents, mids = make_inputs(11, n_tok, n_blocks, dtype)
    aos = layout == "aos"
    cache0 = np.full((n_blocks, BS, HK, 134), 0xA5, dtype=np.uint8)
    got = gpu_store(dev, key, value, slots, rot_t, cents, mids, cache0, dtype, layout, not aos)
    ref = ostore.store(key, value, slots, rot_t, cents, cache0.copy(), block_size=BS, is_aos=aos)

    keep = np.nonzero(slots >= 0)[0]
    blocks, offs = slots[keep] // BS, slots[keep] % BS
    gather = OL.gather_aos if aos else OL.gather_soa
    y = rotated(key[keep], rot_t)
    near_tie = np.abs(y[..., None] - mids.astype(np.float64)).min(-1) < 1e-6
    for h in range(HK):
        gk, gn, gv, gs, gz = gather(got, blocks, offs, h, BS, HK, D)
        rk, rn, rv, rs, rz = gather(ref, blocks, offs, h, BS, HK, D)
        assert np.array_equal(gv, rv), "V codes differ"
        assert np.array_equal(gs, rs) and np.array_equal(gz, rz), "V scale / min differ"
        diff = gk != rk
        assert not np.any(diff & ~near_tie[:, h]), "K index differs away from a midpoint"
        assert np.all(np.abs(gk - rk)[diff] == 1)
        clean = ~diff.any(-1)  # a tie changes sum(c[idx]^2), so the scalar is checked elsewhere
        assert np.all(np.abs(gn - rn)[clean] <= np.abs(rn)[clean] * 2.0 ** -10), "K scalar off by > 1 ulp"
        print(f"head {h}: K index ties {int(diff.sum())}")
    # bytes outside the written records keep the fill
    written = np.zeros(cache0.size, dtype=bool)
    stride = BS * HK * 134
    for blk, off in zip(blocks.astype(np.int64), offs.astype(np.int64)):
        for h in range(HK):
            if aos:
                b0 = blk * stride + (off * HK + h) * 134
                written[b0:b0 + 134] = True
            else:
                b0 = blk * stride + (off * HK + h) * 128
                written[b0:b0 + 128] = True
                meta = blk * stride + BS * HK * 128 + ((h * 3) * BS + off) * 2
                for f in range(3):
                    written[meta + 2 * f * BS:meta + 2 * f * BS + 2] = True
    assert np.array_equal(got.reshape(-1)[~written], cache0.reshape(-1)[~written])
    assert np.array_equal(ref.reshape(-1)[~written], cache0.reshape(-1)[~written])


def check_against_oracle(dev, key, value, slots, rot_t, cents, n_blocks, dtype="f32"):
    mids = ((cents[:-1] + cents[1:]) * np.float32(0.5)).astype(np.float32)
    cache0 = np.zeros((n_blocks, BS, HK, 134), dtype=np.uint8)
    got = gpu_store(dev, key, value, slots, rot_t, cents, mids, cache0, dtype, "soa", True)
    ref = ostore.store(key, value, slots, rot_t, cents, cache0.copy(), block_size=BS)
    keep = np.nonzero(slots >= 0)[0]
    blocks, offs = slots[keep] // BS, slots[keep] % BS
    y = rotated(key[keep], rot_t)
    near_tie = np.abs(y[..., None] - mids.astype(np.float64)).min(-1) < 1e-6
    ties = 0
    for h in range(HK):
        gk, gn, gv, gs, gz = OL.gather_soa(got, blocks, offs, h, BS, HK, D)
        rk, rn, rv, rs, rz = OL.gather_soa(ref, blocks, offs, h, BS, HK, D)
        assert np.array_equal(gv, rv), "V codes differ"
        assert np.array_equal(gs, rs) and np.array_equal(gz, rz), "V scale / min differ"
        diff = gk != rk
        assert not np.any(diff & ~near_tie[:, h]), "K index differs away from a midpoint"
        clean = ~diff.any(-1)
        assert np.all(np.abs(gn - rn)[clean] <= np.abs(rn)[clean] * 2.0 ** -10)
        ties += int(diff.sum())
    return ties


def test_store_codebook_with_close_midpoints(dev):
    """Two midpoints closer than a bucketize table cell: the writer counts midpoints one by
    one instead of using the table; indices still match the oracle's."""
    rng = np.random.default_rng(15)
    n_tok = 200
    key = rng.standard_normal((n_tok, HK, D)).astype(np.float32)
    value = rng.standard_normal((n_tok, HK, D)).astype(np.float32)
    slots = rng.permutation(16 * BS)[:n_tok].astype(np.int32)
    cents = codebook.centroids(D, 4).astype(np.float32).copy()
    cents[7], cents[9] = cents[8] - np.float32(1e-4), cents[8] + np.float32(1e-4)
    mids = (cents[:-1] + cents[1:]) * np.float32(0.5)
    assert np.all(np.diff(cents) > 0) and mids[8] - mids[7] < 2e-4  # midpoints 7, 8 1e-4 apart
    ties = check_against_oracle(dev, key, value, slots, workloads.random_orthogonal(rng, D), cents, 16)
    print(f"K index ties {ties}")


def test_store_values_on_code_boundaries(dev):
    """V rows on a half-step grid: many quotients (v - min) / scale + 0.5 land exactly on an
    integer, where the reciprocal shortcut could round to the other code."""
    rng = np.random.default_rng(16)
    n_tok = 256
    key = rng.standard_normal((n_tok, HK, D)).astype(np.float32)
    steps = rng.integers(0, 31, (n_tok, HK, D)).astype(np.float32)
    steps[..., 0], steps[..., 1] = 0, 30  # range = 15 steps -> scale = step
    step = rng.choice(np.float32([0.5, 0.1, 0.3, 1.7, 3e-3]), (n_tok, HK, 1)).astype(np.float32)
    value = (steps * np.float32(0.5) * step - np.float32(1.3)).astype(np.float32)
    slots = rng.permutation(16 * BS)[:n_tok].astype(np.int32)
    cents = codebook.centroids(D, 4)
    check_against_oracle(dev, key, value, slots, workloads.random_orthogonal(rng, D), cents, 16)


def test_store_then_decode_round_trip(dev):
    """Fill a paged cache with the GPU writer (prefill of 3 sequences), then decode it on
    the GPU and with the oracle."""
    rng = np.random.default_rng(12)
    lens = np.array([700, 129, 1500], dtype=np.int32)
    need = (lens + BS - 1) // BS
    n_blocks = int(need.sum()) + 2
    perm = rng.permutation(n_blocks).astype(np.int32)
    bt = np.zeros((3, int(need.max())), dtype=np.int32)
    pos = 0
    for b in range(3):
        bt[b, :need[b]] = perm[pos:pos + need[b]]
        pos += need[b]
    n_tok = int(lens.sum())
    key, value, _, rot_t, cents, mids = make_inputs(13, n_tok, n_blocks, "bf16")
    slots = np.concatenate([bt[b, np.arange(lens[b]) // BS] * BS + np.arange(lens[b]) % BS
                            for b in range(3)]).astype(np.int32)
    cache0 = np.zeros((n_blocks, BS, HK, 134), dtype=np.uint8)
    cache = gpu_store(dev, key, value, slots, rot_t, cents, mids, cache0, "bf16", "soa", True)
    w = workloads.Workload("stored", rng.standard_normal((3, 32, D), dtype=np.float32), cache, bt,
                           lens, cents, 8, HK)
    mid = torch.full((3, 32, 8, D + 1), float("nan"), device=dev)
    ops.stage1(to_dev(w.q_rot, dev), to_dev(cache, dev), to_dev(bt, dev), to_dev(lens, dev),
               to_dev(w.pair_lut, dev), mid)
    torch.cuda.synchronize()
    ref = native.stage1(w.q_rot, cache, bt, lens, cents, 8, num_kv_heads=HK)
    err = np.nanmax(np.abs(mid.cpu().numpy() - ref))
    print(f"decode of the stored cache: max-abs {err:.3e}")
    assert err <= 1e-4


def test_reference_store_signature_and_skipped_slots(dev):
    key, value, slots, rot_t, cents, mids = make_inputs(14, 40, 4, "f16")
    slots[:] = -1
    slots[5] = 17
    cache0 = np.full((4, BS, HK, 134), 0x3C, dtype=np.uint8)
    cache = to_dev(cache0, dev)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    ops.triton_turboquant_store(t(key).half(), t(value).half(), cache, t(slots), t(rot_t), t(mids),
                                mse_bits=4, key_packed_size=66, value_quant_bits=4,
                                centroids=t(cents), norm_correction=True)
    torch.cuda.synchronize()
    got = cache.cpu().numpy()
    ref = ostore.store(key, value, slots, rot_t, cents, cache0.copy(), block_size=BS)
    changed = got.reshape(-1) != cache0.reshape(-1)
    assert np.array_equal(changed, ref.reshape(-1) != cache0.reshape(-1)), "only slot 17 is written"
    with pytest.raises(RuntimeError):
        ops.triton_turboquant_store(t(key).half(), t(value).half(), cache, t(slots), t(rot_t), t(mids),
                                    mse_bits=3, key_packed_size=66, value_quant_bits=4)


def test_reference_module_names(dev):
    """``tq4_decode.soa_store`` / ``tq4_decode.aos_store`` expose ``triton_turboquant_store``
    with the reference modules' signatures and write what ``ops.store`` writes."""
    from tq4_decode import aos_store, soa_store

    key, value, slots, rot_t, cents, mids = make_inputs(17, 64, 8, "bf16")
    t = lambda a: to_dev(a, dev)  # noqa: E731
    k, v = t(key).bfloat16(), t(value).bfloat16()
    for mod, layout, nc in ((soa_store, "soa", True), (aos_store, "aos", False)):
        a = torch.zeros(8, BS, HK, 134, dtype=torch.uint8, device=dev)
        b = torch.zeros_like(a)
        kwargs = dict(centroids=t(cents), norm_correction=nc) if layout == "soa" else {}
        mod.triton_turboquant_store(k, v, a, t(slots), t(rot_t), t(mids), mse_bits=4,
                                    key_packed_size=66, value_quant_bits=4, **kwargs)
        ops.store(k, v, b, t(slots), t(rot_t), t(mids), t(cents), layout=layout, norm_correction=nc)
        torch.cuda.synchronize()
        assert torch.equal(a, b), layout
        ref = ostore.store(key, value, slots, rot_t, cents, np.zeros((8, BS, HK, 134), np.uint8),
                           block_size=BS, is_aos=layout == "aos")
        keep = np.nonzero(slots >= 0)[0]
        gather = OL.gather_aos if layout == "aos" else OL.gather_soa
        for h in range(HK):
            gv = gather(a.cpu().numpy(), slots[keep] // BS, slots[keep] % BS, h, BS, HK, D)[2]
            rv = gather(ref, slots[keep] // BS, slots[keep] % BS, h, BS, HK, D)[2]
            assert np.array_equal(gv, rv)


def _hadamard(d):
    h = np.ones((1, 1))
    while h.shape[0] < d:
        h = np.block([[h, h], [h, -h]])
    return (h / np.sqrt(d)).astype(np.float32)


@pytest.mark.parametrize("rotation", ["hadamard", "orthogonal"])
@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_store_then_decode_against_unquantized_attention(dev, layout, rotation):
    """The reference's store -> decode check (validation/store_decode.py:90-230): B64 x ctx
    4096, N(0, 1) fp16 keys, values and queries, the Sylvester-Hadamard rotation
    (:45-51) as PiT for both the writer and the query, the writer's cache decoded by the full
    step (rotation, Stage1 over 32 splits, Stage2), and sequence 0 compared with attention
    computed in float64 from the unquantized K / V (:54-67).  The reference publishes the 4-bit
    quantization error of that comparison, output max / mean 0.0187 / 0.0028 and LSE 0.0065 /
    0.0025 (README.md:254-257); the bounds here are twice those, which a norm folded the wrong
    way exceeds.  A seeded random orthogonal rotation as well: it is not symmetric, so the
    writer and the query rotation must agree on its orientation."""
    B, ctx, S, HQ = 64, 4096, 32, 32
    rot = _hadamard(D) if rotation == "hadamard" else workloads.random_orthogonal(np.random.default_rng(9), D)
    cents = codebook.centroids(D, 4)
    mids = ((cents[:-1] + cents[1:]) * np.float32(0.5)).astype(np.float32)
    gen = torch.Generator(device=dev).manual_seed(20260814)
    key = torch.randn(B * ctx, HK, D, generator=gen, device=dev, dtype=torch.float32).half()
    value = torch.randn(B * ctx, HK, D, generator=gen, device=dev, dtype=torch.float32).half()
    query = torch.randn(B, HQ, D, generator=gen, device=dev, dtype=torch.float32).half()
    cache = torch.zeros(B * ctx // BS, BS, HK, 134, dtype=torch.uint8, device=dev)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    ops.store(key, value, cache, torch.arange(B * ctx, dtype=torch.int32, device=dev), t(rot), t(mids),
              t(cents), layout=layout, norm_correction=layout == "soa")
    bt = torch.arange(B * ctx // BS, dtype=torch.int32, device=dev).reshape(B, ctx // BS)
    sl = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    out, lse = ops.full_decode(query, t(rot), cache, bt, sl, t(cents), S, layout=layout,
                               out_dtype=torch.float32)
    torch.cuda.synchronize()
    q0 = query[0].double().cpu().numpy()
    k0 = key[:ctx].double().cpu().numpy()[:, np.arange(HQ) // (HQ // HK)]  # [t, h, d]
    v0 = value[:ctx].double().cpu().numpy()[:, np.arange(HQ) // (HQ // HK)]
    s = np.einsum("hd,thd->ht", q0, k0) / np.sqrt(D)
    m = s.max(axis=1, keepdims=True)
    p = np.exp(s - m)
    ref_lse = (m[:, 0] + np.log(p.sum(axis=1)))
    ref_out = np.einsum("ht,thd->hd", p / p.sum(axis=1, keepdims=True), v0)
    eo = np.abs(out[0].cpu().numpy() - ref_out)
    el = np.abs(lse[0].cpu().numpy() - ref_lse)
    print(f"{layout} {rotation} quantization error vs fp32 attention: output max/mean {eo.max():.4g} / {eo.mean():.4g}, "
          f"LSE max/mean {el.max():.4g} / {el.mean():.4g}")
    assert np.isfinite(out.cpu().numpy()).all() and np.isfinite(lse.cpu().numpy()).all()
    assert eo.max() <= 2 * 0.018739756 and eo.mean() <= 2 * 0.0028449418
    assert el.max() <= 2 * 0.0064659119 and el.mean() <= 2 * 0.0024851561


@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_store_without_norm_correction(dev, layout):
    """``norm_correction=False`` stores ``fp16(||k||)`` as the K scalar (``reference/soa_store.py``
    without NORM_CORRECTION) and changes nothing else: the same inputs written with and without
    it differ only in the K scalars, which then match ||k|| within one fp16 ulp."""
    n_tok, n_blocks = 300, 24
    key, value, slots, rot_t, cents, mids = make_inputs(17, n_tok, n_blocks, "bf16")
    cache0 = np.zeros((n_blocks, BS, HK, 134), dtype=np.uint8)
    with_nc = gpu_store(dev, key, value, slots, rot_t, cents, mids, cache0, "bf16", layout, True)
    raw = gpu_store(dev, key, value, slots, rot_t, cents, mids, cache0, "bf16", layout, False)
    keep = np.nonzero(slots >= 0)[0]
    blocks, offs = slots[keep] // BS, slots[keep] % BS
    gather = OL.gather_aos if layout == "aos" else OL.gather_soa
    norm = np.sqrt((key[keep].astype(np.float64) ** 2).sum(-1))
    for h in range(HK):
        ak, an, av, as_, az = gather(with_nc, blocks, offs, h, BS, HK, D)
        bk, bn, bv, bs_, bz = gather(raw, blocks, offs, h, BS, HK, D)
        assert np.array_equal(ak, bk) and np.array_equal(av, bv)
        assert np.array_equal(as_, bs_) and np.array_equal(az, bz)
    scal = np.zeros(cache0.size, dtype=bool)
    stride = BS * HK * 134
    for blk, off in zip(blocks.astype(np.int64), offs.astype(np.int64)):
        for h in range(HK):
            b0 = (blk * stride + (off * HK + h) * 134 + 64 if layout == "aos"
                  else blk * stride + BS * HK * 128 + (h * 3 * BS + off) * 2)
            scal[b0:b0 + 2] = True
    assert np.array_equal(with_nc.reshape(-1)[~scal], raw.reshape(-1)[~scal]), "bytes other than the K scalar differ"
    stored = raw.reshape(-1)[scal].view(np.float16).astype(np.float64)
    want = []
    for i, (blk, off) in enumerate(zip(blocks.astype(np.int64), offs.astype(np.int64))):
        for h in range(HK):
            b0 = (blk * stride + (off * HK + h) * 134 + 64 if layout == "aos"
                  else blk * stride + BS * HK * 128 + (h * 3 * BS + off) * 2)
            want.append((b0, norm[i, h]))
    want = np.array([v for _, v in sorted(want)])  # in byte order, as `stored`
    assert np.all(np.abs(stored - want) <= np.abs(want) * 2.0 ** -10), "K scalar is not fp16(||k||)"
