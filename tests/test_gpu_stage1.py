"""Stage1 parity on the GPU: HIP kernels (through the C ABI) vs the oracle.

Bar: max-abs <= 1e-4 on mid_o (outputs and LSE, fp32), identical untouched-split
pattern (mid_o is pre-filled with NaN; empty splits must stay NaN).
"""
import numpy as np
import pytest
import torch

from conftest import to_dev
from oracle import native
from tq4_decode import ops, workloads

pytestmark = pytest.mark.gpu
TOL = 1e-4


def run(w, dev, kernel, layout="soa", cache=None):
    cache = w.kv_cache if cache is None else cache
    mid = torch.full((w.batch, w.num_q_heads, w.num_kv_splits, 129), float("nan"), device=dev)
    ops.stage1(to_dev(w.q_rot, dev), to_dev(cache, dev), to_dev(w.block_table, dev),
               to_dev(w.seq_lens, dev), to_dev(w.pair_lut, dev), mid, layout=layout, kernel=kernel)
    torch.cuda.synchronize()
    return mid.cpu().numpy()


def oracle(w, layout="soa", cache=None):
    cache = w.kv_cache if cache is None else cache
    return native.stage1(w.q_rot, cache, w.block_table, w.seq_lens, w.centroids, w.num_kv_splits,
                         num_kv_heads=w.num_kv_heads, block_size=w.block_size,
                         is_aos=layout == "aos")


def assert_parity(got, ref, tol=TOL):
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "untouched-split pattern differs"
    err = np.nanmax(np.abs(got - ref))
    print(f"max-abs {err:.3e}")
    assert err <= tol, f"max-abs {err} > {tol}"


@pytest.mark.parametrize("kernel", ["simple", "xdl"])
@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_store_fixture_b2_ctx256(config1, dev, kernel, layout):
    f = config1
    w = workloads.Workload("config1", f["q_rot"], f[f"cache_{layout}"], f["block_table"],
                           f["seq_lens"], f["centroids"], int(f["num_kv_splits"]),
                           int(f["num_kv_heads"]))
    got = run(w, dev, kernel, layout)
    # the matrix-core kernel holds fp32-grade accuracy on store-written data (f16 hi + lo
    # parts, V codes at the top of the f16 significand): 5e-6, inside the 1e-4 bar
    assert_parity(got, f[f"mid_{layout}"], 5e-6 if kernel == "xdl" else TOL)


@pytest.mark.parametrize("kernel", ["simple", "xdl"])
@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_ragged_with_empty_and_partial_splits(dev, kernel, layout):
    w = workloads.small(101, 6, [1, 3, 17, 100, 257, 999], 32)
    cache = workloads.soa_to_aos(w.kv_cache, w.centroids, 8) if layout == "aos" else None
    assert_parity(run(w, dev, kernel, layout, cache), oracle(w, layout, cache))


@pytest.mark.parametrize("kernel,group", [("simple", 1), ("simple", 2), ("simple", 4), ("simple", 6),
                                          ("simple", 8), ("simple", 16), ("xdl", 1), ("xdl", 2),
                                          ("xdl", 3), ("xdl", 4), ("xdl", 5), ("xdl", 6), ("xdl", 8),
                                          ("xdl", 12), ("xdl", 16), ("xdl", 32)])
def test_gqa_groups(dev, kernel, group):
    """The matrix-core kernel serves a group in waves of 4 (groups up to 4) or 8 q-heads:
    1, 2, 3, 5 and 6 leave padding heads in their wave, 12 and 16 take two waves per
    kv-head, 32 four."""
    hk = 4
    w = workloads.small(102, 3, [77, 300, 1024], 7, num_q_heads=hk * group, num_kv_heads=hk)
    assert_parity(run(w, dev, kernel), oracle(w))


@pytest.mark.parametrize("layout", ["soa", "aos"])
@pytest.mark.parametrize("group", [6, 16])
def test_gqa_6_and_16_on_the_mfma_kernel(dev, layout, group):
    """GQA 6 and 16 (the backend's gfx950 groups besides 8) at 8 kv-heads: many splits per
    wave, an empty and a one-token sequence; auto runs the 16x16x32 kernel."""
    hk = 8
    w = workloads.small(103 + group, 5, [4096, 0, 1, 333, 2049], 32, num_q_heads=hk * group,
                        num_kv_heads=hk)
    cache = workloads.soa_to_aos(w.kv_cache, w.centroids, hk) if layout == "aos" else None
    ref = oracle(w, layout, cache)
    xdl = run(w, dev, "xdl", layout, cache)
    assert_parity(xdl, ref, 1e-5)  # fp32-grade on this data, inside the 1e-4 bar
    assert np.array_equal(run(w, dev, "auto", layout, cache), xdl, equal_nan=True)
    assert_parity(run(w, dev, "simple", layout, cache), ref)


@pytest.mark.parametrize("kernel", ["simple", "xdl"])
@pytest.mark.parametrize("bs", [32, 64, 128, 256])
def test_larger_kv_blocks(dev, kernel, bs):
    w = workloads.small(103, 3, [130, 511, 64], 5, block_size=bs)
    for layout in ("soa", "aos"):
        cache = workloads.soa_to_aos(w.kv_cache, w.centroids, 8, block_size=bs) if layout == "aos" else None
        assert_parity(run(w, dev, kernel, layout, cache), oracle(w, layout, cache))


@pytest.mark.parametrize("bs", [8, 48])
def test_block_sizes_the_mfma_kernel_does_not_take(dev, bs):
    """Block sizes below 16 or not a power of two: "auto" runs the VALU kernel, and asking for
    the 16x16x32 kernel is an error, not a wrong result."""
    w = workloads.small(104, 4, [700, 33, 0, 2000], 8, block_size=bs)
    for layout in ("soa", "aos"):
        cache = workloads.soa_to_aos(w.kv_cache, w.centroids, 8, block_size=bs) if layout == "aos" else None
        assert_parity(run(w, dev, "auto", layout, cache), oracle(w, layout, cache))
        with pytest.raises(RuntimeError, match="power-of-two block_size"):
            run(w, dev, "xdl", layout, cache)


@pytest.mark.parametrize("kernel", ["simple", "xdl"])
@pytest.mark.parametrize("mb,lens", [(4, [1, 60, 33]), (12, [190, 7, 160]), (13, [200, 150, 9]),
                                     (252, [4032, 1000, 2500]), (256, [4096, 17, 3000]),
                                     (260, [4100, 4000, 1])])
def test_block_table_row_widths(dev, kernel, mb, lens):
    """Block-table rows wider than a sequence needs: the entries past its need hold other
    valid block indices, so a kernel that reads a wrong entry changes the result."""
    w = workloads.small(105, 3, lens, 8)
    need = w.block_table.shape[1]
    assert need <= mb
    nb = w.kv_cache.shape[0]
    bt = ((np.arange(3)[:, None] * 7 + np.arange(mb)[None, :] * 3 + 1) % nb).astype(np.int32)
    for b, n in enumerate((w.seq_lens + 15) // 16):
        bt[b, :n] = w.block_table[b, :n]
    w.block_table = bt
    assert_parity(run(w, dev, kernel), oracle(w))


def test_large_scores_rescale_path(dev):
    """q scaled x40: scores span tens of units, so the running max moves often."""
    w = workloads.small(104, 2, [640, 333], 3)
    w.q_rot = (w.q_rot * 40).astype(np.float32)
    assert_parity(run(w, dev, "xdl"), oracle(w))
    assert_parity(run(w, dev, "simple"), oracle(w))


@pytest.mark.parametrize("layout", ["soa", "aos"])
@pytest.mark.parametrize("group", [4, 8])
def test_query_rows_beyond_the_f16_range(dev, layout, group):
    """q rows whose |q * attn_scale * log2 e| reaches 1e5 - 5e5 (past the f16 range of the
    matrix-core operands; they are scaled by a power of two first) next to rows just inside
    it and ordinary rows.  Scores that large make a (split, head) row ill-conditioned when
    its top two tokens lie within a few units: a relative rounding of 2^-22 of the scores
    then moves the output by more than 1e-4 in any fp32 kernel.  So the float64 oracle is
    run twice, the second time with q scaled by 1 + 2^-20, and the rows that move by less
    than 1e-5 (at least 90 % of them) are held to 1e-4 on the outputs and 1e-4 + 2^-20
    relative on the LSE; every row must be finite."""
    from oracle import stage1 as ostage

    hk = 4
    w = workloads.small(109 + group, 3, [700, 64, 1500], 4, num_q_heads=hk * group, num_kv_heads=hk)
    cache = workloads.soa_to_aos(w.kv_cache, w.centroids, hk) if layout == "aos" else w.kv_cache
    q = w.q_rot.copy()
    q[0, 1] *= 2e5
    q[1, :] *= 3e4
    q[2, group] *= 1e6
    w.q_rot = q
    got = run(w, dev, "xdl", layout, None if layout == "soa" else cache)

    def f64(qq):
        return ostage.stage1(qq, cache, w.block_table, w.seq_lens, w.centroids, 4, num_kv_heads=hk,
                             is_aos=layout == "aos")

    ref = f64(q)
    nudged = f64(q.astype(np.float64) * (1 + 2.0 ** -20))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    live = ~np.isnan(ref[..., 0])
    assert np.isfinite(got[live]).all()
    well = live & (np.abs(nudged[..., :128] - ref[..., :128]).max(-1) < 1e-5)
    assert well.sum() >= 0.9 * live.sum()
    err_o = np.abs(got[..., :128] - ref[..., :128])[well].max()
    lse_g, lse_r = got[..., 128][well], ref[..., 128][well]
    print(f"{well.sum()} of {live.sum()} rows well-conditioned; outputs max-abs {err_o:.3e}, "
          f"LSE up to {np.abs(lse_r).max():.3e}")
    assert err_o <= 1e-4
    assert np.all(np.abs(lse_g - lse_r) <= 1e-4 + 2.0 ** -20 * np.abs(lse_r))


@pytest.fixture(scope="module")
def qwen():
    w = workloads.qwen3_4b_b64_ctx4096()
    return w, workloads.soa_to_aos(w.kv_cache, w.centroids, 8)


@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_qwen3_4b_b64_ctx4096_full_size(qwen, dev, layout):
    w, aos = qwen
    cache = aos if layout == "aos" else None
    ref = oracle(w, layout, cache)
    assert_parity(run(w, dev, "auto", layout, cache), ref)


@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_xdl_qwen3_4b_b64_ctx4096_full_size(qwen, dev, layout):
    w, aos = qwen
    cache = aos if layout == "aos" else None
    assert_parity(run(w, dev, "xdl", layout, cache), oracle(w, layout, cache))


@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_xdl_on_store_written_cache_full_size(dev, layout):
    """B64 x ctx 4096 over a cache the GPU writer filled from N(0, 1) keys and values (V
    scales ~0.4 and zero points ~-3, the realistic case for the f16 hi + lo softmax weights,
    unlike the synthetic caches' 0.01-0.1 scales)."""
    from tq4_decode import codebook

    rng = np.random.default_rng(131)
    B, ctx, nb = 64, 4096, 64 * 256
    bt = rng.permutation(nb).astype(np.int32).reshape(B, ctx // 16)
    pos = np.arange(ctx)
    slots = (bt[:, pos // 16] * 16 + pos % 16).reshape(-1).astype(np.int32)
    gen = torch.Generator(device=dev).manual_seed(132)
    key = torch.randn(B * ctx, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
    value = torch.randn(B * ctx, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
    cents = codebook.centroids(128, 4)
    mids = ((cents[:-1] + cents[1:]) * np.float32(0.5)).astype(np.float32)
    rot = workloads.random_orthogonal(rng, 128)
    cache = torch.zeros(nb, 16, 8, 134, dtype=torch.uint8, device=dev)
    ops.store(key, value, cache, to_dev(slots, dev), to_dev(rot, dev), to_dev(mids, dev),
              to_dev(cents, dev), layout=layout, norm_correction=layout == "soa")
    del key, value
    q_rot = rng.standard_normal((B, 32, 128)).astype(np.float32)
    w = workloads.Workload("store_written", q_rot, cache.cpu().numpy(), bt, np.full(B, ctx, np.int32),
                           cents, 32, 8)
    got = run(w, dev, "xdl", layout)
    ref = oracle(w, layout)
    assert_parity(got, ref, 1e-5)


@pytest.mark.parametrize("layout", ["soa", "aos"])
@pytest.mark.parametrize("group", [4, 8])
def test_wave_deal_over_several_lane_chunks(dev, layout, group):
    # 150 sequences (three 64-lane chunks of the kernel's wave deal), about a third empty,
    # lengths 1 .. 700: every live split is written once, every dead one stays NaN
    rng = np.random.default_rng(109)
    lens = rng.integers(1, 700, size=150)
    lens[rng.random(150) < 0.33] = 0
    hk = 2 if group == 8 else 4
    w = workloads.small(109, 150, lens, 32, num_q_heads=hk * group, num_kv_heads=hk)
    cache = workloads.soa_to_aos(w.kv_cache, w.centroids, hk) if layout == "aos" else None
    assert_parity(run(w, dev, "xdl", layout, cache), oracle(w, layout, cache))


def test_runs_of_more_than_64_splits(dev):
    # 72 sequences x 8 kv-heads x 2 parts (GQA-16) = 1152 (sequence, part) pairs: one wave
    # each, so a sequence's wave runs all its live splits -- up to 80 here, past the 64 a
    # wave keeps in its lanes -- next to sequences of fewer splits and an empty one
    rng = np.random.default_rng(111)
    lens = np.concatenate([rng.integers(65, 81, size=24), rng.integers(200, 241, size=24),
                           rng.integers(1, 60, size=23), [0]])
    w = workloads.small(111, 72, lens, 80, num_q_heads=8 * 16, num_kv_heads=8)
    assert_parity(run(w, dev, "xdl"), oracle(w))


def test_wave_deal_gives_a_lone_long_sequence_many_waves(dev):
    # two live sequences out of 64: the deal hands the long one up to one wave per split
    lens = [0] * 64
    lens[5], lens[40] = 4096, 33
    w = workloads.small(110, 64, lens, 32)
    assert_parity(run(w, dev, "xdl"), oracle(w))


@pytest.mark.parametrize("lens", [[1024] * 32, [1000] * 32])
def test_equal_lengths_one_full_round(dev, lens):
    # 8 kv-heads x 32 sequences x 8 waves = 2048 workgroups, one round of the device at two
    # waves per SIMD, each wave a run of 8 of the 64 splits (1000 tokens: splits of 16 tokens,
    # the last one short); every split written exactly once
    w = workloads.small(111, 32, lens, 64)
    assert_parity(run(w, dev, "xdl"), oracle(w))


def test_xdl_ragged_and_gqa8_full_size(dev):
    for w in (workloads.ragged_b64(), workloads.gqa8_b8_ctx32768()):
        assert_parity(run(w, dev, "xdl"), oracle(w))


def test_xdl_and_simple_agree_full_size(qwen, dev):
    w, _ = qwen
    a, b = run(w, dev, "xdl"), run(w, dev, "simple")
    assert_parity(a, b, 1e-5)


def test_ragged_b64_full_size(dev):
    w = workloads.ragged_b64()
    assert_parity(run(w, dev, "auto"), oracle(w))


def test_gqa8_b8_ctx32768_full_size(dev):
    w = workloads.gqa8_b8_ctx32768()
    assert_parity(run(w, dev, "auto"), oracle(w))


def test_reference_call_shapes(qwen, dev):
    w, aos = qwen
    t = lambda a: to_dev(a, dev)  # noqa: E731
    q, bt, sl, cents = t(w.q_rot), t(w.block_table), t(w.seq_lens), t(w.centroids)
    soa_c, aos_c = t(w.kv_cache), t(aos)
    lut = ops.pair_lut_device(cents)
    assert torch.equal(lut.cpu(), torch.from_numpy(w.pair_lut))
    mid_v2 = ops.launch_tq4_v2_stage1(q, soa_c, bt, sl, cents, lut)  # allocates mid_o
    mid_ext = torch.empty_like(mid_v2)
    ops.ext.tq4_cuda_v9(q, soa_c, bt, sl, cents, mid_ext)
    mid_aos = torch.empty_like(mid_v2)
    ops.launch_aos_v1_stage1(q, aos_c, bt, sl, cents, mid_aos)
    torch.cuda.synchronize()
    ref = oracle(w)
    assert_parity(mid_v2.cpu().numpy(), ref)
    assert torch.equal(mid_v2, mid_ext)
    assert_parity(mid_aos.cpu().numpy(), oracle(w, "aos", aos))


@pytest.mark.parametrize("kernel", ["xdl", "simple"])
@pytest.mark.parametrize("layout", ["soa", "aos"])
@pytest.mark.parametrize("group", [4, 6, 8, 16])
def test_sinks(dev, kernel, layout, group):
    """Per-head sink logits enter split 0's softmax (max = sink, sum = 1)."""
    hk = 4
    w = workloads.small(106, 4, [1, 300, 2049, 77], 8, num_q_heads=hk * group, num_kv_heads=hk)
    cache = workloads.soa_to_aos(w.kv_cache, w.centroids, hk) if layout == "aos" else w.kv_cache
    rng = np.random.default_rng(107)
    sinks = rng.normal(0.0, 3.0, hk * group).astype(np.float32)
    sinks[1] = -np.inf
    sinks[2] = 40.0
    mid = torch.full((w.batch, w.num_q_heads, 8, 129), float("nan"), device=dev)
    ops.stage1(to_dev(w.q_rot, dev), to_dev(cache, dev), to_dev(w.block_table, dev),
               to_dev(w.seq_lens, dev), to_dev(w.pair_lut, dev), mid, layout=layout, kernel=kernel,
               sinks=to_dev(sinks, dev))
    torch.cuda.synchronize()
    ref = native_free_oracle(w, cache, layout, sinks)
    assert_parity(mid.cpu().numpy(), ref)


def native_free_oracle(w, cache, layout, sinks):
    from oracle import stage1 as ostage

    return ostage.stage1(w.q_rot, cache, w.block_table, w.seq_lens, w.centroids, w.num_kv_splits,
                         num_kv_heads=w.num_kv_heads, is_aos=layout == "aos", sinks=sinks)


def test_retired_kernel_id_is_rejected(dev):
    """TQ4_KERNEL_MFMA (2), the retired 4x4x4 kernel, returns TQ4_E_UNSUPPORTED and leaves
    mid_o untouched."""
    from tq4_decode import _lib

    w = workloads.small(108, 1, [64], 2)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    q, c, bt, sl, lut = t(w.q_rot), t(w.kv_cache), t(w.block_table), t(w.seq_lens), t(w.pair_lut)
    mid = torch.full((1, 32, 2, 129), float("nan"), device=dev)
    lib = _lib.load()
    rc = lib.tq4_stage1_ex(q.data_ptr(), c.data_ptr(), bt.data_ptr(), sl.data_ptr(), lut.data_ptr(),
                           mid.data_ptr(), 1, 32, 8, 128, 16, bt.size(1), c.stride(0), 2, 0,
                           128 ** -0.5, 2, None, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 2 and b"retired" in lib.tq4_last_error()
    assert torch.isnan(mid).all()


@pytest.mark.parametrize("kernel", ["xdl", "simple"])
@pytest.mark.parametrize("layout", ["soa", "aos"])
@pytest.mark.parametrize("scale", [0.01, 0.3, 2.0])
def test_attention_scales(dev, kernel, layout, scale):
    """Scores scale with attn_scale (the default is 1 / sqrt(D)); at 2.0 the scores reach tens of
    units, so the max rescale path runs too."""
    w = workloads.small(120, 4, [700, 33, 1500, 129], 8)
    cache = workloads.soa_to_aos(w.kv_cache, w.centroids, 8) if layout == "aos" else w.kv_cache
    mid = torch.full((w.batch, w.num_q_heads, w.num_kv_splits, 129), float("nan"), device=dev)
    ops.stage1(to_dev(w.q_rot, dev), to_dev(cache, dev), to_dev(w.block_table, dev), to_dev(w.seq_lens, dev),
               to_dev(w.pair_lut, dev), mid, layout=layout, kernel=kernel, attn_scale=scale)
    torch.cuda.synchronize()
    ref = native.stage1(w.q_rot, cache, w.block_table, w.seq_lens, w.centroids, w.num_kv_splits,
                        num_kv_heads=8, block_size=16, is_aos=layout == "aos", attn_scale=scale)
    assert_parity(mid.cpu().numpy(), ref)
