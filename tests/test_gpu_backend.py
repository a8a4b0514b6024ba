"""The vLLM backend's call path on the GPU.

* The cache view the backend passes: it allocates its cache ``[blocks, Hk, block_size,
  slot]`` and hands decode and store ``kv_cache.transpose(1, 2)``
  (``reference/turboquant_attn.py:536``, ``:565``), a non-contiguous view with strides
  ``(bs*Hk*slot, slot, bs*slot, 1)``.  The entries must give the same bytes / results as
  for the contiguous cache holding the same slots, and match the oracle.
* Graph capture and replay of the decode entry: the launches depend on shapes only, so a
  captured call replays correctly after ``seq_lens`` and ``block_table`` change in place
  (``reference/turboquant_attn.py:368-373``).
* Cache bytes past ``seq_len`` (unwritten slots of a sequence's last block) holding
  non-finite fp16 patterns must not reach the result.

Bars: mid_o max-abs 1e-4 (fp32); fp16 outputs 1e-4 + fp16 rounding (2^-11 relative);
identical results for the view and the contiguous cache.
"""
import numpy as np
import pytest
import torch

from conftest import to_dev
from oracle import native
from oracle import stage1 as ostage
from oracle import store as ostore
from tq4_decode import aos_decode, aos_store, codebook, ops, soa_decode, soa_store, workloads

pytestmark = pytest.mark.gpu
D, HK, BS = 128, 8, 16
SCALE = 128 ** -0.5


def head_major(pm: torch.Tensor, layout: str):
    """The backend's storage ``[blocks, Hk, bs, slot]`` holding the cache ``pm`` (contiguous
    ``[blocks, bs, Hk, slot]``) and its ``transpose(1, 2)`` view: for AoS the view's slot
    (t, h) equals pm's; an SoA block keeps its bytes (its inner layout is the kernels')."""
    nb, bs, hk, slot = pm.shape
    if layout == "aos":
        storage = pm.permute(0, 2, 1, 3).contiguous()
    else:
        storage = pm.reshape(-1).clone().view(nb, hk, bs, slot)
    view = storage.transpose(1, 2)
    assert not view.is_contiguous()
    assert view.stride() == (bs * hk * slot, slot, bs * slot, 1)
    return storage, view


def _mid(dev, w, S):
    return torch.full((w.batch, w.num_q_heads, S, D + 1), float("nan"), device=dev)


def _assert_mid(got, ref, tol=1e-4):
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "untouched-split pattern differs"
    err = np.nanmax(np.abs(got - ref))
    print(f"max-abs {err:.3e}")
    assert err <= tol


@pytest.mark.parametrize("kernel", ["xdl", "simple"])
@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_stage1_takes_the_transposed_view(dev, layout, kernel):
    w = workloads.small(601, 5, [1500, 1, 333, 4096, 64], 32)
    cache = workloads.soa_to_aos(w.kv_cache, w.centroids, HK) if layout == "aos" else w.kv_cache
    t = lambda a: to_dev(a, dev)  # noqa: E731
    pm = t(cache)
    _, view = head_major(pm, layout)
    args = (t(w.q_rot), t(w.block_table), t(w.seq_lens), t(w.pair_lut))
    a, b = _mid(dev, w, 32), _mid(dev, w, 32)
    ops.stage1(args[0], pm, *args[1:], a, layout=layout, kernel=kernel)
    ops.stage1(args[0], view, *args[1:], b, layout=layout, kernel=kernel)
    torch.cuda.synchronize()
    assert torch.equal(a.nan_to_num(7.0), b.nan_to_num(7.0)), "view and contiguous cache differ"
    ref = native.stage1(w.q_rot, cache, w.block_table, w.seq_lens, w.centroids, 32, num_kv_heads=HK,
                        is_aos=layout == "aos")
    _assert_mid(b.cpu().numpy(), ref)


@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_decode_entry_takes_the_backends_cache_view(dev, layout):
    """``{soa,aos}_decode.triton_turboquant_decode_attention`` called exactly as the backend
    calls it: the transposed view, Pi and PiT, fp16 query."""
    rng = np.random.default_rng(602)
    w = workloads.small(602, 5, [1500, 1, 333, 4096, 64], 32)
    cache = workloads.soa_to_aos(w.kv_cache, w.centroids, HK) if layout == "aos" else w.kv_cache
    query = rng.standard_normal((5, 32, D)).astype(np.float16)
    rot_t = workloads.random_orthogonal(rng, D)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    pm = t(cache)
    _, view = head_major(pm, layout)
    mod = aos_decode if layout == "aos" else soa_decode
    Pi, PiT = t(rot_t.T.copy()), t(rot_t)

    def call(c):
        return mod.triton_turboquant_decode_attention(
            t(query), c, t(w.block_table), t(w.seq_lens), Pi, t(w.centroids), SCALE, mse_bits=4,
            key_packed_size=66, value_quant_bits=4, norm_correction=True, PiT=PiT,
            max_num_kv_splits=32).clone()

    a, b = call(pm), call(view)
    torch.cuda.synchronize()
    assert torch.equal(a, b), "view and contiguous cache differ"
    q_rot = (query.astype(np.float64) @ rot_t.astype(np.float64)).astype(np.float32)
    mid = native.stage1(q_rot, cache, w.block_table, w.seq_lens, w.centroids, 32, num_kv_heads=HK,
                        is_aos=layout == "aos")
    ro, _ = native.stage2(mid, w.seq_lens)
    diff = np.abs(b.float().cpu().numpy() - ro)
    print(f"{layout} decode entry (transposed view) fp16 max-abs {diff.max():.3e}")
    assert np.all(diff <= 1e-4 + 2.0 ** -11 * np.abs(ro))


def _store_inputs(dev, seed, n_tok, n_blocks):
    rng = np.random.default_rng(seed)
    key = torch.from_numpy(rng.standard_normal((n_tok, HK, D)).astype(np.float32)).to(dev)
    value = torch.from_numpy(rng.standard_normal((n_tok, HK, D)).astype(np.float32)).to(dev)
    slots = rng.permutation(n_blocks * BS)[:n_tok].astype(np.int32)
    slots[[3, 50]] = -1  # skipped tokens
    return rng, key.to(torch.bfloat16), value.to(torch.bfloat16), to_dev(slots, dev)


@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_store_entry_takes_the_backends_cache_view(dev, layout):
    """``{soa,aos}_store.triton_turboquant_store`` into the transposed view writes what it
    writes into the contiguous cache (same bytes per slot), and decoding that cache through
    the view matches the oracle."""
    n_tok, n_blocks = 400, 30
    rng, key, value, slots = _store_inputs(dev, 603, n_tok, n_blocks)
    cents = codebook.centroids(D, 4)
    mids = ((cents[:-1] + cents[1:]) * np.float32(0.5)).astype(np.float32)
    rot_t = workloads.random_orthogonal(rng, D)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    pm = torch.zeros(n_blocks, BS, HK, 134, dtype=torch.uint8, device=dev)
    storage, view = head_major(torch.zeros_like(pm), layout)
    for c in (pm, view):
        if layout == "aos":
            aos_store.triton_turboquant_store(key, value, c, slots, t(rot_t), t(mids), 4, 66, 4)
        else:
            soa_store.triton_turboquant_store(key, value, c, slots, t(rot_t), t(mids), 4, 66, 4,
                                              centroids=t(cents), norm_correction=True)
    torch.cuda.synchronize()
    if layout == "aos":
        assert torch.equal(view, pm)
    else:
        assert torch.equal(storage.reshape(-1), pm.reshape(-1))
    # V bytes of every written slot equal the oracle writer's (bit-exact)
    ref = np.zeros(tuple(pm.shape), np.uint8)
    ostore.store(key.float().cpu().numpy(), value.float().cpu().numpy(), slots.cpu().numpy(), rot_t,
                 cents, ref, is_aos=layout == "aos")
    got = pm.cpu().numpy()
    if layout == "aos":
        assert np.array_equal(got[..., 66:], ref[..., 66:])
    else:
        data = lambda a: a.reshape(n_blocks, -1)[:, :BS * HK * D].reshape(n_blocks, BS, HK, D)  # noqa: E731
        assert np.array_equal(data(got)[..., 64:], data(ref)[..., 64:])
    # decode through the view: 4 sequences over the written slots
    used = np.sort(slots.cpu().numpy()[slots.cpu().numpy() >= 0])
    blocks = np.unique(used // BS)
    lens = np.array([128, 77, 16 * 6, 1], np.int32)
    bt = np.stack([rng.permutation(blocks)[:8] for _ in range(4)]).astype(np.int32)
    q_rot = rng.standard_normal((4, 32, D)).astype(np.float32)
    mid = torch.full((4, 32, 4, D + 1), float("nan"), device=dev)
    lut = ops.pair_lut_device(t(cents))
    ops.stage1(t(q_rot), view, t(bt), t(lens), lut, mid, layout=layout)
    torch.cuda.synchronize()
    want = native.stage1(q_rot, got, bt, lens, cents, 4, num_kv_heads=HK, is_aos=layout == "aos")
    _assert_mid(mid.cpu().numpy(), want)


@pytest.mark.parametrize("preset", ["fp8", (3, 4), (3, 3)])
@pytest.mark.parametrize("kernel", ["xdl", "simple"])
def test_presets_take_the_head_major_aos_view(dev, preset, kernel):
    """The other presets' writers and Stage1 (AoS slots at the head-major strides)."""
    n_tok, n_blocks = 300, 24
    rng, key, value, slots = _store_inputs(dev, 604, n_tok, n_blocks)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    if preset == "fp8":
        slot = ops.slot_bytes_fp8(D)
    else:
        slot = ops.slot_bytes_preset(D, *preset)
        cents = codebook.centroids(D, preset[0])
        mids = ((cents[:-1] + cents[1:]) * np.float32(0.5)).astype(np.float32)
        rot_t = workloads.random_orthogonal(rng, D)
    pm = torch.zeros(n_blocks, BS, HK, slot, dtype=torch.uint8, device=dev)
    _, view = head_major(torch.zeros_like(pm), "aos")
    for c in (pm, view):
        if preset == "fp8":
            ops.store_fp8(key, value, c, slots, layout="aos")
        else:
            ops.store_preset(key, value, c, slots, t(rot_t), t(mids), t(cents), key_bits=preset[0],
                             value_bits=preset[1], layout="aos", norm_correction=False)
    torch.cuda.synchronize()
    assert torch.equal(view, pm)
    used = slots.cpu().numpy()
    blocks = np.unique(used[used >= 0] // BS)
    lens = np.array([100, 33, 128], np.int32)
    bt = np.stack([rng.permutation(blocks)[:8] for _ in range(3)]).astype(np.int32)
    q = t(rng.standard_normal((3, 32, D)).astype(np.float32))
    a = torch.full((3, 32, 4, D + 1), float("nan"), device=dev)
    b = torch.full_like(a, float("nan"))
    for c, m in ((pm, a), (view, b)):
        if preset == "fp8":
            ops.stage1_fp8(q, c, t(bt), t(lens), m, layout="aos", kernel=kernel)
        else:
            ops.stage1_preset(q, c, t(bt), t(lens), t(cents), m, key_bits=preset[0],
                              value_bits=preset[1], layout="aos", kernel=kernel)
    torch.cuda.synchronize()
    assert torch.equal(a.nan_to_num(7.0), b.nan_to_num(7.0))
    bits = None if preset == "fp8" else preset
    ref = ostage.stage1(q.cpu().numpy(), pm.cpu().numpy(), bt, lens,
                        None if preset == "fp8" else cents, 4, num_kv_heads=HK, is_aos=True,
                        key_fp8=preset == "fp8", **({} if bits is None else {"bits": bits}))
    _assert_mid(b.cpu().numpy(), ref)


class _Holder:
    pass


@pytest.mark.parametrize("batch", [4, 256])
def test_decode_entry_graph_capture_and_replay(dev, batch):
    """Capture the SoA decode entry once (buffers on the holder, warmed up first; no
    allocation or memset in the captured region), then change ``seq_lens`` and
    ``block_table`` in place and replay: every replay equals an eager call on the same
    inputs (bit for bit) and the oracle.  batch 4 runs Stage1 + Stage2; batch 256 gives one
    wave per (sequence, kv-head), the single-split path whose Stage1 writes the output."""
    rng = np.random.default_rng(610 + batch)
    S, mb = 16, 24
    nb = batch * mb + 5
    cache_np = workloads.synthetic_cache(rng, nb, HK)
    query = rng.standard_normal((batch, 32, D)).astype(np.float16)
    rot_t = workloads.random_orthogonal(rng, D)
    cents = codebook.centroids(D, 4)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    cache, q, PiT, Pi, c = t(cache_np), t(query), t(rot_t), t(rot_t.T.copy()), t(cents)
    bt = torch.zeros(batch, mb, dtype=torch.int32, device=dev)
    sl = torch.zeros(batch, dtype=torch.int32, device=dev)
    holder = _Holder()

    def fill():
        lens = rng.integers(1, mb * BS + 1, batch).astype(np.int32)
        lens[0] = mb * BS
        table = rng.permutation(nb)[:batch * mb].astype(np.int32).reshape(batch, mb)
        sl.copy_(t(lens))
        bt.copy_(t(table))
        return lens, table

    def entry():
        return soa_decode.triton_turboquant_decode_attention(
            q, cache, bt, sl, Pi, c, SCALE, mse_bits=4, key_packed_size=66, value_quant_bits=4,
            norm_correction=True, PiT=PiT, buf_holder=holder, max_num_kv_splits=S)

    fill()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            entry()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = entry()
    q_rot = (query.astype(np.float64) @ rot_t.astype(np.float64)).astype(np.float32)
    for rep in range(3):
        lens, table = fill()
        graph.replay()
        torch.cuda.synchronize()
        got = out.float().cpu().numpy().copy()
        eager = entry().float().cpu().numpy()  # eager work between the replays
        torch.cuda.synchronize()
        assert np.array_equal(got, eager), f"replay {rep} differs from the eager call"
        mid = native.stage1(q_rot, cache_np, table, lens, cents, S, num_kv_heads=HK)
        ro, _ = native.stage2(mid, lens)
        diff = np.abs(got - ro)
        print(f"B{batch} replay {rep} fp16 max-abs {diff.max():.3e}")
        assert np.all(diff <= 1e-4 + 2.0 ** -11 * np.abs(ro))


def _poison_past_seq_len(cache, w, layout):
    """Fill every slot past seq_len in each sequence's last block with non-finite fp16
    metadata (NaN norm, +inf scale, -inf zero) and 0xFF code bytes."""
    flat = cache.reshape(cache.shape[0], -1)
    moff = BS * HK * D
    nan, pinf, ninf = (np.array([v], np.uint16).view(np.uint8) for v in (0x7E00, 0x7C00, 0xFC00))
    for b, n in enumerate(w.seq_lens):
        if n % BS == 0:
            continue
        blk = w.block_table[b, (n - 1) // BS]
        for tok in range(n % BS, BS):
            for h in range(HK):
                if layout == "aos":
                    s = (tok * HK + h) * 134
                    flat[blk, s:s + 134] = 0xFF
                    flat[blk, s + 64:s + 66] = nan
                    flat[blk, s + 130:s + 132] = pinf
                    flat[blk, s + 132:s + 134] = ninf
                else:
                    r = (tok * HK + h) * D
                    flat[blk, r:r + D] = 0xFF
                    for f, v in enumerate((nan, pinf, ninf)):
                        m = moff + ((h * 3 + f) * BS + tok) * 2
                        flat[blk, m:m + 2] = v
    return cache


@pytest.mark.parametrize("kernel", ["xdl", "simple"])
@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_non_finite_bytes_past_seq_len(dev, layout, kernel):
    w = workloads.small(620, 6, [37, 250, 1, 1000, 17, 95], 8)
    cache = workloads.soa_to_aos(w.kv_cache, w.centroids, HK) if layout == "aos" else w.kv_cache.copy()
    cache = _poison_past_seq_len(cache, w, layout)
    mid = _mid(dev, w, 8)
    ops.stage1(to_dev(w.q_rot, dev), to_dev(cache, dev), to_dev(w.block_table, dev),
               to_dev(w.seq_lens, dev), to_dev(w.pair_lut, dev), mid, layout=layout, kernel=kernel)
    torch.cuda.synchronize()
    ref = native.stage1(w.q_rot, cache, w.block_table, w.seq_lens, w.centroids, 8, num_kv_heads=HK,
                        is_aos=layout == "aos")
    got = mid.cpu().numpy()
    live = ~np.isnan(ref[..., 0])
    assert np.isfinite(ref[live]).all() and np.isfinite(got[live]).all()
    _assert_mid(got, ref)
