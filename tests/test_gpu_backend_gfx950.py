"""The vLLM backend's two decode call sites on gfx950, called exactly as the backend calls them.

On gfx950 the backend (``reference/turboquant_attn.py:383``) sends every decode through one of:

* ``flydsl_turboquant_decode_attention(**kwargs)`` for GQA 6 / 8 / 16 layers
  (``:1143-1183``) -- here ``tq4_decode.flydsl_decode``;
* ``_dispatch_decode_soa(**kwargs)`` for the others, e.g. the GQA-4 Qwen3-4B shape
  (``:1194-1216``): it loads ``triton_turboquant_decode_attention_soa`` through
  ``_soa_imports()`` (``:87-103``) and filters the kwargs by the target's signature,
  raising for any non-None kwarg the target does not take (``:1241-1257``) -- here
  ``tq4_decode.soa_unified``.

The tests below restate that filter, build the kwargs dicts of those two call sites key for
key, and pass what the backend passes: the ``kv_cache.transpose(1, 2)`` view of its
``[blocks, Hk, block_size, slot]`` SoA cache, the workspace buffers of ``:1133-1141``
(``mid_o`` fp32 ``[B, Hq, S, D+1]``, output in the query dtype, ``lse`` fp32), the layer as
``buf_holder``, and ``PiT``.  Results are checked against the C oracle (rotation in float64,
Stage1, Stage2) and, captured in a graph, on replays after ``seq_lens`` / ``block_table``
change in place.

Bar: output max-abs <= 1e-4 + the output dtype's rounding (2^-11 relative for fp16, 2^-8
for bf16); replays equal an eager call bit for bit.
"""
import inspect

import numpy as np
import pytest
import torch

from conftest import to_dev
from oracle import native
from tq4_decode import codebook, flydsl_decode, soa_unified, workloads

pytestmark = pytest.mark.gpu
D, BS = 128, 16


def dispatch_decode_soa(soa_decode, **kwargs):
    """``_dispatch_decode_soa`` of ``reference/turboquant_attn.py:1241-1257``."""
    accepted = set(inspect.signature(soa_decode).parameters)
    dropped = [k for k, v in kwargs.items() if k not in accepted and v is not None]
    if dropped:
        raise NotImplementedError(f"SoA decode does not support kwargs {sorted(dropped)}")
    return soa_decode(**{k: v for k, v in kwargs.items() if k in accepted})


class Layer:
    """Stands for the attention layer the backend passes as ``buf_holder``."""


def soa_kwargs(q, view, bt, sl, Pi, cents, PiT, bufs, layer, S, max_seq_len):
    """The kwargs of ``reference/turboquant_attn.py:1194-1216`` (4-bit ``_nc`` preset)."""
    mid_o_buf, output_buf, lse_buf = bufs
    return dict(query=q, kv_cache=view, block_table=bt, seq_lens=sl, Pi=Pi, centroids=cents,
                scale=D ** -0.5, mse_bits=4, key_packed_size=66, value_quant_bits=4,
                value_packed_size=68, max_seq_len=max_seq_len, key_fp8=False, norm_correction=True,
                PiT=PiT, mid_o_buf=mid_o_buf, output_buf=output_buf, lse_buf=lse_buf, buf_holder=layer,
                max_num_kv_splits=S, sinks=None, sliding_window=None)


def flydsl_kwargs(*args):
    """The kwargs of ``reference/turboquant_attn.py:1161-1183``: the same minus sliding_window."""
    kw = soa_kwargs(*args)
    del kw["sliding_window"]
    return kw


def head_major_soa(cache):
    """The backend's ``[blocks, Hk, bs, slot]`` storage of an SoA cache (the block's bytes are
    the kernels' own layout) and the ``transpose(1, 2)`` view it passes."""
    nb, bs, hk, slot = cache.shape
    storage = cache.reshape(-1).clone().view(nb, hk, bs, slot)
    view = storage.transpose(1, 2)
    assert view.stride() == (bs * hk * slot, slot, bs * slot, 1) and not view.is_contiguous()
    return storage, view


def workspace(B, Hq, S, dtype, dev):
    """``current_workspace_manager().get_simultaneous(...)`` of ``:1133-1141``."""
    return (torch.empty(B, Hq, S, D + 1, dtype=torch.float32, device=dev),
            torch.empty(B, Hq, D, dtype=dtype, device=dev),
            torch.empty(B, Hq, dtype=torch.float32, device=dev))


def oracle_out(query, rot_t, cache, table, lens, cents, S, hk):
    q_rot = (query.astype(np.float64) @ rot_t.astype(np.float64)).astype(np.float32)
    mid = native.stage1(q_rot, cache, table, lens, cents, S, num_kv_heads=hk)
    return native.stage2(mid, lens)[0]


def rel_bar(dtype):
    return 2.0 ** -11 if dtype == torch.float16 else 2.0 ** -8


def check(got, ref, dtype, what):
    diff = np.abs(got.float().cpu().numpy() - ref)
    print(f"{what}: max-abs {diff.max():.3e}")
    assert np.all(diff <= 1e-4 + rel_bar(dtype) * np.abs(ref)), what


CALL_SITES = {
    # name: (entry, kwargs builder, Hq, Hk)
    "soa_gqa4": (lambda **kw: dispatch_decode_soa(soa_unified.triton_turboquant_decode_attention_soa, **kw),
                 soa_kwargs, 32, 8),
    "flydsl_gqa8": (flydsl_decode.flydsl_turboquant_decode_attention, flydsl_kwargs, 64, 8),
    "flydsl_gqa16": (flydsl_decode.flydsl_turboquant_decode_attention, flydsl_kwargs, 64, 4),
    "flydsl_gqa6": (flydsl_decode.flydsl_turboquant_decode_attention, flydsl_kwargs, 48, 8),
}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("site", sorted(CALL_SITES))
def test_call_site_matches_oracle(dev, site, dtype):
    entry, make_kwargs, hq, hk = CALL_SITES[site]
    rng = np.random.default_rng(700 + hq + hk)
    lens = np.array([1500, 1, 333, 4096, 64], np.int32)
    B, S = len(lens), 32
    w = workloads.small(701 + hq, B, lens, S, num_q_heads=hq, num_kv_heads=hk)
    query = rng.standard_normal((B, hq, D)).astype(np.float32)
    rot_t = workloads.random_orthogonal(rng, D)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    _, view = head_major_soa(t(w.kv_cache))
    q = t(query).to(dtype)
    layer = Layer()
    kw = make_kwargs(q, view, t(w.block_table), t(w.seq_lens), t(rot_t.T.copy()), t(w.centroids),
                     t(rot_t), workspace(B, hq, S, dtype, dev), layer, S, int(lens.max()))
    out = entry(**kw)
    torch.cuda.synchronize()
    assert out.dtype == dtype and tuple(out.shape) == (B, hq, D)
    assert out.data_ptr() == kw["output_buf"].data_ptr(), "the backend's output buffer is used"
    ref = oracle_out(q.float().cpu().numpy(), rot_t, w.kv_cache, w.block_table, lens, w.centroids, S, hk)
    check(out, ref, dtype, f"{site} {dtype}")


def test_soa_adapter_rejects_what_the_reference_rejects(dev):
    """A sliding window is dropped by the filter and raises, as with the reference adapter;
    a value_packed_size that is not the 4-bit preset's raises."""
    w = workloads.small(705, 2, [40, 17], 4)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    rot_t = workloads.random_orthogonal(np.random.default_rng(5), D)
    _, view = head_major_soa(t(w.kv_cache))
    q = torch.randn(2, 32, D, device=dev, dtype=torch.bfloat16)
    kw = soa_kwargs(q, view, t(w.block_table), t(w.seq_lens), t(rot_t.T.copy()), t(w.centroids),
                    t(rot_t), (None, None, None), None, 4, 40)
    f = soa_unified.triton_turboquant_decode_attention_soa
    with pytest.raises(NotImplementedError, match="sliding_window"):
        dispatch_decode_soa(f, **{**kw, "sliding_window": 128})
    with pytest.raises(RuntimeError, match="value_packed_size"):
        dispatch_decode_soa(f, **{**kw, "value_packed_size": 64})
    assert dispatch_decode_soa(f, **kw).shape == (2, 32, D)


@pytest.mark.parametrize("site,batch", [("soa_gqa4", 4), ("soa_gqa4", 256), ("flydsl_gqa8", 6)])
def test_call_site_graph_capture_and_replay(dev, site, batch):
    """Capture the call site once (workspace buffers given, the layer holding the rest,
    warmed up first), then change ``seq_lens`` and ``block_table`` in place and replay:
    every replay equals an eager call on the same inputs bit for bit, and the oracle.  For
    the GQA-4 site batch 256 gives one wave per (sequence, kv-head), the path whose Stage1
    writes the output itself."""
    entry, make_kwargs, hq, hk = CALL_SITES[site]
    rng = np.random.default_rng(720 + batch + hq)
    S, mb = 16, 24
    nb = batch * mb + 5
    cache_np = workloads.synthetic_cache(rng, nb, hk)
    query = rng.standard_normal((batch, hq, D)).astype(np.float32)
    rot_t = workloads.random_orthogonal(rng, D)
    cents = codebook.centroids(D, 4)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    _, view = head_major_soa(t(cache_np))
    q = t(query).to(torch.bfloat16)
    bt = torch.zeros(batch, mb, dtype=torch.int32, device=dev)
    sl = torch.zeros(batch, dtype=torch.int32, device=dev)
    kw = make_kwargs(q, view, bt, sl, t(rot_t.T.copy()), t(cents), t(rot_t),
                     workspace(batch, hq, S, torch.bfloat16, dev), Layer(), S, mb * BS)

    def fill():
        lens = rng.integers(1, mb * BS + 1, batch).astype(np.int32)
        lens[0] = mb * BS
        table = rng.permutation(nb)[:batch * mb].astype(np.int32).reshape(batch, mb)
        sl.copy_(t(lens))
        bt.copy_(t(table))
        return lens, table

    fill()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            entry(**kw)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = entry(**kw)
    qf = q.float().cpu().numpy()
    for rep in range(3):
        lens, table = fill()
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager = entry(**kw).clone()  # eager work between the replays
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {rep} differs from the eager call"
        check(got, oracle_out(qf, rot_t, cache_np, table, lens, cents, S, hk), torch.bfloat16,
              f"{site} B{batch} replay {rep}")
