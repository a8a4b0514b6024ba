"""tq4_full_decode_noalloc through the C ABI: the same results as tq4_full_decode with caller
workspaces (bit for bit: the same kernels on the same inputs), on two calls in a row, the
second with a smaller input, and a clear rejection of shapes beyond its scratch."""
import numpy as np
import pytest
import torch

from conftest import to_dev
from tq4_decode import _lib, codebook, ops, workloads

pytestmark = pytest.mark.gpu
DT = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _inputs(dev, seed, batch, lens, splits, qdtype):
    rng = np.random.default_rng(seed)
    w = workloads.small(seed, batch, lens, splits)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    query = t(rng.standard_normal((batch, 32, 128)).astype(np.float32)).to(qdtype)
    rot = t(workloads.random_orthogonal(rng, 128))
    return w, query, rot, t(w.kv_cache), t(w.block_table), t(w.seq_lens), t(codebook.centroids(128, 4))


def _noalloc(query, rot, cents, cache, bt, sl, splits, out_dtype, sinks=None):
    B, Hq, D = query.shape
    out = torch.full((B, Hq, D), float("nan"), dtype=out_dtype, device=query.device)
    lse = torch.full((B, Hq), float("nan"), device=query.device)
    rc = _lib.load().tq4_full_decode_noalloc(
        query.data_ptr(), DT[query.dtype], rot.data_ptr(), cents.data_ptr(), cache.data_ptr(),
        bt.data_ptr(), sl.data_ptr(), out.data_ptr(), DT[out_dtype], lse.data_ptr(), B, Hq, 8, D, 16,
        bt.size(1), cache.stride(0), splits, 0, 128 ** -0.5,
        None if sinks is None else sinks.data_ptr(), torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "tq4_full_decode_noalloc")
    return out, lse


@pytest.mark.parametrize("qdtype", [torch.float16, torch.float32])
def test_noalloc_full_decode_matches_the_workspace_entry(dev, qdtype):
    # (B, lengths, splits, output dtype): Stage1 + Stage2 over scratch Stage1 rows, then a
    # smaller call; then B256 (one split per sequence: no Stage1 rows), then a small one again
    cases = [(24, [4096] * 12 + [1, 0, 333, 4095, 17, 2048, 64, 100, 1000, 3000, 5, 77], 32, torch.float32),
             (3, [700, 0, 129], 8, torch.bfloat16),
             (256, list(range(0, 2560, 10)), 16, torch.float16),
             (2, [64, 4096], 32, torch.float32)]
    rng = np.random.default_rng(701)
    for i, (B, lens, S, odt) in enumerate(cases):
        w, q, rot, cache, bt, sl, cents = _inputs(dev, 702 + i, B, lens, S, qdtype)
        sinks = torch.from_numpy(rng.normal(0, 2, 32).astype(np.float32)).to(dev) if i == 1 else None
        ref_out, ref_lse = ops.full_decode(q, rot, cache, bt, sl, cents, S, out_dtype=odt, sinks=sinks)
        ref_out, ref_lse = ref_out.clone(), ref_lse.clone()
        out, lse = _noalloc(q, rot, cents, cache, bt, sl, S, odt, sinks)
        torch.cuda.synchronize()
        a, b = out.float().cpu().numpy(), ref_out.float().cpu().numpy()
        assert np.array_equal(np.isnan(a), np.isnan(b)), f"call {i}: NaN pattern differs"
        assert np.array_equal(a[~np.isnan(a)], b[~np.isnan(b)]), f"call {i}: outputs differ"
        assert np.array_equal(lse.cpu().numpy(), ref_lse.cpu().numpy()), f"call {i}: LSE differs"


def test_noalloc_rejects_workspaces_beyond_its_scratch(dev):
    """B64 x 32 heads x 64 splits: 64 x 8 (sequence, kv-head) pairs get several waves, so
    Stage1 writes 64 * 32 * 64 rows of 129 floats (67.6 MB) -- beyond the 40 MiB scratch."""
    w, q, rot, cache, bt, sl, cents = _inputs(dev, 710, 64, [64] * 64, 64, torch.float16)
    lib = _lib.load()
    out = torch.full((64, 32, 128), float("nan"), device=dev)
    lse = torch.full((64, 32), float("nan"), device=dev)
    rc = lib.tq4_full_decode_noalloc(q.data_ptr(), 2, rot.data_ptr(), cents.data_ptr(), cache.data_ptr(),
                                     bt.data_ptr(), sl.data_ptr(), out.data_ptr(), 0, lse.data_ptr(),
                                     64, 32, 8, 128, 16, bt.size(1), cache.stride(0), 64, 0, 128 ** -0.5, None,
                                     torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 1
    assert b"scratch holds" in lib.tq4_last_error()
    assert torch.isnan(out).all() and torch.isnan(lse).all()  # nothing launched
