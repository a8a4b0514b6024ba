"""The full decode step's one-split path with the query rotation inside Stage1.

When every (sequence, kv-head part) gets one wave, ``tq4_full_decode`` runs each sequence as
one split and the Stage1 kernel writes the output rows itself; for fp16 / bf16 queries and
Hk * parts dividing 8, the kernel also rotates the query: one workgroup per sequence holds
its waves, which compute ``query @ rot_t`` into LDS with the rotation launch's operands and
MFMA order.  So the step must be bit-identical to rotation launch + Stage1 (one split) +
Stage2, run separately -- which pins the fused rotation to the rotation launch (itself
within 2e-5 of a float64 matmul, ``test_gpu_stage2.py``) -- and within the oracle's bar.
The fused path leaves the q_rot workspace unwritten (NaN-prefilled here), which shows
that it ran; fp32 queries keep the rotation launch (the workspace is written).

Shapes: (kv-heads, GQA group) with one, two, four and eight waves per sequence, groups with
padding heads (3, 6), two parts per kv-head (16) and four (MQA: one kv-head, 32 q-heads); rows of very large and very small
magnitude; empty and one-token sequences; sinks.
"""
import numpy as np
import pytest
import torch

from conftest import to_dev
from oracle import native
from oracle import stage1 as ostage
from tq4_decode import ops, workloads

pytestmark = pytest.mark.gpu
D = 128


def _case(seed, batch, hk, group, max_len=300):
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, max_len, batch).astype(np.int32)
    lens[[0, batch // 2]] = 0
    lens[1] = 1
    w = workloads.small(seed, batch, lens, 16, num_q_heads=hk * group, num_kv_heads=hk)
    query = rng.standard_normal((batch, hk * group, D)).astype(np.float32)
    query[2, 0] *= 2e3   # rows far from unit scale (inside the fp16 range): the per-row scale
    query[3, 1] *= 1e-6
    return rng, w, query, workloads.random_orthogonal(rng, D)


def _separate(dev, q, r, cache, bt, sl, cents, out_dtype, sinks):
    """Rotation launch + Stage1 with one split + Stage2."""
    q_rot = torch.empty(q.shape, dtype=torch.float32, device=dev)
    ops.rotate_query(q, r, q_rot)
    mid = ops.stage1(q_rot, cache, bt, sl, ops.pair_lut_device(cents), num_kv_splits=1, sinks=sinks)
    return ops.stage2(mid, sl, out_dtype=out_dtype)


# (kv-heads, group, batch): batch * kv-heads * parts fills the device (2048 waves), so the
# step takes the one-split path
SHAPES = [(8, 4, 256), (8, 8, 256), (8, 3, 256), (8, 6, 256), (4, 16, 256), (4, 4, 512), (2, 8, 1024),
          (1, 8, 2048), (1, 32, 512)]


@pytest.mark.parametrize("qdtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hk,group,batch", SHAPES)
def test_fused_rotation_matches_the_separate_launches(dev, hk, group, batch, qdtype):
    rng, w, query, rot_t = _case(800 + 10 * hk + group, batch, hk, group)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    q, r = t(query).to(qdtype), t(rot_t)
    cache, bt, sl, cents = t(w.kv_cache), t(w.block_table), t(w.seq_lens), t(w.centroids)
    ws = ops.DecodeWorkspace(batch, hk * group, 16, dev, torch.bfloat16)
    ws.q_rot.fill_(float("nan"))
    out, lse = ops.full_decode(q, r, cache, bt, sl, cents, 16, out_dtype=torch.bfloat16, workspace=ws)
    ref_out, ref_lse = _separate(dev, q, r, cache, bt, sl, cents, torch.bfloat16, None)
    torch.cuda.synchronize()
    assert torch.isnan(ws.q_rot).all(), "the one-split step rotated inside Stage1"
    a, b = out.float().cpu().numpy(), ref_out.float().cpu().numpy()
    assert np.array_equal(a, b, equal_nan=True), "fused rotation differs from the rotation launch"
    assert np.array_equal(lse.cpu().numpy(), ref_lse.cpu().numpy())
    live = w.seq_lens > 0
    assert np.isnan(a[~live]).all() and np.isneginf(lse.cpu().numpy()[~live]).all()
    qr = (q.float().cpu().numpy().astype(np.float64) @ rot_t.astype(np.float64)).astype(np.float32)
    mid = native.stage1(qr, w.kv_cache, w.block_table, w.seq_lens, w.centroids, 16, num_kv_heads=hk)
    ro, _ = native.stage2(mid, w.seq_lens)
    diff = np.abs(a[live] - ro[live])
    print(f"Hk{hk} G{group} B{batch} {qdtype}: max-abs {diff.max():.3e}")
    assert np.all(diff <= 1e-4 + 2.0 ** -8 * np.abs(ro[live]))


@pytest.mark.parametrize("hk,group", [(8, 4), (4, 16)])
def test_fused_rotation_with_sinks(dev, hk, group):
    rng, w, query, rot_t = _case(830 + group, 256, hk, group)
    sinks = rng.normal(0.0, 3.0, hk * group).astype(np.float32)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    q, r = t(query).half(), t(rot_t)
    cache, bt, sl, cents = t(w.kv_cache), t(w.block_table), t(w.seq_lens), t(w.centroids)
    out, lse = ops.full_decode(q, r, cache, bt, sl, cents, 16, out_dtype=torch.float32, sinks=t(sinks))
    ref_out, ref_lse = _separate(dev, q, r, cache, bt, sl, cents, torch.float32, t(sinks))
    torch.cuda.synchronize()
    a = out.cpu().numpy()
    assert np.array_equal(a, ref_out.cpu().numpy(), equal_nan=True)
    assert np.array_equal(lse.cpu().numpy(), ref_lse.cpu().numpy())
    qr = (q.float().cpu().numpy().astype(np.float64) @ rot_t.astype(np.float64)).astype(np.float32)
    live = w.seq_lens > 0  # (the float64 oracle's Stage2 takes live sequences only)
    ro, _ = ostage.stage2(ostage.stage1(qr[live], w.kv_cache, w.block_table[live], w.seq_lens[live],
                                        w.centroids, 1, num_kv_heads=hk, sinks=sinks), w.seq_lens[live])
    err = np.abs(a[live] - ro).max()
    print(f"sinks Hk{hk} G{group}: max-abs {err:.3e}")
    assert err <= 1e-4


def test_fp32_queries_keep_the_rotation_launch(dev):
    rng, w, query, rot_t = _case(840, 256, 8, 4)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    q, r = t(query), t(rot_t)
    cache, bt, sl, cents = t(w.kv_cache), t(w.block_table), t(w.seq_lens), t(w.centroids)
    ws = ops.DecodeWorkspace(256, 32, 16, dev, torch.float32)
    ws.q_rot.fill_(float("nan"))
    out, lse = ops.full_decode(q, r, cache, bt, sl, cents, 16, out_dtype=torch.float32, workspace=ws)
    ref_out, _ = _separate(dev, q, r, cache, bt, sl, cents, torch.float32, None)
    torch.cuda.synchronize()
    assert not torch.isnan(ws.q_rot).any(), "fp32 queries go through the rotation launch"
    assert np.array_equal(out.cpu().numpy(), ref_out.cpu().numpy(), equal_nan=True)
