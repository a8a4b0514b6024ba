"""The backend's gfx950 decode call sites over seeded random shapes and workspaces: batch,
lengths (empty sequences too), split count, query dtype, the GQA group of each call site, and
workspace buffers that are exact, larger in the batch dimension (their leading block is used),
shaped otherwise (not usable: the call allocates) or absent.

Bar: as the fixed-shape call-site tests -- output max-abs <= 1e-4 + the dtype's rounding
against the C oracle; the backend's output buffer is written in place whenever its leading
block fits; an empty sequence gives a NaN row.
"""
import numpy as np
import pytest
import torch

from conftest import to_dev
from test_gpu_backend_gfx950 import CALL_SITES, D, Layer, check, head_major_soa, oracle_out
from tq4_decode import workloads

pytestmark = pytest.mark.gpu
KINDS = ("exact", "bigger_batch", "other_shape", "none")


def _case(i):
    rng = np.random.default_rng(20261802 + i)
    batch = int(rng.integers(1, 24))
    lens = rng.integers(0, 2500, batch)
    lens[rng.random(batch) < 0.1] = 0
    if lens.max() == 0:
        lens[0] = 17
    return dict(seed=20261802 + i, site=sorted(CALL_SITES)[i % len(CALL_SITES)], batch=batch,
                lens=lens.astype(np.int32), splits=int(rng.choice([1, 4, 16, 32])),
                dtype=str(rng.choice(["bf16", "f16"])), mid=str(rng.choice(KINDS)),
                out=str(rng.choice(KINDS)), lse=str(rng.choice(KINDS)))


CASES = [_case(i) for i in range(24)]


def _id(c):
    return f"{c['site']}-B{c['batch']}-S{c['splits']}-{c['dtype']}-mid_{c['mid']}-out_{c['out']}-lse_{c['lse']}"


def _buffer(kind, shape, dtype, dev, grow):
    if kind == "none":
        return None
    if kind == "bigger_batch":
        shape = (shape[0] + 3,) + tuple(shape[1:])
    elif kind == "other_shape":
        shape = tuple(shape[:grow]) + (shape[grow] + 1,) + tuple(shape[grow + 1:])
    return torch.full(shape, float("nan"), dtype=dtype, device=dev)


@pytest.mark.parametrize("c", CASES, ids=[_id(c) for c in CASES])
def test_call_site_random_shape(dev, c):
    entry, make_kwargs, hq, hk = CALL_SITES[c["site"]]
    dtype = {"bf16": torch.bfloat16, "f16": torch.float16}[c["dtype"]]
    rng = np.random.default_rng(c["seed"])
    lens, B, S = c["lens"], c["batch"], c["splits"]
    w = workloads.small(c["seed"], B, lens, S, num_q_heads=hq, num_kv_heads=hk)
    query = rng.standard_normal((B, hq, D)).astype(np.float32)
    rot_t = workloads.random_orthogonal(rng, D)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    _, view = head_major_soa(t(w.kv_cache))
    q = t(query).to(dtype)
    bufs = (_buffer(c["mid"], (B, hq, S, D + 1), torch.float32, dev, 2),
            _buffer(c["out"], (B, hq, D), dtype, dev, 1),
            _buffer(c["lse"], (B, hq), torch.float32, dev, 1))
    print(_id(c), flush=True)
    kw = make_kwargs(q, view, t(w.block_table), t(w.seq_lens), t(rot_t.T.copy()), t(w.centroids), t(rot_t),
                     bufs, Layer(), S, int(lens.max()))
    out = entry(**kw)
    torch.cuda.synchronize()
    assert out.dtype == dtype and tuple(out.shape) == (B, hq, D)
    if c["out"] in ("exact", "bigger_batch"):
        assert out.data_ptr() == bufs[1].data_ptr(), "the backend's output buffer is used"
    ref = oracle_out(q.float().cpu().numpy(), rot_t, w.kv_cache, w.block_table, lens, w.centroids, S, hk)
    live = lens > 0
    assert torch.isnan(out[torch.from_numpy(~live).to(dev)]).all()
    check(out[torch.from_numpy(live).to(dev)], ref[live], dtype, _id(c))
