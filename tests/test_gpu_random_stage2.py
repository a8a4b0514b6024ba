"""Stage2 over seeded random shapes: batch, q-heads, split counts (up to 300, so merges of one to
ten 32-split chunks) and lengths that leave any number of trailing splits empty, with random
split rows (outputs and LSE spread over 40 units) and NaN in every row Stage1 would not write.

Bar: outputs and LSE within 1e-5 (fp32) of the C oracle's merge; empty sequences give NaN
outputs and -inf LSE.
"""
import numpy as np
import pytest
import torch

from conftest import to_dev
from oracle import native
from tq4_decode import ops

pytestmark = pytest.mark.gpu


def _case(i):
    rng = np.random.default_rng(20261702 + i)
    splits = int(rng.choice([1, 2, 31, 32, 33, 63, 64, 65, 100, 300]))
    batch = int(rng.integers(1, 40))
    lens = rng.integers(0, 4 * splits + 40, batch)
    lens[rng.random(batch) < 0.15] = 0
    return dict(seed=20261702 + i, splits=splits, batch=batch, hq=int(rng.choice([1, 8, 32])),
                lens=lens.astype(np.int32))


CASES = [_case(i) for i in range(24)]


@pytest.mark.parametrize("c", CASES, ids=[f"B{c['batch']}-Hq{c['hq']}-S{c['splits']}" for c in CASES])
def test_stage2_random_shape(dev, c):
    rng = np.random.default_rng(c["seed"])
    B, hq, S, lens = c["batch"], c["hq"], c["splits"], c["lens"]
    mid = rng.standard_normal((B, hq, S, 129)).astype(np.float32)
    mid[..., 128] = rng.uniform(-20, 20, (B, hq, S)).astype(np.float32)
    split_len = (lens + S - 1) // S
    live = np.where(split_len > 0, np.minimum(S, (lens + np.maximum(split_len, 1) - 1) // np.maximum(split_len, 1)), 0)
    for b in range(B):
        mid[b, :, live[b]:, :] = np.nan  # rows Stage1 leaves unwritten
    out, lse = torch.empty(B, hq, 128, device=dev), torch.empty(B, hq, device=dev)
    ops.stage2(to_dev(mid, dev), to_dev(lens, dev), out, lse)
    torch.cuda.synchronize()
    ro, rl = native.stage2(mid, lens)
    got, gl = out.cpu().numpy(), lse.cpu().numpy()
    empty = lens == 0
    assert np.isnan(got[empty]).all() and np.isneginf(gl[empty]).all()
    full = ~empty
    if full.any():
        print(f"max-abs out {np.abs(got[full] - ro[full]).max():.3e} lse {np.abs(gl[full] - rl[full]).max():.3e}")
        assert np.abs(got[full] - ro[full]).max() <= 1e-5
        assert np.abs(gl[full] - rl[full]).max() <= 1e-5
