"""Write the store-semantics parity fixture ``config1_b2_ctx256.npz``.

Workload: batch 2, ctx 256, 32 Q / 8 KV heads, D=128, KV block 16, 4 splits.  Raw
K and V are N(0,1) fp16; K is normalised, rotated by a seeded random orthogonal
128x128 matrix, bucketised on the Lloyd-Max midpoints, packed low-nibble-first,
with the norm-corrected fp16 norm (SoA) or raw fp16 norm (AoS); V is per-token
min/max 4-bit with fp16 scale and min (``reference/soa_store.py:26-116``,
``:223-373``, ``:482-485``; ``reference/aos_store.py:268-325``).  The query is N(0,1)
fp16 and ``q_rot = query.float() @ PiT``.  Identity block table.

Expected outputs come from the float64 oracle (``oracle/stage1.py``).  Usage:
``python tests/golden/make_fixture_config1.py``
"""
from __future__ import annotations

import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import codebook, layout, stage1, store  # noqa: E402

OUT = pathlib.Path(__file__).with_name("config1_b2_ctx256.npz")
SEED = 20261101
B, CTX, HQ, HK, D, BS, S = 2, 256, 32, 8, 128, 16, 4


def main() -> None:
    rng = np.random.default_rng(SEED)
    a = rng.standard_normal((D, D))
    q_mat, r_mat = np.linalg.qr(a)
    rot_t = (q_mat * np.sign(np.diag(r_mat))[None, :]).astype(np.float32)
    cents = codebook.centroids(D, 4)
    nblk = B * CTX // BS
    caches = {}
    for name, aos in (("soa", False), ("aos", True)):
        caches[name] = np.zeros((nblk, BS, HK, layout.slot_bytes(D)), dtype=np.uint8)
    key = rng.standard_normal((B * CTX, HK, D), dtype=np.float32).astype(np.float16)
    value = rng.standard_normal((B * CTX, HK, D), dtype=np.float32).astype(np.float16)
    slots = np.arange(B * CTX, dtype=np.int64)
    for name, aos in (("soa", False), ("aos", True)):
        store.store(key.astype(np.float32), value.astype(np.float32), slots, rot_t, cents,
                    caches[name], block_size=BS, is_aos=aos)
    query = rng.standard_normal((B, HQ, D), dtype=np.float32).astype(np.float16)
    q_rot = (query.astype(np.float64) @ rot_t.astype(np.float64)).astype(np.float32)
    bt = np.arange(nblk, dtype=np.int32).reshape(B, CTX // BS)
    seq = np.full(B, CTX, dtype=np.int32)
    out = {}
    for name, aos in (("soa", False), ("aos", True)):
        mid = stage1.stage1(q_rot, caches[name], bt, seq, cents, S, num_kv_heads=HK,
                            block_size=BS, is_aos=aos)
        o, l = stage1.stage2(mid, seq)
        out[f"mid_{name}"] = mid.astype(np.float32)
        out[f"out_{name}"] = o.astype(np.float32)
        out[f"lse_{name}"] = l.astype(np.float32)
    np.savez_compressed(
        OUT, seed=np.int64(SEED), query=query, rotation_t=rot_t, q_rot=q_rot,
        cache_soa=caches["soa"], cache_aos=caches["aos"], block_table=bt, seq_lens=seq,
        centroids=cents, num_kv_splits=np.int64(S), num_kv_heads=np.int64(HK),
        block_size=np.int64(BS), **out)
    print("wrote", OUT, OUT.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
