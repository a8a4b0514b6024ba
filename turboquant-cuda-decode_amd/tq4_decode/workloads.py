"""Seeded synthetic decode workloads (host side, numpy).

Every input is drawn from one seeded ``numpy.random.Generator`` (PCG64) on the CPU,
so the bytes a kernel reads on the GPU are the bytes a checker reads on the host.

The synthetic cache follows ``baseline/common.py:371-551``: the data region is
uniform random bytes (every byte is a valid pair of 4-bit codes), and the fp16
metadata is ``k_norm in [0.5, 2)``, ``v_scale in [0.01, 0.1)``, ``v_zero in [-0.5, 0.5)``.
``soa_to_aos`` is the lossless converter of ``baseline/common.py:554-672``: the AoS
slot stores the raw norm ``fp16(folded * ||c[idx]||)`` so both layouts decode the
same K.

Named workloads (sizes are the shapes of the decode step they stand for):

* ``qwen3_4b_b64_ctx4096``   B=64, ctx 4096, 32/8 heads, D=128, bs 16, 32 splits,
                              random-permuted block table.
* ``ragged_b64``             B=64, seq_lens ~ U[512, 8192], 32 splits, blocks scattered
                              over a 1.2x-oversized pool.
* ``gqa8_b8_ctx32768``       B=8, ctx 32768, 64/8 heads, 64 splits.
* ``full_b256_ctx2048``      B=256, ctx 2048, 32/8 heads, 16 splits, fp16 query and a
                              128x128 random orthogonal rotation.
"""
from __future__ import annotations

import dataclasses

import numpy as np

from . import codebook
from . import layout as L


@dataclasses.dataclass
class Workload:
    name: str
    q_rot: np.ndarray          # float32 [B, Hq, D]
    kv_cache: np.ndarray       # uint8 [num_blocks, bs, Hk, slot] (SoA bytes)
    block_table: np.ndarray    # int32 [B, max_blocks]
    seq_lens: np.ndarray       # int32 [B]
    centroids: np.ndarray      # float32 [16]
    num_kv_splits: int
    num_kv_heads: int
    block_size: int = 16
    query: np.ndarray | None = None     # fp16 [B, Hq, D] (full-decode workloads)
    rotation_t: np.ndarray | None = None  # float32 [D, D]: q_rot = query @ rotation_t

    @property
    def batch(self):
        return self.q_rot.shape[0]

    @property
    def num_q_heads(self):
        return self.q_rot.shape[1]

    @property
    def head_dim(self):
        return self.q_rot.shape[2]

    @property
    def pair_lut(self):
        return codebook.pair_lut(self.centroids)


def synthetic_cache(rng, num_blocks, num_kv_heads, head_dim=128, block_size=16):
    """SoA cache with uniform random code bytes and valid fp16 metadata."""
    slot = L.slot_bytes(head_dim)
    cache = np.empty((num_blocks, block_size, num_kv_heads, slot), dtype=np.uint8)
    flat = cache.reshape(num_blocks, -1)
    moff = L.meta_offset(block_size, num_kv_heads, head_dim)
    flat[:, :moff] = rng.integers(0, 256, size=(num_blocks, moff), dtype=np.uint8)
    shape = (num_blocks, num_kv_heads, block_size)
    k_norm = (0.5 + 1.5 * rng.random(shape, dtype=np.float32)).astype(np.float16)
    v_scale = (0.01 + 0.09 * rng.random(shape, dtype=np.float32)).astype(np.float16)
    v_zero = (-0.5 + rng.random(shape, dtype=np.float32)).astype(np.float16)
    meta = np.stack([k_norm, v_scale, v_zero], axis=2)  # [blocks, Hk, field, bs]
    flat[:, moff:] = meta.reshape(num_blocks, -1).view(np.uint8)
    return cache


def soa_to_aos(cache, cents, num_kv_heads, head_dim=128, block_size=16, chunk=512):
    """Return the AoS cache holding the same decoded K/V as SoA ``cache``."""
    num_blocks = cache.shape[0]
    half = head_dim // 2
    moff = L.meta_offset(block_size, num_kv_heads, head_dim)
    src = cache.reshape(num_blocks, -1)
    out = np.empty_like(cache)
    c = np.asarray(cents, dtype=np.float32)
    c_sq = c * c
    for b0 in range(0, num_blocks, chunk):
        b1 = min(b0 + chunk, num_blocks)
        data = src[b0:b1, :moff].reshape(b1 - b0, block_size, num_kv_heads, head_dim)
        meta = src[b0:b1, moff:].copy().view(np.float16).reshape(
            b1 - b0, num_kv_heads, L.NUM_SOA_FIELDS, block_size).transpose(0, 3, 1, 2)
        kb = data[..., :half]
        sq = (c_sq[kb & 0xF] + c_sq[kb >> 4]).sum(axis=-1, dtype=np.float32)
        raw = (meta[..., L.SOA_K_NORM].astype(np.float32) * np.sqrt(sq)).astype(np.float16)
        dst = out[b0:b1]
        dst[..., :half] = kb
        as_bytes = lambda x: np.ascontiguousarray(x)[..., None].view(np.uint8)  # noqa: E731
        dst[..., half:half + 2] = as_bytes(raw)
        dst[..., half + 2:head_dim + 2] = data[..., half:]
        dst[..., head_dim + 2:head_dim + 4] = as_bytes(meta[..., L.SOA_V_SCALE])
        dst[..., head_dim + 4:head_dim + 6] = as_bytes(meta[..., L.SOA_V_ZERO])
    return out


def random_orthogonal(rng, d):
    a = rng.standard_normal((d, d))
    q, r = np.linalg.qr(a)
    return (q * np.sign(np.diag(r))[None, :]).astype(np.float32)


def qwen3_4b_b64_ctx4096(seed=20261201, batch=64, ctx=4096, num_splits=32, num_q_heads=32):
    """The headline shape; ``num_q_heads`` other than 32 gives the same cache and block
    table with GQA group num_q_heads / 8."""
    rng = np.random.default_rng(seed)
    hk, hq, d, bs = 8, num_q_heads, 128, 16
    blocks_per_seq = ctx // bs
    nblk = batch * blocks_per_seq
    q_rot = rng.standard_normal((batch, hq, d), dtype=np.float32)
    cache = synthetic_cache(rng, nblk, hk, d, bs)
    bt = rng.permutation(nblk).astype(np.int32).reshape(batch, blocks_per_seq)
    seq = np.full(batch, ctx, dtype=np.int32)
    name = "qwen3_4b_b64_ctx4096" if hq == 32 else f"gqa{hq // hk}_b64_ctx4096"
    return Workload(name, q_rot, cache, bt, seq, codebook.centroids(d, 4), num_splits, hk, bs)


def ragged_b64(seed=20261202, batch=64, lo=512, hi=8192, num_splits=32, max_blocks=512):
    rng = np.random.default_rng(seed)
    hk, hq, d, bs = 8, 32, 128, 16
    seq = rng.integers(lo, hi + 1, size=batch).astype(np.int32)
    need = (seq + bs - 1) // bs
    pool = int(np.ceil(1.2 * need.sum()))
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.zeros((batch, max_blocks), dtype=np.int32)
    pos = 0
    for b in range(batch):
        bt[b, :need[b]] = perm[pos:pos + need[b]]
        pos += need[b]
    q_rot = rng.standard_normal((batch, hq, d), dtype=np.float32)
    cache = synthetic_cache(rng, pool, hk, d, bs)
    return Workload("ragged_b64", q_rot, cache, bt, seq, codebook.centroids(d, 4), num_splits,
                    hk, bs)


def gqa8_b8_ctx32768(seed=20261203, batch=8, ctx=32768, num_splits=64):
    rng = np.random.default_rng(seed)
    hk, hq, d, bs = 8, 64, 128, 16
    bps = ctx // bs
    nblk = batch * bps
    q_rot = rng.standard_normal((batch, hq, d), dtype=np.float32)
    cache = synthetic_cache(rng, nblk, hk, d, bs)
    bt = rng.permutation(nblk).astype(np.int32).reshape(batch, bps)
    seq = np.full(batch, ctx, dtype=np.int32)
    return Workload("gqa8_b8_ctx32768", q_rot, cache, bt, seq, codebook.centroids(d, 4),
                    num_splits, hk, bs)


def full_b256_ctx2048(seed=20261205, batch=256, ctx=2048, num_splits=16):
    rng = np.random.default_rng(seed)
    hk, hq, d, bs = 8, 32, 128, 16
    bps = ctx // bs
    nblk = batch * bps
    query = rng.standard_normal((batch, hq, d), dtype=np.float32).astype(np.float16)
    rot_t = random_orthogonal(rng, d)
    q_rot = (query.astype(np.float32) @ rot_t).astype(np.float32)
    cache = synthetic_cache(rng, nblk, hk, d, bs)
    bt = rng.permutation(nblk).astype(np.int32).reshape(batch, bps)
    seq = np.full(batch, ctx, dtype=np.int32)
    return Workload("full_b256_ctx2048", q_rot, cache, bt, seq, codebook.centroids(d, 4),
                    num_splits, hk, bs, query=query, rotation_t=rot_t)


def small(seed, batch, seq_lens, num_splits, num_q_heads=32, num_kv_heads=8, head_dim=128,
          block_size=16, spare_blocks=3, name="small"):
    """Small random-permuted workload for parity cases (ragged lengths allowed)."""
    rng = np.random.default_rng(seed)
    seq = np.asarray(seq_lens, dtype=np.int32).reshape(batch)
    need = (seq + block_size - 1) // block_size
    max_blocks = int(max(1, need.max()))
    pool = int(need.sum()) + spare_blocks
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.zeros((batch, max_blocks), dtype=np.int32)
    pos = 0
    for b in range(batch):
        bt[b, :need[b]] = perm[pos:pos + need[b]]
        pos += need[b]
    q_rot = rng.standard_normal((batch, num_q_heads, head_dim), dtype=np.float32)
    cache = synthetic_cache(rng, pool, num_kv_heads, head_dim, block_size)
    return Workload(name, q_rot, cache, bt, seq, codebook.centroids(head_dim, 4), num_splits,
                    num_kv_heads, block_size)


WORKLOADS = {
    "qwen3_4b_b64_ctx4096": qwen3_4b_b64_ctx4096,
    "ragged_b64": ragged_b64,
    "gqa8_b8_ctx32768": gqa8_b8_ctx32768,
    "full_b256_ctx2048": full_b256_ctx2048,
}
