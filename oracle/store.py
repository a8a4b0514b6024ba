"""numpy restatement of the TurboQuant 4-bit cache writers (oracle side).

SoA writer (``reference/soa_store.py``):

* launcher ``:482-485``: ``norm = ||k||`` (fp32), ``x_hat = k / (norm + 1e-8)``, ``y = x_hat @ PiT``
* bucketize ``:306-316``: 4-step binary search over the 15 midpoints, going right when
  ``y >= mid`` -- i.e. the index is the count of midpoints ``<= y``
* pack ``:319-325``: low nibble = even dim
* norm correction ``:343-353``: stored K scalar is ``fp16(norm / sqrt(sum c[idx]^2 + 1e-16))``
* V ``:86-116``: ``scale = max((max - min) / 15, 1e-8)``,
  ``code = clamp(int((v - min) / scale + 0.5), 0, 15)``, fp16 scale and fp16 min in the
  per-block metadata region.

AoS writer (``reference/aos_store.py:268-325``): same K indices and V codes, but the slot
stores the raw ``fp16(norm)`` and V scale/zero inline.

Arithmetic is float32 throughout, as in the Triton kernels.  Parity: the exact
packed bytes of the upstream store are "parity unpinned" (they depend on Triton's
fp32 division and reduction order); what is pinned is the round trip -- every field
written here is read back by ``layout.gather_*`` at the positions the decode kernels
use, and every K index is the nearest centroid to ``y`` (brute force).
"""
from __future__ import annotations

import numpy as np

from . import layout


def quantize_keys(key, rot_t, cents):
    """Return ``(idx int64 [N, H, D], norm float32 [N, H], folded float32 [N, H])``."""
    k = np.asarray(key, dtype=np.float32)
    norm = np.sqrt((k.astype(np.float64) ** 2).sum(axis=-1)).astype(np.float32)
    x_hat = k / (norm[..., None] + np.float32(1e-8))
    y = (x_hat.astype(np.float64) @ np.asarray(rot_t, dtype=np.float64)).astype(np.float32)
    c = np.asarray(cents, dtype=np.float32)
    mids = ((c[:-1] + c[1:]) * np.float32(0.5)).astype(np.float32)
    idx = np.searchsorted(mids, y, side="right").astype(np.int64)
    cv = c[idx]
    inv = np.float32(1.0) / np.sqrt((cv * cv).sum(axis=-1, dtype=np.float32) + np.float32(1e-16))
    folded = (norm * inv).astype(np.float32)
    return idx, norm, folded


def quantize_values(value):
    """Return ``(codes int64 [N, H, D], scale float32 [N, H], vmin float32 [N, H])``."""
    v = np.asarray(value, dtype=np.float32)
    vmin = v.min(axis=-1)
    vmax = v.max(axis=-1)
    scale = (vmax - vmin) / np.float32(15.0)
    scale = np.where(scale > np.float32(1e-8), scale, np.float32(1e-8)).astype(np.float32)
    codes = ((v - vmin[..., None]) / scale[..., None] + np.float32(0.5)).astype(np.int32)
    codes = np.clip(codes, 0, 15).astype(np.int64)
    return codes, scale, vmin


def pack_nibbles(codes):
    c = np.asarray(codes, dtype=np.uint8)
    return (c[..., 0::2] & 0xF) | ((c[..., 1::2] & 0xF) << 4)


def _put_fp16(flat, byte_offsets, values):
    u16 = np.asarray(values, dtype=np.float16).view(np.uint16).reshape(-1)
    offs = np.asarray(byte_offsets, dtype=np.int64).reshape(-1)
    flat[offs] = (u16 & 0xFF).astype(np.uint8)
    flat[offs + 1] = (u16 >> 8).astype(np.uint8)


def store(key, value, slot_mapping, rot_t, cents, cache, *, block_size=16, is_aos=False):
    """Write ``key``/``value`` ``[N, Hk, D]`` into ``cache`` (uint8, modified in place)."""
    n_tok, num_kv_heads, head_dim = np.asarray(key).shape
    half = head_dim // 2
    flat = cache.reshape(-1)
    idx, norm, folded = quantize_keys(key, rot_t, cents)
    codes, scale, vmin = quantize_values(value)
    kbytes = pack_nibbles(idx)
    vbytes = pack_nibbles(codes)
    slots = np.asarray(slot_mapping, dtype=np.int64)
    keep = slots >= 0
    blk = slots // block_size
    off = slots % block_size
    stride = layout.block_bytes(block_size, num_kv_heads, head_dim)
    cols = np.arange(half, dtype=np.int64)
    for h in range(num_kv_heads):
        sel = np.nonzero(keep)[0]
        b, t = blk[sel], off[sel]
        if is_aos:
            slot_sz = layout.slot_bytes(head_dim)
            base = b * stride + t * (num_kv_heads * slot_sz) + h * slot_sz
            flat[base[:, None] + cols[None, :]] = kbytes[sel, h]
            _put_fp16(flat, base + half, norm[sel, h])
            flat[base[:, None] + half + 2 + cols[None, :]] = vbytes[sel, h]
            _put_fp16(flat, base + head_dim + 2, scale[sel, h])
            _put_fp16(flat, base + head_dim + 4, vmin[sel, h])
        else:
            data = b * stride + t * (num_kv_heads * head_dim) + h * head_dim
            flat[data[:, None] + cols[None, :]] = kbytes[sel, h]
            flat[data[:, None] + half + cols[None, :]] = vbytes[sel, h]
            meta = b * stride + layout.soa_meta_offset(block_size, num_kv_heads, head_dim)
            fld = lambda f: meta + ((h * layout.NUM_SOA_FIELDS + f) * block_size + t) * 2  # noqa: E731
            _put_fp16(flat, fld(layout.SOA_K_NORM), folded[sel, h])
            _put_fp16(flat, fld(layout.SOA_V_SCALE), scale[sel, h])
            _put_fp16(flat, fld(layout.SOA_V_ZERO), vmin[sel, h])
    return cache


def store_fp8(key, value, slot_mapping, cache, *, block_size=16, is_aos=False):
    """FP8-key preset writer (``reference/soa_store.py:125-212``; AoS ``reference/aos_store.py``):
    K bytes = E4M3 of the raw key (saturating), V as ``quantize_values``."""
    from . import fp8

    n_tok, num_kv_heads, head_dim = np.asarray(key).shape
    flat = cache.reshape(-1)
    kbytes = fp8.encode(np.asarray(key, dtype=np.float32))
    codes, scale, vmin = quantize_values(value)
    vbytes = pack_nibbles(codes)
    slots = np.asarray(slot_mapping, dtype=np.int64)
    sel = np.nonzero(slots >= 0)[0]
    b, t = slots[sel] // block_size, slots[sel] % block_size
    stride = fp8.block_bytes(block_size, num_kv_heads, head_dim)
    rec = fp8.record_bytes(head_dim)
    kcols = np.arange(head_dim, dtype=np.int64)
    vcols = np.arange(head_dim // 2, dtype=np.int64)
    for h in range(num_kv_heads):
        if is_aos:
            slot = fp8.slot_bytes(head_dim)
            base = b * stride + t * (num_kv_heads * slot) + h * slot
            _put_fp16(flat, base + rec, scale[sel, h])
            _put_fp16(flat, base + rec + 2, vmin[sel, h])
        else:
            base = b * stride + t * (num_kv_heads * rec) + h * rec
            meta = b * stride + block_size * num_kv_heads * rec
            fld = lambda f: meta + ((h * fp8.NUM_SOA_FIELDS + f) * block_size + t) * 2  # noqa: E731
            _put_fp16(flat, fld(fp8.SOA_V_SCALE), scale[sel, h])
            _put_fp16(flat, fld(fp8.SOA_V_ZERO), vmin[sel, h])
        flat[base[:, None] + kcols[None, :]] = kbytes[sel, h]
        flat[base[:, None] + head_dim + vcols[None, :]] = vbytes[sel, h]
    return cache
