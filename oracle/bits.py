"""The 3-bit presets (``turboquant_k3v4_nc``: 3-bit K / 4-bit V, ``turboquant_3bit_nc``: 3-bit
K / 3-bit V, ``reference/config.py:30-39``) next to the 4-bit one: bit packing, layout,
gather, writer.  Test infrastructure only.

* Packing (``reference/soa_store.py:319-337`` K, ``:47-83`` V, decode
  ``reference/soa_decode_v1.py:122-132``, ``:271-284``): code ``d`` occupies bits
  ``[b*d, b*d + b)`` of the row's byte string, least significant bit first (4 bits: the low
  nibble is the even dim; 3 bits: eight codes per 24-bit group).
* Layout (``reference/config.py:128-164``): K bytes ``D*kb/8``, V bytes ``D*vb/8``; AoS slot
  ``[K codes | K norm fp16 | V codes | V scale fp16 | V zero fp16]`` padded to even; SoA
  record ``K codes | V codes`` and three fp16 metadata fields ``[h][field][t]`` (K norm,
  V scale, V zero) after the data region.
* V: ``scale = max((max - min) / (2^vb - 1), 1e-8)``, code ``clamp(int((v - min) / scale +
  0.5), 0, 2^vb - 1)``; K: count of the ``2^kb - 1`` midpoints ``<= y``, folded norm with
  norm correction (SoA), raw norm (AoS) -- as the 4-bit writer.

Pinned by: the 4-bit case against the 4-bit oracle (same bytes), a brute-force bit-string
unpack, the write/read round trip, and Stage1 over this layout against torch attention.
"""
from __future__ import annotations

import numpy as np

from .layout import _fp16_at


def key_bytes(d: int, kb: int) -> int:
    return d * kb // 8


def value_bytes(d: int, vb: int) -> int:
    return d * vb // 8


def slot_bytes(d: int, kb: int, vb: int) -> int:
    raw = key_bytes(d, kb) + 2 + value_bytes(d, vb) + 4
    return raw + raw % 2


def record_bytes(d: int, kb: int, vb: int) -> int:
    return key_bytes(d, kb) + value_bytes(d, vb)


def pack(codes, bits: int) -> np.ndarray:
    """``int[..., D]`` -> ``uint8[..., D*bits/8]``, code d at bits ``[bits*d, bits*d+bits)``."""
    c = np.asarray(codes, dtype=np.int64) & ((1 << bits) - 1)
    d = c.shape[-1]
    bitpos = np.arange(d) * bits
    out = np.zeros(c.shape[:-1] + (d * bits // 8,), dtype=np.int64)
    for j in range(bits):  # bit j of every code goes to stream position bits*d + j
        pos = bitpos + j
        bit = (c >> j) & 1
        for p in range(d):
            out[..., pos[p] // 8] |= bit[..., p] << (pos[p] % 8)
    return out.astype(np.uint8)


def unpack(packed, bits: int, d: int) -> np.ndarray:
    p = np.asarray(packed, dtype=np.int64)
    out = np.zeros(p.shape[:-1] + (d,), dtype=np.int64)
    for j in range(bits):
        pos = np.arange(d) * bits + j
        out |= ((p[..., pos // 8] >> (pos % 8)) & 1) << j
    return out


def gather(cache, blocks, offs, kvh, block_size, num_kv_heads, d, kb, vb, is_aos):
    """``(k_idx, k_norm, v_code, v_scale, v_zero)`` of tokens (blocks[i], offs[i])."""
    flat = cache.reshape(-1)
    kbytes, vbytes = key_bytes(d, kb), value_bytes(d, vb)
    slot = slot_bytes(d, kb, vb)
    stride = block_size * num_kv_heads * slot
    blocks = np.asarray(blocks, dtype=np.int64)
    offs = np.asarray(offs, dtype=np.int64)
    kc, vc = np.arange(kbytes), np.arange(vbytes)
    if is_aos:
        base = blocks * stride + offs * (num_kv_heads * slot) + kvh * slot
        kp = flat[base[:, None] + kc]
        vp = flat[base[:, None] + kbytes + 2 + vc]
        norm = _fp16_at(flat, base + kbytes)
        vs, vz = _fp16_at(flat, base + kbytes + 2 + vbytes), _fp16_at(flat, base + kbytes + 4 + vbytes)
    else:
        rec = record_bytes(d, kb, vb)
        base = blocks * stride + offs * (num_kv_heads * rec) + kvh * rec
        kp = flat[base[:, None] + kc]
        vp = flat[base[:, None] + kbytes + vc]
        meta = blocks * stride + block_size * num_kv_heads * rec
        fld = lambda f: meta + ((kvh * 3 + f) * block_size + offs) * 2  # noqa: E731
        norm, vs, vz = _fp16_at(flat, fld(0)), _fp16_at(flat, fld(1)), _fp16_at(flat, fld(2))
    return unpack(kp, kb, d), norm, unpack(vp, vb, d), vs, vz


def quantize_values(value, vb: int):
    v = np.asarray(value, dtype=np.float32)
    top = np.float32((1 << vb) - 1)
    vmin = v.min(axis=-1)
    scale = (v.max(axis=-1) - vmin) / top
    scale = np.where(scale > np.float32(1e-8), scale, np.float32(1e-8)).astype(np.float32)
    codes = ((v - vmin[..., None]) / scale[..., None] + np.float32(0.5)).astype(np.int32)
    return np.clip(codes, 0, int(top)).astype(np.int64), scale, vmin


def store(key, value, slot_mapping, rot_t, cents, cache, kb, vb, *, block_size=16, is_aos=False):
    """Writer of the ``kb``-bit K / ``vb``-bit V preset (norm correction: folded norm in SoA)."""
    from .store import _put_fp16, quantize_keys

    n_tok, hk, d = np.asarray(key).shape
    flat = cache.reshape(-1)
    idx, norm, folded = quantize_keys(key, rot_t, cents)
    codes, scale, vmin = quantize_values(value, vb)
    kp, vp = pack(idx, kb), pack(codes, vb)
    kbytes, vbytes = key_bytes(d, kb), value_bytes(d, vb)
    slot = slot_bytes(d, kb, vb)
    stride = block_size * hk * slot
    slots = np.asarray(slot_mapping, dtype=np.int64)
    sel = np.nonzero(slots >= 0)[0]
    b, t = slots[sel] // block_size, slots[sel] % block_size
    kc, vc = np.arange(kbytes), np.arange(vbytes)
    for h in range(hk):
        if is_aos:
            base = b * stride + t * (hk * slot) + h * slot
            flat[base[:, None] + kc] = kp[sel, h]
            _put_fp16(flat, base + kbytes, norm[sel, h])
            flat[base[:, None] + kbytes + 2 + vc] = vp[sel, h]
            _put_fp16(flat, base + kbytes + 2 + vbytes, scale[sel, h])
            _put_fp16(flat, base + kbytes + 4 + vbytes, vmin[sel, h])
        else:
            rec = record_bytes(d, kb, vb)
            base = b * stride + t * (hk * rec) + h * rec
            flat[base[:, None] + kc] = kp[sel, h]
            flat[base[:, None] + kbytes + vc] = vp[sel, h]
            meta = b * stride + block_size * hk * rec
            fld = lambda f: meta + ((h * 3 + f) * block_size + t) * 2  # noqa: E731
            _put_fp16(flat, fld(0), folded[sel, h])
            _put_fp16(flat, fld(1), scale[sel, h])
            _put_fp16(flat, fld(2), vmin[sel, h])
    return cache
