"""FP8 (OCP E4M3, the "fn" variant: no infinities, NaN = S.1111.111) codec of the FP8-key
preset (``turboquant_k8v4``, ``reference/config.py:20-24``).  Test infrastructure only.

* ``encode``: the store's cast ``k.to(tl.float8e4nv)`` (``reference/soa_store.py:192-193``),
  which on the reference's GPUs rounds to nearest even and saturates to +-448
  ("satfinite"): clamp, then torch's round-to-nearest-even ``float8_e4m3fn`` cast (a
  library routine).  The exact out-of-range behaviour of Triton's cast is parity unpinned
  beyond that (values are clamped here; NaN stays NaN).
* ``decode``: byte -> value by the E4M3 definition (bias 7, 3 mantissa bits, subnormals
  at exponent 0); pinned against torch's ``float8_e4m3fn`` for all 256 bytes.

Layout of the preset (``reference/soa_store.py:391-439``, ``reference/config.py:128-164``):
key_packed_size = D (one byte per dim), value_packed_size = D/2 + 4; AoS slot
``[K fp8 (D) | V codes (D/2) | V scale fp16 | V zero fp16]`` (196 bytes at D = 128); SoA
record ``(t, h)`` = D + D/2 bytes of K then V, metadata fp16 ``[h][field][t]`` with two
fields (0 = V scale, 1 = V zero) after the data region.
"""
from __future__ import annotations

import numpy as np
import torch

E4M3_MAX = 448.0


def decode_table() -> np.ndarray:
    """float64 value of every byte 0..255 (NaN for 0x7F and 0xFF)."""
    b = np.arange(256)
    sign = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 7
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * 2.0 ** (e - 7.0))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return sign * mag


def decode(codes) -> np.ndarray:
    return decode_table()[np.asarray(codes, dtype=np.int64)]


def encode(x) -> np.ndarray:
    """float -> uint8 E4M3 bytes: clamp to +-448, round to nearest even."""
    v = np.asarray(x, dtype=np.float32)
    v = np.where(np.isnan(v), v, np.clip(v, -E4M3_MAX, E4M3_MAX)).astype(np.float32)
    return torch.from_numpy(np.ascontiguousarray(v)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


# ---- preset layout ------------------------------------------------------------------

NUM_SOA_FIELDS = 2
SOA_V_SCALE, SOA_V_ZERO = 0, 1


def slot_bytes(head_dim: int) -> int:
    raw = head_dim + head_dim // 2 + 4
    return raw + raw % 2


def record_bytes(head_dim: int) -> int:
    return head_dim + head_dim // 2


def block_bytes(block_size: int, num_kv_heads: int, head_dim: int) -> int:
    return block_size * num_kv_heads * slot_bytes(head_dim)


def gather(cache, blocks, offs, kvh, block_size, num_kv_heads, head_dim, is_aos):
    """Return ``(k_bytes uint8 [T, D], v_code [T, D], v_scale [T], v_zero [T])``."""
    from .layout import _fp16_at, unpack_nibbles

    flat = cache.reshape(-1)
    stride = block_bytes(block_size, num_kv_heads, head_dim)
    blocks = np.asarray(blocks, dtype=np.int64)
    offs = np.asarray(offs, dtype=np.int64)
    kcols = np.arange(head_dim, dtype=np.int64)
    vcols = np.arange(head_dim // 2, dtype=np.int64)
    if is_aos:
        slot = slot_bytes(head_dim)
        base = blocks * stride + offs * (num_kv_heads * slot) + kvh * slot
        vs, vz = _fp16_at(flat, base + record_bytes(head_dim)), _fp16_at(flat, base + record_bytes(head_dim) + 2)
    else:
        rec = record_bytes(head_dim)
        base = blocks * stride + offs * (num_kv_heads * rec) + kvh * rec
        meta = blocks * stride + block_size * num_kv_heads * rec
        fld = lambda f: meta + ((kvh * NUM_SOA_FIELDS + f) * block_size + offs) * 2  # noqa: E731
        vs, vz = _fp16_at(flat, fld(SOA_V_SCALE)), _fp16_at(flat, fld(SOA_V_ZERO))
    kb = flat[base[:, None] + kcols[None, :]]
    vb = flat[base[:, None] + head_dim + vcols[None, :]]
    return kb, unpack_nibbles(vb), vs, vz
