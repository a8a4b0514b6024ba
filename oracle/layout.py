"""Byte layout of the 4-bit TurboQuant paged KV cache (oracle side).

Restates ``baseline/common.py:38-225`` (constants, SoA block layout) and the AoS
slot layout read by ``reference/aos_decode.py:140-152``, ``:213-221``, ``:282-299``.

Every physical block of the cache tensor ``uint8[num_blocks, bs, Hk, slot]`` is one
run of ``bs * Hk * slot`` bytes (``baseline/common.py:210-214``):

SoA (``baseline/common.py:158-214``)
    data region   ``[t][h][K codes (D/2 B) | V codes (D/2 B)]`` at ``t*Hk*D + h*D``
    meta region   at byte ``bs*Hk*D``: fp16 ``[h][field][t]``; field 0 = K norm
                  (norm-correction folded), 1 = V scale, 2 = V zero (per-token min)
AoS (``reference/aos_decode.py:140-152``)
    slot ``(t, h)`` at ``t*Hk*slot + h*slot``:
    ``[K codes D/2 | raw K norm fp16 | V codes D/2 | V scale fp16 | V zero fp16]``

Nibble order (``reference/soa_store.py:319-325``, ``:97-107``): byte ``j`` holds
dim ``2j`` in its low nibble and dim ``2j+1`` in its high nibble.

Parity: pinned by the reference's own layout asserts (``baseline/common.py:762-775``)
and by a write/read round trip through the independent store restatement.
"""
from __future__ import annotations

import numpy as np

NUM_SOA_FIELDS = 3
SOA_K_NORM, SOA_V_SCALE, SOA_V_ZERO = 0, 1, 2


def slot_bytes(head_dim: int) -> int:
    """K codes + V codes + three fp16 scalars, padded to even (``baseline/common.py:118-136``)."""
    raw = head_dim // 2 + head_dim // 2 + 3 * 2
    return raw + raw % 2


def block_bytes(block_size: int, num_kv_heads: int, head_dim: int) -> int:
    return block_size * num_kv_heads * slot_bytes(head_dim)


def soa_data_bytes(head_dim: int) -> int:
    return head_dim  # D/2 K bytes + D/2 V bytes


def soa_meta_offset(block_size: int, num_kv_heads: int, head_dim: int) -> int:
    return block_size * num_kv_heads * soa_data_bytes(head_dim)


def split_range(seq_len: int, num_splits: int, sid: int) -> tuple[int, int]:
    """Split partition of ``reference/soa_decode_v1.py:101-110``: ceil split length,
    end clipped to ``seq_len``; ``start >= end`` means the split is empty."""
    split_len = -(-seq_len // num_splits)
    start = split_len * sid
    end = min(start + split_len, seq_len)
    return start, end


def unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    """``uint8[..., n]`` -> ``int64[..., 2n]`` with the low nibble first."""
    p = packed.astype(np.int64)
    out = np.empty(p.shape[:-1] + (2 * p.shape[-1],), dtype=np.int64)
    out[..., 0::2] = p & 0xF
    out[..., 1::2] = (p >> 4) & 0xF
    return out


def _fp16_at(flat: np.ndarray, byte_offsets: np.ndarray) -> np.ndarray:
    lo = flat[byte_offsets].astype(np.uint16)
    hi = flat[byte_offsets + 1].astype(np.uint16)
    return (lo | (hi << 8)).view(np.float16).astype(np.float64)


def gather_soa(cache: np.ndarray, blocks: np.ndarray, offs: np.ndarray, kvh: int,
               block_size: int, num_kv_heads: int, head_dim: int):
    """Read K indices, folded K norm, V codes, V scale and V zero of tokens at
    (``blocks[i]``, ``offs[i]``) for kv-head ``kvh`` (``reference/soa_decode_v1.py:156-188``)."""
    flat = cache.reshape(-1)
    stride = block_bytes(block_size, num_kv_heads, head_dim)
    half = head_dim // 2
    base = blocks.astype(np.int64) * stride
    data = base + offs.astype(np.int64) * (num_kv_heads * head_dim) + kvh * head_dim
    cols = np.arange(half, dtype=np.int64)
    k_packed = flat[data[:, None] + cols[None, :]]
    v_packed = flat[data[:, None] + half + cols[None, :]]
    meta = base + soa_meta_offset(block_size, num_kv_heads, head_dim)

    def field(f):
        return _fp16_at(flat, meta + ((kvh * NUM_SOA_FIELDS + f) * block_size + offs) * 2)

    return (unpack_nibbles(k_packed), field(SOA_K_NORM), unpack_nibbles(v_packed),
            field(SOA_V_SCALE), field(SOA_V_ZERO))


def gather_aos(cache: np.ndarray, blocks: np.ndarray, offs: np.ndarray, kvh: int,
               block_size: int, num_kv_heads: int, head_dim: int):
    """Same fields from the AoS slot (``reference/aos_decode.py:140-152``, ``:213-221``,
    ``:282-299``); the K norm returned here is the raw ``||k||``."""
    flat = cache.reshape(-1)
    slot = slot_bytes(head_dim)
    stride = block_bytes(block_size, num_kv_heads, head_dim)
    half = head_dim // 2
    base = (blocks.astype(np.int64) * stride + offs.astype(np.int64) * (num_kv_heads * slot)
            + kvh * slot)
    cols = np.arange(half, dtype=np.int64)
    k_packed = flat[base[:, None] + cols[None, :]]
    v_packed = flat[base[:, None] + half + 2 + cols[None, :]]
    return (unpack_nibbles(k_packed), _fp16_at(flat, base + half), unpack_nibbles(v_packed),
            _fp16_at(flat, base + head_dim + 2), _fp16_at(flat, base + head_dim + 4))
