"""Cache-layout constants of the ``turboquant_4bit_nc`` paged KV cache.

Mirrors the data contract of ``baseline/common.py:38-225`` (SoA) and the AoS slot of
``reference/aos_decode.py:140-152``.  One physical block is ``bs * Hk * slot`` bytes;
``slot = D/2 (K codes) + D/2 (V codes) + 3 fp16 scalars`` (134 B at D=128).

SoA block: data region ``[token][kv_head][K codes | V codes]`` (``D`` bytes per
token-head), then fp16 metadata ``[kv_head][field][token]`` at byte ``bs * Hk * D``
(field 0 folded K norm, 1 V scale, 2 V zero).

AoS slot ``(token, kv_head)`` at ``token*Hk*slot + kv_head*slot``:
``[K codes | raw K norm | V codes | V scale | V zero]``.
"""
from __future__ import annotations

SOA = 0
AOS = 1
# AoS with head-major blocks [Hk][bs][slot]: slot (t, h) at (h * bs + t) * slot.  The vLLM
# backend allocates its cache [blocks, Hk, bs, slot] and hands the kernels
# ``kv_cache.transpose(1, 2)`` (reference/turboquant_attn.py:536, :565); the host layer
# picks this id from that view's strides.
AOS_HEAD_MAJOR = 2
LAYOUTS = {"soa": SOA, "aos": AOS}

NUM_SOA_FIELDS = 3
SOA_K_NORM = 0
SOA_V_SCALE = 1
SOA_V_ZERO = 2

MSE_BITS = 4
VALUE_BITS = 4


def slot_bytes(head_dim: int) -> int:
    raw = head_dim + 3 * 2
    return raw + raw % 2


def slot_bytes_preset(head_dim: int, key_bits: int, value_bits: int) -> int:
    """Slot of the ``key_bits`` / ``value_bits`` presets (``reference/config.py:128-164``):
    K codes + fp16 norm + V codes + fp16 scale + fp16 zero, rounded up to even (3/4: 118,
    3/3: 102, 4/4: 134 at D = 128)."""
    raw = head_dim * key_bits // 8 + 2 + head_dim * value_bits // 8 + 4
    return raw + raw % 2


def slot_bytes_fp8(head_dim: int) -> int:
    """FP8-key preset slot: one E4M3 byte per K dim + V codes + fp16 V scale and zero
    (``reference/config.py:128-164``)."""
    raw = head_dim + head_dim // 2 + 4
    return raw + raw % 2


def block_bytes(block_size: int, num_kv_heads: int, head_dim: int) -> int:
    return block_size * num_kv_heads * slot_bytes(head_dim)


def meta_offset(block_size: int, num_kv_heads: int, head_dim: int) -> int:
    return block_size * num_kv_heads * head_dim


def split_bounds(seq_len: int, num_splits: int, sid: int) -> tuple[int, int]:
    """``split_len = ceil(seq_len / S)``; split ``sid`` covers ``[sid*len, min(+len, seq_len))``."""
    split_len = (seq_len + num_splits - 1) // num_splits
    start = sid * split_len
    return start, min(start + split_len, seq_len)
