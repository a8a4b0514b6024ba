"""numpy float64 restatement of the decode Stage1 / Stage2 / full step.

``stage1`` follows the per-program algorithm of the reference Stage1 oracle kernels:

* split partition and empty-split early return: ``reference/soa_decode_v1.py:101-110``
* paged addressing and field reads: SoA ``:156-188``, AoS ``reference/aos_decode.py:140-152``
* K decode: SoA ``c[idx] * n_t`` (``reference/soa_decode_v1.py:213-254``); AoS with the
  norm correction ``c[idx] / sqrt(sum c^2 + 1e-16) * raw_n_t`` (``reference/aos_decode.py:177-224``)
* score ``n_t * (q . c) * attn_scale``; GQA head ``h`` reads kv-head ``h // G`` (``:99``)
* V decode ``code * scale + zero`` (``reference/soa_decode_v1.py:285-300``)
* softmax over the split, ``mid_o[..., :D] = sum p v / l`` and ``mid_o[..., D] = m + ln l``
  with ``l`` guarded to 1 when not positive (``reference/soa_decode_v1.py:259-314``).

The reference evaluates the softmax online in fp32 (BLOCK_KV-token steps); here it is
evaluated in one shot in float64, which is the exact value those steps approximate.
Splits with ``start >= end`` are left untouched in ``mid_o``.

``stage2`` restates ``baseline/stage2.py:26-55``: merge only the non-empty splits
(recomputed from ``seq_lens``), ``M = max lse``, ``w = exp(lse - M)``,
``out = sum w o / sum w``, ``lse = M + ln sum w``.

``full_decode`` adds the query rotation ``q_rot = query.float() @ PiT``
(``reference/soa_decode_v1.py:532-538``) and the pair-LUT build in front, and casts
the output to the requested dtype (``reference/soa_decode_v1.py:643``).

Parity: pinned against torch's scaled_dot_product_attention / logsumexp on the
decoded K and V (a library routine), against the C restatement ``tq4_oracle.c``,
by the invariant Stage2(Stage1(splits)) == attention over the whole sequence, and
by invariance of that result to the split count.
"""
from __future__ import annotations

import math

import numpy as np

from . import layout

LOG2E = 1.4426950408889634


def decode_kv(cache, blocks, offs, kvh, centroids, is_aos, block_size, num_kv_heads, head_dim):
    """Return float64 ``(K [T, D], V [T, D])`` for the given tokens of one kv-head."""
    c = np.asarray(centroids, dtype=np.float64)
    gather = layout.gather_aos if is_aos else layout.gather_soa
    k_idx, k_norm, v_code, v_scale, v_zero = gather(cache, blocks, offs, kvh,
                                                    block_size, num_kv_heads, head_dim)
    cv = c[k_idx]
    if is_aos:
        cv = cv / np.sqrt((cv * cv).sum(axis=1, keepdims=True) + 1e-16)
    k = cv * k_norm[:, None]
    v = v_code.astype(np.float64) * v_scale[:, None] + v_zero[:, None]
    return k, v


def decode_kv_bits(cache, blocks, offs, kvh, centroids, is_aos, block_size, num_kv_heads, head_dim,
                   key_bits, value_bits):
    """The ``key_bits`` / ``value_bits`` presets (``reference/soa_decode_v1.py:122-132``,
    ``:271-284``): float64 ``(K, V)``, K = c[idx] * stored norm (AoS: c[idx] renormalised,
    ``reference/aos_decode.py:197-205``)."""
    from . import bits

    c = np.asarray(centroids, dtype=np.float64)
    k_idx, k_norm, v_code, v_scale, v_zero = bits.gather(cache, blocks, offs, kvh, block_size,
                                                         num_kv_heads, head_dim, key_bits,
                                                         value_bits, is_aos)
    cv = c[k_idx]
    if is_aos:
        cv = cv / np.sqrt((cv * cv).sum(axis=1, keepdims=True) + 1e-16)
    return cv * k_norm[:, None], v_code.astype(np.float64) * v_scale[:, None] + v_zero[:, None]


def decode_kv_fp8(cache, blocks, offs, kvh, is_aos, block_size, num_kv_heads, head_dim):
    """FP8-key preset: float64 ``(K [T, D], V [T, D])``; K is the E4M3 value of each byte
    (``reference/soa_decode_v1.py:213-230`` with KEY_FP8), no norm."""
    from . import fp8

    kb, v_code, v_scale, v_zero = fp8.gather(cache, blocks, offs, kvh, block_size, num_kv_heads,
                                            head_dim, is_aos)
    return fp8.decode(kb), v_code.astype(np.float64) * v_scale[:, None] + v_zero[:, None]


def stage1(q_rot, cache, block_table, seq_lens, centroids, num_splits, *, num_kv_heads,
           block_size=16, is_aos=False, attn_scale=None, mid_o=None, sinks=None, key_fp8=False,
           bits=None):
    """Return ``mid_o`` float64 ``[B, Hq, S, D+1]``; empty splits keep their prior value
    (NaN when ``mid_o`` is not given).  ``sinks`` ``[Hq]``: split 0 of every sequence starts
    its softmax with max = sink and sum = 1, an extra logit with a zero value
    (``reference/soa_decode_v1.py:134-148``).  ``key_fp8``: the FP8-key preset; ``q_rot``
    is then the unrotated query and ``centroids`` is unused.  ``bits`` ``(key_bits,
    value_bits)``: the bit-width preset layout of ``oracle.bits`` (``centroids`` has
    ``2^key_bits`` entries)."""
    q = np.asarray(q_rot, dtype=np.float64)
    batch, num_q_heads, head_dim = q.shape
    group = num_q_heads // num_kv_heads
    scale = 1.0 / math.sqrt(head_dim) if attn_scale is None else attn_scale
    if mid_o is None:
        mid_o = np.full((batch, num_q_heads, num_splits, head_dim + 1), np.nan)
    bt = np.asarray(block_table)
    for b in range(batch):
        seq_len = int(seq_lens[b])
        for sid in range(num_splits):
            start, end = layout.split_range(seq_len, num_splits, sid)
            if start >= end:
                continue
            tok = np.arange(start, end)
            blocks = bt[b, tok // block_size]
            offs = tok % block_size
            for kvh in range(num_kv_heads):
                if key_fp8:
                    k, v = decode_kv_fp8(cache, blocks, offs, kvh, is_aos, block_size,
                                         num_kv_heads, head_dim)
                elif bits is not None:
                    k, v = decode_kv_bits(cache, blocks, offs, kvh, centroids, is_aos, block_size,
                                          num_kv_heads, head_dim, *bits)
                else:
                    k, v = decode_kv(cache, blocks, offs, kvh, centroids, is_aos,
                                     block_size, num_kv_heads, head_dim)
                heads = slice(kvh * group, (kvh + 1) * group)
                s = (q[b, heads] @ k.T) * scale
                m = s.max(axis=1, keepdims=True)
                sink = None
                if sinks is not None and sid == 0:
                    sink = np.asarray(sinks, dtype=np.float64)[heads][:, None]
                    m = np.maximum(m, sink)
                p = np.exp(s - m)
                denom = p.sum(axis=1, keepdims=True)
                if sink is not None:
                    denom = denom + np.exp(sink - m)
                denom = np.where(denom > 0, denom, 1.0)
                mid_o[b, heads, sid, :head_dim] = (p @ v) / denom
                mid_o[b, heads, sid, head_dim] = (m + np.log(denom))[:, 0]
    return mid_o


def stage2(mid_o, seq_lens):
    """Return ``(out [B, Hq, D], lse [B, Hq])`` float64."""
    mid = np.asarray(mid_o, dtype=np.float64)
    batch, num_q_heads, num_splits, d1 = mid.shape
    out = np.zeros((batch, num_q_heads, d1 - 1))
    lse = np.zeros((batch, num_q_heads))
    for b in range(batch):
        ranges = [layout.split_range(int(seq_lens[b]), num_splits, sid) for sid in range(num_splits)]
        live = [sid for sid, (start, end) in enumerate(ranges) if start < end]
        part = mid[b][:, live, :]
        m = part[:, :, -1].max(axis=1, keepdims=True)
        w = np.exp(part[:, :, -1] - m)
        tot = w.sum(axis=1)
        out[b] = (w[:, :, None] * part[:, :, :-1]).sum(axis=1) / tot[:, None]
        lse[b] = m[:, 0] + np.log(tot)
    return out, lse


def attention_reference(q_rot, cache, block_table, seq_lens, centroids, *, num_kv_heads,
                        block_size=16, is_aos=False, attn_scale=None):
    """Unsplit softmax attention over the whole sequence, float64 ``(out, lse)``."""
    q = np.asarray(q_rot, dtype=np.float64)
    batch, num_q_heads, head_dim = q.shape
    group = num_q_heads // num_kv_heads
    scale = 1.0 / math.sqrt(head_dim) if attn_scale is None else attn_scale
    out = np.zeros((batch, num_q_heads, head_dim))
    lse = np.zeros((batch, num_q_heads))
    for b in range(batch):
        tok = np.arange(int(seq_lens[b]))
        blocks = np.asarray(block_table)[b, tok // block_size]
        offs = tok % block_size
        for kvh in range(num_kv_heads):
            k, v = decode_kv(cache, blocks, offs, kvh, centroids, is_aos, block_size,
                             num_kv_heads, head_dim)
            heads = slice(kvh * group, (kvh + 1) * group)
            s = (q[b, heads] @ k.T) * scale
            m = s.max(axis=1, keepdims=True)
            p = np.exp(s - m)
            out[b, heads] = (p @ v) / p.sum(axis=1, keepdims=True)
            lse[b, heads] = (m + np.log(p.sum(axis=1, keepdims=True)))[:, 0]
    return out, lse


def rotate_query(query, rot_t):
    """``q_rot = query.float() @ PiT`` (``reference/soa_decode_v1.py:532-538``), float64."""
    return np.asarray(query, dtype=np.float64) @ np.asarray(rot_t, dtype=np.float64)


def full_decode(query, rot_t, cache, block_table, seq_lens, centroids, num_splits, *,
                num_kv_heads, block_size=16, is_aos=False):
    """Rotation + Stage1 + Stage2, float64 ``(out, lse, mid_o)``."""
    q_rot = rotate_query(query, rot_t)
    mid = stage1(q_rot, cache, block_table, seq_lens, centroids, num_splits,
                 num_kv_heads=num_kv_heads, block_size=block_size, is_aos=is_aos)
    out, lse = stage2(mid, seq_lens)
    return out, lse, mid
