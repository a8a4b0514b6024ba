"""PyTorch (CPU, fp32) restatement of the reference's fp32 Stage1 math -- the reported CPU
baseline, and a second restatement the tests hold against the numpy oracle.  Test
infrastructure only, like the rest of ``oracle/``.

Follows ``tools/cuda_v1_diagnostic.py:106-224`` (``fp32_reference_one_split``), vectorized
over the kv-heads and splits of a sequence: the split partition ``L = ceil(len / S)``
(``reference/soa_decode_v1.py:101-110``); K/V bytes gathered through the block table (SoA
record ``(t, h)`` and ``[h][field][t]`` fp16 metadata, ``:156-188``; AoS 134-byte slots,
``reference/aos_decode.py:140-152``); nibbles unpacked low-first; ``K = c[idx] * n_t``
(AoS: ``c[idx] / sqrt(sum c^2 + 1e-16) * n_t``, ``reference/aos_decode.py:177-224``);
``V = code * scale + zero``; ``scores = Q K^T * D^-1/2``; per split ``softmax``,
``out = P V`` and ``lse = logsumexp(scores)``.  Empty splits stay NaN.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import layout


def stage1(q_rot, cache, block_table, seq_lens, centroids, num_splits, *, num_kv_heads,
           block_size=16, is_aos=False, attn_scale=None, sequences=None):
    """Return ``mid_o`` float32 ``[B, Hq, S, D+1]`` (rows of sequences not computed and of
    empty splits are NaN); ``sequences`` limits the work to those batch entries."""
    q = torch.as_tensor(np.asarray(q_rot, dtype=np.float32))
    batch, num_q_heads, head_dim = q.shape
    hk, group, half = num_kv_heads, num_q_heads // num_kv_heads, head_dim // 2
    scale = 1.0 / math.sqrt(head_dim) if attn_scale is None else attn_scale
    cache = np.ascontiguousarray(cache)
    flat = torch.from_numpy(cache.reshape(-1))
    flat16 = flat.view(torch.float16)
    stride = int(np.prod(cache.shape[1:]))
    cents = torch.as_tensor(np.asarray(centroids, dtype=np.float32))
    bt = torch.as_tensor(np.asarray(block_table)).long()
    heads = torch.arange(hk)
    cols = torch.arange(half)
    mid = torch.full((batch, num_q_heads, num_splits, head_dim + 1), float("nan"))
    for b in range(batch) if sequences is None else sequences:
        seq_len = int(seq_lens[b])
        if seq_len <= 0:
            continue
        split_len = -(-seq_len // num_splits)
        live = min(num_splits, -(-seq_len // split_len))
        tok = torch.arange(seq_len)
        blocks = bt[b, tok // block_size]
        offs = tok % block_size
        if is_aos:
            base = blocks[:, None] * stride + (offs[:, None] * hk + heads[None, :]) * layout.slot_bytes(head_dim)
            kb = base[..., None] + cols
            vb = base[..., None] + half + 2 + cols
            norm = flat16[(base + half) // 2].float()
            vscale = flat16[(base + head_dim + 2) // 2].float()
            vzero = flat16[(base + head_dim + 4) // 2].float()
        else:
            base = blocks[:, None] * stride + (offs[:, None] * hk + heads[None, :]) * head_dim
            kb = base[..., None] + cols
            vb = kb + half
            meta = (blocks[:, None] * stride + block_size * hk * head_dim
                    + (heads[None, :] * 3 * block_size + offs[:, None]) * 2)
            norm = flat16[meta // 2].float()
            vscale = flat16[(meta + 2 * block_size) // 2].float()
            vzero = flat16[(meta + 4 * block_size) // 2].float()
        kp, vp = flat[kb].long(), flat[vb].long()
        k_idx = torch.stack([kp & 15, kp >> 4], dim=-1).reshape(seq_len, hk, head_dim)
        v_code = torch.stack([vp & 15, vp >> 4], dim=-1).reshape(seq_len, hk, head_dim).float()
        cv = cents[k_idx]
        if is_aos:
            cv = cv / torch.sqrt((cv * cv).sum(-1, keepdim=True) + 1e-16)
        k = cv * norm[..., None]                               # [T, Hk, D]
        v = v_code * vscale[..., None] + vzero[..., None]      # [T, Hk, D]
        qb = q[b].view(hk, group, head_dim)
        s = torch.bmm(qb, k.permute(1, 2, 0).contiguous()) * scale   # [Hk, G, T]
        padded = live * split_len
        sp = torch.full((hk, group, padded), float("-inf"))
        sp[..., :seq_len] = s
        sp = sp.view(hk, group, live, split_len)
        m = sp.amax(-1, keepdim=True)
        p = torch.exp(sp - m)
        den = p.sum(-1, keepdim=True)
        vpad = torch.zeros(hk, padded, head_dim)
        vpad[:, :seq_len] = v.permute(1, 0, 2)
        vpad = vpad.view(hk, live, split_len, head_dim)
        out = torch.matmul(p.permute(0, 2, 1, 3), vpad)         # [Hk, live, G, D]
        out = out / den.permute(0, 2, 1, 3)
        lse = (m + torch.log(den))[..., 0]                        # [Hk, G, live]
        mid[b, :, :live, :head_dim] = out.permute(0, 2, 1, 3).reshape(num_q_heads, live, head_dim)
        mid[b, :, :live, head_dim] = lse.reshape(num_q_heads, live)
    return mid.numpy()
