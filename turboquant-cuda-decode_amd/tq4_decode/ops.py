"""Torch-facing launchers over the C ABI, with the reference harness's call shapes.

Every launcher validates its tensors with the reference's messages
(``cuda/tq4_cuda_v1.cu:468-499``), then calls the HIP library on torch's current
stream of the tensors' device.  Nothing here computes on the host: when the
library is missing, ``_lib.load`` raises.

Reference call shapes kept here:

* ``launch_tq4_v2_stage1(q_rot, kv_cache, block_table, seq_lens, centroids, pair_lut, mid_o=None)``
  -- ``baseline/triton_v2.py:569-706`` (SoA; allocates ``mid_o`` when None)
* ``launch_soa_v1_stage1`` / ``launch_aos_v1_stage1(q_rot, kv_cache, block_table, seq_lens,
  centroids, mid_o)`` -- ``baseline/triton_v1.py:90-203``
* ``launch_stage2(mid_o, seq_lens, output, lse)`` -- ``baseline/stage2.py:58-81``
* ``triton_turboquant_store(key, value, kv_cache, slot_mapping, PiT, midpoints, mse_bits,
  key_packed_size, value_quant_bits, key_fp8=False, centroids=None, norm_correction=False)``
  -- ``reference/soa_store.py:381-524`` (4-bit, 3-bit-key and 3-bit presets, FP8 keys)
* ``ext`` -- object with the CUDA-extension names ``tq4_cuda_v1 .. tq4_cuda_v9``,
  ``tq4_cuda_v7_stage1 / _stage2 / _full`` (``cuda/tq4_cuda_v7_bind.cpp:3-20``), so
  ``cuda_ext = tq4_decode.ext`` drops into ``benchmarks/stage1.py`` / ``full_decode.py``.
"""
from __future__ import annotations

import math

import torch

from . import _lib
from ._lib import Tq4Error  # noqa: F401  (raised by every wrapper)
from .layout import AOS, AOS_HEAD_MAJOR, LAYOUTS, SOA, slot_bytes, slot_bytes_fp8, slot_bytes_preset

KERNELS = {"auto": 0, "simple": 1, "xdl": 3}
DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
HEAD_DIM = 128


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _check_tensor(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    _require(t.is_cuda, f"{name} must be CUDA")
    _require(t.dtype == dtype, f"{name} must be {str(dtype).replace('torch.', '')}")
    _require(t.is_contiguous(), f"{name} must be contiguous")


def _layout_id(layout) -> int:
    if isinstance(layout, str):
        _require(layout in LAYOUTS, f"layout must be one of {sorted(LAYOUTS)}")
        return LAYOUTS[layout]
    _require(layout in (SOA, AOS), "layout must be 0 (SoA) or 1 (AoS)")
    return int(layout)


def _cache_geometry(kv_cache: torch.Tensor, slot_want: int, layout, preset: str = ""):
    """``(block_size, Hk, block stride, ABI layout id)`` of a cache tensor or view.

    Takes the contiguous ``[blocks, block_size, Hk, slot]`` cache and the view the vLLM
    backend passes, ``kv_cache.transpose(1, 2)`` of its ``[blocks, Hk, block_size, slot]``
    allocation (``reference/turboquant_attn.py:536``, ``:565``).  SoA blocks are addressed
    by their own layout, so only the block stride is read (as ``reference/soa_decode_v1.py:579``
    and ``reference/soa_store.py:424`` do); AoS slots follow the view's position and head
    strides (``reference/aos_decode.py:563-565``, ``reference/aos_store.py:375-377``), which
    must describe a position-major or a head-major block.
    """
    _require(kv_cache.is_cuda, "kv_cache must be CUDA")
    _require(kv_cache.dtype == torch.uint8, "kv_cache must be uint8")
    _require(kv_cache.dim() == 4, "kv_cache must be [blocks, block_size, Hk, slot]")
    return block_geometry(tuple(kv_cache.shape), kv_cache.stride(), slot_want, layout, preset)


def block_geometry(shape, strides, slot_want: int, layout, preset: str = ""):
    """The stride rules of ``_cache_geometry`` for a 4-D uint8 ``shape`` / ``strides``."""
    nb, bs, hk, slot = shape
    _require(slot == slot_want, f"requires slot_size={slot_want}{preset}")
    s0, s1, s2, s3 = strides

    def same(size, got, want):  # a dimension of size 1 has no meaningful stride
        return size == 1 or got == want

    _require(same(slot, s3, 1), "kv_cache: the slot bytes must be contiguous (stride(3) == 1)")
    position_major = same(bs, s1, hk * slot) and same(hk, s2, slot)
    head_major = same(bs, s1, slot) and same(hk, s2, bs * slot)
    _require(position_major or head_major,
             "kv_cache: each block must be a contiguous [block_size, Hk, slot] block or the "
             "transpose(1, 2) view of a contiguous [Hk, block_size, slot] block")
    block = bs * hk * slot
    stride = s0 if nb > 1 else max(s0, block)
    _require(stride >= block, "kv_cache: block stride is smaller than a block")
    lid = _layout_id(layout)
    if lid == AOS and not position_major:
        lid = AOS_HEAD_MAJOR
    return bs, hk, stride, lid


def pair_lut_device(centroids: torch.Tensor) -> torch.Tensor:
    """Pair LUT ``[n*n, 2]`` built on the centroids' device (``baseline/common.py:232-257``)."""
    _check_tensor(centroids, "centroids", torch.float32)
    _require(centroids.numel() == 16, "4-bit path requires 16 centroids")
    lut = torch.empty(256, 2, dtype=torch.float32, device=centroids.device)
    _lib.check(_lib.load().tq4_build_pair_lut(centroids.data_ptr(), lut.data_ptr(), 16,
                                              _stream(centroids.device)), "tq4_build_pair_lut")
    return lut


def _check_sinks(sinks, num_q_heads, device):
    if sinks is None:
        return None
    _check_tensor(sinks, "sinks", torch.float32)
    _require(sinks.numel() == num_q_heads and sinks.device == device, "sinks must be fp32 [Hq]")
    return sinks.data_ptr()


def stage1(q_rot, kv_cache, block_table, seq_lens, pair_lut, mid_o=None, *, num_kv_splits=None,
           layout="soa", attn_scale=None, kernel="auto", sinks=None):
    """Stage1 over the 4-bit paged cache; returns ``mid_o [B, Hq, S, D+1]`` (fp32).

    ``S`` comes from ``mid_o`` when given, else from ``num_kv_splits``.  Empty splits
    leave their ``mid_o`` rows untouched.  ``sinks`` (fp32 ``[Hq]``): per-head sink logits
    that split 0's softmax starts from (``reference/soa_decode_v1.py:134-148``).
    """
    for t, n, dt in ((q_rot, "q_rot", torch.float32), (block_table, "block_table", torch.int32),
                     (seq_lens, "seq_lens", torch.int32), (pair_lut, "pair_lut", torch.float32)):
        _check_tensor(t, n, dt)
    _require(q_rot.dim() == 3, "q_rot must be [B, Hq, D]")
    B, Hq, D = q_rot.shape
    _require(D == HEAD_DIM, f"requires D={HEAD_DIM}")
    bs, Hk, stride, lid = _cache_geometry(kv_cache, slot_bytes(D), layout)
    _require(Hq % Hk == 0, "Hq must be a multiple of Hk")
    _require(block_table.dim() == 2 and block_table.size(0) == B, "block_table batch mismatch")
    _require(seq_lens.dim() == 1 and seq_lens.size(0) == B, "seq_lens batch mismatch")
    _require(tuple(pair_lut.shape) == (256, 2), "pair_lut must be [256, 2]")
    if mid_o is None:
        _require(num_kv_splits is not None and num_kv_splits > 0,
                 "num_kv_splits is required when mid_o is None")
        mid_o = torch.empty(B, Hq, num_kv_splits, D + 1, dtype=torch.float32, device=q_rot.device)
    _check_tensor(mid_o, "mid_o", torch.float32)
    S = mid_o.size(2)
    _require(mid_o.dim() == 4 and tuple(mid_o.shape) == (B, Hq, S, D + 1),
             f"mid_o must be [B,{Hq},S,{D + 1}]")
    _require(num_kv_splits is None or num_kv_splits == S, "mid_o split count mismatch")
    devs = {t.device for t in (q_rot, kv_cache, block_table, seq_lens, pair_lut, mid_o)}
    _require(len(devs) == 1, "all tensors must be on the same device")
    scale = 1.0 / math.sqrt(D) if attn_scale is None else float(attn_scale)
    _require(kernel in KERNELS, f"kernel must be one of {sorted(KERNELS)}")
    sinks_ptr = _check_sinks(sinks, Hq, q_rot.device)
    rc = _lib.load().tq4_stage1_ex(
        q_rot.data_ptr(), kv_cache.data_ptr(), block_table.data_ptr(), seq_lens.data_ptr(),
        pair_lut.data_ptr(), mid_o.data_ptr(), B, Hq, Hk, D, bs, block_table.size(1),
        stride, S, lid, scale, KERNELS[kernel], sinks_ptr, _stream(q_rot.device))
    _lib.check(rc, "tq4_stage1")
    return mid_o


def stage2(mid_o, seq_lens, out=None, lse=None, out_dtype=torch.float32):
    """Merge the non-empty splits; returns ``(out [B, Hq, D], lse [B, Hq])``."""
    _check_tensor(mid_o, "mid_o", torch.float32)
    _check_tensor(seq_lens, "seq_lens", torch.int32)
    _require(mid_o.dim() == 4 and mid_o.size(3) == HEAD_DIM + 1, "invalid mid_o shape")
    B, Hq, S, _ = mid_o.shape
    if out is None:
        out = torch.empty(B, Hq, HEAD_DIM, dtype=out_dtype, device=mid_o.device)
    if lse is None:
        lse = torch.empty(B, Hq, dtype=torch.float32, device=mid_o.device)
    _require(out.is_cuda and out.is_contiguous() and out.dtype in DTYPES, "invalid output")
    _require(tuple(out.shape) == (B, Hq, HEAD_DIM), "invalid output shape")
    _check_tensor(lse, "lse", torch.float32)
    _require(tuple(lse.shape) == (B, Hq), "invalid lse shape")
    _require(seq_lens.numel() == B, "seq_lens batch mismatch")
    rc = _lib.load().tq4_stage2(mid_o.data_ptr(), seq_lens.data_ptr(), out.data_ptr(),
                                DTYPES[out.dtype], lse.data_ptr(), B, Hq, HEAD_DIM, S,
                                _stream(mid_o.device))
    _lib.check(rc, "tq4_stage2")
    return out, lse


def rotate_query(query, rotation_t, q_rot=None):
    """``q_rot = query.float() @ rotation_t`` on the GPU (``reference/soa_decode_v1.py:532-538``)."""
    _require(query.is_cuda and query.is_contiguous() and query.dtype in DTYPES, "invalid query")
    _check_tensor(rotation_t, "rotation_t", torch.float32)
    _require(query.size(-1) == HEAD_DIM and tuple(rotation_t.shape) == (HEAD_DIM, HEAD_DIM),
             f"requires D={HEAD_DIM}")
    if q_rot is None:
        q_rot = torch.empty(query.shape, dtype=torch.float32, device=query.device)
    _check_tensor(q_rot, "q_rot", torch.float32)
    rows = query.numel() // HEAD_DIM
    rc = _lib.load().tq4_rotate_query(query.data_ptr(), DTYPES[query.dtype], rotation_t.data_ptr(),
                                      q_rot.data_ptr(), rows, HEAD_DIM, _stream(query.device))
    _lib.check(rc, "tq4_rotate_query")
    return q_rot


def store(key, value, kv_cache, slot_mapping, rotation_t, midpoints, centroids=None, *,
          layout="soa", norm_correction=True):
    """Quantize ``key`` / ``value`` ``[N, Hk, D]`` and write token ``i`` into cache slot
    ``slot_mapping[i]`` (negative slots are skipped); returns ``kv_cache``.

    K: 4-bit Lloyd-Max indices of ``(k / (||k|| + 1e-8)) @ rotation_t`` against
    ``midpoints`` [15]; stored scalar ``fp16(||k|| / ||c[idx]||)`` with
    ``norm_correction`` (needs ``centroids`` [16]), else ``fp16(||k||)``.  V: 4-bit
    uniform codes, fp16 scale and fp16 min.
    """
    _require(key.is_cuda and key.dtype in DTYPES and key.is_contiguous(), "invalid key")
    _require(value.dtype == key.dtype and value.is_contiguous() and value.shape == key.shape,
             "value must match key (shape, dtype, contiguous)")
    _require(key.dim() == 3 and key.size(2) == HEAD_DIM, f"key must be [N, Hk, {HEAD_DIM}]")
    _check_tensor(slot_mapping, "slot_mapping", torch.int32)
    _check_tensor(rotation_t, "rotation_t", torch.float32)
    _check_tensor(midpoints, "midpoints", torch.float32)
    _require(midpoints.numel() == 15, "4-bit keys need 15 midpoints")
    _require(tuple(rotation_t.shape) == (HEAD_DIM, HEAD_DIM), f"rotation must be [{HEAD_DIM}, {HEAD_DIM}]")
    if norm_correction:
        _require(centroids is not None, "norm_correction=True requires centroids")
    if centroids is not None:
        _check_tensor(centroids, "centroids", torch.float32)
        _require(centroids.numel() == 16, "4-bit keys need 16 centroids")
    N, Hk, D = key.shape
    bs, hk, stride, lid = _cache_geometry(kv_cache, slot_bytes(D), layout)
    _require(hk == Hk, "kv_cache must be [blocks, block_size, Hk, slot]")
    _require(slot_mapping.numel() == N, "slot_mapping must have one entry per token")
    devs = {t.device for t in (key, value, kv_cache, slot_mapping, rotation_t, midpoints)}
    _require(len(devs) == 1, "all tensors must be on the same device")
    rc = _lib.load().tq4_store(
        key.data_ptr(), value.data_ptr(), DTYPES[key.dtype], slot_mapping.data_ptr(),
        rotation_t.data_ptr(), midpoints.data_ptr(),
        centroids.data_ptr() if centroids is not None else None, kv_cache.data_ptr(), N, Hk, D,
        bs, stride, lid, int(bool(norm_correction)), _stream(key.device))
    _lib.check(rc, "tq4_store")
    return kv_cache


def stage1_fp8(query, kv_cache, block_table, seq_lens, mid_o=None, *, num_kv_splits=None,
               layout="soa", attn_scale=None, sinks=None, kernel="auto"):
    """Stage1 of the FP8-key preset (``turboquant_k8v4``): ``query`` fp32 ``[B, Hq, D]``
    (not rotated), K one E4M3 byte per dim; returns ``mid_o [B, Hq, S, D+1]``.  ``kernel``:
    "auto" (16x16x32 MFMA where it applies, else VALU), "xdl" or "simple"."""
    for t, n, dt in ((query, "query", torch.float32), (block_table, "block_table", torch.int32),
                     (seq_lens, "seq_lens", torch.int32)):
        _check_tensor(t, n, dt)
    _require(query.dim() == 3 and query.size(2) == HEAD_DIM, f"query must be [B, Hq, {HEAD_DIM}]")
    B, Hq, D = query.shape
    bs, Hk, stride, lid = _cache_geometry(kv_cache, slot_bytes_fp8(D), layout, " (FP8 keys)")
    _require(Hq % Hk == 0, "Hq must be a multiple of Hk")
    _require(block_table.dim() == 2 and block_table.size(0) == B, "block_table batch mismatch")
    _require(seq_lens.dim() == 1 and seq_lens.size(0) == B, "seq_lens batch mismatch")
    if mid_o is None:
        _require(num_kv_splits is not None and num_kv_splits > 0,
                 "num_kv_splits is required when mid_o is None")
        mid_o = torch.empty(B, Hq, num_kv_splits, D + 1, dtype=torch.float32, device=query.device)
    _check_tensor(mid_o, "mid_o", torch.float32)
    S = mid_o.size(2)
    _require(tuple(mid_o.shape) == (B, Hq, S, D + 1), f"mid_o must be [B,{Hq},S,{D + 1}]")
    devs = {t.device for t in (query, kv_cache, block_table, seq_lens, mid_o)}
    _require(len(devs) == 1, "all tensors must be on the same device")
    scale = 1.0 / math.sqrt(D) if attn_scale is None else float(attn_scale)
    _require(kernel in ("auto", "xdl", "simple"), "kernel must be auto, xdl or simple")
    rc = _lib.load().tq4_stage1_fp8_ex(
        query.data_ptr(), kv_cache.data_ptr(), block_table.data_ptr(), seq_lens.data_ptr(),
        mid_o.data_ptr(), B, Hq, Hk, D, bs, block_table.size(1), stride, S, lid, scale,
        _check_sinks(sinks, Hq, query.device), KERNELS[kernel], _stream(query.device))
    _lib.check(rc, "tq4_stage1_fp8")
    return mid_o


def store_fp8(key, value, kv_cache, slot_mapping, *, layout="soa"):
    """Writer of the FP8-key preset: K cast to E4M3 (round to nearest even, saturating at
    +-448), V 4-bit uniform; returns ``kv_cache``."""
    _require(key.is_cuda and key.dtype in DTYPES and key.is_contiguous(), "invalid key")
    _require(value.dtype == key.dtype and value.is_contiguous() and value.shape == key.shape,
             "value must match key (shape, dtype, contiguous)")
    _require(key.dim() == 3 and key.size(2) == HEAD_DIM, f"key must be [N, Hk, {HEAD_DIM}]")
    _check_tensor(slot_mapping, "slot_mapping", torch.int32)
    N, Hk, D = key.shape
    bs, hk, stride, lid = _cache_geometry(kv_cache, slot_bytes_fp8(D), layout, " (FP8 keys)")
    _require(hk == Hk, "kv_cache must be [blocks, block_size, Hk, slot]")
    _require(slot_mapping.numel() == N, "slot_mapping must have one entry per token")
    devs = {t.device for t in (key, value, kv_cache, slot_mapping)}
    _require(len(devs) == 1, "all tensors must be on the same device")
    rc = _lib.load().tq4_store_fp8(
        key.data_ptr(), value.data_ptr(), DTYPES[key.dtype], slot_mapping.data_ptr(),
        kv_cache.data_ptr(), N, Hk, D, bs, stride, lid, _stream(key.device))
    _lib.check(rc, "tq4_store_fp8")
    return kv_cache


PRESETS = ((4, 4), (3, 4), (3, 3))  # (key bits, value bits) of the MSE-key presets


def stage1_preset(q_rot, kv_cache, block_table, seq_lens, centroids, mid_o=None, *, key_bits,
                  value_bits, num_kv_splits=None, layout="soa", attn_scale=None, sinks=None,
                  kernel="auto"):
    """Stage1 of the bit-width presets (``turboquant_k3v4_nc``: 3/4, ``turboquant_3bit_nc``:
    3/3, and 4/4): ``q_rot`` fp32 ``[B, Hq, D]``, ``centroids`` the ``2^key_bits`` Lloyd-Max
    centroids; returns ``mid_o [B, Hq, S, D+1]``.  ``kernel``: "auto" (3/4 and 3/3 on the
    16x16x32 MFMA kernel where it applies, 4/4 and other shapes on the VALU kernel), "xdl" or
    "simple"."""
    _require((key_bits, value_bits) in PRESETS, f"key/value bits must be one of {PRESETS}")
    for t, n, dt in ((q_rot, "q_rot", torch.float32), (block_table, "block_table", torch.int32),
                     (seq_lens, "seq_lens", torch.int32), (centroids, "centroids", torch.float32)):
        _check_tensor(t, n, dt)
    _require(q_rot.dim() == 3 and q_rot.size(2) == HEAD_DIM, f"q_rot must be [B, Hq, {HEAD_DIM}]")
    B, Hq, D = q_rot.shape
    _require(centroids.numel() == 1 << key_bits, f"{key_bits}-bit keys need {1 << key_bits} centroids")
    bs, Hk, stride, lid = _cache_geometry(kv_cache, slot_bytes_preset(D, key_bits, value_bits), layout)
    _require(Hq % Hk == 0, "Hq must be a multiple of Hk")
    _require(block_table.dim() == 2 and block_table.size(0) == B, "block_table batch mismatch")
    _require(seq_lens.dim() == 1 and seq_lens.size(0) == B, "seq_lens batch mismatch")
    if mid_o is None:
        _require(num_kv_splits is not None and num_kv_splits > 0,
                 "num_kv_splits is required when mid_o is None")
        mid_o = torch.empty(B, Hq, num_kv_splits, D + 1, dtype=torch.float32, device=q_rot.device)
    _check_tensor(mid_o, "mid_o", torch.float32)
    S = mid_o.size(2)
    _require(tuple(mid_o.shape) == (B, Hq, S, D + 1), f"mid_o must be [B,{Hq},S,{D + 1}]")
    devs = {t.device for t in (q_rot, kv_cache, block_table, seq_lens, centroids, mid_o)}
    _require(len(devs) == 1, "all tensors must be on the same device")
    scale = 1.0 / math.sqrt(D) if attn_scale is None else float(attn_scale)
    _require(kernel in ("auto", "xdl", "simple"), "kernel must be auto, xdl or simple")
    rc = _lib.load().tq4_stage1_preset_ex(
        q_rot.data_ptr(), kv_cache.data_ptr(), block_table.data_ptr(), seq_lens.data_ptr(),
        centroids.data_ptr(), mid_o.data_ptr(), B, Hq, Hk, D, bs, block_table.size(1),
        stride, S, lid, scale, _check_sinks(sinks, Hq, q_rot.device),
        key_bits, value_bits, KERNELS[kernel], _stream(q_rot.device))
    _lib.check(rc, "tq4_stage1_preset")
    return mid_o


def store_preset(key, value, kv_cache, slot_mapping, rotation_t, midpoints, centroids=None, *,
                 key_bits, value_bits, layout="soa", norm_correction=True):
    """Writer of the bit-width presets: K index = number of the ``2^key_bits - 1``
    ``midpoints`` <= y, V codes at ``value_bits``; otherwise as ``store``."""
    _require((key_bits, value_bits) in PRESETS, f"key/value bits must be one of {PRESETS}")
    _require(key.is_cuda and key.dtype in DTYPES and key.is_contiguous(), "invalid key")
    _require(value.dtype == key.dtype and value.is_contiguous() and value.shape == key.shape,
             "value must match key (shape, dtype, contiguous)")
    _require(key.dim() == 3 and key.size(2) == HEAD_DIM, f"key must be [N, Hk, {HEAD_DIM}]")
    _check_tensor(slot_mapping, "slot_mapping", torch.int32)
    _check_tensor(rotation_t, "rotation_t", torch.float32)
    _check_tensor(midpoints, "midpoints", torch.float32)
    n_mid = (1 << key_bits) - 1
    _require(midpoints.numel() == n_mid, f"{key_bits}-bit keys need {n_mid} midpoints")
    _require(tuple(rotation_t.shape) == (HEAD_DIM, HEAD_DIM), f"rotation must be [{HEAD_DIM}, {HEAD_DIM}]")
    if norm_correction:
        _require(centroids is not None, "norm_correction=True requires centroids")
    if centroids is not None:
        _check_tensor(centroids, "centroids", torch.float32)
        _require(centroids.numel() == n_mid + 1, f"{key_bits}-bit keys need {n_mid + 1} centroids")
    N, Hk, D = key.shape
    bs, hk, stride, lid = _cache_geometry(kv_cache, slot_bytes_preset(D, key_bits, value_bits), layout)
    _require(hk == Hk, "kv_cache must be [blocks, block_size, Hk, slot]")
    _require(slot_mapping.numel() == N, "slot_mapping must have one entry per token")
    devs = {t.device for t in (key, value, kv_cache, slot_mapping, rotation_t, midpoints)}
    _require(len(devs) == 1, "all tensors must be on the same device")
    rc = _lib.load().tq4_store_preset(
        key.data_ptr(), value.data_ptr(), DTYPES[key.dtype], slot_mapping.data_ptr(),
        rotation_t.data_ptr(), midpoints.data_ptr(),
        centroids.data_ptr() if centroids is not None else None, kv_cache.data_ptr(), N, Hk, D,
        bs, stride, lid, int(bool(norm_correction)), key_bits, value_bits, _stream(key.device))
    _lib.check(rc, "tq4_store_preset")
    return kv_cache


class DecodeWorkspace:
    """Preallocated buffers of one full decode step (fixed shapes, reusable)."""

    def __init__(self, batch, num_q_heads, num_kv_splits, device, out_dtype=torch.bfloat16):
        self.q_rot = torch.empty(batch, num_q_heads, HEAD_DIM, dtype=torch.float32, device=device)
        self.pair_lut = torch.empty(256, 2, dtype=torch.float32, device=device)
        self.mid_o = torch.empty(batch, num_q_heads, num_kv_splits, HEAD_DIM + 1,
                                 dtype=torch.float32, device=device)
        self.out = torch.empty(batch, num_q_heads, HEAD_DIM, dtype=out_dtype, device=device)
        self.lse = torch.empty(batch, num_q_heads, dtype=torch.float32, device=device)


def full_decode(query, rotation_t, kv_cache, block_table, seq_lens, centroids, num_kv_splits, *,
                layout="soa", out_dtype=None, attn_scale=None, workspace=None, sinks=None):
    """Rotation + pair LUT + Stage1 + Stage2 in four launches; returns ``(out, lse)``.

    ``out`` is in ``out_dtype`` (default: the query dtype, as ``reference/soa_decode_v1.py:643``).
    """
    _require(query.is_cuda and query.is_contiguous() and query.dtype in DTYPES, "invalid query")
    _check_tensor(rotation_t, "rotation_t", torch.float32)
    _check_tensor(centroids, "centroids", torch.float32)
    _require(centroids.numel() == 16, "4-bit path requires 16 centroids")
    for t, n, dt in ((block_table, "block_table", torch.int32), (seq_lens, "seq_lens", torch.int32)):
        _check_tensor(t, n, dt)
    _require(query.dim() == 3, "query must be [B, Hq, D]")
    B, Hq, D = query.shape
    _require(D == HEAD_DIM, f"requires D={HEAD_DIM}")
    bs, Hk, stride, lid = _cache_geometry(kv_cache, slot_bytes(D), layout)
    out_dtype = query.dtype if out_dtype is None else out_dtype
    ws = workspace or DecodeWorkspace(B, Hq, num_kv_splits, query.device, out_dtype)
    _require(ws.out.dtype == out_dtype and ws.mid_o.shape[:3] == (B, Hq, num_kv_splits),
             "workspace does not match this call")
    scale = 1.0 / math.sqrt(D) if attn_scale is None else float(attn_scale)
    sinks_ptr = _check_sinks(sinks, Hq, query.device)
    rc = _lib.load().tq4_full_decode(
        query.data_ptr(), DTYPES[query.dtype], rotation_t.data_ptr(), centroids.data_ptr(),
        kv_cache.data_ptr(), block_table.data_ptr(), seq_lens.data_ptr(), ws.q_rot.data_ptr(),
        ws.pair_lut.data_ptr(), ws.mid_o.data_ptr(), ws.out.data_ptr(), DTYPES[out_dtype],
        ws.lse.data_ptr(), B, Hq, Hk, D, bs, block_table.size(1), stride,
        num_kv_splits, lid, scale, sinks_ptr, _stream(query.device))
    _lib.check(rc, "tq4_full_decode")
    return ws.out, ws.lse


def _buffer_view(buf, shape, dtype):
    """``buf`` cut to ``shape`` (leading sub-block) when it fits and stays contiguous."""
    if buf is None or buf.dtype != dtype or buf.dim() != len(shape):
        return None
    if any(have < want for have, want in zip(buf.shape, shape)):
        return None
    view = buf[tuple(slice(0, n) for n in shape)]
    return view if view.is_contiguous() else None


def _decode_buffers(query, S, buf_holder, mid_o_buf, output_buf, lse_buf):
    """Workspace of one decode call: the caller's ``mid_o_buf`` / ``output_buf`` /
    ``lse_buf`` when they fit (leading sub-blocks, as ``reference/soa_decode_v1.py:541-560``
    takes them), else buffers kept on ``buf_holder`` and reused by later calls of the same
    shape, so that a captured call replays on the same memory."""
    B, Hq, D = query.shape
    dev = query.device

    def held(name, shape, dtype):
        buf = getattr(buf_holder, name, None) if buf_holder is not None else None
        view = _buffer_view(buf, shape, dtype)
        if view is None:
            view = torch.empty(shape, dtype=dtype, device=dev)
            if buf_holder is not None:
                setattr(buf_holder, name, view)
        return view

    def given(buf, name, shape, dtype):
        view = _buffer_view(buf, shape, dtype)
        return view if view is not None else held(name, shape, dtype)

    ws = DecodeWorkspace.__new__(DecodeWorkspace)
    ws.q_rot = held("_tq4_q_rot_buf", (B, Hq, D), torch.float32)
    ws.pair_lut = held("_tq4_pair_lut_buf", (256, 2), torch.float32)
    ws.mid_o = given(mid_o_buf, "_tq_mid_o_buf", (B, Hq, S, D + 1), torch.float32)
    ws.out = given(output_buf, "_tq_output_buf", (B, Hq, D), query.dtype)
    ws.lse = given(lse_buf, "_tq_lse_buf", (B, Hq), torch.float32)
    return ws


def turboquant_decode_attention(query, kv_cache, block_table, seq_lens, Pi, centroids, scale,
                                mse_bits, key_packed_size, value_quant_bits, key_fp8=False,
                                norm_correction=False, PiT=None, mid_o_buf=None, output_buf=None,
                                lse_buf=None, buf_holder=None, max_num_kv_splits=32, sinks=None, *,
                                layout="soa"):
    """The decode entry of the vLLM backend (``reference/soa_decode_v1.py:485-643``; AoS
    ``reference/aos_decode.py:486-626``): ``q_rot = query @ PiT``, pair LUT, Stage1 over
    ``max_num_kv_splits`` splits, Stage2; returns ``[B, Hq, D]`` in the query dtype.

    ``kv_cache`` is the contiguous ``[blocks, block_size, Hk, slot]`` cache or the backend's
    ``transpose(1, 2)`` view of its ``[blocks, Hk, block_size, slot]`` cache.  Caller buffers
    are used when they fit (``mid_o_buf`` fp32 ``[>=B, Hq, S, D+1]``, ``output_buf``
    ``[>=B, Hq, D]`` in the query dtype, ``lse_buf`` fp32 ``[>=B, Hq]``); the other buffers
    live on ``buf_holder`` when one is given.  The launches depend only on shapes, never on
    ``seq_lens`` or ``block_table`` contents, and nothing is allocated once ``buf_holder``
    holds the buffers, so a call can be captured in a graph and replayed
    (``reference/turboquant_attn.py:368-373``).  ``sinks`` (fp32 ``[Hq]``) enter split 0.
    Built for the 4-bit ``turboquant_4bit_nc`` cache, with ``key_fp8`` the ``turboquant_k8v4``
    cache (unrotated query), and the 3-bit presets ``turboquant_k3v4_nc`` /
    ``turboquant_3bit_nc``, all on the 16x16x32 MFMA Stage1 where it applies (power-of-two
    blocks of 16 tokens or more), else the VALU kernel; 4-bit AoS without norm correction raises ``NotImplementedError``.
    """
    _require(query.dim() == 3 and query.size(2) == HEAD_DIM, f"query must be [B, Hq, {HEAD_DIM}]")
    S = int(max_num_kv_splits)
    ws = _decode_buffers(query, S, buf_holder, mid_o_buf, output_buf, lse_buf)
    if key_fp8:
        _require(value_quant_bits == 4, "FP8 keys are built with 4-bit values")
        _require(key_packed_size == HEAD_DIM, f"key_packed_size must be {HEAD_DIM} for FP8 keys")
        # the unrotated query (reference/soa_decode_v1.py:528-534), as fp32
        ws.q_rot.copy_(query)
        stage1_fp8(ws.q_rot, kv_cache, block_table, seq_lens, ws.mid_o, layout=layout,
                   attn_scale=scale, sinks=sinks)
        stage2(ws.mid_o, seq_lens, ws.out, ws.lse)
        return ws.out
    _require((mse_bits, value_quant_bits) in PRESETS,
             f"MSE key / value bits must be one of {PRESETS}")
    want = HEAD_DIM * mse_bits // 8 + 2
    _require(key_packed_size == want, f"key_packed_size must be {want}")
    if layout == "aos" and not norm_correction:
        raise NotImplementedError("AoS decode is built with the norm correction (the _nc presets)")
    if PiT is None:
        PiT = Pi.t().contiguous()
    query = query.contiguous()
    if mse_bits != 4 or value_quant_bits != 4:
        # 3-bit-key presets: rotation, Stage1 over the preset cache, Stage2
        rotate_query(query, PiT, ws.q_rot)
        stage1_preset(ws.q_rot, kv_cache, block_table, seq_lens, centroids.float().contiguous(),
                      ws.mid_o, key_bits=mse_bits, value_bits=value_quant_bits, layout=layout,
                      attn_scale=scale, sinks=sinks)
        stage2(ws.mid_o, seq_lens, ws.out, ws.lse)
        return ws.out
    out, _ = full_decode(query, PiT, kv_cache, block_table, seq_lens, centroids, S,
                         layout=layout, out_dtype=query.dtype, attn_scale=scale, workspace=ws,
                         sinks=sinks)
    return out


# ---- reference harness call shapes -------------------------------------------------

def launch_tq4_v2_stage1(q_rot, kv_cache, block_table, seq_lens, centroids, pair_lut, mid_o=None,
                         num_kv_splits=32):
    """SoA Stage1 with the ``baseline/triton_v2.py:569-577`` signature."""
    _check_tensor(centroids, "centroids", torch.float32)
    _require(centroids.numel() == 16, "4-bit path requires 16 centroids")
    return stage1(q_rot, kv_cache, block_table, seq_lens, pair_lut, mid_o,
                  num_kv_splits=None if mid_o is not None else num_kv_splits, layout="soa")


def launch_soa_v1_stage1(q_rot, kv_cache, block_table, seq_lens, centroids, mid_o):
    """SoA Stage1 with the ``baseline/triton_v1.py:145-152`` signature."""
    return stage1(q_rot, kv_cache, block_table, seq_lens, pair_lut_device(centroids), mid_o,
                  layout="soa")


def launch_aos_v1_stage1(q_rot, kv_cache, block_table, seq_lens, centroids, mid_o):
    """AoS Stage1 with the ``baseline/triton_v1.py:90-97`` signature."""
    return stage1(q_rot, kv_cache, block_table, seq_lens, pair_lut_device(centroids), mid_o,
                  layout="aos")


def launch_stage2(mid_o, seq_lens, output, lse):
    """Stage2 with the ``baseline/stage2.py:58-63`` signature (writes in place)."""
    stage2(mid_o, seq_lens, output, lse)


def triton_turboquant_store(key, value, kv_cache, slot_mapping, PiT, midpoints, mse_bits,
                            key_packed_size, value_quant_bits, key_fp8=False, centroids=None,
                            norm_correction=False):
    """SoA cache writer with the ``reference/soa_store.py:381-397`` signature: the MSE-key
    presets (4/4, 3/4, 3/3 key / value bits) and FP8 keys with 4-bit values."""
    if key_fp8:  # turboquant_k8v4: no rotation, no codebook
        _require(value_quant_bits == 4 and key_packed_size == HEAD_DIM, "FP8 keys need 4-bit values "
                 f"and key_packed_size {HEAD_DIM}")
        store_fp8(key, value, kv_cache, slot_mapping, layout="soa")
        return
    _store_mse(key, value, kv_cache, slot_mapping, PiT, midpoints, mse_bits, key_packed_size,
               value_quant_bits, centroids, norm_correction, "soa")


def _store_mse(key, value, kv_cache, slot_mapping, PiT, midpoints, mse_bits, key_packed_size,
               value_quant_bits, centroids, norm_correction, layout):
    _require((mse_bits, value_quant_bits) in PRESETS,
             f"MSE key / value bits must be one of {PRESETS}")
    want = HEAD_DIM * mse_bits // 8 + 2
    _require(key_packed_size == want, f"key_packed_size must be {want}")
    if mse_bits == 4 and value_quant_bits == 4:
        store(key, value, kv_cache, slot_mapping, PiT, midpoints, centroids, layout=layout,
              norm_correction=norm_correction)
    else:
        store_preset(key, value, kv_cache, slot_mapping, PiT, midpoints, centroids,
                     key_bits=mse_bits, value_bits=value_quant_bits, layout=layout,
                     norm_correction=norm_correction)


def aos_triton_turboquant_store(key, value, kv_cache, slot_mapping, PiT, midpoints, mse_bits,
                                key_packed_size, value_quant_bits, key_fp8=False):
    """AoS cache writer with the ``reference/aos_store.py:350-361`` signature: the MSE-key
    presets (the slot keeps the raw fp16 norm, no norm correction) and FP8 keys."""
    if key_fp8:  # turboquant_k8v4: no rotation, no codebook
        _require(value_quant_bits == 4 and key_packed_size == HEAD_DIM, "FP8 keys need 4-bit values "
                 f"and key_packed_size {HEAD_DIM}")
        store_fp8(key, value, kv_cache, slot_mapping, layout="aos")
        return
    _store_mse(key, value, kv_cache, slot_mapping, PiT, midpoints, mse_bits, key_packed_size,
               value_quant_bits, None, False, "aos")


class _CudaExtCompat:
    """Methods named like the reference CUDA extension modules (``cuda/tq4_cuda_v*_bind.cpp``).

    ``tq4_cuda_vN(q_rot, kv_cache, block_table, seq_lens, centroids, mid_o)`` runs the SoA
    Stage1 with the split count taken from ``mid_o``; ``tq4_cuda_v7_stage2(mid_o, output,
    lse)`` merges every split of every row, as the reference V7 kernel does
    (``cuda/tq4_cuda_v7.cu:44-47``; it has no ``seq_lens`` argument), or only the non-empty
    splits when ``seq_lens`` is given; ``tq4_cuda_v7_full`` runs Stage1 and Stage2.  The
    object holds no state between calls.

    Precondition of ``tq4_cuda_v7_stage2`` without ``seq_lens`` (the reference kernel's too):
    Stage1 wrote every split row, i.e. every length gives S non-empty splits,
    ``ceil(len / ceil(len / S)) == S`` (true when len is a multiple of S; 77 tokens over 32
    splits of 3 leave 6 empty).  Rows of empty splits are never written (they keep whatever
    the buffer held) and would enter the merge; otherwise pass ``seq_lens``.
    """

    def _stage1(self, q_rot, kv_cache, block_table, seq_lens, centroids, mid_o):
        return launch_soa_v1_stage1(q_rot, kv_cache, block_table, seq_lens, centroids, mid_o)

    def __getattr__(self, name):
        if name.startswith("tq4_cuda_v") and name[len("tq4_cuda_v"):].isdigit():
            return self._stage1
        raise AttributeError(name)

    def tq4_cuda_v7_stage1(self, *args):
        return self._stage1(*args)

    def tq4_cuda_v7_stage2(self, mid_o, output, lse, seq_lens=None):
        if seq_lens is None:
            # every split merged (the caller's precondition: all of them were written); a
            # length of S tokens over S splits makes every split non-empty
            seq_lens = torch.full((mid_o.size(0),), mid_o.size(2), dtype=torch.int32,
                                  device=mid_o.device)
        stage2(mid_o, seq_lens, output, lse)
        return output

    def tq4_cuda_v7_full(self, q_rot, kv_cache, block_table, seq_lens, centroids, mid_o, output,
                         lse):
        self._stage1(q_rot, kv_cache, block_table, seq_lens, centroids, mid_o)
        stage2(mid_o, seq_lens, output, lse)
        return output


ext = _CudaExtCompat()
