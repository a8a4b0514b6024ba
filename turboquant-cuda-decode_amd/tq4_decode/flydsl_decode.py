"""Drop-in for ``reference/flydsl_decode.py`` (vLLM module
``vllm/v1/attention/ops/flydsl_turboquant_decode.py``): the gfx950 decode entry the backend
imports at ``reference/turboquant_attn.py:56-60`` and calls for GQA 6 / 8 / 16 layers
(``:1143-1183``), running this package's gfx950 kernels instead of FlyDSL.

``flydsl_turboquant_decode_attention`` has the signature of
``reference/flydsl_decode.py:559-581`` and the same preset checks (MSE keys at 4 bits, 4-bit
values, 16 centroids, D = 128; ``:604-626``).  Differences, all wider than the reference:

* any block size that is a power of two >= 16 runs on the matrix-core Stage1 (the reference
  takes 16 or 32), and any GQA group on the VALU kernel where the matrix-core one does not
  apply (the reference takes 6, 8, 16);
* ``sinks`` are honoured (split 0's softmax starts from them; the reference ignores them
  with a warning);
* the number of splits is ``max_num_kv_splits``, fixed by the caller, so a captured call
  replays with the same launches (the reference derives its partition count from
  ``block_table.shape[1]`` for the same reason, ``:671-692``).

``is_flydsl_available`` / ``is_flydsl_gqa6_available`` report whether these kernels can run
here: a gfx950 device and the HIP library present.
"""
from __future__ import annotations

from .ops import HEAD_DIM, turboquant_decode_attention

__all__ = ["flydsl_turboquant_decode_attention", "is_flydsl_available", "is_flydsl_gqa6_available"]

_AVAILABLE = None


def is_flydsl_available() -> bool:
    """True on a gfx950 device with the HIP library built (``reference/flydsl_decode.py:56-116``
    gates on gfx950 and an importable FlyDSL)."""
    global _AVAILABLE
    if _AVAILABLE is None:
        try:
            import torch

            from . import _lib

            ok = torch.cuda.is_available() and \
                torch.cuda.get_device_properties(0).gcnArchName.split(":")[0] == "gfx950"
            if ok:
                _lib.load()
            _AVAILABLE = bool(ok)
        except (RuntimeError, OSError, AttributeError):
            _AVAILABLE = False
    return _AVAILABLE


def is_flydsl_gqa6_available() -> bool:
    """GQA 6 runs wherever the kernels run (``reference/flydsl_decode.py:119-128`` needs a
    sibling FlyDSL module for it)."""
    return is_flydsl_available()


def flydsl_turboquant_decode_attention(query, kv_cache, block_table, seq_lens, Pi, centroids, scale,
                                       mse_bits, key_packed_size, value_quant_bits, value_packed_size,
                                       key_fp8=False, norm_correction=False, PiT=None, max_seq_len=0,
                                       mid_o_buf=None, output_buf=None, lse_buf=None, buf_holder=None,
                                       max_num_kv_splits=32, sinks=None):
    """Decode attention over the SoA ``turboquant_4bit_nc`` cache; returns ``[B, Hq, D]`` in
    the query dtype.  ``kv_cache``: the contiguous ``[blocks, block_size, Hk, slot]`` cache or
    the backend's ``transpose(1, 2)`` view of its ``[blocks, Hk, block_size, slot]`` cache."""
    if key_fp8:
        raise AssertionError("FlyDSL supports MSE-key path only")
    if mse_bits != 4:
        raise AssertionError(f"FlyDSL expects mse_bits=4, got {mse_bits}")
    if value_quant_bits != 4:
        raise AssertionError(f"FlyDSL expects value_quant_bits=4, got {value_quant_bits}")
    if query.dim() != 3 or query.size(2) != HEAD_DIM:
        raise AssertionError(f"query must be [B, Hq, {HEAD_DIM}]")
    if centroids.numel() != 16:
        raise AssertionError(f"centroids.numel={centroids.numel()} != 16")
    # key_packed_size / value_packed_size are implied by the preset (the reference drops
    # them too, :598); max_seq_len only sizes the reference's launch
    del key_packed_size, value_packed_size, max_seq_len
    return turboquant_decode_attention(
        query, kv_cache, block_table, seq_lens, Pi, centroids, scale, 4, HEAD_DIM // 2 + 2, 4,
        key_fp8=False, norm_correction=norm_correction, PiT=PiT, mid_o_buf=mid_o_buf,
        output_buf=output_buf, lse_buf=lse_buf, buf_holder=buf_holder,
        max_num_kv_splits=max_num_kv_splits, sinks=sinks, layout="soa")
