"""Drop-in for ``reference/soa_unified.py`` (vLLM module
``vllm/v1/attention/ops/turboquant_soa/triton_turboquant_unified_attention.py``), whose decode
adapter ``triton_turboquant_decode_attention_soa`` the backend's ``_soa_imports()`` loads
(``reference/turboquant_attn.py:87-103``) and calls on gfx950 through
``_dispatch_decode_soa`` (``:1194-1216``, ``:1241-1257``).

Same signature as ``reference/soa_unified.py:1291-1313``, running the gfx950 rotation,
Stage1 and Stage2 on the SoA cache:

* ``value_packed_size`` is checked against the preset: ``ceil(D * value_quant_bits / 8) + 4``
  bytes (codes + fp16 scale and zero, ``reference/config.py:150-157``); any other value
  raises ``RuntimeError``.
* ``max_seq_len`` is a hint the reference only uses to size its launch; the launches here
  depend on shapes alone (graph capture), so it is accepted and unused.
* ``mid_o_buf`` / ``output_buf`` / ``lse_buf`` / ``buf_holder`` are used as workspace when
  they fit (the reference drops all but ``output_buf``); ``sinks`` (fp32 ``[Hq]``) enter
  split 0's softmax.
* There is no ``sliding_window`` parameter, as in the reference: the backend's signature
  filter then raises ``NotImplementedError`` for a layer with a window, exactly as it does
  with the reference adapter.
"""
from __future__ import annotations

import math

from .ops import HEAD_DIM, _require, turboquant_decode_attention

__all__ = ["triton_turboquant_decode_attention_soa", "value_packed_bytes"]


def value_packed_bytes(head_dim: int, value_quant_bits: int) -> int:
    """Packed bytes of one value vector: codes plus fp16 scale and zero
    (``reference/config.py:150-157``)."""
    return math.ceil(head_dim * value_quant_bits / 8) + 4


def triton_turboquant_decode_attention_soa(query, kv_cache, block_table, seq_lens, Pi, centroids,
                                           scale, mse_bits, key_packed_size, value_quant_bits,
                                           value_packed_size, key_fp8=False, norm_correction=False,
                                           PiT=None, max_seq_len=0, mid_o_buf=None, output_buf=None,
                                           lse_buf=None, buf_holder=None, max_num_kv_splits=32,
                                           sinks=None):
    """Decode attention over the SoA TurboQuant cache; returns ``[B, Hq, D]`` in the query
    dtype (``reference/soa_unified.py:1291-1340``).  ``kv_cache`` is the contiguous
    ``[blocks, block_size, Hk, slot]`` cache or the backend's ``transpose(1, 2)`` view."""
    want = value_packed_bytes(HEAD_DIM, value_quant_bits)
    _require(int(value_packed_size) == want,
             f"value_packed_size must be {want} for {value_quant_bits}-bit values, got {value_packed_size}")
    del max_seq_len  # a sizing hint only; every launch here depends on shapes alone
    return turboquant_decode_attention(
        query, kv_cache, block_table, seq_lens, Pi, centroids, scale, mse_bits, key_packed_size,
        value_quant_bits, key_fp8=key_fp8, norm_correction=norm_correction, PiT=PiT,
        mid_o_buf=mid_o_buf, output_buf=output_buf, lse_buf=lse_buf, buf_holder=buf_holder,
        max_num_kv_splits=max_num_kv_splits, sinks=sinks, layout="soa")
