"""Drop-in for ``reference/aos_decode.py`` (and its vLLM copy
``vllm/v1/attention/ops/triton_turboquant_decode.py``, imported by the backend at
``reference/turboquant_attn.py:61-65``): the AoS decode entry
``triton_turboquant_decode_attention`` with the same signature, running the gfx950 kernels."""
from functools import partial

from .ops import turboquant_decode_attention

triton_turboquant_decode_attention = partial(turboquant_decode_attention, layout="aos")
triton_turboquant_decode_attention.__doc__ = turboquant_decode_attention.__doc__

__all__ = ["triton_turboquant_decode_attention"]
