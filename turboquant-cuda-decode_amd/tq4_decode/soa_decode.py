"""Drop-in for ``reference/soa_decode_v1.py`` (the SoA decode entry,
``triton_turboquant_decode_attention``): same signature, running the gfx950 rotation,
Stage1 and Stage2."""
from functools import partial

from .ops import turboquant_decode_attention

triton_turboquant_decode_attention = partial(turboquant_decode_attention, layout="soa")
triton_turboquant_decode_attention.__doc__ = turboquant_decode_attention.__doc__

__all__ = ["triton_turboquant_decode_attention"]
