"""Drop-in for ``reference/soa_store.py`` (and its vLLM copy
``vllm/v1/attention/ops/turboquant_soa/triton_turboquant_store.py``): the SoA cache writer
under the reference's module and function name, running the gfx950 writer."""
from .ops import triton_turboquant_store  # noqa: F401

__all__ = ["triton_turboquant_store"]
