"""Drop-in for ``reference/aos_store.py`` (and its vLLM copy
``vllm/v1/attention/ops/triton_turboquant_store.py``): the AoS cache writer under the
reference's module and function name, running the gfx950 writer."""
from .ops import aos_triton_turboquant_store as triton_turboquant_store  # noqa: F401

__all__ = ["triton_turboquant_store"]
