"""MI355X (gfx950) TurboQuant ``turboquant_4bit_nc`` decode: Stage1 / Stage2 / full step,
and the cache writer.

The compute runs in the HIP library ``libtq4_decode.so`` (C ABI: ``include/tq4_decode.h``);
this package is the torch-facing host side with the reference harness's call shapes.
"""
from . import codebook, layout, workloads  # noqa: F401  (host-side, no GPU needed)

__all__ = [
    "codebook", "layout", "workloads", "ops", "stage1", "stage2", "full_decode",
    "rotate_query", "pair_lut_device", "launch_tq4_v2_stage1", "launch_soa_v1_stage1",
    "launch_aos_v1_stage1", "launch_stage2", "ext", "DecodeWorkspace", "Tq4Error", "store",
    "triton_turboquant_store", "aos_triton_turboquant_store", "turboquant_decode_attention",
    "stage1_fp8", "store_fp8", "stage1_preset", "store_preset",
]


def __getattr__(name):
    # ops imports torch and the HIP library binding; load it on first use
    if name in __all__[3:]:
        import importlib

        ops = importlib.import_module(".ops", __name__)
        return ops if name == "ops" else getattr(ops, name)
    raise AttributeError(name)
