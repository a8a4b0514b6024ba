"""C ABI surface: the library loads, exports every declared symbol, and rejects bad
arguments with a status and message (checks that return before any GPU work)."""
import ctypes
import re
import subprocess

import pytest
import torch

from conftest import ROOT
from tq4_decode import _lib, ops

HEADER = ROOT / "include" / "tq4_decode.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(tq4_\w+)\s*\(", text, re.M)))


def test_header_declares_the_binding_table():
    assert declared() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared():
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                        text=True, check=True).stdout
    exported = set(re.findall(r" T (tq4_\w+)$", nm, re.M))
    assert set(declared()) <= exported
    assert _lib.load().tq4_abi_version() == 106


def _stage1_call(**over):
    args = dict(q=1 << 12, cache=1 << 12, bt=1 << 12, sl=1 << 12, lut=1 << 12, mid=1 << 12, B=2,
                Hq=32, Hk=8, D=128, bs=16, maxb=4, stride=17152, S=4, layout=0, scale=0.088)
    args.update(over)
    return _lib.load().tq4_stage1(args["q"], args["cache"], args["bt"], args["sl"], args["lut"],
                                  args["mid"], args["B"], args["Hq"], args["Hk"], args["D"],
                                  args["bs"], args["maxb"], args["stride"], args["S"],
                                  args["layout"], args["scale"], None)


@pytest.mark.parametrize("over,code,text", [
    (dict(q=0), 1, "null pointer"),
    (dict(B=0), 1, "must be positive"),
    (dict(Hq=30), 1, "multiple of Hk"),
    (dict(D=64), 2, "head_dim 64"),
    (dict(S=65537), 2, "num_kv_splits 65537"),
    (dict(B=65536), 2, "batch 65536"),
    (dict(layout=3), 1, "layout"),
    (dict(stride=100), 1, "requires cache"),
    (dict(cache=(1 << 12) + 2), 1, "16-byte aligned"),
    (dict(scale=-1.0), 1, "attn_scale"),
])
def test_stage1_rejects_bad_arguments(over, code, text):
    assert _stage1_call(**over) == code
    assert text in _lib.load().tq4_last_error().decode()


def test_stage2_and_helpers_reject_bad_arguments():
    lib = _lib.load()
    assert lib.tq4_stage2(None, 1, 1, 0, 1, 1, 1, 128, 4, None) == 1
    assert lib.tq4_stage2(8, 8, 8, 7, 8, 1, 1, 128, 4, None) == 1
    assert "out_dtype" in lib.tq4_last_error().decode()
    assert lib.tq4_stage2(8, 8, 8, 0, 8, 1, 1, 128, 65537, None) == 2
    assert lib.tq4_stage2(8, 8, 8, 0, 8, 65536, 1, 128, 4, None) == 2
    assert "above 65535" in lib.tq4_last_error().decode()
    assert lib.tq4_rotate_query(8, 0, 8, 8, 4, 64, None) == 2
    assert lib.tq4_build_pair_lut(8, 8, 8, None) == 2


def test_python_wrappers_mirror_reference_checks():
    q = torch.zeros(2, 32, 128)
    cache = torch.zeros(4, 16, 8, 134, dtype=torch.uint8)
    bt = torch.zeros(2, 2, dtype=torch.int32)
    sl = torch.zeros(2, dtype=torch.int32)
    lut = torch.zeros(256, 2)
    with pytest.raises(RuntimeError, match="q_rot must be CUDA"):
        ops.stage1(q, cache, bt, sl, lut, num_kv_splits=4)
    with pytest.raises(RuntimeError, match="centroids must be CUDA"):
        ops.launch_soa_v1_stage1(q, cache, bt, sl, torch.zeros(16), torch.zeros(2, 32, 4, 129))


@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_cache_views_the_backend_passes(layout):
    """The contiguous cache and the backend's ``transpose(1, 2)`` view of its head-major
    ``[blocks, Hk, bs, slot]`` cache (reference/turboquant_attn.py:536, :565) are accepted; an
    AoS view of the head-major cache selects the head-major slot strides."""
    from tq4_decode.layout import AOS, AOS_HEAD_MAJOR, SOA

    pm = torch.zeros(6, 16, 8, 134, dtype=torch.uint8)
    hm = torch.zeros(6, 8, 16, 134, dtype=torch.uint8).transpose(1, 2)
    geo = lambda t: ops.block_geometry(tuple(t.shape), t.stride(), 134, layout)  # noqa: E731
    base = SOA if layout == "soa" else AOS
    assert geo(pm) == (16, 8, 17152, base)
    assert geo(hm) == (16, 8, 17152, SOA if layout == "soa" else AOS_HEAD_MAJOR)
    # padded blocks keep their stride; one kv-head: both orders coincide
    padded = torch.zeros(6, 17200, dtype=torch.uint8)[:, :17152].view(6, 16, 8, 134)
    assert geo(padded)[2] == 17200
    one = torch.zeros(6, 1, 16, 134, dtype=torch.uint8).transpose(1, 2)
    assert ops.block_geometry(tuple(one.shape), one.stride(), 134, layout)[3] == base
    bad = [torch.zeros(6, 16, 8, 268, dtype=torch.uint8)[..., ::2],          # strided slot bytes
           torch.zeros(16, 6, 8, 134, dtype=torch.uint8).transpose(0, 1),   # blocks interleaved
           torch.zeros(6, 16, 8, 140, dtype=torch.uint8)[..., :134]]        # padded slots
    for t in bad:
        with pytest.raises(RuntimeError, match="kv_cache"):
            geo(t)
    with pytest.raises(RuntimeError, match="slot_size=134"):
        ops.block_geometry((6, 16, 8, 118), (15104, 944, 118, 1), 134, layout)
