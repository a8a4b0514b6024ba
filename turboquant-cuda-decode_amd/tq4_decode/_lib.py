"""ctypes binding of ``libtq4_decode.so`` (the C ABI in ``include/tq4_decode.h``).

``torch`` is imported first so that the process has a single HIP runtime: the
library's ``libamdhip64.so.7`` dependency then resolves to the copy torch already
loaded, and torch's stream handles are valid in library calls.
"""
from __future__ import annotations

import ctypes
import os
import pathlib

import torch  # noqa: F401  (see module docstring)

# TQ4_DECODE_LIB selects another build of the same library (e.g. for A/B timing).
LIB_PATH = pathlib.Path(os.environ.get("TQ4_DECODE_LIB") or
                        pathlib.Path(__file__).resolve().parent / "libtq4_decode.so")

EXPORTS = (
    "tq4_stage1",
    "tq4_stage1_ex",
    "tq4_stage2",
    "tq4_rotate_query",
    "tq4_build_pair_lut",
    "tq4_full_decode",
    "tq4_full_decode_noalloc",
    "tq4_store",
    "tq4_stage1_fp8",
    "tq4_stage1_fp8_ex",
    "tq4_store_fp8",
    "tq4_stage1_preset",
    "tq4_stage1_preset_ex",
    "tq4_store_preset",
    "tq4_last_error",
    "tq4_abi_version",
    "tq4_time_next_launch",
)

_handle = None

_p, _i, _i64, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
_SIGS = {
    "tq4_stage1": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i64, _i, _i, _f, _p],
    "tq4_stage1_ex": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i64, _i, _i, _f, _i, _p, _p],
    "tq4_stage2": [_p, _p, _p, _i, _p, _i, _i, _i, _i, _p],
    "tq4_rotate_query": [_p, _i, _p, _p, _i, _i, _p],
    "tq4_build_pair_lut": [_p, _p, _i, _p],
    "tq4_full_decode": [_p, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _p, _i, _i, _i, _i, _i,
                        _i, _i64, _i, _i, _f, _p, _p],
    "tq4_full_decode_noalloc": [_p, _i, _p, _p, _p, _p, _p, _p, _i, _p, _i, _i, _i, _i, _i, _i,
                                _i64, _i, _i, _f, _p, _p],
    "tq4_store": [_p, _p, _i, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i64, _i, _i, _p],
    "tq4_last_error": [],
    "tq4_abi_version": [],
    "tq4_time_next_launch": [_p, _p],
    "tq4_stage1_fp8": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i64, _i, _i, _f, _p, _p],
    "tq4_store_fp8": [_p, _p, _i, _p, _p, _i, _i, _i, _i, _i64, _i, _p],
    "tq4_stage1_fp8_ex": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i64, _i, _i, _f, _p, _i, _p],
    "tq4_stage1_preset": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i64, _i, _i, _f, _p, _i,
                          _i, _p],
    "tq4_stage1_preset_ex": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i64, _i, _i, _f, _p, _i,
                             _i, _i, _p],
    "tq4_store_preset": [_p, _p, _i, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i64, _i, _i, _i, _i, _p],
}


class Tq4Error(RuntimeError):
    """A C-ABI call returned a nonzero status."""


def load():
    """Load the library once; fail loudly when it has not been built."""
    global _handle
    if _handle is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP library first "
                "(python __graft_entry__.py, or python -m tq4_decode.build)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, args in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_char_p if name == "tq4_last_error" else ctypes.c_int
        _handle = lib
    return _handle


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().tq4_last_error().decode(errors="replace")
        raise Tq4Error(f"{what} failed (status {rc}): {msg}")
