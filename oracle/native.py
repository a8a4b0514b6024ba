"""ctypes binding of the C oracle ``tq4_oracle.c`` (test infrastructure only)."""
from __future__ import annotations

import ctypes
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libtq4_oracle.so"
_lib = None


def build(force: bool = True) -> pathlib.Path:
    cmd = ["make", "-C", str(HERE)] + (["-B"] if force else [])
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build(force=False)
        _lib = ctypes.CDLL(str(LIB_PATH))
        p, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
        _lib.tq4o_stage1.argtypes = [p, p, p, p, p, p, i32, i32, i32, i32, i32, i32, i64, i32,
                                     i32, f32, i32]
        _lib.tq4o_stage1.restype = i32
        _lib.tq4o_stage2.argtypes = [p, p, p, p, i32, i32, i32, i32, i32]
        _lib.tq4o_stage2.restype = i32
        _lib.tq4o_max_threads.restype = i32
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def default_threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def stage1(q_rot, cache, block_table, seq_lens, cents, num_splits, *, num_kv_heads,
           block_size=16, is_aos=False, attn_scale=None, mid_o=None, threads=None):
    """float32 Stage1; returns ``mid_o`` (NaN-filled where splits are empty unless given)."""
    q = np.ascontiguousarray(q_rot, dtype=np.float32)
    c8 = np.ascontiguousarray(cache).view(np.uint8)
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    c = np.ascontiguousarray(cents, dtype=np.float32)
    batch, num_q_heads, head_dim = q.shape
    if mid_o is None:
        mid_o = np.full((batch, num_q_heads, num_splits, head_dim + 1), np.nan, np.float32)
    stride = block_size * num_kv_heads * (head_dim + 6 + ((head_dim + 6) & 1))
    scale = float(1.0 / np.sqrt(head_dim)) if attn_scale is None else float(attn_scale)
    rc = lib().tq4o_stage1(_ptr(q), _ptr(c8), _ptr(bt), _ptr(sl), _ptr(c), _ptr(mid_o), batch,
                           num_q_heads, num_kv_heads, head_dim, block_size, bt.shape[1], stride,
                           num_splits, int(is_aos), scale,
                           default_threads() if threads is None else threads)
    if rc:
        raise ValueError("tq4o_stage1 rejected its arguments")
    return mid_o


def stage2(mid_o, seq_lens, threads=None):
    mid = np.ascontiguousarray(mid_o, dtype=np.float32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    batch, num_q_heads, num_splits, d1 = mid.shape
    out = np.empty((batch, num_q_heads, d1 - 1), np.float32)
    lse = np.empty((batch, num_q_heads), np.float32)
    rc = lib().tq4o_stage2(_ptr(mid), _ptr(sl), _ptr(out), _ptr(lse), batch, num_q_heads, d1 - 1,
                           num_splits, default_threads() if threads is None else threads)
    if rc:
        raise ValueError("tq4o_stage2 rejected its arguments")
    return out, lse
