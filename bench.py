"""Stage1 benchmark of the MI355X TurboQuant 4-bit decode path.

One step = one Stage1 launch over the whole batch of the Qwen3-4B-shaped decode
workload (B=64, ctx 4096, 32/8 heads, D=128, KV block 16, 32 splits, SoA cache,
random-permuted block table), inputs resident in HBM.  Each timed launch follows a
1 GiB read sweep so the ~316 MB working set is not served from the 256 MB
Infinity Cache (cold cache), and is bracketed by HIP events on the launch stream
(created without the system-scope release fence, so the interval is the kernel's own
duration, as rocprofv3 reports it).

Prints ONE JSON line.  ``value`` is achieved HBM GB/s = algorithmic bytes per launch /
mean launch time; ``roofline`` relates it to MI355X's 8 TB/s; ``cpu_baseline`` is the
C oracle (a port of the reference Stage1 math) timed on this host's cores.

Beside the headline: the other Stage1 workloads of the same kernel (ragged B64, GQA-8
B8 x 32768), Stage2 at the headline shape, the reference-method warm number (100
back-to-back launches), the cache writer, the full decode step, the presets, and the
measured stream ceiling of this GPU (a device copy and a read-only sweep).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--layout soa|aos]
                       [--kernel auto|xdl|simple] [--no-cpu-baseline] [--calibrate-copy]
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import re
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "turboquant-cuda-decode_amd"))
# Kernel arguments in device memory (HIP reads this when it starts, before torch is
# imported below): with them in host memory every wave's first argument read crosses PCIe
# and a Stage1 launch at the headline shape takes ~1.6 us longer.
os.environ.setdefault("HIP_FORCE_DEV_KERNARG", "1")

METRIC = ("Stage1 µs + achieved HBM GB/s (% of peak), B64×ctx4096 Qwen3-4B shape, 1 GPU")
HBM_PEAK_GBS = 8000.0
FLUSH_BYTES = 1 << 30
# untimed launches before each side workload's timed ones: a process's first launches on
# new buffers run 1-3 us slow (the Stage1 headline: ~40 of them)
SIDE_WARMUP = 40
PROFILES = ROOT / "profiles"


def algorithmic_bytes(w) -> int:
    """Bytes a Stage1 launch must move: every live token's 134-byte K/V slot per kv-head,
    q_rot, the used block-table entries, seq_lens, the pair LUT, and the mid_o rows of
    the non-empty splits (D+1 floats per q-head)."""
    import numpy as np

    seq = w.seq_lens.astype(np.int64)
    bs, S = w.block_size, w.num_kv_splits
    kv = int(seq.sum()) * w.num_kv_heads * 134
    q = w.q_rot.nbytes
    bt = int(((seq + bs - 1) // bs).sum()) * 4
    split_len = (seq + S - 1) // S
    live = np.minimum(S, (seq + split_len - 1) // np.maximum(split_len, 1))
    mid = int(live.sum()) * w.num_q_heads * (w.head_dim + 1) * 4
    return kv + q + bt + w.seq_lens.nbytes + 256 * 2 * 4 + mid


def effective_kernel(layout: str, kernel: str) -> str:
    """The kernel a launch runs: ``auto`` picks the 16x16x32 MFMA kernel (xdl) for both
    cache layouts (this workload's GQA group and block size are ones it supports)."""
    return "xdl" if kernel == "auto" else kernel


def traffic_from_profile(name: str):
    """HBM bytes per launch from a committed rocprofv3 PMC summary, if one exists."""
    path = PROFILES / f"{name}_pmc.md"
    if not path.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9][0-9,.]*)", path.read_text())
    return float(m.group(1).replace(",", "")) if m else None


class HipEvents:
    """HIP events on the launch stream, created without the system-scope release fence
    (hipEventDisableSystemFence).  Two ways to take an interval: record a pair around a
    launch (includes the dispatch of the kernel and of the second marker), or hand a pair
    to the library's next kernel launch (``tq4_time_next_launch``: hipExtLaunchKernel
    stamps them with the kernel's own start and end, the duration rocprofv3 reports)."""

    NO_SYSTEM_FENCE = 0x20000000

    def __init__(self, stream: int):
        import ctypes

        self.ct = ctypes
        self.hip = None
        for name in ("libamdhip64.so.7", "libamdhip64.so"):
            try:
                self.hip = ctypes.CDLL(name)  # the runtime torch already loaded
                break
            except OSError:
                continue
        if self.hip is None:
            raise RuntimeError("libamdhip64 not found")
        self.stream = ctypes.c_void_p(stream)

    def pair(self):
        evs = []
        for _ in range(2):
            e = self.ct.c_void_p()
            rc = self.hip.hipEventCreateWithFlags(self.ct.byref(e), self.ct.c_uint(self.NO_SYSTEM_FENCE))
            if rc != 0:
                raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
            evs.append(e)
        return evs

    def record(self, e):
        if self.hip.hipEventRecord(e, self.stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def stamp_next_launch(self, a, b):
        from tq4_decode import _lib

        if _lib.load().tq4_time_next_launch(a, b) != 0:
            raise RuntimeError("tq4_time_next_launch failed")

    def elapsed_ms(self, a, b) -> float:
        ms = self.ct.c_float()
        if self.hip.hipEventElapsedTime(self.ct.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def destroy(self, *evs):
        for e in evs:
            self.hip.hipEventDestroy(e)


def store_times(dev, flush, timer, reps=30, only=None, bits=(4, 4), slots_mode="random"):
    """Cache writer (SoA, bf16 K/V, norm correction) cold, kernel duration: one decode step
    (64 tokens), a prefill chunk (8192 tokens) and a long prefill (65536 tokens, 343 MB: the
    writer's steady state), 8 kv-heads.  ``bits``: key / value bits
    (4/4: tq4_store; 3/4 and 3/3: tq4_store_preset).  Bytes per (token, kv-head): 2 x 256
    read + the slot written, plus 4 of slot mapping per token.  ``slots_mode``: "random"
    (the tokens scattered over the block pool: each block's metadata fields get their tokens
    from different workgroups) or "contiguous" (token t in slot t: blocks filled in order,
    as a prefill of one sequence fills them)."""
    import numpy as np
    import torch

    from tq4_decode import codebook, ops, workloads

    rng = np.random.default_rng(7)
    kb, vb = bits
    slot = ops.slot_bytes_preset(128, kb, vb)
    cents = codebook.centroids(128, kb)
    mids = ((cents[:-1] + cents[1:]) * np.float32(0.5)).astype(np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    rot, c, m = t(workloads.random_orthogonal(rng, 128)), t(cents), t(mids)
    out = {}
    for name, n_tok in (("decode_b64", 64), ("prefill_n8192", 8192), ("prefill_n65536", 65536)):
        if only is not None and name != only:
            continue
        key = torch.randn(n_tok, 8, 128, device=dev, dtype=torch.bfloat16)
        val = torch.randn(n_tok, 8, 128, device=dev, dtype=torch.bfloat16)
        n_blocks = (n_tok + 15) // 16 + 4
        cache = torch.zeros(n_blocks, 16, 8, slot, dtype=torch.uint8, device=dev)
        if slots_mode == "contiguous":
            slots = torch.arange(n_tok, device=dev, dtype=torch.int32)
        else:
            slots = torch.randperm(n_blocks * 16, device=dev)[:n_tok].to(torch.int32)
        times = []
        for i in range(reps + SIDE_WARMUP):
            flush.sum()
            a, b = timer.pair()
            timer.stamp_next_launch(a, b)  # the kernel's own start and end
            if bits == (4, 4):
                ops.store(key, val, cache, slots, rot, m, c)
            else:
                ops.store_preset(key, val, cache, slots, rot, m, c, key_bits=kb, value_bits=vb)
            torch.cuda.synchronize()
            if i >= SIDE_WARMUP:
                times.append(timer.elapsed_ms(a, b) * 1e3)
            timer.destroy(a, b)
        us = statistics.median(times)
        nbytes = n_tok * 8 * (2 * 256 + slot) + n_tok * 4
        out[f"{name}_us"] = round(us, 2)
        out[f"{name}_GBps"] = round(nbytes / us / 1e3, 1)
    return out


def full_decode_time(dev, flush, timer, reps=30):
    """Whole decode step (fp16 query -> rotation + pair LUT -> Stage1 -> Stage2 -> fp16
    out) at B=256 x ctx 2048, 32/8 heads, 16 splits, cold, timed by events around the
    step (it is two or more launches).  Bytes: KV of every token and kv-head + fp16 query
    in + fp16 output and LSE out + block table + rotation."""
    import numpy as np
    import torch

    from tq4_decode import ops, workloads

    w = workloads.full_b256_ctx2048()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    args = (t(w.query).half(), t(w.rotation_t), t(w.kv_cache), t(w.block_table), t(w.seq_lens),
            t(w.centroids), w.num_kv_splits)
    ws = ops.DecodeWorkspace(w.batch, w.num_q_heads, w.num_kv_splits, dev, torch.float16)
    times = []
    for i in range(reps + SIDE_WARMUP):
        flush.sum()
        a, b = timer.pair()
        timer.record(a)
        ops.full_decode(*args, workspace=ws)
        timer.record(b)
        torch.cuda.synchronize()
        if i >= SIDE_WARMUP:
            times.append(timer.elapsed_ms(a, b) * 1e3)
        timer.destroy(a, b)
    us = statistics.median(times)
    rows = w.batch * w.num_q_heads
    nbytes = (int(w.seq_lens.sum()) * w.num_kv_heads * 134 + rows * w.head_dim * 2 * 2 + rows * 4
              + w.block_table.nbytes + w.rotation_t.nbytes)
    return {"workload": "b256_ctx2048_32q8kv_s16_fp16", "us": round(us, 2),
            "GBps": round(nbytes / us / 1e3, 1), "bytes": nbytes}


# Stage1 side workloads of the 4-bit cache beside the headline
GQA_WORKLOADS = ("stage1_ragged_b64", "stage1_gqa8_b8_ctx32768", "stage1_gqa6_b64_ctx4096",
                 "stage1_gqa16_b64_ctx4096", "stage1_mha_b64_ctx4096", "stage1_gqa2_b64_ctx4096")

# preset Stage1 workloads: name -> (preset, SoA record bytes, metadata fields)
PRESET_WORKLOADS = {
    "stage1_fp8_b64_ctx4096": ("fp8", 192, 2),
    "stage1_k3v4_b64_ctx4096": ((3, 4), 112, 3),
    "stage1_3bit_b64_ctx4096": ((3, 3), 96, 3),
}


def stage1_preset_time(dev, flush, timer, name, reps=30, l2_resident=False):
    """Stage1 of a preset (FP8 keys: ``tq4_stage1_fp8``; 3-bit keys: ``tq4_stage1_preset``)
    at the B64 x ctx 4096 shape (32/8 heads, 32 splits), SoA, cold, kernel duration.
    Synthetic cache: random code bytes (E4M3 without NaN codes for FP8 keys), fp16 K norm /
    V scale / V zero in the ranges of the 4-bit workload.  Bytes: one slot per token and
    kv-head + query + block table + mid_o rows.  ``l2_resident``: every sequence's block
    table points at the same 16 blocks, warmed into L2 by a launch before each timed one
    (what the launch costs with HBM taken out; the bytes are the cold launch's)."""
    import numpy as np
    import torch

    from tq4_decode import codebook, ops, workloads

    preset, rec, fields = PRESET_WORKLOADS[name]
    w = workloads.qwen3_4b_b64_ctx4096()
    rng = np.random.default_rng(11)
    nb, bs, hk = w.kv_cache.shape[0], w.block_size, w.num_kv_heads
    slot = rec + 2 * fields
    cache = rng.integers(0, 256, (nb, bs * hk * slot), dtype=np.uint8)
    if preset == "fp8":
        k_region = cache[:, :bs * hk * rec].reshape(nb, bs * hk, rec)[:, :, :128]
        k_region[(k_region & 0x7F) == 0x7F] = 0x38  # no NaN codes
    meta = cache[:, bs * hk * rec:].view(np.float16).reshape(nb, hk, fields, bs)
    if fields == 3:
        meta[:, :, 0] = rng.uniform(0.5, 2.0, (nb, hk, bs)).astype(np.float16)
    meta[:, :, fields - 2] = rng.uniform(0.01, 0.1, (nb, hk, bs)).astype(np.float16)
    meta[:, :, fields - 1] = rng.uniform(-0.5, 0.5, (nb, hk, bs)).astype(np.float16)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    q, c = t(w.q_rot), t(cache.reshape(nb, bs, hk, slot))
    bt, sl = t(w.block_table), t(w.seq_lens)
    if l2_resident:
        bt = (torch.arange(w.block_table.shape[1], dtype=torch.int32, device=dev) % 16).repeat(w.batch, 1)
    mid = torch.empty(w.batch, w.num_q_heads, w.num_kv_splits, w.head_dim + 1, device=dev)
    if preset == "fp8":
        run = lambda: ops.stage1_fp8(q, c, bt, sl, mid)  # noqa: E731
    else:
        cents = t(codebook.centroids(w.head_dim, preset[0]).astype(np.float32))
        run = lambda: ops.stage1_preset(q, c, bt, sl, cents, mid, key_bits=preset[0],  # noqa: E731
                                        value_bits=preset[1])
    times = []
    for i in range(reps + SIDE_WARMUP):
        if l2_resident:
            run()
        else:
            flush.sum()
        a, b = timer.pair()
        timer.stamp_next_launch(a, b)
        run()
        torch.cuda.synchronize()
        if i >= SIDE_WARMUP:
            times.append(timer.elapsed_ms(a, b) * 1e3)
        timer.destroy(a, b)
    us = statistics.median(times)
    nbytes = (int(w.seq_lens.sum()) * hk * slot + w.q_rot.nbytes + w.block_table.nbytes
              + mid.numel() * 4)
    return {"us": round(us, 2), "GBps": round(nbytes / us / 1e3, 1), "bytes": nbytes}


def stage1_workload_time(dev, flush, timer, w, reps=30, kernel="auto"):
    """Stage1 (SoA; ``kernel``: auto, xdl or simple) of another 4-bit workload, cold, kernel
    duration (median of ``reps``); bytes as ``algorithmic_bytes``."""
    import numpy as np
    import torch

    from tq4_decode import ops

    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    q, c, bt, sl, lut = t(w.q_rot), t(w.kv_cache), t(w.block_table), t(w.seq_lens), t(w.pair_lut)
    mid = torch.empty(w.batch, w.num_q_heads, w.num_kv_splits, w.head_dim + 1, device=dev)
    times = []
    for i in range(reps + SIDE_WARMUP):
        flush.sum()
        a, b = timer.pair()
        timer.stamp_next_launch(a, b)
        ops.stage1(q, c, bt, sl, lut, mid, kernel=kernel)
        torch.cuda.synchronize()
        if i >= SIDE_WARMUP:
            times.append(timer.elapsed_ms(a, b) * 1e3)
        timer.destroy(a, b)
    us = statistics.median(times)
    nbytes = algorithmic_bytes(w)
    gbs = nbytes / us / 1e3
    return {"us": round(us, 2), "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "bytes": nbytes}


def stage2_time(dev, flush, timer, w, mid, reps=30):
    """Stage2 over the headline's mid_o (B64 x 32 heads x 32 splits), fp32 output, cold,
    kernel duration.  Bytes: the mid_o rows read, the output rows and LSE written, seq_lens."""
    import numpy as np
    import torch

    from tq4_decode import ops

    sl = torch.from_numpy(np.ascontiguousarray(w.seq_lens)).to(dev)
    out = torch.empty(w.batch, w.num_q_heads, w.head_dim, device=dev)
    lse = torch.empty(w.batch, w.num_q_heads, device=dev)
    times = []
    for i in range(reps + SIDE_WARMUP):
        flush.sum()
        a, b = timer.pair()
        timer.stamp_next_launch(a, b)
        ops.stage2(mid, sl, out, lse)
        torch.cuda.synchronize()
        if i >= SIDE_WARMUP:
            times.append(timer.elapsed_ms(a, b) * 1e3)
        timer.destroy(a, b)
    us = statistics.median(times)
    nbytes = mid.numel() * 4 + out.numel() * 4 + lse.numel() * 4 + w.seq_lens.nbytes
    return {"us": round(us, 2), "GBps": round(nbytes / us / 1e3, 1), "bytes": nbytes,
            "shape": "B64 x 32 q-heads x 32 splits, fp32 out"}


def stream_ceiling(dev, timer, reps=10):
    """This GPU's streaming bandwidth, measured: a 2 x 1 GiB device copy (torch ``copy_``,
    bytes read + written) and a read-only sweep of 2 GiB (torch ``sum``), median of ``reps``,
    events around each launch (the 4 GiB working set is far beyond the Infinity Cache)."""
    import torch

    src = torch.empty(1 << 28, dtype=torch.float32, device=dev).uniform_()
    dst = torch.empty_like(src)
    big = torch.empty(1 << 29, dtype=torch.float32, device=dev).uniform_()
    out = {}
    for name, fn, nbytes in (("copy_GBps", lambda: dst.copy_(src), 2 * src.nbytes),
                             ("read_GBps", lambda: big.sum(), big.nbytes)):
        times = []
        for i in range(reps + 2):
            a, b = timer.pair()
            timer.record(a)
            fn()
            timer.record(b)
            torch.cuda.synchronize()
            if i >= 2:
                times.append(timer.elapsed_ms(a, b))
            timer.destroy(a, b)
        out[name] = round(nbytes / statistics.median(times) / 1e6, 1)
    del src, dst, big
    out["how"] = ("torch copy_ of 1 GiB (2 GiB moved) and torch sum over 2 GiB, events around "
                  "the launch, median of %d" % reps)
    return out


def cpu_baseline(w, threads: int, repeats: int = 3):
    """The reference's fp32 Stage1 math in PyTorch on the host cores (the oracle's
    vectorized restatement of tools/cuda_v1_diagnostic.py:106-224), whole workload."""
    import torch

    from oracle import torch_stage1

    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    times = []
    try:
        for _ in range(repeats):
            t0 = time.perf_counter()
            torch_stage1.stage1(w.q_rot, w.kv_cache, w.block_table, w.seq_lens, w.centroids,
                                w.num_kv_splits, num_kv_heads=w.num_kv_heads)
            times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(prev)
    t = statistics.median(times)
    return {"value": round(algorithmic_bytes(w) / t / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "seconds": round(t, 4),
            "sample": (f"whole workload ({w.batch} seqs x {int(w.seq_lens[0])} tokens, SoA): the "
                       f"reference's fp32 Stage1 math in PyTorch on the CPU (oracle/torch_stage1.py, "
                       f"restating tools/cuda_v1_diagnostic.py:106-224), {threads} torch threads, "
                       f"median of {repeats}")}


def cpu_baseline_c(w, threads: int, repeats: int = 3):
    """The C oracle (Triton V1 program restated, fp32, OpenMP) over the whole workload."""
    from oracle import native

    native.lib()
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        native.stage1(w.q_rot, w.kv_cache, w.block_table, w.seq_lens, w.centroids,
                      w.num_kv_splits, num_kv_heads=w.num_kv_heads, threads=threads)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"value": round(algorithmic_bytes(w) / t / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "seconds": round(t, 4),
            "sample": "whole workload, C oracle tq4o_stage1 (OpenMP), median of %d" % repeats}


def side_workload(args, dev) -> int:
    """One JSON line for a workload beside the headline (the writer or the full step)."""
    import torch

    flush = torch.empty(FLUSH_BYTES // 4, dtype=torch.float32, device=dev).uniform_()
    timer = HipEvents(torch.cuda.current_stream(dev).cuda_stream)
    if args.workload in PRESET_WORKLOADS:
        r = stage1_preset_time(dev, flush, timer, args.workload, reps=args.steps, l2_resident=args.l2_resident)
        us, gbs = r["us"], r["GBps"]
        preset = PRESET_WORKLOADS[args.workload][0]
        label = {"fp8": "FP8-key preset (turboquant_k8v4)", (3, 4): "3-bit-key preset (turboquant_k3v4_nc)",
                 (3, 3): "3-bit preset (turboquant_3bit_nc)"}[preset]
        metric = f"Stage1, {label}, B64 x ctx4096 Qwen3-4B shape: GB/s" + (
            " (L2-resident: every block table on 16 blocks)" if args.l2_resident else "")
        timing = "kernel start/end stamped by hipExtLaunchKernel events, median"
        dtype = ("e4m3 K, 4-bit V" if preset == "fp8" else f"{preset[0]}-bit K, {preset[1]}-bit V") + ", f32 math"
    elif args.workload.startswith("store_"):
        size = args.workload[len("store_"):]
        bits = (4, 4)
        for tag, b in (("k3v4_", (3, 4)), ("3bit_", (3, 3))):
            if size.startswith(tag):
                size, bits = size[len(tag):], b
        r = store_times(dev, flush, timer, reps=args.steps, only=size, bits=bits, slots_mode=args.slots)
        us, gbs = r[f"{size}_us"], r[f"{size}_GBps"]
        entry = "tq4_store" if bits == (4, 4) else f"tq4_store_preset {bits[0]}/{bits[1]}"
        metric = f"cache writer ({entry}, SoA, bf16 K/V, 8 kv-heads, {args.slots} slots) {size}: GB/s"
        timing = "kernel start/end stamped by hipExtLaunchKernel events, median"
        dtype = "bf16 in, f32 math"
    elif args.workload in GQA_WORKLOADS:
        from tq4_decode import workloads

        make = {"stage1_ragged_b64": workloads.ragged_b64, "stage1_gqa8_b8_ctx32768": workloads.gqa8_b8_ctx32768,
                "stage1_gqa6_b64_ctx4096": lambda: workloads.qwen3_4b_b64_ctx4096(num_q_heads=48),
                "stage1_gqa16_b64_ctx4096": lambda: workloads.qwen3_4b_b64_ctx4096(num_q_heads=128),
                "stage1_mha_b64_ctx4096": lambda: workloads.qwen3_4b_b64_ctx4096(num_q_heads=8),
                "stage1_gqa2_b64_ctx4096": lambda: workloads.qwen3_4b_b64_ctx4096(num_q_heads=16)}
        w = make[args.workload]()
        r = stage1_workload_time(dev, flush, timer, w, reps=args.steps, kernel=args.kernel)
        us, gbs = r["us"], r["GBps"]
        metric = {"stage1_ragged_b64": "Stage1, B64 ragged (seq_lens 512..8192), 32/8 heads, 32 splits: GB/s",
                  "stage1_gqa8_b8_ctx32768": "Stage1, B8 x ctx32768, 64/8 heads (GQA-8), 64 splits: GB/s",
                  "stage1_gqa6_b64_ctx4096": "Stage1, B64 x ctx4096, 48/8 heads (GQA-6), 32 splits: GB/s",
                  "stage1_gqa16_b64_ctx4096": "Stage1, B64 x ctx4096, 128/8 heads (GQA-16), 32 splits: GB/s",
                  "stage1_mha_b64_ctx4096": "Stage1, B64 x ctx4096, 8/8 heads (MHA), 32 splits: GB/s",
                  "stage1_gqa2_b64_ctx4096": "Stage1, B64 x ctx4096, 16/8 heads (GQA-2), 32 splits: GB/s"}[
            args.workload] + ("" if args.kernel == "auto" else f" ({args.kernel} kernel)")
        timing = "kernel start/end stamped by hipExtLaunchKernel events, median"
        dtype = "4-bit K/V, f32 math"
    elif args.workload == "stage1_l2_resident":
        import numpy as np

        from tq4_decode import ops, workloads

        # the headline launch with every sequence's block table pointing at the same 16 KV
        # blocks (274 KB, resident in every XCD's L2 after one launch): what the kernel costs
        # when HBM is taken out of the picture
        w = workloads.qwen3_4b_b64_ctx4096()
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
        q, sl, lut = t(w.q_rot), t(w.seq_lens), t(w.pair_lut)
        c = t(w.kv_cache if args.layout == "soa" else workloads.soa_to_aos(w.kv_cache, w.centroids, w.num_kv_heads))
        bt16 = (torch.arange(w.block_table.shape[1], dtype=torch.int32, device=dev) % 16).repeat(w.batch, 1)
        mid = torch.empty(w.batch, w.num_q_heads, w.num_kv_splits, w.head_dim + 1, device=dev)
        times = []
        for i in range(args.steps + SIDE_WARMUP):
            ops.stage1(q, c, bt16, sl, lut, mid, layout=args.layout)  # warms L2 with the 16 blocks
            a, b = timer.pair()
            timer.stamp_next_launch(a, b)
            ops.stage1(q, c, bt16, sl, lut, mid, layout=args.layout)
            torch.cuda.synchronize()
            if i >= SIDE_WARMUP:
                times.append(timer.elapsed_ms(a, b) * 1e3)
            timer.destroy(a, b)
        us = round(statistics.median(times), 2)
        gbs = round(algorithmic_bytes(w) / us / 1e3, 1)
        metric = (f"Stage1, headline shape ({args.layout.upper()}), every KV read an L2 hit (16 shared blocks): "
                  "headline bytes / time, GB/s")
        timing = "kernel start/end stamped by hipExtLaunchKernel events, median"
        dtype = "4-bit K/V, f32 math"
    elif args.workload == "stage2_b64_s32":
        import numpy as np

        from tq4_decode import ops, workloads

        w = workloads.qwen3_4b_b64_ctx4096()
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
        mid = torch.empty(w.batch, w.num_q_heads, w.num_kv_splits, w.head_dim + 1, device=dev)
        ops.stage1(t(w.q_rot), t(w.kv_cache), t(w.block_table), t(w.seq_lens), t(w.pair_lut), mid)
        r = stage2_time(dev, flush, timer, w, mid, reps=args.steps)
        us, gbs = r["us"], r["GBps"]
        metric = "Stage2 over the headline's mid_o (B64 x 32 heads x 32 splits), fp32 out: GB/s"
        timing = "kernel start/end stamped by hipExtLaunchKernel events, median"
        dtype = "f32"
    else:
        r = full_decode_time(dev, flush, timer, reps=args.steps)
        us, gbs = r["us"], r["GBps"]
        metric = "full decode step B256 x ctx2048 (rotation + Stage1 + Stage2): GB/s"
        timing = "events recorded around the step, median"
        dtype = "fp16 in/out, f32 math"
    print(json.dumps({"metric": metric, "value": gbs, "unit": "GB/s", "n_gpus": 1,
                      "steps": args.steps, "ms_per_step": round(us / 1e3, 5),
                      "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                      "dtype": dtype, "data": "synthetic",
                      "config": {"workload": args.workload, **({"l2_resident": True} if args.l2_resident else {})},
                      "timing": timing,
                      # an L2-resident run reads no HBM: its GB/s are the cold launch's bytes over its time
                      "pct_of_hbm_peak": None if args.l2_resident else round(100 * gbs / HBM_PEAK_GBS, 2)}))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # a process's first ~40 cold launches run 1-3 us slow (63-65 us, then 62); 100 untimed
    # launches put the timed ones in the steady state
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--layout", default="soa", choices=["soa", "aos"])
    ap.add_argument("--slots", default="random", choices=["random", "contiguous"],
                    help="writer workloads: token slots scattered over the pool, or in order")
    ap.add_argument("--kernel", default="auto", choices=["auto", "simple", "xdl"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--l2-resident", action="store_true",
                    help="preset workloads: every block table on 16 blocks kept in L2 (HBM taken out)")
    ap.add_argument("--no-variants", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 256 MiB device copy (PMC byte-counter calibration)")
    ap.add_argument("--workload", default="stage1",
                    choices=["stage1", "store_decode_b64", "store_prefill_n8192", "store_prefill_n65536",
                             "full_decode_b256",
                             "store_k3v4_prefill_n8192", "store_3bit_prefill_n8192", "stage1_ragged_b64",
                             "stage1_gqa8_b8_ctx32768", "stage1_gqa6_b64_ctx4096", "stage1_gqa16_b64_ctx4096",
                             "stage1_mha_b64_ctx4096", "stage1_gqa2_b64_ctx4096",
                             "stage2_b64_s32", "stage1_l2_resident",
                             *PRESET_WORKLOADS],
                    help="stage1: the headline (default); the others time only that workload "
                         "(--steps cold launches) and print its own JSON line, e.g. for a profile")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this path has no multi-GPU form "
              f"(--gpus {args.gpus}, WORLD_SIZE {world}); run with --gpus 1", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from tq4_decode import ops, workloads

    dev = torch.device("cuda:0")
    if args.workload != "stage1":
        return side_workload(args, dev)
    w = workloads.qwen3_4b_b64_ctx4096()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    q, bt, sl, lut = t(w.q_rot), t(w.block_table), t(w.seq_lens), t(w.pair_lut)
    caches = {"soa": t(w.kv_cache)}
    if args.layout == "aos" or not args.no_variants:
        caches["aos"] = t(workloads.soa_to_aos(w.kv_cache, w.centroids, w.num_kv_heads))
    mid = torch.empty(w.batch, w.num_q_heads, w.num_kv_splits, w.head_dim + 1, device=dev)
    flush = torch.empty(FLUSH_BYTES // 4, dtype=torch.float32, device=dev).uniform_()
    nbytes = algorithmic_bytes(w)

    def launch(layout, kernel):
        ops.stage1(q, caches[layout], bt, sl, lut, mid, layout=layout, kernel=kernel)

    timer = HipEvents(torch.cuda.current_stream(dev).cuda_stream)

    def cold_times(layout, kernel, steps, warmup, stamped=True):
        """Durations (ms) of `steps` cold launches: the kernel's own start/end stamps, or
        (stamped=False) events recorded around each launch.  The events are created before
        the warm-up, so the GPU does not sit idle (and clock down) between the warm-up and
        the timed launches."""
        ev = [timer.pair() for _ in range(steps)]
        for _ in range(warmup):
            flush.sum()
            launch(layout, kernel)
        torch.cuda.synchronize()
        for a, b in ev:
            flush.sum()  # 1 GiB read sweep: evicts L2 and the Infinity Cache
            if stamped:
                timer.stamp_next_launch(a, b)
                launch(layout, kernel)
            else:
                timer.record(a)
                launch(layout, kernel)
                timer.record(b)
        torch.cuda.synchronize()
        out = [timer.elapsed_ms(a, b) for a, b in ev]
        for e in ev:
            timer.destroy(*e)
        return out

    def warm_time(layout, kernel, iters=100, rounds=5):
        res = []
        a, b = timer.pair()
        for _ in range(rounds):
            for _ in range(10):
                launch(layout, kernel)
            timer.record(a)
            for _ in range(iters):
                launch(layout, kernel)
            timer.record(b)
            torch.cuda.synchronize()
            res.append(timer.elapsed_ms(a, b) / iters)
        timer.destroy(a, b)
        return statistics.median(res)

    torch.cuda.synchronize()
    ms = cold_times(args.layout, args.kernel, args.steps, args.warmup)
    around = cold_times(args.layout, args.kernel, 50, 2, stamped=False)
    mean_ms = statistics.fmean(ms)
    med_ms = statistics.median(ms)
    gbs = nbytes / (mean_ms * 1e-3) / 1e9
    kname = f"stage1_{effective_kernel(args.layout, args.kernel)}_{args.layout}_qwen3_4b_b64_ctx4096"
    traffic = traffic_from_profile(kname)
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(mean_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded CPU generator: uniform random 4-bit code bytes, fp16 "
                "norm/scale/zero, random-permuted block table)",
        "config": {"workload": "qwen3_4b_b64_ctx4096", "batch": w.batch, "ctx": 4096,
                   "q_heads": w.num_q_heads, "kv_heads": w.num_kv_heads, "head_dim": w.head_dim,
                   "block_size": w.block_size, "num_kv_splits": w.num_kv_splits,
                   "layout": args.layout, "kernel": effective_kernel(args.layout, args.kernel),
                   "cache": "cold (1 GiB sweep)"},
        "stage1_us": round(mean_ms * 1e3, 2),
        "stage1_us_median": round(med_ms * 1e3, 2),
        "stage1_us_with_dispatch": round(statistics.fmean(around) * 1e3, 2),
        "timing": "kernel start/end stamped by hipExtLaunchKernel events (the interval "
                  "rocprofv3 reports); stage1_us_with_dispatch: mean of 50 further cold "
                  "launches timed by events recorded around each launch",
        "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "algorithmic_bytes": nbytes,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic},
    }
    # the reference's method: 100 back-to-back launches (benchmarks/stage1.py:32-43); the
    # 316 MB working set then partly stays in the 256 MB Infinity Cache
    result["stage1_us_warm"] = round(warm_time(args.layout, args.kernel) * 1e3, 2)
    if not args.no_variants:
        var = {}
        for layout, kernel in (("aos", "xdl"), ("soa", "simple")):
            vm = statistics.fmean(cold_times(layout, kernel, 50, 5))
            var[f"{layout}_{kernel}_cold_us"] = round(vm * 1e3, 2)
            var[f"{layout}_{kernel}_warm_us"] = round(warm_time(layout, kernel) * 1e3, 2)
        result["variants"] = var
        launch("soa", "xdl")  # mid_o of the headline for Stage2
        result["stage2_b64_s32"] = stage2_time(dev, flush, timer, w, mid)
        del caches
        result["stage1_ragged_b64"] = stage1_workload_time(dev, flush, timer, workloads.ragged_b64())
        result["stage1_gqa8_b8_ctx32768"] = stage1_workload_time(dev, flush, timer,
                                                                 workloads.gqa8_b8_ctx32768())
        result["stream_ceiling"] = stream_ceiling(dev, timer)
        result["store"] = store_times(dev, flush, timer)
        result["full_decode"] = full_decode_time(dev, flush, timer)
        # Stage1 of the other presets at the same B64 x 4096 shape (each in its own layout)
        result["presets"] = {name: stage1_preset_time(dev, flush, timer, name, reps=30)
                             for name in PRESET_WORKLOADS}
    if args.calibrate_copy:
        src = torch.empty(1 << 26, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            flush.sum()
            dst.copy_(src)
        torch.cuda.synchronize()
        result["calibration_copy_bytes"] = src.nbytes
    if not args.no_cpu_baseline:
        # the host cores this process may use, capped by OMP_NUM_THREADS when it is set (a
        # GPU's share of a shared host)
        try:
            threads = len(os.sched_getaffinity(0))
        except AttributeError:
            threads = os.cpu_count() or 1
        cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
        threads = min(threads, cap) if cap > 0 else threads
        result["cpu_baseline"] = cpu_baseline(w, threads)
        result["cpu_baseline_c"] = cpu_baseline_c(w, threads)
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
