"""CPU oracle for the TurboQuant ``turboquant_4bit_nc`` decode path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports, links or
executes anything under ``oracle/``.  Only ``tests/``, ``__graft_entry__.smoke()``
(as the checker) and the ``cpu_baseline`` leg of ``bench.py`` may use it.

Contents (each function cites the reference ``file:line`` it restates):

* ``layout``     byte layout of the SoA / AoS paged cache
                 (``baseline/common.py:38-225``, ``:554-672``).
* ``codebook``   Lloyd-Max codebook and pair LUT
                 (``reference/centroids.py:18-86``, ``baseline/common.py:232-257``).
* ``stage1``     numpy float64 restatement of Stage1 (SoA and AoS), Stage2 and
                 the full decode step (``reference/soa_decode_v1.py:95-314``,
                 ``reference/aos_decode.py:87-313``, ``baseline/stage2.py:26-55``,
                 ``reference/soa_decode_v1.py:532-538``).
* ``store``      numpy restatement of the SoA / AoS cache writers, used to build
                 the store-semantics fixture (``reference/soa_store.py:26-116``,
                 ``:223-373``, ``:482-485``; ``reference/aos_store.py:317-325``).
* ``tq4_oracle.c`` + ``native``  a plain-C float32 restatement of the Triton V1
                 Stage1 programs (one program per (batch, q-head, split), BLOCK_KV=4
                 online softmax) and of Stage2; it is the full-size checker.
* ``torch_stage1`` the reference's fp32 Stage1 math in PyTorch on the CPU
                 (``tools/cuda_v1_diagnostic.py:106-224``), vectorized over the heads
                 and splits of a sequence; the CPU baseline of ``bench.py``.

Pins (what checks each function against something other than itself) live in
``tests/test_oracle_*.py``.  Parity status per function is listed in the module
docstrings; a function without an independent check says "parity unpinned".
"""
