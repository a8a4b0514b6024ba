"""Write the reference Lloyd-Max codebook as a golden vector.

The float32 bits of ``get_centroids(d, bits)`` (``reference/centroids.py:82-86``) are
the one output on this path that no closed form or invariant fixes exactly, so
this script imports that pure-Python function from the reference checkout (read
only) where the reference checkout is present and records its output.  The tests
never run this script; they only read the JSON it wrote.

Usage: ``python tests/golden/make_centroids_golden.py [/root/reference]``
"""
from __future__ import annotations

import importlib.util
import json
import pathlib
import sys

import numpy as np

REF = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
OUT = pathlib.Path(__file__).with_name("centroids_d128_b4.json")


def main() -> None:
    spec = importlib.util.spec_from_file_location("_ref_centroids", REF / "reference" / "centroids.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    cases = []
    for d, bits in ((128, 4), (64, 4), (128, 3)):
        cents, bounds = mod.solve_lloyd_max(d, bits)
        c = cents.numpy().astype(np.float32)
        b = bounds.numpy().astype(np.float32)
        cases.append({
            "d": d,
            "bits": bits,
            "centroids_hex": [f"{v:08x}" for v in c.view(np.uint32).tolist()],
            "boundaries_hex": [f"{v:08x}" for v in b.view(np.uint32).tolist()],
            "centroids": c.tolist(),
        })
    OUT.write_text(json.dumps({"source": "reference/centroids.py:31-86", "cases": cases}, indent=1) + "\n")
    print("wrote", OUT)


if __name__ == "__main__":
    main()
