"""Generate tests/golden/cast_digests.npz: for every scale that per-tensor current scaling can
produce from bf16 data (RN32(a / 448) for every positive finite bf16 magnitude a, plus 1.0),
the digest of the e4m3 cast of all 65536 bf16 bit patterns, computed by the C restatement in
oracle/fp8_cast.c. Run from the repo root: python tests/golden/make_cast_digests.py
"""
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import c_oracle  # noqa: E402
from oracle.fp8_oracle import reachable_scales  # noqa: E402


def main():
    lib = c_oracle()
    scales = reachable_scales()
    out = np.zeros(scales.size, dtype=np.uint64)
    t0 = time.time()
    lib.oracle_cast_digests(scales.ctypes.data, scales.size, out.ctypes.data, os.cpu_count() or 1)
    print(f"{scales.size} scales in {time.time() - t0:.1f}s")
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cast_digests.npz")
    np.savez_compressed(path, scales=scales, digests=out)
    print("wrote", path)


if __name__ == "__main__":
    main()
