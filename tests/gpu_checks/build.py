"""Builds the GPU check libraries of the tests (hipcc, gfx950, the library's own flags)."""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

EXACT_SRC = os.path.join(HERE, "exact_check.hip")
EXACT_LIB = os.path.join(HERE, "libexactcheck.so")


def build(verbose: bool = False) -> str:
    from luminamoon_amd import build_ext

    tmp = EXACT_LIB + ".tmp"
    cmd = [build_ext.hipcc(), *build_ext.HIPCC_FLAGS, "-I", os.path.join(ROOT, "luminamoon_amd", "csrc"),
           "-I", os.path.join(ROOT, "include"), EXACT_SRC, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed building {EXACT_SRC}")
    os.replace(tmp, EXACT_LIB)
    return EXACT_LIB


if __name__ == "__main__":
    print(build(verbose=True))
