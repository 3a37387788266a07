"""Builds the GPU check libraries of the tests (hipcc, gfx950, the library's own flags): the exact
helpers' exhaustive check."""
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


def _build_one(src: str, lib: str, verbose: bool) -> None:
    from luminamoon_amd import build_ext

    tmp = lib + ".tmp"
    cmd = [build_ext.hipcc(), *build_ext.HIPCC_FLAGS, "-I", os.path.join(ROOT, "luminamoon_amd", "csrc"),
           "-I", os.path.join(ROOT, "include"), src, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed building {src}")
    os.replace(tmp, lib)


def build(verbose: bool = False) -> str:
    """Builds libexactcheck.so; returns its path."""
    _build_one(EXACT_SRC, EXACT_LIB, verbose)
    return EXACT_LIB


if __name__ == "__main__":
    print(build(verbose=True))
