"""The library's exact helpers (luminamoon_amd/csrc/lv_exact.h) against their reference definitions
on every input (the check program is tests/gpu_checks/exact_check.hip):

* f32 -> f16 on the hardware converter with the reference's saturation, against the integer
  algorithm of prng.rs:29-67: all 2^32 inputs bit for bit;
* f16 -> f32 against prng.rs:69-96: all 2^16 inputs, where only the signalling NaNs may differ
  (the hardware returns them quietened, same sign);
* sqrt_rn against the IEEE square root (the compiler's correctly rounded one, as Rust's
  f32::sqrt): all 2^32 inputs bit for bit, NaN for NaN;
* xor_fold16 against (z ^ (z >> 16)) & 0xFFFF: all 2^32 inputs.
"""
from __future__ import annotations

import ctypes
import os

import pytest
import torch

pytestmark = pytest.mark.gpu


def _lib():
    from tests.gpu_checks import build as B

    if not os.path.exists(B.EXACT_LIB):
        B.build()
    lib = ctypes.CDLL(B.EXACT_LIB)
    lib.exact_check.restype = ctypes.c_int
    lib.exact_check.argtypes = [ctypes.POINTER(ctypes.c_ulonglong), ctypes.POINTER(ctypes.c_uint32)]
    return lib


def test_exact_helpers_on_every_input():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    counts = (ctypes.c_ulonglong * 5)()
    ex = (ctypes.c_uint32 * 40)()
    print("[case] exact helpers, 3 x 2^32 + 2^16 inputs", flush=True)
    assert _lib().exact_check(counts, ex) == 0
    assert counts[0] == 0, ("f32->f16", [hex(x) for x in ex[0:8]])
    assert counts[1] == 0, ("f16->f32", [hex(x) for x in ex[8:16]])
    # 2 signs x (2^9 - 1) signalling-NaN payloads (exponent all ones, quiet bit clear, mantissa > 0)
    assert counts[2] <= 2 * 511
    assert counts[3] == 0, ("sqrt_rn", [hex(x) for x in ex[24:32]])
    assert counts[4] == 0, ("xor_fold16", [hex(x) for x in ex[32:40]])
