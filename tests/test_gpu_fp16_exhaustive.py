"""The library's fp16 conversions (hardware converters plus the reference's saturation,
luminamoon_amd/csrc/lv_fp16.h) against the reference's integer algorithms (prng.rs:29-96,
restated in tests/gpu_checks/fp16_check.hip), on every input: all 2^32 f32 -> f16 conversions
must agree bit for bit; of the 2^16 f16 -> f32 conversions only the signalling NaNs may differ
(the hardware returns them quietened, same sign), and nothing else."""
from __future__ import annotations

import ctypes
import os

import pytest
import torch

pytestmark = pytest.mark.gpu


def _lib():
    from tests.gpu_checks import build as B

    if not os.path.exists(B.FP16_LIB):
        B.build()
    lib = ctypes.CDLL(B.FP16_LIB)
    lib.fp16_check.restype = ctypes.c_int
    lib.fp16_check.argtypes = [ctypes.POINTER(ctypes.c_ulonglong), ctypes.POINTER(ctypes.c_uint32)]
    return lib


def test_fp16_conversions_on_every_input():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    counts = (ctypes.c_ulonglong * 3)()
    examples = (ctypes.c_uint32 * 16)()
    print("[case] fp16 conversions, 2^32 + 2^16 inputs", flush=True)
    assert _lib().fp16_check(counts, examples) == 0
    f32_to_f16_bad, f16_to_f32_bad, snan_quietened = counts[0], counts[1], counts[2]
    assert f32_to_f16_bad == 0, [hex(x) for x in examples[:8]]
    assert f16_to_f32_bad == 0, [hex(x) for x in examples[8:16]]
    # 2 signs x (2^9 - 1) signalling-NaN payloads (exponent all ones, quiet bit clear, mantissa > 0)
    assert snan_quietened <= 2 * 511
