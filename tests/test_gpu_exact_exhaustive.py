"""The library's exact helpers (luminamoon_amd/csrc/lv_exact.h) against their reference definitions
on every input (the check program is tests/gpu_checks/exact_check.hip):

* f32 -> f16 on the hardware converter with the reference's saturation, against the integer
  algorithm of prng.rs:29-67: all 2^32 inputs bit for bit;
* f16 -> f32 against prng.rs:69-96: all 2^16 inputs, where only the signalling NaNs may differ
  (the hardware returns them quietened, same sign);
* sqrt_rn against the IEEE square root (the compiler's correctly rounded one, as Rust's
  f32::sqrt): all 2^32 inputs bit for bit, NaN for NaN;
* xor_fold16 against (z ^ (z >> 16)) & 0xFFFF: all 2^32 inputs;
* sr_fp16_val, the library's whole fp16 stochastic rounding (the domain's integer add, the wave's
  switch to the integer recipe outside it, then pack_f16_rtz), against prng.rs:98-130 with the
  noise of prng.rs:21-26: all 2^32 inputs x 2 hash inputs;
* sr_bf16_checked (one integer add, with the out-of-range and NaN inputs replaced first when a
  lane of the wave has one) against the reference's integer recipe (prng.rs:137-160): all 2^32
  inputs x 6 noise values;
* sqrt_rn_normal (v_rsq_f32 and one correction, no rescaling) against the IEEE square root on
  every input of its domain, and sqrt_rn_positive (the same without its zero, infinity and NaN
  select) on every input from 2^-96 to the largest finite f32;
* pack_f16_rtz against f32 -> f16 RNE on every finite f16 value and the canonical NaNs (the
  reference's fp16 quantisation never yields an infinity);
* sr_f16_add + pack_f16_rtz (the integer add and round-toward-zero pack) against the reference's
  integer recipe (prng.rs:98-130) on every input of its domain (+-0 and 2^-14 <= |x| < 65504) x 6
  noise values, and its domain test on all 2^32 inputs;
* the guarded fast divisions (div_envelope, div_bound: v_rcp_f32 and the IEEE sequence's own
  fma refinement without its scaling and fix-up steps, taken when a wave-uniform test proves
  them unneeded) against IEEE division: every 2^32 numerator with denominators from n/2 to 2^25,
  T2's clm / env from its own formula for every gradient bit pattern, and the rational bound for
  every step value;
* div_unscaled itself (one Newton step on v_rcp_f32's reciprocal and one correction) against IEEE
  division on all 2^46 pairs of significands in [1, 2), with v_rcp_f32's scaling by the
  denominator's exponent checked for every significand and exponent in [-125, 125]: under the
  guards' conditions every other operand pair is one of these scaled by powers of two.
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
    counts = (ctypes.c_ulonglong * 11)()
    ex = (ctypes.c_uint32 * 88)()
    print("[case] exact helpers, 2^32 inputs x 18 checks + 2 x 2^16", flush=True)
    assert _lib().exact_check(counts, ex) == 0
    assert counts[0] == 0, ("f32->f16", [hex(x) for x in ex[0:8]])
    assert counts[1] == 0, ("f16->f32", [hex(x) for x in ex[8:16]])
    # 2 signs x (2^9 - 1) signalling-NaN payloads (exponent all ones, quiet bit clear, mantissa > 0)
    assert counts[2] <= 2 * 511
    assert counts[3] == 0, ("sqrt_rn", [hex(x) for x in ex[24:32]])
    assert counts[4] == 0, ("xor_fold16", [hex(x) for x in ex[32:40]])
    assert counts[5] == 0, ("sr_fp16_val", [hex(x) for x in ex[40:48]])
    assert counts[6] == 0, ("sr_bf16_checked", [hex(x) for x in ex[48:56]])
    assert counts[7] == 0, ("sqrt_rn_normal / sqrt_rn_positive", [hex(x) for x in ex[56:64]])
    assert counts[8] == 0, ("pack_f16_rtz", [hex(x) for x in ex[64:72]])
    assert counts[9] == 0, ("sr_f16_add", [hex(x) for x in ex[72:80]])
    # domain size, sampled where the low 16 bits are zero: per sign, the zero and the multiples of
    # 2^16 in [0x38800000, 0x477FE000)
    per_sign = 1 + len(range(0x38800000, 0x477FE000, 65536))
    assert counts[10] == 2 * per_sign


def test_guarded_fast_divisions_equal_ieee_division():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    lib = _lib()
    lib.div_check.restype = ctypes.c_int
    lib.div_check.argtypes = [ctypes.POINTER(ctypes.c_ulonglong), ctypes.POINTER(ctypes.c_uint32)]
    counts = (ctypes.c_ulonglong * 4)()
    ex = (ctypes.c_uint32 * 32)()
    print("[case] guarded fast divisions, 2^32 inputs x 5 quotients", flush=True)
    assert lib.div_check(counts, ex) == 0
    assert counts[0] == 0, ("div_envelope", [hex(x) for x in ex[0:8]])
    assert counts[1] == 0, ("T2 clm / env", [hex(x) for x in ex[8:16]])
    assert counts[2] == 0, ("div_bound", [hex(x) for x in ex[16:24]])
    # numerators with 2^-100 <= |n| <= 2^25: 2 signs x 125 binades x 2^23, sampled one in 2^16,
    # with at least 2 of the 3 denominators in range each
    assert counts[3] >= 2 * 125 * 128 * 2


def test_one_correction_division_on_every_significand_pair():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    lib = _lib()
    lib.div_pair_check.restype = ctypes.c_int
    lib.div_pair_check.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int,
                                   ctypes.POINTER(ctypes.c_ulonglong), ctypes.POINTER(ctypes.c_uint32)]
    chunk = 1 << 20
    for first in range(0, 1 << 23, chunk):
        counts = (ctypes.c_ulonglong * 4)()
        ex = (ctypes.c_uint32 * 16)()
        print(f"[case] div_unscaled, denominators {first:#x}..{first + chunk - 1:#x} x 2^23 numerators", flush=True)
        assert lib.div_pair_check(first, chunk, 1 if first == 0 else 0, counts, ex) == 0
        assert counts[0] == 0, ("div_unscaled (dm, nm)", [hex(x) for x in ex[0:8]])
        assert counts[1] == chunk << 23
        if first == 0:
            assert counts[2] == 0, ("v_rcp_f32 scaling (dm, e + 128)", [hex(x) for x in ex[8:16]])
            assert counts[3] == (1 << 23) * 251
