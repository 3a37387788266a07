"""VALU issue rates of the instructions the update's hot path chooses between (the probe is
tests/gpu_checks/issue_rate.hip): each instruction's time per wave instruction per SIMD,
relative to v_add_u32's, is printed, and the one relation the kernels rely on is asserted: the
stochastic-rounding converters (v_cvt_sr_bf16_f32, v_cvt_sr_f16_f32) take at least twice an
integer add's issue time, so the bf16 and fp16 stochastic roundings are integer adds
(csrc/lv_exact.h). Measured on MI355X: about 3.1x."""
from __future__ import annotations

import ctypes
import os

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "gpu_checks", "libissuerate.so")


def test_sr_converters_issue_slower_than_an_integer_add():
    import torch

    if not os.path.exists(LIB):
        pytest.skip("libissuerate.so is not built")
    torch.cuda.init()
    L = ctypes.CDLL(LIB)
    L.lv_rate_name.restype = ctypes.c_char_p
    L.lv_rate_measure.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                  ctypes.POINTER(ctypes.c_int)]
    rates = {}
    for op in range(L.lv_rate_count()):
        ns, khz = ctypes.c_double(), ctypes.c_int()
        assert L.lv_rate_measure(op, 64, 3, ctypes.byref(ns), ctypes.byref(khz)) == 0
        name = L.lv_rate_name(op).decode()
        rates[name] = ns.value
        print(f"{name:22s} {ns.value * khz.value / 1e6:6.2f} cycles at the reported clock", flush=True)
    base = rates["v_add_u32"]
    for name, ns in rates.items():
        print(f"{name:22s} {ns / base:5.2f} x v_add_u32")
    assert rates["v_cvt_sr_bf16_f32"] >= 2.0 * base
    assert rates["v_cvt_sr_f16_f32"] >= 2.0 * base
