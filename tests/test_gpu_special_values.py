"""Non-finite and extreme inputs on the GPU, against the oracle's scalar core (the reference's
default CPU backend).

* Gradients: NaN, +-inf, values past the 1e38 finite cut and past the +-1e18 clamp, the largest
  finite values, subnormals and signed zeros (sanitize_gradient, math.rs:5-11).
* Corrupted state: NaN and +-inf in m, v and p, and subnormal and huge p. These must propagate
  the way the scalar core propagates them:
  - clamp_defect passes NaN through (math.rs:13-16);
  - Rust's max/min drop a NaN operand;
  - stochastic rounding takes its NaN path for bf16 (prng.rs:137-160);
  - the cautious mask tests u*g > 0, which is false for NaN.

The special values sit in whole units (the vector path) and in the partial last unit (the
per-element path). Elements are compared bit for bit, with two exceptions where IEEE 754 leaves
the result open:

- Any two NaNs count as equal; the NaN positions must still match exactly. IEEE 754 does not
  fix which payload an operation returns from two NaN operands, so x86 and gfx950 may differ.
- fp16 params may differ in sign at +-65504. IEEE 754 leaves the sign of a NaN unspecified: for
  an invalid operation (inf/inf, inf - inf, 0 * inf) x86 returns the default NaN with the sign
  bit set (0xFFC00000), while gfx950 returns it with the sign bit clear (0x7FC00000). The
  reference's fp16 stochastic rounding clamps a NaN to the largest finite fp16 and keeps its
  sign (prng.rs:98-130), so a param update that is NaN becomes -65504 on x86 and +65504 here.
  The reference's own GPU path produces the positive default NaN as well.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from tests.parity_util import TensorSet, bits, group_dict, oracle_config

pytestmark = pytest.mark.gpu

NAN, INF = float("nan"), float("inf")
FLT_MAX = float(np.finfo(np.float32).max)
GRAD_SPECIALS = [NAN, INF, -INF, 1e38, -1e38, FLT_MAX, 9.9e37, -1e19, 1e18, -1e18, 1e-40, -1e-45,
                 0.0, -0.0, 1.1754944e-38, -NAN]
M_SPECIALS = [INF, -INF, NAN, 1e38, -3e38, 1e-40, -0.0]
V_SPECIALS = [INF, NAN, 1e38, 1e-40, 0.0]
P_SPECIALS = [NAN, INF, -INF, 1e-40, -0.0, 3e38, -3e38, 1e30]

# tensor 0: 4,133 elements = whole units plus a 37-element tail; tensor 1: 1,000 (one partial unit)
SIZES = [4096 + 37, 1000]
POSITIONS = [[3, 700, 1029, 2050, 3000, 4097, 4116, 4132], [0, 1, 500, 998, 999]]


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


def _inject(t: torch.Tensor, positions, values, shift: int = 0) -> None:
    for k, i in enumerate(positions):
        t[i] = values[(k + shift) % len(values)]


F16_MAX_BITS = 0x7BFF


def _assert_same(a: torch.Tensor, b: torch.Tensor, label: str) -> int:
    """Bitwise equal where not NaN, NaN at the same positions, and for fp16 a sign difference
    allowed at +-65504 (the sign of a default NaN); returns how many elements took an exception."""
    a, b = a.detach().cpu(), b.detach().cpu()
    na, nb = torch.isnan(a.float()), torch.isnan(b.float())
    assert torch.equal(na, nb), f"{label}: NaN at {np.nonzero(na.numpy())[0][:8]} vs {np.nonzero(nb.numpy())[0][:8]}"
    ba, bb = bits(a), bits(b)
    keep = ~na.numpy()
    if a.dtype == torch.float16:  # opposite signs of the largest finite fp16
        keep &= ~(((ba & 0x7FFF) == F16_MAX_BITS) & ((bb & 0x7FFF) == F16_MAX_BITS))
    diff = np.nonzero((ba != bb) & keep)[0]
    if diff.size:
        i = int(diff[0])
        raise AssertionError(f"{label}: {diff.size} elements differ; first at {i}: "
                             f"{a[i].float().item()!r} (0x{int(ba[i]):x}) vs {b[i].float().item()!r} (0x{int(bb[i]):x})")
    return int(np.count_nonzero((ba != bb) & ~keep))


CASES = [
    # buffer, pdt, gdt, sdt, extra group kwargs
    (1, "f32", "f32", "f32", {"lam": 0.3}),
    (2, "f32", "f32", "f32", {}),
    ("T1", "f32", "f32", "f32", {}),
    ("T2", "f32", "f32", "f32", {}),
    (1, "bf16", "bf16", "f32", {}),
    (2, "bf16", "bf16", "f32", {}),
    ("T1", "bf16", "bf16", "f32", {}),
    ("T2", "bf16", "bf16", "f32", {}),
    (2, "bf16", "bf16", "bf16", {"state_precision": "param"}),
    ("T2", "bf16", "bf16", "bf16", {"state_precision": "param"}),
    ("T1", "bf16", "bf16", "bf16", {"state_precision": "param"}),
    ("T2", "f16", "f16", "f32", {}),
    (2, "f16", "f16", "f16", {"state_precision": "param"}),
    ("T1", "f16", "f16", "f16", {"state_precision": "param"}),
    ("T2", "bf16", "bf16", "f32", {"cautious": False, "stochastic_rounding": False}),
]


def _run(O, buffer, pdt, gdt, sdt, extra, corrupt_state: bool, steps: int = 3):
    _need_gpu()
    kw = dict(extra)
    kw.setdefault("lr", 1e-3)
    group = group_dict(buffer=buffer, **kw)
    dual = group["buffer"] in (2, "T2")
    host = TensorSet(SIZES, pdt, gdt, sdt, dual, False, seed=41, m_scale=1e-3)
    if corrupt_state:
        for i, pos in enumerate(POSITIONS):
            _inject(host.m[i], pos, M_SPECIALS, shift=i)
            if dual:
                _inject(host.v[i], pos[1:], V_SPECIALS, shift=i)
            _inject(host.p[i], pos[2:], P_SPECIALS, shift=i)
    dev = host.to("cuda")
    cfg = oracle_config(O, group)
    from luminamoon_amd.optimizer.hip_backend import HipStepper

    st = HipStepper()
    label = f"buffer={buffer} {pdt}/{gdt}/{sdt} {extra} state={'corrupt' if corrupt_state else 'finite'}"
    print(f"[case] special values {label}", flush=True)
    payload = 0
    for s in range(1, steps + 1):
        grads = host.grads(s, 43)
        for i, pos in enumerate(POSITIONS):
            _inject(grads[i], pos, GRAD_SPECIALS, shift=s + i)
        host.oracle_step(O, cfg, grads, s)
        dev.hip_step(st, group, [g.cuda() for g in grads], s)
        torch.cuda.synchronize()
        for i in range(len(SIZES)):
            payload += _assert_same(host.p[i], dev.p[i], f"{label} step {s} p[{i}]")
            payload += _assert_same(host.m[i], dev.m[i], f"{label} step {s} m[{i}]")
            if dual:
                payload += _assert_same(host.v[i], dev.v[i], f"{label} step {s} v[{i}]")
            payload += _assert_same(host.sc[i], dev.sc[i], f"{label} step {s} scratch[{i}]")
    if payload:
        print(f"[info] {label}: {payload} elements differ only in a NaN payload or a NaN sign", flush=True)
    return host


@pytest.mark.parametrize("buffer,pdt,gdt,sdt,extra", CASES, ids=[f"{c[0]}-{c[1]}-{c[3]}-{i}" for i, c in enumerate(CASES)])
def test_special_gradients(oracle_mod, buffer, pdt, gdt, sdt, extra):
    """Finite state, special gradients: sanitize_gradient leaves every value finite, so the
    results are finite and bitwise equal."""
    host = _run(oracle_mod, buffer, pdt, gdt, sdt, extra, corrupt_state=False)
    for i in range(len(SIZES)):
        assert bool(torch.isfinite(host.p[i].float()).all()), "sanitised gradients keep p finite"


@pytest.mark.parametrize("buffer,pdt,gdt,sdt,extra", CASES, ids=[f"{c[0]}-{c[1]}-{c[3]}-{i}" for i, c in enumerate(CASES)])
def test_corrupted_state_propagates_like_the_scalar_core(oracle_mod, buffer, pdt, gdt, sdt, extra):
    host = _run(oracle_mod, buffer, pdt, gdt, sdt, extra, corrupt_state=True)
    if pdt != "f16":  # fp16 stochastic rounding clamps a NaN to +-65504
        assert any(bool(torch.isnan(t.float()).any()) for t in host.p), "a NaN param stays NaN"



# fp16 param values at both ends of the fp16 range: subnormals, the lowest normal binade, the
# largest finite value and zeros. A param that a step leaves below 2^-14 or that a step pushes to
# 65504 or past it is outside the integer add's domain, so its wave takes the reference's integer
# recipe (prng.rs:98-130: the widened field for subnormals, the saturation at 65504).
F16_ENDS = [6e-8, -1.2e-7, 3.1e-6, -4.5e-5, 6.1e-5, -9.2e-5, 1.2e-4, 65504.0, -65504.0, 65000.0,
            -64990.0, 0.0, -0.0, 2.0e-5]


@pytest.mark.parametrize("buffer,sdt,extra", [
    ("T2", "f32", {}),
    ("T2", "f32", {"weight_decay": 0.0}),
    ("T1", "f16", {"state_precision": "param"}),
    (2, "f16", {"state_precision": "param", "weight_decay": 0.0}),
], ids=["T2", "T2-no-wd", "T1-param", "CLM-param-no-wd"])
def test_fp16_params_at_the_ends_of_the_fp16_range(oracle_mod, buffer, sdt, extra):
    """fp16 params from F16_ENDS fill the first 1,500 elements of the first tensor (whole units,
    so mixed waves run the recipe for in-domain lanes too) and every element of the second (the
    per-element path of a partial unit); three steps, bit for bit against the oracle."""
    O = oracle_mod
    _need_gpu()
    kw = dict(extra)
    kw.setdefault("lr", 1e-3)
    group = group_dict(buffer=buffer, **kw)
    dual = group["buffer"] in (2, "T2")
    host = TensorSet(SIZES, "f16", "f16", sdt, dual, False, seed=47, m_scale=1e-3)
    vals = torch.tensor(F16_ENDS, dtype=torch.float32)
    host.p[0][:1500] = vals.repeat(1500 // len(F16_ENDS) + 1)[:1500].to(torch.float16)
    host.p[1][:] = vals.repeat(SIZES[1] // len(F16_ENDS) + 1)[:SIZES[1]].to(torch.float16)
    dev = host.to("cuda")
    cfg = oracle_config(O, group)
    from luminamoon_amd.optimizer.hip_backend import HipStepper

    st = HipStepper()
    label = f"fp16 range ends buffer={buffer} state={sdt} {extra}"
    print(f"[case] {label}", flush=True)
    for s in range(1, 4):
        grads = host.grads(s, 53)
        host.oracle_step(O, cfg, grads, s)
        dev.hip_step(st, group, [g.cuda() for g in grads], s)
        torch.cuda.synchronize()
        for i in range(len(SIZES)):
            assert _assert_same(host.p[i], dev.p[i], f"{label} step {s} p[{i}]") == 0
            assert _assert_same(host.m[i], dev.m[i], f"{label} step {s} m[{i}]") == 0
            if dual:
                assert _assert_same(host.v[i], dev.v[i], f"{label} step {s} v[{i}]") == 0
            assert _assert_same(host.sc[i], dev.sc[i], f"{label} step {s} scratch[{i}]") == 0
    subnormal = [int(((bits(t.cpu()) & 0x7C00) == 0).sum()) - int(((bits(t.cpu()) & 0x7FFF) == 0).sum()) for t in host.p]
    assert sum(subnormal) > 0, "some params stay fp16 subnormals (the recipe's widened field ran)"

def test_radial_with_special_gradients(oracle_mod):
    """Radial bound: the squared norms see only sanitised gradients, so the sums stay finite and
    the f64 sums match the oracle's f64 mode bit for bit."""
    O = oracle_mod
    with O.radial_sum_f64():
        host = _run(O, "T2", "bf16", "bf16", "f32", {"bound_type": "radial"}, corrupt_state=False)
    assert all(math.isfinite(float(sc[4])) for sc in host.sc)
