"""Seeded random option combinations on the GPU, bit for bit against the oracle.

Each case draws every option of the drop-in constructor at once:
- buffer mode, param / grad / state dtypes, master weights;
- cautious, stochastic rounding, bound type (coordinate, radial or none);
- weight decay, fused single pass, and lr, betas, eps, tau, lam, clamp_min, bound_ratio,
  ema_decay and seed;
- a tensor count of 1, 5, or 60 (60 makes a table launch).

This covers the interactions that the hand-picked matrices of test_gpu_parity.py and
test_gpu_radial.py leave out. Radial cases compare with the oracle's f64 sum mode, as in
test_gpu_radial.py. The draws are fixed by the case index, so a failure names a
reproducible case.
"""
from __future__ import annotations

import contextlib

import numpy as np
import pytest
import torch

from tests.parity_util import TensorSet, group_dict, oracle_config

pytestmark = pytest.mark.gpu

N_CASES = 400


def _draw(case: int):
    rng = np.random.default_rng(1000 + case)
    pick = lambda xs: xs[int(rng.integers(len(xs)))]  # noqa: E731
    buffer = pick([1, 2, "T1", "T2"])
    pdt = pick(["f32", "bf16", "bf16", "f16"])
    gdt = pdt if rng.random() < 0.8 else pick(["f32", "bf16", "f16"])
    state = pick(["fp32", "param"])
    master = pick(["none", "semi", "full"]) if pdt != "f32" else "none"
    bound = pick(["coordinate", "coordinate", "radial", "none"])
    kw = dict(
        buffer=buffer, cautious=bool(rng.random() < 0.7), stochastic_rounding=bool(rng.random() < 0.7),
        fused_single_pass=bool(rng.random() < 0.8), master_weights=master, state_precision=state,
        lr=float(10 ** rng.uniform(-4, -2)), betas=(float(rng.uniform(0.8, 0.95)), float(rng.uniform(0.99, 0.9999))),
        eps=float(10 ** rng.uniform(-10, -6)), tau=float(rng.uniform(0.5, 1.0)), lam=float(rng.uniform(0.1, 0.5)),
        weight_decay=pick([0.0, 0.01, 0.08]), cautious_clamp_min=float(rng.uniform(0.2, 0.8)),
        bound_ratio=float(rng.uniform(0.02, 0.1)), seed=int(rng.integers(1, 2 ** 31 - 1)),
        ema_decay=pick(["auto", float(rng.uniform(0.5, 0.95))]),
    )
    if bound == "none":
        kw["bound"] = False
    else:
        kw["bound_type"] = bound
    count = pick([1, 5, 60])
    sizes = [int(np.exp(rng.uniform(0, np.log(20_000)))) + 1 for _ in range(count)]
    return pdt, gdt, kw, sizes


def _state_dtype(pdt: str, kw) -> str:
    if pdt == "f32" or kw["state_precision"] == "fp32" or kw["master_weights"] == "full":
        return "f32"
    return pdt


@pytest.mark.parametrize("case", range(N_CASES))
def test_random_options_bitwise(oracle_mod, case):
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    from luminamoon_amd.optimizer.hip_backend import HipStepper

    O = oracle_mod
    pdt, gdt, kw, sizes = _draw(case)
    group = group_dict(**kw)
    dual = group["buffer"] in (2, "T2")
    master = group["master_weights"] > 0 and pdt != "f32"
    sdt = _state_dtype(pdt, kw)
    host = TensorSet(sizes, pdt, gdt, sdt, dual, master, seed=case, m_scale=1e-3)
    dev = host.to("cuda")
    cfg = oracle_config(O, group)
    st = HipStepper()
    label = f"case {case}: {pdt}/{gdt}/{sdt} {len(sizes)} tensors {kw}"
    print(f"[case] {label}", flush=True)
    radial = group["bound"] and group["bound_type"] == 1
    with O.radial_sum_f64() if radial else contextlib.nullcontext():
        for s in range(1, 4):
            grads = host.grads(s, 77 + case)
            host.oracle_step(O, cfg, grads, s)
            dev.hip_step(st, group, [g.cuda() for g in grads], s)
            torch.cuda.synchronize()
            host.assert_equal(dev, f"{label} step {s}")
