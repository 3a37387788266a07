"""The oracle's AVX-512 backend (a restatement of luminav-simd/src/avx512/*.rs, the reference's CPU
execution path and this build's CPU baseline) against the scalar core.

The reference's own differential test (optimizer/crates/luminav-simd/tests/differential_parity.rs)
holds its AVX-512 kernels to its scalar core bit for bit per element, and its radial-bound
results to 1.5e-6 (the f32 lane sums run in another order). The same two properties are checked
here, plus the documented places where the reference's SIMD code differs from its scalar core.
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.skipif(not O.avx512_available(), reason="CPU without AVX-512")

BF16, F16, F32 = torch.bfloat16, torch.float16, torch.float32


def _bits(t):
    if t is None:
        return None
    return t.view(torch.int16) if t.dtype in (BF16, F16) else t.view(torch.int32)


def _run(backend, buffer, pdt, sdt, n, steps=4, threads=1, seed=7, **cfg_kw):
    rng = np.random.default_rng(seed)
    dual = buffer in (2, "T2")
    p = torch.from_numpy((rng.standard_normal(n) * 0.02).astype(np.float32)).to(pdt)
    m = torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32)).to(sdt)
    v = torch.from_numpy((np.abs(rng.standard_normal(n)) * 1e-6).astype(np.float32)).to(sdt) if dual else None
    master = cfg_kw.get("master_weights", 0)
    mp = p.float().clone() if master else None
    sc = torch.tensor([0, 0, 0, 1, 1, 0], dtype=torch.float32)
    cfg = O.make_config(buffer=buffer, **cfg_kw)
    with O.backend(backend):
        for t in range(1, steps + 1):
            g = rng.standard_normal(n).astype(np.float32) * 1e-3
            g[rng.random(n) < 0.05] = 0.0
            O.step(cfg, [p], [torch.from_numpy(g).to(pdt)], [m], [v], [mp], [sc], [t], [0], threads=threads)
    return {"p": p, "m": m, "v": v, "mp": mp, "scratch": sc}


def _assert_bitwise(a, b, what):
    for k in a:
        if a[k] is None:
            continue
        assert torch.equal(_bits(a[k]), _bits(b[k])), f"{what}: {k} differs in {int((_bits(a[k]) != _bits(b[k])).sum())} elements"


@pytest.mark.parametrize("buffer", [1, 2, "T1", "T2"])
@pytest.mark.parametrize("pdt,sdt", [(F32, F32), (BF16, F32), (BF16, BF16), (F16, F32), (F16, F16)])
def test_avx512_equals_scalar_core_bitwise(buffer, pdt, sdt):
    """Every mode x param/state dtype, ragged sizes (lane tails of 1-15 elements), cautious with the
    fused lagged scale (steps 2-4) and the step-1 two-pass: p, m, v and scratch bit for bit."""
    for n in (1, 15, 16, 17, 1000, 70_001):
        a = _run(O.BACKEND_SCALAR, buffer, pdt, sdt, n)
        b = _run(O.BACKEND_AVX512, buffer, pdt, sdt, n)
        _assert_bitwise(a, b, f"buffer={buffer} {pdt}/{sdt} n={n}")


@pytest.mark.parametrize("opts", [
    dict(cautious=False),
    dict(stochastic_rounding=False),
    dict(fused_single_pass=False),
    dict(master_weights=2),
    dict(bound=False),
    dict(weight_decay=0.0),
])
def test_avx512_equals_scalar_core_options(opts):
    for buffer, pdt in itertools.product([1, 2, "T1", "T2"], [F32, BF16]):
        a = _run(O.BACKEND_SCALAR, buffer, pdt, F32, 4099, steps=3, **opts)
        b = _run(O.BACKEND_AVX512, buffer, pdt, F32, 4099, steps=3, **opts)
        _assert_bitwise(a, b, f"{opts} buffer={buffer} {pdt}")


def test_avx512_multi_chunk_threads():
    """Two 2,097,152-element chunks plus a 37-element tail, one and four threads: the chunk offsets
    of stochastic rounding and the chunk-order mask counts agree with the scalar core."""
    n = 2 * 2_097_152 + 37
    ref = _run(O.BACKEND_SCALAR, "T2", BF16, F32, n, steps=2, threads=4)
    for threads in (1, 4):
        got = _run(O.BACKEND_AVX512, "T2", BF16, F32, n, steps=2, threads=threads)
        _assert_bitwise(ref, got, f"threads={threads}")


@pytest.mark.parametrize("buffer", [1, 2, "T1", "T2"])
def test_avx512_radial_within_reference_tolerance(buffer):
    """Radial bound: the squared norms are f32 lane sums in another order than the scalar core
    (the 16-lane accumulator is reduced 16->8->4->2->1, the chunk tail added one by one), so only
    the bound scale and p move, within the reference's cross-backend tolerance of 1.5e-6
    (differential_parity.rs:16); m and v do not depend on the bound and stay bitwise."""
    n = 100_003
    a = _run(O.BACKEND_SCALAR, buffer, F32, F32, n, steps=3, bound_type=1)
    b = _run(O.BACKEND_AVX512, buffer, F32, F32, n, steps=3, bound_type=1)
    assert torch.equal(_bits(a["m"]), _bits(b["m"]))
    if a["v"] is not None:
        assert torch.equal(_bits(a["v"]), _bits(b["v"]))
    assert float((a["p"] - b["p"]).abs().max()) <= 1.5e-6
    assert abs(float(a["scratch"][4]) - float(b["scratch"][4])) <= 1e-5 * max(1.0, abs(float(a["scratch"][4])))
    assert float(a["scratch"][3]) == float(b["scratch"][3])  # the mask count is exact in both


def _one_step_with(m_value, pdt, sdt):
    """16 elements (one vector, no tail), element 5 of exp_avg set to m_value."""
    out = {}
    for backend in (O.BACKEND_SCALAR, O.BACKEND_AVX512):
        n = 16
        p = torch.full((n,), 0.01, dtype=F32).to(pdt)
        g = torch.full((n,), 1e-3, dtype=F32).to(pdt)
        m = torch.zeros(n, dtype=F32)
        m[5] = m_value
        m = m.to(sdt)
        v = torch.zeros(n, dtype=F32).to(sdt)
        sc = torch.tensor([0, 0, 0, 1, 1, 0], dtype=torch.float32)
        cfg = O.make_config(buffer="T2")
        with O.backend(backend):
            O.step(cfg, [p], [g], [m], [v], [None], [sc], [1], [0])
        out[backend] = (p, m, v)
    return out


def test_documented_divergence_inf_state_through_sr():
    """Where the reference's backends differ, the AVX-512 restatement follows the reference's SIMD
    code: stochastic rounding passes +inf through unchanged (avx512/mod.rs:110-131), where the
    scalar core clamps to the largest finite bf16 (prng.rs:137-154). Finite elements agree."""
    out = _one_step_with(float("inf"), BF16, BF16)
    m_scalar, m_simd = out[O.BACKEND_SCALAR][1], out[O.BACKEND_AVX512][1]
    assert int(_bits(m_scalar)[5]) == 0x7F7F
    assert int(_bits(m_simd)[5]) == 0x7F80
    keep = torch.ones(16, dtype=torch.bool)
    keep[5] = False
    assert torch.equal(_bits(m_scalar)[keep], _bits(m_simd)[keep])
