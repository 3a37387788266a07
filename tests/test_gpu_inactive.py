"""Inactive element ranges on the GPU: a fused bucket's grad=None slices.

The reference steps a fused bucket whose params lack a grad by zeroing their grad slice, stepping
the whole bucket and copying their param/state slices back (python/luminamoon/optimizer/
luminav.py:1426-1603). Those elements therefore count in the bucket's cautious/radial statistics
(n, mask count, squared norms) with g = 0, and their values do not change. The HIP path passes them
as inactive [begin, end) ranges instead: computed with g = 0 for the statistics, never written,
grad not read, and whole 1024-element units inside a range skipped on non-radial passes.

Checked bit for bit against the oracle run the reference's way (zero, step all, restore):
  * at the C-ABI level, with ranges at the tensor start and end, covering whole units, straddling
    unit boundaries, single elements and several ranges inside one unit; for every pass shape
    (two-pass step 1, fused steps, fused_single_pass=False, no-counting single pass, radial
    persistent counting + unit apply), master weights, f16 params, and a multi-tensor call with a
    tensor that is wholly inactive;
  * through LuminaV(fuse_tensors=True) with a grad=None pattern that changes from step to step.
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import pytest
import torch

from tests.parity_util import TensorSet, assert_bitwise, group_dict, oracle_config

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


def _stepper():
    from luminamoon_amd.optimizer.hip_backend import HipStepper

    return HipStepper()


def _ranges(n: int) -> List[Tuple[int, int]]:
    """Sorted, disjoint ranges exercising every unit-coverage case for 1024-, 2048- and
    4096-element units (the last as two 2048-element sub-units): start of tensor, straddling a
    unit or a sub-unit boundary, whole units, single elements, several in one unit, tail."""
    rs = [(0, 5), (1000, 1030), (2048, 5120), (6000, 6001), (6003, 6004), (6010, 6100), (9000, 12288),
          (20000, 20001), (n - 700, n)]
    return [(b, min(e, n)) for b, e in rs if b < n and b < min(e, n)]


def _oracle_step_inactive(O, cfg, host: TensorSet, grads: Sequence[torch.Tensor], step: int,
                          ranges: Sequence[Optional[List[Tuple[int, int]]]]) -> None:
    """The reference's grad=None handling on the oracle: zero the grad slices, step every
    element, restore the param/state/master slices."""
    grads = [g.clone() for g in grads]
    saved = []
    for i, rs in enumerate(ranges):
        for b, e in rs or []:
            grads[i][b:e] = 0
            saved.append((i, b, e, host.p[i][b:e].clone(), host.m[i][b:e].clone(),
                          None if host.v[i] is None else host.v[i][b:e].clone(),
                          None if host.mp[i] is None else host.mp[i][b:e].clone()))
    host.oracle_step(O, cfg, grads, step)
    for i, b, e, p, m, v, mp in saved:
        host.p[i][b:e] = p
        host.m[i][b:e] = m
        if v is not None:
            host.v[i][b:e] = v
        if mp is not None:
            host.mp[i][b:e] = mp


def _tables(ranges):
    return [None if not rs else torch.tensor(rs, dtype=torch.int64, device="cuda") for rs in ranges]


CASES = [
    dict(name="T2 bf16 cautious (two-pass, then fused)", pdt="bf16", sdt="f32", kw=dict(buffer="T2")),
    dict(name="CLM f32 fused_single_pass=False", pdt="f32", sdt="f32", kw=dict(buffer=2, fused_single_pass=False)),
    dict(name="T1 bf16 no cautious (single pass)", pdt="bf16", sdt="f32", kw=dict(buffer="T1", cautious=False)),
    dict(name="TD-CLM f16 master full", pdt="f16", sdt="f32", kw=dict(buffer=1, master_weights="full")),
    dict(name="T2 bf16 bf16-state no SR", pdt="bf16", sdt="bf16", kw=dict(buffer="T2", stochastic_rounding=False)),
    dict(name="T1 bf16 bf16-state cautious (two sub-units)", pdt="bf16", sdt="bf16", kw=dict(buffer="T1")),
    dict(name="T1 f16 fp16-container cautious (two sub-units)", pdt="f16", sdt="f16", kw=dict(buffer="T1")),
    dict(name="radial T2 bf16 cautious", pdt="bf16", sdt="f32", kw=dict(buffer="T2", bound_type="radial"), radial=True),
    dict(name="radial CLM f32 no cautious", pdt="f32", sdt="f32", kw=dict(buffer=2, bound_type="radial", cautious=False),
         radial=True),
]


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_inactive_ranges_match_zero_step_restore(oracle_mod, case):
    _need_gpu()
    O = oracle_mod
    group = group_dict(**case["kw"])
    dual = group["buffer"] in (2, "T2")
    master = group["master_weights"] > 0 and case["pdt"] != "f32"
    sizes = [30_011, 2_000, 4_096]
    # tensor 0: ranges of every kind; tensor 1: wholly inactive; tensor 2: all active
    ranges = [_ranges(sizes[0]), [(0, sizes[1])], None]
    host = TensorSet(sizes, case["pdt"], case["pdt"], case["sdt"], dual, master, seed=77, m_scale=1e-3)
    dev = host.to("cuda")
    tables = _tables(ranges)
    cfg = oracle_config(O, group)
    st = _stepper()
    print(f"[case] inactive {case['name']}", flush=True)
    ctx = O.radial_sum_f64() if case.get("radial") else None
    if ctx is not None:
        ctx.__enter__()
    try:
        for s in range(1, 5):
            grads = host.grads(s, seed=5)
            _oracle_step_inactive(O, cfg, host, grads, s, ranges)
            st.step(group, dev.p, [g.cuda() for g in grads], dev.m, dev.v, dev.mp, dev.sc, [s] * 3, [0, 1, 2],
                    inactive=tables)
            torch.cuda.synchronize()
            host.assert_equal(dev, f"{case['name']} step {s}")
    finally:
        if ctx is not None:
            ctx.__exit__(None, None, None)


def test_inactive_elements_never_written_and_grad_not_read():
    """NaN grads inside inactive ranges must not leak: the kernel never reads them."""
    _need_gpu()
    group = group_dict(buffer="T2")
    n = 10_000
    host = TensorSet([n], "bf16", "bf16", "f32", True, False, seed=3, m_scale=1e-3)
    dev = host.to("cuda")
    rs = [(100, 3000), (5000, 5001), (8192, n)]
    g = host.grads(1, seed=9)[0].cuda()
    for b, e in rs:
        g[b:e] = float("nan")
    p0, m0, v0 = dev.p[0].clone(), dev.m[0].clone(), dev.v[0].clone()
    st = _stepper()
    for s in (1, 2):
        st.step(group, dev.p, [g], dev.m, dev.v, dev.mp, dev.sc, [s], [0], inactive=_tables([rs]))
    torch.cuda.synchronize()
    for b, e in rs:
        assert_bitwise(dev.p[0][b:e], p0[b:e], f"p[{b}:{e}]")
        assert_bitwise(dev.m[0][b:e], m0[b:e], f"m[{b}:{e}]")
        assert_bitwise(dev.v[0][b:e], v0[b:e], f"v[{b}:{e}]")
    assert torch.isfinite(dev.sc[0]).all()
    assert not torch.equal(dev.p[0][3000:5000], p0[3000:5000])


@pytest.mark.parametrize("buffer,pdt", [("T2", torch.bfloat16), (2, torch.float32)])
def test_fused_bucket_grad_none_pattern_matches_reference_semantics(oracle_mod, buffer, pdt):
    """LuminaV(fuse_tensors=True): params without a grad change from step to step; the bucket's
    flat buffers and scratch equal the oracle run with zero-step-restore after every step."""
    _need_gpu()
    from luminamoon_amd import LuminaV
    from tests.parity_util import seeded_tensor

    O = oracle_mod
    shapes = [(3000,), (1,), (64, 64), (777,), (100, 100), (5,)]
    params = [torch.nn.Parameter(seeded_tensor(int(torch.Size(s).numel()), 40 + i, 0.02, pdt).view(s).cuda())
              for i, s in enumerate(shapes)]
    opt = LuminaV(params, lr=2e-3, buffer=buffer, fuse_tensors=True)
    assert len(opt._fused_buckets) == 1
    b = opt._fused_buckets[0]
    group = opt.param_groups[0]
    cfg = oracle_config(O, group)
    sizes = [p.numel() for p in params]
    offs = [0]
    for n in sizes:
        offs.append(offs[-1] + n)
    N = offs[-1]
    dual = buffer in (2, "T2")
    host = TensorSet([N], "bf16" if pdt == torch.bfloat16 else "f32", "bf16" if pdt == torch.bfloat16 else "f32",
                     "f32", dual, False, seed=1)
    host.p[0] = torch.cat([p.detach().cpu().reshape(-1) for p in params])
    none_pattern = [{1, 3}, set(), {0, 5}, {0, 1, 2, 3, 4}, {2}]
    expect_step = [0] * len(params)
    for s, nones in enumerate(none_pattern, 1):
        grads = []
        for i, p in enumerate(params):
            gi = seeded_tensor(sizes[i], 1000 * s + i, 1e-3, pdt).view(p.shape)
            grads.append(gi)
            p.grad = None if i in nones else gi.cuda()
        opt.step()
        flat_g = torch.cat([g.reshape(-1) for g in grads])
        ranges = []
        for i in sorted(nones):
            if ranges and ranges[-1][1] == offs[i]:
                ranges[-1] = (ranges[-1][0], offs[i + 1])
            else:
                ranges.append((offs[i], offs[i + 1]))
        _oracle_step_inactive(O, cfg, host, [flat_g], s, [ranges])
        torch.cuda.synchronize()
        assert_bitwise(b["flat_p"], host.p[0], f"step {s} flat_p")
        assert_bitwise(b["flat_m"], host.m[0], f"step {s} flat_m")
        if dual:
            assert_bitwise(b["flat_v"], host.v[0], f"step {s} flat_v")
        assert_bitwise(b["scratch"], host.sc[0], f"step {s} scratch")
        for i, p in enumerate(params):
            if i not in nones:
                expect_step[i] = s
            assert int(opt.state[p]["step"]) == expect_step[i], f"step {s}: param {i} step count"
