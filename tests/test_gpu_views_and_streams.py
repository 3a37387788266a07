"""Views at any element offset, and one workspace used from two streams, on the GPU.

* Unaligned views. A view that starts k elements past a 16-byte boundary in every one of its
  buffers (a slice of a bucket, a shard) keeps the vector layout: its work units start at the
  first element on a 128-byte line (16 bytes for short tensors) and the head before it is taken
  one element per thread by the tensor's last block. Checked bit for bit against the oracle for
  k = 0..8, 31, 33, 63, 64, 65, for f32, bf16 and 16-bit state
  (the 8-element lane layout), the split lane layout of a master copy beside 16-bit state, sizes
  around the unit size and the head, and inactive ranges that cover the head. Views whose buffers
  disagree on their offset (a shifted grad beside an aligned param and state) go element by element,
  reading consecutive elements across the wave; also bit for bit.
  The reference's Triton kernels take any base offset with masked lanes
  (python/luminamoon/optimizer/triton_kernels.py:156-158).
* Workspace ordering. Two streams stepping disjoint tensor sets back to back through one
  HipStepper share its workspace (count slots); the library makes the second stream wait for the
  first call, so both sets match the oracle bit for bit and the workspace ends zero. The
  reference gives each parameter scratch of its own for the same reason
  (changelogs/LUMINAV_ALGORITHM_CHANGELOG.md:281-283).
"""
from __future__ import annotations

import contextlib
from typing import List, Optional, Sequence, Tuple

import pytest
import torch

from tests.parity_util import TensorSet, group_dict, oracle_config

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


def _stepper():
    from luminamoon_amd.optimizer.hip_backend import HipStepper

    return HipStepper()


def _shifted(t: Optional[torch.Tensor], k: int) -> Optional[torch.Tensor]:
    """A copy of t on the GPU that starts k elements into a fresh (256-byte aligned) buffer."""
    if t is None:
        return None
    big = torch.zeros(t.numel() + 80, dtype=t.dtype, device="cuda")
    big[k:k + t.numel()].copy_(t.reshape(-1))
    return big[k:k + t.numel()]


def _oracle_step_inactive(O, cfg, host: TensorSet, grads: Sequence[torch.Tensor], step: int,
                          ranges: Sequence[Optional[List[Tuple[int, int]]]]) -> None:
    """The reference's grad=None handling on the oracle (luminav.py:1466-1531, 1585-1603): zero the
    grad slices, step every element, restore the param/state/master slices."""
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


def _views_case(O, sizes, pdt, sdt, offs, steps=3, seed=31, ranges=None, grad_offs=None, **gkw):
    """Steps tensors whose p/m/v/master start offs[i] elements into their buffers and whose grads
    start grad_offs[i] (default: the same) elements in, against the oracle."""
    group = group_dict(**gkw)
    dual = group["buffer"] in (2, "T2")
    master = group["master_weights"] > 0 and pdt != "f32"
    host = TensorSet(sizes, pdt, pdt, sdt, dual, master, seed)
    dev = host.to("cpu")
    dev.p = [_shifted(t, k) for t, k in zip(host.p, offs)]
    dev.m = [_shifted(t, k) for t, k in zip(host.m, offs)]
    dev.v = [_shifted(t, k) for t, k in zip(host.v, offs)]
    dev.mp = [_shifted(t, k) for t, k in zip(host.mp, offs)]
    dev.sc = [t.cuda() for t in host.sc]
    goffs = offs if grad_offs is None else grad_offs
    cfg = oracle_config(O, group)
    st = _stepper()
    tables = None
    if ranges is not None:
        tables = [None if not rs else torch.tensor(rs, dtype=torch.int64, device="cuda") for rs in ranges]
    label = f"{gkw} {pdt}/{sdt} sizes={sizes} offs={offs} grad_offs={goffs}"
    print(f"[case] {label}", flush=True)
    for s in range(1, steps + 1):
        grads = host.grads(s, seed)
        if ranges is None:
            host.oracle_step(O, cfg, grads, s)
        else:
            _oracle_step_inactive(O, cfg, host, grads, s, ranges)
        st.step(group, dev.p, [_shifted(g, k) for g, k in zip(grads, goffs)], dev.m, dev.v, dev.mp, dev.sc,
                [s] * len(sizes), list(range(len(sizes))), inactive=tables)
        torch.cuda.synchronize()
        host.assert_equal(dev, f"{label} step {s}")


VIEW_CASES = [
    # name, pdt, sdt, group kwargs
    ("T2 bf16, f32 m/v", "bf16", "f32", dict(buffer="T2", lr=1e-3)),
    ("CLM f32", "f32", "f32", dict(buffer=2, lr=1e-3)),
    ("T1 bf16, bf16 m (8-element lanes)", "bf16", "bf16", dict(buffer="T1", lr=1e-3, state_precision="param")),
    ("T2 bf16, bf16 m/v + semi master (split lanes)", "bf16", "bf16",
     dict(buffer="T2", lr=1e-3, state_precision="param", master_weights="semi")),
    ("TD-CLM f16, fp16 container, no fused pass", "f16", "f16",
     dict(buffer=1, lr=1e-3, state_precision="param", fused_single_pass=False)),
]


@pytest.mark.parametrize("name,pdt,sdt,kw", VIEW_CASES, ids=[c[0] for c in VIEW_CASES])
def test_views_at_every_offset_match_oracle(oracle_mod, name, pdt, sdt, kw):
    """One call over 14 tensors, tensor k starting offs[k] elements past a 256-byte boundary in
    every buffer: 0..8, 31, 33, 63, 64, 65 (heads up to 63 elements to the next 128-byte line,
    or to 16 bytes when the tensor is shorter than that), of sizes around the unit and the head
    (1, shorter than the head, a unit plus the head, whole units after the head, ragged)."""
    _need_gpu()
    offs = [0, 1, 2, 3, 4, 5, 6, 7, 8, 31, 33, 63, 64, 65]
    sizes = [1, 3, 3, 2048 + 61, 4096 + 60, 2 * 2048 + 5, 65_539, 100_000, 1024 + 7, 40, 2048 + 31, 5000, 3000,
             2048 + 63]
    _views_case(oracle_mod, sizes, pdt, sdt, offs, **kw)


def test_views_with_inactive_ranges_over_the_head(oracle_mod):
    """Inactive ranges covering part of the head, the whole head and the first aligned unit, and
    a wholly inactive last unit whose block still takes the head."""
    _need_gpu()
    n = 3 * 1024 + 100
    sizes = [n, n, n, n]
    offs = [1, 5, 3, 7]
    # bf16 p/g with f32 m/v at offset k: head (64 - k) mod 64 (the next 128-byte line)
    ranges = [[(0, 2), (500, 700)],          # part of the head (offset 1: head 63)
              [(0, 59)],                     # exactly the head (offset 5: head 59)
              [(0, 1100), (2000, 2001)],     # the head and the first aligned unit (offset 3: head 61)
              [(2106, n)]]                   # the last unit wholly inactive (offset 7: head 57)
    for kw in (dict(buffer="T2", lr=1e-3), dict(buffer=2, lr=1e-3, cautious=False),
               dict(buffer="T2", lr=1e-3, bound_type="radial")):
        with (oracle_mod.radial_sum_f64() if kw.get("bound_type") == "radial" else contextlib.nullcontext()):
            _views_case(oracle_mod, sizes, "bf16", "f32", offs, ranges=ranges, **kw)


def test_views_whose_buffers_disagree_go_element_by_element(oracle_mod):
    """Grads shifted by 1-5 elements beside an aligned param and state (no head aligns every
    stream): the per-element path, bit for bit."""
    _need_gpu()
    sizes = [1, 1023, 1024 * 3 + 5, 40_000]
    _views_case(oracle_mod, sizes, "bf16", "f32", [0] * 4, grad_offs=[1, 3, 1, 5], buffer="T2", lr=1e-3)
    _views_case(oracle_mod, sizes, "f32", "f32", [0] * 4, grad_offs=[1, 1, 2, 3], buffer=1, lr=1e-3)


def test_two_streams_share_the_workspace_in_order(oracle_mod):
    """Two tensor sets stepped back to back on two streams through one HipStepper (one workspace):
    each call's launches are large enough to still run when the other stream's call is issued.
    Steps 1 (two-pass) to 4 (fused) of each set match the oracle bit for bit, and the workspace
    is all zero at the end. Then the same with the null stream in between."""
    _need_gpu()
    O = oracle_mod
    group = group_dict(buffer="T2", lr=1e-3)
    cfg = oracle_config(O, group)
    sizes = [1 << 22, 3 << 20, 5]
    sets = [TensorSet(sizes, "bf16", "bf16", "f32", True, False, seed) for seed in (41, 42)]
    devs = [h.to("cuda") for h in sets]
    st = _stepper()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    for step in range(1, 5):
        grads = [[g.cuda() for g in h.grads(step, 50 + k)] for k, h in enumerate(sets)]
        torch.cuda.synchronize()
        streams = (s1, s2) if step != 3 else (s1, torch.cuda.default_stream())
        for k, (dev, stream) in enumerate(zip(devs, streams)):
            with torch.cuda.stream(stream):
                dev.hip_step(st, group, grads[k], step)
        torch.cuda.synchronize()
        for k, h in enumerate(sets):
            h.oracle_step(O, cfg, [g.cpu() for g in grads[k]], step, threads=8)
            h.assert_equal(devs[k], f"set {k} step {step}")
    # the null stream, then a side stream, then the null stream again
    for step, stream in ((5, torch.cuda.default_stream()), (6, s2), (7, torch.cuda.default_stream())):
        for k, dev in enumerate(devs):
            g = [x.cuda() for x in sets[k].grads(step, 50 + k)]
            torch.cuda.synchronize()
            with torch.cuda.stream(stream if k == 0 else s1):
                dev.hip_step(st, group, g, step)
        torch.cuda.synchronize()
        for k, h in enumerate(sets):
            h.oracle_step(O, cfg, sets[k].grads(step, 50 + k), step, threads=8)
            h.assert_equal(devs[k], f"set {k} step {step}")
    for ws in st.workspace._bufs.values():
        assert int(torch.count_nonzero(ws)) == 0
