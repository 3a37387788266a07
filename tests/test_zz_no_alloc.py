"""lv_step_multi_noalloc (the entry point for callers that cannot allocate) against
lv_step_multi, through the C ABI, bit for bit: the same tensors stepped by both, two calls in a
row (the second with a smaller input), every buffer and scratch compared after each call; and
its limits refused with a clear error."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from tests.parity_util import TensorSet, assert_bitwise, group_dict

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


def _call_both(lib, group, a, b, grads, step, stepper):
    """Step set `a` with lv_step_multi (the stepper's workspace) and set `b` with
    lv_step_multi_noalloc, from the same packed descriptors layout."""
    from luminamoon_amd.optimizer import hip_backend as H

    n = len(a.sizes)
    pa = stepper.prepare(a.p, grads, a.m, a.v, a.mp, a.sc, [step] * n, list(range(n)))
    stepper.launch(group, pa)
    pb = stepper.prepare(b.p, grads, b.m, b.v, b.mp, b.sc, [step] * n, list(range(n)))
    cfg = H.make_config(group)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.lv_step_multi_noalloc(ctypes.byref(cfg), pb.items, pb.n, ctypes.c_void_p(stream))
    assert rc == 0, lib.lv_last_error()


@pytest.mark.parametrize("buffer,pdt,sdt,extra", [
    ("T2", "bf16", "f32", {}),
    (1, "f32", "f32", {"lam": 0.3, "fused_single_pass": False}),
    (2, "bf16", "bf16", {"state_precision": "param", "master_weights": "full"}),
    ("T1", "bf16", "f32", {"bound_type": "radial"}),
])
def test_noalloc_matches_lv_step_multi(buffer, pdt, sdt, extra):
    _need_gpu()
    from luminamoon_amd.optimizer import hip_backend as H

    lib = H.load_library()
    kw = dict(extra)
    kw.setdefault("lr", 1e-3)
    group = group_dict(buffer=buffer, **kw)
    dual = group["buffer"] in (2, "T2")
    master = group["master_weights"] > 0 and pdt != "f32"
    st = H.HipStepper()
    rng = np.random.default_rng(17)
    # first call: 60 ragged tensors (two inline launches per class here, one table launch in
    # lv_step_multi); second call: a smaller input of 5 tensors
    for call, sizes in enumerate(([int(np.exp(rng.uniform(0, np.log(200_000)))) + 1 for _ in range(60)],
                                  [3, 1025, 2049, 70_001, 7])):
        host = TensorSet(sizes, pdt, pdt, sdt, dual, master, 5 + call)
        a, b = host.to("cuda"), host.to("cuda")
        print(f"[case] noalloc buffer={buffer} {pdt}/{sdt} {extra} call {call} ({len(sizes)} tensors)", flush=True)
        for s in range(1, 4):
            grads = [g.cuda() for g in host.grads(s, 40 + call)]
            _call_both(lib, group, a, b, grads, s, st)
            torch.cuda.synchronize()
            for i in range(len(sizes)):
                assert_bitwise(a.p[i], b.p[i], f"call {call} step {s} p[{i}]")
                assert_bitwise(a.m[i], b.m[i], f"call {call} step {s} m[{i}]")
                if dual:
                    assert_bitwise(a.v[i], b.v[i], f"call {call} step {s} v[{i}]")
                if master:
                    assert_bitwise(a.mp[i], b.mp[i], f"call {call} step {s} mp[{i}]")
                assert_bitwise(a.sc[i], b.sc[i], f"call {call} step {s} scratch[{i}]")


def test_noalloc_limits_are_refused():
    _need_gpu()
    from luminamoon_amd.optimizer import hip_backend as H

    lib = H.load_library()
    st = H.HipStepper()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # more than 256 tensors
    group = group_dict(buffer=1, lr=1e-3)
    host = TensorSet([8] * 257, "f32", "f32", "f32", False, False, 1).to("cuda")
    zeros = [torch.zeros(8, device="cuda") for _ in range(257)]
    prep = st.prepare(host.p, zeros, host.m, host.v, host.mp, host.sc, [1] * 257, list(range(257)))
    cfg = H.make_config(group)
    assert lib.lv_step_multi_noalloc(ctypes.byref(cfg), prep.items, prep.n, stream) == -3
    assert b"256" in lib.lv_last_error()
    # a radial counting launch above 65,536 units (1024-element units with fp32 state)
    rgroup = group_dict(buffer="T2", bound_type="radial", lr=1e-3)
    big = TensorSet([65_536 * 1024 + 1], "bf16", "bf16", "f32", True, False, 2).to("cuda")
    g = torch.zeros(65_536 * 1024 + 1, dtype=torch.bfloat16, device="cuda")
    prep = st.prepare(big.p, [g], big.m, big.v, big.mp, big.sc, [1], [0])
    p0 = big.p[0].clone()
    rcfg = H.make_config(rgroup)
    assert lib.lv_step_multi_noalloc(ctypes.byref(rcfg), prep.items, prep.n, stream) == -3
    assert b"65536" in lib.lv_last_error()
    torch.cuda.synchronize()
    assert torch.equal(big.p[0], p0)
