"""Committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from the
oracle): the oracle must keep reproducing them (CPU), and the HIP path must match them bit for
bit (GPU). Inputs come from the reference's PRNG-based generator, restated in tests/golden/cases.py."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from tests.golden.cases import CASES, inputs, prng
from tests.golden.make_golden import SDT, run_oracle
from tests.parity_util import bits, group_dict

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(HERE, f"{name}.npz")) as z:
        return {k: z[k] for k in z.files}


def test_case_generator_uses_the_pinned_prng(oracle_mod):
    L = oracle_mod.lib()
    idx = np.array([0, 1, 2, 12345, 2 ** 31 - 1, -5], dtype=np.int64).astype(np.int32)
    for seed in (0, 42, 1337, 2 ** 31 - 2):
        assert list(prng(seed, idx)) == [L.lvo_prng(seed, int(i)) for i in idx]


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_reproduces_fixture(oracle_mod, name):
    want = load(name)
    got = run_oracle(name)
    assert set(got) == set(want)
    for k in want:
        assert np.array_equal(got[k].astype(np.uint32), want[k]), (name, k)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_hip_matches_fixture(name):
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    from luminamoon_amd.optimizer.hip_backend import HipStepper

    gk, pdt, sdt, sizes, steps = CASES[name]
    group = group_dict(**gk)
    dual = group["buffer"] in (2, "T2")
    master = group["master_weights"] > 0 and pdt != "f32"
    params, grads = inputs(name)
    p = [x.clone().cuda() for x in params]
    m = [torch.zeros(n, dtype=SDT[sdt], device="cuda") for n in sizes]
    v = [torch.zeros(n, dtype=SDT[sdt], device="cuda") if dual else None for n in sizes]
    mp = [x.float().clone().cuda() if master else None for x in params]
    sc = [torch.tensor([0, 0, 0, 1, 1, 0], dtype=torch.float32, device="cuda") for _ in sizes]
    st = HipStepper()
    print(f"[golden] {name}", flush=True)
    for s in range(steps):
        st.step(group, p, [g.cuda() for g in grads[s]], m, v, mp, sc, [s + 1] * len(sizes), list(range(len(sizes))))
    torch.cuda.synchronize()
    want = load(name)
    for i in range(len(sizes)):
        for key, t in (("p", p[i]), ("m", m[i]), ("v", v[i]), ("mp", mp[i]), ("sc", sc[i])):
            if t is None:
                continue
            assert np.array_equal(bits(t).astype(np.uint32), want[f"{key}{i}"]), (name, key, i)
