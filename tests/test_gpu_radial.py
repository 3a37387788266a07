"""Radial bound on the GPU (bound_type="radial": math.rs:127-239, reference_cpu/dual.rs:134-253,
parallel/dual.rs:176-200 and 260-351).

The HIP kernels add the f32 squares u_eff^2 and p^2 in f64 and round the folded sum to f32 once.
The reference sums in f32, in an order that depends on its CPU backend (16-lane scalar core vs.
AVX-512 reductions), and its own cross-backend test accepts 1.5e-6 absolute
(luminav-simd/tests/differential_parity.rs:16). Two bars here:
  * bit for bit against the oracle in its f64 sum mode (same per-element values, same sums up to
    f64 rounding): every option combination, ragged multi-tensor calls, more tensors than one
    launch holds, tensors summed over several fold chunks and launch pieces;
  * against the oracle in the scalar core's f32 order, on the reference's own differential-parity
    configurations and inputs: m and v bitwise (the scale never feeds them), fp32 params within
    1.5e-6, bf16 params within 1 ULP on a small fraction of elements (a stochastic-rounding
    decision near its threshold can flip when the scale moves in its last bits), the bound scale
    within the f32 summation bound (adds per lane x 2^-24).
The same call twice gives identical bits (fixed-order fold of the unit records).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.parity_util import (DT, TensorSet, assert_bitwise, bits, group_dict, oracle_config, prng_np,
                               reference_pseudo_random)

pytestmark = pytest.mark.gpu

RAGGED = [1, 7, 2047, 2048, 2049, 8191, 65539, 100_000]


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


def _stepper():
    from luminamoon_amd.optimizer.hip_backend import HipStepper

    return HipStepper()




def _run_bitwise(O, sizes, pdt, gdt, sdt, steps=4, seed=31, threads=1, check_workspace=False, **gkw):
    _need_gpu()
    group = group_dict(bound_type="radial", **gkw)
    dual = group["buffer"] in (2, "T2")
    master = group["master_weights"] > 0 and pdt != "f32"
    host = TensorSet(sizes, pdt, gdt, sdt, dual, master, seed)
    dev = host.to("cuda")
    cfg = oracle_config(O, group)
    st = _stepper()
    label = f"radial {gkw} {pdt}/{gdt}/{sdt}"
    print(f"[case] {label} sizes={len(sizes)} max={max(sizes)}", flush=True)
    with O.radial_sum_f64():
        for s in range(1, steps + 1):
            grads = host.grads(s, seed)
            host.oracle_step(O, cfg, grads, s, threads=threads)
            dev.hip_step(st, group, [g.cuda() for g in grads], s)
            torch.cuda.synchronize()
            host.assert_equal(dev, f"{label} step {s}")
            if check_workspace:  # every call leaves the whole workspace zero, radial records included
                for ws in st.workspace._bufs.values():
                    nz = int(torch.count_nonzero(ws))
                    assert nz == 0, f"{label} step {s}: {nz} workspace bytes left set"
    return host


RADIAL_CASES = [
    (2, "f32", "f32", "f32", {}),
    ("T2", "bf16", "bf16", "f32", {}),
    (1, "f32", "f32", "f32", {"lam": 0.3}),
    ("T1", "bf16", "bf16", "f32", {}),
    ("T2", "bf16", "bf16", "f32", {"cautious": False}),
    (2, "bf16", "f32", "f32", {"master_weights": "full"}),
    ("T2", "bf16", "bf16", "f32", {"master_weights": "semi"}),
    ("T1", "f16", "f16", "f16", {"state_precision": "param"}),
    (2, "bf16", "bf16", "bf16", {"state_precision": "param"}),
    ("T2", "bf16", "bf16", "f32", {"fused_single_pass": False}),
    (1, "f32", "f32", "f32", {"cautious": False, "fused_single_pass": False, "weight_decay": 0.0}),
    ("T2", "f32", "f32", "f32", {"stochastic_rounding": False, "lr": 1e-2}),
]


@pytest.mark.parametrize("buffer,pdt,gdt,sdt,extra", RADIAL_CASES,
                         ids=[f"{c[0]}-{c[1]}-{c[2]}-{c[3]}-{i}" for i, c in enumerate(RADIAL_CASES)])
def test_radial_bitwise_vs_oracle_f64_sums(oracle_mod, buffer, pdt, gdt, sdt, extra):
    kw = dict(extra)
    kw.setdefault("lr", 1e-3)
    host = _run_bitwise(oracle_mod, RAGGED, pdt, gdt, sdt, buffer=buffer, **kw)
    # the scale is active on the large tensors (not the r < 1e-4 shortcut)
    assert float(host.sc[-1][4]) < 0.999


def test_radial_many_tensors_and_several_fold_chunks(oracle_mod):
    """64 tensors (two launches sharing the workspace records and tickets) and one tensor of
    19,532 work units, whose records the fold sums in five chunks of 4,096."""
    rng = np.random.default_rng(9)
    sizes = [int(np.exp(rng.uniform(0, np.log(2 ** 14)))) + 1 for _ in range(62)] + [20_000_003, 70_001]
    _run_bitwise(oracle_mod, sizes, "bf16", "bf16", "f32", steps=3, threads=8, buffer="T2", lr=1e-3)


@pytest.mark.parametrize("cap", ["7", "9000"])
def test_radial_launch_split_into_pieces(oracle_mod, monkeypatch, cap):
    """A radial counting launch runs in pieces (at most 2^22 units, one workspace record each)
    with a fold launch after each; a tensor's running sums carry from piece to piece and the
    piece holding its last unit finalises the scratch. LV_MAX_GRID_BLOCKS lowers the piece size:
    7 units (tensors spanning hundreds of pieces, pieces spanning tensors) and 9,000 units (the
    10M-element tensor's 8,833 units in the first piece span three fold chunks of 4,096). Bitwise
    against the oracle's f64 sums over the two-pass first step and the fused steps, and the count
    words and tickets are left zero."""
    monkeypatch.setenv("LV_MAX_GRID_BLOCKS", cap)
    _run_bitwise(oracle_mod, [100_003, 5, 66_000, 2048, 1, 10_000_000], "bf16", "bf16", "f32", steps=3,
                 check_workspace=True, buffer="T2", lr=1e-3)
    _run_bitwise(oracle_mod, [70_001, 2_100_000], "f32", "f32", "f32", steps=2, check_workspace=True, buffer=1,
                 lam=0.3, cautious=False, lr=1e-3)


def test_radial_is_deterministic(oracle_mod):
    """Two runs of the same steps from the same state give the same bits."""
    _need_gpu()
    group = group_dict(buffer="T2", bound_type="radial", lr=1e-3)
    runs = []
    for _ in range(2):
        host = TensorSet([3_000_001, 65539], "bf16", "bf16", "f32", True, False, 4)
        dev = host.to("cuda")
        st = _stepper()
        for s in (1, 2, 3):
            dev.hip_step(st, group, [g.cuda() for g in host.grads(s, 4)], s)
        torch.cuda.synchronize()
        runs.append(dev)
    for i in range(2):
        assert_bitwise(runs[0].p[i], runs[1].p[i], f"p[{i}]")
        assert_bitwise(runs[0].sc[i], runs[1].sc[i], f"scratch[{i}]")


# differential_parity.rs: 131,072 elements, 5 steps, the reference's own configurations
REF_N, REF_STEPS, REF_TOL = 131_072, 5, 1.5e-6
# Relative error of fp32 p is taken against max(|p|, REL_FLOOR): the radial scale's summation
# error moves p by at most lr * |u| * |scale error|, an absolute quantity, so relative error is
# meaningless for p near zero; 1e-3 is the learning rate of these configurations (one step's size).
REL_FLOOR = 1e-3
REF_CONFIGS = [
    # label, buffer, lr, seed, dtype, state dtype, init seed, grad seed base
    ("tdclm_fp32", 1, 1e-3, 1337, "f32", "f32", 42, 1000),   # differential_parity.rs:80-98
    ("tdclm_bf16", 1, 1e-3, 2026, "bf16", "bf16", 77, 2000),  # differential_parity.rs:166-184
    ("dual_bf16", 2, 8e-4, 31415, "bf16", "bf16", 555, 4000),  # differential_parity.rs:347-365
]


@pytest.mark.parametrize("label,buffer,lr,seed,pdt,sdt,init_seed,grad_seed", REF_CONFIGS, ids=[c[0] for c in REF_CONFIGS])
def test_radial_reference_configs_within_reference_tolerance(oracle_mod, label, buffer, lr, seed, pdt, sdt, init_seed,
                                                             grad_seed):
    _need_gpu()
    O = oracle_mod
    L = O.lib()
    idx = np.array([0, 1, 77, 131071], dtype=np.int64)
    assert [int(x) for x in prng_np(init_seed, idx)] == [L.lvo_prng(init_seed, int(i)) for i in idx]
    ema = 0.95 if buffer == 1 else 0.8
    cfg = O.make_config(lr=lr, betas=(0.9, 0.999), weight_decay=0.01, buffer=buffer, bound_type=1, cautious=True,
                        master_weights=0, stochastic_rounding=True, seed=seed, ema_decay=ema)
    group = group_dict(lr=lr, betas=(0.9, 0.999), weight_decay=0.01, buffer=buffer, bound_type="radial", cautious=True,
                       stochastic_rounding=True, seed=seed, tau=0.8, lam=0.3, eps=1e-8, cautious_clamp_min=0.5,
                       bound_ratio=0.05, ema_decay=ema, fused_single_pass=True,
                       state_precision="param" if sdt != "f32" else "fp32")
    dual = buffer == 2
    p_h = reference_pseudo_random(REF_N, init_seed, 0.5, DT[pdt])
    m_h = torch.zeros(REF_N, dtype=DT[sdt])
    v_h = torch.zeros(REF_N, dtype=DT[sdt]) if dual else None
    sc_h = torch.tensor([0, 0, 0, 1, 1, 0], dtype=torch.float32)
    p_d, m_d, sc_d = p_h.cuda(), m_h.cuda(), sc_h.cuda()
    v_d = v_h.cuda() if dual else None
    st = _stepper()
    print(f"[case] radial reference config {label}", flush=True)
    for s in range(1, REF_STEPS + 1):
        g = reference_pseudo_random(REF_N, grad_seed + (s - 1), 0.05, DT[pdt])
        O.step(cfg, [p_h], [g], [m_h], [v_h], [None], [sc_h], [s], [0])  # scalar core's f32 order
        st.step(group, [p_d], [g.cuda()], [m_d], [v_d], [None], [sc_d], [s], [0])
        torch.cuda.synchronize()
        # the scale never feeds m and v: bitwise
        assert_bitwise(m_h, m_d, f"{label} m step {s}")
        if dual:
            assert_bitwise(v_h, v_d, f"{label} v step {s}")
        ph, pd = p_h.float(), p_d.cpu().float()
        if pdt == "f32":
            assert float((ph - pd).abs().max()) <= REF_TOL, f"{label} step {s}"
            # the north star's per-element bound: 1e-6 relative, with |p| floored at REL_FLOOR
            rel = ((ph - pd).abs() / ph.abs().clamp_min(REL_FLOOR)).double()
            k = int(rel.argmax())
            print(f"[radial] {label} step {s}: max rel {float(rel[k]):.3e} at |p| = {abs(float(ph[k])):.3e}, "
                  f"max abs {float((ph - pd).abs().max()):.3e}", flush=True)
            assert float(rel[k]) <= 1e-6, f"{label} step {s}: element {k} rel {float(rel[k]):.3e}"
        else:
            bh, bd = bits(p_h), bits(p_d)
            off = np.abs(bh - bd)
            assert off.max() <= 1, f"{label} step {s}: more than 1 bf16 ULP apart"
            assert np.count_nonzero(off) <= REF_N // 1000, f"{label} step {s}: {np.count_nonzero(off)} flips"
        sh, sd = sc_h.numpy(), sc_d.cpu().numpy()
        assert sh[0] == sd[0] == 0 and sh[1] == sd[1] == 0 and sh[2] == sd[2] == 0 and sh[5] == sd[5] == 0
        assert abs(sh[3] - sd[3]) <= REF_TOL, f"{label} cautious scale step {s}"
        gamma = (REF_N // 16) * 2.0 ** -24  # f32 lane-sum bound of the reference order
        assert abs(sh[4] - sd[4]) <= gamma * abs(sh[4]), f"{label} bound scale step {s}: {sh[4]} vs {sd[4]}"
    assert sd[4] < 0.9999, "the radial scale should be active in these configurations"
