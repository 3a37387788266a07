"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle, bit for bit.

Every case runs several steps (step 1 takes the two-pass path when cautious, later steps the
fused lagged-scale pass) over ragged multi-tensor lists, and compares p, m, v, master and the
6-float scratch after every step. The bar is bitwise equality (fp32 and bf16 alike), which is
stricter than the 1e-6 relative / 1 bf16 ULP tolerance of the target.
"""
from __future__ import annotations

import sys

import pytest
import torch

from tests.parity_util import TensorSet, assert_bitwise, group_dict, oracle_config, seeded_tensor

pytestmark = pytest.mark.gpu

RAGGED = [1, 7, 2047, 2048, 2049, 8191, 65539, 100_000]


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


def _stepper():
    from luminamoon_amd.optimizer.hip_backend import HipStepper

    return HipStepper()


def _run_case(oracle_mod, sizes, pdt, gdt, sdt, steps=5, seed=7, **gkw):
    _need_gpu()
    O = oracle_mod
    group = group_dict(**gkw)
    dual = group["buffer"] in (2, "T2")
    master = group["master_weights"] > 0 and pdt != "f32"
    host = TensorSet(sizes, pdt, gdt, sdt, dual, master, seed)
    dev = host.to("cuda")
    cfg = oracle_config(O, group)
    st = _stepper()
    label = f"{gkw} {pdt}/{gdt}/{sdt}"
    print(f"[case] {label} sizes={len(sizes)}", flush=True)
    for s in range(1, steps + 1):
        grads = host.grads(s, seed)
        host.oracle_step(O, cfg, grads, s)
        dev.hip_step(st, group, [g.cuda() for g in grads], s)
        torch.cuda.synchronize()
        host.assert_equal(dev, f"{label} step {s}")


CASES = [
    # buffer, pdt, gdt, sdt, extra group kwargs
    (2, "f32", "f32", "f32", {}),
    (1, "f32", "f32", "f32", {"lam": 0.3}),
    ("T1", "bf16", "bf16", "f32", {}),
    ("T2", "bf16", "bf16", "f32", {}),
    (2, "bf16", "bf16", "f32", {}),
    (1, "bf16", "bf16", "f32", {}),
    (2, "bf16", "bf16", "bf16", {"state_precision": "param"}),
    ("T2", "bf16", "bf16", "bf16", {"state_precision": "param"}),
    (2, "f16", "f16", "f16", {"state_precision": "param"}),
    ("T1", "f16", "f16", "f16", {"state_precision": "param"}),
    ("T2", "f16", "f16", "f32", {}),
    (2, "bf16", "f32", "f32", {"master_weights": "full"}),
    ("T2", "bf16", "bf16", "f32", {"master_weights": "semi"}),
    (1, "f16", "f16", "f32", {"master_weights": "full"}),
    (2, "f32", "f32", "f32", {"cautious": False}),
    ("T2", "bf16", "bf16", "f32", {"cautious": False, "stochastic_rounding": False}),
    (1, "f32", "f32", "f32", {"cautious": False, "bound": False, "bound_type": "none"}),
    ("T1", "bf16", "bf16", "f32", {"fused_single_pass": False}),
    (2, "f32", "f32", "f32", {"fused_single_pass": False, "weight_decay": 0.0}),
    ("T2", "f32", "f32", "f32", {"stochastic_rounding": False, "lr": 1e-2}),
]


@pytest.mark.parametrize("buffer,pdt,gdt,sdt,extra", CASES, ids=[f"{c[0]}-{c[1]}-{c[2]}-{c[3]}-{i}" for i, c in enumerate(CASES)])
def test_hip_matches_oracle(oracle_mod, buffer, pdt, gdt, sdt, extra):
    kw = dict(extra)
    kw.setdefault("lr", 1e-3)
    _run_case(oracle_mod, RAGGED, pdt, gdt, sdt, buffer=buffer, **kw)


def test_many_tensors_multiple_launches(oracle_mod):
    """64 ragged tensors (more than one kernel-argument table: one table launch) in one call."""
    import numpy as np

    rng = np.random.default_rng(3)
    sizes = [int(np.exp(rng.uniform(0, np.log(2 ** 14)))) + 1 for _ in range(64)]
    _run_case(oracle_mod, sizes, "f32", "f32", "f32", steps=4, buffer=1, lr=8e-4)


# Leading workspace bytes that must be zero between calls (48 x 65 count words 64 B apart and
# 512 B of radial tickets), and the count words of table launches (960 tensors) that follow the
# fixed regions.
ZERO_BYTES = 48 * 65 * 64 + 512
TABLE_SLOT_BYTES = 960 * 65 * 64


@pytest.mark.parametrize("count,buffer,pdt,sdt,extra", [
    (1000, "T2", "bf16", "f32", {}),
    (2000, 1, "f32", "f32", {"lam": 0.3}),
    (1000, 2, "bf16", "f32", {"master_weights": "full"}),
    (1000, 2, "f32", "f32", {"cautious": False}),
    (1000, "T1", "bf16", "bf16", {"state_precision": "param", "fused_single_pass": False}),
], ids=["T2-bf16-1000", "TDCLM-f32-2000", "CLM-master-1000", "CLM-nocautious-1000", "T1-bf16state-twopass-1000"])
def test_table_launches_thousands_of_tensors(oracle_mod, count, buffer, pdt, sdt, extra):
    """More tensors than the kernel-argument table holds: the descriptors go to the workspace
    (up to 960 per launch, the first units stay in the kernel arguments), so 1000 ragged tensors
    are one table launch and an inline launch of 40, and 2000 are 960 + 960 + 80. Every buffer
    and scratch bit for bit over the two-pass first step and fused steps; the count words of both
    kinds of launch are left zero."""
    _table_case(oracle_mod, count, buffer, pdt, sdt, extra)


def test_table_launch_split_into_pieces(oracle_mod, monkeypatch):
    """A table launch cut into pieces of 37 blocks (LV_MAX_GRID_BLOCKS): each piece finds its
    tensors through the first units in the kernel arguments, and counts fold across pieces."""
    monkeypatch.setenv("LV_MAX_GRID_BLOCKS", "37")
    _table_case(oracle_mod, 100, "T2", "bf16", "f32", {})


def test_table_launches_from_two_host_threads(oracle_mod):
    """Two host threads, each with its own stepper (workspace) and stream, step 100-tensor sets
    at the same time: table launches share the device's pinned staging ring, whose slots are
    leased to one call at a time. Both end bit for bit equal to the oracle."""
    import threading

    import numpy as np

    _need_gpu()
    O = oracle_mod
    group = group_dict(buffer="T2", lr=1e-3)
    cfg = oracle_config(O, group)
    rng = np.random.default_rng(5)
    sets = []
    for k in range(2):
        sizes = [int(np.exp(rng.uniform(0, np.log(5000)))) + 1 for _ in range(100)]
        host = TensorSet(sizes, "bf16", "bf16", "f32", True, False, 40 + k)
        sets.append((host, host.to("cuda"), _stepper(), torch.cuda.Stream()))
    steps = 6
    grads = [[host.grads(s, 50 + k) for s in range(1, steps + 1)] for k, (host, _, _, _) in enumerate(sets)]
    dev_grads = [[[g.cuda() for g in gs] for gs in per] for per in grads]
    torch.cuda.synchronize()
    errors = []

    def run(k):
        try:
            host, dev, st, stream = sets[k]
            with torch.cuda.stream(stream):
                for s in range(1, steps + 1):
                    dev.hip_step(st, group, dev_grads[k][s - 1], s)
            stream.synchronize()
        except Exception as e:  # reported below, on the main thread
            errors.append(e)

    threads = [threading.Thread(target=run, args=(k,)) for k in range(2)]
    print("[case] table launches from two host threads", flush=True)
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for k, (host, dev, _, _) in enumerate(sets):
        for s in range(1, steps + 1):
            host.oracle_step(O, cfg, grads[k][s - 1], s)
        host.assert_equal(dev, f"thread {k}")


def _table_case(oracle_mod, count, buffer, pdt, sdt, extra):
    """`count` ragged tensors (plus three larger ones) stepped three times, bitwise against the
    oracle, with the count words of inline and table launches checked zero after every step."""
    import numpy as np

    _need_gpu()
    O = oracle_mod
    rng = np.random.default_rng(count + 7)
    sizes = [int(np.exp(rng.uniform(0, np.log(2 ** 12)))) + 1 for _ in range(count - 3)] + [100_003, 2048, 70_001]
    kw = dict(extra)
    kw.setdefault("lr", 1e-3)
    group = group_dict(buffer=buffer, **kw)
    dual = group["buffer"] in (2, "T2")
    master = group["master_weights"] > 0 and pdt != "f32"
    host = TensorSet(sizes, pdt, pdt, sdt, dual, master, 13)
    dev = host.to("cuda")
    cfg = oracle_config(O, group)
    st = _stepper()
    print(f"[case] table launch {count} tensors buffer={buffer} {pdt}/{sdt} {extra}", flush=True)
    for s in range(1, 4):
        grads = host.grads(s, 13)
        host.oracle_step(O, cfg, grads, s, threads=8)
        dev.hip_step(st, group, [g.cuda() for g in grads], s)
        torch.cuda.synchronize()
        host.assert_equal(dev, f"{count} tensors step {s}")
        for ws in st.workspace._bufs.values():
            assert int(torch.count_nonzero(ws[:ZERO_BYTES])) == 0, f"count words left set (step {s})"
            from luminamoon_amd.optimizer import hip_backend

            fixed = int(hip_backend.load_library().lv_workspace_bytes(1))
            table_words = ws[fixed:fixed + TABLE_SLOT_BYTES]
            assert table_words.numel() == TABLE_SLOT_BYTES
            assert int(torch.count_nonzero(table_words)) == 0, f"table count words left set (step {s})"


def test_mixed_steps_in_one_call(oracle_mod):
    """Tensors at different step counts in one call go to separate launch classes."""
    _need_gpu()
    O = oracle_mod
    group = group_dict(buffer="T2", lr=1e-3)
    cfg = oracle_config(O, group)
    host = TensorSet([5000, 3000, 7001], "bf16", "bf16", "f32", True, False, 11)
    dev = host.to("cuda")
    st = _stepper()
    steps = [1, 3, 2]
    for rnd in range(3):
        grads = host.grads(rnd + 1, 11)
        cur = [s + rnd for s in steps]
        O.step(cfg, host.p, grads, host.m, host.v, host.mp, host.sc, cur, [0, 1, 2])
        st.step(group, dev.p, [g.cuda() for g in grads], dev.m, dev.v, dev.mp, dev.sc, cur, [0, 1, 2])
        torch.cuda.synchronize()
        host.assert_equal(dev, f"mixed round {rnd}")


def test_unaligned_views_use_scalar_path(oracle_mod):
    """Tensors at odd element offsets (not 16-byte aligned) take the per-element path."""
    _need_gpu()
    O = oracle_mod
    group = group_dict(buffer=2, lr=1e-3)
    cfg = oracle_config(O, group)
    n = 10_001
    host = TensorSet([n], "bf16", "bf16", "f32", True, False, 5)
    dev = host.to("cuda")

    def shift(t):
        big = torch.zeros(t.numel() + 1, dtype=t.dtype, device=t.device)
        big[1:].copy_(t)
        return big[1:]

    dev.p, dev.m, dev.v = [shift(dev.p[0])], [shift(dev.m[0])], [shift(dev.v[0])]
    st = _stepper()
    for s in range(1, 4):
        grads = host.grads(s, 5)
        host.oracle_step(O, cfg, grads, s)
        g_dev = shift(grads[0].cuda())
        st.step(group, dev.p, [g_dev], dev.m, dev.v, dev.mp, dev.sc, [s], [0])
        torch.cuda.synchronize()
        host.assert_equal(dev, f"unaligned step {s}")


def test_param_index_seeds_and_large_step(oracle_mod):
    """Non-zero param_index and step counts far from 1 (seed derivation, bias correction)."""
    _need_gpu()
    O = oracle_mod
    group = group_dict(buffer="T2", lr=1e-3)
    cfg = oracle_config(O, group)
    host = TensorSet([4099, 513], "bf16", "bf16", "f32", True, False, 9)
    dev = host.to("cuda")
    st = _stepper()
    pidx = [123456789, 7]
    for s in (1, 2, 1000, 123457):
        grads = host.grads(s % 97, 9)
        O.step(cfg, host.p, grads, host.m, host.v, host.mp, host.sc, [s, s], pidx)
        st.step(group, dev.p, [g.cuda() for g in grads], dev.m, dev.v, dev.mp, dev.sc, [s, s], pidx)
        torch.cuda.synchronize()
        host.assert_equal(dev, f"step {s}")


def test_luminav_readme_example_100_steps(oracle_mod):
    """Config 1: LuminaV(buffer=2) on W[64,10] ~ N(0,1), b[10] = 0, grads N(0,1) from seed 0,
    100 steps; final params, m, v and scratch bitwise equal to the oracle."""
    _need_gpu()
    import numpy as np
    from luminamoon_amd import LuminaV

    O = oracle_mod
    rng = np.random.default_rng(0)
    W0 = rng.standard_normal((64, 10)).astype(np.float32)
    b0 = np.zeros(10, dtype=np.float32)
    gW, gb = [], []
    for _ in range(100):  # draw order: W, then per step gW, gb
        gW.append(rng.standard_normal((64, 10)).astype(np.float32))
        gb.append(rng.standard_normal(10).astype(np.float32))
    W = torch.nn.Parameter(torch.from_numpy(W0).cuda())
    b = torch.nn.Parameter(torch.from_numpy(b0).cuda())
    opt = LuminaV([W, b], lr=8e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.08, tau=0.8, buffer=2)
    group = group_dict(lr=8e-4, weight_decay=0.08, buffer=2)
    cfg = oracle_config(O, group)
    hp = [torch.from_numpy(W0.copy()).reshape(-1), torch.from_numpy(b0.copy())]
    hm = [torch.zeros(640), torch.zeros(10)]
    hv = [torch.zeros(640), torch.zeros(10)]
    hs = [torch.tensor([0, 0, 0, 1, 1, 0], dtype=torch.float32) for _ in range(2)]
    for t in range(100):
        W.grad = torch.from_numpy(gW[t]).cuda()
        b.grad = torch.from_numpy(gb[t]).cuda()
        opt.step()
        O.step(cfg, hp, [torch.from_numpy(gW[t]).reshape(-1), torch.from_numpy(gb[t])], hm, hv, [None, None], hs,
               [t + 1, t + 1], [0, 1])
    torch.cuda.synchronize()
    assert_bitwise(hp[0], W.detach().reshape(-1), "W")
    assert_bitwise(hp[1], b.detach(), "b")
    for i, p in enumerate((W, b)):
        st = opt.state[p]
        assert st["step"] == 100
        assert_bitwise(hm[i], st["exp_avg"].reshape(-1), f"m[{i}]")
        assert_bitwise(hv[i], st["exp_avg_sq"].reshape(-1), f"v[{i}]")
        assert_bitwise(hs[i], st["scratch"], f"scratch[{i}]")


def test_luminav_fused_bucket_matches_oracle_on_flat_buffer(oracle_mod):
    """fuse_tensors=True steps one bucket with param_index 0 and bucket-global offsets."""
    _need_gpu()
    from luminamoon_amd import LuminaV

    O = oracle_mod
    shapes = [(33, 17), (17,), (128, 64), (3,), (255, 9)]
    torch.manual_seed(0)
    params = [torch.nn.Parameter((torch.randn(s) * 0.02).to(torch.bfloat16).cuda()) for s in shapes]
    opt = LuminaV(params, lr=1e-3, buffer="T2", cautious=True, fuse_tensors=True)
    bucket = opt._fused_buckets[0]
    n = bucket["flat_p"].numel()
    group = group_dict(lr=1e-3, buffer="T2", fuse_tensors=True)
    cfg = oracle_config(O, group)
    hp = bucket["flat_p"].detach().cpu().clone()
    hm, hv = torch.zeros(n), torch.zeros(n)
    hs = torch.tensor([0, 0, 0, 1, 1, 0], dtype=torch.float32)
    for t in range(1, 6):
        g = seeded_tensor(n, 100 + t, 1e-3, torch.bfloat16)
        off = 0
        for p in params:
            k = p.numel()
            p.grad.copy_(g[off:off + k].view(p.shape).cuda())
            off += k
        opt.step()
        O.step(cfg, [hp], [g], [hm], [hv], [None], [hs], [t], [0])
    torch.cuda.synchronize()
    assert_bitwise(hp, bucket["flat_p"], "flat_p")
    assert_bitwise(hm, bucket["flat_m"], "flat_m")
    assert_bitwise(hv, bucket["flat_v"], "flat_v")
    assert_bitwise(hs, bucket["scratch"], "scratch")


def test_mask_count_exact_above_2_pow_24(oracle_mod):
    """The cautious count is an exact integer: above 2^24 elements a float count would drift.
    Compares the scratch after a two-pass and a fused step on 2^25 + 3 elements."""
    _need_gpu()
    O = oracle_mod
    group = group_dict(buffer="T2", lr=1e-3)
    cfg = oracle_config(O, group)
    n = (1 << 25) + 3
    host = TensorSet([n], "bf16", "bf16", "f32", True, False, 21)
    dev = host.to("cuda")
    st = _stepper()
    for s in (1, 2):
        grads = host.grads(s, 21)
        host.oracle_step(O, cfg, grads, s, threads=8)
        dev.hip_step(st, group, [g.cuda() for g in grads], s)
        torch.cuda.synchronize()
        host.assert_equal(dev, f"2^25 step {s}")



@pytest.mark.parametrize("buffer,pdt,sdt", [("T2", "bf16", "f32"), ("T1", "bf16", "f32"), (2, "f32", "f32")])
def test_unit_launch_split_into_pieces(oracle_mod, monkeypatch, buffer, pdt, sdt):
    """A unit launch larger than the per-launch block cap runs as several pieces (unit_base);
    LV_MAX_GRID_BLOCKS lowers the cap so small tensors exercise it: pieces of 7 blocks (fewer
    than the 8 XCDs) and of 37 blocks, cutting across tensor boundaries, equal the oracle. The
    mask-count words of a tensor split over pieces fold in whichever piece runs its last block,
    and every call leaves the workspace's count words zeroed."""
    _need_gpu()
    O = oracle_mod
    group = group_dict(buffer=buffer)
    dual = group["buffer"] in (2, "T2")
    sizes = [100_003, 5, 66_000, 2048, 1]
    for cap in ("7", "37"):
        monkeypatch.setenv("LV_MAX_GRID_BLOCKS", cap)
        host = TensorSet(sizes, pdt, pdt, sdt, dual, False, seed=19, m_scale=1e-3)
        dev = host.to("cuda")
        cfg = oracle_config(O, group)
        st = _stepper()
        print(f"[case] split launch cap={cap} buffer={buffer} {pdt}", flush=True)
        for s in range(1, 4):
            grads = host.grads(s, seed=23)
            host.oracle_step(O, cfg, grads, s)
            dev.hip_step(st, group, [g.cuda() for g in grads], s)
            torch.cuda.synchronize()
            host.assert_equal(dev, f"cap {cap} step {s}")
            for ws in st.workspace._bufs.values():  # count words + radial tickets
                zero = ws[:48 * 65 * 64 + 512]
                assert int(torch.count_nonzero(zero)) == 0, f"workspace not left zeroed (cap {cap} step {s})"


@pytest.mark.parametrize("buffer", [1, 2, 3, 4])
@pytest.mark.parametrize("cautious,bound_mode", [(1, 2), (0, 2), (1, 0)])
def test_lv_step_f32_matches_oracle(oracle_mod, buffer, cautious, bound_mode):
    """lv_step_f32, the argument-for-argument twin of the reference's luminav_triton_step_f32
    (luminav_triton_standalone.h:89-111), called through the C ABI on device pointers: four steps
    (two-pass, then fused) bitwise equal to the oracle with the reference's defaults for the
    rest (ema_decay per buffer mode, clamp_min 0.5, SR and fused single pass on)."""
    _need_gpu()
    import ctypes

    import numpy as np

    from luminamoon_amd.optimizer import hip_backend

    O = oracle_mod
    L = hip_backend.load_library()
    n = 70_001
    dual = buffer in (2, 4)
    rng = np.random.default_rng(31 + buffer)
    p0 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    hp, hm = torch.from_numpy(p0.copy()), torch.zeros(n)
    hv = torch.zeros(n) if dual else None
    hs = torch.tensor([0, 0, 0, 1, 1, 0], dtype=torch.float32)
    dp, dm = hp.clone().cuda(), hm.clone().cuda()
    dv = hv.clone().cuda() if dual else None
    ds = hs.clone().cuda()
    code = {1: 1, 2: 2, 3: "T1", 4: "T2"}[buffer]
    cfg = O.make_config(lr=1e-3, buffer=code, cautious=bool(cautious), bound_type=bound_mode, seed=77)
    stream = torch.cuda.current_stream().cuda_stream
    for t in range(1, 5):
        g = torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32))
        dg = g.cuda()
        rc = L.lv_step_f32(dp.data_ptr(), dg.data_ptr(), dm.data_ptr(), dv.data_ptr() if dual else None, None,
                           ds.data_ptr(), n, 1e-3, 0.9, 0.999, 1e-8, 0.08, 0.8, 0.3, buffer, cautious, bound_mode,
                           0.05, t, 77, ctypes.c_void_p(stream))
        assert rc == 0, L.lv_last_error()
        O.step(cfg, [hp], [g], [hm], [hv], [None], [hs], [t], [0])
        torch.cuda.synchronize()
        assert_bitwise(hp, dp, f"step {t} p")
        assert_bitwise(hm, dm, f"step {t} m")
        if dual:
            assert_bitwise(hv, dv, f"step {t} v")
        assert_bitwise(hs, ds, f"step {t} scratch")


if __name__ == "__main__":
    sys.exit(pytest.main([__file__, "-v"]))
