"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle, bit for bit.

Every case runs several steps (step 1 takes the two-pass path when cautious, later steps the
fused lagged-scale pass) over ragged multi-tensor lists, and compares p, m, v, master and the
6-float scratch after every step. The bar is bitwise equality (fp32 and bf16 alike), which is
stricter than the 1e-6 relative / 1 bf16 ULP tolerance of the target.
"""
from __future__ import annotations

import contextlib
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
    # radial sums: the kernels' f64 sums, bitwise against the oracle's f64 sum mode (test_gpu_radial.py)
    radial = group["bound"] and group["bound_type"] == 1
    with (O.radial_sum_f64() if radial else contextlib.nullcontext()):
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
    # 16-bit state with an f32 stream beside it: the split lane layout of 2048-element units
    ("T2", "bf16", "bf16", "bf16", {"state_precision": "param", "master_weights": "semi"}),
    ("T1", "bf16", "f32", "bf16", {"state_precision": "param"}),
    (2, "f16", "f16", "f16", {"state_precision": "param", "master_weights": "semi"}),
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


def assert_workspace_zero(stepper, label):
    """Every call leaves the whole workspace zero (count slots, tickets and radial records)."""
    for ws in stepper.workspace._bufs.values():
        nz = int(torch.count_nonzero(ws))
        assert nz == 0, f"{label}: {nz} workspace bytes left set"


@pytest.mark.parametrize("count,buffer,pdt,sdt,extra", [
    (1000, "T2", "bf16", "f32", {}),
    (2000, 1, "f32", "f32", {"lam": 0.3}),
    (5000, 1, "f32", "f32", {"lam": 0.3, "cautious": True}),
    (1000, 2, "bf16", "f32", {"master_weights": "full"}),
    (1000, 2, "f32", "f32", {"cautious": False}),
    (1000, "T1", "bf16", "bf16", {"state_precision": "param", "fused_single_pass": False}),
    (1000, "T1", "f16", "f16", {"state_precision": "param"}),
], ids=["T2-bf16-1000", "TDCLM-f32-2000", "TDCLM-f32-5000", "CLM-master-1000", "CLM-nocautious-1000",
        "T1-bf16state-twopass-1000", "T1-f16-fp16container-1000"])
def test_table_launches_thousands_of_tensors(oracle_mod, count, buffer, pdt, sdt, extra):
    """More tensors than the kernel-argument table holds: every class is ONE table launch (pair)
    whatever its tensor count, its descriptors in a device table and every group-th tensor's first
    unit in the kernel arguments (2000 tensors: groups of 3; 5000: groups of 6, a second binary
    search in the device table). Every buffer and scratch bit for bit over the two-pass first step
    and fused steps; the whole workspace is left zero."""
    _table_case(oracle_mod, count, buffer, pdt, sdt, extra)


def test_table_upload_skipped_and_reused(oracle_mod):
    """Descriptor tables stay on the device: a step whose table equals one already uploaded
    launches with no upload. Grads alternate between two buffer sets (tables A, B, A, B, ...) and
    a third set appears once (a fresh upload into the least recently used slot); every step bit
    for bit against the oracle."""
    import numpy as np

    _need_gpu()
    O = oracle_mod
    group = group_dict(buffer="T2", lr=1e-3)
    cfg = oracle_config(O, group)
    rng = np.random.default_rng(8)
    sizes = [int(np.exp(rng.uniform(0, np.log(9000)))) + 1 for _ in range(120)]
    host = TensorSet(sizes, "bf16", "bf16", "f32", True, False, 21)
    dev = host.to("cuda")
    st = _stepper()
    bufs = [[torch.empty(n, dtype=torch.bfloat16, device="cuda") for n in sizes] for _ in range(3)]
    print("[case] table upload skip", flush=True)
    for s, which in enumerate((0, 1, 0, 1, 2, 0, 0, 1), start=1):
        grads = host.grads(s, 21)
        for b, g in zip(bufs[which], grads):
            b.copy_(g)
        host.oracle_step(O, cfg, grads, s)
        dev.hip_step(st, group, bufs[which], s)
        torch.cuda.synchronize()
        host.assert_equal(dev, f"step {s} (grad set {which})")
        assert_workspace_zero(st, f"step {s}")


PARTIAL = [1, 3, 4, 5, 1021, 1023, 1024, 1025, 1027, 2045, 2047, 2048, 2049, 3075, 4097, 6143, 65541]


@pytest.mark.parametrize("buffer,pdt,sdt,extra", [
    ("T2", "bf16", "f32", {}),
    ("T2", "bf16", "bf16", {"state_precision": "param"}),
    (2, "f32", "f32", {}),
    (1, "f16", "f16", {"state_precision": "param"}),
    ("T1", "bf16", "f32", {"bound_type": "radial"}),
])
def test_partial_units_keep_the_vector_layout(oracle_mod, buffer, pdt, sdt, extra):
    """A tensor's last, partial unit: every thread's 4-element groups that lie wholly inside the
    tensor take the vector path and only the group straddling the end goes element by element
    (1024-element units with f32 state, 2048 with 16-bit state: sizes around both)."""
    kw = dict(extra)
    kw.setdefault("lr", 1e-3)
    _run_case(oracle_mod, PARTIAL, pdt, pdt, sdt, steps=4, buffer=buffer, **kw)


def test_v_clamp_follows_param_dtype_with_fp16_state_container(oracle_mod):
    """dual.rs:68 clamps v at 65000 for fp16 params only on the reference's native path: the FFI
    worker hands an fp16 state container to the core as bitwise bf16 (worker.rs:107-113). A bf16
    param with an fp16 state container and gradients large enough that v exceeds 65000 keeps the
    unclamped v; an fp16 param is clamped. Through the C ABI, bitwise against the oracle."""
    _need_gpu()
    O = oracle_mod
    for buffer in (2, "T2"):
        for pdt in ("bf16", "f32", "f16"):
            group = group_dict(buffer=buffer, lr=1e-3)
            cfg = oracle_config(O, group)
            host = TensorSet([5000, 2048], pdt, pdt, "f16", True, False, 3)
            dev = host.to("cuda")
            st = _stepper()
            print(f"[case] v clamp buffer={buffer} {pdt} + fp16 state container", flush=True)
            for s in range(1, 4):
                grads = host.grads(s, 3, scale=1.0e4, zero_frac=0.0)
                host.oracle_step(O, cfg, grads, s)
                dev.hip_step(st, group, [g.cuda() for g in grads], s)
                torch.cuda.synchronize()
                host.assert_equal(dev, f"buffer={buffer} {pdt} step {s}")
            vmax = float(dev.v[0].view(torch.bfloat16).float().max())
            assert (vmax <= 65024.0) == (pdt == "f16"), (buffer, pdt, vmax)


def test_table_launch_split_into_pieces(oracle_mod, monkeypatch):
    """A table launch cut into pieces of 37 blocks (LV_MAX_GRID_BLOCKS): each piece finds its
    tensors through the heads in the kernel arguments, and counts fold across pieces."""
    monkeypatch.setenv("LV_MAX_GRID_BLOCKS", "37")
    _table_case(oracle_mod, 100, "T2", "bf16", "f32", {})


def test_table_launches_from_two_host_threads(oracle_mod):
    """Two host threads, each with its own stepper (workspace) and stream, step 100-tensor sets
    at the same time: table launches share the device's descriptor-table ring, whose slots are
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



def test_table_reuse_on_the_null_stream_then_other_streams_and_evictions(oracle_mod):
    """A table launch that reuses its descriptor-table slot on the null stream after null-stream
    readers records no event (the slot is marked pending). One 100-tensor set keeps its grads in
    fixed buffers, so every step reuses the same table: steps 1-3 on the null stream (an upload,
    then two deferred reuses), step 4 on a side stream (the reuse records the pending event and
    waits for it), step 5 on the null stream again, then five other sets on the null stream,
    which rewrite every slot of the device's ring (the pending one included), and step 6 of the
    first set (a fresh upload). Every set ends bit for bit equal to the oracle."""
    import numpy as np

    _need_gpu()
    O = oracle_mod
    group = group_dict(buffer="T2", lr=1e-3)
    cfg = oracle_config(O, group)
    rng = np.random.default_rng(11)

    def make(seed):
        sizes = [int(np.exp(rng.uniform(0, np.log(5000)))) + 1 for _ in range(100)]
        host = TensorSet(sizes, "bf16", "bf16", "f32", True, False, seed)
        return host, host.to("cuda"), _stepper()

    host, dev, st = make(60)
    gbufs = [g.cuda() for g in host.grads(1, 70)]  # fixed addresses: the table stays the same
    side = torch.cuda.Stream()

    def step(s, stream=None):
        gs = host.grads(s, 70 + s)
        ctx = torch.cuda.stream(stream) if stream is not None else torch.cuda.stream(torch.cuda.default_stream())
        with ctx:
            for buf, g in zip(gbufs, gs):
                buf.copy_(g, non_blocking=False)
            dev.hip_step(st, group, gbufs, s)
        host.oracle_step(O, cfg, gs, s)

    print("[case] table reuse: null stream x3, side stream, null stream", flush=True)
    for s in (1, 2, 3):
        step(s)
    torch.cuda.default_stream().synchronize()
    step(4, side)
    side.synchronize()
    step(5)
    torch.cuda.synchronize()
    host.assert_equal(dev, "after the stream changes")
    print("[case] table reuse: five other sets rewrite the ring", flush=True)
    others = [make(80 + k) for k in range(5)]
    for k, (h2, d2, st2) in enumerate(others):
        for s in (1, 2):
            gs = h2.grads(s, 90 + 10 * k + s)
            d2.hip_step(st2, group, [g.cuda() for g in gs], s)
            h2.oracle_step(O, cfg, gs, s)
    step(6)
    torch.cuda.synchronize()
    host.assert_equal(dev, "after the evictions")
    for k, (h2, d2, _) in enumerate(others):
        h2.assert_equal(d2, f"other set {k}")

def _table_case(oracle_mod, count, buffer, pdt, sdt, extra):
    """`count` ragged tensors (plus three larger ones) stepped three times, bitwise against the
    oracle, with the whole workspace checked zero after every step."""
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
        assert_workspace_zero(st, f"{count} tensors step {s}")


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


def test_unaligned_views_by_one_element(oracle_mod):
    """A tensor whose buffers all start one element past a 16-byte boundary: the vector path from
    its first element on a 128-byte line, with the head before it taken by its last block."""
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
            assert_workspace_zero(st, f"cap {cap} step {s}")


@pytest.mark.parametrize("buffer", [1, 2])
@pytest.mark.parametrize("cautious,bound_mode", [(1, 2), (0, 2), (1, 0), (1, 5)])
@pytest.mark.parametrize("master", [False, True])
def test_lv_step_f32_matches_oracle(oracle_mod, buffer, cautious, bound_mode, master):
    """lv_step_f32 with the argument mapping of the reference's luminav_triton_step_f32
    (c_api.rs:108-199) on device pointers: buffer_mode 1 TD-CLM, 2 the dual buffer; bound_mode 1
    radial, 2 coordinate, anything else none; master weights iff a master buffer is passed;
    ema_decay per buffer mode, clamp_min 0.5, stochastic rounding off, fused single pass on. Four
    steps (two-pass, then fused) bitwise equal to the oracle with that configuration."""
    _need_gpu()
    import ctypes

    import numpy as np

    from luminamoon_amd.optimizer import hip_backend

    O = oracle_mod
    L = hip_backend.load_library()
    n = 70_001
    dual = buffer == 2
    rng = np.random.default_rng(31 + buffer + 2 * bound_mode)
    p0 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    hp, hm = torch.from_numpy(p0.copy()), torch.zeros(n)
    hv = torch.zeros(n) if dual else None
    hmp = torch.from_numpy((p0 + 1e-4).astype(np.float32)) if master else None
    hs = torch.tensor([0, 0, 0, 1, 1, 0], dtype=torch.float32)
    dp, dm = hp.clone().cuda(), hm.clone().cuda()
    dv = hv.clone().cuda() if dual else None
    dmp = hmp.clone().cuda() if master else None
    ds = hs.clone().cuda()
    cfg = O.make_config(lr=1e-3, buffer=buffer, cautious=bool(cautious), bound=bound_mode > 0,
                        bound_type=bound_mode if bound_mode in (1, 2) else 0, seed=77, stochastic_rounding=False,
                        master_weights=2 if master else 0)
    stream = torch.cuda.current_stream().cuda_stream
    for t in range(1, 5):
        g = torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32))
        dg = g.cuda()
        rc = L.lv_step_f32(dp.data_ptr(), dg.data_ptr(), dm.data_ptr(), dv.data_ptr() if dual else None,
                           dmp.data_ptr() if master else None, ds.data_ptr(), n, 1e-3, 0.9, 0.999, 1e-8, 0.08, 0.8,
                           0.3, buffer, cautious, bound_mode, 0.05, t, 77, ctypes.c_void_p(stream))
        assert rc == 0, L.lv_last_error()
        O.step(cfg, [hp], [g], [hm], [hv], [hmp], [hs], [t], [0])
        torch.cuda.synchronize()
        assert_bitwise(hp, dp, f"step {t} p")
        assert_bitwise(hm, dm, f"step {t} m")
        if dual:
            assert_bitwise(hv, dv, f"step {t} v")
        if master:
            assert_bitwise(hmp, dmp, f"step {t} master")
        assert_bitwise(hs, ds, f"step {t} scratch")


def test_lv_step_f32_reference_mode_mapping(oracle_mod):
    """Every buffer_mode other than 1 is the dual buffer, which needs exp_avg_sq, and exp_avg_sq
    is taken only for buffer_mode 2 (c_api.rs:120-146): modes 3, 4 and 7, and mode 2 without
    exp_avg_sq, fail with -4 and leave the buffers untouched; an invalid hyper-parameter is -4 too
    (c_api.rs:178-181)."""
    _need_gpu()
    import ctypes

    from luminamoon_amd.optimizer import hip_backend

    L = hip_backend.load_library()
    n = 4096
    p = torch.randn(n, device="cuda") * 0.02
    g, m, v = torch.randn(n, device="cuda") * 1e-3, torch.zeros(n, device="cuda"), torch.zeros(n, device="cuda")
    sc = torch.tensor([0, 0, 0, 1, 1, 0], dtype=torch.float32, device="cuda")
    p0 = p.clone()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for mode, vv in ((3, v), (4, v), (7, v), (2, None)):
        rc = L.lv_step_f32(p.data_ptr(), g.data_ptr(), m.data_ptr(), vv.data_ptr() if vv is not None else None, None,
                           sc.data_ptr(), n, 1e-3, 0.9, 0.999, 1e-8, 0.08, 0.8, 0.3, mode, 1, 2, 0.05, 1, 7, stream)
        assert rc == -4, (mode, rc)
        assert b"exp_avg_sq" in L.lv_last_error()
    rc = L.lv_step_f32(p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(), None, sc.data_ptr(), n, -1.0, 0.9, 0.999,
                       1e-8, 0.08, 0.8, 0.3, 2, 1, 2, 0.05, 1, 7, stream)
    assert rc == -4 and b"learning rate" in L.lv_last_error()
    torch.cuda.synchronize()
    assert torch.equal(p, p0) and int(torch.count_nonzero(m)) == 0


def test_standalone_engine_host_buffers(oracle_mod):
    """The reference's standalone C API (luminav_triton_standalone.h:37-111) on this library:
    engine_create on the current device, platform "rocm", arch the device's gfx name, and
    luminav_triton_step_f32 on HOST buffers (copied to the device, stepped, copied back) for both
    buffer modes, bitwise equal to the oracle over three steps; a NULL engine is -1."""
    _need_gpu()
    import ctypes

    import numpy as np

    from luminamoon_amd.optimizer import hip_backend

    O = oracle_mod
    L = hip_backend.load_library()
    eng = L.luminav_triton_engine_create()
    assert eng
    try:
        assert L.luminav_triton_get_platform(eng) == b"rocm"
        arch = L.luminav_triton_get_arch(eng)
        assert arch.startswith(b"gfx"), arch
        print(f"[case] standalone engine on {arch.decode()}", flush=True)
        P = lambda a: a.ctypes.data_as(ctypes.c_void_p) if a is not None else None  # noqa: E731
        for buffer in (1, 2):
            n = 50_003
            rng = np.random.default_rng(buffer)
            p = (rng.standard_normal(n) * 0.02).astype(np.float32)
            m = np.zeros(n, np.float32)
            v = np.zeros(n, np.float32) if buffer == 2 else None
            sc = np.array([0, 0, 0, 1, 1, 0], np.float32)
            hp, hm, hv, hs = (torch.from_numpy(x.copy()) if x is not None else None for x in (p, m, v, sc))
            cfg = O.make_config(lr=1e-3, buffer=buffer, cautious=True, bound_type=2, seed=5, stochastic_rounding=False)
            for t in range(1, 4):
                g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
                rc = L.luminav_triton_step_f32(eng, P(p), P(g), P(m), P(v), None, P(sc), n, 1e-3, 0.9, 0.999, 1e-8,
                                               0.08, 0.8, 0.3, buffer, 1, 2, 0.05, t, 5)
                assert rc == 0, L.lv_last_error()
                O.step(cfg, [hp], [torch.from_numpy(g)], [hm], [hv], [None], [hs], [t], [0])
                assert_bitwise(hp, torch.from_numpy(p), f"buffer {buffer} step {t} p")
                assert_bitwise(hm, torch.from_numpy(m), f"buffer {buffer} step {t} m")
                if v is not None:
                    assert_bitwise(hv, torch.from_numpy(v), f"buffer {buffer} step {t} v")
                assert_bitwise(hs, torch.from_numpy(sc), f"buffer {buffer} step {t} scratch")
        assert L.luminav_triton_step_f32(None, P(p), P(g), P(m), None, None, P(sc), n, 1e-3, 0.9, 0.999, 1e-8, 0.08,
                                         0.8, 0.3, 1, 1, 2, 0.05, 1, 5) == -1
    finally:
        L.luminav_triton_engine_destroy(eng)


if __name__ == "__main__":
    sys.exit(pytest.main([__file__, "-v"]))
