"""The drop-in optimizer in training loops on the GPU: the reference's own behavioural tests,
restated for ROCm tensors.

* bit-exact resume after state_dict / torch.save / load_state_dict for fp32 and bf16 models, all
  four buffer modes and master weights off / semi / full (eval/modules/checkpoint_test.py:12-88),
  unfused and with fused buckets;
* fused buckets equal unfused tensors with cautious and stochastic rounding off (the reference
  asserts allclose, test_end_to_end_training.py:339-395; here the bits are equal), and zero_grad
  keeps the grad views into the bucket;
* small bucket caps split into several buckets and still track the unfused run
  (test_end_to_end_training.py:437-462);
* tied weights are stepped once and a grad=None parameter inside a bucket is left untouched
  (test_end_to_end_training.py:464-482).
"""
from __future__ import annotations

import copy
import io

import pytest
import torch
import torch.nn as nn

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


def _model(dtype):
    return nn.Sequential(nn.Linear(10, 20), nn.ReLU(), nn.Linear(20, 2)).to(dtype=dtype, device="cuda")


@pytest.mark.parametrize("fuse", [False, True], ids=["unfused", "fused"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_checkpoint_bit_exact_resume(dtype, fuse):
    _need_gpu()
    from luminamoon_amd import LuminaV
    from luminamoon_amd.optimizer.constants import TEMP_STATE_DICT_KEYS

    torch.manual_seed(42)
    for buf in (1, 2, "T1", "T2"):
        for mw in (False, "semi", "full"):
            print(f"[case] resume dtype={dtype} buffer={buf} master={mw} fuse={fuse}", flush=True)
            model_cont = _model(dtype)
            model_res = copy.deepcopy(model_cont)
            kw = dict(lr=1e-3, buffer=buf, bound=True, master_weights=mw, fuse_tensors=fuse)
            opt_cont = LuminaV(model_cont.parameters(), **kw)
            opt_res = LuminaV(model_res.parameters(), **kw)
            batches = [(torch.randn(4, 10, dtype=dtype, device="cuda"), torch.tensor([0, 1, 0, 1], device="cuda"))
                       for _ in range(6)]
            for i in range(5):
                x, y = batches[i]
                for m, opt in ((model_cont, opt_cont), (model_res, opt_res)):
                    loss = nn.CrossEntropyLoss()(m(x).float(), y)
                    opt.zero_grad()
                    loss.backward()
                    opt.step()
            buf_io = io.BytesIO()
            torch.save(opt_res.state_dict(), buf_io)
            buf_io.seek(0)
            opt_loaded = LuminaV(model_res.parameters(), **kw)
            loaded = torch.load(buf_io, weights_only=True)
            opt_loaded.load_state_dict(loaded)
            for st in loaded["state"].values():
                assert not (set(st) & set(TEMP_STATE_DICT_KEYS))
                sc = st["scratch"]
                assert float(sc[0]) == float(sc[1]) == float(sc[2]) == float(sc[5]) == 0.0
            for p in model_res.parameters():
                st = opt_loaded.state[p]
                assert st["scratch"].dtype == torch.float32
                if "master_param" in st:
                    assert st["master_param"].dtype == torch.float32
            x, y = batches[5]
            for m, opt in ((model_cont, opt_cont), (model_res, opt_loaded)):
                loss = nn.CrossEntropyLoss()(m(x).float(), y)
                opt.zero_grad()
                loss.backward()
                opt.step()
            torch.cuda.synchronize()
            for p_c, p_r in zip(model_cont.parameters(), model_res.parameters()):
                assert torch.equal(p_c.view(torch.int16 if dtype == torch.bfloat16 else torch.int32),
                                   p_r.view(torch.int16 if dtype == torch.bfloat16 else torch.int32)), (buf, mw)
            for p_c, p_r in zip(model_cont.parameters(), model_res.parameters()):
                assert torch.equal(opt_cont.state[p_c]["exp_avg"], opt_loaded.state[p_r]["exp_avg"]), (buf, mw)


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("buf", [1, 2, "T1", "T2"])
def test_fused_bucket_equals_unfused_without_cautious_and_sr(buf, dt):
    _need_gpu()
    from luminamoon_amd import LuminaV

    torch.manual_seed(100)
    shapes = [(16, 8), (16,), (32, 16), (32,), (8, 32)]
    pu_list = [nn.Parameter(torch.randn(s, dtype=dt, device="cuda")) for s in shapes]
    pf_list = [nn.Parameter(p.detach().clone()) for p in pu_list]
    kw = dict(lr=2e-3, buffer=buf, cautious=False, bound=True, bound_type="coordinate", stochastic_rounding=False)
    opt_u = LuminaV(pu_list, fuse_tensors=False, **kw)
    opt_f = LuminaV(pf_list, fuse_tensors=True, **kw)
    assert len(opt_f._fused_buckets) == 1
    bucket = opt_f._fused_buckets[0]
    assert bucket["flat_p"].numel() == sum(p.numel() for p in pf_list)
    opt_f.zero_grad(set_to_none=True)
    for p, _, g_slice, _, g_ptr, _, _ in bucket["slices"]:
        assert p.grad is g_slice and p.grad.data_ptr() == g_ptr
    for _ in range(4):
        opt_u.zero_grad(set_to_none=True)
        opt_f.zero_grad(set_to_none=True)
        for pu, pf in zip(pu_list, pf_list):
            g = torch.randn_like(pu) * 0.05
            pu.grad = g.clone()
            pf.grad.copy_(g)
        opt_u.step()
        opt_f.step()
    torch.cuda.synchronize()
    iv = torch.int32 if dt == torch.float32 else torch.int16
    for pu, pf in zip(pu_list, pf_list):
        assert torch.equal(pu.detach().view(iv), pf.detach().view(iv)), f"buffer={buf} dtype={dt}"


def test_small_bucket_cap_splits_and_tracks_unfused():
    _need_gpu()
    from luminamoon_amd import LuminaV

    torch.manual_seed(7)
    shapes = [(32, 16), (16,), (64, 32), (32,), (128, 64)]
    pu_list = [nn.Parameter(torch.randn(s, device="cuda")) for s in shapes]
    pc_list = [nn.Parameter(p.detach().clone()) for p in pu_list]
    opt_u = LuminaV(pu_list, lr=1e-3, buffer=1, fuse_tensors=False)
    opt_c = LuminaV(pc_list, lr=1e-3, buffer=1, fuse_tensors=True, bucket_cap_mb=0.004)
    assert len(opt_c._fused_buckets) >= 2
    for _ in range(5):
        opt_u.zero_grad(set_to_none=True)
        opt_c.zero_grad(set_to_none=True)
        for pu, pc in zip(pu_list, pc_list):
            g = torch.randn_like(pu) * 0.01
            pu.grad = g.clone()
            pc.grad.copy_(g)
        opt_u.step()
        opt_c.step()
    torch.cuda.synchronize()
    for pu, pc in zip(pu_list, pc_list):
        # per-bucket vs per-tensor cautious scale: close, not equal (the reference's own tolerance)
        assert torch.allclose(pu, pc, atol=1e-5, rtol=1e-4)
    sd = opt_c.state_dict()
    reload = [nn.Parameter(p.detach().clone()) for p in pc_list]
    opt_r = LuminaV(reload, lr=1e-3, buffer=1, fuse_tensors=True, bucket_cap_mb=0.004)
    opt_r.load_state_dict(sd)
    assert len(opt_r._fused_buckets) == len(opt_c._fused_buckets)


def test_tied_weights_and_grad_none_isolation_in_bucket():
    _need_gpu()
    from luminamoon_amd import LuminaV

    p_shared = nn.Parameter(torch.ones(16, device="cuda"))
    p_frozen = nn.Parameter(torch.full((16,), 2.0, device="cuda"))
    p_active = nn.Parameter(torch.full((16,), 3.0, device="cuda"))
    opt = LuminaV([p_shared, p_shared, p_frozen, p_active], lr=1e-2, weight_decay=0.1, buffer=2, fuse_tensors=True)
    assert len(opt._fused_buckets[0]["slices"]) == 3
    p_shared.grad = torch.ones_like(p_shared) * 0.5
    p_frozen.grad = None
    p_active.grad = torch.ones_like(p_active) * 0.5
    for _ in range(3):
        opt.step()
    torch.cuda.synchronize()
    assert torch.equal(p_frozen, torch.full((16,), 2.0, device="cuda")), "grad=None param was mutated"
    assert opt.state[p_frozen]["step"] == 0
    assert opt.state[p_active]["step"] == 3
    assert not torch.equal(p_active, torch.full((16,), 3.0, device="cuda"))
    m_frozen = opt.state[p_frozen]["exp_avg"]
    assert torch.count_nonzero(m_frozen) == 0


def test_unfused_descriptor_plan_reuse_and_invalidation(oracle_mod, monkeypatch):
    """Unfused groups reuse their packed descriptors while only grads and step counters change.
    Every way the plan can go stale is driven here -- grads updated in place, new grad tensors,
    a param losing and regaining its grad, param storage replaced, load_state_dict, a changed
    hyper-parameter, new grads while the old ones live on, one grad replaced, a state tensor's
    storage moved in place -- and each step is compared bit for bit with the oracle."""
    _need_gpu()
    from luminamoon_amd import LuminaV
    from tests.parity_util import TensorSet, assert_bitwise, oracle_config, seeded_tensor

    O = oracle_mod
    sizes = [4099, 1, 2048, 70_001]
    host = TensorSet(sizes, "bf16", "bf16", "f32", True, False, seed=11)
    params = [torch.nn.Parameter(t.clone().cuda()) for t in host.p]
    opt = LuminaV(params, lr=3e-3, buffer="T2")
    used = {"fast": 0}
    real = opt._run_unfused_plan

    def spy(group):
        ok = real(group)
        used["fast"] += int(ok)
        return ok

    opt._run_unfused_plan = spy
    # the one-call check of a step (_lv_host.grad_record), when built: count the steps it took
    import luminamoon_amd.optimizer.luminav as L

    record_real = L._grad_record
    taken = {"n": 0}

    def record_spy(*a):
        rec = record_real(*a)
        taken["n"] += rec is not None
        return rec

    if record_real is not None:
        monkeypatch.setattr(L, "_grad_record", record_spy)
    host_steps = [0] * len(sizes)
    kept = []

    def run(s, mode, expect_fast):
        grads = [seeded_tensor(n, 900 + 10 * s + i, 1e-3, torch.bfloat16) for i, n in enumerate(sizes)]
        active = [True] * len(sizes)
        if mode == "drop1":
            active[1] = False
        for i, p in enumerate(params):
            if not active[i]:
                p.grad = None
            elif (mode == "inplace" or (mode == "one" and i > 0)) and p.grad is not None:
                p.grad.copy_(grads[i].cuda())
            else:
                p.grad = grads[i].cuda()
                if mode == "keep":  # the previous grads stay alive: new ids, no weakref death
                    kept.append(p.grad)
        before = used["fast"]
        opt.step()
        torch.cuda.synchronize()
        assert used["fast"] - before == int(expect_fast), f"step {s} ({mode}): plan used {used['fast'] - before}"
        group = opt.param_groups[0]
        cfg = oracle_config(O, group)
        for i in range(len(sizes)):
            if not active[i]:
                continue
            host_steps[i] += 1
            if group["master_weights"] and host.mp[i] is None:  # master weights switched on
                host.mp[i] = host.p[i].float().clone()
            if not group["cautious"]:  # the host layer's scratch forcing (reference luminav.py:1748-1749)
                host.sc[i][3] = 1.0
            O.step(cfg, [host.p[i]], [grads[i]], [host.m[i]], [host.v[i]], [host.mp[i]], [host.sc[i]],
                   [host_steps[i]], [i])
        for i, p in enumerate(params):
            st = opt.state[p]
            if host.mp[i] is not None:
                assert_bitwise(st["master_param"], host.mp[i], f"step {s} ({mode}) mp[{i}]")
            assert_bitwise(p.detach(), host.p[i], f"step {s} ({mode}) p[{i}]")
            assert_bitwise(st["exp_avg"], host.m[i], f"step {s} ({mode}) m[{i}]")
            assert_bitwise(st["exp_avg_sq"], host.v[i], f"step {s} ({mode}) v[{i}]")
            assert_bitwise(st["scratch"], host.sc[i], f"step {s} ({mode}) scratch[{i}]")
            assert int(st["step"]) == host_steps[i]

    run(1, "new", False)      # builds the plan
    run(2, "new", True)       # new grad tensors: pointers refreshed
    run(3, "inplace", True)   # same grad tensors updated in place
    run(4, "drop1", False)    # a param without a grad: slow path, new plan
    run(5, "drop1", True)
    run(6, "new", False)      # it has a grad again
    run(7, "new", True)
    params[2].data = params[2].data.clone()  # param storage moved
    run(8, "new", False)
    run(9, "new", True)
    opt.load_state_dict(opt.state_dict())    # state tensors replaced
    run(10, "new", False)
    run(11, "new", True)
    opt.param_groups[0]["lr"] = 1e-3         # options are read into every launch: the plan stays
    opt.param_groups[0]["cautious"] = False
    run(12, "new", True)
    opt.param_groups[0]["master_weights"] = "full"  # the state layout changes: slow path, new plan
    run(13, "new", False)
    run(14, "new", True)
    # a state entry replaced by a new tensor of the same values (what device-moving helpers do,
    # state[k] = v.to(device)): the plan is dropped, and the new tensor is the one stepped
    st0 = opt.state[params[0]]
    st0["exp_avg"] = st0["exp_avg"].clone()
    run(15, "new", False)
    run(16, "new", True)
    # a parameter's whole state dict replaced (opt.state[p] = {...})
    opt.state[params[1]] = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in opt.state[params[1]].items()}
    run(17, "new", False)
    run(18, "new", True)
    # the optimizer's state map replaced wholesale
    from collections import defaultdict

    opt.state = defaultdict(dict, {k: dict(v) for k, v in opt.state.items()})
    run(19, "new", False)
    run(20, "new", True)
    # every grad a new tensor while the old ones stay alive (all re-pointed at once), then one
    # grad replaced and the rest updated in place (re-pointed one by one)
    run(21, "keep", True)
    run(22, "keep", True)
    run(23, "one", True)
    # a state tensor's storage moved in place (t.data = u, t.set_(u)): the state entry is the same
    # object, so only its data pointer shows it; the plan is dropped and the moved storage stepped
    m0 = opt.state[params[0]]["exp_avg"]
    m0.data = m0.data.clone()
    run(24, "new", False)
    run(25, "new", True)
    v3 = opt.state[params[3]]["exp_avg_sq"]
    v3.set_(v3.clone())
    run(26, "new", False)
    run(27, "new", True)
    sc2 = opt.state[params[2]]["scratch"]
    sc2.data = sc2.data.clone()
    run(28, "new", False)
    run(29, "new", True)
    # the same grad objects updated in place, then new grad objects every step
    # (zero_grad(set_to_none=True)): each step checked and its grads recorded in one C call
    n0 = taken["n"]
    for s, mode in ((30, "inplace"), (31, "inplace"), (32, "new"), (33, "new"), (34, "keep"), (35, "one")):
        run(s, mode, True)
    if record_real is not None:
        assert taken["n"] - n0 == 6, taken


def test_unfused_duplicate_param_raises_like_the_native_seam():
    """LuminaV([w, w]) unfused lists one tensor twice. The reference's native seam rejects it
    (step_pyo3: "Pointer aliasing detected", python_ffi/mod.rs:141-147); here the C ABI does the
    same before any launch, step() raises ValueError, and neither the parameter nor its step
    counter moves. (Fused buckets keep one slice per tied weight instead.)"""
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import warnings

    from luminamoon_amd import LuminaV

    w = torch.nn.Parameter(torch.randn(5000, device="cuda") * 0.02)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")  # torch warns about duplicate parameters in a group
        opt = LuminaV([w, w], lr=1e-3, buffer="T2")
    w.grad = torch.randn_like(w) * 1e-3
    before = w.detach().clone()
    print("[case] unfused duplicate parameter", flush=True)
    with pytest.raises(ValueError, match="Pointer aliasing detected"):
        opt.step()
    torch.cuda.synchronize()
    assert torch.equal(w.detach(), before)
    assert int(opt.state[w]["step"]) == 0


def test_reference_checkpoint_keeps_its_state_dtype(oracle_mod):
    """A checkpoint in the reference's own format -- no state_precision key, bf16 params with bf16
    exp_avg/exp_avg_sq as the reference allocates them (python/luminamoon/optimizer/luminav.py:
    1666-1672) -- resumes with bf16 state in a LuminaV built with the default fp32 state, and the
    next three steps equal the oracle continuing from the same state, bit for bit."""
    _need_gpu()
    from luminamoon_amd import LuminaV
    from tests.parity_util import TensorSet, assert_bitwise, oracle_config

    O = oracle_mod
    sizes = [4099, 70_001]
    host = TensorSet(sizes, "bf16", "bf16", "bf16", True, False, seed=21, m_scale=1e-3)
    params = [nn.Parameter(t.clone().cuda()) for t in host.p]
    opt = LuminaV(params, lr=1e-3, buffer="T2")
    groups = [{k: v for k, v in g.items() if k != "state_precision"} for g in opt.state_dict()["param_groups"]]
    scale = [1.25, 1.5]
    state = {i: {"step": 7, "exp_avg": host.m[i].clone(), "exp_avg_sq": host.v[i].clone(),
                 "scratch": torch.tensor([0.0, 0.0, 0.0, scale[i], 1.0, 0.0]), "buf_count": "T2"}
             for i in range(len(sizes))}
    opt.load_state_dict({"state": state, "param_groups": groups})
    assert opt.param_groups[0]["state_precision"] == "param"
    for p in params:
        assert opt.state[p]["exp_avg"].dtype == torch.bfloat16 and opt.state[p]["exp_avg_sq"].dtype == torch.bfloat16
    for i in range(len(sizes)):
        host.sc[i] = torch.tensor([0.0, 0.0, 0.0, scale[i], 1.0, 0.0])
    cfg = oracle_config(O, opt.param_groups[0])
    for s in (8, 9, 10):
        grads = host.grads(s, 21)
        for p, g in zip(params, grads):
            p.grad = g.cuda()
        opt.step()
        host.oracle_step(O, cfg, grads, s)
        torch.cuda.synchronize()
        for i, p in enumerate(params):
            st = opt.state[p]
            assert_bitwise(p.detach(), host.p[i], f"step {s} p[{i}]")
            assert_bitwise(st["exp_avg"], host.m[i], f"step {s} m[{i}]")
            assert_bitwise(st["exp_avg_sq"], host.v[i], f"step {s} v[{i}]")
            assert_bitwise(st["scratch"], host.sc[i], f"step {s} scratch[{i}]")


def test_bucket_buffers_are_parts_of_one_allocation():
    """A fused bucket's flat p, g, m, v (and master) are parts of ONE device allocation, each on a
    2 MiB boundary in the order p|g|m|v|master, and each is a tensor with a storage of exactly its
    own bytes: torch.save of the params writes the params only, and the allocation lives while
    any part does (the params after the optimizer is gone)."""
    _need_gpu()
    from luminamoon_amd import LuminaV

    sizes = (1000, 3000, 5, 70_001)
    params = [nn.Parameter(torch.randn(n, device="cuda", dtype=torch.bfloat16) * 0.02) for n in sizes]
    for p in params:
        p.grad = torch.randn_like(p) * 1e-3
    opt = LuminaV(params, lr=1e-3, buffer="T2", fuse_tensors=True, master_weights="full")
    opt.step()
    (b,) = opt._fused_buckets
    n = sum(sizes)
    flats = [b["flat_p"], b["flat_g"], b["flat_m"], b["flat_v"], b["flat_mp"]]
    ptrs = [f.data_ptr() for f in flats]
    align = 2 << 20
    assert all(q % align == 0 for q in ptrs)
    for f, q, q_next in zip(flats, ptrs, ptrs[1:]):
        assert q_next - q == -(-f.numel() * f.element_size() // align) * align
    for f in flats:
        assert f.numel() == n
        assert f.untyped_storage().nbytes() == n * f.element_size()
        assert f.untyped_storage().data_ptr() == f.data_ptr()
    buf = io.BytesIO()
    torch.save([p.detach() for p in params], buf)
    assert buf.tell() < n * 2 + 64 * 1024  # the bf16 params, not the whole allocation
    before = [p.detach().clone() for p in params]
    del opt, b, flats
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    junk = torch.full((1 << 22,), 7.0, device="cuda")  # reuse of freed memory would show here
    torch.cuda.synchronize()
    for p, q in zip(params, before):
        assert torch.equal(p.detach(), q)
    del junk
