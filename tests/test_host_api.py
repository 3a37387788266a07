"""Host-side behaviour of the drop-in LuminaV class (no GPU needed).

Mirrors the reference's constructor/error tests (optimizer/tests/test_end_to_end_training.py:82-154,
:290-330), its typo-suggestion known answers (luminav-core/tests/core_tests.rs:113-158), bucket
fusion layout (luminav.py:763-952) and state_dict format (luminav.py:1030-1115).
"""
from __future__ import annotations

import warnings

import pytest
import torch
import torch.nn as nn

from luminamoon_amd import LuminaV
from luminamoon_amd.optimizer.constants import TEMP_STATE_DICT_KEYS
from luminamoon_amd.optimizer.validation import levenshtein, suggest_closest


def P(*shape, dtype=torch.float32):
    return nn.Parameter(torch.randn(*shape, dtype=dtype))


def err(fn):
    with pytest.raises(ValueError) as e:
        fn()
    return str(e.value)


def test_reference_error_strings():
    p = [P(8, 8)]
    assert err(lambda: LuminaV(p, buffer=3)) == (
        "Invalid buffer count: 3. LuminaV only supports buffer=1 (Single-Buffer TD-CLM) or buffer=2 (Dual-Buffer CLM).")
    assert err(lambda: LuminaV(p, bound_type="radal")) == (
        "Invalid bound_type: 'radal'. Expected 'coordinate' or 'radial'. Did you mean 'radial'?")
    assert err(lambda: LuminaV(p, execution="vulkn")) == (
        "Invalid execution mode: 'vulkn'. Expected 'auto', 'vulkan', 'simd', or 'scalar'. Did you mean 'vulkan'?")
    assert "Expected False, 'none', 'semi', or 'full'" in err(lambda: LuminaV(p, master_weights="invalid_mw"))
    assert err(lambda: LuminaV(p, master_weights="sem")) == (
        "Invalid master_weights: 'sem'. Expected False, 'none', 'semi', or 'full'. Did you mean 'semi'?")
    assert err(lambda: LuminaV(p, buffer="duel")) == (
        "Invalid buffer count: 'duel'. LuminaV only supports buffer=1 (Single-Buffer TD-CLM) or buffer=2 (Dual-Buffer CLM). Did you mean 'dual'?")
    e = err(lambda: LuminaV(p, lr=-0.01))
    assert "-0.01" in e and "[0.0, inf)" in e
    e = err(lambda: LuminaV(p, betas=(1.2, 0.999)))
    assert "1.2" in e and "[0.0, 1.0)" in e
    e = err(lambda: LuminaV(p, eps=0.0))
    assert "0.0" in e and "(0.0, inf)" in e
    assert "cautious_clamp_min" in err(lambda: LuminaV(p, cautious_clamp_min=0.0))
    assert "bound_ratio" in err(lambda: LuminaV(p, bound_ratio=-1))
    assert "seed" in err(lambda: LuminaV(p, seed=-1))
    assert "ema_decay" in err(lambda: LuminaV(p, ema_decay=1.0))
    assert "fuse_tensors" in err(lambda: LuminaV(p, fuse_tensors="invalid"))
    assert "prewarm_jit" in err(lambda: LuminaV(p, prewarm_jit="invalid"))
    assert "bucket_cap_mb" in err(lambda: LuminaV(p, bucket_cap_mb=0.0))
    assert "state_precision" in err(lambda: LuminaV(p, state_precision="fp8"))
    with pytest.raises(ValueError):
        LuminaV([], lr=1e-3)


def test_buffer_aliases_and_defaults():
    p = [P(4)]
    for alias, want in (("single", 1), ("TD-CLM", 1), ("clm", 2), ("dual", 2), (" t1 ", "T1"), ("triangle2", "T2"),
                        ("T2", "T2"), (1, 1), (2, 2)):
        assert LuminaV(p, buffer=alias).param_groups[0]["buffer"] == want
    g = LuminaV(p).param_groups[0]
    assert g["lr"] == 3e-4 and g["betas"] == (0.9, 0.999) and g["eps"] == 1e-8 and g["weight_decay"] == 0.08
    assert g["tau"] == 0.8 and g["lam"] == 0.3 and g["cautious"] is True and g["cautious_clamp_min"] == 0.5
    assert g["bound_type"] == 2 and g["bound_ratio"] == 0.05 and g["master_weights"] == 0 and g["seed"] == 1337
    assert g["ema_decay"] == 0.80 and LuminaV(p, buffer="T1").param_groups[0]["ema_decay"] == 0.95
    assert LuminaV(p, master_weights=True).param_groups[0]["master_weights"] == 2
    assert LuminaV(p, master_weights="hybrid").param_groups[0]["master_weights"] == 1
    assert LuminaV(p, bound=False, bound_type="none").param_groups[0]["bound_type"] == 0
    assert LuminaV(p, execution="simd").param_groups[0]["execution"] == 4
    opt = LuminaV(p)
    assert opt.fuse_tensors is False and opt.bucket_cap_mb == 500.0 and opt.prewarm_jit is True


def test_version_gates():
    p = [P(8)]
    assert LuminaV.ALGORITHM_SPEC == "1.6.0"
    assert LuminaV(p, version="1.5.5").version == "1.5.5"
    assert LuminaV(p, version="latest").version == "1.6.0"
    assert "Triangle Family" in err(lambda: LuminaV(p, version="1.5.5", buffer="T2"))
    assert "bucket fusion" in err(lambda: LuminaV(p, version="1.5.4", fuse_tensors=True))
    assert "Invalid LuminaV version format" in err(lambda: LuminaV(p, version="one.two"))
    assert LuminaV.list_versions() == ["1.6.0", "1.5.5", "1.5.4", "1.5.3"]
    assert LuminaV(p).get_capabilities()["supports_triangle_family"] is True
    assert LuminaV.get_capabilities("1.5.3")["allowed_buffers"] == (1, 2)


def test_levenshtein_and_suggestions():
    assert levenshtein("kitten", "sitting") == 3
    assert levenshtein("", "abc") == 3
    assert suggest_closest("radal", ("coordinate", "radial"), 3) == "radial"
    assert suggest_closest("zzzzzzzz", ("coordinate", "radial"), 3) is None
    assert suggest_closest("   ", ("a",), 3) is None


def test_step_on_cpu_tensors_fails_loudly_and_validates_first():
    p = P(8, 8)
    p.grad = torch.randn(8, 8)
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        LuminaV([p]).step()
    nc = nn.Parameter(torch.randn(8, 8).t())
    nc.grad = torch.randn(8, 8)
    assert ".contiguous()" in err(lambda: LuminaV([nc]).step())
    f64 = nn.Parameter(torch.zeros(8, 8, dtype=torch.float64), requires_grad=False)
    f64.grad = torch.zeros(8, 8, dtype=torch.float64)
    e = err(lambda: LuminaV([f64]).step())
    assert "torch.float32" in e and "torch.bfloat16" in e and "torch.float16" in e
    sp = P(4, 4)
    sp.grad = torch.zeros(4, 4).to_sparse()
    with pytest.raises(RuntimeError, match="sparse"):
        LuminaV([sp]).step()
    q = P(3)
    q.grad = None
    LuminaV([q]).step()  # nothing to do: no error, no state
    with pytest.raises(TypeError):
        LuminaV([[1.0, 2.0]])


def test_fsdp_sync_without_distributed_is_disabled():
    opt = LuminaV([P(4)], fsdp_sync=True)
    assert opt.param_groups[0]["fsdp_sync"] is False


def test_bucket_cap_warning():
    p = [P(32)]
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        LuminaV(p, bucket_cap_mb=250.0, fuse_tensors=False)
    assert any("Bounded bucket chunking only applies when" in str(x.message) for x in w)
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        LuminaV(p, fuse_tensors=False)
    assert not any("Bounded bucket chunking only applies when" in str(x.message) for x in w)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("buffer", [1, 2, "T1", "T2"])
def test_bucket_layout_zero_copy(dt, buffer):
    """Views into one flat allocation per (device, dtype) chunk; state dtypes follow the policy."""
    shapes = [(16, 8), (16,), (32, 16), (32,), (8, 32)]
    ps = [P(*s, dtype=dt) for s in shapes]
    before = [p.detach().clone() for p in ps]
    opt = LuminaV(ps, buffer=buffer, fuse_tensors=True)
    assert len(opt._fused_buckets) == 1
    b = opt._fused_buckets[0]
    assert b["flat_p"].numel() == sum(p.numel() for p in ps)
    assert b["state_dtype"] == torch.float32
    assert (b["flat_v"] is not None) == (buffer in (2, "T2"))
    base = b["flat_p"].data_ptr()
    off = 0
    for p, ref in zip(ps, before):
        assert p.data_ptr() == base + off * p.element_size()
        assert torch.equal(p.detach(), ref)
        assert p.grad is not None and p.grad.data_ptr() == b["flat_g"].data_ptr() + off * p.element_size()
        st = opt.state[p]
        assert st["exp_avg"].data_ptr() == b["flat_m"].data_ptr() + off * 4
        assert st["scratch"] is b["scratch"]
        off += p.numel()
    opt.zero_grad(set_to_none=True)
    for p, _, g_slice, _, g_ptr, _, _ in b["slices"]:
        assert p.grad is g_slice and p.grad.data_ptr() == g_ptr
    ref_opt = LuminaV([P(4, dtype=dt)], buffer=buffer, fuse_tensors=True, state_precision="param")
    want = torch.float32 if dt == torch.float32 else dt
    assert ref_opt._fused_buckets[0]["state_dtype"] == want


def test_bucket_cap_partitions_and_tied_weights():
    ps = [P(*s) for s in [(32, 16), (16,), (64, 32), (32,), (128, 64)]]
    opt = LuminaV(ps, buffer=1, fuse_tensors=True, bucket_cap_mb=0.004)
    assert len(opt._fused_buckets) >= 2
    shared, frozen, active = P(16), P(16), P(16)
    opt = LuminaV([shared, shared, frozen, active], lr=1e-2, weight_decay=0.1, buffer=2, fuse_tensors=True)
    assert len(opt._fused_buckets[0]["slices"]) == 3
    chunks = LuminaV._partition_into_bounded_chunks([(i, P(10)) for i in range(5)], 80)
    assert [len(c) for c in chunks] == [2, 2, 1]


def test_state_dict_cleanliness_and_round_trip():
    ps = [P(6, 4), P(4, dtype=torch.bfloat16)]
    opt = LuminaV(ps, master_weights="full")
    # populate state without stepping on a device: same initialiser the step uses
    for p in ps:
        st = opt._init_or_refresh_state(p, opt.param_groups[0])
        st["step"] = 3
        st["scratch"][0] = 5.0
        st["_plan"] = object()
    sd = opt.state_dict()
    for entry in sd["state"].values():
        assert not (set(entry) & TEMP_STATE_DICT_KEYS)
        assert float(entry["scratch"][0]) == 0.0 and float(entry["scratch"][3]) == 1.0
    assert "_validated_sig" not in sd["param_groups"][0]
    assert "master_param" not in sd["state"][0] and "master_param" in sd["state"][1]
    opt2 = LuminaV([nn.Parameter(p.detach().clone()) for p in ps], master_weights="full")
    opt2.load_state_dict(sd)
    for p in opt2.param_groups[0]["params"]:
        st = opt2.state[p]
        assert st["step"] == 3 and st["exp_avg"].dtype == torch.float32 and st["scratch"].numel() == 6
    # fp16 state containers are tagged as bf16 bits, and round-trip into fp32 state exactly
    h = P(8, dtype=torch.float16)
    opt3 = LuminaV([h], state_precision="param")
    st = opt3._init_or_refresh_state(h, opt3.param_groups[0])
    st["exp_avg"].view(torch.bfloat16).copy_(torch.tensor([1.5, -2.25, 3e-30, 0.0, 1e30, -7.0, 0.125, 2.0]).to(torch.bfloat16))
    sd3 = opt3.state_dict()
    assert sd3["state"][0]["_fp16_state_format"] == "bf16_bits"
    opt4 = LuminaV([nn.Parameter(h.detach().clone())], master_weights="full")
    sd3["param_groups"][0]["master_weights"] = "full"  # as test_end_to_end_training.py:262-265
    opt4.load_state_dict(sd3)
    m = opt4.state[opt4.param_groups[0]["params"][0]]["exp_avg"]
    assert m.dtype == torch.float32
    assert torch.equal(m, torch.tensor([1.5, -2.25, 3e-30, 0.0, 1e30, -7.0, 0.125, 2.0]).to(torch.bfloat16).float())


def test_detect_hardware_shape():
    hw = LuminaV.detect_hardware()
    assert hw["backend"] == "hip" and "gpu_dispatch_threshold" in hw and "hip_backend_built" in hw


def test_fsdp_sync_across_ranks_is_refused(monkeypatch):
    """fsdp_sync all-reduces the mask counts across ranks in the reference (fsdp_sync.py:20-38);
    this one-GPU build has no such collective, so it refuses a multi-rank fsdp_sync run instead
    of silently stepping with rank-local scales. One rank, or no process group, is fine."""
    import pytest
    import torch

    from luminamoon_amd import LuminaV

    p = torch.nn.Parameter(torch.zeros(4))
    monkeypatch.setattr(torch.distributed, "is_available", lambda: True)
    monkeypatch.setattr(torch.distributed, "is_initialized", lambda: True)
    monkeypatch.setattr(torch.distributed, "get_world_size", lambda *a, **k: 2)
    with pytest.raises(NotImplementedError, match="fsdp_sync"):
        LuminaV([p], fsdp_sync=True)
    monkeypatch.setattr(torch.distributed, "get_world_size", lambda *a, **k: 1)
    LuminaV([p], fsdp_sync=True)
    monkeypatch.setattr(torch.distributed, "is_initialized", lambda: False)
    LuminaV([p], fsdp_sync=True)


def test_capturable_option_validation_and_guards(monkeypatch):
    """capturable=True: a bool, not with fused buckets; a group holding state steps every
    parameter together (a parameter with state and no grad raises); capturing a group before its
    eager set-up step raises before anything is launched."""
    p = nn.Parameter(torch.zeros(4))
    assert LuminaV([p], capturable=True).param_groups[0]["capturable"] is True
    assert LuminaV([p]).param_groups[0]["capturable"] is False
    with pytest.raises(ValueError, match="capturable"):
        LuminaV([p], capturable="yes")
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        with pytest.raises(ValueError, match="fuse_tensors=False"):
            LuminaV([p], capturable=True, fuse_tensors=True)
    q = nn.Parameter(torch.zeros(4))
    opt = LuminaV([p, q], capturable=True)
    opt.state[q]["step"] = 3
    p.grad = torch.zeros(4)
    with pytest.raises(ValueError, match="steps all of its parameters together"):
        opt.step()
    q.grad = torch.zeros(4)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    with pytest.raises(RuntimeError, match="eager step"):
        opt.step()
    assert opt.state[q]["step"] == 3 and len(opt.state[p]) == 0


def test_bucket_cut_rule():
    """Buckets take params in order while their bytes fit under the cap (a bucket may end exactly
    at the cap); a param that would take a non-empty bucket past it opens the next one, so a param
    larger than the cap sits alone (the reference's rule, luminav.py:763-786)."""
    cut = LuminaV._partition_into_bounded_chunks
    mk = lambda *ns: [(i, torch.empty(n, dtype=torch.float32)) for i, n in enumerate(ns)]  # noqa: E731
    sizes = lambda chunks: [[int(p.numel()) for _, p in c] for c in chunks]  # noqa: E731
    assert cut([], 100) == []
    assert sizes(cut(mk(10, 15), 100)) == [[10, 15]]          # 100 bytes: exactly at the cap
    assert sizes(cut(mk(10, 16), 100)) == [[10], [16]]        # 104 bytes: past it
    assert sizes(cut(mk(50, 3, 2), 100)) == [[50], [3, 2]]    # the first param alone exceeds the cap
    assert sizes(cut(mk(3, 50, 2), 100)) == [[3], [50], [2]]
    assert sizes(cut(mk(5, 5, 5, 5, 5, 5), 40)) == [[5, 5], [5, 5], [5, 5]]
    assert [i for c in cut(mk(7, 1, 30, 2, 2), 40) for i, _ in c] == [0, 1, 2, 3, 4]  # order kept


def test_reference_checkpoint_state_precision_is_inferred():
    """A checkpoint without this build's state_precision key (the reference's format) keeps the
    precision its 16-bit params' state was saved in: bf16 m/v stay bf16 (the reference's default
    for 16-bit params, luminav.py:1666-1672), fp32 m/v stay fp32, whatever the constructor said; a
    checkpoint that carries the key keeps its own value."""
    def make():
        return [P(64, dtype=torch.bfloat16), P(10, dtype=torch.bfloat16)]

    def ckpt(opt, dt, keep_key=False):
        groups = [{k: v for k, v in g.items() if keep_key or k != "state_precision"}
                  for g in opt.state_dict()["param_groups"]]
        state = {i: {"step": 3, "exp_avg": torch.randn(n).to(dt), "exp_avg_sq": torch.rand(n).to(dt),
                     "scratch": torch.tensor([0.0, 0.0, 0.0, 1.0, 1.0, 0.0]), "buf_count": 2}
                 for i, n in enumerate((64, 10))}
        return {"state": state, "param_groups": groups}

    ps = make()
    opt = LuminaV(ps, lr=1e-3)
    opt.load_state_dict(ckpt(opt, torch.bfloat16))
    assert opt.param_groups[0]["state_precision"] == "param"
    assert all(opt.state[p][k].dtype == torch.bfloat16 for p in ps for k in ("exp_avg", "exp_avg_sq"))
    ps = make()
    opt = LuminaV(ps, lr=1e-3, state_precision="param")
    opt.load_state_dict(ckpt(opt, torch.float32))
    assert opt.param_groups[0]["state_precision"] == "fp32"
    assert all(opt.state[p][k].dtype == torch.float32 for p in ps for k in ("exp_avg", "exp_avg_sq"))
    ps = make()
    opt = LuminaV(ps, lr=1e-3, state_precision="fp32")
    opt.load_state_dict(ckpt(opt, torch.bfloat16, keep_key=True))  # this build's own checkpoint
    assert opt.param_groups[0]["state_precision"] == "fp32"
    assert all(opt.state[p][k].dtype == torch.float32 for p in ps for k in ("exp_avg", "exp_avg_sq"))


def test_plan_record_check_and_counter_advance():
    """_lv_host.grad_record gives None whenever the params are not the recorded objects at their
    recorded data pointers, a state tensor's data moved, a grad is missing or does not fit its
    descriptor (CPU tensors never do: the accepting case runs in the GPU plan tests), and rejects
    malformed arguments; advance returns the counters plus one and stores each in its state dict,
    bypassing a dict subclass's __setitem__ as the Python path does."""
    import luminamoon_amd.optimizer.luminav as L
    from luminamoon_amd.optimizer import hip_backend

    host = hip_backend.load_host_ext()
    if host is None or not hasattr(host, "grad_record"):
        pytest.skip("_lv_host.so is not built")
    params = [torch.nn.Parameter(torch.zeros(3)), torch.nn.Parameter(torch.zeros(4, dtype=torch.bfloat16))]
    for p in params:
        p.grad = torch.ones_like(p)
    states = [torch.zeros(3)]
    dts, ns = [torch.float32, torch.bfloat16], [3, 4]
    pid, pp, sp = L._pack_ptrs(list(map(id, params))), L._ptr_record(params), L._ptr_record(states)
    assert host.grad_record(params, pid, pp, states, sp, dts, ns, 0) is None  # CPU grads do not fit
    assert host.grad_record(params[::-1], pid, pp, states, sp, dts, ns, 0) is None
    assert host.grad_record(params, pid, pp, states, L._ptr_record([torch.zeros(3)]), dts, ns, 0) is None
    assert host.grad_record(params, pid[:8], pp, states, sp, dts, ns, 0) is None
    params[1].grad = None
    assert host.grad_record(params, pid, pp, states, sp, dts, ns, 0) is None
    assert host.grad_record([], b"", b"", [], b"", [], [], 0) == b""
    with pytest.raises(ValueError):
        host.grad_record(params, pid, pp, states, sp, dts[:1], ns, 0)
    with pytest.raises(TypeError):
        host.grad_record(params, pid, pp, states, sp, [1, 2], ns, 0)
    with pytest.raises(TypeError):
        host.grad_record(tuple(params), pid, pp, states, sp, dts, ns, 0)

    class Guarded(dict):
        def __setitem__(self, k, v):
            raise AssertionError("the counters bypass __setitem__, as dict.__setitem__ does")

    ds = [{"step": 7}, Guarded(step=2**40), {}]
    out = host.advance(ds, [7, 2**40, 0], "step")
    assert out == [8, 2**40 + 1, 1] and [d["step"] for d in ds] == out
    assert all(a is d["step"] for a, d in zip(out, ds))
    with pytest.raises(ValueError):
        host.advance(ds, [1, 2], "step")
    with pytest.raises(TypeError):
        host.advance([{}, 3], [1, 2], "step")
    with pytest.raises(TypeError):
        host.advance([{}], ["x"], "step")


def test_plan_pointer_helpers_agree_with_python():
    """The step plans' data-pointer checks (the C module _lv_host when built, else Python maps)
    record where each tensor's data is and notice any move; an entry that is not a tensor (a grad
    of None) never matches, and a tensor without storage raises as Tensor.data_ptr does."""
    import luminamoon_amd.optimizer.luminav as L
    from luminamoon_amd.optimizer import hip_backend

    ts = [torch.zeros(3), torch.zeros(5, dtype=torch.bfloat16), torch.zeros(2, 2)[1]]
    rec = L._ptr_record(ts)
    assert L._same_ptrs(ts, rec)
    assert L._same_ptrs(list(ts), L._pack_ptrs([t.data_ptr() for t in ts]))
    moved = [ts[0], ts[1].clone(), ts[2]]
    assert not L._same_ptrs(moved, rec)
    assert not L._same_ptrs(ts[:2], rec)  # a different count
    assert not L._same_ptrs([ts[0], None, ts[2]], rec)
    ts[0].data = ts[0].data.clone()  # storage moved in place, same tensor object
    assert not L._same_ptrs(ts, rec)
    host = hip_backend.load_host_ext()
    if host is not None:
        with pytest.raises(RuntimeError):
            host.ptrs([torch.zeros(4).to_sparse()])
        with pytest.raises(TypeError):
            host.ptrs([torch.zeros(1), 3])
