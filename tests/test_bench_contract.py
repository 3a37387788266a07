"""bench.py's contract on the CPU: it refuses more than one GPU before touching a device, its
workloads have BASELINE.json's shapes and byte counts, and its CPU-baseline leg reports the
fields the bench line carries."""
from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_message():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], cwd=ROOT,
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 2
    line = json.loads(res.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def test_workload_shapes_match_the_configs():
    assert bench.N5 == 6_738_415_616  # Llama-7B shape, one bucket
    assert bench.N4 == 953_223_168    # Llama-1B shape
    assert bench.N3 == 123_570_432    # GPT-2 small
    sizes = bench.cfg2_sizes()
    assert len(sizes) == 64 and min(sizes) >= 1 and max(sizes) <= 2 ** 20 + 1
    assert sum(sizes) == 3_514_803


def test_bytes_per_param_follow_the_buffers():
    """Each buffer read once and written once: p (read + write), g (read), m and v (read + write)."""
    size = {"bf16": 2, "f32": 4}
    for wl in bench.WORKLOADS.values():
        ps = size[wl["pdt"]]
        dual = wl["buffer"] in (2, "T2")
        state = 4  # f32 m (and v)
        assert wl["bytes_per_param"] == 3 * ps + 2 * state * (2 if dual else 1), wl["name"]


def test_variant_workloads():
    """--state param keeps m/v in bf16 (2 + 2 bytes each), --bound radial moves the same bytes."""
    assert bench.workload(5)["bytes_per_param"] == 22
    assert bench.workload(5, state="param")["bytes_per_param"] == 14   # p 2+2, g 2, m 2+2, v 2+2
    assert bench.workload(4, state="param")["bytes_per_param"] == 10   # p 2+2, g 2, m 2+2
    assert bench.workload(3, state="param")["bytes_per_param"] == 28   # fp32 params: fp32 state
    assert bench.workload(5, bound="radial")["bytes_per_param"] == 22
    assert bench.workload(5, state="param")["sdt"] == "bf16"
    assert bench.pmc_traffic_bytes(5, bound="radial") is None
    # an fp32 master copy: p write-only (2), master read + write (8)
    assert bench.workload(5, master="full")["bytes_per_param"] == 28
    assert bench.workload(4, master="semi")["bytes_per_param"] == 20
    assert bench.workload(5, state="param", master="full")["sdt"] == "f32"  # full master keeps fp32 state
    assert bench.workload(5, state="param", master="semi")["bytes_per_param"] == 14 - 2 + 8
    assert bench.workload(5, pdt="f16")["pdt"] == "f16" and bench.workload(5, pdt="f16")["bytes_per_param"] == 22
    with pytest.raises(ValueError):
        bench.workload(3, pdt="f16")
    assert bench.pmc_traffic_bytes(5, master="full") is None


def test_cpu_baseline_with_master_and_fp16():
    wl = dict(bench.workload(5, master="full", pdt="f16"))
    wl["n"] = 1 << 21
    out = bench.cpu_baseline(wl, threads=2, target_s=0.3)
    assert out["value"] > 0 and out["cores"] == 2


def test_pmc_traffic_is_the_algorithmic_bytes_plus_the_count_atomics():
    algorithmic = bench.N5 * 22
    traffic = bench.pmc_traffic_bytes(5)
    blocks = bench.N5 // 256  # one-wave blocks of 256 elements
    # each count atomic writes 32 B (and its return reads a few more)
    assert abs(traffic - (algorithmic + 32 * blocks)) / algorithmic < 1.5e-3
    # the other measured variants: within 0.5% of the algorithmic bytes (+ 32 B per count atomic)
    for key, (bpp, unit) in {(3, "coordinate", "fp32", "none", ""): (28, 256),
                             (4, "coordinate", "fp32", "none", ""): (14, 1024),
                             (4, "coordinate", "param", "none", ""): (10, 2048),
                             (4, "coordinate", "param", "none", "f16"): (10, 2048),
                             (5, "coordinate", "param", "none", ""): (14, 2048)}.items():
        n = {3: bench.N3, 4: bench.N4, 5: bench.N5}[key[0]]
        got = bench.pmc_traffic_bytes(*key)
        want = n * bpp + 32 * (n // unit)
        assert abs(got - want) / want < 5e-3, (key, got, want)
    assert bench.pmc_traffic_bytes(5, state="param", master="full") is None


def test_cpu_baseline_reports_its_fields():
    wl = dict(bench.WORKLOADS[3])
    wl["n"] = 1 << 21
    out = bench.cpu_baseline(wl, threads=2, target_s=0.3)
    assert out["unit"] == "params/s" and out["cores"] == 2 and out["kind"] == "port"
    assert out["value"] > 0 and out["gb_per_s"] > 0
    assert "elements of the same workload" in out["sample"]
    assert "AVX-512" in out["sample"] or "scalar core" in out["sample"]


def test_cpu_threads_follow_the_host_limits(monkeypatch):
    """The CPU baseline uses os.cpu_count() threads unless this process may use fewer (affinity,
    cgroup quota, the box's OMP_NUM_THREADS share), and reports which limit decided, next to the
    host's logical CPUs and physical cores."""
    import os

    import bench

    monkeypatch.delenv("OMP_NUM_THREADS", raising=False)
    ct = bench.cpu_threads()
    assert ct["host_cpus"] == os.cpu_count()
    assert 1 <= ct["threads"] <= os.cpu_count()
    assert ct["threads"] == min(ct["limits"].values()) and ct["limits"]["os.cpu_count"] == os.cpu_count()
    monkeypatch.setenv("OMP_NUM_THREADS", "3")
    ct = bench.cpu_threads()
    assert ct["threads"] == min(3, os.cpu_count()) and ct["limits"]["OMP_NUM_THREADS"] == 3
    if os.cpu_count() > 3:
        assert ct["limited_by"] == "OMP_NUM_THREADS"


def test_cpu_baseline_draws_student_t_grads_for_cfg5():
    """cfg5's sample grads are 1e-3 * t(df=3), like the GPU workload's."""
    import bench

    wl = bench.workload(5)
    assert wl["grad"] == "student_t3"
    out = bench.cpu_baseline(wl, threads=2, target_s=0.3)
    assert out["grads"] == "student_t3" and out["value"] > 0


def _probe_lib():
    import shutil

    if not (os.path.exists(bench.PROBE_LIB) or shutil.which("hipcc") or os.path.exists("/opt/rocm/bin/hipcc")):
        pytest.skip("hipcc is needed to build the stream probe")
    return bench.stream_probe_fn()


def test_stream_probe_rejects_invalid_arguments_before_any_launch():
    """Every invalid call returns 1 from the argument checks (the fake addresses are never used)."""
    fn = _probe_lib()
    a = 1 << 20  # 16-byte aligned stand-ins
    ok = dict(pb=2, sb=4, ns=2, p=a, g=a, m=a, v=a, n=4096)
    bad = [dict(pb=3), dict(sb=8), dict(ns=3), dict(ns=0), dict(p=None), dict(g=None), dict(m=None),
           dict(v=None), dict(n=0), dict(n=4098), dict(p=a + 8), dict(v=a + 4), dict(n=(1 << 24) * 1024)]
    for change in bad:
        c = {**ok, **change}
        assert fn(c["pb"], c["sb"], c["ns"], c["p"], c["g"], c["m"], c["v"], c["n"], None) == 1, change


def test_stream_probe_shapes_reject_invalid_arguments_before_any_launch():
    """lv_stream_probe_shape makes lv_stream_probe's checks in every shape and rejects unknown
    shapes; lv_stream_probe_shape_info describes each shape, shape 0 being the step's own."""
    import ctypes

    _probe_lib()
    lib = bench.stream_probe_lib()
    count = lib.lv_stream_probe_shapes()
    assert count >= 2
    info = (ctypes.c_int * 8)()
    assert lib.lv_stream_probe_shape_info(0, info) == 0 and list(info) == [256, 1, 1, 0, 0, 0, 0, 0]
    for shape in range(count):
        assert lib.lv_stream_probe_shape_info(shape, info) == 0
        assert info[0] in (64, 128, 256, 1024) and info[1] in (1, 2, 4) and all(x in (0, 1) for x in info[2:6])
        assert all(0 <= x < 32 for x in info[6:]) and (info[5] or info[6] == info[7] == 0)
        assert bench.stream_shape_desc(lib, shape)
    assert lib.lv_stream_probe_shape_info(count, info) == 1
    assert lib.lv_stream_probe_shape_info(-1, info) == 1
    assert lib.lv_stream_probe_shape_info(0, None) == 1
    a = 1 << 20
    ok = dict(pb=2, sb=4, ns=2, p=a, g=a, m=a, v=a, n=4096)
    bad = [dict(pb=3), dict(sb=8), dict(ns=3), dict(p=None), dict(v=None), dict(n=0), dict(n=4098),
           dict(p=a + 8), dict(n=(1 << 24) * 1024)]
    for shape in range(count):
        fn = bench.stream_shape_fn(lib, shape)
        for change in bad:
            c = {**ok, **change}
            assert fn(c["pb"], c["sb"], c["ns"], c["p"], c["g"], c["m"], c["v"], c["n"], None) == 1, (shape, change)
    # a one-wave XCD-contiguous grid at lv_stream_probe's largest n would be 2^32 threads
    wave_xcd = [s for s in range(count)
                if lib.lv_stream_probe_shape_info(s, info) == 0 and info[0] == 64 and info[1] == 1 and info[4]]
    assert wave_xcd
    for shape in wave_xcd:
        c = {**ok, "n": ((1 << 24) - 1) * 1024}
        assert bench.stream_shape_fn(lib, shape)(c["pb"], c["sb"], c["ns"], c["p"], c["g"], c["m"], c["v"], c["n"],
                                                 None) == 1
    for shape in (-1, count):
        c = ok
        assert lib.lv_stream_probe_shape(shape, c["pb"], c["sb"], c["ns"], c["p"], c["g"], c["m"], c["v"], c["n"],
                                         None) == 1


def test_every_config_has_default_steps_and_warmup():
    """Each workload times about half a second of steps or more by default (cfg2's ~15 us step
    needs thousands for the bracketing synchronizations to vanish) and warms up first."""
    step_ms = {5: 23.1, 4: 2.13, 3: 0.57, 2: 0.0146}
    for c in bench.WORKLOADS:
        assert bench.DEFAULT_STEPS[c] > 0 and bench.DEFAULT_WARMUP[c] > 0
        assert bench.DEFAULT_STEPS[c] * step_ms[c] >= 400.0, c
