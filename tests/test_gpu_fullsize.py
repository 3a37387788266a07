"""Full-size and shard checks on the GPU.

* cfg5: T2 + cautious, bf16 params/grads, fp32 m/v, one
  6,738,415,616-element bucket. Size-independent checks at full size:
  - the exact cautious count: with m = 0 at step 1 (and m = (1-b1) g at step 2 with the same
    grad), sign(u) = sign(g), so the mask is exactly "g != 0"; the count is an integer torch sum
    and the expected scratch comes from the oracle's pinned cautious-scale / EMA routines;
  - bitwise equality with the oracle on slices that straddle 2^31 and 2^32 (the int32
    offset wraps twice) and on the tail, re-run on the host with index_base = slice start and the
    GPU's pre-step scratch.
* T1 with bf16 params, grads and m and an fp32 master past 2^32 elements: the split lane layout
  of 2048-element units, the same exact-count and slice checks.
* shards: a tensor stepped as slices with index_base equals the whole tensor stepped at once, and
  each shard equals the oracle stepped on it with the same index base (bases across 2^31 and 2^32).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from tests.parity_util import assert_bitwise, group_dict, oracle_config

pytestmark = pytest.mark.gpu

N5 = 32 * (4 * 4096 * 4096 + 3 * 4096 * 11008 + 2 * 4096) + 2 * 32000 * 4096 + 4096


def _need_gpu(min_free_gb: float = 0.0):
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    free, _ = torch.cuda.mem_get_info()
    if free < min_free_gb * 1e9:
        pytest.skip(f"needs {min_free_gb} GB of free HBM")


def test_shards_with_index_base_equal_whole():
    _need_gpu()
    from luminamoon_amd.optimizer.hip_backend import HipStepper

    n = 3 * (1 << 20) + 777
    gen = torch.Generator(device="cuda").manual_seed(3)
    p0 = (torch.randn(n, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
    g = (torch.randn(n, device="cuda", generator=gen) * 1e-3).to(torch.bfloat16)
    group = group_dict(buffer="T2", lr=1e-3, cautious=False)  # no global scale: shards are independent
    st = HipStepper()
    whole = [p0.clone(), torch.zeros(n, device="cuda"), torch.zeros(n, device="cuda"),
             torch.tensor([0, 0, 0, 1, 1, 0.0], device="cuda")]
    cuts = [0, 1_000_003, 2_500_000, n]
    shards = [[p0[a:b].clone(), torch.zeros(b - a, device="cuda"), torch.zeros(b - a, device="cuda"),
               torch.tensor([0, 0, 0, 1, 1, 0.0], device="cuda")] for a, b in zip(cuts, cuts[1:])]
    for t in (1, 2, 3):
        st.step(group, [whole[0]], [g], [whole[1]], [whole[2]], [None], [whole[3]], [t], [0])
        st.step(group, [s[0] for s in shards], [g[a:b] for a, b in zip(cuts, cuts[1:])], [s[1] for s in shards],
                [s[2] for s in shards], [None] * 3, [s[3] for s in shards], [t] * 3, [0] * 3, index_bases=cuts[:-1])
    torch.cuda.synchronize()
    assert_bitwise(torch.cat([s[0] for s in shards]), whole[0], "p")
    assert_bitwise(torch.cat([s[1] for s in shards]), whole[1], "m")
    assert_bitwise(torch.cat([s[2] for s in shards]), whole[2], "v")


@pytest.mark.parametrize("sdt", ["f32", "bf16"])
def test_shards_with_index_base_match_oracle(oracle_mod, sdt):
    """HIP shards stepped with index_base against the oracle stepped on the same shards with the
    same index bases, bit for bit (p, m, v, scratch after each of 3 steps: the two-pass first
    step, then fused). Element i of a shard at index_base a hashes the offset (int32)(a + i): the
    reference's `idx as i32` of the unsharded tensor (reference_cpu/dual.rs:54, prng.rs:4-26); the
    oracle's index_base is pinned to its own whole-tensor run on the CPU (test_oracle_pins.py).
    The shards are slices of flat buffers cut at unaligned points (every buffer of a shard starts
    mid-vector, so they take the vector path after a head), with bf16 params, stochastic rounding
    and cautious on (each shard its own tensor and scratch on both sides), and fp32 or bf16 state.
    Index bases: the cut points themselves, then bases that straddle 2^31 and 2^32 and one past
    2^32 + 2^31."""
    _need_gpu()
    from luminamoon_amd.optimizer.hip_backend import HipStepper

    O = oracle_mod
    n = 3 * (1 << 20) + 777
    cuts = [0, 1_000_003, 2_500_001, n]
    sizes = [b - a for a, b in zip(cuts, cuts[1:])]
    st_dt = torch.float32 if sdt == "f32" else torch.bfloat16
    group = group_dict(buffer="T2", lr=1e-3, state_precision="fp32" if sdt == "f32" else "param")
    cfg = oracle_config(O, group)
    two31, two32 = 1 << 31, 1 << 32
    for bases in (cuts[:-1], [two31 - 400_000, two32 - 1_300_000, two32 + two31 + 5]):
        print(f"[case] shards state={sdt} index_bases={bases}", flush=True)
        gen = torch.Generator(device="cuda").manual_seed(3)
        p = (torch.randn(n, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
        m = torch.zeros(n, dtype=st_dt, device="cuda")
        v = torch.zeros(n, dtype=st_dt, device="cuda")
        dev = [(p[a:b], m[a:b], v[a:b], torch.tensor([0, 0, 0, 1, 1, 0.0], device="cuda"))
               for a, b in zip(cuts, cuts[1:])]
        host = [tuple(t.cpu().clone() for t in d) for d in dev]
        st = HipStepper()
        for t in (1, 2, 3):
            g = (torch.randn(n, device="cuda", generator=gen) * 1e-3).to(torch.bfloat16)
            gs = [g[a:b] for a, b in zip(cuts, cuts[1:])]
            st.step(group, [d[0] for d in dev], gs, [d[1] for d in dev], [d[2] for d in dev], [None] * 3,
                    [d[3] for d in dev], [t] * 3, [0] * 3, index_bases=bases)
            O.step(cfg, [h[0] for h in host], [x.cpu() for x in gs], [h[1] for h in host], [h[2] for h in host],
                   [None] * 3, [h[3] for h in host], [t] * 3, [0] * 3, threads=8, index_bases=bases)
            torch.cuda.synchronize()
            for k, (d, h) in enumerate(zip(dev, host)):
                for name, x, y in zip(("p", "m", "v", "scratch"), h, d):
                    assert_bitwise(x, y, f"step {t} shard {k} (base {bases[k]}, {sizes[k]} elements) {name}")


def test_cfg5_full_bucket_count_and_wrap_slices(oracle_mod):
    _need_gpu(min_free_gb=100)
    from luminamoon_amd.optimizer.hip_backend import HipStepper

    O = oracle_mod
    L = O.lib()
    n = N5
    print(f"[fullsize] cfg5 n={n}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(5)
    p = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    g = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    chunk = 1 << 27
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        z = torch.randn(e - s, device="cuda", generator=gen)
        p[s:e].copy_(z.mul_(0.02))
        z = torch.randn(e - s, device="cuda", generator=gen)
        chi2 = torch.zeros(e - s, device="cuda")
        for _ in range(3):
            w = torch.randn(e - s, device="cuda", generator=gen)
            chi2.addcmul_(w, w)
        z.div_(chi2.div_(3.0).sqrt_())
        z[::20] = 0.0  # exact zeros: 5% of the mask is off
        g[s:e].copy_(z.mul_(1e-3))
        del z, chi2, w
    m = torch.zeros(n, device="cuda")
    v = torch.zeros(n, device="cuda")
    sc = torch.tensor([0, 0, 0, 1, 1, 0.0], device="cuda")
    count = int((g != 0).sum().item())
    group = group_dict(buffer="T2", lr=1e-3)
    cfg = oracle_config(O, group)
    st = HipStepper()
    two32 = 1 << 32
    slices = [(0, 1 << 22), ((1 << 31) - (1 << 21), (1 << 31) + (1 << 21)), (two32 - (1 << 21), two32 + (1 << 21)),
              (n - (1 << 22) - 5, n)]

    # step 1: two-pass; scratch[3] = 1 / clamp(count / n, 0.5, 1) with the count as f32
    st.step(group, [p], [g], [m], [v], [None], [sc], [1], [0])
    torch.cuda.synchronize()
    want1 = L.lvo_cautious_scale(L.lvo_u64_to_f32(count), L.lvo_u64_to_f32(n), 0.5)
    got1 = sc.cpu()
    assert got1[3].item() == want1 and got1[4].item() == 1.0 and got1[0].item() == 0.0

    # step 2: fused, lagged scale; keep host copies of the slices before the step
    before = [(p[a:b].cpu(), g[a:b].cpu(), m[a:b].cpu(), v[a:b].cpu()) for a, b in slices]
    sc_before = got1.clone()
    st.step(group, [p], [g], [m], [v], [None], [sc], [2], [0])
    torch.cuda.synchronize()
    s_exp = (ctypes.c_float * 6)(*[float(x) for x in sc_before])
    s_exp[0] = L.lvo_u64_to_f32(count)
    L.lvo_update_post_step_ema(s_exp, L.lvo_u64_to_f32(n), ctypes.byref(cfg), 1)
    got2 = sc.cpu()
    assert list(got2.numpy().view(np.uint32)) == list(np.array(list(s_exp), dtype=np.float32).view(np.uint32))

    for (a, b), (hp, hg, hm, hv) in zip(slices, before):
        hs = sc_before.clone()
        O.step(cfg, [hp], [hg], [hm], [hv], [None], [hs], [2], [0], threads=8, index_bases=[a])
        print(f"[fullsize] slice [{a}, {b})", flush=True)
        assert_bitwise(hp, p[a:b], f"p[{a}:{b}]")
        assert_bitwise(hm, m[a:b], f"m[{a}:{b}]")
        assert_bitwise(hv, v[a:b], f"v[{a}:{b}]")
    del p, g, m, v
    torch.cuda.empty_cache()


def test_bf16_state_master_past_2_32_split_lanes(oracle_mod):
    """T1 with bf16 params, grads and m and an fp32 master (semi): 2048-element units whose
    threads own two groups of 4 elements 1024 apart (an f32 stream beside 16-bit ones), over
    2^32 + 2^21 + 4101 elements (a 5-element last unit). The cautious count is exact at steps 1
    and 2 (sign(u) = sign(g), as m starts at 0 and then holds a rounding of (1 - b1) g); slices
    across 2^31, 2^32 and the tail equal the oracle bit for bit at step 2."""
    _need_gpu(min_free_gb=60)
    from luminamoon_amd.optimizer.hip_backend import HipStepper

    O = oracle_mod
    L = O.lib()
    n = (1 << 32) + (1 << 21) + 4101
    print(f"[fullsize] T1 bf16 state + semi master n={n}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(11)
    p = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    g = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    chunk = 1 << 27
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        z = torch.randn(e - s, device="cuda", generator=gen)
        p[s:e].copy_(z.mul_(0.02))
        z = torch.randn(e - s, device="cuda", generator=gen)
        z[::20] = 0.0
        g[s:e].copy_(z.mul_(1e-3))
        del z
    mp = torch.empty(n, dtype=torch.float32, device="cuda")
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        mp[s:e].copy_(p[s:e])
    m = torch.zeros(n, dtype=torch.bfloat16, device="cuda")
    sc = torch.tensor([0, 0, 0, 1, 1, 0.0], device="cuda")
    count = int((g != 0).sum().item())
    group = group_dict(buffer="T1", lr=1e-3, master_weights="semi", state_precision="param")
    cfg = oracle_config(O, group)
    st = HipStepper()
    two32 = 1 << 32
    slices = [(0, 1 << 21), ((1 << 31) - (1 << 20), (1 << 31) + (1 << 20)),
              (two32 - (1 << 20) - 3, two32 + (1 << 20)), (n - (1 << 21) - 7, n)]

    st.step(group, [p], [g], [m], [None], [mp], [sc], [1], [0])
    torch.cuda.synchronize()
    want1 = L.lvo_cautious_scale(L.lvo_u64_to_f32(count), L.lvo_u64_to_f32(n), 0.5)
    got1 = sc.cpu()
    assert got1[3].item() == want1 and got1[4].item() == 1.0 and got1[0].item() == 0.0

    before = [(p[a:b].cpu(), g[a:b].cpu(), m[a:b].cpu(), mp[a:b].cpu()) for a, b in slices]
    sc_before = got1.clone()
    st.step(group, [p], [g], [m], [None], [mp], [sc], [2], [0])
    torch.cuda.synchronize()
    s_exp = (ctypes.c_float * 6)(*[float(x) for x in sc_before])
    s_exp[0] = L.lvo_u64_to_f32(count)
    L.lvo_update_post_step_ema(s_exp, L.lvo_u64_to_f32(n), ctypes.byref(cfg), 1)
    got2 = sc.cpu()
    assert list(got2.numpy().view(np.uint32)) == list(np.array(list(s_exp), dtype=np.float32).view(np.uint32))

    for (a, b), (hp, hg, hm, hmp) in zip(slices, before):
        hs = sc_before.clone()
        O.step(cfg, [hp], [hg], [hm], [None], [hmp], [hs], [2], [0], threads=8, index_bases=[a])
        print(f"[fullsize] slice [{a}, {b})", flush=True)
        assert_bitwise(hp, p[a:b], f"p[{a}:{b}]")
        assert_bitwise(hm, m[a:b], f"m[{a}:{b}]")
        assert_bitwise(hmp, mp[a:b], f"master[{a}:{b}]")
    del p, g, m, mp
    torch.cuda.empty_cache()
