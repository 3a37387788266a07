"""BASELINE.json configs as parity cases at their real shapes, through the drop-in LuminaV class:
every final buffer bit for bit against the oracle run on the same inputs.

* cfg2: buffer=1 (TD-CLM, lam 0.3), fp32, 64 ragged unfused tensors (bench.py's
  seeded log-uniform sizes, 3,514,803 elements), grads N(0, 1e-3) with 5% exact zeros, 50 steps.
* cfg3: buffer=2, cautious, fp32, fuse_tensors=True: the GPT-2-small parameter list
  (123,570,432 elements) in one bucket, 3 steps.
* cfg4: buffer="T1" (lam 0.3), bf16 params and grads, fp32 m, fuse_tensors=True:
  the Llama-1B-shaped list (953,223,168 elements) in one bucket, 2 steps.

cfg1 (the README example, 100 steps) is test_gpu_parity.test_luminav_readme_example_100_steps and
cfg5 (6.7e9 elements) is test_gpu_fullsize (exact count + slices across the int32 wraps). The
oracle runs its AVX-512 backend when the host has one: it equals the scalar core bit for bit on
finite inputs (tests/test_oracle_simd.py), and is an order of magnitude faster at these sizes.
"""
from __future__ import annotations

import contextlib

import numpy as np
import pytest
import torch

from tests.parity_util import assert_bitwise, group_dict, oracle_config

pytestmark = pytest.mark.gpu


def _need_gpu(min_free_gb: float = 0.0):
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    free, _ = torch.cuda.mem_get_info()
    if free < min_free_gb * 1e9:
        pytest.skip(f"needs {min_free_gb} GB of free HBM")


def _fast_oracle(O):
    return O.backend(O.BACKEND_AVX512) if O.avx512_available() else contextlib.nullcontext()


def _gpu_normal(n, gen, scale, dtype, zero_every=0):
    x = torch.randn(n, device="cuda", generator=gen).mul_(scale)
    if zero_every:
        x[::zero_every] = 0.0
    return x.to(dtype)


def test_cfg2_64_ragged_unfused_50_steps(oracle_mod):
    _need_gpu()
    import bench
    from luminamoon_amd import LuminaV

    O = oracle_mod
    sizes = bench.cfg2_sizes()
    assert len(sizes) == 64 and sum(sizes) == 3_514_803
    rng = np.random.default_rng(21)
    p0 = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in sizes]
    params = [torch.nn.Parameter(torch.from_numpy(x.copy()).cuda()) for x in p0]
    opt = LuminaV(params, buffer=1, lam=0.3)
    group = group_dict(buffer=1, lam=0.3)
    cfg = oracle_config(O, group)
    hp = [torch.from_numpy(x.copy()) for x in p0]
    hm = [torch.zeros(s) for s in sizes]
    hs = [torch.tensor([0, 0, 0, 1, 1, 0], dtype=torch.float32) for _ in sizes]
    idx = list(range(64))
    print(f"[case] cfg2 64 tensors, {sum(sizes)} elements, 50 steps", flush=True)
    with _fast_oracle(O):
        for t in range(1, 51):
            gs = []
            for s in sizes:
                g = (rng.standard_normal(s) * 1e-3).astype(np.float32)
                g[rng.random(s) < 0.05] = 0.0
                gs.append(torch.from_numpy(g))
            for p, g in zip(params, gs):
                p.grad = g.cuda()
            opt.step()
            O.step(cfg, hp, gs, hm, [None] * 64, [None] * 64, hs, [t] * 64, idx, threads=8)
            if t in (1, 2, 50):
                torch.cuda.synchronize()
                for i, p in enumerate(params):
                    st = opt.state[p]
                    assert_bitwise(hp[i], p.detach(), f"step {t} p[{i}]")
                    assert_bitwise(hm[i], st["exp_avg"], f"step {t} m[{i}]")
                    assert_bitwise(hs[i], st["scratch"], f"step {t} scratch[{i}]")


def _bucket_case(O, shapes, dtype, group_kw, steps, seed, cap_mb):
    from luminamoon_amd import LuminaV

    gen = torch.Generator(device="cuda").manual_seed(seed)
    params = [torch.nn.Parameter(_gpu_normal(int(np.prod(s)), gen, 0.02, dtype).view(s)) for s in shapes]
    opt = LuminaV(params, fuse_tensors=True, bucket_cap_mb=cap_mb, **group_kw)
    assert len(opt._fused_buckets) == 1
    b = opt._fused_buckets[0]
    n = b["flat_p"].numel()
    assert n == sum(int(np.prod(s)) for s in shapes)
    g0, g1 = b["flat_g"].data_ptr(), b["flat_g"].data_ptr() + n * b["flat_g"].element_size()
    assert all(g0 <= p.grad.data_ptr() < g1 for p in params)  # grads are views of the bucket's flat_g
    group = group_dict(fuse_tensors=True, bucket_cap_mb=cap_mb, **group_kw)
    cfg = oracle_config(O, group)
    dual = b["flat_v"] is not None
    hp = b["flat_p"].cpu()
    hm = torch.zeros(n)
    hv = torch.zeros(n) if dual else None
    hs = torch.tensor([0, 0, 0, 1, 1, 0], dtype=torch.float32)
    with _fast_oracle(O):
        for t in range(1, steps + 1):
            g = _gpu_normal(n, gen, 1e-3, dtype)
            off = 0
            for p in params:  # p.grad is the bucket's view of flat_g
                k = p.numel()
                p.grad.copy_(g[off:off + k].view(p.shape))
                off += k
            opt.step()
            O.step(cfg, [hp], [g.cpu()], [hm], [hv], [None], [hs], [t], [0], threads=16)
            del g
    torch.cuda.synchronize()
    assert_bitwise(hp, b["flat_p"], "flat_p")
    assert_bitwise(hm, b["flat_m"], "flat_m")
    if dual:
        assert_bitwise(hv, b["flat_v"], "flat_v")
    assert_bitwise(hs, b["scratch"], "scratch")


def test_cfg3_gpt2_small_bucket(oracle_mod):
    _need_gpu(min_free_gb=8)
    shapes = [s for _ in range(12) for s in ((768, 2304), (768, 768), (768, 3072), (3072, 768))]
    shapes += [(768,)] * 50 + [(50257, 768)]
    print("[case] cfg3 GPT-2-small bucket, CLM cautious fp32, 3 steps", flush=True)
    _bucket_case(oracle_mod, shapes, torch.float32, dict(buffer=2, cautious=True), steps=3, seed=3, cap_mb=500.0)


def test_cfg4_llama1b_bucket(oracle_mod):
    _need_gpu(min_free_gb=24)
    shapes = [s for _ in range(16) for s in ((2048, 2048),) * 4 + ((2048, 5632),) * 3 + ((2048,),) * 2]
    shapes += [(32000, 2048)] * 2 + [(2048,)]
    print("[case] cfg4 Llama-1B bucket, T1 lam 0.3, bf16 + fp32 m, 2 steps", flush=True)
    _bucket_case(oracle_mod, shapes, torch.bfloat16, dict(buffer="T1", lam=0.3), steps=2, seed=4, cap_mb=2048.0)
