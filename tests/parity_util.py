"""Shared helpers for the parity tests: seeded inputs, oracle runs and bitwise comparison.

The oracle (oracle/oracle.py) is the checker here; the product path is luminamoon_amd.
"""
from __future__ import annotations

from typing import Any, Dict, List, Optional, Sequence

import numpy as np
import torch

DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def seeded_tensor(n: int, seed: int, scale: float, dtype: torch.dtype, zero_frac: float = 0.0) -> torch.Tensor:
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * scale).astype(np.float32)
    if zero_frac > 0:
        x[rng.random(n) < zero_frac] = 0.0
    return torch.from_numpy(x).to(dtype)


def prng_np(seed: int, idx: np.ndarray) -> np.ndarray:
    """_prng (prng.rs:21-26) vectorised with the arithmetic of the reference's NumPy restatement
    (validation.py:73-77); tests compare it with the oracle's lvo_prng."""
    z = (idx.astype(np.int64) + int(seed) - 1640531527).astype(np.int32)
    z = (((z ^ (z >> 16)).astype(np.int64) * -2048173461) & 0xFFFFFFFF).astype(np.int32)
    z = (((z ^ (z >> 13)).astype(np.int64) * -1028477387) & 0xFFFFFFFF).astype(np.int32)
    return (z ^ (z >> 16)).astype(np.int32)


def reference_pseudo_random(n: int, seed: int, scale: float, dtype: torch.dtype) -> torch.Tensor:
    """The inputs of the reference's differential-parity tests
    (luminav-simd/tests/differential_parity.rs:18-27): unit = f32(prng / i32::MAX), val = unit *
    scale in f32, rounded to the dtype (RNE, no noise)."""
    r = prng_np(seed, np.arange(n, dtype=np.int64))
    unit = (r.astype(np.float64) / float(2 ** 31 - 1)).astype(np.float32)
    val = unit * np.float32(scale)
    return torch.from_numpy(val).to(dtype)


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().astype(np.int64) & 0xFFFF
    return t.view(torch.int32).numpy().astype(np.int64) & 0xFFFFFFFF


def assert_bitwise(a: torch.Tensor, b: torch.Tensor, label: str) -> None:
    ba, bb = bits(a), bits(b)
    if ba.shape != bb.shape:
        raise AssertionError(f"{label}: shape {ba.shape} vs {bb.shape}")
    diff = np.nonzero(ba != bb)[0]
    if diff.size:
        i = int(diff[0])
        av = a.detach().reshape(-1)[i].float().item()
        bv = b.detach().reshape(-1)[i].float().item()
        raise AssertionError(
            f"{label}: {diff.size} of {ba.size} elements differ; first at {i}: "
            f"{av!r} (0x{int(ba[i]):x}) vs {bv!r} (0x{int(bb[i]):x})"
        )


def group_dict(**kw: Any) -> Dict[str, Any]:
    """A normalised LuminaV param group (the constructor's own validation)."""
    from luminamoon_amd.optimizer.luminav import LuminaV
    from luminamoon_amd.optimizer import constants as C

    g: Dict[str, Any] = dict(
        lr=C.DEFAULT_LR, betas=C.DEFAULT_BETAS, eps=C.DEFAULT_EPS, weight_decay=C.DEFAULT_WEIGHT_DECAY, tau=C.DEFAULT_TAU,
        lam=C.DEFAULT_LAM, cautious=True, cautious_clamp_min=C.DEFAULT_CAUTIOUS_CLAMP_MIN, buffer=2,
        stochastic_rounding=True, bound=True, bound_type="coordinate", bound_ratio=C.DEFAULT_BOUND_RATIO,
        master_weights="none", execution="auto", fused_single_pass=True, fuse_tensors=False,
        bucket_cap_mb=C.DEFAULT_BUCKET_CAP_MB, prewarm_jit=True, ema_decay="auto", fsdp_sync=False,
        seed=C.DEFAULT_OPTIMIZER_SEED, version="1.6.0", state_precision="fp32",
    )
    g.update(kw)
    LuminaV._validate_and_normalize_group(g)
    return g


def oracle_config(O, group: Dict[str, Any]):
    return O.make_config(
        lr=group["lr"], betas=group["betas"], eps=group["eps"], weight_decay=group["weight_decay"], tau=group["tau"],
        lam=group["lam"], cautious=group["cautious"], cautious_clamp_min=group["cautious_clamp_min"],
        buffer=group["buffer"], stochastic_rounding=group["stochastic_rounding"], bound=group["bound"],
        bound_type=group["bound_type"], bound_ratio=group["bound_ratio"], master_weights=group["master_weights"],
        fused_single_pass=group["fused_single_pass"], ema_decay=group["ema_decay"], seed=group["seed"],
    )


class TensorSet:
    """Host copies of p/g/m/v/mp/scratch for a list of tensors, steppable by the oracle,
    plus device copies steppable by the HIP backend."""

    def __init__(self, sizes: Sequence[int], pdt: str, gdt: str, sdt: str, dual: bool, master: bool, seed: int,
                 p_scale: float = 0.02, m_scale: float = 0.0):
        self.sizes = list(sizes)
        self.p: List[torch.Tensor] = []
        self.m: List[torch.Tensor] = []
        self.v: List[Optional[torch.Tensor]] = []
        self.mp: List[Optional[torch.Tensor]] = []
        self.sc: List[torch.Tensor] = []
        self.pdt, self.gdt, self.sdt = DT[pdt], DT[gdt], DT[sdt]
        for i, n in enumerate(self.sizes):
            p = seeded_tensor(n, seed + 17 * i, p_scale, self.pdt)
            self.p.append(p)
            if m_scale > 0:
                self.m.append(seeded_tensor(n, seed + 17 * i + 5, m_scale, self.sdt))
                self.v.append(seeded_tensor(n, seed + 17 * i + 6, m_scale, self.sdt).abs() if dual else None)
            else:
                self.m.append(torch.zeros(n, dtype=self.sdt))
                self.v.append(torch.zeros(n, dtype=self.sdt) if dual else None)
            self.mp.append(p.float().clone() if master else None)
            self.sc.append(torch.tensor([0, 0, 0, 1, 1, 0], dtype=torch.float32))

    def grads(self, step: int, seed: int, scale: float = 1e-3, zero_frac: float = 0.05) -> List[torch.Tensor]:
        return [seeded_tensor(n, seed * 1000 + step * 101 + i, scale, self.gdt, zero_frac) for i, n in enumerate(self.sizes)]

    def to(self, device) -> "TensorSet":
        out = object.__new__(TensorSet)
        out.sizes = self.sizes
        out.pdt, out.gdt, out.sdt = self.pdt, self.gdt, self.sdt
        mv = lambda xs: [None if x is None else x.clone().to(device) for x in xs]  # noqa: E731
        out.p, out.m, out.v, out.mp, out.sc = mv(self.p), mv(self.m), mv(self.v), mv(self.mp), mv(self.sc)
        return out

    def oracle_step(self, O, cfg, grads: Sequence[torch.Tensor], step: int, param_indices=None, threads: int = 1) -> None:
        n = len(self.sizes)
        O.step(cfg, self.p, list(grads), self.m, self.v, self.mp, self.sc, [step] * n,
               param_indices if param_indices is not None else list(range(n)), threads=threads)

    def hip_step(self, stepper, group, grads: Sequence[torch.Tensor], step: int, param_indices=None) -> None:
        n = len(self.sizes)
        stepper.step(group, self.p, list(grads), self.m, self.v, self.mp, self.sc, [step] * n,
                     param_indices if param_indices is not None else list(range(n)))

    def assert_equal(self, other: "TensorSet", label: str, check_scratch: bool = True) -> None:
        for i in range(len(self.sizes)):
            assert_bitwise(self.p[i], other.p[i], f"{label} p[{i}]")
            assert_bitwise(self.m[i], other.m[i], f"{label} m[{i}]")
            if self.v[i] is not None:
                assert_bitwise(self.v[i], other.v[i], f"{label} v[{i}]")
            if self.mp[i] is not None:
                assert_bitwise(self.mp[i], other.mp[i], f"{label} mp[{i}]")
            if check_scratch:
                assert_bitwise(self.sc[i], other.sc[i], f"{label} scratch[{i}]")
