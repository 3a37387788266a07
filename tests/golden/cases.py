"""Golden cases: inputs come from the reference's deterministic generator
generate_pseudo_random_tensor (optimizer/crates/luminav-simd/tests/differential_parity.rs:18-27),
restated here on top of the pinned _prng, so no RNG library version is involved."""
from __future__ import annotations

import numpy as np

I32_MAX = 2147483647


def prng(seed: int, idx: np.ndarray) -> np.ndarray:
    """_prng (prng.rs:21-26) vectorised with int64 products masked to 32 bits."""
    z = (idx.astype(np.int64) + int(seed) - 1640531527).astype(np.int64) & 0xFFFFFFFF
    z = z.astype(np.uint32).view(np.int32).astype(np.int64)
    z = ((z ^ (z >> 16)) * -2048173461) & 0xFFFFFFFF
    z = z.astype(np.uint32).view(np.int32).astype(np.int64)
    z = ((z ^ (z >> 13)) * -1028477387) & 0xFFFFFFFF
    z = z.astype(np.uint32).view(np.int32).astype(np.int64)
    return (z ^ (z >> 16)).astype(np.int32)


def pseudo_random(n: int, seed: int, scale: float) -> np.ndarray:
    """unit = (prng(seed, i) as f64 / i32::MAX as f64) as f32; val = unit * scale (f32)."""
    r = prng(seed, np.arange(n, dtype=np.int64).astype(np.int32))
    unit = (r.astype(np.float64) / float(I32_MAX)).astype(np.float32)
    return (unit * np.float32(scale)).astype(np.float32)


# name: (group kwargs, param dtype, state dtype, sizes, steps, lr)
CASES = {
    "clm_f32_readme": (dict(buffer=2, lr=8e-4, weight_decay=0.08), "f32", "f32", [640, 10], 100),
    "t2_bf16_f32state": (dict(buffer="T2", lr=1e-3), "bf16", "f32", [4099, 7, 2048], 12),
    "tdclm_f32_ragged": (dict(buffer=1, lr=8e-4, lam=0.3), "f32", "f32", [1, 2, 3, 5, 17, 129, 255, 1000, 2049, 4097], 10),
    "t1_bf16_bf16state": (dict(buffer="T1", lr=1e-3, state_precision="param"), "bf16", "bf16", [3001, 65], 10),
    "clm_f16_f16state_master": (dict(buffer=2, lr=1e-3, master_weights="semi", state_precision="param"), "f16", "f16", [1500], 8),
    "t2_bf16_nocautious_fused_off": (dict(buffer="T2", lr=2e-3, cautious=False, fused_single_pass=False), "bf16", "f32", [5000], 6),
}

NP_DT = {"f32": np.float32}


def to_dtype(x32: np.ndarray, dt: str):
    import torch

    t = torch.from_numpy(x32.copy())
    return {"f32": t, "bf16": t.to(torch.bfloat16), "f16": t.to(torch.float16)}[dt]


def inputs(name: str):
    """Initial params and per-step grads (torch CPU tensors) of a case."""
    gk, pdt, sdt, sizes, steps = CASES[name]
    params = [to_dtype(pseudo_random(n, 42 + 31 * i, 0.5), pdt) for i, n in enumerate(sizes)]
    grads = [[to_dtype(pseudo_random(n, 1000 + 97 * s + 7 * i, 0.05), pdt) for i, n in enumerate(sizes)]
             for s in range(steps)]
    return params, grads
