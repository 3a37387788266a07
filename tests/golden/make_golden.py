"""Writes tests/golden/*.npz: oracle outputs for the cases in cases.py (run on the CPU).

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from tests.golden.cases import CASES, inputs  # noqa: E402
from tests.parity_util import bits, group_dict, oracle_config  # noqa: E402

SDT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def run_oracle(name: str):
    gk, pdt, sdt, sizes, steps = CASES[name]
    group = group_dict(**gk)
    cfg = oracle_config(O, group)
    params, grads = inputs(name)
    dual = group["buffer"] in (2, "T2")
    master = group["master_weights"] > 0 and pdt != "f32"
    p = [x.clone() for x in params]
    m = [torch.zeros(n, dtype=SDT[sdt]) for n in sizes]
    v = [torch.zeros(n, dtype=SDT[sdt]) if dual else None for n in sizes]
    mp = [x.float().clone() if master else None for x in params]
    sc = [torch.tensor([0, 0, 0, 1, 1, 0], dtype=torch.float32) for _ in sizes]
    for s in range(steps):
        O.step(cfg, p, grads[s], m, v, mp, sc, [s + 1] * len(sizes), list(range(len(sizes))))
    out = {}
    for i in range(len(sizes)):
        out[f"p{i}"] = bits(p[i])
        out[f"m{i}"] = bits(m[i])
        if v[i] is not None:
            out[f"v{i}"] = bits(v[i])
        if mp[i] is not None:
            out[f"mp{i}"] = bits(mp[i])
        out[f"sc{i}"] = bits(sc[i])
    return out


def main() -> None:
    O.build()
    for name in CASES:
        out = run_oracle(name)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **{k: v.astype(np.uint32) for k, v in out.items()})
        print("wrote", name)


if __name__ == "__main__":
    main()
