"""The stream-floor kernel that bench.py --stream-floor times (libstream_probe.so): on every
element-size combination it writes exactly what it states (p ^= g word by word, m ^= the group's
first gradient word, v ^= the group's first old m word, groups of 4 elements) over the n elements
and nothing past them, so the bandwidth it reports is that of real reads and writes of the whole
buffers."""
from __future__ import annotations

import itertools

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

PAD = 64  # elements past n that must stay as they were


def _run(torch, fn, pb, sb, ns, n, seed):
    rng = np.random.default_rng(seed)
    host = {k: rng.integers(0, 256, size=(n + PAD) * w, dtype=np.uint8)
            for k, w in (("p", pb), ("g", pb), ("m", sb), ("v", sb))}
    dev = {k: torch.from_numpy(x.copy()).cuda() for k, x in host.items()}
    rc = fn(pb, sb, ns, dev["p"].data_ptr(), dev["g"].data_ptr(), dev["m"].data_ptr(),
            dev["v"].data_ptr() if ns == 2 else None, n, None)
    assert rc == 0
    torch.cuda.synchronize()
    out = {k: t.cpu().numpy() for k, t in dev.items()}
    w = {k: x.view(np.uint32) for k, x in host.items()}
    groups = n // 4
    exp = {k: x.copy() for k, x in w.items()}
    exp["p"][:groups * pb] ^= w["g"][:groups * pb]
    gfirst = w["g"][0:groups * pb:pb]
    mfirst = w["m"][0:groups * sb:sb]
    exp["m"][:groups * sb] ^= np.repeat(gfirst, sb)
    if ns == 2:
        exp["v"][:groups * sb] ^= np.repeat(mfirst, sb)
    for k in ("p", "g", "m", "v"):
        assert np.array_equal(out[k].view(np.uint32), exp[k]), (k, pb, sb, ns, n)


@pytest.mark.parametrize("pb,sb,ns", list(itertools.product((2, 4), (2, 4), (1, 2))))
def test_stream_probe_writes_what_it_states(pb, sb, ns):
    import torch

    from tests.test_bench_contract import _probe_lib

    fn = _probe_lib()
    for i, n in enumerate((4, 1024, 3 * 1024 + 520, 40_000)):
        print(f"stream probe pb={pb} sb={sb} ns={ns} n={n}", flush=True)
        _run(torch, fn, pb, sb, ns, n, seed=100 * pb + 10 * sb + ns + i)
