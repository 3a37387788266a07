"""The C ABI library loads here (no GPU), exports every function include/luminav_hip.h declares,
and rejects bad calls on the host before touching the device."""
from __future__ import annotations

import ctypes
import os
import re
import shutil
import subprocess

import pytest

from luminamoon_amd.optimizer import hip_backend as H

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "luminav_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(lv_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(H.LIB_PATH):
        from luminamoon_amd import build_ext

        build_ext.build()
    return H.load_library()


def test_header_declares_expected_entry_points():
    assert declared_functions() == sorted(H.EXPORTED_SYMBOLS)


def test_every_declared_symbol_is_exported(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_version_and_workspace(lib):
    assert lib.lv_version() >= 100
    ws = lib.lv_workspace_bytes(1)
    assert ws % 256 == 0
    # the launches of a call reuse per-launch regions, so the size does not grow with the count
    assert lib.lv_workspace_bytes(48) == ws
    # 48 x 65 count words 64 B apart, 48 tickets, and the radial records of one 2^22-unit piece
    # (2 doubles + a u32 count per unit)
    assert ws >= 48 * 65 * 64 + 48 * 8 + (1 << 22) * 20
    # more than 48 tensors: table launches add count words and a descriptor table for 960 tensors
    assert lib.lv_workspace_bytes(49) == ws + 960 * 65 * 64 + 960 * 80
    assert lib.lv_workspace_bytes(100_000) == lib.lv_workspace_bytes(49)


def _c_layout(struct, fields, tmp_path):
    """sizeof and offsetof of `struct` as gcc lays out include/luminav_hip.h."""
    src = tmp_path / "layout.c"
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "luminav_hip.h"', "int main(void) {",
             f'  printf("%zu\\n", sizeof({struct}));']
    lines += [f'  printf("%zu\\n", offsetof({struct}, {f}));' for f in fields]
    lines += ["  return 0;", "}"]
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    return int(out[0]), [int(x) for x in out[1:]]


@pytest.mark.parametrize("ctype,cname", [(H.LvConfig, "lv_config"), (H.LvTensor, "lv_tensor")])
def test_struct_layouts_match_header(ctype, cname, tmp_path):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    names = [f[0] for f in ctype._fields_]
    size, offsets = _c_layout(cname, names, tmp_path)
    assert ctypes.sizeof(ctype) == size
    assert [getattr(ctype, f).offset for f in names] == offsets


def _cfg(**kw):
    from tests.parity_util import group_dict

    return H.make_config(group_dict(**kw))


def test_host_side_rejections_without_device(lib):
    cfg = _cfg(buffer="T2")
    WS = lib.lv_workspace_bytes(1)
    ws = (ctypes.c_uint8 * WS)()
    t = H.LvTensor()
    assert lib.lv_step_multi(None, ctypes.byref(t), 1, ws, WS, None) == -1
    assert lib.lv_step_multi(ctypes.byref(cfg), None, 0, ws, WS, None) == 0  # nothing to do
    assert lib.lv_step_multi(ctypes.byref(cfg), None, 1, ws, WS, None) == -1
    bad = _cfg(buffer="T2")
    bad.lr = float("nan")
    assert lib.lv_step_multi(ctypes.byref(bad), ctypes.byref(t), 1, ws, WS, None) == -3
    assert b"learning rate" in lib.lv_last_error()
    bad = _cfg(buffer="T2")
    bad.beta2 = 1.0
    assert lib.lv_step_multi(ctypes.byref(bad), ctypes.byref(t), 1, ws, WS, None) == -3
    # a tensor with numel but no pointers
    t.numel, t.step = 10, 1
    assert lib.lv_step_multi(ctypes.byref(cfg), ctypes.byref(t), 1, ws, WS, None) == -1
    assert b"null" in lib.lv_last_error()
    # missing exp_avg_sq in a dual-state mode, missing master for bf16 with master weights
    t.param = t.grad = t.exp_avg = t.scratch = 0x1000
    t.param_dtype = t.grad_dtype = 1
    assert lib.lv_step_multi(ctypes.byref(cfg), ctypes.byref(t), 1, ws, WS, None) == -1
    assert b"exp_avg_sq" in lib.lv_last_error()
    t.exp_avg_sq = 0x2000
    mcfg = _cfg(buffer="T2", master_weights="full")
    assert lib.lv_step_multi(ctypes.byref(mcfg), ctypes.byref(t), 1, ws, WS, None) == -1
    assert b"master_param" in lib.lv_last_error()
    # step 0, a too-small workspace, grad aliasing param
    t.step = 0
    assert lib.lv_step_multi(ctypes.byref(cfg), ctypes.byref(t), 1, ws, WS, None) == -3
    t.step = 1
    assert lib.lv_step_multi(ctypes.byref(cfg), ctypes.byref(t), 1, ws, 8, None) == -3
    t.grad = t.param
    assert lib.lv_step_multi(ctypes.byref(cfg), ctypes.byref(t), 1, ws, WS, None) == -3
    # inactive ranges: a count without a table
    t.grad = 0x3000
    t.n_inactive = 2
    assert lib.lv_step_multi(ctypes.byref(cfg), ctypes.byref(t), 1, ws, WS, None) == -1
    assert b"inactive" in lib.lv_last_error()
    t.n_inactive = 0
    t.grad = t.param
    # more than 48 tensors need the table-launch regions of the workspace
    many = (H.LvTensor * 49)()
    for k in range(49):
        many[k].numel, many[k].step = 10, 1
        many[k].param, many[k].grad, many[k].exp_avg, many[k].exp_avg_sq, many[k].scratch = (
            0x1000, 0x3000, 0x2000, 0x2400, 0x2800)
    assert lib.lv_step_multi(ctypes.byref(cfg), many, 49, ws, WS, None) == -3
    assert b"workspace too small" in lib.lv_last_error()
    # radial: same host checks (the call is never launched here)
    rcfg = _cfg(buffer="T2", bound_type="radial")
    assert lib.lv_step_multi(ctypes.byref(rcfg), ctypes.byref(t), 1, ws, WS, None) == -3
    assert b"aliases" in lib.lv_last_error()


def test_xcd_block_mapping_is_exact_and_bijective():
    """Unit launches send block b to XCD x = b mod X and give each XCD one contiguous range of
    units: unit = x * (G div X) + min(x, G mod X) + b div X. The kernel takes b div X as
    (b * (floor(2^40 / X) + 1)) >> 40 (no integer division in the block prologue): exact for every
    b below the 2^23-block launch cap and X <= 64, and the mapping is a permutation of the grid."""
    import numpy as np

    b = np.arange(1 << 23, dtype=np.uint64)
    for X in range(1, 65):
        recip = np.uint64((1 << 40) // X + 1)
        assert np.array_equal((b * recip) >> np.uint64(40), b // np.uint64(X)), X
    for X in (1, 3, 8, 12):
        for G in list(range(1, 40)) + [1023, 6_580_484]:
            bb = np.arange(G, dtype=np.int64)
            i = (bb.astype(np.uint64) * np.uint64((1 << 40) // X + 1)) >> np.uint64(40)
            x = bb - i.astype(np.int64) * X
            q, r = G // X, G % X
            unit = x * q + np.minimum(x, r) + i.astype(np.int64)
            assert np.array_equal(np.sort(unit), bb), (X, G)
