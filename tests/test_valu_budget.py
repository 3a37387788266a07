"""VALU budget of the unit kernels' hot path, from this build's gfx950 assembly (CPU only).

`tests/gpu_checks/valu_budget.hip` instantiates the unit kernel of each bench workload; hipcc
compiles it to assembly with the library's own flags. The hot path of a kernel is its vector
path over a whole unit (from the `s_setprio` that follows the unit's loads to the block
reduction's `s_barrier`) with every wave-uniform guard on its fast side: the cheapest path
through the control-flow graph, where a guard's slow side is a detour that adds work and an
exec-mask skip (`s_cbranch_execz`) is never taken (some lanes run its body). The path's VALU
instructions per element (4 * H * S per lane: S sub-units of 4 * H elements each) are what
`SQ_INSTS_VALU` per wave counts per element, less the unit's prologue and reduction.

Each kernel's cost must stay within its budget, in issue units: every VALU instruction priced
by its measured issue time on gfx950 (a v_add_u32 is one unit; most 3-operand and bit ops about
1.6; rcp and sqrt about 3), so the costliest classes weigh what they cost. The test fails when a
change adds VALU work to the hot path (a mask carried through a VGPR, a re-created constant, a
slow path laid inline and taken). `python -m pytest tests/test_valu_budget.py -s` prints each
kernel's cost and histogram.
"""
from __future__ import annotations

import collections
import heapq
import os
import re
import shutil
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "gpu_checks", "valu_budget.hip")

# Issue cost of a wave instruction on gfx950, in units of one v_add_u32 (measured 2026-12-02 with
# 8 independent chains per lane, 8 waves per SIMD): the 2-operand f32 add/mul/fma, u32 add/sub,
# and/or/xor, right shifts and moves take about 1; 3-operand integer and bit ops, min/max/med3,
# lshlrev, perm, SDWA forms, conversions, 24/32-bit integer multiplies and the division steps
# (div_scale, div_fmas, div_fixup) about 1.6; rcp, sqrt and rsq about 3.05; a compare and the
# select that reads it about 2.3 for the pair (1.16 each here).
ISSUE_ONE = {
    "v_add_u32", "v_sub_u32", "v_subrev_u32", "v_and_b32", "v_or_b32", "v_xor_b32", "v_not_b32", "v_lshrrev_b32",
    "v_ashrrev_i32", "v_mov_b32", "v_add_f32", "v_sub_f32", "v_subrev_f32", "v_mul_f32", "v_fma_f32", "v_fmac_f32",
    "v_fmaak_f32", "v_fmamk_f32",
}
ISSUE_THREE = {"v_rcp_f32", "v_sqrt_f32", "v_rsq_f32", "v_cvt_sr_bf16_f32", "v_cvt_sr_f16_f32"}


def issue_units(op: str) -> float:
    """Issue cost of one wave instruction, in v_add_u32 units (the table above)."""
    if "_sdwa" in op or "_dpp" in op:
        return 1.55
    base = op.replace("_e32", "").replace("_e64", "")
    if base in ISSUE_ONE:
        return 1.0
    if base in ISSUE_THREE:
        return 3.05
    if base.startswith(("v_cmp", "v_cndmask")):
        return 1.16
    return 1.6


# workload -> (mangled unit_kernel<mode, param dtype, state dtype, pass, flags, table>, elements
# per lane, budget in issue units per element, anchors). A budget is this build's cost rounded up
# to the next multiple of 0.5. The anchors are the per-element counts of the instructions the
# reference's arithmetic needs on the path: every division has one v_rcp_f32 (the IEEE sequence,
# which also ends in one v_div_fixup_f32, or in the 16-bit-state kernels its unscaled form under a
# wave-uniform range test, with no fixup on the hot path), a correctly rounded root one
# v_rsq_f32 (its one-correction form), a hashed (stochastically rounded) stream two v_mul_lo_u32,
# and a stored fp16 value
# half a v_cvt_pkrtz_f16_f32 (two per pack). A walk that skipped real work (a branch the code
# never takes) would miss one of them. Stochastic rounding to bf16 or fp16 is one integer add on
# the path (the v_cvt_sr_bf16_f32 / v_cvt_sr_f16_f32 converters take about 3 times its issue
# time on gfx950), so they are anchored at zero.
#   T2: clm / env, the coordinate bound's quotient; sqrt(v). T1: the same without v.
#   CLM: clm / sigma, the bound's step / b, two tanh quotients; sqrt(v), sqrt(p^2 + 1e-4).
#   TD-CLM: clm / env, step / b, one tanh quotient; sqrt(p^2 + 1e-4).
#   fp16 params add the fp16 safety bound's quotient.
IEEE2 = {"v_rcp_f32": 2, "v_div_fixup_f32": 2}
FAST2 = {"v_rcp_f32": 2, "v_div_fixup_f32": 0}
KERNELS = {
    "cfg5 T2 bf16, f32 m/v": ("_ZN2lv11unit_kernelILi4ELi1ELi0ELi1ELj331ELb0EEEvNS_4ArgsE", 4, 91.5,
                              {**IEEE2, "v_rsq_f32": 1, "v_mul_lo_u32": 2, "v_cvt_sr_bf16_f32": 0}),
    "cfg5 T2 bf16, bf16 m/v": ("_ZN2lv11unit_kernelILi4ELi1ELi1ELi1ELj331ELb0EEEvNS_4ArgsE", 8, 98.5,
                               {**FAST2, "v_rsq_f32": 1, "v_mul_lo_u32": 6, "v_cvt_sr_bf16_f32": 0}),
    "cfg4 T1 bf16, f32 m": ("_ZN2lv11unit_kernelILi3ELi1ELi0ELi1ELj331ELb0EEEvNS_4ArgsE", 4, 74.5,
                            {**IEEE2, "v_mul_lo_u32": 2, "v_cvt_sr_bf16_f32": 0}),
    "cfg4 T1 bf16, bf16 m": ("_ZN2lv11unit_kernelILi3ELi1ELi1ELi1ELj331ELb0EEEvNS_4ArgsE", 16, 72.0,
                             {**FAST2, "v_mul_lo_u32": 4, "v_cvt_sr_bf16_f32": 0}),
    "cfg4 T1 fp16, fp16-container m": ("_ZN2lv11unit_kernelILi3ELi2ELi1ELi1ELj603ELb0EEEvNS_4ArgsE", 16, 95.0,
                                       {"v_rcp_f32": 3, "v_div_fixup_f32": 0, "v_mul_lo_u32": 4,
                                        "v_cvt_sr_bf16_f32": 0, "v_cvt_sr_f16_f32": 0, "v_cvt_pkrtz_f16_f32": 0.5}),
    "cfg3 CLM f32": ("_ZN2lv11unit_kernelILi2ELi0ELi0ELi1ELj75ELb0EEEvNS_4ArgsE", 4, 142.5,
                     {"v_rcp_f32": 4, "v_div_fixup_f32": 4, "v_rsq_f32": 2, "v_mul_lo_u32": 0}),
    "cfg2 TD-CLM f32, table": ("_ZN2lv11unit_kernelILi1ELi0ELi0ELi1ELj75ELb1EEEvNS_4ArgsE", 4, 96.5,
                               {"v_rcp_f32": 3, "v_div_fixup_f32": 3, "v_rsq_f32": 1, "v_mul_lo_u32": 0}),
}

CATEGORIES = [
    ("IEEE division steps", r"v_div_scale|v_rcp_f32|v_div_fmas|v_div_fixup"),
    ("root (v_rsq_f32 or v_sqrt_f32)", r"v_rsq_f32|v_sqrt_f32"),
    ("hash multiply", r"v_mul_lo_u32"),
    ("conversion (SR, f16)", r"v_cvt_"),
    ("compare", r"v_cmp"),
    ("select", r"v_cndmask"),
    ("move", r"v_mov_b32"),
    ("byte permute (16-bit pack)", r"v_perm_b32"),
    ("bitwise / shift", r"v_(xor|and|or|ashr|lshr|lshl|bfe|bfi|alignbit|bitop3)"),
    ("integer add", r"v_(add|sub)_u32|v_(add|sub)_co|v_addc"),
    ("f32 fma / mul / add / min / max", r"v_(fma|fmac|fmaak|fmamk|mul|add|sub|subrev|min|max|min3|max3|med3)_f32"),
]


def _compile(tmp: str) -> str:
    from luminamoon_amd import build_ext

    out = os.path.join(tmp, "valu_budget.s")
    flags = [f for f in build_ext.COMPILE_FLAGS if f != "-fPIC"]
    cmd = [build_ext.hipcc(), *flags, "--cuda-device-only", "-S", "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(ROOT, "luminamoon_amd", "csrc"), SRC, "-o", out]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(res.stdout + res.stderr)
    return out


_BRANCH = ("s_cbranch", "s_branch", "s_endpgm", "s_setpc")


def _blocks(lines: list[str], name: str):
    """The kernel's basic blocks in layout order: [(label or None, [instruction, ...]), ...]. A
    block ends at a label or after a branch (the compiler leaves fall-through blocks unlabelled)."""
    i = next(k for k, l in enumerate(lines) if l.startswith(name + ":"))
    j = next(k for k in range(i, len(lines)) if lines[k].startswith(".Lfunc_end"))
    blocks, label, ins = [], "entry", []
    for l in lines[i + 1:j]:
        m = re.match(r"^(\.LBB\d+_\d+):", l)
        if m:
            if ins or label is not None:
                blocks.append((label, ins))
            label, ins = m.group(1), []
            continue
        t = l.split(";")[0].strip()
        if l.startswith("\t") and t and not t.startswith("."):
            ins.append(t)
            if t.startswith(_BRANCH):
                blocks.append((label, ins))
                label, ins = None, []
    if ins or label is not None:
        blocks.append((label, ins))
    return blocks


def _dest(ins: str) -> str | None:
    """The scalar register an instruction writes, if its first operand is one (SALU results,
    v_cmp_*_e64 masks, saveexec copies)."""
    parts = ins.replace(",", " ").split()
    if len(parts) < 2:
        return None
    d = parts[1]
    return d if re.match(r"^(s\[\d+:\d+\]|s\d+|vcc)$", d) else None


def _overlaps(a: str, b: str) -> bool:
    def regs(r):
        if r == "vcc":
            return {"vcc"}
        m = re.match(r"^s\[(\d+):(\d+)\]$", r)
        if m:
            return {f"s{i}" for i in range(int(m.group(1)), int(m.group(2)) + 1)}
        return {r}
    return bool(regs(a) & regs(b))


def _step(ins: list[str], flags: dict) -> dict:
    """Known constant 64-bit flags (s_mov_b64 sX, -1 or 0) after a block's instructions."""
    flags = dict(flags)
    for x in ins:
        d = _dest(x)
        if d is None:
            continue
        for r in [r for r in flags if _overlaps(r, d)]:
            del flags[r]
        m = re.match(r"^s_mov_b64 (s\[\d+:\d+\]), (-1|0)$", x)
        if m:
            flags[m.group(1)] = int(m.group(2))
    return flags


def _successors(blocks, k, flags):
    """Successors of block k on a path the hot path may take. An exec-masked body is entered by
    some lanes, so it is always on the path: `s_cbranch_execz` (skip the body) falls through and
    `s_cbranch_execnz` (enter the body placed elsewhere) is taken. A branch on vcc = exec & sX,
    with sX a flag the path set to a constant (the compiler's structurizer), goes the one way that
    constant allows (exec is not zero on the hot path)."""
    index = {lab: n for n, (lab, _) in enumerate(blocks) if lab is not None}
    ins = blocks[k][1]
    last = ins[-1] if ins else ""
    if not last.startswith(_BRANCH):
        return [k + 1] if k + 1 < len(blocks) else []
    if last.startswith(("s_endpgm", "s_setpc")):
        return []
    op, target = last.split()[0], last.split()[1]
    if op == "s_branch":
        return [index[target]]
    if op == "s_cbranch_execz":
        return [k + 1]
    if op == "s_cbranch_execnz":
        return [index[target]]
    if op in ("s_cbranch_vccz", "s_cbranch_vccnz") and len(ins) >= 2:
        m = re.match(r"^s_and(n2)?_b64 vcc, exec, (s\[\d+:\d+\])$", ins[-2])
        if m and m.group(2) in flags:
            vcc_set = (flags[m.group(2)] == -1) != bool(m.group(1))
            taken = vcc_set if op == "s_cbranch_vccnz" else not vcc_set
            return [index[target]] if taken else [k + 1]
    return [index[target], k + 1]


def hot_path(path: str, name: str) -> list[str]:
    """Instructions of the cheapest path (in VALU instructions) from the block holding
    `s_setprio` (1, or 0 in the two-sub-unit kernels) to the first block holding `s_barrier`, or,
    in a kernel of one-wave blocks (no barrier), the first holding the count report's atomic."""
    lines = open(path).read().split("\n")
    blocks = _blocks(lines, name)
    marker = ("s_barrier" if any(x.startswith("s_barrier") for _, ins in blocks for x in ins)
              else "global_atomic_add_x2")
    start = next(n for n, (_, ins) in enumerate(blocks) if any(x.startswith("s_setprio") for x in ins))
    cost = [sum(1 for x in ins if x.startswith("v_")) for _, ins in blocks]
    # Dijkstra over (block, known flags)
    s0 = (start, ())
    dist, prev, done = {s0: cost[start]}, {s0: None}, set()
    heap, tick, end = [(cost[start], 0, s0)], 1, None
    while heap:
        c, _, st = heapq.heappop(heap)
        if st in done:
            continue
        done.add(st)
        n, fl = st
        if n != start and any(x.startswith(marker) for x in blocks[n][1]):
            end = st
            break
        flags = _step(blocks[n][1], dict(fl))
        for s in _successors(blocks, n, flags):
            nxt = (s, tuple(sorted(flags.items())))
            if nxt not in done and c + cost[s] < dist.get(nxt, float("inf")):
                dist[nxt], prev[nxt] = c + cost[s], st
                heapq.heappush(heap, (c + cost[s], tick, nxt))
                tick += 1
    assert end is not None, f"{name}: no path from the vector path to the block reduction"
    order, st = [], end
    while st is not None:
        order.append(st[0])
        st = prev[st]
    out = []
    for n in reversed(order):
        ins = blocks[n][1]
        if n == start:
            ins = ins[next(i for i, x in enumerate(ins) if x.startswith("s_setprio")):]
        if n == end[0]:
            ins = ins[:next(i for i, x in enumerate(ins) if x.startswith(marker))]
        out.extend(ins)
    return out


def histogram(ins: list[str]) -> collections.Counter:
    c = collections.Counter()
    for x in ins:
        if not x.startswith("v_"):
            continue
        op = x.split()[0]
        for cat, rx in CATEGORIES:
            if re.match(rx, op):
                c[cat] += 1
                break
        else:
            c["other: " + op] += 1
    return c


@pytest.fixture(scope="module")
def asm():
    from luminamoon_amd import build_ext

    if shutil.which(build_ext.hipcc()) is None and not os.path.exists(build_ext.hipcc()):
        pytest.skip("hipcc not found")
    with tempfile.TemporaryDirectory() as tmp:
        yield _compile(tmp)


def test_hot_path_valu_within_budget(asm):
    rows, missing = [], []
    for what, (name, epl, budget, anchors) in KERNELS.items():
        ins = hot_path(asm, name)
        h = histogram(ins)
        count = sum(h.values()) / epl
        per = sum(issue_units(x.split()[0]) for x in ins if x.startswith("v_")) / epl
        rows.append((what, per, budget))
        print(f"\n{what}: {per:.1f} issue units per element (budget {budget}), {count:.1f} VALU instructions")
        for cat, n in h.most_common():
            print(f"    {cat:34s} {n / epl:6.2f}")
        ops = collections.Counter(x.split()[0].replace("_e32", "").replace("_e64", "") for x in ins)
        for op, want in anchors.items():
            if ops[op] != want * epl:
                missing.append((what, op, ops[op] / epl, want))
    assert not missing, f"hot path does not hold the reference's operations (walk or build changed): {missing}"
    over = [r for r in rows if r[1] > r[2]]
    assert not over, f"hot path over its issue budget: {over}"
