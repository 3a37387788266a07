"""Builds libluminav_hip.so for gfx950 with hipcc (in-tree, into luminamoon_amd/_lib/).

Five objects compiled in parallel and linked into one shared library: the host side and C ABI
(csrc/luminav_hip.hip) and the kernels of each buffer mode (csrc/lv_kernels.hip with
-DLV_MODE=1..4).

Flags that the bitwise-parity contract depends on:
  -ffp-contract=off                          no fused multiply-add except the explicit fmaf calls
  -fhip-fp32-correctly-rounded-divide-sqrt   IEEE division and square root
  -fno-gpu-flush-denormals-to-zero           f32 denormals preserved, as on the CPU
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed-FP32 instructions

And one for speed: -mllvm -amdgpu-atomic-optimizer-strategy=None. A block reports its count with
one atomic from one lane; the optimizer would add a wave reduction around it and a broadcast of
its result (cfg2's 64-tensor table launch: 16.60 against 16.86 us per launch, in one process).
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
HOST_SRC = os.path.join(CSRC, "luminav_hip.hip")
KERNEL_SRC = os.path.join(CSRC, "lv_kernels.hip")
SRC = HOST_SRC
OUT_DIR = os.path.join(HERE, "_lib")
OUT = os.path.join(OUT_DIR, "libluminav_hip.so")
HOST_PTRS_SRC = os.path.join(CSRC, "host_ptrs.cpp")
HOST_PTRS_OUT = os.path.join(OUT_DIR, "_lv_host.so")
ARCH = os.environ.get("LUMINAV_OFFLOAD_ARCH", "gfx950")
MODES = (1, 2, 3, 4)  # LV_BUFFER_TDCLM, _DUAL, _T1, _T2

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wall",
]
COMPILE_FLAGS = [f for f in HIPCC_FLAGS if f != "-shared"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    return "hipcc"


def _run(cmd, what, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed building {what}")


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    jobs = [([hipcc(), *COMPILE_FLAGS, *inc, "-c", HOST_SRC, "-o", os.path.join(OUT_DIR, "host.o")], HOST_SRC)]
    for m in MODES:
        jobs.append(([hipcc(), *COMPILE_FLAGS, *inc, f"-DLV_MODE={m}", "-c", KERNEL_SRC,
                      "-o", os.path.join(OUT_DIR, f"kernels_{m}.o")], f"{KERNEL_SRC} (mode {m})"))
    with ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        for f in [ex.submit(_run, cmd, what, verbose) for cmd, what in jobs]:
            f.result()
    tmp = OUT + ".tmp"
    objs = [os.path.join(OUT_DIR, "host.o")] + [os.path.join(OUT_DIR, f"kernels_{m}.o") for m in MODES]
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp], OUT, verbose)
    os.replace(tmp, OUT)
    for o in objs:
        os.remove(o)
    return OUT


def build_host(verbose: bool = False) -> str:
    """Builds _lv_host.so (csrc/host_ptrs.cpp: the step plans' data-pointer checks, CPU code against
    libtorch's Python API) with torch.utils.cpp_extension, into _lib/."""
    import shutil
    import tempfile

    from torch.utils import cpp_extension

    os.makedirs(OUT_DIR, exist_ok=True)
    with tempfile.TemporaryDirectory() as tmp:
        cpp_extension.load(name="_lv_host", sources=[HOST_PTRS_SRC], build_directory=tmp, extra_cflags=["-O2"],
                           verbose=verbose, is_python_module=False)
        tmp_out = HOST_PTRS_OUT + ".tmp"
        shutil.copyfile(os.path.join(tmp, "_lv_host.so"), tmp_out)
        os.replace(tmp_out, HOST_PTRS_OUT)
    return HOST_PTRS_OUT


if __name__ == "__main__":
    print(build(verbose=True))
    print(build_host(verbose=True))
