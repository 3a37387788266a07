"""The reference's standalone C header against this library (CPU only).

A C program that includes the reference's own `optimizer/include/luminav_triton_standalone.h`
(where it lies under the reference checkout; the test is skipped without it) and this build's
`include/luminav_hip.h` in one translation unit compiles with -Wall -Wextra -Werror: the two
headers declare `luminav_triton_engine_create/destroy/get_platform/get_arch` and
`luminav_triton_step_f32` with the same prototypes and the same engine type (a conflicting
declaration is a compile error), and static assertions tie the reference's status, buffer and
bound codes to this build's. The program then links against libluminav_hip.so and runs: without
a GPU, engine creation returns NULL, the accessors answer "none" (platform) and "unknown" (arch)
for it and a step on it returns the reference's null-pointer status.
"""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
REF_INCLUDE = "/root/reference/optimizer/include"
REF_HEADER = os.path.join(REF_INCLUDE, "luminav_triton_standalone.h")

PROGRAM = r"""
#include <stdio.h>
#include <string.h>
#include "luminav_triton_standalone.h"  /* the reference's header, unchanged */
#include "luminav_hip.h"                /* this build's header: conflicting prototypes fail here */

_Static_assert(LV_STATUS_SUCCESS == LUMINAV_STATUS_SUCCESS, "status");
_Static_assert(LV_STATUS_NULL_POINTER == LUMINAV_STATUS_NULL_POINTER, "status");
_Static_assert(LV_STATUS_NO_DRIVER == LUMINAV_STATUS_NO_DRIVER, "status");
_Static_assert(LV_STATUS_INVALID_CONFIG == LUMINAV_STATUS_INVALID_CONFIG, "status");
_Static_assert(LV_STATUS_EXECUTION_FAILED == LUMINAV_STATUS_EXECUTION_FAILED, "status");
_Static_assert(LV_BUFFER_TDCLM == LUMINAV_BUFFER_TDCLM && LV_BUFFER_DUAL == LUMINAV_BUFFER_DUAL, "buffer");
_Static_assert(LV_BOUND_NONE == LUMINAV_BOUND_NONE && LV_BOUND_RADIAL == LUMINAV_BOUND_RADIAL &&
               LV_BOUND_COORDINATE == LUMINAV_BOUND_COORDINATE, "bound");

int main(void) {
    float p[4] = {0}, g[4] = {0}, m[4] = {0}, v[4] = {0}, sc[6] = {0, 0, 0, 1, 1, 0};
    LuminaVTritonEngine *e = luminav_triton_engine_create();
    if (e) {  /* a GPU is present: the engine works like any other caller's */
        printf("engine %s %s\n", luminav_triton_get_platform(e), luminav_triton_get_arch(e));
        int rc = luminav_triton_step_f32(e, p, g, m, v, NULL, sc, 4, 1e-3f, 0.9f, 0.999f, 1e-8f, 0.01f,
                                         0.8f, 0.3f, LUMINAV_BUFFER_DUAL, 1, LUMINAV_BOUND_COORDINATE,
                                         0.05f, 1, 1337u);
        luminav_triton_engine_destroy(e);
        return rc == LUMINAV_STATUS_SUCCESS ? 0 : 1;
    }
    if (strcmp(luminav_triton_get_platform(NULL), "none") != 0) return 2;  /* the reference's tags: cuda, rocm, none */
    if (strcmp(luminav_triton_get_arch(NULL), "unknown") != 0) return 3;
    int rc = luminav_triton_step_f32(NULL, p, g, m, v, NULL, sc, 4, 1e-3f, 0.9f, 0.999f, 1e-8f, 0.01f,
                                     0.8f, 0.3f, LUMINAV_BUFFER_DUAL, 1, LUMINAV_BOUND_COORDINATE,
                                     0.05f, 1, 1337u);
    if (rc != LUMINAV_STATUS_NULL_POINTER) return 4;
    luminav_triton_engine_destroy(NULL);
    printf("no engine\n");
    return 0;
}
"""


def test_reference_standalone_header_compiles_links_and_runs(tmp_path):
    if not os.path.exists(REF_HEADER):
        pytest.skip("the reference checkout is not present")
    from luminamoon_amd.optimizer import hip_backend

    lib = hip_backend.LIB_PATH
    if not os.path.exists(lib):
        pytest.skip("libluminav_hip.so is not built")
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = tmp_path / "app.c"
    src.write_text(PROGRAM)
    exe = tmp_path / "app"
    libdir = os.path.dirname(lib)
    cmd = [cc, "-std=c11", "-Wall", "-Wextra", "-Werror", "-I", REF_INCLUDE, "-I", os.path.join(ROOT, "include"),
           str(src), "-L", libdir, "-lluminav_hip", f"-Wl,-rpath,{libdir}", "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, (run.returncode, run.stdout, run.stderr)
    assert "no engine" in run.stdout or "engine rocm" in run.stdout
