"""The oracle pins must reject plausible mistakes: each case compiles a copy of the oracle with
one deliberate slip (on the CPU, into a temporary directory) and runs tests/test_oracle_pins.py
against it; the pin suite has to fail."""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "oracle", "luminav_oracle.c")

MUTATIONS = {
    "prng_logical_shift": ("z = (uint32_t)(zi ^ (zi >> 16)) * (uint32_t)(-2048173461);",
                           "z = (uint32_t)(zi ^ (int32_t)((uint32_t)zi >> 16)) * (uint32_t)(-2048173461);"),
    "prng_murmur_constant": ("(uint32_t)(-2048173461)", "0x85EBCA6Bu"),
    "t2_env_drops_eps": ("float env0 = fmaf(k->b1sq, fabsf(m), k->eps);\n        float env1 = fmaf(k->omb1sq, fabsf(g), env0);\n        float env2",
                         "float env0 = fmaf(k->b1sq, fabsf(m), 0.0f);\n        float env1 = fmaf(k->omb1sq, fabsf(g), env0);\n        float env2"),
    "t2_defect_uses_new_m": ("float diff = rclamp(g - m, -1.0e18f, 1.0e18f);\n        v_new",
                             "float diff = rclamp(g - m_new, -1.0e18f, 1.0e18f);\n        v_new"),
    "clm_wrong_coefficient": ("float clm = fmaf(k->b1, m_new, k->omb1 * g);", "float clm = fmaf(k->b1, m_new, k->omb1sq * g);"),
    "sr_bf16_short_noise": ("int32_t noise = lvo_prng(seed, offset) & 0xFFFF;", "int32_t noise = lvo_prng(seed, offset) & 0x7FFF;"),
    "rne_bf16_no_tie_break": ("uint32_t rounded_abs = (abs_bits + 0x7FFFu + lsb) & 0xFFFF0000u;",
                              "uint32_t rounded_abs = (abs_bits + 0x8000u) & 0xFFFF0000u; (void)lsb;"),
    "bound_t2_drops_abs_step": ("float bb = b * (b + fabsf(step));\n    return (bb * step) / fmaf(step, step, bb);\n}\n\n/* math.rs:175-179 */",
                                "float bb = b * b;\n    return (bb * step) / fmaf(step, step, bb);\n}\n\n/* math.rs:175-179 */"),
    "bias_correction_off_by_one": ("1.0 - lvo_powi(b1, (int32_t)(safe + 1))", "1.0 - lvo_powi(b1, (int32_t)safe)"),
    "cautious_scale_no_clamp": ("float m_bar = rclamp(mask_sum / denom, clamp_min, 1.0f);", "float m_bar = mask_sum / denom; (void)clamp_min;"),
    "weight_decay_sign": ("fmaf(-k->lr_wd, p_init, p_init)", "fmaf(k->lr_wd, p_init, p_init)"),
    "sanitize_keeps_inf": ("if (isfinite(g) && fabsf(g) < 1.0e38f)", "if (!isnan(g))"),
    "radial_norm_ignores_cautious_mask": ("float u_eff = k->cautious ? u * (active ? 1.0f : 0.0f) : u;",
                                          "float u_eff = u; (void)active;"),
    "radial_norm_uses_updated_param": ("*p_sq_out = p_init * p_init;", "*p_sq_out = p_upd * p_upd;"),
    # v clamp keyed on the raw fp16 state container instead of the worker's promoted mode
    "v_clamp_on_fp16_state_container": ("p_mode, s_mode, threads,\n                   it->index_base);",
                                        "p_mode, it->state_dtype, threads,\n                   it->index_base);"),
    # the fp16 safety bound with the other mode's form, or with a different floor
    "fp16_safety_tanh_form_swapped": ("    float b = fmaxf(fabsf(p_init) * 0.01f, 1.5e-4f);\n    return b * lvo_tanh_pade(step / b);",
                                      "    float b = fmaxf(fabsf(p_init) * 0.01f, 1.5e-4f);\n    float bb = b * (b + fabsf(step));\n    return (bb * step) / fmaf(step, step, bb);"),
    "fp16_safety_floor_1e4": ("float lvo_fp16_safety_bound_t2(float step, float p_init) {\n    float b = fmaxf(fabsf(p_init) * 0.01f, 1.5e-4f);",
                              "float lvo_fp16_safety_bound_t2(float step, float p_init) {\n    float b = fmaxf(fabsf(p_init) * 0.01f, 1.0e-4f);"),
}


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_pins_reject_mutant(name, tmp_path):
    old, new = MUTATIONS[name]
    src = open(SRC).read()
    assert old in src, f"mutation anchor for {name} not found"
    mutant = tmp_path / "luminav_oracle.c"
    mutant.write_text(src.replace(old, new, 1))
    for other in ("luminav_oracle.h", "luminav_oracle_internal.h", "luminav_oracle_avx512.c"):
        (tmp_path / other).write_text(open(os.path.join(ROOT, "oracle", other)).read())
    lib = tmp_path / "libmutant.so"
    subprocess.run(["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-march=x86-64-v3", "-ffp-contract=off", "-fno-math-errno",
                    "-fopenmp", "-o", str(lib), str(mutant), str(tmp_path / "luminav_oracle_avx512.c"), "-lm"], check=True)
    env = dict(os.environ, LVO_LIB_OVERRIDE=str(lib))
    res = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                          os.path.join(ROOT, "tests", "test_oracle_pins.py")], cwd=ROOT, env=env,
                         capture_output=True, text=True, timeout=600)
    assert res.returncode != 0, f"pins did not catch mutation {name}:\n{res.stdout[-2000:]}"
