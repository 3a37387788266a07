"""Pins for the CPU oracle (oracle/luminav_oracle.c), one group per oracle function.

The reference ships no stored golden vectors for this path and its Rust oracle cannot be built
here (no cargo/rustc, crates.io dependencies), so each oracle function is checked against what
fixes it independently of its own formula:
  - the reference's own known-answer tests (optimizer/crates/luminav-core/tests/core_tests.rs);
  - the reference's independent NumPy restatement of the PRNG (python/luminamoon/optimizer/validation.py:73-77);
  - library routines that compute the same rounding (torch's float->bfloat16 RNE, NumPy's float16);
  - exact rational arithmetic (fractions) for the f64 bias-correction coefficients;
  - statistics (stochastic rounding is unbiased and picks one of the two neighbours);
  - an f64 re-evaluation of the whole update on small inputs, and invariants of the update
    (|u| < 1 for the triangle family, |bounded step| <= b, cautious masking, fused == unfused).
Each check is chosen so that a plausible slip (wrong constant, shift type, operand order,
missing term, wrong sign) fails it.
"""
from __future__ import annotations

import ctypes
import math
from fractions import Fraction

import numpy as np
import pytest
import torch

F = np.float32


def f2u(x: float) -> int:
    return int(np.array([x], dtype=np.float32).view(np.uint32)[0])


def u2f(u: int) -> float:
    return float(np.array([u & 0xFFFFFFFF], dtype=np.uint32).view(np.float32)[0])


# --------------------------------------------------------------------------- PRNG and seeds

def _prng_numpy_reference_style(seed: int, idx: np.ndarray) -> np.ndarray:
    """The reference's NumPy restatement (validation.py:73-77): int64 products masked to 32 bits."""
    z = (idx.astype(np.int64) + int(seed) - 1640531527).astype(np.int32)
    z = (((z ^ (z >> 16)).astype(np.int64) * -2048173461) & 0xFFFFFFFF).astype(np.int32)
    z = (((z ^ (z >> 13)).astype(np.int64) * -1028477387) & 0xFFFFFFFF).astype(np.int32)
    return (z ^ (z >> 16)).astype(np.int32)


def test_prng_closed_form_zero(oracle_mod):
    # core_tests.rs:24-28: _prng(0, 0) expands to a fixed integer.
    assert oracle_mod.lib().lvo_prng(0, 0) == 753291389


def test_prng_matches_reference_numpy_restatement(oracle_mod):
    L = oracle_mod.lib()
    rng = np.random.default_rng(1)
    seeds = rng.integers(0, 2 ** 31 - 1, 4000)
    idx = rng.integers(-(2 ** 31), 2 ** 31 - 1, 4000).astype(np.int32)
    for s, i in zip(seeds[:4000], idx):
        want = int(_prng_numpy_reference_style(int(s), np.array([i]))[0])
        assert L.lvo_prng(int(s), int(i)) == want


def test_prng_is_not_textbook_murmur_fmix32(oracle_mod):
    """The first multiplier is -2048173461 (0x85EB5A6B), not fmix32's 0x85EBCA6B: an oracle that
    assumed MurmurHash3 would fail here."""
    def fmix(seed, idx):
        z = (idx + seed + 0x9E3779B9) & 0xFFFFFFFF
        z = ((z ^ (z >> 16)) * 0x85EBCA6B) & 0xFFFFFFFF
        z = ((z ^ (z >> 13)) * 0xC2B2AE35) & 0xFFFFFFFF
        z ^= z >> 16
        return z - (1 << 32) if z >= 1 << 31 else z
    L = oracle_mod.lib()
    diffs = sum(L.lvo_prng(s, i) != fmix(s, i) for s, i in [(1337, k) for k in range(200)])
    assert diffs > 150


def test_seed_derivation_known_answers(oracle_mod):
    L = oracle_mod.lib()
    sm, sp = ctypes.c_int32(), ctypes.c_int32()
    L.lvo_derive_kernel_seeds(1337, 1, 0, ctypes.byref(sm), ctypes.byref(sp))
    # core_tests.rs:31-37
    assert sm.value == (1337 + 0x9E3779B9) & 0x7FFFFFFF
    assert sp.value == (sm.value + 0x55555555) & 0x7FFFFFFF
    assert L.lvo_derive_variance_seed(sm.value) not in (sm.value, sp.value)
    # u128 wrapping arithmetic (prng.rs:4-13) with Python big integers, large step/param_index
    for seed, step, pidx in [(0, 2 ** 63 + 12345, 2 ** 40 + 7), (4294967295, 2 ** 64 - 1, 2 ** 64 - 1), (7, 3, 99)]:
        raw = (seed + step * 0x9E3779B9 + pidx * 10007) % (1 << 128)
        want_m = raw & 0x7FFFFFFF
        L.lvo_derive_kernel_seeds(seed, step, pidx, ctypes.byref(sm), ctypes.byref(sp))
        assert sm.value == want_m
        assert sp.value == (want_m + 0x55555555) & 0x7FFFFFFF
        assert L.lvo_derive_variance_seed(want_m) == (want_m + 0x2A6D365B) & 0x7FFFFFFF


# --------------------------------------------------------------------------- rounding

def test_rne_bf16_matches_torch(oracle_mod):
    L = oracle_mod.lib()
    rng = np.random.default_rng(2)
    xs = np.concatenate([rng.standard_normal(3000) * 10.0 ** rng.integers(-40, 38, 3000),
                         [0.0, -0.0, 1.0, -1.0, 1e-45, -1e-45, 3.0e38]]).astype(np.float32)
    # exact ties (low 16 bits == 0x8000) with even and odd kept LSB: round half to even
    hi = rng.integers(0x0080, 0x7F7F, 200).astype(np.uint32)
    ties = ((hi << 16) | 0x8000).view(np.float32)
    xs = np.concatenate([xs, ties, -ties])
    want = torch.from_numpy(xs).to(torch.bfloat16).float().numpy()
    got = np.array([L.lvo_rne_bf16(float(x)) for x in xs], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_rne_bf16_overflow_clamps_and_nan(oracle_mod):
    L = oracle_mod.lib()
    # prng.rs:162-178: rounding past the largest bf16 clamps to it instead of +inf
    assert f2u(L.lvo_rne_bf16(u2f(0x7F7FFFFF))) == 0x7F7F0000
    assert f2u(L.lvo_rne_bf16(float("inf"))) == 0x7F7F0000
    assert f2u(L.lvo_rne_bf16(float("-inf"))) == 0xFF7F0000
    assert math.isnan(L.lvo_rne_bf16(float("nan")))


def test_sr_bf16_neighbours_unbiased_and_known_answers(oracle_mod):
    L = oracle_mod.lib()
    val = 1.000123
    for idx in range(64):  # core_tests.rs:41-50
        r = L.lvo_sr_bf16(val, 1337, idx)
        assert f2u(r) & 0xFFFF == 0 and abs(r - val) < 1e-2
    rng = np.random.default_rng(3)
    for x in rng.standard_normal(40) * 10.0 ** rng.integers(-20, 20, 40):
        x = float(np.float32(x))
        lo = u2f(f2u(x) & 0xFFFF0000)
        hi = u2f((f2u(x) & 0xFFFF0000) + 0x10000)
        outs = np.array([L.lvo_sr_bf16(x, 99, i) for i in range(4000)])
        assert set(np.unique(outs)).issubset({lo, hi})
        frac = (abs(x) - abs(lo)) / (abs(hi) - abs(lo))
        p_up = np.mean(outs == hi)
        assert abs(p_up - frac) < 0.04, (x, p_up, frac)
    assert math.isnan(L.lvo_sr_bf16(float("nan"), 1, 2))


def test_fp16_rne_matches_numpy(oracle_mod):
    L = oracle_mod.lib()
    rng = np.random.default_rng(4)
    xs = np.concatenate([rng.standard_normal(4000) * 10.0 ** rng.integers(-9, 5, 4000),
                         [0.0, -0.0, 65504.0, -65504.0, 6e-8, 2.98e-8, 5.96e-8, 1e-9]]).astype(np.float32)
    xs = xs[np.abs(xs) <= 65504.0]
    want = xs.astype(np.float16).view(np.uint16)
    got = np.array([L.lvo_f32_to_f16_bits_rne(float(x)) for x in xs], dtype=np.uint16)
    assert np.array_equal(got, want)
    # overflow saturates to the largest finite value (prng.rs:41-58); NaN -> quiet NaN
    assert L.lvo_f32_to_f16_bits_rne(1e6) == 0x7BFF
    assert L.lvo_f32_to_f16_bits_rne(float("inf")) == 0x7BFF
    assert L.lvo_f32_to_f16_bits_rne(float("nan")) == 0x7E00


def test_fp16_decode_matches_numpy_for_every_pattern(oracle_mod):
    L = oracle_mod.lib()
    pats = np.arange(65536, dtype=np.uint16)
    want = pats.view(np.float16).astype(np.float32)
    got = np.array([L.lvo_f16_bits_to_f32(int(b)) for b in pats], dtype=np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))
    assert np.array_equal(np.isinf(got), np.isinf(want))


def test_sr_fp16_neighbours_and_subnormal_flush(oracle_mod):
    L = oracle_mod.lib()
    for idx in range(64):  # core_tests.rs:41-55
        r = L.lvo_sr_fp16(1.000123, 1337, idx)
        assert abs(r - 1.000123) < 2e-3
    tiny = u2f(102 << 23)
    assert f2u(L.lvo_sr_fp16(tiny, 1337, 0)) == 0
    assert f2u(L.lvo_sr_fp16(-tiny, 1337, 0)) == 0x80000000
    rng = np.random.default_rng(5)
    for x in rng.standard_normal(30) * 10.0 ** rng.integers(-6, 4, 30):
        x32 = np.float32(x)
        h = np.float16(x32)
        cands = {float(np.nextafter(h, np.float16(-np.inf))), float(h), float(np.nextafter(h, np.float16(np.inf)))}
        outs = {L.lvo_sr_fp16(float(x32), 7, i) for i in range(300)}
        assert outs.issubset(cands), (x, outs, cands)


# --------------------------------------------------------------------------- math

def test_tanh_pade_accuracy_and_exact_points(oracle_mod):
    L = oracle_mod.lib()
    xs = np.arange(-10000, 10001) * np.float32(0.001)
    err = max(abs(L.lvo_tanh_pade(float(x)) - math.tanh(float(np.float32(x)))) for x in xs[::7])
    assert err <= 3e-7  # core_tests.rs:62-82
    assert L.lvo_tanh_pade(0.0) == 0.0
    assert L.lvo_tanh_pade(25.0) == 1.0 and L.lvo_tanh_pade(-25.0) == -1.0
    assert math.isnan(L.lvo_tanh_pade(float("nan")))


def test_sanitize_gradient(oracle_mod):
    L = oracle_mod.lib()
    assert L.lvo_sanitize_gradient(float("nan")) == 0.0
    assert L.lvo_sanitize_gradient(float("inf")) == 0.0
    assert L.lvo_sanitize_gradient(2e38) == 0.0
    assert L.lvo_sanitize_gradient(5e37) == float(np.float32(1e18))
    assert L.lvo_sanitize_gradient(-3e20) == float(np.float32(-1e18))
    assert L.lvo_sanitize_gradient(0.25) == 0.25


def _f32(x: Fraction) -> float:
    return float(np.float32(float(x)))


def test_bias_correction_against_exact_rationals(oracle_mod):
    L = oracle_mod.lib()
    out = (ctypes.c_float * 5)()
    L.lvo_bias_correction(1, 0.9, 0.999, 1e-8, 0.8, out)
    assert abs(out[0] - 0.19) < 1e-6  # core_tests.rs:155-157
    for step in (1, 2, 3, 10, 100, 1000, 12345):
        for b1, b2, eps, tau in ((0.9, 0.999, 1e-8, 0.8), (0.95, 0.98, 1e-6, 1.3)):
            L.lvo_bias_correction(step, b1, b2, eps, tau, out)
            B1, B2 = Fraction(float(np.float32(b1))), Fraction(float(np.float32(b2)))
            T, E = Fraction(float(np.float32(tau))), Fraction(float(np.float32(eps)))
            bc1 = 1 - B1 ** (step + 1)
            bc2 = max(1 - B2 ** step, Fraction(1, 10 ** 15))
            c1 = float(bc1 * T) / math.sqrt(float(bc2))
            c2 = bc1 * E * T
            for got, want in ((out[0], float(bc1)), (out[1], float(bc2)), (out[2], c1), (out[3], float(c2))):
                w = np.float32(want)
                assert abs(np.float32(got) - w) <= np.spacing(w), (step, got, want)
            # c_sigma = (0.5 lam) / sqrt(max(f32(bc2), 1e-15)) in f32
            lam = 0.3
            cs = L.lvo_t2_sigma_coeff(step, b2, lam)
            want = np.float32(np.float32(0.5) * np.float32(lam)) / np.float32(math.sqrt(np.float32(float(bc2))))
            assert abs(np.float32(cs) - want) <= 2 * np.spacing(want)


def test_powi_is_repeated_squaring(oracle_mod):
    """f64::powi lowers to compiler-builtins' repeated squaring; its relative error grows with
    the number of squarings (~2^bits(b) ulp), unlike a correctly rounded pow. Exact for powers
    of two and small integer bases."""
    L = oracle_mod.lib()
    for a in (0.9, 0.999, 0.999999, 1.0000001, 0.5):
        for b in (0, 1, 2, 3, 17, 1000, 123457, -3):
            got = L.lvo_powi(a, b)
            exact = float(Fraction(a) ** b)
            k = abs(b).bit_length()
            assert abs(got - exact) <= (k + 1) * 2.0 ** k * 2.3e-16 * abs(exact) + 1e-300, (a, b)
    assert L.lvo_powi(0.5, 40) == 2.0 ** -40
    assert L.lvo_powi(3.0, 20) == 3.0 ** 20


def test_cautious_scale_and_ema_known_answer(oracle_mod):
    O = oracle_mod
    L = O.lib()
    assert L.lvo_cautious_scale(50.0, 100.0, 0.5) == 2.0
    assert L.lvo_cautious_scale(90.0, 100.0, 0.5) == np.float32(1.0) / np.float32(0.9)
    assert L.lvo_cautious_scale(100.0, 100.0, 0.5) == 1.0
    assert L.lvo_cautious_scale(0.0, 0.0, 0.5) == 2.0  # denominator floors at 1
    # core_tests.rs:84-111: mask 50/100, decay 0.8, radial -> cautious 1.2, bound in (0, 1]
    s = (ctypes.c_float * 6)(50.0, 25.0, 100.0, 1.0, 1.0, 0.0)
    cfg = O.make_config(lr=1e-3, cautious_clamp_min=0.5, ema_decay=0.8, bound_type=1, bound_ratio=0.05)
    L.lvo_update_post_step_ema(s, 100.0, ctypes.byref(cfg), 0)
    assert abs(s[3] - 1.2) < 1e-6
    assert 0.0 < s[4] <= 1.0
    assert s[0] == s[1] == s[2] == 0.0


def _t1_radial_expectation(p, g, m, lr, lam, ratio, eps):
    """Closed form of the radial inputs for T1 (no bias correction, no v): u, the cautious mask
    u*g > 0, and the squared norms sum((u*mask)^2), sum(p^2), evaluated in float64 from the f32
    inputs and the f32-rounded coefficients (tdclm.rs:102-109, dual.rs:176-180)."""
    b1sq = np.float32(np.float32(0.9) * np.float32(0.9))
    omb1sq = np.float32(1.0) - b1sq
    p64, g64, m64 = (x.astype(np.float64) for x in (p, g, m))
    u = (float(b1sq) * m64 + float(omb1sq) * g64) / (
        float(b1sq) * np.abs(m64) + float(np.float32(eps)) + float(omb1sq) * np.abs(g64)
        + float(np.float32(lam)) * np.abs(g64 - m64))
    active = u * g64 > 0
    count = int(active.sum())
    return float(np.sum((u * active) ** 2)), float(np.sum(p64 ** 2)), count


def _t1_radial_target(u_sq, p_sq, cs, lr, ratio):
    r = lr * math.sqrt(u_sq) * cs / (ratio * max(math.sqrt(p_sq), 1.0))
    return (1.0 + r) / (1.0 + r + r * r)


@pytest.mark.parametrize("f64_sums", [False, True])
def test_radial_norms_two_pass_and_fused(oracle_mod, f64_sums):
    """The radial scale is built from sum((u*mask)^2) over the cautious mask and sum(p_init^2)
    (dual.rs:279-320 two-pass, dual.rs:176-190 fused + math.rs:188-239 EMA). Checked against the
    closed form from the inputs, with the initial m chosen so that about a third of the mask is off.
    The f64 sum mode must land within 1e-6; the scalar core's f32 lane order within its own
    first-order summation bound, (adds per lane) x 2^-24 (|d ln bs / d ln r| < 1, r ~ sqrt(U/P))."""
    O = oracle_mod
    n = 100_003
    rng = np.random.default_rng(21)
    p0 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    g[::33] = 0.0
    m0 = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    lr, lam, ratio, eps = 1e-2, 0.3, 0.05, 1e-8
    u_sq, p_sq, count = _t1_radial_expectation(p0, g, m0, lr, lam, ratio, eps)
    assert 0.55 * n < count < 0.8 * n  # the mask matters
    cfg = O.make_config(buffer="T1", lr=lr, lam=lam, bound_type=1, bound_ratio=ratio, eps=eps, ema_decay=0.8,
                        weight_decay=0.0)
    import contextlib

    ctx = O.radial_sum_f64() if f64_sums else contextlib.nullcontext()
    tol = 1e-6 if f64_sums else (n // 16 + 1) * 2.0 ** -24
    with ctx:
        # step 1: two passes, scale from this step's norms
        p, m, sc = p0.copy(), m0.copy(), np.array([0, 0, 0, 1, 1, 0], np.float32)
        O.step(cfg, [p], [g], [m], [None], [None], [sc], [1], [0])
        cs = 1.0 / min(max(count / n, 0.5), 1.0)
        want = _t1_radial_target(u_sq, p_sq, cs, lr, ratio)
        assert 0.05 < want < 0.95
        assert abs(sc[4] - want) <= tol * want, (sc[4], want)
        assert sc[3] == np.float32(cs) or abs(sc[3] - cs) <= 1e-6 * cs
        # step 2 from the same inputs: fused pass with lagged scales, EMA of both
        p, m, sc = p0.copy(), m0.copy(), np.array([0, 0, 0, 1.25, 0.8, 0], np.float32)
        O.step(cfg, [p], [g], [m], [None], [None], [sc], [2], [0])
        cs_new = 0.8 * 1.25 + 0.2 * cs
        want2 = 0.8 * 0.8 + 0.2 * _t1_radial_target(u_sq, p_sq, cs_new, lr, ratio)
        assert abs(sc[3] - cs_new) <= 1e-6 * cs_new
        assert abs(sc[4] - want2) <= tol * want2, (sc[4], want2)
        assert sc[0] == sc[1] == sc[2] == sc[5] == 0.0


def test_radial_sum_modes_agree_to_f32_summation_error(oracle_mod):
    """The f64 sum mode (what the HIP kernels compute) and the scalar core's f32 lane order give
    the same bound scale up to the f32 summation bound (131,072 sequential adds per lane in a
    2,097,152-element chunk, then the chunk fold: gamma = 131,074 x 2^-24 = 7.8e-3), on a tensor
    spanning two chunks; m and v never see the scale and stay bitwise equal."""
    O = oracle_mod
    n = 2097152 + 777_777
    rng = np.random.default_rng(22)
    p0 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    cfg = O.make_config(buffer="T2", lr=3e-3, bound_type=1)
    res = []
    for mode in (0, 1):
        O.lib().lvo_set_radial_sum_mode(mode)
        try:
            p, m, v = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
            sc = np.array([0, 0, 0, 1, 1, 0], np.float32)
            O.step(cfg, [p], [g], [m], [v], [None], [sc], [1], [0], threads=4)
            res.append((sc.copy(), p, m, v))
        finally:
            O.lib().lvo_set_radial_sum_mode(0)
    (s0, p_a, m_a, v_a), (s1, p_b, m_b, v_b) = res
    assert np.array_equal(m_a, m_b) and np.array_equal(v_a, v_b)  # the scale never feeds m, v
    gamma = (2097152 // 16 + 2) * 2.0 ** -24
    assert abs(s0[4] - s1[4]) <= gamma * s1[4] and s1[4] < 0.999
    assert np.max(np.abs(p_a - p_b)) <= 1.5e-6  # differential_parity.rs:16 TOLERANCE


def test_radial_scale_properties(oracle_mod):
    L = oracle_mod.lib()
    assert L.lvo_radial_scale(1e-12, 1.0, 1.0, 1e-3, 0.05) == 1.0  # r < 1e-4
    prev = 1.0
    for usq in (1e2, 1e4, 1e6, 1e8):
        sc = L.lvo_radial_scale(usq, 4.0, 1.0, 1e-3, 0.05)
        r = 1e-3 * math.sqrt(usq) / (0.05 * 2.0)
        assert abs(sc - math.tanh(r) / r) < 1e-5 and sc <= prev
        prev = sc
        sc2 = L.lvo_radial_scale_t2(usq, 4.0, 1.0, 1e-3, 0.05)
        assert abs(sc2 - (1 + r) / (r * r + 1 + r)) < 1e-5


def test_coordinate_bounds_are_bounded_and_tangent(oracle_mod):
    L = oracle_mod.lib()
    for p in (0.0, 0.02, -1.5, 30.0):
        b_t = 0.05 * math.sqrt(p * p + 1e-4)
        b_r = 0.05 * (abs(p) + 1e-2)
        for s in (1e-9, -1e-7, 3e-3, -0.2, 50.0):
            t = L.lvo_coordinate_bound(s, p, 0.05)
            r = L.lvo_coordinate_bound_t2(s, p, 0.05)
            assert abs(t) <= b_t * (1 + 1e-6) and abs(r) <= b_r * (1 + 1e-6)
            assert abs(t - b_t * math.tanh(s / b_t)) <= 2e-6 * b_t
            assert abs(r - b_r * (b_r + abs(s)) * s / (s * s + b_r * (b_r + abs(s)))) <= 2e-6 * b_r
            assert math.copysign(1, t) == math.copysign(1, s)
        small = 1e-7 * b_r
        assert abs(L.lvo_coordinate_bound_t2(small, p, 0.05) - small) <= 1e-6 * small
    for p in (0.0, 3.0):  # fp16 safety bound: b = max(|p| * 0.01, 1.5e-4)
        b = max(abs(p) * 0.01, 1.5e-4)
        for s in (1e-6, 0.3):
            assert abs(L.lvo_fp16_safety_bound(s, p)) <= b * (1 + 1e-6)
            assert abs(L.lvo_fp16_safety_bound_t2(s, p)) <= b * (1 + 1e-6)


def test_fp16_safety_bounds_closed_form_per_mode(oracle_mod):
    """apply_fp16_safety_bound{,_t2} (math.rs:175-186): b = max(|p| * 0.01, 1.5e-4), then the
    tanh form b * tanh(s / b) for TD-CLM/CLM and the rational form b(b+|s|) s / (s^2 + b(b+|s|))
    for the triangle family. At |s| = b the two forms differ by 12% (0.762 b vs 0.667 b), and a
    different floor or scale moves b, so swapped forms or a wrong b fail here."""
    L = oracle_mod.lib()
    for p in (0.0, 1e-3, -0.015, 0.02, 3.0, -250.0):
        b = max(abs(p) * 0.01, 1.5e-4)
        for s in (b * 1e-3, -0.5 * b, b, -2.0 * b, 7.5 * b, 1e3 * b):
            t = L.lvo_fp16_safety_bound(s, p)
            r = L.lvo_fp16_safety_bound_t2(s, p)
            bb = b * (b + abs(s))
            assert abs(t - b * math.tanh(s / b)) <= 2e-6 * b, (p, s, t)
            assert abs(r - bb * s / (s * s + bb)) <= 2e-6 * b, (p, s, r)
            assert math.copysign(1, t) == math.copysign(1, s) == math.copysign(1, r)
    # at |s| = b the tanh form is tanh(1) b and the rational one 2/3 b
    assert abs(L.lvo_fp16_safety_bound(1.5e-4, 0.0) - math.tanh(1.0) * 1.5e-4) <= 1e-10
    assert abs(L.lvo_fp16_safety_bound_t2(1.5e-4, 0.0) - 1.0e-4) <= 1e-10


@pytest.mark.parametrize("buffer", [2, "T2"])
def test_v_clamp_follows_the_param_dtype_only(oracle_mod, buffer):
    """The v <= 65000 clamp of the dual-state modes (dual.rs:68-71, dual.rs:160-163) tests
    view.dtype_mode == Float16 || view.state_dtype_mode == Float16. The FFI worker builds that view
    with eff_state_dtype_mode, which maps an fp16 state container to BFloat16 before the core runs
    (worker.rs:107-113 and the view at worker.rs:141-150), so on the reference's native path the
    clamp follows the param dtype alone: a bf16 (or fp32) param with an fp16 state container is
    not clamped, an fp16 param is."""
    O = oracle_mod
    n = 256
    cfg = O.make_config(lr=1e-3, buffer=buffer, cautious=False, stochastic_rounding=False)
    g = torch.full((n,), 1.0e4)  # d^2 = 1e8, so v_new = (1 - beta2) * 1e8 = 1e5 > 65000
    g[1::2] = -1.0e4
    for pdt, clamped in ((torch.bfloat16, False), (torch.float32, False), (torch.float16, True)):
        p = (torch.arange(n, dtype=torch.float32) * 1e-3).to(pdt)
        m = torch.zeros(n, dtype=torch.float16)  # fp16 containers holding bf16 bits
        v = torch.zeros(n, dtype=torch.float16)
        sc = torch.tensor([0, 0, 0, 1, 1, 0], dtype=torch.float32)
        O.step(cfg, [p], [g.to(pdt)], [m], [v], [None], [sc], [1], [0], dtypes=[(
            {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[pdt],) * 2 + (2,)])
        vv = v.view(torch.bfloat16).float()
        assert torch.isfinite(vv).all()
        # unclamped v_new in f32: d = g - m_new (CLM) or g - m (T2) with m = 0, v = (1 - b2) * d^2
        b1, omb2 = np.float32(0.9), np.float32(1.0) - np.float32(0.999)
        gf = np.float32(1.0e4)
        d = gf - (np.float32(1.0) - b1) * gf if buffer == 2 else gf
        want = float(torch.tensor(float(omb2 * (d * d))).to(torch.bfloat16))  # RNE, SR off
        assert want > 65000.0
        if clamped:
            assert torch.equal(vv, torch.full((n,), 65024.0)), pdt  # min(v, 65000) rounded to bf16
        else:
            assert torch.equal(vv, torch.full((n,), want)), (pdt, vv[:4], want)


# --------------------------------------------------------------------------- whole step

def _f64_step(mode, p, g, m, v, step, lr=1e-3, b1=0.9, b2=0.999, eps=1e-8, wd=0.08, tau=0.8, lam=0.3, ratio=0.05,
              cs=1.0, cautious=False):
    """The update re-evaluated in float64 from the reference's formulas (dual.rs, tdclm.rs,
    math.rs), no quantisation (fp32 everything, SR irrelevant). Hyper-parameters are the f32
    values the reference parses (config_parser.rs), so only the rounding of intermediates differs."""
    lr, b1, b2, eps, wd, tau, lam, ratio = (float(np.float32(x)) for x in (lr, b1, b2, eps, wd, tau, lam, ratio))
    g = np.where(np.isfinite(g) & (np.abs(g) < 1e38), np.clip(g, -1e18, 1e18), 0.0)
    bc1 = 1 - b1 ** (step + 1)
    bc2 = max(1 - b2 ** step, 1e-15)
    m_new = b1 * m + (1 - b1) * g
    if mode == 2:
        clm = b1 * m_new + (1 - b1) * g
        d = np.clip(g - m_new, -1e18, 1e18)
        v_new = b2 * v + (1 - b2) * d * d
        sigma = np.sqrt(np.maximum(v_new, 0)) * (bc1 * tau / math.sqrt(bc2)) + eps * bc1 * tau
        u = np.tanh(clm / np.maximum(sigma, 1e-12))
    else:
        clm = b1 * b1 * m + (1 - b1 * b1) * g
        d = np.clip(g - m, -1e18, 1e18)
        if mode == 4:
            v_new = b2 * v + (1 - b2) * d * d
            env = (0.5 * lam / math.sqrt(bc2)) * np.sqrt(v_new) + 0.5 * lam * np.abs(d) + (1 - b1 * b1) * np.abs(g) + b1 * b1 * np.abs(m) + eps
        else:
            v_new = None
            env = lam * np.abs(d) + (1 - b1 * b1) * np.abs(g) + b1 * b1 * np.abs(m) + eps
        u = clm / env
    delta = np.where(u * g > 0, u, 0.0) * cs if cautious else u
    s = lr * delta
    if mode in (3, 4):
        b = ratio * (np.abs(p) + 1e-2)
        s = b * (b + np.abs(s)) * s / (s * s + b * (b + np.abs(s)))
    else:
        b = ratio * np.sqrt(p * p + 1e-4)
        s = b * np.tanh(s / b)
    return (1 - lr * wd) * p - s, m_new, v_new, u


@pytest.mark.parametrize("buffer,code", [(2, 2), (1, 1), ("T1", 3), ("T2", 4)])
def test_full_step_matches_f64_reevaluation(oracle_mod, buffer, code):
    """fp32 oracle vs float64 re-evaluation of the same formulas: agreement to f32 rounding
    noise; a dropped term, wrong sign or swapped operand is far outside it."""
    O = oracle_mod
    rng = np.random.default_rng(11)
    n = 5000
    p0 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    m0 = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    v0 = (rng.random(n) * 1e-6).astype(np.float32)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    step = 7
    cfg = O.make_config(lr=1e-3, buffer=buffer, cautious=False, stochastic_rounding=False)
    p, m = p0.copy(), m0.copy()
    v = v0.copy() if code in (2, 4) else None
    sc = np.array([0, 0, 0, 1, 1, 0], dtype=np.float32)
    O.step(cfg, [p], [g], [m], [v], [None], [sc], [step], [0])
    pw, mw, vw, _ = _f64_step(code, p0.astype(np.float64), g.astype(np.float64), m0.astype(np.float64),
                              v0.astype(np.float64), step)
    # tolerances scale with the magnitude of the summed terms (cancellation-safe)
    m_scale = 0.9 * np.abs(m0) + 0.1 * np.abs(g)
    assert np.all(np.abs(m - mw) <= 4e-7 * m_scale)
    if v is not None:
        v_scale = 0.999 * v0 + 0.001 * (np.abs(g) + np.abs(m0)) ** 2
        assert np.all(np.abs(v - vw) <= 2e-6 * v_scale + 1e-30)
    # per element: the f32 rounding of p itself (2 ulp of |p|) plus 1e-5 of the step
    tol = 2.0 * np.spacing(np.abs(pw).astype(np.float32)).astype(np.float64) + 1e-5 * np.abs(pw - p0)
    assert np.all(np.abs(p.astype(np.float64) - pw) <= tol)
    dp_w = pw - p0
    # a dropped or mis-signed term moves the update by far more than the tolerance
    assert np.max(np.abs(dp_w)) > 1e-4


def test_triangle_family_u_bounded_and_bound_holds(oracle_mod):
    """|u| < 1 for T1/T2 (the envelope dominates |c| by the triangle inequality) and the applied
    step never exceeds b = ratio (|p| + 0.01)."""
    O = oracle_mod
    rng = np.random.default_rng(12)
    n = 20000
    for buffer in ("T1", "T2"):
        p0 = (rng.standard_normal(n) * 0.5).astype(np.float32)
        m = (rng.standard_normal(n) * 3).astype(np.float32)
        v = (rng.random(n) * 10).astype(np.float32) if buffer == "T2" else None
        g = (rng.standard_normal(n) * 5).astype(np.float32)
        p = p0.copy()
        cfg = O.make_config(lr=10.0, weight_decay=0.0, buffer=buffer, cautious=False, stochastic_rounding=False)
        O.step(cfg, [p], [g], [m], [v], [None], [np.array([0, 0, 0, 1, 1, 0], np.float32)], [3], [0])
        b = 0.05 * (np.abs(p0) + 0.01)
        assert np.all(np.abs(p - p0) <= b * (1 + 1e-5))
        _, _, _, u = _f64_step(4 if buffer == "T2" else 3, p0.astype(np.float64), g.astype(np.float64),
                               (m * 0 + m).astype(np.float64), None if v is None else v.astype(np.float64), 3)
        assert np.all(np.abs(u) < 1.0)


def test_cautious_mask_only_updates_aligned_elements(oracle_mod):
    """With cautious on and no weight decay, elements whose u*g <= 0 do not move (dual.rs:186-190)."""
    O = oracle_mod
    rng = np.random.default_rng(13)
    n = 4096
    p0 = (rng.standard_normal(n) * 0.1).astype(np.float32)
    m0 = (rng.standard_normal(n) * 1e-2).astype(np.float32)
    g = (rng.standard_normal(n) * 1e-2).astype(np.float32)
    for buffer, code in ((1, 1), ("T1", 3)):
        p = p0.copy()
        m = m0.copy()
        cfg = O.make_config(lr=1e-2, weight_decay=0.0, buffer=buffer, cautious=True, stochastic_rounding=False)
        sc = np.array([0, 0, 0, 1, 1, 0], dtype=np.float32)
        O.step(cfg, [p], [g], [m], [None], [None], [sc], [1], [0])
        _, _, _, u = _f64_step(code, p0.astype(np.float64), g.astype(np.float64), m0.astype(np.float64), None, 1)
        masked = (u * g) <= 0
        assert masked.sum() > 100 and (~masked).sum() > 100
        assert np.array_equal(p[masked], p0[masked])
        assert np.all(p[~masked] != p0[~masked])
        frac = (~masked).mean()
        assert abs(sc[3] - 1.0 / min(max(frac, 0.5), 1.0)) < 1e-3  # two-pass scale at step 1


def test_fused_equals_unfused_without_cautious_and_sr(oracle_mod):
    """One concatenated tensor == the pieces stepped separately when nothing depends on the
    tensor boundary (cautious off, SR off): luminav.py bucket semantics, test_end_to_end_training.py:339-395."""
    O = oracle_mod
    rng = np.random.default_rng(14)
    sizes = [33, 1, 4096, 70000, 5]
    for buffer in (1, 2, "T1", "T2"):
        dual = buffer in (2, "T2")
        ps = [(rng.standard_normal(k) * 0.02).astype(np.float32) for k in sizes]
        gs = [(rng.standard_normal(k) * 1e-3).astype(np.float32) for k in sizes]
        cfg = O.make_config(lr=2e-3, buffer=buffer, cautious=False, stochastic_rounding=False)
        sep_p = [x.copy() for x in ps]
        sep_m = [np.zeros(k, np.float32) for k in sizes]
        sep_v = [np.zeros(k, np.float32) if dual else None for k in sizes]
        sep_s = [np.array([0, 0, 0, 1, 1, 0], np.float32) for _ in sizes]
        cat_p, cat_g = np.concatenate(ps), np.concatenate(gs)
        cat_m = np.zeros_like(cat_p)
        cat_v = np.zeros_like(cat_p) if dual else None
        cat_s = np.array([0, 0, 0, 1, 1, 0], np.float32)
        for t in range(1, 4):
            O.step(cfg, sep_p, gs, sep_m, sep_v, [None] * len(sizes), sep_s, [t] * len(sizes), list(range(len(sizes))))
            O.step(cfg, [cat_p], [cat_g], [cat_m], [cat_v], [None], [cat_s], [t], [0])
        assert np.array_equal(np.concatenate(sep_p).view(np.uint32), cat_p.view(np.uint32))
        assert np.array_equal(np.concatenate(sep_m).view(np.uint32), cat_m.view(np.uint32))


def test_nan_and_inf_gradients_are_sanitised(oracle_mod):
    """core_tests.rs:160-237: a NaN gradient behaves like a zero gradient; two steps stay finite."""
    O = oracle_mod
    n = 32
    p = np.array([(i + 1) * 0.1 for i in range(n)], dtype=np.float32)
    g = np.array([0.05 if i % 2 == 0 else -0.03 for i in range(n)], dtype=np.float32)
    g_nan = g.copy()
    g_nan[0], g_nan[1] = np.nan, np.inf
    g_zero = g.copy()
    g_zero[0], g_zero[1] = 0.0, 0.0
    for buffer, mw, bt in ((1, 0, 1), (2, 2, 2)):
        outs = []
        for gg in (g_nan, g_zero):
            pp = p.copy()
            mp = p.copy() if mw else None
            m = np.zeros(n, np.float32)
            v = np.zeros(n, np.float32) if buffer == 2 else None
            sc = np.array([0, 0, 0, 1, 1, 0], np.float32)
            cfg = O.make_config(buffer=buffer, bound_type=bt, master_weights=mw)
            for t in (1, 2):
                O.step(cfg, [pp], [gg], [m], [v], [mp], [sc], [t], [0])
            assert np.all(np.isfinite(pp)) and np.all(np.isfinite(m)) and not np.array_equal(pp, p)
            outs.append(pp)
        assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("buffer", [2, "T2"])
@pytest.mark.parametrize("master", [0, 1])
def test_sr_vs_rne_variance_decay_after_spike(oracle_mod, buffer, master):
    """core_tests.rs:239-326: bf16 exp_avg_sq after one 100.0 gradient spike and 599 zero steps:
    round-to-nearest freezes (mean > 8), stochastic rounding decays (mean < 6.5)."""
    O = oracle_mod
    n = 256
    means = {}
    for sr in (False, True):
        p = torch.ones(n, dtype=torch.bfloat16)
        mp = torch.ones(n) if master else None
        m = torch.zeros(n, dtype=torch.bfloat16)
        v = torch.zeros(n, dtype=torch.bfloat16)
        sc = torch.tensor([0, 0, 0, 1, 1, 0], dtype=torch.float32)
        cfg = O.make_config(buffer=buffer, master_weights=master, stochastic_rounding=sr)
        spike = torch.full((n,), 100.0)
        zero = torch.zeros(n)
        for t in range(600):
            O.step(cfg, [p], [spike if t == 0 else zero], [m], [v], [mp], [sc], [t + 1], [0])
        means[sr] = float(v.float().mean())
        assert torch.isfinite(v.float()).all() and (v.float() >= 0).all()
    assert means[False] > 8.0 and means[True] < 6.5, means


def test_threads_and_chunks_do_not_change_results(oracle_mod):
    """2,097,152-element chunks run in parallel give the same bits as one thread, including the
    radial sums (partials fold in chunk order like the scalar core)."""
    O = oracle_mod
    n = 2097152 * 2 + 12345
    rng = np.random.default_rng(15)
    base_p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    for bt in (2, 1):
        res = []
        for threads in (1, 4):
            p = base_p.copy()
            m = np.zeros(n, np.float32)
            v = np.zeros(n, np.float32)
            sc = np.array([0, 0, 0, 1, 1, 0], np.float32)
            cfg = O.make_config(buffer="T2", bound_type=bt)
            for t in (1, 2):
                O.step(cfg, [p], [g], [m], [v], [None], [sc], [t], [0], threads=threads)
            res.append((p, m, v, sc))
        for a, b in zip(res[0], res[1]):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_index_base_reproduces_a_slice(oracle_mod):
    """Checker extension: re-running a slice [a, b) with index_base = a gives the same bits as the
    whole tensor (used to check multi-billion-element buckets slice by slice)."""
    O = oracle_mod
    n = 50000
    rng = np.random.default_rng(16)
    p0 = torch.from_numpy((rng.standard_normal(n) * 0.02).astype(np.float32)).to(torch.bfloat16)
    g = torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32)).to(torch.bfloat16)
    cfg = O.make_config(buffer="T2", cautious=False)
    whole = p0.clone()
    O.step(cfg, [whole], [g], [torch.zeros(n)], [torch.zeros(n)], [None],
           [torch.tensor([0, 0, 0, 1, 1, 0.0])], [5], [0])
    a, b = 12345, 40000
    part = p0[a:b].clone()
    O.step(cfg, [part], [g[a:b].clone()], [torch.zeros(b - a)], [torch.zeros(b - a)], [None],
           [torch.tensor([0, 0, 0, 1, 1, 0.0])], [5], [0], index_bases=[a])
    assert torch.equal(part.view(torch.int16), whole[a:b].view(torch.int16))
