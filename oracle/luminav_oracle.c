/*
 * CPU oracle for the LuminaV optimizer step -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's Rust CPU path.  Each function names
 * the reference file:line it follows.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library; the product package never
 * does.  Build: oracle/Makefile (gcc, -ffp-contract=off, fmaf wherever Rust
 * calls mul_add, IEEE div/sqrt, no fast-math).
 *
 * Parity status of each piece, and the checks that pin it, are listed in
 * tests/test_oracle_pins.py.  Known, documented limits:
 *   - radial-bound f32 sums follow the scalar core's chunk/lane order
 *     (reference_cpu/dual.rs:134-253); the reference's own SIMD backend sums in a
 *     different order, so radial sums are pinned by tolerance, not bitwise.
 *   - f64::powi is restated as compiler-builtins' repeated squaring (the lowering
 *     of llvm.powi); that lowering is not executable here ("parity unpinned" for
 *     the last f64 ulp of bc1/bc2; the f32 coefficients are pinned by exact
 *     rational arithmetic in the tests).
 */
#include "luminav_oracle_internal.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define LVO_ELEM_CHUNK_SIZE 2097152ULL /* reference_cpu/mod.rs:7, parallel/mod.rs:7 */

static __thread char g_err[256];

const char *lvo_last_error(void) { return g_err; }

static int fail(int code, const char *msg) {
    snprintf(g_err, sizeof g_err, "%s", msg);
    return code;
}

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Rust f32::clamp: if x < lo {lo}; if x > hi {hi}; NaN passes through. */
static inline float rclamp(float x, float lo, float hi) {
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}

/* ---------------------------------------------------------------- prng.rs */

/* prng.rs:21-26: wrapping i32 arithmetic, arithmetic right shifts. */
int32_t lvo_prng(int32_t seed, int32_t idx) {
    uint32_t z = (uint32_t)idx + (uint32_t)seed - 1640531527u;
    int32_t zi = (int32_t)z;
    z = (uint32_t)(zi ^ (zi >> 16)) * (uint32_t)(-2048173461);
    zi = (int32_t)z;
    z = (uint32_t)(zi ^ (zi >> 13)) * (uint32_t)(-1028477387);
    zi = (int32_t)z;
    return zi ^ (zi >> 16);
}

/* prng.rs:4-13. Only the low 31 bits survive, so u64 wrapping == u128 wrapping. */
void lvo_derive_kernel_seeds(uint32_t seed, uint64_t step, uint64_t param_index,
                             int32_t *seed_m, int32_t *seed_p) {
    uint64_t raw = (uint64_t)seed + step * 0x9E3779B9ull + param_index * 10007ull;
    int32_t sm = (int32_t)(raw & 0x7FFFFFFFull);
    /* (seed_m as u64): seed_m is non-negative here */
    int32_t sp = (int32_t)(((uint64_t)(int64_t)sm + 0x55555555ull) & 0x7FFFFFFFull);
    *seed_m = sm;
    *seed_p = sp;
}

/* prng.rs:15-18 */
int32_t lvo_derive_variance_seed(int32_t seed_m) {
    return (int32_t)(((uint64_t)(int64_t)seed_m + 0x2A6D365Bull) & 0x7FFFFFFFull);
}

/* prng.rs:29-67 */
uint16_t lvo_f32_to_f16_bits_rne(float val) {
    uint32_t bits = f2u(val);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    int32_t exp = (int32_t)((bits >> 23) & 0xFFu);
    uint32_t mant = bits & 0x007FFFFFu;
    if (exp == 255) return mant != 0 ? (uint16_t)(sign | 0x7E00u) : (uint16_t)(sign | 0x7BFFu);
    int32_t new_exp = exp - 112;
    if (new_exp >= 31) return (uint16_t)(sign | 0x7BFFu);
    if (new_exp <= 0) {
        if (new_exp < -10) return sign;
        uint32_t full_mant = mant | 0x00800000u;
        uint32_t shift = (uint32_t)(14 - new_exp);
        uint32_t half_bit = 1u << (shift - 1);
        uint32_t lsb = (full_mant >> shift) & 1u;
        uint32_t rounded = (full_mant + half_bit - 1u + lsb) >> shift;
        return (uint16_t)(sign | (uint16_t)rounded);
    }
    uint32_t lsb = (mant >> 13) & 1u;
    uint32_t rounded = mant + 0x0FFFu + lsb;
    uint32_t body = ((uint32_t)new_exp << 10) + (rounded >> 13);
    if (body >= 0x7C00u) return (uint16_t)(sign | 0x7BFFu);
    return (uint16_t)(sign | (uint16_t)body);
}

/* prng.rs:69-96 */
float lvo_f16_bits_to_f32(uint16_t bits) {
    uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
    uint32_t exp = (uint32_t)((bits >> 10) & 0x1Fu);
    uint32_t mant = (uint32_t)(bits & 0x03FFu);
    if (exp == 0) {
        if (mant == 0) return u2f(sign);
        uint32_t m = mant, e = 113;
        while ((m & 0x0400u) == 0) { m <<= 1; e -= 1; }
        m &= 0x03FFu;
        return u2f(sign | (e << 23) | (m << 13));
    }
    if (exp == 31) return u2f(sign | 0x7F800000u | (mant << 13));
    return u2f(sign | ((exp + 112u) << 23) | (mant << 13));
}

/* prng.rs:98-125 */
uint16_t lvo_sr_fp16_bits(float v, int32_t seed, int32_t offset) {
    int32_t p_int = (int32_t)f2u(v);
    int32_t abs_int = p_int & 0x7FFFFFFF;
    int32_t exp_f32 = (abs_int >> 23) & 0xFF;
    int32_t raw_sub = 113 - exp_f32;
    int32_t clamped_low = raw_sub > 0 ? raw_sub : 0;
    int32_t sub_shift = clamped_low < 11 ? clamped_low : 11;
    int32_t total_shift = 13 + sub_shift;
    int32_t mask_bits = (int32_t)((1u << total_shift) - 1u);
    int32_t noise = lvo_prng(seed, offset) & mask_bits;
    int32_t added_abs = exp_f32 < 103 ? 0 : (int32_t)(((uint32_t)abs_int + (uint32_t)noise) & (uint32_t)(~mask_bits));
    int32_t rounded_abs = added_abs > 0x477FE000 ? 0x477FE000 : added_abs;
    int32_t sign_bit = p_int & (int32_t)0x80000000u;
    int32_t out_int = sign_bit | rounded_abs;
    return lvo_f32_to_f16_bits_rne(u2f((uint32_t)out_int));
}

float lvo_sr_fp16(float v, int32_t seed, int32_t offset) {
    return lvo_f16_bits_to_f32(lvo_sr_fp16_bits(v, seed, offset)); /* prng.rs:127-130 */
}

float lvo_rne_fp16(float v) { return lvo_f16_bits_to_f32(lvo_f32_to_f16_bits_rne(v)); } /* prng.rs:132-135 */

/* prng.rs:137-154 */
uint16_t lvo_sr_bf16_bits(float v, int32_t seed, int32_t offset) {
    int32_t p_int = (int32_t)f2u(v);
    int32_t abs_int = p_int & 0x7FFFFFFF;
    if (abs_int > 0x7F800000) return (uint16_t)((((uint32_t)p_int) | 0x00400000u) >> 16);
    int32_t noise = lvo_prng(seed, offset) & 0xFFFF;
    int32_t added = (int32_t)(((uint32_t)abs_int + (uint32_t)noise) & 0xFFFF0000u);
    int32_t rounded_abs = (added > 0x7F7F0000 || added < 0) ? 0x7F7F0000 : added;
    int32_t sign_bit = p_int & (int32_t)0x80000000u;
    return (uint16_t)(((uint32_t)(sign_bit | rounded_abs)) >> 16);
}

float lvo_sr_bf16(float v, int32_t seed, int32_t offset) {
    return u2f((uint32_t)lvo_sr_bf16_bits(v, seed, offset) << 16); /* prng.rs:156-160 */
}

/* prng.rs:162-178 */
float lvo_rne_bf16(float v) {
    uint32_t bits = f2u(v);
    uint32_t abs_bits = bits & 0x7FFFFFFFu;
    if (abs_bits > 0x7F800000u) return u2f((bits | 0x00400000u) & 0xFFFF0000u);
    uint32_t sign = bits & 0x80000000u;
    uint32_t lsb = (abs_bits >> 16) & 1u;
    uint32_t rounded_abs = (abs_bits + 0x7FFFu + lsb) & 0xFFFF0000u;
    uint32_t clamped = rounded_abs > 0x7F7F0000u ? 0x7F7F0000u : rounded_abs;
    return u2f(sign | clamped);
}

/* prng.rs:180-195 */
float lvo_quantize(float v, int32_t seed, int32_t offset, int32_t dtype, int32_t use_sr) {
    switch (dtype) {
    case 1: return use_sr ? lvo_sr_bf16(v, seed, offset) : lvo_rne_bf16(v);
    case 2: return use_sr ? lvo_sr_fp16(v, seed, offset) : lvo_rne_fp16(v);
    default: return v;
    }
}

/* ---------------------------------------------------------------- math.rs */

/* math.rs:4-11 */
float lvo_sanitize_gradient(float g) {
    if (isfinite(g) && fabsf(g) < 1.0e38f) return rclamp(g, -1.0e18f, 1.0e18f);
    return 0.0f;
}

/* compiler-builtins __powidf2 (the lowering of llvm.powi used by f64::powi). */
double lvo_powi(double a, int32_t b) {
    int recip = b < 0;
    uint32_t pw = recip ? (uint32_t)(-(int64_t)b) : (uint32_t)b;
    double mul = 1.0;
    for (;;) {
        if (pw & 1u) mul *= a;
        pw >>= 1;
        if (pw == 0) break;
        a *= a;
    }
    return recip ? 1.0 / mul : mul;
}

/* math.rs:27-68 */
void lvo_bias_correction(uint64_t step, float beta1, float beta2, float eps, float tau, float *out) {
    uint64_t safe = step > 1 ? step : 1;
    double b1 = (double)beta1, b2 = (double)beta2, t = (double)tau, e = (double)eps;
    double bc1 = safe < 2147483647ull ? 1.0 - lvo_powi(b1, (int32_t)(safe + 1))
                                      : 1.0 - pow(b1, (double)(safe + 1));
    double bc2_raw = safe <= 2147483647ull ? 1.0 - lvo_powi(b2, (int32_t)safe)
                                           : 1.0 - pow(b2, (double)safe);
    double bc2 = fmax(bc2_raw, 1.0e-15);
    out[0] = (float)bc1;
    out[1] = (float)bc2;
    out[2] = (float)((bc1 * t) / sqrt(bc2));
    out[3] = (float)(e * bc1 * t);
    out[4] = eps;
}

/* math.rs:70-81 */
float lvo_t2_sigma_coeff(uint64_t step, float beta2, float lam) {
    uint64_t safe = step > 1 ? step : 1;
    double b2 = (double)beta2;
    double bc2_raw = safe <= 2147483647ull ? 1.0 - lvo_powi(b2, (int32_t)safe)
                                           : 1.0 - pow(b2, (double)safe);
    float bc2 = (float)fmax(bc2_raw, 1.0e-15);
    return (0.5f * lam) / sqrtf(fmaxf(bc2, 1.0e-15f));
}

/* math.rs:83-118 */
float lvo_tanh_pade(float x_in) {
    if (isnan(x_in)) return NAN;
    const float A13 = -2.7607684e-16f, A11 = 2.000188e-13f, A9 = -8.604672e-11f,
                A7 = 5.122297e-8f, A5 = 1.4857224e-5f, A3 = 6.3726193e-4f, A1 = 4.8935246e-3f;
    const float B6 = 1.1982584e-6f, B4 = 1.1853471e-4f, B2 = 2.2684346e-3f, B0 = 4.8935246e-3f;
    float x = rclamp(x_in, -7.9988117f, 7.9988117f);
    float x2 = x * x;
    float p = fmaf(A13, x2, A11);
    float q = fmaf(B6, x2, B4);
    p = fmaf(p, x2, A9);
    q = fmaf(q, x2, B2);
    p = fmaf(p, x2, A7);
    q = fmaf(q, x2, B0);
    p = fmaf(p, x2, A5);
    p = fmaf(p, x2, A3);
    p = fmaf(p, x2, A1);
    return (x * p) / q;
}

/* math.rs:120-125 */
float lvo_cautious_scale(float mask_sum, float total, float clamp_min) {
    float denom = fmaxf(total, 1.0f);
    float m_bar = rclamp(mask_sum / denom, clamp_min, 1.0f);
    return 1.0f / m_bar;
}

/* math.rs:127-144 */
float lvo_radial_scale(float u_sq, float p_sq, float cs, float lr, float ratio) {
    float norm_p = sqrtf(fmaxf(p_sq, 0.0f));
    float norm_d = sqrtf(fmaxf(u_sq, 0.0f)) * cs;
    float radius = ratio * fmaxf(norm_p, 1.0f);
    float r = (lr * norm_d) / radius;
    if (r < 1.0e-4f) return 1.0f;
    return lvo_tanh_pade(r) / fmaxf(r, 1.0e-8f);
}

/* math.rs:146-160 */
float lvo_radial_scale_t2(float u_sq, float p_sq, float cs, float lr, float ratio) {
    float norm_p = sqrtf(fmaxf(p_sq, 0.0f));
    float norm_d = sqrtf(fmaxf(u_sq, 0.0f)) * cs;
    float radius = ratio * fmaxf(norm_p, 1.0f);
    float r = (lr * norm_d) / fmaxf(radius, 1.0e-12f);
    float one_plus_r = 1.0f + r;
    return one_plus_r / fmaf(r, r, one_plus_r);
}

/* math.rs:162-166 */
float lvo_coordinate_bound(float step, float p_init, float ratio) {
    float b = ratio * sqrtf(fmaf(p_init, p_init, 1.0e-4f));
    return b * lvo_tanh_pade(step / b);
}

/* math.rs:168-173 */
float lvo_coordinate_bound_t2(float step, float p_init, float ratio) {
    float b = ratio * (fabsf(p_init) + 1.0e-2f);
    float bb = b * (b + fabsf(step));
    return (bb * step) / fmaf(step, step, bb);
}

/* math.rs:175-179 */
float lvo_fp16_safety_bound(float step, float p_init) {
    float b = fmaxf(fabsf(p_init) * 0.01f, 1.5e-4f);
    return b * lvo_tanh_pade(step / b);
}

/* math.rs:181-186 */
float lvo_fp16_safety_bound_t2(float step, float p_init) {
    float b = fmaxf(fabsf(p_init) * 0.01f, 1.5e-4f);
    float bb = b * (b + fabsf(step));
    return (bb * step) / fmaf(step, step, bb);
}

static inline int effective_bound(const lvo_config *c) { /* config.rs:368-375 */
    return (c->bound && c->bound_ratio > 0.0f) ? c->bound_type : 0;
}

static inline void reset_accumulators(float *s) { s[0] = 0.0f; s[1] = 0.0f; s[2] = 0.0f; s[5] = 0.0f; } /* state.rs:105-111 */

/* math.rs:188-239. `triangle` selects the radial target form (is_triangle_family). */
void lvo_update_post_step_ema(float *s, float total, const lvo_config *cfg, int32_t triangle) {
    int bound = effective_bound(cfg);
    if (cfg->cautious) {
        float target = lvo_cautious_scale(s[0], total, cfg->cautious_clamp_min);
        float old = s[3];
        s[3] = fmaf(cfg->ema_decay, old, (1.0f - cfg->ema_decay) * target);
    }
    if (bound == 1) {
        float cs = cfg->cautious ? s[3] : 1.0f;
        float target = triangle ? lvo_radial_scale_t2(s[1], s[2], cs, cfg->lr, cfg->bound_ratio)
                                : lvo_radial_scale(s[1], s[2], cs, cfg->lr, cfg->bound_ratio);
        float old = s[4];
        s[4] = fmaf(cfg->ema_decay, old, (1.0f - cfg->ema_decay) * target);
    }
    reset_accumulators(s);
}

/* math.rs:241-261 */
static float reduce_sum_16(const float *l) {
    float s8[8], s4[4];
    for (int i = 0; i < 8; i++) s8[i] = l[i] + l[i + 8];
    for (int i = 0; i < 4; i++) s4[i] = s8[i] + s8[i + 4];
    float s2_0 = s4[0] + s4[2];
    float s2_1 = s4[1] + s4[3];
    return s2_0 + s2_1;
}

float lvo_u64_to_f32(uint64_t x) { return (float)x; } /* Rust `as f32`: round to nearest even */

/* config.rs:329-366 */
int lvo_validate_config(const lvo_config *c) {
    if (!isfinite(c->lr) || c->lr < 0.0f) return fail(LVO_ERR_CONFIG, "Invalid learning rate");
    if (!isfinite(c->beta1) || !(c->beta1 >= 0.0f && c->beta1 < 1.0f)) return fail(LVO_ERR_CONFIG, "Invalid beta1 parameter");
    if (!isfinite(c->beta2) || !(c->beta2 >= 0.0f && c->beta2 < 1.0f)) return fail(LVO_ERR_CONFIG, "Invalid beta2 parameter");
    if (!isfinite(c->eps) || c->eps <= 0.0f) return fail(LVO_ERR_CONFIG, "Invalid epsilon value");
    if (!isfinite(c->weight_decay) || c->weight_decay < 0.0f) return fail(LVO_ERR_CONFIG, "Invalid weight_decay value");
    if (!isfinite(c->tau) || c->tau <= 0.0f) return fail(LVO_ERR_CONFIG, "Invalid tau parameter");
    if (!isfinite(c->lam) || c->lam < 0.0f) return fail(LVO_ERR_CONFIG, "Invalid lam parameter");
    if (!isfinite(c->cautious_clamp_min) || c->cautious_clamp_min <= 0.0f || c->cautious_clamp_min > 1.0f)
        return fail(LVO_ERR_CONFIG, "Invalid cautious_clamp_min");
    if (!isfinite(c->bound_ratio) || c->bound_ratio <= 0.0f) return fail(LVO_ERR_CONFIG, "Invalid bound_ratio");
    if (!isfinite(c->ema_decay) || c->ema_decay <= 0.0f || c->ema_decay >= 1.0f) return fail(LVO_ERR_CONFIG, "Invalid ema_decay");
    if (c->buffer < 1 || c->buffer > 4) return fail(LVO_ERR_CONFIG, "Invalid buffer count");
    if (c->bound_type < 0 || c->bound_type > 2) return fail(LVO_ERR_CONFIG, "Invalid bound_type");
    if (c->master_weights < 0 || c->master_weights > 2) return fail(LVO_ERR_CONFIG, "Invalid master_weights");
    return LVO_OK;
}

/* ------------------------------------------------------- per-element core */

/* u for one element; m_new / v_new are returned for the apply step.
 * CLM: dual.rs:63-74; T2: dual.rs:492-506; TD-CLM / T1: tdclm.rs:102-109. */
static inline float compute_u(const coef_t *k, float g, float m, float v, float *m_new_out, float *v_new_out) {
    float m_new = fmaf(k->b1, m, k->omb1 * g);
    float u, v_new = 0.0f;
    if (k->mode == 2) {
        float clm = fmaf(k->b1, m_new, k->omb1 * g);
        float diff = rclamp(g - m_new, -1.0e18f, 1.0e18f);
        v_new = fmaf(k->b2, v, k->omb2 * (diff * diff));
        if (k->clamp_v) v_new = fminf(v_new, 65000.0f);
        float sigma = fmaf(sqrtf(fmaxf(v_new, 0.0f)), k->c1, k->c2);
        u = lvo_tanh_pade(clm / fmaxf(sigma, 1.0e-12f));
    } else if (k->mode == 4) {
        float clm = fmaf(k->b1sq, m, k->omb1sq * g);
        float diff = rclamp(g - m, -1.0e18f, 1.0e18f);
        v_new = fmaf(k->b2, v, k->omb2 * (diff * diff));
        if (k->clamp_v) v_new = fminf(v_new, 65000.0f);
        float env0 = fmaf(k->b1sq, fabsf(m), k->eps);
        float env1 = fmaf(k->omb1sq, fabsf(g), env0);
        float env2 = fmaf(k->lam1, fabsf(diff), env1);
        float env = fmaf(k->c_sigma, sqrtf(fmaxf(v_new, 0.0f)), env2);
        u = clm / env;
    } else {
        float clm = fmaf(k->b1sq, m, k->omb1sq * g);
        float diff = rclamp(g - m, -1.0e18f, 1.0e18f);
        float env0 = fmaf(k->b1sq, fabsf(m), k->eps);
        float env1 = fmaf(k->omb1sq, fabsf(g), env0);
        float env = fmaf(k->lam, fabsf(diff), env1);
        u = clm / env;
    }
    *m_new_out = m_new;
    *v_new_out = v_new;
    return u;
}

/* Apply + store for one element (dual.rs:168-228 and the matching blocks of tdclm.rs).
 * Returns 1 when the cautious mask is active. */
static inline int apply_elem(const coef_t *k, const view_t *w, uint64_t idx, float cs, float bs,
                             float *u_sq_out, float *p_sq_out) {
    int32_t off = (int32_t)(uint32_t)(k->index_base + idx);
    float p_init = k->has_master ? w->mp[idx] : w->p[idx];
    float g = lvo_sanitize_gradient(w->g[idx]);
    float m = w->m[idx];
    float v = k->dual_state ? w->v[idx] : 0.0f;
    float m_new, v_new;
    float u = compute_u(k, g, m, v, &m_new, &v_new);
    int active = (u * g) > 0.0f;
    float m_mask = active ? 1.0f : 0.0f;

    w->m[idx] = lvo_quantize(m_new, k->seed_m, off, k->s_mode, k->sr);
    if (k->dual_state) w->v[idx] = lvo_quantize(v_new, k->seed_v, off, k->s_mode, k->sr);

    float delta = k->cautious ? (u * m_mask) * cs : u;
    float step = k->lr * delta;
    if (k->bound == 1) {
        step *= bs;
    } else if (k->bound == 2) {
        step = k->triangle ? lvo_coordinate_bound_t2(step, p_init, k->ratio)
                           : lvo_coordinate_bound(step, p_init, k->ratio);
    }
    if (k->fp16_param)
        step = k->triangle ? lvo_fp16_safety_bound_t2(step, p_init) : lvo_fp16_safety_bound(step, p_init);
    float p_dec = k->wd_nonzero ? fmaf(-k->lr_wd, p_init, p_init) : p_init;
    float p_upd = p_dec - step;
    if (k->has_master) {
        w->mp[idx] = p_upd;
        w->p[idx] = lvo_quantize(p_upd, k->seed_p, off, k->p_mode, 0);
    } else {
        w->p[idx] = lvo_quantize(p_upd, k->seed_p, off, k->p_mode, k->sr);
    }
    if (u_sq_out) {
        float u_eff = k->cautious ? u * m_mask : u;
        *u_sq_out = u_eff * u_eff;
        *p_sq_out = p_init * p_init;
    }
    return active;
}

/* Pass-1 counting for one element (dual.rs:279-320, dual.rs:720-763, tdclm.rs:232-265). */
static inline int count_elem(const coef_t *k, const view_t *w, uint64_t idx, float *u_sq_out, float *p_sq_out) {
    float g = lvo_sanitize_gradient(w->g[idx]);
    float m = w->m[idx];
    float v = k->dual_state ? w->v[idx] : 0.0f;
    float m_new, v_new;
    float u = compute_u(k, g, m, v, &m_new, &v_new);
    int active = (u * g) > 0.0f;
    if (u_sq_out) {
        float u_eff = k->cautious ? u * (active ? 1.0f : 0.0f) : u;
        float p_val = k->has_master ? w->mp[idx] : w->p[idx];
        *u_sq_out = u_eff * u_eff;
        *p_sq_out = p_val * p_val;
    }
    return active;
}

int lvo_i_apply_elem(const coef_t *k, const view_t *w, uint64_t idx, float cs, float bs, float *u_sq_out,
                     float *p_sq_out) {
    return apply_elem(k, w, idx, cs, bs, u_sq_out, p_sq_out);
}

int lvo_i_count_elem(const coef_t *k, const view_t *w, uint64_t idx, float *u_sq_out, float *p_sq_out) {
    return count_elem(k, w, idx, u_sq_out, p_sq_out);
}

/* luminav-simd/src/lib.rs:38-60 (the AVX-512 backend's feature test) */
int lvo_i_cpu_has_avx512(void) {
#if defined(__x86_64__)
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512dq") &&
           __builtin_cpu_supports("avx512bw") && __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("fma");
#else
    return 0;
#endif
}

/* Chunk backend: 0 = the scalar core (default, what the HIP kernels are checked against);
 * 1 = the restatement of luminav-simd's AVX-512 chunk kernels (avx512/dual.rs, avx512/tdclm.rs),
 * the reference's own CPU execution path. The f64 radial sum mode always uses the scalar core. */
static int g_backend = 0;

int32_t lvo_set_backend(int32_t backend) {
    if (backend != 0 && backend != 1) return fail(LVO_ERR_CONFIG, "unknown backend");
    if (backend == 1 && !lvo_i_cpu_has_avx512()) return fail(LVO_ERR_EXEC, "this CPU lacks AVX-512 (avx512f/dq/bw/vl + fma)");
    g_backend = backend;
    return LVO_OK;
}

int32_t lvo_backend(void) { return g_backend; }

/* Radial sum mode (checker option, not a reference behaviour): 0 = the scalar core's f32 lane
 * and chunk order (default); 1 = every f32 square added in f64, rounded to f32 once -- the
 * order-independent sum the HIP kernels compute, so they can be compared bit for bit. */
static int g_radial_sum_f64 = 0;
void lvo_set_radial_sum_mode(int32_t mode) { g_radial_sum_f64 = mode ? 1 : 0; }
int32_t lvo_radial_sum_mode(void) { return g_radial_sum_f64; }

/* One 2,097,152-element chunk of a counting pass: lane sums exactly as the scalar core. */
static chunk_metrics run_chunk(const coef_t *k, const view_t *w, uint64_t start, uint64_t end,
                               int apply, float cs, float bs) {
    if (g_backend == 1 && !g_radial_sum_f64) return lvo_i_avx512_chunk(k, w, start, end, apply, cs, bs);
    chunk_metrics cm = {0, 0.0f, 0.0f, 0.0, 0.0};
    uint64_t len = end - start;
    uint64_t simd_len = len & ~15ull;
    float ul[16] = {0}, pl[16] = {0};
    float ut = 0.0f, pt = 0.0f;
    int radial = k->bound == 1;
    for (uint64_t li = 0; li < len; li++) {
        uint64_t idx = start + li;
        float usq = 0.0f, psq = 0.0f;
        int act = apply ? apply_elem(k, w, idx, cs, bs, radial ? &usq : NULL, &psq)
                        : count_elem(k, w, idx, radial ? &usq : NULL, &psq);
        if (k->cautious && act) cm.mask += 1;
        if (radial) {
            if (g_radial_sum_f64) { cm.du += (double)usq; cm.dp += (double)psq; }
            else if (li < simd_len) { ul[li & 15] += usq; pl[li & 15] += psq; }
            else { ut += usq; pt += psq; }
        }
    }
    if (radial) {
        cm.u_sq = reduce_sum_16(ul) + ut;
        cm.p_sq = reduce_sum_16(pl) + pt;
    }
    return cm;
}

/* Runs a counting pass over all chunks; partials fold in chunk order like the scalar core. */
static chunk_metrics run_counting(const coef_t *k, const view_t *w, uint64_t n, int apply,
                                  float cs, float bs, int threads) {
    uint64_t nchunks = (n + LVO_ELEM_CHUNK_SIZE - 1) / LVO_ELEM_CHUNK_SIZE;
    chunk_metrics tot = {0, 0.0f, 0.0f, 0.0, 0.0};
    if (threads > 1 && nchunks > 1) {
        chunk_metrics *parts = (chunk_metrics *)malloc(nchunks * sizeof(chunk_metrics));
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
        for (int64_t c = 0; c < (int64_t)nchunks; c++) {
            uint64_t s = (uint64_t)c * LVO_ELEM_CHUNK_SIZE;
            uint64_t e = s + LVO_ELEM_CHUNK_SIZE < n ? s + LVO_ELEM_CHUNK_SIZE : n;
            parts[c] = run_chunk(k, w, s, e, apply, cs, bs);
        }
        for (uint64_t c = 0; c < nchunks; c++) {
            tot.mask += parts[c].mask;
            tot.u_sq += parts[c].u_sq;
            tot.p_sq += parts[c].p_sq;
            tot.du += parts[c].du;
            tot.dp += parts[c].dp;
        }
        free(parts);
    } else {
        for (uint64_t c = 0; c < nchunks; c++) {
            uint64_t s = c * LVO_ELEM_CHUNK_SIZE;
            uint64_t e = s + LVO_ELEM_CHUNK_SIZE < n ? s + LVO_ELEM_CHUNK_SIZE : n;
            chunk_metrics cm = run_chunk(k, w, s, e, apply, cs, bs);
            tot.mask += cm.mask;
            tot.u_sq += cm.u_sq;
            tot.p_sq += cm.p_sq;
            tot.du += cm.du;
            tot.dp += cm.dp;
        }
    }
    if (g_radial_sum_f64) {
        tot.u_sq = (float)tot.du;
        tot.p_sq = (float)tot.dp;
    }
    return tot;
}

/* Non-counting single pass (dual.rs:52-121, dual.rs:481-553). */
static void run_plain(const coef_t *k, const view_t *w, uint64_t n, int threads) {
    if (g_backend == 1) {
        /* avx512/dual.rs:891-918: the same 2,097,152-element chunks, serial or in parallel */
        uint64_t nchunks = (n + LVO_ELEM_CHUNK_SIZE - 1) / LVO_ELEM_CHUNK_SIZE;
#pragma omp parallel for num_threads(threads > 1 ? threads : 1) schedule(dynamic, 1) if (threads > 1 && nchunks > 1)
        for (int64_t c = 0; c < (int64_t)nchunks; c++) {
            uint64_t s = (uint64_t)c * LVO_ELEM_CHUNK_SIZE;
            uint64_t e = s + LVO_ELEM_CHUNK_SIZE < n ? s + LVO_ELEM_CHUNK_SIZE : n;
            (void)lvo_i_avx512_chunk(k, w, s, e, 1, 1.0f, 1.0f);
        }
        return;
    }
    if (threads > 1 && n > LVO_ELEM_CHUNK_SIZE) {
        uint64_t nchunks = (n + LVO_ELEM_CHUNK_SIZE - 1) / LVO_ELEM_CHUNK_SIZE;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
        for (int64_t c = 0; c < (int64_t)nchunks; c++) {
            uint64_t s = (uint64_t)c * LVO_ELEM_CHUNK_SIZE;
            uint64_t e = s + LVO_ELEM_CHUNK_SIZE < n ? s + LVO_ELEM_CHUNK_SIZE : n;
            for (uint64_t i = s; i < e; i++) apply_elem(k, w, i, 1.0f, 1.0f, NULL, NULL);
        }
    } else {
        for (uint64_t i = 0; i < n; i++) apply_elem(k, w, i, 1.0f, 1.0f, NULL, NULL);
    }
}

/*
 * The scalar core for one decoded tensor: single_step_dual_scalar / single_step_t2_scalar
 * (dual.rs:14-888) and single_step_single_buffer_impl (tdclm.rs:34-392).
 */
static int core_step(const lvo_config *cfg, const view_t *w, float *scratch, uint64_t n,
                     uint64_t step, uint64_t param_index, int p_mode, int s_mode_raw, int threads,
                     uint64_t index_base) {
    int rc = lvo_validate_config(cfg);
    if (rc != LVO_OK) return rc;
    if (n == 0) return LVO_OK;
    coef_t k;
    memset(&k, 0, sizeof k);
    k.mode = cfg->buffer;
    k.triangle = (cfg->buffer == 3 || cfg->buffer == 4);
    k.dual_state = (cfg->buffer == 2 || cfg->buffer == 4);
    k.has_master = cfg->master_weights != 0;
    if (k.dual_state && !w->v) return fail(LVO_ERR_EXEC, "Dual-buffer mode requires an initialized exp_avg_sq buffer");
    if (k.has_master && !w->mp) return fail(LVO_ERR_EXEC, "Master weight mode requires an initialized master_param buffer");
    k.fp16_param = p_mode == 2;
    k.clamp_v = (p_mode == 2 || s_mode_raw == 2);
    k.p_mode = p_mode;
    k.s_mode = s_mode_raw == 2 ? 1 : s_mode_raw; /* fp16 state -> bitwise bf16 (dual.rs:40-45) */
    k.cautious = cfg->cautious != 0;
    k.sr = cfg->stochastic_rounding != 0;
    k.bound = effective_bound(cfg);
    k.wd_nonzero = cfg->weight_decay != 0.0f;
    k.lr = cfg->lr;
    k.b1 = cfg->beta1;
    k.b2 = cfg->beta2;
    k.omb1 = 1.0f - k.b1;
    k.omb2 = 1.0f - k.b2;
    k.b1sq = k.b1 * k.b1;
    k.omb1sq = 1.0f - k.b1sq;
    k.lam = cfg->lam;
    k.lam1 = 0.5f * cfg->lam;
    k.eps = cfg->eps;
    k.lr_wd = cfg->lr * cfg->weight_decay;
    k.ratio = cfg->bound_ratio;
    float bc[5];
    lvo_bias_correction(step, cfg->beta1, cfg->beta2, cfg->eps, cfg->tau, bc);
    k.c1 = bc[2];
    k.c2 = bc[3];
    k.c_sigma = lvo_t2_sigma_coeff(step, cfg->beta2, cfg->lam);
    lvo_derive_kernel_seeds(cfg->seed, step, param_index, &k.seed_m, &k.seed_p);
    k.seed_v = lvo_derive_variance_seed(k.seed_m);
    k.index_base = index_base;

    float total = (float)n;
    int radial = k.bound == 1;
    if (!k.cautious && !radial) {
        /* single pass without statistics (dual.rs:52-121, tdclm.rs:67-68) */
        run_plain(&k, w, n, threads);
        reset_accumulators(scratch);
    } else if (cfg->fused_single_pass && step > 1) {
        /* lagged scales, count, EMA (dual.rs:122-259, dual.rs:554-700, tdclm.rs:70-212) */
        scratch[0] = scratch[1] = scratch[2] = 0.0f;
        float cs = scratch[3], bs = scratch[4];
        chunk_metrics t = run_counting(&k, w, n, 1, cs, bs, threads);
        scratch[0] = (float)t.mask;
        scratch[1] = t.u_sq;
        scratch[2] = t.p_sq;
        lvo_update_post_step_ema(scratch, total, cfg, k.triangle);
    } else {
        /* two passes (dual.rs:260-439, dual.rs:701-885, tdclm.rs:213-389) */
        scratch[0] = scratch[1] = scratch[2] = 0.0f;
        chunk_metrics t = run_counting(&k, w, n, 0, 1.0f, 1.0f, threads);
        float mask_sum = (float)t.mask;
        scratch[0] = mask_sum;
        scratch[1] = t.u_sq;
        scratch[2] = t.p_sq;
        float cs = k.cautious ? lvo_cautious_scale(mask_sum, total, cfg->cautious_clamp_min) : 1.0f;
        float bs = 1.0f;
        if (radial)
            bs = k.triangle ? lvo_radial_scale_t2(t.u_sq, t.p_sq, cs, cfg->lr, cfg->bound_ratio)
                            : lvo_radial_scale(t.u_sq, t.p_sq, cs, cfg->lr, cfg->bound_ratio);
        run_counting(&k, w, n, 1, cs, bs, threads);
        reset_accumulators(scratch);
        scratch[3] = cs;
        scratch[4] = bs;
    }
    return LVO_OK;
}

/* ------------------------------------------------------- worker.rs wrapper */

/* worker.rs:35-53 (serial decode, as the reference does) */
static float *decode(const void *ptr, uint64_t n, int mode) {
    float *dst = (float *)malloc((n ? n : 1) * sizeof(float));
    if (!dst) return NULL;
    const uint16_t *h = (const uint16_t *)ptr;
    if (mode == 1) {
        for (uint64_t i = 0; i < n; i++) dst[i] = u2f((uint32_t)h[i] << 16);
    } else {
        for (uint64_t i = 0; i < n; i++) dst[i] = lvo_f16_bits_to_f32(h[i]);
    }
    return dst;
}

/* worker.rs:55-75 */
static void encode(void *ptr, const float *src, uint64_t n, int mode) {
    uint16_t *h = (uint16_t *)ptr;
    if (mode == 1) {
        for (uint64_t i = 0; i < n; i++) h[i] = (uint16_t)(f2u(src[i]) >> 16);
    } else {
        for (uint64_t i = 0; i < n; i++) h[i] = lvo_f32_to_f16_bits_rne(src[i]);
    }
}

/* worker.rs:77-179 */
static int process_item(const lvo_config *cfg, const lvo_tensor *it, int threads) {
    uint64_t n = it->numel;
    int p_mode = it->param_dtype, g_mode = it->grad_dtype;
    int s_mode = it->state_dtype == 2 ? 1 : it->state_dtype; /* worker.rs:107-113 */
    float *pbuf = NULL, *gbuf = NULL, *mbuf = NULL, *vbuf = NULL;
    view_t w;
    memset(&w, 0, sizeof w);
    int rc = LVO_OK;

    if (p_mode != 0) { pbuf = decode(it->param, n, p_mode); w.p = pbuf; }
    else w.p = (float *)it->param;
    w.mp = it->master_param;
    if (w.mp && p_mode == 0 && (void *)w.mp == it->param) w.mp = NULL; /* worker.rs:95-98 */
    if (g_mode != 0) { gbuf = decode(it->grad, n, g_mode); w.g = gbuf; }
    else w.g = (const float *)it->grad;
    if (s_mode != 0) {
        mbuf = decode(it->exp_avg, n, s_mode);
        w.m = mbuf;
        if (it->exp_avg_sq) { vbuf = decode(it->exp_avg_sq, n, s_mode); w.v = vbuf; }
    } else {
        w.m = (float *)it->exp_avg;
        w.v = (float *)it->exp_avg_sq;
    }
    if ((p_mode != 0 && !pbuf) || (g_mode != 0 && !gbuf) || (s_mode != 0 && !mbuf) ||
        (s_mode != 0 && it->exp_avg_sq && !vbuf)) {
        rc = fail(LVO_ERR_EXEC, "out of host memory");
        goto done;
    }

    float scratch[6];
    memcpy(scratch, it->scratch, sizeof scratch);
    lvo_config item_cfg = *cfg;
    if (p_mode == 0 && w.mp == NULL) item_cfg.master_weights = 0; /* worker.rs:153-156 */
    /* The core sees the promoted state mode (worker.rs:107-113 builds the view with
     * eff_state_dtype_mode, worker.rs:141-150), so an fp16 state container never reaches the
     * core as Float16: the v <= 65000 clamp (dual.rs:68) then follows the param dtype alone. */
    rc = core_step(&item_cfg, &w, scratch, n, it->step, it->param_index, p_mode, s_mode, threads,
                   it->index_base);
    if (rc != LVO_OK) goto done;

    if (p_mode != 0) encode(it->param, pbuf, n, p_mode);
    if (s_mode != 0) {
        encode(it->exp_avg, mbuf, n, s_mode);
        if (it->exp_avg_sq) encode(it->exp_avg_sq, vbuf, n, s_mode);
    }
    memcpy(it->scratch, scratch, sizeof scratch);
done:
    free(pbuf);
    free(gbuf);
    free(mbuf);
    free(vbuf);
    return rc;
}

int lvo_step_multi(const lvo_config *cfg, const lvo_tensor *items, int count, int threads) {
    if (!cfg || (count > 0 && !items)) return fail(LVO_ERR_NULL, "null pointer");
    int rc = lvo_validate_config(cfg);
    if (rc != LVO_OK) return rc;
    for (int i = 0; i < count; i++) {
        const lvo_tensor *it = &items[i];
        if (it->numel == 0) continue;
        if (!it->param || !it->grad || !it->exp_avg || !it->scratch) return fail(LVO_ERR_NULL, "null tensor pointer");
    }
    if (threads > 1 && count > 1) {
        /* python_ffi/mod.rs:354-359: items in parallel, each item single-threaded */
        int err = LVO_OK;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
        for (int i = 0; i < count; i++) {
            if (items[i].numel == 0) continue;
            int r = process_item(cfg, &items[i], 1);
            if (r != LVO_OK) {
#pragma omp critical
                err = r;
            }
        }
        return err;
    }
    for (int i = 0; i < count; i++) {
        if (items[i].numel == 0) continue;
        rc = process_item(cfg, &items[i], threads);
        if (rc != LVO_OK) return rc;
    }
    return LVO_OK;
}
