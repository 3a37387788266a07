/*
 * AVX-512 chunk kernels of the CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A C restatement of the reference's CPU execution path, luminav-simd's AVX-512 chunk kernels
 * (optimizer/crates/luminav-simd/src/avx512/mod.rs, avx512/dual.rs, avx512/tdclm.rs): 16 lanes
 * per vector with the reference's operation order, fma placement and lane-wise radial
 * accumulation, the ragged tail of each chunk on the scalar core (as the reference's kernels
 * do). Selected with lvo_set_backend(1); only tests/ and bench.py's cpu_baseline use it.
 *
 * Per element it equals the scalar core bit for bit on finite data (the reference's own
 * differential_parity.rs property). Where the reference's two backends differ, this file follows
 * the SIMD code: a masked-off u becomes +0 (maskz_mov) where the scalar core forms u * 0 (sign of
 * zero, NaN for an infinite u); SR/RNE pass +-inf and NaN through unchanged (mod.rs:110-148)
 * where the scalar core clamps or quiets; Padé tanh propagates the input NaN (mod.rs:252-282);
 * the chunk tail's squares are added one by one to the reduced lane sum (dual.rs:232-374).
 */
#pragma GCC target("avx512f,avx512dq,avx512bw,avx512vl,fma")
#include <immintrin.h>
#include <stdint.h>

#include "luminav_oracle_internal.h"

/* avx512/mod.rs:60-77: 16 -> 8 -> 4 -> 2 -> 1 */
static inline float reduce_add(__m512 v) {
    __m256 s256 = _mm256_add_ps(_mm512_castps512_ps256(v), _mm512_extractf32x8_ps(v, 1));
    __m128 s128 = _mm_add_ps(_mm256_castps256_ps128(s256), _mm256_extractf128_ps(s256, 1));
    __m128 s64 = _mm_add_ps(s128, _mm_movehl_ps(s128, s128));
    __m128 s32 = _mm_add_ss(s64, _mm_movehdup_ps(s64));
    return _mm_cvtss_f32(s32);
}

/* avx512/mod.rs:79-86 (NaN passes: vmaxps/vminps return the second operand) */
static inline __m512 clamp_diff(__m512 v) {
    return _mm512_min_ps(_mm512_set1_ps(1.0e18f), _mm512_max_ps(_mm512_set1_ps(-1.0e18f), v));
}

/* avx512/mod.rs:88-95 */
static inline __m512 sanitize(__m512 g) {
    __mmask16 ord = _mm512_cmp_ps_mask(g, g, _CMP_ORD_Q);
    __mmask16 lt = _mm512_cmp_ps_mask(_mm512_abs_ps(g), _mm512_set1_ps(1.0e38f), _CMP_LT_OQ);
    return _mm512_maskz_mov_ps(ord & lt, clamp_diff(g));
}

/* avx512/mod.rs:97-108: the prng.rs:21-26 hash in 16 lanes */
static inline __m512i prng16(__m512i seed, __m512i off) {
    __m512i z = _mm512_add_epi32(_mm512_add_epi32(off, seed), _mm512_set1_epi32(-1640531527));
    z = _mm512_mullo_epi32(_mm512_xor_si512(z, _mm512_srai_epi32(z, 16)), _mm512_set1_epi32(-2048173461));
    z = _mm512_mullo_epi32(_mm512_xor_si512(z, _mm512_srai_epi32(z, 13)), _mm512_set1_epi32(-1028477387));
    return _mm512_xor_si512(z, _mm512_srai_epi32(z, 16));
}

/* avx512/mod.rs:110-131 */
static inline __m512 sr_bf16(__m512 p, __m512i seed, __m512i off) {
    __m512i pi = _mm512_castps_si512(p);
    __m512i a = _mm512_and_epi32(pi, _mm512_set1_epi32(0x7FFFFFFF));
    __mmask16 fin = _mm512_cmpgt_epi32_mask(_mm512_set1_epi32(0x7F800000), a);
    __m512i noise = _mm512_and_epi32(prng16(seed, off), _mm512_set1_epi32(0xFFFF));
    __m512i added = _mm512_and_epi32(_mm512_add_epi32(a, noise), _mm512_set1_epi32(~0xFFFF));
    __m512i r = _mm512_min_epi32(added, _mm512_set1_epi32(0x7F7F0000));
    __m512i sign = _mm512_and_epi32(pi, _mm512_set1_epi32(INT32_MIN));
    return _mm512_mask_blend_ps(fin, p, _mm512_castsi512_ps(_mm512_or_epi32(sign, r)));
}

/* avx512/mod.rs:133-148 */
static inline __m512 rne_bf16(__m512 p) {
    __m512i pi = _mm512_castps_si512(p);
    __m512i a = _mm512_and_epi32(pi, _mm512_set1_epi32(0x7FFFFFFF));
    __mmask16 fin = _mm512_cmpgt_epi32_mask(_mm512_set1_epi32(0x7F800000), a);
    __m512i lsb = _mm512_and_epi32(_mm512_srli_epi32(a, 16), _mm512_set1_epi32(1));
    __m512i bias = _mm512_add_epi32(_mm512_set1_epi32(0x7FFF), lsb);
    __m512i added = _mm512_and_epi32(_mm512_add_epi32(a, bias), _mm512_set1_epi32(~0xFFFF));
    __m512i r = _mm512_min_epi32(added, _mm512_set1_epi32(0x7F7F0000));
    __m512i sign = _mm512_and_epi32(pi, _mm512_set1_epi32(INT32_MIN));
    return _mm512_mask_blend_ps(fin, p, _mm512_castsi512_ps(_mm512_or_epi32(sign, r)));
}

/* avx512/mod.rs:150-196: vector SR to fp16 precision; lanes outside the fast path's range send
 * the whole vector through the scalar core (prng.rs:98-130) lane by lane. */
static inline __m512 sr_fp16(__m512 val, __m512i seed, __m512i off) {
    __m512i pi = _mm512_castps_si512(val);
    __m512i a = _mm512_and_si512(pi, _mm512_set1_epi32(0x7FFFFFFF));
    __m512i e = _mm512_and_si512(_mm512_srli_epi32(a, 23), _mm512_set1_epi32(0xFF));
    __m512i sub = _mm512_min_epi32(_mm512_max_epi32(_mm512_sub_epi32(_mm512_set1_epi32(113), e), _mm512_setzero_si512()),
                                   _mm512_set1_epi32(11));
    __m512i shift = _mm512_add_epi32(_mm512_set1_epi32(13), sub);
    __m512i one = _mm512_set1_epi32(1);
    __m512i mask_bits = _mm512_sub_epi32(_mm512_sllv_epi32(one, shift), one);
    __m512i noise = _mm512_and_si512(prng16(seed, off), mask_bits);
    __m512i not_mask = _mm512_xor_si512(mask_bits, _mm512_set1_epi32(-1));
    __m512i added = _mm512_and_si512(_mm512_add_epi32(a, noise), not_mask);
    __mmask16 not_under = _mm512_cmp_epi32_mask(e, _mm512_set1_epi32(103), _MM_CMPINT_NLT);
    __m512i r = _mm512_maskz_mov_epi32(not_under, added);
    __m512i sign = _mm512_and_si512(pi, _mm512_set1_epi32(INT32_MIN));
    __m512i out = _mm512_or_si512(sign, r);
    __m512i e_out = _mm512_srli_epi32(r, 23);
    __mmask16 valid = _mm512_cmp_epi32_mask(e, _mm512_set1_epi32(142), _MM_CMPINT_LE) &
                      _mm512_cmp_epi32_mask(e_out, _mm512_set1_epi32(142), _MM_CMPINT_LE);
    if (valid == 0xFFFF) return _mm512_castsi512_ps(out);
    float lanes[16];
    int32_t seeds[16], offs[16];
    _mm512_storeu_ps(lanes, val);
    _mm512_storeu_si512(seeds, seed);
    _mm512_storeu_si512(offs, off);
    for (int i = 0; i < 16; i++) lanes[i] = lvo_sr_fp16(lanes[i], seeds[i], offs[i]);
    return _mm512_loadu_ps(lanes);
}

/* avx512/mod.rs:198-226 */
static inline __m512 rne_fp16(__m512 val) {
    __m512i pi = _mm512_castps_si512(val);
    __m512i a = _mm512_and_si512(pi, _mm512_set1_epi32(0x7FFFFFFF));
    __m512i e = _mm512_and_si512(_mm512_srli_epi32(a, 23), _mm512_set1_epi32(0xFF));
    __m512i lsb = _mm512_and_si512(_mm512_srli_epi32(a, 13), _mm512_set1_epi32(1));
    __m512i bias = _mm512_add_epi32(_mm512_set1_epi32(0x0FFF), lsb);
    __m512i added = _mm512_and_si512(_mm512_add_epi32(a, bias), _mm512_set1_epi32(~0x1FFF));
    __mmask16 normal = _mm512_cmp_epi32_mask(e, _mm512_set1_epi32(113), _MM_CMPINT_NLT);
    __mmask16 under = _mm512_cmp_epi32_mask(e, _mm512_set1_epi32(102), _MM_CMPINT_LT);
    __m512i r = _mm512_maskz_mov_epi32(normal, added);
    __m512i sign = _mm512_and_si512(pi, _mm512_set1_epi32(INT32_MIN));
    __m512i out = _mm512_or_si512(sign, r);
    __m512i e_out = _mm512_srli_epi32(r, 23);
    __mmask16 valid = (normal | under) & _mm512_cmp_epi32_mask(e, _mm512_set1_epi32(142), _MM_CMPINT_LE) &
                      _mm512_cmp_epi32_mask(e_out, _mm512_set1_epi32(142), _MM_CMPINT_LE);
    if (valid == 0xFFFF) return _mm512_castsi512_ps(out);
    float lanes[16];
    _mm512_storeu_ps(lanes, val);
    for (int i = 0; i < 16; i++) lanes[i] = lvo_rne_fp16(lanes[i]);
    return _mm512_loadu_ps(lanes);
}

/* avx512/mod.rs:228-250 */
static inline __m512 quantize(__m512 v, __m512i seed, __m512i off, int mode, int sr) {
    if (mode == 1) return sr ? sr_bf16(v, seed, off) : rne_bf16(v);
    if (mode == 2) return sr ? sr_fp16(v, seed, off) : rne_fp16(v);
    return v;
}

/* avx512/mod.rs:252-282: [13/6] Padé with the reference's coefficients, Horner with fma */
static inline __m512 tanh_pade(__m512 x_in) {
    __m512 x = _mm512_min_ps(_mm512_set1_ps(7.9988117f), _mm512_max_ps(_mm512_set1_ps(-7.9988117f), x_in));
    __m512 x2 = _mm512_mul_ps(x, x);
    __m512 p = _mm512_fmadd_ps(_mm512_set1_ps(-2.7607684e-16f), x2, _mm512_set1_ps(2.000188e-13f));
    __m512 q = _mm512_fmadd_ps(_mm512_set1_ps(1.1982584e-6f), x2, _mm512_set1_ps(1.1853471e-4f));
    p = _mm512_fmadd_ps(p, x2, _mm512_set1_ps(-8.604672e-11f));
    q = _mm512_fmadd_ps(q, x2, _mm512_set1_ps(2.2684346e-3f));
    p = _mm512_fmadd_ps(p, x2, _mm512_set1_ps(5.122297e-8f));
    q = _mm512_fmadd_ps(q, x2, _mm512_set1_ps(4.8935246e-3f));
    p = _mm512_fmadd_ps(p, x2, _mm512_set1_ps(1.4857224e-5f));
    p = _mm512_fmadd_ps(p, x2, _mm512_set1_ps(6.3726193e-4f));
    p = _mm512_fmadd_ps(p, x2, _mm512_set1_ps(4.8935246e-3f));
    return _mm512_div_ps(_mm512_mul_ps(x, p), q);
}

/* avx512/mod.rs:284-294 */
static inline __m512 coordinate_bound(__m512 step, __m512 p_init, __m512 ratio) {
    __m512 bi = _mm512_mul_ps(ratio, _mm512_sqrt_ps(_mm512_fmadd_ps(p_init, p_init, _mm512_set1_ps(1.0e-4f))));
    return _mm512_mul_ps(bi, tanh_pade(_mm512_div_ps(step, bi)));
}

/* avx512/mod.rs:296-309 */
static inline __m512 coordinate_bound_t2(__m512 step, __m512 p_init, __m512 ratio) {
    __m512 bi = _mm512_mul_ps(ratio, _mm512_add_ps(_mm512_abs_ps(p_init), _mm512_set1_ps(1.0e-2f)));
    __m512 bb = _mm512_mul_ps(bi, _mm512_add_ps(bi, _mm512_abs_ps(step)));
    return _mm512_div_ps(_mm512_mul_ps(bb, step), _mm512_fmadd_ps(step, step, bb));
}

/* avx512/mod.rs:311-333 */
static inline __m512 fp16_safety_bound(__m512 step, __m512 p_init, int triangle) {
    __m512 bs = _mm512_max_ps(_mm512_mul_ps(_mm512_abs_ps(p_init), _mm512_set1_ps(0.01f)), _mm512_set1_ps(1.5e-4f));
    if (!triangle) return _mm512_mul_ps(bs, tanh_pade(_mm512_div_ps(step, bs)));
    __m512 bb = _mm512_mul_ps(bs, _mm512_add_ps(bs, _mm512_abs_ps(step)));
    return _mm512_div_ps(_mm512_mul_ps(bb, step), _mm512_fmadd_ps(step, step, bb));
}

/* u of 16 lanes; m_new / v_new for the apply path: the u computation of the chunk kernels
 * (CLM and T2 in avx512/dual.rs:29-374, TD-CLM and T1 in avx512/tdclm.rs:27-286). */
static inline __m512 compute_u16(const coef_t *k, __m512 g, __m512 m, __m512 v, __m512 *m_new, __m512 *v_new) {
    __m512 g_scaled = _mm512_mul_ps(_mm512_set1_ps(k->omb1), g);
    *m_new = _mm512_fmadd_ps(_mm512_set1_ps(k->b1), m, g_scaled);
    *v_new = _mm512_setzero_ps();
    if (k->mode == 2) {
        __m512 clm = _mm512_fmadd_ps(_mm512_set1_ps(k->b1), *m_new, g_scaled);
        __m512 diff = clamp_diff(_mm512_sub_ps(g, *m_new));
        __m512 vn = _mm512_fmadd_ps(_mm512_set1_ps(k->b2), v, _mm512_mul_ps(_mm512_set1_ps(k->omb2), _mm512_mul_ps(diff, diff)));
        if (k->clamp_v) vn = _mm512_min_ps(vn, _mm512_set1_ps(65000.0f));
        *v_new = vn;
        __m512 sigma = _mm512_fmadd_ps(_mm512_sqrt_ps(_mm512_max_ps(vn, _mm512_setzero_ps())), _mm512_set1_ps(k->c1),
                                       _mm512_set1_ps(k->c2));
        return tanh_pade(_mm512_div_ps(clm, _mm512_max_ps(sigma, _mm512_set1_ps(1.0e-12f))));
    }
    __m512 clm = _mm512_fmadd_ps(_mm512_set1_ps(k->b1sq), m, _mm512_mul_ps(_mm512_set1_ps(k->omb1sq), g));
    __m512 diff = clamp_diff(_mm512_sub_ps(g, m));
    __m512 env0 = _mm512_fmadd_ps(_mm512_set1_ps(k->b1sq), _mm512_abs_ps(m), _mm512_set1_ps(k->eps));
    __m512 env1 = _mm512_fmadd_ps(_mm512_set1_ps(k->omb1sq), _mm512_abs_ps(g), env0);
    if (k->mode == 4) {
        __m512 vn = _mm512_fmadd_ps(_mm512_set1_ps(k->b2), v, _mm512_mul_ps(_mm512_set1_ps(k->omb2), _mm512_mul_ps(diff, diff)));
        if (k->clamp_v) vn = _mm512_min_ps(vn, _mm512_set1_ps(65000.0f));
        *v_new = vn;
        __m512 env2 = _mm512_fmadd_ps(_mm512_set1_ps(k->lam1), _mm512_abs_ps(diff), env1);
        __m512 env = _mm512_fmadd_ps(_mm512_set1_ps(k->c_sigma), _mm512_sqrt_ps(_mm512_max_ps(vn, _mm512_setzero_ps())), env2);
        return _mm512_div_ps(clm, env);
    }
    __m512 env = _mm512_fmadd_ps(_mm512_set1_ps(k->lam), _mm512_abs_ps(diff), env1);
    return _mm512_div_ps(clm, env);
}

/* avx512/mod.rs:335-342: (int32)(chunk_offset + i) + lane, wrapping */
static inline __m512i offsets16(uint32_t base) {
    return _mm512_add_epi32(_mm512_set1_epi32((int32_t)base),
                            _mm512_set_epi32(15, 14, 13, 12, 11, 10, 9, 8, 7, 6, 5, 4, 3, 2, 1, 0));
}

/*
 * One chunk [start, end). apply = 1: dual_single_pass_chunk_avx512 / dual_pass2_chunk_avx512
 * (avx512/dual.rs:29-374, 555-854) and tdclm_single_pass_chunk_avx512 / tdclm_pass2_chunk_avx512
 * (avx512/tdclm.rs:27-286, 398-614); apply = 0: dual_pass1_chunk_avx512 (avx512/dual.rs:376-553)
 * and tdclm_pass1_chunk_avx512 (avx512/tdclm.rs:288-396).
 */
chunk_metrics lvo_i_avx512_chunk(const coef_t *k, const view_t *w, uint64_t start, uint64_t end, int apply,
                                 float cs, float bs) {
    chunk_metrics cm = {0, 0.0f, 0.0f, 0.0, 0.0};
    const uint64_t len = end - start;
    const uint64_t simd_len = len & ~15ull;
    const int radial = k->bound == 1;
    const __m512 zero = _mm512_setzero_ps();
    const __m512i seed_m = _mm512_set1_epi32(k->seed_m), seed_p = _mm512_set1_epi32(k->seed_p),
                  seed_v = _mm512_set1_epi32(k->seed_v);
    __m512 acc_u = zero, acc_p = zero;
    for (uint64_t i = 0; i < simd_len; i += 16) {
        const uint64_t idx = start + i;
        const __m512 g = sanitize(_mm512_loadu_ps(w->g + idx));
        const __m512 m = _mm512_loadu_ps(w->m + idx);
        const __m512 v = k->dual_state ? _mm512_loadu_ps(w->v + idx) : zero;
        __m512 m_new, v_new;
        const __m512 u = compute_u16(k, g, m, v, &m_new, &v_new);
        const __mmask16 act = _mm512_cmp_ps_mask(_mm512_mul_ps(u, g), zero, _CMP_GT_OQ);
        const __m512 u_masked = _mm512_maskz_mov_ps(act, u);
        __m512 p_init;
        if (apply || radial) p_init = _mm512_loadu_ps((k->has_master ? w->mp : w->p) + idx);
        else p_init = zero;
        if (apply) {
            const __m512i off = offsets16((uint32_t)(k->index_base + idx));
            _mm512_storeu_ps(w->m + idx, quantize(m_new, seed_m, off, k->s_mode, k->sr));
            if (k->dual_state) _mm512_storeu_ps(w->v + idx, quantize(v_new, seed_v, off, k->s_mode, k->sr));
            const __m512 delta = k->cautious ? _mm512_mul_ps(u_masked, _mm512_set1_ps(cs)) : u;
            __m512 step = _mm512_mul_ps(_mm512_set1_ps(k->lr), delta);
            if (k->bound == 1) step = _mm512_mul_ps(step, _mm512_set1_ps(bs));
            else if (k->bound == 2)
                step = k->triangle ? coordinate_bound_t2(step, p_init, _mm512_set1_ps(k->ratio))
                                   : coordinate_bound(step, p_init, _mm512_set1_ps(k->ratio));
            if (k->fp16_param) step = fp16_safety_bound(step, p_init, k->triangle);
            const __m512 p_dec = k->wd_nonzero ? _mm512_fnmadd_ps(_mm512_set1_ps(k->lr_wd), p_init, p_init) : p_init;
            const __m512 p_upd = _mm512_sub_ps(p_dec, step);
            if (k->has_master) {
                _mm512_storeu_ps(w->mp + idx, p_upd);
                _mm512_storeu_ps(w->p + idx, quantize(p_upd, seed_p, off, k->p_mode, 0));
            } else {
                _mm512_storeu_ps(w->p + idx, quantize(p_upd, seed_p, off, k->p_mode, k->sr));
            }
        }
        if (k->cautious) cm.mask += (uint64_t)__builtin_popcount((unsigned)act);
        if (radial) {
            const __m512 ue = k->cautious ? u_masked : u;
            acc_u = _mm512_add_ps(acc_u, _mm512_mul_ps(ue, ue));
            acc_p = _mm512_add_ps(acc_p, _mm512_mul_ps(p_init, p_init));
        }
    }
    if (radial) {
        cm.u_sq = reduce_add(acc_u);
        cm.p_sq = reduce_add(acc_p);
    }
    for (uint64_t idx = start + simd_len; idx < end; idx++) {
        float usq = 0.0f, psq = 0.0f;
        int act = apply ? lvo_i_apply_elem(k, w, idx, cs, bs, radial ? &usq : NULL, &psq)
                        : lvo_i_count_elem(k, w, idx, radial ? &usq : NULL, &psq);
        if (k->cautious && act) cm.mask += 1;
        if (radial) {
            cm.u_sq += usq;
            cm.p_sq += psq;
        }
    }
    return cm;
}
