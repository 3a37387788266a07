/*
 * Internal interface between the scalar oracle (luminav_oracle.c) and its AVX-512 chunk
 * backend (luminav_oracle_avx512.c) -- TEST INFRASTRUCTURE ONLY, like the rest of oracle/.
 */
#ifndef LUMINAV_ORACLE_INTERNAL_H
#define LUMINAV_ORACLE_INTERNAL_H

#include <stdint.h>

#include "luminav_oracle.h"

/* Per-tensor, per-step constants of the element update. */
typedef struct {
    int mode;        /* 1 TD-CLM, 2 CLM, 3 T1, 4 T2 */
    int triangle;    /* T1 / T2: rational coordinate bound */
    int dual_state;  /* CLM / T2: exp_avg_sq present */
    int clamp_v;     /* fp16 param or fp16 state: v <= 65000 */
    int fp16_param;
    int cautious, sr, bound, has_master, wd_nonzero;
    int p_mode, s_mode;
    float lr, b1, b2, omb1, omb2, b1sq, omb1sq, lam, lam1, eps, c1, c2, c_sigma, lr_wd, ratio;
    int32_t seed_m, seed_p, seed_v;
    uint64_t index_base;
} coef_t;

/* Decoded f32 views of one tensor (worker.rs:35-53 decodes 16-bit buffers to f32 first). */
typedef struct {
    float *p;           /* decoded f32 param */
    float *mp;          /* master or NULL */
    const float *g;     /* decoded f32 grad */
    float *m;
    float *v;           /* NULL for TD-CLM / T1 */
} view_t;

/* ChunkMetrics (avx512/mod.rs:32-48) plus the f64 sums of the checker's f64 radial mode. */
typedef struct {
    uint64_t mask;
    float u_sq, p_sq;
    double du, dp;
} chunk_metrics;

/* Scalar element update / count of the scalar core; the SIMD chunk kernels use them for the
 * ragged tail of a chunk, as the reference's do (e.g. avx512/dual.rs:253-355). */
int lvo_i_apply_elem(const coef_t *k, const view_t *w, uint64_t idx, float cs, float bs, float *u_sq_out,
                     float *p_sq_out);
int lvo_i_count_elem(const coef_t *k, const view_t *w, uint64_t idx, float *u_sq_out, float *p_sq_out);

/* 1 when the CPU has avx512f/dq/bw/vl and fma (luminav-simd/src/lib.rs:38-60). */
int lvo_i_cpu_has_avx512(void);

/* One chunk [start, end) of a pass with the reference's AVX-512 kernels: apply = 1 is
 * *_single_pass_chunk_avx512 / *_pass2_chunk_avx512 (update and store; metrics accumulated),
 * apply = 0 is *_pass1_chunk_avx512 (count only). */
chunk_metrics lvo_i_avx512_chunk(const coef_t *k, const view_t *w, uint64_t start, uint64_t end, int apply,
                                 float cs, float bs);

#endif
