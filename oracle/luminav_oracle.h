/*
 * CPU oracle for the LuminaV optimizer step -- TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference's Rust CPU implementation
 * (optimizer/crates/luminav-core + optimizer/src/python_ffi/worker.rs) used as
 * the parity checker for the HIP product path and as the timed CPU baseline in
 * bench.py.  Nothing in luminamoon_amd/ may link, load or call it; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg do.
 *
 * Layout of the structs is the oracle's own; codes follow the reference enums:
 *   buffer       1 TD-CLM, 2 CLM (dual), 3 T1, 4 T2   (luminav-core/src/config.rs:54-59)
 *   bound_type   0 none, 1 radial, 2 coordinate         (config.rs:128-132)
 *   master       0 none, 1 semi, 2 full                  (config.rs:170-174)
 *   dtype        0 f32, 1 bf16, 2 f16                    (config.rs:217-221)
 */
#ifndef LUMINAV_ORACLE_H
#define LUMINAV_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lvo_config {
    float lr, beta1, beta2, eps, weight_decay, tau, lam;
    float cautious_clamp_min, bound_ratio, ema_decay;
    int32_t buffer;
    int32_t cautious;
    int32_t stochastic_rounding;
    int32_t bound;
    int32_t bound_type;
    int32_t master_weights;
    int32_t fused_single_pass;
    uint32_t seed;
} lvo_config;

/* One work item, host pointers (worker.rs:7-21). exp_avg_sq / master_param may be NULL. */
typedef struct lvo_tensor {
    void *param;
    const void *grad;
    void *exp_avg;
    void *exp_avg_sq;
    float *master_param;
    float *scratch;          /* float[6] */
    uint64_t numel;
    uint64_t step;
    uint64_t param_index;
    int32_t param_dtype;
    int32_t grad_dtype;
    int32_t state_dtype;
    int32_t reserved;
    /* Checker-only extension: element i of this item uses SR offset (i32)(index_base + i), so a
     * slice [a, b) of a larger tensor can be re-run on its own (index_base = a). The reference
     * always starts at 0 (reference_cpu/dual.rs:54). */
    uint64_t index_base;
} lvo_tensor;

/* status codes */
#define LVO_OK 0
#define LVO_ERR_NULL (-1)
#define LVO_ERR_CONFIG (-3)
#define LVO_ERR_EXEC (-4)

/* scalar primitives (exported so the tests can pin each one) */
int32_t lvo_prng(int32_t seed, int32_t idx);
void lvo_derive_kernel_seeds(uint32_t seed, uint64_t step, uint64_t param_index,
                             int32_t *seed_m, int32_t *seed_p);
int32_t lvo_derive_variance_seed(int32_t seed_m);
float lvo_sanitize_gradient(float g);
float lvo_tanh_pade(float x);
uint16_t lvo_f32_to_f16_bits_rne(float v);
float lvo_f16_bits_to_f32(uint16_t bits);
uint16_t lvo_sr_fp16_bits(float v, int32_t seed, int32_t offset);
float lvo_sr_fp16(float v, int32_t seed, int32_t offset);
float lvo_rne_fp16(float v);
uint16_t lvo_sr_bf16_bits(float v, int32_t seed, int32_t offset);
float lvo_sr_bf16(float v, int32_t seed, int32_t offset);
float lvo_rne_bf16(float v);
float lvo_quantize(float v, int32_t seed, int32_t offset, int32_t dtype, int32_t use_sr);
/* out[5] = {bc1_nes, bc2, c1, c2, effective_eps} */
void lvo_bias_correction(uint64_t step, float beta1, float beta2, float eps, float tau, float *out);
float lvo_t2_sigma_coeff(uint64_t step, float beta2, float lam);
double lvo_powi(double a, int32_t b);
float lvo_cautious_scale(float mask_sum, float total, float clamp_min);
float lvo_radial_scale(float u_sq, float p_sq, float cs, float lr, float ratio);
float lvo_radial_scale_t2(float u_sq, float p_sq, float cs, float lr, float ratio);
float lvo_coordinate_bound(float step, float p_init, float ratio);
float lvo_coordinate_bound_t2(float step, float p_init, float ratio);
float lvo_fp16_safety_bound(float step, float p_init);
float lvo_fp16_safety_bound_t2(float step, float p_init);
void lvo_update_post_step_ema(float *scratch, float total, const lvo_config *cfg, int32_t triangle);
float lvo_u64_to_f32(uint64_t x);

/* Radial-bound sum mode (checker option): 0 (default) = the scalar core's f32 16-lane / chunk
 * order (reference_cpu/dual.rs:134-253, parallel/dual.rs:192-200); 1 = each f32 square added
 * in f64 and rounded to f32 once (the HIP kernels' order-independent sum). Process-global. */
void lvo_set_radial_sum_mode(int32_t mode);
int32_t lvo_radial_sum_mode(void);

/* Chunk backend, process-global: 0 (default) = the scalar core (luminav-core reference_cpu,
 * what the HIP kernels are checked against bit for bit); 1 = the restatement of the reference's
 * AVX-512 chunk kernels (luminav-simd/src/avx512/{mod,dual,tdclm}.rs), its CPU execution path.
 * Returns LVO_OK, or LVO_ERR_EXEC when the CPU lacks avx512f/dq/bw/vl + fma. */
int32_t lvo_set_backend(int32_t backend);
int32_t lvo_backend(void);

/* Validate like LuminaVConfig::validate (config.rs:329-366). Returns LVO_OK or LVO_ERR_CONFIG. */
int lvo_validate_config(const lvo_config *cfg);

/*
 * Step `count` work items in place, exactly like step_pyo3 -> process_work_item ->
 * single_step_*_scalar (python_ffi/mod.rs:201-391, worker.rs:77-179).
 * threads <= 1: one thread, item after item (scalar core).
 * threads  > 1: items in parallel when count > 1, else 2,097,152-element chunks in
 *               parallel (luminav-simd/src/lib.rs:62-150, parallel/mod.rs:7); per-element
 *               results are identical to threads == 1.
 */
int lvo_step_multi(const lvo_config *cfg, const lvo_tensor *items, int count, int threads);

const char *lvo_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
