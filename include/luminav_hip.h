/*
 * luminav_hip.h -- C ABI of the MI355X-native LuminaV optimizer step (libluminav_hip.so).
 *
 * Plain pointers and sizes only. Every tensor pointer is a device (HBM) pointer on the
 * current HIP device; `stream` is a hipStream_t passed as void* (NULL = default stream).
 * All calls are asynchronous on `stream`: no host synchronisation, no allocation on the
 * steady-state path.
 *
 * Codes follow the reference enums:
 *   buffer       1 TD-CLM, 2 CLM (dual), 3 T1, 4 T2  (optimizer/crates/luminav-core/src/config.rs:54-59)
 *   bound_type   0 none, 1 radial, 2 coordinate        (config.rs:128-132)
 *   master       0 none, 1 semi, 2 full                 (config.rs:170-174)
 *   dtype        0 f32, 1 bf16, 2 f16                   (config.rs:217-221)
 * Status codes are the reference's (optimizer/include/luminav_triton_standalone.h:25-29).
 */
#ifndef LUMINAV_HIP_H
#define LUMINAV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LV_STATUS_SUCCESS 0
#define LV_STATUS_NULL_POINTER -1
#define LV_STATUS_NO_DRIVER -2
#define LV_STATUS_INVALID_CONFIG -3
#define LV_STATUS_EXECUTION_FAILED -4

#define LV_BUFFER_TDCLM 1
#define LV_BUFFER_DUAL 2
#define LV_BUFFER_T1 3
#define LV_BUFFER_T2 4

#define LV_BOUND_NONE 0
#define LV_BOUND_RADIAL 1
#define LV_BOUND_COORDINATE 2

#define LV_DTYPE_F32 0
#define LV_DTYPE_BF16 1
#define LV_DTYPE_F16 2

/* Hyper-parameters; mirrors LuminaVConfig (optimizer/crates/luminav-core/src/config.rs:274-295)
 * minus the host-only fields (execution, fsdp_sync). Floats are the f32 values the reference
 * parses (optimizer/src/python_ffi/config_parser.rs:9-199). */
typedef struct lv_config {
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
} lv_config;

/* One tensor (or one fused bucket). Mirrors a step_pyo3 work item
 * (optimizer/src/python_ffi/worker.rs:7-21): exp_avg_sq is NULL for buffer 1/T1, master_param
 * is NULL without master weights, scratch is the 6-float per-tensor ScratchBuffer
 * (luminav-core/src/state.rs:4-117). step is the already-incremented step count. */
typedef struct lv_tensor {
    void *param;
    const void *grad;
    void *exp_avg;
    void *exp_avg_sq;
    float *master_param;
    float *scratch;
    uint64_t numel;
    uint64_t step;
    uint64_t param_index;
    int32_t param_dtype;
    int32_t grad_dtype;
    int32_t state_dtype;
    int32_t reserved;
    /* Element i uses stochastic-rounding offset (int32)(index_base + i). 0 for a whole tensor
     * (the reference's `idx as i32`, reference_cpu/dual.rs:54); a shard of a larger tensor passes
     * its global start so its bits equal the unsharded step. */
    uint64_t index_base;
    /* Optional inactive element ranges: `inactive` points to 2 x n_inactive uint64 values in
     * device memory, sorted and disjoint [begin, end) pairs of element indices of this tensor.
     * Their elements count in the cautious / radial statistics as if their gradient were zero,
     * but are never written (param, state and master keep their values) and their grad is not
     * read. This is the reference's grad=None slice of a fused bucket -- zero the grad slice,
     * step the whole bucket, restore the slice (python/luminamoon/optimizer/luminav.py:1466-1531,
     * luminav.py:1585-1603) -- without the copies. NULL / 0: every element is active. */
    const uint64_t *inactive;
    uint64_t n_inactive;
} lv_tensor;

/* Library version, major*10000 + minor*100 + patch. */
int lv_version(void);

/* Bytes of device workspace lv_step_multi needs for a call with n_tensors tensors (the launches
 * of a call reuse per-launch regions): 195 KiB of cautious mask-count words (48 tensors per
 * launch x 65 words x 64 bytes) and 512 bytes of radial-fold tickets, which must be zero before a
 * call, then 35 KiB of radial running sums and chunk records and 80 MiB of radial unit records
 * (one launch piece of 2^22 units x 20 bytes), which need no clearing. Above 48 tensors, table
 * launches (up to 960 tensors each) add 3.8 MiB of count words, which must be zero, and a 75 KiB
 * descriptor table. The caller allocates it once,
 * zero-filled; the kernels leave the count words and tickets zeroed again after every call, so it
 * is reused from step to step. Calls that share one workspace must not overlap. After a call
 * that returned LV_STATUS_EXECUTION_FAILED (a launch failed part-way), zero the workspace again
 * before reusing it. */
size_t lv_workspace_bytes(int n_tensors);

/*
 * One optimizer step over `count` tensors, in place, asynchronous on `stream`.
 * Replaces the reference's GPU seam LuminaVGpuMixin._step_gpu_group
 * (python/luminamoon/optimizer/gpu_backend.py:2603-2733) and the CPU seam
 * step_pyo3 -> process_work_item (optimizer/src/python_ffi/mod.rs:201-391,
 * optimizer/src/python_ffi/worker.rs:77-179) with one multi-tensor launch per
 * (dtype, step, pass) class instead of one launch per tensor.
 * Returns LV_STATUS_* ; lv_last_error() describes a failure.
 */
int lv_step_multi(const lv_config *cfg, const lv_tensor *tensors, int count,
                  void *workspace, size_t workspace_bytes, void *stream);

/*
 * Single fp32 tensor step on device pointers, argument-for-argument the reference's
 * luminav_triton_step_f32 (optimizer/include/luminav_triton_standalone.h:89-111) without the
 * engine handle; ema_decay is the reference default for the buffer mode, cautious_clamp_min
 * 0.5, stochastic rounding and fused single pass on (config.rs:297-321). Uses an internal
 * per-device workspace allocated on first use: calls on one device share it, so calls on
 * different streams must not overlap in time (stream-ordered calls on one stream are fine).
 */
int lv_step_f32(float *param, const float *grad, float *exp_avg, float *exp_avg_sq,
                float *master_param, float *scratch, size_t num_elements, float lr, float beta1,
                float beta2, float eps, float weight_decay, float tau, float lam, int buffer_mode,
                int cautious, int bound_mode, float bound_ratio, uint64_t step, uint32_t seed,
                void *stream);

/* Description of the last error on this thread ("" if none). */
const char *lv_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* LUMINAV_HIP_H */
