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

/* Workspace. lv_step_multi needs caller-owned device memory, 256-byte aligned, ZERO-FILLED before
 * its first use; every call leaves all of it zero again (the kernels re-zero the cautious count
 * slots and tickets they use, and the radial fold zeroes every record it reads), so one workspace
 * serves every later call, whatever its tensors or options. Calls that share a workspace are
 * ordered by the library: a call on another stream than the workspace's previous call first
 * waits for that call (an event the library records after it; after a call on the NULL stream the
 * event is recorded only when another stream needs it). One host thread at a time may call with a
 * given workspace. After a call that returned LV_STATUS_EXECUTION_FAILED (a launch failed
 * part-way), zero it again before reusing it.
 * Layout of one call: 195 KiB of inline count slots (48 tensors x 65 slots x 64 B) and 2 KiB of
 * radial tickets and running sums; with more than 48 tensors in a launch class, table count
 * slots (per tensor, one fold slot plus the smallest power of two of slots that keeps every slot
 * at <= 64 blocks, at most 64; 64 B each); with the radial bound,
 * 32 B of chunk record per 4096 units and 20 B of unit record per unit, up to one piece of 2^22
 * units (80 MiB). No radial space is needed without the radial bound. */

/* Bytes of workspace any call with n_tensors tensors can need (64 count slots per tensor and a
 * full radial piece: an upper bound for callers that do not inspect their tensors). */
size_t lv_workspace_bytes(int n_tensors);

/* Bytes of workspace this call needs (the same arguments as lv_step_multi; step counters and
 * pointers do not matter, only the sizes, the count and whether the radial bound is on). */
size_t lv_workspace_bytes_for(const lv_config *cfg, const lv_tensor *tensors, int count);

/*
 * One optimizer step over `count` tensors, in place, asynchronous on `stream`.
 * Replaces the reference's GPU seam LuminaVGpuMixin._step_gpu_group
 * (python/luminamoon/optimizer/gpu_backend.py:2603-2733) and the CPU seam
 * step_pyo3 -> process_work_item (optimizer/src/python_ffi/mod.rs:201-391,
 * optimizer/src/python_ffi/worker.rs:77-179) with one multi-tensor launch (pair) per
 * (dtype, step, pass) class instead of one launch per tensor: up to 48 tensors in the kernel
 * arguments, any number above that from a descriptor table in device memory. The tables belong to
 * the library (a small ring per device, allocated on first use and grown when a call needs more);
 * a call whose table equals one already on the device launches with no upload.
 * Validation follows step_pyo3 (mod.rs:57-173): null pointers (-1), dtype codes, master and
 * exp_avg_sq presence, and pointer aliasing (-3 with the reference's "Pointer aliasing detected"
 * messages): no param, exp_avg, exp_avg_sq, master_param or scratch buffer may appear twice or
 * overlap another, and no grad may overlap any of them.
 * Returns LV_STATUS_* ; lv_last_error() describes a failure.
 */
int lv_step_multi(const lv_config *cfg, const lv_tensor *tensors, int count,
                  void *workspace, size_t workspace_bytes, void *stream);

/*
 * Graph-capture-safe stepping (the reference keeps per-parameter scratch pointers stable for CUDA
 * graph capture, changelogs/LUMINAV_ALGORITHM_CHANGELOG.md:283-284; its kernels still take the
 * step count and coefficients as launch arguments). lv_step_multi_graph takes the step count
 * from a caller-owned record in DEVICE memory instead: each call first advances record->step on
 * the device and writes that step's bias-correction coefficients and seed base into the record
 * (a one-thread kernel, the same f64 arithmetic as the host path), then runs lv_step_multi's
 * launches reading them from there. So a HIP graph captured around a call replays one correct
 * step per replay. The call uses inline launches only (no descriptor upload, no event, no memset,
 * no allocation); the tensors' `step` fields are ignored: every tensor of the call shares the
 * record's count. Passes are those of a step >= 2: with cautious or radial and the fused single
 * pass, a first step (record->step == 0 before the call) is refused on the device (status 1, the
 * counter and every buffer unchanged); take it through lv_step_multi and set record->step to 1.
 * Results are bit for bit lv_step_multi's for the same step counts. Workspace: as lv_step_multi
 * without table count slots, but the library does not order these calls across streams (a
 * capturing stream cannot wait on an event recorded outside its capture): calls that share a
 * workspace must be ordered by the caller, e.g. one workspace per set of tensors stepped
 * together, as the tensors themselves require.
 */
typedef struct lv_step_record {
    uint64_t step;          /* steps taken; each call adds one on the device before stepping */
    float c1, c2, c_sigma;  /* written by each call: its step's coefficients (math.rs:27-81) */
    uint32_t seed_base;     /* written by each call: seed + step * 0x9E3779B9 (prng.rs:4-13) */
    uint32_t status;        /* 0, or 1 when the last call refused a first step */
    uint32_t reserved;
} lv_step_record;

int lv_step_multi_graph(const lv_config *cfg, const lv_tensor *tensors, int count, lv_step_record *record,
                        void *workspace, size_t workspace_bytes, void *stream);

/*
 * lv_step_multi without allocation: no counterpart in the reference. For callers that cannot
 * allocate device memory -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc. Same arguments, validation, launches and results (bit for bit) as
 * lv_step_multi, with no workspace argument: it uses a scratch array the library holds on each
 * device (1,514,496 bytes, kept until the process ends) and calls no allocating routine.
 * Limits, refused with LV_STATUS_INVALID_CONFIG: at most 256 tensors per call, and radial-bound
 * counting launches of at most 65,536 work units (about 67M elements with fp32 state). Classes
 * above 48 tensors run as several inline launches (no descriptor tables). Every call on a device
 * shares that device's array: calls that overlap in time on one device (two streams, two host
 * threads) race and must not be issued; stream-ordered calls are fine. Each call leaves the array
 * zero; after a call that failed part-way the next call clears it first.
 */
int lv_step_multi_noalloc(const lv_config *cfg, const lv_tensor *tensors, int count, void *stream);

/*
 * Single fp32 tensor step with luminav_triton_step_f32's argument mapping
 * (optimizer/crates/luminav-triton-aot/src/c_api.rs:108-199): buffer_mode 1 is TD-CLM and every
 * other value the dual buffer (c_api.rs:143-146); exp_avg_sq is used only when buffer_mode == 2
 * (c_api.rs:120-124), so any other dual-buffer call fails; bound_mode 1 radial, 2 coordinate,
 * anything else no bound; master weights iff master_param != NULL; cautious_clamp_min 0.5,
 * ema_decay the buffer mode's default, stochastic rounding off, fused single pass on; status -1
 * for a null param/grad/exp_avg/scratch and -4 for every other failure (c_api.rs:178-181).
 * The one deliberate difference: device pointers and a stream instead of the engine and host
 * buffers (luminav_triton_step_f32 below takes those). The step runs like lv_step_multi's (the
 * reference CPU core's pass selection). Uses an internal per-device workspace allocated on first
 * use: calls on one device share it, and a call on another stream than the previous one waits for
 * it (as lv_step_multi's workspace ordering).
 */
int lv_step_f32(float *param, const float *grad, float *exp_avg, float *exp_avg_sq,
                float *master_param, float *scratch, size_t num_elements, float lr, float beta1,
                float beta2, float eps, float weight_decay, float tau, float lam, int buffer_mode,
                int cautious, int bound_mode, float bound_ratio, uint64_t step, uint32_t seed,
                void *stream);

/*
 * The reference's standalone C API (optimizer/include/luminav_triton_standalone.h:21-111,
 * optimizer/crates/luminav-triton-aot/src/c_api.rs:9-199), same names, signatures and status
 * codes, so a C program written against that header links against this library unchanged.
 * luminav_triton_engine_create: the current HIP device and a stream of its own; NULL when no
 * device is present. get_platform: "rocm" ("none" for NULL). get_arch: the device's gfx name,
 * e.g. "gfx950" ("unknown" for NULL). luminav_triton_step_f32 takes HOST buffers: it copies
 * them to the device, steps as lv_step_f32 does, copies param, exp_avg, exp_avg_sq (mode 2),
 * master_param and scratch back and returns when done. Calls on one engine are serialised.
 */
typedef struct LuminaVTritonEngine LuminaVTritonEngine;
LuminaVTritonEngine *luminav_triton_engine_create(void);
void luminav_triton_engine_destroy(LuminaVTritonEngine *engine);
const char *luminav_triton_get_platform(const LuminaVTritonEngine *engine);
const char *luminav_triton_get_arch(const LuminaVTritonEngine *engine);
int luminav_triton_step_f32(LuminaVTritonEngine *engine, float *param, const float *grad,
                            float *exp_avg, float *exp_avg_sq, float *master_param, float *scratch,
                            size_t num_elements, float lr, float beta1, float beta2, float eps,
                            float weight_decay, float tau, float lam, int buffer_mode, int cautious,
                            int bound_mode, float bound_ratio, uint64_t step, uint32_t seed);

/* Description of the last error on this thread ("" if none). */
const char *lv_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* LUMINAV_HIP_H */
