// VALU issue rates on gfx950 for the instructions on the update's hot paths: each kernel runs 8
// independent chains per lane of one instruction (inline asm, so nothing is folded or reordered;
// the compare + select kernel chains the pair and is timed per pair), 256 per loop iteration,
// with 8 blocks of 4 waves per CU (8 waves per SIMD). The time per wave instruction per SIMD,
// relative to v_add_u32's, is the instruction's issue cost. Only VALU instructions on registers: no memory access but one store per lane at the
// end. Test infrastructure: built by __graft_entry__.build() into tests/gpu_checks/libissuerate.so
// and run by tests/test_gpu_issue_rate.py.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

#define LV_RATE_KERNEL(NAME, ASM, ...)                                                                 \
    __global__ void __launch_bounds__(256) NAME(uint32_t *out, int iters, uint32_t seed) {          \
        uint32_t a0 = seed + threadIdx.x, a1 = a0 * 3u, a2 = a0 * 5u, a3 = a0 * 7u;                  \
        uint32_t a4 = a0 ^ 0x3f800000u, a5 = a1 ^ 0x3f800000u, a6 = a2 ^ 0x3f800000u, a7 = a3 ^ 0x3f800000u; \
        const uint32_t b = 0x3f812345u + blockIdx.x, c = 0x3f7edcbau;                               \
        for (int i = 0; i < iters; i++) {                                                           \
            _Pragma("unroll") for (int k = 0; k < 32; k++) {                                        \
                asm volatile(ASM : "+v"(a0) : "v"(b), "v"(c) __VA_ARGS__);                           \
                asm volatile(ASM : "+v"(a1) : "v"(b), "v"(c) __VA_ARGS__);                           \
                asm volatile(ASM : "+v"(a2) : "v"(b), "v"(c) __VA_ARGS__);                           \
                asm volatile(ASM : "+v"(a3) : "v"(b), "v"(c) __VA_ARGS__);                           \
                asm volatile(ASM : "+v"(a4) : "v"(b), "v"(c) __VA_ARGS__);                           \
                asm volatile(ASM : "+v"(a5) : "v"(b), "v"(c) __VA_ARGS__);                           \
                asm volatile(ASM : "+v"(a6) : "v"(b), "v"(c) __VA_ARGS__);                           \
                asm volatile(ASM : "+v"(a7) : "v"(b), "v"(c) __VA_ARGS__);                           \
            }                                                                                       \
        }                                                                                           \
        out[blockIdx.x * 256 + threadIdx.x] = a0 ^ a1 ^ a2 ^ a3 ^ a4 ^ a5 ^ a6 ^ a7;                 \
    }

LV_RATE_KERNEL(r_add_u32, "v_add_u32 %0, %0, %1")
LV_RATE_KERNEL(r_sub_u32, "v_sub_u32 %0, %0, %1")
LV_RATE_KERNEL(r_and_b32, "v_and_b32 %0, %0, %1")
LV_RATE_KERNEL(r_or_b32, "v_or_b32 %0, %0, %1")
LV_RATE_KERNEL(r_xor_b32, "v_xor_b32 %0, %0, %1")
LV_RATE_KERNEL(r_lshrrev_b32, "v_lshrrev_b32 %0, %1, %0")
LV_RATE_KERNEL(r_ashrrev_i32, "v_ashrrev_i32 %0, %1, %0")
LV_RATE_KERNEL(r_mov_b32, "v_mov_b32 %0, %1")
LV_RATE_KERNEL(r_add_f32, "v_add_f32 %0, %0, %1")
LV_RATE_KERNEL(r_mul_f32, "v_mul_f32 %0, %0, %1")
LV_RATE_KERNEL(r_fma_f32, "v_fma_f32 %0, %0, %1, %2")
LV_RATE_KERNEL(r_fmac_f32, "v_fmac_f32 %0, %1, %2")
LV_RATE_KERNEL(r_add_f32_abs, "v_add_f32_e64 %0, |%0|, %1")
LV_RATE_KERNEL(r_lshlrev_b32, "v_lshlrev_b32 %0, %1, %0")
LV_RATE_KERNEL(r_min_f32, "v_min_f32 %0, %0, %1")
LV_RATE_KERNEL(r_med3_f32, "v_med3_f32 %0, %0, %1, %2")
LV_RATE_KERNEL(r_maximum3_f32, "v_maximum3_f32 %0, |%0|, |%1|, %2")
LV_RATE_KERNEL(r_bfe_u32, "v_bfe_u32 %0, %0, %1, %2")
LV_RATE_KERNEL(r_bfi_b32, "v_bfi_b32 %0, %0, %1, %2")
LV_RATE_KERNEL(r_add3_u32, "v_add3_u32 %0, %0, %1, %2")
LV_RATE_KERNEL(r_lshl_add_u32, "v_lshl_add_u32 %0, %0, %1, %2")
LV_RATE_KERNEL(r_and_or_b32, "v_and_or_b32 %0, %0, %1, %2")
LV_RATE_KERNEL(r_perm_b32, "v_perm_b32 %0, %0, %1, %2")
LV_RATE_KERNEL(r_xor_sdwa, "v_xor_b32_sdwa %0, %0, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:WORD_0")
LV_RATE_KERNEL(r_cmp_cndmask, "v_cmp_gt_f32 vcc, %0, %1\n v_cndmask_b32 %0, %0, %1, vcc", : "vcc")
LV_RATE_KERNEL(r_cvt_f32_u32, "v_cvt_f32_u32 %0, %0")
LV_RATE_KERNEL(r_cvt_pkrtz, "v_cvt_pkrtz_f16_f32 %0, %0, %1")
LV_RATE_KERNEL(r_mul_u32_u24, "v_mul_u32_u24 %0, %0, %1")
LV_RATE_KERNEL(r_mul_lo_u32, "v_mul_lo_u32 %0, %0, %1")
LV_RATE_KERNEL(r_div_scale_f32, "v_div_scale_f32 %0, vcc, %0, %1, %2", : "vcc")
LV_RATE_KERNEL(r_div_fmas_f32, "v_div_fmas_f32 %0, %0, %1, %2")
LV_RATE_KERNEL(r_div_fixup_f32, "v_div_fixup_f32 %0, %0, %1, %2")
LV_RATE_KERNEL(r_rcp_f32, "v_rcp_f32 %0, %0")
LV_RATE_KERNEL(r_sqrt_f32, "v_sqrt_f32 %0, %0")
LV_RATE_KERNEL(r_rsq_f32, "v_rsq_f32 %0, %0")
LV_RATE_KERNEL(r_cvt_sr_bf16, "v_cvt_sr_bf16_f32 %0, %1, %2")
LV_RATE_KERNEL(r_cvt_sr_f16, "v_cvt_sr_f16_f32 %0, %1, %2")

typedef void (*RateFn)(uint32_t *, int, uint32_t);
struct RateOp {
    const char *name;
    RateFn fn;
};
const RateOp kOps[] = {
    {"v_add_u32", r_add_u32},
    {"v_sub_u32", r_sub_u32},
    {"v_and_b32", r_and_b32},
    {"v_or_b32", r_or_b32},
    {"v_xor_b32", r_xor_b32},
    {"v_lshrrev_b32", r_lshrrev_b32},
    {"v_ashrrev_i32", r_ashrrev_i32},
    {"v_mov_b32", r_mov_b32},
    {"v_add_f32", r_add_f32},
    {"v_mul_f32", r_mul_f32},
    {"v_fma_f32", r_fma_f32},
    {"v_fmac_f32", r_fmac_f32},
    {"v_add_f32 |abs|", r_add_f32_abs},
    {"v_lshlrev_b32", r_lshlrev_b32},
    {"v_min_f32", r_min_f32},
    {"v_med3_f32", r_med3_f32},
    {"v_maximum3_f32", r_maximum3_f32},
    {"v_bfe_u32", r_bfe_u32},
    {"v_bfi_b32", r_bfi_b32},
    {"v_add3_u32", r_add3_u32},
    {"v_lshl_add_u32", r_lshl_add_u32},
    {"v_and_or_b32", r_and_or_b32},
    {"v_perm_b32", r_perm_b32},
    {"v_xor_b32_sdwa", r_xor_sdwa},
    {"v_cmp_gt_f32 + v_cndmask_b32 (per pair)", r_cmp_cndmask},
    {"v_cvt_f32_u32", r_cvt_f32_u32},
    {"v_cvt_pkrtz_f16_f32", r_cvt_pkrtz},
    {"v_mul_u32_u24", r_mul_u32_u24},
    {"v_mul_lo_u32", r_mul_lo_u32},
    {"v_div_scale_f32", r_div_scale_f32},
    {"v_div_fmas_f32", r_div_fmas_f32},
    {"v_div_fixup_f32", r_div_fixup_f32},
    {"v_rcp_f32", r_rcp_f32},
    {"v_sqrt_f32", r_sqrt_f32},
    {"v_rsq_f32", r_rsq_f32},
    {"v_cvt_sr_bf16_f32", r_cvt_sr_bf16},
    {"v_cvt_sr_f16_f32", r_cvt_sr_f16},
};
constexpr int kNumOps = (int)(sizeof(kOps) / sizeof(kOps[0]));

}  // namespace

extern "C" int lv_rate_count() { return kNumOps; }

extern "C" const char *lv_rate_name(int op) { return (op >= 0 && op < kNumOps) ? kOps[op].name : nullptr; }

// Best of `reps` timed launches of instruction `op`'s kernel, `iters` loop iterations each, in
// nanoseconds per wave instruction per SIMD (8 waves per SIMD x iters x 256 instructions). Also
// returns the device's reported clock in kHz. 0 on success, 1 for an invalid argument, 2 for a
// HIP error.
extern "C" int lv_rate_measure(int op, int iters, int reps, double *ns_per_instr, int *clock_khz) {
    if (op < 0 || op >= kNumOps || iters <= 0 || reps <= 0 || !ns_per_instr || !clock_khz) return 1;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 2;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 2;
    if (hipDeviceGetAttribute(clock_khz, hipDeviceAttributeClockRate, dev) != hipSuccess) return 2;
    const int blocks = cus * 8;
    uint32_t *out = nullptr;
    if (hipMalloc(&out, (size_t)blocks * 256 * sizeof(uint32_t)) != hipSuccess) return 2;
    hipEvent_t a = nullptr, b = nullptr;
    int rc = 0;
    float best = 1e30f;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) rc = 2;
    if (rc == 0) {
        kOps[op].fn<<<blocks, 256>>>(out, 2, 1u);  // warm-up
        if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess) rc = 2;
    }
    for (int r = 0; rc == 0 && r < reps; r++) {
        float ms = 0.0f;
        if (hipEventRecord(a) != hipSuccess) { rc = 2; break; }
        kOps[op].fn<<<blocks, 256>>>(out, iters, 1u + (uint32_t)r);
        if (hipGetLastError() != hipSuccess || hipEventRecord(b) != hipSuccess || hipEventSynchronize(b) != hipSuccess ||
            hipEventElapsedTime(&ms, a, b) != hipSuccess) {
            rc = 2;
            break;
        }
        if (ms < best) best = ms;
    }
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    (void)hipFree(out);
    if (rc == 0) *ns_per_instr = (double)best * 1e6 / (8.0 * iters * 256.0);
    return rc;
}
