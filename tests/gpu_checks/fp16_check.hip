// Exhaustive check of the library's fp16 conversions (luminamoon_amd/csrc/lv_fp16.h) against the
// reference's integer algorithms, restated here from optimizer/crates/luminav-core/src/prng.rs:
// f32 -> f16 (prng.rs:29-67) over all 2^32 inputs, f16 -> f32 (prng.rs:69-96) over all 2^16.
// Test infrastructure: built by __graft_entry__.build() into tests/gpu_checks/libfp16check.so
// and run by tests/test_gpu_fp16_exhaustive.py.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "lv_fp16.h"

namespace {

// prng.rs:29-67, integer form
__device__ uint32_t ref_f32_to_f16(uint32_t bits) {
    uint32_t sign = (bits >> 16) & 0x8000u;
    int32_t exp = (int32_t)((bits >> 23) & 0xFFu);
    uint32_t mant = bits & 0x007FFFFFu;
    if (exp == 255) return sign | (mant != 0 ? 0x7E00u : 0x7BFFu);
    int32_t ne = exp - 112;
    if (ne >= 31) return sign | 0x7BFFu;
    if (ne <= 0) {
        if (ne < -10) return sign;
        uint32_t fm = mant | 0x00800000u;
        uint32_t sh = (uint32_t)(14 - ne);
        uint32_t half = 1u << (sh - 1);
        return sign | ((fm + half - 1u + ((fm >> sh) & 1u)) >> sh);
    }
    uint32_t r = mant + 0x0FFFu + ((mant >> 13) & 1u);
    uint32_t body = ((uint32_t)ne << 10) + (r >> 13);
    return body >= 0x7C00u ? (sign | 0x7BFFu) : (sign | body);
}

// prng.rs:69-96, integer form
__device__ uint32_t ref_f16_to_f32(uint32_t h) {
    uint32_t sign = (h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x03FFu;
    if (exp == 0) {
        if (mant == 0) return sign;
        uint32_t lz = __clz(mant) - 21;
        return sign | ((113u - lz) << 23) | (((mant << lz) & 0x03FFu) << 13);
    }
    if (exp == 31) return sign | 0x7F800000u | (mant << 13);
    return sign | ((exp + 112u) << 23) | (mant << 13);
}

// out[0]: f32 -> f16 mismatches; out[1]: f16 -> f32 mismatches where either side is not NaN;
// out[2]: f16 -> f32 results that differ but are both NaN with the same sign; ex[0..7] and
// ex[8..15] the first inputs of the first two kinds.
__global__ void check_f32_to_f16(uint32_t base, unsigned long long *out, uint32_t *ex) {
    const uint32_t i = base + blockIdx.x * blockDim.x + threadIdx.x;
    if (lv::f32_to_f16_rne(__uint_as_float(i)) != ref_f32_to_f16(i)) {
        const unsigned long long k = atomicAdd(&out[0], 1ull);
        if (k < 8) ex[k] = i;
    }
}

__global__ void check_f16_to_f32(unsigned long long *out, uint32_t *ex) {
    const uint32_t h = blockIdx.x * blockDim.x + threadIdx.x;  // grid covers exactly 2^16
    const uint32_t got = __float_as_uint(lv::f16_to_f32(h));
    const uint32_t want = ref_f16_to_f32(h);
    if (got == want) return;
    const bool both_nan = (got & 0x7FFFFFFFu) > 0x7F800000u && (want & 0x7FFFFFFFu) > 0x7F800000u;
    if (both_nan && (got >> 31) == (want >> 31)) {
        atomicAdd(&out[2], 1ull);
        return;
    }
    const unsigned long long k = atomicAdd(&out[1], 1ull);
    if (k < 8) ex[8 + k] = h;
}

}  // namespace

extern "C" int fp16_check(unsigned long long *host_counts /* 3 */, uint32_t *host_examples /* 16 */) {
    unsigned long long *out = nullptr;
    uint32_t *ex = nullptr;
    if (hipMalloc(&out, 3 * sizeof(unsigned long long)) != hipSuccess) return -1;
    if (hipMalloc(&ex, 16 * sizeof(uint32_t)) != hipSuccess) return -1;
    if (hipMemset(out, 0, 3 * sizeof(unsigned long long)) != hipSuccess) return -1;
    if (hipMemset(ex, 0, 16 * sizeof(uint32_t)) != hipSuccess) return -1;
    const uint32_t per = 1u << 24;  // 65536 blocks of 256 per launch; 256 launches cover 2^32
    for (uint64_t base = 0; base < (1ull << 32); base += per)
        check_f32_to_f16<<<per / 256, 256>>>((uint32_t)base, out, ex);
    check_f16_to_f32<<<(1u << 16) / 256, 256>>>(out, ex);
    int rc = hipDeviceSynchronize() == hipSuccess ? 0 : -2;
    if (rc == 0 && hipMemcpy(host_counts, out, 3 * sizeof(unsigned long long), hipMemcpyDeviceToHost) != hipSuccess)
        rc = -3;
    if (rc == 0 && hipMemcpy(host_examples, ex, 16 * sizeof(uint32_t), hipMemcpyDeviceToHost) != hipSuccess) rc = -3;
    (void)hipFree(out);
    (void)hipFree(ex);
    return rc;
}
