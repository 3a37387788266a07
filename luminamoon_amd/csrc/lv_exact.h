// Exact helpers on gfx950's hardware instructions, each equal to its reference definition on every
// input (tests/test_gpu_exact_exhaustive.py runs all 2^32 inputs of each).
//
// f32 -> f16 (prng.rs:29-67): round to nearest even, subnormals included, but saturating: an
// overflow and an infinity become the largest finite value (+-65504), and a NaN the canonical
// quiet NaN 0x7E00, keeping the sign. v_cvt_f16_f32 rounds to nearest even with IEEE overflow to
// infinity; the fix-up maps its infinities and NaNs to the reference's values.
//
// f16 -> f32 (prng.rs:69-96): exact, subnormals included. v_cvt_f32_f16 is exact too and
// differs only on signalling NaNs, which it returns quietened (the payload and the sign kept),
// where the reference keeps the bits; both are NaN.
//
// sqrt_rn: the IEEE (correctly rounded) square root, as Rust's f32::sqrt. v_sqrt_f32 is within
// 1 ulp; the neighbour test below picks the correctly rounded one of s - ulp, s, s + ulp from the
// signs of the exact remainders x - s'*s (one fma each). Inputs below 2^-96 are scaled by 2^32
// first so that the remainders stay normal (the root scales by exactly 2^16). It matches the
// compiler's correctly rounded sqrt on all 2^32 inputs (NaN for NaN) in 3 fewer instructions:
// zero, infinity and NaN need no separate class test here.
//
// xor_fold16(z) = (z ^ (z >> 16)) & 0xFFFF, the low half of the reference PRNG's last mixing
// step (prng.rs:25) that bf16 stochastic rounding uses as noise, in one SDWA instruction.
//
// The fp16 conversions need fp16 denormals enabled, the HIP default for gfx950 code objects.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace lv {

__device__ __forceinline__ uint32_t f32_to_f16_rne(float val) {
    const _Float16 h = (_Float16)val;  // v_cvt_f16_f32: round to nearest even
    const uint32_t a = (uint32_t)__builtin_bit_cast(uint16_t, h) & 0x7FFFu;
    const uint32_t sign = (__float_as_uint(val) >> 16) & 0x8000u;
    const uint32_t r = a < 0x7C00u ? a : (a == 0x7C00u ? 0x7BFFu : 0x7E00u);
    return sign | r;
}

__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);  // v_cvt_f32_f16: exact
}

__device__ __forceinline__ float sqrt_rn(float x) {
    const bool small = x < 0x1p-96f;
    const float xs = small ? x * 0x1p32f : x;
    float s = __builtin_amdgcn_sqrtf(xs);  // v_sqrt_f32, within 1 ulp
    const float sd = __uint_as_float(__float_as_uint(s) - 1u);
    const float su = __uint_as_float(__float_as_uint(s) + 1u);
    const float rd = __builtin_fmaf(-sd, s, xs);
    const float ru = __builtin_fmaf(-su, s, xs);
    s = rd <= 0.0f ? sd : s;
    s = ru > 0.0f ? su : s;
    return small ? s * 0x1p-16f : s;
}

__device__ __forceinline__ uint32_t xor_fold16(uint32_t z) {
    uint32_t r;
    asm("v_xor_b32_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:WORD_0"
        : "=v"(r)
        : "v"(z));
    return r;
}

}  // namespace lv
