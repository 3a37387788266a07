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
// sqrt_rn_positive, the same root for 2^-96 <= x <= the largest finite f32, from v_rsq_f32
// instead: with y = rsq(x), g = x * y and h = y / 2, one correction g + (x - g^2) * h (the
// remainder exact in one fma) is the correctly rounded root on every input of that domain
// (checked on all of them). 5 instructions, about 7 integer adds of issue time on gfx950 against
// the neighbour test's 11.7 (v_sqrt_f32 and v_rsq_f32 issue alike). sqrt_rn_normal extends it to
// +-0, +inf and NaN, where g is NaN, with one compare and select (about 9.4).
//
// xor_fold16(z) = (z ^ (z >> 16)) & 0xFFFF, the low half of the reference PRNG's last mixing
// step (prng.rs:25) that bf16 stochastic rounding uses as noise, in one SDWA instruction.
//
// sr_bf16_checked: bf16 stochastic rounding (prng.rs:137-160) as one integer add. For
// |v| <= the largest finite bf16 (0x7F7F0000; NaN excluded) the reference's recipe -- 16 noise
// bits added to |v|'s bits, the low half dropped, the sign put back -- is the high half of
// bits(v) + noise: the sum never carries into the sign bit and never passes 0x7F7FFFFF, so the
// reference's saturation never applies. The other inputs are first replaced by values whose sum
// with any noise has the reference's high half (sr_bf16_prep): a magnitude above the largest
// finite bf16 (inf included), which the reference always rounds to +-0x7F7F, by +-0x7F7F0000;
// a NaN by its quietened upper half (bits | 0x00400000, prng.rs:141-143) with a zero low half.
// The replacement runs only when a lane of the wave needs it (one compare per value). The
// result is an f32 whose HIGH half holds the bf16 bits; its low half is NOT zero, so it is only
// good for storing the high half. (gfx950's v_cvt_sr_bf16_f32 gives the same bits on its
// domain but takes about 3 times an integer add's issue time.)
//
// sr_f16_add: fp16 stochastic rounding (prng.rs:98-130) on its common domain, +-0 and
// 2^-14 <= |v| < 65504 (sr_f16_domain). There the reference adds 13 noise bits (the low 13 of the
// hash) to |v|'s bits and clears those 13 bits: an fp16 normal or zero, at most 65504. That is the
// round-toward-zero fp16 conversion of bits(v) + noise (v_cvt_pkrtz_f16_f32, pack_f16_rtz): the
// sum never carries into the sign bit, stays below 0x47800000 (RTZ gives at most 65504), and for
// +-0 is an f32 far below the smallest fp16 subnormal, which converts to +-0. Outside the domain
// callers take the integer recipe: below 2^-14 the reference widens both the cleared field and
// the noise to 13 + k bits. (gfx950's v_cvt_sr_f16_f32 gives the same bits on the domain but takes
// about 3 times an integer add's issue time, plus a shift to place its noise.)
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

// The neighbour test alone: correctly rounded for x >= 2^-96, +-0, +inf and NaN (no rescaling).
__device__ __forceinline__ float sqrt_rn_neighbours(float x) {
    float s = __builtin_amdgcn_sqrtf(x);  // v_sqrt_f32, within 1 ulp
    const float sd = __uint_as_float(__float_as_uint(s) - 1u);
    const float su = __uint_as_float(__float_as_uint(s) + 1u);
    const float rd = __builtin_fmaf(-sd, s, x);
    const float ru = __builtin_fmaf(-su, s, x);
    s = rd <= 0.0f ? sd : s;
    s = ru > 0.0f ? su : s;
    return s;
}

// One correction from v_rsq_f32: correctly rounded for 2^-96 <= x <= the largest finite f32.
__device__ __forceinline__ float sqrt_rn_positive(float x) {
    const float y = __builtin_amdgcn_rsqf(x);
    const float g = x * y;
    const float h = 0.5f * y;
    const float r = __builtin_fmaf(-g, g, x);
    return __builtin_fmaf(r, h, g);
}

// The same for x >= 2^-96, +-0, +inf and NaN: x * rsq(x) is NaN exactly for +-0, +inf and NaN
// (0 * inf, inf * 0), which are returned as they are (a signalling NaN is not quietened).
__device__ __forceinline__ float sqrt_rn_normal(float x) {
    const float s = sqrt_rn_positive(x);
    return __builtin_isnan(x * __builtin_amdgcn_rsqf(x)) ? x : s;
}

__device__ __forceinline__ float sqrt_rn(float x) {
    const bool small = x < 0x1p-96f;
    const float xs = small ? x * 0x1p32f : x;
    const float s = sqrt_rn_neighbours(xs);
    return small ? s * 0x1p-16f : s;
}

__device__ __forceinline__ uint32_t xor_fold16(uint32_t z) {
    uint32_t r;
    asm("v_xor_b32_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:WORD_0"
        : "=v"(r)
        : "v"(z));
    return r;
}

// Two f32 values packed as fp16 bits, low half first, with one v_cvt_pkrtz_f16_f32 (round toward
// zero). For values that are already fp16 values (every result of the reference's fp16
// quantisation: finite fp16 values, +-65504, signed zeros, subnormals, or the canonical quiet NaN
// +-0x7FC00000) it is exact, and the canonical NaN becomes the reference's +-0x7E00; for
// sr_f16_add's sums it is the truncation that completes the stochastic rounding.
__device__ __forceinline__ uint32_t pack_f16_rtz(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
}

// Largest finite bf16 as an f32.
constexpr uint32_t kBf16MaxBits = 0x7F7F0000u;

// +-largest finite bf16 for a magnitude above it (inf included), v itself otherwise (NaN included).
__device__ __forceinline__ float bf16_saturate(float v) {
    const bool big = __builtin_fabsf(v) > __uint_as_float(kBf16MaxBits);  // false for NaN
    return big ? __uint_as_float((__float_as_uint(v) & 0x80000000u) | kBf16MaxBits) : v;
}

// True where sr_bf16_add needs sr_bf16_prep first: |v| above the largest finite bf16, or NaN.
__device__ __forceinline__ bool sr_bf16_odd(float v) {
    return !(__builtin_fabsf(v) <= __uint_as_float(kBf16MaxBits));
}

// v itself where |v| <= the largest finite bf16; otherwise the value whose sum with any 16-bit
// noise has the reference's rounding of v in its high half.
__device__ __forceinline__ float sr_bf16_prep(float v) {
    const uint32_t quiet = (__float_as_uint(v) | 0x00400000u) & 0xFFFF0000u;
    return v != v ? __uint_as_float(quiet) : bf16_saturate(v);
}

// The add alone: the reference's rounding of v (high half) for |v| <= the largest finite bf16
// and for sr_bf16_prep's values; `noise` is the 16-bit noise in the low half.
__device__ __forceinline__ float sr_bf16_add(float v, uint32_t noise) {
    return __uint_as_float(__float_as_uint(v) + noise);
}

__device__ __forceinline__ float sr_bf16_checked(float v, uint32_t noise) {
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(sr_bf16_odd(v)) != 0, 0)) v = sr_bf16_prep(v);
    return sr_bf16_add(v, noise);
}

__device__ __forceinline__ bool sr_f16_domain(float v) {
    const float a = __builtin_fabsf(v);
    // false for NaN; & and | (not && and ||) keep the three compares free of branches
    return (a < 65504.0f) & ((a >= 0x1p-14f) | (a == 0.0f));
}

// bits(v) + noise, noise in [0, 0x1FFF]: the reference's rounding of v after pack_f16_rtz, for v
// in sr_f16_domain.
__device__ __forceinline__ float sr_f16_add(float v, uint32_t noise) {
    return __uint_as_float(__float_as_uint(v) + noise);
}

}  // namespace lv
