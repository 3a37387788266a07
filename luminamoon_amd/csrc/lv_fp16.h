// fp16 conversions with the reference's semantics (optimizer/crates/luminav-core/src/prng.rs:29-96),
// on gfx950's hardware converters.
//
// f32 -> f16 (prng.rs:29-67): round to nearest even, subnormals included, but saturating: an
// overflow and an infinity become the largest finite value (+-65504), and a NaN the canonical
// quiet NaN 0x7E00, keeping the sign. v_cvt_f16_f32 rounds to nearest even with IEEE overflow to
// infinity; the fix-up maps its infinities and NaNs to the reference's values. The result equals
// the reference's integer algorithm for every one of the 2^32 inputs
// (tests/test_gpu_fp16_exhaustive.py).
//
// f16 -> f32 (prng.rs:69-96): exact, subnormals included. v_cvt_f32_f16 is exact too and
// differs only on signalling NaNs, which it returns quietened (the payload and the sign kept),
// where the reference keeps the bits; both are NaN.
//
// Both need fp16 denormals enabled, the HIP default for gfx950 code objects.
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

}  // namespace lv
