// Exhaustive check of the library's exact helpers (luminamoon_amd/csrc/lv_exact.h) against their
// reference definitions, every input:
//   f32 -> f16 against the reference's integer algorithm (prng.rs:29-67, restated here), 2^32;
//   f16 -> f32 against prng.rs:69-96 (restated here), 2^16;
//   sqrt_rn against the compiler's correctly rounded square root (IEEE, as Rust's f32::sqrt), 2^32;
//   xor_fold16 against (z ^ (z >> 16)) & 0xFFFF with the arithmetic shift of prng.rs:25, 2^32;
//   sr_fp16_val (the library's whole fp16 stochastic rounding: the domain's integer add, the wave's
//     switch to the integer recipe, pack_f16_rtz) against prng.rs:98-130 with prng.rs:21-26's noise,
//     2 hash inputs per input, 2 x 2^32;
//   sr_bf16_checked against the reference's bf16 stochastic rounding (prng.rs:137-160, restated here)
//     with 6 noise values per input (0, 1, 0x7FFF, 0x8000, 0xFFFF and a hash of the input), 6 x 2^32;
//   sqrt_rn_normal against the IEEE square root on its domain (x >= 2^-96, +-0, +inf, NaN), and
//     sqrt_rn_positive on its own (2^-96 <= x <= the largest finite f32);
//   pack_f16_rtz on every f16 value (and the canonical NaNs) against f32 -> f16 RNE, 2^16;
//   sr_f16_add + pack_f16_rtz against the reference's fp16 stochastic rounding (prng.rs:98-130,
//     restated here) on every input of its domain (sr_f16_domain) with 6 noise values per input (0, 1, 0xFFF,
//     0x1000, 0x1FFF and a hash of the input), and the domain test against its definition, 2^32;
//   the guarded fast divisions (div_envelope, div_bound) against IEEE division (div_check).
// Test infrastructure: built by __graft_entry__.build() into tests/gpu_checks/libexactcheck.so
// and run by tests/test_gpu_exact_exhaustive.py.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "lv_device.h"
#include "lv_exact.h"

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

__device__ bool is_nan(uint32_t b) { return (b & 0x7FFFFFFFu) > 0x7F800000u; }

// prng.rs:137-160 with the 16-bit noise given: the bf16 bits
__device__ uint32_t ref_sr_bf16(uint32_t p, uint32_t noise) {
    const uint32_t a = p & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return ((p | 0x00400000u) & 0xFFFF0000u) >> 16;
    uint32_t added = (a + noise) & 0xFFFF0000u;
    if (added > 0x7F7F0000u) added = 0x7F7F0000u;
    return ((p & 0x80000000u) | added) >> 16;
}

// prng.rs:98-130 with the noise given (its low 13 + k bits are used): the result's f32 bits
__device__ uint32_t ref_sr_f16(uint32_t pu, uint32_t noise) {
    const int32_t p = (int32_t)pu;
    const int32_t a = p & 0x7FFFFFFF;
    const int32_t ex = (a >> 23) & 0xFF;
    int32_t sub = 113 - ex;
    sub = sub > 0 ? sub : 0;
    sub = sub < 11 ? sub : 11;
    const uint32_t mask = (1u << (13 + sub)) - 1u;
    const int32_t added = ex < 103 ? 0 : (int32_t)(((uint32_t)a + (noise & mask)) & ~mask);
    const int32_t r = added > 0x477FE000 ? 0x477FE000 : added;
    return (uint32_t)((p & (int32_t)0x80000000u) | r);
}

// prng.rs:21-26: wrapping i32 arithmetic, arithmetic right shifts; z0 = idx + seed - 1640531527.
__device__ uint32_t ref_prng(uint32_t z0) {
    int32_t z = (int32_t)z0;
    z = (int32_t)((uint32_t)(z ^ (z >> 16)) * (uint32_t)-2048173461);
    z = (int32_t)((uint32_t)(z ^ (z >> 13)) * (uint32_t)-1028477387);
    return (uint32_t)(z ^ (z >> 16));
}

__device__ uint32_t mix32(uint32_t z) {
    z ^= z >> 16;
    z *= 0x7FEB352Du;
    z ^= z >> 15;
    z *= 0x846CA68Bu;
    return z ^ (z >> 16);
}

__device__ void record(unsigned long long *count, uint32_t *ex, uint32_t input) {
    const unsigned long long k = atomicAdd(count, 1ull);
    if (k < 8) ex[k] = input;
}

// Counters: [0] f32->f16 mismatches, [1] f16->f32 mismatches other than quietened signalling
// NaNs, [2] quietened signalling NaNs (same sign), [3] sqrt_rn mismatches (two NaNs are equal),
// [4] xor_fold16 mismatches, [5] sr_fp16_val (input, either hash input), [6] sr_bf16_checked
// (input, any noise), [7] sqrt_rn_normal and sqrt_rn_positive on their domains, [8] pack_f16_rtz, [9] sr_f16_add on its
// domain (input, any noise) or a domain test that disagrees with its definition, [10] inputs in
// the sr_f16_domain
// (not a mismatch: the size of the domain checked); ex[8 * c + k] holds the first inputs of
// counter c.
__global__ void check_2_32(uint32_t base, unsigned long long *out, uint32_t *ex) {
    const uint32_t i = base + blockIdx.x * blockDim.x + threadIdx.x;
    if (lv::f32_to_f16_rne(__uint_as_float(i)) != ref_f32_to_f16(i)) record(&out[0], ex + 0, i);
    const uint32_t s = __float_as_uint(lv::sqrt_rn(__uint_as_float(i)));
    const uint32_t s_ref = __float_as_uint(__builtin_sqrtf(__uint_as_float(i)));
    if (s != s_ref && !(is_nan(s) && is_nan(s_ref))) record(&out[3], ex + 24, i);
    if (lv::xor_fold16(i) != ((i ^ (uint32_t)((int32_t)i >> 16)) & 0xFFFFu)) record(&out[4], ex + 32, i);
    const uint32_t zs[2] = {i * 0x9E3779B9u, mix32(i ^ 0x5bd1e995u)};
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const uint32_t got = lv::pack_f16_rtz(lv::sr_fp16_val(__uint_as_float(i), zs[k]), 0.0f);
        if (got != ref_f32_to_f16(ref_sr_f16(i, ref_prng(zs[k])))) record(&out[5], ex + 40, i);
    }
    const uint32_t h = mix32(i);
    const uint32_t noises[6] = {0u, 1u, 0x7FFFu, 0x8000u, 0xFFFFu, h & 0xFFFFu};
#pragma unroll
    for (int k = 0; k < 6; k++) {
        const uint32_t got = __float_as_uint(lv::sr_bf16_checked(__uint_as_float(i), noises[k])) >> 16;
        if (got != ref_sr_bf16(i, noises[k])) record(&out[6], ex + 48, i);
    }
    const float x = __uint_as_float(i);
    const uint32_t mag = i & 0x7FFFFFFFu;
    const bool in_dom = mag == 0u || (mag >= 0x38800000u && mag < 0x477FE000u);  // 2^-14, 65504
    if (lv::sr_f16_domain(x) != in_dom) record(&out[9], ex + 72, i);
    if (in_dom) {
        if ((i & 0xFFFFu) == 0u) atomicAdd(&out[10], 1ull);  // sampled: one in 2^16
        const uint32_t nf[6] = {0u, 1u, 0x0FFFu, 0x1000u, 0x1FFFu, h & 0x1FFFu};
#pragma unroll
        for (int k = 0; k < 6; k++) {
            const uint32_t got = lv::pack_f16_rtz(lv::sr_f16_add(x, nf[k]), 0.0f);
            if (got != ref_f32_to_f16(ref_sr_f16(i, nf[k]))) record(&out[9], ex + 72, i);
        }
    }
    if (!(x < 0x1p-96f) || x == 0.0f) {
        const uint32_t n = __float_as_uint(lv::sqrt_rn_normal(x));
        if (n != s_ref && !(is_nan(n) && is_nan(s_ref))) record(&out[7], ex + 56, i);
        if (x >= 0x1p-96f && x <= 0x1.fffffep127f && __float_as_uint(lv::sqrt_rn_positive(x)) != s_ref)
            record(&out[7], ex + 56, i);
    }
}

// pack_f16_rtz: every finite f16 value h (as f32), and the canonical quiet NaNs, against the
// reference's f32 -> f16 RNE; the packed word holds the value in both halves. The infinities are
// not in the domain: the reference's fp16 quantisation saturates them to +-65504 (prng.rs:29-67,
// prng.rs:98-130), so no quantised value is infinite.
__global__ void check_pack_f16(unsigned long long *out, uint32_t *ex) {
    const uint32_t h = blockIdx.x * blockDim.x + threadIdx.x;  // grid covers exactly 2^16
    if ((h & 0x7FFFu) == 0x7C00u) return;
    uint32_t xb = ref_f16_to_f32(h);
    if (is_nan(xb)) xb = (xb & 0x80000000u) | 0x7FC00000u;  // quantisation yields canonical NaNs only
    const float x = __uint_as_float(xb);
    const uint32_t want = ref_f32_to_f16(xb);
    if (lv::pack_f16_rtz(x, x) != (want | (want << 16))) record(&out[8], ex + 64, h);
}

__global__ void check_f16_to_f32(unsigned long long *out, uint32_t *ex) {
    const uint32_t h = blockIdx.x * blockDim.x + threadIdx.x;  // grid covers exactly 2^16
    const uint32_t got = __float_as_uint(lv::f16_to_f32(h));
    const uint32_t want = ref_f16_to_f32(h);
    if (got == want) return;
    if (is_nan(got) && is_nan(want) && (got >> 31) == (want >> 31)) {
        atomicAdd(&out[2], 1ull);
        return;
    }
    record(&out[1], ex + 8, h);
}

}  // namespace

constexpr int kCounters = 11;

extern "C" int exact_check(unsigned long long *host_counts /* kCounters */, uint32_t *host_examples /* 8 x kCounters */) {
    unsigned long long *out = nullptr;
    uint32_t *ex = nullptr;
    if (hipMalloc(&out, kCounters * sizeof(unsigned long long)) != hipSuccess) return -1;
    if (hipMalloc(&ex, 8 * kCounters * sizeof(uint32_t)) != hipSuccess) return -1;
    if (hipMemset(out, 0, kCounters * sizeof(unsigned long long)) != hipSuccess) return -1;
    if (hipMemset(ex, 0, 8 * kCounters * sizeof(uint32_t)) != hipSuccess) return -1;
    const uint32_t per = 1u << 24;  // 65536 blocks of 256 per launch; 256 launches cover 2^32
    for (uint64_t base = 0; base < (1ull << 32); base += per) check_2_32<<<per / 256, 256>>>((uint32_t)base, out, ex);
    check_f16_to_f32<<<(1u << 16) / 256, 256>>>(out, ex);
    check_pack_f16<<<(1u << 16) / 256, 256>>>(out, ex);
    int rc = hipDeviceSynchronize() == hipSuccess ? 0 : -2;
    if (rc == 0 &&
        hipMemcpy(host_counts, out, kCounters * sizeof(unsigned long long), hipMemcpyDeviceToHost) != hipSuccess)
        rc = -3;
    if (rc == 0 && hipMemcpy(host_examples, ex, 8 * kCounters * sizeof(uint32_t), hipMemcpyDeviceToHost) != hipSuccess)
        rc = -3;
    (void)hipFree(out);
    (void)hipFree(ex);
    return rc;
}

namespace {

// A float with the exponent drawn from [lo, hi] (unbiased exponents) and a random mantissa.
__device__ float rand_float(uint32_t h, int lo, int hi) {
    const uint32_t span = (uint32_t)(hi - lo + 1);
    const int e = lo + (int)((h >> 23) % span);
    return __uint_as_float(((uint32_t)(e + 127) << 23) | (mix32(h) & 0x007FFFFFu));
}

__device__ bool same_bits(float a, float b) {
    const uint32_t x = __float_as_uint(a), y = __float_as_uint(b);
    return x == y || (is_nan(x) && is_nan(y));
}

// The guarded fast divisions (lv_device.h: div_unscaled under div_envelope's and div_bound's
// tests) against the IEEE quotient the compiler's own division gives. Counters: [0] div_envelope
// on all 2^32 numerators x 3 denominators in [|n| / 2, 2^25]; [1] T2's clm / env from its own
// formula (compute_u) on all 2^32 gradient bit patterns x a random state; [2] the rational bound
// (bb * s) / (s * s + bb) through div_bound on all 2^32 step bit patterns x a random b (a zero
// quotient may differ in sign there: zero_ok); [3] the pairs checked in [0], sampled one input in
// 2^16 (not mismatches: the size of the domain checked).
__global__ void check_div(uint32_t base, unsigned long long *out, uint32_t *ex) {
    const uint32_t i = base + blockIdx.x * blockDim.x + threadIdx.x;
    const float n = __uint_as_float(i);
    const float an = __builtin_fabsf(n);
    // [0]: d from |n| / 2 (at least 2^-101) to 2^25, when that range is not empty
    if (an >= 0x1p-100f && an <= 0x1p25f) {
        const int elo = (int)((__float_as_uint(an) >> 23) & 0xFFu) - 128;  // exponent of |n| / 2
        const float ds[3] = {an, rand_float(mix32(i ^ 0x1234567u), elo < -101 ? -101 : elo, 24),
                             __builtin_fmaxf(an * 0.5f, 0x1p-101f)};
#pragma unroll
        for (int k = 0; k < 3; k++) {
            const float d = ds[k];
            if (!(d >= an * 0.5f && d <= 0x1p25f)) continue;
            if (!same_bits(lv::div_envelope(n, d), n / d)) record(&out[0], ex + 0, i);
            if ((i & 0xFFFFu) == 0u) atomicAdd(&out[3], 1ull);  // sampled: one in 2^16
        }
    }
    // [1]: T2's masked direction, g = the input bits, m, v from a hash of it
    {
        const uint32_t h = mix32(i * 0x9E3779B9u);
        const float g = n;
        const float m = (h & 1u ? -1.0f : 1.0f) * rand_float(h, -40, 4);
        const float v = rand_float(mix32(h), -60, 2);
        const float b1sq = 0.9f * 0.9f, omb1sq = 1.0f - b1sq, lam1 = 0.15f, eps = 1e-8f, c_sigma = 0.1503f;
        const float clm = __builtin_fmaf(b1sq, m, omb1sq * g);
        const float diff = g - m;
        const float env0 = __builtin_fmaf(b1sq, __builtin_fabsf(m), eps);
        const float env1 = __builtin_fmaf(omb1sq, __builtin_fabsf(g), env0);
        const float env2 = __builtin_fmaf(lam1, __builtin_fabsf(diff), env1);
        const float env = __builtin_fmaf(c_sigma, __builtin_sqrtf(v), env2);
        if (!same_bits(lv::div_envelope(clm, env), clm / env)) record(&out[1], ex + 8, i);
    }
    // [2]: the rational bound over every step value s, b = ratio * (|p| + 0.01) for a random p
    {
        const uint32_t h = mix32(i ^ 0xA5A5A5A5u);
        const float s = n;
        const float b = rand_float(h, -50, 6);
        const float bb = b * (b + __builtin_fabsf(s));
        const float num = bb * s, den = __builtin_fmaf(s, s, bb);
        bool fast;
        const float got = lv::div_bound(num, den, __builtin_amdgcn_ballot_w64(s == 0.0f && b >= 0x1p-46f), fast);
        const float want = num / den;
        const bool ok = same_bits(got, want) || (got == 0.0f && want == 0.0f);
        if (!ok) record(&out[2], ex + 16, i);
    }
}

}  // namespace

extern "C" int div_check(unsigned long long *host_counts /* 4 */, uint32_t *host_examples /* 8 x 4 */) {
    unsigned long long *out = nullptr;
    uint32_t *ex = nullptr;
    if (hipMalloc(&out, 4 * sizeof(unsigned long long)) != hipSuccess) return -1;
    if (hipMalloc(&ex, 32 * sizeof(uint32_t)) != hipSuccess) return -1;
    if (hipMemset(out, 0, 4 * sizeof(unsigned long long)) != hipSuccess) return -1;
    if (hipMemset(ex, 0, 32 * sizeof(uint32_t)) != hipSuccess) return -1;
    const uint32_t per = 1u << 24;
    for (uint64_t b = 0; b < (1ull << 32); b += per) check_div<<<per / 256, 256>>>((uint32_t)b, out, ex);
    int rc = hipDeviceSynchronize() == hipSuccess ? 0 : -2;
    if (rc == 0 && hipMemcpy(host_counts, out, 4 * sizeof(unsigned long long), hipMemcpyDeviceToHost) != hipSuccess)
        rc = -3;
    if (rc == 0 && hipMemcpy(host_examples, ex, 32 * sizeof(uint32_t), hipMemcpyDeviceToHost) != hipSuccess) rc = -3;
    (void)hipFree(out);
    (void)hipFree(ex);
    return rc;
}

namespace {

// div_unscaled against IEEE division on every pair of significands: n = 1.nm, d = 1.dm, both in
// [1, 2), for the 2^23 numerators nm and the denominators dm in [dm0, dm0 + gridDim.x). Under the
// guards of div_envelope and div_bound every intermediate of div_unscaled is these pairs' scaled
// by powers of two: v_rcp_f32 scales with d's exponent (check_rcp_scale), e0 does not depend on
// it, q0, r1 and the quotient are normal, and the residual n - d * q0 is exact wherever its scaled
// value is subnormal (a multiple of 2^-147 there), so every rounding scales too. Counters: [0]
// mismatches (ex: dm, nm pairs), [1] pairs checked.
__global__ void check_div_pairs(uint32_t dm0, unsigned long long *out, uint32_t *ex) {
    const uint32_t dm = dm0 + blockIdx.x;
    const float d = __uint_as_float(0x3F800000u | dm);
    for (uint32_t nm = threadIdx.x; nm < (1u << 23); nm += blockDim.x) {
        const float n = __uint_as_float(0x3F800000u | nm);
        if (__float_as_uint(lv::div_unscaled(n, d)) != __float_as_uint(n / d)) {
            const unsigned long long k = atomicAdd(&out[0], 1ull);
            if (k < 4) {
                ex[2 * k] = dm;
                ex[2 * k + 1] = nm;
            }
        }
    }
    if (threadIdx.x == 0) atomicAdd(&out[1], 1ull << 23);
}

// v_rcp_f32 on d = 1.dm * 2^e against v_rcp_f32(1.dm) * 2^-e, for every significand and every e
// with 2^e and 2^-e normal (e in [-126, 126] less the ends): the reciprocal's significand does
// not depend on d's exponent. Counters: [2] mismatches (ex: dm, e + 128), [3] pairs checked.
__global__ void check_rcp_scale(unsigned long long *out, uint32_t *ex) {
    const uint32_t dm = blockIdx.x * blockDim.x + threadIdx.x;
    if (dm >= (1u << 23)) return;
    const float base = __builtin_amdgcn_rcpf(__uint_as_float(0x3F800000u | dm));
    for (int e = -125; e <= 125; e++) {
        const float d = __uint_as_float(((uint32_t)(127 + e) << 23) | dm);
        const float want = __builtin_ldexpf(base, -e);
        if (__float_as_uint(__builtin_amdgcn_rcpf(d)) != __float_as_uint(want)) {
            const unsigned long long k = atomicAdd(&out[2], 1ull);
            if (k < 4) {
                ex[8 + 2 * k] = dm;
                ex[8 + 2 * k + 1] = (uint32_t)(e + 128);
            }
        }
    }
    if ((dm & 255u) == 0u) atomicAdd(&out[3], 256ull * 251ull);
}

}  // namespace

// div_unscaled on the significand pairs with denominators [dm_first, dm_first + dm_count), and
// (with_rcp) v_rcp_f32's scaling over every exponent. Counters as check_div_pairs and
// check_rcp_scale: 4, examples 16. Returns 0, or negative on a HIP error or a range outside 2^23.
extern "C" int div_pair_check(uint32_t dm_first, uint32_t dm_count, int with_rcp, unsigned long long *host_counts,
                              uint32_t *host_examples) {
    if (dm_first > (1u << 23) || dm_count > (1u << 23) - dm_first) return -5;
    unsigned long long *out = nullptr;
    uint32_t *ex = nullptr;
    if (hipMalloc(&out, 4 * sizeof(unsigned long long)) != hipSuccess) return -1;
    if (hipMalloc(&ex, 16 * sizeof(uint32_t)) != hipSuccess) return -1;
    if (hipMemset(out, 0, 4 * sizeof(unsigned long long)) != hipSuccess) return -1;
    if (hipMemset(ex, 0, 16 * sizeof(uint32_t)) != hipSuccess) return -1;
    const uint32_t per = 1u << 14;
    for (uint32_t b = 0; b < dm_count; b += per)
        check_div_pairs<<<dm_count - b < per ? dm_count - b : per, 256>>>(dm_first + b, out, ex);
    if (with_rcp) check_rcp_scale<<<(1u << 23) / 256, 256>>>(out, ex);
    int rc = hipDeviceSynchronize() == hipSuccess ? 0 : -2;
    if (rc == 0 && hipMemcpy(host_counts, out, 4 * sizeof(unsigned long long), hipMemcpyDeviceToHost) != hipSuccess)
        rc = -3;
    if (rc == 0 && hipMemcpy(host_examples, ex, 16 * sizeof(uint32_t), hipMemcpyDeviceToHost) != hipSuccess) rc = -3;
    (void)hipFree(out);
    (void)hipFree(ex);
    return rc;
}

// The graph launches' per-step coefficients computed on the device (lv::step_coeffs, the function
// the step record kernel calls), for the host to compare with its own: out[4 * i ..] = c1, c2,
// c_sigma (bits) and the seed base of steps[i].
__global__ void coeff_kernel(const uint64_t *steps, int n, float b1, float b2, float eps, float tau, float lam,
                             uint32_t seed, uint32_t *out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const lv::StepCoeffs k = lv::step_coeffs(steps[i], b1, b2, eps, tau, lam);
    out[4 * i] = __float_as_uint(k.c1);
    out[4 * i + 1] = __float_as_uint(k.c2);
    out[4 * i + 2] = __float_as_uint(k.c_sigma);
    out[4 * i + 3] = lv::step_seed_base(seed, steps[i]);
}

extern "C" int coeff_check(const uint64_t *host_steps, int n, float b1, float b2, float eps, float tau, float lam,
                           uint32_t seed, uint32_t *host_out) {
    uint64_t *steps = nullptr;
    uint32_t *out = nullptr;
    if (n <= 0) return 0;
    if (hipMalloc(&steps, (size_t)n * sizeof(uint64_t)) != hipSuccess) return -1;
    if (hipMalloc(&out, (size_t)n * 4 * sizeof(uint32_t)) != hipSuccess) return -1;
    int rc = hipMemcpy(steps, host_steps, (size_t)n * sizeof(uint64_t), hipMemcpyHostToDevice) == hipSuccess ? 0 : -2;
    if (rc == 0) {
        coeff_kernel<<<(n + 255) / 256, 256>>>(steps, n, b1, b2, eps, tau, lam, seed, out);
        rc = hipDeviceSynchronize() == hipSuccess ? 0 : -3;
    }
    if (rc == 0 && hipMemcpy(host_out, out, (size_t)n * 4 * sizeof(uint32_t), hipMemcpyDeviceToHost) != hipSuccess) rc = -4;
    (void)hipFree(steps);
    (void)hipFree(out);
    return rc;
}
