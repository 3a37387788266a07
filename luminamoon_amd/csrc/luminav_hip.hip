// MI355X (gfx950) LuminaV optimizer step: HIP kernels + C ABI (include/luminav_hip.h).
//
// One multi-tensor launch per (pass, step, dtype) class of tensors: up to 48 descriptors in the
// kernel arguments (inline launch), or up to 960 uploaded to the workspace through pinned staging
// with their first units in the kernel arguments (table launch). Each tensor is cut into work
// units of 1024 elements (2048 with 16-bit state); every block of a unit launch updates exactly
// one unit and exits. A thread moves 4 consecutive elements of each 1024-element half with
// vector loads/stores (16 bytes for f32, 8 for 16-bit types) and falls back to per-element
// access for the partial last unit and for tensors whose pointers are not 16-byte aligned.
// The cautious mask is counted exactly: each block reports its integer count and its completion
// in one atomic on one of 64 spread u64 slot words per tensor; the block that completes the
// tensor holds the exact total and finalises the 6-float scratch on the device, so a steady step
// is one launch and needs no host synchronisation.
//
// Radial bound (counting passes): the same unit launch, run in pieces of at most kRadialPiece
// units. Each block sums sum(u_eff^2) and sum(p^2) of its unit from the f32 squares in f64 (per
// thread, then a fixed-order wave/block reduction) and stores them, with its mask count, as the
// unit's record in the workspace with plain stores; a fold launch after each piece (the kernel
// boundary makes the records visible, so the streaming kernel needs no fence) sums the records
// of each tensor in unit order, carries the tensor's running sum from piece to piece, and
// finalises the scratch in the piece that holds the tensor's last unit. The result (rounded to
// f32 once) is the exactly rounded sum up to f64 rounding, and bitwise deterministic on any
// device (the summation tree depends only on the unit and piece sizes). The reference's own f32
// sums depend on its CPU backend (16-lane order in reference_cpu/dual.rs:134-253 vs. AVX-512
// reductions in avx512/dual.rs), so radial results match it to its cross-backend tolerance, not
// bit for bit.
//
// Per-element arithmetic follows the reference's scalar core operation for operation
// (optimizer/crates/luminav-core/src/reference_cpu/dual.rs, reference_cpu/tdclm.rs,
// math.rs, prng.rs): explicit fmaf exactly where the Rust code calls mul_add, separately
// rounded products elsewhere (built with -ffp-contract=off), IEEE division and square root,
// so results are bitwise equal to the reference CPU implementation.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

#include "luminav_hip.h"
#include "lv_exact.h"

namespace lv {

constexpr int kThreads = 256;
constexpr uint32_t kHalf = kThreads * 4;     // a thread owns 4 consecutive elements of each half

// Halves per work unit of a unit launch. With f32 state the step is HBM-bound and 1024-element
// units stream best (measured in one process: T2 bf16/f32 23.2 vs 23.6 ms, T1 bf16/f32 2.17 vs
// 2.25 ms, CLM and TD-CLM f32 0.58 vs 0.63 ms and 0.41 vs 0.44 ms for 1024 vs 2048). With 16-bit
// state, stochastic rounding of m (and v) makes the step VALU-bound and 2048-element units are
// faster (T2 bf16/bf16 3.05 vs 3.40 ms, T1 bf16/bf16 2.22 vs 2.49 ms).
constexpr int unit_halves(int mode, int pt, int st) {
    (void)mode;
    (void)pt;
    return st == LV_DTYPE_F32 ? 1 : 2;
}
constexpr int kMaxDesc = 48;                 // tensors per inline launch (kernel argument table, < 4 KiB)
constexpr uint32_t kSlots = 64;              // cautious-count slots per tensor (unit launches)
constexpr uint32_t kSlotWords = kSlots + 1;  // + one fold word per tensor
constexpr uint32_t kSlotStride = 8;          // u64 per slot: one slot per 64-byte segment
// Slot word: mask count << kTicketBits | blocks that reported. A tensor has < 2^32 units of
// >= 1024 elements and at most 2^42 elements, so a slot sees <= 2^26 blocks (27 bits) and
// counts <= 2^36 elements (37 bits). Fold word: count << 7 | slots completed (<= 64).
constexpr int kTicketBits = 27;
constexpr int kFoldBits = 7;
constexpr uint32_t kMaxGrid = 1u << 23;      // blocks per unit launch (grid x 256 threads < 2^32)
// Radial counting launches: units per piece (one workspace record each: 2 doubles + a u32 count),
// and unit records one fold block sums into a chunk record.
constexpr uint32_t kRadialPiece = 1u << 22;
constexpr uint32_t kFoldChunk = 4096;  // fold blocks per full piece: kRadialPiece / kFoldChunk
constexpr int kFoldBatch = 16;         // unit records a fold thread loads before adding them
constexpr uint32_t kMaxChunks = kRadialPiece / kFoldChunk + kMaxDesc;  // chunks of one piece
// A chunk's mask count (<= kFoldChunk units x 2048 elements) fits the u32 chunk sums; the
// sums over chunks run in u64.
static_assert((uint64_t)kFoldChunk * 2048u <= 0xFFFFFFFFull, "chunk counts fit 32 bits");

enum Pass : int { kSingle = 0, kFused = 1, kCount = 2, kApply = 3 };

enum Flags : uint32_t {
    kFDynamic = 1u << 31,  // template flag set: read the flags from the launch arguments
    kFCautious = 1u << 0,
    kFSR = 1u << 1,
    kFMaster = 1u << 2,
    kFWeightDecay = 1u << 3,
    kFClampV = 1u << 4,
    kFRadial = 1u << 5,
    kFCoordinate = 1u << 6,
};

// One tensor of a launch (80 bytes): in the kernel arguments (inline launches) or in the
// workspace (table launches).
struct Desc {
    void *p;
    const void *g;
    void *m;
    void *v;
    float *mp;
    float *scratch;
    uint64_t n;
    uint32_t unit_begin;  // first work unit of this tensor in the launch's unit space
    uint32_t pidx;        // low 32 bits of param_index (seeds only need idx * 10007 mod 2^31)
    uint32_t ibase;       // low 32 bits of index_base (the SR offset is taken mod 2^32)
    uint32_t nskip;       // inactive [begin, end) ranges in `skip` (sorted, disjoint)
    const uint64_t *skip;
};

// Radial-bound sums of a run of units: sum u_eff^2, sum p^2 (f64), mask count.
struct RadialSum {
    double su, sp;
    unsigned long long cnt, pad;
};

// Launch-uniform constants: hyper-parameters, per-step coefficients, tensor table.
struct Args {
    float lr, b1, b2, omb1, omb2, b1sq, omb1sq, eps, lam, lam1, neg_lr_wd, ratio;
    float c1, c2, c_sigma, ema, ema_c, clamp_min;
    uint32_t seed_base;  // low 32 bits of seed + step * 0x9E3779B9 (prng.rs:4-13)
    uint32_t flags;      // Flags | grad dtype << 8
    uint32_t total_units;
    uint32_t unit_base;  // unit launches: the blocks cover units [unit_base, unit_base + grid)
    uint32_t xcds;       // unit launches: XCDs the device dispatches workgroups over (>= 1)
    uint32_t xcd_q, xcd_r;  // unit launches: grid / xcds and grid % xcds of this launch
    int32_t ndesc;
    uint32_t piece_units;  // radial launches: units of the current piece ([unit_base, + piece_units))
    uint32_t pad_;
    uint64_t xcd_recip;  // unit launches: floor(2^40 / xcds) + 1, so b / xcds == (b * xcd_recip) >> 40
    unsigned long long *slots;    // non-radial counting launches: kSlotWords count words per tensor
    unsigned long long *tickets;  // radial fold: finished chunks of the piece, per tensor (left zero)
    RadialSum *run;               // radial fold: per tensor, the sums of the pieces folded so far
    RadialSum *chunks;            // radial fold: one record per chunk of the piece
    double *unit_sq;              // radial: per unit of the piece, (sum u_eff^2, sum p^2)
    uint32_t *unit_cnt;           // radial: per unit of the piece, the mask count
    const Desc *dtab;             // table launches: the tensor table in device memory
    union {
        Desc d[kMaxDesc];  // inline launches: the tensor table
        uint32_t ubegin[kMaxDesc * sizeof(Desc) / sizeof(uint32_t)];  // table launches: first unit per tensor
    };
};

// Table launches: up to kTableMax tensors, their descriptors uploaded to the workspace and their
// first units in the kernel arguments (where the inline table would be).
constexpr int kTableMax = kMaxDesc * (int)(sizeof(Desc) / sizeof(uint32_t));  // 960

static_assert(sizeof(Desc) == 80, "descriptor layout");
static_assert(sizeof(Args) <= 4096, "kernel arguments must fit in 4 KiB");

// ------------------------------------------------------------------ device math

__device__ __forceinline__ float bits_f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f_bits(float f) { return __float_as_uint(f); }

// Rust f32::clamp: NaN passes through.
__device__ __forceinline__ float rclamp(float x, float lo, float hi) {
    x = x < lo ? lo : x;
    return x > hi ? hi : x;
}

// prng.rs:21-26 -- wrapping i32 arithmetic, arithmetic right shifts.
// The multipliers are the reference's decimal i32 constants; the first one is close to, but not,
// MurmurHash3's fmix32 constant.
// The hash input is z0 = idx + seed + kPrngAdd (wrapping); callers form z0 themselves, so a
// thread adds a per-stream base once and each element only its constant offset.
// prng_mixed is the state before the last step, z ^ (z >> 16).
constexpr uint32_t kPrngAdd = (uint32_t)-1640531527;  // wrapping_sub(1_640_531_527)

__device__ __forceinline__ int32_t prng_mixed(uint32_t z0) {
    constexpr uint32_t kMul1 = (uint32_t)-2048173461;
    constexpr uint32_t kMul2 = (uint32_t)-1028477387;
    int32_t z = (int32_t)z0;
    z = (int32_t)((uint32_t)(z ^ (z >> 16)) * kMul1);
    return (int32_t)((uint32_t)(z ^ (z >> 13)) * kMul2);
}

__device__ __forceinline__ int32_t prng(uint32_t z0) {
    const int32_t z = prng_mixed(z0);
    return z ^ (z >> 16);
}

// prng.rs:137-160 (value form: f32 carrying the bf16 bits). Branch-free: both the finite and
// the NaN result are formed and one is selected, so a wave never splits on NaN lanes.
__device__ __forceinline__ float sr_bf16(float v, uint32_t z0) {
    uint32_t p = f_bits(v);
    uint32_t a = p & 0x7FFFFFFFu;
    uint32_t noise = xor_fold16((uint32_t)prng_mixed(z0));  // prng(z0) & 0xFFFF
    uint32_t added = (a + noise) & 0xFFFF0000u;  // a <= 0x7F800000 when used: no wrap, never "negative"
    uint32_t r = added > 0x7F7F0000u ? 0x7F7F0000u : added;
    uint32_t fin = (p & 0x80000000u) | r;
    uint32_t nan = (p | 0x00400000u) & 0xFFFF0000u;
    return bits_f(a > 0x7F800000u ? nan : fin);
}

// prng.rs:162-178
__device__ __forceinline__ float rne_bf16(float v) {
    uint32_t b = f_bits(v);
    uint32_t a = b & 0x7FFFFFFFu;
    uint32_t r = (a + 0x7FFFu + ((a >> 16) & 1u)) & 0xFFFF0000u;
    r = r > 0x7F7F0000u ? 0x7F7F0000u : r;
    uint32_t fin = (b & 0x80000000u) | r;
    uint32_t nan = (b | 0x00400000u) & 0xFFFF0000u;
    return bits_f(a > 0x7F800000u ? nan : fin);
}

// f32_to_f16_rne (prng.rs:29-67) and f16_to_f32 (prng.rs:69-96) are in lv_exact.h.

// prng.rs:98-130
__device__ __forceinline__ float sr_fp16(float v, uint32_t z0) {
    int32_t p = (int32_t)f_bits(v);
    int32_t a = p & 0x7FFFFFFF;
    int32_t ex = (a >> 23) & 0xFF;
    int32_t sub = 113 - ex;
    sub = sub > 0 ? sub : 0;
    sub = sub < 11 ? sub : 11;
    int32_t mask = (int32_t)((1u << (13 + sub)) - 1u);
    int32_t noise = prng(z0) & mask;
    int32_t added = ex < 103 ? 0 : (int32_t)(((uint32_t)a + (uint32_t)noise) & (uint32_t)(~mask));
    int32_t r = added > 0x477FE000 ? 0x477FE000 : added;
    // The reference converts sign | r to fp16 and back (prng.rs:129). That is the identity here,
    // because sign | r is already an fp16 value. r is one of:
    // - 0, or 65504;
    // - the sign bit alone (-0.0), when a NaN's magnitude plus the noise wraps past 2^31;
    // - a value with its (13 + sub) low bits clear. For ex >= 113 that leaves 10 fraction bits
    //   below 65504 (an fp16 normal). For 103 <= ex <= 112 it leaves a multiple of 2^-24 below
    //   2^-13 (fp16 subnormals and the lowest normal binade).
    return bits_f((uint32_t)((p & (int32_t)0x80000000u) | r));
}

__device__ __forceinline__ float rne_fp16(float v) { return f16_to_f32(f32_to_f16_rne(v)); }

// prng.rs:180-195; dtype is a compile-time constant at every call site. z0 is the element's
// hash input for the buffer's seed (offset + seed + kPrngAdd).
template <int DT>
__device__ __forceinline__ float quantize(float v, uint32_t z0, bool sr) {
    if constexpr (DT == LV_DTYPE_BF16) {
        return sr ? sr_bf16(v, z0) : rne_bf16(v);
    } else if constexpr (DT == LV_DTYPE_F16) {
        return sr ? sr_fp16(v, z0) : rne_fp16(v);
    } else {
        return v;
    }
}

// math.rs:4-11. |g| < 1e38 is false for NaN and +-inf, so one compare also covers is_finite;
// on that path g is not NaN and med3 is exactly the clamp.
__device__ __forceinline__ float sanitize(float g) {
    return fabsf(g) < 1.0e38f ? __builtin_amdgcn_fmed3f(g, -1.0e18f, 1.0e18f) : 0.0f;
}

// math.rs:13-16 (clamp_defect): NaN passes through like Rust's f32::clamp.
__device__ __forceinline__ float clamp_defect(float d) {
    return __builtin_isnan(d) ? d : __builtin_amdgcn_fmed3f(d, -1.0e18f, 1.0e18f);
}

// math.rs:83-118 -- [13/6] Pade tanh, Horner with fma.
__device__ __forceinline__ float tanh_pade(float x_in) {
    if (__builtin_isnan(x_in)) return bits_f(0x7FC00000u);  // Rust f32::NAN
    float x = rclamp(x_in, -7.9988117f, 7.9988117f);
    float x2 = x * x;
    float p = __builtin_fmaf(-2.7607684e-16f, x2, 2.000188e-13f);
    float q = __builtin_fmaf(1.1982584e-6f, x2, 1.1853471e-4f);
    p = __builtin_fmaf(p, x2, -8.604672e-11f);
    q = __builtin_fmaf(q, x2, 2.2684346e-3f);
    p = __builtin_fmaf(p, x2, 5.122297e-8f);
    q = __builtin_fmaf(q, x2, 4.8935246e-3f);
    p = __builtin_fmaf(p, x2, 1.4857224e-5f);
    p = __builtin_fmaf(p, x2, 6.3726193e-4f);
    p = __builtin_fmaf(p, x2, 4.8935246e-3f);
    return (x * p) / q;
}

// math.rs:162-186
template <bool TRI>
__device__ __forceinline__ float coordinate_bound(float step, float p_init, float ratio) {
    if constexpr (TRI) {
        float b = ratio * (fabsf(p_init) + 1.0e-2f);
        float bb = b * (b + fabsf(step));
        return (bb * step) / __builtin_fmaf(step, step, bb);
    } else {
        float b = ratio * sqrt_rn(__builtin_fmaf(p_init, p_init, 1.0e-4f));
        return b * tanh_pade(step / b);
    }
}

template <bool TRI>
__device__ __forceinline__ float fp16_safety_bound(float step, float p_init) {
    float b = __builtin_fmaxf(fabsf(p_init) * 0.01f, 1.5e-4f);
    if constexpr (TRI) {
        float bb = b * (b + fabsf(step));
        return (bb * step) / __builtin_fmaf(step, step, bb);
    } else {
        return b * tanh_pade(step / b);
    }
}

// math.rs:120-125
__device__ __forceinline__ float cautious_scale(float mask_sum, float total, float clamp_min) {
    float denom = __builtin_fmaxf(total, 1.0f);
    return 1.0f / rclamp(mask_sum / denom, clamp_min, 1.0f);
}

// math.rs:127-160: radial trust-region scale from the squared norms. TRI selects the rational
// form of the triangle family (T1/T2), otherwise tanh(r)/r.
template <bool TRI>
__device__ __forceinline__ float radial_scale(float u_sq, float p_sq, float cs, float lr, float ratio) {
    float norm_p = __builtin_sqrtf(__builtin_fmaxf(p_sq, 0.0f));
    float norm_d = __builtin_sqrtf(__builtin_fmaxf(u_sq, 0.0f)) * cs;
    float radius = ratio * __builtin_fmaxf(norm_p, 1.0f);
    if constexpr (TRI) {
        float r = (lr * norm_d) / __builtin_fmaxf(radius, 1.0e-12f);
        float one_plus_r = 1.0f + r;
        return one_plus_r / __builtin_fmaf(r, r, one_plus_r);
    } else {
        float r = (lr * norm_d) / radius;
        if (r < 1.0e-4f) return 1.0f;
        return tanh_pade(r) / __builtin_fmaxf(r, 1.0e-8f);
    }
}

// Round-to-nearest-even u64 -> f32 (Rust `as f32`), exact integer algorithm.
__device__ __forceinline__ float u64_to_f32_rn(uint64_t x) {
    if ((x >> 24) == 0) return (float)(uint32_t)x;
    int bits = 64 - __clzll((long long)x);
    int sh = bits - 24;
    uint64_t mant = x >> sh;
    uint64_t rem = x & ((1ull << sh) - 1ull);
    uint64_t half = 1ull << (sh - 1);
    if (rem > half || (rem == half && (mant & 1ull))) mant += 1ull;
    return ldexpf((float)(uint32_t)mant, sh);
}

// u, m_new, v_new for one element.
// CLM: dual.rs:63-74.  T2: dual.rs:492-506.  TD-CLM / T1: tdclm.rs:102-109.
template <int MODE>
__device__ __forceinline__ float compute_u(const Args &a, bool clamp_v, float g, float m, float v,
                                           float &m_new, float &v_new) {
    m_new = __builtin_fmaf(a.b1, m, a.omb1 * g);
    if constexpr (MODE == LV_BUFFER_DUAL) {
        float clm = __builtin_fmaf(a.b1, m_new, a.omb1 * g);
        float diff = clamp_defect(g - m_new);
        v_new = __builtin_fmaf(a.b2, v, a.omb2 * (diff * diff));
        if (clamp_v) v_new = __builtin_fminf(v_new, 65000.0f);
        float sigma = __builtin_fmaf(sqrt_rn(__builtin_fmaxf(v_new, 0.0f)), a.c1, a.c2);
        return tanh_pade(clm / __builtin_fmaxf(sigma, 1.0e-12f));
    } else if constexpr (MODE == LV_BUFFER_T2) {
        float clm = __builtin_fmaf(a.b1sq, m, a.omb1sq * g);
        float diff = clamp_defect(g - m);
        v_new = __builtin_fmaf(a.b2, v, a.omb2 * (diff * diff));
        if (clamp_v) v_new = __builtin_fminf(v_new, 65000.0f);
        float env0 = __builtin_fmaf(a.b1sq, fabsf(m), a.eps);
        float env1 = __builtin_fmaf(a.omb1sq, fabsf(g), env0);
        float env2 = __builtin_fmaf(a.lam1, fabsf(diff), env1);
        float env = __builtin_fmaf(a.c_sigma, sqrt_rn(__builtin_fmaxf(v_new, 0.0f)), env2);
        return clm / env;
    } else {
        float clm = __builtin_fmaf(a.b1sq, m, a.omb1sq * g);
        float diff = clamp_defect(g - m);
        float env0 = __builtin_fmaf(a.b1sq, fabsf(m), a.eps);
        float env1 = __builtin_fmaf(a.omb1sq, fabsf(g), env0);
        float env = __builtin_fmaf(a.lam, fabsf(diff), env1);
        v_new = 0.0f;
        return clm / env;
    }
}

// ------------------------------------------------------------------ loads / stores

template <int DT>
__device__ __forceinline__ float load1(const void *base, uint64_t i) {
    if constexpr (DT == LV_DTYPE_F32) {
        return static_cast<const float *>(base)[i];
    } else if constexpr (DT == LV_DTYPE_BF16) {
        return bits_f((uint32_t) static_cast<const uint16_t *>(base)[i] << 16);
    } else {
        return f16_to_f32(static_cast<const uint16_t *>(base)[i]);
    }
}

template <int DT>
__device__ __forceinline__ void store1(void *base, uint64_t i, float x) {
    if constexpr (DT == LV_DTYPE_F32) {
        static_cast<float *>(base)[i] = x;
    } else if constexpr (DT == LV_DTYPE_BF16) {
        static_cast<uint16_t *>(base)[i] = (uint16_t)(f_bits(x) >> 16);
    } else {
        static_cast<uint16_t *>(base)[i] = (uint16_t)f32_to_f16_rne(x);
    }
}

__device__ __forceinline__ float load1_dyn(int dt, const void *base, uint64_t i) {
    if (dt == LV_DTYPE_BF16) return load1<LV_DTYPE_BF16>(base, i);
    if (dt == LV_DTYPE_F32) return load1<LV_DTYPE_F32>(base, i);
    return load1<LV_DTYPE_F16>(base, i);
}

// One thread's 4 or 8 elements as raw vectors, kept undecoded while the loads are in flight.
// Vector-path loads and stores are non-temporal: the step streams every byte exactly once, so
// nothing is worth keeping in L2 or the MALL, and streaming hints measurably raise HBM
// throughput for this 4-read/3-write pattern.
// Layout of a work unit of H 1024-element halves: thread t owns elements [4t, 4t+4) of each
// half, so every wave-wide load or store instruction covers one contiguous span (1 KiB for
// f32, 512 B for 16-bit types). 32-bit types use `a` (first half) and `b` (second half);
// 16-bit types pack both halves into `a` (.xy first half, .zw second half).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct Raw8 {
    u32x4 a, b;
};

// H (1 or 2) is the number of 1024-element halves in the unit: a thread moves 4 * H elements.
template <int DT, int H>
__device__ __forceinline__ Raw8 load_raw(const void *base, uint64_t h0) {
    Raw8 r;
    if constexpr (DT == LV_DTYPE_F32) {
        const float *f = static_cast<const float *>(base);
        r.a = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(f + h0));
        if constexpr (H == 2) r.b = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(f + h0 + kHalf));
        else r.b = u32x4{0, 0, 0, 0};
    } else {
        const uint16_t *h = static_cast<const uint16_t *>(base);
        u32x2 x = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(h + h0));
        u32x2 y = u32x2{0, 0};
        if constexpr (H == 2) y = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(h + h0 + kHalf));
        r.a = u32x4{x.x, x.y, y.x, y.y};
        r.b = u32x4{0, 0, 0, 0};
    }
    return r;
}

template <int H>
__device__ __forceinline__ Raw8 load_raw_dyn(int dt, const void *base, uint64_t h0) {
    if (dt == LV_DTYPE_F32) return load_raw<LV_DTYPE_F32, H>(base, h0);
    return load_raw<LV_DTYPE_BF16, H>(base, h0);  // 16-bit types share the raw layout
}

// Stores 4 * H values in the same layout; 16-bit values are already exact in the target
// type (quantised), so bf16 is a truncation (worker.rs:55-63) and f16 an exact RNE encode.
template <int DT, int H>
__device__ __forceinline__ void store_raw(void *base, uint64_t h0, const float in[8]) {
    if constexpr (DT == LV_DTYPE_F32) {
        float *f = static_cast<float *>(base);
        __builtin_nontemporal_store(f32x4{in[0], in[1], in[2], in[3]}, reinterpret_cast<f32x4 *>(f + h0));
        if constexpr (H == 2)
            __builtin_nontemporal_store(f32x4{in[4], in[5], in[6], in[7]}, reinterpret_cast<f32x4 *>(f + h0 + kHalf));
    } else {
        uint32_t ws[4];
#pragma unroll
        for (int k = 0; k < 2 * H; k++) {
            uint32_t lo, hi;
            if constexpr (DT == LV_DTYPE_BF16) {
                lo = f_bits(in[2 * k]) >> 16;
                hi = f_bits(in[2 * k + 1]) & 0xFFFF0000u;
            } else {
                lo = f32_to_f16_rne(in[2 * k]);
                hi = f32_to_f16_rne(in[2 * k + 1]) << 16;
            }
            ws[k] = lo | hi;
        }
        uint16_t *h = static_cast<uint16_t *>(base);
        __builtin_nontemporal_store(u32x2{ws[0], ws[1]}, reinterpret_cast<u32x2 *>(h + h0));
        if constexpr (H == 2) __builtin_nontemporal_store(u32x2{ws[2], ws[3]}, reinterpret_cast<u32x2 *>(h + h0 + kHalf));
    }
}

template <int DT, int H>
__device__ __forceinline__ void decode_raw(const Raw8 &r, float out[8]) {
    if constexpr (DT == LV_DTYPE_F32) {
        out[0] = bits_f(r.a.x); out[1] = bits_f(r.a.y); out[2] = bits_f(r.a.z); out[3] = bits_f(r.a.w);
        if constexpr (H == 2) {
            out[4] = bits_f(r.b.x); out[5] = bits_f(r.b.y); out[6] = bits_f(r.b.z); out[7] = bits_f(r.b.w);
        }
    } else {
        uint32_t ws[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
        for (int k = 0; k < 2 * H; k++) {
            if constexpr (DT == LV_DTYPE_BF16) {
                out[2 * k] = bits_f(ws[k] << 16);
                out[2 * k + 1] = bits_f(ws[k] & 0xFFFF0000u);
            } else {
                out[2 * k] = f16_to_f32(ws[k] & 0xFFFFu);
                out[2 * k + 1] = f16_to_f32(ws[k] >> 16);
            }
        }
    }
}

template <int H>
__device__ __forceinline__ void decode_raw_dyn(int dt, const Raw8 &r, float out[8]) {
    if (dt == LV_DTYPE_BF16) decode_raw<LV_DTYPE_BF16, H>(r, out);
    else if (dt == LV_DTYPE_F32) decode_raw<LV_DTYPE_F32, H>(r, out);
    else decode_raw<LV_DTYPE_F16, H>(r, out);
}

// The loads of one work unit that are in flight while the previous unit computes.
// p holds the param or, with master weights, the f32 master: one field for both, so that the
// run-time choice never becomes a select between two register arrays (which the compiler would
// place in scratch memory).
struct Inflight {
    Raw8 p, g, m, v;
};

// ------------------------------------------------------------------ element update

struct Seeds {
    int32_t m, p, v;
};

// Hash inputs of one element offset for the m, p and v streams.
struct HashIn {
    uint32_t m, p, v;
};

__device__ __forceinline__ HashIn hash_in(const Seeds &sd, uint32_t off) {
    return {off + (uint32_t)sd.m + kPrngAdd, off + (uint32_t)sd.p + kPrngAdd, off + (uint32_t)sd.v + kPrngAdd};
}

// Apply path for one element: dual.rs:150-228 and the matching blocks of dual.rs / tdclm.rs.
// Returns the cautious mask bit; u_eff is the (masked) direction whose square feeds the radial
// norm (dual.rs:176-180).
template <int MODE, int PT, int ST>
__device__ __forceinline__ uint32_t apply_elem(const Args &a, uint32_t flags, const HashIn &z,
                                               float cs, float bs, float p_init, float g_raw, float &m_io,
                                               float &v_io, float &p_out, float &mp_out, float &u_eff) {
    constexpr bool kTri = (MODE == LV_BUFFER_T1 || MODE == LV_BUFFER_T2);
    constexpr bool kDual = (MODE == LV_BUFFER_DUAL || MODE == LV_BUFFER_T2);
    const bool sr = flags & kFSR;
    float g = sanitize(g_raw);
    float m_new, v_new;
    float u = compute_u<MODE>(a, flags & kFClampV, g, m_io, v_io, m_new, v_new);
    bool active = (u * g) > 0.0f;
    float m_mask = active ? 1.0f : 0.0f;
    m_io = quantize<ST>(m_new, z.m, sr);
    if constexpr (kDual) v_io = quantize<ST>(v_new, z.v, sr);
    u_eff = (flags & kFCautious) ? u * m_mask : u;
    float delta = (flags & kFCautious) ? u_eff * cs : u;
    float step = a.lr * delta;
    if (flags & kFRadial) step *= bs;
    else if (flags & kFCoordinate) step = coordinate_bound<kTri>(step, p_init, a.ratio);
    if constexpr (PT == LV_DTYPE_F16) step = fp16_safety_bound<kTri>(step, p_init);
    float p_dec = (flags & kFWeightDecay) ? __builtin_fmaf(a.neg_lr_wd, p_init, p_init) : p_init;
    float p_upd = p_dec - step;
    if (flags & kFMaster) {
        mp_out = p_upd;
        p_out = quantize<PT>(p_upd, z.p, false);
    } else {
        p_out = quantize<PT>(p_upd, z.p, sr);
    }
    return active ? 1u : 0u;
}

// Counting path for one element (dual.rs:279-303, dual.rs:720-746, tdclm.rs:232-248).
template <int MODE>
__device__ __forceinline__ uint32_t count_elem(const Args &a, uint32_t flags, float g_raw, float m, float v,
                                               float &u_eff) {
    float g = sanitize(g_raw);
    float m_new, v_new;
    float u = compute_u<MODE>(a, flags & kFClampV, g, m, v, m_new, v_new);
    bool active = (u * g) > 0.0f;
    u_eff = (flags & kFCautious) ? u * (active ? 1.0f : 0.0f) : u;
    return active ? 1u : 0u;
}

// ------------------------------------------------------------------ scratch finalisation

// Last block of tensor t: dual.rs:255-259 + math.rs:188-239 (fused), dual.rs:330-351 +
// dual.rs:436-438 (two-pass count).  Thread 0 only. Slots 3/4 end at 1.0 when cautious /
// radial is off, the value the reference's host layer forces before every step
// (luminav.py:1748-1751).
template <int MODE, int PASS>
__device__ void finalize_scratch(const Args &a, bool radial, const Desc &D, unsigned long long mask_count,
                                 float u_sq, float p_sq) {
    constexpr bool kTri = (MODE == LV_BUFFER_T1 || MODE == LV_BUFFER_T2);
    float *s = D.scratch;
    const bool cautious = a.flags & kFCautious;
    float mask_sum = u64_to_f32_rn(mask_count);
    float total = u64_to_f32_rn(D.n);
    float s3, s4 = 1.0f;
    if constexpr (PASS == kFused) {
        s3 = cautious ? __builtin_fmaf(a.ema, s[3], a.ema_c * cautious_scale(mask_sum, total, a.clamp_min)) : 1.0f;
        if (radial)
            s4 = __builtin_fmaf(a.ema, s[4], a.ema_c * radial_scale<kTri>(u_sq, p_sq, s3, a.lr, a.ratio));
    } else {
        s3 = cautious ? cautious_scale(mask_sum, total, a.clamp_min) : 1.0f;
        if (radial) s4 = radial_scale<kTri>(u_sq, p_sq, s3, a.lr, a.ratio);
    }
    s[0] = 0.0f;
    s[1] = 0.0f;
    s[2] = 0.0f;
    s[3] = s3;
    s[4] = s4;
    s[5] = 0.0f;
}

// Butterfly sum over the 64 lanes; every lane ends with the same, order-fixed value.
__device__ __forceinline__ double wave_sum(double x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
    return x;
}

__device__ __forceinline__ uint32_t wave_sum(uint32_t x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
    return x;
}

__device__ __forceinline__ unsigned long long wave_sum(unsigned long long x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)x, off, 64);
        const uint32_t hi = __shfl_xor((uint32_t)(x >> 32), off, 64);
        x += ((unsigned long long)hi << 32) | lo;
    }
    return x;
}

// Block-wide sums in a fixed order (lanes by butterfly, then the 4 waves in order); the result
// is valid in thread 0, which reads the shared slots after the barrier: a second call by the
// same block needs a barrier in between.
struct BlockSums {
    double su[kThreads / 64];
    double sp[kThreads / 64];
    unsigned long long cnt[kThreads / 64];
};

template <typename C>
__device__ __forceinline__ void block_sums(BlockSums &sh, double &su, double &sp, C &cnt) {
    su = wave_sum(su);
    sp = wave_sum(sp);
    cnt = wave_sum(cnt);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sh.su[w] = su;
        sh.sp[w] = sp;
        sh.cnt[w] = cnt;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        su = sh.su[0];
        sp = sh.sp[0];
        cnt = (C)sh.cnt[0];
#pragma unroll
        for (int k = 1; k < kThreads / 64; k++) {
            su += sh.su[k];
            sp += sh.sp[k];
            cnt += (C)sh.cnt[k];
        }
    }
}

__device__ __forceinline__ double load_relaxed(const double *p) {
    uint64_t b = __hip_atomic_load(reinterpret_cast<const uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __longlong_as_double((long long)b);
}

// ------------------------------------------------------------------ per-unit work

// First unit of tensor t, and its descriptor, in an inline or a table launch.
template <bool TABLE>
__device__ __forceinline__ uint32_t unit_begin_of(const Args &a, int t) {
    if constexpr (TABLE) return a.ubegin[t];
    else return a.d[t].unit_begin;
}

template <bool TABLE>
__device__ __forceinline__ const Desc &desc_of(const Args &a, int t) {
    if constexpr (TABLE) return a.dtab[t];
    else return a.d[t];
}

// What a block needs to know about the tensor that owns its current unit.
struct View {
    uint32_t t_begin, t_end;  // the tensor's unit range in the launch
    uint64_t n;
    bool vec_ok;              // every pointer 16-byte aligned: whole units take the vector path
    float cs, bs;             // cautious / radial scale read from the scratch (fused, apply)
    Seeds sd;
    uint32_t ibase;
};

template <int MODE, int PASS, bool TABLE>
__device__ __forceinline__ View open_view(const Args &a, const Desc &D, int t, uint32_t flags, uint32_t unit) {
    constexpr bool kDual = (MODE == LV_BUFFER_DUAL || MODE == LV_BUFFER_T2);
    View tv;
    tv.t_begin = unit_begin_of<TABLE>(a, t);
    tv.t_end = (t + 1 < a.ndesc) ? unit_begin_of<TABLE>(a, t + 1) : a.total_units;
    tv.n = D.n;
    uintptr_t al = (uintptr_t)D.p | (uintptr_t)D.g | (uintptr_t)D.m;
    if (kDual) al |= (uintptr_t)D.v;
    if (flags & kFMaster) al |= (uintptr_t)D.mp;
    tv.vec_ok = (al & 15u) == 0;
    tv.ibase = D.ibase;
    uint32_t raw = a.seed_base + D.pidx * 10007u;
    tv.sd.m = (int32_t)(raw & 0x7FFFFFFFu);
    tv.sd.p = (int32_t)(((uint32_t)tv.sd.m + 0x55555555u) & 0x7FFFFFFFu);
    tv.sd.v = (int32_t)(((uint32_t)tv.sd.m + 0x2A6D365Bu) & 0x7FFFFFFFu);
    tv.cs = 1.0f;
    tv.bs = 1.0f;
    if constexpr (PASS == kFused || PASS == kApply) {
        tv.cs = D.scratch[3];
        tv.bs = D.scratch[4];
    }
    if constexpr (PASS == kSingle) {
        // reset_accumulators (state.rs:105-111) with the host-side forcing of slots 3/4
        // that the reference applies when cautious/radial are off (luminav.py:1748-1751).
        if (unit == tv.t_begin && threadIdx.x == 0) {
            float *sc = D.scratch;
            sc[0] = 0.0f; sc[1] = 0.0f; sc[2] = 0.0f; sc[3] = 1.0f; sc[4] = 1.0f; sc[5] = 0.0f;
        }
    }
    return tv;
}

// Vector loads of one whole, aligned unit.
template <int MODE, int PT, int ST, int PASS, int H>
__device__ __forceinline__ Inflight issue_unit(const Desc &D, const View &tv, uint32_t flags, bool radial, uint32_t u) {
    constexpr bool kDual = (MODE == LV_BUFFER_DUAL || MODE == LV_BUFFER_T2);
    const int gdt = (int)((flags >> 8) & 3u);
    Inflight f;
    const uint64_t e = (uint64_t)(u - tv.t_begin) * (kHalf * H) + (uint64_t)threadIdx.x * 4u;
    f.g = load_raw_dyn<H>(gdt, D.g, e);
    f.m = load_raw<ST, H>(D.m, e);
    if constexpr (kDual) f.v = load_raw<ST, H>(D.v, e);
    if (PASS != kCount || radial) {  // the count pass reads p only for the radial norm
        if (flags & kFMaster) f.p = load_raw<LV_DTYPE_F32, H>(D.mp, e);
        else f.p = load_raw<PT, H>(D.p, e);
    }
    return f;
}

// Update (or count) one whole, aligned unit from its loaded vectors and store it.
template <int MODE, int PT, int ST, int PASS, int H>
__device__ __forceinline__ void process_unit(const Args &a, const Desc &D, const View &tv, uint32_t flags, bool radial,
                                             const Inflight &cur, uint32_t u, uint32_t &cnt, double &su, double &sp) {
    constexpr bool kDual = (MODE == LV_BUFFER_DUAL || MODE == LV_BUFFER_T2);
    constexpr bool kCounting = (PASS == kFused || PASS == kCount);
    const int gdt = (int)((flags >> 8) & 3u);
    const bool master = flags & kFMaster;
    const uint64_t e0 = (uint64_t)(u - tv.t_begin) * (kHalf * H) + (uint64_t)threadIdx.x * 4u;
    float g[8], m[8], v[8];
    decode_raw_dyn<H>(gdt, cur.g, g);
    decode_raw<ST, H>(cur.m, m);
    if constexpr (kDual) decode_raw<ST, H>(cur.v, v);
    if constexpr (PASS == kCount) {
        float pin[8];
        if (radial) {
            if (master) decode_raw<LV_DTYPE_F32, H>(cur.p, pin);
            else decode_raw<PT, H>(cur.p, pin);
        }
#pragma unroll
        for (int j = 0; j < 4 * H; j++) {
            float ue;
            // every lane of the wave is on this path: count the wave's mask bits in one ballot
            cnt += (uint32_t)__popcll(__ballot(count_elem<MODE>(a, flags, g[j], m[j], kDual ? v[j] : 0.0f, ue)));
            if (radial) {
                su += (double)(ue * ue);
                sp += (double)(pin[j] * pin[j]);
            }
        }
    } else {
        float pin[8], pout[8], mpout[8];
        if (master) decode_raw<LV_DTYPE_F32, H>(cur.p, pin);
        else decode_raw<PT, H>(cur.p, pin);
        // the thread's hash inputs at its first element (offsets wrap at 2^32 as (int32)idx does)
        const HashIn zb = hash_in(tv.sd, (uint32_t)e0 + tv.ibase);
#pragma unroll
        for (int j = 0; j < 4 * H; j++) {
            float vj = kDual ? v[j] : 0.0f;
            float ue;
            const uint32_t jj = j < 4 ? (uint32_t)j : kHalf + (uint32_t)j - 4u;  // a constant once unrolled
            const HashIn zj = {zb.m + jj, zb.p + jj, zb.v + jj};
            uint32_t act = apply_elem<MODE, PT, ST>(a, flags, zj, tv.cs, tv.bs, pin[j], g[j], m[j], vj, pout[j],
                                                    mpout[j], ue);
            if constexpr (kDual) v[j] = vj;
            if constexpr (kCounting) {
                cnt += (uint32_t)__popcll(__ballot(act));  // the wave's count (all lanes active here)
                if (radial) {
                    su += (double)(ue * ue);
                    sp += (double)(pin[j] * pin[j]);
                }
            }
        }
        store_raw<PT, H>(D.p, e0, pout);
        if (master) store_raw<LV_DTYPE_F32, H>(D.mp, e0, mpout);
        store_raw<ST, H>(D.m, e0, m);
        if constexpr (kDual) store_raw<ST, H>(D.v, e0, v);
    }
}

// Per-element path for one unit: the partial last unit of a tensor and unaligned tensors.
// nskip > 0: the unit overlaps the tensor's inactive ranges, `first` is the first range that ends
// after the unit's first element. Inactive elements are computed with a zero gradient (they count
// in the statistics) and not stored.
template <int MODE, int PT, int ST, int PASS, int H>
__device__ __forceinline__ void scalar_unit(const Args &a, const Desc &D, const View &tv, uint32_t flags, bool radial,
                                            uint32_t u, uint32_t &cnt, double &su, double &sp, uint32_t nskip = 0,
                                            uint32_t first = 0) {
    constexpr bool kDual = (MODE == LV_BUFFER_DUAL || MODE == LV_BUFFER_T2);
    constexpr bool kCounting = (PASS == kFused || PASS == kCount);
    constexpr uint64_t kPer = 4 * H;  // consecutive elements per thread
    const int gdt = (int)((flags >> 8) & 3u);
    const bool master = flags & kFMaster;
    const uint64_t e0 = (uint64_t)(u - tv.t_begin) * (kHalf * H) + (uint64_t)threadIdx.x * kPer;
    const uint64_t e1 = (e0 + kPer < tv.n) ? e0 + kPer : tv.n;
    uint32_t r = first;
    for (uint64_t i = e0; i < e1; i++) {
        bool inactive = false;
        if (nskip) {
            while (r < nskip && D.skip[2 * r + 1] <= i) r++;
            inactive = r < nskip && D.skip[2 * r] <= i;
        }
        float g = inactive ? 0.0f : load1_dyn(gdt, D.g, i);
        float m = load1<ST>(D.m, i);
        float v = kDual ? load1<ST>(D.v, i) : 0.0f;
        if constexpr (PASS == kCount) {
            float ue;
            cnt += count_elem<MODE>(a, flags, g, m, v, ue);
            if (radial) {
                float pin = master ? D.mp[i] : load1<PT>(D.p, i);
                su += (double)(ue * ue);
                sp += (double)(pin * pin);
            }
        } else {
            float pin = master ? D.mp[i] : load1<PT>(D.p, i);
            float pout, mpout, ue;
            uint32_t act = apply_elem<MODE, PT, ST>(a, flags, hash_in(tv.sd, (uint32_t)i + tv.ibase), tv.cs, tv.bs,
                                                    pin, g, m, v, pout, mpout, ue);
            if (!inactive) {
                store1<PT>(D.p, i, pout);
                if (master) D.mp[i] = mpout;
                store1<ST>(D.m, i, m);
                if constexpr (kDual) store1<ST>(D.v, i, v);
            }
            if constexpr (kCounting) {
                cnt += act;
                if (radial) {
                    su += (double)(ue * ue);
                    sp += (double)(pin * pin);
                }
            }
        }
    }
}

// How the tensor's inactive ranges cover the elements [e0, e1): 0 not at all, 1 partly, 2 fully.
// `first` receives the first range that ends after e0. Block-uniform.
__device__ __forceinline__ int inactive_cover(const Desc &D, uint64_t e0, uint64_t e1, uint32_t &first) {
    uint32_t lo = 0, hi = D.nskip;
    while (lo < hi) {
        uint32_t mid = (lo + hi) >> 1;
        if (D.skip[2 * mid + 1] <= e0) lo = mid + 1;
        else hi = mid;
    }
    first = lo;
    if (lo == D.nskip) return 0;
    const uint64_t b = D.skip[2 * lo], e = D.skip[2 * lo + 1];
    if (b >= e1) return 0;
    return (b <= e0 && e >= e1) ? 2 : 1;
}

// Index of the tensor that owns `unit`: binary search of the unit ranges.
template <bool TABLE>
__device__ __forceinline__ int find_tensor(const Args &a, uint32_t unit) {
    int lo = 0, hi = a.ndesc - 1;
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (unit_begin_of<TABLE>(a, mid) <= unit) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// ------------------------------------------------------------------ the kernels

// Counting unit launches: thread 0 of every block reports its exact mask count and the block's
// completion in ONE 64-bit atomic (count << kTicketBits | 1) on one of the tensor's kSlots slot
// words (slot = unit index in the tensor mod kSlots, 64 B apart, so the atomics spread over
// L2 channels). The block whose report completes a slot (its ticket reaches the slot's block
// count) holds that slot's whole count in the value its own atomic returned, re-zeroes the slot
// and reports count << kFoldBits | 1 on the tensor's fold word; the block that completes the
// fold word holds the tensor's exact count and finalises the scratch. Every decision reads only
// the value returned by an atomic on that same word, so no fence is needed (a device-scope
// release fence per block measured 7x slower); integer sums are exact in any order, so the
// result is deterministic. Wholly inactive units report a zero count.
template <int MODE, int PASS>
__device__ __forceinline__ void report_count(const Args &a, int t, const Desc &D, const View &tv, uint32_t unit,
                                             uint32_t count) {
    const uint32_t n_units = tv.t_end - tv.t_begin;
    const uint32_t k = unit - tv.t_begin;
    const uint32_t s = k % kSlots;
    unsigned long long *words = a.slots + (size_t)t * kSlotWords * kSlotStride;
    unsigned long long *slot = words + (size_t)s * kSlotStride;
    constexpr unsigned long long kTicketMask = (1ull << kTicketBits) - 1ull;
    const unsigned long long old = __hip_atomic_fetch_add(slot, ((unsigned long long)count << kTicketBits) | 1ull,
                                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t expect = n_units / kSlots + (s < n_units % kSlots ? 1u : 0u);
    if ((uint32_t)(old & kTicketMask) + 1u != expect) return;
    const unsigned long long slot_count = (old >> kTicketBits) + count;
    __hip_atomic_store(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned long long *fold = words + (size_t)kSlots * kSlotStride;
    const unsigned long long prev = __hip_atomic_fetch_add(fold, (slot_count << kFoldBits) | 1ull, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t nslots = n_units < kSlots ? n_units : kSlots;
    if ((uint32_t)(prev & ((1ull << kFoldBits) - 1ull)) + 1u != nslots) return;
    __hip_atomic_store(fold, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    finalize_scratch<MODE, PASS>(a, false, D, (prev >> kFoldBits) + slot_count, 0.0f, 0.0f);
}

// Unit launch: each block updates exactly one work unit (1024 or 2048 elements, unit_halves) and
// exits.
// The hardware keeps every CU full with fresh blocks, so the loads of some blocks overlap the
// arithmetic of others without a software pipeline; on MI355X this launch shape streams HBM
// faster than any persistent grid-stride loop over the same buffers (measured: 23.4 vs 26.5 ms
// for the 6.7e9-element T2 step; 2048-element units: 23.7 ms). Counting passes report each
// block's exact mask count (report_count), and the last block of each tensor finalises its
// scratch, so a step is one launch. Radial counting passes instead store each unit's record
// (mask count and f64 squared-norm sums) for fold_kernel.
// FL is either kFDynamic (flags read at run time) or the exact flag word of the launch, in
// which case every option test folds at compile time and the per-element code is straight-line.
// TABLE: the tensor table is in device memory (a.dtab) and the first units in a.ubegin.
template <int MODE, int PT, int ST, int PASS, uint32_t FL, bool TABLE>
__global__ void __launch_bounds__(kThreads) unit_kernel(const Args a) {
    constexpr bool kCounting = (PASS == kFused || PASS == kCount);
    __shared__ BlockSums sh;

    const uint32_t flags = (FL & kFDynamic) ? a.flags : FL;
    const bool radial = kCounting && (flags & kFRadial);  // squared norms summed in this pass
    // Workgroups are dispatched to the XCDs round-robin (block b runs on XCD b mod X). Map them so
    // that each XCD streams one contiguous range of units (measured ~1% faster than b -> b).
    // Every block is short-lived, so its prologue is on the critical path: b / X comes from the
    // host's reciprocal (exact for b < 2^23 and X <= 64) instead of an integer division, which
    // measured 1.3% of the cfg5 step.
    const uint32_t b = blockIdx.x;
    const uint32_t i = (uint32_t)(((uint64_t)b * a.xcd_recip) >> 40);
    const uint32_t x = b - i * a.xcds;
    const uint32_t unit = a.unit_base + x * a.xcd_q + (x < a.xcd_r ? x : a.xcd_r) + i;
    const int t = find_tensor<TABLE>(a, unit);
    const Desc &D = desc_of<TABLE>(a, t);
    const View tv = open_view<MODE, PASS, TABLE>(a, D, t, flags, unit);
    uint32_t cnt = 0;
    double su = 0.0, sp = 0.0;  // radial: sum u_eff^2, sum p^2
    constexpr int H = unit_halves(MODE, PT, ST);
    int cover = 0;
    uint32_t first = 0;
    if (D.nskip) {
        const uint64_t e0 = (uint64_t)(unit - tv.t_begin) * (kHalf * H);
        cover = inactive_cover(D, e0, e0 + kHalf * H < tv.n ? e0 + kHalf * H : tv.n, first);
        // A wholly inactive unit has a zero gradient (its mask count is 0) and writes nothing;
        // its elements still enter the radial norms.
        if (!kCounting && cover == 2) return;
    }
    // Vector path: cnt ends as the wave's count (the same in every lane, from ballots); per-element
    // path: cnt is the lane's count.
    const bool vec = cover == 0 && tv.vec_ok && unit < tv.t_begin + (uint32_t)(tv.n / (kHalf * H));
    if (vec) {
        const Inflight f = issue_unit<MODE, PT, ST, PASS, H>(D, tv, flags, radial, unit);
        // Waves whose loads are in flight outrank freshly started ones, so a SIMD finishes (and
        // stores) the units it holds before new blocks add loads: ~0.5% more HBM throughput.
        __builtin_amdgcn_s_setprio(1);
        process_unit<MODE, PT, ST, PASS, H>(a, D, tv, flags, radial, f, unit, cnt, su, sp);
    } else if (cover != 2 || radial) {
        scalar_unit<MODE, PT, ST, PASS, H>(a, D, tv, flags, radial, unit, cnt, su, sp, cover ? D.nskip : 0, first);
    }
    if constexpr (kCounting) {
        if (radial) {
            uint32_t lane_cnt = vec ? ((threadIdx.x & 63) == 0 ? cnt : 0u) : cnt;
            block_sums(sh, su, sp, lane_cnt);
            cnt = lane_cnt;
            if (threadIdx.x == 0) {
                const uint32_t k = unit - a.unit_base;  // < piece_units
                a.unit_sq[2 * (size_t)k] = su;
                a.unit_sq[2 * (size_t)k + 1] = sp;
                a.unit_cnt[k] = cnt;
            }
        } else {
            if (!vec) cnt = wave_sum(cnt);  // block-uniform branch
            if ((threadIdx.x & 63) == 0) sh.cnt[threadIdx.x >> 6] = cnt;
            __syncthreads();
            if (threadIdx.x == 0) {
                uint32_t tot = 0;
#pragma unroll
                for (int k = 0; k < kThreads / 64; k++) tot += (uint32_t)sh.cnt[k];
                report_count<MODE, PASS>(a, t, D, tv, unit, tot);
            }
        }
    }
}

// Units of tensor t inside the piece [ub, ue) of the launch's unit space: [lo, hi).
__host__ __device__ inline void piece_span(const Args &a, int t, uint32_t ub, uint32_t ue, uint32_t &lo, uint32_t &hi) {
    const uint32_t tb = a.d[t].unit_begin;
    const uint32_t te = (t + 1 < a.ndesc) ? a.d[t + 1].unit_begin : a.total_units;
    lo = tb > ub ? tb : ub;
    hi = te < ue ? te : ue;
    if (hi < lo) hi = lo;
}

// Radial fold, one launch after each piece of a radial counting launch. The piece's units are
// cut, per tensor, into chunks of kFoldChunk; block j sums the unit records of chunk j into
// chunk record j (thread k adds records k, k + 256, ... in order, kFoldBatch loads in flight,
// then the fixed block order), and the block that completes a tensor's chunks (per-tensor
// ticket, release/acquire fences: <= 1072 blocks per piece, after a kernel boundary that already
// wrote the L2 back) sums the tensor's chunk records in order, adds them after the running sum
// of the earlier pieces, and either stores the new running sum or, in the piece that holds the
// tensor's last unit, finalises the scratch. Every sum runs in an order fixed by the unit and
// piece sizes.
template <int MODE, int PASS>
__global__ void __launch_bounds__(kThreads) fold_kernel(const Args a) {
    __shared__ BlockSums sh;
    __shared__ uint32_t last;
    const uint32_t ub = a.unit_base, ue = a.unit_base + a.piece_units;
    uint32_t j = blockIdx.x, cbase = 0, lo = 0, hi = 0, nc = 0;
    int t = 0;
    for (; t < a.ndesc; t++) {  // block-uniform; the grid is exactly the piece's chunk count
        piece_span(a, t, ub, ue, lo, hi);
        nc = (hi - lo + kFoldChunk - 1) / kFoldChunk;
        if (j < nc) break;
        j -= nc;
        cbase += nc;
    }
    if (t == a.ndesc) return;
    const uint32_t u0 = lo + j * kFoldChunk;
    const uint32_t u1 = (hi - u0 > kFoldChunk) ? u0 + kFoldChunk : hi;
    double su = 0.0, sp = 0.0;
    uint32_t cnt = 0;
    const uint32_t k0 = u0 - ub, k1 = u1 - ub;  // piece-relative record indices, <= kRadialPiece
    const double2 *sq = reinterpret_cast<const double2 *>(a.unit_sq);
    for (uint32_t kb = k0; kb < k1; kb += kFoldBatch * kThreads) {  // block-uniform
        double2 x[kFoldBatch];
        uint32_t c[kFoldBatch];
#pragma unroll
        for (int r = 0; r < kFoldBatch; r++) {
            const uint32_t k = kb + r * kThreads + threadIdx.x;
            const uint32_t kc = k < k1 ? k : k0;  // always in range, so every load can issue at once
            x[r] = sq[kc];
            c[r] = a.unit_cnt[kc];
        }
#pragma unroll
        for (int r = 0; r < kFoldBatch; r++) {
            if (kb + r * kThreads + threadIdx.x < k1) {
                su += x[r].x;
                sp += x[r].y;
                cnt += c[r];
            }
        }
    }
    block_sums(sh, su, sp, cnt);
    if (threadIdx.x == 0) {
        RadialSum *r = a.chunks + cbase + j;
        r->su = su;
        r->sp = sp;
        r->cnt = cnt;
        __threadfence();
        const unsigned long long prev = atomicAdd(&a.tickets[t], 1ull);
        last = (prev + 1ull == (unsigned long long)nc) ? 1u : 0u;
    }
    __syncthreads();
    if (!last) return;  // block-uniform
    __threadfence();
    su = 0.0;
    sp = 0.0;
    unsigned long long total = 0;
    for (uint32_t k = threadIdx.x; k < nc; k += kThreads) {
        const RadialSum *r = a.chunks + cbase + k;
        su += load_relaxed(&r->su);
        sp += load_relaxed(&r->sp);
        total += __hip_atomic_load(&r->cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    block_sums(sh, su, sp, total);
    if (threadIdx.x == 0) {
        RadialSum &run = a.run[t];
        if (lo != a.d[t].unit_begin) {  // earlier pieces hold the tensor's first units
            su = run.su + su;
            sp = run.sp + sp;
            total += run.cnt;
        }
        const uint32_t te = (t + 1 < a.ndesc) ? a.d[t + 1].unit_begin : a.total_units;
        if (hi == te) {
            finalize_scratch<MODE, PASS>(a, true, a.d[t], total, (float)su, (float)sp);
        } else {
            run.su = su;
            run.sp = sp;
            run.cnt = total;
        }
        __hip_atomic_store(&a.tickets[t], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ------------------------------------------------------------------ host side

using KernelFn = void (*)(Args);

// Flag word of the specialised ("static") instantiation: the reference defaults (cautious in
// the counting passes, stochastic rounding, weight decay, coordinate bound, no master, grad
// dtype = param dtype, v clamp for fp16 params).
constexpr uint32_t static_flags(int PT, int PASS) {
    return (PASS != kSingle ? (uint32_t)kFCautious : 0u) | (uint32_t)kFSR | (uint32_t)kFWeightDecay |
           (uint32_t)kFCoordinate | (PT == LV_DTYPE_F16 ? (uint32_t)kFClampV : 0u) | ((uint32_t)PT << 8);
}

// The same defaults with bound_type="radial" (the radial passes never run SINGLE).
constexpr uint32_t radial_flags(int PT) {
    return ((uint32_t)kFCautious | (uint32_t)kFSR | (uint32_t)kFWeightDecay | (uint32_t)kFRadial |
            (PT == LV_DTYPE_F16 ? (uint32_t)kFClampV : 0u) | ((uint32_t)PT << 8));
}

// Table launches (many small tensors, launch-bound) use the run-time-flag kernel only.
template <int MODE, int PT, int ST, int PASS>
KernelFn pick_flags(uint32_t flags, bool table) {
    constexpr uint32_t kStatic = static_flags(PT, PASS);
    constexpr uint32_t kRadial = radial_flags(PT);
    if (table) return unit_kernel<MODE, PT, ST, PASS, kFDynamic, true>;
    if (flags == kStatic) return unit_kernel<MODE, PT, ST, PASS, kStatic, false>;
    if (flags == kRadial) return unit_kernel<MODE, PT, ST, PASS, kRadial, false>;
    if constexpr (PASS == kFused) {
        // The steady step of common departures from the defaults: master weights, no stochastic
        // rounding, no weight decay. Where the step is VALU-bound the run-time-flag kernel costs
        // more: T2 with master weights and bf16 m/v on the cfg5 shape, 25.3 -> 23.2 ms.
        constexpr uint32_t kMaster = kStatic | kFMaster;
        constexpr uint32_t kNoSR = kStatic & ~(uint32_t)kFSR;
        constexpr uint32_t kNoWD = kStatic & ~(uint32_t)kFWeightDecay;
        if (flags == kMaster) return unit_kernel<MODE, PT, ST, PASS, kMaster, false>;
        if (flags == kNoSR) return unit_kernel<MODE, PT, ST, PASS, kNoSR, false>;
        if (flags == kNoWD) return unit_kernel<MODE, PT, ST, PASS, kNoWD, false>;
    }
    return unit_kernel<MODE, PT, ST, PASS, kFDynamic, false>;
}

template <int MODE, int PT, int ST>
KernelFn pick_pass(int pass, uint32_t flags, bool table) {
    switch (pass) {
    case kSingle: return pick_flags<MODE, PT, ST, kSingle>(flags, table);
    case kFused: return pick_flags<MODE, PT, ST, kFused>(flags, table);
    case kCount: return pick_flags<MODE, PT, ST, kCount>(flags, table);
    default: return pick_flags<MODE, PT, ST, kApply>(flags, table);
    }
}

template <int MODE, int PT>
KernelFn pick_state(int st, int pass, uint32_t flags, bool table) {
    return st == LV_DTYPE_F32 ? pick_pass<MODE, PT, LV_DTYPE_F32>(pass, flags, table)
                              : pick_pass<MODE, PT, LV_DTYPE_BF16>(pass, flags, table);
}

template <int MODE>
KernelFn pick_param(int pt, int st, int pass, uint32_t flags, bool table) {
    switch (pt) {
    case LV_DTYPE_F32: return pick_state<MODE, LV_DTYPE_F32>(st, pass, flags, table);
    case LV_DTYPE_BF16: return pick_state<MODE, LV_DTYPE_BF16>(st, pass, flags, table);
    default: return pick_state<MODE, LV_DTYPE_F16>(st, pass, flags, table);
    }
}

static KernelFn pick_kernel(int mode, int pt, int st, int pass, uint32_t flags, bool table) {
    switch (mode) {
    case LV_BUFFER_TDCLM: return pick_param<LV_BUFFER_TDCLM>(pt, st, pass, flags, table);
    case LV_BUFFER_DUAL: return pick_param<LV_BUFFER_DUAL>(pt, st, pass, flags, table);
    case LV_BUFFER_T1: return pick_param<LV_BUFFER_T1>(pt, st, pass, flags, table);
    default: return pick_param<LV_BUFFER_T2>(pt, st, pass, flags, table);
    }
}

template <int MODE>
KernelFn pick_fold_pass(int pass) {
    return pass == kFused ? fold_kernel<MODE, kFused> : fold_kernel<MODE, kCount>;
}

static KernelFn pick_fold(int mode, int pass) {
    switch (mode) {
    case LV_BUFFER_TDCLM: return pick_fold_pass<LV_BUFFER_TDCLM>(pass);
    case LV_BUFFER_DUAL: return pick_fold_pass<LV_BUFFER_DUAL>(pass);
    case LV_BUFFER_T1: return pick_fold_pass<LV_BUFFER_T1>(pass);
    default: return pick_fold_pass<LV_BUFFER_T2>(pass);
    }
}

static thread_local char g_err[512];

static int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

// compiler-builtins' __powidf2 (the lowering of Rust f64::powi): repeated squaring.
static double powi_rs(double a, int32_t b) {
    bool recip = b < 0;
    uint32_t pw = recip ? (uint32_t)(-(int64_t)b) : (uint32_t)b;
    double mul = 1.0;
    for (;;) {
        if (pw & 1u) mul *= a;
        pw >>= 1;
        if (pw == 0) break;
        a *= a;
    }
    return recip ? 1.0 / mul : mul;
}

struct StepCoeffs {
    float c1, c2, c_sigma;
};

// math.rs:27-81
static StepCoeffs step_coeffs(uint64_t step, float beta1, float beta2, float eps, float tau, float lam) {
    uint64_t safe = step > 1 ? step : 1;
    double b1 = (double)beta1, b2 = (double)beta2;
    double bc1 = safe < 2147483647ull ? 1.0 - powi_rs(b1, (int32_t)(safe + 1)) : 1.0 - std::pow(b1, (double)(safe + 1));
    double bc2_raw = safe <= 2147483647ull ? 1.0 - powi_rs(b2, (int32_t)safe) : 1.0 - std::pow(b2, (double)safe);
    double bc2 = std::fmax(bc2_raw, 1.0e-15);
    StepCoeffs c;
    c.c1 = (float)((bc1 * (double)tau) / std::sqrt(bc2));
    c.c2 = (float)((double)eps * bc1 * (double)tau);
    float bc2f = (float)bc2;
    c.c_sigma = (0.5f * lam) / std::sqrt(std::fmax(bc2f, 1.0e-15f));
    return c;
}

static int validate_config(const lv_config *c) {
    auto fin = [](float x) { return std::isfinite(x); };
    if (!fin(c->lr) || c->lr < 0.0f) return fail(LV_STATUS_INVALID_CONFIG, "Invalid learning rate: %g", c->lr);
    if (!fin(c->beta1) || !(c->beta1 >= 0.0f && c->beta1 < 1.0f))
        return fail(LV_STATUS_INVALID_CONFIG, "Invalid beta1 parameter: %g", c->beta1);
    if (!fin(c->beta2) || !(c->beta2 >= 0.0f && c->beta2 < 1.0f))
        return fail(LV_STATUS_INVALID_CONFIG, "Invalid beta2 parameter: %g", c->beta2);
    if (!fin(c->eps) || c->eps <= 0.0f) return fail(LV_STATUS_INVALID_CONFIG, "Invalid epsilon value: %g", c->eps);
    if (!fin(c->weight_decay) || c->weight_decay < 0.0f)
        return fail(LV_STATUS_INVALID_CONFIG, "Invalid weight_decay value: %g", c->weight_decay);
    if (!fin(c->tau) || c->tau <= 0.0f) return fail(LV_STATUS_INVALID_CONFIG, "Invalid tau parameter: %g", c->tau);
    if (!fin(c->lam) || c->lam < 0.0f) return fail(LV_STATUS_INVALID_CONFIG, "Invalid lam parameter: %g", c->lam);
    if (!fin(c->cautious_clamp_min) || c->cautious_clamp_min <= 0.0f || c->cautious_clamp_min > 1.0f)
        return fail(LV_STATUS_INVALID_CONFIG, "Invalid cautious_clamp_min: %g", c->cautious_clamp_min);
    if (!fin(c->bound_ratio) || c->bound_ratio <= 0.0f)
        return fail(LV_STATUS_INVALID_CONFIG, "Invalid bound_ratio: %g", c->bound_ratio);
    if (!fin(c->ema_decay) || c->ema_decay <= 0.0f || c->ema_decay >= 1.0f)
        return fail(LV_STATUS_INVALID_CONFIG, "Invalid ema_decay: %g", c->ema_decay);
    if (c->buffer < 1 || c->buffer > 4) return fail(LV_STATUS_INVALID_CONFIG, "Invalid buffer count: %d", c->buffer);
    if (c->bound_type < 0 || c->bound_type > 2)
        return fail(LV_STATUS_INVALID_CONFIG, "Invalid bound_type: %d", c->bound_type);
    if (c->master_weights < 0 || c->master_weights > 2)
        return fail(LV_STATUS_INVALID_CONFIG, "Invalid master_weights: %d", c->master_weights);
    return LV_STATUS_SUCCESS;
}

// XCDs of the current device (hipDeviceAttributeNumberOfXccs; 1 if unknown).
static uint32_t device_xcds() {
    static std::mutex mu;
    static std::vector<std::pair<int, uint32_t>> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    std::lock_guard<std::mutex> lk(mu);
    for (const auto &e : cache)
        if (e.first == dev) return e.second;
    int x = 0;
    if (hipDeviceGetAttribute(&x, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || x < 1 || x > 64) x = 1;
    cache.push_back({dev, (uint32_t)x});
    return (uint32_t)x;
}

struct Item {
    int idx;      // position in the caller's array (workspace slot)
    int pass;     // first pass of this tensor
    int pt, gt, st;
    bool master;
    bool clampv;  // fp16 param or fp16 state container: v <= 65000 (dual.rs:68-71)
    uint64_t step;
};

static int launch_one(KernelFn fn, const Args &args, uint32_t grid, uint32_t threads, hipStream_t stream) {
    void *kargs[] = {const_cast<Args *>(&args)};
    hipError_t e = hipLaunchKernel(reinterpret_cast<const void *>(fn), dim3(grid), dim3(threads), kargs, 0, stream);
    if (e != hipSuccess) return fail(LV_STATUS_EXECUTION_FAILED, "kernel launch failed: %s", hipGetErrorString(e));
    return LV_STATUS_SUCCESS;
}

// Gives the tensors of a launch consecutive ranges of units of `unit_elems` elements. A table
// launch (`table` = its descriptors in host staging memory) keeps the first units both in the
// staged descriptors and in the kernel arguments.
static int assign_units(Args &args, uint32_t unit_elems, Desc *table) {
    uint64_t units = 0;
    for (int k = 0; k < args.ndesc; k++) {
        Desc &D = table ? table[k] : args.d[k];
        D.unit_begin = (uint32_t)units;
        if (table) args.ubegin[k] = (uint32_t)units;
        units += (D.n + unit_elems - 1) / unit_elems;
        if (units > 0xFFFFFFFFull) return fail(LV_STATUS_INVALID_CONFIG, "too many work units in one launch");
    }
    args.total_units = (uint32_t)units;
    return LV_STATUS_SUCCESS;
}

// Pinned host staging for the descriptor tables of table launches: kStageSlots tables per
// device, used round-robin. A slot is written only after the upload that last read it has
// finished (its event), so the host rarely waits and the uploads stay asynchronous. A slot is
// leased to one call from acquire_staging until its upload is enqueued (release_staging), so
// host threads stepping on the same device never write the same slot.
constexpr int kStageSlots = 4;

struct Staging {
    int dev;
    Desc *host;
    hipEvent_t ev[kStageSlots];
    bool used[kStageSlots];  // an upload was enqueued from the slot (its event was recorded)
    bool busy[kStageSlots];  // leased to a call that has not enqueued its upload yet
    int next;
};

struct StagingLease {
    Staging *S = nullptr;
    int slot = -1;
    Desc *table = nullptr;
    hipEvent_t ev = nullptr;
};

static std::mutex g_stage_mu;
static std::vector<Staging *> g_stage;

// Leases a staging table of the current device, free for the host to write. Allocates the
// device's ring on first use (the only allocation of the step path, once per device and process).
static int acquire_staging(StagingLease &lease) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(LV_STATUS_NO_DRIVER, "no HIP device");
    std::unique_lock<std::mutex> lk(g_stage_mu);
    Staging *S = nullptr;
    for (Staging *x : g_stage)
        if (x->dev == dev) S = x;
    if (!S) {
        void *h = nullptr;
        if (hipHostMalloc(&h, sizeof(Desc) * kTableMax * kStageSlots, hipHostMallocDefault) != hipSuccess)
            return fail(LV_STATUS_EXECUTION_FAILED, "pinned staging allocation failed");
        Staging fresh{};
        fresh.dev = dev;
        fresh.host = static_cast<Desc *>(h);
        for (int k = 0; k < kStageSlots; k++) {
            if (hipEventCreateWithFlags(&fresh.ev[k], hipEventDisableTiming) != hipSuccess) {
                for (int j = 0; j < k; j++) (void)hipEventDestroy(fresh.ev[j]);
                (void)hipHostFree(h);
                return fail(LV_STATUS_EXECUTION_FAILED, "event creation failed");
            }
        }
        S = new Staging(fresh);  // kept until the process ends
        g_stage.push_back(S);
    }
    int k = S->next;
    while (S->busy[k]) {  // every slot leased by other threads' calls: wait for one to enqueue
        lk.unlock();
        std::this_thread::yield();
        lk.lock();
        k = S->next;
    }
    S->next = (k + 1) % kStageSlots;
    if (S->used[k] && hipEventSynchronize(S->ev[k]) != hipSuccess)
        return fail(LV_STATUS_EXECUTION_FAILED, "staging event wait failed");
    S->busy[k] = true;
    lease.S = S;
    lease.slot = k;
    lease.table = S->host + (size_t)k * kTableMax;
    lease.ev = S->ev[k];
    return LV_STATUS_SUCCESS;
}

// Ends a lease: `enqueued` says whether an upload from the slot was enqueued (and its event
// recorded after it).
static void release_staging(StagingLease &lease, bool enqueued) {
    if (!lease.S) return;
    std::lock_guard<std::mutex> lk(g_stage_mu);
    if (enqueued) lease.S->used[lease.slot] = true;
    lease.S->busy[lease.slot] = false;
    lease.S = nullptr;
}

// Table launches: assigns the units of the args.ndesc descriptors staged in `table` and
// uploads them to args.dtab on the stream; `staged` is recorded after the upload. The launches
// of the class (COUNT and APPLY use the same unit size) then read the uploaded table.
static int stage_table(Args &args, int mode, int pt, int st, Desc *table, hipEvent_t staged, hipStream_t stream) {
    int rc = assign_units(args, kHalf * unit_halves(mode, pt, st), table);
    if (rc != LV_STATUS_SUCCESS) return rc;
    if (hipMemcpyAsync(const_cast<Desc *>(args.dtab), table, sizeof(Desc) * args.ndesc, hipMemcpyHostToDevice,
                       stream) != hipSuccess ||
        hipEventRecord(staged, stream) != hipSuccess)
        return fail(LV_STATUS_EXECUTION_FAILED, "descriptor upload failed");
    return LV_STATUS_SUCCESS;
}

// Inline launch: the descriptors are in args.d and get their units here. Table launch: the
// table was staged (stage_table).
static int launch(Args &args, int mode, int pt, int st, int pass, hipStream_t stream, bool table = false) {
    KernelFn fn = pick_kernel(mode, pt, st, pass, args.flags, table);
    const bool radial = (pass == kFused || pass == kCount) && (args.flags & kFRadial);
    if (table && radial) return fail(LV_STATUS_INVALID_CONFIG, "radial counting launches are inline");
    if (!table) {
        int rc = assign_units(args, kHalf * unit_halves(mode, pt, st), nullptr);
        if (rc != LV_STATUS_SUCCESS) return rc;
    }
    if (args.total_units == 0) return LV_STATUS_SUCCESS;
    int rc = LV_STATUS_SUCCESS;
    // Unit launches, in pieces of at most kMaxGrid blocks (kRadialPiece for radial counting, the
    // records of one piece; LV_MAX_GRID_BLOCKS lowers the cap, so tests can split small launches).
    // A counting launch folds its counts in its last blocks; a radial one runs fold_kernel after
    // every piece.
    args.xcds = device_xcds();
    // b / X == (b * recip) >> 40 for b < 2^23 = kMaxGrid and X <= 64: recip exceeds 2^40 / X by at
    // most 1, so the product exceeds b * 2^40 / X by less than b < 2^23, i.e. by < 2^-17 after the
    // shift, while the fraction of b / X is at most 1 - 1/X <= 1 - 2^-6.
    static_assert(kMaxGrid <= (1u << 23), "the reciprocal is exact for grids up to 2^23 blocks");
    static_assert(kRadialPiece <= kMaxGrid, "a radial piece is one unit launch");
    args.xcd_recip = ((uint64_t)1 << 40) / args.xcds + 1;
    uint32_t max_grid = radial ? kRadialPiece : kMaxGrid;
    if (const char *e = std::getenv("LV_MAX_GRID_BLOCKS")) {
        long v = std::atol(e);
        if (v > 0 && (uint32_t)v < max_grid) max_grid = (uint32_t)v;
    }
    KernelFn fold = radial ? pick_fold(mode, pass) : nullptr;
    for (uint32_t ub = 0; ub < args.total_units; ub += std::min<uint32_t>(max_grid, args.total_units - ub)) {
        const uint32_t grid = std::min<uint32_t>(max_grid, args.total_units - ub);
        args.unit_base = ub;
        args.piece_units = grid;
        args.xcd_q = grid / args.xcds;
        args.xcd_r = grid % args.xcds;
        rc = launch_one(fn, args, grid, kThreads, stream);
        if (rc != LV_STATUS_SUCCESS) return rc;
        if (radial) {
            uint32_t chunks = 0;
            for (int t = 0; t < args.ndesc; t++) {
                uint32_t lo, hi;
                piece_span(args, t, ub, ub + grid, lo, hi);
                chunks += (hi - lo + kFoldChunk - 1) / kFoldChunk;
            }
            rc = launch_one(fold, args, chunks, kThreads, stream);
            if (rc != LV_STATUS_SUCCESS) return rc;
        }
    }
    args.unit_base = 0;
    return LV_STATUS_SUCCESS;
}

}  // namespace lv

// ====================================================================== C ABI

extern "C" {

int lv_version(void) { return 200; }

// Layout (every region a multiple of 256 B):
//   [count words: kMaxDesc x kSlotWords words, 64 B apart][radial tickets: kMaxDesc u64, 512 B]
//     -- kZeroBytes that must be zero before a call; every launch leaves them zeroed again --
//   [radial running sums: kMaxDesc RadialSum][chunk records: kMaxChunks RadialSum]
//   [unit records: kRadialPiece x (2 doubles)][unit counts: kRadialPiece x u32]   = kFixedBytes
// and, when a call has more than kMaxDesc tensors (table launches):
//   [count words: kTableMax x kSlotWords words, 64 B apart] (zero, like the first region)
//   [descriptor table: kTableMax x Desc]
// Everything is reused by every launch of a call (stream-ordered).
static constexpr size_t kSlotBytes = (size_t)lv::kMaxDesc * lv::kSlotWords * lv::kSlotStride * sizeof(unsigned long long);
static constexpr size_t kTicketBytes = 512;
static constexpr size_t kZeroBytes = kSlotBytes + kTicketBytes;
static constexpr size_t kRunBytes = (size_t)lv::kMaxDesc * sizeof(lv::RadialSum);
static constexpr size_t kChunkBytes = (size_t)lv::kMaxChunks * sizeof(lv::RadialSum);
static constexpr size_t kUnitSqBytes = (size_t)lv::kRadialPiece * 2 * sizeof(double);
static constexpr size_t kUnitCntBytes = (size_t)lv::kRadialPiece * sizeof(uint32_t);
static constexpr size_t kFixedBytes = kZeroBytes + kRunBytes + kChunkBytes + kUnitSqBytes + kUnitCntBytes;
static constexpr size_t kTableSlotBytes =
    (size_t)lv::kTableMax * lv::kSlotWords * lv::kSlotStride * sizeof(unsigned long long);
static constexpr size_t kTableDescBytes = (size_t)lv::kTableMax * sizeof(lv::Desc);
static_assert(kSlotBytes % 256 == 0 && kRunBytes % 256 == 0 && kChunkBytes % 256 == 0, "region alignment");
static_assert(kFixedBytes % 256 == 0 && kTableSlotBytes % 256 == 0 && kTableDescBytes % 256 == 0, "region alignment");
static_assert(lv::kMaxDesc * sizeof(unsigned long long) <= kTicketBytes, "ticket region");
static_assert(sizeof(lv::RadialSum) == 32, "radial record layout");

size_t lv_workspace_bytes(int n_tensors) {
    // the launches of a call reuse per-launch regions; table launches need their own words
    return kFixedBytes + (n_tensors > lv::kMaxDesc ? kTableSlotBytes + kTableDescBytes : 0);
}

const char *lv_last_error(void) { return lv::g_err; }

int lv_step_multi(const lv_config *cfg, const lv_tensor *tensors, int count, void *workspace,
                  size_t workspace_bytes, void *stream_ptr) {
    using namespace lv;
    g_err[0] = 0;
    if (!cfg) return fail(LV_STATUS_NULL_POINTER, "config is NULL");
    if (count < 0) return fail(LV_STATUS_INVALID_CONFIG, "negative tensor count");
    if (count == 0) return LV_STATUS_SUCCESS;
    if (!tensors) return fail(LV_STATUS_NULL_POINTER, "tensor list is NULL");
    int rc = validate_config(cfg);
    if (rc != LV_STATUS_SUCCESS) return rc;
    const int bound = (cfg->bound && cfg->bound_ratio > 0.0f) ? cfg->bound_type : LV_BOUND_NONE;  // config.rs:368-375
    const bool dual = cfg->buffer == LV_BUFFER_DUAL || cfg->buffer == LV_BUFFER_T2;
    const bool cautious = cfg->cautious != 0;
    if (!workspace) return fail(LV_STATUS_NULL_POINTER, "workspace is NULL");
    if (workspace_bytes < lv_workspace_bytes(count))
        return fail(LV_STATUS_INVALID_CONFIG, "workspace too small: %zu < %zu", workspace_bytes, lv_workspace_bytes(count));
    if (((uintptr_t)workspace & 15u) != 0) return fail(LV_STATUS_INVALID_CONFIG, "workspace must be 16-byte aligned");

    std::vector<Item> items;
    items.reserve(count);
    for (int i = 0; i < count; i++) {
        const lv_tensor &T = tensors[i];
        if (T.numel == 0) continue;
        if (!T.param || !T.grad || !T.exp_avg || !T.scratch)
            return fail(LV_STATUS_NULL_POINTER, "tensor %d: null param/grad/exp_avg/scratch pointer", i);
        if (dual && !T.exp_avg_sq)
            return fail(LV_STATUS_NULL_POINTER, "tensor %d: Dual-buffer mode requires an initialized exp_avg_sq buffer", i);
        if (T.param_dtype < 0 || T.param_dtype > 2 || T.grad_dtype < 0 || T.grad_dtype > 2 || T.state_dtype < 0 ||
            T.state_dtype > 2)
            return fail(LV_STATUS_INVALID_CONFIG, "tensor %d: invalid dtype code", i);
        if (T.step == 0) return fail(LV_STATUS_INVALID_CONFIG, "tensor %d: step must be >= 1", i);
        if (T.numel > (uint64_t)0xFFFFFFFFull * kHalf)
            return fail(LV_STATUS_INVALID_CONFIG, "tensor %d: too many elements", i);
        // worker.rs:95-98 and worker.rs:153-156: an fp32 param aliasing its master has none.
        bool mp_present = T.master_param && !(T.param_dtype == LV_DTYPE_F32 && (void *)T.master_param == T.param);
        bool master = cfg->master_weights != 0 && mp_present;
        if (cfg->master_weights != 0 && !mp_present && T.param_dtype != LV_DTYPE_F32)
            return fail(LV_STATUS_NULL_POINTER, "tensor %d: Master weight mode requires an initialized master_param buffer", i);
        if (T.grad == T.param || T.grad == T.exp_avg)
            return fail(LV_STATUS_INVALID_CONFIG, "tensor %d: grad aliases mutable state", i);  // mod.rs:310-318
        if (T.n_inactive && !T.inactive) return fail(LV_STATUS_NULL_POINTER, "tensor %d: inactive ranges pointer is NULL", i);
        if (T.n_inactive > 0xFFFFFFFFull) return fail(LV_STATUS_INVALID_CONFIG, "tensor %d: too many inactive ranges", i);
        Item it;
        it.idx = i;
        it.pt = T.param_dtype;
        it.gt = T.grad_dtype;
        it.st = T.state_dtype == LV_DTYPE_F32 ? LV_DTYPE_F32 : LV_DTYPE_BF16;  // fp16 state -> bf16 bits (worker.rs:107-113)
        it.master = master;
        it.clampv = T.param_dtype == LV_DTYPE_F16 || T.state_dtype == LV_DTYPE_F16;
        it.step = T.step;
        if (!cautious && bound != LV_BOUND_RADIAL) it.pass = kSingle;
        else if (cfg->fused_single_pass && T.step > 1) it.pass = kFused;
        else it.pass = kCount;
        items.push_back(it);
    }
    if (items.empty()) return LV_STATUS_SUCCESS;

    // Launch classes: identical (pass, step, dtypes, master). Stable order keeps the caller's order.
    std::stable_sort(items.begin(), items.end(), [](const Item &x, const Item &y) {
        if (x.pass != y.pass) return x.pass < y.pass;
        if (x.step != y.step) return x.step < y.step;
        if (x.pt != y.pt) return x.pt < y.pt;
        if (x.gt != y.gt) return x.gt < y.gt;
        if (x.st != y.st) return x.st < y.st;
        if (x.clampv != y.clampv) return x.clampv < y.clampv;
        return x.master < y.master;
    });

    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    char *ws = static_cast<char *>(workspace);
    // Radial counting launches fold per tensor after each piece, which needs the inline table.
    const bool table_ok = bound != LV_BOUND_RADIAL;
    size_t begin = 0;
    while (begin < items.size()) {
        const Item &h = items[begin];
        size_t cls_end = begin + 1;
        while (cls_end < items.size()) {
            const Item &x = items[cls_end];
            if (x.pass != h.pass || x.step != h.step || x.pt != h.pt || x.gt != h.gt || x.st != h.st ||
                x.master != h.master || x.clampv != h.clampv)
                break;
            cls_end++;
        }
        // One launch (pair) per kMaxDesc tensors of the class, or per kTableMax tensors when more
        // than kMaxDesc remain and the class can use a table launch.
        while (begin < cls_end) {
            const size_t left = cls_end - begin;
            const bool table = table_ok && left > (size_t)kMaxDesc;
            const size_t end = begin + std::min(left, (size_t)(table ? kTableMax : kMaxDesc));
            Args args;
            std::memset(&args, 0, sizeof args);
            args.lr = cfg->lr;
            args.b1 = cfg->beta1;
            args.b2 = cfg->beta2;
            args.omb1 = 1.0f - cfg->beta1;
            args.omb2 = 1.0f - cfg->beta2;
            args.b1sq = cfg->beta1 * cfg->beta1;
            args.omb1sq = 1.0f - args.b1sq;
            args.eps = cfg->eps;
            args.lam = cfg->lam;
            args.lam1 = 0.5f * cfg->lam;
            args.neg_lr_wd = -(cfg->lr * cfg->weight_decay);
            args.ratio = cfg->bound_ratio;
            StepCoeffs sc = step_coeffs(h.step, cfg->beta1, cfg->beta2, cfg->eps, cfg->tau, cfg->lam);
            args.c1 = sc.c1;
            args.c2 = sc.c2;
            args.c_sigma = sc.c_sigma;
            args.ema = cfg->ema_decay;
            args.ema_c = 1.0f - cfg->ema_decay;
            args.clamp_min = cfg->cautious_clamp_min;
            args.seed_base = (uint32_t)((uint64_t)cfg->seed + h.step * 0x9E3779B9ull);
            uint32_t flags = 0;
            if (cautious) flags |= kFCautious;
            if (cfg->stochastic_rounding) flags |= kFSR;
            if (h.master) flags |= kFMaster;
            if (cfg->weight_decay != 0.0f) flags |= kFWeightDecay;
            if (h.clampv) flags |= kFClampV;
            if (bound == LV_BOUND_COORDINATE) flags |= kFCoordinate;
            if (bound == LV_BOUND_RADIAL) flags |= kFRadial;
            flags |= (uint32_t)h.gt << 8;
            args.flags = flags;
            args.ndesc = (int32_t)(end - begin);
            StagingLease lease;
            if (table) {
                rc = acquire_staging(lease);
                if (rc != LV_STATUS_SUCCESS) return rc;
            }
            Desc *staged = lease.table;
            for (size_t k = begin; k < end; k++) {
                const lv_tensor &T = tensors[items[k].idx];
                Desc &D = table ? staged[k - begin] : args.d[k - begin];
                D.p = T.param;
                D.g = T.grad;
                D.m = T.exp_avg;
                D.v = T.exp_avg_sq;
                D.mp = items[k].master ? T.master_param : nullptr;
                D.scratch = T.scratch;
                D.n = T.numel;
                D.unit_begin = 0;  // set per launch (the unit size depends on the launch shape)
                D.pidx = (uint32_t)T.param_index;
                D.ibase = (uint32_t)T.index_base;
                D.nskip = (uint32_t)T.n_inactive;
                D.skip = T.n_inactive ? T.inactive : nullptr;
            }
            args.slots = reinterpret_cast<unsigned long long *>(table ? ws + kFixedBytes : ws);
            args.tickets = reinterpret_cast<unsigned long long *>(ws + kSlotBytes);
            args.run = reinterpret_cast<RadialSum *>(ws + kZeroBytes);
            args.chunks = reinterpret_cast<RadialSum *>(ws + kZeroBytes + kRunBytes);
            args.unit_sq = reinterpret_cast<double *>(ws + kZeroBytes + kRunBytes + kChunkBytes);
            args.unit_cnt = reinterpret_cast<uint32_t *>(ws + kZeroBytes + kRunBytes + kChunkBytes + kUnitSqBytes);
            if (table) {
                args.dtab = reinterpret_cast<const Desc *>(ws + kFixedBytes + kTableSlotBytes);
                rc = stage_table(args, cfg->buffer, h.pt, h.st, staged, lease.ev, stream);
                release_staging(lease, rc == LV_STATUS_SUCCESS);
                if (rc != LV_STATUS_SUCCESS) return rc;
            }
            if (h.pass == kCount) {
                rc = launch(args, cfg->buffer, h.pt, h.st, kCount, stream, table);
                if (rc == LV_STATUS_SUCCESS) rc = launch(args, cfg->buffer, h.pt, h.st, kApply, stream, table);
            } else {
                rc = launch(args, cfg->buffer, h.pt, h.st, h.pass, stream, table);
            }
            if (rc != LV_STATUS_SUCCESS) return rc;
            begin = end;
        }
    }
    return LV_STATUS_SUCCESS;
}

int lv_step_f32(float *param, const float *grad, float *exp_avg, float *exp_avg_sq, float *master_param,
                float *scratch, size_t num_elements, float lr, float beta1, float beta2, float eps,
                float weight_decay, float tau, float lam, int buffer_mode, int cautious, int bound_mode,
                float bound_ratio, uint64_t step, uint32_t seed, void *stream) {
    using namespace lv;
    static std::mutex mu;
    static void *ws[64] = {nullptr};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(LV_STATUS_NO_DRIVER, "no HIP device");
    {
        std::lock_guard<std::mutex> lk(mu);
        if (!ws[dev]) {
            void *p = nullptr;
            if (hipMalloc(&p, lv_workspace_bytes(1)) != hipSuccess) return fail(LV_STATUS_EXECUTION_FAILED, "hipMalloc failed");
            if (hipMemset(p, 0, lv_workspace_bytes(1)) != hipSuccess) return fail(LV_STATUS_EXECUTION_FAILED, "hipMemset failed");
            ws[dev] = p;
        }
    }
    lv_config c;
    c.lr = lr;
    c.beta1 = beta1;
    c.beta2 = beta2;
    c.eps = eps;
    c.weight_decay = weight_decay;
    c.tau = tau;
    c.lam = lam;
    c.cautious_clamp_min = 0.5f;
    c.bound_ratio = bound_ratio;
    c.ema_decay = (buffer_mode == LV_BUFFER_TDCLM || buffer_mode == LV_BUFFER_T1) ? 0.95f : 0.80f;
    c.buffer = buffer_mode;
    c.cautious = cautious;
    c.stochastic_rounding = 1;
    c.bound = 1;
    c.bound_type = bound_mode;
    c.master_weights = master_param ? 2 : 0;
    c.fused_single_pass = 1;
    c.seed = seed;
    lv_tensor t;
    std::memset(&t, 0, sizeof t);
    t.param = param;
    t.grad = grad;
    t.exp_avg = exp_avg;
    t.exp_avg_sq = exp_avg_sq;
    t.master_param = master_param;
    t.scratch = scratch;
    t.numel = num_elements;
    t.step = step;
    t.param_index = 0;
    t.param_dtype = t.grad_dtype = t.state_dtype = LV_DTYPE_F32;
    int rc = lv_step_multi(&c, &t, 1, ws[dev], lv_workspace_bytes(1), stream);
    if (rc == LV_STATUS_EXECUTION_FAILED) {
        // a launch failed part-way: its count words may hold partial counts; start clean
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (hipStreamSynchronize(s) == hipSuccess) (void)hipMemset(ws[dev], 0, lv_workspace_bytes(1));
    }
    return rc;
}

}  // extern "C"
