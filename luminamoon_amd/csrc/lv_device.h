// Device side of the MI355X LuminaV step: constants, descriptor and argument layouts, the exact
// per-element arithmetic, the unit kernel, the radial fold kernel and the kernel pickers. Included
// by the per-mode kernel units (lv_kernels.hip, one object per buffer mode so that they compile in
// parallel) and, for the layouts alone, by the host side (luminav_hip.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "luminav_hip.h"
#include "lv_exact.h"

namespace lv {

// Address spaces of the kernels' memory accesses. Every stream, scratch and range pointer a kernel
// dereferences points to global memory (1), and a table launch's descriptor table is constant
// while the launch runs (4). Pointers read from that table carry no address space of their own,
// so without these casts the compiler accessed the streams with flat instructions, read the
// descriptor with vector loads and waited for them before the first stream load; with them it
// reads the descriptor in one batch of scalar loads and streams with global instructions (cfg2's
// 64-tensor table launch: 14.46 against 16.56 us per launch, in one process).
#define LV_GLOBAL __attribute__((address_space(1)))
#define LV_CONSTANT __attribute__((address_space(4)))

constexpr int kThreads = 256;
constexpr uint32_t kHalf = kThreads * 4;     // unit granule: 4 elements per thread; a unit is 1 or 2 of them

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
// Slot word: mask count << kTicketBits | blocks that reported. A tensor has < 2^32 units (of
// >= 256 elements; at most 2^40 elements), so a slot sees <= 2^26 blocks (27 bits) and counts
// <= 2^36 elements (37 bits). Fold word: count << 7 | slots completed (<= 64).
constexpr int kTicketBits = 27;
constexpr int kFoldBits = 7;
constexpr uint32_t kMaxGrid = 1u << 23;      // blocks per unit launch (grid x 256 threads < 2^32)
// Blocks per identity-mapped unit launch (one XCD: b / 1 is exact for any b). One-wave blocks:
// 2^25 x 64 threads < 2^32, so a cfg5 step (26.3M one-wave units) is one launch.
constexpr uint32_t kMaxGridIdentity = 1u << 25;
// Radial counting launches: units per piece (one workspace record each: 2 doubles + a u32 count),
// and unit records one fold block sums into a chunk record.
constexpr uint32_t kRadialPiece = 1u << 22;
constexpr uint32_t kFoldChunk = 4096;  // fold blocks per full piece: kRadialPiece / kFoldChunk
constexpr int kFoldBatch = 16;         // unit records a fold thread loads before adding them
constexpr uint32_t kMaxChunks = kRadialPiece / kFoldChunk + kMaxDesc;  // chunks of one piece
// A chunk's mask count (<= kFoldChunk units x 4096 elements) fits the u32 chunk sums; the
// sums over chunks run in u64.
static_assert((uint64_t)kFoldChunk * 4096u <= 0xFFFFFFFFull, "chunk counts fit 32 bits");

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

// Flag word of the specialised ("static") instantiation: the reference defaults (cautious in
// the counting passes, stochastic rounding, weight decay, coordinate bound, no master, grad
// dtype = param dtype, v clamp for fp16 params).
constexpr uint32_t static_flags(int PT, int PASS) {
    return (PASS != kSingle ? (uint32_t)kFCautious : 0u) | (uint32_t)kFSR | (uint32_t)kFWeightDecay |
           (uint32_t)kFCoordinate | (PT == LV_DTYPE_F16 ? (uint32_t)kFClampV : 0u) | ((uint32_t)PT << 8);
}

// Sub-units per work unit (each 1024 * unit_halves elements) of the kernel for this mode, dtypes,
// pass and flag word (the launch's word; the run-time-flag kernels have 1). A block of 2 issues
// the loads of both sub-units before it computes the first, so the second's memory latency hides
// behind the first's arithmetic. That pays where the step is VALU-bound and the kernel keeps full
// occupancy with the extra registers: T1 with 16-bit state and 16-bit params, reference-default
// flags (in one process, bf16-state cfg4 1.653 -> 1.612 ms, fp16 cfg4 1.996 -> 1.904 ms). With
// 2 sub-units the T2 and TD-CLM 16-bit kernels and T1's other flag words need more registers than
// 8 waves per SIMD leave, and spill.
constexpr int unit_subs(int mode, int pt, int st, int pass, uint32_t flags) {
    return (mode == LV_BUFFER_T1 && st != LV_DTYPE_F32 && pt != LV_DTYPE_F32 && flags == static_flags(pt, pass)) ? 2 : 1;
}

// Blocks per CU a unit kernel must fit (its launch bounds). Without a bound the compiler takes the
// registers for a second sub-unit's loads out of occupancy (102 SGPRs: 7 waves per SIMD, where
// the bound keeps 8 and 78 SGPRs): 1.635 against 1.612 ms for bf16-state cfg4.
constexpr int unit_min_blocks(int mode, int pt, int st, int pass, uint32_t flags) {
    return unit_subs(mode, pt, st, pass, flags) > 1 ? 8 : 1;
}

// Threads per block of the unit kernel for this mode, dtypes, pass, flag word (the launch's word;
// the run-time-flag kernels have 256) and launch kind. Two steady inline steps with f32 state and
// the reference defaults run one-wave blocks (units of 256 elements), which launch() maps block b
// to unit b. In one process on the same buffers, against 256-thread blocks:
// - CLM in f32 (cfg3's kernel): 0.938-0.966x (cfg3, and a 1e9-element bucket);
// - T2 with bf16 params (the headline's kernel): 0.966x at 1e9 elements, 0.959x at 3.5e9, and
//   0.992-1.005x at cfg5's 6.7e9 (five processes).
// The other kernels keep 256: T1 with f32 state ran 1.040-1.046x with one-wave blocks (cfg4),
// TD-CLM's table launch of 64 tensors (cfg2) 1.03x (its inline buckets 0.980-0.986x).
constexpr int unit_threads(int mode, int pt, int st, int pass, uint32_t flags, bool table) {
    const bool one_wave = (mode == LV_BUFFER_DUAL && pt == LV_DTYPE_F32) || (mode == LV_BUFFER_T2 && pt == LV_DTYPE_BF16);
    return (!table && one_wave && st == LV_DTYPE_F32 && pass == kFused && flags == static_flags(pt, pass)) ? 64 : kThreads;
}

// Elements per work unit of a unit launch.
constexpr uint32_t unit_elems(int mode, int pt, int st, int pass, uint32_t flags, bool table) {
    return 4u * (uint32_t)unit_threads(mode, pt, st, pass, flags, table) * (uint32_t)unit_halves(mode, pt, st) *
           (uint32_t)unit_subs(mode, pt, st, pass, flags);
}
constexpr uint32_t kMaxUnitElems = 4 * kHalf;
constexpr uint32_t kMinUnitElems = 4 * 64;  // one-wave blocks, one group of 4 per lane

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
    uint32_t nskip : 24;  // inactive [begin, end) ranges in `skip` (sorted, disjoint)
    // vec: every stream is aligned at element `head` (< 64; to a 128-byte line where the views
    // allow it, else to 16 bytes), so the tensor's work units start there and whole units take
    // the vector path; the `head` elements before it are taken one per thread by the block of the
    // tensor's last unit. Set by the host from the pointers.
    uint32_t head : 6;
    uint32_t vec : 1;
    uint32_t : 1;
    const uint64_t *skip;
};

// A tensor of a table launch, in device memory: its descriptor, the end of its unit range and the
// first of its count slots (64-byte slot index into Args::slots; the tensor has
// table_count_slots(units) slots and one fold slot after them).
struct TDesc {
    Desc d;
    uint32_t unit_end;
    uint32_t slot_base;
};

// Count slots of a tensor of `units` work units: the smallest power of two that keeps every slot at
// <= 64 blocks, at most kSlots (a tensor of <= 64 units has one, whose last block finalises it
// without the fold word). Inline launches reserve kSlotWords slot words per tensor; table
// launches lay the tensors' slots out back to back.
__host__ __device__ inline uint32_t table_count_slots(uint32_t units) {
    const uint32_t c = (units + 63u) >> 6;
    if (c <= 1u) return 1u;
    if (c >= kSlots) return kSlots;
    return 1u << (32 - __builtin_clz(c - 1u));
}

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
    uint32_t group;        // table launches: tensors per head (ubegin[h] is tensor h * group's first unit)
    uint32_t nheads;       // table launches: entries of ubegin
    uint32_t bound_floor;  // 1 when bound_ratio >= 2^-40: the coordinate bound's b * b is a normal number
    uint32_t ranges;       // kRange* facts about the hyper-parameters (the host tests them per launch)
    uint64_t xcd_recip;  // unit launches: floor(2^40 / xcds) + 1, so b / xcds == (b * xcd_recip) >> 40
    unsigned long long *slots;    // counting launches: count slots (inline: kSlotWords per tensor, in order)
    unsigned long long *tickets;  // radial fold: finished chunks of the piece, per tensor (left zero)
    RadialSum *run;               // radial fold: per tensor, the sums of the pieces folded so far
    RadialSum *chunks;            // radial fold: one record per chunk of the piece
    double *unit_sq;              // radial: per unit of the piece, (sum u_eff^2, sum p^2)
    uint32_t *unit_cnt;           // radial: per unit of the piece, the mask count
    const TDesc *dtab;            // table launches: the tensor table in device memory
    const lv_step_record *step_rec;  // graph launches: this step's coefficients (else c1..seed_base above)
    union {
        Desc d[kMaxDesc];  // inline launches: the tensor table
        uint32_t ubegin[kMaxDesc * sizeof(Desc) / sizeof(uint32_t)];  // table launches: first unit per head
    };
};

// Table launches: any number of tensors in device memory; the kernel arguments hold the first unit
// of every group-th tensor (the heads, where the inline table would be), so a block finds its
// tensor by a binary search of the heads and, above kTableHeads tensors, of its head's group.
constexpr int kTableHeads = kMaxDesc * (int)(sizeof(Desc) / sizeof(uint32_t));  // 960

static_assert(sizeof(Desc) == 80, "descriptor layout");
static_assert(sizeof(TDesc) == 88, "table descriptor layout");
static_assert(sizeof(Args) <= 4096, "kernel arguments must fit in 4 KiB");

// Args::ranges. kRangeM: |beta1| and |1 - beta1| are at most 2^64, so m' = beta1 m + (1 - beta1) g
// stays below 2^126 whenever |g| <= 1e18 and |g - m| <= 1e18. kRangeP: bound_floor, and
// |lr * weight_decay| is at most 2^32, so a param the coordinate bound's fast quotient took
// (|p| <= 2^52.5, |step| <= 2^11.5: div_bound) decays and steps to below 2^86.
enum : uint32_t { kRangeM = 1u, kRangeP = 2u };

// ------------------------------------------------------------------ per-step coefficients

// compiler-builtins' __powidf2 (the lowering of Rust f64::powi): repeated squaring.
__host__ __device__ inline double powi_rs(double a, int32_t b) {
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

// math.rs:27-81, on the host for every launch and on the device for graph launches (the step
// record kernel): IEEE f64 products, quotient and square root (correctly rounded on both sides),
// so both give the same bits. Above 2^31 - 1 steps the reference switches to f64::powf, here the
// platform's pow (not pinned against the reference's).
__host__ __device__ inline StepCoeffs step_coeffs(uint64_t step, float beta1, float beta2, float eps, float tau,
                                                  float lam) {
    uint64_t safe = step > 1 ? step : 1;
    double b1 = (double)beta1, b2 = (double)beta2;
    double bc1 = safe < 2147483647ull ? 1.0 - powi_rs(b1, (int32_t)(safe + 1)) : 1.0 - pow(b1, (double)(safe + 1));
    double bc2_raw = safe <= 2147483647ull ? 1.0 - powi_rs(b2, (int32_t)safe) : 1.0 - pow(b2, (double)safe);
    double bc2 = fmax(bc2_raw, 1.0e-15);
    StepCoeffs c;
    c.c1 = (float)((bc1 * (double)tau) / sqrt(bc2));
    c.c2 = (float)((double)eps * bc1 * (double)tau);
    float bc2f = (float)bc2;
    c.c_sigma = (0.5f * lam) / sqrtf(fmaxf(bc2f, 1.0e-15f));
    return c;
}

// Seed base of a step: low 32 bits of seed + step * 0x9E3779B9 (prng.rs:4-13).
__host__ __device__ inline uint32_t step_seed_base(uint32_t seed, uint64_t step) {
    return (uint32_t)((uint64_t)seed + step * 0x9E3779B9ull);
}

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

// prng.rs:137-160 (sr_bf16_checked in lv_exact.h) with the noise prng(z0) & 0xFFFF. Returns an
// f32 whose HIGH half holds the bf16 bits (the low half is not zero: store it, do not compute
// with it).
__device__ __forceinline__ float sr_bf16(float v, uint32_t z0) {
    return sr_bf16_checked(v, xor_fold16((uint32_t)prng_mixed(z0)));
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

// prng.rs:98-130 as an f32 whose round-toward-zero fp16 conversion (pack_f16_rtz) is the
// reference's result. On sr_f16_domain (lv_exact.h: +-0 and fp16 normal results below 65504)
// that is v's bits plus the 13 noise bits prng(z0) & 0x1FFF (sr_f16_add); when any active lane of
// the wave is outside the domain, the wave takes the integer recipe below (the one the reference
// states), whose result is itself an fp16 value.
__device__ __forceinline__ float sr_fp16_val(float v, uint32_t z0) {
    const uint32_t z = (uint32_t)prng_mixed(z0);
    // the domain's result, replaced below in the rare waves that need the recipe (computing it
    // first lets both paths leave the result in one register)
    const float fast = sr_f16_add(v, xor_fold16(z) & 0x1FFFu);
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(!sr_f16_domain(v)) == 0, 1)) return fast;
    int32_t p = (int32_t)f_bits(v);
    int32_t a = p & 0x7FFFFFFF;
    int32_t ex = (a >> 23) & 0xFF;
    int32_t sub = 113 - ex;
    sub = sub > 0 ? sub : 0;
    sub = sub < 11 ? sub : 11;
    int32_t mask = (int32_t)((1u << (13 + sub)) - 1u);
    int32_t noise = ((int32_t)z ^ ((int32_t)z >> 16)) & mask;  // prng(z0)
    int32_t added = ex < 103 ? 0 : (int32_t)(((uint32_t)a + (uint32_t)noise) & (uint32_t)(~mask));
    int32_t r = added > 0x477FE000 ? 0x477FE000 : added;
    // The reference converts sign | r to fp16 and back (prng.rs:129). sign | r is already an fp16
    // value, so that round trip is the identity and pack_f16_rtz converts it exactly. r is one of:
    // - 0, or 65504;
    // - the sign bit alone (-0.0), when a NaN's magnitude plus the noise wraps past 2^31;
    // - a value with its (13 + sub) low bits clear. For ex >= 113 that leaves 10 fraction bits
    //   below 65504 (an fp16 normal). For 103 <= ex <= 112 it leaves a multiple of 2^-24 below
    //   2^-13 (fp16 subnormals and the lowest normal binade).
    return bits_f((uint32_t)((p & (int32_t)0x80000000u) | r));
}

// The same with the fp16 bits in the low half (high half zero), for element-wise stores.
__device__ __forceinline__ float sr_fp16(float v, uint32_t z0) { return bits_f(pack_f16_rtz(sr_fp16_val(v, z0), 0.0f)); }

// prng.rs:29-67: fp16 bits in the low half (high half zero), like sr_fp16.
__device__ __forceinline__ float rne_fp16(float v) { return bits_f(f32_to_f16_rne(v)); }

// The same as an fp16 value in an f32 (exact for pack_f16_rtz), like sr_fp16_val.
__device__ __forceinline__ float rne_fp16_val(float v) { return f16_to_f32(f32_to_f16_rne(v)); }

// prng.rs:180-195; dtype is a compile-time constant at every call site. z0 is the element's
// hash input for the buffer's seed (offset + seed + kPrngAdd). The result is only stored:
// bf16 results hold the bf16 bits in the high half, fp16 results the fp16 bits in the low half.
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

// Wave-uniform fast paths. Each exact helper below has a cheap common case (an input in the range
// where the helper is the identity, or needs no rescaling); when every active lane of the wave is
// in it, one compare per element and a scalar branch replace the general sequence. The general
// sequence still runs, for the whole wave, whenever any lane needs it, so results are unchanged.
__device__ __forceinline__ bool wave_all(bool c) { return __builtin_amdgcn_ballot_w64(!c) == 0; }

// How an element's cautious mask bit is counted: not at all (SINGLE pass), into the lane's own
// count, or into the wave's count (every lane of the wave present; cnt is the same in every lane).
enum : int { kTallyNone = 0, kTallyLane = 1, kTallyWave = 2 };

// Adds the mask bit where it is computed. For the wave count the empty asm holds the ballot's
// popcount in an SGPR at this point: otherwise the compiler sinks every element's ballot past the
// wave-uniform branches that follow and carries each lane mask across them through a VGPR (a
// v_cndmask and a v_cmp per element).
template <int TALLY>
__device__ __forceinline__ void tally(uint32_t &cnt, bool active) {
    if constexpr (TALLY == kTallyWave) {
        uint32_t c = (uint32_t)__popcll(__builtin_amdgcn_ballot_w64(active));
        asm volatile("" : "+s"(c));
        cnt += c;
    } else if constexpr (TALLY == kTallyLane) {
        cnt += active ? 1u : 0u;
    }
}

// math.rs:4-11. |g| < 1e38 is false for NaN and +-inf, so one compare also covers is_finite;
// on that path g is not NaN and med3 is exactly the clamp. |g| <= 1e18 (false for NaN) leaves g
// unchanged.
__device__ __forceinline__ float sanitize(float g) {
    if (__builtin_expect(wave_all(fabsf(g) <= 1.0e18f), 1)) return g;
    return fabsf(g) < 1.0e38f ? __builtin_amdgcn_fmed3f(g, -1.0e18f, 1.0e18f) : 0.0f;
}

// math.rs:13-16 (clamp_defect): NaN passes through like Rust's f32::clamp; |d| <= 1e18 is the
// identity.
__device__ __forceinline__ float clamp_defect(float d) {
    if (__builtin_expect(wave_all(fabsf(d) <= 1.0e18f), 1)) return d;
    return __builtin_isnan(d) ? d : __builtin_amdgcn_fmed3f(d, -1.0e18f, 1.0e18f);
}

// The same, telling whether every lane of the wave took the identity (|d| <= 1e18, no NaN).
__device__ __forceinline__ float clamp_defect(float d, bool &identity) {
    identity = wave_all(fabsf(d) <= 1.0e18f);
    if (__builtin_expect(identity, 1)) return d;
    return __builtin_isnan(d) ? d : __builtin_amdgcn_fmed3f(d, -1.0e18f, 1.0e18f);
}

// fma(a, |x|, c) as ONE v_fma_f32 with the abs source modifier (a wave-uniform). Written as
// __builtin_fmaf(a, fabsf(x), c) the compiler materialises |x| with a v_and_b32 and uses the
// 2-operand v_fmac_f32: one more VALU instruction for the same result.
__device__ __forceinline__ float fma_abs(float a, float x, float c) {
    float r;
    asm("v_fma_f32 %0, %1, |%2|, %3" : "=v"(r) : "s"(a), "v"(x), "v"(c));
    return r;
}

// Correctly rounded sqrt (sqrt_rn in lv_exact.h) with its small-input rescaling skipped when no
// lane of the wave needs it (x >= 2^-96, +-0, +inf and NaN need none).
__device__ __forceinline__ float sqrt_cr(float x) {
    if (__builtin_expect(wave_all(!(x < 0x1p-96f) || x == 0.0f), 1)) return sqrt_rn_normal(x);
    return sqrt_rn(x);
}

// Three constants of tanh_pade: the clamp bound and the leading coefficients of its numerator and
// denominator. An fma or median instruction takes at most one literal or SGPR operand on gfx950,
// so each of these needs a VGPR; the vector path passes copies made once per unit (in_vgpr), which
// the compiler would otherwise re-create with a v_mov at every call.
struct PadeK {
    float hi, p0, q0;
};
constexpr PadeK kPade = {7.9988117f, -2.7607684e-16f, 1.1982584e-6f};

// A wave-uniform value copied to a VGPR once. A VOP3 instruction reads at most one SGPR on gfx950,
// so an fma with two uniform operands needs one of them in a VGPR; the asm copy cannot be
// re-created, where the compiler would otherwise re-create it (a v_mov) for every element.
__device__ __forceinline__ float in_vgpr(float x) {
    float r;
    asm("v_mov_b32 %0, %1" : "=v"(r) : "s"(x));
    return r;
}

// math.rs:83-118 -- [13/6] Pade tanh, Horner with fma. c holds kPade's values.
__device__ __forceinline__ float tanh_pade(float x_in, const PadeK &c = kPade) {
    if (__builtin_isnan(x_in)) return bits_f(0x7FC00000u);  // Rust f32::NAN
    // x_in is not NaN here, so the median of three is exactly the clamp
    float x = __builtin_amdgcn_fmed3f(x_in, -7.9988117f, c.hi);
    float x2 = x * x;
    float p = __builtin_fmaf(c.p0, x2, 2.000188e-13f);
    float q = __builtin_fmaf(c.q0, x2, 1.1853471e-4f);
    p = __builtin_fmaf(p, x2, -8.604672e-11f);
    q = __builtin_fmaf(q, x2, 2.2684346e-3f);
    p = __builtin_fmaf(p, x2, 5.122297e-8f);
    q = __builtin_fmaf(q, x2, 4.8935246e-3f);
    p = __builtin_fmaf(p, x2, 1.4857224e-5f);
    p = __builtin_fmaf(p, x2, 6.3726193e-4f);
    p = __builtin_fmaf(p, x2, 4.8935246e-3f);
    return (x * p) / q;
}

// IEEE f32 division in five instructions: v_rcp_f32, one Newton step on the reciprocal (r1), the
// product q0 = n * r1 and one correction by its exact residual, q0 + (n - d * q0) * r1 (Markstein's
// final step). The compiler's correctly rounded quotient is 11 instructions, about 15.5 integer
// adds of issue time on gfx950 (v_div_scale on both operands, v_rcp_f32, the refinement,
// v_div_fmas and v_div_fixup; the scale, fmas and fixup steps issue at about 1.6 each, v_rcp at
// 3). This equals n / d bit for bit on every pair of significands: n and d in [1, 2), all 2^46
// pairs, checked on the GPU against the compiler's division, with v_rcp_f32's result checked to
// scale exactly with d's exponent over [-125, 125] (tests/gpu_checks/exact_check.hip). Other
// exponents scale every step when |n| >= 2^-100, 2^-125 <= |n / d| (no overflow) and
// 2^-125 <= d <= 2^125: r1, q0 and the quotient are then normal, and the residual n - d * q0, a
// multiple of 2^-147, is exact wherever it is subnormal, so every rounding scales with the
// operands. Callers test their own sufficient condition, wave-uniformly, and otherwise divide as
// usual.
__device__ __forceinline__ float div_unscaled(float n, float d) {
    const float r0 = __builtin_amdgcn_rcpf(d);
    const float e0 = __builtin_fmaf(-d, r0, 1.0f);
    const float r1 = __builtin_fmaf(e0, r0, r0);
    const float q0 = n * r1;
    const float e1 = __builtin_fmaf(-d, q0, n);
    return __builtin_fmaf(e1, r1, q0);
}

// clm / env of T1, T2 and TD-CLM, where |clm| <= env up to rounding (env adds the
// magnitudes of clm's two terms and non-negative ones): with |clm| >= 2^-100 and env <= 2^25,
// env >= 2^-101 is normal, the quotient is at least 2^-125 and the exponents are at most one
// apart, so div_unscaled is exact. NaNs and infinities fail one of the two compares.
__device__ __forceinline__ float div_envelope(float n, float d) {
    const uint64_t small = __builtin_amdgcn_ballot_w64(!(__builtin_fabsf(n) >= 0x1p-100f));
    const uint64_t large = __builtin_amdgcn_ballot_w64(!(d <= 0x1p25f));
    if (__builtin_expect((small | large) == 0, 1)) return div_unscaled(n, d);
    return n / d;
}

// (bb * s) / (s * s + bb) of the rational bounds, bb = b (b + |s|) > 0. Its magnitude is at most
// sqrt(bb) / 2 <= sqrt(d) / 2 (AM-GM), so |n| >= 2^-100 puts d above 2^-66, and with d <= 2^25
// the quotient lies in [2^-125, 2^12.5]: div_unscaled is exact. A NaN or infinite d fails the
// test. `zero_lane`: this lane's step is a masked cautious step, an exact +-0 (so n is one and
// d = bb, a normal number below 2^25 when the caller knows a floor on b); div_unscaled then
// gives a zero of either sign, and that sign is lost anyway where the caller also knows weight
// decay is on: the decayed param p + (-lr wd) p is never -0, and p_dec - (+-0) is the same for
// every other p_dec.
// `zero_lanes` is a wave mask (the ballot of the lanes whose step is such a zero, or 0), and the
// test's masks are combined on the scalar unit: a ballot of a combined condition would go through
// a VGPR (a select and a compare per element).
// `fast` tells the caller which way the wave went: on the fast side every lane has d <= 2^25.
__device__ __forceinline__ float div_bound(float n, float d, uint64_t zero_lanes, bool &fast) {
    const uint64_t small = __builtin_amdgcn_ballot_w64(!(__builtin_fabsf(n) >= 0x1p-100f));
    const uint64_t large = __builtin_amdgcn_ballot_w64(!(d <= 0x1p25f));
    fast = ((small & ~zero_lanes) | large) == 0;
    if (__builtin_expect(fast, 1)) return div_unscaled(n, d);
    return n / d;
}

// math.rs:162-186. TRI: zero_lanes as for div_bound, with the floor b >= ratio * 0.01 >= 2^-46.7
// (the caller's bound_floor) giving bb >= 2^-93. `fast`: the wave took div_bound's fast side,
// where d = step^2 + bb <= 2^25 bounds b^2 <= bb, so |p_init| <= 2^12.5 / ratio, and the result,
// at most sqrt(bb) / 2, is at most 2^11.5 (false when FAST is off).
template <bool TRI, bool FAST = false>
__device__ __forceinline__ float coordinate_bound(float step, float p_init, float ratio, const PadeK &c, uint64_t zero_lanes,
                                                  bool &fast) {
    fast = false;
    if constexpr (TRI) {
        float b = ratio * (fabsf(p_init) + 1.0e-2f);
        float bb = b * (b + fabsf(step));
        if constexpr (FAST) return div_bound(bb * step, __builtin_fmaf(step, step, bb), zero_lanes, fast);
        return (bb * step) / __builtin_fmaf(step, step, bb);
    } else {
        // p^2 + 1e-4 is at least 1e-4 (or NaN or +inf), where the root needs no rescaling
        float b = ratio * sqrt_rn_normal(__builtin_fmaf(p_init, p_init, 1.0e-4f));
        return b * tanh_pade(step / b, c);
    }
}

// TRI: zero_lanes as for div_bound; here b >= 1.5e-4 always (f32::max returns 1.5e-4 for a NaN
// p too), so bb >= 2.25e-8.
template <bool TRI, bool FAST = false>
__device__ __forceinline__ float fp16_safety_bound(float step, float p_init, const PadeK &c = kPade,
                                                   uint64_t zero_lanes = 0) {
    float b = __builtin_fmaxf(fabsf(p_init) * 0.01f, 1.5e-4f);
    if constexpr (TRI) {
        float bb = b * (b + fabsf(step));
        bool fast;
        if constexpr (FAST) return div_bound(bb * step, __builtin_fmaf(step, step, bb), zero_lanes, fast);
        return (bb * step) / __builtin_fmaf(step, step, bb);
    } else {
        return b * tanh_pade(step / b, c);
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

// Uniform constants an element's update reads from VGPRs: a.eps and the tanh constants (kPade).
// The vector path copies them to VGPRs once per unit (lane_consts); the per-element path uses
// them as they are.
struct LaneK {
    float eps;
    PadeK pade;
};

// What compute_u<FAST> found out about the wave (wave-uniform bits):
// kKnownM: every lane's defect |g - m| is at most 1e18 (clamp_defect was the identity), so with
//   |g| <= 1e18 (sanitize) |m| <= 2e18; with Args::ranges' kRangeM, m' is then below 2^126.
// kKnownV (T2): every lane's v' lies in [2^-96, the largest finite bf16]: no lane's root needs the
//   small-input rescaling or the clamp at 0, and no lane's bf16 rounding of v' needs the
//   saturation or NaN handling (sr_bf16_checked).
enum : uint32_t { kKnownM = 1u, kKnownV = 2u };

// u, m_new, v_new for one element.
// CLM: dual.rs:63-74.  T2: dual.rs:492-506.  TD-CLM / T1: tdclm.rs:102-109.
// FAST: the triangle envelope's quotient through div_envelope (kernels whose time is their VALU
// work: 16-bit state or fp16 params; the f32-state kernels stream at the HBM's rate and measured
// level or 1.3% slower with the guard's branches), and `known` (kKnown*) for T1 and T2. T2's root
// of v' takes one range test for both of kKnownV's facts (a subtraction and one unsigned compare
// of the bits: below 2^-96, negative, NaN and above the largest bf16 all fall outside) instead of
// the clamp at 0 and the root's own two compares.
template <int MODE, bool FAST>
__device__ __forceinline__ float compute_u(const Args &a, const StepCoeffs &k, const LaneK &lk, bool clamp_v, float g,
                                           float m, float v, float &m_new, float &v_new, uint32_t &known) {
    known = 0;
    m_new = __builtin_fmaf(a.b1, m, a.omb1 * g);
    if constexpr (MODE == LV_BUFFER_DUAL) {
        float clm = __builtin_fmaf(a.b1, m_new, a.omb1 * g);
        float diff = clamp_defect(g - m_new);
        v_new = __builtin_fmaf(a.b2, v, a.omb2 * (diff * diff));
        if (clamp_v) v_new = __builtin_fminf(v_new, 65000.0f);
        float sigma = __builtin_fmaf(sqrt_cr(__builtin_fmaxf(v_new, 0.0f)), k.c1, k.c2);
        return tanh_pade(clm / __builtin_fmaxf(sigma, 1.0e-12f), lk.pade);
    } else if constexpr (MODE == LV_BUFFER_T2) {
        float clm = __builtin_fmaf(a.b1sq, m, a.omb1sq * g);
        if constexpr (FAST) {
            bool defect_ok;
            const float diff = clamp_defect(g - m, defect_ok);
            v_new = __builtin_fmaf(a.b2, v, a.omb2 * (diff * diff));
            if (clamp_v) v_new = __builtin_fminf(v_new, 65000.0f);
            const float env0 = __builtin_fmaf(a.b1sq, fabsf(m), lk.eps);
            const float env1 = __builtin_fmaf(a.omb1sq, fabsf(g), env0);
            const float env2 = fma_abs(a.lam1, diff, env1);
            const bool v_ok = wave_all(f_bits(v_new) - 0x0F800000u <= kBf16MaxBits - 0x0F800000u);
            float root;
            if (__builtin_expect(v_ok, 1)) root = sqrt_rn_positive(v_new);  // v_new in [2^-96, 0x7F7F0000]
            else root = sqrt_cr(__builtin_fmaxf(v_new, 0.0f));
            known = (defect_ok ? kKnownM : 0u) | (v_ok ? kKnownV : 0u);
            return div_envelope(clm, __builtin_fmaf(k.c_sigma, root, env2));
        }
        float diff = clamp_defect(g - m);
        v_new = __builtin_fmaf(a.b2, v, a.omb2 * (diff * diff));
        if (clamp_v) v_new = __builtin_fminf(v_new, 65000.0f);
        float env0 = __builtin_fmaf(a.b1sq, fabsf(m), lk.eps);
        float env1 = __builtin_fmaf(a.omb1sq, fabsf(g), env0);
        float env2 = __builtin_fmaf(a.lam1, fabsf(diff), env1);
        float env = __builtin_fmaf(k.c_sigma, sqrt_cr(__builtin_fmaxf(v_new, 0.0f)), env2);
        return clm / env;
    } else {
        float clm = __builtin_fmaf(a.b1sq, m, a.omb1sq * g);
        v_new = 0.0f;
        if constexpr (FAST && MODE == LV_BUFFER_T1) {
            bool defect_ok;
            const float diff = clamp_defect(g - m, defect_ok);
            const float env0 = __builtin_fmaf(a.b1sq, fabsf(m), lk.eps);
            const float env1 = __builtin_fmaf(a.omb1sq, fabsf(g), env0);
            known = defect_ok ? kKnownM : 0u;
            return div_envelope(clm, fma_abs(a.lam, diff, env1));
        }
        float diff = clamp_defect(g - m);
        float env0 = __builtin_fmaf(a.b1sq, fabsf(m), lk.eps);
        float env1 = __builtin_fmaf(a.omb1sq, fabsf(g), env0);
        float env = __builtin_fmaf(a.lam, fabsf(diff), env1);
        return FAST ? div_envelope(clm, env) : clm / env;
    }
}

template <int MODE, bool FAST = false>
__device__ __forceinline__ float compute_u(const Args &a, const StepCoeffs &k, const LaneK &lk, bool clamp_v, float g,
                                           float m, float v, float &m_new, float &v_new) {
    uint32_t known;
    return compute_u<MODE, FAST>(a, k, lk, clamp_v, g, m, v, m_new, v_new, known);
}

// ------------------------------------------------------------------ loads / stores

template <int DT>
__device__ __forceinline__ float load1(const void *base, uint64_t i) {
    if constexpr (DT == LV_DTYPE_F32) {
        return ((const LV_GLOBAL float *)base)[i];
    } else if constexpr (DT == LV_DTYPE_BF16) {
        return bits_f((uint32_t)((const LV_GLOBAL uint16_t *)base)[i] << 16);
    } else {
        return f16_to_f32(((const LV_GLOBAL uint16_t *)base)[i]);
    }
}

template <int DT>
__device__ __forceinline__ void store1(void *base, uint64_t i, float x) {
    if constexpr (DT == LV_DTYPE_F32) {
        ((LV_GLOBAL float *)base)[i] = x;
    } else if constexpr (DT == LV_DTYPE_BF16) {
        ((LV_GLOBAL uint16_t *)base)[i] = (uint16_t)(f_bits(x) >> 16);
    } else {
        ((LV_GLOBAL uint16_t *)base)[i] = (uint16_t)f_bits(x);  // fp16 bits in the low half
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
// Layout of a work unit of 1024 * H elements. With H = 1 (f32 state) thread t owns [4t, 4t + 4):
// every wave-wide f32 access is one 16-byte load or store per lane over 1 KiB. With H = 2
// (16-bit state) thread t owns two groups of 4, at 4t and at 4t + HS (lane_split):
// - HS = 4, when every stream is 16-bit: the 8 consecutive elements [8t, 8t + 8), so a 16-bit
//   stream moves them in ONE 16-byte access per lane (1 KiB per wave instruction);
// - HS = 1024, when an f32 stream (a master copy, f32 grads) comes with the 16-bit ones: each
//   group is contiguous across the wave, so the f32 stream moves 1 KiB per wave instruction
//   (two adjacent 16-byte accesses per lane would stride 32 B and cost ~6% of the semi-master
//   bf16-state step) and a 16-bit stream 512 B.
// 32-bit types use `a` (the first group) and `b` (the second); 16-bit types pack all eight into
// `a` (.x = elements 0-1, ..., .w = 6-7).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct Raw8 {
    u32x4 a, b;
};

// H (1 or 2) is the number of 1024-element halves in the unit: a thread moves 4 * H elements, in
// groups of 4 at h0 and (H = 2) h0 + HS.
template <int DT, int H, uint32_t HS = 4>
__device__ __forceinline__ Raw8 load_raw(const void *base, uint64_t h0) {
    Raw8 r;
    if constexpr (DT == LV_DTYPE_F32) {
        const LV_GLOBAL float *f = (const LV_GLOBAL float *)base;
        r.a = __builtin_nontemporal_load((const LV_GLOBAL u32x4 *)(f + h0));
        if constexpr (H == 2) r.b = __builtin_nontemporal_load((const LV_GLOBAL u32x4 *)(f + h0 + HS));
        else r.b = u32x4{0, 0, 0, 0};
    } else {
        const LV_GLOBAL uint16_t *h = (const LV_GLOBAL uint16_t *)base;
        if constexpr (H == 2 && HS == 4) {
            r.a = __builtin_nontemporal_load((const LV_GLOBAL u32x4 *)(h + h0));
        } else {
            const u32x2 x = __builtin_nontemporal_load((const LV_GLOBAL u32x2 *)(h + h0));
            if constexpr (H == 2) {
                const u32x2 y = __builtin_nontemporal_load((const LV_GLOBAL u32x2 *)(h + h0 + HS));
                r.a = u32x4{x.x, x.y, y.x, y.y};
            } else {
                r.a = u32x4{x.x, x.y, 0, 0};
            }
        }
        r.b = u32x4{0, 0, 0, 0};
    }
    return r;
}

template <int H, uint32_t HS = 4>
__device__ __forceinline__ Raw8 load_raw_dyn(int dt, const void *base, uint64_t h0) {
    if (dt == LV_DTYPE_F32) return load_raw<LV_DTYPE_F32, H, HS>(base, h0);
    return load_raw<LV_DTYPE_BF16, H, HS>(base, h0);  // 16-bit types share the raw layout
}

// Stores 4 * H values in the same layout; 16-bit values are already quantised: a bf16 value is
// the high half of its register (worker.rs:55-63); an fp16 value is an f32 whose round-toward-zero
// conversion is the fp16 result (sr_fp16_val, rne_fp16_val: quantize_lane).
template <int DT, int H, uint32_t HS = 4>
__device__ __forceinline__ void store_raw(void *base, uint64_t h0, const float in[8]) {
    if constexpr (DT == LV_DTYPE_F32) {
        LV_GLOBAL float *f = (LV_GLOBAL float *)base;
        __builtin_nontemporal_store(f32x4{in[0], in[1], in[2], in[3]}, (LV_GLOBAL f32x4 *)(f + h0));
        if constexpr (H == 2)
            __builtin_nontemporal_store(f32x4{in[4], in[5], in[6], in[7]}, (LV_GLOBAL f32x4 *)(f + h0 + HS));
    } else {
        uint32_t ws[4];
#pragma unroll
        for (int k = 0; k < 2 * H; k++) {
            if constexpr (DT == LV_DTYPE_BF16) {
                // the high halves of both values in one v_perm_b32 (bytes 2-3 of each)
                ws[k] = __builtin_amdgcn_perm(f_bits(in[2 * k + 1]), f_bits(in[2 * k]), 0x07060302u);
            } else {
                // fp16 values (or sr_fp16_val's sums) converted and packed in one instruction
                ws[k] = pack_f16_rtz(in[2 * k], in[2 * k + 1]);
            }
        }
        LV_GLOBAL uint16_t *h = (LV_GLOBAL uint16_t *)base;
        if constexpr (H == 2 && HS == 4) {
            __builtin_nontemporal_store(u32x4{ws[0], ws[1], ws[2], ws[3]}, (LV_GLOBAL u32x4 *)(h + h0));
        } else {
            __builtin_nontemporal_store(u32x2{ws[0], ws[1]}, (LV_GLOBAL u32x2 *)(h + h0));
            if constexpr (H == 2) __builtin_nontemporal_store(u32x2{ws[2], ws[3]}, (LV_GLOBAL u32x2 *)(h + h0 + HS));
        }
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

// The param's update from the masked direction u (dual.rs:150-228 and the matching blocks of
// dual.rs / tdclm.rs): the cautious scale cs, the radial scale bs or the coordinate bound, the
// fp16 safety bound, weight decay. u_eff is the masked direction whose square feeds the radial
// norm (dual.rs:176-180).
// active_lanes: the ballot of `active`, taken where the compare is (a lane mask kept across
// branches would be rebuilt from a VGPR).
// The cautious scale cs of a unit for its active lanes, and 0 * cs for its masked ones: the
// reference's (u * mask) * cs (dual.rs:150-160) is u * cs where mask = 1 and (u * 0) * cs where
// mask = 0, and (u * 0) * cs equals u * (0 * cs) bit for bit for every u and cs (a zero whose sign
// is sign(u) xor sign(cs), or NaN when u or cs is NaN or infinite), so an element's delta is ONE
// multiply by a select of the two. The vector path keeps both in VGPRs (a select reads at most one
// scalar operand).
struct CsPair {
    float on, off;
};

__device__ __forceinline__ CsPair cs_pair(float cs) { return {cs, 0.0f * cs}; }

// Both in VGPRs, copied once per unit.
__device__ __forceinline__ CsPair cs_pair_vgpr(float cs) {
    CsPair r;
    asm("v_mov_b32 %0, %1" : "=v"(r.on) : "s"(cs));
    asm("v_mul_f32 %0, 0, %1" : "=v"(r.off) : "v"(r.on));
    return r;
}

// p_fast: the coordinate bound took div_bound's fast side in every lane of the wave (FAST only), so
// with Args::ranges' kRangeP the updated param is finite and below 2^86 in every lane.
template <int MODE, int PT, bool FAST = false>
__device__ __forceinline__ float param_update(const Args &a, const LaneK &lk, uint32_t flags, const CsPair &cs, float bs,
                                              float p_init, float u, bool active, uint64_t active_lanes,
                                              float &u_eff, bool &p_fast) {
    constexpr bool kTri = (MODE == LV_BUFFER_T1 || MODE == LV_BUFFER_T2);
    float m_mask = active ? 1.0f : 0.0f;
    u_eff = (flags & kFCautious) ? u * m_mask : u;  // read by the radial passes only
    float delta = (flags & kFCautious) ? u * (active ? cs.on : cs.off) : u;
    float step = a.lr * delta;
    // masked steps are exact +-0s whose sign the weight decay makes irrelevant (div_bound): the
    // wave's mask of them, from the ballot of the cautious compare itself
    const uint64_t masked = ((flags & kFCautious) && (flags & kFWeightDecay)) ? ~active_lanes : 0;
    p_fast = false;
    if (flags & kFRadial) step *= bs;
    else if (flags & kFCoordinate)
        step = coordinate_bound<kTri, FAST>(step, p_init, a.ratio, lk.pade, a.bound_floor ? masked : 0, p_fast);
    if constexpr (PT == LV_DTYPE_F16) step = fp16_safety_bound<kTri, FAST>(step, p_init, lk.pade, masked);
    float p_dec = (flags & kFWeightDecay) ? __builtin_fmaf(a.neg_lr_wd, p_init, p_init) : p_init;
    return p_dec - step;
}

// quantize<DT> where the caller may know (`in_range`, wave-uniform) that every lane's value is
// finite and at most the largest finite bf16: then a bf16 stochastic rounding is the add alone,
// without sr_bf16_checked's compare.
template <int DT>
__device__ __forceinline__ float quantize_known(float v, uint32_t z0, bool sr, bool in_range) {
    if constexpr (DT == LV_DTYPE_BF16) {
        if (!sr) return rne_bf16(v);
        const uint32_t noise = xor_fold16((uint32_t)prng_mixed(z0));
        if (__builtin_expect(in_range, 1)) return sr_bf16_add(v, noise);
        return sr_bf16_checked(v, noise);
    } else {
        return quantize<DT>(v, z0, sr);
    }
}

// Apply path for one element. Counts the cautious mask bit into cnt (TALLY). m and v are
// quantised as soon as they are known: the hashes of their stochastic rounding then overlap the
// param's bound (each wave-uniform guard limits how far the compiler moves code). With master
// weights p is rounded to nearest from the master (the master keeps the f32 value).
// With 16-bit state (kFast) the roundings skip the range tests compute_u and param_update have
// already settled for the whole wave (kKnownM with kRangeM for m', kKnownV for v', the coordinate
// bound's fast side with kRangeP for p).
template <int MODE, int PT, int ST, int TALLY>
__device__ __forceinline__ void apply_elem(const Args &a, const StepCoeffs &k, const LaneK &lk, uint32_t flags, const HashIn &z,
                                           const CsPair &cs, float bs, float p_init, float g_raw, float &m_io,
                                           float &v_io, float &p_out, float &mp_out, float &u_eff, uint32_t &cnt) {
    constexpr bool kDual = (MODE == LV_BUFFER_DUAL || MODE == LV_BUFFER_T2);
    constexpr bool kFast = ST != LV_DTYPE_F32;  // the guarded divisions where VALU work is the bound
    const bool sr = flags & kFSR;
    float g = sanitize(g_raw);
    float m_new, v_new;
    uint32_t known;
    float u = compute_u<MODE, kFast>(a, k, lk, flags & kFClampV, g, m_io, v_io, m_new, v_new, known);
    bool active = (u * g) > 0.0f;
    const uint64_t active_lanes = __builtin_amdgcn_ballot_w64(active);
    tally<TALLY>(cnt, active);
    m_io = quantize_known<ST>(m_new, z.m, sr, (known & kKnownM) && (a.ranges & kRangeM));
    if constexpr (kDual) v_io = quantize_known<ST>(v_new, z.v, sr, known & kKnownV);
    bool p_fast;
    float p_upd = param_update<MODE, PT, kFast>(a, lk, flags, cs, bs, p_init, u, active, active_lanes, u_eff, p_fast);
    if (flags & kFMaster) {
        mp_out = p_upd;
        p_out = quantize<PT>(p_upd, z.p, false);
    } else {
        p_out = quantize_known<PT>(p_upd, z.p, sr, p_fast && (a.ranges & kRangeP));
    }
}

// apply_elem without the quantisation: m_io and v_io receive m' and v', p_out the updated param
// (and mp_out too, with master weights), all in f32, for quantize_lane. FAST as for compute_u.
// `known` receives compute_u's facts (kKnown*).
template <int MODE, int PT, int TALLY, bool FAST>
__device__ __forceinline__ void update_elem(const Args &a, const StepCoeffs &k, const LaneK &lk, uint32_t flags,
                                            const CsPair &cs, float bs, float p_init, float g_raw, float &m_io, float &v_io,
                                            float &p_out, float &mp_out, float &u_eff, uint32_t &cnt, uint32_t &known) {
    constexpr bool kDual = (MODE == LV_BUFFER_DUAL || MODE == LV_BUFFER_T2);
    float g = sanitize(g_raw);
    float m_new, v_new;
    float u = compute_u<MODE, FAST>(a, k, lk, flags & kFClampV, g, m_io, v_io, m_new, v_new, known);
    bool active = (u * g) > 0.0f;
    const uint64_t active_lanes = __builtin_amdgcn_ballot_w64(active);
    tally<TALLY>(cnt, active);
    m_io = m_new;
    if constexpr (kDual) v_io = v_new;
    bool p_fast;
    p_out = param_update<MODE, PT, FAST>(a, lk, flags, cs, bs, p_init, u, active, active_lanes, u_eff, p_fast);
    if (flags & kFMaster) mp_out = p_out;
}

// The vector path's quantisation of a thread's N = 4H updated values of m, v (kDual) and p: the
// values quantize<> gives element by element (element j's hash input is its stream's base plus
// j's offset from the thread's first element: j, or HS + j - 4 in the second group of 4). The
// bf16 stochastic roundings (one integer add each, sr_bf16_add) share ONE test: when any of the
// lane's values to round is NaN or has |x| above the largest finite bf16 in any lane of the wave,
// all of them go through sr_bf16_prep first (the identity for the others). The maximum of the
// magnitudes is NaN-propagating (v_maximum3_f32), so the test `!(max <= largest)` sees NaNs.
// mv_known (wave-uniform): every lane's m (and v) values are known finite and at most the largest
// finite bf16 (kKnownM with kRangeM, and kKnownV), so they stay out of the test.
template <int ST, int PT, bool kDual, int N, uint32_t HS>
__device__ __forceinline__ void quantize_lane(uint32_t flags, const HashIn &zb, float m[8], float v[8], float p[8],
                                              bool mv_known = false) {
    const bool sr = flags & kFSR;
    const bool psr = sr && !(flags & kFMaster);
    constexpr bool kBfMV = ST == LV_DTYPE_BF16;  // m (and v) rounded stochastically to bf16 when sr
    constexpr bool kBfP = PT == LV_DTYPE_BF16;   // p rounded stochastically to bf16 when psr
    const bool mv_sr = kBfMV && sr, p_sr = kBfP && psr;
    const bool mv_test = mv_sr && !mv_known;
    if (mv_test || p_sr) {
        float mx = 0.0f;
#pragma unroll
        for (int j = 0; j < N; j++) {
            if (mv_test) {
                mx = __builtin_elementwise_maximum(mx, __builtin_fabsf(m[j]));
                if constexpr (kDual) mx = __builtin_elementwise_maximum(mx, __builtin_fabsf(v[j]));
            }
            if (p_sr) mx = __builtin_elementwise_maximum(mx, __builtin_fabsf(p[j]));
        }
        if (__builtin_expect(!wave_all(mx <= __uint_as_float(kBf16MaxBits)), 0)) {
#pragma unroll
            for (int j = 0; j < N; j++) {
                if (mv_test) {
                    m[j] = sr_bf16_prep(m[j]);
                    if constexpr (kDual) v[j] = sr_bf16_prep(v[j]);
                }
                if (p_sr) p[j] = sr_bf16_prep(p[j]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < N; j++) {
        const uint32_t off = j < 4 ? (uint32_t)j : HS + (uint32_t)(j - 4);
        if (mv_sr) {
            m[j] = sr_bf16_add(m[j], xor_fold16((uint32_t)prng_mixed(zb.m + off)));
            if constexpr (kDual) v[j] = sr_bf16_add(v[j], xor_fold16((uint32_t)prng_mixed(zb.v + off)));
        } else {
            m[j] = quantize<ST>(m[j], zb.m + off, sr);
            if constexpr (kDual) v[j] = quantize<ST>(v[j], zb.v + off, sr);
        }
        if (p_sr) p[j] = sr_bf16_add(p[j], xor_fold16((uint32_t)prng_mixed(zb.p + off)));
        else if constexpr (PT == LV_DTYPE_F16) p[j] = psr ? sr_fp16_val(p[j], zb.p + off) : rne_fp16_val(p[j]);
        else p[j] = quantize<PT>(p[j], zb.p + off, psr);
    }
}

// Counting path for one element (dual.rs:279-303, dual.rs:720-746, tdclm.rs:232-248).
template <int MODE, int TALLY>
__device__ __forceinline__ void count_elem(const Args &a, const StepCoeffs &k, const LaneK &lk, uint32_t flags, float g_raw,
                                           float m, float v, float &u_eff, uint32_t &cnt) {
    float g = sanitize(g_raw);
    float m_new, v_new;
    float u = compute_u<MODE>(a, k, lk, flags & kFClampV, g, m, v, m_new, v_new);
    bool active = (u * g) > 0.0f;
    tally<TALLY>(cnt, active);
    u_eff = (flags & kFCautious) ? u * (active ? 1.0f : 0.0f) : u;
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
    LV_GLOBAL float *s = (LV_GLOBAL float *)D.scratch;
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
template <int TPB>
struct BlockSums {
    double su[TPB / 64];
    double sp[TPB / 64];
    unsigned long long cnt[TPB / 64];
};

template <int TPB, typename C>
__device__ __forceinline__ void block_sums(BlockSums<TPB> &sh, double &su, double &sp, C &cnt) {
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
        for (int k = 1; k < TPB / 64; k++) {
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

// The device table of a table launch, read through the constant address space.
__device__ __forceinline__ const LV_CONSTANT TDesc *table_of(const Args &a) {
    return (const LV_CONSTANT TDesc *)a.dtab;
}

// A copy of the descriptor of tensor t of a table launch (a reference into the table would not
// carry its address space), field by field.
static_assert(sizeof(Desc) == 80, "table_desc copies every field of Desc: extend it with the struct");
__device__ __forceinline__ Desc table_desc(const Args &a, int t) {
    const LV_CONSTANT Desc &c = table_of(a)[t].d;
    Desc d;
    d.p = c.p;
    d.g = c.g;
    d.m = c.m;
    d.v = c.v;
    d.mp = c.mp;
    d.scratch = c.scratch;
    d.n = c.n;
    d.unit_begin = c.unit_begin;
    d.pidx = c.pidx;
    d.ibase = c.ibase;
    d.nskip = c.nskip;
    d.head = c.head;
    d.vec = c.vec;
    d.skip = c.skip;
    return d;
}

// What a block needs to know about the tensor that owns its current unit.
struct View {
    uint32_t t_begin, t_end;  // the tensor's unit range in the launch
    uint32_t slot_base;       // its first count slot (64-byte index into Args::slots)
    uint64_t n;
    bool vec_ok;              // every stream aligned at element `head`: whole units vectorised
    uint32_t head;            // elements before the first aligned element (vec_ok only; else 0)
    float cs, bs;             // cautious / radial scale read from the scratch (fused, apply)
    Seeds sd;
    uint32_t ibase;
    StepCoeffs k;             // this step's c1, c2, c_sigma (kernel arguments, or the step record)
    bool skip;                // graph launch whose step record refused the step: change nothing
};

// What a block needs to address its unit: the tensor's first unit, size and alignment. In inline
// launches everything else a block reads before its arithmetic (open_step) waits until its stream
// loads are in flight: each dependent scalar load before the first vector load delays every
// block's loads by a scalar-cache round trip, and a block lives only a few microseconds.
__device__ __forceinline__ View open_view(const Desc &D) {
    View tv;
    tv.t_begin = D.unit_begin;
    tv.n = D.n;
    tv.vec_ok = D.vec;
    tv.head = D.vec ? D.head : 0u;
    return tv;
}

// The rest of the view: the tensor's unit end and count slots, this step's coefficients and seeds
// (the kernel arguments, or the step record of a graph launch) and the scales in the scratch.
template <int MODE, int PASS, bool TABLE>
__device__ __forceinline__ void open_step(const Args &a, const Desc &D, int t, uint32_t unit, View &tv) {
    if constexpr (TABLE) {
        tv.t_end = table_of(a)[t].unit_end;
        tv.slot_base = table_of(a)[t].slot_base;
    } else {
        tv.t_end = (t + 1 < a.ndesc) ? a.d[t + 1].unit_begin : a.total_units;
        tv.slot_base = (uint32_t)t * kSlotWords;
    }
    tv.ibase = D.ibase;
    // The scales are loaded before the step record is read, so that a graph launch waits for both
    // loads at once rather than for one after the other.
    float cs = 1.0f, bs = 1.0f;
    if constexpr (PASS == kFused || PASS == kApply) {
        cs = ((const LV_GLOBAL float *)D.scratch)[3];
        bs = ((const LV_GLOBAL float *)D.scratch)[4];
    }
    uint32_t seed_base = a.seed_base;
    tv.k = {a.c1, a.c2, a.c_sigma};
    tv.skip = false;
    if (a.step_rec) {  // graph launch: the coefficients the step record kernel wrote for this step
        const lv_step_record *r = a.step_rec;
        tv.k = {r->c1, r->c2, r->c_sigma};
        seed_base = r->seed_base;
        tv.skip = r->status != 0;
    }
    uint32_t raw = seed_base + D.pidx * 10007u;
    tv.sd.m = (int32_t)(raw & 0x7FFFFFFFu);
    tv.sd.p = (int32_t)(((uint32_t)tv.sd.m + 0x55555555u) & 0x7FFFFFFFu);
    tv.sd.v = (int32_t)(((uint32_t)tv.sd.m + 0x2A6D365Bu) & 0x7FFFFFFFu);
    if constexpr ((PASS == kFused || PASS == kApply) && !TABLE) {
        // Read after the stream loads, the scales come back through the vector memory path; the
        // values are block-uniform and stay in scalar registers.
        cs = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, cs)));
        bs = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, bs)));
    }
    // Table launches read the scales here, before the stream loads, and the compiler may use scalar
    // loads: a launch writes a tensor's scales only in the block that completes its count, after
    // every block of the tensor has read them.
    tv.cs = cs;
    tv.bs = bs;
    if constexpr (PASS == kSingle) {
        // reset_accumulators (state.rs:105-111) with the host-side forcing of slots 3/4
        // that the reference applies when cautious/radial are off (luminav.py:1748-1751).
        if (unit == tv.t_begin && threadIdx.x == 0 && !tv.skip) {
            LV_GLOBAL float *sc = (LV_GLOBAL float *)D.scratch;
            sc[0] = 0.0f; sc[1] = 0.0f; sc[2] = 0.0f; sc[3] = 1.0f; sc[4] = 1.0f; sc[5] = 0.0f;
        }
    }
}

// Vector loads of one thread's 4 * H elements: [e, e + 4) and (H = 2) [e + HS, e + HS + 4).
template <int MODE, int PT, int ST, int PASS, int H, uint32_t HS = 4>
__device__ __forceinline__ Inflight issue_at(const Desc &D, uint32_t flags, bool radial, uint64_t e) {
    constexpr bool kDual = (MODE == LV_BUFFER_DUAL || MODE == LV_BUFFER_T2);
    const int gdt = (int)((flags >> 8) & 3u);
    Inflight f;
    f.g = load_raw_dyn<H, HS>(gdt, D.g, e);
    f.m = load_raw<ST, H, HS>(D.m, e);
    if constexpr (kDual) f.v = load_raw<ST, H, HS>(D.v, e);
    if (PASS != kCount || radial) {  // the count pass reads p only for the radial norm
        if (flags & kFMaster) f.p = load_raw<LV_DTYPE_F32, H, HS>(D.mp, e);
        else f.p = load_raw<PT, H, HS>(D.p, e);
    }
    return f;
}

// The LaneK of the vector path: VGPR copies of the constants that mode reads with another uniform
// operand. eps is read by T1, T2 and TD-CLM, the tanh constants by CLM and TD-CLM (tanh_pade).
// CLM with 16-bit state keeps the tanh constants as they are: there the extra VGPRs would cost
// some of its kernels a wave of occupancy (T2's eps costs none of its kernels one).
template <int MODE, int H>
__device__ __forceinline__ LaneK lane_consts(const Args &a) {
    LaneK lk{a.eps, kPade};
    if constexpr (MODE == LV_BUFFER_T1 || MODE == LV_BUFFER_TDCLM || MODE == LV_BUFFER_T2) lk.eps = in_vgpr(a.eps);
    if constexpr (MODE == LV_BUFFER_TDCLM || (MODE == LV_BUFFER_DUAL && H == 1))
        lk.pade = PadeK{in_vgpr(kPade.hi), in_vgpr(kPade.p0), in_vgpr(kPade.q0)};
    return lk;
}

// Update (or count) the 4 * H elements loaded by issue_at(e0) and store them. BALLOT: every lane
// of the wave is here, and cnt accumulates the wave's count (the same in every lane) from ballots;
// otherwise cnt accumulates the lane's own count.
template <int MODE, int PT, int ST, int PASS, int H, bool BALLOT, uint32_t HS = 4>
__device__ __forceinline__ void process_at(const Args &a, const Desc &D, const View &tv, uint32_t flags, bool radial,
                                           const Inflight &cur, uint64_t e0, uint32_t &cnt, double &su, double &sp) {
    constexpr bool kDual = (MODE == LV_BUFFER_DUAL || MODE == LV_BUFFER_T2);
    constexpr bool kCounting = (PASS == kFused || PASS == kCount);
    constexpr int kTally = !kCounting ? kTallyNone : (BALLOT ? kTallyWave : kTallyLane);
    const int gdt = (int)((flags >> 8) & 3u);
    const bool master = flags & kFMaster;
    const LaneK lk = lane_consts<MODE, H>(a);
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
            count_elem<MODE, kTally>(a, tv.k, lk, flags, g[j], m[j], kDual ? v[j] : 0.0f, ue, cnt);
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
        const CsPair csp = cs_pair_vgpr(tv.cs);
        uint32_t known_all = ~0u;  // the kKnown* facts that hold for all of the lane's elements
#pragma unroll
        for (int j = 0; j < 4 * H; j++) {
            float vj = kDual ? v[j] : 0.0f;
            float ue;
            if constexpr (PT == LV_DTYPE_F16) {
                // fp16 params: the lane's values are quantised together below (2% faster on the
                // fp16-container cfg4 step than element by element)
                uint32_t known;
                update_elem<MODE, PT, kTally, ST != LV_DTYPE_F32>(a, tv.k, lk, flags, csp, tv.bs, pin[j], g[j], m[j], vj,
                                                                   pout[j], mpout[j], ue, cnt, known);
                known_all &= known;
            } else {
                // quantised element by element: each hash then overlaps the next element's arithmetic
                // (quantising the lane's bf16 values together after all of them measured 4% slower)
                const uint32_t off = j < 4 ? (uint32_t)j : HS + (uint32_t)(j - 4);  // element offset from e0
                const HashIn zj = {zb.m + off, zb.p + off, zb.v + off};
                apply_elem<MODE, PT, ST, kTally>(a, tv.k, lk, flags, zj, csp, tv.bs, pin[j], g[j], m[j], vj, pout[j],
                                                 mpout[j], ue, cnt);
            }
            if constexpr (kDual) v[j] = vj;
            if (kCounting && radial) {
                su += (double)(ue * ue);
                sp += (double)(pin[j] * pin[j]);
            }
        }
        if constexpr (PT == LV_DTYPE_F16) {
            const bool m_known = (known_all & kKnownM) && (a.ranges & kRangeM);
            const bool v_known = !kDual || (known_all & kKnownV);
            quantize_lane<ST, PT, kDual, 4 * H, HS>(flags, zb, m, v, pout, m_known && v_known);
        }
        store_raw<PT, H, HS>(D.p, e0, pout);
        if (master) store_raw<LV_DTYPE_F32, H, HS>(D.mp, e0, mpout);
        store_raw<ST, H, HS>(D.m, e0, m);
        if constexpr (kDual) store_raw<ST, H, HS>(D.v, e0, v);
    }
}

// Per-element path for the elements [e_begin, e_end) of one thread (partially inactive units,
// unaligned tensors, and the last few elements of a tensor). nskip > 0: the tensor's inactive
// ranges, `first` the first range that ends after the unit's first element. Inactive elements are
// computed with a zero gradient (they count in the statistics) and not stored. cnt accumulates the
// lane's own count.
template <int MODE, int PT, int ST, int PASS>
__device__ __forceinline__ void scalar_range(const Args &a, const Desc &D, const View &tv, uint32_t flags, bool radial,
                                             uint64_t e_begin, uint64_t e_end, uint32_t &cnt, double &su, double &sp,
                                             uint32_t nskip = 0, uint32_t first = 0) {
    constexpr bool kDual = (MODE == LV_BUFFER_DUAL || MODE == LV_BUFFER_T2);
    constexpr bool kCounting = (PASS == kFused || PASS == kCount);
    const int gdt = (int)((flags >> 8) & 3u);
    const bool master = flags & kFMaster;
    uint32_t r = first;
    for (uint64_t i = e_begin; i < e_end; i++) {
        bool inactive = false;
        if (nskip) {
            while (r < nskip && ((const LV_GLOBAL uint64_t *)D.skip)[2 * r + 1] <= i) r++;
            inactive = r < nskip && ((const LV_GLOBAL uint64_t *)D.skip)[2 * r] <= i;
        }
        float g = inactive ? 0.0f : load1_dyn(gdt, D.g, i);
        float m = load1<ST>(D.m, i);
        float v = kDual ? load1<ST>(D.v, i) : 0.0f;
        if constexpr (PASS == kCount) {
            float ue;
            count_elem<MODE, kTallyLane>(a, tv.k, LaneK{a.eps, kPade}, flags, g, m, v, ue, cnt);
            if (radial) {
                float pin = master ? D.mp[i] : load1<PT>(D.p, i);
                su += (double)(ue * ue);
                sp += (double)(pin * pin);
            }
        } else {
            float pin = master ? D.mp[i] : load1<PT>(D.p, i);
            float pout, mpout, ue;
            apply_elem<MODE, PT, ST, kCounting ? kTallyLane : kTallyNone>(
                a, tv.k, LaneK{a.eps, kPade}, flags, hash_in(tv.sd, (uint32_t)i + tv.ibase), cs_pair(tv.cs), tv.bs, pin, g, m, v,
                pout, mpout, ue, cnt);
            if (!inactive) {
                store1<PT>(D.p, i, pout);
                if (master) D.mp[i] = mpout;
                store1<ST>(D.m, i, m);
                if constexpr (kDual) store1<ST>(D.v, i, v);
            }
            if (kCounting && radial) {
                su += (double)(ue * ue);
                sp += (double)(pin * pin);
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
        if (((const LV_GLOBAL uint64_t *)D.skip)[2 * mid + 1] <= e0) lo = mid + 1;
        else hi = mid;
    }
    first = lo;
    if (lo == D.nskip) return 0;
    const uint64_t b = ((const LV_GLOBAL uint64_t *)D.skip)[2 * lo], e = ((const LV_GLOBAL uint64_t *)D.skip)[2 * lo + 1];
    if (b >= e1) return 0;
    return (b <= e0 && e >= e1) ? 2 : 1;
}

// Index of the tensor that owns `unit`: binary search of the unit ranges. Table launches search
// the heads in the kernel arguments, then (groups of more than one tensor) the head's group in
// the device table. Every tensor of a launch has at least one unit, so the ranges are strictly
// increasing.
template <bool TABLE>
__device__ __forceinline__ int find_tensor(const Args &a, uint32_t unit) {
    if constexpr (!TABLE) {
        int lo = 0, hi = a.ndesc - 1;
        while (lo < hi) {
            int mid = (lo + hi + 1) >> 1;
            if (a.d[mid].unit_begin <= unit) lo = mid;
            else hi = mid - 1;
        }
        return lo;
    } else {
        int lo = 0, hi = (int)a.nheads - 1;
        while (lo < hi) {
            int mid = (lo + hi + 1) >> 1;
            if (a.ubegin[mid] <= unit) lo = mid;
            else hi = mid - 1;
        }
        if (a.group == 1) return lo;
        int tlo = lo * (int)a.group;
        int thi = tlo + (int)a.group - 1;
        if (thi > a.ndesc - 1) thi = a.ndesc - 1;
        while (tlo < thi) {
            int mid = (tlo + thi + 1) >> 1;
            if (table_of(a)[mid].d.unit_begin <= unit) tlo = mid;
            else thi = mid - 1;
        }
        return tlo;
    }
}

// ------------------------------------------------------------------ the kernels

// Counting unit launches: thread 0 of every block reports its exact mask count and the block's
// completion in ONE 64-bit atomic (count << kTicketBits | 1) on one of the tensor's S count slots
// (slot = unit index in the tensor mod S, 64 B apart, so the atomics spread over L2 channels;
// S = table_count_slots(units): the smallest power of two keeping every slot at <= 64 blocks, at
// most 64). The block whose report completes a slot (its ticket reaches the slot's block count)
// holds that slot's whole count in the value its own atomic returned and re-zeroes the slot; a
// tensor of one slot (<= 64 units) is then complete, and that block finalises the scratch. With
// more slots it reports count << kFoldBits | 1 on the tensor's fold slot (the one after its count
// slots), and the block that completes the fold slot holds the tensor's exact count and
// finalises the scratch. Every decision reads only the value
// returned by an atomic on that same word, so no fence is needed (a device-scope release fence
// per block measured 7x slower); integer sums are exact in any order, so the result is
// deterministic. Wholly inactive units report a zero count.
template <int MODE, int PASS, bool TABLE>
__device__ __forceinline__ void report_count(const Args &a, const Desc &D, const View &tv, uint32_t unit,
                                             uint32_t count) {
    const uint32_t n_units = tv.t_end - tv.t_begin;
    const uint32_t k = unit - tv.t_begin;
    // slot s of S takes units k = s (mod S): n_units / S blocks, plus one for s < n_units % S
    const uint32_t S = table_count_slots(n_units);  // a power of two, <= 64 blocks per slot
    const uint32_t s = k & (S - 1u);
    const uint32_t nslots = n_units < S ? n_units : S;
    unsigned long long *words = a.slots + (size_t)tv.slot_base * kSlotStride;
    unsigned long long *slot = words + (size_t)s * kSlotStride;
    constexpr unsigned long long kTicketMask = (1ull << kTicketBits) - 1ull;
    const unsigned long long old = __hip_atomic_fetch_add(slot, ((unsigned long long)count << kTicketBits) | 1ull,
                                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t expect = (n_units >> __builtin_ctz(S)) + (s < (n_units & (S - 1u)) ? 1u : 0u);
    if ((uint32_t)(old & kTicketMask) + 1u != expect) return;
    const unsigned long long slot_count = (old >> kTicketBits) + count;
    __hip_atomic_store(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (nslots == 1u) {  // a tensor of <= 64 units: its one slot holds its whole count
        finalize_scratch<MODE, PASS>(a, false, D, slot_count, 0.0f, 0.0f);
        return;
    }
    unsigned long long *fold = words + (size_t)nslots * kSlotStride;
    const unsigned long long prev = __hip_atomic_fetch_add(fold, (slot_count << kFoldBits) | 1ull, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT);
    if ((uint32_t)(prev & ((1ull << kFoldBits) - 1ull)) + 1u != nslots) return;
    __hip_atomic_store(fold, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    finalize_scratch<MODE, PASS>(a, false, D, (prev >> kFoldBits) + slot_count, 0.0f, 0.0f);
}

// Offset in elements of a thread's second group of 4 in a 2048-element unit (the layout above
// load_raw): 4, so that the thread's 8 elements are consecutive, unless the launch may move an
// f32 stream beside its 16-bit ones (a master copy, f32 grads, or a flag word known only at run
// time), then 1024.
constexpr uint32_t lane_split(int H, uint32_t FL) {
    return (H == 2 && ((FL & kFDynamic) || (FL & kFMaster) || ((FL >> 8) & 3u) == LV_DTYPE_F32)) ? kHalf : 4u;
}

// One sub-unit [ub, ub + 1024 * H) of a block that does not take the whole-unit vector path: the
// partial last unit of an aligned tensor (whole groups of 4 as vectors), streams with no common
// 16-byte alignment (element by element, coalesced across the wave), or inactive ranges
// (`cover`: 0 none, 1 partly, 2 wholly; `first` the first range that ends after ub). cnt
// accumulates the lane's own count.
template <int MODE, int PT, int ST, int PASS, int H, uint32_t HS, int TPB>
__device__ __forceinline__ void subunit_nonvec(const Args &a, const Desc &D, const View &tv, uint32_t flags, bool radial,
                                               uint64_t ub, int cover, uint32_t first, uint32_t &cnt, double &su,
                                               double &sp) {
    constexpr bool kCounting = (PASS == kFused || PASS == kCount);
    if (!kCounting && cover == 2) return;  // wholly inactive: nothing to write
    if (cover == 0 && tv.vec_ok) {
        const uint64_t es = ub + (uint64_t)threadIdx.x * (HS == 4 ? 4u * H : 4u);
#pragma unroll
        for (int h = 0; h < H; h++) {
            const uint64_t e = es + (uint64_t)h * HS;
            if (e + 4u <= tv.n) {
                const Inflight f = issue_at<MODE, PT, ST, PASS, 1>(D, flags, radial, e);
                process_at<MODE, PT, ST, PASS, 1, false>(a, D, tv, flags, radial, f, e, cnt, su, sp);
            } else if (e < tv.n) {
                scalar_range<MODE, PT, ST, PASS>(a, D, tv, flags, radial, e, tv.n, cnt, su, sp);
            }
        }
    } else if (cover == 0) {
#pragma unroll 1
        for (uint32_t j = 0; j < 4u * H; j++) {
            const uint64_t e = ub + (uint64_t)j * TPB + threadIdx.x;
            if (e < tv.n) scalar_range<MODE, PT, ST, PASS>(a, D, tv, flags, radial, e, e + 1, cnt, su, sp);
        }
    } else if (cover != 2 || radial) {
        const uint64_t eb = ub + (uint64_t)threadIdx.x * (4u * H);
        const uint64_t ee = eb + 4u * H < tv.n ? eb + 4u * H : tv.n;
        scalar_range<MODE, PT, ST, PASS>(a, D, tv, flags, radial, eb, ee, cnt, su, sp, cover ? D.nskip : 0, first);
    }
}

// Unit launch: each block updates exactly one work unit (256, 1024, 2048 or 4096 elements: unit_elems) and
// exits.
// The hardware keeps every CU full with fresh blocks, so the loads of some blocks overlap the
// arithmetic of others without a software pipeline; on MI355X this launch shape streams HBM
// faster than any persistent grid-stride loop over the same buffers (measured: 23.4 vs 26.5 ms
// for the 6.7e9-element T2 step; 2048-element units: 23.7 ms). Counting passes report each
// block's exact mask count (report_count), and the last block of each tensor finalises its
// scratch, so a step is one launch. Radial counting passes instead store each unit's record
// (mask count and f64 squared-norm sums) for fold_kernel.
// A tensor's partial last unit keeps the vector layout: each thread's 4-element groups that lie
// wholly inside the tensor take the vector path, and only the one group that straddles the end
// goes element by element.
// FL is either kFDynamic (flags read at run time) or the exact flag word of the launch, in
// which case every option test folds at compile time and the per-element code is straight-line.
// TABLE: the tensor table is in device memory (a.dtab) and the heads in a.ubegin.
template <int MODE, int PT, int ST, int PASS, uint32_t FL, bool TABLE>
__global__ void __launch_bounds__(unit_threads(MODE, PT, ST, PASS, FL, TABLE), unit_min_blocks(MODE, PT, ST, PASS, FL))
    unit_kernel(const Args a) {
    constexpr bool kCounting = (PASS == kFused || PASS == kCount);
    constexpr int TPB = unit_threads(MODE, PT, ST, PASS, FL, TABLE);  // threads per block
    __shared__ BlockSums<TPB> sh;

    const uint32_t flags = (FL & kFDynamic) ? a.flags : FL;
    const bool radial = kCounting && (flags & kFRadial);  // squared norms summed in this pass
    // Workgroups are dispatched to the XCDs round-robin (block b runs on XCD b mod X). Map them so
    // that each XCD streams one contiguous range of units, or, where the host passes X = 1, block
    // b on unit b (which launches take which mapping: launch() in luminav_hip.hip).
    // Every block is short-lived, so its prologue is on the critical path: b / X comes from the
    // host's reciprocal (exact for b < 2^23 and X <= 64) instead of an integer division, which
    // measured 1.3% of the cfg5 step.
    // With one XCD the mapping is b itself: an identity-mapped launch has up to kMaxGridIdentity
    // = 2^25 blocks, past the reciprocal's range (b * recip overflows 64 bits from b = 2^24).
    const uint32_t b = blockIdx.x;
    uint32_t unit;
    if (a.xcds == 1) {
        unit = a.unit_base + b;
    } else {
        const uint32_t i = (uint32_t)(((uint64_t)b * a.xcd_recip) >> 40);
        const uint32_t x = b - i * a.xcds;
        unit = a.unit_base + x * a.xcd_q + (x < a.xcd_r ? x : a.xcd_r) + i;
    }
    const int t = find_tensor<TABLE>(a, unit);
    Desc table_d;
    if constexpr (TABLE) table_d = table_desc(a, t);
    const Desc &D = TABLE ? table_d : a.d[t];
    View tv = open_view(D);
    // Table launches (many small tensors, latency-bound, descriptors in device memory) read the
    // rest of the view first: issued behind the stream loads, those reads queue after them
    // (cfg2's 64-tensor launch: 20.6 vs 18.7 us). Inline launches stream and read it afterwards.
    if constexpr (TABLE) {
        open_step<MODE, PASS, TABLE>(a, D, t, unit, tv);
        if (tv.skip) return;  // block-uniform: the whole launch leaves every buffer as it was
    }
    uint32_t cnt = 0;
    double su = 0.0, sp = 0.0;  // radial: sum u_eff^2, sum p^2
    constexpr int H = unit_halves(MODE, PT, ST);
    constexpr int S = unit_subs(MODE, PT, ST, PASS, FL);
    constexpr uint32_t HS = lane_split(H, FL);
    static_assert(H == 1 || TPB == kThreads, "16-bit state splits its lanes at 1024 elements");
    constexpr uint64_t kSub = 4ull * TPB * H;  // elements per sub-unit
    constexpr uint64_t kUnit = kSub * S;
    // units start at the tensor's first 16-byte aligned element (tv.head > 0: an unaligned view)
    const uint64_t ubase = (uint64_t)(unit - tv.t_begin) * kUnit + tv.head;
    // Whether this block also takes the head. One-wave kernels (identity-mapped, heads of up to 255
    // elements) use the tensor's first unit, whose block starts early in the launch: with the last
    // unit, whose head round trips fall on the launch's tail, a 2^27-element T2 view at +1
    // element ran 1.030x the aligned view, with the first 1.022x (and with the head spread over
    // the first units' blocks, 64 elements each, 1.036x). The others keep the last unit, which
    // also keeps the radial sums' fold order. Only after open_step: tv.t_end is set there.
    const auto takes_head = [&]() {
        if constexpr (TPB == kThreads) return tv.head && unit + 1u == tv.t_end;
        else return tv.head && unit == tv.t_begin;
    };
    int cover = 0;
    uint32_t first = 0;
    if (D.nskip) cover = inactive_cover(D, ubase, ubase + kUnit < tv.n ? ubase + kUnit : tv.n, first);
    // Vector path over a whole unit: cnt ends as the wave's count (the same in every lane, from
    // ballots); every other path: cnt is the lane's count.
    const bool fast = cover == 0 && tv.vec_ok;
    const bool vec = fast && ubase + kUnit <= tv.n;
    const uint64_t e0 = ubase + (uint64_t)threadIdx.x * (HS == 4 ? 4u * H : 4u);  // the first group
    if (vec) {
        Inflight f[S];
#pragma unroll
        for (int sub = 0; sub < S; sub++)
            f[sub] = issue_at<MODE, PT, ST, PASS, H, HS>(D, flags, radial, e0 + (uint64_t)sub * kSub);
        if constexpr (!TABLE) {
            __builtin_amdgcn_sched_barrier(0);  // every stream load is issued before the step's reads
            open_step<MODE, PASS, TABLE>(a, D, t, unit, tv);
            // A graph step refused by its step record changes nothing (block-uniform; the loads
            // above only read).
            if (tv.skip) return;
        }
        // Waves whose loads are in flight outrank freshly started ones, so a SIMD finishes (and
        // stores) the units it holds before new blocks add loads: ~0.5% more HBM throughput. The
        // two-sub-unit kernels already hold their next loads in flight and keep the default
        // priority (fp16 cfg4 0.995x and 0.991x, bf16-state cfg4 0.9995x, in one process each); the
        // explicit priority 0 costs one scalar instruction and marks the same point in the code.
        __builtin_amdgcn_s_setprio(S == 1 ? 1 : 0);
#pragma unroll
        for (int sub = 0; sub < S; sub++)
            process_at<MODE, PT, ST, PASS, H, true, HS>(a, D, tv, flags, radial, f[sub], e0 + (uint64_t)sub * kSub, cnt,
                                                       su, sp);
    } else {
        if constexpr (!TABLE) {
            open_step<MODE, PASS, TABLE>(a, D, t, unit, tv);
            if (tv.skip) return;  // block-uniform: the whole launch leaves every buffer as it was
        }
        // A wholly inactive unit has a zero gradient (its mask count is 0) and writes nothing;
        // its elements still enter the radial norms.
        if (!kCounting && cover == 2 && !takes_head()) return;
        if constexpr (S == 1) {
            subunit_nonvec<MODE, PT, ST, PASS, H, HS, TPB>(a, D, tv, flags, radial, ubase, cover, first, cnt, su, sp);
        } else {
#pragma unroll 1
            for (int sub = 0; sub < S; sub++) {
                const uint64_t ub = ubase + (uint64_t)sub * kSub;  // this sub-unit's first element
                if (ub >= tv.n) break;
                uint32_t sfirst = 0;
                const int scover = D.nskip ? inactive_cover(D, ub, ub + kSub < tv.n ? ub + kSub : tv.n, sfirst) : 0;
                subunit_nonvec<MODE, PT, ST, PASS, H, HS, TPB>(a, D, tv, flags, radial, ub, scover, sfirst, cnt, su, sp);
            }
        }
    }
    // An unaligned view's head [0, tv.head) (its streams are aligned from element tv.head on; at
    // most 255 elements) is taken by one block, after its unit, element j in thread j mod TPB.
    // Block-uniform; its count joins cnt as the wave's (vector path) or the lane's count.
    if (takes_head()) {
        uint32_t hc = 0, hfirst = 0;
        const int hcover = D.nskip ? inactive_cover(D, 0, tv.head, hfirst) : 0;
        if (kCounting || hcover != 2) {
            if constexpr (TPB == kThreads) {  // a head of at most 63 elements: one per thread
                if (threadIdx.x < tv.head)
                    scalar_range<MODE, PT, ST, PASS>(a, D, tv, flags, radial, threadIdx.x, threadIdx.x + 1, hc, su, sp,
                                                     hcover ? D.nskip : 0, hfirst);
            } else {
                for (uint32_t j = threadIdx.x; j < tv.head; j += TPB)
                    scalar_range<MODE, PT, ST, PASS>(a, D, tv, flags, radial, j, j + 1, hc, su, sp, hcover ? D.nskip : 0,
                                                     hfirst);
            }
        }
        if constexpr (kCounting) cnt += vec ? wave_sum(hc) : hc;
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
                for (int k = 0; k < TPB / 64; k++) tot += (uint32_t)sh.cnt[k];
                report_count<MODE, PASS, TABLE>(a, D, tv, unit, tot);
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
// piece sizes. Every record is zeroed once it has been read, so the call leaves the whole
// workspace zero (a later call may use the same bytes as count words).
template <int MODE, int PASS>
__global__ void __launch_bounds__(kThreads) fold_kernel(const Args a) {
    __shared__ BlockSums<kThreads> sh;
    __shared__ uint32_t last;
    if (a.step_rec && a.step_rec->status != 0) return;  // refused graph step: the unit launch wrote nothing
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
    double2 *sq = reinterpret_cast<double2 *>(a.unit_sq);
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
            const uint32_t k = kb + r * kThreads + threadIdx.x;
            if (k < k1) {
                su += x[r].x;
                sp += x[r].y;
                cnt += c[r];
                sq[k] = double2{0.0, 0.0};
                a.unit_cnt[k] = 0u;
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
        RadialSum *r = a.chunks + cbase + k;
        su += load_relaxed(&r->su);
        sp += load_relaxed(&r->sp);
        total += __hip_atomic_load(&r->cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        r->su = 0.0;
        r->sp = 0.0;
        r->cnt = 0ull;
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
            run.su = 0.0;
            run.sp = 0.0;
            run.cnt = 0ull;
        } else {
            run.su = su;
            run.sp = sp;
            run.cnt = total;
        }
        __hip_atomic_store(&a.tickets[t], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ------------------------------------------------------------------ kernel pickers

using KernelFn = void (*)(Args);


// The same defaults with bound_type="radial" (the radial passes never run SINGLE).
constexpr uint32_t radial_flags(int PT) {
    return ((uint32_t)kFCautious | (uint32_t)kFSR | (uint32_t)kFWeightDecay | (uint32_t)kFRadial |
            (PT == LV_DTYPE_F16 ? (uint32_t)kFClampV : 0u) | ((uint32_t)PT << 8));
}

// Table launches (many small tensors) have the reference defaults specialised too: on cfg2's 64
// tensors the run-time-flag table kernel took 22.5 us per launch and the specialised one 19.2,
// level with a memory-only twin (19.4).
template <int MODE, int PT, int ST, int PASS>
KernelFn pick_flags(uint32_t flags, bool table) {
    constexpr uint32_t kStatic = static_flags(PT, PASS);
    constexpr uint32_t kRadial = radial_flags(PT);
    if (table) {
        if (flags == kStatic) return unit_kernel<MODE, PT, ST, PASS, kStatic, true>;
        return unit_kernel<MODE, PT, ST, PASS, kFDynamic, true>;
    }
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

template <int MODE>
KernelFn pick_fold_pass(int pass) {
    return pass == kFused ? fold_kernel<MODE, kFused> : fold_kernel<MODE, kCount>;
}

// One per buffer mode, each defined in its own kernel unit (lv_kernels.hip built with LV_MODE).
KernelFn pick_kernel_tdclm(int pt, int st, int pass, uint32_t flags, bool table);
KernelFn pick_kernel_clm(int pt, int st, int pass, uint32_t flags, bool table);
KernelFn pick_kernel_t1(int pt, int st, int pass, uint32_t flags, bool table);
KernelFn pick_kernel_t2(int pt, int st, int pass, uint32_t flags, bool table);
KernelFn pick_fold_tdclm(int pass);
KernelFn pick_fold_clm(int pass);
KernelFn pick_fold_t1(int pass);
KernelFn pick_fold_t2(int pass);

}  // namespace lv
