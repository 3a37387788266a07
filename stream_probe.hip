// The stream floor of a step: a kernel that reads and writes exactly the buffers one optimizer
// step streams (p and the state read and written, the gradient read), with the same element
// sizes, unit shape (256 threads, 1024 elements per block, 4 consecutive elements per thread) and
// non-temporal vector accesses, and no arithmetic, tensor lookup, count or scalar prologue. Its
// bandwidth is what this hardware gives that read/write mix; the step kernel's own rate is read
// against it. Not part of the optimizer library: bench.py loads it for --stream-floor.
//
// Each output depends on its inputs, so no load is dead: p ^= g word by word, m ^= the thread's
// first gradient word, v ^= the thread's first (old) m word.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

namespace {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int BYTES> struct Words;  // 4 elements of BYTES each
template <> struct Words<2> { using T = u32x2; };
template <> struct Words<4> { using T = u32x4; };

constexpr uint32_t kThreads = 256;
constexpr uint32_t kUnit = 1024;  // elements per block

template <int P, int S, int NS>
__global__ void __launch_bounds__(kThreads) stream_probe_kernel(void *p, const void *g, void *m, void *v, uint64_t n) {
    using PV = typename Words<P>::T;
    using SV = typename Words<S>::T;
    const uint64_t e = (uint64_t)blockIdx.x * kUnit + (uint64_t)threadIdx.x * 4u;
    if (e + 4u > n) return;  // n is a multiple of 4: whole groups only
    PV *pp = reinterpret_cast<PV *>(static_cast<char *>(p) + e * P);
    const PV *gp = reinterpret_cast<const PV *>(static_cast<const char *>(g) + e * P);
    SV *mp = reinterpret_cast<SV *>(static_cast<char *>(m) + e * S);
    const PV gv = __builtin_nontemporal_load(gp);
    const SV mv = __builtin_nontemporal_load(mp);
    SV vv{};
    if constexpr (NS == 2) vv = __builtin_nontemporal_load(reinterpret_cast<const SV *>(static_cast<char *>(v) + e * S));
    const PV pv = __builtin_nontemporal_load(pp);
    __builtin_nontemporal_store(pv ^ gv, pp);
    __builtin_nontemporal_store(mv ^ gv.x, mp);
    if constexpr (NS == 2) __builtin_nontemporal_store(vv ^ mv.x, reinterpret_cast<SV *>(static_cast<char *>(v) + e * S));
}

template <int P, int S, int NS>
hipError_t launch(void *p, const void *g, void *m, void *v, uint64_t n, uint32_t blocks, hipStream_t stream) {
    stream_probe_kernel<P, S, NS><<<blocks, kThreads, 0, stream>>>(p, g, m, v, n);
    return hipGetLastError();
}

// Other shapes of the same stream (lv_stream_probe_shape): T threads per block, G groups of 4
// elements per thread, T * 4 apart (a block covers T * 4 * G elements; every access is contiguous
// across the wave), non-temporal (NT) or plain loads and stores, one block per block-sized piece
// or a persistent grid that strides over the pieces, and block b on piece b or XCD-contiguous
// (blocks go to the 8 XCDs round robin, so block b takes piece (b mod 8) * ceil(pieces / 8) +
// b / 8 and each XCD streams one contiguous eighth). Every group's loads are issued before its
// stores, as in the step. The same outputs as stream_probe_kernel for every shape.
template <int P, int S, int NS, int T, int G, bool NT>
__device__ __forceinline__ void shape_piece(char *p, const char *g, char *m, char *v, uint64_t n, uint64_t piece) {
    using PV = typename Words<P>::T;
    using SV = typename Words<S>::T;
    constexpr uint64_t kElems = (uint64_t)T * 4u * G;
    PV pv[G], gv[G];
    SV mv[G], vv[G];
    bool ok[G];
#pragma unroll
    for (int k = 0; k < G; k++) {
        const uint64_t e = piece * kElems + (uint64_t)k * T * 4u + (uint64_t)threadIdx.x * 4u;
        ok[k] = e + 4u <= n;
        if (!ok[k]) continue;
        const PV *gp = reinterpret_cast<const PV *>(g + e * P);
        const SV *mp = reinterpret_cast<const SV *>(m + e * S);
        const PV *pp = reinterpret_cast<const PV *>(p + e * P);
        gv[k] = NT ? __builtin_nontemporal_load(gp) : *gp;
        mv[k] = NT ? __builtin_nontemporal_load(mp) : *mp;
        if constexpr (NS == 2) {
            const SV *vp = reinterpret_cast<const SV *>(v + e * S);
            vv[k] = NT ? __builtin_nontemporal_load(vp) : *vp;
        }
        pv[k] = NT ? __builtin_nontemporal_load(pp) : *pp;
    }
#pragma unroll
    for (int k = 0; k < G; k++) {
        if (!ok[k]) continue;
        const uint64_t e = piece * kElems + (uint64_t)k * T * 4u + (uint64_t)threadIdx.x * 4u;
        PV *pp = reinterpret_cast<PV *>(p + e * P);
        SV *mp = reinterpret_cast<SV *>(m + e * S);
        const PV po = pv[k] ^ gv[k];
        const SV mo = mv[k] ^ gv[k].x;
        if (NT) {
            __builtin_nontemporal_store(po, pp);
            __builtin_nontemporal_store(mo, mp);
        } else {
            *pp = po;
            *mp = mo;
        }
        if constexpr (NS == 2) {
            SV *vp = reinterpret_cast<SV *>(v + e * S);
            const SV vo = vv[k] ^ mv[k].x;
            if (NT) __builtin_nontemporal_store(vo, vp);
            else *vp = vo;
        }
    }
}

template <int P, int S, int NS, int T, int G, bool NT, bool PERSIST, bool XCD>
__global__ void __launch_bounds__(T) shape_kernel(void *p, const void *g, void *m, void *v, uint64_t n,
                                                  uint64_t pieces) {
    char *pc = static_cast<char *>(p);
    const char *gc = static_cast<const char *>(g);
    char *mc = static_cast<char *>(m);
    char *vc = static_cast<char *>(v);
    if constexpr (PERSIST) {
        for (uint64_t piece = blockIdx.x; piece < pieces; piece += gridDim.x)
            shape_piece<P, S, NS, T, G, NT>(pc, gc, mc, vc, n, piece);
    } else if constexpr (XCD) {
        const uint64_t per = (pieces + 7u) / 8u;  // the grid is 8 * per blocks
        const uint64_t piece = (uint64_t)(blockIdx.x % 8u) * per + blockIdx.x / 8u;
        if (piece < pieces) shape_piece<P, S, NS, T, G, NT>(pc, gc, mc, vc, n, piece);
    } else {
        shape_piece<P, S, NS, T, G, NT>(pc, gc, mc, vc, n, blockIdx.x);
    }
}

// The step's shape and mapping (256 threads, 4 elements per thread, XCD-contiguous) with buffer
// loads and stores whose cache policy bits are set explicitly: LA for the loads, SA for the stores
// (bit 0 sc0, bit 1 nt, bit 4 sc1). The buffer of each stream spans exactly the block's elements,
// so lanes past the last element load zeros and store nothing.
template <int BYTES> struct Buf;
template <> struct Buf<2> {  // 4 elements of 2 bytes: 8 bytes a lane
    using T = u32x2;
    template <int AUX> static __device__ T load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
        return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, AUX);
    }
    template <int AUX> static __device__ void store(T x, __amdgpu_buffer_rsrc_t r, uint32_t off) {
        __builtin_amdgcn_raw_buffer_store_b64(x, r, off, 0, AUX);
    }
};
template <> struct Buf<4> {  // 4 elements of 4 bytes: 16 bytes a lane
    using T = u32x4;
    template <int AUX> static __device__ T load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
        return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
    }
    template <int AUX> static __device__ void store(T x, __amdgpu_buffer_rsrc_t r, uint32_t off) {
        __builtin_amdgcn_raw_buffer_store_b128(x, r, off, 0, AUX);
    }
};

constexpr int kRsrcWord3 = 0x00020000;  // raw (untyped) buffer access, as for gfx9-family dword loads

template <int P, int S, int NS, int LA, int SA>
__global__ void __launch_bounds__(kThreads) policy_kernel(void *p, const void *g, void *m, void *v, uint64_t n,
                                                          uint64_t pieces) {
    const uint64_t per = (pieces + 7u) / 8u;  // the grid is 8 * per blocks
    const uint64_t piece = (uint64_t)(blockIdx.x % 8u) * per + blockIdx.x / 8u;
    if (piece >= pieces) return;
    const uint64_t e0 = piece * kUnit;
    const int cnt = (int)(n - e0 < kUnit ? n - e0 : kUnit);  // elements of this block
    auto rsrc = [&](const void *base, int bytes) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(static_cast<const char *>(base)) + e0 * bytes, 0,
                                                 cnt * bytes, kRsrcWord3);
    };
    const __amdgpu_buffer_rsrc_t rp = rsrc(p, P), rg = rsrc(g, P), rm = rsrc(m, S);
    const uint32_t op = threadIdx.x * 4u * P, os = threadIdx.x * 4u * S;
    const auto gv = Buf<P>::template load<LA>(rg, op);
    const auto mv = Buf<S>::template load<LA>(rm, os);
    typename Buf<S>::T vv{};
    const __amdgpu_buffer_rsrc_t rv = rsrc(NS == 2 ? v : m, S);  // unused when there is no v
    if constexpr (NS == 2) vv = Buf<S>::template load<LA>(rv, os);
    const auto pv = Buf<P>::template load<LA>(rp, op);
    Buf<P>::template store<SA>(pv ^ gv, rp, op);
    Buf<S>::template store<SA>(mv ^ gv.x, rm, os);
    if constexpr (NS == 2) Buf<S>::template store<SA>(vv ^ mv.x, rv, os);
}

struct ShapeInfo {
    int threads, groups;
    bool nt, persist, xcd;
    int buffer, load_aux, store_aux;  // buffer: policy_kernel with the given cache policy bits
};

// The shapes: 0 is stream_probe_kernel's (the step's unit shape); 7 adds the step's XCD mapping.
constexpr ShapeInfo kShapes[] = {
    {256, 1, true, false, false, 0, 0, 0},   // 0: 1024 elements per block
    {256, 2, true, false, false, 0, 0, 0},   // 1: 2048 per block, two groups 1024 apart
    {256, 4, true, false, false, 0, 0, 0},   // 2: 4096 per block, four groups 1024 apart
    {1024, 1, true, false, false, 0, 0, 0},  // 3: 4096 per block of 1024 threads
    {64, 1, true, false, false, 0, 0, 0},    // 4: 256 per block of one wave
    {256, 1, true, true, false, 0, 0, 0},    // 5: 1024-element pieces, 8 blocks per CU striding over them
    {256, 1, false, false, false, 0, 0, 0},  // 6: shape 0 with plain loads and stores
    {256, 1, true, false, true, 0, 0, 0},    // 7: shape 0, XCD-contiguous (the step's mapping)
    {64, 1, true, false, true, 0, 0, 0},     // 8: shape 4, XCD-contiguous
    {128, 1, true, false, false, 0, 0, 0},   // 9: 512 per block of two waves
    {128, 1, true, false, true, 0, 0, 0},    // 10: shape 9, XCD-contiguous
    {64, 2, true, false, true, 0, 0, 0},     // 11: 512 per block of one wave, XCD-contiguous
    {256, 1, true, false, true, 1, 2, 2},    // 12: shape 7 as buffer accesses: loads nt, stores nt
    {256, 1, true, false, true, 1, 18, 18},  // 13: loads nt sc1, stores nt sc1
    {256, 1, true, false, true, 1, 3, 19},   // 14: loads sc0 nt, stores sc0 nt sc1
    {256, 1, true, false, true, 1, 2, 0},    // 15: loads nt, stores default
    {256, 1, false, false, true, 1, 0, 2},   // 16: loads default, stores nt
    {256, 1, true, false, true, 1, 2, 17},   // 17: loads nt, stores sc0 sc1
};
constexpr int kNumShapes = (int)(sizeof(kShapes) / sizeof(kShapes[0]));

uint64_t shape_pieces(const ShapeInfo &si, uint64_t n) {
    const uint64_t per = (uint64_t)si.threads * 4u * si.groups;
    return (n + per - 1) / per;
}

// Blocks of a shape's grid before a persistent grid's cap.
uint64_t shape_blocks(const ShapeInfo &si, uint64_t n) {
    const uint64_t pieces = shape_pieces(si, n);
    return si.xcd ? (pieces + 7u) / 8u * 8u : pieces;
}

template <int P, int S, int NS, int SH>
hipError_t launch_shape(void *p, const void *g, void *m, void *v, uint64_t n, hipStream_t stream) {
    constexpr ShapeInfo si = kShapes[SH];
    const uint64_t pieces = shape_pieces(si, n);
    uint64_t blocks = shape_blocks(si, n);
    if constexpr (si.buffer) {
        policy_kernel<P, S, NS, si.load_aux, si.store_aux><<<(uint32_t)blocks, kThreads, 0, stream>>>(p, g, m, v, n,
                                                                                                     pieces);
        return hipGetLastError();
    }
    if (si.persist) {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return hipErrorUnknown;
        blocks = std::min<uint64_t>(pieces, (uint64_t)cus * 8u);
    }
    shape_kernel<P, S, NS, si.threads, si.groups, si.nt, si.persist, si.xcd>
        <<<(uint32_t)blocks, si.threads, 0, stream>>>(p, g, m, v, n, pieces);
    return hipGetLastError();
}

template <int P, int S, int NS>
hipError_t launch_shape_of(int shape, void *p, const void *g, void *m, void *v, uint64_t n, hipStream_t stream) {
    switch (shape) {
    case 0: return launch_shape<P, S, NS, 0>(p, g, m, v, n, stream);
    case 1: return launch_shape<P, S, NS, 1>(p, g, m, v, n, stream);
    case 2: return launch_shape<P, S, NS, 2>(p, g, m, v, n, stream);
    case 3: return launch_shape<P, S, NS, 3>(p, g, m, v, n, stream);
    case 4: return launch_shape<P, S, NS, 4>(p, g, m, v, n, stream);
    case 5: return launch_shape<P, S, NS, 5>(p, g, m, v, n, stream);
    case 6: return launch_shape<P, S, NS, 6>(p, g, m, v, n, stream);
    case 7: return launch_shape<P, S, NS, 7>(p, g, m, v, n, stream);
    case 8: return launch_shape<P, S, NS, 8>(p, g, m, v, n, stream);
    case 9: return launch_shape<P, S, NS, 9>(p, g, m, v, n, stream);
    case 10: return launch_shape<P, S, NS, 10>(p, g, m, v, n, stream);
    case 11: return launch_shape<P, S, NS, 11>(p, g, m, v, n, stream);
    case 12: return launch_shape<P, S, NS, 12>(p, g, m, v, n, stream);
    case 13: return launch_shape<P, S, NS, 13>(p, g, m, v, n, stream);
    case 14: return launch_shape<P, S, NS, 14>(p, g, m, v, n, stream);
    case 15: return launch_shape<P, S, NS, 15>(p, g, m, v, n, stream);
    case 16: return launch_shape<P, S, NS, 16>(p, g, m, v, n, stream);
    default: return launch_shape<P, S, NS, 17>(p, g, m, v, n, stream);
    }
}

}  // namespace

// One pass over n elements. param_bytes (p and g) and state_bytes (m, and v when nstate == 2) are
// 2 or 4; n must be a positive multiple of 4 with at most 2^24 - 1 blocks of 1024; every pointer
// 16-byte aligned (v may be NULL when nstate == 1). Returns 0, 1 for invalid arguments, 2 when the
// launch fails. Asynchronous on `stream` (a hipStream_t, NULL for the default stream).
extern "C" int lv_stream_probe(int param_bytes, int state_bytes, int nstate, void *p, const void *g, void *m,
                               void *v, uint64_t n, void *stream) {
    if ((param_bytes != 2 && param_bytes != 4) || (state_bytes != 2 && state_bytes != 4)) return 1;
    if (nstate != 1 && nstate != 2) return 1;
    if (!p || !g || !m || (nstate == 2 && !v)) return 1;
    if (n == 0 || n % 4u != 0) return 1;
    const uint64_t blocks = (n + kUnit - 1) / kUnit;
    if (blocks >= (1ull << 24)) return 1;  // blocks * 256 threads stays below 2^32
    const uintptr_t al = (uintptr_t)p | (uintptr_t)g | (uintptr_t)m | (nstate == 2 ? (uintptr_t)v : 0u);
    if (al & 15u) return 1;
    const uint32_t b = (uint32_t)blocks;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int key = (param_bytes == 4 ? 4 : 0) | (state_bytes == 4 ? 2 : 0) | (nstate == 2 ? 1 : 0);
    hipError_t rc;
    switch (key) {
    case 0: rc = launch<2, 2, 1>(p, g, m, v, n, b, st); break;
    case 1: rc = launch<2, 2, 2>(p, g, m, v, n, b, st); break;
    case 2: rc = launch<2, 4, 1>(p, g, m, v, n, b, st); break;
    case 3: rc = launch<2, 4, 2>(p, g, m, v, n, b, st); break;
    case 4: rc = launch<4, 2, 1>(p, g, m, v, n, b, st); break;
    case 5: rc = launch<4, 2, 2>(p, g, m, v, n, b, st); break;
    case 6: rc = launch<4, 4, 1>(p, g, m, v, n, b, st); break;
    default: rc = launch<4, 4, 2>(p, g, m, v, n, b, st); break;
    }
    return rc == hipSuccess ? 0 : 2;
}

// Number of shapes lv_stream_probe_shape takes (0 .. count - 1).
extern "C" int lv_stream_probe_shapes(void) { return kNumShapes; }

// Threads per block, 4-element groups per thread, non-temporal (1/0), persistent (1/0),
// XCD-contiguous (1/0), buffer accesses (1/0) and, for those, the load and store cache policy bits
// (bit 0 sc0, bit 1 nt, bit 4 sc1) of a shape, into out[8]. Returns 0, or 1 for an unknown shape or
// a NULL out.
extern "C" int lv_stream_probe_shape_info(int shape, int *out) {
    if (shape < 0 || shape >= kNumShapes || !out) return 1;
    out[0] = kShapes[shape].threads;
    out[1] = kShapes[shape].groups;
    out[2] = kShapes[shape].nt ? 1 : 0;
    out[3] = kShapes[shape].persist ? 1 : 0;
    out[4] = kShapes[shape].xcd ? 1 : 0;
    out[5] = kShapes[shape].buffer;
    out[6] = kShapes[shape].load_aux;
    out[7] = kShapes[shape].store_aux;
    return 0;
}

// lv_stream_probe in one of the shapes above (the same arguments and checks, the same outputs).
extern "C" int lv_stream_probe_shape(int shape, int param_bytes, int state_bytes, int nstate, void *p, const void *g,
                                     void *m, void *v, uint64_t n, void *stream) {
    if (shape < 0 || shape >= kNumShapes) return 1;
    if ((param_bytes != 2 && param_bytes != 4) || (state_bytes != 2 && state_bytes != 4)) return 1;
    if (nstate != 1 && nstate != 2) return 1;
    if (!p || !g || !m || (nstate == 2 && !v)) return 1;
    if (n == 0 || n % 4u != 0) return 1;
    if ((n + kUnit - 1) / kUnit >= (1ull << 24)) return 1;  // lv_stream_probe's limit
    if (shape_blocks(kShapes[shape], n) * (uint64_t)kShapes[shape].threads >= (1ull << 32)) return 1;
    const uintptr_t al = (uintptr_t)p | (uintptr_t)g | (uintptr_t)m | (nstate == 2 ? (uintptr_t)v : 0u);
    if (al & 15u) return 1;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int key = (param_bytes == 4 ? 4 : 0) | (state_bytes == 4 ? 2 : 0) | (nstate == 2 ? 1 : 0);
    hipError_t rc;
    switch (key) {
    case 0: rc = launch_shape_of<2, 2, 1>(shape, p, g, m, v, n, st); break;
    case 1: rc = launch_shape_of<2, 2, 2>(shape, p, g, m, v, n, st); break;
    case 2: rc = launch_shape_of<2, 4, 1>(shape, p, g, m, v, n, st); break;
    case 3: rc = launch_shape_of<2, 4, 2>(shape, p, g, m, v, n, st); break;
    case 4: rc = launch_shape_of<4, 2, 1>(shape, p, g, m, v, n, st); break;
    case 5: rc = launch_shape_of<4, 2, 2>(shape, p, g, m, v, n, st); break;
    case 6: rc = launch_shape_of<4, 4, 1>(shape, p, g, m, v, n, st); break;
    default: rc = launch_shape_of<4, 4, 2>(shape, p, g, m, v, n, st); break;
    }
    return rc == hipSuccess ? 0 : 2;
}
