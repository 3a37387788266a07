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
