// MI355X (gfx950) LuminaV optimizer step: host side and C ABI (include/luminav_hip.h). The device
// side (layouts, exact arithmetic, kernels) is lv_device.h; the kernels of each buffer mode are
// instantiated in their own object (lv_kernels.hip).
//
// One multi-tensor launch (pair) per (pass, step, dtype) class of tensors: up to 48 descriptors
// in the kernel arguments (inline launch), or any number from a descriptor table in device memory
// (table launch: the library keeps a small ring of tables per device and launches with no upload
// when the table is unchanged). Each tensor is cut into work units of 1024 elements (2048 with
// 16-bit state); every block of a unit launch updates exactly one unit and exits. A thread moves 4
// consecutive elements of each 1024-element half with vector loads/stores (16 bytes for f32, 8 for
// 16-bit types); a tensor's last, partial unit keeps that layout and only the one 4-element group
// straddling its end goes element by element; tensors whose pointers are not 16-byte aligned go
// element by element. The cautious mask is counted exactly: each block reports its integer count
// and its completion in one atomic on one of the tensor's spread u64 slot words; the block that
// completes the tensor holds the exact total and finalises the 6-float scratch on the device, so a
// steady step is one launch and needs no host synchronisation.
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
#include <cstddef>
#include <cstring>
#include <mutex>
#include <new>
#include <thread>
#include <vector>

#include "luminav_hip.h"
#include "lv_device.h"

namespace lv {

// ------------------------------------------------------------------ host side

static KernelFn pick_kernel(int mode, int pt, int st, int pass, uint32_t flags, bool table) {
    switch (mode) {
    case LV_BUFFER_TDCLM: return pick_kernel_tdclm(pt, st, pass, flags, table);
    case LV_BUFFER_DUAL: return pick_kernel_clm(pt, st, pass, flags, table);
    case LV_BUFFER_T1: return pick_kernel_t1(pt, st, pass, flags, table);
    default: return pick_kernel_t2(pt, st, pass, flags, table);
    }
}

static KernelFn pick_fold(int mode, int pass) {
    switch (mode) {
    case LV_BUFFER_TDCLM: return pick_fold_tdclm(pass);
    case LV_BUFFER_DUAL: return pick_fold_clm(pass);
    case LV_BUFFER_T1: return pick_fold_t1(pass);
    default: return pick_fold_t2(pass);
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

// f32-state unit launches of at most this many blocks map block b to unit b (launch()).
constexpr uint32_t kIdentityMapUnits = 1u << 21;

// XCDs of the current device (hipDeviceAttributeNumberOfXccs; 1 if unknown).
static uint32_t device_xcds() {
    static std::mutex mu;
    static uint32_t cache[64] = {0};  // per device; 0 = not queried yet (no allocation here)
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    std::lock_guard<std::mutex> lk(mu);
    if (cache[dev]) return cache[dev];
    int x = 0;
    if (hipDeviceGetAttribute(&x, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || x < 1 || x > 64) x = 1;
    cache[dev] = (uint32_t)x;
    return (uint32_t)x;
}

struct Item {
    int idx;   // position in the caller's array
    int pass;  // first pass of this tensor
    int pt, gt, st;
    bool master;
    uint64_t step;
};

// Launch classes: identical (pass, step, dtypes, master); within a class the caller's order.
static bool item_less(const Item &x, const Item &y) {
    if (x.pass != y.pass) return x.pass < y.pass;
    if (x.step != y.step) return x.step < y.step;
    if (x.pt != y.pt) return x.pt < y.pt;
    if (x.gt != y.gt) return x.gt < y.gt;
    if (x.st != y.st) return x.st < y.st;
    if (x.master != y.master) return x.master < y.master;
    return x.idx < y.idx;
}

static bool same_class(const Item &x, const Item &y) {
    return x.pass == y.pass && x.step == y.step && x.pt == y.pt && x.gt == y.gt && x.st == y.st && x.master == y.master;
}

static int launch_one(KernelFn fn, const Args &args, uint32_t grid, uint32_t threads, hipStream_t stream) {
    void *kargs[] = {const_cast<Args *>(&args)};
    hipError_t e = hipLaunchKernel(reinterpret_cast<const void *>(fn), dim3(grid), dim3(threads), kargs, 0, stream);
    if (e != hipSuccess) return fail(LV_STATUS_EXECUTION_FAILED, "kernel launch failed: %s", hipGetErrorString(e));
    return LV_STATUS_SUCCESS;
}

static uint64_t units_of(uint64_t n, uint32_t unit_elems) { return (n + unit_elems - 1) / unit_elems; }

// Count slots a tensor of `units` work units takes in a table launch: its count slots and its fold
// slot.
static uint64_t table_slots_of(uint64_t units) {
    return (uint64_t)table_count_slots(units > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)units) + 1;
}

static int dtype_bytes(int dt) { return dt == LV_DTYPE_F32 ? 4 : 2; }

// ------------------------------------------------------------------ pointer aliasing

// One buffer of one tensor of a call: [b, e) in bytes.
struct Span {
    uintptr_t b, e;
    int item;  // position in the caller's array
    int kind;  // 0 param, 1 exp_avg, 2 exp_avg_sq, 3 master_param, 4 scratch
};

// step_pyo3's anti-aliasing rules (optimizer/src/python_ffi/mod.rs:131-173), with the reference's
// messages: an item's grad must not be its param or exp_avg; no param, exp_avg, exp_avg_sq,
// master_param (other than an fp32 param's own pointer) or scratch pointer may appear twice in a
// call; no grad may equal any of them. The reference compares start pointers only; a launch runs
// every tensor of a class concurrently, so buffers that merely overlap would race as well: they
// are rejected too. `spans` has room for 5 entries per item.
static int check_aliasing(const lv_tensor *T, const Item *items, int nitems, Span *spans) {
    for (int k = 0; k < nitems; k++) {
        const lv_tensor &t = T[items[k].idx];
        if (t.grad == t.param || t.grad == t.exp_avg)
            return fail(LV_STATUS_INVALID_CONFIG,
                        "Pointer aliasing detected: grad_ptr 0x%llx aliases mutable state at param index %llu.",
                        (unsigned long long)(uintptr_t)t.grad, (unsigned long long)t.param_index);
    }
    int ns = 0;
    for (int k = 0; k < nitems; k++) {
        const int i = items[k].idx;
        const lv_tensor &t = T[i];
        const uint64_t n = t.numel;
        const uintptr_t p = (uintptr_t)t.param, m = (uintptr_t)t.exp_avg;
        spans[ns++] = {p, p + n * (uint64_t)dtype_bytes(t.param_dtype), i, 0};
        spans[ns++] = {m, m + n * (uint64_t)dtype_bytes(t.state_dtype), i, 1};
        if (t.exp_avg_sq) {
            const uintptr_t v = (uintptr_t)t.exp_avg_sq;
            spans[ns++] = {v, v + n * (uint64_t)dtype_bytes(t.state_dtype), i, 2};
        }
        if (t.master_param && (void *)t.master_param != t.param) {
            const uintptr_t mp = (uintptr_t)t.master_param;
            spans[ns++] = {mp, mp + n * 4u, i, 3};
        }
        const uintptr_t s = (uintptr_t)t.scratch;
        spans[ns++] = {s, s + 6u * sizeof(float), i, 4};
    }
    std::sort(spans, spans + ns, [](const Span &x, const Span &y) {
        if (x.b != y.b) return x.b < y.b;
        return x.item != y.item ? x.item < y.item : x.kind < y.kind;
    });
    uintptr_t reach = 0;  // end of the furthest-reaching span so far
    int reach_k = -1;
    for (int k = 0; k < ns; k++) {
        const Span &s = spans[k];
        if (k > 0 && s.b == spans[k - 1].b) {
            const char *what = s.kind == 2 ? "mutable exp_avg_sq pointer" : s.kind == 3 ? "mutable master_param pointer"
                                                                                        : "mutable pointer";
            return fail(LV_STATUS_INVALID_CONFIG,
                        "Pointer aliasing detected in step_pyo3: %s 0x%llx is referenced multiple times.", what,
                        (unsigned long long)s.b);
        }
        if (reach_k >= 0 && s.b < reach) {
            const Span &o = spans[reach_k];
            return fail(LV_STATUS_INVALID_CONFIG,
                        "Pointer aliasing detected: mutable buffers of param index %llu (0x%llx) and param index %llu "
                        "(0x%llx) overlap.",
                        (unsigned long long)T[o.item].param_index, (unsigned long long)o.b,
                        (unsigned long long)T[s.item].param_index, (unsigned long long)s.b);
        }
        if (s.e > reach) {
            reach = s.e;
            reach_k = k;
        }
    }
    // The mutable spans are now sorted and disjoint: each grad is checked by a binary search.
    for (int k = 0; k < nitems; k++) {
        const lv_tensor &t = T[items[k].idx];
        const uintptr_t gb = (uintptr_t)t.grad, ge = gb + t.numel * (uint64_t)dtype_bytes(t.grad_dtype);
        int lo = 0, hi = ns;  // first span starting at or after ge
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (spans[mid].b < ge) lo = mid + 1;
            else hi = mid;
        }
        if (lo > 0 && spans[lo - 1].e > gb)
            return fail(LV_STATUS_INVALID_CONFIG,
                        "Pointer aliasing detected: grad_ptr 0x%llx aliases mutable state at param index %llu.",
                        (unsigned long long)gb, (unsigned long long)t.param_index);
    }
    return LV_STATUS_SUCCESS;
}

// ------------------------------------------------------------------ workspace layout

// A call's workspace, every region a multiple of 256 bytes:
//   [inline count slots: kMaxDesc x kSlotWords slots of 64 B][radial tickets: 512 B]
//   [radial running sums: kMaxDesc records][radial chunk records: one per kFoldChunk units + kMaxDesc]
//   [table count slots: the call's table launches][radial unit records: 16 B + 4 B per unit]
// The caller zero-fills it once; every call leaves all of it zero again (the kernels re-zero the
// count slots and tickets, the radial fold zeroes every record it reads), so calls with different
// layouts can share one workspace.
constexpr size_t kSlotBytes = (size_t)kMaxDesc * kSlotWords * kSlotStride * sizeof(unsigned long long);
constexpr size_t kTicketBytes = 512;
constexpr size_t kRunBytes = (size_t)kMaxDesc * sizeof(RadialSum);
static_assert(kSlotBytes % 256 == 0 && kRunBytes % 256 == 0, "region alignment");
static_assert(kMaxDesc * sizeof(unsigned long long) <= kTicketBytes, "ticket region");
static_assert(sizeof(RadialSum) == 32, "radial record layout");

constexpr size_t round256(size_t x) { return (x + 255) & ~(size_t)255; }

struct Layout {
    unsigned long long *slots = nullptr;   // inline count slots
    unsigned long long *tslots = nullptr;  // table count slots
    unsigned long long *tickets = nullptr;
    RadialSum *run = nullptr, *chunks = nullptr;
    double *unit_sq = nullptr;
    uint32_t *unit_cnt = nullptr;
    uint64_t table_slots = 0;    // table count slots available (0: no table launches)
    uint32_t radial_units = 0;   // unit records available: the largest radial launch piece
    bool radial_split = true;    // a radial launch above radial_units runs in pieces (else: refused)
};

constexpr size_t chunk_bytes(uint32_t radial_units) {
    return radial_units ? round256(((size_t)(radial_units + kFoldChunk - 1) / kFoldChunk + kMaxDesc) * sizeof(RadialSum))
                        : 0;
}

constexpr size_t layout_bytes(uint64_t table_slots, uint32_t radial_units) {
    return kSlotBytes + kTicketBytes + kRunBytes + chunk_bytes(radial_units) +
           round256(table_slots * kSlotStride * sizeof(unsigned long long)) + (size_t)radial_units * 16u +
           round256((size_t)radial_units * 4u);
}

static Layout make_layout(char *ws, uint64_t table_slots, uint32_t radial_units) {
    Layout L;
    size_t off = 0;
    L.slots = reinterpret_cast<unsigned long long *>(ws + off);
    off += kSlotBytes;
    L.tickets = reinterpret_cast<unsigned long long *>(ws + off);
    off += kTicketBytes;
    L.run = reinterpret_cast<RadialSum *>(ws + off);
    off += kRunBytes;
    L.chunks = reinterpret_cast<RadialSum *>(ws + off);
    off += chunk_bytes(radial_units);
    L.tslots = reinterpret_cast<unsigned long long *>(ws + off);
    off += round256(table_slots * kSlotStride * sizeof(unsigned long long));
    L.unit_sq = reinterpret_cast<double *>(ws + off);
    off += (size_t)radial_units * 16u;
    L.unit_cnt = reinterpret_cast<uint32_t *>(ws + off);
    L.table_slots = table_slots;
    L.radial_units = radial_units;
    return L;
}

// What a call needs, from its tensors alone (an upper bound over every class the call forms):
// table count slots when more than kMaxDesc tensors step, and radial unit records up to one piece
// when the config uses the radial bound. Units are counted at the smallest unit size of table and
// radial launches, 1024 elements (the one-wave blocks of unit_threads are inline launches only).
static void call_needs(const lv_config *cfg, const lv_tensor *T, int count, uint64_t &table_slots, uint32_t &radial_units) {
    table_slots = 0;
    radial_units = 0;
    if (!cfg || !T || count <= 0) return;
    const bool radial = cfg->bound && cfg->bound_ratio > 0.0f && cfg->bound_type == LV_BOUND_RADIAL;
    uint64_t units = 0, slots = 0;
    int active = 0;
    for (int i = 0; i < count; i++) {
        if (T[i].numel == 0) continue;
        active++;
        const uint64_t u = units_of(T[i].numel, kHalf);
        units += u;
        slots += table_slots_of(u);
    }
    if (active > kMaxDesc && !radial) table_slots = slots;
    if (radial) radial_units = (uint32_t)std::min<uint64_t>(units, kRadialPiece);
}

// ------------------------------------------------------------------ descriptor tables

// Table launches read their descriptors from device tables owned by the library: a ring of
// kRingSlots per device, each with a pinned host mirror of the bytes it last uploaded. A call
// whose table equals a slot's bytes launches from that slot with no upload; otherwise the least
// recently used slot is rewritten after the launches that last read it have finished (its event),
// and the new table is uploaded on the caller's stream. A slot is leased to one call from
// acquisition until its launches are enqueued and its event recorded; a call on another stream
// that reuses a slot first waits for the slot's earlier readers, so the event always covers
// every reader. A call on the null stream that reuses the slot the previous null-stream call
// left (the steady step of a many-tensor group) records no event: the slot is marked `pending`,
// and whoever next needs the event records it on the null stream first, which covers every
// reader enqueued there (the null stream cannot be destroyed, so that record is always valid).
// That spares one hipEventRecord of host time per step.
constexpr int kRingSlots = 4;

struct TableSlot {
    TDesc *dev = nullptr;
    TDesc *host = nullptr;
    size_t cap = 0;   // descriptors each buffer holds
    size_t len = 0;   // descriptors of the table last uploaded (0: none)
    hipEvent_t ev = nullptr;
    hipStream_t last = nullptr;
    bool used = false;     // ev has been recorded
    bool pending = false;  // readers enqueued on the null stream (last) after ev was recorded
    bool busy = false;
    uint64_t stamp = 0;
};

struct TableRing {
    int dev = 0;
    TableSlot slot[kRingSlots];
    uint64_t clock = 0;
};

static std::mutex g_ring_mu;
static std::vector<TableRing *> g_rings;  // one per device, kept until the process ends

struct TableLease {
    TableSlot *s = nullptr;
    bool uploaded = false;
};

// Records a leased slot's deferred event on the null stream (see above); false on failure.
static bool record_pending(TableSlot &s) {
    if (hipEventRecord(s.ev, nullptr) != hipSuccess) return false;
    s.pending = false;
    return true;
}

static int acquire_table(const TDesc *want, size_t n, hipStream_t stream, TableLease &lease) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(LV_STATUS_NO_DRIVER, "no HIP device");
    std::unique_lock<std::mutex> lk(g_ring_mu);
    TableRing *R = nullptr;
    for (TableRing *r : g_rings)
        if (r->dev == dev) R = r;
    if (!R) {
        R = new TableRing();
        R->dev = dev;
        g_rings.push_back(R);
    }
    for (;;) {
        for (TableSlot &s : R->slot) {
            if (s.busy || s.len != n || std::memcmp(s.host, want, n * sizeof(TDesc)) != 0) continue;
            s.busy = true;
            s.stamp = ++R->clock;
            lk.unlock();
            lease.s = &s;
            lease.uploaded = false;
            if (s.used && s.last != stream &&
                ((s.pending && !record_pending(s)) || hipStreamWaitEvent(stream, s.ev, 0) != hipSuccess)) {
                lk.lock();
                s.busy = false;
                return fail(LV_STATUS_EXECUTION_FAILED, "descriptor table wait failed");
            }
            return LV_STATUS_SUCCESS;
        }
        TableSlot *pick = nullptr;
        for (TableSlot &s : R->slot)
            if (!s.busy && (!pick || s.stamp < pick->stamp)) pick = &s;
        if (pick) {
            pick->busy = true;
            pick->stamp = ++R->clock;
            lease.s = pick;
            break;
        }
        lk.unlock();  // every slot leased by other threads' calls
        std::this_thread::yield();
        lk.lock();
    }
    lk.unlock();
    TableSlot &s = *lease.s;
    auto give_back = [&](int rc) {
        std::lock_guard<std::mutex> g(g_ring_mu);
        s.busy = false;
        lease.s = nullptr;
        return rc;
    };
    if (!s.ev && hipEventCreateWithFlags(&s.ev, hipEventDisableTiming) != hipSuccess)
        return give_back(fail(LV_STATUS_EXECUTION_FAILED, "event creation failed"));
    if (s.used && ((s.pending && !record_pending(s)) || hipEventSynchronize(s.ev) != hipSuccess))
        return give_back(fail(LV_STATUS_EXECUTION_FAILED, "descriptor table event wait failed"));
    s.len = 0;
    if (s.cap < n) {
        // the slot's readers and its last upload have finished (its event): both buffers are free
        if (s.dev) (void)hipFree(s.dev);
        if (s.host) (void)hipHostFree(s.host);
        s.dev = nullptr;
        s.host = nullptr;
        s.cap = 0;
        const size_t cap = std::max<size_t>(n + n / 2, 64);
        void *d = nullptr, *h = nullptr;
        if (hipMalloc(&d, cap * sizeof(TDesc)) != hipSuccess)
            return give_back(fail(LV_STATUS_EXECUTION_FAILED, "descriptor table allocation failed"));
        if (hipHostMalloc(&h, cap * sizeof(TDesc), hipHostMallocDefault) != hipSuccess) {
            (void)hipFree(d);
            return give_back(fail(LV_STATUS_EXECUTION_FAILED, "pinned descriptor staging allocation failed"));
        }
        s.dev = static_cast<TDesc *>(d);
        s.host = static_cast<TDesc *>(h);
        s.cap = cap;
    }
    std::memcpy(s.host, want, n * sizeof(TDesc));
    if (hipMemcpyAsync(s.dev, s.host, n * sizeof(TDesc), hipMemcpyHostToDevice, stream) != hipSuccess)
        return give_back(fail(LV_STATUS_EXECUTION_FAILED, "descriptor upload failed"));
    s.len = n;
    lease.uploaded = true;
    return LV_STATUS_SUCCESS;
}

// Ends a lease after the launches that read the slot were enqueued on `stream` (or failed).
static int release_table(TableLease &lease, hipStream_t stream) {
    if (!lease.s) return LV_STATUS_SUCCESS;
    TableSlot &s = *lease.s;
    if (stream == nullptr && !lease.uploaded && s.used && s.last == nullptr) {
        // a reuse on the null stream after null-stream readers: defer the record
        std::lock_guard<std::mutex> g(g_ring_mu);
        s.pending = true;
        s.busy = false;
        lease.s = nullptr;
        return LV_STATUS_SUCCESS;
    }
    const bool ok = hipEventRecord(s.ev, stream) == hipSuccess;
    std::lock_guard<std::mutex> g(g_ring_mu);
    if (ok) {
        s.used = true;
        s.pending = false;
        s.last = stream;
    } else {
        s.len = 0;  // nothing certain covers this slot's readers: never reuse its bytes
        (void)hipStreamSynchronize(stream);
    }
    s.busy = false;
    lease.s = nullptr;
    return ok ? LV_STATUS_SUCCESS : fail(LV_STATUS_EXECUTION_FAILED, "descriptor table event record failed");
}

// ------------------------------------------------------------------ workspace ordering

// Calls that share a workspace share its count slots and radial records, so each must start after
// the previous one has finished. Calls on one stream are ordered by the stream; a call on another
// stream first waits for an event that follows the previous call. The library keeps one such
// record per workspace address (a handful per process; kept until it ends). A call on a non-null
// stream records its event right after its launches. A call on the null stream records none: the
// next call from another stream records it on the null stream first, which covers everything
// enqueued there (the null stream cannot be destroyed, so that late record is always valid), so
// the steady step on the null stream pays no event. The reference gives every parameter scratch
// of its own for the same reason (changelogs/LUMINAV_ALGORITHM_CHANGELOG.md:281-283).
struct WsOrder {
    const void *ws = nullptr;
    hipEvent_t ev = nullptr;
    hipStream_t last = nullptr;
    bool called = false;   // a call has used the workspace
    bool recorded = false;  // ev follows the last call (else: the last call was on the null stream)
};

static std::mutex g_order_mu;
static std::vector<WsOrder *> g_orders;

// Makes `stream` wait for the previous call on workspace `ws` when that call ran on another
// stream. Returns the workspace's record (locked by the caller's sequencing: one host thread per
// workspace at a time, as the header requires).
static int order_before(const void *ws, hipStream_t stream, WsOrder *&out) {
    WsOrder *o = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_order_mu);
        for (WsOrder *x : g_orders)
            if (x->ws == ws) o = x;
        if (!o) {
            o = new (std::nothrow) WsOrder();
            if (!o) return fail(LV_STATUS_EXECUTION_FAILED, "workspace order record allocation failed");
            o->ws = ws;
            g_orders.push_back(o);
        }
    }
    out = o;
    if (!o->called || o->last == stream) return LV_STATUS_SUCCESS;
    if (!o->ev && hipEventCreateWithFlags(&o->ev, hipEventDisableTiming) != hipSuccess)
        return fail(LV_STATUS_EXECUTION_FAILED, "event creation failed");
    if (!o->recorded) {  // the previous call ran on the null stream
        if (hipEventRecord(o->ev, nullptr) != hipSuccess) return fail(LV_STATUS_EXECUTION_FAILED, "event record failed");
        o->recorded = true;
    }
    if (hipStreamWaitEvent(stream, o->ev, 0) != hipSuccess)
        return fail(LV_STATUS_EXECUTION_FAILED, "stream wait on the previous workspace user failed");
    return LV_STATUS_SUCCESS;
}

// After a call's launches on `stream` were enqueued.
static int order_after(WsOrder *o, hipStream_t stream) {
    o->called = true;
    o->last = stream;
    o->recorded = false;
    if (stream == nullptr) return LV_STATUS_SUCCESS;  // recorded late, if another stream needs it
    if (!o->ev && hipEventCreateWithFlags(&o->ev, hipEventDisableTiming) != hipSuccess)
        return fail(LV_STATUS_EXECUTION_FAILED, "event creation failed");
    if (hipEventRecord(o->ev, stream) != hipSuccess) return fail(LV_STATUS_EXECUTION_FAILED, "event record failed");
    o->recorded = true;
    return LV_STATUS_SUCCESS;
}

// ------------------------------------------------------------------ launches

// Unit launches of one class over args.total_units units, in pieces of at most kMaxGrid blocks
// (kMaxGridIdentity when block b maps to unit b)
// (`radial_piece` for radial counting launches, the unit records of one piece; LV_MAX_GRID_BLOCKS
// lowers the cap, so tests can split small launches). A counting launch folds its counts in its
// last blocks; a radial one runs fold_kernel after every piece.
static int launch(Args &args, int mode, int pt, int st, int pass, hipStream_t stream, bool table, uint32_t radial_piece) {
    KernelFn fn = pick_kernel(mode, pt, st, pass, args.flags, table);
    const bool radial = (pass == kFused || pass == kCount) && (args.flags & kFRadial);
    if (table && radial) return fail(LV_STATUS_INVALID_CONFIG, "radial counting launches are inline");
    if (args.total_units == 0) return LV_STATUS_SUCCESS;
    // The block mapping. XCD-contiguous (each XCD streams one contiguous eighth of the units) is
    // the default. f32-state launches of one-wave blocks, and of up to kIdentityMapUnits 256-thread
    // blocks, map block b to unit b instead (xcds = 1). Against the XCD-contiguous mapping, in one
    // process on the same buffers: 256-thread f32-state launches ran 0.5-3.3% faster (cfg2's
    // 64-tensor table launch, cfg3, cfg4, and T2 buckets of 2.5e8-2e9 elements) and larger ones
    // 1.2-2.9% slower (T1 at 4e9, T2 at 3.5e9-6.7e9 elements); one-wave T2 blocks ran 3-4% faster
    // at 1e9 and 3.5e9 elements and 2% faster at 6.7e9; 16-bit-state launches ran level to 4.6%
    // slower. Results are the same either way: units are independent and the count is exact in
    // any order.
    const bool identity_map = st == LV_DTYPE_F32 && !radial &&
                              (lv::unit_threads(mode, pt, st, pass, args.flags, table) < kThreads ||
                               args.total_units <= kIdentityMapUnits);
    args.xcds = identity_map ? 1u : device_xcds();
    // b / X == (b * recip) >> 40 for b < 2^23 = kMaxGrid and X <= 64: recip exceeds 2^40 / X by at
    // most 1, so the product exceeds b * 2^40 / X by less than b < 2^23, i.e. by < 2^-17 after the
    // shift, while the fraction of b / X is at most 1 - 1/X <= 1 - 2^-6.
    // With X = 1 (identity-mapped launches) the kernel takes unit = base + b and skips this
    // product, which would overflow 64 bits from b = 2^24 (recip = 2^40 + 1).
    static_assert(kMaxGrid <= (1u << 23), "the reciprocal is exact for grids up to 2^23 blocks");
    static_assert(kRadialPiece <= kMaxGrid, "a radial piece is one unit launch");
    args.xcd_recip = ((uint64_t)1 << 40) / args.xcds + 1;
    // identity-mapped launches are of one-wave blocks or of at most kIdentityMapUnits blocks
    static_assert((uint64_t)kMaxGridIdentity * 64 < (1ull << 32) && kIdentityMapUnits <= kMaxGrid, "grid x threads < 2^32");
    uint32_t max_grid = radial ? radial_piece : (identity_map ? kMaxGridIdentity : kMaxGrid);
    if (const char *e = std::getenv("LV_MAX_GRID_BLOCKS")) {
        long v = std::atol(e);
        if (v > 0 && (uint32_t)v < max_grid) max_grid = (uint32_t)v;
    }
    if (max_grid == 0) return fail(LV_STATUS_INVALID_CONFIG, "no radial unit records in the workspace");
    KernelFn fold = radial ? pick_fold(mode, pass) : nullptr;
    for (uint32_t ub = 0; ub < args.total_units; ub += std::min<uint32_t>(max_grid, args.total_units - ub)) {
        const uint32_t grid = std::min<uint32_t>(max_grid, args.total_units - ub);
        args.unit_base = ub;
        args.piece_units = grid;
        args.xcd_q = grid / args.xcds;
        args.xcd_r = grid % args.xcds;
        int rc = launch_one(fn, args, grid, lv::unit_threads(mode, pt, st, pass, args.flags, table), stream);
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

// Where a tensor's vector layout starts: the smallest h < 64 at which every stream the kernel moves
// (param, grad, exp_avg, exp_avg_sq in the two-buffer modes, the master copy) starts a 128-byte
// line, or failing that the smallest h < 8 at which every stream is 16-byte aligned (the vector
// accesses' own alignment). A view that starts k elements past a line in all of its buffers (a
// slice of a bucket, a shard) so keeps whole-line accesses per wave: with only 16-byte alignment
// every wave instruction straddles one more line and the non-temporal stores write partial lines
// (a +1-element T2 view ran 6% slower than the aligned one). Buffers that disagree, or a tensor
// of at most h elements, get no vector layout and go element by element.
static bool head_for(const lv_tensor &T, const Item &it, bool dual, uint32_t align, uint32_t limit, uint32_t &head) {
    struct Stream {
        uintptr_t addr;
        int bytes;
    } st[5];
    int ns = 0;
    st[ns++] = {(uintptr_t)T.param, dtype_bytes(it.pt)};
    st[ns++] = {(uintptr_t)T.grad, dtype_bytes(it.gt)};
    st[ns++] = {(uintptr_t)T.exp_avg, dtype_bytes(it.st)};
    if (dual) st[ns++] = {(uintptr_t)T.exp_avg_sq, dtype_bytes(it.st)};
    if (it.master) st[ns++] = {(uintptr_t)T.master_param, 4};
    head = 0;
    for (uint32_t h = 0; h < limit; h++) {
        bool ok = true;
        for (int k = 0; k < ns && ok; k++)
            ok = ((st[k].addr + (uintptr_t)h * (uintptr_t)st[k].bytes) & (uintptr_t)(align - 1u)) == 0;
        if (ok) {
            if ((uint64_t)h >= T.numel) return false;
            head = h;
            return true;
        }
    }
    return false;
}

// For kernels of one-wave blocks (units of kMinUnitElems elements): the smallest h < kMinUnitElems
// at which every stream starts a whole unit of its own element size, that is at an element index
// (address / element size) that is a multiple of kMinUnitElems, so each block moves the same
// whole 512-byte (16-bit) and 1 KiB (f32) pieces of its streams as in an aligned tensor. A view
// at +k elements of aligned buffers has h = 256 - k. Against the 128-byte-line head, a 2^27-element
// T2 view at +1, +33 and +63 elements ran 1.033-1.037x the aligned view in one-wave blocks.
static bool unit_head(const lv_tensor &T, const Item &it, bool dual, uint32_t &head) {
    struct Stream {
        uintptr_t addr;
        int bytes;
    } st[5];
    int ns = 0;
    st[ns++] = {(uintptr_t)T.param, dtype_bytes(it.pt)};
    st[ns++] = {(uintptr_t)T.grad, dtype_bytes(it.gt)};
    st[ns++] = {(uintptr_t)T.exp_avg, dtype_bytes(it.st)};
    if (dual) st[ns++] = {(uintptr_t)T.exp_avg_sq, dtype_bytes(it.st)};
    if (it.master) st[ns++] = {(uintptr_t)T.master_param, 4};
    uint64_t e = 0;
    for (int k = 0; k < ns; k++) {
        if (st[k].addr % (uintptr_t)st[k].bytes) return false;
        const uint64_t ek = (uint64_t)(st[k].addr / (uintptr_t)st[k].bytes) % kMinUnitElems;
        if (k && ek != e) return false;
        e = ek;
    }
    head = (uint32_t)((kMinUnitElems - e) % kMinUnitElems);
    return (uint64_t)head < T.numel;
}

static bool vector_head(const lv_tensor &T, const Item &it, bool dual, uint32_t unit_elems, uint32_t &head) {
    if (unit_elems == kMinUnitElems && unit_head(T, it, dual, head)) return true;
    return head_for(T, it, dual, 128u, 64u, head) || head_for(T, it, dual, 16u, 8u, head);
}

static void fill_desc(Desc &D, const lv_tensor &T, const Item &it, bool dual, uint32_t unit_elems) {
    D.p = T.param;
    D.g = T.grad;
    D.m = T.exp_avg;
    D.v = T.exp_avg_sq;
    D.mp = it.master ? T.master_param : nullptr;
    D.scratch = T.scratch;
    D.n = T.numel;
    D.unit_begin = 0;
    D.pidx = (uint32_t)T.param_index;
    D.ibase = (uint32_t)T.index_base;
    D.nskip = (uint32_t)T.n_inactive;  // < 2^24 (prepare_call)
    uint32_t head = 0;
    D.vec = vector_head(T, it, dual, unit_elems, head) ? 1u : 0u;
    D.head = head;
    D.skip = T.n_inactive ? T.inactive : nullptr;
}

// Work units of a tensor: they start at its vector head, so an unaligned view may have one fewer
// than an aligned tensor of the same size (never more: call_needs counts from element 0).
static uint64_t desc_units(const Desc &D, uint32_t unit_elems) {
    return units_of(D.n - (D.vec ? D.head : 0u), unit_elems);
}

static void fill_args_common(Args &args, const lv_config *cfg, const Item &h, int bound) {
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
    args.bound_floor = cfg->bound_ratio >= 0x1p-40f ? 1u : 0u;
    // facts the kernels' stochastic roundings rely on (kRangeM, kRangeP): false for NaNs
    if (std::fabs(args.b1) <= 0x1p64f && std::fabs(args.omb1) <= 0x1p64f) args.ranges |= kRangeM;
    if (args.bound_floor && std::fabs(args.neg_lr_wd) <= 0x1p32f) args.ranges |= kRangeP;
    StepCoeffs sc = step_coeffs(h.step, cfg->beta1, cfg->beta2, cfg->eps, cfg->tau, cfg->lam);
    args.c1 = sc.c1;
    args.c2 = sc.c2;
    args.c_sigma = sc.c_sigma;
    args.ema = cfg->ema_decay;
    args.ema_c = 1.0f - cfg->ema_decay;
    args.clamp_min = cfg->cautious_clamp_min;
    args.seed_base = step_seed_base(cfg->seed, h.step);
    uint32_t flags = 0;
    if (cfg->cautious) flags |= kFCautious;
    if (cfg->stochastic_rounding) flags |= kFSR;
    if (h.master) flags |= kFMaster;
    if (cfg->weight_decay != 0.0f) flags |= kFWeightDecay;
    // v <= 65000 for fp16 params only: the FFI worker hands the core an fp16 *state* container as
    // bitwise bf16 (worker.rs:107-113, 141-150), so the core's fp16-state test (dual.rs:68) never
    // fires on that path.
    if (h.pt == LV_DTYPE_F16) flags |= kFClampV;
    if (bound == LV_BOUND_COORDINATE) flags |= kFCoordinate;
    if (bound == LV_BOUND_RADIAL) flags |= kFRadial;
    flags |= (uint32_t)h.gt << 8;
    args.flags = flags;
}

// The launches of one class (or of one inline group of at most kMaxDesc tensors of it).
static int launch_class(Args &args, const lv_config *cfg, const Item &h, hipStream_t stream, bool table,
                        uint32_t radial_piece) {
    if (h.pass == kCount) {
        int rc = launch(args, cfg->buffer, h.pt, h.st, kCount, stream, table, radial_piece);
        if (rc != LV_STATUS_SUCCESS) return rc;
        return launch(args, cfg->buffer, h.pt, h.st, kApply, stream, table, radial_piece);
    }
    return launch(args, cfg->buffer, h.pt, h.st, h.pass, stream, table, radial_piece);
}

// An item's step count and first pass: dual.rs:52, dual.rs:122, dual.rs:260; tdclm.rs:67-68.
static void set_step(Item &it, const lv_config *cfg, int bound, uint64_t step) {
    it.step = step;
    if (!cfg->cautious && bound != LV_BOUND_RADIAL) it.pass = kSingle;
    else if (cfg->fused_single_pass && step > 1) it.pass = kFused;
    else it.pass = kCount;
}

// Validates a call and forms its items (tensors with elements), in the caller's order.
// `items` has room for `count` entries and `spans` for 5 per entry.
static int prepare_call(const lv_config *cfg, const lv_tensor *tensors, int count, Item *items, int &nitems,
                        Span *spans) {
    nitems = 0;
    const bool dual = cfg->buffer == LV_BUFFER_DUAL || cfg->buffer == LV_BUFFER_T2;
    const int bound = (cfg->bound && cfg->bound_ratio > 0.0f) ? cfg->bound_type : LV_BOUND_NONE;  // config.rs:368-375
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
        if (T.numel > (uint64_t)0xFFFFFFFFull * kMinUnitElems)
            return fail(LV_STATUS_INVALID_CONFIG, "tensor %d: too many elements", i);
        // worker.rs:95-98 and worker.rs:153-156: an fp32 param aliasing its master has none.
        const bool mp_present = T.master_param && !(T.param_dtype == LV_DTYPE_F32 && (void *)T.master_param == T.param);
        const bool master = cfg->master_weights != 0 && mp_present;
        if (cfg->master_weights != 0 && !mp_present && T.param_dtype != LV_DTYPE_F32)
            return fail(LV_STATUS_NULL_POINTER, "tensor %d: Master weight mode requires an initialized master_param buffer", i);
        if (T.n_inactive && !T.inactive) return fail(LV_STATUS_NULL_POINTER, "tensor %d: inactive ranges pointer is NULL", i);
        if (T.n_inactive > 0xFFFFFFull)
            return fail(LV_STATUS_INVALID_CONFIG, "tensor %d: too many inactive ranges (at most 2^24 - 1)", i);
        Item it;
        it.idx = i;
        it.pt = T.param_dtype;
        it.gt = T.grad_dtype;
        it.st = T.state_dtype == LV_DTYPE_F32 ? LV_DTYPE_F32 : LV_DTYPE_BF16;  // fp16 state -> bf16 bits (worker.rs:107-113)
        it.master = master;
        set_step(it, cfg, bound, T.step);
        items[nitems++] = it;
    }
    return check_aliasing(tensors, items, nitems, spans);
}

// Launches every class of a prepared call. `items` is sorted here. Classes run one launch (pair)
// each: a table launch when more than kMaxDesc tensors share a class and the layout has table
// slots (radial counting classes stay inline: their fold walks the launch's tensor list), else
// inline launches of up to kMaxDesc tensors.
static int run_call(const lv_config *cfg, const lv_tensor *tensors, Item *items, int nitems, const Layout &L,
                    hipStream_t stream, std::vector<TDesc> *tab_buf, const lv_step_record *rec = nullptr) {
    const int bound = (cfg->bound && cfg->bound_ratio > 0.0f) ? cfg->bound_type : LV_BOUND_NONE;
    const bool dual = cfg->buffer == LV_BUFFER_DUAL || cfg->buffer == LV_BUFFER_T2;
    std::sort(items, items + nitems, item_less);
    for (int begin = 0; begin < nitems;) {
        const Item &h = items[begin];
        int cls_end = begin + 1;
        while (cls_end < nitems && same_class(items[cls_end], h)) cls_end++;
        const bool radial = bound == LV_BOUND_RADIAL && h.pass != kSingle;
        const bool table = !radial && L.table_slots > 0 && tab_buf && cls_end - begin > kMaxDesc;
        if (table) {
            const int n = cls_end - begin;
            Args args;
            fill_args_common(args, cfg, h, bound);
            args.step_rec = rec;
            const uint32_t unit_elems = lv::unit_elems(cfg->buffer, h.pt, h.st, h.pass, args.flags, true);
            std::vector<TDesc> &tab = *tab_buf;
            if (tab.size() < (size_t)n) tab.resize((size_t)n);
            uint64_t units = 0, slot = 0;
            for (int k = 0; k < n; k++) {
                const lv_tensor &T = tensors[items[begin + k].idx];
                TDesc &E = tab[(size_t)k];
                std::memset(&E, 0, sizeof E);
                fill_desc(E.d, T, items[begin + k], dual, unit_elems);
                const uint64_t u = desc_units(E.d, unit_elems);
                E.d.unit_begin = (uint32_t)units;
                units += u;
                if (units > 0xFFFFFFFFull) return fail(LV_STATUS_INVALID_CONFIG, "too many work units in one launch");
                E.unit_end = (uint32_t)units;
                E.slot_base = (uint32_t)slot;
                slot += table_slots_of(u);
            }
            if (slot > L.table_slots)
                return fail(LV_STATUS_INVALID_CONFIG, "workspace too small: %llu table count slots needed, %llu present",
                            (unsigned long long)slot, (unsigned long long)L.table_slots);
            args.ndesc = n;
            args.total_units = (uint32_t)units;
            args.group = (uint32_t)((n + kTableHeads - 1) / kTableHeads);
            args.nheads = (uint32_t)((n + args.group - 1) / args.group);
            for (uint32_t hd = 0; hd < args.nheads; hd++) args.ubegin[hd] = tab[(size_t)hd * args.group].d.unit_begin;
            args.slots = L.tslots;
            args.tickets = L.tickets;
            TableLease lease;
            int rc = acquire_table(tab.data(), (size_t)n, stream, lease);
            if (rc != LV_STATUS_SUCCESS) return rc;
            args.dtab = lease.s->dev;
            rc = launch_class(args, cfg, h, stream, true, 0);
            const int rr = release_table(lease, stream);
            if (rc != LV_STATUS_SUCCESS) return rc;
            if (rr != LV_STATUS_SUCCESS) return rr;
            begin = cls_end;
            continue;
        }
        while (begin < cls_end) {
            const int end = begin + std::min(cls_end - begin, kMaxDesc);
            Args args;
            fill_args_common(args, cfg, h, bound);
            args.step_rec = rec;
            const uint32_t unit_elems = lv::unit_elems(cfg->buffer, h.pt, h.st, h.pass, args.flags, false);
            args.ndesc = end - begin;
            uint64_t units = 0;
            for (int k = begin; k < end; k++) {
                Desc &D = args.d[k - begin];
                const lv_tensor &T = tensors[items[k].idx];
                fill_desc(D, T, items[k], dual, unit_elems);
                D.unit_begin = (uint32_t)units;
                units += desc_units(D, unit_elems);
                if (units > 0xFFFFFFFFull) return fail(LV_STATUS_INVALID_CONFIG, "too many work units in one launch");
            }
            args.total_units = (uint32_t)units;
            if (radial && units > L.radial_units && !L.radial_split)
                return fail(LV_STATUS_INVALID_CONFIG,
                            "radial launch of %llu work units exceeds the %u unit records of this entry point",
                            (unsigned long long)units, L.radial_units);
            args.slots = L.slots;
            args.tickets = L.tickets;
            args.run = L.run;
            args.chunks = L.chunks;
            args.unit_sq = L.unit_sq;
            args.unit_cnt = L.unit_cnt;
            const int rc = launch_class(args, cfg, h, stream, false, L.radial_units);
            if (rc != LV_STATUS_SUCCESS) return rc;
            begin = end;
        }
    }
    return LV_STATUS_SUCCESS;
}

// lv_step_multi's host scratch, one per thread, grown on demand and reused (no allocation per
// call in the steady state), and the last call it validated: a call whose config and tensors
// (every field but the step counters, which only set the passes) are byte for byte those of that
// call takes its items without validating again. Validation depends on nothing else.
struct CallScratch {
    std::vector<Item> items;
    std::vector<Span> spans;
    std::vector<TDesc> tab;
    std::vector<lv_tensor> last;  // step fields zeroed
    std::vector<Item> last_items;
    lv_config last_cfg;
    int last_nitems = -1;

    static bool same_but_step(const lv_tensor &a, const lv_tensor &b) {
        constexpr size_t s0 = offsetof(lv_tensor, step), s1 = s0 + sizeof(uint64_t);
        const char *x = reinterpret_cast<const char *>(&a), *y = reinterpret_cast<const char *>(&b);
        return std::memcmp(x, y, s0) == 0 && std::memcmp(x + s1, y + s1, sizeof(lv_tensor) - s1) == 0;
    }

    bool same_as_last(const lv_config *cfg, const lv_tensor *t, int count) const {
        if (last_nitems < 0 || last.size() != (size_t)count || std::memcmp(&last_cfg, cfg, sizeof *cfg) != 0) return false;
        for (int i = 0; i < count; i++)
            if (!same_but_step(last[(size_t)i], t[i])) return false;
        return true;
    }

    void remember(const lv_config *cfg, const lv_tensor *t, int count, int nitems) {
        last.assign(t, t + count);
        for (lv_tensor &x : last) x.step = 0;
        last_items.assign(items.begin(), items.begin() + nitems);
        last_cfg = *cfg;
        last_nitems = nitems;
    }
};
static thread_local CallScratch t_call;
static_assert(sizeof(lv_config) == 18 * 4, "lv_config has no padding (compared with memcmp)");
static_assert(sizeof(lv_tensor) == 112, "lv_tensor layout (compared with memcmp)");

// The configuration luminav_triton_step_f32 builds from its arguments (c_api.rs:143-176).
static void f32_config(lv_config &c, float lr, float beta1, float beta2, float eps, float weight_decay, float tau,
                       float lam, int buffer_mode, int cautious, int bound_mode, float bound_ratio, bool master,
                       uint32_t seed) {
    c.lr = lr;
    c.beta1 = beta1;
    c.beta2 = beta2;
    c.eps = eps;
    c.weight_decay = weight_decay;
    c.tau = tau;
    c.lam = lam;
    c.cautious_clamp_min = 0.5f;
    c.bound_ratio = bound_ratio;
    c.buffer = buffer_mode == LV_BUFFER_TDCLM ? LV_BUFFER_TDCLM : LV_BUFFER_DUAL;
    c.ema_decay = c.buffer == LV_BUFFER_TDCLM ? 0.95f : 0.80f;  // BufferMode::default_ema_decay
    c.cautious = cautious != 0;
    c.stochastic_rounding = 0;
    c.bound = bound_mode > 0;
    c.bound_type = bound_mode == LV_BOUND_RADIAL ? LV_BOUND_RADIAL
                   : bound_mode == LV_BOUND_COORDINATE ? LV_BOUND_COORDINATE : LV_BOUND_NONE;
    c.master_weights = master ? 2 : 0;
    c.fused_single_pass = 1;
    c.seed = seed;
}

// Per-device zero-filled workspaces of lv_step_f32 and the engines, grown on demand.
struct OwnedWorkspace {
    void *p = nullptr;
    size_t bytes = 0;
};

// A single-tensor fp32 step with luminav_triton_step_f32's argument mapping on device pointers.
// Every failure other than a null pointer is LV_STATUS_EXECUTION_FAILED, as there (c_api.rs:178-181).
static int step_f32_device(OwnedWorkspace &ws, float *param, const float *grad, float *exp_avg, float *exp_avg_sq,
                           float *master_param, float *scratch, size_t n, float lr, float beta1, float beta2, float eps,
                           float weight_decay, float tau, float lam, int buffer_mode, int cautious, int bound_mode,
                           float bound_ratio, uint64_t step, uint32_t seed, hipStream_t stream) {
    if (!param || !grad || !exp_avg || !scratch) return fail(LV_STATUS_NULL_POINTER, "null param/grad/exp_avg/scratch pointer");
    lv_config c;
    f32_config(c, lr, beta1, beta2, eps, weight_decay, tau, lam, buffer_mode, cautious, bound_mode, bound_ratio,
               master_param != nullptr, seed);
    if (validate_config(&c) != LV_STATUS_SUCCESS) return LV_STATUS_EXECUTION_FAILED;  // message already set
    if (n == 0) return LV_STATUS_SUCCESS;
    float *v = buffer_mode == LV_BUFFER_DUAL ? exp_avg_sq : nullptr;  // c_api.rs:120-124
    if (c.buffer == LV_BUFFER_DUAL && !v)
        return fail(LV_STATUS_EXECUTION_FAILED, "Dual-buffer mode requires an initialized exp_avg_sq buffer");
    lv_tensor t;
    std::memset(&t, 0, sizeof t);
    t.param = param;
    t.grad = grad;
    t.exp_avg = exp_avg;
    t.exp_avg_sq = v;
    t.master_param = master_param;
    t.scratch = scratch;
    t.numel = n;
    t.step = step;
    t.param_dtype = t.grad_dtype = t.state_dtype = LV_DTYPE_F32;
    uint64_t tslots;
    uint32_t runits;
    call_needs(&c, &t, 1, tslots, runits);
    const size_t need = layout_bytes(tslots, runits);
    if (ws.bytes < need) {
        if (ws.p) {
            if (hipStreamSynchronize(stream) != hipSuccess || hipFree(ws.p) != hipSuccess)
                return fail(LV_STATUS_EXECUTION_FAILED, "workspace release failed");
            ws.p = nullptr;
            ws.bytes = 0;
        }
        void *p = nullptr;
        if (hipMalloc(&p, need) != hipSuccess) return fail(LV_STATUS_EXECUTION_FAILED, "hipMalloc failed");
        if (hipMemset(p, 0, need) != hipSuccess) {
            (void)hipFree(p);
            return fail(LV_STATUS_EXECUTION_FAILED, "hipMemset failed");
        }
        ws.p = p;
        ws.bytes = need;
    }
    Item it;
    Span spans[5];
    int nitems = 0;
    int rc = prepare_call(&c, &t, 1, &it, nitems, spans);
    if (rc == LV_STATUS_SUCCESS && nitems) {
        Layout L = make_layout(static_cast<char *>(ws.p), tslots, runits);
        WsOrder *order = nullptr;
        rc = order_before(ws.p, stream, order);
        if (rc == LV_STATUS_SUCCESS) {
            rc = run_call(&c, &t, &it, nitems, L, stream, nullptr);
            const int ro = order_after(order, stream);
            if (rc == LV_STATUS_SUCCESS) rc = ro;
        }
        if (rc == LV_STATUS_EXECUTION_FAILED) {
            // a launch failed part-way: its count words may hold partial counts; start clean
            if (hipStreamSynchronize(stream) == hipSuccess) (void)hipMemset(ws.p, 0, ws.bytes);
        }
    }
    return rc == LV_STATUS_SUCCESS || rc == LV_STATUS_NULL_POINTER ? rc : LV_STATUS_EXECUTION_FAILED;
}

// ------------------------------------------------------------------ no-allocation entry point

// lv_step_multi_noalloc's workspace: inline count slots for 48 tensors per launch and radial
// records for launches of up to kNoAllocRadialUnits units (one piece, so its radial sums follow
// the same summation tree as lv_step_multi's). No table slots: classes above 48 tensors run as
// several inline launches, which give the same bits. One copy per device, zero at load; every
// call leaves it zero again, and a call that failed part-way marks it for a clearing kernel
// before the next call.
constexpr uint32_t kNoAllocRadialUnits = 1u << 16;
constexpr int kNoAllocMaxTensors = 256;
constexpr size_t kNoAllocBytes = layout_bytes(0, kNoAllocRadialUnits);
static_assert(kNoAllocBytes == 1514496, "no-allocation scratch size");

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

__global__ void __launch_bounds__(kThreads) zero_fill(uint4 *p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (size_t)gridDim.x * kThreads)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// Graph launches: advances the call's step record on the device and writes that step's
// coefficients for the unit kernels that follow on the stream (one thread). A call whose passes
// assume a lagged scale (need_two: cautious or radial with the fused single pass) refuses a first
// step: status 1, counter unchanged, and the unit kernels then change nothing.
__global__ void __launch_bounds__(64) step_record_kernel(lv_step_record *r, float b1, float b2, float eps, float tau,
                                                         float lam, uint32_t seed, int need_two) {
    if (threadIdx.x != 0) return;
    const uint64_t s = r->step + 1;
    if (need_two && s < 2) {
        r->status = 1u;
        return;
    }
    const StepCoeffs k = step_coeffs(s, b1, b2, eps, tau, lam);
    r->step = s;
    r->c1 = k.c1;
    r->c2 = k.c2;
    r->c_sigma = k.c_sigma;
    r->seed_base = step_seed_base(seed, s);
    r->status = 0u;
}

struct NoAllocScratch {
    std::mutex mu;
    void *ptr[64] = {nullptr};  // `scratch` on each device (hipGetSymbolAddress)
    bool dirty[64] = {false};   // a call failed part-way: clear before the next one
};
static NoAllocScratch g_noalloc;

}  // namespace lv

// The reference's standalone engine handle (luminav_triton_standalone.h:21-22): a device, a stream
// and device staging for the host buffers of luminav_triton_step_f32.
struct LuminaVTritonEngine {
    int device = 0;
    hipStream_t stream = nullptr;
    char arch[64] = {0};
    void *buf = nullptr;  // device copies of param, grad, exp_avg, exp_avg_sq, master_param, scratch
    size_t buf_bytes = 0;
    lv::OwnedWorkspace ws;
    std::mutex mu;
};

// ====================================================================== C ABI

extern "C" {

int lv_version(void) { return 400; }

size_t lv_workspace_bytes(int n_tensors) {
    // any call with n_tensors tensors: every tensor with kSlots count slots in a table launch, and
    // one full radial piece
    const uint64_t tslots = n_tensors > lv::kMaxDesc ? (uint64_t)n_tensors * lv::kSlotWords : 0;
    return lv::layout_bytes(tslots, lv::kRadialPiece);
}

size_t lv_workspace_bytes_for(const lv_config *cfg, const lv_tensor *tensors, int count) {
    uint64_t tslots;
    uint32_t runits;
    lv::call_needs(cfg, tensors, count, tslots, runits);
    return lv::layout_bytes(tslots, runits);
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
    if (!workspace) return fail(LV_STATUS_NULL_POINTER, "workspace is NULL");
    if (((uintptr_t)workspace & 255u) != 0) return fail(LV_STATUS_INVALID_CONFIG, "workspace must be 256-byte aligned");
    uint64_t tslots;
    uint32_t runits;
    call_needs(cfg, tensors, count, tslots, runits);
    const size_t need = layout_bytes(tslots, runits);
    if (workspace_bytes < need)
        return fail(LV_STATUS_INVALID_CONFIG, "workspace too small: %zu < %zu (lv_workspace_bytes_for)", workspace_bytes,
                    need);
    CallScratch &cs = t_call;
    if (cs.items.size() < (size_t)count) cs.items.resize((size_t)count);
    int nitems = 0;
    if (cs.same_as_last(cfg, tensors, count)) {
        // validated before: the items again, with this call's step counters
        const int bound = (cfg->bound && cfg->bound_ratio > 0.0f) ? cfg->bound_type : LV_BOUND_NONE;
        nitems = cs.last_nitems;
        for (int k = 0; k < nitems; k++) {
            cs.items[(size_t)k] = cs.last_items[(size_t)k];
            set_step(cs.items[(size_t)k], cfg, bound, tensors[cs.items[(size_t)k].idx].step);
        }
    } else {
        if (cs.spans.size() < (size_t)count * 5) cs.spans.resize((size_t)count * 5);
        rc = prepare_call(cfg, tensors, count, cs.items.data(), nitems, cs.spans.data());
        if (rc != LV_STATUS_SUCCESS) {
            cs.last_nitems = -1;
            return rc;
        }
        cs.remember(cfg, tensors, count, nitems);
    }
    if (nitems == 0) return LV_STATUS_SUCCESS;
    const Layout L = make_layout(static_cast<char *>(workspace), tslots, runits);
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    WsOrder *order = nullptr;
    rc = order_before(workspace, stream, order);
    if (rc != LV_STATUS_SUCCESS) return rc;
    rc = run_call(cfg, tensors, cs.items.data(), nitems, L, stream, &cs.tab);
    const int ro = order_after(order, stream);
    return rc != LV_STATUS_SUCCESS ? rc : ro;
}

int lv_step_multi_noalloc(const lv_config *cfg, const lv_tensor *tensors, int count, void *stream_ptr) {
    using namespace lv;
    g_err[0] = 0;
    if (!cfg) return fail(LV_STATUS_NULL_POINTER, "config is NULL");
    if (count < 0) return fail(LV_STATUS_INVALID_CONFIG, "negative tensor count");
    if (count == 0) return LV_STATUS_SUCCESS;
    if (!tensors) return fail(LV_STATUS_NULL_POINTER, "tensor list is NULL");
    if (count > kNoAllocMaxTensors)
        return fail(LV_STATUS_INVALID_CONFIG, "%d tensors exceed the %d of lv_step_multi_noalloc (use lv_step_multi)",
                    count, kNoAllocMaxTensors);
    int rc = validate_config(cfg);
    if (rc != LV_STATUS_SUCCESS) return rc;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(LV_STATUS_NO_DRIVER, "no HIP device");
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    char *ws = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_noalloc.mu);
        if (!g_noalloc.ptr[dev]) {
            void *p = nullptr;
            // with this device current: its own copy of the array
            if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p)
                return fail(LV_STATUS_EXECUTION_FAILED, "cannot resolve the no-allocation scratch on device %d", dev);
            g_noalloc.ptr[dev] = p;
        }
        ws = static_cast<char *>(g_noalloc.ptr[dev]);
        if (g_noalloc.dirty[dev]) {
            hipLaunchKernelGGL(zero_fill, dim3(64), dim3(kThreads), 0, stream, reinterpret_cast<uint4 *>(ws),
                               kNoAllocBytes / sizeof(uint4));
            if (hipGetLastError() != hipSuccess) return fail(LV_STATUS_EXECUTION_FAILED, "scratch clearing failed");
            g_noalloc.dirty[dev] = false;
        }
    }
    Item items[kNoAllocMaxTensors];
    Span spans[kNoAllocMaxTensors * 5];
    int nitems = 0;
    rc = prepare_call(cfg, tensors, count, items, nitems, spans);
    if (rc != LV_STATUS_SUCCESS || nitems == 0) return rc;
    Layout L = make_layout(ws, 0, kNoAllocRadialUnits);
    L.radial_split = false;
    rc = run_call(cfg, tensors, items, nitems, L, stream, nullptr);
    if (rc == LV_STATUS_EXECUTION_FAILED) {
        std::lock_guard<std::mutex> lk(g_noalloc.mu);
        g_noalloc.dirty[dev] = true;
    }
    return rc;
}

int lv_step_multi_graph(const lv_config *cfg, const lv_tensor *tensors, int count, lv_step_record *record,
                        void *workspace, size_t workspace_bytes, void *stream_ptr) {
    using namespace lv;
    g_err[0] = 0;
    if (!cfg) return fail(LV_STATUS_NULL_POINTER, "config is NULL");
    if (!record) return fail(LV_STATUS_NULL_POINTER, "step record is NULL");
    if (count < 0) return fail(LV_STATUS_INVALID_CONFIG, "negative tensor count");
    if (count == 0) return LV_STATUS_SUCCESS;
    if (!tensors) return fail(LV_STATUS_NULL_POINTER, "tensor list is NULL");
    int rc = validate_config(cfg);
    if (rc != LV_STATUS_SUCCESS) return rc;
    if (!workspace) return fail(LV_STATUS_NULL_POINTER, "workspace is NULL");
    if (((uintptr_t)workspace & 255u) != 0) return fail(LV_STATUS_INVALID_CONFIG, "workspace must be 256-byte aligned");
    if (((uintptr_t)record & 7u) != 0) return fail(LV_STATUS_INVALID_CONFIG, "step record must be 8-byte aligned");
    uint64_t tslots;
    uint32_t runits;
    call_needs(cfg, tensors, count, tslots, runits);
    const size_t need = layout_bytes(0, runits);  // inline launches only
    if (workspace_bytes < need)
        return fail(LV_STATUS_INVALID_CONFIG, "workspace too small: %zu < %zu", workspace_bytes, need);
    CallScratch &cs = t_call;
    if (cs.items.size() < (size_t)count) cs.items.resize((size_t)count);
    if (cs.spans.size() < (size_t)count * 5) cs.spans.resize((size_t)count * 5);
    int nitems = 0;
    rc = prepare_call(cfg, tensors, count, cs.items.data(), nitems, cs.spans.data());
    cs.last_nitems = -1;  // items below get graph passes: not a cache entry for lv_step_multi
    if (rc != LV_STATUS_SUCCESS || nitems == 0) return rc;
    // Every step a replay takes is a later one: passes as for step >= 2, one class per dtype set.
    const int bound = (cfg->bound && cfg->bound_ratio > 0.0f) ? cfg->bound_type : LV_BOUND_NONE;
    for (int k = 0; k < nitems; k++) set_step(cs.items[(size_t)k], cfg, bound, 2);
    const bool need_two = (cfg->cautious || bound == LV_BOUND_RADIAL) && cfg->fused_single_pass;
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    hipLaunchKernelGGL(step_record_kernel, dim3(1), dim3(64), 0, stream, record, cfg->beta1, cfg->beta2, cfg->eps,
                       cfg->tau, cfg->lam, cfg->seed, need_two ? 1 : 0);
    if (hipGetLastError() != hipSuccess) return fail(LV_STATUS_EXECUTION_FAILED, "step record launch failed");
    const Layout L = make_layout(static_cast<char *>(workspace), 0, runits);
    return run_call(cfg, tensors, cs.items.data(), nitems, L, stream, nullptr, record);
}

int lv_step_f32(float *param, const float *grad, float *exp_avg, float *exp_avg_sq, float *master_param,
                float *scratch, size_t num_elements, float lr, float beta1, float beta2, float eps,
                float weight_decay, float tau, float lam, int buffer_mode, int cautious, int bound_mode,
                float bound_ratio, uint64_t step, uint32_t seed, void *stream) {
    using namespace lv;
    static std::mutex mu;
    static OwnedWorkspace ws[64];
    g_err[0] = 0;
    if (!param || !grad || !exp_avg || !scratch) return fail(LV_STATUS_NULL_POINTER, "null param/grad/exp_avg/scratch pointer");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(LV_STATUS_EXECUTION_FAILED, "no HIP device");
    std::lock_guard<std::mutex> lk(mu);
    return step_f32_device(ws[dev], param, grad, exp_avg, exp_avg_sq, master_param, scratch, num_elements, lr, beta1,
                           beta2, eps, weight_decay, tau, lam, buffer_mode, cautious, bound_mode, bound_ratio, step,
                           seed, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------------------------
// The reference's standalone C API (optimizer/include/luminav_triton_standalone.h:37-111,
// optimizer/crates/luminav-triton-aot/src/c_api.rs), same names, signatures and status codes:
// host buffers in, host buffers out, one synchronous step per call on the engine's own stream.

LuminaVTritonEngine *luminav_triton_engine_create(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) return nullptr;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return nullptr;
    LuminaVTritonEngine *e = new (std::nothrow) LuminaVTritonEngine();
    if (!e) return nullptr;
    e->device = dev;
    size_t k = 0;  // "gfx950:sramecc+:xnack-" -> "gfx950"
    while (k + 1 < sizeof e->arch && prop.gcnArchName[k] && prop.gcnArchName[k] != ':') {
        e->arch[k] = prop.gcnArchName[k];
        k++;
    }
    e->arch[k] = 0;
    if (hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess) {
        delete e;
        return nullptr;
    }
    return e;
}

void luminav_triton_engine_destroy(LuminaVTritonEngine *engine) {
    if (!engine) return;
    int prev = 0;
    const bool have_prev = hipGetDevice(&prev) == hipSuccess;
    if (hipSetDevice(engine->device) == hipSuccess) {
        (void)hipStreamSynchronize(engine->stream);
        if (engine->buf) (void)hipFree(engine->buf);
        if (engine->ws.p) (void)hipFree(engine->ws.p);
        (void)hipStreamDestroy(engine->stream);
    }
    if (have_prev) (void)hipSetDevice(prev);
    delete engine;
}

const char *luminav_triton_get_platform(const LuminaVTritonEngine *engine) { return engine ? "rocm" : "none"; }

const char *luminav_triton_get_arch(const LuminaVTritonEngine *engine) {
    return engine && engine->arch[0] ? engine->arch : "unknown";
}

int luminav_triton_step_f32(LuminaVTritonEngine *engine, float *param, const float *grad, float *exp_avg,
                            float *exp_avg_sq, float *master_param, float *scratch, size_t num_elements, float lr,
                            float beta1, float beta2, float eps, float weight_decay, float tau, float lam,
                            int buffer_mode, int cautious, int bound_mode, float bound_ratio, uint64_t step,
                            uint32_t seed) {
    using namespace lv;
    g_err[0] = 0;
    if (!engine || !param || !grad || !exp_avg || !scratch)
        return fail(LV_STATUS_NULL_POINTER, "null engine/param/grad/exp_avg/scratch pointer");
    std::lock_guard<std::mutex> lk(engine->mu);
    int prev = 0;
    const bool have_prev = hipGetDevice(&prev) == hipSuccess;
    if (hipSetDevice(engine->device) != hipSuccess) return fail(LV_STATUS_EXECUTION_FAILED, "cannot select the engine's device");
    const size_t n = num_elements;
    float *v_host = buffer_mode == LV_BUFFER_DUAL ? exp_avg_sq : nullptr;  // c_api.rs:120-124
    const size_t arr = round256(n * sizeof(float));
    const size_t bytes = arr * (3 + (v_host ? 1 : 0) + (master_param ? 1 : 0)) + 256;
    int rc = LV_STATUS_SUCCESS;
    if (engine->buf_bytes < bytes) {
        if (engine->buf) (void)hipFree(engine->buf);
        engine->buf = nullptr;
        engine->buf_bytes = 0;
        if (hipMalloc(&engine->buf, bytes) != hipSuccess) {
            engine->buf = nullptr;
            rc = fail(LV_STATUS_EXECUTION_FAILED, "device staging allocation failed");
        } else {
            engine->buf_bytes = bytes;
        }
    }
    if (rc == LV_STATUS_SUCCESS) {
        char *b = static_cast<char *>(engine->buf);
        float *dp = reinterpret_cast<float *>(b);
        float *dg = reinterpret_cast<float *>(b + arr);
        float *dm = reinterpret_cast<float *>(b + 2 * arr);
        size_t off = 3 * arr;
        float *dv = nullptr, *dmp = nullptr;
        if (v_host) { dv = reinterpret_cast<float *>(b + off); off += arr; }
        if (master_param) { dmp = reinterpret_cast<float *>(b + off); off += arr; }
        float *ds = reinterpret_cast<float *>(b + off);
        hipStream_t s = engine->stream;
        const size_t nb = n * sizeof(float);
        bool ok = hipMemcpyAsync(dp, param, nb, hipMemcpyHostToDevice, s) == hipSuccess &&
                  hipMemcpyAsync(dg, grad, nb, hipMemcpyHostToDevice, s) == hipSuccess &&
                  hipMemcpyAsync(dm, exp_avg, nb, hipMemcpyHostToDevice, s) == hipSuccess &&
                  (!dv || hipMemcpyAsync(dv, v_host, nb, hipMemcpyHostToDevice, s) == hipSuccess) &&
                  (!dmp || hipMemcpyAsync(dmp, master_param, nb, hipMemcpyHostToDevice, s) == hipSuccess) &&
                  hipMemcpyAsync(ds, scratch, 6 * sizeof(float), hipMemcpyHostToDevice, s) == hipSuccess;
        if (!ok) rc = fail(LV_STATUS_EXECUTION_FAILED, "host-to-device copy failed");
        if (rc == LV_STATUS_SUCCESS)
            rc = step_f32_device(engine->ws, dp, dg, dm, dv, dmp, ds, n, lr, beta1, beta2, eps, weight_decay, tau, lam,
                                 buffer_mode, cautious, bound_mode, bound_ratio, step, seed, s);
        if (rc == LV_STATUS_SUCCESS) {
            ok = hipMemcpyAsync(param, dp, nb, hipMemcpyDeviceToHost, s) == hipSuccess &&
                 hipMemcpyAsync(exp_avg, dm, nb, hipMemcpyDeviceToHost, s) == hipSuccess &&
                 (!dv || hipMemcpyAsync(v_host, dv, nb, hipMemcpyDeviceToHost, s) == hipSuccess) &&
                 (!dmp || hipMemcpyAsync(master_param, dmp, nb, hipMemcpyDeviceToHost, s) == hipSuccess) &&
                 hipMemcpyAsync(scratch, ds, 6 * sizeof(float), hipMemcpyDeviceToHost, s) == hipSuccess;
            if (!ok) rc = fail(LV_STATUS_EXECUTION_FAILED, "device-to-host copy failed");
        }
        if (hipStreamSynchronize(s) != hipSuccess && rc == LV_STATUS_SUCCESS)
            rc = fail(LV_STATUS_EXECUTION_FAILED, "step failed on the device");
    }
    if (have_prev) (void)hipSetDevice(prev);
    return rc;
}

}  // extern "C"
