// va_internal.hpp — shared host/device internals of libva_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/va_hip.h"
#include "va_keys.hpp"
#include "va_plan.hpp"

// ---------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------

// The GPU context: one device, one stream, a grow-only scratch arena.
// Replaces Metal4Context (device + command queue, Core/Metal4Context.swift:183-269)
// and its BufferPool (Core/BufferPool.swift:89-200).
struct va_context {
    int device = 0;
    hipStream_t stream = nullptr;
    bool owns_stream = false;
    int num_cus = 256;
    std::string last_error;
    // test/tuning overrides of the exact top-k scan (0 = automatic)
    uint64_t opt_candidate_cap = 0;
    uint64_t opt_sample_rows = 0;
    uint64_t opt_sample_rank = 0;  // VA_OPT_SAMPLE_RANK: 0 automatic, else min(value, k)
    uint32_t opt_screen = 0;  // VA_OPT_SCREEN: 0 auto, 1 off, 2 forced where it applies
    // scratch arena: partial results, counters, candidate buffers
    char* scratch = nullptr;
    size_t scratch_bytes = 0;
    // while set (the allocation-free entry point), scratch comes from this fixed device block
    // instead of the arena: reserve() checks the size and never allocates
    char* fixed_scratch = nullptr;
    size_t fixed_scratch_bytes = 0;
    // side buffer: per-call device inputs that a scan reads beside its scratch arena (PQ
    // distance tables); grow-only like the arena, so a call need not wait before returning
    char* side = nullptr;
    size_t side_bytes = 0;
    // pinned host word used to read back small counters
    uint32_t* host_word = nullptr;
    // phase profiling of the top-k scan (va_context_set_profiling): a ring of records whose
    // events are read when a record is reused or the timings are asked for, so a profiled scan
    // never waits on the host
    int profiling = 0;  // 0 off, 1 every phase, 2 the scan phase alone
    static constexpr int kScanRing = 16;
    struct ScanRecord {
        hipEvent_t ev[5] = {nullptr, nullptr, nullptr, nullptr, nullptr};
        uint32_t* dev_word = nullptr;   // device scratch of the record's counts
        uint32_t* host_word = nullptr;  // pinned: [0] overflowed rows, [1] reranked rows
        bool pending = false, sampled = false, fallback = false, has_ovf = false, has_rerank = false;
        bool light = false;  // profiling level 2: events 1 and 2 only
        va_scan_timings t{};
    } rec[kScanRing];
    int rec_next = 0, rec_last = -1;
    va_scan_timings rec_sum{};  // phase times summed over the scans folded since the last reset
    uint32_t rec_count = 0;
    va_scan_timings last_scan{};  // the scan being enqueued (static fields)
    // extra streams for independent launches that overlap (default priority); created on
    // first use, with the events that fork them from and join them back into `stream`.  Three,
    // so that with `stream` they fit HIP's default of four hardware queues per process
    // (streams beyond that share a queue and serialise).
    static constexpr int kAux = 3;
    hipStream_t aux[kAux] = {nullptr, nullptr, nullptr};
    hipEvent_t fork_ev = nullptr;
    hipEvent_t join_ev[kAux] = {nullptr, nullptr, nullptr};
};

namespace va {

// *out = the context's side buffer, grown to at least `bytes` (growth waits for the stream).
va_status side_reserve(va_context* ctx, size_t bytes, void** out);

// Records an error message on the context and returns the status.
va_status fail(va_context* ctx, va_status st, const char* fmt, ...);

// Makes ctx->aux[0 .. n) wait for the work queued so far on ctx->stream (creating every aux
// stream on first use).
va_status aux_fork(va_context* ctx, int n = va_context::kAux);
// Makes ctx->stream wait for the work queued so far on ctx->aux[0 .. n).
va_status aux_join(va_context* ctx, int n = va_context::kAux);

// Joins ctx->aux[0 .. n) into ctx->stream when it leaves scope unless join() ran first, so an
// error return between a fork and its join still orders the aux work before anything the caller
// queues next (scratch buffers the aux work writes are reused by later calls).
struct AuxJoinGuard {
    va_context* ctx;
    int n;
    bool armed = true;
    AuxJoinGuard(va_context* c, int k) : ctx(c), n(k) {}
    va_status join() {
        armed = false;
        return aux_join(ctx, n);
    }
    ~AuxJoinGuard() {
        if (armed) (void)aux_join(ctx, n);
    }
    AuxJoinGuard(const AuxJoinGuard&) = delete;
    AuxJoinGuard& operator=(const AuxJoinGuard&) = delete;
};

// Sends what the code in the scope queues on ctx->stream to another stream (an aux stream, forked
// from ctx->stream before the scope and joined after it).
struct StreamScope {
    va_context* ctx;
    hipStream_t prev;
    StreamScope(va_context* c, hipStream_t s) : ctx(c), prev(c->stream) { c->stream = s; }
    ~StreamScope() { ctx->stream = prev; }
    StreamScope(const StreamScope&) = delete;
    StreamScope& operator=(const StreamScope&) = delete;
};

// Makes `ctx->device` current for the lifetime of the guard.
struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        (void)hipGetDevice(&prev);
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        (void)hipGetDevice(&cur);
        if (prev >= 0 && cur != prev) (void)hipSetDevice(prev);
    }
};

// Bump allocator over the context's scratch arena (or its fixed block, see va_context).  Sizes
// are rounded to 256 B.  reserve() grows the arena (synchronising the stream first) before any
// carve(); with a fixed block it only checks that `total` fits.
struct Scratch {
    va_context* ctx;
    size_t off = 0;
    explicit Scratch(va_context* c) : ctx(c) {}
    static size_t round(size_t b) { return scratch_round(b); }
    va_status reserve(size_t total);
    // after the carves: they stayed within the `reserved` bytes (a planning mistake is an error,
    // not an out-of-bounds carve)
    va_status verify(size_t reserved) const {
        if (off > reserved)
            return fail(ctx, VA_ERR_HIP, "scratch carves of %zu bytes exceed the %zu reserved", off, reserved);
        return VA_OK;
    }
    template <typename T>
    T* carve(size_t count) {
        size_t b = round(count * sizeof(T));
        T* p = reinterpret_cast<T*>((ctx->fixed_scratch ? ctx->fixed_scratch : ctx->scratch) + off);
        off += b;
        return p;
    }
};

// Bytes of dense keys one launch of the exact scan may write (the threshold sample, the dense
// path, the overflow rescan): 256 MiB, or a quarter of a fixed scratch block.
size_t dense_budget(const va_context* ctx);
// whether the device-side overflow fallback's buffers for `rows` rows fit beside `need` bytes
bool fb_fits(const va_context* ctx, size_t need, uint32_t rows, uint32_t N, uint32_t k);


// Allocation-free entry point: resolves the device address of the fixed scratch block of
// `device` (called once per device, with that device current, when a context is created).
void noalloc_setup_device(int device);

}  // namespace va

#define VA_CHECK_HIP(ctx, expr)                                                                   \
    do {                                                                                          \
        hipError_t _e = (expr);                                                                   \
        if (_e != hipSuccess)                                                                     \
            return va::fail((ctx), _e == hipErrorOutOfMemory ? VA_ERR_OOM : VA_ERR_HIP, "%s: %s (%s:%d)", \
                            #expr, hipGetErrorString(_e), __FILE__, __LINE__);                    \
    } while (0)

#define VA_CHECK_LAUNCH(ctx) VA_CHECK_HIP(ctx, hipGetLastError())

#define VA_CHECK_STATUS(expr)          \
    do {                               \
        va_status _s = (expr);         \
        if (_s != VA_OK) return _s;    \
    } while (0)

#define VA_REQUIRE(ctx, cond, ...)                                     \
    do {                                                               \
        if (!(cond)) return va::fail((ctx), VA_ERR_INVALID_ARG, __VA_ARGS__); \
    } while (0)

// ---------------------------------------------------------------------------
// ordering keys shared by every top-K kernel
// ---------------------------------------------------------------------------
namespace va {

constexpr uint32_t kSentinel = 0xFFFFFFFFu;
// MI355X: 8 XCDs of 32 CUs, each with its own 4 MB L2; workgroup w is dispatched to XCD w % 8.
constexpr uint32_t kXcds = 8;

inline uint32_t ceil_div(uint64_t a, uint64_t b) { return uint32_t((a + b - 1) / b); }

// ---------------------------------------------------------------------------
// Global -> LDS direct loads (CDNA buffer loads with the lds modifier)
// ---------------------------------------------------------------------------
// A buffer resource covers [base, base + bytes); a load whose offset is at or past `bytes`
// reads nothing and returns zeros, which is how out-of-tile rows and columns are padded.
// Offsets are kept below 2^31 so kDmaSkip is always out of range.
typedef int dma_rsrc __attribute__((ext_vector_type(4)));
constexpr uint32_t kDmaSkip = 0x80000000u;
constexpr uint32_t kDmaMaxBytes = 0x7FFFFFF0u;

__device__ __forceinline__ dma_rsrc make_dma_rsrc(const void* base, uint32_t bytes) {
    const uint64_t p = reinterpret_cast<uint64_t>(base);
    dma_rsrc r;
    r[0] = __builtin_amdgcn_readfirstlane(int(uint32_t(p)));
    r[1] = __builtin_amdgcn_readfirstlane(int(uint32_t(p >> 32) & 0xFFFFu));  // stride 0
    r[2] = __builtin_amdgcn_readfirstlane(int(bytes));                        // num_records
    r[3] = 0x00020000;                                                         // gfx9 data format
    return r;
}

// One wave-wide 16-byte-per-lane load into LDS: lane i's bytes land at lds_addr + 16*i, so a
// wave fills 1 KiB of contiguous LDS per call.  lds_addr must be wave-uniform.  The load is
// invisible to the compiler's wait-count tracking: callers wait with wait_vmcnt<> themselves
// before a barrier that publishes the data.  M0 is set here and nowhere else in the kernels
// that use this (the compiler keeps nothing in M0 on gfx9 across these loops); M0 is a
// reserved register, whose clobbers the compiler does not honour, so it is not listed.
__device__ __forceinline__ void lds_dma16(const dma_rsrc& rsrc, uint32_t voff, uint32_t lds_addr) {
    // The operands are wave-uniform by contract; readfirstlane keeps them in SGPRs where the
    // compiler's divergence analysis cannot prove it (a no-op for values already in SGPRs).
    dma_rsrc r;
    r[0] = __builtin_amdgcn_readfirstlane(rsrc[0]);
    r[1] = __builtin_amdgcn_readfirstlane(rsrc[1]);
    r[2] = __builtin_amdgcn_readfirstlane(rsrc[2]);
    r[3] = __builtin_amdgcn_readfirstlane(rsrc[3]);
    const uint32_t l = __builtin_amdgcn_readfirstlane(lds_addr);
    // one wait state between the M0 write and the LDS-DMA load that reads it
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(l), "v"(voff), "s"(r)
                 : "memory");
}

// The same load with a wave-uniform byte offset soff added to every lane's address (an SGPR
// operand: no per-lane arithmetic).  Callers keep voff + soff inside each in-range lane's row
// and make out-of-range lanes fail the range check through voff alone, so the result does not
// depend on whether the check includes soff.
__device__ __forceinline__ void lds_dma16_so(const dma_rsrc& rsrc, uint32_t voff, uint32_t soff, uint32_t lds_addr) {
    dma_rsrc r;
    r[0] = __builtin_amdgcn_readfirstlane(rsrc[0]);
    r[1] = __builtin_amdgcn_readfirstlane(rsrc[1]);
    r[2] = __builtin_amdgcn_readfirstlane(rsrc[2]);
    r[3] = __builtin_amdgcn_readfirstlane(rsrc[3]);
    const uint32_t l = __builtin_amdgcn_readfirstlane(lds_addr);
    const uint32_t so = __builtin_amdgcn_readfirstlane(soff);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(l), "v"(voff), "s"(r), "s"(so)
                 : "memory");
}

// The one-dword form: lane i's 4 bytes land at lds_addr + 4*i (256 B per wave).  Used as an L2
// prefetch whose data is not needed.
__device__ __forceinline__ void lds_dma4(const dma_rsrc& rsrc, uint32_t voff, uint32_t lds_addr) {
    dma_rsrc r;
    r[0] = __builtin_amdgcn_readfirstlane(rsrc[0]);
    r[1] = __builtin_amdgcn_readfirstlane(rsrc[1]);
    r[2] = __builtin_amdgcn_readfirstlane(rsrc[2]);
    r[3] = __builtin_amdgcn_readfirstlane(rsrc[3]);
    const uint32_t l = __builtin_amdgcn_readfirstlane(lds_addr);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :
                 : "s"(l), "v"(voff), "s"(r)
                 : "memory");
}

// s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding: vmcnt in bits 3:0 and 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// LDS byte address of a pointer into __shared__ memory (low half of the flat address).
__device__ __forceinline__ uint32_t lds_addr_of(const void* p) {
    return uint32_t(reinterpret_cast<uintptr_t>(p));
}

}  // namespace va

// ---------------------------------------------------------------------------
// internal launchers shared between translation units
// ---------------------------------------------------------------------------
namespace va {

// Epilogue operations of the distance GEMM.
enum DistOp : int {
    OP_L2SQ = 0,     // |q|^2 + |x|^2 - 2 q.x  (clamped at 0)
    OP_L2 = 1,       // sqrt(OP_L2SQ)
    OP_COS_SIM = 2,  // q.x / (|q||x|), 0 below FLT_MIN, clamped to [-1, 1]
    OP_COS_DIST = 3, // 1 - OP_COS_SIM
    OP_DOT = 4,      // q.x
    OP_ABS_DOT = 5,  // |q.x|
    OP_NEG_DOT = 6,  // -q.x
};
DistOp metric_op(va_metric m);

// Output modes of the distance GEMM.
enum DistOut : int {
    OUT_VALUES = 0,  // out_f[q * ldo + n] = value
    OUT_KEYS = 1,    // out_k[q * ldo + n] = key_of_float(value)
    OUT_FILTER = 2,  // append (key, n) to the query's candidate list when key <= thr[q]
    OUT_ARGMIN = 3,  // best[q] = min over rows of (key << 32 | row id) (64-bit atomic min)
};


// A device-planned list-major launch (IVF): tiles of TQ queries x TN rows over the lists of one
// tile shape, enumerated by pre[] (the exclusive prefix over the lists of their tile counts for
// this shape; pre[C] tiles in all).  List l is probed by the queries qlist[qoff[l] .. qoff[l+1])
// (the launch's qrow) and holds the row positions roff[l] .. roff[l+1] (its sample prefix when
// sample is set).  Tile t of list l covers row block (t - pre[l]) / query blocks and query block
// (t - pre[l]) % query blocks: the query blocks of a row block are neighbouring tiles, so a long
// list probed by many queries is read from HBM about once, not once per query block.
struct ListPlan {
    const uint32_t* pre = nullptr;   // [C + 1]
    const uint32_t* qoff = nullptr;  // [C + 1]
    const uint32_t* roff = nullptr;  // [C + 1]
    uint32_t C = 0;
    uint32_t sample = 0;
    uint32_t grid = 0;  // workgroups of the persistent launch (host)
};
#ifdef __HIPCC__
__device__ inline void plan_tile(const ListPlan& p, uint32_t t, uint32_t TQ, uint32_t TN, uint32_t& qs, uint32_t& qc,
                                 uint32_t& rs, uint32_t& rc) {
    uint32_t lo = 0, hi = p.C - 1;  // the last list l with pre[l] <= t
    while (lo < hi) {
        const uint32_t mid = (lo + hi + 1) >> 1;
        if (p.pre[mid] <= t) lo = mid;
        else hi = mid - 1;
    }
    const uint32_t l = lo, local = t - p.pre[lo];
    const uint32_t nq = p.qoff[l + 1] - p.qoff[l];
    const uint32_t len = p.roff[l + 1] - p.roff[l];
    const uint32_t n = p.sample ? ivf_sample_rows(len) : len;
    const uint32_t nqb = (nq + TQ - 1) / TQ;
    const uint32_t rb = local / nqb, qb = local % nqb;
    qs = p.qoff[l] + qb * TQ;
    qc = min(TQ, nq - qb * TQ);
    rs = p.roff[l] + rb * TN;
    rc = min(TN, n - rb * TN);
}
// plan_tile for a tile t at or after one of list h (pre[h] <= t): the list is found by galloping
// up from h (one load while t stays in h's list, as a persistent workgroup's tiles of a long list
// do) instead of a binary search over all lists.  Returns the list.
__device__ inline uint32_t plan_tile_after(const ListPlan& p, uint32_t t, uint32_t h, uint32_t TQ, uint32_t TN,
                                           uint32_t& qs, uint32_t& qc, uint32_t& rs, uint32_t& rc) {
    uint32_t lo = h, hi = h + 1, step = 1;  // pre[lo] <= t; find hi with pre[hi] > t (or hi = C)
    while (hi < p.C && p.pre[hi] <= t) {
        lo = hi;
        step *= 2;
        hi = min(p.C, lo + step);
    }
    hi -= 1;  // the answer lies in [lo, hi]
    while (lo < hi) {
        const uint32_t mid = (lo + hi + 1) >> 1;
        if (p.pre[mid] <= t) lo = mid;
        else hi = mid - 1;
    }
    const uint32_t l = lo, local = t - p.pre[lo];
    const uint32_t nq = p.qoff[l + 1] - p.qoff[l];
    const uint32_t len = p.roff[l + 1] - p.roff[l];
    const uint32_t n = p.sample ? ivf_sample_rows(len) : len;
    const uint32_t nqb = (nq + TQ - 1) / TQ;
    const uint32_t rb = local / nqb, qb = local % nqb;
    qs = p.qoff[l] + qb * TQ;
    qc = min(TQ, nq - qb * TQ);
    rs = p.roff[l] + rb * TN;
    rc = min(TN, n - rb * TN);
    return l;
}
// plan_tile_after with the list found by the whole wave: lane i tests list base + 1 + i, so a
// tile within 64 lists of the last one found costs one load round instead of a gallop's and a
// binary search's several dependent loads (a persistent workgroup's next tile is often tens of
// lists on, most of them without tiles in its group).  Every lane of the wave must call it with
// the same t and h (pre[h] <= t); every lane gets the same tile.
__device__ inline uint32_t plan_tile_after_wave(const ListPlan& p, uint32_t t, uint32_t h, uint32_t TQ, uint32_t TN,
                                                uint32_t& qs, uint32_t& qc, uint32_t& rs, uint32_t& rc) {
    const uint32_t lane = __lane_id();
    uint32_t base = h;  // pre[base] <= t
    for (;;) {
        const uint32_t l = base + 1u + lane;
        const bool le = l < p.C && p.pre[l] <= t;  // a prefix of the lanes (pre is non-decreasing)
        const uint32_t c = uint32_t(__popcll(__ballot(le)));
        base += c;
        if (c < 64u) break;
    }
    const uint32_t l = base, local = t - p.pre[l];
    const uint32_t nq = p.qoff[l + 1] - p.qoff[l];
    const uint32_t len = p.roff[l + 1] - p.roff[l];
    const uint32_t n = p.sample ? ivf_sample_rows(len) : len;
    const uint32_t nqb = (nq + TQ - 1) / TQ;
    const uint32_t rb = local / nqb, qb = local % nqb;
    qs = p.qoff[l] + qb * TQ;
    qc = min(TQ, nq - qb * TQ);
    rs = p.roff[l] + rb * TN;
    rc = min(TN, n - rb * TN);
    return l;
}
// plan_tile with the list found by a 64-way search of the whole wave: each round lane i tests an
// evenly spaced list of the remaining range, which shrinks 64-fold (two rounds over 4,096 lists,
// where a binary search is twelve dependent loads), from a list h with pre[h] <= t (a wave's
// previous tile's list, or 0).  Every lane of the wave must call it with the same t and h; every
// lane gets the same tile.  Returns the list.
__device__ inline uint32_t plan_tile_wave(const ListPlan& p, uint32_t t, uint32_t h, uint32_t TQ, uint32_t TN,
                                          uint32_t& qs, uint32_t& qc, uint32_t& rs, uint32_t& rc) {
    const uint32_t lane = __lane_id();
    uint32_t lo = h, hi = p.C;  // pre[lo] <= t; the answer lies in [lo, hi)
    while (hi - lo > 1) {
        const uint32_t step = (hi - lo + 63) / 64;
        const uint32_t l = lo + lane * step;
        const bool le = l < hi && p.pre[l] <= t;  // a prefix of the lanes (pre is non-decreasing); lane 0 holds
        const uint32_t c = uint32_t(__popcll(__ballot(le)));
        lo = __builtin_amdgcn_readfirstlane(lo + (c - 1) * step);
        hi = __builtin_amdgcn_readfirstlane(min(hi, lo + step));
    }
    const uint32_t l = lo, local = t - p.pre[l];
    const uint32_t nq = p.qoff[l + 1] - p.qoff[l];
    const uint32_t len = p.roff[l + 1] - p.roff[l];
    const uint32_t n = p.sample ? ivf_sample_rows(len) : len;
    const uint32_t nqb = (nq + TQ - 1) / TQ;
    const uint32_t rb = local / nqb, qb = local % nqb;
    qs = p.qoff[l] + qb * TQ;
    qc = min(TQ, nq - qb * TQ);
    rs = p.roff[l] + rb * TN;
    rc = min(TN, n - rb * TN);
    return l;
}
#endif

struct DistArgs {
    const float* q = nullptr;   // query rows
    const uint32_t* qrow = nullptr;  // optional query-row indirection (query i reads row qrow[i])
    uint64_t q_rows = 0;             // rows addressable from q when qrow is set (0 = unknown)
    int64_t ldq = 0;
    const float* x = nullptr;   // database rows
    int64_t ldx = 0;
    uint32_t Q = 0, N = 0, D = 0;
    DistOp op = OP_L2SQ;
    DistOut out = OUT_VALUES;
    float* out_f = nullptr;
    uint32_t* out_k = nullptr;
    int64_t ldo = 0;
    // filter mode
    const uint32_t* thr = nullptr;
    uint32_t* cnt = nullptr;
    uint32_t* cand_key = nullptr;
    uint32_t* cand_id = nullptr;
    uint32_t cap = 0;
    uint32_t id_base = 0;  // added to database row ids in filter mode
    // argmin mode: packed (key, row) minimum per query, initialised to ~0 by the caller
    unsigned long long* best = nullptr;
    // filter launches: the id of database row position p is ids[p] (nullptr: id_base + p)
    const uint32_t* ids = nullptr;
    // gather launches (the exact rerank of screened candidates): workgroup b takes query
    // b / gtiles and the rows gather[q * gcap + j] for j in [128 t, 128 t + 128) of its list of
    // min(gcount[q], gcap) rows, t = b % gtiles; keys go to out_k[q * ldo + j].  1x1 tiles,
    // OUT_KEYS only.
    const uint32_t* gather = nullptr;
    const uint32_t* gcount = nullptr;
    uint32_t gcap = 0;
    uint32_t gtiles = 0;
    // device-planned list-major (IVF) launches (plan.pre set): persistent over the plan's
    // tiles; query i of a tile is row qrow[qs + i]; Q / N are ignored then
    ListPlan plan;
    int wq = 0;  // waves along queries (tiles of 32*wq queries); 0 = from Q
    int wn = 0;  // waves along rows (tiles of 128*wn rows); 0 = 4/wq.  wq x wn in {1x4, 2x2, 4x1}, and
                 // for OUT_FILTER also 1x1, 2x1
};

// Tile shape of launch_dist for a given wq: queries and database rows per workgroup.
inline uint32_t dist_tile_queries(int wq) { return 32u * uint32_t(wq); }
inline uint32_t dist_tile_rows(int wn) { return 128u * uint32_t(wn); }

// Launch the MFMA distance GEMM.  Chooses the tile shape from Q.
va_status launch_dist(va_context* ctx, const DistArgs& a);

// Row-wise exact top-k selection (one workgroup per row).
struct SelectArgs {
    // source of items: either a dense key matrix (ids = column index) or candidate lists
    const uint32_t* keys = nullptr;  // [rows x ld] keys, or candidate keys [rows x cap]
    const uint32_t* ids = nullptr;   // candidate ids [rows x cap] (nullptr: id = column index)
    const uint32_t* counts = nullptr; // per-row counts (candidate mode); nullptr: n for every row
    int64_t ld = 0;
    uint32_t n = 0;        // items per row (dense) or capacity (candidate mode)
    uint32_t rows = 0;
    uint32_t k = 0;
    uint32_t id_offset = 0;        // added to output ids
    const uint32_t* row_map = nullptr;  // output row for each input row (nullptr: identity)
    // device row count (rows past it are skipped; rows is then the host bound), or nullptr
    const uint32_t* rows_dev = nullptr;
    // outputs (row stride out_ld, default k)
    int64_t out_ld = 0;
    uint32_t* out_idx = nullptr;   // [rows x k]
    uint32_t* out_key = nullptr;   // [rows x k] keys (optional)
    float* out_f = nullptr;        // [rows x k] float values (optional)
    int32_t* out_i32 = nullptr;    // [rows x k] int32 values (optional)
    int key_kind = 0;              // 0 float asc, 1 float desc, 2 int32, 3 uint32 (for value outputs)
    // threshold mode: write only the k-th smallest key per row (ignores outputs above)
    uint32_t* out_kth = nullptr;
    // overflow detection (candidate mode): rows whose count exceeds n, or is below min_count,
    // are listed here
    uint32_t* overflow_count = nullptr;
    uint32_t* overflow_rows = nullptr;
    uint32_t min_count = 0;
    // every key is below 2^key_bits (Hamming distances: a few bits); up to 11 bits the k-th
    // smallest key comes from one histogram pass instead of four byte passes
    uint32_t key_bits = 32;
};
va_status launch_select(va_context* ctx, const SelectArgs& a);

// assign[i] = the nearest centroid of row i by L2^2 (ties -> lower centroid) on the fp32 MFMA
// distance kernel with the argmin epilogue; best is N words of scratch
va_status nearest_centroids(va_context* ctx, const float* x, const float* cen, uint32_t N, uint32_t C, uint32_t D,
                            unsigned long long* best, uint32_t* assign);
// CSR lists from assignments: ids = row ids grouped by centroid in row order (stable sort),
// offsets[C + 1].  Synchronises the context's stream.
va_status csr_from_assignments(va_context* ctx, const uint32_t* assign, uint32_t N, uint32_t C, uint32_t* ids,
                               uint32_t* offsets);

// fill a device u32 array (graph-safe replacement for hipMemsetAsync)
va_status fill_u32(va_context* ctx, uint32_t* p, uint64_t n, uint32_t v);

// Exact top-k over any key producer (fp32 distances, int8 dots, Hamming distances).
// The Q x N key matrix is never materialised:
//   1. sample pass: keys of every query against a strided sample of S rows; the k-th
//      smallest sample key is an upper bound tau_q of the query's true k-th key;
//   2. filter pass: every (query, row) key <= tau_q is appended to the query's candidate
//      list (atomic counter, capacity `cap`);
//   3. select: exact (key, id) top-k of each candidate list;
//   4. rows whose list overflowed are recomputed exactly, chunk by chunk (rare).
// Small databases (N <= sample) go straight to dense keys + select.
struct FbArgs;  // the device-side overflow fallback (va_fallback.hpp)

struct KeyProducer {
    // keys for queries [q0, q0+nq) (or rows qrow[0..nq) when qrow != nullptr) against
    // database rows c0 + j*stride, j < cols, written to out_k[i * ldo + j]
    virtual va_status dense(const uint32_t* qrow, uint32_t q0, uint32_t nq, uint32_t c0, uint32_t cols,
                            uint32_t stride, uint32_t* out_k, int64_t ldo) = 0;
    // filter pass over all queries and all rows
    virtual va_status filter(const uint32_t* thr, uint32_t* cnt, uint32_t* ckey, uint32_t* cid, uint32_t cap) = 0;
    // every key the producer makes is below 2^key_bits()
    virtual uint32_t key_bits() const { return 32; }
    // one pass of the device-side overflow fallback (fb_pass_kernel over the producer's keys)
    virtual va_status fallback_pass(const FbArgs& a, int pass) = 0;
    virtual ~KeyProducer() = default;
};

struct ScanOutputs {
    uint32_t* idx = nullptr;
    float* f = nullptr;        // key_kind 0
    int32_t* i32 = nullptr;    // key_kind 2
    uint32_t* key = nullptr;   // raw keys (Hamming distances)
    int key_kind = 0;
    // rows excluded from the search (skip[row] != 0; the deleted rows of an index), or nullptr:
    // their keys become kAbsentKey before every selection
    const uint8_t* skip = nullptr;
};

// keys[r * ld + j] = kAbsentKey for the rows + j * stride (j < cols) that skip excludes
va_status mask_dense_keys(va_context* ctx, uint32_t* keys, uint32_t rows, uint32_t cols, int64_t ld, uint32_t row0,
                          uint32_t stride, const uint8_t* skip);
// keys[r * ld + i] (and keys2, when given) = kAbsentKey for the excluded ids[r * ld + i],
// i < min(counts[r], cap); with id_map the list holds positions p and the row id is id_map[p]
va_status mask_list_keys(va_context* ctx, uint32_t* keys, uint32_t* keys2, const uint32_t* ids, const uint32_t* counts,
                         uint32_t rows, uint32_t cap, int64_t ld, const uint8_t* skip,
                         const uint32_t* id_map = nullptr);

va_status exact_topk_scan(va_context* ctx, KeyProducer& kp, uint32_t Q, uint32_t N, uint32_t k,
                          const ScanOutputs& out);

// IVF scan / search (probe + scan) whose results exclude the rows whose skip byte, indexed by row
// id, is set (an index's deletions): excluded rows become absent keys before every selection of
// the scan, its threshold samples and its device fallback included.  skip = nullptr: va_ivf_scan /
// va_ivf_search.
va_status ivf_scan_masked(va_context* ctx, const va_ivf* ivf, const float* queries, uint32_t num_queries,
                          const uint32_t* probes, uint32_t nprobe, uint32_t k, uint32_t* out_idx, float* out_dist,
                          const uint8_t* skip);
va_status ivf_search_masked(va_context* ctx, const va_ivf* ivf, const float* queries, uint32_t num_queries,
                            uint32_t nprobe, uint32_t k, uint32_t* out_idx, float* out_dist, const uint8_t* skip);
uint32_t ivf_num_lists(const va_ivf* ivf);

// Plan of the sampled scan: S sample rows (every stride-th row), candidate capacity per query,
// queries per sample launch; direct = the database is small enough for dense keys.
// The order statistic of the sample that becomes a query's threshold (k, or a smaller rank whose
// lists are checked before use; va_scan.hip)
uint32_t sample_rank(const va_context* ctx, uint32_t k, uint64_t S, uint32_t N, bool masked);
// sample size, strided sample step and candidate capacity of an exact top-k scan
ScanPlan plan_scan(const va_context* ctx, uint32_t Q, uint32_t N, uint32_t k);

// Exact top-k of the listed query rows (device list) by dense keys over the whole database in
// chunks (the path of queries whose candidate list overflowed).  Writes base's outputs at the
// listed rows; rows excluded by skip (may be nullptr) are absent.  Synchronises the stream.
va_status rescan_rows(va_context* ctx, KeyProducer& kp, uint32_t N, uint32_t k, const SelectArgs& base,
                      const uint32_t* rows_dev, uint32_t n_rows, const uint8_t* skip = nullptr);

// Takes the next profiling record of the ring, folding the scan it held first (that scan is
// long finished in steady state).  nullptr on failure.
va_context::ScanRecord* profile_record(va_context* ctx);
// Waits for a pending record's events and adds its phase times to the context's totals.
void profile_fold(va_context* ctx, va_context::ScanRecord& r);
// Enqueues sum(v[0..n)) into *out (one workgroup).
va_status sum_u32_into(va_context* ctx, const uint32_t* v, uint32_t n, uint32_t* out);

// hipEvent marks of the scan phases (no-ops unless profiling is on).  Nothing here waits: the
// events are read when the record is reused or the timings are asked for.
struct ScanPhaseMarks {
    va_context* ctx;
    va_context::ScanRecord* r = nullptr;
    explicit ScanPhaseMarks(va_context* c) : ctx(c) {}
    va_status mark(int i) {
        if (!ctx->profiling) return VA_OK;
        if (ctx->profiling == 2 && i != 1 && i != 2) return VA_OK;  // the scan phase alone
        if (i == 0 || !r) r = profile_record(ctx);
        if (!r) return VA_ERR_HIP;
        r->light = ctx->profiling == 2;
        VA_CHECK_HIP(ctx, hipEventRecord(r->ev[i], ctx->stream));
        return VA_OK;
    }
    // profiling only: the device count of overflowed rows, read with the record
    va_status count_overflow(const uint32_t* dev_count) {
        if (ctx->profiling != 1 || !r) return VA_OK;
        VA_CHECK_HIP(ctx, hipMemcpyAsync(r->host_word, dev_count, 4, hipMemcpyDeviceToHost, ctx->stream));
        r->has_ovf = true;
        return VA_OK;
    }
    // profiling only: the sum of a device array (rows re-scored by the rerank), read with the record
    va_status count_sum(const uint32_t* v, uint32_t n) {
        if (ctx->profiling != 1 || !r) return VA_OK;
        VA_CHECK_STATUS(sum_u32_into(ctx, v, n, r->dev_word));
        VA_CHECK_HIP(ctx, hipMemcpyAsync(r->host_word + 1, r->dev_word, 4, hipMemcpyDeviceToHost, ctx->stream));
        r->has_rerank = true;
        return VA_OK;
    }
    // events: 0 start, 1 after sample, 2 after scan, 3 after select, 4 end
    va_status finish(bool sampled, bool fallback) {
        if (!ctx->profiling || !r) return VA_OK;
        if (!r->light) VA_CHECK_HIP(ctx, hipEventRecord(r->ev[4], ctx->stream));
        r->sampled = sampled;
        r->fallback = fallback;
        r->t = ctx->last_scan;
        r->pending = true;
        ctx->rec_last = int(r - ctx->rec);
        return VA_OK;
    }
};

// The fp32 top-k with an fp16 screening pass (va_screen.hip): the same result as
// exact_topk_scan over F32 keys, bit for bit, from a cheaper filtering scan.
struct ScreenInput {
    const float* q = nullptr;
    const float* x = nullptr;
    uint32_t Q = 0, N = 0, D = 0;
    DistOp op = OP_L2SQ;
    // optional fp16 shadow of x (shadow_pitch(D) halves per row) and its squared norms: the
    // filtering scan then reads it instead of converting x
    const _Float16* xh = nullptr;
    const float* xn = nullptr;
    // optional with the shadow: xe[j] >= |fp16(x_j) - x_j| (build_shadow's errs); the candidates'
    // intervals then use the measured rounding errors (narrower than the worst case)
    const float* xe = nullptr;
};
// Exact top-k of device queries against a device database (va_fused_topk's body).  shadow /
// norms: an fp16 shadow of x (see build_shadow) or nullptr; skip: rows excluded, or nullptr.
va_status flat_topk(va_context* ctx, DistOp op, const float* q, const float* x, uint32_t Q, uint32_t N, uint32_t D,
                    uint32_t k, uint32_t* out_idx, float* out_dist, const _Float16* shadow = nullptr,
                    const float* norms = nullptr, const uint8_t* skip = nullptr, const float* errs = nullptr);
// Halves per row of an fp16 shadow (D rounded up to a multiple of 64).
uint32_t shadow_pitch(uint32_t D);
// shadow[r * shadow_pitch(D) + d] = fp16(x[r * D + d]) (RNE, zeros past D), norms[r] = |x_r|^2
// in fp32, for rows r < N.  norm_err (may be nullptr; norms may then be nullptr): {|x_r|^2, an
// upper bound of |fp16(x_r) - x_r|} per row (infinite past the fp16 range); errs (may be
// nullptr): that upper bound alone.
va_status build_shadow(va_context* ctx, const float* x, uint32_t N, uint32_t D, _Float16* shadow, float* norms,
                       float2* norm_err = nullptr, float* errs = nullptr);
// Pieces of the screened scan shared with the IVF list scan (va_screen.hip).  The bound itself
// is va_screen_bound.hpp's.
struct ScreenBound;
// qh[q * shadow_pitch(D) + d] = fp16(q[q * D + d] * 2^sc_q) (the query's scale puts its largest
// entry in [2^14, 2^15)), qinfo[q] = {|q|^2, |q|, 2^-sc_q, c0 * 2^-25 * 2^-sc_q}; qerr (may be
// nullptr): an upper bound of the norm of the (unscaled) rounding error of each query's fp16 image.
// zero0[0 .. n0) and zero1[0 .. n1) are cleared by the same launch (a search's counters).
va_status screen_prepare_queries(va_context* ctx, const float* q, uint32_t Q, uint32_t D, _Float16* qh,
                                 float4* qinfo, float c0, float* qerr = nullptr, uint32_t* zero0 = nullptr,
                                 uint32_t n0 = 0, uint32_t* zero1 = nullptr, uint32_t n1 = 0);
// Candidate lists of screened pairs, in place: (unscaled fp16 dot, |x|^2) -> (key of the upper
// bound, key of the lower bound) of the pair's fp32 key, for i < min(cnt[q], cap).
va_status screen_list_bounds(va_context* ctx, const ScreenBound& b, const float4* qinfo, float* dot, float* xx,
                             const uint32_t* cnt, uint32_t cap, uint32_t Q);
// Rerank lists: rr[q * rcap ..] = the cand_id of the candidates with lower bound <= bound[q];
// queries whose candidates overflowed (cnt > cap) or whose list outgrows rcap get rcount 0 and
// are appended to ovf_rows (ovf_cnt[0] counts them; ovf_cnt[1] receives the longest list).
va_status screen_compact(va_context* ctx, const uint32_t* cnt, const uint32_t* cand_lo, const uint32_t* cand_id,
                         const uint32_t* bound, uint32_t cap, uint32_t Q, uint32_t* rr, uint32_t* rcount, uint32_t rcap,
                         uint32_t* ovf_cnt, uint32_t* ovf_rows);
// Whether the screened path applies (metric, alignment, sizes, VA_OPT_SCREEN).
bool screen_applies(const va_context* ctx, const ScreenInput& in, uint32_t k);
va_status screened_topk_scan(va_context* ctx, const ScreenInput& in, KeyProducer& exact, uint32_t k,
                             const ScanOutputs& out);

}  // namespace va
