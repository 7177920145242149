// ztcp_rows.h -- row geometry and LDS hand-off helpers shared by the fused
// egress and ingress kernels.
//
// A row is one 64-byte keystream block position of the payload, for all pages
// of a workgroup (lane = page).  Row slots in LDS hold 16 words per page; the
// 16-byte quads of a page are XOR-swizzled so that both lane-per-page access
// and the transposed four-lanes-per-page access used for coalesced global
// stores are free of bank conflicts.
#pragma once

#include "ztcp_params.h"

namespace ztcp {

constexpr int kRowWords = 64 * 16;         // one row: 64 pages x 16 words

// Word offset of quad q (16 bytes) of page `pg` inside a row slot.  The quad
// index is XOR-swizzled by page so that lane-per-page accesses and the
// transposed four-lanes-per-page accesses are both free of bank conflicts.
__device__ __forceinline__ uint32_t quad_word(int pg, int q) {
    return (uint32_t)(pg * 16 + ((q ^ ((pg >> 1) & 3)) << 2));
}

__device__ __forceinline__ uint4 lds_quad(const uint32_t* row, int pg, int q) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(row + quad_word(pg, q));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void lds_put_quad(uint32_t* row, int pg, int q, uint4 x) {
    *reinterpret_cast<uint4*>(row + quad_word(pg, q)) = x;
}

// Byte offsets of the four quads of one page inside a row slot, computed once
// per lane (the swizzle depends only on the page).
struct PageQuads {
    uint32_t off[4];
    __device__ __forceinline__ void init(int pg) {
#pragma unroll
        for (int q = 0; q < 4; ++q) off[q] = quad_word(pg, q) * 4u;
    }
};

// Loaded as a 4 x u32 vector: reading a uint4 struct lets the compiler turn
// the 64-bit word views of the quad into a second, overlapping LDS read.
__device__ __forceinline__ uint4 lds_quad_at(const uint32_t* row, uint32_t byte_off) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(row) + byte_off);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void lds_put_quad_at(uint32_t* row, uint32_t byte_off, uint4 x) {
    *reinterpret_cast<uint4*>(reinterpret_cast<char*>(row) + byte_off) = x;
}

// Phase timers (builds with ZTCP_PHASE_TIMERS only; the product library has
// none of this code).  Each workgroup keeps kTimerSlots 64-bit counters in
// LDS right after its other LDS data: shader-clock counts (s_memtime) of the
// start-up, of the waits of each wave role and of the end, relative to the
// clock at which the wave left the workgroup's first barrier.  Thread 0
// copies them to the call's timer record at the end of the kernel.
#ifdef ZTCP_PHASE_TIMERS
constexpr bool kPhaseTimers = true;
#else
constexpr bool kPhaseTimers = false;
#endif
constexpr int kTimerSlots = 48;        // 64-bit counters per workgroup
constexpr int kTimerMaxWg = 4096;      // workgroups with a record
constexpr int kTraceRows = 1024;       // rows traced in workgroup 0: [4][kTraceRows] u32 after the records
constexpr int kTimerLdsWords = kPhaseTimers ? 2 * kTimerSlots : 0;
enum TimerSlot : int {
    kTmMacRowsBegin = 0,   // MAC / verify wave: header absorbed, payload rows begin
    kTmMacFirstRow = 1,    // MAC / verify wave: first payload row absorbed
    kTmMacRowsEnd = 2,     // MAC / verify wave: last payload row absorbed
    kTmMacEnd = 3,         // MAC / verify wave: tag done
    kTmWgEnd = 4,          // after the workgroup's last barrier
    kTmProdFirstRow = 5,   // earliest clock at which a producer / decoder published a row (min)
    kTmProdLast = 6,       // latest clock at which a producer / decoder ran out of rows (max)
    kTmProdBusy = 7,       // sum over producer / decoder waves of (exit - start)
    kTmMacWait = 8,        // [8] MAC / verify wave: clocks waiting for a row, by payload row / 64
    kTmMacMiss = 16,       // [8] MAC / verify wave: rows not ready when first tested, by row / 64
    kTmRingWait = 24,      // producers / decoders: waiting for ring space
    kTmStageWait = 25,     // egress producers: staging slot free; ingress decoders: scales ready
    kTmFreeWait = 26,      // ingress scale rows: staging slot free
    kTmStorerWait = 27,    // egress storer: waiting for a row
    kTmFeedWait = 28,      // feeder: waiting (scale row stored, ring space)
    kTmStorerEnd = 29,     // egress storer: done
    kTmFeedEnd = 30,       // feeder: done
    kTmProdWaves = 31,     // producer / decoder waves that ran
    kTmRows = 32,          // rows made by producers / decoders
    kTmProdSetup = 33,     // earliest producer / decoder done with its page setup (descriptor, nonce cache)
    kTmProdLoaded = 34,    // earliest producer / decoder holding its first row's data (egress: quantized)
    // written to the record by thread 0 directly
    kTmAbsStart = 40,      // s_memtime after the first barrier
    kTmAbsEnd = 41,        // s_memtime after the last barrier
    kTmRealStart = 42,     // s_memrealtime (100 MHz) after the first barrier
    kTmRealEnd = 43,       // s_memrealtime after the last barrier
};

__device__ __forceinline__ uint64_t phase_clock() {
    if constexpr (kPhaseTimers) return __builtin_amdgcn_s_memtime();
    return 0;
}
__device__ __forceinline__ void tm_add(uint32_t* tm, int slot, uint64_t v) {
    if constexpr (kPhaseTimers) {
        if ((threadIdx.x & 63) == 0)
            __hip_atomic_fetch_add(reinterpret_cast<unsigned long long*>(tm) + slot, (unsigned long long)v,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}
__device__ __forceinline__ void tm_max(uint32_t* tm, int slot, uint64_t v) {
    if constexpr (kPhaseTimers) {
        if ((threadIdx.x & 63) == 0)
            __hip_atomic_fetch_max(reinterpret_cast<unsigned long long*>(tm) + slot, (unsigned long long)v,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}
__device__ __forceinline__ void tm_min(uint32_t* tm, int slot, uint64_t v) {
    if constexpr (kPhaseTimers) {
        if ((threadIdx.x & 63) == 0)
            __hip_atomic_fetch_min(reinterpret_cast<unsigned long long*>(tm) + slot, (unsigned long long)v,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}
// Clears the LDS counters (min slots start at all ones); every thread of the
// workgroup calls it before the first barrier.
__device__ __forceinline__ void tm_clear(uint32_t* tm) {
    if constexpr (kPhaseTimers) {
        if ((int)threadIdx.x < kTimerSlots)
            reinterpret_cast<unsigned long long*>(tm)[threadIdx.x] =
                (threadIdx.x == kTmProdFirstRow || threadIdx.x == kTmProdSetup || threadIdx.x == kTmProdLoaded)
                    ? ~0ull : 0ull;
    }
}
// Workgroup 0's row trace (timer builds): 32-bit clocks since the first
// barrier at which each payload row reached the ring (trace[r]) and at which
// the MAC / verify wave absorbed it (trace[kTraceRows + r]); for a group of
// four rows from r whose flags that wave found incomplete, the clocks it
// then waited for the group's rows (trace[2 kTraceRows + r]); the words from
// 3 kTraceRows stay zero.
__device__ __forceinline__ uint32_t* trace_of(unsigned long long* timers) {
    if constexpr (kPhaseTimers) {
        if (timers && blockIdx.x == 0)
            return reinterpret_cast<uint32_t*>(timers + (size_t)kTimerMaxWg * kTimerSlots);
    }
    return nullptr;
}
// Workgroup 0, every thread, before the first barrier: zero the slow-path
// words of the trace (fast-path rows leave them 0).
__device__ __forceinline__ void tm_trace_clear(unsigned long long* timers) {
    if constexpr (kPhaseTimers) {
        uint32_t* trace = trace_of(timers);
        if (!trace) return;
        for (int i = threadIdx.x; i < 2 * kTraceRows; i += blockDim.x) trace[2 * kTraceRows + i] = 0u;
        __threadfence_block();
    }
}
// Trace words are stored through a global pointer: a store through a
// generic pointer is a flat store, which the wave's LDS waits also wait for,
// so the traced wave would stall for each trace store's write latency.
__device__ __forceinline__ void tm_trace_put(uint32_t* trace, int idx, uint32_t v) {
    if constexpr (kPhaseTimers) ((__attribute__((address_space(1))) uint32_t*)trace)[idx] = v;
}
__device__ __forceinline__ void tm_trace(uint32_t* trace, int idx, uint64_t t0) {
    if constexpr (kPhaseTimers) {
        if (trace && idx >= 0 && idx < 4 * kTraceRows && (threadIdx.x & 63) == 0)
            tm_trace_put(trace, idx, (uint32_t)(phase_clock() - t0));
    }
}

// Thread 0, after the last barrier: the LDS counters and the absolute clocks
// into this workgroup's record (kTimerSlots words) of the call's buffer.
__device__ __forceinline__ void tm_flush(const uint32_t* tm, unsigned long long* rec, uint64_t start,
                                         uint64_t real_start) {
    if constexpr (kPhaseTimers) {
        if (!rec || threadIdx.x != 0) return;
        const uint64_t end = __builtin_amdgcn_s_memtime();
        const uint64_t real_end = __builtin_amdgcn_s_memrealtime();
        unsigned long long* r = rec + (size_t)blockIdx.x * kTimerSlots;
        const unsigned long long* t = reinterpret_cast<const unsigned long long*>(tm);
        for (int i = 0; i < kTimerSlots; ++i) r[i] = t[i];
        r[kTmWgEnd] = end - start;
        r[kTmAbsStart] = start;
        r[kTmAbsEnd] = end;
        r[kTmRealStart] = real_start;
        r[kTmRealEnd] = real_end;
    }
}

// Where a wave's bounded waits report an expiry: the device's sticky
// diagnostics, the call's own diagnostics (ingress) and an LDS word of the
// workgroup, which the kernel reads after its last barrier to fail every
// page of the workgroup closed.  `tm` and `t0` serve the phase timers only.
struct Waiter {
    uint32_t* dev_diag;
    uint32_t* call_diag;   // nullptr: no per-call record
    uint32_t* expired;     // LDS
    uint32_t spin_limit;
    uint32_t call_tag;     // WaitSink::call_tag
    uint32_t* tm;          // LDS phase-timer counters (timer builds)
    uint64_t t0;           // clock at which the wave left the first barrier (timer builds)
    uint32_t* trace;       // workgroup 0's row trace (timer builds), else nullptr
};

__device__ __forceinline__ Waiter make_waiter(const WaitSink& s, uint32_t* expired_lds, uint32_t* tm = nullptr,
                                              uint64_t t0 = 0) {
    return Waiter{s.dev_diag, s.call_diag, expired_lds, s.spin_limit, s.call_tag, tm, t0, nullptr};
}

// Waits until *flag >= want (monotonic counters; want <= 0 returns at once).
// Bounded: after spin_limit polls the wait records DIAG (device and call
// diagnostics, the workgroup's LDS word) and returns; the caller carries on,
// and the kernel fails the workgroup's pages at its end.  Once any wait of
// the workgroup has expired, its hand-offs are broken and later waits may
// never be satisfied: every wait that finds the LDS word set returns at its
// next poll instead of spinning out its own bound, so a broken workgroup
// ends about one bound after its first expiry.  TSLOT >= 0: timer builds add
// the clocks spent here to that phase-timer slot.
template <uint32_t DIAG, int TSLOT = -1>
__device__ __forceinline__ void wait_ge(const uint32_t* flag, int32_t want, const Waiter& w) {
    if ((int32_t)__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= want) return;
    [[maybe_unused]] const uint64_t t_in = (kPhaseTimers && TSLOT >= 0) ? phase_clock() : 0;
    for (uint32_t spin = 0;; ++spin) {
        if (__hip_atomic_load(w.expired, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0u) break;
        if (spin >= w.spin_limit) {
            if ((threadIdx.x & 63) == 0) {
                atomicOr(w.dev_diag, DIAG);
                if (w.call_diag) {
                    // egress calls carry a tag (the host reads the slot back
                    // by tag); ingress calls or in their kernel's bit
                    if constexpr (DIAG == kDiagEgressWait) atomicMax(w.call_diag, w.call_tag);
                    else atomicOr(w.call_diag, DIAG);
                }
            }
            __hip_atomic_store(w.expired, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        if ((int32_t)__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= want) break;
    }
    if constexpr (kPhaseTimers && TSLOT >= 0) tm_add(w.tm, TSLOT, phase_clock() - t_in);
}

// Marks 16 words as produced here: the computation of w[] stays before the
// code that follows (an empty asm that reads and rewrites them), which keeps
// the compiler from sinking it below a wait loop.
__device__ __forceinline__ void pin_words(uint32_t (&w)[16]) {
    asm volatile("" : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(w[4]), "+v"(w[5]), "+v"(w[6]),
                      "+v"(w[7]), "+v"(w[8]), "+v"(w[9]), "+v"(w[10]), "+v"(w[11]), "+v"(w[12]), "+v"(w[13]),
                      "+v"(w[14]), "+v"(w[15]));
}

__device__ __forceinline__ void publish(uint32_t* flag, uint32_t value) {
    __hip_atomic_store(flag, value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// A hand-off through LDS whose data this wave read or wrote in LDS only: the
// LDS unit performs a wave's LDS operations in issue order, so every access
// issued before the flag store has been performed when another wave reads
// the flag.  The empty asm keeps the compiler from moving those accesses
// past the store; unlike a release, the store does not wait for this wave's
// LDS reads still in flight (the MAC wave's prefetched rows).
__device__ __forceinline__ void publish_lds(uint32_t* flag, uint32_t value) {
    asm volatile("" ::: "memory");
    __hip_atomic_store(flag, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// A SIMD issues the oldest of its ready waves first, so four worker waves of
// equal priority progress at very different speeds (the youngest one's first
// row finishes about four times later than the oldest one's).  Rows are
// handed out in order while the MAC wave consumes them in order, so a row
// held by a starved wave stalls the chain.  A worker therefore raises its
// priority by how soon the MAC wave absorbs the row it is making: `lead` =
// payload row - rows absorbed (wave-uniform).
__device__ __forceinline__ void set_row_priority(int32_t lead) {
    if (lead <= 4) __builtin_amdgcn_s_setprio(3);
    else if (lead <= 10) __builtin_amdgcn_s_setprio(2);
    else if (lead <= 18) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
}

// set_row_priority for payload row `row` from the rows absorbed so far.
// Workers call it again while they make a row: a row taken far ahead of the
// MAC / verify wave starts at a low priority, and if its wave is the
// youngest on its SIMD it is starved by the older ones until it is the row
// that holds up the chain (a group of rows waiting for its last member).
__device__ __forceinline__ void refresh_row_priority(const uint32_t* used, int32_t row) {
    set_row_priority(
        row - (int32_t)__builtin_amdgcn_readfirstlane(
                  __hip_atomic_load(used, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)));
}

// ---------------------------------------------------------------------------
// The MAC wave's side of a ring of row slots holding the payload in order:
// payload row r sits in slot r % ring_len once flag[slot] = r + 1, and the
// wave publishes `used` = rows absorbed, which frees their slots.
// ---------------------------------------------------------------------------

// Rows per readiness test and per release of the MAC / verify wave.  Ring
// lengths are multiples of it, so a group's four flags are one aligned
// 16-byte LDS read.  Against a test and a release per row this takes about
// 70 clocks per row off the chain (a probe of the MAC wave alone in the
// kernel: 1,836 clocks per row with per-row flags and releases, 1,790
// without the flag reads, 1,808 without the releases).
constexpr int kMacGroup = 4;

// The four ready flags of the group at `slot`, read before any of the
// group's data (LDS operations of a wave are performed in order, and a row's
// maker writes the row before it releases its flag: a flag read that shows
// the row guarantees that a later data read holds it).  The read goes
// through an LDS pointer and is kept in place by compiler barriers, not by
// `volatile`: a volatile read of a generic pointer was compiled as a flat
// load with system-coherence bits followed at once by a wait for every
// outstanding memory operation of the wave (about 1 % of both kernels).
__device__ __forceinline__ uint4 mac_flags4(const uint32_t* ring_flags, int32_t slot) {
    asm volatile("" ::: "memory");  // read afresh: other waves write the flags
    const u32x4 v = *(const __attribute__((address_space(3))) u32x4*)(ring_flags + slot);
    asm volatile("" ::: "memory");  // the data reads stay after the flag read
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Whether rows row0 .. row0 + 3 (those below total) are all in the ring.
// Every lane read the same words: a vector compare and a ballot cost the
// chain nothing measurable, where v_readfirstlane of a flag cost it about
// 66 clocks.
__device__ __forceinline__ bool mac_ready4(const uint4 f, int32_t row0, int32_t total) {
    const bool ok = ((int32_t)f.x > row0 || row0 >= total) && ((int32_t)f.y > row0 + 1 || row0 + 1 >= total) &&
                    ((int32_t)f.z > row0 + 2 || row0 + 2 >= total) && ((int32_t)f.w > row0 + 3 || row0 + 3 >= total);
    return __builtin_amdgcn_ballot_w64(!ok) == 0ull;
}

__device__ __forceinline__ void mac_row_data(const uint32_t* ring, const PageQuads& pq, int32_t slot, uint4 (&x)[4]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) x[q] = lds_quad_at(ring + slot * kRowWords, pq.off[q]);
}

// Absorbs payload rows [0, total) from a ring of RING slots, four rows per
// group.  The group's flags are read, then the data of its first two rows,
// while the previous group's last two rows are absorbed; at the group's
// start one ballot tests all four flags (if any row is missing, the wave
// takes that group a row at a time, below); the data of its third and
// fourth rows are read while its first two are absorbed.  Every read thus
// has two rows' absorption to complete before it is used, and the wave
// publishes `used` once per group.  Reads past the last row fetch
// slots that are never absorbed.  The caller completes every load it has
// issued before the call: a load still counted as in flight where the loop
// begins would turn the loop's LDS waits into full waits.
template <int RING, uint32_t DIAG>
__device__ __forceinline__ void mac_rows(const Waiter& wt, const uint32_t* ring, const uint32_t* ring_flags,
                                         uint32_t* used, const PageQuads& pq, Sip& s, int32_t total) {
    static_assert(RING % kMacGroup == 0 && kMacGroup == 4, "a group's flags are one aligned 16-byte read");
    uint4 b0[4], b1[4], b2[4], b3[4];
    int32_t gs = 0;  // ring slot of the group's first row
    uint4 fl = mac_flags4(ring_flags, 0);
    mac_row_data(ring, pq, 0, b0);
    mac_row_data(ring, pq, 1, b1);
    [[maybe_unused]] auto traced = [&](int32_t row) {
        if constexpr (kPhaseTimers) {
            if (row == 0) tm_add(wt.tm, kTmMacFirstRow, phase_clock() - wt.t0);
            tm_trace(wt.trace, kTraceRows + row, wt.t0);
        }
    };
    // A row taken alone: waited for, read, absorbed and released at once.
    auto one_row = [&](int32_t row, int32_t slot, uint64_t& waited) {
        [[maybe_unused]] const uint64_t t_in = phase_clock();
        wait_ge<DIAG>(ring_flags + slot, row + 1, wt);
        if constexpr (kPhaseTimers) waited += phase_clock() - t_in;
        mac_row_data(ring, pq, slot, b2);
        s.absorb64(b2);
        traced(row);
        publish(used, (uint32_t)(row + 1));
    };
    // Whole groups.  The inner loop takes ready groups and has one exit, to
    // the code for a group with a row missing, which rejoins it with the
    // next group's flags and first two rows in fl, b0 and b1, as the inner
    // loop leaves them.  (A loop with its exits between the rows of a group
    // had the compiler copy the chain's state and the prefetched rows to
    // other registers and back on every iteration.)
    const int32_t full = total & ~(kMacGroup - 1);
    int32_t r = 0;
#pragma unroll 1
    while (r < full) {
#pragma unroll 1
        for (; r < full; r += kMacGroup) {
            if (__builtin_expect(!mac_ready4(fl, r, total), 0)) break;
            const int32_t ns = gs + kMacGroup == RING ? 0 : gs + kMacGroup;
            mac_row_data(ring, pq, gs + 2, b2);
            s.absorb64(b0);
            traced(r);
            mac_row_data(ring, pq, gs + 3, b3);
            s.absorb64(b1);
            traced(r + 1);
            fl = mac_flags4(ring_flags, ns);
            mac_row_data(ring, pq, ns, b0);
            s.absorb64(b2);
            traced(r + 2);
            mac_row_data(ring, pq, ns + 1, b1);
            s.absorb64(b3);
            traced(r + 3);
            publish(used, (uint32_t)(r + kMacGroup));
            gs = ns;
        }
        if (r >= full) break;
        // A row of the group is missing (most often its last, held by a
        // worker that fell behind): take the group a row at a time, each as
        // soon as it is in the ring, and release each slot at once, so that
        // the rows already there are absorbed while the wave waits for the
        // missing one.
        const int32_t ns = gs + kMacGroup == RING ? 0 : gs + kMacGroup;
        [[maybe_unused]] uint64_t waited = 0;
#pragma unroll 1
        for (int i = 0; i < kMacGroup; ++i) one_row(r + i, gs + i, waited);
        if constexpr (kPhaseTimers) {
            const int b = min(r >> 6, 7);
            tm_add(wt.tm, kTmMacWait + b, waited);
            tm_add(wt.tm, kTmMacMiss + b, 1);
            if (wt.trace && (threadIdx.x & 63) == 0 && r < kTraceRows)
                tm_trace_put(wt.trace, 2 * kTraceRows + r, (uint32_t)waited);
        }
        fl = mac_flags4(ring_flags, ns);
        mac_row_data(ring, pq, ns, b0);
        mac_row_data(ring, pq, ns + 1, b1);
        gs = ns;
        r += kMacGroup;
    }
    // the last total % 4 rows, one at a time
    [[maybe_unused]] uint64_t waited = 0;
#pragma unroll 1
    for (int32_t i = 0; r < total; ++r, ++i) one_row(r, gs + i, waited);
    if constexpr (kPhaseTimers) tm_add(wt.tm, kTmMacWait + min(full >> 6, 7), waited);
    publish(used, (uint32_t)total);
}

// ---------------------------------------------------------------------------
// Loads four lanes per page.  A load of 16 bytes per lane from 64 pages
// touches 64 lines per instruction; four lanes per page read 64 contiguous
// bytes of 16 pages (on all 256 workgroups at once: 4.8 TB/s against
// 3.1 TB/s, a probe over 16,384 pages).  Lane 16 r + c takes quad r of page
// 16 i + c in load i; the four 16-lane rows of four such loads are then
// transposed (row_transpose) so that every lane holds its own page's quads.
// ---------------------------------------------------------------------------

typedef uint32_t ztcp_u32x2 __attribute__((ext_vector_type(2)));

// a = [a0, a1, b0, b1], b = [a2, a3, b2, b3] in 16-lane rows
__device__ __forceinline__ void swap_halves(uint32_t& a, uint32_t& b) {
    const ztcp_u32x2 r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}
// a = [a0, b0, a2, b2], b = [a1, b1, a3, b3] in 16-lane rows
__device__ __forceinline__ void swap_rows(uint32_t& a, uint32_t& b) {
    const ztcp_u32x2 r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}

// 4 x 4 transpose of the 16-lane rows of four registers of 16 bytes, R0 =
// a[0..3], R1 = a[4..7], R2 = b[0..3], R3 = b[4..7]: afterwards row r of Rq
// holds what row q of Rr held.
__device__ __forceinline__ void row_transpose(uint32_t (&a)[8], uint32_t (&b)[8]) {
#pragma unroll
    for (int d = 0; d < 8; ++d) swap_halves(a[d], b[d]);  // (R0, R2), (R1, R3)
#pragma unroll
    for (int d = 0; d < 4; ++d) {                         // (R0, R1), (R2, R3)
        swap_rows(a[d], a[4 + d]);
        swap_rows(b[d], b[4 + d]);
    }
}

// p of lanes c, 16 + c, 32 + c, 48 + c, for every lane of column c.
__device__ __forceinline__ void column_ptrs(const void* p, const uint8_t* (&out)[4]) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        lo[i] = (uint32_t)v;
        hi[i] = (uint32_t)(v >> 32);
    }
    swap_halves(lo[0], lo[2]);
    swap_halves(lo[1], lo[3]);
    swap_rows(lo[0], lo[1]);
    swap_rows(lo[2], lo[3]);
    swap_halves(hi[0], hi[2]);
    swap_halves(hi[1], hi[3]);
    swap_rows(hi[0], hi[1]);
    swap_rows(hi[2], hi[3]);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = reinterpret_cast<const uint8_t*>(((uint64_t)hi[i] << 32) | lo[i]);
}

// Row geometry of one section (all values wave-uniform).
struct SecRows {
    int32_t kind, nblk, rpu, n_units;
    int32_t code_begin;
    int32_t qunit_begin;  // units of quantized sections before this one (staging order)
    int32_t gpv, col, src;
    uint32_t q_off, s_off;
};

__device__ __forceinline__ SecRows sec_rows(const Layout& lay, int si, int32_t code_begin, int32_t qunit_begin) {
    SecRows s;
    s.kind = ZTCP_SEC_FIELD(lay, si, kind);
    s.nblk = code_rows_per_unit(s.kind);
    s.rpu = s.nblk + (s.kind != kSecRaw ? 1 : 0);
    s.n_units = ZTCP_SEC_FIELD(lay, si, n_units);
    s.code_begin = code_begin;
    s.qunit_begin = qunit_begin;
    s.gpv = ZTCP_SEC_FIELD(lay, si, gpv);
    s.col = ZTCP_SEC_FIELD(lay, si, col);
    s.src = ZTCP_SEC_FIELD(lay, si, src);
    s.q_off = ZTCP_SEC_FIELD(lay, si, q_off);
    s.s_off = ZTCP_SEC_FIELD(lay, si, s_off);
    return s;
}

__device__ __forceinline__ int32_t total_code_rows(const Layout& lay) {
    int32_t t = 0;
#pragma unroll
    for (int si = 0; si < 3; ++si) {
        if (si >= lay.n_sec) continue;
        const int32_t kind = ZTCP_SEC_FIELD(lay, si, kind);
        t += ZTCP_SEC_FIELD(lay, si, n_units) * code_rows_per_unit(kind);
    }
    return t;
}

// One code row of a layout, by its index among the page's code rows.
struct Row {
    int32_t valid;
    int32_t u, j;     // unit in section, code block in unit
    int32_t g;        // unit index among the page's quantized units (staging slot order)
    int32_t cidx;     // code row index = production order
    int32_t mrow;     // row index in the MAC wave's order (code rows and scale rows)
    int32_t block;    // payload block index (keystream counter - 1)
    SecRows s;
};

// Code row t: the payload's code blocks in order (egress: also the order of
// production).
__device__ __forceinline__ Row row_info(const Layout& lay, int32_t t) {
    Row row{};
    int32_t cb = 0, qb = 0;
#pragma unroll
    for (int si = 0; si < 3; ++si) {
        if (si >= lay.n_sec || row.valid) continue;
        const SecRows s = sec_rows(lay, si, cb, qb);
        const int32_t n = s.n_units * s.nblk;
        if (t >= cb && t < cb + n) {
            const int32_t local = t - cb;
            row.valid = 1;
            row.u = local / s.nblk;  // nblk is 8, 4 or 16
            row.j = local - row.u * s.nblk;
            row.g = s.qunit_begin + row.u;
            row.cidx = t;
            row.mrow = t + qb;  // the scale rows of earlier sections come first
            row.block = (int32_t)(s.q_off / 64u) + local;
            row.s = s;
        }
        cb += n;
        if (s.kind != kSecRaw) qb += s.n_units;
    }
    return row;
}

}  // namespace ztcp
