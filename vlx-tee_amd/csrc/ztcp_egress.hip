// ztcp_egress.hip -- fused cold-page egress for gfx950:
// quantize -> ChaCha20 -> SipHash-2-4-128 in one kernel, one HBM read of the
// hot page and one HBM write of the blob.  Replaces the per-page encoder
// encode_one_cold_page_into_cpu (cpp:1103-1426) driven by
// fused_encode_cold_pages_peak_into_cpu (cpp:1904-2004).
//
// Work decomposition (one workgroup = up to 64 pages, 16 waves, four per
// SIMD, or 12 for the int4-per-32 and asym8 kinds; lane = page in every
// wave):
//   * A "row" is one 64-byte keystream block position of the payload, for all
//     pages of the workgroup.  Every payload block is exactly one row: a code
//     row (4 int8 / e4m3 / int4-per-32 groups, 8 int4 groups, 2 raw groups
//     or 1 asym8 group) or a scale row (the 64 parameter bytes of one unit).
//   * Eleven producer waves (on SIMDs 1-3; eight in the 12-wave kernels)
//     take code rows in order from an LDS counter.  A code
//     row quantizes its groups (loaded a row ahead; the int4 rows four lanes
//     per page, transposed between the wave's 16-lane rows afterwards),
//     stages the scales in LDS, computes the keystream, XORs, and writes the
//     ciphertext into a ring of row slots in LDS at its place in payload
//     order.
//   * A storer wave (wave 1, SIMD 1) stores every code row from the ring to
//     the blobs, in payload order, transposed (four lanes per page, 64
//     contiguous bytes per page per store).  After a unit's last code row
//     it also makes the unit's scale row: it encrypts the staged scales in
//     their slot, and stores them the same way, freeing the slot, together
//     with the next scale rows of the section, eight at a time.  Producers issue
//     no stores: a wave's wait for its own loads also waits for every store
//     it issued before them, which exposed the int4 rows' second loads; and
//     the MAC wave's SIMD is kept free of stores.
//   * Wave 0 runs SipHash for one page per lane, at raised priority on SIMD
//     0.  It absorbs the header, then the payload rows in order from the
//     ring, so it never reads global memory.  Scale rows reach the ring
//     through a feeder wave (wave 4, also on SIMD 0): a scale row is stored
//     long before the MAC wave reaches it (after all of its section's code
//     rows), and the feeder copies it back from the blob once its stores
//     have completed.  Waves 8 and 12 exit at once: producers there slow the
//     MAC chain down more than they add.
//   * Hand-offs are monotonic LDS counters with workgroup-scope
//     release/acquire: ring_flag[slot] = payload row index + 1 when written,
//     mac_used = rows absorbed and stored = rows stored (a slot is free once
//     both have passed it), stage_flag[slot] = unit + 1 when a scale row
//     has read its staging slot, scale_flag[slot] = unit + 1 once the scale
//     row's stores have completed.  Every wait is bounded; an
//     expired wait sets a sticky diagnostic bit and the kernel still ends.
//     Waits only point backwards in row order, so progress never depends on
//     a later row.
// Requires every section to hold a multiple of 32 groups (Layout::aligned),
// payload == required and 16-byte aligned pointers; otherwise the host routes
// the call to the generic kernels.
#include "ztcp_rows.h"

namespace ztcp {

namespace {

// 16 waves, four per SIMD, 128 VGPRs each: the MAC wave (0) and the
// scale-row feeder (4) on SIMD 0 (waves 8 and 12 exit at once: producers
// there slow the MAC chain down more than they add), the storer (1) and
// eleven producers on the other three SIMDs.  The kernels of the int4-per-32
// and asym8 kinds run 12 waves, three per SIMD (eight producers): their
// quantizers need more than 128 VGPRs, and 168 keep them out of scratch
// memory.
template <int FAM>
constexpr int egress_waves() { return FAM <= 1 ? 16 : 12; }  // family 2's quantizers need 168 VGPRs
constexpr int kRing = 24;             // payload rows between their makers and the MAC wave
constexpr int kStage = 13;            // units whose scales are staged at once
constexpr int kScaleGroup = 8;        // scale rows stored together (at most kScaleGroup - 1 held)
constexpr int kLdsStage = kRing * kRowWords;
constexpr int kScaleSlots = 64;       // scale rows the feeder wave may still be waiting for
constexpr int kLdsFlags = kLdsStage + kStage * kRowWords;
constexpr int kFlagRing = 0;                          // [kRing] MAC row index + 1
constexpr int kFlagStage = kFlagRing + kRing;         // [kStage] unit + 1: staging slot free
constexpr int kFlagScale = kFlagStage + kStage;       // [kScaleSlots] unit + 1: scale row stored
constexpr int kFlagMacUsed = kFlagScale + kScaleSlots;  // rows absorbed by the MAC wave
constexpr int kFlagStored = kFlagMacUsed + 1;         // rows passed by the storer wave
constexpr int kFlagTask = kFlagStored + 1;            // next code row to hand out
constexpr int kFlagExpired = kFlagTask + 1;           // 1: a bounded wait of the workgroup expired
constexpr int kNumFlags = (kFlagExpired + 2) & ~1;    // even: the blob table after it is 8-byte aligned
constexpr int kLdsBlobs = kLdsFlags + kNumFlags;      // 64 blob pointers (8-byte aligned)
constexpr int kLdsTimers = kLdsBlobs + 2 * 64;        // phase-timer counters (timer builds only)
constexpr int kLdsWords = kLdsTimers + kTimerLdsWords;
static_assert(kLdsWords * 4 <= 160 * 1024, "LDS budget of one CU");
static_assert(kScaleGroup <= kStage, "held scale rows must leave a staging slot for the unit that completes their group");
static_assert(kLdsBlobs % 2 == 0 && kLdsTimers % 2 == 0, "blob table and timers must be 8-byte aligned");

__device__ __forceinline__ int32_t total_rows(const Layout& lay) {
    int32_t t = 0;
#pragma unroll
    for (int si = 0; si < 3; ++si) {
        if (si >= lay.n_sec) continue;
        const int32_t kind = ZTCP_SEC_FIELD(lay, si, kind);
        const int32_t rpu = code_rows_per_unit(kind) + (kind != kSecRaw ? 1 : 0);
        t += ZTCP_SEC_FIELD(lay, si, n_units) * rpu;
    }
    return t;
}

__device__ __forceinline__ void load_group(const uint8_t* p, uint32_t w[8]) {
    const uint4 a = ldg16(p, 0), b = ldg16(p, 1);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

// Issues the hot loads of half h of a code row: 16-element chunks
// [4h, 4h + 4) of the row's 4, 8 (int4, int4 per 32) or 2 (raw) chunks.
__device__ __forceinline__ void load_half(const EgressParams& p, const EgressPage& pg, const Row& row, int h,
                                          uint32_t (&w)[4][8]) {
    const int ng = chunks_per_row(row.s.kind);
    const uint8_t* src = row.s.src ? pg.v : pg.k;
    GroupCursor cur = group_cursor(row.u * row.s.nblk * ng + row.j * ng + 4 * h, row.s.gpv, row.s.col, p.head_dim);
    const uint32_t skip = (uint32_t)(p.head_dim - row.s.gpv * 16) * 2u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (i < ng) {
            load_group(src + cur.off, w[i]);
            cur.step(row.s.gpv, skip);
        }
    }
}

// Half h of a code row with four lanes per page: load i (0..7) gives lane
// 16 r + c quad 4 (i / 4) + r of page 16 (i % 4) + c, 64 contiguous bytes per
// page per load; row_untranspose then gives every lane its own page's eight
// quads.  Needs the half's four chunks contiguous (tq_row).
__device__ __forceinline__ void load_half_t(const EgressParams& p, const EgressPage& pg, const Row& row, int h,
                                            uint32_t (&w)[4][8]) {
    const int ng = chunks_per_row(row.s.kind);
    const GroupCursor cur = group_cursor(row.u * row.s.nblk * ng + row.j * ng + 4 * h, row.s.gpv, row.s.col, p.head_dim);
    const uint32_t r16 = (threadIdx.x >> 4 & 3u) * 16u;
    const uint8_t* pm[4];
    column_ptrs(row.s.src ? pg.v : pg.k, pm);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint4 v = ldg16(pm[i & 3] + cur.off + (uint32_t)(i >> 2) * 64u + r16, 0);
        w[i >> 1][(i & 1) * 4 + 0] = v.x;
        w[i >> 1][(i & 1) * 4 + 1] = v.y;
        w[i >> 1][(i & 1) * 4 + 2] = v.z;
        w[i >> 1][(i & 1) * 4 + 3] = v.w;
    }
}
__device__ __forceinline__ void row_untranspose(uint32_t (&w)[4][8]) {
    row_transpose(w[0], w[1]);
    row_transpose(w[2], w[3]);
}

struct ProducerCtx {
    const EgressParams* p;
    EgressPage pg;
    uint32_t n0, n1, n2;
    ChaChaNonceCache nc;
    uint32_t* lds;
    int lane;
    // Transposed row stores: store k of a row writes quad (lane & 3) of page
    // 16 k + (lane >> 2).  Past the last page of a partial workgroup the lane
    // writes page 0's quad instead, the same bytes page 0's own lane writes,
    // so every store is unconditional (a store under a branch makes the
    // compiler wait for all outstanding stores before the next row's loads).
    uint8_t* sb[4];   // blob of the page stored by store k
    uint32_t sq[4];   // byte offset of that page's quad inside a row slot
    Waiter wt;

    __device__ __forceinline__ void init_stores(int ppw) {
        const uint64_t* blobs = reinterpret_cast<const uint64_t*>(lds + kLdsBlobs);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int pr = 16 * k + (lane >> 2);
            const int pe = pr < ppw ? pr : 0;
            sb[k] = reinterpret_cast<uint8_t*>(blobs[pe]);
            sq[k] = quad_word(pe, lane & 3) * 4u;
        }
    }
};

// Stores one row slot to the blobs, each store instruction writing 64
// contiguous bytes of 16 pages.  The four quads are read first, so the row
// costs one LDS round trip.  The stores are issued after the next row's
// loads, so the wave's wait for those loads does not include them (vector
// memory operations complete in issue order).
__device__ __forceinline__ void store_row(const uint32_t* slot, const ProducerCtx& c, uint32_t blob_off) {
    uint4 x[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) x[k] = lds_quad_at(slot, c.sq[k]);
#pragma unroll
    for (int k = 0; k < 4; ++k) stg16(c.sb[k] + blob_off, c.lane & 3, x[k]);
}

// Quantizes groups w[0..3] (int8: 4 code words each, int4: 2) into pt[] and
// their fp16 scales into sc[] (two per word, low half first).
template <int DT, int BITS>
__device__ __forceinline__ void quant_half(const uint32_t (&w)[4][8], uint32_t* pt, uint32_t* sc) {
    constexpr int CW = BITS == 8 ? 4 : 2;
#pragma unroll
    for (int i = 0; i < 4; i += 2) {
        uint32_t qa[4], qb[4];
        const uint32_t sa = quant_group<DT, BITS>(w[i], qa);
        const uint32_t sbb = quant_group<DT, BITS>(w[i + 1], qb);
#pragma unroll
        for (int t = 0; t < CW; ++t) {
            pt[CW * i + t] = qa[t];
            pt[CW * (i + 1) + t] = qb[t];
        }
        sc[i / 2] = sa | (sbb << 16);
    }
}

// e4m3 groups w[0..3] into pt[0..15] and their scales into sc[0..1].
template <int DT>
__device__ __forceinline__ void quant_half_e4m3(const uint32_t (&w)[4][8], uint32_t* pt, uint32_t* sc) {
#pragma unroll
    for (int i = 0; i < 4; i += 2) {
        const uint32_t sa = quant_group_e4m3<DT>(w[i], pt + 4 * i);
        const uint32_t sbb = quant_group_e4m3<DT>(w[i + 1], pt + 4 * (i + 1));
        sc[i / 2] = sa | (sbb << 16);
    }
}

// Two int4 groups of 32 elements (chunks w[0..1], w[2..3]) into pt[0..7];
// returns their scales (first in the low half).
template <int DT>
__device__ __forceinline__ uint32_t quant_half_int4g32(const uint32_t (&w)[4][8], uint32_t* pt) {
    const uint32_t sa = quant_group32_int4<DT>(w[0], w[1], pt);
    const uint32_t sbb = quant_group32_int4<DT>(w[2], w[3], pt + 4);
    return sa | (sbb << 16);
}

// The scale row of unit g (payload block `block`), made by the storer wave
// once it has stored the unit's last code row: every code row of the unit
// stages its scales before it releases its ring row, so all of them are in
// the staging slot by then.  Encrypts the staged scales in place, stores the
// block transposed and frees the staging slot; that the stores have
// completed is published later (publish_scales).
__device__ __forceinline__ void encrypt_scale_row(const ProducerCtx& c, int32_t g, uint32_t block) {
    const EgressParams& p = *c.p;
    uint32_t ks[16];
    chacha_block_cached(p.key, c.nc, 1u + block, c.n0, c.n1, c.n2, ks);
    uint32_t* stage = c.lds + kLdsStage + (g % kStage) * kRowWords;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint4 s = lds_quad(stage, c.lane, q);
        lds_put_quad(stage, c.lane, q,
                     make_uint4(s.x ^ ks[4 * q], s.y ^ ks[4 * q + 1], s.z ^ ks[4 * q + 2], s.w ^ ks[4 * q + 3]));
    }
}
// Stores unit g's encrypted scale row (payload block `block`) from its
// staging slot and frees the slot.
__device__ __forceinline__ void store_scale_row(const ProducerCtx& c, int32_t g, uint32_t block) {
    uint32_t* flags = c.lds + kLdsFlags;
    store_row(c.lds + kLdsStage + (g % kStage) * kRowWords, c, (uint32_t)kHeader + 64u * block);
    publish(&flags[kFlagStage + g % kStage], (uint32_t)g + 1u);  // the release follows the slot reads
}

// Publishes that scale rows [from, to) are in the blobs, for the feeder.
__device__ __forceinline__ void publish_scales(uint32_t* flags, int32_t from, int32_t to) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's stores have completed
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
#pragma unroll 1
    for (int32_t g = from; g < to; ++g) publish(&flags[kFlagScale + g % kScaleSlots], (uint32_t)g + 1u);
}

// Whether a row of this kind quantizes eight 16-element chunks (int4, int4 per
// 32): those rows load their chunks in two halves of four.
template <int FAM>
__device__ __forceinline__ bool two_halves(int32_t kind) {
    return kind == kSecInt4 || (FAM == 2 && kind == kSecInt4G32);
}

// Quantizes a row's first four chunks (w) into pt[] and its parameter words
// into sc[] (raw rows copy their two chunks).
template <int DT, int FAM>
__device__ __forceinline__ void quant_first(int32_t kind, const uint32_t (&w)[4][8], uint32_t (&pt)[16],
                                            uint32_t (&sc)[4]) {
    if (kind == kSecInt8) {
        quant_half<DT, 8>(w, pt, sc);
    } else if (kind == kSecInt4) {
        quant_half<DT, 4>(w, pt, sc);
    } else if (FAM == 0 || kind == kSecRaw) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            pt[t] = w[0][t];
            pt[8 + t] = w[1][t];
        }
    } else if constexpr (FAM >= 1) {
        if (FAM == 1 || kind == kSecE4m3) quant_half_e4m3<DT>(w, pt, sc);
        else if constexpr (FAM == 2) {
            if (kind == kSecInt4G32) sc[0] = quant_half_int4g32<DT>(w, pt);
            else sc[0] = quant_group64_asym8<DT>(w, pt);
        }
    }
}

// The first half of a row's chunks: loads them, and once they have arrived
// quantizes them and issues the loads of the second half (rows of eight
// chunks), which then arrive during the row's first double rounds.  Run at
// the end of the previous row, whose last rounds cover the first half's
// loads.
// Whether a row's hot loads are made four lanes per page: the rows that read
// 256 hot bytes per page (int4, int4 per 32) when each half is four
// contiguous chunks (groups per vector a multiple of 4).  The rows of 128
// hot bytes per page (int8, e4m3, asym8) measured slower that way.
template <int FAM>
__device__ __forceinline__ bool tq_row(const Row& row) {
    return (row.s.gpv & 3) == 0 &&
           ((FAM == 0 && row.s.kind == kSecInt4) || (FAM == 2 && row.s.kind == kSecInt4G32));
}
template <int FAM>
__device__ __forceinline__ void load_half_any(const EgressParams& p, const EgressPage& pg, const Row& row, int h,
                                              uint32_t (&w)[4][8]) {
    if (tq_row<FAM>(row)) load_half_t(p, pg, row, h, w);
    else load_half(p, pg, row, h, w);
}

template <int DT, int FAM>
__device__ __forceinline__ void first_half(const EgressParams& p, const EgressPage& pg, const Row& row,
                                           uint32_t (&w)[4][8], uint32_t (&pt)[16], uint32_t (&sc)[4]) {
    if (tq_row<FAM>(row)) row_untranspose(w);
    quant_first<DT, FAM>(row.s.kind, w, pt, sc);
    if (two_halves<FAM>(row.s.kind)) load_half_any<FAM>(p, pg, row, 1, w);
}

// One code row.  pt / sc hold the row's first half quantized (first_half, at
// the end of the previous row) and w the second half's chunks when the row
// has two, loaded since; the second half is quantized after four double
// rounds.  The next row's first four chunks are loaded into w then, and at
// the end of this row first_half runs for the next row.  Every kind of row
// issues the next row's loads at the same point, into the same registers,
// so that no path has to move a register whose load is still in flight
// (such a move would make the wave wait for it).
template <int DT, int FAM>
__device__ __forceinline__ void code_row(const ProducerCtx& c, const Row& row, const Row& nxt,
                                         uint32_t (&w)[4][8], uint32_t (&pt)[16], uint32_t (&sc)[4]) {
    const EgressParams& p = *c.p;
    uint32_t* flags = c.lds + kLdsFlags;
    const int32_t kind = row.s.kind;
    ChaChaState st;
    st.start_cached(p.key, c.nc, 1u + (uint32_t)row.block);
    st.double_rounds<4>();
    // the priority is refreshed after four and after seven double rounds;
    // pin_words keeps the rounds on their side of each refresh
    pin_words(st.x);
    refresh_row_priority(&flags[kFlagMacUsed], row.mrow);
    // the second half's scale words go to variables of their own: stores
    // into sc at other indices than the first half's let the compiler merge
    // the two quantizer calls into one store at a runtime index, which puts
    // sc in scratch memory
    uint32_t s2 = 0u, s3 = 0u;
    if (two_halves<FAM>(kind) && tq_row<FAM>(row)) row_untranspose(w);  // the second half
    if (kind == kSecInt4) {
        uint32_t t[2];
        quant_half<DT, 4>(w, pt + 8, t);
        s2 = t[0];
        s3 = t[1];
    } else if (FAM == 2 && kind == kSecInt4G32) {
        s2 = quant_half_int4g32<DT>(w, pt + 8);
    }
    if (nxt.valid) load_half_any<FAM>(p, c.pg, nxt, 0, w);
    st.double_rounds<3>();
    pin_words(st.x);
    refresh_row_priority(&flags[kFlagMacUsed], row.mrow);
    st.double_rounds<2>();
    if (kind != kSecRaw) {
        // the unit's staging slot is free once unit g - kStage's scale row is done
        uint32_t* stage = c.lds + kLdsStage + (row.g % kStage) * kRowWords;
        wait_ge<kDiagEgressWait, kTmStageWait>(&flags[kFlagStage + row.g % kStage], row.g - kStage + 1, c.wt);
        // parameter words of this row: 2 (int8, e4m3, int4 per 32), 4 (int4)
        // or 1 (asym8), at logical words j * sw .. of this lane's page.  One
        // branch per count: a loop bounded by a runtime count would index sc
        // at run time and put it in scratch memory.
        const int sw = param_words_per_row(kind);
        if (sw == 4) {  // int4: two words per half
            stage[quad_word(c.lane, row.j) + 0] = sc[0];
            stage[quad_word(c.lane, row.j) + 1] = sc[1];
            stage[quad_word(c.lane, row.j) + 2] = s2;
            stage[quad_word(c.lane, row.j) + 3] = s3;
        } else if (sw == 2) {  // int8, e4m3: both words from the first half; int4 per 32: one per half
            const int wd = row.j * 2;
            const bool split = FAM == 2 && kind == kSecInt4G32;
            stage[quad_word(c.lane, wd >> 2) + (wd & 3)] = sc[0];
            stage[quad_word(c.lane, wd >> 2) + (wd & 3) + 1] = split ? s2 : sc[1];
        } else {
            stage[quad_word(c.lane, row.j >> 2) + (row.j & 3)] = sc[0];
        }
    }
    uint32_t ks[16];
    st.finish(p.key, 1u + (uint32_t)row.block, c.n0, c.n1, c.n2, ks);
    // the row's ciphertext is complete before the ring waits: left to
    // itself, the compiler sinks the last rounds below the waits (their
    // results are only used after them), so a wave that finds the ring full
    // would wait first and compute afterwards
#pragma unroll
    for (int i = 0; i < 16; ++i) ks[i] ^= pt[i];
    pin_words(ks);
    uint32_t* slot = c.lds + (row.mrow % kRing) * kRowWords;
    wait_ge<kDiagEgressWait, kTmRingWait>(&flags[kFlagMacUsed], row.mrow - kRing + 1, c.wt);
    wait_ge<kDiagEgressWait, kTmRingWait>(&flags[kFlagStored], row.mrow - kRing + 1, c.wt);
#pragma unroll
    for (int q = 0; q < 4; ++q)
        lds_put_quad(slot, c.lane, q, make_uint4(ks[4 * q], ks[4 * q + 1], ks[4 * q + 2], ks[4 * q + 3]));
    publish(&flags[kFlagRing + row.mrow % kRing], (uint32_t)row.mrow + 1u);  // the storer wave stores it
    tm_trace(c.wt.trace, row.mrow, c.wt.t0);
    if (nxt.valid) first_half<DT, FAM>(p, c.pg, nxt, w, pt, sc);
}

template <int DT, int FAM>
__device__ void egress_produce(const EgressParams& p, int64_t page0, int ppw, uint32_t* lds) {
    ProducerCtx c;
    c.p = &p;
    c.lane = threadIdx.x & 63;
    c.pg = egress_page(p, page0 + (c.lane < ppw ? c.lane : 0));
    c.n0 = (uint32_t)c.pg.seq;
    c.n1 = (uint32_t)(c.pg.seq >> 32);
    c.n2 = c.pg.nonce2;
    c.nc.init(p.key, c.n0, c.n1, c.n2);
    c.lds = lds;
    c.wt = make_waiter(p.sink, lds + kLdsFlags + kFlagExpired, lds + kLdsTimers, phase_clock());
    c.wt.trace = trace_of(p.timers);
    const int32_t total = total_code_rows(p.lay);
    // The page descriptor and kernel argument loads above complete here,
    // before the loop: a load still counted as in flight where the loop
    // begins makes the compiler wait for every outstanding memory operation
    // wherever the loop uses its result.
    __builtin_amdgcn_s_waitcnt(0);
    if constexpr (kPhaseTimers) tm_min(c.wt.tm, kTmProdSetup, phase_clock() - c.wt.t0);
    uint32_t* flags = lds + kLdsFlags;
    // code rows are handed out in order from an LDS counter, one row ahead of
    // the one being made (so its groups can be prefetched): a slower wave
    // simply takes fewer rows
    // (also reads how many rows the MAC wave has absorbed, for the priority)
    int32_t used = 0;
    auto grab = [&]() -> int32_t {
        uint32_t t = 0;
        const uint32_t u = __hip_atomic_load(&flags[kFlagMacUsed], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (c.lane == 0)
            t = __hip_atomic_fetch_add(&flags[kFlagTask], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        used = (int32_t)__builtin_amdgcn_readfirstlane(u);
        return (int32_t)__builtin_amdgcn_readfirstlane(t);
    };
    uint32_t w[4][8];
    uint32_t pt[16], sc[4];
    int32_t t = grab();
    Row cur = row_info(p.lay, t);
    if (cur.valid) {
        load_half_any<FAM>(p, c.pg, cur, 0, w);
        first_half<DT, FAM>(p, c.pg, cur, w, pt, sc);
        if constexpr (kPhaseTimers) tm_min(c.wt.tm, kTmProdLoaded, phase_clock() - c.wt.t0);
    }
    [[maybe_unused]] int32_t made = 0;
#pragma unroll 1
    while (t < total) {
        const int32_t tn = grab();
        set_row_priority(cur.mrow - used);
        const Row nxt = row_info(p.lay, tn);
        code_row<DT, FAM>(c, cur, nxt, w, pt, sc);
        if constexpr (kPhaseTimers) {
            if (made++ == 0) tm_min(c.wt.tm, kTmProdFirstRow, phase_clock() - c.wt.t0);
        }
        t = tn;
        cur = nxt;
    }
    if constexpr (kPhaseTimers) {
        const uint64_t now = phase_clock() - c.wt.t0;
        tm_max(c.wt.tm, kTmProdLast, now);
        tm_add(c.wt.tm, kTmProdBusy, now);
        tm_add(c.wt.tm, kTmProdWaves, 1);
        tm_add(c.wt.tm, kTmRows, (uint64_t)made);
    }
}

// Section sizes of the page layout in scalar registers: code rows and scale
// rows per section, and the payload offset of each section's scales.  The
// values pass through an empty asm so that the compiler keeps them in
// registers instead of reloading them from the kernel arguments inside the
// MAC loop (a scalar load there would make the wave wait for its LDS reads).
struct MacPlan {
    int32_t nc0, nc1, nc2;     // code rows per section
    int32_t ns0, ns1, ns2;     // scale rows per section (0 for raw sections)
    uint32_t so0, so1, so2;    // payload offset of the section's scales
    int32_t total;             // rows absorbed after the header

    __device__ __forceinline__ void init(const Layout& lay) {
        int32_t nc[3], ns[3];
        uint32_t so[3];
#pragma unroll
        for (int si = 0; si < 3; ++si) {
            const bool on = si < lay.n_sec;
            const int32_t kind = ZTCP_SEC_FIELD(lay, si, kind);
            const int32_t nu = ZTCP_SEC_FIELD(lay, si, n_units);
            nc[si] = on ? nu * code_rows_per_unit(kind) : 0;
            ns[si] = on && kind != kSecRaw ? nu : 0;
            so[si] = ZTCP_SEC_FIELD(lay, si, s_off);
        }
        nc0 = nc[0]; nc1 = nc[1]; nc2 = nc[2];
        ns0 = ns[0]; ns1 = ns[1]; ns2 = ns[2];
        so0 = so[0]; so1 = so[1]; so2 = so[2];
        asm volatile("" : "+s"(nc0), "+s"(nc1), "+s"(nc2), "+s"(ns0), "+s"(ns1), "+s"(ns2));
        asm volatile("" : "+s"(so0), "+s"(so1), "+s"(so2));
        total = nc0 + nc1 + nc2 + ns0 + ns1 + ns2;
    }
    __device__ __forceinline__ int32_t nc(int32_t si) const { return si == 0 ? nc0 : (si == 1 ? nc1 : (si == 2 ? nc2 : 0)); }
    __device__ __forceinline__ int32_t ns(int32_t si) const { return si == 0 ? ns0 : (si == 1 ? ns1 : (si == 2 ? ns2 : 0)); }
};

template <int DT>
__device__ void egress_mac(const EgressParams& p, int64_t page0, int ppw, uint32_t* lds, uint64_t t0) {
    const int lane = threadIdx.x & 63;
    const bool active = lane < ppw;
    const EgressPage pg = egress_page(p, page0 + (active ? lane : 0));
    uint8_t* blob = pg.blob;
    if (active) {  // header (cpp:1129-1140)
        stg16(blob, 0, make_uint4((uint32_t)p.hdr0, (uint32_t)(p.hdr0 >> 32), (uint32_t)pg.hdr1,
                                  (uint32_t)(pg.hdr1 >> 32)));
        stg16(blob, 1, make_uint4((uint32_t)pg.token, (uint32_t)(pg.token >> 32), (uint32_t)pg.seq,
                                  (uint32_t)(pg.seq >> 32)));
    }
    Sip s;
    s.init(p.mk0, p.mk1);
    const uint64_t hdr[4] = {p.hdr0, pg.hdr1, pg.token, pg.seq};
    s.absorb_words<4>(hdr);
    PageQuads pq;
    pq.init(lane);
    MacPlan m;
    m.init(p.lay);
    // Rows arrive in MAC order in the ring (code rows from the producers,
    // scale rows from the feeder), so the next row is always the next slot.
    Waiter wt = make_waiter(p.sink, lds + kLdsFlags + kFlagExpired, lds + kLdsTimers, t0);
    wt.trace = trace_of(p.timers);
    __builtin_amdgcn_s_waitcnt(0);
    if constexpr (kPhaseTimers) tm_add(wt.tm, kTmMacRowsBegin, phase_clock() - t0);
    mac_rows<kRing, kDiagEgressWait>(wt, lds, lds + kLdsFlags + kFlagRing, lds + kLdsFlags + kFlagMacUsed, pq, s,
                                     m.total);
    if constexpr (kPhaseTimers) tm_add(wt.tm, kTmMacRowsEnd, phase_clock() - t0);
    uint64_t lo, hi;
    s.finish((uint64_t)((kHeader + p.payload) & 0xFFu) << 56, lo, hi);
    if (active)
        stg16(blob + kHeader + p.payload, 0,
              make_uint4((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)));
    if constexpr (kPhaseTimers) tm_add(wt.tm, kTmMacEnd, phase_clock() - t0);
}

// Scale-row feeder (a wave on the MAC wave's SIMD, almost idle): copies each
// section's encrypted scale rows from the blobs into the ring, at their place
// in the MAC wave's order, where the MAC wave reads them like code rows.  A scale row is stored long
// before the MAC wave reaches it (after all of its section's code rows), so
// it is no longer in L2; the feeder takes that latency instead of the MAC
// chain.  Within a section the next row's loads are in flight while the
// current one is written; a section's first row is never waited for before
// the previous section's rows are all in the ring, so the MAC wave never
// depends on a row that needs it to progress first.
__device__ __forceinline__ void feed_load(const Waiter& wt, const uint32_t* lds, const uint8_t* src,
                                          int32_t g, uint4 (&x)[4]) {
    wait_ge<kDiagEgressWait, kTmFeedWait>(lds + kLdsFlags + kFlagScale + g % kScaleSlots, g + 1, wt);
    if (src) {
#pragma unroll
        for (int q = 0; q < 4; ++q) x[q] = ldg16(src, q);
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) x[q] = make_uint4(0u, 0u, 0u, 0u);
    }
}

__device__ __forceinline__ void feed_put(const Waiter& wt, uint32_t* lds, const PageQuads& pq, int32_t rs,
                                         const uint4 (&x)[4]) {
    uint32_t* flags = lds + kLdsFlags;
    wait_ge<kDiagEgressWait, kTmFeedWait>(&flags[kFlagMacUsed], rs - kRing + 1, wt);
    wait_ge<kDiagEgressWait, kTmFeedWait>(&flags[kFlagStored], rs - kRing + 1, wt);
    uint32_t* slot = lds + (rs % kRing) * kRowWords;
#pragma unroll
    for (int q = 0; q < 4; ++q) lds_put_quad_at(slot, pq.off[q], x[q]);
    publish(&flags[kFlagRing + rs % kRing], (uint32_t)rs + 1u);
    tm_trace(wt.trace, rs, wt.t0);
}

__device__ void egress_scale_feed(const EgressParams& p, uint32_t* lds) {
    const int lane = threadIdx.x & 63;
    const uint8_t* blob = reinterpret_cast<const uint8_t*>(reinterpret_cast<const uint64_t*>(lds + kLdsBlobs)[lane]);
    PageQuads pq;
    pq.init(lane);
    MacPlan m;
    m.init(p.lay);
    Waiter wt = make_waiter(p.sink, lds + kLdsFlags + kFlagExpired, lds + kLdsTimers, phase_clock());
    wt.trace = trace_of(p.timers);
    int32_t g0 = 0, r0 = 0;  // scale rows / MAC rows before the section
#pragma unroll
    for (int si = 0; si < 3; ++si) {
        const int32_t n = m.ns(si);
        const int32_t rs = r0 + m.nc(si);  // MAC row of the section's first scale row
        const uint32_t so = si == 0 ? m.so0 : (si == 1 ? m.so1 : m.so2);
        const uint8_t* base = blob ? blob + kHeader + so : nullptr;
        uint4 a[4], b[4];
        if (n > 0) feed_load(wt, lds, base, g0, a);
#pragma unroll 1
        for (int32_t j = 0; j < n; j += 2) {
            if (j + 1 < n) feed_load(wt, lds, base ? base + 64u * (uint32_t)(j + 1) : nullptr, g0 + j + 1, b);
            feed_put(wt, lds, pq, rs + j, a);
            if (j + 1 >= n) break;
            if (j + 2 < n) feed_load(wt, lds, base ? base + 64u * (uint32_t)(j + 2) : nullptr, g0 + j + 2, a);
            feed_put(wt, lds, pq, rs + j + 1, b);
        }
        g0 += n;
        r0 = rs + n;
    }
    if constexpr (kPhaseTimers) tm_max(wt.tm, kTmFeedEnd, phase_clock() - wt.t0);
}

// Storer (one wave on SIMD 1): stores every code row from the ring to the
// blobs, in payload order (the MAC order), transposed -- four lanes per page,
// 64 contiguous bytes of 16 pages per store instruction -- and publishes
// `stored` = rows passed; a ring slot is rewritten only once the MAC wave and
// the storer have both passed it.  Once it has stored a unit's last code row
// it also makes the unit's scale row (every code row stages its scales before
// releasing its ring row), so the producers never wait for a unit to fill.
// A section's scale rows are neighbours in the blob: the storer keeps each
// encrypted one in its staging slot until it has made the next ones and
// stores them kScaleGroup at a time (the section's last ones as they come),
// so that the 128-byte lines they share are written at once instead of one
// unit apart, when the first half is often evicted and written back alone.
// Holding them creates no cycle of waits: the MAC wave reaches a section's
// scale rows after all of its code rows, and a producer of unit g waits for
// the slot of unit g - kStage, which is stored at the latest with unit
// g - kStage + kScaleGroup - 1, a unit before g (kScaleGroup <= kStage).
// That a scale row's stores have completed is published for the feeder
// before the storer next waits for a row, or once four are outstanding: the
// storer issues no loads, so those waits only cover its own stores.  Stores
// are kept off the producers, whose waits for their own loads would
// otherwise also wait for every store they issued before those loads, and
// off the MAC wave's SIMD, where the data and address reads of scattered
// stores take register-file cycles from the chain.
__device__ void egress_store_rows(const EgressParams& p, int64_t page0, int ppw, uint32_t* lds) {
    ProducerCtx c;
    c.p = &p;
    c.lane = threadIdx.x & 63;
    c.pg = egress_page(p, page0 + (c.lane < ppw ? c.lane : 0));
    c.n0 = (uint32_t)c.pg.seq;
    c.n1 = (uint32_t)(c.pg.seq >> 32);
    c.n2 = c.pg.nonce2;
    c.nc.init(p.key, c.n0, c.n1, c.n2);
    c.lds = lds;
    c.wt = make_waiter(p.sink, lds + kLdsFlags + kFlagExpired, lds + kLdsTimers, phase_clock());
    c.init_stores(ppw);
    uint32_t* flags = lds + kLdsFlags;
    // a slot is reused only once stored: never let the producers sharing
    // this SIMD starve the storer
    __builtin_amdgcn_s_setprio(2);
    __builtin_amdgcn_s_waitcnt(0);
    int32_t r = 0, g0 = 0;      // payload row; quantized units before the section
    int32_t made = 0, pub = 0;  // scale rows made / published as stored
    int32_t held = 0;           // encrypted scale rows waiting in their slots for the rest of their group
#pragma unroll
    for (int si = 0; si < 3; ++si) {
        if (si >= p.lay.n_sec) continue;
        const int32_t kind = ZTCP_SEC_FIELD(p.lay, si, kind);
        const int32_t nu = ZTCP_SEC_FIELD(p.lay, si, n_units);
        const int32_t nblk = code_rows_per_unit(kind);  // 4, 8 or 16
        const uint32_t sblk = ZTCP_SEC_FIELD(p.lay, si, s_off) / 64u;
        const bool quant = kind != kSecRaw;
        const int32_t ncode = nu * nblk;
#pragma unroll 1
        for (int32_t cr = 0; cr < ncode; ++cr, ++r) {
            const uint32_t* f = &flags[kFlagRing + r % kRing];
            if (pub < made &&
                (int32_t)__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < r + 1) {
                publish_scales(flags, pub, made);
                pub = made;
            }
            wait_ge<kDiagEgressWait, kTmStorerWait>(f, r + 1, c.wt);
            store_row(lds + (r % kRing) * kRowWords, c, (uint32_t)kHeader + 64u * (uint32_t)r);
            publish(&flags[kFlagStored], (uint32_t)r + 1u);  // the release orders the slot reads before it
            if (quant && (cr & (nblk - 1)) == nblk - 1) {
                const int32_t u = cr / nblk;
                encrypt_scale_row(c, g0 + u, sblk + (uint32_t)u);
                if (held < kScaleGroup - 1 && u + 1 < nu) {
                    ++held;
                } else {
#pragma unroll 1
                    for (int32_t h = u - held; h <= u; ++h) store_scale_row(c, g0 + h, sblk + (uint32_t)h);
                    made += held + 1;
                    held = 0;
                    if (made - pub >= 4) {
                        publish_scales(flags, pub, made);
                        pub = made;
                    }
                }
            }
        }
        if (quant) {  // the section's scale rows reach the ring through the feeder
#pragma unroll 1
            for (int32_t i = 0; i < nu; ++i, ++r) publish(&flags[kFlagStored], (uint32_t)r + 1u);
            g0 += nu;
        }
    }
    publish_scales(flags, pub, made);
    if constexpr (kPhaseTimers) tm_max(c.wt.tm, kTmStorerEnd, phase_clock() - c.wt.t0);
}

// FAM 0: the reference's section kinds (int8, int4, raw); FAM 1: also e4m3
// (16 waves, as FAM 0); FAM 2: also int4 per 32 and asym8, whose 32- and
// 64-element groups need the most registers (12 waves, 168 VGPRs each).
// Separate instantiations keep each kind's registers out of the kernels of
// layouts that do not use it.
template <int DT, int FAM>
__global__ __launch_bounds__(64 * egress_waves<FAM>()) void egress_fused_kernel(EgressParams p) {
    extern __shared__ __align__(16) uint32_t lds[];
    const int64_t page0 = (int64_t)blockIdx.x * p.ppw;
    const int ppw = (int)min((int64_t)p.ppw, p.batch - page0);
    for (int i = threadIdx.x; i < kNumFlags; i += blockDim.x) lds[kLdsFlags + i] = 0u;
    tm_clear(lds + kLdsTimers);
    tm_trace_clear(p.timers);
    if (threadIdx.x < 64) {
        uint64_t* blobs = reinterpret_cast<uint64_t*>(lds + kLdsBlobs);
        blobs[threadIdx.x] = (int)threadIdx.x < ppw ? reinterpret_cast<uint64_t>(egress_page(p, page0 + threadIdx.x).blob)
                                                    : 0ull;  // null past the last page
    }
    __syncthreads();
    [[maybe_unused]] const uint64_t t0 = phase_clock();
    [[maybe_unused]] const uint64_t rt0 = kPhaseTimers ? __builtin_amdgcn_s_memrealtime() : 0;
    const int wave = threadIdx.x >> 6;
    if (wave == 0) {
        __builtin_amdgcn_s_setprio(3);
        egress_mac<DT>(p, page0, ppw, lds, t0);
    } else if (wave == 4) {
        egress_scale_feed(p, lds);
    } else if ((wave & 3) == 0) {
        // the rest of the MAC wave's SIMD stays idle
    } else if (wave == 1) {
        egress_store_rows(p, page0, ppw, lds);
    } else {
        egress_produce<DT, FAM>(p, page0, ppw, lds);
    }
    // Fail closed: if any bounded wait of the workgroup expired, its rows may
    // have been read or overwritten out of turn, so no blob of the workgroup
    // may verify.  The MAC wave's lanes, which stored the headers, zero the
    // first 16 header bytes (magic 0: every ingress rejects the page with
    // status 1).  Same lanes, same addresses: the stores stay in order.
    __syncthreads();
    tm_flush(lds + kLdsTimers, p.timers, t0, rt0);
    if (__hip_atomic_load(lds + kLdsFlags + kFlagExpired, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0u &&
        (int)threadIdx.x < ppw) {
        uint8_t* blob = reinterpret_cast<uint8_t*>(reinterpret_cast<const uint64_t*>(lds + kLdsBlobs)[threadIdx.x]);
        stg16(blob, 0, make_uint4(0u, 0u, 0u, 0u));
    }
}

// ---------------------------------------------------------------------------
// Small batches (at most kSmallMaxPpw pages per workgroup, reference kinds).
// With a few pages per workgroup, lane = page leaves most lanes of the
// producer waves idle, and each row still costs a whole wave's keystream
// block: the chain then waits for rows made one page at a time.  Here lane
// = (code row, page) instead: three producer waves make the code rows of
// every page 192 at a time (load, quantize, keystream, XOR), write each to
// the blob and to a copy of the page's whole payload in LDS, and stage its
// scales; once every code row is made they encrypt the scale rows the same
// way.  The MAC wave (0, one page per lane) absorbs the payload in order
// from LDS as the producers' passes complete, two rows of LDS reads ahead,
// so it never reads global memory and waits only for the first pass.
// ---------------------------------------------------------------------------
constexpr int kSmallWaves = 4;        // MAC wave + three producer waves
constexpr int kSmRowWords = 16;       // one 64-byte payload row of one page
constexpr int kSmallMaxPpw = 4;       // pages per workgroup up to which the small kernel runs
constexpr int kSmallTasks = 64 * (kSmallWaves - 1);  // tasks per producer pass
constexpr int kSmFlagPass = 0;        // [3] passes completed by producer wave 1..3
constexpr int kSmFlagScales = 3;      // producer waves done with the scale rows
constexpr int kSmFlagExpired = 4;     // 1: a bounded wait of the workgroup expired
constexpr int kSmFlags = 16;          // flag words
constexpr int kSmPay = kSmFlags + kTimerLdsWords;  // the payload copy (64-byte aligned)

// Payload block of the scale row of quantized unit g (staging order).
__device__ __forceinline__ int32_t scale_block(const Layout& lay, int32_t g) {
    int32_t blk = 0, q = 0;
    bool found = false;
#pragma unroll
    for (int si = 0; si < 3; ++si) {
        if (si >= lay.n_sec || found) continue;
        if (ZTCP_SEC_FIELD(lay, si, kind) == kSecRaw) continue;
        const int32_t nu = ZTCP_SEC_FIELD(lay, si, n_units);
        if (g < q + nu) {
            blk = (int32_t)(ZTCP_SEC_FIELD(lay, si, s_off) / 64u) + (g - q);
            found = true;
        }
        q += nu;
    }
    return blk;
}

__device__ __forceinline__ void put_row(uint32_t* lds_row, uint8_t* blob_row, const uint32_t (&x)[16]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint4 v = make_uint4(x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]);
        *reinterpret_cast<uint4*>(lds_row + 4 * q) = v;
        stg16(blob_row, q, v);
    }
}

// Producer wave pw (0..2).  Task t of pass k = 192 k + 64 pw + lane is code
// row t / ppw of page t % ppw, so a pass holds whole rows of every page.
template <int DT>
__device__ void small_produce(const EgressParams& p, int64_t page0, int ppw, int32_t nrow, int32_t nq,
                              uint32_t* lds, uint64_t t0) {
    const int pw = (int)(threadIdx.x >> 6) - 1;
    const int lane = threadIdx.x & 63;
    uint32_t* flags = lds;
    uint32_t* pay = lds + kSmPay;
    uint32_t* stage = pay + (size_t)ppw * nrow * kSmRowWords;
    const Waiter wt = make_waiter(p.sink, flags + kSmFlagExpired, lds + kSmFlags, t0);
    const int32_t ntask = total_code_rows(p.lay) * ppw;
    const int32_t npass = (ntask + kSmallTasks - 1) / kSmallTasks;
#pragma unroll 1
    for (int32_t k = 0; k < npass; ++k) {
        const int32_t t = k * kSmallTasks + pw * 64 + lane;
        if (t < ntask) {
            const int32_t i = t % ppw;
            const Row row = row_info(p.lay, t / ppw);
            const EgressPage pg = egress_page(p, page0 + i);
            // both halves' loads first, then the keystream while they are in flight
            uint32_t w[4][8], w2[4][8], pt[16], sc[4];
            const bool two = row.s.kind == kSecInt4;
            load_half(p, pg, row, 0, w);
            if (two) load_half(p, pg, row, 1, w2);
            uint32_t ks[16];
            chacha_block(p.key, 1u + (uint32_t)row.block, (uint32_t)pg.seq, (uint32_t)(pg.seq >> 32), pg.nonce2, ks);
            quant_first<DT, 0>(row.s.kind, w, pt, sc);
            uint32_t s2 = 0u, s3 = 0u;
            if (two) {
                uint32_t t2[2];
                quant_half<DT, 4>(w2, pt + 8, t2);
                s2 = t2[0];
                s3 = t2[1];
            }
#pragma unroll
            for (int q = 0; q < 16; ++q) ks[q] ^= pt[q];
            put_row(pay + ((size_t)i * nrow + row.block) * kSmRowWords, pg.blob + kHeader + 64u * (uint32_t)row.block,
                    ks);
            // the unit's 16 parameter words: 2 per int8 row, 4 per int4 row
            uint32_t* st = stage + ((size_t)i * nq + row.g) * kSmRowWords;
            if (row.s.kind == kSecInt4) {
                st[4 * row.j + 0] = sc[0];
                st[4 * row.j + 1] = sc[1];
                st[4 * row.j + 2] = s2;
                st[4 * row.j + 3] = s3;
            } else if (row.s.kind == kSecInt8) {
                st[2 * row.j + 0] = sc[0];
                st[2 * row.j + 1] = sc[1];
            }
        }
        publish(&flags[kSmFlagPass + pw], (uint32_t)k + 1u);
        if constexpr (kPhaseTimers) {
            if (k == 0) tm_min(wt.tm, kTmProdFirstRow, phase_clock() - t0);
        }
    }
    // scale rows, once every wave has staged all of its scales
#pragma unroll 1
    for (int w2 = 0; w2 < kSmallWaves - 1; ++w2) wait_ge<kDiagEgressWait>(&flags[kSmFlagPass + w2], npass, wt);
    const int32_t nst = nq * ppw;
#pragma unroll 1
    for (int32_t t = pw * 64 + lane; t < nst; t += kSmallTasks) {
        const int32_t i = t % ppw, g = t / ppw;
        const EgressPage pg = egress_page(p, page0 + i);
        const int32_t blk = scale_block(p.lay, g);
        uint32_t ks[16];
        chacha_block(p.key, 1u + (uint32_t)blk, (uint32_t)pg.seq, (uint32_t)(pg.seq >> 32), pg.nonce2, ks);
        const uint32_t* st = stage + ((size_t)i * nq + g) * kSmRowWords;
#pragma unroll
        for (int q = 0; q < 16; ++q) ks[q] ^= st[q];
        put_row(pay + ((size_t)i * nrow + blk) * kSmRowWords, pg.blob + kHeader + 64u * (uint32_t)blk, ks);
    }
    __builtin_amdgcn_s_waitcnt(0);
    if (lane == 0) __hip_atomic_fetch_add(&flags[kSmFlagScales], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    if constexpr (kPhaseTimers) {
        tm_max(wt.tm, kTmProdLast, phase_clock() - t0);
        tm_add(wt.tm, kTmProdWaves, 1);
    }
}

// The MAC wave: header, then payload rows 0..nrow-1 of page `lane` from LDS.
// A code row is read once the pass holding its last page's task is complete
// in all three producer waves, a scale row once every wave has made its
// scale rows.
template <int DT>
__device__ void small_mac(const EgressParams& p, int64_t page0, int ppw, int32_t nrow, uint32_t* lds, uint64_t t0) {
    const int lane = threadIdx.x & 63;
    const bool active = lane < ppw;
    const EgressPage pg = egress_page(p, page0 + (active ? lane : 0));
    uint32_t* flags = lds;
    const uint32_t* mine = lds + kSmPay + (size_t)(active ? lane : 0) * nrow * kSmRowWords;
    if (active) {  // header (cpp:1129-1140)
        stg16(pg.blob, 0, make_uint4((uint32_t)p.hdr0, (uint32_t)(p.hdr0 >> 32), (uint32_t)pg.hdr1,
                                     (uint32_t)(pg.hdr1 >> 32)));
        stg16(pg.blob, 1, make_uint4((uint32_t)pg.token, (uint32_t)(pg.token >> 32), (uint32_t)pg.seq,
                                     (uint32_t)(pg.seq >> 32)));
    }
    Sip s;
    s.init(p.mk0, p.mk1);
    const uint64_t hdr[4] = {p.hdr0, pg.hdr1, pg.token, pg.seq};
    s.absorb_words<4>(hdr);
    const Waiter wt = make_waiter(p.sink, flags + kSmFlagExpired, lds + kSmFlags, t0);
    const int32_t ncode = total_code_rows(p.lay);
    int32_t r = 0;         // payload rows fetched
    int32_t c = 0;         // code rows absorbed
    int32_t ready = 0;     // code rows complete for every page
    bool scales = false;   // scale rows complete
    auto fetch = [&](uint4 (&x)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) x[q] = *reinterpret_cast<const uint4*>(mine + r * kSmRowWords + 4 * q);
        ++r;
    };
    __builtin_amdgcn_s_waitcnt(0);
    if constexpr (kPhaseTimers) tm_add(wt.tm, kTmMacRowsBegin, phase_clock() - t0);
    // Sections in payload order, each its code rows then its scale rows; the
    // code rows in runs that end where the completed passes end, so the
    // loop itself has no per-row test.
#pragma unroll 1
    for (int si = 0; si < 3; ++si) {
        if (si >= p.lay.n_sec) continue;
        const int32_t kind = ZTCP_SEC_FIELD(p.lay, si, kind);
        const int32_t nu = ZTCP_SEC_FIELD(p.lay, si, n_units);
        int32_t left = nu * code_rows_per_unit(kind);
#pragma unroll 1
        while (left > 0) {
            if (c >= ready) {
                [[maybe_unused]] const uint64_t t_in = phase_clock();
                const int32_t need = (c * ppw + ppw - 1) / kSmallTasks + 1;  // passes
#pragma unroll 1
                for (int w2 = 0; w2 < kSmallWaves - 1; ++w2)
                    wait_ge<kDiagEgressWait>(&flags[kSmFlagPass + w2], need, wt);
                ready = min(ncode, need * kSmallTasks / ppw);
                if constexpr (kPhaseTimers) {
                    tm_add(wt.tm, kTmMacWait + min(r >> 6, 7), phase_clock() - t_in);
                    if (c == 0) tm_add(wt.tm, kTmMacFirstRow, phase_clock() - t0);
                }
            }
            const int32_t n = min(left, ready - c);
            sip_stream64(s, (uint32_t)n, fetch);
            c += n;
            left -= n;
        }
        if (kind != kSecRaw) {
            if (!scales) {
                [[maybe_unused]] const uint64_t t_in = phase_clock();
                wait_ge<kDiagEgressWait>(&flags[kSmFlagScales], kSmallWaves - 1, wt);
                scales = true;
                if constexpr (kPhaseTimers) tm_add(wt.tm, kTmMacWait + min(r >> 6, 7), phase_clock() - t_in);
            }
            sip_stream64(s, (uint32_t)nu, fetch);
        }
    }
    if constexpr (kPhaseTimers) tm_add(wt.tm, kTmMacRowsEnd, phase_clock() - t0);
    uint64_t lo, hi;
    s.finish((uint64_t)((kHeader + p.payload) & 0xFFu) << 56, lo, hi);
    if (active)
        stg16(pg.blob + kHeader + p.payload, 0,
              make_uint4((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)));
    if constexpr (kPhaseTimers) tm_add(wt.tm, kTmMacEnd, phase_clock() - t0);
}

template <int DT>
__global__ __launch_bounds__(64 * kSmallWaves) void egress_small_kernel(EgressParams p) {
    extern __shared__ __align__(16) uint32_t lds[];
    const int64_t page0 = (int64_t)blockIdx.x * p.ppw;
    const int ppw = (int)min((int64_t)p.ppw, p.batch - page0);
    const int32_t nrow = (int32_t)(p.payload / 64u);
    const int32_t nq = nrow - total_code_rows(p.lay);
    if (threadIdx.x < kSmFlags) lds[threadIdx.x] = 0u;
    tm_clear(lds + kSmFlags);
    __syncthreads();
    [[maybe_unused]] const uint64_t t0 = phase_clock();
    [[maybe_unused]] const uint64_t rt0 = kPhaseTimers ? __builtin_amdgcn_s_memrealtime() : 0;
    if (threadIdx.x < 64) {
        __builtin_amdgcn_s_setprio(3);
        small_mac<DT>(p, page0, ppw, nrow, lds, t0);
    } else {
        small_produce<DT>(p, page0, ppw, nrow, nq, lds, t0);
    }
    // fail closed, as in egress_fused_kernel: the MAC lanes zero the headers
    __syncthreads();
    tm_flush(lds + kSmFlags, p.timers, t0, rt0);
    if (__hip_atomic_load(lds + kSmFlagExpired, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0u &&
        (int)threadIdx.x < ppw)
        stg16(egress_page(p, page0 + threadIdx.x).blob, 0, make_uint4(0u, 0u, 0u, 0u));
}

}  // namespace

// Zeroes every blob of a call (a synchronous egress whose bounded wait
// expired: fail closed, as the reference's wrapper zeroes out_blobs on any
// failure, nfc:597-600).  One workgroup per page, 16 bytes per thread.
__global__ void egress_zero_blobs_kernel(EgressParams p) {
    uint8_t* blob = egress_page(p, (int64_t)blockIdx.x).blob;
    for (uint32_t i = threadIdx.x; i < p.blob_bytes / 16u; i += blockDim.x) stg16(blob, i, make_uint4(0u, 0u, 0u, 0u));
    for (uint32_t i = (p.blob_bytes & ~15u) + threadIdx.x; i < p.blob_bytes; i += blockDim.x) blob[i] = 0;
}

size_t egress_fused_lds_bytes() { return (size_t)kLdsWords * sizeof(uint32_t); }

hipError_t launch_egress_zero_blobs(const EgressParams& p, hipStream_t s) {
    if (p.batch > 0x7FFFFFFF) return hipErrorInvalidValue;
    hipLaunchKernelGGL(egress_zero_blobs_kernel, dim3((uint32_t)p.batch), dim3(256), 0, s, p);
    return hipGetLastError();
}

// LDS of egress_small_kernel: flags, the payload of every page and the
// staged parameters of every quantized unit.
static size_t egress_small_lds_bytes(const EgressParams& p) {
    int64_t nq = 0;
    for (int si = 0; si < p.lay.n_sec; ++si)
        if (p.lay.sec[si].kind != kSecRaw) nq += p.lay.sec[si].n_units;
    return sizeof(uint32_t) * ((size_t)kSmPay + (size_t)p.ppw * (p.payload / 64u + (size_t)nq) * kSmRowWords);
}

hipError_t launch_egress_fused(const EgressParams& p, int dtype, hipStream_t s) {
    const int64_t grid = (p.batch + p.ppw - 1) / p.ppw;
    const size_t lds = egress_fused_lds_bytes();  // above 64 KiB: gfx950 has 160 KiB per CU
    int fam = 0;  // the kind family of the layout (egress_fused_kernel)
    for (int si = 0; si < p.lay.n_sec; ++si) {
        const int32_t kind = p.lay.sec[si].kind;
        if (kind == kSecAsym8 || kind == kSecInt4G32) fam = 2;
        else if (is_extension_kind(kind) && fam < 1) fam = 1;
    }
    const size_t small_lds = egress_small_lds_bytes(p);
    if (fam == 0 && p.ppw <= kSmallMaxPpw && small_lds <= 160u * 1024u) {
        const dim3 g((uint32_t)grid), b(64 * kSmallWaves);
        if (dtype == kHotBf16) hipLaunchKernelGGL(egress_small_kernel<kHotBf16>, g, b, small_lds, s, p);
        else hipLaunchKernelGGL(egress_small_kernel<kHotFp16>, g, b, small_lds, s, p);
        return hipGetLastError();
    }
    const dim3 g((uint32_t)grid),
        b((uint32_t)(64 * (fam == 0 ? egress_waves<0>() : (fam == 1 ? egress_waves<1>() : egress_waves<2>()))));
    if (dtype == kHotBf16) {
        if (fam == 2) hipLaunchKernelGGL((egress_fused_kernel<kHotBf16, 2>), g, b, lds, s, p);
        else if (fam == 1) hipLaunchKernelGGL((egress_fused_kernel<kHotBf16, 1>), g, b, lds, s, p);
        else hipLaunchKernelGGL((egress_fused_kernel<kHotBf16, 0>), g, b, lds, s, p);
    } else {
        if (fam == 2) hipLaunchKernelGGL((egress_fused_kernel<kHotFp16, 2>), g, b, lds, s, p);
        else if (fam == 1) hipLaunchKernelGGL((egress_fused_kernel<kHotFp16, 1>), g, b, lds, s, p);
        else hipLaunchKernelGGL((egress_fused_kernel<kHotFp16, 0>), g, b, lds, s, p);
    }
    return hipGetLastError();
}

}  // namespace ztcp
