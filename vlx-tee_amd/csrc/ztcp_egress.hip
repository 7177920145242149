// ztcp_egress.hip -- fused cold-page egress for gfx950:
// quantize -> ChaCha20 -> SipHash-2-4-128 in one kernel, one HBM read of the
// hot page and one HBM write of the blob.  Replaces the per-page encoder
// encode_one_cold_page_into_cpu (cpp:1103-1426) driven by
// fused_encode_cold_pages_peak_into_cpu (cpp:1904-2004).
//
// Work decomposition (one workgroup = up to 64 pages, 12 waves; lane = page
// in every wave):
//   * A "row" is one 64-byte keystream block position of the payload, for all
//     pages of the workgroup.  Every payload block is exactly one row: a code
//     row (4 int8 groups, 8 int4 groups or 2 raw groups) or a scale row (the
//     32 fp16 scales of one unit = 32 groups).  Rows are produced unit by
//     unit: a unit's code rows, then its scale row.
//   * Nine producer waves take code rows in order from an LDS counter.  A
//     code row quantizes its groups (loaded ahead, four at a time, while a
//     keystream is being computed), stages the scales in LDS, computes the
//     keystream, XORs, and writes the ciphertext into a ring of row slots in
//     LDS.  From the slot it stores the row to the blobs transposed: four
//     lanes per page, 64 contiguous bytes per page per store.  The wave that
//     stages a unit's last scales (an LDS counter per staging slot) also
//     makes the unit's scale row: it encrypts the staged scales and stores
//     them the same way.
//   * Wave 0 runs SipHash for one page per lane, at raised priority on a SIMD
//     of its own (waves 4 and 8, which the dispatcher places on that SIMD,
//     exit at once).  It absorbs the header, then the payload in order:
//     code rows straight from the LDS ring (no global read-back), scale rows
//     from the blobs once their stores have completed.
//   * Hand-offs are monotonic LDS counters with workgroup-scope
//     release/acquire: ring_flag[slot] = code row index + 1 when produced,
//     mac_used = code rows absorbed (frees ring slots), stage_flag[slot] =
//     unit + 1 when a scale row has read its staging slot, scale_flag[slot] =
//     unit + 1 once the scale row's stores have completed.  Every
//     wait is bounded; an expired wait sets a sticky diagnostic bit and the
//     kernel still ends.  Waits only point backwards in row order, so
//     progress never depends on a later row.
// Requires every section to hold a multiple of 32 groups (Layout::aligned),
// payload == required and 16-byte aligned pointers; otherwise the host routes
// the call to the generic kernels.
#include "ztcp_rows.h"

namespace ztcp {

namespace {

constexpr int kRing = 24;             // code rows between producers and the MAC wave
constexpr int kStage = 8;             // units whose scales are staged at once
constexpr int kLdsStage = kRing * kRowWords;
constexpr int kScaleSlots = 64;      // scale rows the MAC wave may still be waiting for
constexpr int kLdsFlags = kLdsStage + kStage * kRowWords;
constexpr int kFlagRing = 0;                          // [kRing] code row index + 1
constexpr int kFlagStage = kFlagRing + kRing;         // [kStage] unit + 1: staging slot free
constexpr int kFlagCount = kFlagStage + kStage;       // [kStage] code rows staged in the slot
constexpr int kFlagScale = kFlagCount + kStage;       // [kScaleSlots] unit + 1: scale row stored
constexpr int kFlagMacUsed = kFlagScale + kScaleSlots;  // code rows absorbed by the MAC wave
constexpr int kFlagTask = kFlagMacUsed + 1;           // next code row to hand out
constexpr int kNumFlags = kFlagMacUsed + 4;
constexpr int kLdsBlobs = kLdsFlags + kNumFlags;      // 64 blob pointers (8-byte aligned)
constexpr int kLdsWords = kLdsBlobs + 2 * 64;
static_assert(kLdsBlobs % 2 == 0, "blob table must be 8-byte aligned");

struct Row {
    int32_t valid;
    int32_t scale;    // 1: last code row of its unit (quantized sections)
    int32_t u, j;     // unit in section, code block in unit
    int32_t g;        // unit index among the page's quantized units (staging slot order)
    int32_t cidx;     // code row index = production order
    int32_t block;    // payload block index (keystream counter - 1)
    SecRows s;
};

// Code row t: the payload's code blocks in order, which is also the order of
// production.  A unit's scale row is produced right after its last code row,
// by the same wave.
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
            row.scale = s.kind != kSecRaw && row.j == s.nblk - 1;
            row.g = s.qunit_begin + row.u;
            row.cidx = t;
            row.block = (int32_t)(s.q_off / 64u) + local;
            row.s = s;
        }
        cb += n;
        if (s.kind != kSecRaw) qb += s.n_units;
    }
    return row;
}


__device__ __forceinline__ int32_t total_rows(const Layout& lay) {
    int32_t t = 0;
#pragma unroll
    for (int si = 0; si < 3; ++si) {
        if (si >= lay.n_sec) continue;
        const int32_t kind = ZTCP_SEC_FIELD(lay, si, kind);
        const int32_t rpu = kind == kSecInt8 ? 9 : (kind == kSecInt4 ? 5 : 16);
        t += ZTCP_SEC_FIELD(lay, si, n_units) * rpu;
    }
    return t;
}

__device__ __forceinline__ void load_group(const uint8_t* p, uint32_t w[8]) {
    const uint4 a = ldg16(p, 0), b = ldg16(p, 1);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

// Issues the hot loads of half h of a code row: groups [4h, 4h + 4) of the
// row's 4 (int8), 8 (int4) or 2 (raw) groups.
__device__ __forceinline__ void load_half(const EgressParams& p, const EgressPage& pg, const Row& row, int h,
                                          uint32_t (&w)[4][8]) {
    const int ng = row.s.kind == kSecInt8 ? 4 : (row.s.kind == kSecInt4 ? 8 : 2);
    const uint8_t* src = row.s.src ? pg.v : pg.k;
    GroupCursor cur = group_cursor(row.u * 32 + row.j * ng + 4 * h, row.s.gpv, row.s.col, p.head_dim);
    const uint32_t skip = (uint32_t)(p.head_dim - row.s.gpv * 16) * 2u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (i < ng) {
            load_group(src + cur.off, w[i]);
            cur.step(row.s.gpv, skip);
        }
    }
}

// Stores one row slot to the blobs: lane l writes quad (l & 3) of page
// 16 k + (l >> 2), so each store instruction writes 64 contiguous bytes of 16
// pages.  The blob pointers come from the workgroup's LDS table (null past
// the last page).
__device__ __forceinline__ void store_row(const uint32_t* slot, const uint32_t* lds, uint32_t blob_off,
                                          int lane) {
    const uint64_t* blobs = reinterpret_cast<const uint64_t*>(lds + kLdsBlobs);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int pr = 16 * k + (lane >> 2), q = lane & 3;
        const uint4 x = lds_quad(slot, pr, q);
        uint8_t* b = reinterpret_cast<uint8_t*>(blobs[pr]);
        if (b) stg16(b + blob_off, q, x);
    }
}

struct ProducerCtx {
    const EgressParams* p;
    EgressPage pg;
    uint32_t n0, n1, n2;
    ChaChaNonceCache nc;
    uint32_t* lds;
    int lane;
};

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

// One code row.  w holds the row's first four groups (loaded a row ahead);
// an int4 row loads its second four during the first half of the keystream.
// The next row's first groups are loaded as soon as w is free.
template <int DT, int KIND>
__device__ __forceinline__ void code_row(const ProducerCtx& c, const Row& row, const Row& nxt, bool prefetch,
                                         uint32_t (&w)[4][8]) {
    constexpr int SW = KIND == kSecInt8 ? 2 : (KIND == kSecInt4 ? 4 : 0);  // scale words per row
    const EgressParams& p = *c.p;
    uint32_t* flags = c.lds + kLdsFlags;
    uint32_t pt[16];
    uint32_t sc[4];
    ChaChaState st;
    st.start_cached(p.key, c.nc, 1u + (uint32_t)row.block);
    if constexpr (KIND == kSecRaw) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            pt[t] = w[0][t];
            pt[8 + t] = w[1][t];
        }
        if (prefetch) load_half(p, c.pg, nxt, 0, w);
        st.double_rounds<9>();
    } else if constexpr (KIND == kSecInt8) {
        quant_half<DT, 8>(w, pt, sc);
        if (prefetch) load_half(p, c.pg, nxt, 0, w);
        st.double_rounds<9>();
    } else {
        quant_half<DT, 4>(w, pt, sc);
        load_half(p, c.pg, row, 1, w);
        st.double_rounds<4>();
        quant_half<DT, 4>(w, pt + 8, sc + 2);
        if (prefetch) load_half(p, c.pg, nxt, 0, w);
        st.double_rounds<5>();
    }
    if constexpr (SW > 0) {
        // the unit's staging slot is free once unit g - kStage's scale row is done
        uint32_t* stage = c.lds + kLdsStage + (row.g % kStage) * kRowWords;
        wait_ge<kDiagEgressWait>(&flags[kFlagStage + row.g % kStage], row.g - kStage + 1, p.state);
#pragma unroll
        for (int t = 0; t < SW; ++t) {
            const int wd = row.j * SW + t;  // logical scale word of this lane's page
            stage[quad_word(c.lane, wd >> 2) + (wd & 3)] = sc[t];
        }
    }
    uint32_t ks[16];
    st.finish(p.key, 1u + (uint32_t)row.block, c.n0, c.n1, c.n2, ks);
    uint32_t* slot = c.lds + (row.cidx % kRing) * kRowWords;
    wait_ge<kDiagEgressWait>(&flags[kFlagMacUsed], row.cidx - kRing + 1, p.state);
#pragma unroll
    for (int q = 0; q < 4; ++q)
        lds_put_quad(slot, c.lane, q,
                     make_uint4(pt[4 * q] ^ ks[4 * q], pt[4 * q + 1] ^ ks[4 * q + 1],
                                pt[4 * q + 2] ^ ks[4 * q + 2], pt[4 * q + 3] ^ ks[4 * q + 3]));
    store_row(slot, c.lds, (uint32_t)kHeader + 64u * (uint32_t)row.block, c.lane);
    publish(&flags[kFlagRing + row.cidx % kRing], (uint32_t)row.cidx + 1u);
}

// The scale row of row.u's unit, run by the wave that staged the unit's last
// scales: encrypts the staged scales in place and stores the block.  Frees
// the staging slot at once; the stores' completion is published later
// (publish_scale) so that the wave does not wait for them here.
__device__ __forceinline__ void scale_row(const ProducerCtx& c, const Row& row) {
    const EgressParams& p = *c.p;
    uint32_t* flags = c.lds + kLdsFlags;
    const uint32_t block = row.s.s_off / 64u + (uint32_t)row.u;
    uint32_t ks[16];
    chacha_block_cached(p.key, c.nc, 1u + block, c.n0, c.n1, c.n2, ks);
    uint32_t* stage = c.lds + kLdsStage + (row.g % kStage) * kRowWords;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint4 s = lds_quad(stage, c.lane, q);
        lds_put_quad(stage, c.lane, q,
                     make_uint4(s.x ^ ks[4 * q], s.y ^ ks[4 * q + 1], s.z ^ ks[4 * q + 2], s.w ^ ks[4 * q + 3]));
    }
    store_row(stage, c.lds, (uint32_t)kHeader + 64u * block, c.lane);
    flags[kFlagCount + row.g % kStage] = 0u;
    publish(&flags[kFlagStage + row.g % kStage], (uint32_t)row.g + 1u);
}

// Publishes that scale row g is in the blobs, for the MAC wave to read.
__device__ __forceinline__ void publish_scale(uint32_t* flags, int32_t g) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's stores have completed
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    publish(&flags[kFlagScale + g % kScaleSlots], (uint32_t)g + 1u);
}

template <int DT>
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
    const int32_t total = total_code_rows(p.lay);
    uint32_t* flags = lds + kLdsFlags;
    // code rows are handed out in order from an LDS counter, one row ahead of
    // the one being made (so its groups can be prefetched): a slower wave
    // simply takes fewer rows
    auto grab = [&]() -> int32_t {
        uint32_t t = 0;
        if (c.lane == 0)
            t = __hip_atomic_fetch_add(&flags[kFlagTask], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        return (int32_t)__builtin_amdgcn_readfirstlane(t);
    };
    uint32_t w[4][8];
    int32_t t = grab();
    Row cur = row_info(p.lay, t);
    if (cur.valid) load_half(p, c.pg, cur, 0, w);
    int32_t pending = -1;  // scale row whose store completion is not yet published
#pragma unroll 1
    while (t < total) {
        if (pending >= 0) {  // the wave waits for this row's prefetched groups here anyway
            publish_scale(flags, pending);
            pending = -1;
        }
        const int32_t tn = grab();
        const Row nxt = row_info(p.lay, tn);
        if (cur.s.kind == kSecInt8)
            code_row<DT, kSecInt8>(c, cur, nxt, nxt.valid, w);
        else if (cur.s.kind == kSecInt4)
            code_row<DT, kSecInt4>(c, cur, nxt, nxt.valid, w);
        else
            code_row<DT, kSecRaw>(c, cur, nxt, nxt.valid, w);
        if (cur.s.kind != kSecRaw) {
            // count the unit's staged code rows; whoever stages the last one
            // encrypts the unit's scales
            uint32_t old = 0;
            if (c.lane == 0)
                old = __hip_atomic_fetch_add(&flags[kFlagCount + cur.g % kStage], 1u, __ATOMIC_ACQ_REL,
                                             __HIP_MEMORY_SCOPE_WORKGROUP);
            old = __builtin_amdgcn_readfirstlane(old);
            if (old == (uint32_t)cur.s.nblk - 1u) {
                scale_row(c, cur);
                pending = cur.g;
            }
        }
        t = tn;
        cur = nxt;
    }
    if (pending >= 0) publish_scale(flags, pending);
}

// The MAC wave's view of the payload: each section's code rows (LDS ring),
// then its scale rows (blobs).
struct MacFeed {
    int32_t si, phase, i;
    int32_t cidx;
    int32_t code_begin, qunit_begin;

    __device__ __forceinline__ void fetch(const EgressParams& p, const uint8_t* pay, const uint32_t* lds,
                                          int lane, uint4 (&x)[4], int32_t& tag) {
        const uint32_t* flags = lds + kLdsFlags;
        const SecRows s = sec_rows(p.lay, si, code_begin, qunit_begin);
        if (phase == 0) {
            const uint32_t* slot = lds + (cidx % kRing) * kRowWords;
            wait_ge<kDiagEgressWait>(&flags[kFlagRing + cidx % kRing], cidx + 1, p.state);
#pragma unroll
            for (int q = 0; q < 4; ++q) x[q] = lds_quad(slot, lane, q);
            tag = cidx + 1;
            ++cidx;
            if (++i == s.n_units * s.nblk) {
                i = 0;
                phase = s.kind != kSecRaw ? 1 : 2;
            }
        } else {
            const int32_t g = s.qunit_begin + i;
            wait_ge<kDiagEgressWait>(&flags[kFlagScale + g % kScaleSlots], g + 1, p.state);
            const uint8_t* q = pay + s.s_off + 64u * (uint32_t)i;
            x[0] = ldg16(q, 0); x[1] = ldg16(q, 1); x[2] = ldg16(q, 2); x[3] = ldg16(q, 3);
            tag = 0;
            if (++i == s.n_units) phase = 2;
        }
        if (phase == 2) {  // next section
            code_begin += s.n_units * s.nblk;
            if (s.kind != kSecRaw) qunit_begin += s.n_units;
            ++si;
            phase = 0;
            i = 0;
        }
    }
};

template <int DT>
__device__ void egress_mac(const EgressParams& p, int64_t page0, int ppw, uint32_t* lds) {
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
    const uint8_t* pay = blob + kHeader;
    uint32_t* used = lds + kLdsFlags + kFlagMacUsed;
    MacFeed feed{0, 0, 0, 0, 0, 0};
    const int32_t total = total_rows(p.lay);
    // three chunks in flight: two fetched ahead of the one being absorbed; a
    // code row's ring slot is released once it has been absorbed
    uint4 x0[4], x1[4], x2[4];
    int32_t t0 = 0, t1 = 0, t2 = 0;
    if (total > 0) feed.fetch(p, pay, lds, lane, x0, t0);
    if (total > 1) feed.fetch(p, pay, lds, lane, x1, t1);
#pragma unroll 1
    for (int32_t c = 0; c < total; c += 3) {
        if (c + 2 < total) feed.fetch(p, pay, lds, lane, x2, t2);
        s.absorb64(x0);
        if (t0) publish(used, (uint32_t)t0);
        if (c + 1 >= total) break;
        if (c + 3 < total) feed.fetch(p, pay, lds, lane, x0, t0);
        s.absorb64(x1);
        if (t1) publish(used, (uint32_t)t1);
        if (c + 2 >= total) break;
        if (c + 4 < total) feed.fetch(p, pay, lds, lane, x1, t1);
        s.absorb64(x2);
        if (t2) publish(used, (uint32_t)t2);
    }
    uint64_t lo, hi;
    s.finish((uint64_t)((kHeader + p.payload) & 0xFFu) << 56, lo, hi);
    if (active)
        stg16(blob + kHeader + p.payload, 0,
              make_uint4((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)));
}

template <int DT>
__global__ __launch_bounds__(kFusedThreads) void egress_fused_kernel(EgressParams p) {
    extern __shared__ __align__(16) uint32_t lds[];
    const int64_t page0 = (int64_t)blockIdx.x * p.ppw;
    const int ppw = (int)min((int64_t)p.ppw, p.batch - page0);
    for (int i = threadIdx.x; i < kNumFlags; i += blockDim.x) lds[kLdsFlags + i] = 0u;
    if (threadIdx.x < 64) {
        uint64_t* blobs = reinterpret_cast<uint64_t*>(lds + kLdsBlobs);
        blobs[threadIdx.x] = (int)threadIdx.x < ppw ? reinterpret_cast<uint64_t>(egress_page(p, page0 + threadIdx.x).blob)
                                                    : 0ull;  // no stores past the last page
    }
    __syncthreads();
    const int wave = threadIdx.x >> 6;
    if (wave == 0) {
        __builtin_amdgcn_s_setprio(3);
        egress_mac<DT>(p, page0, ppw, lds);
        return;
    }
    if ((wave & 3) == 0) return;  // leave the MAC wave's SIMD to it
    egress_produce<DT>(p, page0, ppw, lds);
}

}  // namespace

size_t egress_fused_lds_bytes() { return (size_t)kLdsWords * sizeof(uint32_t); }

hipError_t launch_egress_fused(const EgressParams& p, int dtype, hipStream_t s) {
    const int64_t grid = (p.batch + p.ppw - 1) / p.ppw;
    const size_t lds = egress_fused_lds_bytes();  // above 64 KiB: gfx950 has 160 KiB per CU
    if (dtype == kHotBf16)
        hipLaunchKernelGGL(egress_fused_kernel<kHotBf16>, dim3((uint32_t)grid), dim3(kFusedThreads), lds, s, p);
    else
        hipLaunchKernelGGL(egress_fused_kernel<kHotFp16>, dim3((uint32_t)grid), dim3(kFusedThreads), lds, s, p);
    return hipGetLastError();
}

}  // namespace ztcp
