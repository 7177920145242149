// ztcp_ingress.hip -- fused cold-page ingress for gfx950:
// verify (header, AAD, SipHash tag) -> ChaCha20 decrypt -> dequantize, one
// HBM read of the blob and one HBM write of the hot page.  Replaces the
// per-page decoder of fused_decode_cold_pages_peak_into_cpu (cpp:2309-2463).
//
// One workgroup handles up to 64 pages with 16 waves, four per SIMD (lane =
// page in every wave):
//   * Every page is decoded according to its own header flags.  The
//     workgroup's layout is that of its first page with valid flags; pages
//     with that layout go through the row pipeline below, pages with another
//     valid layout are decoded afterwards unit by unit, pages with invalid
//     flags are not decoded (they fail with status 1).
//   * Twelve decoder waves (on SIMDs 1-3) take rows in order from an LDS
//     counter, each with its ciphertext block loaded one row ahead.  A
//     unit's scale row is decrypted into an LDS staging slot four units ahead
//     of its code rows.  A code row first puts its ciphertext into a ring of
//     row slots in LDS, at its place in payload order, then decrypts, takes
//     its scales from staging and dequantizes two groups at a time into a
//     per-wave LDS tile, from which the wave stores them transposed: four
//     lanes per page, so each store writes the two groups (64 bytes,
//     contiguous within a head vector) of 16 pages.
//   * Wave 0 verifies one page per lane at raised priority on SIMD 0:
//     magic/version (status 1), AAD tenant/model/layer/token hash (status
//     2), the SipHash-2-4-128 tag over header || ciphertext (status 3), then
//     flags and payload size (status 1), in the reference's order
//     (cpp:2313-2355).  It reads the payload's 64-byte rows in order from the
//     ring: code rows come from the decoders, every other row (scales,
//     padding) from a feeder wave (wave 4, on SIMD 0 as well), which copies
//     them from the blob so that the verify wave's chain never waits for
//     global memory.  Waves 8 and 12 exit at once.
//   * Decoding is speculative: a page whose verdict is not OK has its outputs
//     zeroed before the kernel ends (per-page mode) or by the finalize kernel
//     (all-or-nothing mode, which zeroes every output, cpp:2481-2486).
//     Outputs are only valid after the call returns OK, as with the
//     reference.
//   * Hand-offs are monotonic LDS counters (ring flags, mac_used,
//     scale_ready, scale_free) with workgroup-scope release/acquire; every
//     wait is bounded and only points backwards in payload or task order.
// Requires 16-byte aligned blobs / outputs, blob_bytes % 16 == 0 and every
// layout aligned to 64-byte units; otherwise the host uses the generic path.
#include "ztcp_rows.h"

namespace ztcp {

namespace {

constexpr int kIngressWaves = 16;
constexpr int kIngressThreads = 64 * kIngressWaves;
constexpr int kDecoderWaves = 12;  // the waves on SIMDs 1-3
constexpr int kRing = 16;          // payload rows between their makers and the verify wave
constexpr int kStage = 8;          // units whose decrypted scales are staged at once
constexpr int kLookahead = 4;      // a unit's scale row is handed out this many units early
constexpr int kLdsStage = kRing * kRowWords;
constexpr int kLdsTile = kLdsStage + kStage * kRowWords;       // per decoder wave: 2 groups per page
constexpr int kLdsFlags = kLdsTile + kDecoderWaves * kRowWords;
constexpr int kFlagRing = 0;                         // [kRing] payload row index + 1
constexpr int kFlagReady = kFlagRing + kRing;        // [kStage] unit + 1: scales decrypted
constexpr int kFlagFree = kFlagReady + kStage;       // [kStage] unit + 1: scales consumed
constexpr int kFlagCount = kFlagFree + kStage;       // [kStage] code rows that took their scales
constexpr int kFlagMacUsed = kFlagCount + kStage;    // payload rows absorbed by the verify wave
constexpr int kFlagTask = kFlagMacUsed + 1;          // next row to hand out
constexpr int kFlagStatus = kFlagTask + 1;           // [64] verdicts
constexpr int kFlagNaN = kFlagStatus + 64;           // [64] 1: the page has an inf / NaN scale
constexpr int kFlagExpired = kFlagNaN + 64;          // 1: a bounded wait of the workgroup expired
constexpr int kNumFlags = (kFlagExpired + 2) & ~1;   // even: the pointer table after it is 8-byte aligned
constexpr int kLdsPtrs = kLdsFlags + kNumFlags;      // [2][64] output pointers (K, V)
constexpr int kLdsLayouts = kLdsPtrs + 2 * 2 * 64;   // [kNumLayouts] Layout, one per header flags value
constexpr int kLayoutWords = (int)(sizeof(Layout) / 4);
constexpr int kLdsHeaders = (kLdsLayouts + kNumLayouts * kLayoutWords + 3) & ~3;  // [64] 32-byte headers
constexpr int kLdsTimers = kLdsHeaders + 64 * 8;       // phase-timer counters (timer builds only)
constexpr int kLdsWords = kLdsTimers + kTimerLdsWords;
static_assert(kLdsHeaders % 4 == 0, "header table must be 16-byte aligned");
static_assert(sizeof(Layout) % 4 == 0, "Layout is copied word by word");
static_assert(kLdsWords * 4 <= 160 * 1024, "LDS budget of one CU");
static_assert(kLdsPtrs % 2 == 0, "pointer table must be 8-byte aligned");
static_assert(kStage >= kLookahead + 1, "a scale row only waits for units whose code rows come before it");

__device__ __forceinline__ void load_block(const uint8_t* p, uint32_t w[16]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint4 a = ldg16(p, i);
        w[4 * i] = a.x; w[4 * i + 1] = a.y; w[4 * i + 2] = a.z; w[4 * i + 3] = a.w;
    }
}

__device__ __forceinline__ void store_group(uint8_t* p, const uint32_t o[8]) {
    stg16(p, 0, make_uint4(o[0], o[1], o[2], o[3]));
    stg16(p, 1, make_uint4(o[4], o[5], o[6], o[7]));
}

// Layout index (preset - 1) * 4 + rope_mode of a header's flags, or -1 when
// the flags are invalid, not enabled for this call (lay_ok: the extension
// layouts only with ZTCP_EXT_LAYOUTS) or the payload is too short for them.
__device__ __forceinline__ int layout_index(const IngressParams& p, uint32_t h0x) {
    const uint32_t flags = h0x >> 24, preset = flags & 0x0Fu, rope_mode = flags >> 4;
    if (preset < 1u || preset > 6u || rope_mode > 3u) return -1;
    const int li = (int)((preset - 1u) * 4u + rope_mode);
    return ((p.lay_ok >> li) & 1u) ? li : -1;
}

// Extension kinds (family 1 kernels only): compile-time row geometry
// (ztcp_layout.h) and the dequantization of chunks 2 pc, 2 pc + 1 (32
// elements, 16 packed hot words) of a decrypted code row pt with the row's
// parameter words sc.
template <int KIND>
struct ExtRows {
    static constexpr int kChunks = KIND == kSecInt4G32 ? 8 : 4;       // 16-element chunks per row
    static constexpr int kParamWords = KIND == kSecAsym8 ? 1 : 2;     // parameter words per row
    static constexpr int kRowsPerUnit = KIND == kSecAsym8 ? 16 : 8;   // code rows per unit
};

template <int DT, int KIND>
__device__ __forceinline__ void dequant_pair_ext(const uint32_t* pt, const uint32_t* sc, int pc, uint32_t o[16]) {
    if constexpr (KIND == kSecInt4G32) {  // group pc: 32 elements, one scale
        const uint32_t sb = (pc & 1) ? (sc[pc >> 1] >> 16) : (sc[pc >> 1] & 0xFFFFu);
        dequant_group_int4<DT>(pt + 4 * pc, sb, o);
        dequant_group_int4<DT>(pt + 4 * pc + 2, sb, o + 8);
    } else if constexpr (KIND == kSecAsym8) {  // half pc of the row's one group
        dequant_asym8_16<DT>(pt + 8 * pc, sc[0], o);
        dequant_asym8_16<DT>(pt + 8 * pc + 4, sc[0], o + 8);
    } else {  // e4m3: groups 2 pc, 2 pc + 1 of 16 elements
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int gi = 2 * pc + h;
            const uint32_t sbits = (gi & 1) ? (sc[gi >> 1] >> 16) : (sc[gi >> 1] & 0xFFFFu);
            dequant_group_e4m3<DT>(pt + 4 * gi, sbits, o + 8 * h);
        }
    }
}

// ---------------------------------------------------------------------------
// Unit-by-unit decode for pages whose layout is not the workgroup's.
// ---------------------------------------------------------------------------

template <int DT, int KIND>
__device__ __forceinline__ void decode_ext_unit(const IngressParams& p, const uint8_t* pay, uint8_t* out,
                                                int32_t lu, int32_t gpv, int32_t col, uint32_t q_off,
                                                uint32_t s_off, uint32_t n0, uint32_t n1, uint32_t n2,
                                                uint32_t* nan_flag) {
    using G = ExtRows<KIND>;
    GroupCursor cur = group_cursor(lu * G::kRowsPerUnit * G::kChunks, gpv, col, p.head_dim);
    const uint32_t skip = (uint32_t)(p.head_dim - gpv * 16) * 2u;
    const uint32_t s_unit = s_off + (uint32_t)lu * 64u;
    uint32_t sc[16];
    load_block(pay + s_unit, sc);
    uint32_t ks[16];
    chacha_block(p.key, 1u + s_unit / 64u, n0, n1, n2, ks);
#pragma unroll
    for (int i = 0; i < 16; ++i) sc[i] ^= ks[i];
    if (params_nonfinite(sc)) *nan_flag = 1u;
    const uint32_t code0 = q_off + (uint32_t)lu * (uint32_t)G::kRowsPerUnit * 64u;
#pragma unroll 1
    for (int j = 0; j < G::kRowsPerUnit; ++j) {
        uint32_t ct[16];
        load_block(pay + code0 + (uint32_t)j * 64u, ct);
        chacha_block(p.key, 1u + code0 / 64u + (uint32_t)j, n0, n1, n2, ks);
#pragma unroll
        for (int i = 0; i < 16; ++i) ct[i] ^= ks[i];
#pragma unroll
        for (int pc = 0; pc < G::kChunks / 2; ++pc) {
            uint32_t o[16];
            dequant_pair_ext<DT, KIND>(ct, sc, pc, o);
            store_group(out + cur.off, o);
            cur.step(gpv, skip);
            store_group(out + cur.off, o + 8);
            cur.step(gpv, skip);
        }
#pragma unroll
        for (int t = 0; t < 16 - G::kParamWords; ++t) sc[t] = sc[t + G::kParamWords];
    }
}

template <int DT, int KIND>
__device__ __forceinline__ void decode_quant_unit(const IngressParams& p, const uint8_t* pay,
                                                  uint8_t* out, int32_t lu, int32_t gpv,
                                                  int32_t col, uint32_t q_off, uint32_t s_off,
                                                  uint32_t n0, uint32_t n1, uint32_t n2, uint32_t* nan_flag) {
    constexpr int GPB = KIND == kSecInt8 ? 4 : 8;
    constexpr int NBLK = 32 / GPB;
    constexpr int CW = KIND == kSecInt8 ? 4 : 2;
    const int32_t G0 = lu * 32;
    GroupCursor cur = group_cursor(G0, gpv, col, p.head_dim);
    const uint32_t skip = (uint32_t)(p.head_dim - gpv * 16) * 2u;
    const uint32_t s_unit = s_off + (uint32_t)lu * 64u;
    uint32_t sc[16];
    load_block(pay + s_unit, sc);
    uint32_t ks[16];
    chacha_block(p.key, 1u + s_unit / 64u, n0, n1, n2, ks);
#pragma unroll
    for (int i = 0; i < 16; ++i) sc[i] ^= ks[i];
    if (params_nonfinite(sc)) *nan_flag = 1u;
    const uint32_t code0 = q_off + (uint32_t)(G0 * CW * 4);
#pragma unroll 1
    for (int j = 0; j < NBLK; ++j) {
        uint32_t ct[16];
        load_block(pay + code0 + (uint32_t)j * 64u, ct);
        chacha_block(p.key, 1u + code0 / 64u + (uint32_t)j, n0, n1, n2, ks);
#pragma unroll
        for (int i = 0; i < 16; ++i) ct[i] ^= ks[i];
#pragma unroll
        for (int i = 0; i < GPB; ++i) {
            const uint32_t sbits = (i & 1) ? (sc[i >> 1] >> 16) : (sc[i >> 1] & 0xFFFFu);
            uint32_t o[8];
            if constexpr (KIND == kSecInt8) dequant_group_int8<DT>(ct + 4 * i, sbits, o);
            else dequant_group_int4<DT>(ct + 2 * i, sbits, o);
            store_group(out + cur.off, o);
            cur.step(gpv, skip);
        }
#pragma unroll
        for (int t = 0; t < 16 - GPB / 2; ++t) sc[t] = sc[t + GPB / 2];
    }
}

__device__ __forceinline__ void decode_raw_unit(const IngressParams& p, const uint8_t* pay,
                                                uint8_t* out, int32_t lu, int32_t gpv,
                                                int32_t col, uint32_t q_off, uint32_t n0,
                                                uint32_t n1, uint32_t n2) {
    const int32_t G0 = lu * 32;
    GroupCursor cur = group_cursor(G0, gpv, col, p.head_dim);
    const uint32_t skip = (uint32_t)(p.head_dim - gpv * 16) * 2u;
    const uint32_t code0 = q_off + (uint32_t)G0 * 32u;
#pragma unroll 1
    for (int j = 0; j < 16; ++j) {
        uint32_t ct[16], ks[16];
        load_block(pay + code0 + (uint32_t)j * 64u, ct);
        chacha_block(p.key, 1u + code0 / 64u + (uint32_t)j, n0, n1, n2, ks);
#pragma unroll
        for (int i = 0; i < 16; ++i) ct[i] ^= ks[i];
        store_group(out + cur.off, ct);
        cur.step(gpv, skip);
        store_group(out + cur.off, ct + 8);
        cur.step(gpv, skip);
    }
}

template <int DT, int FAM>
__device__ __forceinline__ void decode_unit(const IngressParams& p, const Layout& lay, int64_t page, int32_t u,
                            uint32_t n0, uint32_t n1, uint32_t n2, uint32_t* nan_flag) {
    const int si = section_of_unit(lay, u);
    const int32_t kind = ZTCP_SEC_FIELD(lay, si, kind);
    const int32_t srcsel = ZTCP_SEC_FIELD(lay, si, src);
    const int32_t col = ZTCP_SEC_FIELD(lay, si, col);
    const int32_t gpv = ZTCP_SEC_FIELD(lay, si, gpv);
    const int32_t lu = u - ZTCP_SEC_FIELD(lay, si, unit_begin);
    const uint32_t q_off = ZTCP_SEC_FIELD(lay, si, q_off);
    const uint32_t s_off = ZTCP_SEC_FIELD(lay, si, s_off);
    const uint8_t* pay = ingress_blob(p, page) + kHeader;
    uint8_t* out = srcsel ? ingress_v(p, page) : ingress_k(p, page);
    if (kind == kSecInt8)
        decode_quant_unit<DT, kSecInt8>(p, pay, out, lu, gpv, col, q_off, s_off, n0, n1, n2, nan_flag);
    else if (kind == kSecInt4)
        decode_quant_unit<DT, kSecInt4>(p, pay, out, lu, gpv, col, q_off, s_off, n0, n1, n2, nan_flag);
    else if (kind == kSecRaw)
        decode_raw_unit(p, pay, out, lu, gpv, col, q_off, n0, n1, n2);
    else if constexpr (FAM == 1) {
        if (kind == kSecE4m3)
            decode_ext_unit<DT, kSecE4m3>(p, pay, out, lu, gpv, col, q_off, s_off, n0, n1, n2, nan_flag);
        else if (kind == kSecInt4G32)
            decode_ext_unit<DT, kSecInt4G32>(p, pay, out, lu, gpv, col, q_off, s_off, n0, n1, n2, nan_flag);
        else
            decode_ext_unit<DT, kSecAsym8>(p, pay, out, lu, gpv, col, q_off, s_off, n0, n1, n2, nan_flag);
    }
}

// ---------------------------------------------------------------------------
// Row pipeline.
// ---------------------------------------------------------------------------

// Row t of the decode order.  Per section of U units: the scale rows of units
// 0 .. L-1, then the units' code rows, two units at a time with the scale
// rows of units u + L and u + 1 + L (L = kLookahead) between them (task_info
// below), so a unit's scales are decrypted while the units before it are
// being decoded.
struct Task {
    int32_t valid;
    int32_t scale;    // 1: scale row of unit u
    int32_t u, j;     // unit in section, code block in unit
    int32_t g;        // unit index among the page's quantized units (staging order)
    int32_t cidx;     // code row index (payload order of the code rows)
    int32_t mrow;     // payload row of a code row (its place in the ring)
    int32_t block;    // payload block index (keystream counter - 1)
    SecRows s;
};

template <int FAM>
__device__ __forceinline__ int32_t div_nblk(int32_t x, int32_t kind) {  // nblk = 8, 4, 16
    if constexpr (FAM == 1) {
        const int32_t nblk = code_rows_per_unit(kind);
        return nblk == 8 ? x / 8 : (nblk == 4 ? x / 4 : x / 16);
    }
    return kind == kSecInt8 ? x / 8 : (kind == kSecInt4 ? x / 4 : x / 16);
}
template <int FAM>
__device__ __forceinline__ int32_t div_rpu2(int32_t x, int32_t kind) {  // 2 (nblk + 1) = 18, 10, 34
    if constexpr (FAM == 1) {
        const int32_t nblk = code_rows_per_unit(kind);
        return nblk == 8 ? x / 18 : (nblk == 4 ? x / 10 : x / 34);
    }
    return kind == kSecInt8 ? x / 18 : x / 10;
}

// Task t of the workgroup layout.  A quantized section hands out the scale
// rows of its first kLookahead units, then its units' code rows two units
// at a time with the scale rows of the two units kLookahead further on
// between them: code rows of u, scale rows of u + L and u + 1 + L, code
// rows of u + 1.  Neighbouring scale rows share 128-byte lines in the blob,
// and decoders that take them one after the other read those lines at once.
template <int FAM>
__device__ __forceinline__ Task task_info(const Layout& lay, int32_t t) {
    Task k{};
    int32_t tb = 0, cb = 0, qb = 0;
#pragma unroll
    for (int si = 0; si < 3; ++si) {
        if (si >= lay.n_sec || k.valid) continue;
        const SecRows s = sec_rows(lay, si, cb, qb);
        const bool quant = s.kind != kSecRaw;
        const int32_t n = s.n_units * s.nblk + (quant ? s.n_units : 0);
        if (t >= tb && t < tb + n) {
            int32_t x = t - tb;
            k.valid = 1;
            if (!quant) {
                k.u = div_nblk<FAM>(x, s.kind);
                k.j = x - k.u * s.nblk;
            } else {
                const int32_t pre = min(kLookahead, s.n_units);
                const int32_t full = max(s.n_units - kLookahead, 0);  // units followed by a scale row
                if (x < pre) {
                    k.scale = 1;
                    k.u = x;
                } else if ((x -= pre) < full * s.rpu) {
                    const int32_t span = 2 * s.rpu, pairs = full >> 1;
                    int32_t u0, off;
                    if (x < pairs * span) {
                        const int32_t p2 = div_rpu2<FAM>(x, s.kind);
                        u0 = 2 * p2;
                        off = x - p2 * span;
                    } else {  // an odd last unit: its code rows, then one scale row
                        u0 = full - 1;
                        off = x - pairs * span;
                    }
                    if (off < s.nblk) {
                        k.u = u0;
                        k.j = off;
                    } else if (off <= s.nblk + 1) {
                        k.scale = 1;
                        k.u = u0 + kLookahead + (off - s.nblk);
                    } else {
                        k.u = u0 + 1;
                        k.j = off - s.nblk - 2;
                    }
                } else {
                    x -= full * s.rpu;
                    const int32_t u = div_nblk<FAM>(x, s.kind);
                    k.u = full + u;
                    k.j = x - u * s.nblk;
                }
            }
            k.g = s.qunit_begin + k.u;
            k.cidx = cb + k.u * s.nblk + k.j;
            k.mrow = k.cidx + qb;  // a section's codes follow the scale rows of the sections before it
            k.block = k.scale ? (int32_t)(s.s_off / 64u) + k.u : (int32_t)(s.q_off / 64u) + k.u * s.nblk + k.j;
            k.s = s;
        }
        tb += n;
        cb += s.n_units * s.nblk;
        if (quant) qb += s.n_units;
    }
    return k;
}

__device__ __forceinline__ int32_t total_tasks(const Layout& lay) {
    int32_t t = 0;
#pragma unroll
    for (int si = 0; si < 3; ++si) {
        if (si >= lay.n_sec) continue;
        const int32_t kind = ZTCP_SEC_FIELD(lay, si, kind);
        t += ZTCP_SEC_FIELD(lay, si, n_units) * (code_rows_per_unit(kind) + (kind != kSecRaw ? 1 : 0));
    }
    return t;
}

// The payload row that sets a task's urgency: a code task's own row; a
// scale task is as urgent as the first code row of its unit.
__device__ __forceinline__ int32_t task_lead_row(const Task& k) {
    return k.scale ? (int32_t)(k.s.q_off / 64u) + k.u * k.s.nblk : k.mrow;
}

struct DecoderCtx {
    const IngressParams* p;
    const uint8_t* pay;     // this lane's page payload
    uint32_t n0, n1, n2;    // this lane's page nonce (from its header)
    ChaChaNonceCache nc;
    uint32_t* lds;
    uint32_t* tile;         // this wave's dequantized tile
    PageQuads pq;           // this lane's quads in a row slot
    Waiter wt;
    int lane;
    // Transposed tile stores: store k (0..3) writes quad (lane & 3) of page
    // 16 k + (lane >> 2), whose output pointer is entry 16 k + (lane >> 2)
    // of the pointer table.  Past the last page of a partial workgroup the
    // table holds page 0's pointers, and the tile holds page 0's data (those
    // lanes decode page 0), so every store is unconditional: a store under a
    // branch makes the compiler wait for all outstanding stores before the
    // next row's loads.  The quad swizzle of page 16 k + i equals that of
    // page i, so store k's tile offset is tq0 + 1024 k bytes.
    uint32_t tq0;

    __device__ __forceinline__ void init_stores() { tq0 = quad_word(lane >> 2, lane & 3) * 4u; }

    // 16 on odd lanes, else 0: the second quad of the 32 bytes that a lane
    // pair stores.  Bits 4-5 of tq0 are (lane & 3) ^ ((lane >> 3) & 3) and
    // bit 7 is (lane >> 3) & 1, so bit 4 of tq0 ^ (tq0 >> 3) is lane & 1.
    // Recomputed at each store by instructions the compiler cannot hoist: a
    // value held across the task loop is one VGPR more than the BF16 kernel
    // of the extension kinds has at 16 waves, and the allocator spills it
    // (a scratch reload, which waits for every load in flight).
    __device__ __forceinline__ uint32_t odd16() const {
        uint32_t r;
        asm volatile("v_lshrrev_b32 %0, 3, %1\n\tv_xor_b32 %0, %0, %1\n\tv_and_b32 %0, 16, %0"
                     : "=&v"(r)
                     : "v"(tq0));
        return r;
    }
};

template <int DT, int KIND>
__device__ __forceinline__ void code_task(const DecoderCtx& c, const Task& k, uint32_t (&ct)[16],
                                          const Task& nxt) {
    constexpr int GPB = KIND == kSecInt8 ? 4 : (KIND == kSecInt4 ? 8 : 2);
    constexpr int SW = GPB / 2;  // scale words of this row
    const IngressParams& p = *c.p;
    uint32_t* flags = c.lds + kLdsFlags;
    // ciphertext to the verify wave, at its place in payload order
    uint32_t* slot = c.lds + (k.mrow % kRing) * kRowWords;
    wait_ge<kDiagIngressWait, kTmRingWait>(&flags[kFlagMacUsed], k.mrow - kRing + 1, c.wt);
#pragma unroll
    for (int q = 0; q < 4; ++q)
        lds_put_quad_at(slot, c.pq.off[q], make_uint4(ct[4 * q], ct[4 * q + 1], ct[4 * q + 2], ct[4 * q + 3]));
    publish(&flags[kFlagRing + k.mrow % kRing], (uint32_t)k.mrow + 1u);
    tm_trace(c.wt.trace, k.mrow, c.wt.t0);
    // this row is out: the rest of the task runs at the urgency of the next
    if (nxt.valid) refresh_row_priority(&flags[kFlagMacUsed], task_lead_row(nxt));
    uint32_t pt[16];
    {
        uint32_t ks[16];
        chacha_block_cached(p.key, c.nc, 1u + (uint32_t)k.block, c.n0, c.n1, c.n2, ks);
#pragma unroll
        for (int i = 0; i < 16; ++i) pt[i] = ct[i] ^ ks[i];
    }
    if (nxt.valid) load_block(c.pay + 64u * (uint32_t)nxt.block, ct);
    uint32_t sc[SW];
    if constexpr (KIND != kSecRaw) {
        const int slot_s = k.g % kStage;
        wait_ge<kDiagIngressWait, kTmStageWait>(&flags[kFlagReady + slot_s], k.g + 1, c.wt);
        const uint32_t* stage = c.lds + kLdsStage + slot_s * kRowWords;
        if constexpr (KIND == kSecInt8) {  // words 2j, 2j + 1 of the page's scale row
            const uint32_t* w = stage + quad_word(c.lane, k.j >> 1) + 2 * (k.j & 1);
            sc[0] = w[0];
            sc[1] = w[1];
        } else {  // words 4j .. 4j + 3
            const uint4 v = lds_quad(stage, c.lane, k.j);
            sc[0] = v.x; sc[1] = v.y; sc[2] = v.z; sc[3] = v.w;
        }
        // the last code row of the unit to take its scales frees the slot
        uint32_t old = 0;
        if (c.lane == 0)
            old = __hip_atomic_fetch_add(&flags[kFlagCount + slot_s], 1u, __ATOMIC_ACQ_REL,
                                         __HIP_MEMORY_SCOPE_WORKGROUP);
        old = __builtin_amdgcn_readfirstlane(old);
        if (old == (uint32_t)k.s.nblk - 1u) {
            flags[kFlagCount + slot_s] = 0u;
            publish(&flags[kFlagFree + slot_s], (uint32_t)k.g + 1u);
        }
    }
    // output offsets of the row's groups, walked in (vec, group) order
    GroupCursor cur = group_cursor(k.u * 32 + k.j * GPB, k.s.gpv, k.s.col, p.head_dim);
    const uint32_t skip = (uint32_t)(p.head_dim - k.s.gpv * 16) * 2u;
    const bool to_v = k.s.src != 0;
#pragma unroll
    for (int pc = 0; pc < GPB / 2; ++pc) {
        uint32_t o[16];
        if constexpr (KIND == kSecRaw) {
#pragma unroll
            for (int i = 0; i < 16; ++i) o[i] = pt[i];
        } else {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int gi = 2 * pc + h;
                const uint32_t sbits = (gi & 1) ? (sc[gi >> 1] >> 16) : (sc[gi >> 1] & 0xFFFFu);
                if constexpr (KIND == kSecInt8) dequant_group_int8<DT>(pt + 4 * gi, sbits, o + 8 * h);
                else dequant_group_int4<DT>(pt + 2 * gi, sbits, o + 8 * h);
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
            lds_put_quad_at(c.tile, c.pq.off[q], make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]));
        const uint32_t off_a = cur.off;
        cur.step(k.s.gpv, skip);
        const uint32_t off_b = cur.off;
        cur.step(k.s.gpv, skip);
        // lanes 4i, 4i + 1 store the first group's two quads, 4i + 2, 4i + 3 the second's
        const uint32_t off = ((c.lane & 2) ? off_b : off_a) + c.odd16();
        const uint64_t* ptab = reinterpret_cast<const uint64_t*>(c.lds + kLdsPtrs) + (to_v ? 64 : 0) + (c.lane >> 2);
        uint4 x[4];
        uint8_t* out[4];
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
            x[s4] = lds_quad_at(c.tile, c.tq0 + 1024u * (uint32_t)s4);
            out[s4] = reinterpret_cast<uint8_t*>(ptab[16 * s4]);
        }
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) stg16(out[s4] + off, 0, x[s4]);
    }
}

// code_task for the extension kinds (family 1): the same steps with the
// kind's row geometry (ExtRows) and dequantizer.
template <int DT, int KIND>
__device__ __forceinline__ void code_task_ext(const DecoderCtx& c, const Task& k, uint32_t (&ct)[16],
                                              const Task& nxt) {
    using G = ExtRows<KIND>;
    const IngressParams& p = *c.p;
    uint32_t* flags = c.lds + kLdsFlags;
    uint32_t* slot = c.lds + (k.mrow % kRing) * kRowWords;
    wait_ge<kDiagIngressWait, kTmRingWait>(&flags[kFlagMacUsed], k.mrow - kRing + 1, c.wt);
#pragma unroll
    for (int q = 0; q < 4; ++q)
        lds_put_quad_at(slot, c.pq.off[q], make_uint4(ct[4 * q], ct[4 * q + 1], ct[4 * q + 2], ct[4 * q + 3]));
    publish(&flags[kFlagRing + k.mrow % kRing], (uint32_t)k.mrow + 1u);
    tm_trace(c.wt.trace, k.mrow, c.wt.t0);
    // this row is out: the rest of the task runs at the urgency of the next
    if (nxt.valid) refresh_row_priority(&flags[kFlagMacUsed], task_lead_row(nxt));
    uint32_t pt[16];
    {
        uint32_t ks[16];
        chacha_block_cached(p.key, c.nc, 1u + (uint32_t)k.block, c.n0, c.n1, c.n2, ks);
#pragma unroll
        for (int i = 0; i < 16; ++i) pt[i] = ct[i] ^ ks[i];
    }
    if (nxt.valid) load_block(c.pay + 64u * (uint32_t)nxt.block, ct);
    uint32_t sc[2];
    const int slot_s = k.g % kStage;
    wait_ge<kDiagIngressWait, kTmStageWait>(&flags[kFlagReady + slot_s], k.g + 1, c.wt);
    const uint32_t* stage = c.lds + kLdsStage + slot_s * kRowWords;
    if constexpr (G::kParamWords == 2) {  // words 2j, 2j + 1 of the page's parameter row
        const uint32_t* w = stage + quad_word(c.lane, k.j >> 1) + 2 * (k.j & 1);
        sc[0] = w[0];
        sc[1] = w[1];
    } else {  // word j
        sc[0] = stage[quad_word(c.lane, k.j >> 2) + (k.j & 3)];
        sc[1] = 0u;
    }
    uint32_t old = 0;
    if (c.lane == 0)
        old = __hip_atomic_fetch_add(&flags[kFlagCount + slot_s], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old == (uint32_t)k.s.nblk - 1u) {
        flags[kFlagCount + slot_s] = 0u;
        publish(&flags[kFlagFree + slot_s], (uint32_t)k.g + 1u);
    }
    GroupCursor cur = group_cursor((k.u * G::kRowsPerUnit + k.j) * G::kChunks, k.s.gpv, k.s.col, p.head_dim);
    const uint32_t skip = (uint32_t)(p.head_dim - k.s.gpv * 16) * 2u;
    const bool to_v = k.s.src != 0;
#pragma unroll
    for (int pc = 0; pc < G::kChunks / 2; ++pc) {
        uint32_t o[16];
        dequant_pair_ext<DT, KIND>(pt, sc, pc, o);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            lds_put_quad_at(c.tile, c.pq.off[q], make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]));
        const uint32_t off_a = cur.off;
        cur.step(k.s.gpv, skip);
        const uint32_t off_b = cur.off;
        cur.step(k.s.gpv, skip);
        const uint32_t off = ((c.lane & 2) ? off_b : off_a) + c.odd16();
        const uint64_t* ptab = reinterpret_cast<const uint64_t*>(c.lds + kLdsPtrs) + (to_v ? 64 : 0) + (c.lane >> 2);
        uint4 x[4];
        uint8_t* out[4];
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
            x[s4] = lds_quad_at(c.tile, c.tq0 + 1024u * (uint32_t)s4);
            out[s4] = reinterpret_cast<uint8_t*>(ptab[16 * s4]);
        }
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) stg16(out[s4] + off, 0, x[s4]);
    }
}

__device__ __forceinline__ void scale_task(const DecoderCtx& c, const Task& k, uint32_t (&ct)[16],
                                           const Task& nxt) {
    const IngressParams& p = *c.p;
    uint32_t* flags = c.lds + kLdsFlags;
    uint32_t sc[16];
    {
        uint32_t ks[16];
        chacha_block_cached(p.key, c.nc, 1u + (uint32_t)k.block, c.n0, c.n1, c.n2, ks);
#pragma unroll
        for (int i = 0; i < 16; ++i) sc[i] = ct[i] ^ ks[i];
    }
    if (nxt.valid) load_block(c.pay + 64u * (uint32_t)nxt.block, ct);
    if (params_nonfinite(sc)) flags[kFlagNaN + c.lane] = 1u;
    const int slot_s = k.g % kStage;
    wait_ge<kDiagIngressWait, kTmFreeWait>(&flags[kFlagFree + slot_s], k.g - kStage + 1, c.wt);
    uint32_t* stage = c.lds + kLdsStage + slot_s * kRowWords;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        lds_put_quad_at(stage, c.pq.off[q], make_uint4(sc[4 * q], sc[4 * q + 1], sc[4 * q + 2], sc[4 * q + 3]));
    publish(&flags[kFlagReady + slot_s], (uint32_t)k.g + 1u);
}

template <int DT, int FAM>
__device__ __forceinline__ void decode_rows(const DecoderCtx& c, const Layout& lay) {
    uint32_t* flags = c.lds + kLdsFlags;
    // (also reads how many rows the verify wave has absorbed, for the priority)
    int32_t used = 0;
    auto grab = [&]() -> int32_t {
        uint32_t t = 0;
        const uint32_t u = __hip_atomic_load(&flags[kFlagMacUsed], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (c.lane == 0)
            t = __hip_atomic_fetch_add(&flags[kFlagTask], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        used = (int32_t)__builtin_amdgcn_readfirstlane(u);
        return (int32_t)__builtin_amdgcn_readfirstlane(t);
    };
    const int32_t total = total_tasks(lay);
    int32_t t = grab();
    Task k = task_info<FAM>(lay, t);
    uint32_t ct[16];
    if constexpr (kPhaseTimers) tm_min(c.wt.tm, kTmProdSetup, phase_clock() - c.wt.t0);
    if (k.valid) load_block(c.pay + 64u * (uint32_t)k.block, ct);
    // The layout, descriptor and pointer-table reads complete here, before
    // the loop: a load still counted as in flight where the loop begins makes
    // the compiler wait for every outstanding memory operation wherever the
    // loop uses its result.
    __builtin_amdgcn_s_waitcnt(0);
    if constexpr (kPhaseTimers) tm_min(c.wt.tm, kTmProdLoaded, phase_clock() - c.wt.t0);
    [[maybe_unused]] int32_t made = 0;
#pragma unroll 1
    while (t < total) {
        const int32_t tn = grab();
        if constexpr (kPhaseTimers) {
            if (made++ == 1) tm_min(c.wt.tm, kTmProdFirstRow, phase_clock() - c.wt.t0);
        }
        set_row_priority(task_lead_row(k) - used);
        const Task nxt = task_info<FAM>(lay, tn);
        if (k.scale)
            scale_task(c, k, ct, nxt);
        else if (k.s.kind == kSecInt8)
            code_task<DT, kSecInt8>(c, k, ct, nxt);
        else if (k.s.kind == kSecInt4)
            code_task<DT, kSecInt4>(c, k, ct, nxt);
        else if (FAM == 0 || k.s.kind == kSecRaw)
            code_task<DT, kSecRaw>(c, k, ct, nxt);
        else if constexpr (FAM == 1) {
            if (k.s.kind == kSecE4m3)
                code_task_ext<DT, kSecE4m3>(c, k, ct, nxt);
            else if (k.s.kind == kSecInt4G32)
                code_task_ext<DT, kSecInt4G32>(c, k, ct, nxt);
            else
                code_task_ext<DT, kSecAsym8>(c, k, ct, nxt);
        }
        t = tn;
        k = nxt;
    }
    if constexpr (kPhaseTimers) {
        const uint64_t now = phase_clock() - c.wt.t0;
        tm_max(c.wt.tm, kTmProdLast, now);
        tm_add(c.wt.tm, kTmProdBusy, now);
        tm_add(c.wt.tm, kTmProdWaves, 1);
        tm_add(c.wt.tm, kTmRows, (uint64_t)made);
    }
}

// Feeder: copies every payload row that is not a code row of the workgroup
// layout (scale rows, padding; all rows when no page has a usable layout)
// from the blob into the ring, in payload order, two rows in flight.  It
// depends only on the verify wave freeing slots, so the rows before any row
// it waits for are always in the ring already.
__device__ __forceinline__ void feed_put(const Waiter& wt, uint32_t* lds, const PageQuads& pq, int32_t r,
                                         const uint4 (&x)[4]) {
    uint32_t* flags = lds + kLdsFlags;
    wait_ge<kDiagIngressWait, kTmFeedWait>(&flags[kFlagMacUsed], r - kRing + 1, wt);
    uint32_t* slot = lds + (r % kRing) * kRowWords;
#pragma unroll
    for (int q = 0; q < 4; ++q) lds_put_quad_at(slot, pq.off[q], x[q]);
    publish(&flags[kFlagRing + r % kRing], (uint32_t)r + 1u);
    tm_trace(wt.trace, r, wt.t0);
}

__device__ void ingress_feed(const IngressParams& p, uint32_t* lds, const Layout& lay, bool has_lay,
                             const uint8_t* pay, int lane) {
    PageQuads pq;
    pq.init(lane);
    Waiter wt = make_waiter(p.sink, lds + kLdsFlags + kFlagExpired, lds + kLdsTimers, phase_clock());
    wt.trace = trace_of(p.timers);
    const int32_t total = (int32_t)(p.payload / 64u);
    // payload rows [cb_i, ce_i) are section i's code rows (decoders)
    int32_t cb[3], ce[3];
#pragma unroll
    for (int si = 0; si < 3; ++si) {
        const bool on = has_lay && si < lay.n_sec;
        const int32_t kind = ZTCP_SEC_FIELD(lay, si, kind);
        cb[si] = on ? (int32_t)(ZTCP_SEC_FIELD(lay, si, q_off) / 64u) : 0;
        ce[si] = cb[si] + (on ? ZTCP_SEC_FIELD(lay, si, n_units) * code_rows_per_unit(kind) : 0);
    }
    auto next_fed = [&](int32_t r) {
#pragma unroll
        for (int si = 0; si < 3; ++si) r = (r >= cb[si] && r < ce[si]) ? ce[si] : r;
        return r;
    };
    // loads past the last row read the last row again (never put)
    auto load = [&](int32_t r, uint4 (&x)[4]) {
        const uint8_t* q = pay + 64u * (uint32_t)min(r, total - 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = ldg16(q, i);
    };
    int32_t ra = next_fed(0);
    if (ra >= total) return;
    struct FeedEnd {  // the feeder's end time, on every return path
        const Waiter& w;
        __device__ ~FeedEnd() {
            if constexpr (kPhaseTimers) tm_max(w.tm, kTmFeedEnd, phase_clock() - w.t0);
        }
    } feed_end{wt};
    uint4 a[4], b[4];
    load(ra, a);
    int32_t rb = next_fed(ra + 1);
    load(rb, b);
#pragma unroll 1
    for (;;) {
        feed_put(wt, lds, pq, ra, a);
        if (rb >= total) break;
        ra = next_fed(rb + 1);
        load(ra, a);
        feed_put(wt, lds, pq, rb, b);
        if (ra >= total) break;
        rb = next_fed(ra + 1);
        load(rb, b);
    }
}

// The checks of one page in the reference's order (cpp:2313-2355), given
// its header words and the xor of the stored and computed tags.
__device__ __forceinline__ int32_t page_verdict(const IngressParams& p, int64_t page, const uint4 h0, const uint4 h1,
                                                uint32_t tag_diff) {
    const uint64_t tok = ingress_token(p, page);
    const uint32_t layer = ingress_layer(p, page);
    const uint32_t magic = h0.x & 0xFFFFu, version = (h0.x >> 16) & 0xFFu;
    if (magic != kMagic || version != kVersion) return 1;
    if (h0.y != p.exp_tenant || h0.z != p.exp_model || (h0.w & 0xFFFFu) != layer || lo64(h1) != tok) return 2;
    if (tag_diff != 0u) return 3;
    if (layout_index(p, h0.x) < 0) return 1;
    return 0;
}

// Verdict of one page (cpp:2313-2355).  The payload's full 64-byte rows
// come from the ring; its last (payload % 64) bytes and the tag are loaded
// with the header.
__device__ __forceinline__ int32_t verify_page(const IngressParams& p, int64_t page, uint32_t* lds, int lane,
                                               const uint4 h0, const uint4 h1, uint64_t t0) {
    const uint8_t* blob = ingress_blob(p, page);
    const uint8_t* pay = blob + kHeader;
    const int32_t total = (int32_t)(p.payload / 64u);
    const uint32_t tail0 = (uint32_t)total * 64u;
    const int ntail = (int)((p.payload - tail0) / 16u);  // 0..3 chunks of 16 bytes
    uint4 tl[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) tl[i] = ldg16(pay + min(tail0 + 16u * (uint32_t)i, p.payload), 0);
    const uint4 tag = ldg16(pay + p.payload, 0);
    Sip s;
    s.init(p.mk0, p.mk1);
    const uint64_t hdr[4] = {lo64(h0), hi64(h0), lo64(h1), hi64(h1)};
    s.absorb_words<4>(hdr);
    PageQuads pq;
    pq.init(lane);
    Waiter st = make_waiter(p.sink, lds + kLdsFlags + kFlagExpired, lds + kLdsTimers, t0);
    st.trace = trace_of(p.timers);
    __builtin_amdgcn_s_waitcnt(0);
    if constexpr (kPhaseTimers) tm_add(st.tm, kTmMacRowsBegin, phase_clock() - t0);
    mac_rows<kRing, kDiagIngressWait>(st, lds, lds + kLdsFlags + kFlagRing, lds + kLdsFlags + kFlagMacUsed, pq, s,
                                      total);
    if constexpr (kPhaseTimers) tm_add(st.tm, kTmMacRowsEnd, phase_clock() - t0);
#pragma unroll
    for (int i = 0; i < 3; ++i)
        if (i < ntail) s.absorb(tl[i]);
    uint64_t lo, hi;
    s.finish((uint64_t)((kHeader + p.payload) & 0xFFu) << 56, lo, hi);
    const uint32_t diff = (tag.x ^ (uint32_t)lo) | (tag.y ^ (uint32_t)(lo >> 32)) |
                          (tag.z ^ (uint32_t)hi) | (tag.w ^ (uint32_t)(hi >> 32));
    if constexpr (kPhaseTimers) tm_add(st.tm, kTmMacEnd, phase_clock() - t0);
    return page_verdict(p, page, h0, h1, diff);
}

// Pages of a workgroup whose valid layout is not the workgroup's: unit by
// unit, one page per wave (after the barrier that ends the row pipeline).
template <int DT, int FAM, int NWAVES>
__device__ __forceinline__ void decode_other_layouts(const IngressParams& p, int64_t page0, bool active, int li,
                                                     int li_wg, const uint4 h0, const uint4 h1,
                                                     const Layout* layouts, uint32_t* nan) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint64_t other = __ballot(active && li >= 0 && li != li_wg);
    if (other) {
        int n = 0;
#pragma unroll 1
        for (uint64_t m = other; m; m &= m - 1, ++n) {
            if (n % NWAVES != wave) continue;
            const int pl = (int)__builtin_ctzll(m);
            const int lp = __builtin_amdgcn_readlane(li, pl);
            const Layout& L2 = layouts[lp];
            const uint32_t a0 = __builtin_amdgcn_readlane(h1.z, pl), a1 = __builtin_amdgcn_readlane(h1.w, pl);
            const uint32_t a2 = __builtin_amdgcn_readlane(h0.w, pl);
            const uint32_t m2 = ((a2 & 0xFFFFu) << 16) | (a2 >> 16);
#pragma unroll 1
            for (int u = lane; u < L2.n_units; u += 64)
                decode_unit<DT, FAM>(p, L2, page0 + pl, u, a0, a1, m2, &nan[pl]);
        }
        __builtin_amdgcn_s_waitcnt(0);  // every decode store has completed before the zeroing
    }
    __syncthreads();
}

// The end of an ingress workgroup (every thread): NaN rewrite of verified
// pages, fail closed after an expired wait, verdicts out, and the per-page
// policy's zeroing.  status / nan: one word per page of the workgroup (LDS).
template <int DT>
__device__ __forceinline__ void ingress_epilogue(const IngressParams& p, int64_t page0, int ppw, uint32_t* status,
                                                 const uint32_t* nan, const uint32_t* expired_word, uint32_t* tm,
                                                 uint64_t t0, uint64_t rt0) {
    // Verified pages with an inf / NaN scale (only possible when |values| pass
    // 65504 times the code range, so with BF16 data): their NaN outputs are
    // rewritten as the reference's conversions write them.  Every store to
    // them has completed (the barriers that end the decode and the other
    // layouts' decode, before this call).
#pragma unroll 1
    for (int pl = 0; pl < ppw; ++pl) {
        if (nan[pl] == 0u || status[pl] != 0u) continue;
        const int64_t n16 = p.page_bytes / 16;
        uint8_t* k = ingress_k(p, page0 + pl);
        uint8_t* v = ingress_v(p, page0 + pl);
        for (int64_t i = threadIdx.x; i < 2 * n16; i += blockDim.x) {
            uint8_t* b = i < n16 ? k : v;
            if (!b) continue;
            const uint4 x = ldg16(b, i % n16);
            uint32_t w[8] = {x.x, x.y, x.z, x.w, 0u, 0u, 0u, 0u};
            canonical_nans<DT>(w);
            stg16(b, i % n16, make_uint4(w[0], w[1], w[2], w[3]));
        }
        __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();
    // Fail closed: after an expired bounded wait, a page's verdict and its
    // decoded bytes may come from rows handed over out of turn, so every page
    // of the workgroup fails with ZTCP_ERR_DEVICE and its outputs are zeroed
    // like any failing page's.
    const bool expired = *expired_word != 0u;
    if (expired && (int)threadIdx.x < ppw) status[threadIdx.x] = (uint32_t)ZTCP_ERR_DEVICE;
    __syncthreads();
    tm_flush(tm, p.timers, t0, rt0);
    if ((int)threadIdx.x < ppw) {
        const int32_t st = (int32_t)status[threadIdx.x];
        const int64_t pg = page0 + threadIdx.x;
        if (p.page_status) p.page_status[pg] = st;
        if (st != 0) atomicMin(&p.call->fail, ((unsigned long long)pg << 8) | (unsigned long long)st);
    }
    if (p.per_page) {  // extension: zero only the failing pages
        const int64_t n16 = p.page_bytes / 16;
#pragma unroll 1
        for (int pl = 0; pl < ppw; ++pl) {
            if (status[pl] == 0u) continue;
            uint8_t* k = ingress_k(p, page0 + pl);
            for (int64_t i = threadIdx.x; i < n16; i += blockDim.x) stg16(k, i, make_uint4(0, 0, 0, 0));
            uint8_t* v = ingress_v(p, page0 + pl);
            if (v)
                for (int64_t i = threadIdx.x; i < n16; i += blockDim.x) stg16(v, i, make_uint4(0, 0, 0, 0));
        }
    }
}

template <int DT, int FAM>
__global__ __launch_bounds__(kIngressThreads) void ingress_fused_kernel(IngressParams p) {
    extern __shared__ __align__(16) uint32_t lds[];
    const int64_t page0 = (int64_t)blockIdx.x * p.ppw;
    const int ppw = (int)min((int64_t)p.ppw, p.batch - page0);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const bool active = lane < ppw;
    const int64_t page = page0 + (active ? lane : 0);
    const uint8_t* blob = ingress_blob(p, page);
    // the 64 headers are loaded once, into LDS, for every wave
    uint4* hdrs = reinterpret_cast<uint4*>(lds + kLdsHeaders);
    if (threadIdx.x < 64) {
        hdrs[2 * threadIdx.x] = ldg16(blob, 0);
        hdrs[2 * threadIdx.x + 1] = ldg16(blob, 1);
    }
    // the 24 layouts live in LDS: a table in registers or in the kernel
    // arguments would be copied to scratch memory once indexed by a variable
    Layout* layouts = reinterpret_cast<Layout*>(lds + kLdsLayouts);
    if (threadIdx.x < kNumLayouts) layouts[threadIdx.x] = ingress_layout(p, (int)threadIdx.x);
    uint32_t* flags = lds + kLdsFlags;
    for (int i = threadIdx.x; i < kNumFlags; i += blockDim.x) flags[i] = 0u;
    tm_clear(lds + kLdsTimers);
    tm_trace_clear(p.timers);
    if (threadIdx.x < 64) {
        // Pages outside the row pipeline (another layout, invalid flags) get
        // its stores too: those of another layout are decoded again below,
        // after every row store has completed; failing pages are zeroed.
        uint64_t* ptrs = reinterpret_cast<uint64_t*>(lds + kLdsPtrs);
        uint8_t* k = ingress_k(p, page);
        uint8_t* v = ingress_v(p, page);
        ptrs[threadIdx.x] = reinterpret_cast<uint64_t>(k);
        ptrs[64 + threadIdx.x] = reinterpret_cast<uint64_t>(v ? v : k);
    }
    __syncthreads();
    [[maybe_unused]] const uint64_t t0 = phase_clock();
    [[maybe_unused]] const uint64_t rt0 = kPhaseTimers ? __builtin_amdgcn_s_memrealtime() : 0;
    // every wave derives the workgroup layout from the 64 headers itself
    const uint4 h0 = hdrs[2 * lane], h1 = hdrs[2 * lane + 1];
    const int li = layout_index(p, h0.x);
    const uint64_t any_valid = __ballot(active && li >= 0);
    const int li_wg = any_valid ? __builtin_amdgcn_readlane(li, (int)__builtin_ctzll(any_valid)) : -1;
    const bool has_lay = li_wg >= 0;
    const Layout& lay = layouts[has_lay ? li_wg : 0];
    if (wave == 0) {
        __builtin_amdgcn_s_setprio(3);
        flags[kFlagStatus + lane] = (uint32_t)verify_page(p, page, lds, lane, h0, h1, t0);
    } else if (wave == 4) {
        ingress_feed(p, lds, lay, has_lay, blob + kHeader, lane);
    } else if ((wave & 3) != 0 && has_lay) {  // waves 8 and 12 share SIMD 0 and idle
        DecoderCtx c;
        c.p = &p;
        c.pay = blob + kHeader;
        c.n0 = h1.z;  // nonce from the page's own header (cpp:2357-2365)
        c.n1 = h1.w;
        c.n2 = ((h0.w & 0xFFFFu) << 16) | (h0.w >> 16);
        c.nc.init(p.key, c.n0, c.n1, c.n2);
        c.lds = lds;
        c.tile = lds + kLdsTile + (wave - 1 - (wave >> 2)) * kRowWords;
        c.lane = lane;
        c.pq.init(lane);
        c.wt = make_waiter(p.sink, lds + kLdsFlags + kFlagExpired, lds + kLdsTimers, t0);
        c.wt.trace = trace_of(p.timers);
        c.init_stores();
        decode_rows<DT, FAM>(c, lay);
    }
    __builtin_amdgcn_s_waitcnt(0);  // every row store has completed
    __syncthreads();
    decode_other_layouts<DT, FAM, kIngressWaves>(p, page0, active, li, li_wg, h0, h1, layouts, flags + kFlagNaN);
    ingress_epilogue<DT>(p, page0, ppw, flags + kFlagStatus, flags + kFlagNaN, flags + kFlagExpired,
                         lds + kLdsTimers, t0, rt0);
}

// ---------------------------------------------------------------------------
// Small batches (at most kSiMaxPpw pages per workgroup, the reference's
// kinds).  As in egress_small_kernel: with lane = page most lanes of the row
// pipeline idle and the verify wave's chain waits for rows decoded one page
// at a time.  Here three loader waves copy every payload row of every page
// into LDS, lane = (row, page), 192 rows per pass, publishing their passes;
// the verify wave (one page per lane) absorbs the rows from LDS as the passes
// complete, so its chain runs at the lone rate.  After their load passes the
// same waves decode the pages with the workgroup's layout, lane = (unit,
// page), with the unit decoder the row-pipeline kernel uses for pages of
// another layout (scale row first, then the unit's code rows, from the
// blobs, which the loads have just brought into L2).  Pages of another valid
// layout are decoded unit by unit afterwards, and the epilogue is the
// row-pipeline kernel's.
// ---------------------------------------------------------------------------
constexpr int kSiWaves = 4;
constexpr int kSiMaxPpw = 4;
constexpr int kSiTasks = 64 * (kSiWaves - 1);  // tasks per pass
constexpr int kSiRowWords = 16;                // one 64-byte payload row of one page
constexpr int kSiFlagPass = 0;                 // [3] load passes completed by loader wave 1..3
constexpr int kSiFlagExpired = 4;              // 1: a bounded wait of the workgroup expired
constexpr int kSiFlagStatus = 8;               // [4] verdicts
constexpr int kSiFlagNaN = 12;                 // [4] 1: the page has an inf / NaN scale
constexpr int kSiFlags = 16;
constexpr int kSiTimers = kSiFlags;                                     // phase timers (timer builds)
constexpr int kSiHeaders = kSiTimers + kTimerLdsWords;                  // [4] 32-byte headers
constexpr int kSiLayouts = kSiHeaders + kSiMaxPpw * 8;                  // [kNumLayouts] Layout
constexpr int kSiPay = (kSiLayouts + kNumLayouts * kLayoutWords + 15) & ~15;  // payload copies, 64-byte aligned
static_assert(kSiHeaders % 4 == 0, "header table must be 16-byte aligned");

// Verdict of page `lane` (< ppw) from its payload copy in LDS.
__device__ __forceinline__ int32_t small_verify(const IngressParams& p, int64_t page0, int ppw, int32_t nrow,
                                                uint32_t* lds, const uint4 h0, const uint4 h1, uint64_t t0) {
    const int lane = threadIdx.x & 63;
    const bool active = lane < ppw;
    const int64_t page = page0 + (active ? lane : 0);
    const uint8_t* pay = ingress_blob(p, page) + kHeader;
    const uint32_t tail0 = (uint32_t)nrow * 64u;
    const int ntail = (int)((p.payload - tail0) / 16u);  // 0..3 chunks of 16 bytes
    uint4 tl[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) tl[i] = ldg16(pay + min(tail0 + 16u * (uint32_t)i, p.payload), 0);
    const uint4 tag = ldg16(pay + p.payload, 0);
    Sip s;
    s.init(p.mk0, p.mk1);
    const uint64_t hdr[4] = {lo64(h0), hi64(h0), lo64(h1), hi64(h1)};
    s.absorb_words<4>(hdr);
    uint32_t* flags = lds;
    const uint32_t* mine = lds + kSiPay + (size_t)(active ? lane : 0) * nrow * kSiRowWords;
    const Waiter wt = make_waiter(p.sink, flags + kSiFlagExpired, lds + kSiTimers, t0);
    int32_t r = 0;  // rows fetched
    auto fetch = [&](uint4 (&x)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) x[q] = *reinterpret_cast<const uint4*>(mine + r * kSiRowWords + 4 * q);
        ++r;
    };
    __builtin_amdgcn_s_waitcnt(0);
    if constexpr (kPhaseTimers) tm_add(wt.tm, kTmMacRowsBegin, phase_clock() - t0);
    int32_t done = 0, ready = 0;
#pragma unroll 1
    while (done < nrow) {
        if (done >= ready) {  // the pass that loads row `done` of the last page
            [[maybe_unused]] const uint64_t t_in = phase_clock();
            const int32_t need = (done * ppw + ppw - 1) / kSiTasks + 1;
#pragma unroll 1
            for (int w2 = 0; w2 < kSiWaves - 1; ++w2) wait_ge<kDiagIngressWait>(&flags[kSiFlagPass + w2], need, wt);
            ready = min(nrow, need * kSiTasks / ppw);
            if constexpr (kPhaseTimers) {
                tm_add(wt.tm, kTmMacWait + min(done >> 6, 7), phase_clock() - t_in);
                if (done == 0) tm_add(wt.tm, kTmMacFirstRow, phase_clock() - t0);
            }
        }
        const int32_t n = ready - done;
        sip_stream64(s, (uint32_t)n, fetch);
        done += n;
    }
    if constexpr (kPhaseTimers) tm_add(wt.tm, kTmMacRowsEnd, phase_clock() - t0);
#pragma unroll
    for (int i = 0; i < 3; ++i)
        if (i < ntail) s.absorb(tl[i]);
    uint64_t lo, hi;
    s.finish((uint64_t)((kHeader + p.payload) & 0xFFu) << 56, lo, hi);
    const uint32_t diff = (tag.x ^ (uint32_t)lo) | (tag.y ^ (uint32_t)(lo >> 32)) |
                          (tag.z ^ (uint32_t)hi) | (tag.w ^ (uint32_t)(hi >> 32));
    if constexpr (kPhaseTimers) tm_add(wt.tm, kTmMacEnd, phase_clock() - t0);
    return page_verdict(p, page, h0, h1, diff);
}

template <int DT>
__device__ void small_load_decode(const IngressParams& p, int64_t page0, int ppw, int32_t nrow, uint32_t* lds,
                                  int li_wg, uint64_t t0) {
    const int lw = (int)(threadIdx.x >> 6) - 1;
    const int lane = threadIdx.x & 63;
    uint32_t* flags = lds;
    uint32_t* pay = lds + kSiPay;
    const uint4* hdrs = reinterpret_cast<const uint4*>(lds + kSiHeaders);
    const Waiter wt = make_waiter(p.sink, flags + kSiFlagExpired, lds + kSiTimers, t0);
    const int32_t ntask = nrow * ppw;
    const int32_t npass = (ntask + kSiTasks - 1) / kSiTasks;
#pragma unroll 1
    for (int32_t k = 0; k < npass; ++k) {
        const int32_t t = k * kSiTasks + lw * 64 + lane;
        if (t < ntask) {
            const int32_t r = t / ppw, i = t - r * ppw;
            const uint8_t* src = ingress_blob(p, page0 + i) + kHeader + 64u * (uint32_t)r;
            uint32_t* dst = pay + ((size_t)i * nrow + r) * kSiRowWords;
            uint4 x[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) x[q] = ldg16(src, q);
#pragma unroll
            for (int q = 0; q < 4; ++q) *reinterpret_cast<uint4*>(dst + 4 * q) = x[q];
        }
        publish(&flags[kSiFlagPass + lw], (uint32_t)k + 1u);
        if constexpr (kPhaseTimers) {
            if (k == 0) tm_min(wt.tm, kTmProdFirstRow, phase_clock() - t0);
        }
    }
    if (li_wg >= 0) {
        // the units of the pages with the workgroup's layout, lane = (unit,
        // page), from the blobs (in L2 since the loads above)
        const Layout& lay = reinterpret_cast<const Layout*>(lds + kSiLayouts)[li_wg];
        const int32_t ntask2 = lay.n_units * ppw;
#pragma unroll 1
        for (int32_t t = lw * 64 + lane; t < ntask2; t += kSiTasks) {
            const int32_t u = t / ppw, i = t - u * ppw;
            const uint4 h0 = hdrs[2 * i], h1 = hdrs[2 * i + 1];
            if (layout_index(p, h0.x) != li_wg) continue;
            const uint32_t n2 = ((h0.w & 0xFFFFu) << 16) | (h0.w >> 16);  // nonce (cpp:2357-2365)
            decode_unit<DT, 0>(p, lay, page0 + i, u, h1.z, h1.w, n2, &flags[kSiFlagNaN + i]);
        }
    }
    if constexpr (kPhaseTimers) {
        tm_max(wt.tm, kTmProdLast, phase_clock() - t0);
        tm_add(wt.tm, kTmProdWaves, 1);
    }
}

// One workgroup per CU at most (grid = batch / pages per workgroup <= CU
// count), one wave per SIMD: registers need not be shared.
template <int DT>
__global__ __launch_bounds__(64 * kSiWaves) __attribute__((amdgpu_waves_per_eu(1, 1)))
void ingress_small_kernel(IngressParams p) {
    extern __shared__ __align__(16) uint32_t lds[];
    const int64_t page0 = (int64_t)blockIdx.x * p.ppw;
    const int ppw = (int)min((int64_t)p.ppw, p.batch - page0);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const bool active = lane < ppw;
    const int32_t nrow = (int32_t)(p.payload / 64u);
    uint32_t* flags = lds;
    uint4* hdrs = reinterpret_cast<uint4*>(lds + kSiHeaders);
    if ((int)threadIdx.x < ppw) {
        const uint8_t* b = ingress_blob(p, page0 + threadIdx.x);
        hdrs[2 * threadIdx.x] = ldg16(b, 0);
        hdrs[2 * threadIdx.x + 1] = ldg16(b, 1);
    }
    Layout* layouts = reinterpret_cast<Layout*>(lds + kSiLayouts);
    if (threadIdx.x < kNumLayouts) layouts[threadIdx.x] = ingress_layout(p, (int)threadIdx.x);
    if (threadIdx.x < kSiFlags) flags[threadIdx.x] = 0u;
    tm_clear(lds + kSiTimers);
    __syncthreads();
    [[maybe_unused]] const uint64_t t0 = phase_clock();
    [[maybe_unused]] const uint64_t rt0 = kPhaseTimers ? __builtin_amdgcn_s_memrealtime() : 0;
    // every wave derives the workgroup layout from the headers itself
    const int lp = active ? lane : 0;
    const uint4 h0 = hdrs[2 * lp], h1 = hdrs[2 * lp + 1];
    const int li = layout_index(p, h0.x);
    const uint64_t any_valid = __ballot(active && li >= 0);
    const int li_wg = any_valid ? __builtin_amdgcn_readlane(li, (int)__builtin_ctzll(any_valid)) : -1;
    if (wave == 0) {
        __builtin_amdgcn_s_setprio(3);
        const int32_t v = small_verify(p, page0, ppw, nrow, lds, h0, h1, t0);
        if (active) flags[kSiFlagStatus + lane] = (uint32_t)v;
    } else {
        small_load_decode<DT>(p, page0, ppw, nrow, lds, li_wg, t0);
    }
    __builtin_amdgcn_s_waitcnt(0);  // every decode store has completed
    __syncthreads();
    decode_other_layouts<DT, 0, kSiWaves>(p, page0, active, li, li_wg, h0, h1, layouts, flags + kSiFlagNaN);
    ingress_epilogue<DT>(p, page0, ppw, flags + kSiFlagStatus, flags + kSiFlagNaN, flags + kSiFlagExpired,
                         lds + kSiTimers, t0, rt0);
}

}  // namespace

// All-or-nothing epilogue (cpp:2481-2486): if any page failed, zero both
// outputs entirely.  Every block reads the failure word once.
__global__ void ingress_finalize_kernel(IngressParams p) {
    if (p.call->fail == ~0ull) return;
    const int64_t n16 = p.page_bytes / 16;
    const int64_t total = n16 * p.batch;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t page = i / n16, off = i - page * n16;
        stg16(ingress_k(p, page), off, make_uint4(0, 0, 0, 0));
        uint8_t* v = ingress_v(p, page);
        if (v) stg16(v, off, make_uint4(0, 0, 0, 0));
    }
}

__global__ void reset_call_kernel(CallState* call) {
    call->fail = ~0ull;
    call->diag = 0u;
}

hipError_t launch_ingress_fused(const IngressParams& p, int dtype, hipStream_t s) {
    const int64_t grid = (p.batch + p.ppw - 1) / p.ppw;
    const size_t lds = (size_t)kLdsWords * sizeof(uint32_t);  // above 64 KiB: gfx950 has 160 KiB per CU
    // family 1 (the extension kinds) only when the call enables the extension layouts
    const bool ext = (p.lay_ok >> 12) != 0u;  // bits of presets 4..6 (index (preset - 1) * 4 + rope_mode)
    const bool ext_rope = (p.lay_ok & 0x888u) != 0u;  // RoPE mode 3 of presets 1..3
    // small batches of the reference's kinds: every page's payload in LDS
    const size_t small_lds = sizeof(uint32_t) * ((size_t)kSiPay + (size_t)p.ppw * (p.payload / 64u) * kSiRowWords);
    if (!ext && !ext_rope && p.ppw <= kSiMaxPpw && small_lds <= 160u * 1024u) {
        const dim3 g((uint32_t)grid), b(64 * kSiWaves);
        if (dtype == kHotBf16) hipLaunchKernelGGL(ingress_small_kernel<kHotBf16>, g, b, small_lds, s, p);
        else hipLaunchKernelGGL(ingress_small_kernel<kHotFp16>, g, b, small_lds, s, p);
        return hipGetLastError();
    }
    if (dtype == kHotBf16) {
        if (ext || ext_rope)
            hipLaunchKernelGGL((ingress_fused_kernel<kHotBf16, 1>), dim3((uint32_t)grid), dim3(kIngressThreads), lds, s, p);
        else
            hipLaunchKernelGGL((ingress_fused_kernel<kHotBf16, 0>), dim3((uint32_t)grid), dim3(kIngressThreads), lds, s, p);
    } else {
        if (ext || ext_rope)
            hipLaunchKernelGGL((ingress_fused_kernel<kHotFp16, 1>), dim3((uint32_t)grid), dim3(kIngressThreads), lds, s, p);
        else
            hipLaunchKernelGGL((ingress_fused_kernel<kHotFp16, 0>), dim3((uint32_t)grid), dim3(kIngressThreads), lds, s, p);
    }
    return hipGetLastError();
}

hipError_t launch_ingress_finalize(const IngressParams& p, hipStream_t s) {
    const int64_t total = (p.page_bytes / 16) * p.batch;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(ingress_finalize_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_reset_call(CallState* call, hipStream_t s) {
    hipLaunchKernelGGL(reset_call_kernel, dim3(1), dim3(1), 0, s, call);
    return hipGetLastError();
}

}  // namespace ztcp
