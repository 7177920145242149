// ztcp_ingress.hip -- fused cold-page ingress for gfx950:
// verify (header, AAD, SipHash tag) -> ChaCha20 decrypt -> dequantize, one
// HBM read of the blob and one HBM write of the hot page.  Replaces the
// per-page decoder of fused_decode_cold_pages_peak_into_cpu (cpp:2309-2463).
//
// One workgroup handles up to 64 pages with 12 waves (lane = page):
//   * Every page is decoded according to its own header flags.  The
//     workgroup's layout is that of its first page with valid flags; pages
//     with that layout go through the row pipeline below, pages with another
//     valid layout are decoded afterwards unit by unit, pages with invalid
//     flags are not decoded (they fail with status 1).
//   * Nine decoder waves take rows in order from an LDS counter, each with
//     its ciphertext block loaded one row ahead.  A unit's scale row is
//     decrypted into an LDS staging slot two units ahead of its code rows.  A
//     code row first puts its ciphertext into a ring of row slots in LDS for
//     the verify wave, then decrypts, takes its scales from staging and
//     dequantizes two groups at a time into a per-wave LDS tile, from which
//     the wave stores them transposed: four lanes per page, so each store
//     writes the two groups (64 bytes, contiguous within a head vector) of
//     16 pages.
//   * Wave 0 verifies one page per lane at raised priority on a SIMD of its
//     own (waves 4 and 8, which the dispatcher places there, exit at once):
//     magic/version (status 1), AAD tenant/model/layer/token hash (status
//     2), the SipHash-2-4-128 tag over header || ciphertext (status 3), then
//     flags and payload size (status 1), in the reference's order
//     (cpp:2313-2355).  Code rows of the workgroup's layout come from the
//     LDS ring, every other 64-byte chunk (scales, padding) from the blob.
//   * Decoding is speculative: a page whose verdict is not OK has its outputs
//     zeroed before the kernel ends (per-page mode) or by the finalize kernel
//     (all-or-nothing mode, which zeroes every output, cpp:2481-2486).
//     Outputs are only valid after the call returns OK, as with the
//     reference.
//   * Hand-offs are monotonic LDS counters (ring_flag, mac_used, scale_ready,
//     scale_free) with workgroup-scope release/acquire; every wait is bounded
//     and only points backwards in row order.
// Requires 16-byte aligned blobs / outputs, blob_bytes % 16 == 0 and every
// layout aligned to 64-byte units; otherwise the host uses the generic path.
#include "ztcp_rows.h"

namespace ztcp {

namespace {

constexpr int kRing = 16;        // code rows between decoders and the verify wave
constexpr int kStage = 8;        // units whose decrypted scales are staged at once
constexpr int kLookahead = 2;    // a unit's scale row is handed out this many units early
constexpr int kLdsStage = kRing * kRowWords;
constexpr int kLdsTile = kLdsStage + kStage * kRowWords;       // per decoder wave: 2 groups per page
constexpr int kLdsFlags = kLdsTile + kProducerWaves * kRowWords;
constexpr int kFlagRing = 0;                         // [kRing] code row index + 1
constexpr int kFlagReady = kFlagRing + kRing;        // [kStage] unit + 1: scales decrypted
constexpr int kFlagFree = kFlagReady + kStage;       // [kStage] unit + 1: scales consumed
constexpr int kFlagCount = kFlagFree + kStage;       // [kStage] code rows that took their scales
constexpr int kFlagMacUsed = kFlagCount + kStage;    // code rows absorbed by the verify wave
constexpr int kFlagTask = kFlagMacUsed + 1;          // next row to hand out
constexpr int kFlagStatus = kFlagTask + 1;           // [64] verdicts
constexpr int kNumFlags = kFlagStatus + 64;
constexpr int kLdsPtrs = kLdsFlags + kNumFlags + (kNumFlags & 1);  // [2][64] output pointers
constexpr int kLdsLayouts = kLdsPtrs + 2 * 2 * 64;   // [9] Layout, one per header flags value
constexpr int kLayoutWords = (int)(sizeof(Layout) / 4);
constexpr int kLdsWords = kLdsLayouts + 9 * kLayoutWords;
static_assert(sizeof(Layout) % 4 == 0, "Layout is copied word by word");

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

// Layout index (preset - 1) * 3 + rope_mode of a header's flags, or -1 when
// the flags are invalid or the payload is too short for them.
__device__ __forceinline__ int layout_index(const IngressParams& p, uint32_t h0x) {
    const uint32_t flags = h0x >> 24, preset = flags & 0x0Fu, rope_mode = flags >> 4;
    if (preset < 1u || preset > 3u || rope_mode > 2u) return -1;
    const int li = (int)((preset - 1u) * 3u + rope_mode);
    return ((p.lay_ok >> li) & 1u) ? li : -1;
}

// ---------------------------------------------------------------------------
// Unit-by-unit decode for pages whose layout is not the workgroup's.
// ---------------------------------------------------------------------------

template <int DT, int KIND>
__device__ __forceinline__ void decode_quant_unit(const IngressParams& p, const uint8_t* pay,
                                                  uint8_t* out, int32_t lu, int32_t gpv,
                                                  int32_t col, uint32_t q_off, uint32_t s_off,
                                                  uint32_t n0, uint32_t n1, uint32_t n2) {
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

template <int DT>
__device__ __forceinline__ void decode_unit(const IngressParams& p, const Layout& lay, int64_t page, int32_t u,
                            uint32_t n0, uint32_t n1, uint32_t n2) {
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
        decode_quant_unit<DT, kSecInt8>(p, pay, out, lu, gpv, col, q_off, s_off, n0, n1, n2);
    else if (kind == kSecInt4)
        decode_quant_unit<DT, kSecInt4>(p, pay, out, lu, gpv, col, q_off, s_off, n0, n1, n2);
    else
        decode_raw_unit(p, pay, out, lu, gpv, col, q_off, n0, n1, n2);
}

// ---------------------------------------------------------------------------
// Row pipeline.
// ---------------------------------------------------------------------------

// Row t of the decode order.  Per section of U units: the scale rows of units
// 0 .. L-1, then for each unit u its code rows followed by the scale row of
// unit u + L (L = kLookahead), so a unit's scales are decrypted while the
// units before it are being decoded.
struct Task {
    int32_t valid;
    int32_t scale;    // 1: scale row of unit u
    int32_t u, j;     // unit in section, code block in unit
    int32_t g;        // unit index among the page's quantized units (staging order)
    int32_t cidx;     // code row index (payload order)
    int32_t block;    // payload block index (keystream counter - 1)
    SecRows s;
};

__device__ __forceinline__ int32_t div_nblk(int32_t x, int32_t kind) {  // nblk = 8, 4, 16
    return kind == kSecInt8 ? x / 8 : (kind == kSecInt4 ? x / 4 : x / 16);
}
__device__ __forceinline__ int32_t div_rpu(int32_t x, int32_t kind) {  // nblk + 1 = 9, 5
    return kind == kSecInt8 ? x / 9 : x / 5;
}

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
                k.u = div_nblk(x, s.kind);
                k.j = x - k.u * s.nblk;
            } else {
                const int32_t pre = min(kLookahead, s.n_units);
                const int32_t full = max(s.n_units - kLookahead, 0);  // units followed by a scale row
                if (x < pre) {
                    k.scale = 1;
                    k.u = x;
                } else if ((x -= pre) < full * s.rpu) {
                    const int32_t u = div_rpu(x, s.kind), r = x - u * s.rpu;
                    k.scale = r == s.nblk;
                    k.u = k.scale ? u + kLookahead : u;
                    k.j = k.scale ? 0 : r;
                } else {
                    x -= full * s.rpu;
                    const int32_t u = div_nblk(x, s.kind);
                    k.u = full + u;
                    k.j = x - u * s.nblk;
                }
            }
            k.g = s.qunit_begin + k.u;
            k.cidx = cb + k.u * s.nblk + k.j;
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
        t += ZTCP_SEC_FIELD(lay, si, n_units) * (kind == kSecInt8 ? 9 : (kind == kSecInt4 ? 5 : 16));
    }
    return t;
}

// Byte offset of group G of a section inside the page's K or V buffer.
__device__ __forceinline__ uint32_t group_offset(const SecRows& s, int32_t G, int32_t head_dim) {
    const int32_t vec = G / s.gpv, gi = G - vec * s.gpv;
    return (uint32_t)vec * (uint32_t)head_dim * 2u + (uint32_t)(s.col + gi * 16) * 2u;
}

struct DecoderCtx {
    const IngressParams* p;
    const uint8_t* pay;     // this lane's page payload
    uint32_t n0, n1, n2;    // this lane's page nonce (from its header)
    ChaChaNonceCache nc;
    uint32_t* lds;
    uint32_t* tile;         // this wave's dequantized tile
    int lane;
};

// Stores the wave's tile (two groups G, G + 1 of 64 pages) transposed: lane l
// writes 16 bytes of page 16 k + (l >> 2).
__device__ __forceinline__ void store_tile(const DecoderCtx& c, const SecRows& s, int32_t G) {
    const uint64_t* ptrs = reinterpret_cast<const uint64_t*>(c.lds + kLdsPtrs) + (s.src ? 64 : 0);
    const int q = c.lane & 3;
    const uint32_t off = group_offset(s, G + (q >> 1), c.p->head_dim) + 16u * (uint32_t)(q & 1);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int pr = 16 * k + (c.lane >> 2);
        const uint4 x = lds_quad(c.tile, pr, q);
        uint8_t* out = reinterpret_cast<uint8_t*>(ptrs[pr]);
        if (out) stg16(out + off, 0, x);
    }
}

template <int DT, int KIND>
__device__ __forceinline__ void code_task(const DecoderCtx& c, const Task& k, uint32_t (&ct)[16],
                                          const Task& nxt) {
    constexpr int GPB = KIND == kSecInt8 ? 4 : (KIND == kSecInt4 ? 8 : 2);
    constexpr int SW = GPB / 2;  // scale words of this row
    const IngressParams& p = *c.p;
    uint32_t* flags = c.lds + kLdsFlags;
    // ciphertext to the verify wave
    uint32_t* slot = c.lds + (k.cidx % kRing) * kRowWords;
    wait_ge<kDiagIngressWait>(&flags[kFlagMacUsed], k.cidx - kRing + 1, p.state);
#pragma unroll
    for (int q = 0; q < 4; ++q)
        lds_put_quad(slot, c.lane, q, make_uint4(ct[4 * q], ct[4 * q + 1], ct[4 * q + 2], ct[4 * q + 3]));
    publish(&flags[kFlagRing + k.cidx % kRing], (uint32_t)k.cidx + 1u);
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
        wait_ge<kDiagIngressWait>(&flags[kFlagReady + slot_s], k.g + 1, p.state);
        const uint32_t* stage = c.lds + kLdsStage + slot_s * kRowWords;
#pragma unroll
        for (int t = 0; t < SW; ++t) {
            const int wd = k.j * SW + t;
            sc[t] = stage[quad_word(c.lane, wd >> 2) + (wd & 3)];
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
    const int32_t G0 = k.u * 32 + k.j * GPB;
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
            lds_put_quad(c.tile, c.lane, q, make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]));
        store_tile(c, k.s, G0 + 2 * pc);
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
    const int slot_s = k.g % kStage;
    wait_ge<kDiagIngressWait>(&flags[kFlagFree + slot_s], k.g - kStage + 1, p.state);
    uint32_t* stage = c.lds + kLdsStage + slot_s * kRowWords;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        lds_put_quad(stage, c.lane, q, make_uint4(sc[4 * q], sc[4 * q + 1], sc[4 * q + 2], sc[4 * q + 3]));
    publish(&flags[kFlagReady + slot_s], (uint32_t)k.g + 1u);
}

template <int DT>
__device__ __forceinline__ void decode_rows(const DecoderCtx& c, const Layout& lay) {
    uint32_t* flags = c.lds + kLdsFlags;
    auto grab = [&]() -> int32_t {
        uint32_t t = 0;
        if (c.lane == 0)
            t = __hip_atomic_fetch_add(&flags[kFlagTask], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        return (int32_t)__builtin_amdgcn_readfirstlane(t);
    };
    const int32_t total = total_tasks(lay);
    int32_t t = grab();
    Task k = task_info(lay, t);
    uint32_t ct[16];
    if (k.valid) load_block(c.pay + 64u * (uint32_t)k.block, ct);
#pragma unroll 1
    while (t < total) {
        const int32_t tn = grab();
        const Task nxt = task_info(lay, tn);
        if (k.scale)
            scale_task(c, k, ct, nxt);
        else if (k.s.kind == kSecInt8)
            code_task<DT, kSecInt8>(c, k, ct, nxt);
        else if (k.s.kind == kSecInt4)
            code_task<DT, kSecInt4>(c, k, ct, nxt);
        else
            code_task<DT, kSecRaw>(c, k, ct, nxt);
        t = tn;
        k = nxt;
    }
}

// The verify wave's view of the payload: each section's code rows of the
// workgroup layout from the LDS ring, everything else from the blob.
struct VerifyFeed {
    int32_t si, phase, i, cidx, code_begin;
    uint32_t off;  // payload offset of the next chunk

    __device__ __forceinline__ void fetch(const IngressParams& p, const Layout& lay, bool has_lay,
                                          const uint8_t* pay, const uint32_t* lds, int lane, uint4 (&x)[4],
                                          int32_t& tag) {
        tag = 0;
        if (has_lay && si < lay.n_sec) {
            const SecRows s = sec_rows(lay, si, code_begin, 0);
            if (phase == 0) {
                const uint32_t* slot = lds + (cidx % kRing) * kRowWords;
                wait_ge<kDiagIngressWait>(&lds[kLdsFlags + kFlagRing + cidx % kRing], cidx + 1, p.state);
#pragma unroll
                for (int q = 0; q < 4; ++q) x[q] = lds_quad(slot, lane, q);
                tag = cidx + 1;
                ++cidx;
                off += 64u;
                if (++i == s.n_units * s.nblk) {
                    i = 0;
                    phase = s.kind != kSecRaw ? 1 : 2;
                }
            } else {
                const uint8_t* q = pay + off;
                x[0] = ldg16(q, 0); x[1] = ldg16(q, 1); x[2] = ldg16(q, 2); x[3] = ldg16(q, 3);
                off += 64u;
                if (++i == s.n_units) phase = 2;
            }
            if (phase == 2) {
                code_begin += s.n_units * s.nblk;
                ++si;
                phase = 0;
                i = 0;
            }
            return;
        }
        const uint8_t* q = pay + off;  // padding (or no usable layout in the workgroup)
        x[0] = ldg16(q, 0); x[1] = ldg16(q, 1); x[2] = ldg16(q, 2); x[3] = ldg16(q, 3);
        off += 64u;
    }
};

// Verdict of one page (cpp:2313-2355).
__device__ __forceinline__ int32_t verify_page(const IngressParams& p, int64_t page, const Layout& lay, bool has_lay,
                               const uint32_t* lds, uint32_t* used, int lane) {
    const uint8_t* blob = ingress_blob(p, page);
    const uint4 h0 = ldg16(blob, 0), h1 = ldg16(blob, 1);
    Sip s;
    s.init(p.mk0, p.mk1);
    const uint64_t hdr[4] = {lo64(h0), hi64(h0), lo64(h1), hi64(h1)};
    s.absorb_words<4>(hdr);
    const uint8_t* pay = blob + kHeader;
    const int32_t total = (int32_t)(p.payload / 64u);
    VerifyFeed feed{0, 0, 0, 0, 0, 0u};
    uint4 x0[4], x1[4], x2[4];
    int32_t t0 = 0, t1 = 0, t2 = 0;
    if (total > 0) feed.fetch(p, lay, has_lay, pay, lds, lane, x0, t0);
    if (total > 1) feed.fetch(p, lay, has_lay, pay, lds, lane, x1, t1);
#pragma unroll 1
    for (int32_t c = 0; c < total; c += 3) {
        if (c + 2 < total) feed.fetch(p, lay, has_lay, pay, lds, lane, x2, t2);
        s.absorb64(x0);
        if (t0) publish(used, (uint32_t)t0);
        if (c + 1 >= total) break;
        if (c + 3 < total) feed.fetch(p, lay, has_lay, pay, lds, lane, x0, t0);
        s.absorb64(x1);
        if (t1) publish(used, (uint32_t)t1);
        if (c + 2 >= total) break;
        if (c + 4 < total) feed.fetch(p, lay, has_lay, pay, lds, lane, x1, t1);
        s.absorb64(x2);
        if (t2) publish(used, (uint32_t)t2);
    }
#pragma unroll 1
    for (uint32_t o = (uint32_t)total * 64u; o < p.payload; o += 16u) s.absorb(ldg16(pay + o, 0));
    uint64_t lo, hi;
    s.finish((uint64_t)((kHeader + p.payload) & 0xFFu) << 56, lo, hi);
    const uint4 tag = ldg16(pay + p.payload, 0);
    const uint32_t diff = (tag.x ^ (uint32_t)lo) | (tag.y ^ (uint32_t)(lo >> 32)) |
                          (tag.z ^ (uint32_t)hi) | (tag.w ^ (uint32_t)(hi >> 32));
    const uint32_t magic = h0.x & 0xFFFFu, version = (h0.x >> 16) & 0xFFu;
    if (magic != kMagic || version != kVersion) return 1;
    const uint64_t tok = lo64(h1);
    if (h0.y != p.exp_tenant || h0.z != p.exp_model || (h0.w & 0xFFFFu) != ingress_layer(p, page) ||
        tok != ingress_token(p, page))
        return 2;
    if (diff != 0u) return 3;
    if (layout_index(p, h0.x) < 0) return 1;
    return 0;
}

template <int DT>
__global__ __launch_bounds__(kFusedThreads) void ingress_fused_kernel(IngressParams p) {
    extern __shared__ __align__(16) uint32_t lds[];
    const int64_t page0 = (int64_t)blockIdx.x * p.ppw;
    const int ppw = (int)min((int64_t)p.ppw, p.batch - page0);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const bool active = lane < ppw;
    const int64_t page = page0 + (active ? lane : 0);
    // every wave derives the workgroup layout from the 64 headers itself
    const uint8_t* blob = ingress_blob(p, page);
    const uint4 h0 = ldg16(blob, 0), h1 = ldg16(blob, 1);
    const int li = layout_index(p, h0.x);
    const uint64_t any_valid = __ballot(active && li >= 0);
    const int li_wg = any_valid ? __builtin_amdgcn_readlane(li, (int)__builtin_ctzll(any_valid)) : -1;
    const uint64_t rows_mask = __ballot(active && li >= 0 && li == li_wg);
    const bool has_lay = li_wg >= 0;
    // the nine layouts live in LDS: a table in registers or in the kernel
    // arguments would be copied to scratch memory once indexed by a variable
    Layout* layouts = reinterpret_cast<Layout*>(lds + kLdsLayouts);
    if (threadIdx.x < 9) layouts[threadIdx.x] = ingress_layout(p, (int)threadIdx.x);
    uint32_t* flags = lds + kLdsFlags;
    for (int i = threadIdx.x; i < kNumFlags; i += blockDim.x) flags[i] = 0u;
    if (threadIdx.x < 64) {
        uint64_t* ptrs = reinterpret_cast<uint64_t*>(lds + kLdsPtrs);
        const bool rows = (rows_mask >> threadIdx.x) & 1ull;
        ptrs[threadIdx.x] = rows ? reinterpret_cast<uint64_t>(ingress_k(p, page)) : 0ull;
        ptrs[64 + threadIdx.x] = rows ? reinterpret_cast<uint64_t>(ingress_v(p, page)) : 0ull;
    }
    __syncthreads();
    const Layout& lay = layouts[has_lay ? li_wg : 0];
    if (wave == 0) {
        __builtin_amdgcn_s_setprio(3);
        flags[kFlagStatus + lane] = (uint32_t)verify_page(p, page, lay, has_lay, lds, &flags[kFlagMacUsed], lane);
    } else if ((wave & 3) != 0) {  // waves 4 and 8 share the verify wave's SIMD: they idle
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
        if (has_lay) decode_rows<DT>(c, lay);
        // pages with another valid layout: unit by unit, one page per wave
        const uint64_t other = __ballot(active && li >= 0 && li != li_wg);
        if (other) {
            const int dw = wave - 1 - (wave >> 2);
            int n = 0;
#pragma unroll 1
            for (uint64_t m = other; m; m &= m - 1, ++n) {
                if (n % kProducerWaves != dw) continue;
                const int pl = (int)__builtin_ctzll(m);
                const int lp = __builtin_amdgcn_readlane(li, pl);
                const Layout& L2 = layouts[lp];
                const uint32_t a0 = __builtin_amdgcn_readlane(h1.z, pl), a1 = __builtin_amdgcn_readlane(h1.w, pl);
                const uint32_t a2 = __builtin_amdgcn_readlane(h0.w, pl);
                const uint32_t m2 = ((a2 & 0xFFFFu) << 16) | (a2 >> 16);
#pragma unroll 1
                for (int u = lane; u < L2.n_units; u += 64) decode_unit<DT>(p, L2, page0 + pl, u, a0, a1, m2);
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // every decode store has completed before the verdicts
    __syncthreads();
    if ((int)threadIdx.x < ppw) {
        const int32_t st = (int32_t)flags[kFlagStatus + threadIdx.x];
        const int64_t pg = page0 + threadIdx.x;
        if (p.page_status) p.page_status[pg] = st;
        if (st != 0) atomicMin(&p.state->fail, ((unsigned long long)pg << 8) | (unsigned long long)st);
    }
    if (p.per_page) {  // extension: zero only the failing pages
        const int64_t n16 = p.page_bytes / 16;
#pragma unroll 1
        for (int pl = 0; pl < ppw; ++pl) {
            if (flags[kFlagStatus + pl] == 0u) continue;
            uint8_t* k = ingress_k(p, page0 + pl);
            for (int64_t i = threadIdx.x; i < n16; i += blockDim.x) stg16(k, i, make_uint4(0, 0, 0, 0));
            uint8_t* v = ingress_v(p, page0 + pl);
            if (v)
                for (int64_t i = threadIdx.x; i < n16; i += blockDim.x) stg16(v, i, make_uint4(0, 0, 0, 0));
        }
    }
}

}  // namespace

// All-or-nothing epilogue (cpp:2481-2486): if any page failed, zero both
// outputs entirely.  Every block reads the failure word once.
__global__ void ingress_finalize_kernel(IngressParams p) {
    if (p.state->fail == ~0ull) return;
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

__global__ void reset_fail_kernel(DeviceState* st) { st->fail = ~0ull; }

hipError_t launch_ingress_fused(const IngressParams& p, int dtype, hipStream_t s) {
    const int64_t grid = (p.batch + p.ppw - 1) / p.ppw;
    const size_t lds = (size_t)kLdsWords * sizeof(uint32_t);  // above 64 KiB: gfx950 has 160 KiB per CU
    if (dtype == kHotBf16)
        hipLaunchKernelGGL(ingress_fused_kernel<kHotBf16>, dim3((uint32_t)grid), dim3(kFusedThreads), lds, s, p);
    else
        hipLaunchKernelGGL(ingress_fused_kernel<kHotFp16>, dim3((uint32_t)grid), dim3(kFusedThreads), lds, s, p);
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

hipError_t launch_reset_fail(DeviceState* st, hipStream_t s) {
    hipLaunchKernelGGL(reset_fail_kernel, dim3(1), dim3(1), 0, s, st);
    return hipGetLastError();
}

}  // namespace ztcp
