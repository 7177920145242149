// ztcp_params.h -- kernel argument blocks and launch helpers shared by the
// egress, ingress and generic translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ztcp.h"
#include "ztcp_device.h"
#include "ztcp_layout.h"

namespace ztcp {

// Diagnostic bits (or-ed by kernels).
constexpr uint32_t kDiagEgressWait = 1u;   // a bounded wait of the fused egress kernel expired
constexpr uint32_t kDiagIngressWait = 2u;  // a bounded wait of the fused ingress kernel expired

// Bounded waits give up after this many s_sleep(1) polls (about 30 ms).
constexpr uint32_t kSpinLimit = 1u << 20;

// Per-device library state (allocated once per device by the host side):
// sticky diagnostic bits, read and cleared by ztcp_device_diag.
struct DeviceState {
    uint32_t diag;
    uint32_t pad[3];
};

// Per-call ingress state: every ingress call owns one for its duration, so
// concurrent calls on one device (other streams, other threads) never see
// each other's verdicts.  Reset by the call's first kernel.
struct CallState {
    unsigned long long fail;   // (page_index << 8) | status of the lowest failing page; ~0 = none
    uint32_t diag;             // kDiag* bits of waits that expired during this call
    uint32_t pad;
};

// What a bounded wait reports to when it expires.  Ingress or-s its kDiag*
// bit into the call's diag word (reset by the call's first kernel); egress
// raises it to the call's tag instead (atomic max of a per-device call
// counter, never below 16), so the host learns of an expiry in this call
// without a reset kernel: the word equals the tag only if this call wrote it.
struct WaitSink {
    uint32_t* dev_diag;        // DeviceState::diag (sticky, per device)
    uint32_t* call_diag;       // CallState::diag, or nullptr
    uint32_t spin_limit;       // polls before giving up
    uint32_t call_tag;         // 0: or the kDiag* bit into call_diag; else max it with this tag
};

struct EgressParams {
    const uint8_t* k;              // contiguous K pages (hot elements, 2 bytes each)
    const uint8_t* v;              // contiguous V pages or nullptr
    const int64_t* token_hashes;   // [batch]
    uint8_t* blobs;                // [batch, blob_bytes]
    const ztcp_page_desc* descs;   // descriptor mode when non-null
    int64_t batch;
    int64_t page_bytes;            // T*H*D*2
    int32_t vecs, head_dim;
    uint32_t payload;              // expected_payload_bytes
    uint32_t blob_bytes;
    Layout lay;
    ChaKey key;
    uint64_t mk0, mk1;
    uint64_t hdr0;                 // header bytes 0..7 (magic, version, flags, tenant)
    uint64_t hdr1;                 // header bytes 8..15 (model, layer, head group);
                                   // descriptor mode: only the model hash is used
    uint32_t nonce2;               // (layer_id << 16) | head_group_id
    uint64_t base_seq;
    int32_t ppw;                   // pages per workgroup
    WaitSink sink;
    unsigned long long* timers;    // phase-timer records, one per workgroup (timer builds; else nullptr)
};

struct IngressParams {
    const uint8_t* blobs;          // [batch, blob_bytes]
    const int64_t* token_hashes;   // expected token hashes [batch]
    uint8_t* out_k;
    uint8_t* out_v;                // nullptr for MLA single buffer
    const ztcp_page_desc* descs;
    int32_t* page_status;          // may be null
    int64_t batch;
    int64_t page_bytes;
    int32_t vecs, head_dim;
    uint32_t blob_bytes;
    uint32_t payload;              // blob_bytes - 48
    int32_t rope_dim, has_v;       // geometry of the page layouts (ingress_layout)
    uint32_t lay_ok;               // bit (preset - 1) * 4 + rope_mode: valid layout, payload >= required
    int32_t n_units;               // generic path: 16-element groups per page
    ChaKey key;
    uint64_t mk0, mk1;
    uint32_t exp_tenant, exp_model;
    uint32_t exp_layer;
    int32_t per_page;              // zero failing pages in-kernel
    int32_t ppw;
    CallState* call;               // this call's failure word and diagnostics
    WaitSink sink;
    unsigned long long* timers;    // phase-timer records, one per workgroup (timer builds; else nullptr)
};

// Page addressing (contiguous batch or descriptor array).
struct EgressPage {
    const uint8_t* k;
    const uint8_t* v;
    uint8_t* blob;
    uint64_t token;
    uint64_t seq;
    uint64_t hdr1;    // header bytes 8..15: model, layer, head group
    uint32_t nonce2;  // (layer_id << 16) | head_group_id
};

__device__ __forceinline__ EgressPage egress_page(const EgressParams& p, int64_t page) {
    EgressPage e;
    if (p.descs) {
        const ztcp_page_desc& d = p.descs[page];
        e.k = (const uint8_t*)d.k;
        e.v = (const uint8_t*)d.v;
        e.blob = d.blob;
        e.token = (uint64_t)d.token_hash;
        e.seq = d.sequence_nonce;
        e.hdr1 = (p.hdr1 & 0xFFFFFFFFull) | ((uint64_t)d.layer_id << 32) | ((uint64_t)d.head_group_id << 48);
        e.nonce2 = ((uint32_t)d.layer_id << 16) | (uint32_t)d.head_group_id;
    } else {
        e.k = p.k + page * p.page_bytes;
        e.v = p.v ? p.v + page * p.page_bytes : nullptr;
        e.blob = p.blobs + page * (int64_t)p.blob_bytes;
        e.token = (uint64_t)p.token_hashes[page];
        e.seq = p.base_seq + (uint64_t)page;  // cpp:1979
        e.hdr1 = p.hdr1;
        e.nonce2 = p.nonce2;
    }
    return e;
}

// Layout of header flags index li = (preset - 1) * 4 + rope_mode, computed
// in registers (no table in the kernel arguments).
__device__ __forceinline__ Layout ingress_layout(const IngressParams& p, int li) {
    Layout L;
    build_layout(li / 4 + 1, li % 4, p.vecs, p.head_dim, p.rope_dim, p.has_v != 0, L);
    return L;
}

__device__ __forceinline__ const uint8_t* ingress_blob(const IngressParams& p, int64_t page) {
    return p.descs ? (const uint8_t*)p.descs[page].blob : p.blobs + page * (int64_t)p.blob_bytes;
}
__device__ __forceinline__ uint8_t* ingress_k(const IngressParams& p, int64_t page) {
    return p.descs ? (uint8_t*)p.descs[page].k : p.out_k + page * p.page_bytes;
}
// nullptr when the page has no V buffer (MLA single buffer).
__device__ __forceinline__ uint8_t* ingress_v(const IngressParams& p, int64_t page) {
    if (p.descs) return (uint8_t*)p.descs[page].v;
    return p.out_v ? p.out_v + page * p.page_bytes : nullptr;
}
__device__ __forceinline__ uint64_t ingress_token(const IngressParams& p, int64_t page) {
    return (uint64_t)(p.descs ? p.descs[page].token_hash : p.token_hashes[page]);
}
__device__ __forceinline__ uint32_t ingress_layer(const IngressParams& p, int64_t page) {
    return p.descs ? (uint32_t)p.descs[page].layer_id : p.exp_layer;
}

// Field of section `si` (0..2) selected without dynamic indexing.
#define ZTCP_SEC_FIELD(lay, si, f) \
    ((si) == 0 ? (lay).sec[0].f : ((si) == 1 ? (lay).sec[1].f : (lay).sec[2].f))

__device__ __forceinline__ int section_of_unit(const Layout& lay, int u) {
    return (lay.n_sec > 1 && u >= lay.sec[1].unit_begin)
               ? ((lay.n_sec > 2 && u >= lay.sec[2].unit_begin) ? 2 : 1)
               : 0;
}

// Byte offset of a section's groups inside a page buffer, walked in (vec,
// group) row-major order: 32 bytes per group, `skip` extra bytes at the end of
// each vector (the columns outside the section).
struct GroupCursor {
    uint32_t off;
    int32_t g;
    __device__ __forceinline__ void step(int32_t gpv, uint32_t skip) {
        off += 32u;
        if (++g == gpv) { g = 0; off += skip; }
    }
};

__device__ __forceinline__ GroupCursor group_cursor(int32_t G0, int32_t gpv, int32_t col, int32_t head_dim) {
    const int32_t vec = G0 / gpv, g = G0 - vec * gpv;
    return GroupCursor{(uint32_t)vec * (uint32_t)head_dim * 2u + (uint32_t)(col + g * 16) * 2u, g};
}

// Host-side launchers (defined in the .hip translation units).
hipError_t launch_egress_fused(const EgressParams& p, int dtype, hipStream_t s);
hipError_t launch_ingress_fused(const IngressParams& p, int dtype, hipStream_t s);
hipError_t launch_egress_generic(const EgressParams& p, int dtype, hipStream_t s);
hipError_t launch_egress_zero_blobs(const EgressParams& p, hipStream_t s);
hipError_t launch_ingress_generic_impl(const IngressParams& p, int dtype, int32_t* status,
                                       hipStream_t s);
hipError_t launch_ingress_finalize(const IngressParams& p, hipStream_t s);
hipError_t launch_reset_call(CallState* call, hipStream_t s);
hipError_t launch_chacha_xor(const uint8_t* src, uint8_t* dst, size_t len, ChaKey key,
                             uint32_t ctr, uint32_t n0, uint32_t n1, uint32_t n2, hipStream_t s);
hipError_t launch_selftest(unsigned int* bad, hipStream_t s);
hipError_t launch_siphash(const uint8_t* data, size_t len, uint64_t mk0, uint64_t mk1,
                          uint8_t* tag, hipStream_t s);

}  // namespace ztcp
