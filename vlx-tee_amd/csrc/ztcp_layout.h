// ztcp_layout.h -- payload layout of one cold page, shared by host and device.
//
// A payload is up to three sections followed by zero padding (encode order
// cpp:1376-1422, decode order cpp:2418-2461):
//   1. K RoPE columns [0, rope_dim): int8 (PRESERVE_FP8) or raw hot bytes
//      (PRESERVE_RAW); absent for QUANTIZE_ALL or rope_dim == 0.
//   2. K remaining columns (all columns for QUANTIZE_ALL): int4 for INT4_SYM,
//      int8 otherwise.
//   3. V, all columns (absent for MLA single-buffer pages): int4 for INT4_SYM
//      and K8V4_ASYM, int8 for FP8_ONLY.
// A quantized section is [codes of every (vec, group) in row-major order]
// [fp16 scale of every (vec, group) in the same order] (cpp:1146-1374); a raw
// section is the hot bytes of each vec's columns in vec order (cpp:1379-1386).
//
// The GPU kernels cut every section into units of 32 consecutive groups: a
// unit's codes occupy 512 (int8) / 256 (int4) / 1024 (raw) payload bytes and
// its scales exactly one 64-byte ChaCha20 block.  When every section holds a
// multiple of 32 groups, all unit boundaries fall on 64-byte keystream blocks.
#pragma once

#include <stdint.h>

#ifdef __HIPCC__
#define ZTCP_HD __host__ __device__
#else
#define ZTCP_HD
#endif

namespace ztcp {

enum SectionKind : int32_t { kSecInt8 = 0, kSecInt4 = 1, kSecRaw = 2 };

struct Section {
    int32_t kind;        // SectionKind
    int32_t src;         // 0 = K buffer, 1 = V buffer
    int32_t col;         // first column inside the head vector
    int32_t gpv;         // 16-element groups per vector in this section
    int32_t n_groups;    // vecs * gpv
    int32_t unit_begin;  // index of the section's first unit in the page
    int32_t n_units;     // ceil(n_groups / 32)
    uint32_t q_off;      // payload offset of the codes (or raw bytes)
    uint32_t s_off;      // payload offset of the scales (quantized sections)
    uint32_t bytes;      // section bytes (codes + scales)
};

struct Layout {
    Section sec[3];
    int32_t n_sec;
    int32_t n_units;     // units in the page
    uint32_t required;   // unpadded payload bytes (cpp:1439-1474)
    int32_t aligned;     // every section holds a multiple of 32 groups
};

ZTCP_HD inline int32_t code_bytes_per_group(int32_t kind) {
    return kind == kSecInt8 ? 16 : (kind == kSecInt4 ? 8 : 32);
}

ZTCP_HD inline Section make_section(int32_t kind, int32_t src, int32_t col, int32_t width, int64_t vecs,
                                   uint32_t off, int32_t units) {
    Section s;
    s.kind = kind;
    s.src = src;
    s.col = col;
    s.gpv = width / 16;
    s.n_groups = (int32_t)(vecs * s.gpv);
    s.unit_begin = units;
    s.n_units = (s.n_groups + 31) / 32;
    s.q_off = off;
    const uint32_t code = (uint32_t)s.n_groups * (uint32_t)code_bytes_per_group(kind);
    s.s_off = off + code;
    s.bytes = code + (kind == kSecRaw ? 0u : 2u * (uint32_t)s.n_groups);
    return s;
}

// c ? x : y field by field (a select of whole structs would go through memory
// on the device).
ZTCP_HD inline Section pick(bool c, const Section& x, const Section& y) {
    return Section{c ? x.kind : y.kind,         c ? x.src : y.src,         c ? x.col : y.col,
                   c ? x.gpv : y.gpv,           c ? x.n_groups : y.n_groups,
                   c ? x.unit_begin : y.unit_begin, c ? x.n_units : y.n_units,
                   c ? x.q_off : y.q_off,       c ? x.s_off : y.s_off,     c ? x.bytes : y.bytes};
}

// Returns false for preset / rope_mode outside 1..3 / 0..2 (cpp:1447-1449).
// Written with selects only (no indexed stores), so that a Layout built on the
// device from wave-uniform flags stays in scalar registers.
ZTCP_HD inline bool build_layout(int64_t preset, int64_t rope_mode, int64_t vecs, int64_t head_dim,
                                 int64_t rope_dim, bool has_v, Layout& L) {
    if (preset < 1 || preset > 3 || rope_mode < 0 || rope_mode > 2) return false;
    // candidate sections in payload order: K RoPE columns, the other K columns, V
    const bool pa = rope_mode != 0 && rope_dim > 0;
    const int64_t kq = rope_mode == 0 ? head_dim : head_dim - rope_dim;
    const bool pb = kq > 0, pc = has_v;
    const Section a = make_section(rope_mode == 2 ? kSecRaw : kSecInt8, 0, 0, pa ? (int32_t)rope_dim : 0, vecs, 0u, 0);
    const uint32_t off_b = pa ? a.bytes : 0u;
    const int32_t units_b = pa ? a.n_units : 0;
    const Section b = make_section(preset == 1 ? kSecInt4 : kSecInt8, 0, rope_mode == 0 ? 0 : (int32_t)rope_dim,
                                   pb ? (int32_t)kq : 0, vecs, off_b, units_b);
    const uint32_t off_c = off_b + (pb ? b.bytes : 0u);
    const int32_t units_c = units_b + (pb ? b.n_units : 0);
    const Section c = make_section((preset == 1 || preset == 2) ? kSecInt4 : kSecInt8, 1, 0,
                                   pc ? (int32_t)head_dim : 0, vecs, off_c, units_c);
    const uint32_t end = off_c + (pc ? c.bytes : 0u);
    const int32_t units = units_c + (pc ? c.n_units : 0);
    const Section e{kSecInt8, 0, 0, 0, 0, units, 0, end, end, 0};  // unused slot
    const Section c_or_e = pick(pc, c, e);
    const Section b_or_c = pick(pb, b, c_or_e);
    L.sec[0] = pick(pa, a, b_or_c);
    L.sec[1] = pick(pa, b_or_c, pick(pb && pc, c, e));
    L.sec[2] = pick(pa && pb && pc, c, e);
    L.n_sec = (pa ? 1 : 0) + (pb ? 1 : 0) + (pc ? 1 : 0);
    L.n_units = units;
    L.required = end;
    L.aligned = (!pa || a.n_groups % 32 == 0) && (!pb || b.n_groups % 32 == 0) && (!pc || c.n_groups % 32 == 0);
    return true;
}

}  // namespace ztcp
