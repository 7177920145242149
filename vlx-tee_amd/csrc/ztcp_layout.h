// ztcp_layout.h -- payload layout of one cold page, shared by host and device.
//
// A payload is up to three sections followed by zero padding (encode order
// cpp:1376-1422, decode order cpp:2418-2461):
//   1. K RoPE columns [0, rope_dim): int8 (PRESERVE_FP8), raw hot bytes
//      (PRESERVE_RAW) or e4m3 (PRESERVE_E4M3, extension); absent for
//      QUANTIZE_ALL or rope_dim == 0.
//   2. K remaining columns (all columns for QUANTIZE_ALL).
//   3. V, all columns (absent for MLA single-buffer pages).
// Section kinds per preset (K remaining columns / V):
//   1 INT4_SYM  int4 / int4        2 K8V4       int8 / int4
//   3 FP8_ONLY  int8 / int8        (the reference's presets, 16-element groups)
//   4 K8V4_ASYM asym8 per 64 / int4 per 32        (extensions, no counterpart
//   5 FP8_E4M3  e4m3 / e4m3                        in the reference)
//   6 INT4_SYM_G32 int4 per 32 / int4 per 32
// A quantized section is [codes of every (vec, group) in row-major order]
// [parameters of every (vec, group) in the same order] (cpp:1146-1374): an
// fp16 scale per group, and for asym8 the scale then the zero point as a
// little-endian u16.  A raw section is the hot bytes of each vec's columns in
// vec order (cpp:1379-1386).
//
// The GPU kernels cut every section into units whose parameters fill exactly
// one 64-byte ChaCha20 block: 32 groups (16 for asym8, whose groups carry
// 4 parameter bytes).  A unit's codes are a whole number of 64-byte blocks
// ("code rows"): 8 (int8, e4m3, int4 per 32), 4 (int4) or 16 (asym8, raw).
// When every section holds a whole number of units, all unit boundaries fall
// on 64-byte keystream blocks.  Within a page buffer, a section is walked in
// 16-element chunks (32 hot bytes): every group is 1, 2 or 4 chunks.
#pragma once

#include <stdint.h>

#ifdef __HIPCC__
#define ZTCP_HD __host__ __device__
#else
#define ZTCP_HD
#endif

namespace ztcp {

enum SectionKind : int32_t {
    kSecInt8 = 0,     // int8 symmetric, 16-element groups (reference)
    kSecInt4 = 1,     // int4 symmetric, 16-element groups (reference)
    kSecRaw = 2,      // hot bytes (reference)
    kSecE4m3 = 3,     // FP8 e4m3, 16-element groups (extension)
    kSecInt4G32 = 4,  // int4 symmetric, 32-element groups (extension)
    kSecAsym8 = 5,    // int8 asymmetric (scale, zero point), 64-element groups (extension)
};

struct Section {
    int32_t kind;        // SectionKind
    int32_t src;         // 0 = K buffer, 1 = V buffer
    int32_t col;         // first column inside the head vector
    int32_t gpv;         // 16-element chunks per vector in this section
    int32_t n_groups;    // groups: vecs * width / group elements
    int32_t unit_begin;  // index of the section's first unit in the page
    int32_t n_units;     // ceil(n_groups / groups per unit)
    uint32_t q_off;      // payload offset of the codes (or raw bytes)
    uint32_t s_off;      // payload offset of the parameters (quantized sections)
    uint32_t bytes;      // section bytes (codes + parameters)
};

struct Layout {
    Section sec[3];
    int32_t n_sec;
    int32_t n_units;     // units in the page
    uint32_t required;   // unpadded payload bytes (cpp:1439-1474)
    int32_t aligned;     // every section holds a whole number of units
};

// Per-kind geometry (selects only: the kind is a runtime, wave-uniform value).
ZTCP_HD inline int32_t group_elems(int32_t kind) {  // elements per group
    return kind == kSecInt4G32 ? 32 : (kind == kSecAsym8 ? 64 : 16);
}
ZTCP_HD inline int32_t code_bytes_per_group(int32_t kind) {
    return kind == kSecInt4 ? 8 : (kind == kSecRaw ? 32 : (kind == kSecAsym8 ? 64 : 16));
}
ZTCP_HD inline int32_t param_bytes_per_group(int32_t kind) {
    return kind == kSecRaw ? 0 : (kind == kSecAsym8 ? 4 : 2);
}
ZTCP_HD inline int32_t groups_per_unit(int32_t kind) { return kind == kSecAsym8 ? 16 : 32; }
// 64-byte code rows per unit: 8, 4 (int4), 16 (raw, asym8)
ZTCP_HD inline int32_t code_rows_per_unit(int32_t kind) {
    return kind == kSecInt4 ? 4 : ((kind == kSecRaw || kind == kSecAsym8) ? 16 : 8);
}
// groups in one code row: 4, 8 (int4), 2 (raw), 1 (asym8)
ZTCP_HD inline int32_t groups_per_row(int32_t kind) {
    return kind == kSecInt4 ? 8 : (kind == kSecRaw ? 2 : (kind == kSecAsym8 ? 1 : 4));
}
// 16-element chunks of hot data in one code row: 4, 8 (int4, int4 per 32), 2 (raw)
ZTCP_HD inline int32_t chunks_per_row(int32_t kind) {
    return (kind == kSecInt4 || kind == kSecInt4G32) ? 8 : (kind == kSecRaw ? 2 : 4);
}
// parameter words (4 bytes) one code row contributes to its unit's parameter row
ZTCP_HD inline int32_t param_words_per_row(int32_t kind) {
    return kind == kSecInt4 ? 4 : (kind == kSecAsym8 ? 1 : 2);
}

ZTCP_HD inline Section make_section(int32_t kind, int32_t src, int32_t col, int32_t width, int64_t vecs,
                                   uint32_t off, int32_t units) {
    Section s;
    s.kind = kind;
    s.src = src;
    s.col = col;
    s.gpv = width / 16;
    s.n_groups = (int32_t)(vecs * (width / group_elems(kind)));
    s.unit_begin = units;
    s.n_units = (s.n_groups + groups_per_unit(kind) - 1) / groups_per_unit(kind);
    s.q_off = off;
    const uint32_t code = (uint32_t)s.n_groups * (uint32_t)code_bytes_per_group(kind);
    s.s_off = off + code;
    s.bytes = code + (uint32_t)param_bytes_per_group(kind) * (uint32_t)s.n_groups;
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

// Number of header-flag layouts: presets 1..6 x RoPE modes 0..3, index
// (preset - 1) * 4 + rope_mode.
constexpr int kNumLayouts = 24;

ZTCP_HD inline bool flags_valid(int64_t preset, int64_t rope_mode) {
    return preset >= 1 && preset <= 6 && rope_mode >= 0 && rope_mode <= 3;
}
ZTCP_HD inline int32_t rope_section_kind(int64_t rope_mode) {
    return rope_mode == 2 ? kSecRaw : (rope_mode == 3 ? kSecE4m3 : kSecInt8);
}
ZTCP_HD inline int32_t kmain_section_kind(int64_t preset) {
    return preset == 1 ? kSecInt4
                       : (preset == 4 ? kSecAsym8
                                      : (preset == 5 ? kSecE4m3 : (preset == 6 ? kSecInt4G32 : kSecInt8)));
}
ZTCP_HD inline int32_t v_section_kind(int64_t preset) {
    return (preset == 1 || preset == 2) ? kSecInt4
                                        : (preset == 3 ? kSecInt8 : (preset == 5 ? kSecE4m3 : kSecInt4G32));
}
ZTCP_HD inline bool is_extension_kind(int32_t kind) { return kind >= kSecE4m3; }

// Returns false for preset / rope_mode outside 1..6 / 0..3 (the reference
// accepts 1..3 / 0..2, cpp:1447-1449) and for an extension kind whose group
// does not divide its section's width.  Written with selects only (no indexed
// stores), so that a Layout built on the device from wave-uniform flags stays
// in scalar registers.
ZTCP_HD inline bool build_layout(int64_t preset, int64_t rope_mode, int64_t vecs, int64_t head_dim,
                                 int64_t rope_dim, bool has_v, Layout& L) {
    if (!flags_valid(preset, rope_mode)) return false;
    // candidate sections in payload order: K RoPE columns, the other K columns, V
    const bool pa = rope_mode != 0 && rope_dim > 0;
    const int64_t kq = rope_mode == 0 ? head_dim : head_dim - rope_dim;
    const bool pb = kq > 0, pc = has_v;
    const int32_t ka = rope_section_kind(rope_mode), kb = kmain_section_kind(preset), kc = v_section_kind(preset);
    if ((pa && rope_dim % group_elems(ka)) || (pb && kq % group_elems(kb)) || (pc && head_dim % group_elems(kc)))
        return false;
    const Section a = make_section(ka, 0, 0, pa ? (int32_t)rope_dim : 0, vecs, 0u, 0);
    const uint32_t off_b = pa ? a.bytes : 0u;
    const int32_t units_b = pa ? a.n_units : 0;
    const Section b = make_section(kb, 0, rope_mode == 0 ? 0 : (int32_t)rope_dim, pb ? (int32_t)kq : 0, vecs,
                                   off_b, units_b);
    const uint32_t off_c = off_b + (pb ? b.bytes : 0u);
    const int32_t units_c = units_b + (pb ? b.n_units : 0);
    const Section c = make_section(kc, 1, 0, pc ? (int32_t)head_dim : 0, vecs, off_c, units_c);
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
    L.aligned = (!pa || a.n_groups % groups_per_unit(ka) == 0) && (!pb || b.n_groups % groups_per_unit(kb) == 0) &&
                (!pc || c.n_groups % groups_per_unit(kc) == 0);
    return true;
}

}  // namespace ztcp
