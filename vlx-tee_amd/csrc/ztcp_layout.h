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

// Returns false for preset / rope_mode outside 1..3 / 0..2 (cpp:1447-1449).
ZTCP_HD inline bool build_layout(int64_t preset, int64_t rope_mode, int64_t vecs,
                                 int64_t head_dim, int64_t rope_dim, bool has_v, Layout& L) {
    if (preset < 1 || preset > 3 || rope_mode < 0 || rope_mode > 2) return false;
    int32_t kinds[3], srcs[3], cols[3], widths[3];
    int n = 0;
    if (rope_mode == 2 && rope_dim > 0) {
        kinds[n] = kSecRaw; srcs[n] = 0; cols[n] = 0; widths[n] = (int32_t)rope_dim; ++n;
    } else if (rope_mode == 1 && rope_dim > 0) {
        kinds[n] = kSecInt8; srcs[n] = 0; cols[n] = 0; widths[n] = (int32_t)rope_dim; ++n;
    }
    const int64_t kq = rope_mode == 0 ? head_dim : head_dim - rope_dim;
    const int64_t kc = rope_mode == 0 ? 0 : rope_dim;
    if (kq > 0) {
        kinds[n] = preset == 1 ? kSecInt4 : kSecInt8; srcs[n] = 0;
        cols[n] = (int32_t)kc; widths[n] = (int32_t)kq; ++n;
    }
    if (has_v) {
        kinds[n] = (preset == 1 || preset == 2) ? kSecInt4 : kSecInt8; srcs[n] = 1;
        cols[n] = 0; widths[n] = (int32_t)head_dim; ++n;
    }
    uint32_t off = 0;
    int32_t units = 0;
    bool aligned = true;
    for (int i = 0; i < 3; ++i) {
        Section& s = L.sec[i];
        if (i >= n) {
            s = Section{kSecInt8, 0, 0, 0, 0, units, 0, off, off, 0};
            continue;
        }
        s.kind = kinds[i];
        s.src = srcs[i];
        s.col = cols[i];
        s.gpv = widths[i] / 16;
        s.n_groups = (int32_t)(vecs * s.gpv);
        s.unit_begin = units;
        s.n_units = (s.n_groups + 31) / 32;
        s.q_off = off;
        const uint32_t code = (uint32_t)s.n_groups * (uint32_t)code_bytes_per_group(s.kind);
        const uint32_t scales = s.kind == kSecRaw ? 0u : 2u * (uint32_t)s.n_groups;
        s.s_off = off + code;
        s.bytes = code + scales;
        off += s.bytes;
        units += s.n_units;
        if (s.n_groups % 32 != 0) aligned = false;
    }
    L.n_sec = n;
    L.n_units = units;
    L.required = off;
    L.aligned = aligned ? 1 : 0;
    return true;
}

}  // namespace ztcp
