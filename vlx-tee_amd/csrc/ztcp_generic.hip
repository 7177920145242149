// ztcp_generic.hip -- layout-agnostic egress / ingress kernels and the
// known-answer hooks.
//
// The fused kernels need every section cut into whole 64-byte keystream
// blocks.  Geometries where that does not hold (T*H not a multiple of 32 for
// some section, payload padding beyond the required size, blob sizes that
// are not multiples of 16, unaligned descriptors) are handled here with the
// same device arithmetic (ztcp_device.h), decomposed differently:
//   egress:  one thread per (page, 64-byte payload block) builds that block's
//            plaintext from the groups that overlap it, XORs the keystream
//            and stores bytes; then one thread per page writes the header
//            and runs SipHash over header || ciphertext.
//   ingress: one thread per page verifies; one thread per (page, group)
//            decrypts the group's code and scale bytes and dequantizes; then
//            failing pages are zeroed (per page, or all-or-nothing).
// Byte-granular loads and stores keep every access in bounds for any
// alignment.  This path is correct for every geometry the reference accepts;
// the fused kernels are the fast path.
#include "ztcp_params.h"

namespace ztcp {

// Bytes [off, off + len) of the keystream of a payload (counter 1 at offset 0).
__device__ void keystream_bytes(const ChaKey& key, uint32_t n0, uint32_t n1, uint32_t n2,
                                uint32_t off, uint32_t len, uint8_t* out) {
    uint32_t blk = 0xFFFFFFFFu;
    uint32_t ks[16];
    for (uint32_t i = 0; i < len; ++i) {
        const uint32_t b = (off + i) / 64u;
        if (b != blk) {
            chacha_block(key, 1u + b, n0, n1, n2, ks);
            blk = b;
        }
        const uint32_t r = (off + i) % 64u;
        out[i] = (uint8_t)(ks[r / 4] >> (8 * (r % 4)));
    }
}

__device__ __forceinline__ void load_group_u16(const uint8_t* p, uint32_t w[8]) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
    for (int i = 0; i < 8; ++i) w[i] = (uint32_t)h[2 * i] | ((uint32_t)h[2 * i + 1] << 16);
}

// 16-element chunk g of a section whose vectors hold gpv chunks.
__device__ __forceinline__ const uint8_t* group_ptr(const uint8_t* base, int64_t head_dim,
                                                    int32_t gpv, int32_t col, int64_t g) {
    const int64_t vec = g / gpv, gg = g % gpv;
    return base + (vec * head_dim + col + gg * 16) * 2;
}

// One group of any quantized kind: code bytes (up to 64) and the parameter
// word (fp16 scale, and for asym8 the zero point in bits 16..31).  grp points
// at the group's first element; its 16, 32 or 64 elements are contiguous.
template <int DT>
__device__ void quant_any(const uint8_t* grp, int32_t kind, uint8_t codes[64], uint32_t& prm) {
    uint32_t w[4][8];
    const int nch = group_elems(kind) / 16;
    for (int c = 0; c < 4; ++c) {
        if (c < nch) load_group_u16(grp + 32 * c, w[c]);
        else for (int i = 0; i < 8; ++i) w[c][i] = 0u;
    }
    uint32_t q[16];
    for (int i = 0; i < 16; ++i) q[i] = 0u;
    if (kind == kSecInt8) prm = quant_group_int8<DT>(w[0], q);
    else if (kind == kSecInt4) prm = quant_group_int4<DT>(w[0], q);
    else if (kind == kSecE4m3) prm = quant_group_e4m3<DT>(w[0], q);
    else if (kind == kSecInt4G32) prm = quant_group32_int4<DT>(w[0], w[1], q);
    else prm = quant_group64_asym8<DT>(w, q);
    for (int i = 0; i < 64; ++i) codes[i] = (uint8_t)(q[i / 4] >> (8 * (i % 4)));
}

template <int DT>
__global__ void egress_generic_blocks_kernel(EgressParams p, int64_t nblk) {
    const int64_t total = p.batch * nblk;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t page = t / nblk;
        const uint32_t lo = (uint32_t)(t - page * nblk) * 64u;
        const uint32_t hi = min(lo + 64u, p.payload);
        uint8_t pt[64];
        for (int i = 0; i < 64; ++i) pt[i] = 0;
        for (int si = 0; si < 3; ++si) {
            if (si >= p.lay.n_sec) break;
            const Section S = p.lay.sec[si];
            const EgressPage pg = egress_page(p, page);
            const uint8_t* src = S.src ? pg.v : pg.k;
            if (S.kind == kSecRaw) {
                const uint32_t a = max(lo, S.q_off), b = min(hi, S.q_off + S.bytes);
                for (uint32_t x = a; x < b; ++x) {
                    const uint32_t r = x - S.q_off;
                    pt[x - lo] = group_ptr(src, p.head_dim, S.gpv, S.col, r / 32u)[r % 32u];
                }
                continue;
            }
            const uint32_t bpg = (uint32_t)code_bytes_per_group(S.kind);
            const uint32_t ppg = (uint32_t)param_bytes_per_group(S.kind);
            const int64_t cpg = group_elems(S.kind) / 16;  // 16-element chunks per group
            const uint32_t code_end = S.s_off;
            const uint32_t sc_end = S.q_off + S.bytes;
            // code bytes overlapping [lo, hi)
            uint32_t a = max(lo, S.q_off), b = min(hi, code_end);
            if (a < b) {
                for (uint32_t g = (a - S.q_off) / bpg; g <= (b - 1 - S.q_off) / bpg; ++g) {
                    uint8_t codes[64];
                    uint32_t prm;
                    quant_any<DT>(group_ptr(src, p.head_dim, S.gpv, S.col, g * cpg), S.kind, codes, prm);
                    for (uint32_t i = 0; i < bpg; ++i) {
                        const uint32_t x = S.q_off + g * bpg + i;
                        if (x >= a && x < b) pt[x - lo] = codes[i];
                    }
                }
            }
            // parameter bytes overlapping [lo, hi)
            a = max(lo, S.s_off);
            b = min(hi, sc_end);
            if (a < b) {
                for (uint32_t g = (a - S.s_off) / ppg; g <= (b - 1 - S.s_off) / ppg; ++g) {
                    uint8_t codes[64];
                    uint32_t prm;
                    quant_any<DT>(group_ptr(src, p.head_dim, S.gpv, S.col, g * cpg), S.kind, codes, prm);
                    for (uint32_t i = 0; i < ppg; ++i) {
                        const uint32_t x = S.s_off + ppg * g + i;
                        if (x >= a && x < b) pt[x - lo] = (uint8_t)(prm >> (8 * i));
                    }
                }
            }
        }
        const EgressPage pg = egress_page(p, page);
        uint32_t ks[16];
        chacha_block(p.key, 1u + lo / 64u, (uint32_t)pg.seq, (uint32_t)(pg.seq >> 32), pg.nonce2, ks);
        uint8_t* dst = pg.blob + kHeader + lo;
        for (uint32_t i = 0; i < hi - lo; ++i) dst[i] = pt[i] ^ (uint8_t)(ks[i / 4] >> (8 * (i % 4)));
    }
}

__device__ __forceinline__ uint64_t load_u64_bytes(const uint8_t* p) {
    uint64_t v = 0;
    for (int i = 0; i < 8; ++i) v |= (uint64_t)p[i] << (8 * i);
    return v;
}

// SipHash over data[0, len) with byte loads; the final word folds len & 0xff.
__device__ void siphash_bytes(Sip& s, const uint8_t* data, uint64_t len, uint64_t& lo, uint64_t& hi) {
    const uint64_t nw = len / 8;
    for (uint64_t i = 0; i < nw; ++i) s.absorb(load_u64_bytes(data + 8 * i));
    uint64_t last = (len & 0xFFull) << 56;
    for (uint64_t b = 0; b < (len & 7ull); ++b) last |= (uint64_t)data[nw * 8 + b] << (8 * b);
    s.finish(last, lo, hi);
}

__global__ void egress_generic_mac_kernel(EgressParams p) {
    const int64_t page = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (page >= p.batch) return;
    const EgressPage pg = egress_page(p, page);
    uint8_t* blob = pg.blob;
    const uint64_t hw[4] = {p.hdr0, pg.hdr1, pg.token, pg.seq};
    for (int i = 0; i < 32; ++i) blob[i] = (uint8_t)(hw[i / 8] >> (8 * (i % 8)));
    Sip s;
    s.init(p.mk0, p.mk1);
    uint64_t lo, hi;
    siphash_bytes(s, blob, (uint64_t)kHeader + p.payload, lo, hi);
    uint8_t* tag = blob + kHeader + p.payload;
    for (int i = 0; i < 8; ++i) {
        tag[i] = (uint8_t)(lo >> (8 * i));
        tag[8 + i] = (uint8_t)(hi >> (8 * i));
    }
}

__global__ void ingress_generic_verify_kernel(IngressParams p, int32_t* status) {
    const int64_t page = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (page >= p.batch) return;
    const uint8_t* blob = ingress_blob(p, page);
    const uint64_t w0 = load_u64_bytes(blob), w1 = load_u64_bytes(blob + 8);
    const uint64_t tok = load_u64_bytes(blob + 16);
    Sip s;
    s.init(p.mk0, p.mk1);
    uint64_t lo, hi;
    siphash_bytes(s, blob, (uint64_t)kHeader + p.payload, lo, hi);
    const uint8_t* tag = blob + kHeader + p.payload;
    const uint64_t tlo = load_u64_bytes(tag), thi = load_u64_bytes(tag + 8);
    const uint32_t magic = (uint32_t)(w0 & 0xFFFFu), version = (uint32_t)((w0 >> 16) & 0xFFu);
    const uint32_t flags = (uint32_t)((w0 >> 24) & 0xFFu);
    int32_t st = 0;
    if (magic != kMagic || version != kVersion) st = 1;
    else if ((uint32_t)(w0 >> 32) != p.exp_tenant || (uint32_t)w1 != p.exp_model ||
             (uint32_t)((w1 >> 32) & 0xFFFFu) != ingress_layer(p, page) || tok != ingress_token(p, page))
        st = 2;
    else if ((tlo ^ lo) | (thi ^ hi)) st = 3;
    else {
        const uint32_t preset = flags & 0x0Fu, rope_mode = flags >> 4;
        if (!flags_valid(preset, rope_mode) || !((p.lay_ok >> ((preset - 1u) * 4u + rope_mode)) & 1u))
            st = 1;
    }
    status[page] = st;
    if (st != 0) atomicMin(&p.call->fail, ((unsigned long long)page << 8) | (unsigned long long)st);
}

template <int DT>
__global__ void ingress_generic_decode_kernel(IngressParams p, int64_t groups_per_page) {
    const int64_t total = p.batch * groups_per_page;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t page = t / groups_per_page;
        int64_t gi = t - page * groups_per_page;
        const uint8_t* blob = ingress_blob(p, page);
        const uint64_t w0 = load_u64_bytes(blob), w1 = load_u64_bytes(blob + 8);
        const uint64_t seq = load_u64_bytes(blob + 24);
        const uint32_t flags = (uint32_t)((w0 >> 24) & 0xFFu);
        const uint32_t preset = flags & 0x0Fu, rope_mode = flags >> 4;
        if (!flags_valid(preset, rope_mode)) continue;
        const int li = (int)((preset - 1u) * 4u + rope_mode);
        if (!((p.lay_ok >> li) & 1u)) continue;
        const Layout L = ingress_layout(p, li);
        int si = 0;
        while (si < L.n_sec - 1 && gi >= L.sec[si].n_groups) gi -= L.sec[si++].n_groups;
        const Section S = L.sec[si];
        if (gi >= S.n_groups) continue;
        const uint32_t n0 = (uint32_t)seq, n1 = (uint32_t)(seq >> 32);
        const uint32_t layer = (uint32_t)((w1 >> 32) & 0xFFFFu), hg = (uint32_t)(w1 >> 48);
        const uint32_t n2 = (layer << 16) | hg;
        const uint8_t* pay = blob + kHeader;
        uint8_t* out = S.src ? ingress_v(p, page) : ingress_k(p, page);
        const int64_t ges = group_elems(S.kind), gpvec = (int64_t)S.gpv * 16 / ges;  // groups per vector
        uint8_t* dst = out + ((gi / gpvec) * p.head_dim + S.col + (gi % gpvec) * ges) * 2;
        if (S.kind == kSecRaw) {
            uint8_t ks[32];
            keystream_bytes(p.key, n0, n1, n2, S.q_off + (uint32_t)gi * 32u, 32u, ks);
            for (int i = 0; i < 32; ++i) dst[i] = pay[S.q_off + gi * 32 + i] ^ ks[i];
            continue;
        }
        const uint32_t bpg = (uint32_t)code_bytes_per_group(S.kind);
        const uint32_t ppg = (uint32_t)param_bytes_per_group(S.kind);
        uint8_t ks[64], sk[4];
        keystream_bytes(p.key, n0, n1, n2, S.q_off + (uint32_t)gi * bpg, bpg, ks);
        keystream_bytes(p.key, n0, n1, n2, S.s_off + ppg * (uint32_t)gi, ppg, sk);
        uint32_t prm = 0;
        for (uint32_t i = 0; i < ppg; ++i) prm |= (uint32_t)(pay[S.s_off + ppg * gi + i] ^ sk[i]) << (8 * i);
        uint32_t q[16];
        for (int i = 0; i < 16; ++i) q[i] = 0u;
        for (uint32_t i = 0; i < bpg; ++i)
            q[i / 4] |= (uint32_t)(pay[S.q_off + gi * bpg + i] ^ ks[i]) << (8 * (i % 4));
        uint32_t o[32];
        if (S.kind == kSecInt8) dequant_group_int8<DT>(q, prm, o);
        else if (S.kind == kSecInt4) dequant_group_int4<DT>(q, prm, o);
        else if (S.kind == kSecE4m3) dequant_group_e4m3<DT>(q, prm, o);
        else if (S.kind == kSecInt4G32) {
            dequant_group_int4<DT>(q, prm, o);
            dequant_group_int4<DT>(q + 2, prm, o + 8);
        } else {
            for (int c = 0; c < 4; ++c) dequant_asym8_16<DT>(q + 4 * c, prm, o + 8 * c);
        }
        if ((prm & 0x7C00u) == 0x7C00u)  // an inf / NaN scale: NaN outputs as the reference writes them
            for (int c = 0; c < 4; ++c) canonical_nans<DT>(o + 8 * c);
        for (int64_t i = 0; i < 2 * ges; ++i) dst[i] = (uint8_t)(o[i / 4] >> (8 * (i % 4)));
    }
}

// Zero failing pages (per-page mode) or, when any page failed, every page
// (all-or-nothing); byte stores keep any alignment legal.
__global__ void ingress_generic_zero_kernel(IngressParams p, const int32_t* status, int all) {
    if (all && p.call->fail == ~0ull) return;
    const int64_t total = p.page_bytes * p.batch;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t page = i / p.page_bytes, off = i - page * p.page_bytes;
        if (!all && status[page] == 0) continue;
        ingress_k(p, page)[off] = 0;
        uint8_t* v = ingress_v(p, page);
        if (v) v[off] = 0;
    }
}

// ---- known-answer hooks (cpp:2499-2538) ------------------------------------

__global__ void chacha_xor_kernel(const uint8_t* src, uint8_t* dst, uint64_t len, ChaKey key,
                                  uint32_t ctr, uint32_t n0, uint32_t n1, uint32_t n2) {
    const uint64_t nblk = (len + 63) / 64;
    for (uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nblk;
         b += (uint64_t)gridDim.x * blockDim.x) {
        uint32_t ks[16];
        chacha_block(key, ctr + (uint32_t)b, n0, n1, n2, ks);
        const uint64_t lo = b * 64, n = min((uint64_t)64, len - lo);
        for (uint64_t i = 0; i < n; ++i) dst[lo + i] = src[lo + i] ^ (uint8_t)(ks[i / 4] >> (8 * (i % 4)));
    }
}

__global__ void siphash_kernel(const uint8_t* data, uint64_t len, uint64_t mk0, uint64_t mk1,
                               uint8_t* tag) {
    if (blockIdx.x != 0 || threadIdx.x != 0) return;
    Sip s;
    s.init(mk0, mk1);
    uint64_t lo, hi;
    siphash_bytes(s, data, len, lo, hi);
    for (int i = 0; i < 8; ++i) {
        tag[i] = (uint8_t)(lo >> (8 * i));
        tag[8 + i] = (uint8_t)(hi >> (8 * i));
    }
}

// ---- self-test of the fast quantizer arithmetic -------------------------------
// Thread i covers magnitude bits i of both hot dtypes (amax candidates) and,
// for i < 0x7C00, the fp16 scale with bits i (reciprocal candidates).
// Violations: an int8 / int4 fast scale that is a normal fp16 value but
// differs from fp16(amax / C) by IEEE division, an e4m3 fast scale that
// differs from fp16(amax / 448) at all, or a fast reciprocal that differs
// from 1 / s.
__global__ void selftest_kernel(unsigned int* bad) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= 0x8000u) return;
    uint32_t n = 0;
    const float cand[2] = {__uint_as_float(i << 16), f16_to_f32(i)};
    for (int d = 0; d < 2; ++d) {
        const float a = cand[d] > 1e-6f ? cand[d] : 1e-6f;
        if (!(a < __builtin_inff())) continue;
        const uint32_t f8 = scale_fast<8>(a), f4 = scale_fast<4>(a);
        if (f8 >= 0x0400u && f8 < 0x7C00u && f8 != f32_to_f16(a / 127.0f)) ++n;
        if (f4 >= 0x0400u && f4 < 0x7C00u && f4 != f32_to_f16(a / 7.0f)) ++n;
        if (scale_e4m3(a) != f32_to_f16(a / 448.0f)) ++n;  // e4m3: every result
    }
    if (i > 0 && i < 0x7C00u) {
        const float sv = f16_to_f32(i);
        if (__float_as_uint(recip_fast(sv)) != __float_as_uint(1.0f / sv)) ++n;
    }
    if (n) atomicAdd(bad, n);
}

// The hardware e4m3 conversions the kernels use, against the bit-exact
// software forms (f32_to_e4m3_sat, e4m3_to_f32_sw; the oracle's conversion is
// the software one, pinned by torch.float8_e4m3fn).  Thread i covers the fp32
// values (i << 16) | o for five low halves o: every bf16 pattern (which
// includes every rounding tie of e4m3) and values just above and below them;
// threads below 256 also decode code i in each byte position.  Violations
// are counted.
__global__ void selftest_e4m3_kernel(unsigned int* bad) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= 0x10000u) return;
    uint32_t n = 0;
    const uint32_t lows[5] = {0x0000u, 0x0001u, 0x7FFFu, 0x8000u, 0xFFFFu};
    for (int k = 0; k < 5; k += 2) {
        const float a = __uint_as_float((i << 16) | lows[k]);
        const float b = __uint_as_float((i << 16) | lows[k < 4 ? k + 1 : k]);
        const uint32_t hw = e4m3_pair_hw(e4m3_operand(a), e4m3_operand(b));
        if (a == a && (hw & 0xFFu) != f32_to_e4m3_sat(a)) ++n;
        if (b == b && (hw >> 8) != f32_to_e4m3_sat(b)) ++n;
    }
    if (i < 256u) {  // code i in each byte position of a word
        const float sw = e4m3_to_f32_sw(i);
        const float h[4] = {e4m3_byte_to_f32<0>(i), e4m3_byte_to_f32<1>(i << 8), e4m3_byte_to_f32<2>(i << 16),
                            e4m3_byte_to_f32<3>(i << 24)};
        for (int b = 0; b < 4; ++b)
            if (!(h[b] != h[b] && sw != sw) && __float_as_uint(h[b]) != __float_as_uint(sw)) ++n;
    }
    if (n) atomicAdd(bad, n);
}

hipError_t launch_selftest(unsigned int* bad, hipStream_t s) {
    hipLaunchKernelGGL(selftest_kernel, dim3(0x8000 / 256), dim3(256), 0, s, bad);
    hipLaunchKernelGGL(selftest_e4m3_kernel, dim3(0x10000 / 256), dim3(256), 0, s, bad);
    return hipGetLastError();
}

// ---- launchers ---------------------------------------------------------------

static uint32_t grid_for(int64_t items, int block, int64_t cap = 65536) {
    int64_t g = (items + block - 1) / block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (uint32_t)g;
}

hipError_t launch_egress_generic(const EgressParams& p, int dtype, hipStream_t s) {
    const int64_t nblk = ((int64_t)p.payload + 63) / 64;
    if (nblk > 0) {
        const uint32_t g = grid_for(p.batch * nblk, 256);
        if (dtype == kHotBf16)
            hipLaunchKernelGGL(egress_generic_blocks_kernel<kHotBf16>, dim3(g), dim3(256), 0, s, p, nblk);
        else
            hipLaunchKernelGGL(egress_generic_blocks_kernel<kHotFp16>, dim3(g), dim3(256), 0, s, p, nblk);
    }
    hipLaunchKernelGGL(egress_generic_mac_kernel, dim3(grid_for(p.batch, 64)), dim3(64), 0, s, p);
    return hipGetLastError();
}

// `status` must hold p.batch entries (the caller's array or library scratch).
hipError_t launch_ingress_generic_impl(const IngressParams& p, int dtype, int32_t* status,
                                       hipStream_t s) {
    hipLaunchKernelGGL(ingress_generic_verify_kernel, dim3(grid_for(p.batch, 64)), dim3(64), 0, s, p,
                       status);
    const int64_t gpp = (int64_t)p.n_units;  // groups per page (see host)
    if (dtype == kHotBf16)
        hipLaunchKernelGGL(ingress_generic_decode_kernel<kHotBf16>, dim3(grid_for(p.batch * gpp, 256)),
                           dim3(256), 0, s, p, gpp);
    else
        hipLaunchKernelGGL(ingress_generic_decode_kernel<kHotFp16>, dim3(grid_for(p.batch * gpp, 256)),
                           dim3(256), 0, s, p, gpp);
    hipLaunchKernelGGL(ingress_generic_zero_kernel, dim3(grid_for(p.page_bytes * p.batch, 256, 8192)),
                       dim3(256), 0, s, p, status, p.per_page ? 0 : 1);
    return hipGetLastError();
}

hipError_t launch_chacha_xor(const uint8_t* src, uint8_t* dst, size_t len, ChaKey key, uint32_t ctr,
                             uint32_t n0, uint32_t n1, uint32_t n2, hipStream_t s) {
    const uint32_t g = grid_for((int64_t)((len + 63) / 64), 256);
    hipLaunchKernelGGL(chacha_xor_kernel, dim3(g), dim3(256), 0, s, src, dst, (uint64_t)len, key, ctr,
                       n0, n1, n2);
    return hipGetLastError();
}

hipError_t launch_siphash(const uint8_t* data, size_t len, uint64_t mk0, uint64_t mk1, uint8_t* tag,
                          hipStream_t s) {
    hipLaunchKernelGGL(siphash_kernel, dim3(1), dim3(64), 0, s, data, (uint64_t)len, mk0, mk1, tag);
    return hipGetLastError();
}

}  // namespace ztcp
