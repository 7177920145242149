/*
 * ztcp_oracle.c -- CPU restatement of the ZTCP fused cold-page codec
 * (profile S of research/baseline_codec/csrc/fused_cold_page_cpu.cpp).
 *
 * TEST INFRASTRUCTURE ONLY: the CPU reference the HIP path is compared with.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Build: gcc -O2 -std=c11 -ffp-contract=off (never -ffast-math); the fp32
 * operations below are evaluated exactly in the order the reference writes
 * them.  Built by oracle/build.py.
 *
 * Parity pins (tests/test_oracle_*.py):
 *   ChaCha20      RFC 8439 2.3.2 / 2.4.2 / A.1 / A.2 known answers.
 *   SipHash-128   Aumasson-Bernstein vectors_sip128 (key 00..0f, msg 00..3f).
 *   fp16/bf16     numpy float16 / torch bfloat16 conversions, exhaustively.
 *   quantizers    closed forms + the compiled reference (oracle/_ref).
 *   pages         byte-identical blobs and outputs vs the compiled reference
 *                 (oracle/_ref) for every preset x rope mode, FP16; committed
 *                 golden fixtures in tests/golden/.
 */
#define _GNU_SOURCE
#include "ztcp_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define ZO_MAGIC 0x5A54u
#define ZO_VERSION 1u
#define ZO_HEADER 32u
#define ZO_TAG 16u
#define ZO_GS 16

/* ------------------------------------------------------------------------ */
/* Bit casts and IEEE conversions (c10::Half / c10::BFloat16 semantics).    */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* fp32 -> fp16, round to nearest even, subnormals kept, overflow to inf.
 * NaN becomes sign | 0x7E00 (c10's software conversion, which the
 * reference's at::Half assignments use on x86). */
uint16_t zo_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 */
    if (ax >= 0x38800000u) {                                   /* >= 2^-14 */
        uint32_t r = ax - (112u << 23);
        r += 0xFFFu + ((r >> 13) & 1u);
        return (uint16_t)(sign | (r >> 13));
    }
    uint32_t e = ax >> 23;
    if (e == 0) return (uint16_t)sign; /* fp32 subnormal or zero: < 2^-126 */
    uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126u - e; /* value / 2^-24 = mant * 2^(e-126) */
    if (shift > 24) return (uint16_t)sign;
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float zo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0x1F) return u2f(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return u2f(sign);
        /* subnormal: m * 2^-24, exact in fp32 */
        float v = (float)m * u2f(0x33800000u); /* 2^-24 */
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* fp32 -> bf16 round to nearest even; NaN -> 0x7FC0 (c10::BFloat16). */
uint16_t zo_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float zo_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

static inline float hot_to_f32(uint16_t v, int dtype) {
    return dtype == ZO_BF16 ? zo_bf16_to_f32(v) : zo_f16_to_f32(v);
}
static inline uint16_t f32_to_hot(float f, int dtype) {
    return dtype == ZO_BF16 ? zo_f32_to_bf16(f) : zo_f32_to_f16(f);
}

/* ------------------------------------------------------------------------ */
/* ChaCha20 (RFC 8439 2.3), cpp:157-188 (scalar block), cpp:356-398 (XOR).   */
/* ------------------------------------------------------------------------ */

static inline uint32_t rotl32(uint32_t x, int b) { return (x << b) | (x >> (32 - b)); }
static inline uint64_t rotl64(uint64_t x, int b) { return (x << b) | (x >> (64 - b)); }
static inline uint32_t ld32(const uint8_t* p) { uint32_t v; memcpy(&v, p, 4); return v; }
static inline uint64_t ld64(const uint8_t* p) { uint64_t v; memcpy(&v, p, 8); return v; }

#define QR(a, b, c, d)                        \
    do {                                      \
        a += b; d = rotl32(d ^ a, 16);        \
        c += d; b = rotl32(b ^ c, 12);        \
        a += b; d = rotl32(d ^ a, 8);         \
        c += d; b = rotl32(b ^ c, 7);         \
    } while (0)

void zo_chacha20_block(const uint32_t key[8], uint32_t counter,
                       const uint32_t nonce[3], uint8_t out[64]) {
    uint32_t s[16] = {0x61707865u, 0x3320646Eu, 0x79622D32u, 0x6B206574u,
                      key[0], key[1], key[2], key[3],
                      key[4], key[5], key[6], key[7],
                      counter, nonce[0], nonce[1], nonce[2]};
    uint32_t x[16];
    memcpy(x, s, sizeof x);
    for (int i = 0; i < 10; ++i) {
        QR(x[0], x[4], x[8], x[12]);
        QR(x[1], x[5], x[9], x[13]);
        QR(x[2], x[6], x[10], x[14]);
        QR(x[3], x[7], x[11], x[15]);
        QR(x[0], x[5], x[10], x[15]);
        QR(x[1], x[6], x[11], x[12]);
        QR(x[2], x[7], x[8], x[13]);
        QR(x[3], x[4], x[9], x[14]);
    }
    for (int i = 0; i < 16; ++i) {
        uint32_t w = x[i] + s[i];
        memcpy(out + 4 * i, &w, 4);
    }
}

/* Keystream for bytes [0, len) starting at block `counter`; cpp:356-398. */
static void chacha_xor_words(const uint8_t* src, uint8_t* dst, size_t len,
                             const uint32_t key[8], uint32_t counter,
                             const uint32_t nonce[3]) {
    uint8_t ks[64];
    size_t off = 0;
    while (off < len) {
        zo_chacha20_block(key, counter++, nonce, ks);
        size_t n = len - off < 64 ? len - off : 64;
        for (size_t j = 0; j < n; ++j) dst[off + j] = src[off + j] ^ ks[j];
        off += n;
    }
}

void zo_chacha20_xor(const uint8_t* src, uint8_t* dst, size_t len,
                     const uint8_t key32[32], uint32_t counter,
                     const uint8_t nonce12[12]) {
    /* cpp:2499-2524: key and nonce bytes are read as little-endian words. */
    uint32_t key[8], nonce[3];
    for (int i = 0; i < 8; ++i) key[i] = ld32(key32 + 4 * i);
    for (int i = 0; i < 3; ++i) nonce[i] = ld32(nonce12 + 4 * i);
    chacha_xor_words(src, dst, len, key, counter, nonce);
}

/* ------------------------------------------------------------------------ */
/* SipHash-2-4-128, cpp:401-471.                                            */
/* ------------------------------------------------------------------------ */

typedef struct { uint64_t v0, v1, v2, v3; } sip_t;

static inline void sipround(sip_t* s) {
    s->v0 += s->v1; s->v1 = rotl64(s->v1, 13); s->v1 ^= s->v0; s->v0 = rotl64(s->v0, 32);
    s->v2 += s->v3; s->v3 = rotl64(s->v3, 16); s->v3 ^= s->v2;
    s->v0 += s->v3; s->v3 = rotl64(s->v3, 21); s->v3 ^= s->v0;
    s->v2 += s->v1; s->v1 = rotl64(s->v1, 17); s->v1 ^= s->v2; s->v2 = rotl64(s->v2, 32);
}

static inline void sip_absorb(sip_t* s, uint64_t m) { /* cpp:418-423 */
    s->v3 ^= m;
    sipround(s);
    sipround(s);
    s->v0 ^= m;
}

void zo_siphash128(const uint8_t* data, size_t len, uint64_t mk0, uint64_t mk1,
                   uint8_t tag[16]) {
    sip_t s; /* cpp:404-409 (128-bit variant: v1 ^= 0xee) */
    s.v0 = 0x736F6D6570736575ull ^ mk0;
    s.v1 = 0x646F72616E646F6Dull ^ mk1 ^ 0xEEull;
    s.v2 = 0x6C7967656E657261ull ^ mk0;
    s.v3 = 0x7465646279746573ull ^ mk1;
    size_t nw = len / 8;
    for (size_t i = 0; i < nw; ++i) sip_absorb(&s, ld64(data + 8 * i));
    /* cpp:438-444: last word = (len & 0xff) << 56 | tail bytes */
    uint64_t last = (uint64_t)(len & 0xFFu) << 56;
    for (size_t b = 0; b < (len & 7u); ++b) last |= (uint64_t)data[nw * 8 + b] << (8 * b);
    sip_absorb(&s, last);
    /* cpp:447-456 */
    s.v2 ^= 0xEEull;
    for (int i = 0; i < 4; ++i) sipround(&s);
    uint64_t lo = s.v0 ^ s.v1 ^ s.v2 ^ s.v3;
    s.v1 ^= 0xDDull;
    for (int i = 0; i < 4; ++i) sipround(&s);
    uint64_t hi = s.v0 ^ s.v1 ^ s.v2 ^ s.v3;
    memcpy(tag, &lo, 8);
    memcpy(tag + 8, &hi, 8);
}

/* ------------------------------------------------------------------------ */
/* Group-16 quantizers, profile S (cpp:735-753, cpp:806-824) and            */
/* dequantizers (cpp:772-776, cpp:846-853).                                 */
/* ------------------------------------------------------------------------ */

/* x86 float->int conversion of NaN / out-of-range yields INT_MIN (the
 * reference's static_casts compile to cvttss2si); only NaN reaches it here. */
static inline int f32_to_int_x86(float f) {
    if (f != f || f >= 2147483648.0f || f < -2147483648.0f) return INT32_MIN;
    return (int)f;
}

void zo_quant_group16_int8(const uint16_t* src, int dtype, uint8_t q[16],
                           uint16_t* scale_f16) {
    float amax = 1e-6f;
    float vals[16];
    for (int i = 0; i < 16; ++i) {
        float v = hot_to_f32(src[i], dtype);
        vals[i] = v;
        float av = fabsf(v);
        if (av > amax) amax = av;
    }
    uint16_t sh = zo_f32_to_f16(amax / 127.0f);
    *scale_f16 = sh;
    float inv = 1.0f / zo_f16_to_f32(sh);
    for (int i = 0; i < 16; ++i) {
        float qf = nearbyintf(vals[i] * inv);
        if (qf < -127.0f) qf = -127.0f;
        if (qf > 127.0f) qf = 127.0f;
        /* static_cast<int8_t>(qf): int conversion, then the low byte */
        q[i] = (uint8_t)(f32_to_int_x86(qf) & 0xFF);
    }
}

void zo_quant_group16_int4(const uint16_t* src, int dtype, uint8_t q[8],
                           uint16_t* scale_f16) {
    float amax = 1e-6f;
    float vals[16];
    for (int i = 0; i < 16; ++i) {
        float v = hot_to_f32(src[i], dtype);
        vals[i] = v;
        float av = fabsf(v);
        if (av > amax) amax = av;
    }
    uint16_t sh = zo_f32_to_f16(amax / 7.0f);
    *scale_f16 = sh;
    float inv = 1.0f / zo_f16_to_f32(sh);
    for (int i = 0; i < 8; ++i) {
        float q0 = nearbyintf(vals[2 * i] * inv) + 8.0f;
        float q1 = nearbyintf(vals[2 * i + 1] * inv) + 8.0f;
        int u0 = f32_to_int_x86(q0);
        int u1 = f32_to_int_x86(q1);
        u0 = u0 < 0 ? 0 : (u0 > 15 ? 15 : u0);
        u1 = u1 < 0 ? 0 : (u1 > 15 ? 15 : u1);
        q[i] = (uint8_t)((u0 & 0x0F) | ((u1 & 0x0F) << 4)); /* cpp:823 */
    }
}

void zo_dequant_group16_int8(const uint8_t q[16], uint16_t scale_f16, int dtype,
                             uint16_t* dst) {
    float s = zo_f16_to_f32(scale_f16);
    for (int i = 0; i < 16; ++i) dst[i] = f32_to_hot((float)(int8_t)q[i] * s, dtype);
}

void zo_dequant_group16_int4(const uint8_t q[8], uint16_t scale_f16, int dtype,
                             uint16_t* dst) {
    float s = zo_f16_to_f32(scale_f16);
    for (int i = 0; i < 8; ++i) {
        float v0 = (float)(q[i] & 0x0F) - 8.0f;
        float v1 = (float)((q[i] >> 4) & 0x0F) - 8.0f;
        dst[2 * i] = f32_to_hot(v0 * s, dtype);
        dst[2 * i + 1] = f32_to_hot(v1 * s, dtype);
    }
}

/* ------------------------------------------------------------------------ */
/* Extension codes (no counterpart in the reference; defined by this codec). */
/* They follow profile S's shape: an fp32 statistic, an fp16 scale rounded  */
/* once, inv = 1 / f32(scale), codes by round-to-nearest-even, and a        */
/* dequantization whose product is exact in fp32 followed by one RNE to the  */
/* hot dtype.                                                               */
/* ------------------------------------------------------------------------ */

/* fp32 -> OCP FP8 e4m3 ("e4m3fn": bias 7, no infinities, NaN 0x7F/0xFF,
 * largest finite 448), saturating: |x| >= 448 gives +-448, NaN gives 0x7F;
 * otherwise round to nearest even (subnormal step 2^-9). */
uint8_t zo_f32_to_e4m3(float x) {
    if (x != x) return 0x7F;
    const uint8_t sign = (uint8_t)((f2u(x) >> 24) & 0x80u);
    const float a = fabsf(x);
    if (a >= 448.0f) return (uint8_t)(sign | 0x7E);
    if (a < 0.015625f) { /* below 2^-6: multiples of 2^-9; a * 512 is exact */
        return (uint8_t)(sign | (uint8_t)nearbyintf(a * 512.0f)); /* 8 -> 0x08 = 2^-6 */
    }
    const uint32_t u = f2u(a);
    int e = (int)(u >> 23) - 127;                /* -6 .. 8 */
    uint32_t m = (u & 0x7FFFFFu) | 0x800000u;    /* 24-bit significand */
    uint32_t r = m >> 20, rem = m & 0xFFFFFu;   /* keep 1 + 3 bits */
    if (rem > 0x80000u || (rem == 0x80000u && (r & 1u))) r++;
    if (r == 16u) { r = 8u; e++; }
    return (uint8_t)(sign | (uint8_t)(((uint32_t)(e + 7) << 3) | (r & 7u)));
}

float zo_e4m3_to_f32(uint8_t c) {
    const uint32_t e = (c >> 3) & 0xFu, m = c & 7u;
    float v;
    if (e == 0xFu && m == 7u) v = u2f(0x7FC00000u);
    else if (e == 0) v = (float)m * 0.001953125f; /* m * 2^-9, exact */
    else v = u2f(((e + 120u) << 23) | (m << 20));
    return (c & 0x80u) ? -v : v;
}

static float group_amax(const uint16_t* src, int dtype, int n, float* vals) {
    float amax = 1e-6f;
    for (int i = 0; i < n; ++i) {
        float v = hot_to_f32(src[i], dtype);
        vals[i] = v;
        float av = fabsf(v);
        if (av > amax) amax = av;
    }
    return amax;
}

/* FP8 e4m3, 16-element group: s = fp16(amax / 448), codes e4m3(v * inv).
 * A NaN product (0 * inf when the scale underflows to 0, or a NaN input)
 * gives code 0, as the reference's integer conversion of NaN gives code 0
 * in its int8 quantizer (cpp:735-753): a group too small for an fp16 scale
 * decodes to zeros, never to NaN. */
void zo_quant_group16_e4m3(const uint16_t* src, int dtype, uint8_t q[16],
                           uint16_t* scale_f16) {
    float vals[16];
    const float amax = group_amax(src, dtype, 16, vals);
    const uint16_t sh = zo_f32_to_f16(amax / 448.0f);
    *scale_f16 = sh;
    const float inv = 1.0f / zo_f16_to_f32(sh);
    for (int i = 0; i < 16; ++i) {
        const float x = vals[i] * inv;
        q[i] = x != x ? 0 : zo_f32_to_e4m3(x);
    }
}

void zo_dequant_group16_e4m3(const uint8_t q[16], uint16_t scale_f16, int dtype,
                             uint16_t* dst) {
    const float s = zo_f16_to_f32(scale_f16);
    for (int i = 0; i < 16; ++i) dst[i] = f32_to_hot(zo_e4m3_to_f32(q[i]) * s, dtype);
}

/* INT4 symmetric over a 32-element group: the int4 formula of cpp:806-824
 * with the absmax taken over 32 elements; 16 code bytes, one fp16 scale. */
void zo_quant_group32_int4(const uint16_t* src, int dtype, uint8_t q[16],
                           uint16_t* scale_f16) {
    float vals[32];
    const float amax = group_amax(src, dtype, 32, vals);
    const uint16_t sh = zo_f32_to_f16(amax / 7.0f);
    *scale_f16 = sh;
    const float inv = 1.0f / zo_f16_to_f32(sh);
    for (int i = 0; i < 16; ++i) {
        int u0 = f32_to_int_x86(nearbyintf(vals[2 * i] * inv) + 8.0f);
        int u1 = f32_to_int_x86(nearbyintf(vals[2 * i + 1] * inv) + 8.0f);
        u0 = u0 < 0 ? 0 : (u0 > 15 ? 15 : u0);
        u1 = u1 < 0 ? 0 : (u1 > 15 ? 15 : u1);
        q[i] = (uint8_t)((u0 & 0x0F) | ((u1 & 0x0F) << 4));
    }
}

void zo_dequant_group32_int4(const uint8_t q[16], uint16_t scale_f16, int dtype,
                             uint16_t* dst) {
    zo_dequant_group16_int4(q, scale_f16, dtype, dst);
    zo_dequant_group16_int4(q + 8, scale_f16, dtype, dst + 16);
}

/* INT8 asymmetric over a 64-element group.  The range always includes 0:
 * lo = min(0, min v), hi = max(0, max v); s = fp16(max(1e-6, hi - lo) / 255);
 * zero point z = clamp(rne(-lo * inv), 0, 255); q = clamp(rne(v * inv) + z,
 * 0, 255).  Parameters on the wire: fp16 scale, then z as a little-endian
 * u16.  Dequantized: f32(q - z) * f32(s), exact in fp32, one RNE. */
void zo_quant_group64_asym8(const uint16_t* src, int dtype, uint8_t q[64],
                            uint16_t* scale_f16, uint16_t* zero) {
    float vals[64];
    float lo = 0.0f, hi = 0.0f;
    for (int i = 0; i < 64; ++i) {
        float v = hot_to_f32(src[i], dtype);
        vals[i] = v;
        if (v < lo) lo = v;
        if (v > hi) hi = v;
    }
    float range = hi - lo;
    if (!(range > 1e-6f)) range = 1e-6f;
    const uint16_t sh = zo_f32_to_f16(range / 255.0f);
    *scale_f16 = sh;
    const float inv = 1.0f / zo_f16_to_f32(sh);
    float zf = nearbyintf(-lo * inv);
    if (zf < 0.0f) zf = 0.0f;
    if (zf > 255.0f) zf = 255.0f;
    const int z = f32_to_int_x86(zf) & 0xFF;
    *zero = (uint16_t)z;
    for (int i = 0; i < 64; ++i) {
        float qf = nearbyintf(vals[i] * inv) + (float)z;
        if (qf < 0.0f) qf = 0.0f;
        if (qf > 255.0f) qf = 255.0f;
        q[i] = (uint8_t)(f32_to_int_x86(qf) & 0xFF);
    }
}

void zo_dequant_group64_asym8(const uint8_t q[64], uint16_t scale_f16, uint16_t zero,
                              int dtype, uint16_t* dst) {
    const float s = zo_f16_to_f32(scale_f16);
    for (int i = 0; i < 64; ++i) dst[i] = f32_to_hot((float)((int)q[i] - (int)zero) * s, dtype);
}

/* ------------------------------------------------------------------------ */
/* Sizing: cpp:1439-1474 (native, unpadded) and spec:203-246 (padded).      */
/* ------------------------------------------------------------------------ */

/* Section kinds.  INT8 / INT4 / RAW are the reference's (16-element groups,
 * cpp:1157-1374); E4M3, INT4G32 and ASYM8 are this codec's extensions. */
enum { SEC_INT8 = 0, SEC_INT4 = 1, SEC_RAW = 2, SEC_E4M3 = 3, SEC_INT4G32 = 4, SEC_ASYM8 = 5 };
static const int SEC_GES[6] = {16, 16, 16, 16, 32, 64}; /* elements per group */
static const int SEC_CB[6] = {16, 8, 32, 16, 16, 64};   /* code bytes per group */
static const int SEC_PB[6] = {2, 2, 0, 2, 2, 4};        /* scale / zero bytes per group */

/* Presets 1..3 and RoPE modes 0..2 are the reference's (cpp:1447-1449);
 * presets 4..6 and RoPE mode 3 are extensions:
 *   4 K8V4_ASYM     K: int8 asymmetric per 64 (ASYM8), V: int4 per 32 (INT4G32)
 *   5 FP8_E4M3      K and V: e4m3 per 16 (E4M3)
 *   6 INT4_SYM_G32  K and V: int4 per 32 (INT4G32)
 *   RoPE mode 3     PRESERVE_E4M3: the RoPE columns as e4m3 per 16.
 * Returns -1 for flags outside these. */
static int rope_kind(int64_t rope_mode) {
    return rope_mode == 1 ? SEC_INT8 : (rope_mode == 2 ? SEC_RAW : (rope_mode == 3 ? SEC_E4M3 : -1));
}
static int kmain_kind(int64_t preset) {
    static const int k[7] = {-1, SEC_INT4, SEC_INT8, SEC_INT8, SEC_ASYM8, SEC_E4M3, SEC_INT4G32};
    return preset >= 1 && preset <= 6 ? k[preset] : -1;
}
static int v_kind(int64_t preset) {
    static const int k[7] = {-1, SEC_INT4, SEC_INT4, SEC_INT8, SEC_INT4G32, SEC_E4M3, SEC_INT4G32};
    return preset >= 1 && preset <= 6 ? k[preset] : -1;
}
static int flags_valid(int64_t preset, int64_t rope_mode) {
    return preset >= 1 && preset <= 6 && rope_mode >= 0 && rope_mode <= 3;
}

/* Bytes of one section of `width` columns over `vecs` vectors; (size_t)-1
 * when an extension kind's group does not divide the width.  For the
 * reference's kinds this is the reference's per-column formula
 * (cpp:1450-1472: one code per column, one scale per whole group). */
static size_t section_bytes(int kind, int64_t vecs, int64_t width) {
    switch (kind) {
    case SEC_RAW: return (size_t)vecs * (size_t)width * 2u;
    case SEC_INT8: return (size_t)(vecs * width) + (size_t)vecs * (size_t)(width / ZO_GS) * 2u;
    case SEC_INT4: return (size_t)(vecs * (width / 2)) + (size_t)vecs * (size_t)(width / ZO_GS) * 2u;
    default:
        if (width % SEC_GES[kind]) return (size_t)-1;
        return (size_t)vecs * (size_t)(width / SEC_GES[kind]) * (size_t)(SEC_CB[kind] + SEC_PB[kind]);
    }
}

size_t zo_required_payload(int64_t preset, int64_t rope_mode, int64_t vecs,
                           int64_t head_dim, int64_t rope_dim, int has_v) {
    if (!flags_valid(preset, rope_mode)) return (size_t)-1;
    size_t req = 0, b;
    if (rope_mode != 0 && rope_dim > 0) {
        if ((b = section_bytes(rope_kind(rope_mode), vecs, rope_dim)) == (size_t)-1) return b;
        req += b;
    }
    const int64_t kq = rope_mode == 0 ? head_dim : head_dim - rope_dim;
    if (kq > 0) {
        if ((b = section_bytes(kmain_kind(preset), vecs, kq)) == (size_t)-1) return b;
        req += b;
    }
    if (has_v) {
        if ((b = section_bytes(v_kind(preset), vecs, head_dim)) == (size_t)-1) return b;
        req += b;
    }
    return req;
}

size_t zo_payload_bytes(int64_t preset, int64_t rope_mode, int64_t vecs,
                        int64_t head_dim, int64_t rope_dim, int has_v) {
    size_t r = zo_required_payload(preset, rope_mode, vecs, head_dim, rope_dim, has_v);
    if (r == (size_t)-1) return r;
    return (r + 3u) & ~(size_t)3u;
}

/* ------------------------------------------------------------------------ */
/* Page layout: a payload is up to three sections, each [codes][fp16 scales] */
/* (or raw hot bytes), then zero padding.  cpp:1376-1422 (encode order),    */
/* cpp:2418-2461 (decode order), cpp:1146-1374 (section byte maps).          */
/* ------------------------------------------------------------------------ */

typedef struct {
    int kind;        /* SEC_* */
    int src;         /* 0 = K, 1 = V */
    int64_t col;     /* first column */
    int64_t width;   /* columns covered */
} zo_section;

static int build_sections(int64_t preset, int64_t rope_mode, int64_t head_dim,
                          int64_t rope_dim, int has_v, zo_section out[3]) {
    int n = 0;
    if (rope_mode != 0 && rope_dim > 0) out[n++] = (zo_section){rope_kind(rope_mode), 0, 0, rope_dim};
    const int64_t kq = rope_mode == 0 ? head_dim : head_dim - rope_dim;
    const int64_t kc = rope_mode == 0 ? 0 : rope_dim;
    if (kq > 0) out[n++] = (zo_section){kmain_kind(preset), 0, kc, kq};
    if (has_v) out[n++] = (zo_section){v_kind(preset), 1, 0, head_dim};
    return n;
}

/* Codes and parameters of group `gi` of a quantized section.  params[0] is
 * the fp16 scale, params[1] the zero point (ASYM8 only). */
static void quant_group_kind(int kind, const uint16_t* grp, int dtype, uint8_t* q,
                             uint16_t params[2]) {
    switch (kind) {
    case SEC_INT8: zo_quant_group16_int8(grp, dtype, q, &params[0]); break;
    case SEC_INT4: zo_quant_group16_int4(grp, dtype, q, &params[0]); break;
    case SEC_E4M3: zo_quant_group16_e4m3(grp, dtype, q, &params[0]); break;
    case SEC_INT4G32: zo_quant_group32_int4(grp, dtype, q, &params[0]); break;
    default: zo_quant_group64_asym8(grp, dtype, q, &params[0], &params[1]); break;
    }
}

static void dequant_group_kind(int kind, const uint8_t* q, const uint16_t params[2], int dtype,
                               uint16_t* out) {
    switch (kind) {
    case SEC_INT8: zo_dequant_group16_int8(q, params[0], dtype, out); break;
    case SEC_INT4: zo_dequant_group16_int4(q, params[0], dtype, out); break;
    case SEC_E4M3: zo_dequant_group16_e4m3(q, params[0], dtype, out); break;
    case SEC_INT4G32: zo_dequant_group32_int4(q, params[0], dtype, out); break;
    default: zo_dequant_group64_asym8(q, params[0], params[1], dtype, out); break;
    }
}

/* Plaintext payload of one page (section bytes, then zero padding). */
static void page_plaintext(const uint16_t* k, const uint16_t* v, int dtype,
                           int64_t vecs, int64_t head_dim, int64_t rope_dim,
                           int64_t preset, int64_t rope_mode, size_t payload_len,
                           uint8_t* plain) {
    zo_section secs[3];
    int ns = build_sections(preset, rope_mode, head_dim, rope_dim, v != NULL, secs);
    size_t off = 0;
    for (int s = 0; s < ns; ++s) {
        const uint16_t* src = secs[s].src ? v : k;
        const int64_t w = secs[s].width, col = secs[s].col;
        if (secs[s].kind == SEC_RAW) { /* cpp:1379-1386 */
            for (int64_t r = 0; r < vecs; ++r) {
                memcpy(plain + off, src + r * head_dim + col, (size_t)w * 2u);
                off += (size_t)w * 2u;
            }
            continue;
        }
        const int kind = secs[s].kind, ges = SEC_GES[kind];
        const int64_t groups = w / ges;
        const int bpg = SEC_CB[kind], pb = SEC_PB[kind];
        uint8_t* qb = plain + off;
        uint8_t* sb = qb + (size_t)(vecs * groups * bpg);
        for (int64_t r = 0; r < vecs; ++r) {
            for (int64_t g = 0; g < groups; ++g) {
                const uint16_t* grp = src + r * head_dim + col + g * ges;
                const int64_t gi = r * groups + g;
                uint16_t prm[2] = {0, 0};
                quant_group_kind(kind, grp, dtype, qb + gi * bpg, prm);
                memcpy(sb + gi * pb, prm, (size_t)pb); /* little-endian u16s */
            }
        }
        off += (size_t)(vecs * groups * (bpg + pb));
    }
    if (off < payload_len) memset(plain + off, 0, payload_len - off); /* cpp:1411-1422 */
}

static void pack_header(uint8_t h[32], uint8_t flags, uint32_t tenant, uint32_t model,
                        uint16_t layer, uint16_t hg, uint64_t tok, uint64_t seq) {
    /* cpp:61-75, cpp:1129-1140: packed little-endian header */
    uint16_t magic = ZO_MAGIC;
    memcpy(h + 0, &magic, 2);
    h[2] = ZO_VERSION;
    h[3] = flags;
    memcpy(h + 4, &tenant, 4);
    memcpy(h + 8, &model, 4);
    memcpy(h + 12, &layer, 2);
    memcpy(h + 14, &hg, 2);
    memcpy(h + 16, &tok, 8);
    memcpy(h + 24, &seq, 8);
}

static void key_words(uint64_t k0, uint64_t k1, uint64_t k2, uint64_t k3, uint32_t key[8]) {
    /* cpp:85-100 */
    const uint64_t k[4] = {k0, k1, k2, k3};
    for (int i = 0; i < 4; ++i) {
        key[2 * i] = (uint32_t)(k[i] & 0xFFFFFFFFull);
        key[2 * i + 1] = (uint32_t)(k[i] >> 32);
    }
}

static void nonce_words(uint64_t seq, uint16_t layer, uint16_t hg, uint32_t nonce[3]) {
    /* cpp:102-110, fqc:157-166 */
    nonce[0] = (uint32_t)(seq & 0xFFFFFFFFull);
    nonce[1] = (uint32_t)(seq >> 32);
    nonce[2] = ((uint32_t)layer << 16) | (uint32_t)hg;
}

/* cpp:1103-1426 (encode_one_cold_page_into_cpu).  The reference interleaves
 * quantize / encrypt / MAC in one stream; the result is, byte for byte,
 * ct = plaintext ^ keystream(counter 1..) and tag = SipHash(header || ct). */
static void encode_page(const zo_egress_args* a, int64_t b, uint8_t* plain) {
    const int64_t vecs = a->num_tokens * a->num_heads;
    const int64_t elems = vecs * a->head_dim;
    const size_t blob_bytes = ZO_HEADER + (size_t)a->expected_payload_bytes + ZO_TAG;
    const uint16_t* k = (const uint16_t*)a->k_pages + b * elems;
    const uint16_t* v = a->v_pages ? (const uint16_t*)a->v_pages + b * elems : NULL;
    uint8_t* blob = a->out_blobs + (size_t)b * blob_bytes;
    const uint64_t seq = a->base_sequence_nonce + (uint64_t)b; /* cpp:1979 */
    const uint8_t flags = (uint8_t)((a->preset & 0x0F) | ((a->rope_mode & 0x0F) << 4));
    pack_header(blob, flags, a->tenant_id_hash, a->model_id_hash, a->layer_id,
                a->head_group_id, (uint64_t)a->token_hashes[b], seq);
    const size_t plen = (size_t)a->expected_payload_bytes;
    page_plaintext(k, v, a->dtype, vecs, a->head_dim, a->rope_dim, a->preset,
                   a->rope_mode, plen, plain);
    uint32_t key[8], nonce[3];
    key_words(a->k0, a->k1, a->k2, a->k3, key);
    nonce_words(seq, a->layer_id, a->head_group_id, nonce);
    chacha_xor_words(plain, blob + ZO_HEADER, plen, key, 1u, nonce); /* cpp:497 */
    zo_siphash128(blob, ZO_HEADER + plen, a->mk0, a->mk1, blob + ZO_HEADER + plen);
    memset(plain, 0, plen);
}

/* Per-page decode lambda, cpp:2309-2463. */
static int decode_page(const zo_ingress_args* a, int64_t b, uint8_t* plain) {
    const int64_t vecs = a->num_tokens * a->num_heads;
    const int64_t elems = vecs * a->head_dim;
    const size_t total = (size_t)a->blob_bytes;
    const size_t plen = total - ZO_HEADER - ZO_TAG;
    const uint8_t* blob = a->blobs + (size_t)b * total;
    uint16_t magic; uint32_t tenant, model; uint16_t layer, hg; uint64_t tok, seq;
    memcpy(&magic, blob, 2);
    const uint8_t version = blob[2], flags = blob[3];
    memcpy(&tenant, blob + 4, 4);
    memcpy(&model, blob + 8, 4);
    memcpy(&layer, blob + 12, 2);
    memcpy(&hg, blob + 14, 2);
    memcpy(&tok, blob + 16, 8);
    memcpy(&seq, blob + 24, 8);
    if (magic != ZO_MAGIC || version != ZO_VERSION) return 1;
    if (tenant != a->expected_tenant_hash || model != a->expected_model_hash ||
        layer != a->expected_layer_id || tok != (uint64_t)a->expected_token_hashes[b])
        return 2;
    uint8_t tag[16];
    zo_siphash128(blob, ZO_HEADER + plen, a->mk0, a->mk1, tag);
    uint8_t diff = 0;
    for (int i = 0; i < 16; ++i) diff |= (uint8_t)(tag[i] ^ blob[ZO_HEADER + plen + i]);
    if (diff) return 3;
    const int preset = flags & 0x0F, rope_mode = (flags >> 4) & 0x0F;
    const int has_v = !a->is_mla_single_buffer;
    size_t req = zo_required_payload(preset, rope_mode, vecs, a->head_dim, a->rope_dim, has_v);
    if (req == (size_t)-1 || plen < req) return 1;

    uint32_t key[8], nonce[3];
    key_words(a->k0, a->k1, a->k2, a->k3, key);
    nonce_words(seq, layer, hg, nonce);
    chacha_xor_words(blob + ZO_HEADER, plain, plen, key, 1u, nonce);

    uint16_t* ko = (uint16_t*)a->out_k + b * elems;
    uint16_t* vo = has_v ? (uint16_t*)a->out_v + b * elems : NULL;
    zo_section secs[3];
    int ns = build_sections(preset, rope_mode, a->head_dim, a->rope_dim, has_v, secs);
    size_t off = 0;
    for (int s = 0; s < ns; ++s) {
        uint16_t* dst = secs[s].src ? vo : ko;
        const int64_t w = secs[s].width, col = secs[s].col;
        if (secs[s].kind == SEC_RAW) {
            for (int64_t r = 0; r < vecs; ++r) {
                memcpy(dst + r * a->head_dim + col, plain + off, (size_t)w * 2u);
                off += (size_t)w * 2u;
            }
            continue;
        }
        const int kind = secs[s].kind, ges = SEC_GES[kind];
        const int64_t groups = w / ges;
        const int bpg = SEC_CB[kind], pb = SEC_PB[kind];
        const uint8_t* qb = plain + off;
        const uint8_t* sb = qb + (size_t)(vecs * groups * bpg);
        for (int64_t r = 0; r < vecs; ++r) {
            for (int64_t g = 0; g < groups; ++g) {
                const int64_t gi = r * groups + g;
                uint16_t prm[2] = {0, 0};
                memcpy(prm, sb + gi * pb, (size_t)pb);
                uint16_t* out = dst + r * a->head_dim + col + g * ges;
                dequant_group_kind(kind, qb + gi * bpg, prm, a->dtype, out);
            }
        }
        off += (size_t)(vecs * groups * (bpg + pb));
    }
    memset(plain, 0, plen);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Batch drivers: contiguous page chunks per thread (cpp:1858-1898).        */
/* ------------------------------------------------------------------------ */

typedef struct {
    const zo_egress_args* e;
    const zo_ingress_args* i;
    int32_t* status;
    int64_t begin, end;
} zo_job;

static void* egress_worker(void* p) {
    zo_job* j = (zo_job*)p;
    uint8_t* plain = (uint8_t*)malloc((size_t)j->e->expected_payload_bytes + 64);
    for (int64_t b = j->begin; b < j->end; ++b) encode_page(j->e, b, plain);
    free(plain);
    return NULL;
}

static void* ingress_worker(void* p) {
    zo_job* j = (zo_job*)p;
    uint8_t* plain = (uint8_t*)malloc((size_t)j->i->blob_bytes + 64);
    for (int64_t b = j->begin; b < j->end; ++b) j->status[b] = decode_page(j->i, b, plain);
    free(plain);
    return NULL;
}

static void run_chunks(int64_t n, int threads, zo_job proto, void* (*fn)(void*)) {
    if (threads > n) threads = (int)n;
    if (threads <= 1) {
        proto.begin = 0;
        proto.end = n;
        fn(&proto);
        return;
    }
    pthread_t* th = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
    zo_job* jobs = (zo_job*)calloc((size_t)threads, sizeof(zo_job));
    const int64_t chunk = (n + threads - 1) / threads;
    int started = 0;
    for (int t = 0; t < threads; ++t) {
        jobs[t] = proto;
        jobs[t].begin = t * chunk;
        jobs[t].end = jobs[t].begin + chunk < n ? jobs[t].begin + chunk : n;
        if (jobs[t].begin >= jobs[t].end) break;
        pthread_create(&th[t], NULL, fn, &jobs[t]);
        started++;
    }
    for (int t = 0; t < started; ++t) pthread_join(th[t], NULL);
    free(jobs);
    free(th);
}

static int geometry_ok(int64_t batch, int64_t T, int64_t H, int64_t D, int64_t R) {
    /* cpp:1925-1957 */
    return batch > 0 && T > 0 && H > 0 && D >= 16 && D % 16 == 0 && R >= 0 && R <= D &&
           R % 16 == 0;
}

int zo_egress_batch(const zo_egress_args* a, int threads) {
    if (!geometry_ok(a->batch, a->num_tokens, a->num_heads, a->head_dim, a->rope_dim)) return -1;
    size_t req = zo_required_payload(a->preset, a->rope_mode, a->num_tokens * a->num_heads,
                                     a->head_dim, a->rope_dim, a->v_pages != NULL);
    if (req == (size_t)-1 || a->expected_payload_bytes < (int64_t)req) return -1;
    zo_job proto = {a, NULL, NULL, 0, 0};
    run_chunks(a->batch, threads, proto, egress_worker);
    return 0;
}

int zo_ingress_batch(const zo_ingress_args* a, int32_t* status, int all_or_nothing,
                     int threads) {
    if (!geometry_ok(a->batch, a->num_tokens, a->num_heads, a->head_dim, a->rope_dim)) return -1;
    if (a->blob_bytes <= (int64_t)(ZO_HEADER + ZO_TAG)) return -1;
    int32_t* st = status ? status : (int32_t*)calloc((size_t)a->batch, sizeof(int32_t));
    zo_job proto = {NULL, a, st, 0, 0};
    run_chunks(a->batch, threads, proto, ingress_worker);
    const int64_t elems = a->num_tokens * a->num_heads * a->head_dim;
    int first = 0;
    for (int64_t b = 0; b < a->batch; ++b) {
        if (st[b] == 0) continue;
        if (!first) first = st[b];
        if (!all_or_nothing) {
            memset((uint16_t*)a->out_k + b * elems, 0, (size_t)elems * 2u);
            if (!a->is_mla_single_buffer)
                memset((uint16_t*)a->out_v + b * elems, 0, (size_t)elems * 2u);
        }
    }
    if (first && all_or_nothing) { /* cpp:2481-2486 */
        memset(a->out_k, 0, (size_t)(a->batch * elems) * 2u);
        if (!a->is_mla_single_buffer) memset(a->out_v, 0, (size_t)(a->batch * elems) * 2u);
    }
    if (!status) free(st);
    return first;
}

/* ------------------------------------------------------------------------ */
/* Array helpers for exhaustive conversion checks.                          */
/* ------------------------------------------------------------------------ */

void zo_f32_to_f16_array(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = zo_f32_to_f16(src[i]);
}
void zo_f32_to_bf16_array(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = zo_f32_to_bf16(src[i]);
}
void zo_f16_to_f32_array(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = zo_f16_to_f32(src[i]);
}
/* n groups of 16 hot elements -> codes (16 or 8 bytes per group) + scales */
void zo_quant_groups(const uint16_t* src, int dtype, int bits, size_t n, uint8_t* q,
                     uint16_t* scales) {
    for (size_t g = 0; g < n; ++g) {
        if (bits == 8)
            zo_quant_group16_int8(src + 16 * g, dtype, q + 16 * g, scales + g);
        else
            zo_quant_group16_int4(src + 16 * g, dtype, q + 8 * g, scales + g);
    }
}
void zo_dequant_groups(const uint8_t* q, const uint16_t* scales, int dtype, int bits,
                       size_t n, uint16_t* dst) {
    for (size_t g = 0; g < n; ++g) {
        if (bits == 8)
            zo_dequant_group16_int8(q + 16 * g, scales[g], dtype, dst + 16 * g);
        else
            zo_dequant_group16_int4(q + 8 * g, scales[g], dtype, dst + 16 * g);
    }
}

/* Extension kinds over n groups (kind 3 = E4M3 / 16 elements, 4 = INT4G32 /
 * 32, 5 = ASYM8 / 64); params holds two u16 per group (scale, zero point). */
int zo_quant_groups_ext(int kind, const uint16_t* src, int dtype, size_t n, uint8_t* q,
                        uint16_t* params) {
    if (kind < SEC_E4M3 || kind > SEC_ASYM8) return -1;
    for (size_t g = 0; g < n; ++g) {
        params[2 * g] = params[2 * g + 1] = 0;
        quant_group_kind(kind, src + (size_t)SEC_GES[kind] * g, dtype, q + (size_t)SEC_CB[kind] * g,
                         params + 2 * g);
    }
    return 0;
}
int zo_dequant_groups_ext(int kind, const uint8_t* q, const uint16_t* params, int dtype, size_t n,
                          uint16_t* dst) {
    if (kind < SEC_E4M3 || kind > SEC_ASYM8) return -1;
    for (size_t g = 0; g < n; ++g)
        dequant_group_kind(kind, q + (size_t)SEC_CB[kind] * g, params + 2 * g, dtype,
                           dst + (size_t)SEC_GES[kind] * g);
    return 0;
}
void zo_f32_to_e4m3_array(const float* src, uint8_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = zo_f32_to_e4m3(src[i]);
}
void zo_e4m3_to_f32_array(const uint8_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = zo_e4m3_to_f32(src[i]);
}
