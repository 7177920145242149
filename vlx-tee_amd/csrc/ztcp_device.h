// ztcp_device.h -- gfx950 device primitives of the cold-page codec:
// RFC 8439 ChaCha20 block, SipHash-2-4-128, fp16/bf16 conversions and the
// group-16 quantizers / dequantizers, bit-exact with the reference's portable
// fp32 path (research/baseline_codec/csrc/fused_cold_page_cpu.cpp, "cpp").
//
// Exactness rules this file relies on (all sources are built with
// -ffp-contract=off, without fast-math, with IEEE mode and fp32 denormals on):
//   * fp32 '/' is correctly rounded (HIP's default), '*' and '+' are IEEE RNE.
//   * (_Float16)x and (__bf16)x are round-to-nearest-even (v_cvt_f16_f32,
//     v_cvt_pk_bf16_f32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ztcp {

constexpr uint32_t kMagic = 0x5A54u;
constexpr uint32_t kVersion = 1u;
constexpr int kHeader = 32;
constexpr int kTag = 16;
constexpr int kHotFp16 = 0;
constexpr int kHotBf16 = 1;

// ---------------------------------------------------------------------------
// ChaCha20 block function, RFC 8439 section 2.3 (cpp:113-189).  State words
// 0..3 constants, 4..11 key, 12 block counter, 13..15 nonce.  One 64-byte
// block per lane; the key stays in scalar registers.
// ---------------------------------------------------------------------------

struct ChaKey {
    uint32_t w[8];
};

__device__ __forceinline__ uint32_t rotl32(uint32_t x, int n) {
    return (x << n) | (x >> (32 - n));
}

#define ZTCP_QR(a, b, c, d)            \
    a += b; d = rotl32(d ^ a, 16);     \
    c += d; b = rotl32(b ^ c, 12);     \
    a += b; d = rotl32(d ^ a, 8);      \
    c += d; b = rotl32(b ^ c, 7);

// Keystream block `ctr` for nonce (n0, n1, n2) into ks[16] (little-endian words).
__device__ __forceinline__ void chacha_block(const ChaKey& key, uint32_t ctr, uint32_t n0,
                                             uint32_t n1, uint32_t n2, uint32_t ks[16]) {
    uint32_t x0 = 0x61707865u, x1 = 0x3320646Eu, x2 = 0x79622D32u, x3 = 0x6B206574u;
    uint32_t x4 = key.w[0], x5 = key.w[1], x6 = key.w[2], x7 = key.w[3];
    uint32_t x8 = key.w[4], x9 = key.w[5], x10 = key.w[6], x11 = key.w[7];
    uint32_t x12 = ctr, x13 = n0, x14 = n1, x15 = n2;
#pragma unroll
    for (int i = 0; i < 10; ++i) {
        ZTCP_QR(x0, x4, x8, x12)
        ZTCP_QR(x1, x5, x9, x13)
        ZTCP_QR(x2, x6, x10, x14)
        ZTCP_QR(x3, x7, x11, x15)
        ZTCP_QR(x0, x5, x10, x15)
        ZTCP_QR(x1, x6, x11, x12)
        ZTCP_QR(x2, x7, x8, x13)
        ZTCP_QR(x3, x4, x9, x14)
    }
    ks[0] = x0 + 0x61707865u;  ks[1] = x1 + 0x3320646Eu;
    ks[2] = x2 + 0x79622D32u;  ks[3] = x3 + 0x6B206574u;
    ks[4] = x4 + key.w[0];     ks[5] = x5 + key.w[1];
    ks[6] = x6 + key.w[2];     ks[7] = x7 + key.w[3];
    ks[8] = x8 + key.w[4];     ks[9] = x9 + key.w[5];
    ks[10] = x10 + key.w[6];   ks[11] = x11 + key.w[7];
    ks[12] = x12 + ctr;        ks[13] = x13 + n0;
    ks[14] = x14 + n1;         ks[15] = x15 + n2;
}

// ---------------------------------------------------------------------------
// SipHash-2-4 with 128-bit output (cpp:401-471).
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint64_t rotl64(uint64_t x, int n) {
    return (x << n) | (x >> (64 - n));
}

struct Sip {
    uint64_t v0, v1, v2, v3;

    __device__ __forceinline__ void init(uint64_t mk0, uint64_t mk1) {
        v0 = 0x736F6D6570736575ull ^ mk0;
        v1 = 0x646F72616E646F6Dull ^ mk1 ^ 0xEEull;
        v2 = 0x6C7967656E657261ull ^ mk0;
        v3 = 0x7465646279746573ull ^ mk1;
    }
    __device__ __forceinline__ void round() {
        v0 += v1; v1 = rotl64(v1, 13); v1 ^= v0; v0 = rotl64(v0, 32);
        v2 += v3; v3 = rotl64(v3, 16); v3 ^= v2;
        v0 += v3; v3 = rotl64(v3, 21); v3 ^= v0;
        v2 += v1; v1 = rotl64(v1, 17); v1 ^= v2; v2 = rotl64(v2, 32);
    }
    __device__ __forceinline__ void absorb(uint64_t m) {
        v3 ^= m;
        round();
        round();
        v0 ^= m;
    }
    // Final word = (total_len & 0xff) << 56 | tail bytes (cpp:458-470), then
    // the 128-bit finalization (cpp:447-456).
    __device__ __forceinline__ void finish(uint64_t last_word, uint64_t& lo, uint64_t& hi) {
        absorb(last_word);
        v2 ^= 0xEEull;
        round(); round(); round(); round();
        lo = v0 ^ v1 ^ v2 ^ v3;
        v1 ^= 0xDDull;
        round(); round(); round(); round();
        hi = v0 ^ v1 ^ v2 ^ v3;
    }
};

__device__ __forceinline__ uint64_t lo64(uint4 a) { return (uint64_t)a.x | ((uint64_t)a.y << 32); }
__device__ __forceinline__ uint64_t hi64(uint4 a) { return (uint64_t)a.z | ((uint64_t)a.w << 32); }

// ---------------------------------------------------------------------------
// Hot dtype conversions.
// ---------------------------------------------------------------------------

__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
__device__ __forceinline__ uint32_t f32_to_f16(float f) {  // RNE
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {  // RNE
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

template <int DT>
__device__ __forceinline__ float hot_lo(uint32_t w) {  // element in bits 0..15
    if constexpr (DT == kHotBf16) return __uint_as_float(w << 16);
    else return f16_to_f32(w & 0xFFFFu);
}
template <int DT>
__device__ __forceinline__ float hot_hi(uint32_t w) {  // element in bits 16..31
    if constexpr (DT == kHotBf16) return __uint_as_float(w & 0xFFFF0000u);
    else return f16_to_f32(w >> 16);
}
// Two fp32 values -> packed hot pair (lo in bits 0..15), RNE.
template <int DT>
__device__ __forceinline__ uint32_t pack_hot(float lo, float hi) {
    if constexpr (DT == kHotBf16) return f32_to_bf16(lo) | (f32_to_bf16(hi) << 16);
    else return f32_to_f16(lo) | (f32_to_f16(hi) << 16);
}

// ---------------------------------------------------------------------------
// Group-16 quantizers, profile S of the reference:
//   int8 (cpp:735-753): amax = max(1e-6, max|v|); s = fp16(amax / 127);
//        inv = 1 / f32(s); q = clamp(nearbyintf(v * inv), -127, 127)
//   int4 (cpp:806-824): s = fp16(amax / 7);
//        q = clamp(int(nearbyintf(v * inv) + 8), 0, 15); byte i = q[2i] | q[2i+1] << 4
// Input: a group as 8 words (element 2i in the low half of word i).
//
// Fast path: for finite inputs and a nonzero scale, |v * inv| is bounded
// (<= 190), so clamp-then-round equals round-then-clamp, and adding 1.5*2^23
// (+8 for int4) rounds to nearest-even in the same fp32 add: the low bits of
// the sum are the code.  Groups holding NaN / inf, or an int8 scale that
// underflows to 0 (amax <= 3.79e-6), take the exact emulation of the x86
// conversions instead (NaN -> 0 after the int conversion).
// ---------------------------------------------------------------------------

template <int DT>
__device__ __forceinline__ uint32_t group_amax_bits(const uint32_t w[8]) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    u16x2 m = __builtin_bit_cast(u16x2, w[0] & 0x7FFF7FFFu);
#pragma unroll
    for (int i = 1; i < 8; ++i)
        m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[i] & 0x7FFF7FFFu));
    return m.x > m.y ? m.x : m.y;
}

template <int DT>
__device__ __forceinline__ float bits_to_f32(uint32_t b) {
    if constexpr (DT == kHotBf16) return __uint_as_float(b << 16);
    else return f16_to_f32(b);
}

// Scale bits and reciprocal for a group; returns true for the exact path.
template <int DT, int BITS>
__device__ __forceinline__ bool group_scale(const uint32_t w[8], uint32_t& scale_bits,
                                            float& inv) {
    const uint32_t ab = group_amax_bits<DT>(w);
    const uint32_t inf_bits = DT == kHotBf16 ? 0x7F80u : 0x7C00u;
    const float amax_v = bits_to_f32<DT>(ab);
    const float amax = amax_v > 1e-6f ? amax_v : 1e-6f;
    scale_bits = f32_to_f16(amax / (BITS == 8 ? 127.0f : 7.0f));
    inv = 1.0f / f16_to_f32(scale_bits);
    return ab >= inf_bits || scale_bits == 0;
}

// Exact amax for groups that hold NaN (the reference skips NaN: `av > amax`).
template <int DT, int BITS>
__device__ __noinline__ void group_scale_exact(const uint32_t w[8], uint32_t& scale_bits,
                                               float& inv) {
    float amax = 1e-6f;
    for (int i = 0; i < 8; ++i) {
        float a = fabsf(hot_lo<DT>(w[i]));
        float b = fabsf(hot_hi<DT>(w[i]));
        if (a > amax) amax = a;
        if (b > amax) amax = b;
    }
    scale_bits = f32_to_f16(amax / (BITS == 8 ? 127.0f : 7.0f));
    inv = 1.0f / f16_to_f32(scale_bits);
}

__device__ __forceinline__ uint32_t code8_exact(float y) {
    float r = rintf(y);
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    return r != r ? 0u : ((uint32_t)(int)r & 0xFFu);
}
__device__ __forceinline__ uint32_t code4_exact(float y) {
    float r = rintf(y) + 8.0f;
    int u = r != r ? INT32_MIN : (int)r;
    u = u < 0 ? 0 : (u > 15 ? 15 : u);
    return (uint32_t)u;
}

// Pack byte 0 of four words into one word.
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0C0C0400u);
    const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x0C0C0400u);
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// int8: 16 elements -> 4 code words; returns the fp16 scale bits.
template <int DT>
__device__ __forceinline__ uint32_t quant_group_int8(const uint32_t w[8], uint32_t q[4]) {
    uint32_t sb;
    float inv;
    if (!group_scale<DT, 8>(w, sb, inv)) {
        uint32_t t[16];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float a = __builtin_amdgcn_fmed3f(hot_lo<DT>(w[i]) * inv, -127.0f, 127.0f);
            float b = __builtin_amdgcn_fmed3f(hot_hi<DT>(w[i]) * inv, -127.0f, 127.0f);
            t[2 * i] = __float_as_uint(a + 12582912.0f);
            t[2 * i + 1] = __float_as_uint(b + 12582912.0f);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) q[j] = pack_low_bytes(t[4 * j], t[4 * j + 1], t[4 * j + 2], t[4 * j + 3]);
        return sb;
    }
    group_scale_exact<DT, 8>(w, sb, inv);
    for (int j = 0; j < 4; ++j) {
        uint32_t c0 = code8_exact(hot_lo<DT>(w[2 * j]) * inv);
        uint32_t c1 = code8_exact(hot_hi<DT>(w[2 * j]) * inv);
        uint32_t c2 = code8_exact(hot_lo<DT>(w[2 * j + 1]) * inv);
        uint32_t c3 = code8_exact(hot_hi<DT>(w[2 * j + 1]) * inv);
        q[j] = c0 | (c1 << 8) | (c2 << 16) | (c3 << 24);
    }
    return sb;
}

// int4: 16 elements -> 2 code words; returns the fp16 scale bits.
template <int DT>
__device__ __forceinline__ uint32_t quant_group_int4(const uint32_t w[8], uint32_t q[2]) {
    uint32_t sb;
    float inv;
    if (!group_scale<DT, 4>(w, sb, inv)) {
        uint32_t b[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float lo = __builtin_amdgcn_fmed3f(hot_lo<DT>(w[i]) * inv, -8.0f, 7.0f);
            float hi = __builtin_amdgcn_fmed3f(hot_hi<DT>(w[i]) * inv, -8.0f, 7.0f);
            // bits 0..3 of each sum hold q + 8; bits 4..7 are zero.
            b[i] = (__float_as_uint(hi + 12582920.0f) << 4) | __float_as_uint(lo + 12582920.0f);
        }
        q[0] = pack_low_bytes(b[0], b[1], b[2], b[3]);
        q[1] = pack_low_bytes(b[4], b[5], b[6], b[7]);
        return sb;
    }
    group_scale_exact<DT, 4>(w, sb, inv);
    for (int j = 0; j < 2; ++j) {
        uint32_t word = 0;
        for (int i = 0; i < 4; ++i) {
            uint32_t e = w[4 * j + i];
            uint32_t lo = code4_exact(hot_lo<DT>(e) * inv);
            uint32_t hi = code4_exact(hot_hi<DT>(e) * inv);
            word |= (lo | (hi << 4)) << (8 * i);
        }
        q[j] = word;
    }
    return sb;
}

// ---------------------------------------------------------------------------
// Dequantizers (cpp:772-776, cpp:846-853): out = hot(f32(q) * f32(s)).  The
// product is exact in fp32 (|q| <= 128, s has 11 significant bits), so the
// only rounding is the final RNE conversion.
// ---------------------------------------------------------------------------

// 16 int8 codes (4 words) -> 8 packed hot words.
template <int DT>
__device__ __forceinline__ void dequant_group_int8(const uint32_t q[4], uint32_t scale_bits,
                                                   uint32_t out[8]) {
    const float s = f16_to_f32(scale_bits & 0xFFFFu);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int32_t w = (int32_t)q[j];
        float e0 = (float)((w << 24) >> 24) * s;
        float e1 = (float)((w << 16) >> 24) * s;
        float e2 = (float)((w << 8) >> 24) * s;
        float e3 = (float)(w >> 24) * s;
        out[2 * j] = pack_hot<DT>(e0, e1);
        out[2 * j + 1] = pack_hot<DT>(e2, e3);
    }
}

// 16 int4 codes (2 words) -> 8 packed hot words.
template <int DT>
__device__ __forceinline__ void dequant_group_int4(const uint32_t q[2], uint32_t scale_bits,
                                                   uint32_t out[8]) {
    const float s = f16_to_f32(scale_bits & 0xFFFFu);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t lo = q[j] & 0x0F0F0F0Fu;         // elements 0,2,4,6 of the word
        const uint32_t hi = (q[j] >> 4) & 0x0F0F0F0Fu;  // elements 1,3,5,7
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float a = ((float)((lo >> (8 * i)) & 0xFFu) - 8.0f) * s;
            float b = ((float)((hi >> (8 * i)) & 0xFFu) - 8.0f) * s;
            out[4 * j + i] = pack_hot<DT>(a, b);
        }
    }
}

}  // namespace ztcp
