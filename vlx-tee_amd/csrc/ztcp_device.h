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

// The first column round touches the block counter only in its first
// quarter round (x0, x4, x8, x12).  For one page -- fixed key and nonce --
// the other three quarter rounds give the same twelve words for every block,
// so a lane computes them once per page and starts every block from there;
// with a wave-uniform counter the remaining quarter round runs on the scalar
// unit.  This removes three of the 80 quarter rounds from each block's VALU
// work.
struct ChaChaNonceCache {
    uint32_t c[12];  // x1, x5, x9, x13, x2, x6, x10, x14, x3, x7, x11, x15 after column round 1

    __device__ __forceinline__ void init(const ChaKey& key, uint32_t n0, uint32_t n1, uint32_t n2) {
        uint32_t x1 = 0x3320646Eu, x5 = key.w[1], x9 = key.w[5], x13 = n0;
        uint32_t x2 = 0x79622D32u, x6 = key.w[2], x10 = key.w[6], x14 = n1;
        uint32_t x3 = 0x6B206574u, x7 = key.w[3], x11 = key.w[7], x15 = n2;
        ZTCP_QR(x1, x5, x9, x13)
        ZTCP_QR(x2, x6, x10, x14)
        ZTCP_QR(x3, x7, x11, x15)
        c[0] = x1; c[1] = x5; c[2] = x9; c[3] = x13;
        c[4] = x2; c[5] = x6; c[6] = x10; c[7] = x14;
        c[8] = x3; c[9] = x7; c[10] = x11; c[11] = x15;
    }
};

// The same block function split in two, so that a caller can interleave
// other work (loads, quantization) between the halves of the 10 double rounds.
struct ChaChaState {
    uint32_t x[16];

    __device__ __forceinline__ void start(const ChaKey& key, uint32_t ctr, uint32_t n0, uint32_t n1,
                                          uint32_t n2) {
        x[0] = 0x61707865u; x[1] = 0x3320646Eu; x[2] = 0x79622D32u; x[3] = 0x6B206574u;
#pragma unroll
        for (int i = 0; i < 8; ++i) x[4 + i] = key.w[i];
        x[12] = ctr; x[13] = n0; x[14] = n1; x[15] = n2;
    }
    // start() followed by the first double round, the column round taken
    // from the page's cache.
    __device__ __forceinline__ void start_cached(const ChaKey& key, const ChaChaNonceCache& nc, uint32_t ctr) {
        x[0] = 0x61707865u; x[4] = key.w[0]; x[8] = key.w[4]; x[12] = ctr;
        ZTCP_QR(x[0], x[4], x[8], x[12])
        x[1] = nc.c[0]; x[5] = nc.c[1]; x[9] = nc.c[2];  x[13] = nc.c[3];
        x[2] = nc.c[4]; x[6] = nc.c[5]; x[10] = nc.c[6]; x[14] = nc.c[7];
        x[3] = nc.c[8]; x[7] = nc.c[9]; x[11] = nc.c[10]; x[15] = nc.c[11];
        ZTCP_QR(x[0], x[5], x[10], x[15])
        ZTCP_QR(x[1], x[6], x[11], x[12])
        ZTCP_QR(x[2], x[7], x[8], x[13])
        ZTCP_QR(x[3], x[4], x[9], x[14])
    }
    template <int N>
    __device__ __forceinline__ void double_rounds() {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            ZTCP_QR(x[0], x[4], x[8], x[12])
            ZTCP_QR(x[1], x[5], x[9], x[13])
            ZTCP_QR(x[2], x[6], x[10], x[14])
            ZTCP_QR(x[3], x[7], x[11], x[15])
            ZTCP_QR(x[0], x[5], x[10], x[15])
            ZTCP_QR(x[1], x[6], x[11], x[12])
            ZTCP_QR(x[2], x[7], x[8], x[13])
            ZTCP_QR(x[3], x[4], x[9], x[14])
        }
    }
    // Feed-forward (RFC 8439 2.3): ks = rounds(state) + state.
    __device__ __forceinline__ void finish(const ChaKey& key, uint32_t ctr, uint32_t n0, uint32_t n1,
                                           uint32_t n2, uint32_t ks[16]) const {
        ks[0] = x[0] + 0x61707865u;  ks[1] = x[1] + 0x3320646Eu;
        ks[2] = x[2] + 0x79622D32u;  ks[3] = x[3] + 0x6B206574u;
#pragma unroll
        for (int i = 0; i < 8; ++i) ks[4 + i] = x[4 + i] + key.w[i];
        ks[12] = x[12] + ctr; ks[13] = x[13] + n0;
        ks[14] = x[14] + n1;  ks[15] = x[15] + n2;
    }
};

// Keystream block `ctr` of a page whose first column round is cached.
__device__ __forceinline__ void chacha_block_cached(const ChaKey& key, const ChaChaNonceCache& nc, uint32_t ctr,
                                                    uint32_t n0, uint32_t n1, uint32_t n2, uint32_t ks[16]) {
    ChaChaState st;
    st.start_cached(key, nc, ctr);
    st.double_rounds<9>();
    st.finish(key, ctr, n0, n1, n2, ks);
}

// ---------------------------------------------------------------------------
// SipHash-2-4 with 128-bit output (cpp:401-471).
// One page per lane; the chain is strictly sequential, so its cost is the
// number of VALU issues per 8-byte word.  gfx950 forms used:
//   * 64-bit add          -> v_lshl_add_u64 (shift 0);
//   * rotate by n < 32    -> two v_alignbit_b32 on the 32-bit halves;
//   * rotate by 32        -> never executed: v0's rotation is folded into the
//                            add that follows it (v_add_co_u32 +
//                            v_addc_co_u32 on exchanged halves), and v2 is
//                            kept rotated by 32 between rounds, so the add
//                            that opens the next round reads it the same way;
//   * the next word's "v3 ^= m" is folded into the previous round's last
//     "v3 ^= v0" as a three-input xor (v_bitop3_b32, truth table 0x96).
// Measured on a lone wave: ~206 shader clocks per word (~212 with an
// explicit v_pk_mov_b32 exchange for each rotation by 32).
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint64_t add_u64(uint64_t a, uint64_t b) {
    uint64_t r;
    asm("v_lshl_add_u64 %0, %1, 0, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
// rotl(a, 32) + b, with the rotation done by reading a's halves exchanged.
// The carry goes through VCC in one asm block: with the carry in an SGPR
// pair the compiler put a wait state (s_nop) between the two halves, a few
// hundred per workgroup's chain.
__device__ __forceinline__ uint64_t add_rot32_u64(uint64_t a, uint64_t b) {
    uint32_t lo, hi;
    asm("v_add_co_u32_e32 %0, vcc, %2, %3\n\tv_addc_co_u32_e32 %1, vcc, %4, %5, vcc"
        : "=&v"(lo), "=v"(hi)
        : "v"((uint32_t)(a >> 32)), "v"((uint32_t)b), "v"((uint32_t)a), "v"((uint32_t)(b >> 32))
        : "vcc");
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t rot32_u64(uint64_t a) { return (a << 32) | (a >> 32); }
__device__ __forceinline__ uint32_t xor3_u32(uint32_t a, uint32_t b, uint32_t c) {
    uint32_t r;
    asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0x96" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
__device__ __forceinline__ uint64_t rotl_u64(uint64_t x, int n) {  // 0 < n < 32
    const uint32_t lo = (uint32_t)x, hi = (uint32_t)(x >> 32);
    const uint32_t nl = __builtin_amdgcn_alignbit(lo, hi, 32 - n);
    const uint32_t nh = __builtin_amdgcn_alignbit(hi, lo, 32 - n);
    return ((uint64_t)nh << 32) | nl;
}
__device__ __forceinline__ uint64_t xor3_u64(uint64_t a, uint64_t b, uint64_t c) {
    return ((uint64_t)xor3_u32((uint32_t)(a >> 32), (uint32_t)(b >> 32), (uint32_t)(c >> 32)) << 32) |
           xor3_u32((uint32_t)a, (uint32_t)b, (uint32_t)c);
}

struct Sip {
    // v2r holds rotl(v2, 32): SipRound ends with v2 = rotl(v2, 32), and
    // keeping it that way lets the next round's "v2 += v3" read the halves
    // exchanged instead of moving them.
    uint64_t v0, v1, v2r, v3;

    __device__ __forceinline__ void init(uint64_t mk0, uint64_t mk1) {
        v0 = 0x736F6D6570736575ull ^ mk0;
        v1 = 0x646F72616E646F6Dull ^ mk1 ^ 0xEEull;
        v2r = rot32_u64(0x6C7967656E657261ull ^ mk0);
        v3 = 0x7465646279746573ull ^ mk1;
    }
    // SipRound (cpp:401-416); with INJ the final v3 also takes "^ next", the
    // next message word's v3 injection.
    template <bool INJ>
    __device__ __forceinline__ void round_(uint64_t next) {
        v0 = add_u64(v0, v1);
        uint64_t v2 = add_rot32_u64(v2r, v3);  // v2 += v3
        v1 = rotl_u64(v1, 13) ^ v0;
        v3 = rotl_u64(v3, 16) ^ v2;
        v0 = add_rot32_u64(v0, v3);            // v0 = rotl(v0, 32) + v3
        v2 = add_u64(v2, v1);
        v3 = INJ ? xor3_u64(rotl_u64(v3, 21), v0, next) : (rotl_u64(v3, 21) ^ v0);
        v1 = rotl_u64(v1, 17) ^ v2;
        v2r = v2;                              // v2 = rotl(v2, 32), held rotated
    }
    __device__ __forceinline__ void round() { round_<false>(0); }
    // Compression of one word whose "v3 ^= m" was already applied; the next
    // word's injection is fused into the second round.
    __device__ __forceinline__ void compress_then_inject(uint64_t m, uint64_t next) {
        round_<false>(0);
        round_<true>(next);
        v0 ^= m;
    }
    __device__ __forceinline__ void absorb(uint64_t m) {
        v3 ^= m;
        round();
        round();
        v0 ^= m;
    }
    __device__ __forceinline__ void absorb(uint32_t mlo, uint32_t mhi) {
        absorb((uint64_t)mlo | ((uint64_t)mhi << 32));
    }
    // n consecutive words w[0..n-1]: one injection xor per chunk instead of
    // one per word.
    template <int N>
    __device__ __forceinline__ void absorb_words(const uint64_t (&w)[N]) {
        v3 ^= w[0];
#pragma unroll
        for (int i = 0; i + 1 < N; ++i) compress_then_inject(w[i], w[i + 1]);
        round();
        round();
        v0 ^= w[N - 1];
    }
    __device__ __forceinline__ void absorb(uint4 q) {  // two little-endian words
        const uint64_t w[2] = {(uint64_t)q.x | ((uint64_t)q.y << 32), (uint64_t)q.z | ((uint64_t)q.w << 32)};
        absorb_words<2>(w);
    }
    __device__ __forceinline__ void absorb64(const uint4 (&c)[4]) {  // eight words
        uint64_t w[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[2 * i] = (uint64_t)c[i].x | ((uint64_t)c[i].y << 32);
            w[2 * i + 1] = (uint64_t)c[i].z | ((uint64_t)c[i].w << 32);
        }
        absorb_words<8>(w);
    }
    // absorb64 with after_word(i) called after word i (i = 0..7), so that a
    // caller can spread other work (memory instructions) over the chain.
    template <class F>
    __device__ __forceinline__ void absorb64_with(const uint4 (&c)[4], F&& after_word) {
        uint64_t w[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[2 * i] = (uint64_t)c[i].x | ((uint64_t)c[i].y << 32);
            w[2 * i + 1] = (uint64_t)c[i].z | ((uint64_t)c[i].w << 32);
        }
        v3 ^= w[0];
#pragma unroll
        for (int i = 0; i < 7; ++i) {
            compress_then_inject(w[i], w[i + 1]);
            after_word(i);
        }
        round();
        round();
        v0 ^= w[7];
        after_word(7);
    }
    // Final word = (total_len & 0xff) << 56 | tail bytes (cpp:458-470), then
    // the 128-bit finalization (cpp:447-456).
    __device__ __forceinline__ void finish(uint64_t last_word, uint64_t& lo, uint64_t& hi) {
        absorb(last_word);
        v2r ^= 0xEEull << 32;  // v2 ^= 0xee
        round(); round(); round(); round();
        lo = v0 ^ v1 ^ rot32_u64(v2r) ^ v3;
        v1 ^= 0xDDull;
        round(); round(); round(); round();
        hi = v0 ^ v1 ^ rot32_u64(v2r) ^ v3;
    }
};

// Absorbs `total` consecutive 64-byte chunks delivered by fetch(uint4[4]),
// with the loads of two chunks in flight ahead of the one being absorbed.
template <class F>
__device__ __forceinline__ void sip_stream64(Sip& s, uint32_t total, F&& fetch) {
    uint4 x0[4], x1[4], x2[4];
    if (total > 0u) fetch(x0);
    if (total > 1u) fetch(x1);
#pragma unroll 1
    for (uint32_t c = 0; c < total; c += 3u) {
        if (c + 2u < total) fetch(x2);
        s.absorb64(x0);
        if (c + 1u >= total) break;
        if (c + 3u < total) fetch(x0);
        s.absorb64(x1);
        if (c + 2u >= total) break;
        if (c + 4u < total) fetch(x1);
        s.absorb64(x2);
    }
}

__device__ __forceinline__ uint64_t lo64(uint4 a) { return (uint64_t)a.x | ((uint64_t)a.y << 32); }
__device__ __forceinline__ uint64_t hi64(uint4 a) { return (uint64_t)a.z | ((uint64_t)a.w << 32); }

// 16-byte global loads and stores through global-address-space pointers:
// they stay on the global_* path (in-order vmcnt accounting, so a prefetched
// load is not waited for together with newer ones) instead of flat_*.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) u32x4* gptr_ro;
typedef __attribute__((address_space(1))) u32x4* gptr_rw;

__device__ __forceinline__ uint4 ldg16(const void* p, int64_t i = 0) {
    const u32x4 v = ((gptr_ro)p)[i];
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void stg16(void* p, int64_t i, uint4 x) {
    ((gptr_rw)p)[i] = u32x4{x.x, x.y, x.z, x.w};
}

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
// Two fp32 values -> packed hot pair (lo in bits 0..15), RNE.  The bf16 pair
// goes through one two-wide conversion (a single v_cvt_pk_bf16_f32); two
// scalar conversions cost a conversion, a shift and an or per element.
typedef float ztcp_float2 __attribute__((ext_vector_type(2)));
typedef __bf16 ztcp_bf16x2 __attribute__((ext_vector_type(2)));
template <int DT>
__device__ __forceinline__ uint32_t pack_hot(float lo, float hi) {
    if constexpr (DT == kHotBf16) {
        const ztcp_float2 f = {lo, hi};
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, ztcp_bf16x2));
    } else {
        return f32_to_f16(lo) | (f32_to_f16(hi) << 16);
    }
}

// ---------------------------------------------------------------------------
// Group-16 quantizers, profile S of the reference:
//   int8 (cpp:735-753): amax = max(1e-6, max|v|); s = fp16(amax / 127);
//        inv = 1 / f32(s); q = clamp(nearbyintf(v * inv), -127, 127)
//   int4 (cpp:806-824): s = fp16(amax / 7);
//        q = clamp(int(nearbyintf(v * inv) + 8), 0, 15); byte i = q[2i] | q[2i+1] << 4
// Input: a group as 8 words (element 2i in the low half of word i).
//
// Fast path (every group whose scale is a normal fp16 number and whose
// elements are finite):
//   * s is computed as q0 = amax * (1/C), q = fma(fma(-q0, C, amax), 1/C, q0)
//     (a corrected quotient) and inv as a Newton-refined v_rcp_f32.  Both are
//     checked exhaustively against correctly rounded division
//     (ztcp_selftest): the reciprocal equals 1/s for every positive finite
//     fp16 s, and fp16(q) equals fp16(amax / C) for every amax the fp16 and
//     bf16 hot dtypes can produce whenever the result is a normal fp16 value.
//   * with a normal s, |v * inv| <= C * (1 + 2^-10) < C + 0.5, so no clamp is
//     needed, and adding 1.5 * 2^23 (+8 for int4) rounds to nearest-even in
//     that same fp32 add: the low bits of the sum are the code.
// Every other group (NaN / inf elements, a zero, subnormal or infinite
// scale) takes the exact emulation: IEEE division and the x86 conversions
// (NaN -> 0 after the int conversion), identical to the reference.
// ---------------------------------------------------------------------------

struct GroupCodes {
    uint32_t q0, q1, q2, q3;  // code words (int4 uses q0, q1)
    uint32_t scale;           // fp16 scale bits
};

// Exact emulation of the reference for one group.  Inlined (in a cold block
// at each use): a call would make the caller save registers to scratch
// around it, and scratch reloads count as memory operations in flight where
// the rare path joins the fast one, which makes the compiler wait for every
// outstanding load and store there.
template <int DT, int BITS>
__device__ __forceinline__ GroupCodes quant_group_exact(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                                     uint32_t w4, uint32_t w5, uint32_t w6, uint32_t w7) {
    const uint32_t w[8] = {w0, w1, w2, w3, w4, w5, w6, w7};
    float amax = 1e-6f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float a = fabsf(hot_lo<DT>(w[i]));
        const float b = fabsf(hot_hi<DT>(w[i]));
        if (a > amax) amax = a;
        if (b > amax) amax = b;
    }
    GroupCodes r;
    r.scale = f32_to_f16(amax / (BITS == 8 ? 127.0f : 7.0f));
    const float inv = 1.0f / f16_to_f32(r.scale);
    uint32_t q[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < (BITS == 8 ? 4 : 2); ++j) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (BITS == 8) {
                const uint32_t e = w[2 * j + (i >> 1)];
                const float v = (i & 1) ? hot_hi<DT>(e) : hot_lo<DT>(e);
                float rr = rintf(v * inv);
                if (rr < -127.0f) rr = -127.0f;
                if (rr > 127.0f) rr = 127.0f;
                const uint32_t c = rr != rr ? 0u : ((uint32_t)(int)rr & 0xFFu);
                word |= c << (8 * i);
            } else {
                const uint32_t e = w[4 * j + i];
                uint32_t nib[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float v = h ? hot_hi<DT>(e) : hot_lo<DT>(e);
                    const float rr = rintf(v * inv) + 8.0f;
                    int u = rr != rr ? INT32_MIN : (int)rr;
                    nib[h] = (uint32_t)(u < 0 ? 0 : (u > 15 ? 15 : u));
                }
                word |= (nib[0] | (nib[1] << 4)) << (8 * i);
            }
        }
        q[j] = word;
    }
    r.q0 = q[0]; r.q1 = q[1]; r.q2 = q[2]; r.q3 = q[3];
    return r;
}

// amax / C in fp32 for the fast paths: a corrected quotient (see above), one
// fp32 rounding.
template <int CI>
__device__ __forceinline__ float quotient_fast(float amax) {
    constexpr float C = (float)CI;
    constexpr float rC = 1.0f / (float)CI;
    const float q0 = amax * rC;
    const float r = __builtin_fmaf(-q0, C, amax);
    return __builtin_fmaf(r, rC, q0);
}

// The int8 / int4 scale fp16(amax / C), C = 127 / 7; valid when the result is
// normal.  The compiler folds the last fma and the fp16 conversion into one
// mixed-precision instruction, which rounds once from the exact value where
// the reference rounds to fp32 first; ztcp_selftest shows the two agree for
// every amax of both hot dtypes whenever the result is a normal fp16 value
// (the quantizers send every other scale to their exact path).
template <int BITS>
__device__ __forceinline__ uint32_t scale_fast(float amax) {
    return f32_to_f16(quotient_fast<BITS == 8 ? 127 : 7>(amax));
}

// The e4m3 scale fp16(amax / 448) for every amax >= 1e-6: the quotient equals
// the IEEE one for every amax of both hot dtypes, and the empty asm keeps its
// fp32 rounding, so fp16 subnormal results round as the reference's do
// (ztcp_selftest checks every amax).
__device__ __forceinline__ uint32_t scale_e4m3(float amax) {
    float q = quotient_fast<448>(amax);
    asm volatile("" : "+v"(q));
    return f32_to_f16(q);
}

// 1 / s for a positive finite fp16 value s: Newton-refined v_rcp_f32.
__device__ __forceinline__ float recip_fast(float s) {
    const float r0 = __builtin_amdgcn_rcpf(s);
    const float e = __builtin_fmaf(-s, r0, 1.0f);
    return __builtin_fmaf(e, r0, r0);
}

// Pack byte 0 of four words into one word.
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0C0C0400u);
    const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x0C0C0400u);
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// The 16 elements of a group as fp32 (element 2i from the low half of word i).
template <int DT>
__device__ __forceinline__ void hot_floats(const uint32_t w[8], float f[16]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        f[2 * i] = hot_lo<DT>(w[i]);
        f[2 * i + 1] = hot_hi<DT>(w[i]);
    }
}

// max(1e-6, max |f|) by v_max3.  It equals the reference's compare loop
// whenever the result is finite: a NaN element is either skipped, as the
// compare loop skips it, or makes the result NaN, which sends the group to
// the caller's exact path.  (The int8 and int4 fast paths then still write
// the reference's code 0 for a skipped NaN element: the low bits of a NaN
// sum are zero.)
__device__ __forceinline__ float amax16(const float f[16]) {
    float m0 = __builtin_fmaxf(__builtin_fmaxf(fabsf(f[0]), fabsf(f[1])), fabsf(f[2]));
    float m1 = __builtin_fmaxf(__builtin_fmaxf(fabsf(f[3]), fabsf(f[4])), fabsf(f[5]));
    float m2 = __builtin_fmaxf(__builtin_fmaxf(fabsf(f[6]), fabsf(f[7])), fabsf(f[8]));
    float m3 = __builtin_fmaxf(__builtin_fmaxf(fabsf(f[9]), fabsf(f[10])), fabsf(f[11]));
    float m4 = __builtin_fmaxf(__builtin_fmaxf(fabsf(f[12]), fabsf(f[13])), fabsf(f[14]));
    m0 = __builtin_fmaxf(__builtin_fmaxf(m0, m1), m2);
    m3 = __builtin_fmaxf(__builtin_fmaxf(m3, m4), fabsf(f[15]));
    return __builtin_fmaxf(__builtin_fmaxf(m0, m3), 1e-6f);
}

// int4 codes of 16 elements with a normal scale: with |v * inv| <= 7 * (1 +
// 2^-10) < 7.5 no clamp is needed, and adding 1.5 * 2^23 + 8 rounds to
// nearest even in that fp32 add; bits 0..3 of each sum hold q + 8 and bits
// 4..7 are zero.  Element 2i goes to the low nibble of byte i.
__device__ __forceinline__ void int4_codes_fast(const float f[16], float inv, uint32_t& q0, uint32_t& q1) {
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        b[i] = (__float_as_uint(f[2 * i + 1] * inv + 12582920.0f) << 4) | __float_as_uint(f[2 * i] * inv + 12582920.0f);
    q0 = pack_low_bytes(b[0], b[1], b[2], b[3]);
    q1 = pack_low_bytes(b[4], b[5], b[6], b[7]);
}

// One group: code words (4 for int8, 2 for int4, the rest zero) and the fp16
// scale bits, returned by value from both paths so that the caller's
// registers never go through memory.
template <int DT, int BITS>
__device__ __forceinline__ GroupCodes quant_group_codes(const uint32_t w[8]) {
    float f[16];
    hot_floats<DT>(w, f);
    const float amax = amax16(f);
    const uint32_t sb = scale_fast<BITS>(amax);
    // exact path: NaN / inf elements (amax not < inf), scale zero / subnormal / inf
    const bool special = !(amax < __builtin_inff()) || (sb - 0x0400u) >= (0x7C00u - 0x0400u);
    if (__builtin_expect(special, 0))
        return quant_group_exact<DT, BITS>(w[0], w[1], w[2], w[3], w[4], w[5], w[6], w[7]);
    const float inv = recip_fast(f16_to_f32(sb));
    GroupCodes r;
    r.scale = sb;
    if constexpr (BITS == 8) {
        uint32_t t[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) t[i] = __float_as_uint(f[i] * inv + 12582912.0f);
        r.q0 = pack_low_bytes(t[0], t[1], t[2], t[3]);
        r.q1 = pack_low_bytes(t[4], t[5], t[6], t[7]);
        r.q2 = pack_low_bytes(t[8], t[9], t[10], t[11]);
        r.q3 = pack_low_bytes(t[12], t[13], t[14], t[15]);
    } else {
        int4_codes_fast(f, inv, r.q0, r.q1);
        r.q2 = 0u;
        r.q3 = 0u;
    }
    return r;
}

// Array form: q[0..3] (int4 fills q[0], q[1]); returns the fp16 scale bits.
template <int DT, int BITS>
__device__ __forceinline__ uint32_t quant_group(const uint32_t w[8], uint32_t q[4]) {
    const GroupCodes r = quant_group_codes<DT, BITS>(w);
    q[0] = r.q0; q[1] = r.q1; q[2] = r.q2; q[3] = r.q3;
    return r.scale;
}

template <int DT>
__device__ __forceinline__ uint32_t quant_group_int8(const uint32_t w[8], uint32_t q[4]) {
    return quant_group<DT, 8>(w, q);
}
template <int DT>
__device__ __forceinline__ uint32_t quant_group_int4(const uint32_t w[8], uint32_t q[2]) {
    uint32_t t[4];
    const uint32_t sb = quant_group<DT, 4>(w, t);
    q[0] = t[0];
    q[1] = t[1];
    return sb;
}

// ---------------------------------------------------------------------------
// Dequantizers (cpp:772-776, cpp:846-853): out = hot(f32(q) * f32(s)).  The
// product is exact in fp32 (|q| <= 128, s has 11 significant bits), so the
// only rounding is the final RNE conversion.
// ---------------------------------------------------------------------------

// NaN outputs as the reference's conversions write them (c10::BFloat16:
// every NaN is 0x7FC0; c10::Half: sign | 0x7E00); the hardware conversions
// keep other payloads and, for bf16, the sign.
template <int DT>
__device__ __forceinline__ void canonical_nans(uint32_t out[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t lo = out[i] & 0xFFFFu, hi = out[i] >> 16;
        if constexpr (DT == kHotBf16) {
            lo = (lo & 0x7FFFu) > 0x7F80u ? 0x7FC0u : lo;
            hi = (hi & 0x7FFFu) > 0x7F80u ? 0x7FC0u : hi;
        } else {
            lo = (lo & 0x7FFFu) > 0x7C00u ? ((lo & 0x8000u) | 0x7E00u) : lo;
            hi = (hi & 0x7FFFu) > 0x7C00u ? ((hi & 0x8000u) | 0x7E00u) : hi;
        }
        out[i] = lo | (hi << 16);
    }
}

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
    // Nibble n ^ 8 is n - 8 in 4-bit two's complement.  Moved to the high
    // half of a byte it is the signed byte 16 (n - 8), which one sign-
    // extending conversion per element turns into fp32 (as the int8 codes
    // are); times s / 16 (exact: a power-of-two scaling of an fp16 value)
    // that is exactly (n - 8) * s, with the same sign of zero, infinities
    // and NaNs as the reference's (float)(n - 8) * s.
    const float s16 = f16_to_f32(scale_bits & 0xFFFFu) * 0.0625f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t x = q[j] ^ 0x88888888u;
        const int32_t hi = (int32_t)(x & 0xF0F0F0F0u);          // byte i: 16 x element 2i + 1
        const int32_t lo = (int32_t)((x << 4) & 0xF0F0F0F0u);   // byte i: 16 x element 2i
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = (float)((lo << (24 - 8 * i)) >> 24) * s16;  // element 2i
            const float b = (float)((hi << (24 - 8 * i)) >> 24) * s16;  // element 2i + 1
            out[4 * j + i] = pack_hot<DT>(a, b);
        }
    }
}

// Whether any of the 32 fp16 halves of a decrypted parameter row is inf or
// NaN (an asym8 row's zero points, 0..255, never look so).  A finite scale
// times an integer code is never NaN; a non-finite one makes NaN outputs,
// which the kernels then rewrite with canonical_nans.
__device__ __forceinline__ bool params_nonfinite(const uint32_t sc[16]) {
    uint32_t any = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t e = sc[i] & 0x7C007C00u;
        any |= ((e & 0xFFFFu) == 0x7C00u) | ((e >> 16) == 0x7C00u);
    }
    return any != 0u;
}

// ---------------------------------------------------------------------------
// Extension codes (no counterpart in the reference; the oracle's
// zo_quant_group16_e4m3 / zo_quant_group32_int4 / zo_quant_group64_asym8
// define them).  Same shape as profile S: an fp32 statistic, an fp16 scale
// rounded once from an IEEE division, inv = 1 / f32(scale) (IEEE), codes by
// round-to-nearest-even; dequantization is an exact fp32 product and one RNE.
// ---------------------------------------------------------------------------

// fp32 -> OCP e4m3 ("e4m3fn") saturating at +-448, round to nearest even.
// NaN inputs are the caller's (they give +-448 here).
__device__ __forceinline__ uint32_t f32_to_e4m3_sat(float x) {
    const uint32_t sign = (__float_as_uint(x) >> 24) & 0x80u;
    const float a = __builtin_fminf(__builtin_fabsf(x), 448.0f);
    const uint32_t u = __float_as_uint(a);
    // normal range: keep 3 mantissa bits with RNE; the carry runs into the
    // exponent, which is rebased from 127 to 7 (120 << 3 = 960)
    const uint32_t nrm = ((u + 0x7FFFFu + ((u >> 20) & 1u)) >> 20) - 960u;
    // below 2^-6: multiples of 2^-9 (a * 512 is exact); 8 is the code of 2^-6
    const uint32_t sub = (uint32_t)__builtin_rintf(a * 512.0f);
    return sign | (a < 0.015625f ? sub : nrm);
}

// e4m3 code (bits 0..7 of c) -> fp32, exact; 0x7F / 0xFF -> NaN.  The
// dequantizers use the hardware form below; this one is what ztcp_selftest
// compares it with.
__device__ __forceinline__ float e4m3_to_f32_sw(uint32_t c) {
    const uint32_t m7 = c & 0x7Fu;
    const float nrm = __uint_as_float((m7 << 20) + 0x3C000000u);  // exponent rebased 7 -> 127
    const float sub = (float)(c & 7u) * 0.001953125f;              // m * 2^-9
    float v = m7 < 8u ? sub : nrm;
    v = m7 == 0x7Fu ? __builtin_nanf("") : v;
    return __uint_as_float(__float_as_uint(v) | ((c & 0x80u) << 24));
}

// Byte B of word c -> fp32 by v_cvt_f32_fp8 (exact: every e4m3 value is an
// fp32 value).
template <int B>
__device__ __forceinline__ float e4m3_byte_to_f32(uint32_t c) {
    return __builtin_amdgcn_cvt_f32_fp8((int)c, B);
}

// a * b as a plain fp32 multiply.  For fp16 data the compiler otherwise folds
// the f16 <-> f32 conversion next to a product into v_fma_mix* with a +0
// addend, which turns a -0 product into +0; e4m3 has a negative zero code
// (0x80) that the codec keeps (the integer codes never produce -0).
template <int DT>
__device__ __forceinline__ float mul_keep_sign(float a, float b) {
    if constexpr (DT == kHotFp16) {
        asm volatile("" : "+v"(a));
        float r = a * b;
        asm volatile("" : "+v"(r));
        return r;
    }
    return a * b;
}

template <int DT>
__device__ __forceinline__ float group_amax16(const uint32_t w[8]) {
    float amax = 1e-6f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float a = __builtin_fabsf(hot_lo<DT>(w[i]));
        const float b = __builtin_fabsf(hot_hi<DT>(w[i]));
        amax = a > amax ? a : amax;
        amax = b > amax ? b : amax;
    }
    return amax;
}

// The same conversion by gfx950's v_cvt_pk_fp8_f32 (OCP e4m3, round to
// nearest even) of a value already clamped to [-448, 448]: two values per
// instruction, low byte first.  ztcp_selftest checks it against
// f32_to_e4m3_sat on every bf16 pattern and its neighbours (every rounding
// tie of e4m3 is a bf16 value).
__device__ __forceinline__ uint32_t e4m3_pair_hw(float a, float b) {
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xFFFFu;
}

// Clamp for the conversion; a NaN product (a scale that underflowed to 0, or
// a NaN element) becomes 0 and so code 0.
__device__ __forceinline__ float e4m3_operand(float x) {
    return x != x ? 0.0f : __builtin_amdgcn_fmed3f(x, -448.0f, 448.0f);
}

// e4m3 codes of one 16-element chunk with inv: 4 words, byte i = element i.
template <int DT>
__device__ __forceinline__ void e4m3_codes(const uint32_t w[8], float inv, uint32_t q[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t e0 = w[2 * j], e1 = w[2 * j + 1];
        const uint32_t lo = e4m3_pair_hw(e4m3_operand(mul_keep_sign<DT>(hot_lo<DT>(e0), inv)),
                                         e4m3_operand(mul_keep_sign<DT>(hot_hi<DT>(e0), inv)));
        const uint32_t hi = e4m3_pair_hw(e4m3_operand(mul_keep_sign<DT>(hot_lo<DT>(e1), inv)),
                                         e4m3_operand(mul_keep_sign<DT>(hot_hi<DT>(e1), inv)));
        q[j] = lo | (hi << 16);
    }
}

// max |element| of a group as a 16-bit pattern: bf16 and fp16 magnitudes
// order like their bit patterns, and every NaN pattern lies above +inf's.
__device__ __forceinline__ uint32_t amax_bits16(const uint32_t w[8]) {
    using u16x2 = unsigned short __attribute__((ext_vector_type(2)));
    u16x2 m = __builtin_bit_cast(u16x2, w[0] & 0x7FFF7FFFu);
#pragma unroll
    for (int i = 1; i < 8; ++i) m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[i] & 0x7FFF7FFFu));
    return m.x > m.y ? m.x : m.y;
}

// FP8 e4m3, 16-element group: s = fp16(amax / 448), IEEE division and
// reciprocal, codes by the saturating conversion with NaN -> 0 (the oracle's
// zo_quant_group16_e4m3).  Cold path for groups with NaN or infinite
// elements and for zero or infinite scales.
template <int DT>
__device__ __forceinline__ GroupCodes e4m3_group_exact(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                                     uint32_t w4, uint32_t w5, uint32_t w6, uint32_t w7) {
    const uint32_t w[8] = {w0, w1, w2, w3, w4, w5, w6, w7};
    GroupCodes r;
    r.scale = f32_to_f16(group_amax16<DT>(w) / 448.0f);
    uint32_t q[4];
    e4m3_codes<DT>(w, 1.0f / f16_to_f32(r.scale), q);
    r.q0 = q[0]; r.q1 = q[1]; r.q2 = q[2]; r.q3 = q[3];
    return r;
}

// The same codes with finite elements and a finite nonzero scale: amax from
// the 16-bit magnitudes, the scale by scale_e4m3, the reciprocal by recip_fast
// (exact for every positive finite fp16 value); the products are finite, so
// the clamp alone prepares them for the conversion.
template <int DT>
__device__ __forceinline__ GroupCodes e4m3_group_codes(const uint32_t w[8]) {
    const uint32_t mb = amax_bits16(w);
    const float m = DT == kHotBf16 ? __uint_as_float(mb << 16) : f16_to_f32(mb);
    const uint32_t sb = scale_e4m3(__builtin_fmaxf(m, 1e-6f));
    const bool special = mb >= (DT == kHotBf16 ? 0x7F80u : 0x7C00u) || sb == 0u || sb >= 0x7C00u;
    if (__builtin_expect(special, 0))
        return e4m3_group_exact<DT>(w[0], w[1], w[2], w[3], w[4], w[5], w[6], w[7]);
    const float inv = recip_fast(f16_to_f32(sb));
    GroupCodes r;
    r.scale = sb;
    uint32_t q[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t e0 = w[2 * j], e1 = w[2 * j + 1];
        const uint32_t lo =
            e4m3_pair_hw(__builtin_amdgcn_fmed3f(mul_keep_sign<DT>(hot_lo<DT>(e0), inv), -448.0f, 448.0f),
                         __builtin_amdgcn_fmed3f(mul_keep_sign<DT>(hot_hi<DT>(e0), inv), -448.0f, 448.0f));
        const uint32_t hi =
            e4m3_pair_hw(__builtin_amdgcn_fmed3f(mul_keep_sign<DT>(hot_lo<DT>(e1), inv), -448.0f, 448.0f),
                         __builtin_amdgcn_fmed3f(mul_keep_sign<DT>(hot_hi<DT>(e1), inv), -448.0f, 448.0f));
        q[j] = lo | (hi << 16);
    }
    r.q0 = q[0]; r.q1 = q[1]; r.q2 = q[2]; r.q3 = q[3];
    return r;
}

// FP8 e4m3, 16-element group.  Returns the scale bits.
template <int DT>
__device__ __forceinline__ uint32_t quant_group_e4m3(const uint32_t w[8], uint32_t q[4]) {
    const GroupCodes r = e4m3_group_codes<DT>(w);
    q[0] = r.q0; q[1] = r.q1; q[2] = r.q2; q[3] = r.q3;
    return r.scale;
}

// int4 codes of one 16-element chunk with inv (the reference's int4 formula,
// cpp:806-824): 2 words, element 2i in the low nibble of byte i.
template <int DT>
__device__ __forceinline__ void int4_codes(const uint32_t w[8], float inv, uint32_t q[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t e = w[4 * j + i];
            uint32_t nib[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float v = h ? hot_hi<DT>(e) : hot_lo<DT>(e);
                float rr = __builtin_rintf(v * inv) + 8.0f;
                rr = rr != rr ? 0.0f : rr;  // NaN: the x86 conversion gives INT_MIN, clamped to 0
                rr = rr < 0.0f ? 0.0f : (rr > 15.0f ? 15.0f : rr);
                nib[h] = (uint32_t)rr;
            }
            word |= (nib[0] | (nib[1] << 4)) << (8 * i);
        }
        q[j] = word;
    }
}

// int4 over a 32-element group (chunks a, b): s = fp16(max(amax_a, amax_b) / 7),
// IEEE division and reciprocal (the oracle's zo_quant_group32_int4).  Cold
// path for groups with non-finite elements and for scales that are not
// normal fp16 values.
template <int DT>
__device__ __forceinline__ uint32_t int4g32_exact(const uint32_t a[8], const uint32_t b[8], uint32_t q[4]) {
    const float ma = group_amax16<DT>(a), mb = group_amax16<DT>(b);
    const uint32_t sb = f32_to_f16((mb > ma ? mb : ma) / 7.0f);
    const float inv = 1.0f / f16_to_f32(sb);
    int4_codes<DT>(a, inv, q);
    int4_codes<DT>(b, inv, q + 2);
    return sb;
}

// int4 codes of 16 elements (words w) with a normal scale, each element
// converted where it is used: the int4_codes_fast sums without a float array.
template <int DT>
__device__ __forceinline__ void int4_codes_fast_w(const uint32_t w[8], float inv, uint32_t& q0, uint32_t& q1) {
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        b[i] = (__float_as_uint(hot_hi<DT>(w[i]) * inv + 12582920.0f) << 4) |
               __float_as_uint(hot_lo<DT>(w[i]) * inv + 12582920.0f);
    q0 = pack_low_bytes(b[0], b[1], b[2], b[3]);
    q1 = pack_low_bytes(b[4], b[5], b[6], b[7]);
}

// The same with the int4 fast path of profile S (scale_fast, recip_fast and
// rounding by the 1.5 * 2^23 sum) whenever the elements are finite and the
// scale is a normal fp16 value.  amax comes from the 16-bit magnitudes of
// both chunks (amax_bits16), so no chunk is held as fp32 values.
template <int DT>
__device__ __forceinline__ uint32_t quant_group32_int4(const uint32_t a[8], const uint32_t b[8], uint32_t q[4]) {
    const uint32_t ma = amax_bits16(a), mbits = amax_bits16(b);
    const uint32_t mb = ma > mbits ? ma : mbits;
    const float m = DT == kHotBf16 ? __uint_as_float(mb << 16) : f16_to_f32(mb);
    const uint32_t sb = scale_fast<4>(__builtin_fmaxf(m, 1e-6f));
    const bool special = mb >= (DT == kHotBf16 ? 0x7F80u : 0x7C00u) || (sb - 0x0400u) >= (0x7C00u - 0x0400u);
    if (__builtin_expect(special, 0)) return int4g32_exact<DT>(a, b, q);
    const float inv = recip_fast(f16_to_f32(sb));
    int4_codes_fast_w<DT>(a, inv, q[0], q[1]);
    int4_codes_fast_w<DT>(b, inv, q[2], q[3]);
    return sb;
}

// int8 asymmetric over a 64-element group (4 chunks): lo = min(0, min v),
// hi = max(0, max v), s = fp16(max(1e-6, hi - lo) / 255), z = clamp(rne(-lo *
// inv), 0, 255), q = clamp(rne(v * inv) + z, 0, 255); NaN codes are 0.
// Returns scale bits | zero point << 16 (the group's parameter word).
//
// Exact emulation for groups with non-finite elements or a zero / infinite
// scale (inlined in a cold block, as quant_group_exact).
template <int DT>
__device__ __forceinline__ uint32_t asym8_exact(const uint32_t (&w)[4][8], uint32_t q[16]) {
    float lo = 0.0f, hi = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float v = (i & 1) ? hot_hi<DT>(w[c][i >> 1]) : hot_lo<DT>(w[c][i >> 1]);
            lo = v < lo ? v : lo;
            hi = v > hi ? v : hi;
        }
    }
    float range = hi - lo;
    range = range > 1e-6f ? range : 1e-6f;
    const uint32_t sb = f32_to_f16(range / 255.0f);
    const float inv = 1.0f / f16_to_f32(sb);
    float zf = __builtin_rintf(-lo * inv);
    zf = zf != zf ? 0.0f : zf;
    zf = zf < 0.0f ? 0.0f : (zf > 255.0f ? 255.0f : zf);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t word = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t e = w[c][2 * j + (i >> 1)];
                const float v = (i & 1) ? hot_hi<DT>(e) : hot_lo<DT>(e);
                float qf = __builtin_rintf(v * inv) + zf;
                qf = qf != qf ? 0.0f : qf;
                qf = qf < 0.0f ? 0.0f : (qf > 255.0f ? 255.0f : qf);
                word |= (uint32_t)qf << (8 * i);
            }
            q[4 * c + j] = word;
        }
    }
    return sb | ((uint32_t)zf << 16);
}

// Order-preserving signed keys of the two 16-bit floats (fp16 or bf16) of a
// word: k = b ^ ((b >> 15) & 0x7FFF) per half, so that key order is the
// floats' order, -0 just below +0, and NaN patterns outside +-inf.  The
// transform is its own inverse.
typedef short ztcp_short2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ ztcp_short2 order_keys(uint32_t w) {
    const ztcp_short2 x = __builtin_bit_cast(ztcp_short2, w);
    return x ^ ((x >> (short)15) & (short)0x7FFF);
}
__device__ __forceinline__ uint32_t key_bits(short k) {
    return (uint32_t)(uint16_t)(k ^ ((k >> 15) & 0x7FFF));
}
template <int DT>
__device__ __forceinline__ float hot_bits_to_f32(uint32_t b) {
    if constexpr (DT == kHotBf16) return __uint_as_float(b << 16);
    else return f16_to_f32(b);
}

// Fast path (finite elements, a positive finite scale): |v * inv| <= 255 *
// (1 + 2^-10) (x 1.5 for a subnormal scale), so adding 1.5 * 2^23 rounds
// v * inv to nearest-even in that same add and the low bits of the sum are
// rne(v * inv) + 2^22; the zero point is added and the result clamped as
// integers.  The group's minimum and maximum come from packed 16-bit keys of
// the raw elements (two per instruction); a NaN element makes one of them a
// NaN and the group takes the exact path, as do infinities and a zero or
// infinite scale.  A -0 minimum gives the same range and zero point as the
// reference-style compares (which keep +0).
template <int DT>
__device__ __forceinline__ uint32_t quant_group64_asym8(const uint32_t (&w)[4][8], uint32_t q[16]) {
    ztcp_short2 kmin = {0, 0}, kmax = {0, 0};  // keys of +0: the range always includes 0
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const ztcp_short2 k = order_keys(w[c][i]);
            kmin = __builtin_elementwise_min(kmin, k);
            kmax = __builtin_elementwise_max(kmax, k);
        }
    }
    const float lo = hot_bits_to_f32<DT>(key_bits(kmin.x < kmin.y ? kmin.x : kmin.y));
    const float hi = hot_bits_to_f32<DT>(key_bits(kmax.x > kmax.y ? kmax.x : kmax.y));
    float range = hi - lo;
    range = range > 1e-6f ? range : 1e-6f;
    const uint32_t sb = f32_to_f16(range / 255.0f);
    const bool special = !(hi < __builtin_inff()) || !(lo > -__builtin_inff()) || sb == 0u || sb >= 0x7C00u;
    if (__builtin_expect(special, 0)) return asym8_exact<DT>(w, q);
    const float inv = recip_fast(f16_to_f32(sb));
    float zf = __builtin_rintf(-lo * inv);
    zf = zf < 0.0f ? 0.0f : (zf > 255.0f ? 255.0f : zf);
    const uint32_t z = (uint32_t)zf;
    const uint32_t bias = 0x4B400000u - z;  // bits of 1.5 * 2^23, less the zero point
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t t[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t e = w[c][2 * j + (i >> 1)];
                const float v = (i & 1) ? hot_hi<DT>(e) : hot_lo<DT>(e);
                const int32_t d = (int32_t)(__float_as_uint(v * inv + 12582912.0f) - bias);
                t[i] = (uint32_t)(d < 0 ? 0 : (d > 255 ? 255 : d));  // v_med3_i32
            }
            q[4 * c + j] = pack_low_bytes(t[0], t[1], t[2], t[3]);
        }
    }
    return sb | (z << 16);
}

// 16 e4m3 codes (4 words) -> 8 packed hot words.
template <int DT>
__device__ __forceinline__ void dequant_group_e4m3(const uint32_t q[4], uint32_t scale_bits, uint32_t out[8]) {
    const float s = f16_to_f32(scale_bits & 0xFFFFu);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        out[2 * j] = pack_hot<DT>(mul_keep_sign<DT>(e4m3_byte_to_f32<0>(q[j]), s),
                                  mul_keep_sign<DT>(e4m3_byte_to_f32<1>(q[j]), s));
        out[2 * j + 1] = pack_hot<DT>(mul_keep_sign<DT>(e4m3_byte_to_f32<2>(q[j]), s),
                                      mul_keep_sign<DT>(e4m3_byte_to_f32<3>(q[j]), s));
    }
}

// 16 asym8 codes (4 words) of a group with parameter word (scale | zero << 16)
// -> 8 packed hot words: hot(f32(q - z) * f32(s)).
template <int DT>
__device__ __forceinline__ void dequant_asym8_16(const uint32_t q[4], uint32_t prm, uint32_t out[8]) {
    const float s = f16_to_f32(prm & 0xFFFFu);
    const int32_t z = (int32_t)(prm >> 16);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t w = q[j];
        const float e0 = (float)((int32_t)(w & 0xFFu) - z) * s;
        const float e1 = (float)((int32_t)((w >> 8) & 0xFFu) - z) * s;
        const float e2 = (float)((int32_t)((w >> 16) & 0xFFu) - z) * s;
        const float e3 = (float)((int32_t)(w >> 24) - z) * s;
        out[2 * j] = pack_hot<DT>(e0, e1);
        out[2 * j + 1] = pack_hot<DT>(e2, e3);
    }
}

}  // namespace ztcp
