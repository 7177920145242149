// ztcp_ingress.hip -- fused cold-page ingress for gfx950:
// verify (header, AAD, SipHash tag) -> ChaCha20 decrypt -> dequantize, one
// HBM read of the blob and one HBM write of the hot page.  Replaces the
// per-page decoder of fused_decode_cold_pages_peak_into_cpu (cpp:2309-2463).
//
// One workgroup handles up to 64 pages with 12 waves:
//   * wave 0 verifies one page per lane: magic/version (status 1), AAD
//     tenant/model/layer/token hash (status 2), the SipHash-2-4-128 tag over
//     header || ciphertext (status 3), then flags and payload size (status 1),
//     in the reference's order (cpp:2313-2355).
//   * waves on the other three SIMDs decrypt and dequantize (page, unit)
//     items concurrently (waves 4 and 8 share the verify wave's SIMD and exit),
//     each page according to its own header flags.  This is speculative: a
//     page whose verdict is not OK has its outputs zeroed before the kernel
//     ends (per-page mode) or by the finalize kernel (all-or-nothing mode,
//     which zeroes every output, cpp:2481-2486).  Outputs are only valid after
//     the call returns OK, as with the reference.
// Requires 16-byte aligned blobs / outputs, blob_bytes % 16 == 0 and every
// layout aligned to 64-byte units; otherwise the host uses the generic path.
#include "ztcp_params.h"

namespace ztcp {

__device__ __forceinline__ void xor_block(uint32_t ct[16], const uint32_t ks[16]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) ct[i] ^= ks[i];
}

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
    xor_block(sc, ks);
    const uint32_t code0 = q_off + (uint32_t)(G0 * CW * 4);
#pragma unroll 1
    for (int j = 0; j < NBLK; ++j) {
        uint32_t ct[16];
        load_block(pay + code0 + (uint32_t)j * 64u, ct);
        chacha_block(p.key, 1u + code0 / 64u + (uint32_t)j, n0, n1, n2, ks);
        xor_block(ct, ks);
#pragma unroll
        for (int i = 0; i < GPB; ++i) {
            const uint32_t sbits = (i & 1) ? (sc[i >> 1] >> 16) : (sc[i >> 1] & 0xFFFFu);
            uint32_t o[8];
            if constexpr (KIND == kSecInt8) dequant_group_int8<DT>(ct + 4 * i, sbits, o);
            else dequant_group_int4<DT>(ct + 2 * i, sbits, o);
            store_group(out + cur.off, o);
            cur.step(gpv, skip);
        }
        // consume this block's scales
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
        xor_block(ct, ks);
        store_group(out + cur.off, ct);
        cur.step(gpv, skip);
        store_group(out + cur.off, ct + 8);
        cur.step(gpv, skip);
    }
}

template <int DT>
__device__ void decode_unit(const IngressParams& p, const Layout& lay, int64_t page, int32_t u,
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

// Verdict of one page (cpp:2313-2355); the MAC covers header || payload,
// read two 64-byte chunks ahead of the chunk being absorbed.
__device__ int32_t verify_page(const IngressParams& p, int64_t page) {
    const uint8_t* blob = ingress_blob(p, page);
    const uint4 h0 = ldg16(blob, 0), h1 = ldg16(blob, 1);
    Sip s;
    s.init(p.mk0, p.mk1);
    // header || payload = n16 16-byte words (payload % 16 == 0 on this path)
    const uint32_t n16 = (kHeader + p.payload) / 16u;
    const uint32_t n64 = n16 / 4u;
    uint32_t next = 0;
    sip_stream64(s, n64, [&](uint4 (&x)[4]) {
        x[0] = ldg16(blob, next); x[1] = ldg16(blob, next + 1u);
        x[2] = ldg16(blob, next + 2u); x[3] = ldg16(blob, next + 3u);
        next += 4u;
    });
#pragma unroll 1
    for (uint32_t k = n64 * 4u; k < n16; ++k) s.absorb(ldg16(blob, k));
    uint64_t lo, hi;
    s.finish((uint64_t)((kHeader + p.payload) & 0xFFu) << 56, lo, hi);
    const uint4 tag = ldg16(blob, n16);
    const uint32_t diff = (tag.x ^ (uint32_t)lo) | (tag.y ^ (uint32_t)(lo >> 32)) |
                          (tag.z ^ (uint32_t)hi) | (tag.w ^ (uint32_t)(hi >> 32));
    const uint32_t magic = h0.x & 0xFFFFu, version = (h0.x >> 16) & 0xFFu, flags = h0.x >> 24;
    if (magic != kMagic || version != kVersion) return 1;
    const uint64_t tok = (uint64_t)h1.x | ((uint64_t)h1.y << 32);
    if (h0.y != p.exp_tenant || h0.z != p.exp_model || (h0.w & 0xFFFFu) != ingress_layer(p, page) ||
        tok != ingress_token(p, page))
        return 2;
    if (diff != 0u) return 3;
    const uint32_t preset = flags & 0x0Fu, rope_mode = flags >> 4;
    if (preset < 1u || preset > 3u || rope_mode > 2u) return 1;
    if (!p.lay_ok[(preset - 1u) * 3u + rope_mode]) return 1;
    return 0;
}

template <int DT>
__global__ __launch_bounds__(kFusedThreads) void ingress_fused_kernel(IngressParams p) {
    __shared__ int32_t status[64];
    const int64_t page0 = (int64_t)blockIdx.x * p.ppw;
    const int ppw = (int)min((int64_t)p.ppw, p.batch - page0);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nwaves = blockDim.x >> 6;
    if (wave == 0) {
        __builtin_amdgcn_s_setprio(3);
        const int32_t st = verify_page(p, page0 + (lane < ppw ? lane : 0));
        status[lane] = st;
    } else if ((wave & 3) != 0) {  // waves 4 and 8 share the verify wave's SIMD: they idle
        const int items = ppw * p.n_units;
        const int n_batches = (items + 63) / 64;
        const int dec = wave - 1 - (wave >> 2);
        const int ndec = nwaves - 1 - ((nwaves - 1) >> 2);
#pragma unroll 1
        for (int b = dec; b < n_batches; b += ndec) {
            const int item = b * 64 + lane;
            if (item >= items) continue;
            const int u = item / ppw;
            const int64_t page = page0 + (item - u * ppw);
            const uint8_t* hq = ingress_blob(p, page);
            const uint4 h0 = ldg16(hq, 0), h1 = ldg16(hq, 1);
            const uint32_t flags = h0.x >> 24, preset = flags & 0x0Fu, rope_mode = flags >> 4;
            const bool valid = preset >= 1u && preset <= 3u && rope_mode <= 2u &&
                               p.lay_ok[(preset - 1u) * 3u + rope_mode];
            const int li = valid ? (int)((preset - 1u) * 3u + rope_mode) : -1;
            // nonce from the page's own header (cpp:2357-2365)
            const uint32_t n0 = h1.z, n1 = h1.w;
            const uint32_t n2 = ((h0.w & 0xFFFFu) << 16) | (h0.w >> 16);
            // one pass per distinct layout present in the wave (normally one)
#pragma unroll 1
            for (int l = 0; l < 9; ++l) {
                if (!__any(li == l)) continue;
                if (li == l) decode_unit<DT>(p, p.lay[l], page, u, n0, n1, n2);
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // every decode store has completed before the verdicts
    __syncthreads();
    if ((int)threadIdx.x < ppw) {
        const int32_t st = status[threadIdx.x];
        const int64_t page = page0 + threadIdx.x;
        if (p.page_status) p.page_status[page] = st;
        if (st != 0)
            atomicMin(&p.state->fail, ((unsigned long long)page << 8) | (unsigned long long)st);
    }
    if (p.per_page) {  // extension: zero only the failing pages
        const int64_t n16 = p.page_bytes / 16;
#pragma unroll 1
        for (int pl = 0; pl < ppw; ++pl) {
            if (status[pl] == 0) continue;
            uint8_t* k = ingress_k(p, page0 + pl);
            for (int64_t i = threadIdx.x; i < n16; i += blockDim.x) stg16(k, i, make_uint4(0, 0, 0, 0));
            uint8_t* v = ingress_v(p, page0 + pl);
            if (v)
                for (int64_t i = threadIdx.x; i < n16; i += blockDim.x) stg16(v, i, make_uint4(0, 0, 0, 0));
        }
    }
}

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
    const int waves = kFusedWaves;
    const int64_t grid = (p.batch + p.ppw - 1) / p.ppw;
    if (dtype == kHotBf16)
        hipLaunchKernelGGL(ingress_fused_kernel<kHotBf16>, dim3((uint32_t)grid), dim3(64 * waves), 0, s, p);
    else
        hipLaunchKernelGGL(ingress_fused_kernel<kHotFp16>, dim3((uint32_t)grid), dim3(64 * waves), 0, s, p);
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
