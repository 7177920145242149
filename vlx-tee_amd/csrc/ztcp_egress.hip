// ztcp_egress.hip -- fused cold-page egress for gfx950:
// quantize -> ChaCha20 -> SipHash-2-4-128 in one kernel, one HBM read of the
// hot page and one HBM write of the blob.  Replaces the per-page encoder
// encode_one_cold_page_into_cpu (cpp:1103-1426) driven by
// fused_encode_cold_pages_peak_into_cpu (cpp:1904-2004).
//
// Work decomposition (one workgroup = up to 64 pages, 16 waves):
//   * wave 0 (the MAC wave) owns one page per lane.  SipHash is a strictly
//     sequential chain per page, so 64 pages share one wave's instruction
//     stream; the wave runs at raised priority and walks the page in MAC
//     order, reading back ciphertext the producers wrote (still in L2).
//   * waves 1..15 (producers) take "batches" of 64 (page, unit) items.  A
//     unit is 32 consecutive groups of one section: its codes (4/8/16
//     keystream blocks) and its 64-byte scale block.  A lane loads its groups,
//     computes each keystream block while the loads are in flight, quantizes,
//     XORs and stores.  Plaintext never leaves registers.
//   * a producer publishes a finished batch through a workgroup-scope release
//     on an LDS flag; the MAC wave acquires the flag before reading.  The MAC
//     wave never blocks producers, and its wait is bounded (sticky diag flag).
// Requires every section to hold a multiple of 32 groups (Layout::aligned),
// payload == required, 16-byte aligned pointers; otherwise the host routes the
// call to the generic kernels.
#include "ztcp_params.h"

namespace ztcp {

constexpr uint32_t kSpinLimit = 1u << 22;

__device__ __forceinline__ void wait_flag(const uint32_t* flag, DeviceState* st) {
    if (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) != 0u) return;
    for (uint32_t spin = 0;; ++spin) {
        __builtin_amdgcn_s_sleep(8);
        if (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) != 0u) return;
        if (spin >= kSpinLimit) {
            atomicOr(&st->diag, kDiagEgressWait);
            return;
        }
    }
}

__device__ __forceinline__ void load_group(const uint8_t* p, uint32_t w[8]) {
    const uint4 a = reinterpret_cast<const uint4*>(p)[0];
    const uint4 b = reinterpret_cast<const uint4*>(p)[1];
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

__device__ __forceinline__ void store_block(uint8_t* dst, const uint32_t pt[16], const uint32_t ks[16]) {
    uint4* d = reinterpret_cast<uint4*>(dst);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        d[i] = make_uint4(pt[4 * i] ^ ks[4 * i], pt[4 * i + 1] ^ ks[4 * i + 1],
                          pt[4 * i + 2] ^ ks[4 * i + 2], pt[4 * i + 3] ^ ks[4 * i + 3]);
}

struct GroupCursor {  // (vec, group) walk over a section in row-major order
    int64_t vec;
    int32_t g;
    __device__ __forceinline__ void step(int32_t gpv) {
        if (++g == gpv) { g = 0; ++vec; }
    }
};

// One unit of a quantized section.  GPB = groups per 64-byte code block
// (4 for int8, 8 for int4).
template <int DT, int KIND>
__device__ __forceinline__ void produce_quant_unit(const EgressParams& p, const uint8_t* src,
                                                   uint8_t* pay, int32_t lu, int32_t gpv,
                                                   int32_t col, uint32_t q_off, uint32_t s_off,
                                                   uint32_t n0, uint32_t n1, uint32_t n2) {
    constexpr int GPB = KIND == kSecInt8 ? 4 : 8;
    constexpr int NBLK = 32 / GPB;
    constexpr int CW = KIND == kSecInt8 ? 4 : 2;  // code words per group
    const int32_t G0 = lu * 32;
    GroupCursor cur{G0 / gpv, G0 % gpv};
    const int64_t row = (int64_t)p.head_dim * 2;
    uint32_t sc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) sc[i] = 0;
    const uint32_t blk0 = 1u + (q_off + (uint32_t)G0 * (uint32_t)(CW * 4)) / 64u;
#pragma unroll 1
    for (int j = 0; j < NBLK; ++j) {
        uint32_t w[GPB][8];
#pragma unroll
        for (int i = 0; i < GPB; ++i) {
            load_group(src + cur.vec * row + (int64_t)(col + cur.g * 16) * 2, w[i]);
            cur.step(gpv);
        }
        uint32_t ks[16];
        chacha_block(p.key, blk0 + (uint32_t)j, n0, n1, n2, ks);
        uint32_t pt[16];
        uint32_t s[GPB];
#pragma unroll
        for (int i = 0; i < GPB; ++i) {
            if constexpr (KIND == kSecInt8) s[i] = quant_group_int8<DT>(w[i], pt + 4 * i);
            else s[i] = quant_group_int4<DT>(w[i], pt + 2 * i);
        }
        // append this block's GPB scales (GPB/2 words) to the 16-word scale block
#pragma unroll
        for (int t = 0; t < 16 - GPB / 2; ++t) sc[t] = sc[t + GPB / 2];
#pragma unroll
        for (int i = 0; i < GPB / 2; ++i) sc[16 - GPB / 2 + i] = s[2 * i] | (s[2 * i + 1] << 16);
        store_block(pay + q_off + (uint32_t)(G0 * CW * 4) + (uint32_t)j * 64u, pt, ks);
    }
    const uint32_t s_unit = s_off + (uint32_t)lu * 64u;
    uint32_t ks[16];
    chacha_block(p.key, 1u + s_unit / 64u, n0, n1, n2, ks);
    store_block(pay + s_unit, sc, ks);
}

// One unit of a raw (PRESERVE_RAW) section: 32 groups of hot bytes.
__device__ __forceinline__ void produce_raw_unit(const EgressParams& p, const uint8_t* src,
                                                 uint8_t* pay, int32_t lu, int32_t gpv,
                                                 int32_t col, uint32_t q_off, uint32_t n0,
                                                 uint32_t n1, uint32_t n2) {
    const int32_t G0 = lu * 32;
    GroupCursor cur{G0 / gpv, G0 % gpv};
    const int64_t row = (int64_t)p.head_dim * 2;
    const uint32_t blk0 = 1u + (q_off + (uint32_t)G0 * 32u) / 64u;
#pragma unroll 1
    for (int j = 0; j < 16; ++j) {
        uint32_t pt[16];
        load_group(src + cur.vec * row + (int64_t)(col + cur.g * 16) * 2, pt);
        cur.step(gpv);
        load_group(src + cur.vec * row + (int64_t)(col + cur.g * 16) * 2, pt + 8);
        cur.step(gpv);
        uint32_t ks[16];
        chacha_block(p.key, blk0 + (uint32_t)j, n0, n1, n2, ks);
        store_block(pay + q_off + (uint32_t)G0 * 32u + (uint32_t)j * 64u, pt, ks);
    }
}

template <int DT>
__device__ void produce_unit(const EgressParams& p, int64_t page, int32_t u) {
    const int si = section_of_unit(p.lay, u);
    const int32_t kind = ZTCP_SEC_FIELD(p.lay, si, kind);
    const int32_t srcsel = ZTCP_SEC_FIELD(p.lay, si, src);
    const int32_t col = ZTCP_SEC_FIELD(p.lay, si, col);
    const int32_t gpv = ZTCP_SEC_FIELD(p.lay, si, gpv);
    const int32_t lu = u - ZTCP_SEC_FIELD(p.lay, si, unit_begin);
    const uint32_t q_off = ZTCP_SEC_FIELD(p.lay, si, q_off);
    const uint32_t s_off = ZTCP_SEC_FIELD(p.lay, si, s_off);
    const EgressPage pg = egress_page(p, page);
    const uint8_t* src = srcsel ? pg.v : pg.k;
    uint8_t* pay = pg.blob + kHeader;
    const uint32_t n0 = (uint32_t)pg.seq, n1 = (uint32_t)(pg.seq >> 32);
    if (kind == kSecInt8)
        produce_quant_unit<DT, kSecInt8>(p, src, pay, lu, gpv, col, q_off, s_off, n0, n1, pg.nonce2);
    else if (kind == kSecInt4)
        produce_quant_unit<DT, kSecInt4>(p, src, pay, lu, gpv, col, q_off, s_off, n0, n1, pg.nonce2);
    else
        produce_raw_unit(p, src, pay, lu, gpv, col, q_off, n0, n1, pg.nonce2);
}

// SipHash over n64 consecutive 64-byte chunks, next chunk prefetched.
__device__ __forceinline__ void absorb_chunks(Sip& s, const uint4* ptr, int n64) {
    if (n64 <= 0) return;
    uint4 a0 = ptr[0], a1 = ptr[1], a2 = ptr[2], a3 = ptr[3];
#pragma unroll 1
    for (int c = 0; c < n64; ++c) {
        const int nx = c + 1 < n64 ? c + 1 : c;
        const uint4 b0 = ptr[4 * nx], b1 = ptr[4 * nx + 1], b2 = ptr[4 * nx + 2], b3 = ptr[4 * nx + 3];
        s.absorb(lo64(a0)); s.absorb(hi64(a0));
        s.absorb(lo64(a1)); s.absorb(hi64(a1));
        s.absorb(lo64(a2)); s.absorb(hi64(a2));
        s.absorb(lo64(a3)); s.absorb(hi64(a3));
        a0 = b0; a1 = b1; a2 = b2; a3 = b3;
    }
}

template <int DT>
__device__ void egress_mac(const EgressParams& p, int64_t page0, int ppw, const uint32_t* done) {
    const int lane = threadIdx.x & 63;
    const bool active = lane < ppw;
    const int64_t page = page0 + (active ? lane : 0);
    const EgressPage pg = egress_page(p, page);
    uint8_t* blob = pg.blob;
    if (active) {  // header (cpp:1129-1140)
        uint4* h = reinterpret_cast<uint4*>(blob);
        h[0] = make_uint4((uint32_t)p.hdr0, (uint32_t)(p.hdr0 >> 32), (uint32_t)pg.hdr1,
                          (uint32_t)(pg.hdr1 >> 32));
        h[1] = make_uint4((uint32_t)pg.token, (uint32_t)(pg.token >> 32), (uint32_t)pg.seq,
                          (uint32_t)(pg.seq >> 32));
    }
    Sip s;
    s.init(p.mk0, p.mk1);
    s.absorb(p.hdr0);
    s.absorb(pg.hdr1);
    s.absorb(pg.token);
    s.absorb(pg.seq);
    const uint8_t* pay = blob + kHeader;
#pragma unroll 1
    for (int si = 0; si < p.lay.n_sec; ++si) {
        const int32_t kind = ZTCP_SEC_FIELD(p.lay, si, kind);
        const int32_t ub = ZTCP_SEC_FIELD(p.lay, si, unit_begin);
        const int32_t nu = ZTCP_SEC_FIELD(p.lay, si, n_units);
        const uint32_t q_off = ZTCP_SEC_FIELD(p.lay, si, q_off);
        const uint32_t s_off = ZTCP_SEC_FIELD(p.lay, si, s_off);
        const int32_t unit_bytes = 32 * code_bytes_per_group(kind);
#pragma unroll 1
        for (int32_t lu = 0; lu < nu; ++lu) {
            const int32_t u = ub + lu;
            const int32_t b0 = (u * ppw) / 64, b1 = (u * ppw + ppw - 1) / 64;
            wait_flag(&done[b0], p.state);
            if (b1 != b0) wait_flag(&done[b1], p.state);
            absorb_chunks(s, reinterpret_cast<const uint4*>(pay + q_off + (uint32_t)(lu * unit_bytes)),
                          unit_bytes / 64);
        }
        if (kind != kSecRaw) absorb_chunks(s, reinterpret_cast<const uint4*>(pay + s_off), nu);
    }
    uint64_t lo, hi;
    s.finish((uint64_t)((kHeader + p.payload) & 0xFFu) << 56, lo, hi);
    if (active)
        *reinterpret_cast<uint4*>(blob + kHeader + p.payload) =
            make_uint4((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32));
}

template <int DT>
__global__ __launch_bounds__(1024) void egress_fused_kernel(EgressParams p) {
    extern __shared__ uint32_t done[];
    const int64_t page0 = (int64_t)blockIdx.x * p.ppw;
    const int ppw = (int)min((int64_t)p.ppw, p.batch - page0);
    const int items = ppw * p.lay.n_units;
    const int n_batches = (items + 63) / 64;
    for (int i = threadIdx.x; i < n_batches; i += blockDim.x) done[i] = 0u;
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nwaves = blockDim.x >> 6;
    if (wave == 0) {
        __builtin_amdgcn_s_setprio(3);
        egress_mac<DT>(p, page0, ppw, done);
        return;
    }
#pragma unroll 1
    for (int b = wave - 1; b < n_batches; b += nwaves - 1) {
        const int item = b * 64 + lane;
        if (item < items) {
            const int u = item / ppw;
            produce_unit<DT>(p, page0 + (item - u * ppw), u);
        }
        __builtin_amdgcn_s_waitcnt(0);  // every store of this batch has completed
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0) __hip_atomic_store(&done[b], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}

hipError_t launch_egress_fused(const EgressParams& p, int dtype, int waves, hipStream_t s) {
    const int64_t grid = (p.batch + p.ppw - 1) / p.ppw;
    const size_t lds = (size_t)p.n_batches * sizeof(uint32_t);
    if (dtype == kHotBf16)
        hipLaunchKernelGGL(egress_fused_kernel<kHotBf16>, dim3((uint32_t)grid), dim3(64 * waves), lds, s, p);
    else
        hipLaunchKernelGGL(egress_fused_kernel<kHotFp16>, dim3((uint32_t)grid), dim3(64 * waves), lds, s, p);
    return hipGetLastError();
}

}  // namespace ztcp
