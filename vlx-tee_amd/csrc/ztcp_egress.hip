// ztcp_egress.hip -- fused cold-page egress for gfx950:
// quantize -> ChaCha20 -> SipHash-2-4-128 in one kernel, one HBM read of the
// hot page and one HBM write of the blob.  Replaces the per-page encoder
// encode_one_cold_page_into_cpu (cpp:1103-1426) driven by
// fused_encode_cold_pages_peak_into_cpu (cpp:1904-2004).
//
// Work decomposition (one workgroup = up to 64 pages, 12 waves):
//   * wave 0 (the MAC wave) owns one page per lane.  SipHash is a strictly
//     sequential chain per page, so 64 pages share one wave's instruction
//     stream and the kernel can never be shorter than one page's chain
//     (~240 cycles per 8-byte word on an otherwise idle SIMD).  The MAC wave
//     therefore runs at raised priority on a SIMD of its own: waves 4 and 8,
//     which the dispatcher places on the same SIMD, exit at once.  It
//     walks the page in MAC order, reading back ciphertext the producers
//     wrote, two 64-byte chunks ahead of the one it absorbs.
//   * the other 9 waves (producers) take "batches" of 64 (page, unit)
//     items.  A unit is 32 consecutive groups of one section: its codes
//     (4 / 8 / 16 keystream blocks) and its 64-byte scale block.  A lane
//     issues the loads of a block's groups, computes the block's keystream
//     while they are in flight, quantizes, XORs and stores.  Plaintext never
//     leaves registers.
//   * a producer publishes a finished batch through a workgroup-scope release
//     on an LDS flag; the MAC wave acquires the flag before reading a unit.
//     The MAC wave never blocks producers, and its wait is bounded (a sticky
//     diagnostic flag records an expired wait and the kernel still ends).
// Requires every section to hold a multiple of 32 groups (Layout::aligned),
// payload == required and 16-byte aligned pointers; otherwise the host routes
// the call to the generic kernels.
#include "ztcp_params.h"

namespace ztcp {

constexpr uint32_t kSpinLimit = 1u << 22;

__device__ __forceinline__ void wait_flag(const uint32_t* flag, DeviceState* st) {
    if (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) != 0u) return;
    for (uint32_t spin = 0;; ++spin) {
        __builtin_amdgcn_s_sleep(2);
        if (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) != 0u) return;
        if (spin >= kSpinLimit) {
            atomicOr(&st->diag, kDiagEgressWait);
            return;
        }
    }
}

__device__ __forceinline__ void load_group(const uint8_t* p, uint32_t w[8]) {
    const uint4 a = ldg16(p, 0), b = ldg16(p, 1);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

__device__ __forceinline__ void store_block(uint8_t* dst, const uint32_t pt[16], const uint32_t ks[16]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
        stg16(dst, i, make_uint4(pt[4 * i] ^ ks[4 * i], pt[4 * i + 1] ^ ks[4 * i + 1],
                                 pt[4 * i + 2] ^ ks[4 * i + 2], pt[4 * i + 3] ^ ks[4 * i + 3]));
}

// One unit of a quantized section.  GPB = groups per 64-byte code block
// (4 for int8, 8 for int4).  Per block: quantize the groups loaded during the
// previous block's keystream, issue the next block's loads, compute this
// block's keystream, XOR and store.  The unit's 32 scales are staged in this
// lane's LDS slot (word-major, so lanes hit distinct banks) and encrypted as
// the unit's scale block at the end.
template <int DT, int KIND>
__device__ __forceinline__ void produce_quant_unit(const EgressParams& p, const uint8_t* src,
                                                   uint8_t* pay, int32_t lu, int32_t gpv,
                                                   int32_t col, uint32_t q_off, uint32_t s_off,
                                                   uint32_t n0, uint32_t n1, uint32_t n2,
                                                   uint32_t* slot) {
    constexpr int GPB = KIND == kSecInt8 ? 4 : 8;
    constexpr int NBLK = 32 / GPB;
    constexpr int CW = KIND == kSecInt8 ? 4 : 2;  // code words per group
    const int32_t G0 = lu * 32;
    GroupCursor cur = group_cursor(G0, gpv, col, p.head_dim);
    const uint32_t skip = (uint32_t)(p.head_dim - gpv * 16) * 2u;
    const uint32_t blk0 = 1u + (q_off + (uint32_t)G0 * (uint32_t)(CW * 4)) / 64u;
    uint8_t* code = pay + q_off + (uint32_t)(G0 * CW * 4);
    uint32_t w[GPB][8];
#pragma unroll
    for (int i = 0; i < GPB; ++i) {
        load_group(src + cur.off, w[i]);
        cur.step(gpv, skip);
    }
#pragma unroll 1
    for (int j = 0; j < NBLK; ++j) {
        uint32_t pt[16];
#pragma unroll
        for (int i = 0; i < GPB; i += 2) {
            uint32_t qa[4], qb[4];
            const uint32_t sa = quant_group<DT, KIND == kSecInt8 ? 8 : 4>(w[i], qa);
            const uint32_t sbb = quant_group<DT, KIND == kSecInt8 ? 8 : 4>(w[i + 1], qb);
#pragma unroll
            for (int t = 0; t < CW; ++t) {
                pt[CW * i + t] = qa[t];
                pt[CW * (i + 1) + t] = qb[t];
            }
            slot[(j * (GPB / 2) + i / 2) * 64] = sa | (sbb << 16);
        }
        if (j + 1 < NBLK) {
#pragma unroll
            for (int i = 0; i < GPB; ++i) {
                load_group(src + cur.off, w[i]);
                cur.step(gpv, skip);
            }
        }
        uint32_t ks[16];
        chacha_block(p.key, blk0 + (uint32_t)j, n0, n1, n2, ks);
        store_block(code + (uint32_t)j * 64u, pt, ks);
    }
    uint32_t sc[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) sc[t] = slot[t * 64];
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
    GroupCursor cur = group_cursor(G0, gpv, col, p.head_dim);
    const uint32_t skip = (uint32_t)(p.head_dim - gpv * 16) * 2u;
    const uint32_t blk0 = 1u + (q_off + (uint32_t)G0 * 32u) / 64u;
    uint32_t pt[16];
    load_group(src + cur.off, pt);
    cur.step(gpv, skip);
    load_group(src + cur.off, pt + 8);
    cur.step(gpv, skip);
#pragma unroll 1
    for (int j = 0; j < 16; ++j) {
        uint32_t ks[16];
        chacha_block(p.key, blk0 + (uint32_t)j, n0, n1, n2, ks);
        store_block(pay + q_off + (uint32_t)G0 * 32u + (uint32_t)j * 64u, pt, ks);
        if (j + 1 < 16) {
            load_group(src + cur.off, pt);
            cur.step(gpv, skip);
            load_group(src + cur.off, pt + 8);
            cur.step(gpv, skip);
        }
    }
}

template <int DT>
__device__ void produce_unit(const EgressParams& p, int64_t page, int32_t u, uint32_t* slot) {
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
        produce_quant_unit<DT, kSecInt8>(p, src, pay, lu, gpv, col, q_off, s_off, n0, n1, pg.nonce2, slot);
    else if (kind == kSecInt4)
        produce_quant_unit<DT, kSecInt4>(p, src, pay, lu, gpv, col, q_off, s_off, n0, n1, pg.nonce2, slot);
    else
        produce_raw_unit(p, src, pay, lu, gpv, col, q_off, n0, n1, pg.nonce2);
}

// Walks the payload's 64-byte chunks in MAC order, waiting for each unit's
// batch flags before its first chunk is read.
struct MacCursor {
    int32_t seg;
    uint32_t i;

    __device__ __forceinline__ void fetch(const EgressParams& p, const uint8_t* pay, int ppw,
                                          const uint32_t* done, uint4 (&x)[4]) {
        const MacSeg s = p.seg[seg];
        if (s.chunks_per_unit && i % (uint32_t)s.chunks_per_unit == 0u) {
            const int32_t u = s.unit0 + (int32_t)(i / (uint32_t)s.chunks_per_unit);
            const int32_t b0 = (u * ppw) / 64, b1 = (u * ppw + ppw - 1) / 64;
            wait_flag(&done[b0], p.state);
            if (b1 != b0) wait_flag(&done[b1], p.state);
        }
        const uint8_t* q = pay + s.off + 64u * i;
        x[0] = ldg16(q, 0); x[1] = ldg16(q, 1); x[2] = ldg16(q, 2); x[3] = ldg16(q, 3);
        if (++i == s.n) { ++seg; i = 0; }
    }
};

template <int DT>
__device__ void egress_mac(const EgressParams& p, int64_t page0, int ppw, const uint32_t* done) {
    const int lane = threadIdx.x & 63;
    const bool active = lane < ppw;
    const int64_t page = page0 + (active ? lane : 0);
    const EgressPage pg = egress_page(p, page);
    uint8_t* blob = pg.blob;
    if (active) {  // header (cpp:1129-1140)
        stg16(blob, 0, make_uint4((uint32_t)p.hdr0, (uint32_t)(p.hdr0 >> 32), (uint32_t)pg.hdr1,
                                  (uint32_t)(pg.hdr1 >> 32)));
        stg16(blob, 1, make_uint4((uint32_t)pg.token, (uint32_t)(pg.token >> 32), (uint32_t)pg.seq,
                                  (uint32_t)(pg.seq >> 32)));
    }
    Sip s;
    s.init(p.mk0, p.mk1);
    s.absorb(p.hdr0);
    s.absorb(pg.hdr1);
    s.absorb(pg.token);
    s.absorb(pg.seq);
    const uint8_t* pay = blob + kHeader;
    MacCursor cur{0, 0};
    sip_stream64(s, p.mac_chunks, [&](uint4 (&x)[4]) { cur.fetch(p, pay, ppw, done, x); });
    uint64_t lo, hi;
    s.finish((uint64_t)((kHeader + p.payload) & 0xFFu) << 56, lo, hi);
    if (active)
        stg16(blob + kHeader + p.payload, 0,
              make_uint4((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)));
}

// Dynamic LDS: scale staging for the producer waves (16 words x 64 lanes
// each), then one completion flag per batch.
constexpr int kStageWords = kProducerWaves * 16 * 64;

template <int DT>
__global__ __launch_bounds__(kFusedThreads) void egress_fused_kernel(EgressParams p) {
    extern __shared__ uint32_t lds[];
    uint32_t* done = lds + kStageWords;
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
    if ((wave & 3) == 0) return;  // leave the MAC wave's SIMD to it
    const int prod = wave - 1 - (wave >> 2);
    const int nprod = nwaves - 1 - ((nwaves - 1) >> 2);
    if (prod >= kProducerWaves) return;  // never: launched with kFusedWaves waves
    uint32_t* slot = lds + prod * 16 * 64 + lane;
#pragma unroll 1
    for (int b = prod; b < n_batches; b += nprod) {
        const int item = b * 64 + lane;
        if (item < items) {
            const int u = item / ppw;
            produce_unit<DT>(p, page0 + (item - u * ppw), u, slot);
        }
        __builtin_amdgcn_s_waitcnt(0);  // every store of this batch has completed
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0) __hip_atomic_store(&done[b], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}

hipError_t launch_egress_fused(const EgressParams& p, int dtype, hipStream_t s) {
    const int waves = kFusedWaves;
    const int64_t grid = (p.batch + p.ppw - 1) / p.ppw;
    const size_t lds = ((size_t)kStageWords + (size_t)p.n_batches) * sizeof(uint32_t);
    if (dtype == kHotBf16)
        hipLaunchKernelGGL(egress_fused_kernel<kHotBf16>, dim3((uint32_t)grid), dim3(64 * waves), lds, s, p);
    else
        hipLaunchKernelGGL(egress_fused_kernel<kHotFp16>, dim3((uint32_t)grid), dim3(64 * waves), lds, s, p);
    return hipGetLastError();
}

}  // namespace ztcp
