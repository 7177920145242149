// ztcp_capi_example.cpp -- a C++ caller of the C ABI in include/ztcp.h, as a
// serving stack would link it: no torch, plain device buffers from the HIP
// runtime.  Built next to libztcp_hip.so by vlx-tee_amd/build.py.
//
// Encodes 64 pages of 16 tokens x 4 KV heads x head_dim 128 (BF16, INT4_SYM +
// PRESERVE_FP8) twice, through the contiguous entry point and the descriptor
// form, checks that the blobs agree, decodes them, checks that a tampered
// blob is rejected with every output zeroed, and writes the blobs and the
// decoded K and V pages to the file named by argv[1] (for a comparison with
// an independent implementation).  Page values come from a 64-bit LCG
// (state * 6364136223846793005 + 1442695040888963407, seed 2024): element i
// takes the next state x and is the bf16 pattern sign = bit 63 of x, exponent
// 120 + (x >> 56) % 11, mantissa (x >> 40) & 0x7F; K first, then V.
// Exit status 0 on success; a message on stderr otherwise.
#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/ztcp.h"

namespace {

constexpr int64_t kPages = 64, kTokens = 16, kHeads = 4, kDim = 128, kRope = 64;
constexpr uint32_t kTenant = 0x1234ABCDu, kModel = 0x0BADF00Du;
constexpr uint16_t kLayer = 7, kHeadGroup = 1;
constexpr uint64_t kBaseSeq = 1000;

int fail(const char* what, int rc) {
    std::fprintf(stderr, "ztcp_capi_example: %s: %d (%s; %s)\n", what, rc, ztcp_strerror(rc), ztcp_last_error());
    return 1;
}

bool hip_ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    std::fprintf(stderr, "ztcp_capi_example: %s: %s\n", what, hipGetErrorString(e));
    return false;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s OUT_FILE\n", argv[0]);
        return 2;
    }
    const ztcp_geometry g{kTokens, kHeads, kDim, kRope, ZTCP_HOT_BF16, 0};
    const size_t payload = ztcp_payload_bytes(&g, ZTCP_INT4_SYM, ZTCP_PRESERVE_FP8);
    const size_t blob_bytes = ztcp_blob_bytes(&g, ZTCP_INT4_SYM, ZTCP_PRESERVE_FP8);
    if (payload == (size_t)-1 || blob_bytes != payload + ZTCP_HEADER_BYTES + ZTCP_TAG_BYTES) return fail("sizing", -1);
    const size_t elems = (size_t)(kPages * kTokens * kHeads * kDim);
    std::vector<uint16_t> hot(2 * elems);
    uint64_t x = 2024;
    for (auto& h : hot) {
        x = x * 6364136223846793005ull + 1442695040888963407ull;
        h = (uint16_t)(((x >> 63) << 15) | ((120u + (uint32_t)((x >> 56) % 11u)) << 7) | ((x >> 40) & 0x7Fu));
    }
    std::vector<int64_t> tok(kPages);
    for (int64_t i = 0; i < kPages; ++i) tok[i] = (int64_t)(0x9E3779B97F4A7C15ull * (uint64_t)(i + 1));
    const ztcp_keys keys{0x0706050403020100ull, 0x0F0E0D0C0B0A0908ull, 0x1716151413121110ull,
                         0x1F1E1D1C1B1A1918ull, 0x2726252423222120ull, 0x2F2E2D2C2B2A2928ull};
    const ztcp_aad aad{kTenant, kModel, kLayer, kHeadGroup};

    void *k = nullptr, *v = nullptr, *ko = nullptr, *vo = nullptr, *descs = nullptr;
    int64_t* dtok = nullptr;
    uint8_t *blobs = nullptr, *blobs2 = nullptr;
    int32_t* status = nullptr;
    const size_t page_bytes = elems / kPages * 2;
    if (!hip_ok(hipMalloc(&k, elems * 2), "hipMalloc") || !hip_ok(hipMalloc(&v, elems * 2), "hipMalloc") ||
        !hip_ok(hipMalloc(&ko, elems * 2), "hipMalloc") || !hip_ok(hipMalloc(&vo, elems * 2), "hipMalloc") ||
        !hip_ok(hipMalloc((void**)&dtok, sizeof(int64_t) * kPages), "hipMalloc") ||
        !hip_ok(hipMalloc((void**)&blobs, blob_bytes * kPages), "hipMalloc") ||
        !hip_ok(hipMalloc((void**)&blobs2, blob_bytes * kPages), "hipMalloc") ||
        !hip_ok(hipMalloc((void**)&status, sizeof(int32_t) * kPages), "hipMalloc") ||
        !hip_ok(hipMalloc(&descs, sizeof(ztcp_page_desc) * kPages), "hipMalloc"))
        return 1;
    if (!hip_ok(hipMemcpy(k, hot.data(), elems * 2, hipMemcpyHostToDevice), "hipMemcpy") ||
        !hip_ok(hipMemcpy(v, hot.data() + elems, elems * 2, hipMemcpyHostToDevice), "hipMemcpy") ||
        !hip_ok(hipMemcpy(dtok, tok.data(), sizeof(int64_t) * kPages, hipMemcpyHostToDevice), "hipMemcpy"))
        return 1;

    // contiguous batch (fused_encode_cold_pages_peak_into_cpu's arguments)
    int rc = ztcp_egress_peak_into(k, v, dtok, blobs, kPages, &g, ZTCP_INT4_SYM, ZTCP_PRESERVE_FP8, (int64_t)payload,
                                   &aad, kBaseSeq, &keys, nullptr);
    if (rc != ZTCP_OK) return fail("ztcp_egress_peak_into", rc);
    // the descriptor form with the same per-page fields
    std::vector<ztcp_page_desc> d(kPages);
    for (int64_t i = 0; i < kPages; ++i)
        d[i] = ztcp_page_desc{(char*)k + i * page_bytes, (char*)v + i * page_bytes, blobs2 + i * blob_bytes, tok[i],
                              kBaseSeq + (uint64_t)i, kLayer, kHeadGroup, 0u};
    if (!hip_ok(hipMemcpy(descs, d.data(), sizeof(ztcp_page_desc) * kPages, hipMemcpyHostToDevice), "hipMemcpy"))
        return 1;
    rc = ztcp_egress_batch((const ztcp_page_desc*)descs, kPages, &g, ZTCP_INT4_SYM, ZTCP_PRESERVE_FP8,
                           (int64_t)payload, kTenant, kModel, &keys, nullptr);
    if (rc != ZTCP_OK) return fail("ztcp_egress_batch", rc);
    std::vector<uint8_t> b1(blob_bytes * kPages), b2(blob_bytes * kPages);
    if (!hip_ok(hipMemcpy(b1.data(), blobs, b1.size(), hipMemcpyDeviceToHost), "hipMemcpy") ||
        !hip_ok(hipMemcpy(b2.data(), blobs2, b2.size(), hipMemcpyDeviceToHost), "hipMemcpy"))
        return 1;
    if (b1 != b2) return fail("contiguous and descriptor blobs differ", -1);

    rc = ztcp_ingress_peak_into(blobs, (int64_t)blob_bytes, dtok, ko, vo, kPages, &g, kTenant, kModel, kLayer, &keys,
                                status, 0u, nullptr);
    if (rc != ZTCP_OK) return fail("ztcp_ingress_peak_into", rc);
    std::vector<uint16_t> dec(2 * elems);
    if (!hip_ok(hipMemcpy(dec.data(), ko, elems * 2, hipMemcpyDeviceToHost), "hipMemcpy") ||
        !hip_ok(hipMemcpy(dec.data() + elems, vo, elems * 2, hipMemcpyDeviceToHost), "hipMemcpy"))
        return 1;

    // one flipped ciphertext bit of page 9: the MAC check rejects it, and the
    // reference's all-or-nothing policy zeroes every output
    uint8_t byte = 0;
    uint8_t* target = blobs2 + 9 * blob_bytes + ZTCP_HEADER_BYTES + 100;
    if (!hip_ok(hipMemcpy(&byte, target, 1, hipMemcpyDeviceToHost), "hipMemcpy")) return 1;
    byte ^= 0x20;
    if (!hip_ok(hipMemcpy(target, &byte, 1, hipMemcpyHostToDevice), "hipMemcpy")) return 1;
    rc = ztcp_ingress_peak_into(blobs2, (int64_t)blob_bytes, dtok, ko, vo, kPages, &g, kTenant, kModel, kLayer, &keys,
                                status, 0u, nullptr);
    if (rc != ZTCP_ERR_MAC) return fail("tampered ingress did not report ZTCP_ERR_MAC", rc);
    std::vector<uint16_t> zero(2 * elems, 0xFFFF);
    if (!hip_ok(hipMemcpy(zero.data(), ko, elems * 2, hipMemcpyDeviceToHost), "hipMemcpy") ||
        !hip_ok(hipMemcpy(zero.data() + elems, vo, elems * 2, hipMemcpyDeviceToHost), "hipMemcpy"))
        return 1;
    for (uint16_t z : zero)
        if (z) return fail("tampered ingress left nonzero outputs", -1);

    std::FILE* f = std::fopen(argv[1], "wb");
    if (!f) return fail("cannot open the output file", -1);
    const bool wrote = std::fwrite(b1.data(), 1, b1.size(), f) == b1.size() &&
                       std::fwrite(dec.data(), 2, dec.size(), f) == dec.size();
    if (std::fclose(f) != 0 || !wrote) return fail("cannot write the output file", -1);
    for (void* p : {k, v, ko, vo, descs, (void*)dtok, (void*)blobs, (void*)blobs2, (void*)status}) (void)hipFree(p);
    std::printf("ztcp_capi_example: %lld pages, %zu-byte blobs: contiguous == descriptor, round trip ok, "
                "tampered page rejected\n", (long long)kPages, blob_bytes);
    return 0;
}
