// ztcp_abi.hip -- host side of the C ABI declared in include/ztcp.h.
//
// Argument checks follow the reference's TORCH_CHECK lists
// (cpp:1925-1957 egress, cpp:2267-2296 ingress) and return ZTCP_EINVAL /
// ZTCP_EOVERLAP instead of raising.  Each call picks the fused kernels
// (ztcp_egress.hip / ztcp_ingress.hip) when the page layout is cut into whole
// 64-byte keystream blocks and every pointer is 16-byte aligned, otherwise
// the generic kernels (ztcp_generic.hip).
#include <mutex>
#include <vector>

#include "ztcp_params.h"

using namespace ztcp;

namespace {


struct DeviceCtx {
    DeviceState* state = nullptr;
    unsigned long long* host_fail = nullptr;  // pinned
    int32_t* status_scratch = nullptr;
    int64_t status_cap = 0;
    int cu_count = 0;
};

std::mutex g_mu;
std::vector<DeviceCtx> g_ctx;

// Per-device library state, created on the first call on that device.
int device_ctx(DeviceCtx** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return ZTCP_EHIP;
    std::lock_guard<std::mutex> lock(g_mu);
    if ((int)g_ctx.size() <= dev) g_ctx.resize(dev + 1);
    DeviceCtx& c = g_ctx[dev];
    if (!c.state) {
        DeviceState* st = nullptr;
        if (hipMalloc(&st, sizeof(DeviceState)) != hipSuccess) return ZTCP_EHIP;
        DeviceState init{};
        init.fail = ~0ull;
        if (hipMemcpy(st, &init, sizeof init, hipMemcpyHostToDevice) != hipSuccess) return ZTCP_EHIP;
        if (hipHostMalloc(&c.host_fail, sizeof(unsigned long long), hipHostMallocDefault) != hipSuccess)
            return ZTCP_EHIP;
        if (hipDeviceGetAttribute(&c.cu_count, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return ZTCP_EHIP;
        c.state = st;
    }
    *out = &c;
    return ZTCP_OK;
}

int status_scratch(DeviceCtx* c, int64_t n, int32_t** out) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (c->status_cap < n) {
        if (c->status_scratch) (void)hipFree(c->status_scratch);
        c->status_scratch = nullptr;
        c->status_cap = 0;
        if (hipMalloc(&c->status_scratch, (size_t)n * sizeof(int32_t)) != hipSuccess) return ZTCP_EHIP;
        c->status_cap = n;
    }
    *out = c->status_scratch;
    return ZTCP_OK;
}

bool geometry_ok(const ztcp_geometry* g) {  // cpp:1925-1935
    return g && g->num_tokens > 0 && g->num_heads > 0 && g->head_dim >= 16 && g->head_dim % 16 == 0 &&
           g->rope_dim >= 0 && g->rope_dim <= g->head_dim && g->rope_dim % 16 == 0 &&
           (g->hot_dtype == ZTCP_HOT_FP16 || g->hot_dtype == ZTCP_HOT_BF16) &&
           g->num_tokens * g->num_heads * g->head_dim < (int64_t)1 << 30;
}

bool overlap(const void* a, int64_t an, const void* b, int64_t bn) {  // cpp:1428-1437
    if (!a || !b || an <= 0 || bn <= 0) return false;
    const uintptr_t as = (uintptr_t)a, ae = as + (uintptr_t)an;
    const uintptr_t bs = (uintptr_t)b, be = bs + (uintptr_t)bn;
    return as < be && bs < ae;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

ChaKey key_words(const ztcp_keys* k) {  // cpp:85-100
    ChaKey key;
    const uint64_t w[4] = {k->k0, k->k1, k->k2, k->k3};
    for (int i = 0; i < 4; ++i) {
        key.w[2 * i] = (uint32_t)w[i];
        key.w[2 * i + 1] = (uint32_t)(w[i] >> 32);
    }
    return key;
}

int pages_per_group(int64_t batch, int cu_count) {
    int64_t ppw = (batch + cu_count - 1) / (cu_count > 0 ? cu_count : 1);
    if (ppw < 1) ppw = 1;
    if (ppw > 64) ppw = 64;
    return (int)ppw;
}

int egress_common(const void* k, const void* v, const int64_t* tok, uint8_t* blobs,
                  const ztcp_page_desc* descs, int64_t batch, const ztcp_geometry* g,
                  int64_t preset, int64_t rope_mode, int64_t expected_payload, const ztcp_aad* aad,
                  uint64_t base_seq, const ztcp_keys* keys, hipStream_t stream) {
    if (!geometry_ok(g) || batch <= 0 || !aad || !keys) return ZTCP_EINVAL;
    if (!flags_valid(preset, rope_mode)) return ZTCP_EINVAL;
    const int64_t vecs = g->num_tokens * g->num_heads;
    const bool has_v = descs ? !g->is_mla_single_buffer : (v != nullptr);
    Layout lay;
    if (!build_layout(preset, rope_mode, vecs, g->head_dim, g->rope_dim, has_v, lay)) return ZTCP_EINVAL;
    if (expected_payload < (int64_t)lay.required || expected_payload > ((int64_t)1 << 31))
        return ZTCP_EINVAL;  // cpp:1955-1957
    const int64_t blob_bytes = kHeader + expected_payload + kTag;
    const int64_t page_bytes = vecs * g->head_dim * 2;
    if (!descs) {
        if (!k || !tok || !blobs) return ZTCP_EINVAL;
        const int64_t out_n = blob_bytes * batch;  // cpp:1949-1951
        if (overlap(blobs, out_n, k, page_bytes * batch) || overlap(blobs, out_n, v, page_bytes * batch) ||
            overlap(blobs, out_n, tok, 8 * batch))
            return ZTCP_EOVERLAP;
    }
    DeviceCtx* ctx = nullptr;
    int rc = device_ctx(&ctx);
    if (rc) return rc;

    EgressParams p{};
    p.k = (const uint8_t*)k;
    p.v = (const uint8_t*)v;
    p.token_hashes = tok;
    p.blobs = blobs;
    p.descs = descs;
    p.batch = batch;
    p.page_bytes = page_bytes;
    p.vecs = (int32_t)vecs;
    p.head_dim = (int32_t)g->head_dim;
    p.payload = (uint32_t)expected_payload;
    p.blob_bytes = (uint32_t)blob_bytes;
    p.lay = lay;
    p.key = key_words(keys);
    p.mk0 = keys->mk0;
    p.mk1 = keys->mk1;
    const uint64_t flags = (uint64_t)((preset & 0x0F) | ((rope_mode & 0x0F) << 4));
    p.hdr0 = (uint64_t)kMagic | ((uint64_t)kVersion << 16) | (flags << 24) |
             ((uint64_t)aad->tenant_id_hash << 32);
    p.hdr1 = (uint64_t)aad->model_id_hash | ((uint64_t)aad->layer_id << 32) |
             ((uint64_t)aad->head_group_id << 48);
    p.nonce2 = ((uint32_t)aad->layer_id << 16) | (uint32_t)aad->head_group_id;  // cpp:108-109
    p.base_seq = base_seq;
    p.ppw = pages_per_group(batch, ctx->cu_count);
    p.state = ctx->state;

    const bool fast = lay.aligned && expected_payload == (int64_t)lay.required && blob_bytes % 16 == 0 &&
                      (descs || (aligned16(k) && aligned16(v) && aligned16(blobs)));
    hipError_t e = fast ? launch_egress_fused(p, g->hot_dtype, stream)
                        : launch_egress_generic(p, g->hot_dtype, stream);
    return e == hipSuccess ? ZTCP_OK : ZTCP_EHIP;
}

int ingress_common(const uint8_t* blobs, int64_t blob_bytes, const int64_t* tok, void* out_k,
                   void* out_v, const ztcp_page_desc* descs, int64_t batch, const ztcp_geometry* g,
                   uint32_t tenant, uint32_t model, uint16_t layer, const ztcp_keys* keys,
                   int32_t* page_status, uint32_t flags, hipStream_t stream) {
    if (!geometry_ok(g) || batch <= 0 || !keys) return ZTCP_EINVAL;
    if (blob_bytes <= (int64_t)(kHeader + kTag) || blob_bytes > ((int64_t)1 << 31)) return ZTCP_EINVAL;
    if ((flags & ZTCP_ASYNC) && !page_status) return ZTCP_EINVAL;
    const bool mla = g->is_mla_single_buffer != 0;
    const int64_t vecs = g->num_tokens * g->num_heads;
    const int64_t page_bytes = vecs * g->head_dim * 2;
    if (!descs) {
        if (!blobs || !tok || !out_k) return ZTCP_EINVAL;
        if (!mla && !out_v) return ZTCP_EINVAL;  // cpp:2288
        const int64_t kn = page_bytes * batch, bn = blob_bytes * batch;
        if (overlap(out_k, kn, blobs, bn) || overlap(out_k, kn, tok, 8 * batch) ||
            (!mla && (overlap(out_v, kn, blobs, bn) || overlap(out_v, kn, tok, 8 * batch) ||
                      overlap(out_k, kn, out_v, kn))))  // cpp:2283, cpp:2293-2294
            return ZTCP_EOVERLAP;
    }
    DeviceCtx* ctx = nullptr;
    int rc = device_ctx(&ctx);
    if (rc) return rc;

    IngressParams p{};
    p.blobs = blobs;
    p.token_hashes = tok;
    p.out_k = (uint8_t*)out_k;
    p.out_v = mla ? nullptr : (uint8_t*)out_v;
    p.descs = descs;
    p.page_status = page_status;
    p.batch = batch;
    p.page_bytes = page_bytes;
    p.vecs = (int32_t)vecs;
    p.head_dim = (int32_t)g->head_dim;
    p.blob_bytes = (uint32_t)blob_bytes;
    p.payload = (uint32_t)(blob_bytes - kHeader - kTag);
    p.rope_dim = (int32_t)g->rope_dim;
    p.has_v = mla ? 0 : 1;
    bool all_aligned = true;
    const bool ext = (flags & ZTCP_EXT_LAYOUTS) != 0;
    for (int preset = 1; preset <= (ext ? 6 : 3); ++preset) {
        for (int rm = 0; rm <= (ext ? 3 : 2); ++rm) {
            const int i = (preset - 1) * 4 + rm;
            Layout lay;
            // an extension layout whose groups do not divide the geometry is
            // simply not a valid header for it (status 1)
            if (!build_layout(preset, rm, vecs, g->head_dim, g->rope_dim, !mla, lay)) continue;
            if (p.payload >= lay.required) p.lay_ok |= 1u << i;
            all_aligned = all_aligned && lay.aligned;
        }
    }
    p.key = key_words(keys);
    p.mk0 = keys->mk0;
    p.mk1 = keys->mk1;
    p.exp_tenant = tenant;
    p.exp_model = model;
    p.exp_layer = layer;
    p.per_page = (flags & ZTCP_PER_PAGE) ? 1 : 0;
    p.state = ctx->state;
    p.ppw = pages_per_group(batch, ctx->cu_count);

    const bool fast = all_aligned && blob_bytes % 16 == 0 &&
                      (descs || (aligned16(blobs) && aligned16(out_k) && (mla || aligned16(out_v))));
    hipError_t e = launch_reset_fail(p.state, stream);
    if (e == hipSuccess) {
        if (fast) {
            e = launch_ingress_fused(p, g->hot_dtype, stream);
            if (e == hipSuccess && !p.per_page) e = launch_ingress_finalize(p, stream);
        } else {
            p.n_units = (int32_t)(vecs * (g->head_dim / 16) * (mla ? 1 : 2));  // groups per page
            int32_t* status = page_status;
            if (!status) {
                rc = status_scratch(ctx, batch, &status);
                if (rc) return rc;
            }
            e = launch_ingress_generic_impl(p, g->hot_dtype, status, stream);
        }
    }
    if (e != hipSuccess) return ZTCP_EHIP;
    if (flags & ZTCP_ASYNC) return ZTCP_OK;
    if (hipMemcpyAsync(ctx->host_fail, &p.state->fail, sizeof(unsigned long long), hipMemcpyDeviceToHost,
                       stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess)
        return ZTCP_EHIP;
    const unsigned long long f = *ctx->host_fail;
    return f == ~0ull ? ZTCP_OK : (int)(f & 0xFFu);
}

}  // namespace

extern "C" {

size_t ztcp_required_payload_bytes(const ztcp_geometry* g, int64_t preset, int64_t rope_mode) {
    if (!g) return (size_t)-1;
    Layout lay;
    if (!build_layout(preset, rope_mode, g->num_tokens * g->num_heads, g->head_dim, g->rope_dim,
                      !g->is_mla_single_buffer, lay))
        return (size_t)-1;
    return lay.required;
}

size_t ztcp_payload_bytes(const ztcp_geometry* g, int64_t preset, int64_t rope_mode) {
    const size_t r = ztcp_required_payload_bytes(g, preset, rope_mode);
    return r == (size_t)-1 ? r : ((r + 3u) & ~(size_t)3u);  // spec:244-246
}

size_t ztcp_blob_bytes(const ztcp_geometry* g, int64_t preset, int64_t rope_mode) {
    const size_t r = ztcp_payload_bytes(g, preset, rope_mode);
    return r == (size_t)-1 ? r : r + kHeader + kTag;
}

int ztcp_egress_peak_into(const void* k_pages, const void* v_pages, const int64_t* page_token_hashes,
                          uint8_t* out_blobs, int64_t batch, const ztcp_geometry* g, int64_t preset,
                          int64_t rope_mode, int64_t expected_payload_bytes, const ztcp_aad* aad,
                          uint64_t base_sequence_nonce, const ztcp_keys* keys, void* stream) {
    if (g && g->is_mla_single_buffer && v_pages) return ZTCP_EINVAL;
    return egress_common(k_pages, v_pages, page_token_hashes, out_blobs, nullptr, batch, g, preset,
                         rope_mode, expected_payload_bytes, aad, base_sequence_nonce, keys,
                         (hipStream_t)stream);
}

int ztcp_egress_batch(const ztcp_page_desc* pages, int64_t n_pages, const ztcp_geometry* g,
                      int64_t preset, int64_t rope_mode, int64_t expected_payload_bytes,
                      uint32_t tenant_id_hash, uint32_t model_id_hash, const ztcp_keys* keys,
                      void* stream) {
    if (!pages) return ZTCP_EINVAL;
    const ztcp_aad aad{tenant_id_hash, model_id_hash, 0, 0};  // layer / head group per page
    return egress_common(nullptr, nullptr, nullptr, nullptr, pages, n_pages, g, preset, rope_mode,
                         expected_payload_bytes, &aad, 0, keys, (hipStream_t)stream);
}

int ztcp_ingress_peak_into(const uint8_t* cold_blobs, int64_t blob_bytes,
                           const int64_t* expected_token_hashes, void* out_k_pages, void* out_v_pages,
                           int64_t batch, const ztcp_geometry* g, uint32_t expected_tenant_hash,
                           uint32_t expected_model_hash, uint16_t expected_layer_id,
                           const ztcp_keys* keys, int32_t* page_status, uint32_t flags, void* stream) {
    return ingress_common(cold_blobs, blob_bytes, expected_token_hashes, out_k_pages, out_v_pages, nullptr,
                          batch, g, expected_tenant_hash, expected_model_hash, expected_layer_id, keys,
                          page_status, flags, (hipStream_t)stream);
}

int ztcp_ingress_batch(const ztcp_page_desc* pages, int64_t n_pages, int64_t blob_bytes,
                       const ztcp_geometry* g, uint32_t expected_tenant_hash, uint32_t expected_model_hash,
                       const ztcp_keys* keys, int32_t* page_status, uint32_t flags, void* stream) {
    if (!pages) return ZTCP_EINVAL;
    return ingress_common(nullptr, blob_bytes, nullptr, nullptr, nullptr, pages, n_pages, g,
                          expected_tenant_hash, expected_model_hash, 0, keys, page_status, flags,
                          (hipStream_t)stream);
}

int ztcp_chacha20_xor(const uint8_t* src, uint8_t* dst, size_t len, const uint8_t key[32],
                      uint32_t initial_counter, const uint8_t nonce[12], void* stream) {
    if (!key || !nonce || (len && (!src || !dst))) return ZTCP_EINVAL;
    if (len == 0) return ZTCP_OK;
    ChaKey k;
    uint32_t n[3];
    for (int i = 0; i < 8; ++i)
        k.w[i] = (uint32_t)key[4 * i] | ((uint32_t)key[4 * i + 1] << 8) | ((uint32_t)key[4 * i + 2] << 16) |
                 ((uint32_t)key[4 * i + 3] << 24);
    for (int i = 0; i < 3; ++i)
        n[i] = (uint32_t)nonce[4 * i] | ((uint32_t)nonce[4 * i + 1] << 8) |
               ((uint32_t)nonce[4 * i + 2] << 16) | ((uint32_t)nonce[4 * i + 3] << 24);
    return launch_chacha_xor(src, dst, len, k, initial_counter, n[0], n[1], n[2], (hipStream_t)stream) ==
                   hipSuccess
               ? ZTCP_OK
               : ZTCP_EHIP;
}

int ztcp_siphash128(const uint8_t* data, size_t len, uint64_t mk0, uint64_t mk1, uint8_t* tag16,
                    void* stream) {
    if (!tag16 || (len && !data)) return ZTCP_EINVAL;
    return launch_siphash(data, len, mk0, mk1, tag16, (hipStream_t)stream) == hipSuccess ? ZTCP_OK
                                                                                       : ZTCP_EHIP;
}

int ztcp_selftest(void) {
    unsigned int* bad = nullptr;
    if (hipMalloc(&bad, sizeof(unsigned int)) != hipSuccess) return ZTCP_EHIP;
    unsigned int h = 0;
    int rc = ZTCP_OK;
    if (hipMemcpy(bad, &h, sizeof h, hipMemcpyHostToDevice) != hipSuccess ||
        launch_selftest(bad, nullptr) != hipSuccess ||
        hipMemcpy(&h, bad, sizeof h, hipMemcpyDeviceToHost) != hipSuccess)
        rc = ZTCP_EHIP;
    (void)hipFree(bad);
    return rc == ZTCP_OK ? (int)h : rc;
}

int ztcp_device_diag(void) {
    DeviceCtx* ctx = nullptr;
    int rc = device_ctx(&ctx);
    if (rc) return rc;
    uint32_t d = 0;
    if (hipDeviceSynchronize() != hipSuccess) return ZTCP_EHIP;
    if (hipMemcpy(&d, &ctx->state->diag, sizeof d, hipMemcpyDeviceToHost) != hipSuccess) return ZTCP_EHIP;
    const uint32_t zero = 0;
    if (hipMemcpy(&ctx->state->diag, &zero, sizeof zero, hipMemcpyHostToDevice) != hipSuccess)
        return ZTCP_EHIP;
    return (int)d;
}

const char* ztcp_strerror(int code) {
    switch (code) {
        case ZTCP_OK: return "ok";
        case ZTCP_ERR_HEADER: return "KV_INTEGRITY_ERROR: Invalid cold-page header magic, version, or flags";
        case ZTCP_ERR_AAD: return "CROSS_TENANT_CONTAMINATION: Cold-page AAD mismatch";
        case ZTCP_ERR_MAC: return "KV_INTEGRITY_ERROR: Cold-page MAC verification failed";
        case ZTCP_EINVAL: return "invalid argument";
        case ZTCP_EOVERLAP: return "outputs must not alias or overlap input tensors";
        case ZTCP_EHIP: return "HIP runtime error";
        case ZTCP_EDEVICE: return "device-side bounded wait expired";
        default: return "unknown error";
    }
}

}  // extern "C"
