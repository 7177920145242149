// ztcp_abi.hip -- host side of the C ABI declared in include/ztcp.h.
//
// Argument checks follow the reference's TORCH_CHECK lists
// (cpp:1925-1957 egress, cpp:2267-2296 ingress) and return ZTCP_EINVAL /
// ZTCP_EOVERLAP instead of raising.  Each call picks the fused kernels
// (ztcp_egress.hip / ztcp_ingress.hip) when the page layout is cut into whole
// 64-byte keystream blocks and every pointer is 16-byte aligned, otherwise
// the generic kernels (ztcp_generic.hip).
#include <atomic>
#include <mutex>
#include <thread>
#include <vector>

#include "ztcp_params.h"
#include "ztcp_rows.h"
#ifdef ZTCP_PHASE_TIMERS
#include "../../include/ztcp_timers.h"
#endif

using namespace ztcp;

namespace {

// Per-call ingress state: a pool of CallState slots per device.  A call takes
// a free slot for its duration; a synchronous call returns it after reading
// the verdict, an asynchronous one records an event after its last kernel and
// the slot is free again once that event has completed.
constexpr int kCallSlots = 64;

struct DeviceCtx {
    DeviceState* state = nullptr;      // sticky diagnostics (ztcp_device_diag)
    CallState* calls = nullptr;        // [kCallSlots], device
    CallState* host_calls = nullptr;   // [kCallSlots], pinned: verdict read-back
    hipEvent_t done[kCallSlots] = {};
    bool busy[kCallSlots] = {};        // taken by a call
    bool pending[kCallSlots] = {};     // released by an asynchronous call: free once done[k] completes
    bool poisoned[kCallSlots] = {};    // lost to a failed release (its stream may still write it)
    int next = 0;
    int cu_count = 0;
    uint32_t egress_tag = 15;          // last egress call tag (WaitSink::call_tag), 16 and up
};

std::mutex g_mu;                       // guards g_ctx and every DeviceCtx's slot bookkeeping
std::vector<DeviceCtx*> g_ctx;
std::atomic<uint32_t> g_spin_limit{kSpinLimit};
thread_local const char* t_last_error = "";

int fail_arg(int rc, const char* why) {
    t_last_error = why;
    return rc;
}

// Per-device library state, created on the first call on that device.
int device_ctx(DeviceCtx** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return ZTCP_EHIP;
    std::lock_guard<std::mutex> lock(g_mu);
    if ((int)g_ctx.size() <= dev) g_ctx.resize(dev + 1, nullptr);
    if (!g_ctx[dev]) {
        DeviceCtx* c = new DeviceCtx();
        const DeviceState init{};
        bool ok = hipMalloc(&c->state, sizeof(DeviceState)) == hipSuccess &&
                  hipMemcpy(c->state, &init, sizeof init, hipMemcpyHostToDevice) == hipSuccess &&
                  hipMalloc(&c->calls, sizeof(CallState) * kCallSlots) == hipSuccess &&
                  hipHostMalloc(&c->host_calls, sizeof(CallState) * kCallSlots, hipHostMallocDefault) == hipSuccess &&
                  hipDeviceGetAttribute(&c->cu_count, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess;
        // A slot's event only tells the host that the device is done with the
        // slot's CallState, which only later device work touches: a device-scope
        // release suffices, and spares each asynchronous call the system-scope
        // fence (an L2 writeback and invalidate on every XCD).
        for (int i = 0; ok && i < kCallSlots; ++i)
            ok = hipEventCreateWithFlags(&c->done[i], hipEventDisableTiming | hipEventReleaseToDevice) == hipSuccess;
        if (!ok) return ZTCP_EHIP;  // the partial context is left unused (one per device, process lifetime)
        g_ctx[dev] = c;
    }
    *out = g_ctx[dev];
    return ZTCP_OK;
}

// A free call slot: one never used, released by a synchronous call, or
// released by an asynchronous call whose event has completed.  A slot held by
// a call still in progress is never handed out (its event is stale then).
// When every slot is taken, waits for an asynchronous call to complete, or,
// when synchronous calls in progress hold them all, for one of those to end;
// when every slot is lost to failed releases, returns ZTCP_EHIP.
int acquire_call(DeviceCtx* c, int* slot) {
    std::unique_lock<std::mutex> lock(g_mu);
    for (;;) {
        int wait_on = -1, held = 0;
        for (int i = 0; i < kCallSlots; ++i) {
            const int k = (c->next + i) % kCallSlots;
            if (c->poisoned[k]) continue;
            if (c->busy[k]) {
                if (!c->pending[k]) {  // a call still holds it
                    ++held;
                    continue;
                }
                const hipError_t q = hipEventQuery(c->done[k]);
                if (q == hipErrorNotReady) {
                    if (wait_on < 0) wait_on = k;
                    continue;
                }
                if (q != hipSuccess) return ZTCP_EHIP;
            }
            c->busy[k] = true;
            c->pending[k] = false;
            c->next = (k + 1) % kCallSlots;
            *slot = k;
            return ZTCP_OK;
        }
        if (wait_on < 0 && held == 0) return fail_arg(ZTCP_EHIP, "every call slot of the device is lost to failed releases");
        lock.unlock();
        if (wait_on >= 0) {
            if (hipEventSynchronize(c->done[wait_on]) != hipSuccess) return ZTCP_EHIP;
        } else {
            std::this_thread::yield();
        }
        lock.lock();
    }
}

// Asynchronous release: the slot is free once the work enqueued on `stream`
// so far has completed.  Synchronous release: free now.
int release_call(DeviceCtx* c, int slot, hipStream_t stream, bool async) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (async) {
        if (hipEventRecord(c->done[slot], stream) == hipSuccess) {
            c->pending[slot] = true;
            return ZTCP_OK;
        }
        // The event did not record: wait for the stream instead.  If that
        // fails too, the slot's kernels may still write it: it stays out of
        // use for good (acquire_call skips it and fails once all are lost).
        if (hipStreamSynchronize(stream) != hipSuccess) {
            c->poisoned[slot] = true;
            return ZTCP_EHIP;
        }
    }
    c->busy[slot] = false;
    c->pending[slot] = false;
    return ZTCP_OK;
}

#ifdef ZTCP_PHASE_TIMERS
// Phase-timer records of the last fused launch per direction (diagnostic
// build only): one buffer per direction, on the device of the first launch.
static_assert(kTimerSlots == ZTCP_TIMER_SLOTS && kTimerMaxWg == ZTCP_TIMER_MAX_WORKGROUPS &&
                  kTraceRows == ZTCP_TRACE_ROWS, "timer record size");
unsigned long long* g_timer_buf[2] = {nullptr, nullptr};
int64_t g_timer_wgs[2] = {0, 0};
unsigned long long* timer_record(int dir, int64_t grid) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (grid > ZTCP_TIMER_MAX_WORKGROUPS) return nullptr;
    if (!g_timer_buf[dir] &&
        hipMalloc(&g_timer_buf[dir], sizeof(unsigned long long) * (kTimerSlots * ZTCP_TIMER_MAX_WORKGROUPS +
                                                                     2 * kTraceRows)) != hipSuccess)
        return g_timer_buf[dir] = nullptr;
    g_timer_wgs[dir] = grid;
    return g_timer_buf[dir];
}
#else
unsigned long long* timer_record(int, int64_t) { return nullptr; }
#endif

WaitSink wait_sink(DeviceCtx* c, CallState* call) {
    return WaitSink{&c->state->diag, call ? &call->diag : nullptr, g_spin_limit.load(std::memory_order_relaxed)};
}

// The reference's dimension checks (cpp:1934-1935 egress, cpp:2277-2278
// ingress) with its messages; `what` names the page tensor.
int check_geometry(const ztcp_geometry* g, int64_t batch, const char* dims_msg) {
    if (!g) return fail_arg(ZTCP_EINVAL, "geometry must not be NULL");
    if (!(batch > 0 && g->num_tokens > 0 && g->num_heads > 0 && g->head_dim >= 16 && g->head_dim % 16 == 0))
        return fail_arg(ZTCP_EINVAL, dims_msg);
    if (!(g->rope_dim >= 0 && g->rope_dim <= g->head_dim && g->rope_dim % 16 == 0))
        return fail_arg(ZTCP_EINVAL, "Invalid rope_dim");
    if (g->hot_dtype != ZTCP_HOT_FP16 && g->hot_dtype != ZTCP_HOT_BF16)
        return fail_arg(ZTCP_EINVAL, "hot_dtype must be ZTCP_HOT_FP16 or ZTCP_HOT_BF16");
    if (g->num_tokens * g->num_heads * g->head_dim >= (int64_t)1 << 30)
        return fail_arg(ZTCP_EINVAL, "page too large (num_tokens * num_heads * head_dim must be below 2^30)");
    return ZTCP_OK;
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
                  uint64_t base_seq, const ztcp_keys* keys, uint32_t flags, hipStream_t stream) {
    t_last_error = "";
    // the reference's order (cpp:1934-1957): dimensions, overlaps, preset and
    // RoPE mode, payload size
    int rc = check_geometry(g, batch, "Invalid k_pages dimensions");
    if (rc) return rc;
    if (!aad || !keys) return fail_arg(ZTCP_EINVAL, "aad and keys must not be NULL");
    const int64_t blob_bytes = kHeader + expected_payload + kTag;
    const int64_t vecs = g->num_tokens * g->num_heads;
    const int64_t page_bytes = vecs * g->head_dim * 2;
    if (!descs) {
        if (!k || !blobs) return fail_arg(ZTCP_EINVAL, "k_pages and out_blobs must not be NULL");
        if (!tok) return fail_arg(ZTCP_EINVAL, "page_token_hashes must not be NULL");
        const int64_t out_n = blob_bytes * batch;  // cpp:1940, cpp:1949-1951
        if (overlap(blobs, out_n, k, page_bytes * batch) || overlap(blobs, out_n, tok, 8 * batch))
            return fail_arg(ZTCP_EOVERLAP, "out_blobs must not alias or overlap input tensors");
        if (overlap(blobs, out_n, v, page_bytes * batch))
            return fail_arg(ZTCP_EOVERLAP, "out_blobs must not alias or overlap v_pages");
    }
    // cpp:1952-1953; the extension presets only when the call asks for them
    const bool ext = (flags & ZTCP_EXT_LAYOUTS) != 0;
    if (preset < 1 || preset > (ext ? 6 : 3))
        return fail_arg(ZTCP_EINVAL, ext ? "Invalid preset (must be 1..6)" : "Invalid preset (must be 1..3)");
    if (rope_mode < 0 || rope_mode > (ext ? 3 : 2))
        return fail_arg(ZTCP_EINVAL, ext ? "Invalid rope_mode (must be 0..3)" : "Invalid rope_mode (must be 0..2)");
    const bool has_v = descs ? !g->is_mla_single_buffer : (v != nullptr);
    Layout lay;
    if (!build_layout(preset, rope_mode, vecs, g->head_dim, g->rope_dim, has_v, lay))
        return fail_arg(ZTCP_EINVAL, "head_dim / rope_dim not divisible by the extension preset's group size");
    if (expected_payload < (int64_t)lay.required)
        return fail_arg(ZTCP_EINVAL, "expected_payload_bytes smaller than required payload");  // cpp:1955-1957
    if (expected_payload > ((int64_t)1 << 31))
        return fail_arg(ZTCP_EINVAL, "expected_payload_bytes too large (at most 2^31)");
    DeviceCtx* ctx = nullptr;
    rc = device_ctx(&ctx);
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
    const uint64_t hflags = (uint64_t)((preset & 0x0F) | ((rope_mode & 0x0F) << 4));
    p.hdr0 = (uint64_t)kMagic | ((uint64_t)kVersion << 16) | (hflags << 24) |
             ((uint64_t)aad->tenant_id_hash << 32);
    p.hdr1 = (uint64_t)aad->model_id_hash | ((uint64_t)aad->layer_id << 32) |
             ((uint64_t)aad->head_group_id << 48);
    p.nonce2 = ((uint32_t)aad->layer_id << 16) | (uint32_t)aad->head_group_id;  // cpp:108-109
    p.base_seq = base_seq;
    p.ppw = pages_per_group(batch, ctx->cu_count);

    const bool fast = lay.aligned && expected_payload == (int64_t)lay.required && blob_bytes % 16 == 0 &&
                      (descs || (aligned16(k) && aligned16(v) && aligned16(blobs)));
    const bool async = (flags & ZTCP_ASYNC) != 0;
    if (!fast) {  // the generic kernels have no hand-offs, hence no bounded waits
        p.sink = wait_sink(ctx, nullptr);
        const hipError_t e = launch_egress_generic(p, g->hot_dtype, stream);
        if (e == hipSuccess && !async && hipStreamSynchronize(stream) != hipSuccess) return ZTCP_EHIP;
        return e == hipSuccess ? ZTCP_OK : ZTCP_EHIP;
    }
    // The fused kernel reports an expired bounded wait into this call's slot,
    // raising its diag word to the call's tag (no reset kernel needed).
    int slot = 0;
    rc = acquire_call(ctx, &slot);
    if (rc) return rc;
    CallState* call = ctx->calls + slot;
    uint32_t tag;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        tag = ctx->egress_tag = ctx->egress_tag == 0xFFFFFFFFu ? 16u : ctx->egress_tag + 1u;
    }
    p.sink = wait_sink(ctx, call);
    p.sink.call_tag = tag;
    p.timers = timer_record(0, (batch + p.ppw - 1) / p.ppw);
    hipError_t e = launch_egress_fused(p, g->hot_dtype, stream);
    if (e == hipSuccess && !async) e = hipMemcpyAsync(ctx->host_calls + slot, call, sizeof(CallState),
                                                      hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess && !async) e = hipStreamSynchronize(stream);
    const bool expired = e == hipSuccess && !async && ctx->host_calls[slot].diag == tag;
    if (expired) {  // fail closed: every blob of the call is zeroed before the call returns
        e = launch_egress_zero_blobs(p, stream);
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
    }
    const int rel = release_call(ctx, slot, stream, async || e != hipSuccess);
    if (e != hipSuccess) return ZTCP_EHIP;
    if (rel) return rel;
    return expired ? ZTCP_EDEVICE : ZTCP_OK;
}

// An ingress call's validated parameters: the reference's argument checks
// (cpp:2267-2296) and the kernel argument block, without any device state.
struct IngressCall {
    IngressParams p{};
    int dtype = 0;
    bool fast = false;
    bool async = false;
};

int ingress_prepare(const uint8_t* blobs, int64_t blob_bytes, const int64_t* tok, void* out_k, void* out_v,
                    const ztcp_page_desc* descs, int64_t batch, const ztcp_geometry* g, uint32_t tenant,
                    uint32_t model, uint16_t layer, const ztcp_keys* keys, int32_t* page_status, uint32_t flags,
                    int cu_count, IngressCall* out) {
    t_last_error = "";
    int rc = check_geometry(g, batch, "Invalid out_k_pages dimensions");
    if (rc) return rc;
    if (!keys) return fail_arg(ZTCP_EINVAL, "keys must not be NULL");
    if (blob_bytes <= (int64_t)(kHeader + kTag)) return fail_arg(ZTCP_EINVAL, "cold_blob too small");  // cpp:2282
    if (blob_bytes > ((int64_t)1 << 31)) return fail_arg(ZTCP_EINVAL, "cold_blob too large (at most 2^31 bytes)");
    if ((flags & ZTCP_ASYNC) && !page_status)
        return fail_arg(ZTCP_EINVAL, "ZTCP_ASYNC needs page_status (the verdicts' only destination)");
    const bool mla = g->is_mla_single_buffer != 0;
    const int64_t vecs = g->num_tokens * g->num_heads;
    const int64_t page_bytes = vecs * g->head_dim * 2;
    if (!descs) {
        if (!blobs || !out_k) return fail_arg(ZTCP_EINVAL, "cold_blobs and out_k_pages must not be NULL");
        if (!tok) return fail_arg(ZTCP_EINVAL, "expected_token_hashes must not be NULL");
        const int64_t kn = page_bytes * batch, bn = blob_bytes * batch;
        if (overlap(out_k, kn, blobs, bn) || overlap(out_k, kn, tok, 8 * batch))  // cpp:2283
            return fail_arg(ZTCP_EOVERLAP, "out_k_pages must not alias or overlap input tensors");
        if (!mla && !out_v) return fail_arg(ZTCP_EINVAL, "out_v_pages is required for non-MLA geometry");  // cpp:2288
        if (!mla && overlap(out_k, kn, out_v, kn))  // cpp:2292
            return fail_arg(ZTCP_EOVERLAP, "out_k_pages and out_v_pages must not alias or overlap in memory");
        if (!mla && (overlap(out_v, kn, blobs, bn) || overlap(out_v, kn, tok, 8 * batch)))  // cpp:2293-2294
            return fail_arg(ZTCP_EOVERLAP, "out_v_pages must not alias or overlap input tensors");
    }
    IngressParams& p = out->p;
    p = IngressParams{};
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
    p.ppw = pages_per_group(batch, cu_count);
    p.n_units = (int32_t)(vecs * (g->head_dim / 16) * (mla ? 1 : 2));  // generic path: groups per page
    out->dtype = g->hot_dtype;
    out->async = (flags & ZTCP_ASYNC) != 0;
    out->fast = all_aligned && blob_bytes % 16 == 0 &&
                (descs || (aligned16(blobs) && aligned16(out_k) && (mla || aligned16(out_v))));
    return ZTCP_OK;
}

// Enqueues an ingress call whose CallState is `call`: reset, kernels,
// finalize, and for a synchronous call the verdict's read-back into
// `result`.  `status` is the per-page status array of the generic path when
// the caller gave none (nullptr: a stream-ordered allocation of its own).
hipError_t ingress_enqueue(IngressCall& c, CallState* call, int32_t* status, const WaitSink& sink,
                           CallState* result, hipStream_t stream) {
    IngressParams& p = c.p;
    p.call = call;
    p.sink = sink;
    if (p.page_status) status = p.page_status;
    bool own_status = false;
    hipError_t e = launch_reset_call(call, stream);
    if (e == hipSuccess && !c.fast && !status) {
        e = hipMallocAsync((void**)&status, (size_t)p.batch * sizeof(int32_t), stream);
        own_status = e == hipSuccess;
    }
    if (e == hipSuccess) {
        if (c.fast) p.timers = timer_record(1, (p.batch + p.ppw - 1) / p.ppw);
        e = c.fast ? launch_ingress_fused(p, c.dtype, stream) : launch_ingress_generic_impl(p, c.dtype, status, stream);
        if (e == hipSuccess && c.fast && !p.per_page) e = launch_ingress_finalize(p, stream);
    }
    if (own_status && hipFreeAsync(status, stream) != hipSuccess && e == hipSuccess) e = hipErrorUnknown;
    if (e == hipSuccess && !c.async) e = hipMemcpyAsync(result, call, sizeof(CallState), hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess && !c.async) e = hipStreamSynchronize(stream);
    return e;
}

int verdict(const CallState& r) {
    if (r.diag) return ZTCP_EDEVICE;
    return r.fail == ~0ull ? ZTCP_OK : (int)(r.fail & 0xFFu);
}

int ingress_common(const uint8_t* blobs, int64_t blob_bytes, const int64_t* tok, void* out_k,
                   void* out_v, const ztcp_page_desc* descs, int64_t batch, const ztcp_geometry* g,
                   uint32_t tenant, uint32_t model, uint16_t layer, const ztcp_keys* keys,
                   int32_t* page_status, uint32_t flags, hipStream_t stream) {
    DeviceCtx* ctx = nullptr;
    IngressCall c;
    int rc = ingress_prepare(blobs, blob_bytes, tok, out_k, out_v, descs, batch, g, tenant, model, layer, keys,
                             page_status, flags, 0, &c);
    if (rc) return rc;
    rc = device_ctx(&ctx);
    if (rc) return rc;
    c.p.ppw = pages_per_group(batch, ctx->cu_count);
    int slot = 0;
    rc = acquire_call(ctx, &slot);
    if (rc) return rc;
    CallState* call = ctx->calls + slot;
    const hipError_t e = ingress_enqueue(c, call, nullptr, wait_sink(ctx, call), ctx->host_calls + slot, stream);
    // read the verdict while the slot (and its read-back area) is still ours
    const CallState r = (e == hipSuccess && !c.async) ? ctx->host_calls[slot] : CallState{~0ull, 0u, 0u};
    // a failed launch leaves the slot to an event, as the kernels before it
    // may still run
    const int rel = release_call(ctx, slot, stream, c.async || e != hipSuccess);
    if (e != hipSuccess) return ZTCP_EHIP;
    if (rel) return rel;
    return c.async ? ZTCP_OK : verdict(r);
}

// ---------------------------------------------------------------------------
// Ingress without allocation (ztcp_ingress_peak_into_noalloc): the call's
// device state lives in `scratch`, a file-scope device array each GPU holds
// one copy of until the process ends, instead of the per-device slot pool
// and the stream-ordered status allocation.
//   [0, 16)                      CallState (failure word, diagnostics)
//   [16, 32)                     DeviceState (sticky diagnostics of this path)
//   [256, 256 + 4 * kNoAllocPages)  per-page status of the generic path
// Every call on a GPU uses the same array: calls that overlap on one GPU
// race, and the array keeps the last call's contents (the call state is
// reset by the call's first kernel).
// ---------------------------------------------------------------------------
constexpr int64_t kNoAllocPages = ZTCP_NOALLOC_MAX_PAGES;
constexpr size_t kScratchStatusOff = 256;
constexpr size_t kScratchBytes = kScratchStatusOff + sizeof(int32_t) * (size_t)kNoAllocPages;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
static_assert(sizeof(CallState) == 16 && sizeof(DeviceState) == 16, "scratch layout");

constexpr int kMaxDevices = 64;
struct NoAllocDevice {
    unsigned char* scratch = nullptr;  // this device's copy of `scratch` (hipGetSymbolAddress)
    int cu_count = 0;
};
NoAllocDevice g_noalloc[kMaxDevices];
std::mutex g_noalloc_mu;

// Once per device, with that device current: the device address of its copy
// of `scratch`.  The array's name is a host-side stand-in, never passed to a
// kernel or copy; only this address is.
int noalloc_device(NoAllocDevice** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return ZTCP_EHIP;
    if (dev < 0 || dev >= kMaxDevices) return fail_arg(ZTCP_EINVAL, "device index out of range for the no-allocation path");
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    NoAllocDevice& d = g_noalloc[dev];
    if (!d.scratch) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return ZTCP_EHIP;
        if (hipDeviceGetAttribute(&d.cu_count, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return ZTCP_EHIP;
        d.scratch = (unsigned char*)ptr;
    }
    *out = &d;
    return ZTCP_OK;
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

int ztcp_egress_peak_into_ext(const void* k_pages, const void* v_pages, const int64_t* page_token_hashes,
                              uint8_t* out_blobs, int64_t batch, const ztcp_geometry* g, int64_t preset,
                              int64_t rope_mode, int64_t expected_payload_bytes, const ztcp_aad* aad,
                              uint64_t base_sequence_nonce, const ztcp_keys* keys, uint32_t flags,
                              void* stream) {
    if (g && g->is_mla_single_buffer && v_pages)
        return fail_arg(ZTCP_EINVAL, "v_pages must be NULL for an MLA single-buffer geometry");
    return egress_common(k_pages, v_pages, page_token_hashes, out_blobs, nullptr, batch, g, preset,
                         rope_mode, expected_payload_bytes, aad, base_sequence_nonce, keys, flags,
                         (hipStream_t)stream);
}

int ztcp_egress_peak_into(const void* k_pages, const void* v_pages, const int64_t* page_token_hashes,
                          uint8_t* out_blobs, int64_t batch, const ztcp_geometry* g, int64_t preset,
                          int64_t rope_mode, int64_t expected_payload_bytes, const ztcp_aad* aad,
                          uint64_t base_sequence_nonce, const ztcp_keys* keys, void* stream) {
    return ztcp_egress_peak_into_ext(k_pages, v_pages, page_token_hashes, out_blobs, batch, g, preset, rope_mode,
                                     expected_payload_bytes, aad, base_sequence_nonce, keys, 0u, stream);
}

int ztcp_egress_batch_ext(const ztcp_page_desc* pages, int64_t n_pages, const ztcp_geometry* g,
                          int64_t preset, int64_t rope_mode, int64_t expected_payload_bytes,
                          uint32_t tenant_id_hash, uint32_t model_id_hash, const ztcp_keys* keys,
                          uint32_t flags, void* stream) {
    if (!pages) return fail_arg(ZTCP_EINVAL, "pages must not be NULL");
    const ztcp_aad aad{tenant_id_hash, model_id_hash, 0, 0};  // layer / head group per page
    return egress_common(nullptr, nullptr, nullptr, nullptr, pages, n_pages, g, preset, rope_mode,
                         expected_payload_bytes, &aad, 0, keys, flags, (hipStream_t)stream);
}

int ztcp_egress_batch(const ztcp_page_desc* pages, int64_t n_pages, const ztcp_geometry* g,
                      int64_t preset, int64_t rope_mode, int64_t expected_payload_bytes,
                      uint32_t tenant_id_hash, uint32_t model_id_hash, const ztcp_keys* keys,
                      void* stream) {
    return ztcp_egress_batch_ext(pages, n_pages, g, preset, rope_mode, expected_payload_bytes, tenant_id_hash,
                                 model_id_hash, keys, 0u, stream);
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
    if (!pages) return fail_arg(ZTCP_EINVAL, "pages must not be NULL");
    return ingress_common(nullptr, blob_bytes, nullptr, nullptr, nullptr, pages, n_pages, g,
                          expected_tenant_hash, expected_model_hash, 0, keys, page_status, flags,
                          (hipStream_t)stream);
}

int ztcp_ingress_peak_into_noalloc(const uint8_t* cold_blobs, int64_t blob_bytes,
                                   const int64_t* expected_token_hashes, void* out_k_pages, void* out_v_pages,
                                   int64_t batch, const ztcp_geometry* g, uint32_t expected_tenant_hash,
                                   uint32_t expected_model_hash, uint16_t expected_layer_id,
                                   const ztcp_keys* keys, int32_t* page_status, uint32_t flags, void* stream) {
    if (batch > kNoAllocPages)
        return fail_arg(ZTCP_ESCRATCH, "batch exceeds ZTCP_NOALLOC_MAX_PAGES (the no-allocation scratch capacity)");
    // a synchronous call copies its verdict to the host and waits for the
    // stream, neither of which a stream under capture allows
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing((hipStream_t)stream, &cap) != hipSuccess) return ZTCP_EHIP;
    if (cap != hipStreamCaptureStatusNone && !(flags & ZTCP_ASYNC))
        return fail_arg(ZTCP_EINVAL, "a stream under capture needs ZTCP_ASYNC (verdicts in page_status)");
    IngressCall c;
    int rc = ingress_prepare(cold_blobs, blob_bytes, expected_token_hashes, out_k_pages, out_v_pages, nullptr, batch,
                             g, expected_tenant_hash, expected_model_hash, expected_layer_id, keys, page_status,
                             flags, 0, &c);
    if (rc) return rc;
    NoAllocDevice* d = nullptr;
    rc = noalloc_device(&d);
    if (rc) return rc;
    c.p.ppw = pages_per_group(batch, d->cu_count);
    CallState* call = reinterpret_cast<CallState*>(d->scratch);
    DeviceState* sticky = reinterpret_cast<DeviceState*>(d->scratch + sizeof(CallState));
    int32_t* status = reinterpret_cast<int32_t*>(d->scratch + kScratchStatusOff);
    CallState result{~0ull, 0u, 0u};  // pageable: the read-back allocates nothing
    const WaitSink sink{&sticky->diag, &call->diag, g_spin_limit.load(std::memory_order_relaxed)};
    const hipError_t e = ingress_enqueue(c, call, status, sink, &result, (hipStream_t)stream);
    if (e != hipSuccess) return ZTCP_EHIP;
    return c.async ? ZTCP_OK : verdict(result);
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
    // the library's sticky word when the allocating entry points have set up
    // this device, and the no-allocation path's when that path has: reading
    // them allocates nothing
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return ZTCP_EHIP;
    if (hipDeviceSynchronize() != hipSuccess) return ZTCP_EHIP;
    uint32_t* words[2] = {nullptr, nullptr};
    {
        std::lock_guard<std::mutex> lock(g_mu);
        if (dev < (int)g_ctx.size() && g_ctx[dev]) words[0] = &g_ctx[dev]->state->diag;
    }
    {
        std::lock_guard<std::mutex> lock(g_noalloc_mu);
        if (dev < kMaxDevices && g_noalloc[dev].scratch)
            words[1] = &reinterpret_cast<DeviceState*>(g_noalloc[dev].scratch + sizeof(CallState))->diag;
    }
    uint32_t all = 0;
    for (uint32_t* w : words) {
        if (!w) continue;
        uint32_t d = 0;
        const uint32_t zero = 0;
        if (hipMemcpy(&d, w, sizeof d, hipMemcpyDeviceToHost) != hipSuccess ||
            hipMemcpy(w, &zero, sizeof zero, hipMemcpyHostToDevice) != hipSuccess)
            return ZTCP_EHIP;
        all |= d;
    }
    return (int)all;
}

int64_t ztcp_debug_spin_limit(int64_t n) {
    const uint32_t v = n < 0 ? kSpinLimit : (n > (int64_t)0xFFFFFFFFu ? 0xFFFFFFFFu : (uint32_t)n);
    return (int64_t)g_spin_limit.exchange(v);
}

const char* ztcp_strerror(int code) {
    switch (code) {
        case ZTCP_OK: return "ok";
        case ZTCP_ERR_HEADER: return "KV_INTEGRITY_ERROR: Invalid cold-page header magic, version, or flags";
        case ZTCP_ERR_AAD: return "CROSS_TENANT_CONTAMINATION: Cold-page AAD mismatch";
        case ZTCP_ERR_MAC: return "KV_INTEGRITY_ERROR: Cold-page MAC verification failed";
        case ZTCP_ERR_DEVICE: return "KV_INTEGRITY_ERROR: page rejected after a device-side wait expired";
        case ZTCP_EINVAL: return "invalid argument";
        case ZTCP_EOVERLAP: return "outputs must not alias or overlap input tensors";
        case ZTCP_EHIP: return "HIP runtime error";
        case ZTCP_EDEVICE: return "device-side bounded wait expired; outputs zeroed";
        case ZTCP_ESCRATCH: return "batch exceeds ZTCP_NOALLOC_MAX_PAGES";
        default: return "unknown error";
    }
}

const char* ztcp_last_error(void) { return t_last_error; }

#ifdef ZTCP_PHASE_TIMERS
int64_t ztcp_phase_timers_read(int32_t direction, uint64_t* out, int64_t max_words) {
    if (direction < 0 || direction > 1 || (!out && max_words > 0)) return ZTCP_EINVAL;
    if (hipDeviceSynchronize() != hipSuccess) return ZTCP_EHIP;
    unsigned long long* buf = nullptr;
    int64_t n = 0;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        buf = g_timer_buf[direction];
        n = g_timer_wgs[direction] * kTimerSlots;
    }
    if (!buf || n == 0) return 0;
    if (n > max_words) return ZTCP_EINVAL;
    if (hipMemcpy(out, buf, sizeof(uint64_t) * (size_t)n, hipMemcpyDeviceToHost) != hipSuccess) return ZTCP_EHIP;
    return n;
}

int64_t ztcp_phase_trace_read(int32_t direction, uint32_t* out, int64_t max_words) {
    if (direction < 0 || direction > 1 || (!out && max_words > 0)) return ZTCP_EINVAL;
    if (hipDeviceSynchronize() != hipSuccess) return ZTCP_EHIP;
    unsigned long long* buf = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        buf = g_timer_buf[direction];
    }
    if (!buf) return 0;
    if (max_words < 4 * kTraceRows) return ZTCP_EINVAL;
    if (hipMemcpy(out, buf + (size_t)kTimerSlots * ZTCP_TIMER_MAX_WORKGROUPS, sizeof(uint32_t) * 4 * kTraceRows,
                  hipMemcpyDeviceToHost) != hipSuccess)
        return ZTCP_EHIP;
    return 4 * kTraceRows;
}
#endif

}  // extern "C"
