// ztcp_serving.hip -- the serving-side steps on either side of the codec:
//   * the hit bitmap of a batch's per-page ingress verdicts: the PoisonShield
//     per-page fallback (research/paper/main.tex:173), where a page that fails
//     its checks reads as a miss and the serving engine recomputes it;
//   * the egress wire ring: blobs leave HBM into pinned host slots on a copy
//     stream of the ring's own, ordered after the producer's stream by an
//     event, so the next batch's egress overlaps the copy.  The reference
//     only models this step (blob bytes over a link after the codec,
//     research/benchmarks/bench_cold_page_pipeline.py:1089-1162).
#include <mutex>
#include <new>
#include <vector>

#include "ztcp_params.h"

namespace {

// One page per lane.  Packed: the wave's 64 verdicts become one ballot, page
// i in bit i % 8 of byte i / 8 (least significant bit first), written by the
// wave's first eight lanes; bits past the last page are 0.  Unpacked: one
// byte (0 / 1) per page.
__global__ void hit_bitmap_kernel(const int32_t* status, int64_t n, uint8_t* out, int32_t packed) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool hit = i < n && status[i] == 0;
    if (!packed) {
        if (i < n) out[i] = hit ? 1u : 0u;
        return;
    }
    const uint64_t m = __ballot(hit);
    const int lane = (int)(threadIdx.x & 63u);
    const int64_t byte0 = (i - lane) / 8;  // the wave's first page is a multiple of 64
    if (lane < 8 && byte0 + lane < (n + 7) / 8) out[byte0 + lane] = (uint8_t)(m >> (8 * lane));
}

}  // namespace

struct ztcp_wire_ring {
    int device = 0;
    size_t slot_bytes = 0;
    std::vector<uint8_t*> slots;       // pinned host memory (hipHostMalloc)
    std::vector<size_t> sizes;         // bytes of the last copy into each slot
    std::vector<hipEvent_t> done;      // recorded on the copy stream after each copy
    std::vector<bool> used;            // a copy was ever enqueued into the slot
    hipEvent_t ready = nullptr;        // the producer stream's position at a push
    hipStream_t copy = nullptr;        // default priority
    int next = 0;
    std::mutex mu;                     // pushes from several threads take slots in turn
};

namespace {

void ring_free(ztcp_wire_ring* r) {
    for (uint8_t* s : r->slots)
        if (s) (void)hipHostFree(s);
    for (hipEvent_t e : r->done)
        if (e) (void)hipEventDestroy(e);
    if (r->ready) (void)hipEventDestroy(r->ready);
    if (r->copy) (void)hipStreamDestroy(r->copy);
    delete r;
}

}  // namespace

extern "C" {

int ztcp_hit_bitmap(const int32_t* page_status, int64_t n, uint8_t* out, int32_t packed, void* stream) {
    if (n < 0 || (n > 0 && (!page_status || !out))) return ZTCP_EINVAL;
    if (n == 0) return ZTCP_OK;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(hit_bitmap_kernel, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, page_status,
                       n, out, packed ? 1 : 0);
    return hipGetLastError() == hipSuccess ? ZTCP_OK : ZTCP_EHIP;
}

int ztcp_wire_ring_create(size_t slot_bytes, int32_t n_slots, ztcp_wire_ring** out) {
    if (!out || slot_bytes == 0 || n_slots <= 0) return ZTCP_EINVAL;
    *out = nullptr;
    ztcp_wire_ring* r = new (std::nothrow) ztcp_wire_ring;
    if (!r) return ZTCP_EHIP;
    r->slot_bytes = slot_bytes;
    bool ok = hipGetDevice(&r->device) == hipSuccess &&
              hipStreamCreateWithFlags(&r->copy, hipStreamNonBlocking) == hipSuccess &&
              hipEventCreateWithFlags(&r->ready, hipEventDisableTiming) == hipSuccess;
    for (int i = 0; ok && i < n_slots; ++i) {
        uint8_t* s = nullptr;
        hipEvent_t e = nullptr;
        ok = hipHostMalloc((void**)&s, slot_bytes, hipHostMallocDefault) == hipSuccess;
        if (ok) ok = hipEventCreateWithFlags(&e, hipEventDisableTiming) == hipSuccess;
        r->slots.push_back(s);
        r->done.push_back(e);
        r->sizes.push_back(0);
        r->used.push_back(false);
    }
    if (!ok) {
        ring_free(r);
        return ZTCP_EHIP;
    }
    *out = r;
    return ZTCP_OK;
}

int ztcp_wire_ring_destroy(ztcp_wire_ring* ring) {
    if (!ring) return ZTCP_EINVAL;
    int dev = 0;
    const bool switch_dev = hipGetDevice(&dev) == hipSuccess && dev != ring->device;
    if (switch_dev) (void)hipSetDevice(ring->device);
    const hipError_t e = hipStreamSynchronize(ring->copy);  // no copy may land in freed memory
    ring_free(ring);
    if (switch_dev) (void)hipSetDevice(dev);
    return e == hipSuccess ? ZTCP_OK : ZTCP_EHIP;
}

int ztcp_wire_ring_push(ztcp_wire_ring* ring, const uint8_t* blobs, size_t nbytes, void* stream, int32_t* slot) {
    if (!ring || !slot || (nbytes > 0 && !blobs)) return ZTCP_EINVAL;
    if (nbytes > ring->slot_bytes) return ZTCP_EINVAL;
    std::lock_guard<std::mutex> lock(ring->mu);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return ZTCP_EHIP;
    if (dev != ring->device && hipSetDevice(ring->device) != hipSuccess) return ZTCP_EHIP;
    const int i = ring->next;
    // the slot's previous bytes stay valid until here: its copy has landed
    // and is overwritten only now, n_slots pushes later
    bool ok = !ring->used[i] || hipEventSynchronize(ring->done[i]) == hipSuccess;
    if (ok) ok = hipEventRecord(ring->ready, (hipStream_t)stream) == hipSuccess;
    if (ok) ok = hipStreamWaitEvent(ring->copy, ring->ready, 0) == hipSuccess;
    if (ok && nbytes > 0)
        ok = hipMemcpyAsync(ring->slots[i], blobs, nbytes, hipMemcpyDeviceToHost, ring->copy) == hipSuccess;
    if (ok) ok = hipEventRecord(ring->done[i], ring->copy) == hipSuccess;
    if (dev != ring->device) (void)hipSetDevice(dev);
    if (!ok) return ZTCP_EHIP;
    ring->used[i] = true;
    ring->sizes[i] = nbytes;
    ring->next = (i + 1) % (int)ring->slots.size();
    *slot = i;
    return ZTCP_OK;
}

int ztcp_wire_ring_wait(ztcp_wire_ring* ring, int32_t slot, const uint8_t** host, size_t* nbytes) {
    if (!ring || !host || !nbytes || slot < 0 || slot >= (int32_t)ring->slots.size()) return ZTCP_EINVAL;
    hipEvent_t ev = nullptr;
    {
        std::lock_guard<std::mutex> lock(ring->mu);
        if (!ring->used[slot]) return ZTCP_EINVAL;
        ev = ring->done[slot];
        *host = ring->slots[slot];
        *nbytes = ring->sizes[slot];
    }
    return hipEventSynchronize(ev) == hipSuccess ? ZTCP_OK : ZTCP_EHIP;
}

}  // extern "C"
