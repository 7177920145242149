/*
 * ztcp.h -- C ABI of the MI355X (gfx950) ZTCP fused cold-page codec.
 *
 * Egress:  quantize -> ChaCha20 (RFC 8439) -> SipHash-2-4-128 Encrypt-then-MAC.
 * Ingress: verify tag and AAD -> decrypt -> dequantize, rejecting tampered pages.
 *
 * Every entry point below replaces one function of the reference's native
 * module `ztcp_fused_cold_page_cpp` (research/baseline_codec/csrc/
 * fused_cold_page_cpu.cpp, "cpp" below), as bound by its Python wrapper
 * research/baseline_codec/native_fused_codec.py ("nfc").  Arguments keep the
 * reference's names, meaning and order; torch tensors become plain device
 * pointers plus the sizes the tensors carried.
 *
 * Conventions
 *  - Page data, blobs, token hashes and status arrays are DEVICE pointers.
 *  - Hot pages are [batch, num_tokens, num_heads, head_dim] elements of
 *    `hot_dtype` (FP16 = the reference's only dtype, cpp:1499; BF16 = extension:
 *    the byte layout is unchanged, scales stay fp16 on the wire).
 *  - A blob is 32-byte header || payload || 16-byte tag (spec:17-51).
 *  - Calls are enqueued on `stream` (a hipStream_t; NULL = the default stream)
 *    and, like the reference's, are synchronous: they return once the work
 *    is done, with its verdict.  With ZTCP_ASYNC (the entry points that take
 *    flags) a call returns once enqueued: ingress verdicts are then read from
 *    `page_status`, and an egress failure shows in the blobs (below).
 *  - Calls may overlap freely (several streams, several host threads): each
 *    call keeps its failure record in device state of its own, which the call
 *    holds until its work on the stream has completed.
 *  - Fail closed: the fused kernels' hand-offs use bounded waits.  If one
 *    expires (a device-side fault, never expected), every later wait of the
 *    same workgroup ends at once, ingress fails every page of the affected
 *    workgroup with ZTCP_ERR_DEVICE and zeroes its outputs, and egress writes
 *    the affected workgroup's blobs with a zero header magic, which every
 *    ingress rejects (status 1).  A synchronous call then returns
 *    ZTCP_EDEVICE, egress after zeroing every blob of the call (the
 *    reference's wrapper zeroes out_blobs on any failure, nfc:597-600).
 *    Either way ztcp_device_diag reports it.
 *  - Keys are passed by value and never retained (nfc:173-174 unpacks them
 *    into the same little-endian u64 words).
 *  - Errors are return codes, never exceptions: negative = argument / runtime
 *    error (the TORCH_CHECK list of cpp:1925-1957, cpp:2267-2296);
 *    positive = integrity verdict of the lowest failing page (cpp:2231-2245).
 */
#ifndef ZTCP_H
#define ZTCP_H

#include <stddef.h>
#include <stdint.h>

/* Every entry point is exported from the library, which is built with hidden
 * default visibility: the library exports exactly what its headers declare. */
#ifndef ZTCP_API
#if defined(__GNUC__) || defined(__clang__)
#define ZTCP_API __attribute__((visibility("default")))
#else
#define ZTCP_API
#endif
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Wire constants: spec:47-51, cpp:55-58. */
#define ZTCP_MAGIC 0x5A54u
#define ZTCP_VERSION 1u
#define ZTCP_HEADER_BYTES 32u
#define ZTCP_TAG_BYTES 16u

/* QuantPreset (spec:54-59) and RoPEMode (spec:62-67). */
enum { ZTCP_INT4_SYM = 1, ZTCP_K8V4_ASYM = 2, ZTCP_FP8_ONLY = 3 };
enum { ZTCP_QUANTIZE_ALL = 0, ZTCP_PRESERVE_FP8 = 1, ZTCP_PRESERVE_RAW = 2 };
/* Extension presets and RoPE mode (no counterpart in the reference, which
 * rejects these header flags; same header, framing, cipher and MAC):
 *   ZTCP_K8V4_ASYM_G64   K: int8 asymmetric per 64 elements (fp16 scale + u16
 *                        zero point), V: int4 symmetric per 32 elements
 *   ZTCP_FP8_E4M3        K and V: OCP FP8 e4m3 per 16 elements (fp16 scale
 *                        = amax / 448, saturating round-to-nearest-even)
 *   ZTCP_INT4_SYM_G32    K and V: int4 symmetric per 32 elements
 *   ZTCP_PRESERVE_E4M3   the RoPE columns as e4m3 per 16 elements
 * A group must not straddle a section: the extension kinds need section
 * widths divisible by 64 (int8 asymmetric) or 32 (int4 per 32); otherwise the
 * sizing functions return (size_t)-1 and egress returns ZTCP_EINVAL. */
enum { ZTCP_K8V4_ASYM_G64 = 4, ZTCP_FP8_E4M3 = 5, ZTCP_INT4_SYM_G32 = 6 };
enum { ZTCP_PRESERVE_E4M3 = 3 };
enum { ZTCP_HOT_FP16 = 0, ZTCP_HOT_BF16 = 1 };

/* Integrity verdicts: the reference's per-page status codes (cpp:2056-2057). */
#define ZTCP_OK 0
#define ZTCP_ERR_HEADER 1  /* KV_INTEGRITY_ERROR: magic, version, flags or size */
#define ZTCP_ERR_AAD 2     /* CROSS_TENANT_CONTAMINATION: tenant/model/layer/token */
#define ZTCP_ERR_MAC 3     /* KV_INTEGRITY_ERROR: MAC verification failed */
/* Per-page status only (no counterpart in the reference): the page's
 * workgroup hit an expired bounded wait; the page is rejected and zeroed. */
#define ZTCP_ERR_DEVICE 4
/* Argument / runtime errors. */
#define ZTCP_EINVAL (-1)   /* a TORCH_CHECK of the reference would fail */
#define ZTCP_EOVERLAP (-2) /* an output aliases an input (cpp:1428-1437) */
#define ZTCP_EHIP (-3)     /* the HIP runtime reported an error */
#define ZTCP_EDEVICE (-4)  /* a kernel's bounded wait expired: outputs are zeroed
                              (ingress: all of them; egress: every blob of the
                              call; see ztcp_device_diag) */
#define ZTCP_ESCRATCH (-5) /* batch larger than ZTCP_NOALLOC_MAX_PAGES
                              (ztcp_ingress_peak_into_noalloc only) */

/* Call flags. */
#define ZTCP_ASYNC 0x1u          /* enqueue only.  Ingress: verdicts land in page_status.
                                    Egress: an expired wait shows only as blobs with a
                                    zero header magic and in ztcp_device_diag */
#define ZTCP_PER_PAGE 0x2u       /* ingress extension: keep verified pages, zero failing
                                    ones; default is the reference's all-or-nothing */
#define ZTCP_EXT_LAYOUTS 0x4u    /* extension: the extension presets / RoPE mode.  Ingress
                                    without it fails such headers with status 1, egress
                                    (the *_ext entry points) without it rejects them with
                                    ZTCP_EINVAL, as the reference's flags check does
                                    (cpp:1447-1449) */

typedef struct ztcp_geometry {
    int64_t num_tokens;   /* tokens per page */
    int64_t num_heads;    /* KV heads per page */
    int64_t head_dim;     /* >= 16, multiple of 16 */
    int64_t rope_dim;     /* leading RoPE columns of K, multiple of 16 */
    int32_t hot_dtype;    /* ZTCP_HOT_FP16 / ZTCP_HOT_BF16 */
    int32_t is_mla_single_buffer; /* 1: K only (no V buffer) */
} ztcp_geometry;

/* Per-batch AAD fields of the header (cpp:61-75). */
typedef struct ztcp_aad {
    uint32_t tenant_id_hash;
    uint32_t model_id_hash;
    uint16_t layer_id;
    uint16_t head_group_id;
} ztcp_aad;

/* Session keys as the reference passes them: encryption key k0..k3 (LE u64
 * words of the 32-byte key, cpp:85-100), MAC key mk0, mk1 (nfc:173-174). */
typedef struct ztcp_keys {
    uint64_t k0, k1, k2, k3;
    uint64_t mk0, mk1;
} ztcp_keys;

/* One page of a paged (non-contiguous) KV pool, possibly spanning layers.
 * Egress reads k/v and writes blob; ingress reads blob and writes k/v.  v is
 * NULL for MLA single-buffer pages.  k, v and blob must be 16-byte aligned.
 * The per-page fields replace the batch-wide ones of the contiguous form:
 *   egress:  token_hash, sequence_nonce, layer_id, head_group_id go into the
 *            page's header and nonce (cpp:1129-1140, cpp:102-110);
 *   ingress: token_hash and layer_id are the page's expected AAD values
 *            (cpp:2317-2323); sequence_nonce / head_group_id are not compared,
 *            as in the reference. */
typedef struct ztcp_page_desc {
    void* k;
    void* v;
    uint8_t* blob;
    int64_t token_hash;
    uint64_t sequence_nonce;
    uint16_t layer_id;
    uint16_t head_group_id;
    uint32_t reserved;
} ztcp_page_desc;

/* Payload bytes padded to 4 (spec:203-246, what nfc passes as
 * expected_payload_bytes); (size_t)-1 for invalid preset / rope_mode.  The
 * extension presets 4..6 and RoPE mode 3 are sized as well. */
ZTCP_API size_t ztcp_payload_bytes(const ztcp_geometry* g, int64_t preset, int64_t rope_mode);
/* Unpadded minimum payload for header flags: required_payload_bytes_for_flags
 * (cpp:1439-1474); (size_t)-1 for invalid flags. */
ZTCP_API size_t ztcp_required_payload_bytes(const ztcp_geometry* g, int64_t preset, int64_t rope_mode);
/* 32 + ztcp_payload_bytes + 16 (spec:248-250 cold_blob_bytes). */
ZTCP_API size_t ztcp_blob_bytes(const ztcp_geometry* g, int64_t preset, int64_t rope_mode);

/* Batch egress into a preallocated [batch, 32 + expected_payload_bytes + 16]
 * buffer.  Replaces fused_encode_cold_pages_peak_into_cpu (cpp:1904-2004):
 * page b is read at b * T*H*D elements, encoded with token_hashes[b] and
 * sequence_nonce = base_sequence_nonce + b, and written at b * blob_bytes.
 * Presets 1..3 and RoPE modes 0..2, as the reference (cpp:1947-1948). */
ZTCP_API int ztcp_egress_peak_into(const void* k_pages, const void* v_pages,
                          const int64_t* page_token_hashes, uint8_t* out_blobs,
                          int64_t batch, const ztcp_geometry* g, int64_t preset,
                          int64_t rope_mode, int64_t expected_payload_bytes,
                          const ztcp_aad* aad, uint64_t base_sequence_nonce,
                          const ztcp_keys* keys, void* stream);
/* The same with call flags: ZTCP_ASYNC; ZTCP_EXT_LAYOUTS admits the
 * extension presets 4..6 and RoPE mode 3 (no counterpart in the reference). */
ZTCP_API int ztcp_egress_peak_into_ext(const void* k_pages, const void* v_pages,
                              const int64_t* page_token_hashes, uint8_t* out_blobs,
                              int64_t batch, const ztcp_geometry* g, int64_t preset,
                              int64_t rope_mode, int64_t expected_payload_bytes,
                              const ztcp_aad* aad, uint64_t base_sequence_nonce,
                              const ztcp_keys* keys, uint32_t flags, void* stream);

/* Descriptor form of the same egress for paged, multi-layer KV pools:
 * `pages` is a DEVICE array of n_pages descriptors; tenant and model hashes
 * come from `tenant_id_hash` / `model_id_hash`, every other header field from
 * the page's descriptor.  Same encoding as ztcp_egress_peak_into. */
ZTCP_API int ztcp_egress_batch(const ztcp_page_desc* pages, int64_t n_pages,
                      const ztcp_geometry* g, int64_t preset, int64_t rope_mode,
                      int64_t expected_payload_bytes, uint32_t tenant_id_hash,
                      uint32_t model_id_hash, const ztcp_keys* keys, void* stream);
/* The same with call flags: ZTCP_ASYNC, ZTCP_EXT_LAYOUTS (the extension
 * presets / RoPE mode). */
ZTCP_API int ztcp_egress_batch_ext(const ztcp_page_desc* pages, int64_t n_pages,
                          const ztcp_geometry* g, int64_t preset, int64_t rope_mode,
                          int64_t expected_payload_bytes, uint32_t tenant_id_hash,
                          uint32_t model_id_hash, const ztcp_keys* keys, uint32_t flags,
                          void* stream);

/* Batch ingress into preallocated outputs.  Replaces
 * fused_decode_cold_pages_peak_into_cpu (cpp:2250-2496): every page is
 * checked in the reference's order (magic/version -> 1, tenant/model/layer/
 * token hash -> 2, SipHash tag -> 3, flags/size -> 1), decrypted and
 * dequantized according to its own header flags.  Default (all-or-nothing):
 * if any page fails, both outputs are zeroed and the verdict of the lowest
 * failing page is returned (ZTCP_EDEVICE when a bounded wait expired).
 * page_status (DEVICE int32[batch], may be NULL) receives every page's
 * verdict (0..4). */
ZTCP_API int ztcp_ingress_peak_into(const uint8_t* cold_blobs, int64_t blob_bytes,
                           const int64_t* expected_token_hashes, void* out_k_pages,
                           void* out_v_pages, int64_t batch, const ztcp_geometry* g,
                           uint32_t expected_tenant_hash, uint32_t expected_model_hash,
                           uint16_t expected_layer_id, const ztcp_keys* keys,
                           int32_t* page_status, uint32_t flags, void* stream);

/* Ingress that allocates nothing.  No counterpart in the reference: for
 * callers that cannot allocate device or pinned memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid it).  Same arguments,
 * checks, kernels and results as ztcp_ingress_peak_into; the call's device
 * state (failure word, diagnostics, and the per-page status array the
 * generic kernels need when page_status is NULL) lives in a fixed device
 * array of about 256 KiB that each GPU holds until the process ends, so
 * batches are limited to ZTCP_NOALLOC_MAX_PAGES pages (ZTCP_ESCRATCH beyond).
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (other streams, other threads) race and must be serialized by the caller.
 * The array is set up on the first call on each device.  Only a ZTCP_ASYNC
 * call can be recorded into a HIP graph (a synchronous one copies its verdict
 * to the host and waits for the stream): a synchronous call on a stream under
 * capture returns ZTCP_EINVAL.  ztcp_device_diag reads this path's sticky
 * diagnostics without allocating. */
#define ZTCP_NOALLOC_MAX_PAGES 65536
ZTCP_API int ztcp_ingress_peak_into_noalloc(const uint8_t* cold_blobs, int64_t blob_bytes,
                                   const int64_t* expected_token_hashes, void* out_k_pages,
                                   void* out_v_pages, int64_t batch, const ztcp_geometry* g,
                                   uint32_t expected_tenant_hash, uint32_t expected_model_hash,
                                   uint16_t expected_layer_id, const ztcp_keys* keys,
                                   int32_t* page_status, uint32_t flags, void* stream);

/* Descriptor form of the same ingress (blob in, k/v out; the expected token
 * hash and layer id of each page come from its descriptor). */
ZTCP_API int ztcp_ingress_batch(const ztcp_page_desc* pages, int64_t n_pages, int64_t blob_bytes,
                       const ztcp_geometry* g, uint32_t expected_tenant_hash,
                       uint32_t expected_model_hash, const ztcp_keys* keys,
                       int32_t* page_status, uint32_t flags, void* stream);

/* Known-answer hooks.  ztcp_chacha20_xor replaces chacha20_rfc8439_xor_cpu
 * (cpp:2499-2524): dst = src ^ ChaCha20(key, nonce, counter..).
 * ztcp_siphash128 replaces siphash24_128_cpu (cpp:2526-2538).  key, nonce
 * are HOST byte arrays; data and outputs are DEVICE pointers. */
ZTCP_API int ztcp_chacha20_xor(const uint8_t* src, uint8_t* dst, size_t len, const uint8_t key[32],
                      uint32_t initial_counter, const uint8_t nonce[12], void* stream);
ZTCP_API int ztcp_siphash128(const uint8_t* data, size_t len, uint64_t mk0, uint64_t mk1,
                    uint8_t* tag16, void* stream);

/* Self-check of the device arithmetic the fused quantizer relies on: for
 * every amax the FP16 and BF16 hot dtypes can produce, the fast scale (a
 * corrected quotient) equals fp16(amax / 127) and fp16(amax / 7) by IEEE
 * division whenever it is a normal fp16 value, and the Newton-refined
 * reciprocal equals 1 / s for every positive finite fp16 scale; and the
 * hardware e4m3 conversions (v_cvt_pk_fp8_f32, v_cvt_f32_fp8) the extension
 * kinds use equal the bit-exact software conversions on every bf16 pattern,
 * its neighbours and all 256 codes.  Returns the number of violations
 * (0 = pass) or a negative error.  A test hook like the
 * reference's (cpp:2499-2538); it has no counterpart of its own there. */
ZTCP_API int ztcp_selftest(void);

/* Device-side diagnostics of the current device: returns and clears the
 * sticky flags a kernel's bounded waits set (0 = none).  Synchronizes; sets
 * nothing up and allocates nothing. */
ZTCP_API int ztcp_device_diag(void);

/* Test hook for the fail-closed paths (no counterpart in the reference):
 * sets the number of polls after which the fused kernels' bounded waits give
 * up, for calls made afterwards in this process; n < 0 restores the default
 * (about 30 ms).  n = 0 makes every wait that is not already satisfied expire
 * at once, so a test can drive the expiry handling to completion without a
 * fault.  Returns the previous value. */
ZTCP_API int64_t ztcp_debug_spin_limit(int64_t n);

/* Serving-side steps around the codec (vlx-tee_amd/csrc/ztcp_serving.hip).
 *
 * Hit bitmap of per-page ingress verdicts: the PoisonShield per-page fallback
 * (research/paper/main.tex:173), where a page that fails AAD, MAC or
 * freshness checks is not written to hot memory and reads as a miss in the
 * serving engine's hit bitmap, so the engine recomputes that prefix instead
 * of failing the worker.  The reference describes the step but has no
 * function for it.  page_status: DEVICE int32[n] as the per-page ingress
 * writes it.  packed = 0: out is DEVICE uint8[n], 1 where the verdict is 0;
 * packed = 1: out is DEVICE uint8[(n + 7) / 8], page i in bit i % 8 of byte
 * i / 8 (least significant bit first), trailing bits 0.  Enqueued on stream. */
ZTCP_API int ztcp_hit_bitmap(const int32_t* page_status, int64_t n, uint8_t* out, int32_t packed, void* stream);

/* Egress wire ring: a batch of blobs leaves HBM into the next of n_slots
 * pinned host slots, on a copy stream of the ring's own that waits for the
 * work already queued on the producer's stream (the egress launch that wrote
 * the blobs), so the next batch's egress overlaps the copy.  The reference
 * models this step only (research/benchmarks/bench_cold_page_pipeline.py:
 * 1089-1162: blob bytes over a link after the codec).
 *   create:  n_slots slots of slot_bytes on the current device.
 *   push:    copies nbytes (<= slot_bytes) of DEVICE blobs into the next
 *            slot, after the work queued on `stream`; *slot = its index.  A
 *            slot is reused n_slots pushes later, after its previous copy
 *            has landed, so the bytes wait returned stay valid until then.
 *            Pushes from several host threads take slots in turn.
 *   wait:    blocks until that slot's copy has landed; *host and *nbytes
 *            give its bytes (HOST memory owned by the ring).
 *   destroy: waits for the copies in flight, then frees the ring. */
typedef struct ztcp_wire_ring ztcp_wire_ring;
ZTCP_API int ztcp_wire_ring_create(size_t slot_bytes, int32_t n_slots, ztcp_wire_ring** ring);
ZTCP_API int ztcp_wire_ring_push(ztcp_wire_ring* ring, const uint8_t* blobs, size_t nbytes, void* stream,
                        int32_t* slot);
ZTCP_API int ztcp_wire_ring_wait(ztcp_wire_ring* ring, int32_t slot, const uint8_t** host, size_t* nbytes);
ZTCP_API int ztcp_wire_ring_destroy(ztcp_wire_ring* ring);

/* Short description of a return code. */
ZTCP_API const char* ztcp_strerror(int code);

/* Why the calling thread's last call returned ZTCP_EINVAL or ZTCP_EOVERLAP:
 * the reference's TORCH_CHECK message for the same condition where it has
 * one ("" when the last call succeeded). */
ZTCP_API const char* ztcp_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* ZTCP_H */
