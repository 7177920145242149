/*
 * ztcp_oracle.h -- CPU restatement of the ZTCP fused cold-page codec.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the CPU reference the HIP path is compared
 * against (tests/, __graft_entry__.smoke(), and bench.py's cpu_baseline leg).
 * Nothing on the product path links, loads or calls it.
 *
 * It restates the reference's portable scalar arithmetic ("profile S": the
 * `#else` branches the reference compiles on any non-NEON host) of
 * research/baseline_codec/csrc/fused_cold_page_cpu.cpp, function by function;
 * every definition in ztcp_oracle.c cites the reference lines it follows.
 *
 * Hot dtypes: ZO_FP16 is the reference's only dtype (cpp:1499); ZO_BF16 is
 * an extension beyond the reference (f32 widening of bf16, fp16 scales on the
 * wire, bf16 round-to-nearest-even on dequantize).
 */
#ifndef ZTCP_ORACLE_H
#define ZTCP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ZO_FP16 = 0, ZO_BF16 = 1 };

/* ---- primitives -------------------------------------------------------- */
uint16_t zo_f32_to_f16(float f);
float zo_f16_to_f32(uint16_t h);
uint16_t zo_f32_to_bf16(float f);
float zo_bf16_to_f32(uint16_t b);

void zo_chacha20_block(const uint32_t key[8], uint32_t counter,
                       const uint32_t nonce[3], uint8_t out[64]);
void zo_chacha20_xor(const uint8_t* src, uint8_t* dst, size_t len,
                     const uint8_t key32[32], uint32_t counter,
                     const uint8_t nonce12[12]);
void zo_siphash128(const uint8_t* data, size_t len, uint64_t mk0, uint64_t mk1,
                   uint8_t tag[16]);

/* One 16-element group.  src holds 16 raw hot elements (fp16 or bf16 bits). */
void zo_quant_group16_int8(const uint16_t* src, int dtype, uint8_t q[16],
                           uint16_t* scale_f16);
void zo_quant_group16_int4(const uint16_t* src, int dtype, uint8_t q[8],
                           uint16_t* scale_f16);
void zo_dequant_group16_int8(const uint8_t q[16], uint16_t scale_f16, int dtype,
                             uint16_t* dst);
void zo_dequant_group16_int4(const uint8_t q[8], uint16_t scale_f16, int dtype,
                             uint16_t* dst);

/* Extension codes (no counterpart in the reference): FP8 e4m3 per 16
 * elements, int4 per 32, int8 asymmetric per 64 (scale, zero point). */
uint8_t zo_f32_to_e4m3(float x);
float zo_e4m3_to_f32(uint8_t c);
void zo_quant_group16_e4m3(const uint16_t* src, int dtype, uint8_t q[16], uint16_t* scale_f16);
void zo_dequant_group16_e4m3(const uint8_t q[16], uint16_t scale_f16, int dtype, uint16_t* dst);
void zo_quant_group32_int4(const uint16_t* src, int dtype, uint8_t q[16], uint16_t* scale_f16);
void zo_dequant_group32_int4(const uint8_t q[16], uint16_t scale_f16, int dtype, uint16_t* dst);
void zo_quant_group64_asym8(const uint16_t* src, int dtype, uint8_t q[64], uint16_t* scale_f16,
                            uint16_t* zero);
void zo_dequant_group64_asym8(const uint8_t q[64], uint16_t scale_f16, uint16_t zero, int dtype,
                              uint16_t* dst);

/* ---- sizing ------------------------------------------------------------ */
/* Unpadded payload bytes for header flags; (size_t)-1 for invalid flags.
 * Presets 1..3 / RoPE modes 0..2 are the reference's; presets 4 (K8V4_ASYM),
 * 5 (FP8_E4M3), 6 (INT4_SYM_G32) and RoPE mode 3 (PRESERVE_E4M3) are
 * extensions, valid only where their group size divides the section width. */
size_t zo_required_payload(int64_t preset, int64_t rope_mode, int64_t vecs,
                           int64_t head_dim, int64_t rope_dim, int has_v);
/* Payload padded to a 4-byte boundary (the size the Python wrapper passes). */
size_t zo_payload_bytes(int64_t preset, int64_t rope_mode, int64_t vecs,
                        int64_t head_dim, int64_t rope_dim, int has_v);

/* ---- pages and batches ------------------------------------------------- */
typedef struct zo_egress_args {
    const void* k_pages;          /* [B, T, H, D] hot elements */
    const void* v_pages;          /* same shape, or NULL (MLA single buffer) */
    const int64_t* token_hashes;  /* [B] */
    uint8_t* out_blobs;           /* [B, 32 + expected_payload + 16] */
    int64_t batch, num_tokens, num_heads, head_dim, rope_dim;
    int32_t dtype;
    int64_t preset, rope_mode, expected_payload_bytes;
    uint32_t tenant_id_hash, model_id_hash;
    uint16_t layer_id, head_group_id;
    uint64_t base_sequence_nonce;
    uint64_t k0, k1, k2, k3, mk0, mk1;
} zo_egress_args;

typedef struct zo_ingress_args {
    const uint8_t* blobs;         /* [B, blob_bytes] */
    int64_t blob_bytes;
    const int64_t* expected_token_hashes;
    void* out_k;                  /* [B, T, H, D] */
    void* out_v;                  /* NULL when is_mla_single_buffer */
    int64_t batch, num_tokens, num_heads, head_dim, rope_dim;
    int32_t dtype, is_mla_single_buffer;
    uint32_t expected_tenant_hash, expected_model_hash;
    uint16_t expected_layer_id;
    uint64_t k0, k1, k2, k3, mk0, mk1;
} zo_ingress_args;

/* Encode a batch.  threads <= 1 runs serially; otherwise contiguous page
 * chunks on that many pthreads.  Returns 0, or -1 on invalid arguments. */
int zo_egress_batch(const zo_egress_args* a, int threads);

/* Decode a batch.  status[b] (may be NULL) receives 0 OK, 1 header/flags/size,
 * 2 AAD mismatch, 3 MAC failure.  all_or_nothing != 0 zeroes every output when
 * any page fails (the reference's batch contract); otherwise only failing
 * pages are zeroed.  Returns the status of the lowest failing page, or 0;
 * -1 on invalid arguments. */
int zo_ingress_batch(const zo_ingress_args* a, int32_t* status,
                     int all_or_nothing, int threads);

/* ---- array helpers (exhaustive conversion / quantizer checks) ---------- */
void zo_f32_to_f16_array(const float* src, uint16_t* dst, size_t n);
void zo_f32_to_bf16_array(const float* src, uint16_t* dst, size_t n);
void zo_f16_to_f32_array(const uint16_t* src, float* dst, size_t n);
void zo_quant_groups(const uint16_t* src, int dtype, int bits, size_t n, uint8_t* q,
                     uint16_t* scales);
void zo_dequant_groups(const uint8_t* q, const uint16_t* scales, int dtype, int bits,
                       size_t n, uint16_t* dst);

int zo_quant_groups_ext(int kind, const uint16_t* src, int dtype, size_t n, uint8_t* q,
                        uint16_t* params);
int zo_dequant_groups_ext(int kind, const uint8_t* q, const uint16_t* params, int dtype, size_t n,
                          uint16_t* dst);
void zo_f32_to_e4m3_array(const float* src, uint8_t* dst, size_t n);
void zo_e4m3_to_f32_array(const uint8_t* src, float* dst, size_t n);

#ifdef __cplusplus
}
#endif
#endif
