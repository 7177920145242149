/*
 * ztcp_keyring.h -- C ABI of the session key ring that guards the cold-page
 * codec's keys and nonces (host code, no GPU).
 *
 * Replaces the reference's EphemeralSessionKeyRing
 * (research/baseline_codec/fused_quant_crypto.py, "fqc", lines 99-659): the
 * per-(tenant, session) key derivation, the nonce burn before encryption, the
 * monotonic per-slot freshness watermarks checked after decryption, and the
 * generation-bound crypto-shred.  Semantics follow the reference method by
 * method (each declaration cites it); the state lives in native memory behind
 * one mutex per key ring.
 *
 * Strings are NUL-terminated UTF-8 (tenant and session ids, as the reference
 * formats them into the derivation label).  Keys are 32-byte buffers.
 *
 * Return codes: 0 = success, negative = failure.  The failure's message (the
 * reference's exception text) is available from ztcp_keyring_last_error() on
 * the calling thread until its next key-ring call.
 */
#ifndef ZTCP_KEYRING_H
#define ZTCP_KEYRING_H

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

#define ZTCP_KR_EINVAL (-1)        /* ValueError (bad argument) */
#define ZTCP_KR_ESTALE (-10)       /* StalePageReplayError (fqc:64-65) */
#define ZTCP_KR_ENONCE (-11)       /* NonceReuseError (fqc:68-69) */
#define ZTCP_KR_ESHREDDED (-12)    /* SessionShreddedError (fqc:72-73) */
#define ZTCP_KR_ENOMEM (-13)       /* allocation failed */
#define ZTCP_KR_ERANDOM (-14)      /* the OS random source failed */

typedef struct ztcp_keyring ztcp_keyring;
/* A staged nonce reservation (fqc:76-97): owns copies of the session keys,
 * the burned nonces and the slot watermarks to commit.  Created by
 * ztcp_keyring_preflight_egress, freed by ztcp_keyring_release_reservation. */
typedef struct ztcp_reservation ztcp_reservation;

/* One decoded header for the batch freshness check (fqc:543-603). */
typedef struct ztcp_freshness_record {
    uint32_t model_id_hash;
    uint16_t layer_id;
    uint16_t head_group_id;
    uint64_t page_token_hash;
    uint64_t sequence_nonce;
} ztcp_freshness_record;

/* EphemeralSessionKeyRing(deployment_pepper) (fqc:125-157): the pepper must be
 * at least 32 bytes. */
ZTCP_API int ztcp_keyring_create(const uint8_t* pepper, size_t pepper_len, ztcp_keyring** out);
/* Zeroizes every key buffer and frees the key ring.  Release every
 * reservation first: any still registered are zeroized and freed here, and
 * their handles must not be used afterwards. */
ZTCP_API void ztcp_keyring_destroy(ztcp_keyring* kr);

/* derive_or_get (fqc:196-239): the session's keys, deriving them on first use
 * (HMAC-SHA256 of the pepper over "tenant:session:gen=G:" || 32 random bytes,
 * then HMAC-SHA256 labels "ztcp-cold-page-enc-v1\x01" / "...mac-v1\x02").
 * Any output pointer may be NULL. */
ZTCP_API int ztcp_keyring_derive_or_get(ztcp_keyring* kr, const char* tenant, const char* session,
                               uint8_t enc_key[32], uint8_t mac_key[32], uint64_t* generation);
/* The same derivation with the 32 "random" bytes supplied by the caller, for
 * known-answer tests of the derivation only (no counterpart in the
 * reference; production callers use ztcp_keyring_derive_or_get). */
ZTCP_API int ztcp_keyring_derive_with_secret_for_test(ztcp_keyring* kr, const char* tenant, const char* session,
                                             const uint8_t secret[32], uint8_t enc_key[32],
                                             uint8_t mac_key[32], uint64_t* generation);

/* next_sequence_nonce (fqc:241-255): a fresh range [base, base + count). */
ZTCP_API int ztcp_keyring_next_sequence_nonce(ztcp_keyring* kr, const char* tenant, const char* session,
                                     uint64_t count, uint64_t* base);

/* preflight_validate_egress (fqc:257-341): checks every page of an egress
 * batch (page b: sequence base + b, token_hashes[b]) against the slot
 * watermarks (stale -> ZTCP_KR_ESTALE) and the burned nonces (reuse ->
 * ZTCP_KR_ENONCE), then burns the batch's nonces and returns a reservation. */
ZTCP_API int ztcp_keyring_preflight_egress(ztcp_keyring* kr, const char* tenant, const char* session,
                                  uint32_t model_id_hash, uint16_t layer_id, uint16_t head_group_id,
                                  uint64_t base_sequence_nonce, const uint64_t* token_hashes, size_t n,
                                  ztcp_reservation** out);
/* begin_egress_execution (fqc:356-395): the reservation's key snapshots, or
 * ZTCP_KR_ESHREDDED if its generation was shredded. */
ZTCP_API int ztcp_keyring_begin_egress(ztcp_keyring* kr, const char* tenant, const char* session,
                              ztcp_reservation* res, uint8_t enc_key[32], uint8_t mac_key[32]);
/* commit_egress (fqc:397-434): advances the slot watermarks monotonically. */
ZTCP_API int ztcp_keyring_commit_egress(ztcp_keyring* kr, const char* tenant, const char* session,
                               ztcp_reservation* res);
/* release_egress_reservation (fqc:436-458): zeroizes and frees it. */
ZTCP_API void ztcp_keyring_release_reservation(ztcp_keyring* kr, const char* tenant, const char* session,
                                      ztcp_reservation* res);
/* Last sequence nonce of a reservation (base + n - 1). */
ZTCP_API uint64_t ztcp_reservation_last_sequence(const ztcp_reservation* res);
/* Key generation a reservation is bound to (fqc:87, _StagedNonceReservation.generation). */
ZTCP_API uint64_t ztcp_reservation_generation(const ztcp_reservation* res);

/* begin_ingress (fqc:460-471). */
ZTCP_API int ztcp_keyring_begin_ingress(ztcp_keyring* kr, const char* tenant, const char* session,
                               uint64_t* generation, uint8_t enc_key[32], uint8_t mac_key[32]);
/* verify_and_update_freshness (fqc:473-541); each optional check is enabled
 * by a non-NULL pointer. */
ZTCP_API int ztcp_keyring_verify_freshness(ztcp_keyring* kr, const char* tenant, const char* session,
                                  uint32_t model_id_hash, uint16_t layer_id, uint16_t head_group_id,
                                  uint64_t page_token_hash, uint64_t sequence_nonce,
                                  const uint64_t* min_sequence_nonce,
                                  const uint64_t* expected_sequence_nonce,
                                  const uint64_t* expected_generation);
/* verify_and_update_freshness_batch (fqc:543-603): all records are checked
 * before any watermark moves. */
ZTCP_API int ztcp_keyring_verify_freshness_batch(ztcp_keyring* kr, const char* tenant, const char* session,
                                        const ztcp_freshness_record* records, size_t n,
                                        const uint64_t* min_sequence_nonce,
                                        const uint64_t* expected_generation);
/* finish_ingress (fqc:605-618). */
ZTCP_API int ztcp_keyring_finish_ingress(ztcp_keyring* kr, const char* tenant, const char* session,
                                uint64_t expected_generation);

/* crypto_shred_session (fqc:647-650): 1 if the session existed, else 0. */
ZTCP_API int ztcp_keyring_shred_session(ztcp_keyring* kr, const char* tenant, const char* session);
/* crypto_shred_tenant (fqc:652-658): the number of sessions shredded. */
ZTCP_API int ztcp_keyring_shred_tenant(ztcp_keyring* kr, const char* tenant);

/* Message of the calling thread's last failing key-ring call ("" if none). */
ZTCP_API const char* ztcp_keyring_last_error(void);

/* SHA-256 (FIPS 180-4) and HMAC-SHA256 (RFC 2104) of the derivation, exposed
 * for known-answer tests. */
ZTCP_API void ztcp_sha256(const uint8_t* data, size_t len, uint8_t out[32]);
ZTCP_API void ztcp_hmac_sha256(const uint8_t* key, size_t key_len, const uint8_t* data, size_t len, uint8_t out[32]);

#ifdef __cplusplus
}
#endif
#endif /* ZTCP_KEYRING_H */
