"""Session key ring of the cold-page codec: Python face of the native key ring.

The state and every check live in native code (include/ztcp_keyring.h,
csrc/ztcp_keyring.cpp) behind one mutex; this module gives it the API of the
reference's ``EphemeralSessionKeyRing``
(research/baseline_codec/fused_quant_crypto.py:99-659) -- same method names,
argument names and order, return shapes, exception classes and messages --
so the codec class and callers written against the reference run unchanged.

Differences:
  * key material never leaves native memory except as copies: ``derive_or_get``
    returns fresh ``bytearray`` copies (zeroing them does not shred the
    session; ``crypto_shred_session`` does), and a reservation's key snapshots
    are native;
  * ``preflight_validate_egress`` returns ``(reservation, reservation,
    last_seq)``: the staged slot watermarks live inside the native
    reservation, so the second element is the reservation itself and
    ``commit_egress`` takes its watermarks from there (the reference's legacy
    plain-``set`` staging form is not supported);
  * token hashes may be given as a list of ints or as a 1-D integer tensor /
    array (no per-page Python objects on the fast path);
  * ``verify_and_update_freshness_batch`` also accepts the headers' 24-byte
    tails (``blob[8:32]``: model hash, layer, head group, token hash,
    sequence nonce -- the native record layout) as an ``(n, 24)`` uint8 array;
  * tenant and session ids may not contain NUL characters (``ValueError``).
"""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np

from . import _native as N

_M64 = (1 << 64) - 1

# Native freshness record (include/ztcp_keyring.h): the header's bytes 8..32.
RECORD_DTYPE = np.dtype([("model_id_hash", "<u4"), ("layer_id", "<u2"), ("head_group_id", "<u2"),
                         ("page_token_hash", "<u8"), ("sequence_nonce", "<u8")])
assert RECORD_DTYPE.itemsize == 24


class KVIntegrityError(RuntimeError):
    """A cold page failed MAC authentication (fqc:56-57)."""


class CrossTenantContaminationError(KVIntegrityError):
    """A cold page's AAD does not match the requesting tenant/model/layer (fqc:60-61)."""


class StalePageReplayError(KVIntegrityError):
    """A cold page's sequence_nonce is older than the latest slot version (fqc:64-65)."""


class NonceReuseError(ValueError):
    """An encode would reuse a ChaCha20 nonce under the same session key (fqc:68-69)."""


class SessionShreddedError(RuntimeError):
    """The session's ephemeral key was crypto-shredded (fqc:72-73)."""


_ERRORS = {
    N.KR_EINVAL: ValueError,
    N.KR_ESTALE: StalePageReplayError,
    N.KR_ENONCE: NonceReuseError,
    N.KR_ESHREDDED: SessionShreddedError,
    N.KR_ENOMEM: MemoryError,
    N.KR_ERANDOM: OSError,
}


def _raise(rc: int) -> None:
    if rc >= 0:
        return
    msg = N.lib().ztcp_keyring_last_error().decode("utf-8", "replace")
    raise _ERRORS.get(rc, RuntimeError)(msg or f"key ring error {rc}")


def _id(s: str) -> bytes:
    if not isinstance(s, str):
        raise TypeError(f"tenant and session ids must be str, got {type(s).__name__}")
    if "\x00" in s:
        raise ValueError("tenant and session ids must not contain NUL characters")
    return s.encode("utf-8")


def _u64_array(token_hashes) -> np.ndarray:
    """Token hashes as a contiguous uint64 array (values taken mod 2**64)."""
    try:
        import torch

        if isinstance(token_hashes, torch.Tensor):
            if token_hashes.dtype.is_floating_point or token_hashes.dtype.is_complex:
                raise TypeError("token hashes must be integers")
            t = token_hashes.reshape(-1).to(device="cpu", dtype=torch.int64)
            return np.ascontiguousarray(t.numpy().view(np.uint64))
    except ImportError:  # pragma: no cover - torch is always present with the codec
        pass
    if isinstance(token_hashes, np.ndarray):
        if token_hashes.dtype.kind not in "iu":
            raise TypeError("token hashes must be integers")
        flat = token_hashes.reshape(-1)
        if flat.dtype.kind == "i":
            flat = flat.astype(np.int64, copy=False).view(np.uint64)
        return np.ascontiguousarray(flat, dtype=np.uint64)
    return np.fromiter((int(t) & _M64 for t in token_hashes), dtype=np.uint64)


class _StagedNonceReservation:
    """Handle of a native staged nonce reservation (fqc:76-97).

    Owns native copies of the session keys, the burned nonces' slot
    watermarks and the last sequence nonce; released (zeroized, unregistered,
    freed) by ``release_egress_reservation`` or when collected."""

    __slots__ = ("_ring", "_ptr", "tenant_id", "session_id", "generation", "last_sequence")

    def __init__(self, ring: "EphemeralSessionKeyRing", ptr: int, tenant_id: str, session_id: str):
        self._ring = ring
        self._ptr = ptr
        self.tenant_id = tenant_id
        self.session_id = session_id
        L = N.lib()
        self.generation = int(L.ztcp_reservation_generation(ptr))
        self.last_sequence = int(L.ztcp_reservation_last_sequence(ptr))

    def _release(self) -> None:
        ptr, self._ptr = self._ptr, None
        if ptr is not None and self._ring._h is not None:
            N.lib().ztcp_keyring_release_reservation(self._ring._h, _id(self.tenant_id),
                                                     _id(self.session_id), ptr)

    def __del__(self):
        try:
            self._release()
        except Exception:
            pass


class EphemeralSessionKeyRing:
    """Per-tenant / per-session ephemeral keys, nonce uniqueness, freshness and
    crypto-shredding (fqc:99-659), held in native memory.

    Every state transition is one native call under the key ring's mutex (the
    reference's re-entrant lock); ctypes releases the GIL around it."""

    def __init__(self, deployment_pepper: bytes):
        pepper = bytes(deployment_pepper)
        if len(pepper) < 32:  # fqc:155-157
            raise ValueError("deployment_pepper must be at least 32 bytes")
        h = C.c_void_p()
        _raise(N.lib().ztcp_keyring_create(pepper, len(pepper), C.byref(h)))
        self._h = h.value

    def close(self) -> None:
        """Zeroize every key buffer and free the native key ring."""
        h, self._h = self._h, None
        if h is not None:
            N.lib().ztcp_keyring_destroy(h)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _handle(self) -> int:
        if self._h is None:
            raise SessionShreddedError("key ring is closed")
        return self._h

    @staticmethod
    def pack_chacha20_nonce(sequence_nonce: int, layer_id: int, head_group_id: int) -> bytes:
        """96-bit ChaCha20 nonce: sequence (64 b) || layer (16 b) || head group (16 b) (fqc:159-166)."""
        seq = sequence_nonce & _M64
        loc = ((layer_id & 0xFFFF) << 16) | (head_group_id & 0xFFFF)
        return struct.pack("<3I", seq & 0xFFFFFFFF, seq >> 32, loc)

    # ---- keys ------------------------------------------------------------------

    def derive_or_get(self, tenant_id: str, session_id: str) -> tuple[bytearray, bytearray, int, int]:
        """(enc_key_32b, mac_key_32b, k0_u64, k1_u64) of the session (fqc:196-239)."""
        enc, mac = (C.c_uint8 * 32)(), (C.c_uint8 * 32)()
        gen = C.c_uint64()
        _raise(N.lib().ztcp_keyring_derive_or_get(self._handle(), _id(tenant_id), _id(session_id),
                                                  enc, mac, C.byref(gen)))
        e, m = bytearray(enc), bytearray(mac)
        C.memset(enc, 0, 32)
        C.memset(mac, 0, 32)
        k0, k1 = struct.unpack("<QQ", e[:16])
        return e, m, k0, k1

    def session_generation(self, tenant_id: str, session_id: str) -> int:
        """Current key generation of an active session (derives it on first use)."""
        gen = C.c_uint64()
        _raise(N.lib().ztcp_keyring_derive_or_get(self._handle(), _id(tenant_id), _id(session_id),
                                                  None, None, C.byref(gen)))
        return gen.value

    def next_sequence_nonce(self, tenant_id: str, session_id: str, count: int = 1) -> int:
        """A fresh monotonic sequence_nonce range [base, base + count) (fqc:241-255)."""
        if count < 1:
            raise ValueError("count must be >= 1")
        base = C.c_uint64()
        _raise(N.lib().ztcp_keyring_next_sequence_nonce(self._handle(), _id(tenant_id), _id(session_id),
                                                        count & _M64, C.byref(base)))
        return base.value

    # ---- egress transaction ----------------------------------------------------------

    def preflight_validate_egress(self, tenant_id: str, session_id: str, model_id_hash: int,
                                  layer_id: int, head_group_id: int, base_sequence_nonce: int,
                                  token_hashes) -> tuple[_StagedNonceReservation, _StagedNonceReservation, int]:
        """Validate and burn the batch's ChaCha20 nonces before encryption (fqc:257-341)."""
        th = _u64_array(token_hashes)
        if th.size == 0:
            raise ValueError("token_hashes must be non-empty")
        res = C.c_void_p()
        _raise(N.lib().ztcp_keyring_preflight_egress(
            self._handle(), _id(tenant_id), _id(session_id), model_id_hash & 0xFFFFFFFF,
            layer_id & 0xFFFF, head_group_id & 0xFFFF, base_sequence_nonce & _M64,
            th.ctypes.data, th.size, C.byref(res)))
        r = _StagedNonceReservation(self, res.value, tenant_id, session_id)
        return r, r, r.last_sequence

    def _reservation(self, staged_nonces) -> int:
        if not isinstance(staged_nonces, _StagedNonceReservation) or staged_nonces._ring is not self:
            raise TypeError("staged_nonces must be a reservation returned by this key ring's "
                            "preflight_validate_egress")
        if staged_nonces._ptr is None:
            raise SessionShreddedError(
                f"Session ({staged_nonces.tenant_id}, {staged_nonces.session_id}) generation "
                f"{staged_nonces.generation} reservation was already released")
        return staged_nonces._ptr

    def begin_egress_execution(self, tenant_id: str, session_id: str, staged_nonces) -> tuple[bytes, bytes]:
        """Key snapshots of a reservation whose generation is still live (fqc:356-395)."""
        enc, mac = (C.c_uint8 * 32)(), (C.c_uint8 * 32)()
        _raise(N.lib().ztcp_keyring_begin_egress(self._handle(), _id(tenant_id), _id(session_id),
                                                 self._reservation(staged_nonces), enc, mac))
        e, m = bytes(enc), bytes(mac)
        C.memset(enc, 0, 32)
        C.memset(mac, 0, 32)
        return e, m

    def commit_egress(self, tenant_id: str, session_id: str, staged_nonces, staged_slots=None,
                      last_seq: int | None = None) -> None:
        """Advance the reservation's slot watermarks monotonically (fqc:397-434)."""
        _raise(N.lib().ztcp_keyring_commit_egress(self._handle(), _id(tenant_id), _id(session_id),
                                                  self._reservation(staged_nonces)))

    def release_egress_reservation(self, tenant_id: str, session_id: str, staged_nonces) -> None:
        """Zeroize the reservation's key copies and unregister it (fqc:436-458)."""
        if isinstance(staged_nonces, _StagedNonceReservation) and staged_nonces._ring is self:
            staged_nonces._release()

    # ---- ingress transaction ---------------------------------------------------------

    def begin_ingress(self, tenant_id: str, session_id: str) -> tuple[int, bytes, bytes]:
        """(generation, enc_key, mac_key) snapshots for an ingress decode (fqc:460-471)."""
        enc, mac = (C.c_uint8 * 32)(), (C.c_uint8 * 32)()
        gen = C.c_uint64()
        _raise(N.lib().ztcp_keyring_begin_ingress(self._handle(), _id(tenant_id), _id(session_id),
                                                  C.byref(gen), enc, mac))
        e, m = bytes(enc), bytes(mac)
        C.memset(enc, 0, 32)
        C.memset(mac, 0, 32)
        return gen.value, e, m

    @staticmethod
    def _opt(v: int | None):
        return None if v is None else C.byref(C.c_uint64(v & _M64))

    def verify_and_update_freshness(self, tenant_id: str, session_id: str, model_id_hash: int,
                                    layer_id: int, head_group_id: int, page_token_hash: int,
                                    sequence_nonce: int, min_sequence_nonce: int | None = None,
                                    expected_sequence_nonce: int | None = None,
                                    expected_generation: int | None = None) -> None:
        """Freshness contract after MAC authentication (fqc:473-541)."""
        _raise(N.lib().ztcp_keyring_verify_freshness(
            self._handle(), _id(tenant_id), _id(session_id), model_id_hash & 0xFFFFFFFF,
            layer_id & 0xFFFF, head_group_id & 0xFFFF, page_token_hash & _M64, sequence_nonce & _M64,
            self._opt(min_sequence_nonce), self._opt(expected_sequence_nonce),
            self._opt(expected_generation)))

    def verify_and_update_freshness_batch(self, tenant_id: str, session_id: str, records,
                                          min_sequence_nonce: int | None = None,
                                          expected_generation: int | None = None) -> None:
        """All-or-nothing freshness check of a batch of decoded headers (fqc:543-603).

        ``records``: (model_id_hash, layer_id, head_group_id, token_hash,
        sequence_nonce) tuples, or an ``(n, 24)`` uint8 array of header bytes
        8..32, or an array of ``RECORD_DTYPE``."""
        if isinstance(records, np.ndarray) and records.dtype == np.uint8:
            if records.ndim != 2 or records.shape[1] != 24:
                raise ValueError("header-tail records must have shape (n, 24)")
            arr = np.ascontiguousarray(records).view(RECORD_DTYPE).reshape(-1)
        elif isinstance(records, np.ndarray) and records.dtype == RECORD_DTYPE:
            arr = np.ascontiguousarray(records.reshape(-1))
        else:
            arr = np.array([(m & 0xFFFFFFFF, l & 0xFFFF, g & 0xFFFF, t & _M64, s & _M64)
                            for m, l, g, t, s in records], dtype=RECORD_DTYPE)
        _raise(N.lib().ztcp_keyring_verify_freshness_batch(
            self._handle(), _id(tenant_id), _id(session_id), arr.ctypes.data if arr.size else None,
            arr.size, self._opt(min_sequence_nonce), self._opt(expected_generation)))

    def finish_ingress(self, tenant_id: str, session_id: str, expected_generation: int) -> None:
        """The session generation is still live right before decoded pages are returned (fqc:605-618)."""
        _raise(N.lib().ztcp_keyring_finish_ingress(self._handle(), _id(tenant_id), _id(session_id),
                                                   expected_generation & _M64))

    # ---- crypto-shred -------------------------------------------------------------

    def crypto_shred_session(self, tenant_id: str, session_id: str) -> bool:
        """Zero the session's key buffers and revoke its in-flight operations (fqc:647-650)."""
        rc = N.lib().ztcp_keyring_shred_session(self._handle(), _id(tenant_id), _id(session_id))
        _raise(rc)
        return rc == 1

    def crypto_shred_tenant(self, tenant_id: str) -> int:
        """Shred every active session of a tenant; returns how many (fqc:652-658)."""
        rc = N.lib().ztcp_keyring_shred_tenant(self._handle(), _id(tenant_id))
        _raise(rc)
        return rc

    # ---- known-answer hooks --------------------------------------------------------

    def _derive_with_secret_for_test(self, tenant_id: str, session_id: str,
                                     secret: bytes) -> tuple[bytes, bytes, int]:
        """Derivation with caller-supplied 32 "random" bytes (tests of the key schedule only)."""
        if len(secret) != 32:
            raise ValueError("secret must be 32 bytes")
        enc, mac = (C.c_uint8 * 32)(), (C.c_uint8 * 32)()
        gen = C.c_uint64()
        _raise(N.lib().ztcp_keyring_derive_with_secret_for_test(
            self._handle(), _id(tenant_id), _id(session_id), bytes(secret), enc, mac, C.byref(gen)))
        return bytes(enc), bytes(mac), gen.value


def sha256(data: bytes) -> bytes:
    """Native SHA-256 (FIPS 180-4) of the key schedule."""
    out = (C.c_uint8 * 32)()
    N.lib().ztcp_sha256(bytes(data), len(data), out)
    return bytes(out)


def hmac_sha256(key: bytes, data: bytes) -> bytes:
    """Native HMAC-SHA256 (RFC 2104) of the key schedule."""
    out = (C.c_uint8 * 32)()
    N.lib().ztcp_hmac_sha256(bytes(key), len(key), bytes(data), len(data), out)
    return bytes(out)
