"""Plain-Python restatement of the reference's session key ring.

TEST INFRASTRUCTURE ONLY: tests/ compare the native key ring
(include/ztcp_keyring.h) with this model, operation by operation, on the
same inputs.  Nothing in the product imports it.

It restates EphemeralSessionKeyRing
(research/baseline_codec/fused_quant_crypto.py, "fqc") with the standard
library's ``hmac`` / ``hashlib`` for the key schedule; each method cites the
lines it follows.  Error classes are given by name (the tests map them to the
product's exception classes) and messages are the reference's text.

Pinned by: the standard library's HMAC-SHA256 (an independent implementation
of RFC 2104 / FIPS 180-4), and by the reference benchmark's own key-ring
assertions (research/benchmarks/bench_cold_page_pipeline.py:216-610: nonce
reuse, stale replay, out-of-order commit, shred + re-derive) which the tests
run against this model and the native ring alike.
"""
from __future__ import annotations

import hashlib
import hmac
import os
import threading

M64 = (1 << 64) - 1


class ModelError(Exception):
    """An error of the model: ``kind`` is the reference's exception class name."""

    def __init__(self, kind: str, msg: str):
        super().__init__(msg)
        self.kind = kind


class Reservation:
    """fqc:76-97: the staged nonces' generation, key copies, revocation flag."""

    def __init__(self, key, generation, enc, mac, slots, last_seq):
        self.key = key
        self.generation = generation
        self.enc = bytearray(enc)
        self.mac = bytearray(mac)
        self.slots = slots
        self.last_seq = last_seq
        self.revoked = False

    def zeroize(self):
        self.enc[:] = bytes(len(self.enc))
        self.mac[:] = bytes(len(self.mac))


class KeyRingModel:
    def __init__(self, pepper: bytes):
        if len(pepper) < 32:  # fqc:155-157
            raise ModelError("ValueError", "deployment_pepper must be at least 32 bytes")
        self.pepper = bytes(pepper)
        self.lock = threading.RLock()
        self.keys: dict = {}          # (tenant, session) -> (enc bytearray, mac bytearray)
        self.gen: dict = {}
        self.shredded: dict = {}
        self.used: dict = {}          # -> set of 12-byte nonces
        self.marks: dict = {}         # -> {(model, layer, hg, token): seq}
        self.max_seq: dict = {}
        self.inflight: dict = {}      # ((tenant, session), gen) -> [Reservation]

    # fqc:168-194
    def _active_gen(self, key) -> int:
        if key not in self.keys:
            raise ModelError("SessionShreddedError", f"Session {key} key is missing or crypto-shredded")
        enc, mac = self.keys[key]
        if not any(enc) or not any(mac):
            raise ModelError("SessionShreddedError", f"Session {key} key buffer was zeroized or crypto-shredded")
        if key not in self.gen:
            self.gen[key] = self.shredded.get(key, 0) + 1
        return self.gen[key]

    # fqc:196-239
    def _derive(self, key, secret: bytes):
        g = max(self.gen.get(key, 0), self.shredded.get(key, 0)) + 1
        self.gen[key] = g
        label = f"{key[0]}:{key[1]}:gen={g}:".encode("utf-8")
        prk = hmac.new(self.pepper, label + bytes(secret), hashlib.sha256).digest()
        enc = bytearray(hmac.new(prk, b"ztcp-cold-page-enc-v1\x01", hashlib.sha256).digest())
        mac = bytearray(hmac.new(prk, b"ztcp-cold-page-mac-v1\x02", hashlib.sha256).digest())
        self.keys[key] = (enc, mac)
        self.used[key] = set()
        self.marks[key] = {}
        self.max_seq[key] = 0
        self.inflight[(key, g)] = []

    def derive_or_get(self, tenant, session, secret: bytes | None = None):
        with self.lock:
            key = (tenant, session)
            if key in self.keys:
                g = self._active_gen(key)
            else:
                self._derive(key, os.urandom(32) if secret is None else secret)
                g = self.gen[key]
            enc, mac = self.keys[key]
            return bytes(enc), bytes(mac), g

    # fqc:241-255
    def next_sequence_nonce(self, tenant, session, count=1):
        if count < 1:
            raise ModelError("ValueError", "count must be >= 1")
        with self.lock:
            key = (tenant, session)
            if key not in self.keys:
                self.derive_or_get(tenant, session)
            self._active_gen(key)
            base = self.max_seq.get(key, 0) + 1
            self.max_seq[key] = base + count - 1
            return base

    # fqc:257-341
    def preflight(self, tenant, session, model, layer, hg, base, token_hashes):
        if len(token_hashes) == 0:
            raise ModelError("ValueError", "token_hashes must be non-empty")
        with self.lock:
            key = (tenant, session)
            if key not in self.keys:
                self.derive_or_get(tenant, session)
            g = self._active_gen(key)
            used = self.used.setdefault(key, set())
            marks = self.marks.setdefault(key, {})
            loc = (((layer & 0xFFFF) << 16) | (hg & 0xFFFF)).to_bytes(4, "little")
            staged, slots = set(), {}
            for i, th in enumerate(token_hashes):
                seq = (base + i) & M64
                slot = (model & 0xFFFFFFFF, layer & 0xFFFF, hg & 0xFFFF, th & M64)
                prev = slots[slot] if slot in slots else marks.get(slot, 0)
                if seq < prev:
                    raise ModelError("StalePageReplayError",
                                     f"STALE_PAGE_REPLAY: Cannot encode cold page with stale sequence_nonce={seq} < latest={prev}")
                nonce = seq.to_bytes(8, "little") + loc
                if nonce in used or nonce in staged:
                    raise ModelError("NonceReuseError",
                                     f"NONCE_REUSE_DETECTED: Final 96-bit ChaCha20 nonce {nonce.hex()} already used under session {key}")
                staged.add(nonce)
                slots[slot] = seq
            enc, mac = self.keys[key]
            last = (base + len(token_hashes) - 1) & M64
            r = Reservation(key, g, enc, mac, slots, last)
            self.inflight.setdefault((key, g), []).append(r)
            used.update(staged)
            if last > self.max_seq.get(key, 0):
                self.max_seq[key] = last
            return r

    def _check_res(self, key, r, when):
        g = r.generation
        if (r.revoked or key not in self.keys or self.gen.get(key) != g
                or self.shredded.get(key, 0) >= g):
            r.zeroize()
            raise ModelError("SessionShreddedError",
                             f"Session ({key[0]}, {key[1]}) generation {g} was crypto-shredded {when}")

    # fqc:356-395
    def begin_egress(self, tenant, session, r):
        with self.lock:
            key = (tenant, session)
            self._check_res(key, r, "before or during egress")
            if not any(r.enc) or not any(r.mac):
                r.zeroize()
                raise ModelError("SessionShreddedError",
                                 f"Session ({tenant}, {session}) generation {r.generation} key buffer was zeroized")
            return bytes(r.enc), bytes(r.mac)

    # fqc:397-434
    def commit_egress(self, tenant, session, r):
        with self.lock:
            key = (tenant, session)
            self._check_res(key, r, "before commit")
            marks = self.marks.setdefault(key, {})
            for slot, seq in r.slots.items():
                if seq > marks.get(slot, 0):
                    marks[slot] = seq
            if r.last_seq > self.max_seq.get(key, 0):
                self.max_seq[key] = r.last_seq

    # fqc:436-458
    def release(self, tenant, session, r):
        with self.lock:
            r.zeroize()
            lst = self.inflight.get(((tenant, session), r.generation))
            if lst is not None and r in lst:
                lst.remove(r)

    # fqc:460-471
    def begin_ingress(self, tenant, session):
        with self.lock:
            key = (tenant, session)
            if key not in self.keys:
                raise ModelError("SessionShreddedError",
                                 f"Session ({tenant}, {session}) key is missing or crypto-shredded")
            g = self._active_gen(key)
            enc, mac = self.keys[key]
            return g, bytes(enc), bytes(mac)

    def _ingress_gen(self, key, expected_generation):
        if key not in self.keys:
            raise ModelError("SessionShreddedError",
                             f"Session ({key[0]}, {key[1]}) key is missing or crypto-shredded")
        cur = self._active_gen(key)
        if expected_generation is not None and (
                cur != expected_generation or self.shredded.get(key, 0) >= expected_generation):
            raise ModelError("SessionShreddedError",
                             f"Session ({key[0]}, {key[1]}) generation {expected_generation} was crypto-shredded during ingress")

    # fqc:473-541
    def verify_freshness(self, tenant, session, model, layer, hg, token, seq, min_seq=None,
                         expected_seq=None, expected_generation=None):
        with self.lock:
            key = (tenant, session)
            self._ingress_gen(key, expected_generation)
            seq &= M64
            if expected_seq is not None and seq != (expected_seq & M64):
                raise ModelError("StalePageReplayError",
                                 f"STALE_PAGE_REPLAY: Cold-page sequence_nonce={seq} != expected_sequence_nonce={expected_seq & M64}")
            if min_seq is not None and seq < (min_seq & M64):
                raise ModelError("StalePageReplayError",
                                 f"STALE_PAGE_REPLAY: Cold-page sequence_nonce={seq} < min_sequence_nonce={min_seq & M64}")
            marks = self.marks.setdefault(key, {})
            slot = (model & 0xFFFFFFFF, layer & 0xFFFF, hg & 0xFFFF, token & M64)
            latest = marks.get(slot, 0)
            if seq < latest:
                raise ModelError("StalePageReplayError",
                                 f"STALE_PAGE_REPLAY: Cold-page sequence_nonce={seq} is older than latest slot version={latest}")
            if seq > latest:
                marks[slot] = seq
            if seq > self.max_seq.get(key, 0):
                self.max_seq[key] = seq

    # fqc:543-603
    def verify_freshness_batch(self, tenant, session, records, min_seq=None, expected_generation=None):
        with self.lock:
            key = (tenant, session)
            self._ingress_gen(key, expected_generation)
            marks = self.marks.setdefault(key, {})
            top = self.max_seq.get(key, 0)
            staged = {}
            for m, l, g, t, s in records:
                s &= M64
                if min_seq is not None and s < (min_seq & M64):
                    raise ModelError("StalePageReplayError",
                                     f"STALE_PAGE_REPLAY: Cold-page sequence_nonce={s} < min_sequence_nonce={min_seq & M64}")
                slot = (m & 0xFFFFFFFF, l & 0xFFFF, g & 0xFFFF, t & M64)
                latest = staged[slot] if slot in staged else marks.get(slot, 0)
                if s < latest:
                    raise ModelError("StalePageReplayError",
                                     f"STALE_PAGE_REPLAY: Cold-page sequence_nonce={s} is older than latest slot version={latest}")
                if s > latest:
                    staged[slot] = s
                top = max(top, s)
            marks.update(staged)
            self.max_seq[key] = top

    # fqc:605-618
    def finish_ingress(self, tenant, session, expected_generation):
        with self.lock:
            key = (tenant, session)
            if (key not in self.keys or self.gen.get(key) != expected_generation
                    or self.shredded.get(key, 0) >= expected_generation):
                raise ModelError("SessionShreddedError",
                                 f"Session ({tenant}, {session}) generation {expected_generation} was crypto-shredded during ingress")

    # fqc:620-645
    def _shred(self, key) -> bool:
        g = self.gen.get(key, 1)
        bufs = self.keys.pop(key, None)
        if bufs is not None:
            for b in bufs:
                b[:] = bytes(len(b))
        for r in self.inflight.pop((key, g), []):
            r.revoked = True
            r.zeroize()
        self.used.pop(key, None)
        self.marks.pop(key, None)
        self.max_seq.pop(key, None)
        if bufs is not None:
            self.shredded[key] = max(self.shredded.get(key, 0), g)
        return bufs is not None

    # fqc:647-658
    def shred_session(self, tenant, session) -> bool:
        with self.lock:
            return self._shred((tenant, session))

    def shred_tenant(self, tenant) -> int:
        with self.lock:
            keys = [k for k in self.keys if k[0] == tenant]
            for k in keys:
                self._shred(k)
            return len(keys)
