"""Session key ring (include/ztcp_keyring.h): key schedule, nonce burn,
freshness watermarks and crypto-shred.  Host code, no GPU.

* SHA-256 / HMAC-SHA256 are pinned by FIPS 180-4 and RFC 4231 known answers
  and by the standard library on every length around the block boundaries.
* The key derivation (fqc:196-239) is pinned by the standard library's HMAC
  over the reference's labels, with the 32 random bytes supplied.
* The state machine is run against the plain-Python model in
  oracle/keyring_model.py: the reference benchmark's own key-ring assertions
  (research/benchmarks/bench_cold_page_pipeline.py:404-610) on both, then a
  seeded random operation sequence compared call by call (result, error class
  and message).
"""
from __future__ import annotations

import hashlib
import hmac
import random
import struct
import threading

import numpy as np
import pytest


@pytest.fixture(scope="module")
def KR(pkg):
    import vlx_tee_amd.keyring as KR

    return KR


@pytest.fixture(scope="module")
def M():
    from oracle import keyring_model as M

    return M


PEPPER = bytes(range(7, 7 + 48))


# ---- SHA-256 and HMAC -------------------------------------------------------------

SHA_KAT = [  # FIPS 180-4 examples (NIST CSRC "SHA256.pdf" / "SHA2_Additional.pdf")
    (b"", "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"),
    (b"abc", "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"),
    (b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq",
     "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"),
    (b"a" * 1_000_000, "cdc76e5c9914fb9281a1c7e284d73e67f1809a48a497200e046d39ccc7112cd0"),
]

HMAC_KAT = [  # RFC 4231 test cases 1, 2, 3, 4, 6, 7 (HMAC-SHA-256)
    (b"\x0b" * 20, b"Hi There", "b0344c61d8db38535ca8afceaf0bf12b881dc200c9833da726e9376c2e32cff7"),
    (b"Jefe", b"what do ya want for nothing?",
     "5bdcc146bf60754e6a042426089575c75a003f089d2739839dec58b964ec3843"),
    (b"\xaa" * 20, b"\xdd" * 50, "773ea91e36800e46854db8ebd09181a72959098b3ef8c122d9635514ced565fe"),
    (bytes(range(1, 26)), b"\xcd" * 50, "82558a389a443c0ea4cc819899f2083a85f0faa3e578f8077a2e3ff46729665b"),
    (b"\xaa" * 131, b"Test Using Larger Than Block-Size Key - Hash Key First",
     "60e431591ee0b67f0d8a26aacbf5b77f8e0bc6213728c5140546040f0ee37f54"),
    (b"\xaa" * 131, b"This is a test using a larger than block-size key and a larger than block-size "
     b"data. The key needs to be hashed before being used by the HMAC algorithm.",
     "9b09ffa71b942fcb27635fbcd5b0e944bfdc63644f0713938a7f51535c3a35e2"),
]


@pytest.mark.parametrize("msg,want", SHA_KAT, ids=["empty", "abc", "448bit", "million_a"])
def test_sha256_fips_vectors(KR, msg, want):
    assert KR.sha256(msg).hex() == want


def test_sha256_every_length_around_blocks(KR):
    rng = np.random.default_rng(1)
    for n in list(range(0, 200)) + [1000, 4095, 4096, 4097]:
        m = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert KR.sha256(m) == hashlib.sha256(m).digest(), n


@pytest.mark.parametrize("key,msg,want", HMAC_KAT, ids=["tc1", "tc2", "tc3", "tc4", "tc6", "tc7"])
def test_hmac_rfc4231(KR, key, msg, want):
    assert KR.hmac_sha256(key, msg).hex() == want


def test_hmac_key_lengths(KR):
    rng = np.random.default_rng(2)
    for kl in (0, 1, 31, 32, 63, 64, 65, 128, 200):
        for ml in (0, 1, 55, 56, 64, 119, 300):
            k = rng.integers(0, 256, kl, dtype=np.uint8).tobytes()
            m = rng.integers(0, 256, ml, dtype=np.uint8).tobytes()
            assert KR.hmac_sha256(k, m) == hmac.new(k, m, hashlib.sha256).digest(), (kl, ml)


# ---- key schedule -------------------------------------------------------------------

def _schedule(pepper: bytes, tenant: str, session: str, gen: int, secret: bytes):
    """fqc:214-231 with the standard library."""
    prk = hmac.new(pepper, f"{tenant}:{session}:gen={gen}:".encode() + secret, hashlib.sha256).digest()
    return (hmac.new(prk, b"ztcp-cold-page-enc-v1\x01", hashlib.sha256).digest(),
            hmac.new(prk, b"ztcp-cold-page-mac-v1\x02", hashlib.sha256).digest())


def test_key_derivation_known_answer(KR, M):
    ring = KR.EphemeralSessionKeyRing(PEPPER)
    model = M.KeyRingModel(PEPPER)
    secret = bytes(range(100, 132))
    for tenant, session in [("tenant-alpha-bank", "sess-001"), ("ténänt", "s:1"), ("", "")]:
        enc, mac, gen = ring._derive_with_secret_for_test(tenant, session, secret)
        assert gen == 1
        assert (enc, mac) == _schedule(PEPPER, tenant, session, 1, secret)
        assert model.derive_or_get(tenant, session, secret) == (enc, mac, 1)
        e2, m2, k0, k1 = ring.derive_or_get(tenant, session)  # cached
        assert (bytes(e2), bytes(m2)) == (enc, mac) and (k0, k1) == struct.unpack("<QQ", enc[:16])
    # a shredded session re-derives under the next generation
    assert ring.crypto_shred_session("tenant-alpha-bank", "sess-001")
    enc, mac, gen = ring._derive_with_secret_for_test("tenant-alpha-bank", "sess-001", secret)
    assert gen == 2 and (enc, mac) == _schedule(PEPPER, "tenant-alpha-bank", "sess-001", 2, secret)
    with pytest.raises(ValueError):
        ring._derive_with_secret_for_test("tenant-alpha-bank", "sess-001", secret)  # already active


def test_random_derivation_is_fresh(KR):
    ring = KR.EphemeralSessionKeyRing(PEPPER)
    e1, m1, _, _ = ring.derive_or_get("t", "s")
    assert any(e1) and any(m1) and e1 != m1
    assert ring.crypto_shred_session("t", "s")
    e2, m2, _, _ = ring.derive_or_get("t", "s")
    assert e2 != e1 and m2 != m1
    other = KR.EphemeralSessionKeyRing(PEPPER)
    assert other.derive_or_get("t", "s")[0] not in (e1, e2)


def test_pepper_and_argument_errors(KR):
    with pytest.raises(ValueError, match="at least 32 bytes"):
        KR.EphemeralSessionKeyRing(b"x" * 31)
    ring = KR.EphemeralSessionKeyRing(PEPPER)
    with pytest.raises(ValueError, match="count must be >= 1"):
        ring.next_sequence_nonce("t", "s", 0)
    with pytest.raises(ValueError, match="token_hashes must be non-empty"):
        ring.preflight_validate_egress("t", "s", 1, 2, 3, 4, [])
    with pytest.raises(ValueError, match="NUL"):
        ring.derive_or_get("t\x00", "s")
    with pytest.raises(TypeError):
        ring.begin_egress_execution("t", "s", {b"not a reservation"})


# ---- the reference benchmark's key-ring assertions, on both implementations ------------

class _Native:
    """The product key ring behind the model's method names."""

    def __init__(self, KR):
        self.KR = KR
        self.r = KR.EphemeralSessionKeyRing(PEPPER)

    def derive_or_get(self, t, s):
        e, m, _, _ = self.r.derive_or_get(t, s)
        return bytes(e), bytes(m), self.r.session_generation(t, s)

    def next_sequence_nonce(self, t, s, count=1):
        return self.r.next_sequence_nonce(t, s, count)

    def preflight(self, t, s, model, layer, hg, base, ths):
        res, _, _ = self.r.preflight_validate_egress(t, s, model, layer, hg, base, ths)
        return res

    def begin_egress(self, t, s, res):
        return self.r.begin_egress_execution(t, s, res)

    def commit_egress(self, t, s, res):
        return self.r.commit_egress(t, s, res, res, res.last_sequence)

    def release(self, t, s, res):
        return self.r.release_egress_reservation(t, s, res)

    def begin_ingress(self, t, s):
        return self.r.begin_ingress(t, s)

    def verify_freshness(self, t, s, model, layer, hg, token, seq, min_seq=None, expected_seq=None,
                         expected_generation=None):
        return self.r.verify_and_update_freshness(t, s, model, layer, hg, token, seq, min_seq,
                                                  expected_seq, expected_generation)

    def verify_freshness_batch(self, t, s, records, min_seq=None, expected_generation=None):
        return self.r.verify_and_update_freshness_batch(t, s, records, min_seq, expected_generation)

    def finish_ingress(self, t, s, gen):
        return self.r.finish_ingress(t, s, gen)

    def shred_session(self, t, s):
        return self.r.crypto_shred_session(t, s)

    def shred_tenant(self, t):
        return self.r.crypto_shred_tenant(t)


@pytest.fixture(params=["native", "model"])
def ring(request, KR, M):
    if request.param == "native":
        return _Native(KR)
    return M.KeyRingModel(PEPPER)


def _kind(exc) -> str:
    return getattr(exc, "kind", type(exc).__name__)


def _expect(kind, fn, *a, match=None, **kw):
    try:
        fn(*a, **kw)
    except Exception as exc:  # noqa: BLE001
        assert _kind(exc) == kind, (kind, exc)
        if match is not None:
            assert str(exc) == match, str(exc)
        return exc
    raise AssertionError(f"expected {kind}")


def _encode(ring, t, s, seq, token, layer=14, hg=0, model=0xABCD):
    res = ring.preflight(t, s, model, layer, hg, seq, [token])
    try:
        ring.begin_egress(t, s, res)
        ring.commit_egress(t, s, res)
    finally:
        ring.release(t, s, res)


def test_nonce_reuse_and_stale_replay(ring):
    t, s, tok = "tenant-alpha-bank", "sess-peak-sec", 0x1234_5678_9ABC_DEF0
    _encode(ring, t, s, 10, tok)
    # same sequence nonce, layer and head group -> the same ChaCha20 nonce
    _expect("NonceReuseError", ring.preflight, t, s, 0xABCD, 14, 0, 10, [tok],
            match="NONCE_REUSE_DETECTED: Final 96-bit ChaCha20 nonce 0a00000000000000" "00000e00"
            f" already used under session {(t, s)}")
    # another layer gives another nonce
    _encode(ring, t, s, 10, tok, layer=15)
    # v2 of the slot, then v1 cannot be re-encoded or re-read
    _encode(ring, t, s, 11, tok)
    _expect("StalePageReplayError", ring.preflight, t, s, 0xABCD, 14, 0, 9, [tok],
            match="STALE_PAGE_REPLAY: Cannot encode cold page with stale sequence_nonce=9 < latest=11")
    gen, _, _ = ring.begin_ingress(t, s)
    ring.verify_freshness(t, s, 0xABCD, 14, 0, tok, 11, expected_generation=gen)  # legitimate re-read
    _expect("StalePageReplayError", ring.verify_freshness, t, s, 0xABCD, 14, 0, tok, 10,
            match="STALE_PAGE_REPLAY: Cold-page sequence_nonce=10 is older than latest slot version=11")
    _expect("StalePageReplayError", ring.verify_freshness, t, s, 0xABCD, 14, 0, tok, 12, None, 13,
            match="STALE_PAGE_REPLAY: Cold-page sequence_nonce=12 != expected_sequence_nonce=13")
    _expect("StalePageReplayError", ring.verify_freshness, t, s, 0xABCD, 14, 0, tok, 12, 20,
            match="STALE_PAGE_REPLAY: Cold-page sequence_nonce=12 < min_sequence_nonce=20")
    ring.finish_ingress(t, s, gen)


def test_failed_encode_keeps_nonce_burned(ring):
    t, s = "tenant-alpha-bank", "sess-code003"
    res = ring.preflight(t, s, 1, 14, 0, 25, [5])
    ring.release(t, s, res)  # the kernel step failed: no commit
    _expect("NonceReuseError", ring.preflight, t, s, 1, 14, 0, 25, [5])
    # the watermark did not move: an older sequence for the slot is still accepted
    _encode(ring, t, s, 24, 5)


def test_out_of_order_commit_keeps_watermark(ring):
    t, s = "tenant-alpha-bank", "sess-code003"
    low = ring.preflight(t, s, 1, 14, 0, 30, [77])
    high = ring.preflight(t, s, 1, 14, 0, 31, [77])
    ring.begin_egress(t, s, high)
    ring.commit_egress(t, s, high)
    ring.release(t, s, high)
    ring.begin_egress(t, s, low)
    ring.commit_egress(t, s, low)  # late commit of seq 30 does not roll back 31
    ring.release(t, s, low)
    _expect("StalePageReplayError", ring.verify_freshness, t, s, 1, 14, 0, 77, 30)
    ring.verify_freshness(t, s, 1, 14, 0, 77, 31)


def test_shred_revokes_in_flight_and_rederives(ring):
    t, s = "tenant-alpha-bank", "sess-001"
    e1, m1, g1 = ring.derive_or_get(t, s)
    assert g1 == 1
    res = ring.preflight(t, s, 1, 2, 3, 100, [1, 2, 3])
    gen, _, _ = ring.begin_ingress(t, s)
    assert ring.shred_session(t, s) is True
    assert ring.shred_session(t, s) is False
    _expect("SessionShreddedError", ring.begin_egress, t, s, res,
            match=f"Session ({t}, {s}) generation 1 was crypto-shredded before or during egress")
    _expect("SessionShreddedError", ring.commit_egress, t, s, res,
            match=f"Session ({t}, {s}) generation 1 was crypto-shredded before commit")
    ring.release(t, s, res)
    _expect("SessionShreddedError", ring.begin_ingress, t, s,
            match=f"Session ({t}, {s}) key is missing or crypto-shredded")
    _expect("SessionShreddedError", ring.finish_ingress, t, s, gen,
            match=f"Session ({t}, {s}) generation 1 was crypto-shredded during ingress")
    e2, m2, g2 = ring.derive_or_get(t, s)
    assert g2 == 2 and e2 != e1 and m2 != m1
    # an ingress begun under generation 1 cannot finish under generation 2
    _expect("SessionShreddedError", ring.verify_freshness, t, s, 1, 2, 3, 1, 100, None, None, gen,
            match=f"Session ({t}, {s}) generation 1 was crypto-shredded during ingress")
    # nonces and watermarks start afresh under the new key
    _encode(ring, t, s, 100, 1, layer=2, hg=3, model=1)


def test_shred_tenant(ring):
    for s in ("a", "b", "c"):
        ring.derive_or_get("tenant-x", s)
    ring.derive_or_get("tenant-y", "a")
    assert ring.shred_tenant("tenant-x") == 3
    assert ring.shred_tenant("tenant-x") == 0
    ring.begin_ingress("tenant-y", "a")


def test_sequence_allocation(ring):
    t, s = "t", "s"
    assert ring.next_sequence_nonce(t, s) == 1
    assert ring.next_sequence_nonce(t, s, 5) == 2
    assert ring.next_sequence_nonce(t, s) == 7
    res = ring.preflight(t, s, 1, 1, 1, 100, [1, 2, 3])
    ring.release(t, s, res)
    assert ring.next_sequence_nonce(t, s) == 103  # preflight raised the session maximum
    ring.verify_freshness(t, s, 9, 9, 9, 9, 500)
    assert ring.next_sequence_nonce(t, s) == 501


def test_batch_freshness_is_all_or_nothing(ring):
    t, s = "t", "s"
    ring.derive_or_get(t, s)
    ring.verify_freshness(t, s, 1, 0, 0, 2, 50)  # slot B at 50
    recs = [(1, 0, 0, 1, 40), (1, 0, 0, 1, 41), (1, 0, 0, 2, 49)]  # slot A twice, then a stale B
    _expect("StalePageReplayError", ring.verify_freshness_batch, t, s, recs,
            match="STALE_PAGE_REPLAY: Cold-page sequence_nonce=49 is older than latest slot version=50")
    ring.verify_freshness(t, s, 1, 0, 0, 1, 1)  # slot A did not move
    # within one batch a slot may not go backwards either
    _expect("StalePageReplayError", ring.verify_freshness_batch, t, s, [(1, 0, 0, 3, 9), (1, 0, 0, 3, 8)])
    _expect("StalePageReplayError", ring.verify_freshness_batch, t, s, [(1, 0, 0, 4, 9)], 10,
            match="STALE_PAGE_REPLAY: Cold-page sequence_nonce=9 < min_sequence_nonce=10")
    ring.verify_freshness_batch(t, s, recs[:2])
    _expect("StalePageReplayError", ring.verify_freshness, t, s, 1, 0, 0, 1, 40)


def test_header_tail_records(KR):
    """The codec hands the key ring header bytes 8..32 unparsed."""
    from vlx_tee_amd.spec import pack_header

    ring = KR.EphemeralSessionKeyRing(PEPPER)
    ring.derive_or_get("t", "s")
    hdrs = np.frombuffer(b"".join(pack_header(2, 1, 7, 0xDEADBEEF, 14, 3, (1 << 64) - 5, 1000 + i)
                                  for i in range(4)), dtype=np.uint8).reshape(4, 32)
    ring.verify_and_update_freshness_batch("t", "s", hdrs[:, 8:32])
    with pytest.raises(KR.StalePageReplayError, match="sequence_nonce=1002 is older than latest slot version=1003"):
        ring.verify_and_update_freshness("t", "s", 0xDEADBEEF, 14, 3, (1 << 64) - 5, 1002)


def test_concurrent_same_nonce_race(KR):
    """bench_cold_page_pipeline.py:486-528: of two racing encodes of one nonce
    exactly one succeeds."""
    ring = KR.EphemeralSessionKeyRing(PEPPER)
    for trial in range(20):
        barrier = threading.Barrier(2)
        out = []

        def work(tok):
            barrier.wait(timeout=10)
            try:
                res, _, _ = ring.preflight_validate_egress("t", "race", 1, 14, 0, 20 + 1000 * trial, [tok])
                ring.release_egress_reservation("t", "race", res)
                out.append("ok")
            except KR.NonceReuseError:
                out.append("reuse")

        th = [threading.Thread(target=work, args=(tok,)) for tok in (1, 2)]
        for x in th:
            x.start()
        for x in th:
            x.join()
        assert sorted(out) == ["ok", "reuse"]


def test_reservation_generation_and_release(KR):
    ring = KR.EphemeralSessionKeyRing(PEPPER)
    res, slots, last = ring.preflight_validate_egress("t", "s", 1, 1, 1, (1 << 64) - 2, [1, 2, 3])
    assert slots is res and res.generation == 1
    assert last == 0  # the sequence wraps mod 2**64 as the reference masks it
    ring.release_egress_reservation("t", "s", res)
    with pytest.raises(KR.SessionShreddedError, match="already released"):
        ring.commit_egress("t", "s", res, slots, last)
    ring.release_egress_reservation("t", "s", res)  # idempotent
    ring.close()
    with pytest.raises(KR.SessionShreddedError, match="closed"):
        ring.derive_or_get("t", "s")


# ---- seeded random operation sequence: native vs model ----------------------------------

def _run(impl, op, args):
    try:
        return ("ok", op(impl, *args))
    except Exception as exc:  # noqa: BLE001
        return (_kind(exc), str(exc))


def test_random_operations_match_model(KR, M):
    for seed in (1234, 99):
        random_operations(KR, M, seed)


def random_operations(KR, M, seed, steps=3000):
    rng = random.Random(seed)
    nat, mod = _Native(KR), M.KeyRingModel(PEPPER)
    tenants, sessions = ["ta", "tb"], ["s1", "s2"]
    held = []  # (native reservation, model reservation, tenant, session)
    gens = {}

    def pick():
        return rng.choice(tenants), rng.choice(sessions)

    for step in range(steps):
        r = rng.random()
        t, s = pick()
        if r < 0.12:
            a = (t, s)
            rn, rm = _run(nat, lambda i, *x: i.derive_or_get(*x)[2], a), _run(mod, lambda i, *x: i.derive_or_get(*x)[2], a)
        elif r < 0.18:
            a = (t, s, rng.randint(1, 5))
            rn, rm = _run(nat, lambda i, *x: i.next_sequence_nonce(*x), a), _run(mod, lambda i, *x: i.next_sequence_nonce(*x), a)
        elif r < 0.40:
            n = rng.randint(1, 4)
            a = (t, s, rng.randint(0, 1), rng.randint(0, 1), 0, rng.randint(0, 40),
                 [rng.randint(0, 3) for _ in range(n)])
            rn = _run(nat, lambda i, *x: i.preflight(*x), a)
            rm = _run(mod, lambda i, *x: i.preflight(*x), a)
            if rn[0] == "ok" and rm[0] == "ok":
                held.append((rn[1], rm[1], t, s))
                rn, rm = ("ok", None), ("ok", None)
        elif r < 0.58 and held:
            k = rng.randrange(len(held))
            hn, hm, ht, hs = held[k]
            what = rng.random()
            if what < 0.35:
                rn = _run(nat, lambda i: i.begin_egress(ht, hs, hn) and None, ())
                rm = _run(mod, lambda i: i.begin_egress(ht, hs, hm) and None, ())
            elif what < 0.75:
                rn = _run(nat, lambda i: i.commit_egress(ht, hs, hn), ())
                rm = _run(mod, lambda i: i.commit_egress(ht, hs, hm), ())
            else:
                nat.release(ht, hs, hn)
                mod.release(ht, hs, hm)
                held.pop(k)
                rn = rm = ("ok", None)
        elif r < 0.68:
            a = (t, s)
            rn = _run(nat, lambda i, *x: i.begin_ingress(*x)[0], a)
            rm = _run(mod, lambda i, *x: i.begin_ingress(*x)[0], a)
            if rn[0] == "ok":
                gens[(t, s)] = rn[1]
        elif r < 0.80:
            a = (t, s, rng.randint(0, 1), rng.randint(0, 1), 0, rng.randint(0, 3), rng.randint(0, 45),
                 rng.choice([None, rng.randint(0, 30)]), rng.choice([None, None, rng.randint(0, 45)]),
                 rng.choice([None, gens.get((t, s)), rng.randint(1, 3)]))
            rn = _run(nat, lambda i, *x: i.verify_freshness(*x), a)
            rm = _run(mod, lambda i, *x: i.verify_freshness(*x), a)
        elif r < 0.90:
            recs = [(rng.randint(0, 1), rng.randint(0, 1), 0, rng.randint(0, 3), rng.randint(0, 45))
                    for _ in range(rng.randint(0, 4))]
            a = (t, s, recs, rng.choice([None, rng.randint(0, 20)]),
                 rng.choice([None, gens.get((t, s))]))
            rn = _run(nat, lambda i, *x: i.verify_freshness_batch(*x), a)
            rm = _run(mod, lambda i, *x: i.verify_freshness_batch(*x), a)
        elif r < 0.94:
            a = (t, s, rng.choice([gens.get((t, s), 1), 1, 2]))
            rn = _run(nat, lambda i, *x: i.finish_ingress(*x), a)
            rm = _run(mod, lambda i, *x: i.finish_ingress(*x), a)
        elif r < 0.985:
            rn = _run(nat, lambda i: i.shred_session(t, s), ())
            rm = _run(mod, lambda i: i.shred_session(t, s), ())
        else:
            rn = _run(nat, lambda i: i.shred_tenant(t), ())
            rm = _run(mod, lambda i: i.shred_tenant(t), ())
        assert rn == rm, (step, r, rn, rm)
    for hn, hm, ht, hs in held:
        nat.release(ht, hs, hn)
