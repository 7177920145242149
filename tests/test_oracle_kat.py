"""Known answers pinning the oracle's ChaCha20 and SipHash-2-4-128.

RFC 8439 test vectors (sections 2.3.2, 2.4.2, A.1) are typed from the RFC;
SipHash-128 is pinned by the first Aumasson-Bernstein vector (key 00..0f,
empty message) and, for every other length, by the reference's own compiled
implementation (siphash24_128_cpu, cpp:2526-2538).
"""
import numpy as np
import pytest
import torch

KEY_0_31 = bytes(range(32))


def test_rfc8439_block_2_3_2(O):
    nonce = bytes.fromhex("000000090000004a00000000")
    ks = O.chacha20_xor(bytes(64), KEY_0_31, 1, nonce)
    assert ks.hex() == (
        "10f1e7e4d13b5915500fdd1fa32071c4c7d1f4c733c068030422aa9ac3d46c4e"
        "d2826446079faa0914c2d705d98b02a2b5129cd1de164eb9cbd083e8a2503c4e")


def test_rfc8439_encryption_2_4_2(O):
    nonce = bytes.fromhex("000000000000004a00000000")
    pt = (b"Ladies and Gentlemen of the class of '99: If I could offer you only one tip "
          b"for the future, sunscreen would be it.")
    ct = O.chacha20_xor(pt, KEY_0_31, 1, nonce)
    assert ct.hex() == (
        "6e2e359a2568f98041ba0728dd0d6981e97e7aec1d4360c20a27afccfd9fae0b"
        "f91b65c5524733ab8f593dabcd62b3571639d624e65152ab8f530c359f0861d8"
        "07ca0dbf500d6a6156a38e088a22b65e52bc514d16ccf806818ce91ab7793736"
        "5af90bbf74a35be6b40b8eedf2785e42874d")
    assert O.chacha20_xor(ct, KEY_0_31, 1, nonce) == pt


def test_rfc8439_a1_zero_key(O):
    ks = O.chacha20_xor(bytes(64), bytes(32), 0, bytes(12))
    assert ks.hex() == (
        "76b8e0ada0f13d90405d6ae55386bd28bdd219b8a08ded1aa836efcc8b770dc7"
        "da41597c5157488d7724e03fb8d84a376a43b8f41518a11cc387b669b2ee6586")


def test_chacha_counter_continuity(O):
    """Bytes of block c+1 of one call equal block 0 of a call at counter c+1."""
    nonce = bytes(range(12))
    a = O.chacha20_xor(bytes(200), KEY_0_31, 7, nonce)
    b = O.chacha20_xor(bytes(136), KEY_0_31, 8, nonce)
    assert a[64:] == b


def test_siphash128_first_vector(O):
    k = bytes(range(16))
    mk0, mk1 = int.from_bytes(k[:8], "little"), int.from_bytes(k[8:], "little")
    assert O.siphash128(b"", mk0, mk1).hex() == "a3817f04ba25a8e66df67214c7550293"


def test_siphash128_vectors_vs_reference(O, ref):
    k = bytes(range(16))
    mk0, mk1 = int.from_bytes(k[:8], "little"), int.from_bytes(k[8:], "little")
    for n in range(0, 130):
        msg = bytes(i & 0xFF for i in range(n))
        t_ref = bytes(ref.siphash24_128_cpu(torch.tensor(list(msg), dtype=torch.uint8), mk0, mk1).tolist())
        assert O.siphash128(msg, mk0, mk1) == t_ref, n


def test_siphash128_random_keys_vs_reference(O, ref):
    rng = np.random.default_rng(3)
    for _ in range(40):
        n = int(rng.integers(0, 300))
        msg = rng.integers(0, 256, size=n, dtype=np.uint8)
        mk0, mk1 = (int(x) for x in rng.integers(0, 2**63, size=2))
        t_ref = bytes(ref.siphash24_128_cpu(torch.from_numpy(msg.copy()), mk0, mk1).tolist())
        assert O.siphash128(msg.tobytes(), mk0, mk1) == t_ref


def test_chacha_vs_reference(O, ref):
    rng = np.random.default_rng(4)
    for _ in range(20):
        n = int(rng.integers(1, 700))
        data = rng.integers(0, 256, size=n, dtype=np.uint8)
        key = rng.integers(0, 256, size=32, dtype=np.uint8)
        nonce = rng.integers(0, 256, size=12, dtype=np.uint8)
        ctr = int(rng.integers(0, 2**32 - 20))
        out = ref.chacha20_rfc8439_xor_cpu(torch.from_numpy(data.copy()), torch.from_numpy(key.copy()),
                                           ctr, torch.from_numpy(nonce.copy())).numpy().tobytes()
        assert O.chacha20_xor(data.tobytes(), key.tobytes(), ctr, nonce.tobytes()) == out
