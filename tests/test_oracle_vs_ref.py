"""The oracle against the reference's own compiled codec (oracle/_ref).

Blobs must be byte-identical and decoded pages bit-identical for every preset
x RoPE mode, regular and odd geometries, padding, zero / tiny groups, and the
batch decoder's verdicts must agree for the reference's tamper cases
(bench_cold_page_pipeline.py:318-401)."""
import numpy as np
import pytest
import torch

KEYS = dict(k0=0x0123456789ABCDEF, k1=0xFEDCBA9876543210, mk0=0x1111222233334444,
            mk1=0x5555666677778888, k2=0xDEADBEEFCAFEF00D, k3=0x0BADC0DE12345678)
TEN, MOD, LAYER, HG, BASE = 0xAABBCCDD, 0x11223344, 7, 3, 1000

GEOMS = [(16, 4, 128, 64, False), (4, 2, 64, 16, False), (3, 1, 48, 32, True),
         (2, 2, 32, 0, False), (5, 3, 16, 16, False), (64, 1, 576, 64, True)]


def _pages(rng, B, T, H, D, R, mla, zero=False):
    k = (rng.standard_normal((B, T, H, D)) * 0.5).astype(np.float16)
    if R:
        k[..., :R] *= 8
    v = None if mla else (rng.standard_normal((B, T, H, D)) * 0.3).astype(np.float16)
    if zero:
        k[0, 0, 0, :16] = 0
        k[-1, 0, 0, -16:] = np.float16(1e-7)
        if v is not None:
            v[0, 0, 0, :] = 0
    return k, v


def _ref_encode(ref, k, v, th, preset, rm, R, exp):
    out = torch.empty((k.shape[0], 48 + exp), dtype=torch.uint8)
    ref.fused_encode_cold_pages_peak_into_cpu(
        torch.from_numpy(k), None if v is None else torch.from_numpy(v), torch.from_numpy(th), out,
        preset, rm, R, exp, TEN, MOD, LAYER, HG, BASE, KEYS["k0"], KEYS["k1"], KEYS["mk0"],
        KEYS["mk1"], KEYS["k2"], KEYS["k3"])
    return out.numpy()


def _ref_decode(ref, blobs, th, T, H, D, R, mla, tenant=TEN, model=MOD, layer=LAYER):
    B = blobs.shape[0]
    ko = torch.empty((B, T, H, D), dtype=torch.float16)
    vo = None if mla else torch.empty_like(ko)
    try:
        ref.fused_decode_cold_pages_peak_into_cpu(
            torch.from_numpy(blobs), torch.from_numpy(th), ko, vo, R, mla, tenant, model, layer,
            KEYS["k0"], KEYS["k1"], KEYS["mk0"], KEYS["mk1"], KEYS["k2"], KEYS["k3"])
        err = None
    except RuntimeError as e:
        err = str(e)
    return err, ko.numpy().view(np.uint16), None if vo is None else vo.numpy().view(np.uint16)


def _oracle_decode(O, blobs, th, T, H, D, R, mla, tenant=TEN, model=MOD, layer=LAYER):
    return O.ingress_batch(blobs, th, num_tokens=T, num_heads=H, head_dim=D, rope_dim=R,
                           is_mla_single_buffer=mla, dtype=O.FP16, expected_tenant_hash=tenant,
                           expected_model_hash=model, expected_layer_id=layer, **KEYS)


@pytest.mark.parametrize("geo", GEOMS)
def test_encode_decode_match_reference(O, ref, geo):
    T, H, D, R, mla = geo
    rng = np.random.default_rng(hash(geo) & 0xFFFF)
    for preset in (1, 2, 3):
        for rm in (0, 1, 2):
            for zero in (False, True):
                B = 3
                k, v = _pages(rng, B, T, H, D, R, mla, zero)
                th = rng.integers(-2**62, 2**62, B).astype(np.int64)
                exp = O.payload_bytes(preset, rm, T * H, D, R, not mla)
                for pad in (0, 68):
                    a = _ref_encode(ref, k, v, th, preset, rm, R, exp + pad)
                    b = O.egress_batch(k.view(np.uint16), None if mla else v.view(np.uint16), th,
                                       dtype=O.FP16, preset=preset, rope_mode=rm, rope_dim=R,
                                       expected_payload_bytes=exp + pad, tenant_id_hash=TEN,
                                       model_id_hash=MOD, layer_id=LAYER, head_group_id=HG,
                                       base_sequence_nonce=BASE, **KEYS)
                    assert np.array_equal(a, b), (preset, rm, zero, pad)
                    err, rk, rv = _ref_decode(ref, a, th, T, H, D, R, mla)
                    rc, st, ok, ov = _oracle_decode(O, b, th, T, H, D, R, mla)
                    assert err is None and rc == 0
                    assert np.array_equal(rk, ok)
                    if not mla:
                        assert np.array_equal(rv, ov)


def _verdict(err):
    if err is None:
        return 0
    if "CROSS_TENANT" in err:
        return 2
    return 3 if "MAC" in err else 1


def test_tamper_verdicts_match_reference(O, ref):
    """bench:318-401 tamper cases + header corruption, on a 4-page batch."""
    T, H, D, R, mla = 16, 4, 128, 64, False
    rng = np.random.default_rng(9)
    k, v = _pages(rng, 4, T, H, D, R, mla)
    th = np.arange(4, dtype=np.int64) + 77
    exp = O.payload_bytes(1, 1, T * H, D, R, True)
    blobs = _ref_encode(ref, k, v, th, 1, 1, R, exp)
    vecs = T * H
    s_rope = 32 + vecs * R
    q_nope = s_rope + vecs * (R // 16) * 2
    q_v = q_nope + vecs * ((D - R) // 2) + vecs * ((D - R) // 16) * 2

    def case(mut, **exp_kw):
        b = blobs.copy()
        mut(b)
        err, rk, rv = _ref_decode(ref, b, th, T, H, D, R, mla, **exp_kw)
        rc, st, ok, ov = _oracle_decode(O, b, th, T, H, D, R, mla, **exp_kw)
        assert rc == _verdict(err), (err, rc, st)
        assert np.array_equal(rk, ok) and np.array_equal(rv, ov)  # zeroed on failure
        return rc, st

    def flip(i, j):
        return lambda b: b.__setitem__((i, j), b[i, j] ^ 1)

    def swap16(b):
        x = b[1, q_nope:q_nope + 16].copy()
        b[1, q_nope:q_nope + 16] = b[1, q_nope + 16:q_nope + 32]
        b[1, q_nope + 16:q_nope + 32] = x

    def paired(b):
        b[2, q_v] ^= 1
        b[2, q_v + 16] ^= 1

    assert case(lambda b: None)[0] == 0
    assert case(flip(0, blobs.shape[1] // 2))[0] == 3      # 3.3 midpoint bit
    assert case(flip(1, s_rope))[0] == 3                  # 3.6 rope scale
    assert case(swap16)[0] == 3                           # 3.7 NoPE block swap
    assert case(paired)[0] == 3                           # 3.8 paired V flips
    assert case(flip(3, 0))[0] == 1                       # magic
    assert case(flip(3, 2))[0] == 1                       # version
    assert case(flip(2, 3))[0] == 3                       # flags (MAC'd)
    assert case(flip(1, 4))[0] == 2                       # tenant hash bit
    assert case(flip(1, 12))[0] == 2                      # layer bit
    assert case(flip(1, 16))[0] == 2                      # token hash bit
    assert case(flip(1, 24))[0] == 3                      # sequence nonce (MAC only)
    assert case(flip(0, blobs.shape[1] - 1))[0] == 3      # tag byte
    # 3.9 AAD mismatches on the expectation side
    assert case(lambda b: None, tenant=TEN ^ 1)[0] == 2
    assert case(lambda b: None, model=MOD ^ 1)[0] == 2
    assert case(lambda b: None, layer=LAYER + 1)[0] == 2
    # lowest failing page wins
    def two(b):
        b[3, 40] ^= 1
        b[1, 5] ^= 1
    rc, st = case(two)
    assert rc == 2 and list(st) == [0, 2, 0, 3]
