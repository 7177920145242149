"""Extension presets on the HIP path against the oracle, through the C ABI.

Presets 4 (int8 asymmetric per 64 / int4 per 32), 5 (e4m3 per 16), 6 (int4
per 32) and RoPE mode 3 (RoPE columns as e4m3) have no counterpart in the
reference; the oracle defines them (tests/test_oracle_ext.py pins it).  Blobs
must be byte-identical and decoded pages bit-identical to the oracle's, on the
fused kernels (aligned geometries) and the generic ones; without
ZTCP_EXT_LAYOUTS an extension header fails the flags check (status 1), as it
does in the reference.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

KEYS = dict(k0=0x0123456789ABCDEF, k1=0xFEDCBA9876543210, mk0=0x1111222233334444,
            mk1=0x5555666677778888, k2=0xDEADBEEFCAFEF00D, k3=0x0BADC0DE12345678)
TEN, MOD, LAYER, HG, BASE = 0xAABBCCDD, 0x11223344, 7, 3, 1000
DT = {"fp16": torch.float16, "bf16": torch.bfloat16}
EXT = [(p, r) for p in range(1, 7) for r in range(4) if p >= 4 or r == 3]


def _pages(seed, B, T, H, D, R, mla, dtype):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((B, T, H, D)).astype(np.float32) * 0.7
    if R:
        k[..., :R] *= 8
    k[0, 0, 0, :64] = 0                       # an all-zero group of every kind
    k[-1, 0, 0, :64] = np.abs(k[-1, 0, 0, :64])  # one-signed groups
    v = None if mla else (rng.standard_normal((B, T, H, D)) * 0.4).astype(np.float32)
    if v is not None:
        v[-1, -1, -1, :32] = -np.abs(v[-1, -1, -1, :32])
    return torch.from_numpy(k).to(dtype), (None if v is None else torch.from_numpy(v).to(dtype))


def _bits(t):
    return None if t is None else t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _odt(O, dtype):
    return O.BF16 if dtype == torch.bfloat16 else O.FP16


def _egress(H, O, k, v, th, preset, rm, R):
    dev = torch.device("cuda")
    B, T, Hh, D = k.shape
    exp = O.payload_bytes(preset, rm, T * Hh, D, R, v is not None)
    out = torch.full((B, 48 + exp), 0xA5, dtype=torch.uint8, device=dev)
    H.fused_encode_cold_pages_peak_into(k.to(dev), None if v is None else v.to(dev), torch.from_numpy(th),
                                        out, preset, rm, R, exp, TEN, MOD, LAYER, HG, BASE, KEYS["k0"],
                                        KEYS["k1"], KEYS["mk0"], KEYS["mk1"], KEYS["k2"], KEYS["k3"],
                                        ext_layouts=True)
    torch.cuda.synchronize()
    want = O.egress_batch(_bits(k), _bits(v), th, dtype=_odt(O, k.dtype), preset=preset, rope_mode=rm,
                          rope_dim=R, expected_payload_bytes=exp, tenant_id_hash=TEN, model_id_hash=MOD,
                          layer_id=LAYER, head_group_id=HG, base_sequence_nonce=BASE, **KEYS)
    return out.cpu().numpy(), want


def _ingress(H, O, blobs, th, shape, R, mla, dtype, *, ext=True, per_page=False):
    dev = torch.device("cuda")
    B = blobs.shape[0]
    ko = torch.full((B,) + shape, 7.0, dtype=dtype, device=dev)
    vo = None if mla else torch.full_like(ko, 7.0)
    st = torch.full((B,), -9, dtype=torch.int32, device=dev)
    err = None
    try:
        H.fused_decode_cold_pages_peak_into(torch.from_numpy(blobs).to(dev), torch.from_numpy(th), ko, vo, R,
                                            mla, TEN, MOD, LAYER, KEYS["k0"], KEYS["k1"], KEYS["mk0"],
                                            KEYS["mk1"], KEYS["k2"], KEYS["k3"], page_status=st,
                                            per_page=per_page, ext_layouts=ext)
    except RuntimeError as e:
        err = str(e)
    torch.cuda.synchronize()
    rc, ost, ok, ov = O.ingress_batch(blobs, th, num_tokens=shape[0], num_heads=shape[1], head_dim=shape[2],
                                      rope_dim=R, is_mla_single_buffer=mla, dtype=_odt(O, dtype),
                                      expected_tenant_hash=TEN, expected_model_hash=MOD,
                                      expected_layer_id=LAYER, all_or_nothing=not per_page, **KEYS)
    return err, st.cpu().numpy(), _bits(ko.cpu()), _bits(None if vo is None else vo.cpu()), rc, ost, ok, ov


GEOMS = [  # tokens, heads, head_dim, rope, mla, pages
    (16, 4, 128, 64, False, 64),     # c0 page shape (fused)
    (16, 8, 128, 64, False, 40),     # c2 page shape (fused)
    (64, 1, 576, 64, True, 6),       # c4 page shape (fused)
    (2, 16, 32, 16, False, 300),     # several pages per workgroup; wide groups do not fit
    (3, 1, 128, 64, True, 5),        # generic path (vecs % 16 != 0)
    (16, 2, 128, 0, False, 9),       # rope_dim 0
]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("geo", GEOMS, ids=lambda g: "x".join(map(str, g[:4])) + ("m" if g[4] else ""))
def test_ext_roundtrip_matches_oracle(hip, O, geo, dtype):
    T, Hh, D, R, mla, B = geo
    k, v = _pages(hash(geo) & 0xFFFF, B, T, Hh, D, R, mla, DT[dtype])
    th = (np.arange(B, dtype=np.int64) * 7919) ^ 0x5A5A
    ran = 0
    for preset, rm in EXT:
        if O.required_payload(preset, rm, T * Hh, D, R, not mla) < 0:
            continue  # a group wider than its section
        print(f"case T{T} H{Hh} D{D} R{R} mla={mla} B{B} {dtype} preset={preset} rope={rm}", flush=True)
        got, want = _egress(hip, O, k, v, th, preset, rm, R)
        assert np.array_equal(got, want), (preset, rm)
        err, st, gk, gv, rc, ost, ok, ov = _ingress(hip, O, got, th, (T, Hh, D), R, mla, DT[dtype])
        assert err is None and rc == 0 and (st == 0).all(), (preset, rm, err)
        assert np.array_equal(gk, ok), (preset, rm)
        if not mla:
            assert np.array_equal(gv, ov), (preset, rm)
        ran += 1
    assert ran > 0
    assert hip.device_diag() == 0


@pytest.mark.parametrize("preset,rm", [(4, 1), (5, 3), (6, 0), (2, 3)])
def test_ext_headers_rejected_without_opt_in(hip, O, preset, rm):
    """The reference's flags check rejects presets > 3 / RoPE mode 3 (status 1,
    KV_INTEGRITY_ERROR); so does ingress without ZTCP_EXT_LAYOUTS."""
    T, Hh, D, R, mla, B = 16, 4, 128, 64, False, 8
    k, v = _pages(5, B, T, Hh, D, R, mla, torch.bfloat16)
    th = np.arange(B, dtype=np.int64)
    got, want = _egress(hip, O, k, v, th, preset, rm, R)
    assert np.array_equal(got, want)
    err, st, gk, gv, *_ = _ingress(hip, O, got, th, (T, Hh, D), R, mla, torch.bfloat16, ext=False, per_page=True)
    assert err is not None and "KV_INTEGRITY_ERROR" in err
    assert (st == 1).all()
    assert not gk.any() and not gv.any()


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_ext_mixed_layouts_in_one_batch(hip, O, dtype):
    """Pages of reference and extension layouts in one workgroup: the first
    page's layout goes through the row pipeline, the others unit by unit."""
    T, Hh, D, R, mla = 16, 4, 128, 64, False
    k, v = _pages(9, 12, T, Hh, D, R, mla, DT[dtype])
    th = np.arange(12, dtype=np.int64) + 40
    flags = [(4, 3), (2, 1), (5, 0), (6, 1), (1, 3), (4, 1)]
    # every page at the largest blob size: a payload longer than its layout is
    # accepted, and the tag covers the zero padding
    width = max(O.payload_bytes(p_, r_, T * Hh, D, R, True) for p_, r_ in flags) + 48
    blobs = np.zeros((12, width), dtype=np.uint8)
    dev = torch.device("cuda")
    for i, (preset, rm) in enumerate(flags):
        sl = slice(2 * i, 2 * i + 2)
        out = torch.empty((2, width), dtype=torch.uint8, device=dev)
        hip.fused_encode_cold_pages_peak_into(k[sl].to(dev), v[sl].to(dev), torch.from_numpy(th[sl]), out,
                                              preset, rm, R, width - 48, TEN, MOD, LAYER, HG, BASE + 2 * i,
                                              KEYS["k0"], KEYS["k1"], KEYS["mk0"], KEYS["mk1"], KEYS["k2"],
                                              KEYS["k3"], ext_layouts=True)
        torch.cuda.synchronize()
        blobs[sl] = out.cpu().numpy()
        want = O.egress_batch(_bits(k[sl]), _bits(v[sl]), th[sl], dtype=_odt(O, k.dtype), preset=preset,
                              rope_mode=rm, rope_dim=R, expected_payload_bytes=width - 48, tenant_id_hash=TEN,
                              model_id_hash=MOD, layer_id=LAYER, head_group_id=HG,
                              base_sequence_nonce=BASE + 2 * i, **KEYS)
        assert np.array_equal(blobs[sl], want), (preset, rm)
    for first in (0, 5):  # the row pipeline on an extension layout, then on a reference one
        order = np.r_[2 * first:12, 0:2 * first]
        err, st, gk, gv, rc, ost, ok, ov = _ingress(hip, O, blobs[order], th[order], (T, Hh, D), R, mla,
                                                    DT[dtype])
        assert err is None and rc == 0 and (st == 0).all()
        assert np.array_equal(gk, ok) and np.array_equal(gv, ov)


def test_ext_tamper_matrix(hip, O):
    T, Hh, D, R, mla, B = 16, 8, 128, 64, False, 16
    k, v = _pages(11, B, T, Hh, D, R, mla, torch.bfloat16)
    th = np.arange(B, dtype=np.int64)
    for preset, rm in [(4, 3), (5, 1), (6, 3)]:
        got, _ = _egress(hip, O, k, v, th, preset, rm, R)
        bad = got.copy()
        L = bad.shape[1]
        bad[1, 0] ^= 1            # magic -> 1
        bad[3, 5] ^= 4            # tenant -> 2
        bad[5, 3] ^= 0x10         # flags (under the MAC) -> 3
        bad[7, 40] ^= 0x80        # payload -> 3
        bad[9, L - 20] ^= 1       # payload tail -> 3
        bad[11, L - 3] ^= 2       # tag -> 3
        err, st, gk, gv, rc, ost, ok, ov = _ingress(hip, O, bad, th, (T, Hh, D), R, mla, torch.bfloat16,
                                                    per_page=True)
        want = np.zeros(B, dtype=np.int32)
        want[[1, 3, 5, 7, 9, 11]] = [1, 2, 3, 3, 3, 3]
        assert np.array_equal(st, want) and np.array_equal(ost, want)
        assert np.array_equal(gk, ok) and np.array_equal(gv, ov)


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_ext_special_values(hip, O, dtype):
    """Non-finite, tiny and huge groups take the exact paths of the
    quantizers (zero / infinite scales, NaN codes -> 0) and the NaN outputs
    of infinite scales are written as c10 writes them: bytes == oracle."""
    T, Hh, D, R, mla, B = 16, 4, 128, 64, False, 4
    k, v = _pages(13, B, T, Hh, D, R, mla, DT[dtype])
    big = 60000.0 if dtype == "fp16" else 3.0e38
    k[1, 0, 0, 64:128] = float("nan")
    k[1, 0, 1, 70] = float("inf")
    k[1, 0, 2, 80] = -float("inf")
    k[1, 1, 0, 64:128] = 1e-7
    k[1, 1, 1, 64:128] = big
    k[1, 1, 2, 64:96] = -big
    k[2, 0, 0, :64] = float("nan")
    v[2, 0, 0, :32] = float("inf")
    v[2, 0, 1, 5] = float("nan")
    v[3, 0, 0, :] = 3e-8
    k[3, 2, 1, 64:128:3] = -0.0      # negative zeros: e4m3 code 0x80 decodes to -0
    v[3, 1, 1, ::5] = -0.0
    v[3, 1, 2, :16] = -1e-30         # products that round to -0 in e4m3
    th = np.arange(B, dtype=np.int64)
    # the reference's presets too: a scale that overflows fp16 decodes to NaN,
    # which must be written as the reference's conversions write it
    for preset, rm in [(4, 3), (5, 3), (6, 3), (4, 1), (1, 1), (2, 2), (3, 0)]:
        got, want = _egress(hip, O, k, v, th, preset, rm, R)
        assert np.array_equal(got, want), (preset, rm)
        err, st, gk, gv, rc, ost, ok, ov = _ingress(hip, O, got, th, (T, Hh, D), R, mla, DT[dtype])
        assert err is None and rc == 0
        assert np.array_equal(gk, ok) and np.array_equal(gv, ov), (preset, rm)


def _asym8_tie_groups(fp16: bool):
    """64-element groups whose codes (and, fp16 only, zero point) fall on
    exact ties: scale 1/16 (range 255/16), values (2k + 1) / 32."""
    k = np.arange(62)
    ties = (2 * k + 1) / 32.0
    groups = [np.concatenate([[0.0, 255 / 16], ties]), np.concatenate([[0.0, -255 / 16], -ties])]
    if fp16:
        groups.append(np.concatenate([[-253 / 32, 257 / 32], ties[:31], -ties[:31]]))
    return groups


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_ext_asym8_ties(hip, O, dtype):
    """asym8 groups on exact rounding ties (codes and zero points round to
    even in the oracle, tests/test_oracle_ext.py): the kernels' codes, blobs
    and decoded pages equal the oracle's."""
    T, Hh, D, R, mla, B = 16, 4, 128, 64, False, 8
    k, v = _pages(29, B, T, Hh, D, R, mla, DT[dtype])
    groups = _asym8_tie_groups(dtype == "fp16")
    kf = k.float()
    i = 0
    for b in range(B):
        for t in range(0, T, 3):
            for h in range(Hh):
                kf[b, t, h, R:] = torch.from_numpy(groups[i % len(groups)].astype(np.float32))
                i += 1
    k = kf.to(DT[dtype])
    assert torch.equal(k.float()[0, 0, 0, R:], torch.from_numpy(groups[0].astype(np.float32)))
    th = np.arange(B, dtype=np.int64) + 40
    for preset, rm in [(4, 3), (4, 1)]:
        got, want = _egress(hip, O, k, v, th, preset, rm, R)
        assert np.array_equal(got, want), (preset, rm)
        err, st, gk, gv, rc, ost, ok, ov = _ingress(hip, O, got, th, (T, Hh, D), R, mla, DT[dtype])
        assert err is None and rc == 0 and (st == 0).all()
        assert np.array_equal(gk, ok) and np.array_equal(gv, ov), (preset, rm)
