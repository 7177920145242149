"""HIP path against the oracle, through the C ABI (python mirror -> libztcp_hip.so).

Byte-exact blobs (header, codes, scales, ciphertext, tags) and bit-exact
decoded pages for FP16 (the reference's dtype) and BF16 (extension), every
preset x RoPE mode, fused and generic kernels, contiguous and descriptor
forms; the reference's tamper cases; per-page and all-or-nothing policies.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

KEYS = dict(k0=0x0123456789ABCDEF, k1=0xFEDCBA9876543210, mk0=0x1111222233334444,
            mk1=0x5555666677778888, k2=0xDEADBEEFCAFEF00D, k3=0x0BADC0DE12345678)
TEN, MOD, LAYER, HG, BASE = 0xAABBCCDD, 0x11223344, 7, 3, 1000
DT = {"fp16": torch.float16, "bf16": torch.bfloat16}


def _pages(seed, B, T, H, D, R, mla, dtype):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((B, T, H, D)).astype(np.float32) * 0.7
    if R:
        k[..., :R] *= 8
    k[0, 0, 0, :16] = 0
    v = None if mla else (rng.standard_normal((B, T, H, D)) * 0.4).astype(np.float32)
    kt = torch.from_numpy(k).to(dtype)
    vt = None if v is None else torch.from_numpy(v).to(dtype)
    return kt, vt


def _bits(t):
    return None if t is None else t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _odt(O, dtype):
    return O.BF16 if dtype == torch.bfloat16 else O.FP16


def _egress_both(H, O, k, v, th, preset, rm, R, exp):
    dev = torch.device("cuda")
    B = k.shape[0]
    out = torch.full((B, 48 + exp), 0xA5, dtype=torch.uint8, device=dev)
    H.fused_encode_cold_pages_peak_into(k.to(dev), None if v is None else v.to(dev),
                                        torch.from_numpy(th), out, preset, rm, R, exp, TEN, MOD,
                                        LAYER, HG, BASE, KEYS["k0"], KEYS["k1"], KEYS["mk0"],
                                        KEYS["mk1"], KEYS["k2"], KEYS["k3"])
    torch.cuda.synchronize()
    want = O.egress_batch(_bits(k), _bits(v), th, dtype=_odt(O, k.dtype), preset=preset,
                          rope_mode=rm, rope_dim=R, expected_payload_bytes=exp, tenant_id_hash=TEN,
                          model_id_hash=MOD, layer_id=LAYER, head_group_id=HG,
                          base_sequence_nonce=BASE, **KEYS)
    return out.cpu().numpy(), want


def _ingress_both(H, O, blobs, th, T, Hh, D, R, mla, dtype, per_page=False, **exp_kw):
    dev = torch.device("cuda")
    B = blobs.shape[0]
    ko = torch.full((B, T, Hh, D), 7.0, dtype=dtype, device=dev)
    vo = None if mla else torch.full_like(ko, 7.0)
    st = torch.full((B,), -9, dtype=torch.int32, device=dev)
    err = None
    try:
        H.fused_decode_cold_pages_peak_into(torch.from_numpy(blobs).to(dev), torch.from_numpy(th), ko,
                                            vo, R, mla, exp_kw.get("tenant", TEN),
                                            exp_kw.get("model", MOD), exp_kw.get("layer", LAYER),
                                            KEYS["k0"], KEYS["k1"], KEYS["mk0"], KEYS["mk1"],
                                            KEYS["k2"], KEYS["k3"], page_status=st, per_page=per_page)
    except RuntimeError as e:
        err = str(e)
    torch.cuda.synchronize()
    rc, ost, ok, ov = O.ingress_batch(blobs, th, num_tokens=T, num_heads=Hh, head_dim=D, rope_dim=R,
                                      is_mla_single_buffer=mla, dtype=_odt(O, dtype),
                                      expected_tenant_hash=exp_kw.get("tenant", TEN),
                                      expected_model_hash=exp_kw.get("model", MOD),
                                      expected_layer_id=exp_kw.get("layer", LAYER),
                                      all_or_nothing=not per_page, **KEYS)
    return err, st.cpu().numpy(), _bits(ko.cpu()), _bits(None if vo is None else vo.cpu()), rc, ost, ok, ov


def _verdict(err):
    if err is None:
        return 0
    if "CROSS_TENANT" in err:
        return 2
    return 3 if "MAC" in err else 1


GEOMS = [  # tokens, heads, head_dim, rope, mla, pages   (fast path unless noted)
    # egress: up to 4 pages per workgroup (<= 1024 pages) run the small-batch
    # kernel for the reference's presets, larger batches the row-pipeline one
    (16, 4, 128, 64, False, 64),     # c0 page shape
    (16, 8, 128, 64, False, 40),     # c2 page shape
    (64, 1, 576, 64, True, 6),       # c4 page shape
    (2, 16, 32, 16, False, 700),     # several pages per workgroup (small-batch kernel)
    (16, 4, 128, 64, False, 1333),   # row pipeline, 6 pages per workgroup, the last one partial
    (3, 1, 48, 32, True, 5),         # generic path (vecs % 32 != 0)
    (5, 3, 16, 16, False, 4),        # generic path
    (16, 2, 64, 0, False, 9),        # rope_dim 0
]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("geo", GEOMS, ids=lambda g: "x".join(map(str, g[:4])) + ("m" if g[4] else ""))
def test_roundtrip_matches_oracle(hip, O, geo, dtype):
    T, Hh, D, R, mla, B = geo
    k, v = _pages(hash(geo) & 0xFFFF, B, T, Hh, D, R, mla, DT[dtype])
    th = (np.arange(B, dtype=np.int64) * 7919) ^ 0x5A5A
    for preset in (1, 2, 3):
        for rm in (0, 1, 2):
            print(f"case T{T} H{Hh} D{D} R{R} mla={mla} B{B} {dtype} preset={preset} rope={rm}", flush=True)
            exp = O.payload_bytes(preset, rm, T * Hh, D, R, not mla)
            got, want = _egress_both(hip, O, k, v, th, preset, rm, R, exp)
            assert np.array_equal(got, want), (preset, rm)
            err, st, gk, gv, rc, ost, ok, ov = _ingress_both(hip, O, got, th, T, Hh, D, R, mla, DT[dtype])
            assert err is None and rc == 0 and (st == 0).all()
            assert np.array_equal(gk, ok)
            if not mla:
                assert np.array_equal(gv, ov)
    assert hip.device_diag() == 0


@pytest.mark.parametrize("pad", [4, 16, 48, 68, 80, 128, 132])
def test_padded_payload(hip, O, pad):
    """Payload longer than the layout: egress always takes the generic
    kernels; ingress takes the fused kernel when the blob size is a multiple
    of 16 (padding rows and a 16/32/48-byte tail on the verify path) and the
    generic kernels otherwise."""
    T, Hh, D, R, mla, B = 16, 4, 128, 64, False, 5
    k, v = _pages(3, B, T, Hh, D, R, mla, torch.bfloat16)
    th = np.arange(B, dtype=np.int64)
    exp = O.payload_bytes(2, 1, T * Hh, D, R, True) + pad
    got, want = _egress_both(hip, O, k, v, th, 2, 1, R, exp)
    assert np.array_equal(got, want)
    err, st, gk, gv, rc, ost, ok, ov = _ingress_both(hip, O, got, th, T, Hh, D, R, mla, torch.bfloat16)
    assert err is None and rc == 0
    assert np.array_equal(gk, ok) and np.array_equal(gv, ov)


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("first_bad", [False, True])
def test_mixed_layouts_in_one_batch(hip, O, dtype, first_bad):
    """One ingress batch whose pages carry different header flags (each page
    decodes under its own preset / rope mode, cpp:2340-2341), padded to one
    blob size; optionally the first page's flags are invalid, so another page
    sets the workgroup's layout."""
    T, Hh, D, R, mla, B = 16, 4, 128, 64, False, 520  # > 256 pages: several pages per workgroup
    k, v = _pages(29, B, T, Hh, D, R, mla, DT[dtype])
    th = np.arange(B, dtype=np.int64) * 31 + 5
    combos = [(3, 0), (1, 1), (2, 2), (1, 0), (2, 1), (3, 1)]
    exp = max(O.payload_bytes(p, rm, T * Hh, D, R, True) for p, rm in combos)
    blobs = np.zeros((B, 48 + exp), dtype=np.uint8)
    kb, vb = _bits(k), _bits(v)
    for i in range(B):
        p, rm = combos[(i * 5) % len(combos)]
        blobs[i] = O.egress_batch(kb[i:i + 1], vb[i:i + 1], th[i:i + 1], dtype=_odt(O, DT[dtype]), preset=p,
                                  rope_mode=rm, rope_dim=R, expected_payload_bytes=exp, tenant_id_hash=TEN,
                                  model_id_hash=MOD, layer_id=LAYER, head_group_id=HG,
                                  base_sequence_nonce=BASE + i, **KEYS)[0]
    if first_bad:
        blobs[0, 3] = 0x07  # flags byte: preset 7 (invalid); fails the MAC first
    print(f"case mixed layouts {dtype} first_bad={first_bad}", flush=True)
    err, st, gk, gv, rc, ost, ok, ov = _ingress_both(hip, O, blobs, th, T, Hh, D, R, mla, DT[dtype],
                                                      per_page=True)
    assert np.array_equal(st, ost)
    assert (st[1:] == 0).all() and st[0] == (3 if first_bad else 0)
    assert np.array_equal(gk, ok) and np.array_equal(gv, ov)
    assert hip.device_diag() == 0


@pytest.mark.parametrize("per_page", [False, True])
def test_tamper_matrix(hip, O, per_page):
    """bench_cold_page_pipeline.py:318-401 on the GPU path, plus header cases."""
    T, Hh, D, R, mla, B = 16, 4, 128, 64, False, 4
    k, v = _pages(5, B, T, Hh, D, R, mla, torch.float16)
    th = np.arange(B, dtype=np.int64) + 77
    exp = O.payload_bytes(1, 1, T * Hh, D, R, True)
    blobs, want = _egress_both(hip, O, k, v, th, 1, 1, R, exp)
    assert np.array_equal(blobs, want)
    vecs = T * Hh
    s_rope = 32 + vecs * R
    q_nope = s_rope + vecs * (R // 16) * 2
    q_v = q_nope + vecs * ((D - R) // 2) + vecs * ((D - R) // 16) * 2
    L = blobs.shape[1]

    def flip(*ij):
        def f(b):
            for i, j in ij:
                b[i, j] ^= 1
        return f

    def swap16(b):
        x = b[1, q_nope:q_nope + 16].copy()
        b[1, q_nope:q_nope + 16] = b[1, q_nope + 16:q_nope + 32]
        b[1, q_nope + 16:q_nope + 32] = x

    cases = [
        (lambda b: None, {}, [0, 0, 0, 0]),
        (flip((0, L // 2)), {}, [3, 0, 0, 0]),
        (flip((1, s_rope)), {}, [0, 3, 0, 0]),
        (swap16, {}, [0, 3, 0, 0]),
        (flip((2, q_v), (2, q_v + 16)), {}, [0, 0, 3, 0]),
        (flip((3, 0)), {}, [0, 0, 0, 1]),
        (flip((3, 2)), {}, [0, 0, 0, 1]),
        (flip((2, 3)), {}, [0, 0, 3, 0]),
        (flip((1, 4)), {}, [0, 2, 0, 0]),
        (flip((1, 12)), {}, [0, 2, 0, 0]),
        (flip((1, 16)), {}, [0, 2, 0, 0]),
        (flip((1, 24)), {}, [0, 3, 0, 0]),
        (flip((0, L - 1)), {}, [3, 0, 0, 0]),
        (lambda b: None, {"tenant": TEN ^ 1}, [2, 2, 2, 2]),
        (lambda b: None, {"model": MOD ^ 1}, [2, 2, 2, 2]),
        (lambda b: None, {"layer": LAYER + 1}, [2, 2, 2, 2]),
        (flip((3, 40), (1, 5)), {}, [0, 2, 0, 3]),
    ]
    for mut, kw, expect in cases:
        b = blobs.copy()
        mut(b)
        err, st, gk, gv, rc, ost, ok, ov = _ingress_both(hip, O, b, th, T, Hh, D, R, mla,
                                                         torch.float16, per_page=per_page, **kw)
        assert list(st) == expect and list(ost) == expect
        assert _verdict(err) == rc == next((s for s in expect if s), 0)
        assert np.array_equal(gk, ok) and np.array_equal(gv, ov)
        if not per_page and rc:
            assert not gk.any() and not gv.any()  # all-or-nothing zeroing (cpp:2483-2486)
    assert hip.device_diag() == 0


def test_descriptor_multilayer_matches_per_layer_oracle(hip, O, pkg):
    import vlx_tee_amd.pages as P

    T, Hh, D, R, B, per_layer = 16, 8, 128, 64, 96, 32
    dev = torch.device("cuda")
    k, v = _pages(17, B, T, Hh, D, R, False, torch.bfloat16)
    kd, vd = k.to(dev), v.to(dev)
    th = np.arange(B, dtype=np.int64) * 3 + 1
    seq = np.arange(B, dtype=np.uint64) + 500
    layers = (np.arange(B) // per_layer).astype(np.uint16)
    for preset, rm in [(2, 1), (1, 1), (3, 0)]:
        exp = O.payload_bytes(preset, rm, T * Hh, D, R, True)
        blobs = torch.zeros((B, 48 + exp), dtype=torch.uint8, device=dev)
        descs = P.build_descriptors(kd, vd, blobs, th, seq, layers, np.full(B, HG))
        P.egress(descs, B, num_tokens=T, num_heads=Hh, head_dim=D, rope_dim=R, dtype=torch.bfloat16,
                 is_mla_single_buffer=False, preset=preset, rope_mode=rm, expected_payload_bytes=exp,
                 tenant_id_hash=TEN, model_id_hash=MOD, **KEYS)
        torch.cuda.synchronize()
        got = blobs.cpu().numpy()
        for l0 in range(0, B, per_layer):
            sl = slice(l0, l0 + per_layer)
            want = O.egress_batch(_bits(k[sl]), _bits(v[sl]), th[sl], dtype=O.BF16, preset=preset,
                                  rope_mode=rm, rope_dim=R, expected_payload_bytes=exp,
                                  tenant_id_hash=TEN, model_id_hash=MOD, layer_id=int(layers[l0]),
                                  head_group_id=HG, base_sequence_nonce=int(seq[l0]), **KEYS)
            assert np.array_equal(got[sl], want), (preset, rm, l0)
        ko = torch.zeros_like(kd)
        vo = torch.zeros_like(vd)
        descs_in = P.build_descriptors(ko, vo, blobs, th, seq, layers)
        rc = P.ingress(descs_in, B, 48 + exp, num_tokens=T, num_heads=Hh, head_dim=D, rope_dim=R,
                       dtype=torch.bfloat16, is_mla_single_buffer=False, expected_tenant_hash=TEN,
                       expected_model_hash=MOD, **KEYS)
        assert rc == 0
        rc2, st2, ok, ov = O.ingress_batch(got[:per_layer], th[:per_layer], num_tokens=T,
                                           num_heads=Hh, head_dim=D, rope_dim=R,
                                           is_mla_single_buffer=False, dtype=O.BF16,
                                           expected_tenant_hash=TEN, expected_model_hash=MOD,
                                           expected_layer_id=0, **KEYS)
        assert rc2 == 0
        assert np.array_equal(_bits(ko[:per_layer].cpu()), ok)
        assert np.array_equal(_bits(vo[:per_layer].cpu()), ov)
        # a wrong expected layer for one page is an AAD failure for that page only
        layers_bad = layers.copy()
        layers_bad[B - 1] ^= 1
        st = torch.zeros(B, dtype=torch.int32, device=dev)
        descs_bad = P.build_descriptors(ko, vo, blobs, th, seq, layers_bad)
        rc = P.ingress(descs_bad, B, 48 + exp, num_tokens=T, num_heads=Hh, head_dim=D, rope_dim=R,
                       dtype=torch.bfloat16, is_mla_single_buffer=False, expected_tenant_hash=TEN,
                       expected_model_hash=MOD, page_status=st, per_page=True, **KEYS)
        s = st.cpu().numpy()
        assert rc == 2 and s[B - 1] == 2 and (s[:B - 1] == 0).all()
        assert not ko[B - 1].any() and ko[0].any()


def test_overlap_and_argument_errors(hip):
    dev = torch.device("cuda")
    buf = torch.zeros(16384 + 12336, dtype=torch.uint8, device=dev)
    k = buf[:16384].view(torch.float16).view(1, 16, 4, 128)
    v = torch.zeros_like(k)
    th = torch.zeros(1, dtype=torch.int64)
    with pytest.raises(RuntimeError, match="overlap"):  # cpp:1949-1951
        hip.fused_encode_cold_pages_peak_into(k, v, th, buf[4096:4096 + 12336].view(1, 12336), 1, 1,
                                              64, 12288, 0, 0, 0, 0, 0, 1, 2, 3, 4)
    out = torch.zeros((1, 12336), dtype=torch.uint8, device=dev)
    with pytest.raises(RuntimeError, match="preset"):
        hip.fused_encode_cold_pages_peak_into(k, v, th, out, 7, 1, 64, 12288, 0, 0, 0, 0, 0, 1, 2, 3, 4)
    with pytest.raises(RuntimeError, match="rope_mode"):
        hip.fused_encode_cold_pages_peak_into(k, v, th, out, 1, 4, 64, 12288, 0, 0, 0, 0, 0, 1, 2, 3, 4)
    with pytest.raises(RuntimeError, match="smaller than required"):
        hip.fused_encode_cold_pages_peak_into(k, v, th, torch.zeros((1, 12332), dtype=torch.uint8,
                                                                    device=dev),
                                              1, 1, 64, 12284, 0, 0, 0, 0, 0, 1, 2, 3, 4)


def test_kat_hooks_on_gpu(hip, O):
    dev = torch.device("cuda")
    key = torch.arange(32, dtype=torch.uint8)
    nonce = torch.tensor([0, 0, 0, 9, 0, 0, 0, 0x4A, 0, 0, 0, 0], dtype=torch.uint8)
    ks = hip.chacha20_rfc8439_xor(torch.zeros(64, dtype=torch.uint8, device=dev), key, 1, nonce)
    assert bytes(ks.cpu().tolist()).hex().startswith("10f1e7e4d13b5915500fdd1fa32071c4")
    rng = np.random.default_rng(1)
    for n in (0, 1, 7, 8, 9, 63, 64, 65, 1000, 4096 + 5):
        data = rng.integers(0, 256, size=n, dtype=np.uint8)
        mk0, mk1 = 0x0706050403020100, 0x0F0E0D0C0B0A0908
        tag = hip.siphash24_128(torch.from_numpy(data).to(dev), mk0, mk1)
        assert bytes(tag.cpu().tolist()) == O.siphash128(data.tobytes(), mk0, mk1)
        if n:
            kb = rng.integers(0, 256, size=32, dtype=np.uint8)
            nb = rng.integers(0, 256, size=12, dtype=np.uint8)
            ct = hip.chacha20_rfc8439_xor(torch.from_numpy(data).to(dev), torch.from_numpy(kb), 3,
                                          torch.from_numpy(nb))
            assert ct.cpu().numpy().tobytes() == O.chacha20_xor(data.tobytes(), kb.tobytes(), 3,
                                                                nb.tobytes())


def test_fast_quantizer_arithmetic_selftest(hip):
    """Exhaustive device check of the fast scale / reciprocal (ztcp_selftest)."""
    assert hip.N.lib().ztcp_selftest() == 0


# Payloads of 21, 10 and 31 rows (4k + 1, 4k + 2, 4k + 3) whose sections
# hold whole 32-group units, so the fused kernels take them: the MAC / verify
# wave takes rows four at a time and the last total % 4 rows one at a time;
# 64 pages run the small-batch kernels, 1,100 the row pipelines (5 pages per
# workgroup, the last one partial).
PARTIAL_GROUPS = [(1, 8, 64, 64, 1, 2), (1, 2, 256, 0, 1, 0), (1, 8, 128, 64, 1, 2)]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("B", [64, 1100])
@pytest.mark.parametrize("geo", PARTIAL_GROUPS, ids=lambda g: f"T{g[0]}H{g[1]}D{g[2]}R{g[3]}p{g[4]}r{g[5]}")
def test_partial_last_mac_group(hip, O, geo, B, dtype):
    T, Hh, D, R, preset, rm = geo
    k, v = _pages(61 + B, B, T, Hh, D, R, False, DT[dtype])
    th = np.arange(B, dtype=np.int64) * 3 + 1
    exp = O.payload_bytes(preset, rm, T * Hh, D, R, True)
    assert exp % 64 == 0 and (exp // 64) % 4 != 0
    got, want = _egress_both(hip, O, k, v, th, preset, rm, R, exp)
    assert np.array_equal(got, want)
    err, st, gk, gv, rc, ost, ok, ov = _ingress_both(hip, O, want, th, T, Hh, D, R, False, DT[dtype])
    assert err is None and rc == 0 and (st == 0).all()
    assert np.array_equal(gk, ok) and np.array_equal(gv, ov)
