"""The session-bound codec class on the GPU (drop-in for NativeCppFusedColdPageCodec).

Follows the reference benchmark's security suite on its native codec
(research/benchmarks/bench_cold_page_pipeline.py:172-610, tests 3.1-3.12) on
the reference's GQA geometry (64 tokens, 8 KV heads, head_dim 128, RoPE 64),
with pages and blobs resident on the GPU.  Blobs are compared byte for byte
with the oracle's encoder under the session's derived keys, decoded pages with
the oracle's decoder.
"""
from __future__ import annotations

import dataclasses
import struct
import threading
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from fidelity import BAR, attention_fidelity, reference_pages

pytestmark = pytest.mark.gpu

TENANT, MODEL, LAYER = "tenant-alpha-bank", "Qwen/Qwen3.6-35B-A3B", 14
TOKENS = list(range(1000, 1064))


@pytest.fixture(scope="module")
def C(pkg):
    import vlx_tee_amd.codec as C

    return C


@pytest.fixture(scope="module")
def S(pkg):
    import vlx_tee_amd.spec as S

    return S


def _geom(S, mla=False):
    if mla:
        return S.ColdPageGeometry(num_tokens=64, num_kv_heads=1, head_dim=576, rope_dim=64,
                                  is_mla_single_buffer=True)
    return S.ColdPageGeometry(num_tokens=64, num_kv_heads=8, head_dim=128, rope_dim=64)


def _pages(geo, n=None, seed=0, dtype=torch.float16):
    g = torch.Generator(device="cpu").manual_seed(seed)
    shape = (geo.num_tokens, geo.num_kv_heads, geo.head_dim)
    if n is not None:
        shape = (n,) + shape
    k = (torch.randn(shape, generator=g) * 2).to(dtype).cuda()
    v = None if geo.is_mla_single_buffer else (torch.randn(shape, generator=g)).to(dtype).cuda()
    return k, v


def _i64(h: int) -> int:
    return struct.unpack("<q", struct.pack("<Q", h & ((1 << 64) - 1)))[0]


def _session_keys(ring, tenant, session):
    enc, mac, _, _ = ring.derive_or_get(tenant, session)
    k0, k1, k2, k3 = struct.unpack("<4Q", bytes(enc))
    mk0, mk1 = struct.unpack("<2Q", bytes(mac)[:16])
    return dict(k0=k0, k1=k1, k2=k2, k3=k3, mk0=mk0, mk1=mk1)


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _oracle_blobs(O, geo, k, v, ths, aad, keys):
    dt = O.BF16 if k.dtype == torch.bfloat16 else O.FP16
    kb = _bits(k if k.dim() == 4 else k.unsqueeze(0))
    vb = None if v is None else _bits(v if v.dim() == 4 else v.unsqueeze(0))
    return O.egress_batch(kb, vb, np.array(ths, dtype=np.int64), dtype=dt, preset=int(aad.preset),
                          rope_mode=int(aad.rope_mode), rope_dim=geo.rope_dim,
                          expected_payload_bytes=geo.payload_bytes(aad.preset, aad.rope_mode),
                          tenant_id_hash=aad.tenant_id_hash, model_id_hash=aad.model_id_hash,
                          layer_id=aad.layer_id, head_group_id=aad.head_group_id,
                          base_sequence_nonce=aad.sequence_nonce, **keys)


def _oracle_decode(O, geo, blobs, ths, tenant, model, layer, keys, dtype=torch.float16):
    return O.ingress_batch(blobs, np.array(ths, dtype=np.int64), num_tokens=geo.num_tokens,
                           num_heads=geo.num_kv_heads, head_dim=geo.head_dim, rope_dim=geo.rope_dim,
                           is_mla_single_buffer=geo.is_mla_single_buffer,
                           dtype=O.BF16 if dtype == torch.bfloat16 else O.FP16,
                           expected_tenant_hash=tenant, expected_model_hash=model,
                           expected_layer_id=layer, **keys)


def test_single_page_security_suite(pkg, O, C, S):
    """bench_cold_page_pipeline.py:172-258 (tests 3.1-3.4) on the HIP codec."""
    geo = _geom(S)
    ring = C.EphemeralSessionKeyRing(bytes(range(40)))
    codec = C.NativeCppFusedColdPageCodec(geo, ring)
    k, v = _pages(geo)
    aad = S.ColdPageAAD.from_context(TENANT, MODEL, LAYER, TOKENS, sequence_nonce=1)
    th = aad.page_token_hash
    blob = codec.encode_cold_page_tensor(k, v, TENANT, "sess-001", aad)
    keys = _session_keys(ring, TENANT, "sess-001")
    want = _oracle_blobs(O, geo, k, v, [_i64(th)], aad, keys)
    assert np.array_equal(blob.cpu().numpy(), want[0])
    # 3.1 round trip
    kd, vd = codec.decode_cold_page_tensor(blob, TENANT, "sess-001", MODEL, LAYER, th)
    rc, _, ok, ov = _oracle_decode(O, geo, want, [_i64(th)], aad.tenant_id_hash, aad.model_id_hash, LAYER, keys)
    assert rc == 0 and np.array_equal(_bits(kd), ok[0]) and np.array_equal(_bits(vd), ov[0])
    # 3.2 another tenant's session asks for this blob
    ring.derive_or_get("tenant-beta-defense", "sess-beta-009")
    with pytest.raises(C.CrossTenantContaminationError, match="CROSS_TENANT_CONTAMINATION"):
        codec.decode_cold_page_tensor(blob, "tenant-beta-defense", "sess-beta-009", MODEL, LAYER, th)
    # 3.3 one flipped ciphertext bit
    bad = blob.clone()
    bad[bad.numel() // 2] ^= 1
    with pytest.raises(C.KVIntegrityError) as ei:
        codec.decode_cold_page_tensor(bad, TENANT, "sess-001", MODEL, LAYER, th)
    assert not isinstance(ei.value, C.CrossTenantContaminationError)
    # 3.4 crypto-shred, then re-derivation cannot open the archived blob
    assert ring.crypto_shred_session(TENANT, "sess-001") is True
    with pytest.raises(C.SessionShreddedError):
        codec.decode_cold_page_tensor(blob, TENANT, "sess-001", MODEL, LAYER, th)
    new_keys = _session_keys(ring, TENANT, "sess-001")
    assert new_keys != keys
    with pytest.raises(C.KVIntegrityError):
        codec.decode_cold_page_tensor(blob, TENANT, "sess-001", MODEL, LAYER, th)


def test_peak_path_security_suite(pkg, O, C, S):
    """bench_cold_page_pipeline.py:260-482 (tests 3.5-3.11) on the HIP codec."""
    geo = _geom(S)
    ring = C.EphemeralSessionKeyRing(bytes(range(1, 41)))
    codec = C.NativeCppFusedColdPageCodec(geo, ring)
    k_ref, v_ref = reference_pages(geo.num_tokens, geo.num_kv_heads, geo.head_dim, geo.rope_dim, False, 1,
                                   torch.float16)
    k_ref, v_ref = k_ref[0], v_ref[0]
    k, v = k_ref.cuda(), v_ref.cuda()
    sess = "sess-peak-sec"
    aad1 = S.ColdPageAAD.from_context(TENANT, MODEL, LAYER, TOKENS, sequence_nonce=10,
                                      preset=S.QuantPreset.INT4_SYM, rope_mode=S.RoPEMode.PRESERVE_FP8)
    th = aad1.page_token_hash
    th_t = torch.tensor([_i64(th)], dtype=torch.int64)
    nbytes = geo.cold_blob_bytes(aad1.preset, aad1.rope_mode)
    out1 = torch.empty((1, nbytes), dtype=torch.uint8, device="cuda")
    codec.encode_cold_pages_peak_into(k.unsqueeze(0), v.unsqueeze(0), th_t, out1, TENANT, sess, aad1)
    keys = _session_keys(ring, TENANT, sess)
    assert np.array_equal(out1.cpu().numpy(), _oracle_blobs(O, geo, k, v, [_i64(th)], aad1, keys))
    # 3.5 round trip and a legitimate re-read of the same version
    k1, v1 = codec.decode_cold_page_tensor(out1[0], TENANT, sess, MODEL, LAYER, th)
    k2, _ = codec.decode_cold_page_tensor(out1[0], TENANT, sess, MODEL, LAYER, th)
    assert torch.equal(k1, k2)
    # the reference's acceptance bar on its own page distribution (tests/fidelity.py)
    assert attention_fidelity(k_ref, v_ref, k1, v1) > BAR
    # 3.6-3.8 scale tamper, swapped 16-byte NoPE blocks, paired V-block flips
    vecs, gs, r = geo.vectors_per_buffer, geo.group_size, geo.rope_dim
    s_rope = 32 + vecs * r
    q_nope = s_rope + vecs * (r // gs) * 2
    q_v = q_nope + vecs * (geo.nope_dim // 2) + vecs * (geo.nope_dim // gs) * 2
    t1 = out1[0].clone()
    t1[s_rope] ^= 1
    t2 = out1[0].clone()
    t2[q_nope:q_nope + 16], t2[q_nope + 16:q_nope + 32] = out1[0, q_nope + 16:q_nope + 32].clone(), \
        out1[0, q_nope:q_nope + 16].clone()
    t3 = out1[0].clone()
    t3[q_v] ^= 1
    t3[q_v + 16] ^= 1
    for bad in (t1, t2, t3):
        with pytest.raises(C.KVIntegrityError, match="MAC verification failed"):
            codec.decode_cold_page_tensor(bad, TENANT, sess, MODEL, LAYER, th)
    # 3.9 AAD mismatch on tenant, model, layer, token hash
    for bt, bm, bl, btok in (("tenant-beta-defense", MODEL, LAYER, th), (TENANT, "Qwen/Other-Model", LAYER, th),
                             (TENANT, MODEL, LAYER + 1, th), (TENANT, MODEL, LAYER, th ^ 1)):
        ring.derive_or_get(bt, sess)
        with pytest.raises(C.CrossTenantContaminationError):
            codec.decode_cold_page_tensor(out1[0], bt, sess, bm, bl, btok)
    # 3.10a same nonce again: rejected before anything is written
    before = out1.clone()
    with pytest.raises(C.NonceReuseError, match="NONCE_REUSE_DETECTED"):
        codec.encode_cold_pages_peak_into(k.unsqueeze(0), v.unsqueeze(0), th_t, out1, TENANT, sess, aad1)
    assert torch.equal(out1, before)
    # 3.10b distinct sequence nonces never share a ChaCha20 nonce
    assert ring.pack_chacha20_nonce((1 << 32) | 7, 14, 0) != ring.pack_chacha20_nonce((2 << 32) | 7, 14, 0)
    # 3.10c version 2 of the slot; version 1 is now a stale replay
    aad2 = dataclasses.replace(aad1, sequence_nonce=11)
    out2 = torch.empty_like(out1)
    codec.encode_cold_pages_peak_into(k.unsqueeze(0), v.unsqueeze(0), th_t, out2, TENANT, sess, aad2)
    codec.decode_cold_page_tensor(out2[0], TENANT, sess, MODEL, LAYER, th)
    ok = torch.full((1,) + tuple(k.shape), 7.0, dtype=torch.float16, device="cuda")
    ov = torch.full_like(ok, 7.0)
    with pytest.raises(C.StalePageReplayError, match="is older than latest slot version=11"):
        codec.decode_cold_pages_peak_into(out1, th_t, ok, ov, TENANT, sess, MODEL, LAYER)
    assert not ok.any() and not ov.any()  # outputs zeroed on failure
    # 3.11 shred + re-derive: the archived blob stays closed
    assert ring.crypto_shred_session(TENANT, sess)
    ring.derive_or_get(TENANT, sess)
    with pytest.raises(C.KVIntegrityError):
        codec.decode_cold_page_tensor(out2[0], TENANT, sess, MODEL, LAYER, th)


def test_transactional_session_state(pkg, C, S):
    """bench_cold_page_pipeline.py:484-610 (test 3.12) on the HIP codec."""
    geo = _geom(S)
    ring = C.EphemeralSessionKeyRing(bytes(range(2, 42)))
    codec = C.NativeCppFusedColdPageCodec(geo, ring)
    k, v = _pages(geo, seed=2)
    sess = "sess-code003"
    ring.derive_or_get(TENANT, sess)
    base = S.ColdPageAAD.from_context(TENANT, MODEL, LAYER, TOKENS, sequence_nonce=10,
                                      preset=S.QuantPreset.INT4_SYM, rope_mode=S.RoPEMode.PRESERVE_FP8)
    th = base.page_token_hash
    nbytes = geo.cold_blob_bytes(base.preset, base.rope_mode)
    # 3.12a two racing encodes of one nonce: exactly one succeeds
    barrier = threading.Barrier(2)

    def worker(aad_w, th_w):
        out = torch.empty((1, nbytes), dtype=torch.uint8, device="cuda")
        barrier.wait(timeout=10)
        codec.encode_cold_pages_peak_into(k.unsqueeze(0), v.unsqueeze(0),
                                          torch.tensor([_i64(th_w)], dtype=torch.int64), out, TENANT,
                                          sess, aad_w)
        return out

    with ThreadPoolExecutor(max_workers=2) as pool:
        futs = [pool.submit(worker, dataclasses.replace(base, sequence_nonce=20, page_token_hash=th), th),
                pool.submit(worker, dataclasses.replace(base, sequence_nonce=20, page_token_hash=th ^ 3), th ^ 3)]
        outcomes = []
        for f in futs:
            try:
                f.result(timeout=60)
                outcomes.append("ok")
            except C.NonceReuseError:
                outcomes.append("nonce_reuse")
    assert sorted(outcomes) == ["nonce_reuse", "ok"]
    # 3.12b a failed encode (wrong page shape) still burns its nonce
    fail = dataclasses.replace(base, sequence_nonce=25)
    with pytest.raises(RuntimeError, match="does not match geometry"):
        codec.encode_cold_page_tensor(k[:1], v, TENANT, sess, fail)
    with pytest.raises(C.NonceReuseError):
        codec.encode_cold_page_tensor(k, v, TENANT, sess, fail)
    # 3.12c out-of-order commit does not roll back the slot watermark
    orig = codec.keyring.preflight_validate_egress
    low_ready, high_done = threading.Event(), threading.Event()

    def ordered(*a, **kw):
        res = orig(*a, **kw)
        if kw.get("session_id") == sess and kw.get("base_sequence_nonce") == 30:
            low_ready.set()
            assert high_done.wait(timeout=30)
        return res

    codec.keyring.preflight_validate_egress = ordered
    try:
        with ThreadPoolExecutor(max_workers=1) as pool:
            f_low = pool.submit(codec.encode_cold_page_tensor, k, v, TENANT, sess,
                                dataclasses.replace(base, sequence_nonce=30))
            assert low_ready.wait(timeout=30)
            blob31 = codec.encode_cold_page_tensor(k, v, TENANT, sess, dataclasses.replace(base, sequence_nonce=31))
            high_done.set()
            blob30 = f_low.result(timeout=60)
    finally:
        codec.keyring.preflight_validate_egress = orig
    with pytest.raises(C.StalePageReplayError):
        codec.decode_cold_page_tensor(blob30, TENANT, sess, MODEL, LAYER, th)
    codec.decode_cold_page_tensor(blob31, TENANT, sess, MODEL, LAYER, th)


@pytest.mark.parametrize("mla,dtype", [(False, torch.float16), (False, torch.bfloat16), (True, torch.bfloat16)])
def test_batch_paths_vs_oracle(pkg, O, C, S, mla, dtype):
    """encode_cold_pages_batch_tensor / decode_cold_pages_batch_tensor /
    decode_cold_pages_peak_into (nfc:284-520) on 8 pages, against the oracle;
    then one tampered page fails the whole batch and zeroes every output."""
    geo = _geom(S, mla)
    ring = C.EphemeralSessionKeyRing(bytes(range(3, 43)))
    codec = C.NativeCppFusedColdPageCodec(geo, ring, dtype=dtype)
    B = 8
    k, v = _pages(geo, B, seed=3, dtype=dtype)
    sess = "sess-batch"
    aad = S.ColdPageAAD(S.hash32(TENANT), S.hash32(MODEL), LAYER, 0, ring.next_sequence_nonce(TENANT, sess, B),
                        preset=S.QuantPreset.K8V4_ASYM, rope_mode=S.RoPEMode.PRESERVE_FP8, head_group_id=2)
    ths = [_i64(S.hash64_tokens(range(64 * i, 64 * i + 64))) for i in range(B)]
    th_t = torch.tensor(ths, dtype=torch.int64)
    blobs = codec.encode_cold_pages_batch_tensor(k, v, th_t, TENANT, sess, aad)
    keys = _session_keys(ring, TENANT, sess)
    want = _oracle_blobs(O, geo, k, v, ths, aad, keys)
    assert np.array_equal(blobs.cpu().numpy(), want)
    rc, _, ok, ov = _oracle_decode(O, geo, want, ths, aad.tenant_id_hash, aad.model_id_hash, LAYER, keys, dtype)
    assert rc == 0
    kd, vd = codec.decode_cold_pages_batch_tensor(blobs, th_t.cuda(), TENANT, sess, MODEL, LAYER)
    assert kd.dtype == dtype and np.array_equal(_bits(kd), ok)
    assert (vd is None) == mla and (mla or np.array_equal(_bits(vd), ov))
    ko = torch.empty_like(k)
    vo = None if mla else torch.empty_like(v)
    codec.decode_cold_pages_peak_into(blobs, th_t, ko, vo, TENANT, sess, MODEL, LAYER,
                                      min_sequence_nonce=aad.sequence_nonce)
    assert torch.equal(ko, kd) and (mla or torch.equal(vo, vd))
    # a replayed batch below the caller's floor
    with pytest.raises(C.StalePageReplayError, match="min_sequence_nonce"):
        codec.decode_cold_pages_peak_into(blobs, th_t, ko, vo, TENANT, sess, MODEL, LAYER,
                                          min_sequence_nonce=aad.sequence_nonce + 1)
    assert not ko.any()
    # one tampered page: all-or-nothing
    bad = blobs.clone()
    bad[5, 100] ^= 0x40
    ko.fill_(1)
    with pytest.raises(C.KVIntegrityError, match="MAC verification failed"):
        codec.decode_cold_pages_peak_into(bad, th_t, ko, vo, TENANT, sess, MODEL, LAYER)
    assert not ko.any() and (mla or not vo.any())
    # argument checks and aliasing
    if not mla:
        with pytest.raises(RuntimeError, match="must not alias or overlap"):
            codec.decode_cold_pages_peak_into(blobs, th_t, ko, ko, TENANT, sess, MODEL, LAYER)
    with pytest.raises(RuntimeError, match="does not match batch geometry"):
        codec.decode_cold_pages_peak_into(blobs[:4], th_t[:4], ko, vo, TENANT, sess, MODEL, LAYER)
    aad_next = dataclasses.replace(aad, sequence_nonce=ring.next_sequence_nonce(TENANT, sess, B))
    with pytest.raises(RuntimeError, match="out_blobs_u8 must not alias"):
        aliased = k.view(torch.uint8).reshape(-1)[:blobs.numel()].view(blobs.shape)
        codec.encode_cold_pages_peak_into(k, v, th_t, aliased, TENANT, sess, aad_next)


@pytest.mark.parametrize("mla,preset,rope", [(False, 4, 3), (False, 5, 1), (True, 6, 3)])
def test_codec_class_extension_presets(pkg, O, C, S, mla, preset, rope):
    """The session-bound codec with the extension presets: batch encode ==
    oracle; decode needs accept_extension_layouts (otherwise the reference's
    flags check rejects the page: KVIntegrityError, outputs zeroed)."""
    geo = _geom(S, mla)
    ring = C.EphemeralSessionKeyRing(bytes(range(5, 45)))
    codec = C.NativeCppFusedColdPageCodec(geo, ring, dtype=torch.bfloat16, accept_extension_layouts=True)
    strict = C.NativeCppFusedColdPageCodec(geo, ring, dtype=torch.bfloat16)
    B = 4
    k, v = _pages(geo, B, seed=9, dtype=torch.bfloat16)
    sess = "sess-ext"
    aad = S.ColdPageAAD(S.hash32(TENANT), S.hash32(MODEL), LAYER, 0, ring.next_sequence_nonce(TENANT, sess, B),
                        preset=S.QuantPreset(preset), rope_mode=S.RoPEMode(rope), head_group_id=1)
    ths = [_i64(S.hash64_tokens(range(64 * i, 64 * i + 64))) for i in range(B)]
    th_t = torch.tensor(ths, dtype=torch.int64)
    blobs = codec.encode_cold_pages_batch_tensor(k, v, th_t, TENANT, sess, aad)
    keys = _session_keys(ring, TENANT, sess)
    want = _oracle_blobs(O, geo, k, v, ths, aad, keys)
    assert np.array_equal(blobs.cpu().numpy(), want)
    rc, _, ok, ov = _oracle_decode(O, geo, want, ths, aad.tenant_id_hash, aad.model_id_hash, LAYER, keys,
                                   torch.bfloat16)
    assert rc == 0
    ko = torch.full_like(k, 3.0)
    vo = None if mla else torch.full_like(v, 3.0)
    with pytest.raises(C.KVIntegrityError):
        strict.decode_cold_pages_peak_into(blobs, th_t, ko, vo, TENANT, sess, MODEL, LAYER)
    assert not ko.any() and (mla or not vo.any())
    kd, vd = codec.decode_cold_pages_batch_tensor(blobs, th_t.cuda(), TENANT, sess, MODEL, LAYER)
    assert np.array_equal(_bits(kd), ok) and (mla or np.array_equal(_bits(vd), ov))
