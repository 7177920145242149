"""Full-size workloads on the GPU path (16,384 pages each), through the descriptor API.

At these sizes the whole batch is checked through properties that do not need
the oracle (every page verifies, a second encode is identical, tampering one
page changes no other page's output) and a seeded sample of pages is checked
byte for byte against the oracle (blobs and decoded pages).

* 1 GiB BF16 prefix, K8V4 + PRESERVE_FP8 (4096 tokens x 64 layers).
* The same prefix under the reference's FP8_ONLY preset (int8 everywhere,
  QUANTIZE_ALL) with one bit flipped in 1% of pages: every tampered page is
  rejected with the verdict its bit implies (cpp:2313-2355) and zeroed,
  every other page decodes exactly as without tampering.
* DeepSeek-MLA single buffer: 64-token pages of 576 values, INT4_SYM latent
  + PRESERVE_FP8 RoPE.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SAMPLE = 24


@pytest.fixture(scope="module")
def W(pkg):
    import vlx_tee_amd.workloads as W
    return W


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _encode(pkg, W, name):
    import vlx_tee_amd.pages as P
    w = W.WORKLOADS[name]
    dev = torch.device("cuda")
    keys = W.session_keys()
    k, v = W.generate(w, dev, torch.bfloat16)
    th, seq, layers = W.page_metadata(w)
    blobs = torch.empty((w.n_pages, w.blob_bytes), dtype=torch.uint8, device=dev)
    d = P.build_descriptors(k, v, blobs, th, seq, layers)
    geo = dict(num_tokens=w.num_tokens, num_heads=w.num_heads, head_dim=w.head_dim,
               rope_dim=w.rope_dim, dtype=torch.bfloat16, is_mla_single_buffer=w.mla)
    P.egress(d, w.n_pages, preset=w.preset, rope_mode=w.rope_mode,
             expected_payload_bytes=w.payload_bytes, tenant_id_hash=W.TENANT_HASH,
             model_id_hash=W.MODEL_HASH, **geo, **keys)
    torch.cuda.synchronize()
    return w, keys, k, v, th, seq, layers, blobs, geo


def _decode(pkg, W, w, keys, blobs, th, seq, layers, geo, per_page):
    import vlx_tee_amd.pages as P
    ko = torch.full((w.n_pages, w.num_tokens, w.num_heads, w.head_dim), 3.0, dtype=torch.bfloat16,
                    device=blobs.device)
    vo = None if w.mla else torch.full_like(ko, 3.0)
    st = torch.full((w.n_pages,), -1, dtype=torch.int32, device=blobs.device)
    d = P.build_descriptors(ko, vo, blobs, th, seq, layers)
    rc = P.ingress(d, w.n_pages, w.blob_bytes, expected_tenant_hash=W.TENANT_HASH,
                   expected_model_hash=W.MODEL_HASH, page_status=st, per_page=per_page, **geo, **keys)
    torch.cuda.synchronize()
    return rc, st.cpu().numpy(), ko, vo


def _sample_vs_oracle(O, W, w, keys, k, v, blobs, ko, vo, th, seq, layers, pages):
    """Sampled pages: blob bytes from the oracle's encoder, decoded pages from
    the oracle's decoder (each page with its own layer id and sequence nonce)."""
    for pg in pages:
        kb = _bits(k[pg:pg + 1])
        vb = None if v is None else _bits(v[pg:pg + 1])
        want = O.egress_batch(kb, vb, th[pg:pg + 1], dtype=O.BF16, preset=w.preset,
                              rope_mode=w.rope_mode, rope_dim=w.rope_dim,
                              expected_payload_bytes=w.payload_bytes, tenant_id_hash=W.TENANT_HASH,
                              model_id_hash=W.MODEL_HASH, layer_id=int(layers[pg]), head_group_id=0,
                              base_sequence_nonce=int(seq[pg]), **keys)
        got = blobs[pg:pg + 1].cpu().numpy()
        assert np.array_equal(got, want), f"page {pg}: blob differs from the oracle"
        rc, st, ok, ov = O.ingress_batch(got, th[pg:pg + 1], num_tokens=w.num_tokens,
                                         num_heads=w.num_heads, head_dim=w.head_dim,
                                         rope_dim=w.rope_dim, is_mla_single_buffer=w.mla,
                                         dtype=O.BF16, expected_tenant_hash=W.TENANT_HASH,
                                         expected_model_hash=W.MODEL_HASH,
                                         expected_layer_id=int(layers[pg]), **keys)
        assert rc == 0
        assert np.array_equal(_bits(ko[pg:pg + 1]), ok), f"page {pg}: decoded K differs"
        if vo is not None:
            assert np.array_equal(_bits(vo[pg:pg + 1]), ov), f"page {pg}: decoded V differs"


def _sample(n, seed):
    return np.sort(np.random.default_rng(seed).choice(n, size=SAMPLE, replace=False))


@pytest.mark.parametrize("name", ["c2_k8v4_prefix1g", "c2_int4_prefix1g", "c4_mla_int4"])
def test_full_prefix_roundtrip(pkg, O, W, name):
    print(f"case {name}: encode", flush=True)
    w, keys, k, v, th, seq, layers, blobs, geo = _encode(pkg, W, name)
    first = blobs.clone()
    import vlx_tee_amd.pages as P
    d = P.build_descriptors(k, v, blobs, th, seq, layers)
    P.egress(d, w.n_pages, preset=w.preset, rope_mode=w.rope_mode,
             expected_payload_bytes=w.payload_bytes, tenant_id_hash=W.TENANT_HASH,
             model_id_hash=W.MODEL_HASH, **geo, **keys)
    torch.cuda.synchronize()
    assert torch.equal(first, blobs), "egress is not deterministic"
    del first
    print(f"case {name}: decode", flush=True)
    rc, st, ko, vo = _decode(pkg, W, w, keys, blobs, th, seq, layers, geo, per_page=False)
    assert rc == 0 and (st == 0).all()
    print(f"case {name}: sample vs oracle", flush=True)
    _sample_vs_oracle(O, W, w, keys, k, v, blobs, ko, vo, th, seq, layers, _sample(w.n_pages, 7))
    import vlx_tee_amd.native_hip_codec as H
    assert H.device_diag() == 0


def _expected_verdict(byte):
    """Verdict of a page with one flipped bit at blob byte `byte` (cpp:2313-2355):
    magic / version -> 1; tenant, model, layer, token hash -> 2; anything else
    the MAC covers (flags, head group, sequence nonce, payload) -> 3."""
    if byte < 3:
        return 1
    if 4 <= byte < 14 or 16 <= byte < 24:
        return 2
    return 3


def test_fp8only_tamper_stress_full_prefix(pkg, O, W):
    print("case c3_fp8only_tamper: encode", flush=True)
    w, keys, k, v, th, seq, layers, blobs, geo = _encode(pkg, W, "c3_fp8only_tamper")
    rc, st, ko_clean, vo_clean = _decode(pkg, W, w, keys, blobs, th, seq, layers, geo, per_page=True)
    assert rc == 0 and (st == 0).all()
    pages, bits = W.tamper_plan(w, w.blob_bytes)
    assert len(pages) == round(0.01 * w.n_pages)
    tampered = blobs.clone()
    idx = torch.from_numpy(pages).to(blobs.device)
    cols = torch.from_numpy(bits // 8).to(blobs.device)
    masks = torch.from_numpy((1 << (bits % 8)).astype(np.uint8)).to(blobs.device)
    tampered[idx, cols] = tampered[idx, cols] ^ masks
    print(f"case c3_fp8only_tamper: decode with {len(pages)} tampered pages", flush=True)
    rc, st, ko, vo = _decode(pkg, W, w, keys, tampered, th, seq, layers, geo, per_page=True)
    want = np.zeros(w.n_pages, dtype=np.int32)
    want[pages] = [_expected_verdict(int(b) // 8) for b in bits]
    assert np.array_equal(st, want)
    # PoisonShield hit bitmap: False exactly at the tampered slots
    import vlx_tee_amd.serving as SV
    hits = SV.hit_bitmap(torch.from_numpy(st).to(blobs.device)).cpu().numpy()
    assert hits.sum() == w.n_pages - len(pages) and not hits[pages].any()
    assert rc == int(want[pages[0]])  # the lowest failing page's verdict
    # tampered pages zeroed, every other page exactly as without tampering
    ko_clean[idx] = 0
    vo_clean[idx] = 0
    assert torch.equal(ko, ko_clean) and torch.equal(vo, vo_clean)
    # all-or-nothing (the reference's policy): every output zeroed, lowest verdict returned
    rc2, st2, ko2, vo2 = _decode(pkg, W, w, keys, tampered, th, seq, layers, geo, per_page=False)
    assert rc2 == rc and np.array_equal(st2, want)
    assert not ko2.any() and not vo2.any()
    # the oracle agrees on a sample of tampered pages and of untouched pages
    print("case c3_fp8only_tamper: sample vs oracle", flush=True)
    tb = tampered.cpu().numpy()
    for pg in list(pages[:8]):
        rc_o, st_o, _, _ = O.ingress_batch(tb[pg:pg + 1], th[pg:pg + 1], num_tokens=w.num_tokens,
                                           num_heads=w.num_heads, head_dim=w.head_dim,
                                           rope_dim=w.rope_dim, is_mla_single_buffer=w.mla,
                                           dtype=O.BF16, expected_tenant_hash=W.TENANT_HASH,
                                           expected_model_hash=W.MODEL_HASH,
                                           expected_layer_id=int(layers[pg]), **keys)
        assert int(st_o[0]) == int(st[pg]), f"page {pg}: verdict differs from the oracle"
    clean = np.setdiff1d(np.arange(w.n_pages), pages)
    _sample_vs_oracle(O, W, w, keys, k, v, blobs, ko, vo, th, seq, layers,
                      np.sort(np.random.default_rng(3).choice(clean, size=SAMPLE, replace=False)))


def test_wire_ring_egress_copy(pkg, W):
    """The egress wire step: a full prefix's blobs leave HBM through a ring of
    two pinned host slots, a quarter of the pages per push, byte for byte."""
    import time
    import vlx_tee_amd.serving as SV
    print("case c2_k8v4_prefix1g: encode for the wire ring", flush=True)
    w, keys, k, v, th, seq, layers, blobs, geo = _encode(pkg, W, "c2_k8v4_prefix1g")
    del k, v
    torch.cuda.synchronize()
    q = w.n_pages // 4
    ring = SV.WireRing(q * w.blob_bytes, n_slots=2)
    host = blobs.cpu()
    t0 = time.perf_counter()
    got = []
    for part in range(4):
        slot = ring.push(blobs[part * q:(part + 1) * q])
        if part >= 1:
            got.append(ring.wait((slot + 1) % 2).clone())
    got.append(ring.wait(slot).clone())
    dt = time.perf_counter() - t0
    print(f"wire ring: {blobs.numel() / dt / 1e9:.1f} GB/s device-to-pinned-host "
          f"({blobs.numel()} blob bytes, 4 pushes)", flush=True)
    for part in range(4):
        assert torch.equal(got[part], host[part * q:(part + 1) * q].reshape(-1))
    with pytest.raises(ValueError):
        ring.push(blobs)  # larger than a slot
