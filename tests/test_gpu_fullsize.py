"""Full-size workloads on the GPU path (16,384 pages each), through the descriptor API.

At these sizes the whole batch is checked through properties that do not need
the oracle (every page verifies, a second encode is identical, tampering one
page changes no other page's output) and a seeded sample of pages is checked
byte for byte against the oracle (blobs and decoded pages); a second test
compares every page of every workload's batch with the oracle.

* 1 GiB BF16 prefix, K8V4 + PRESERVE_FP8 (4096 tokens x 64 layers).
* The same prefix under the reference's FP8_ONLY preset (int8 everywhere,
  QUANTIZE_ALL) with one bit flipped in 1% of pages: every tampered page is
  rejected with the verdict its bit implies (cpp:2313-2355) and zeroed,
  every other page decodes exactly as without tampering.
* DeepSeek-MLA single buffer: 64-token pages of 576 values, INT4_SYM latent
  + PRESERVE_FP8 RoPE.
* The same three workloads as the task words them, with the extension kinds:
  K int8 asymmetric per 64 + e4m3 RoPE / V int4 per 32; FP8 e4m3 with 1% of
  the pages tampered; MLA latent int4 per 32 + e4m3 RoPE.
* A paged KV pool: K, V and blob slots drawn independently from larger
  pools, descriptors in shuffled order; same blobs and pages as the
  contiguous batch.
* The two small batches exactly as specified (64 and 256 pages of 16 tokens x
  4 KV heads x 128, INT4_SYM + PRESERVE_FP8, N(0,1) with RoPE columns x8 and
  1% of the channels x20, seed-7 keys, nonce = page index): every blob and
  every decoded page against the oracle, FP16 and BF16.
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
             model_id_hash=W.MODEL_HASH, ext_layouts=w.extension, **geo, **keys)
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
                   expected_model_hash=W.MODEL_HASH, page_status=st, per_page=per_page,
                   ext_layouts=w.extension, **geo, **keys)
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


@pytest.mark.parametrize("name", ["c2_k8v4_prefix1g", "c2_int4_prefix1g", "c4_mla_int4",
                                  "c2_k8v4asym_prefix1g", "c4_mla_int4g32"])
def test_full_prefix_roundtrip(pkg, O, W, name):
    print(f"case {name}: encode", flush=True)
    w, keys, k, v, th, seq, layers, blobs, geo = _encode(pkg, W, name)
    first = blobs.clone()
    import vlx_tee_amd.pages as P
    d = P.build_descriptors(k, v, blobs, th, seq, layers)
    P.egress(d, w.n_pages, preset=w.preset, rope_mode=w.rope_mode,
             expected_payload_bytes=w.payload_bytes, tenant_id_hash=W.TENANT_HASH,
             model_id_hash=W.MODEL_HASH, ext_layouts=w.extension, **geo, **keys)
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


@pytest.mark.parametrize("name", ["c2_k8v4_prefix1g", "c2_int4_prefix1g", "c4_mla_int4", "c3_fp8only_tamper",
                                  "c2_k8v4asym_prefix1g", "c4_mla_int4g32", "c3_e4m3_tamper"])
def test_full_prefix_every_page_vs_oracle(pkg, O, W, name):
    """The whole 16,384-page batch byte for byte (the tamper workloads before
    any tampering): every blob (codes, scales, ciphertext, tag) equals the
    oracle encoder's and every decoded page equals the oracle decoder's, one
    layer (its own layer id and first sequence nonce) per oracle call."""
    import os
    threads = max(1, min(16, os.cpu_count() or 1))
    print(f"case {name}: encode", flush=True)
    w, keys, k, v, th, seq, layers, blobs, geo = _encode(pkg, W, name)
    rc, st, ko, vo = _decode(pkg, W, w, keys, blobs, th, seq, layers, geo, per_page=False)
    assert rc == 0 and (st == 0).all()
    ppl = w.pages_per_layer
    for a in range(0, w.n_pages, ppl):
        b = min(a + ppl, w.n_pages)
        layer = int(layers[a])
        assert (layers[a:b] == layer).all() and (seq[a:b] == seq[a] + np.arange(b - a, dtype=np.uint64)).all()
        if a % (16 * ppl) == 0:
            print(f"case {name}: pages {a}..{b - 1} vs oracle", flush=True)
        want = O.egress_batch(_bits(k[a:b]), None if v is None else _bits(v[a:b]), th[a:b], dtype=O.BF16,
                              preset=w.preset, rope_mode=w.rope_mode, rope_dim=w.rope_dim,
                              expected_payload_bytes=w.payload_bytes, tenant_id_hash=W.TENANT_HASH,
                              model_id_hash=W.MODEL_HASH, layer_id=layer, head_group_id=0,
                              base_sequence_nonce=int(seq[a]), threads=threads, **keys)
        got = blobs[a:b].cpu().numpy()
        bad = np.nonzero((got != want).any(axis=1))[0]
        assert bad.size == 0, f"pages {(a + bad[:8]).tolist()}: blob differs from the oracle"
        orc, ost, ok, ov = O.ingress_batch(got, th[a:b], num_tokens=w.num_tokens, num_heads=w.num_heads,
                                           head_dim=w.head_dim, rope_dim=w.rope_dim,
                                           is_mla_single_buffer=w.mla, dtype=O.BF16,
                                           expected_tenant_hash=W.TENANT_HASH,
                                           expected_model_hash=W.MODEL_HASH, expected_layer_id=layer,
                                           threads=threads, **keys)
        assert orc == 0
        assert np.array_equal(_bits(ko[a:b]), ok), f"layer {layer}: decoded K differs from the oracle"
        if vo is not None:
            assert np.array_equal(_bits(vo[a:b]), ov), f"layer {layer}: decoded V differs from the oracle"


_DESC = np.dtype([("k", "<u8"), ("v", "<u8"), ("blob", "<u8"), ("token_hash", "<i8"),
                  ("sequence_nonce", "<u8"), ("layer_id", "<u2"), ("head_group_id", "<u2"),
                  ("reserved", "<u4")])


def _pool_descs(kpool, vpool, bpool, sk, sv, sb, th, seq, layers, order):
    """Descriptor i for page order[i], whose K, V and blob sit in pool slots
    sk / sv / sb of that page."""
    pb = kpool[0].numel() * kpool.element_size()
    j = order
    d = np.zeros(len(order), dtype=_DESC)
    d["k"] = np.uint64(kpool.data_ptr()) + sk[j].astype(np.uint64) * np.uint64(pb)
    d["v"] = np.uint64(vpool.data_ptr()) + sv[j].astype(np.uint64) * np.uint64(pb)
    d["blob"] = np.uint64(bpool.data_ptr()) + sb[j].astype(np.uint64) * np.uint64(bpool.size(1))
    d["token_hash"] = th[j]
    d["sequence_nonce"] = seq[j]
    d["layer_id"] = layers[j]
    return torch.from_numpy(d.view(np.uint8).reshape(len(order), _DESC.itemsize).copy()).to(kpool.device)


def test_descriptors_over_a_scattered_pool(pkg, W):
    """A paged KV pool: 2,048 pages of the K8V4 prefix (8 layers) whose K, V
    and blob slots are drawn independently from pools three times as large,
    with the descriptors in shuffled order (layers interleaved).  Egress and
    ingress over those descriptors give exactly the blobs and pages of the
    contiguous batch."""
    import vlx_tee_amd.pages as P
    print("case scattered pool: contiguous batch", flush=True)
    w = W.WORKLOADS["c2_k8v4_prefix1g"]
    n, dev = 2048, torch.device("cuda")
    keys = W.session_keys()
    k, v = W.generate(w, dev, torch.bfloat16, n_pages=n)
    th, seq, layers = W.page_metadata(w, 0, n)
    geo = dict(num_tokens=w.num_tokens, num_heads=w.num_heads, head_dim=w.head_dim, rope_dim=w.rope_dim,
               dtype=torch.bfloat16, is_mla_single_buffer=False)
    eg = dict(preset=w.preset, rope_mode=w.rope_mode, expected_payload_bytes=w.payload_bytes,
              tenant_id_hash=W.TENANT_HASH, model_id_hash=W.MODEL_HASH, **geo, **keys)
    ig = dict(expected_tenant_hash=W.TENANT_HASH, expected_model_hash=W.MODEL_HASH, per_page=False, **geo, **keys)
    blobs = torch.empty((n, w.blob_bytes), dtype=torch.uint8, device=dev)
    P.egress(P.build_descriptors(k, v, blobs, th, seq, layers), n, **eg)
    ko, vo = torch.empty_like(k), torch.empty_like(v)
    st = torch.full((n,), -1, dtype=torch.int32, device=dev)
    assert P.ingress(P.build_descriptors(ko, vo, blobs, th, seq, layers), n, w.blob_bytes, page_status=st, **ig) == 0
    torch.cuda.synchronize()

    print("case scattered pool: descriptors over the pool", flush=True)
    rng = np.random.default_rng(11)
    slots = 3 * n
    sk, sv, sb = (rng.permutation(slots)[:n] for _ in range(3))
    order = rng.permutation(n)
    kpool = torch.zeros((slots,) + tuple(k.shape[1:]), dtype=k.dtype, device=dev)
    vpool = torch.zeros_like(kpool)
    bpool = torch.zeros((slots, w.blob_bytes), dtype=torch.uint8, device=dev)
    kpool[torch.from_numpy(sk).to(dev)] = k
    vpool[torch.from_numpy(sv).to(dev)] = v
    P.egress(_pool_descs(kpool, vpool, bpool, sk, sv, sb, th, seq, layers, order), n, **eg)
    torch.cuda.synchronize()
    assert torch.equal(bpool[torch.from_numpy(sb).to(dev)], blobs)

    # decode from the pool's blob slots into other scattered slots
    ok_s, ov_s = rng.permutation(slots)[:n], rng.permutation(slots)[:n]
    kout = torch.full_like(kpool, 3.0)
    vout = torch.full_like(vpool, 3.0)
    st.fill_(-1)
    d = _pool_descs(kout, vout, bpool, ok_s, ov_s, sb, th, seq, layers, order)
    assert P.ingress(d, n, w.blob_bytes, page_status=st, **ig) == 0
    torch.cuda.synchronize()
    assert torch.equal(kout[torch.from_numpy(ok_s).to(dev)], ko)
    assert torch.equal(vout[torch.from_numpy(ov_s).to(dev)], vo)


def _expected_verdict(byte):
    """Verdict of a page with one flipped bit at blob byte `byte` (cpp:2313-2355):
    magic / version -> 1; tenant, model, layer, token hash -> 2; anything else
    the MAC covers (flags, head group, sequence nonce, payload) -> 3."""
    if byte < 3:
        return 1
    if 4 <= byte < 14 or 16 <= byte < 24:
        return 2
    return 3


@pytest.mark.parametrize("name", ["c3_fp8only_tamper", "c3_e4m3_tamper"])
def test_tamper_stress_full_prefix(pkg, O, W, name):
    print(f"case {name}: encode", flush=True)
    w, keys, k, v, th, seq, layers, blobs, geo = _encode(pkg, W, name)
    rc, st, ko_clean, vo_clean = _decode(pkg, W, w, keys, blobs, th, seq, layers, geo, per_page=True)
    assert rc == 0 and (st == 0).all()
    pages, bits = W.tamper_plan(w, w.blob_bytes)
    assert len(pages) == round(0.01 * w.n_pages)
    tampered = blobs.clone()
    idx = torch.from_numpy(pages).to(blobs.device)
    cols = torch.from_numpy(bits // 8).to(blobs.device)
    masks = torch.from_numpy((1 << (bits % 8)).astype(np.uint8)).to(blobs.device)
    tampered[idx, cols] = tampered[idx, cols] ^ masks
    print(f"case {name}: decode with {len(pages)} tampered pages", flush=True)
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
    print(f"case {name}: sample vs oracle", flush=True)
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


def test_wire_ring_egress_copy(pkg, O, W):
    """The egress wire step: a full prefix's blobs leave HBM through a ring of
    two pinned host slots, a quarter of the pages per push.  The pushes are
    issued right after the egress launch, with no synchronization: the ring's
    copy stream must wait for the kernel through its event.  The slots are
    compared with the blobs read back after a full synchronization, and a
    sample of pages with the oracle."""
    import time
    import vlx_tee_amd.pages as P
    import vlx_tee_amd.serving as SV
    w = W.WORKLOADS["c2_k8v4_prefix1g"]
    dev = torch.device("cuda")
    keys = W.session_keys()
    k, v = W.generate(w, dev, torch.bfloat16)
    th, seq, layers = W.page_metadata(w)
    blobs = torch.zeros((w.n_pages, w.blob_bytes), dtype=torch.uint8, device=dev)
    d = P.build_descriptors(k, v, blobs, th, seq, layers)
    geo = dict(num_tokens=w.num_tokens, num_heads=w.num_heads, head_dim=w.head_dim, rope_dim=w.rope_dim,
               dtype=torch.bfloat16, is_mla_single_buffer=w.mla)
    q = w.n_pages // 4
    ring = SV.WireRing(q * w.blob_bytes, n_slots=2)
    torch.cuda.synchronize()
    print("case c2_k8v4_prefix1g: egress + wire ring pushes, no synchronization between", flush=True)
    t0 = time.perf_counter()
    P.egress(d, w.n_pages, preset=w.preset, rope_mode=w.rope_mode, expected_payload_bytes=w.payload_bytes,
             tenant_id_hash=W.TENANT_HASH, model_id_hash=W.MODEL_HASH, asynchronous=True, **geo, **keys)
    got = []
    for part in range(4):
        slot = ring.push(blobs[part * q:(part + 1) * q])
        if part >= 1:
            got.append(ring.wait((slot + 1) % 2).clone())
    got.append(ring.wait(slot).clone())
    dt = time.perf_counter() - t0
    print(f"wire ring: egress + {blobs.numel() / 1e9:.3f} GB to pinned host in {dt * 1e3:.1f} ms", flush=True)
    torch.cuda.synchronize()
    host = blobs.cpu()
    for part in range(4):
        assert torch.equal(got[part], host[part * q:(part + 1) * q].reshape(-1))
    ring_pages = torch.cat(got).view(w.n_pages, w.blob_bytes).numpy()
    for pg in _sample(w.n_pages, 11)[:8]:
        want = O.egress_batch(_bits(k[pg:pg + 1]), _bits(v[pg:pg + 1]), th[pg:pg + 1], dtype=O.BF16, preset=w.preset,
                              rope_mode=w.rope_mode, rope_dim=w.rope_dim, expected_payload_bytes=w.payload_bytes,
                              tenant_id_hash=W.TENANT_HASH, model_id_hash=W.MODEL_HASH,
                              layer_id=int(layers[pg]), head_group_id=0, base_sequence_nonce=int(seq[pg]), **keys)
        assert np.array_equal(ring_pages[pg:pg + 1], want), f"page {pg}: ring bytes differ from the oracle"
    with pytest.raises(ValueError):
        ring.push(blobs)  # larger than a slot


@pytest.mark.parametrize("name", ["c0_int4_gqa64", "c1_int4_gqa256"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_small_batch_workloads_exact(pkg, O, W, name, dtype):
    """64- and 256-page INT4_SYM + PRESERVE_FP8 batches through the reference's
    peak entry point form (cpp:1904-2004): every blob (ciphertext and tag) and
    every decoded page equals the oracle's."""
    import vlx_tee_amd.native_hip_codec as H
    w = W.WORKLOADS[name]
    print(f"case {name} {dtype}", flush=True)
    keys = W.session_keys()
    k, v = W.generate(w, "cpu", dtype)
    th = torch.arange(w.n_pages, dtype=torch.int64)
    dev = torch.device("cuda")
    out = torch.full((w.n_pages, w.blob_bytes), 0xA5, dtype=torch.uint8, device=dev)
    H.fused_encode_cold_pages_peak_into(k.to(dev), v.to(dev), th, out, w.preset, w.rope_mode, w.rope_dim,
                                        w.payload_bytes, W.TENANT_HASH, W.MODEL_HASH, 0, 0, 0, keys["k0"],
                                        keys["k1"], keys["mk0"], keys["mk1"], keys["k2"], keys["k3"])
    torch.cuda.synchronize()
    odt = O.BF16 if dtype == torch.bfloat16 else O.FP16
    want = O.egress_batch(_bits(k), _bits(v), th.numpy(), dtype=odt, preset=w.preset, rope_mode=w.rope_mode,
                          rope_dim=w.rope_dim, expected_payload_bytes=w.payload_bytes,
                          tenant_id_hash=W.TENANT_HASH, model_id_hash=W.MODEL_HASH, layer_id=0,
                          head_group_id=0, base_sequence_nonce=0, **keys)
    got = out.cpu().numpy()
    assert np.array_equal(got, want), f"{int((got != want).any(axis=1).sum())} blobs differ from the oracle"
    ko, vo = torch.full_like(k, 3.0, device=dev), torch.full_like(v, 3.0, device=dev)
    H.fused_decode_cold_pages_peak_into(out, th, ko, vo, w.rope_dim, False, W.TENANT_HASH, W.MODEL_HASH, 0,
                                        keys["k0"], keys["k1"], keys["mk0"], keys["mk1"], keys["k2"], keys["k3"])
    rc, st, ok, ov = O.ingress_batch(want, th.numpy(), num_tokens=w.num_tokens, num_heads=w.num_heads,
                                     head_dim=w.head_dim, rope_dim=w.rope_dim, is_mla_single_buffer=False,
                                     dtype=odt, expected_tenant_hash=W.TENANT_HASH,
                                     expected_model_hash=W.MODEL_HASH, expected_layer_id=0, **keys)
    assert rc == 0
    assert np.array_equal(_bits(ko), ok) and np.array_equal(_bits(vo), ov)
